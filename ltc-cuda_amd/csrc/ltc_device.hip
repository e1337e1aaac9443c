// gfx950 kernels for the LTC fused ODE-solver path.
//
// Math (restated from ltc.py:42-63; gradients as csrc/ltc_kernels.cu:627-667
// and :323-338 compute them):
//   sensory  sn[b,t,h] = sum_d Ws*sig(Ss*(x-Ms))*Es,  sd[b,t,h] = sum_d Ws*sig(...)
//   unfold   a_ij = sig(S_ij*(v_i - M_ij))
//            n_j = sum_i a_ij*WE_ij + sn_j,  q_j = sum_i a_ij*WP_ij + sd_j
//            v_j <- (C_j*v_j + G_j*L_j + n_j) / (C_j + G_j + q_j + eps)
//
// Layout choices (all buffers in HBM, fp32):
//  * Lanes of a wave run over the OUTPUT neuron and each thread loops over a
//    slice of the reduction axis. Row-major [i][j] parameters are then read
//    as one contiguous 1 KiB float4 line per wave, with no transpose for the
//    forward and no cross-lane reduction inside the synapse loop.
//  * The four per-synapse operands travel as one float4 {S', c', WE, WP}
//    with S' = -S*log2(e) and c' = S*M*log2(e), so the gate is
//    rcp(1 + exp2(fma(S', v, c'))): one FMA, one v_exp_f32, one add and one
//    v_rcp_f32 per synapse.
//  * The sensory term depends on x only, so it is computed for every (b,t)
//    in one parallel pass before the sequential unfold loop.
//  * The unfold loop runs in one persistent launch: a workgroup owns NB batch
//    rows for all T*U unfolds, with the state in LDS and, when they fit,
//    each thread's synapse operands in registers for the whole launch.
//  * Backward: a reverse-time chain kernel produces dL/dv for every unfold
//    and saves alpha/beta; parameter gradients are then reduced over
//    (t,k,b) by separate kernels into partial buffers that a finalize kernel
//    sums in a fixed order. No atomics anywhere, so every result is bitwise
//    reproducible run to run.
#include <type_traits>

#include "ltc_internal.h"

namespace ltc {

thread_local LaunchEvents* g_launch_events = nullptr;

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegLn2 = -0.69314718055994531f;
constexpr float kLn2 = 0.69314718055994531f;

// The device's sticky fault flag: raised when a call's workgroups gave up
// waiting for each other (a gated fill after a cluster launch, or the fused
// row backward's finalize), read and cleared by the host (device_fault).
__device__ int g_fault;

// Exchange words between workgroups: {value bits, tag} written and read
// whole as 64-bit agent-scope atomics, so no fence or counter is needed.
__device__ __forceinline__ void xch_put(unsigned long long* w, float v, unsigned tag) {
  const unsigned long long word =
      (unsigned long long)__float_as_uint(v) | ((unsigned long long)tag << 32);
  __hip_atomic_store(w, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long xch_get(unsigned long long* w) {
  return __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// sigmoid(z) for zp = -z*log2(e). v_exp_f32 saturates to +inf for large zp
// and rcp(inf) = 0, while exp2 of a large negative zp is 0 and rcp(1) = 1, so
// both saturated limits are exact and a*(1-a) is 0 there (never inf/inf).
__device__ __forceinline__ float gate(float zp) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(zp));
}

// Workgroup barrier that orders LDS only. Global loads issued before it stay
// in flight (no vmcnt(0) wait), which lets the next unfold's operands stream
// in while the workgroup synchronises.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Sum of v over the wave, in every lane (xor butterfly).
// Sum of x over the four 16-lane groups of a wave, in every lane. gfx950's
// v_permlane32_swap / v_permlane16_swap exchange halves and rows of a wave
// in the VALU: after the two steps every lane holds (x0 + x2) + (x1 + x3)
// with the same bits.
__device__ __forceinline__ float group_sum4(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Sum of x over the eight 8-lane groups of a wave, in every lane: the two
// swaps of group_sum4, then DPP row_ror:8, which hands each lane the value
// of the lane 8 away within its 16-lane row.
__device__ __forceinline__ float group_sum8(float x) {
  x = group_sum4(x);
  const float y = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf,
                                                             0xf, false));
  return x + y;
}

// Sum of v over the wave, in every lane with the same bits, without LDS
// traffic: group_sum4 across the four 16-lane rows, then DPP row_ror by 8,
// 4, 2 and 1 within each row. Each step is a butterfly (the vector being
// rotated has period twice the shift), so both lanes of a pair add the
// same two values.
__device__ __forceinline__ float wave_sum(float v) {
  v = group_sum4(v);
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x122, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x121, 0xf, 0xf, false));
  return v;
}

// Largest value of v over the wave, as a wave-uniform value.
__device__ __forceinline__ int wave_max(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
  return __builtin_amdgcn_readfirstlane(v);
}

// Balanced lane order of a compacted kernel. Its synapse lanes (one per
// thread: a column's chunk of entries) hold different entry counts n <= 16,
// and a wave runs as many slots as its fullest lane. Ranking the lanes by
// count, largest first (ties by lane index), and giving the r-th ranked lane
// to thread r puts lanes of nearly equal counts in each wave, so waves run
// few padding slots, and the long waves and the short ones spread over the
// SIMDs (the workgroups of a CU place each wave index on different SIMDs).
// n: the count of this thread's own lane (lane = tid); returns the lane this
// thread evaluates. Every thread of the workgroup must call it (it holds two
// workgroup barriers). LDS: perm [nthr] ints, wcnt [nthr / 64][17] ints.
__device__ __forceinline__ int balanced_lane(int n, int tid, int nthr, int* perm, int* wcnt) {
  const int lane = tid & 63, w = tid >> 6, nw = nthr >> 6;
  const unsigned long long below = (1ull << lane) - 1ull;
  int local = 0;
#pragma unroll
  for (int v = 0; v <= 16; ++v) {
    const unsigned long long m = __ballot(n == v);
    if (n == v) local = __popcll(m & below);
    if (lane == 0) wcnt[w * 17 + v] = __popcll(m);
  }
  __syncthreads();
  // wave 0, lane v < 17: start[w][v] = (lanes of any wave with count > v)
  // + (lanes of count v in waves before w), written over wcnt in place
  if (w == 0) {
    int tot = 0;
    if (lane <= 16)
      for (int x = 0; x < nw; ++x) tot += wcnt[x * 17 + lane];
    int above = 0;
#pragma unroll
    for (int v = 1; v <= 16; ++v) {
      const int t = __shfl(tot, v, 64);
      if (v > lane) above += t;
    }
    if (lane <= 16) {
      int run = above;
      for (int x = 0; x < nw; ++x) {
        const int c = wcnt[x * 17 + lane];
        wcnt[x * 17 + lane] = run;
        run += c;
      }
    }
  }
  __syncthreads();
  perm[wcnt[w * 17 + n] + local] = tid;
  __syncthreads();
  return perm[tid];
}

// Sum of the K partials base[0], base[stride], ..., base[(K-1)*stride]: all K
// LDS reads are issued before the first add, then a fixed pairwise tree.
template <int K, class V>
__device__ __forceinline__ V tree_sum(const V* base, int stride) {
  V v[K];
#pragma unroll
  for (int s = 0; s < K; ++s) v[s] = base[s * stride];
#pragma unroll
  for (int w = 1; w < K; w *= 2) {
#pragma unroll
    for (int s = 0; s + w < K; s += 2 * w) v[s] += v[s + w];
  }
  return v[0];
}

// KS (a power of two <= 16) is a runtime value: groups of four reads are in
// flight together and summed pairwise, groups are added in order.
template <class V>
__device__ __forceinline__ V ks_sum(const V* base, int stride, int KS) {
  if (KS < 4) return KS == 2 ? base[0] + base[stride] : base[0];
  V acc = tree_sum<4>(base, stride);
  for (int g = 4; g < KS; g += 4) acc += tree_sum<4>(base + g * stride, stride);
  return acc;
}

// KS = 8 or 16 (the cluster kernels): all KS reads in flight together, one
// LDS round trip, then a fixed pairwise tree.
template <class V>
__device__ __forceinline__ V ks_sum_wide(const V* base, int stride, int KS) {
  return KS == 16 ? tree_sum<16>(base, stride) : tree_sum<8>(base, stride);
}

// Any KS (a power of two <= 16) in one LDS round trip: for the kernels whose
// threads finish one or two rows, where the extra registers are free.
template <class V>
__device__ __forceinline__ V ks_sum_1r(const V* base, int stride, int KS) {
  switch (KS) {
    case 16: return tree_sum<16>(base, stride);
    case 8: return tree_sum<8>(base, stride);
    case 4: return tree_sum<4>(base, stride);
    case 2: return base[0] + base[stride];
    default: return base[0];
  }
}

// Operand images read through a buffer resource: the wave-uniform row offset
// is the scalar offset and the lane's column the vector offset, so no
// per-load address arithmetic runs on the VALU. Reads past `bytes` return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t image_rsrc(const float4* base, long long bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float4*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ float4 image_load(__amdgpu_buffer_rsrc_t r, int lane_bytes,
                                             int row_bytes) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, lane_bytes,
                                                                           row_bytes, 0));
}

// Streams operand rows [r0, r0 + RC) of one image column (RC a multiple of 8)
// through a double buffer of four rows, calling f(operand, row) for each row.
// r0 must be wave-uniform. The prefetch past the chunk reads the next chunk's
// rows, or zeros past the image.
// As stream_rows, calling f4(operands, row) once per group of four rows.
template <class F4>
__device__ __forceinline__ void stream_rows4(__amdgpu_buffer_rsrc_t rs, int lane_bytes, int r0,
                                             int RC, int Hp, F4&& f4) {
  const int rowb = Hp * 16;
  const int sb = r0 * rowb;
  float4 pa[4], pb[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) pa[q] = image_load(rs, lane_bytes, sb + q * rowb);
  for (int rr = 0; rr < RC; rr += 8) {
    const int s0 = sb + rr * rowb;
#pragma unroll
    for (int q = 0; q < 4; ++q) pb[q] = image_load(rs, lane_bytes, s0 + (4 + q) * rowb);
    __builtin_amdgcn_sched_barrier(0);
    f4(pa, r0 + rr);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < 4; ++q) pa[q] = image_load(rs, lane_bytes, s0 + (8 + q) * rowb);
    __builtin_amdgcn_sched_barrier(0);
    f4(pb, r0 + rr + 4);
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <class F>
__device__ __forceinline__ void stream_rows(__amdgpu_buffer_rsrc_t rs, int lane_bytes, int r0,
                                            int RC, int Hp, F&& f) {
  const int rowb = Hp * 16;
  const int sb = r0 * rowb;
  float4 pa[4], pb[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) pa[q] = image_load(rs, lane_bytes, sb + q * rowb);
  for (int rr = 0; rr < RC; rr += 8) {
    const int s0 = sb + rr * rowb;
#pragma unroll
    for (int q = 0; q < 4; ++q) pb[q] = image_load(rs, lane_bytes, s0 + (4 + q) * rowb);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < 4; ++q) f(pa[q], r0 + rr + q);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < 4; ++q) pa[q] = image_load(rs, lane_bytes, s0 + (8 + q) * rowb);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < 4; ++q) f(pb[q], r0 + rr + 4 + q);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ---------------------------------------------------------------------------
// Compacted image columns (one wave per column). op(r, v, act) gives row r's
// operand and whether it can contribute; a ballot over each 64 rows gives the
// active rows their entry numbers in ascending row order. With nch chunks,
// entry e goes to chunk e % nch, slot e / nch, so a dense column gives every
// chunk the rows ks, ks + nch, ... and all lanes of a chunk the same row per
// slot. Slots past the column's count get zero operands and row 0. The image
// has nrows rows (slots of all chunks) of `stride` columns.
// ---------------------------------------------------------------------------
template <class Op>
__device__ __forceinline__ void compact_column(int col, int nrows, int stride, int nch, int lane,
                                               float4* cimg, int* cidx, int* ccnt, Op op) {
  const int sc = nrows / nch;
  auto at = [&](int e) { return (long long)((e % nch) * sc + e / nch) * stride + col; };
  int n = 0;
  for (int r0 = 0; r0 < nrows; r0 += 64) {
    const int r = r0 + lane;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    bool act = false;
    op(r, v, act);
    const unsigned long long m = __ballot(act);
    if (act) {
      const long long a = at(n + __popcll(m & ((1ULL << lane) - 1ULL)));
      cimg[a] = v;
      cidx[a] = r;
    }
    n += __popcll(m);
  }
  for (int e = n + lane; e < nrows; e += 64) {
    const long long a = at(e);
    cimg[a] = make_float4(0.f, 0.f, 0.f, 0.f);
    cidx[a] = 0;
  }
  if (lane == 0) ccnt[col] = n;
}

// Compacted columns a prep launch builds: Hp forward columns when cF is set,
// then Hp chain columns when the chain image is built and cB is set.
__host__ __device__ inline int cmp_columns(const Prepped& pp, int Hp, int Dp, bool fwd, bool bwd,
                                            bool sens) {
  return ((fwd && pp.cF != nullptr) ? Hp : 0) + ((bwd && pp.cB != nullptr) ? Hp : 0) +
         ((sens && pp.sF != nullptr) ? (pp.sFfull ? Hp : (Dp / 64) * Hp) : 0);
}

// Compacted sensory forward column (one wave per 64-input chunk c and neuron
// h): the chunk's inputs whose sensory weight for h is nonzero, with the
// forward operands op(d) gives.
template <class Op>
__device__ __forceinline__ void compact_sens_column(const Prepped& pp, int col, int Hp, int D,
                                                    int H, int lane, Op op) {
  if (pp.sFfull) {
    // one list per neuron h = col over all of D (Dp rows)
    const int Dp = (D + 63) & ~63;
    compact_column(col, Dp, Hp, 1, lane, pp.sF, pp.sFi, pp.sFn, [&](int d, float4& v, bool& act) {
      if (d < D && col < H) {
        v = op((long long)d * H + col);
        act = v.w != 0.f;
      }
    });
    return;
  }
  const int c = col / Hp, h = col - c * Hp;
  const long long cb = (long long)c * 64 * Hp;
  compact_column(h, 64, Hp, 1, lane, pp.sF + cb, pp.sFi + cb, pp.sFn + (long long)c * Hp,
                 [&](int dl, float4& v, bool& act) {
                   const int d = c * 64 + dl;
                   if (d < D && h < H) {
                     v = op((long long)d * H + h);
                     act = v.w != 0.f;
                   }
                 });
}

// ---------------------------------------------------------------------------
// Parameter images (one launch, flat index space over three segments).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prep_kernel(RawParams rp, Prepped pp, int H, int D,
                                                   int Hp, int Dp, int bwd, int segs,
                                                   int nflat_blocks, int nchf, int nchb) {
  if ((int)blockIdx.x >= nflat_blocks) {
    // Compacted columns, one per wave (forward, then chain).
    const int lane = threadIdx.x & 63;
    int col = ((int)blockIdx.x - nflat_blocks) * 4 + (int)(threadIdx.x >> 6);
    const bool fwd_c = (segs & kPrepRec) && pp.cF != nullptr;
    auto operand = [&](int i, int j, float4& v) {
      const long long e = (long long)i * H + j;
      const float S = rp.sigma[e], M = rp.mu[e];
      v = make_float4(-S * kLog2e, S * M * kLog2e, rp.w_erev[e], rp.w_pos[e]);
    };
    if (fwd_c) {
      if (col < Hp) {
        const int j = col;
        compact_column(j, Hp, Hp, nchf, lane, pp.cF, pp.cFi, pp.cFn, [&](int i, float4& v, bool& act) {
          if (i < H && j < H) {
            operand(i, j, v);
            act = v.z != 0.f || v.w != 0.f;
          }
        });
        return;
      }
      col -= Hp;
    }
    if (bwd && (segs & kPrepRec) && pp.cB != nullptr) {
      if (col < Hp) {
        // The fused chain (bwd == 1) keeps every real synapse (it also forms
        // the parameter gradients); the unfused one (bwd == 2, folded
        // operands) only those that add to dL/dv.
        const int i = col;
        compact_column(i, Hp, Hp, nchb, lane, pp.cB, pp.cBi, pp.cBn, [&](int j, float4& v, bool& act) {
          if (i < H && j < H) {
            operand(i, j, v);
            if (bwd == 2) {
              v = make_float4(v.x, v.y, v.x * v.z, v.x * v.w);
              act = v.z != 0.f || v.w != 0.f;
            } else {
              act = true;
            }
          }
        });
        return;
      }
      col -= Hp;
    }
    if ((segs & kPrepSens) && pp.sF != nullptr && col < (pp.sFfull ? Hp : (Dp / 64) * Hp)) {
      compact_sens_column(pp, col, Hp, D, H, lane, [&](long long e) {
        const float Ss = rp.s_sigma[e], Ms = rp.s_mu[e], Ws = rp.s_wpos[e];
        return make_float4(-Ss * kLog2e, Ss * Ms * kLog2e, Ws * rp.s_erev[e], Ws);
      });
    }
    return;
  }
  long long tid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long nrec = (segs & kPrepRec) ? (long long)Hp * Hp : 0;
  const long long nsens = (segs & kPrepSens) ? (long long)Dp * Hp : 0;
  if (tid < nrec) {
    const int i = (int)(tid / Hp), j = (int)(tid - (long long)i * Hp);
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (i < H && j < H) {
      const long long e = (long long)i * H + j;
      const float S = rp.sigma[e], M = rp.mu[e];
      v = make_float4(-S * kLog2e, S * M * kLog2e, rp.w_erev[e], rp.w_pos[e]);
    }
    pp.recF[tid] = v;
    // bwd == 2: the chain's image carries S'*WE and S'*WP (folded; see
    // bwd_synapse_folded); bwd == 1 keeps WE, WP for the fused chain.
    if (bwd) pp.recB[(long long)j * Hp + i] = bwd == 2 ? make_float4(v.x, v.y, v.x * v.z, v.x * v.w) : v;
    return;
  }
  tid -= nrec;
  if (tid < nsens) {
    const int d = (int)(tid / Hp), h = (int)(tid - (long long)d * Hp);
    float4 f = make_float4(0.f, 0.f, 0.f, 0.f), g = f;
    if (d < D && h < H) {
      const long long e = (long long)d * H + h;
      const float Ss = rp.s_sigma[e], Ms = rp.s_mu[e], Es = rp.s_erev[e], Ws = rp.s_wpos[e];
      f = make_float4(-Ss * kLog2e, Ss * Ms * kLog2e, Ws * Es, Ws);
      g = make_float4(-Ss * kLog2e, Ss * Ms * kLog2e, Es, Ws * Ss);
    }
    if (bwd)
      pp.sensB[(long long)h * Dp + d] = g;
    else if (pp.sF == nullptr)  // the compacted image replaces the dense one
      pp.sensF[tid] = f;
    return;
  }
  tid -= nsens;
  if ((segs & kPrepNeuron) && tid < 3LL * Hp) {
    const int q = (int)(tid / Hp), j = (int)(tid - (long long)q * Hp);
    const float* src = q == 0 ? rp.cm : (q == 1 ? rp.gleak : rp.vleak);
    pp.neuron[tid] = j < H ? src[j] : 0.f;
  }
}

// ---------------------------------------------------------------------------
// Sensory forward for all (b,t) rows at once.
// Block 256 = 4 waves, lane -> h (64 neurons per workgroup). Each float4
// operand read from L2 is reused for RPW rows held in registers; x is staged
// through LDS 64 inputs at a time and read as a broadcast.
//   DS = 1: the 4 waves own 4 groups of RPW rows (4*RPW rows per workgroup)
//           and each walks all of D (large B*T: operands shared through L1);
//   DS = 4: the 4 waves split D into quarters over the same RPW rows and meet
//           in LDS (small B*T: 4x shorter dependent load chains per thread).
// grid (Hp/64, ceil(BT / rows_per_workgroup)).
// ---------------------------------------------------------------------------
template <int RPW, int DS>
__global__ __launch_bounds__(256) void sens_fwd_kernel(const float* __restrict__ x, Strides3 xs,
                                                       int T, int D, int BT, int Hp,
                                                       const float4* __restrict__ sensF,
                                                       float* __restrict__ sn,
                                                       float* __restrict__ sd) {
  constexpr int ROWS = (DS == 1 ? 4 : 1) * RPW;
  constexpr int XLD = ROWS + 4;  // padded staged row, 16-byte aligned
  __shared__ __align__(16) float xsh[64 * XLD];
  __shared__ float2 part[DS == 1 ? 1 : 3][RPW][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int h = blockIdx.x * 64 + lane;
  const int row0 = blockIdx.y * ROWS;
  const int rw = DS == 1 ? w * RPW : 0;  // first staged row of this wave
  float an[RPW], ad[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) an[r] = ad[r] = 0.f;

  // The x values of a 64-input chunk are loaded into registers one chunk
  // ahead, so the loads travel while the previous chunk is evaluated. Lane l
  // of wave w stages input d0 + l of rows w, w + 4, ...; the row bases are
  // wave-uniform and computed once.
  constexpr int NXF = (ROWS + 3) / 4;
  const int wu = __builtin_amdgcn_readfirstlane(w);
  const float* xrow[NXF];
#pragma unroll
  for (int i = 0; i < NXF; ++i) {
    const int r = wu + 4 * i, row = row0 + r;
    xrow[i] = nullptr;
    if (r < ROWS && row < BT) {
      const int b = row / T, t = row - b * T;
      xrow[i] = x + b * xs.b + t * xs.t;
    }
  }
  // The loads are unconditional (a lane past the rows or past D reads x[0],
  // and the stash writes 0 instead) so that none sits behind a branch and
  // each waits only for its own data.
  float xv[NXF];
  auto fetch = [&](int d0) {
    const int d = d0 + lane;
    const long long off = (long long)d * xs.c;
#pragma unroll
    for (int i = 0; i < NXF; ++i) xv[i] = *((xrow[i] != nullptr && d < D) ? xrow[i] + off : x);
  };
  if (D > 0) fetch(0);
  for (int d0 = 0; d0 < D; d0 += 64) {
    const bool dok = d0 + lane < D;
#pragma unroll
    for (int i = 0; i < NXF; ++i)
      if (wu + 4 * i < ROWS)
        xsh[lane * XLD + wu + 4 * i] = (dok && xrow[i] != nullptr) ? xv[i] : 0.f;
    __syncthreads();
    fetch(d0 + 64);
    const float4* pcol = sensF + (long long)d0 * Hp + h;
    if constexpr (DS == 1) {
      // All 64 inputs of the chunk (rows past D are zero in the image and in
      // xsh, so they add exact zeros), operands loaded four at a time one
      // group ahead (the last group reloads itself).
      float4 pc[4], pn[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) pc[i] = pcol[(long long)i * Hp];
      for (int gq = 0; gq < 16; ++gq) {
        const int gn = gq < 15 ? gq + 1 : 15;
#pragma unroll
        for (int i = 0; i < 4; ++i) pn[i] = pcol[(long long)(gn * 4 + i) * Hp];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float* xr = xsh + (gq * 4 + i) * XLD + rw;
#pragma unroll
          for (int r = 0; r < RPW; ++r) {
            const float a = gate(fmaf(pc[i].x, xr[r], pc[i].y));
            an[r] = fmaf(a, pc[i].z, an[r]);
            ad[r] = fmaf(a, pc[i].w, ad[r]);
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) pc[i] = pn[i];
      }
    } else {
      // The wave's 64/DS inputs of the chunk: all operand loads in flight at
      // once. Rows past D are zero in the image and zero in xsh, so they add
      // exact zeros.
      constexpr int QD = 64 / DS;
      const int dlo = w * QD;
      float4 pq[QD];
#pragma unroll
      for (int i = 0; i < QD; ++i) pq[i] = pcol[(long long)(dlo + i) * Hp];
#pragma unroll
      for (int i = 0; i < QD; ++i) {
        const float* xr = xsh + (dlo + i) * XLD + rw;
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          const float a = gate(fmaf(pq[i].x, xr[r], pq[i].y));
          an[r] = fmaf(a, pq[i].z, an[r]);
          ad[r] = fmaf(a, pq[i].w, ad[r]);
        }
      }
    }
    __syncthreads();
  }
  if constexpr (DS != 1) {
    if (w > 0) {
#pragma unroll
      for (int r = 0; r < RPW; ++r) part[w - 1][r][lane] = make_float2(an[r], ad[r]);
    }
    __syncthreads();
    if (w > 0) return;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const float2 v = part[q][r][lane];
        an[r] += v.x;
        ad[r] += v.y;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int row = row0 + rw + r;
    if (row < BT) {
      sn[(long long)row * Hp + h] = an[r];
      sd[(long long)row * Hp + h] = ad[r];
    }
  }
}

// ---------------------------------------------------------------------------
// Sensory forward over the compacted image (module path): sens_fwd_kernel's
// layout and staging (lane -> neuron h, 64-input chunks of the rows staged in
// LDS one chunk ahead), but in each chunk a lane walks only the inputs whose
// weight is nonzero (sF, sFi: [chunk][64 slots][Hp], ascending input within
// the chunk; sFn: [chunk][Hp] counts), so a wave runs as many slots as its
// fullest neuron has entries in the chunk instead of 64, and each lane reads
// its slot's input at its own LDS address. With DS = 4 the four waves take
// quarters of each chunk's slots. Slots past a count hold zero operands
// (input 0) and add zero.
// ---------------------------------------------------------------------------
// LN (DS = 1, D <= 64): x is the raw input, and each wave applies the
// module's LayerNorm + affine to its rows of the staged chunk in place, with
// ln_row's arithmetic, so the sums are those over the prep launch's rows.
template <int RPW, int DS, bool LN = false>
__global__ __launch_bounds__(256) void sens_fwd_cmp_kernel(const float* __restrict__ x, Strides3 xs,
                                                           int T, int D, int BT, int Hp,
                                                           const float4* __restrict__ sF,
                                                           const int* __restrict__ sFi,
                                                           const int* __restrict__ sFn,
                                                           float* __restrict__ sn,
                                                           float* __restrict__ sd, LnAff la) {
  static_assert(!LN || DS == 1, "the row normalisation runs in the row-group layout");
  constexpr int ROWS = (DS == 1 ? 4 : 1) * RPW;
  constexpr int XLD = ROWS + 4;  // padded staged row, 16-byte aligned
  __shared__ __align__(16) float xsh[64 * XLD];
  __shared__ float2 part[DS == 1 ? 1 : 3][RPW][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int h = blockIdx.x * 64 + lane;
  const int row0 = blockIdx.y * ROWS;
  const int rw = DS == 1 ? w * RPW : 0;
  float an[RPW], ad[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) an[r] = ad[r] = 0.f;
  // x staging as in sens_fwd_kernel: lane l of wave w loads input d0 + l of
  // rows w, w + 4, ... one chunk ahead
  constexpr int NXF = (ROWS + 3) / 4;
  const int wu = __builtin_amdgcn_readfirstlane(w);
  const float* xrow[NXF];
#pragma unroll
  for (int i = 0; i < NXF; ++i) {
    const int r = wu + 4 * i, row = row0 + r;
    xrow[i] = nullptr;
    if (r < ROWS && row < BT) {
      const int b = row / T, t = row - b * T;
      xrow[i] = x + b * xs.b + t * xs.t;
    }
  }
  float xv[NXF];
  auto fetch = [&](int d0) {
    const int d = d0 + lane;
    const long long off = (long long)d * xs.c;
#pragma unroll
    for (int i = 0; i < NXF; ++i) xv[i] = *((xrow[i] != nullptr && d < D) ? xrow[i] + off : x);
  };
  if (D > 0) fetch(0);
  for (int d0 = 0; d0 < D; d0 += 64) {
    const bool dok = d0 + lane < D;
#pragma unroll
    for (int i = 0; i < NXF; ++i)
      if (wu + 4 * i < ROWS)
        xsh[lane * XLD + wu + 4 * i] = (dok && xrow[i] != nullptr) ? xv[i] : 0.f;
    const long long cb = (long long)(d0 >> 6) * 64 * Hp;
    // this chunk's slots of the wave, in groups of four
    const int nsw = (wave_max(sFn[(d0 >> 6) * Hp + h]) + 3) & ~3;
    int s0 = 0, s1 = nsw;
    if constexpr (DS != 1) {
      const int q = ((nsw + 4 * DS - 1) / (4 * DS)) * 4;
      s0 = min(nsw, w * q);
      s1 = min(nsw, s0 + q);
    }
    __syncthreads();
    fetch(d0 + 64);
    if constexpr (LN) {
      // the only chunk (D <= 64): this wave's rows, lane = input
      const bool in = lane < D;
      const float lw = in ? la.ln_w[lane] : 0.f, lb = in ? la.ln_b[lane] : 0.f;
      const float iw = in ? la.input_w[lane] : 0.f, ib = in ? la.input_b[lane] : 0.f;
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        float* px = xsh + lane * XLD + rw + r;
        const float v = *px;
        const float mean = wave_sum(v) / (float)D;
        const float dv = in ? v - mean : 0.f;
        const float rstd = 1.0f / sqrtf(wave_sum(fmaf(dv, dv, 0.f)) / (float)D + la.eps);
        const float xn = (v - mean) * rstd * lw + lb;
        *px = in ? xn * iw + ib : 0.f;
      }
    }
    if (s0 < s1) {
      const float4* pcol = sF + cb + h;
      const int* icol = sFi + cb + h;
      float4 pc[4], pn[4];
      int dc[4], dn[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pc[i] = pcol[(long long)(s0 + i) * Hp];
        dc[i] = icol[(long long)(s0 + i) * Hp];
      }
      for (int s = s0; s < s1; s += 4) {
        // the next group's operands travel while this one is evaluated (the
        // last group reloads itself)
        const int sn4 = s + 4 < s1 ? s + 4 : s;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pn[i] = pcol[(long long)(sn4 + i) * Hp];
          dn[i] = icol[(long long)(sn4 + i) * Hp];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float* xr = xsh + dc[i] * XLD + rw;
          float xq[RPW];
          if constexpr (RPW % 4 == 0) {
#pragma unroll
            for (int r = 0; r < RPW; r += 4) {
              const float4 q4 = *reinterpret_cast<const float4*>(xr + r);
              xq[r] = q4.x;
              xq[r + 1] = q4.y;
              xq[r + 2] = q4.z;
              xq[r + 3] = q4.w;
            }
          } else {
#pragma unroll
            for (int r = 0; r < RPW; ++r) xq[r] = xr[r];
          }
#pragma unroll
          for (int r = 0; r < RPW; ++r) {
            const float a = gate(fmaf(pc[i].x, xq[r], pc[i].y));
            an[r] = fmaf(a, pc[i].z, an[r]);
            ad[r] = fmaf(a, pc[i].w, ad[r]);
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pc[i] = pn[i];
          dc[i] = dn[i];
        }
      }
    }
    __syncthreads();
  }
  if constexpr (DS != 1) {
    if (w > 0) {
#pragma unroll
      for (int r = 0; r < RPW; ++r) part[w - 1][r][lane] = make_float2(an[r], ad[r]);
    }
    __syncthreads();
    if (w > 0) return;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const float2 v = part[q][r][lane];
        an[r] += v.x;
        ad[r] += v.y;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int row = row0 + rw + r;
    if (row < BT) {
      sn[(long long)row * Hp + h] = an[r];
      sd[(long long)row * Hp + h] = ad[r];
    }
  }
}

// ---------------------------------------------------------------------------
// Persistent forward unfold loop.
// One workgroup owns NB batch rows for all T*U unfolds. blockDim = Hp*KS:
// thread (o = tid % Hp, ks = tid / Hp) accumulates the partial n_o, q_o over
// presynaptic i in [ks*RC, ks*RC + RC) for every row; partials meet in LDS
// and thread (o, ks) finishes rows b = ks, ks+KS, ... of column o.
// RCP > 0: the RC = RCP float4 operands of the thread live in registers.
// ---------------------------------------------------------------------------
struct FwdK {
  const float4* recF;
  const float* neuron;
  const float* sn;
  const float* sd;
  const float* state0;
  float* out;
  float* hfin;
  float* vsave;
  float* densave;
  int B, T, H, Hp, U, KS, RC;
  float eps;
  // Compacted forward image (the single-row forward): operands, row indices,
  // column counts.
  const float4* cimg;
  const int* cidx;
  const int* ccnt;
};

template <int NB>
__device__ __forceinline__ void fwd_synapse(const float4 p, const float* vs, int Hp, int r,
                                            float* na, float* qa) {
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const float a = gate(fmaf(p.x, vs[b * Hp + r], p.y));
    na[b] = fmaf(a, p.z, na[b]);
    qa[b] = fmaf(a, p.w, qa[b]);
  }
}

// G register-resident synapses (rows r .. r+G-1) for every row of the tile,
// with the G*NB gates evaluated in phases (arguments, exponentials,
// reciprocals) before the sums, which keep fwd_synapse's order.
// Synapses per phased group: fewer at 8+ rows, whose gates already fill the
// registers; none at one row (measured slower there: C2 forward +1%).
template <int NB>
constexpr int kFwdGroup = NB == 1 ? 1 : (NB >= 8 ? 2 : 4);

template <int NB, int G>
__device__ __forceinline__ void fwd_synapses(const float4* p, const float* vs, int Hp, int r,
                                             float* na, float* qa) {
  float z[G][NB];
#pragma unroll
  for (int i = 0; i < G; ++i)
#pragma unroll
    for (int b = 0; b < NB; ++b) z[i][b] = fmaf(p[i].x, vs[b * Hp + r + i], p[i].y);
#pragma unroll
  for (int i = 0; i < G; ++i)
#pragma unroll
    for (int b = 0; b < NB; ++b) z[i][b] = 1.0f + __builtin_amdgcn_exp2f(z[i][b]);
#pragma unroll
  for (int i = 0; i < G; ++i)
#pragma unroll
    for (int b = 0; b < NB; ++b) z[i][b] = __builtin_amdgcn_rcpf(z[i][b]);
#pragma unroll
  for (int i = 0; i < G; ++i)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      na[b] = fmaf(z[i][b], p[i].z, na[b]);
      qa[b] = fmaf(z[i][b], p[i].w, qa[b]);
    }
}

// The NB state values of LDS row r in the compacted kernels' [Hp][NB] layout.
template <int NB>
__device__ __forceinline__ void lds_rows(const float* base, int byte_off, float (&v)[NB]) {
  const char* at = reinterpret_cast<const char*>(base) + byte_off;
  if constexpr (NB % 4 == 0) {
#pragma unroll
    for (int q = 0; q < NB; q += 4) {
      const float4 w = *reinterpret_cast<const float4*>(at + q * 4);
      v[q] = w.x;
      v[q + 1] = w.y;
      v[q + 2] = w.z;
      v[q + 3] = w.w;
    }
  } else if constexpr (NB == 2) {
    const float2 w = *reinterpret_cast<const float2*>(at);
    v[0] = w.x;
    v[1] = w.y;
  } else {
    v[0] = *reinterpret_cast<const float*>(at);
  }
}

// Two compacted forward synapses (slots with LDS row offsets o0, o1) for every
// row of the tile, gates in phases as in fwd_synapses.
template <int NB>
__device__ __forceinline__ void fwd_synapses_cmp(const float4* p, const float* vs, int o0, int o1,
                                                 float* na, float* qa) {
  float z[2][NB];
  lds_rows<NB>(vs, o0, z[0]);
  lds_rows<NB>(vs, o1, z[1]);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int b = 0; b < NB; ++b) z[i][b] = fmaf(p[i].x, z[i][b], p[i].y);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int b = 0; b < NB; ++b) z[i][b] = 1.0f + __builtin_amdgcn_exp2f(z[i][b]);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int b = 0; b < NB; ++b) z[i][b] = __builtin_amdgcn_rcpf(z[i][b]);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      na[b] = fmaf(z[i][b], p[i].z, na[b]);
      qa[b] = fmaf(z[i][b], p[i].w, qa[b]);
    }
}

// With register-resident operands (RCP > 0) the kernel reads the compacted
// image (CMP): thread (o, ks) holds the entries ks, ks + KS, ... of column o,
// the wave runs as many slots as its fullest lane (wave-uniform branches
// around unused pairs), the state sits in LDS as [Hp][NB] so that a slot's NB
// values are one read at a per-lane row, and the slot row offsets stay in
// registers (no table read before a slot pair's state reads).
template <int NB, int RCP>
__global__ __launch_bounds__(ode_max_threads(NB)) void ode_fwd_kernel(FwdK k) {
  constexpr int MO = ode_owned_rows(NB);
  constexpr bool CMP = RCP > 0;
  extern __shared__ float4 lds4[];
  const int Hp = k.Hp, H = k.H, KS = k.KS, B = k.B, T = k.T, U = k.U;
  const int RC = RCP > 0 ? RCP : k.RC;
  float* vs = reinterpret_cast<float*>(lds4);            // [NB][Hp] ([Hp][NB] with CMP)
  float2* red = reinterpret_cast<float2*>(vs + NB * Hp);  // [KS][NB][Hp]
  // CMP: the compacted kernels' slot-table space [RCP/4][threads] (int4); this
  // kernel keeps its offsets in registers and uses only the space after it
  int4* slot_tab = reinterpret_cast<int4*>(red + KS * NB * Hp);
  auto vat = [&](int b, int j) { return CMP ? j * NB + b : b * Hp + j; };
  const int tid = threadIdx.x, nthr = blockDim.x;
  // Hp is a multiple of 64, so ks is uniform across each wave.
  const int ks = __builtin_amdgcn_readfirstlane(tid / Hp), o = tid - ks * Hp;
  const __amdgpu_buffer_rsrc_t rsF = image_rsrc(k.recF, (long long)Hp * Hp * 16);
  const int b0 = blockIdx.x * NB;
  const int r0 = ks * RC;

  const float C = k.neuron[o], G = k.neuron[Hp + o], L = k.neuron[2 * Hp + o];
  const float GL = G * L, CG = C + G;

  float4 preg[RCP > 0 ? RCP : 1];
  int ix[RCP > 0 ? RCP : 1];  // CMP: slot row offsets, in registers
  int nslot = 0;  // CMP: slots the wave runs
  // Synapse lane of this thread: (chunk sks, column so). With CMP the lanes
  // are dealt in balanced order (balanced_lane); the owner role below keeps
  // (ks, o).
  int sks = ks, so = o;
  if constexpr (CMP) {
    int* perm = reinterpret_cast<int*>(slot_tab + (RCP / 4) * nthr);  // [threads]
    const int cnt0 = k.ccnt[o];
    const int lane_id = balanced_lane(cnt0 > ks ? (cnt0 - 1 - ks) / KS + 1 : 0, tid, nthr,
                                      perm, perm + nthr);
    sks = lane_id / Hp;
    so = lane_id - sks * Hp;
    const int cnt = k.ccnt[so];
    nslot = wave_max(cnt > sks ? (cnt - 1 - sks) / KS + 1 : 0);
#pragma unroll
    for (int rr = 0; rr < RCP; ++rr) {
      const long long a = (long long)(sks * RCP + rr) * Hp + so;
      preg[rr] = k.cimg[a];
      ix[rr] = k.cidx[a] * NB * 4;
    }
  }

  for (int e = tid; e < NB * Hp; e += blockDim.x) {
    const int b = e / Hp, j = e - b * Hp;
    vs[vat(b, j)] = (k.state0 != nullptr && b0 + b < B && j < H)
                        ? k.state0[(long long)(b0 + b) * H + j]
                        : 0.f;
  }
  lds_barrier();

  // Sensory sums of step t are requested one step ahead (software pipeline).
  float snr[MO], sdr[MO], snn[MO], sdn[MO];
  auto load_sens = [&](int t, float (&sn_)[MO], float (&sd_)[MO]) {
#pragma unroll
    for (int m = 0; m < MO; ++m) {
      const int b = ks + m * KS;
      sn_[m] = sd_[m] = 0.f;
      if (b < NB && b0 + b < B) {
        const long long e = ((long long)(b0 + b) * T + t) * Hp + o;
        sn_[m] = k.sn[e];
        sd_[m] = k.sd[e];
      }
    }
  };
  if (T > 0) load_sens(0, snr, sdr);
  for (int t = 0; t < T; ++t) {
    if (t + 1 < T) load_sens(t + 1, snn, sdn);
    for (int u = 0; u < U; ++u) {
      float na[NB], qa[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) na[b] = qa[b] = 0.f;
      if constexpr (CMP) {
        // Wave-uniform slot count: the skipped pairs branch around.
#pragma unroll
        for (int q = 0; q < RCP / 4; ++q) {
          if (4 * q < nslot) {
            fwd_synapses_cmp<NB>(preg + 4 * q, vs, ix[4 * q], ix[4 * q + 1], na, qa);
            if (4 * q + 2 < nslot)
              fwd_synapses_cmp<NB>(preg + 4 * q + 2, vs, ix[4 * q + 2], ix[4 * q + 3], na, qa);
          }
        }
      } else {
        // Operands stream from L2, the next four requested while the current
        // four are evaluated.
        if constexpr (kFwdGroup<NB> == 4) {
          stream_rows4(rsF, o * 16, r0, RC, Hp, [&](const float4* p, int r) {
            fwd_synapses<NB, 4>(p, vs, Hp, r, na, qa);
          });
        } else {
          stream_rows(rsF, o * 16, r0, RC, Hp,
                      [&](const float4 p, int r) { fwd_synapse<NB>(p, vs, Hp, r, na, qa); });
        }
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) red[(sks * NB + b) * Hp + so] = make_float2(na[b], qa[b]);
      lds_barrier();
#pragma unroll
      for (int m = 0; m < MO; ++m) {
        const int b = ks + m * KS;
        if (b < NB) {
          const float2 nq = NB <= 2 ? ks_sum_1r(red + b * Hp + o, NB * Hp, KS)
                                    : ks_sum(red + b * Hp + o, NB * Hp, KS);
          const float n = nq.x, q = nq.y;
          const float vold = vs[vat(b, o)];
          const float den = CG + (q + sdr[m]) + k.eps;
          const float num = C * vold + GL + (n + snr[m]);
          // 1/den from v_rcp_f32 (within 1 ulp): the new state is num/den to
          // about 2 ulp, and the reciprocal is what the backward multiplies
          // by, so it is saved in place of den.
          const float rden = __builtin_amdgcn_rcpf(den);
          const float vnew = o < H ? num * rden : 0.f;
          const bool live = b0 + b < B;
          if (k.vsave != nullptr && live) {
            const long long e = ((long long)(t * U + u) * B + b0 + b) * Hp + o;
            k.vsave[e] = vold;
            k.densave[e] = rden;
          }
          vs[vat(b, o)] = vnew;
          if (u == U - 1 && live && o < H) k.out[((long long)(b0 + b) * T + t) * H + o] = vnew;
        }
      }
      lds_barrier();
    }
    if (t + 1 < T) {
#pragma unroll
      for (int m = 0; m < MO; ++m) {
        snr[m] = snn[m];
        sdr[m] = sdn[m];
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MO; ++m) {
    const int b = ks + m * KS;
    if (b < NB && b0 + b < B) {
      const float v = vs[vat(b, o)];
      if (o < H) k.hfin[(long long)(b0 + b) * H + o] = v;
      if (k.vsave != nullptr) k.vsave[((long long)T * U * B + b0 + b) * Hp + o] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Persistent reverse-time chain: dL/dv for every unfold.
// Same thread layout as the forward with the roles swapped: o is the
// presynaptic neuron i whose gradient is being formed and the thread loops
// over postsynaptic j in [ks*RC, ks*RC + RC), reading the transposed image
// recB[j][i]. alpha_j, beta_j of each unfold are broadcast through LDS.
// ---------------------------------------------------------------------------
struct BwdK {
  const float4* recB;
  const float* neuron;
  const float* vsave;
  const float* densave;
  const float* gout;
  Strides3 gs;
  const float* ghfin;
  float2* absave;   // alpha/beta per unfold, for rec_grad_kernel (unused when fused)
  float* dsn;
  float* dsd;
  float* npart;
  float* gstate;
  float* rpart;     // per-workgroup recurrent partials [grid][4][Hp][Hp] (fused only)
  int B, T, H, Hp, U, KS, RC;
  // Compacted chain image (the single-row fused chain): operands, row
  // indices, column counts.
  const float4* cimg;
  const int* cidx;
  const int* ccnt;
  // Exchange words with tag 1: the fused row backward (Hp = 64) sends dL/dsn,
  // dL/dsd of each (row, step) as [B*T][2][64] words instead of into dsn /
  // dsd; the Hp = 128 chain with recurrent-gradient companions sends each
  // unfold's alpha/beta as [B][T*U][2][128] words instead of into absave.
  unsigned long long* rbw;
};

// The recurrent-gradient companions of the Hp = 128 chain: the forward image
// {S', c', WE, WP} and their wait budget (recF null: no companions).
struct RecC {
  const float4* recF;
  long long spin;
  int* status;  // the status word, after all words
  // Sensory companions (sensB null: none): each step's dL/dsn, dL/dsd as
  // words [B][T][2][128] from the chain (instead of dsn / dsd), then the
  // words [B][T][128] that hand the first half's dL/dxa to the second; the
  // rows xa, the backward sensory image, and their outputs: one sensory
  // partial per row [B][4][Hp][Dp]; the LayerNorm backward's dL/dx and one
  // column partial per row [B][4][Dp].
  unsigned long long* sw;
  const float* xa;
  const float4* sensB;
  float* spart;
  LnBuf ln;
  const float* input_w;
  const float* ln_w;
  const float* ln_b;
  float* gx;
  float* lnpart;
  int D, Dp;
};

// One synapse (i = o, j = r) of the chain for every row of the tile. With
// FUSE the parameter-gradient sums of this synapse ride along in gacc:
// {sum alpha*a, sum beta*a, sum delta, sum delta*v_i}.
template <int NB, bool FUSE>
__device__ __forceinline__ void bwd_synapse(const float4 p, const float2* ab, int Hp, int r,
                                            const float* vi, float* acc, float4& gacc) {
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const float2 c = ab[b * Hp + r];
    const float a = gate(fmaf(p.x, vi[b], p.y));
    const float a2 = fmaf(-a, a, a);
    const float dl = fmaf(c.x, p.z, c.y * p.w) * a2;
    acc[b] = fmaf(dl, p.x, acc[b]);
    if constexpr (FUSE) {
      gacc.x = fmaf(c.x, a, gacc.x);
      gacc.y = fmaf(c.y, a, gacc.y);
      gacc.z += dl;
      gacc.w = fmaf(dl, vi[b], gacc.w);
    }
  }
}

// Chain synapse with the folded image {S', c', S'*WE, S'*WP}: the S' factor of
// dL/dv_i rides in the image, so each row costs one multiply less.
template <int NB>
__device__ __forceinline__ void bwd_synapse_folded(const float4 p, const float2* ab, int Hp, int r,
                                                   const float* vi, float* acc) {
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const float2 c = ab[b * Hp + r];
    const float a = gate(fmaf(p.x, vi[b], p.y));
    const float a2 = fmaf(-a, a, a);
    acc[b] = fmaf(fmaf(c.x, p.z, c.y * p.w), a2, acc[b]);
  }
}

// bwd_synapse_folded for a compacted slot: the NB alpha/beta pairs of its row
// from the [Hp][NB] float2 layout at byte offset `off`.
template <int NB>
__device__ __forceinline__ void bwd_synapse_folded_cmp(const float4 p, const float2* ab, int off,
                                                       const float* vi, float* acc) {
  float2 c[NB];
  const char* at = reinterpret_cast<const char*>(ab) + off;
  if constexpr (NB % 2 == 0) {
#pragma unroll
    for (int b = 0; b < NB; b += 2) {
      const float4 w = *reinterpret_cast<const float4*>(at + b * 8);
      c[b] = make_float2(w.x, w.y);
      c[b + 1] = make_float2(w.z, w.w);
    }
  } else {
    c[0] = *reinterpret_cast<const float2*>(at);
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const float a = gate(fmaf(p.x, vi[b], p.y));
    const float a2 = fmaf(-a, a, a);
    acc[b] = fmaf(fmaf(c[b].x, p.z, c[b].y * p.w), a2, acc[b]);
  }
}

// Operands of unfold n for the synapse phase (all rows, column o) and for the
// rows this thread finishes (1/den, v^k, v^{k+1}).
template <int NB, int MO>
__device__ __forceinline__ void bwd_load_unfold(const BwdK& k, long long n, int b0, int ks, int o,
                                                float (&vi)[NB], float (&den)[MO],
                                                float (&vk)[MO], float (&vk1)[MO]) {
  const long long BHp = (long long)k.B * k.Hp;
#pragma unroll
  for (int b = 0; b < NB; ++b) vi[b] = b0 + b < k.B ? k.vsave[(n * k.B + b0 + b) * k.Hp + o] : 0.f;
#pragma unroll
  for (int m = 0; m < MO; ++m) {
    const int b = ks + m * k.KS;
    den[m] = 1.f;
    vk[m] = vk1[m] = 0.f;
    if (b < NB && b0 + b < k.B && o < k.H) {
      const long long e = (n * k.B + b0 + b) * k.Hp + o;
      den[m] = k.densave[e];
      vk[m] = k.vsave[e];
      vk1[m] = k.vsave[e + BHp];
    }
  }
}

template <int NB, int MO>
__device__ __forceinline__ void bwd_load_gout(const BwdK& k, int t, int b0, int ks, int o,
                                              float (&go)[MO]) {
#pragma unroll
  for (int m = 0; m < MO; ++m) {
    const int b = ks + m * k.KS;
    go[m] = 0.f;
    if (b < NB && b0 + b < k.B && o < k.H) go[m] = k.gout[(b0 + b) * k.gs.b + t * k.gs.t + o * k.gs.c];
  }
}

// FUSE (register-resident operands only): each operand also carries its
// gradient accumulators, which removes the separate parameter-gradient pass
// and its second gate evaluation.
// Unfused with register-resident operands (CMP: RCP > 0, !FUSE) the kernel
// reads the compacted folded image: only synapses with a nonzero weight add
// to dL/dv (the parameter gradients come from rec_grad_kernel over every
// synapse). Thread (o, ks) holds the entries ks, ks + KS, ... of column o,
// alpha/beta sit in LDS as [Hp][NB], and the slot row offsets come from an
// LDS table [RCP/4][threads] of int4.
template <int NB, int RCP, bool FUSE>
__global__ __launch_bounds__(ode_max_threads(NB)) void ode_bwd_kernel(BwdK k) {
  static_assert(!FUSE || RCP > 0, "fused gradients need register-resident operands");
  constexpr int MO = ode_owned_rows(NB);
  constexpr bool CMP = !FUSE && RCP > 0;
  extern __shared__ float4 lds4[];
  const int Hp = k.Hp, H = k.H, KS = k.KS, B = k.B, T = k.T, U = k.U;
  const int RC = RCP > 0 ? RCP : k.RC;
  float2* ab = reinterpret_cast<float2*>(lds4);        // [NB][Hp] ([Hp][NB] with CMP)
  float* red = reinterpret_cast<float*>(ab + NB * Hp);  // [KS][NB][Hp]
  int4* slot_tab = reinterpret_cast<int4*>(red + KS * NB * Hp);  // CMP: [RCP/4][threads]
  auto abat = [&](int b, int col) { return CMP ? col * NB + b : b * Hp + col; };
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int ks = __builtin_amdgcn_readfirstlane(tid / Hp), o = tid - ks * Hp;
  const __amdgpu_buffer_rsrc_t rsB = image_rsrc(k.recB, (long long)Hp * Hp * 16);
  const int b0 = blockIdx.x * NB;
  const int r0 = ks * RC;
  const float C = k.neuron[o];

  float4 preg[RCP > 0 ? RCP : 1];
  float4 gacc[FUSE ? RCP : 1];
  int nslot = 0;  // CMP: slots the wave runs
  if constexpr (CMP) {
    const int cnt = k.ccnt[o];
    nslot = wave_max(cnt > ks ? (cnt - 1 - ks) / KS + 1 : 0);
    int ix[RCP];
#pragma unroll
    for (int rr = 0; rr < RCP; ++rr) {
      const long long a = (long long)(ks * RCP + rr) * Hp + o;
      preg[rr] = k.cimg[a];
      ix[rr] = k.cidx[a] * NB * 8;
    }
#pragma unroll
    for (int q = 0; q < RCP / 4; ++q)
      slot_tab[q * nthr + tid] = make_int4(ix[4 * q], ix[4 * q + 1], ix[4 * q + 2], ix[4 * q + 3]);
  } else if constexpr (RCP > 0) {
#pragma unroll
    for (int rr = 0; rr < RCP; ++rr) preg[rr] = k.recB[(long long)(r0 + rr) * Hp + o];
  }
  if constexpr (FUSE) {
#pragma unroll
    for (int rr = 0; rr < RCP; ++rr) gacc[rr] = make_float4(0.f, 0.f, 0.f, 0.f);
  }

  float g[MO], pC[MO], pGv[MO], pA[MO];
#pragma unroll
  for (int m = 0; m < MO; ++m) {
    const int b = ks + m * KS;
    g[m] = 0.f;
    pC[m] = pGv[m] = pA[m] = 0.f;
    if (k.ghfin != nullptr && b < NB && b0 + b < B && o < H) g[m] = k.ghfin[(long long)(b0 + b) * H + o];
  }
  if (T == 0) return;

  // Operands of the current unfold, software-pipelined one unfold ahead.
  float cvi[NB], cden[MO], cvk[MO], cvk1[MO];
  float nvi[NB], nden[MO], nvk[MO], nvk1[MO];
  float gcur[MO], gnext[MO];
#pragma unroll
  for (int m = 0; m < MO; ++m) gnext[m] = 0.f;
  bwd_load_unfold<NB, MO>(k, (long long)T * U - 1, b0, ks, o, cvi, cden, cvk, cvk1);
  bwd_load_gout<NB, MO>(k, T - 1, b0, ks, o, gcur);

  for (int t = T - 1; t >= 0; --t) {
    if (t > 0) bwd_load_gout<NB, MO>(k, t - 1, b0, ks, o, gnext);
    float accA[MO], accB[MO];
#pragma unroll
    for (int m = 0; m < MO; ++m) {
      accA[m] = accB[m] = 0.f;
      g[m] += gcur[m];
    }
    for (int u = U - 1; u >= 0; --u) {
      const long long n = (long long)t * U + u;
      if (n > 0) bwd_load_unfold<NB, MO>(k, n - 1, b0, ks, o, nvi, nden, nvk, nvk1);
      float gdir[MO];
#pragma unroll
      for (int m = 0; m < MO; ++m) {
        const int b = ks + m * KS;
        gdir[m] = 0.f;
        if (b < NB) {
          float al = 0.f, be = 0.f;
          const bool live = b0 + b < B;
          if (live && o < H) {
            const float rden = cden[m];  // saved 1/den
            al = g[m] * rden;
            be = -g[m] * cvk1[m] * rden;
            accA[m] += al;
            accB[m] += be;
            pC[m] += al * (cvk[m] - cvk1[m]);
            pGv[m] += al * cvk1[m];
            pA[m] += al;
            gdir[m] = al * C;
          }
          ab[abat(b, o)] = make_float2(al, be);
          if (!FUSE && live) k.absave[(n * B + b0 + b) * Hp + o] = make_float2(al, be);
        }
      }
      lds_barrier();
      float acc[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[b] = 0.f;
      if constexpr (FUSE) {
#pragma unroll
        for (int rr = 0; rr < RCP; ++rr)
          bwd_synapse<NB, true>(preg[rr], ab, Hp, r0 + rr, cvi, acc, gacc[rr]);
      } else if constexpr (CMP) {
        // Wave-uniform slot count: the skipped pairs branch around.
#pragma unroll
        for (int q = 0; q < RCP / 4; ++q) {
          if (4 * q < nslot) {
            const int4 of = slot_tab[q * nthr + tid];
            bwd_synapse_folded_cmp<NB>(preg[4 * q], ab, of.x, cvi, acc);
            bwd_synapse_folded_cmp<NB>(preg[4 * q + 1], ab, of.y, cvi, acc);
            if (4 * q + 2 < nslot) {
              bwd_synapse_folded_cmp<NB>(preg[4 * q + 2], ab, of.z, cvi, acc);
              bwd_synapse_folded_cmp<NB>(preg[4 * q + 3], ab, of.w, cvi, acc);
            }
          }
        }
      } else {
        // Streamed (folded) operands, double-buffered four at a time.
        stream_rows(rsB, o * 16, r0, RC, Hp, [&](const float4 p, int r) {
          bwd_synapse_folded<NB>(p, ab, Hp, r, cvi, acc);
        });
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) red[(ks * NB + b) * Hp + o] = acc[b];
      lds_barrier();
#pragma unroll
      for (int m = 0; m < MO; ++m) {
        const int b = ks + m * KS;
        if (b < NB) {
          const float s = NB <= 2 ? ks_sum_1r(red + b * Hp + o, NB * Hp, KS)
                                  : ks_sum(red + b * Hp + o, NB * Hp, KS);
          g[m] = o < H ? fmaf(kNegLn2, s, gdir[m]) : 0.f;
        }
      }
      if (n > 0) {
#pragma unroll
        for (int b = 0; b < NB; ++b) cvi[b] = nvi[b];
#pragma unroll
        for (int m = 0; m < MO; ++m) {
          cden[m] = nden[m];
          cvk[m] = nvk[m];
          cvk1[m] = nvk1[m];
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MO; ++m) {
      const int b = ks + m * KS;
      if (b < NB && b0 + b < B) {
        const long long e = ((long long)(b0 + b) * T + t) * Hp + o;
        k.dsn[e] = accA[m];
        k.dsd[e] = accB[m];
      }
      gcur[m] = gnext[m];
    }
  }
#pragma unroll
  for (int m = 0; m < MO; ++m) {
    const int b = ks + m * KS;
    if (b < NB && b0 + b < B) {
      if (k.gstate != nullptr && o < H) k.gstate[(long long)(b0 + b) * H + o] = g[m];
      float* np = k.npart + (long long)(b0 + b) * 3 * Hp + o;
      np[0] = pC[m];
      np[Hp] = pGv[m];
      np[2 * Hp] = pA[m];
    }
  }
  if constexpr (FUSE) {
    // This workgroup's share of the recurrent parameter gradients, synapse
    // (i = o, j = r0 + rr), layout [workgroup][4][i][j] as rec_grad_kernel's.
    // A thread holds RCP consecutive j of one i, so each plane goes through a
    // padded [Hp][Hp+1] LDS tile and leaves in whole rows (scattered 16-byte
    // pieces cost one cache line each).
    const long long HH = (long long)Hp * Hp;
    float* tile = reinterpret_cast<float*>(lds4);
    float* out = k.rpart + (long long)blockIdx.x * 4 * HH;
    const int nthr = blockDim.x;
#pragma unroll
    for (int pl = 0; pl < 4; ++pl) {
      __syncthreads();  // the LDS is free (chain buffers or the previous plane)
#pragma unroll
      for (int rr = 0; rr < RCP; ++rr) {
        const float4 v = gacc[rr];
        tile[o * (Hp + 1) + r0 + rr] = pl == 0 ? v.x : pl == 1 ? v.y : pl == 2 ? v.z : v.w;
      }
      __syncthreads();
      for (int e = tid; e < Hp * Hp; e += nthr) {
        const int i = e / Hp, j = e - i * Hp;
        out[pl * HH + e] = tile[i * (Hp + 1) + j];
      }
    }
  }
}

// Single-row forward at Hp = 64 with wave-owned columns: 4 waves, wave w owns
// the 16 output columns j = 16w + (lane & 15), and the lane's row group
// g = lane >> 4 holds the compacted entries g, g + 4, ... of column j (the
// rows i whose synapse (i -> j) has a nonzero weight, ascending), with their
// operands and LDS row offsets in registers. The wave runs NS slots, its
// fullest lane's count (at Hp = 128 as row128_slots rounds it), in a loop
// unrolled for that NS.
// A column's sums over its four row groups finish inside the wave
// (group_sum4), so an unfold has one LDS round trip: the new state goes to a
// double-buffered LDS row and, after the unfold's one barrier, every lane
// reads its slots' rows back. A buffer is rewritten one unfold after it was
// read, across that barrier. (8 waves of 8 columns, summed with group_sum8,
// measured slower at C1: 27.1 against 25.9 us.)
// Wave-owned single-row forward layouts: waves of 16 columns with 4 row
// groups per column (group_sum4); HP = 64 runs 4 waves of 16 slots per lane,
// HP = 128 8 waves of 32 (two waves per SIMD, so each wave has 256
// registers for its slots' operands).
// Slot count a single-row Hp = 128 wave runs for its fullest lane's nslot:
// multiples of four up to 12 and from 28, even counts between (where the
// counts of half-dense masks fall), so a wave runs at most one padding slot
// there.
__device__ __forceinline__ int row128_slots(int nslot) {
  if (nslot <= 12) return nslot <= 4 ? 4 : (nslot <= 8 ? 8 : 12);
  if (nslot <= 28) return (nslot + 1) & ~1;
  return 32;
}

template <int HP>
struct RowWave {
  static_assert(HP == 64 || HP == 128, "single-row wave layouts");
  static constexpr int kGroups = 4;
  static constexpr int kSlots = HP / kGroups;
  static constexpr int kThreads = HP * kGroups;
};

// Byte offset of slot r from offsets packed two per register (16 bits each).
template <int N>
__device__ __forceinline__ int slot_offset(const unsigned (&ix)[N], int r) {
  return (int)((r & 1) ? (ix[r >> 1] >> 16) : (ix[r >> 1] & 0xFFFFu));
}

template <int NS, int HP>
__device__ __forceinline__ void fwd_row_wave_loop(const FwdK& k,
                                                  const float4 (&preg)[RowWave<HP>::kSlots],
                                                  const unsigned (&ix)[RowWave<HP>::kSlots / 2],
                                                  float* vsh, int j, bool lead, bool col, float v) {
  constexpr int TS = kRowSensSteps, NT = RowWave<HP>::kThreads;
  const int H = k.H, B = k.B, T = k.T, U = k.U;
  const int b0 = blockIdx.x;
  const float C = k.neuron[j], G = k.neuron[HP + j], L = k.neuron[2 * HP + j];
  const float GL = G * L, CG = C + G;
  // The row's sensory sums go through LDS, TS steps at a time: loaded into
  // registers a step ahead, their wait would be a vmcnt(0) at every step
  // boundary (the compiler cannot count the stores issued since across the
  // loop), which also waits for every vsave/densave/out store in flight.
  float* ssh = vsh + 2 * HP;  // [2][TS][HP]: sn, sd of the staged steps
  // Direct global-to-LDS copies of 64-float segments (no registers held),
  // the waves taking segments in turn.
  auto stage = [&](int t0) {
    const int nseg = min(T - t0, TS) * HP / 64;
    const long long base = ((long long)b0 * T + t0) * HP;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    for (int q = w; q < 2 * nseg; q += NT / 64) {
      const int a = q >= nseg ? 1 : 0, sg = q - a * nseg;
      __builtin_amdgcn_global_load_lds(
          static_cast<const void*>((a ? k.sd : k.sn) + base + sg * 64 + lane),
          (__attribute__((address_space(3))) void*)(ssh + a * TS * HP + sg * 64), 4, 0, 0);
    }
  };
  if (T > 0) stage(0);
  // One wait for the operands and the first staged steps, before the loop:
  // otherwise the loop's first use of them carries a vmcnt(0) wait every
  // unfold, which on gfx9 also waits for the previous unfold's vsave/densave
  // stores.
  __builtin_amdgcn_s_waitcnt(0);
  lds_barrier();
  float snr = 0.f, sdr = 0.f;
  int t = 0, u = 0;
  // One unfold reading state buffer P (compile-time, so the per-lane row
  // offsets are the whole LDS address) and writing buffer P ^ 1.
  auto unfold = [&](auto pc) {
    constexpr int P = decltype(pc)::value;
    if (u == 0) {
      const int ts = t % TS;
      if (ts == 0 && t > 0) {
        // every wave read the previous block's last step U unfolds ago
        stage(t);
        __builtin_amdgcn_s_waitcnt(0);
        lds_barrier();
      }
      snr = ssh[ts * HP + j];
      sdr = ssh[(TS + ts) * HP + j];
    }
    const char* vr = reinterpret_cast<const char*>(vsh + P * HP);
    // Gates in phases (states, arguments, exponentials, reciprocals), in
    // groups of at most ZG slots; the sums keep their order.
    constexpr int ZG = HP == 64 ? 16 : 8;
    float na = 0.f, qa = 0.f;
#pragma unroll
    for (int r0 = 0; r0 < NS; r0 += ZG) {
      constexpr int Z = NS < ZG ? NS : ZG;
      float z[Z];
#pragma unroll
      for (int q = 0; q < Z; ++q)
        if (r0 + q < NS) z[q] = *reinterpret_cast<const float*>(vr + slot_offset(ix, r0 + q));
#pragma unroll
      for (int q = 0; q < Z; ++q)
        if (r0 + q < NS) z[q] = fmaf(preg[r0 + q].x, z[q], preg[r0 + q].y);
#pragma unroll
      for (int q = 0; q < Z; ++q)
        if (r0 + q < NS) z[q] = 1.0f + __builtin_amdgcn_exp2f(z[q]);
#pragma unroll
      for (int q = 0; q < Z; ++q)
        if (r0 + q < NS) z[q] = __builtin_amdgcn_rcpf(z[q]);
#pragma unroll
      for (int q = 0; q < Z; ++q) {
        if (r0 + q < NS) {
          na = fmaf(z[q], preg[r0 + q].z, na);
          qa = fmaf(z[q], preg[r0 + q].w, qa);
        }
      }
    }
    na = group_sum4(na);
    qa = group_sum4(qa);
    const float den = CG + (qa + sdr) + k.eps;
    const float num = C * v + GL + (na + snr);
    const float rden = __builtin_amdgcn_rcpf(den);
    const float vnew = col ? num * rden : 0.f;
    if (lead) {
      vsh[(P ^ 1) * HP + j] = vnew;
      if (k.vsave != nullptr) {
        const long long e = ((long long)(t * U + u) * B + b0) * HP + j;
        k.vsave[e] = v;
        k.densave[e] = rden;
      }
      if (u == U - 1 && col) k.out[((long long)b0 * T + t) * H + j] = vnew;
    }
    lds_barrier();
    v = vnew;
    if (++u == U) {
      u = 0;
      ++t;
    }
  };
  const long long N = (long long)T * U;
  long long n = 0;
  for (; n + 1 < N; n += 2) {
    unfold(std::integral_constant<int, 0>{});
    unfold(std::integral_constant<int, 1>{});
  }
  if (n < N) unfold(std::integral_constant<int, 0>{});
  if (lead) {
    if (col) k.hfin[(long long)b0 * H + j] = v;
    if (k.vsave != nullptr) k.vsave[((long long)T * U * B + b0) * HP + j] = v;
  }
}

template <int HP>
__global__ __launch_bounds__(RowWave<HP>::kThreads) void ode_fwd_row_wave_kernel(FwdK k) {
  constexpr int RC = RowWave<HP>::kSlots, G = RowWave<HP>::kGroups, CW = 64 / G;
  extern __shared__ float4 lds4[];
  float* vsh = reinterpret_cast<float*>(lds4);  // [2][HP], the state by unfold parity
  const int H = k.H;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int g = lane / CW;
  const int j = (tid >> 6) * CW + (lane & (CW - 1));  // output column of this lane
  const bool lead = g == 0;                           // one lane per column stores
  const bool col = j < H;
  const int cnt = k.ccnt[j];
  const int nslot = wave_max(cnt > g ? (cnt - 1 - g) / G + 1 : 0);
  float4 preg[RC];
  unsigned ix[RC / 2];  // LDS byte offsets of the slots' rows, two 16-bit halves each
#pragma unroll
  for (int rr = 0; rr < RC; rr += 2) {
    const long long a = (long long)(g * RC + rr) * HP + j;
    preg[rr] = k.cimg[a];
    preg[rr + 1] = k.cimg[a + HP];
    ix[rr / 2] = (unsigned)(k.cidx[a] * 4) | ((unsigned)(k.cidx[a + HP] * 4) << 16);
  }
  const float v = (k.state0 != nullptr && col) ? k.state0[(long long)blockIdx.x * H + j] : 0.f;
  if (lead) vsh[j] = v;
  if constexpr (HP == 64) {
    switch (nslot) {
#define LTC_FRW(N) \
  case N: fwd_row_wave_loop<N, HP>(k, preg, ix, vsh, j, lead, col, v); break;
      case 0: LTC_FRW(1) LTC_FRW(2) LTC_FRW(3) LTC_FRW(4) LTC_FRW(5) LTC_FRW(6) LTC_FRW(7)
      LTC_FRW(8) LTC_FRW(9) LTC_FRW(10) LTC_FRW(11) LTC_FRW(12) LTC_FRW(13) LTC_FRW(14)
      LTC_FRW(15)
      default: fwd_row_wave_loop<16, HP>(k, preg, ix, vsh, j, lead, col, v); break;
#undef LTC_FRW
    }
  } else {
    // padding slots add zeros
    switch (row128_slots(nslot)) {
#define LTC_FRW(N) \
  case N: fwd_row_wave_loop<N, HP>(k, preg, ix, vsh, j, lead, col, v); break;
      LTC_FRW(4) LTC_FRW(8) LTC_FRW(12) LTC_FRW(14) LTC_FRW(16) LTC_FRW(18) LTC_FRW(20)
      LTC_FRW(22) LTC_FRW(24) LTC_FRW(26) LTC_FRW(28)
      default: fwd_row_wave_loop<32, HP>(k, preg, ix, vsh, j, lead, col, v); break;
#undef LTC_FRW
    }
  }
}

// Stages, for one row's single-workgroup chain, the block of unfolds ending at
// nhi (at most kRowChainUnfolds of them, down to unfold 0): v^n for n = n_lo
// ... nhi + 1, 1/den and dL/dout of the steps they cover, as rows of HP
// floats at vst ([SU + 1][HP] v, then [SU][HP] 1/den, then [SU][HP]
// dL/dout). Each wave copies 64-float segments (wave-uniform kinds) with
// direct global-to-LDS loads, which hold no registers; columns past H get
// 1/den = 1 and dL/dout = 0 by LDS stores. NT threads take part; nothing
// waits here (the caller waits for vmcnt(0), then a workgroup barrier).
template <int HP, int NT, bool FULL>
__device__ __forceinline__ void chain_stage(const BwdK& k, int b0, long long nhi, float* vst,
                                            long long& n_lo, int& t_lo) {
  constexpr int SU = kRowChainUnfolds, SPR = HP / 64;
  const int H = k.H, B = k.B, U = k.U;
  float* rst = vst + (SU + 1) * HP;
  float* gst = rst + SU * HP;
  n_lo = nhi - SU + 1 > 0 ? nhi - SU + 1 : 0;
  t_lo = (int)(n_lo / U);
  const int nu = (int)(nhi - n_lo + 1), nt = (int)(nhi / U) - t_lo + 1;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
  for (int q = w; q < (2 * nu + nt + 1) * SPR; q += NT / 64) {
    const int r = q / SPR, c = (q - r * SPR) * 64 + lane;
    const bool cl = FULL || c < H;
    const float* src;
    float* dst;
    bool ld = true;
    float fill = 0.f;
    if (r <= nu) {
      src = k.vsave + ((n_lo + r) * B + b0) * HP + c;
      dst = vst + r * HP + (c - lane);
    } else if (r <= 2 * nu) {
      const int rr = r - nu - 1;
      src = k.densave + ((n_lo + rr) * B + b0) * HP + c;
      dst = rst + rr * HP + (c - lane);
      ld = cl;
      fill = 1.f;
    } else {
      const int tt = r - 2 * nu - 1;
      src = k.gout + (long long)b0 * k.gs.b + (long long)(t_lo + tt) * k.gs.t +
            (long long)c * k.gs.c;
      dst = gst + tt * HP + (c - lane);
      ld = cl;
    }
    if (ld)
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(src),
                                       (__attribute__((address_space(3))) void*)dst, 4, 0, 0);
    else
      dst[lane] = fill;
  }
}

// Fused single-row chain at Hp = 64 with wave-owned presynaptic neurons: 8
// waves, wave w owns i = 8w + (lane & 7), and the lane's group jg = lane >> 3
// holds the compacted entries jg, jg + 8, ... of column i (its postsynaptic
// j: every real synapse on the boundary, those with a nonzero mask entry on
// the module path), with their operands, four gradient sums and LDS offsets
// in registers. The wave runs NS slots, its fullest lane's count, in a loop
// unrolled for that NS. dL/dv_i finishes inside the wave
// (group_sum8), so an unfold has one LDS round trip: alpha/beta of every
// column go to a double-buffered LDS row and, after the unfold's one barrier,
// every lane reads its slots' pairs back. The unfold loop runs in pairs so
// that the buffer of each unfold is known at compile time.
template <int NS, bool FULL>
__device__ __forceinline__ void bwd_row_wave_loop(const BwdK& k, const float4 (&preg)[8],
                                                  const int (&jx)[8], float4 (&gacc)[8],
                                                  float2* abs_, int i, bool lead) {
  constexpr int HP = 64, SU = kRowChainUnfolds;
  const int H = k.H, B = k.B, T = k.T, U = k.U;
  const int b0 = blockIdx.x;
  const bool col = FULL || i < H;
  const float C = k.neuron[i];
  float g = (k.ghfin != nullptr && col) ? k.ghfin[(long long)b0 * H + i] : 0.f;
  float pC = 0.f, pGv = 0.f, pA = 0.f;
  // The row's saved pre-states v^k (also v_i of the synapses), 1/den and
  // dL/dout go through LDS, SU unfolds at a time, so the loop issues no
  // global load: waiting for one loaded a step ahead would be a vmcnt(0) (the
  // compiler cannot count the word stores issued since), which also waits
  // for every store in flight.
  float* vst = reinterpret_cast<float*>(abs_ + 2 * HP);  // [SU + 1][64] v^n, n = n_lo...
  float* rst = vst + (SU + 1) * HP;                     // [SU][64] 1/den
  float* gst = rst + SU * HP;                           // [SU][64] dL/dout, steps t_lo...
  long long n_lo = 0;
  int t_lo = 0;
  auto stage = [&](long long nhi) {
    chain_stage<HP, 512, FULL>(k, b0, nhi, vst, n_lo, t_lo);
  };
  stage((long long)T * U - 1);
  __builtin_amdgcn_s_waitcnt(0);
  lds_barrier();
  float accA = 0.f, accB = 0.f;
  int t = T - 1, u = U - 1;
  auto unfold = [&](auto pc) {
    constexpr int P = decltype(pc)::value;
    const long long n = (long long)t * U + u;
    if (n < n_lo) {
      // every wave read the previous block's rows before this unfold's barrier
      stage(n);
      __builtin_amdgcn_s_waitcnt(0);
      lds_barrier();
    }
    const int nr = (int)(n - n_lo);
    const float cvk = vst[nr * HP + i], cvk1 = vst[(nr + 1) * HP + i];
    const float crd = rst[nr * HP + i];
    if (u == U - 1) {
      accA = accB = 0.f;
      g += gst[(t - t_lo) * HP + i];
    }
    float al = 0.f, be = 0.f;
    if (col) {
      al = g * crd;  // saved 1/den
      be = -g * cvk1 * crd;
    }
    if (lead) {
      abs_[P * HP + i] = make_float2(al, be);
      accA += al;
      accB += be;
      pC += al * (cvk - cvk1);
      pGv += al * cvk1;
      pA += al;
    }
    const float gdir = al * C;
    // The gates depend on v^k only: evaluated in phases ahead of the barrier.
    float ga[NS];
#pragma unroll
    for (int rr = 0; rr < NS; ++rr) ga[rr] = fmaf(preg[rr].x, cvk, preg[rr].y);
#pragma unroll
    for (int rr = 0; rr < NS; ++rr) ga[rr] = 1.0f + __builtin_amdgcn_exp2f(ga[rr]);
#pragma unroll
    for (int rr = 0; rr < NS; ++rr) ga[rr] = __builtin_amdgcn_rcpf(ga[rr]);
    lds_barrier();
    const char* ar = reinterpret_cast<const char*>(abs_ + P * HP);
    float2 abj[NS];
#pragma unroll
    for (int rr = 0; rr < NS; ++rr) abj[rr] = *reinterpret_cast<const float2*>(ar + jx[rr]);
    float acc = 0.f;
#pragma unroll
    for (int rr = 0; rr < NS; ++rr) {
      const float4 p = preg[rr];
      const float cx = abj[rr].x, cy = abj[rr].y;
      const float a = ga[rr];
      const float a2 = fmaf(-a, a, a);
      const float dl = fmaf(cx, p.z, cy * p.w) * a2;
      acc = fmaf(dl, p.x, acc);
      gacc[rr].x = fmaf(cx, a, gacc[rr].x);
      gacc[rr].y = fmaf(cy, a, gacc[rr].y);
      gacc[rr].z += dl;
      gacc[rr].w = fmaf(dl, cvk, gacc[rr].w);
    }
    const float sum = group_sum8(acc);
    g = col ? fmaf(kNegLn2, sum, gdir) : 0.f;
    if (u == 0) {
      if (lead) {
        const long long e = ((long long)b0 * T + t) * HP + i;
        if (k.rbw != nullptr) {
          xch_put(k.rbw + 2 * e - i, accA, 1u);
          xch_put(k.rbw + 2 * e - i + HP, accB, 1u);
        } else {
          k.dsn[e] = accA;
          k.dsd[e] = accB;
        }
      }
      --t;
      u = U - 1;
    } else {
      --u;
    }
  };
  const long long N = (long long)T * U;
  long long m = 0;
  for (; m + 1 < N; m += 2) {
    unfold(std::integral_constant<int, 0>{});
    unfold(std::integral_constant<int, 1>{});
  }
  if (m < N) unfold(std::integral_constant<int, 0>{});
  if (lead) {
    if (k.gstate != nullptr && col) k.gstate[(long long)b0 * H + i] = g;
    float* np = k.npart + (long long)b0 * 3 * HP + i;
    np[0] = pC;
    np[HP] = pGv;
    np[2 * HP] = pA;
  }
}

template <bool FULL>
__device__ __forceinline__ void bwd_row_wave_body(const BwdK& k) {
  constexpr int HP = 64, RC = 8;
  extern __shared__ float4 lds4[];
  float2* abs_ = reinterpret_cast<float2*>(lds4);  // [2][64] alpha/beta by unfold parity
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int jg = lane >> 3;
  const int i = (tid >> 6) * 8 + (lane & 7);  // presynaptic neuron (and its own alpha/beta column)
  const bool lead = jg == 0;                  // one lane per neuron keeps the sums and stores
  const int cnt = k.ccnt[i];
  const int nmine = cnt > jg ? (cnt - 1 - jg) / 8 + 1 : 0;
  const int nslot = wave_max(nmine);
  float4 preg[RC], gacc[RC];
  int jx[RC];
#pragma unroll
  for (int rr = 0; rr < RC; ++rr) {
    const long long a = (long long)(jg * RC + rr) * HP + i;
    preg[rr] = k.cimg[a];
    jx[rr] = k.cidx[a] * 8;
    gacc[rr] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (k.T == 0) return;
  switch (nslot) {
    case 0:
    case 1: bwd_row_wave_loop<1, FULL>(k, preg, jx, gacc, abs_, i, lead); break;
    case 2: bwd_row_wave_loop<2, FULL>(k, preg, jx, gacc, abs_, i, lead); break;
    case 3: bwd_row_wave_loop<3, FULL>(k, preg, jx, gacc, abs_, i, lead); break;
    case 4: bwd_row_wave_loop<4, FULL>(k, preg, jx, gacc, abs_, i, lead); break;
    case 5: bwd_row_wave_loop<5, FULL>(k, preg, jx, gacc, abs_, i, lead); break;
    case 6: bwd_row_wave_loop<6, FULL>(k, preg, jx, gacc, abs_, i, lead); break;
    case 7: bwd_row_wave_loop<7, FULL>(k, preg, jx, gacc, abs_, i, lead); break;
    default: bwd_row_wave_loop<8, FULL>(k, preg, jx, gacc, abs_, i, lead); break;
  }
  // Recurrent-gradient partials through four padded [64][65] LDS planes at
  // once, whole rows out (layout [workgroup][4][i][j]); each lane places its
  // entries' sums at their columns j. Places without an entry are left as
  // they are (their synapses are masked or padding, and the finalize does not
  // read them).
  constexpr int TLD = HP + 1, PL = HP * TLD;
  constexpr int NT = 512, PER = 4 * HP * HP / NT;
  float* tile = reinterpret_cast<float*>(lds4);
  float* out = k.rpart + (long long)blockIdx.x * 4 * HP * HP;
  __syncthreads();
#pragma unroll
  for (int rr = 0; rr < RC; ++rr) {
    if (rr < nmine) {
      const float4 v4 = gacc[rr];
      const int e = i * TLD + (jx[rr] >> 3);
      tile[e] = v4.x;
      tile[PL + e] = v4.y;
      tile[2 * PL + e] = v4.z;
      tile[3 * PL + e] = v4.w;
    }
  }
  __syncthreads();
  float vals[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int e = tid + q * NT;
    const int pl = e >> 12, ii = (e >> 6) & 63, jj = e & 63;
    vals[q] = tile[pl * PL + ii * TLD + jj];
  }
#pragma unroll
  for (int q = 0; q < PER; ++q) out[tid + q * NT] = vals[q];
}

template <bool FULL>
__global__ __launch_bounds__(512) void ode_bwd_row_wave_kernel(BwdK k) {
  bwd_row_wave_body<FULL>(k);
}

// Single-row chain at Hp = 128, unfused (the recurrent parameter gradients
// come from rec_grad_kernel over the saved alpha/beta): 8 waves; wave w owns
// the presynaptic neurons i = 16w + (lane & 15), and the lane's group
// jg = lane >> 4 holds the folded compacted entries jg, jg + 4, ... of row i
// (the postsynaptic j with S'*WE or S'*WP nonzero, at most 32), with their
// operands and LDS offsets in registers. As in the Hp = 64 chain: one barrier
// and one LDS round trip per unfold, dL/dv_i summed inside the wave
// (group_sum4), the saved rows staged in LDS; alpha/beta of each unfold
// also go to absave.
template <int NS, bool FULL>
__device__ __forceinline__ void bwd_row_wave128_loop(const BwdK& k, const float4 (&preg)[32],
                                                     const unsigned (&jx)[16], float2* abs_, int i,
                                                     bool lead, unsigned long long* sw) {
  constexpr int HP = 128, SU = kRowChainUnfolds;
  const int H = k.H, B = k.B, T = k.T, U = k.U;
  const int b0 = blockIdx.x;
  const bool col = FULL || i < H;
  const float C = k.neuron[i];
  float g = (k.ghfin != nullptr && col) ? k.ghfin[(long long)b0 * H + i] : 0.f;
  float pC = 0.f, pGv = 0.f, pA = 0.f;
  float* vst = reinterpret_cast<float*>(abs_ + 2 * HP);  // [SU + 1][HP] v^n, n = n_lo...
  float* rst = vst + (SU + 1) * HP;                     // [SU][HP] 1/den
  float* gst = rst + SU * HP;                           // [SU][HP] dL/dout, steps t_lo...
  long long n_lo = 0;
  int t_lo = 0;
  chain_stage<HP, 512, FULL>(k, b0, (long long)T * U - 1, vst, n_lo, t_lo);
  __builtin_amdgcn_s_waitcnt(0);
  lds_barrier();
  float accA = 0.f, accB = 0.f;
  int t = T - 1, u = U - 1;
  auto unfold = [&](auto pc) {
    constexpr int P = decltype(pc)::value;
    const long long n = (long long)t * U + u;
    if (n < n_lo) {
      // every wave read the previous block's rows before this unfold's barrier
      chain_stage<HP, 512, FULL>(k, b0, n, vst, n_lo, t_lo);
      __builtin_amdgcn_s_waitcnt(0);
      lds_barrier();
    }
    const int nr = (int)(n - n_lo);
    const float cvk = vst[nr * HP + i], cvk1 = vst[(nr + 1) * HP + i];
    const float crd = rst[nr * HP + i];
    if (u == U - 1) {
      accA = accB = 0.f;
      g += gst[(t - t_lo) * HP + i];
    }
    float al = 0.f, be = 0.f;
    if (col) {
      al = g * crd;  // saved 1/den
      be = -g * cvk1 * crd;
    }
    if (lead) {
      abs_[P * HP + i] = make_float2(al, be);
      if (k.rbw != nullptr) {
        unsigned long long* wd = k.rbw + ((long long)b0 * T * U + n) * 2 * HP + i;
        xch_put(wd, al, 1u);
        xch_put(wd + HP, be, 1u);
      } else {
        k.absave[(n * B + b0) * HP + i] = make_float2(al, be);
      }
      accA += al;
      accB += be;
      pC += al * (cvk - cvk1);
      pGv += al * cvk1;
      pA += al;
    }
    const float gdir = al * C;
    // The gates depend on v^k only: evaluated in phases ahead of the barrier.
    float ga[NS];
#pragma unroll
    for (int rr = 0; rr < NS; ++rr) ga[rr] = fmaf(preg[rr].x, cvk, preg[rr].y);
#pragma unroll
    for (int rr = 0; rr < NS; ++rr) ga[rr] = 1.0f + __builtin_amdgcn_exp2f(ga[rr]);
#pragma unroll
    for (int rr = 0; rr < NS; ++rr) ga[rr] = __builtin_amdgcn_rcpf(ga[rr]);
    lds_barrier();
    const char* ar = reinterpret_cast<const char*>(abs_ + P * HP);
    float acc = 0.f;
#pragma unroll
    for (int rr = 0; rr < NS; ++rr) {
      const float2 c = *reinterpret_cast<const float2*>(ar + slot_offset(jx, rr));
      const float a = ga[rr];
      const float a2 = fmaf(-a, a, a);
      acc = fmaf(fmaf(c.x, preg[rr].z, c.y * preg[rr].w), a2, acc);
    }
    const float sum = group_sum4(acc);
    g = col ? fmaf(kNegLn2, sum, gdir) : 0.f;
    if (u == 0) {
      if (lead) {
        const long long e = ((long long)b0 * T + t) * HP + i;
        if (sw != nullptr) {
          // to the row's sensory companions: [B][T][2][128] words
          xch_put(sw + e + (long long)(b0 * T + t) * HP, accA, 1u);
          xch_put(sw + e + (long long)(b0 * T + t + 1) * HP, accB, 1u);
        } else {
          k.dsn[e] = accA;
          k.dsd[e] = accB;
        }
      }
      --t;
      u = U - 1;
    } else {
      --u;
    }
  };
  const long long N = (long long)T * U;
  long long m = 0;
  for (; m + 1 < N; m += 2) {
    unfold(std::integral_constant<int, 0>{});
    unfold(std::integral_constant<int, 1>{});
  }
  if (m < N) unfold(std::integral_constant<int, 0>{});
  if (lead) {
    if (k.gstate != nullptr && col) k.gstate[(long long)b0 * H + i] = g;
    float* np = k.npart + (long long)b0 * 3 * HP + i;
    np[0] = pC;
    np[HP] = pGv;
    np[2 * HP] = pA;
  }
}

// Companion of the Hp = 128 chain for batch row b and the postsynaptic
// neurons j in [64 jt, 64 jt + 64) (module path): the recurrent
// parameter-gradient sums of rec_grad_kernel for the row, formed while the
// row's chain workgroup publishes each unfold's alpha/beta (latest unfold
// first). 8 waves; lane l of wave w holds the 16 synapses (i = 16w + s,
// j = 64 jt + l) with their forward operands and the four sums
// {sum alpha*a, sum beta*a, sum d, sum d*v_i}, d = (alpha*WE + beta*WP) a(1-a),
// in registers. Per unfold 128 threads wait for the 64 alpha/beta pairs while
// 128 others stage v_i of the unfold's pre-state; one barrier per unfold (two
// LDS buffers by unfold parity). At the end the companion writes its half of
// the row's partial [b][4][Hp][Hp] and returns its words to tag 0, so a second
// backward over the same forward waits for its own. A wait that runs out of
// the budget sets the status word (after the words) and the companion writes
// no partial; the finalize then writes NaN into every output.
template <bool FULL>
__device__ __forceinline__ void rec_companion128(const BwdK& k, const RecC& rc, int b, int jt) {
  constexpr int HP = 128;
  extern __shared__ float4 lds4[];
  float2* ab = reinterpret_cast<float2*>(lds4);       // [2][64] alpha/beta of the unfold
  float* vv = reinterpret_cast<float*>(ab + 2 * 64);  // [2][HP] v_i of the unfold
  int* flag = reinterpret_cast<int*>(vv + 2 * HP);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int j = jt * 64 + lane;
  const long long N = (long long)k.T * k.U;
  const int B = k.B;
  float4 q[16], acc[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    q[r] = rc.recF[(long long)(16 * w + r) * HP + j];
    acc[r] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (tid == 0) *flag = 0;
  __syncthreads();
  unsigned long long* words = k.rbw + (long long)b * N * 2 * HP;
  for (long long n = N - 1; n >= 0; --n) {
    const int par = (int)(n & 1);
    if (tid < 128) {
      const int qq = tid >> 6;  // 0: alpha, 1: beta
      unsigned long long* wd = words + (n * 2 + qq) * HP + jt * 64 + lane;
      bool ok = rc.spin > 0;
      unsigned long long v = 0;
      if (ok) {
        v = xch_get(wd);
        const long long t0 = wall_clock64();
        while ((unsigned)(v >> 32) != 1u) {
          if (wall_clock64() - t0 > rc.spin) {
            ok = false;
            break;
          }
          v = xch_get(wd);
        }
      }
      reinterpret_cast<float*>(ab + par * 64)[lane * 2 + qq] = __uint_as_float((unsigned)v);
      if (!ok) *flag = 1;
    } else if (tid < 256) {
      const int i = tid - 128;
      vv[par * HP + i] = k.vsave[(n * B + b) * HP + i];
    }
    __syncthreads();
    if (*flag) break;
    const float2 c = ab[par * 64 + lane];
    const float* vr = vv + par * HP + 16 * w;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float vi = vr[r];
      const float a = gate(fmaf(q[r].x, vi, q[r].y));
      const float a2 = fmaf(-a, a, a);
      acc[r].x = fmaf(c.x, a, acc[r].x);
      acc[r].y = fmaf(c.y, a, acc[r].y);
      const float dl = fmaf(c.x, q[r].z, c.y * q[r].w) * a2;
      acc[r].z += dl;
      acc[r].w = fmaf(dl, vi, acc[r].w);
    }
  }
  const bool gave_up = *flag != 0;
  if (!gave_up) {
    const long long HH = (long long)HP * HP;
    float* out = k.rpart + (long long)b * 4 * HH;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const long long e = (long long)(16 * w + r) * HP + j;
      out[e] = acc[r].x;
      out[HH + e] = acc[r].y;
      out[2 * HH + e] = acc[r].z;
      out[3 * HH + e] = acc[r].w;
    }
  }
  // this companion's words back to tag 0, every unfold consumed
  for (long long e = tid; e < N * 128; e += (long long)blockDim.x) {
    const long long n = e >> 7;
    const int r = (int)(e & 127);
    xch_put(words + (n * 2 + (r >> 6)) * HP + jt * 64 + (r & 63), 0.f, 0u);
  }
  if (gave_up && tid == 0)
    __hip_atomic_store(rc.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sensory companion of the Hp = 128 chain for batch row b and the neurons
// h in [64 jt, 64 jt + 64) (module path, D <= 64 * DC <= 128): the sensory
// backward of the row's T steps for those neurons, as the row's chain
// workgroup publishes each step's dL/dsn, dL/dsd (latest step first), in
// the fused row backward's layout (8 waves; lane l and wave w hold the DC*8
// synapses d = l + 64*kk, h = 64 jt + 8w + m with their operands and four
// gradient sums; the second 64 inputs' operands in LDS). Per step 128
// threads wait for the step's 128 words while the others stage its row of
// xa; after the synapses, the 8 per-wave partials of dL/dxa[d] are summed in
// a fixed order. The first half (jt = 0) hands its sum to the second as one
// word per input; wave 0 of the second half waits for it, adds its own sum
// (dL/dxa = first + second, as the two-partial LayerNorm backward adds them)
// and finishes the row's LayerNorm backward as ln_bwd_kernel does: dL/dx and
// the column sums of the LayerNorm and input-affine gradients. The second
// half is later in the grid than the first, so it never waits on a workgroup
// dispatched after it. At the end each companion writes its half of the row's
// sensory partial (the second also its LayerNorm column partial) and returns
// the words it consumed to tag 0; a wait that runs out sets the status word
// and no partial is written.
template <int DC>
__device__ __forceinline__ void sens_companion128(const BwdK& k, const RecC& rc, int b, int jt) {
  constexpr int HP = 128, NX = 64 * DC;
  extern __shared__ float4 lds4[];
  float4* qsh = lds4;  // [8][8][64] operands of the second 64 inputs (DC = 2)
  float2* absh = reinterpret_cast<float2*>(lds4 + (DC - 1) * 8 * 8 * 64);  // [64] of the step
  float* xsh = reinterpret_cast<float*>(absh + 64);  // [NX] the step's xa row
  float* dxr = xsh + NX;                             // [8][NX] per-wave dL/dxa partials
  int* flag = reinterpret_cast<int*>(dxr + 8 * NX);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int T = k.T, D = rc.D, Dp = rc.Dp;
  const int h0 = 64 * jt + 8 * w;
  const bool fin = jt == 1 && w == 0;  // the wave that finishes the LayerNorm backward
  // one 64-bit base, 32-bit offsets: the image rows of this wave's 8 neurons
  const float4* srow = rc.sensB + (long long)h0 * Dp + lane;
  float4 q[8], sa[DC][8];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    q[m] = srow[m * Dp];
    if constexpr (DC == 2) qsh[(w * 8 + m) * 64 + lane] = srow[m * Dp + 64];
#pragma unroll
    for (int kk = 0; kk < DC; ++kk) sa[kk][m] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float iw[DC], lw[DC], lb[DC], cw[DC], cb[DC], cl[DC], cbl[DC];
#pragma unroll
  for (int kk = 0; kk < DC; ++kk) {
    const int d = lane + 64 * kk;
    const bool in = fin && d < D;
    iw[kk] = in ? rc.input_w[d] : 0.f;
    lw[kk] = in ? rc.ln_w[d] : 0.f;
    lb[kk] = in ? rc.ln_b[d] : 0.f;
    cw[kk] = cb[kk] = cl[kk] = cbl[kk] = 0.f;
  }
  if (tid == 0) *flag = 0;
  __syncthreads();
  unsigned long long* words = rc.sw + (long long)b * T * 2 * HP;
  // the row's dL/dxa hand-over words, [T][128]
  unsigned long long* dxw = rc.sw + (long long)k.B * T * 2 * HP + (long long)b * T * HP;
  for (int t = T - 1; t >= 0; --t) {
    const long long row = (long long)b * T + t;
    // the finishing wave's LayerNorm inputs of the row, requested before the wait
    float mean = 0.f, rstd = 0.f, xr[DC];
    if (fin) {
      mean = rc.ln.stats[2 * row];
      rstd = rc.ln.stats[2 * row + 1];
      const float* xrow = rc.ln.x + (long long)b * rc.ln.xs.b + (long long)t * rc.ln.xs.t;
#pragma unroll
      for (int kk = 0; kk < DC; ++kk) {
        const int d = lane + 64 * kk;
        xr[kk] = d < D ? xrow[(long long)d * rc.ln.xs.c] : 0.f;
      }
    }
    if (tid < 128) {
      const int qq = tid >> 6;  // 0: dL/dsn, 1: dL/dsd
      unsigned long long* wd = words + ((long long)t * 2 + qq) * HP + 64 * jt + lane;
      bool ok = rc.spin > 0;
      unsigned long long v = 0;
      if (ok) {
        v = xch_get(wd);
        const long long t0 = wall_clock64();
        while ((unsigned)(v >> 32) != 1u) {
          if (wall_clock64() - t0 > rc.spin) {
            ok = false;
            break;
          }
          v = xch_get(wd);
        }
      }
      reinterpret_cast<float*>(absh)[lane * 2 + qq] = __uint_as_float((unsigned)v);
      if (!ok) *flag = 1;
    } else if (tid - 128 < NX) {
      const int d = tid - 128;
      xsh[d] = d < D ? rc.xa[row * D + d] : 0.f;
    }
    __syncthreads();
    if (*flag) break;
#pragma unroll
    for (int kk = 0; kk < DC; ++kk) {
      const float xv = xsh[lane + 64 * kk];
      float dxp = 0.f;
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const float2 cc = absh[8 * w + m];
        const float4 p = kk == 0 ? q[m] : qsh[(w * 8 + m) * 64 + lane];
        const float a = gate(fmaf(p.x, xv, p.y));
        const float a2 = fmaf(-a, a, a);
        const float gm = fmaf(cc.x, p.z, cc.y);
        sa[kk][m].x = fmaf(gm, a, sa[kk][m].x);
        sa[kk][m].y = fmaf(cc.x, a, sa[kk][m].y);
        const float ga2 = gm * a2;
        sa[kk][m].z += ga2;
        sa[kk][m].w = fmaf(ga2, xv, sa[kk][m].w);
        dxp = fmaf(ga2, p.w, dxp);
      }
      dxr[w * NX + lane + 64 * kk] = dxp;
      // one block of 64 inputs at a time (keeps the live registers in bounds)
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();
    if (jt == 0) {
      if (tid < D) {
        float sxa = 0.f;
#pragma unroll
        for (int ww = 0; ww < 8; ++ww) sxa += dxr[ww * NX + tid];
        xch_put(dxw + (long long)t * HP + tid, sxa, 1u);
      }
    } else if (w == 0) {
      float xh[DC], gxh[DC];
      float s1 = 0.f, s2 = 0.f;
      bool ok = true;
#pragma unroll
      for (int kk = 0; kk < DC; ++kk) {
        const int d = lane + 64 * kk;
        xh[kk] = gxh[kk] = 0.f;
        if (d < D) {
          float own = 0.f;
#pragma unroll
          for (int ww = 0; ww < 8; ++ww) own += dxr[ww * NX + d];
          unsigned long long* wd = dxw + (long long)t * HP + d;
          unsigned long long v = xch_get(wd);
          const long long t0 = wall_clock64();
          while ((unsigned)(v >> 32) != 1u) {
            if (wall_clock64() - t0 > rc.spin) {
              ok = false;
              break;
            }
            v = xch_get(wd);
          }
          const float gxa = __uint_as_float((unsigned)v) + own;
          xh[kk] = (xr[kk] - mean) * rstd;
          const float xn = xh[kk] * lw[kk] + lb[kk];
          const float gxn = gxa * iw[kk];
          gxh[kk] = gxn * lw[kk];
          cw[kk] = fmaf(gxa, xn, cw[kk]);
          cb[kk] += gxa;
          cl[kk] = fmaf(gxn, xh[kk], cl[kk]);
          cbl[kk] += gxn;
          s1 += gxh[kk];
          s2 = fmaf(gxh[kk], xh[kk], s2);
        }
      }
      // seen by every wave after the next step's first barrier, or the one below
      if (!ok) *flag = 1;
      const float m1 = wave_sum(s1) / (float)D, m2 = wave_sum(s2) / (float)D;
#pragma unroll
      for (int kk = 0; kk < DC; ++kk) {
        const int d = lane + 64 * kk;
        if (d < D) rc.gx[row * D + d] = rstd * (gxh[kk] - m1 - xh[kk] * m2);
      }
    }
  }
  __syncthreads();
  const bool gave_up = *flag != 0;
  if (!gave_up) {
    // this half of the row's sensory partial, layout [4][Hp][Dp] as sens_bwd_kernel's
    const long long DH = (long long)Dp * HP;
    float* out = rc.spart + (long long)b * 4 * DH;
#pragma unroll
    for (int kk = 0; kk < DC; ++kk)
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const long long e = (long long)(h0 + m) * Dp + lane + 64 * kk;
        out[e] = sa[kk][m].x;
        out[DH + e] = sa[kk][m].y;
        out[2 * DH + e] = sa[kk][m].z;
        out[3 * DH + e] = sa[kk][m].w;
      }
    if (fin) {
      float* lo = rc.lnpart + (long long)b * 4 * Dp;
#pragma unroll
      for (int kk = 0; kk < DC; ++kk) {
        const int d = lane + 64 * kk;
        if (d < Dp) {
          lo[d] = cw[kk];
          lo[Dp + d] = cb[kk];
          lo[2 * Dp + d] = cl[kk];
          lo[3 * Dp + d] = cbl[kk];
        }
      }
    }
  }
  // this companion's words back to tag 0, every step consumed (the second
  // half also clears the row's hand-over words)
  for (int e = tid; e < T * 128; e += (int)blockDim.x) {
    const int t = e >> 7, r = e & 127;
    xch_put(words + ((long long)t * 2 + (r >> 6)) * HP + 64 * jt + (r & 63), 0.f, 0u);
    if (jt == 1) xch_put(dxw + e, 0.f, 0u);
  }
  if (gave_up && tid == 0)
    __hip_atomic_store(rc.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <bool FULL, int DC = 1>
__global__ __launch_bounds__(512) void ode_bwd_row_wave128_kernel(BwdK k, RecC rc) {
  constexpr int HP = 128, RC = 32;
  // With recurrent-gradient companions (rc.recF set): workgroups [0, B) are
  // the chains, [Bc, Bc + B) and [2 Bc, 2 Bc + B) the companions of the
  // postsynaptic halves (Bc = B rounded up to 8, so that a row's companions
  // run on its chain's XCD), the ones between return at once. The chains
  // come first in the grid, so they are dispatched before their companions.
  if (rc.recF != nullptr && (int)blockIdx.x >= k.B) {
    // with sensory companions (rc.sensB set) also [3 Bc, 3 Bc + B) and
    // [4 Bc, 4 Bc + B) for the two 64-neuron halves
    const int Bc = (k.B + 7) / 8 * 8, g = (int)blockIdx.x;
    const int kind = g / Bc, b = g % Bc;
    if (b < k.B) {
      if (kind == 1 || kind == 2)
        rec_companion128<FULL>(k, rc, b, kind - 1);
      else if ((kind == 3 || kind == 4) && rc.sensB != nullptr)
        sens_companion128<DC>(k, rc, b, kind - 3);
    }
    return;
  }
  extern __shared__ float4 lds4[];
  float2* abs_ = reinterpret_cast<float2*>(lds4);  // [2][128] alpha/beta by unfold parity
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int jg = lane >> 4;
  const int i = (tid >> 6) * 16 + (lane & 15);  // presynaptic neuron of this lane
  const bool lead = jg == 0;                    // one lane per neuron keeps the sums and stores
  const int cnt = k.ccnt[i];
  const int nslot = wave_max(cnt > jg ? (cnt - 1 - jg) / 4 + 1 : 0);
  float4 preg[RC];
  unsigned jx[RC / 2];  // LDS byte offsets of the slots' alpha/beta, two 16-bit halves each
#pragma unroll
  for (int rr = 0; rr < RC; rr += 2) {
    const long long a = (long long)(jg * RC + rr) * HP + i;
    preg[rr] = k.cimg[a];
    preg[rr + 1] = k.cimg[a + HP];
    jx[rr / 2] = (unsigned)(k.cidx[a] * 8) | ((unsigned)(k.cidx[a + HP] * 8) << 16);
  }
  if (k.T == 0) return;
  // padding slots add zeros
  switch (row128_slots(nslot)) {
#define LTC_BRW(N) \
  case N: bwd_row_wave128_loop<N, FULL>(k, preg, jx, abs_, i, lead, rc.sw); break;
    LTC_BRW(4) LTC_BRW(8) LTC_BRW(12) LTC_BRW(14) LTC_BRW(16) LTC_BRW(18) LTC_BRW(20)
    LTC_BRW(22) LTC_BRW(24) LTC_BRW(26) LTC_BRW(28)
    default: bwd_row_wave128_loop<32, FULL>(k, preg, jx, abs_, i, lead, rc.sw); break;
#undef LTC_BRW
  }
}

// Companion of the fused row backward for batch row b (module path): the
// sensory backward and the LayerNorm backward of the row's T steps, as the
// chain workgroup of the row publishes each step's dL/dsn, dL/dsd (latest
// step first). 8 waves; lane l and wave w hold the DC*8 sensory synapses
// (d = l + 64*kk, h = 8w + m) with their operands and four gradient sums
// {sum gm*a, sum dsn*a, sum gm*a', sum gm*a'*x} (gm = dsn*E + dsd,
// a' = a(1 - a)) in registers, as sens_bwd_kernel forms them. Per step:
// 128 threads wait for the step's words while the others stage its input row
// in LDS; each thread then adds its synapses' terms and its partial of
// dL/dxa[d] over its 8 neurons; wave 0 sums the 8 partials of every d in a
// fixed order and finishes the row's LayerNorm backward as ln_bwd_kernel
// does, accumulating the column sums. Every wait is bounded by c.spin ticks;
// a companion that runs out sets the status word (after the words) and
// leaves, and the finalize then writes NaN into every output of the call.
template <int DC>
__device__ __forceinline__ void row_companion(const BwdK& k, const RowCompanion& c,
                                              const float4* sensB, int D, int Dp, int b) {
  constexpr int HP = 64, NX = 64 * DC;
  extern __shared__ float4 lds4[];
  // The operands of the second 64 inputs (DC = 2) stay in LDS, [8][8][64]
  // float4, the first 64's in registers.
  float4* qsh = lds4;
  float2* absh = reinterpret_cast<float2*>(lds4 + (DC - 1) * 8 * 8 * 64);  // [64] of the step
  float* xsh = reinterpret_cast<float*>(absh + HP);  // [NX] the step's input row
  float* dxr = xsh + NX;                             // [8][NX] per-wave dL/dxa partials
  int* flag = reinterpret_cast<int*>(dxr + 8 * NX);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int T = k.T;
  // one 64-bit base, 32-bit offsets: the image rows of this wave's 8 neurons
  const float4* srow = sensB + (long long)(8 * w) * Dp + lane;
  float4 q[8], sa[DC][8];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    q[m] = srow[m * Dp];
    if constexpr (DC == 2) qsh[(w * 8 + m) * 64 + lane] = srow[m * Dp + 64];
#pragma unroll
    for (int kk = 0; kk < DC; ++kk) sa[kk][m] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float iw[DC], lw[DC], lb[DC], cw[DC], cb[DC], cl[DC], cbl[DC];
#pragma unroll
  for (int kk = 0; kk < DC; ++kk) {
    const int d = lane + 64 * kk;
    iw[kk] = d < D ? c.input_w[d] : 0.f;
    lw[kk] = d < D ? c.ln_w[d] : 0.f;
    lb[kk] = d < D ? c.ln_b[d] : 0.f;
    cw[kk] = cb[kk] = cl[kk] = cbl[kk] = 0.f;
  }
  if (tid == 0) *flag = 0;
  __syncthreads();
  for (int t = T - 1; t >= 0; --t) {
    const long long row = (long long)b * T + t;
    // wave 0's LayerNorm inputs of the row, requested before the wait
    float mean = 0.f, rstd = 0.f, xr[DC];
    if (w == 0) {
      mean = c.ln.stats[2 * row];
      rstd = c.ln.stats[2 * row + 1];
      const float* xrow = c.ln.x + (long long)b * c.ln.xs.b + (long long)t * c.ln.xs.t;
#pragma unroll
      for (int kk = 0; kk < DC; ++kk) {
        const int d = lane + 64 * kk;
        xr[kk] = d < D ? xrow[(long long)d * c.ln.xs.c] : 0.f;
      }
    }
    if (tid < 2 * HP) {
      unsigned long long* wd = c.words + (row * 2 + (tid >> 6)) * HP + (tid & 63);
      bool ok = c.spin > 0;
      if (ok) {
        unsigned long long v = xch_get(wd);
        const long long t0 = wall_clock64();
        while ((unsigned)(v >> 32) != 1u) {
          if (wall_clock64() - t0 > c.spin) {
            ok = false;
            break;
          }
          v = xch_get(wd);
        }
        reinterpret_cast<float*>(absh)[(tid & 63) * 2 + (tid >> 6)] = __uint_as_float((unsigned)v);
      }
      if (!ok) *flag = 1;
    } else if (tid - 2 * HP < NX) {
      const int d = tid - 2 * HP;
      xsh[d] = d < D ? c.xa[row * D + d] : 0.f;
    }
    __syncthreads();
    if (*flag) break;
#pragma unroll
    for (int kk = 0; kk < DC; ++kk) {
      const float xv = xsh[lane + 64 * kk];
      float dxp = 0.f;
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const float2 cc = absh[8 * w + m];
        const float4 p = kk == 0 ? q[m] : qsh[(w * 8 + m) * 64 + lane];
        const float a = gate(fmaf(p.x, xv, p.y));
        const float a2 = fmaf(-a, a, a);
        const float gm = fmaf(cc.x, p.z, cc.y);
        sa[kk][m].x = fmaf(gm, a, sa[kk][m].x);
        sa[kk][m].y = fmaf(cc.x, a, sa[kk][m].y);
        const float ga2 = gm * a2;
        sa[kk][m].z += ga2;
        sa[kk][m].w = fmaf(ga2, xv, sa[kk][m].w);
        dxp = fmaf(ga2, p.w, dxp);
      }
      dxr[w * NX + lane + 64 * kk] = dxp;
      // one block of 64 inputs at a time (keeps the live registers in bounds)
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();
    if (w == 0) {
      float xh[DC], gxh[DC];
      float s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int kk = 0; kk < DC; ++kk) {
        const int d = lane + 64 * kk;
        xh[kk] = gxh[kk] = 0.f;
        if (d < D) {
          float gxa = 0.f;
#pragma unroll
          for (int ww = 0; ww < 8; ++ww) gxa += dxr[ww * NX + d];
          xh[kk] = (xr[kk] - mean) * rstd;
          const float xn = xh[kk] * lw[kk] + lb[kk];
          const float gxn = gxa * iw[kk];
          gxh[kk] = gxn * lw[kk];
          cw[kk] = fmaf(gxa, xn, cw[kk]);
          cb[kk] += gxa;
          cl[kk] = fmaf(gxn, xh[kk], cl[kk]);
          cbl[kk] += gxn;
          s1 += gxh[kk];
          s2 = fmaf(gxh[kk], xh[kk], s2);
        }
      }
      const float m1 = wave_sum(s1) / (float)D, m2 = wave_sum(s2) / (float)D;
#pragma unroll
      for (int kk = 0; kk < DC; ++kk) {
        const int d = lane + 64 * kk;
        if (d < D) c.gx[row * D + d] = rstd * (gxh[kk] - m1 - xh[kk] * m2);
      }
    }
  }
  // The row's words back to tag 0, every step consumed: another backward
  // over the same forward (whose prep launch cleared them) then waits for its
  // own chain's words instead of reading these.
  for (int e = tid; e < T * 2 * HP; e += (int)blockDim.x)
    xch_put(c.words + (long long)b * T * 2 * HP + e, 0.f, 0u);
  if (*flag) {
    if (tid == 0)
      __hip_atomic_store(reinterpret_cast<int*>(c.words + (long long)k.B * T * 128), 1,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  // One sensory partial per row, layout [4][Hp][Dp] as sens_bwd_kernel's.
  const long long DH = (long long)Dp * HP;
  float* out = c.spart + (long long)b * 4 * DH;
#pragma unroll
  for (int kk = 0; kk < DC; ++kk)
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const long long e = (long long)(8 * w + m) * Dp + lane + 64 * kk;
      out[e] = sa[kk][m].x;
      out[DH + e] = sa[kk][m].y;
      out[2 * DH + e] = sa[kk][m].z;
      out[3 * DH + e] = sa[kk][m].w;
    }
  if (w == 0) {
    float* lo = c.lnpart + (long long)b * 4 * Dp;
#pragma unroll
    for (int kk = 0; kk < DC; ++kk) {
      const int d = lane + 64 * kk;
      lo[d] = cw[kk];
      lo[Dp + d] = cb[kk];
      lo[2 * Dp + d] = cl[kk];
      lo[3 * Dp + d] = cbl[kk];
    }
  }
}

// Fused row backward: workgroups [0, B) run the chain of their batch row
// (bwd_row_wave_body, publishing dL/dsn, dL/dsd as words), workgroups
// [Bc, Bc + B) the companions (Bc = B rounded up to 8, so that the companion
// of row b runs on the same XCD as its chain workgroup); the ones between
// return at once. The chain workgroups come first in the grid, so they are
// dispatched before the companions that wait on them.
template <bool FULL, int DC>
__global__ __launch_bounds__(512) void ode_bwd_row_fused_kernel(BwdK k, RowCompanion c,
                                                                const float4* sensB, int D, int Dp,
                                                                int Bc) {
  const int g = blockIdx.x;
  if (g < k.B) {
    bwd_row_wave_body<FULL>(k);
  } else if (g >= Bc && g - Bc < k.B) {
    row_companion<DC>(k, c, sensB, D, Dp, g - Bc);
  }
}

// ---------------------------------------------------------------------------
// Recurrent parameter gradients, reduced over n = (t,k,b).
// grid (Hp/64, Hp/32, NCH), block 256: lane -> j, wave w -> 8 presynaptic i.
// Per synapse and n:  a = gate, a2 = a(1-a), h = alpha*WE + beta*WP,
//   sWE += alpha*a, sWP += beta*a, sD += h*a2, sDv += h*a2*v_i
// and the finalize kernel forms dM = -S*sD and dS = sDv - M*sD.
// ---------------------------------------------------------------------------
constexpr int RG_NT = 32;

struct RecGK {
  const float4* recF;
  const float* vsave;
  const float2* absave;
  float* rpart;
  int Hp;
  long long N, nper;
};

__global__ __launch_bounds__(256) void rec_grad_kernel(RecGK k) {
  __shared__ __align__(16) float vsh[RG_NT][32];
  __shared__ __align__(16) float2 absh[RG_NT][64];
  const int Hp = k.Hp;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int jb = blockIdx.x * 64, ib = blockIdx.y * 32;
  const int j = jb + lane, i0 = ib + w * 8;
  float4 p[8];
#pragma unroll
  for (int ii = 0; ii < 8; ++ii) p[ii] = k.recF[(long long)(i0 + ii) * Hp + j];
  float sWE[8], sWP[8], sD[8], sDv[8];
#pragma unroll
  for (int ii = 0; ii < 8; ++ii) sWE[ii] = sWP[ii] = sD[ii] = sDv[ii] = 0.f;

  const long long nb = (long long)blockIdx.z * k.nper;
  const long long ne = min(k.N, nb + k.nper);
  // A chunk's v_i and alpha/beta rows are loaded into registers one chunk
  // ahead, so the loads travel while the previous chunk is evaluated.
  constexpr int NV = RG_NT * 32 / 256, NA = RG_NT * 64 / 256;
  float nv[NV];
  float2 nab[NA];
  auto fetch = [&](long long n0) {
#pragma unroll
    for (int q = 0; q < NV; ++q) {
      const int e = threadIdx.x + q * 256;
      const long long n = n0 + (e >> 5);
      nv[q] = n < ne ? k.vsave[n * Hp + ib + (e & 31)] : 0.f;
    }
#pragma unroll
    for (int q = 0; q < NA; ++q) {
      const int e = threadIdx.x + q * 256;
      const long long n = n0 + (e >> 6);
      nab[q] = n < ne ? k.absave[n * Hp + jb + (e & 63)] : make_float2(0.f, 0.f);
    }
  };
  if (nb < ne) fetch(nb);
  for (long long n0 = nb; n0 < ne; n0 += RG_NT) {
#pragma unroll
    for (int q = 0; q < NV; ++q) {
      const int e = threadIdx.x + q * 256;
      vsh[e >> 5][e & 31] = nv[q];
    }
#pragma unroll
    for (int q = 0; q < NA; ++q) {
      const int e = threadIdx.x + q * 256;
      absh[e >> 6][e & 63] = nab[q];
    }
    __syncthreads();
    if (n0 + RG_NT < ne) fetch(n0 + RG_NT);
    const int cnt = (int)min((long long)RG_NT, ne - n0);
    for (int nn = 0; nn < cnt; ++nn) {
      const float2 c = absh[nn][lane];
      const float4 va = *reinterpret_cast<const float4*>(&vsh[nn][w * 8]);
      const float4 vb = *reinterpret_cast<const float4*>(&vsh[nn][w * 8 + 4]);
      const float v[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
#pragma unroll
      for (int ii = 0; ii < 8; ++ii) {
        const float a = gate(fmaf(p[ii].x, v[ii], p[ii].y));
        const float a2 = fmaf(-a, a, a);
        sWE[ii] = fmaf(c.x, a, sWE[ii]);
        sWP[ii] = fmaf(c.y, a, sWP[ii]);
        const float dl = fmaf(c.x, p[ii].z, c.y * p[ii].w) * a2;
        sD[ii] += dl;
        sDv[ii] = fmaf(dl, v[ii], sDv[ii]);
      }
    }
    __syncthreads();
  }
  const long long HH = (long long)Hp * Hp;
  float* out = k.rpart + (long long)blockIdx.z * 4 * HH;
#pragma unroll
  for (int ii = 0; ii < 8; ++ii) {
    const long long e = (long long)(i0 + ii) * Hp + j;
    out[e] = sWE[ii];
    out[HH + e] = sWP[ii];
    out[2 * HH + e] = sD[ii];
    out[3 * HH + e] = sDv[ii];
  }
}

// ---------------------------------------------------------------------------
// Sensory forward over the compacted image as one list per neuron over all of
// D (sFfull; sens_full_list). sens_fwd_cmp_kernel's layout with four row
// groups (lane -> neuron h, wave w -> rows w*RPW ...), but the block's rows of
// x are staged whole (Dp inputs, one barrier) and each lane walks its neuron's
// entries over all of D. A wave then runs its fullest neuron's total count,
// rounded up to four, instead of the fullest count of every 64-input chunk
// rounded up to four: at half-dense masks about 148 slots against 4 x 44.
// The entries come in ascending input order, as over the chunks in turn, so
// the sums take the same terms in the same order as in sens_fwd_cmp_kernel
// (padding slots add exact zeros there between chunks, here at the end).
// ---------------------------------------------------------------------------
template <int RPW>
__global__ __launch_bounds__(256) void sens_fwd_full_kernel(const float* __restrict__ x,
                                                            Strides3 xs, int T, int D, int Dp,
                                                            int BT, int Hp,
                                                            const float4* __restrict__ sF,
                                                            const int* __restrict__ sFi,
                                                            const int* __restrict__ sFn,
                                                            float* __restrict__ sn,
                                                            float* __restrict__ sd) {
  constexpr int ROWS = 4 * RPW;
  constexpr int XLD = ROWS + 4;  // padded staged row, 16-byte aligned
  extern __shared__ float4 lds4[];
  float* xsh = reinterpret_cast<float*>(lds4);  // [Dp][XLD]
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int h = blockIdx.x * 64 + lane;
  const int row0 = blockIdx.y * ROWS;
  const int rw = w * RPW;
  // Stage x: lane l of wave w loads input d0 + l of rows w, w + 4, ...
  const int wu = __builtin_amdgcn_readfirstlane(w);
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int r = wu + 4 * i, row = row0 + r;
    const float* xr = nullptr;
    if (row < BT) {
      const int b = row / T, t = row - b * T;
      xr = x + b * xs.b + t * xs.t;
    }
    for (int d0 = 0; d0 < Dp; d0 += 64) {
      const int d = d0 + lane;
      xsh[d * XLD + r] = (xr != nullptr && d < D) ? xr[(long long)d * xs.c] : 0.f;
    }
  }
  float an[RPW], ad[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) an[r] = ad[r] = 0.f;
  const int nsw = (wave_max(sFn[h]) + 3) & ~3;
  __syncthreads();
  if (nsw > 0) {
    const float4* pcol = sF + h;
    const int* icol = sFi + h;
    float4 pc[4], pn[4];
    int dc[4], dn[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pc[i] = pcol[(long long)i * Hp];
      dc[i] = icol[(long long)i * Hp];
    }
    for (int s = 0; s < nsw; s += 4) {
      // the next group's operands travel while this one is evaluated (the
      // last group reloads itself)
      const int sn4 = s + 4 < nsw ? s + 4 : s;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pn[i] = pcol[(long long)(sn4 + i) * Hp];
        dn[i] = icol[(long long)(sn4 + i) * Hp];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float* xr = xsh + dc[i] * XLD + rw;
        float xq[RPW];
        if constexpr (RPW % 4 == 0) {
#pragma unroll
          for (int r = 0; r < RPW; r += 4) {
            const float4 q4 = *reinterpret_cast<const float4*>(xr + r);
            xq[r] = q4.x;
            xq[r + 1] = q4.y;
            xq[r + 2] = q4.z;
            xq[r + 3] = q4.w;
          }
        } else {
#pragma unroll
          for (int r = 0; r < RPW; ++r) xq[r] = xr[r];
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          const float a = gate(fmaf(pc[i].x, xq[r], pc[i].y));
          an[r] = fmaf(a, pc[i].z, an[r]);
          ad[r] = fmaf(a, pc[i].w, ad[r]);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pc[i] = pn[i];
        dc[i] = dn[i];
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int row = row0 + rw + r;
    if (row < BT) {
      sn[(long long)row * Hp + h] = an[r];
      sd[(long long)row * Hp + h] = ad[r];
    }
  }
}

// ---------------------------------------------------------------------------
// Sensory backward over all (b,t) rows.
// grid (Dp/64, Hp/32, NRC), block 256: lane -> d, wave w -> 8 neurons h.
// With A = dL/dsn, Bq = dL/dsd, gamma = A*Es + Bq, a2 = a(1-a):
//   s1 += gamma*a, s2 += A*a, s3 += gamma*a2, s4 += gamma*a2*x,
//   dx_d += gamma*a2*Ws*Ss   (summed over h; waves meet in LDS, h-blocks in
//   the finalize kernel).
// Finalize: dWs = s1, dEs = Ws*s2, dMs = -Ss*Ws*s3, dSs = Ws*(s4 - Ms*s3).
// ---------------------------------------------------------------------------
constexpr int SB_RT = 32;

struct SensBK {
  const float* x;
  Strides3 xs;
  const float4* sensB;
  const float* dsn;
  const float* dsd;
  float* spart;
  float* dxpart;
  int T, D, Dp, Hp, BT, rows_per;
};

__global__ __launch_bounds__(256) void sens_bwd_kernel(SensBK k) {
  __shared__ __align__(16) float2 absh[SB_RT][32];
  __shared__ float xsh[SB_RT][64];
  __shared__ float dxr[4][SB_RT][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int db = blockIdx.x * 64, hb = blockIdx.y;
  const int d = db + lane, h0 = hb * 32 + w * 8;
  const int Dp = k.Dp, Hp = k.Hp;
  float4 q[8];
#pragma unroll
  for (int hh = 0; hh < 8; ++hh) q[hh] = k.sensB[(long long)(h0 + hh) * Dp + d];
  float s1[8], s2[8], s3[8], s4[8];
#pragma unroll
  for (int hh = 0; hh < 8; ++hh) s1[hh] = s2[hh] = s3[hh] = s4[hh] = 0.f;

  const int rb = blockIdx.z * k.rows_per;
  const int re = min(k.BT, rb + k.rows_per);
  // A chunk's staged values (dL/dsn, dL/dsd of its rows for this block's 32
  // neurons, and its x rows) are loaded into registers one chunk ahead, so
  // the loads travel while the previous chunk is evaluated.
  constexpr int NA = SB_RT * 32 / 256, NX = SB_RT * 64 / 256;
  float2 na[NA];
  float nx[NX];
  auto fetch = [&](int r0) {
    const int cnt = min(SB_RT, re - r0);
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int e = threadIdx.x + i * 256;
      const int rr = e >> 5, hh = e & 31;
      na[i] = make_float2(0.f, 0.f);
      if (rr < cnt) {
        const long long ix = (long long)(r0 + rr) * Hp + hb * 32 + hh;
        na[i] = make_float2(k.dsn[ix], k.dsd[ix]);
      }
    }
    // x rows r0 + wv + 4i, wave-uniform: one division per chunk, then steps
    // of four rows
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int dg = db + (int)(threadIdx.x & 63);
    int b = (r0 + wv) / k.T, t = r0 + wv - b * k.T;
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      nx[i] = 0.f;
      if (wv + 4 * i < cnt && dg < k.D) nx[i] = k.x[b * k.xs.b + t * k.xs.t + dg * k.xs.c];
      t += 4;
      while (t >= k.T) {
        t -= k.T;
        ++b;
      }
    }
  };
  if (rb < re) fetch(rb);
  for (int r0 = rb; r0 < re; r0 += SB_RT) {
    const int cnt = min(SB_RT, re - r0);
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int e = threadIdx.x + i * 256;
      absh[e >> 5][e & 31] = na[i];
    }
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      const int e = threadIdx.x + i * 256;
      xsh[e >> 6][e & 63] = nx[i];
    }
    __syncthreads();
    if (r0 + SB_RT < re) fetch(r0 + SB_RT);
    for (int rr = 0; rr < cnt; ++rr) {
      const float xv = xsh[rr][lane];
      float dxp = 0.f;
#pragma unroll
      for (int hh = 0; hh < 8; ++hh) {
        const float2 c = absh[rr][w * 8 + hh];
        const float a = gate(fmaf(q[hh].x, xv, q[hh].y));
        const float a2 = fmaf(-a, a, a);
        const float gm = fmaf(c.x, q[hh].z, c.y);
        s1[hh] = fmaf(gm, a, s1[hh]);
        s2[hh] = fmaf(c.x, a, s2[hh]);
        const float ga2 = gm * a2;
        s3[hh] += ga2;
        s4[hh] = fmaf(ga2, xv, s4[hh]);
        dxp = fmaf(ga2, q[hh].w, dxp);
      }
      dxr[w][rr][lane] = dxp;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < cnt * 64; e += 256) {
      const int rr = e >> 6, dd = e & 63;
      const float s = dxr[0][rr][dd] + dxr[1][rr][dd] + dxr[2][rr][dd] + dxr[3][rr][dd];
      k.dxpart[((long long)hb * k.BT + r0 + rr) * Dp + db + dd] = s;
    }
    __syncthreads();
  }
  const long long DH = (long long)Dp * Hp;
  float* out = k.spart + (long long)blockIdx.z * 4 * DH;
#pragma unroll
  for (int hh = 0; hh < 8; ++hh) {
    const long long e = (long long)(h0 + hh) * Dp + d;
    out[e] = s1[hh];
    out[DH + e] = s2[hh];
    out[2 * DH + e] = s3[hh];
    out[3 * DH + e] = s4[hh];
  }
}

// ---------------------------------------------------------------------------
// Module-path sensory backward over the unmasked synapses only. A synapse
// whose mask entry is 0 has Ws = 0: its four leaf gradients are zero and it
// adds nothing to dL/dx, so it can be skipped. Same grid, rows and staging as
// sens_bwd_kernel (64 inputs x 32 neurons per block), but each thread's lane
// is one input d and one group of 8 neurons, and holds only that group's
// unmasked synapses of d, in ascending neuron order (NS = the wave's longest
// list, the loop instantiated per NS). The block's 256 lanes run in balanced
// order (balanced_lane), so each wave holds lists of nearly equal length. A
// slot's dL/dsn, dL/dsd come from its neuron's column of the staged rows (a
// per-lane LDS read; 32 float2 fill the 64 banks once). Partials of masked
// synapses stay unwritten: the module finalize writes zero gradients for
// them without reading their partials.
// ---------------------------------------------------------------------------
template <int NS>
__device__ __forceinline__ void sens_bwd_cmp_rows(const SensBK& k, const float4 (&q)[8],
                                                  unsigned hsel, int nmine, int ld, int g,
                                                  int db, int hb, float2 (*absh)[32],
                                                  float (*xsh)[64], float (*dxr)[SB_RT][64]) {
  float s1[NS], s2[NS], s3[NS], s4[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) s1[i] = s2[i] = s3[i] = s4[i] = 0.f;
  const int Dp = k.Dp, Hp = k.Hp;
  const int rb = blockIdx.z * k.rows_per;
  const int re = min(k.BT, rb + k.rows_per);
  constexpr int NA = SB_RT * 32 / 256, NX = SB_RT * 64 / 256;
  float2 na[NA];
  float nx[NX];
  auto fetch = [&](int r0) {
    const int cnt = min(SB_RT, re - r0);
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int e = threadIdx.x + i * 256;
      const int rr = e >> 5, hh = e & 31;
      na[i] = make_float2(0.f, 0.f);
      if (rr < cnt) {
        const long long ix = (long long)(r0 + rr) * Hp + hb * 32 + hh;
        na[i] = make_float2(k.dsn[ix], k.dsd[ix]);
      }
    }
    // x rows r0 + wv + 4i, wave-uniform: one division per chunk, then steps
    // of four rows
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int dg = db + (int)(threadIdx.x & 63);
    int b = (r0 + wv) / k.T, t = r0 + wv - b * k.T;
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      nx[i] = 0.f;
      if (wv + 4 * i < cnt && dg < k.D) nx[i] = k.x[b * k.xs.b + t * k.xs.t + dg * k.xs.c];
      t += 4;
      while (t >= k.T) {
        t -= k.T;
        ++b;
      }
    }
  };
  // the column of each slot's neuron in the staged rows
  int col[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) col[i] = g * 8 + ((hsel >> (3 * i)) & 7);
  if (rb < re) fetch(rb);
  for (int r0 = rb; r0 < re; r0 += SB_RT) {
    const int cnt = min(SB_RT, re - r0);
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int e = threadIdx.x + i * 256;
      absh[e >> 5][e & 31] = na[i];
    }
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      const int e = threadIdx.x + i * 256;
      xsh[e >> 6][e & 63] = nx[i];
    }
    __syncthreads();
    if (r0 + SB_RT < re) fetch(r0 + SB_RT);
    for (int rr = 0; rr < cnt; ++rr) {
      const float xv = xsh[rr][ld];
      float dxp = 0.f;
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const float2 c = absh[rr][col[i]];
        const float a = gate(fmaf(q[i].x, xv, q[i].y));
        const float a2 = fmaf(-a, a, a);
        const float gm = fmaf(c.x, q[i].z, c.y);
        s1[i] = fmaf(gm, a, s1[i]);
        s2[i] = fmaf(c.x, a, s2[i]);
        const float ga2 = gm * a2;
        s3[i] += ga2;
        s4[i] = fmaf(ga2, xv, s4[i]);
        dxp = fmaf(ga2, q[i].w, dxp);
      }
      dxr[g][rr][ld] = dxp;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < cnt * 64; e += 256) {
      const int rr = e >> 6, dd = e & 63;
      const float sum = dxr[0][rr][dd] + dxr[1][rr][dd] + dxr[2][rr][dd] + dxr[3][rr][dd];
      k.dxpart[((long long)hb * k.BT + r0 + rr) * Dp + db + dd] = sum;
    }
    __syncthreads();
  }
  const long long DH = (long long)Dp * Hp;
  float* out = k.spart + (long long)blockIdx.z * 4 * DH;
  const int d = db + ld, h0 = hb * 32 + g * 8;
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    if (i < nmine) {
      const long long e = (long long)(h0 + ((hsel >> (3 * i)) & 7)) * Dp + d;
      out[e] = s1[i];
      out[DH + e] = s2[i];
      out[2 * DH + e] = s3[i];
      out[3 * DH + e] = s4[i];
    }
  }
}

__global__ __launch_bounds__(256) void sens_bwd_cmp_kernel(SensBK k,
                                                           const float* __restrict__ smask,
                                                           int H) {
  __shared__ __align__(16) float2 absh[SB_RT][32];
  __shared__ float xsh[SB_RT][64];
  __shared__ float dxr[4][SB_RT][64];
  __shared__ int perm[256 + 4 * 17];
  const int tid = threadIdx.x;
  const int db = blockIdx.x * 64, hb = blockIdx.y;
  const int D = k.D, Dp = k.Dp;
  // Unmasked synapses of a lane (input d, neurons h0 .. h0 + 7), as a bit set.
  auto keep_bits = [&](int d, int h0) {
    unsigned m = 0;
    if (d < D) {
      const float* row = smask + (long long)d * H;
#pragma unroll
      for (int hh = 0; hh < 8; ++hh)
        if (h0 + hh < H && row[h0 + hh] != 0.f) m |= 1u << hh;
    }
    return m;
  };
  const unsigned m0 = keep_bits(db + (tid & 63), hb * 32 + (tid >> 6) * 8);
  const int lane_id = balanced_lane(__popc(m0), tid, 256, perm, perm + 256);
  const int ld = lane_id & 63, g = lane_id >> 6;
  const int d = db + ld, h0 = hb * 32 + g * 8;
  unsigned m = keep_bits(d, h0);
  const int nmine = __popc(m);
  // The lane's unmasked synapses in ascending neuron order: operands in
  // q[0 .. nmine), neuron offsets as 3-bit fields of hsel.
  float4 q[8];
  unsigned hsel = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    q[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (m != 0) {
      const int hh = __builtin_ctz(m);
      m &= m - 1;
      q[i] = k.sensB[(long long)(h0 + hh) * Dp + d];
      hsel |= (unsigned)hh << (3 * i);
    }
  }
  switch (wave_max(nmine)) {
#define LTC_SBC(N) \
  case N: sens_bwd_cmp_rows<N>(k, q, hsel, nmine, ld, g, db, hb, absh, xsh, dxr); break;
    LTC_SBC(1) LTC_SBC(2) LTC_SBC(3) LTC_SBC(4) LTC_SBC(5) LTC_SBC(6) LTC_SBC(7)
    default: sens_bwd_cmp_rows<8>(k, q, hsel, nmine, ld, g, db, hb, absh, xsh, dxr); break;
#undef LTC_SBC
  }
}

// ---------------------------------------------------------------------------
// Finalize: fixed-order sums of every partial buffer, then the closed forms.
// Flat index space in four segments: (H*H recurrent) + (H neurons) +
// (D*H sensory) + (BT*D x). A launch covers [base, base + count) of it, so
// the per-step entry points can finalize only the recurrent/neuron half or
// only the sensory/x half.
// ---------------------------------------------------------------------------
struct FinK {
  RawParams rp;
  const float* rpart;
  const float* spart;
  const float* dxpart;
  const float* npart;
  GradOut g;
  int B, D, H, Hp, Dp, NCH, NRC, HB, BT;  // B, NCH: counts of neuron / recurrent partials
  long long base, count;
};

// Sum of n strided partials with 8 loads in flight per round.
__device__ __forceinline__ float sum_partials(const float* p, long long stride, int n) {
  float acc = 0.f;
  int z = 0;
  for (; z + 8 <= n; z += 8) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = p[(long long)(z + i) * stride];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += v[i];
  }
  for (; z < n; ++z) acc += p[(long long)z * stride];
  return acc;
}

// sum_partials of P planes (plane q at p + q*pstep) with the loads of all
// planes in flight together; each plane's sum keeps the same order.
template <int P>
__device__ __forceinline__ void sum_partials_planes(const float* p, long long pstep,
                                                    long long stride, int n, float (&acc)[P]) {
#pragma unroll
  for (int q = 0; q < P; ++q) acc[q] = 0.f;
  int z = 0;
  for (; z + 8 <= n; z += 8) {
    float v[P][8];
#pragma unroll
    for (int q = 0; q < P; ++q)
#pragma unroll
      for (int i = 0; i < 8; ++i) v[q][i] = p[q * pstep + (long long)(z + i) * stride];
#pragma unroll
    for (int q = 0; q < P; ++q)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[q] += v[q][i];
  }
  for (; z < n; ++z) {
#pragma unroll
    for (int q = 0; q < P; ++q) acc[q] += p[q * pstep + (long long)z * stride];
  }
}

// First pass of a long partial sum: dst[r][n] = sum of src rows
// [r*rpb, min(M, (r+1)*rpb)) at column n (row stride `stride`), in row order.
__global__ __launch_bounds__(256) void sum_rows_kernel(const float* __restrict__ src,
                                                       long long stride, int M, long long N,
                                                       int rpb, float* __restrict__ dst) {
  const long long n = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int r0 = (int)blockIdx.y * rpb;
  const int cnt = M - r0 < rpb ? M - r0 : rpb;
  dst[(long long)blockIdx.y * N + n] = sum_partials(src + (long long)r0 * stride + n, stride, cnt);
}

__global__ __launch_bounds__(256) void finalize_kernel(FinK k) {
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= k.count) return;
  long long tid = k.base + gid;
  const int H = k.H, D = k.D, Hp = k.Hp, Dp = k.Dp;
  const long long nrec = (long long)H * H, nsens = (long long)D * H;
  if (tid < nrec) {
    const int i = (int)(tid / H), j = (int)(tid - (long long)i * H);
    const long long HH = (long long)Hp * Hp;
    const float* src = k.rpart + (long long)i * Hp + j;
    float sp[4];
    sum_partials_planes<4>(src, HH, 4 * HH, k.NCH, sp);
    const float s0 = sp[0], s1 = sp[1], s2 = sp[2], s3 = sp[3];
    k.g.w_erev[tid] = s0;
    k.g.w_pos[tid] = s1;
    k.g.mu[tid] = -k.rp.sigma[tid] * s2;
    k.g.sigma[tid] = s3 - k.rp.mu[tid] * s2;
    return;
  }
  tid -= nrec;
  if (tid < H) {
    const int j = (int)tid;
    const float* src = k.npart + j;
    float sp[3];
    sum_partials_planes<3>(src, Hp, 3LL * Hp, k.B, sp);
    const float c = sp[0], gv = sp[1], ga = sp[2];
    k.g.cm[j] = c;
    k.g.gleak[j] = k.rp.vleak[j] * ga - gv;
    k.g.vleak[j] = k.rp.gleak[j] * ga;
    return;
  }
  tid -= H;
  if (tid < nsens) {
    // h-major walk so the partial reads are contiguous in d
    const int h = (int)(tid / D), d = (int)(tid - (long long)h * D);
    const long long DH = (long long)Dp * Hp;
    const float* src = k.spart + (long long)h * Dp + d;
    float sp[4];
    sum_partials_planes<4>(src, DH, 4 * DH, k.NRC, sp);
    const float s1 = sp[0], s2 = sp[1], s3 = sp[2], s4 = sp[3];
    const long long e = (long long)d * H + h;
    const float Ws = k.rp.s_wpos[e], Ss = k.rp.s_sigma[e], Ms = k.rp.s_mu[e];
    k.g.s_wpos[e] = s1;
    k.g.s_erev[e] = Ws * s2;
    k.g.s_mu[e] = -Ss * Ws * s3;
    k.g.s_sigma[e] = Ws * (s4 - Ms * s3);
    return;
  }
  tid -= nsens;
  if (tid < (long long)k.BT * D) {
    const long long row = tid / D;
    const int d = (int)(tid - row * D);
    k.g.x[tid] = sum_partials(k.dxpart + row * Dp + d, (long long)k.BT * Dp, k.HB);
  }
}

// Copies `rows` rows of `cols` floats between row pitches (in floats) and
// writes zeros into dst columns [cols, dst_ld): pads (B,H) into [B][Hp] and
// strips the padding again.
__global__ __launch_bounds__(256) void copy_rows_kernel(const float* __restrict__ src,
                                                        long long src_ld, float* __restrict__ dst,
                                                        long long dst_ld, long long rows,
                                                        int cols) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * dst_ld) return;
  const long long r = i / dst_ld;
  const int c = (int)(i - r * dst_ld);
  dst[i] = c < cols ? src[r * src_ld + c] : 0.f;
}

// ---------------------------------------------------------------------------
// Module path: pre-transforms and LayerNorm inside the library.
// ---------------------------------------------------------------------------

// torch's softplus (beta 1, threshold 20) and its derivative z/(z+1), z = e^x.
// softplus(x) = max(x, 0) + log(1 + y), y = e^-|x| in (0, 1], with log(1 + y)
// formed from the hardware exp2/log2 as log(u) * (y / (u - 1)), u = fl(1 + y),
// which corrects for the rounding of 1 + y (Goldberg, "What every computer
// scientist should know about floating-point arithmetic", 1991, Theorem 4):
// a few ulp, branch-free, in about 13 instructions where log1pf(expf(x))
// takes about 150. Above 20 the second term is below half an ulp of x, so
// the result is x, as with torch's threshold; NaN stays NaN.
__device__ __forceinline__ float softplus_t(float x) {
  const float y = __builtin_amdgcn_exp2f(-fabsf(x) * kLog2e);
  const float u = 1.0f + y;
  const float l = (__builtin_amdgcn_logf(u) * kLn2) * (y * __builtin_amdgcn_rcpf(u - 1.0f));
  return fmaxf(x, 0.f) + (u == 1.0f ? y : l);
}
__device__ __forceinline__ float softplus_grad(float x) {
  if (x > 20.f) return 1.f;
  const float z = expf(x);
  return z / (z + 1.f);
}



// One (b,t) row's LayerNorm + affine (the row blocks of prep_leaf_kernel):
// the row in registers, CPL values per lane, two-pass mean/variance,
// xa = ((x - mean)*rstd*ln_w + ln_b)*input_w + input_b. load() issues the
// row's and the four per-column vectors' loads together (one memory round
// trip precedes the two reductions); finish() leaves every lane of the wave
// with the row statistics and its xa values (xo; 0 past D).
template <int CPL>
struct LnRow {
  float xv[CPL], lw[CPL], lb[CPL], iw[CPL], ib[CPL];
  __device__ __forceinline__ void load(const LeafParams& lp, const LnBuf& ln, int row, int D,
                                       int T) {
    const int lane = threadIdx.x & 63;
    const int b = row / T, t = row - b * T;
    const float* xr = ln.x + b * ln.xs.b + t * ln.xs.t;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int d = lane + 64 * c;
      const bool in = d < D;
      xv[c] = in ? xr[d * ln.xs.c] : 0.f;
      lw[c] = in ? lp.ln_w[d] : 0.f;
      lb[c] = in ? lp.ln_b[d] : 0.f;
      iw[c] = in ? lp.input_w[d] : 0.f;
      ib[c] = in ? lp.input_b[d] : 0.f;
    }
  }
  __device__ __forceinline__ void finish(const LeafParams& lp, int D, float (&xo)[CPL],
                                         float& mean, float& rstd) {
    const int lane = threadIdx.x & 63;
    float sum = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) sum += xv[c];
    mean = wave_sum(sum) / (float)D;
    float sq = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int d = lane + 64 * c;
      const float dv = d < D ? xv[c] - mean : 0.f;
      sq = fmaf(dv, dv, sq);
    }
    rstd = 1.0f / sqrtf(wave_sum(sq) / (float)D + lp.ln_eps);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const float xn = (xv[c] - mean) * rstd * lw[c] + lb[c];
      xo[c] = lane + 64 * c < D ? xn * iw[c] + ib[c] : 0.f;
    }
  }
};

template <int CPL>
__device__ __forceinline__ void ln_row(const LeafParams& lp, const LnBuf& ln, int row, int D,
                                       int T, float (&xo)[CPL], float& mean, float& rstd) {
  LnRow<CPL> r;
  r.load(lp, ln, row, D, T);
  r.finish(lp, D, xo, mean, rstd);
}

// Threads per block of the prep launch when it forms the sensory sums.
constexpr int kPrepSensThreads = 512;

// The sensory sums of one (b,t) row for neurons [64*hb, 64*hb + 64), inside
// the prep launch (prep_sens_fused), one 512-thread block per (row, 64
// neurons). Lane -> four neurons h..h+3, h = 64*hb + 4*(lane & 15); input
// group g = 4*w + (lane >> 4) of wave w (32 groups) -> inputs d = g + 32*i.
// The five sensory leaves are read as 16-byte rows of four neurons (H % 4 ==
// 0 and 16-byte aligned leaves, checked by the caller): 10*CPL loads per
// thread, all in flight at once, and each synapse's operands are formed
// from them (zero past D or H). Each wave normalises the whole row itself
// (LnRow) and reads its inputs' xa from its own copy in LDS. The 32
// groups' sums meet in a fixed order: the four lane groups (group_sum4),
// then the waves in LDS. The blocks with hb == 0 save
// xa and the row statistics for the backward, after the sums (stores count
// against the load counter, so storing earlier would delay the barrier).
template <int CPL>
__device__ __forceinline__ void ln_sens_row(const LeafParams& lp, const LnBuf& ln, int row,
                                            int hb, int H, int D, int Hp, int T, float* sn,
                                            float* sd) {
  constexpr int NW = kPrepSensThreads / 64;
  __shared__ float4 part[NW - 1][2][16];
  __shared__ __align__(16) float xs[NW][64 * CPL];
  constexpr int NI = 2 * CPL;  // inputs per thread
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int h = hb * 64 + 4 * (lane & 15);
  const int g = 4 * w + (lane >> 4);
  const bool hok = h < H;  // H % 4 == 0: all four neurons or none
  // The row's loads first, then the operands' (clamped to element 0,
  // selected afterwards) in the order of use: the load counter is in order,
  // so the LayerNorm waits only for the row, and each input's synapses only
  // for their own operands, while the rest stream in.
  // (Scheduling barriers keep the compiler from moving the row's loads
  // behind the operands', the LayerNorm ahead of the operand loads, or
  // operand arithmetic into the LayerNorm, where it would wait for them.)
  LnRow<CPL> lr;
  lr.load(lp, ln, row, D, T);
  __builtin_amdgcn_sched_barrier(0);
  float4 lsw[NI], lsm[NI], lse[NI], lsu[NI], lss[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int d = g + 4 * NW * i;
    const long long e = (d < D && hok) ? (long long)d * H + h : 0;
    lsw[i] = *reinterpret_cast<const float4*>(lp.s_w + e);
    lsm[i] = *reinterpret_cast<const float4*>(lp.s_mask + e);
    lse[i] = *reinterpret_cast<const float4*>(lp.s_erev + e);
    lsu[i] = *reinterpret_cast<const float4*>(lp.s_mu + e);
    lss[i] = *reinterpret_cast<const float4*>(lp.s_sigma + e);
  }
  __builtin_amdgcn_sched_barrier(0);
  float xo[CPL], mean, rstd;
  lr.finish(lp, D, xo, mean, rstd);
  __builtin_amdgcn_sched_barrier(0);
  // Each wave reads only its own copy of the row: an in-wave LDS round trip,
  // ordered by fences at wave scope, with no workgroup barrier.
#pragma unroll
  for (int c = 0; c < CPL; ++c) xs[w][64 * c + lane] = xo[c];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float an[4] = {0.f, 0.f, 0.f, 0.f}, ad[4] = {0.f, 0.f, 0.f, 0.f};
  // One synapse: w_pos = softplus(w) * mask (the mask zeroed past D or H,
  // where the clamped loads hold element 0's finite values, so the synapse
  // adds exact zeros), gate argument sigma*log2(e)*(mu - xa), and the sums
  // n += (a*w_pos)*erev, d += a*w_pos.
  auto syn = [&](int j, float sw, float sm, float se, float su, float ss, float xa) {
    const float t = gate((su - xa) * (ss * kLog2e)) * (softplus_t(sw) * sm);
    an[j] = fmaf(t, se, an[j]);
    ad[j] += t;
  };
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int d = g + 4 * NW * i;  // < 64 * CPL
    const bool ok = d < D && hok;
    const float xa = xs[w][d];
    const float4 m = lsm[i];
    syn(0, lsw[i].x, ok ? m.x : 0.f, lse[i].x, lsu[i].x, lss[i].x, xa);
    syn(1, lsw[i].y, ok ? m.y : 0.f, lse[i].y, lsu[i].y, lss[i].y, xa);
    syn(2, lsw[i].z, ok ? m.z : 0.f, lse[i].z, lsu[i].z, lss[i].z, xa);
    syn(3, lsw[i].w, ok ? m.w : 0.f, lse[i].w, lsu[i].w, lss[i].w, xa);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    an[j] = group_sum4(an[j]);
    ad[j] = group_sum4(ad[j]);
  }
  if (w > 0 && lane < 16) {
    part[w - 1][0][lane] = make_float4(an[0], an[1], an[2], an[3]);
    part[w - 1][1][lane] = make_float4(ad[0], ad[1], ad[2], ad[3]);
  }
  __syncthreads();
  if (w > 0) return;
  if (lane < 16) {
    float4 tn = make_float4(an[0], an[1], an[2], an[3]);
    float4 td = make_float4(ad[0], ad[1], ad[2], ad[3]);
#pragma unroll
    for (int q = 0; q < NW - 1; ++q) {
      const float4 vn = part[q][0][lane], vd = part[q][1][lane];
      tn = make_float4(tn.x + vn.x, tn.y + vn.y, tn.z + vn.z, tn.w + vn.w);
      td = make_float4(td.x + vd.x, td.y + vd.y, td.z + vd.z, td.w + vd.w);
    }
    *reinterpret_cast<float4*>(sn + (long long)row * Hp + h) = tn;
    *reinterpret_cast<float4*>(sd + (long long)row * Hp + h) = td;
  }
  if (hb == 0) {
    float* xrow = ln.xa + (long long)row * D;
#pragma unroll
    for (int c = 0; c < CPL; ++c)
      if (lane + 64 * c < D) xrow[lane + 64 * c] = xo[c];
    if (lane == 0) {
      ln.stats[2LL * row] = mean;
      ln.stats[2LL * row + 1] = rstd;
    }
  }
}

// Parameter images from the leaves (same flat segments as prep_kernel), plus
// LayerNorm + affine of the (b,t) rows in trailing blocks of the same launch
// (ln_row; D <= kModuleMaxD), one wave per row, or with FS one block per
// (row, 64 neurons) that also forms the row's sensory sums (ln_sens_row).
// recb: 0 no chain image, 1 plain {S', c', WE, WP} (fused chain), 2 folded
// {S', c', S'*WE, S'*WP}; sensf / sensb: write the forward / backward
// sensory image. recF and the neuron vector are always written.
// CPL: row values each lane keeps (D <= 64 * CPL <= kModuleMaxD).
template <int CPL, bool FS>
__global__ __launch_bounds__(FS ? kPrepSensThreads : 256) void prep_leaf_kernel(LeafParams lp, Prepped pp, int H, int D,
                                                        int Hp, int Dp, int recb, int sensf,
                                                        int sensb, int nprep_blocks, int ncmp_blocks,
                                                        int nchf, int nchb, LnBuf ln, int T,
                                                        int BT, unsigned long long* clr,
                                                        long long nclr, float* sn, float* sd) {
  if ((int)blockIdx.x >= nprep_blocks && (int)blockIdx.x < nprep_blocks + ncmp_blocks) {
    // Compacted columns, one per wave: forward (synapses whose w_pos or w_erev
    // is nonzero), then chain (synapses whose mask entry is nonzero).
    const int lane = threadIdx.x & 63;
    int col = ((int)blockIdx.x - nprep_blocks) * (int)(blockDim.x >> 6) + (int)(threadIdx.x >> 6);
    auto operand = [&](int i, int j, float4& v) {
      const long long e = (long long)i * H + j;
      const float S = lp.sigma[e], M = lp.mu[e];
      const float wp = softplus_t(lp.w[e]) * lp.mask[e];
      v = make_float4(-S * kLog2e, S * M * kLog2e, wp * lp.erev[e], wp);
    };
    if (pp.cF != nullptr) {
      if (col < Hp) {
        const int j = col;
        compact_column(j, Hp, Hp, nchf, lane, pp.cF, pp.cFi, pp.cFn, [&](int i, float4& v, bool& act) {
          if (i < H && j < H) {
            operand(i, j, v);
            act = v.z != 0.f || v.w != 0.f;
          }
        });
        return;
      }
      col -= Hp;
    }
    if (recb && pp.cB != nullptr) {
      if (col < Hp) {
        // The fused chain (recb == 1) keeps the synapses whose mask entry is
        // nonzero; the unfused one (recb == 2, folded operands) those that
        // add to dL/dv.
        const int i = col;
        compact_column(i, Hp, Hp, nchb, lane, pp.cB, pp.cBi, pp.cBn, [&](int j, float4& v, bool& act) {
          if (i < H && j < H) {
            if (recb == 2) {
              operand(i, j, v);
              v = make_float4(v.x, v.y, v.x * v.z, v.x * v.w);
              act = v.z != 0.f || v.w != 0.f;
            } else if (lp.mask[(long long)i * H + j] != 0.f) {
              operand(i, j, v);
              act = true;
            }
          }
        });
        return;
      }
      col -= Hp;
    }
    if (pp.sF != nullptr && col < (pp.sFfull ? Hp : (Dp / 64) * Hp)) {
      compact_sens_column(pp, col, Hp, D, H, lane, [&](long long e) {
        const float Ss = lp.s_sigma[e], Ms = lp.s_mu[e];
        const float Ws = softplus_t(lp.s_w[e]) * lp.s_mask[e];
        return make_float4(-Ss * kLog2e, Ss * Ms * kLog2e, Ws * lp.s_erev[e], Ws);
      });
    }
    return;
  }
  if ((int)blockIdx.x >= nprep_blocks) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int blk = (int)blockIdx.x - nprep_blocks - ncmp_blocks;
    if constexpr (FS) {
      const int hbn = Hp / 64;
      ln_sens_row<CPL>(lp, ln, blk / hbn, blk - (blk / hbn) * hbn, H, D, Hp, T, sn, sd);
      return;
    }
    const int row = blk * 4 + w;
    if (row >= BT) return;
    float xo[CPL], mean, rstd;
    ln_row<CPL>(lp, ln, row, D, T, xo, mean, rstd);
    float* xrow = ln.xa + (long long)row * D;
#pragma unroll
    for (int c = 0; c < CPL; ++c)
      if (lane + 64 * c < D) xrow[lane + 64 * c] = xo[c];
    if (lane == 0) {
      ln.stats[2LL * row] = mean;
      ln.stats[2LL * row + 1] = rstd;
    }
    return;
  }
  long long tid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long nrec = (long long)Hp * Hp;
  const long long nsens = (long long)Dp * Hp;
  if (tid < nrec) {
    const int i = (int)(tid / Hp), j = (int)(tid - (long long)i * Hp);
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (i < H && j < H) {
      const long long e = (long long)i * H + j;
      const float S = lp.sigma[e], M = lp.mu[e];
      const float wp = softplus_t(lp.w[e]) * lp.mask[e];
      v = make_float4(-S * kLog2e, S * M * kLog2e, wp * lp.erev[e], wp);
    }
    pp.recF[tid] = v;
    // recb == 2: the chain's image carries S'*WE and S'*WP (folded; see
    // bwd_synapse_folded); recb == 1 keeps WE, WP for the fused chain.
    if (recb)
      pp.recB[(long long)j * Hp + i] = recb == 2 ? make_float4(v.x, v.y, v.x * v.z, v.x * v.w) : v;
    return;
  }
  tid -= nrec;
  if (tid < nsens) {
    const int d = (int)(tid / Hp), h = (int)(tid - (long long)d * Hp);
    float4 f = make_float4(0.f, 0.f, 0.f, 0.f), g = f;
    if (d < D && h < H) {
      const long long e = (long long)d * H + h;
      const float Ss = lp.s_sigma[e], Ms = lp.s_mu[e], Es = lp.s_erev[e];
      const float Ws = softplus_t(lp.s_w[e]) * lp.s_mask[e];
      f = make_float4(-Ss * kLog2e, Ss * Ms * kLog2e, Ws * Es, Ws);
      g = make_float4(-Ss * kLog2e, Ss * Ms * kLog2e, Es, Ws * Ss);
    }
    if (sensb) pp.sensB[(long long)h * Dp + d] = g;
    if (sensf) pp.sensF[tid] = f;
    return;
  }
  tid -= nsens;
  if (tid < 3LL * Hp) {
    const int q = (int)(tid / Hp), j = (int)(tid - (long long)q * Hp);
    float v = 0.f;
    if (j < H) {
      if (q == 0) v = softplus_t(lp.cm[j]) / lp.dtU;
      else if (q == 1) v = softplus_t(lp.gleak[j]);
      else v = lp.vleak[j];
    }
    pp.neuron[tid] = v;
    return;
  }
  tid -= 3LL * Hp;
  // the exchange words and status word of the fused backward forms (tag 0),
  // four words per thread in two 16-byte stores (the words are 256-byte aligned)
  const long long e = 4 * tid;
  if (e + 4 <= nclr) {
    uint4* q = reinterpret_cast<uint4*>(clr + e);
    q[0] = make_uint4(0u, 0u, 0u, 0u);
    q[1] = make_uint4(0u, 0u, 0u, 0u);
  } else {
    for (long long r = e; r < nclr; ++r) clr[r] = 0ULL;
  }
}

// LayerNorm + affine backward. Block 256 = 4 waves, `rpb` rows per block (4
// or 16), each wave takes rows w, w+4, ...; CPL column slots per lane (D <=
// 64*CPL). With gxa = dL/dxa (sum of the h-block partials),
// xh = (x - mean)*rstd, gxn = gxa*input_w, gxh = gxn*ln_w:
//   dx = rstd*(gxh - mean_d(gxh) - xh*mean_d(gxh*xh))
// and the column sums dinput_w = sum gxa*xn, dinput_b = sum gxa,
// dln_w = sum gxn*xh, dln_b = sum gxn are accumulated per lane, combined over
// the 4 waves in LDS in a fixed order and written as one partial per block.
template <int CPL>
__global__ __launch_bounds__(256) void ln_bwd_kernel(LeafParams lp, LnBuf ln, const float* dxpart,
                                                     float* gx, float* lnpart, int T, int D,
                                                     int Dp, int BT, int HB, int rpb) {
  __shared__ float col[4][64 * CPL];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  float cw[CPL], cb[CPL], cl[CPL], cbl[CPL];
  float iw[CPL], lw[CPL], lb[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int d = lane + 64 * c;
    cw[c] = cb[c] = cl[c] = cbl[c] = 0.f;
    iw[c] = d < D ? lp.input_w[d] : 0.f;
    lw[c] = d < D ? lp.ln_w[d] : 0.f;
    lb[c] = d < D ? lp.ln_b[d] : 0.f;
  }
  const long long hstride = (long long)BT * Dp;
  for (int i = w; i < rpb; i += 4) {
    const int row = blockIdx.x * rpb + i;
    if (row >= BT) break;
    const int b = row / T, t = row - b * T;
    const float* xr = ln.x + b * ln.xs.b + t * ln.xs.t;
    const float mean = ln.stats[2LL * row], rstd = ln.stats[2LL * row + 1];
    float xh[CPL], gxh[CPL];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int d = lane + 64 * c;
      xh[c] = gxh[c] = 0.f;
      if (d < D) {
        float gxa = 0.f;
        const float* pp = dxpart + (long long)row * Dp + d;
        // Unrolled so that the partials' loads are in flight together (the
        // adds keep their fixed order); less deep at the widest rows, whose
        // registers already hold 16 columns.
        constexpr int UNR = CPL <= 8 ? 8 : 4;
#pragma unroll UNR
        for (int hb = 0; hb < HB; ++hb) gxa += pp[hb * hstride];
        xh[c] = (xr[d * ln.xs.c] - mean) * rstd;
        const float xn = xh[c] * lw[c] + lb[c];
        const float gxn = gxa * iw[c];
        gxh[c] = gxn * lw[c];
        cw[c] = fmaf(gxa, xn, cw[c]);
        cb[c] += gxa;
        cl[c] = fmaf(gxn, xh[c], cl[c]);
        cbl[c] += gxn;
        s1 += gxh[c];
        s2 = fmaf(gxh[c], xh[c], s2);
      }
    }
    const float m1 = wave_sum(s1) / (float)D, m2 = wave_sum(s2) / (float)D;
    float* go = gx + (long long)row * D;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int d = lane + 64 * c;
      if (d < D) go[d] = rstd * (gxh[c] - m1 - xh[c] * m2);
    }
  }
  // Fixed-order combine of the 4 waves' column sums.
  for (int wv = 0; wv < 4; ++wv) {
    if (w == wv) {
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int d = lane + 64 * c;
        if (d < D) {
          if (wv == 0) {
            col[0][d] = cw[c];
            col[1][d] = cb[c];
            col[2][d] = cl[c];
            col[3][d] = cbl[c];
          } else {
            col[0][d] += cw[c];
            col[1][d] += cb[c];
            col[2][d] += cl[c];
            col[3][d] += cbl[c];
          }
        }
      }
    }
    __syncthreads();
  }
  float* out = lnpart + (long long)blockIdx.x * 4 * Dp;
  for (int e = threadIdx.x; e < 4 * D; e += 256) {
    const int q = e / D, d = e - q * D;
    out[(long long)q * Dp + d] = col[q][d];
  }
}

// Finalize of the module path: partial sums as finalize_kernel, then the
// chain rule through the pre-transforms to the module's leaves.
struct FinLeafK {
  LeafParams lp;
  const float* rpart;
  const float* spart;
  const float* npart;
  const float* lnpart;
  LeafGrads g;
  int B, D, H, Hp, Dp, NCH, NRC, NLN;  // B, NCH: counts of neuron / recurrent partials
  // Fused row backward: its status word, and the two outputs written before
  // the finalize (dL/dx over nx floats, dL/dh0 over ns floats), which also
  // become NaN when the status is set.
  const int* status;
  float* gstate;
  long long nx, ns;
};

// Every output this thread owns, NaN (a fused row backward gave up).
__device__ __forceinline__ void finalize_leaf_poison(const FinLeafK& k, long long tid) {
  const float nan = __builtin_nanf("");
  const long long nrec = (long long)k.H * k.H, nsens = (long long)k.D * k.H;
  if (tid == 0) __hip_atomic_store(&g_fault, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (tid < nrec) {
    k.g.w[tid] = k.g.erev[tid] = k.g.mu[tid] = k.g.sigma[tid] = nan;
    return;
  }
  tid -= nrec;
  if (tid < nsens) {
    k.g.s_w[tid] = k.g.s_erev[tid] = k.g.s_mu[tid] = k.g.s_sigma[tid] = nan;
    return;
  }
  tid -= nsens;
  if (tid < k.H) {
    k.g.cm[tid] = k.g.gleak[tid] = k.g.vleak[tid] = nan;
    return;
  }
  tid -= k.H;
  if (tid < k.D) {
    k.g.input_w[tid] = k.g.input_b[tid] = k.g.ln_w[tid] = k.g.ln_b[tid] = nan;
    return;
  }
  tid -= k.D;
  if (tid < k.nx) {
    k.g.x[tid] = nan;
    return;
  }
  tid -= k.nx;
  if (tid < k.ns && k.gstate != nullptr) k.gstate[tid] = nan;
}

// One plane's sum over n partials at stride `stride`, in partial order, up to
// 32 loads in flight at once. Loads past the n-th reload the last partial and
// add zero instead, which leaves the sum bitwise unchanged (it starts at +0,
// and a round-to-nearest sum is never -0 unless both terms are). The address
// advances by one stride per load (up to the last partial), and the adds take
// their bound from a copy of the count that the compiler cannot see through:
// 32 separately formed 64-bit offsets, or the loads' 32 bound conditions kept
// for the adds, would be live in scalar registers at once and spill them.
__device__ __forceinline__ float sum_partials_plane(const float* p, long long stride, int n) {
  float acc = 0.f;
  for (int z = 0; z < n; z += 32) {
    float v[32];
    const float* q = p + (long long)z * stride;
    const int m = n - z;  // partials left from z on, >= 1
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      v[i] = *q;
      if (i + 1 < m) q += stride;
    }
    int ma = m;
    asm volatile("" : "+s"(ma));
#pragma unroll
    for (int i = 0; i < 32; ++i) acc += i < ma ? v[i] : 0.f;
  }
  return acc;
}

// Lane L's value of each group of four lanes (DPP quad permute).
template <int L>
__device__ __forceinline__ float quad_lane(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), L * 0x55, 0xf, 0xf, false));
}

// Four threads per output element: lane q of the quad sums partial plane q,
// the quad exchanges the sums, and lane q writes the element's q-th
// gradient. The sums run in partial order, so the results are those of one
// thread summing all planes, with a quarter of its dependent loads. With a
// gave-up status, one thread per output (every leaf gradient, dL/dx, dL/dh0)
// writes NaN instead.
__global__ __launch_bounds__(256) void finalize_leaf_kernel(FinLeafK k) {
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (k.status != nullptr &&
      __hip_atomic_load(k.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
    finalize_leaf_poison(k, gid);
    return;
  }
  const int H = k.H, D = k.D, Hp = k.Hp, Dp = k.Dp;
  const long long nrec = (long long)H * H, nsens = (long long)D * H;
  // every branch below is uniform over a quad: its lanes share e
  long long e = gid >> 2;
  const int q = (int)(gid & 3);
  if (e < nrec) {
    const int i = (int)(e / H), j = (int)(e - (long long)i * H);
    const long long HH = (long long)Hp * Hp;
    const float mk = k.lp.mask[e];
    if (mk == 0.f) {
      // A masked synapse's four gradients are zero; the compacted chain
      // leaves its partials unwritten.
      float* dst = q == 0 ? k.g.w : (q == 1 ? k.g.erev : (q == 2 ? k.g.mu : k.g.sigma));
      dst[e] = 0.f;
      return;
    }
    const float s = sum_partials_plane(k.rpart + q * HH + (long long)i * Hp + j, 4 * HH, k.NCH);
    const float dwe = quad_lane<0>(s), dwp = quad_lane<1>(s);
    const float sd = quad_lane<2>(s), sdv = quad_lane<3>(s);
    const float wv = k.lp.w[e];
    if (q == 0) {
      // w_pos feeds the synapse directly and through w_erev = w_pos * erev.
      k.g.w[e] = (dwp + dwe * k.lp.erev[e]) * mk * softplus_grad(wv);
    } else if (q == 1) {
      k.g.erev[e] = dwe * (softplus_t(wv) * mk);
    } else if (q == 2) {
      k.g.mu[e] = -k.lp.sigma[e] * sd;
    } else {
      k.g.sigma[e] = sdv - k.lp.mu[e] * sd;
    }
    return;
  }
  e -= nrec;
  if (e < nsens) {
    const int h = (int)(e / D), d = (int)(e - (long long)h * D);
    const long long o = (long long)d * H + h;
    const float mk = k.lp.s_mask[o];
    if (mk == 0.f) {
      // A masked synapse's four gradients are zero; the compacted sensory
      // backward leaves its partials unwritten.
      float* dst = q == 0 ? k.g.s_w : (q == 1 ? k.g.s_erev : (q == 2 ? k.g.s_mu : k.g.s_sigma));
      dst[o] = 0.f;
      return;
    }
    const long long DH = (long long)Dp * Hp;
    const float s = sum_partials_plane(k.spart + q * DH + (long long)h * Dp + d, 4 * DH, k.NRC);
    const float s1 = quad_lane<0>(s), s2 = quad_lane<1>(s);
    const float s3 = quad_lane<2>(s), s4 = quad_lane<3>(s);
    const float sw = k.lp.s_w[o];
    const float Ws = softplus_t(sw) * mk;
    if (q == 0) {
      k.g.s_w[o] = s1 * mk * softplus_grad(sw);
    } else if (q == 1) {
      k.g.s_erev[o] = Ws * s2;
    } else if (q == 2) {
      k.g.s_mu[o] = -k.lp.s_sigma[o] * Ws * s3;
    } else {
      k.g.s_sigma[o] = Ws * (s4 - k.lp.s_mu[o] * s3);
    }
    return;
  }
  e -= nsens;
  if (e < H) {
    const int j = (int)e;
    // three planes: C, G*v and the G*L term
    const float s = q < 3 ? sum_partials_plane(k.npart + q * Hp + j, 3LL * Hp, k.B) : 0.f;
    const float c = quad_lane<0>(s), gv = quad_lane<1>(s), ga = quad_lane<2>(s);
    const float gl = k.lp.gleak[j];
    if (q == 0)
      k.g.cm[j] = c / k.lp.dtU * softplus_grad(k.lp.cm[j]);
    else if (q == 1)
      k.g.gleak[j] = (k.lp.vleak[j] * ga - gv) * softplus_grad(gl);
    else if (q == 2)
      k.g.vleak[j] = softplus_t(gl) * ga;
    return;
  }
  e -= H;
  if (e < D) {
    const int d = (int)e;
    const float s = sum_partials_plane(k.lnpart + q * Dp + d, 4LL * Dp, k.NLN);
    float* dst = q == 0 ? k.g.input_w : (q == 1 ? k.g.input_b : (q == 2 ? k.g.ln_w : k.g.ln_b));
    dst[d] = s;
  }
}

// ---------------------------------------------------------------------------
// Cluster ODE kernels (H >= 256 with few batch rows per CU).
// A cluster of CP workgroups advances NB batch rows together. Member p owns
// the 64 columns [64p, 64p + 64) and keeps only that column slice of the
// operand image, so every operand it reads serves NB rows while all CUs have
// work. Workgroup g runs on XCD g % 8 and is member g % CP, so an XCD's L2
// holds only the slices of the members it runs.
// After every unfold each member publishes its new column values as 64-bit
// words {value bits, unfold tag} (agent-scope atomic stores) and reads the
// other members' words until their tags are current. A word is written and
// read whole, so no fence or counter is involved. Two slots alternate by tag
// parity: a member overwrites a slot only after all partners have published
// the following unfold, which they do after they finished reading that slot.
// Every wait is bounded (a budget of ticks of the 100 MHz wall clock, a
// kernel argument). A member that gives up sets *status, writes NaN into its
// final state and returns; its partners then give up the same way, so the
// grid always drains. The host then overwrites every output of the call with
// NaN and raises the device's fault flag (launch_fill with a gate).
// Exchange layout: [cluster][2 slots][CP members][NB rows][64 columns] words,
// cleared (tag 0) before every launch; tags start at 1.
// ---------------------------------------------------------------------------
constexpr int kClW = 64;                    // columns per cluster member


// Reads the (CP-1)*PER words of the other members for unfold `tag`, XB per
// thread at a time. For each word: pre(x, a) is called once before the first
// poll (to start the loads its delivery needs), deliver(x, a, value) once the
// tag is current; a = q*PER + b*64 + col is the word's offset in the slot and
// x its index in the batch. Returns false if a wait ran out; with a budget
// of spin <= 0 ticks, at the first wait, before any word is read.
constexpr int kXchBatch = 2;

template <int PER, int XB = kXchBatch, class Pre, class Deliver>
__device__ __forceinline__ bool xch_gather(unsigned long long* slot, int p, int nwords, int tid,
                                           int nthr, unsigned tag, long long spin, Pre&& pre,
                                           Deliver&& deliver) {
  if (spin <= 0) return false;
  for (int e0 = tid; e0 < nwords; e0 += XB * nthr) {
    unsigned long long w[XB];
    int at[XB];
    bool wait[XB];
#pragma unroll
    for (int x = 0; x < XB; ++x) {
      const int e = e0 + x * nthr;
      wait[x] = e < nwords;
      at[x] = e + (e / PER >= p ? PER : 0);  // skip this member's own words
      if (wait[x]) {
        w[x] = xch_get(slot + at[x]);
        pre(x, at[x]);
      }
    }
    const long long t0 = wall_clock64();
    for (;;) {
      bool any = false;
#pragma unroll
      for (int x = 0; x < XB; ++x) {
        if (wait[x]) {
          if ((unsigned)(w[x] >> 32) == tag) {
            wait[x] = false;
            deliver(x, at[x], __uint_as_float((unsigned)w[x]));
          } else {
            any = true;
          }
        }
      }
      if (!any) break;
      if (wall_clock64() - t0 > spin) return false;
#pragma unroll
      for (int x = 0; x < XB; ++x)
        if (wait[x]) w[x] = xch_get(slot + at[x]);
    }
  }
  return true;
}

// Cluster and member of workgroup g. Workgroup g runs on XCD g % 8. By
// default member p = g % CP, so the members of a cluster spread over the XCDs
// and each XCD's L2 holds only the operand-image columns of the members it
// runs (what the streamed forms read every unfold). With `xcd_local` (used
// when operands are register-resident and NCL is a multiple of 8) all members
// of a cluster run on one XCD instead: cluster cl lives on XCD cl % 8, so the
// saved rows all its members read come through one L2.
__device__ __forceinline__ void cluster_coords(int g, int CP, bool xcd_local, int& p, int& cl) {
  if (xcd_local) {
    const int xcd = g & 7, slot = g >> 3;
    const int q = slot / CP;
    p = slot - q * CP;
    cl = xcd + 8 * q;
  } else {
    cl = g / CP;
    p = g - cl * CP;
  }
}

struct FwdCK {
  const float4* recF;  // [Hp + 8][Hp]: 8 zero rows of slack for the streamed prefetch
  const float* neuron;
  const float* sn;
  const float* sd;
  const float* state0;
  float* out;
  float* hfin;
  float* vsave;
  float* densave;
  unsigned long long* xch;
  int* status;
  long long spin;  // wait budget of each exchange, wall-clock ticks
  int B, T, H, Hp, U, KS, RC, CP;
  int xcd_local;   // cluster_coords: all members of a cluster on one XCD
  float eps;
  // Compacted forward image (RC = 16): operands, row indices, column counts.
  const float4* cimg;
  const int* cidx;
  const int* ccnt;
  int R0;  // first batch row of this launch (launches take NCL * NB rows each)
};



// RCP = 16 (Hp = 256): the compacted image (CMP). Thread (o, ks) holds the
// entries ks, ks + 16, ... of column c's active rows, and the wave runs as
// many slots as its fullest lane; the state sits in LDS as [Hp][NB] so that a
// slot's NB values are one read at a per-lane row. Slot row offsets live in
// an LDS table [4][threads] of int4.
template <int NB, int RCP>
__global__ __launch_bounds__(1024) void ode_fwd_cl_kernel(FwdCK k) {
  constexpr int PER = NB * kClW;
  constexpr bool CMP = RCP == 16;
  extern __shared__ float4 lds4[];
  __shared__ int gave_up;
  const int Hp = k.Hp, H = k.H, KS = k.KS, B = k.B, T = k.T, U = k.U, CP = k.CP;
  const int RC = RCP > 0 ? RCP : k.RC;
  float* vs = reinterpret_cast<float*>(lds4);            // [NB][Hp] ([Hp][NB] with CMP)
  float2* red = reinterpret_cast<float2*>(vs + NB * Hp);  // [KS][NB][64]
  int4* slot_tab = reinterpret_cast<int4*>(red + KS * NB * kClW);  // CMP: [4][threads]
  auto vat = [&](int b, int j) { return CMP ? j * NB + b : b * Hp + j; };
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int ks = __builtin_amdgcn_readfirstlane(tid >> 6), o = tid & 63;
  int p, cl;
  cluster_coords(blockIdx.x, CP, k.xcd_local != 0, p, cl);
  const int c = p * kClW + o;  // output column of this thread
  const int b0 = k.R0 + cl * NB;
  const int r0 = ks * RC;
  const bool owner = ks < NB;  // finishes row ks of column c (the plan keeps KS >= NB)
  const __amdgpu_buffer_rsrc_t rsF = image_rsrc(k.recF, (long long)Hp * Hp * 16);
  const int bo = ks;
  const bool live = owner && b0 + bo < B;
  unsigned long long* xbase = k.xch + (long long)cl * 2 * CP * PER;
  const int nwords = (CP - 1) * PER;

  const float C = k.neuron[c], G = k.neuron[Hp + c], L = k.neuron[2 * Hp + c];
  const float GL = G * L, CG = C + G;

  float4 preg[RCP > 0 ? RCP : 1];
  int nslot = 0;  // CMP: slots the wave runs
  // Synapse lane of this thread (chunk sks, member column so): with CMP in
  // balanced order (balanced_lane); the owner and exchange roles keep (ks, o).
  int sks = ks, so = o;
  if constexpr (CMP) {
    int* perm = reinterpret_cast<int*>(slot_tab + (RCP / 4) * nthr);  // [threads]
    const int cnt0 = k.ccnt[c];
    const int lane_id = balanced_lane(cnt0 > ks ? (cnt0 - 1 - ks) / kCmpChunks + 1 : 0, tid,
                                      nthr, perm, perm + nthr);
    sks = lane_id >> 6;
    so = lane_id & 63;
    const int sc = p * kClW + so;
    const int cnt = k.ccnt[sc];
    nslot = wave_max(cnt > sks ? (cnt - 1 - sks) / kCmpChunks + 1 : 0);
    int ix[RCP];
#pragma unroll
    for (int rr = 0; rr < RCP; ++rr) {
      const long long a = (long long)(sks * RCP + rr) * Hp + sc;
      preg[rr] = k.cimg[a];
      ix[rr] = k.cidx[a] * NB * 4;
    }
#pragma unroll
    for (int q = 0; q < RCP / 4; ++q)
      slot_tab[q * nthr + tid] = make_int4(ix[4 * q], ix[4 * q + 1], ix[4 * q + 2], ix[4 * q + 3]);
  } else if constexpr (RCP > 0) {
#pragma unroll
    for (int rr = 0; rr < RCP; ++rr) preg[rr] = k.recF[(long long)(r0 + rr) * Hp + c];
  }
  if (tid == 0) gave_up = 0;
  for (int e = tid; e < NB * Hp; e += nthr) {
    const int b = e / Hp, j = e - b * Hp;
    vs[vat(b, j)] = (k.state0 != nullptr && b0 + b < B && j < H)
                        ? k.state0[(long long)(b0 + b) * H + j]
                        : 0.f;
  }
  lds_barrier();

  float snr = 0.f, sdr = 0.f, snn = 0.f, sdn = 0.f;
  auto load_sens = [&](int t, float& a, float& d) {
    a = d = 0.f;
    if (live) {
      const long long e = ((long long)(b0 + bo) * T + t) * Hp + c;
      a = k.sn[e];
      d = k.sd[e];
    }
  };
  if (T > 0) load_sens(0, snr, sdr);
  for (int t = 0; t < T; ++t) {
    if (t + 1 < T) load_sens(t + 1, snn, sdn);
    for (int u = 0; u < U; ++u) {
      float na[NB], qa[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) na[b] = qa[b] = 0.f;
      if constexpr (CMP) {
        // Wave-uniform slot count: the skipped pairs branch around.
#pragma unroll
        for (int q = 0; q < RCP / 4; ++q) {
          if (4 * q < nslot) {
            const int4 of = slot_tab[q * nthr + tid];
            fwd_synapses_cmp<NB>(preg + 4 * q, vs, of.x, of.y, na, qa);
            if (4 * q + 2 < nslot) fwd_synapses_cmp<NB>(preg + 4 * q + 2, vs, of.z, of.w, na, qa);
          }
        }
      } else if constexpr (RCP > 0) {
#pragma unroll
        for (int rr = 0; rr < RCP; rr += kFwdGroup<NB>)
          fwd_synapses<NB, kFwdGroup<NB>>(preg + rr, vs, Hp, r0 + rr, na, qa);
      } else {
        if constexpr (kFwdGroup<NB> == 4) {
          stream_rows4(rsF, c * 16, r0, RC, Hp, [&](const float4* p, int r) {
            fwd_synapses<NB, 4>(p, vs, Hp, r, na, qa);
          });
        } else {
          stream_rows(rsF, c * 16, r0, RC, Hp,
                      [&](const float4 p, int r) { fwd_synapse<NB>(p, vs, Hp, r, na, qa); });
        }
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) red[(sks * NB + b) * kClW + so] = make_float2(na[b], qa[b]);
      lds_barrier();
      const unsigned tag = (unsigned)(t * U + u + 1);
      unsigned long long* slot = xbase + (long long)(tag & 1) * CP * PER;
      if (owner) {
        const float2 nq = ks_sum_wide(red + bo * kClW + o, NB * kClW, KS);
        const float vold = vs[vat(bo, c)];
        const float den = CG + (nq.y + sdr) + k.eps;
        const float num = C * vold + GL + (nq.x + snr);
        const float rden = __builtin_amdgcn_rcpf(den);
        const float vnew = c < H ? num * rden : 0.f;
        // Publish first: the partners wait on it, the other stores on nothing.
        xch_put(slot + p * PER + bo * kClW + o, vnew, tag);
        if (k.vsave != nullptr && live) {
          const long long e = ((long long)(t * U + u) * B + b0 + bo) * Hp + c;
          k.vsave[e] = vold;
          k.densave[e] = rden;
        }
        vs[vat(bo, c)] = vnew;
        if (u == U - 1 && live && c < H) k.out[((long long)(b0 + bo) * T + t) * H + c] = vnew;
      }
      const bool ok = xch_gather<PER>(
          slot, p, nwords, tid, nthr, tag, k.spin, [](int, int) {},
          [&](int, int a, float v) {
            const int q = a / PER, r = a - q * PER;
            vs[vat(r >> 6, q * kClW + (r & 63))] = v;
          });
      if (!ok) gave_up = 1;
      lds_barrier();
      if (gave_up) {
        if (live && c < H) k.hfin[(long long)(b0 + bo) * H + c] = __builtin_nanf("");
        if (tid == 0) __hip_atomic_store(k.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
      }
    }
    snr = snn;
    sdr = sdn;
  }
  if (live) {
    const float v = vs[vat(bo, c)];
    if (c < H) k.hfin[(long long)(b0 + bo) * H + c] = v;
    if (k.vsave != nullptr) k.vsave[((long long)T * U * B + b0 + bo) * Hp + c] = v;
  }
}

// The compacted cluster forward (register-resident operands, RC = 16) with
// its NB >= 2 rows in two groups of NB/2 that take turns, so that each
// group's exchange travels while the other group's synapses are evaluated.
// Phase (g, n) evaluates group g's rows at unfold n. After the phase's one
// barrier, the owners of group g (waves 0 .. NB-1, which the SIMDs issue
// first) finish v_g^{n+1} of the member's columns and publish it, tag n + 1,
// at the start of the next phase, ahead of their own synapses, while the
// other waves go straight on. A phase also gathers the partners' columns of
// the other group's newest state: each gathering thread issues its word's
// load halfway through its synapse slots and writes the value into LDS before
// the barrier. Two barriers per unfold, as in the one-group form, but the
// owners' reduction and the exchange no longer sit between the unfolds.
// Exchange words as in ode_fwd_cl_kernel: [cluster][2 slots][CP][NB][64], a
// group's rows at [g*NB/2, (g+1)*NB/2); each group's tags rise by one per
// unfold and alternate the two slots, so a slot is overwritten only after
// every partner has published the group's following state, which it does
// after it has gathered the slot's words. Waits are bounded as there.
template <int NB>
__global__ __launch_bounds__(1024) void ode_fwd_cl2_kernel(FwdCK k) {
  static_assert(NB == 2 || NB == 4 || NB == 8, "two groups of rows");
  constexpr int HB = NB / 2, RCP = 16, PER = NB * kClW, PERG = HB * kClW;
  extern __shared__ float4 lds4[];
  __shared__ int gave_up;
  const int Hp = k.Hp, H = k.H, KS = k.KS, B = k.B, T = k.T, U = k.U, CP = k.CP;
  float* vs = reinterpret_cast<float*>(lds4);                          // [Hp][NB]
  float2* red = reinterpret_cast<float2*>(vs + NB * Hp);               // [2][KS][HB][64]
  int4* slot_tab = reinterpret_cast<int4*>(red + 2 * KS * HB * kClW);  // [4][threads]
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int ks = __builtin_amdgcn_readfirstlane(tid >> 6), o = tid & 63;
  int p, cl;
  cluster_coords(blockIdx.x, CP, k.xcd_local != 0, p, cl);
  const int c = p * kClW + o;
  const int b0 = k.R0 + cl * NB;
  const bool owner = ks < NB;  // finishes row bo = ks of column c (the plan keeps KS >= NB)
  const int bo = ks, og = ks / HB;
  const bool live = owner && b0 + bo < B;
  unsigned long long* xbase = k.xch + (long long)cl * 2 * CP * PER;
  const float C = k.neuron[c], G = k.neuron[Hp + c], L = k.neuron[2 * Hp + c];
  const float GL = G * L, CG = C + G;

  // Synapse lane in balanced order, as in ode_fwd_cl_kernel.
  float4 preg[RCP];
  int nslot, sks, so;
  {
    int* perm = reinterpret_cast<int*>(slot_tab + (RCP / 4) * nthr);
    const int cnt0 = k.ccnt[c];
    const int lane_id = balanced_lane(cnt0 > ks ? (cnt0 - 1 - ks) / kCmpChunks + 1 : 0, tid,
                                      nthr, perm, perm + nthr);
    sks = lane_id >> 6;
    so = lane_id & 63;
    const int sc = p * kClW + so;
    const int cnt = k.ccnt[sc];
    nslot = wave_max(cnt > sks ? (cnt - 1 - sks) / kCmpChunks + 1 : 0);
    int ix[RCP];
#pragma unroll
    for (int rr = 0; rr < RCP; ++rr) {
      const long long a = (long long)(sks * RCP + rr) * Hp + sc;
      preg[rr] = k.cimg[a];
      ix[rr] = k.cidx[a] * NB * 4;
    }
#pragma unroll
    for (int q = 0; q < RCP / 4; ++q)
      slot_tab[q * nthr + tid] = make_int4(ix[4 * q], ix[4 * q + 1], ix[4 * q + 2], ix[4 * q + 3]);
  }
  if (tid == 0) gave_up = 0;
  for (int e = tid; e < NB * Hp; e += nthr) {
    const int b = e / Hp, j = e - b * Hp;
    vs[j * NB + b] = (k.state0 != nullptr && b0 + b < B && j < H)
                         ? k.state0[(long long)(b0 + b) * H + j]
                         : 0.f;
  }
  lds_barrier();

  // This thread's word of a group gather (threads below (CP - 1) * PERG):
  // partner member gm, row gr of the group, column gc.
  const bool gth = tid < (CP - 1) * PERG;
  int gm = 0, gr = 0, gc = 0;
  if (gth) {
    const int q = tid / PERG, r = tid - q * PERG;
    gm = q + (q >= p ? 1 : 0);
    gr = r / kClW;
    gc = r - gr * kClW;
  }
  const long long N = (long long)T * U;
  float snr = 0.f, sdr = 0.f;  // owners: their row's sensory sums at the current step
  float vlast = 0.f;           // owners: their column's newest state
  bool pend = false;           // owners: a finish of their group is due
  float2 pnq = make_float2(0.f, 0.f);
  long long pn = 0;
  int pt = 0, pu = 0;  // pn's step and unfold within the step
  auto load_sens = [&](int t) {
    snr = sdr = 0.f;
    if (live) {
      const long long e = ((long long)(b0 + bo) * T + t) * Hp + c;
      snr = k.sn[e];
      sdr = k.sd[e];
    }
  };
  // The owners' finish of unfold pn: v^{pn+1} of (row bo, column c) from the
  // reduced sums pnq; publish (when a partner needs it), saved state, output.
  auto finish = [&](bool publish) {
    const int t = pt, u = pu;
    const float vold = vs[c * NB + bo];
    const float den = CG + (pnq.y + sdr) + k.eps;
    const float num = C * vold + GL + (pnq.x + snr);
    const float rden = __builtin_amdgcn_rcpf(den);
    const float vnew = c < H ? num * rden : 0.f;
    if (publish) {
      const unsigned tag = (unsigned)(pn + 1);
      xch_put(xbase + (long long)(tag & 1) * CP * PER + p * PER + bo * kClW + o, vnew, tag);
    }
    if (k.vsave != nullptr && live) {
      const long long e = (pn * B + b0 + bo) * Hp + c;
      k.vsave[e] = vold;
      k.densave[e] = rden;
    }
    vs[c * NB + bo] = vnew;
    vlast = vnew;
    if (u == U - 1) {
      if (live && c < H) k.out[((long long)(b0 + bo) * T + t) * H + c] = vnew;
      if (t + 1 < T) load_sens(t + 1);
    }
  };
  if (owner && T > 0) load_sens(0);
  // step t and unfold u within it, stepped with n
  int t = 0, u = 0;
  auto step = [&] {
    if (++u == U) {
      u = 0;
      ++t;
    }
  };
  for (long long n = 0; n < N; ++n, step()) {
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      if (pend) {
        pend = false;
        finish(true);
      }
      // The other group's newest state: v_0^{n+1} (published at the start
      // of this phase) while evaluating group 1, v_1^n while evaluating
      // group 0; not needed past the last unfold or before the first.
      const int gg = 1 - g;
      const long long gtag = g == 1 ? n + 1 : n;
      const bool need = g == 1 ? n + 1 < N : n > 0;
      unsigned long long* gw = xbase + (long long)(gtag & 1) * CP * PER + gm * PER +
                               (gg * HB + gr) * kClW + gc;
      unsigned long long w = 0;
      float na[HB], qa[HB];
#pragma unroll
      for (int b = 0; b < HB; ++b) na[b] = qa[b] = 0.f;
      // the slot count, opaque here so that the slot branches' conditions are
      // not held as lane masks across the loop
      int nsl = nslot;
      asm volatile("" : "+s"(nsl));
#pragma unroll
      for (int q = 0; q < RCP / 4; ++q) {
        if (q == RCP / 8 && need && gth) w = xch_get(gw);
        if (4 * q < nsl) {
          const int4 of = slot_tab[q * nthr + tid];
          fwd_synapses_cmp<HB>(preg + 4 * q, vs + g * HB, of.x, of.y, na, qa);
          if (4 * q + 2 < nsl)
            fwd_synapses_cmp<HB>(preg + 4 * q + 2, vs + g * HB, of.z, of.w, na, qa);
        }
      }
      float2* rg = red + g * KS * HB * kClW;
#pragma unroll
      for (int b = 0; b < HB; ++b) rg[(sks * HB + b) * kClW + so] = make_float2(na[b], qa[b]);
      if (k.spin <= 0) {
        gave_up = 1;  // a budget of 0: give up at the first wait, as xch_gather does
      } else if (need && gth) {
        const long long t0 = wall_clock64();
        bool ok = true;
        while ((unsigned)(w >> 32) != (unsigned)gtag) {
          if (wall_clock64() - t0 > k.spin) {
            ok = false;
            break;
          }
          w = xch_get(gw);
        }
        if (ok)
          vs[(gm * kClW + gc) * NB + gg * HB + gr] = __uint_as_float((unsigned)w);
        else
          gave_up = 1;
      }
      lds_barrier();
      if (gave_up) {
        if (live && c < H) k.hfin[(long long)(b0 + bo) * H + c] = __builtin_nanf("");
        if (tid == 0) __hip_atomic_store(k.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
      }
      if (owner && og == g) {
        pnq = ks_sum_wide(rg + (bo - g * HB) * kClW + o, HB * kClW, KS);
        pn = n;
        pt = t;
        pu = u;
        pend = true;
      }
    }
  }
  // group 1's last finish: nothing gathers v_1^N
  if (pend) finish(false);
  if (live) {
    if (c < H) k.hfin[(long long)(b0 + bo) * H + c] = vlast;
    if (k.vsave != nullptr) k.vsave[((long long)T * U * B + b0 + bo) * Hp + c] = vlast;
  }
}

// Fused chain synapse phase with streamed operands (RCS rows per thread,
// fully unrolled so that each row's four gradient sums stay in registers).
// Members are 32 columns wide, so a wave holds two reduction chunks: its
// lower half reads rows [srow0, srow0 + RCS), its upper half the RCS rows
// after them. The upper half's row offset rides in its per-lane byte offset,
// so the row walk stays a scalar offset. Rows come four at a time, the next
// four requested while the current four are evaluated; nothing is requested
// past the chunk, so no load is left in flight when the phase ends.
//   jrow0  this thread's first postsynaptic row (for alpha/beta in LDS)
template <int NB, int RCS>
__device__ __forceinline__ void chain_fused_stream(__amdgpu_buffer_rsrc_t rs, int lane_bytes,
                                                   int srow0, int jrow0, int Hp,
                                                   const float2* ab, const float* vi,
                                                   float* acc, float4 (&gacc)[RCS]) {
  static_assert(RCS % 8 == 0, "rows come in groups of eight");
  const int rowb = Hp * 16;
  const int sb = srow0 * rowb;
  float4 pa[4], pb[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) pa[q] = image_load(rs, lane_bytes, sb + q * rowb);
#pragma unroll
  for (int rr = 0; rr < RCS; rr += 8) {
#pragma unroll
    for (int q = 0; q < 4; ++q) pb[q] = image_load(rs, lane_bytes, sb + (rr + 4 + q) * rowb);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      bwd_synapse<NB, true>(pa[q], ab, Hp, jrow0 + rr + q, vi, acc, gacc[rr + q]);
      asm volatile("" : "+v"(gacc[rr + q].x), "+v"(gacc[rr + q].y), "+v"(gacc[rr + q].z),
                   "+v"(gacc[rr + q].w));
    }
    __builtin_amdgcn_sched_barrier(0);
    if (rr + 8 < RCS) {  // no prefetch past the chunk: nothing would use it
#pragma unroll
      for (int q = 0; q < 4; ++q) pa[q] = image_load(rs, lane_bytes, sb + (rr + 8 + q) * rowb);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      bwd_synapse<NB, true>(pb[q], ab, Hp, jrow0 + rr + 4 + q, vi, acc, gacc[rr + 4 + q]);
      asm volatile("" : "+v"(gacc[rr + 4 + q].x), "+v"(gacc[rr + 4 + q].y),
                   "+v"(gacc[rr + 4 + q].z), "+v"(gacc[rr + 4 + q].w));
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Copies rows [b0, b0 + NB) of one [B][HP] slice (rows < B only) into LDS
// [NB][HP] with direct global-to-LDS loads, 16 bytes per lane; a wave fills
// 1 KiB of LDS per instruction. NT threads take part. Nothing waits here:
// the caller waits for vmcnt(0) and then a workgroup barrier before it reads
// the block.
template <int NB, int HP, int NT>
__device__ __forceinline__ void rows_to_lds_fixed(const float* slice, int b0, int B, float* dst,
                                                  int tid) {
  constexpr int units = NB * HP / 4, upr = HP / 4;
  const int lane = tid & 63;
#pragma unroll
  for (int i = 0; i < (units + NT - 1) / NT; ++i) {
    const int u0 = i * NT + (tid & ~63);
    const int u = u0 + lane;
    if (u < units && b0 + u / upr < B)
      __builtin_amdgcn_global_load_lds(
          static_cast<const void*>(slice + (long long)b0 * HP + 4LL * u),
          (__attribute__((address_space(3))) void*)(dst + 4 * u0), 16, 0, 0);
  }
}

// Waits for this wave's outstanding global loads (and stores), including
// the direct-to-LDS ones; LDS and export counters are not waited on.
__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(0x0F70); }

struct BwdCK {
  const float4* recB;  // [Hp][Hp] (+ slack rows)
  const float* neuron;
  const float* vsave;
  const float* densave;
  const float* gout;
  Strides3 gs;
  const float* ghfin;
  float2* absave;
  float* dsn;
  float* dsd;
  float* npart;
  float* gstate;
  float* rpart;  // FUSE: one recurrent-gradient partial per cluster, [NCL][4][Hp][Hp]
  unsigned long long* xch;
  int* status;
  long long spin;  // wait budget of each exchange, wall-clock ticks
  int B, T, H, Hp, U, KS, RC, CP;
  int xcd_local;   // cluster_coords: all members of a cluster on one XCD
  // Compacted chain image (fused, RC = 16): operands, row indices, column counts.
  const float4* cimg;
  const int* cidx;
  const int* ccnt;
  int R0;  // first batch row of this launch (launches take NCL * NB rows each)
};

// One compacted chain synapse for every row of the tile: alpha/beta of its
// row come from the [Hp][NB] float2 layout at byte offset `off` (one 8*NB
// byte read per lane), the rest as bwd_synapse<NB, true>.
template <int NB>
__device__ __forceinline__ void bwd_synapse_cmp(const float4 p, const float2* ab, int off,
                                                const float* vi, float* acc, float4& gacc) {
  float2 c[NB];
  const char* at = reinterpret_cast<const char*>(ab) + off;
  if constexpr (NB % 2 == 0) {
#pragma unroll
    for (int b = 0; b < NB; b += 2) {
      const float4 w = *reinterpret_cast<const float4*>(at + b * 8);
      c[b] = make_float2(w.x, w.y);
      c[b + 1] = make_float2(w.z, w.w);
    }
  } else {
    c[0] = *reinterpret_cast<const float2*>(at);
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const float a = gate(fmaf(p.x, vi[b], p.y));
    const float a2 = fmaf(-a, a, a);
    const float dl = fmaf(c[b].x, p.z, c[b].y * p.w) * a2;
    acc[b] = fmaf(dl, p.x, acc[b]);
    gacc.x = fmaf(c[b].x, a, gacc.x);
    gacc.y = fmaf(c[b].y, a, gacc.y);
    gacc.z += dl;
    gacc.w = fmaf(dl, vi[b], gacc.w);
  }
}

// bwd_synapse_cmp over operands (x, y, E, w x), w factored out of dL/darg:
// dl = (alpha E + beta) a (1 - a) is dL/darg / w, so dL/dv_i takes dl (w x)
// and the last two gradient sums (of dL/darg and dL/darg v_i) come out
// divided by w, which the caller multiplies back once at the end. One
// multiply per synapse-row fewer.
template <int NB>
__device__ __forceinline__ void bwd_synapse_cmpe(const float4 p, const float2* ab, int off,
                                                 const float* vi, float* acc, float4& gacc) {
  float2 c[NB];
  const char* at = reinterpret_cast<const char*>(ab) + off;
  if constexpr (NB % 2 == 0) {
#pragma unroll
    for (int b = 0; b < NB; b += 2) {
      const float4 w = *reinterpret_cast<const float4*>(at + b * 8);
      c[b] = make_float2(w.x, w.y);
      c[b + 1] = make_float2(w.z, w.w);
    }
  } else {
    c[0] = *reinterpret_cast<const float2*>(at);
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const float a = gate(fmaf(p.x, vi[b], p.y));
    const float a2 = fmaf(-a, a, a);
    const float dl = fmaf(c[b].x, p.z, c[b].y) * a2;
    acc[b] = fmaf(dl, p.w, acc[b]);
    gacc.x = fmaf(c[b].x, a, gacc.x);
    gacc.y = fmaf(c[b].y, a, gacc.y);
    gacc.z += dl;
    gacc.w = fmaf(dl, vi[b], gacc.w);
  }
}

// Cluster chain: member p forms dL/dv_i for its JW columns i (reduction over
// every postsynaptic j) and publishes them; alpha_j/beta_j of the other
// members' columns are then rebuilt from the published dL/dv_j and the saved
// 1/den_j, v_j, so only one value per (row, column) crosses the cluster.
// Thread (o, ks): column i = p*JW + o, postsynaptic rows [ks*RC, ks*RC + RC).
// FUSE (JW = 32, the unfolded image): the thread also accumulates the four
// recurrent parameter-gradient sums of its synapses over all rows and
// unfolds, and writes one partial per cluster, so the separate
// parameter-gradient pass and its gate evaluation go away. Its operands are
// register-resident (RCP rows) or streamed (RCS rows, chain_fused_stream).
// FUSE with RCP = 16 (Hp = 256) reads the compacted image (CMP): thread
// (o, ks) holds the entries ks, ks + 16, ... of column c's synapses, the wave
// runs as many slots as its fullest lane, alpha/beta sit in LDS as [Hp][NB]
// float2 (a slot's NB pairs at one per-lane row), and the slot row offsets
// come from an LDS table [4][threads] of int4. Each slot's gradient sums go
// to its synapse's place in the partial; synapses without an entry are
// never written.
template <int NB, int JW, int RCP, bool FUSE, int RCS = 0>
__global__ __launch_bounds__(FUSE ? 512 : 1024) void ode_bwd_cl_kernel(BwdCK k) {
  static_assert(!FUSE || RCP > 0 || RCS > 0, "the fused chain needs a compile-time row count");
  static_assert(RCS == 0 || (FUSE && JW == 32 && RCP == 0), "streamed fusion: 32-column members");
  constexpr int NACC = FUSE ? (RCP > 0 ? RCP : RCS) : 1;  // synapses with gradient sums
  constexpr int PER = NB * JW;
  // Saved forward values through LDS prefetch: only where the synapse phase
  // issues no loads of its own (register-resident operands), since the load
  // counter is in order and the prefetch would delay the operands' waits.
  constexpr bool PF = FUSE && RCP > 0;
  constexpr bool CMP = FUSE && RCP == 16;
  constexpr int HPC = 16 * NACC;  // Hp of the fused forms (512 threads, 16 chunks)
  extern __shared__ float4 lds4[];
  __shared__ int gave_up;
  const int Hp = k.Hp, H = k.H, KS = k.KS, B = k.B, T = k.T, U = k.U, CP = k.CP;
  const int RC = RCP > 0 ? RCP : (RCS > 0 ? RCS : k.RC);
  // alpha/beta: [NB][Hp], or with CMP [Hp][ABS] float2, rows padded to
  // ABS = NB + 2 pairs so that the per-lane row reads of 16 lanes spread over
  // 16 bank groups instead of 4
  constexpr int ABS = CMP ? NB + 2 : NB;
  float2* ab = reinterpret_cast<float2*>(lds4);
  float* red = reinterpret_cast<float*>(ab + ABS * Hp);  // [KS][NB][JW]
  // PF: saved forward values of the cluster's rows, fetched one synapse
  // phase ahead of use: 1/den of unfold n-1, and v of slots n and n-1.
  float* pden = red + KS * NB * JW;                     // [NB][Hp]
  float* pv = pden + NB * Hp;                           // [2][NB][Hp]
  int4* slot_tab = reinterpret_cast<int4*>(pv + 2 * NB * Hp);  // CMP: [4][threads]
  auto abat = [&](int b, int col) { return CMP ? col * ABS + b : b * Hp + col; };
  const int tid = threadIdx.x, nthr = blockDim.x;
  // With JW = 64 ks is uniform across each wave; with JW = 32 a wave holds two.
  const int ks = JW == 64 ? __builtin_amdgcn_readfirstlane(tid / JW) : tid / JW;
  const int o = tid % JW;
  int p, cl;
  cluster_coords(blockIdx.x, CP, k.xcd_local != 0, p, cl);
  const int c = p * JW + o;
  const int b0 = k.R0 + cl * NB;
  const int r0 = ks * RC;
  const bool owner = ks < NB;
  const int bo = ks;
  const bool live = owner && b0 + bo < B;
  unsigned long long* xbase = k.xch + (long long)cl * 2 * CP * PER;
  const int nwords = (CP - 1) * PER;
  const long long BHp = (long long)B * Hp;
  const float C = k.neuron[c];
  if (T == 0) return;

  float4 preg[RCP > 0 ? RCP : 1];
  int nmine = 0, nslot = 0;  // CMP: this lane's entries, slots the wave runs
  // Synapse lane of this thread (chunk sks, column sc = presynaptic neuron of
  // its synapses): with CMP in balanced order (balanced_lane); the owner and
  // exchange roles keep (ks, c).
  int sks = ks, so = o;
  if constexpr (CMP) {
    int* perm = reinterpret_cast<int*>(slot_tab + (RCP / 4) * nthr);  // [threads]
    const int cnt0 = k.ccnt[c];
    const int lane_id = balanced_lane(cnt0 > ks ? (cnt0 - 1 - ks) / kCmpChunks + 1 : 0, tid,
                                      nthr, perm, perm + nthr);
    sks = lane_id / JW;
    so = lane_id - sks * JW;
    const int cnt = k.ccnt[p * JW + so];
    nmine = cnt > sks ? (cnt - 1 - sks) / kCmpChunks + 1 : 0;
    nslot = wave_max(nmine);
    int ix[RCP];
#pragma unroll
    for (int rr = 0; rr < RCP; ++rr) {
      const long long a = (long long)(sks * RCP + rr) * Hp + p * JW + so;
      preg[rr] = k.cimg[a];
      ix[rr] = k.cidx[a] * ABS * 8;
    }
#pragma unroll
    for (int q = 0; q < RCP / 4; ++q)
      slot_tab[q * nthr + tid] = make_int4(ix[4 * q], ix[4 * q + 1], ix[4 * q + 2], ix[4 * q + 3]);
  } else if constexpr (RCP > 0) {
#pragma unroll
    for (int rr = 0; rr < RCP; ++rr) preg[rr] = k.recB[(long long)(r0 + rr) * Hp + c];
  }
  const int sc = p * JW + so;  // column of this thread's synapses
  float4 gacc[NACC];
  if constexpr (FUSE) {
#pragma unroll
    for (int rr = 0; rr < NACC; ++rr) gacc[rr] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (tid == 0) gave_up = 0;

  // Owner state: g = dL/dv of (row bo, column c) after the current unfold.
  float g = 0.f, gdir = 0.f, accA = 0.f, accB = 0.f, pC = 0.f, pGv = 0.f, pA = 0.f;
  // alpha/beta of unfold n for the owned entry; accumulates the per-step and
  // per-row sums that the sensory and neuron gradients need.
  auto own_ab = [&](long long n, float den, float vk, float vk1) {
    float al = 0.f, be = 0.f;
    gdir = 0.f;
    if (live && c < H) {
      const float rden = den;  // saved 1/den
      al = g * rden;
      be = -g * vk1 * rden;
      accA += al;
      accB += be;
      pC += al * (vk - vk1);
      pGv += al * vk1;
      pA += al;
      gdir = al * C;
    }
    ab[abat(bo, c)] = make_float2(al, be);
    if (!FUSE && live) k.absave[(n * B + b0 + bo) * Hp + c] = make_float2(al, be);
  };
  auto gout_at = [&](int b, int t, int col) {
    return k.gout[(long long)(b0 + b) * k.gs.b + (long long)t * k.gs.t + (long long)col * k.gs.c];
  };
  // Word offset a = q*PER + b*JW + col-in-member of a slot -> (row, column).
  auto word_rc = [&](int a, int& b, int& col) {
    const int q = a / PER, r = a - q * PER;
    b = r / JW;
    col = q * JW + (r - b * JW);
  };

  const long long n_last = (long long)T * U - 1;
  if (owner) {
    if (live && c < H) {
      g = gout_at(bo, T - 1, c);
      if (k.ghfin != nullptr) g += k.ghfin[(long long)(b0 + bo) * H + c];
    }
    float den = 1.f, vk = 0.f, vk1 = 0.f;
    if (live) {
      const long long e = (n_last * B + b0 + bo) * Hp + c;
      den = k.densave[e];
      vk = k.vsave[e];
      vk1 = k.vsave[e + BHp];
    }
    own_ab(n_last, den, vk, vk1);
  }
  // The other members' columns for the last unfold come straight from the
  // output gradients (no exchange needed yet).
  for (int e = tid; e < nwords; e += nthr) {
    int b, col;
    word_rc(e + (e / PER >= p ? PER : 0), b, col);
    float al = 0.f, be = 0.f;
    if (b0 + b < B && col < H) {
      float gg = gout_at(b, T - 1, col);
      if (k.ghfin != nullptr) gg += k.ghfin[(long long)(b0 + b) * H + col];
      const long long ee = (n_last * B + b0 + b) * Hp + col;
      const float rden = k.densave[ee];  // saved 1/den
      al = gg * rden;
      be = -gg * k.vsave[ee + BHp] * rden;
    }
    ab[abat(b, col)] = make_float2(al, be);
  }
  // v of slot n_last, the post-unfold state of unfold n_last - 1.
  if constexpr (PF)
    rows_to_lds_fixed<NB, HPC, 512>(k.vsave + n_last * BHp, b0, B, pv + (n_last & 1) * NB * HPC,
                                    tid);
  lds_barrier();

  float cvi[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
    cvi[b] = b0 + b < B ? k.vsave[(n_last * B + b0 + b) * Hp + sc] : 0.f;

  for (long long n = n_last; n >= 0; --n) {
    const int t = (int)(n / U), u = (int)(n - (long long)t * U);
    // PF: the saved values that unfold n-1's alpha/beta need, in flight
    // during the synapse phase (v of slot n is already resident).
    if constexpr (PF) {
      if (n > 0) {
        rows_to_lds_fixed<NB, HPC, 512>(k.densave + (n - 1) * BHp, b0, B, pden, tid);
        rows_to_lds_fixed<NB, HPC, 512>(k.vsave + (n - 1) * BHp, b0, B,
                                        pv + ((n - 1) & 1) * NB * HPC, tid);
      }
    }
    // Output gradient entering at this step boundary (owner only).
    float gnext = 0.f;
    if (n > 0 && u == 0 && live && c < H) gnext = gout_at(bo, t - 1, c);
    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.f;
    if constexpr (FUSE && RCS > 0) {
      // Wave w holds chunks 2w (lower half) and 2w + 1 (upper half).
      const int srow0 = __builtin_amdgcn_readfirstlane((tid >> 6) * 2 * RCS);
      const int lane_bytes = c * 16 + ((tid >> 5) & 1) * RCS * Hp * 16;
      const __amdgpu_buffer_rsrc_t rsB = image_rsrc(k.recB, (long long)Hp * Hp * 16);
      chain_fused_stream<NB, RCS>(rsB, lane_bytes, srow0, r0, Hp, ab, cvi, acc, gacc);
    } else if constexpr (CMP) {
      // Wave-uniform slot count: the skipped pairs branch around.
#pragma unroll
      for (int q = 0; q < RCP / 4; ++q) {
        if (4 * q < nslot) {
          const int4 of = slot_tab[q * nthr + tid];
          const int off[4] = {of.x, of.y, of.z, of.w};
#pragma unroll
          for (int h = 0; h < 4; h += 2) {
            if (4 * q + h < nslot) {
#pragma unroll
              for (int i = 0; i < 2; ++i) {
                const int rr = 4 * q + h + i;
                bwd_synapse_cmp<NB>(preg[rr], ab, off[h + i], cvi, acc, gacc[rr]);
                asm volatile("" : "+v"(gacc[rr].x), "+v"(gacc[rr].y), "+v"(gacc[rr].z),
                             "+v"(gacc[rr].w));
              }
            }
          }
        }
      }
    } else if constexpr (FUSE) {
#pragma unroll
      for (int rr = 0; rr < RCP; ++rr) {
        bwd_synapse<NB, true>(preg[rr], ab, Hp, r0 + rr, cvi, acc, gacc[rr]);
        // Pin the accumulators here: otherwise the compiler sinks these sums
        // past the barrier and keeps every synapse's temporaries alive.
        asm volatile("" : "+v"(gacc[rr].x), "+v"(gacc[rr].y), "+v"(gacc[rr].z), "+v"(gacc[rr].w));
      }
    } else if constexpr (RCP > 0) {
#pragma unroll
      for (int rr = 0; rr < RCP; ++rr) bwd_synapse_folded<NB>(preg[rr], ab, Hp, r0 + rr, cvi, acc);
    } else {
      static_assert(FUSE || RCP > 0 || JW == 64, "streamed operands need wave-uniform rows");
      const __amdgpu_buffer_rsrc_t rsB = image_rsrc(k.recB, (long long)Hp * Hp * 16);
      stream_rows(rsB, c * 16, r0, RC, Hp, [&](const float4 pw, int r) {
        bwd_synapse_folded<NB>(pw, ab, Hp, r, cvi, acc);
      });
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) red[(sks * NB + b) * JW + so] = acc[b];
    // Without PF: the saved values of unfold n-1, requested now and consumed
    // after the exchange, whose wait covers their latency.
    float nden = 1.f, nvk = 0.f, nvk1 = 0.f;
    if constexpr (PF) {
      // The prefetched blocks have long arrived; make them visible to all waves.
      wait_vm();
    } else if (n > 0) {
#pragma unroll
      for (int b = 0; b < NB; ++b)
        acc[b] = b0 + b < B ? k.vsave[((n - 1) * B + b0 + b) * Hp + c] : 0.f;
      if (live) {
        const long long e = ((n - 1) * B + b0 + bo) * Hp + c;
        nden = k.densave[e];
        nvk = k.vsave[e];
        nvk1 = k.vsave[e + BHp];
      }
    }
    lds_barrier();
    // ab and red of unfold n are consumed: publish dL/dv^n and build unfold
    // n-1's alpha/beta.
    const unsigned tag = (unsigned)n;
    unsigned long long* slot = xbase + (long long)(tag & 1) * CP * PER;
    if (owner) {
      const float s = ks_sum_wide(red + bo * JW + o, NB * JW, KS);
      g = c < H ? fmaf(kNegLn2, s, gdir) : 0.f;
      // Publish first: the partners wait on it, the other stores on nothing.
      if (n > 0) {
        g += gnext;
        xch_put(slot + p * PER + bo * JW + o, g, tag);
      }
      if (u == 0 && live) {
        const long long e = ((long long)(b0 + bo) * T + t) * Hp + c;
        k.dsn[e] = accA;
        k.dsd[e] = accB;
      }
      if (u == 0) accA = accB = 0.f;
    }
    if (n > 0 && PF) {
      const float* vn = pv + (n & 1) * NB * Hp;         // v of slot n
      const float* vm = pv + ((n - 1) & 1) * NB * Hp;   // v of slot n-1
      const bool ok = xch_gather<PER, kXchBatch>(
          slot, p, nwords, tid, nthr, tag, k.spin, [](int, int) {},
          [&](int, int a, float gg) {
            int b, col;
            word_rc(a, b, col);
            float al = 0.f, be = 0.f;
            if (b0 + b < B && col < H) {
              const float rden = pden[b * Hp + col];  // saved 1/den
              al = gg * rden;
              be = -gg * vn[b * Hp + col] * rden;
            }
            ab[abat(b, col)] = make_float2(al, be);
          });
      if (!ok) gave_up = 1;
      if (owner) own_ab(n - 1, pden[bo * Hp + c], vm[bo * Hp + c], vn[bo * Hp + c]);
#pragma unroll
      for (int b = 0; b < NB; ++b) cvi[b] = b0 + b < B ? vm[b * Hp + sc] : 0.f;
    } else if (n > 0) {
      // Words in flight per thread: 4 for the streamed fused chain (7.5 words
      // per thread at Hp = 512; two poll rounds instead of four), else 2.
      constexpr int XB = (FUSE && RCS > 0) ? 4 : kXchBatch;
      float pden_[XB], pvk1[XB];
      const bool ok = xch_gather<PER, XB>(
          slot, p, nwords, tid, nthr, tag, k.spin,
          [&](int x, int a) {
            int b, col;
            word_rc(a, b, col);
            pden_[x] = 1.f;
            pvk1[x] = 0.f;
            if (b0 + b < B) {
              const long long ee = ((n - 1) * B + b0 + b) * Hp + col;
              pden_[x] = k.densave[ee];
              pvk1[x] = k.vsave[ee + BHp];
            }
          },
          [&](int x, int a, float gg) {
            int b, col;
            word_rc(a, b, col);
            float al = 0.f, be = 0.f;
            if (b0 + b < B && col < H) {
              const float rden = pden_[x];  // saved 1/den
              al = gg * rden;
              be = -gg * pvk1[x] * rden;
            }
            ab[abat(b, col)] = make_float2(al, be);
          });
      if (!ok) gave_up = 1;
      if (owner) own_ab(n - 1, nden, nvk, nvk1);
#pragma unroll
      for (int b = 0; b < NB; ++b) cvi[b] = acc[b];
    }
    lds_barrier();
    if (gave_up) {
      if (k.gstate != nullptr && live && c < H)
        k.gstate[(long long)(b0 + bo) * H + c] = __builtin_nanf("");
      if (tid == 0) __hip_atomic_store(k.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
  }
  if (live) {
    if (k.gstate != nullptr && c < H) k.gstate[(long long)(b0 + bo) * H + c] = g;
    float* np = k.npart + (long long)(b0 + bo) * 3 * Hp + c;
    np[0] = pC;
    np[Hp] = pGv;
    np[2 * Hp] = pA;
  }
  if constexpr (FUSE) {
    // This cluster's share of the recurrent parameter gradients for synapses
    // (i = sc, j = r0 + rr), layout [cluster][4][i][j] as rec_grad_kernel's.
    const long long HH = (long long)Hp * Hp;
    if constexpr (CMP) {
      float* out = k.rpart + (long long)(k.R0 / NB + cl) * 4 * HH + (long long)sc * Hp;
#pragma unroll
      for (int rr = 0; rr < NACC; ++rr) {
        if (rr < nmine) {
          const int j = k.cidx[(long long)(sks * RCP + rr) * Hp + sc];
          out[j] = gacc[rr].x;
          out[HH + j] = gacc[rr].y;
          out[2 * HH + j] = gacc[rr].z;
          out[3 * HH + j] = gacc[rr].w;
        }
      }
    } else {
      float* out = k.rpart + (long long)(k.R0 / NB + cl) * 4 * HH + (long long)c * Hp + r0;
#pragma unroll
      for (int rr = 0; rr < NACC; ++rr) {
        out[rr] = gacc[rr].x;
        out[HH + rr] = gacc[rr].y;
        out[2 * HH + rr] = gacc[rr].z;
        out[3 * HH + rr] = gacc[rr].w;
      }
    }
  }
}

// The compacted fused cluster chain (register-resident operands, Hp = 256,
// 32-column members of 512 threads) with its NB >= 2 rows in two groups of
// NB/2 that take turns, as ode_fwd_cl2_kernel does for the forward. Phase
// (g, n) runs group g's synapses at unfold n (reverse time). After the
// phase's one barrier the owners of group g (waves of ks < NB, which the SIMDs
// issue first) reduce dL/dv^n of their columns and publish it (tag n) at the
// start of the next phase, and that next phase, which gathers the partners'
// words of group g halfway through its slots, rebuilds group g's alpha/beta
// of unfold n-1 before its barrier. The saved 1/den and v of the cluster's
// rows come through LDS prefetches issued in group 1's phases two phases
// ahead of use (after that phase's word loads, so the word waits do not wait
// for them): 1/den of two unfolds and v of three slots. The four gradient
// sums of each synapse take the rows in the same order as the one-group
// kernel; a slot's operands are (x, y, E, w x), w factored out of dL/darg
// (bwd_synapse_cmpe), and its alpha/beta row offset stays in a register.
template <int NB>
__global__ __launch_bounds__(512) void ode_bwd_cl2_kernel(BwdCK k) {
  static_assert(NB == 2 || NB == 4 || NB == 8, "two groups of rows");
  constexpr int JW = 32, RCP = 16, HB = NB / 2, PER = NB * JW, PERG = HB * JW;
  constexpr int ABS = NB + 2;  // padded alpha/beta rows, as in ode_bwd_cl_kernel
  constexpr int HPC = 16 * RCP;  // Hp = 256
  constexpr int XW = 2;          // gather words per thread and group: (CP-1)*PERG <= 2*512
  extern __shared__ float4 lds4[];
  __shared__ int gave_up;
  const int Hp = k.Hp, H = k.H, KS = k.KS, B = k.B, T = k.T, U = k.U, CP = k.CP;
  float2* ab = reinterpret_cast<float2*>(lds4);                  // [Hp][ABS]
  float* red = reinterpret_cast<float*>(ab + ABS * Hp);         // [2][KS][HB][JW]
  float* pden = red + 2 * KS * HB * JW;                         // [2][NB][Hp] by unfold parity
  float* pv = pden + 2 * NB * Hp;                               // [3][NB][Hp] by slot mod 3
  // [4][threads] int4 of the compacted kernels' slot table, of which this
  // kernel only uses the space after it (balanced_lane's scratch)
  int4* slot_tab = reinterpret_cast<int4*>(pv + 3 * NB * Hp);
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int ks = tid / JW, o = tid % JW;
  int p, cl;
  cluster_coords(blockIdx.x, CP, k.xcd_local != 0, p, cl);
  const int c = p * JW + o;
  const int b0 = k.R0 + cl * NB;
  const bool owner = ks < NB;
  const int bo = ks, og = ks / HB;
  const bool live = owner && b0 + bo < B;
  unsigned long long* xbase = k.xch + (long long)cl * 2 * CP * PER;
  const long long BHp = (long long)B * Hp;
  const float C = k.neuron[c];
  if (T == 0) return;
  auto pden_at = [&](long long m) { return pden + (m & 1) * NB * Hp; };
  auto pv_at = [&](long long m) { return pv + (m % 3) * NB * Hp; };
  // v slot r (an unfold index mod 3, kept by the loop instead of divided)
  auto pv_slot = [&](int r) { return pv + r * NB * Hp; };
  auto mod3_next = [](int r) { return r == 2 ? 0 : r + 1; };
  auto mod3_prev = [](int r) { return r == 0 ? 2 : r - 1; };

  float4 preg[RCP];
  int ix[RCP];  // slot row offsets, in registers
  int nmine, nslot, sks, so;
  {
    int* perm = reinterpret_cast<int*>(slot_tab + (RCP / 4) * nthr);
    const int cnt0 = k.ccnt[c];
    const int lane_id = balanced_lane(cnt0 > ks ? (cnt0 - 1 - ks) / kCmpChunks + 1 : 0, tid,
                                      nthr, perm, perm + nthr);
    sks = lane_id / JW;
    so = lane_id - sks * JW;
    const int cnt = k.ccnt[p * JW + so];
    nmine = cnt > sks ? (cnt - 1 - sks) / kCmpChunks + 1 : 0;
    nslot = wave_max(nmine);
#pragma unroll
    for (int rr = 0; rr < RCP; ++rr) {
      const long long a = (long long)(sks * RCP + rr) * Hp + p * JW + so;
      // image operands (x, y, w E, w) -> (x, y, E, w x); an entry with
      // w = 0 (a padding slot) contributes nothing either way
      const float4 q = k.cimg[a];
      preg[rr] = make_float4(q.x, q.y, q.w != 0.f ? q.z / q.w : 0.f, q.w * q.x);
      ix[rr] = k.cidx[a] * ABS * 8;
    }
  }
  const int sc = p * JW + so;
  float4 gacc[RCP];
#pragma unroll
  for (int rr = 0; rr < RCP; ++rr) gacc[rr] = make_float4(0.f, 0.f, 0.f, 0.f);
  if (tid == 0) gave_up = 0;

  // Owner state, as in ode_bwd_cl_kernel.
  float g = 0.f, gdir = 0.f, accA = 0.f, accB = 0.f, pC = 0.f, pGv = 0.f, pA = 0.f;
  auto own_ab = [&](float den, float vk, float vk1) {
    float al = 0.f, be = 0.f;
    gdir = 0.f;
    if (live && c < H) {
      al = g * den;  // saved 1/den
      be = -g * vk1 * den;
      accA += al;
      accB += be;
      pC += al * (vk - vk1);
      pGv += al * vk1;
      pA += al;
      gdir = al * C;
    }
    ab[c * ABS + bo] = make_float2(al, be);
  };
  auto gout_at = [&](int b, int t, int col) {
    return k.gout[(long long)(b0 + b) * k.gs.b + (long long)t * k.gs.t + (long long)col * k.gs.c];
  };
  auto prefetch = [&](long long m) {  // 1/den of unfold m, v of slot m
    rows_to_lds_fixed<NB, HPC, 512>(k.densave + m * BHp, b0, B, pden_at(m), tid);
    rows_to_lds_fixed<NB, HPC, 512>(k.vsave + m * BHp, b0, B, pv_at(m), tid);
  };

  const long long n_last = (long long)T * U - 1;
  // Unfold n_last's alpha/beta of every column from the output gradients.
  if (owner) {
    if (live && c < H) {
      g = gout_at(bo, T - 1, c);
      if (k.ghfin != nullptr) g += k.ghfin[(long long)(b0 + bo) * H + c];
    }
    float den = 1.f, vk = 0.f, vk1 = 0.f;
    if (live) {
      const long long e = (n_last * B + b0 + bo) * Hp + c;
      den = k.densave[e];
      vk = k.vsave[e];
      vk1 = k.vsave[e + BHp];
    }
    own_ab(den, vk, vk1);
  }
  for (int e = tid; e < (CP - 1) * PER; e += nthr) {
    const int q = e / PER, r = e - q * PER, b = r / JW;
    const int col = (q + (q >= p ? 1 : 0)) * JW + (r - b * JW);
    float al = 0.f, be = 0.f;
    if (b0 + b < B && col < H) {
      float gg = gout_at(b, T - 1, col);
      if (k.ghfin != nullptr) gg += k.ghfin[(long long)(b0 + b) * H + col];
      const long long ee = (n_last * B + b0 + b) * Hp + col;
      const float rden = k.densave[ee];
      al = gg * rden;
      be = -gg * k.vsave[ee + BHp] * rden;
    }
    ab[col * ABS + b] = make_float2(al, be);
  }
  // The prefetched rows the first three phases read: v of slots n_last and
  // n_last - 1, 1/den of unfold n_last - 1.
  rows_to_lds_fixed<NB, HPC, 512>(k.vsave + n_last * BHp, b0, B, pv_at(n_last), tid);
  if (n_last > 0) prefetch(n_last - 1);
  wait_vm();
  lds_barrier();

  // This thread's gather words (x < XW): partner member, row of the group, column.
  int gm[XW], gr[XW], gcl[XW];
  bool gth[XW];
#pragma unroll
  for (int x = 0; x < XW; ++x) {
    const int e = tid + x * nthr;
    // With two or more rows per group the word count (CP - 1) * PERG is a
    // multiple of 64, so a wave gathers all its words or none: a scalar
    // branch instead of a lane mask.
    if constexpr (HB >= 2)
      gth[x] = __builtin_amdgcn_readfirstlane(e) < (CP - 1) * PERG;
    else
      gth[x] = e < (CP - 1) * PERG;
    const int q = e / PERG, r = e - q * PERG;
    gm[x] = q + (q >= p ? 1 : 0);
    gr[x] = r / JW;
    gcl[x] = gm[x] * JW + (r - gr[x] * JW);
  }
  bool pend = false;  // owners: their group's finish is due
  long long pn = 0;
  int pn3 = 0, pt = 0, pu = 0;  // pn mod 3, its step and unfold within the step
  float gnext = 0.f;
  // step t, unfold u within it and n mod 3, stepped with n
  int t = T - 1, u = U - 1, n3 = (int)(n_last % 3);
  for (long long n = n_last; n >= 0; --n) {
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      // (e) the owners of the previous phase's group: dL/dv^{pn}, published
      // for the partners' alpha/beta of unfold pn - 1.
      bool own_next = false;
      if (pend) {
        pend = false;
        const float* rg = red + og * KS * HB * JW;
        const float s = ks_sum_wide(rg + (bo - og * HB) * JW + o, HB * JW, KS);
        g = c < H ? fmaf(kNegLn2, s, gdir) : 0.f;
        if (pn > 0) {
          g += gnext;
          const unsigned tag = (unsigned)pn;
          xch_put(xbase + (long long)(tag & 1) * CP * PER + p * PER + bo * JW + o, g, tag);
          own_next = true;
        }
        if (pu == 0 && live) {
          const long long e = ((long long)(b0 + bo) * T + pt) * Hp + c;
          k.dsn[e] = accA;
          k.dsd[e] = accB;
        }
        if (pu == 0) accA = accB = 0.f;
      }
      // The output gradient entering at this unfold's step boundary.
      if (owner && og == gi) gnext = (n > 0 && u == 0 && live && c < H) ? gout_at(bo, t - 1, c) : 0.f;
      // (a) group gi's synapses at unfold n; the other group's newest words
      // are loaded halfway: group 0's dL/dv^n while running group 1, group
      // 1's dL/dv^{n+1} while running group 0.
      const int gg = 1 - gi;
      const long long gtag = gi == 1 ? n : n + 1;
      const bool need = gi == 1 ? n > 0 : n < n_last;
      const long long am = gtag - 1;  // the unfold whose alpha/beta the words rebuild
      unsigned long long* gslot = xbase + (long long)(gtag & 1) * CP * PER;
      unsigned long long w[XW];
      // 1/den and v^{am+1} of the gathered words' rows and columns, read
      // from LDS when the word loads are issued, so that the rebuild after
      // the poll does not wait for LDS
      float rdn[XW], rvk[XW], odn = 0.f, ovk = 0.f, ovk1 = 0.f;
      const float* dn = pden_at(am);
      const float* vk1 = pv_slot(gi == 1 ? n3 : mod3_next(n3));  // slot am + 1 = gtag
      float cvi[HB], acc[HB];
      // The slot count, opaque to the compiler here: otherwise it keeps the
      // slot branches' conditions as lane masks across the loop, which spill
      // and are reloaded every phase.
      int nsl = nslot;
      asm volatile("" : "+s"(nsl));
      const float* vn = pv_slot(n3);
#pragma unroll
      for (int b = 0; b < HB; ++b) {
        cvi[b] = b0 + gi * HB + b < B ? vn[(gi * HB + b) * Hp + sc] : 0.f;
        acc[b] = 0.f;
      }
#pragma unroll
      for (int q = 0; q < RCP / 4; ++q) {
        if (q == RCP / 8) {
#pragma unroll
          for (int x = 0; x < XW; ++x)
            if (need && gth[x])
              w[x] = xch_get(gslot + gm[x] * PER + (gg * HB + gr[x]) * JW + (gcl[x] - gm[x] * JW));
#pragma unroll
          for (int x = 0; x < XW; ++x) {
            rdn[x] = rvk[x] = 0.f;
            if (need && gth[x]) {
              const int e = (gg * HB + gr[x]) * Hp + gcl[x];
              rdn[x] = dn[e];
              rvk[x] = vk1[e];
            }
          }
          // the owners' own entry likewise
          if (own_next) {
            odn = pden_at(pn - 1)[bo * Hp + c];
            ovk = pv_slot(mod3_prev(pn3))[bo * Hp + c];
            ovk1 = pv_slot(pn3)[bo * Hp + c];
          }
          // group 1's phases issue the prefetch of unfold n - 2, after the
          // word loads
          if (gi == 1 && n >= 2) {
            // 1/den of unfold n - 2, v of slot n - 2 (n - 2 = n + 1 mod 3)
            rows_to_lds_fixed<NB, HPC, 512>(k.densave + (n - 2) * BHp, b0, B, pden_at(n), tid);
            rows_to_lds_fixed<NB, HPC, 512>(k.vsave + (n - 2) * BHp, b0, B,
                                            pv_slot(mod3_next(n3)), tid);
          }
        }
        if (4 * q < nsl) {
          const int off[4] = {ix[4 * q], ix[4 * q + 1], ix[4 * q + 2], ix[4 * q + 3]};
#pragma unroll
          for (int h = 0; h < 4; h += 2) {
            if (4 * q + h < nsl) {
#pragma unroll
              for (int i = 0; i < 2; ++i) {
                const int rr = 4 * q + h + i;
                bwd_synapse_cmpe<HB>(preg[rr], ab + gi * HB, off[h + i], cvi, acc, gacc[rr]);
                asm volatile("" : "+v"(gacc[rr].x), "+v"(gacc[rr].y), "+v"(gacc[rr].z),
                             "+v"(gacc[rr].w));
              }
            }
          }
        }
      }
      // (b) the group's partials
      float* rgi = red + gi * KS * HB * JW;
#pragma unroll
      for (int b = 0; b < HB; ++b) rgi[(sks * HB + b) * JW + so] = acc[b];
      // (c) the other group's alpha/beta of unfold am from the partners'
      // words, and the owners' own entry of the group they just finished
      if (k.spin <= 0) {
        gave_up = 1;  // a budget of 0: give up at the first wait, as xch_gather does
      } else if (need) {
#pragma unroll
        for (int x = 0; x < XW; ++x) {
          if (!gth[x]) continue;
          const long long t0 = wall_clock64();
          bool ok = true;
          unsigned long long* wa =
              gslot + gm[x] * PER + (gg * HB + gr[x]) * JW + (gcl[x] - gm[x] * JW);
          while ((unsigned)(w[x] >> 32) != (unsigned)gtag) {
            if (wall_clock64() - t0 > k.spin) {
              ok = false;
              break;
            }
            w[x] = xch_get(wa);
          }
          if (!ok) {
            gave_up = 1;
            continue;
          }
          const int b = gg * HB + gr[x], col = gcl[x];
          float al = 0.f, be = 0.f;
          if (b0 + b < B && col < H) {
            const float gv = __uint_as_float((unsigned)w[x]);
            const float rden = rdn[x];
            al = gv * rden;
            be = -gv * rvk[x] * rden;
          }
          ab[col * ABS + b] = make_float2(al, be);
        }
      }
      if (own_next) own_ab(odn, ovk, ovk1);
      // the prefetch issued in the previous (group 1) phase, visible to
      // every wave after this barrier
      if (gi == 0) wait_vm();
      lds_barrier();
      if (gave_up) {
        if (k.gstate != nullptr && live && c < H)
          k.gstate[(long long)(b0 + bo) * H + c] = __builtin_nanf("");
        if (tid == 0) __hip_atomic_store(k.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
      }
      if (owner && og == gi) {
        pn = n;
        pn3 = n3;
        pt = t;
        pu = u;
        pend = true;
      }
    }
    n3 = mod3_prev(n3);
    if (--u < 0) {
      u = U - 1;
      --t;
    }
  }
  // group 1's finish of unfold 0 (nothing is published at unfold 0)
  if (pend) {
    const float* rg = red + og * KS * HB * JW;
    const float s = ks_sum_wide(rg + (bo - og * HB) * JW + o, HB * JW, KS);
    g = c < H ? fmaf(kNegLn2, s, gdir) : 0.f;
    if (live) {
      const long long e = ((long long)(b0 + bo) * T) * Hp + c;
      k.dsn[e] = accA;
      k.dsd[e] = accB;
    }
  }
  if (live) {
    if (k.gstate != nullptr && c < H) k.gstate[(long long)(b0 + bo) * H + c] = g;
    float* np = k.npart + (long long)(b0 + bo) * 3 * Hp + c;
    np[0] = pC;
    np[Hp] = pGv;
    np[2 * Hp] = pA;
  }
  // This cluster's share of the recurrent parameter gradients, layout
  // [cluster][4][i][j], as ode_bwd_cl_kernel writes it.
  const long long HH = (long long)Hp * Hp;
  float* out = k.rpart + (long long)(k.R0 / NB + cl) * 4 * HH + (long long)sc * Hp;
  // The image entries are indexed again from a copy of sks the compiler
  // cannot match with the preload's, so that it does not keep the preload's
  // addresses (or every w) live across the loop.
  int sks_end = sks;
  asm volatile("" : "+v"(sks_end));
#pragma unroll
  for (int rr = 0; rr < RCP; ++rr) {
    if (rr < nmine) {
      const long long a = (long long)(sks_end * RCP + rr) * Hp + sc;
      const int j = k.cidx[a];
      const float w = k.cimg[a].w;  // the factor the last two sums left out
      out[j] = gacc[rr].x;
      out[HH + j] = gacc[rr].y;
      out[2 * HH + j] = gacc[rr].z * w;
      out[3 * HH + j] = gacc[rr].w * w;
    }
  }
}

// Clears the cluster exchange words (tag 0) and the status word before a
// cluster launch; a kernel rather than a memset so that graph capture
// records a kernel node.
__global__ __launch_bounds__(256) void clear_words_kernel(unsigned long long* w, long long n,
                                                          int* status) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) w[i] = 0ULL;
  if (i == 0 && status != nullptr) *status = 0;
}


// Segment list fill/copy (see FillList). Grid-stride over the concatenated
// segments; with a gate, every thread first reads it and leaves when it is 0.
__global__ __launch_bounds__(256) void fill_list_kernel(FillList fl) {
  if (fl.gate != nullptr) {
    if (__hip_atomic_load(fl.gate, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) return;
    if (blockIdx.x == 0 && threadIdx.x == 0)
      __hip_atomic_store(&g_fault, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const long long stride = (long long)gridDim.x * blockDim.x;
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  long long base = 0;
  for (int sgi = 0; sgi < fl.nseg; ++sgi) {
    const FillSeg sg = fl.seg[sgi];
    for (; i < base + sg.n; i += stride) {
      const long long e = i - base;
      sg.dst[e] = sg.src != nullptr ? sg.src[e] : fl.value;
    }
    base += sg.n;
  }
}

// ---------------------------------------------------------------------------
// Template dispatch helpers.
// ---------------------------------------------------------------------------
size_t fwd_lds_bytes(const Plan& p) { return (size_t)fwd_lds(p); }
size_t bwd_lds_bytes(const Plan& p) { return (size_t)chain_lds(p); }

template <int NB>
hipError_t fwd_by_rcp(const Plan& p, const FwdK& a, hipStream_t s) {
  const dim3 grid((p.B + NB - 1) / NB), block(p.Hp * p.KS);
  const size_t lds = fwd_lds_bytes(p);
  const int rcp = (p.RC == 4 || p.RC == 8 || p.RC == 16) ? p.RC : 0;
  if constexpr (NB == 1) {
    if (row_wave128_fwd(p)) {
      LTC_LAUNCH((ode_fwd_row_wave_kernel<128>), grid, dim3(512), lds, s, a);
      return hipGetLastError();
    }
    if (row_kernels(p)) {
      // the launch plan gives every single-row forward at Hp = 64 RC = 16
      if (rcp != 16) return hipErrorInvalidValue;
      LTC_LAUNCH((ode_fwd_row_wave_kernel<64>), grid, dim3(256), lds, s, a);
      return hipGetLastError();
    }
  }
  switch (rcp) {
    case 4: LTC_LAUNCH((ode_fwd_kernel<NB, 4>), grid, block, lds, s, a); break;
    case 8: LTC_LAUNCH((ode_fwd_kernel<NB, 8>), grid, block, lds, s, a); break;
    case 16: LTC_LAUNCH((ode_fwd_kernel<NB, 16>), grid, block, lds, s, a); break;
    default: LTC_LAUNCH((ode_fwd_kernel<NB, 0>), grid, block, lds, s, a); break;
  }
  return hipGetLastError();
}

template <int NB>
hipError_t bwd_by_rcp(const Plan& p, const BwdK& a, hipStream_t s) {
  const dim3 grid((p.B + NB - 1) / NB), block(p.Hp * p.KSB);
  const size_t lds = bwd_lds_bytes(p);
  const int rcp = (p.RCB == 4 || p.RCB == 8 || p.RCB == 16) ? p.RCB : 0;
#define LTC_BWD(R, F) LTC_LAUNCH((ode_bwd_kernel<NB, R, F>), grid, block, lds, s, a)
  if constexpr (NB == 1) {
    if (row_kernels(p)) {
      // the launch plan gives every single-row chain at Hp = 64 FUSE, RCB = 8
      if (!p.FUSE || rcp != 8) return hipErrorInvalidValue;
      if (p.H == 64)
        LTC_LAUNCH((ode_bwd_row_wave_kernel<true>), grid, block, lds, s, a);
      else
        LTC_LAUNCH((ode_bwd_row_wave_kernel<false>), grid, block, lds, s, a);
      return hipGetLastError();
    }
    if (row_wave128_bwd(p)) {
      const RecC none{};
      if (p.H == 128)
        LTC_LAUNCH((ode_bwd_row_wave128_kernel<true>), grid, dim3(512), lds, s, a, none);
      else
        LTC_LAUNCH((ode_bwd_row_wave128_kernel<false>), grid, dim3(512), lds, s, a, none);
      return hipGetLastError();
    }
  }
  if (p.FUSE) {
    // Only the spill-free pairs of ode_fuse_ok() are instantiated.
    if constexpr (ode_fuse_ok(NB, 8)) {
      if (rcp == 8) LTC_BWD(8, true);
    }
    if constexpr (ode_fuse_ok(NB, 4)) {
      if (rcp == 4) LTC_BWD(4, true);
    }
  } else {
    switch (rcp) {
      case 4: LTC_BWD(4, false); break;
      case 8: LTC_BWD(8, false); break;
      case 16: LTC_BWD(16, false); break;
      default: LTC_BWD(0, false); break;
    }
  }
#undef LTC_BWD
  return hipGetLastError();
}

// Cluster path: grid NCL * CP, 64 * KS threads. The forward keeps its operands
// in registers when RC = 16, otherwise they stream (RC is a multiple of 8).
size_t fwd_cl_lds_bytes(const Plan& p) { return (size_t)cluster_fwd_lds(p); }
size_t bwd_cl_lds_bytes(const Plan& p) { return (size_t)cluster_bwd_lds(p); }

// Clears the exchange words before a cluster launch; the status word only
// before the first launch of a call, so a give-up in an earlier launch of the
// call stays reported.
hipError_t clear_cluster(const Plan& p, const ClusterBuf& cb, bool bwd, hipStream_t s,
                         bool status = true) {
  const long long n = bwd ? cluster_words_bwd(p) : cluster_words(p);
  LTC_LAUNCH(clear_words_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
             cb.xch, n, status ? cb.status : nullptr);
  return hipGetLastError();
}

template <int NB>
hipError_t fwd_cl_by_rcp(const Plan& p, const FwdCK& a, hipStream_t s) {
  const dim3 grid(p.NCL * p.CP), block(64 * p.KS);
  const size_t lds = fwd_cl_lds_bytes(p);
  if (p.RC == 16 && NB >= 2)
    LTC_LAUNCH((ode_fwd_cl2_kernel<(NB >= 2 ? NB : 2)>), grid, block, lds, s, a);
  else if (p.RC == 16)
    LTC_LAUNCH((ode_fwd_cl_kernel<NB, 16>), grid, block, lds, s, a);
  else
    LTC_LAUNCH((ode_fwd_cl_kernel<NB, 0>), grid, block, lds, s, a);
  return hipGetLastError();
}

template <int NB>
hipError_t bwd_cl_by_rcp(const Plan& p, const BwdCK& a, hipStream_t s) {
  const dim3 grid(p.NCLB * p.CPB), block(p.JWB * p.KSB);
  const size_t lds = bwd_cl_lds_bytes(p);
  if (p.FUSE) {
    // 32-column members, 512 threads: 16 register-resident synapses each
    // (Hp = 256) or 32 streamed ones (Hp = 512).
    if (p.JWB != 32 || p.KSB != 16) return hipErrorInvalidConfiguration;
    if (p.RCB == 16 && NB >= 2)
      LTC_LAUNCH((ode_bwd_cl2_kernel<(NB >= 2 ? NB : 2)>), grid, block, lds, s, a);
    else if (p.RCB == 16)
      LTC_LAUNCH((ode_bwd_cl_kernel<NB, 32, 16, true>), grid, block, lds, s, a);
    else if (p.RCB == 32)
      LTC_LAUNCH((ode_bwd_cl_kernel<NB, 32, 0, true, 32>), grid, block, lds, s, a);
    else
      return hipErrorInvalidConfiguration;
  } else {
    // Streamed operands (a register-resident form spilled at 1024 threads
    // and measured slower).
    LTC_LAUNCH((ode_bwd_cl_kernel<NB, 64, 0, false>), grid, block, lds, s, a);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_prep(const Plan& p, const RawParams& rp, const Prepped& pp, bool bwd,
                       hipStream_t s, int segs) {
  const long long total = ((segs & kPrepRec) ? (long long)p.Hp * p.Hp : 0) +
                          ((segs & kPrepSens) ? (long long)p.Dp * p.Hp : 0) +
                          ((segs & kPrepNeuron) ? 3LL * p.Hp : 0);
  if (total == 0) return hipSuccess;
  const int nflat = (int)((total + 255) / 256);
  const bool rec = (segs & kPrepRec) != 0;
  const int ncmp = (cmp_columns(pp, p.Hp, p.Dp, rec, rec && bwd, (segs & kPrepSens) != 0) + 3) / 4;
  LTC_LAUNCH(prep_kernel, dim3((unsigned)(nflat + ncmp)), dim3(256), 0, s, rp, pp, p.H,
                     p.D, p.Hp, p.Dp, bwd ? (p.FUSE ? 1 : 2) : 0, segs, nflat, cmp_chunks_fwd(p),
                     cmp_chunks_bwd(p));
  return hipGetLastError();
}

hipError_t launch_fill(const FillList& fl, hipStream_t s) {
  long long total = 0;
  for (int i = 0; i < fl.nseg; ++i) total += fl.seg[i].n;
  if (total == 0) return hipSuccess;
  // A gated fill (after a cluster launch) usually does nothing: a small grid
  // keeps its cost to one short launch.
  const long long cap = fl.gate != nullptr ? 256 : 2048;
  long long blocks = (total + 255) / 256;
  if (blocks > cap) blocks = cap;
  LTC_LAUNCH(fill_list_kernel, dim3((unsigned)blocks), dim3(256), 0, s, fl);
  return hipGetLastError();
}

hipError_t device_fault(int* value, bool clear) {
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return e;
  int v = 0;
  e = hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_fault), sizeof(int), 0, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return e;
  if (clear && v != 0) {
    const int zero = 0;
    e = hipMemcpyToSymbol(HIP_SYMBOL(g_fault), &zero, sizeof(int), 0, hipMemcpyHostToDevice);
    if (e != hipSuccess) return e;
  }
  *value = v;
  return hipSuccess;
}

hipError_t launch_copy_rows(const float* src, long long src_ld, float* dst, long long dst_ld,
                            long long rows, int cols, hipStream_t s) {
  const long long n = rows * dst_ld;
  if (n == 0) return hipSuccess;
  LTC_LAUNCH(copy_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src,
                     src_ld, dst, dst_ld, rows, cols);
  return hipGetLastError();
}

hipError_t launch_sens_fwd(const Plan& p, const float* x, Strides3 xs, const Prepped& pp,
                           float* sn, float* sd, hipStream_t s) {
  const int BT = p.B * p.T;
  const int hb = p.Hp / 64;
  const dim3 block(256);
  const SensGeom geo = sens_fwd_geom(p);
  const bool split_d = geo.split_d;
  const int rpw = geo.rpw, rows_of = split_d ? 1 : 4;
  const dim3 grid(hb, (BT + rows_of * rpw - 1) / (rows_of * rpw));
#define LTC_SENS(R, DSV)                                                                        \
  do {                                                                                          \
    if (pp.sF != nullptr)                                                                       \
      LTC_LAUNCH((sens_fwd_cmp_kernel<R, DSV>), grid, block, 0, s, x, xs, p.T, p.D, BT, \
                         p.Hp, pp.sF, pp.sFi, pp.sFn, sn, sd, LnAff{});                         \
    else                                                                                        \
      LTC_LAUNCH((sens_fwd_kernel<R, DSV>), grid, block, 0, s, x, xs, p.T, p.D, BT,     \
                         p.Hp, pp.sensF, sn, sd);                                               \
  } while (0)
  if (pp.sF != nullptr && (pp.sFi == nullptr || pp.sFn == nullptr)) return hipErrorInvalidValue;
  if (pp.sF != nullptr && pp.sFfull) {
    // one list per neuron over all of D; the block's rows of x staged whole
    if (split_d || p.Dp > 256) return hipErrorInvalidValue;
#define LTC_SENSF(R)                                                                          \
  LTC_LAUNCH((sens_fwd_full_kernel<R>), grid, block, (size_t)p.Dp * (4 * R + 4) * 4, s, x, xs, \
             p.T, p.D, p.Dp, BT, p.Hp, pp.sF, pp.sFi, pp.sFn, sn, sd)
    switch (rpw) {
      case 8: LTC_SENSF(8); break;
      case 4: LTC_SENSF(4); break;
      case 2: LTC_SENSF(2); break;
      default: LTC_SENSF(1); break;
    }
#undef LTC_SENSF
    return hipGetLastError();
  }
  if (split_d) {
    switch (rpw) {
      case 8: LTC_SENS(8, 4); break;
      case 4: LTC_SENS(4, 4); break;
      case 2: LTC_SENS(2, 4); break;
      default: LTC_SENS(1, 4); break;
    }
  } else {
    switch (rpw) {
      case 8: LTC_SENS(8, 1); break;
      case 4: LTC_SENS(4, 1); break;
      case 2: LTC_SENS(2, 1); break;
      default: LTC_SENS(1, 1); break;
    }
  }
#undef LTC_SENS
  return hipGetLastError();
}

hipError_t launch_sens_fwd_ln(const Plan& p, const float* x, Strides3 xs, const Prepped& pp,
                              const LnAff& la, float* sn, float* sd, hipStream_t s) {
  if (!sens_fwd_ln_fusable(p) || pp.sF == nullptr || pp.sFi == nullptr || pp.sFn == nullptr)
    return hipErrorInvalidValue;
  const int BT = p.B * p.T;
  const SensGeom geo = sens_fwd_geom(p);
  const dim3 grid(p.Hp / 64, (BT + 4 * geo.rpw - 1) / (4 * geo.rpw)), block(256);
#define LTC_SENSLN(R)                                                                      \
  LTC_LAUNCH((sens_fwd_cmp_kernel<R, 1, true>), grid, block, 0, s, x, xs, p.T, p.D, BT, \
                     p.Hp, pp.sF, pp.sFi, pp.sFn, sn, sd, la)
  switch (geo.rpw) {
    case 8: LTC_SENSLN(8); break;
    case 4: LTC_SENSLN(4); break;
    case 2: LTC_SENSLN(2); break;
    default: LTC_SENSLN(1); break;
  }
#undef LTC_SENSLN
  return hipGetLastError();
}

hipError_t launch_ode_fwd(const Plan& p, const Prepped& pp, const float* sn, const float* sd,
                          const float* state0, float eps, float* out, float* hfin,
                          float* vsave, float* densave, const ClusterBuf& cb, hipStream_t s) {
  if (p.CP > 0) {
    // Register-resident operands (RC = 16) read no image from L2 in the loop.
    const int xl = (p.RC == 16 && p.NCL % 8 == 0) ? 1 : 0;
    FwdCK a{pp.recF, pp.neuron, sn, sd, state0, out, hfin, vsave, densave, cb.xch, cb.status,
            cb.spin, p.B, p.T, p.H, p.Hp, p.U, p.KS, p.RC, p.CP, xl, eps,
            pp.cF, pp.cFi, pp.cFn, 0};
    if (cmp_fwd(p) && (pp.cF == nullptr || pp.cFi == nullptr || pp.cFn == nullptr))
      return hipErrorInvalidValue;
    // One launch per NCL * NB rows (more than one only at Hp > 1024); the
    // exchange words are cleared before each, in stream order.
    for (int l = 0; l < p.LCH; ++l) {
      hipError_t e = clear_cluster(p, cb, false, s, l == 0);
      if (e != hipSuccess) return e;
      a.R0 = l * p.NCL * p.NB;
      switch (p.NB) {
        case 8: e = fwd_cl_by_rcp<8>(p, a, s); break;
        case 4: e = fwd_cl_by_rcp<4>(p, a, s); break;
        case 2: e = fwd_cl_by_rcp<2>(p, a, s); break;
        default: e = fwd_cl_by_rcp<1>(p, a, s); break;
      }
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  FwdK a{pp.recF, pp.neuron, sn, sd, state0, out, hfin, vsave, densave,
         p.B, p.T, p.H, p.Hp, p.U, p.KS, p.RC, eps, pp.cF, pp.cFi, pp.cFn};
  if (cmp_fwd(p) && (pp.cF == nullptr || pp.cFi == nullptr || pp.cFn == nullptr))
    return hipErrorInvalidValue;
  switch (p.NB) {
    case 16: return fwd_by_rcp<16>(p, a, s);
    case 8: return fwd_by_rcp<8>(p, a, s);
    case 4: return fwd_by_rcp<4>(p, a, s);
    case 2: return fwd_by_rcp<2>(p, a, s);
    default: return fwd_by_rcp<1>(p, a, s);
  }
}

hipError_t launch_ode_bwd(const Plan& p, const Prepped& pp, const float* vsave,
                          const float* densave, const float* gout, Strides3 gs,
                          const float* ghfin, float2* absave, float* dsn, float* dsd,
                          float* npart, float* gstate, float* rpart, const ClusterBuf& cb,
                          hipStream_t s) {
  if (p.CP > 0) {
    // The register-resident fused chain (Hp = 256) prefetches saved rows that
    // every member of a cluster reads: keep a cluster on one XCD.
    const int xl = (chain_prefetches(p) && p.NCLB % 8 == 0) ? 1 : 0;
    BwdCK a{pp.recB, pp.neuron, vsave, densave, gout, gs, ghfin, absave, dsn, dsd, npart,
            gstate, rpart, cb.xch, cb.status, cb.spin, p.B, p.T, p.H, p.Hp, p.U, p.KSB, p.RCB,
            p.CPB, xl, pp.cB, pp.cBi, pp.cBn, 0};
    if (cmp_bwd(p) && (pp.cB == nullptr || pp.cBi == nullptr || pp.cBn == nullptr))
      return hipErrorInvalidValue;
    for (int l = 0; l < p.LCHB; ++l) {
      hipError_t e = clear_cluster(p, cb, true, s, l == 0);
      if (e != hipSuccess) return e;
      a.R0 = l * p.NCLB * p.NBB;
      switch (p.NBB) {
        case 8: e = bwd_cl_by_rcp<8>(p, a, s); break;
        case 4: e = bwd_cl_by_rcp<4>(p, a, s); break;
        case 2: e = bwd_cl_by_rcp<2>(p, a, s); break;
        default: e = bwd_cl_by_rcp<1>(p, a, s); break;
      }
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  BwdK a{pp.recB, pp.neuron, vsave, densave, gout, gs, ghfin, absave, dsn, dsd, npart, gstate,
         rpart, p.B, p.T, p.H, p.Hp, p.U, p.KSB, p.RCB, pp.cB, pp.cBi, pp.cBn, nullptr};
  if (cmp_bwd(p) && (pp.cB == nullptr || pp.cBi == nullptr || pp.cBn == nullptr))
    return hipErrorInvalidValue;
  switch (p.NB) {
    case 16: return bwd_by_rcp<16>(p, a, s);
    case 8: return bwd_by_rcp<8>(p, a, s);
    case 4: return bwd_by_rcp<4>(p, a, s);
    case 2: return bwd_by_rcp<2>(p, a, s);
    default: return bwd_by_rcp<1>(p, a, s);
  }
}

hipError_t launch_ode_bwd_row128_rec(const Plan& p, const Prepped& pp, const float* vsave,
                                     const float* densave, const float* gout, Strides3 gs,
                                     const float* ghfin, float* dsn, float* dsd, float* npart,
                                     float* gstate, float* rpart, unsigned long long* words,
                                     long long spin, const RowCompanion* sc, hipStream_t s) {
  if (!row128_rec_fused(p) || pp.cB == nullptr || pp.cBi == nullptr || pp.cBn == nullptr ||
      pp.recF == nullptr || words == nullptr)
    return hipErrorInvalidValue;
  const bool sens = sc != nullptr;
  if (sens && (!row128_sens_fused(p) || pp.sensB == nullptr || sc->xa == nullptr ||
               sc->spart == nullptr || sc->lnpart == nullptr || sc->gx == nullptr ||
               sc->ln.stats == nullptr || sc->ln.x == nullptr))
    return hipErrorInvalidValue;
  BwdK a{pp.recB, pp.neuron, vsave, densave, gout, gs, ghfin, nullptr, dsn, dsd, npart, gstate,
         rpart, p.B, p.T, p.H, p.Hp, p.U, p.KSB, p.RCB, pp.cB, pp.cBi, pp.cBn, words};
  const long long nrec = (long long)p.B * p.T * p.U * 256;
  unsigned long long* sw = sens ? words + nrec : nullptr;
  int* status = reinterpret_cast<int*>(words + row_bwd_words(p) - 1);
  RecC rc{pp.recF, spin, status, sw, nullptr, nullptr, nullptr, {}, nullptr, nullptr, nullptr,
          nullptr, nullptr, p.D, p.Dp};
  if (sens) {
    rc.xa = sc->xa;
    rc.sensB = pp.sensB;
    rc.spart = sc->spart;
    rc.ln = sc->ln;
    rc.input_w = sc->input_w;
    rc.ln_w = sc->ln_w;
    rc.ln_b = sc->ln_b;
    rc.gx = sc->gx;
    rc.lnpart = sc->lnpart;
  }
  const int Bc = (p.B + 7) / 8 * 8;
  const dim3 grid((unsigned)((sens ? 4 : 2) * Bc + p.B)), block(512);
  // the chain's LDS (its staged rows), or a sensory companion's when larger
  const size_t lds = sens ? (size_t)chain_launch_lds(p) : bwd_lds_bytes(p);
#define LTC_W128(F, C) \
  LTC_LAUNCH((ode_bwd_row_wave128_kernel<F, C>), grid, block, lds, s, a, rc)
  if (p.H == 128) {
    if (p.Dp > 64) LTC_W128(true, 2); else LTC_W128(true, 1);
  } else {
    if (p.Dp > 64) LTC_W128(false, 2); else LTC_W128(false, 1);
  }
#undef LTC_W128
  return hipGetLastError();
}

hipError_t launch_ode_bwd_row_fused(const Plan& p, const Prepped& pp, const float* vsave,
                                    const float* densave, const float* gout, Strides3 gs,
                                    const float* ghfin, float* npart, float* gstate, float* rpart,
                                    const RowCompanion& rc, hipStream_t s) {
  if (!row_bwd_fused(p) || pp.cB == nullptr || pp.sensB == nullptr || rc.words == nullptr)
    return hipErrorInvalidValue;
  BwdK a{pp.recB, pp.neuron, vsave, densave, gout, gs, ghfin, nullptr, nullptr, nullptr,
         npart, gstate, rpart, p.B, p.T, p.H, p.Hp, p.U, p.KSB, p.RCB, pp.cB, pp.cBi, pp.cBn,
         rc.words};
  const int Bc = (p.B + 7) / 8 * 8;
  const dim3 grid((unsigned)(Bc + p.B)), block(512);
  const int DC = p.Dp / 64;
  // the chain's LDS (its gradient tile), or the companion's when larger
  const size_t lds = (size_t)chain_launch_lds(p);
#define LTC_RBF(F, C) \
  LTC_LAUNCH((ode_bwd_row_fused_kernel<F, C>), grid, block, lds, s, a, rc, pp.sensB, p.D, p.Dp, Bc)
  if (p.H == 64) {
    if (DC == 1) LTC_RBF(true, 1); else LTC_RBF(true, 2);
  } else {
    if (DC == 1) LTC_RBF(false, 1); else LTC_RBF(false, 2);
  }
#undef LTC_RBF
  return hipGetLastError();
}

hipError_t launch_rec_grad(const Plan& p, const Prepped& pp, const float* vsave,
                           const float2* absave, float* rpart, hipStream_t s) {
  const long long nper = (p.N + p.NCH - 1) / p.NCH;
  RecGK a{pp.recF, vsave, absave, rpart, p.Hp, p.N, nper};
  LTC_LAUNCH(rec_grad_kernel, dim3(p.Hp / 64, p.Hp / 32, p.NCH), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_sens_bwd(const Plan& p, const float* x, Strides3 xs, const Prepped& pp,
                           const float* dsn, const float* dsd, float* spart, float* dxpart,
                           hipStream_t s, const float* smask) {
  const int BT = p.B * p.T;
  const int rows_per = (BT + p.NRC - 1) / p.NRC;
  SensBK a{x, xs, pp.sensB, dsn, dsd, spart, dxpart, p.T, p.D, p.Dp, p.Hp, BT, rows_per};
  const dim3 grid(p.Dp / 64, p.Hp / 32, p.NRC);
  if (smask != nullptr)
    LTC_LAUNCH(sens_bwd_cmp_kernel, grid, dim3(256), 0, s, a, smask, p.H);
  else
    LTC_LAUNCH(sens_bwd_kernel, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

// Applies the first pass to the recurrent and neuron partials when they are
// long; returns the partial pointers and counts the finalize kernel sums.
struct Partials {
  const float* rpart;
  int nrec;
  const float* npart;
  int nneuron;
};

hipError_t presum(const Plan& p, const float* rpart, const float* npart, const PresumBuf& ps,
                  hipStream_t s, Partials& out) {
  out = Partials{rpart, p.NCH, npart, p.B};
  auto pass = [&](const float* src, int M, long long N, float* dst) {
    const int parts = presum_parts(M);
    const int rpb = (M + parts - 1) / parts;
    LTC_LAUNCH(sum_rows_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)parts),
                       dim3(256), 0, s, src, N, M, N, rpb, dst);
    return parts;
  };
  if (presum_parts(p.NCH) > 0) {
    out.nrec = pass(rpart, p.NCH, 4LL * p.Hp * p.Hp, ps.rec);
    out.rpart = ps.rec;
  }
  if (presum_parts(p.B) > 0) {
    out.nneuron = pass(npart, p.B, 3LL * p.Hp, ps.neuron);
    out.npart = ps.neuron;
  }
  return hipGetLastError();
}

hipError_t launch_finalize(const Plan& p, const RawParams& rp, const float* rpart,
                           const float* spart, const float* dxpart, const float* npart,
                           const PresumBuf& ps, const GradOut& g, hipStream_t s, int segs) {
  const int BT = p.B * p.T;
  Partials pt{rpart, p.NCH, npart, p.B};
  if (segs & kFinRec) {
    hipError_t e = presum(p, rpart, npart, ps, s, pt);
    if (e != hipSuccess) return e;
  }
  const long long nrn = (long long)p.H * p.H + p.H;
  const long long nsx = (long long)p.D * p.H + (long long)BT * p.D;
  const long long base = (segs & kFinRec) ? 0 : nrn;
  const long long count = ((segs & kFinRec) ? nrn : 0) + ((segs & kFinSens) ? nsx : 0);
  if (count == 0) return hipSuccess;
  FinK a{rp, pt.rpart, spart, dxpart, pt.npart, g, pt.nneuron, p.D, p.H, p.Hp, p.Dp, pt.nrec,
         p.NRC, p.Hp / 32, BT, base, count};
  const unsigned blocks = (unsigned)((count + 255) / 256);
  LTC_LAUNCH(finalize_kernel, dim3(blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_prep_leaf(const Plan& p, const LeafParams& lp, const Prepped& pp, int images,
                            const LnBuf* ln, hipStream_t s, unsigned long long* clear_words,
                            long long nclear, float* sn, float* sd) {
  if (clear_words == nullptr) nclear = 0;
  const bool fs = sn != nullptr;
  if (fs && (ln == nullptr || sd == nullptr || !prep_sens_fused(p))) return hipErrorInvalidValue;
  const int threads = fs ? kPrepSensThreads : 256;
  const long long total =
      (long long)p.Hp * p.Hp + (long long)p.Dp * p.Hp + 3LL * p.Hp + (nclear + 3) / 4;
  const int nprep = (int)((total + threads - 1) / threads);
  const int BT = p.B * p.T;
  const int nln = ln ? (fs ? BT * (p.Hp / 64) : (BT + 3) / 4) : 0;
  LnBuf lb = ln ? *ln : LnBuf{nullptr, {0, 0, 0}, nullptr, nullptr};
  const bool bwd = (images & kLeafBwdImages) != 0;
  const int wpb = threads / 64;  // compacted columns per block, one per wave
  const int ncmp = (cmp_columns(pp, p.Hp, p.Dp, true, bwd, true) + wpb - 1) / wpb;
  // With the sensory sums formed in the row blocks, or the sensory launch
  // reading the compacted image, nothing reads sensF.
  const int sensf = (images & kLeafFwdImages) && !fs && pp.sF == nullptr ? 1 : 0;
#define LTC_PREPL(C, F)                                                                           \
  LTC_LAUNCH((prep_leaf_kernel<C, F>), dim3(nprep + ncmp + nln), dim3(threads), 0, s, lp, pp, \
                     p.H, p.D, p.Hp, p.Dp, bwd ? (p.FUSE ? 1 : 2) : 0, sensf, bwd ? 1 : 0, nprep, \
                     ncmp, cmp_chunks_fwd(p), cmp_chunks_bwd(p), lb, p.T, BT, clear_words,       \
                     nclear, sn, sd)
  if (fs) {
    if (p.D <= 64) LTC_PREPL(1, true);
    else LTC_PREPL(2, true);
  } else if (nln == 0 || p.D <= 64) LTC_PREPL(1, false);
  else if (p.D <= 128) LTC_PREPL(2, false);
  else if (p.D <= 256) LTC_PREPL(4, false);
  else if (p.D <= 512) LTC_PREPL(8, false);
  else LTC_PREPL(16, false);
#undef LTC_PREPL
  return hipGetLastError();
}

// Rows per LayerNorm-backward block: one per wave (more loads in flight) up
// to 4096 rows, four per wave beyond (fewer column partials).
int ln_rows_per_block(const Plan& p) {
  const long long BT = (long long)p.B * p.T;
  if (BT > 4096) return 16;
  // up to 1024 rows: the fewest rows per block that keep the column partials
  // at 64 or fewer, which the finalize sums without a pre-sum launch
  for (int rpb : {4, 8, 16})
    if ((BT + rpb - 1) / rpb <= 64) return rpb;
  return 4;
}

int ln_bwd_blocks(const Plan& p) {
  const int rpb = ln_rows_per_block(p);
  return (p.B * p.T + rpb - 1) / rpb;
}

hipError_t launch_ln_bwd(const Plan& p, const LeafParams& lp, const LnBuf& ln,
                         const float* dxpart, float* gx, float* lnpart, hipStream_t s) {
  const dim3 grid(ln_bwd_blocks(p)), block(256);
  // the dL/dxa partials per row: those of the 32-neuron blocks
  const int rpb = ln_rows_per_block(p), BT = p.B * p.T, HB = p.Hp / 32;
#define LTC_LNB(C) LTC_LAUNCH((ln_bwd_kernel<C>), grid, block, 0, s, lp, ln, dxpart, gx, lnpart, p.T, p.D, p.Dp, BT, HB, rpb)
  if (p.D <= 64) LTC_LNB(1);
  else if (p.D <= 128) LTC_LNB(2);
  else if (p.D <= 256) LTC_LNB(4);
  else if (p.D <= 512) LTC_LNB(8);
  else LTC_LNB(16);
#undef LTC_LNB
  return hipGetLastError();
}

hipError_t launch_finalize_leaf(const Plan& p, const LeafParams& lp, const float* rpart,
                                const float* spart, const float* npart, const float* lnpart,
                                const PresumBuf& ps, const LeafGrads& g, hipStream_t s,
                                const int* status, float* gstate) {
  Partials pt;
  hipError_t e = presum(p, rpart, npart, ps, s, pt);
  if (e != hipSuccess) return e;
  // one LayerNorm partial per row when the sensory companions formed them
  int nln = row128_sens_fused(p) ? p.B : ln_bwd_blocks(p);
  if (presum_parts(nln) > 0) {
    const int parts = presum_parts(nln), rpb = (nln + parts - 1) / parts;
    const long long N = 4LL * p.Dp;
    LTC_LAUNCH(sum_rows_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)parts),
                       dim3(256), 0, s, lnpart, N, nln, N, rpb, ps.ln);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    lnpart = ps.ln;
    nln = parts;
  }
  const long long nx = status ? (long long)p.B * p.T * p.D : 0;
  const long long ns = status && gstate ? (long long)p.B * p.H : 0;
  FinLeafK a{lp, pt.rpart, spart, pt.npart, lnpart, g, pt.nneuron, p.D, p.H, p.Hp, p.Dp,
             pt.nrec, p.NRC, nln, status, gstate, nx, ns};
  // four threads per output element, or one per output when a gave-up status
  // turns them all into NaN
  const long long nel = (long long)p.H * p.H + (long long)p.D * p.H + p.H + p.D;
  const long long total = 4 * nel > nel + nx + ns ? 4 * nel : nel + nx + ns;
  const unsigned blocks = (unsigned)((total + 255) / 256);
  LTC_LAUNCH(finalize_leaf_kernel, dim3(blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_finalize_leaf_fused(const Plan& p, const LeafParams& lp, const float* rpart,
                                      const float* spart, const float* npart,
                                      const float* lnpart, const PresumBuf& ps,
                                      const LeafGrads& g, const int* status, float* gstate,
                                      hipStream_t s) {
  if (!row_bwd_fused(p)) return hipErrorInvalidValue;
  Partials pt;
  hipError_t e = presum(p, rpart, npart, ps, s, pt);
  if (e != hipSuccess) return e;
  const long long nx = (long long)p.B * p.T * p.D, ns = (long long)p.B * p.H;
  // one sensory and one LayerNorm partial per batch row (B <= 64)
  FinLeafK a{lp, pt.rpart, spart, pt.npart, lnpart, g, pt.nneuron, p.D, p.H, p.Hp, p.Dp,
             pt.nrec, p.B, p.B, status, gstate, nx, ns};
  // four threads per output element, or one per output (every leaf gradient,
  // dL/dx and dL/dh0) when a gave-up status turns them all into NaN
  const long long nel = (long long)p.H * p.H + (long long)p.D * p.H + p.H + p.D;
  const long long total = 4 * nel > nel + nx + ns ? 4 * nel : nel + nx + ns;
  const unsigned blocks = (unsigned)((total + 255) / 256);
  LTC_LAUNCH(finalize_leaf_kernel, dim3(blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace ltc
