// Internal interface between the C-ABI layer (ltc_capi.hip) and the gfx950
// kernels (ltc_device.hip). Not installed; the public surface is
// include/ltc_capi.h.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace ltc {

// Kernel timing (ltc_timing_enable). While a timed call runs on a thread, the
// hook hands every kernel that call launches a pair of events, and the kernel
// is launched with hipExtLaunchKernel, which records the pair around the
// kernel's own execution: the interval is the kernel's duration, with no
// marker command between the two events and the kernel.
struct LaunchEvents {
  virtual bool take(hipEvent_t* start, hipEvent_t* stop) = 0;
};
extern thread_local LaunchEvents* g_launch_events;

#define LTC_LAUNCH(K, GRID, BLOCK, LDS, S, ...)                                          \
  do {                                                                                   \
    hipEvent_t ltc_ev_a_ = nullptr, ltc_ev_b_ = nullptr;                                 \
    if (::ltc::g_launch_events != nullptr &&                                             \
        ::ltc::g_launch_events->take(&ltc_ev_a_, &ltc_ev_b_))                            \
      hipExtLaunchKernelGGL(K, GRID, BLOCK, LDS, S, ltc_ev_a_, ltc_ev_b_, 0, __VA_ARGS__); \
    else                                                                                 \
      hipLaunchKernelGGL(K, GRID, BLOCK, LDS, S, __VA_ARGS__);                           \
  } while (0)

// Threads per workgroup of the persistent ODE kernels for NB batch rows per
// workgroup. More rows per thread means more live registers, so fewer
// threads; the same bound is the kernels' __launch_bounds__.
constexpr int ode_max_threads(int nb) { return nb <= 1 ? 1024 : (nb <= 4 ? 512 : 256); }

// Rows each thread finishes per unfold (the compile-time size of its per-row
// registers). The launch plan keeps ceil(NB / KS) within it: KS >= 4 when NB >= 4.
constexpr int ode_owned_rows(int nb) { return nb <= 2 ? nb : nb / 4; }

// (NB, RC) pairs whose chain kernel can also keep the four recurrent
// gradient accumulators of every register-resident operand without spilling
// at the register budget __launch_bounds__(ode_max_threads(NB)) leaves
// (checked against the compiled code objects: zero scratch). One row at
// Hp = 64 uses the single-row chain instead (ode_bwd_row_wave_kernel).
constexpr bool ode_fuse_ok(int nb, int rc) {
  return (nb == 4 && (rc == 4 || rc == 8)) || (nb == 8 && (rc == 4 || rc == 8)) ||
         (nb == 16 && rc == 4);
}

// Kernel ids for the optional event-timing facility.
enum KernelId : int {
  K_PREP = 0,
  K_SENS_FWD,
  K_ODE_FWD,
  K_ODE_BWD,
  K_REC_GRAD,
  K_SENS_BWD,
  K_LN_BWD,
  K_FINALIZE,
  K_COUNT
};

// Shapes and launch choices shared by every kernel of one call.
struct Plan {
  int B, T, D, H, U;
  int Hp, Dp;      // H and D rounded up to 64 (one wave of lanes per 64 columns)
  int NB;          // batch rows per workgroup in the persistent ODE kernels
  int KS;          // forward: split of the reduction axis across waves of one workgroup
  int RC;          // forward: reduction chunk per thread = Hp / KS
  int KSB;         // chain (backward) kernel: the same split
  int RCB;         // chain kernel: Hp / KSB
  bool FUSE;       // recurrent parameter gradients accumulated inside the chain kernel
  int CP;          // cluster path: workgroups per cluster (0 = one workgroup per NB rows)
  int NCL;         // cluster path: clusters = ceil(B / NB); grid = NCL * CP
  // Cluster path, chain kernel: its own geometry (equal to the forward's
  // unless the chain is fused): CPB members of JWB columns, NBB rows per
  // cluster, NCLB clusters.
  int CPB, JWB, NBB, NCLB;
  int NCH;         // partials of the recurrent parameter-gradient reduction
  int NRC;         // row-chunks of the sensory backward reduction
  long long N;     // T * U * B unfold instances
  // Cluster path, launches per call: 1, or with Hp > 1024 (no single-workgroup
  // form covers a row) as many as take the B rows NCL * NB at a time, each
  // launch holding at most one workgroup per CU. Forward and chain.
  int LCH, LCHB;
};

// Derived, zero-padded parameter images built once per call by the prep kernel.
//   recF[i][j] = {-S*log2e, S*M*log2e, WE, WP} of synapse (i -> j), [Hp][Hp]
//   recB[j][i] = the same float4, transposed, [Hp][Hp]
//   sensF[d][h] = {-Ss*log2e, Ss*Ms*log2e, Ws*Es, Ws}, [Dp][Hp]
//   sensB[h][d] = {-Ss*log2e, Ss*Ms*log2e, Es, Ws*Ss}, [Hp][Dp]
//   neuron = C[Hp], G[Hp], L[Hp]
//
// Compacted recurrent images (cmp_fwd / cmp_bwd): per column, the synapses
// that can contribute, in ascending row order; with NC chunks (cmp_chunks_*)
// of Hp/NC slots, entry e of column c sits in chunk e % NC, slot e / NC:
//   cF[(ks*Hp/NC + s)*Hp + j]  forward operand of column j (postsynaptic), rows i
//                           with WE or WP nonzero (a synapse with both zero adds
//                           exact zeros to the forward sums);
//   cB[(ks*Hp/NC + s)*Hp + i]  chain operand of column i (presynaptic), rows j: every
//                           real synapse, or on the module path only those whose
//                           mask entry is nonzero (the others have zero gradients);
//   cFi / cBi               the row index of each slot (0 in padding slots);
//   cFn / cBn               the entry count of each column.
// Padding slots hold zero operands, which add exact zeros. Null when the plan
// does not use the compacted kernels.
struct Prepped {
  float4* recF;
  float4* recB;
  float4* sensF;
  float4* sensB;
  float* neuron;
  float4* cF;
  int* cFi;
  int* cFn;
  float4* cB;
  int* cBi;
  int* cBn;
  // Compacted sensory forward image (module path): per 64-input chunk and
  // neuron h, the chunk's inputs whose sensory weight for h is nonzero,
  // ascending, as [chunk][64 slots][Hp] operands and input indices within
  // the chunk, and [chunk][Hp] counts.
  float4* sF;
  int* sFi;
  int* sFn;
  // 1: the same image as one list per neuron over all of D instead
  // ([slot][Hp] operands and input indices, [Hp] counts; sens_full_list)
  int sFfull;
};
// Chunks (and slots per chunk) of a compacted image column at Hp = 256.
constexpr int kCmpChunks = 16;
// LDS of the compacted kernels' slot table: one int per slot per thread.
inline long long cmp_index_lds(int threads) { return (long long)threads * kCmpChunks * 4; }
// LDS scratch of the balanced lane order (balanced_lane in the device code):
// one int per thread and 17 per wave.
inline long long balance_lds(long long threads) { return threads * 4 + (threads / 64) * 17 * 4; }
// The compacted cluster chain pads each alpha/beta row by two pairs.
inline long long cmp_pad_lds(int hp) { return 16LL * hp; }

struct RawParams {
  const float* w_pos;
  const float* w_erev;
  const float* mu;
  const float* sigma;
  const float* s_mu;
  const float* s_sigma;
  const float* s_erev;
  const float* s_wpos;
  const float* cm;
  const float* gleak;
  const float* vleak;
};

struct Strides3 {
  long long b, t, c;
};

// Module-level leaves (reference ltc.py:150-186) for the fused module path:
// the pre-transforms of ltc.py:259-283 are then computed inside the kernels.
//   w_pos = softplus(w)*mask, w_erev = w_pos*erev, cm_t = softplus(cm)/dtU,
//   gleak_pos = softplus(gleak), sensory_w_pos = softplus(s_w)*s_mask,
//   xa = LayerNorm(x; ln_w, ln_b, ln_eps)*input_w + input_b.
struct LeafParams {
  const float* w;
  const float* erev;
  const float* mask;
  const float* mu;
  const float* sigma;
  const float* s_w;
  const float* s_erev;
  const float* s_mask;
  const float* s_mu;
  const float* s_sigma;
  const float* gleak;
  const float* vleak;
  const float* cm;
  const float* input_w;
  const float* input_b;
  const float* ln_w;
  const float* ln_b;
  float dtU;     // dt / ode_unfolds, as the fp32 scalar torch divides by
  float ln_eps;
};

// LayerNorm + affine of the module path: per (b,t) row, xa written contiguous
// [B*T][D] and (mean, rstd) in stats [B*T][2].
struct LnBuf {
  const float* x;  // raw input, strided
  Strides3 xs;
  float* xa;
  float* stats;
};

// Largest input width the module path handles (LayerNorm rows in registers).
constexpr int kModuleMaxD = 1024;

// Segments of the parameter images that a prep launch builds: the recurrent
// images, the sensory images and the per-neuron vectors.
constexpr int kPrepRec = 1, kPrepSens = 2, kPrepNeuron = 4;
constexpr int kPrepAll = kPrepRec | kPrepSens | kPrepNeuron;
hipError_t launch_prep(const Plan& p, const RawParams& rp, const Prepped& pp, bool bwd,
                       hipStream_t s, int segs = kPrepAll);
// Copies rows x cols floats from pitch src_ld to pitch dst_ld (both in
// floats), zero-filling dst columns [cols, dst_ld).
hipError_t launch_copy_rows(const float* src, long long src_ld, float* dst, long long dst_ld,
                            long long rows, int cols, hipStream_t s);
// Module path: images from the leaves; with ln != nullptr the same launch
// also normalises every (b,t) row of x. `images` selects the forward
// (sensF) and backward (recB, sensB) images; recF and neuron are always built.
constexpr int kLeafFwdImages = 1;
constexpr int kLeafBwdImages = 2;
// With sn != nullptr (only when prep_sens_fused(p)), the row blocks also
// compute every row's sensory sums into sn / sd, forming the sensory operands
// from the leaves, and the separate sensory launch is skipped.
hipError_t launch_prep_leaf(const Plan& p, const LeafParams& lp, const Prepped& pp, int images,
                            const LnBuf* ln, hipStream_t s, unsigned long long* clear_words = nullptr,
                            long long nclear = 0, float* sn = nullptr, float* sd = nullptr);
hipError_t launch_sens_fwd(const Plan& p, const float* x, Strides3 xs, const Prepped& pp,
                           float* sn, float* sd, hipStream_t s);
// Geometry of the sensory forward launch: rows per wave, and whether the
// four waves split D (few rows) instead of taking a row group each.
struct SensGeom {
  int rpw;
  bool split_d;
};
inline SensGeom sens_fwd_geom(const Plan& p) {
  const long long BT = (long long)p.B * p.T, hb = p.Hp / 64;
  // Many rows: 4 row groups per workgroup sharing operands through L1.
  // Few rows: split D over the waves instead, so each thread's chain of
  // dependent operand loads is 4x shorter.
  const bool split_d = hb * ((BT + 3) / 4) < 512;
  const int rows_of = split_d ? 1 : 4;
  int rpw = 8;
  while (rpw > 1 && hb * ((BT + rows_of * rpw - 1) / (rows_of * rpw)) < 1024) rpw >>= 1;
  return {rpw, split_d};
}
// The compacted sensory image as one list per neuron over all of D (for
// sens_fwd_full_kernel, which stages the block's rows of x whole): with four
// row groups per workgroup and 64 < Dp <= 256. With Dp = 64 the per-chunk
// image is already one list per neuron.
inline bool sens_full_list(const Plan& p) {
  return p.Dp > 64 && p.Dp <= 256 && !sens_fwd_geom(p).split_d;
}
// The module forward's sensory sums inside the prep launch: when a block
// per (row, 64 neurons) fits the chip at once (at most 256 of them) and a
// row fits two 64-input chunks, such blocks of the prep launch normalise
// their row and form its sums themselves, which saves a dependent launch.
// They read the sensory leaves as 16-byte rows of four neurons, so H % 4 == 0
// here and the caller also checks that the five sensory leaves are 16-byte
// aligned.
inline bool prep_sens_fused(const Plan& p) {
  return (long long)p.B * p.T * (p.Hp / 64) <= 256 && p.D >= 1 && p.D <= 128 && p.H % 4 == 0;
}
// LayerNorm + affine of the raw input rows, applied by the compacted sensory
// launch itself when the rows fit one 64-input chunk and the launch takes
// four row groups per workgroup (the module's no-grad forward then skips the
// prep launch's row normalisation, whose output nothing else reads).
struct LnAff {
  const float* ln_w;
  const float* ln_b;
  const float* input_w;
  const float* input_b;
  float eps;
};
inline bool sens_fwd_ln_fusable(const Plan& p) { return p.D <= 64 && !sens_fwd_geom(p).split_d; }
hipError_t launch_sens_fwd_ln(const Plan& p, const float* x, Strides3 xs, const Prepped& pp,
                              const LnAff& la, float* sn, float* sd, hipStream_t s);
// Cluster path scratch: exchange words and a status word (nonzero after a
// cluster member gave up waiting for its partners), plus the wait budget of
// every exchange in ticks of the 100 MHz wall clock (<= 0: a member gives up
// at its first wait, which the tests use to force the give-up path).
struct ClusterBuf {
  unsigned long long* xch;
  int* status;
  long long spin;
};
// Default wait budget: 0.2 s.
constexpr long long kDefaultSpinTicks = 20000000;

// Writes a list of contiguous float segments in one launch: each segment is
// either copied from `src` or, with src == nullptr, filled with `value`. With
// `gate` set, the launch does nothing unless *gate != 0, and then it also
// raises the device's sticky fault flag (read by device_fault()): the
// cluster paths use this to overwrite every output of a call with NaN after a
// member gave up. A kernel, not hipMemsetAsync, so that a captured call
// records kernel nodes only.
struct FillSeg {
  float* dst;
  const float* src;
  long long n;
};
constexpr int kMaxFillSegs = 20;
struct FillList {
  FillSeg seg[kMaxFillSegs];
  int nseg;
  float value;
  const int* gate;
};
hipError_t launch_fill(const FillList& fl, hipStream_t s);
// Adds a segment (ignored when dst is null or n is 0).
inline void fill_add(FillList& fl, float* dst, const float* src, long long n) {
  if (dst != nullptr && n > 0 && fl.nseg < kMaxFillSegs) fl.seg[fl.nseg++] = FillSeg{dst, src, n};
}
// The current device's sticky fault flag: reads it (after waiting for the
// device) and clears it when `clear` is set. Returns the HIP status.
hipError_t device_fault(int* value, bool clear);
// Exchange words of one cluster launch (forward / chain).
inline long long cluster_words(const Plan& p) { return 2LL * p.NCL * p.CP * p.NB * 64; }
inline long long cluster_words_bwd(const Plan& p) {
  return 2LL * p.NCLB * p.CPB * p.NBB * p.JWB;
}
// Rows of slack after the [Hp][Hp] operand images that the cluster kernels'
// streamed prefetch may read.
constexpr int kImageSlackRows = 8;
// LDS bytes of one cluster chain member: alpha/beta [NB][Hp] float2, the
// reduction partials [KS][NB][JW], and with `pf` three [NB][Hp] blocks of
// saved forward values (1/den of one unfold, v of two slots) prefetched ahead
// of use.
// Saved values the prefetching chain keeps per (row, column): 1/den of one
// unfold and v of two slots (12 bytes), or in the two-group form
// (ode_bwd_cl2_kernel, NB >= 2) 1/den of two unfolds and v of three slots.
inline long long chain_pf_bytes(int nb) { return nb >= 2 ? 20 : 12; }
inline long long cluster_chain_lds(int nb, int hp, int ks, int jw, bool pf) {
  return (long long)nb * hp * 8 + (long long)ks * nb * jw * 4 +
         (pf ? chain_pf_bytes(nb) * nb * hp : 0);
}
// The cluster chain prefetches saved values when its operands are
// register-resident: the fused form at Hp = 256.
inline bool chain_prefetches(const Plan& p) { return p.FUSE && p.CP > 0 && p.Hp == 256; }
// One row per workgroup at Hp = 64: the wave-owned single-row forward
// (RC = 16) and fused chain (RCB = 8), one barrier per unfold.
inline bool row_kernels(const Plan& p) { return p.CP == 0 && p.NB == 1 && p.Hp == 64; }
// Kernels that read compacted images: the cluster forward and the fused
// cluster chain with register-resident operands (16 rows per thread,
// Hp = 256), and the single-row forward (4 row groups of 16) and fused chain
// (8 groups of 8) at Hp = 64. The chunk count is the number of row groups a
// column's entries are dealt over.
// The single-workgroup forward with register-resident operands (RC of 4, 8 or
// 16) reads one too, its entries dealt over its KS row chunks.
// One row per workgroup at Hp = 128: the wave-owned single-row forward (8
// waves of 16 columns, the compacted image in 4 chunks of 32 slots).
inline bool row_wave128_fwd(const Plan& p) {
  return p.CP == 0 && p.NB == 1 && p.Hp == 128 && p.KS == 8 && p.RC == 16;
}
// The unfused single-row chain at Hp = 128 (ode_bwd_row_wave128_kernel: 8
// waves of 16 neurons, the folded compacted image in 4 chunks of 32 slots).
inline bool row_wave128_bwd(const Plan& p) {
  return p.CP == 0 && p.NB == 1 && p.Hp == 128 && !p.FUSE && p.KSB == 8 && p.RCB == 16;
}
inline bool generic_fwd_cmp(const Plan& p) {
  return p.CP == 0 && !row_kernels(p) && (p.RC == 4 || p.RC == 8 || p.RC == 16);
}
inline bool cmp_fwd(const Plan& p) {
  return (p.CP > 0 && p.Hp == 256 && p.KS == 16 && p.RC == 16) || (row_kernels(p) && p.RC == 16) ||
         generic_fwd_cmp(p);
}
// The unfused single-workgroup chain with register-resident operands reads a
// compacted folded image (only synapses that add to dL/dv).
inline bool generic_bwd_cmp(const Plan& p) {
  return p.CP == 0 && !row_kernels(p) && !p.FUSE && (p.RCB == 4 || p.RCB == 8 || p.RCB == 16);
}
inline bool cmp_bwd(const Plan& p) {
  return (p.CP > 0 && p.FUSE && p.Hp == 256 && p.JWB == 32 && p.KSB == 16 && p.RCB == 16) ||
         (row_kernels(p) && p.FUSE && p.RCB == 8) || generic_bwd_cmp(p);
}
// Module-path backward at Hp = 64 with one row per workgroup, Dp <= 128 and
// B <= 64: the sensory and LayerNorm backward run inside the chain launch, in
// one companion workgroup per batch row that takes each step's dL/dsn, dL/dsd
// from its row's chain workgroup as {value, tag} words (row_bwd_words of
// them: [B*T][2][64], then a status word).
inline bool row_bwd_fused(const Plan& p) {
  return row_kernels(p) && p.FUSE && p.RCB == 8 && p.Dp <= 128 && p.B >= 1 && p.B <= 64;
}
// Module-path backward at Hp = 128 with one row per workgroup (the unfused
// single-row chain) and B <= 64: the recurrent parameter-gradient sums are
// formed inside the chain launch, in two companion workgroups per batch row
// (64 postsynaptic neurons each) that take each unfold's alpha/beta from the
// row's chain workgroup as {value, tag} words ([B][T*U][2][128], then a
// status word), instead of by rec_grad_kernel afterwards: one recurrent
// partial per row. The words live in the module's saved buffer from the
// forward to the backward, 2 KiB per (row, unfold), so the companions are
// chosen only while they take at most 64 MiB (B*T*U <= 32768); longer
// sequences save alpha/beta for rec_grad_kernel instead (8 bytes per neuron
// and unfold, in the backward's workspace).
constexpr long long kRow128WordUnfolds = 32768;
inline bool row128_rec_fused(const Plan& p) {
  return row_wave128_bwd(p) && p.B >= 1 && p.B <= 64 &&
         (long long)p.B * p.T * p.U <= kRow128WordUnfolds;
}
// With Dp <= 128 the sensory and LayerNorm backward also run in companion
// workgroups of that launch, two per row (64 neurons each), taking each
// step's dL/dsn, dL/dsd as words [B][T][2][128] after the alpha/beta words;
// the first hands its dL/dxa sums to the second as words [B][T][128], which
// finishes the LayerNorm backward. They write one sensory partial and one
// LayerNorm column partial per row, and dL/dx.
inline bool row128_sens_fused(const Plan& p) { return row128_rec_fused(p) && p.Dp <= 128; }
// Exchange words of the fused row backward (row_bwd_fused) or of the Hp = 128
// chain with recurrent-gradient companions (row128_rec_fused); the last one
// is the status word.
inline long long row_bwd_words(const Plan& p) {
  if (row_bwd_fused(p)) return (long long)p.B * p.T * 128 + 1;
  if (row128_rec_fused(p))
    return (long long)p.B * p.T * p.U * 256 + (row128_sens_fused(p) ? (long long)p.B * p.T * 384 : 0) + 1;
  return 0;
}
inline int cmp_chunks_fwd(const Plan& p) {
  return (row_kernels(p) || row_wave128_fwd(p)) ? 4 : (p.CP > 0 ? kCmpChunks : p.KS);
}
inline int cmp_chunks_bwd(const Plan& p) {
  return row_kernels(p) ? 8 : (row_wave128_bwd(p) ? 4 : (p.CP > 0 ? kCmpChunks : p.KSB));
}
// Dynamic LDS of a cluster chain member (cluster_chain_lds) plus, with the
// compacted image, its slot table.
inline long long cluster_bwd_lds(const Plan& p) {
  return cluster_chain_lds(p.NBB, p.Hp, p.KSB, p.JWB, chain_prefetches(p)) +
         (cmp_bwd(p) ? cmp_index_lds(p.JWB * p.KSB) + cmp_pad_lds(p.Hp) +
                           balance_lds(p.JWB * p.KSB)
                     : 0);
}
// Dynamic LDS of a cluster forward member: state rows [NB][Hp], the KS
// partials [KS][NB][64] float2, and with the compacted image the slot table.
inline long long cluster_fwd_lds(const Plan& p) {
  return (long long)p.NB * p.Hp * 4 + (long long)p.KS * p.NB * 64 * 8 +
         (cmp_fwd(p) ? cmp_index_lds(64 * p.KS) + balance_lds(64 * p.KS) : 0);
}
// Dynamic LDS of the single-workgroup forward: state rows and the KS
// partials, or the wave-owned single-row forward's state and staged sums.
// Steps of sensory sums the single-row forward stages in LDS at a time, and
// unfolds of saved states the single-row chain stages.
constexpr int kRowSensSteps = 32;
constexpr int kRowChainUnfolds = 48;
inline long long fwd_lds(const Plan& p) {
  // with the compacted image, the slot table (one int per slot per thread)
  // and the balanced lane order's scratch (one int per thread, 17 per wave)
  const long long thr = (long long)p.Hp * p.KS;
  const long long base = (long long)p.NB * p.Hp * 4 + (long long)p.KS * p.NB * p.Hp * 8 +
                         (generic_fwd_cmp(p) ? thr * p.RC * 4 + balance_lds(thr) : 0);
  // the wave-owned single-row forms: the double-buffered state and the
  // staged sensory sums
  const long long wave = 2LL * p.Hp * 4 + 2LL * kRowSensSteps * p.Hp * 4;
  if (row_wave128_fwd(p)) return wave;
  const long long row = row_kernels(p) ? wave : 0;
  return base > row ? base : row;
}

// Dynamic LDS of the single-workgroup chain (ode_bwd_kernel): alpha/beta rows
// and the KS partials, or the wave-owned single-row chain's alpha/beta and
// staged rows; with FUSE at least one padded [Hp][Hp+1] plane (all four in
// the single-row chain at Hp = 64), through which the recurrent-gradient
// partials are transposed for coalesced stores.
inline long long chain_lds(const Plan& p) {
  // with the compacted image, the slot table: one int per slot per thread
  long long base = (long long)p.NB * p.Hp * 8 + (long long)p.KSB * p.NB * p.Hp * 4 +
                   (generic_bwd_cmp(p) ? (long long)p.Hp * p.KSB * p.RCB * 4 : 0);
  // the wave-owned single-row chains: alpha/beta by parity and the staged
  // v^k, 1/den and dL/dout rows
  const long long waveb = 2LL * p.Hp * 8 + (3LL * kRowChainUnfolds + 1) * p.Hp * 4;
  if (row_wave128_bwd(p)) return waveb;
  if (row_kernels(p) && waveb > base) base = waveb;
  const long long plane =
      p.FUSE ? (row_kernels(p) ? 4LL : 1LL) * p.Hp * (p.Hp + 1) * 4 : 0;
  return base > plane ? base : plane;
}

// Dynamic LDS of a sensory companion workgroup (the fused row backward at
// Hp = 64, and the sensory companions of the Hp = 128 chain), over DC
// 64-input blocks: the operands of every block past the first
// [8 waves][8][64] float4, one [64] float2 row, the [9][64 * DC] float sums
// and a flag word.
inline long long sens_companion_lds(int DC) {
  return (long long)(DC - 1) * 8 * 8 * 64 * 16 + 64 * 8 + 9LL * 64 * DC * 4 + 16;
}
// Dynamic LDS the module backward's chain launch requests: the chain's own,
// or its sensory companions' when larger (a recurrent-gradient companion of
// the Hp = 128 chain needs about 2 KB, under the chain's staging).
inline long long chain_launch_lds(const Plan& p) {
  const long long c = chain_lds(p);
  if (!row_bwd_fused(p) && !row128_sens_fused(p)) return c;
  const long long comp = sens_companion_lds(p.Dp / 64);
  return c > comp ? c : comp;
}

hipError_t launch_ode_fwd(const Plan& p, const Prepped& pp, const float* sn, const float* sd,
                          const float* state0, float eps, float* out, float* hfin,
                          float* vsave, float* densave, const ClusterBuf& cb, hipStream_t s);
hipError_t launch_ode_bwd(const Plan& p, const Prepped& pp, const float* vsave,
                          const float* densave, const float* gout, Strides3 gs,
                          const float* ghfin, float2* absave, float* dsn, float* dsd,
                          float* npart, float* gstate, float* rpart, const ClusterBuf& cb,
                          hipStream_t s);
hipError_t launch_rec_grad(const Plan& p, const Prepped& pp, const float* vsave,
                           const float2* absave, float* rpart, hipStream_t s);
// smask (the module path's sensory mask, (D,H)): skip the masked synapses
// (sens_bwd_cmp_kernel), whose partials stay unwritten.
hipError_t launch_sens_bwd(const Plan& p, const float* x, Strides3 xs, const Prepped& pp,
                           const float* dsn, const float* dsd, float* spart, float* dxpart,
                           hipStream_t s, const float* smask = nullptr);
struct GradOut {
  float* x;        // (B,T,D) contiguous
  float* w_pos;    // (H,H)
  float* w_erev;
  float* mu;
  float* sigma;
  float* s_mu;     // (D,H)
  float* s_sigma;
  float* s_erev;
  float* s_wpos;
  float* cm;       // (H)
  float* gleak;
  float* vleak;
};
// Long partial sums (the per-row neuron partials over B, the recurrent
// gradient partials over NCH) get a parallel first pass into at most 64
// partials each: presum_parts(M) of them, or 0 when M is small enough to sum
// directly. The scratch buffers hold presum_parts(NCH) * 4*Hp*Hp and
// presum_parts(B) * 3*Hp floats.
inline int presum_parts(int m) {
  if (m <= 64) return 0;
  const int rpb = (m + 63) / 64 > 32 ? (m + 63) / 64 : 32;
  return (m + rpb - 1) / rpb;
}
struct PresumBuf {
  float* rec;     // presum_parts(NCH) x 4*Hp*Hp
  float* neuron;  // presum_parts(B) x 3*Hp
  float* ln;      // module path: presum_parts(ln_bwd_blocks) x 4*Dp
};
// Gradient groups a finalize launch writes: the recurrent and per-neuron
// gradients (from rpart, npart) and the sensory and input gradients (from
// spart, dxpart).
constexpr int kFinRec = 1, kFinSens = 2, kFinAll = kFinRec | kFinSens;
hipError_t launch_finalize(const Plan& p, const RawParams& rp, const float* rpart,
                           const float* spart, const float* dxpart, const float* npart,
                           const PresumBuf& ps, const GradOut& g, hipStream_t s,
                           int segs = kFinAll);

// Module path backward.
struct LeafGrads {
  float* x;  // (B,T,D) raw-input gradient, contiguous
  float* w;
  float* erev;
  float* mu;
  float* sigma;
  float* s_w;
  float* s_erev;
  float* s_mu;
  float* s_sigma;
  float* gleak;
  float* vleak;
  float* cm;
  float* input_w;
  float* input_b;
  float* ln_w;
  float* ln_b;
};
// LayerNorm/affine backward per row, from the h-block partials of dL/dxa;
// writes dL/dx and per-block column partials lnpart[nblk][4][Dp].
int ln_bwd_blocks(const Plan& p);
hipError_t launch_ln_bwd(const Plan& p, const LeafParams& lp, const LnBuf& ln,
                         const float* dxpart, float* gx, float* lnpart, hipStream_t s);
// With a status word (the companions of a row128_rec_fused chain), every
// output (also dL/dx and dL/dh0 = gstate) becomes NaN when it is set.
hipError_t launch_finalize_leaf(const Plan& p, const LeafParams& lp, const float* rpart,
                                const float* spart, const float* npart, const float* lnpart,
                                const PresumBuf& ps, const LeafGrads& g, hipStream_t s,
                                const int* status = nullptr, float* gstate = nullptr);

// Fused row backward (row_bwd_fused): the chain of every batch row plus one
// companion workgroup per row for its sensory and LayerNorm backward. The
// companions write the sensory partials (one per row, [B][4][Hp][Dp]), the
// LayerNorm column partials ([B][4][Dp]) and dL/dx; a companion that runs out
// of its wait budget sets *status instead.
struct RowCompanion {
  const float* xa;     // [B*T][D] LayerNorm + affine output (the sensory input)
  LnBuf ln;            // raw input and row statistics
  const float* input_w;
  const float* ln_w;
  const float* ln_b;
  float* spart;
  float* lnpart;
  float* gx;
  unsigned long long* words;  // row_bwd_words(p), cleared before the launch
  long long spin;
};
// The Hp = 128 chain with recurrent-gradient companions (row128_rec_fused):
// rpart receives one partial per batch row, [B][4][Hp][Hp]; a companion that
// runs out of its wait budget sets the status word after the words.
// With sc (row128_sens_fused), also the sensory companions, which run the
// sensory and LayerNorm backward as RowCompanion describes (its words and
// spin unused: those of this call hold).
hipError_t launch_ode_bwd_row128_rec(const Plan& p, const Prepped& pp, const float* vsave,
                                     const float* densave, const float* gout, Strides3 gs,
                                     const float* ghfin, float* dsn, float* dsd, float* npart,
                                     float* gstate, float* rpart, unsigned long long* words,
                                     long long spin, const RowCompanion* sc, hipStream_t s);
hipError_t launch_ode_bwd_row_fused(const Plan& p, const Prepped& pp, const float* vsave,
                                    const float* densave, const float* gout, Strides3 gs,
                                    const float* ghfin, float* npart, float* gstate, float* rpart,
                                    const RowCompanion& rc, hipStream_t s);
// The module finalize after a fused row backward: B sensory and B LayerNorm
// partials, and with *status set every output (also dL/dx and dL/dh0) NaN.
hipError_t launch_finalize_leaf_fused(const Plan& p, const LeafParams& lp, const float* rpart,
                                      const float* spart, const float* npart,
                                      const float* lnpart, const PresumBuf& ps,
                                      const LeafGrads& g, const int* status, float* gstate,
                                      hipStream_t s);

}  // namespace ltc
