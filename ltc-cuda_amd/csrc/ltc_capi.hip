// C-ABI entry points of libltc_hip.so (declared in include/ltc_capi.h).
// Validates arguments before touching the device, chooses the launch plan,
// carves the caller's workspace and enqueues the kernels on the caller's
// stream. Allocates no device memory.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/ltc_capi.h"
#include "ltc_internal.h"

// Scratch of the no-allocation forward (ltc_full_forward_noalloc): one array
// per device, held until the process ends. In host code `scratch` names a
// host-side shadow, never the device array: its device address comes from
// hipGetSymbolAddress, once per device, and only that address is passed on.
static __device__ __align__(256) unsigned char scratch[LTC_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

long long round_up(long long v, long long m) { return (v + m - 1) / m * m; }

// Compute units of the current device (cached per device). Without a device
// the plan is made for MI355X's 256.
int device_cus() {
  constexpr int kMaxDev = 64;
  static int cache[kMaxDev] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) {
    (void)hipGetLastError();
    return 256;
  }
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n < 1) {
      (void)hipGetLastError();
      n = 256;
    }
    cache[dev] = n;
  }
  return cache[dev];
}

// Cluster path (H > 192): CP = Hp/64 workgroups share NB rows, one 64-column
// slice each, so every operand serves NB rows while up to one workgroup per
// CU runs. The whole grid must be resident at once (members wait on each
// other), so it is used only when NCL * CP <= CUs, with at most 1024 threads
// and at most one CU's LDS per workgroup (one workgroup fits on any CU).
// Dynamic LDS of a forward cluster member, leaving room for its static flag word.
constexpr long long kClusterLds = 60 * 1024;

// LDS one workgroup may allocate on the current device (cached per device),
// less 1 KiB for static variables. Without a device the plan is made for
// MI355X's 160 KiB.
long long chain_lds_limit() {
  constexpr int kMaxDev = 64;
  static int cache[kMaxDev] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) {
    (void)hipGetLastError();
    return 159 * 1024;
  }
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
        n < 65536) {
      (void)hipGetLastError();
      n = 65536;
    }
    cache[dev] = n;
  }
  return cache[dev] - 1024;
}

// Hp = 256 and 512: the chain runs as clusters of Hp/32 members of 32
// columns with 512 threads, each thread holding the four gradient sums of its
// Hp/16 synapses in registers (operands register-resident at Hp = 256,
// streamed at 512), which removes the separate parameter-gradient pass.
void plan_fused_chain(ltc::Plan& p, int ncu) {
  if (p.Hp != 256 && p.Hp != 512) return;
  const int cp = p.Hp / 32, slots = ncu / cp;
  for (int nb : {1, 2, 4, 8}) {
    const int ncl = (p.B + nb - 1) / nb;
    if (ncl > slots) continue;
    // at Hp = 256 the compacted chain adds its slot table
    if (ltc::cluster_chain_lds(nb, p.Hp, 16, 32, p.Hp == 256) +
            (p.Hp == 256 ? ltc::cmp_index_lds(512) + ltc::cmp_pad_lds(p.Hp) + ltc::balance_lds(512)
                         : 0) >
        chain_lds_limit())
      continue;
    p.CPB = cp;
    p.JWB = 32;
    p.NBB = nb;
    p.NCLB = ncl;
    p.KSB = 16;
    p.RCB = p.Hp / 16;
    p.FUSE = true;
    return;
  }
}

// Cluster geometry with NB rows per cluster: the largest KS (16 or 8, RC a
// multiple of 8, KS >= NB) whose forward and chain LDS fit; 0 if none.
int cluster_ks(const ltc::Plan& p, int nb) {
  for (int ks = 16; ks >= nb && ks >= 8; ks >>= 1) {
    if ((p.Hp / ks) % 8 != 0) continue;  // streamed operands come eight rows at a time
    const long long lf = (long long)nb * p.Hp * 4 + (long long)ks * nb * 64 * 8;
    if (lf > kClusterLds || ltc::cluster_chain_lds(nb, p.Hp, ks, 64, false) > chain_lds_limit())
      continue;
    if (p.Hp == 256 && ks == 16 &&
        lf + ltc::cmp_index_lds(64 * ks) + ltc::balance_lds(64 * ks) > chain_lds_limit())
      continue;
    return ks;
  }
  return 0;
}

// Hp > 1024: one thread per column no longer fits one workgroup, so the
// cluster form runs every batch size. When the rows do not fit one launch of
// at most one workgroup per CU, the call makes LCH launches, each taking the
// next NCL * NB rows (rows are independent): the fewest rows per cluster
// that fit B in one launch, else the most the LDS allows.
bool plan_cluster_wide(ltc::Plan& p, int ncu) {
  if (p.Hp <= 1024 || p.B < 1) return false;
  const int cp = p.Hp / 64;
  const int slots = ncu / cp;
  if (slots < 1) return false;
  int best_nb = 0, best_ks = 0;
  for (int nb : {1, 2, 4, 8}) {
    const int ks = cluster_ks(p, nb);
    if (ks == 0) continue;
    best_nb = nb;
    best_ks = ks;
    if ((p.B + nb - 1) / nb <= slots) break;
  }
  if (best_nb == 0) return false;
  const int nb = best_nb, ks = best_ks;
  const int need = (p.B + nb - 1) / nb;
  const int ncl = need < slots ? need : slots;
  p.CP = cp;
  p.NCL = ncl;
  p.NB = nb;
  p.KS = p.KSB = ks;
  p.RC = p.RCB = p.Hp / ks;
  p.FUSE = false;
  p.CPB = cp;
  p.JWB = 64;
  p.NBB = nb;
  p.NCLB = ncl;
  p.LCH = p.LCHB = (p.B + ncl * nb - 1) / (ncl * nb);
  return true;
}

bool plan_cluster(ltc::Plan& p, int ncu) {
  if (p.Hp < 256 || p.B < 1) return false;
  if (p.Hp > 1024) return plan_cluster_wide(p, ncu);
  const int cp = p.Hp / 64;
  const int slots = ncu / cp;
  for (int nb : {1, 2, 4, 8}) {
    const int ncl = (p.B + nb - 1) / nb;
    if (ncl > slots) continue;
    for (int ks = 16; ks >= nb && ks >= 8; ks >>= 1) {
      if ((p.Hp / ks) % 8 != 0) continue;  // streamed operands come eight rows at a time
      const long long lf = (long long)nb * p.Hp * 4 + (long long)ks * nb * 64 * 8;
      if (lf > kClusterLds || ltc::cluster_chain_lds(nb, p.Hp, ks, 64, false) > chain_lds_limit())
        continue;
      // the compacted forward (Hp = 256, 16 rows per thread) adds its slot
      // table and the balanced lane order's scratch
      if (p.Hp == 256 && ks == 16 &&
          lf + ltc::cmp_index_lds(64 * ks) + ltc::balance_lds(64 * ks) > chain_lds_limit())
        continue;
      p.CP = cp;
      p.NCL = ncl;
      p.NB = nb;
      p.KS = p.KSB = ks;
      p.RC = p.RCB = p.Hp / ks;
      p.FUSE = false;
      p.CPB = cp;
      p.JWB = 64;
      p.NBB = nb;
      p.NCLB = ncl;
      plan_fused_chain(p, ncu);
      return true;
    }
  }
  return false;
}

// ---------------------------------------------------------------------------
// Launch plan
// ---------------------------------------------------------------------------
ltc::Plan make_plan_uncached(int B, int T, int D, int H, int U, int ncu) {
  ltc::Plan p{};
  p.B = B;
  p.T = T;
  p.D = D;
  p.H = H;
  p.U = U;
  p.Hp = (int)round_up(H > 0 ? H : 1, 64);
  p.Dp = (int)round_up(D > 0 ? D : 1, 64);
  // Rows per persistent workgroup: keep at least 256 workgroups (one per CU)
  // while B allows, and reuse each synapse operand NB times otherwise.
  // At Hp = 64 the operands of every thread stay in registers, so reuse over
  // more rows buys nothing, while more workgroups per CU hide latency
  // (measured: NB = 4 beats 8 and 16 for both ODE kernels at large B).
  p.NB = 1;
  for (int nb : {16, 8, 4, 2}) {
    if (p.Hp <= 64 && nb > 4) continue;
    if ((B + nb - 1) / nb >= 256) {
      p.NB = nb;
      break;
    }
  }
  // Split of the reduction axis: as many waves as the thread bound allows,
  // with LDS partials under 64 KiB and at least 4 synapses per thread. When
  // even KS = 1 does not fit, fewer rows per workgroup.
  auto lds_fwd = [&](int nb, int k) {
    return (long long)nb * p.Hp * 4 + (long long)k * nb * p.Hp * 8;
  };
  auto lds_bwd = [&](int nb, int k) {
    return (long long)nb * p.Hp * 8 + (long long)k * nb * p.Hp * 4;
  };
  // KS is a power of two <= 16, so it always divides Hp/4 (Hp is a multiple
  // of 64). With NB >= 4 rows, KS >= 4 keeps the rows each thread finishes
  // within ode_owned_rows(NB). When no split fits, fewer rows per workgroup.
  auto pick_ks = [&](int nb, int want, bool bwd) {
    const int cap = ltc::ode_max_threads(nb) / p.Hp;
    const int ks_min = nb >= 4 ? 4 : 1;
    int ks = 0;
    for (int k = 16; k >= 1; k >>= 1) {
      if (k <= cap && k <= want) {
        ks = k;
        break;
      }
    }
    auto fits = [&](int k) {
      return k >= ks_min && p.Hp / k >= 4 &&
             (bwd ? lds_bwd(nb, k) : lds_fwd(nb, k)) <= 65536;
    };
    while (ks > ks_min && !fits(ks)) ks >>= 1;
    return fits(ks) ? ks : 0;
  };
  // Per-unfold latency is lowest with one wave per SIMD for the forward at
  // small H with one row per workgroup (fewer partials, same VALU work per
  // CU). With several rows per workgroup at Hp = 64 (many workgroups per CU)
  // eight chunks per column measured faster: the compacted forward's waves,
  // in balanced lane order, then hold 8 entries each at most (C5 forward
  // 79.2 -> 76.8 us). The chain kernel keeps the widest split, whose
  // register-resident operands carry the fused gradient accumulators.
  const int want_f = p.Hp <= 64 ? (p.NB >= 2 ? 8 : 4) : 16;
  for (;;) {
    const int kf = pick_ks(p.NB, want_f, false), kb = pick_ks(p.NB, 16, true);
    if ((kf > 0 && kb > 0) || p.NB == 1) {
      p.KS = kf > 0 ? kf : 1;
      p.KSB = kb > 0 ? kb : 1;
      break;
    }
    p.NB >>= 1;
  }
  p.RC = p.Hp / p.KS;
  p.RCB = p.Hp / p.KSB;
  p.N = (long long)T * U * B;
  // When each thread's synapse operands fit in registers (RC in {4, 8, 16}),
  // the chain kernel also accumulates the recurrent parameter gradients and
  // writes one partial per workgroup.
  p.FUSE = ltc::ode_fuse_ok(p.NB, p.RCB);
  // One row at Hp = 64: the single-row fused chain with 8 waves of 8 synapses.
  if (p.NB == 1 && p.Hp == 64) {
    p.KSB = 8;
    p.RCB = 8;
    p.FUSE = true;
  }
  p.CP = p.NCL = 0;
  p.CPB = p.NBB = p.NCLB = 0;
  p.JWB = 64;
  p.LCH = p.LCHB = 1;
  plan_cluster(p, ncu);
  // Recurrent parameter-gradient chunks: about 1024 workgroups, at least 32
  // unfold instances each, at most 64 partials per synapse.
  if (p.FUSE) {
    // One partial per chain workgroup, or per chain cluster.
    p.NCH = p.CP > 0 ? p.NCLB : (B + p.NB - 1) / p.NB;
    if (p.NCH < 1) p.NCH = 1;
  } else {
    const long long bpc = (long long)(p.Hp / 64) * (p.Hp / 32);
    long long nch = (1024 + bpc - 1) / bpc;
    if (nch > 64) nch = 64;
    const long long cap = (p.N + 31) / 32;
    if (nch > cap) nch = cap;
    if (nch < 1) nch = 1;
    const long long nper = (p.N + nch - 1) / nch;
    p.NCH = (int)(nper > 0 ? (p.N + nper - 1) / nper : 1);
    if (p.NCH < 1) p.NCH = 1;
  }
  // Sensory backward row chunks, at least 8 rows each: blocks for two full
  // rounds of the CUs at three resident blocks each (the sensory backward
  // kernels' registers and LDS allow three), so that no lone last round of
  // blocks runs on a third of each CU (C3 0.383 -> 0.359 ms, C4 0.437 ->
  // 0.423 ms against 1024 blocks).
  {
    const long long BT = (long long)B * T;
    const long long bpc = (long long)(p.Dp / 64) * (p.Hp / 32);
    long long nrc = (6LL * ncu + bpc - 1) / bpc;
    if (nrc > 64) nrc = 64;
    const long long cap = (BT + 7) / 8;
    if (nrc > cap) nrc = cap;
    if (nrc < 1) nrc = 1;
    const long long per = (BT + nrc - 1) / nrc;
    p.NRC = (int)(per > 0 ? (BT + per - 1) / per : 1);
    if (p.NRC < 1) p.NRC = 1;
  }
  return p;
}

// The plans of the last few sizes asked for on this thread: a training step
// asks for the same sizes several times (saved-buffer and workspace sizes,
// then the call itself, forward and backward).
ltc::Plan make_plan(int B, int T, int D, int H, int U, int ncu = device_cus()) {
  constexpr int kKey = 7;
  struct Entry {
    int key[kKey];
    ltc::Plan p;
  };
  constexpr int kEntries = 4;
  thread_local Entry cache[kEntries];
  thread_local int used = 0, next = 0;
  // the plan also depends on the device's per-workgroup LDS limit
  const int key[kKey] = {B, T, D, H, U, ncu, (int)chain_lds_limit()};
  for (int i = 0; i < used; ++i) {
    const Entry& e = cache[i];
    bool hit = true;
    for (int k = 0; k < kKey; ++k) hit = hit && e.key[k] == key[k];
    if (hit) return e.p;
  }
  Entry& e = cache[next];
  for (int i = 0; i < kKey; ++i) e.key[i] = key[i];
  e.p = make_plan_uncached(B, T, D, H, U, ncu);
  next = (next + 1) % kEntries;
  if (used < kEntries) ++used;
  return e.p;
}

// Carves 256-byte aligned regions out of one workspace in a fixed order; the
// same walk computes the total size (base == nullptr).
struct Carver {
  char* base;
  long long off = 0;
  template <class Tp>
  Tp* take(long long count) {
    const long long at = round_up(off, 256);
    off = at + count * (long long)sizeof(Tp);
    return base ? reinterpret_cast<Tp*>(base + at) : nullptr;
  }
};

// Operand image rows: the cluster kernels' streamed prefetch may read a few
// rows past the end.
long long image_rows(const ltc::Plan& p) { return p.Hp + (p.CP > 0 ? ltc::kImageSlackRows : 0); }

// Wait budget of the cluster exchanges (ltc_set_cluster_spin_ticks).
std::atomic<long long> g_spin{ltc::kDefaultSpinTicks};

// Compacted images of the register-resident cluster kernels (forward / chain).
void carve_cmp(const ltc::Plan& p, Carver& c, ltc::Prepped& pp, bool fwd, bool bwd) {
  const long long n = (long long)p.Hp * p.Hp;
  if (fwd && ltc::cmp_fwd(p)) {
    pp.cF = c.take<float4>(n);
    pp.cFi = c.take<int>(n);
    pp.cFn = c.take<int>(p.Hp);
  }
  if (bwd && ltc::cmp_bwd(p)) {
    pp.cB = c.take<float4>(n);
    pp.cBi = c.take<int>(n);
    pp.cBn = c.take<int>(p.Hp);
  }
}

ltc::ClusterBuf carve_cluster(const ltc::Plan& p, Carver& c, bool bwd) {
  ltc::ClusterBuf cb{nullptr, nullptr, g_spin.load(std::memory_order_relaxed)};
  if (p.CP > 0) {
    cb.xch = c.take<unsigned long long>(bwd ? ltc::cluster_words_bwd(p) : ltc::cluster_words(p));
    cb.status = c.take<int>(1);
  }
  return cb;
}

struct FwdWs {
  ltc::Prepped pp;
  float* sn;
  float* sd;
  ltc::ClusterBuf cb;
};

// The compacted sensory forward image (per 64-input chunk and neuron, the
// inputs with a nonzero sensory weight), which the forward's sensory launch
// reads instead of the dense image.
void carve_sens_cmp(const ltc::Plan& p, Carver& c, ltc::Prepped& pp) {
  const long long n = (long long)p.Dp * p.Hp;
  pp.sF = c.take<float4>(n);
  pp.sFi = c.take<int>(n);
  pp.sFn = c.take<int>((long long)(p.Dp / 64) * p.Hp);
  pp.sFfull = ltc::sens_full_list(p) ? 1 : 0;
}

// sens: with the compacted sensory image (every forward that runs the
// sensory launch).
FwdWs carve_fwd(const ltc::Plan& p, Carver& c, bool sens = true) {
  FwdWs w{};
  w.pp.recF = c.take<float4>(image_rows(p) * p.Hp);
  w.pp.sensF = c.take<float4>((long long)p.Dp * p.Hp);
  w.pp.neuron = c.take<float>(3LL * p.Hp);
  carve_cmp(p, c, w.pp, true, false);
  w.sn = c.take<float>((long long)p.B * p.T * p.Hp);
  w.sd = c.take<float>((long long)p.B * p.T * p.Hp);
  w.cb = carve_cluster(p, c, false);
  if (sens) carve_sens_cmp(p, c, w.pp);
  return w;
}

struct BwdWs {
  ltc::Prepped pp;
  float2* absave;
  float* dsn;
  float* dsd;
  float* npart;
  float* rpart;
  float* spart;
  float* dxpart;
  ltc::ClusterBuf cb;
  ltc::PresumBuf ps;
};

// images = false: the caller brings the parameter images (the module path
// keeps them in its saved buffer).
BwdWs carve_bwd(const ltc::Plan& p, Carver& c, bool images = true) {
  BwdWs w{};
  if (images) {
    w.pp.recF = c.take<float4>(image_rows(p) * p.Hp);
    w.pp.recB = c.take<float4>(image_rows(p) * p.Hp);
    w.pp.sensB = c.take<float4>((long long)p.Dp * p.Hp);
    w.pp.neuron = c.take<float>(3LL * p.Hp);
    // the forward's as well: the per-step backward recomputes a forward unfold
    carve_cmp(p, c, w.pp, true, true);
  }
  w.absave = p.FUSE ? nullptr : c.take<float2>(p.N * p.Hp);
  w.dsn = c.take<float>((long long)p.B * p.T * p.Hp);
  w.dsd = c.take<float>((long long)p.B * p.T * p.Hp);
  w.npart = c.take<float>((long long)p.B * 3 * p.Hp);
  // recurrent partials: NCH chunks, or one per batch row (Hp = 128 chain with
  // recurrent-gradient companions)
  const long long nch = ltc::row128_rec_fused(p) && p.B > p.NCH ? p.B : p.NCH;
  w.rpart = c.take<float>(nch * 4 * p.Hp * p.Hp);
  // sensory partials: NRC row chunks, or one per batch row (fused row backward,
  // or the sensory companions of the Hp = 128 chain)
  const bool per_row = ltc::row_bwd_fused(p) || ltc::row128_sens_fused(p);
  const long long nrc = per_row && p.B > p.NRC ? p.B : p.NRC;
  w.spart = c.take<float>(nrc * 4 * p.Dp * p.Hp);
  w.dxpart = c.take<float>((long long)(p.Hp / 32) * p.B * p.T * p.Dp);
  w.cb = carve_cluster(p, c, true);
  w.ps.rec = c.take<float>((long long)ltc::presum_parts(p.NCH) * 4 * p.Hp * p.Hp);
  w.ps.neuron = c.take<float>((long long)ltc::presum_parts(p.B) * 3 * p.Hp);
  w.ps.ln = c.take<float>((long long)ltc::presum_parts(ltc::ln_bwd_blocks(p)) * 4 * p.Dp);
  return w;
}

// LayerNorm column partials of the module backward: one per ln_bwd block, or
// one per batch row when the fused row backward forms them.
long long module_ln_parts(const ltc::Plan& p) {
  const long long n = ltc::ln_bwd_blocks(p);
  return (ltc::row_bwd_fused(p) || ltc::row128_sens_fused(p)) && p.B > n ? p.B : n;
}

// Module-path extras: the normalised input and its row statistics live in the
// saved buffer when training (the backward reads them), else in the workspace.
struct LnWs {
  float* xa;
  float* stats;
};

LnWs carve_ln(const ltc::Plan& p, Carver& c) {
  LnWs w{};
  w.xa = c.take<float>((long long)p.B * p.T * p.D);
  w.stats = c.take<float>(2LL * p.B * p.T);
  return w;
}

long long saved_floats(const ltc::Plan& p) {
  // vsave: T*U+1 slots of (B,Hp); densave (1/den): T*U slots of (B,Hp).
  return ((long long)p.T * p.U + 1) * p.B * p.Hp + (long long)p.T * p.U * p.B * p.Hp;
}

// Every parameter image of a training step: the forward builds them all in
// one launch and the backward reads them from the saved buffer.
ltc::Prepped carve_images(const ltc::Plan& p, Carver& c) {
  ltc::Prepped pp{};
  pp.recF = c.take<float4>(image_rows(p) * p.Hp);
  pp.recB = c.take<float4>(image_rows(p) * p.Hp);
  pp.sensF = c.take<float4>((long long)p.Dp * p.Hp);
  pp.sensB = c.take<float4>((long long)p.Dp * p.Hp);
  pp.neuron = c.take<float>(3LL * p.Hp);
  carve_cmp(p, c, pp, true, true);
  return pp;
}

// The fused row backward's exchange words and status word, after the images
// in the module's saved buffer (cleared by the forward's prep launch).
unsigned long long* carve_row_words(const ltc::Plan& p, Carver& c) {
  const long long n = ltc::row_bwd_words(p);
  return n > 0 ? c.take<unsigned long long>(n) : nullptr;
}

long long module_saved_floats(const ltc::Plan& p) {
  // boundary saved buffer, then xa and stats, then the parameter images, each
  // at 64-float (256-byte) alignment
  Carver c{nullptr};
  c.take<float>(saved_floats(p));
  carve_ln(p, c);
  carve_images(p, c);
  carve_row_words(p, c);
  return (c.off + 3) / 4;
}

int check_dims(int B, int T, int D, int H, int U) {
  if (B < 0 || T < 0 || D < 1 || H < 1)
    return fail(LTC_EINVAL, "dimensions must satisfy B >= 0, T >= 0, D >= 1, H >= 1");
  if (U < 1) return fail(LTC_EINVAL, "ode_unfolds must be >= 1");
  if (H > LTC_MAX_HIDDEN)
    return fail(LTC_EUNSUPPORTED, "hidden size H = " + std::to_string(H) + " exceeds " +
                                      std::to_string(LTC_MAX_HIDDEN));
  // above 1024 only the cluster form covers a row: Hp/64 workgroups at once
  if (H > 1024 && (H + 63) / 64 > device_cus())
    return fail(LTC_EUNSUPPORTED, "hidden size H = " + std::to_string(H) +
                                      " needs " + std::to_string((H + 63) / 64) +
                                      " co-resident workgroups; the device has " +
                                      std::to_string(device_cus()) + " CUs");
  if ((long long)B * T * (D > H ? D : H) > (1LL << 40))
    return fail(LTC_EUNSUPPORTED, "problem too large");
  return LTC_OK;
}

// ---------------------------------------------------------------------------
// Event timing
// ---------------------------------------------------------------------------
const char* const kNames[ltc::K_COUNT] = {"ltc_prep",     "ltc_sens_fwd", "ltc_ode_fwd",
                                          "ltc_ode_bwd",  "ltc_rec_grad", "ltc_sens_bwd",
                                          "ltc_ln_bwd",   "ltc_finalize"};

struct Timing {
  std::mutex mu;
  bool on = false;
  // One timed call: the event pairs of the kernels it launched.
  struct Rec {
    int id;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> ev;
  };
  std::vector<Rec> pending;
  std::vector<hipEvent_t> pool;
  double total_ms[ltc::K_COUNT] = {};
  long long count[ltc::K_COUNT] = {};

  hipEvent_t get() {
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
  // A call's time is the sum of its kernels' durations; calls count once.
  void drain() {
    for (auto& r : pending) {
      double sum = 0.0;
      bool ok = !r.ev.empty();
      for (auto& pr : r.ev) {
        float ms = 0.f;
        if (hipEventSynchronize(pr.second) == hipSuccess &&
            hipEventElapsedTime(&ms, pr.first, pr.second) == hipSuccess)
          sum += ms;
        else
          ok = false;
        pool.push_back(pr.first);
        pool.push_back(pr.second);
      }
      if (ok) {
        total_ms[r.id] += sum;
        count[r.id] += 1;
      }
    }
    pending.clear();
  }
};

Timing& timing() {
  static Timing* t = new Timing();  // never destroyed: events may outlive static teardown
  return *t;
}

// Hands each kernel of one timed call an event pair from the pool.
struct CallEvents : ltc::LaunchEvents {
  Timing& tm;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> ev;
  explicit CallEvents(Timing& t) : tm(t) {}
  bool take(hipEvent_t* a, hipEvent_t* b) override {
    std::lock_guard<std::mutex> g(tm.mu);
    *a = tm.get();
    *b = tm.get();
    if (*a == nullptr || *b == nullptr) {
      if (*a) tm.pool.push_back(*a);
      if (*b) tm.pool.push_back(*b);
      return false;
    }
    ev.emplace_back(*a, *b);
    return true;
  }
};

// Runs one library call's launches; when timing is enabled, each of its
// kernels is timed by its own execution (hipExtLaunchKernel events).
template <class F>
hipError_t timed(int id, hipStream_t s, F&& launch) {
  (void)s;
  Timing& tm = timing();
  if (!tm.on) return launch();
  CallEvents ce(tm);
  ltc::LaunchEvents* prev = ltc::g_launch_events;
  ltc::g_launch_events = &ce;
  const hipError_t err = launch();
  ltc::g_launch_events = prev;
  if (!ce.ev.empty()) {
    std::lock_guard<std::mutex> g(tm.mu);
    tm.pending.push_back({id, std::move(ce.ev)});
  }
  return err;
}

int hip_fail(const char* what, hipError_t e) {
  return fail(LTC_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

// Runs a fill list (zero-fills and copies of a degenerate call, or the NaN
// fill after a cluster launch) and reports a failed launch.
int run_fill(const ltc::FillList& fl, hipStream_t s) {
  const hipError_t e = ltc::launch_fill(fl, s);
  return e == hipSuccess ? LTC_OK : hip_fail("fill launch", e);
}

ltc::FillList zero_list() {
  ltc::FillList fl{};
  fl.value = 0.f;
  return fl;
}

// After a call whose ODE kernels ran as clusters: every output listed is
// overwritten with NaN, and the device's fault flag raised, when a member of
// the call gave up waiting (its status word is set); otherwise nothing runs.
ltc::FillList poison_list(const ltc::ClusterBuf& cb) {
  ltc::FillList fl{};
  fl.value = __builtin_nanf("");
  fl.gate = cb.status;
  return fl;
}

// Device address of this device's scratch array (looked up on the first call
// on each device, with that device current); nullptr after a failed lookup,
// with the message set.
void* noalloc_scratch() {
  constexpr int kMaxDev = 64;
  static std::mutex mu;
  static void* addr[kMaxDev] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    hip_fail("hipGetDevice", e);
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDev) {
    fail(LTC_EUNSUPPORTED, "device index " + std::to_string(dev) + " out of range");
    return nullptr;
  }
  std::lock_guard<std::mutex> g(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      hip_fail("hipGetSymbolAddress(scratch)", e != hipSuccess ? e : hipErrorInvalidSymbol);
      return nullptr;
    }
    addr[dev] = p;
  }
  return addr[dev];
}

}  // namespace

extern "C" {

int ltc_abi_version(void) { return LTC_ABI_VERSION; }

const char* ltc_last_error(void) { return g_err.c_str(); }

int ltc_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

long long ltc_saved_floats(int B, int T, int H, int ode_unfolds) {
  if (B < 0 || T < 0 || H < 1 || ode_unfolds < 1) return -1;
  return saved_floats(make_plan(B, T, 1, H, ode_unfolds));
}

long long ltc_fwd_workspace_bytes(int B, int T, int D, int H, int ode_unfolds) {
  if (check_dims(B, T, D, H, ode_unfolds) != LTC_OK) return -1;
  const ltc::Plan p = make_plan(B, T, D, H, ode_unfolds);
  Carver c{nullptr};
  carve_fwd(p, c);
  return round_up(c.off, 256);
}

long long ltc_bwd_workspace_bytes(int B, int T, int D, int H, int ode_unfolds) {
  if (check_dims(B, T, D, H, ode_unfolds) != LTC_OK) return -1;
  const ltc::Plan p = make_plan(B, T, D, H, ode_unfolds);
  Carver c{nullptr};
  carve_bwd(p, c);
  return round_up(c.off, 256);
}

int ltc_full_forward(const float* x, long long sxb, long long sxt, long long sxd,
                     const float* state, const float* w_pos, const float* w_erev,
                     const float* mu, const float* sigma, const float* sensory_mu,
                     const float* sensory_sigma, const float* sensory_erev,
                     const float* sensory_w_pos, const float* cm_t, const float* gleak_pos,
                     const float* vleak, int B, int T, int D, int H, int ode_unfolds,
                     float epsilon, int save_intermediates, float* out, float* h_final,
                     float* saved, void* workspace, long long workspace_bytes, void* stream) {
  g_err.clear();
  int rc = check_dims(B, T, D, H, ode_unfolds);
  if (rc != LTC_OK) return rc;
  if (!w_pos || !w_erev || !mu || !sigma || !sensory_mu || !sensory_sigma || !sensory_erev ||
      !sensory_w_pos || !cm_t || !gleak_pos || !vleak)
    return fail(LTC_EINVAL, "parameter pointer is NULL");
  if (B > 0 && (!state || !h_final)) return fail(LTC_EINVAL, "state/h_final pointer is NULL");
  if ((long long)B * T > 0 && (!x || !out)) return fail(LTC_EINVAL, "x/out pointer is NULL");
  if (save_intermediates && !saved) return fail(LTC_EINVAL, "saved pointer is NULL");
  const ltc::Plan p = make_plan(B, T, D, H, ode_unfolds);
  Carver need{nullptr};
  carve_fwd(p, need);
  if (workspace_bytes < need.off || (need.off > 0 && !workspace))
    return fail(LTC_EINVAL, "workspace too small: need " + std::to_string(need.off) + " bytes");
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
    return fail(LTC_EINVAL, "workspace must be 256-byte aligned");
  if (B == 0) return LTC_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (T == 0) {
    // No steps: the final state is the initial state.
    ltc::FillList fl = zero_list();
    ltc::fill_add(fl, h_final, state, (long long)B * H);
    return run_fill(fl, s);
  }

  Carver c{static_cast<char*>(workspace)};
  const FwdWs w = carve_fwd(p, c);
  const ltc::RawParams rp{w_pos, w_erev, mu, sigma, sensory_mu, sensory_sigma, sensory_erev,
                          sensory_w_pos, cm_t, gleak_pos, vleak};
  const ltc::Strides3 xs{sxb, sxt, sxd};
  float* vsave = save_intermediates ? saved : nullptr;
  float* densave = save_intermediates ? saved + ((long long)T * ode_unfolds + 1) * B * p.Hp : nullptr;

  hipError_t e;
  e = timed(ltc::K_PREP, s, [&] { return ltc::launch_prep(p, rp, w.pp, false, s); });
  if (e != hipSuccess) return hip_fail("prep launch", e);
  e = timed(ltc::K_SENS_FWD, s, [&] { return ltc::launch_sens_fwd(p, x, xs, w.pp, w.sn, w.sd, s); });
  if (e != hipSuccess) return hip_fail("sensory forward launch", e);
  e = timed(ltc::K_ODE_FWD, s, [&] {
    return ltc::launch_ode_fwd(p, w.pp, w.sn, w.sd, state, epsilon, out, h_final, vsave, densave,
                               w.cb, s);
  });
  if (e != hipSuccess) return hip_fail("ODE forward launch", e);
  if (p.CP > 0) {
    ltc::FillList fl = poison_list(w.cb);
    ltc::fill_add(fl, out, nullptr, (long long)B * T * H);
    ltc::fill_add(fl, h_final, nullptr, (long long)B * H);
    ltc::fill_add(fl, saved, nullptr, save_intermediates ? saved_floats(p) : 0);
    return run_fill(fl, s);
  }
  return LTC_OK;
}

int ltc_full_forward_noalloc(const float* x, long long sxb, long long sxt, long long sxd,
                             const float* state, const float* w_pos, const float* w_erev,
                             const float* mu, const float* sigma, const float* sensory_mu,
                             const float* sensory_sigma, const float* sensory_erev,
                             const float* sensory_w_pos, const float* cm_t,
                             const float* gleak_pos, const float* vleak, int B, int T, int D,
                             int H, int ode_unfolds, float epsilon, int save_intermediates,
                             float* out, float* h_final, float* saved, void* stream) {
  g_err.clear();
  const int rc = check_dims(B, T, D, H, ode_unfolds);
  if (rc != LTC_OK) return rc;
  Carver need{nullptr};
  carve_fwd(make_plan(B, T, D, H, ode_unfolds), need);
  if (need.off > LTC_NOALLOC_SCRATCH_BYTES)
    return fail(LTC_EUNSUPPORTED,
                "these sizes need " + std::to_string(need.off) +
                    " bytes of scratch; the no-allocation forward holds " +
                    std::to_string(LTC_NOALLOC_SCRATCH_BYTES) +
                    " (use ltc_full_forward with a workspace)");
  void* ws = noalloc_scratch();
  if (ws == nullptr) return LTC_EHIP;
  return ltc_full_forward(x, sxb, sxt, sxd, state, w_pos, w_erev, mu, sigma, sensory_mu,
                          sensory_sigma, sensory_erev, sensory_w_pos, cm_t, gleak_pos, vleak, B,
                          T, D, H, ode_unfolds, epsilon, save_intermediates, out, h_final, saved,
                          ws, LTC_NOALLOC_SCRATCH_BYTES, stream);
}

int ltc_full_backward(const float* x, long long sxb, long long sxt, long long sxd,
                      const float* w_pos, const float* w_erev, const float* mu,
                      const float* sigma, const float* sensory_mu, const float* sensory_sigma,
                      const float* sensory_erev, const float* sensory_w_pos, const float* cm_t,
                      const float* gleak_pos, const float* vleak, const float* saved,
                      const float* grad_out, long long sgb, long long sgt, long long sgh,
                      const float* grad_h_final, int B, int T, int D, int H, int ode_unfolds,
                      float epsilon, float* grad_x, float* grad_state, float* grad_w_pos,
                      float* grad_w_erev, float* grad_mu, float* grad_sigma,
                      float* grad_sensory_mu, float* grad_sensory_sigma,
                      float* grad_sensory_erev, float* grad_sensory_w_pos, float* grad_cm_t,
                      float* grad_gleak_pos, float* grad_vleak, void* workspace,
                      long long workspace_bytes, void* stream) {
  g_err.clear();
  (void)epsilon;  // the saved denominators already include it
  int rc = check_dims(B, T, D, H, ode_unfolds);
  if (rc != LTC_OK) return rc;
  if (!w_pos || !w_erev || !mu || !sigma || !sensory_mu || !sensory_sigma || !sensory_erev ||
      !sensory_w_pos || !cm_t || !gleak_pos || !vleak)
    return fail(LTC_EINVAL, "parameter pointer is NULL");
  if (!grad_w_pos || !grad_w_erev || !grad_mu || !grad_sigma || !grad_sensory_mu ||
      !grad_sensory_sigma || !grad_sensory_erev || !grad_sensory_w_pos || !grad_cm_t ||
      !grad_gleak_pos || !grad_vleak)
    return fail(LTC_EINVAL, "gradient output pointer is NULL");
  if (B > 0 && !grad_state) return fail(LTC_EINVAL, "grad_state pointer is NULL");
  if ((long long)B * T > 0 && (!x || !grad_out || !grad_x || !saved))
    return fail(LTC_EINVAL, "x/grad_out/grad_x/saved pointer is NULL");
  const ltc::Plan p = make_plan(B, T, D, H, ode_unfolds);
  Carver need{nullptr};
  carve_bwd(p, need);
  if (workspace_bytes < need.off || (need.off > 0 && !workspace))
    return fail(LTC_EINVAL, "workspace too small: need " + std::to_string(need.off) + " bytes");
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
    return fail(LTC_EINVAL, "workspace must be 256-byte aligned");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);

  if ((long long)B * T == 0) {
    // No unfolds: parameter gradients are zero and dL/dh0 = dL/dh_final.
    ltc::FillList fl = zero_list();
    for (float* z : {grad_w_pos, grad_w_erev, grad_mu, grad_sigma})
      ltc::fill_add(fl, z, nullptr, (long long)H * H);
    for (float* z : {grad_sensory_mu, grad_sensory_sigma, grad_sensory_erev, grad_sensory_w_pos})
      ltc::fill_add(fl, z, nullptr, (long long)D * H);
    for (float* z : {grad_cm_t, grad_gleak_pos, grad_vleak}) ltc::fill_add(fl, z, nullptr, H);
    ltc::fill_add(fl, grad_state, grad_h_final, (long long)B * H);
    return run_fill(fl, s);
  }

  Carver c{static_cast<char*>(workspace)};
  const BwdWs w = carve_bwd(p, c);
  const ltc::RawParams rp{w_pos, w_erev, mu, sigma, sensory_mu, sensory_sigma, sensory_erev,
                          sensory_w_pos, cm_t, gleak_pos, vleak};
  const ltc::Strides3 xs{sxb, sxt, sxd};
  const ltc::Strides3 gs{sgb, sgt, sgh};
  const float* vsave = saved;
  const float* densave = saved + ((long long)T * ode_unfolds + 1) * B * p.Hp;
  const ltc::GradOut go{grad_x, grad_w_pos, grad_w_erev, grad_mu, grad_sigma, grad_sensory_mu,
                        grad_sensory_sigma, grad_sensory_erev, grad_sensory_w_pos, grad_cm_t,
                        grad_gleak_pos, grad_vleak};

  hipError_t e;
  e = timed(ltc::K_PREP, s, [&] { return ltc::launch_prep(p, rp, w.pp, true, s); });
  if (e != hipSuccess) return hip_fail("prep launch", e);
  e = timed(ltc::K_ODE_BWD, s, [&] {
    return ltc::launch_ode_bwd(p, w.pp, vsave, densave, grad_out, gs, grad_h_final, w.absave,
                               w.dsn, w.dsd, w.npart, grad_state, w.rpart, w.cb, s);
  });
  if (e != hipSuccess) return hip_fail("ODE backward launch", e);
  if (!p.FUSE) {
    e = timed(ltc::K_REC_GRAD, s,
              [&] { return ltc::launch_rec_grad(p, w.pp, vsave, w.absave, w.rpart, s); });
    if (e != hipSuccess) return hip_fail("recurrent gradient launch", e);
  }
  e = timed(ltc::K_SENS_BWD, s, [&] {
    return ltc::launch_sens_bwd(p, x, xs, w.pp, w.dsn, w.dsd, w.spart, w.dxpart, s);
  });
  if (e != hipSuccess) return hip_fail("sensory backward launch", e);
  e = timed(ltc::K_FINALIZE, s, [&] {
    return ltc::launch_finalize(p, rp, w.rpart, w.spart, w.dxpart, w.npart, w.ps, go, s);
  });
  if (e != hipSuccess) return hip_fail("finalize launch", e);
  if (p.CP > 0) {
    ltc::FillList fl = poison_list(w.cb);
    ltc::fill_add(fl, grad_x, nullptr, (long long)B * T * D);
    ltc::fill_add(fl, grad_state, nullptr, (long long)B * H);
    for (float* z : {grad_w_pos, grad_w_erev, grad_mu, grad_sigma})
      ltc::fill_add(fl, z, nullptr, (long long)H * H);
    for (float* z : {grad_sensory_mu, grad_sensory_sigma, grad_sensory_erev, grad_sensory_w_pos})
      ltc::fill_add(fl, z, nullptr, (long long)D * H);
    for (float* z : {grad_cm_t, grad_gleak_pos, grad_vleak}) ltc::fill_add(fl, z, nullptr, H);
    return run_fill(fl, s);
  }
  return LTC_OK;
}

long long ltc_module_saved_floats(int B, int T, int D, int H, int ode_unfolds) {
  if (check_dims(B, T, D, H, ode_unfolds) != LTC_OK || D > ltc::kModuleMaxD) return -1;
  return module_saved_floats(make_plan(B, T, D, H, ode_unfolds));
}

long long ltc_module_fwd_workspace_bytes(int B, int T, int D, int H, int ode_unfolds) {
  if (check_dims(B, T, D, H, ode_unfolds) != LTC_OK || D > ltc::kModuleMaxD) return -1;
  const ltc::Plan p = make_plan(B, T, D, H, ode_unfolds);
  Carver c{nullptr};
  carve_fwd(p, c);
  carve_ln(p, c);  // used when nothing is saved (inference)
  return round_up(c.off, 256);
}

long long ltc_module_bwd_workspace_bytes(int B, int T, int D, int H, int ode_unfolds) {
  if (check_dims(B, T, D, H, ode_unfolds) != LTC_OK || D > ltc::kModuleMaxD) return -1;
  const ltc::Plan p = make_plan(B, T, D, H, ode_unfolds);
  Carver c{nullptr};
  carve_bwd(p, c, false);
  c.take<float>(module_ln_parts(p) * 4 * p.Dp);
  return round_up(c.off, 256);
}

namespace {

int check_leaves(const ltc::LeafParams& lp) {
  if (!lp.w || !lp.erev || !lp.mask || !lp.mu || !lp.sigma || !lp.s_w || !lp.s_erev ||
      !lp.s_mask || !lp.s_mu || !lp.s_sigma || !lp.gleak || !lp.vleak || !lp.cm ||
      !lp.input_w || !lp.input_b || !lp.ln_w || !lp.ln_b)
    return fail(LTC_EINVAL, "parameter pointer is NULL");
  if (!(lp.dtU > 0.f)) return fail(LTC_EINVAL, "dt / ode_unfolds must be positive");
  return LTC_OK;
}

}  // namespace

int ltc_module_forward(const float* x, long long sxb, long long sxt, long long sxd,
                       const float* state, const float* w, const float* erev, const float* mask,
                       const float* mu, const float* sigma, const float* sensory_w,
                       const float* sensory_erev, const float* sensory_mask,
                       const float* sensory_mu, const float* sensory_sigma, const float* gleak,
                       const float* vleak, const float* cm, const float* input_w,
                       const float* input_b, const float* ln_weight, const float* ln_bias,
                       int B, int T, int D, int H, int ode_unfolds, float dt, float epsilon,
                       float ln_eps, int save_intermediates, float* out, float* h_final,
                       float* saved, void* workspace, long long workspace_bytes, void* stream) {
  g_err.clear();
  int rc = check_dims(B, T, D, H, ode_unfolds);
  if (rc != LTC_OK) return rc;
  if (D > ltc::kModuleMaxD)
    return fail(LTC_EUNSUPPORTED, "module path handles D <= " + std::to_string(ltc::kModuleMaxD));
  const ltc::LeafParams lp{w, erev, mask, mu, sigma, sensory_w, sensory_erev, sensory_mask,
                           sensory_mu, sensory_sigma, gleak, vleak, cm, input_w, input_b,
                           ln_weight, ln_bias, (float)((double)dt / ode_unfolds), ln_eps};
  rc = check_leaves(lp);
  if (rc != LTC_OK) return rc;
  if (B > 0 && !h_final) return fail(LTC_EINVAL, "h_final pointer is NULL");
  if ((long long)B * T > 0 && (!x || !out)) return fail(LTC_EINVAL, "x/out pointer is NULL");
  if (save_intermediates && !saved) return fail(LTC_EINVAL, "saved pointer is NULL");
  const ltc::Plan p = make_plan(B, T, D, H, ode_unfolds);
  Carver need{nullptr};
  carve_fwd(p, need);
  carve_ln(p, need);
  if (workspace_bytes < need.off || (need.off > 0 && !workspace))
    return fail(LTC_EINVAL, "workspace too small: need " + std::to_string(need.off) + " bytes");
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
    return fail(LTC_EINVAL, "workspace must be 256-byte aligned");
  if (B == 0) return LTC_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (T == 0) {
    ltc::FillList fl = zero_list();
    ltc::fill_add(fl, h_final, state, (long long)B * H);
    return run_fill(fl, s);
  }
  Carver c{static_cast<char*>(workspace)};
  const FwdWs wfw = carve_fwd(p, c);
  LnWs lw = carve_ln(p, c);
  ltc::Prepped pp = wfw.pp;
  int images = ltc::kLeafFwdImages;
  float* vsave = nullptr;
  float* densave = nullptr;
  unsigned long long* row_words = nullptr;
  if (save_intermediates) {
    // Training: LayerNorm rows and every parameter image go to the saved
    // buffer, so the backward starts with the chain (no image launch).
    vsave = saved;
    densave = saved + ((long long)T * ode_unfolds + 1) * B * p.Hp;
    Carver sc{reinterpret_cast<char*>(saved)};
    sc.take<float>(saved_floats(p));
    lw = carve_ln(p, sc);
    pp = carve_images(p, sc);
    row_words = carve_row_words(p, sc);
    images |= ltc::kLeafBwdImages;
  }
  const ltc::LnBuf ln{x, {sxb, sxt, sxd}, lw.xa, lw.stats};
  const ltc::Strides3 xas{(long long)T * D, D, 1};
  // Few rows: the prep launch forms the sensory sums too (one launch fewer).
  auto al16 = [](const float* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const bool sens_in_prep = ltc::prep_sens_fused(p) && al16(sensory_w) && al16(sensory_erev) &&
                            al16(sensory_mask) && al16(sensory_mu) && al16(sensory_sigma);
  // otherwise the sensory launch reads the compacted image (in the workspace)
  pp.sF = sens_in_prep ? nullptr : wfw.pp.sF;
  pp.sFi = sens_in_prep ? nullptr : wfw.pp.sFi;
  pp.sFn = sens_in_prep ? nullptr : wfw.pp.sFn;
  pp.sFfull = wfw.pp.sFfull;
  // Without saving, nothing but the sensory launch reads the normalised rows:
  // when they fit one 64-input chunk, it normalises them itself.
  const bool ln_in_sens = !save_intermediates && !sens_in_prep && ltc::sens_fwd_ln_fusable(p);
  hipError_t e;
  e = timed(ltc::K_PREP, s, [&] {
    return ltc::launch_prep_leaf(p, lp, pp, images, ln_in_sens ? nullptr : &ln, s, row_words,
                                 row_words ? ltc::row_bwd_words(p) : 0,
                                 sens_in_prep ? wfw.sn : nullptr, sens_in_prep ? wfw.sd : nullptr);
  });
  if (e != hipSuccess) return hip_fail("prep launch", e);
  if (ln_in_sens) {
    const ltc::LnAff la{ln_weight, ln_bias, input_w, input_b, ln_eps};
    e = timed(ltc::K_SENS_FWD, s, [&] {
      return ltc::launch_sens_fwd_ln(p, x, ltc::Strides3{sxb, sxt, sxd}, pp, la, wfw.sn, wfw.sd,
                                     s);
    });
    if (e != hipSuccess) return hip_fail("sensory forward launch", e);
  } else if (!sens_in_prep) {
    e = timed(ltc::K_SENS_FWD, s,
              [&] { return ltc::launch_sens_fwd(p, lw.xa, xas, pp, wfw.sn, wfw.sd, s); });
    if (e != hipSuccess) return hip_fail("sensory forward launch", e);
  }
  e = timed(ltc::K_ODE_FWD, s, [&] {
    return ltc::launch_ode_fwd(p, pp, wfw.sn, wfw.sd, state, epsilon, out, h_final, vsave,
                               densave, wfw.cb, s);
  });
  if (e != hipSuccess) return hip_fail("ODE forward launch", e);
  if (p.CP > 0) {
    ltc::FillList fl = poison_list(wfw.cb);
    ltc::fill_add(fl, out, nullptr, (long long)B * T * H);
    ltc::fill_add(fl, h_final, nullptr, (long long)B * H);
    ltc::fill_add(fl, saved, nullptr, save_intermediates ? saved_floats(p) : 0);
    return run_fill(fl, s);
  }
  return LTC_OK;
}

int ltc_module_backward(const float* x, long long sxb, long long sxt, long long sxd,
                        const float* w, const float* erev, const float* mask, const float* mu,
                        const float* sigma, const float* sensory_w, const float* sensory_erev,
                        const float* sensory_mask, const float* sensory_mu,
                        const float* sensory_sigma, const float* gleak, const float* vleak,
                        const float* cm, const float* input_w, const float* input_b,
                        const float* ln_weight, const float* ln_bias, const float* saved,
                        const float* grad_out, long long sgb, long long sgt, long long sgh,
                        const float* grad_h_final, int B, int T, int D, int H, int ode_unfolds,
                        float dt, float epsilon, float ln_eps, float* grad_x, float* grad_state,
                        float* grad_w, float* grad_erev, float* grad_mu, float* grad_sigma,
                        float* grad_sensory_w, float* grad_sensory_erev, float* grad_sensory_mu,
                        float* grad_sensory_sigma, float* grad_gleak, float* grad_vleak,
                        float* grad_cm, float* grad_input_w, float* grad_input_b,
                        float* grad_ln_weight, float* grad_ln_bias, void* workspace,
                        long long workspace_bytes, void* stream) {
  g_err.clear();
  (void)epsilon;  // the saved denominators already include it
  int rc = check_dims(B, T, D, H, ode_unfolds);
  if (rc != LTC_OK) return rc;
  if (D > ltc::kModuleMaxD)
    return fail(LTC_EUNSUPPORTED, "module path handles D <= " + std::to_string(ltc::kModuleMaxD));
  const ltc::LeafParams lp{w, erev, mask, mu, sigma, sensory_w, sensory_erev, sensory_mask,
                           sensory_mu, sensory_sigma, gleak, vleak, cm, input_w, input_b,
                           ln_weight, ln_bias, (float)((double)dt / ode_unfolds), ln_eps};
  rc = check_leaves(lp);
  if (rc != LTC_OK) return rc;
  const ltc::LeafGrads lg{grad_x, grad_w, grad_erev, grad_mu, grad_sigma, grad_sensory_w,
                          grad_sensory_erev, grad_sensory_mu, grad_sensory_sigma, grad_gleak,
                          grad_vleak, grad_cm, grad_input_w, grad_input_b, grad_ln_weight,
                          grad_ln_bias};
  if (!lg.w || !lg.erev || !lg.mu || !lg.sigma || !lg.s_w || !lg.s_erev || !lg.s_mu ||
      !lg.s_sigma || !lg.gleak || !lg.vleak || !lg.cm || !lg.input_w || !lg.input_b ||
      !lg.ln_w || !lg.ln_b)
    return fail(LTC_EINVAL, "gradient output pointer is NULL");
  if ((long long)B * T > 0 && (!x || !grad_out || !grad_x || !saved))
    return fail(LTC_EINVAL, "x/grad_out/grad_x/saved pointer is NULL");
  const ltc::Plan p = make_plan(B, T, D, H, ode_unfolds);
  Carver need{nullptr};
  carve_bwd(p, need, false);
  need.take<float>((long long)module_ln_parts(p) * 4 * p.Dp);
  if (workspace_bytes < need.off || (need.off > 0 && !workspace))
    return fail(LTC_EINVAL, "workspace too small: need " + std::to_string(need.off) + " bytes");
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
    return fail(LTC_EINVAL, "workspace must be 256-byte aligned");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if ((long long)B * T == 0) {
    ltc::FillList fl = zero_list();
    for (float* z : {grad_w, grad_erev, grad_mu, grad_sigma})
      ltc::fill_add(fl, z, nullptr, (long long)H * H);
    for (float* z : {grad_sensory_w, grad_sensory_erev, grad_sensory_mu, grad_sensory_sigma})
      ltc::fill_add(fl, z, nullptr, (long long)D * H);
    for (float* z : {grad_gleak, grad_vleak, grad_cm}) ltc::fill_add(fl, z, nullptr, H);
    for (float* z : {grad_input_w, grad_input_b, grad_ln_weight, grad_ln_bias})
      ltc::fill_add(fl, z, nullptr, D);
    ltc::fill_add(fl, grad_state, grad_h_final, (long long)B * H);
    return run_fill(fl, s);
  }
  Carver c{static_cast<char*>(workspace)};
  BwdWs wb = carve_bwd(p, c, false);
  float* lnpart = c.take<float>((long long)module_ln_parts(p) * 4 * p.Dp);
  Carver sc{const_cast<char*>(reinterpret_cast<const char*>(saved))};
  sc.take<float>(saved_floats(p));
  const LnWs lw = carve_ln(p, sc);
  wb.pp = carve_images(p, sc);  // built by the forward (ltc_module_forward)
  unsigned long long* row_words = carve_row_words(p, sc);  // cleared by the forward
  const ltc::LnBuf ln{x, {sxb, sxt, sxd}, lw.xa, lw.stats};
  const ltc::Strides3 xas{(long long)T * D, D, 1};
  const ltc::Strides3 gs{sgb, sgt, sgh};
  const float* vsave = saved;
  const float* densave = saved + ((long long)T * ode_unfolds + 1) * B * p.Hp;
  hipError_t e;
  if (ltc::row_bwd_fused(p)) {
    // The sensory and LayerNorm backward run inside the chain launch.
    const ltc::RowCompanion rc{lw.xa, ln, input_w, ln_weight, ln_bias, wb.spart, lnpart,
                               grad_x, row_words, g_spin.load(std::memory_order_relaxed)};
    e = timed(ltc::K_ODE_BWD, s, [&] {
      return ltc::launch_ode_bwd_row_fused(p, wb.pp, vsave, densave, grad_out, gs, grad_h_final,
                                           wb.npart, grad_state, wb.rpart, rc, s);
    });
    if (e != hipSuccess) return hip_fail("ODE backward launch", e);
    const int* status = reinterpret_cast<const int*>(row_words + ltc::row_bwd_words(p) - 1);
    e = timed(ltc::K_FINALIZE, s, [&] {
      return ltc::launch_finalize_leaf_fused(p, lp, wb.rpart, wb.spart, wb.npart, lnpart, wb.ps,
                                             lg, status, grad_state, s);
    });
    if (e != hipSuccess) return hip_fail("finalize launch", e);
    return LTC_OK;
  }
  // At Hp = 128 (one row per workgroup) the recurrent-gradient sums are formed
  // inside the chain launch by companion workgroups: one partial per row.
  ltc::Plan pf = p;
  const int* status = nullptr;
  const bool sens_comp = ltc::row128_sens_fused(p);
  if (ltc::row128_rec_fused(p)) {
    // with D <= 128 the sensory and LayerNorm backward run in that launch too
    unsigned long long* words = row_words;
    const long long spin = g_spin.load(std::memory_order_relaxed);
    const ltc::RowCompanion sc{lw.xa, ln, input_w, ln_weight, ln_bias, wb.spart, lnpart,
                               grad_x, words, spin};
    e = timed(ltc::K_ODE_BWD, s, [&] {
      return ltc::launch_ode_bwd_row128_rec(p, wb.pp, vsave, densave, grad_out, gs,
                                            grad_h_final, wb.dsn, wb.dsd, wb.npart, grad_state,
                                            wb.rpart, words, spin, sens_comp ? &sc : nullptr, s);
    });
    if (e != hipSuccess) return hip_fail("ODE backward launch", e);
    pf.NCH = p.B;
    if (sens_comp) pf.NRC = p.B;
    status = reinterpret_cast<const int*>(words + ltc::row_bwd_words(p) - 1);
  } else {
    e = timed(ltc::K_ODE_BWD, s, [&] {
      return ltc::launch_ode_bwd(p, wb.pp, vsave, densave, grad_out, gs, grad_h_final,
                                 wb.absave, wb.dsn, wb.dsd, wb.npart, grad_state, wb.rpart, wb.cb,
                                 s);
    });
    if (e != hipSuccess) return hip_fail("ODE backward launch", e);
    if (!p.FUSE) {
      e = timed(ltc::K_REC_GRAD, s,
                [&] { return ltc::launch_rec_grad(p, wb.pp, vsave, wb.absave, wb.rpart, s); });
      if (e != hipSuccess) return hip_fail("recurrent gradient launch", e);
    }
  }
  if (!sens_comp) {
    e = timed(ltc::K_SENS_BWD, s, [&] {
      return ltc::launch_sens_bwd(p, lw.xa, xas, wb.pp, wb.dsn, wb.dsd, wb.spart, wb.dxpart, s,
                                  lp.s_mask);
    });
    if (e != hipSuccess) return hip_fail("sensory backward launch", e);
  }
  if (!sens_comp) {
    e = timed(ltc::K_LN_BWD, s,
              [&] { return ltc::launch_ln_bwd(p, lp, ln, wb.dxpart, grad_x, lnpart, s); });
    if (e != hipSuccess) return hip_fail("LayerNorm backward launch", e);
  }
  e = timed(ltc::K_FINALIZE, s, [&] {
    return ltc::launch_finalize_leaf(pf, lp, wb.rpart, wb.spart, wb.npart, lnpart, wb.ps, lg, s,
                                     status, grad_state);
  });
  if (e != hipSuccess) return hip_fail("finalize launch", e);
  if (p.CP > 0) {
    ltc::FillList fl = poison_list(wb.cb);
    ltc::fill_add(fl, grad_x, nullptr, (long long)B * T * D);
    ltc::fill_add(fl, grad_state, nullptr, (long long)B * H);
    for (float* z : {grad_w, grad_erev, grad_mu, grad_sigma})
      ltc::fill_add(fl, z, nullptr, (long long)H * H);
    for (float* z : {grad_sensory_w, grad_sensory_erev, grad_sensory_mu, grad_sensory_sigma})
      ltc::fill_add(fl, z, nullptr, (long long)D * H);
    for (float* z : {grad_gleak, grad_vleak, grad_cm}) ltc::fill_add(fl, z, nullptr, H);
    for (float* z : {grad_input_w, grad_input_b, grad_ln_weight, grad_ln_bias})
      ltc::fill_add(fl, z, nullptr, D);
    return run_fill(fl, s);
  }
  return LTC_OK;
}

// ---------------------------------------------------------------------------
// Per-step entry points of the reference (csrc/ltc_kernels.cu:674-950): one
// time step's sensory sums, one step's U unfolds, and their backward passes,
// as thin wrappers over the same kernels with T = 1.
// ---------------------------------------------------------------------------
namespace {

struct SensWs {
  ltc::Prepped pp;
  float* sn;    // [B][Hp]
  float* sd;
  float* spart;
  float* dxpart;
};

SensWs carve_sens(const ltc::Plan& p, Carver& c, bool bwd) {
  SensWs w{};
  const long long img = (long long)p.Dp * p.Hp;
  if (bwd)
    w.pp.sensB = c.take<float4>(img);
  else
    w.pp.sensF = c.take<float4>(img);
  w.sn = c.take<float>((long long)p.B * p.Hp);
  w.sd = c.take<float>((long long)p.B * p.Hp);
  if (bwd) {
    // sensory partials: NRC row chunks, or one per batch row (fused row backward)
  const long long nrc = ltc::row_bwd_fused(p) && p.B > p.NRC ? p.B : p.NRC;
  w.spart = c.take<float>(nrc * 4 * p.Dp * p.Hp);
    w.dxpart = c.take<float>((long long)(p.Hp / 32) * p.B * p.Dp);
  }
  return w;
}

// One-step unfold workspace: the full-path regions with T = 1 (the backward
// also recomputes the forward, so it holds both), plus the padded sensory
// sums, the recomputed unfold states and a scratch final state.
struct UnfoldWs {
  FwdWs f;
  BwdWs b;
  float* vsave;  // saved_floats(p)
  float* hscr;   // [B][H]
};

UnfoldWs carve_unfold(const ltc::Plan& p, Carver& c, bool bwd) {
  UnfoldWs w{};
  w.f = carve_fwd(p, c, false);
  if (bwd) {
    w.b = carve_bwd(p, c);
    w.hscr = c.take<float>((long long)p.B * p.H);
  }
  w.vsave = c.take<float>(saved_floats(p));
  return w;
}

int check_ws(long long need, void* workspace, long long workspace_bytes) {
  if (workspace_bytes < need || (need > 0 && !workspace))
    return fail(LTC_EINVAL, "workspace too small: need " + std::to_string(need) + " bytes");
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
    return fail(LTC_EINVAL, "workspace must be 256-byte aligned");
  return LTC_OK;
}

int check_step_dims(int B, int D, int H, int U) {
  if (B < 0 || D < 1 || H < 1) return fail(LTC_EINVAL, "dimensions must satisfy B >= 0, D >= 1, H >= 1");
  return check_dims(B, 1, D, H, U);
}

}  // namespace

long long ltc_sensory_fwd_workspace_bytes(int B, int D, int H) {
  if (check_step_dims(B, D, H, 1) != LTC_OK) return -1;
  const ltc::Plan p = make_plan(B, 1, D, H, 1);
  Carver c{nullptr};
  carve_sens(p, c, false);
  return round_up(c.off, 256);
}

long long ltc_sensory_bwd_workspace_bytes(int B, int D, int H) {
  if (check_step_dims(B, D, H, 1) != LTC_OK) return -1;
  const ltc::Plan p = make_plan(B, 1, D, H, 1);
  Carver c{nullptr};
  carve_sens(p, c, true);
  return round_up(c.off, 256);
}

long long ltc_ode_unfold_fwd_workspace_bytes(int B, int H, int ode_unfolds) {
  if (check_step_dims(B, 1, H, ode_unfolds) != LTC_OK) return -1;
  const ltc::Plan p = make_plan(B, 1, 1, H, ode_unfolds);
  Carver c{nullptr};
  carve_unfold(p, c, false);
  return round_up(c.off, 256);
}

long long ltc_ode_unfold_bwd_workspace_bytes(int B, int H, int ode_unfolds) {
  if (check_step_dims(B, 1, H, ode_unfolds) != LTC_OK) return -1;
  const ltc::Plan p = make_plan(B, 1, 1, H, ode_unfolds);
  Carver c{nullptr};
  carve_unfold(p, c, true);
  return round_up(c.off, 256);
}

int ltc_sensory_fwd(const float* inputs, long long sib, long long sid,
                    const float* sensory_sigma, const float* sensory_mu,
                    const float* sensory_w_pos, const float* sensory_erev, int B, int D, int H,
                    float* w_num_sensory, float* w_den_sensory, void* workspace,
                    long long workspace_bytes, void* stream) {
  g_err.clear();
  int rc = check_step_dims(B, D, H, 1);
  if (rc != LTC_OK) return rc;
  if (!sensory_sigma || !sensory_mu || !sensory_w_pos || !sensory_erev)
    return fail(LTC_EINVAL, "parameter pointer is NULL");
  if (B > 0 && (!inputs || !w_num_sensory || !w_den_sensory))
    return fail(LTC_EINVAL, "inputs/w_num_sensory/w_den_sensory pointer is NULL");
  const ltc::Plan p = make_plan(B, 1, D, H, 1);
  Carver need{nullptr};
  carve_sens(p, need, false);
  rc = check_ws(need.off, workspace, workspace_bytes);
  if (rc != LTC_OK) return rc;
  if (B == 0) return LTC_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  Carver c{static_cast<char*>(workspace)};
  const SensWs w = carve_sens(p, c, false);
  const ltc::RawParams rp{nullptr, nullptr, nullptr, nullptr, sensory_mu, sensory_sigma,
                          sensory_erev, sensory_w_pos, nullptr, nullptr, nullptr};
  hipError_t e;
  e = timed(ltc::K_PREP, s, [&] { return ltc::launch_prep(p, rp, w.pp, false, s, ltc::kPrepSens); });
  if (e != hipSuccess) return hip_fail("prep launch", e);
  e = timed(ltc::K_SENS_FWD, s, [&] {
    return ltc::launch_sens_fwd(p, inputs, ltc::Strides3{sib, 0, sid}, w.pp, w.sn, w.sd, s);
  });
  if (e != hipSuccess) return hip_fail("sensory forward launch", e);
  e = ltc::launch_copy_rows(w.sn, p.Hp, w_num_sensory, H, B, H, s);
  if (e == hipSuccess) e = ltc::launch_copy_rows(w.sd, p.Hp, w_den_sensory, H, B, H, s);
  if (e != hipSuccess) return hip_fail("copy launch", e);
  return LTC_OK;
}

int ltc_sensory_bwd(const float* grad_w_num, const float* grad_w_den, const float* inputs,
                    long long sib, long long sid, const float* sensory_sigma,
                    const float* sensory_mu, const float* sensory_w_pos,
                    const float* sensory_erev, int B, int D, int H, float* grad_inputs,
                    float* grad_sensory_sigma, float* grad_sensory_mu,
                    float* grad_sensory_w_pos, float* grad_sensory_erev, void* workspace,
                    long long workspace_bytes, void* stream) {
  g_err.clear();
  int rc = check_step_dims(B, D, H, 1);
  if (rc != LTC_OK) return rc;
  if (!sensory_sigma || !sensory_mu || !sensory_w_pos || !sensory_erev)
    return fail(LTC_EINVAL, "parameter pointer is NULL");
  if (!grad_sensory_sigma || !grad_sensory_mu || !grad_sensory_w_pos || !grad_sensory_erev)
    return fail(LTC_EINVAL, "gradient output pointer is NULL");
  if (B > 0 && (!grad_w_num || !grad_w_den || !inputs || !grad_inputs))
    return fail(LTC_EINVAL, "grad_w_num/grad_w_den/inputs/grad_inputs pointer is NULL");
  const ltc::Plan p = make_plan(B, 1, D, H, 1);
  Carver need{nullptr};
  carve_sens(p, need, true);
  rc = check_ws(need.off, workspace, workspace_bytes);
  if (rc != LTC_OK) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (B == 0) {
    ltc::FillList fl = zero_list();
    for (float* z : {grad_sensory_sigma, grad_sensory_mu, grad_sensory_w_pos, grad_sensory_erev})
      ltc::fill_add(fl, z, nullptr, (long long)D * H);
    return run_fill(fl, s);
  }
  Carver c{static_cast<char*>(workspace)};
  const SensWs w = carve_sens(p, c, true);
  const ltc::RawParams rp{nullptr, nullptr, nullptr, nullptr, sensory_mu, sensory_sigma,
                          sensory_erev, sensory_w_pos, nullptr, nullptr, nullptr};
  const ltc::Strides3 xs{sib, 0, sid};
  ltc::GradOut go{};
  go.x = grad_inputs;
  go.s_mu = grad_sensory_mu;
  go.s_sigma = grad_sensory_sigma;
  go.s_erev = grad_sensory_erev;
  go.s_wpos = grad_sensory_w_pos;
  hipError_t e;
  e = timed(ltc::K_PREP, s, [&] { return ltc::launch_prep(p, rp, w.pp, true, s, ltc::kPrepSens); });
  if (e != hipSuccess) return hip_fail("prep launch", e);
  e = ltc::launch_copy_rows(grad_w_num, H, w.sn, p.Hp, B, H, s);
  if (e == hipSuccess) e = ltc::launch_copy_rows(grad_w_den, H, w.sd, p.Hp, B, H, s);
  if (e != hipSuccess) return hip_fail("copy launch", e);
  e = timed(ltc::K_SENS_BWD, s, [&] {
    return ltc::launch_sens_bwd(p, inputs, xs, w.pp, w.sn, w.sd, w.spart, w.dxpart, s);
  });
  if (e != hipSuccess) return hip_fail("sensory backward launch", e);
  e = timed(ltc::K_FINALIZE, s, [&] {
    return ltc::launch_finalize(p, rp, nullptr, w.spart, w.dxpart, nullptr, ltc::PresumBuf{},
                                go, s, ltc::kFinSens);
  });
  if (e != hipSuccess) return hip_fail("finalize launch", e);
  return LTC_OK;
}

int ltc_ode_unfold_fwd(const float* state, const float* w_pos, const float* w_erev,
                       const float* mu, const float* sigma, const float* w_num_sensory,
                       const float* w_den_sensory, const float* cm_t, const float* gleak_pos,
                       const float* vleak, int B, int H, int ode_unfolds, float epsilon,
                       int save_intermediates, float* state_out, float* v_buffer,
                       void* workspace, long long workspace_bytes, void* stream) {
  g_err.clear();
  int rc = check_step_dims(B, 1, H, ode_unfolds);
  if (rc != LTC_OK) return rc;
  if (!w_pos || !w_erev || !mu || !sigma || !cm_t || !gleak_pos || !vleak)
    return fail(LTC_EINVAL, "parameter pointer is NULL");
  if (B > 0 && (!state || !w_num_sensory || !w_den_sensory || !state_out))
    return fail(LTC_EINVAL, "state/w_num_sensory/w_den_sensory/state_out pointer is NULL");
  if (B > 0 && save_intermediates && !v_buffer)
    return fail(LTC_EINVAL, "v_buffer pointer is NULL");
  const ltc::Plan p = make_plan(B, 1, 1, H, ode_unfolds);
  Carver need{nullptr};
  carve_unfold(p, need, false);
  rc = check_ws(need.off, workspace, workspace_bytes);
  if (rc != LTC_OK) return rc;
  if (B == 0) return LTC_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  Carver c{static_cast<char*>(workspace)};
  const UnfoldWs w = carve_unfold(p, c, false);
  const ltc::RawParams rp{w_pos, w_erev, mu, sigma, nullptr, nullptr, nullptr, nullptr,
                          cm_t, gleak_pos, vleak};
  float* vsave = save_intermediates ? w.vsave : nullptr;
  float* densave = save_intermediates ? w.vsave + ((long long)ode_unfolds + 1) * B * p.Hp : nullptr;
  hipError_t e;
  e = timed(ltc::K_PREP, s, [&] {
    return ltc::launch_prep(p, rp, w.f.pp, false, s, ltc::kPrepRec | ltc::kPrepNeuron);
  });
  if (e != hipSuccess) return hip_fail("prep launch", e);
  e = ltc::launch_copy_rows(w_num_sensory, H, w.f.sn, p.Hp, B, H, s);
  if (e == hipSuccess) e = ltc::launch_copy_rows(w_den_sensory, H, w.f.sd, p.Hp, B, H, s);
  if (e != hipSuccess) return hip_fail("copy launch", e);
  // T = 1: the kernel's (B,T,H) output and its final state are the same (B,H)
  // values, written by the same thread.
  e = timed(ltc::K_ODE_FWD, s, [&] {
    return ltc::launch_ode_fwd(p, w.f.pp, w.f.sn, w.f.sd, state, epsilon, state_out, state_out,
                               vsave, densave, w.f.cb, s);
  });
  if (e != hipSuccess) return hip_fail("ODE forward launch", e);
  if (save_intermediates) {
    e = ltc::launch_copy_rows(vsave, p.Hp, v_buffer, H, (long long)ode_unfolds * B, H, s);
    if (e != hipSuccess) return hip_fail("copy launch", e);
  }
  if (p.CP > 0) {
    ltc::FillList fl = poison_list(w.f.cb);
    ltc::fill_add(fl, state_out, nullptr, (long long)B * H);
    ltc::fill_add(fl, v_buffer, nullptr, save_intermediates ? (long long)ode_unfolds * B * H : 0);
    return run_fill(fl, s);
  }
  return LTC_OK;
}

int ltc_ode_unfold_bwd(const float* v_buffer, const float* w_pos, const float* w_erev,
                       const float* mu, const float* sigma, const float* w_num_sensory,
                       const float* w_den_sensory, const float* cm_t, const float* gleak_pos,
                       const float* vleak, const float* grad_output, int B, int H,
                       int ode_unfolds, float epsilon, float* grad_v,
                       float* grad_w_num_sensory, float* grad_w_den_sensory,
                       float* grad_w_pos, float* grad_w_erev, float* grad_mu,
                       float* grad_sigma, float* grad_cm_t, float* grad_gleak_pos,
                       float* grad_vleak, void* workspace, long long workspace_bytes,
                       void* stream) {
  g_err.clear();
  int rc = check_step_dims(B, 1, H, ode_unfolds);
  if (rc != LTC_OK) return rc;
  if (!w_pos || !w_erev || !mu || !sigma || !cm_t || !gleak_pos || !vleak)
    return fail(LTC_EINVAL, "parameter pointer is NULL");
  if (!grad_w_pos || !grad_w_erev || !grad_mu || !grad_sigma || !grad_cm_t || !grad_gleak_pos ||
      !grad_vleak)
    return fail(LTC_EINVAL, "gradient output pointer is NULL");
  if (B > 0 && (!v_buffer || !w_num_sensory || !w_den_sensory || !grad_output || !grad_v ||
                !grad_w_num_sensory || !grad_w_den_sensory))
    return fail(LTC_EINVAL, "v_buffer/sensory/grad_output/grad_v pointer is NULL");
  const ltc::Plan p = make_plan(B, 1, 1, H, ode_unfolds);
  Carver need{nullptr};
  carve_unfold(p, need, true);
  rc = check_ws(need.off, workspace, workspace_bytes);
  if (rc != LTC_OK) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (B == 0) {
    ltc::FillList fl = zero_list();
    for (float* z : {grad_w_pos, grad_w_erev, grad_mu, grad_sigma})
      ltc::fill_add(fl, z, nullptr, (long long)H * H);
    for (float* z : {grad_cm_t, grad_gleak_pos, grad_vleak}) ltc::fill_add(fl, z, nullptr, H);
    return run_fill(fl, s);
  }
  Carver c{static_cast<char*>(workspace)};
  const UnfoldWs w = carve_unfold(p, c, true);
  const ltc::RawParams rp{w_pos, w_erev, mu, sigma, nullptr, nullptr, nullptr, nullptr,
                          cm_t, gleak_pos, vleak};
  const int U = ode_unfolds;
  float* vsave = w.vsave;
  float* densave = w.vsave + ((long long)U + 1) * B * p.Hp;
  ltc::GradOut go{};
  go.w_pos = grad_w_pos;
  go.w_erev = grad_w_erev;
  go.mu = grad_mu;
  go.sigma = grad_sigma;
  go.cm = grad_cm_t;
  go.gleak = grad_gleak_pos;
  go.vleak = grad_vleak;
  hipError_t e;
  // Backward-mode images (recF for the recompute and rec_grad, recB for the
  // chain) and the per-neuron vectors.
  e = timed(ltc::K_PREP, s, [&] {
    return ltc::launch_prep(p, rp, w.b.pp, true, s, ltc::kPrepRec | ltc::kPrepNeuron);
  });
  if (e != hipSuccess) return hip_fail("prep launch", e);
  e = ltc::launch_copy_rows(w_num_sensory, H, w.f.sn, p.Hp, B, H, s);
  if (e == hipSuccess) e = ltc::launch_copy_rows(w_den_sensory, H, w.f.sd, p.Hp, B, H, s);
  if (e != hipSuccess) return hip_fail("copy launch", e);
  // The unfold states and reciprocal denominators, recomputed from v_buffer[0] (the
  // reference's backward kernels recompute each unfold from its saved
  // pre-state, csrc/ltc_kernels.cu:549-668).
  e = timed(ltc::K_ODE_FWD, s, [&] {
    return ltc::launch_ode_fwd(p, w.b.pp, w.f.sn, w.f.sd, v_buffer, epsilon, w.hscr, w.hscr,
                               vsave, densave, w.f.cb, s);
  });
  if (e != hipSuccess) return hip_fail("ODE forward launch", e);
  // dL/dv^U enters as the output gradient of the single step.
  const ltc::Strides3 gs{H, 0, 1};
  e = timed(ltc::K_ODE_BWD, s, [&] {
    return ltc::launch_ode_bwd(p, w.b.pp, vsave, densave, grad_output, gs, nullptr, w.b.absave,
                               w.b.dsn, w.b.dsd, w.b.npart, grad_v, w.b.rpart, w.b.cb, s);
  });
  if (e != hipSuccess) return hip_fail("ODE backward launch", e);
  if (!p.FUSE) {
    e = timed(ltc::K_REC_GRAD, s,
              [&] { return ltc::launch_rec_grad(p, w.b.pp, vsave, w.b.absave, w.b.rpart, s); });
    if (e != hipSuccess) return hip_fail("recurrent gradient launch", e);
  }
  e = ltc::launch_copy_rows(w.b.dsn, p.Hp, grad_w_num_sensory, H, B, H, s);
  if (e == hipSuccess) e = ltc::launch_copy_rows(w.b.dsd, p.Hp, grad_w_den_sensory, H, B, H, s);
  if (e != hipSuccess) return hip_fail("copy launch", e);
  e = timed(ltc::K_FINALIZE, s, [&] {
    return ltc::launch_finalize(p, rp, w.b.rpart, nullptr, nullptr, w.b.npart, w.b.ps, go, s,
                                ltc::kFinRec);
  });
  if (e != hipSuccess) return hip_fail("finalize launch", e);
  if (p.CP > 0) {
    // Either the recompute (forward) or the chain may have given up; both
    // status words gate the same fill.
    for (const ltc::ClusterBuf* cb : {&w.f.cb, &w.b.cb}) {
      ltc::FillList fl = poison_list(*cb);
      for (float* z : {grad_v, grad_w_num_sensory, grad_w_den_sensory})
        ltc::fill_add(fl, z, nullptr, (long long)B * H);
      for (float* z : {grad_w_pos, grad_w_erev, grad_mu, grad_sigma})
        ltc::fill_add(fl, z, nullptr, (long long)H * H);
      for (float* z : {grad_cm_t, grad_gleak_pos, grad_vleak}) ltc::fill_add(fl, z, nullptr, H);
      const int rc = run_fill(fl, s);
      if (rc != LTC_OK) return rc;
    }
  }
  return LTC_OK;
}

int ltc_launch_plan(int B, int T, int D, int H, int ode_unfolds, long long* out, int n) {
  if (check_dims(B, T, D, H, ode_unfolds) != LTC_OK || !out || n < 0) return -1;
  const ltc::Plan p = make_plan(B, T, D, H, ode_unfolds);
  // Columns each workgroup of the ODE kernels owns: all Hp, or one member's.
  const long long cols = p.CP > 0 ? 64 : p.Hp;
  const long long colsb = p.CP > 0 ? p.JWB : p.Hp;
  const long long nbb = p.CP > 0 ? p.NBB : p.NB;
  const long long v[LTC_PLAN_FIELDS] = {
      p.Hp, p.Dp, p.NB, p.KS, p.RC, cols * p.KS,
      p.CP > 0 ? ltc::cluster_fwd_lds(p) : ltc::fwd_lds(p),
      p.CP > 0 ? ltc::cluster_bwd_lds(p) : ltc::chain_launch_lds(p),
      p.NCH, p.NRC, p.CP > 0 ? (long long)p.NCL * p.CP : (B + p.NB - 1) / p.NB,
      p.FUSE ? 1 : 0, p.KSB, p.RCB, colsb * p.KSB, p.CP, p.NCL, p.CPB, nbb,
      p.CP > 0 ? (long long)p.NCLB * p.CPB : (B + p.NB - 1) / p.NB,
      ltc::cmp_fwd(p) ? 1 : 0, ltc::cmp_bwd(p) ? 1 : 0, ltc::prep_sens_fused(p) ? 1 : 0,
      ltc::row_bwd_fused(p) ? 1 : 0, ltc::row128_rec_fused(p) ? 1 : 0, p.LCH, p.LCHB,
      ltc::sens_full_list(p) ? 1 : 0};
  const int m = n < LTC_PLAN_FIELDS ? n : LTC_PLAN_FIELDS;
  for (int i = 0; i < m; ++i) out[i] = v[i];
  return m;
}

int ltc_device_status(int clear) {
  g_err.clear();
  int v = 0;
  const hipError_t e = ltc::device_fault(&v, clear != 0);
  if (e != hipSuccess) return hip_fail("device status read", e);
  if (v != 0)
    return fail(LTC_EHIP,
                "a launch on this device gave up waiting for its partner workgroups (a "
                "cluster, or a fused row backward's companions: the grid was not resident at "
                "once); every output of that call was set to NaN");
  return LTC_OK;
}

long long ltc_set_cluster_spin_ticks(long long ticks) {
  if (ticks < 0) return -1;
  return g_spin.exchange(ticks);
}

int ltc_timing_enable(int on) {
  Timing& tm = timing();
  std::lock_guard<std::mutex> g(tm.mu);
  tm.drain();
  tm.on = on != 0;
  for (int i = 0; i < ltc::K_COUNT; ++i) {
    tm.total_ms[i] = 0.0;
    tm.count[i] = 0;
  }
  return LTC_OK;
}

int ltc_timing_read(int kernel_id, double* total_ms, long long* launches) {
  if (kernel_id < 0 || kernel_id >= ltc::K_COUNT || !total_ms || !launches)
    return fail(LTC_EINVAL, "bad kernel id or NULL output");
  Timing& tm = timing();
  std::lock_guard<std::mutex> g(tm.mu);
  tm.drain();
  *total_ms = tm.total_ms[kernel_id];
  *launches = tm.count[kernel_id];
  return LTC_OK;
}

int ltc_kernel_count(void) { return ltc::K_COUNT; }

const char* ltc_kernel_name(int kernel_id) {
  if (kernel_id < 0 || kernel_id >= ltc::K_COUNT) return "";
  return kNames[kernel_id];
}

}  // extern "C"
