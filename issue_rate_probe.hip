// Issue-rate probe for bench.py's mix-aware VALU bound: how many lane
// operations per CU per clock gfx950 issues for an FP32 FMA, a v_exp_f32 and a
// v_rcp_f32, and for the forward synapse mix (fma, exp, add, rcp, two fma).
// Each lane runs 8 independent dependency chains and each CU holds 16 waves,
// so latency is hidden and the result is the throughput. The ratio of the FMA
// rate to a transcendental's rate is the cost `r` of that transcendental in
// FMA issue slots.
//
// Built by __graft_entry__.build() (or bench.py --build-probe) into
// ./issue_rate_probe; bench.py runs it before it touches the GPU and prints
// its JSON line into the bench record. Not part of the library.
#include <hip/hip_runtime.h>

#include <cstdio>

namespace {

constexpr int kChains = 8;
constexpr int kIters = 16384;
constexpr int kThreads = 256;

// Block 0's first thread reads the shader clock counter (clock64, which
// counts engine clocks) and the constant 100 MHz wall clock (wall_clock64)
// at its start and end, so the host learns the engine clock the kernel ran at.
template <int OP>
__global__ __launch_bounds__(kThreads) void chains(float* out, float seed, long long* clk) {
  const bool probe = blockIdx.x == 0 && threadIdx.x == 0;
  if (probe) {
    clk[0] = clock64();
    clk[1] = wall_clock64();
  }
  float v[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c) v[c] = seed + 0.03125f * c + 1e-7f * threadIdx.x;
  for (int it = 0; it < kIters; ++it) {
#pragma unroll
    for (int c = 0; c < kChains; ++c) {
      if constexpr (OP == 0) {
        v[c] = fmaf(v[c], 0.9990234f, 0.0009765625f);
      } else if constexpr (OP == 1) {
        v[c] = __builtin_amdgcn_exp2f(-v[c]);
      } else if constexpr (OP == 2) {
        v[c] = __builtin_amdgcn_rcpf(v[c]);  // alternates between x and 1/x
      } else {
        // one forward synapse: gate argument, exp2, 1 + e, rcp, then two
        // accumulations (folded back into the chain to keep it dependent)
        const float a = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(fmaf(v[c], -1.25f, 0.5f)));
        v[c] = fmaf(a, 0.25f, fmaf(a, 0.125f, v[c] * 0.5f));
      }
    }
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < kChains; ++c) s += v[c];
  out[(long long)blockIdx.x * kThreads + threadIdx.x] = s;
  if (probe) {
    clk[2] = clock64();
    clk[3] = wall_clock64();
  }
}

// Engine clock (Hz) of the last launch from block 0's counters, or 0.
double measured_clock(const long long* dclk, int wall_hz) {
  long long h[4] = {0, 0, 0, 0};
  if (hipMemcpy(h, dclk, sizeof(h), hipMemcpyDeviceToHost) != hipSuccess) return 0.0;
  const long long cyc = h[2] - h[0], wall = h[3] - h[1];
  return (cyc > 0 && wall > 0) ? (double)cyc / (double)wall * wall_hz : 0.0;
}

// Best rate over the repetitions, in lane-ops per CU per engine clock: the
// clock each repetition ran at is measured (block 0's counters), so the rate
// holds per clock whatever the clock; *clk_used is that repetition's clock.
template <int OP>
double rate(float* out, long long* dclk, int blocks, int cus, int wall_hz, float seed,
            hipEvent_t a, hipEvent_t b, double* clk_used) {
  double best = 0.0;
  // enough repetitions (about 0.3 s over the four kernels) for the engine
  // clock to settle from idle
  for (int rep = 0; rep < 12; ++rep) {
    if (hipEventRecord(a, nullptr) != hipSuccess) return -1.0;
    hipLaunchKernelGGL(chains<OP>, dim3(blocks), dim3(kThreads), 0, nullptr, out, seed, dclk);
    if (hipGetLastError() != hipSuccess) return -1.0;
    if (hipEventRecord(b, nullptr) != hipSuccess || hipEventSynchronize(b) != hipSuccess) return -1.0;
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, a, b) != hipSuccess || ms <= 0.f) return -1.0;
    const double clk_hz = measured_clock(dclk, wall_hz);
    if (clk_hz <= 0.0) return -1.0;
    const double lane_ops = (double)blocks * kThreads * kIters * kChains;
    const double per_cu_clk = lane_ops / (ms * 1e-3) / cus / clk_hz;
    if (rep > 0 && per_cu_clk > best) {  // rep 0 warms up
      best = per_cu_clk;
      *clk_used = clk_hz;
    }
  }
  return best;
}

}  // namespace

int main() {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, 0) != hipSuccess) {
    std::printf("{\"error\": \"no HIP device\"}\n");
    return 1;
  }
  const int cus = prop.multiProcessorCount;
  int wall_khz = 0;
  if (hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, 0) != hipSuccess ||
      wall_khz <= 0)
    wall_khz = 100000;  // 100 MHz on gfx9
  const int wall_hz = wall_khz * 1000;
  const int blocks = cus * 16 * 64 / kThreads;  // 16 waves per CU
  float* out = nullptr;
  long long* dclk = nullptr;
  if (hipMalloc(&out, sizeof(float) * blocks * kThreads) != hipSuccess) return 1;
  if (hipMalloc(&dclk, 4 * sizeof(long long)) != hipSuccess) return 1;
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return 1;
  double cf = 0, ce = 0, cr = 0, cs = 0;
  const double fma = rate<0>(out, dclk, blocks, cus, wall_hz, 0.5f, a, b, &cf);
  const double ex = rate<1>(out, dclk, blocks, cus, wall_hz, 0.5f, a, b, &ce);
  const double rc = rate<2>(out, dclk, blocks, cus, wall_hz, 1.5f, a, b, &cr);
  const double syn = rate<3>(out, dclk, blocks, cus, wall_hz, 0.5f, a, b, &cs);
  (void)hipFree(out);
  (void)hipFree(dclk);
  if (fma <= 0 || ex <= 0 || rc <= 0 || syn <= 0) {
    std::printf("{\"error\": \"timing failed\"}\n");
    return 1;
  }
  // lane-ops per CU per engine clock (the clock each kernel ran at, measured);
  // r = FMA rate / rate.
  std::printf(
      "{\"arch\": \"%s\", \"cus\": %d, \"clock_mhz\": %.0f, \"clock_mhz_measured\": "
      "{\"fma\": %.0f, \"exp\": %.0f, \"rcp\": %.0f, \"synapse\": %.0f}, "
      "\"waves_per_cu\": 16, "
      "\"chains_per_lane\": %d, \"fma_per_cu_clk\": %.2f, \"exp_per_cu_clk\": %.2f, "
      "\"rcp_per_cu_clk\": %.2f, \"synapse_per_cu_clk\": %.3f, \"r_exp\": %.3f, "
      "\"r_rcp\": %.3f, \"synapse_slots\": %.3f}\n",
      prop.gcnArchName, cus, prop.clockRate / 1e3, cf / 1e6, ce / 1e6, cr / 1e6, cs / 1e6,
      kChains, fma, ex, rc, syn, fma / ex, fma / rc, fma / syn);
  return 0;
}
