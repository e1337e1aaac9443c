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

template <int OP>
__global__ __launch_bounds__(kThreads) void chains(float* out, float seed) {
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
}

template <int OP>
double rate(float* out, int blocks, int cus, double clk_hz, float seed, hipEvent_t a, hipEvent_t b) {
  double best = 0.0;
  // enough repetitions (about 0.3 s over the four kernels) for bench.py's
  // sysfs clock sampler to see the engine clock while they run
  for (int rep = 0; rep < 12; ++rep) {
    if (hipEventRecord(a, nullptr) != hipSuccess) return -1.0;
    hipLaunchKernelGGL(chains<OP>, dim3(blocks), dim3(kThreads), 0, nullptr, out, seed);
    if (hipGetLastError() != hipSuccess) return -1.0;
    if (hipEventRecord(b, nullptr) != hipSuccess || hipEventSynchronize(b) != hipSuccess) return -1.0;
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, a, b) != hipSuccess || ms <= 0.f) return -1.0;
    const double lane_ops = (double)blocks * kThreads * kIters * kChains;
    const double per_cu_clk = lane_ops / (ms * 1e-3) / cus / clk_hz;
    if (rep > 0 && per_cu_clk > best) best = per_cu_clk;  // rep 0 warms up
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
  const double clk_hz = prop.clockRate * 1e3;
  const int blocks = cus * 16 * 64 / kThreads;  // 16 waves per CU
  float* out = nullptr;
  if (hipMalloc(&out, sizeof(float) * blocks * kThreads) != hipSuccess) return 1;
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return 1;
  const double fma = rate<0>(out, blocks, cus, clk_hz, 0.5f, a, b);
  const double ex = rate<1>(out, blocks, cus, clk_hz, 0.5f, a, b);
  const double rc = rate<2>(out, blocks, cus, clk_hz, 1.5f, a, b);
  const double syn = rate<3>(out, blocks, cus, clk_hz, 0.5f, a, b);
  (void)hipFree(out);
  if (fma <= 0 || ex <= 0 || rc <= 0 || syn <= 0) {
    std::printf("{\"error\": \"timing failed\"}\n");
    return 1;
  }
  // lane-ops per CU per clock at the reported clock; r = FMA rate / rate.
  std::printf(
      "{\"arch\": \"%s\", \"cus\": %d, \"clock_mhz\": %.0f, \"waves_per_cu\": 16, "
      "\"chains_per_lane\": %d, \"fma_per_cu_clk\": %.2f, \"exp_per_cu_clk\": %.2f, "
      "\"rcp_per_cu_clk\": %.2f, \"synapse_per_cu_clk\": %.3f, \"r_exp\": %.3f, "
      "\"r_rcp\": %.3f, \"synapse_slots\": %.3f}\n",
      prop.gcnArchName, cus, clk_hz / 1e6, kChains, fma, ex, rc, syn, fma / ex, fma / rc,
      fma / syn);
  return 0;
}
