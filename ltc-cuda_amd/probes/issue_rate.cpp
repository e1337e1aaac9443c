// Issue-rate probe for the roofline of the LTC kernels: measures lane-operations
// per CU per clock for FP32 FMA, v_exp_f32, v_rcp_f32, and the forward synapse
// mix (fma, exp, add, rcp, three fma-class ops). 16 waves per CU, 8 independent
// dependency chains per lane. Output is read against 64 lane-slots/CU/clk.
// Build: python ltc-cuda_amd/build.py (writes ltc-cuda_amd/probes/issue_rate).
#include <hip/hip_runtime.h>
#include <cstdio>
#define CH 8
template <int OP>
__global__ __launch_bounds__(256) void k(float* out, int iters, float seed) {
  float x[CH];
  #pragma unroll
  for (int c = 0; c < CH; ++c) x[c] = seed + 0.01f * c + 1e-6f * threadIdx.x;
  for (int it = 0; it < iters; ++it) {
    #pragma unroll
    for (int c = 0; c < CH; ++c) {
      if (OP == 0) x[c] = fmaf(x[c], 0.999f, 0.0001f);
      if (OP == 1) x[c] = __builtin_amdgcn_exp2f(-x[c]);
      if (OP == 2) x[c] = __builtin_amdgcn_rcpf(-x[c]);
      if (OP == 3) { // synapse: fma, exp, add, rcp, fma, fma (accumulators folded back)
        float a = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(fmaf(x[c], -1.3f, 0.4f)));
        x[c] = fmaf(a, 0.3f, fmaf(a, 0.2f, x[c] * 0.5f));
      }
    }
  }
  float s = 0; 
  #pragma unroll
  for (int c = 0; c < CH; ++c) s += x[c];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}
int main() {
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, 0) != hipSuccess) return 1;
  printf("CUs %d clock %d kHz\n", p.multiProcessorCount, p.clockRate);
  const int blocks = p.multiProcessorCount * 16, threads = 256, iters = 2048;
  float* out = nullptr;
  if (hipMalloc(&out, sizeof(float) * blocks * threads) != hipSuccess) return 1;
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return 1;
  const char* names[4] = {"fma", "exp", "rcp", "synapse(6 instr)"};
  for (int op = 0; op < 4; ++op) {
    for (int rep = 0; rep < 2; ++rep) {
      (void)hipEventRecord(a);
      if (op == 0) hipLaunchKernelGGL(k<0>, dim3(blocks), dim3(threads), 0, 0, out, iters, 0.5f);
      if (op == 1) hipLaunchKernelGGL(k<1>, dim3(blocks), dim3(threads), 0, 0, out, iters, 0.5f);
      if (op == 2) hipLaunchKernelGGL(k<2>, dim3(blocks), dim3(threads), 0, 0, out, iters, 1.5f);
      if (op == 3) hipLaunchKernelGGL(k<3>, dim3(blocks), dim3(threads), 0, 0, out, iters, 0.5f);
      (void)hipEventRecord(b);
      (void)hipEventSynchronize(b);
      float ms = 0.f;
      (void)hipEventElapsedTime(&ms, a, b);
      double ops = (double)blocks * threads * iters * CH;   // per-lane operations (chains x iters)
      double per_cu_clk = ops / (ms * 1e-3) / p.multiProcessorCount / (p.clockRate * 1e3);
      if (rep) printf("%-18s %8.3f ms  %.2f lane-ops/CU/clk (64 = full rate)\n", names[op], ms, per_cu_clk);
    }
  }
  (void)hipFree(out);
  return 0;
}
