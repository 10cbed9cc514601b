// Throughput ceiling of the exact int8 epilogue on one SIMD: per "block", T
// V_MFMA_I32_32X32X32_I8 tiles, each followed by its 16 x (v_cvt_f32_i32, v_fma_f32)
// epilogue, with double-buffered accumulators and operands that change every
// block (so nothing is folded away); also MFMA alone and MFMA + fma without the
// conversion.  Operands live in registers: this is the bound no memory
// hierarchy can raise.
#include <hip/hip_runtime.h>
#include <cstdio>
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int T, bool EPI, bool CVT>
__global__ __launch_bounds__(256) void k(int iters, const float* sc_in, float* out) {
  i32x4 a = {(int)threadIdx.x, 1, 2, 3};
  i32x4 b[T];
  for (int t = 0; t < T; ++t) b[t] = (i32x4){3, t, 1, (int)threadIdx.x};
  const i32x16 z = {0};
  f32x16 f[T];
  for (int t = 0; t < T; ++t) for (int e = 0; e < 16; ++e) f[t][e] = 0.f;
  i32x16 acc[2][T];
  float s = sc_in[threadIdx.x & 31];
  for (int t = 0; t < T; ++t) acc[0][t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b[t], z, 0, 0, 0);
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      a[0] += 1;
#pragma unroll
      for (int t = 0; t < T; ++t) acc[h ^ 1][t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b[t], z, 0, 0, 0);
      if (EPI) {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            f[t][e] = CVT ? fmaf((float)acc[h][t][e], s, f[t][e]) : fmaf(__int_as_float(acc[h][t][e]), s, f[t][e]);
      } else {
#pragma unroll
        for (int t = 0; t < T; ++t) a[1] ^= acc[h][t][0];
      }
      s += 1.0f;
    }
  }
  float r = a[1];
  for (int t = 0; t < T; ++t) for (int e = 0; e < 16; ++e) r += f[t][e];
  out[blockIdx.x * blockDim.x + threadIdx.x] = r;
}

template <int T, bool EPI, bool CVT>
void run(const char* name, int cus, float* sc, float* out) {
  hipEvent_t e0, e1; (void)hipEventCreate(&e0); (void)hipEventCreate(&e1);
  for (int wps : {1, 2, 4}) {
    const int blocks = cus * wps, iters = 2048;
    hipLaunchKernelGGL((k<T, EPI, CVT>), dim3(blocks), dim3(256), 0, 0, 8, sc, out);
    (void)hipDeviceSynchronize();
    (void)hipEventRecord(e0);
    hipLaunchKernelGGL((k<T, EPI, CVT>), dim3(blocks), dim3(256), 0, 0, iters, sc, out);
    (void)hipEventRecord(e1); (void)hipEventSynchronize(e1);
    float ms; (void)hipEventElapsedTime(&ms, e0, e1);
    const double ops = 2.0 * 32768 * T * 2.0 * iters * blocks * 4;
    printf("%-28s T=%d waves/SIMD=%d : %7.1f TOPS  (%.1f clk per tile-block @2.4GHz)\n", name, T, wps,
           ops / ms / 1e9, (ms * 1e-3 * 2.4e9) / (2.0 * iters * T) / wps);
  }
}

int main() {
  hipDeviceProp_t p; (void)hipGetDeviceProperties(&p, 0);
  const int cus = p.multiProcessorCount;
  float *sc, *out; (void)hipMalloc(&sc, 4096); (void)hipMalloc(&out, sizeof(float) * 256 * cus * 4);
  (void)hipMemset(sc, 0, 4096);
  run<1, false, true>("mfma only", cus, sc, out);
  run<2, false, true>("mfma only", cus, sc, out);
  run<1, true, true>("mfma + cvt + fma", cus, sc, out);
  run<2, true, true>("mfma + cvt + fma", cus, sc, out);
  run<4, true, true>("mfma + cvt + fma", cus, sc, out);
  run<2, true, false>("mfma + fma (no cvt)", cus, sc, out);
  run<4, true, false>("mfma + fma (no cvt)", cus, sc, out);
  return 0;
}
