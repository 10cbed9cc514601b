// LDS read-pattern probe: the lane -> address maps of the GEMM's fragment and
// scale reads and of the attention's Q reads, each next to a linear read of the
// same width, one kernel per pattern (2048 workgroups of 4 wavefronts, every
// wavefront reading its own 2 KiB window of a 16 KiB buffer).  Profile it with
//   rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS SQ_ACTIVE_INST_LDS SQ_WAVES -- ./probe_lds
// to count bank-conflict cycles per pattern.  Not part of the library.
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>

typedef int v4i __attribute__((ext_vector_type(4)));

template <int PAT>
__global__ __launch_bounds__(256) void probe(int iters, int* out) {
  __shared__ __attribute__((aligned(16))) int8_t s[16384];
  for (int i = threadIdx.x; i < 16384 / 4; i += 256)
    reinterpret_cast<uint32_t*>(s)[i] = (uint32_t)i * 2654435761u;
  __syncthreads();
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  int off;
  if (PAT == 0) {  // 16x16 GEMM fragment, 8 bytes per lane
    const int q = l >> 4;
    off = ((q >> 1) * 32 + (l & 15)) * 16 + (q & 1) * 8;
  } else if (PAT == 1) {
    off = 8 * l;  // linear, 8 bytes per lane
  } else if (PAT == 2) {
    off = (l & 15) * 16;  // GEMM activation scales: 16 distinct 16-byte slots, broadcast
  } else if (PAT == 3) {
    off = 16 * l;  // linear, 16 bytes per lane
  } else {
    off = (l & 31) * 272 + 16 * (l >> 5);  // attention Q plane rows (136 halves)
  }
  off += w * 2048;
  // every iteration reads a different 16 KiB-wrapped address, and the values
  // are summed (not xor-ed, which would cancel in pairs), so no read folds away
  int acc = 0;
  for (int it = 0; it < iters; ++it) {
    const int o = (off + it * 4096) & 16383;
    if (PAT == 0 || PAT == 1) {
      const int64_t v = *reinterpret_cast<const int64_t*>(s + o);
      acc += (int)v + (int)(v >> 32) * (it | 1);
    } else {
      const v4i v = *reinterpret_cast<const v4i*>(s + o);
      acc += (v[0] + v[1] + v[2] + v[3]) * (it | 1);
    }
  }
  out[blockIdx.x * 256 + threadIdx.x] = acc;
}

int main() {
  int* out = nullptr;
  if (hipMalloc(&out, 2048 * 256 * sizeof(int)) != hipSuccess) return 1;
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return 1;
  const int iters = 1024, blocks = 2048;
  auto run = [&](auto kernel, const char* name) {
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(256), 0, 0, iters, out);
    if (hipDeviceSynchronize() != hipSuccess) return;
    (void)hipEventRecord(e0);
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(256), 0, 0, iters, out);
    (void)hipEventRecord(e1);
    (void)hipEventSynchronize(e1);
    float ms = 0.f;
    (void)hipEventElapsedTime(&ms, e0, e1);
    printf("%-28s %8.3f ms\n", name, ms);
  };
  run(probe<0>, "gemm16 fragment (b64)");
  run(probe<1>, "linear (b64)");
  run(probe<2>, "gemm scales, broadcast (b128)");
  run(probe<3>, "linear (b128)");
  run(probe<4>, "attention Q rows (b128)");
  return 0;
}
