// Shared device helpers for the gfx950 int8-nk kernels.
//
// All kernels are built with -ffp-contract=off: every fused multiply-add below
// is an explicit fmaf(), every other product and sum is rounded on its own, so
// the order of roundings is the one written here and nothing else.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ovh {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBlockK = 32;  // activation quantisation block (k values)

__host__ __device__ inline int64_t kb_of(int64_t K) { return (K + 31) / 32; }

// Byte k of row m of int8 activation codes with Kp bytes per row: row-major
// [M][Kp], or tile-major (the weight tile layout: 1 KiB per 32-row x 32-k
// tile, tiles row-tile-major; inside a tile the 16-row half h = m / 16 % 2 at
// 512 h, then k-group g = k / 8 % 4 at 128 g, then 8 bytes per row), which the
// GEMM moves as 1 KiB contiguous DMA and reads as conflict-free 8-byte
// fragments.  A store of 4 bytes at a k aligned to 4 stays inside one row's
// 8-byte piece; 16 bytes of a row are two pieces 128 bytes apart.
__host__ __device__ inline int64_t act_index(int64_t m, int64_t k, int64_t Kp, bool tiled) {
  if (!tiled) return m * Kp + k;
  return ((m >> 5) * (Kp >> 5) + (k >> 5)) * 1024 + ((m >> 4) & 1) * 512 + ((k >> 3) & 3) * 128 +
         (m & 15) * 8 + (k & 7);
}

// q = clamp(RNE(v*inv), -127, 127), where a product that x86 cvtps_epi32 cannot
// represent (NaN, |x| >= 2^31) becomes INT_MIN and so clamps to -127, as in the
// reference quantiser (cpp/src/backend/cpu/gemm.cpp:412-415).
__device__ __forceinline__ int quant_q(float v, float inv) {
  const float x = __fmul_rn(v, inv);
  if (!(fabsf(x) < 2147483648.0f)) return -127;
  const float r = rintf(x);
  return (int)fminf(fmaxf(r, -127.f), 127.f);
}

// Correctly rounded fp32 square root (what x86 sqrtss returns).  v_sqrt_f32 alone
// is a 1-ulp approximation; the f64 square root is expanded to a correctly
// rounded sequence, and rounding a correctly rounded 53-bit root to 24 bits is
// again correctly rounded (53 >= 2*24 + 2, so the double rounding is innocuous).
__device__ __forceinline__ float sqrt_rn(float x) { return (float)__dsqrt_rn((double)x); }

// Max over the 8 lanes of an aligned 8-lane group (one 32-k block, 4 values per
// lane), by DPP lane moves (no LDS round trip): the pair (quad_perm 1,0,3,2),
// the quad (quad_perm 2,3,0,1), then the other quad of the 8 (row_half_mirror:
// lane i of the 8 reads lane 7 - i).  The max of a set does not depend on the
// order it is taken in.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float group8_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  return v;
}

// sum_{j<8} of lane j's p, added in lane order (every lane gets it); the lane
// values are read as scalars (v_readlane), not through LDS.
__device__ __forceinline__ float sum_lanes8_in_order(float p) {
  float sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), 0));
#pragma unroll
  for (int j = 1; j < 8; ++j)
    sum = __fadd_rn(sum, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), j)));
  return sum;
}

// One 32-k block spread over an 8-lane group, 4 values per lane: computes the
// block's amax, packs this lane's 4 int8 codes (0 for invalid slots, i.e. the
// K-tail padding) into *codes and returns the block scale amax/127.
__device__ __forceinline__ float quant_block_lane(const float v[4], int nvalid, uint32_t* codes) {
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (i < nvalid) a = fmaxf(a, fabsf(v[i]));
  const float amax = group8_max(a);
  const float inv = amax > 0.f ? __fdiv_rn(127.0f, amax) : 0.f;
  uint32_t packed = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = i < nvalid ? quant_q(v[i], inv) : 0;
    packed |= (uint32_t)(uint8_t)(int8_t)q << (8 * i);
  }
  *codes = packed;
  return __fdiv_rn(amax, 127.0f);
}

// RMSNorm + block quantisation of one row of 256*P columns (P <= 4) by one
// wavefront (lane = the lane index), as rmsnorm_quantize_f32 computes it
// (cpp/src/backend/cpu/gemm.cpp:638-707; the same order as the general
// rmsnorm_quantize_kernel): lane l owns
// k = 256p + 4l..+3, which is also the 4-value slot of quantisation block
// 8p + l/8, so the row never has to be re-read.  For the sum of squares the
// row is staged in LDS (xt: kRmsRowLds<P> floats of this wavefront's own)
// transposed, chain j (elements j, j+8, ...) as one contiguous run, and lanes
// 0..7 stream their chains with ds_read_b128; the 8 chains are added in order.
template <int P>
constexpr int kRmsRowLds = 8 * (32 * P + 4);
// rms_quant_row_wvals takes the row's values and its lane's norm weights
// already loaded (xv[p], wv[p] = elements 256p + 4l..+3).
template <int P>
__device__ __forceinline__ void rms_quant_row_wvals(const f32x4 (&xv)[P], const f32x4 (&wv)[P],
                                                    float eps, int8_t* __restrict__ aq,
                                                    float* __restrict__ asc, int64_t r, bool tiled,
                                                    int lane, float* xt) {
  constexpr int cols = 256 * P, T = cols / 8, TP = T + 4;  // chain length, padded LDS row
  // element 256p + 4l + c -> chain 4(l&1) + c, position 32p + l/2
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int c = 0; c < 4; ++c) xt[(4 * (lane & 1) + c) * TP + 32 * p + (lane >> 1)] = xv[p][c];
  // the writes of the other lanes of this wavefront land before the reads
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float part = 0.f;
  if (lane < 8) {
    float acc = 0.f;
#pragma unroll 8
    for (int t = 0; t < T; t += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(&xt[lane * TP + t]);
      acc = fmaf(v[0], v[0], acc);
      acc = fmaf(v[1], v[1], acc);
      acc = fmaf(v[2], v[2], acc);
      acc = fmaf(v[3], v[3], acc);
    }
    part = acc;
  }
  const float sum = sum_lanes8_in_order(part);
  const float scale =
      __fdiv_rn(1.f, sqrt_rn(__fadd_rn(__fdiv_rn(sum, (float)cols), eps)));
#pragma unroll
  for (int p = 0; p < P; ++p) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __fmul_rn(__fmul_rn(xv[p][i], scale), wv[p][i]);
    uint32_t codes;
    const float s = quant_block_lane(v, 4, &codes);
    *reinterpret_cast<uint32_t*>(aq + act_index(r, 256 * p + 4 * lane, cols, tiled)) = codes;
    if ((lane & 7) == 0) asc[r * (cols / 32) + 8 * p + (lane >> 3)] = s;
  }
}

template <int P>
__device__ __forceinline__ void rms_quant_row_vals(const f32x4 (&xv)[P], const float* __restrict__ w,
                                                   float eps, int8_t* __restrict__ aq,
                                                   float* __restrict__ asc, int64_t r, bool tiled,
                                                   int lane, float* xt) {
  f32x4 wv[P];
#pragma unroll
  for (int p = 0; p < P; ++p) wv[p] = *reinterpret_cast<const f32x4*>(w + 256 * p + 4 * lane);
  rms_quant_row_wvals<P>(xv, wv, eps, aq, asc, r, tiled, lane, xt);
}

template <int P>
__device__ __forceinline__ void rms_quant_row(const float* __restrict__ row,
                                              const float* __restrict__ w, float eps,
                                              int8_t* __restrict__ aq, float* __restrict__ asc,
                                              int64_t r, bool tiled, int lane, float* xt) {
  f32x4 xv[P];
#pragma unroll
  for (int p = 0; p < P; ++p) xv[p] = *reinterpret_cast<const f32x4*>(row + 256 * p + 4 * lane);
  rms_quant_row_vals<P>(xv, w, eps, aq, asc, r, tiled, lane, xt);
}

// silu(g) * u as the reference's exp256 lanes compute it (ops_cpu.cpp:75-92,
// 144-198 as its GCC build compiles them: the range reduction x - n*ln2 and
// the final "1 + p*2^n" are fused).
__device__ __forceinline__ float silu_up_lane(float g, float u) {
  float x = __fsub_rn(0.0f, g);
  x = fminf(x, 88.0f);   // minps(x, 88) yields 88 for NaN, as fminf does
  x = fmaxf(x, -87.0f);
  const float n = rintf(__fmul_rn(x, 1.4426950408889634f));
  const float r = fmaf(-n, 0.6931471805599453f, x);
  float p = 1.0f / 720;
  p = fmaf(p, r, 1.0f / 120);
  p = fmaf(p, r, 1.0f / 24);
  p = fmaf(p, r, 1.0f / 6);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ni = (int)n;
  const float sc = __int_as_float((ni + 127) << 23);
  const float d = fmaf(p, sc, 1.0f);
  return __fmul_rn(__fdiv_rn(g, d), u);
}

// Workgroup id -> (n tile, m tile), XCD-aware.  Workgroups are dispatched to the
// 8 XCDs round-robin (id % 8).  The n tiles are split into 8 contiguous ranges of
// `per` tiles (padded: the grid has 8*per*m_tiles workgroups and those landing on
// a padding tile return at once); XCD x walks its range m-tile by m-tile, so the
// weight rows an XCD reads stay in its own L2.
__device__ __forceinline__ bool tile_of(int id, int n_tiles, int& nt, int& mt) {
  const int per = (n_tiles + 7) >> 3;
  const int xcd = id & 7, slot = id >> 3;
  nt = xcd * per + slot % per;
  mt = slot / per;
  return nt < n_tiles;
}

__host__ __device__ inline int64_t grid_size(int64_t n_tiles, int64_t m_tiles) {
  return 8 * ((n_tiles + 7) / 8) * m_tiles;
}

// An L2 prefetch carried by a launch for the launch after it: `wgs` extra
// workgroups per XCD, appended to the grid, load one dword of every 128-byte
// line of `p` (all of it on every XCD, or with `slice` XCD x its eighth
// [x bytes / 8, (x + 1) bytes / 8)) after `sleep` rounds of s_sleep 127 (~8k
// clocks each, so that the launch's own first loads go first).  The lines stay
// in the XCD's L2 across the launch boundary: the next launch's first reads of
// its weight then hit there instead of HBM.  Nothing is written.
struct L2Prefetch {
  const int8_t* p = nullptr;
  int64_t bytes = 0;
  int wgs = 0;
  int sleep = 0;
  int slice = 0;
};

// Compute units of the current device (0 if the query fails).
inline int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  return cus;
}

// The body of prefetch workgroup j of XCD xcd (blockDim.x threads).
__device__ __forceinline__ void l2_prefetch(const L2Prefetch& pf, int j, int xcd) {
  for (int i = 0; i < pf.sleep; ++i) __builtin_amdgcn_s_sleep(127);
  const int64_t lo = pf.slice ? pf.bytes * xcd / 8 : 0;
  const int64_t hi = pf.slice ? pf.bytes * (xcd + 1) / 8 : pf.bytes;
  const int64_t per = (hi - lo + pf.wgs - 1) / pf.wgs;
  const int64_t b0 = lo + j * per, b1 = b0 + per < hi ? b0 + per : hi;
  const int64_t stride = (int64_t)blockDim.x * 128;
  uint32_t acc = 0;
#pragma unroll 8
  for (int64_t off = b0 + (int64_t)threadIdx.x * 128; off + 4 <= b1; off += stride)
    acc ^= *reinterpret_cast<const uint32_t*>(pf.p + off);
  asm volatile("" ::"v"(acc));  // the loads are kept (and waited for) without a store
}

// s_waitcnt vmcnt(N) lgkmcnt(0) (gfx9 encoding; expcnt left alone): this
// wavefront's DMA ops older than the last N have landed in LDS and its own LDS
// reads have returned.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

// LDS destination of global_load_lds (address space 3).
typedef __attribute__((address_space(3))) void lds_void_t;

}  // namespace ovh
