/*
 * ovoracle.c — CPU restatement of OVNative's int8-nk quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker and the CPU
 * baseline for the HIP implementation in ovnative_amd/.  Nothing in the
 * product links, loads or calls it; only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg do.
 *
 * Every function restates one piece of the reference's arithmetic, in the
 * reference's operation order, so that its outputs are the reference's bits.
 * References are relative to the AFun9/ovnative tree:
 *
 *   ovo_quantize_weight_rows   tools/convert_weights.py:130-135  (quantize_int8)
 *   ovo_quantize_u8            cpp/src/backend/cpu/gemm.cpp:379-430 (quantize_a_u8),
 *                              entry point :709-720 (s8_nk_quantize)
 *   ovo_rmsnorm_f32            cpp/src/backend/cpu/ops_cpu.cpp:38-62 (rmsnorm_avx2)
 *   ovo_rmsnorm_quantize_u8    cpp/src/backend/cpu/gemm.cpp:638-707 (rmsnorm_quantize_avx2)
 *   ovo_exp256                 cpp/src/backend/cpu/ops_cpu.cpp:75-92 (exp256_ps, one lane)
 *   ovo_silu_mul_f32           cpp/src/backend/cpu/ops_cpu.cpp:126-136 (silu_mul_avx2)
 *   ovo_silu_mul_quantize_u8   cpp/src/backend/cpu/ops_cpu.cpp:144-198 (silu_mul_quant_avx2)
 *   ovo_block_dots             cpp/src/backend/cpu/gemm.cpp:455-474 (acc - 128*wsum per block)
 *   ovo_linear_q               cpp/src/backend/cpu/gemm.cpp:432-504 (vnni_tile_at epilogue)
 *   ovo_pack / ovo_linear_q_packed   the same arithmetic on AVX-512 VNNI, for timing
 *   ovo_linear_f32             cpp/src/backend/cpu/gemm.cpp:64-110, 283-330, 884-905
 *                              (linear_f32_ld: Mat's fp32 branch, the fp32 audio head)
 *
 * "The reference's arithmetic" means the reference as its own build compiles it:
 * g++ -O3 -std=c++17.  For C++, GCC's default is -ffp-contract=fast, so some
 * mul/add pairs written separately in the source are single fused operations in
 * the reference binary (exp256's range reduction, "1 + exp" in silu, the
 * RMSNorm scalar tail).  Those places are called out below.
 *
 * Numerics that the restatement must keep (and that the HIP kernels keep):
 *   - activation blocks are 32 k wide; scale = amax/127.0f, inv = 127.0f/amax
 *     (0 when amax == 0), q = clamp(RNE(a*inv), -127, 127); a product that
 *     cvtps_epi32 cannot represent (NaN, |x| >= 2^31) becomes INT_MIN and
 *     therefore clamps to -127;
 *   - the reference stores q + 128 as u8 and pads the K tail with byte 0;
 *   - per output: f = fma((float)acc_b, asc[m,b], f) for b = 0..Kb-1, then
 *     o = f * wscale[n]; the residual variant then rounds o + C separately.
 *
 * Build: oracle/Makefile (gcc, ISO C, -ffp-contract=off so that no mul+add
 * pair is fused behind our back: the reference is built with -std=c++17,
 * under which GCC does not contract either).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#if defined(__x86_64__)
#include <immintrin.h>
#endif

#define OVO_API __attribute__((visibility("default")))

/* OVO_PLANT selects a deliberate mistake, for tests/test_oracle.py to prove the
 * golden vectors catch it (never set in a normal build):
 *   1 unfused exp256 range reduction   2 sequential RMSNorm sum
 *   3 unfused block epilogue           4 truncating quantiser
 *   5 wrong zero point (127)           6 weight scale floor skipped
 *   7 attention scale applied after the lane sum
 *   8 RoPE rotation with both products rounded (no fma)
 *   9 softmax through libm expf everywhere (no exp256) */
#ifndef OVO_PLANT
#define OVO_PLANT 0
#endif

static inline int64_t kb_of(int64_t K) { return (K + 31) / 32; }

/* cvtps_epi32 semantics in round-to-nearest-even mode. */
static inline int32_t cvt_rne_i32(float x) {
  if (!(fabsf(x) < 2147483648.0f)) return INT32_MIN;
  if (OVO_PLANT == 4) return (int32_t)x;
  return (int32_t)nearbyintf(x);
}

static inline uint8_t quant_u8(float v, float inv) {
  int32_t z = cvt_rne_i32(v * inv);
  z = z < -127 ? -127 : (z > 127 ? 127 : z);
  return (uint8_t)(z + 128);
}

/* Quantise `kn` (<= 32) values of one block into q[0..31]; returns the block scale. */
static float quant_block_u8(const float* v, int64_t kn, uint8_t* q) {
  float amax = 0.f;
  for (int64_t i = 0; i < kn; ++i) {
    const float a = fabsf(v[i]);
    amax = a > amax ? a : amax;
  }
  const float scale = amax / 127.0f;
  const float inv = amax > 0.f ? 127.0f / amax : 0.f;
  for (int64_t i = 0; i < kn; ++i) q[i] = quant_u8(v[i], inv);
  for (int64_t i = kn; i < 32; ++i) q[i] = 0;
  return scale;
}

OVO_API int64_t ovo_quant_bytes(int64_t M, int64_t K) { return M * kb_of(K) * 32; }
OVO_API int64_t ovo_quant_scales(int64_t M, int64_t K) { return M * kb_of(K); }

/* tools/convert_weights.py:130-135: per output row, scale = max(absmax/127, 1e-12)
 * in float32; q = clip(rint(w/scale), -127, 127). */
OVO_API void ovo_quantize_weight_rows(int64_t N, int64_t K, const float* W, int8_t* q,
                                      float* scale) {
  const float floor_scale = 1e-12f;
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const float* row = W + n * K;
    float amax = 0.f;
    for (int64_t k = 0; k < K; ++k) {
      const float a = fabsf(row[k]);
      amax = a > amax ? a : amax;
    }
    float s = amax / 127.0f;
    if (OVO_PLANT != 6) s = s > floor_scale ? s : floor_scale;
    scale[n] = s;
    for (int64_t k = 0; k < K; ++k) {
      float r = rintf(row[k] / s);
      r = r < -127.f ? -127.f : (r > 127.f ? 127.f : r);
      q[n * K + k] = (int8_t)r;
    }
  }
}

/* cpp/src/backend/cpu/gemm.cpp:379-430 */
OVO_API void ovo_quantize_u8(int64_t M, int64_t K, const float* A, uint8_t* aq, float* asc) {
  if (M <= 0 || K <= 0) return;
  const int64_t Kb = kb_of(K), Kp = Kb * 32;
#pragma omp parallel for schedule(static) if (M >= 32)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t b = 0; b < Kb; ++b) {
      const int64_t k0 = b * 32, kn = (K - k0 < 32) ? (K - k0) : 32;
      asc[m * Kb + b] = quant_block_u8(A + m * K + k0, kn, aq + m * Kp + k0);
    }
  }
}

/* Row scale of cpp/src/backend/cpu/ops_cpu.cpp:38-62: eight fma partial sums
 * (element i feeds partial i%8, in increasing i), summed left to right, then
 * the scalar tail (cols % 8) added one square at a time. */
static float rms_scale(const float* row, int64_t cols, float eps) {
  float lanes[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int64_t i = 0;
  if (OVO_PLANT == 2) {
    float seq = 0.f;
    for (; i < cols; ++i) seq = fmaf(row[i], row[i], seq);
    return 1.f / sqrtf(seq / (float)cols + eps);
  }
  for (; i + 8 <= cols; i += 8)
    for (int j = 0; j < 8; ++j) lanes[j] = fmaf(row[i + j], row[i + j], lanes[j]);
  float sum = lanes[0];
  for (int j = 1; j < 8; ++j) sum = sum + lanes[j];
  /* The scalar tail loop (`sum += row[i]*row[i]`, at most 7 iterations) is what
   * GCC 11 vectorises: with 4 or more elements left, the first 4 squares are
   * rounded (vmulps xmm) and added in order; every remaining element is one
   * fused vfmadd231ss. */
  const int64_t t = cols - i;
  int64_t j = 0;
  if (t >= 4)
    for (; j < 4; ++j) {
      const float sq = row[i + j] * row[i + j];
      sum = sum + sq;
    }
  for (; j < t; ++j) sum = fmaf(row[i + j], row[i + j], sum);
  return 1.f / sqrtf(sum / (float)cols + eps);
}

OVO_API void ovo_rmsnorm_f32(float* dst, const float* src, const float* w, int64_t rows,
                             int64_t cols, float eps) {
#pragma omp parallel for schedule(static) if (rows >= 32)
  for (int64_t r = 0; r < rows; ++r) {
    const float* row = src + r * cols;
    const float s = rms_scale(row, cols, eps);
    for (int64_t i = 0; i < cols; ++i) dst[r * cols + i] = (row[i] * s) * w[i];
  }
}

/* cpp/src/backend/cpu/gemm.cpp:638-707 — byte-identical to rmsnorm then quantise. */
OVO_API void ovo_rmsnorm_quantize_u8(int64_t rows, int64_t cols, const float* x, const float* w,
                                     float eps, uint8_t* aq, float* asc) {
  if (rows <= 0 || cols <= 0) return;
  const int64_t Kb = kb_of(cols), Kp = Kb * 32;
#pragma omp parallel for schedule(static) if (rows >= 32)
  for (int64_t r = 0; r < rows; ++r) {
    const float* row = x + r * cols;
    const float s = rms_scale(row, cols, eps);
    float v[32];
    for (int64_t b = 0; b < Kb; ++b) {
      const int64_t k0 = b * 32, kn = (cols - k0 < 32) ? (cols - k0) : 32;
      for (int64_t i = 0; i < kn; ++i) v[i] = (row[k0 + i] * s) * w[k0 + i];
      asc[r * Kb + b] = quant_block_u8(v, kn, aq + r * Kp + k0);
    }
  }
}

/* One lane of exp256_ps, cpp/src/backend/cpu/ops_cpu.cpp:75-92, as GCC 11 compiles
 * it for the reference (-O3 -std=c++17; for C++ GCC's default is
 * -ffp-contract=fast): clamp to [-87, 88], n = RNE(x*log2e), r = x - n*ln2 as ONE
 * fused op (vfnmadd), degree-6 Horner with fma, then 2^n built in the exponent
 * field.  Returns the polynomial p and the power sc separately because the
 * caller decides how p*sc is rounded: alone it is a plain multiply (softmax),
 * under "1 + exp(..)" GCC fuses it into fma(p, sc, 1) (silu). */
static inline void exp256_parts(float x, float* p_out, float* sc_out) {
  x = x < 88.0f ? x : 88.0f; /* minps returns the second operand on NaN */
  x = x > -87.0f ? x : -87.0f;
  const float n = nearbyintf(x * 1.4426950408889634f);
  const float r = OVO_PLANT == 1 ? x - n * 0.6931471805599453f
                                 : fmaf(-n, 0.6931471805599453f, x);
  float p = 1.0f / 720;
  p = fmaf(p, r, 1.0f / 120);
  p = fmaf(p, r, 1.0f / 24);
  p = fmaf(p, r, 1.0f / 6);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int32_t ni = cvt_rne_i32(n);
  const uint32_t bits = (uint32_t)(ni + 127) << 23;
  memcpy(sc_out, &bits, 4);
  *p_out = p;
}

OVO_API float ovo_exp256(float x) {
  float p, sc;
  exp256_parts(x, &p, &sc);
  return p * sc;
}

/* silu(g)*u on an 8-wide SIMD lane (ops_cpu.cpp:126-142): d = 1 + exp(0 - g)
 * compiles to fma(p, sc, 1); then (g / d) * u.  The scalar tail (ops_cpu.cpp:23)
 * calls libm expf and rounds every step. */
static inline float silu_up_lane(float g, float u) {
  float p, sc;
  exp256_parts(0.0f - g, &p, &sc);
  const float d = fmaf(p, sc, 1.0f);
  return (g / d) * u;
}
static inline float silu_up_tail(float g, float u) { return (g / (1.f + expf(-g))) * u; }

/* cpp/src/backend/cpu/ops_cpu.cpp:126-136: lanes in groups of 8 from the start
 * of the buffer, the n % 8 tail through libm. */
OVO_API void ovo_silu_mul_f32(float* out, const float* g, const float* u, int64_t n) {
  int64_t i = 0;
  for (; i + 8 <= n; i += 8)
    for (int j = 0; j < 8; ++j) out[i + j] = silu_up_lane(g[i + j], u[i + j]);
  for (; i < n; ++i) out[i] = silu_up_tail(g[i], u[i]);
}

/* cpp/src/backend/cpu/ops_cpu.cpp:144-198: per row and 32-k block, groups of 8
 * from the block start use exp256, the block's kn % 8 tail uses libm. */
OVO_API void ovo_silu_mul_quantize_u8(int64_t M, int64_t K, const float* gate, const float* up,
                                      uint8_t* aq, float* asc) {
  if (M <= 0 || K <= 0) return;
  const int64_t Kb = kb_of(K), Kp = Kb * 32;
#pragma omp parallel for schedule(static) if (M >= 32)
  for (int64_t r = 0; r < M; ++r) {
    const float* gr = gate + r * K;
    const float* ur = up + r * K;
    float v[32];
    for (int64_t b = 0; b < Kb; ++b) {
      const int64_t k0 = b * 32, kn = (K - k0 < 32) ? (K - k0) : 32;
      const int64_t kv = (kn / 8) * 8;
      int64_t i = 0;
      for (; i < kv; ++i) v[i] = silu_up_lane(gr[k0 + i], ur[k0 + i]);
      for (; i < kn; ++i) v[i] = silu_up_tail(gr[k0 + i], ur[k0 + i]);
      asc[r * Kb + b] = quant_block_u8(v, kn, aq + r * Kp + k0);
    }
  }
}

/* Per-block int32 products, gemm.cpp:455-474: Σ u8·w over the block minus
 * 128·Σ w, i.e. Σ q·w with q = u8 - 128 (pads are 0 in both operands).
 * out[(m*N + n)*Kb + b]. */
OVO_API void ovo_block_dots(int64_t M, int64_t N, int64_t K, const uint8_t* aq, const int8_t* W,
                            int32_t* out) {
  const int64_t Kb = kb_of(K), Kp = Kb * 32;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      const uint8_t* a = aq + m * Kp;
      const int8_t* w = W + n * K;
      for (int64_t b = 0; b < Kb; ++b) {
        const int64_t k0 = b * 32, kn = (K - k0 < 32) ? (K - k0) : 32;
        int32_t acc = 0, wsum = 0;
        for (int64_t k = 0; k < kn; ++k) {
          acc += (int32_t)a[k0 + k] * (int32_t)w[k0 + k];
          wsum += w[k0 + k];
        }
        out[(m * N + n) * Kb + b] = acc - (OVO_PLANT == 5 ? 127 : 128) * wsum;
      }
    }
  }
}

/* gemm.cpp:432-504, one output at a time: the block epilogue, the column scale,
 * and the separately rounded residual add.  C has leading dimension ldc. */
OVO_API void ovo_linear_q(int64_t M, int64_t N, int64_t K, const uint8_t* aq, const float* asc,
                          const int8_t* W, const float* wscale, float* C, int64_t ldc,
                          int accumulate) {
  if (M <= 0 || N <= 0 || K <= 0) return;
  const int64_t Kb = kb_of(K), Kp = Kb * 32;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      const uint8_t* a = aq + m * Kp;
      const int8_t* w = W + n * K;
      float f = 0.f;
      for (int64_t b = 0; b < Kb; ++b) {
        const int64_t k0 = b * 32, kn = (K - k0 < 32) ? (K - k0) : 32;
        int32_t acc = 0;
        for (int64_t k = 0; k < kn; ++k)
          acc += ((int32_t)a[k0 + k] - (OVO_PLANT == 5 ? 127 : 128)) * (int32_t)w[k0 + k];
        f = OVO_PLANT == 3 ? f + (float)acc * asc[m * Kb + b]
                           : fmaf((float)acc, asc[m * Kb + b], f);
      }
      float o = f * wscale[n];
      if (accumulate) o = o + C[m * ldc + n];
      C[m * ldc + n] = o;
    }
  }
}

/* gemm.cpp:884-905 -> linear_f32_ld_avx2 :283-330: C[i, j] (+)= sum_k A[i, k] W[k, j],
 * W stored [K, N].  Every output is one fma chain over k from +0, in k order:
 * columns in full groups of 8 in micro_f32_8x8 (:64-110), and the N % 8 column
 * tail in the lambda's scalar loop "acc += a[k] * W[k*N+j]" (:297-303), which
 * the reference binary also fuses (it is compiled inside the avx2/fma function
 * with GCC's default -ffp-contract=fast).  accumulate: C_old + acc, rounded
 * once more. */
OVO_API void ovo_linear_f32(int64_t M, int64_t N, int64_t K, const float* A, const float* W,
                            float* C, int64_t ldc, int accumulate) {
  if (M <= 0 || N <= 0 || K <= 0) return;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t i = 0; i < M; ++i) {
    for (int64_t j = 0; j < N; ++j) {
      const float* a = A + i * K;
      float acc = 0.f;
      for (int64_t k = 0; k < K; ++k)
        acc = OVO_PLANT == 10 ? acc + a[k] * W[k * N + j] : fmaf(a[k], W[k * N + j], acc);
      float* c = C + i * ldc + j;
      *c = accumulate ? *c + acc : acc;
    }
  }
}

/* ------------------------------------------------------------------------
 * AVX-512 VNNI form of ovo_linear_q (identical bits; used for CPU timing).
 *
 * Packed weights: panels of 16 output rows; inside a panel one 64-byte group
 * per 4 k holds byte j*4+l = W[n0+j][4g+l] (the operand shape vpdpbusd needs);
 * wsum[b*Npad + n] = Σ_{k in block b} W[n,k] removes the +128 zero point.
 * ---------------------------------------------------------------------- */
static inline int64_t npad16(int64_t N) { return ((N + 15) / 16) * 16; }

OVO_API int64_t ovo_packed_bytes(int64_t N, int64_t K) { return npad16(N) * kb_of(K) * 32; }
OVO_API int64_t ovo_wsum_elems(int64_t N, int64_t K) { return npad16(N) * kb_of(K); }

OVO_API void ovo_pack(int64_t N, int64_t K, const int8_t* W, int8_t* packed, int32_t* wsum) {
  const int64_t Kb = kb_of(K), Np = npad16(N), G = Kb * 8;
  memset(packed, 0, (size_t)(Np * Kb * 32));
  memset(wsum, 0, sizeof(int32_t) * (size_t)(Np * Kb));
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const int64_t p = n / 16, j = n % 16;
    for (int64_t k = 0; k < K; ++k) {
      const int64_t g = k / 4, l = k % 4;
      packed[(p * G + g) * 64 + j * 4 + l] = W[n * K + k];
      wsum[(k / 32) * Np + n] += W[n * K + k];
    }
  }
}

OVO_API int ovo_fast_available(void) {
#if defined(__x86_64__)
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
         __builtin_cpu_supports("avx512vnni");
#else
  return 0;
#endif
}

#if defined(__x86_64__)
#define OVO_AVX512 __attribute__((target("avx512f,avx512bw,avx512vl,avx512vnni")))

/* 4 rows x 32 columns (two panels) per call. */
OVO_AVX512 static void tile_4x32(int64_t m0, int rows, int64_t p0, int npanels, int64_t N,
                                 int64_t Kb, int64_t Kp, int64_t Np, const uint8_t* aq,
                                 const float* asc, const int8_t* packed, const int32_t* wsum,
                                 const float* wscale, float* C, int64_t ldc, int accumulate) {
  const int64_t G = Kb * 8;
  const uint8_t* ar[4];
  for (int r = 0; r < 4; ++r) ar[r] = aq + (m0 + (r < rows ? r : 0)) * Kp;
  __m512 f[4][2];
  for (int r = 0; r < 4; ++r) f[r][0] = f[r][1] = _mm512_setzero_ps();
  const int8_t* w0 = packed + p0 * G * 64;
  const int8_t* w1 = packed + (p0 + (npanels > 1 ? 1 : 0)) * G * 64;
  for (int64_t b = 0; b < Kb; ++b) {
    __m512i c[4][2];
    for (int r = 0; r < 4; ++r) c[r][0] = c[r][1] = _mm512_setzero_si512();
    for (int gg = 0; gg < 8; ++gg) {
      const int64_t g = b * 8 + gg;
      const __m512i b0 = _mm512_loadu_si512((const void*)(w0 + g * 64));
      const __m512i b1 = _mm512_loadu_si512((const void*)(w1 + g * 64));
      for (int r = 0; r < 4; ++r) {
        uint32_t a4;
        memcpy(&a4, ar[r] + 4 * g, 4);
        const __m512i av = _mm512_set1_epi32((int)a4);
        c[r][0] = _mm512_dpbusd_epi32(c[r][0], av, b0);
        c[r][1] = _mm512_dpbusd_epi32(c[r][1], av, b1);
      }
    }
    for (int h = 0; h < 2; ++h) {
      const int64_t n0 = (p0 + h) * 16;
      if (n0 >= Np) continue;
      const __m512i corr =
          _mm512_slli_epi32(_mm512_loadu_si512((const void*)(wsum + b * Np + n0)), 7);
      for (int r = 0; r < rows; ++r) {
        const __m512 v = _mm512_cvtepi32_ps(_mm512_sub_epi32(c[r][h], corr));
        f[r][h] = _mm512_fmadd_ps(v, _mm512_set1_ps(asc[(m0 + r) * Kb + b]), f[r][h]);
      }
    }
  }
  for (int h = 0; h < npanels; ++h) {
    const int64_t n0 = (p0 + h) * 16;
    const int64_t nv = (N - n0 < 16) ? (N - n0) : 16;
    if (nv <= 0) continue;
    const __mmask16 mk = (__mmask16)((1u << nv) - 1u);
    const __m512 ws = _mm512_maskz_loadu_ps(mk, wscale + n0);
    for (int r = 0; r < rows; ++r) {
      float* cp = C + (m0 + r) * ldc + n0;
      __m512 o = _mm512_mul_ps(f[r][h], ws);
      if (accumulate) o = _mm512_add_ps(o, _mm512_maskz_loadu_ps(mk, cp));
      _mm512_mask_storeu_ps(cp, mk, o);
    }
  }
}

OVO_AVX512 static void linear_q_packed_avx512(int64_t M, int64_t N, int64_t K,
                                              const uint8_t* aq, const float* asc,
                                              const int8_t* packed, const int32_t* wsum,
                                              const float* wscale, float* C, int64_t ldc,
                                              int accumulate) {
  const int64_t Kb = kb_of(K), Kp = Kb * 32, Np = npad16(N);
  const int64_t pairs = (Np / 16 + 1) / 2, rblocks = (M + 3) / 4;
#pragma omp parallel for collapse(2) schedule(dynamic, 4)
  for (int64_t pp = 0; pp < pairs; ++pp) {
    for (int64_t rb = 0; rb < rblocks; ++rb) {
      const int64_t p0 = pp * 2;
      const int np = (p0 + 1 < Np / 16) ? 2 : 1;
      const int64_t m0 = rb * 4;
      const int rows = (int)((M - m0 < 4) ? (M - m0) : 4);
      tile_4x32(m0, rows, p0, np, N, Kb, Kp, Np, aq, asc, packed, wsum, wscale, C, ldc,
                accumulate);
    }
  }
}
#endif

/* Returns 0 on success, -1 when the AVX-512 VNNI form is unavailable. */
OVO_API int ovo_linear_q_packed(int64_t M, int64_t N, int64_t K, const uint8_t* aq,
                                const float* asc, const int8_t* packed, const int32_t* wsum,
                                const float* wscale, float* C, int64_t ldc, int accumulate) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
#if defined(__x86_64__)
  if (ovo_fast_available()) {
    linear_q_packed_avx512(M, N, K, aq, asc, packed, wsum, wscale, C, ldc, accumulate);
    return 0;
  }
#endif
  return -1;
}

OVO_API int ovo_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ========================================================================
 * The rest of one decoder layer and the LM around the linears.
 *
 *   ovo_rope_tables     cpp/src/backend/cpu/ops_cpu.cpp:945-993 (qk_norm_rope_f32
 *                       table build: inv_freq in double, angle and cos/sin in float)
 *   ovo_qk_norm_rope    cpp/src/backend/cpu/ops_cpu.cpp:266-299, 301-318
 *                       (norm_rope_head_avx2 / qk_norm_rope_avx2, half % 8 == 0)
 *   ovo_attention_head  cpp/src/backend/cpu/ops_cpu.cpp:586-786
 *                       (attention_head_avx2_rb4; rb2 at :332-578 has the same
 *                       per-row arithmetic), run under FTZ/DAZ like the reference
 *   ovo_attention       cpp/src/model/lm.cpp:259-276 (GQA loop over segments/heads)
 *   ovo_embed           cpp/src/model/lm.cpp:180-198, mat.cpp:57-67 (Emb::gather)
 *   ovo_guided_sample   cpp/src/model/tts.cpp:91-101, 296-326 (parity unpinned against
 *                       a reference binary; pinned by properties)
 * ====================================================================== */

/* FTZ/DAZ as enable_flush_to_zero() sets them (ops_cpu.cpp:1132-1136). */
static inline unsigned ftz_enter(void) {
#if defined(__x86_64__)
  const unsigned old = _mm_getcsr();
  _mm_setcsr(old | 0x8040u);
  return old;
#else
  return 0;
#endif
}
static inline void ftz_leave(unsigned old) {
#if defined(__x86_64__)
  _mm_setcsr(old);
#else
  (void)old;
#endif
}

/* cos/sin tables [rows, D/2]: inv_freq[i] = (float)pow(theta, -2i/D) in double,
 * angle = (float)pos * inv_freq[i] in float, then cosf/sinf. */
OVO_API void ovo_rope_tables(int64_t rows, const int64_t* pos, int D, float theta,
                             float* cos_tab, float* sin_tab) {
  const int half = D / 2;
  float inv_freq[512];
  if (half > 512) return;
  for (int i = 0; i < half; ++i)
    inv_freq[i] = (float)pow((double)theta, -2.0 * i / (double)D);
  for (int64_t r = 0; r < rows; ++r) {
    const float p = (float)pos[r];
    for (int i = 0; i < half; ++i) {
      const float angle = p * inv_freq[i];
      cos_tab[r * half + i] = cosf(angle);
      sin_tab[r * half + i] = sinf(angle);
    }
  }
}

/* The row's sum of squares in the order of an 8-lane fma accumulator: lane j
 * takes elements j, j+8, ...; lanes summed left to right.  D % 8 == 0. */
static inline float lanes8_sumsq(const float* v, int D) {
  float lanes[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int i = 0; i + 8 <= D; i += 8)
    for (int j = 0; j < 8; ++j) lanes[j] = fmaf(v[i + j], v[i + j], lanes[j]);
  float sum = lanes[0];
  for (int j = 1; j < 8; ++j) sum = sum + lanes[j];
  return sum;
}

static void norm_rope_head(float* v, const float* w, const float* c, const float* sn, int D,
                           float eps) {
  const int half = D / 2;
  const float sum = lanes8_sumsq(v, D);
  const float scale = 1.f / sqrtf(sum / (float)D + eps);
  for (int i = 0; i < half; ++i) {
    const float na = (v[i] * scale) * w[i];
    const float nb = (v[i + half] * scale) * w[i + half];
    /* _mm256_fmsub_ps(na, c, nb*sn) and _mm256_fmadd_ps(na, sn, nb*c) */
    if (OVO_PLANT == 8) {
      v[i] = na * c[i] - nb * sn[i];
      v[i + half] = na * sn[i] + nb * c[i];
      continue;
    }
    v[i] = fmaf(na, c[i], -(nb * sn[i]));
    v[i + half] = fmaf(na, sn[i], nb * c[i]);
  }
}

/* q [rows, n_heads*D], k [rows, n_kv_heads*D] in place.  Returns -1 when
 * D/2 % 8 != 0 (the reference then takes its scalar fallback, not restated). */
OVO_API int ovo_qk_norm_rope(float* q, float* k, const float* qw, const float* kw, int64_t rows,
                             int n_heads, int n_kv_heads, int D, const float* cos_tab,
                             const float* sin_tab, float eps) {
  if (D <= 0 || (D / 2) % 8 != 0) return -1;
  const int half = D / 2;
#pragma omp parallel for schedule(static) if (rows >= 16)
  for (int64_t r = 0; r < rows; ++r) {
    const float* c = cos_tab + r * half;
    const float* sn = sin_tab + r * half;
    for (int h = 0; h < n_heads; ++h)
      norm_rope_head(q + (r * n_heads + h) * D, qw, c, sn, D, eps);
    for (int h = 0; h < n_kv_heads; ++h)
      norm_rope_head(k + (r * n_kv_heads + h) * D, kw, c, sn, D, eps);
  }
  return 0;
}

/* hsum256: ((v0+v4) + (v1+v5)) + ((v2+v6) + (v3+v7)). */
static inline float hsum8(const float* v) {
  const float l0 = v[0] + v[4], l1 = v[1] + v[5], l2 = v[2] + v[6], l3 = v[3] + v[7];
  return (l0 + l1) + (l2 + l3);
}

/* One head, S queries attending to S keys (fp32, additive bias [S, S] or NULL).
 * Scores: 8 fma lanes over d, each lane times scale, hsum8, plus bias.  A row
 * whose max is below -1e29 is fully masked and gets zeros.  Softmax: exp256 on
 * the first S/8*8 keys (lane sums, hsum8), libm expf on the tail, one 1/sum
 * multiply.  Output: sequential fma over keys.  D % 8 == 0. */
OVO_API int ovo_attention_head(const float* q, int64_t q_stride, const float* k, const float* v,
                               int64_t kv_stride, const float* bias, int S, int D, float scale,
                               float* out, int64_t out_stride) {
  if (S <= 0) return 0;
  if (D <= 0 || D % 8 != 0) return -1;
  const unsigned csr = ftz_enter();
  float* p = (float*)malloc(sizeof(float) * (size_t)S);
  if (!p) { ftz_leave(csr); return -1; }
  for (int s = 0; s < S; ++s) {
    const float* qr = q + (int64_t)s * q_stride;
    const float* br = bias ? bias + (int64_t)s * S : NULL;
    float mx = -INFINITY;
    for (int t = 0; t < S; ++t) {
      const float* kr = k + (int64_t)t * kv_stride;
      float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int d = 0; d + 8 <= D; d += 8)
        for (int j = 0; j < 8; ++j) a[j] = fmaf(qr[d + j], kr[d + j], a[j]);
      float val;
      if (OVO_PLANT == 7) {
        val = hsum8(a) * scale;
      } else {
        for (int j = 0; j < 8; ++j) a[j] = a[j] * scale;
        val = hsum8(a);
      }
      if (br) val = val + br[t];
      p[t] = val;
      mx = val > mx ? val : mx;
    }
    float* orow = out + (int64_t)s * out_stride;
    if (mx < -1e29f) {
      for (int d = 0; d < D; ++d) orow[d] = 0.f;
      continue;
    }
    float sumv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int i = 0;
    for (; i + 8 <= S; i += 8)
      for (int j = 0; j < 8; ++j) {
        const float e = OVO_PLANT == 9 ? expf(p[i + j] - mx) : ovo_exp256(p[i + j] - mx);
        p[i + j] = e;
        sumv[j] = sumv[j] + e;
      }
    float sum = hsum8(sumv);
    for (; i < S; ++i) {
      const float e = expf(p[i] - mx);
      p[i] = e;
      sum = sum + e;
    }
    const float inv = 1.f / sum;
    for (i = 0; i < S; ++i) p[i] = p[i] * inv;
    for (int d = 0; d < D; ++d) {
      float r = 0.f;
      for (int t = 0; t < S; ++t) r = fmaf(p[t], v[(int64_t)t * kv_stride + d], r);
      orow[d] = r;
    }
  }
  free(p);
  ftz_leave(csr);
  return 0;
}

/* run_layer's attention loop (lm.cpp:259-276): for every segment and query head
 * h, KV head h / (n_heads / n_kv_heads); offsets are element offsets into q/out
 * (q_off) and k/v (kv_off); the output has the same layout as q. */
OVO_API int ovo_attention(int n_segs, const float* const* bias, const int32_t* rows,
                          const int64_t* q_off, const int64_t* kv_off, int n_heads,
                          int n_kv_heads, int D, const float* q, const float* k, const float* v,
                          float scale, float* out) {
  if (n_kv_heads <= 0 || n_heads % n_kv_heads != 0) return -1;
  const int group = n_heads / n_kv_heads;
  const int64_t QD = (int64_t)n_heads * D, KVD = (int64_t)n_kv_heads * D;
  int rc = 0;
#pragma omp parallel for collapse(2) schedule(dynamic, 1) reduction(| : rc)
  for (int s = 0; s < n_segs; ++s)
    for (int h = 0; h < n_heads; ++h) {
      const int kv = h / group;
      rc |= ovo_attention_head(q + q_off[s] + (int64_t)h * D, QD, k + kv_off[s] + (int64_t)kv * D,
                               v + kv_off[s] + (int64_t)kv * D, KVD, bias ? bias[s] : NULL,
                               rows[s], D, scale, out + q_off[s] + (int64_t)h * D, QD);
    }
  return rc ? -1 : 0;
}

/* LM::embed (lm.cpp:180-198): row (b, s) with audio_mask set sums, from 0.f in
 * codebook order, audio_emb[ids[b, c, s] + offsets[c]]; otherwise copies
 * tok_emb[ids[b, 0, s]].  Tables are fp32 (tok_q/aud_q NULL) or int8 with one
 * scale per row, gathered as (float)q * scale (mat.cpp:57-67).  Returns -1 on an
 * id out of range (the reference throws). */
OVO_API int ovo_embed(int batch, int seq, int C, int64_t H, const int64_t* ids,
                      const uint8_t* mask, const float* tok_w, const int8_t* tok_q,
                      const float* tok_s, int64_t tok_rows, const float* aud_w,
                      const int8_t* aud_q, const float* aud_s, int64_t aud_rows,
                      const int64_t* offsets, float* out) {
  for (int b = 0; b < batch; ++b)
    for (int s = 0; s < seq; ++s) {
      const int64_t row = (int64_t)b * seq + s;
      float* o = out + row * H;
      if (mask[row]) {
        for (int64_t h = 0; h < H; ++h) o[h] = 0.f;
        for (int c = 0; c < C; ++c) {
          const int64_t id = ids[((int64_t)b * C + c) * seq + s] + offsets[c];
          if (id < 0 || id >= aud_rows) return -1;
          for (int64_t h = 0; h < H; ++h) {
            const float e = aud_w ? aud_w[id * H + h] : (float)aud_q[id * H + h] * aud_s[id];
            o[h] = o[h] + e;
          }
        }
      } else {
        const int64_t id = ids[(int64_t)b * C * seq + s];
        if (id < 0 || id >= tok_rows) return -1;
        for (int64_t h = 0; h < H; ++h)
          o[h] = tok_w ? tok_w[id * H + h] : (float)tok_q[id * H + h] * tok_s[id];
      }
    }
  return 0;
}

/* ------------------------------------------------------------------------
 * Guided sampling, cpp/src/model/tts.cpp:91-101 (log_softmax) and :296-326,
 * per (codebook c, target frame t) on token-major planes [S, C*V]: cond at
 * its last target_len positions, uncond at its first (the device form,
 * cuda_lm.cu:679-690).  tts.cpp is compiled for baseline x86-64 (no FMA
 * contraction), so every product and sum rounds on its own.
 *
 * cpu_alias = 1 reproduces the host path exactly, including that it calls
 * log_softmax(lp_mix, V, lp_mix) in place: the function's last loop then reads
 * x[i] after its second loop overwrote it with exp(x[i] - m), so the host's
 * guided log-probabilities are exp(mix - m) - lse.  cpu_alias = 0 is the
 * reference's device sampler (cuda_lm.cu:720-756), which an accelerator backend
 * uses: mix - lse.  The argmax agrees except where exp() underflows to ties;
 * the scores differ.  Parity unpinned against a reference binary (tts.cpp needs
 * the whole pipeline to build); pinned by the properties in
 * tests/test_oracle_layer.py.
 * ---------------------------------------------------------------------- */
static void log_softmax_row(const float* x, int n, float* out) {
  float m = -INFINITY;
  for (int i = 0; i < n; ++i) m = x[i] > m ? x[i] : m;
  float sum = 0.f;
  for (int i = 0; i < n; ++i) {
    out[i] = expf(x[i] - m);
    sum = sum + out[i];
  }
  const float lse = logf(sum) + m;
  for (int i = 0; i < n; ++i) out[i] = x[i] - lse;
}

OVO_API int ovo_guided_sample(const float* cond, int cond_seq, const float* uncond, int C, int V,
                              int target_len, float guidance, float layer_penalty, int mask_id,
                              int cpu_alias, int32_t* pred, float* scores) {
  if (target_len <= 0 || target_len > cond_seq || V <= 0) return -1;
  const int64_t CV = (int64_t)C * V;
  float* buf = (float*)malloc(sizeof(float) * 4 * (size_t)V);
  if (!buf) return -1;
  float *lp_c = buf, *lp_u = buf + V, *mix = buf + 2 * V, *tmp = buf + 3 * V;
  for (int idx = 0; idx < C * target_len; ++idx) {
    const int c = idx / target_len, t = idx - c * target_len;
    const float* lc = cond + (int64_t)(cond_seq - target_len + t) * CV + (int64_t)c * V;
    const float* lu = uncond + (int64_t)t * CV + (int64_t)c * V;
    log_softmax_row(lc, V, lp_c);
    log_softmax_row(lu, V, lp_u);
    if (guidance != 0.f) {
      for (int v = 0; v < V; ++v) mix[v] = lp_c[v] + guidance * (lp_c[v] - lp_u[v]);
      if (cpu_alias) {
        log_softmax_row(mix, V, mix);
      } else {
        log_softmax_row(mix, V, tmp);
        memcpy(mix, tmp, sizeof(float) * (size_t)V);
      }
    } else {
      memcpy(mix, lp_c, sizeof(float) * (size_t)V);
    }
    if (mask_id >= 0 && mask_id < V) mix[mask_id] = -INFINITY;
    int best = 0;
    float best_val = -INFINITY;
    for (int v = 0; v < V; ++v)
      if (mix[v] > best_val) {
        best_val = mix[v];
        best = v;
      }
    pred[idx] = best;
    scores[idx] = best_val - (float)c * layer_penalty;
  }
  free(buf);
  return 0;
}
