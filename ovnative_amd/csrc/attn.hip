// Attention side of one decoder layer for gfx950: RoPE tables, fused per-head
// RMSNorm + RoPE, and bidirectional GQA attention with an additive bias.
#include <atomic>
#include <cstdint>
#include <type_traits>

#include "attn.h"
#include "ovh_common.h"
#include "qk_common.h"

namespace ovh {

// ---------------------------------------------------------------------------
// RoPE tables, as cpp/src/backend/cpu/ops_cpu.cpp:958-993 builds them:
// inv_freq = (float)pow(theta, -2i/D) in double, angle = (float)pos * inv_freq
// in float.  cos/sin of the float angle are evaluated in double and rounded
// once, i.e. correctly rounded; libm's cosf/sinf are within one ulp of that.
__global__ __launch_bounds__(256) void rope_table_kernel(int64_t rows, const int64_t* __restrict__ pos,
                                                         int half, int D, double theta,
                                                         float* __restrict__ cos_tab,
                                                         float* __restrict__ sin_tab) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * half) return;
  const int64_t r = i / half;
  const int d = (int)(i - r * half);
  const float inv_freq = (float)pow(theta, -2.0 * d / (double)D);
  const float angle = __fmul_rn((float)pos[r], inv_freq);
  cos_tab[i] = (float)cos((double)angle);
  sin_tab[i] = (float)sin((double)angle);
}

hipError_t launch_rope_tables(int64_t rows, const int64_t* pos, int D, float theta,
                              float* cos_tab, float* sin_tab, hipStream_t st) {
  const int half = D / 2;
  const int64_t n = rows * half;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     rows, pos, half, D, (double)theta, cos_tab, sin_tab);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Per-head RMSNorm then RoPE, cpp/src/backend/cpu/ops_cpu.cpp:266-318
// (norm_rope_head_avx2).  One wavefront per (row, head); lane t < D/2 owns the
// rotation pair (t, t + D/2).  The sum of squares reproduces the reference's
// 8-lane fma accumulator: chain j takes elements j, j+8, ... in order, and the
// 8 chains are added left to right, so the norm scale is the reference's bits.
// Lane t < D/2 of the wavefront returns the normalised, rotated pair (t, t + D/2)
// of the head vector v in (oa, ob); the other lanes return false.
template <int D>
__device__ __forceinline__ bool norm_rope_pair(const float* __restrict__ v,
                                               const float* __restrict__ w,
                                               const float* __restrict__ cos_row,
                                               const float* __restrict__ sin_row, float eps,
                                               int lane, float& oa, float& ob) {
  constexpr int half = D / 2;
  const bool own = lane < half;
  const float a = own ? v[lane] : 0.f;
  const float b = own ? v[lane + half] : 0.f;

  // Chain j = lane % 8 (lanes 8.. compute copies that are not used).
  const int j = lane & 7;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < D / 8; ++i) {
    const int d = j + 8 * i;
    const float x = (8 * i < half) ? __shfl(a, d) : __shfl(b, d - half);
    s = fmaf(x, x, s);
  }
  float sum = __shfl(s, 0);
#pragma unroll
  for (int c = 1; c < 8; ++c) sum = __fadd_rn(sum, __shfl(s, c));
  const float scale = __fdiv_rn(1.f, sqrt_rn(__fadd_rn(__fdiv_rn(sum, (float)D), eps)));
  if (!own) return false;
  const float c = cos_row[lane], sn = sin_row[lane];
  const float na = __fmul_rn(__fmul_rn(a, scale), w[lane]);
  const float nb = __fmul_rn(__fmul_rn(b, scale), w[lane + half]);
  oa = fmaf(na, c, -__fmul_rn(nb, sn));
  ob = fmaf(na, sn, __fmul_rn(nb, c));
  return true;
}

template <int D>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(float* __restrict__ q,
                                                           float* __restrict__ k,
                                                           const float* __restrict__ qw,
                                                           const float* __restrict__ kw,
                                                           int64_t rows, int n_heads,
                                                           int n_kv_heads,
                                                           const float* __restrict__ cos_tab,
                                                           const float* __restrict__ sin_tab,
                                                           float eps) {
  constexpr int half = D / 2;
  const int lane = threadIdx.x & 63;
  const int heads = n_heads + n_kv_heads;
  const int64_t task = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (task >= rows * heads) return;  // whole wavefront leaves together
  const int64_t r = task / heads;
  const int h = (int)(task - r * heads);
  float* v = h < n_heads ? q + (r * n_heads + h) * D : k + (r * n_kv_heads + (h - n_heads)) * D;
  float oa, ob;
  if (!norm_rope_pair<D>(v, h < n_heads ? qw : kw, cos_tab + r * half, sin_tab + r * half, eps,
                         lane, oa, ob))
    return;
  v[lane] = oa;
  v[lane + half] = ob;
}

hipError_t launch_qk_norm_rope(float* q, float* k, const float* qw, const float* kw,
                               int64_t rows, int n_heads, int n_kv_heads, int D,
                               const float* cos_tab, const float* sin_tab, float eps,
                               hipStream_t st) {
  const int64_t tasks = rows * (n_heads + n_kv_heads);
  if (tasks <= 0) return hipSuccess;
  const dim3 grid((unsigned)((tasks + 3) / 4));
  if (D == 128)
    hipLaunchKernelGGL(qk_norm_rope_kernel<128>, grid, dim3(256), 0, st, q, k, qw, kw, rows,
                       n_heads, n_kv_heads, cos_tab, sin_tab, eps);
  else
    hipLaunchKernelGGL(qk_norm_rope_kernel<64>, grid, dim3(256), 0, st, q, k, qw, kw, rows,
                       n_heads, n_kv_heads, cos_tab, sin_tab, eps);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// GQA attention (fp32): out[s] = softmax(q[s]·K^T * scale + bias[s]) · V per
// segment and query head, KV head = head / group.  Semantics of
// cpp/src/backend/cpu/ops_cpu.cpp:907-943 / :586-786: a query row whose largest
// biased score is below -1e29 (fully masked) gets zeros.
//
// Work split: one workgroup per (segment, head, 32 query rows); its 4
// wavefronts take every 4th block of 32 keys and keep a flash-style running
// max / sum / output, merged through LDS at the end.  Products run on the fp32
// matrix core (V_MFMA_F32_32X32X2_F32):
//   * scores are computed transposed, S^T = K · Q^T, so each lane ends up with
//     16 keys of ONE query (lane % 32); the softmax row statistics are then a
//     per-lane reduction plus one exchange with lane ^ 32;
//   * those 16 probabilities are exactly the A operand that P · V needs from
//     this lane (query = lane % 32, key = the same 16 keys), so P never leaves
//     registers;
//   * the head dimension is split so that each lane loads float4s: for scores
//     lane (r, h) holds d = 8c + 4h + e (c < 16, e < 4) of its key/query row;
//     for P · V output column j of block c' is d = 4j + c'.
// Loads of K, V, Q rows past the segment end are clamped to its last row (and
// masked out of the softmax / not stored), so every access stays in bounds.
constexpr int kAttnD = 128;
constexpr int kAttnQ = 32;   // query rows per workgroup
constexpr int kAttnK = 32;   // keys per block
constexpr int kAttnWaves = 4;

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__global__ __launch_bounds__(256, 2) void attention_kernel(AttnArgs args) {
  __shared__ float part[kAttnWaves][kAttnQ][kAttnD];  // per-wave unnormalised outputs
  __shared__ float mstat[kAttnWaves][kAttnQ], lstat[kAttnWaves][kAttnQ];
  __shared__ float alpha_s[kAttnWaves][kAttnQ];

  const AttnSeg seg = args.segs[blockIdx.z];
  const int S = seg.rows;
  const int q0 = blockIdx.x * kAttnQ;
  if (q0 >= S) return;  // uniform for the workgroup
  const int h = blockIdx.y, kvh = h / args.group;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r32 = lane & 31, hf = lane >> 5;

  const float* qb = args.q + seg.q_off + (int64_t)h * kAttnD;
  const float* kb = args.k + seg.kv_off + (int64_t)kvh * kAttnD;
  const float* vb = args.v + seg.kv_off + (int64_t)kvh * kAttnD;
  const float* bias = seg.bias;

  // Q row of this lane (query q0 + r32), d = 8c + 4hf + e.
  f32x4 qv[16];
  {
    const int qr = min(q0 + r32, S - 1);
    const float* src = qb + (int64_t)qr * args.q_stride + 4 * hf;
#pragma unroll
    for (int c = 0; c < 16; ++c) qv[c] = *reinterpret_cast<const f32x4*>(src + 8 * c);
  }
  const int qrow_b = min(q0 + r32, S - 1);  // bias row (clamped)

  f32x16 o[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[c][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  const int nblk = (S + kAttnK - 1) / kAttnK;
  for (int blk = wave; blk < nblk; blk += kAttnWaves) {
    const int t0 = blk * kAttnK;
    // ---- S^T = K Q^T for 32 keys x 32 queries
    f32x16 st;
#pragma unroll
    for (int e = 0; e < 16; ++e) st[e] = 0.f;
    {
      const int kr = min(t0 + r32, S - 1);
      const float* src = kb + (int64_t)kr * args.kv_stride + 4 * hf;
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const f32x4 kv4 = *reinterpret_cast<const f32x4*>(src + 8 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e) st = mfma_f32(kv4[e], qv[c][e], st);
      }
    }
    // ---- scale, bias, mask; key of element e is t0 + 8(e/4) + 4hf + e%4
    float p[16];
    float bmax = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int t = t0 + 8 * (e >> 2) + 4 * hf + (e & 3);
      float x = __fmul_rn(st[e], args.scale);
      if (bias) x = __fadd_rn(x, bias[(int64_t)qrow_b * S + min(t, S - 1)]);
      x = t < S ? x : -INFINITY;
      p[e] = x;
      bmax = fmaxf(bmax, x);
    }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
    const float m_new = fmaxf(m_run, bmax);  // finite: key t0 is always valid
    const float alpha = expf(m_run - m_new);
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      p[e] = expf(p[e] - m_new);
      psum = __fadd_rn(psum, p[e]);
    }
    psum = __fadd_rn(psum, __shfl_xor(psum, 32));
    l_run = fmaf(l_run, alpha, psum);
    m_run = m_new;

    // ---- rescale O rows: row i of o[c][e] is query 8(e/4) + 4hf + e%4, whose
    // alpha lives in lane i; exchange through this wave's LDS slot.
    if (hf == 0) alpha_s[wave][r32] = alpha;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 a4 = *reinterpret_cast<const f32x4*>(&alpha_s[wave][8 * g + 4 * hf]);
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) o[c][4 * g + e] = __fmul_rn(o[c][4 * g + e], a4[e]);
    }
    __builtin_amdgcn_wave_barrier();

    // ---- O += P V: step kk uses key t0 + 8(kk/4) + 4hf + kk%4 (= this lane's p[kk])
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      const int t = min(t0 + 8 * (kk >> 2) + 4 * hf + (kk & 3), S - 1);
      const f32x4 v4 = *reinterpret_cast<const f32x4*>(vb + (int64_t)t * args.kv_stride + 4 * r32);
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = mfma_f32(p[kk], v4[c], o[c]);
    }
  }

  // ---- merge the 4 key splits: raw partial outputs and (max, sum) per query
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int i = 8 * (e >> 2) + 4 * hf + (e & 3);
    f32x4 w4;
#pragma unroll
    for (int c = 0; c < 4; ++c) w4[c] = o[c][e];
    *reinterpret_cast<f32x4*>(&part[wave][i][4 * r32]) = w4;
  }
  if (hf == 0) {
    mstat[wave][r32] = m_run;
    lstat[wave][r32] = l_run;
  }
  __syncthreads();
  const int qi = threadIdx.x >> 3, d0 = (threadIdx.x & 7) * 16;
  if (q0 + qi >= S) return;
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, mstat[w][qi]);
  float* dst = args.out + seg.q_off + (int64_t)(q0 + qi) * args.out_stride + (int64_t)h * kAttnD + d0;
  if (M < -1e29f) {  // fully masked row
#pragma unroll
    for (int j = 0; j < 16; j += 4) *reinterpret_cast<f32x4*>(dst + j) = f32x4{0.f, 0.f, 0.f, 0.f};
    return;
  }
  float f[kAttnWaves], L = 0.f;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) {
    f[w] = mstat[w][qi] == -INFINITY ? 0.f : expf(mstat[w][qi] - M);
    L = fmaf(lstat[w][qi], f[w], L);
  }
  const float inv = __fdiv_rn(1.f, L);
#pragma unroll
  for (int j = 0; j < 16; j += 4) {
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(&part[w][qi][d0 + j]);
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = fmaf(x[c], f[w], acc[c]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = __fmul_rn(acc[c], inv);
    *reinterpret_cast<f32x4*>(dst + j) = acc;
  }
}

hipError_t launch_attention(const AttnArgs& args, int max_rows, hipStream_t st) {
  if (args.n_segs <= 0 || max_rows <= 0) return hipSuccess;
  const dim3 grid((unsigned)((max_rows + kAttnQ - 1) / kAttnQ), (unsigned)args.n_heads,
                  (unsigned)args.n_segs);
  hipLaunchKernelGGL(attention_kernel, grid, dim3(256), 0, st, args);
  return hipGetLastError();
}


// ---------------------------------------------------------------------------
// Split-f16 attention.  fp32 x = hi + lo with hi = f16(x) and lo = f16(x - hi):
// hi*hi + hi*lo + lo*hi carries the product to ~2^-22 relative (lo*lo is
// dropped), and each term is exact in the fp32 accumulator, so three
// V_MFMA_F32_32X32X16_F16 replace eight V_MFMA_F32_32X32X2_F32 per 32x32x16
// product: 5.3x less matrix-core time than the fp32 kernel above, same
// structure otherwise.  Values beyond the f16 range would become inf: the split
// pass reports them through `overflow` (the reference's own GPU path runs its
// activations in fp16 too, cuda_lm.cu:1086-1160).

__device__ __forceinline__ f32x16 mfma_h(h8 a, h8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// ---- f16 hi/lo planes of K and V --------------------------------------------
// Tile-major (see AttnSplit): per (KV head, 32-key block) 8 fragments of 64
// lanes x 8 halves, each the 16 bytes one lane reads for one matrix-core
// operand, so a wavefront's fragment load is 1 KiB of contiguous memory.

// V (and K) of one 32-key x 32-dim tile (key tile `kt` of segment `s`, dims
// 32*dq..+31 of KV head `kvh`).  V goes through LDS: head-dim row 32j + r holds
// d = 4r + j, stored key position m holds key m with bits 2 and 3 swapped, and
// fragment 4*(m/16) + j, lane r + 32*((m/8)%2) of the block holds the 8 keys
// of that lane; keys past the segment are 0.  K: with `write_k` the tile's k
// values, otherwise only zeros for keys past the segment (the real keys come
// from the qk-norm/RoPE wavefronts).  `tile` is 32 x 33 floats of LDS.
// Returns true when a value is beyond f16.
__device__ __forceinline__ bool split_v_tile(const AttnArgs& a, const AttnSplit& sp, int s, int kt,
                                             int kvh, int dq, float (*tile)[33], bool write_k,
                                             bool k_pad = true) {
  const AttnSeg seg = a.segs[s];
  const int t0 = kt * 32;
  const int64_t nkb = sp.vt_cols / 32, kb = sp.vt_off[s] / 32 + kt;
  bool bad = false;
  {
    const int key = threadIdx.x >> 3, c4 = (threadIdx.x & 7) * 4;
    const bool real = t0 + key < seg.rows;
    if (write_k || (k_pad && !real)) {
      f32x4 x = f32x4{0.f, 0.f, 0.f, 0.f};
      if (real)
        x = *reinterpret_cast<const f32x4*>(a.k + seg.kv_off + (int64_t)(t0 + key) * a.kv_stride +
                                            kvh * kAttnD + dq * 32 + c4);
      h4 hh, ll;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bad |= !(fabsf(x[j]) < 65504.f);
        _Float16 hi, lo;
        split16(x[j], hi, lo);
        hh[j] = hi;
        ll[j] = lo;
      }
      const int64_t ki = k_tile_index(kvh, nkb, kb, key, dq * 32 + c4);
      *reinterpret_cast<h4*>(sp.kh + ki) = hh;
      *reinterpret_cast<h4*>(sp.kl + ki) = ll;
    }
  }
  {
    const int key = threadIdx.x >> 3, c4 = (threadIdx.x & 7) * 4;
    f32x4 x = f32x4{0.f, 0.f, 0.f, 0.f};
    if (t0 + key < seg.rows)
      x = *reinterpret_cast<const f32x4*>(a.v + seg.kv_off + (int64_t)(t0 + key) * a.kv_stride +
                                          kvh * kAttnD + dq * 32 + c4);
#pragma unroll
    for (int j = 0; j < 4; ++j) tile[key][c4 + j] = x[j];
  }
  __syncthreads();
  if (threadIdx.x < 128) {
    const int dl = threadIdx.x >> 2, kg = threadIdx.x & 3;
    const int d = dq * 32 + dl;
    h8 h, l;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int m = 8 * kg + i;                                        // stored position
      const int key = (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1);     // swap bits 2 and 3
      const float x = tile[key][dl];
      bad |= !(fabsf(x) < 65504.f);
      _Float16 hi, lo;
      split16(x, hi, lo);
      h[i] = hi;
      l[i] = lo;
    }
    const int64_t vi =
        ((((int64_t)kvh * nkb + kb) * 8 + 4 * (kg >> 1) + (d & 3)) * 64 + (d >> 2) + 32 * (kg & 1)) * 8;
    *reinterpret_cast<h8*>(sp.vh + vi) = h;
    *reinterpret_cast<h8*>(sp.vl + vi) = l;
  }
  return bad;
}

// V tiles of one launch: blockIdx -> (segment, key tile, kv head, dim quarter).
__device__ __forceinline__ bool split_v_job(const AttnArgs& a, const AttnSplit& sp, int64_t job,
                                            int ktiles, float (*tile)[33], bool write_k) {
  const int per_seg = ktiles * sp.n_kv_heads * 4;
  const int s = (int)(job / per_seg);
  int r = (int)(job - (int64_t)s * per_seg);
  const int kt = r / (sp.n_kv_heads * 4);
  r -= kt * sp.n_kv_heads * 4;
  if (kt * 32 >= a.segs[s].rows) return false;  // uniform for the workgroup
  return split_v_tile(a, sp, s, kt, r >> 2, r & 3, tile, write_k);
}

// Standalone split of K and V for one attention call: one workgroup per
// (segment, key tile, KV head, dim quarter).
__global__ __launch_bounds__(256) void split_kv_kernel(AttnArgs a, AttnSplit sp, int ktiles) {
  __shared__ float tile[32][33];
  if (split_v_job(a, sp, (int64_t)blockIdx.x, ktiles, tile, true)) atomicOr(sp.overflow, 1u);
}

// The runner's form of qk-norm + RoPE + plane split, in one launch.  The first
// q_blocks workgroups: q in place, 32 (row, head) vectors per workgroup, 8
// lanes each.  The rest: one workgroup per (segment, 32-key tile, KV head,
// quarter qd): keys 8qd..8qd+7 of the tile normalised and rotated the same way
// (8 lanes per key), staged in LDS and written to the K planes 16 bytes per
// slot (keys past the segment as zeros), and the tile's V dims 32qd..+31.
__global__ __launch_bounds__(256) void qk_norm_rope_split_kernel(
    float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ qw,
    const float* __restrict__ kw, int64_t rows, int n_heads, const float* __restrict__ cos_tab,
    const float* __restrict__ sin_tab, float eps, int64_t q_blocks, int ktiles, AttnArgs a,
    AttnSplit sp) {
  constexpr int D = kAttnD, half = D / 2;
  __shared__ float tile[32][33];
  __shared__ float kt_s[8][D + 4];  // 8 keys of a tile, normalised and rotated
  const int j = threadIdx.x & 7;
  if ((int64_t)blockIdx.x < q_blocks) {
    const int64_t task = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    if (task >= rows * n_heads) return;  // whole 8-lane groups leave together
    const int64_t r = task / n_heads;
    float* v = q + task * D;  // q rows are n_heads * D wide
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = v[j + 8 * i];
    norm_rope_lanes8(x, qw, cos_tab + r * half, sin_tab + r * half, eps, j);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[j + 8 * i] = x[i];
    return;
  }
  // (segment, key tile, KV head, quarter)
  const int64_t job = (int64_t)blockIdx.x - q_blocks;
  const int per_seg = ktiles * sp.n_kv_heads * 4;
  const int s = (int)(job / per_seg);
  int rem = (int)(job - (int64_t)s * per_seg);
  const int ktile = rem / (sp.n_kv_heads * 4);
  rem -= ktile * sp.n_kv_heads * 4;
  const int kvh = rem >> 2, qd = rem & 3;
  const AttnSeg seg = a.segs[s];
  const int t0 = ktile * 32;
  if (t0 >= seg.rows) return;  // uniform for the workgroup
  const int64_t r0 = seg.kv_off / a.kv_stride;  // the segment's first k row
  bool bad = false;
  if (threadIdx.x < 64) {
    const int kq = threadIdx.x >> 3, key = 8 * qd + kq;
    float x[16];
    if (t0 + key < seg.rows) {
      const int64_t r = r0 + t0 + key;
      const float* kr = k + r * a.kv_stride + (int64_t)kvh * D;
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = kr[j + 8 * i];
      norm_rope_lanes8(x, kw, cos_tab + r * half, sin_tab + r * half, eps, j);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) kt_s[kq][j + 8 * i] = x[i];
  }
  __syncthreads();
  if (threadIdx.x < 128) {
    // slots: (key, 8-dim group g) -> fragment g/2, lane key + 32*(g%2)
    const int64_t nkb = sp.vt_cols / 32, kb = sp.vt_off[s] / 32 + ktile;
    {
      const int kq = threadIdx.x & 7, key = 8 * qd + kq, g = threadIdx.x >> 3;
      h8 hh, ll;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xv = kt_s[kq][8 * g + e];
        bad |= !(fabsf(xv) < 65504.f);
        _Float16 hi, lo;
        split16(xv, hi, lo);
        hh[e] = hi;
        ll[e] = lo;
      }
      const int64_t ki = k_tile_index(kvh, nkb, kb, key, 8 * g);
      *reinterpret_cast<h8*>(sp.kh + ki) = hh;
      *reinterpret_cast<h8*>(sp.kl + ki) = ll;
    }
  }
  bad |= split_v_tile(a, sp, s, ktile, kvh, qd, tile, false, false);
  if (bad) atomicOr(sp.overflow, 1u);
}

// Attention over the planes.  Same work split as attention_kernel (one
// workgroup per (segment, head, 32 queries), 4 wavefronts over 32-key blocks,
// merged through LDS); the Q planes of the workgroup sit in LDS, the softmax
// runs in base 2 (scores scaled by log2(e), V_EXP_F32), and each wavefront loads
// the K and V fragments of its next block while it computes the current one.
constexpr int kQPad = kAttnD + 8;  // LDS row of a Q plane, in halves
constexpr int kPartRow = kAttnD + 4;  // LDS row of a merge partial, in floats
// The split forms' lazy softmax reference: a row's exponents are taken
// against a value at most this far (base 2) below its largest score so far.
constexpr float kLazyLog2 = 8.0f;
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kMaskedLog2 = -1e29f * kLog2e;

// The mask word of a segment without a mask: every key visible.
__device__ const uint32_t kAllVisible[1] = {0xffffffffu};

template <bool kBits>
__global__ __launch_bounds__(256, 2) void attention_split_kernel(AttnArgs args, AttnSplit sp,
                                                                 int qtiles, int per_xcd) {
  // The Q planes (2 x 32 x kQPad halves) alias the start of `part`, which is
  // written only after every wavefront has left the key loop.  Rows of `part`
  // are padded by 16 bytes, so that the merge's reads (one query row per lane)
  // spread over the banks.
  __shared__ __attribute__((aligned(16))) float part[kAttnWaves][kAttnQ][kPartRow];
  __shared__ float mstat[kAttnWaves][kAttnQ], lstat[kAttnWaves][kAttnQ];
  __shared__ float alpha_s[kAttnWaves][kAttnQ];
  _Float16* qs_h = reinterpret_cast<_Float16*>(&part[0][0][0]);
  _Float16* qs_l = qs_h + kAttnQ * kQPad;

  // prefetch workgroups (sp.pf, sp.pf.wgs per XCD) follow the 8 * per_xcd
  // attention workgroups
  if ((int)blockIdx.x >= 8 * per_xcd) {
    l2_prefetch(sp.pf, ((int)blockIdx.x - 8 * per_xcd) >> 3, (int)blockIdx.x & 7);
    return;
  }
  // XCD-aware task order: workgroups reach the 8 XCDs round-robin (id % 8);
  // XCD x takes the x-th contiguous range of tasks, and tasks are numbered
  // (segment, KV head, head in group, query tile)-major, so the two heads of a
  // KV group and all their query tiles read K/V planes held in one L2.
  const int task = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
  if (task >= args.n_segs * args.n_heads * qtiles) return;
  const int qt = task % qtiles;
  const int sh = task / qtiles;  // segment * n_heads + head; heads of a KV group adjacent
  const int sidx = sh / args.n_heads;
  const int h = sh - sidx * args.n_heads, kvh = h / args.group;
  const AttnSeg seg = args.segs[sidx];
  const int S = seg.rows;
  const int q0 = qt * kAttnQ;
  if (q0 >= S) return;
  // wave index in a scalar register: the key loop's trip count and block
  // starts are then uniform and its loads unconditional
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int r32 = lane & 31, hf = lane >> 5;

  // ---- Q rows q0..q0+31 of head h (16 values per thread): loaded first, so
  // that the K prefetch below is in flight while they are split into the
  // hi/lo planes in LDS
  const int q_row = threadIdx.x >> 3, q_c0 = (threadIdx.x & 7) * 16;
  f32x4 qx[4];
  {
    const int qr = min(q0 + q_row, S - 1);
    const float* src = args.q + seg.q_off + (int64_t)qr * args.q_stride + (int64_t)h * kAttnD + q_c0;
#pragma unroll
    for (int j = 0; j < 4; ++j) qx[j] = *reinterpret_cast<const f32x4*>(src + 4 * j);
  }

  // Wave-uniform bases of this (KV head, segment)'s tiles and 32-bit per-lane
  // byte offsets (the launcher checks that every offset fits), so the loads
  // take a scalar base; fragment j of key block b is 1 KiB at (8b + j) KiB.
  const int64_t tiles0 = ((int64_t)kvh * (sp.vt_cols / 32) + sp.vt_off[sidx] / 32) * kTileHalves;
  const _Float16* __restrict__ khb = sp.kh + tiles0;
  const _Float16* __restrict__ klb = sp.kl + tiles0;
  const _Float16* __restrict__ vhb = sp.vh + tiles0;
  const _Float16* __restrict__ vlb = sp.vl + tiles0;

  // Mask of this lane's query row: bit words (kBits) or the additive bias row.
  // Without mask words every block reads the one all-visible word, so the
  // word's load is unconditional.
  const int qrow = min(q0 + r32, S - 1);
  // (global address space spelled out: through the select the compiler would
  // otherwise emit a flat load, which it can only wait for with vmcnt(0))
  typedef const __attribute__((address_space(1))) uint32_t gword;
  const bool has_bits = kBits && seg.bits;  // uniform
  const gword* mrow = has_bits ? (const gword*)(seg.bits + (int64_t)qrow * ((S + 31) >> 5))
                               : (const gword*)kAllVisible;
  const int mstep = has_bits ? 1 : 0;
  const float* brow = !kBits && seg.bias ? seg.bias + (int64_t)qrow * S : nullptr;
  const bool bias_vec = brow && (S & 3) == 0 && (reinterpret_cast<uintptr_t>(seg.bias) & 15) == 0;
  const float sl2 = args.scale * kLog2e;
  constexpr float kMaskedBias = -1e30f * kLog2e;  // the mask's bias, in base-2 units

  h8 kh[8], kl[8], vh[8], vl[8];  // K: chunk c; V: 8 * (16-key chunk) + ... index 4c + db
  auto ld = [](const _Float16* base, uint32_t elem) __attribute__((always_inline)) {
    return *reinterpret_cast<const h8*>(reinterpret_cast<const char*>(base) + 2u * elem);
  };
  auto load_k = [&](int t0) {
    const uint32_t off = (uint32_t)(t0 >> 5) * kTileHalves + 8u * (uint32_t)lane;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      kh[c] = ld(khb, off + 512 * c);
      kl[c] = ld(klb, off + 512 * c);
    }
  };
  auto load_v = [&](int t0) {
    const uint32_t off = (uint32_t)(t0 >> 5) * kTileHalves + 8u * (uint32_t)lane;
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // j = 4 * (16-key chunk) + head-dim block
      vh[j] = ld(vhb, off + 512 * j);
      vl[j] = ld(vlb, off + 512 * j);
    }
  };

  f32x16 o[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[c][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  // The mask form prefetches the next block's K and V; the float-bias form has
  // 16 more live values per lane and loads K and V at the start of each block.
  // No load sits under a branch inside the key loop (where the paths join the
  // compiler would wait for every load in flight): the wavefront's last block
  // is peeled off as the one that prefetches nothing.
  constexpr bool kPrefetch = kBits;
  const int nblk = (S + kAttnK - 1) / kAttnK;
  const int nb = wave < nblk ? (nblk - 1 - wave) / kAttnWaves + 1 : 0;  // this wavefront's blocks
  // unconditional (a wavefront without blocks loads one it will not use)
  if (kPrefetch) load_k(min(wave, nblk - 1) * kAttnK);
  {
    h8 hh[2], ll[2];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        _Float16 a, b;
        split16(qx[j][e], a, b);
        hh[j >> 1][4 * (j & 1) + e] = a;
        ll[j >> 1][4 * (j & 1) + e] = b;
      }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      *reinterpret_cast<h8*>(qs_h + q_row * kQPad + q_c0 + 8 * j) = hh[j];
      *reinterpret_cast<h8*>(qs_l + q_row * kQPad + q_c0 + 8 * j) = ll[j];
    }
  }
  // V of the first block only once Q has landed (the split above waits for
  // it): the launch-wide burst of first-block loads that Q queues behind is
  // then K alone (attention 14.70 -> 14.52 us per launch at 2 x 300).  The
  // scheduling barrier keeps the compiler from hoisting the loads back.
  __builtin_amdgcn_sched_barrier(0);
  if (kPrefetch) load_v(min(wave, nblk - 1) * kAttnK);
  // Q planes written: this wavefront's LDS stores done, then the barrier.  Not
  // __syncthreads(), whose release fence would also wait for the K/V prefetch
  // (vmcnt(0)); the empty asm keeps the compiler from moving LDS accesses
  // across the barrier.
  wait_vm_lgkm<63>();
  asm volatile("s_barrier" ::: "memory");

  auto key_block = [&](int blk, auto next) __attribute__((always_inline)) {
    constexpr bool kNext = kPrefetch && decltype(next)::value;
    const int t0 = blk * kAttnK;
    const int t_next = t0 + kAttnWaves * kAttnK;
    if (!kPrefetch) {
      load_k(t0);
      load_v(t0);
    }
    // this lane's 16 mask bits: bit 8g + i = key t0 + 8g + 4hf + i
    const uint32_t mword = mrow[blk * mstep] >> (4 * hf);
    // ---- S^T = K Q^T (32 keys x 32 queries), three f16 products per chunk
    f32x16 st;
#pragma unroll
    for (int e = 0; e < 16; ++e) st[e] = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const h8 qh = *reinterpret_cast<const h8*>(qs_h + r32 * kQPad + 16 * c + 8 * hf);
      const h8 ql = *reinterpret_cast<const h8*>(qs_l + r32 * kQPad + 16 * c + 8 * hf);
      st = mfma_h(kl[c], qh, st);
      st = mfma_h(kh[c], ql, st);
      st = mfma_h(kh[c], qh, st);
    }
    // the next block's fragments reuse these registers: keep the loads after
    // the products that read them
    __builtin_amdgcn_sched_barrier(0);
    if (kNext) load_k(t_next);

    // bias of this lane's 16 keys (key of element e: t0 + 8(e/4) + 4hf + e%4),
    // base-2 units
    float bv[16];
    if (kBits) {
      // every key of every lane visible (most blocks): no bias, the same bits
      if (has_bits && !__all((mword & 0x0F0F0F0Fu) == 0x0F0F0F0Fu)) {
#pragma unroll
        for (int e = 0; e < 16; ++e)
          bv[e] = mword & (1u << (8 * (e >> 2) + (e & 3))) ? 0.f : kMaskedBias;
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) bv[e] = 0.f;
      }
    } else if (brow) {
      if (bias_vec) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int tg = t0 + 8 * g + 4 * hf;
          f32x4 b4 = f32x4{0.f, 0.f, 0.f, 0.f};
          if (tg < S) b4 = *reinterpret_cast<const f32x4*>(brow + tg);
#pragma unroll
          for (int e = 0; e < 4; ++e) bv[4 * g + e] = b4[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) bv[e] = brow[min(t0 + 8 * (e >> 2) + 4 * hf + (e & 3), S - 1)];
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) bv[e] = __fmul_rn(bv[e], kLog2e);
    }

    // ---- base-2 softmax statistics
    float p[16];
    float bmax = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e)
      p[e] = (kBits || brow) ? fmaf(st[e], sl2, bv[e]) : __fmul_rn(st[e], sl2);
    // keys past the segment: the partial block, if any, is the last one the
    // wavefront takes (uniform)
    if (!decltype(next)::value && t0 + kAttnK > S) {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (t0 + 8 * (e >> 2) + 4 * hf + (e & 3) >= S) p[e] = -INFINITY;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) bmax = fmaxf(bmax, p[e]);
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
    // The row's reference m_run (the exponents are taken against it) moves
    // only when a score exceeds it by more than kLazyLog2, so p <= 2^kLazyLog2;
    // then the output and the sum are rescaled, in most blocks not at all.
    const bool up = bmax > m_run + kLazyLog2;
    const float m_new = up ? bmax : m_run;
    const float m_ref = m_new == -INFINITY ? 0.f : m_new;  // all keys so far at -inf
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      p[e] = __builtin_amdgcn_exp2f(p[e] - m_ref);
      psum = __fadd_rn(psum, p[e]);
    }
    psum = __fadd_rn(psum, __shfl_xor(psum, 32));
    // a row that keeps its reference gets alpha = 1: l_run + psum, o unchanged
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_ref);
    l_run = fmaf(l_run, alpha, psum);
    if (__any(up)) {  // uniform
      if (hf == 0) alpha_s[wave][r32] = alpha;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 a4 = *reinterpret_cast<const f32x4*>(&alpha_s[wave][8 * g + 4 * hf]);
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e) o[c][4 * g + e] = __fmul_rn(o[c][4 * g + e], a4[e]);
      }
      __builtin_amdgcn_wave_barrier();
    }
    m_run = m_new;

    // ---- O += P V: 16-key chunk c takes this lane's p[8c .. 8c+7]
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      h8 ph, pl;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        _Float16 a, b;
        split16(p[8 * c + j], a, b);
        ph[j] = a;
        pl[j] = b;
      }
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        o[db] = mfma_h(pl, vh[4 * c + db], o[db]);
        o[db] = mfma_h(ph, vl[4 * c + db], o[db]);
        o[db] = mfma_h(ph, vh[4 * c + db], o[db]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (kNext) load_v(t_next);
  };
  for (int i = 0; i + 1 < nb; ++i) key_block(wave + i * kAttnWaves, std::true_type{});
  if (nb > 0) key_block(wave + (nb - 1) * kAttnWaves, std::false_type{});

  __syncthreads();  // every wavefront is done with the Q planes
  // merge the 4 key splits (output column of block db, lane r32: d = 4*r32 + db)
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int i = 8 * (e >> 2) + 4 * hf + (e & 3);
    f32x4 w4;
#pragma unroll
    for (int c = 0; c < 4; ++c) w4[c] = o[c][e];
    *reinterpret_cast<f32x4*>(&part[wave][i][4 * r32]) = w4;
  }
  if (hf == 0) {
    mstat[wave][r32] = m_run;
    lstat[wave][r32] = l_run;
  }
  __syncthreads();
  // One query row per lane, 16 columns each: wavefront w takes the 32-column
  // block w of every row, lanes l and l + 32 its two halves
  static_assert(kAttnWaves * 32 == kAttnD, "one 32-column block per wavefront");
  const int qi = lane & 31, d0 = 32 * wave + 16 * hf;
  const bool valid = q0 + qi < S;  // the pair exchange below needs both lanes
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, mstat[w][qi]);
  float ov[16];
  if (M < kMaskedLog2) {  // fully masked row (largest biased score below -1e29)
#pragma unroll
    for (int j = 0; j < 16; ++j) ov[j] = 0.f;
  } else {
    float f[kAttnWaves], L = 0.f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      f[w] = mstat[w][qi] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mstat[w][qi] - M);
      L = fmaf(lstat[w][qi], f[w], L);
    }
    const float inv = __fdiv_rn(1.f, L);
#pragma unroll
    for (int j = 0; j < 16; j += 4) {
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(&part[w][qi][d0 + j]);
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] = fmaf(x[c], f[w], acc[c]);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) ov[j + c] = __fmul_rn(acc[c], inv);
    }
  }
  if (sp.aq) {
    const int64_t row = seg.q_off / args.q_stride + q0 + qi;
    // s8_nk_quantize of this 32-column block: amax over the lane pair, then
    // the same scale and rounding as quantize_kernel (quant_block_lane).
    float a = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) a = fmaxf(a, fabsf(ov[j]));
    const float amax = fmaxf(a, __shfl_xor(a, 32));
    const float qinv = amax > 0.f ? __fdiv_rn(127.0f, amax) : 0.f;
    i32x4 codes;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint32_t packed = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        packed |= (uint32_t)(uint8_t)(int8_t)quant_q(ov[4 * c + e], qinv) << (8 * e);
      codes[c] = (int)packed;
    }
    if (!valid) return;
    const int64_t col = (int64_t)h * kAttnD + d0;
    if (sp.aq_tiled) {  // the row's 16 codes are two 8-byte pieces of the tile
      *reinterpret_cast<int2*>(sp.aq + act_index(row, col, args.out_stride, true)) =
          int2{codes[0], codes[1]};
      *reinterpret_cast<int2*>(sp.aq + act_index(row, col + 8, args.out_stride, true)) =
          int2{codes[2], codes[3]};
    } else {
      *reinterpret_cast<i32x4*>(sp.aq + row * args.out_stride + col) = codes;
    }
    if (hf == 0) sp.asc[row * (args.out_stride / 32) + col / 32] = __fdiv_rn(amax, 127.0f);
    return;
  }
  if (!valid) return;
  float* dst = args.out + seg.q_off + (int64_t)(q0 + qi) * args.out_stride + (int64_t)h * kAttnD + d0;
#pragma unroll
  for (int j = 0; j < 16; j += 4)
    *reinterpret_cast<f32x4*>(dst + j) = f32x4{ov[j], ov[j + 1], ov[j + 2], ov[j + 3]};
}


// ---------------------------------------------------------------------------
// Long-sequence form of the split-f16 attention.  In the form above every
// workgroup (32 query rows) streams its KV head's whole planes through its
// wavefronts' registers; at seq 1024 that is ~1 MB per workgroup per head and
// the L2 -> CU traffic, not the matrix core, sets the time.  Here a workgroup
// covers 128 query-head rows: its 4 wavefronts are the G heads of one KV group
// times 128/G queries (wave w: head kvh*G + w%G, rows 32*(w/G)..+31 of the
// tile), each 32-key block of K and V is moved into LDS once (DMA, double
// buffered) and read by all four, and every wavefront walks all keys itself, so
// there is no merge.  Per element the arithmetic is the form above's (three f16
// products, base-2 online softmax, same masks, same quantised epilogue).
// LDS planes of a block: the block's 8 fragments of each global plane as they
// are stored (1 KiB each, lane-linear), so the DMA copies them verbatim and a
// wavefront's fragment read is 64 contiguous 16-byte slots (conflict-free).
constexpr int kLdsPlane = 32 * kAttnD;  // halves per plane per block
// The long-sequence form pays once its workgroups (segments x KV heads x
// 128-row tiles) fill the chip about one and a half times over; below that
// the form above, with 4x the workgroups, is faster.  MI355X, 16/8 heads,
// us (short form / this form, tasks of this form): 2 x 300 15.1 / 22.9 (80),
// 8 x 300 39.5 / 41.7 (320), 4 x 768 87.6 / 80.4 (384), 2 x 1024 76.3 / 73.3
// (256), 8 x 512 86.0 / 65.7 (512), 16 x 300 73.7 / 63.0 (640).
constexpr int kLdsMinTasks = 384;
// The threshold in use (ovh_set_attention_long_min_tasks), process-wide.
std::atomic<int64_t> g_long_min_tasks{kLdsMinTasks};

template <bool kBits>
__global__ __launch_bounds__(256, 2) void attention_split_lds_kernel(AttnArgs args, AttnSplit sp,
                                                                     int qtiles, int per_xcd) {
  // Double buffer as two arrays (kh, kl, vh, vl planes each): with the block
  // loop unrolled by parity, a block's reads and the next block's DMA touch
  // different arrays, which the compiler can tell apart (one array would make
  // it wait for the DMA before every read).
  __shared__ __attribute__((aligned(16))) _Float16 kv0[4][kLdsPlane];
  __shared__ __attribute__((aligned(16))) _Float16 kv1[4][kLdsPlane];
  __shared__ float xs[kAttnWaves][kAttnQ];                               // per-wave row exchange
  __shared__ float ms[kAttnWaves][kAttnQ];
  const int G = args.group;  // 4 % G == 0 (host)
  // wave index in a scalar register: `live` and the block loop are uniform
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int r32 = lane & 31, hf = lane >> 5;
  const int n_kv = args.n_heads / G;
  const int task = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
  if (task >= args.n_segs * n_kv * qtiles) return;
  const int qt = task % qtiles;
  const int sk = task / qtiles;  // segment * n_kv + kv head
  const int sidx = sk / n_kv;
  const int kvh = sk - sidx * n_kv;
  const AttnSeg seg = args.segs[sidx];
  const int S = seg.rows;
  const int QT = kAttnWaves * kAttnQ / G;  // queries per workgroup
  if (qt * QT >= S) return;               // uniform for the workgroup
  const int h = kvh * G + wave % G;
  const int q0 = qt * QT + kAttnQ * (wave / G);
  const bool live = q0 < S;  // uniform for the wavefront; dead ones still move data

  // ---- Q fragments in registers: chunk c = d 16c + 8hf .. +7 of row q0 + r32
  h8 qh[8], ql[8];
  {
    const int qr = min(q0 + r32, S - 1);
    const float* src = args.q + seg.q_off + (int64_t)qr * args.q_stride + (int64_t)h * kAttnD + 8 * hf;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(src + 16 * c);
      const f32x4 x1 = *reinterpret_cast<const f32x4*>(src + 16 * c + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        _Float16 a, b;
        split16(x0[j], a, b);
        qh[c][j] = a;
        ql[c][j] = b;
        split16(x1[j], a, b);
        qh[c][4 + j] = a;
        ql[c][4 + j] = b;
      }
    }
  }

  // ---- DMA sources.  Wave w moves plane w of each block (8 x 1 KiB):
  // K planes (w < 2): slot s = 64 i + lane -> key s/16, chunk (s%16) ^ (key&15);
  // V planes: slot s -> row s/4, chunk (s%4) ^ ((row>>2)&3).
  const _Float16* plane = (wave == 0 ? sp.kh : wave == 1 ? sp.kl : wave == 2 ? sp.vh : sp.vl) +
                          ((int64_t)kvh * (sp.vt_cols / 32) + sp.vt_off[sidx] / 32) * kTileHalves;
  auto issue = [&](int blk, auto odd) __attribute__((always_inline)) {
    const _Float16* pb = plane + (int64_t)blk * kTileHalves;  // the block's tiles
    _Float16* dst = decltype(odd)::value ? &kv1[wave][0] : &kv0[wave][0];
#pragma unroll
    for (int i = 0; i < 8; ++i)  // fragment i of this wavefront's plane
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(pb + 512 * i + 8 * lane),
                                       (lds_void_t*)(dst + 512 * i), 16, 0, 0);
  };

  // mask words as in attention_split_kernel: the all-visible word when the
  // segment has none, so the load is unconditional
  typedef const __attribute__((address_space(1))) uint32_t gword;
  const int qrow = min(q0 + r32, S - 1);
  const bool has_bits = kBits && seg.bits;  // uniform
  const gword* mrow = has_bits ? (const gword*)(seg.bits + (int64_t)qrow * ((S + 31) >> 5))
                               : (const gword*)kAllVisible;
  const int mstep = has_bits ? 1 : 0;
  const float* brow = !kBits && seg.bias ? seg.bias + (int64_t)qrow * S : nullptr;
  const float sl2 = args.scale * kLog2e;
  constexpr float kMaskedBias = -1e30f * kLog2e;

  f32x16 o[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[c][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const int lslot = 8 * lane;  // this lane's 16 bytes in an LDS fragment

  // The last block is peeled off as the one that issues no DMA, so no load
  // sits under a branch inside the loop.
  const int nblk = (S + kAttnK - 1) / kAttnK;
  issue(0, std::false_type{});
  // block blk (odd: blk % 2 == 1, its planes in kv1), then the next block's DMA
  auto key_block = [&](int blk, auto next, auto odd) __attribute__((always_inline)) {
    constexpr bool kOdd = decltype(odd)::value;
    // this lane's mask word, loaded ahead of the DMA issue so that waiting for
    // it leaves the next block's DMA in flight
    const uint32_t mword_raw = kBits ? (uint32_t)mrow[blk * mstep] : 0u;
    wait_vm_lgkm<0>();              // this wavefront's DMA for block blk (and Q) landed
    __builtin_amdgcn_s_barrier();   // ... and the others'; block blk-1's slot is free
    if constexpr (decltype(next)::value) issue(blk + 1, std::integral_constant<bool, !kOdd>{});
    if (!live) return;
    const int t0 = blk * kAttnK;
    const _Float16* kb = kOdd ? &kv1[0][0] : &kv0[0][0];
    // ---- S^T = K Q^T
    f32x16 st;
#pragma unroll
    for (int e = 0; e < 16; ++e) st[e] = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int off = 512 * c + lslot;
      const h8 khf = *reinterpret_cast<const h8*>(kb + off);
      const h8 klf = *reinterpret_cast<const h8*>(kb + kLdsPlane + off);
      st = mfma_h(klf, qh[c], st);
      st = mfma_h(khf, ql[c], st);
      st = mfma_h(khf, qh[c], st);
    }
    // ---- bias of this lane's 16 keys (key of element e: t0 + 8(e/4) + 4hf + e%4)
    float bv[16];
    if (kBits) {
      const uint32_t mword = mword_raw >> (4 * hf);
      // every key of every lane visible (most blocks): no bias, the same bits
      if (has_bits && !__all((mword & 0x0F0F0F0Fu) == 0x0F0F0F0Fu)) {
#pragma unroll
        for (int e = 0; e < 16; ++e)
          bv[e] = mword & (1u << (8 * (e >> 2) + (e & 3))) ? 0.f : kMaskedBias;
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) bv[e] = 0.f;
      }
    } else if (brow) {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        bv[e] = __fmul_rn(brow[min(t0 + 8 * (e >> 2) + 4 * hf + (e & 3), S - 1)], kLog2e);
    }
    float p[16];
    float bmax = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e)
      p[e] = (kBits || brow) ? fmaf(st[e], sl2, bv[e]) : __fmul_rn(st[e], sl2);
    // keys past the segment: the partial block, if any, is the last one the
    // wavefront takes (uniform)
    if (!decltype(next)::value && t0 + kAttnK > S) {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (t0 + 8 * (e >> 2) + 4 * hf + (e & 3) >= S) p[e] = -INFINITY;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) bmax = fmaxf(bmax, p[e]);
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
    // lazy reference, as in attention_split_kernel
    const bool up = bmax > m_run + kLazyLog2;
    const float m_new = up ? bmax : m_run;
    const float m_ref = m_new == -INFINITY ? 0.f : m_new;
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      p[e] = __builtin_amdgcn_exp2f(p[e] - m_ref);
      psum = __fadd_rn(psum, p[e]);
    }
    psum = __fadd_rn(psum, __shfl_xor(psum, 32));
    // a row that keeps its reference gets alpha = 1: l_run + psum, o unchanged
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_ref);
    l_run = fmaf(l_run, alpha, psum);
    if (__any(up)) {  // uniform
      if (hf == 0) xs[wave][r32] = alpha;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 a4 = *reinterpret_cast<const f32x4*>(&xs[wave][8 * g + 4 * hf]);
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e) o[c][4 * g + e] = __fmul_rn(o[c][4 * g + e], a4[e]);
      }
      __builtin_amdgcn_wave_barrier();
    }
    m_run = m_new;

    // ---- O += P V
    const _Float16* vb = kb + 2 * kLdsPlane;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      h8 ph, pl;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        _Float16 a, b;
        split16(p[8 * c + j], a, b);
        ph[j] = a;
        pl[j] = b;
      }
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int off = 512 * (4 * c + db) + lslot;
        const h8 vhf = *reinterpret_cast<const h8*>(vb + off);
        const h8 vlf = *reinterpret_cast<const h8*>(vb + kLdsPlane + off);
        o[db] = mfma_h(pl, vhf, o[db]);
        o[db] = mfma_h(ph, vlf, o[db]);
        o[db] = mfma_h(ph, vhf, o[db]);
      }
    }
  };
  int blk = 0;
  for (; blk + 2 < nblk; blk += 2) {
    key_block(blk, std::true_type{}, std::false_type{});
    __builtin_amdgcn_sched_barrier(0);  // one block's registers at a time
    key_block(blk + 1, std::true_type{}, std::true_type{});
  }
  if (blk + 1 < nblk) {  // two blocks left (uniform)
    key_block(blk, std::true_type{}, std::false_type{});
    __builtin_amdgcn_sched_barrier(0);
    key_block(blk + 1, std::false_type{}, std::true_type{});
  } else {
    key_block(blk, std::false_type{}, std::false_type{});
  }
  if (!live) return;

  // ---- epilogue: row i of o[c][e] is query q0 + 8(e/4) + 4hf + e%4, column
  // d = 4*r32 + c; its l and m live in lane i (exchanged through LDS)
  if (hf == 0) {
    xs[wave][r32] = l_run;
    ms[wave][r32] = m_run;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const f32x4 l4 = *reinterpret_cast<const f32x4*>(&xs[wave][8 * g + 4 * hf]);
    const f32x4 m4 = *reinterpret_cast<const f32x4*>(&ms[wave][8 * g + 4 * hf]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 8 * g + 4 * hf + e;
      const bool valid = q0 + i < S;
      f32x4 v;
      if (m4[e] < kMaskedLog2) {  // fully masked row
        v = f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
        const float inv = __fdiv_rn(1.f, l4[e]);
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = __fmul_rn(o[c][4 * g + e], inv);
      }
      if (sp.aq) {
        // 32-column block = lanes r32 = 8b..8b+7 of this half: amax by xor 1, 2, 4
        float a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        a = fmaxf(a, __shfl_xor(a, 1));
        a = fmaxf(a, __shfl_xor(a, 2));
        a = fmaxf(a, __shfl_xor(a, 4));
        const float qinv = a > 0.f ? __fdiv_rn(127.0f, a) : 0.f;
        uint32_t packed = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          packed |= (uint32_t)(uint8_t)(int8_t)quant_q(v[c], qinv) << (8 * c);
        if (valid) {
          const int64_t row = seg.q_off / args.q_stride + q0 + i;
          const int64_t col = (int64_t)h * kAttnD + 4 * r32;
          *reinterpret_cast<uint32_t*>(sp.aq + act_index(row, col, args.out_stride, sp.aq_tiled)) =
              packed;
          if ((r32 & 7) == 0) sp.asc[row * (args.out_stride / 32) + col / 32] = __fdiv_rn(a, 127.0f);
        }
      } else if (valid) {
        float* dst = args.out + seg.q_off + (int64_t)(q0 + i) * args.out_stride +
                     (int64_t)h * kAttnD + 4 * r32;
        *reinterpret_cast<f32x4*>(dst) = v;
      }
    }
  }
}

namespace {
// resident workgroups per CU of the short form: a property of the kernel on
// the architecture
template <bool kBits>
int split_occupancy() {
  static const int occ = [] {
    int o = 0;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, attention_split_kernel<kBits>, 256, 0) ==
                   hipSuccess
               ? o
               : 0;
  }();
  return occ;
}
}  // namespace

hipError_t launch_attention_split(const AttnArgs& args, const AttnSplit& sp, int max_rows,
                                  hipStream_t st) {
  if (args.n_segs <= 0 || max_rows <= 0) return hipSuccess;
  const int ktiles = (max_rows + 31) / 32;
  const int64_t jobs = (int64_t)args.n_segs * ktiles * sp.n_kv_heads * 4;
  hipLaunchKernelGGL(split_kv_kernel, dim3((unsigned)jobs), dim3(256), 0, st, args, sp, ktiles);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_attention_split_only(args, sp, max_rows, false, st);
}

hipError_t launch_attention_split_only(const AttnArgs& args, const AttnSplit& sp, int max_rows,
                                       bool mask_bits, hipStream_t st) {
  if (args.n_segs <= 0 || max_rows <= 0) return hipSuccess;
  if (sp.aq) {  // quantised output: whole rows of one stride, 32-column blocks
    if (args.q_stride != args.out_stride || args.out_stride % 32 != 0 || !sp.asc)
      return hipErrorInvalidValue;
    for (int i = 0; i < args.n_segs; ++i)
      if (args.segs[i].q_off % args.q_stride != 0) return hipErrorInvalidValue;
  }
  // per-lane offsets into one KV head's tiles are 32-bit, in bytes
  // (vt_cols / 32 blocks x 8 KiB)
  if (256 * (uint64_t)sp.vt_cols >= (1ull << 32) || sp.vt_cols % 32 != 0) return hipErrorInvalidValue;
  // The long form holds the G heads of a KV group in its 4 wavefronts, so it
  // needs 4 % G == 0 (then QT >= 32; any other G, up to n_heads, takes the
  // short form below, which has no limit on G).
  const bool lds_ok = args.group > 0 && kAttnWaves % args.group == 0;
  const int QT = lds_ok ? kAttnWaves * kAttnQ / args.group : 1;  // query rows per long-form workgroup
  const int lds_qtiles = (max_rows + QT - 1) / QT;
  const int lds_tasks = lds_ok ? args.n_segs * (args.n_heads / args.group) * lds_qtiles : 0;
  if (lds_ok && lds_tasks >= g_long_min_tasks.load(std::memory_order_relaxed)) {
    // a chip's worth of long-form workgroups: K/V blocks shared through LDS
    // by 128 query-head rows
    const int qtiles = lds_qtiles;
    const int tasks = lds_tasks;
    const int per_xcd = (tasks + 7) / 8;
    const dim3 grid((unsigned)(8 * per_xcd));
    if (mask_bits)
      hipLaunchKernelGGL(attention_split_lds_kernel<true>, grid, dim3(256), 0, st, args, sp, qtiles,
                         per_xcd);
    else
      hipLaunchKernelGGL(attention_split_lds_kernel<false>, grid, dim3(256), 0, st, args, sp,
                         qtiles, per_xcd);
    return hipGetLastError();
  }
  // 1-D grid of 8 * per_xcd workgroups (XCD-aware task order in the kernel),
  // then the prefetch workgroups
  const int qtiles = (max_rows + kAttnQ - 1) / kAttnQ;
  const int tasks = args.n_segs * args.n_heads * qtiles;
  const int per_xcd = (tasks + 7) / 8;
  // the prefetch workgroups only where all of them are resident beside the
  // attention's own (else they would run after them and lengthen the launch)
  auto kernel = mask_bits ? attention_split_kernel<true> : attention_split_kernel<false>;
  AttnSplit s = sp;
  if (!s.pf.p || s.pf.bytes <= 0 || s.pf.wgs <= 0 ||
      8 * (int64_t)(per_xcd + s.pf.wgs) >
          (int64_t)(mask_bits ? split_occupancy<true>() : split_occupancy<false>()) * device_cus())
    s.pf.wgs = 0;
  const dim3 grid((unsigned)(8 * per_xcd + 8 * s.pf.wgs));
  hipLaunchKernelGGL(kernel, grid, dim3(256), 0, st, args, s, qtiles, per_xcd);
  return hipGetLastError();
}

hipError_t launch_qk_norm_rope_split(float* q, float* k, const float* qw, const float* kw,
                                     int64_t rows, int n_heads, int n_kv_heads,
                                     const float* cos_tab, const float* sin_tab, float eps,
                                     const AttnArgs& args, const AttnSplit& sp, int max_rows,
                                     hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  if (args.kv_stride != (int64_t)n_kv_heads * kAttnD || sp.n_kv_heads != n_kv_heads)
    return hipErrorInvalidValue;
  const int64_t q_blocks = (rows * n_heads + 31) / 32;
  const int ktiles = (max_rows + 31) / 32;
  const int64_t kv_jobs = args.n_segs > 0 ? (int64_t)args.n_segs * ktiles * n_kv_heads * 4 : 0;
  hipLaunchKernelGGL(qk_norm_rope_split_kernel, dim3((unsigned)(q_blocks + kv_jobs)), dim3(256), 0,
                     st, q, k, qw, kw, rows, n_heads, cos_tab, sin_tab, eps, q_blocks, ktiles,
                     args, sp);
  return hipGetLastError();
}

int64_t attention_long_min_tasks() { return g_long_min_tasks.load(std::memory_order_relaxed); }
void set_attention_long_min_tasks(int64_t tasks) {
  g_long_min_tasks.store(tasks, std::memory_order_relaxed);
}

}  // namespace ovh
