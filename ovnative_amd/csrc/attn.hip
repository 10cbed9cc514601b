// Attention side of one decoder layer for gfx950: RoPE tables, fused per-head
// RMSNorm + RoPE, and bidirectional GQA attention with an additive bias.
#include "attn.h"
#include "ovh_common.h"

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
  const float* w = h < n_heads ? qw : kw;
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
  if (!own) return;
  const float c = cos_tab[r * half + lane], sn = sin_tab[r * half + lane];
  const float na = __fmul_rn(__fmul_rn(a, scale), w[lane]);
  const float nb = __fmul_rn(__fmul_rn(b, scale), w[lane + half]);
  v[lane] = fmaf(na, c, -__fmul_rn(nb, sn));
  v[lane + half] = fmaf(na, sn, __fmul_rn(nb, c));
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

}  // namespace ovh
