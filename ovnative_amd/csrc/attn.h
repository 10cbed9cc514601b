// Attention-side kernels of one decoder layer: RoPE tables, fused per-head
// RMSNorm + RoPE, and GQA attention over segments.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace ovh {

constexpr int kAttnMaxSegs = 32;  // segments per attention launch

struct AttnSeg {
  const float* bias;  // [rows, rows] additive, or nullptr
  int32_t rows;
  int64_t q_off;      // element offset into q and out
  int64_t kv_off;     // element offset into k and v
};

struct AttnArgs {
  const float* q;
  const float* k;
  const float* v;
  float* out;
  int64_t q_stride, kv_stride, out_stride;
  int32_t n_heads, group;
  float scale;
  int32_t n_segs;
  AttnSeg segs[kAttnMaxSegs];
};

// cos/sin [rows, D/2] from int64 positions (device).
hipError_t launch_rope_tables(int64_t rows, const int64_t* pos, int D, float theta,
                              float* cos_tab, float* sin_tab, hipStream_t st);
// q [rows, n_heads*D], k [rows, n_kv_heads*D] in place; D = 64 or 128.
hipError_t launch_qk_norm_rope(float* q, float* k, const float* qw, const float* kw,
                               int64_t rows, int n_heads, int n_kv_heads, int D,
                               const float* cos_tab, const float* sin_tab, float eps,
                               hipStream_t st);
// head_dim 128; args.n_segs <= kAttnMaxSegs; max_rows = largest segment.
hipError_t launch_attention(const AttnArgs& args, int max_rows, hipStream_t st);

}  // namespace ovh
