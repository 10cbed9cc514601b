// Attention-side kernels of one decoder layer: RoPE tables, fused per-head
// RMSNorm + RoPE, and GQA attention over segments.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

#include "ovh_common.h"

namespace ovh {

constexpr int kAttnMaxSegs = 32;  // segments per attention launch

struct AttnSeg {
  const float* bias;  // [rows, rows] additive, or nullptr
  int32_t rows;
  int64_t q_off;      // element offset into q and out
  int64_t kv_off;     // element offset into k and v
  // Split-f16 kernel, mask form (launch_attention_split_only with mask_bits):
  // bit t % 32 of word [row * ((rows + 31) / 32) + t / 32] set = key t visible
  // (bias 0), clear = bias -1e30; nullptr = no mask.
  const uint32_t* bits;
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

// Split-f16 attention (three f16 matrix-core products per fp32 product).
// K and V are split once per call into f16 hi/lo planes, tile-major: each
// segment's keys in 32-key blocks (padded with zeros; block index
// kb = vt_off[s] / 32 + key / 32), and per (KV head kvh, block kb) 8 fragments
// of 64 lanes x 8 halves at halves ((kvh * vt_cols/32 + kb) * 8 + f) * 512 +
// lane * 8, each the 16 bytes one lane reads for one matrix-core operand:
//   kh, kl : fragment f = 16-dim chunk, lane = key % 32 + 32 * ((d / 8) % 2),
//            half = d % 8;
//   vh, vl : head-dim rows permuted (row 32j + r holds d = 4r + j) and key
//            positions permuted inside 16-key groups (bits 2 and 3 swapped);
//            fragment f = 4 * (position / 16) + j, lane = r + 32 * ((position
//            / 8) % 2), half = position % 8.
// Each plane holds n_kv_heads * 128 * vt_cols halves;
// vt_off[s] = sum over earlier segments of round_up(rows, 32).
struct AttnSplit {
  _Float16* kh;
  _Float16* kl;
  _Float16* vh;
  _Float16* vl;
  int64_t vt_cols;
  int64_t vt_off[kAttnMaxSegs];
  int32_t n_kv_heads;
  uint32_t* overflow;  // set non-zero when a |k| or |v| is beyond the f16 range
  // Optional: the output quantised per 32-column block as s8_nk_quantize does
  // (codes [rows][out_stride], scales [rows][out_stride / 32]) instead of the
  // fp32 `out`; needs q_stride == out_stride and segment q offsets in whole rows.
  int8_t* aq;
  float* asc;
  bool aq_tiled;  // codes tile-major (act_index), as the runner's GEMM reads them
  // Optional: the next launch's weight into the L2s by extra workgroups
  // (l2_prefetch; the runner passes the o_proj weight)
  L2Prefetch pf;
};
// Splits K and V of the segments into the planes, then attends.
hipError_t launch_attention_split(const AttnArgs& args, const AttnSplit& sp, int max_rows,
                                  hipStream_t st);
// Attention alone, over planes already written (launch_qk_norm_rope_split); the
// segments' masks from AttnSeg::bits when mask_bits, else from AttnSeg::bias.
hipError_t launch_attention_split_only(const AttnArgs& args, const AttnSplit& sp, int max_rows,
                                       bool mask_bits, hipStream_t st);
// launch_qk_norm_rope (D = 128) that also writes the planes of the roped k rows
// of args' segments (args.kv_stride = n_kv_heads * 128) and of their V, in one
// launch.
hipError_t launch_qk_norm_rope_split(float* q, float* k, const float* qw, const float* kw,
                                     int64_t rows, int n_heads, int n_kv_heads,
                                     const float* cos_tab, const float* sin_tab, float eps,
                                     const AttnArgs& args, const AttnSplit& sp, int max_rows,
                                     hipStream_t st);

// From how many long-form workgroups (segments x KV heads x 128-row query
// tiles) the split attention takes its long-sequence kernel; process-wide.
int64_t attention_long_min_tasks();
void set_attention_long_min_tasks(int64_t tasks);
}  // namespace ovh
