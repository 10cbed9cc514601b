// Device-resident LM runner for gfx950: the accelerator plugin of the reference
// LM (cpp/src/backend/cuda/cuda_lm.h:26-57) rebuilt on the int8-nk HIP
// operators.  Host code is plain C++17 around HIP; the numerics of every step
// are those of the reference's CPU int8-nk forward (cpp/src/model/lm.cpp:217-401):
//
//   x = embed(ids)                                         lm.cpp:180-198
//   per layer (lm.cpp:217-322):
//     aq = rmsnorm_quantize(x, input_ln)                   one activation quantisation
//     q|k|v = linear_q_sliced(aq, qkv)                     merged q/k/v weight
//     q, k = qk_norm_rope(q, k)                            per-head RMSNorm + RoPE
//     a = attention(q, k, v, bias)                         GQA, fp32
//     x += linear(a, o)                                    quantise a, residual add
//     aq = rmsnorm_quantize(x, post_ln)
//     g|u = linear_q_sliced(aq, gate_up)
//     x += linear_q(silu_mul_quantize(g, u), down)
//   logits = linear(rmsnorm(x, final_norm), audio_heads)   lm.cpp:383-385
//
// The final norm and the head's activation quantisation are one fused kernel
// (rmsnorm_quantize is byte-identical to rmsnorm followed by s8_nk_quantize).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <numeric>
#include <random>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/ovnative_amd.h"
#include "attn.h"
#include "ovh_common.h"
#include "status.h"
#include "quant.h"
#include "weight.h"

namespace ovh {

// ---------------------------------------------------------------------------
// Embedding (lm.cpp:180-198, Emb::gather mat.cpp:57-67): a row with its audio
// mask set is the sum, from 0 in codebook order, of audio_emb[ids[b,c,s] +
// offsets[c]]; any other row is token_emb[ids[b,0,s]].  Tables are fp32, or
// int8 with one scale per row gathered as float(q) * scale.  Ids were range-
// checked on the host.
struct EmbTable {
  const float* f32;
  const int8_t* i8;
  const float* scale;
  int64_t rows;
};

__device__ __forceinline__ float emb_at(const EmbTable& t, int64_t id, int64_t H, int64_t h) {
  return t.f32 ? t.f32[id * H + h] : __fmul_rn((float)t.i8[id * H + h], t.scale[id]);
}

// Columns h..h+3 of table row id (H % 4 == 0): one 4- or 16-byte load; zeros
// for an id outside the table.
__device__ __forceinline__ f32x4 emb4(const EmbTable& t, int64_t id, int64_t H, int64_t h) {
  if (id < 0 || id >= t.rows) return f32x4{0.f, 0.f, 0.f, 0.f};
  if (t.f32) return *reinterpret_cast<const f32x4*>(t.f32 + id * H + h);
  const uint32_t q = *reinterpret_cast<const uint32_t*>(t.i8 + id * H + h);
  const float sc = t.scale[id];
  f32x4 r;
#pragma unroll
  for (int k = 0; k < 4; ++k) r[k] = __fmul_rn((float)(int8_t)(q >> (8 * k)), sc);
  return r;
}

// The attention masks of the forward's segments as AttnSeg::bits words (bit
// t % 32 of word [row * ((rows + 31) / 32) + t / 32] set = key t visible),
// done by extra workgroups of the embedding launch: four rows per workgroup,
// one wavefront per row, 64 keys per ballot.
struct MaskJob {
  const uint8_t* mask;  // [rows, rows], non-zero = visible
  uint32_t* bits;
  int32_t rows;
  int32_t first;  // first workgroup of this job, counted from the mask part
};
struct MaskJobs {
  int32_t n;
  MaskJob job[kAttnMaxSegs];
};
constexpr int kEmbMaxC = 16;  // codebooks the vector path holds in registers
// The first layer's input norm in the embedding launch (rmsnorm_quantize of
// each embedded row, tile-major codes): w null = off.  Vector path, H = 256 P
// with P <= 4.
struct EmbNorm {
  const float* w;
  float eps;
  int8_t* aq;
  float* asc;
};

__global__ __launch_bounds__(256) void embed_kernel(const int64_t* __restrict__ ids,
                                                    const uint8_t* __restrict__ mask, int seq,
                                                    int C, int64_t H, EmbTable tok, EmbTable aud,
                                                    const int64_t* __restrict__ offsets,
                                                    float* __restrict__ out, int64_t T,
                                                    MaskJobs mj, EmbNorm nrm) {
  const int64_t wg = blockIdx.x;
  if (wg >= T) {
    const int64_t mw = wg - T;
    int j = 0;
    while (j + 1 < mj.n && mw >= mj.job[j + 1].first) ++j;
    const MaskJob jb = mj.job[j];
    const int r = (int)(mw - jb.first) * 4 + (int)(threadIdx.x >> 6);
    if (r >= jb.rows) return;
    const int lane = threadIdx.x & 63, words = (jb.rows + 31) >> 5;
    const uint8_t* src = jb.mask + (int64_t)r * jb.rows;
    for (int t0 = 0; t0 < jb.rows; t0 += 64) {
      const int t = t0 + lane;
      const uint64_t vis = __ballot(t < jb.rows && src[t < jb.rows ? t : 0] != 0);
      const int w = (t0 >> 5) + lane;  // lanes 0 and 1 write the two words
      if (lane < 2 && w < words) jb.bits[(int64_t)r * words + w] = (uint32_t)(vis >> (32 * lane));
    }
    return;
  }
  const int64_t row = wg;
  const int64_t b = row / seq, s = row - b * seq;
  float* o = out + row * H;
  // The host has range-checked every id; an id outside its table (which that
  // check rules out) reads nothing and contributes zeros.
  if ((H & 3) == 0 && C <= kEmbMaxC) {
    if (mask[row]) {
      for (int64_t h = 4 * (int64_t)threadIdx.x; h < H; h += 4 * (int64_t)blockDim.x) {
        // every codebook's values are loaded before the sum, which runs from 0
        // in codebook order as above
        f32x4 e[kEmbMaxC];
#pragma unroll
        for (int c = 0; c < kEmbMaxC; ++c)
          if (c < C) e[c] = emb4(aud, ids[(b * C + c) * seq + s] + offsets[c], H, h);
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < kEmbMaxC; ++c)
          if (c < C)
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[k] = __fadd_rn(acc[k], e[c][k]);
        *reinterpret_cast<f32x4*>(o + h) = acc;
      }
    } else {
      const int64_t id = ids[b * C * seq + s];
      for (int64_t h = 4 * (int64_t)threadIdx.x; h < H; h += 4 * (int64_t)blockDim.x)
        *reinterpret_cast<f32x4*>(o + h) = emb4(tok, id, H, h);
    }
    if (nrm.w) {
      // the workgroup's stores of the row are visible to it after the barrier;
      // one wavefront normalises and quantises it as rmsnorm_quantize_rows
      __shared__ float xt[kRmsRowLds<4>];
      __syncthreads();
      if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        switch (H >> 8) {
          case 1:
            rms_quant_row<1>(o, nrm.w, nrm.eps, nrm.aq, nrm.asc, row, true, lane, xt);
            break;
          case 2:
            rms_quant_row<2>(o, nrm.w, nrm.eps, nrm.aq, nrm.asc, row, true, lane, xt);
            break;
          case 3:
            rms_quant_row<3>(o, nrm.w, nrm.eps, nrm.aq, nrm.asc, row, true, lane, xt);
            break;
          default:
            rms_quant_row<4>(o, nrm.w, nrm.eps, nrm.aq, nrm.asc, row, true, lane, xt);
            break;
        }
      }
    }
    return;
  }
  if (mask[row]) {
    for (int64_t h = threadIdx.x; h < H; h += blockDim.x) {
      float acc = 0.f;
      for (int c = 0; c < C; ++c) {
        const int64_t id = ids[(b * C + c) * seq + s] + offsets[c];
        acc = __fadd_rn(acc, id >= 0 && id < aud.rows ? emb_at(aud, id, H, h) : 0.f);
      }
      o[h] = acc;
    }
  } else {
    const int64_t id = ids[b * C * seq + s];
    const bool ok = id >= 0 && id < tok.rows;
    for (int64_t h = threadIdx.x; h < H; h += blockDim.x) o[h] = ok ? emb_at(tok, id, H, h) : 0.f;
  }
}

// bias = attn ? 0 : -1e30 (lm.cpp:367).
__global__ __launch_bounds__(256) void mask_to_bias_kernel(const uint8_t* __restrict__ m,
                                                           float* __restrict__ bias, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) bias[i] = m[i] ? 0.f : -1e30f;
}

// ---------------------------------------------------------------------------
// Guided sampling for one (codebook c, target frame t) per workgroup, the
// per-step pass of cpp/src/model/tts.cpp:296-326 (device form as in
// cuda_lm.cu:679-758): log_softmax of the conditional and unconditional
// logits, lp = lc + g * (lc - lu) renormalised by a second log_softmax (when
// g != 0), the mask token excluded, argmax (lowest index on ties) and
// score = max - c * layer_penalty.  Both planes are token-major [S, C*V]: cond
// at its last target_len positions, uncond at its first target_len positions.
constexpr int kSampleThreads = 256;
constexpr int kSampleMaxPer = 8;  // vocab <= 2048

struct ArgMax {
  float v;
  int i;
};

__device__ __forceinline__ ArgMax better(ArgMax a, ArgMax b) {
  return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}

__device__ float block_max(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < kSampleThreads / 64; ++i) r = fmaxf(r, red[i]);
  return r;
}

__device__ float block_sum(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = __fadd_rn(v, __shfl_xor(v, o));
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < kSampleThreads / 64; ++i) r = __fadd_rn(r, red[i]);
  return r;
}

__global__ __launch_bounds__(kSampleThreads) void guided_sample_kernel(
    const float* __restrict__ cond, int cond_seq, const float* __restrict__ uncond, int C, int V,
    int target_len, float guidance, float layer_penalty, int mask_id, int32_t* __restrict__ pred,
    float* __restrict__ scores, const uint32_t* __restrict__ flag_src,
    uint32_t* __restrict__ flag_dst) {
  __shared__ float red[kSampleThreads / 64];
  // the runner's overflow flag rides back with the results
  if (blockIdx.x == 0 && threadIdx.x == 0) *flag_dst = *flag_src;
  __shared__ ArgMax ared[kSampleThreads / 64];
  const int idx = blockIdx.x;
  const int c = idx / target_len, t = idx - c * target_len;
  const int64_t CV = (int64_t)C * V;
  const float* lc = cond + (int64_t)(cond_seq - target_len + t) * CV + (int64_t)c * V;
  const float* lu = uncond + (int64_t)t * CV + (int64_t)c * V;

  float xc[kSampleMaxPer], xu[kSampleMaxPer];
  float mc = -INFINITY, mu = -INFINITY;
#pragma unroll
  for (int i = 0; i < kSampleMaxPer; ++i) {
    const int j = threadIdx.x + i * kSampleThreads;
    xc[i] = j < V ? lc[j] : -INFINITY;
    xu[i] = j < V ? lu[j] : -INFINITY;
    mc = fmaxf(mc, xc[i]);
    mu = fmaxf(mu, xu[i]);
  }
  mc = block_max(mc, red);
  mu = block_max(mu, red);
  float sc = 0.f, su = 0.f;
#pragma unroll
  for (int i = 0; i < kSampleMaxPer; ++i) {
    const int j = threadIdx.x + i * kSampleThreads;
    if (j < V) {
      sc = __fadd_rn(sc, expf(__fsub_rn(xc[i], mc)));
      su = __fadd_rn(su, expf(__fsub_rn(xu[i], mu)));
    }
  }
  sc = block_sum(sc, red);
  su = block_sum(su, red);
  const float lse_c = __fadd_rn(logf(sc), mc), lse_u = __fadd_rn(logf(su), mu);

  float lp[kSampleMaxPer];
  float m2 = -INFINITY;
#pragma unroll
  for (int i = 0; i < kSampleMaxPer; ++i) {
    const float pc = __fsub_rn(xc[i], lse_c);
    const float pu = __fsub_rn(xu[i], lse_u);
    // tts.cpp is built for baseline x86-64 (no FMA): product and sum round separately
    lp[i] = guidance != 0.f ? __fadd_rn(pc, __fmul_rn(guidance, __fsub_rn(pc, pu))) : pc;
    const int j = threadIdx.x + i * kSampleThreads;
    if (j < V) m2 = fmaxf(m2, lp[i]);
  }
  float lse2 = 0.f;
  if (guidance != 0.f) {
    m2 = block_max(m2, red);
    float s2 = 0.f;
#pragma unroll
    for (int i = 0; i < kSampleMaxPer; ++i) {
      const int j = threadIdx.x + i * kSampleThreads;
      if (j < V) s2 = __fadd_rn(s2, expf(__fsub_rn(lp[i], m2)));
    }
    s2 = block_sum(s2, red);
    lse2 = __fadd_rn(logf(s2), m2);
  }
  ArgMax best{-INFINITY, 0x7fffffff};
#pragma unroll
  for (int i = 0; i < kSampleMaxPer; ++i) {
    const int j = threadIdx.x + i * kSampleThreads;
    if (j < V && j != mask_id) {
      const float v = guidance != 0.f ? __fsub_rn(lp[i], lse2) : lp[i];
      best = better(best, ArgMax{v, j});
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    ArgMax other{__shfl_xor(best.v, o), __shfl_xor(best.i, o)};
    best = better(best, other);
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) ared[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    ArgMax r = ared[0];
    for (int i = 1; i < kSampleThreads / 64; ++i) r = better(r, ared[i]);
    // argmax over an all -inf row stays at index 0, as the reference's loop does
    pred[idx] = r.i == 0x7fffffff ? 0 : r.i;
    scores[idx] = __fsub_rn(r.v, __fmul_rn((float)c, layer_penalty));
  }
}

}  // namespace ovh

// ===========================================================================
// The runner.
struct OvhLm {
  OvhLmConfig cfg{};
  hipStream_t st = nullptr;
  struct Layer {
    OvhWeight* qkv = nullptr;
    OvhWeight* o = nullptr;
    OvhWeight* gate_up = nullptr;
    OvhWeight* down = nullptr;
    float* ln1 = nullptr;
    float* ln2 = nullptr;
    float* qn = nullptr;
    float* kn = nullptr;
  };
  std::vector<Layer> layers;
  // the audio head: int8 (nk / kn), or fp32 [K, N] as the reference's default
  // int8 checkpoint keeps it (f32 planes, see ovh_linear_f32)
  OvhWeight* head = nullptr;
  float* final_norm = nullptr;
  ovh::EmbTable tok{}, aud{};
  int64_t tok_rows = 0, aud_rows = 0;
  std::vector<int64_t> offsets;
  int64_t* d_offsets = nullptr;
  std::vector<void*> allocs;
  // forward workspace (grow-only)
  char* arena = nullptr;
  size_t arena_cap = 0;
  float* logits = nullptr;
  bool device_sampling = false;
  std::vector<float> host_flat;
  // Pinned host staging: a forward's inputs go up in one copy (h_in, guarded by
  // in_done so a copy in flight is never overwritten); a sample's results come
  // back in one copy of d_out = [overflow flag | pad to 64 B][pred n][scores n].
  char* h_in = nullptr;
  size_t h_in_cap = 0;
  hipEvent_t in_done = nullptr;
  char* d_out = nullptr;
  char* h_out = nullptr;
  int64_t sample_cap = 0;
  // gate/up GEMM with silu(gate)*up quantised in its epilogue (inter % 64 == 0)
  bool silu_fused = false;
  // attention: split-f16 products (default) or fp32; overflow flag of the split
  bool attn_split = true;
  // The forward's launches as one HIP graph, captured per layout (graph_key)
  // and replayed; own_st is the runner's stream when the caller gave none
  // (graphs are not captured on the legacy default stream).
  bool use_graphs = true;
  hipGraphExec_t graph = nullptr;
  std::vector<int64_t> graph_key;
  hipStream_t own_st = nullptr;
  uint32_t* d_overflow = nullptr;
  // o_proj and down with the following RMSNorm + quantise in the same launch
  // (GemmMode kAccumNorm) where the layout allows it; their band counters
  // (zeroed when allocated, then only advanced by the launches)
  bool norm_fused = true;
  // o_proj's weight into the L2s by prefetch workgroups of the attention launch
  bool prefetch = true;
  unsigned long long* d_band = nullptr;
  int64_t band_words = 0;
  // RoPE tables of the last position list (rebuilt only when it changes)
  std::vector<int64_t> tab_pos;
  std::vector<float> tab_host;
  float* d_tab = nullptr;
  size_t tab_cap = 0;
  // In-runner recovery: the fallbacks taken (OVH_LM_RECOVERED_*), a condition
  // to force on the next forward (OVH_LM_FORCE_*), and the host inputs of the
  // last forward that left its logits on the device without synchronising,
  // so that the sample which finds its flags set can run it again.
  int recovered = 0;
  uint32_t last_flags = 0;  // the flag word of the last flagged forward
  int force = 0;
  struct LastForward {
    bool valid = false;
    int batch = 0, seq = 0;
    std::vector<int64_t> ids, pos, seg_row0;
    std::vector<uint8_t> am, masks;  // the segments' masks, concatenated
    std::vector<int> seg_rows;
    std::vector<int64_t> mask_off;   // offset of each segment's mask, -1: none
  } last;
  // Stage timer (ovh_lm_set_profile): events recorded between the stages of
  // the last forward, their labels, and the per-label sums.
  bool profile = false, profile_print = false;
  std::vector<hipEvent_t> prof_ev;
  std::vector<const char*> prof_lab;
  size_t prof_n = 0;
  std::vector<std::pair<const char*, double>> prof_ms;

  ~OvhLm() {
    for (auto& L : layers) {
      ovh_weight_free(L.qkv);
      ovh_weight_free(L.o);
      ovh_weight_free(L.gate_up);
      ovh_weight_free(L.down);
    }
    ovh_weight_free(head);
    for (void* p : allocs) (void)hipFree(p);
    if (arena) (void)hipFree(arena);
    if (in_done) (void)hipEventSynchronize(in_done);
    if (in_done) (void)hipEventDestroy(in_done);
    if (h_in) (void)hipHostFree(h_in);
    if (d_out) (void)hipFree(d_out);
    if (h_out) (void)hipHostFree(h_out);
    if (d_tab) (void)hipFree(d_tab);
    if (d_overflow) (void)hipFree(d_overflow);
    if (d_band) (void)hipFree(d_band);
    if (graph) (void)hipGraphExecDestroy(graph);
    for (hipEvent_t e : prof_ev) (void)hipEventDestroy(e);
    if (own_st) (void)hipStreamDestroy(own_st);
  }
};

namespace {

using ovh::set_error;

// Prefetch workgroups per XCD (l2_prefetch) in the attention launch for the
// o_proj weight, MI355X, LM step at M = 600 (320 attention workgroups, two
// fit a CU): o_proj 12.56 -> 11.76 us and the attention unchanged, with one
// s_sleep round first (without it the loads meet the attention's own first
// loads and it takes 2.4 us longer).
constexpr int kPfAttnWgs = 8;

struct TensorIndex {
  std::unordered_map<std::string, const OvhTensorView*> by_name;
  const OvhTensorView* find(const std::string& n) const {
    auto it = by_name.find(n);
    return it == by_name.end() ? nullptr : it->second;
  }
};

int missing(const std::string& name) {
  return set_error(OV_ERR_INVALID_ARG, "LM weights: tensor not found: '" + name + "'");
}

int upload_bytes(OvhLm& L, const void* src, size_t n, void** out) {
  void* d = nullptr;
  OVH_HIP(hipMalloc(&d, n ? n : 1), "hipMalloc(LM tensor)");
  L.allocs.push_back(d);
  if (n) OVH_HIP(hipMemcpyAsync(d, src, n, hipMemcpyHostToDevice, L.st), "upload LM tensor");
  *out = d;
  return OV_OK;
}

// fp32 vector of `expect` elements (make_norm, mat.cpp:130-139).
int load_norm(OvhLm& L, const TensorIndex& ix, const std::string& name, int64_t expect,
              float** out) {
  const OvhTensorView* t = ix.find(name);
  if (!t) return missing(name);
  int64_t n = 1;
  for (int i = 0; i < t->ndim; ++i) n *= t->dims[i];
  if (t->dtype != 0 || n != expect || !t->data)
    return set_error(OV_ERR_INVALID_ARG, name + ": expected " + std::to_string(expect) +
                                             " fp32 elements");
  void* d = nullptr;
  const int rc = upload_bytes(L, t->data, sizeof(float) * (size_t)n, &d);
  *out = static_cast<float*>(d);
  return rc;
}

// An int8 linear weight with per-output-channel scales, OVW1 layout 0 ([N,K],
// "nk") or 1 ([K,N], "kn"): make_linear, mat.cpp:69-106.
int load_linear(const OvhLm& L, const TensorIndex& ix, const std::string& name, int64_t N,
                int64_t K, OvhWeight** out) {
  const OvhTensorView* t = ix.find(name);
  if (!t) return missing(name);
  if (t->ndim != 2) return set_error(OV_ERR_INVALID_ARG, name + ": expected a 2-D weight");
  if (t->dtype != 1 || !t->quantized || !t->scales)
    return set_error(OV_ERR_NOT_IMPLEMENTED,
                     name + ": the HIP runner takes int8 weights with per-channel scales");
  const int layout = t->transposed ? 1 : 0;
  const int64_t n = layout ? t->dims[1] : t->dims[0], k = layout ? t->dims[0] : t->dims[1];
  if (n != N || k != K || t->n_scales != N)
    return set_error(OV_ERR_INVALID_ARG, name + ": shape mismatch (expected N=" +
                                             std::to_string(N) + ", K=" + std::to_string(K) + ")");
  return ovh_weight_upload(N, K, static_cast<const int8_t*>(t->data), t->scales, layout, L.st, out);
}

// The audio head (make_linear, mat.cpp:69-106, as LM's constructor loads it):
// int8 with per-channel scales in either layout, or fp32 stored pre-transposed
// [K, N] (the reference's fp32 encoding; an fp32 [N, K] tensor is an error
// there too).
int load_head(const OvhLm& L, const TensorIndex& ix, const std::string& name, int64_t N,
              int64_t K, OvhWeight** out) {
  const OvhTensorView* t = ix.find(name);
  if (!t) return missing(name);
  if (t->ndim != 2 || t->dtype != 0) return load_linear(L, ix, name, N, K, out);
  if (!t->transposed)
    return set_error(OV_ERR_INVALID_ARG,
                     name + ": expected a pre-transposed weight or an int8 [N,K] weight");
  if (t->dims[0] != K || t->dims[1] != N || !t->data)
    return set_error(OV_ERR_INVALID_ARG, name + ": shape mismatch (expected [K=" +
                                             std::to_string(K) + ", N=" + std::to_string(N) + "])");
  return ovh::weight_upload_f32(N, K, static_cast<const float*>(t->data), 1, L.st, out);
}

// Embedding table [rows, H]: fp32, or int8 + per-row scale (make_emb, mat.cpp:108-128).
int load_emb(OvhLm& L, const TensorIndex& ix, const std::string& name, int64_t H,
             ovh::EmbTable* tab, int64_t* rows) {
  const OvhTensorView* t = ix.find(name);
  if (!t) return missing(name);
  if (t->ndim != 2 || t->transposed || t->dims[1] != H)
    return set_error(OV_ERR_INVALID_ARG, name + ": expected a row-major [rows, hidden] table");
  *rows = t->dims[0];
  void* d = nullptr;
  *tab = ovh::EmbTable{nullptr, nullptr, nullptr, t->dims[0]};
  if (t->dtype == 0) {
    int rc = upload_bytes(L, t->data, sizeof(float) * (size_t)(t->dims[0] * H), &d);
    tab->f32 = static_cast<const float*>(d);
    return rc;
  }
  if (t->dtype == 1 && t->quantized && t->scales && t->n_scales == t->dims[0]) {
    int rc = upload_bytes(L, t->data, (size_t)(t->dims[0] * H), &d);
    if (rc != OV_OK) return rc;
    tab->i8 = static_cast<const int8_t*>(d);
    rc = upload_bytes(L, t->scales, sizeof(float) * (size_t)t->dims[0], &d);
    tab->scale = static_cast<const float*>(d);
    return rc;
  }
  return set_error(OV_ERR_INVALID_ARG, name + ": unsupported dtype for an embedding");
}

int build(OvhLm& L, const TensorIndex& ix) {
  const OvhLmConfig& c = L.cfg;
  const int64_t H = c.hidden, QD = (int64_t)c.n_heads * c.head_dim,
                KVD = (int64_t)c.n_kv_heads * c.head_dim, I = c.inter;
  int rc = load_emb(L, ix, "llm.embed_tokens.weight", H, &L.tok, &L.tok_rows);
  if (rc == OV_OK) rc = load_emb(L, ix, "audio_embeddings.weight", H, &L.aud, &L.aud_rows);
  if (rc != OV_OK) return rc;
  if (L.aud_rows != (int64_t)c.n_codebooks * c.audio_vocab)
    return set_error(OV_ERR_INVALID_ARG, "audio embedding rows mismatch");
  rc = load_head(L, ix, "audio_heads.weight", (int64_t)c.n_codebooks * c.audio_vocab, H, &L.head);
  if (rc == OV_OK && L.head->f32 && (H % 256 != 0 || H > 1024))
    rc = set_error(OV_ERR_NOT_IMPLEMENTED,
                   "an fp32 audio head needs hidden a multiple of 256, at most 1024");
  if (rc == OV_OK) rc = load_norm(L, ix, "llm.norm.weight", H, &L.final_norm);
  if (rc != OV_OK) return rc;
  const OvhTensorView* offs = ix.find("codebook_layer_offsets");
  if (!offs) return missing("codebook_layer_offsets");
  if (offs->dtype != 3 || offs->ndim < 1 || offs->dims[0] != c.n_codebooks || !offs->data)
    return set_error(OV_ERR_INVALID_ARG, "codebook_layer_offsets: unexpected size");
  L.offsets.assign(static_cast<const int64_t*>(offs->data),
                   static_cast<const int64_t*>(offs->data) + c.n_codebooks);
  void* d = nullptr;
  rc = upload_bytes(L, L.offsets.data(), sizeof(int64_t) * L.offsets.size(), &d);
  if (rc != OV_OK) return rc;
  L.d_offsets = static_cast<int64_t*>(d);

  L.layers.resize((size_t)c.n_layers);
  for (int i = 0; i < c.n_layers; ++i) {
    const std::string p = "llm.layers." + std::to_string(i) + ".";
    OvhLm::Layer& Y = L.layers[(size_t)i];
    rc = load_norm(L, ix, p + "input_layernorm.weight", H, &Y.ln1);
    if (rc == OV_OK) rc = load_norm(L, ix, p + "post_attention_layernorm.weight", H, &Y.ln2);
    if (rc == OV_OK) rc = load_norm(L, ix, p + "self_attn.q_norm.weight", c.head_dim, &Y.qn);
    if (rc == OV_OK) rc = load_norm(L, ix, p + "self_attn.k_norm.weight", c.head_dim, &Y.kn);
    OvhWeight *q = nullptr, *k = nullptr, *v = nullptr, *g = nullptr, *u = nullptr;
    if (rc == OV_OK) rc = load_linear(L, ix, p + "self_attn.q_proj.weight", QD, H, &q);
    if (rc == OV_OK) rc = load_linear(L, ix, p + "self_attn.k_proj.weight", KVD, H, &k);
    if (rc == OV_OK) rc = load_linear(L, ix, p + "self_attn.v_proj.weight", KVD, H, &v);
    if (rc == OV_OK) rc = load_linear(L, ix, p + "self_attn.o_proj.weight", H, QD, &Y.o);
    if (rc == OV_OK) rc = load_linear(L, ix, p + "mlp.gate_proj.weight", I, H, &g);
    if (rc == OV_OK) rc = load_linear(L, ix, p + "mlp.up_proj.weight", I, H, &u);
    if (rc == OV_OK) rc = load_linear(L, ix, p + "mlp.down_proj.weight", H, I, &Y.down);
    // q/k/v and gate/up merged once at load time (combine_packed, lm.cpp:57-94).
    if (rc == OV_OK) {
      const OvhWeight* parts[3] = {q, k, v};
      rc = ovh_weight_concat(parts, 3, L.st, &Y.qkv);
    }
    if (rc == OV_OK) {
      if (L.silu_fused) {  // rows interleaved for the SiLU-fused GEMM epilogue
        rc = ovh::weight_interleave16(g, u, L.st, &Y.gate_up);
      } else {
        const OvhWeight* parts[2] = {g, u};
        rc = ovh_weight_concat(parts, 2, L.st, &Y.gate_up);
      }
    }
    ovh_weight_free(q);
    ovh_weight_free(k);
    ovh_weight_free(v);
    ovh_weight_free(g);
    ovh_weight_free(u);
    if (rc != OV_OK) return rc;
  }
  OVH_HIP(hipStreamSynchronize(L.st), "LM upload");
  return OV_OK;
}

// One attention segment as given by the caller (host mask, nullable).
struct SegIn {
  const uint8_t* mask;  // [rows, rows], 1 = attend; nullptr = all attend
  int rows;
  int64_t row0;
};

// RoPE cos/sin tables [T, D/2] for the position list, built on the host exactly
// as qk_norm_rope_f32 builds its cached tables (cpp/src/backend/cpu/ops_cpu.cpp:
// 958-993): inv_freq = (float)pow(theta, -2i/D) in double, angle = (float)pos *
// inv_freq in float, then libm cosf / sinf, so the tables are the reference's
// bits.  Like the reference, the tables are cached by position list: a decode
// loop whose positions do not change builds and uploads them once.
int rope_tables_cached(OvhLm& L, const int64_t* pos, int64_t T, float** cos_out,
                       float** sin_out) {
  const int D = L.cfg.head_dim, half = D / 2;
  const size_t n = (size_t)T * half;
  const bool same = (int64_t)L.tab_pos.size() == T &&
                    std::equal(L.tab_pos.begin(), L.tab_pos.end(), pos);
  if (!same) {
    if (2 * n > L.tab_cap) {
      if (L.d_tab) OVH_HIP(hipFree(L.d_tab), "hipFree(rope tables)");
      L.d_tab = nullptr;
      L.tab_cap = 0;
      OVH_HIP(hipMalloc(reinterpret_cast<void**>(&L.d_tab), sizeof(float) * 2 * n),
              "hipMalloc(rope tables)");
      L.tab_cap = 2 * n;
    }
    std::vector<float> inv_freq((size_t)half);
    for (int i = 0; i < half; ++i)
      inv_freq[(size_t)i] = (float)std::pow((double)L.cfg.rope_theta, -2.0 * i / (double)D);
    L.tab_host.resize(2 * n);
    for (int64_t r = 0; r < T; ++r) {
      const float p = (float)pos[r];
      for (int i = 0; i < half; ++i) {
        const float angle = p * inv_freq[(size_t)i];
        L.tab_host[(size_t)r * half + i] = std::cos(angle);
        L.tab_host[n + (size_t)r * half + i] = std::sin(angle);
      }
    }
    OVH_HIP(hipMemcpyAsync(L.d_tab, L.tab_host.data(), sizeof(float) * 2 * n,
                           hipMemcpyHostToDevice, L.st),
            "upload rope tables");
    L.tab_pos.assign(pos, pos + T);
  }
  *cos_out = L.d_tab;
  *sin_out = L.d_tab + n;
  return OV_OK;
}

bool all_ones(const uint8_t* m, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    if (!m[i]) return false;
  return true;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// The stage timer's sums for the forward just enqueued: waits for its last
// event, then adds each stage's time (from the mark before it) to its label,
// labels in the order they first appear.
int stage_times(OvhLm& L) {
  L.prof_ms.clear();
  if (L.prof_n < 2) return OV_OK;
  OVH_HIP(hipEventSynchronize(L.prof_ev[L.prof_n - 1]), "stage timer: hipEventSynchronize");
  for (size_t i = 1; i < L.prof_n; ++i) {
    float ms = 0.f;
    OVH_HIP(hipEventElapsedTime(&ms, L.prof_ev[i - 1], L.prof_ev[i]),
            "stage timer: hipEventElapsedTime");
    auto it = std::find_if(L.prof_ms.begin(), L.prof_ms.end(), [&](const auto& kv) {
      return std::strcmp(kv.first, L.prof_lab[i]) == 0;
    });
    if (it == L.prof_ms.end())
      L.prof_ms.emplace_back(L.prof_lab[i], (double)ms);
    else
      it->second += ms;
  }
  if (L.profile_print) {
    std::fprintf(stderr, "[hip-stage]");
    for (const auto& kv : L.prof_ms) std::fprintf(stderr, " %s=%.3f", kv.first, kv.second);
    std::fprintf(stderr, "\n");
  }
  return OV_OK;
}

// Forward over T rows laid out as `batch` x `seq` for the embedding's id indexing
// ([batch, C, seq]), attention split into `segs`.
int forward_rows(OvhLm& L, int batch, int seq, const std::vector<SegIn>& segs,
                 const int64_t* ids, const uint8_t* audio_mask, const int64_t* pos) {
  const OvhLmConfig& c = L.cfg;
  const int64_t T = (int64_t)batch * seq;
  const int64_t H = c.hidden, D = c.head_dim, QD = (int64_t)c.n_heads * D,
                KVD = (int64_t)c.n_kv_heads * D, I = c.inter, C = c.n_codebooks,
                CV = (int64_t)c.n_codebooks * c.audio_vocab;
  // Id range checks (Emb::gather throws on these, mat.cpp:58-60).
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t s = 0; s < seq; ++s) {
      const int64_t row = b * seq + s;
      if (audio_mask[row]) {
        for (int64_t cb = 0; cb < C; ++cb) {
          const int64_t id = ids[(b * C + cb) * seq + s] + L.offsets[(size_t)cb];
          if (id < 0 || id >= L.aud_rows)
            return set_error(OV_ERR_INVALID_ARG, "embedding id out of range: " + std::to_string(id));
        }
      } else {
        const int64_t id = ids[b * C * seq + s];
        if (id < 0 || id >= L.tok_rows)
          return set_error(OV_ERR_INVALID_ARG, "embedding id out of range: " + std::to_string(id));
      }
    }
  // Masks that are all ones add a zero bias: skip them.
  // The split attention takes masks as bit words, the fp32 kernel as biases.
  const bool split = L.attn_split && (int)segs.size() <= ovh::kAttnMaxSegs;
  // Activation codes tile-major on the main path (split attention, SiLU in the
  // gate/up epilogue, a hidden width the RMSNorm rows kernel takes): every
  // GEMM then moves its A tiles as 1 KiB contiguous DMA.  Rows are padded to a
  // multiple of 128 (the tallest GEMM tile reads whole tiles).
  // tile-major codes need the 16x16 GEMM for every projection that reads them
  // (K a multiple of 128: H, and inter for down)
  const bool tiled = split && L.silu_fused && H % 256 == 0 && H <= 1024 && I % 128 == 0;
  const int64_t Tpad = (T + 127) / 128 * 128;
  // From f16_min_rows() rows (when set) the GEMMs take int8-valued f16
  // operands: every int8 weight gets its f16 copy (made once, before any
  // capture) and the codes are widened into one arena buffer ahead of each GEMM.
  const int64_t f16_rows = ovh::f16_min_rows();
  bool f16 = tiled && f16_rows > 0 && T >= f16_rows;
  for (const OvhLm::Layer& Y : L.layers)
    if (f16)
      f16 = ovh::weight_f16(Y.qkv, L.st) && ovh::weight_f16(Y.o, L.st) &&
            ovh::weight_f16(Y.gate_up, L.st) && ovh::weight_f16(Y.down, L.st);
  if (f16 && !L.head->f32) f16 = ovh::weight_f16(L.head, L.st);
  // the residual GEMMs' fused norm: tile-major codes, the int8 GEMM form,
  // below 2048 rows (from there, on 64-row bands, it measured no faster than
  // the separate norm: config 5 forward 39.5 against 39.4 ms)
  const bool nfuse = L.norm_fused && tiled && !f16 && T < 2048 && ovh::norm_fusable();
  // a condition forced from the host (ovh_lm_force_condition) for this forward
  const int force = L.force;
  L.force = 0;
  const int xcd_test = (force & OVH_LM_FORCE_XCD) ? 1 : 0;
  // L2 prefetch of o_proj's weight by the attention launch (below 2048 rows,
  // int8 form).  With the fused norm every XCD reads the whole weight (its own
  // row bands), so every XCD loads all of it; the plain residual launch's XCDs
  // read an eighth each.  The launcher adds the workgroups only where they fit
  // beside the attention's own.
  const bool pf_on = L.prefetch && split && !f16 && T < 2048;
  auto prefetch_of = [&](const OvhWeight* w, int wgs) {
    ovh::L2Prefetch p;
    if (!pf_on) return p;
    p.p = w->w.q;
    p.bytes = w->w.Npad * w->w.Kp;
    p.wgs = wgs;
    p.sleep = 1;
    p.slice = nfuse ? 0 : 1;
    return p;
  };
  const bool emb_norm = nfuse && C <= ovh::kEmbMaxC && !L.layers.empty();
  if (nfuse && ovh::band_counter_words(T) > L.band_words) {
    // before any capture; the old counters may still be in use by the stream
    OVH_HIP(hipStreamSynchronize(L.st), "hipStreamSynchronize");
    if (L.d_band) OVH_HIP(hipFree(L.d_band), "hipFree(band counters)");
    L.d_band = nullptr;
    L.band_words = 0;
    const int64_t words = ovh::band_counter_words(2048);
    OVH_HIP(hipMalloc(reinterpret_cast<void**>(&L.d_band), sizeof(unsigned long long) * words),
            "hipMalloc(band counters)");
    OVH_HIP(hipMemset(L.d_band, 0, sizeof(unsigned long long) * words), "hipMemset(band counters)");
    L.band_words = words;
  }
  if (nfuse && (force & OVH_LM_FORCE_BAND_WAIT)) {
    // the first band's counter one short of a launch boundary: its first
    // arrival finds the counter off the boundary, the others wait for an
    // arrival that never comes until their bounded wait runs out
    OVH_HIP(hipStreamSynchronize(L.st), "hipStreamSynchronize");
    const unsigned long long off = ovh::kBandRound - 1;
    OVH_HIP(hipMemcpy(L.d_band, &off, sizeof off, hipMemcpyHostToDevice), "force band counter");
  }
  std::vector<int64_t> bias_off(segs.size(), -1), bits_off(segs.size(), -1);
  int64_t bias_elems = 0, bits_words = 0;
  for (size_t i = 0; i < segs.size(); ++i) {
    const int64_t n = (int64_t)segs[i].rows * segs[i].rows;
    if (segs[i].mask && !all_ones(segs[i].mask, n)) {
      bias_off[i] = bias_elems;
      bias_elems += n;
      bits_off[i] = bits_words;
      bits_words += (int64_t)segs[i].rows * ((segs[i].rows + 31) / 32);
    }
  }
  const int64_t Kp_max = 32 * ovh::kb_of(I > QD ? (I > H ? I : H) : (QD > H ? QD : H));
  const int64_t Kb_max = Kp_max / 32;
  struct Buf {
    size_t off, bytes;
  };
  size_t cur = 0;
  auto take = [&](size_t bytes) {
    Buf b{cur, bytes};
    cur = align256(cur + bytes);
    return b;
  };
  // inputs, contiguous for one upload: ids | audio mask | attention masks
  const size_t ids_bytes = sizeof(int64_t) * (size_t)(T * C);
  // q/k/v GEMM with qk-norm + RoPE and the K/V planes in its epilogue (the
  // split attention path with tile-major codes; heads are 128 wide)
  const bool qkv_fused = tiled && (int)segs.size() <= ovh::kQkvMaxSegs;
  const size_t in_ids = 0, in_am = ids_bytes,                      // byte offsets
               in_mask = in_am + (((size_t)T + 7) & ~(size_t)7),
               in_qf = (in_mask + (size_t)bias_elems + 63) & ~(size_t)63,
               in_bytes = in_qf + (qkv_fused ? sizeof(ovh::QkvFuse) : 0);
  const Buf b_in = take(in_bytes),
            b_bias = take(split ? 0 : sizeof(float) * (size_t)bias_elems),
            b_bits = take(split ? sizeof(uint32_t) * (size_t)bits_words : 0),
            b_x = take(sizeof(float) * (size_t)(T * H)),
            b_aq = take((size_t)(Tpad * Kp_max)), b_asc = take(sizeof(float) * (size_t)(T * Kb_max)),
            b_q = take(sizeof(float) * (size_t)(T * QD)), b_k = take(sizeof(float) * (size_t)(T * KVD)),
            b_v = take(sizeof(float) * (size_t)(T * KVD)), b_at = take(sizeof(float) * (size_t)(T * QD)),
            b_g = take(sizeof(float) * (size_t)(Tpad * I)),  // also the SiLU codes, Tpad rows
            b_u = take(sizeof(float) * (size_t)(T * I)),
            b_lg = take(sizeof(float) * (size_t)(T * CV));
  // the post-attention norm's codes when o_proj writes them (its own operand,
  // the attention's codes, is still being read by the other bands)
  const Buf b_aq2 = take(nfuse ? (size_t)(Tpad * H) : 0),
            b_asc2 = take(nfuse ? sizeof(float) * (size_t)(T * (H / 32)) : 0);
  // fp32 head: the final norm's output as f16 hi/lo planes and row scales
  const bool head_f32 = L.head->f32;
  const size_t hplane = head_f32 ? sizeof(_Float16) * (size_t)ovh::f32_plane_halves(T, H) : 0;
  const Buf b_aq16 = take(f16 ? sizeof(_Float16) * (size_t)(Tpad * Kp_max) : 0);
  const Buf b_hh = take(hplane), b_hl = take(hplane),
            b_hs = take(head_f32 ? sizeof(float) * (size_t)Tpad : 0);
  // split-f16 attention planes (K and V tile-major, segments padded to 32 keys)
  int64_t vt_cols = 0;
  std::vector<int64_t> vt_off(segs.size());
  for (size_t i = 0; i < segs.size(); ++i) {
    vt_off[i] = vt_cols;
    vt_cols += (segs[i].rows + 31) / 32 * 32;
  }
  const Buf b_kh = take(split ? sizeof(_Float16) * (size_t)(KVD * vt_cols) : 0),
            b_kl = take(split ? sizeof(_Float16) * (size_t)(KVD * vt_cols) : 0),
            b_vh = take(split ? sizeof(_Float16) * (size_t)(KVD * vt_cols) : 0),
            b_vl = take(split ? sizeof(_Float16) * (size_t)(KVD * vt_cols) : 0);
  if (cur > L.arena_cap) {
    if (L.arena) OVH_HIP(hipFree(L.arena), "hipFree(arena)");
    L.arena = nullptr;
    L.arena_cap = 0;
    const size_t want = cur + cur / 4 + ((size_t)1 << 20);
    OVH_HIP(hipMalloc(reinterpret_cast<void**>(&L.arena), want), "hipMalloc(arena)");
    L.arena_cap = want;
  }
  auto at = [&](const Buf& b) { return static_cast<void*>(L.arena + b.off); };
  char* d_in = static_cast<char*>(at(b_in));
  int64_t* d_ids = reinterpret_cast<int64_t*>(d_in + in_ids);
  uint8_t* d_am = reinterpret_cast<uint8_t*>(d_in + in_am);
  uint8_t* d_mask = reinterpret_cast<uint8_t*>(d_in + in_mask);
  const ovh::QkvFuse* d_qf = reinterpret_cast<const ovh::QkvFuse*>(d_in + in_qf);
  float* x = static_cast<float*>(at(b_x));
  int8_t* aq = static_cast<int8_t*>(at(b_aq));
  float* asc = static_cast<float*>(at(b_asc));
  float* q = static_cast<float*>(at(b_q));
  float* k = static_cast<float*>(at(b_k));
  float* v = static_cast<float*>(at(b_v));
  float* att = static_cast<float*>(at(b_at));
  float* gate = static_cast<float*>(at(b_g));
  float* up = static_cast<float*>(at(b_u));
  float* logits = static_cast<float*>(at(b_lg));
  _Float16* aq16 = f16 ? static_cast<_Float16*>(at(b_aq16)) : nullptr;
  int8_t* aq2 = static_cast<int8_t*>(at(b_aq2));
  float* asc2 = static_cast<float*>(at(b_asc2));
  hipStream_t st = L.st;

  // stage the inputs in pinned memory (after the previous upload has left it)
  if (!L.in_done) OVH_HIP(hipEventCreateWithFlags(&L.in_done, hipEventDisableTiming), "hipEventCreate");
  OVH_HIP(hipEventSynchronize(L.in_done), "staging wait");
  if (in_bytes > L.h_in_cap) {
    if (L.h_in) OVH_HIP(hipHostFree(L.h_in), "hipHostFree(staging)");
    L.h_in = nullptr;
    L.h_in_cap = 0;
    const size_t want = in_bytes + in_bytes / 4 + 4096;
    OVH_HIP(hipHostMalloc(reinterpret_cast<void**>(&L.h_in), want, hipHostMallocDefault),
            "hipHostMalloc(staging)");
    L.h_in_cap = want;
  }
  std::memcpy(L.h_in + in_ids, ids, ids_bytes);
  std::memcpy(L.h_in + in_am, audio_mask, (size_t)T);
  for (size_t i = 0; i < segs.size(); ++i)
    if (bias_off[i] >= 0)
      std::memcpy(L.h_in + in_mask + bias_off[i], segs[i].mask,
                  (size_t)segs[i].rows * (size_t)segs[i].rows);
  if (qkv_fused) {
    // the layout-wide part of the fused q/k/v epilogue, uploaded with the inputs
    ovh::QkvFuse qf{};
    qf.QD = (int32_t)QD;
    qf.KVD = (int32_t)KVD;
    qf.n_segs = (int32_t)segs.size();
    for (size_t i = 0; i < segs.size(); ++i) {
      qf.row0[i] = (int32_t)segs[i].row0;
      qf.rows[i] = segs[i].rows;
      qf.vt_off[i] = vt_off[i];
    }
    qf.nkb = vt_cols / 32;
    qf.eps = c.rms_eps;
    qf.q = q;
    qf.kh = static_cast<_Float16*>(at(b_kh));
    qf.kl = static_cast<_Float16*>(at(b_kl));
    qf.vh = static_cast<_Float16*>(at(b_vh));
    qf.vl = static_cast<_Float16*>(at(b_vl));
    qf.overflow = L.d_overflow;
    std::memcpy(L.h_in + in_qf, &qf, sizeof qf);  // the RoPE tables are set below
  }
  // each segment's mask: bias rows (fp32 attention) or bit words (split form)
  std::vector<OvhAttnSegment> asegs(segs.size());
  std::vector<const uint32_t*> seg_bits(segs.size(), nullptr);
  for (size_t i = 0; i < segs.size(); ++i) {
    const float* bias = nullptr;
    if (bias_off[i] >= 0) {
      if (split)
        seg_bits[i] = static_cast<uint32_t*>(at(b_bits)) + bits_off[i];
      else
        bias = static_cast<float*>(at(b_bias)) + bias_off[i];
    }
    asegs[i] = OvhAttnSegment{bias, segs[i].rows, segs[i].row0 * QD, segs[i].row0 * KVD};
  }
  float *cosb = nullptr, *sinb = nullptr;
  int rc = rope_tables_cached(L, pos, T, &cosb, &sinb);
  if (rc != OV_OK) return rc;
  if (qkv_fused) {
    ovh::QkvFuse* hq = reinterpret_cast<ovh::QkvFuse*>(L.h_in + in_qf);
    hq->cos_tab = cosb;
    hq->sin_tab = sinb;
  }

  const float scale = 1.f / std::sqrt((float)D);
  ovh::AttnArgs aargs{};
  ovh::AttnSplit sp{};
  int max_rows = 0;
  if (split) {
    aargs.k = k; aargs.v = v; aargs.q = q; aargs.out = att;
    aargs.q_stride = QD; aargs.kv_stride = KVD; aargs.out_stride = QD;
    aargs.n_heads = c.n_heads; aargs.group = c.n_heads / c.n_kv_heads; aargs.scale = scale;
    aargs.n_segs = (int)asegs.size();
    for (size_t i = 0; i < asegs.size(); ++i) {
      aargs.segs[i] = ovh::AttnSeg{nullptr, asegs[i].rows, asegs[i].q_off, asegs[i].kv_off,
                                   seg_bits[i]};
      sp.vt_off[i] = vt_off[i];
      max_rows = asegs[i].rows > max_rows ? asegs[i].rows : max_rows;
    }
    sp.kh = static_cast<_Float16*>(at(b_kh));
    sp.kl = static_cast<_Float16*>(at(b_kl));
    sp.vh = static_cast<_Float16*>(at(b_vh));
    sp.vl = static_cast<_Float16*>(at(b_vl));
    sp.vt_cols = vt_cols;
    sp.n_kv_heads = c.n_kv_heads;
    sp.overflow = L.d_overflow;
    sp.aq = aq;  // attention writes the o_proj input already quantised
    sp.asc = asc;
    sp.aq_tiled = tiled;
  }
  // stage timer: an event after each stage, labelled with the stage
  L.prof_n = 0;
  auto mark = [&](const char* label) -> int {
    if (!L.profile) return OV_OK;
    if (L.prof_n == L.prof_ev.size()) {
      hipEvent_t e = nullptr;
      OVH_HIP(hipEventCreate(&e), "hipEventCreate(stage timer)");
      L.prof_ev.push_back(e);
      L.prof_lab.push_back(nullptr);
    }
    L.prof_lab[L.prof_n] = label;
    OVH_HIP(hipEventRecord(L.prof_ev[L.prof_n++], st), "hipEventRecord(stage timer)");
    return OV_OK;
  };
  if ((rc = mark("start")) != OV_OK) return rc;
  // The inputs go up first, in one copy; the staging buffer may be refilled
  // once it is done.
  OVH_HIP(hipMemcpyAsync(d_in, L.h_in, in_bytes, hipMemcpyHostToDevice, st), "upload inputs");
  OVH_HIP(hipEventRecord(L.in_done, st), "hipEventRecord");
  // Everything else the forward does on the device, in stream order: masks,
  // embedding, the layers, final norm and head.
  auto enqueue = [&]() -> int {
    int rc = OV_OK;
    auto norm_q = [&](const float* w) -> int {
      if (!tiled) return ovh_rmsnorm_quantize(T, H, x, w, c.rms_eps, aq, asc, st);
      OVH_HIP(ovh::launch_rmsnorm_quantize(T, H, x, w, c.rms_eps, aq, asc, st, true),
              "rmsnorm launch");
      return OV_OK;
    };
    // masks: bit words (split form, built by the embedding launch) or fp32 bias
    ovh::MaskJobs mj{};
    int64_t mask_wgs = 0;
    for (size_t i = 0; i < segs.size(); ++i) {
      if (bias_off[i] < 0) continue;
      const uint8_t* m = d_mask + bias_off[i];
      if (split) {
        mj.job[mj.n++] = ovh::MaskJob{m, const_cast<uint32_t*>(seg_bits[i]), segs[i].rows,
                                      (int32_t)mask_wgs};
        mask_wgs += (segs[i].rows + 3) / 4;
      } else {
        const int64_t n = (int64_t)segs[i].rows * segs[i].rows;
        hipLaunchKernelGGL(ovh::mask_to_bias_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256),
                           0, st, m, const_cast<float*>(asegs[i].bias), n);
        OVH_HIP(hipGetLastError(), "mask_to_bias launch");
      }
    }
    // with nfuse, the first layer's input norm runs in the embedding launch
    const ovh::EmbNorm en{emb_norm ? L.layers[0].ln1 : nullptr, c.rms_eps, aq, asc};
    hipLaunchKernelGGL(ovh::embed_kernel, dim3((unsigned)(T + mask_wgs)), dim3(256), 0, st, d_ids,
                       d_am, seq, (int)C, H, L.tok, L.aud, L.d_offsets, x, T, mj, en);
    OVH_HIP(hipGetLastError(), "embed launch");
    if ((rc = mark("prep+embed")) != OV_OK) return rc;
    const int64_t qkv_n[3] = {QD, KVD, KVD};
    float* qkv_c[3] = {q, k, v};
    const int64_t gu_n[2] = {I, I};
    float* gu_c[2] = {gate, up};
    for (size_t li = 0; li < L.layers.size(); ++li) {
      const OvhLm::Layer& Y = L.layers[li];
      // with nfuse, the embedding launch (layer 0) or the previous layer's down
      // launch normalised x into aq/asc
      if (!(li == 0 ? emb_norm : nfuse) && (rc = norm_q(Y.ln1)) != OV_OK) return rc;
      if (qkv_fused) {
        // q/k/v GEMM + qk-norm/RoPE + K/V planes in one launch, then attention
        ovh::GemmArgs ga;
        ga.M = (int)T;
        ga.N = (int)(QD + 2 * KVD);
        ga.Kb = (int)ovh::kb_of(H);
        ga.Kp = 32 * ovh::kb_of(H);
        ga.aq = aq;
        ga.asc = asc;
        ga.a_tiled = 1;
        ga.W = Y.qkv->w.q;
        ga.ws = Y.qkv->w.scale;
        ga.qf = d_qf;
        ga.qnw = Y.qn;
        ga.knw = Y.kn;
        ga.qkv_q_tiles = (int)(QD / 128);
        if (f16) {
          OVH_HIP(ovh::launch_widen_f16(aq, aq16, Tpad * ga.Kp, st), "widen codes");
          ga.W16 = Y.qkv->w.q16;
          ga.aq16 = aq16;
        }
        OVH_HIP(ovh::launch_gemm(ga, ovh::kQkvNorm, st), "q/k/v + qk-norm launch");
        if ((rc = mark("qkv")) != OV_OK) return rc;
        sp.pf = prefetch_of(Y.o, kPfAttnWgs);
        OVH_HIP(ovh::launch_attention_split_only(aargs, sp, max_rows, true, st), "attention launch");
        sp.pf = ovh::L2Prefetch{};
      } else if ((rc = ovh::linear_q_sliced(T, aq, asc, Y.qkv, qkv_n, qkv_c, 3, st, tiled, aq16,
                                            f16)) != OV_OK || (rc = mark("qkv")) != OV_OK) {
        return rc;
      } else if (split) {
        // q/k norm + RoPE, f16 planes of k and V, then attention
        OVH_HIP(ovh::launch_qk_norm_rope_split(q, k, Y.qn, Y.kn, T, c.n_heads, c.n_kv_heads, cosb,
                                               sinb, c.rms_eps, aargs, sp, max_rows, st),
                "qk_norm_rope launch");
        if ((rc = mark("qk_norm_rope")) != OV_OK) return rc;
        OVH_HIP(ovh::launch_attention_split_only(aargs, sp, max_rows, true, st), "attention launch");
      } else {
        if ((rc = ovh_qk_norm_rope(q, k, Y.qn, Y.kn, T, c.n_heads, c.n_kv_heads, (int)D, cosb,
                                   sinb, c.rms_eps, st)) != OV_OK ||
            (rc = mark("qk_norm_rope")) != OV_OK)
          return rc;
        if ((rc = ovh_attention(asegs.data(), (int)asegs.size(), c.n_heads, c.n_kv_heads, (int)D, q,
                                QD, k, v, KVD, scale, att, QD, st)) != OV_OK)
          return rc;
      }
      if (!split && (rc = ovh_s8_nk_quantize(T, QD, att, aq, asc, st)) != OV_OK) return rc;
      if ((rc = mark("attn")) != OV_OK) return rc;
      // x += o_proj(attention), then the post-attention norm's codes: in one
      // launch into aq2/asc2, or a second launch into aq/asc
      const int8_t* naq = nfuse ? aq2 : aq;
      const float* nasc = nfuse ? asc2 : asc;
      if (nfuse) {
        if ((rc = ovh::linear_q_norm(T, aq, asc, Y.o, x, H, Y.ln2, c.rms_eps, aq2, asc2, L.d_band,
                                     L.d_overflow, st, xcd_test)) != OV_OK ||
            (rc = mark("o_proj")) != OV_OK)
          return rc;
      } else {
        if ((rc = ovh::linear_q(T, aq, asc, Y.o, x, H, 1, st, tiled, aq16, f16)) != OV_OK) return rc;
        if ((rc = mark("o_proj")) != OV_OK) return rc;
        if ((rc = norm_q(Y.ln2)) != OV_OK) return rc;
      }
      // the norm after down: the next layer's input norm, or the final norm of
      // an int8 head
      const bool last = li + 1 == L.layers.size();
      const float* next_ln = last ? (head_f32 ? nullptr : L.final_norm) : L.layers[li + 1].ln1;
      if (L.silu_fused) {
        // h = silu(gate) * up, quantised, straight from the gate/up GEMM into the
        // (otherwise unused) gate/up buffers: codes [T][I], scales [T][I/32]
        ovh::GemmArgs ga;
        ga.M = (int)T;
        ga.N = (int)(2 * I);
        ga.Kb = (int)ovh::kb_of(H);
        ga.Kp = 32 * ovh::kb_of(H);
        ga.aq = naq;
        ga.asc = nasc;
        ga.W = Y.gate_up->w.q;
        ga.ws = Y.gate_up->w.scale;
        ga.hq = reinterpret_cast<int8_t*>(gate);
        ga.hsc = up;
        ga.hKp = I;
        ga.a_tiled = tiled;
        ga.h_tiled = tiled;
        if (f16) {
          OVH_HIP(ovh::launch_widen_f16(aq, aq16, Tpad * ga.Kp, st), "widen codes");
          ga.W16 = Y.gate_up->w.q16;
          ga.aq16 = aq16;
        }
        OVH_HIP(ovh::launch_gemm(ga, ovh::kSiluQuant, st), "gate/up + silu launch");
        if ((rc = mark("gate_up")) != OV_OK) return rc;
        if (nfuse && next_ln) {
          if ((rc = ovh::linear_q_norm(T, ga.hq, ga.hsc, Y.down, x, H, next_ln, c.rms_eps, aq, asc,
                                       L.d_band, L.d_overflow, st, xcd_test)) != OV_OK)
            return rc;
        } else if ((rc = ovh::linear_q(T, ga.hq, ga.hsc, Y.down, x, H, 1, st, tiled, aq16, f16)) !=
                   OV_OK) {
          return rc;
        }
      } else {
        if ((rc = ovh_linear_q_sliced(T, aq, asc, Y.gate_up, gu_n, gu_c, 2, st)) != OV_OK) return rc;
        if ((rc = mark("gate_up")) != OV_OK) return rc;
        if ((rc = ovh_silu_mul_quantize(T, I, gate, up, aq, asc, st)) != OV_OK) return rc;
        if ((rc = mark("silu")) != OV_OK) return rc;
        if ((rc = ovh_linear_q(T, aq, asc, Y.down, x, H, 1, st)) != OV_OK) return rc;
      }
      if ((rc = mark("down")) != OV_OK) return rc;
    }
    if (head_f32) {
      // rmsnorm_f32 then Mat's fp32 product (lm.cpp:383-385)
      const ovh::F32Weight& fw = L.head->fw;
      ovh::GemmF32Args ha;
      ha.M = (int)T;
      ha.N = (int)fw.N;
      ha.Ks = fw.Ks;
      ha.ahi = static_cast<_Float16*>(at(b_hh));
      ha.alo = static_cast<_Float16*>(at(b_hl));
      ha.ascale = static_cast<float*>(at(b_hs));
      ha.whi = fw.hi;
      ha.wlo = fw.lo;
      ha.wscale = fw.scale;
      ha.C = logits;
      ha.ldc = CV;
      OVH_HIP(ovh::launch_rmsnorm_split(T, H, x, L.final_norm, c.rms_eps, fw.Ks,
                                        static_cast<_Float16*>(at(b_hh)),
                                        static_cast<_Float16*>(at(b_hl)),
                                        static_cast<float*>(at(b_hs)), st),
              "final norm (split) launch");
      OVH_HIP(ovh::launch_gemm_f32(ha, st), "fp32 head launch");
      return mark("final_norm+head");
    }
    if (!nfuse && (rc = norm_q(L.final_norm)) != OV_OK) return rc;
    if ((rc = ovh::linear_q(T, aq, asc, L.head, logits, CV, 0, st, tiled, aq16, f16)) != OV_OK)
      return rc;
    return mark("final_norm+head");
  };

  if (!L.use_graphs || L.profile) {
    if ((rc = enqueue()) != OV_OK) return rc;
    if (L.profile && (rc = stage_times(L)) != OV_OK) return rc;
  } else {
    // One graph per forward layout: the shapes, the segments and their masks,
    // and every buffer address the launches take.  A changed layout (other
    // lengths, a grown arena, new RoPE tables) is captured anew; the same
    // layout replays over the new inputs the upload above brought.
    std::vector<int64_t> key = {batch, seq, split, L.silu_fused, f16, nfuse, pf_on, xcd_test,
                                (int64_t)(intptr_t)L.d_band, (int64_t)segs.size(),
                                (int64_t)in_bytes, (int64_t)(intptr_t)L.arena,
                                (int64_t)(intptr_t)cosb, (int64_t)(intptr_t)sinb};
    for (size_t i = 0; i < segs.size(); ++i) {
      key.push_back(segs[i].rows);
      key.push_back(segs[i].row0);
      key.push_back(bias_off[i]);
      key.push_back(bits_off[i]);
    }
    if (!L.graph || key != L.graph_key) {
      if (L.graph) OVH_HIP(hipGraphExecDestroy(L.graph), "hipGraphExecDestroy");
      L.graph = nullptr;
      L.graph_key.clear();
      OVH_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "begin capture");
      const int erc = enqueue();
      hipGraph_t g = nullptr;
      const hipError_t e = hipStreamEndCapture(st, &g);
      if (erc != OV_OK) {
        if (g) (void)hipGraphDestroy(g);
        return erc;
      }
      OVH_HIP(e, "end capture");
      const hipError_t ei = hipGraphInstantiate(&L.graph, g, nullptr, nullptr, 0);
      (void)hipGraphDestroy(g);
      if (ei != hipSuccess) L.graph = nullptr;
      OVH_HIP(ei, "hipGraphInstantiate");
      L.graph_key = key;
    }
    OVH_HIP(hipGraphLaunch(L.graph, st), "hipGraphLaunch");
  }
  L.logits = logits;
  return OV_OK;
}

// The runner's flag word (d_overflow): kFlagAttn, |k| or |v| beyond the f16
// range of the split attention (set by the q/k/v epilogue or the plane
// split); ovh::kNormErrWait / kNormErrXcd, a fused residual + norm launch's
// band hand-off failed.  Read, and cleared, where the runner synchronises
// with the host.
constexpr uint32_t kFlagAttn = 1u;
constexpr uint32_t kFlagNorm = ovh::kNormErrWait | ovh::kNormErrXcd;

int take_flags(OvhLm& L, uint32_t* flag) {
  *flag = 0;
  OVH_HIP(hipMemcpy(flag, L.d_overflow, sizeof *flag, hipMemcpyDeviceToHost), "read runner flags");
  if (*flag) {
    L.last_flags = *flag;
    const uint32_t zero = 0;
    OVH_HIP(hipMemcpy(L.d_overflow, &zero, sizeof zero, hipMemcpyHostToDevice),
            "clear runner flags");
  }
  return OV_OK;
}

int flag_error(uint32_t flag) {
  if (flag & kFlagNorm)
    return set_error(OV_ERR_INTERNAL, "residual GEMM + norm: the row bands' hand-off failed "
                                      "again with the norm as a launch of its own");
  return set_error(OV_ERR_INTERNAL, "attention inputs beyond the f16 range with the fp32 "
                                    "attention form selected");
}

// Switch to the exact fallbacks the flag calls for and keep them; false when
// a flagged condition has no fallback left (its form is already off).
int fall_back(OvhLm& L, uint32_t flag, bool* ok) {
  *ok = true;
  if (flag & kFlagAttn) {
    if (!L.attn_split) *ok = false;
    L.attn_split = false;
    L.recovered |= OVH_LM_RECOVERED_ATTENTION;
  }
  if (flag & kFlagNorm) {
    if (!L.norm_fused) *ok = false;
    L.norm_fused = false;
    L.recovered |= OVH_LM_RECOVERED_NORM;
    // the counters may stand anywhere now: from zero if the fused norm is
    // switched on again
    if (L.d_band) {
      OVH_HIP(hipStreamSynchronize(L.st), "hipStreamSynchronize");
      OVH_HIP(hipMemset(L.d_band, 0, sizeof(unsigned long long) * (size_t)L.band_words),
              "reset band counters");
    }
  }
  return OV_OK;
}

// The forward the runner may have to run again: its host inputs, kept when it
// left the logits on the device without synchronising.
int keep_last(OvhLm& L, int batch, int seq, const std::vector<SegIn>& segs, const int64_t* ids,
              const uint8_t* audio_mask, const int64_t* pos) {
  OvhLm::LastForward& f = L.last;
  const int64_t T = (int64_t)batch * seq;
  f.valid = false;
  f.batch = batch;
  f.seq = seq;
  f.ids.assign(ids, ids + T * L.cfg.n_codebooks);
  f.am.assign(audio_mask, audio_mask + T);
  f.pos.assign(pos, pos + T);
  f.seg_rows.clear();
  f.seg_row0.clear();
  f.mask_off.clear();
  f.masks.clear();
  for (const SegIn& g : segs) {
    f.seg_rows.push_back(g.rows);
    f.seg_row0.push_back(g.row0);
    if (g.mask) {
      f.mask_off.push_back((int64_t)f.masks.size());
      f.masks.insert(f.masks.end(), g.mask, g.mask + (size_t)g.rows * (size_t)g.rows);
    } else {
      f.mask_off.push_back(-1);
    }
  }
  f.valid = true;
  return OV_OK;
}

int run_last(OvhLm& L) {
  const OvhLm::LastForward& f = L.last;
  std::vector<SegIn> segs(f.seg_rows.size());
  for (size_t i = 0; i < segs.size(); ++i)
    segs[i] = SegIn{f.mask_off[i] < 0 ? nullptr : f.masks.data() + f.mask_off[i], f.seg_rows[i],
                    f.seg_row0[i]};
  return forward_rows(L, f.batch, f.seq, segs, f.ids.data(), f.am.data(), f.pos.data());
}

bool config_ok(const OvhLmConfig& c) {
  return c.n_layers > 0 && c.hidden > 0 && c.n_heads > 0 && c.n_kv_heads > 0 &&
         c.n_heads % c.n_kv_heads == 0 && c.head_dim == 128 && c.inter > 0 &&
         c.audio_vocab > 1 && c.audio_vocab <= ovh::kSampleThreads * ovh::kSampleMaxPer &&
         c.n_codebooks > 0 && c.hidden % 64 == 0 && ((int64_t)c.n_heads * c.head_dim) % 64 == 0 &&
         ((int64_t)c.n_kv_heads * c.head_dim) % 64 == 0 && c.inter % 64 == 0;
}

}  // namespace

extern "C" {

int ovh_lm_create(const OvhLmConfig* cfg, const OvhTensorView* tensors, int n_tensors,
                  void* stream, OvhLm** out) {
  if (!out) return set_error(OV_ERR_INVALID_ARG, "out is null");
  *out = nullptr;
  if (!cfg || !tensors || n_tensors <= 0) return set_error(OV_ERR_INVALID_ARG, "no config/tensors");
  if (!config_ok(*cfg))
    return set_error(OV_ERR_NOT_IMPLEMENTED,
                     "LM config: the HIP runner needs head_dim 128, n_heads % n_kv_heads == 0, "
                     "projection widths that are multiples of 64 and audio_vocab <= 2048");
  TensorIndex ix;
  for (int i = 0; i < n_tensors; ++i)
    if (tensors[i].name) ix.by_name[tensors[i].name] = &tensors[i];
  OvhLm* L = new (std::nothrow) OvhLm();
  if (!L) return set_error(OV_ERR_INTERNAL, "out of host memory");
  L->cfg = *cfg;
  L->st = static_cast<hipStream_t>(stream);
  if (!L->st) {
    // A stream of the runner's own, created with the default flags: it stays
    // ordered with the legacy default stream the caller uses, and the forward
    // can be captured into a graph on it.
    if (hipStreamCreate(&L->own_st) != hipSuccess) {
      delete L;
      return set_error(OV_ERR_INTERNAL, "hipStreamCreate");
    }
    L->st = L->own_st;
  }
  // the SiLU-fused gate/up GEMM takes K = hidden in 4-block stages (hidden a
  // multiple of 128); other widths compose the sliced GEMM and silu_mul_quantize
  L->silu_fused = cfg->inter % 64 == 0 && cfg->hidden % 128 == 0;
  // the stage timer from the environment, printing as the reference's does
  if (std::getenv("OVH_LM_PROFILE")) L->profile = L->profile_print = true;
  int rc = OV_OK;
  if (hipMalloc(reinterpret_cast<void**>(&L->d_overflow), sizeof(uint32_t)) != hipSuccess ||
      hipMemset(L->d_overflow, 0, sizeof(uint32_t)) != hipSuccess)
    rc = set_error(OV_ERR_INTERNAL, "hipMalloc(overflow flag)");
  if (rc == OV_OK) rc = build(*L, ix);
  if (rc != OV_OK) {
    (void)hipStreamSynchronize(L->st);
    delete L;
    return rc;
  }
  *out = L;
  return OV_OK;
}

void ovh_lm_destroy(OvhLm* lm) {
  if (!lm) return;
  (void)hipStreamSynchronize(lm->st);
  delete lm;
}

int ovh_lm_forward(OvhLm* lm, int batch, int seq, const int64_t* input_ids,
                   const uint8_t* audio_mask, const uint8_t* attn_mask,
                   const int64_t* position_ids, float* logits) {
  if (!lm) return set_error(OV_ERR_INVALID_ARG, "lm is null");
  if (batch <= 0 || seq <= 0) return set_error(OV_ERR_INVALID_ARG, "batch and seq must be positive");
  if (!input_ids || !audio_mask || !attn_mask || !position_ids)
    return set_error(OV_ERR_INVALID_ARG, "null host input");
  std::vector<SegIn> segs((size_t)batch);
  for (int b = 0; b < batch; ++b)
    segs[(size_t)b] = SegIn{attn_mask + (int64_t)b * seq * seq, seq, (int64_t)b * seq};
  int rc = forward_rows(*lm, batch, seq, segs, input_ids, audio_mask, position_ids);
  if (rc != OV_OK) return rc;
  // logits left on the device: the sample that reads them checks the flags
  if (!logits || lm->device_sampling)
    return keep_last(*lm, batch, seq, segs, input_ids, audio_mask, position_ids);
  lm->last.valid = false;
  // [B*S, C*V] on the device -> [B, C, S, V] on the host (cuda_lm.cu:1184-1199).
  const int C = lm->cfg.n_codebooks, V = lm->cfg.audio_vocab;
  const size_t n = (size_t)batch * seq * C * V;
  lm->host_flat.resize(n);
  for (;;) {
    OVH_HIP(hipMemcpyAsync(lm->host_flat.data(), lm->logits, sizeof(float) * n,
                           hipMemcpyDeviceToHost, lm->st),
            "download logits");
    OVH_HIP(hipStreamSynchronize(lm->st), "forward sync");
    uint32_t flag = 0;
    bool ok = true;
    if ((rc = take_flags(*lm, &flag)) != OV_OK) return rc;
    if (!flag) break;
    // the forward again on the fallback its flags call for
    if ((rc = fall_back(*lm, flag, &ok)) != OV_OK) return rc;
    if (!ok) return flag_error(flag);
    if ((rc = forward_rows(*lm, batch, seq, segs, input_ids, audio_mask, position_ids)) != OV_OK)
      return rc;
  }
  for (int b = 0; b < batch; ++b)
    for (int cb = 0; cb < C; ++cb)
      for (int s = 0; s < seq; ++s)
        std::memcpy(logits + (((size_t)b * C + cb) * seq + s) * V,
                    lm->host_flat.data() + ((size_t)b * seq + s) * C * V + (size_t)cb * V,
                    sizeof(float) * (size_t)V);
  return OV_OK;
}

int ovh_lm_forward_cfg(OvhLm* lm, int cond_seq, int uncond_seq, const int64_t* input_ids,
                       const uint8_t* audio_mask, const uint8_t* cond_attn,
                       const uint8_t* uncond_attn, const int64_t* position_ids, float* logits) {
  if (!lm) return set_error(OV_ERR_INVALID_ARG, "lm is null");
  if (cond_seq <= 0 || uncond_seq <= 0)
    return set_error(OV_ERR_INVALID_ARG, "forward_cfg: both segments must be non-empty");
  if (!input_ids || !audio_mask || !cond_attn || !uncond_attn || !position_ids)
    return set_error(OV_ERR_INVALID_ARG, "null host input");
  const int rows = cond_seq + uncond_seq;
  std::vector<SegIn> segs = {SegIn{cond_attn, cond_seq, 0}, SegIn{uncond_attn, uncond_seq, cond_seq}};
  int rc = forward_rows(*lm, 1, rows, segs, input_ids, audio_mask, position_ids);
  if (rc != OV_OK) return rc;
  if (!logits || lm->device_sampling)
    return keep_last(*lm, 1, rows, segs, input_ids, audio_mask, position_ids);
  lm->last.valid = false;
  const size_t n = (size_t)rows * lm->cfg.n_codebooks * lm->cfg.audio_vocab;
  for (;;) {
    OVH_HIP(hipMemcpyAsync(logits, lm->logits, sizeof(float) * n, hipMemcpyDeviceToHost, lm->st),
            "download logits");
    OVH_HIP(hipStreamSynchronize(lm->st), "forward sync");
    uint32_t flag = 0;
    bool ok = true;
    if ((rc = take_flags(*lm, &flag)) != OV_OK) return rc;
    if (!flag) return OV_OK;
    if ((rc = fall_back(*lm, flag, &ok)) != OV_OK) return rc;
    if (!ok) return flag_error(flag);
    if ((rc = forward_rows(*lm, 1, rows, segs, input_ids, audio_mask, position_ids)) != OV_OK)
      return rc;
  }
}

const void* ovh_lm_last_logits(const OvhLm* lm) { return lm ? lm->logits : nullptr; }

void ovh_lm_set_device_sampling(OvhLm* lm, int on) {
  if (lm) lm->device_sampling = on != 0;
}

void ovh_lm_set_attention(OvhLm* lm, int split_f16) {
  if (lm) lm->attn_split = split_f16 != 0;
}

void ovh_lm_set_graphs(OvhLm* lm, int on) {
  if (lm) lm->use_graphs = on != 0;
}

void ovh_lm_set_fused_norm(OvhLm* lm, int on) {
  if (lm) lm->norm_fused = on != 0;
}

void ovh_lm_set_prefetch(OvhLm* lm, int on) {
  if (lm) lm->prefetch = on != 0;
}

int ovh_lm_recovered(const OvhLm* lm) { return lm ? lm->recovered : 0; }

int ovh_lm_last_flags(const OvhLm* lm) { return lm ? (int)lm->last_flags : 0; }

void ovh_lm_force_condition(OvhLm* lm, int what) {
  if (lm) lm->force = what & (OVH_LM_FORCE_BAND_WAIT | OVH_LM_FORCE_XCD);
}

void ovh_lm_set_profile(OvhLm* lm, int on) {
  if (!lm) return;
  lm->profile = on != 0;
  if (!on) lm->profile_print = false;
}

int ovh_lm_stage_times(const OvhLm* lm, double* ms, const char** names, int n) {
  if (!lm) return 0;
  const int k = (int)lm->prof_ms.size();
  for (int i = 0; i < k && i < n; ++i) {
    if (ms) ms[i] = lm->prof_ms[(size_t)i].second;
    if (names) names[i] = lm->prof_ms[(size_t)i].first;
  }
  return k;
}

int ovh_lm_sample(OvhLm* lm, const void* cond, int cond_seq, const void* uncond, int uncond_seq,
                  int target_len, float guidance, float layer_penalty, int32_t* pred,
                  float* scores) {
  if (!lm) return set_error(OV_ERR_INVALID_ARG, "lm is null");
  if (!cond || !uncond || !pred || !scores) return set_error(OV_ERR_INVALID_ARG, "null argument");
  if (target_len <= 0 || target_len > cond_seq || target_len > uncond_seq)
    return set_error(OV_ERR_INVALID_ARG, "sample: need 0 < target_len <= both plane lengths");
  const int C = lm->cfg.n_codebooks, V = lm->cfg.audio_vocab;
  const int64_t n = (int64_t)C * target_len;
  constexpr size_t kHead = 64;  // the runner's flag word, padded
  if (n > lm->sample_cap) {
    OVH_HIP(hipStreamSynchronize(lm->st), "sample sync");
    if (lm->d_out) OVH_HIP(hipFree(lm->d_out), "hipFree");
    if (lm->h_out) OVH_HIP(hipHostFree(lm->h_out), "hipHostFree");
    lm->d_out = nullptr;
    lm->h_out = nullptr;
    lm->sample_cap = 0;
    const size_t bytes = kHead + 8 * (size_t)n;
    OVH_HIP(hipMalloc(reinterpret_cast<void**>(&lm->d_out), bytes), "hipMalloc(sample out)");
    OVH_HIP(hipHostMalloc(reinterpret_cast<void**>(&lm->h_out), bytes, hipHostMallocDefault),
            "hipHostMalloc(sample out)");
    lm->sample_cap = n;
  }
  const size_t bytes = kHead + 8 * (size_t)n;
  int32_t* d_pred = reinterpret_cast<int32_t*>(lm->d_out + kHead);
  float* d_scores = reinterpret_cast<float*>(lm->d_out + kHead + 4 * (size_t)n);
  for (;;) {
    // The mask token is the last audio id (kMaskId = 1024 with audio_vocab
    // 1025, cpp/src/model/tts.cpp:17).
    hipLaunchKernelGGL(ovh::guided_sample_kernel, dim3((unsigned)n), dim3(ovh::kSampleThreads), 0,
                       lm->st, static_cast<const float*>(cond), cond_seq,
                       static_cast<const float*>(uncond), C, V, target_len, guidance,
                       layer_penalty, V - 1, d_pred, d_scores, lm->d_overflow,
                       reinterpret_cast<uint32_t*>(lm->d_out));
    OVH_HIP(hipGetLastError(), "guided sample launch");
    OVH_HIP(hipMemcpyAsync(lm->h_out, lm->d_out, bytes, hipMemcpyDeviceToHost, lm->st),
            "download sample");
    OVH_HIP(hipStreamSynchronize(lm->st), "sample sync");
    uint32_t flag;
    std::memcpy(&flag, lm->h_out, sizeof flag);
    if (!flag) break;
    int rc = take_flags(*lm, &flag);
    if (rc != OV_OK) return rc;
    // Planes of the last forward (logits left on the device): that forward
    // again on its fallback, then this sample on its new logits (the arena
    // may have moved: same offsets).
    const char* base = reinterpret_cast<const char*>(lm->logits);
    // the last forward's logits: [rows][C * V], ids [C * rows]
    const size_t plane_bytes = lm->last.valid ? sizeof(float) * lm->last.ids.size() * (size_t)V : 0;
    auto own = [&](const void* p) {
      const char* c = static_cast<const char*>(p);
      return base && c >= base && c < base + plane_bytes;
    };
    if (!lm->last.valid || !own(cond) || !own(uncond))
      return set_error(OV_ERR_INTERNAL,
                       (flag & kFlagNorm)
                           ? "the last forward's residual GEMM + norm hand-off failed: its "
                             "logits are not to be used (ovh_lm_set_fused_norm(lm, 0))"
                           : "the last forward's attention inputs were beyond the f16 range: its "
                             "logits are not to be used (ovh_lm_set_attention(lm, 0))");
    const ptrdiff_t oc = static_cast<const char*>(cond) - base,
                    ou = static_cast<const char*>(uncond) - base;
    bool ok = true;
    if ((rc = fall_back(*lm, flag, &ok)) != OV_OK) return rc;
    if (!ok) return flag_error(flag);
    if ((rc = run_last(*lm)) != OV_OK) return rc;
    cond = reinterpret_cast<const char*>(lm->logits) + oc;
    uncond = reinterpret_cast<const char*>(lm->logits) + ou;
  }
  std::memcpy(pred, lm->h_out + kHead, 4 * (size_t)n);
  std::memcpy(scores, lm->h_out + kHead + 4 * (size_t)n, 4 * (size_t)n);
  return OV_OK;
}


// The CFG decoding loop of Pipeline::run_sampling (cpp/src/model/tts.cpp:165-364)
// on the accelerator branch (use_cuda: the B = 2 batch and the device sampler).
// Batch: row 0 = the full prompt, row 1 = the target slice of the prompt in its
// first T positions (full attention among them) and mask tokens attending only
// to themselves after that.  Schedule ts = t_shift*t / (1 + (t_shift-1)*t), per
// step ceil(total * (ts[s+1] - ts[s])) positions (the last step takes the rest).
// Each step: forward, guided argmax per (codebook, frame), Gumbel noise from
// std::mt19937(seed) / uniform_real_distribution<float>(0, 1) in row-major
// (codebook, frame) order, already-decoded positions at -inf, then the top-k
// positions take their predicted token in both rows.
int ovh_lm_generate(OvhLm* lm, const int64_t* prompt_ids, const uint8_t* prompt_audio_mask,
                    int seq, int target_len, const OvhGenOptions* opt, int64_t* tokens) {
  if (!lm || !prompt_ids || !prompt_audio_mask || !opt || !tokens)
    return set_error(OV_ERR_INVALID_ARG, "generate: null argument");
  if (seq <= 0 || target_len <= 0 || target_len > seq || opt->num_steps <= 0)
    return set_error(OV_ERR_INVALID_ARG, "generate: need 0 < target_len <= seq and num_steps > 0");
  const int C = lm->cfg.n_codebooks, V = lm->cfg.audio_vocab, S = seq, T = target_len;
  const int64_t mask_id = V - 1;  // kMaskId = 1024 for audio_vocab 1025 (tts.cpp:17)
  const size_t CS = (size_t)C * S;
  std::vector<int64_t> ids(2 * CS, mask_id);
  std::vector<uint8_t> amask(2 * (size_t)S, 0);
  std::vector<uint8_t> attn(2 * (size_t)S * S, 0);
  std::vector<int64_t> pos(2 * (size_t)S);
  std::memcpy(ids.data(), prompt_ids, sizeof(int64_t) * CS);
  std::memcpy(amask.data(), prompt_audio_mask, (size_t)S);
  std::fill(attn.begin(), attn.begin() + (size_t)S * S, (uint8_t)1);
  for (int c = 0; c < C; ++c)
    for (int t = 0; t < T; ++t)
      ids[CS + (size_t)c * S + t] = prompt_ids[(size_t)c * S + (S - T + t)];
  for (int t = 0; t < T; ++t) {
    amask[(size_t)S + t] = 1;
    for (int j = 0; j < T; ++j) attn[((size_t)S + t) * S + j] = 1;
  }
  for (int t = T; t < S; ++t) attn[((size_t)S + t) * S + t] = 1;
  for (int b = 0; b < 2; ++b)
    for (int i = 0; i < S; ++i) pos[(size_t)b * S + i] = i;

  const int steps = opt->num_steps;
  std::vector<double> ts((size_t)steps + 1);
  for (int i = 0; i <= steps; ++i) {
    const double t = (double)i / steps;
    ts[(size_t)i] = opt->t_shift * t / (1.0 + (opt->t_shift - 1.0) * t);
  }
  const int64_t total = (int64_t)T * C;
  std::vector<int> sched((size_t)steps, 0);
  int64_t rem = total;
  for (int st = 0; st < steps; ++st) {
    const int64_t num =
        st == steps - 1
            ? rem
            : std::min<int64_t>((int64_t)std::ceil(total * (ts[(size_t)st + 1] - ts[(size_t)st])), rem);
    sched[(size_t)st] = (int)num;
    rem -= num;
  }

  std::vector<int64_t> tok((size_t)total, mask_id);
  std::vector<float> scores((size_t)total);
  std::vector<int32_t> pred((size_t)total);
  std::vector<size_t> order((size_t)total);
  std::mt19937 rng(opt->seed);
  std::uniform_real_distribution<float> uni(0.f, 1.f);
  const bool prev = lm->device_sampling;
  lm->device_sampling = true;
  int rc = OV_OK;
  const size_t plane = (size_t)S * C * V;
  for (int st = 0; st < steps && rc == OV_OK; ++st) {
    const int k = sched[(size_t)st];
    if (k <= 0) continue;
    rc = ovh_lm_forward(lm, 2, S, ids.data(), amask.data(), attn.data(), pos.data(), nullptr);
    if (rc != OV_OK) break;
    const float* dev = lm->logits;
    rc = ovh_lm_sample(lm, dev, S, dev + plane, S, T, opt->guidance_scale, opt->layer_penalty,
                       pred.data(), scores.data());
    if (rc != OV_OK) break;
    for (size_t i = 0; i < scores.size(); ++i) {
      float u = uni(rng);
      u = std::max(u, 1e-10f);
      const float g = -std::log(-std::log(u) + 1e-10f);
      scores[i] = scores[i] / opt->position_temperature + g;
    }
    for (size_t i = 0; i < tok.size(); ++i)
      if (tok[i] != mask_id) scores[i] = -INFINITY;
    std::iota(order.begin(), order.end(), (size_t)0);
    const int kk = std::min<int>(k, (int)order.size());
    std::partial_sort(order.begin(), order.begin() + kk, order.end(),
                      [&](size_t a, size_t b) { return scores[a] > scores[b]; });
    for (int i = 0; i < kk; ++i) {
      const size_t idx = order[(size_t)i];
      if (!std::isfinite(scores[idx])) break;
      tok[idx] = pred[idx];
      const size_t c = idx / (size_t)T, t = idx % (size_t)T;
      ids[c * S + (S - T + t)] = pred[idx];
      ids[CS + c * S + t] = pred[idx];
    }
  }
  lm->device_sampling = prev;
  if (rc != OV_OK) return rc;
  std::memcpy(tokens, tok.data(), sizeof(int64_t) * tok.size());
  return OV_OK;
}

}  // extern "C"
