// ref_shim.cpp — extern "C" wrappers over the reference's own CPU int8-nk API
// (cpp/include/ovnative/ov_gemm.h, cpp/src/model/ops.h), so that Python tests
// and the CPU-baseline leg of bench.py can call the compiled reference.
//
// TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile into oracle/_ref/ from the
// reference sources where they lie; nothing in the product loads it.
// Exceptions thrown by the reference become negative return codes here.
#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <vector>

#include "model/lm.h"
#include "model/ops.h"
#include "ovnative/ov_gemm.h"
#include "ovnative/ov_weights.h"

#define REF_API extern "C" __attribute__((visibility("default")))

REF_API int ovref_vnni_available() { return ov::cpu_vnni_available() ? 1 : 0; }
REF_API const char* ovref_kernel_name() { return ov::cpu_kernel_name(); }
REF_API void ovref_enable_ftz() { ov::enable_flush_to_zero(); }

REF_API int ovref_s8_nk_quantize(int64_t M, int64_t K, const float* A, uint8_t* aq, float* asc) {
  try { ov::s8_nk_quantize(M, K, A, aq, asc); return 0; } catch (const std::exception&) { return -1; }
}
REF_API int ovref_rmsnorm_quantize(int64_t rows, int64_t cols, const float* x, const float* w,
                                   float eps, uint8_t* aq, float* asc) {
  try { ov::rmsnorm_quantize_f32(rows, cols, x, w, eps, aq, asc); return 0; }
  catch (const std::exception&) { return -1; }
}
REF_API int ovref_silu_mul_quantize(int64_t M, int64_t K, const float* g, const float* u,
                                    uint8_t* aq, float* asc) {
  try { ov::silu_mul_quantize_f32(M, K, g, u, aq, asc); return 0; }
  catch (const std::exception&) { return -1; }
}
REF_API void ovref_rmsnorm_into(float* dst, const float* src, const float* w, int64_t rows,
                                int64_t cols, float eps) {
  ov::rmsnorm_into_f32(dst, src, w, rows, cols, eps);
}
REF_API void ovref_silu_mul(float* out, const float* g, const float* u, int64_t n) {
  ov::silu_mul_f32(out, g, u, n);
}
REF_API int64_t ovref_packed_bytes(int64_t N, int64_t K) { return ov::s8_nk_packed_bytes(N, K); }
REF_API int64_t ovref_wsum_elems(int64_t N, int64_t K) { return ov::s8_nk_wsum_elems(N, K); }
REF_API void ovref_pack(int64_t N, int64_t K, const int8_t* W, int8_t* packed, int32_t* wsum) {
  ov::s8_nk_pack(N, K, W, packed, wsum);
}
REF_API int ovref_linear_packed_q(int64_t M, int64_t N, int64_t K, const uint8_t* aq,
                                  const float* asc, const int8_t* packed, const int32_t* wsum,
                                  const float* scale, float* C, int accumulate) {
  try {
    if (accumulate)
      ov::linear_s8_nk_packed_q_add(M, N, K, aq, asc, packed, wsum, scale, C);
    else
      ov::linear_s8_nk_packed_q(M, N, K, aq, asc, packed, wsum, scale, C);
    return 0;
  } catch (const std::exception&) { return -1; }
}
// linear_f32_ld (gemm.cpp:884-905): Mat's fp32 branch, W [K, N].
REF_API int ovref_linear_f32(int64_t M, int64_t N, int64_t K, const float* A, const float* W,
                             float* C, int64_t ldc, int accumulate) {
  try { ov::linear_f32_ld(M, N, K, A, W, C, ldc, accumulate != 0); return 0; }
  catch (const std::exception&) { return -1; }
}
REF_API int ovref_linear_packed(int64_t M, int64_t N, int64_t K, const float* A,
                                const int8_t* packed, const int32_t* wsum, const float* scale,
                                float* C, int accumulate) {
  try {
    if (accumulate)
      ov::linear_s8_nk_packed_add(M, N, K, A, packed, wsum, scale, C);
    else
      ov::linear_s8_nk_packed(M, N, K, A, packed, wsum, scale, C);
    return 0;
  } catch (const std::exception&) { return -1; }
}
// Returns -2 for std::invalid_argument (bad slice widths), -1 for other errors.
REF_API int ovref_linear_packed_q_sliced(int64_t M, int64_t K, const uint8_t* aq, const float* asc,
                                         const int8_t* packed, const int32_t* wsum,
                                         const float* scale, const int64_t* slice_n,
                                         float* const* slice_c, int n_slices) {
  std::vector<ov::S8NkSlice> s(static_cast<size_t>(n_slices > 0 ? n_slices : 0));
  for (int i = 0; i < n_slices; ++i) s[static_cast<size_t>(i)] = {slice_n[i], slice_c[i]};
  try {
    ov::linear_s8_nk_packed_q_sliced(M, K, aq, asc, packed, wsum, scale, s.data(), n_slices);
    return 0;
  } catch (const std::invalid_argument&) { return -2; }
  catch (const std::exception&) { return -1; }
}
REF_API void ovref_qk_norm_rope(float* q, float* k, const float* qw, const float* kw, int64_t rows,
                                int n_heads, int n_kv_heads, int head_dim, const int64_t* pos,
                                float theta, float eps) {
  ov::qk_norm_rope_f32(q, k, qw, kw, rows, n_heads, n_kv_heads, head_dim, pos, theta, eps);
}
REF_API void ovref_attention_head(const float* q, int64_t q_stride, const float* k, const float* v,
                                  int64_t kv_stride, const float* bias, int S, int D, float scale,
                                  float* out, int64_t out_stride) {
  ov::attention_head_f32(q, q_stride, k, v, kv_stride, bias, S, D, scale, out, out_stride);
}

// OVW1 reader (cpp/src/core/weight_file.cpp): opens files written by
// ovnative_amd/ovw1.py so the tests can check them against the reference loader.
REF_API void* ovref_ovw1_open(const char* path, char* err, size_t n) {
  try {
    return new ov::WeightFile(ov::WeightFile::Open(path));
  } catch (const std::exception& e) {
    if (err && n) std::snprintf(err, n, "%s", e.what());
    return nullptr;
  }
}
REF_API void ovref_ovw1_close(void* h) { delete static_cast<ov::WeightFile*>(h); }
REF_API int ovref_ovw1_count(void* h) {
  return static_cast<int>(static_cast<ov::WeightFile*>(h)->tensors().size());
}
REF_API int ovref_ovw1_get(void* h, const char* name, int* dtype, int* ndim, int64_t* dims,
                           int* transposed, int* quantized, const void** data, int64_t* nbytes,
                           const float** scales, int64_t* n_scales, uint32_t* stored_crc,
                           uint32_t* computed_crc) {
  const auto* wf = static_cast<ov::WeightFile*>(h);
  const ov::Tensor* t = wf->Find(name);
  if (!t) return -1;
  *dtype = static_cast<int>(t->dtype);
  *ndim = t->shape.ndim;
  for (int k = 0; k < 4; ++k) dims[k] = t->shape.dims[k];
  *transposed = t->transposed ? 1 : 0;
  *quantized = t->quantized ? 1 : 0;
  *data = t->data;
  *nbytes = t->nbytes;
  *scales = t->scales;
  *n_scales = t->n_scales;
  *stored_crc = wf->StoredCrc(*t);
  *computed_crc = wf->ComputeCrc(*t);
  return 0;
}

// The reference LM (cpp/src/model/lm.cpp) over an OVW1 file: LM::forward and
// LM::forward_cfg on the host, for the LM parity pin and the CPU baseline.
struct RefLm {
  ov::WeightFile wf;
  ov::LM lm;
  RefLm(ov::WeightFile&& w, const ov::LMConfig& c) : wf(std::move(w)), lm(wf, c) {}
};
REF_API void* ovref_lm_open(const char* path, int n_layers, int hidden, int n_heads,
                            int n_kv_heads, int head_dim, int inter, int vocab, int audio_vocab,
                            int n_codebooks, float rms_eps, float rope_theta, char* err,
                            size_t n) {
  try {
    ov::LMConfig c;
    c.n_layers = n_layers; c.hidden = hidden; c.n_heads = n_heads; c.n_kv_heads = n_kv_heads;
    c.head_dim = head_dim; c.inter = inter; c.vocab = vocab; c.audio_vocab = audio_vocab;
    c.n_codebooks = n_codebooks; c.rms_eps = rms_eps; c.rope_theta = rope_theta;
    return new RefLm(ov::WeightFile::Open(path), c);
  } catch (const std::exception& e) {
    if (err && n) std::snprintf(err, n, "%s", e.what());
    return nullptr;
  }
}
REF_API void ovref_lm_close(void* h) { delete static_cast<RefLm*>(h); }
REF_API int ovref_lm_forward(void* h, int batch, int seq, const int64_t* ids, const uint8_t* amask,
                             const uint8_t* attn, const int64_t* pos, float* logits) {
  try {
    static_cast<RefLm*>(h)->lm.forward(batch, seq, ids, amask, attn, pos, logits);
    return 0;
  } catch (const std::exception&) { return -1; }
}
REF_API int ovref_lm_forward_cfg(void* h, int cond_seq, int uncond_seq, const int64_t* ids,
                                 const uint8_t* amask, const uint8_t* cond_attn,
                                 const uint8_t* uncond_attn, const int64_t* pos, float* logits) {
  try {
    static_cast<RefLm*>(h)->lm.forward_cfg(cond_seq, uncond_seq, ids, amask, cond_attn,
                                           uncond_attn, pos, logits);
    return 0;
  } catch (const std::exception&) { return -1; }
}
