/* ovnative_amd.h — C ABI of the MI355X (gfx950) int8-nk quantized-linear path.
 *
 * This is the drop-in boundary for OVNative's quantized linear layers.  Each
 * entry point replaces one function of the reference's CPU operator API
 * (cpp/include/ovnative/ov_gemm.h, namespace ov) with the same argument
 * meaning, except that every buffer is DEVICE memory and every call is
 * enqueued on a caller-supplied HIP stream (`stream` = hipStream_t, NULL for
 * the null stream).  Calls are asynchronous with respect to the host.
 *
 * Status codes are the reference C ABI's (cpp/include/ovnative/ovnative.h:18-23).
 * Errors never throw across this boundary; a failing call returns a negative
 * status and leaves a message for ovh_last_error() on the calling thread.
 * Degenerate sizes (M, N or K <= 0) return OV_OK without doing anything, as the
 * reference does (cpp/src/backend/cpu/gemm.cpp:761).
 *
 * Activation format on the device.  The reference quantises activations per
 * row and 32-k block to u8 = q + 128 (cpp/src/backend/cpu/gemm.cpp:379-430).
 * Here the same q is stored signed: aq is int8 [M, Kp], Kp = 32*ceil(K/32),
 * with aq_s8 = aq_u8 - 128 for every real k and 0 in the K-tail padding (the
 * reference pads u8 with 0; the matching weight bytes are 0 either way), and
 * asc is fp32 [M, ceil(K/32)], identical to the reference's scales.
 *
 * Weight format on the device.  OVW1 int8 weights carry one fp32 scale per
 * output channel (tools/convert_weights.py:130-135).  ovh_weight_upload() takes
 * either OVW1 layout (0 = [N, K] "nk", 1 = [K, N] "kn"; the integers and scales
 * are the same, cpp/src/model/mat.cpp:69-106) and builds the device layout the
 * kernels read; the handle owns that memory.
 *
 * Threading: a handle may be used from any thread; calls that write the same
 * output buffer must be ordered by the caller (same stream), as with the
 * reference's synchronous API.
 */
#ifndef OVNATIVE_AMD_H
#define OVNATIVE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__) || defined(__clang__)
#pragma GCC visibility push(default)
#endif

#define OVH_ABI_VERSION 1

/* Status codes: same values as cpp/include/ovnative/ovnative.h:18-23. */
#ifndef OV_OK
#define OV_OK 0
#define OV_ERR_INVALID_ARG (-1)
#define OV_ERR_IO (-2)
#define OV_ERR_NOT_IMPLEMENTED (-3)
#define OV_ERR_INTERNAL (-4)
#endif

typedef struct OvhWeight OvhWeight;

/* Message of the last failing call on this thread ("" if none). */
const char* ovh_last_error(void);
/* The same message into a caller-owned buffer, the reference's C ABI
 * convention (`char* err, size_t err_len` of ov_engine_create / ov_tts,
 * cpp/include/ovnative/ovnative.h:42-57): at most err_len - 1 bytes and a NUL
 * (nothing when err is NULL or err_len is 0); returns the message's full
 * length, so a caller can tell it was truncated. */
size_t ovh_copy_last_error(char* err, size_t err_len);

/* ABI version and the device the library runs on, e.g. "hip:gfx950 (256 CUs)".
 * Plays the role of ov_engine_backend() (cpp/include/ovnative/ovnative.h:49)
 * and cpu_kernel_name() (cpp/include/ovnative/ov_gemm.h:122). */
int ovh_abi_version(void);
int ovh_backend_name(char* buf, size_t len);

/* Activation buffer sizes; replace s8_nk_quant_bytes / s8_nk_quant_scales
 * (cpp/include/ovnative/ov_gemm.h:95-96, gemm.cpp:623-631). */
int64_t ovh_quant_bytes(int64_t M, int64_t K);
int64_t ovh_quant_scales(int64_t M, int64_t K);

/* ---- weights --------------------------------------------------------------
 * Replaces the load-time repack s8_nk_pack (ov_gemm.h:60-63, gemm.cpp:584-621)
 * and make_linear's layout dispatch (mat.cpp:69-106).  `q` is int8 in OVW1
 * layout `layout` (0: [N,K], 1: [K,N]); `scale` has N floats.  Host pointers
 * for ovh_weight_upload, device pointers for ovh_weight_from_device.  The
 * handle's memory is allocated here and freed by ovh_weight_free. */
int ovh_weight_upload(int64_t N, int64_t K, const int8_t* q, const float* scale, int layout,
                      void* stream, OvhWeight** out);
int ovh_weight_from_device(int64_t N, int64_t K, const int8_t* q, const float* scale,
                           int layout, void* stream, OvhWeight** out);
/* Concatenate weights with equal K along N (q/k/v -> qkv, gate/up -> gate_up);
 * replaces combine_packed (cpp/src/model/lm.cpp:57-94).  Each part's N must be
 * a positive multiple of 64, as the reference requires. */
int ovh_weight_concat(const OvhWeight* const* parts, int n_parts, void* stream, OvhWeight** out);
void ovh_weight_free(OvhWeight* w);
int64_t ovh_weight_n(const OvhWeight* w);
int64_t ovh_weight_k(const OvhWeight* w);
/* Copy the weight back as OVW1 layout-0 int8 [N,K] + fp32 scales (device
 * pointers); used by tests to prove the layout transform is lossless. */
int ovh_weight_download(const OvhWeight* w, int8_t* q_nk, float* scale, void* stream);

/* ---- activation quantisers ------------------------------------------------ */
/* s8_nk_quantize (ov_gemm.h:97, gemm.cpp:709-720 -> quantize_a_u8 :379-430).
 * A fp32 [M,K] -> aq int8 [M,Kp], asc fp32 [M,Kb]. */
int ovh_s8_nk_quantize(int64_t M, int64_t K, const float* A, int8_t* aq, float* asc,
                       void* stream);
/* rmsnorm_quantize_f32 (ov_gemm.h:118-119, gemm.cpp:722-756 -> :638-707):
 * xn = (x * 1/sqrt(mean(x^2)+eps)) * w, quantised without materialising xn. */
int ovh_rmsnorm_quantize(int64_t rows, int64_t cols, const float* x, const float* w, float eps,
                         int8_t* aq, float* asc, void* stream);
/* silu_mul_quantize_f32 (ov_gemm.h:84-85, ops_cpu.cpp:1138-1168 -> :144-198):
 * silu(gate)*up quantised per 32-k block. */
int ovh_silu_mul_quantize(int64_t M, int64_t K, const float* gate, const float* up, int8_t* aq,
                          float* asc, void* stream);

/* ---- GEMM ------------------------------------------------------------------
 * C[m, n] = wscale[n] * sum_b fma-chain(float(acc_b[m,n]) * asc[m,b]) with
 * acc_b the exact int32 dot product of block b; bit-identical to the reference's
 * epilogue (gemm.cpp:469-502).  C has leading dimension ldc >= N.  The codes
 * aq and the block scales asc are device pointers aligned to 16 bytes (the
 * kernels move them by 16-byte DMA; OV_ERR_INVALID_ARG otherwise), as every
 * allocation of the device allocator is.
 *
 * linear_s8_nk_packed_q (ov_gemm.h:98-100, gemm.cpp:758-774): accumulate = 0.
 * linear_s8_nk_packed_q_add (ov_gemm.h:78-80, gemm.cpp:847-862): accumulate = 1,
 * C = C + P with P rounded first (the reference's "keep mul/add separate"). */
int ovh_linear_q(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w, float* C,
                 int64_t ldc, int accumulate, void* stream);
/* ovh_linear_q with the codes aq tile-major (the LM runner's layout, described
 * at ovh_block_dots_tiled; a buffer of ovh_tiled_codes_bytes(M, K)); the same
 * results bit for bit.  K must be a multiple of 128.  No reference counterpart
 * (layout of this library); it runs the GEMM the way the runner does. */
int ovh_linear_q_tiled(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w,
                       float* C, int64_t ldc, int accumulate, void* stream);
/* The residual projection and the RMSNorm + quantise that follows it, in one
 * launch: x [M][ldx] += P as ovh_linear_q_tiled with accumulate = 1 (codes aq
 * tile-major; lm.cpp:281 o_proj mul_add, lm.cpp:311 down mul_q_add), then
 * rmsnorm_quantize_f32 of the updated rows (lm.cpp:292 and :232,
 * gemm.cpp:638-707) with weight nw into codes nq (tile-major,
 * ovh_tiled_codes_bytes(M, N)) and scales nsc [M][N / 32]; x, nq and nsc hold
 * the bits of those two calls.  N = 256 P with P <= 4, K a multiple of 128.
 * band_cnt: ovh_band_counter_bytes(R) of device memory, R >= M, zeroed by
 * the caller before its first use, then passed unchanged to every later call
 * on that device (each launch moves its counters on to the next launch
 * boundary, whatever its N); calls sharing one run in stream order.  Its first
 * 4 bytes turn non-zero if the row bands' hand-off failed: bit 1 (value 2) a
 * workgroup's wait for the rest of its band ran out (only possible when other
 * work keeps the device from holding the band's workgroups) or a counter was
 * not at a launch boundary; bit 2 (value 4) a workgroup ran on another XCD
 * than its band's.  The outputs of that call are then not to be used (the
 * same result comes from ovh_linear_q_tiled + ovh_rmsnorm_quantize).  Needs a
 * device of 8 XCDs (MI355X), else OV_ERR_NOT_IMPLEMENTED.  No reference
 * counterpart as one call (the LM runner's o_proj / down launch). */
int ovh_linear_q_norm(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w, float* x,
                      int64_t ldx, const float* nw, float eps, int8_t* nq, float* nsc,
                      void* band_cnt, void* stream);
int64_t ovh_band_counter_bytes(int64_t max_rows);
/* linear_s8_nk_packed_q_sliced (ov_gemm.h:105-111, gemm.cpp:776-827): one launch
 * over a concatenated weight, slice s (N = slice_n[s], a positive multiple of
 * 64, summing to the weight's N) written to slice_c[s] with leading dimension
 * slice_n[s].  Invalid slices -> OV_ERR_INVALID_ARG (the reference throws
 * std::invalid_argument). */
int ovh_linear_q_sliced(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w,
                        const int64_t* slice_n, float* const* slice_c, int n_slices,
                        void* stream);
/* One launch over up to 8 independent ovh_linear_q problems (each its own
 * codes, scales, weight, output and M; all in the store form, or all in the
 * residual form: accumulate applies to every member).  No counterpart in the
 * reference, which runs such GEMMs one after another
 * (linear_s8_nk_packed_q, gemm.cpp:758-774, one call per projection in
 * lm.cpp:241-311); the results are those of ovh_linear_q bit for bit.  For
 * the skinny shapes (M < 256), where one launch per GEMM leaves most of the
 * GPU waiting on launch latency instead of streaming weights.  Every member's
 * K must be a multiple of 128 (OV_ERR_NOT_IMPLEMENTED otherwise).  When every
 * member has M <= 128 and K of 1024, 2048 or 3072, with codes and scales
 * 16-byte aligned, the launch stages each member's activation rows in LDS once
 * and streams the weights straight into registers (same bits). */
typedef struct OvhGemmGroup {
  int64_t M;
  const int8_t* aq;  /* row-major codes [M][Kp] */
  const float* asc;  /* [M][Kb] */
  const OvhWeight* w;
  float* C;          /* [M][ldc] */
  int64_t ldc;
} OvhGemmGroup;
int ovh_linear_q_grouped(const OvhGemmGroup* groups, int n_groups, int accumulate, void* stream);
/* linear_s8_nk_packed / _packed_add (ov_gemm.h:67-75, gemm.cpp:829-845, :864-882):
 * quantise A (fp32 [M,K]) into a library-owned workspace, then ovh_linear_q. */
int ovh_linear(int64_t M, const float* A, const OvhWeight* w, float* C, int64_t ldc,
               int accumulate, void* stream);
/* The f16-operand GEMM form: no counterpart in the reference (a choice of
 * matrix-core instruction inside this library).  From `rows` rows on (0, the
 * default: never) the int8 GEMMs (ovh_linear_q, _tiled, _sliced, ovh_linear,
 * ovh_silu_gate_linear and the LM runner's projections; not
 * ovh_linear_noalloc) run V_MFMA_F32_16X16X32_F16 on int8-valued f16 copies
 * of the weights and codes: its fp32 block products are the int32 dots
 * exactly, so the results are the same bit for bit.  Costs a 2-byte-per-element
 * f16 copy of each weight (made on its first such call outside graph capture)
 * and a widened copy of the codes per call.  Process-wide; returns the
 * previous setting (negative rows: unchanged, a query). */
int64_t ovh_set_f16_min_rows(int64_t rows);
/* The split-f16 attention's two kernels (ovh_attention_split and the LM
 * runner): from `tasks` long-form workgroups on (segments x KV heads x 128-row
 * query tiles; default 384, 0 = whenever 4 % (n_heads / n_kv_heads) == 0) the
 * long-sequence kernel, which shares each key block through LDS, else the
 * short one, which splits the keys over four wavefronts and merges.  Both are
 * within the operator's tolerance of the reference; they sum in another
 * order, so a batch and its requests run alone give the same bits only when
 * they take the same kernel.  No reference counterpart (the CUDA runner picks
 * its attention kernel from the sequence length, cuda_lm.cu:1106-1115).
 * Process-wide; returns the previous setting (negative: unchanged, a query). */
int64_t ovh_set_attention_long_min_tasks(int64_t tasks);
/* ovh_linear without any allocation: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The codes and scales
 * go to a fixed 16 MiB device array per GPU (held from the first call on that
 * GPU until the process ends), so M * (Kp + 4 * Kb) plus up to 255 bytes of
 * alignment must fit in 16 MiB (M <= 14563 at K = 1024, M <= 4854 at
 * K = 3072); larger calls return OV_ERR_INVALID_ARG.  Every call on one GPU
 * shares that array: calls that overlap on one GPU (other streams, other
 * threads) race; order them on one stream.  Same results, bit for bit, as
 * ovh_linear. */
int ovh_linear_noalloc(int64_t M, const float* A, const OvhWeight* w, float* C, int64_t ldc,
                       int accumulate, void* stream);

/* ---- fp32 linear (Mat's fp32 branch) ----------------------------------------
 * Mat::mul / mul_add on an fp32 weight (cpp/src/model/mat.cpp:11-13, :40-42 ->
 * linear_f32_ld, cpp/src/backend/cpu/gemm.cpp:884-905): C = A W (accumulate 0)
 * or C = C + A W (accumulate 1, the sum rounded separately), A fp32 [M, K], W
 * fp32 [K, N].  The reference's default int8 checkpoint keeps the audio head
 * in this form (tools/convert_weights.py --int8-keep audio_heads).  Computed on
 * the f16 matrix cores from hi/lo splits of power-of-two-scaled operands
 * (hi*hi + hi*lo + lo*hi, fp32 sums): not the reference's bits (its fma chain
 * over k), a few fp32 ulps of sum_k |A W| from them.  The weight is uploaded
 * once from host memory, OVW1 layout 0 ([N, K]) or 1 ([K, N], the reference's
 * fp32 encoding); ovh_linear_f32 allocates its split activations stream-ordered. */
int ovh_weight_upload_f32(int64_t N, int64_t K, const float* w, int layout, void* stream,
                          OvhWeight** out);
int ovh_weight_is_f32(const OvhWeight* w);
int ovh_linear_f32(int64_t M, const float* A, const OvhWeight* w, float* C, int64_t ldc,
                   int accumulate, void* stream);

/* Debug: the exact int32 dot product of every (m, n, block); out is int32
 * [M, N, Kb].  The reference keeps these in registers (gemm.cpp:455-474); this
 * exposes them for the bit-exactness check.  They come from the kernel and
 * tile that ovh_linear_q launches for the same M and weight (same DMA ring,
 * fragment reads and block products; the per-block values are written out
 * where ovh_linear_q folds them into the fp32 chain). */
int ovh_block_dots(int64_t M, const int8_t* aq, const OvhWeight* w, int32_t* out, void* stream);
/* The same with the codes tile-major, the layout the LM runner keeps its
 * activation codes in: 1 KiB tiles of 32 rows x 32 k, row tile major then
 * k block; inside a tile byte (m/16 % 2)*512 + (k/8 % 4)*128 + (m % 16)*8 +
 * k % 8; rows padded to a multiple of 128 (ovh_tiled_codes_bytes).  K must be
 * a multiple of 128.  No reference counterpart (layout of this library). */
int ovh_block_dots_tiled(int64_t M, const int8_t* aq, const OvhWeight* w, int32_t* out,
                         void* stream);
int64_t ovh_tiled_codes_bytes(int64_t M, int64_t K);

/* Diagnostics, no reference counterpart: read `bytes` of device memory at src
 * once (bytes a positive multiple of 128 KiB) through one load path of the
 * GEMM kernels: 0 DMA into LDS, 16 bytes a lane (the tiles of the 16x16
 * kernels); 1 DMA into LDS, 4 bytes a lane; 2 16-byte vector loads; 3 8-byte
 * buffer loads (the weight stream of the skinny grouped kernel).  Nothing is
 * written.  For calibrating hardware byte counters (FETCH_SIZE) against a
 * known byte count on exactly the paths the GEMMs use. */
int ovh_diag_read(const void* src, int64_t bytes, int path, void* stream);

/* ---- SiLU-gated MLP input ---------------------------------------------------
 * The reference composes gate/up -> silu*up -> quantise for the down
 * projection (cpp/src/model/lm.cpp:293-311: linear_s8_nk_packed_q_sliced over
 * the merged gate/up, then silu_mul_quantize_f32, ops_cpu.cpp:1138-1168).
 * Here it is one GEMM whose epilogue forms gate and up (the fp32 values the
 * sliced GEMM would store), silu(gate)*up with the reference's exp256 lane
 * arithmetic, and its per-32-column block quantisation: hq int8 [M, I] and
 * hsc fp32 [M, I/32] are byte-identical to silu_mul_quantize_f32's output
 * (as signed codes, see above) for the same inputs.
 *
 * ovh_weight_gate_up builds the operand from gate and up weights [I, K] (I a
 * multiple of 64; rows interleaved in 16-row groups); that handle is only
 * accepted by ovh_silu_gate_linear.  K must be a multiple of 128
 * (OV_ERR_NOT_IMPLEMENTED otherwise). */
int ovh_weight_gate_up(const OvhWeight* gate, const OvhWeight* up, void* stream, OvhWeight** out);
int ovh_silu_gate_linear(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* gate_up,
                         int8_t* hq, float* hsc, void* stream);

/* ---- attention side of a decoder layer (fp32) ------------------------------- */

/* One attention segment: `rows` query rows starting at element offset q_off of
 * q and out, attending to the `rows` keys at element offset kv_off of k and v,
 * with an optional additive bias [rows, rows] (device; NULL = none).  Same
 * fields and meaning as ov::AttnSegment (cpp/src/model/lm.h:42-51). */
typedef struct OvhAttnSegment {
  const float* bias;
  int32_t rows;
  int64_t q_off;
  int64_t kv_off;
} OvhAttnSegment;

/* RoPE cos/sin tables [rows, head_dim/2] from device int64 positions, as
 * qk_norm_rope_f32 builds them (ops_cpu.cpp:958-993): inv_freq = (float)
 * pow(theta, -2i/D) in double, angle = (float)pos * inv_freq.  cos/sin are
 * correctly rounded (libm's cosf/sinf are within one ulp of them). */
int ovh_rope_tables(int64_t rows, const int64_t* pos, int head_dim, float theta, float* cos_tab,
                    float* sin_tab, void* stream);
/* qk_norm_rope_f32 (ops.h, ops_cpu.cpp:945-1016 -> :266-318): per-head RMSNorm
 * (weights qw / kw [head_dim]) then RoPE, in place on q [rows, n_heads*D] and
 * k [rows, n_kv_heads*D], with the tables of ovh_rope_tables.  Bit-identical
 * to the reference for the same tables.  head_dim 64 or 128. */
int ovh_qk_norm_rope(float* q, float* k, const float* qw, const float* kw, int64_t rows,
                     int n_heads, int n_kv_heads, int head_dim, const float* cos_tab,
                     const float* sin_tab, float eps, void* stream);
/* The attention loop of LM::run_layer (lm.cpp:259-276) over attention_head_f32
 * (ops.h, ops_cpu.cpp:907-943): for each segment and query head h (KV head
 * h / (n_heads / n_kv_heads)), out = softmax(q k^T * scale + bias) v in fp32,
 * zeros for a fully masked row (max < -1e29).  q/out rows have stride q_stride
 * / out_stride, k/v rows kv_stride (elements).  head_dim 128.  segs is HOST
 * memory (any count; launched 32 segments at a time). */
int ovh_attention(const OvhAttnSegment* segs, int n_segs, int n_heads, int n_kv_heads,
                  int head_dim, const float* q, int64_t q_stride, const float* k, const float* v,
                  int64_t kv_stride, float scale, float* out, int64_t out_stride, void* stream);
/* The same attention with the products split into f16 hi/lo parts on the f16
 * matrix core (hi*hi + hi*lo + lo*hi, ~2^-22 relative; 5x less matrix-core
 * time than the fp32 form).  No reference counterpart beyond ovh_attention's.
 * |k| and |v| must stay below 65504 (OV_ERR_INVALID_ARG otherwise); strides a
 * multiple of 8, kv_off a whole number of rows, at most 32 segments.  Allocates
 * its split workspace stream-ordered and synchronises the stream. */
int ovh_attention_split(const OvhAttnSegment* segs, int n_segs, int n_heads, int n_kv_heads,
                        int head_dim, const float* q, int64_t q_stride, const float* k,
                        const float* v, int64_t kv_stride, float scale, float* out,
                        int64_t out_stride, void* stream);

/* ---- weights: OVW1 files -------------------------------------------------- */

/* A tensor of a checkpoint: same fields as ov::Tensor
 * (cpp/include/ovnative/ov_types.h).  dtype: 0 f32, 1 i8, 2 f16, 3 i64 (ov::DType);
 * transposed = OVW1 layout 1 (2-D linear weight stored [in, out]); quantized =
 * per-output-channel int8 with n_scales fp32 scales.  data/scales are HOST memory. */
typedef struct OvhTensorView {
  const char* name;
  int32_t dtype;
  int32_t ndim;
  int64_t dims[4];
  int32_t transposed;
  int32_t quantized;
  const void* data;
  int64_t nbytes;
  const float* scales;
  int64_t n_scales;
  uint32_t crc;
} OvhTensorView;

typedef struct OvhWeightFile OvhWeightFile;

/* WeightFile::Open (ov_weights.h:29, weight_file.cpp): mmap an OVW1 file and
 * check it the way the reference loader does (magic, version, file size, index,
 * names, payload and scale bounds, byte size = shape x dtype).  Format errors
 * return OV_ERR_IO (the reference throws std::runtime_error). */
int ovh_ovw1_open(const char* path, OvhWeightFile** out);
void ovh_ovw1_close(OvhWeightFile* wf);
/* tensors() / Find() / n_params() (ov_weights.h:36-43); views live until close. */
int ovh_ovw1_count(const OvhWeightFile* wf);
const OvhTensorView* ovh_ovw1_tensors(const OvhWeightFile* wf);
const OvhTensorView* ovh_ovw1_find(const OvhWeightFile* wf, const char* name);
uint64_t ovh_ovw1_n_params(const OvhWeightFile* wf);
/* ComputeCrc (ov_weights.h:45): CRC-32 of tensor `index`'s payload, to compare
 * with the stored OvhTensorView.crc. */
uint32_t ovh_ovw1_compute_crc(const OvhWeightFile* wf, int index);

/* ---- LM runner: the accelerator plugin of cpp/src/backend/cuda/cuda_lm.h ------ */

/* ov::LMConfig (cpp/src/model/lm.h:17-29). */
typedef struct OvhLmConfig {
  int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, inter, vocab, audio_vocab,
      n_codebooks;
  float rms_eps, rope_theta;
} OvhLmConfig;

typedef struct OvhLm OvhLm;

/* LmRunnerCreate (cuda_lm.h:31): uploads the LM's tensors (the reference's names,
 * lm.cpp:96-149) and merges q/k/v and gate/up.  Linear weights must be int8 with
 * per-channel scales, OVW1 layout 0 or 1; embeddings fp32 or int8.  All work is
 * enqueued on `stream` (hipStream_t), which the runner keeps using.  Returns
 * OV_ERR_NOT_IMPLEMENTED for configurations the HIP kernels do not cover (the
 * reference's factory returns null and the caller stays on the CPU). */
int ovh_lm_create(const OvhLmConfig* cfg, const OvhTensorView* tensors, int n_tensors,
                  void* stream, OvhLm** out);
/* LmRunnerDelete. */
void ovh_lm_destroy(OvhLm* lm);
/* LmRunnerForward / LmRunnerForwardThunk (cuda_lm.h:34-36, :50-52) = LM::forward
 * (lm.h:65-73): host inputs ids [B, 8, S] int64, audio_mask [B, S], attn_mask
 * [B, S, S] (1 = attend), position_ids [B, S]; logits host [B, C, S, V], or NULL
 * (or device sampling on) to leave them on the device only. */
int ovh_lm_forward(OvhLm* lm, int batch, int seq, const int64_t* input_ids,
                   const uint8_t* audio_mask, const uint8_t* attn_mask,
                   const int64_t* position_ids, float* logits);
/* LM::forward_cfg (lm.h:75-82): ragged CFG batch, cond_seq rows then uncond_seq
 * rows; ids [C, rows] codebook-major, logits host [rows, C*V] token-major (or NULL). */
int ovh_lm_forward_cfg(OvhLm* lm, int cond_seq, int uncond_seq, const int64_t* input_ids,
                       const uint8_t* audio_mask, const uint8_t* cond_attn,
                       const uint8_t* uncond_attn, const int64_t* position_ids, float* logits);
/* LmRunnerLastLogitsThunk (cuda_lm.h:42): device logits [rows, C*V] of the last forward. */
const void* ovh_lm_last_logits(const OvhLm* lm);
/* LmRunnerSetDeviceSampling (cuda_lm.h:46). */
void ovh_lm_set_device_sampling(OvhLm* lm, int on);
/* Attention kernel of the runner: 1 = split-f16 products (default), 0 = fp32
 * products.  No reference counterpart (the CUDA runner picks its attention
 * kernel from the sequence length and environment variables, cuda_lm.cu:1106-1115). */
void ovh_lm_set_attention(OvhLm* lm, int split_f16);
/* Forward launches: 1 = captured once per layout into a HIP graph and replayed
 * (default), 0 = launched one by one.  Both give the same bits.  No reference
 * counterpart (the CUDA runner launches its kernels one by one). */
void ovh_lm_set_graphs(OvhLm* lm, int on);
/* o_proj and down with the RMSNorm + quantise that follows each of them in the
 * same launch: 1 = where the layout allows it (default; below 2048 rows, int8
 * GEMM form, tile-major codes), 0 = the norm as a launch of its own.  Both give
 * the same bits.  No reference counterpart (lm.cpp:339-401 runs the norm as a
 * step of its own). */
void ovh_lm_set_fused_norm(OvhLm* lm, int on);
/* L2 prefetch of o_proj's weight: 1 = the attention launch carries workgroups
 * that load it into the L2 of every XCD that reads it, below 2048 rows and
 * where they fit beside the attention's own workgroups (default), 0 = off.
 * Nothing is written: both give the same bits.  No reference counterpart. */
void ovh_lm_set_prefetch(OvhLm* lm, int on);
/* LmRunnerSampleThunk (cuda_lm.h:39-41): the per-step guidance + argmax pass
 * (tts.cpp:296-326) on device logit planes; pred/scores host [C, target_len]. */
int ovh_lm_sample(OvhLm* lm, const void* cond, int cond_seq, const void* uncond, int uncond_seq,
                  int target_len, float guidance, float layer_penalty, int32_t* pred,
                  float* scores);
/* In-runner recovery, as the CUDA runner's forward falls back to its cuBLAS
 * path when the fused attention cannot run (cuda_lm.cu:586-606, :620-622).
 * Two conditions that only a finished forward shows make the default kernels'
 * results unusable: |k| or |v| beyond the f16 range of the split-f16
 * attention, and a fused residual + norm launch whose row-band hand-off failed
 * (ovh_linear_q_norm's error bits).  Wherever the runner synchronises with the
 * host (ovh_lm_forward with host logits, ovh_lm_forward_cfg, ovh_lm_sample on
 * the last forward's own logits, hence every step of ovh_lm_generate) it
 * checks for them, runs that forward again on the exact fallback (the fp32
 * attention form, the norm as a launch of its own: the bits those settings
 * give when chosen from the start), keeps the fallback for later forwards,
 * and returns OV_OK.  ovh_lm_recovered: the fallbacks taken so far, a mask of
 * OVH_LM_RECOVERED_*.  No reference counterpart as a call. */
#define OVH_LM_RECOVERED_ATTENTION 1
#define OVH_LM_RECOVERED_NORM 2
int ovh_lm_recovered(const OvhLm* lm);
/* The conditions behind the last recovery (0 if none): bit 0 (value 1) the
 * attention's inputs beyond f16, bit 1 (2) a band's hand-off wait ran out or
 * its counter was off a launch boundary, bit 2 (4) a workgroup of the fused
 * norm launch on another XCD than its band's. */
int ovh_lm_last_flags(const OvhLm* lm);
/* Test support: force a condition the recovery handles on the next forward,
 * from the host, with every kernel still ending normally.
 * OVH_LM_FORCE_BAND_WAIT puts the first row band's counter off its launch
 * boundary (the hand-off reports it, and that band's bounded waits run out);
 * OVH_LM_FORCE_XCD makes every fused launch's XCD placement check fail.
 * No reference counterpart. */
#define OVH_LM_FORCE_BAND_WAIT 1
#define OVH_LM_FORCE_XCD 2
void ovh_lm_force_condition(OvhLm* lm, int what);
/* Stage timer, as the reference's OV_CUDA_PROFILE events (cuda_lm.cu:994-1022,
 * :1036-1197): with on = 1 each forward launches its kernels one by one with
 * HIP events between the stages and waits for them; ovh_lm_stage_times then
 * gives the last forward's milliseconds per stage, summed over the layers
 * (ms[i], i < n), and the stage labels (names[i] if names is not NULL), and
 * returns the number of stages.  Stages: "prep+embed" (input upload, masks,
 * embedding), "qkv" (the q/k/v GEMM with qk-norm and RoPE), "attn", "o_proj"
 * (with the norm after it when fused), "gate_up" (with SiLU), "down" (with
 * the next norm when fused), "final_norm+head"; a norm that runs as a launch
 * of its own counts with the stage after it, as in the reference.  The
 * environment variable OVH_LM_PROFILE, set when the runner is created, turns
 * it on and prints one "[hip-stage]" line per forward to stderr. */
void ovh_lm_set_profile(OvhLm* lm, int on);
int ovh_lm_stage_times(const OvhLm* lm, double* ms, const char** names, int n);

/* ---- the CFG decoding loop ----------------------------------------------- */

/* The sampling fields of TtsOptions (cpp/src/model/tts.h:26-36); the reference's
 * defaults are 32, 2.0, 0.1, 5.0, 5.0, 1234. */
typedef struct OvhGenOptions {
  int32_t num_steps;
  float guidance_scale, t_shift, layer_penalty, position_temperature;
  uint32_t seed;
} OvhGenOptions;

/* Pipeline::run_sampling (cpp/src/model/tts.cpp:165-364) on the accelerator
 * branch: the B = 2 CFG batch, `num_steps` forwards with device guided
 * sampling, Gumbel position noise from std::mt19937(seed), top-k unmasking.
 * prompt_ids [C, seq] and prompt_audio_mask [seq] as Pipeline::build_prompt
 * makes them (the last target_len positions hold the mask token); tokens out
 * [C, target_len], host memory.  Uses the runner's stream; synchronous. */
int ovh_lm_generate(OvhLm* lm, const int64_t* prompt_ids, const uint8_t* prompt_audio_mask,
                    int seq, int target_len, const OvhGenOptions* opt, int64_t* tokens);

#if defined(__GNUC__) || defined(__clang__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif

#endif /* OVNATIVE_AMD_H */
