// The device weight behind the ABI's opaque OvhWeight handle, and the
// library-internal weight transforms the runner uses.
#pragma once

#include <hip/hip_runtime.h>

#include "gemm.h"

struct OvhWeight {
  ovh::DeviceWeight w;
  // rows interleaved gate/up in 16-row groups (weight_interleave16): only the
  // SiLU-fused operator takes such a weight
  bool silu_pair = false;
  // an fp32 weight (ovh_weight_upload_f32): f16 planes in fw, w unused except
  // for N and K; only ovh_linear_f32 takes it
  bool f32 = false;
  ovh::F32Weight fw;
};

namespace ovh {
// gate [I, K] and up [I, K] (I % 64 == 0) -> one weight of 2I rows in which
// 32-row block tile c holds gate rows 16c..16c+15 then up rows 16c..16c+15
// (scales alike): the operand of the SiLU-fused GEMM mode.
int weight_interleave16(const OvhWeight* gate, const OvhWeight* up, hipStream_t st,
                        OvhWeight** out);
// ovh_linear_q / ovh_linear_q_sliced, with the codes aq tile-major
// (act_index; rows up to a multiple of 128 readable) when a_tiled.  From
// f16_min_rows() rows (when set; K a multiple of 128) they run the f16-operand
// GEMM form:
// the codes are widened into f16_codes when given (2 x ovh_tiled_codes_bytes),
// else into a stream-ordered allocation.  f16_ok = false keeps the int8 form.
int linear_q(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w, float* C,
             int64_t ldc, int accumulate, hipStream_t st, bool a_tiled,
             _Float16* f16_codes = nullptr, bool f16_ok = true);
int linear_q_sliced(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w,
                    const int64_t* slice_n, float* const* slice_c, int n_slices, hipStream_t st,
                    bool a_tiled, _Float16* f16_codes = nullptr, bool f16_ok = true);
// x [M][ldx] += linear_q(aq, w) (N = w's N, tile-major codes), then
// rmsnorm_quantize of the updated rows with weight nw into codes nq
// (tile-major) and scales nsc, in the same launch (GemmMode kAccumNorm:
// N = 256 P with P <= 4, K a multiple of 128).  band_cnt: the launch's band
// counters (band_counter_words(M) or more, zero when allocated, kept for
// every later launch); err gets kNormErrWait / kNormErrXcd (gemm.h) when the
// band hand-off failed.  xcd_test: GemmArgs::xcd_test (0 in use).
int linear_q_norm(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w, float* x,
                  int64_t ldx, const float* nw, float eps, int8_t* nq, float* nsc,
                  unsigned long long* band_cnt, uint32_t* err, hipStream_t st, int xcd_test = 0);
// The int8-valued f16 copy of w's tiles (DeviceWeight::q16) for the large-M
// GEMM form, made on first call (hipMalloc, widened on st, then st synchronised;
// serialised over threads).  False where it cannot be made now: during graph
// capture on st, or out of device memory; the int8 form then runs.
bool weight_f16(const OvhWeight* w, hipStream_t st);
// fp32 weight from host memory, OVW1 layout 0 ([N,K]) or 1 ([K,N])
int weight_upload_f32(int64_t N, int64_t K, const float* w, int layout, hipStream_t st,
                      OvhWeight** out);
}  // namespace ovh
