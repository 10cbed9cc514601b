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
// (act_index; rows up to a multiple of 128 readable) when a_tiled.
int linear_q(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w, float* C,
             int64_t ldc, int accumulate, hipStream_t st, bool a_tiled);
int linear_q_sliced(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w,
                    const int64_t* slice_n, float* const* slice_c, int n_slices, hipStream_t st,
                    bool a_tiled);
// fp32 weight from host memory, OVW1 layout 0 ([N,K]) or 1 ([K,N])
int weight_upload_f32(int64_t N, int64_t K, const float* w, int layout, hipStream_t st,
                      OvhWeight** out);
}  // namespace ovh
