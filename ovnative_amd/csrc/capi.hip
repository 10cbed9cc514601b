// extern "C" entry points of libovnative_amd.so (declared in include/ovnative_amd.h).
//
// Argument checking and error reporting follow the reference's operator API
// (cpp/include/ovnative/ov_gemm.h): degenerate sizes are a silent no-op, bad
// slice widths are an invalid argument, and a failure never escapes as an
// exception — it becomes a status code plus a per-thread message.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/ovnative_amd.h"
#include "attn.h"
#include "gemm.h"
#include "ovh_common.h"
#include "quant.h"
#include "status.h"
#include "weight.h"


namespace {
thread_local std::string t_err;
}  // namespace

namespace ovh {
int set_error(int code, const std::string& msg) {
  t_err = msg;
  return code;
}
int hip_error(hipError_t e, const char* what) {
  return set_error(OV_ERR_INTERNAL, std::string(what) + ": " + hipGetErrorString(e));
}
}  // namespace ovh

namespace {

int fail(int code, const std::string& msg) { return ovh::set_error(code, msg); }
int hip_fail(hipError_t e, const char* what) { return ovh::hip_error(e, what); }

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int new_weight(int64_t N, int64_t K, OvhWeight** out) {
  auto* h = new (std::nothrow) OvhWeight();
  if (!h) return fail(OV_ERR_INTERNAL, "out of host memory");
  ovh::DeviceWeight& w = h->w;
  w.N = N;
  w.K = K;
  w.Kb = ovh::kb_of(K);
  w.Kp = w.Kb * 32;
  w.Npad = (N + ovh::kRowPad - 1) / ovh::kRowPad * ovh::kRowPad;
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&w.q), (size_t)(w.Npad * w.Kp));
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&w.scale), sizeof(float) * (size_t)w.Npad);
  if (e != hipSuccess) {
    if (w.q) (void)hipFree(w.q);
    delete h;
    return hip_fail(e, "hipMalloc(weight)");
  }
  *out = h;
  return OV_OK;
}

int check_gemm_operands(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w) {
  if (!w) return fail(OV_ERR_INVALID_ARG, "weight handle is null");
  if (w->silu_pair)
    return fail(OV_ERR_INVALID_ARG, "weight is an interleaved gate/up operand: use "
                                    "ovh_silu_gate_linear");
  if (w->f32) return fail(OV_ERR_INVALID_ARG, "weight is fp32: use ovh_linear_f32");
  if (M > 0x7fffffff || w->w.N > 0x7fffffff)
    return fail(OV_ERR_INVALID_ARG, "M and N must fit in 31 bits");
  if (!aq || !asc) return fail(OV_ERR_INVALID_ARG, "aq/asc must be device pointers");
  if (!aligned16(aq)) return fail(OV_ERR_INVALID_ARG, "aq must be 16-byte aligned");
  if (!aligned16(asc)) return fail(OV_ERR_INVALID_ARG, "asc must be 16-byte aligned");
  return OV_OK;
}

std::mutex g_f16_mu;  // making a weight's f16 copy
std::atomic<int64_t> g_f16_min_rows{0};

// The f16 GEMM form for M rows: the weight's f16 copy (made here on first use)
// and the codes widened to tile-major f16, into f16_codes when given (2 x
// ovh_tiled_codes_bytes), else into *ws from the stream-ordered allocator (the
// caller frees it after the launch).  Leaves a alone where the form does not
// apply (the form off or M below its row threshold, K not a multiple of 128,
// no copy made).
int f16_operands(int64_t M, const int8_t* aq, bool a_tiled, const OvhWeight* w,
                 _Float16* f16_codes, hipStream_t st, ovh::GemmArgs& a, _Float16** ws,
                 bool f16_ok = true) {
  *ws = nullptr;
  const int64_t min_rows = ovh::f16_min_rows();
  if (!f16_ok || min_rows <= 0 || M < min_rows || w->w.Kb % 4 != 0 || !ovh::weight_f16(w, st))
    return OV_OK;
  const int64_t bytes = (M + 127) / 128 * 128 * w->w.Kp;
  _Float16* codes = f16_codes;
  if (!codes) {
    // no stream-ordered allocation into a graph being captured: int8 form
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
      return OV_OK;
    OVH_HIP(hipMallocAsync(reinterpret_cast<void**>(ws), sizeof(_Float16) * (size_t)bytes, st),
            "hipMallocAsync(f16 codes)");
    codes = *ws;
  }
  const hipError_t e = a_tiled ? ovh::launch_widen_f16(aq, codes, bytes, st)
                               : ovh::launch_codes_to_f16_tiled(M, w->w.Kp, aq, codes, st);
  if (e != hipSuccess) {
    if (*ws) (void)hipFreeAsync(*ws, st);
    *ws = nullptr;
    return hip_fail(e, "widen codes to f16");
  }
  a.W16 = w->w.q16;
  a.aq16 = codes;
  a.a_tiled = 1;
  return OV_OK;
}

// Launch, then release the f16 codes workspace (stream order).
int launch_with_ws(const ovh::GemmArgs& a, ovh::GemmMode mode, _Float16* ws, hipStream_t st) {
  const hipError_t e = ovh::launch_gemm(a, mode, st);
  if (ws) (void)hipFreeAsync(ws, st);
  OVH_HIP(e, "gemm launch");
  return OV_OK;
}

ovh::GemmArgs base_args(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w) {
  ovh::GemmArgs a;
  a.M = (int)M;
  a.N = (int)w->w.N;
  a.Kb = (int)w->w.Kb;
  a.Kp = w->w.Kp;
  a.aq = aq;
  a.asc = asc;
  a.W = w->w.q;
  a.ws = w->w.scale;
  return a;
}

}  // namespace

namespace ovh {
int64_t f16_min_rows() { return g_f16_min_rows.load(std::memory_order_relaxed); }
void set_f16_min_rows(int64_t rows) { g_f16_min_rows.store(rows, std::memory_order_relaxed); }

bool weight_f16(const OvhWeight* w, hipStream_t st) {
  if (w->w.q16) return true;
  // not while a graph is being captured: hipMalloc and the synchronisation
  // below are not allowed there (the int8 form runs instead)
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return false;
  std::lock_guard<std::mutex> lock(g_f16_mu);
  if (w->w.q16) return true;
  const int64_t n = w->w.Npad * w->w.Kp;
  _Float16* p = nullptr;
  if (hipMalloc(reinterpret_cast<void**>(&p), sizeof(_Float16) * (size_t)n) != hipSuccess) {
    (void)hipGetLastError();  // out of memory: keep the int8 form
    return false;
  }
  // finished before any stream may read it
  if (launch_widen_f16(w->w.q, p, n, st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess) {
    (void)hipGetLastError();
    (void)hipFree(p);
    return false;
  }
  const_cast<OvhWeight*>(w)->w.q16 = p;
  return true;
}

int weight_interleave16(const OvhWeight* gate, const OvhWeight* up, hipStream_t st,
                        OvhWeight** out) {
  *out = nullptr;
  if (!gate || !up || gate->silu_pair || up->silu_pair || gate->f32 || up->f32 ||
      gate->w.N != up->w.N ||
      gate->w.K != up->w.K || gate->w.N % 64 != 0)
    return fail(OV_ERR_INVALID_ARG, "interleave: gate/up need equal shapes, rows a multiple of 64");
  OvhWeight* h = nullptr;
  const int rc = new_weight(2 * gate->w.N, gate->w.K, &h);
  if (rc != OV_OK) return rc;
  const hipError_t e = launch_weight_interleave16(gate->w, up->w, h->w, st);
  if (e != hipSuccess) {
    ovh_weight_free(h);
    return hip_fail(e, "weight interleave");
  }
  h->silu_pair = true;
  *out = h;
  return OV_OK;
}
}  // namespace ovh

namespace ovh {
int weight_upload_f32(int64_t N, int64_t K, const float* wsrc, int layout, hipStream_t st,
                      OvhWeight** out) {
  *out = nullptr;
  if (N <= 0 || K <= 0) return fail(OV_ERR_INVALID_ARG, "weight dims must be positive");
  if (layout != 0 && layout != 1) return fail(OV_ERR_INVALID_ARG, "layout must be 0 (nk) or 1 (kn)");
  if (!wsrc) return fail(OV_ERR_INVALID_ARG, "weight is null");
  auto* h = new (std::nothrow) OvhWeight();
  if (!h) return fail(OV_ERR_INTERNAL, "out of host memory");
  h->f32 = true;
  h->w.N = N;
  h->w.K = K;
  F32Weight& fw = h->fw;
  fw.N = N;
  fw.K = K;
  fw.Np = (N + 127) / 128 * 128;
  fw.Ks = (K + 15) / 16;
  const size_t plane = sizeof(_Float16) * (size_t)f32_plane_halves(N, K);
  float* staging = nullptr;
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&fw.hi), plane);
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&fw.lo), plane);
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&fw.scale), sizeof(float) * (size_t)fw.Np);
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&staging), sizeof(float) * (size_t)(N * K));
  if (e == hipSuccess)
    e = hipMemcpyAsync(staging, wsrc, sizeof(float) * (size_t)(N * K), hipMemcpyHostToDevice, st);
  if (e == hipSuccess) e = launch_f32_weight(N, K, staging, layout, fw, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);  // staging is freed below
  if (staging) (void)hipFree(staging);
  if (e != hipSuccess) {
    ovh_weight_free(h);
    return hip_fail(e, "fp32 weight upload");
  }
  *out = h;
  return OV_OK;
}

int linear_q(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w, float* C,
             int64_t ldc, int accumulate, hipStream_t st, bool a_tiled, _Float16* f16_codes,
             bool f16_ok) {
  if (M <= 0) return OV_OK;
  int rc = check_gemm_operands(M, aq, asc, w);
  if (rc != OV_OK) return rc;
  if (!C) return fail(OV_ERR_INVALID_ARG, "C is null");
  if (ldc < w->w.N) return fail(OV_ERR_INVALID_ARG, "ldc < N");
  ovh::GemmArgs a = base_args(M, aq, asc, w);
  a.a_tiled = a_tiled;
  a.nslices = 1;
  a.start[0] = 0;
  a.start[1] = (int)w->w.N;
  a.out[0] = C;
  a.ld[0] = ldc;
  _Float16* ws = nullptr;
  if ((rc = f16_operands(M, aq, a_tiled, w, f16_codes, st, a, &ws, f16_ok)) != OV_OK) return rc;
  return launch_with_ws(a, accumulate ? ovh::kAccumulate : ovh::kStore, ws, st);
}

int linear_q_norm(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w, float* x,
                  int64_t ldx, const float* nw, float eps, int8_t* nq, float* nsc,
                  unsigned long long* band_cnt, uint32_t* err, hipStream_t st, int xcd_test) {
  if (M <= 0) return OV_OK;
  int rc = check_gemm_operands(M, aq, asc, w);
  if (rc != OV_OK) return rc;
  if (!x || !nw || !nq || !nsc || !band_cnt || !err)
    return fail(OV_ERR_INVALID_ARG, "residual + norm GEMM: null operand");
  if (ldx < w->w.N) return fail(OV_ERR_INVALID_ARG, "ldx < N");
  if (!ovh::norm_fusable())
    return fail(OV_ERR_NOT_IMPLEMENTED,
                "residual + norm GEMM: needs a device of 8 XCDs (the row bands' placement)");
  ovh::GemmArgs a = base_args(M, aq, asc, w);
  a.a_tiled = 1;
  a.nslices = 1;
  a.start[0] = 0;
  a.start[1] = (int)w->w.N;
  a.out[0] = x;
  a.ld[0] = ldx;
  a.nw = nw;
  a.neps = eps;
  a.nq = nq;
  a.nsc = nsc;
  a.n_tiled = 1;
  a.band_cnt = band_cnt;
  a.norm_err = err;
  a.xcd_test = xcd_test;
  OVH_HIP(ovh::launch_gemm(a, ovh::kAccumNorm, st), "residual + norm gemm launch");
  return OV_OK;
}

int linear_q_sliced(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w,
                    const int64_t* slice_n, float* const* slice_c, int n_slices, hipStream_t st,
                    bool a_tiled, _Float16* f16_codes, bool f16_ok) {
  if (M <= 0 || n_slices <= 0) return OV_OK;
  int rc = check_gemm_operands(M, aq, asc, w);
  if (rc != OV_OK) return rc;
  if (!slice_n || !slice_c) return fail(OV_ERR_INVALID_ARG, "slices are null");
  if (n_slices > ovh::kMaxSlices)
    return fail(OV_ERR_INVALID_ARG, "sliced GEMM: at most 8 slices");
  ovh::GemmArgs a = base_args(M, aq, asc, w);
  a.a_tiled = a_tiled;
  int64_t total = 0;
  a.nslices = n_slices;
  for (int s = 0; s < n_slices; ++s) {
    if (slice_n[s] <= 0 || slice_n[s] % 64 != 0 || !slice_c[s])
      return fail(OV_ERR_INVALID_ARG, "sliced GEMM: each slice N must be a positive multiple of 64");
    a.start[s] = (int)total;
    a.out[s] = slice_c[s];
    a.ld[s] = slice_n[s];
    total += slice_n[s];
  }
  if (total != w->w.N)
    return fail(OV_ERR_INVALID_ARG, "sliced GEMM: slice widths must sum to the weight's N");
  a.start[n_slices] = (int)total;
  _Float16* ws = nullptr;
  if ((rc = f16_operands(M, aq, a_tiled, w, f16_codes, st, a, &ws, f16_ok)) != OV_OK) return rc;
  return launch_with_ws(a, ovh::kStore, ws, st);
}
}  // namespace ovh

extern "C" {

const char* ovh_last_error(void) { return t_err.c_str(); }

size_t ovh_copy_last_error(char* err, size_t err_len) {
  if (err && err_len > 0) {
    const size_t n = t_err.size() < err_len - 1 ? t_err.size() : err_len - 1;
    std::memcpy(err, t_err.data(), n);
    err[n] = '\0';
  }
  return t_err.size();
}

int ovh_abi_version(void) { return OVH_ABI_VERSION; }

int ovh_backend_name(char* buf, size_t len) {
  int dev = 0;
  OVH_HIP(hipGetDevice(&dev), "hipGetDevice");
  hipDeviceProp_t p;
  OVH_HIP(hipGetDeviceProperties(&p, dev), "hipGetDeviceProperties");
  if (buf && len) std::snprintf(buf, len, "hip:%s (%d CUs)", p.gcnArchName, p.multiProcessorCount);
  return OV_OK;
}

int64_t ovh_quant_bytes(int64_t M, int64_t K) {
  return (M <= 0 || K <= 0) ? 0 : M * ovh::kb_of(K) * 32;
}
int64_t ovh_quant_scales(int64_t M, int64_t K) {
  return (M <= 0 || K <= 0) ? 0 : M * ovh::kb_of(K);
}

// ---- weights ----------------------------------------------------------------

int ovh_weight_from_device(int64_t N, int64_t K, const int8_t* q, const float* scale, int layout,
                           void* stream, OvhWeight** out) {
  if (!out) return fail(OV_ERR_INVALID_ARG, "out is null");
  *out = nullptr;
  if (N <= 0 || K <= 0) return fail(OV_ERR_INVALID_ARG, "weight dims must be positive");
  if (layout != 0 && layout != 1) return fail(OV_ERR_INVALID_ARG, "layout must be 0 (nk) or 1 (kn)");
  if (!q || !scale) return fail(OV_ERR_INVALID_ARG, "q/scale are null");
  OvhWeight* h = nullptr;
  const int rc = new_weight(N, K, &h);
  if (rc != OV_OK) return rc;
  const hipError_t e = ovh::launch_weight_layout(N, K, q, layout, scale, h->w, as_stream(stream));
  if (e != hipSuccess) {
    ovh_weight_free(h);
    return hip_fail(e, "weight layout");
  }
  *out = h;
  return OV_OK;
}

int ovh_weight_upload(int64_t N, int64_t K, const int8_t* q, const float* scale, int layout,
                      void* stream, OvhWeight** out) {
  if (!out) return fail(OV_ERR_INVALID_ARG, "out is null");
  *out = nullptr;
  if (N <= 0 || K <= 0) return fail(OV_ERR_INVALID_ARG, "weight dims must be positive");
  if (!q || !scale) return fail(OV_ERR_INVALID_ARG, "q/scale are null");
  int8_t* dq = nullptr;
  float* ds = nullptr;
  const hipStream_t st = as_stream(stream);
  OVH_HIP(hipMalloc(reinterpret_cast<void**>(&dq), (size_t)(N * K)), "hipMalloc(staging)");
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&ds), sizeof(float) * (size_t)N);
  if (e == hipSuccess) e = hipMemcpyAsync(dq, q, (size_t)(N * K), hipMemcpyHostToDevice, st);
  if (e == hipSuccess)
    e = hipMemcpyAsync(ds, scale, sizeof(float) * (size_t)N, hipMemcpyHostToDevice, st);
  int rc = OV_OK;
  if (e != hipSuccess) {
    rc = hip_fail(e, "weight upload");
  } else {
    rc = ovh_weight_from_device(N, K, dq, ds, layout, stream, out);
    if (rc == OV_OK) {
      e = hipStreamSynchronize(st);  // staging buffers are freed below
      if (e != hipSuccess) {
        ovh_weight_free(*out);
        *out = nullptr;
        rc = hip_fail(e, "weight upload sync");
      }
    }
  }
  (void)hipFree(dq);
  if (ds) (void)hipFree(ds);
  return rc;
}

int ovh_weight_concat(const OvhWeight* const* parts, int n_parts, void* stream, OvhWeight** out) {
  if (!out) return fail(OV_ERR_INVALID_ARG, "out is null");
  *out = nullptr;
  if (!parts || n_parts <= 0) return fail(OV_ERR_INVALID_ARG, "no parts");
  int64_t N = 0;
  const int64_t K = parts[0] ? parts[0]->w.K : 0;
  for (int i = 0; i < n_parts; ++i) {
    if (!parts[i] || parts[i]->silu_pair || parts[i]->f32 || parts[i]->w.K != K ||
        parts[i]->w.N % 64 != 0)
      return fail(OV_ERR_INVALID_ARG, "concat: parts need equal K and N a multiple of 64");
    N += parts[i]->w.N;
  }
  OvhWeight* h = nullptr;
  const int rc = new_weight(N, K, &h);
  if (rc != OV_OK) return rc;
  const hipStream_t st = as_stream(stream);
  ovh::DeviceWeight& w = h->w;
  hipError_t e = hipSuccess;
  int64_t row = 0;
  for (int i = 0; i < n_parts && e == hipSuccess; ++i) {
    const ovh::DeviceWeight& p = parts[i]->w;
    e = hipMemcpyAsync(w.q + row * w.Kp, p.q, (size_t)(p.N * p.Kp), hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess)
      e = hipMemcpyAsync(w.scale + row, p.scale, sizeof(float) * (size_t)p.N,
                         hipMemcpyDeviceToDevice, st);
    row += p.N;
  }
  if (e == hipSuccess && w.Npad > N) {
    e = hipMemsetAsync(w.q + N * w.Kp, 0, (size_t)((w.Npad - N) * w.Kp), st);
    if (e == hipSuccess)
      e = hipMemsetAsync(w.scale + N, 0, sizeof(float) * (size_t)(w.Npad - N), st);
  }
  if (e != hipSuccess) {
    ovh_weight_free(h);
    return hip_fail(e, "weight concat");
  }
  *out = h;
  return OV_OK;
}

void ovh_weight_free(OvhWeight* h) {
  if (!h) return;
  if (h->w.q) (void)hipFree(h->w.q);
  if (h->w.scale) (void)hipFree(h->w.scale);
  if (h->w.q16) (void)hipFree(h->w.q16);
  if (h->fw.hi) (void)hipFree(h->fw.hi);
  if (h->fw.lo) (void)hipFree(h->fw.lo);
  if (h->fw.scale) (void)hipFree(h->fw.scale);
  delete h;
}

int ovh_weight_upload_f32(int64_t N, int64_t K, const float* w, int layout, void* stream,
                          OvhWeight** out) {
  if (!out) return fail(OV_ERR_INVALID_ARG, "out is null");
  return ovh::weight_upload_f32(N, K, w, layout, as_stream(stream), out);
}

int ovh_linear_f32(int64_t M, const float* A, const OvhWeight* w, float* C, int64_t ldc,
                   int accumulate, void* stream) {
  if (M <= 0) return OV_OK;
  if (!w || !A || !C) return fail(OV_ERR_INVALID_ARG, "null argument");
  if (!w->f32) return fail(OV_ERR_INVALID_ARG, "linear_f32: the weight is not fp32");
  if (M > 0x7fffffff || w->w.N > 0x7fffffff)
    return fail(OV_ERR_INVALID_ARG, "M and N must fit in 31 bits");
  if (ldc < w->w.N) return fail(OV_ERR_INVALID_ARG, "ldc < N");
  const hipStream_t st = as_stream(stream);
  const ovh::F32Weight& fw = w->fw;
  const size_t plane = sizeof(_Float16) * (size_t)ovh::f32_plane_halves(M, fw.K);
  const size_t rows = (size_t)((M + 127) / 128 * 128);
  char* ws = nullptr;
  OVH_HIP(hipMallocAsync(reinterpret_cast<void**>(&ws), 2 * plane + sizeof(float) * rows, st),
          "hipMallocAsync(linear_f32)");
  ovh::GemmF32Args a;
  a.M = (int)M;
  a.N = (int)fw.N;
  a.Ks = fw.Ks;
  _Float16* hi = reinterpret_cast<_Float16*>(ws);
  _Float16* lo = reinterpret_cast<_Float16*>(ws + plane);
  float* sc = reinterpret_cast<float*>(ws + 2 * plane);
  a.ahi = hi;
  a.alo = lo;
  a.ascale = sc;
  a.whi = fw.hi;
  a.wlo = fw.lo;
  a.wscale = fw.scale;
  a.C = C;
  a.ldc = ldc;
  a.accumulate = accumulate != 0;
  hipError_t e = ovh::launch_f32_split(M, fw.K, A, fw.Ks, hi, lo, sc, st);
  if (e == hipSuccess) e = ovh::launch_gemm_f32(a, st);
  (void)hipFreeAsync(ws, st);
  if (e != hipSuccess) return hip_fail(e, "linear_f32 launch");
  return OV_OK;
}

int64_t ovh_weight_n(const OvhWeight* w) { return w ? w->w.N : 0; }
int ovh_weight_is_f32(const OvhWeight* w) { return w && w->f32 ? 1 : 0; }
int64_t ovh_weight_k(const OvhWeight* w) { return w ? w->w.K : 0; }

int ovh_weight_download(const OvhWeight* w, int8_t* q_nk, float* scale, void* stream) {
  if (!w || !q_nk || !scale) return fail(OV_ERR_INVALID_ARG, "null argument");
  if (w->f32) return fail(OV_ERR_INVALID_ARG, "weight_download: the weight is fp32");
  const hipStream_t st = as_stream(stream);
  hipError_t e = ovh::launch_weight_to_nk(w->w, q_nk, st);
  if (e == hipSuccess)
    e = hipMemcpyAsync(scale, w->w.scale, sizeof(float) * (size_t)w->w.N,
                       hipMemcpyDeviceToDevice, st);
  if (e != hipSuccess) return hip_fail(e, "weight download");
  return OV_OK;
}

// ---- quantisers ---------------------------------------------------------------

int ovh_s8_nk_quantize(int64_t M, int64_t K, const float* A, int8_t* aq, float* asc,
                       void* stream) {
  if (M <= 0 || K <= 0) return OV_OK;
  if (!A || !aq || !asc) return fail(OV_ERR_INVALID_ARG, "null device pointer");
  if (((uintptr_t)aq & 3u) != 0) return fail(OV_ERR_INVALID_ARG, "aq must be 4-byte aligned");
  OVH_HIP(ovh::launch_quantize(M, K, A, aq, asc, as_stream(stream)), "quantize launch");
  return OV_OK;
}

int ovh_rmsnorm_quantize(int64_t rows, int64_t cols, const float* x, const float* w, float eps,
                         int8_t* aq, float* asc, void* stream) {
  if (rows <= 0 || cols <= 0) return OV_OK;
  if (!x || !w || !aq || !asc) return fail(OV_ERR_INVALID_ARG, "null device pointer");
  if (((uintptr_t)aq & 3u) != 0) return fail(OV_ERR_INVALID_ARG, "aq must be 4-byte aligned");
  if (ovh::rmsnorm_quantize_smem(cols) > 160 * 1024)
    return fail(OV_ERR_INVALID_ARG, "rmsnorm_quantize: cols too large for one LDS row stage");
  OVH_HIP(ovh::launch_rmsnorm_quantize(rows, cols, x, w, eps, aq, asc, as_stream(stream)),
          "rmsnorm_quantize launch");
  return OV_OK;
}

int ovh_silu_mul_quantize(int64_t M, int64_t K, const float* gate, const float* up, int8_t* aq,
                          float* asc, void* stream) {
  if (M <= 0 || K <= 0) return OV_OK;
  if (!gate || !up || !aq || !asc) return fail(OV_ERR_INVALID_ARG, "null device pointer");
  if (((uintptr_t)aq & 3u) != 0) return fail(OV_ERR_INVALID_ARG, "aq must be 4-byte aligned");
  OVH_HIP(ovh::launch_silu_mul_quantize(M, K, gate, up, aq, asc, as_stream(stream)),
          "silu_mul_quantize launch");
  return OV_OK;
}

// ---- GEMM -----------------------------------------------------------------------

int ovh_linear_q(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w, float* C,
                 int64_t ldc, int accumulate, void* stream) {
  return ovh::linear_q(M, aq, asc, w, C, ldc, accumulate, as_stream(stream), false);
}

int ovh_linear_q_tiled(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w,
                       float* C, int64_t ldc, int accumulate, void* stream) {
  if (M > 0 && w && w->w.Kb % 4 != 0)
    return fail(OV_ERR_NOT_IMPLEMENTED, "linear_q_tiled: K must be a multiple of 128");
  return ovh::linear_q(M, aq, asc, w, C, ldc, accumulate, as_stream(stream), true);
}

// band_cnt: the hand-off error word in the first counter slot, then the band
// slots for launches of up to max_rows rows (band_counter_words)
int64_t ovh_band_counter_bytes(int64_t max_rows) {
  if (max_rows < 1) max_rows = 1;
  return (int64_t)sizeof(unsigned long long) *
         (ovh::kBandCntStride + ovh::band_counter_words(max_rows));
}

int ovh_linear_q_norm(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w, float* x,
                      int64_t ldx, const float* nw, float eps, int8_t* nq, float* nsc,
                      void* band_cnt, void* stream) {
  if (M <= 0) return OV_OK;
  if (!w) return fail(OV_ERR_INVALID_ARG, "weight is null");
  if (w->w.Kb % 4 != 0)
    return fail(OV_ERR_NOT_IMPLEMENTED, "linear_q_norm: K must be a multiple of 128");
  if (w->w.N % 256 != 0 || w->w.N > 1024)
    return fail(OV_ERR_NOT_IMPLEMENTED, "linear_q_norm: N must be 256, 512, 768 or 1024");
  if (!band_cnt) return fail(OV_ERR_INVALID_ARG, "band_cnt is null");
  auto* cnt = static_cast<unsigned long long*>(band_cnt);
  return ovh::linear_q_norm(M, aq, asc, w, x, ldx, nw, eps, nq, nsc, cnt + ovh::kBandCntStride,
                            reinterpret_cast<uint32_t*>(cnt), as_stream(stream));
}

int ovh_linear_q_sliced(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* w,
                        const int64_t* slice_n, float* const* slice_c, int n_slices,
                        void* stream) {
  return ovh::linear_q_sliced(M, aq, asc, w, slice_n, slice_c, n_slices, as_stream(stream), false);
}

int ovh_linear_q_grouped(const OvhGemmGroup* groups, int n_groups, int accumulate,
                         void* stream) {
  if (n_groups <= 0) return OV_OK;
  if (!groups) return fail(OV_ERR_INVALID_ARG, "groups is null");
  if (n_groups > ovh::kMaxGroups)
    return fail(OV_ERR_INVALID_ARG, "grouped GEMM: at most 8 groups");
  ovh::GemmGroups gg;
  for (int g = 0; g < n_groups; ++g) {
    const OvhGemmGroup& m = groups[g];
    if (m.M <= 0) continue;  // an empty member: nothing to launch
    int rc = check_gemm_operands(m.M, m.aq, m.asc, m.w);
    if (rc != OV_OK) return rc;
    if (!m.C) return fail(OV_ERR_INVALID_ARG, "C is null");
    if (m.ldc < m.w->w.N) return fail(OV_ERR_INVALID_ARG, "ldc < N");
    if (m.w->w.Kb % 4 != 0)
      return fail(OV_ERR_NOT_IMPLEMENTED, "grouped GEMM: K must be a multiple of 128");
    ovh::GemmArgs a = base_args(m.M, m.aq, m.asc, m.w);
    a.nslices = 1;
    a.start[0] = 0;
    a.start[1] = (int)m.w->w.N;
    a.out[0] = m.C;
    a.ld[0] = m.ldc;
    gg.args[gg.n++] = a;
  }
  if (gg.n == 0) return OV_OK;
  OVH_HIP(ovh::launch_gemm_grouped(gg, accumulate ? ovh::kAccumulate : ovh::kStore,
                                   as_stream(stream)),
          "grouped gemm launch");
  return OV_OK;
}

}  // extern "C"

namespace {
// ovh_linear's quantised copy of A.  One workspace per (device, stream), kept
// from the first eager call on that stream until the process ends and grown
// when a call needs more: eager calls on one stream are ordered by the stream,
// calls on different streams never share one.  Growth frees the old buffer and
// allocates the new one on the calling stream (hipFreeAsync/hipMallocAsync),
// after that stream's earlier work.  A call under graph capture never touches
// the workspace: it allocates and frees in the graph (memory nodes), so the
// graph owns its buffer, stays valid when a later eager call grows (frees)
// the workspace, and shares nothing with eager calls or with replays on other
// streams.  A stream destroyed while a call on it is still running must not be
// replaced by a new stream of the same handle before that call ends.
struct LinearWorkspace {
  int device;
  hipStream_t stream;
  void* ptr;
  size_t bytes;
};
constexpr int kMaxLinearWorkspaces = 256;
std::mutex g_ws_mu;
LinearWorkspace g_ws[kMaxLinearWorkspaces];
int g_ws_n = 0;

// The workspace of the current device and stream st with at least `bytes`
// (*ptr), or *ptr = nullptr and *owned = true after a stream-ordered
// allocation the caller frees (capture, or more streams than the table holds).
int linear_workspace(hipStream_t st, size_t bytes, void** ptr, bool* owned) {
  *ptr = nullptr;
  *owned = false;
  int dev = 0;
  OVH_HIP(hipGetDevice(&dev), "hipGetDevice");
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  OVH_HIP(hipStreamIsCapturing(st, &cap), "hipStreamIsCapturing");
  if (cap != hipStreamCaptureStatusNone) {
    // the graph's own buffer (see above)
    OVH_HIP(hipMallocAsync(ptr, bytes, st), "hipMallocAsync(linear workspace, captured)");
    *owned = true;
    return OV_OK;
  }
  std::lock_guard<std::mutex> lock(g_ws_mu);
  LinearWorkspace* ws = nullptr;
  for (int i = 0; i < g_ws_n; ++i)
    if (g_ws[i].device == dev && g_ws[i].stream == st) ws = &g_ws[i];
  if (ws && ws->bytes >= bytes) {
    *ptr = ws->ptr;
    return OV_OK;
  }
  if (!ws && g_ws_n == kMaxLinearWorkspaces) {
    OVH_HIP(hipMallocAsync(ptr, bytes, st), "hipMallocAsync(linear workspace)");
    *owned = true;
    return OV_OK;
  }
  if (!ws) {
    ws = &g_ws[g_ws_n++];
    *ws = LinearWorkspace{dev, st, nullptr, 0};
  }
  if (ws->ptr) {
    (void)hipFreeAsync(ws->ptr, st);
    ws->ptr = nullptr;
    ws->bytes = 0;
  }
  const size_t grown = bytes + bytes / 4;  // room for a somewhat larger M next time
  OVH_HIP(hipMallocAsync(&ws->ptr, grown, st), "hipMallocAsync(linear workspace)");
  ws->bytes = grown;
  *ptr = ws->ptr;
  return OV_OK;
}
}  // namespace

extern "C" {

int ovh_linear(int64_t M, const float* A, const OvhWeight* w, float* C, int64_t ldc,
               int accumulate, void* stream) {
  if (M <= 0) return OV_OK;
  if (!w || !A) return fail(OV_ERR_INVALID_ARG, "null argument");
  const hipStream_t st = as_stream(stream);
  // K a multiple of 128: the codes tile-major (the layout the 16x16 GEMM reads
  // as contiguous 1 KiB tiles), else row-major; the scales [M][Kb] follow at
  // the next 256-byte boundary
  const bool tiled = w->w.Kb % 4 == 0;
  const size_t code_bytes =
      ((tiled ? (size_t)ovh_tiled_codes_bytes(M, w->w.K) : (size_t)M * (size_t)w->w.Kp) + 255) &
      ~(size_t)255;
  void* ws = nullptr;
  bool owned = false;
  int rc = linear_workspace(st, code_bytes + sizeof(float) * (size_t)M * (size_t)w->w.Kb, &ws,
                            &owned);
  if (rc != OV_OK) return rc;
  int8_t* aq = static_cast<int8_t*>(ws);
  float* asc = reinterpret_cast<float*>(aq + code_bytes);
  if (tiled) {
    const hipError_t e = ovh::launch_quantize(M, w->w.K, A, aq, asc, st, true);
    rc = e == hipSuccess ? ovh::linear_q(M, aq, asc, w, C, ldc, accumulate, st, true)
                         : hip_fail(e, "quantize launch");
  } else {
    rc = ovh_s8_nk_quantize(M, w->w.K, A, aq, asc, stream);
    if (rc == OV_OK) rc = ovh_linear_q(M, aq, asc, w, C, ldc, accumulate, stream);
  }
  if (owned) (void)hipFreeAsync(ws, st);
  return rc;
}

namespace {
int block_dots(int64_t M, const int8_t* aq, const OvhWeight* w, int32_t* out, void* stream,
               bool tiled) {
  if (M <= 0) return OV_OK;
  int rc = check_gemm_operands(M, aq, reinterpret_cast<const float*>(aq), w);
  if (rc != OV_OK) return rc;
  if (!out) return fail(OV_ERR_INVALID_ARG, "out is null");
  if (tiled && w->w.Kb % 4 != 0)
    return fail(OV_ERR_INVALID_ARG, "block_dots_tiled: K must be a multiple of 128");
  ovh::GemmArgs a = base_args(M, aq, nullptr, w);
  a.asc = nullptr;
  a.a_tiled = tiled;
  a.start[1] = (int)w->w.N;
  a.dump = out;
  OVH_HIP(ovh::launch_gemm(a, ovh::kDumpBlocks, as_stream(stream)), "gemm launch");
  return OV_OK;
}
}  // namespace

int ovh_block_dots(int64_t M, const int8_t* aq, const OvhWeight* w, int32_t* out, void* stream) {
  return block_dots(M, aq, w, out, stream, false);
}

int ovh_diag_read(const void* src, int64_t bytes, int path, void* stream) {
  if (!src) return fail(OV_ERR_INVALID_ARG, "src is null");
  if (path < 0 || path > 3) return fail(OV_ERR_INVALID_ARG, "path must be 0 .. 3");
  if (bytes <= 0 || bytes % (128 * 1024) != 0 || bytes > (int64_t(128) << 30))
    return fail(OV_ERR_INVALID_ARG, "bytes must be a positive multiple of 128 KiB (at most 128 GiB)");
  OVH_HIP(ovh::launch_read_paths(static_cast<const int8_t*>(src), bytes, path, as_stream(stream)),
          "diag read launch");
  return OV_OK;
}

// ---- allocation-free linear -------------------------------------------------
// ovh_linear quantises A into a stream-ordered allocation; this variant puts
// the codes and scales in a fixed device array instead.  Each device holds its
// own copy of `scratch` (a file-scope device array) from the first call on it
// until the process ends; its device address is looked up once per device with
// that device current and kept in g_scratch.  In host code the array's name is
// not a device address: only the looked-up pointer reaches kernels.
}  // extern "C"

namespace {
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) int8_t scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

int scratch_of_current_device(void** out) {
  int dev = 0;
  OVH_HIP(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(OV_ERR_NOT_IMPLEMENTED, "linear_noalloc: device index beyond 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    OVH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!p) return fail(OV_ERR_INTERNAL, "hipGetSymbolAddress(scratch) returned null");
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return OV_OK;
}
}  // namespace

extern "C" {

int ovh_linear_noalloc(int64_t M, const float* A, const OvhWeight* w, float* C, int64_t ldc,
                       int accumulate, void* stream) {
  if (M <= 0) return OV_OK;
  if (!w || !A) return fail(OV_ERR_INVALID_ARG, "null argument");
  // codes at offset 0 ([M][Kp], or tile-major as in ovh_linear when K is a
  // multiple of 128 and the rows padded to 128 still fit), scales [M][Kb] at
  // the next 256-byte boundary; the quantiser writes every code and scale the
  // GEMM uses (K-tail padding included; rows of a tile past M are read but
  // their outputs dropped), so nothing has to start at zero
  const size_t scale_bytes = sizeof(float) * (size_t)M * (size_t)w->w.Kb;
  const size_t tiled_bytes = ((size_t)ovh_tiled_codes_bytes(M, w->w.K) + 255) & ~(size_t)255;
  const bool tiled = w->w.Kb % 4 == 0 && tiled_bytes + scale_bytes <= kNoAllocScratchBytes;
  const size_t code_bytes =
      tiled ? tiled_bytes : ((size_t)M * (size_t)w->w.Kp + 255) & ~(size_t)255;
  const size_t need = code_bytes + scale_bytes;
  if (M > ((int64_t)1 << 31) || need > kNoAllocScratchBytes)
    return fail(OV_ERR_INVALID_ARG,
                "linear_noalloc: M * (Kp + 4 * Kb) = " + std::to_string(need) +
                    " bytes exceeds the 16 MiB scratch (use ovh_linear)");
  void* base = nullptr;
  int rc = scratch_of_current_device(&base);
  if (rc != OV_OK) return rc;
  int8_t* aq = static_cast<int8_t*>(base);
  float* asc = reinterpret_cast<float*>(static_cast<char*>(base) + code_bytes);
  if (tiled) {
    const hipError_t e = ovh::launch_quantize(M, w->w.K, A, aq, asc, as_stream(stream), true);
    if (e != hipSuccess) return hip_fail(e, "quantize launch");
  } else {
    rc = ovh_s8_nk_quantize(M, w->w.K, A, aq, asc, stream);
  }
  // the int8 GEMM form at every M (the f16 form would allocate)
  if (rc == OV_OK)
    rc = ovh::linear_q(M, aq, asc, w, C, ldc, accumulate, as_stream(stream), tiled, nullptr, false);
  return rc;
}

int64_t ovh_set_f16_min_rows(int64_t rows) {
  const int64_t prev = ovh::f16_min_rows();
  if (rows >= 0) ovh::set_f16_min_rows(rows);
  return prev;
}

int64_t ovh_set_attention_long_min_tasks(int64_t tasks) {
  const int64_t prev = ovh::attention_long_min_tasks();
  if (tasks >= 0) ovh::set_attention_long_min_tasks(tasks);
  return prev;
}

int ovh_block_dots_tiled(int64_t M, const int8_t* aq, const OvhWeight* w, int32_t* out,
                         void* stream) {
  return block_dots(M, aq, w, out, stream, true);
}

int64_t ovh_tiled_codes_bytes(int64_t M, int64_t K) {
  return (M <= 0 || K <= 0) ? 0 : (M + 127) / 128 * 128 * ovh::kb_of(K) * 32;
}

// ---- SiLU-fused gate/up ------------------------------------------------------

int ovh_weight_gate_up(const OvhWeight* gate, const OvhWeight* up, void* stream, OvhWeight** out) {
  if (!out) return fail(OV_ERR_INVALID_ARG, "out is null");
  return ovh::weight_interleave16(gate, up, as_stream(stream), out);
}

int ovh_silu_gate_linear(int64_t M, const int8_t* aq, const float* asc, const OvhWeight* gate_up,
                         int8_t* hq, float* hsc, void* stream) {
  if (M <= 0) return OV_OK;
  if (!gate_up) return fail(OV_ERR_INVALID_ARG, "weight handle is null");
  if (!gate_up->silu_pair)
    return fail(OV_ERR_INVALID_ARG, "silu_gate_linear: the weight must come from ovh_weight_gate_up");
  if (M > 0x7fffffff || gate_up->w.N > 0x7fffffff)
    return fail(OV_ERR_INVALID_ARG, "M and N must fit in 31 bits");
  if (!aq || !asc || !hq || !hsc) return fail(OV_ERR_INVALID_ARG, "null device pointer");
  if (!aligned16(aq) || ((uintptr_t)hq & 3u) != 0)
    return fail(OV_ERR_INVALID_ARG, "aq must be 16-byte and hq 4-byte aligned");
  if (gate_up->w.Kb % 4 != 0)
    return fail(OV_ERR_NOT_IMPLEMENTED, "silu_gate_linear: K must be a multiple of 128");
  ovh::GemmArgs a;
  a.M = (int)M;
  a.N = (int)gate_up->w.N;
  a.Kb = (int)gate_up->w.Kb;
  a.Kp = gate_up->w.Kp;
  a.aq = aq;
  a.asc = asc;
  a.W = gate_up->w.q;
  a.ws = gate_up->w.scale;
  a.hq = hq;
  a.hsc = hsc;
  a.hKp = gate_up->w.N / 2;  // I, a multiple of 64
  _Float16* ws = nullptr;
  const int rc = f16_operands(M, aq, false, gate_up, nullptr, as_stream(stream), a, &ws);
  if (rc != OV_OK) return rc;
  return launch_with_ws(a, ovh::kSiluQuant, ws, as_stream(stream));
}


int ovh_rope_tables(int64_t rows, const int64_t* pos, int head_dim, float theta, float* cos_tab,
                    float* sin_tab, void* stream) {
  if (rows <= 0) return OV_OK;
  if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > 1024)
    return fail(OV_ERR_INVALID_ARG, "rope_tables: head_dim must be even and <= 1024");
  if (!pos || !cos_tab || !sin_tab) return fail(OV_ERR_INVALID_ARG, "null device pointer");
  OVH_HIP(ovh::launch_rope_tables(rows, pos, head_dim, theta, cos_tab, sin_tab, as_stream(stream)),
          "rope tables launch");
  return OV_OK;
}

int ovh_qk_norm_rope(float* q, float* k, const float* qw, const float* kw, int64_t rows,
                     int n_heads, int n_kv_heads, int head_dim, const float* cos_tab,
                     const float* sin_tab, float eps, void* stream) {
  if (rows <= 0) return OV_OK;
  if (head_dim != 64 && head_dim != 128)
    return fail(OV_ERR_NOT_IMPLEMENTED, "qk_norm_rope: head_dim must be 64 or 128");
  if (n_heads < 0 || n_kv_heads < 0 || n_heads + n_kv_heads <= 0)
    return fail(OV_ERR_INVALID_ARG, "qk_norm_rope: bad head counts");
  if ((n_heads && (!q || !qw)) || (n_kv_heads && (!k || !kw)) || !cos_tab || !sin_tab)
    return fail(OV_ERR_INVALID_ARG, "null device pointer");
  OVH_HIP(ovh::launch_qk_norm_rope(q, k, qw, kw, rows, n_heads, n_kv_heads, head_dim, cos_tab,
                                   sin_tab, eps, as_stream(stream)),
          "qk_norm_rope launch");
  return OV_OK;
}

int ovh_attention(const OvhAttnSegment* segs, int n_segs, int n_heads, int n_kv_heads,
                  int head_dim, const float* q, int64_t q_stride, const float* k, const float* v,
                  int64_t kv_stride, float scale, float* out, int64_t out_stride, void* stream) {
  if (n_segs <= 0) return OV_OK;
  if (!segs) return fail(OV_ERR_INVALID_ARG, "segs is null");
  if (head_dim != 128) return fail(OV_ERR_NOT_IMPLEMENTED, "attention: head_dim must be 128");
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || n_heads > 65535)
    return fail(OV_ERR_INVALID_ARG, "attention: n_heads must be a positive multiple of n_kv_heads");
  if (!q || !k || !v || !out) return fail(OV_ERR_INVALID_ARG, "null device pointer");
  if (q_stride < (int64_t)n_heads * head_dim || out_stride < (int64_t)n_heads * head_dim ||
      kv_stride < (int64_t)n_kv_heads * head_dim)
    return fail(OV_ERR_INVALID_ARG, "attention: row strides smaller than the head span");
  if ((q_stride | kv_stride | out_stride) & 3)
    return fail(OV_ERR_INVALID_ARG, "attention: strides must be multiples of 4 elements");
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 15u)
    return fail(OV_ERR_INVALID_ARG, "attention: q/k/v/out must be 16-byte aligned");
  for (int s = 0; s < n_segs; ++s) {
    if (segs[s].rows < 0 || segs[s].q_off < 0 || segs[s].kv_off < 0 || (segs[s].q_off & 3) ||
        (segs[s].kv_off & 3))
      return fail(OV_ERR_INVALID_ARG, "attention: bad segment (rows/offsets)");
  }
  for (int s0 = 0; s0 < n_segs; s0 += ovh::kAttnMaxSegs) {
    ovh::AttnArgs a{};
    a.q = q; a.k = k; a.v = v; a.out = out;
    a.q_stride = q_stride; a.kv_stride = kv_stride; a.out_stride = out_stride;
    a.n_heads = n_heads; a.group = n_heads / n_kv_heads; a.scale = scale;
    a.n_segs = n_segs - s0 < ovh::kAttnMaxSegs ? n_segs - s0 : ovh::kAttnMaxSegs;
    int max_rows = 0;
    for (int i = 0; i < a.n_segs; ++i) {
      const OvhAttnSegment& g = segs[s0 + i];
      a.segs[i] = ovh::AttnSeg{g.bias, g.rows, g.q_off, g.kv_off, nullptr};
      max_rows = g.rows > max_rows ? g.rows : max_rows;
    }
    OVH_HIP(ovh::launch_attention(a, max_rows, as_stream(stream)), "attention launch");
  }
  return OV_OK;
}

int ovh_attention_split(const OvhAttnSegment* segs, int n_segs, int n_heads, int n_kv_heads,
                        int head_dim, const float* q, int64_t q_stride, const float* k,
                        const float* v, int64_t kv_stride, float scale, float* out,
                        int64_t out_stride, void* stream) {
  if (n_segs <= 0) return OV_OK;
  if (n_segs > ovh::kAttnMaxSegs)
    return fail(OV_ERR_INVALID_ARG, "attention_split: at most 32 segments per call");
  if (!segs) return fail(OV_ERR_INVALID_ARG, "segs is null");
  if (head_dim != 128) return fail(OV_ERR_NOT_IMPLEMENTED, "attention: head_dim must be 128");
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || n_heads > 65535)
    return fail(OV_ERR_INVALID_ARG, "attention: n_heads must be a positive multiple of n_kv_heads");
  if (!q || !k || !v || !out) return fail(OV_ERR_INVALID_ARG, "null device pointer");
  if (q_stride < (int64_t)n_heads * head_dim || out_stride < (int64_t)n_heads * head_dim ||
      kv_stride < (int64_t)n_kv_heads * head_dim)
    return fail(OV_ERR_INVALID_ARG, "attention: row strides smaller than the head span");
  if ((q_stride | kv_stride | out_stride) & 7)
    return fail(OV_ERR_INVALID_ARG, "attention_split: strides must be multiples of 8 elements");
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 15u)
    return fail(OV_ERR_INVALID_ARG, "attention: q/k/v/out must be 16-byte aligned");
  ovh::AttnArgs a{};
  a.q = q; a.k = k; a.v = v; a.out = out;
  a.q_stride = q_stride; a.kv_stride = kv_stride; a.out_stride = out_stride;
  a.n_heads = n_heads; a.group = n_heads / n_kv_heads; a.scale = scale; a.n_segs = n_segs;
  ovh::AttnSplit sp{};
  int max_rows = 0;
  for (int s = 0; s < n_segs; ++s) {
    const OvhAttnSegment& g = segs[s];
    if (g.rows < 0 || g.q_off < 0 || g.kv_off < 0 || (g.q_off & 7) || g.kv_off % kv_stride)
      return fail(OV_ERR_INVALID_ARG, "attention_split: bad segment (rows/offsets; kv_off must "
                                      "be a whole number of k rows)");
    a.segs[s] = ovh::AttnSeg{g.bias, g.rows, g.q_off, g.kv_off, nullptr};
    sp.vt_off[s] = sp.vt_cols;
    sp.vt_cols += (g.rows + 31) / 32 * 32;
    max_rows = g.rows > max_rows ? g.rows : max_rows;
  }
  sp.n_kv_heads = n_kv_heads;
  hipStream_t st = as_stream(stream);
  const size_t vbytes = sizeof(_Float16) * (size_t)((int64_t)n_kv_heads * head_dim * sp.vt_cols);
  const size_t kbytes = vbytes;  // K and V planes are both tile-major over the padded keys
  char* ws = nullptr;
  const size_t total = 2 * kbytes + 2 * vbytes + 256;
  OVH_HIP(hipMallocAsync(reinterpret_cast<void**>(&ws), total, st), "hipMallocAsync(split)");
  sp.kh = reinterpret_cast<_Float16*>(ws);
  sp.kl = reinterpret_cast<_Float16*>(ws + kbytes);
  sp.vh = reinterpret_cast<_Float16*>(ws + 2 * kbytes);
  sp.vl = reinterpret_cast<_Float16*>(ws + 2 * kbytes + vbytes);
  sp.overflow = reinterpret_cast<uint32_t*>(ws + 2 * kbytes + 2 * vbytes);
  hipError_t e = hipMemsetAsync(sp.overflow, 0, sizeof(uint32_t), st);
  if (e == hipSuccess) e = ovh::launch_attention_split(a, sp, max_rows, st);
  uint32_t flag = 0;
  if (e == hipSuccess) e = hipMemcpyAsync(&flag, sp.overflow, sizeof flag, hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  (void)hipFreeAsync(ws, st);
  if (e != hipSuccess) return hip_fail(e, "attention_split");
  if (flag)
    return fail(OV_ERR_INVALID_ARG, "attention_split: |k| or |v| beyond the f16 range; use "
                                    "ovh_attention");
  return OV_OK;
}

}  // extern "C"
