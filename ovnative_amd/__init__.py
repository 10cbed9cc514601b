"""ovnative_amd — MI355X (gfx950) int8-nk quantized-linear path for OVNative-class LMs.

The product is ``libovnative_amd.so``: hand-written HIP kernels behind the C ABI
declared in ``include/ovnative_amd.h``.  This module is a thin ctypes binding
of that ABI for Python callers (tests, benchmarks): buffers are torch CUDA
tensors, which on ROCm are HIP device allocations, and every call is enqueued
on torch's current stream.

There is no CPU fallback: if the library is missing, or a call fails, an
exception is raised.  The Python names follow the reference's operator API
(``cpp/include/ovnative/ov_gemm.h``): ``s8_nk_quantize``, ``rmsnorm_quantize``,
``silu_mul_quantize``, ``linear_q`` (= ``linear_s8_nk_packed_q[_add]``),
``linear_q_sliced``, ``linear`` (= ``linear_s8_nk_packed[_add]``).
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libovnative_amd.so")

OV_OK = 0
OV_ERR_INVALID_ARG = -1
OV_ERR_IO = -2
OV_ERR_NOT_IMPLEMENTED = -3
OV_ERR_INTERNAL = -4

# Every symbol include/ovnative_amd.h declares, with its ctypes signature.
_i64, _f32, _p, _int = C.c_int64, C.c_float, C.c_void_p, C.c_int
SIGNATURES = {
    "ovh_last_error": (C.c_char_p, []),
    "ovh_abi_version": (_int, []),
    "ovh_backend_name": (_int, [C.c_char_p, C.c_size_t]),
    "ovh_quant_bytes": (_i64, [_i64, _i64]),
    "ovh_quant_scales": (_i64, [_i64, _i64]),
    "ovh_weight_upload": (_int, [_i64, _i64, _p, _p, _int, _p, C.POINTER(_p)]),
    "ovh_weight_from_device": (_int, [_i64, _i64, _p, _p, _int, _p, C.POINTER(_p)]),
    "ovh_weight_concat": (_int, [C.POINTER(_p), _int, _p, C.POINTER(_p)]),
    "ovh_weight_free": (None, [_p]),
    "ovh_weight_n": (_i64, [_p]),
    "ovh_weight_k": (_i64, [_p]),
    "ovh_weight_download": (_int, [_p, _p, _p, _p]),
    "ovh_s8_nk_quantize": (_int, [_i64, _i64, _p, _p, _p, _p]),
    "ovh_rmsnorm_quantize": (_int, [_i64, _i64, _p, _p, _f32, _p, _p, _p]),
    "ovh_silu_mul_quantize": (_int, [_i64, _i64, _p, _p, _p, _p, _p]),
    "ovh_linear_q": (_int, [_i64, _p, _p, _p, _p, _i64, _int, _p]),
    "ovh_linear_q_sliced": (_int, [_i64, _p, _p, _p, _p, _p, _int, _p]),
    "ovh_linear": (_int, [_i64, _p, _p, _p, _i64, _int, _p]),
    "ovh_block_dots": (_int, [_i64, _p, _p, _p, _p]),
    "ovh_rope_tables": (_int, [_i64, _p, _int, _f32, _p, _p, _p]),
    "ovh_qk_norm_rope": (_int, [_p, _p, _p, _p, _i64, _int, _int, _int, _p, _p, _f32, _p]),
    "ovh_attention": (_int, [_p, _int, _int, _int, _int, _p, _i64, _p, _p, _i64, _f32, _p,
                             _i64, _p]),
}


class AttnSegment(C.Structure):
    """OvhAttnSegment (same fields as ov::AttnSegment, cpp/src/model/lm.h:46-51)."""
    _fields_ = [("bias", C.c_void_p), ("rows", C.c_int32), ("q_off", C.c_int64),
                ("kv_off", C.c_int64)]


class OvhError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"ovnative_amd error {code}: {msg}")
        self.code = code


class InvalidArgument(OvhError, ValueError):
    pass


_LIB = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Load libovnative_amd.so (raises if it has not been built)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def _check(rc: int) -> None:
    if rc != OV_OK:
        msg = load().ovh_last_error().decode(errors="replace")
        if rc == OV_ERR_INVALID_ARG:
            raise InvalidArgument(rc, msg)
        raise OvhError(rc, msg)


# ---------------------------------------------------------------------------
# torch plumbing (device memory and streams only)

def _torch():
    import torch
    return torch


def _stream():
    torch = _torch()
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dptr(t) -> C.c_void_p:
    if t is None:
        return C.c_void_p(0)
    if not t.is_cuda:
        raise ValueError("expected a device (cuda) tensor")
    if not t.is_contiguous():
        raise ValueError("expected a contiguous tensor")
    return C.c_void_p(t.data_ptr())


def kb_of(K: int) -> int:
    return (K + 31) // 32


def backend_name() -> str:
    buf = C.create_string_buffer(128)
    _check(load().ovh_backend_name(buf, 128))
    return buf.value.decode()


class Weight:
    """Device-resident int8 weight with per-output-channel fp32 scales.

    ``q`` is OVW1 int8 in ``layout`` 0 ([N, K]) or 1 ([K, N]); ``scale`` has N
    floats (tools/convert_weights.py:130-135).  Host numpy arrays are uploaded,
    device tensors are consumed in place.
    """

    def __init__(self, handle: int, N: int, K: int):
        self.handle = C.c_void_p(handle)
        self.N, self.K = N, K
        self.Kb = kb_of(K)

    @classmethod
    def from_host(cls, q, scale, layout: int = 0) -> "Weight":
        import numpy as np
        q = np.ascontiguousarray(q, dtype=np.int8)
        scale = np.ascontiguousarray(scale, dtype=np.float32)
        N, K = (q.shape if layout == 0 else q.shape[::-1])
        h = C.c_void_p()
        _check(load().ovh_weight_upload(N, K, q.ctypes.data, scale.ctypes.data, layout, _stream(),
                                        C.byref(h)))
        return cls(h.value, N, K)

    @classmethod
    def from_device(cls, q, scale, layout: int = 0) -> "Weight":
        N, K = (q.shape if layout == 0 else q.shape[::-1])
        h = C.c_void_p()
        _check(load().ovh_weight_from_device(N, K, _dptr(q), _dptr(scale), layout, _stream(),
                                             C.byref(h)))
        return cls(h.value, N, K)

    @classmethod
    def concat(cls, parts) -> "Weight":
        arr = (C.c_void_p * len(parts))(*[p.handle.value for p in parts])
        h = C.c_void_p()
        _check(load().ovh_weight_concat(arr, len(parts), _stream(), C.byref(h)))
        return cls(h.value, sum(p.N for p in parts), parts[0].K)

    def download(self):
        """(q [N, K] int8, scale [N] fp32) device tensors in OVW1 layout 0."""
        torch = _torch()
        q = torch.empty((self.N, self.K), dtype=torch.int8, device="cuda")
        s = torch.empty((self.N,), dtype=torch.float32, device="cuda")
        _check(load().ovh_weight_download(self.handle, _dptr(q), _dptr(s), _stream()))
        return q, s

    def free(self) -> None:
        if self.handle and self.handle.value:
            load().ovh_weight_free(self.handle)
            self.handle = C.c_void_p(0)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _quant_out(M: int, K: int):
    torch = _torch()
    aq = torch.empty((M, kb_of(K) * 32), dtype=torch.int8, device="cuda")
    asc = torch.empty((M, kb_of(K)), dtype=torch.float32, device="cuda")
    return aq, asc


def s8_nk_quantize(A, out=None):
    """A fp32 [M, K] -> (aq int8 [M, Kp], asc fp32 [M, Kb]) (gemm.cpp:379-430)."""
    M, K = A.shape
    aq, asc = out if out is not None else _quant_out(M, K)
    _check(load().ovh_s8_nk_quantize(M, K, _dptr(A), _dptr(aq), _dptr(asc), _stream()))
    return aq, asc


def rmsnorm_quantize(x, w, eps: float = 1e-6, out=None):
    """Fused RMSNorm + quantise (gemm.cpp:638-707)."""
    M, K = x.shape
    aq, asc = out if out is not None else _quant_out(M, K)
    _check(load().ovh_rmsnorm_quantize(M, K, _dptr(x), _dptr(w), eps, _dptr(aq), _dptr(asc),
                                       _stream()))
    return aq, asc


def silu_mul_quantize(gate, up, out=None):
    """silu(gate)*up quantised per 32-k block (ops_cpu.cpp:144-198)."""
    M, K = gate.shape
    aq, asc = out if out is not None else _quant_out(M, K)
    _check(load().ovh_silu_mul_quantize(M, K, _dptr(gate), _dptr(up), _dptr(aq), _dptr(asc),
                                        _stream()))
    return aq, asc


def linear_q(aq, asc, w: Weight, C=None, accumulate: bool = False):
    """C[M, N] (+)= int8 GEMM with the reference epilogue (gemm.cpp:432-504)."""
    torch = _torch()
    M = aq.shape[0]
    if C is None:
        C = torch.zeros((M, w.N), dtype=torch.float32, device="cuda")
    _check(load().ovh_linear_q(M, _dptr(aq), _dptr(asc), w.handle, _dptr(C), C.shape[1],
                               int(bool(accumulate)), _stream()))
    return C


def linear_q_sliced(aq, asc, w: Weight, slice_n, outs=None):
    """One launch over a concatenated weight, one output per slice (gemm.cpp:776-827)."""
    torch = _torch()
    M = aq.shape[0]
    if outs is None:
        outs = [torch.empty((M, n), dtype=torch.float32, device="cuda") for n in slice_n]
    ns = (C.c_int64 * len(slice_n))(*slice_n)
    ptrs = (C.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
    _check(load().ovh_linear_q_sliced(M, _dptr(aq), _dptr(asc), w.handle, ns, ptrs,
                                      len(slice_n), _stream()))
    return outs


def linear(A, w: Weight, C=None, accumulate: bool = False):
    """Quantise fp32 A then GEMM (linear_s8_nk_packed[_add], gemm.cpp:829-882)."""
    torch = _torch()
    M = A.shape[0]
    if C is None:
        C = torch.zeros((M, w.N), dtype=torch.float32, device="cuda")
    _check(load().ovh_linear(M, _dptr(A), w.handle, _dptr(C), C.shape[1], int(bool(accumulate)),
                             _stream()))
    return C


def block_dots(aq, w: Weight):
    """Exact int32 per-(m, n, block) dot products from the MFMA code path."""
    torch = _torch()
    M = aq.shape[0]
    out = torch.empty((M, w.N, w.Kb), dtype=torch.int32, device="cuda")
    _check(load().ovh_block_dots(M, _dptr(aq), w.handle, _dptr(out), _stream()))
    return out


# ---------------------------------------------------------------------------
# attention side of a decoder layer

def rope_tables(pos, head_dim: int, theta: float = 1e6):
    """cos/sin [rows, head_dim/2] for device int64 positions."""
    torch = _torch()
    pos = pos.contiguous()
    c = torch.empty(pos.numel(), head_dim // 2, dtype=torch.float32, device=pos.device)
    s = torch.empty_like(c)
    _check(load().ovh_rope_tables(pos.numel(), _dptr(pos), head_dim, theta, _dptr(c), _dptr(s),
                                  _stream()))
    return c, s


def qk_norm_rope(q, k, qw, kw, n_heads: int, n_kv_heads: int, head_dim: int, cos_tab, sin_tab,
                 eps: float = 1e-6) -> None:
    """In place on q [rows, n_heads*D] and k [rows, n_kv_heads*D] (qk_norm_rope_f32)."""
    _check(load().ovh_qk_norm_rope(_dptr(q), _dptr(k), _dptr(qw), _dptr(kw), q.shape[0], n_heads,
                                   n_kv_heads, head_dim, _dptr(cos_tab), _dptr(sin_tab), eps,
                                   _stream()))


def attention(q, k, v, segs, n_heads: int, n_kv_heads: int, head_dim: int = 128, scale=None,
              out=None):
    """GQA attention over segments (LM::run_layer's loop over attention_head_f32).

    segs: list of (bias tensor [rows, rows] or None, rows, q_row0, kv_row0) with row
    offsets into q [T, n_heads*D] and k/v [T, n_kv_heads*D]."""
    torch = _torch()
    if scale is None:
        scale = float(torch.tensor(1.0) / torch.sqrt(torch.tensor(float(head_dim))))
    if out is None:
        out = torch.zeros_like(q)
    arr = (AttnSegment * max(1, len(segs)))()
    for i, (bias, rows, qr, kr) in enumerate(segs):
        arr[i] = AttnSegment(0 if bias is None else _dptr(bias).value, rows,
                             qr * q.stride(0), kr * k.stride(0))
    _check(load().ovh_attention(C.cast(arr, C.c_void_p), len(segs), n_heads, n_kv_heads,
                                head_dim, _dptr(q), q.stride(0), _dptr(k), _dptr(v), k.stride(0),
                                scale, _dptr(out), out.stride(0), _stream()))
    return out
