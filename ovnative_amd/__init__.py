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
    "ovh_linear_q_tiled": (_int, [_i64, _p, _p, _p, _p, _i64, _int, _p]),
    "ovh_linear_q_norm": (_int, [_i64, _p, _p, _p, _p, _i64, _p, _f32, _p, _p, _p, _p]),
    "ovh_band_counter_bytes": (_i64, [_i64]),
    "ovh_linear": (_int, [_i64, _p, _p, _p, _i64, _int, _p]),
    "ovh_linear_noalloc": (_int, [_i64, _p, _p, _p, _i64, _int, _p]),
    "ovh_weight_upload_f32": (_int, [_i64, _i64, _p, _int, _p, C.POINTER(_p)]),
    "ovh_weight_is_f32": (_int, [_p]),
    "ovh_linear_f32": (_int, [_i64, _p, _p, _p, _i64, _int, _p]),
    "ovh_block_dots": (_int, [_i64, _p, _p, _p, _p]),
    "ovh_diag_read": (_int, [_p, _i64, _int, _p]),
    "ovh_block_dots_tiled": (_int, [_i64, _p, _p, _p, _p]),
    "ovh_tiled_codes_bytes": (_i64, [_i64, _i64]),
    "ovh_set_f16_min_rows": (_i64, [_i64]),
    "ovh_set_attention_long_min_tasks": (_i64, [_i64]),
    "ovh_copy_last_error": (C.c_size_t, [C.c_char_p, C.c_size_t]),
    "ovh_linear_q_grouped": (_int, [_p, _int, _int, _p]),
    "ovh_weight_gate_up": (_int, [_p, _p, _p, C.POINTER(_p)]),
    "ovh_silu_gate_linear": (_int, [_i64, _p, _p, _p, _p, _p, _p]),
    "ovh_rope_tables": (_int, [_i64, _p, _int, _f32, _p, _p, _p]),
    "ovh_qk_norm_rope": (_int, [_p, _p, _p, _p, _i64, _int, _int, _int, _p, _p, _f32, _p]),
    "ovh_attention": (_int, [_p, _int, _int, _int, _int, _p, _i64, _p, _p, _i64, _f32, _p,
                             _i64, _p]),
    "ovh_ovw1_open": (_int, [C.c_char_p, C.POINTER(_p)]),
    "ovh_ovw1_close": (None, [_p]),
    "ovh_ovw1_count": (_int, [_p]),
    "ovh_ovw1_tensors": (_p, [_p]),
    "ovh_ovw1_find": (_p, [_p, C.c_char_p]),
    "ovh_ovw1_n_params": (C.c_uint64, [_p]),
    "ovh_ovw1_compute_crc": (C.c_uint32, [_p, _int]),
    "ovh_lm_create": (_int, [_p, _p, _int, _p, C.POINTER(_p)]),
    "ovh_lm_destroy": (None, [_p]),
    "ovh_lm_forward": (_int, [_p, _int, _int, _p, _p, _p, _p, _p]),
    "ovh_lm_forward_cfg": (_int, [_p, _int, _int, _p, _p, _p, _p, _p, _p]),
    "ovh_lm_last_logits": (_p, [_p]),
    "ovh_lm_set_device_sampling": (None, [_p, _int]),
    "ovh_lm_sample": (_int, [_p, _p, _int, _p, _int, _int, _f32, _f32, _p, _p]),
    "ovh_lm_generate": (_int, [_p, _p, _p, _int, _int, _p, _p]),
    "ovh_attention_split": (_int, [_p, _int, _int, _int, _int, _p, _i64, _p, _p, _i64, _f32, _p,
                                   _i64, _p]),
    "ovh_lm_set_attention": (None, [_p, _int]),
    "ovh_lm_set_graphs": (None, [_p, _int]),
    "ovh_lm_set_fused_norm": (None, [_p, _int]),
    "ovh_lm_set_prefetch": (None, [_p, _int]),
    "ovh_lm_recovered": (_int, [_p]),
    "ovh_lm_last_flags": (_int, [_p]),
    "ovh_lm_force_condition": (None, [_p, _int]),
    "ovh_lm_set_profile": (None, [_p, _int]),
    "ovh_lm_stage_times": (_int, [_p, _p, _p, _int]),
}

# ovh_lm_recovered bits and ovh_lm_force_condition conditions (ovnative_amd.h)
RECOVERED_ATTENTION, RECOVERED_NORM = 1, 2
FORCE_BAND_WAIT, FORCE_XCD = 1, 2


class GenOptions(C.Structure):
    """OvhGenOptions = the sampling fields of TtsOptions (cpp/src/model/tts.h:26-36)."""
    _fields_ = [("num_steps", C.c_int32), ("guidance_scale", C.c_float), ("t_shift", C.c_float),
                ("layer_penalty", C.c_float), ("position_temperature", C.c_float),
                ("seed", C.c_uint32)]

    def __init__(self, **kw):
        d = dict(num_steps=32, guidance_scale=2.0, t_shift=0.1, layer_penalty=5.0,
                 position_temperature=5.0, seed=1234)
        d.update(kw)
        super().__init__(**d)


class TensorView(C.Structure):
    """OvhTensorView (same fields as ov::Tensor, cpp/include/ovnative/ov_types.h)."""
    _fields_ = [("name", C.c_char_p), ("dtype", C.c_int32), ("ndim", C.c_int32),
                ("dims", C.c_int64 * 4), ("transposed", C.c_int32), ("quantized", C.c_int32),
                ("data", C.c_void_p), ("nbytes", C.c_int64), ("scales", C.c_void_p),
                ("n_scales", C.c_int64), ("crc", C.c_uint32)]


class LmConfig(C.Structure):
    """OvhLmConfig = ov::LMConfig (cpp/src/model/lm.h:17-29); defaults are the reference's."""
    _fields_ = [(n, C.c_int32) for n in ("n_layers", "hidden", "n_heads", "n_kv_heads",
                                         "head_dim", "inter", "vocab", "audio_vocab",
                                         "n_codebooks")] + \
               [("rms_eps", C.c_float), ("rope_theta", C.c_float)]

    def __init__(self, **kw):
        d = dict(n_layers=28, hidden=1024, n_heads=16, n_kv_heads=8, head_dim=128, inter=3072,
                 vocab=151676, audio_vocab=1025, n_codebooks=8, rms_eps=1e-6, rope_theta=1e6)
        d.update(kw)
        super().__init__(**d)


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
    def from_host_f32(cls, w, layout: int = 1) -> "Weight":
        """fp32 weight: layout 1 = [K, N] (the reference's fp32 encoding), 0 = [N, K]."""
        import numpy as np
        w = np.ascontiguousarray(w, dtype=np.float32)
        N, K = (w.shape if layout == 0 else w.shape[::-1])
        h = C.c_void_p()
        _check(load().ovh_weight_upload_f32(N, K, w.ctypes.data, layout, _stream(), C.byref(h)))
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


def tile_major(aq, M: int = None):
    """Row-major codes [M, Kp] (device) -> the runner's tile-major layout (1 KiB
    tiles of 32 rows x 32 k; inside a tile (m/16 % 2)*512 + (k/8 % 4)*128 +
    (m%16)*8 + k%8), rows zero-padded to a multiple of 128."""
    torch = _torch()
    M = aq.shape[0] if M is None else M
    Kp = aq.shape[1]
    Mp = (M + 127) // 128 * 128
    a = torch.zeros((Mp, Kp), dtype=torch.int8, device=aq.device)
    a[:M] = aq[:M]
    return a.view(Mp // 32, 2, 16, Kp // 32, 4, 8).permute(0, 3, 1, 4, 2, 5).contiguous().view(-1)


def linear_q_tiled(aq_tiled, asc, w: Weight, M: int, C=None, accumulate: bool = False):
    """linear_q on tile-major codes (tile_major), as the LM runner runs it."""
    torch = _torch()
    if C is None:
        C = torch.zeros((M, w.N), dtype=torch.float32, device="cuda")
    _check(load().ovh_linear_q_tiled(M, _dptr(aq_tiled), _dptr(asc), w.handle, _dptr(C),
                                     C.shape[1], int(bool(accumulate)), _stream()))
    return C


def band_counters(max_rows: int = 2048):
    """Zeroed device memory for linear_q_norm's band counters, for calls of up
    to max_rows rows: allocate one per device and output width N, and pass it
    to every call (stream-ordered)."""
    torch = _torch()
    return torch.zeros(load().ovh_band_counter_bytes(max_rows) // 8, dtype=torch.int64,
                       device="cuda")


def linear_q_norm(aq_tiled, asc, w: Weight, x, nw, band_cnt, eps: float = 1e-6):
    """x[M, N] += linear_q_tiled(aq_tiled, asc, w), then rmsnorm_quantize of the
    updated rows with weight nw, in one launch (lm.cpp:281 + :292, :311 + :232).
    Returns (codes tile-major, zero past row M; scales [M, N / 32])."""
    torch = _torch()
    M, N = x.shape
    nq = torch.zeros(load().ovh_tiled_codes_bytes(M, N), dtype=torch.int8, device="cuda")
    nsc = torch.empty((M, N // 32), dtype=torch.float32, device="cuda")
    _check(load().ovh_linear_q_norm(M, _dptr(aq_tiled), _dptr(asc), w.handle, _dptr(x), N,
                                    _dptr(nw), eps, _dptr(nq), _dptr(nsc), _dptr(band_cnt),
                                    _stream()))
    return nq, nsc


class GemmGroup(C.Structure):
    _fields_ = [("M", C.c_int64), ("aq", C.c_void_p), ("asc", C.c_void_p), ("w", C.c_void_p),
                ("C", C.c_void_p), ("ldc", C.c_int64)]


def linear_q_grouped(problems, outs=None, accumulate: bool = False):
    """ovh_linear_q_grouped: problems = [(aq, asc, Weight), ...] (row-major codes),
    one launch; returns the outputs ([M, N] fp32 each, or `outs` updated)."""
    torch = _torch()
    if outs is None:
        outs = [torch.empty((aq.shape[0], w.N), dtype=torch.float32, device="cuda")
                for aq, _, w in problems]
    arr = (GemmGroup * max(1, len(problems)))()
    for aq, asc, w in problems:
        # the C ABI takes M from here and cannot see the buffers' sizes
        if aq.dim() != 2 or aq.shape[1] < 32 * w.Kb or asc.shape[0] != aq.shape[0]:
            raise InvalidArgument(OV_ERR_INVALID_ARG, "grouped GEMM: codes must be [M, Kp] row-major "
                                  "with block scales [M, Kb]")
    for i, ((aq, asc, w), c) in enumerate(zip(problems, outs)):
        arr[i] = GemmGroup(aq.shape[0], _dptr(aq).value, _dptr(asc).value, w.handle.value,
                           _dptr(c).value, c.shape[1])
    _check(load().ovh_linear_q_grouped(arr, len(problems), int(bool(accumulate)), _stream()))
    return outs


def set_f16_min_rows(rows: int) -> int:
    """ovh_set_f16_min_rows: GEMMs of at least `rows` rows (0: none, the
    default) run the f16-operand form, bit-identical to the int8 form; returns
    the previous setting."""
    return int(load().ovh_set_f16_min_rows(int(rows)))


def set_attention_long_min_tasks(tasks: int) -> int:
    """ovh_set_attention_long_min_tasks: from how many long-form workgroups the
    split attention takes its long-sequence kernel (default 384; 0: whenever
    the head grouping allows it); returns the previous setting."""
    return int(load().ovh_set_attention_long_min_tasks(int(tasks)))


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


def linear_f32(A, w: Weight, C=None, accumulate: bool = False):
    """Mat's fp32 branch: C (+)= A W on the f16 matrix cores (hi/lo splits)."""
    torch = _torch()
    M = A.shape[0]
    if C is None:
        C = torch.zeros((M, w.N), dtype=torch.float32, device="cuda")
    _check(load().ovh_linear_f32(M, _dptr(A), w.handle, _dptr(C), C.shape[1],
                                 int(bool(accumulate)), _stream()))
    return C


def block_dots(aq, w: Weight, M: int = None, tiled: bool = False):
    """Exact int32 per-(m, n, block) dot products from the kernel ovh_linear_q
    launches for the same shape; ``tiled``: aq holds tile-major codes (the LM
    runner's layout; pass M, since the buffer holds padded rows)."""
    torch = _torch()
    M = aq.shape[0] if M is None else M
    out = torch.empty((M, w.N, w.Kb), dtype=torch.int32, device="cuda")
    fn = load().ovh_block_dots_tiled if tiled else load().ovh_block_dots
    _check(fn(M, _dptr(aq), w.handle, _dptr(out), _stream()))
    return out


READ_DMA16, READ_DMA4, READ_VEC16, READ_BUF8 = 0, 1, 2, 3


def diag_read(t, path: int) -> None:
    """Read tensor t's bytes once through one load path of the GEMM kernels
    (READ_*), for calibrating hardware byte counters; t's size must be a
    multiple of 128 KiB."""
    _check(load().ovh_diag_read(_dptr(t), t.numel() * t.element_size(), path, _stream()))


def gate_up_weight(gate: Weight, up: Weight) -> Weight:
    """The SiLU-fused operand of gate and up [I, K] (ovh_weight_gate_up)."""
    h = C.c_void_p()
    _check(load().ovh_weight_gate_up(gate.handle, up.handle, _stream(), C.byref(h)))
    return Weight(h.value, 2 * gate.N, gate.K)


def silu_gate_linear(aq, asc, gate_up: Weight, out=None):
    """(hq int8 [M, I], hsc fp32 [M, I/32]) = quantised silu(aq.gate) * (aq.up),
    byte-identical to linear_q_sliced -> silu_mul_quantize (lm.cpp:293-311)."""
    torch = _torch()
    M, I = aq.shape[0], gate_up.N // 2
    if out is None:
        out = (torch.empty((M, I), dtype=torch.int8, device="cuda"),
               torch.empty((M, I // 32), dtype=torch.float32, device="cuda"))
    hq, hsc = out
    _check(load().ovh_silu_gate_linear(M, _dptr(aq), _dptr(asc), gate_up.handle, _dptr(hq),
                                       _dptr(hsc), _stream()))
    return hq, hsc


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
              out=None, split: bool = False):
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
    fn = load().ovh_attention_split if split else load().ovh_attention
    _check(fn(C.cast(arr, C.c_void_p), len(segs), n_heads, n_kv_heads, head_dim, _dptr(q),
              q.stride(0), _dptr(k), _dptr(v), k.stride(0), scale, _dptr(out), out.stride(0),
              _stream()))
    return out


# ---------------------------------------------------------------------------
# OVW1 files and the LM runner

class WeightFile:
    """An mmapped OVW1 checkpoint (ovh_ovw1_open = WeightFile::Open)."""

    def __init__(self, path: str):
        lib = load()
        h = C.c_void_p()
        _check(lib.ovh_ovw1_open(os.fsencode(path), C.byref(h)))
        self.handle = h
        n = lib.ovh_ovw1_count(h)
        base = lib.ovh_ovw1_tensors(h)
        self.views = (TensorView * n).from_address(base) if n else (TensorView * 0)()

    def __len__(self):
        return len(self.views)

    def names(self):
        return [v.name.decode() for v in self.views]

    def find(self, name: str):
        p = load().ovh_ovw1_find(self.handle, name.encode())
        return None if not p else TensorView.from_address(p)

    def crc_ok(self) -> bool:
        lib = load()
        return all(lib.ovh_ovw1_compute_crc(self.handle, i) == v.crc
                   for i, v in enumerate(self.views))

    def close(self):
        if self.handle:
            load().ovh_ovw1_close(self.handle)
            self.handle = None
            self.views = (TensorView * 0)()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def views_from_tensors(tensors):
    """TensorView array over host numpy arrays (ovw1.Tensor list); the returned
    keepalive list must outlive the views."""
    import numpy as np
    dt = {np.dtype(np.float32): 0, np.dtype(np.int8): 1, np.dtype(np.float16): 2,
          np.dtype(np.int64): 3}
    arr = (TensorView * len(tensors))()
    keep = []
    for i, t in enumerate(tensors):
        a = np.ascontiguousarray(t.array)
        name = t.name.encode()
        keep += [a, name]
        v = arr[i]
        v.name, v.dtype, v.ndim = name, dt[a.dtype], a.ndim
        for k in range(a.ndim):
            v.dims[k] = a.shape[k]
        v.transposed = 1 if t.layout == 1 else 0
        v.data, v.nbytes = a.ctypes.data, a.nbytes
        if t.scales is not None:
            sc = np.ascontiguousarray(t.scales, dtype=np.float32)
            keep.append(sc)
            v.quantized, v.scales, v.n_scales = 1, sc.ctypes.data, sc.size
    return arr, keep


class LM:
    """The HIP LM runner (ovh_lm_* = the accelerator plugin of cuda_lm.h); all
    work runs on torch's current stream at construction time."""

    def __init__(self, cfg: LmConfig, views, n: int):
        lib = load()
        self.cfg = cfg
        h = C.c_void_p()
        _check(lib.ovh_lm_create(C.byref(cfg), C.cast(views, C.c_void_p), n, _stream(),
                                 C.byref(h)))
        self.handle = h

    @classmethod
    def from_file(cls, path: str, cfg: LmConfig):
        wf = WeightFile(path)
        try:
            return cls(cfg, wf.views, len(wf))
        finally:
            wf.close()

    @classmethod
    def from_tensors(cls, tensors, cfg: LmConfig):
        views, keep = views_from_tensors(tensors)
        lm = cls(cfg, views, len(tensors))
        del keep
        return lm

    def forward(self, ids, audio_mask, attn_mask, pos, host_logits: bool = True):
        """ids [B, C, S] int64, audio_mask [B, S] u8, attn_mask [B, S, S] u8, pos [B, S]
        int64 (numpy); returns logits [B, C, S, V] (numpy) or None."""
        import numpy as np
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        am = np.ascontiguousarray(audio_mask, dtype=np.uint8)
        at = np.ascontiguousarray(attn_mask, dtype=np.uint8)
        pos = np.ascontiguousarray(pos, dtype=np.int64)
        B, Cb, S = ids.shape
        out = np.empty((B, Cb, S, self.cfg.audio_vocab), np.float32) if host_logits else None
        _check(load().ovh_lm_forward(self.handle, B, S, ids.ctypes.data, am.ctypes.data,
                                     at.ctypes.data, pos.ctypes.data,
                                     None if out is None else out.ctypes.data))
        return out

    def forward_cfg(self, cond_seq, uncond_seq, ids, audio_mask, cond_attn, uncond_attn, pos,
                    host_logits: bool = True):
        import numpy as np
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        am = np.ascontiguousarray(audio_mask, dtype=np.uint8)
        ca = np.ascontiguousarray(cond_attn, dtype=np.uint8)
        ua = np.ascontiguousarray(uncond_attn, dtype=np.uint8)
        pos = np.ascontiguousarray(pos, dtype=np.int64)
        rows = cond_seq + uncond_seq
        CV = self.cfg.n_codebooks * self.cfg.audio_vocab
        out = np.empty((rows, CV), np.float32) if host_logits else None
        _check(load().ovh_lm_forward_cfg(self.handle, cond_seq, uncond_seq, ids.ctypes.data,
                                         am.ctypes.data, ca.ctypes.data, ua.ctypes.data,
                                         pos.ctypes.data,
                                         None if out is None else out.ctypes.data))
        return out

    def last_logits_ptr(self) -> int:
        return load().ovh_lm_last_logits(self.handle) or 0

    def set_device_sampling(self, on: bool) -> None:
        load().ovh_lm_set_device_sampling(self.handle, int(bool(on)))

    def set_attention(self, split_f16: bool) -> None:
        load().ovh_lm_set_attention(self.handle, int(bool(split_f16)))

    def set_graphs(self, on: bool) -> None:
        """Replay the forward as a captured HIP graph (default) or launch its kernels one by one."""
        load().ovh_lm_set_graphs(self.handle, int(bool(on)))

    def set_fused_norm(self, on: bool) -> None:
        """Run each RMSNorm after o_proj / down in the same launch (default) or as its own."""
        load().ovh_lm_set_fused_norm(self.handle, int(bool(on)))

    def set_prefetch(self, on: bool) -> None:
        """Prefetch o_proj's weight into L2 from the attention launch (default) or not."""
        load().ovh_lm_set_prefetch(self.handle, int(bool(on)))

    def recovered(self) -> int:
        """Fallbacks the runner took after a forward's flags (RECOVERED_* bits)."""
        return load().ovh_lm_recovered(self.handle)

    def last_flags(self) -> int:
        """The condition bits behind the last recovery (ovh_lm_last_flags)."""
        return load().ovh_lm_last_flags(self.handle)

    def force_condition(self, what: int) -> None:
        """Test support: force FORCE_BAND_WAIT / FORCE_XCD on the next forward."""
        load().ovh_lm_force_condition(self.handle, int(what))

    def set_profile(self, on: bool) -> None:
        """Stage timer on (eager launches with HIP events between stages) or off."""
        load().ovh_lm_set_profile(self.handle, int(bool(on)))

    def stage_times(self) -> dict:
        """The last profiled forward's milliseconds per stage, in stage order."""
        lib = load()
        n = lib.ovh_lm_stage_times(self.handle, None, None, 0)
        ms = (C.c_double * max(n, 1))()
        names = (C.c_char_p * max(n, 1))()
        n = lib.ovh_lm_stage_times(self.handle, C.cast(ms, C.c_void_p), C.cast(names, C.c_void_p),
                                   n)
        return {names[i].decode(): float(ms[i]) for i in range(n)}

    def sample(self, cond_ptr: int, cond_seq: int, uncond_ptr: int, uncond_seq: int,
               target_len: int, guidance: float, layer_penalty: float):
        import numpy as np
        n = self.cfg.n_codebooks * target_len
        pred = np.empty(n, np.int32)
        scores = np.empty(n, np.float32)
        _check(load().ovh_lm_sample(self.handle, C.c_void_p(cond_ptr), cond_seq,
                                    C.c_void_p(uncond_ptr), uncond_seq, target_len, guidance,
                                    layer_penalty, pred.ctypes.data, scores.ctypes.data))
        return pred.reshape(self.cfg.n_codebooks, target_len), \
            scores.reshape(self.cfg.n_codebooks, target_len)

    def generate(self, prompt_ids, audio_mask, target_len: int, opts=None):
        """Pipeline::run_sampling on the device: prompt_ids [C, S] int64, audio_mask [S];
        returns tokens [C, target_len]."""
        import numpy as np
        ids = np.ascontiguousarray(prompt_ids, dtype=np.int64)
        am = np.ascontiguousarray(audio_mask, dtype=np.uint8)
        Cb, S = ids.shape
        out = np.empty((Cb, target_len), np.int64)
        o = opts if opts is not None else GenOptions()
        _check(load().ovh_lm_generate(self.handle, ids.ctypes.data, am.ctypes.data, S, target_len,
                                      C.byref(o), out.ctypes.data))
        return out

    def close(self):
        if getattr(self, "handle", None):
            load().ovh_lm_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
