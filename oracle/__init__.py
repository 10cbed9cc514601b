"""CPU oracle for the int8-nk quantized-linear path (TEST INFRASTRUCTURE ONLY).

Two numpy-facing bindings live here:

* ``Oracle``   — our C restatement (``oracle/ovoracle.c`` -> ``liboracle.so``),
  the parity checker for the HIP kernels and the "port" CPU baseline;
* ``Reference`` — the reference's own CPU kernels compiled from
  ``/root/reference/cpp/src/backend/cpu/{gemm,ops_cpu,conv_cpu}.cpp`` plus our
  extern "C" shim (``oracle/_ref/libovref.so``), used to pin the restatement and
  as the "reference" CPU baseline where its AVX-VNNI dispatch is available.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
import this package.  The product (``ovnative_amd``) never does.

Byte formats follow the reference: activations are quantised per 32-k block to
``u8 = q + 128`` (K tail padded with byte 0) with one fp32 scale per block
(``cpp/src/backend/cpu/gemm.cpp:379-430``); weights are int8 ``[N, K]`` with one
fp32 scale per output row (``tools/convert_weights.py:130-135``).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libovref.so")
REF_TREE = "/root/reference/cpp"

_i64 = C.c_int64
_f32 = C.c_float
_p = C.c_void_p


def build(ref: bool = True) -> None:
    """Compile liboracle.so (and oracle/_ref when the reference tree is mounted)."""
    subprocess.run(["make", "-s", "-B", "-C", HERE, "all"], check=True)
    if ref and os.path.isdir(REF_TREE):
        subprocess.run(["make", "-s", "-B", "-C", HERE, "ref"], check=True)


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def kb_of(K: int) -> int:
    return (K + 31) // 32


class Oracle:
    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            build(ref=False)
        self.lib = L = C.CDLL(path)
        sig = {
            "ovo_quant_bytes": (_i64, [_i64, _i64]),
            "ovo_quant_scales": (_i64, [_i64, _i64]),
            "ovo_quantize_weight_rows": (None, [_i64, _i64, _p, _p, _p]),
            "ovo_quantize_u8": (None, [_i64, _i64, _p, _p, _p]),
            "ovo_rmsnorm_f32": (None, [_p, _p, _p, _i64, _i64, _f32]),
            "ovo_rmsnorm_quantize_u8": (None, [_i64, _i64, _p, _p, _f32, _p, _p]),
            "ovo_exp256": (_f32, [_f32]),
            "ovo_silu_mul_f32": (None, [_p, _p, _p, _i64]),
            "ovo_silu_mul_quantize_u8": (None, [_i64, _i64, _p, _p, _p, _p]),
            "ovo_block_dots": (None, [_i64, _i64, _i64, _p, _p, _p]),
            "ovo_linear_q": (None, [_i64, _i64, _i64, _p, _p, _p, _p, _p, _i64, C.c_int]),
            "ovo_linear_f32": (None, [_i64, _i64, _i64, _p, _p, _p, _i64, C.c_int]),
            "ovo_packed_bytes": (_i64, [_i64, _i64]),
            "ovo_wsum_elems": (_i64, [_i64, _i64]),
            "ovo_pack": (None, [_i64, _i64, _p, _p, _p]),
            "ovo_fast_available": (C.c_int, []),
            "ovo_linear_q_packed": (C.c_int, [_i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _i64,
                                              C.c_int]),
            "ovo_num_threads": (C.c_int, []),
            "ovo_rope_tables": (None, [_i64, _p, C.c_int, _f32, _p, _p]),
            "ovo_qk_norm_rope": (C.c_int, [_p, _p, _p, _p, _i64, C.c_int, C.c_int, C.c_int, _p,
                                           _p, _f32]),
            "ovo_attention_head": (C.c_int, [_p, _i64, _p, _p, _i64, _p, C.c_int, C.c_int, _f32,
                                             _p, _i64]),
            "ovo_attention": (C.c_int, [C.c_int, _p, _p, _p, _p, C.c_int, C.c_int, C.c_int, _p,
                                        _p, _p, _f32, _p]),
            "ovo_embed": (C.c_int, [C.c_int, C.c_int, C.c_int, _i64, _p, _p, _p, _p, _p, _i64, _p,
                                    _p, _p, _i64, _p, _p]),
            "ovo_guided_sample": (C.c_int, [_p, C.c_int, _p, C.c_int, C.c_int, C.c_int, _f32, _f32,
                                            C.c_int, C.c_int, _p, _p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args

    # -- weights -----------------------------------------------------------
    def quantize_weight_rows(self, W: np.ndarray):
        W = np.ascontiguousarray(W, dtype=np.float32)
        N, K = W.shape
        q = np.empty((N, K), np.int8)
        s = np.empty(N, np.float32)
        self.lib.ovo_quantize_weight_rows(N, K, _ptr(W), _ptr(q), _ptr(s))
        return q, s

    # -- activation quantizers (reference u8 format) ------------------------
    def quantize(self, A: np.ndarray):
        A = np.ascontiguousarray(A, dtype=np.float32)
        M, K = A.shape
        aq = np.empty((M, kb_of(K) * 32), np.uint8)
        asc = np.empty((M, kb_of(K)), np.float32)
        self.lib.ovo_quantize_u8(M, K, _ptr(A), _ptr(aq), _ptr(asc))
        return aq, asc

    def rmsnorm(self, x: np.ndarray, w: np.ndarray, eps: float = 1e-6):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        out = np.empty_like(x)
        self.lib.ovo_rmsnorm_f32(_ptr(out), _ptr(x), _ptr(w), x.shape[0], x.shape[1], eps)
        return out

    def rmsnorm_quantize(self, x: np.ndarray, w: np.ndarray, eps: float = 1e-6):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        M, K = x.shape
        aq = np.empty((M, kb_of(K) * 32), np.uint8)
        asc = np.empty((M, kb_of(K)), np.float32)
        self.lib.ovo_rmsnorm_quantize_u8(M, K, _ptr(x), _ptr(w), eps, _ptr(aq), _ptr(asc))
        return aq, asc

    def exp256(self, x: float) -> float:
        return float(self.lib.ovo_exp256(x))

    def silu_mul(self, g: np.ndarray, u: np.ndarray):
        g = np.ascontiguousarray(g, dtype=np.float32)
        u = np.ascontiguousarray(u, dtype=np.float32)
        out = np.empty_like(g)
        self.lib.ovo_silu_mul_f32(_ptr(out), _ptr(g), _ptr(u), g.size)
        return out

    def silu_mul_quantize(self, g: np.ndarray, u: np.ndarray):
        g = np.ascontiguousarray(g, dtype=np.float32)
        u = np.ascontiguousarray(u, dtype=np.float32)
        M, K = g.shape
        aq = np.empty((M, kb_of(K) * 32), np.uint8)
        asc = np.empty((M, kb_of(K)), np.float32)
        self.lib.ovo_silu_mul_quantize_u8(M, K, _ptr(g), _ptr(u), _ptr(aq), _ptr(asc))
        return aq, asc

    # -- GEMM ----------------------------------------------------------------
    def block_dots(self, aq: np.ndarray, W: np.ndarray) -> np.ndarray:
        """int32 [M, N, Kb]: Σ_{k in block} (aq-128)·W[n,k]."""
        W = np.ascontiguousarray(W, dtype=np.int8)
        N, K = W.shape
        M = aq.shape[0]
        out = np.empty((M, N, kb_of(K)), np.int32)
        self.lib.ovo_block_dots(M, N, K, _ptr(aq), _ptr(W), _ptr(out))
        return out

    def linear_q(self, aq, asc, W, wscale, C=None, accumulate=False) -> np.ndarray:
        W = np.ascontiguousarray(W, dtype=np.int8)
        N, K = W.shape
        M = aq.shape[0]
        if C is None:
            C = np.zeros((M, N), np.float32)
        else:
            C = np.array(C, dtype=np.float32, copy=True, order="C")
        wscale = np.ascontiguousarray(wscale, dtype=np.float32)
        self.lib.ovo_linear_q(M, N, K, _ptr(aq), _ptr(asc), _ptr(W), _ptr(wscale), _ptr(C),
                              C.shape[1], int(bool(accumulate)))
        return C

    def linear_f32(self, A, W_kn, C=None, accumulate=False):
        """linear_f32_ld (gemm.cpp:884-905): C (+)= A W, W stored [K, N] fp32."""
        A = np.ascontiguousarray(A, dtype=np.float32)
        W_kn = np.ascontiguousarray(W_kn, dtype=np.float32)
        K, N = W_kn.shape
        M = A.shape[0]
        C = np.zeros((M, N), np.float32) if C is None else \
            np.array(C, dtype=np.float32, copy=True, order="C")
        self.lib.ovo_linear_f32(M, N, K, _ptr(A), _ptr(W_kn), _ptr(C), C.shape[1],
                                int(bool(accumulate)))
        return C

    def linear(self, A, W, wscale, C=None, accumulate=False):
        """Quantise fp32 activations, then linear_q (gemm.cpp:829-845 / :864-882)."""
        aq, asc = self.quantize(A)
        return self.linear_q(aq, asc, W, wscale, C, accumulate)

    # -- packed AVX-512 form (timing) ---------------------------------------
    def fast_available(self) -> bool:
        return bool(self.lib.ovo_fast_available())

    def pack(self, W: np.ndarray):
        W = np.ascontiguousarray(W, dtype=np.int8)
        N, K = W.shape
        packed = np.empty(self.lib.ovo_packed_bytes(N, K), np.int8)
        wsum = np.empty(self.lib.ovo_wsum_elems(N, K), np.int32)
        self.lib.ovo_pack(N, K, _ptr(W), _ptr(packed), _ptr(wsum))
        return packed, wsum

    def linear_q_packed(self, aq, asc, packed, wsum, N, K, wscale, C, accumulate=False):
        rc = self.lib.ovo_linear_q_packed(aq.shape[0], N, K, _ptr(aq), _ptr(asc), _ptr(packed),
                                          _ptr(wsum), _ptr(wscale), _ptr(C), C.shape[1],
                                          int(bool(accumulate)))
        if rc != 0:
            raise RuntimeError("AVX-512 VNNI not available on this host")
        return C

    def num_threads(self) -> int:
        return int(self.lib.ovo_num_threads())

    # -- the rest of the layer ----------------------------------------------
    def rope_tables(self, pos: np.ndarray, D: int, theta: float = 1e6):
        pos = np.ascontiguousarray(pos, dtype=np.int64)
        c = np.empty((pos.size, D // 2), np.float32)
        s = np.empty((pos.size, D // 2), np.float32)
        self.lib.ovo_rope_tables(pos.size, _ptr(pos), D, theta, _ptr(c), _ptr(s))
        return c, s

    def qk_norm_rope(self, q, k, qw, kw, n_heads, n_kv_heads, D, pos=None, theta=1e6,
                     eps=1e-6, tables=None):
        """Returns new (q, k); q [rows, n_heads*D], k [rows, n_kv_heads*D]."""
        q = np.array(q, dtype=np.float32, copy=True, order="C")
        k = np.array(k, dtype=np.float32, copy=True, order="C")
        qw = np.ascontiguousarray(qw, dtype=np.float32)
        kw = np.ascontiguousarray(kw, dtype=np.float32)
        c, s = tables if tables is not None else self.rope_tables(pos, D, theta)
        c = np.ascontiguousarray(c, dtype=np.float32)
        s = np.ascontiguousarray(s, dtype=np.float32)
        rc = self.lib.ovo_qk_norm_rope(_ptr(q), _ptr(k), _ptr(qw), _ptr(kw), q.shape[0],
                                       n_heads, n_kv_heads, D, _ptr(c), _ptr(s), eps)
        if rc != 0:
            raise ValueError("qk_norm_rope: head_dim/2 must be a multiple of 8")
        return q, k

    def attention_head(self, q, k, v, bias=None, scale=None):
        """q, k, v [S, D] (one head), bias [S, S] or None."""
        q = np.ascontiguousarray(q, dtype=np.float32)
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        S, D = q.shape
        scale = np.float32(1.0) / np.sqrt(np.float32(D)) if scale is None else scale
        out = np.empty((S, D), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        rc = self.lib.ovo_attention_head(_ptr(q), D, _ptr(k), _ptr(v), D,
                                         None if b is None else _ptr(b), S, D, float(scale),
                                         _ptr(out), D)
        if rc != 0:
            raise ValueError("attention_head: head_dim must be a multiple of 8")
        return out

    def attention(self, q, k, v, segs, n_heads, n_kv_heads, D, scale=None):
        """GQA over segments: segs = [(bias or None, rows, q_row0, kv_row0)] with row
        offsets into q [T, n_heads*D] and k/v [T, n_kv_heads*D]."""
        q = np.ascontiguousarray(q, dtype=np.float32)
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        scale = np.float32(1.0) / np.sqrt(np.float32(D)) if scale is None else scale
        out = np.zeros_like(q)
        n = len(segs)
        keep = [None if b is None else np.ascontiguousarray(b, dtype=np.float32)
                for b, *_ in segs]
        bias = (C.c_void_p * n)(*[None if b is None else b.ctypes.data for b in keep])
        rows = np.array([r for _, r, _, _ in segs], np.int32)
        qo = np.array([qr * n_heads * D for _, _, qr, _ in segs], np.int64)
        ko = np.array([kr * n_kv_heads * D for _, _, _, kr in segs], np.int64)
        rc = self.lib.ovo_attention(n, C.cast(bias, C.c_void_p), _ptr(rows), _ptr(qo), _ptr(ko),
                                    n_heads, n_kv_heads, D, _ptr(q), _ptr(k), _ptr(v),
                                    float(scale), _ptr(out))
        if rc != 0:
            raise ValueError("attention: bad head configuration")
        return out

    def embed(self, ids, mask, tok, aud, offsets, tok_scale=None, aud_scale=None):
        """ids [B, C, S] int64, mask [B, S] u8; tables fp32, or int8 with per-row scales."""
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        mask = np.ascontiguousarray(mask, dtype=np.uint8)
        offsets = np.ascontiguousarray(offsets, dtype=np.int64)
        B, Cb, S = ids.shape
        H = tok.shape[1]
        out = np.empty((B * S, H), np.float32)
        tf = tok if tok.dtype == np.float32 else None
        af = aud if aud.dtype == np.float32 else None
        tq = None if tf is not None else np.ascontiguousarray(tok, dtype=np.int8)
        aqq = None if af is not None else np.ascontiguousarray(aud, dtype=np.int8)
        ptr = lambda a: None if a is None else _ptr(np.ascontiguousarray(a))
        rc = self.lib.ovo_embed(B, S, Cb, H, _ptr(ids), _ptr(mask), ptr(tf), ptr(tq),
                                ptr(tok_scale), tok.shape[0], ptr(af), ptr(aqq), ptr(aud_scale),
                                aud.shape[0], _ptr(offsets), _ptr(out))
        if rc != 0:
            raise ValueError("embed: id out of range")
        return out

    def guided_sample(self, cond, cond_seq, uncond, C_, V, target_len, guidance, layer_penalty,
                      mask_id=None, cpu_alias=False):
        """cond [cond_seq, C*V], uncond [>= target_len, C*V] token-major logit planes.
        cpu_alias=True reproduces tts.cpp's in-place log_softmax quirk (host path);
        the default is the device sampler's arithmetic (cuda_lm.cu:720-756)."""
        cond = np.ascontiguousarray(cond, dtype=np.float32)
        uncond = np.ascontiguousarray(uncond, dtype=np.float32)
        n = C_ * target_len
        pred = np.empty(n, np.int32)
        scores = np.empty(n, np.float32)
        rc = self.lib.ovo_guided_sample(_ptr(cond), cond_seq, _ptr(uncond), C_, V, target_len,
                                        guidance, layer_penalty, V - 1 if mask_id is None else mask_id,
                                        int(bool(cpu_alias)), _ptr(pred), _ptr(scores))
        if rc != 0:
            raise ValueError("guided_sample: bad sizes")
        return pred.reshape(C_, target_len), scores.reshape(C_, target_len)

    # -- the LM forward, composed from the restated pieces ------------------
    def _linear_fast(self, aq, asc, W, wscale, C=None, accumulate=False):
        """linear_q through the AVX-512 VNNI form when the host has it (same bits,
        tests/test_oracle.py::test_fast_path_matches_scalar)."""
        if not self.fast_available():
            return self.linear_q(aq, asc, W, wscale, C, accumulate)
        N, K = W.shape
        packed, wsum = self.pack(W)
        out = np.zeros((aq.shape[0], N), np.float32) if C is None else \
            np.array(C, dtype=np.float32, copy=True, order="C")
        return self.linear_q_packed(aq, asc, packed, wsum, N, K,
                                    np.ascontiguousarray(wscale, dtype=np.float32), out, accumulate)

    def lm_forward(self, cfg, tensors, ids, audio_mask, segs, pos, attention=None):
        """LM::run_layer / forward (cpp/src/model/lm.cpp:217-401) on the int8-nk
        path: `tensors` maps the reference's tensor names to (array, scales,
        transposed); ids [B, C, S]; segs = [(mask [rows, rows] u8 or None, rows,
        row0)]; pos [T].  Returns logits [T, C*V] token-major.  `attention`, if
        given, replaces the attention step: attention(q, k, v, segs) -> out (the
        tests pass the device kernel here to isolate every other step)."""
        g = lambda n: tensors[n]

        def lin(name):
            a, sc, tr = g(name)
            return (np.ascontiguousarray(a.T) if tr else a), sc

        H, NH, NKV, D = cfg["hidden"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
        eps, theta = cfg.get("rms_eps", 1e-6), cfg.get("rope_theta", 1e6)
        tok, tok_s, _ = g("llm.embed_tokens.weight")
        aud, aud_s, _ = g("audio_embeddings.weight")
        offs = g("codebook_layer_offsets")[0]
        x = self.embed(ids, audio_mask, tok, aud, offs, tok_s, aud_s)
        tables = self.rope_tables(pos, D, theta)
        asegs = [(None if m is None else np.where(m != 0, 0.0, -1e30).astype(np.float32), r, r0, r0)
                 for m, r, r0 in segs]
        for li in range(cfg["n_layers"]):
            p = f"llm.layers.{li}."
            aq, asc = self.rmsnorm_quantize(x, g(p + "input_layernorm.weight")[0], eps)
            lq = self._linear_fast
            q = lq(aq, asc, *lin(p + "self_attn.q_proj.weight"))
            k = lq(aq, asc, *lin(p + "self_attn.k_proj.weight"))
            v = lq(aq, asc, *lin(p + "self_attn.v_proj.weight"))
            q, k = self.qk_norm_rope(q, k, g(p + "self_attn.q_norm.weight")[0],
                                     g(p + "self_attn.k_norm.weight")[0], NH, NKV, D, eps=eps,
                                     tables=tables)
            att = (self.attention(q, k, v, asegs, NH, NKV, D) if attention is None
                   else attention(q, k, v, asegs))
            aq, asc = self.quantize(att)
            x = lq(aq, asc, *lin(p + "self_attn.o_proj.weight"), C=x, accumulate=True)
            aq, asc = self.rmsnorm_quantize(x, g(p + "post_attention_layernorm.weight")[0], eps)
            gate = lq(aq, asc, *lin(p + "mlp.gate_proj.weight"))
            up = lq(aq, asc, *lin(p + "mlp.up_proj.weight"))
            aq, asc = self.silu_mul_quantize(gate, up)
            x = lq(aq, asc, *lin(p + "mlp.down_proj.weight"), C=x, accumulate=True)
        head, head_s, head_t = g("audio_heads.weight")
        if head_s is None:
            # the fp32 head of the reference's default int8 checkpoint, stored
            # [K, N] (lm.cpp:383-385: rmsnorm_f32, then Mat's fp32 branch)
            if not head_t:
                raise ValueError("audio_heads.weight: an fp32 head must be stored [K, N]")
            return self.linear_f32(self.rmsnorm(x, g("llm.norm.weight")[0], eps), head)
        aq, asc = self.rmsnorm_quantize(x, g("llm.norm.weight")[0], eps)
        return self._linear_fast(aq, asc, *lin("audio_heads.weight"))


class Reference:
    """The reference's compiled CPU kernels (see ``oracle/ref_shim.cpp``)."""

    def __init__(self, path: str = REF_LIB_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.lib = L = C.CDLL(path)
        sig = {
            "ovref_vnni_available": (C.c_int, []),
            "ovref_kernel_name": (C.c_char_p, []),
            "ovref_enable_ftz": (None, []),
            "ovref_s8_nk_quantize": (C.c_int, [_i64, _i64, _p, _p, _p]),
            "ovref_rmsnorm_quantize": (C.c_int, [_i64, _i64, _p, _p, _f32, _p, _p]),
            "ovref_silu_mul_quantize": (C.c_int, [_i64, _i64, _p, _p, _p, _p]),
            "ovref_rmsnorm_into": (None, [_p, _p, _p, _i64, _i64, _f32]),
            "ovref_silu_mul": (None, [_p, _p, _p, _i64]),
            "ovref_packed_bytes": (_i64, [_i64, _i64]),
            "ovref_wsum_elems": (_i64, [_i64, _i64]),
            "ovref_pack": (None, [_i64, _i64, _p, _p, _p]),
            "ovref_linear_packed_q": (C.c_int, [_i64, _i64, _i64, _p, _p, _p, _p, _p, _p,
                                                C.c_int]),
            "ovref_linear_packed": (C.c_int, [_i64, _i64, _i64, _p, _p, _p, _p, _p, C.c_int]),
            "ovref_linear_f32": (C.c_int, [_i64, _i64, _i64, _p, _p, _p, _i64, C.c_int]),
            "ovref_linear_packed_q_sliced": (C.c_int, [_i64, _i64, _p, _p, _p, _p, _p, _p, _p,
                                                       C.c_int]),
            "ovref_qk_norm_rope": (None, [_p, _p, _p, _p, _i64, C.c_int, C.c_int, C.c_int, _p,
                                          _f32, _f32]),
            "ovref_attention_head": (None, [_p, _i64, _p, _p, _i64, _p, C.c_int, C.c_int, _f32,
                                            _p, _i64]),
            "ovref_ovw1_open": (_p, [C.c_char_p, C.c_char_p, C.c_size_t]),
            "ovref_ovw1_close": (None, [_p]),
            "ovref_ovw1_count": (C.c_int, [_p]),
            "ovref_ovw1_get": (C.c_int, [_p, C.c_char_p] + [_p] * 11),
            "ovref_lm_open": (_p, [C.c_char_p] + [C.c_int] * 9 + [_f32, _f32, C.c_char_p,
                                                                  C.c_size_t]),
            "ovref_lm_close": (None, [_p]),
            "ovref_lm_forward": (C.c_int, [_p, C.c_int, C.c_int, _p, _p, _p, _p, _p]),
            "ovref_lm_forward_cfg": (C.c_int, [_p, C.c_int, C.c_int, _p, _p, _p, _p, _p, _p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args

    def vnni_available(self) -> bool:
        return bool(self.lib.ovref_vnni_available())

    def lm_open(self, path, cfg):
        """The reference LM (lm.cpp) on an OVW1 checkpoint; cfg = LMConfig fields."""
        err = C.create_string_buffer(512)
        keys = ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim", "inter", "vocab",
                "audio_vocab", "n_codebooks")
        h = self.lib.ovref_lm_open(os.fsencode(path), *[int(cfg[k]) for k in keys],
                                   float(cfg.get("rms_eps", 1e-6)),
                                   float(cfg.get("rope_theta", 1e6)), err, 512)
        if not h:
            raise RuntimeError(err.value.decode())
        return h

    def lm_close(self, h):
        self.lib.ovref_lm_close(h)

    def lm_forward(self, h, cfg, ids, audio_mask, attn_mask, pos):
        """LM::forward: returns logits [B, C, S, V]."""
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        am = np.ascontiguousarray(audio_mask, dtype=np.uint8)
        at = np.ascontiguousarray(attn_mask, dtype=np.uint8)
        pos = np.ascontiguousarray(pos, dtype=np.int64)
        B, Cb, S = ids.shape
        out = np.empty((B, Cb, S, int(cfg["audio_vocab"])), np.float32)
        if self.lib.ovref_lm_forward(h, B, S, _ptr(ids), _ptr(am), _ptr(at), _ptr(pos), _ptr(out)):
            raise RuntimeError("reference LM::forward failed")
        return out

    def ovw1_read(self, path, names):
        """Open `path` with the reference loader (WeightFile::Open); returns
        (n_tensors, {name: dict(dtype, dims, transposed, quantized, data bytes,
        scales, stored_crc, computed_crc)}).  Raises RuntimeError with the
        loader's message on a format error."""
        err = C.create_string_buffer(512)
        h = self.lib.ovref_ovw1_open(os.fsencode(path), err, 512)
        if not h:
            raise RuntimeError(err.value.decode())
        try:
            out = {}
            for name in names:
                dt, nd, tr, qu = C.c_int(), C.c_int(), C.c_int(), C.c_int()
                dims = (C.c_int64 * 4)()
                data, sc = C.c_void_p(), C.c_void_p()
                nb, ns = C.c_int64(), C.c_int64()
                scrc, ccrc = C.c_uint32(), C.c_uint32()
                rc = self.lib.ovref_ovw1_get(h, name.encode(), C.byref(dt), C.byref(nd), dims,
                                             C.byref(tr), C.byref(qu), C.byref(data), C.byref(nb),
                                             C.byref(sc), C.byref(ns), C.byref(scrc),
                                             C.byref(ccrc))
                if rc != 0:
                    out[name] = None
                    continue
                raw = C.string_at(data.value, nb.value) if nb.value else b""
                scales = (np.frombuffer(C.string_at(sc.value, 4 * ns.value), np.float32).copy()
                          if qu.value and ns.value else None)
                out[name] = dict(dtype=dt.value, dims=tuple(dims[:nd.value]), transposed=tr.value,
                                 quantized=qu.value, data=raw, scales=scales,
                                 stored_crc=scrc.value, computed_crc=ccrc.value)
            return self.lib.ovref_ovw1_count(h), out
        finally:
            self.lib.ovref_ovw1_close(h)

    def qk_norm_rope(self, q, k, qw, kw, n_heads, n_kv_heads, D, pos, theta=1e6, eps=1e-6):
        q = np.array(q, dtype=np.float32, copy=True, order="C")
        k = np.array(k, dtype=np.float32, copy=True, order="C")
        qw = np.ascontiguousarray(qw, dtype=np.float32)
        kw = np.ascontiguousarray(kw, dtype=np.float32)
        pos = np.ascontiguousarray(pos, dtype=np.int64)
        self.lib.ovref_qk_norm_rope(_ptr(q), _ptr(k), _ptr(qw), _ptr(kw), q.shape[0], n_heads,
                                    n_kv_heads, D, _ptr(pos), theta, eps)
        return q, k

    def attention_head(self, q, k, v, bias=None, scale=None):
        q = np.ascontiguousarray(q, dtype=np.float32)
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        S, D = q.shape
        scale = np.float32(1.0) / np.sqrt(np.float32(D)) if scale is None else scale
        out = np.empty((S, D), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        self.lib.ovref_attention_head(_ptr(q), D, _ptr(k), _ptr(v), D,
                                      None if b is None else _ptr(b), S, D, float(scale),
                                      _ptr(out), D)
        return out

    def kernel_name(self) -> str:
        return self.lib.ovref_kernel_name().decode()

    def quantize(self, A):
        A = np.ascontiguousarray(A, dtype=np.float32)
        M, K = A.shape
        aq = np.empty((M, kb_of(K) * 32), np.uint8)
        asc = np.empty((M, kb_of(K)), np.float32)
        if self.lib.ovref_s8_nk_quantize(M, K, _ptr(A), _ptr(aq), _ptr(asc)) != 0:
            raise RuntimeError("reference s8_nk_quantize failed")
        return aq, asc

    def rmsnorm_quantize(self, x, w, eps=1e-6):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        M, K = x.shape
        aq = np.empty((M, kb_of(K) * 32), np.uint8)
        asc = np.empty((M, kb_of(K)), np.float32)
        if self.lib.ovref_rmsnorm_quantize(M, K, _ptr(x), _ptr(w), eps, _ptr(aq), _ptr(asc)):
            raise RuntimeError("reference rmsnorm_quantize failed")
        return aq, asc

    def silu_mul_quantize(self, g, u):
        g = np.ascontiguousarray(g, dtype=np.float32)
        u = np.ascontiguousarray(u, dtype=np.float32)
        M, K = g.shape
        aq = np.empty((M, kb_of(K) * 32), np.uint8)
        asc = np.empty((M, kb_of(K)), np.float32)
        if self.lib.ovref_silu_mul_quantize(M, K, _ptr(g), _ptr(u), _ptr(aq), _ptr(asc)):
            raise RuntimeError("reference silu_mul_quantize failed")
        return aq, asc

    def rmsnorm(self, x, w, eps=1e-6):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        out = np.empty_like(x)
        self.lib.ovref_rmsnorm_into(_ptr(out), _ptr(x), _ptr(w), x.shape[0], x.shape[1], eps)
        return out

    def silu_mul(self, g, u):
        g = np.ascontiguousarray(g, dtype=np.float32)
        u = np.ascontiguousarray(u, dtype=np.float32)
        out = np.empty_like(g)
        self.lib.ovref_silu_mul(_ptr(out), _ptr(g), _ptr(u), g.size)
        return out

    def pack(self, W):
        W = np.ascontiguousarray(W, dtype=np.int8)
        N, K = W.shape
        packed = np.empty(self.lib.ovref_packed_bytes(N, K), np.int8)
        wsum = np.empty(self.lib.ovref_wsum_elems(N, K), np.int32)
        self.lib.ovref_pack(N, K, _ptr(W), _ptr(packed), _ptr(wsum))
        return packed, wsum

    def linear_q_packed(self, aq, asc, packed, wsum, N, K, wscale, C, accumulate=False):
        wscale = np.ascontiguousarray(wscale, dtype=np.float32)
        if self.lib.ovref_linear_packed_q(aq.shape[0], N, K, _ptr(aq), _ptr(asc), _ptr(packed),
                                          _ptr(wsum), _ptr(wscale), _ptr(C),
                                          int(bool(accumulate))):
            raise RuntimeError("reference linear_s8_nk_packed_q failed")
        return C

    def linear_q(self, aq, asc, W, wscale, C=None, accumulate=False):
        W = np.ascontiguousarray(W, dtype=np.int8)
        N, K = W.shape
        packed, wsum = self.pack(W)
        if C is None:
            C = np.zeros((aq.shape[0], N), np.float32)
        else:
            C = np.array(C, dtype=np.float32, copy=True, order="C")
        return self.linear_q_packed(aq, asc, packed, wsum, N, K, wscale, C, accumulate)

    def linear(self, A, W, wscale, C=None, accumulate=False):
        A = np.ascontiguousarray(A, dtype=np.float32)
        W = np.ascontiguousarray(W, dtype=np.int8)
        N, K = W.shape
        packed, wsum = self.pack(W)
        C = np.zeros((A.shape[0], N), np.float32) if C is None else np.array(C, np.float32)
        wscale = np.ascontiguousarray(wscale, dtype=np.float32)
        if self.lib.ovref_linear_packed(A.shape[0], N, K, _ptr(A), _ptr(packed), _ptr(wsum),
                                        _ptr(wscale), _ptr(C), int(bool(accumulate))):
            raise RuntimeError("reference linear_s8_nk_packed failed")
        return C

    def block_dots(self, aq, W):
        """Per-block int32 through the reference's public API: with asc one-hot on
        block b and wscale = 1, the epilogue returns fma(float(acc_b), 1, 0) =
        float(acc_b), exact because |acc_b| < 2^24."""
        W = np.ascontiguousarray(W, dtype=np.int8)
        N, K = W.shape
        M, Kb = aq.shape[0], kb_of(K)
        packed, wsum = self.pack(W)
        ones = np.ones(N, np.float32)
        out = np.empty((M, N, Kb), np.int32)
        for b in range(Kb):
            asc = np.zeros((M, Kb), np.float32)
            asc[:, b] = 1.0
            C = np.zeros((M, N), np.float32)
            self.linear_q_packed(aq, asc, packed, wsum, N, K, ones, C)
            out[:, :, b] = C.astype(np.int32)
        return out

    def linear_f32(self, A, W_kn, C=None, accumulate=False):
        A = np.ascontiguousarray(A, dtype=np.float32)
        W_kn = np.ascontiguousarray(W_kn, dtype=np.float32)
        K, N = W_kn.shape
        M = A.shape[0]
        C = np.zeros((M, N), np.float32) if C is None else \
            np.array(C, dtype=np.float32, copy=True, order="C")
        if self.lib.ovref_linear_f32(M, N, K, _ptr(A), _ptr(W_kn), _ptr(C), C.shape[1],
                                     int(bool(accumulate))):
            raise RuntimeError("reference linear_f32_ld failed")
        return C

    def linear_q_sliced(self, aq, asc, W_slices, scale_slices):
        """Merged [sum N, K] matrix with one C per slice (gemm.cpp:776-827)."""
        K = W_slices[0].shape[1]
        Wc = np.ascontiguousarray(np.concatenate(W_slices, axis=0), dtype=np.int8)
        sc = np.ascontiguousarray(np.concatenate(scale_slices), dtype=np.float32)
        packed, wsum = self.pack(Wc)
        Ns = np.array([w.shape[0] for w in W_slices], np.int64)
        outs = [np.zeros((aq.shape[0], int(n)), np.float32) for n in Ns]
        ptrs = (C.c_void_p * len(outs))(*[o.ctypes.data for o in outs])
        rc = self.lib.ovref_linear_packed_q_sliced(aq.shape[0], K, _ptr(aq), _ptr(asc),
                                                   _ptr(packed), _ptr(wsum), _ptr(sc),
                                                   _ptr(Ns), C.cast(ptrs, C.c_void_p),
                                                   len(outs))
        if rc == -2:
            raise ValueError("sliced GEMM: each slice N must be a positive multiple of 64")
        if rc != 0:
            raise RuntimeError("reference sliced GEMM failed")
        return outs


def reference_available() -> bool:
    return os.path.exists(REF_LIB_PATH)


# ---------------------------------------------------------------------------
# The CFG decoding loop's host logic (cpp/src/model/tts.cpp:165-364), for the
# tests of ovh_lm_generate.  The per-step forward + guided argmax is passed in
# (the tests pass the device runner's own, so only this logic is compared).

def mt19937_u32(seed: int, n: int) -> np.ndarray:
    """n raw outputs of std::mt19937(seed) (init_genrand seeding = numpy's legacy
    integer seeding; pinned by the C++ standard's known answer, [rand.predef])."""
    bg = np.random.MT19937()
    bg._legacy_seeding(seed)
    return bg.random_raw(n).astype(np.uint32)


def uniform_float01(x: np.ndarray) -> np.ndarray:
    """std::uniform_real_distribution<float>(0, 1) on one 32-bit draw each, as
    libstdc++'s generate_canonical<float, 24> computes it: float(x) / 2^32,
    values rounding up to 1 replaced by nextafter(1, 0)."""
    r = np.asarray(x, np.uint32).astype(np.float32) / np.float32(4294967296.0)
    return np.where(r >= 1, np.nextafter(np.float32(1), np.float32(0)), r).astype(np.float32)


def cfg_schedule(num_steps: int, t_shift: float, total: int):
    """tts.cpp:231-249: shifted time grid in double from the float option, per-step
    counts (the last takes the rest)."""
    import math
    t_shift = float(np.float32(t_shift))  # TtsOptions::t_shift is a float
    ts = [t_shift * (i / num_steps) / (1.0 + (t_shift - 1.0) * (i / num_steps))
          for i in range(num_steps + 1)]
    sched, rem = [], total
    for s in range(num_steps):
        num = rem if s == num_steps - 1 else min(math.ceil(total * (ts[s + 1] - ts[s])), rem)
        sched.append(int(num))
        rem -= num
    return sched


def run_sampling(step_fn, prompt_ids, audio_mask, target_len, C_, V, num_steps=32,
                 guidance=2.0, t_shift=0.1, layer_penalty=5.0, position_temperature=5.0,
                 seed=1234):
    """tts.cpp:165-364 (accelerator branch).  step_fn(ids, amask, attn, pos) ->
    (pred [C, T], scores [C, T]) runs the B = 2 forward and the guided argmax."""
    libm = C.CDLL("libm.so.6")
    libm.logf.restype = C.c_float
    libm.logf.argtypes = [C.c_float]
    S, T = prompt_ids.shape[1], target_len
    mask_id = V - 1
    ids = np.full((2, C_, S), mask_id, np.int64)
    ids[0] = prompt_ids
    ids[1, :, :T] = prompt_ids[:, S - T:]
    am = np.zeros((2, S), np.uint8)
    am[0] = audio_mask
    am[1, :T] = 1
    attn = np.zeros((2, S, S), np.uint8)
    attn[0] = 1
    attn[1, :T, :T] = 1
    attn[1, np.arange(T, S), np.arange(T, S)] = 1
    pos = np.tile(np.arange(S, dtype=np.int64), (2, 1))
    tokens = np.full(C_ * T, mask_id, np.int64)
    draws = iter(uniform_float01(mt19937_u32(seed, num_steps * C_ * T + 1)))
    for k in cfg_schedule(num_steps, t_shift, C_ * T):
        if k <= 0:
            continue
        pred, scores = step_fn(ids, am, attn, pos)
        pred = pred.reshape(-1)
        scores = scores.reshape(-1).astype(np.float32).copy()
        for i in range(scores.size):
            u = max(float(next(draws)), float(np.float32(1e-10)))
            inner = np.float32(-np.float32(libm.logf(u))) + np.float32(1e-10)
            g = -np.float32(libm.logf(float(inner)))
            scores[i] = np.float32(scores[i] / np.float32(position_temperature)) + g
        scores[tokens != mask_id] = -np.inf
        order = np.argsort(-scores, kind="stable")
        for idx in order[:min(k, scores.size)]:
            if not np.isfinite(scores[idx]):
                break
            tokens[idx] = pred[idx]
            c, t = divmod(int(idx), T)
            ids[0, c, S - T + t] = pred[idx]
            ids[1, c, t] = pred[idx]
    return tokens.reshape(C_, T)
