"""Write the golden vectors for the int8-nk path from the COMPILED REFERENCE.

Run in the build container (where /root/reference is mounted):

    make -C oracle ref && python tests/golden/gen_golden.py

Every expected output below comes from the reference's own CPU kernels
(cpp/src/backend/cpu/gemm.cpp, ops_cpu.cpp), compiled from source by
oracle/Makefile into oracle/_ref/libovref.so and called through its public API
(ov_gemm.h).  Inputs are seeded synthetic data shaped like the reference's own
tests (cpp/tests/test_gemm.cpp:462-508: tails in M%4, N%8, K%32) plus one
slice of BASELINE config 1 (K=1024 with 8 outlier channels x20).  The files
are plain .npz (no pickles): inputs and expected outputs only.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import Reference  # noqa: E402


def act(rng, M, K, outliers=0, scale=1.0):
    A = (rng.standard_normal((M, K)) * scale).astype(np.float32)
    if outliers:
        cols = rng.choice(K, size=min(outliers, K), replace=False)
        A[:, cols] *= 20.0
    return A


def main() -> None:
    ref = Reference()
    assert ref.vnni_available(), "the reference's VNNI path must be live to generate fixtures"
    rng = np.random.default_rng(20261201)
    out = {}

    # -- s8_nk_quantize (gemm.cpp:379-430) -------------------------------------
    qcases = [(4, 16), (5, 33), (9, 69), (1, 9), (2, 1024), (7, 13), (3, 3072), (16, 1024)]
    for i, (M, K) in enumerate(qcases):
        A = act(rng, M, K, outliers=2 if K >= 32 else 0)
        if i == 1:
            A[1, :32] = 0.0          # an all-zero block: scale 0, codes 128
        if i == 2:
            A[0, 40] = 1e-41         # a subnormal in a block of normals
        aq, asc = ref.quantize(A)
        out[f"quant{i}_A"], out[f"quant{i}_aq"], out[f"quant{i}_asc"] = A, aq, asc

    # -- rmsnorm_quantize_f32 (gemm.cpp:638-707) ---------------------------------
    rcases = [(7, 33), (8, 1024), (3, 7), (5, 69), (4, 12), (6, 3072)]
    for i, (M, K) in enumerate(rcases):
        x = act(rng, M, K, scale=rng.uniform(0.2, 8.0))
        w = rng.uniform(0.1, 1.1, K).astype(np.float32)
        aq, asc = ref.rmsnorm_quantize(x, w, 1e-6)
        out[f"rms{i}_x"], out[f"rms{i}_w"] = x, w
        out[f"rms{i}_aq"], out[f"rms{i}_asc"] = aq, asc
        out[f"rms{i}_xn"] = ref.rmsnorm(x, w, 1e-6)   # rmsnorm_into_f32 (ops_cpu.cpp:38-62)

    # -- silu_mul_quantize_f32 (ops_cpu.cpp:144-198) -------------------------------
    scases = [(7, 69), (8, 1024), (3, 3072), (2, 40)]
    for i, (M, K) in enumerate(scases):
        g = (rng.standard_normal((M, K)) * 4.0).astype(np.float32)
        u = rng.standard_normal((M, K)).astype(np.float32)
        g[0, :4] = [-100.0, 100.0, 0.0, -0.0]   # clamp ends of exp256 and signed zeros
        aq, asc = ref.silu_mul_quantize(g, u)
        out[f"silu{i}_g"], out[f"silu{i}_u"] = g, u
        out[f"silu{i}_aq"], out[f"silu{i}_asc"] = aq, asc
        out[f"silu{i}_act"] = ref.silu_mul(g, u)   # silu_mul_f32 (ops_cpu.cpp:126-136)

    # -- linear_s8_nk_packed_q / _q_add + per-block int32 (gemm.cpp:432-504) -------
    gcases = [(4, 8, 16), (5, 17, 33), (9, 7, 69), (1, 33, 9), (7, 69, 33), (2, 128, 1024),
              (16, 96, 1024)]
    for i, (M, N, K) in enumerate(gcases):
        A = act(rng, M, K, outliers=8 if K >= 1024 else 1)
        W = rng.integers(-127, 128, (N, K)).astype(np.int8)
        ws = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
        Cin = rng.standard_normal((M, N)).astype(np.float32)
        aq, asc = ref.quantize(A)
        out[f"gemm{i}_A"], out[f"gemm{i}_W"], out[f"gemm{i}_ws"], out[f"gemm{i}_Cin"] = A, W, ws, Cin
        out[f"gemm{i}_C"] = ref.linear_q(aq, asc, W, ws)
        out[f"gemm{i}_Cadd"] = ref.linear_q(aq, asc, W, ws, Cin, accumulate=True)
        if M * N * K <= 300_000:
            out[f"gemm{i}_blocks"] = ref.block_dots(aq, W)

    # -- BASELINE config 1 slice: weights from fp32 via the OVW1 quantiser ----------
    Wf = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float32)
    A = act(rng, 8, 1024, outliers=8)
    from oracle import Oracle
    q, s = Oracle().quantize_weight_rows(Wf)   # pinned separately by tests/test_oracle.py
    aq, asc = ref.quantize(A)
    out["c1_A"], out["c1_Wf"], out["c1_q"], out["c1_s"] = A, Wf, q, s
    out["c1_C"] = ref.linear_q(aq, asc, q, s)

    # -- linear_s8_nk_packed_q_sliced (gemm.cpp:776-827) -----------------------------
    A = act(rng, 7, 96)
    Ws = [rng.integers(-127, 128, (n, 96)).astype(np.int8) for n in (128, 64, 64)]
    ss = [rng.uniform(1e-4, 1e-2, w.shape[0]).astype(np.float32) for w in Ws]
    aq, asc = ref.quantize(A)
    outs = ref.linear_q_sliced(aq, asc, Ws, ss)
    out["sl_A"] = A
    for j, (w, s_, o) in enumerate(zip(Ws, ss, outs)):
        out[f"sl_W{j}"], out[f"sl_s{j}"], out[f"sl_C{j}"] = w, s_, o

    # -- qk_norm_rope_f32 (ops_cpu.cpp:945-1016, tables built from positions) ------
    for i, (rows, nh, nkv, D) in enumerate([(5, 4, 2, 128), (3, 2, 1, 64), (4, 16, 8, 128)]):
        q = (rng.standard_normal((rows, nh * D)) * rng.uniform(0.5, 4.0)).astype(np.float32)
        k = rng.standard_normal((rows, nkv * D)).astype(np.float32)
        qw = rng.uniform(0.3, 1.7, D).astype(np.float32)
        kw = rng.uniform(0.3, 1.7, D).astype(np.float32)
        pos = rng.integers(0, 4000, rows).astype(np.int64)
        pos[0] = 0                                  # cos 1, sin 0: the norm alone
        qo, ko = ref.qk_norm_rope(q, k, qw, kw, nh, nkv, D, pos, 1e6, 1e-6)
        for name, arr in dict(q=q, k=k, qw=qw, kw=kw, pos=pos, qo=qo, ko=ko).items():
            out[f"qknr{i}_{name}"] = arr
        out[f"qknr{i}_dims"] = np.array([rows, nh, nkv, D], np.int64)

    # -- attention_head_f32 (ops_cpu.cpp:907-943 -> :586-786) ----------------------
    acases = [(1, 128, 1.0, False), (7, 128, 1.0, True), (33, 128, 3.0, True),
              (70, 128, 12.0, False), (19, 64, 1.0, True)]
    for i, (S, D, mag, masked) in enumerate(acases):
        q = (rng.standard_normal((S, D)) * mag).astype(np.float32)
        k = rng.standard_normal((S, D)).astype(np.float32)
        v = rng.standard_normal((S, D)).astype(np.float32)
        bias = np.zeros((S, S), np.float32)
        if masked:
            bias[rng.random((S, S)) < 0.4] = -1e30
            bias[0, :] = -1e30                      # a fully masked row -> zeros
        o = ref.attention_head(q, k, v, bias if masked else None)
        for name, arr in dict(q=q, k=k, v=v, bias=bias, out=o).items():
            out[f"attn{i}_{name}"] = arr
        out[f"attn{i}_masked"] = np.array(int(masked), np.int64)

    # -- linear_f32_ld (gemm.cpp:884-905): Mat's fp32 branch, W [K, N] ---------
    # (the fp32 audio head of the default int8 checkpoint); N % 8 tails included
    fcases = [(3, 16, 24), (9, 40, 100), (8, 69, 33), (2, 136, 64), (17, 7, 1024)]
    for i, (M, N, K) in enumerate(fcases):
        A = act(rng, M, K, scale=rng.uniform(0.5, 3.0))
        W = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
        Cin = rng.standard_normal((M, N)).astype(np.float32)
        out[f"lf32{i}_A"], out[f"lf32{i}_W"], out[f"lf32{i}_Cin"] = A, W, Cin
        out[f"lf32{i}_C"] = ref.linear_f32(A, W)
        out[f"lf32{i}_Cadd"] = ref.linear_f32(A, W, Cin, accumulate=True)

    path = os.path.join(HERE, "int8nk_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
