"""CPU tests: pin the oracle (our C restatement of the int8-nk path).

Each function of oracle/ovoracle.c is pinned three ways where possible:
  1. against the golden vectors written from the compiled reference
     (tests/golden/gen_golden.py);
  2. against the compiled reference itself on fresh seeded inputs
     (oracle/_ref; skipped where it is not built);
  3. against what the mathematics fixes: the lossless known-answer GEMM of
     cpp/tests/test_gemm.cpp:114-146, integer brute force for the per-block
     dot products, closed-form quantiser bounds, exp accuracy.
"""
import ctypes
import math

import numpy as np
import pytest

from conftest import u8_to_s8  # noqa: F401


def bits(a):
    return np.ascontiguousarray(a).view(np.int32)


# ---------------------------------------------------------------------------
# 1. golden vectors

def _cases(golden, prefix):
    return sorted({k.split("_")[0] for k in golden if k.startswith(prefix)})


def test_quantize_golden(golden, oracle):
    for c in _cases(golden, "quant"):
        aq, asc = oracle.quantize(golden[c + "_A"])
        assert np.array_equal(aq, golden[c + "_aq"]), c
        assert np.array_equal(bits(asc), bits(golden[c + "_asc"])), c


def test_rmsnorm_quantize_golden(golden, oracle):
    for c in _cases(golden, "rms"):
        aq, asc = oracle.rmsnorm_quantize(golden[c + "_x"], golden[c + "_w"], 1e-6)
        assert np.array_equal(aq, golden[c + "_aq"]), c
        assert np.array_equal(bits(asc), bits(golden[c + "_asc"])), c


def test_silu_mul_quantize_golden(golden, oracle):
    for c in _cases(golden, "silu"):
        aq, asc = oracle.silu_mul_quantize(golden[c + "_g"], golden[c + "_u"])
        assert np.array_equal(aq, golden[c + "_aq"]), c
        assert np.array_equal(bits(asc), bits(golden[c + "_asc"])), c


def test_gemm_golden(golden, oracle):
    for c in _cases(golden, "gemm"):
        A, W, ws, Cin = (golden[c + s] for s in ("_A", "_W", "_ws", "_Cin"))
        aq, asc = oracle.quantize(A)
        assert np.array_equal(bits(oracle.linear_q(aq, asc, W, ws)), bits(golden[c + "_C"])), c
        Cadd = oracle.linear_q(aq, asc, W, ws, Cin, accumulate=True)
        assert np.array_equal(bits(Cadd), bits(golden[c + "_Cadd"])), c
        if c + "_blocks" in golden:
            assert np.array_equal(oracle.block_dots(aq, W), golden[c + "_blocks"]), c


def test_c1_slice_golden(golden, oracle):
    q, s = oracle.quantize_weight_rows(golden["c1_Wf"])
    assert np.array_equal(q, golden["c1_q"]) and np.array_equal(bits(s), bits(golden["c1_s"]))
    aq, asc = oracle.quantize(golden["c1_A"])
    assert np.array_equal(bits(oracle.linear_q(aq, asc, q, s)), bits(golden["c1_C"]))


def test_sliced_golden(golden, oracle):
    aq, asc = oracle.quantize(golden["sl_A"])
    for j in range(3):
        C = oracle.linear_q(aq, asc, golden[f"sl_W{j}"], golden[f"sl_s{j}"])
        assert np.array_equal(bits(C), bits(golden[f"sl_C{j}"])), j


# ---------------------------------------------------------------------------
# 2. against the compiled reference on fresh inputs

@pytest.mark.parametrize("M,N,K", [(3, 24, 40), (13, 70, 100), (33, 64, 1024), (8, 200, 3072)])
def test_against_reference(reference, oracle, M, N, K):
    rng = np.random.default_rng(M * 1000 + N + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    A[:, rng.integers(0, K, 4)] *= 20
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    ws = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    aq_o, asc_o = oracle.quantize(A)
    aq_r, asc_r = reference.quantize(A)
    assert np.array_equal(aq_o, aq_r) and np.array_equal(bits(asc_o), bits(asc_r))
    assert np.array_equal(bits(oracle.linear_q(aq_o, asc_o, W, ws)),
                          bits(reference.linear_q(aq_r, asc_r, W, ws)))
    x = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    w = rng.uniform(0.1, 1.1, K).astype(np.float32)
    a, b = oracle.rmsnorm_quantize(x, w), reference.rmsnorm_quantize(x, w)
    assert np.array_equal(a[0], b[0]) and np.array_equal(bits(a[1]), bits(b[1]))
    assert np.array_equal(bits(oracle.rmsnorm(x, w)), bits(reference.rmsnorm(x, w)))
    g = (rng.standard_normal((M, K)) * 4).astype(np.float32)
    u = rng.standard_normal((M, K)).astype(np.float32)
    a, b = oracle.silu_mul_quantize(g, u), reference.silu_mul_quantize(g, u)
    assert np.array_equal(a[0], b[0]) and np.array_equal(bits(a[1]), bits(b[1]))
    assert np.array_equal(bits(oracle.silu_mul(g, u)), bits(reference.silu_mul(g, u)))


def test_tail_widths_against_reference(reference, oracle):
    """Every K%8 / K%32 tail the RMSNorm and SiLU reductions can see."""
    rng = np.random.default_rng(7)
    for K in list(range(1, 41)) + [69, 1023, 1025]:
        x = (rng.standard_normal((5, K)) * rng.uniform(0.1, 30)).astype(np.float32)
        w = rng.uniform(0.1, 1.1, K).astype(np.float32)
        assert np.array_equal(bits(oracle.rmsnorm(x, w)), bits(reference.rmsnorm(x, w))), K
        a, b = oracle.rmsnorm_quantize(x, w), reference.rmsnorm_quantize(x, w)
        assert np.array_equal(a[0], b[0]) and np.array_equal(bits(a[1]), bits(b[1])), K


def test_fast_path_matches_scalar(oracle):
    if not oracle.fast_available():
        pytest.skip("no AVX-512 VNNI on this host")
    rng = np.random.default_rng(3)
    for (M, N, K) in [(5, 17, 33), (64, 300, 1024), (7, 16, 3072)]:
        A = rng.standard_normal((M, K)).astype(np.float32)
        W = rng.integers(-127, 128, (N, K)).astype(np.int8)
        ws = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
        aq, asc = oracle.quantize(A)
        packed, wsum = oracle.pack(W)
        for acc in (False, True):
            Cin = rng.standard_normal((M, N)).astype(np.float32)
            C = Cin.copy() if acc else np.zeros((M, N), np.float32)
            oracle.linear_q_packed(aq, asc, packed, wsum, N, K, ws, C, accumulate=acc)
            ref = oracle.linear_q(aq, asc, W, ws, Cin if acc else None, accumulate=acc)
            assert np.array_equal(bits(C), bits(ref)), (M, N, K, acc)


# ---------------------------------------------------------------------------
# 3. what the mathematics fixes

@pytest.mark.parametrize("M,N,K", [(4, 8, 16), (5, 17, 33), (9, 7, 69), (1, 33, 9), (2, 1024, 1024)])
def test_lossless_known_answer(oracle, M, N, K):
    """cpp/tests/test_gemm.cpp:114-146: activations 0.5*U{-127..127} with 63.5 at every
    block start, so amax/127 = 0.5 exactly and quantisation is lossless; the GEMM must
    then equal a double-precision product within rel 1e-5 (it is exact in practice)."""
    rng = np.random.default_rng(1234 + M + N + K)
    A = 0.5 * rng.integers(-127, 128, (M, K)).astype(np.float32)
    A[:, ::32] = 63.5
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    ws = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    aq, asc = oracle.quantize(A)
    assert np.all(asc == np.float32(0.5))
    C = oracle.linear_q(aq, asc, W, ws)
    R = (A.astype(np.float64) @ W.astype(np.float64).T) * ws.astype(np.float64)
    rel = np.abs(C - R).max() / (np.abs(R).max() + 1e-12)
    assert rel <= 1e-5


def test_block_dots_brute_force(oracle):
    rng = np.random.default_rng(11)
    M, N, K = 6, 9, 75
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    aq, _ = oracle.quantize(A)
    q = aq[:, :K].astype(np.int64) - 128
    Kb = (K + 31) // 32
    want = np.zeros((M, N, Kb), np.int64)
    for b in range(Kb):
        sl = slice(32 * b, min(K, 32 * b + 32))
        want[:, :, b] = q[:, sl] @ W[:, sl].astype(np.int64).T
    assert np.array_equal(oracle.block_dots(aq, W), want)


def test_quantizer_closed_form(oracle):
    """scale = amax/127 per block; every dequantised value is within scale/2 of its
    input; the block max maps to +-127; zero blocks give scale 0 and code 128;
    K-tail padding bytes are 0."""
    rng = np.random.default_rng(5)
    M, K = 9, 77
    A = (rng.standard_normal((M, K)) * rng.uniform(0.01, 100, (M, 1))).astype(np.float32)
    A[2, 32:64] = 0.0
    aq, asc = oracle.quantize(A)
    Kb = (K + 31) // 32
    for m in range(M):
        for b in range(Kb):
            blk = A[m, 32 * b:min(K, 32 * b + 32)]
            amax = np.float32(np.abs(blk).max())
            assert asc[m, b] == np.float32(amax / np.float32(127.0))
            q = aq[m, 32 * b:32 * b + len(blk)].astype(np.int32) - 128
            if amax == 0:
                assert np.all(q == 0)
                continue
            assert np.abs(q).max() == 127
            assert np.all(np.abs(q * np.float64(asc[m, b]) - blk) <= asc[m, b] * 0.5 * (1 + 1e-5))
    assert np.all(aq[:, K:] == 0)


def test_weight_quantization_closed_form(oracle):
    """tools/convert_weights.py:130-135: per row scale = max(absmax/127, 1e-12); the row's
    absmax element maps to +-127; |q*scale - w| <= scale/2; an all-zero row keeps scale
    1e-12 and codes 0."""
    rng = np.random.default_rng(9)
    W = (rng.standard_normal((12, 300)) * 0.02).astype(np.float32)
    W[3] = 0.0
    q, s = oracle.quantize_weight_rows(W)
    assert s[3] == np.float32(1e-12) and np.all(q[3] == 0)
    for n in (0, 1, 5, 11):
        amax = np.float32(np.abs(W[n]).max())
        assert s[n] == np.float32(amax / np.float32(127.0))
        assert np.abs(q[n]).max() == 127
        assert np.all(np.abs(q[n] * np.float64(s[n]) - W[n]) <= s[n] * 0.5 * (1 + 1e-5))


def test_exp256_accuracy_and_clamps(oracle):
    """ops_cpu.cpp:72-74 claims max relative error ~1e-7 on the clamped range."""
    worst = 0.0
    for x in np.linspace(-87, 88, 20001, dtype=np.float32):
        e = oracle.exp256(float(x))
        worst = max(worst, abs(e - math.exp(float(x))) / math.exp(float(x)))
    assert worst < 6e-7
    assert oracle.exp256(200.0) == oracle.exp256(88.0)
    assert oracle.exp256(-200.0) == oracle.exp256(-87.0)


def test_fused_equals_unfused(oracle):
    """Byte-identity invariants of cpp/tests/test_gemm.cpp:182-201, 300-351."""
    rng = np.random.default_rng(1)
    for (M, K) in [(8, 1024), (7, 33)]:
        x = rng.uniform(-1, 1, (M, K)).astype(np.float32)
        w = rng.uniform(0.1, 1.1, K).astype(np.float32)
        a, b = oracle.rmsnorm_quantize(x, w), oracle.quantize(oracle.rmsnorm(x, w))
        assert np.array_equal(a[0], b[0]) and np.array_equal(bits(a[1]), bits(b[1]))
    g = rng.uniform(-1, 1, (8, 1024)).astype(np.float32)
    u = rng.uniform(-1, 1, (8, 1024)).astype(np.float32)
    a, b = oracle.silu_mul_quantize(g, u), oracle.quantize(oracle.silu_mul(g, u))
    assert np.array_equal(a[0], b[0]) and np.array_equal(bits(a[1]), bits(b[1]))
    A = rng.uniform(-1, 1, (8, 1024)).astype(np.float32)
    W = rng.integers(-127, 128, (64, 1024)).astype(np.int8)
    ws = rng.uniform(1e-4, 1e-2, 64).astype(np.float32)
    Cin = rng.uniform(-1, 1, (8, 64)).astype(np.float32)
    aq, asc = oracle.quantize(A)
    P = oracle.linear_q(aq, asc, W, ws)
    assert np.array_equal(bits(oracle.linear_q(aq, asc, W, ws, Cin, accumulate=True)),
                          bits((Cin + P).astype(np.float32)))


def golden_mismatches(o, golden):
    """Names of the golden checks that oracle `o` fails."""
    bad = []
    for c in _cases(golden, "lf32"):
        A, W, Cin = golden[c + "_A"], golden[c + "_W"], golden[c + "_Cin"]
        if not (np.array_equal(bits(o.linear_f32(A, W)), bits(golden[c + "_C"])) and
                np.array_equal(bits(o.linear_f32(A, W, Cin, True)), bits(golden[c + "_Cadd"]))):
            bad.append(c)
    for c in _cases(golden, "quant"):
        aq, asc = o.quantize(golden[c + "_A"])
        if not (np.array_equal(aq, golden[c + "_aq"]) and
                np.array_equal(bits(asc), bits(golden[c + "_asc"]))):
            bad.append(c)
    for c in _cases(golden, "rms"):
        aq, asc = o.rmsnorm_quantize(golden[c + "_x"], golden[c + "_w"], 1e-6)
        xn = o.rmsnorm(golden[c + "_x"], golden[c + "_w"], 1e-6)
        if not (np.array_equal(aq, golden[c + "_aq"]) and
                np.array_equal(bits(asc), bits(golden[c + "_asc"])) and
                np.array_equal(bits(xn), bits(golden[c + "_xn"]))):
            bad.append(c)
    for c in _cases(golden, "silu"):
        aq, asc = o.silu_mul_quantize(golden[c + "_g"], golden[c + "_u"])
        act = o.silu_mul(golden[c + "_g"], golden[c + "_u"])
        if not (np.array_equal(aq, golden[c + "_aq"]) and
                np.array_equal(bits(asc), bits(golden[c + "_asc"])) and
                np.array_equal(bits(act), bits(golden[c + "_act"]))):
            bad.append(c)
    for c in _cases(golden, "gemm"):
        A, W, ws = golden[c + "_A"], golden[c + "_W"], golden[c + "_ws"]
        aq, asc = o.quantize(A)
        ok = np.array_equal(bits(o.linear_q(aq, asc, W, ws)), bits(golden[c + "_C"]))
        if c + "_blocks" in golden:
            ok = ok and np.array_equal(o.block_dots(aq, W), golden[c + "_blocks"])
        if not ok:
            bad.append(c)
    q, sc = o.quantize_weight_rows(golden["c1_Wf"])
    if not (np.array_equal(q, golden["c1_q"]) and np.array_equal(bits(sc), bits(golden["c1_s"]))):
        bad.append("c1")
    for c in _cases(golden, "qknr"):
        rows, nh, nkv, D = (int(x) for x in golden[c + "_dims"])
        qo, ko = o.qk_norm_rope(golden[c + "_q"], golden[c + "_k"], golden[c + "_qw"],
                                golden[c + "_kw"], nh, nkv, D, golden[c + "_pos"])
        if not (np.array_equal(bits(qo), bits(golden[c + "_qo"])) and
                np.array_equal(bits(ko), bits(golden[c + "_ko"]))):
            bad.append(c)
    for c in _cases(golden, "attn"):
        bias = golden[c + "_bias"] if int(golden[c + "_masked"]) else None
        out = o.attention_head(golden[c + "_q"], golden[c + "_k"], golden[c + "_v"], bias)
        if not np.array_equal(bits(out), bits(golden[c + "_out"])):
            bad.append(c)
    return bad


def test_golden_f32_intermediates(golden, oracle):
    assert golden_mismatches(oracle, golden) == []


def test_weight_scale_floor(oracle):
    """An all-zero row keeps the 1e-12 floor (plant 6 removes it)."""
    q, s = oracle.quantize_weight_rows(np.zeros((2, 40), np.float32))
    assert np.all(s == np.float32(1e-12)) and np.all(q == 0)


@pytest.mark.parametrize("plant", [1, 2, 3, 4, 5, 7, 8, 9, 10])
def test_planted_mistakes_are_caught(golden, plant, tmp_path):
    """Rebuild the oracle with one deliberate, plausible mistake (OVO_PLANT in
    oracle/ovoracle.c) and check that the golden vectors reject it."""
    import subprocess
    from oracle import HERE, Oracle
    lib = tmp_path / f"liboracle_plant{plant}.so"
    subprocess.run(["gcc", "-std=c11", "-O2", "-ffp-contract=off", "-fopenmp", "-fPIC", "-shared",
                    f"-DOVO_PLANT={plant}", "-o", str(lib), f"{HERE}/ovoracle.c", "-lm"],
                   check=True)
    assert golden_mismatches(Oracle(str(lib)), golden) != []


def test_linear_f32_closed_form_and_reference(oracle, reference):
    """linear_f32 (Mat's fp32 branch): integer-valued operands with sums below
    2^24 give the exact integer product whatever the order; a K = 1 product is
    one correctly rounded multiply; and on random data the oracle's fma chain is
    the compiled reference's linear_f32_ld bit for bit (N % 8 tails included)."""
    rng = np.random.default_rng(31)
    A = rng.integers(-50, 51, (13, 70)).astype(np.float32)
    W = rng.integers(-50, 51, (70, 29)).astype(np.float32)
    exact = A.astype(np.int64) @ W.astype(np.int64)
    assert np.array_equal(oracle.linear_f32(A, W), exact.astype(np.float32))
    a1 = rng.standard_normal((5, 1)).astype(np.float32)
    w1 = rng.standard_normal((1, 11)).astype(np.float32)
    assert np.array_equal(bits(oracle.linear_f32(a1, w1)), bits((a1 * w1).astype(np.float32)))
    for M, N, K in ((7, 8200 // 40, 1024), (3, 13, 5), (40, 64, 300)):
        A = rng.standard_normal((M, K)).astype(np.float32)
        W = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
        Cin = rng.standard_normal((M, N)).astype(np.float32)
        assert np.array_equal(bits(oracle.linear_f32(A, W)), bits(reference.linear_f32(A, W)))
        assert np.array_equal(bits(oracle.linear_f32(A, W, Cin, True)),
                              bits(reference.linear_f32(A, W, Cin, True)))
