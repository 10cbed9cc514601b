"""GPU parity tests: the HIP path through the C ABI vs the oracle and the golden
vectors written from the compiled reference.

Bar: integer/byte outputs (activation codes, per-block int32 dot products) are
bit-exact; fp32 outputs (scales, GEMM results) are bit-exact too, because the
kernels keep the reference's operation order (f = fma(float(acc_b), asc, f) in
block order, then * wscale, then + C rounded separately).  The north-star
tolerance for fp32 (max relative error 1e-3) is therefore met with zero error;
tests that only need that tolerance say so.
"""
import ctypes
import os

import numpy as np
import pytest

from conftest import u8_to_s8

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import ovnative_amd
    ovnative_amd.load()  # fail loudly if the HIP library is missing
    torch.cuda.set_device(0)
    yield
    torch.cuda.synchronize()


def bits(a):
    return np.ascontiguousarray(a).view(np.int32)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def cases(golden, prefix):
    return sorted({k.split("_")[0] for k in golden if k.startswith(prefix)})


def glibc_expf_differs(g):
    """True where glibc expf(-g) != exp(-g) correctly rounded (the silu tail uses
    libm in the reference and a double-precision exp on the GPU)."""
    libm = ctypes.CDLL("libm.so.6")
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    out = np.zeros(g.shape, bool)
    for idx, x in np.ndenumerate(g):
        out[idx] = np.float32(libm.expf(float(-x))) != np.float32(np.exp(-np.float64(x)))
    return out


# ---------------------------------------------------------------------------
# quantisers vs golden vectors (compiled reference)

def test_quantize_golden(golden):
    import ovnative_amd as ov
    for c in cases(golden, "quant"):
        A = golden[c + "_A"]
        aq, asc = ov.s8_nk_quantize(dev(A))
        assert np.array_equal(host(aq), u8_to_s8(golden[c + "_aq"], A.shape[1])), c
        assert np.array_equal(bits(host(asc)), bits(golden[c + "_asc"])), c


def test_rmsnorm_quantize_golden(golden):
    import ovnative_amd as ov
    for c in cases(golden, "rms"):
        x, w = golden[c + "_x"], golden[c + "_w"]
        aq, asc = ov.rmsnorm_quantize(dev(x), dev(w), 1e-6)
        assert np.array_equal(host(aq), u8_to_s8(golden[c + "_aq"], x.shape[1])), c
        assert np.array_equal(bits(host(asc)), bits(golden[c + "_asc"])), c


def test_silu_mul_quantize_golden(golden):
    import ovnative_amd as ov
    for c in cases(golden, "silu"):
        g, u = golden[c + "_g"], golden[c + "_u"]
        K = g.shape[1]
        aq, asc = ov.silu_mul_quantize(dev(g), dev(u))
        aq, asc = host(aq), host(asc)
        want_aq, want_asc = u8_to_s8(golden[c + "_aq"], K), golden[c + "_asc"]
        # rows whose libm-tail inputs have a misrounded glibc expf are excused
        ok_rows = np.ones(g.shape[0], bool)
        kv_tail = K % 32 % 8
        if kv_tail:
            tail = g[:, K - kv_tail:]
            ok_rows = ~glibc_expf_differs(tail).any(axis=1)
        assert ok_rows.sum() >= g.shape[0] - 1
        assert np.array_equal(aq[ok_rows], want_aq[ok_rows]), c
        assert np.array_equal(bits(asc[ok_rows]), bits(want_asc[ok_rows])), c


# ---------------------------------------------------------------------------
# GEMM vs golden vectors

def test_gemm_golden(golden):
    import ovnative_amd as ov
    for c in cases(golden, "gemm"):
        A, W, ws, Cin = (golden[c + s] for s in ("_A", "_W", "_ws", "_Cin"))
        w = ov.Weight.from_host(W, ws, layout=0)
        aq, asc = ov.s8_nk_quantize(dev(A))
        C = ov.linear_q(aq, asc, w)
        assert np.array_equal(bits(host(C)), bits(golden[c + "_C"])), c
        Cacc = dev(Cin)
        ov.linear_q(aq, asc, w, Cacc, accumulate=True)
        assert np.array_equal(bits(host(Cacc)), bits(golden[c + "_Cadd"])), c
        if c + "_blocks" in golden:
            assert np.array_equal(host(ov.block_dots(aq, w)), golden[c + "_blocks"]), c


def test_gemm_golden_kn_layout(golden):
    """OVW1 layout=1 ([K,N]) weights give the same bits (mat.cpp:73-85)."""
    import ovnative_amd as ov
    for c in ("gemm1", "gemm4", "gemm5"):
        A, W, ws = golden[c + "_A"], golden[c + "_W"], golden[c + "_ws"]
        w = ov.Weight.from_host(np.ascontiguousarray(W.T), ws, layout=1)
        aq, asc = ov.s8_nk_quantize(dev(A))
        assert np.array_equal(bits(host(ov.linear_q(aq, asc, w))), bits(golden[c + "_C"])), c


def test_c1_slice_golden(golden):
    import ovnative_amd as ov
    w = ov.Weight.from_host(golden["c1_q"], golden["c1_s"])
    aq, asc = ov.s8_nk_quantize(dev(golden["c1_A"]))
    assert np.array_equal(bits(host(ov.linear_q(aq, asc, w))), bits(golden["c1_C"]))


def test_sliced_golden(golden):
    import ovnative_amd as ov
    parts = [ov.Weight.from_host(golden[f"sl_W{j}"], golden[f"sl_s{j}"]) for j in range(3)]
    merged = ov.Weight.concat(parts)
    aq, asc = ov.s8_nk_quantize(dev(golden["sl_A"]))
    outs = ov.linear_q_sliced(aq, asc, merged, [128, 64, 64])
    for j, o in enumerate(outs):
        assert np.array_equal(bits(host(o)), bits(golden[f"sl_C{j}"])), j


# ---------------------------------------------------------------------------
# against the oracle at BASELINE shapes

def _rand_problem(rng, M, N, K, outliers=8):
    A = rng.standard_normal((M, K)).astype(np.float32)
    A[:, rng.choice(K, size=min(outliers, K), replace=False)] *= 20
    Wf = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    return A, Wf


def _oracle_linear(oracle, A, q, s, Cin=None):
    aq, asc = oracle.quantize(A)
    if oracle.fast_available():
        packed, wsum = oracle.pack(q)
        C = np.zeros((A.shape[0], q.shape[0]), np.float32) if Cin is None else Cin.copy()
        return oracle.linear_q_packed(aq, asc, packed, wsum, q.shape[0], q.shape[1], s, C,
                                      accumulate=Cin is not None)
    return oracle.linear_q(aq, asc, q, s, Cin, accumulate=Cin is not None)


@pytest.mark.parametrize("M,N,K", [
    (256, 3072, 1024),
    (128, 2048, 1024), (128, 1024, 1024), (128, 1024, 2048), (128, 3072, 1024),
    (128, 1024, 3072),   # config 2: q, k/v, o, gate/up, down at M = 2 x 64
    (600, 4096, 1024), (600, 6144, 1024), (600, 1024, 3072),  # config 3/4: qkv, gate/up, down
    (1, 1024, 1024), (5, 200, 96), (33, 130, 1000), (65, 64, 32),
    (520, 192, 1152),    # 512 <= M < 1024, Kb % 8 != 0: the 3-stage ring
    (700, 2112, 1024),   # 512 <= M < 1024, N >= 2048: 64x32 tiles of 2 wavefronts
    (300, 1024, 2048),   # 256 <= M < 512, N < 2048: 8-block stages, 3-stage ring
    (1200, 1024, 3072),  # 1024 <= M < 2048, N < 2048: 32x32 tiles of 2 wavefronts
    (1200, 4096, 1024),  # 1024 <= M < 2048, N >= 2048: 64x64 tiles, 3-stage ring
])
def test_linear_vs_oracle(oracle, M, N, K):
    import ovnative_amd as ov
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    A, Wf = _rand_problem(rng, M, N, K)
    q, s = oracle.quantize_weight_rows(Wf)
    w = ov.Weight.from_host(q, s)
    dA = dev(A)
    aq, asc = ov.s8_nk_quantize(dA)
    aq_r, asc_r = oracle.quantize(A)
    assert np.array_equal(host(aq), u8_to_s8(aq_r, K))
    assert np.array_equal(bits(host(asc)), bits(asc_r))
    C = host(ov.linear_q(aq, asc, w))
    want = _oracle_linear(oracle, A, q, s)
    assert np.array_equal(bits(C), bits(want))
    # residual variant (o_proj / down)
    Cin = rng.standard_normal((M, N)).astype(np.float32)
    Cacc = dev(Cin)
    ov.linear_q(aq, asc, w, Cacc, accumulate=True)
    assert np.array_equal(bits(host(Cacc)), bits(_oracle_linear(oracle, A, q, s, Cin)))
    # fp32 tolerance of the north star, against the double-precision dequantised product
    R = (A.astype(np.float64) @ (q.astype(np.float64) * s[:, None].astype(np.float64)).T)
    assert np.abs(C - R).max() / np.abs(R).max() < 5e-2  # quantisation noise bound, not parity


BAND_EDGES = (127, 128, 129, 255, 256, 511, 512, 1023, 1024, 2047, 2048)


@pytest.mark.parametrize("N,K", [(1024, 1024), (2048, 1024), (6144, 1024), (1024, 3072)])
def test_linear_tile_band_edges(oracle, N, K):
    """On both sides of every row count where launch_gemm changes tile shape
    (128, 256, 512, 1024, 2048; with N = 1024 / 2048 / 6144 and K = 1024 /
    3072, the N and K conditions of the dispatch): the store and residual
    forms, on row-major and tile-major codes, are the oracle's bits
    (gemm.cpp:432-504) on sampled rows, the first and last among them."""
    import ovnative_amd as ov
    rng = np.random.default_rng(N + K)
    Mmax = max(BAND_EDGES)
    A, Wf = _rand_problem(rng, Mmax, N, K)
    q, s = oracle.quantize_weight_rows(Wf)
    w = ov.Weight.from_host(q, s)
    Cin = rng.standard_normal((Mmax, N)).astype(np.float32)
    for M in BAND_EDGES:
        aq, asc = ov.s8_nk_quantize(dev(A[:M]))
        t = ov.tile_major(aq)
        rows = np.unique(np.concatenate([[0, M - 1], rng.choice(M, 6, replace=False)]))
        want = _oracle_linear(oracle, A[rows], q, s)
        want_acc = _oracle_linear(oracle, A[rows], q, s, Cin[rows])
        for name, C in (("rowmajor", ov.linear_q(aq, asc, w)),
                        ("tilemajor", ov.linear_q_tiled(t, asc, w, M))):
            assert np.array_equal(bits(host(C)[rows]), bits(want)), (M, name)
        for name, fn in (("rowmajor", lambda C: ov.linear_q(aq, asc, w, C, accumulate=True)),
                         ("tilemajor",
                          lambda C: ov.linear_q_tiled(t, asc, w, M, C, accumulate=True))):
            C = dev(Cin[:M])
            fn(C)
            assert np.array_equal(bits(host(C)[rows]), bits(want_acc)), (M, name, "residual")


def test_linear_random_shapes(oracle):
    """Seeded random shapes (M up to 2600; N and K ragged, or multiples of 128
    / 256 as the LM's are): ovh_linear_q is the oracle's bits on sampled rows,
    and where the shape allows them ovh_linear_q_tiled and ovh_linear_q_norm
    (== the residual launch then ovh_rmsnorm_quantize) are too."""
    import ovnative_amd as ov
    rng = np.random.default_rng(2026)
    for _ in range(24):
        M = int(rng.choice([rng.integers(1, 300), rng.integers(300, 2600)]))
        N = int(rng.choice([rng.integers(1, 700), 256 * rng.integers(1, 5), 2048, 3072]))
        K = int(rng.choice([rng.integers(1, 600), 128 * rng.integers(1, 25), 1024, 3072]))
        A, Wf = _rand_problem(rng, M, N, K, outliers=min(8, K))
        q, s = oracle.quantize_weight_rows(Wf)
        w = ov.Weight.from_host(q, s)
        aq, asc = ov.s8_nk_quantize(dev(A))
        rows = np.unique(np.concatenate([[0, M - 1], rng.choice(M, min(M, 5), replace=False)]))
        want = _oracle_linear(oracle, A[rows], q, s)
        assert np.array_equal(bits(host(ov.linear_q(aq, asc, w))[rows]), bits(want)), (M, N, K)
        if K % 128:
            continue
        t = ov.tile_major(aq)
        got = host(ov.linear_q_tiled(t, asc, w, M))[rows]
        assert np.array_equal(bits(got), bits(want)), (M, N, K, "tiled")
        if N % 256 or N > 1024:
            continue
        x0 = rng.standard_normal((M, N)).astype(np.float32)
        nw = dev(rng.uniform(0.5, 1.5, N).astype(np.float32))
        cnt = ov.band_counters(max(M, 2048))
        x = dev(x0)
        nq, nsc = ov.linear_q_norm(t, asc, w, x, nw, cnt, 1e-6)
        want_x = dev(x0)
        ov.linear_q_tiled(t, asc, w, M, want_x, accumulate=True)
        want_q, want_s = ov.rmsnorm_quantize(want_x, nw, 1e-6)
        assert np.array_equal(bits(host(x)), bits(host(want_x))), (M, N, K, "norm")
        assert np.array_equal(host(nq), tile_major(host(want_q), M)), (M, N, K, "norm codes")
        assert np.array_equal(bits(host(nsc)), bits(host(want_s))), (M, N, K, "norm scales")
        assert host(cnt)[0] == 0


@pytest.mark.parametrize("M", [129, 511, 512, 1023, 1024, 2047, 2048])
def test_silu_gate_linear_band_edges(oracle, M):
    """The SiLU-fused gate/up on both sides of its tile-shape changes (128,
    512, 1024, 2048 rows): the reference's gate/up GEMM then
    silu_mul_quantize_f32 (lm.cpp:293-311) byte for byte, on sampled rows."""
    import ovnative_amd as ov
    rng = np.random.default_rng(500 + M)
    I, K = 3072, 1024
    A = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    qg, sg = oracle.quantize_weight_rows((rng.standard_normal((I, K)) * 0.02).astype(np.float32))
    qu, su = oracle.quantize_weight_rows((rng.standard_normal((I, K)) * 0.02).astype(np.float32))
    gu = ov.gate_up_weight(ov.Weight.from_host(qg, sg), ov.Weight.from_host(qu, su))
    aq, asc = ov.s8_nk_quantize(dev(A))
    hq, hsc = ov.silu_gate_linear(aq, asc, gu)
    rows = np.unique(np.concatenate([[0, M - 1], rng.choice(M, 6, replace=False)]))
    hq_r, hsc_r = oracle.silu_mul_quantize(_oracle_linear(oracle, A[rows], qg, sg),
                                           _oracle_linear(oracle, A[rows], qu, su))
    assert np.array_equal(host(hq)[rows], u8_to_s8(hq_r, I))
    assert np.array_equal(bits(host(hsc)[rows]), bits(hsc_r))


def test_diag_read_paths():
    """The byte-counter calibration reads run on every load path and leave the
    buffer as it was; sizes that are not a multiple of 128 KiB and unknown paths
    are refused."""
    import ovnative_amd as ov
    t = torch.arange(1 << 16, dtype=torch.float32, device="cuda")  # 256 KiB
    ref = t.clone()
    for path in (ov.READ_DMA16, ov.READ_DMA4, ov.READ_VEC16, ov.READ_BUF8):
        ov.diag_read(t, path)
    torch.cuda.synchronize()
    assert torch.equal(t, ref)
    with pytest.raises(ov.InvalidArgument):
        ov.diag_read(t[:1000], ov.READ_DMA16)
    with pytest.raises(ov.InvalidArgument):
        ov.diag_read(t, 4)


def test_linear_q_refuses_unaligned_scales():
    """The GEMMs move codes and block scales by 16-byte DMA: scales that are
    not 16-byte aligned are refused (single and grouped entry points) rather
    than read from a rounded address; aligned copies of the same values give
    the usual result."""
    import ovnative_amd as ov
    rng = np.random.default_rng(71)
    M, N, K = 64, 256, 1024
    A = rng.standard_normal((M, K)).astype(np.float32)
    w = ov.Weight.from_host(rng.integers(-127, 128, (N, K), dtype=np.int8),
                            (rng.random(N) * 1e-3 + 1e-4).astype(np.float32))
    aq, asc = ov.s8_nk_quantize(dev(A))
    flat = torch.empty(asc.numel() + 1, dtype=torch.float32, device="cuda")
    mis = flat[1:].view(M, -1)  # 4 bytes past a 16-byte boundary
    mis.copy_(asc)
    with pytest.raises(ov.InvalidArgument):
        ov.linear_q(aq, mis, w)
    with pytest.raises(ov.InvalidArgument):
        ov.linear_q_grouped([(aq, mis, w)])
    assert np.array_equal(bits(host(ov.linear_q(aq, mis.clone(), w))),
                          bits(host(ov.linear_q(aq, asc, w))))


def test_block_dots_exact_at_scale(oracle):
    """Per-block int32 sums from the MFMA path equal integer brute force (sampled rows)."""
    import ovnative_amd as ov
    rng = np.random.default_rng(99)
    M, N, K = 600, 1024, 3072
    A, Wf = _rand_problem(rng, M, N, K)
    q, s = oracle.quantize_weight_rows(Wf)
    w = ov.Weight.from_host(q, s)
    aq, asc = ov.s8_nk_quantize(dev(A))
    blocks = host(ov.block_dots(aq, w))
    rows = rng.choice(M, 24, replace=False)
    aq_h = host(aq).astype(np.int64)
    for m in rows:
        want = (aq_h[m].reshape(-1, 32)[None, :, :] *
                np.pad(q, ((0, 0), (0, aq_h.shape[1] - K))).astype(np.int64).reshape(N, -1, 32)
                ).sum(axis=2)
        assert np.array_equal(blocks[m], want), m


def test_large_m_properties(oracle):
    """M = 16384 (config 5 rows): sampled rows bit-exact vs the oracle; row order does
    not change a row's result (rows are independent)."""
    import ovnative_amd as ov
    rng = np.random.default_rng(5)
    M, N, K = 16384, 1024, 1024
    A, Wf = _rand_problem(rng, M, N, K)
    q, s = oracle.quantize_weight_rows(Wf)
    w = ov.Weight.from_host(q, s)
    dA = dev(A)
    aq, asc = ov.s8_nk_quantize(dA)
    C = host(ov.linear_q(aq, asc, w))
    rows = np.sort(rng.choice(M, 64, replace=False))
    want = _oracle_linear(oracle, A[rows], q, s)
    assert np.array_equal(bits(C[rows]), bits(want))
    perm = rng.permutation(M)
    aq2, asc2 = ov.s8_nk_quantize(dev(A[perm]))
    C2 = host(ov.linear_q(aq2, asc2, w))
    assert np.array_equal(bits(C2), bits(C[perm]))


def _sample_rows(rng, M, n):
    """Rows of every large-M tile position: the first and last rows, the 64-row
    tile edges around them, and random rows."""
    edge = {0, 1, 31, 32, 63, 64, 127, 128, M // 2, M - 65, M - 64, M - 2, M - 1}
    return np.array(sorted(edge | set(rng.choice(M, n, replace=False).tolist())))


@pytest.mark.parametrize("which", ["silu_gate_up", "residual_k3072", "qkv_sliced_n4096"])
def test_large_m_int8_form_sampled_rows(oracle, which):
    """The default int8 GEMM form at M = 16384 (8 requests x
    CFG 2 x seq 1024), i.e. the large-M tiles the runner takes from 2048 rows,
    on the LM's shapes: the SiLU-fused gate/up (N = 2 x 3072, codes and scales
    vs the oracle's sliced GEMM then silu_mul_quantize_f32), the down
    projection's residual form (K = 3072, tile-major codes as the runner
    passes them, accumulating into a random fp32 hidden state) and the merged
    q/k/v sliced into three outputs (N = 2048 + 1024 + 1024); sampled rows
    bit-exact vs the oracle."""
    import ovnative_amd as ov
    rng = np.random.default_rng({"silu_gate_up": 71, "residual_k3072": 72,
                                 "qkv_sliced_n4096": 73}[which])
    M = 16384
    if which == "silu_gate_up":
        I, K = 3072, 1024
        A = (rng.standard_normal((M, K)) * 2).astype(np.float32)
        qg, sg = oracle.quantize_weight_rows((rng.standard_normal((I, K)) * 0.02).astype(np.float32))
        qu, su = oracle.quantize_weight_rows((rng.standard_normal((I, K)) * 0.02).astype(np.float32))
        gu = ov.gate_up_weight(ov.Weight.from_host(qg, sg), ov.Weight.from_host(qu, su))
        aq, asc = ov.s8_nk_quantize(dev(A))
        hq, hsc = ov.silu_gate_linear(aq, asc, gu)
        hq, hsc = host(hq), host(hsc)
        rows = _sample_rows(rng, M, 40)
        hq_r, hsc_r = oracle.silu_mul_quantize(_oracle_linear(oracle, A[rows], qg, sg),
                                               _oracle_linear(oracle, A[rows], qu, su))
        assert np.array_equal(hq[rows], u8_to_s8(hq_r, I))
        assert np.array_equal(bits(hsc[rows]), bits(hsc_r))
    elif which == "residual_k3072":
        N, K = 1024, 3072
        A, Wf = _rand_problem(rng, M, N, K)
        q, s = oracle.quantize_weight_rows(Wf)
        w = ov.Weight.from_host(q, s)
        aq, asc = ov.s8_nk_quantize(dev(A))
        Cin = rng.standard_normal((M, N)).astype(np.float32)
        C = dev(Cin)
        ov.linear_q_tiled(ov.tile_major(aq), asc, w, M, C, accumulate=True)
        C = host(C)
        rows = _sample_rows(rng, M, 40)
        want = _oracle_linear(oracle, A[rows], q, s, Cin[rows])
        assert np.array_equal(bits(C[rows]), bits(want))
    else:
        K = 1024
        A, Wf = _rand_problem(rng, M, 4096, K)
        q, s = oracle.quantize_weight_rows(Wf)
        w = ov.Weight.from_host(q, s)
        aq, asc = ov.s8_nk_quantize(dev(A))
        outs = ov.linear_q_sliced(aq, asc, w, [2048, 1024, 1024])
        got = np.concatenate([host(o) for o in outs], axis=1)
        rows = _sample_rows(rng, M, 40)
        assert np.array_equal(bits(got[rows]), bits(_oracle_linear(oracle, A[rows], q, s)))


# ---------------------------------------------------------------------------
# the f16-operand GEMM form (opt-in, here from 2048 rows): int8-valued f16
# weights and codes, exact block products out of the f16 matrix core.  Rows are
# independent, so the int8 form over row chunks below the threshold gives every
# row's expected bits at full size; sampled rows are checked against the oracle
# as well.

F16_MIN_ROWS = 2048


@pytest.fixture
def f16_form():
    import ovnative_amd as ov
    prev = ov.set_f16_min_rows(F16_MIN_ROWS)
    assert prev == 0  # off unless asked for
    yield
    ov.set_f16_min_rows(prev)


def _by_chunks(M, fn, chunk=1024):
    assert chunk < F16_MIN_ROWS
    for r0 in range(0, M, chunk):
        fn(r0, min(M, r0 + chunk))


@pytest.mark.parametrize("M,N,K", [(2048, 4096, 1024), (16384, 4096, 1024), (4133, 1024, 3072),
                                   (16384, 8200, 1024), (2111, 1024, 2048), (3000, 96, 128)])
def test_f16_form_equals_int8_form(oracle, f16_form, M, N, K):
    """Store and residual forms, row-major and tile-major codes: every row of the
    f16 form equals the int8 form's, sampled rows equal the oracle (q/k/v N = 4096,
    the head's 8200 columns, K = 2048 / 3072 of o_proj / down, ragged M)."""
    import ovnative_amd as ov
    rng = np.random.default_rng(M + 3 * N + K)
    A, Wf = _rand_problem(rng, M, N, K)
    q, s = oracle.quantize_weight_rows(Wf)
    w = ov.Weight.from_host(q, s)
    aq, asc = ov.s8_nk_quantize(dev(A))
    C = ov.linear_q(aq, asc, w)
    ref = torch.empty_like(C)

    def part(r0, r1):
        ref[r0:r1] = ov.linear_q(aq[r0:r1], asc[r0:r1], w)
    _by_chunks(M, part)
    C_h = host(C)
    assert np.array_equal(bits(C_h), bits(host(ref)))
    rows = np.sort(rng.choice(M, 32, replace=False))
    assert np.array_equal(bits(C_h[rows]), bits(_oracle_linear(oracle, A[rows], q, s)))
    del C, ref
    Cin = rng.standard_normal((M, N)).astype(np.float32)
    c1, c2 = dev(Cin), dev(Cin)
    ov.linear_q_tiled(ov.tile_major(aq), asc, w, M, c1, accumulate=True)

    def part_acc(r0, r1):
        ov.linear_q(aq[r0:r1], asc[r0:r1], w, c2[r0:r1], accumulate=True)
    _by_chunks(M, part_acc)
    assert np.array_equal(bits(host(c1)), bits(host(c2)))


def test_f16_form_sliced(oracle, f16_form):
    """The sliced GEMM (q/k/v into three outputs) in the f16 form."""
    import ovnative_amd as ov
    rng = np.random.default_rng(31)
    M, K = 3000, 1024
    A, Wf = _rand_problem(rng, M, 4096, K)
    q, s = oracle.quantize_weight_rows(Wf)
    w = ov.Weight.from_host(q, s)
    aq, asc = ov.s8_nk_quantize(dev(A))
    outs = ov.linear_q_sliced(aq, asc, w, [2048, 1024, 1024])
    full = host(ov.linear_q(aq[:1000], asc[:1000], w))
    got = np.concatenate([host(o) for o in outs], axis=1)
    assert np.array_equal(bits(got[:1000]), bits(full))
    rows = np.sort(rng.choice(M, 16, replace=False))
    assert np.array_equal(bits(got[rows]), bits(_oracle_linear(oracle, A[rows], q, s)))


def test_f16_form_silu_gate_linear(oracle, f16_form):
    """The SiLU-fused gate/up at M = 16384 (config 5, N = 2 x 3072): codes and
    scales of every row equal the int8 form's, sampled rows the oracle's
    composition (sliced GEMM, then silu_mul_quantize_f32)."""
    import ovnative_amd as ov
    rng = np.random.default_rng(61)
    M, I, K = 16384, 3072, 1024
    A = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    qg, sg = oracle.quantize_weight_rows((rng.standard_normal((I, K)) * 0.02).astype(np.float32))
    qu, su = oracle.quantize_weight_rows((rng.standard_normal((I, K)) * 0.02).astype(np.float32))
    gu = ov.gate_up_weight(ov.Weight.from_host(qg, sg), ov.Weight.from_host(qu, su))
    aq, asc = ov.s8_nk_quantize(dev(A))
    hq, hsc = ov.silu_gate_linear(aq, asc, gu)
    hq2, hsc2 = torch.empty_like(hq), torch.empty_like(hsc)

    def part(r0, r1):
        a, b = ov.silu_gate_linear(aq[r0:r1], asc[r0:r1], gu)
        hq2[r0:r1], hsc2[r0:r1] = a, b
    _by_chunks(M, part)
    hq, hsc = host(hq), host(hsc)
    assert np.array_equal(hq, host(hq2)) and np.array_equal(bits(hsc), bits(host(hsc2)))
    rows = np.sort(rng.choice(M, 24, replace=False))
    hq_r, hsc_r = oracle.silu_mul_quantize(_oracle_linear(oracle, A[rows], qg, sg),
                                           _oracle_linear(oracle, A[rows], qu, su))
    assert np.array_equal(hq[rows], u8_to_s8(hq_r, I))
    assert np.array_equal(bits(hsc[rows]), bits(hsc_r))


# ---------------------------------------------------------------------------
# grouped launch: several independent GEMMs, each member's bits those of its own
# ovh_linear_q

def test_linear_q_grouped_equals_separate(oracle):
    """The seven projections of a layer at M = 128 in one
    launch, then members of ragged M (1, 37, 300: other tile bands) with the
    residual form; every member equals ovh_linear_q, one against the oracle."""
    import ovnative_amd as ov
    rng = np.random.default_rng(12)
    H, QD, KVD, I = 1024, 2048, 1024, 3072
    shapes = [(QD, H), (KVD, H), (KVD, H), (H, QD), (I, H), (I, H), (H, I)]
    acts = {}
    probs, hostw = [], []
    for n, k in shapes:
        if k not in acts:
            acts[k] = rng.standard_normal((128, k)).astype(np.float32)
        q, s = oracle.quantize_weight_rows((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        hostw.append((q, s))
        aq, asc = ov.s8_nk_quantize(dev(acts[k]))
        probs.append((aq, asc, ov.Weight.from_host(q, s)))
    outs = ov.linear_q_grouped(probs)
    for (aq, asc, w), c in zip(probs, outs):
        assert np.array_equal(bits(host(c)), bits(host(ov.linear_q(aq, asc, w))))
    q, s = hostw[3]
    assert np.array_equal(bits(host(outs[3])), bits(_oracle_linear(oracle, acts[QD], q, s)))
    # ragged M, residual form
    mixed = []
    for M, (n, k) in [(1, (1024, 1024)), (37, (512, 2048)), (300, (1024, 3072))]:
        A = rng.standard_normal((M, k)).astype(np.float32)
        q, s = oracle.quantize_weight_rows((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        aq, asc = ov.s8_nk_quantize(dev(A))
        mixed.append((aq, asc, ov.Weight.from_host(q, s)))
    cins = [rng.standard_normal((p[0].shape[0], p[2].N)).astype(np.float32) for p in mixed]
    got = [dev(c) for c in cins]
    ov.linear_q_grouped(mixed, got, accumulate=True)
    for (aq, asc, w), g, c in zip(mixed, got, cins):
        want = dev(c)
        ov.linear_q(aq, asc, w, want, accumulate=True)
        assert np.array_equal(bits(host(g)), bits(host(want)))


@pytest.mark.parametrize("accumulate", [False, True], ids=["store", "residual"])
def test_linear_q_grouped_skinny(oracle, accumulate):
    """The skinny-M form of the grouped launch (every member M <= 128 and K a
    multiple of 1024 up to 3072: weights streamed into registers, activation
    slab in LDS; 128 / 64 / 32 rows per workgroup for K = 1024 / 2048 / 3072):
    ragged M (1 .. 128), widths that are not multiples of the 64-column
    workgroup (96, 200, 1000), both output forms; every member equals its own
    ovh_linear_q bit for bit and one the oracle."""
    import ovnative_amd as ov
    rng = np.random.default_rng(31 + accumulate)
    cases = [(1, 1024, 1024), (17, 200, 2048), (64, 96, 3072), (100, 1000, 1024),
             (128, 2048, 3072), (33, 1024, 2048), (128, 3072, 1024), (5, 512, 3072)]
    probs, host_in = [], []
    for M, n, k in cases:
        A = rng.standard_normal((M, k)).astype(np.float32)
        A[:, rng.choice(k, 8, replace=False)] *= 20
        q, s = oracle.quantize_weight_rows((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        aq, asc = ov.s8_nk_quantize(dev(A))
        probs.append((aq, asc, ov.Weight.from_host(q, s)))
        host_in.append((A, q, s))
    cins = [rng.standard_normal((M, n)).astype(np.float32) for M, n, _ in cases]
    got = [dev(c) for c in cins]
    for i in range(0, len(probs), 4):  # two launches of four members
        ov.linear_q_grouped(probs[i:i + 4], got[i:i + 4], accumulate=accumulate)
    for (aq, asc, w), g, c in zip(probs, got, cins):
        want = dev(c)
        ov.linear_q(aq, asc, w, want, accumulate=accumulate)
        assert np.array_equal(bits(host(g)), bits(host(want)))
    A, q, s = host_in[4]
    ref = _oracle_linear(oracle, A, q, s, cins[4] if accumulate else None)
    assert np.array_equal(bits(host(got[4])), bits(ref))


@pytest.mark.parametrize("Ms", [(600, 601, 37), (2100, 128, 5), (128, 128, 128), (129, 128, 1)],
                         ids=["mid", "large", "skinny_edge", "past_skinny_edge"])
def test_linear_q_grouped_tile_bands(oracle, Ms):
    """The grouped launch takes one tile shape for all members, chosen by the
    largest M (the skinny kernel up to 128 rows, 32x32 tiles in the mid band,
    128x64 tiles from 2048 rows): every member, small ones included, still
    equals its own ovh_linear_q."""
    import ovnative_amd as ov
    rng = np.random.default_rng(sum(Ms))
    probs = []
    for M, (n, k) in zip(Ms, [(1024, 2048), (4096, 1024), (1024, 3072)]):
        A = rng.standard_normal((M, k)).astype(np.float32)
        q, s = oracle.quantize_weight_rows((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        aq, asc = ov.s8_nk_quantize(dev(A))
        probs.append((aq, asc, ov.Weight.from_host(q, s)))
    outs = ov.linear_q_grouped(probs)
    for (aq, asc, w), c in zip(probs, outs):
        assert np.array_equal(bits(host(c)), bits(host(ov.linear_q(aq, asc, w))))


def test_linear_q_grouped_random(oracle):
    """Seeded random groups of 1 to 8 members (M 1 .. 200, so that some groups
    take the skinny kernel and some the 16x16 tiles; N ragged or the LM's; K a
    multiple of 128, mostly the LM's 1024 / 2048 / 3072), store and residual
    forms: every member equals its own ovh_linear_q bit for bit."""
    import ovnative_amd as ov
    rng = np.random.default_rng(808)
    for it in range(10):
        n_mem = int(rng.integers(1, 9))
        probs, cins = [], []
        for _ in range(n_mem):
            M = int(rng.integers(1, 201 if it % 2 else 129))
            N = int(rng.choice([rng.integers(1, 700), 1024, 2048, 3072]))
            K = int(rng.choice([1024, 2048, 3072, 128 * rng.integers(1, 12)]))
            A = rng.standard_normal((M, K)).astype(np.float32)
            q, s = oracle.quantize_weight_rows((rng.standard_normal((N, K)) * 0.02)
                                               .astype(np.float32))
            aq, asc = ov.s8_nk_quantize(dev(A))
            probs.append((aq, asc, ov.Weight.from_host(q, s)))
            cins.append(rng.standard_normal((M, N)).astype(np.float32))
        accumulate = bool(it % 3 == 0)
        got = [dev(c) for c in cins]
        ov.linear_q_grouped(probs, got, accumulate=accumulate)
        for j, ((aq, asc, w), g, c) in enumerate(zip(probs, got, cins)):
            want = dev(c)
            ov.linear_q(aq, asc, w, want, accumulate=accumulate)
            assert np.array_equal(bits(host(g)), bits(host(want))), (it, j)


def test_linear_q_grouped_errors(oracle):
    import ovnative_amd as ov
    rng = np.random.default_rng(3)
    q, s = oracle.quantize_weight_rows((rng.standard_normal((64, 96)) * 0.1).astype(np.float32))
    w = ov.Weight.from_host(q, s)
    aq, asc = ov.s8_nk_quantize(dev(rng.standard_normal((5, 96)).astype(np.float32)))
    with pytest.raises(ov.OvhError):       # K = 96: not a multiple of 128
        ov.linear_q_grouped([(aq, asc, w)])
    q2, s2 = oracle.quantize_weight_rows((rng.standard_normal((64, 128)) * 0.1).astype(np.float32))
    w2 = ov.Weight.from_host(q2, s2)
    aq2, asc2 = ov.s8_nk_quantize(dev(rng.standard_normal((5, 128)).astype(np.float32)))
    with pytest.raises(ov.InvalidArgument):  # nine members
        ov.linear_q_grouped([(aq2, asc2, w2)] * 9)
    assert ov.linear_q_grouped([]) == []


# ---------------------------------------------------------------------------
# fused producers at LM shapes vs the oracle

@pytest.mark.parametrize("M,K", [(600, 1024), (128, 1024), (1, 1024), (40, 256), (7, 512), (4099, 1024),
                                 (9, 768), (13, 100), (5, 1280)])
def test_rmsnorm_quantize_vs_oracle(oracle, M, K):
    import ovnative_amd as ov
    rng = np.random.default_rng(M + K)
    x = (rng.standard_normal((M, K)) * rng.uniform(0.5, 4)).astype(np.float32)
    w = rng.uniform(0.1, 1.1, K).astype(np.float32)
    aq, asc = ov.rmsnorm_quantize(dev(x), dev(w), 1e-6)
    aq_r, asc_r = oracle.rmsnorm_quantize(x, w, 1e-6)
    assert np.array_equal(host(aq), u8_to_s8(aq_r, K))
    assert np.array_equal(bits(host(asc)), bits(asc_r))


@pytest.mark.parametrize("M,K", [(600, 3072), (128, 3072), (3, 64)])
def test_silu_mul_quantize_vs_oracle(oracle, M, K):
    import ovnative_amd as ov
    rng = np.random.default_rng(M * K)
    g = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    u = rng.standard_normal((M, K)).astype(np.float32)
    aq, asc = ov.silu_mul_quantize(dev(g), dev(u))
    aq_r, asc_r = oracle.silu_mul_quantize(g, u)
    assert np.array_equal(host(aq), u8_to_s8(aq_r, K))
    assert np.array_equal(bits(host(asc)), bits(asc_r))


# ---------------------------------------------------------------------------
# boundary behaviour

def test_linear_quantizes_internally(oracle):
    """ovh_linear (= linear_s8_nk_packed[_add]) == quantise + linear_q."""
    import ovnative_amd as ov
    rng = np.random.default_rng(8)
    A, Wf = _rand_problem(rng, 70, 192, 1024)
    q, s = oracle.quantize_weight_rows(Wf)
    w = ov.Weight.from_host(q, s)
    C = host(ov.linear(dev(A), w))
    assert np.array_equal(bits(C), bits(_oracle_linear(oracle, A, q, s)))
    Cin = rng.standard_normal((70, 192)).astype(np.float32)
    Cacc = dev(Cin)
    ov.linear(dev(A), w, Cacc, accumulate=True)
    assert np.array_equal(bits(host(Cacc)), bits(_oracle_linear(oracle, A, q, s, Cin)))


# tile-major codes inside (K = 1000: a K tail; 994: no 4-float vector loads),
# then row-major codes (K = 96)
@pytest.mark.parametrize("K", [1024, 1000, 994, 96])
def test_linear_workspace_growth_and_streams(oracle, K):
    """ovh_linear keeps its quantised copy of A per stream and grows it: rows
    rising and falling on the current stream and on a second stream, every
    result against the oracle."""
    import ovnative_amd as ov
    rng = np.random.default_rng(K)
    _, Wf = _rand_problem(rng, 1, 256, K)
    q, s = oracle.quantize_weight_rows(Wf)
    w = ov.Weight.from_host(q, s)
    side = torch.cuda.Stream()
    for M in (40, 700, 17, 1500, 300):
        A, _ = _rand_problem(rng, M, 1, K)
        want = bits(_oracle_linear(oracle, A, q, s))
        assert np.array_equal(bits(host(ov.linear(dev(A), w))), want), M
        dA = dev(A)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            C = ov.linear(dA, w)
        torch.cuda.current_stream().wait_stream(side)
        assert np.array_equal(bits(host(C)), want), M


def test_linear_in_a_graph(oracle):
    """ovh_linear captured in a graph on a stream whose workspace would fit:
    the captured call still quantises into a buffer the graph owns, so every
    replay equals the eager result, also after eager calls on the capture
    stream that grow (free and reallocate) that stream's workspace, and when
    the graph is replayed on another stream."""
    import ovnative_amd as ov
    rng = np.random.default_rng(21)
    A, Wf = _rand_problem(rng, 200, 512, 1024)
    q, s = oracle.quantize_weight_rows(Wf)
    w = ov.Weight.from_host(q, s)
    want = bits(_oracle_linear(oracle, A, q, s))
    s0, s1 = torch.cuda.Stream(), torch.cuda.Stream()
    dA, C = dev(A), torch.zeros((200, 512), dtype=torch.float32, device="cuda")
    A2, _ = _rand_problem(rng, 300, 1, 1024)
    A3, _ = _rand_problem(rng, 1500, 1, 1024)
    dA2, dA3 = dev(A2), dev(A3)
    with torch.cuda.stream(s0):
        ov.linear(dA2, w)                       # the workspace now holds 300 rows
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s0):
        ov.linear(dA, w, C)
    want2 = bits(_oracle_linear(oracle, A2, q, s))
    want3 = bits(_oracle_linear(oracle, A3, q, s))
    for rep in range(3):
        C.fill_(7.0)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(host(C)), want), rep
        with torch.cuda.stream(s0):
            C3 = ov.linear(dA3, w)              # grows the workspace: frees the old buffer
            C2 = ov.linear(dA2, w)
        torch.cuda.synchronize()
        assert np.array_equal(bits(host(C3)), want3), rep
        assert np.array_equal(bits(host(C2)), want2), rep
        C.fill_(7.0)
        torch.cuda.synchronize()
        with torch.cuda.stream(s1):
            g.replay()                          # the graph's buffer, not s1's or s0's
        with torch.cuda.stream(s0):
            C2 = ov.linear(dA2, w)
        torch.cuda.synchronize()
        assert np.array_equal(bits(host(C)), want), rep
        assert np.array_equal(bits(host(C2)), want2), rep


def test_ldc_and_slices_errors(oracle):
    import ovnative_amd as ov
    rng = np.random.default_rng(4)
    A, Wf = _rand_problem(rng, 9, 128, 64)
    q, s = oracle.quantize_weight_rows(Wf)
    w = ov.Weight.from_host(q, s)
    aq, asc = ov.s8_nk_quantize(dev(A))
    # ldc > N writes a strided sub-block and leaves the rest untouched
    big = torch.full((9, 200), 7.0, device="cuda")
    ov.load().ovh_linear_q(9, ov._dptr(aq), ov._dptr(asc), w.handle, ov._dptr(big), 200, 0,
                           ov._stream())
    big = host(big)
    assert np.array_equal(bits(big[:, :128]), bits(_oracle_linear(oracle, A, q, s)))
    assert np.all(big[:, 128:] == 7.0)
    with pytest.raises(ov.InvalidArgument):
        ov.linear_q_sliced(aq, asc, w, [96, 32])      # not multiples of 64
    with pytest.raises(ov.InvalidArgument):
        ov.linear_q_sliced(aq, asc, w, [64])          # does not sum to N
    with pytest.raises(ov.InvalidArgument):
        ov.linear_q(aq, asc, w, torch.zeros((9, 64), device="cuda"))  # ldc < N


def test_weight_layout_roundtrip():
    import ovnative_amd as ov
    rng = np.random.default_rng(6)
    for (N, K) in [(7, 69), (130, 1024), (64, 33)]:
        q = rng.integers(-127, 128, (N, K)).astype(np.int8)
        s = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
        for layout, src in ((0, q), (1, np.ascontiguousarray(q.T))):
            w = ov.Weight.from_host(src, s, layout=layout)
            dq, ds = w.download()
            assert np.array_equal(host(dq), q) and np.array_equal(bits(host(ds)), bits(s))
            wd = ov.Weight.from_device(dev(src), dev(s), layout=layout)
            dq, ds = wd.download()
            assert np.array_equal(host(dq), q)


def test_concat_sliced_equals_separate(oracle):
    """Sliced merged GEMM (qkv at LM shape) == three separate GEMMs, byte for byte
    (cpp/tests/test_gemm.cpp:240-297)."""
    import ovnative_amd as ov
    rng = np.random.default_rng(12)
    M, K = 300, 1024
    A = rng.standard_normal((M, K)).astype(np.float32)
    parts, hs = [], []
    for n in (2048, 1024, 1024):
        q, s = oracle.quantize_weight_rows((rng.standard_normal((n, K)) * 0.02).astype(np.float32))
        parts.append((q, s))
        hs.append(ov.Weight.from_host(q, s))
    merged = ov.Weight.concat(hs)
    aq, asc = ov.s8_nk_quantize(dev(A))
    outs = ov.linear_q_sliced(aq, asc, merged, [2048, 1024, 1024])
    for (q, s), h, o in zip(parts, hs, outs):
        assert np.array_equal(bits(host(o)), bits(host(ov.linear_q(aq, asc, h))))


def test_empty_inputs_are_no_ops():
    """M = 0 (and K = 0 for the quantisers) returns OK without touching any
    buffer, as the reference's early returns do (cpp/src/backend/cpu/gemm.cpp:710,
    :724, :761, :779)."""
    import ovnative_amd as ov
    rng = np.random.default_rng(21)
    q = rng.integers(-127, 128, (64, 96)).astype(np.int8)
    w = ov.Weight.from_host(q, rng.uniform(1e-3, 1e-2, 64).astype(np.float32))
    e = torch.empty((0, 96), device="cuda")
    aq, asc = ov.s8_nk_quantize(e)
    assert aq.shape == (0, 96) and asc.shape == (0, 3)
    aq, asc = ov.rmsnorm_quantize(e, torch.ones(96, device="cuda"))
    assert aq.shape == (0, 96)
    aq, asc = ov.silu_mul_quantize(e, e)
    assert aq.shape == (0, 96)
    assert ov.linear_q(aq, asc, w).shape == (0, 64)
    assert ov.linear(e, w).shape == (0, 64)
    assert [o.shape for o in ov.linear_q_sliced(aq, asc, w, [64])] == [(0, 64)]
    # a zero-width quantiser call writes nothing: a sentinel survives
    lib = ov.load()
    A = torch.randn(4, 32, device="cuda")
    aq = torch.full((4, 32), 7, dtype=torch.int8, device="cuda")
    asc = torch.full((4, 1), 3.0, device="cuda")
    for rows, cols in ((0, 32), (4, 0)):
        assert lib.ovh_s8_nk_quantize(rows, cols, ctypes.c_void_p(A.data_ptr()),
                                      ctypes.c_void_p(aq.data_ptr()),
                                      ctypes.c_void_p(asc.data_ptr()), None) == 0
    torch.cuda.synchronize()
    assert bool((aq == 7).all()) and bool((asc == 3.0).all())


# ---------------------------------------------------------------------------
# per-block int32 of the production kernel, and the SiLU-fused gate/up operator

def tile_major(aq: np.ndarray, M: int) -> np.ndarray:
    """Row-major codes [M, Kp] -> the runner's tile-major layout (1 KiB tiles of
    32 rows x 32 k; inside a tile (m/16 % 2)*512 + (k/8 % 4)*128 + (m%16)*8 + k%8),
    rows padded with zeros to a multiple of 128."""
    Kp = aq.shape[1]
    Mp = (M + 127) // 128 * 128
    a = np.zeros((Mp, Kp), np.int8)
    a[:M] = aq[:M]
    # [mt, h, r, kb, g, e] -> [mt, kb, h, g, r, e]
    t = a.reshape(Mp // 32, 2, 16, Kp // 32, 4, 8).transpose(0, 3, 1, 4, 2, 5)
    return np.ascontiguousarray(t).reshape(-1)


def _brute_blocks(aq_rows: np.ndarray, q: np.ndarray) -> np.ndarray:
    """Integer brute force: [rows, N, Kb] int64 block dot products."""
    Kp = aq_rows.shape[1]
    N, K = q.shape
    w = np.zeros((N, Kp), np.int64)
    w[:, :K] = q
    w = w.reshape(N, Kp // 32, 32)
    return np.stack([(a.astype(np.int64).reshape(1, Kp // 32, 32) * w).sum(axis=2)
                     for a in aq_rows])


@pytest.mark.parametrize("M,N,K", [
    (256, 3072, 1024),
    (600, 4096, 1024), (600, 6144, 1024),   # config 3: q/k/v, gate/up
    (600, 1024, 3072), (600, 1024, 2048),   # config 3: down, o_proj
    (128, 1024, 3072), (128, 2048, 1024),   # config 2 (3-stage ring tiles)
    (2400, 1024, 1024), (1200, 4096, 1024),  # 128x64 and 64x64 tiles
])
@pytest.mark.parametrize("tiled", [False, True], ids=["rowmajor", "tilemajor"])
def test_block_dots_production_kernel(oracle, M, N, K, tiled):
    """ovh_block_dots / _tiled run the kernel and tile ovh_linear_q launches for
    the shape (K a multiple of 128: the 16x16 kernel): its per-block int32 sums
    equal integer brute force on sampled rows (gemm.cpp:455-474), with the codes
    row-major (the C ABI's format) and tile-major (the runner's)."""
    import ovnative_amd as ov
    rng = np.random.default_rng(M + 3 * N + 7 * K + tiled)
    A, Wf = _rand_problem(rng, M, N, K)
    q, s = oracle.quantize_weight_rows(Wf)
    w = ov.Weight.from_host(q, s)
    aq, asc = ov.s8_nk_quantize(dev(A))
    aq_h = host(aq)
    if tiled:
        t = tile_major(aq_h, M)
        assert t.size == ov.load().ovh_tiled_codes_bytes(M, K)
        blocks = ov.block_dots(dev(t), w, M=M, tiled=True)
    else:
        blocks = ov.block_dots(aq, w)
    rows = np.sort(np.concatenate([rng.choice(M, min(M, 20), replace=False), [M - 1]]))
    got = blocks[torch.from_numpy(rows).cuda()].cpu().numpy()
    want = _brute_blocks(aq_h[rows], q)
    assert np.array_equal(got.astype(np.int64), want)


@pytest.mark.parametrize("M,N,K", [(600, 1024, 2048), (600, 1024, 3072), (128, 4096, 1024),
                                   (37, 320, 256)])
def test_linear_q_tiled_equals_rowmajor(oracle, M, N, K):
    """ovh_linear_q_tiled (the runner's tile-major codes) gives ovh_linear_q's
    bits, store and residual forms; the device layout helper matches the
    host restatement of the layout."""
    import ovnative_amd as ov
    rng = np.random.default_rng(M + N + K)
    A, Wf = _rand_problem(rng, M, N, K)
    q, s = oracle.quantize_weight_rows(Wf)
    w = ov.Weight.from_host(q, s)
    aq, asc = ov.s8_nk_quantize(dev(A))
    t = ov.tile_major(aq)
    assert np.array_equal(host(t), tile_major(host(aq), M))
    assert np.array_equal(bits(host(ov.linear_q_tiled(t, asc, w, M))),
                          bits(host(ov.linear_q(aq, asc, w))))
    Cin = rng.standard_normal((M, N)).astype(np.float32)
    c1, c2 = dev(Cin), dev(Cin)
    ov.linear_q(aq, asc, w, c1, accumulate=True)
    ov.linear_q_tiled(t, asc, w, M, c2, accumulate=True)
    assert np.array_equal(bits(host(c1)), bits(host(c2)))


@pytest.mark.parametrize("M,N,K", [(600, 1024, 2048), (600, 1024, 3072), (128, 1024, 3072),
                                   (1, 1024, 2048), (37, 256, 512), (300, 512, 1024),
                                   (1320, 1024, 2048), (2047, 768, 1024), (2048, 1024, 2048),
                                   (4133, 1024, 3072), (2400, 256, 1024),
                                   # both sides of the tile-shape changes (256, 512, 1024 rows;
                                   # K = 1024 with 8-block stages, 1152 without)
                                   (255, 1024, 1024), (256, 1024, 1152), (511, 512, 3072),
                                   (512, 1024, 1152), (1023, 1024, 2048), (1024, 256, 1024)])
def test_linear_q_norm_equals_two_calls(oracle, M, N, K):
    """ovh_linear_q_norm (the runner's o_proj / down launch, with the RMSNorm +
    quantise that follows it: lm.cpp:281 + :292, :311 + :232) gives the bits of
    ovh_linear_q_tiled in its residual form followed by ovh_rmsnorm_quantize,
    codes tile-major, over repeated calls on one counter buffer (32-row bands
    below 2048 rows, 64-row bands from 2048); the norm's codes and scales are
    also the oracle's rmsnorm_quantize of the updated rows."""
    import ovnative_amd as ov
    rng = np.random.default_rng(7 * M + N + K)
    A, Wf = _rand_problem(rng, M, N, K)
    q, s = oracle.quantize_weight_rows(Wf)
    w = ov.Weight.from_host(q, s)
    aq, asc = ov.s8_nk_quantize(dev(A))
    t = ov.tile_major(aq)
    nw_h = rng.uniform(0.1, 1.1, N).astype(np.float32)
    nw = dev(nw_h)
    cnt = ov.band_counters(M)
    Cin = rng.standard_normal((M, N)).astype(np.float32)
    want_x = dev(Cin)
    ov.linear_q_tiled(t, asc, w, M, want_x, accumulate=True)
    want_q, want_s = ov.rmsnorm_quantize(want_x, nw, 1e-6)
    aq_r, asc_r = oracle.rmsnorm_quantize(host(want_x), nw_h, 1e-6)
    assert np.array_equal(host(want_q), u8_to_s8(aq_r, N))
    assert np.array_equal(bits(host(want_s)), bits(asc_r))
    for rep in range(3):
        x = dev(Cin)
        nq, nsc = ov.linear_q_norm(t, asc, w, x, nw, cnt, 1e-6)
        assert np.array_equal(bits(host(x)), bits(host(want_x))), rep
        assert np.array_equal(host(nq), tile_major(host(want_q), M)), rep
        assert np.array_equal(bits(host(nsc)), bits(host(want_s))), rep
    assert host(cnt)[0] == 0  # no hand-off wait ran out


def test_linear_q_norm_wait_running_out_is_flagged(oracle):
    """A helper whose wait for the rest of its band runs out flags the counter
    buffer's error word (the condition forced from the host: band 0's counter
    set to 1, so the band's last arrival waits for a count the launch never
    reaches; its wait is bounded, ~0.1 s), and a clean buffer works again."""
    import ovnative_amd as ov
    rng = np.random.default_rng(5)
    A, Wf = _rand_problem(rng, 32, 1024, 1024)
    q, s = oracle.quantize_weight_rows(Wf)
    w = ov.Weight.from_host(q, s)
    aq, asc = ov.s8_nk_quantize(dev(A))
    t = ov.tile_major(aq)
    nw = dev(rng.uniform(0.5, 1.5, 1024).astype(np.float32))
    cnt = ov.band_counters()
    stride = 64  # 64-bit words per counter slot: the error word's slot, then band 0's
    cnt[stride] = 1
    ov.linear_q_norm(t, asc, w, dev(np.zeros((32, 1024), np.float32)), nw, cnt)
    torch.cuda.synchronize()
    assert host(cnt)[0] != 0
    cnt.zero_()
    x = dev(np.zeros((32, 1024), np.float32))
    nq, nsc = ov.linear_q_norm(t, asc, w, x, nw, cnt)
    want_x = dev(np.zeros((32, 1024), np.float32))
    ov.linear_q_tiled(t, asc, w, 32, want_x, accumulate=True)
    want_q, want_s = ov.rmsnorm_quantize(want_x, nw, 1e-6)
    assert host(cnt)[0] == 0
    assert np.array_equal(host(nq), tile_major(host(want_q), 32))
    assert np.array_equal(bits(host(nsc)), bits(host(want_s)))


def test_linear_q_norm_counters_shared_across_widths(oracle):
    """One counter buffer for launches of different widths and heights in any
    order (each launch's band counters move on to the next launch boundary
    whatever its column-tile count): every launch equals the two-call form and
    the error word stays 0; the 64-row bands from 2048 rows share it too."""
    import ovnative_amd as ov
    rng = np.random.default_rng(9)
    cnt = ov.band_counters(4096)
    for M, N, K in [(600, 1024, 2048), (600, 256, 1024), (300, 512, 1024), (600, 1024, 3072),
                    (37, 768, 1024), (2100, 1024, 1024), (600, 256, 1024), (2100, 512, 1024),
                    (600, 1024, 2048)]:
        A, Wf = _rand_problem(rng, M, N, K)
        q, s = oracle.quantize_weight_rows(Wf)
        w = ov.Weight.from_host(q, s)
        aq, asc = ov.s8_nk_quantize(dev(A))
        t = ov.tile_major(aq)
        nw = dev(rng.uniform(0.5, 1.5, N).astype(np.float32))
        x0 = rng.standard_normal((M, N)).astype(np.float32)
        x = dev(x0)
        nq, nsc = ov.linear_q_norm(t, asc, w, x, nw, cnt)
        want_x = dev(x0)
        ov.linear_q_tiled(t, asc, w, M, want_x, accumulate=True)
        want_q, want_s = ov.rmsnorm_quantize(want_x, nw, 1e-6)
        assert host(cnt)[0] == 0, (M, N, K)
        assert np.array_equal(bits(host(x)), bits(host(want_x))), (M, N, K)
        assert np.array_equal(host(nq), tile_major(host(want_q), M)), (M, N, K)
        assert np.array_equal(bits(host(nsc)), bits(host(want_s))), (M, N, K)
        # between launches every band word stands at a launch boundary (0 or
        # 2^15 arrivals) with its per-XCD arrival fields cleared
        words = host(cnt).view(np.uint64)[64::64]
        assert np.all((words & np.uint64(0x7FFF)) == 0) and np.all((words >> np.uint64(16)) == 0)


def test_linear_q_norm_errors(oracle):
    import ovnative_amd as ov
    q, s = oracle.quantize_weight_rows(np.ones((1024, 1100), np.float32) * 0.01)
    w = ov.Weight.from_host(q, s)          # K = 1100: 35 blocks, not a multiple of 4
    aq, asc = ov.s8_nk_quantize(dev(np.ones((4, 1100), np.float32)))
    x = dev(np.zeros((4, 1024), np.float32))
    nw = dev(np.ones(1024, np.float32))
    cnt = ov.band_counters()
    with pytest.raises(ov.OvhError, match="multiple of 128"):
        ov.linear_q_norm(ov.tile_major(aq), asc, w, x, nw, cnt)
    q, s = oracle.quantize_weight_rows(np.ones((320, 1024), np.float32) * 0.01)
    w = ov.Weight.from_host(q, s)          # N = 320
    aq, asc = ov.s8_nk_quantize(dev(np.ones((4, 1024), np.float32)))
    with pytest.raises(ov.OvhError, match="N must be"):
        ov.linear_q_norm(ov.tile_major(aq), asc, w, dev(np.zeros((4, 320), np.float32)),
                         dev(np.ones(320, np.float32)), cnt)


@pytest.mark.parametrize("M", [1, 100, 128, 256, 600, 2400])
def test_silu_gate_linear_vs_oracle(oracle, M):
    """ovh_silu_gate_linear (gate/up GEMM with silu*up and its quantisation in the
    epilogue) == the reference's composition: the sliced gate/up GEMM, then
    silu_mul_quantize_f32 (lm.cpp:293-311), byte for byte, in every tile band of
    the fused kernel; also equal to the device's own unfused composition."""
    import ovnative_amd as ov
    rng = np.random.default_rng(40 + M)
    I, K = 3072, 1024
    A = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    qg, sg = oracle.quantize_weight_rows((rng.standard_normal((I, K)) * 0.02).astype(np.float32))
    qu, su = oracle.quantize_weight_rows((rng.standard_normal((I, K)) * 0.02).astype(np.float32))
    wg, wu = ov.Weight.from_host(qg, sg), ov.Weight.from_host(qu, su)
    gu = ov.gate_up_weight(wg, wu)
    aq, asc = ov.s8_nk_quantize(dev(A))
    hq, hsc = ov.silu_gate_linear(aq, asc, gu)
    hq, hsc = host(hq), host(hsc)
    gate = _oracle_linear(oracle, A, qg, sg)
    up = _oracle_linear(oracle, A, qu, su)
    hq_r, hsc_r = oracle.silu_mul_quantize(gate, up)
    assert np.array_equal(hq, u8_to_s8(hq_r, I))
    assert np.array_equal(bits(hsc), bits(hsc_r))
    merged = ov.Weight.concat([wg, wu])
    g_d, u_d = ov.linear_q_sliced(aq, asc, merged, [I, I])
    hq2, hsc2 = ov.silu_mul_quantize(g_d, u_d)
    assert np.array_equal(host(hq2), hq) and np.array_equal(bits(host(hsc2)), bits(hsc))


def test_silu_gate_linear_small_width_and_errors(oracle):
    """I = 320 (N = 640, not a multiple of 256) at M = 37; a plain weight is
    refused by the fused operator and the interleaved one by the plain GEMMs;
    K = 96 is not covered (OV_ERR_NOT_IMPLEMENTED)."""
    import ovnative_amd as ov
    rng = np.random.default_rng(77)
    M, I, K = 37, 320, 256
    A = rng.standard_normal((M, K)).astype(np.float32)
    qg, sg = oracle.quantize_weight_rows((rng.standard_normal((I, K)) * 0.05).astype(np.float32))
    qu, su = oracle.quantize_weight_rows((rng.standard_normal((I, K)) * 0.05).astype(np.float32))
    wg, wu = ov.Weight.from_host(qg, sg), ov.Weight.from_host(qu, su)
    gu = ov.gate_up_weight(wg, wu)
    aq, asc = ov.s8_nk_quantize(dev(A))
    hq, hsc = ov.silu_gate_linear(aq, asc, gu)
    hq_r, hsc_r = oracle.silu_mul_quantize(_oracle_linear(oracle, A, qg, sg),
                                           _oracle_linear(oracle, A, qu, su))
    assert np.array_equal(host(hq), u8_to_s8(hq_r, I))
    assert np.array_equal(bits(host(hsc)), bits(hsc_r))
    with pytest.raises(ov.InvalidArgument):
        ov.silu_gate_linear(aq, asc, wg)
    with pytest.raises(ov.InvalidArgument):
        ov.linear_q(aq, asc, gu)
    with pytest.raises(ov.InvalidArgument):
        ov.Weight.concat([gu, wg])
    q96 = rng.integers(-127, 128, (64, 96)).astype(np.int8)
    s96 = np.full(64, 1e-2, np.float32)
    g96 = ov.gate_up_weight(ov.Weight.from_host(q96, s96), ov.Weight.from_host(q96, s96))
    aq96, asc96 = ov.s8_nk_quantize(dev(rng.standard_normal((5, 96)).astype(np.float32)))
    with pytest.raises(ov.OvhError) as e:
        ov.silu_gate_linear(aq96, asc96, g96)
    assert e.value.code == ov.OV_ERR_NOT_IMPLEMENTED


# ---------------------------------------------------------------------------
# Mat's fp32 branch (the fp32 audio head): split-f16 matrix-core products

# |gpu - reference| <= F32_TOL * sum_k |A[m,k] W[k,n]| per output: the split
# keeps ~22 bits of each operand (hi + lo; lo*lo dropped, ~2^-22 relative per
# product) and both sides sum in fp32 in different orders.
F32_TOL = 2.0 ** -18


def _check_f32(got, want, A, W):
    bound = np.abs(A.astype(np.float64)) @ np.abs(W.astype(np.float64))
    err = np.abs(got.astype(np.float64) - want)
    ratio = float((err / np.maximum(bound, 1e-30)).max())
    rel = float(err.max() / max(np.abs(want).max(), 1e-30))
    print(f"linear_f32 {A.shape} x {W.shape}: max |d| / sum|aw| = {ratio:.3g}, "
          f"max |d| / max|ref| = {rel:.3g}")
    assert ratio <= F32_TOL
    assert rel <= 1e-3   # the north star's fp32 bar


@pytest.mark.parametrize("M,N,K", [(600, 8200, 1024), (37, 69, 100), (1, 64, 16), (130, 136, 33),
                                   (256, 1024, 3072)])
def test_linear_f32_vs_oracle(oracle, M, N, K):
    """ovh_linear_f32 against the oracle's linear_f32_ld (the reference's fma chain,
    pinned bit for bit to the compiled reference): store and accumulate, weights
    uploaded in both OVW1 layouts; (600, 8200, 1024) is the fp32 audio head at
    BASELINE config 4."""
    import ovnative_amd as ov
    rng = np.random.default_rng(M + N + K)
    A = (rng.standard_normal((M, K)) * rng.uniform(0.5, 4)).astype(np.float32)
    A[:, rng.integers(0, K, 3)] *= 20
    W = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    want = oracle.linear_f32(A, W)
    w_kn = ov.Weight.from_host_f32(W, layout=1)
    got = host(ov.linear_f32(dev(A), w_kn))
    _check_f32(got, want, A, W)
    w_nk = ov.Weight.from_host_f32(np.ascontiguousarray(W.T), layout=0)
    assert np.array_equal(bits(host(ov.linear_f32(dev(A), w_nk))), bits(got))
    Cin = rng.standard_normal((M, N)).astype(np.float32)
    c = dev(Cin)
    ov.linear_f32(dev(A), w_kn, c, accumulate=True)
    assert np.array_equal(bits(host(c)), bits((Cin + got).astype(np.float32)))


def test_linear_f32_ranges_and_errors(oracle):
    """Power-of-two row and column scales keep tiny and huge operands in f16's
    range (values near 1e-30 and 1e30 in different rows/columns), an all-zero row
    gives zeros, and the int8 operators refuse an fp32 weight (and back)."""
    import ovnative_amd as ov
    rng = np.random.default_rng(3)
    M, N, K = 6, 40, 64
    A = rng.standard_normal((M, K)).astype(np.float32)
    A[1] *= 1e-30
    A[2] *= 1e30
    A[3] = 0
    W = rng.standard_normal((K, N)).astype(np.float32)
    W[:, 5] *= 1e-25
    W[:, 6] *= 1e-10
    want = oracle.linear_f32(A, W)
    w = ov.Weight.from_host_f32(W)
    got = host(ov.linear_f32(dev(A), w))
    assert np.all(got[3] == 0)
    _check_f32(got, want, A, W)
    aq, asc = ov.s8_nk_quantize(dev(A))
    with pytest.raises(ov.InvalidArgument):
        ov.linear_q(aq, asc, w)
    q, s = oracle.quantize_weight_rows(rng.standard_normal((N, K)).astype(np.float32))
    with pytest.raises(ov.InvalidArgument):
        ov.linear_f32(dev(A), ov.Weight.from_host(q, s))
