"""GPU parity for the attention side of a decoder layer, through the C ABI.

Bars:
  * RoPE tables: within 1 ulp of the oracle (libm cosf/sinf vs correctly
    rounded cos/sin of the same float angle);
  * qk-norm + RoPE: bit-exact for the same tables;
  * attention (fp32, different summation order on the matrix core): max
    absolute error <= ATTN_TOL * max(1, max|ref|) per case, and fully masked
    rows exactly zero.  ATTN_TOL = 2e-5 is 50x tighter than the north-star
    fp32 bar (max relative error 1e-3).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

ATTN_TOL = 2e-5


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import ovnative_amd
    ovnative_amd.load()
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


def _cases(golden, prefix):
    return sorted({k.split("_")[0] for k in golden if k.startswith(prefix)})


def test_rope_tables(oracle):
    import ovnative_amd as ov
    pos = np.concatenate([np.arange(300), [0, 1023, 4095, 40000, 65535]]).astype(np.int64)
    c, s = ov.rope_tables(dev(pos), 128, 1e6)
    rc, rs = oracle.rope_tables(pos, 128, 1e6)
    for got, want in ((host(c), rc), (host(s), rs)):
        ulps = np.abs(bits(got).astype(np.int64) - bits(want).astype(np.int64))
        assert ulps.max() <= 1
        assert (ulps > 0).mean() < 0.01


def test_qk_norm_rope_golden(golden, oracle):
    import ovnative_amd as ov
    for c in _cases(golden, "qknr"):
        rows, nh, nkv, D = (int(x) for x in golden[c + "_dims"])
        ct, st = oracle.rope_tables(golden[c + "_pos"], D, 1e6)
        q, k = dev(golden[c + "_q"]), dev(golden[c + "_k"])
        ov.qk_norm_rope(q, k, dev(golden[c + "_qw"]), dev(golden[c + "_kw"]), nh, nkv, D,
                        dev(ct), dev(st), 1e-6)
        assert np.array_equal(bits(host(q)), bits(golden[c + "_qo"])), c
        assert np.array_equal(bits(host(k)), bits(golden[c + "_ko"])), c


@pytest.mark.parametrize("rows,nh,nkv,D", [(600, 16, 8, 128), (37, 4, 2, 64), (1, 16, 8, 128)])
def test_qk_norm_rope_vs_oracle(oracle, rows, nh, nkv, D):
    import ovnative_amd as ov
    rng = np.random.default_rng(rows + D)
    q = (rng.standard_normal((rows, nh * D)) * 3).astype(np.float32)
    k = rng.standard_normal((rows, nkv * D)).astype(np.float32)
    qw = rng.uniform(0.2, 2.0, D).astype(np.float32)
    kw = rng.uniform(0.2, 2.0, D).astype(np.float32)
    pos = rng.integers(0, 3000, rows).astype(np.int64)
    # bit-exact with the oracle's own tables ...
    ct, st = oracle.rope_tables(pos, D)
    qo, ko = oracle.qk_norm_rope(q, k, qw, kw, nh, nkv, D, tables=(ct, st))
    qd, kd = dev(q), dev(k)
    ov.qk_norm_rope(qd, kd, dev(qw), dev(kw), nh, nkv, D, dev(ct), dev(st))
    assert np.array_equal(bits(host(qd)), bits(qo)) and np.array_equal(bits(host(kd)), bits(ko))
    # ... and within a few ulp with the device tables
    c2, s2 = ov.rope_tables(dev(pos), D)
    qd, kd = dev(q), dev(k)
    ov.qk_norm_rope(qd, kd, dev(qw), dev(kw), nh, nkv, D, c2, s2)
    np.testing.assert_allclose(host(qd), qo, rtol=0, atol=4e-7 * np.abs(qo).max())
    np.testing.assert_allclose(host(kd), ko, rtol=0, atol=4e-7 * np.abs(ko).max())


def _attn_err(got, want):
    return float(np.abs(got - want).max() / max(1.0, float(np.abs(want).max())))


def test_attention_golden(golden):
    import ovnative_amd as ov
    for c in _cases(golden, "attn"):
        q, k, v = golden[c + "_q"], golden[c + "_k"], golden[c + "_v"]
        S, D = q.shape
        if D != 128:
            continue
        masked = int(golden[c + "_masked"])
        bias = dev(golden[c + "_bias"]) if masked else None
        out = host(ov.attention(dev(q), dev(k), dev(v), [(bias, S, 0, 0)], 1, 1, 128))
        want = golden[c + "_out"]
        assert _attn_err(out, want) <= ATTN_TOL, c
        dead = np.all(want == 0, axis=1)
        assert np.all(out[dead] == 0), c


def _segments(rng, seg_rows, masked):
    segs, biases, r0 = [], [], 0
    for rows in seg_rows:
        b = None
        if masked:
            b = np.where(rng.random((rows, rows)) < 0.3, -1e30, 0.0).astype(np.float32)
            b[rows // 2] = -1e30            # a fully masked row
        segs.append((b, rows, r0, r0))
        r0 += rows
    return segs, r0


@pytest.mark.parametrize("split", [False, True], ids=["fp32", "split_f16"])
@pytest.mark.parametrize("seg_rows,nh,nkv,masked", [
    ([300, 300], 16, 8, False),   # BASELINE config 3/4: CFG batch 2, seq 300
    ([300, 260], 16, 8, True),    # ragged CFG (cond S, uncond T) with masks
    ([1024], 16, 8, False),       # one sequence of config 5
    ([700, 650], 16, 8, True),    # long segments, masked
    ([700] * 11, 16, 8, True),    # many long segments (split: the LDS-shared K/V form)
    ([640, 3], 8, 2, True),       # KV group of 4, a segment shorter than the tile
    ([700], 4, 4, False),         # KV group of 1
    ([1, 33, 64, 65], 4, 2, True),
    ([7], 2, 2, False),
    ([40, 33], 256, 1, True),     # a KV group of 256 heads (more than a workgroup's rows)
])
def test_attention_vs_oracle(oracle, seg_rows, nh, nkv, masked, split):
    import ovnative_amd as ov
    rng = np.random.default_rng(sum(seg_rows) + nh)
    D = 128
    segs, T = _segments(rng, seg_rows, masked)
    q = rng.standard_normal((T, nh * D)).astype(np.float32)
    k = rng.standard_normal((T, nkv * D)).astype(np.float32)
    v = rng.standard_normal((T, nkv * D)).astype(np.float32)
    want = oracle.attention(q, k, v, segs, nh, nkv, D)
    dsegs = [(None if b is None else dev(b), rows, r0, k0) for b, rows, r0, k0 in segs]
    got = host(ov.attention(dev(q), dev(k), dev(v), dsegs, nh, nkv, D, split=split))
    err = _attn_err(got, want)
    print(f"attention {'split' if split else 'fp32'} {seg_rows} nh={nh} nkv={nkv} "
          f"masked={masked}: max err {err:.3g}")
    assert err <= ATTN_TOL
    dead = np.all(want == 0, axis=1)
    assert np.all(got[dead] == 0)


@pytest.mark.parametrize("seg_rows,nh,nkv,masked", [
    ([300, 300], 16, 8, False),   # config 3/4 in the long form
    ([300, 260], 16, 8, True),
    ([640, 3], 8, 2, True),       # a segment shorter than the 128-row tile: dead wavefronts
    ([1, 33, 64, 65], 4, 2, True),
    ([700], 4, 4, False),         # KV group of 1
    ([7], 2, 2, False),
])
def test_attention_long_form_forced(oracle, seg_rows, nh, nkv, masked):
    """The long-sequence split form (K/V blocks through LDS, every wavefront
    walking all keys; chosen by workgroup count, here forced for every size
    with ovh_set_attention_long_min_tasks(0)) on short and ragged segments,
    where some of its wavefronts have no query rows and only move K/V: within
    the attention tolerance of the oracle (ops_cpu.cpp:907-943), fully masked
    rows exactly zero, and the threshold restored afterwards."""
    import ovnative_amd as ov
    rng = np.random.default_rng(7 * sum(seg_rows) + nh)
    D = 128
    segs, T = _segments(rng, seg_rows, masked)
    q = rng.standard_normal((T, nh * D)).astype(np.float32)
    k = rng.standard_normal((T, nkv * D)).astype(np.float32)
    v = rng.standard_normal((T, nkv * D)).astype(np.float32)
    want = oracle.attention(q, k, v, segs, nh, nkv, D)
    dsegs = [(None if b is None else dev(b), rows, r0, k0) for b, rows, r0, k0 in segs]
    prev = ov.set_attention_long_min_tasks(0)
    try:
        got = host(ov.attention(dev(q), dev(k), dev(v), dsegs, nh, nkv, D, split=True))
    finally:
        assert ov.set_attention_long_min_tasks(prev) == 0
    assert _attn_err(got, want) <= ATTN_TOL
    dead = np.all(want == 0, axis=1)
    assert np.all(got[dead] == 0)


def test_attention_random_segments(oracle):
    """Seeded random segment layouts (1 to 4 segments of 1 to 700 rows, KV
    groups of 1, 2 and 4, with and without masks), each through the fp32 form,
    the split form as chosen by size, and the split form's long kernel forced:
    within the attention tolerance of the oracle, fully masked rows zero."""
    import ovnative_amd as ov
    rng = np.random.default_rng(4242)
    D = 128
    for _ in range(8):
        nh, nkv = [(16, 8), (8, 2), (4, 4), (2, 1)][rng.integers(4)]
        rows = [int(r) for r in rng.integers(1, 701, rng.integers(1, 5))]
        segs, T = _segments(rng, rows, bool(rng.integers(2)))
        q = rng.standard_normal((T, nh * D)).astype(np.float32)
        k = rng.standard_normal((T, nkv * D)).astype(np.float32)
        v = rng.standard_normal((T, nkv * D)).astype(np.float32)
        want = oracle.attention(q, k, v, segs, nh, nkv, D)
        dead = np.all(want == 0, axis=1)
        dsegs = [(None if b is None else dev(b), r, r0, k0) for b, r, r0, k0 in segs]
        for split, long_min in ((False, None), (True, None), (True, 0)):
            prev = ov.set_attention_long_min_tasks(long_min) if long_min is not None else None
            try:
                got = host(ov.attention(dev(q), dev(k), dev(v), dsegs, nh, nkv, D, split=split))
            finally:
                if prev is not None:
                    ov.set_attention_long_min_tasks(prev)
            assert _attn_err(got, want) <= ATTN_TOL, (rows, nh, nkv, split, long_min)
            assert np.all(got[dead] == 0), (rows, nh, nkv, split, long_min)


def test_attention_sharp_and_argument_errors(oracle):
    """Large logits (softmax close to one-hot) and the ABI's argument checks."""
    import ovnative_amd as ov
    rng = np.random.default_rng(99)
    S, D = 96, 128
    q = (rng.standard_normal((S, D)) * 12).astype(np.float32)
    k = rng.standard_normal((S, D)).astype(np.float32)
    v = rng.standard_normal((S, D)).astype(np.float32)
    want = oracle.attention_head(q, k, v)
    got = host(ov.attention(dev(q), dev(k), dev(v), [(None, S, 0, 0)], 1, 1, D))
    assert _attn_err(got, want) <= ATTN_TOL
    with pytest.raises(ov.OvhError):
        ov.attention(dev(q[:, :64]), dev(k[:, :64]), dev(v[:, :64]), [(None, S, 0, 0)], 1, 1, 64)
    with pytest.raises(ov.InvalidArgument):
        ov.attention(dev(q), dev(k), dev(v), [(None, S, 0, 0)], 3, 2, D)


def test_attention_split_golden_and_range(golden):
    """The split-f16 form on the reference's golden cases, and its f16-range check."""
    import ovnative_amd as ov
    for c in _cases(golden, "attn"):
        q, k, v = golden[c + "_q"], golden[c + "_k"], golden[c + "_v"]
        S, D = q.shape
        if D != 128:
            continue
        bias = dev(golden[c + "_bias"]) if int(golden[c + "_masked"]) else None
        out = host(ov.attention(dev(q), dev(k), dev(v), [(bias, S, 0, 0)], 1, 1, 128,
                                split=True))
        assert _attn_err(out, golden[c + "_out"]) <= ATTN_TOL, c
    rng = np.random.default_rng(5)
    q = rng.standard_normal((16, 128)).astype(np.float32)
    v = rng.standard_normal((16, 128)).astype(np.float32)
    v[3, 7] = 1e5                                   # beyond f16
    with pytest.raises(ov.InvalidArgument):
        ov.attention(dev(q), dev(q), dev(v), [(None, 16, 0, 0)], 1, 1, 128, split=True)
