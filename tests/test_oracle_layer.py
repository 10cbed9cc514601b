"""CPU pins for the oracle's attention-side restatements (qk-norm + RoPE,
attention, embedding): golden vectors from the compiled reference, the live
reference where it is built, and properties the mathematics fixes."""
import numpy as np
import pytest


def bits(a):
    return np.ascontiguousarray(a).view(np.int32)


def _cases(golden, prefix):
    return sorted({k.split("_")[0] for k in golden if k.startswith(prefix)})


def test_qk_norm_rope_golden(golden, oracle):
    for c in _cases(golden, "qknr"):
        rows, nh, nkv, D = (int(x) for x in golden[c + "_dims"])
        qo, ko = oracle.qk_norm_rope(golden[c + "_q"], golden[c + "_k"], golden[c + "_qw"],
                                     golden[c + "_kw"], nh, nkv, D, golden[c + "_pos"])
        assert np.array_equal(bits(qo), bits(golden[c + "_qo"])), c
        assert np.array_equal(bits(ko), bits(golden[c + "_ko"])), c


def test_attention_golden(golden, oracle):
    for c in _cases(golden, "attn"):
        bias = golden[c + "_bias"] if int(golden[c + "_masked"]) else None
        out = oracle.attention_head(golden[c + "_q"], golden[c + "_k"], golden[c + "_v"], bias)
        assert np.array_equal(bits(out), bits(golden[c + "_out"])), c


@pytest.mark.parametrize("S,D,mag", [(5, 128, 1.0), (64, 128, 8.0), (300, 128, 1.0),
                                     (41, 64, 2.0), (9, 16, 1.0)])
def test_attention_against_reference(reference, oracle, S, D, mag):
    rng = np.random.default_rng(S * 7 + D)
    q = (rng.standard_normal((S, D)) * mag).astype(np.float32)
    k = rng.standard_normal((S, D)).astype(np.float32)
    v = rng.standard_normal((S, D)).astype(np.float32)
    bias = np.where(rng.random((S, S)) < 0.3, -1e30, 0.0).astype(np.float32)
    bias[-1] = -1e30
    for b in (None, bias):
        assert np.array_equal(bits(oracle.attention_head(q, k, v, b)),
                              bits(reference.attention_head(q, k, v, b)))


def test_qk_norm_rope_against_reference(reference, oracle):
    rng = np.random.default_rng(5)
    rows, nh, nkv, D = 40, 16, 8, 128
    q = (rng.standard_normal((rows, nh * D)) * 2).astype(np.float32)
    k = rng.standard_normal((rows, nkv * D)).astype(np.float32)
    qw = rng.uniform(0.2, 2.0, D).astype(np.float32)
    kw = rng.uniform(0.2, 2.0, D).astype(np.float32)
    pos = rng.integers(0, 20000, rows)
    a = oracle.qk_norm_rope(q, k, qw, kw, nh, nkv, D, pos)
    b = reference.qk_norm_rope(q, k, qw, kw, nh, nkv, D, pos)
    assert np.array_equal(bits(a[0]), bits(b[0])) and np.array_equal(bits(a[1]), bits(b[1]))


def test_rope_tables_closed_form(oracle):
    """inv_freq = theta^(-2i/D); pos 0 gives cos 1, sin 0; every entry is within
    one ulp of cos/sin of the float angle evaluated in double."""
    pos = np.array([0, 1, 7, 299, 1023, 40000], np.int64)
    D, theta = 128, 1e6
    c, s = oracle.rope_tables(pos, D, theta)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    inv = (theta ** (-2.0 * np.arange(D // 2) / D)).astype(np.float32)
    ang = pos.astype(np.float32)[:, None] * inv[None, :]
    for got, fn in ((c, np.cos), (s, np.sin)):
        want = fn(ang.astype(np.float64)).astype(np.float32)
        assert np.abs(bits(got).astype(np.int64) - bits(want).astype(np.int64)).max() <= 1


def test_qk_norm_rope_properties(oracle):
    """At pos 0 the rotation is the identity, so the output is the per-head norm
    alone; at any position each (i, i+D/2) pair keeps its length."""
    rng = np.random.default_rng(11)
    rows, nh, nkv, D = 3, 2, 1, 128
    q = rng.standard_normal((rows, nh * D)).astype(np.float32)
    k = rng.standard_normal((rows, nkv * D)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, D).astype(np.float32)
    qo, _ = oracle.qk_norm_rope(q, k, w, w, nh, nkv, D, np.zeros(rows, np.int64))
    x = q.reshape(rows, nh, D).astype(np.float64)
    ref = x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(qo.reshape(rows, nh, D), ref, rtol=2e-6, atol=1e-7)
    qo, _ = oracle.qk_norm_rope(q, k, w, w, nh, nkv, D, np.array([5, 77, 3000]))
    y = qo.reshape(rows, nh, D).astype(np.float64)
    h = D // 2
    np.testing.assert_allclose(y[..., :h] ** 2 + y[..., h:] ** 2,
                               ref[..., :h] ** 2 + ref[..., h:] ** 2, rtol=1e-5, atol=1e-9)


def test_attention_properties(oracle):
    """One visible key returns that key's value row; q = 0 gives the mean of V;
    a fully masked row is zero."""
    rng = np.random.default_rng(3)
    S, D = 37, 128
    q = rng.standard_normal((S, D)).astype(np.float32)
    k = rng.standard_normal((S, D)).astype(np.float32)
    v = rng.standard_normal((S, D)).astype(np.float32)
    bias = np.full((S, S), -1e30, np.float32)
    pick = rng.integers(0, S, S)
    bias[np.arange(S), pick] = 0.0
    bias[5] = -1e30
    out = oracle.attention_head(q, k, v, bias)
    rows = np.arange(S) != 5
    np.testing.assert_allclose(out[rows], v[pick[rows]], rtol=1e-7, atol=1e-30)
    assert np.all(out[5] == 0.0)
    out = oracle.attention_head(np.zeros_like(q), k, v)
    np.testing.assert_allclose(out, np.broadcast_to(v.astype(np.float64).mean(0), (S, D)),
                               rtol=0, atol=2e-6)


def test_attention_gqa_loop(oracle):
    """The multi-segment GQA driver equals per-head calls (KV head = h / group)."""
    rng = np.random.default_rng(4)
    nh, nkv, D = 4, 2, 64
    segs_rows = [9, 6]
    T = sum(segs_rows)
    q = rng.standard_normal((T, nh * D)).astype(np.float32)
    k = rng.standard_normal((T, nkv * D)).astype(np.float32)
    v = rng.standard_normal((T, nkv * D)).astype(np.float32)
    b1 = np.where(rng.random((6, 6)) < 0.3, -1e30, 0).astype(np.float32)
    segs = [(None, 9, 0, 0), (b1, 6, 9, 9)]
    out = oracle.attention(q, k, v, segs, nh, nkv, D)
    for bias, rows, r0, _ in segs:
        for h in range(nh):
            kv = h // (nh // nkv)
            want = oracle.attention_head(q[r0:r0 + rows, h * D:(h + 1) * D],
                                         k[r0:r0 + rows, kv * D:(kv + 1) * D],
                                         v[r0:r0 + rows, kv * D:(kv + 1) * D], bias)
            assert np.array_equal(bits(out[r0:r0 + rows, h * D:(h + 1) * D]), bits(want))


def test_embed_brute_force(oracle):
    rng = np.random.default_rng(8)
    B, Cb, S, H, V = 2, 8, 6, 32, 11
    tok = rng.standard_normal((50, H)).astype(np.float32)
    aud = rng.standard_normal((Cb * V, H)).astype(np.float32)
    offs = np.arange(Cb, dtype=np.int64) * V
    ids = rng.integers(0, V, (B, Cb, S)).astype(np.int64)
    mask = (rng.random((B, S)) < 0.5).astype(np.uint8)
    out = oracle.embed(ids, mask, tok, aud, offs)
    for b in range(B):
        for s in range(S):
            if mask[b, s]:
                acc = np.zeros(H, np.float32)
                for c in range(Cb):
                    acc = (acc + aud[ids[b, c, s] + offs[c]]).astype(np.float32)
                want = acc
            else:
                want = tok[ids[b, 0, s]]
            assert np.array_equal(bits(out[b * S + s]), bits(want))
    # int8 tables with per-row scales: gathered as float(q) * scale
    tq = rng.integers(-127, 128, tok.shape).astype(np.int8)
    ts = rng.uniform(1e-3, 1e-2, tok.shape[0]).astype(np.float32)
    aq = rng.integers(-127, 128, aud.shape).astype(np.int8)
    as_ = rng.uniform(1e-3, 1e-2, aud.shape[0]).astype(np.float32)
    out = oracle.embed(ids, mask, tq, aq, offs, ts, as_)
    b, s = np.argwhere(mask == 0)[0]
    assert np.array_equal(bits(out[b * S + s]),
                          bits(tq[ids[b, 0, s]].astype(np.float32) * ts[ids[b, 0, s]]))
    with pytest.raises(ValueError):
        bad = ids.copy()
        bad[0, 0, :] = 10_000
        oracle.embed(bad, np.zeros_like(mask), tok, aud, offs)


def _np_guided(cond, cond_seq, uncond, C, V, T, g, pen, mask_id):
    """float64 statement of tts.cpp:296-326 (log_softmax, mix, mask, argmax)."""
    def lsm(x):
        m = x.max()
        return x - (np.log(np.exp(x - m).sum()) + m)
    pred = np.zeros((C, T), np.int64)
    score = np.zeros((C, T))
    gap = np.zeros((C, T))
    for c in range(C):
        for t in range(T):
            lc = lsm(cond[cond_seq - T + t, c * V:(c + 1) * V].astype(np.float64))
            lu = lsm(uncond[t, c * V:(c + 1) * V].astype(np.float64))
            mix = lsm(lc + g * (lc - lu)) if g != 0 else lc
            mix[mask_id] = -np.inf
            srt = np.sort(mix)
            pred[c, t], score[c, t], gap[c, t] = mix.argmax(), srt[-1] - c * pen, srt[-1] - srt[-2]
    return pred, score, gap


@pytest.mark.parametrize("g", [0.0, 2.0])
def test_guided_sample_properties(oracle, g):
    rng = np.random.default_rng(int(g * 10) + 1)
    C, V, S, T = 8, 1025, 12, 7
    cond = (rng.standard_normal((S, C * V)) * 3).astype(np.float32)
    uncond = (rng.standard_normal((T, C * V)) * 3).astype(np.float32)
    cond[S - T, 1024] = 100.0          # the mask token never wins
    pred, score = oracle.guided_sample(cond, S, uncond, C, V, T, g, 5.0)
    want, wscore, gap = _np_guided(cond, S, uncond, C, V, T, g, 5.0, 1024)
    clear = gap > 1e-4
    assert np.array_equal(pred[clear], want[clear]) and np.all(pred != 1024)
    np.testing.assert_allclose(score, wscore, rtol=0, atol=2e-5)


def test_guided_sample_invariants(oracle):
    """What tts.cpp:296-326 fixes independently of rounding: (1) with the
    unconditional logits equal to the conditional ones the guidance term
    vanishes, so g = 2 picks what g = 0 picks, with the same score up to the
    second log_softmax's rounding; (2) log_softmax removes a constant added to
    one (codebook, frame) row of either plane; (3) the layer penalty only
    subtracts c * penalty from codebook c's scores; (4) the mask token (the last
    id) is never chosen, even as the largest logit."""
    rng = np.random.default_rng(44)
    C, V, S, T = 8, 1025, 10, 6
    cond = (rng.standard_normal((S, C * V)) * 2).astype(np.float32)
    uncond = (rng.standard_normal((T, C * V)) * 2).astype(np.float32)
    cond[S - T + 2, 3 * V + V - 1] = 50.0
    uncond[2, 3 * V + V - 1] = 50.0
    p0, s0 = oracle.guided_sample(cond, S, cond[S - T:], C, V, T, 0.0, 5.0)
    p2, s2 = oracle.guided_sample(cond, S, cond[S - T:], C, V, T, 2.0, 5.0)
    assert np.array_equal(p0, p2)
    np.testing.assert_allclose(s2, s0, rtol=0, atol=4e-6)
    base_p, base_s = oracle.guided_sample(cond, S, uncond, C, V, T, 2.0, 5.0)
    _, _, gap = _np_guided(cond, S, uncond, C, V, T, 2.0, 5.0, V - 1)
    clear = gap > 1e-4
    c2, u2 = cond.copy(), uncond.copy()
    c2[S - T + 1, 2 * V:3 * V] += 3.0       # (codebook 2, frame 1) of the cond plane
    u2[4, 5 * V:6 * V] -= 7.0               # (codebook 5, frame 4) of the uncond plane
    sh_p, sh_s = oracle.guided_sample(c2, S, u2, C, V, T, 2.0, 5.0)
    assert np.array_equal(sh_p[clear], base_p[clear])
    np.testing.assert_allclose(sh_s, base_s, rtol=0, atol=2e-5)
    np_p, np_s = oracle.guided_sample(cond, S, uncond, C, V, T, 2.0, 0.0)
    assert np.array_equal(np_p, base_p)
    np.testing.assert_allclose(np_s - 5.0 * np.arange(C)[:, None], base_s, rtol=0, atol=8e-6)
    assert np.all(base_p != V - 1) and np.all(p0 != V - 1)


def test_guided_sample_host_alias_quirk(oracle):
    """tts.cpp's host path renormalises lp_mix with log_softmax(x, n, x) in place,
    so its guided values are exp(mix - m) - lse (the function's last loop reads
    the overwritten x).  Same argmax as the device form wherever exp() does not
    underflow; scores are 1 - lse instead of max(mix) - lse."""
    rng = np.random.default_rng(21)
    C, V, S, T = 8, 1025, 6, 4
    cond = rng.standard_normal((S, C * V)).astype(np.float32)
    uncond = rng.standard_normal((T, C * V)).astype(np.float32)
    p_dev, s_dev = oracle.guided_sample(cond, S, uncond, C, V, T, 2.0, 5.0)
    p_cpu, s_cpu = oracle.guided_sample(cond, S, uncond, C, V, T, 2.0, 5.0, cpu_alias=True)
    assert np.array_equal(p_dev, p_cpu)
    # host score = exp(mix_best - m) - lse - c*pen with mix_best = m: 1 - lse - c*pen,
    # device score = m - lse - c*pen, so host - device = 1 - m  (m = max mix)
    want, _, _ = _np_guided(cond, S, uncond, C, V, T, 2.0, 5.0, 1024)
    assert np.array_equal(p_dev, want)
    assert not np.allclose(s_dev, s_cpu)


@pytest.mark.parametrize("layout,batch,seq,text,head_fp32", [
    ("nk", 2, 40, 8, False), ("nk", 1, 17, 5, False), ("kn", 2, 24, 6, False),
    ("nk", 2, 30, 6, True)], ids=["nk-b2", "nk-b1", "kn-b2", "nk-b2-fp32head"])
def test_lm_forward_against_reference(reference, oracle, tmp_path, layout, batch, seq, text,
                                      head_fp32):
    """The oracle's forward (composition of the restated pieces) is bit-identical to
    the reference's LM::forward (lm.cpp, compiled from source) on an OVW1 file
    written by ovnative_amd/ovw1.py.  For kn checkpoints the reference CPU takes
    its non-VNNI fp32-activation kernel (mat.cpp:82-90, no activation
    quantisation), a different arithmetic; the HIP path computes int8-nk numerics
    for both layouts, so kn is only checked to stay close (cosine >= 0.9999).
    fp32head: the audio head fp32 [K, N], as the reference's default int8
    checkpoint keeps it (final rmsnorm_f32, then Mat's fp32 branch)."""
    from lm_fixture import SMALL, make_inputs, make_lm
    from ovnative_amd import ovw1
    if not reference.vnni_available():
        pytest.skip("the reference's int8-nk VNNI path is not available on this host")
    ts, table = make_lm(5, SMALL, layout=layout, head_fp32=head_fp32)
    path = str(tmp_path / "lm.ovw")
    ovw1.write(path, ts)
    ids, am, attn, pos = make_inputs(6, SMALL, batch, seq, text)
    h = reference.lm_open(path, SMALL)
    try:
        ref = reference.lm_forward(h, SMALL, ids, am, attn, pos)
    finally:
        reference.lm_close(h)
    segs = [(attn[b], seq, b * seq) for b in range(batch)]
    got = oracle.lm_forward(SMALL, table, ids, am, segs, pos.reshape(-1))
    Cb, V = SMALL["n_codebooks"], SMALL["audio_vocab"]
    ref_flat = ref.transpose(0, 2, 1, 3).reshape(batch * seq, Cb * V)
    if layout == "nk":
        assert np.array_equal(bits(got), bits(ref_flat))
    else:
        cos = (got.astype(np.float64) * ref_flat).sum() / (
            np.linalg.norm(got.astype(np.float64)) * np.linalg.norm(ref_flat.astype(np.float64)))
        assert cos >= 0.9999


def test_guided_sample_known_answer(oracle):
    """The hand-worked case of lm_fixture.SAMPLER_CASE (derived there from
    tts.cpp:296-326): the oracle's device-form sampler picks the hand-derived
    tokens with the hand-derived scores (to fp32 rounding), and the case
    separates the plausible mistakes: g = -2 computes the flipped guidance sign
    (lc - 2 (lc - lu)) and picks tokens 1 and 2, g = 0 picks token 1 in
    codebook 0, and the scores are far from the values without the second
    log-softmax (1.9445, -7.0313)."""
    from lm_fixture import SAMPLER_CASE as K
    cond = np.array(K["cond"], np.float32)
    uncond = np.array(K["uncond"], np.float32)

    def run(g):
        return oracle.guided_sample(cond, 1, uncond, K["C"], K["V"], K["T"], g, K["penalty"])
    pred, scores = run(K["guidance"])
    assert np.array_equal(pred, np.array(K["pred"]))
    np.testing.assert_allclose(scores, np.array(K["scores"]), rtol=0, atol=2e-6)
    assert np.array_equal(run(-K["guidance"])[0], np.array([[1], [2]]))
    assert run(0.0)[0][0, 0] == 1
    assert np.abs(scores - np.array([[1.9445], [-7.0313]])).min() > 0.05
