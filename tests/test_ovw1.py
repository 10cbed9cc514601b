"""OVW1 writer (ovnative_amd/ovw1.py) and reader (ovh_ovw1_* in the HIP library,
host code only) against the reference's own loader (weight_file.cpp, compiled
into oracle/_ref) and against the format's closed-form properties.  CPU only."""
import math
import os
import struct
import zlib
from fractions import Fraction

import numpy as np
import pytest

from lm_fixture import SMALL, make_lm
from ovnative_amd import ovw1


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    ts, table = make_lm(1, dict(SMALL, n_layers=1), layout="kn")
    ts.append(ovw1.Tensor("extra.f16", np.arange(6, dtype=np.float16).reshape(2, 3)))
    path = str(tmp_path_factory.mktemp("ovw") / "lm.ovw")
    size = ovw1.write(path, ts)
    return path, size, ts


def test_layout_closed_form(ckpt):
    path, size, ts = ckpt
    raw = open(path, "rb").read()
    assert len(raw) == size and size % 64 == 0
    magic, ver, mode, n, hb, idx, names_off, data_off, fsize, flags, params = \
        struct.unpack_from("<8sIIIIQQQQQQ", raw, 0)
    assert (magic, ver, mode, n, hb, idx, fsize) == (b"OMNIVOIC", 1, 1, len(ts), 128, 128, size)
    assert names_off % 64 == 0 and data_off % 64 == 0 and flags == 3
    names = sorted(t.name for t in ts)
    for i, name in enumerate(names):
        d = struct.unpack_from("<IIBBBB4IIQQQQ", raw, 128 + 64 * i)
        no, nl, dt, nd, lay, qu = d[:6]
        aux_n, crc, doff, nb, aoff = d[10:]
        assert raw[names_off + no:names_off + no + nl].decode() == name
        assert doff % 64 == 0 and (aoff % 64 == 0)
        assert zlib.crc32(raw[doff:doff + nb]) == crc


def test_reader_roundtrip(ckpt):
    import ovnative_amd as ov
    path, size, ts = ckpt
    wf = ov.WeightFile(path)
    try:
        assert sorted(wf.names()) == sorted(t.name for t in ts) and wf.crc_ok()
        for t in ts:
            v = wf.find(t.name)
            assert v is not None and v.ndim == t.array.ndim
            assert tuple(v.dims[:v.ndim]) == t.array.shape
            assert v.transposed == (t.layout == 1)
            got = np.ctypeslib.as_array((np.ctypeslib.ctypes.c_uint8 * v.nbytes).from_address(v.data))
            assert got.tobytes() == np.ascontiguousarray(t.array).tobytes()
            if t.scales is not None:
                assert v.quantized and v.n_scales == t.scales.size
                sc = np.ctypeslib.as_array((np.ctypeslib.ctypes.c_float * v.n_scales).from_address(v.scales))
                assert np.array_equal(sc, t.scales)
        assert wf.find("no.such.tensor") is None
    finally:
        wf.close()


def test_reference_loader_reads_our_files(reference, ckpt):
    path, size, ts = ckpt
    n, got = reference.ovw1_read(path, [t.name for t in ts])
    assert n == len(ts)
    for t in ts:
        g = got[t.name]
        assert g["dims"] == t.array.shape and g["transposed"] == (t.layout == 1)
        assert g["data"] == np.ascontiguousarray(t.array).tobytes()
        assert g["stored_crc"] == g["computed_crc"]
        assert g["quantized"] == (t.scales is not None)
        if t.scales is not None:
            assert np.array_equal(g["scales"], t.scales)


@pytest.mark.parametrize("damage", ["magic", "version", "truncate", "payload_size"])
def test_reader_rejects_damaged_files(reference, ckpt, tmp_path, damage):
    """Both readers refuse the same damaged files (the reference throws)."""
    import ovnative_amd as ov
    path, size, ts = ckpt
    raw = bytearray(open(path, "rb").read())
    if damage == "magic":
        raw[0:8] = b"NOTOVW1!"
    elif damage == "version":
        raw[8:12] = struct.pack("<I", 2)
    elif damage == "truncate":
        raw = raw[:-64]
    else:  # first descriptor's nbytes no longer matches its shape
        nb_off = 128 + 48
        raw[nb_off:nb_off + 8] = struct.pack("<Q", struct.unpack_from("<Q", raw, nb_off)[0] + 1)
    bad = tmp_path / "bad.ovw"
    bad.write_bytes(bytes(raw))
    with pytest.raises(ov.OvhError) as e:
        ov.WeightFile(str(bad))
    assert e.value.code == ov.OV_ERR_IO
    with pytest.raises(RuntimeError):
        reference.ovw1_read(str(bad), [])


def test_quantize_int8_matches_oracle(oracle):
    """The writer's quantiser is convert_weights.py's; the oracle restates it in C."""
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((64, 333)) * 0.02).astype(np.float32)
    w[3] = 0.0
    q, s = ovw1.quantize_int8(w)
    q2, s2 = oracle.quantize_weight_rows(w)
    assert np.array_equal(q, q2) and np.array_equal(s.view(np.int32), s2.view(np.int32))
    t = ovw1.linear_int8("x", w, "kn")
    assert t.layout == 1 and np.array_equal(t.array, q.T)


def _round_f32(x: Fraction) -> Fraction:
    """The float32 nearest to the rational x (ties to even), for normal |x|."""
    if x == 0:
        return Fraction(0)
    sign, x = (-1 if x < 0 else 1), abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    while Fraction(2) ** e > x:
        e -= 1
    while Fraction(2) ** (e + 1) <= x:
        e += 1
    ulp = Fraction(2) ** (e - 23)
    m = x / ulp
    r = math.floor(m)
    if m - r > Fraction(1, 2) or (m - r == Fraction(1, 2) and r % 2 == 1):
        r += 1
    return sign * r * ulp


def _rne_int(x: Fraction) -> int:
    r = math.floor(x)
    if x - r > Fraction(1, 2) or (x - r == Fraction(1, 2) and r % 2 == 1):
        r += 1
    return r


def _quantize_exact(w: np.ndarray):
    """tools/convert_weights.py:130-135 in exact arithmetic: scale = the float32
    nearest absmax / 127 (floored at float32(1e-12)); q = clip(RNE(the float32
    nearest w / scale), -127, 127)."""
    q = np.zeros(w.shape, np.int64)
    s = np.zeros(w.shape[0], np.float32)
    floor = Fraction(float(np.float32(1e-12)))
    for r in range(w.shape[0]):
        am = max(abs(Fraction(float(v))) for v in w[r])
        sc = max(_round_f32(am / 127) if am else Fraction(0), floor)
        s[r] = np.float32(float(sc))
        for c in range(w.shape[1]):
            q[r, c] = min(127, max(-127, _rne_int(_round_f32(Fraction(float(w[r, c])) / sc))
                                   if w[r, c] != 0 else 0))
    return q.astype(np.int8), s


def test_quantize_int8_exact_arithmetic(oracle):
    """quantize_int8 (the product's Python writer) and the oracle's C restatement
    equal the exact-arithmetic statement of convert_weights.py:130-135 on rows
    built to separate plausible mistakes: exact .5 ties (round half to even, not
    away: 0.5 -> 0, 1.5 -> 2, 2.5 -> 2), quotients where multiplying by a
    rounded reciprocal lands on the other integer than dividing does, the
    absmax element (exactly +-127), an all-zero row (the 1e-12 floor) and
    random rows."""
    rows = []
    # absmax 127/128 -> scale 2^-7 exactly; w = (k + 1/2) 2^-7 -> ties
    rows.append(np.array([127 / 128] + [(k + 0.5) / 128 for k in range(8)] +
                         [-(k + 0.5) / 128 for k in range(8)], np.float32))
    # division vs reciprocal: rint(w / s) != rint(w * (1 / s)) in float32
    for am, w in ((0.11075115948915482, 0.10857102274894714),
                  (0.07779009640216827, -0.06584594398736954),
                  (0.057323209941387177, 0.041751157492399216),
                  (0.016390521079301834, -0.008453378453850746),
                  (0.0901048481464386, 0.03795755282044411),
                  (0.1104719266295433, 0.06393453478813171)):
        r = np.zeros(17, np.float32)
        r[0], r[1] = am, w
        rows.append(r)
    rows.append(np.zeros(17, np.float32))
    rng = np.random.default_rng(8)
    rows += list((rng.standard_normal((6, 17)) * 0.02).astype(np.float32))
    W = np.stack(rows)
    want_q, want_s = _quantize_exact(W)
    assert list(want_q[0, 1:9]) == [0, 2, 2, 4, 4, 6, 6, 8]
    for k in range(6):   # the traps do separate the two readings
        am, w = np.float32(W[1 + k, 0]), np.float32(W[1 + k, 1])
        s = np.float32(am / np.float32(127))
        assert np.rint(w / s) != np.rint(w * (np.float32(1) / s))
    q, s = ovw1.quantize_int8(W)
    assert np.array_equal(q, want_q) and np.array_equal(s.view(np.int32), want_s.view(np.int32))
    q2, s2 = oracle.quantize_weight_rows(W)
    assert np.array_equal(q2, want_q) and np.array_equal(s2.view(np.int32), want_s.view(np.int32))
