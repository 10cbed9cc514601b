"""OVW1 writer (ovnative_amd/ovw1.py) and reader (ovh_ovw1_* in the HIP library,
host code only) against the reference's own loader (weight_file.cpp, compiled
into oracle/_ref) and against the format's closed-form properties.  CPU only."""
import os
import struct
import zlib

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
