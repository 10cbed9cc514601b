"""OVW1 checkpoint writer and int8 weight quantiser (numpy only).

Writes the reference's on-disk format (docs/weight-format.en.md, the layout
that tools/convert_weights.py:198-244 produces and cpp/src/core/weight_file.cpp
reads): a 128-byte header, one 64-byte descriptor per tensor (sorted by name),
a NUL-separated names blob, then 64-byte aligned payloads, each quantised
tensor's fp32 scales right after its payload.  Every payload carries its CRC-32.
The C++ reader of this package is ``ovh_ovw1_open`` (ovnative_amd/csrc/ovw1.cpp).
"""
from __future__ import annotations

import struct
import zlib
from dataclasses import dataclass
from typing import Iterable, Optional

import numpy as np

MAGIC = b"OMNIVOIC"
VERSION = 1
HEADER_BYTES = 128
DESC_BYTES = 64
ALIGN = 64
_HEADER = struct.Struct("<8sIIIIQQQQQQ")     # 72 bytes used of the 128-byte header
_DESC = struct.Struct("<IIBBBB4IIQQQQ")      # 64 bytes
DT_F32, DT_I8, DT_F16, DT_I64 = 0, 1, 2, 3
_DTYPES = {np.dtype(np.float32): DT_F32, np.dtype(np.int8): DT_I8,
           np.dtype(np.float16): DT_F16, np.dtype(np.int64): DT_I64}


def _align(x: int) -> int:
    return (x + ALIGN - 1) // ALIGN * ALIGN


@dataclass
class Tensor:
    """One stored tensor.  ``layout`` 1 marks a 2-D linear weight stored [in, out];
    ``scales`` (fp32, one per output channel) marks per-channel int8."""
    name: str
    array: np.ndarray
    layout: int = 0
    scales: Optional[np.ndarray] = None


def quantize_int8(w: np.ndarray):
    """Per-output-channel symmetric int8 of a [out, in] matrix
    (tools/convert_weights.py:130-135): scale = max(absmax/127, 1e-12) in fp32,
    q = clip(rint(w/scale), -127, 127)."""
    w = np.asarray(w, dtype=np.float32)
    absmax = np.abs(w).max(axis=1, keepdims=True)
    scale = np.maximum(absmax / np.float32(127.0), np.float32(1e-12)).astype(np.float32)
    q = np.clip(np.rint(w / scale), -127, 127).astype(np.int8)
    return q, scale.reshape(-1)


def linear_int8(name: str, w: np.ndarray, layout: str = "nk") -> Tensor:
    """An fp32 [out, in] linear weight as the converter stores it in int8:
    ``nk`` = q [out, in] (layout 0), ``kn`` = q.T [in, out] (layout 1)."""
    q, s = quantize_int8(w)
    if layout == "kn":
        return Tensor(name, np.ascontiguousarray(q.T), 1, s)
    if layout != "nk":
        raise ValueError(f"unknown int8 layout {layout!r}")
    return Tensor(name, q, 0, s)


def write(path: str, tensors: Iterable[Tensor], n_params: int = 0) -> int:
    """Write an OVW1 file; returns its size in bytes."""
    ts = sorted(tensors, key=lambda t: t.name)
    for t in ts:
        t.array = np.ascontiguousarray(t.array)
        if t.array.dtype not in _DTYPES:
            raise TypeError(f"{t.name}: unsupported dtype {t.array.dtype}")
        if t.array.ndim > 4:
            raise ValueError(f"{t.name}: rank > 4")
        if t.scales is not None:
            t.scales = np.ascontiguousarray(t.scales, dtype=np.float32)
    names_off = _align(HEADER_BYTES + DESC_BYTES * len(ts))
    blob = bytearray()
    name_off = []
    for t in ts:
        name_off.append(len(blob))
        blob += t.name.encode("utf-8") + b"\0"
    cursor = _align(names_off + len(blob))
    data_off = cursor
    offs = []
    for t in ts:
        d = _align(cursor)
        cursor = d + t.array.nbytes
        a = 0
        if t.scales is not None:
            a = _align(cursor)
            cursor = a + t.scales.nbytes
        offs.append((d, a))
    size = _align(cursor)
    int8 = any(t.array.dtype == np.int8 for t in ts)
    with open(path, "wb") as f:
        f.truncate(size)
        f.seek(HEADER_BYTES)
        for t, no, (d, a) in zip(ts, name_off, offs):
            dims = list(t.array.shape) + [0] * (4 - t.array.ndim)
            crc = zlib.crc32(memoryview(t.array).cast("B")) & 0xFFFFFFFF
            f.write(_DESC.pack(no, len(t.name.encode("utf-8")), _DTYPES[t.array.dtype],
                               t.array.ndim, t.layout, 1 if t.scales is not None else 0, *dims,
                               0 if t.scales is None else t.scales.size, crc, d, t.array.nbytes,
                               a))
        f.seek(names_off)
        f.write(bytes(blob))
        for t, (d, a) in zip(ts, offs):
            f.seek(d)
            f.write(memoryview(t.array).cast("B"))
            if t.scales is not None:
                f.seek(a)
                f.write(memoryview(t.scales).cast("B"))
        f.seek(0)
        f.write(_HEADER.pack(MAGIC, VERSION, 1 if int8 else 0, len(ts), HEADER_BYTES,
                             HEADER_BYTES, names_off, data_off, size, (1 if int8 else 0) | 2,
                             n_params or sum(t.array.size for t in ts)))
    return size
