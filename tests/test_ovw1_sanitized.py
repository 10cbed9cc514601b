"""The OVW1 reader (ovnative_amd/csrc/ovw1.cpp, host C++ that parses untrusted
files) built with AddressSanitizer and UndefinedBehaviorSanitizer and run over a
valid checkpoint and hundreds of truncated and corrupted copies of it: every
damaged file must come back as an error status (or, for damage the format does
not detect, as readable views), with no out-of-bounds access, overflow or other
undefined behaviour reported.  CPU only (host code; g++ with libasan/libubsan)."""
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

from lm_fixture import SMALL, make_lm
from ovnative_amd import ovw1

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

DRIVER = r"""
#include <cstdio>
#include <cstring>
#include <string>
#include "ovnative_amd.h"
namespace ovh {
static std::string g_msg;
int set_error(int code, const std::string& msg) { g_msg = msg; return code; }
}
int main(int argc, char** argv) {
  int opened = 0;
  for (int i = 1; i < argc; ++i) {
    OvhWeightFile* wf = nullptr;
    const int rc = ovh_ovw1_open(argv[i], &wf);
    if (rc != OV_OK) { if (wf) return 3; continue; }
    ++opened;
    const int n = ovh_ovw1_count(wf);
    const OvhTensorView* v = ovh_ovw1_tensors(wf);
    unsigned sum = 0;
    for (int t = 0; t < n; ++t) {
      const unsigned char* d = static_cast<const unsigned char*>(v[t].data);
      if (v[t].nbytes > 0) sum += d[0] + d[v[t].nbytes - 1];
      if (v[t].scales && v[t].n_scales > 0) sum += (unsigned)v[t].scales[v[t].n_scales - 1];
      sum += ovh_ovw1_compute_crc(wf, t);
      // a duplicated name finds its first tensor, as WeightFile::Find does (a
      // damaged name with a NUL inside is not found by its C string at all)
      const OvhTensorView* f = ovh_ovw1_find(wf, v[t].name);
      if (f && (std::strcmp(f->name, v[t].name) != 0 || f > &v[t])) { ovh_ovw1_close(wf); return 4; }
    }
    sum += (unsigned)ovh_ovw1_n_params(wf);
    ovh_ovw1_close(wf);
    std::printf("%s %d %u\n", argv[i], n, sum);
  }
  std::printf("opened %d of %d\n", opened, argc - 1);
  return 0;
}
"""


def _mutants(blob: bytes, rng):
    hdr = struct.Struct("<8sIIIIQQQQQQ")
    magic, ver, mode, nt, hb, idx, names, data, fsize, flags, npar = hdr.unpack_from(blob, 0)
    out = []
    for cut in sorted({0, 1, 7, 8, 71, 72, 127, 128, idx + 1, idx + 63, idx + 64 * nt - 1,
                       names, names + 5, data - 1, data, data + 17, len(blob) // 2,
                       len(blob) - 65, len(blob) - 1}):
        if 0 <= cut < len(blob):
            out.append(blob[:cut])
    def put(off, fmt, val):
        b = bytearray(blob)
        struct.pack_into(fmt, b, off, val)
        return bytes(b)
    big = (1 << 64) - 64
    for off, fmt, val in ((20, "<I", 1 << 30), (20, "<I", nt + 1), (24, "<Q", big),
                          (32, "<Q", big), (40, "<Q", big), (48, "<Q", len(blob) + 64),
                          (16, "<I", 0), (8, "<I", 2), (0, "<8s", b"OMNIVOIX")):
        out.append(put(off, fmt, val))
    # descriptor fields of tensor 0 and of the last tensor: name_off/len, dtype,
    # ndim, dims (products past 2^63), aux_n, data_off, nbytes, aux_off
    for t in (0, nt - 1):
        d = idx + 64 * t
        for off, fmt, val in ((0, "<I", 1 << 31), (4, "<I", 1 << 20), (8, "<B", 9),
                              (9, "<B", 5), (9, "<B", 0), (12, "<I", 0xFFFFFFFF),
                              (16, "<I", 0xFFFFFFFF), (28, "<I", 0xFFFFFFFF),
                              (40, "<Q", big), (48, "<Q", big), (48, "<Q", 1),
                              (56, "<Q", big), (56, "<Q", len(blob) - 2)):
            out.append(put(d + off, fmt, val))
    # random byte damage in the header, the index and the names
    for _ in range(300):
        b = bytearray(blob)
        for _ in range(int(rng.integers(1, 6))):
            b[int(rng.integers(0, data))] = int(rng.integers(0, 256))
        out.append(bytes(b))
    return out


def test_ovw1_reader_under_sanitizers(tmp_path):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no g++")
    drv = tmp_path / "driver.cpp"
    drv.write_text(DRIVER)
    exe = tmp_path / "ovw1_san"
    cmd = [cxx, "-std=c++17", "-g", "-O1", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           f"-I{ROOT}/include", str(drv), f"{ROOT}/ovnative_amd/csrc/ovw1.cpp", "-o", str(exe)]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0 and ("asan" in r.stdout.lower() or "ubsan" in r.stdout.lower()):
        pytest.skip("sanitizer runtimes not installed: " + r.stdout[-300:])
    assert r.returncode == 0, r.stdout[-3000:]
    ts, _ = make_lm(3, dict(SMALL, n_layers=1))
    good = tmp_path / "good.ovw"
    ovw1.write(str(good), ts)
    blob = good.read_bytes()
    rng = np.random.default_rng(99)
    files = [str(good)]
    for i, m in enumerate(_mutants(blob, rng)):
        p = tmp_path / f"m{i}.ovw"
        p.write_bytes(m)
        files.append(str(p))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([str(exe)] + files, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                       text=True, env=env)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
    lines = r.stdout.splitlines()
    assert lines[0].startswith(str(good))       # the valid file opens
    assert lines[-1].startswith("opened ")
    print(lines[-1])
