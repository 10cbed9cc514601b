"""The reference-side C++ shims of the repository's integration guide (every
```cpp block of the top-level guide the test reads) compile against the
reference's own headers (cpp/src/model/lm.h, tts.h, ov_weights.h) and
include/ovnative_amd.h, and the runner thunks have exactly the plugin's
function-pointer types (static_asserts in the shim: LM::CudaForwardFn,
CudaLogitsFn, CudaSampleFn, lm.h:86-106).  CPU only; needs the reference tree
and a C++17 compiler (skipped where /root/reference is not mounted)."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference/cpp"


def _blocks():
    text = open(os.path.join(ROOT, "INTEGRATION.md"), encoding="utf-8").read()
    return re.findall(r"```cpp\n(.*?)```", text, flags=re.S)


def test_integration_shims_compile(tmp_path):
    if not os.path.isdir(REF):
        pytest.skip("reference tree not mounted")
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no g++")
    blocks = _blocks()
    assert len(blocks) >= 5
    src = tmp_path / "shims.cpp"
    src.write_text("\n".join(blocks) + "\nint main() { return 0; }\n")
    cmd = [cxx, "-std=c++17", "-fsyntax-only", "-D__HIP_PLATFORM_AMD__",
           f"-I{ROOT}/include", f"-I{REF}/include", f"-I{REF}/src", "-I/opt/rocm/include",
           str(src)]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-4000:]
