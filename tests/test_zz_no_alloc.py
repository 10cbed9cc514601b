"""ovh_linear_noalloc (the allocation-free variant of ovh_linear) through the C
ABI against ovh_linear on the same inputs: bit-identical results on two calls
in a row (the second smaller, so it runs over what the first left in the shared
device array), the residual form, and the size limit."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import ovnative_amd
    ovnative_amd.load()
    torch.cuda.set_device(0)
    yield
    torch.cuda.synchronize()


def _call(fn, A, w, C, accumulate):
    import ovnative_amd as ov
    ov._check(fn(A.shape[0], ov._dptr(A), w.handle, ov._dptr(C), C.shape[1], int(accumulate),
                 ov._stream()))
    torch.cuda.synchronize()
    return C.cpu().numpy()


def _weight(rng, N, K):
    import ovnative_amd as ov
    q = rng.integers(-127, 128, (N, K)).astype(np.int8)
    s = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    return ov.Weight.from_host(q, s)


def test_noalloc_matches_linear_twice():
    import ovnative_amd as ov
    lib = ov.load()
    rng = np.random.default_rng(2024)
    cases = [(600, 1024, 3072, True), (37, 200, 1000, False)]   # second call smaller
    for M, N, K, acc in cases:
        w = _weight(rng, N, K)
        A = torch.from_numpy((rng.standard_normal((M, K)) * 3).astype(np.float32)).cuda()
        Cin = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).cuda()
        want = _call(lib.ovh_linear, A, w, Cin.clone(), acc)
        got = _call(lib.ovh_linear_noalloc, A, w, Cin.clone(), acc)
        assert np.array_equal(got.view(np.int32), want.view(np.int32)), (M, N, K)


def test_noalloc_size_limit():
    import ovnative_amd as ov
    lib = ov.load()
    rng = np.random.default_rng(7)
    w = _weight(rng, 64, 3072)
    M = 4855                                    # 4855 * (3072 + 384) > 16 MiB
    A = torch.zeros((M, 3072), device="cuda")
    C = torch.zeros((M, 64), device="cuda")
    rc = lib.ovh_linear_noalloc(M, ov._dptr(A), w.handle, ov._dptr(C), 64, 0, ov._stream())
    assert rc == ov.OV_ERR_INVALID_ARG
    assert b"16 MiB" in lib.ovh_last_error()
    M = 4854                                    # fits
    A = torch.from_numpy(rng.standard_normal((M, 3072)).astype(np.float32)).cuda()
    C = torch.zeros((M, 64), device="cuda")
    want = _call(lib.ovh_linear, A, w, C.clone(), False)
    got = _call(lib.ovh_linear_noalloc, A, w, C.clone(), False)
    assert np.array_equal(got.view(np.int32), want.view(np.int32))
