"""GEMM tile configs at the LM step's shapes (M = 600 by default) with the weights cold, as the
step reads them: each timed pass walks ~600 MB of distinct weights (more than the
256 MB last-level cache), activation codes tile-major as the runner holds them.
Prints the per-launch mean of each config (residual o_proj / down, q/k/v, and
the SiLU-fused gate/up variants of tune_gemm_silu_v), fastest first.

    python3 ovnative_amd/tune/tune_cold.py [M]
"""
import ctypes as C, sys, os, math
R = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, R)
import torch, ovnative_amd as ov
torch.cuda.set_device(0)
lib = C.CDLL(os.path.join(R, 'ovnative_amd/tune/libgemm_tune.so'))
lib.tune_gemm_at.argtypes = [C.c_int]*4 + [C.c_void_p]*5 + [C.c_int, C.c_void_p, C.c_int]
lib.tune_gemm_silu_v.argtypes = [C.c_int]*4 + [C.c_void_p]*6 + [C.c_int64, C.c_int, C.c_void_p]
class DW(C.Structure):
    _fields_ = [('N', C.c_int64), ('K', C.c_int64), ('Npad', C.c_int64), ('Kb', C.c_int64), ('Kp', C.c_int64), ('q', C.c_void_p), ('scale', C.c_void_p)]
st = torch.cuda.current_stream().cuda_stream
M = int(sys.argv[1]) if len(sys.argv) > 1 else 600
def weights(N, K):
    n = math.ceil(600e6 / (N * K)); ws = []
    for _ in range(n):
        q = torch.randint(-127, 128, (N, K), dtype=torch.int8, device='cuda')
        s = torch.rand(N, device='cuda') * 1e-3 + 1e-4
        w = ov.Weight.from_device(q, s); ws.append((w, DW.from_address(w.handle.value)))
    return ws
def timed(run, n):
    run(); torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(); run(); e1.record(); torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n * 1e3
def acts(K):
    A = torch.randn(M, K, device='cuda'); aq, asc = ov.s8_nk_quantize(A)
    at = ov.Weight.from_device(aq.view(torch.int8)[:, :K].contiguous(), torch.ones(M, device='cuda'))
    return at, DW.from_address(at.handle.value).q, asc
for (N, K, acc, cfgs) in [(1024, 2048, 1, [8, 16, 14, 18, 45, 46, 47, 40, 41, 44]),
                          (1024, 3072, 1, [8, 16, 14, 18, 45, 46, 47, 40, 41, 44]),
                          (4096, 1024, 0, [9, 42, 43, 48, 49, 13, 15, 12])]:
    ws = weights(N, K); at, ap, asc = acts(K)
    Cc = torch.zeros(M, N, device='cuda'); res = []
    for cfg in cfgs:
        def run():
            for w, dw in ws:
                rc = lib.tune_gemm_at(cfg, M, N, K // 32, ap, asc.data_ptr(), dw.q, dw.scale, Cc.data_ptr(), acc, st, 1)
                assert rc == 0, (cfg, rc)
        res.append((timed(run, len(ws)), cfg))
    res.sort()
    print(f"cold M={M} N={N} K={K} acc={acc} ({len(ws)} weights): " + "  ".join(f"c{c}:{t:.2f}" for t, c in res), flush=True)
    for w, _ in ws: w.free()
    del ws
# SiLU gate/up, interleaved weights
N, K = 6144, 1024; inter = N // 2
ws = weights(N, K); at, ap, asc = acts(K)
hq = torch.zeros(((M + 127) // 128 * 128) * inter, dtype=torch.int8, device='cuda')
hsc = torch.zeros(M * (inter // 32), device='cuda'); res = []
for v in range(10):
    def run():
        for w, dw in ws:
            rc = lib.tune_gemm_silu_v(v, M, N, K // 32, ap, asc.data_ptr(), dw.q, dw.scale, hq.data_ptr(), hsc.data_ptr(), inter, 1, st)
            assert rc == 0, (v, rc)
    res.append((timed(run, len(ws)), v))
res.sort()
print(f"cold SiLU M={M} N={N} K={K} ({len(ws)} weights): " + "  ".join(f"s{c}:{t:.2f}" for t, c in res), flush=True)
