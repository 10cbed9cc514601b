"""Run one GEMM tile config on one shape repeatedly (profiling driver):

    python3 ovnative_amd/tune/one_gemm.py CFG M N K REPS [ACCUMULATE]

CFG indexes the configs of gemm_tune.hip (4 = 128x64, 2 = 64x64, 7 = 32x32;
10 = the 16x16-tile 128x64 x 8-wave kernel the product uses for gate/up at M = 600)."""
import ctypes as C, sys, os
sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
import torch, ovnative_amd as ov
cfg, M, N, K, reps = (int(x) for x in sys.argv[1:6])
acc = int(sys.argv[6]) if len(sys.argv) > 6 else 0  # 1: C += (the residual form)
torch.cuda.set_device(0)
lib = C.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), 'libgemm_tune.so'))
lib.tune_gemm.argtypes = [C.c_int]*4 + [C.c_void_p]*5 + [C.c_int, C.c_void_p]
class DW(C.Structure):
    _fields_ = [('N', C.c_int64), ('K', C.c_int64), ('Npad', C.c_int64), ('Kb', C.c_int64), ('Kp', C.c_int64), ('q', C.c_void_p), ('scale', C.c_void_p)]
q = torch.randint(-127, 128, (N, K), dtype=torch.int8, device='cuda')
s = torch.rand(N, device='cuda') * 1e-3 + 1e-4
w = ov.Weight.from_device(q, s); dw = DW.from_address(w.handle.value)
A = torch.randn(M, K, device='cuda'); aq, asc = ov.s8_nk_quantize(A)
Cc = torch.zeros(M, N, device='cuda')
st = torch.cuda.current_stream().cuda_stream
for _ in range(reps):
    lib.tune_gemm(cfg, M, N, K // 32, aq.data_ptr(), asc.data_ptr(), dw.q, dw.scale, Cc.data_ptr(), acc, st)
torch.cuda.synchronize()
print("done", cfg, M, N, K, reps)
