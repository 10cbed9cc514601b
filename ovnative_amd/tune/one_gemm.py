"""Run one GEMM tile config on one shape repeatedly (profiling driver):

    python3 ovnative_amd/tune/one_gemm.py CFG M N K REPS [ACCUMULATE]

CFG indexes the configs of gemm_tune.hip with row-major activation codes as
ovh_s8_nk_quantize writes them (8 = the 16x16-tile 32x32 x 4-wave kernel the
product uses for o_proj/down at M = 600 and the C ABI's residual GEMM; 32 =
128x64 x 8 waves, block by block, for M >= 2048), or sV for the SiLU-fused
gate/up variant V of tune_gemm_silu_v (s1 = the product's at M = 600) on
tile-major codes, as the runner launches it (N = 2 x inter, interleaved
gate/up weight rows; the weight values are random)."""
import ctypes as C, sys, os
sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
import torch, ovnative_amd as ov
cfg_s = sys.argv[1]
M, N, K, reps = (int(x) for x in sys.argv[2:6])
acc = int(sys.argv[6]) if len(sys.argv) > 6 else 0  # 1: C += (the residual form)
torch.cuda.set_device(0)
lib = C.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), 'libgemm_tune.so'))
lib.tune_gemm.argtypes = [C.c_int]*4 + [C.c_void_p]*5 + [C.c_int, C.c_void_p]
lib.tune_gemm_silu_v.argtypes = [C.c_int]*4 + [C.c_void_p]*6 + [C.c_int64, C.c_int, C.c_void_p]


class DW(C.Structure):
    _fields_ = [('N', C.c_int64), ('K', C.c_int64), ('Npad', C.c_int64), ('Kb', C.c_int64),
                ('Kp', C.c_int64), ('q', C.c_void_p), ('scale', C.c_void_p)]


q = torch.randint(-127, 128, (N, K), dtype=torch.int8, device='cuda')
s = torch.rand(N, device='cuda') * 1e-3 + 1e-4
w = ov.Weight.from_device(q, s); dw = DW.from_address(w.handle.value)
A = torch.randn(M, K, device='cuda'); aq, asc = ov.s8_nk_quantize(A)
st = torch.cuda.current_stream().cuda_stream
if cfg_s.startswith('s'):
    # tile-major codes: the weight tile layout of the same rows (rows past M zero)
    at = ov.Weight.from_device(aq.view(torch.int8)[:, :K].contiguous(), torch.ones(M, device='cuda'))
    dat = DW.from_address(at.handle.value)
    inter = N // 2
    hq = torch.zeros(((M + 127) // 128 * 128) * inter, dtype=torch.int8, device='cuda')
    hsc = torch.zeros(M * (inter // 32), device='cuda')
    for _ in range(reps):
        rc = lib.tune_gemm_silu_v(int(cfg_s[1:]), M, N, K // 32, dat.q, asc.data_ptr(), dw.q,
                                  dw.scale, hq.data_ptr(), hsc.data_ptr(), inter, 1, st)
        assert rc == 0, rc
else:
    Cc = torch.zeros(M, N, device='cuda')
    for _ in range(reps):
        rc = lib.tune_gemm(int(cfg_s), M, N, K // 32, aq.data_ptr(), asc.data_ptr(), dw.q,
                           dw.scale, Cc.data_ptr(), acc, st)
        assert rc == 0, rc
torch.cuda.synchronize()
print("done", cfg_s, M, N, K, reps)
