"""Sweep every GEMM tile config over the LM shapes; checks each against the
product kernel bit for bit and prints per-config time.

    python3 ovnative_amd/tune/tune_gemm.py [CFG,CFG,...] [--tiled]

--tiled: the activation codes tile-major, as the runner holds them (the 16x16
configs only, 8 and up); default: row-major, as ovh_s8_nk_quantize writes them.
"""
import ctypes as C, sys, os
ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import torch, ovnative_amd as ov
torch.cuda.set_device(0)
lib = C.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), 'libgemm_tune.so'))
lib.tune_gemm.argtypes = [C.c_int]*4 + [C.c_void_p]*5 + [C.c_int, C.c_void_p]
lib.tune_gemm_at.argtypes = [C.c_int]*4 + [C.c_void_p]*5 + [C.c_int, C.c_void_p, C.c_int]
tiled = '--tiled' in sys.argv
argv = [a for a in sys.argv[1:] if a != '--tiled']
class DW(C.Structure):
    _fields_ = [('N', C.c_int64), ('K', C.c_int64), ('Npad', C.c_int64), ('Kb', C.c_int64), ('Kp', C.c_int64), ('q', C.c_void_p), ('scale', C.c_void_p)]
# 0-7: the 32x32-tile kernel (register-staged); 8-24: the 16x16-tile kernel
# (LDS DMA ring, software-pipelined stage loop): s<BN>x<BM>w<waves>[b<blocks per
# stage>][n<ring stages>]; 30-35: 16x16 tiles with the block-by-block stage loop (b...)
cfgs = {0: '128x128', 1: '64x128', 2: '64x64', 3: '32x64', 4: '128x64', 5: '32x128', 6: '64x32', 7: '32x32',
        8: 's32x32w4', 9: 's64x32w4', 10: 's128x64w8', 11: 's128x64w8n3', 12: 's64x32w8',
        13: 's64x64w4n3', 14: 's32x32w4b8', 15: 's64x32w4xn3', 16: 's32x32w4n3', 17: 's32x32w4n4',
        18: 's32x32w4b8n3', 19: 's32x64w4n3', 20: 's32x32w4n6', 21: 's64x32w4n4', 22: 's128x64w8n4',
        23: 's64x32w4n3', 24: 's64x64w4n4',
        30: 'b32x32w4', 31: 'b64x32w4', 32: 'b128x64w8', 33: 'b128x64w8n3', 34: 'b32x32w4n4',
        35: 'b64x32w4xn3', 40: 's32x32w2m', 41: 's32x32w2n', 42: 's64x32w2', 43: 's64x32w2m',
        44: 's32x32w2n3', 45: 's32x32w2nb8', 46: 's32x32w2mb8', 47: 's32x32w4b16', 48: 's64x32w2b8',
        49: 's64x32w4b8'}
if argv:
    cfgs = {k: v for k, v in cfgs.items() if str(k) in argv[0].split(',')}
if tiled:
    cfgs = {k: v for k, v in cfgs.items() if k >= 8}
shapes = [(600, 6144, 1024), (600, 4096, 1024), (600, 1024, 2048), (600, 1024, 3072), (600, 8192, 1024),
          (600, 2048, 1024), (600, 3072, 1024),
          (128, 4096, 1024), (128, 6144, 1024), (128, 1024, 2048), (128, 1024, 3072), (128, 2048, 1024), (128, 1024, 1024),
          (256, 3072, 1024), (16384, 6144, 1024), (16384, 1024, 3072)]
st = torch.cuda.current_stream()
for (M, N, K) in shapes:
    q = torch.randint(-127, 128, (N, K), dtype=torch.int8, device='cuda')
    s = torch.rand(N, device='cuda') * 1e-3 + 1e-4
    w = ov.Weight.from_device(q, s)
    dw = DW.from_address(w.handle.value)
    A = torch.randn(M, K, device='cuda')
    aq, asc = ov.s8_nk_quantize(A)
    ref = ov.linear_q(aq, asc, w)
    a_ptr = aq.data_ptr()
    if tiled:  # the same codes in the weight tile order (rows past M zero)
        at = ov.Weight.from_device(aq.view(torch.int8)[:, :K].contiguous(), torch.ones(M, device='cuda'))
        a_ptr = DW.from_address(at.handle.value).q
    res = []
    for cfg, name in cfgs.items():
        C_ = torch.empty(M, N, device='cuda')
        args = (cfg, M, N, K // 32, a_ptr, asc.data_ptr(), dw.q, dw.scale, C_.data_ptr(), 0,
                st.cuda_stream, int(tiled))
        rc = lib.tune_gemm_at(*args); torch.cuda.synchronize()
        ok = rc == 0 and torch.equal(C_.view(torch.int32), ref.view(torch.int32))
        n = 30 if M * N * K < 1e11 else 8
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for _ in range(3): lib.tune_gemm_at(*args)
        e0.record()
        for _ in range(n): lib.tune_gemm_at(*args)
        e1.record(); torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / n * 1e3
        res.append((us, name, ok))
    res.sort()
    print(f"M={M} N={N} K={K}{' tiled' if tiled else ''}: "
          + "  ".join(f"{nm}:{us:.1f}us{'' if ok else '!BAD'}" for us, nm, ok in res)
          + f"  | best {2*M*N*K/res[0][0]/1e6:.0f} TOPS", flush=True)
