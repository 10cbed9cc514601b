"""BASELINE config 2 with cold weights: the seven projections of a layer (q, k, v,
o, gate, up, down) at M = 128, over 28 layers of distinct int8 weights (440 MB,
more than the 256 MB last-level cache, so every weight comes from HBM), through
the product entry point (ovh_linear_q).  Prints per projection the mean time per
launch and the weight-read rate (int8 bytes + fp32 scales / time).

    python3 ovnative_amd/tune/skinny_layer.py [M] [CFG]

CFG (optional) runs a gemm_tune.hip config instead of the product dispatch."""
import ctypes as C, sys, os
sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
import torch, ovnative_amd as ov
M = int(sys.argv[1]) if len(sys.argv) > 1 else 128
cfg = int(sys.argv[2]) if len(sys.argv) > 2 else None
torch.cuda.set_device(0)
H, QD, KVD, I, L = 1024, 2048, 1024, 3072, 28
shapes = [("q", QD, H), ("k", KVD, H), ("v", KVD, H), ("o", H, QD), ("gate", I, H), ("up", I, H),
          ("down", H, I)]
g = torch.Generator(device="cuda").manual_seed(3)
lib = None
if cfg is not None:
    lib = C.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), 'libgemm_tune.so'))
    lib.tune_gemm.argtypes = [C.c_int]*4 + [C.c_void_p]*5 + [C.c_int, C.c_void_p]

    class DW(C.Structure):
        _fields_ = [('N', C.c_int64), ('K', C.c_int64), ('Npad', C.c_int64), ('Kb', C.c_int64),
                    ('Kp', C.c_int64), ('q', C.c_void_p), ('scale', C.c_void_p)]
layers = []
for _ in range(L):
    ws = []
    for name, n, k in shapes:
        q = torch.randint(-127, 128, (n, k), generator=g, device="cuda", dtype=torch.int8)
        s = torch.rand(n, generator=g, device="cuda") * 1e-3 + 1e-4
        ws.append(ov.Weight.from_device(q, s))
    layers.append(ws)
acts = {k: ov.s8_nk_quantize(torch.randn((M, k), generator=g, device="cuda")) for k in (H, QD, I)}
outs = {n: torch.zeros((M, n), device="cuda") for n in (QD, KVD, H, I)}
st = torch.cuda.current_stream().cuda_stream


def run(j, w):
    name, n, k = shapes[j]
    aq, asc = acts[k]
    if lib is None:
        # the C ABI entry itself: a Python wrapper per launch would leave the
        # GPU waiting on the host at these kernel times
        ov.load().ovh_linear_q(M, aq.data_ptr(), asc.data_ptr(), w.handle, outs[n].data_ptr(), n,
                               0, st)
    else:
        dw = DW.from_address(w.handle.value)
        lib.tune_gemm(cfg, M, n, k // 32, aq.data_ptr(), asc.data_ptr(), dw.q, dw.scale,
                      outs[n].data_ptr(), 0, st)


for ws in layers:  # warm-up (code, allocator); weights are evicted again below
    for j, w in enumerate(ws):
        run(j, w)
torch.cuda.synchronize()
tot_b, tot_t = 0, 0.0
for j, (name, n, k) in enumerate(shapes):
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for ws in layers:
        run(j, ws[j])
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / L * 1e3
    b = n * k + 4 * n
    tot_b += b
    tot_t += us
    print(f"{name:5s} N={n:5d} K={k:5d}: {us:6.2f} us/launch  {b / us / 1e3:7.1f} GB/s weights", flush=True)
print(f"seven projections: {tot_b / 1e6:.2f} MB in {tot_t:.2f} us = {tot_b / tot_t / 1e3:.0f} GB/s "
      f"({tot_b / tot_t / 1e3 / 80:.1f} % of 8 TB/s), M={M}, "
      f"{'product dispatch' if cfg is None else f'config {cfg}'}", flush=True)
