#!/usr/bin/env python3
"""Benchmark of the int8-nk LM path on one MI355X.

Workload (the one the metric is quoted on): one CFG
decoding step of the 28-layer Qwen3-0.6B-shaped LM at seq 300, CFG batch 2
(cond = 40 text + 260 audio positions, uncond = the 260 target positions, as
cpp/src/model/tts.cpp:175-213 builds the batch; M = 600 rows), run by the HIP
LM runner (ovh_lm_*, the cuda_lm.h plugin contract):

    embed -> 28 x [rmsnorm+quant, qkv (merged), qk-norm+RoPE, GQA attention,
    quant + o_proj (+= x), rmsnorm+quant, gate/up (merged), silu*up+quant,
    down (+= x)] -> final rmsnorm+quant -> int8 audio head (1024 -> 8 x 1025)
    -> device guided sampling (guidance 2, layer penalty 5).

Weights are random ~N(0, 0.02), int8-quantised per output channel (440 MB of
linears plus the head and int8 embedding tables, resident in HBM before timing);
inputs are synthetic token ids.

value    = int8 linear throughput of the whole step: 2*M*N*K summed over every
           linear of the forward, divided by the measured step time (attention,
           norms, embedding and sampling included in that time), TOPS;
roofline = the kernel with the largest share of the step: the residual GEMM
           (o_proj, K=2048, and down, K=3072; M=600, N=1024, accumulating into
           the fp32 hidden state), 28 launches of each on distinct weights with
           tile-major codes, replayed as a HIP graph as the step runs them and
           timed with HIP events on the stream they run on; bound = the roof its
           algorithmic intensity binds (HBM: 339 int8 ops per byte, below the
           625 ridge), with the epilogue-VALU ceiling as a second line;
cpu_baseline = the reference's own LM::forward (cpp/src/model/lm.cpp, compiled
           from source into oracle/_ref) on the same checkpoint and batch, on
           the host's cores, when its AVX-VNNI int8-nk dispatch is available;
           else the oracle's restatement (a port) on a shorter model.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# CPU baseline placement: OpenMP threads bound close to the cores they start
# on, one per core; set before any OpenMP runtime starts.
os.environ.setdefault("OMP_PROC_BIND", "close")
os.environ.setdefault("OMP_PLACES", "cores")
try:  # the CPUs this process may use, read before OpenMP binds the main thread
    CPUS_ALLOWED = len(os.sched_getaffinity(0))
except (AttributeError, OSError):
    CPUS_ALLOWED = os.cpu_count()

CFG = dict(n_layers=28, hidden=1024, n_heads=16, n_kv_heads=8, head_dim=128, inter=3072,
           vocab=151676, audio_vocab=1025, n_codebooks=8, rms_eps=1e-6, rope_theta=1e6)
SEQ, TEXT, CFG_BATCH = 300, 40, 2
PEAK_INT8_TOPS = 5000.0


def linear_ops(cfg: dict, M: int, layers: int) -> int:
    H, QD = cfg["hidden"], cfg["n_heads"] * cfg["head_dim"]
    KVD, I = cfg["n_kv_heads"] * cfg["head_dim"], cfg["inter"]
    per_layer = 2 * M * (H * (QD + 2 * KVD) + QD * H + 2 * H * I + I * H)
    return layers * per_layer + 2 * M * H * cfg["n_codebooks"] * cfg["audio_vocab"]


def attention_flops(cfg: dict, seq: int, batch: int, layers: int) -> int:
    return layers * batch * cfg["n_heads"] * 4 * seq * seq * cfg["head_dim"]


NORM_TRAFFIC = "gemm_residual_norm_m600_traffic.json"


def residual_traffic(name="gemm_residual_m600_traffic.json"):
    """HBM bytes per launch of the residual GEMM (mean of the o_proj and down
    launches), or of the kernel another committed PMC summary names (FETCH_SIZE
    + WRITE_SIZE, scaled by the copy-kernel calibration)."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            return json.load(f)["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--layers", type=int, default=CFG["n_layers"])
    p.add_argument("--cpu-seconds", type=float, default=15.0,
                   help="wall-clock budget of the CPU-baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--workload", choices=("step", "m16384", "linear", "skinny", "layer",
                                          "residual"),
                   default="step",
                   help="step: BASELINE config 4 (the metric); m16384: config 5, one forward "
                        "of 8 requests x CFG 2 x seq 1024 (M = 16384); linear: config 1, one "
                        "quantise + int8 linear at M=256, K=1024, N=3072; skinny: config 2, a "
                        "layer's seven projections at M=2x64, weights cold; layer: config 3, "
                        "one decoder layer at M=2x300; residual: the roofline kernel alone "
                        "(with a 64 MiB copy for counter calibration)")
    return p.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# checkpoint and inputs

def make_checkpoint(cfg: dict, seed: int = 0):
    """Random int8 checkpoint with the reference's tensor names and encodings
    (linears int8 [N, K] + per-row scales, embeddings int8 + per-row scales,
    fp32 norms): fp32 weights drawn on the GPU, quantised on the host by
    ovw1.quantize_int8 (the converter's quantisation, tools/convert_weights.py:
    130-135), returned as host arrays."""
    import numpy as np
    import torch
    from ovnative_amd import ovw1
    g = torch.Generator(device="cuda").manual_seed(seed)

    def q8(rows, cols):
        qs, ss = [], []
        for r0 in range(0, rows, 16384):  # row chunks bound the host temporaries
            n = min(16384, rows - r0)
            w = (torch.randn((n, cols), generator=g, device="cuda") * 0.02).cpu().numpy()
            q, s = ovw1.quantize_int8(w)
            qs.append(q)
            ss.append(s)
        return np.concatenate(qs), np.concatenate(ss)

    def norm(n):
        return (1.0 + 0.1 * torch.randn(n, generator=g, device="cuda")).float().cpu().numpy()

    H, D, I = cfg["hidden"], cfg["head_dim"], cfg["inter"]
    QD, KVD = cfg["n_heads"] * D, cfg["n_kv_heads"] * D
    CV = cfg["n_codebooks"] * cfg["audio_vocab"]
    ts = []
    for name, rows in (("llm.embed_tokens.weight", cfg["vocab"]), ("audio_embeddings.weight", CV),
                       ("audio_heads.weight", CV)):
        q, s = q8(rows, H)
        ts.append(ovw1.Tensor(name, q, 0, s))
    ts.append(ovw1.Tensor("llm.norm.weight", norm(H)))
    ts.append(ovw1.Tensor("codebook_layer_offsets",
                          np.arange(cfg["n_codebooks"], dtype=np.int64) * cfg["audio_vocab"]))
    for i in range(cfg["n_layers"]):
        p = f"llm.layers.{i}."
        for name, n in (("input_layernorm", H), ("post_attention_layernorm", H),
                        ("self_attn.q_norm", D), ("self_attn.k_norm", D)):
            ts.append(ovw1.Tensor(p + name + ".weight", norm(n)))
        for name, (n, k) in (("self_attn.q_proj", (QD, H)), ("self_attn.k_proj", (KVD, H)),
                             ("self_attn.v_proj", (KVD, H)), ("self_attn.o_proj", (H, QD)),
                             ("mlp.gate_proj", (I, H)), ("mlp.up_proj", (I, H)),
                             ("mlp.down_proj", (H, I))):
            q, s = q8(n, k)
            ts.append(ovw1.Tensor(p + name + ".weight", q, 0, s))
    return ts


def make_inputs(cfg: dict, seed: int = 1, seq: int = SEQ, text: int = TEXT):
    """The CFG batch of tts.cpp:175-213: row 0 = cond prompt (text + audio),
    row 1 = uncond (the target slice, then mask tokens attending to themselves)."""
    import numpy as np
    rng = np.random.default_rng(seed)
    Cb, V, S, TEXT_ = cfg["n_codebooks"], cfg["audio_vocab"], seq, text
    T = S - TEXT_
    ids = np.full((2, Cb, S), V - 1, np.int64)
    ids[0, :, TEXT_:] = rng.integers(0, V - 1, (Cb, T))
    ids[0, 0, :TEXT_] = rng.integers(0, cfg["vocab"], TEXT_)
    ids[1, :, :T] = ids[0, :, TEXT_:]
    am = np.zeros((2, S), np.uint8)
    am[0, TEXT_:] = 1
    am[1, :T] = 1
    attn = np.ones((2, S, S), np.uint8)
    attn[1] = 0
    attn[1, :T, :T] = 1
    attn[1, np.arange(T, S), np.arange(T, S)] = 1
    pos = np.tile(np.arange(S, dtype=np.int64), (2, 1))
    return ids, am, attn, pos, T


def make_requests(cfg: dict, requests: int, seq: int, text: int = TEXT):
    """`requests` independent CFG pairs stacked into one batch of 2*requests rows."""
    import numpy as np
    parts = [make_inputs(cfg, seed=10 + r, seq=seq, text=text)[:4] for r in range(requests)]
    return tuple(np.concatenate([p[i] for p in parts]) for i in range(4))


# ---------------------------------------------------------------------------
# GPU

class LmStep:
    def __init__(self, cfg: dict, tensors):
        import ovnative_amd as ov
        self.cfg = cfg
        self.lm = ov.LM.from_tensors(tensors, ov.LmConfig(**cfg))
        self.lm.set_device_sampling(True)
        self.ids, self.am, self.attn, self.pos, self.T = make_inputs(cfg)
        self.plane = SEQ * cfg["n_codebooks"] * cfg["audio_vocab"] * 4

    def run(self):
        """One CFG decoding step: forward (logits stay on the device) and the
        guidance/argmax pass; returns (pred, scores) on the host."""
        self.lm.forward(self.ids, self.am, self.attn, self.pos, host_logits=False)
        base = self.lm.last_logits_ptr()
        return self.lm.sample(base, SEQ, base + self.plane, SEQ, self.T, 2.0, 5.0)


def residual_bytes(cfg: dict, M: int) -> float:
    """Algorithmic HBM bytes of one residual launch, the mean of o_proj (K = heads
    x 128) and down (K = inter): int8 weight N*K and its fp32 scales 4N, int8
    codes M*Kp and fp32 block scales 4*M*Kb, the fp32 residual read and written
    (4*M*N each)."""
    H, QD, I = cfg["hidden"], cfg["n_heads"] * cfg["head_dim"], cfg["inter"]

    def one(K):
        Kb = (K + 31) // 32
        return H * K + 4 * H + M * 32 * Kb + 4 * M * Kb + 8 * M * H
    return (one(QD) + one(I)) / 2


def norm_out_bytes(cfg: dict, M: int) -> float:
    """Algorithmic HBM bytes the fused RMSNorm + quantise adds to a residual
    launch: its codes M*N and fp32 block scales 4*M*N/32 written, its weight 4N
    read (the updated rows it normalises are the launch's own output, read back
    from L2)."""
    H = cfg["hidden"]
    return M * H + 4 * M * (H // 32) + 4 * H


# Epilogue ceiling of the int8 GEMM with the reference's exact epilogue: per
# output and 32-k block one v_cvt_f32_i32 and one v_fma_f32; a wave64 VALU
# instruction takes 4 clocks on a 16-lane SIMD, so a 16x16x32 block product
# (16384 ops, 4 outputs per lane) costs 32 VALU clocks: 512 ops per clock per
# SIMD, x 1024 SIMDs x 2.4 GHz.
VALU_CEIL_TOPS = 512 * 1024 * 2.4e9 / 1e12
HBM_PEAK_GBS = 8000.0
RIDGE_OPS_PER_BYTE = PEAK_INT8_TOPS * 1e12 / (HBM_PEAK_GBS * 1e9)


def roofline_entry(kernel: str, ops: float, nbytes: float, ms: float, traffic=None, **extra):
    """The binding roof from the algorithmic intensity (ops / bytes against the
    ridge, 625 int8 ops per byte), achieved against it, and the epilogue-VALU
    ceiling as a second reference line."""
    tops = ops / (ms * 1e-3) / 1e12
    if ops / nbytes < RIDGE_OPS_PER_BYTE:
        gbs = nbytes / (ms * 1e-3) / 1e9
        e = {"bound": "hbm", "kernel": kernel, "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
             "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}
    else:
        e = {"bound": "mfma", "kernel": kernel, "achieved": round(tops, 2),
             "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s", "frac": round(tops / PEAK_INT8_TOPS, 4)}
    e.update({"traffic": traffic, "avg_ms": round(ms, 5), "algorithmic_bytes": round(nbytes),
              "ops_per_launch": round(ops), "int8_tops": round(tops, 2),
              "valu_epilogue_ceiling": {"tops": round(VALU_CEIL_TOPS, 1),
                                        "frac": round(tops / VALU_CEIL_TOPS, 4)}})
    e.update(extra)
    return e


def time_residual(cfg: dict, layers: int, M: int, reps: int = 4, eager: bool = True,
                  norm: bool = False):
    """The residual GEMM as the step runs it: `layers` o_proj (K = heads*128) and
    `layers` down (K = inter) launches on distinct weights with tile-major codes
    (the runner's layout), accumulating into one fp32 [M, hidden] buffer,
    captured once as a HIP graph (the runner replays its forward as one) and
    replayed between one pair of HIP events on the stream it runs on.  Each of
    the `reps` passes has its own weights (reps x 140 MB at the LM shape), so,
    as in the step, where 440 MB of weights go by between two uses of one
    weight, every launch reads its weight from HBM rather than from the 256 MB
    last-level cache.  Also timed: the same launches eagerly through the C ABI
    with row-major codes.  With `norm`, the same launches as the step makes them
    below 2048 rows, each with the RMSNorm + quantise that follows it
    (ovh_linear_q_norm: o_proj with the post-attention norm, down with the next
    layer's input norm), captured and replayed the same way.  Returns
    dict(graph_ms, eager_ms, graph_norm_ms per launch, ops per launch on
    average)."""
    import torch
    import ovnative_amd as ov
    H, QD, I = cfg["hidden"], cfg["n_heads"] * cfg["head_dim"], cfg["inter"]
    g = torch.Generator(device="cuda").manual_seed(7)

    def weight(n, k):
        q = torch.randint(-127, 128, (n, k), generator=g, device="cuda", dtype=torch.int8)
        s = torch.rand(n, generator=g, device="cuda") * 1e-3 + 1e-4
        return ov.Weight.from_device(q, s)

    wo = [weight(H, QD) for _ in range(layers * reps)]
    wd = [weight(H, I) for _ in range(layers * reps)]
    ao = ov.s8_nk_quantize(torch.randn((M, QD), generator=g, device="cuda"))
    ad = ov.s8_nk_quantize(torch.randn((M, I), generator=g, device="cuda"))
    to, td = ov.tile_major(ao[0]), ov.tile_major(ad[0])
    x = torch.zeros((M, H), device="cuda")

    # straight through the C ABI: at ~10 us per launch a Python wrapper per call
    # would leave the GPU waiting on the host
    lib = ov.load()

    def launches(fn, a_o, a_d, st):
        for a, b in zip(wo, wd):
            if fn(M, a_o.data_ptr(), ao[1].data_ptr(), a.handle, x.data_ptr(), H, 1, st) != 0 or \
               fn(M, a_d.data_ptr(), ad[1].data_ptr(), b.handle, x.data_ptr(), H, 1, st) != 0:
                raise RuntimeError(ov.load().ovh_last_error().decode())

    n = reps * 2 * layers
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out = {"ops": (2 * M * H * QD + 2 * M * H * I) / 2}
    if eager:
        st = torch.cuda.current_stream().cuda_stream
        launches(lib.ovh_linear_q, ao[0], ad[0], st)   # warm-up
        torch.cuda.synchronize()
        e0.record()
        launches(lib.ovh_linear_q, ao[0], ad[0], st)
        e1.record()
        torch.cuda.synchronize()
        out["eager_ms"] = e0.elapsed_time(e1) / n
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launches(lib.ovh_linear_q_tiled, to, td, side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        launches(lib.ovh_linear_q_tiled, to, td, torch.cuda.current_stream().cuda_stream)
    graph.replay()  # warm-up; the timed replay starts on the set used longest ago
    torch.cuda.synchronize()
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    out["graph_ms"] = e0.elapsed_time(e1) / n
    del graph
    if norm:
        nw = [torch.rand(H, generator=g, device="cuda") + 0.5 for _ in range(2)]
        nq = torch.zeros(lib.ovh_tiled_codes_bytes(M, H), dtype=torch.int8, device="cuda")
        nsc = torch.empty((M, H // 32), device="cuda")
        cnt = ov.band_counters(M)

        def launches_norm(st):
            for a, b in zip(wo, wd):
                for (t, sc, w, v) in ((to, ao[1], a, nw[0]), (td, ad[1], b, nw[1])):
                    if lib.ovh_linear_q_norm(M, t.data_ptr(), sc.data_ptr(), w.handle,
                                             x.data_ptr(), H, v.data_ptr(), cfg["rms_eps"],
                                             nq.data_ptr(), nsc.data_ptr(), cnt.data_ptr(),
                                             st) != 0:
                        raise RuntimeError(ov.load().ovh_last_error().decode())
        graph = torch.cuda.CUDAGraph()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            launches_norm(side.cuda_stream)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            launches_norm(torch.cuda.current_stream().cuda_stream)
        graph.replay()
        torch.cuda.synchronize()
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        out["graph_norm_ms"] = e0.elapsed_time(e1) / n
        if int(cnt[0].item()) != 0:
            raise RuntimeError("residual + norm: a band hand-off wait ran out")
        del graph
    for w in wo + wd:
        w.free()
    return out


def counter_calibration() -> None:
    """Untimed reads of known size that PMC runs of the counter workloads scale
    their byte counters by: a 64 MiB device copy (64 MiB read and 64 MiB
    written), then the same 64 MiB read once through each load path of the
    GEMM kernels (ovh_diag_read: DMA into LDS 16 and 4 bytes a lane, 16-byte
    vector loads, 8-byte buffer loads), which shows whether one scale holds for
    the GEMMs' own loads."""
    import torch
    import ovnative_amd as ov
    src = torch.ones(16 << 20, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    junk = torch.empty(1 << 28, device="cuda")  # 1 GiB: evicts src between the reads
    for path in (ov.READ_DMA16, ov.READ_DMA4, ov.READ_VEC16, ov.READ_BUF8):
        junk.fill_(0.0)
        ov.diag_read(src, path)
    torch.cuda.synchronize()
    del src, dst, junk


def run_residual(args) -> None:
    """The roofline kernel alone, for counter runs: a 64 MiB device copy (the
    calibration the HBM byte counters are scaled by) and one replay of the
    step's residual GEMM launches (time_residual, cold weights)."""
    import torch
    M = SEQ * CFG_BATCH
    counter_calibration()
    rs = time_residual(CFG, args.layers, M, eager=False, norm=True)
    nbytes = residual_bytes(CFG, M)
    print(json.dumps({"workload": "the residual GEMM launches of the step (o_proj and down, "
                                  "M=600, weights cold, graph replay), plain and with the "
                                  "following RMSNorm + quantise (the roofline kernel), after a "
                                  "64 MiB copy calibration",
                      "roofline": roofline_entry("gemm16 residual + norm", rs["ops"],
                                                 nbytes + norm_out_bytes(CFG, M),
                                                 rs["graph_norm_ms"],
                                                 residual_traffic(NORM_TRAFFIC)),
                      "plain_residual": roofline_entry("gemm16 residual", rs["ops"], nbytes,
                                                       rs["graph_ms"], residual_traffic())}),
          flush=True)


# ---------------------------------------------------------------------------
# CPU baseline (reported beside the GPU, not optimised)

def host_cpu() -> dict:
    """What the CPU baseline ran on: the CPU model, the CPUs this process may
    use, and the OpenMP settings."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "cpus_allowed": CPUS_ALLOWED, "cpus_online": os.cpu_count(),
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS"),
            "OMP_PROC_BIND": os.environ.get("OMP_PROC_BIND"),
            "OMP_PLACES": os.environ.get("OMP_PLACES")}


def cpu_baseline(cfg: dict, tensors, budget_s: float, batch=None):
    """batch = (ids, am, attn, pos) (default: the config-4 CFG batch)."""
    import oracle
    ids, am, attn, pos = batch if batch is not None else make_inputs(cfg)[:4]
    B, S = am.shape
    M = B * S
    threads = oracle.Oracle().num_threads()
    ref = None
    if oracle.reference_available():
        try:
            r = oracle.Reference()
            ref = r if r.vnni_available() else None
        except OSError:
            ref = None
    if ref is not None:
        from ovnative_amd import ovw1
        with tempfile.TemporaryDirectory() as d:
            path = os.path.join(d, "lm.ovw")
            ovw1.write(path, tensors)
            h = ref.lm_open(path, cfg)
            try:
                ref.lm_forward(h, cfg, ids, am, attn, pos)     # warm-up
                times = []
                t_end = time.perf_counter() + budget_s
                while len(times) < 2 or (time.perf_counter() < t_end and len(times) < 30):
                    t0 = time.perf_counter()
                    ref.lm_forward(h, cfg, ids, am, attn, pos)
                    times.append(time.perf_counter() - t0)
            finally:
                ref.lm_close(h)
        sec = statistics.median(times)
        ops = linear_ops(cfg, M, cfg["n_layers"])
        return {
            "value": round(ops / sec / 1e12, 4),
            "unit": "TOPS",
            "cores": threads,
            "kind": "reference",
            "sample": (f"reference LM::forward (lm.cpp, {ref.kernel_name()} int8-nk kernels) on the "
                       f"same checkpoint: {cfg['n_layers']} layers, B={B}, S={S}, median of "
                       f"{len(times)} forwards (host sampling pass not included)"),
            "ms_per_step": round(sec * 1e3, 2),
            "isa": ref.kernel_name(),
            "host": host_cpu(),
        }
    # No reference VNNI dispatch on this host: time the oracle's restatement on a
    # 2-layer prefix of the same model and scale per layer.
    o = oracle.Oracle()
    if not o.fast_available():
        return None
    nl = 2
    table = {t.name: (t.array, t.scales, t.layout == 1) for t in tensors}
    segs = [(attn[b], S, b * S) for b in range(B)]
    sub = dict(cfg, n_layers=nl)
    o.lm_forward(sub, table, ids, am, segs, pos.reshape(-1))
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 2 or (time.perf_counter() < t_end and len(times) < 10):
        t0 = time.perf_counter()
        o.lm_forward(sub, table, ids, am, segs, pos.reshape(-1))
        times.append(time.perf_counter() - t0)
    sec = statistics.median(times)
    ops = linear_ops(cfg, M, nl)
    return {
        "value": round(ops / sec / 1e12, 4),
        "unit": "TOPS",
        "cores": threads,
        "kind": "port",
        "sample": f"oracle restatement, {nl}-layer prefix at B={B} S={S}, median of {len(times)}",
        "ms_per_step": None,
        "host": host_cpu(),
    }


def bench_line(args, value, unit, ms, config, roofline, cpu, wall, dtype="int8"):
    return {
        "metric": "int8 linear TOPS & % roofline; LM ms/step (seq 300, CFG batch 2)",
        "value": value,
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic",
        "config": config,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "wall_s": wall,
    }


def linear_inputs(M=256, K=1024, N=3072, seed=1234):
    """A fp32 [M, K] ~N(0, 1) with 8 outlier channels x20, W
    fp32 [N, K] ~N(0, 0.02) quantised per output channel as
    tools/convert_weights.py:130-135 does (float32 scale = max(absmax/127,
    1e-12), q = clip(rint(w / scale), -127, 127))."""
    import numpy as np
    rng = np.random.default_rng(seed)
    A = rng.standard_normal((M, K)).astype(np.float32)
    A[:, rng.choice(K, 8, replace=False)] *= np.float32(20.0)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    s = np.maximum(np.abs(W).max(axis=1) / np.float32(127.0), np.float32(1e-12)).astype(np.float32)
    q = np.clip(np.rint(W / s[:, None]), -127, 127).astype(np.int8)
    return A, q, s


def run_linear(args) -> None:
    """the int8-nk linear of fp32 activations,
    linear_s8_nk_packed (quantise A per 32-k block, then the int8 GEMM) as
    ovh_linear on device-resident inputs: one step = that call (its codes
    tile-major inside).  Also timed: the reference's q path as two calls
    (ovh_s8_nk_quantize + ovh_linear_q, row-major codes), and the GEMM alone on
    tile-major codes for the roofline (HBM-bound: 6.60 MB of algorithmic
    traffic against 1.61 GOP)."""
    import numpy as np
    import torch
    import ovnative_amd as ov
    M, K, N = 256, 1024, 3072
    A, q, s = linear_inputs(M, K, N)
    w = ov.Weight.from_host(q, s)
    lib = ov.load()
    st = torch.cuda.current_stream().cuda_stream
    dA = torch.from_numpy(A).cuda()
    Kb = (K + 31) // 32
    aq = torch.empty((M, 32 * Kb), dtype=torch.int8, device="cuda")
    asc = torch.empty((M, Kb), dtype=torch.float32, device="cuda")
    C_ = torch.empty((M, N), dtype=torch.float32, device="cuda")
    qargs = (M, K, dA.data_ptr(), aq.data_ptr(), asc.data_ptr(), st)
    largs = (M, aq.data_ptr(), asc.data_ptr(), w.handle, C_.data_ptr(), N, 0, st)
    fargs = (M, dA.data_ptr(), w.handle, C_.data_ptr(), N, 0, st)
    aqt = ov.tile_major(ov.s8_nk_quantize(dA)[0])
    targs = (M, aqt.data_ptr(), asc.data_ptr(), w.handle, C_.data_ptr(), N, 0, st)

    def timed(fns, reps):
        for _ in range(args.warmup):
            for f, a in fns:
                if f(*a) != 0:
                    raise RuntimeError("C ABI call failed")
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            for f, a in fns:
                f(*a)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    t0 = time.perf_counter()
    reps = max(args.steps, 200)
    ms_step = timed([(lib.ovh_linear, fargs)], reps)
    ms_pair = timed([(lib.ovh_s8_nk_quantize, qargs), (lib.ovh_linear_q, largs)], reps)
    ms_gemm_rm = timed([(lib.ovh_linear_q, largs)], reps)
    ms_gemm = timed([(lib.ovh_linear_q_tiled, targs)], reps)
    ms_quant = timed([(lib.ovh_s8_nk_quantize, qargs)], reps)
    wall = time.perf_counter() - t0
    ops = 2 * M * N * K
    gemm_bytes = N * K + 4 * N + M * 32 * Kb + 4 * M * Kb + 4 * M * N
    log(f"config 1: ovh_linear {ms_step * 1e3:.2f} us; as two calls {ms_pair * 1e3:.2f} us "
        f"(quantise {ms_quant * 1e3:.2f}, linear {ms_gemm_rm * 1e3:.2f}); the GEMM on tile-major "
        f"codes {ms_gemm * 1e3:.2f} us = {gemm_bytes / ms_gemm / 1e6:.0f} GB/s")
    cpu = None
    if not args.no_cpu:
        import oracle
        impl, kind = None, None
        if oracle.reference_available():
            try:
                r = oracle.Reference()
                if r.vnni_available():
                    impl, kind = r, "reference"
            except OSError:
                impl = None
        if impl is None:
            o = oracle.Oracle()
            if o.fast_available():
                impl, kind = o, "port"
        if impl is not None:
            packed, wsum = impl.pack(q)
            Cc = np.zeros((M, N), np.float32)
            times = []
            t_end = time.perf_counter() + min(args.cpu_seconds, 10.0)
            while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 500):
                t1 = time.perf_counter()
                caq, casc = impl.quantize(A)
                impl.linear_q_packed(caq, casc, packed, wsum, N, K, s, Cc)
                times.append(time.perf_counter() - t1)
            sec = statistics.median(times)
            cpu = {"value": round(ops / sec / 1e12, 4), "unit": "TOPS",
                   "cores": oracle.Oracle().num_threads(), "host": host_cpu(), "kind": kind,
                   "sample": (f"s8_nk_quantize + linear_s8_nk_packed_q at M={M}, K={K}, N={N} "
                              f"({'reference gemm.cpp' if kind == 'reference' else 'oracle restatement'}"
                              f"), median of {len(times)}"),
                   "ms_per_step": round(sec * 1e3, 4)}
    frac_gb = gemm_bytes / ms_gemm / 1e6
    line = bench_line(
        args, round(ops / (ms_step * 1e-3) / 1e12, 2), "TOPS", round(ms_step, 5),
        {"workload": (f"BASELINE config 1: ovh_linear (linear_s8_nk_packed): A fp32 [{M},{K}] "
                      f"(~N(0,1), 8 outlier channels x20) quantised per 32-k block, then the "
                      f"int8-nk linear to C fp32 [{M},{N}] (W ~N(0,0.02), per-channel int8), inputs "
                      "resident in HBM"),
         "model": "single linear (MLP up-proj shape)", "global_batch": M, "seq_len": 1,
         "parallelism": "single GPU", "two_calls_ms": round(ms_pair, 5),
         "quantize_ms": round(ms_quant, 5), "linear_rowmajor_ms": round(ms_gemm_rm, 5),
         "linear_tiled_ms": round(ms_gemm, 5)},
        {"bound": "hbm", "kernel": f"gemm16 store, tile-major codes (M={M}, N={N}, K={K})",
         "achieved": round(frac_gb, 1), "peak": 8000.0, "unit": "GB/s",
         "frac": round(frac_gb / 8000.0, 4),
         "traffic": residual_traffic("gemm_linear_m256_traffic.json"), "avg_ms": round(ms_gemm, 5),
         "algorithmic_bytes": gemm_bytes},
        cpu, round(wall, 3))
    w.free()
    print(json.dumps(line), flush=True)


def run_skinny(args) -> None:
    """the seven projections of a layer at M = 2 x 64, weights
    cold (28 layers of distinct weights, 440 MB, rotated so every launch streams
    its weight from HBM): in one ovh_linear_q_grouped launch per layer (value =
    weight bytes, int8 + fp32 scales, of the seven / that launch's time), and
    for comparison one ovh_linear_q per projection and the merged q/k/v and
    gate/up weights the runner launches (ovh_linear_q_sliced)."""
    import numpy as np
    import torch
    import ovnative_amd as ov
    M, L = 128, 28
    H, QD, KVD, I = CFG["hidden"], CFG["n_heads"] * CFG["head_dim"], \
        CFG["n_kv_heads"] * CFG["head_dim"], CFG["inter"]
    shapes = [("q", QD, H), ("k", KVD, H), ("v", KVD, H), ("o", H, QD), ("gate", I, H),
              ("up", I, H), ("down", H, I)]
    # the calibration the HBM byte counters of a PMC run are scaled by (a
    # 64 MiB device copy), untimed
    counter_calibration()
    g = torch.Generator(device="cuda").manual_seed(3)
    layers, host0 = [], None
    for li in range(L):
        ws = []
        for name, n, k in shapes:
            q = torch.randint(-127, 128, (n, k), generator=g, device="cuda", dtype=torch.int8)
            s = torch.rand(n, generator=g, device="cuda") * 1e-3 + 1e-4
            ws.append(ov.Weight.from_device(q, s))
            if li == 0:
                host0 = (host0 or []) + [(q.cpu().numpy(), s.cpu().numpy())]
        ws.append(ov.Weight.concat(ws[0:3]))   # merged q/k/v, as the runner holds it
        ws.append(ov.Weight.concat(ws[4:6]))   # merged gate/up
        layers.append(ws)
    A = {k: torch.randn((M, k), generator=g, device="cuda") for k in (H, QD, I)}
    acts = {k: ov.s8_nk_quantize(a) for k, a in A.items()}
    outs = {n: torch.zeros((M, n), device="cuda") for n in (QD, KVD, H, I)}
    lib = ov.load()
    st = torch.cuda.current_stream().cuda_stream
    import ctypes as C
    qkv_n = (C.c_int64 * 3)(QD, KVD, KVD)
    qkv_c = (C.c_void_p * 3)(outs[QD].data_ptr(), outs[KVD].data_ptr(), outs[KVD].data_ptr())
    gu_n = (C.c_int64 * 2)(I, I)
    gu_c = (C.c_void_p * 2)(outs[I].data_ptr(), outs[I].data_ptr())

    grp = (ov.GemmGroup * 7)()
    lib_grouped = lib.ovh_linear_q_grouped

    def call(j, ws):
        if j == 9:  # the seven in one grouped launch
            for i, (name, n, k) in enumerate(shapes):
                aq, asc = acts[k]
                grp[i] = ov.GemmGroup(M, aq.data_ptr(), asc.data_ptr(), ws[i].handle.value,
                                      outs_g[i].data_ptr(), n)
            return lib_grouped(grp, 7, 0, st)
        if j < 7:
            name, n, k = shapes[j]
            aq, asc = acts[k]
            return lib.ovh_linear_q(M, aq.data_ptr(), asc.data_ptr(), ws[j].handle,
                                    outs[n].data_ptr(), n, 0, st)
        aq, asc = acts[H]
        if j == 7:
            return lib.ovh_linear_q_sliced(M, aq.data_ptr(), asc.data_ptr(), ws[7].handle, qkv_n,
                                           qkv_c, 3, st)
        return lib.ovh_linear_q_sliced(M, aq.data_ptr(), asc.data_ptr(), ws[8].handle, gu_n,
                                       gu_c, 2, st)

    outs_g = [torch.zeros((M, n), device="cuda") for _, n, _ in shapes]
    for ws in layers:
        for j in range(10):
            if call(j, ws) != 0:
                raise RuntimeError("C ABI call failed")
    torch.cuda.synchronize()
    for i, (name, n, k) in enumerate(shapes):  # the grouped launch == the separate ones
        call(i, layers[-1])
        call(9, layers[-1])
        torch.cuda.synchronize()
        if not torch.equal(outs_g[i], outs[n]):
            raise RuntimeError(f"grouped GEMM differs from ovh_linear_q for {name}")
    t0 = time.perf_counter()
    per = {}
    names = [s[0] for s in shapes] + ["qkv (merged)", "gate/up (merged)", "grouped (seven)"]
    wbytes = [n * k + 4 * n for _, n, k in shapes]
    wbytes += [sum(wbytes[0:3]), sum(wbytes[4:6]), sum(wbytes[0:7])]
    for j, nm in enumerate(names):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for ws in layers:
            call(j, ws)
        e1.record()
        torch.cuda.synchronize()
        per[nm] = e0.elapsed_time(e1) / L
    wall = time.perf_counter() - t0
    seven_ms = sum(per[s[0]] for s in shapes)
    seven_b = sum(wbytes[:7])
    merged_ms = per["qkv (merged)"] + per["o"] + per["gate/up (merged)"] + per["down"]
    grouped_ms = per["grouped (seven)"]
    gbs = seven_b / grouped_ms / 1e6
    # algorithmic bytes of the grouped launch: the weights, each distinct
    # activation's codes and block scales once, the fp32 outputs
    alg_b = seven_b + sum(M * k + 4 * M * (k // 32) for k in (H, QD, I)) + \
        sum(4 * M * n for _, n, _ in shapes)
    for j, nm in enumerate(names):
        log(f"config 2: {nm:17s} {per[nm] * 1e3:7.2f} us  {wbytes[j] / per[nm] / 1e6:7.1f} GB/s")
    log(f"config 2: seven projections one launch each {seven_ms * 1e3:.1f} us = "
        f"{seven_b / seven_ms / 1e6:.0f} GB/s; runner's four launches (qkv, o, gate/up, down) "
        f"{merged_ms * 1e3:.1f} us = {seven_b / merged_ms / 1e6:.0f} GB/s; one grouped launch "
        f"{grouped_ms * 1e3:.1f} us = {gbs:.0f} GB/s")
    for ws in layers:
        for w in ws:
            w.free()
    ops = sum(2 * M * n * k for _, n, k in shapes)
    cpu = None
    if not args.no_cpu:
        import oracle
        impl, kind = None, None
        if oracle.reference_available():
            try:
                r = oracle.Reference()
                if r.vnni_available():
                    impl, kind = r, "reference"
            except OSError:
                impl = None
        if impl is None:
            o = oracle.Oracle()
            if o.fast_available():
                impl, kind = o, "port"
        if impl is not None:
            packs = [impl.pack(q) for q, _ in host0]
            hacts = {k: impl.quantize(a.cpu().numpy()) for k, a in A.items()}
            houts = [np.zeros((M, n), np.float32) for _, n, _ in shapes]

            def layer():
                for j, (name, n, k) in enumerate(shapes):
                    aq, asc = hacts[k]
                    impl.linear_q_packed(aq, asc, packs[j][0], packs[j][1], n, k, host0[j][1],
                                         houts[j])
            layer()
            times = []
            t_end = time.perf_counter() + min(args.cpu_seconds, 10.0)
            while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 200):
                t1 = time.perf_counter()
                layer()
                times.append(time.perf_counter() - t1)
            sec = statistics.median(times)
            cpu = {"value": round(seven_b / sec / 1e9, 2), "unit": "GB/s",
                   "cores": oracle.Oracle().num_threads(), "host": host_cpu(), "kind": kind,
                   "sample": (f"linear_s8_nk_packed_q of the seven projections at M={M} "
                              f"({'reference gemm.cpp' if kind == 'reference' else 'oracle restatement'}"
                              f", one layer's weights, warm in the host caches), median of "
                              f"{len(times)}: {sec * 1e3:.3f} ms = {ops / sec / 1e12:.2f} TOPS"),
                   "ms_per_step": round(sec * 1e3, 4)}
    line = bench_line(
        args, round(gbs, 1), "GB/s", round(grouped_ms, 5),
        {"workload": (f"BASELINE config 2: the seven projections of one layer at M=2x64 in one "
                      f"ovh_linear_q_grouped launch, weights cold from HBM ({L} layers rotated, "
                      f"{L * seven_b / 1e6:.0f} MB); value = weight bytes / launch time"),
         "model": "Qwen3-0.6B-shaped layer projections", "global_batch": 2, "seq_len": 64,
         "parallelism": "single GPU",
         "per_projection_us": {nm: round(per[nm] * 1e3, 2) for nm in names},
         "separate_launches_us": round(seven_ms * 1e3, 2),
         "separate_launches_gbs": round(seven_b / seven_ms / 1e6, 1),
         "runner_launches_us": round(merged_ms * 1e3, 2),
         "runner_launches_gbs": round(seven_b / merged_ms / 1e6, 1)},
        {"bound": "hbm", "kernel": (f"skinny_grouped_kernel store, seven projections in one "
                                    f"launch (M={M}, weights cold); achieved = algorithmic "
                                    f"bytes (weights, codes and scales of the three "
                                    f"activations, fp32 outputs) / launch time"),
         "achieved": round(alg_b / grouped_ms / 1e6, 1), "peak": 8000.0, "unit": "GB/s",
         "frac": round(alg_b / grouped_ms / 1e6 / 8000.0, 4),
         "traffic": residual_traffic("gemm_grouped_m128_traffic.json"),
         "algorithmic_bytes": alg_b, "avg_ms": round(grouped_ms, 5)},
        cpu, round(wall, 3))
    print(json.dumps(line), flush=True)


def run_layer(args) -> None:
    """one decoder layer at M = 2 x 300 (the config-4 CFG batch),
    measured as the difference of the runner's forward at 2 layers and at 1 layer
    (same embedding, final norm and head on both sides), with the reference's
    LM::forward timed the same way on the host."""
    import torch
    import ovnative_amd as ov
    cfg2 = dict(CFG, n_layers=2)
    cfg1 = dict(CFG, n_layers=1)
    t_setup = time.perf_counter()
    tensors = make_checkpoint(cfg2)
    ids, am, attn, pos, _ = make_inputs(cfg2)
    log(f"checkpoint {time.perf_counter() - t_setup:.1f}s")
    t0 = time.perf_counter()
    ms = {}
    for n, cfg in ((1, cfg1), (2, cfg2)):
        lm = ov.LM.from_tensors(tensors, ov.LmConfig(**cfg))
        for _ in range(max(args.warmup, 3)):
            lm.forward(ids, am, attn, pos, host_logits=False)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = max(args.steps, 50)
        e0.record()
        for _ in range(reps):
            lm.forward(ids, am, attn, pos, host_logits=False)
        e1.record()
        torch.cuda.synchronize()
        ms[n] = e0.elapsed_time(e1) / reps
        lm.close()
    wall = time.perf_counter() - t0
    M = SEQ * CFG_BATCH
    layer_ms = ms[2] - ms[1]
    layer_ops = linear_ops(cfg1, M, 1) - linear_ops(cfg1, M, 0)
    tops = layer_ops / (layer_ms * 1e-3) / 1e12
    log(f"config 3: forward 1 layer {ms[1]:.3f} ms, 2 layers {ms[2]:.3f} ms -> layer "
        f"{layer_ms * 1e3:.1f} us ({tops:.1f} linear TOPS)")
    rs = time_residual(CFG, 1, M, reps=16, norm=True)
    cpu = None
    if not args.no_cpu:
        import oracle
        if oracle.reference_available():
            try:
                ref = oracle.Reference()
                ref = ref if ref.vnni_available() else None
            except OSError:
                ref = None
            if ref is not None:
                from ovnative_amd import ovw1
                sec = {}
                with tempfile.TemporaryDirectory() as d:
                    path = os.path.join(d, "lm.ovw")
                    ovw1.write(path, tensors)
                    for n, cfg in ((1, cfg1), (2, cfg2)):
                        h = ref.lm_open(path, cfg)
                        try:
                            ref.lm_forward(h, cfg, ids, am, attn, pos)
                            times = []
                            t_end = time.perf_counter() + args.cpu_seconds / 2
                            while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 30):
                                t1 = time.perf_counter()
                                ref.lm_forward(h, cfg, ids, am, attn, pos)
                                times.append(time.perf_counter() - t1)
                        finally:
                            ref.lm_close(h)
                        sec[n] = (statistics.median(times), len(times))
                layer_s = sec[2][0] - sec[1][0]
                cpu = {"value": round(layer_ops / layer_s / 1e12, 4), "unit": "TOPS",
                       "cores": oracle.Oracle().num_threads(), "host": host_cpu(), "kind": "reference",
                       "sample": (f"reference LM::forward at 2 layers (median of {sec[2][1]}) minus "
                                  f"1 layer (median of {sec[1][1]}), B=2, S={SEQ}"),
                       "ms_per_step": round(layer_s * 1e3, 3)}
    line = bench_line(
        args, round(tops, 2), "TOPS", round(layer_ms, 5),
        {"workload": (f"BASELINE config 3: one Qwen3-0.6B-shaped decoder layer at M=2x{SEQ} (the "
                      "config-4 CFG batch): RMSNorm+quant, merged q/k/v, qk-norm+RoPE, GQA "
                      "attention (split-f16), o_proj (+= x) with the next RMSNorm+quant in the "
                      "same launch, gate/up+SiLU, down (+= x) with the next layer's "
                      "RMSNorm+quant; runner forward at 2 layers minus 1 layer"),
         "model": "one decoder layer (hidden 1024, 16/8 heads x 128, inter 3072)",
         "global_batch": CFG_BATCH, "seq_len": SEQ, "parallelism": "single GPU",
         "layer_linear_gop": round(layer_ops / 1e9, 3),
         "forward_1_layer_ms": round(ms[1], 4), "forward_2_layers_ms": round(ms[2], 4)},
        roofline_entry(f"gemm16 residual + norm (o_proj K=2048 and down K=3072; M={M}, N=1024, "
                       "+= x, then RMSNorm + quantise of the updated rows in the same launch; "
                       "one layer's weights, cache-hot as in this workload; graph replay, "
                       "tile-major codes)", rs["ops"], residual_bytes(CFG, M) + norm_out_bytes(CFG, M),
                       rs["graph_norm_ms"], avg_ms_plain_residual=round(rs["graph_ms"], 5),
                       avg_ms_plain_residual_eager_rowmajor=round(rs["eager_ms"], 5)),
        cpu, round(wall, 3))
    print(json.dumps(line), flush=True)


def run_m16384(args, cfg: dict, tensors) -> None:
    """8 concurrent requests x CFG 2 x seq 1024 (M = 16384)
    through the 28-layer LM; one step = one forward (logits left on the device)."""
    import torch
    import ovnative_amd as ov
    requests, seq = 8, 1024
    batch = make_requests(cfg, requests, seq)
    ids, am, attn, pos = batch
    B = 2 * requests
    M = B * seq
    lm = ov.LM.from_tensors(tensors, ov.LmConfig(**cfg))
    lm.set_device_sampling(True)

    def timed(steps):
        for _ in range(args.warmup):
            lm.forward(ids, am, attn, pos, host_logits=False)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            lm.forward(ids, am, attn, pos, host_logits=False)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps, time.perf_counter() - t0

    ms_step, wall = timed(args.steps)
    ops = linear_ops(cfg, M, args.layers)
    tops = ops / (ms_step * 1e-3) / 1e12
    log(f"M={M} forward {ms_step:.2f} ms ({tops:.1f} linear TOPS)")
    # the opt-in f16-operand GEMM form on the same forward (same logits bit for bit)
    prev = ov.set_f16_min_rows(2048)
    try:
        ms_f16, _ = timed(max(1, args.steps // 2))
    finally:
        ov.set_f16_min_rows(prev)
    lm.close()
    log(f"M={M} forward with the f16 GEMM form {ms_f16:.2f} ms "
        f"({ops / (ms_f16 * 1e-3) / 1e12:.1f} linear TOPS)")
    rs = time_residual(cfg, args.layers, M, reps=1)
    cpu = None if args.no_cpu else cpu_baseline(cfg, tensors, args.cpu_seconds, batch)
    line = {
        "metric": "int8 linear TOPS & % roofline; LM ms/step (seq 300, CFG batch 2)",
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": (f"BASELINE config 5: one forward of the {args.layers}-layer LM over "
                         f"{requests} requests x CFG 2 x seq {seq} (M={M}; each request the "
                         "tts.cpp cond/uncond pair), logits left on the device"),
            "model": "Qwen3-0.6B-shaped LM (hidden 1024, 16/8 heads x 128, inter 3072, 28 layers)",
            "global_batch": B,
            "seq_len": seq,
            "parallelism": "single GPU",
            "step_linear_gop": round(ops / 1e9, 2),
            "step_attention_gflop": round(attention_flops(cfg, seq, B, args.layers) / 1e9, 2),
            "f16_gemm_form": {"ms_per_step": round(ms_f16, 4),
                              "linear_tops": round(ops / (ms_f16 * 1e-3) / 1e12, 2),
                              "note": "ovh_set_f16_min_rows(2048): int8-valued f16 operands, "
                                      "same logits; off by default"},
        },
        "roofline": roofline_entry(
            f"gemm16 residual (o_proj K=2048 and down K=3072; M={M}, N=1024, += x; graph "
            "replay, tile-major codes)", rs["ops"], residual_bytes(cfg, M), rs["graph_ms"],
            avg_ms_eager_rowmajor=round(rs["eager_ms"], 5)),
        "cpu_baseline": cpu,
        "wall_s": round(wall, 3),
    }
    print(json.dumps(line), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is designed, not launched, in this build.", file=sys.stderr)
        sys.exit(2)
    import torch
    import ovnative_amd as ov
    ov.load()
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    if args.workload == "linear":
        run_linear(args)
        return
    if args.workload == "layer":
        run_layer(args)
        return
    if args.workload == "skinny":
        run_skinny(args)
        return
    if args.workload == "residual":
        run_residual(args)
        return
    cfg = dict(CFG, n_layers=args.layers)
    M = SEQ * CFG_BATCH
    t_setup = time.perf_counter()
    tensors = make_checkpoint(cfg)
    if args.workload == "m16384":
        run_m16384(args, cfg, tensors)
        return
    step = LmStep(cfg, tensors)
    log(f"checkpoint + upload {time.perf_counter() - t_setup:.1f}s")
    for _ in range(args.warmup):
        step.run()
    torch.cuda.synchronize()

    t0 = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step.run()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = e0.elapsed_time(e1) / args.steps
    ops = linear_ops(cfg, M, args.layers)
    tops = ops / (ms_step * 1e-3) / 1e12
    log(f"LM step {ms_step:.3f} ms ({tops:.1f} linear TOPS)")

    # BASELINE config 4's second figure: the end-to-end LM time of a 32-step
    # decode (ovh_lm_generate = tts.cpp's run_sampling on the device runner:
    # forwards, device sampling, host Gumbel/top-k, id updates), wall clock.
    import ovnative_amd as ov
    T = SEQ - TEXT
    prompt = step.ids[0].copy()
    prompt[:, TEXT:] = cfg["audio_vocab"] - 1
    amask = step.am[0].copy()
    opts = ov.GenOptions(num_steps=32)
    step.lm.generate(prompt, amask, T, opts)          # warm-up (tables, arena)
    torch.cuda.synchronize()
    t_gen = time.perf_counter()
    step.lm.generate(prompt, amask, T, opts)
    gen_ms = (time.perf_counter() - t_gen) * 1e3
    log(f"32-step decode {gen_ms:.1f} ms")

    rs = time_residual(cfg, args.layers, M, norm=True)
    step.lm.close()

    cpu = None if args.no_cpu else cpu_baseline(cfg, tensors, args.cpu_seconds)

    line = {
        "metric": "int8 linear TOPS & % roofline; LM ms/step (seq 300, CFG batch 2)",
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": (f"one CFG decoding step of the {args.layers}-layer LM: forward at B=2, "
                         f"S={SEQ} ({TEXT} text + {SEQ - TEXT} audio; uncond = target slice), "
                         "int8-nk linears, GQA attention (split-f16 matrix-core products, fp32 "
                         "softmax), head 1024->8x1025, device guided sampling"),
            "model": "Qwen3-0.6B-shaped LM (hidden 1024, 16/8 heads x 128, inter 3072, 28 layers)",
            "global_batch": CFG_BATCH,
            "seq_len": SEQ,
            "parallelism": "single GPU",
            "step_linear_gop": round(ops / 1e9, 2),
            "step_attention_gflop": round(attention_flops(cfg, SEQ, CFG_BATCH, args.layers) / 1e9, 2),
            "lm_32_steps_ms": round(gen_ms, 2),
            "lm_32_steps_note": "ovh_lm_generate wall clock: 32 forwards + device sampling + host top-k",
        },
        "roofline": roofline_entry(
            "gemm16 residual + norm (o_proj K=2048 and down K=3072; M=600, N=1024, += x, then "
            "RMSNorm + quantise of the updated rows in the same launch), launched as the step "
            "launches it: graph replay, tile-major codes, weights cold from HBM (as the step's "
            "down launches read theirs; its o_proj launches find their weight prefetched into "
            "L2 by the attention launch and run ~2.5 us shorter)",
            rs["ops"], residual_bytes(cfg, M) + norm_out_bytes(cfg, M), rs["graph_norm_ms"],
            residual_traffic(NORM_TRAFFIC),
            avg_ms_plain_residual=round(rs["graph_ms"], 5),
            avg_ms_plain_residual_eager_rowmajor=round(rs["eager_ms"], 5)),
        "cpu_baseline": cpu,
        "wall_s": round(wall, 3),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
