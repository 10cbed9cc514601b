#!/usr/bin/env python3
"""Benchmark of the int8-nk quantized-linear path on one MI355X.

Workload (the one the metric is quoted on): the
28-layer Qwen3-0.6B-shaped LM at seq 300, CFG batch 2 (M = 600 rows), one step
= every int8 linear of one LM forward with its fused activation quantisers, in
the order LM::run_layer issues them (cpp/src/model/lm.cpp:217-322):

    rmsnorm+quant -> qkv (merged, sliced)     -> quant(attn) -> o_proj (+= x)
    rmsnorm+quant -> gate/up (merged, sliced) -> silu*up+quant -> down (+= x)

then the final rmsnorm+quant and the int8 audio head (1024 -> 8192).  The
attention core between qkv and o_proj is not part of this path yet: o_proj
reads the q projection in its place.  28 distinct layers of random int8 weights
(~N(0, 0.02), per-channel scales; 440 MB, more than the 256 MB MALL) are
resident in HBM before timing starts; activations are synthetic ~N(0, 1).

value   = int8 linear throughput of the whole step, TOPS (2*M*N*K summed over
          every linear, divided by the measured step time);
roofline = the dominant kernel (merged gate/up GEMM, M=600 N=6144 K=1024),
          timed with HIP events on the stream it runs on, against the dense
          int8 MFMA peak;
cpu_baseline = the same step on the host's cores through the reference's own
          compiled int8-nk kernels (oracle/_ref) when its AVX-VNNI dispatch is
          available there, else through the oracle's AVX-512 VNNI port.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

H, QD, KVD, INTER, LAYERS, HEAD_N = 1024, 2048, 1024, 3072, 28, 8192
SEQ, CFG_BATCH = 300, 2
M_DEFAULT = SEQ * CFG_BATCH
PEAK_INT8_TOPS = 5000.0
PEAK_HBM_GBS = 8000.0


def step_linear_ops(M: int, layers: int = LAYERS) -> int:
    per_layer = 2 * M * (H * (QD + 2 * KVD) + QD * H + H * 2 * INTER + INTER * H)
    return layers * per_layer + 2 * M * H * HEAD_N


def gate_up_traffic():
    """HBM bytes per launch of the merged gate/up GEMM, from the committed PMC
    summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration)."""
    path = os.path.join(ROOT, "profiles", "gemm_gate_up_m600_traffic.json")
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
    p.add_argument("--m", type=int, default=M_DEFAULT, help="rows (CFG batch x seq)")
    p.add_argument("--layers", type=int, default=LAYERS)
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="wall-clock budget of the CPU-baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    return p.parse_args()


# ---------------------------------------------------------------------------
# GPU step

class GpuStep:
    def __init__(self, M: int, layers: int, seed: int = 0):
        import torch
        import ovnative_amd as ov
        self.ov, self.torch, self.M, self.layers = ov, torch, M, layers
        g = torch.Generator(device="cuda").manual_seed(seed)
        dev = "cuda"

        def qweight(N, K):
            w = torch.randn((N, K), generator=g, device=dev) * 0.02
            s = (w.abs().amax(dim=1) / 127.0).clamp_min(1e-12)
            q = torch.clamp(torch.round(w / s[:, None]), -127, 127).to(torch.int8)
            return ov.Weight.from_device(q.contiguous(), s.contiguous().float(), layout=0)

        self.L = []
        for _ in range(layers):
            q_, k_, v_ = qweight(QD, H), qweight(KVD, H), qweight(KVD, H)
            gate, up = qweight(INTER, H), qweight(INTER, H)
            layer = {
                "qkv": ov.Weight.concat([q_, k_, v_]),
                "o": qweight(H, QD),
                "gate_up": ov.Weight.concat([gate, up]),
                "down": qweight(H, INTER),
                "ln1": (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).contiguous(),
                "ln2": (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).contiguous(),
            }
            for w in (q_, k_, v_, gate, up):
                w.free()
            self.L.append(layer)
        self.head = qweight(HEAD_N, H)
        self.final_ln = torch.ones(H, device=dev)
        torch.cuda.synchronize()

        e = lambda *s, dt=torch.float32: torch.empty(s, dtype=dt, device=dev)  # noqa: E731
        self.x0 = torch.randn((M, H), generator=g, device=dev)
        self.x = e(M, H)
        self.aq_h, self.asc_h = e(M, H, dt=torch.int8), e(M, H // 32)
        self.aq_o, self.asc_o = e(M, QD, dt=torch.int8), e(M, QD // 32)
        self.aq_d, self.asc_d = e(M, INTER, dt=torch.int8), e(M, INTER // 32)
        self.q, self.k, self.v = e(M, QD), e(M, KVD), e(M, KVD)
        self.gate, self.up = e(M, INTER), e(M, INTER)
        self.logits = e(M, HEAD_N)

    def time_gate_up(self, reps: int = 4) -> float:
        """Average duration (ms) of the dominant kernel, the merged gate/up GEMM:
        reps x layers back-to-back launches (each layer's own weights, as in the
        step) between one pair of HIP events on the stream they run on."""
        ov, torch = self.ov, self.torch
        ov.rmsnorm_quantize(self.x0, self.L[0]["ln2"], 1e-6, out=(self.aq_h, self.asc_h))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            for L in self.L:
                ov.linear_q_sliced(self.aq_h, self.asc_h, L["gate_up"], [INTER, INTER],
                                   outs=[self.gate, self.up])
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / (reps * len(self.L))

    def run(self):
        ov, torch = self.ov, self.torch
        self.x.copy_(self.x0)
        for L in self.L:
            ov.rmsnorm_quantize(self.x, L["ln1"], 1e-6, out=(self.aq_h, self.asc_h))
            ov.linear_q_sliced(self.aq_h, self.asc_h, L["qkv"], [QD, KVD, KVD],
                               outs=[self.q, self.k, self.v])
            ov.s8_nk_quantize(self.q, out=(self.aq_o, self.asc_o))  # attention output stand-in
            ov.linear_q(self.aq_o, self.asc_o, L["o"], self.x, accumulate=True)
            ov.rmsnorm_quantize(self.x, L["ln2"], 1e-6, out=(self.aq_h, self.asc_h))
            ov.linear_q_sliced(self.aq_h, self.asc_h, L["gate_up"], [INTER, INTER],
                               outs=[self.gate, self.up])
            ov.silu_mul_quantize(self.gate, self.up, out=(self.aq_d, self.asc_d))
            ov.linear_q(self.aq_d, self.asc_d, L["down"], self.x, accumulate=True)
        ov.rmsnorm_quantize(self.x, self.final_ln, 1e-6, out=(self.aq_h, self.asc_h))
        ov.linear_q(self.aq_h, self.asc_h, self.head, self.logits)


# ---------------------------------------------------------------------------
# CPU baseline (reported beside the GPU, not optimised)

def cpu_baseline(M: int, layers: int, budget_s: float):
    import numpy as np
    import oracle
    from oracle import Oracle

    rng = np.random.default_rng(0)

    def qw(N, K):
        return (rng.integers(-127, 128, (N, K), dtype=np.int8),
                rng.uniform(1e-4, 1e-3, N).astype(np.float32))

    ref = None
    if oracle.reference_available():
        try:
            r = oracle.Reference()
            if r.vnni_available():
                ref = r
        except OSError:
            ref = None
    orc = Oracle()
    if ref is None and not orc.fast_available():
        return None
    kind = "reference" if ref is not None else "port"
    impl = ref if ref is not None else orc

    # The sample: `nl` layers of the same step (every projection and quantiser of
    # a layer), weights packed once outside the timed region like the reference's
    # load-time s8_nk_pack.
    nl = min(layers, 4)
    packs = []
    for _ in range(nl):
        L = {}
        for name, (N, K) in (("q", (QD, H)), ("k", (KVD, H)), ("v", (KVD, H)), ("o", (H, QD)),
                             ("gate", (INTER, H)), ("up", (INTER, H)), ("down", (H, INTER))):
            q, s = qw(N, K)
            L[name] = (impl.pack(q), N, K, s)
        L["ln1"] = rng.uniform(0.5, 1.5, H).astype(np.float32)
        L["ln2"] = rng.uniform(0.5, 1.5, H).astype(np.float32)
        packs.append(L)
    x0 = rng.standard_normal((M, H)).astype(np.float32)

    def lin(aq, asc, ent, C, acc):
        (packed, wsum), N, K, s = ent
        impl.linear_q_packed(aq, asc, packed, wsum, N, K, s, C, accumulate=acc)

    def run_layers():
        x = x0.copy()
        for L in packs:
            aq, asc = impl.rmsnorm_quantize(x, L["ln1"], 1e-6)
            q = np.zeros((M, QD), np.float32)
            k = np.zeros((M, KVD), np.float32)
            v = np.zeros((M, KVD), np.float32)
            lin(aq, asc, L["q"], q, False)
            lin(aq, asc, L["k"], k, False)
            lin(aq, asc, L["v"], v, False)
            aqo, asco = impl.quantize(q)
            lin(aqo, asco, L["o"], x, True)
            aq, asc = impl.rmsnorm_quantize(x, L["ln2"], 1e-6)
            gate = np.zeros((M, INTER), np.float32)
            up = np.zeros((M, INTER), np.float32)
            lin(aq, asc, L["gate"], gate, False)
            lin(aq, asc, L["up"], up, False)
            aqd, ascd = impl.silu_mul_quantize(gate, up)
            lin(aqd, ascd, L["down"], x, True)
        return x

    run_layers()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        run_layers()
        times.append(time.perf_counter() - t0)
    per_layer_s = statistics.median(times) / nl
    ops_layer = step_linear_ops(M, 1) - 2 * M * H * HEAD_N
    cores = orc.num_threads()
    return {
        "value": round(ops_layer / per_layer_s / 1e12, 4),
        "unit": "TOPS",
        "cores": cores,
        "kind": kind,
        "sample": (f"{nl} decoder layers' int8 linears + quantisers at M={M} "
                   f"(median of {len(times)} reps, {ops_layer * nl / 1e9:.1f} GOP each); "
                   f"ms/layer {per_layer_s * 1e3:.2f}; "
                   f"{'reference gemm.cpp VNNI kernels' if kind == 'reference' else 'oracle AVX-512 VNNI port'}"),
        "ms_per_layer": round(per_layer_s * 1e3, 3),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is described in DESIGN.md, not launched.", file=sys.stderr)
        sys.exit(2)
    import torch
    import ovnative_amd as ov
    ov.load()
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    M = args.m
    step = GpuStep(M, args.layers)
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
    ops = step_linear_ops(M, args.layers)
    tops = ops / (ms_step * 1e-3) / 1e12

    gu_ms = step.time_gate_up()
    gu_ops = 2 * M * (2 * INTER) * H
    gu_tops = gu_ops / (gu_ms * 1e-3) / 1e12

    cpu = None if args.no_cpu else cpu_baseline(M, args.layers, args.cpu_seconds)

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
            "workload": (f"LM int8-linear step: {args.layers} layers x (qkv, o, gate/up, down) + "
                         f"head 1024->{HEAD_N}, M={M} (seq {SEQ} x CFG batch {CFG_BATCH}), "
                         "fused rmsnorm/silu quantisers; attention core not included"),
            "model": "Qwen3-0.6B-shaped LM (hidden 1024, 16/8 heads, inter 3072)",
            "global_batch": CFG_BATCH,
            "seq_len": SEQ,
            "parallelism": "single GPU",
            "step_gop": round(ops / 1e9, 2),
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "gemm_i8 gate/up merged (M=600, N=6144, K=1024)",
            "achieved": round(gu_tops, 2),
            "peak": PEAK_INT8_TOPS,
            "unit": "TFLOP/s",
            "frac": round(gu_tops / PEAK_INT8_TOPS, 4),
            "traffic": gate_up_traffic(),
            "avg_ms": round(gu_ms, 5),
        },
        "cpu_baseline": cpu,
        "wall_s": round(wall, 3),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
