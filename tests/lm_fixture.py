"""Random LM checkpoints for the tests: the reference's tensor names and
encodings (tools/convert_weights.py: int8 linears per output channel in the nk
or kn layout, int8 embedding tables with per-row scales, fp32 norms), with
weights ~N(0, 0.02) and norm weights near 1."""
from __future__ import annotations

import numpy as np

from ovnative_amd import ovw1

SMALL = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=128, inter=512,
             vocab=300, audio_vocab=33, n_codebooks=8, rms_eps=1e-6, rope_theta=1e6)
# One decoder layer at the LM's real widths with the real
# 8 x 1025 audio head; the text table is cut to 2048 rows (it only has to hold
# the mask id the unconditional row carries in its text slots).
FULL1 = dict(n_layers=1, hidden=1024, n_heads=16, n_kv_heads=8, head_dim=128, inter=3072,
             vocab=2048, audio_vocab=1025, n_codebooks=8, rms_eps=1e-6, rope_theta=1e6)
# all 28 layers at the real widths (440 MB of int8 weights).
FULL28 = dict(FULL1, n_layers=28)


def make_lm(seed: int, cfg: dict, layout: str = "nk", emb_int8: bool = True,
            head_fp32: bool = False):
    """Returns (tensors for ovw1.write / views, {name: (array, scales, transposed)}).
    head_fp32: the audio head stays fp32, stored [K, N], as the reference's
    default int8 checkpoint keeps it (tools/convert_weights.py --int8-keep)."""
    rng = np.random.default_rng(seed)
    H, NH, NKV, D, I = cfg["hidden"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["inter"]
    Cb, V = cfg["n_codebooks"], cfg["audio_vocab"]
    ts = []

    def lin(name, n, k):
        ts.append(ovw1.linear_int8(name, (rng.standard_normal((n, k)) * 0.02).astype(np.float32),
                                   layout))

    def norm(name, n):
        ts.append(ovw1.Tensor(name, rng.uniform(0.8, 1.2, n).astype(np.float32)))

    def emb(name, rows):
        w = (rng.standard_normal((rows, H)) * 0.02).astype(np.float32)
        if emb_int8:
            q, s = ovw1.quantize_int8(w)
            ts.append(ovw1.Tensor(name, q, 0, s))
        else:
            ts.append(ovw1.Tensor(name, w))

    emb("llm.embed_tokens.weight", cfg["vocab"])
    emb("audio_embeddings.weight", Cb * V)
    if head_fp32:
        w = (rng.standard_normal((Cb * V, H)) * 0.02).astype(np.float32)
        ts.append(ovw1.Tensor("audio_heads.weight", np.ascontiguousarray(w.T), 1))
    else:
        lin("audio_heads.weight", Cb * V, H)
    norm("llm.norm.weight", H)
    ts.append(ovw1.Tensor("codebook_layer_offsets", np.arange(Cb, dtype=np.int64) * V))
    for i in range(cfg["n_layers"]):
        p = f"llm.layers.{i}."
        norm(p + "input_layernorm.weight", H)
        norm(p + "post_attention_layernorm.weight", H)
        norm(p + "self_attn.q_norm.weight", D)
        norm(p + "self_attn.k_norm.weight", D)
        lin(p + "self_attn.q_proj.weight", NH * D, H)
        lin(p + "self_attn.k_proj.weight", NKV * D, H)
        lin(p + "self_attn.v_proj.weight", NKV * D, H)
        lin(p + "self_attn.o_proj.weight", H, NH * D)
        lin(p + "mlp.gate_proj.weight", I, H)
        lin(p + "mlp.up_proj.weight", I, H)
        lin(p + "mlp.down_proj.weight", H, I)
    table = {t.name: (t.array, t.scales, t.layout == 1) for t in ts}
    return ts, table


def make_inputs(seed: int, cfg: dict, batch: int, seq: int, text: int):
    """A CFG-style batch like tts.cpp:175-213 builds: `text` text positions then
    audio positions in row 0; row 1 holds only the target audio (attends within
    its first seq - text positions, diagonal for the tail)."""
    rng = np.random.default_rng(seed)
    Cb, V = cfg["n_codebooks"], cfg["audio_vocab"]
    ids = rng.integers(0, V - 1, (batch, Cb, seq)).astype(np.int64)
    ids[:, 0, :text] = rng.integers(0, cfg["vocab"], (batch, text))
    amask = np.zeros((batch, seq), np.uint8)
    amask[:, text:] = 1
    attn = np.ones((batch, seq, seq), np.uint8)
    if batch > 1:
        # row 1: the target slice of row 0 in its first T positions, the mask
        # token elsewhere (tts.cpp:190-198)
        T = seq - text
        ids[1] = V - 1
        ids[1, :, :T] = ids[0, :, text:]
        attn[1] = 0
        attn[1, :T, :T] = 1
        attn[1, np.arange(T, seq), np.arange(T, seq)] = 1
        amask[1] = 0
        amask[1, :T] = 1
    pos = np.tile(np.arange(seq, dtype=np.int64), (batch, 1))
    return ids, amask, attn, pos


# A hand-worked case of the guided sampling pass (tts.cpp:296-326, the device
# form of cuda_lm.cu:679-758): V = 4 (token 3 is the mask token), 2 codebooks,
# one frame, guidance g = 2, layer penalty 5.  With lc = log_softmax(cond) and
# lu = log_softmax(uncond), mix = lc + g (lc - lu) = 3 cond - 2 uncond - K (K
# a constant per row), then lp2 = log_softmax(mix), argmax over the non-mask
# tokens, score = max lp2 - c * penalty:
#   codebook 0: cond [0, 2, 1.5, 0], uncond [0, 3, 0.5, 0]: 3c - 2u = [0, 0, 3.5, 0]
#     -> token 2, score 3.5 - ln(3 + e^3.5) = -0.0867208058559692;
#   codebook 1: cond [1, 0, 0, 5], uncond [0, 0, 1, 5]: 3c - 2u = [3, 0, -2, 5]
#     -> token 0 (the mask token's 5 is excluded), score
#     3 - ln(e^3 + 1 + e^-2 + e^5) - 5 = -7.1336433595320905.
# Plausible mistakes move the answer: the guidance term's sign flipped
# (-lc + 2 lu: [0, 4, -0.5, 0] and [-1, 0, 2, 5]) picks tokens 1 and 2; no
# guidance picks token 1 in codebook 0; the mask token not excluded picks 3 in
# codebook 1; without the second log-softmax the scores are 1.9445 and
# -7.0313; the penalty on codebook 0 instead of 1 moves both scores by 5.
SAMPLER_CASE = dict(
    cond=[[0.0, 2.0, 1.5, 0.0, 1.0, 0.0, 0.0, 5.0]],      # [frames, C * V], codebook-major
    uncond=[[0.0, 3.0, 0.5, 0.0, 0.0, 0.0, 1.0, 5.0]],
    C=2, V=4, T=1, guidance=2.0, penalty=5.0,
    pred=[[2], [0]], scores=[[-0.0867208058559692], [-7.1336433595320905]])
