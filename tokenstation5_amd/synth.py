"""Seeded synthetic inputs in GGML block layouts, for the benchmark configs.

No checkpoint or dataset is reachable, so every weight is random-init with the
field distributions the benchmark configs state:

* Q4_K (144 B per 256 values): ``d``, ``dmin`` = f16(|N(0,1)| * 0.01); the 12
  packed scale/min bytes uniform (every byte pattern encodes eight 6-bit scales
  and eight 6-bit mins, so uniform bytes are uniform scales and mins in
  [0, 63]); the 128 nibble bytes uniform (quants uniform in [0, 15]).
* Q6_K (210 B): ql / qh uniform bytes, int8 sub-scales uniform, ``d`` as Q4_K's.
* Q8_0 (34 B): ``d`` as above, int8 quants uniform.
* Norm weights fp32 N(1, 0.02).

Each tensor draws from its own generator, seeded by (seed, crc32(name)), so a
tensor is the same whatever else is generated. Layouts follow
engine/src/quants.cpp:74-205 (block byte order) and engine/src/gguf.cpp:38-46
(block sizes).
"""
from __future__ import annotations

import zlib

import numpy as np

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 3, 6, 7, 8, 12, 13, 14, 30
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22),
         Q5_1: (32, 24), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}
TYPE_NAME = {F32: "F32", F16: "F16", BF16: "BF16", Q4_0: "Q4_0", Q4_1: "Q4_1", Q5_0: "Q5_0",
             Q5_1: "Q5_1", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}


def row_bytes(t: int, ne0: int) -> int:
    bv, bb = BLOCK[t]
    if ne0 % bv:
        raise ValueError(f"row of {ne0} values is not a whole number of {TYPE_NAME[t]} blocks")
    return ne0 // bv * bb


def rng_for(seed: int, name: str) -> np.random.Generator:
    return np.random.default_rng([seed, zlib.crc32(name.encode())])


def _half_bytes(v: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(v.astype(np.float16)).view(np.uint8).reshape(-1, 2)


def _scale(rng: np.random.Generator, n: int) -> np.ndarray:
    return _half_bytes(np.abs(rng.standard_normal(n)) * 0.01)


def pack_scale_min(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Eight 6-bit scales and mins per row -> the 12 packed K-quant bytes that
    engine/src/quants.cpp:64-72 unpacks (sub-blocks 0-3 in the low 6 bits of
    bytes j and j+4; 4-7 split over byte j+8's nibbles and the top bits)."""
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    out = np.empty((sc.shape[0], 12), np.uint8)
    out[:, 0:4] = sc[:, 0:4] | ((sc[:, 4:8] >> 4) << 6)
    out[:, 4:8] = m[:, 0:4] | ((m[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:8] & 15) | ((m[:, 4:8] & 15) << 4)
    return out


def blocks(t: int, n_blocks: int, rng: np.random.Generator, centered: bool = False, dscale: float = 0.01) -> np.ndarray:
    """n_blocks blocks of type t as a (n_blocks, block_bytes) uint8 array.

    centered (Q4_K only): dmin = 8 d and each min = round(7.5 scale / 8), so a
    sub-block's values centre near zero instead of near 7.5 d scale. The
    benchmark's distribution has every weight's mean far above zero, which
    makes a random model's output almost independent of its input; the
    centred variant is for parity tests whose argmax should vary with it.
    dscale (centred Q4_K only): d = f16(|N(0,1)| * dscale)."""
    bb = BLOCK[t][1]
    out = np.frombuffer(rng.bytes(n_blocks * bb), dtype=np.uint8).reshape(n_blocks, bb).copy()
    if t == Q4_K and centered:
        d = (np.abs(rng.standard_normal(n_blocks)) * dscale).astype(np.float16)
        out[:, 0:2] = np.ascontiguousarray(d).view(np.uint8).reshape(-1, 2)
        out[:, 2:4] = _half_bytes(d.astype(np.float32) * 8)
        sc = rng.integers(0, 64, size=(n_blocks, 8))
        out[:, 4:16] = pack_scale_min(sc, np.rint(sc * 7.5 / 8))
    elif t == Q4_K or t == Q5_K:
        out[:, 0:2] = _scale(rng, n_blocks)
        out[:, 2:4] = _scale(rng, n_blocks)
    elif t == Q6_K:
        out[:, 208:210] = _scale(rng, n_blocks)
    elif t in (Q8_0, Q4_0, Q5_0):
        out[:, 0:2] = _scale(rng, n_blocks)
    elif t in (Q4_1, Q5_1):
        out[:, 0:2] = _scale(rng, n_blocks)
        out[:, 2:4] = _scale(rng, n_blocks)
    elif t == F16:
        out[:] = _half_bytes(rng.standard_normal(n_blocks)).reshape(n_blocks, 2)
    elif t == F32:
        out[:] = rng.standard_normal(n_blocks).astype(np.float32).view(np.uint8).reshape(n_blocks, 4)
    return out


def tensor(t: int, ne0: int, ne1: int, seed: int, name: str, centered: bool = False,
           dscale: float = 0.01) -> np.ndarray:
    """A (ne1, row_bytes) uint8 matrix of type t: rows are output rows."""
    rb = row_bytes(t, ne0)
    bv, bb = BLOCK[t]
    b = blocks(t, ne0 // bv * ne1, rng_for(seed, name), centered, dscale)
    return b.reshape(ne1, rb)


def norm_weight(n: int, seed: int, name: str) -> np.ndarray:
    """fp32 N(1, 0.02) as raw bytes (a GGUF F32 tensor)."""
    v = (1.0 + 0.02 * rng_for(seed, name).standard_normal(n)).astype(np.float32)
    return v.view(np.uint8).reshape(1, 4 * n)


# --- models -------------------------------------------------------------------

LLAMA_8B = dict(arch="llama", n_vocab=128256, n_embd=4096, n_layer=32, n_ff=14336, n_head=32, n_head_kv=8,
                head_dim=128, rope_base=500000.0, rms_eps=1e-5, wtype=Q4_K, head_type=Q6_K, embd_type=Q4_K)

# The speculative-decoding pair (draft: 896-wide matrices in Q8_0 because 896
# is not a multiple of 256; ffn_down, 4864 wide, in Q4_K; head tied).
DRAFT_0P5B = dict(arch="qwen2", n_vocab=151936, n_embd=896, n_layer=24, n_ff=4864, n_head=14, n_head_kv=2,
                  head_dim=64, rope_base=1000000.0, rms_eps=1e-6, wtype=Q8_0, down_type=Q4_K, head_type=None,
                  embd_type=Q8_0)
TARGET_14B = dict(arch="qwen2", n_vocab=151936, n_embd=5120, n_layer=48, n_ff=13824, n_head=40, n_head_kv=8,
                  head_dim=128, rope_base=1000000.0, rms_eps=1e-6, wtype=Q4_K, head_type=Q6_K, embd_type=Q4_K)

# Small models of the same families for parity tests (CPU-oracle sized).
TINY_LLAMA = dict(arch="llama", n_vocab=1000, n_embd=512, n_layer=2, n_ff=1536, n_head=4, n_head_kv=1,
                  head_dim=128, rope_base=500000.0, rms_eps=1e-5, wtype=Q4_K, head_type=Q6_K, embd_type=Q4_K)
TINY_DRAFT = dict(arch="qwen2", n_vocab=1000, n_embd=448, n_layer=2, n_ff=768, n_head=7, n_head_kv=1,
                  head_dim=64, rope_base=1000000.0, rms_eps=1e-6, wtype=Q8_0, down_type=Q4_K, head_type=None,
                  embd_type=Q8_0)
# The same shapes with centred Q4_K weights (input-dependent argmax).
TINY_LLAMA_C = dict(TINY_LLAMA, centered=True)
TINY_DRAFT_C = dict(TINY_DRAFT, centered=True)
# Llama 3.1's RoPE: a rope_freqs.weight tensor of per-frequency divisors
# (with base 10000, so that 12-72 positions turn the slow frequencies too).
TINY_LLAMA31 = dict(TINY_LLAMA_C, rope_freqs=True, rope_base=10000.0)
# Qwen 3's layer: per-head q/k norms, neox RoPE, no biases.
TINY_QWEN3 = dict(TINY_LLAMA_C, arch="qwen3", rope_base=1000000.0, rms_eps=1e-6)
# Gemma 3's layer (engine/src/model.cpp:44-63): head_dim 256 as in its 1B-12B
# models, per-head q/k norms, norms after attention and the FFN, GELU, a
# scaled embedding, tied Q6_K head (one small block scale for every row, so
# that no row outweighs the others and the layers, not the token's own
# embedding, decide the next token); 7 layers so that layer 5 is global and
# the others slide, over an 8-key window that short sequences already cross;
# linear RoPE scaling by 8 on the global layer, as Gemma 3 4B-27B have it.
TINY_GEMMA3 = dict(arch="gemma3", n_vocab=1000, n_embd=512, n_layer=7, n_ff=1536, n_head=4, n_head_kv=1,
                   head_dim=256, rope_base=1000000.0, rms_eps=1e-6, swa_window=8, wtype=Q4_K, head_type=None,
                   embd_type=Q6_K, centered=True, embd_d=5e-6, rope_scaling_factor=8.0)


def _extra_norms(hp: dict, p: str):
    """(name, length) of a layer's per-head q/k norms (qwen3, gemma3) and
    Gemma 3's norms after attention and the FFN (engine/src/model.cpp:108-116)."""
    if hp["arch"] in ("qwen3", "gemma3"):
        yield p + "attn_q_norm.weight", hp["head_dim"]
        yield p + "attn_k_norm.weight", hp["head_dim"]
    if hp["arch"] == "gemma3":
        yield p + "post_attention_norm.weight", hp["n_embd"]
        yield p + "post_ffw_norm.weight", hp["n_embd"]


def rope_divisors(hp: dict) -> np.ndarray:
    """RoPE divisors per frequency, as Llama 3.1's GGUFs store them in
    rope_freqs.weight (1 for the fastest frequencies up to 8 for the
    slowest): here a ramp over the whole range, so that a test model's
    short sequences already feel every one."""
    n = hp.get("rope_dims", hp["head_dim"]) // 2
    return (1.0 + 7.0 * (np.arange(n) / (n - 1)) ** 2).astype(np.float32)


def model_tensors(hp: dict, seed: int):
    """GGUF tensors of a random-init model: {name: (type, ne0, ne1, (ne1, row_bytes) uint8)}.

    Names and shapes follow engine/src/model.cpp:89-119 (ne0 is the input
    width of a matrix, ne1 its output rows)."""
    E, F, H, HKV, HD, V = (hp[k] for k in ("n_embd", "n_ff", "n_head", "n_head_kv", "head_dim", "n_vocab"))
    wt = hp["wtype"]
    out = {}

    def mat(name, t, ne0, ne1):
        out[name] = (t, ne0, ne1, tensor(t, ne0, ne1, seed, name, hp.get("centered", False), hp.get("dscale", 0.01)))

    t, ne0, ne1 = hp["embd_type"], E, V
    emb = tensor(t, ne0, ne1, seed, "token_embd.weight", hp.get("centered", False), hp.get("dscale", 0.01))
    if hp.get("embd_d") and t == Q6_K:  # one block scale for every row: no row outweighs the rest as a tied head
        b = emb.reshape(-1, BLOCK[t][1])
        b[:, 208:210] = _half_bytes(np.full(b.shape[0], hp["embd_d"]))
    out["token_embd.weight"] = (t, ne0, ne1, emb)
    out["output_norm.weight"] = (F32, E, 1, norm_weight(E, seed, "output_norm.weight"))
    if hp.get("rope_freqs"):
        f = rope_divisors(hp)
        out["rope_freqs.weight"] = (F32, f.size, 1, f.view(np.uint8).reshape(1, -1))
    if hp.get("head_type") is not None:
        mat("output.weight", hp["head_type"], E, V)
    for i in range(hp["n_layer"]):
        p = f"blk.{i}."
        for name, n in _extra_norms(hp, p):
            out[name] = (F32, n, 1, norm_weight(n, seed, name))
        out[p + "attn_norm.weight"] = (F32, E, 1, norm_weight(E, seed, p + "attn_norm.weight"))
        out[p + "ffn_norm.weight"] = (F32, E, 1, norm_weight(E, seed, p + "ffn_norm.weight"))
        mat(p + "attn_q.weight", wt, E, H * HD)
        mat(p + "attn_k.weight", wt, E, HKV * HD)
        mat(p + "attn_v.weight", wt, E, HKV * HD)
        mat(p + "attn_output.weight", wt, H * HD, E)
        mat(p + "ffn_gate.weight", wt, E, F)
        mat(p + "ffn_up.weight", wt, E, F)
        mat(p + "ffn_down.weight", hp.get("down_type", wt), F, E)
    return out


def tensor_specs(hp: dict):
    """(name, type, ne0, ne1) of every tensor of a model (engine/src/model.cpp:89-119 names),
    for weights generated in HBM (ts5hip Model.synth_tensor)."""
    E, F, H, HKV, HD, V = (hp[k] for k in ("n_embd", "n_ff", "n_head", "n_head_kv", "head_dim", "n_vocab"))
    wt = hp["wtype"]
    yield "token_embd.weight", hp["embd_type"], E, V
    yield "output_norm.weight", F32, E, 1
    if hp.get("head_type") is not None:
        yield "output.weight", hp["head_type"], E, V
    for i in range(hp["n_layer"]):
        p = f"blk.{i}."
        for name, n in _extra_norms(hp, p):
            yield name, F32, n, 1
        yield p + "attn_norm.weight", F32, E, 1
        yield p + "ffn_norm.weight", F32, E, 1
        yield p + "attn_q.weight", wt, E, H * HD
        yield p + "attn_k.weight", wt, E, HKV * HD
        yield p + "attn_v.weight", wt, E, HKV * HD
        yield p + "attn_output.weight", wt, H * HD, E
        yield p + "ffn_gate.weight", wt, E, F
        yield p + "ffn_up.weight", wt, E, F
        yield p + "ffn_down.weight", hp.get("down_type", wt), F, E


def weight_bytes(hp: dict) -> dict:
    """Bytes per tensor role of a model of these hyperparameters (no generation)."""
    E, F, H, HKV, HD, V = (hp[k] for k in ("n_embd", "n_ff", "n_head", "n_head_kv", "head_dim", "n_vocab"))
    wt = hp["wtype"]
    dt = hp.get("down_type", wt)
    layer = (row_bytes(wt, E) * (H * HD + 2 * HKV * HD + 2 * F) + row_bytes(wt, H * HD) * E
             + row_bytes(dt, F) * E)
    head_t = hp["head_type"] if hp.get("head_type") is not None else hp["embd_type"]
    return dict(layer=layer, layers=layer * hp["n_layer"], head=row_bytes(head_t, E) * V,
                norms=4 * E * (2 * hp["n_layer"] + 1), embd_row=row_bytes(hp["embd_type"], E))
