"""TEST INFRASTRUCTURE: writes GGUF v3 files of synthetic models.

Only used to hand models to ts5's own CPU code (oracle/_ref) when golden
vectors are made. The layout is the one engine/src/gguf.cpp:94-170 reads:
magic, version, tensor and key counts, typed key/value pairs, tensor infos
(name, dims, type, offset into the data section), then the data section at
the next multiple of general.alignment (32), each tensor at a multiple of 32.
"""
from __future__ import annotations

import struct

import numpy as np

T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR = 4, 5, 6, 7, 8, 9


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(v):
    if isinstance(v, bool):
        return struct.pack("<I", T_BOOL) + struct.pack("<B", int(v))
    if isinstance(v, int):
        return struct.pack("<I", T_I32) + struct.pack("<i", v)
    if isinstance(v, float):
        return struct.pack("<I", T_F32) + struct.pack("<f", v)
    if isinstance(v, str):
        return struct.pack("<I", T_STR) + _str(v)
    if isinstance(v, list):
        if all(isinstance(x, str) for x in v):
            return struct.pack("<IIQ", T_ARR, T_STR, len(v)) + b"".join(_str(x) for x in v)
        return struct.pack("<IIQ", T_ARR, T_I32, len(v)) + b"".join(struct.pack("<i", x) for x in v)
    raise TypeError(type(v))


def write(path: str, kv: dict, tensors: dict) -> None:
    """tensors: {name: (ggml_type, ne0, ne1, uint8 array of the raw bytes)}."""
    head = [b"GGUF", struct.pack("<IQQ", 3, len(tensors), len(kv))]
    for k, v in kv.items():
        head.append(_str(k) + _value(v))
    off = 0
    infos, blobs = [], []
    for name, (t, ne0, ne1, data) in tensors.items():
        dims = [ne0] if ne1 == 1 and name.endswith("norm.weight") else [ne0, ne1]
        infos.append(_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
                     + struct.pack("<IQ", t, off))
        raw = np.ascontiguousarray(data).tobytes()
        pad = (-len(raw)) % 32
        blobs.append(raw + b"\0" * pad)
        off += len(raw) + pad
    header = b"".join(head + infos)
    header += b"\0" * ((-len(header)) % 32)
    with open(path, "wb") as f:
        f.write(header)
        for b in blobs:
            f.write(b)


def model_kv(hp: dict, vocab_pieces: bool = True) -> dict:
    """Metadata for a synthetic model of hyperparameters hp (synth.py's dicts)."""
    a = hp["arch"]
    kv = {
        "general.architecture": a,
        "general.alignment": 32,
        f"{a}.embedding_length": hp["n_embd"],
        f"{a}.block_count": hp["n_layer"],
        f"{a}.feed_forward_length": hp["n_ff"],
        f"{a}.attention.head_count": hp["n_head"],
        f"{a}.attention.head_count_kv": hp["n_head_kv"],
        f"{a}.attention.key_length": hp["head_dim"],
        f"{a}.context_length": 32768,
        f"{a}.attention.layer_norm_rms_epsilon": float(hp["rms_eps"]),
        f"{a}.rope.freq_base": float(hp["rope_base"]),
        f"{a}.rope.dimension_count": hp["head_dim"],
    }
    if hp.get("swa_window"):
        kv[f"{a}.attention.sliding_window"] = hp["swa_window"]
    if hp.get("rope_scaling_factor"):
        kv[f"{a}.rope.scaling.type"] = "linear"
        kv[f"{a}.rope.scaling.factor"] = float(hp["rope_scaling_factor"])
    if vocab_pieces:
        # Pieces that decode back to "<id>" (no merges, no end-of-generation).
        kv["tokenizer.ggml.model"] = "gpt2"
        kv["tokenizer.ggml.tokens"] = [f"<{i}>" for i in range(hp["n_vocab"])]
    return kv
