"""Writes the golden vectors under tests/golden/ from ts5's own CPU code.

Run in a container that holds the reference (it builds oracle/_ref first):

    python tests/golden/make_golden.py

Every input is regenerated from a seed by tokenstation5_amd/synth.py (numpy
PCG64), so the fixtures hold only seeds, small inputs, and the reference's
outputs (plus sha256 digests of the regenerated inputs, so a change in the
generator shows up as a fixture mismatch instead of a silent drift).
The reference runs here only; its files never travel with the fixtures.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import gguf_writer  # noqa: E402
import oracle  # noqa: E402
from tokenstation5_amd import synth  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
MODEL_SEED = 1234


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def fp16_inputs(seed: int = 7) -> np.ndarray:
    """fp32 bit patterns covering f16's range edges, then random ones."""
    rng = np.random.default_rng(seed)
    edges = []
    for e in range(90, 160):  # exponents around f16's normal / subnormal / overflow range
        for m in (0, 1, 0xFFF, 0x1000, 0x1001, 0x2000, 0x3000, 0x7FE000, 0x7FF000, 0x7FFFFF):
            edges.append((e << 23) | m)
    edges += [0, 0x7F800000, 0x7FC00000, 0x7F800001, 0x477FE000, 0x477FF000, 0x477FEFFF]
    edges = np.array(edges, np.uint32)
    edges = np.concatenate([edges, edges | 0x80000000])
    rand = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    small = (np.abs(rng.standard_normal(1 << 16)) * 1e-4).astype(np.float32).view(np.uint32)
    return np.concatenate([edges, rand, small])


def golden_fp16():
    R = oracle.ref()
    halves = np.arange(65536, dtype=np.uint32)
    h2f = np.array([R.ts5r_fp16_to_fp32(int(h)) for h in halves], np.float32)
    xs = fp16_inputs()
    f2h = np.array([R.ts5r_fp32_to_fp16(float(v)) for v in xs.view(np.float32)], np.uint16)
    np.savez_compressed(os.path.join(OUT, "fp16.npz"), h2f_sha=sha(h2f.view(np.uint32)),
                        f2h_seed=7, f2h_inputs_sha=sha(xs), f2h_sha=sha(f2h), f2h_head=f2h[:4096],
                        h2f_head=h2f.view(np.uint32)[:4096])


def special_blocks(t: int) -> np.ndarray:
    """Hand-made blocks: zero, f16-subnormal, negative and large scales."""
    bb = synth.BLOCK[t][1]
    rng = np.random.default_rng(99)
    out = []
    for d_bits in (0x0000, 0x0001, 0x03FF, 0x0400, 0x8123, 0x3C00, 0x7BFF, 0x2E66):
        b = np.frombuffer(rng.bytes(bb), np.uint8).copy()
        d = np.array([d_bits], np.uint16).view(np.uint8)
        if t in (synth.Q4_K, synth.Q5_K, synth.Q4_1, synth.Q5_1):
            b[0:2] = d
            b[2:4] = np.array([d_bits ^ 0x0201], np.uint16).view(np.uint8)
        elif t == synth.Q6_K:
            b[208:210] = d
        elif t in (synth.Q8_0, synth.Q4_0, synth.Q5_0):
            b[0:2] = d
        out.append(b)
    return np.stack(out)


def golden_quants():
    R = oracle.ref()
    res = {}
    for t in (synth.Q4_0, synth.Q4_1, synth.Q5_0, synth.Q5_1, synth.Q8_0, synth.Q4_K, synth.Q5_K, synth.Q6_K,
              synth.F16, synth.BF16):
        bv, bb = synth.BLOCK[t]
        nb = 16 if bv == 256 else (64 if bv == 32 else 2048)
        blocks = synth.blocks(t, nb, np.random.default_rng([5, t]))
        if bv > 1:
            blocks = np.concatenate([blocks, special_blocks(t)])
        n = blocks.shape[0] * bv
        y = np.empty(n, np.float32)
        rc = R.ts5r_dequantize_row(t, np.ascontiguousarray(blocks).ctypes.data, y, n)
        assert rc == 0, t
        res[f"t{t}_blocks"] = blocks
        res[f"t{t}_values"] = y
    np.savez_compressed(os.path.join(OUT, "quants.npz"), **res)


def write_model(hp: dict, path: str) -> dict:
    tensors = synth.model_tensors(hp, MODEL_SEED)
    gguf_writer.write(path, gguf_writer.model_kv(hp), tensors)
    return tensors


def check_schedule(R, path, n, kv, nv):
    """ts5 check's order (engine/src/checks.cpp:119-124): n-4 tokens in one
    call with every position's logits, then 4 single-token calls."""
    toks = np.array([(17 + i * 7919) % nv for i in range(n)], np.int32)
    h = R.ts5r_cpu_open(path.encode(), 64, kv)
    assert h, R.ts5r_last_error()
    single = min(4, n // 2)
    batch = n - single
    out = np.empty((n, nv), np.float32)
    assert R.ts5r_cpu_forward(h, toks[:batch].copy(), batch, 0, out.ctypes.data, 1) == 0
    for i in range(batch, n):
        assert R.ts5r_cpu_forward(h, toks[i:i + 1].copy(), 1, i, out[i:].ctypes.data, 0) == 0
    R.ts5r_cpu_close(h)
    return toks, out


MODELS = {"tiny_llama": synth.TINY_LLAMA, "tiny_draft": synth.TINY_DRAFT, "tiny_llama_c": synth.TINY_LLAMA_C,
          "tiny_draft_c": synth.TINY_DRAFT_C, "tiny_gemma3": synth.TINY_GEMMA3, "tiny_qwen3": synth.TINY_QWEN3,
          "tiny_llama31": synth.TINY_LLAMA31}


def golden_models(names=None):
    """Each model's check-schedule logits (f32, f16, q8 caches) and 64 greedy
    ids; `names` regenerates only those (the manifest keeps the others)."""
    R = oracle.ref()
    mpath = os.path.join(OUT, "models.json")
    manifest = json.load(open(mpath)) if names and os.path.exists(mpath) else {}
    with tempfile.TemporaryDirectory() as d:
        for name, hp in MODELS.items():
            if names and name not in names:
                continue
            path = os.path.join(d, name + ".gguf")
            tensors = write_model(hp, path)
            digests = {k: sha(v[3]) for k, v in tensors.items()}
            nv = hp["n_vocab"]
            res = {}
            for kv in (0, 1, 2):
                toks, lg = check_schedule(R, path, 12, kv, nv)
                res[f"kv{kv}_tokens"] = toks
                res[f"kv{kv}_logits"] = lg
            # Greedy generation, 64 tokens, no speculation.
            prompt = np.array([(17 + 31 * i) % nv for i in range(8)], np.int32)
            ids = np.zeros(64, np.int32)
            stats = np.zeros(3, np.int32)
            n = R.ts5r_generate(path.encode(), b"", 128, 2, prompt, prompt.size, 0.0, 0.95, 40, 1, 0, 64, ids,
                                stats)
            assert n == 64, (n, R.ts5r_last_error())
            res["greedy_prompt"] = prompt
            res["greedy_q8_ids"] = ids
            # The same with an f16 cache (KvType::F16, the Vulkan backend's default).
            ids16 = np.zeros(64, np.int32)
            n = R.ts5r_generate(path.encode(), b"", 128, 1, prompt, prompt.size, 0.0, 0.95, 40, 1, 0, 64, ids16,
                                stats)
            assert n == 64, (n, R.ts5r_last_error())
            res["greedy_f16_ids"] = ids16
            np.savez_compressed(os.path.join(OUT, f"model_{name}.npz"), **res)
            manifest[name] = dict(seed=MODEL_SEED, hparams={k: v for k, v in hp.items()}, tensor_sha256=digests)
    with open(mpath, "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)


# ts5 check's test tokens need a vocabulary past 1000 (engine/src/checks.cpp:22-26).
TINY_CHECK = dict(synth.TINY_LLAMA_C, n_vocab=2048)
CHECK_N = 16


def golden_check():
    """`ts5 check` run by the reference itself (run_check with its CPU backend
    in the GPU's place) on a small GGUF: the .ts5ref files it saves next to
    the model (f16 and q8 caches), byte for byte, and its result."""
    R = oracle.ref()
    res = {}
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "check.gguf")
        write_model(TINY_CHECK, path)
        res["gguf_sha"] = np.frombuffer(hashlib.sha256(open(path, "rb").read()).digest(), np.uint8)
        for kv, suffix in ((1, ".ts5ref"), (2, ".q8.ts5ref")):
            out = (C.c_double * 5)()
            assert R.ts5r_check(path.encode(), kv, CHECK_N, out) == 0, R.ts5r_last_error()
            res[f"kv{kv}_result"] = np.array(list(out), np.float64)
            res[f"kv{kv}_file"] = np.frombuffer(open(path + suffix, "rb").read(), np.uint8)
    np.savez_compressed(os.path.join(OUT, "check.npz"), **res)


def sampler_table(seed: int, rows: int, nv: int) -> np.ndarray:
    return (np.random.default_rng(seed).standard_normal((rows, nv)) * 3.0).astype(np.float32)


SAMPLER_CASES = [  # (temperature, top_p, top_k): the benchmark's, the engine's defaults, greedy, no top-k
    (0.7, 0.9, 40), (0.7, 0.95, 40), (0.0, 0.95, 40), (1.0, 0.9, 0), (0.3, 1.0, 5)]


def golden_sampler():
    R = oracle.ref()
    nv, rows = 128256, 24
    table = sampler_table(11, rows, nv)
    res = dict(table_seed=11, rows=rows, n_vocab=nv, table_sha=sha(table))
    for i, (T, p, k) in enumerate(SAMPLER_CASES):
        out = np.zeros(rows, np.int32)
        n = R.ts5r_sample_table(table, rows, nv, T, p, k, 42 + i, rows, out)
        assert n == rows, (n, R.ts5r_last_error())
        res[f"case{i}"] = np.array([T, p, k], np.float64)
        res[f"ids{i}"] = out
    np.savez_compressed(os.path.join(OUT, "sampler.npz"), **res)


def golden_speculation():
    """Engine::generate with prompt-lookup drafting and with a draft model
    (the tiny draft, and the target as its own drafter)."""
    R = oracle.ref()
    res = {}
    with tempfile.TemporaryDirectory() as d:
        tp = os.path.join(d, "t.gguf")
        dp = os.path.join(d, "d.gguf")
        write_model(synth.TINY_LLAMA_C, tp)
        write_model(synth.TINY_DRAFT_C, dp)
        nv = synth.TINY_LLAMA["n_vocab"]
        base = [(5 + 13 * i) % nv for i in range(10)]
        # The plain greedy continuation of `base`, then `base` again: prompt
        # lookup finds that continuation and drafts it.
        ids = np.zeros(16, np.int32)
        first = np.array(base, np.int32)
        assert R.ts5r_generate(tp.encode(), b"", 256, 2, first, first.size, 0.0, 0.9, 40, 3, 0, 16, ids,
                               np.zeros(3, np.int32)) == 16
        prompt = np.array(base + list(ids) + base, np.int32)
        res["prompt"] = prompt
        cases = {"plain": (b"", 0), "lookup4": (b"", 4), "draft_model4": (dp.encode(), 4),
                 "self_draft4": (tp.encode(), 4)}
        for name, (drafter, k) in cases.items():
            for T, tag in ((0.0, "greedy"), (0.7, "t07")):
                ids = np.zeros(48, np.int32)
                stats = np.zeros(3, np.int32)
                n = R.ts5r_generate(tp.encode(), drafter, 256, 2, prompt, prompt.size, T, 0.9, 40, 3, k, 48, ids,
                                    stats)
                assert n == 48, (name, n, R.ts5r_last_error())
                res[f"{name}_{tag}_ids"] = ids
                res[f"{name}_{tag}_stats"] = stats
    np.savez_compressed(os.path.join(OUT, "speculation.npz"), **res)


def main():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "all", "ref"], check=True)
    os.environ.pop("TS5_DRAFT", None)
    os.environ.pop("TS5_ADAPT", None)
    os.environ.pop("TS5_SWA_WINDOW", None)
    if len(sys.argv) > 1:  # model fixtures only: make_golden.py tiny_gemma3 ...
        golden_models(sys.argv[1:])
        print("model fixtures written:", " ".join(sys.argv[1:]))
        return
    golden_fp16()
    golden_quants()
    golden_models()
    golden_sampler()
    golden_speculation()
    golden_check()
    print("golden vectors written to", OUT)


if __name__ == "__main__":
    main()
