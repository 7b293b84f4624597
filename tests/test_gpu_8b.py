"""Full-size parity: the cfg2 8B (32 layers, hidden 4096, FFN 14336, 32/8
heads of 128, vocab 128256, Q4_K layers, Q6_K head, q8 KV cache) through the
C ABI against the CPU oracle (the restatement of ts5's CpuBackend, pinned bit
for bit to the reference's own logits by tests/test_oracle.py), from the same
host weights on both sides.

Bars:
* logits: the reference's own GPU-vs-CPU check for a q8 cache
  (engine/src/checks.cpp:145-159: max|diff| / max|ref| <= 2e-2) plus cosine
  > 0.999 (engine/tests/compare.py:51-55), and relative L2 <= 1e-2;
* greedy decode: 100 % argmax agreement over the first 64 generated tokens of
  the device-resident greedy loop, checked by teacher forcing (the oracle runs
  the GPU's 64 ids as one batch: each row's argmax must be the next id; a
  CPU batch gives every row bit for bit what single-token steps give), free
  running with an f16 cache, and step by step on the reference's own cache
  state with a q8 cache (whose 1/127 rounding steps the two sides' last-bit
  differences can land on either side of; the free-running q8 run reports
  where it first parts from the reference).

The greedy part uses centred Q4_K weights (synth.blocks): with the benchmark's
distribution every weight's mean is far above zero and a random model's
argmax hardly depends on its input, so agreement there would prove little."""
import os
import time

import numpy as np
import pytest

import oracle
from tokenstation5_amd import synth, ts5hip

pytestmark = pytest.mark.gpu
SEED = 8_000_000_008
THREADS = min(16, os.cpu_count() or 1)  # the GPU box's share of host cores


def say(msg):
    print(f"[8b] {msg}", flush=True)


@pytest.fixture(scope="module")
def ctx():
    c = ts5hip.Context(0)
    yield c
    c.close()


def check_rows(got, want, tag, tol=2e-2):
    worst = 0.0
    for r in range(want.shape[0]):
        g, w = got[r].astype(np.float64), want[r].astype(np.float64)
        d = np.abs(g - w).max() / np.abs(w).max()
        cos = float(np.dot(g, w) / (np.linalg.norm(g) * np.linalg.norm(w)))
        rel = float(np.linalg.norm(g - w) / np.linalg.norm(w))
        worst = max(worst, d)
        assert d <= tol and cos > 0.999 and rel <= 1e-2, (tag, r, d, cos, rel)
    say(f"{tag}: {want.shape[0]} rows, worst max|diff|/max|ref| {worst:.2e}")


def test_8b_prompt_logits_cfg2_weights(ctx):
    """The benchmark's own weight distribution: an 8-token prompt, every
    position's logits (the batched matrix-core path), then one decode step
    (the single-token path), against the oracle."""
    hp = dict(synth.LLAMA_8B)
    t0 = time.time()
    tensors = synth.model_tensors(hp, SEED)
    say(f"cfg2 host weights generated ({time.time() - t0:.1f} s)")
    m = ts5hip.Model(ctx, hp, 64)
    m.set_tensors(tensors)
    prompt = np.random.default_rng(1).integers(0, hp["n_vocab"], 9).astype(np.int32)
    got = m.forward(prompt[:8], 0, all_logits=True)
    step = m.forward(prompt[8:], 8)
    m.close()
    ref = oracle.Model(hp, tensors, 64, 2, threads=THREADS)
    t0 = time.time()
    want = ref.forward(prompt, 0, all_logits=True)
    say(f"oracle: 9 tokens in {time.time() - t0:.1f} s")
    check_rows(got, want[:8], "cfg2 prompt")
    check_rows(step, want[8:], "cfg2 decode step")


@pytest.fixture(scope="module")
def centred():
    hp = dict(synth.LLAMA_8B, centered=True)
    t0 = time.time()
    tensors = synth.model_tensors(hp, SEED + 1)
    say(f"centred host weights generated ({time.time() - t0:.1f} s)")
    return hp, tensors


@pytest.mark.parametrize("kv", [ts5hip.KV_F16, ts5hip.KV_Q8])
def test_8b_greedy_64_tokens(ctx, centred, kv):
    hp, tensors = centred
    m = ts5hip.Model(ctx, hp, 96, kv)
    m.set_tensors(tensors)
    prompt = np.random.default_rng(2).integers(0, hp["n_vocab"], 4).astype(np.int32)
    lg = m.forward(prompt, 0)[0]
    first = int(np.argmax(lg))
    ids = np.concatenate([[first], m.generate_greedy(first, prompt.size, 63)]).astype(np.int32)
    say(f"GPU greedy ids[:12] {list(ids[:12])}, {np.unique(ids).size} distinct of 64")
    seq = np.concatenate([prompt, ids[:-1]]).astype(np.int32)
    got = m.forward(seq, 0, all_logits=True)  # the same 67 positions as one batch on the GPU
    m.close()
    ref = oracle.Model(hp, tensors, 96, kv, threads=THREADS)
    t0 = time.time()
    want = ref.forward(seq, 0, all_logits=True)
    say(f"oracle (kv {kv}): {seq.size} tokens teacher-forced in {time.time() - t0:.1f} s ({THREADS} threads)")
    picks = np.argmax(want[prompt.size - 1:], axis=1)
    div = next((i for i in range(64) if picks[i] != ids[i]), None)
    msg = "64 of 64 greedy tokens agree"
    if div is not None:
        row = want[prompt.size - 1 + div]
        top2 = np.sort(row)[-2:]
        msg = (f"first divergence at generated token {div}: GPU {ids[div]}, oracle {picks[div]} "
               f"(oracle top-2 gap {top2[1] - top2[0]:.3e} of max {top2[1]:.3e})")
    say(f"kv {kv} free-running: {msg}")
    assert np.unique(ids).size > 8  # the centred model's argmax follows its input
    if kv == ts5hip.KV_F16:
        # An f16 cache rounds each value to 11 bits: both sides' caches agree
        # and the whole 64-token continuation must be the reference's.
        assert div is None, msg
        check_rows(got, want, "centred 67 positions", tol=5e-3)
    # A q8 cache rounds each 32-value block to 1/127 of its largest value:
    # inputs differing in their last bits (fp32 GPU sums against the
    # reference's fp64) land on different sides of a rounding boundary now
    # and then, and this random model's near one-hot attention (scores of
    # several thousand) can turn one such step into another token. The GPU's
    # two paths agree with each other; per-step parity on the reference's own
    # cache state is test_8b_q8_steps_on_reference_cache.


def test_8b_q8_steps_on_reference_cache(ctx, centred):
    """64 decode steps of the centred 8B with a q8 cache, each on the
    oracle's exact cache state (every earlier position's K and V written into
    the GPU's cache through ts5hip_kv_write, which stores already-rounded
    values exactly): every step's greedy pick equals the oracle's and its
    logits are within the reference's q8 check bar."""
    hp, tensors = centred
    L, W = hp["n_layer"], hp["n_head_kv"] * hp["head_dim"]
    prompt = np.random.default_rng(2).integers(0, hp["n_vocab"], 4).astype(np.int32)
    m = ts5hip.Model(ctx, hp, 96, ts5hip.KV_Q8)
    m.set_tensors(tensors)
    first = int(np.argmax(m.forward(prompt, 0)[0]))
    ids = np.concatenate([[first], m.generate_greedy(first, prompt.size, 63)]).astype(np.int32)
    seq = np.concatenate([prompt, ids[:-1]]).astype(np.int32)
    ref = oracle.Model(hp, tensors, 96, ts5hip.KV_Q8, threads=THREADS)
    want = ref.forward(seq, 0, all_logits=True)
    cache = [[ref.kv(which, layer)[:seq.size].copy() for which in (0, 1)] for layer in range(L)]
    for layer in range(L):
        for which in (0, 1):
            m.kv_write(layer, which, 0, cache[layer][which])
    picks, worst = 0, 0.0
    for i in range(64):
        p = prompt.size - 1 + i
        got = m.forward(seq[p:p + 1], p)[0]  # overwrites slot p with the GPU's own K / V of that token
        for layer in range(L):
            for which in (0, 1):
                m.kv_write(layer, which, p, cache[layer][which][p:p + 1])
        g, w = got.astype(np.float64), want[p].astype(np.float64)
        d = np.abs(g - w).max() / np.abs(w).max()
        worst = max(worst, d)
        assert int(np.argmax(got)) == int(np.argmax(want[p])), (i, d)
        assert d <= 2e-2, (i, d)
        picks += 1
    say(f"q8 on the reference's cache state: {picks} of 64 steps pick the oracle's token, worst "
        f"max|diff|/max|ref| {worst:.2e}")
    m.close()
