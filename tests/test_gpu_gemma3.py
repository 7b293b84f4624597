"""Gemma 3 through the C ABI (engine/src/model.cpp:44-63, engine/src/cpu_backend.cpp:120-266):
the scaled embedding, q/k norms, head dimension 256, sliding layers (five of six) that see only
their last swa_window keys with their own RoPE base, the global layer, GELU, and the norms after
attention and the FFN, on synth.TINY_GEMMA3 (8-key window, so every sequence here crosses it).

Against the reference's own CPU backend (tests/golden/model_tiny_gemma3.npz, written by
make_golden.py from engine/src/cpu_backend.cpp; the oracle restates it bit for bit): the check
schedule's logits at the reference's bars (engine/src/checks.cpp:152-159: max|diff| / max|ref|
<= 5e-3 with an f16 cache, 2e-2 with q8) and its 64 greedy ids. Against the oracle: a 40-token
prompt chunk (the matmuls and the per-query windowed attention), verify batches of 5 and 12,
and single tokens after them; the same at head dimension 128 (27B's attention shape), also
over a 9000-position cache, and at Gemma 3 1B's layer width over a 700-token prompt past its
512-key window. A GGUF file loads to
the same logits, and the engine's self-drafting output equals plain greedy decoding."""
import os

import numpy as np
import pytest

import gguf_writer
import make_golden
import oracle
from tokenstation5_amd import synth, ts5hip

pytestmark = pytest.mark.gpu
G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
HP = synth.TINY_GEMMA3
BAR = {ts5hip.KV_F16: 5e-3, ts5hip.KV_Q8: 2e-2}


@pytest.fixture(scope="module")
def ctx():
    c = ts5hip.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def tensors():
    return synth.model_tensors(HP, make_golden.MODEL_SEED)


def rows_within(got, want, tol, what):
    for r in range(want.shape[0]):
        d = np.abs(got[r].astype(np.float64) - want[r]).max() / np.abs(want[r]).max()
        assert d <= tol, (what, r, d)


def model(ctx, tensors, kv, n_ctx=128):
    m = ts5hip.Model(ctx, HP, n_ctx, kv)
    m.set_tensors(tensors)
    return m


@pytest.mark.parametrize("graphs", ["1", "0"])
@pytest.mark.parametrize("kv,key", [(ts5hip.KV_F16, "kv1"), (ts5hip.KV_Q8, "kv2")])
def test_check_schedule_logits(ctx, tensors, monkeypatch, graphs, kv, key):
    """n-4 tokens in one call with every position's logits, then 4 single
    tokens (engine/src/checks.cpp:119-124), against the reference's logits."""
    monkeypatch.setenv("TS5HIP_GRAPHS", graphs)
    g = np.load(os.path.join(G, "model_tiny_gemma3.npz"))
    toks, want = g[f"{key}_tokens"], g[f"{key}_logits"]
    m = model(ctx, tensors, kv, 64)
    n = toks.size
    got = np.empty_like(want)
    got[:n - 4] = m.forward(toks[:n - 4], 0, all_logits=True)
    for i in range(n - 4, n):
        got[i] = m.forward(toks[i:i + 1], i)[0]
    rows_within(got, want, BAR[kv], "check schedule")
    assert np.mean(np.argmax(got, 1) == np.argmax(want, 1)) >= 0.9
    m.close()


@pytest.mark.parametrize("kv", [ts5hip.KV_F16, ts5hip.KV_Q8])
def test_prompt_chunk_verify_and_decode(ctx, tensors, kv):
    """A 40-token prompt chunk (past 16 tokens: the chunk matmuls, each query
    over its own window), verify batches of 5 and 12 tokens (RoPE and the
    K/V append inside the attention), then single tokens, each against the
    oracle fed the same tokens at the same positions."""
    m = model(ctx, tensors, kv)
    ref = oracle.Model(HP, tensors, 128, kv)
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, HP["n_vocab"], 40).astype(np.int32)
    rows_within(m.forward(prompt, 0, all_logits=True), ref.forward(prompt, 0, all_logits=True), BAR[kv], "prompt")
    pos = prompt.size
    for n in (5, 12):
        toks = rng.integers(0, HP["n_vocab"], n).astype(np.int32)
        rows_within(m.forward(toks, pos, all_logits=True), ref.forward(toks, pos, all_logits=True), BAR[kv],
                    f"verify {n}")
        pos += n
    for i in range(6):
        t = rng.integers(0, HP["n_vocab"], 1).astype(np.int32)
        rows_within(m.forward(t, pos), ref.forward(t, pos), BAR[kv], f"token {pos}")
        pos += 1
    m.close()


@pytest.mark.parametrize("graphs", ["1", "0"])
def test_greedy_64_f16(ctx, tensors, monkeypatch, graphs):
    """64 greedy ids with an f16 cache equal the reference's
    (Engine::generate over its CPU backend)."""
    monkeypatch.setenv("TS5HIP_GRAPHS", graphs)
    g = np.load(os.path.join(G, "model_tiny_gemma3.npz"))
    prompt, want = g["greedy_prompt"], list(g["greedy_f16_ids"])
    m = model(ctx, tensors, ts5hip.KV_F16)
    first = int(np.argmax(m.forward(prompt, 0)[0]))
    ids = [first] + list(m.generate_greedy(first, prompt.size, 63))
    assert ids == want, next(i for i in range(64) if ids[i] != want[i])
    m.close()


def test_greedy_64_q8(ctx, tensors):
    """With a q8 cache: the reference's 64 ids, or a first difference at a
    step where the oracle (bit-identical to the reference) fed the GPU's own
    tokens has its top two logits within q8 rounding of each other."""
    g = np.load(os.path.join(G, "model_tiny_gemma3.npz"))
    prompt, want = g["greedy_prompt"], list(g["greedy_q8_ids"])
    m = model(ctx, tensors, ts5hip.KV_Q8)
    first = int(np.argmax(m.forward(prompt, 0)[0]))
    ids = [first] + list(m.generate_greedy(first, prompt.size, 63))
    if ids != want:
        k = next(i for i in range(64) if ids[i] != want[i])
        ref = oracle.Model(HP, tensors, 128, ts5hip.KV_Q8)
        lg = ref.forward(prompt, 0)[0]
        for i in range(k):
            lg = ref.forward(np.array([ids[i]], np.int32), prompt.size + i)[0]
        top = np.sort(lg)[-2:]
        gap = (top[1] - top[0]) / np.abs(lg).max()
        print(f"gemma3 q8 greedy: first difference at token {k}, oracle top-2 gap {gap:.2e} of the largest logit")
        assert gap < 2e-2, (k, gap)
        assert ids[k] in np.argsort(lg)[-2:], k
    m.close()


# Head dimension 128 with two query heads a KV head (Gemma 3 27B's attention
# shape): decode on the LDS kernel with windows, the global layer's q8 prompt
# chunks on the matrix cores and its verify batches on the multi-query kernel.
HP128 = dict(HP, n_head=8, n_head_kv=4, head_dim=128)
# Gemma 3 1B's layer (1152 wide: Q8_0 rows, not whole Q4_K super-blocks;
# window 512), seven layers so that one is global, and a smaller vocabulary.
HP1B = dict(HP, n_embd=1152, n_ff=6912, n_layer=7, swa_window=512, wtype=synth.Q8_0, embd_type=synth.Q8_0,
            n_vocab=4096, centered=False)


@pytest.mark.parametrize("hp,kv,n_prompt", [(HP128, ts5hip.KV_Q8, 40), (HP128, ts5hip.KV_F16, 40),
                                            (HP1B, ts5hip.KV_Q8, 700)])
def test_other_shapes_against_oracle(ctx, hp, kv, n_prompt):
    tensors = synth.model_tensors(hp, 11)
    n_ctx = n_prompt + 32
    m = ts5hip.Model(ctx, hp, n_ctx, kv)
    m.set_tensors(tensors)
    ref = oracle.Model(hp, tensors, n_ctx, kv)
    rng = np.random.default_rng(9)
    prompt = rng.integers(0, hp["n_vocab"], n_prompt).astype(np.int32)
    rows_within(m.forward(prompt, 0), ref.forward(prompt, 0), BAR[kv], "prompt")
    pos = n_prompt
    toks = rng.integers(0, hp["n_vocab"], 5).astype(np.int32)
    rows_within(m.forward(toks, pos, all_logits=True), ref.forward(toks, pos, all_logits=True), BAR[kv], "verify")
    pos += 5
    for i in range(4):
        t = rng.integers(0, hp["n_vocab"], 1).astype(np.int32)
        rows_within(m.forward(t, pos), ref.forward(t, pos), BAR[kv], f"token {pos}")
        pos += 1
    m.close()


@pytest.mark.parametrize("kv", [ts5hip.KV_Q8, ts5hip.KV_F16])
def test_decode_over_long_cache(ctx, kv):
    """Single tokens at positions past 8192 at head dimension 128: the global
    layer over all 8990 earlier positions on the matrix-core one-query
    attention (k_attn_m1), the sliding layers over their last 8 keys. Both
    caches first hold the same values as the cache keeps them
    (ts5hip_kv_write; the oracle's own cache array), then each token against
    the oracle at the reference's bars."""
    hp = HP128
    tensors = synth.model_tensors(hp, 13)
    n_ctx, p0 = 9000, 8990
    m = ts5hip.Model(ctx, hp, n_ctx, kv)
    m.set_tensors(tensors)
    ref = oracle.Model(hp, tensors, n_ctx, kv)
    rng = np.random.default_rng(8)
    W = hp["n_head_kv"] * hp["head_dim"]
    for layer in range(hp["n_layer"]):
        for which in (0, 1):
            x = (rng.standard_normal((p0, W)) * 2.0).astype(np.float32)
            if kv == ts5hip.KV_Q8:  # per 32 values sc = f16(amax / 127), q = rint(v / sc)
                b = x.reshape(-1, 32)
                sc = (np.abs(b).max(1) / np.float32(127)).astype(np.float16).astype(np.float32)
                x = (np.clip(np.rint(b / sc[:, None]), -127, 127) * sc[:, None]).astype(np.float32).reshape(p0, W)
            else:
                x = x.astype(np.float16).astype(np.float32)
            m.kv_write(layer, which, 0, x)
            ref.kv(which, layer)[:p0] = x
    for i in range(5):
        t = rng.integers(0, hp["n_vocab"], 1).astype(np.int32)
        rows_within(m.forward(t, p0 + i), ref.forward(t, p0 + i), BAR[kv], f"token {p0 + i}")
    m.close()


def test_gguf_load(ctx, tensors, tmp_path):
    """The same tensors from a GGUF file: the loader derives Gemma 3's
    hyperparameters (model.cpp:44-63) and the logits are bit-identical."""
    path = str(tmp_path / "gemma3.gguf")
    gguf_writer.write(path, gguf_writer.model_kv(HP), tensors)
    prompt = np.random.default_rng(3).integers(0, HP["n_vocab"], 30).astype(np.int32)
    m = model(ctx, tensors, ts5hip.KV_F16, 64)
    want = m.forward(prompt, 0, all_logits=True)
    f = ts5hip.load_model(ctx, path, n_ctx=64, kv=ts5hip.KV_F16)
    assert np.array_equal(f.forward(prompt, 0, all_logits=True).view(np.uint32), want.view(np.uint32))
    f.close()
    m.close()


def test_self_draft_equals_greedy(ctx, tensors):
    """The decode driver drafting with the model itself (verify batches over
    the sliding windows) gives the plain greedy output."""
    prompt = np.random.default_rng(5).integers(0, HP["n_vocab"], 20).astype(np.int32)
    m = model(ctx, tensors, ts5hip.KV_F16)
    e = ts5hip.Engine(m)
    plain, st0 = e.generate(prompt, max_tokens=40, draft=0)
    e.close()
    m2, d = model(ctx, tensors, ts5hip.KV_F16), model(ctx, tensors, ts5hip.KV_F16)
    e2 = ts5hip.Engine(m2)
    e2.set_drafter(d)
    spec, st = e2.generate(prompt, max_tokens=40, draft=4, adapt=False)
    assert list(spec) == list(plain)
    assert st[3] > 0, st
    e2.close()
    for x in (m, m2, d):
        x.close()
