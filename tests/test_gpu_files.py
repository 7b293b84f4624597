"""GGUF files into HBM (ts5hip_model_load) and `ts5 check` over this backend
(ts5hip_check_run), through the C ABI.

Bars: a model loaded from a GGUF file computes exactly what the same tensors
set by name compute (bit-identical logits: the same bytes reach HBM, Q6_K /
Q8_0 repacked on the way); an automatic context takes the training context
in an f16 cache when that fits (engine/src/vk_backend.cpp:620-648); the check
passes against the reference's own saved logits (the .ts5ref files its
run_check wrote, tests/golden/check.npz) at its bars, and fails on a model
that is not the reference's."""
import json
import os

import numpy as np
import pytest

import gguf_writer
import make_golden
from tokenstation5_amd import synth, ts5hip

pytestmark = pytest.mark.gpu
G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MODELS = json.load(open(os.path.join(G, "models.json")))


@pytest.fixture(scope="module")
def ctx():
    c = ts5hip.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("name", ["tiny_llama_c", "tiny_draft_c"])
@pytest.mark.parametrize("threads", [1, 3])
def test_load_equals_set_tensors(ctx, tmp_path, name, threads):
    hp = dict(MODELS[name]["hparams"])
    tensors = synth.model_tensors(hp, make_golden.MODEL_SEED)
    path = str(tmp_path / f"{name}.gguf")
    gguf_writer.write(path, gguf_writer.model_kv(hp), tensors)
    m = ts5hip.load_model(ctx, path, n_ctx=64, kv=ts5hip.KV_Q8, threads=threads)
    assert m.n_ctx() == 64 and m.kv_type() == ts5hip.KV_Q8
    ref = ts5hip.Model(ctx, hp, 64)
    ref.set_tensors(tensors)
    toks = np.array([(7 + 13 * i) % hp["n_vocab"] for i in range(20)], np.int32)
    a = m.forward(toks, 0, all_logits=True)
    b = ref.forward(toks, 0, all_logits=True)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert list(m.generate_greedy(int(np.argmax(a[-1])), 20, 8)) == list(ref.generate_greedy(int(np.argmax(b[-1])), 20, 8))
    m.close()
    ref.close()


def test_load_auto_context(ctx, tmp_path):
    """n_ctx 0: the training context (32768 in these files) fits the GPU many
    times over in f16, so a q8 request gets an f16 cache of 32768 positions."""
    hp = synth.TINY_LLAMA
    path = str(tmp_path / "m.gguf")
    gguf_writer.write(path, gguf_writer.model_kv(hp), synth.model_tensors(hp, 3))
    m = ts5hip.load_model(ctx, path, n_ctx=0, kv=ts5hip.KV_Q8)
    assert m.n_ctx() == 32768 and m.kv_type() == ts5hip.KV_F16 and m.chosen_kv == ts5hip.KV_F16
    lg = m.forward(np.array([1, 2, 3], np.int32), 0)
    assert np.isfinite(lg).all()
    m.close()
    with pytest.raises(ts5hip.Ts5HipError):
        ts5hip.load_model(ctx, str(tmp_path / "missing.gguf"))


@pytest.mark.parametrize("kv", [ts5hip.KV_F16, ts5hip.KV_Q8])
def test_check_against_reference_file(ctx, tmp_path, kv):
    hp, n = make_golden.TINY_CHECK, make_golden.CHECK_N
    path = str(tmp_path / "check.gguf")
    gguf_writer.write(path, gguf_writer.model_kv(hp), synth.model_tensors(hp, make_golden.MODEL_SEED))
    g = np.load(os.path.join(G, "check.npz"))
    with open(ts5hip.ref_path(path, kv), "wb") as f:
        f.write(bytes(g[f"kv{kv}_file"]))
    m = ts5hip.load_model(ctx, path, n_ctx=n, kv=kv)
    r = m.check_run(path, n)
    print(f"kv {kv}: max |diff| {r.max_diff:.3g} ({r.rel:.2g} of the largest logit) at {r.worst}, "
          f"same top {r.same_top}/{r.n}, {r.gpu_ms:.1f} ms")
    assert r.pass_ and r.saved and r.n == n and r.same_top == n
    # The same with the logits handed over, and against another model's (it must fail).
    ref = ts5hip.ref_load(path, n, hp["n_vocab"], kv)
    assert m.check_run(None, n, ref).pass_
    other = ts5hip.Model(ctx, hp, n, kv)
    other.set_tensors(synth.model_tensors(hp, make_golden.MODEL_SEED + 1))
    assert not other.check_run(path, n).pass_
    m.close()
    other.close()
