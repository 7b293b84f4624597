"""The decode driver (ts5hip_engine_generate: Engine::generate with
prompt-lookup and draft-model speculation) against the reference's own runs:
tests/golden/speculation.npz holds the ids and the drafted / accepted counts
of engine/src/engine.cpp on its CPU backend (make_golden.py), for the tiny
target with no drafting, lookup drafting, a draft model, and itself as the
draft model, greedy and at T = 0.7 (top_p 0.9, top_k 40, seed 3, q8 cache,
256-token context, 48 tokens).

Bars: the same ids and counts; and the greedy output with any drafting equal
to the output without (the reference's own claim, engine/src/engine.cpp:
186-190)."""
import json
import os

import numpy as np
import pytest

import make_golden
from tokenstation5_amd import synth, ts5hip

pytestmark = pytest.mark.gpu
G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MODELS = json.load(open(os.path.join(G, "models.json")))
SPEC = np.load(os.path.join(G, "speculation.npz"))
CASES = {"plain": (None, 0), "lookup4": (None, 4), "draft_model4": ("tiny_draft_c", 4),
         "self_draft4": ("tiny_llama_c", 4)}


@pytest.fixture(scope="module")
def ctx():
    c = ts5hip.Context(0)
    yield c
    c.close()


def load(ctx, name, n_ctx=256):
    hp = dict(MODELS[name]["hparams"])
    m = ts5hip.Model(ctx, hp, n_ctx)
    m.set_tensors(synth.model_tensors(hp, make_golden.MODEL_SEED))
    return m


@pytest.mark.parametrize("temp,tag", [(0.0, "greedy"), (0.7, "t07")])
@pytest.mark.parametrize("case", list(CASES))
def test_generate_matches_reference(ctx, case, temp, tag):
    drafter, k = CASES[case]
    m = load(ctx, "tiny_llama_c")
    e = ts5hip.Engine(m)
    dm = load(ctx, drafter) if drafter else None
    e.set_drafter(dm)
    ids, st = e.generate(SPEC["prompt"], temperature=temp, top_p=0.9, top_k=40, max_tokens=48, seed=3, draft=k)
    want_ids, want_st = SPEC[f"{case}_{tag}_ids"], SPEC[f"{case}_{tag}_stats"]
    div = next((i for i in range(48) if ids[i] != want_ids[i]), None)
    assert div is None, f"first divergence at {div}: {ids[div]} vs {want_ids[div]}"
    assert list(st[2:5]) == list(want_st), (st, want_st)  # generated, drafted, accepted
    if k and case != "plain":
        assert st[3] > 0  # speculation happened
    e.close()


def test_drafting_keeps_greedy_output(ctx):
    m = load(ctx, "tiny_llama_c")
    base = None
    for k in (0, 1, 4, 7):
        e = ts5hip.Engine(m)
        ids, st = e.generate(SPEC["prompt"], temperature=0.0, max_tokens=40, seed=1, draft=k)
        if base is None:
            base = list(ids)
        assert list(ids) == base, k
        e.close()


def test_prefix_reuse_and_errors(ctx):
    """A second request sharing a prefix re-evaluates only the rest
    (engine/src/engine.cpp:157-165); an empty or too long prompt fails."""
    m = load(ctx, "tiny_llama_c", n_ctx=96)
    e = ts5hip.Engine(m)
    p = SPEC["prompt"]
    ids1, st1 = e.generate(p, max_tokens=8, draft=0)
    assert st1[1] == p.size
    ids2, st2 = e.generate(np.concatenate([p, ids1[:3]]), max_tokens=8, draft=0)
    assert st2[1] == 1  # all but the last prompt token were cached; that one is evaluated again
    ref = ts5hip.Engine(load(ctx, "tiny_llama_c", n_ctx=96))
    ids3, _ = ref.generate(np.concatenate([p, ids1[:3]]), max_tokens=8, draft=0)
    assert list(ids2) == list(ids3)
    with pytest.raises(ts5hip.Ts5HipError):
        e.generate(np.zeros(0, np.int32))
    with pytest.raises(ts5hip.Ts5HipError):
        e.generate(np.ones(96, np.int32))
    e.close()
    ref.close()


def test_end_of_generation_stops(ctx):
    m = load(ctx, "tiny_llama_c")
    e = ts5hip.Engine(m)
    ids, _ = e.generate(SPEC["prompt"], max_tokens=20, draft=0)
    stop = int(ids[5])
    first = int(np.argmax(ids == stop))
    ids2, st2 = ts5hip.Engine(m).generate(SPEC["prompt"], max_tokens=20, draft=4, eog=[stop])
    assert list(ids2) == list(ids[:first]) and st2[5] == 1


def test_logits_topk_rows(ctx):
    """The GPU pick over the rows of a verify-shaped forward: each row's top 40
    (and top 1) equal a stable descending sort of the row read on the host."""
    m = load(ctx, "tiny_llama_c")
    toks = SPEC["prompt"][:6]
    m.forward_in_place(toks[:-5], 0)
    m.ctx.check(ts5hip.lib().ts5hip_forward_in_place(m.h, toks[-5:].ctypes.data, 5, toks.size - 5, 1))
    v, i = m.logits_topk(0, 5, 40)
    v1, i1 = m.logits_topk(2, 3, 1)
    rows = m.forward_in_place(toks[-5:], toks.size - 5, all_logits=True)  # the same rows, read on the host
    for r in range(5):
        want = np.argsort(-rows[r], kind="stable")[:40]
        assert list(i[r]) == list(want) and np.array_equal(v[r], rows[r][want]), r
    assert list(i1[:, 0]) == [int(np.argmax(rows[r])) for r in range(2, 5)]
    with pytest.raises(ts5hip.Ts5HipError):
        m.logits_topk(3, 3, 5)


def test_sample_with_ties_equals_reference_heap(ctx):
    """Logits full of ties (a zero output head: every logit 0) leave the
    candidates to the order of Engine::sample's heap: the draw must then come
    from the whole row on the host and equal the oracle's restatement of
    engine/src/engine.cpp:16-46 (pinned to the reference by sampler.npz)."""
    import oracle
    hp = dict(MODELS["tiny_llama_c"]["hparams"])
    tensors = synth.model_tensors(hp, make_golden.MODEL_SEED)
    t, ne0, ne1, data = tensors["output.weight"]
    tensors["output.weight"] = (t, ne0, ne1, np.zeros_like(data))
    m = ts5hip.Model(ctx, hp, 64)
    m.set_tensors(tensors)
    lg = m.forward(SPEC["prompt"][:4], 0)[0]
    assert np.all(lg == 0)
    smp, ref = ts5hip.Sampler(9), oracle.Sampler(9)
    for k, p in ((40, 0.9), (5, 1.0), (0, 0.5)):
        for _ in range(6):
            assert m.sample(smp, 0, 0.7, p, k) == ref.sample(lg, 0.7, p, k), (k, p)
