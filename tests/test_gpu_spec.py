"""cfg5's speculative decoding at its stated shapes, through the decode driver
(ts5hip_engine_generate): the 24-layer, 896-wide Q8_0 draft model (vocab
151936, tied head) proposing k = 4 tokens per step for the 48-layer,
5120-wide, 40/8-head Q4_K target (vocab 151936, Q6_K head) and for the
32-layer 8B of cfg2, after a 2048-token prompt of uniform ids, 128 generated
tokens (engine/src/engine.cpp:75-129, :186-195; the reference's own run,
engine/tests/run.sh:222-229).

Bars: the greedy output with drafting is the output without it, token for
token (a draft is kept only when the target's own pick equals it,
engine/src/engine.cpp:186-190), and speculation did happen (drafted > 0;
with the target itself as the draft model, drafts were also accepted).
Weights are centred Q4_K (synth.blocks), so the targets' picks follow their
input and prompt lookup seldom finds a match: the draft model does the
drafting."""
import numpy as np
import pytest

from tokenstation5_amd import synth, ts5hip

pytestmark = pytest.mark.gpu
PROMPT = 2048
GEN = 128


@pytest.fixture(scope="module")
def ctx():
    c = ts5hip.Context(0)
    yield c
    c.close()


def synth_model(ctx, hp, n_ctx, seed):
    m = ts5hip.Model(ctx, hp, n_ctx)
    for name, t, ne0, ne1 in synth.tensor_specs(hp):
        m.synth_tensor(name, t, ne0, ne1, seed, centered=True)
    return m


@pytest.fixture(scope="module")
def drafter(ctx):
    m = synth_model(ctx, synth.DRAFT_0P5B, PROMPT + GEN + 16, 51)
    yield m
    m.close()


TARGETS = {"target_48x5120": synth.TARGET_14B, "llama_8b": synth.LLAMA_8B}


@pytest.mark.parametrize("name", list(TARGETS))
def test_draft_model_keeps_greedy_output(ctx, drafter, name):
    hp = TARGETS[name]
    target = synth_model(ctx, hp, PROMPT + GEN + 16, 52)
    prompt = np.random.default_rng(5).integers(0, hp["n_vocab"], PROMPT).astype(np.int32)
    base_ids, base_st = ts5hip.Engine(target).generate(prompt, temperature=0.0, max_tokens=GEN, draft=0)
    e = ts5hip.Engine(target)
    e.set_drafter(drafter)
    ids, st = e.generate(prompt, temperature=0.0, max_tokens=GEN, draft=4)
    print(f"{name}: drafted {st[3]}, accepted {st[4]}; ids[:8] {list(ids[:8])}, "
          f"{np.unique(ids).size} distinct of {ids.size}")
    assert list(ids) == list(base_ids)
    assert st[2] == GEN and st[3] > 0 and base_st[3] == 0
    e.close()
    target.close()


def test_self_draft_is_accepted(ctx):
    """The target as its own draft model (a second instance of the same
    weights; the reference's self-draft run): the drafts are its single-token
    greedy picks, which the batched verify forward reproduces almost always."""
    hp = TARGETS["llama_8b"]
    target = synth_model(ctx, hp, PROMPT + GEN + 16, 53)
    twin = synth_model(ctx, hp, PROMPT + GEN + 16, 53)
    prompt = np.random.default_rng(6).integers(0, hp["n_vocab"], PROMPT).astype(np.int32)
    base_ids, _ = ts5hip.Engine(target).generate(prompt, temperature=0.0, max_tokens=GEN, draft=0)
    e = ts5hip.Engine(target)
    e.set_drafter(twin)
    ids, st = e.generate(prompt, temperature=0.0, max_tokens=GEN, draft=4)
    print(f"self-draft: drafted {st[3]}, accepted {st[4]}")
    assert list(ids) == list(base_ids)
    assert st[3] > 0 and st[4] >= 0.8 * st[3]
    e.close()
    twin.close()
    target.close()
