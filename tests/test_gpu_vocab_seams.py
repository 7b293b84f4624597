"""The draft model at the vocabulary seams, through the decode driver
(ts5hip_engine_generate), as ts5's own suite forces them
(engine/tests/run.sh:230-274; engine/src/engine.cpp:78-88, :122-123):

* a drafter whose weight rows are padded past the target's vocabulary, and a
  target padded past the drafter's: the output is the target's own, and the
  drafter keeps proposing (drafted and accepted > 0, still drafting);
* a target that picks a token in its pad range (past the drafter's embedding
  rows): the drafter is stopped, the output stays the target's own;
* a drafter that picks a row past the target's vocabulary: only that draft is
  lost, the drafter keeps drafting.

The drafter is the target itself with 128 padded rows (pad rows are zero
blocks: logit 0, below a centred model's largest logit), so its drafts are
mostly accepted. A "hot" pad row is a copy of a real output row with its
block scales doubled: its logit is twice that row's, so it wins wherever that
row's logit is positive and above half the maximum."""
import numpy as np
import pytest

from tokenstation5_amd import synth, ts5hip

pytestmark = pytest.mark.gpu
HP = dict(synth.TINY_LLAMA_C)
PAD = 128
SEED = 77
N_CTX = 512
GEN = 100


@pytest.fixture(scope="module")
def ctx():
    c = ts5hip.Context(0)
    yield c
    c.close()


def padded(tensors, hp, hot_from=None):
    """The model with PAD zero rows after its embedding and output rows; with
    hot_from = r, pad row 4 (token n_vocab + 4) is output row r with every
    Q6_K block's d doubled."""
    out = dict(tensors)
    for name in ("token_embd.weight", "output.weight"):
        t, ne0, ne1, rows = tensors[name]
        more = np.zeros((PAD, rows.shape[1]), np.uint8)
        if name == "output.weight" and hot_from is not None:
            assert t == synth.Q6_K
            row = rows[hot_from].copy().reshape(-1, 210)
            d = row[:, 208:210].copy().view(np.float16).astype(np.float32) * 2
            row[:, 208:210] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
            more[4] = row.reshape(-1)
        out[name] = (t, ne0, ne1 + PAD, np.concatenate([rows, more]))
    return dict(hp, n_vocab=hp["n_vocab"] + PAD), out


def model(ctx, hp, tensors):
    m = ts5hip.Model(ctx, hp, N_CTX)
    m.set_tensors(tensors)
    return m


@pytest.fixture(scope="module")
def base():
    tensors = synth.model_tensors(HP, SEED)
    prompt = np.random.default_rng(9).integers(0, HP["n_vocab"], 48).astype(np.int32)
    return tensors, prompt


def run(target, drafter, prompt):
    """(ids without drafting, ids with the drafter, stats, drafter state)."""
    plain, st0 = ts5hip.Engine(target).generate(prompt, temperature=0.0, max_tokens=GEN, draft=0)
    assert st0[3] == 0
    e = ts5hip.Engine(target)
    e.set_drafter(drafter)
    ids, st = e.generate(prompt, temperature=0.0, max_tokens=GEN, draft=7, adapt=False)
    state = e.drafter_state()
    e.close()
    return plain, ids, st, state


@pytest.mark.parametrize("wider", ["drafter", "target"])
def test_padded_vocabulary_keeps_drafting(ctx, base, wider):
    tensors, prompt = base
    php, ptensors = padded(tensors, HP)
    if wider == "drafter":
        target, drafter = model(ctx, HP, tensors), model(ctx, php, ptensors)
    else:
        target, drafter = model(ctx, php, ptensors), model(ctx, HP, tensors)
    plain, ids, st, state = run(target, drafter, prompt)
    print(f"{wider} padded: drafted {st[3]}, accepted {st[4]}, drafter state {state}")
    assert list(ids) == list(plain)
    assert state == 1 and st[3] > 0 and st[4] > 0
    target.close()
    drafter.close()


def hot_row(ctx, tensors, prompt):
    """A real token the plain model picks early, with a positive logit."""
    m = model(ctx, HP, tensors)
    lg = m.forward(prompt, 0)[0]
    first = int(np.argmax(lg))
    ids = [first] + list(m.generate_greedy(first, prompt.size, 7))
    m.close()
    assert lg[first] > 0
    return ids[0]


def test_target_pick_past_drafter_rows_stops_drafter(ctx, base):
    tensors, prompt = base
    hot = hot_row(ctx, tensors, prompt)
    php, ptensors = padded(tensors, HP, hot_from=hot)
    target, drafter = model(ctx, php, ptensors), model(ctx, HP, tensors)
    plain, ids, st, state = run(target, drafter, prompt)
    pad_tok = HP["n_vocab"] + 4
    print(f"hot target: pad token at {list(plain).index(pad_tok) if pad_tok in plain else None}, "
          f"drafted {st[3]}, accepted {st[4]}, drafter state {state}")
    assert pad_tok in list(plain)  # the target does pick into its pad range
    assert list(ids) == list(plain)
    assert state == 2  # the drafter could not embed that token: stopped
    target.close()
    drafter.close()


def test_drafter_pick_past_target_rows_loses_that_draft(ctx, base):
    tensors, prompt = base
    hot = hot_row(ctx, tensors, prompt)
    php, ptensors = padded(tensors, HP, hot_from=hot)
    target, drafter = model(ctx, HP, tensors), model(ctx, php, ptensors)
    # The padded drafter on its own does pick its pad row on this prompt.
    lg = drafter.forward(prompt, 0)[0]
    first = int(np.argmax(lg))
    alone = [first] + list(drafter.generate_greedy(first, prompt.size, GEN - 1))
    assert HP["n_vocab"] + 4 in alone
    plain, ids, st, state = run(target, drafter, prompt)
    print(f"hot drafter: drafted {st[3]}, accepted {st[4]}, drafter state {state}")
    assert list(ids) == list(plain)
    assert state == 1
    target.close()
    drafter.close()
