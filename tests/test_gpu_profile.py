"""Backend::take_profile over this backend (engine/src/backend.h:40-43), with
TS5_PROFILE=1 set when the model is made: GPU time per kernel and weight role,
as ts5's per-dispatch timestamps report it (engine/src/vk_backend.cpp:347-358,
:737-749, :926-932).

Bars: every launch of a decode token and of a prompt batch appears under its
kernel and weight role with the exact launch count the token loop makes
(n_layer per layer kernel and token, one head per token), with the token's
kernels replayed as a HIP graph (an event node after each) or launched
directly; so does a verify batch (its own graph); the per-kernel times add
up to no more than the forward calls' GPU time; the profiled run computes
exactly what the unprofiled one computes; taking the profile empties it; a
model made without TS5_PROFILE reports nothing."""
import re

import numpy as np
import pytest

from tokenstation5_amd import synth, ts5hip

pytestmark = pytest.mark.gpu
HP = dict(synth.TINY_LLAMA_C)


@pytest.fixture(scope="module")
def ctx():
    c = ts5hip.Context(0)
    yield c
    c.close()


def model(ctx, profile, monkeypatch, graphs="1"):
    monkeypatch.setenv("TS5HIP_GRAPHS", graphs)
    if profile:
        monkeypatch.setenv("TS5_PROFILE", profile)
    else:
        monkeypatch.delenv("TS5_PROFILE", raising=False)
    m = ts5hip.Model(ctx, HP, 128)
    m.set_tensors(synth.model_tensors(HP, 21))
    assert m.token_path() == ("graphs" if graphs == "1" else "direct")
    return m


def parse(text):
    """{label: (ms, calls)} and the forward calls' GPU ms."""
    calls = re.search(r"forward calls, \d+ tokens, ([0-9.]+) ms GPU", text)
    rows = {}
    for line in text.splitlines():
        m = re.match(r"\s+(\S+(?: \S+)?)\s+([0-9.]+) ms\s+[0-9.]+%\s+(\d+) calls", line)
        if m:
            rows[m.group(1)] = (float(m.group(2)), int(m.group(3)))
    return rows, float(calls.group(1)) if calls else None


@pytest.mark.parametrize("graphs", ["1", "0"])
def test_profile_per_kernel(ctx, monkeypatch, graphs):
    L = HP["n_layer"]
    prompt = np.arange(3, 40, dtype=np.int32)
    plain = model(ctx, None, monkeypatch, graphs)
    want = plain.forward(prompt, 0)[0]
    want_ids = plain.generate_greedy(int(np.argmax(want)), prompt.size, 8)
    batch = np.array([5, 9, 11, 13, 17], np.int32)
    want_batch = plain.forward(batch, prompt.size + 8, all_logits=True)
    assert plain.take_profile() == ""
    plain.close()

    m = model(ctx, "1", monkeypatch, graphs)
    got = m.forward(prompt, 0)[0]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    pf, total = parse(m.take_profile())
    assert pf["embed_q4_k token_embd"][1] == 1
    assert pf.get("attention_prompt", (0, 0))[1] == L or pf.get("attention_q8 batch", (0, 0))[1] == L, pf
    assert any(k.endswith(" attn_qkv") and k.startswith(("matmul", "act_quant")) for k in pf), pf
    assert sum(v[0] for v in pf.values()) <= total * 1.01 + 0.05

    ids = m.generate_greedy(int(np.argmax(got)), prompt.size, 8)
    assert list(ids) == list(want_ids)
    text = m.take_profile()
    pf, total = parse(text)
    print(text)
    for label in ("matvec_q4_k attn_qkv", "attention_q8 decode", "matvec_q4_k attn_output",
                  "matvec_glu_q4_k ffn_gate+up", "matvec_q4_k ffn_down"):
        assert pf[label][1] == 8 * L, (label, pf.get(label))
    assert pf["matvec_argmax_q6_k output"][1] == 8 and pf["embed_q4_k token_embd"][1] == 8
    assert all(v[0] > 0 for v in pf.values())
    assert sum(v[0] for v in pf.values()) <= total * 1.01 + 0.05

    got_batch = m.forward(batch, prompt.size + 8, all_logits=True)
    assert np.array_equal(got_batch.view(np.uint32), want_batch.view(np.uint32))
    pf, total = parse(m.take_profile())
    att = [v[1] for k, v in pf.items() if k.startswith("attention")]
    assert sum(att) == L, pf
    assert any(k.endswith(" ffn_down") for k in pf) and all(v[0] > 0 for v in pf.values()), pf
    assert sum(v[0] for v in pf.values()) <= total * 1.01 + 0.05
    assert m.take_profile() == ""
    m.close()
