"""The CPU oracle pinned against ts5's own CPU code (golden vectors made by
tests/golden/make_golden.py from engine/src/*.cpp) and against closed forms.

These run on the CPU only."""
import hashlib
import json
import os

import numpy as np
import pytest

import make_golden
import oracle
from tokenstation5_amd import synth

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_fp16_to_fp32_all_halves():
    f = np.load(os.path.join(G, "fp16.npz"))
    L = oracle.lib()
    h2f = np.array([L.ts5o_fp16_to_fp32(h) for h in range(65536)], np.float32).view(np.uint32)
    assert np.array_equal(h2f[:4096], f["h2f_head"])
    assert sha(h2f) == str(f["h2f_sha"])
    # Closed form: every finite half is exactly numpy's float16 value.
    ref = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32).view(np.uint32)
    finite = np.isfinite(np.arange(65536, dtype=np.uint16).view(np.float16))
    assert np.array_equal(h2f[finite], ref[finite])


def test_fp32_to_fp16_rounding():
    f = np.load(os.path.join(G, "fp16.npz"))
    xs = make_golden.fp16_inputs(int(f["f2h_seed"]))
    assert sha(xs) == str(f["f2h_inputs_sha"])
    L = oracle.lib()
    got = np.array([L.ts5o_fp32_to_fp16(float(v)) for v in xs.view(np.float32)], np.uint16)
    assert np.array_equal(got[:4096], f["f2h_head"])
    assert sha(got) == str(f["f2h_sha"])
    # Closed form: numpy's float32 -> float16 is IEEE round-to-nearest-even.
    v = xs.view(np.float32)
    ok = ~np.isnan(v)
    with np.errstate(over="ignore"):
        assert np.array_equal(got[ok], v[ok].astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("t", [synth.Q4_0, synth.Q4_1, synth.Q5_0, synth.Q5_1, synth.Q8_0, synth.Q4_K, synth.Q5_K,
                               synth.Q6_K, synth.F16, synth.BF16])
def test_dequantize_matches_reference(t):
    q = np.load(os.path.join(G, "quants.npz"))
    blocks, want = q[f"t{t}_blocks"], q[f"t{t}_values"]
    got = oracle.dequantize(t, blocks, want.size)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q4_k_closed_form():
    """y = d*sc*q - dmin*m per sub-block, from the fields unpacked by hand."""
    rng = np.random.default_rng(3)
    sc = rng.integers(0, 64, (32, 8))
    m = rng.integers(0, 64, (32, 8))
    b = synth.blocks(synth.Q4_K, 32, rng)
    b[:, 4:16] = synth.pack_scale_min(sc, m)
    got = oracle.dequantize(synth.Q4_K, b, 32 * 256).reshape(32, 8, 32)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    qs = b[:, 16:].reshape(32, 4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=2).reshape(32, 8, 32)  # sub-block 2g low, 2g+1 high
    want = (d[:, None] * sc).astype(np.float32)[:, :, None] * q - (dmin[:, None] * m).astype(np.float32)[:, :, None]
    assert np.array_equal(got, want.astype(np.float32))


def test_q6_k_closed_form():
    rng = np.random.default_rng(4)
    b = synth.blocks(synth.Q6_K, 16, rng)
    got = oracle.dequantize(synth.Q6_K, b, 16 * 256).reshape(16, 2, 4, 32)
    d = b[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
    for blk in range(16):
        for h in range(2):
            ql, qh = b[blk, 64 * h:64 * h + 64].astype(int), b[blk, 128 + 32 * h:160 + 32 * h].astype(int)
            sc = b[blk, 192 + 8 * h:200 + 8 * h].view(np.int8).astype(int)
            for c in range(4):
                low = (ql[32 * (c & 1):32 * (c & 1) + 32] >> (4 * (c >> 1))) & 15
                q = low | (((qh >> (2 * c)) & 3) << 4)
                s = np.repeat(sc[2 * c:2 * c + 2], 16)
                want = (np.float32(d[blk]) * s.astype(np.float32)) * (q - 32).astype(np.float32)
                assert np.array_equal(got[blk, h, c], want.astype(np.float32)), (blk, h, c)


def test_matmul_brute_force():
    """The fp64-accumulated matvec against numpy in float64 over the same
    dequantized rows (a transposed operand or dropped block fails)."""
    rows, ne0 = 96, 1024
    for t in (synth.Q4_K, synth.Q6_K, synth.Q8_0):
        w = synth.tensor(t, ne0, rows, 5, "m")
        x = np.random.default_rng(6).standard_normal((3, ne0)).astype(np.float32)
        y = oracle.matmul(t, w, ne0, x, threads=3)
        deq = np.stack([oracle.dequantize(t, w[r], ne0) for r in range(rows)]).astype(np.float64)
        want = x.astype(np.float64) @ deq.T
        assert np.allclose(y, want, rtol=1e-6, atol=1e-6 * np.abs(want).max())


def test_rmsnorm_closed_form():
    x = np.random.default_rng(1).standard_normal(4096).astype(np.float32) * 1e3
    w = (1 + 0.02 * np.random.default_rng(2).standard_normal(4096)).astype(np.float32)
    got = oracle.rmsnorm(x, w, 1e-5)
    s = np.float32(1.0) / np.sqrt(np.float32(np.mean(x.astype(np.float64) ** 2)) + np.float32(1e-5))
    assert np.allclose(got, x * s * w, rtol=1e-6)


def test_round_kv_q8_properties():
    rng = np.random.default_rng(8)
    v = (rng.standard_normal(4096) * rng.choice([1e-3, 1, 1e4], 4096)).astype(np.float32)
    r = oracle.round_kv(2, v).reshape(-1, 32)
    vb = v.reshape(-1, 32)
    sc = (np.abs(vb).max(1) / np.float32(127)).astype(np.float16).astype(np.float32)
    q = r / sc[:, None]
    assert np.array_equal(q, np.rint(q))           # integers times the f16 scale
    assert np.abs(q).max() <= 127
    assert np.array_equal(q, np.clip(np.rint(vb / sc[:, None]), -127, 127))  # nearest, ties to even
    assert np.array_equal(oracle.round_kv(1, v), v.astype(np.float16).astype(np.float32))


def test_rope_rotation():
    v = np.random.default_rng(9).standard_normal(128).astype(np.float32)
    assert np.array_equal(oracle.rope(v, 128, 0, 500000.0, False), v)  # position 0: identity
    for neox in (False, True):
        r = oracle.rope(v, 128, 1234, 500000.0, neox)
        assert np.isclose(np.linalg.norm(r), np.linalg.norm(v), rtol=1e-5)
        c, s = oracle.rope_cs(128, 1234, 500000.0)
        a = np.arange(64) if neox else 2 * np.arange(64)
        b = a + 64 if neox else a + 1
        assert np.array_equal(r[a], (v[a] * c - v[b] * s).astype(np.float32))
        assert np.array_equal(r[b], (v[a] * s + v[b] * c).astype(np.float32))
    # The frequency of pair i is base^(-2i/n): pair 0 turns by `pos` radians.
    c, s = oracle.rope_cs(128, 3, 500000.0)
    assert np.isclose(c[0], np.cos(3.0)) and np.isclose(s[0], np.sin(3.0))


def test_attention_softmax():
    H, HKV, HD, n = 8, 2, 64, 37
    rng = np.random.default_rng(10)
    q = rng.standard_normal(H * HD).astype(np.float32)
    kc = rng.standard_normal((n, HKV * HD)).astype(np.float32)
    vc = rng.standard_normal((n, HKV * HD)).astype(np.float32)
    got = oracle.attention(q, kc, vc, H, HKV, HD, n - 1, 0.125)
    for h in range(H):
        kh = h // (H // HKV)
        s = kc[:, kh * HD:(kh + 1) * HD].astype(np.float64) @ q[h * HD:(h + 1) * HD] * 0.125
        p = np.exp(s - s.max())
        want = (p / p.sum()) @ vc[:, kh * HD:(kh + 1) * HD].astype(np.float64)
        assert np.allclose(got[h * HD:(h + 1) * HD], want, rtol=1e-5, atol=1e-6)


def test_attention_window():
    """lo > 0 (a sliding layer's window): the softmax over keys lo..pos only."""
    H, HKV, HD, n, lo = 4, 1, 256, 30, 22
    rng = np.random.default_rng(12)
    q = rng.standard_normal(H * HD).astype(np.float32)
    kc = rng.standard_normal((n, HKV * HD)).astype(np.float32)
    vc = rng.standard_normal((n, HKV * HD)).astype(np.float32)
    got = oracle.attention(q, kc, vc, H, HKV, HD, n - 1, 0.0625, lo=lo)
    want = oracle.attention(q, kc[lo:], vc[lo:], H, HKV, HD, n - 1 - lo, 0.0625)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-7)
    # A window of one key returns that key's values.
    one = oracle.attention(q, kc, vc, H, HKV, HD, n - 1, 0.0625, lo=n - 1)
    assert np.allclose(one, np.tile(vc[n - 1], H), rtol=0, atol=1e-7)


def test_geglu_against_erf_gelu():
    """The tanh form of GELU stays within 1e-3 of x * Phi(x) (its published
    error is a few 1e-4), is 0 at 0, x for large x and 0 for very negative x."""
    from scipy.special import erf
    x = np.linspace(-8, 8, 4001).astype(np.float32)
    u = np.ones_like(x)
    got = oracle.geglu(x, u).astype(np.float64)
    exact = 0.5 * x * (1 + erf(x / np.sqrt(2.0)))
    assert np.abs(got - exact).max() < 1e-3
    assert oracle.geglu(np.float32([0.0]), np.float32([3.0]))[0] == 0.0
    big = oracle.geglu(np.float32([12.0, -12.0]), np.float32([2.0, 2.0]))
    assert big[0] == 24.0 and abs(big[1]) < 1e-30
    # The up projection multiplies.
    assert np.allclose(oracle.geglu(x, 3 * u), 3 * got, rtol=1e-6, atol=1e-7)


def _check_model(name):
    hp = dict(json.load(open(os.path.join(G, "models.json")))[name]["hparams"])
    digests = json.load(open(os.path.join(G, "models.json")))[name]["tensor_sha256"]
    tensors = synth.model_tensors(hp, make_golden.MODEL_SEED)
    assert {k: sha(v[3]) for k, v in tensors.items()} == digests
    g = np.load(os.path.join(G, f"model_{name}.npz"))
    for kv in (0, 1, 2):  # f32, f16 and q8 caches
        toks, want = g[f"kv{kv}_tokens"], g[f"kv{kv}_logits"]
        m = oracle.Model(hp, tensors, 64, kv)
        n = toks.size
        batch = n - 4
        got = np.empty_like(want)
        got[:batch] = m.forward(toks[:batch], 0, all_logits=True)
        for i in range(batch, n):
            got[i] = m.forward(toks[i:i + 1], i)[0]
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, kv)
    return hp, tensors, g


@pytest.mark.parametrize("name", ["tiny_llama", "tiny_draft", "tiny_llama_c", "tiny_draft_c", "tiny_gemma3",
                                  "tiny_qwen3", "tiny_llama31"])
def test_model_logits_match_reference(name):
    _check_model(name)


@pytest.mark.parametrize("name", ["tiny_llama_c", "tiny_draft_c", "tiny_gemma3", "tiny_qwen3", "tiny_llama31"])
@pytest.mark.parametrize("kv,key", [(2, "greedy_q8_ids"), (1, "greedy_f16_ids")])
def test_greedy_decode_matches_reference(name, kv, key):
    hp = dict(json.load(open(os.path.join(G, "models.json")))[name]["hparams"])
    g = np.load(os.path.join(G, f"model_{name}.npz"))
    m = oracle.Model(hp, synth.model_tensors(hp, make_golden.MODEL_SEED), 128, kv)
    prompt = g["greedy_prompt"]
    lg = m.forward(prompt, 0)[0]
    ids = []
    for i in range(64):
        ids.append(int(np.argmax(lg)))
        lg = m.forward(np.array([ids[-1]]), prompt.size + i)[0]
    assert ids == list(g[key])


def test_sampler_matches_reference():
    s = np.load(os.path.join(G, "sampler.npz"))
    table = make_golden.sampler_table(int(s["table_seed"]), int(s["rows"]), int(s["n_vocab"]))
    assert sha(table) == str(s["table_sha"])
    for i, (T, p, k) in enumerate(make_golden.SAMPLER_CASES):
        smp = oracle.Sampler(42 + i)
        got = [smp.sample(table[r], T, p, k) for r in range(table.shape[0])]
        assert got == list(s[f"ids{i}"]), i
        # The same draws from the top-k candidates alone (what a GPU top-k hands over).
        if T > 0 and k > 0:
            smp = oracle.Sampler(42 + i)
            got2 = []
            for r in range(table.shape[0]):
                ids = np.argsort(-table[r], kind="stable")[:k].astype(np.int32)
                got2.append(smp.sample_topk(ids, table[r][ids], T, p))
            assert got2 == got, i
