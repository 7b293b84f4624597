"""The GGML matrix types beyond Q4_K / Q6_K / Q8_0 that ts5 runs on its GPU
(engine/src/vk_backend.cpp:156-170: Q4_0, Q4_1, Q5_0, Q5_1, Q5_K, F16, F32),
through the C ABI. The quantized ones are unpacked at upload into one exact
layout (int8 quants, an fp32 scale and min per 32 values) that the Q8_0
kernels read with a min term; F16 / F32 rows have a matvec of their own (the
one-token kernel per token in batches).

Bars: unpack bit-exact against the reference's own dequantize_row outputs
(tests/golden/quants.npz, written from engine/src/quants.cpp by
make_golden.py) and against the oracle on random blocks; one-token matvec in
every mode (plain, residual, fused norm + gate/up + SiLU, greedy pick) and
several-token matmuls (1-16 tokens, and a 70-token prompt chunk) within the
same bars as Q8_0's (relative L2 <= 1e-3, and <= 2e-6 where the 23-bit
activation is the only rounding); a model whose every matrix role takes
these types (q, k and v of different types in one layer) gives the oracle's
logits within the reference's q8 check bar and its greedy tokens, and loads
from a GGUF file to the same logits."""
import os

import numpy as np
import pytest

import gguf_writer
import oracle
from tokenstation5_amd import synth, ts5hip

pytestmark = pytest.mark.gpu
G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NEW = [synth.Q4_0, synth.Q4_1, synth.Q5_0, synth.Q5_1, synth.Q5_K]
FLOAT = [synth.F16, synth.F32]


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


@pytest.fixture(scope="module")
def ctx():
    c = ts5hip.Context(0)
    yield c
    c.close()


def test_supported():
    for t in NEW + FLOAT:
        assert ts5hip.lib().ts5hip_supports_type(t) == 1, t
    # An int8 byte and 8 bytes of (scale, min) per 32 values, each array on 256-byte boundaries.
    assert ts5hip.lib().ts5hip_weight_bytes(synth.Q4_0, 4096, 64) == 4096 * 64 + 4096 * 64 // 32 * 8
    assert ts5hip.lib().ts5hip_weight_bytes(synth.Q5_K, 96, 1) < 0  # not whole 256-value blocks


@pytest.mark.parametrize("t", NEW)
def test_dequantize_bit_exact_golden(ctx, t):
    """HBM-layout unpack == the reference's dequantize_row on its golden
    blocks (zero, subnormal, negative and large f16 scales and mins)."""
    q = np.load(os.path.join(G, "quants.npz"))
    blocks, want = q[f"t{t}_blocks"], q[f"t{t}_values"]
    ne0 = synth.BLOCK[t][0]
    rows = blocks.shape[0]
    w = ctx.weight(t, ne0, rows, blocks.reshape(rows, -1))
    y = ctx.alloc(want.nbytes)
    ctx.dequantize(t, w, ne0, rows, y)
    got = y.download(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("t", NEW)
def test_dequantize_bit_exact_random(ctx, t):
    ne0, rows = 4096, 24
    W = synth.tensor(t, ne0, rows, 31, f"deq_new{t}")
    w = ctx.weight(t, ne0, rows, W)
    y = ctx.alloc(ne0 * rows * 4)
    ctx.dequantize(t, w, ne0, rows, y)
    got = y.download(np.float32).reshape(rows, ne0)
    want = np.stack([oracle.dequantize(t, W[r], ne0) for r in range(rows)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t", NEW + FLOAT)
@pytest.mark.parametrize("ne0,rows", [(4096, 1024), (896, 4864), (512, 37)])
def test_matvec_modes(ctx, t, ne0, rows):
    if ne0 % synth.BLOCK[t][0]:
        pytest.skip("rows of whole blocks")
    rng = np.random.default_rng(ne0 * 7 + rows + t)
    W = synth.tensor(t, ne0, rows, 41, f"mvn{t}_{ne0}")
    U = synth.tensor(t, ne0, rows, 42, f"mvu{t}_{ne0}")
    x = rng.standard_normal(ne0).astype(np.float32)
    nw = (1 + 0.02 * rng.standard_normal(ne0)).astype(np.float32)
    w, u = ctx.weight(t, ne0, rows, W), ctx.weight(t, ne0, rows, U)
    want = oracle.matmul(t, W, ne0, x)[0]
    y = ctx.alloc(rows * 4)
    ctx.matvec(t, w, ne0, rows, ctx.to_device(x), y)
    got = y.download(np.float32)
    assert rel_l2(got, want) <= 2e-6, rel_l2(got, want)
    y0 = rng.standard_normal(rows).astype(np.float32)
    ya = ctx.to_device(y0)
    ctx.matvec(t, w, ne0, rows, ctx.to_device(x), ya, accumulate=True)
    assert rel_l2(ya.download(np.float32), y0 + want) <= 2e-6
    h = oracle.rmsnorm(x, nw, 1e-6)
    wg = oracle.swiglu(oracle.matmul(t, W, ne0, h)[0], oracle.matmul(t, U, ne0, h)[0])
    yg = ctx.alloc(rows * 4)
    ctx.matvec_glu(t, w, u, ne0, rows, ctx.to_device(x), yg, norm_w=ctx.to_device(nw), eps=1e-6)
    assert rel_l2(yg.download(np.float32), wg) <= 1e-5
    out = ctx.alloc(4)
    yl = ctx.alloc(rows * 4)
    ctx.matvec_argmax(t, w, ne0, rows, ctx.to_device(x), yl, out)
    logits = yl.download(np.float32)
    assert int(out.download(np.int32)[0]) == int(np.argmax(logits))
    assert rel_l2(logits, want) <= 2e-6


@pytest.mark.parametrize("t", NEW + FLOAT)
@pytest.mark.parametrize("M", [1, 5, 16, 70])
def test_matmul_tokens(ctx, t, M):
    """Several tokens: k_gemm_small up to 16, the int8 matrix-core k_gemm past
    it; F16 / F32 rows the one-token matvec per token."""
    ne0, rows = 1536, 520
    rng = np.random.default_rng(M + 10 * t)
    W = synth.tensor(t, ne0, rows, 51, f"mm{t}")
    U = synth.tensor(t, ne0, rows, 52, f"mmu{t}")
    x = rng.standard_normal((M, ne0)).astype(np.float32)
    w, u = ctx.weight(t, ne0, rows, W), ctx.weight(t, ne0, rows, U)
    y = ctx.alloc(M * rows * 4)
    ctx.matmul(t, w, ne0, rows, ctx.to_device(x), M, y)
    want = oracle.matmul(t, W, ne0, x)
    got = y.download(np.float32, (M, rows))
    for k in range(M):
        assert rel_l2(got[k], want[k]) <= 2e-6, (k, rel_l2(got[k], want[k]))
    yg = ctx.alloc(M * rows * 4)
    ctx.matmul_glu(t, w, u, ne0, rows, ctx.to_device(x), M, yg)
    wg = oracle.swiglu(want, oracle.matmul(t, U, ne0, x))
    gg = yg.download(np.float32, (M, rows))
    for k in range(M):
        assert rel_l2(gg[k], wg[k]) <= 1e-5, (k, rel_l2(gg[k], wg[k]))


# A model whose matrices take every new type: per layer q, k and v of
# different types (q and k first in the shared buffer, then v of another type
# moves them apart), wo, gate/up, down; token_embd and the head too.
HP = dict(synth.TINY_LLAMA)
TYPES = {
    "token_embd.weight": synth.Q4_0,
    "output.weight": synth.Q5_1,
    "blk.0.attn_q.weight": synth.Q5_0, "blk.0.attn_k.weight": synth.Q5_0, "blk.0.attn_v.weight": synth.Q8_0,
    "blk.0.attn_output.weight": synth.Q4_1, "blk.0.ffn_gate.weight": synth.Q5_K, "blk.0.ffn_up.weight": synth.Q5_K,
    "blk.0.ffn_down.weight": synth.Q5_1,
    "blk.1.attn_q.weight": synth.Q4_1, "blk.1.attn_k.weight": synth.Q5_1, "blk.1.attn_v.weight": synth.Q5_K,
    "blk.1.attn_output.weight": synth.Q5_K, "blk.1.ffn_gate.weight": synth.Q4_0, "blk.1.ffn_up.weight": synth.Q4_0,
    "blk.1.ffn_down.weight": synth.Q4_K,
}


# Float matrices in every role that can hold one: the head (F16), attention
# output (F32), q / k / v, gate / up (F16) and down (F32).
FLOAT_TYPES = {
    "output.weight": synth.F16, "blk.0.attn_output.weight": synth.F32, "blk.1.attn_q.weight": synth.F16,
    "blk.1.attn_k.weight": synth.F16, "blk.1.attn_v.weight": synth.F16, "blk.1.ffn_gate.weight": synth.F16,
    "blk.1.ffn_up.weight": synth.F16, "blk.1.ffn_down.weight": synth.F32,
}


def mixed_tensors(seed=61, types=TYPES):
    tensors = synth.model_tensors(HP, seed)
    for name, t in types.items():
        _, ne0, ne1, _ = tensors[name]
        if t in FLOAT:  # N(0, 0.05^2) values, the quantized matrices' scale
            v = np.random.default_rng([seed, ne0, ne1, t]).standard_normal((ne1, ne0)) * 0.05
            raw = np.ascontiguousarray(v.astype(np.float16 if t == synth.F16 else np.float32)).view(np.uint8)
            tensors[name] = (t, ne0, ne1, raw.reshape(ne1, -1))
        else:
            tensors[name] = (t, ne0, ne1, synth.tensor(t, ne0, ne1, seed, name))
    return tensors


@pytest.mark.parametrize("kv,types", [(ts5hip.KV_F16, "quant"), (ts5hip.KV_Q8, "quant"), (ts5hip.KV_F16, "float")])
def test_mixed_type_model(ctx, tmp_path, kv, types):
    tensors = mixed_tensors(types=TYPES if types == "quant" else dict(TYPES, **FLOAT_TYPES))
    m = ts5hip.Model(ctx, HP, 96, kv)
    m.set_tensors(tensors)
    ref = oracle.Model(HP, tensors, 96, kv)
    prompt = np.random.default_rng(3).integers(0, HP["n_vocab"], 40).astype(np.int32)
    got = m.forward(prompt, 0, all_logits=True)  # prompt chunk: the matrix-core matmuls
    want = ref.forward(prompt, 0, all_logits=True)
    for r in range(prompt.size):
        d = np.abs(got[r].astype(np.float64) - want[r]).max() / np.abs(want[r]).max()
        assert d <= (2e-2 if kv == ts5hip.KV_Q8 else 5e-3), (r, d)
    first = int(np.argmax(got[-1]))
    assert first == int(np.argmax(want[-1]))
    ids = m.generate_greedy(first, prompt.size, 12)  # one-token matvecs, graph replay
    tok, exp = first, []
    for i in range(12):
        tok = int(np.argmax(ref.forward(np.array([tok], np.int32), prompt.size + i)[0]))
        exp.append(tok)
    if kv == ts5hip.KV_F16:
        assert list(ids) == exp
    else:
        assert list(ids)[:4] == exp[:4]  # q8 rounding steps may part them later, as for Q4_K models
    # The same tensors from a GGUF file load to the same logits.
    path = str(tmp_path / "mixed.gguf")
    gguf_writer.write(path, gguf_writer.model_kv(HP), tensors)
    f = ts5hip.load_model(ctx, path, n_ctx=96, kv=kv)
    assert np.array_equal(f.forward(prompt, 0, all_logits=True).view(np.uint32), got.view(np.uint32))
    f.close()
    m.close()
