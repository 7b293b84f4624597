"""The several-token projections (ts5hip_matmul, ts5hip_matmul_glu: the
speculative verify step and prompt chunks) against the oracle's fp64 matmul
(engine/src/cpu_backend.cpp:18-41 at n > 1), through the C ABI.

Bars: rel-L2 <= 1e-3 per token against the oracle, like the one-token
matvec; and against that matvec, row by row, the same integer products in
another summation order (rel-L2 <= 2e-5)."""
import numpy as np
import pytest

import oracle
from tokenstation5_amd import synth, ts5hip

pytestmark = pytest.mark.gpu
REL_L2 = 1e-3


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


@pytest.fixture(scope="module")
def ctx():
    c = ts5hip.Context(0)
    yield c
    c.close()


def run_matmul(ctx, t, W, ne0, rows, x, norm=None, eps=1e-5, accumulate=None):
    ntok = x.shape[0]
    w = ctx.weight(t, ne0, rows, W)
    y = ctx.to_device(accumulate if accumulate is not None else np.zeros((ntok, rows), np.float32))
    ctx.matmul(t, w, ne0, rows, ctx.to_device(x), ntok, y, norm_w=None if norm is None else ctx.to_device(norm),
               eps=eps, accumulate=accumulate is not None)
    return y.download(np.float32, (ntok, rows)).reshape(ntok, rows)


SHAPES = [
    (synth.Q4_K, 4096, 1024),
    (synth.Q4_K, 14336, 512),   # ffn_down: 56 blocks a row
    (synth.Q4_K, 256, 37),      # one block, ragged rows
    (synth.Q6_K, 4096, 515),
    (synth.Q6_K, 512, 1000),
    (synth.Q8_0, 896, 300),     # the draft's 896-wide matrices
    (synth.Q8_0, 4864, 128),
]


@pytest.mark.parametrize("t,ne0,rows", SHAPES)
@pytest.mark.parametrize("ntok", [1, 2, 5, 16, 17, 70])
def test_matmul_vs_oracle(ctx, t, ne0, rows, ntok):
    W = synth.tensor(t, ne0, rows, 1, f"mm{t}_{ne0}_{rows}")
    x = np.random.default_rng(ne0 + rows + ntok).standard_normal((ntok, ne0)).astype(np.float32)
    got = run_matmul(ctx, t, W, ne0, rows, x)
    want = oracle.matmul(t, W, ne0, x)
    for i in range(ntok):
        assert rel_l2(got[i], want[i]) <= REL_L2, (i, rel_l2(got[i], want[i]))


@pytest.mark.parametrize("t,ne0,rows", [(synth.Q4_K, 4096, 1000), (synth.Q4_K, 14336, 256), (synth.Q4_K, 256, 37)])
@pytest.mark.parametrize("ntok", [17, 64, 65, 130, 256])
def test_matmul_prompt_q4k_vs_oracle(ctx, t, ne0, rows, ntok):
    """Q4_K batches past 16 tokens take the fp16 matrix-core path (activations
    as hi + lo fp16 planes, about 22 bits): ragged token tiles of 64 and row
    tiles of 128, one-block rows, split-K over 56 blocks. Its error is far
    below the shared bar, so it is held to 2e-5."""
    W = synth.tensor(t, ne0, rows, 7, f"pf{ne0}_{rows}")
    x = np.random.default_rng(ne0 + 3 * rows + ntok).standard_normal((ntok, ne0)).astype(np.float32)
    got = run_matmul(ctx, t, W, ne0, rows, x)
    want = oracle.matmul(t, W, ne0, x)
    for i in range(ntok):
        assert rel_l2(got[i], want[i]) <= 2e-5, (i, rel_l2(got[i], want[i]))


@pytest.mark.parametrize("t,ne0,rows", [(synth.Q4_K, 4096, 1024), (synth.Q6_K, 4096, 515), (synth.Q8_0, 896, 300)])
def test_matmul_rows_equal_matvec(ctx, t, ne0, rows):
    """Each token's row against the one-token matvec of the same input."""
    W = synth.tensor(t, ne0, rows, 2, f"mv{t}")
    x = np.random.default_rng(3).standard_normal((9, ne0)).astype(np.float32)
    got = run_matmul(ctx, t, W, ne0, rows, x)
    w = ctx.weight(t, ne0, rows, W)
    for i in range(x.shape[0]):
        y = ctx.to_device(np.zeros(rows, np.float32))
        ctx.matvec(t, w, ne0, rows, ctx.to_device(x[i]), y)
        assert rel_l2(got[i], y.download(np.float32)) <= 2e-5, i


def test_matmul_norm_and_accumulate(ctx):
    """rmsnorm fused per token, accumulation into the residual, inputs from
    1e-6 to 1e7 across tokens (scales are per 32 values per token)."""
    rng = np.random.default_rng(8)
    ne0, rows, ntok = 4096, 640, 24
    W = synth.tensor(synth.Q4_K, ne0, rows, 4, "acc")
    x = rng.standard_normal((ntok, ne0)).astype(np.float32) * np.logspace(-6, 7, ntok, dtype=np.float32)[:, None]
    nw = (1 + 0.02 * rng.standard_normal(ne0)).astype(np.float32)
    want = oracle.matmul(synth.Q4_K, W, ne0, np.stack([oracle.rmsnorm(r, nw, 1e-5) for r in x]))
    y0 = (rng.standard_normal((ntok, rows)) * np.abs(want).mean()).astype(np.float32)
    got = run_matmul(ctx, synth.Q4_K, W, ne0, rows, x, norm=nw, accumulate=y0.copy())
    for i in range(ntok):
        assert rel_l2(got[i], y0[i].astype(np.float64) + want[i]) <= REL_L2, i
    got = run_matmul(ctx, synth.Q4_K, W, ne0, rows, x[:5] * 0)
    assert np.array_equal(got, np.zeros_like(got))


@pytest.mark.parametrize("t,ne0,rows", [(synth.Q6_K, 4096, 515), (synth.Q6_K, 512, 1000), (synth.Q8_0, 896, 300),
                                         (synth.Q8_0, 4864, 128)])
@pytest.mark.parametrize("ntok", [130, 256])
def test_matmul_prompt_chunk_vs_oracle(ctx, t, ne0, rows, ntok):
    """Q6_K and Q8_0 at prompt-chunk sizes (the int8 matrix-core path in
    64-token tiles, ragged at 130): the shared bar per token."""
    W = synth.tensor(t, ne0, rows, 9, f"pc{t}_{ne0}_{rows}")
    x = np.random.default_rng(ne0 + 5 * rows + ntok).standard_normal((ntok, ne0)).astype(np.float32)
    got = run_matmul(ctx, t, W, ne0, rows, x)
    want = oracle.matmul(t, W, ne0, x)
    for i in range(ntok):
        assert rel_l2(got[i], want[i]) <= REL_L2, (i, rel_l2(got[i], want[i]))


@pytest.mark.parametrize("t,ne0,rows", [(synth.Q4_K, 4096, 1536), (synth.Q4_K, 4096, 14336), (synth.Q8_0, 896, 4864)])
@pytest.mark.parametrize("ntok", [1, 5, 40, 256])
def test_matmul_glu_vs_oracle(ctx, t, ne0, rows, ntok):
    """silu(Wg x') * (Wu x') per token (engine/src/cpu_backend.cpp:253-261)."""
    rng = np.random.default_rng(rows + ntok)
    Wg = synth.tensor(t, ne0, rows, 5, "gate")
    Wu = synth.tensor(t, ne0, rows, 6, "up")
    x = rng.standard_normal((ntok, ne0)).astype(np.float32)
    nw = (1 + 0.02 * rng.standard_normal(ne0)).astype(np.float32)
    xn = np.stack([oracle.rmsnorm(r, nw, 1e-6) for r in x])
    want = oracle.swiglu(oracle.matmul(t, Wg, ne0, xn), oracle.matmul(t, Wu, ne0, xn))
    y = ctx.alloc(ntok * rows * 4)
    ctx.matmul_glu(t, ctx.weight(t, ne0, rows, Wg), ctx.weight(t, ne0, rows, Wu), ne0, rows, ctx.to_device(x), ntok,
                   y, norm_w=ctx.to_device(nw), eps=1e-6)
    got = y.download(np.float32, (ntok, rows)).reshape(ntok, rows)
    for i in range(ntok):
        assert rel_l2(got[i], want[i]) <= REL_L2, i


def test_matmul_rejects_bad_arguments(ctx):
    W = synth.tensor(synth.Q4_K, 256, 16, 7, "bad")
    w = ctx.weight(synth.Q4_K, 256, 16, W)
    y = ctx.alloc(16 * 4)
    x = ctx.to_device(np.zeros(256, np.float32))
    with pytest.raises(ts5hip.Ts5HipError):
        ctx.matmul(synth.Q4_K, w, 256, 16, x, 0, y)
    with pytest.raises(ts5hip.Ts5HipError):
        ctx.matmul(synth.Q4_K, w, 100, 16, x, 1, y)
