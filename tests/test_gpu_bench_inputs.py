"""The benchmark's own plumbing, through the C ABI: the synthetic KV caches
cfg3 times attention on (ts5hip_kv_synth) and the per-launch event marks
behind cfg1's median (ts5hip_timer_mark / ts5hip_timer_marks).

Bars: a q8 cache is what the q8 rule makes of N(0,1) values (per 32 values
the scale is an f16 and the largest |q| is exactly 127, engine/src/
cpu_backend.cpp:78-90), with the values' mean and spread of N(0,1); an f16
cache holds N(0,1) values; the same seed gives the same cache; marks give one
positive interval per launch between them."""
import numpy as np
import pytest

from tokenstation5_amd import ts5hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = ts5hip.Context(0)
    yield c
    c.close()


def test_kv_synth_q8_and_f16(ctx):
    n = 32 * 4096
    v, s = ctx.alloc(n), ctx.alloc(n // 16)
    ctx.kv_synth(5, n, ts5hip.KV_Q8, v, s)
    q = v.download(np.int8).astype(np.int32).reshape(-1, 32)
    sc = s.download(np.float16).astype(np.float64)
    assert (sc > 0).all() and (np.abs(q).max(axis=1) == 127).all()
    x = q * sc[:, None]
    assert abs(x.mean()) < 0.02 and abs(x.std() - 1) < 0.02
    # The largest |value| of a block of 32 N(0,1) draws: 2.347 on average
    # (the mean over these 4096 blocks has a spread of about 0.007).
    assert 2.30 < (127 * sc).mean() < 2.40
    v2, s2 = ctx.alloc(n), ctx.alloc(n // 16)
    ctx.kv_synth(5, n, ts5hip.KV_Q8, v2, s2)
    assert np.array_equal(v2.download(np.int8), q.reshape(-1).astype(np.int8))
    h = ctx.alloc(2 * n)
    ctx.kv_synth(6, n, ts5hip.KV_F16, h)
    f = h.download(np.float16).astype(np.float64)
    assert np.isfinite(f).all() and abs(f.mean()) < 0.02 and abs(f.std() - 1) < 0.02
    with pytest.raises(ts5hip.Ts5HipError):
        ctx.kv_synth(5, 33, ts5hip.KV_Q8, v, s)


def test_timer_marks(ctx):
    x = ctx.to_device(np.ones(4096 * 256, np.float32))
    y = ctx.alloc(4096 * 256 * 4)
    w = ctx.to_device(np.ones(4096, np.float32))
    for i in range(5):
        ctx.timer_mark(i)
        ctx.rmsnorm(x, w, 1e-5, 4096, 256, y)
    ctx.timer_mark(5)
    ms = ctx.timer_marks(6)
    assert ms.shape == (5,) and (ms > 0).all() and (ms < 100).all()
