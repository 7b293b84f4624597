"""ts5hip_attn_decode_noalloc (the entry point that allocates nothing: its
partials and merge counters live in a static device array) against
ts5hip_attn_decode, through the C ABI: bit-identical outputs (the same kernels
and split counts) on two calls in a row, the second smaller; both within the
1e-3 relative L2 bar of the CPU oracle; a call needing more partials than the
array holds is refused."""
import numpy as np
import pytest

import oracle
from tokenstation5_amd import ts5hip

pytestmark = pytest.mark.gpu


def q8_cache(rng, B, HKV, n_ctx, HD):
    vals = rng.standard_normal((B, HKV, n_ctx, HD), dtype=np.float32)
    blocks = vals.reshape(-1, 32)
    sc = (np.abs(blocks).max(1) / np.float32(127)).astype(np.float16)
    scf = sc.astype(np.float32)
    q = np.clip(np.rint(blocks / scf[:, None]), -127, 127).astype(np.int8)
    deq = (q.astype(np.float32) * scf[:, None]).reshape(vals.shape)
    return q.reshape(vals.shape), sc.reshape(B, HKV, n_ctx, HD // 32), deq


def test_attn_decode_noalloc_matches_allocating_entry_point():
    ctx = ts5hip.Context(0)
    H, HKV, HD = 32, 8, 128
    scale = float(np.float32(1) / np.sqrt(np.float32(HD)))
    for B, n, split in ((4, 8192, 0), (1, 1000, 0), (1, 3000, 47)):  # the second call is smaller
        rng = np.random.default_rng(B * 1000 + n)
        k8, ks, kd = q8_cache(rng, B, HKV, n, HD)
        v8, vs, vd = q8_cache(rng, B, HKV, n, HD)
        q = rng.standard_normal((B, H * HD)).astype(np.float32)
        args = (ctx.to_device(q), B, H, HKV, HD, ctx.to_device(k8), ctx.to_device(ks), ctx.to_device(v8),
                ctx.to_device(vs), n, ctx.to_device(np.full(B, n, np.int32)), 1, scale)
        want_out, got_out = ctx.alloc(q.nbytes), ctx.alloc(q.nbytes)
        ctx.attn_decode(*args, want_out, n_split=split)
        ctx.attn_decode_noalloc(*args, got_out, n_split=split)
        want, got = want_out.download(np.float32, (B, H * HD)), got_out.download(np.float32, (B, H * HD))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (B, n)
        for b in range(B):
            kc = kd[b].transpose(1, 0, 2).reshape(n, HKV * HD)
            vc = vd[b].transpose(1, 0, 2).reshape(n, HKV * HD)
            ref = oracle.attention(q[b], kc, vc, H, HKV, HD, n - 1, scale)
            assert np.linalg.norm(got[b] - ref) / np.linalg.norm(ref) <= 1e-3, (B, n, b)
    # 16 queries x 64 splits x 8 KV heads need ~17 MB of partials: refused, not overrun.
    z = ctx.to_device(np.zeros((16, H * HD), np.float32))
    c8 = ctx.to_device(np.zeros((16, HKV, 64, HD), np.int8))
    cs = ctx.to_device(np.zeros((16, HKV, 64, HD // 32), np.float16))
    with pytest.raises(ts5hip.Ts5HipError):
        ctx.attn_decode_noalloc(z, 16, H, HKV, HD, c8, cs, c8, cs, 64, ctx.to_device(np.full(16, 64, np.int32)), 1,
                                scale, ctx.alloc(16 * H * HD * 4), n_split=64)
    ctx.close()
