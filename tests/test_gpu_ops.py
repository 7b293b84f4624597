"""Per-op parity of the HIP kernels with the CPU oracle (a restatement of
ts5's engine/src/cpu_backend.cpp and quants.cpp, pinned to the reference's own
outputs by tests/test_oracle.py), through the C ABI.

Bars: unpack and q8 KV rounding bit-exact; matvec and attention relative L2
error <= 1e-3 against the oracle's fp64-accumulated results."""
import os

import numpy as np
import pytest

import oracle
from tokenstation5_amd import synth, ts5hip

pytestmark = pytest.mark.gpu
G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
REL_L2 = 1e-3


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


@pytest.fixture(scope="module")
def ctx():
    c = ts5hip.Context(0)
    assert c.arch.startswith("gfx950"), c.arch
    yield c
    c.close()


# ---- unpack -------------------------------------------------------------------------

@pytest.mark.parametrize("t", [synth.Q4_K, synth.Q6_K, synth.Q8_0])
def test_dequantize_bit_exact_golden(ctx, t):
    """HBM-layout unpack == the reference's dequantize_row (golden blocks,
    including zero, subnormal, negative and large f16 scales)."""
    q = np.load(os.path.join(G, "quants.npz"))
    blocks, want = q[f"t{t}_blocks"], q[f"t{t}_values"]
    bv = synth.BLOCK[t][0]
    rows = blocks.shape[0] if bv == 32 else blocks.shape[0]
    ne0 = bv
    w = ctx.weight(t, ne0, rows, blocks.reshape(rows, -1))
    y = ctx.alloc(want.nbytes)
    ctx.dequantize(t, w, ne0, rows, y)
    got = y.download(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_f16_unpack_every_half(ctx):
    h = np.arange(65536, dtype=np.uint16)
    w = ctx.to_device(h)
    y = ctx.alloc(65536 * 4)
    ctx.dequantize(synth.F16, w, 65536, 1, y)
    got = y.download(np.float32).view(np.uint32)
    want = np.array([oracle.lib().ts5o_fp16_to_fp32(int(v)) for v in h], np.float32).view(np.uint32)
    finite = np.isfinite(h.view(np.float16))
    assert np.array_equal(got[finite], want[finite])
    assert np.all(np.isnan(got[~finite].view(np.float32)) == np.isnan(want[~finite].view(np.float32)))


@pytest.mark.parametrize("t,ne0,rows", [(synth.Q4_K, 4096, 64), (synth.Q6_K, 4096, 32), (synth.Q8_0, 896, 50),
                                        (synth.Q4_K, 14336, 3)])
def test_dequantize_bit_exact_random(ctx, t, ne0, rows):
    W = synth.tensor(t, ne0, rows, 11, f"deq{t}")
    w = ctx.weight(t, ne0, rows, W)
    y = ctx.alloc(ne0 * rows * 4)
    ctx.dequantize(t, w, ne0, rows, y)
    got = y.download(np.float32).reshape(rows, ne0)
    want = np.stack([oracle.dequantize(t, W[r], ne0) for r in range(rows)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---- activations ----------------------------------------------------------------------

XQ_MAX = 2 ** 22 - 1


def act_unpack(buf, n, ntok=1):
    """(X values, scale, sum, isum) of ntok activations from the device:
    X = 65536 hi + 256 mid + lo from the three int8 planes."""
    ab = ts5hip.Context.act_bytes(n)
    raw = buf.download(np.uint8)[:ab * ntok].reshape(ntok, ab)
    al = lambda v: -(-v // 256) * 256  # noqa: E731
    planes = [raw[:, k * al(n):k * al(n) + n].view(np.int8).astype(np.int64) for k in range(3)]
    X = 65536 * planes[0] + 256 * planes[1] + planes[2]
    assert np.abs(planes[0]).max() <= 64
    o = 3 * al(n)
    sc = raw[:, o:o + n // 32 * 4].copy().view(np.float32)
    o += al(n // 32 * 4)
    sm = raw[:, o:o + n // 32 * 4].copy().view(np.float32)
    o += al(n // 32 * 4)
    isum = raw[:, o:o + n // 16 * 4].copy().view(np.int32)
    return X, sc, sm, isum


@pytest.mark.parametrize("n,norm", [(4096, True), (14336, False), (896, True)])
def test_act_quantize(ctx, n, norm):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * rng.choice([1e-3, 1.0, 1e4], n)).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(n)).astype(np.float32)
    dx, dw = ctx.to_device(x), ctx.to_device(w)
    act = ctx.alloc(ctx.act_bytes(n))
    ctx.act_quantize(dx, dw if norm else None, 1e-5, n, 1, act)
    X, sc, sm, isum = act_unpack(act, n)
    ref = oracle.rmsnorm(x, w, 1e-5) if norm else x
    rb = ref.reshape(-1, 32)
    assert np.abs(X).max() <= XQ_MAX
    # Per sub-block the scale is max|x| / XQ_MAX and every value within half a step.
    assert np.allclose(sc[0], np.abs(rb).max(1) / XQ_MAX, rtol=1e-5)
    # Nearest step, up to the fp32 roundings of v * (XQ_MAX / amax) (a few ulp of |v|).
    err = np.abs(X[0].reshape(-1, 32) * sc[0][:, None].astype(np.float64) - rb)
    assert np.all(err <= 0.5 * sc[0][:, None] + 4 * 2.0 ** -24 * np.abs(rb) + 1e-30)
    assert np.allclose(sm[0], rb.astype(np.float64).sum(1), rtol=1e-4, atol=1e-6 * np.abs(rb).max())
    assert np.array_equal(isum[0], X[0].reshape(-1, 16).sum(1))


@pytest.mark.parametrize("n", [4096, 1000, 8192])  # one pass in registers up to 4096, else two passes
def test_rmsnorm(ctx, n):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((3, n)) * 1e6).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(n)).astype(np.float32)
    y = ctx.alloc(x.nbytes)
    ctx.rmsnorm(ctx.to_device(x), ctx.to_device(w), 1e-5, n, 3, y)
    got = y.download(np.float32, (3, n))
    want = np.stack([oracle.rmsnorm(x[t], w, 1e-5) for t in range(3)])
    assert rel_l2(got, want) < 1e-6


# ---- matvec -----------------------------------------------------------------------------

def run_matvec(ctx, t, W, ne0, rows, x, accumulate=None, norm=None, eps=1e-5):
    w = ctx.weight(t, ne0, rows, W)
    y = ctx.to_device(accumulate if accumulate is not None else np.zeros(rows, np.float32))
    ctx.matvec(t, w, ne0, rows, ctx.to_device(x), y, norm_w=None if norm is None else ctx.to_device(norm), eps=eps,
               accumulate=accumulate is not None)
    return y.download(np.float32)


@pytest.mark.parametrize("t,ne0,rows", [
    (synth.Q4_K, 4096, 4096),     # cfg1
    (synth.Q4_K, 4096, 1024),     # wk/wv (2 rows a wave)
    (synth.Q4_K, 4096, 6144),     # fused QKV (3 rows a wave)
    (synth.Q4_K, 14336, 4096),    # ffn_down
    (synth.Q4_K, 4864, 896),      # the draft's ffn_down (19 blocks per row)
    (synth.Q4_K, 4352, 37),       # 17 blocks: split 9 + 8 across waves, ragged rows
    (synth.Q4_K, 256, 37),        # one block, ragged rows
    (synth.Q4_K, 5120, 7168),     # 20 blocks a row (the 14B-class QKV): row-packed steps of 4 blocks
    (synth.Q4_K, 3072, 1000),     # 12 blocks, row-packed, rows past the last group's
    (synth.Q4_K, 5120, 37),       # row-packed, fewer rows than one group of 16
    (synth.Q6_K, 4096, 4096),
    (synth.Q6_K, 512, 1000),
    (synth.Q8_0, 896, 896),       # the draft's 896-wide matrices
    (synth.Q8_0, 896, 4864),
    (synth.Q8_0, 32, 5),
])
def test_matvec_vs_oracle(ctx, t, ne0, rows):
    W = synth.tensor(t, ne0, rows, 1, f"mv{t}_{ne0}_{rows}")
    x = np.random.default_rng(ne0 + rows).standard_normal(ne0).astype(np.float32)
    got = run_matvec(ctx, t, W, ne0, rows, x)
    want = oracle.matmul(t, W, ne0, x)[0]
    assert rel_l2(got, want) <= REL_L2, rel_l2(got, want)


def test_matvec_centered_weights(ctx):
    """Zero-mean Q4_K weights (outputs not dominated by the weight mean)."""
    W = synth.tensor(synth.Q4_K, 4096, 512, 2, "centered", centered=True)
    x = np.random.default_rng(9).standard_normal(4096).astype(np.float32)
    got = run_matvec(ctx, synth.Q4_K, W, 4096, 512, x)
    want = oracle.matmul(synth.Q4_K, W, 4096, x)[0]
    assert rel_l2(got, want) <= REL_L2


@pytest.mark.parametrize("t,ne0,rows,centered", [(synth.Q4_K, 4096, 2048, True), (synth.Q4_K, 14336, 512, True),
                                                  (synth.Q4_K, 4096, 2048, False), (synth.Q6_K, 4096, 1024, False),
                                                  (synth.Q8_0, 896, 1024, False)])
def test_matvec_precision(ctx, t, ne0, rows, centered):
    """The activation keeps 23 significant bits per 32 values (65536 hi +
    256 mid + lo), the precision of the fp32 input the reference multiplies
    (engine/src/cpu_backend.cpp:30): against the fp64-accumulated oracle the
    one-token matvec and the several-token matmul (5 tokens, the verify
    batch) stay within 2e-6 relative L2, far inside the 1e-3 bar, also on
    zero-mean rows whose outputs cancel."""
    W = synth.tensor(t, ne0, rows, 8, f"prec{t}_{ne0}", centered=centered)
    rng = np.random.default_rng(ne0 + rows)
    x = rng.standard_normal((5, ne0)).astype(np.float32)
    got = run_matvec(ctx, t, W, ne0, rows, x[0])
    want = oracle.matmul(t, W, ne0, x)
    assert rel_l2(got, want[0]) <= 2e-6, rel_l2(got, want[0])
    w = ctx.weight(t, ne0, rows, W)
    y = ctx.alloc(5 * rows * 4)
    ctx.matmul(t, w, ne0, rows, ctx.to_device(x), 5, y)
    got5 = y.download(np.float32, (5, rows))
    for k in range(5):
        assert rel_l2(got5[k], want[k]) <= 2e-6, (k, rel_l2(got5[k], want[k]))


@pytest.mark.parametrize("ne0,rows", [(1024, 256), (14336, 200), (5120, 300), (5120, 5120)])
def test_matvec_accumulate_and_scales(ctx, ne0, rows):
    """Input magnitudes from 1e-6 to 1e7 (the activation scale is per 32
    values), and accumulation into an existing fp32 vector (y += W x), for
    rows of one step (1024 wide: 4 blocks, row-packed), rows whose blocks
    the workgroup's waves split, and 5120-wide rows on row-packed steps."""
    W = synth.tensor(synth.Q4_K, ne0, rows, 3, f"acc{ne0}")
    rng = np.random.default_rng(4)
    for scale in (1e-6, 1.0, 1e7):
        x = (rng.standard_normal(ne0) * scale).astype(np.float32)
        want = oracle.matmul(synth.Q4_K, W, ne0, x)[0]
        assert rel_l2(run_matvec(ctx, synth.Q4_K, W, ne0, rows, x), want) <= REL_L2, scale
        y0 = (rng.standard_normal(rows) * np.abs(want).mean()).astype(np.float32)
        got = run_matvec(ctx, synth.Q4_K, W, ne0, rows, x, accumulate=y0.copy())
        assert rel_l2(got, y0.astype(np.float64) + want) <= REL_L2, scale


def test_matvec_zero_input(ctx):
    W = synth.tensor(synth.Q6_K, 256, 64, 5, "zero")
    got = run_matvec(ctx, synth.Q6_K, W, 256, 64, np.zeros(256, np.float32))
    assert np.array_equal(got, np.zeros(64, np.float32))


def test_matvec_fused_rmsnorm(ctx):
    """The norm before a projection fused into the matvec's prologue:
    W rmsnorm(x) (engine/src/cpu_backend.cpp:48-53, :193)."""
    rng = np.random.default_rng(12)
    x = (rng.standard_normal(4096) * 3e5).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(4096)).astype(np.float32)
    W = synth.tensor(synth.Q4_K, 4096, 6144, 4, "qkv")
    got = run_matvec(ctx, synth.Q4_K, W, 4096, 6144, x, norm=w, eps=1e-5)
    want = oracle.matmul(synth.Q4_K, W, 4096, oracle.rmsnorm(x, w, 1e-5))[0]
    assert rel_l2(got, want) <= REL_L2


@pytest.mark.parametrize("t,ne0,rows", [(synth.Q6_K, 4096, 128256), (synth.Q8_0, 896, 151936), (synth.Q6_K, 512, 1000)])
def test_head_argmax(ctx, t, ne0, rows):
    """cfg4's head: logits = W rmsnorm(h), and the greedy id equals the
    first maximum of those logits (bit-exact token id), within 1e-3 of the
    oracle's logits."""
    rng = np.random.default_rng(rows)
    W = synth.tensor(t, ne0, rows, 5, f"head{t}")
    h = rng.standard_normal(ne0).astype(np.float32)
    nw = (1 + 0.02 * rng.standard_normal(ne0)).astype(np.float32)
    w = ctx.weight(t, ne0, rows, W)
    y, out = ctx.alloc(rows * 4), ctx.alloc(4)
    for rep in range(3):  # the workgroup counter resets itself between launches
        ctx.matvec_argmax(t, w, ne0, rows, ctx.to_device(h), y, out, norm_w=ctx.to_device(nw), eps=1e-5)
        lg = y.download(np.float32)
        assert int(out.download(np.int32)[0]) == int(np.argmax(lg)), rep
    want = oracle.matmul(t, W, ne0, oracle.rmsnorm(h, nw, 1e-5))[0]
    assert rel_l2(lg, want) <= REL_L2


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 6, 8, 9, 16])
@pytest.mark.parametrize("ne0,rows,mode", [(4096, 1000, "store"), (14336, 528, "add"), (512, 37, "glu"),
                                           (4096, 9000, "add"), (4096, 4100, "glu"), (14336, 4200, "add"),
                                           (4096, 6144, "store"), (5120, 7168, "store"), (5120, 5120, "add")])
def test_q4k_small_batch_matmul(ctx, M, ne0, rows, mode):
    """The Q4_K matmul of 1-16 tokens (k_gemm_m up to 8, k_gemm_small past
    it; up to 5 tokens over inputs up to 4096 wide, k_gemm_mx): every token's
    rows within 2e-6 relative L2 of the oracle, in each mode (plain,
    accumulating into a residual, fused gate/up + SiLU), with row counts that
    leave partial 16-row tiles; 9000 and 4100 rows give k_gemm_mx 4 and 2
    row tiles a workgroup, some of them past the last row, and 6144 rows
    (the 8B's QKV) 2 tiles of one matrix; inputs past 4096 wide (5120: the
    14B-class QKV and wo; 14336) take k_gemm_mw over quantized records
    (4200 rows: 263 tiles over 256 workgroups)."""
    rng = np.random.default_rng(M * 100 + rows)
    W = synth.tensor(synth.Q4_K, ne0, rows, 21, f"sb{ne0}", centered=True)
    x = rng.standard_normal((M, ne0)).astype(np.float32)
    w = ctx.weight(synth.Q4_K, ne0, rows, W)
    if mode == "glu":
        U = synth.tensor(synth.Q4_K, ne0, rows, 22, f"sbu{ne0}", centered=True)
        y = ctx.alloc(M * rows * 4)
        ctx.matmul_glu(synth.Q4_K, w, ctx.weight(synth.Q4_K, ne0, rows, U), ne0, rows, ctx.to_device(x), M, y)
        want = oracle.swiglu(oracle.matmul(synth.Q4_K, W, ne0, x), oracle.matmul(synth.Q4_K, U, ne0, x))
    elif mode == "add":
        y0 = rng.standard_normal((M, rows)).astype(np.float32)
        y = ctx.to_device(y0)
        ctx.matmul(synth.Q4_K, w, ne0, rows, ctx.to_device(x), M, y, accumulate=True)
        want = y0.astype(np.float64) + oracle.matmul(synth.Q4_K, W, ne0, x)
    else:
        y = ctx.alloc(M * rows * 4)
        ctx.matmul(synth.Q4_K, w, ne0, rows, ctx.to_device(x), M, y)
        want = oracle.matmul(synth.Q4_K, W, ne0, x)
    got = y.download(np.float32, (M, rows))
    for k in range(M):
        assert rel_l2(got[k], want[k]) <= 2e-6, (k, rel_l2(got[k], want[k]))


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 6])
@pytest.mark.parametrize("ne0,rows,mode", [(4096, 1000, "store"), (512, 515, "add"), (4096, 20000, "store"),
                                           (4096, 40008, "store")])
def test_q6k_small_batch_matmul(ctx, M, ne0, rows, mode):
    """The Q6_K matmul of 1-6 tokens (up to 5: centred quants and two MFMAs
    per 32 values, on k_gemm_mh without a residual, k_gemm_m with one;
    k_gemm_small past it): every token's rows within 2e-6 relative L2 of the
    oracle; a ragged last row tile, and (40008 rows, 2501 tiles) more tiles
    than the launch has waves, as the verify batch's head has."""
    rng = np.random.default_rng(M * 1000 + rows)
    W = synth.tensor(synth.Q6_K, ne0, rows, 23, f"q6sb{ne0}_{rows}")
    x = rng.standard_normal((M, ne0)).astype(np.float32)
    w = ctx.weight(synth.Q6_K, ne0, rows, W)
    if mode == "add":
        y0 = rng.standard_normal((M, rows)).astype(np.float32)
        y = ctx.to_device(y0)
        ctx.matmul(synth.Q6_K, w, ne0, rows, ctx.to_device(x), M, y, accumulate=True)
        want = y0.astype(np.float64) + oracle.matmul(synth.Q6_K, W, ne0, x)
    else:
        y = ctx.alloc(M * rows * 4)
        ctx.matmul(synth.Q6_K, w, ne0, rows, ctx.to_device(x), M, y)
        want = oracle.matmul(synth.Q6_K, W, ne0, x)
    got = y.download(np.float32, (M, rows))
    for k in range(M):
        assert rel_l2(got[k], want[k]) <= 2e-6, (k, rel_l2(got[k], want[k]))


@pytest.mark.parametrize("t,ne0,rows", [(synth.Q4_K, 4096, 14336), (synth.Q8_0, 896, 4864), (synth.Q4_K, 512, 64),
                                        (synth.Q4_K, 5120, 13824), (synth.Q4_K, 3072, 1001)])
def test_glu_vs_oracle(ctx, t, ne0, rows):
    Wg = synth.tensor(t, ne0, rows, 6, "gate")
    Wu = synth.tensor(t, ne0, rows, 6, "up")
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(ne0) * 50).astype(np.float32)
    nw = (1 + 0.02 * rng.standard_normal(ne0)).astype(np.float32)
    wg, wu = ctx.weight(t, ne0, rows, Wg), ctx.weight(t, ne0, rows, Wu)
    y = ctx.alloc(rows * 4)
    ctx.matvec_glu(t, wg, wu, ne0, rows, ctx.to_device(x), y, norm_w=ctx.to_device(nw), eps=1e-6)
    got = y.download(np.float32)
    h = oracle.rmsnorm(x, nw, 1e-6)
    want = oracle.swiglu(oracle.matmul(t, Wg, ne0, h)[0], oracle.matmul(t, Wu, ne0, h)[0])
    assert rel_l2(got, want) <= REL_L2


# ---- RoPE + q8 KV append, attention ---------------------------------------------------------

@pytest.mark.parametrize("H,HKV,HD,neox,ntok,pos0", [(32, 8, 128, False, 1, 4095), (14, 2, 64, True, 3, 17),
                                                     (4, 1, 128, False, 5, 0)])
def test_rope_kv_append(ctx, H, HKV, HD, neox, ntok, pos0):
    """q rotated and K/V rounded to q8 exactly as the CPU path does it."""
    n_ctx = pos0 + ntok + 3
    rng = np.random.default_rng(H + pos0)
    R = (H + 2 * HKV) * HD
    qkv = (rng.standard_normal((ntok, R)) * rng.choice([1.0, 300.0], (ntok, R))).astype(np.float32)
    bias = (rng.standard_normal(R) * 0.1).astype(np.float32) if neox else None
    rope = ctx.rope_table(HD, n_ctx, 1e6 if neox else 500000.0)
    pos = ctx.to_device(np.array([pos0], np.int32))
    q_out = ctx.alloc(ntok * H * HD * 4)
    k8, v8 = ctx.alloc(HKV * n_ctx * HD).zero(), ctx.alloc(HKV * n_ctx * HD).zero()
    ks, vs = ctx.alloc(HKV * n_ctx * HD // 16).zero(), ctx.alloc(HKV * n_ctx * HD // 16).zero()
    ctx.rope_kv_append(ctx.to_device(qkv), ntok, pos, H, HKV, HD, HD, neox, rope, n_ctx, q_out, k8, ks, v8, vs,
                       bias=None if bias is None else ctx.to_device(bias))
    q = q_out.download(np.float32, (ntok, H, HD))
    K8 = k8.download(np.int8, (HKV, n_ctx, HD)).astype(np.float32)
    V8 = v8.download(np.int8, (HKV, n_ctx, HD)).astype(np.float32)
    KS = ks.download(np.float16, (HKV, n_ctx, HD // 32)).astype(np.float32)
    VS = vs.download(np.float16, (HKV, n_ctx, HD // 32)).astype(np.float32)
    base = 1e6 if neox else 500000.0
    for t in range(ntok):
        v = qkv[t] + (bias if bias is not None else 0)
        p = pos0 + t
        for h in range(H):
            want = oracle.rope(v[h * HD:(h + 1) * HD], HD, p, base, neox)
            assert np.array_equal(q[t, h].view(np.uint32), want.view(np.uint32)), (t, h)
        for h in range(HKV):
            kw = oracle.round_kv(2, oracle.rope(v[(H + h) * HD:(H + h + 1) * HD], HD, p, base, neox))
            vw = oracle.round_kv(2, v[(H + HKV + h) * HD:(H + HKV + h + 1) * HD])
            kg = (K8[h, p].reshape(-1, 32) * KS[h, p][:, None]).ravel()
            vg = (V8[h, p].reshape(-1, 32) * VS[h, p][:, None]).ravel()
            assert np.array_equal(kg, kw), (t, h)
            assert np.array_equal(vg, vw), (t, h)


def q8_cache(rng, B, HKV, n_ctx, HD):
    """K/V ~ N(0,1) rounded by the q8 rule: (int8, f16 scale) and fp32 values."""
    vals = rng.standard_normal((B, HKV, n_ctx, HD), dtype=np.float32)
    blocks = vals.reshape(-1, 32)
    amax = np.abs(blocks).max(1)
    sc = (amax / np.float32(127)).astype(np.float16)
    scf = sc.astype(np.float32)
    q = np.clip(np.rint(blocks / scf[:, None]), -127, 127).astype(np.int8)
    deq = (q.astype(np.float32) * scf[:, None]).reshape(vals.shape)
    return q.reshape(vals.shape), sc.reshape(B, HKV, n_ctx, HD // 32), deq


@pytest.mark.parametrize("B,ctxlen,H,HKV,HD", [(1, 8192, 32, 8, 128), (4, 8192, 32, 8, 128), (16, 8192, 32, 8, 128),
                                               (1, 32768, 32, 8, 128), (4, 32768, 32, 8, 128),
                                               (16, 32768, 32, 8, 128), (1, 1000, 32, 8, 128),
                                               (2, 33, 14, 2, 64), (3, 1, 32, 8, 128),
                                               (1, 700, 4, 1, 256), (3, 1500, 8, 4, 256), (2, 4096, 16, 8, 256)])
def test_attention_vs_oracle(ctx, B, ctxlen, H, HKV, HD):
    """cfg3: one query per sequence over its q8 cache, full context, scale 1/sqrt(HD);
    every cfg3 shape (B 1, 4, 16 x 8192, 32768 keys) with the default split count."""
    rng = np.random.default_rng(B * 7 + ctxlen)
    q8, sc, deq = q8_cache(rng, B, HKV, ctxlen, HD)
    v8, vsc, vdeq = q8_cache(rng, B, HKV, ctxlen, HD)
    q = rng.standard_normal((B, H * HD)).astype(np.float32)
    scale = float(np.float32(1) / np.sqrt(np.float32(HD)))
    out = ctx.alloc(q.nbytes)
    nk = ctx.to_device(np.full(B, ctxlen, np.int32))
    ctx.attn_decode(ctx.to_device(q), B, H, HKV, HD, ctx.to_device(q8), ctx.to_device(sc), ctx.to_device(v8),
                    ctx.to_device(vsc), ctxlen, nk, 1, scale, out)
    got = out.download(np.float32, (B, H * HD))
    for b in range(B):
        kc = deq[b].transpose(1, 0, 2).reshape(ctxlen, HKV * HD)
        vc = vdeq[b].transpose(1, 0, 2).reshape(ctxlen, HKV * HD)
        want = oracle.attention(q[b], kc, vc, H, HKV, HD, ctxlen - 1, scale)
        assert rel_l2(got[b], want) <= REL_L2, (b, rel_l2(got[b], want))


@pytest.mark.parametrize("kv", ["q8", "f16"])
@pytest.mark.parametrize("H,HKV", [(8, 8), (16, 8), (40, 8), (28, 4), (64, 8)])
def test_attention_matrix_core_one_query(ctx, kv, H, HKV):
    """The matrix-core one-query kernel (k_attn_m1: queries on caches of their
    own, head dimension 128) for every query-head group it takes (G 1, 2, 5,
    7, 8; G 4 is cfg3's), q8 and f16, each sequence with its own key count
    (a whole number of 128-key steps, a ragged tail, a short cache of 5
    keys), against the oracle at 2e-5 relative L2."""
    HD, ctxlen, B = 128, 1000, 3
    n_keys = np.array([ctxlen, ctxlen - 37, 5], np.int32)
    rng = np.random.default_rng(H * 3 + HKV)
    if kv == "q8":
        k8, ks, kd = q8_cache(rng, B, HKV, ctxlen, HD)
        v8, vs, vd = q8_cache(rng, B, HKV, ctxlen, HD)
    else:
        kd = rng.standard_normal((B, HKV, ctxlen, HD), dtype=np.float32).astype(np.float16)
        vd = rng.standard_normal((B, HKV, ctxlen, HD), dtype=np.float32).astype(np.float16)
    q = rng.standard_normal((B, H * HD)).astype(np.float32)
    scale = float(np.float32(1) / np.sqrt(np.float32(HD)))
    out = ctx.alloc(q.nbytes)
    nk = ctx.to_device(n_keys)
    if kv == "q8":
        ctx.attn_decode(ctx.to_device(q), B, H, HKV, HD, ctx.to_device(k8), ctx.to_device(ks), ctx.to_device(v8),
                        ctx.to_device(vs), ctxlen, nk, 1, scale, out)
    else:
        ctx.attn_decode_f16(ctx.to_device(q), B, H, HKV, HD, ctx.to_device(kd), ctx.to_device(vd), ctxlen, nk, 1,
                            scale, out)
    got = out.download(np.float32, (B, H * HD))
    for b in range(B):
        n = int(n_keys[b])
        kc = kd[b].astype(np.float32).transpose(1, 0, 2).reshape(ctxlen, HKV * HD)[:n]
        vc = vd[b].astype(np.float32).transpose(1, 0, 2).reshape(ctxlen, HKV * HD)[:n]
        want = oracle.attention(q[b], kc, vc, H, HKV, HD, n - 1, scale)
        assert rel_l2(got[b], want) <= 2e-5, (b, rel_l2(got[b], want))


@pytest.mark.parametrize("B,ctxlen,H,HKV,HD,n_split", [(1, 8192, 32, 8, 128, 0), (4, 8192, 32, 8, 128, 0),
                                                       (16, 8192, 32, 8, 128, 0), (1, 32768, 32, 8, 128, 0),
                                                       (4, 32768, 32, 8, 128, 0), (16, 32768, 32, 8, 128, 0),
                                                       (2, 70, 14, 2, 64, 0), (1, 5000, 32, 8, 128, 64),
                                                       (1, 700, 4, 1, 256, 0), (2, 3000, 8, 4, 256, 0)])
def test_attention_f16_vs_oracle(ctx, B, ctxlen, H, HKV, HD, n_split):
    """cfg3's attention over an f16 cache (KvType::F16, the reference's
    default; each value the nearest half of N(0,1)), long contexts included."""
    rng = np.random.default_rng(B * 11 + ctxlen)
    k = rng.standard_normal((B, HKV, ctxlen, HD), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((B, HKV, ctxlen, HD), dtype=np.float32).astype(np.float16)
    q = rng.standard_normal((B, H * HD)).astype(np.float32)
    scale = float(np.float32(1) / np.sqrt(np.float32(HD)))
    out = ctx.alloc(q.nbytes)
    ctx.attn_decode_f16(ctx.to_device(q), B, H, HKV, HD, ctx.to_device(k), ctx.to_device(v), ctxlen,
                        ctx.to_device(np.full(B, ctxlen, np.int32)), 1, scale, out, n_split=n_split)
    got = out.download(np.float32, (B, H * HD))
    for b in range(B):
        kc = k[b].astype(np.float32).transpose(1, 0, 2).reshape(ctxlen, HKV * HD)
        vc = v[b].astype(np.float32).transpose(1, 0, 2).reshape(ctxlen, HKV * HD)
        want = oracle.attention(q[b], kc, vc, H, HKV, HD, ctxlen - 1, scale)
        assert rel_l2(got[b], want) <= REL_L2, (b, rel_l2(got[b], want))


def test_attention_most_work_items_twice(ctx):
    """B * HKV = 4096 (the per-op entry point's limit) with 8 key splits each:
    every (query, KV head) merge counter counts 8 workgroups and its last one
    merges, 32768 workgroups in all; run twice (the counters must be back at
    zero), and one more query refused."""
    rng = np.random.default_rng(11)
    B, H, HKV, HD, n = 512, 32, 8, 64, 200
    q8, sc, deq = q8_cache(rng, B, HKV, n, HD)
    v8, vsc, vdeq = q8_cache(rng, B, HKV, n, HD)
    q = rng.standard_normal((B, H * HD)).astype(np.float32)
    args = (ctx.to_device(q8), ctx.to_device(sc), ctx.to_device(v8), ctx.to_device(vsc), n,
            ctx.to_device(np.full(B, n, np.int32)), 1, 0.125)
    dq = ctx.to_device(q)
    for _ in range(2):
        out = ctx.alloc(q.nbytes)
        ctx.attn_decode(dq, B, H, HKV, HD, *args, out, n_split=8)
        got = out.download(np.float32, (B, H * HD))
        for b in range(0, B, 7):
            kc = deq[b].transpose(1, 0, 2).reshape(n, HKV * HD)
            vc = vdeq[b].transpose(1, 0, 2).reshape(n, HKV * HD)
            assert rel_l2(got[b], oracle.attention(q[b], kc, vc, H, HKV, HD, n - 1, 0.125)) <= REL_L2, b
    with pytest.raises(ts5hip.Ts5HipError):
        ctx.attn_decode(ctx.to_device(np.zeros((B + 1, H * HD), np.float32)), B + 1, H, HKV, HD, *args,
                        ctx.alloc((B + 1) * H * HD * 4))


def test_attention_splits_agree(ctx):
    """Any split count gives the same softmax (merge of partials)."""
    rng = np.random.default_rng(5)
    B, H, HKV, HD, n = 1, 32, 8, 128, 3000
    q8, sc, _ = q8_cache(rng, B, HKV, n, HD)
    v8, vsc, _ = q8_cache(rng, B, HKV, n, HD)
    q = ctx.to_device(rng.standard_normal((B, H * HD)).astype(np.float32))
    dq8, dsc, dv8, dvs = ctx.to_device(q8), ctx.to_device(sc), ctx.to_device(v8), ctx.to_device(vsc)
    nk = ctx.to_device(np.array([n], np.int32))
    outs = []
    for split in (1, 7, 47, 64):
        out = ctx.alloc(H * HD * 4)
        ctx.attn_decode(q, B, H, HKV, HD, dq8, dsc, dv8, dvs, n, nk, 1, 0.0883883, out, n_split=split)
        outs.append(out.download(np.float32))
    for o in outs[1:]:
        assert rel_l2(o, outs[0]) < 1e-5


@pytest.mark.parametrize("n_split", [0, 32])
def test_attention_verify_batch(ctx, n_split):
    """The verify batch of speculative decoding: 5 consecutive queries of one
    cache at ~4.3k keys (the default split count, then 32 splits: 40 KV-head
    merges each with many concurrent mergers), against the oracle."""
    rng = np.random.default_rng(12 + n_split)
    H, HKV, HD, n_ctx, p0, B = 32, 8, 128, 4400, 4300, 5
    q8, sc, deq = q8_cache(rng, 1, HKV, n_ctx, HD)
    v8, vsc, vdeq = q8_cache(rng, 1, HKV, n_ctx, HD)
    q = rng.standard_normal((B, H * HD)).astype(np.float32)
    scale = float(np.float32(1) / np.sqrt(np.float32(HD)))
    out = ctx.alloc(q.nbytes)
    ctx.attn_decode(ctx.to_device(q), B, H, HKV, HD, ctx.to_device(q8), ctx.to_device(sc), ctx.to_device(v8),
                    ctx.to_device(vsc), n_ctx, ctx.to_device(np.array([p0], np.int32)), 0, scale, out,
                    n_split=n_split)
    got = out.download(np.float32, (B, H * HD))
    kc = deq[0].transpose(1, 0, 2).reshape(n_ctx, HKV * HD)
    vc = vdeq[0].transpose(1, 0, 2).reshape(n_ctx, HKV * HD)
    for b in range(B):
        want = oracle.attention(q[b], kc, vc, H, HKV, HD, p0 + b, scale)
        assert rel_l2(got[b], want) <= REL_L2, (b, rel_l2(got[b], want))


@pytest.mark.parametrize("B,H,HKV,n_ctx,p0,n_split", [(2, 32, 8, 4400, 4300, 32), (8, 32, 8, 3000, 2990, 32),
                                                     (16, 8, 8, 1200, 1100, 16), (16, 16, 8, 700, 600, 0),
                                                     (6, 40, 8, 2100, 2000, 40), (4, 64, 8, 900, 800, 7),
                                                     (5, 32, 8, 64, 10, 32), (5, 32, 8, 300, 0, 1),
                                                     (3, 4, 1, 5000, 4096, 64), (5, 32, 8, 4200, 4094, 61)])
def test_attention_batch_matrix_cores(ctx, B, H, HKV, n_ctx, p0, n_split):
    """One cache, 2-16 consecutive queries, B x G <= 32 rows of head
    dimension 128: the batch's queries together in each work item, on the
    matrix cores (fp16 hi + lo query and p planes, exact int8 keys and
    values), against the oracle to 2e-5: G 1-8, splits from 1 (one work
    item writes the output) to 64, short slices, keys from position 0,
    split boundaries between the batch's queries."""
    rng = np.random.default_rng(B * 31 + H + n_ctx + n_split)
    HD = 128
    q8, sc, deq = q8_cache(rng, 1, HKV, n_ctx, HD)
    v8, vsc, vdeq = q8_cache(rng, 1, HKV, n_ctx, HD)
    q = (rng.standard_normal((B, H * HD)) * 2).astype(np.float32)
    scale = float(np.float32(1) / np.sqrt(np.float32(HD)))
    out = ctx.alloc(q.nbytes)
    ctx.attn_decode(ctx.to_device(q), B, H, HKV, HD, ctx.to_device(q8), ctx.to_device(sc), ctx.to_device(v8),
                    ctx.to_device(vsc), n_ctx, ctx.to_device(np.array([p0], np.int32)), 0, scale, out,
                    n_split=n_split)
    got = out.download(np.float32, (B, H * HD))
    kc = deq[0].transpose(1, 0, 2).reshape(n_ctx, HKV * HD)
    vc = vdeq[0].transpose(1, 0, 2).reshape(n_ctx, HKV * HD)
    for b in range(B):
        want = oracle.attention(q[b], kc, vc, H, HKV, HD, p0 + b, scale)
        assert rel_l2(got[b], want) <= 2e-5, (b, rel_l2(got[b], want))


def test_attention_causal_batch(ctx):
    """kv_per_batch = 0: query b at position p0 + b sees keys 0..p0+b."""
    rng = np.random.default_rng(6)
    H, HKV, HD, n_ctx, p0, B = 8, 2, 64, 200, 150, 4
    q8, sc, deq = q8_cache(rng, 1, HKV, n_ctx, HD)
    v8, vsc, vdeq = q8_cache(rng, 1, HKV, n_ctx, HD)
    q = rng.standard_normal((B, H * HD)).astype(np.float32)
    out = ctx.alloc(q.nbytes)
    ctx.attn_decode(ctx.to_device(q), B, H, HKV, HD, ctx.to_device(q8), ctx.to_device(sc), ctx.to_device(v8),
                    ctx.to_device(vsc), n_ctx, ctx.to_device(np.array([p0], np.int32)), 0, 0.125, out)
    got = out.download(np.float32, (B, H * HD))
    kc = deq[0].transpose(1, 0, 2).reshape(n_ctx, HKV * HD)
    vc = vdeq[0].transpose(1, 0, 2).reshape(n_ctx, HKV * HD)
    for b in range(B):
        want = oracle.attention(q[b], kc, vc, H, HKV, HD, p0 + b, 0.125)
        assert rel_l2(got[b], want) <= REL_L2


@pytest.mark.parametrize("nq,p0,n_ctx,H,HKV,HD", [(64, 0, 64, 32, 8, 128), (256, 3840, 4096, 32, 8, 128),
                                                (100, 1000, 2048, 8, 2, 128), (37, 5, 64, 4, 1, 128),
                                                (130, 300, 512, 16, 16, 128), (50, 200, 300, 16, 8, 128),
                                                (40, 700, 1000, 64, 8, 128), (17, 4079, 4096, 32, 8, 128),
                                                (5, 4091, 4096, 32, 8, 128), (16, 1000, 2048, 8, 2, 128),
                                                (1, 100, 200, 32, 8, 128),
                                                (256, 1792, 2048, 14, 2, 64), (60, 0, 60, 14, 2, 64),
                                                (100, 400, 600, 12, 4, 64), (33, 90, 200, 48, 3, 64),
                                                (256, 768, 1024, 40, 8, 128), (70, 10, 100, 28, 4, 128)])
def test_attention_prompt_vs_oracle(ctx, nq, p0, n_ctx, H, HKV, HD):
    """Prompt chunks on the matrix cores: query t at p0 + t over keys 0..p0+t (one split
    up to 256 keys, then up to 16 merged splits; ragged query blocks; GQA groups 1-8 at
    head dimension 128, and groups that leave rows of the 128 idle: 7 and 3 and 16 at
    head dimension 64 (the 0.5B draft's 14/2 heads), 5 and 7 at 128 (14B-class 40/8,
    28/4)). A few queries (5, 16, 1) take the same kernel. The path keeps ~22-bit
    operands, so it is held to 2e-5, not the shared 1e-3."""
    rng = np.random.default_rng(nq + p0 + H)
    q8, sc, deq = q8_cache(rng, 1, HKV, n_ctx, HD)
    v8, vsc, vdeq = q8_cache(rng, 1, HKV, n_ctx, HD)
    q = (rng.standard_normal((nq, H * HD)) * 3).astype(np.float32)
    scale = float(np.float32(1) / np.sqrt(np.float32(HD)))
    out = ctx.alloc(q.nbytes)
    ctx.attn_prompt(ctx.to_device(q), nq, H, HKV, HD, ctx.to_device(q8), ctx.to_device(sc), ctx.to_device(v8),
                    ctx.to_device(vsc), n_ctx, p0, scale, out)
    got = out.download(np.float32, (nq, H * HD))
    kc = deq[0].transpose(1, 0, 2).reshape(n_ctx, HKV * HD)
    vc = vdeq[0].transpose(1, 0, 2).reshape(n_ctx, HKV * HD)
    for t in range(nq):
        want = oracle.attention(q[t], kc, vc, H, HKV, HD, p0 + t, scale)
        assert rel_l2(got[t], want) <= 2e-5, (t, rel_l2(got[t], want))


@pytest.mark.parametrize("nq,p0,n_ctx,H,HKV,HD", [(64, 0, 64, 32, 8, 128), (256, 3840, 4096, 32, 8, 128),
                                                (100, 1000, 2048, 8, 2, 128), (37, 5, 64, 4, 1, 128),
                                                (130, 300, 512, 16, 16, 128), (17, 4079, 4096, 32, 8, 128),
                                                (1, 100, 200, 32, 8, 128), (256, 1792, 2048, 14, 2, 64),
                                                (100, 400, 600, 12, 4, 64), (256, 768, 1024, 40, 8, 128)])
def test_attention_prompt_f16_vs_oracle(ctx, nq, p0, n_ctx, H, HKV, HD):
    """Prompt chunks over an f16 cache (each value the nearest half of N(0,1))
    on the matrix cores, K and V as stored: one split and merged splits,
    ragged query blocks, GQA groups 1-8 at head dimension 128 and 7, 3, 5 with
    idle rows, held to 2e-5 like the q8 path."""
    rng = np.random.default_rng(nq + p0 + H + 7)
    k = rng.standard_normal((HKV, n_ctx, HD), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((HKV, n_ctx, HD), dtype=np.float32).astype(np.float16)
    q = (rng.standard_normal((nq, H * HD)) * 3).astype(np.float32)
    scale = float(np.float32(1) / np.sqrt(np.float32(HD)))
    out = ctx.alloc(q.nbytes)
    ctx.attn_prompt_f16(ctx.to_device(q), nq, H, HKV, HD, ctx.to_device(k), ctx.to_device(v), n_ctx, p0, scale, out)
    got = out.download(np.float32, (nq, H * HD))
    kc = k.astype(np.float32).transpose(1, 0, 2).reshape(n_ctx, HKV * HD)
    vc = v.astype(np.float32).transpose(1, 0, 2).reshape(n_ctx, HKV * HD)
    for t in range(nq):
        want = oracle.attention(q[t], kc, vc, H, HKV, HD, p0 + t, scale)
        assert rel_l2(got[t], want) <= 2e-5, (t, rel_l2(got[t], want))


def test_attention_prompt_large_values_and_bad_shapes(ctx):
    """Queries of 1e6 (past fp16: each row is scaled by a power of two first), keys of
    1e3; then shapes the path does not take are refused, not guessed."""
    H, HKV, HD, n_ctx, p0, nq = 8, 2, 128, 96, 10, 40
    rng = np.random.default_rng(11)
    q8, sc, deq = q8_cache(rng, 1, HKV, n_ctx, HD)
    sc = (sc.astype(np.float32) * 1000).astype(np.float16)
    deq = (q8.astype(np.float32).reshape(-1, 32) * sc.astype(np.float32).reshape(-1, 1)).reshape(deq.shape)
    v8, vsc, vdeq = q8_cache(rng, 1, HKV, n_ctx, HD)
    q = (rng.standard_normal((nq, H * HD)) * 1e6).astype(np.float32)
    out = ctx.alloc(q.nbytes)
    ctx.attn_prompt(ctx.to_device(q), nq, H, HKV, HD, ctx.to_device(q8), ctx.to_device(sc), ctx.to_device(v8),
                    ctx.to_device(vsc), n_ctx, p0, 0.088, out)
    got = out.download(np.float32, (nq, H * HD))
    kc = deq[0].transpose(1, 0, 2).reshape(n_ctx, HKV * HD)
    vc = vdeq[0].transpose(1, 0, 2).reshape(n_ctx, HKV * HD)
    for t in range(nq):
        want = oracle.attention(q[t], kc, vc, H, HKV, HD, p0 + t, 0.088)
        assert rel_l2(got[t], want) <= 2e-5, t
    with pytest.raises(ts5hip.Ts5HipError):  # head dimension 256 (Gemma 3) takes the per-query kernel
        ctx.attn_prompt(ctx.to_device(q), nq, 4, 2, 256, ctx.to_device(q8), ctx.to_device(sc), ctx.to_device(v8),
                        ctx.to_device(vsc), n_ctx, p0, 0.088, out)
    with pytest.raises(ts5hip.Ts5HipError):
        ctx.attn_prompt(ctx.to_device(q), nq, H, HKV, HD, ctx.to_device(q8), ctx.to_device(sc), ctx.to_device(v8),
                        ctx.to_device(vsc), n_ctx, n_ctx - nq + 1, 0.088, out)


# ---- sampling reductions ------------------------------------------------------------------------

def test_argmax_first_maximum(ctx):
    rng = np.random.default_rng(8)
    x = rng.standard_normal((3, 128256)).astype(np.float32)
    x[1, 777] = x[1, 99999] = 50.0   # a tie: the lower id wins (std::max_element)
    x[2, :] = 1.0                    # all equal: id 0
    out = ctx.alloc(12)
    ctx.argmax(ctx.to_device(x), 128256, 3, out)
    got = out.download(np.int32)
    assert list(got) == [int(np.argmax(x[0])), 777, 0]


@pytest.mark.parametrize("n,k", [(128256, 40), (151936, 64), (1000, 5), (128256, 1)])
def test_topk(ctx, n, k):
    rng = np.random.default_rng(n + k)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    x[10] = x[20] = x.max() + 1  # tie at the top: ascending id
    vals, ids = ctx.alloc(k * 4), ctx.alloc(k * 4)
    ctx.topk(ctx.to_device(x), n, k, vals, ids)
    want = np.argsort(-x, kind="stable")[:k]
    assert list(ids.download(np.int32)) == list(want)
    assert np.array_equal(vals.download(np.float32), x[want])


@pytest.mark.parametrize("case", ["all_equal", "int_ties", "signed_zeros", "minus_inf", "two_slices", "n_is_k",
                                  "one"])
def test_topk_edge_cases(ctx, case):
    """The top k in rank order (larger value, then smaller id, as a stable
    descending sort) where the selection is exact only by its tie handling:
    a row of one value (more tied entries than the gather holds: the sorted
    lists are merged), small integers (ties at the k-th), -0 and +0 across
    the cut (equal values, ranked by id), -inf entries, a last slice of one
    logit, n == k."""
    rng = np.random.default_rng(sum(map(ord, case)))
    n, k = 128256, 40
    if case == "all_equal":
        x = np.ones(n, np.float32)
    elif case == "int_ties":
        x = np.rint(rng.standard_normal(n) * 2).astype(np.float32)
    elif case == "signed_zeros":
        n, k = 5000, 64
        x = -np.abs(rng.standard_normal(n)).astype(np.float32) - 1
        x[rng.choice(n, 30, replace=False)] = 0.0
        x[rng.choice(n, 30, replace=False)] = -0.0
        x[rng.choice(n, 20, replace=False)] = 1.0
    elif case == "minus_inf":
        x = rng.standard_normal(n).astype(np.float32)
        x[rng.choice(n, n - 50, replace=False)] = -np.inf
    elif case == "two_slices":
        n, k = 1025, 64
        x = rng.standard_normal(n).astype(np.float32)
        x[1024] = 9.0
    elif case == "n_is_k":
        n, k = 64, 64
        x = rng.standard_normal(n).astype(np.float32)
    else:
        n, k = 1, 1
        x = np.array([-3.0], np.float32)
    vals, ids = ctx.alloc(k * 4), ctx.alloc(k * 4)
    ctx.topk(ctx.to_device(x), n, k, vals, ids)
    want = np.argsort(-x, kind="stable")[:k]
    assert list(ids.download(np.int32)) == list(want)
    assert np.array_equal(vals.download(np.float32), x[want])


def test_sampling_cfg4_matches_reference_draws(ctx):
    """cfg4's sampling step: GPU top-40 then the host draw (T 0.7, p 0.9) gives
    the reference engine's ids on the golden logit table."""
    import make_golden
    s = np.load(os.path.join(G, "sampler.npz"))
    table = make_golden.sampler_table(int(s["table_seed"]), int(s["rows"]), int(s["n_vocab"]))
    T, p, k = make_golden.SAMPLER_CASES[0]
    smp = ts5hip.Sampler(42)
    vals, ids = ctx.alloc(k * 4), ctx.alloc(k * 4)
    got = []
    for r in range(table.shape[0]):
        ctx.topk(ctx.to_device(table[r]), table.shape[1], k, vals, ids)
        got.append(smp.draw(ids.download(np.int32), vals.download(np.float32), T, p))
    assert got == list(s["ids0"])
