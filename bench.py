"""Benchmark of ts5's batch-1 token loop on one MI355X (BASELINE.json cfg2).

A Llama-style 8B (32 layers, hidden 4096, FFN 14336, 32/8 heads of 128,
vocab 128256) with random-init Q4_K weights (Q6_K head) and fp32 norms is
generated in HBM; a 4096-token prompt of uniform ids is prefilled into the q8
KV cache; then --steps greedy decode steps run at batch 1, each token the
argmax of the previous step's logits, one HIP graph replay per token. The
timed region is exactly those steps, bracketed by device synchronisation.

Beside the decode rate it reports:
  roofline      the dominant kernel (fused gate/up + SiLU, 45 % of a token's
                bytes) timed with HIP events on the library's stream over
                launches that rotate through > 1 GiB of weights (so the
                256 MB Infinity Cache cannot serve them), against 8 TB/s.
  cpu_baseline  the CPU oracle (a restatement of ts5's CPU backend,
                engine/src/cpu_backend.cpp) decoding a few tokens of the same
                model shape at ~4k keys on the host cores.

    python bench.py [--steps 256] [--warmup 8] [--gpus 1]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from tokenstation5_amd import synth, ts5hip  # noqa: E402

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the roofline kernel, from rocprofv3 --pmc runs of
# `bench.py --roofline-only` (profiles/glu_roofline_counters.md): FETCH_SIZE
# 32,477.4 KiB and WRITE_SIZE 448 KiB per dispatch, scaled by what the same
# counters read for the one-pass RMSNorm stream of 256 MiB in and 256 MiB out
# (131,237.4 and 262,144 KiB: factors 1.9975 and 1.0). 1.011 x the algorithmic
# bytes.
GLU_TRAFFIC_BYTES = 66888639
PROMPT = 4096
SEED = 20241201


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def decode_bench(ctx, hp, steps: int, warmup: int, prompt_len: int = PROMPT):
    """The timed decode; also the prompt's prefill rate and the cost of a
    5-token verify batch (one token + 4 drafts, all logits) against one step."""
    n_ctx = prompt_len + max(steps, warmup) + 16
    m = ts5hip.Model(ctx, hp, n_ctx)
    t0 = time.time()
    for name, t, ne0, ne1 in synth.tensor_specs(hp):
        m.synth_tensor(name, t, ne0, ne1, SEED)
    ctx.sync()
    log(f"weights generated in HBM ({time.time() - t0:.1f} s)")
    prompt = np.random.default_rng(SEED).integers(0, hp["n_vocab"], prompt_len).astype(np.int32)
    m.forward(prompt[:256], 0, logits=False)  # first use: graphs, batch buffers
    t0 = time.time()
    m.forward(prompt[:-1], 0, logits=False)
    prefill_s = time.time() - t0
    first = int(m.generate_greedy(int(prompt[-1]), prompt_len - 1, 1)[0])
    log(f"prefill of {prompt_len - 1} tokens: {prefill_s:.2f} s ({(prompt_len - 1) / prefill_s:.0f} tok/s, "
        f"256-token batches)")
    if warmup:
        m.generate_greedy(first, prompt_len, warmup)
    ctx.sync()
    ctx.timer_begin()
    ids = m.generate_greedy(first, prompt_len, steps)
    ms = ctx.timer_end()
    log(f"{steps} decode steps: {ms:.2f} ms ({steps / ms * 1e3:.1f} tok/s); ids[:8] {list(ids[:8])}")
    # Speculative verification at the end of the context: 5 tokens with every
    # position's logits, against a single step, both end to end (host logits).
    pos = prompt_len + steps
    batch = np.array(ids[-5:], np.int32)
    times = {}
    for n in (1, 5, 1, 5):
        t0 = time.time()
        for _ in range(10):
            m.forward(batch[:n], pos, all_logits=n > 1)
        times[n] = (time.time() - t0) / 10 * 1e3
    log(f"verify: 1 token {times[1]:.3f} ms, 5 tokens {times[5]:.3f} ms ({times[5] / times[1]:.2f}x)")
    m.close()
    extra = dict(prefill_tok_s=round((prompt_len - 1) / prefill_s, 1), step_ms_host=round(times[1], 3),
                 verify5_ms_host=round(times[5], 3), verify5_over_step=round(times[5] / times[1], 3))
    return ms, ids, extra


def glu_roofline(ctx, hp, launches: int = 200):
    """Fused gate/up + SiLU (k_mv_glu) alone on the library's stream, HIP events
    around `launches` launches cycling through > 1 GiB of weight copies (a
    token sweeps 4.3 GB of weights, so none of its matrices is still in the
    256 MB Infinity Cache when it comes round again). The stream is first
    given other work first (RMSNorm over 1 GiB, ~0.4 ms, once per 10 timed
    launches), during which the host queues every timed launch: the events
    then time kernels back to back, not the host's launch rate (which a
    profiler slows to ~40 us a launch)."""
    E, F = hp["n_embd"], hp["n_ff"]
    wb = ctx.weight_bytes(synth.Q4_K, E, F)
    copies = max(2, -(-(1100 << 20) // (2 * wb)))
    gates = [ctx.weight_synth(synth.Q4_K, E, F, 100 + i) for i in range(copies)]
    ups = [ctx.weight_synth(synth.Q4_K, E, F, 200 + i) for i in range(copies)]
    rng = np.random.default_rng(1)
    x = ctx.to_device((rng.standard_normal(E) * 100).astype(np.float32))
    nw = ctx.to_device((1 + 0.02 * rng.standard_normal(E)).astype(np.float32))
    out = ctx.alloc(F * 4)
    for i in range(copies):
        ctx.matvec_glu(synth.Q4_K, gates[i], ups[i], E, F, x, out, norm_w=nw, eps=1e-5)
    busy_n, busy_rows = 4096, 65536
    bx, by = ctx.alloc(busy_n * busy_rows * 4), ctx.alloc(busy_n * busy_rows * 4)
    ones = ctx.to_device(np.ones(busy_n, np.float32))
    bx.zero()
    ctx.sync()
    for _ in range(max(2, launches // 10)):
        ctx.rmsnorm(bx, ones, 1e-5, busy_n, busy_rows, by)
    ctx.timer_begin()
    for i in range(launches):
        ctx.matvec_glu(synth.Q4_K, gates[i % copies], ups[i % copies], E, F, x, out, norm_w=nw, eps=1e-5)
    ms = ctx.timer_end()
    avg_us = ms * 1e3 / launches
    # Weights, the fp32 input and norm weight, the fp32 output.
    algo = 2 * E // 256 * F * 144 + 2 * 4 * E + 4 * F
    achieved = algo / (avg_us * 1e-6) / 1e9
    for b in gates + ups + [bx, by]:
        b.free()
    return dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                frac=round(achieved / HBM_PEAK_GBS, 4), traffic=GLU_TRAFFIC_BYTES,
                kernel="k_mv<Q4K,1,4,MV_GLU> (ffn rmsnorm+gate+up+SiLU, 14336x4096 x2)", avg_us=round(avg_us, 2),
                algorithmic_bytes=int(algo))


_busy = {}


def queue_busy(ctx, launches: int):
    """After a sync, `launches` RMSNorm launches over 1 GiB (~0.4 ms each) on
    the library's stream: the host queues the timed launches behind them."""
    if ctx not in _busy:
        bx, by = ctx.alloc(4096 * 65536 * 4), ctx.alloc(4096 * 65536 * 4)
        bx.zero()
        _busy[ctx] = (bx, by, ctx.to_device(np.ones(4096, np.float32)))
    bx, by, ones = _busy[ctx]
    ctx.sync()
    for _ in range(launches):
        ctx.rmsnorm(bx, ones, 1e-5, 4096, 65536, by)


def timed(ctx, fn, n: int, warm: int = 3, busy: bool = True) -> float:
    """Mean microseconds of fn(i) over n calls on the library's stream, HIP
    events around them (after `warm` untimed ones). With `busy`, the stream is
    first given RMSNorm work over 1 GiB (~0.4 ms a launch, enough for the host
    to queue every timed launch meanwhile), so that the events time kernels
    back to back rather than the host's launch rate."""
    for i in range(warm):
        fn(i)
    if busy:
        queue_busy(ctx, 2 + n // 10)
    else:
        ctx.sync()
    ctx.timer_begin()
    for i in range(n):
        fn(i)
    return ctx.timer_end() * 1e3 / n


def free_busy(ctx):
    for b in _busy.pop(ctx, ())[:2]:
        b.free()


def timed_groups(ctx, fn, n: int, group: int, warm: int = 3) -> np.ndarray:
    """Microseconds per launch of fn(i) in each of n / group groups of
    back-to-back launches: an event on the library's stream between groups
    (group 1: between every two launches, which then also times the event's
    own gap), the launches queued behind ~0.4 ms RMSNorm launches so that the
    host's launch rate is not timed."""
    for i in range(warm):
        fn(i)
    queue_busy(ctx, 2 + n // 10)
    for i in range(n):
        if i % group == 0:
            ctx.timer_mark(i // group)
        fn(i)
    ctx.timer_mark(n // group)
    return ctx.timer_marks(n // group + 1).astype(np.float64) * 1e3 / group


def cfg1_matvec(ctx):
    """cfg1: the 4096x4096 Q4_K matvec alone, 40 rotated copies (378 MB, past
    the 256 MB Infinity Cache), 200 launches: the mean (events around all
    200), the median over 20 groups of 10 back-to-back launches, and the
    median of launches timed one by one (an event between every two, whose
    gap it includes)."""
    E = 4096
    copies = 40
    ws = [ctx.weight_synth(synth.Q4_K, E, E, 300 + i) for i in range(copies)]
    x = ctx.to_device(np.random.default_rng(1).standard_normal(E).astype(np.float32))
    y = ctx.alloc(E * 4)
    run = lambda i: ctx.matvec(synth.Q4_K, ws[i % copies], E, E, x, y)
    mean = timed(ctx, run, 200)
    med = float(np.median(timed_groups(ctx, run, 200, 10)))
    iso = float(np.median(timed_groups(ctx, run, 200, 1)))
    algo = E * E // 256 * 144 + 4 * E + 4 * E  # 9,469,952 B
    for w in ws:
        w.free()
    return dict(us_median=round(med, 2), gbs_median=round(algo / med / 1e3, 1), us_mean=round(mean, 2),
                gbs_mean=round(algo / mean / 1e3, 1), us_median_one_by_one=round(iso, 2), bytes=algo)


def cfg3_attention(ctx):
    """cfg3: flash decode over q8 (and f16) caches, one query per sequence,
    32/8 heads of 128, every key. K and V are drawn N(0,1) on the device and
    stored as the cache keeps them (q8: round_kv per 32 values; f16), q is
    N(0,1). Buffers are rotated so each launch reads past the Infinity Cache
    (> 300 MB of caches in rotation)."""
    H, HKV, HD = 32, 8, 128
    scale = float(np.float32(1) / np.sqrt(np.float32(HD)))
    out = {}
    for B in (1, 4, 16):
        for n in (8192, 32768):
            for kvn, f16 in (("q8", False), ("f16", True)):
                vb = 2 if f16 else 1
                cache = B * HKV * n * HD * vb
                copies = max(1, -(-(300 << 20) // (2 * cache)))
                bufs = []
                nval = B * HKV * n * HD
                kvt = ts5hip.KV_F16 if f16 else ts5hip.KV_Q8
                for c in range(copies):
                    k, v = ctx.alloc(cache), ctx.alloc(cache)
                    sk = sv = None
                    if not f16:
                        sk, sv = ctx.alloc(cache // 16), ctx.alloc(cache // 16)
                    ctx.kv_synth(1000 * B + 10 * c + 1, nval, kvt, k, sk)
                    ctx.kv_synth(1000 * B + 10 * c + 2, nval, kvt, v, sv)
                    bufs.append((k, sk, v, sv))
                q = ctx.to_device(np.random.default_rng(B).standard_normal((B, H * HD)).astype(np.float32))
                o = ctx.alloc(B * H * HD * 4)
                nk = ctx.to_device(np.full(B, n, np.int32))

                def run(i):
                    k, sk, v, sv = bufs[i % copies]
                    if f16:
                        ctx.attn_decode_f16(q, B, H, HKV, HD, k, v, n, nk, 1, scale, o)
                    else:
                        ctx.attn_decode(q, B, H, HKV, HD, k, sk, v, sv, n, nk, 1, scale, o)

                us = timed(ctx, run, 40 if B * n <= 65536 else 10)
                algo = B * n * HKV * 2 * HD * (vb + (0 if f16 else 2 / 32)) + 2 * B * H * HD * 4
                out[f"{kvn}_B{B}_{n // 1024}k"] = dict(us=round(us, 1), gbs=round(algo / us / 1e3, 1))
                for t in bufs:
                    for b in t:
                        if b is not None:
                            b.free()
    return out


def cfg4_head_sampling(ctx):
    """cfg4: the Q6_K head 128256x4096 (431 MB, two copies in rotation), then
    the GPU top-40 and the host draw at T 0.7, p 0.9; and the head with the
    greedy pick fused in."""
    E, V = 4096, 128256
    ws = [ctx.weight_synth(synth.Q6_K, E, V, 400 + i) for i in range(2)]
    rng = np.random.default_rng(4)
    h = ctx.to_device(rng.standard_normal(E).astype(np.float32))
    nw = ctx.to_device((1 + 0.02 * rng.standard_normal(E)).astype(np.float32))
    y, out = ctx.alloc(V * 4), ctx.alloc(4)
    head = timed(ctx, lambda i: ctx.matvec(synth.Q6_K, ws[i % 2], E, V, h, y, norm_w=nw, eps=1e-5), 50)
    fused = timed(ctx, lambda i: ctx.matvec_argmax(synth.Q6_K, ws[i % 2], E, V, h, y, out, norm_w=nw, eps=1e-5), 50)
    vals, ids = ctx.alloc(40 * 4), ctx.alloc(40 * 4)
    topk = timed(ctx, lambda i: ctx.topk(y, V, 40, vals, ids), 50)
    smp = ts5hip.Sampler(7)
    t0 = time.perf_counter()
    for _ in range(100):
        smp.draw(ids.download(np.int32), vals.download(np.float32), 0.7, 0.9)
    draw_us = (time.perf_counter() - t0) / 100 * 1e6
    for w in ws:
        w.free()
    algo = V * E // 256 * 210 + 4 * E * 2 + 4 * V
    return dict(head_us=round(head, 1), head_gbs=round(algo / head / 1e3, 1), head_argmax_us=round(fused, 1),
                topk40_us=round(topk, 1), host_draw_us=round(draw_us, 1),
                step_us=round(head + topk + draw_us, 1))


def cfg5_speculation(ctx, gen: int = 512, prompt_len: int = 2048):
    """cfg5: the 24-layer 896-wide draft model proposing k = 4 per step for
    the 48-layer 5120-wide target and for the 8B, after a 2048-token prompt
    of uniform ids, 512 tokens, greedy (random-init weights of the configs'
    own distribution). Per target: tok/s without and with drafting, output
    equality, drafted / accepted by source (prompt lookup, draft model), a
    5-token verify forward against one step, and the draft model's time per
    drafted token. Q4_K weights are centred (synth.blocks): with the configs'
    own distribution every weight's mean is far above zero, a random model's
    argmax hardly depends on its input (one token repeated), and prompt lookup
    rather than the draft model would do all the drafting."""
    n_ctx = prompt_len + gen + 16
    draft = ts5hip.Model(ctx, synth.DRAFT_0P5B, n_ctx)
    for name, t, ne0, ne1 in synth.tensor_specs(synth.DRAFT_0P5B):
        draft.synth_tensor(name, t, ne0, ne1, SEED + 5, centered=True)
    res = {}
    for tag, hp in (("target_48x5120", synth.TARGET_14B), ("llama_8b", synth.LLAMA_8B)):
        m = ts5hip.Model(ctx, hp, n_ctx)
        for name, t, ne0, ne1 in synth.tensor_specs(hp):
            m.synth_tensor(name, t, ne0, ne1, SEED + 5, centered=True)
        prompt = np.random.default_rng(5).integers(0, hp["n_vocab"], prompt_len).astype(np.int32)
        runs, sources = {}, {}
        for k in (0, 4):
            e = ts5hip.Engine(m)
            e.set_drafter(draft if k else None)
            e.generate(prompt, temperature=0.0, max_tokens=8, draft=k)  # the prompt cached on both models
            t0 = time.time()
            ids, st = e.generate(prompt, temperature=0.0, max_tokens=gen, draft=k)
            dt = time.time() - t0
            runs[k] = (ids, st, dt)
            sources[k] = e.draft_sources()
            e.close()
        pos = prompt_len + 8
        batch = np.array(runs[0][0][:5], np.int32)

        def fwd(model, n):  # the engine's call: every row's logits kept in HBM
            ctx.check(ts5hip.lib().ts5hip_forward_in_place(model.h, batch.ctypes.data, n, pos, int(n > 1)))

        step = timed(ctx, lambda i: fwd(m, 1), 10, 2, busy=False)
        verify = timed(ctx, lambda i: fwd(m, 5), 10, 2, busy=False)
        dstep = timed(ctx, lambda i: fwd(draft, 1), 10, 2, busy=False)
        (ids0, st0, dt0), (ids4, st4, dt4) = runs[0], runs[4]
        same = bool(np.array_equal(ids0, ids4))
        div = None
        if not same:
            # Where drafting changed the greedy output, and how close the
            # undrafted run's top two logits were there (the verify batches
            # write the cache through the batch kernels, whose float sums
            # run in another order than the single-step kernels').
            d = next((i for i in range(min(len(ids0), len(ids4))) if ids0[i] != ids4[i]), min(len(ids0), len(ids4)))
            if d < min(len(ids0), len(ids4)):
                lg = m.forward(prompt, 0, logits=d == 0)  # its last row predicts ids0[0]
                for i in range(d):  # ids0[i] at prompt_len + i predicts ids0[i + 1]
                    lg = m.forward(np.array([ids0[i]], np.int32), prompt_len + i, logits=i == d - 1)
                row = np.sort(np.asarray(lg[0], np.float64))
                div = dict(at=int(d), top2_gap_rel=float((row[-1] - row[-2]) / abs(row[-1])))
        res[tag] = dict(tok_s_draft0=round(gen / dt0, 1), tok_s_draft4=round(gen / dt4, 1),
                        same_output=same, first_divergence=div, distinct_ids=int(np.unique(ids0).size),
                        drafted=int(st4[3]), accepted=int(st4[4]), **sources[4],
                        step_ms=round(step / 1e3, 3), verify5_ms=round(verify / 1e3, 3),
                        verify5_over_step=round(verify / step, 3), draft_ms_per_token=round(dstep / 1e3, 3))
        log(f"cfg5 {tag}: {res[tag]}")
        m.close()
    draft.close()
    return res


def draft_only(prompt_len: int = 2048, steps: int = 32):
    """cfg5's draft model alone (centred random weights generated in HBM): the
    prompt, then `steps` greedy tokens of the device-resident loop, timed on
    the host around the loop."""
    ctx = ts5hip.Context(0)
    hp = synth.DRAFT_0P5B
    m = ts5hip.Model(ctx, hp, prompt_len + steps + 16)
    for name, t, ne0, ne1 in synth.tensor_specs(hp):
        m.synth_tensor(name, t, ne0, ne1, SEED + 5, centered=True)
    prompt = np.random.default_rng(5).integers(0, hp["n_vocab"], prompt_len).astype(np.int32)
    first = int(np.argmax(m.forward(prompt, 0)[0]))
    ctx.sync()
    t0 = time.perf_counter()
    m.generate_greedy(first, prompt_len, steps)
    dt = time.perf_counter() - t0
    print(json.dumps({"draft_ms_per_token": round(dt / steps * 1e3, 3), "steps": steps, "prompt": prompt_len}),
          flush=True)
    m.close()
    ctx.close()


def kernel_profile(hp, prompt_len: int = PROMPT, steps: int = 32):
    """take_profile with TS5_PROFILE=1 over cfg2's decode: GPU time per kernel
    and weight role of `steps` greedy tokens after the prompt, from event nodes
    in the token's graph (or, with TS5HIP_GRAPHS=0, events after its direct
    launches)."""
    os.environ["TS5_PROFILE"] = "1"
    ctx = ts5hip.Context(0)
    m = ts5hip.Model(ctx, hp, prompt_len + steps + 16)
    for name, t, ne0, ne1 in synth.tensor_specs(hp):
        m.synth_tensor(name, t, ne0, ne1, SEED)
    prompt = np.random.default_rng(SEED).integers(0, hp["n_vocab"], prompt_len).astype(np.int32)
    m.forward(prompt[:-1], 0, logits=False)
    first = int(m.generate_greedy(int(prompt[-1]), prompt_len - 1, 1)[0])
    m.take_profile()  # the prompt's and the first token's
    m.generate_greedy(first, prompt_len, steps)
    print(f"token path: {m.token_path()}")
    print(m.take_profile(), flush=True)
    m.close()
    ctx.close()


def roofline_only(hp):
    """The roofline kernel's launches alone, then one RMSNorm over 256 MiB
    (k_rmsnorm_reg: 16384 rows of 4096 values, each row held in registers
    between its sum and its write, so it reads 256 MiB once and writes 256 MiB
    once): the known-size stream that scales the hardware counters
    (FETCH_SIZE, WRITE_SIZE) of a rocprofv3 --pmc run of this mode."""
    ctx = ts5hip.Context(0)
    roof = glu_roofline(ctx, hp, launches=40)
    n, rows = 4096, 16384
    x = ctx.alloc(n * rows * 4)
    y = ctx.alloc(n * rows * 4)
    x.zero()
    w = ctx.to_device(np.ones(n, np.float32))
    ctx.rmsnorm(x, w, 1e-5, n, rows, y)
    ctx.sync()
    ctx.close()
    print(json.dumps({"roofline": roof, "stream_kernel": "k_rmsnorm", "stream_read_bytes": n * rows * 4,
                      "stream_write_bytes": n * rows * 4}), flush=True)


def prefill_only(hp, prompt_len: int = PROMPT):
    """The prompt alone (for rocprofv3 runs of the prefill kernels): one
    256-token chunk to warm up, then the prompt's prefill into the q8 cache,
    timed with HIP events on the library's stream."""
    ctx = ts5hip.Context(0)
    m = ts5hip.Model(ctx, hp, prompt_len + 16)
    for name, t, ne0, ne1 in synth.tensor_specs(hp):
        m.synth_tensor(name, t, ne0, ne1, SEED)
    prompt = np.random.default_rng(SEED).integers(0, hp["n_vocab"], prompt_len).astype(np.int32)
    m.forward(prompt[:256], 0, logits=False)
    ctx.sync()
    ctx.timer_begin()
    m.forward(prompt, 0, logits=False)
    ms = ctx.timer_end()
    m.close()
    ctx.close()
    print(json.dumps({"prefill_tokens": prompt_len, "prefill_ms": round(ms, 2),
                      "prefill_tok_s": round(prompt_len / ms * 1e3, 1)}), flush=True)


def verify_only(hp, prompt_len: int = PROMPT, reps: int = 20):
    """The verify batch alone (for rocprofv3 runs of the several-token
    kernels): after the prompt, `reps` forwards of 5 tokens (one token + 4
    drafts, every row's logits kept in HBM, as the engine's speculative step
    calls it) and `reps` single-token forwards at the same position, each
    set timed with HIP events on the library's stream."""
    ctx = ts5hip.Context(0)
    m = ts5hip.Model(ctx, hp, prompt_len + 16)
    for name, t, ne0, ne1 in synth.tensor_specs(hp):
        m.synth_tensor(name, t, ne0, ne1, SEED)
    prompt = np.random.default_rng(SEED).integers(0, hp["n_vocab"], prompt_len).astype(np.int32)
    m.forward(prompt, 0, logits=False)
    batch = np.ascontiguousarray(prompt[-5:])

    def fwd(n):
        ctx.check(ts5hip.lib().ts5hip_forward_in_place(m.h, batch.ctypes.data, n, prompt_len, int(n > 1)))

    step = timed(ctx, lambda i: fwd(1), reps, 2, busy=False)
    verify = timed(ctx, lambda i: fwd(5), reps, 2, busy=False)
    m.close()
    ctx.close()
    print(json.dumps({"step_us": round(step, 1), "verify5_us": round(verify, 1),
                      "verify5_over_step": round(verify / step, 3)}), flush=True)


def cpu_baseline(hp, steps: int = 4, keys: int = PROMPT):
    """The CPU oracle (the restatement of ts5's CPU backend: per-row dequant,
    fp64 dots, rows striped over threads) on the host cores: the cfg2 8B
    decoding `steps` tokens at `keys` cached positions (KV seeded with random
    q8-rounded values), and cfg1's matvec and cfg4's head with all threads
    and with one."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle  # test infrastructure: the checker, timed only as the CPU baseline

    nproc = os.cpu_count() or 1
    threads = min(nproc, 16)  # the GPU box's share of host cores
    rng = np.random.default_rng(3)
    W1 = synth.tensor(synth.Q4_K, 4096, 4096, SEED, "cfg1")
    x1 = rng.standard_normal(4096).astype(np.float32)

    def best_ms(fn, reps):
        t = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            t.append((time.perf_counter() - t0) * 1e3)
        return float(np.median(t))

    cfg1_ms = best_ms(lambda: oracle.matmul(synth.Q4_K, W1, 4096, x1, threads=threads), 9)
    cfg1_ms_1t = best_ms(lambda: oracle.matmul(synth.Q4_K, W1, 4096, x1, threads=1), 3)
    t0 = time.time()
    tensors = synth.model_tensors(hp, SEED)
    log(f"cpu baseline: host weights generated ({time.time() - t0:.1f} s)")
    head = tensors["output.weight"][3]
    cfg4_ms = best_ms(lambda: oracle.matmul(synth.Q6_K, head, 4096, x1, threads=threads), 3)
    cfg4_ms_1t = best_ms(lambda: oracle.matmul(synth.Q6_K, head, 4096, x1, threads=1), 1)
    m = oracle.Model(hp, tensors, keys + steps + 1, 2, threads=threads)
    for layer in range(hp["n_layer"]):
        for which in (0, 1):
            kv = m.kv(which, layer)
            kv[:keys] = oracle.round_kv(2, rng.standard_normal(kv[:keys].size).astype(np.float32)).reshape(keys, -1)
    tok = np.array([1], np.int32)
    m.forward(tok, keys)  # warm
    t0 = time.time()
    for i in range(steps):
        lg = m.forward(tok, keys + 1 + i)
        tok = np.array([int(np.argmax(lg[0]))], np.int32)
    dt = time.time() - t0
    return dict(value=round(steps / dt, 4), unit="tok/s", cores=threads, kind="port", nproc=nproc,
                sample=f"{steps} greedy decode steps of the cfg2 8B shape at {keys} seeded q8 keys, "
                       f"oracle/cpu_forward.cpp (per-row dequant, fp64 dots, rows over {threads} of {nproc} "
                       f"host threads); cfg1 / cfg4 matvecs median of 9 / 3 runs",
                cfg1_matvec_ms=round(cfg1_ms, 2), cfg1_matvec_ms_1thread=round(cfg1_ms_1t, 2),
                cfg4_head_ms=round(cfg4_ms, 1), cfg4_head_ms_1thread=round(cfg4_ms_1t, 1))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--prompt", type=int, default=PROMPT, help="prompt length (cfg2: 4096)")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the roofline kernel's launches and a 256 MiB device copy (for rocprofv3 --pmc)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the prompt's prefill, timed on the device (for rocprofv3 runs)")
    ap.add_argument("--verify-only", action="store_true",
                    help="only 5-token verify forwards and single steps, device-timed (for rocprofv3 runs)")
    ap.add_argument("--no-configs", action="store_true", help="skip the cfg1/cfg3/cfg4/cfg5 measurements")
    ap.add_argument("--no-spec", action="store_true", help="skip cfg5 (draft model + two targets, ~1 min)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the cfg2 decode and its JSON line (for rocprofv3 runs)")
    ap.add_argument("--draft-only", action="store_true",
                    help="only cfg5's draft model: a 2048-token prompt, then 32 greedy tokens (for rocprofv3 runs)")
    ap.add_argument("--target-only", action="store_true",
                    help="only cfg5's 48x5120 target: a 2048-token prompt, then greedy decode (for rocprofv3 runs)")
    ap.add_argument("--cfg3-only", action="store_true",
                    help="only cfg3's attention configurations and their JSON (for rocprofv3 runs)")
    ap.add_argument("--kernel-profile", action="store_true",
                    help="only take_profile (TS5_PROFILE=1) of 32 decode tokens: GPU time per kernel and role")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this backend runs ts5's token loop on one GPU (batch 1); "
              "there is no multi-GPU path to measure.", file=sys.stderr)
        sys.exit(2)
    hp = dict(synth.LLAMA_8B)
    if args.roofline_only:
        roofline_only(hp)
        return
    if args.prefill_only:
        prefill_only(hp, args.prompt)
        return
    if args.verify_only:
        verify_only(hp, args.prompt)
        return
    if args.draft_only:
        draft_only()
        return
    if args.kernel_profile:
        kernel_profile(hp, args.prompt)
        return
    if args.target_only:
        ctx = ts5hip.Context(0)
        steps = min(args.steps, 64)
        ms, _, extra = decode_bench(ctx, dict(synth.TARGET_14B), steps, args.warmup, 2048)
        print(json.dumps({"target_48x5120_tok_s": round(steps / ms * 1e3, 1), **extra}), flush=True)
        ctx.close()
        return
    if args.cfg3_only:
        ctx = ts5hip.Context(0)
        print(json.dumps({"cfg3_attention": cfg3_attention(ctx)}), flush=True)
        ctx.close()
        return
    ctx = ts5hip.Context(0)
    log(f"device {ctx.arch}, {ctx.n_cu} CUs, {ctx.hbm / 2**30:.0f} GiB")
    ms, ids, extra = decode_bench(ctx, hp, args.steps, args.warmup, args.prompt)
    configs = {}
    if args.decode_only:
        roof = None
        args.no_cpu = True
    else:
        roof = glu_roofline(ctx, hp)
        log(f"roofline: {roof}")
        if not args.no_configs:
            configs["cfg1_q4k_matvec_4096"] = cfg1_matvec(ctx)
            log(f"cfg1: {configs['cfg1_q4k_matvec_4096']}")
            configs["cfg3_attention"] = cfg3_attention(ctx)
            log(f"cfg3: {configs['cfg3_attention']}")
            configs["cfg4_head_sampling"] = cfg4_head_sampling(ctx)
            log(f"cfg4: {configs['cfg4_head_sampling']}")
            free_busy(ctx)
            if not args.no_spec:
                configs["cfg5_speculation"] = cfg5_speculation(ctx)
    ctx.close()
    cpu = None if args.no_cpu else cpu_baseline(hp)
    if cpu:
        log(f"cpu baseline: {cpu}")
    value = args.steps / (ms / 1e3)
    wb = synth.weight_bytes(hp)
    token_bytes = wb["layers"] + wb["head"] + wb["norms"] + wb["embd_row"] + \
        (hp["n_layer"]) * (args.prompt + args.steps / 2) * hp["n_head_kv"] * hp["head_dim"] * 2 * (1 + 2 / 32)
    print(json.dumps({
        "metric": "decode tok/s (8B Q4_K, bs1, 4k ctx, 1 GPU)",
        "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "q4_k/q6_k weights, int8 x 23-bit activation dot (exact int32), fp32 accum",
        "data": "synthetic (random-init weights generated in HBM, uniform prompt ids)",
        "config": {"workload": "cfg2: Llama-style 8B decode, 4096-token prompt, greedy, q8 KV",
                   "global_batch": 1, "seq_len": args.prompt, "parallelism": "none (1 GPU)",
                   "decode_hbm_gbs": round(token_bytes * value / 1e9, 1),
                   "decode_roofline_frac": round(token_bytes * value / 1e9 / HBM_PEAK_GBS, 4), **extra,
                   **configs},
        "roofline": roof, "cpu_baseline": cpu,
    }), flush=True)


if __name__ == "__main__":
    main()
