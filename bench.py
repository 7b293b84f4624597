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
# 32,442.0 KiB and WRITE_SIZE 448 KiB per dispatch, scaled by what the same
# counters read for the one-pass RMSNorm stream of 256 MiB in and 256 MiB out
# (131,226.9 and 262,144 KiB: factors 1.9976 and 1.0). 1.010 x the algorithmic
# bytes.
GLU_TRAFFIC_BYTES = 66821554
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


def cpu_baseline(hp, steps: int = 3, keys: int = PROMPT):
    """The CPU oracle decoding `steps` tokens of the same model shape at
    `keys` cached positions (KV seeded with random q8-rounded values)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle  # test infrastructure: the checker, timed only as the CPU baseline

    threads = min(os.cpu_count() or 1, 16)
    t0 = time.time()
    tensors = synth.model_tensors(hp, SEED)
    log(f"cpu baseline: host weights generated ({time.time() - t0:.1f} s)")
    m = oracle.Model(hp, tensors, keys + steps + 1, 2, threads=threads)
    rng = np.random.default_rng(3)
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
    return dict(value=round(steps / dt, 4), unit="tok/s", cores=threads, kind="port",
                sample=f"{steps} greedy decode steps of the cfg2 8B shape at {keys} seeded q8 keys, "
                       f"oracle/cpu_forward.cpp (fp64 dots, rows over {threads} threads)")


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
    ctx = ts5hip.Context(0)
    log(f"device {ctx.arch}, {ctx.n_cu} CUs, {ctx.hbm / 2**30:.0f} GiB")
    ms, ids, extra = decode_bench(ctx, hp, args.steps, args.warmup, args.prompt)
    roof = glu_roofline(ctx, hp)
    log(f"roofline: {roof}")
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
        "vs_baseline": None, "dtype": "q4_k/q6_k weights, int8 x int16 dot, fp32 accum",
        "data": "synthetic (random-init weights generated in HBM, uniform prompt ids)",
        "config": {"workload": "cfg2: Llama-style 8B decode, 4096-token prompt, greedy, q8 KV",
                   "global_batch": 1, "seq_len": args.prompt, "parallelism": "none (1 GPU)",
                   "decode_hbm_gbs": round(token_bytes * value / 1e9, 1),
                   "decode_roofline_frac": round(token_bytes * value / 1e9 / HBM_PEAK_GBS, 4), **extra},
        "roofline": roof, "cpu_baseline": cpu,
    }), flush=True)


if __name__ == "__main__":
    main()
