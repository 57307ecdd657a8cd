#!/usr/bin/env python3
"""Verified tokens/s of the speculative-decoding verify step on one MI355X.

Workload (configs[1], the metric's single-GPU case): the 16-layer 1B decoder (hidden 2048,
32/8 heads of 64, SwiGLU 8192, vocab 32000) with random int8 per-output-channel weights and a
tied bf16 head; one stream with 8192 cached tokens (paged KV, pages of 16, K/V ~ N(0, 1)); a
linear chain of k = 4 drafts per step; greedy acceptance with rollback of rejected rows.

Drafts come from the reference's replay drafter (kernels.metal:1695-1724): before timing, a
plain greedy decode records the target's own continuation; each verify step then drafts that
trace with a seeded 35% mistake rate (per-position agreement ~65%), so acceptance behaves as
with a real drafter and the emitted tokens must reproduce the trace (checked).

A step is one verify pass over the 5 rows (embed, 16 layers, head, sampler, accept, replay
drafter), captured once as a HIP graph and replayed back to back; `value` = tokens emitted
over the timed steps / their wall time, inputs resident in HBM.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "silicon-violetto_amd"))

METRIC = "verified tok/s @1 & 32 seqs, 8k ctx, k=4; verify-step HBM GB/s % of peak"
HBM_PEAK_GBS = 8000.0
KV_BYTES_PER_TOKEN_LAYER = 8 * 64 * 2 * 2  # NKV x D x bf16 x (K, V)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--ctx", type=int, default=8192)
    ap.add_argument("--draft", type=int, default=4, help="drafts per step (k)")
    ap.add_argument("--mistake-rate", type=float, default=0.35)
    ap.add_argument("--profile-reps", type=int, default=5, help="steps timed per kernel with hipEvents")
    ap.add_argument("--cpu-steps", type=int, default=2, help="oracle steps for the CPU baseline (0: skip)")
    ap.add_argument("--seed", type=int, default=0)
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for {max(args.gpus, world)}); "
              "streams shard across GPUs with no exchange, see DESIGN.md", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import violetto
    from violetto import _lib as L
    from violetto.model import CONFIG_SHAPE, SyntheticModel, rope_freq

    assert torch.cuda.is_available(), "bench.py needs an MI355X"
    shape = CONFIG_SHAPE
    ctx, k = args.ctx, args.draft
    rows = k + 1
    n_steps = args.warmup + args.steps + args.profile_reps + 4
    trace_n = rows * n_steps + 32
    max_seq_len = ctx + trace_n + 64

    t_setup = time.perf_counter()
    log(f"generating the 16-layer int8 model on the GPU (seed {args.seed})")
    model = SyntheticModel.generate(shape, int8=True, seed=args.seed, device="cuda")
    freq = rope_freq(500000.0, shape.head_dim)
    eng = violetto.Engine(shape, max_seqs=1, max_step_tokens=16, max_seq_len=max_seq_len, max_head_rows=16,
                          kv_tokens=max_seq_len, page_shift=4, attn_scale=0.125, freq=freq)
    eng.set_model(model)
    slot = eng.new_seq()
    eng.bench_fill(slot, ctx)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed + 1)
    kd, vd = eng.kv_cache()
    for t in (kd, vd):
        t.copy_(torch.randn(t.shape, generator=gen, device="cuda", dtype=torch.float32).to(torch.bfloat16))
    torch.cuda.synchronize()
    rng = np.random.default_rng(args.seed)
    t0 = int(rng.integers(0, shape.vocab_real))

    # The target's greedy continuation (plain decode, one row per step, graph-replayed).
    log(f"recording a {trace_n}-token greedy trace from position {ctx}")
    eng.set_feed(slot, ctx, t0)
    eng.plan([(slot, [L.FEED_ROW], False, 1)], extra_keys=trace_n + 8)
    eng.graph_capture(0)
    feed = eng.view("d_feed", (16,))
    trace = [t0]
    for _ in range(trace_n):
        eng.graph_replay(1)
        eng.sync()
        trace.append(int(feed[0].item()))
    tr = eng.view("d_trace", (1, max_seq_len))
    tr.zero_()
    tr[0, ctx:ctx + len(trace)] = torch.tensor(trace, dtype=torch.int32, device="cuda")
    eng.view("d_trace_len", (1,)).fill_(ctx + len(trace))
    torch.cuda.synchronize()

    # The verify step: run [input, d1..dk] from the GPU-fed rows; accept; replay drafts.
    eng.set_feed(slot, ctx, t0)
    eng.set_replay(args.seed + 7, args.mistake_rate)
    info = eng.plan([(slot, [L.FEED_ROW + i for i in range(rows)], True)], extra_keys=rows * n_steps + 8)
    eng.graph_capture(L.STEP_REPLAY)
    lens = eng.view("d_lens", (1,))
    eng.graph_replay(args.warmup)
    eng.sync()
    torch.cuda.synchronize()
    len0 = int(lens[0].item())
    log(f"setup {time.perf_counter() - t_setup:.1f} s; split {info.split} keys x {info.max_splits} splits; timing "
        f"{args.steps} steps")

    torch.cuda.synchronize()
    eng.sync()
    t_a = time.perf_counter()
    eng.graph_replay(args.steps)
    eng.sync()
    torch.cuda.synchronize()
    t_b = time.perf_counter()
    len1 = int(lens[0].item())
    emitted = len1 - len0
    secs = t_b - t_a
    ms_step = secs / args.steps * 1e3
    value = emitted / secs
    # Lossless check: the sequence's next input is the trace's token at its position.
    lossless = int(feed[0].item()) == trace[len1 - ctx]
    log(f"{emitted} tokens in {args.steps} steps ({emitted / args.steps:.2f}/step), {ms_step:.4f} ms/step, "
        f"{value:.0f} tok/s, trace reproduced: {lossless}")

    # Per-kernel durations, hipEvents on the engine's stream around each kernel.
    prof = eng.profile_step(L.STEP_REPLAY, reps=args.profile_reps)
    per_step_ms = {kk: v[0] / args.profile_reps for kk, v in prof.items() if v[1]}
    dominant = max(prof, key=lambda kk: prof[kk][0])
    H, F, V = shape.hidden, shape.ffn, shape.vocab
    mat_bytes = {"qkv": shape.qkv_width * H + 2 * shape.qkv_width, "o": H * H + 2 * H,
                 "gate_up": 2 * F * H + 2 * 2 * F, "down": H * F + 2 * H, "head": V * H * 2}
    ctx_mid = (len0 + len1) / 2
    attn_bytes = ctx_mid * KV_BYTES_PER_TOKEN_LAYER + rows * 2 * 8 * 64 * 2
    bytes_per_launch = mat_bytes.get(dominant, attn_bytes if dominant == "attn" else 0)
    d_ms, d_n = prof[dominant]
    d_avg_ms = d_ms / d_n
    achieved = bytes_per_launch / (d_avg_ms * 1e-3) / 1e9
    step_bytes = shape.weight_bytes(int8=True) + shape.n_layers * attn_bytes + rows * H * 2
    step_gbs = step_bytes / (ms_step * 1e-3) / 1e9
    log("per step (ms): " + ", ".join(f"{kk} {v:.4f}" for kk, v in per_step_ms.items()))

    cpu = None
    if args.cpu_steps > 0:
        cpu = cpu_baseline(args, shape, model, eng, kd, vd, trace, ctx, rows, freq)

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "verified tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights x fp32 activations (bf16 hi+lo MFMA, fp32 accumulate)",
        "data": "synthetic (random N(0,0.02) int8 weights, N(0,1) bf16 KV, replayed greedy drafts)",
        "config": {"workload": "configs[1]: 16-layer int8 1B verify step, 1 stream, 8192 ctx, k=4 chain, greedy, "
                               "KV rollback", "streams": 1, "ctx": ctx, "k": k, "rows_per_step": rows,
                   "draft_mistake_rate": args.mistake_rate},
        "emitted_per_step": round(emitted / args.steps, 3),
        "lossless_trace_check": lossless,
        "roofline": {"bound": "hbm", "kernel": dominant, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_launch": int(bytes_per_launch), "avg_launch_us": round(d_avg_ms * 1e3, 3)},
        "step_roofline": {"bytes_per_step": int(step_bytes), "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS,
                          "unit": "GB/s", "frac": round(step_gbs / HBM_PEAK_GBS, 4)},
        "kernel_ms_per_step": {kk: round(v, 4) for kk, v in per_step_ms.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    eng.close()
    return 0


def cpu_baseline(args, shape, model, eng, kd, vd, trace, ctx, rows, freq):
    """The oracle's verify step (C, OpenMP over output rows and heads) on this host's cores, on
    the same workload: args.cpu_steps steps of the 16-layer model at this context."""
    import numpy as np
    import torch

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    from violetto import _lib as L

    log(f"CPU baseline: copying the model to host, {args.cpu_steps} oracle steps")
    emb, lay, sc = oracle.host_weights(model)
    max_len = ctx + 16 * (args.cpu_steps + 2)
    ref = oracle.OracleEngine(L, shape, emb, lay, sc, max_seqs=1, max_seq_len=max_len, kv_tokens=max_len,
                              attn_scale=0.125, freq=freq)
    s = ref.new_seq()
    ref.bench_fill(s, ctx)
    pages = eng.seq_pages(0)[: ref.n_pages]
    assert pages == ref.pool.pages(s)[: len(pages)]
    n = min(ref.n_pages, kd.shape[1])
    ref.k[:, :n] = kd[:, :n].view(torch.int16).cpu().numpy().view(np.uint16)
    ref.v[:, :n] = vd[:, :n].view(torch.int16).cpu().numpy().view(np.uint16)
    ref.set_feed(s, ctx, trace[0])
    tr = np.zeros((1, max_len), np.uint32)
    m = min(len(trace), max_len - ctx)
    tr[0, ctx:ctx + m] = trace[:m]
    tr_len = np.array([ctx + m], np.uint32)
    ra = L.ReplayArgs(max_len, args.seed + 7, args.mistake_rate, shape.vocab_real)
    run_in = [L.RunIn(s, 0, rows, 0, rows, 1)]
    oracle.replay_draft(L, run_in, ref.lens, ref.feed, tr, tr_len, ra, ref.tree)
    emitted, secs = 0, 0.0
    for _ in range(args.cpu_steps):
        t_a = time.perf_counter()
        ids, _, em, _ = ref.step([(s, [L.FEED_ROW + i for i in range(rows)], True)])
        secs += time.perf_counter() - t_a
        emitted += int(em[0])
        oracle.replay_draft(L, run_in, ref.lens, ref.feed, tr, tr_len, ra, ref.tree)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    log(f"CPU: {emitted} tokens in {secs:.2f} s over {args.cpu_steps} steps, {threads} threads")
    return {"value": round(emitted / secs, 3), "unit": "verified tok/s", "cores": threads, "kind": "port",
            "sample": f"{args.cpu_steps} verify steps of the configs[1] workload (16 layers, 1 stream, {ctx} ctx, "
                      f"k={rows - 1}) by the C oracle, OpenMP over output rows and attention heads; "
                      f"{secs / args.cpu_steps:.2f} s/step"}


if __name__ == "__main__":
    sys.exit(main())
