#!/usr/bin/env python3
"""Verified tokens/s of the speculative-decoding verify step on one MI355X.

Model: the 16-layer 1B decoder of BASELINE.json (hidden 2048, 32/8 heads of 64, SwiGLU 8192,
vocab 32000), random int8 per-output-channel weights (N(0, 0.02) quantised), tied bf16 head;
paged KV cache (pages of 16 tokens) filled with N(0, 1) bf16.

`value` is configs[1] (the metric's 1-stream case): one stream at 8192 cached tokens, a
linear chain of k = 4 drafts per step, greedy acceptance with rollback of rejected rows.
The line also carries configs[2] (`streams32`): 32 streams with contexts U[1024, 8192],
page tables shuffled over a shared pool, T = 0.7 sampling with per-stream Philox seeds;
verify rows = 160.

Drafts come from the reference's replay drafter (kernels.metal:1695-1724): before timing, a
plain decode (greedy, or sampled with the streams' seeds) records the target's own
continuation; each verify step then drafts that trace with a seeded 35% mistake rate
(~65% per-position agreement), so acceptance behaves as with a real drafter and the emitted
tokens must reproduce the trace (checked: `lossless_trace_check`).

A step is one verify pass (embed, 16 layers, head, sampler, accept + replay drafter),
captured once as a HIP graph and replayed back to back; value = tokens emitted over the
timed steps / their wall time, with every input resident in HBM.
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
MFMA_BF16_PEAK_TFLOPS = 2500.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def sample_order(tok: int, vocab: int) -> int:
    """Position of id `tok` in the sampler's fixed order: thread t of 1024 owns ids t, t + 1024,
    ... in turn (kernels.metal:1484-1576)."""
    t, j = tok % 1024, tok // 1024
    return t * (vocab // 1024) + min(t, vocab % 1024) + j


def kv_bytes_per_token(shape) -> int:
    return shape.n_layers * shape.n_kv_heads * shape.head_dim * 2 * 2  # layers x heads x dims x bf16 x (K, V)


def run_workload(args, model, shape, *, streams: int, ctxs: list[int], temperature: float, shuffle: bool,
                 steps: int, warmup: int, profile_reps: int, seed: int, int8: bool = True, tree: bool = False):
    """Build the engine state for `streams` sequences, record their trace, time `steps`
    graph-replayed verify steps. Returns a dict of results (and the engine for reuse).

    tree: each stream verifies the fixed 16-node draft tree TREE_PARENTS every step (node ids
    random, drawn once; no replay drafter, no trace): the configs[4] workload."""
    import ctypes as C

    import numpy as np
    import torch

    import violetto
    from violetto import _lib as L
    from violetto.model import rope_freq

    k = args.draft
    rows = 16 if tree else k + 1
    n_steps = warmup + 2 * steps + profile_reps + 4  # the timed steps run twice (the re-run classifies)
    trace_n = rows * n_steps + 32
    max_ctx = max(ctxs)
    max_seq_len = max_ctx + trace_n + 64
    page = 16
    kv_tokens = sum(-(-(c + trace_n + 64) // page) * page for c in ctxs)
    freq = rope_freq(500000.0, shape.head_dim)
    eng = violetto.Engine(shape, max_seqs=streams, max_step_tokens=max(16, streams * rows),
                          max_seq_len=max_seq_len, max_head_rows=max(16, streams * rows), kv_tokens=kv_tokens,
                          page_shift=4, attn_scale=0.125, freq=freq, split_keys=args.split_keys,
                          options=L.OPT_LAYERS_KERNEL if args.layers_kernel else 0)
    eng.set_model(model)
    rng = np.random.default_rng(seed)
    slots = [eng.new_seq() for _ in range(streams)]
    seeds = [seed * 1000 + s + 1 for s in slots]
    for s, sd in zip(slots, seeds):
        eng.set_sampling(s, temperature, 1.0, sd)
    if shuffle:  # pages taken one at a time by randomly ordered sequences: shuffled tables
        left = {s: c for s, c in zip(slots, ctxs)}
        while left:
            s = int(rng.choice(list(left)))
            n = min(page, left[s])
            eng.bench_fill(s, n)
            left[s] -= n
            if left[s] == 0:
                del left[s]
    else:
        for s, c in zip(slots, ctxs):
            eng.bench_fill(s, c)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 1)
    kd, vd = eng.kv_cache()
    for t in (kd, vd):
        for l0 in range(0, t.shape[0], 4):
            t[l0:l0 + 4].copy_(torch.randn(t[l0:l0 + 4].shape, generator=gen, device="cuda").to(torch.bfloat16))
    torch.cuda.synchronize()
    first = [int(x) for x in rng.integers(0, shape.vocab_real, streams)]

    traces = None
    if tree:
        # The tree (parent, depth, ancestry mask per node: kernels.metal:64-72) and random node ids
        # as GPU-fed rows; accept leaves them in place (no replay drafter), so every step verifies
        # the same tree after the stream's newest token.
        depth = [0] * 16
        sees = [1] * 16
        for i in range(1, 16):
            depth[i] = depth[TREE_PARENTS[i]] + 1
            sees[i] = sees[TREE_PARENTS[i]] | (1 << i)
        nodes = np.array([depth[i] | ((0xFF if TREE_PARENTS[i] is None else TREE_PARENTS[i]) << 8) | (sees[i] << 16)
                          for i in range(16)], np.uint32)
        d_tree = eng.view("d_tree", (streams, 16))
        d_feed = eng.view("d_feed", (streams, 16))
        for s, c, t in zip(slots, ctxs, first):
            eng.set_feed(s, c, t)
            ids = np.concatenate([[t], rng.integers(0, shape.vocab_real, 15)]).astype(np.uint32)
            d_feed[s].copy_(torch.from_numpy(ids.view(np.int32)))
            d_tree[s].copy_(torch.from_numpy(nodes.view(np.int32)))
        torch.cuda.synchronize()
        info = eng.plan([(s, [L.FEED_ROW + i for i in range(rows)], True) for s in slots],
                        extra_keys=rows * n_steps + 8)
        eng.graph_capture(0)
        feed = d_feed
    else:
        # The target's own continuation: plain decode, one row per stream and step.
        log(f"{streams} stream(s): recording a {trace_n}-token trace per stream")
        for s, c, t in zip(slots, ctxs, first):
            eng.set_feed(s, c, t)
        eng.plan([(s, [L.FEED_ROW], False, 1) for s in slots], extra_keys=trace_n + 8)
        eng.graph_capture(0)
        feed = eng.view("d_feed", (streams, 16))
        traces = [[t] for t in first]
        for _ in range(trace_n):
            eng.graph_replay(1)
            eng.sync()
            col = feed[:, 0].cpu().tolist()
            for i, s in enumerate(slots):
                traces[i].append(int(col[s]))
        tr = eng.view("d_trace", (streams, max_seq_len))
        tr.zero_()
        for i, s in enumerate(slots):
            tr[s, ctxs[i]:ctxs[i] + len(traces[i])] = torch.tensor(traces[i], dtype=torch.int32, device="cuda")
        tl = eng.view("d_trace_len", (streams,))
        for i, s in enumerate(slots):
            tl[s] = ctxs[i] + len(traces[i])
        torch.cuda.synchronize()

        # Verify steps: [input, d1..dk] per stream from the GPU-fed rows; accept; replay drafts.
        for s, c, t in zip(slots, ctxs, first):
            eng.set_feed(s, c, t)
        eng.set_replay(seed + 7, args.mistake_rate)
        info = eng.plan([(s, [L.FEED_ROW + i for i in range(rows)], True) for s in slots],
                        extra_keys=rows * n_steps + 8)
        eng.graph_capture(L.STEP_REPLAY)
    lens = eng.view("d_lens", (streams,))
    divergences = []
    outv = eng.view("d_out_ids", (streams * rows,))
    seen = set()

    def checked_step(w, leg):
        """One replay, each stream's emitted tokens checked against its plain decode. Where they
        first differ, the distance between the drawn and the recorded id in the sampler's fixed
        order says what moved the draw: 1 is the neighbouring id (a CDF edge that the two
        computations' fp32 rounding put on different sides of the uniform)."""
        before = lens.cpu().numpy().astype(np.int64)
        eng.graph_replay(1)
        eng.sync()
        after = lens.cpu().numpy().astype(np.int64)
        out = outv.cpu().numpy().view(np.uint32)
        for i, s in enumerate(slots):
            if s in seen:
                continue
            got = [int(x) for x in out[rows * i: rows * i + after[s] - before[s]]]
            off = int(before[s]) - ctxs[i] + 1
            want = traces[i][off: off + len(got)]
            if got != want:
                m = next(j for j in range(len(got)) if j >= len(want) or got[j] != want[j])
                seen.add(s)
                divergences.append({"stream": s, "leg": leg, "step": w, "position": int(before[s]) + m,
                                    "order_distance": None if m >= len(want) else
                                    abs(sample_order(got[m], shape.vocab) - sample_order(want[m], shape.vocab))})
        return int((after - before).sum())

    if tree:
        eng.graph_replay(warmup)
        eng.sync()
    else:
        for w in range(warmup):
            checked_step(w, "warmup")
    # The state the timed steps start from (sequence state and K/V cache, on the device): after
    # timing, the same steps are re-run from it one at a time to classify every stream that leaves
    # its trace during them (graph replays are deterministic: the re-run emits the same tokens).
    snap = None
    if not tree:
        snap = {nm: eng.view(nm, shp).clone() for nm, shp in
                (("d_lens", (streams,)), ("d_feed", (streams * 16,)), ("d_tree", (streams * 16,)),
                 ("d_gen", (streams * C.sizeof(L.GenState) // 4,)))}
        snap["k"], snap["v"] = kd.clone(), vd.clone()
    len0 = lens.cpu().numpy().astype(np.int64)
    log(f"split {info.split} keys, grid {info.max_splits} splits; timing {steps} steps")
    torch.cuda.synchronize()
    eng.sync()
    t_a = time.perf_counter()
    eng.graph_replay(steps)
    eng.sync()
    torch.cuda.synchronize()
    t_b = time.perf_counter()
    len1 = lens.cpu().numpy().astype(np.int64)
    emitted = int((len1 - len0).sum())
    secs = t_b - t_a
    ms_step = secs / steps * 1e3
    fed = feed[:, 0].cpu().tolist()
    # Lossless check (bench_spec.rs:119-139): each stream's last emitted token is the one its plain
    # decode produced at that position.
    same = None if tree else [int(fed[s]) == traces[i][int(len1[s]) - ctxs[i]] for i, s in enumerate(slots)]
    lossless = None if tree else all(same)
    log(f"{emitted} tokens in {steps} steps ({emitted / steps:.2f}/step), {ms_step:.4f} ms/step, "
        f"{emitted / secs:.0f} tok/s, traces reproduced: {lossless}"
        + ("" if tree else f" ({sum(same)} of {len(same)} streams)"))

    prof = eng.profile_step(L.STEP_REPLAY, reps=profile_reps)
    per_step_ms = {kk: v[0] / profile_reps for kk, v in prof.items() if v[1]}
    rerun_emitted = None
    if snap is not None:
        for nm, shp in (("d_lens", (streams,)), ("d_feed", (streams * 16,)), ("d_tree", (streams * 16,)),
                        ("d_gen", (streams * C.sizeof(L.GenState) // 4,))):
            eng.view(nm, shp).copy_(snap[nm])
        kd.copy_(snap["k"])
        vd.copy_(snap["v"])
        del snap
        torch.cuda.synchronize()
        rerun_emitted = sum(checked_step(w, "timed") for w in range(steps))
        log(f"re-run of the timed steps: {rerun_emitted} tokens (timed: {emitted}); "
            f"{len(divergences)} stream(s) left the trace, order distances "
            f"{[d['order_distance'] for d in divergences]}")
    ctx_mid = float(((len0 + len1) / 2).sum())
    H, F, V = shape.hidden, shape.ffn, shape.vocab
    n_rows = streams * rows
    def wbytes(m, kk):  # int8 + one bf16 scale per row, or bf16
        return m * kk + 2 * m if int8 else 2 * m * kk

    mat_bytes = {"qkv": wbytes(shape.qkv_width, H), "o": wbytes(H, H), "gate_up": wbytes(2 * F, H),
                 "down": wbytes(H, F), "head": V * H * 2}
    attn_bytes = ctx_mid * kv_bytes_per_token(shape) / shape.n_layers + n_rows * 2 * shape.n_kv_heads * \
        shape.head_dim * 2
    step_bytes = shape.weight_bytes(int8=int8) + shape.n_layers * attn_bytes + n_rows * H * 2
    # the persistent layer kernel: every layer's four matrices and its attention's K/V
    layers_bytes = shape.n_layers * (sum(mat_bytes[kk] for kk in ("qkv", "o", "gate_up", "down")) + attn_bytes)
    mat_elems = {"qkv": shape.qkv_width * H, "o": H * H, "gate_up": 2 * F * H, "down": H * F}
    flops = 2 * n_rows * (shape.n_layers * sum(mat_elems.values()) + V * H)
    res = dict(eng=eng, kd=kd, vd=vd, traces=traces, ctxs=ctxs, slots=slots, seeds=seeds, replay_seed=seed + 7,
               steps=steps, warmup=warmup,
               emitted=emitted, secs=secs, ms_step=ms_step, value=emitted / secs, lossless=lossless,
               lossless_streams=None if tree else sum(same), divergences=divergences, prof=prof,
               rerun_emitted=rerun_emitted,
               per_step_ms=per_step_ms, attn_bytes=attn_bytes, mat_bytes=mat_bytes, step_bytes=step_bytes,
               layers_bytes=layers_bytes,
               flops=flops, info=info, rows=rows, mat_elems=mat_elems, n_rows=n_rows)
    return res


# configs[4]'s 16-node tree: root 0; children 1-4; two children under each (5-12); one leaf
# under each of 5, 6, 7 (13-15). The config's 1 + 4 + 8 + 8 = 21 nodes exceed the reference's
# 16 fed rows per run, so the last level keeps three leaves.
TREE_PARENTS = [None, 0, 0, 0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 5, 6, 7]


def extra_object(res, workload, rows, reps, key=None):
    return {"value": round(res["value"], 2), "unit": "verified tok/s", "ms_per_step": round(res["ms_step"], 5),
            "steps": res["steps"], "emitted_per_step": round(res["emitted"] / res["steps"], 3),
            "lossless_trace_check": res["lossless"], "config": {"workload": workload, "rows_per_step": rows},
            "roofline": roofline_of(res, reps, key), "step_roofline": step_roofline(res),
            "gemm_roofline": gemm_roofline(res),
            "kernel_ms_per_step": {kk: round(v, 4) for kk, v in res["per_step_ms"].items()}}


def gemm_roofline(res):
    """The verify step's GEMMs against the dense bf16 matrix-core peak: algorithmic flops per
    launch (2 n m k for n rows, the reference's product) / the kind's mean launch duration (the
    same hipExtLaunchKernelGGL events as `roofline`). The kernels run every product twice (bf16
    hi and lo halves of the fp32 activations), so `frac_hi_lo` counts the matrix-core work done.
    Meaningful at many rows (the GEMM path); below 17 rows the matmuls are HBM-bound GEMVs."""
    prof = res["prof"]
    per = {}
    for kk, elems in res["mat_elems"].items():
        if kk in prof and prof[kk][1]:
            us = prof[kk][0] / prof[kk][1] * 1e3
            tf = 2.0 * res["n_rows"] * elems / (us * 1e-6) / 1e12
            per[kk] = {"avg_launch_us": round(us, 3), "achieved": round(tf, 1)}
    if not per:
        return None
    dom = max(per, key=lambda kk: res["mat_elems"][kk])
    a = per[dom]["achieved"]
    return {"bound": "mfma", "kernel": dom, "achieved": a, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(a / MFMA_BF16_PEAK_TFLOPS, 4), "frac_hi_lo": round(2 * a / MFMA_BF16_PEAK_TFLOPS, 4),
            "flops_per_launch": int(2 * res["n_rows"] * res["mat_elems"][dom]), "avg_launch_us": per[dom]["avg_launch_us"],
            "per_matrix": per}


def roofline_of(res, profile_reps, workload=None):
    """The time-dominant kernel (most milliseconds per step; `layers`, the persistent kernel that
    runs every layer of a 1-8 row step, counts all its layers' weights and cached K/V) against
    the HBM peak: algorithmic bytes per launch / its mean duration (hipExtLaunchKernelGGL
    start/stop events around the kernel's own execution, over `profile_reps` steps of the timed
    workload). `by_bytes` gives the same for the kernel with the most algorithmic bytes per step
    where that is another one. `traffic` is the measured HBM bytes per launch (rocprofv3
    FETCH_SIZE + WRITE_SIZE, calibrated) from profiles/hbm_traffic.json when it holds this
    workload's kernel."""
    prof = res["prof"]
    per_launch = dict(res["mat_bytes"])
    per_launch["attn"] = res["attn_bytes"]
    per_launch["layers"] = res["layers_bytes"]
    live = [kk for kk in per_launch if kk in prof and prof[kk][1]]
    per_step_bytes = {kk: per_launch[kk] * prof[kk][1] / profile_reps for kk in live}
    per_step_ms = {kk: prof[kk][0] / profile_reps for kk in live}

    def of(kk):
        d_ms, d_n = prof[kk]
        d_avg_ms = d_ms / d_n
        achieved = per_launch[kk] / (d_avg_ms * 1e-3) / 1e9
        traffic = None
        tf = ROOT / "profiles" / "hbm_traffic.json"
        if workload and tf.exists():
            t = json.loads(tf.read_text()).get(workload, {}).get(kk)
            if t:
                traffic = int(t["fetch_bytes"] + t["write_bytes"])
        return {"bound": "hbm", "kernel": kk, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "bytes_per_launch": int(per_launch[kk]),
                "avg_launch_us": round(d_avg_ms * 1e3, 3), "ms_per_step": round(per_step_ms[kk], 4)}

    by_time = max(per_step_ms, key=per_step_ms.get)
    by_bytes = max(per_step_bytes, key=per_step_bytes.get)
    out = of(by_time)
    out["selected_by"] = "time"
    if by_bytes != by_time:
        b = of(by_bytes)
        out["by_bytes"] = {k: b[k] for k in ("kernel", "achieved", "frac", "bytes_per_launch", "avg_launch_us")}
    return out


def step_roofline(res):
    gbs = res["step_bytes"] / (res["ms_step"] * 1e-3) / 1e9
    tflops = res["flops"] / (res["ms_step"] * 1e-3) / 1e12
    bound_ms = max(res["step_bytes"] / (HBM_PEAK_GBS * 1e9), res["flops"] / (MFMA_BF16_PEAK_TFLOPS * 1e12)) * 1e3
    return {"bytes_per_step": int(res["step_bytes"]), "achieved_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "flops_per_step": int(res["flops"]), "achieved_tflops": round(tflops, 2),
            "roofline_ms": round(bound_ms, 4), "frac": round(bound_ms / res["ms_step"], 4)}


def run_drafter(args, streams: int, ctx: int, steps: int, reps: int = 3):
    """The drafter's pass (drafter.rs:278-447) after each verify step, at the reference drafter's
    shape (tools/spec/drafter.py: 2 layers of hidden 1280, 10 x 128 query heads over 2 kv heads,
    ffn 3328, two-tap convolutions, inject, window 1024; export.py: int8 groups of 64, the head
    over a 16384-id draft vocabulary in groups of 8) on a 4-layer target of the reference's
    dimensions (its depth does not enter the drafter's cost): `streams` slots `ctx` tokens in,
    blocks of 8 rows (the bonus token and 7 drafts, drafter.py BLOCK), each step verifying the
    tree the drafter wrote the step before. Graph-replayed steps with and without the pass; the
    pass's own kernels timed by hipEvents (kind "draft")."""
    import dataclasses

    import torch

    import violetto
    from violetto import _lib as L
    from violetto.drafter import SyntheticDrafter
    from violetto.model import REFERENCE_SHAPE, SyntheticModel, rope_freq

    shape = dataclasses.replace(REFERENCE_SHAPE, n_layers=4)
    rows = 8
    n_steps = 2 * (steps + reps) + 16
    max_seq_len = ctx + rows * n_steps + 64
    model = SyntheticModel.generate(shape, int8=True, seed=args.seed, device="cuda", group=64)
    eng = violetto.Engine(shape, max_seqs=streams, max_step_tokens=max(64, streams * rows), max_seq_len=max_seq_len,
                          max_head_rows=streams * rows, kv_tokens=streams * (max_seq_len + 16), page_shift=4,
                          attn_scale=0.1, freq=rope_freq(500000.0, shape.head_dim))
    eng.set_model(model)
    d = SyntheticDrafter.generate(shape, n_layers=2, taps=(1, 3), v=16384, window=1024, seed=args.seed + 5,
                                  device="cuda", group=64, head_group=8)
    eng.set_drafter(d)
    slots = [eng.new_seq() for _ in range(streams)]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed + 9)
    for s in slots:
        eng.bench_fill(s, ctx)
        eng.set_feed(s, ctx, int(torch.randint(0, shape.vocab_real, (1,), generator=gen, device="cuda")))
        eng.set_draft_rows(s, rows)
    kd, vd = eng.kv_cache()
    kr, vr, _ = eng.draft_rings()
    for t in (kd, vd, kr, vr):
        t.copy_(torch.randn(t.shape, generator=gen, device="cuda").to(torch.bfloat16))
    torch.cuda.synchronize()
    # the first step drafts from the bonus token; later steps verify the drafter's trees
    eng.plan([(s, [L.FEED_ROW], False, 1) for s in slots], extra_keys=8)
    eng.encode(L.STEP_DRAFT)
    eng.sync()
    out = {}
    for flags, key in ((0, "verify_only"), (L.STEP_DRAFT, "verify_and_draft")):
        eng.plan([(s, [L.FEED_ROW + i for i in range(rows)], True) for s in slots], extra_keys=rows * (steps + reps + 4))
        eng.graph_capture(flags)
        eng.graph_replay(2)
        eng.sync()
        t_a = time.perf_counter()
        eng.graph_replay(steps)
        eng.sync()
        out[key] = (time.perf_counter() - t_a) / steps * 1e3
    prof = eng.profile_step(L.STEP_DRAFT, reps=reps)
    per_step = {kk: v[0] / reps for kk, v in prof.items() if v[1]}
    # the bytes one pass reads: every drafter matrix once in its file format (the head's int8
    # groups of 8 included, read here as the exact bf16 hi + lo pair: 4 bytes a weight)
    file_bytes = sum(w.numel() * w.element_size() + (0 if sc is None else sc.numel() * 2) for w, sc in d.mats.values())
    head_w, head_s = d.mats["head"]
    read_bytes = file_bytes - head_w.numel() - head_s.numel() * 2 + 4 * head_w.numel()
    draft_ms = per_step.get("draft", float("nan"))
    eng.close()
    del model, d
    torch.cuda.empty_cache()
    gbs = file_bytes / (draft_ms * 1e-3) / 1e9
    return {"config": {"workload": f"drafter pass: {streams} slot(s) x {ctx} ctx, blocks of {rows} rows, reference "
                                   "drafter shape (2 layers, hidden 1280, v 16384, convs + inject, window 1024)",
                       "streams": streams, "ctx": ctx, "block_rows": rows},
            "ms_per_step_verify_only": round(out["verify_only"], 5),
            "ms_per_step_verify_and_draft": round(out["verify_and_draft"], 5),
            "draft_pass_ms": round(draft_ms, 5),
            "draft_weight_bytes": int(file_bytes), "draft_bytes_read": int(read_bytes),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
            "kernel_ms_per_step": {kk: round(v, 4) for kk, v in per_step.items()}}


def run_reference_model(args, streams: int, ctx: int, steps: int):
    """The reference's own model shape (engine/src/model.rs:6-21: Limite, 48 layers of hidden
    1280, 10 x 128 query heads over 2 kv heads, ffn 3328, vocabulary 151680; every fourth layer
    global, the others sliding-window layers of 1024 keys; value embeddings, gates, XSA, MUDD;
    int8 groups of 64, its own int8 head) with random weights, `streams` sequences `ctx` tokens
    in. Two graph-replayed steps, each timed over `steps`:
      - plain decode, one row per sequence (what docs/performance.md's "plain" column measures:
        one token per sequence per step whatever the weights, so its tok/s is comparable);
      - a verify step of an 8-row block per sequence plus the drafter's pass (the reference
        drafter's shape, tapping layers 35 and 47 as tools/spec/drafter.py TAPS), the step the
        reference's "with the drafter" column runs; random weights accept nothing, so only its
        time is reported."""
    import torch

    import violetto
    from violetto import _lib as L
    from violetto.drafter import SyntheticDrafter
    from violetto.model import REFERENCE_SHAPE, SyntheticModel, generate_extras, rope_freq

    shape = REFERENCE_SHAPE
    rows = 8
    max_seq_len = ctx + (rows + 1) * (2 * steps + 16) + 64
    model = SyntheticModel.generate(shape, int8=True, seed=args.seed, device="cuda", group=64)
    model = model.with_extras(generate_extras(shape, seed=args.seed + 3, device="cuda", window=1024)).with_head(64)
    eng = violetto.Engine(shape, max_seqs=streams, max_step_tokens=max(64, streams * rows), max_seq_len=max_seq_len,
                          max_head_rows=streams * rows, kv_tokens=streams * (max_seq_len + 16), page_shift=4,
                          attn_scale=0.1, freq=rope_freq(500000.0, shape.head_dim), local=model.extras.local,
                          window=1024)
    eng.set_model(model)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed + 11)
    slots = [eng.new_seq() for _ in range(streams)]
    for s in slots:
        eng.bench_fill(s, ctx)
        eng.set_feed(s, ctx, int(torch.randint(0, shape.vocab_real, (1,), generator=gen, device="cuda")))
    kd, vd = eng.kv_cache()
    kl, vl, _ = eng.local_cache()
    for t in (kd, vd, kl, vl):
        for l0 in range(0, t.shape[0], 4):
            t[l0:l0 + 4].copy_(torch.randn(t[l0:l0 + 4].shape, generator=gen, device="cuda").to(torch.bfloat16))
    torch.cuda.synchronize()
    out = {}
    # plain decode
    eng.plan([(s, [L.FEED_ROW], False, 1) for s in slots], extra_keys=steps + 8)
    eng.graph_capture(0)
    eng.graph_replay(3)
    eng.sync()
    t_a = time.perf_counter()
    eng.graph_replay(steps)
    eng.sync()
    ms = (time.perf_counter() - t_a) / steps * 1e3
    out["plain_decode"] = {"ms_per_step": round(ms, 4), "tok_per_s": round(streams / ms * 1e3, 1)}
    prof = eng.profile_step(0, reps=2)
    out["plain_decode"]["kernel_ms_per_step"] = {kk: round(v[0] / 2, 4) for kk, v in prof.items() if v[1]}
    # verify an 8-row block per sequence, then the drafter's pass
    d = SyntheticDrafter.generate(shape, n_layers=2, taps=(35, 47), v=16384, window=1024, seed=args.seed + 5,
                                  device="cuda", group=64, head_group=8)
    eng.set_drafter(d)
    for s in slots:
        eng.set_draft_rows(s, rows)
    kr, vr, _ = eng.draft_rings()
    for t in (kr, vr):
        t.copy_(torch.randn(t.shape, generator=gen, device="cuda").to(torch.bfloat16))
    eng.plan([(s, [L.FEED_ROW], False, 1) for s in slots], extra_keys=8)
    eng.encode(L.STEP_DRAFT)
    eng.sync()
    eng.plan([(s, [L.FEED_ROW + i for i in range(rows)], True) for s in slots], extra_keys=rows * (steps + 8))
    eng.graph_capture(L.STEP_DRAFT)
    eng.graph_replay(2)
    eng.sync()
    t_a = time.perf_counter()
    eng.graph_replay(steps)
    eng.sync()
    ms = (time.perf_counter() - t_a) / steps * 1e3
    prof = eng.profile_step(L.STEP_DRAFT, reps=2)
    per = {kk: round(v[0] / 2, 4) for kk, v in prof.items() if v[1]}
    out["verify_and_draft"] = {"ms_per_step": round(ms, 4), "draft_ms": per.get("draft"), "kernel_ms_per_step": per}
    eng.close()
    del d
    torch.cuda.empty_cache()
    if streams == 1:
        # prefill (docs/performance.md's prefill table): one prompt of `ctx` tokens in chunks of
        # 512 rows, each a step with its head row only on the last chunk, host planning included
        chunk = 512
        eng = violetto.Engine(shape, max_seqs=1, max_step_tokens=chunk, max_seq_len=ctx + 64, max_head_rows=16,
                              kv_tokens=ctx + 64, page_shift=4, attn_scale=0.1, freq=rope_freq(500000.0, shape.head_dim),
                              local=model.extras.local, window=1024)
        eng.set_model(model)
        prompt = torch.randint(0, shape.vocab_real, (ctx,), generator=gen, device="cuda").cpu().tolist()
        for rep in range(2):  # the first pass warms the kernels and the allocator
            s0 = eng.new_seq()
            torch.cuda.synchronize()
            t_a = time.perf_counter()
            for c0 in range(0, ctx, chunk):
                last = c0 + chunk >= ctx
                eng.step([(s0, prompt[c0:c0 + chunk], False, 1 if last else 0)])
            eng.sync()
            secs = time.perf_counter() - t_a
            eng.free_seq(s0)
        out["prefill"] = {"tokens": ctx, "chunk": chunk, "seconds": round(secs, 4), "tok_per_s": round(ctx / secs, 1)}
        eng.close()
    del model
    torch.cuda.empty_cache()
    return {"config": {"workload": f"reference model (Limite 48 layers, int8 groups of 64, window 1024, MUDD, value "
                                   f"embeddings), {streams} sequence(s) x {ctx} ctx, random weights",
                       "streams": streams, "ctx": ctx}, **out}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--ctx", type=int, default=8192)
    ap.add_argument("--draft", type=int, default=4, help="drafts per step (k)")
    ap.add_argument("--mistake-rate", type=float, default=0.35)
    ap.add_argument("--profile-reps", type=int, default=5, help="steps timed per kernel with hipEvents")
    ap.add_argument("--cpu-steps", type=int, default=2, help="oracle steps for the CPU baselines (0: skip)")
    ap.add_argument("--cpu-streams", type=int, default=4,
                    help="streams of configs[2] in its CPU baseline's sample (0: skip that baseline)")
    ap.add_argument("--streams32-steps", type=int, default=30, help="timed steps of configs[2] (0: skip)")
    ap.add_argument("--long-steps", type=int, default=20,
                    help="timed steps of configs[3] (bf16 weights, 65536 ctx, 1 and 8 streams; 0: skip)")
    ap.add_argument("--tree-steps", type=int, default=20, help="timed steps of configs[4] (16-node trees x 32; 0: skip)")
    ap.add_argument("--drafter-steps", type=int, default=20,
                    help="timed steps of the drafter's pass (1 and 32 slots, reference drafter shape; 0: skip)")
    ap.add_argument("--refmodel-steps", type=int, default=20,
                    help="timed steps of the reference's own model (plain decode and verify + draft, 1 and 32 "
                         "sequences at 8192 ctx; 0: skip)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--split-keys", type=int, default=0, help="attention keys per split (0: the engine's choice)")
    ap.add_argument("--layers-kernel", action="store_true",
                    help="run 1-8 row steps on the persistent layer kernel (SV_OPT_LAYERS_KERNEL)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="end with 4 elementwise passes over 256 MiB (the known-size kernel that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE into bytes)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for {max(args.gpus, world)} GPUs). "
              "Streams would shard across GPUs (one engine and page pool per GPU, a full weight "
              "replica each) with no exchange per step.", file=sys.stderr)
        return 2

    import torch

    from violetto.model import CONFIG_SHAPE, SyntheticModel

    assert torch.cuda.is_available(), "bench.py needs an MI355X"
    shape = CONFIG_SHAPE
    log(f"generating the 16-layer int8 model on the GPU (seed {args.seed})")
    model = SyntheticModel.generate(shape, int8=True, seed=args.seed, device="cuda")

    r1 = run_workload(args, model, shape, streams=1, ctxs=[args.ctx], temperature=0.0, shuffle=False,
                      steps=args.steps, warmup=args.warmup, profile_reps=args.profile_reps, seed=args.seed)
    log("per step (ms): " + ", ".join(f"{kk} {v:.4f}" for kk, v in r1["per_step_ms"].items()))
    cpu = cpu_baseline(args, shape, model, r1, [0], "configs[1]", 0.0) if args.cpu_steps > 0 else None
    r1["eng"].close()

    s32 = None
    if args.streams32_steps > 0:
        import numpy as np

        rng = np.random.default_rng(args.seed + 100)
        ctxs = [int(x) for x in rng.integers(1024, 8193, 32)]
        r2 = run_workload(args, model, shape, streams=32, ctxs=ctxs, temperature=0.7, shuffle=True,
                          steps=args.streams32_steps, warmup=8, profile_reps=2, seed=args.seed + 1)
        log("32 streams, per step (ms): " + ", ".join(f"{kk} {v:.4f}" for kk, v in r2["per_step_ms"].items()))
        cpu2 = (cpu_baseline(args, shape, model, r2, list(range(args.cpu_streams)), "configs[2]", 0.7)
                if args.cpu_steps > 0 and args.cpu_streams > 0 else None)
        s32 = {"value": round(r2["value"], 2), "unit": "verified tok/s", "ms_per_step": round(r2["ms_step"], 5),
               "steps": r2["steps"], "emitted_per_step": round(r2["emitted"] / r2["steps"], 3),
               "lossless_trace_check": r2["lossless"], "lossless_streams": r2["lossless_streams"],
               "divergences": r2["divergences"], "emitted": r2["emitted"], "rerun_emitted": r2["rerun_emitted"],
               "config": {"workload": "configs[2]: 32 streams, ctx U[1024,8192] (mean %d), shuffled page tables, "
                                      "k=4, T=0.7 Philox-seeded sample-and-match" % int(np.mean(ctxs)),
                          "rows_per_step": 32 * r2["rows"]},
               "roofline": roofline_of(r2, 2, "configs[2]"), "step_roofline": step_roofline(r2),
               "gemm_roofline": gemm_roofline(r2), "cpu_baseline": cpu2,
               "kernel_ms_per_step": {kk: round(v, 4) for kk, v in r2["per_step_ms"].items()}}
        r2["eng"].close()

    s64 = None
    if args.tree_steps > 0:
        r4 = run_workload(args, model, shape, streams=32, ctxs=[4096] * 32, temperature=0.7, shuffle=True,
                          steps=args.tree_steps, warmup=3, profile_reps=2, seed=args.seed + 4, tree=True)
        log("trees, per step (ms): " + ", ".join(f"{kk} {v:.4f}" for kk, v in r4["per_step_ms"].items()))
        s64 = extra_object(r4, "configs[4]: 32 streams x 16-node draft tree (random node ids), 4096 ctx, T=0.7 "
                               "Philox-seeded sample-and-match, accepted path compacted", 32 * 16, 2, "configs[4]")
        r4["eng"].close()
    del model
    torch.cuda.empty_cache()
    long_ctx = None
    if args.long_steps > 0:
        log(f"generating the 16-layer bf16 model on the GPU (seed {args.seed})")
        model16 = SyntheticModel.generate(shape, int8=False, seed=args.seed, device="cuda")
        long_ctx = {}
        for streams in (1, 8):
            r3 = run_workload(args, model16, shape, streams=streams, ctxs=[65536] * streams, temperature=0.0,
                              shuffle=False, steps=args.long_steps, warmup=3, profile_reps=2, seed=args.seed + 3,
                              int8=False)
            log(f"65536 ctx x {streams}, per step (ms): " + ", ".join(f"{kk} {v:.4f}" for kk, v in r3["per_step_ms"].items()))
            long_ctx[f"streams{streams}"] = extra_object(
                r3, f"configs[3]: bf16 weights, {streams} stream(s) x 65536 ctx, k=4 chain, greedy, KV rollback",
                streams * r3["rows"], 2, f"configs[3]x{streams}")
            if streams == 1 and args.cpu_steps > 0:
                # one oracle step (about 2 GB of bf16 weights and 64k keys per layer on the host)
                steps_saved, args.cpu_steps = args.cpu_steps, 1
                long_ctx["streams1"]["cpu_baseline"] = cpu_baseline(args, shape, model16, r3, [0], "configs[3]x1", 0.0)
                args.cpu_steps = steps_saved
            r3["eng"].close()
            torch.cuda.empty_cache()
        del model16

    drafter = None
    if args.drafter_steps > 0:
        drafter = {}
        for streams in (1, 32):
            log(f"drafter pass, {streams} slot(s)")
            drafter[f"streams{streams}"] = run_drafter(args, streams, 4096, args.drafter_steps)
            log(f"  {drafter[f'streams{streams}']}")

    refmodel = None
    if args.refmodel_steps > 0:
        refmodel = {}
        for streams in (1, 32):
            log(f"reference model, {streams} sequence(s)")
            refmodel[f"streams{streams}"] = run_reference_model(args, streams, 8192, args.refmodel_steps)
            log(f"  {refmodel[f'streams{streams}']}")

    line = {
        "metric": METRIC,
        "value": round(r1["value"], 2),
        "unit": "verified tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r1["ms_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights x fp32 activations (bf16 hi+lo MFMA, fp32 accumulate)",
        "data": "synthetic (random N(0,0.02) int8 weights, N(0,1) bf16 KV, replayed drafts of the target's own decode)",
        "config": {"workload": "configs[1]: 16-layer int8 1B verify step, 1 stream, 8192 ctx, k=4 chain, greedy, "
                               "KV rollback", "streams": 1, "ctx": args.ctx, "k": args.draft,
                   "rows_per_step": r1["rows"], "draft_mistake_rate": args.mistake_rate},
        "emitted_per_step": round(r1["emitted"] / args.steps, 3),
        "lossless_trace_check": r1["lossless"],
        "roofline": roofline_of(r1, args.profile_reps, "configs[1]"),
        "step_roofline": step_roofline(r1),
        "kernel_ms_per_step": {kk: round(v, 4) for kk, v in r1["per_step_ms"].items()},
        "cpu_baseline": cpu,
        "streams32": s32,
        "long_ctx_bf16": long_ctx,
        "trees32": s64,
        "drafter": drafter,
        "reference_model": refmodel,
    }
    print(json.dumps(line), flush=True)
    if args.calibrate_copy:
        # an elementwise kernel of known traffic: reads and writes 64 Mi floats (256 MiB each)
        src = torch.empty(64 << 20, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(4):
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        log("calibration: 4 elementwise passes over 256 MiB (read 256 MiB, write 256 MiB each)")
    return 0


def cpu_baseline(args, shape, model, res, picks, workload, temperature):
    """The oracle's verify step (C, OpenMP over output rows and heads) on this host's cores, on a
    bounded sample of a measured workload: args.cpu_steps verify steps of the 16-layer model for
    the streams `picks` (indices into the workload's streams), each at its context with the same
    cached K/V (copied by position from the GPU), sampling seeds and replayed drafts. Returns the
    cpu_baseline object; matches_gpu: the oracle emitted the GPU's recorded continuation."""
    import numpy as np
    import torch

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    from violetto import _lib as L
    from violetto.model import rope_freq

    eng, kd, vd, rows = res["eng"], res["kd"], res["vd"], res["rows"]
    log(f"CPU baseline ({workload}): copying the model to host, {len(picks)} stream(s), {args.cpu_steps} oracle steps")
    emb, lay, sc = oracle.host_weights(model)
    ctxs = [res["ctxs"][i] for i in picks]
    traces = [res["traces"][i] for i in picks]
    max_len = max(ctxs) + 16 * (args.cpu_steps + 2)
    ref = oracle.OracleEngine(L, shape, emb, lay, sc, max_seqs=len(picks), max_seq_len=max_len,
                              kv_tokens=len(picks) * max_len, attn_scale=0.125, freq=rope_freq(500000.0, shape.head_dim))
    tr = np.zeros((len(picks), max_len), np.uint32)
    tr_len = np.zeros(len(picks), np.uint32)
    run_in, runs = [], []
    for j, (i, ctx, trace) in enumerate(zip(picks, ctxs, traces)):
        s = ref.new_seq()
        ref.bench_fill(s, ctx)
        gpu_pages = eng.seq_pages(res["slots"][i])[: len(ref.pool.pages(s))]
        idx = torch.tensor(gpu_pages, device=kd.device)
        ref.k[:, ref.pool.pages(s)] = kd[:, idx].view(torch.int16).cpu().numpy().view(np.uint16)
        ref.v[:, ref.pool.pages(s)] = vd[:, idx].view(torch.int16).cpu().numpy().view(np.uint16)
        ref.set_sampling(s, temperature, 1.0, res["seeds"][i])
        ref.set_feed(s, ctx, trace[0])
        m = min(len(trace), max_len - ctx)
        tr[s, ctx:ctx + m] = trace[:m]
        tr_len[s] = ctx + m
        run_in.append(L.RunIn(s, rows * j, rows, rows * j, rows, 1))
        runs.append((s, [L.FEED_ROW + r for r in range(rows)], True))
    ra = L.ReplayArgs(max_len, res["replay_seed"], args.mistake_rate, shape.vocab_real)
    oracle.replay_draft(L, run_in, ref.lens, ref.feed, tr, tr_len, ra, ref.tree)
    emitted, secs, agree = 0, 0.0, True
    for _ in range(args.cpu_steps):
        pos = [int(ref.lens[s]) for s, _, _ in runs]
        t_a = time.perf_counter()
        ids, _, em, _ = ref.step(runs)
        secs += time.perf_counter() - t_a
        emitted += int(em.sum())
        for j, (s, _, _) in enumerate(runs):
            got = [int(x) for x in ids[rows * j: rows * j + int(em[j])]]
            want = traces[j][pos[j] - ctxs[j] + 1: pos[j] - ctxs[j] + 1 + int(em[j])]
            agree = agree and got == want
        oracle.replay_draft(L, run_in, ref.lens, ref.feed, tr, tr_len, ra, ref.tree)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    log(f"CPU ({workload}): {emitted} tokens in {secs:.2f} s over {args.cpu_steps} steps, {threads} threads; "
        f"oracle tokens = GPU trace: {agree}")
    return {"value": round(emitted / secs, 3), "unit": "verified tok/s", "cores": threads, "kind": "port",
            "matches_gpu": agree,
            "sample": f"{args.cpu_steps} verify steps of {len(picks)} of the workload's streams ({workload}: 16 "
                      f"layers, contexts {ctxs}, k={rows - 1}) by the C oracle, OpenMP over output rows and "
                      f"attention heads; {secs / args.cpu_steps:.2f} s/step; emitted tokens equal the GPU's: {agree}"}


if __name__ == "__main__":
    sys.exit(main())
