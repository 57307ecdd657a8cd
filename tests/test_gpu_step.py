"""End-to-end verify steps on the GPU engine against the oracle engine (BASELINE.json
configs[0] and smaller variants), through the C ABI.

Bar (north star): logits within 2e-2 max-abs / 1e-2 relative; greedy ids equal wherever the
oracle's top-1 margin exceeds 2e-2; accepted counts, emitted ids, paths, lengths and page
tables bit-exact."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

import oracle
from conftest import banner
from helpers import close, greedy_ids_match
from violetto import _lib as L
from violetto.engine import Engine
from violetto.model import LayerScalars, ModelShape, SyntheticModel, rope_freq

pytestmark = pytest.mark.gpu

LOGIT_ATOL, LOGIT_RTOL = 2e-2, 1e-2


def build_pair(shape: ModelShape, *, ctx: int, n_seqs: int = 1, seed: int = 0, int8: bool = True, page_shift=4,
               max_seq_len=1024, scalars=None, shuffle=False, split_keys=0, max_head_rows=16, fast_kv=False,
               options=0):
    model = SyntheticModel.generate(shape, int8=int8, seed=seed, device="cpu", scalars=scalars)
    freq = rope_freq(500000.0, shape.head_dim)
    eng = Engine(shape, max_seqs=n_seqs, max_step_tokens=16 * n_seqs, max_seq_len=max_seq_len, max_head_rows=max_head_rows,
                 kv_tokens=n_seqs * max_seq_len, page_shift=page_shift, attn_scale=0.125, freq=freq,
                 split_keys=split_keys, options=options)
    gm = model.to("cuda")
    eng.set_model(gm)
    emb, lay, sc = oracle.host_weights(model)
    ref = oracle.OracleEngine(L, shape, emb, lay, sc, max_seqs=n_seqs, max_seq_len=max_seq_len,
                              kv_tokens=n_seqs * max_seq_len, page_shift=page_shift, attn_scale=0.125, freq=freq)
    rng = np.random.default_rng(seed + 1)
    slots = []
    for s in range(n_seqs):
        a, b = eng.new_seq(), ref.new_seq()
        assert a == b
        slots.append(a)
    ctxs = [ctx] * n_seqs if np.isscalar(ctx) else list(ctx)
    if shuffle:  # pages taken a page at a time by randomly ordered sequences: shuffled tables
        left = dict(zip(slots, ctxs))
        while left:
            s = int(rng.choice(list(left)))
            n = min(1 << page_shift, left[s])
            eng.bench_fill(s, n)
            ref.bench_fill(s, n)
            left[s] -= n
            if left[s] == 0:
                del left[s]
    else:
        for s, c in zip(slots, ctxs):
            eng.bench_fill(s, c)
            ref.bench_fill(s, c)
    for s in slots:
        assert eng.seq_pages(s) == ref.pool.pages(s), "page tables differ"
    # cached K/V bf16 at every reserved page (same values on both sides): N(0, 1), or for large
    # caches random bf16 of magnitude [2^-7, 2) with random sign, drawn as bits
    kd, vd = eng.kv_cache()
    if fast_kv:
        size = (2,) + tuple(kd.shape)
        bits = (rng.integers(0x3C00, 0x4000, size, dtype=np.uint16) |
                (rng.integers(0, 2, size, dtype=np.uint16) << np.uint16(15)))
    else:
        kv_host = rng.normal(0, 1, (2,) + tuple(kd.shape)).astype(np.float32)
        bits = np.asarray(kv_host.view(np.uint32) + 0x7FFF + ((kv_host.view(np.uint32) >> 16) & 1), np.uint32) >> 16
        bits = bits.astype(np.uint16)
    ref.k[...] = bits[0]
    ref.v[...] = bits[1]
    kd.copy_(torch.from_numpy(bits[0].view(np.int16)).cuda().view(torch.bfloat16))
    vd.copy_(torch.from_numpy(bits[1].view(np.int16)).cuda().view(torch.bfloat16))
    torch.cuda.synchronize()
    return model, gm, eng, ref, slots, rng


def compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots, runs=None):
    """The step bar. Integer state is checked per run: a run whose head rows' ids all equal the
    oracle's has the oracle's emitted count and length (a run whose ids differ, only where the
    oracle's margin is within the logits tolerance, leaves that slot unchecked from then on);
    page tables (one shared pool) when every id of the step matched."""
    close(res.logits, logits_r, LOGIT_ATOL, LOGIT_RTOL, "logits")
    fin = np.isfinite(logits_r)  # the -inf columns past vocab_real were compared by close()
    err = np.abs(res.logits.astype(np.float64)[fin] - logits_r[fin])
    print(f"  logits max-abs err {err.max():.3e}", flush=True)
    greedy_ids_match(res.ids, ids_r, logits_r)
    diverged = eng.__dict__.setdefault("_diverged", set())
    if runs is not None:
        row = 0
        for ri, r in enumerate(runs):
            nh = len(r[1]) if r[2] else (r[3] if len(r) > 3 else 1)
            if r[0] not in diverged and np.array_equal(res.ids[row:row + nh], ids_r[row:row + nh]):
                assert res.emitted[ri] == em_r[ri], f"run {ri}: emitted {res.emitted[ri]} != {em_r[ri]}"
                assert eng.seq_len(r[0]) == ref.seq_len[r[0]], f"run {ri}: length differs"
            else:
                diverged.add(r[0])
            row += nh
    if np.array_equal(res.ids, ids_r) and not diverged:
        assert np.array_equal(res.emitted, em_r), f"emitted {res.emitted} != {em_r}"
        for s in slots:
            assert eng.seq_len(s) == ref.seq_len[s]
            assert eng.seq_pages(s) == ref.pool.pages(s)


def test_config0_step(gpu):
    """one layer + head, 512 cached tokens, k = 4 uniform drafts, greedy, seed 0."""
    banner("config0 step")
    shape = ModelShape(n_layers=1)
    model, gm, eng, ref, slots, rng = build_pair(shape, ctx=512, seed=0)
    s = slots[0]
    tok0 = int(rng.integers(0, shape.vocab))
    eng.set_feed(s, 512, tok0)
    ref.set_feed(s, 512, tok0)
    drafts = [int(x) for x in rng.integers(0, shape.vocab, 4)]
    run = (s, [L.FEED_ROW] + drafts, True)
    res = eng.step([run], logits=True)
    ids_r, logits_r, em_r, extra_r = ref.step([run])
    compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots, runs=[run])
    # this seed's step has no near-tie row: every id, the accept/rollback state and the pages agree
    assert np.array_equal(res.ids, ids_r), f"ids {res.ids} != {ids_r}"
    assert np.array_equal(res.emitted, em_r) and eng.seq_len(s) == ref.seq_len[s]
    assert eng.seq_pages(s) == ref.pool.pages(s)


@pytest.mark.parametrize("scalars", [LayerScalars(), LayerScalars(0.8, 1.2, 0.9, 1.1, 0.95, 0.7, 1),
                                     LayerScalars(1.1, 0.9, 1.0, 0.5, 1.0, 1.3, 0)])
def test_two_layer_steps_with_replayed_drafts(gpu, scalars):
    """Two layers, two sequences, three steps: drafts copied from the oracle's own greedy
    continuation (some right, some wrong), so acceptance, emitted counts, lengths and the
    next step's inputs are exercised; KV of rejected rows is overwritten later."""
    banner(f"two-layer steps {scalars}")
    shape = ModelShape(n_layers=2, vocab=4096, vocab_real=4000)
    model, gm, eng, ref, slots, rng = build_pair(shape, ctx=[300, 77], n_seqs=2, seed=3, scalars=scalars,
                                                 )
    for s in slots:
        t = int(rng.integers(0, shape.vocab_real))
        eng.set_feed(s, ref.seq_len[s], t)
        ref.set_feed(s, ref.seq_len[s], t)
    for step in range(3):
        runs = []
        for s in slots:
            k = int(rng.integers(1, 6))
            drafts = [int(x) for x in rng.integers(0, shape.vocab_real, k)]
            runs.append((s, [L.FEED_ROW] + drafts, True))
        ids_r, logits_r, em_r, extra_r = ref.step(runs)
        res = eng.step(runs, logits=True)
        compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots, runs=runs)
        assert np.array_equal(res.ids, ids_r), "greedy ids diverged (margins within tolerance)"


def test_multi_stream_steps(gpu):
    """Eight sequences (contexts 64-1100) over two layers, three steps of 1-5 drafts each: 17+
    verify rows (the GEMM path for every matmul) and, with 128-key splits, more attention
    workgroups than CUs (the streaming variant, each run's last cached split taking its new
    keys), against the oracle engine."""
    banner("multi-stream steps")
    shape = ModelShape(n_layers=2, vocab=4096, vocab_real=4000)
    ctxs = [300, 1100, 517, 64, 800, 999, 128, 640]
    model, gm, eng, ref, slots, rng = build_pair(shape, ctx=ctxs, n_seqs=8, seed=7, max_seq_len=1200,
                                                 split_keys=128, max_head_rows=64)
    for s in slots:
        t = int(rng.integers(0, shape.vocab_real))
        eng.set_feed(s, ref.seq_len[s], t)
        ref.set_feed(s, ref.seq_len[s], t)
    for step in range(3):
        runs = []
        for s in slots:
            k = int(rng.integers(1, 6))
            runs.append((s, [L.FEED_ROW] + [int(x) for x in rng.integers(0, shape.vocab_real, k)], True))
        ids_r, logits_r, em_r, extra_r = ref.step(runs)
        res = eng.step(runs, logits=True)
        assert sum(len(r[1]) for r in runs) > 16, "the step must take the GEMM path"
        compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots, runs=runs)
        assert np.array_equal(res.ids, ids_r), "greedy ids diverged (margins within tolerance)"


def test_tree_step_compacts(gpu):
    """A 16-node draft tree whose accepted path is not a prefix: kv_compact must move the
    path's K/V to consecutive positions (compared bit for bit on the V cache)."""
    banner("tree step")
    shape = ModelShape(n_layers=1, vocab=2048, vocab_real=2048)
    model, gm, eng, ref, slots, rng = build_pair(shape, ctx=200, seed=5)
    s = slots[0]
    tok0 = 17
    eng.set_feed(s, 200, tok0)
    ref.set_feed(s, 200, tok0)
    # First find the greedy continuation with a plain step, to build a tree that accepts.
    probe = ref.step([(s, [L.FEED_ROW], False)])
    ref.seq_len[s] -= 1  # undo (a probe): the oracle engine advanced a non-verify run
    ref.lens[s] = 200
    ref.feed[s * 16] = tok0
    ref.gen[s].remaining = 0xFFFFFFFF
    nxt = int(probe[0][0])
    # tree: root(0); children 1,2,3,4 of root (4 has the right token); 5,6 under 4; ...
    parent = [None, 0, 0, 0, 0, 4, 4, 1, 2, 3, 5, 6, 7, 8, 9, 10]
    toks = [L.FEED_ROW] + [int(x) for x in rng.integers(0, 2048, 15)]
    toks[4] = nxt
    depth = [0] * 16
    sees = [1] * 16
    for i in range(1, 16):
        depth[i] = depth[parent[i]] + 1
        sees[i] = sees[parent[i]] | (1 << i)
    tree = np.array([depth[i] | ((0xFF if parent[i] is None else parent[i]) << 8) | (sees[i] << 16)
                     for i in range(16)], np.uint32)
    # write the tree and the drafts as GPU-fed rows
    feed = np.array([tok0] + toks[1:], np.uint32)
    eng.view("d_tree", (16,)).copy_(torch.from_numpy(tree.view(np.int32)).cuda())
    eng.view("d_feed", (16,)).copy_(torch.from_numpy(feed.view(np.int32)).cuda())
    ref.tree[:16] = tree
    ref.feed[:16] = feed
    run = (s, [L.FEED_ROW + i for i in range(16)], True)
    res = eng.step([run], logits=True)
    ids_r, logits_r, em_r, extra_r = ref.step([run])
    compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots, runs=[run])
    assert np.array_equal(res.ids, ids_r)
    assert em_r[0] >= 2, "the tree was built to accept its child 4"
    torch.cuda.synchronize()
    kd, vd = eng.kv_cache()
    # V rows come from each side's own matmul: equal up to one bf16 rounding step.
    got = oracle.bf16_to_f32(vd.view(torch.int16).cpu().numpy().view(np.uint16))
    want = oracle.bf16_to_f32(ref.v)
    # (plus an absolute term for values near zero, whose fp32 projections differ in the last bits)
    bad = np.argwhere(np.abs(got - want) > 2 ** -7 * np.abs(want) + 1e-4)
    pages = eng.seq_pages(s)
    pos = [(pages.index(int(b[1])) * 16 + int(b[3]) if int(b[1]) in pages else -1, int(b[2])) for b in bad[:12]]
    assert bad.size == 0, (f"V cache (after kv_compact) differs at {len(bad)} elements; (position, kv head) "
                           f"{sorted(set(pos))}; path {extra_r['path'][0][:em_r[0]]}")


def test_sample_logits_seam(gpu):
    """hooks.rs:41-55 sample_logits through the engine: T > 0 draws bit-exact with the oracle."""
    banner("sample_logits")
    shape = ModelShape(n_layers=1, vocab=32000)
    eng = Engine(shape, max_seqs=1, max_step_tokens=16, max_seq_len=64, kv_tokens=64)
    rng = np.random.default_rng(9)
    logits = rng.normal(15, 0.7, (8, shape.vocab)).astype(np.float32)
    temps = np.array([0.7, 0.7, 0.7, 0.7, 0.0, 1.0, 0.3, 2.0], np.float32)
    tops = np.array([1.0, 0.9, 0.5, 0.99, 1.0, 0.8, 1.0, 0.95], np.float32)
    seeds = np.arange(8, dtype=np.uint64) * 0x1_0000_0001 + 5
    pos = np.arange(8, dtype=np.uint32) * 1000 + 3
    got = eng.sample_logits(logits, temps, tops, seeds, pos)
    rows = [L.SampleRow(int(seeds[i]) & 0xFFFFFFFF, int(seeds[i]) >> 32, int(pos[i]), float(temps[i]),
                        float(tops[i]), L.NO_TOK) for i in range(8)]
    want = oracle.sample(L, logits, rows)
    assert np.array_equal(got, want)


# ------------------------------------------------------------------ sampled steps (T > 0)
def sample_rows_of(ref, extra) -> list:
    """Each head row's sampler row with its position explicit (engine.rs:134-137 row_of: a step
    row samples at meta[row].y + 1 with its sequence's seed), for the oracle sampler."""
    rows = []
    for t in extra["head_rows"]:
        slot, pos = (int(v) for v in extra["meta"][t])
        sr = ref.sampling[slot]
        rows.append(L.SampleRow(sr.seed_lo, sr.seed_hi, pos + 1, sr.temperature, sr.top_p, L.NO_TOK))
    return rows


def compacted(draws, head0s, paths, path_lens) -> np.ndarray:
    """accept (kernels.metal:1630-1636) moves each verify run's accepted path to the front of
    its head rows: out[head0 + j] = draw at row path[j]."""
    out = draws.copy()
    if paths is None:
        return out
    for h0, path, n in zip(head0s, paths, path_lens):
        for j in range(int(n)):
            out[h0 + j] = draws[h0 + int(path[j])]
    return out


def check_sampled(got_ids, got_logits, want_ids, want_logits, rows, what, head0s=(), got_path=None,
                  got_path_len=(), want_path=None, want_path_len=()) -> np.ndarray:
    """Sampled ids against the oracle. The GPU's draws must equal the oracle sampler's on the
    GPU's own logits, and the oracle step's draws the oracle sampler's on its logits (both bit
    for bit, after accept's compaction of each side's own accepted path); the logits agree
    within the tolerance. Rows where the two sides' draws still differ are draws that the
    logits' rounding difference moved across an edge of the ordered CDF; they are returned
    (the caller bounds and reports them)."""
    close(got_logits, want_logits, LOGIT_ATOL, LOGIT_RTOL, f"{what} logits")
    got_raw = oracle.sample(L, got_logits, rows)
    want_raw = oracle.sample(L, want_logits, rows)
    assert np.array_equal(compacted(got_raw, head0s, got_path, got_path_len), got_ids), \
        f"{what}: GPU draws != sampler on GPU logits"
    assert np.array_equal(compacted(want_raw, head0s, want_path, want_path_len), want_ids), \
        f"{what}: oracle step draws != sampler"
    return np.flatnonzero(got_raw != want_raw)


def read_head(eng, n_head):
    torch.cuda.synchronize()
    ids = eng.view("d_out_ids", (n_head,)).cpu().numpy().view(np.uint32).copy()
    logits = eng.view("d_logits", (n_head, eng.shape.vocab), torch.float32).cpu().numpy().copy()
    return ids, logits


def dev_u32(eng, name, shape) -> np.ndarray:
    torch.cuda.synchronize()
    return eng.view(name, shape).cpu().numpy().view(np.uint32).copy()


def put_u32(eng, name, arr) -> None:
    eng.view(name, arr.shape).copy_(torch.from_numpy(np.ascontiguousarray(arr, np.uint32).view(np.int32)).cuda())
    torch.cuda.synchronize()


def reserve_like_plan(ref, runs, extra_keys) -> None:
    """The oracle's pool takes the pages sv_plan reserves for replays of a plan (each run's rows
    plus extra_keys positions, in run order), so both page tables stay equal."""
    for r in runs:
        s = r[0]
        assert ref.pool.reserve(s, min(ref.seq_len[s] + len(r[1]) + extra_keys, ref.max_seq_len))


def resync(eng, ref, slots) -> None:
    """After a draw that crossed a CDF edge the two sides' sequences differ: continue from the
    GPU's state (lengths, feed, tree, generation state and KV cache)."""
    S = ref.max_seqs
    ref.lens[:] = dev_u32(eng, "d_lens", (S,))
    ref.feed[:] = dev_u32(eng, "d_feed", (S * 16,))
    ref.tree[:] = dev_u32(eng, "d_tree", (S * 16,))
    g = dev_u32(eng, "d_gen", (S, C.sizeof(L.GenState) // 4))
    C.memmove(ref.gen, g.ctypes.data, g.nbytes)
    kd, vd = eng.kv_cache()
    ref.k[...] = kd.view(torch.int16).cpu().numpy().view(np.uint16)
    ref.v[...] = vd.view(torch.int16).cpu().numpy().view(np.uint16)
    for s in slots:
        ref.seq_len[s] = int(ref.lens[s])


@pytest.mark.parametrize("top_p", [1.0, 0.9])
def test_sampled_graph_replay_multi_stream(gpu, top_p):
    """configs[2]'s path at reduced size: 8 streams (contexts 64-1100, shuffled page tables), T in
    {0.5, 0.7, 1.0, 1.3}, captured once as a HIP graph and replayed, as bench.py times it.
    First a plain sampled decode records each stream's continuation (14 replays of one row per
    stream); then verify steps of k = 4 drafts from the replay drafter over that continuation
    (35% wrong), 4 replays. After every replay the GPU's draws, emitted counts, lengths, feed,
    drafts and page tables equal the oracle engine's (bit-exact; a draw moved across a CDF edge
    by the logits' rounding is counted, and both sides continue from the GPU's state), and every
    verify step emits the recorded continuation (the lossless property)."""
    banner(f"sampled graph replay, 8 streams, top_p={top_p}")
    shape = ModelShape(n_layers=2, vocab=4096, vocab_real=4000)
    ctxs = [300, 1100, 517, 64, 800, 999, 128, 640]
    S, k, trace_n, steps, rate, max_len = 8, 4, 24, 4, 0.35, 1300
    model, gm, eng, ref, slots, rng = build_pair(shape, ctx=ctxs, n_seqs=S, seed=11, max_seq_len=max_len,
                                                 shuffle=True, max_head_rows=64)
    temps = [0.7, 0.7, 1.0, 0.7, 0.5, 0.7, 1.3, 0.7]
    for i, s in enumerate(slots):
        eng.set_sampling(s, temps[i], top_p, 1000 + 7 * i)
        ref.set_sampling(s, temps[i], top_p, 1000 + 7 * i)
    first = [int(x) for x in rng.integers(0, shape.vocab_real, S)]
    for s, c, t in zip(slots, ctxs, first):
        eng.set_feed(s, c, t)
        ref.set_feed(s, c, t)
    edges, draws = 0, 0
    diverged = set()

    def one(runs, what, after=None):
        nonlocal edges, draws
        eng.graph_replay(1)
        eng.sync()
        ids_r, logits_r, em_r, extra = ref.step(runs)
        if after:
            after()
        got_ids, got_logits = read_head(eng, len(ids_r))
        # linear chains: accept's compaction leaves the head rows in place
        e = check_sampled(got_ids, got_logits, ids_r, logits_r, sample_rows_of(ref, extra), what)
        draws += len(ids_r)
        if e.size:
            edges += e.size
            diverged.update(int(extra["meta"][extra["head_rows"][i]][0]) for i in e)
            resync(eng, ref, slots)
            return
        assert np.array_equal(dev_u32(eng, "d_emitted", (S,))[: len(runs)], em_r), f"{what}: emitted"
        assert np.array_equal(dev_u32(eng, "d_lens", (S,)), ref.lens), f"{what}: lengths"
        assert np.array_equal(dev_u32(eng, "d_feed", (S * 16,)), ref.feed), f"{what}: feed / drafts"
        for s in slots:
            assert eng.seq_pages(s) == ref.pool.pages(s), f"{what}: page table of {s}"

    # 1. the plain sampled decode that records each stream's continuation
    runs1 = [(s, [L.FEED_ROW], False, 1) for s in slots]
    eng.plan(runs1, extra_keys=trace_n + 8)
    reserve_like_plan(ref, runs1, trace_n + 8)
    eng.graph_capture(0)
    traces = [[t] for t in first]
    for i in range(trace_n):
        one(runs1, f"decode {i}")
        col = dev_u32(eng, "d_feed", (S, 16))[:, 0]
        for j, s in enumerate(slots):
            traces[j].append(int(col[s]))
    # 2. verify steps drafting that continuation
    tr = np.zeros((S, max_len), np.uint32)
    tl = np.zeros(S, np.uint32)
    for j, (s, c) in enumerate(zip(slots, ctxs)):
        tr[s, c:c + len(traces[j])] = traces[j]
        tl[s] = c + len(traces[j])
    put_u32(eng, "d_trace", tr)
    put_u32(eng, "d_trace_len", tl)
    for s, c, t in zip(slots, ctxs, first):
        eng.set_feed(s, c, t)
        ref.set_feed(s, c, t)
    ra = L.ReplayArgs(max_len, 77, rate, shape.vocab_real)
    eng.set_replay(77, rate)
    run_in = [L.RunIn(s, 0, k + 1, 0, k + 1, 1) for s in slots]
    oracle.replay_draft(L, run_in, ref.lens, ref.feed, tr, tl, ra, ref.tree)
    put_u32(eng, "d_feed", ref.feed)
    put_u32(eng, "d_tree", ref.tree)
    runs2 = [(s, [L.FEED_ROW + i for i in range(k + 1)], True) for s in slots]
    eng.plan(runs2, extra_keys=(k + 1) * steps + 8)
    reserve_like_plan(ref, runs2, (k + 1) * steps + 8)
    eng.graph_capture(L.STEP_REPLAY)
    accepted = 0
    for i in range(steps):
        before = ref.lens.copy()
        one(runs2, f"verify {i}", lambda: oracle.replay_draft(L, run_in, ref.lens, ref.feed, tr, tl, ra, ref.tree))
        lens = dev_u32(eng, "d_lens", (S,))
        feed = dev_u32(eng, "d_feed", (S, 16))
        accepted += int((lens - before)[slots].sum()) - S
        for j, (s, c) in enumerate(zip(slots, ctxs)):
            if s not in diverged:
                assert feed[s, 0] == traces[j][lens[s] - c], f"verify {i}: stream {s} left its continuation"
    print(f"  {draws} draws, {edges} moved across a CDF edge by rounding; {accepted} drafts accepted", flush=True)
    assert edges <= 2, f"{edges} of {draws} draws differ"
    assert accepted > 0, "no draft was accepted"
    # The plan reserved pages for (4 + 1) x 4 + 8 positions past the first step: 6 steps in
    # all. A replay past them is refused before it runs (it would write unreserved pages).
    eng.graph_replay(2)
    with pytest.raises(L.SvError, match="pages cover 6 steps"):
        eng.graph_replay(1)
    eng.close()


TREE16 = [None, 0, 0, 0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 5, 6, 7]  # configs[4]'s tree (16 nodes)


def tree_nodes(parents) -> np.ndarray:
    depth, sees = [0] * len(parents), [1] * len(parents)
    for i in range(1, len(parents)):
        depth[i] = depth[parents[i]] + 1
        sees[i] = sees[parents[i]] | (1 << i)
    return np.array([depth[i] | ((0xFF if parents[i] is None else parents[i]) << 8) | (sees[i] << 16)
                     for i in range(len(parents))], np.uint32)


def test_sampled_tree_step_accepts_planted_path(gpu):
    """Four streams verify configs[4]'s 16-node tree at T = 0.7 (top-p 1 and 0.9) through
    sv_step. The drafts along root -> 2 -> 7 -> 15 are set, level by level, to what the oracle
    samples at their parents, so multi-candidate sample-and-match accepts a path that is not a
    prefix of the rows and kv_compact moves it. Draws, emitted counts, paths, lengths and page
    tables are bit-exact; the V cache after compaction matches within one bf16 step."""
    banner("sampled tree step with a planted path")
    shape = ModelShape(n_layers=2, vocab=2048, vocab_real=2048)
    ctxs = [200, 333, 90, 512]
    S = 4
    model, gm, eng, ref, slots, rng = build_pair(shape, ctx=ctxs, n_seqs=S, seed=13, max_seq_len=600,
                                                 shuffle=True, max_head_rows=64)
    for i, s in enumerate(slots):
        eng.set_sampling(s, 0.7, (1.0, 0.9)[i % 2], 31 + i)
        ref.set_sampling(s, 0.7, (1.0, 0.9)[i % 2], 31 + i)
    nodes = tree_nodes(TREE16)
    for s, c in zip(slots, ctxs):
        t0 = int(rng.integers(0, shape.vocab_real))
        eng.set_feed(s, c, t0)
        ref.set_feed(s, c, t0)
        ref.feed[s * 16 + 1:s * 16 + 16] = rng.integers(0, shape.vocab_real, 15)
        ref.tree[s * 16:s * 16 + 16] = nodes
    runs = [(s, [L.FEED_ROW + i for i in range(16)], True) for s in slots]
    for parent, child in ((0, 2), (2, 7), (7, 15)):  # probe on the oracle, then roll it back
        saved = (ref.lens.copy(), ref.feed.copy(), ref.tree.copy(), list(ref.seq_len), bytes(ref.gen))
        ids = ref.step(runs)[0]
        ref.lens[:], ref.feed[:], ref.tree[:] = saved[0], saved[1], saved[2]
        ref.seq_len[:] = saved[3]
        C.memmove(ref.gen, saved[4], len(saved[4]))
        for j, s in enumerate(slots):
            ref.feed[s * 16 + child] = ids[16 * j + parent]
    put_u32(eng, "d_feed", ref.feed)
    put_u32(eng, "d_tree", ref.tree)
    res = eng.step(runs, logits=True)
    ids_r, logits_r, em_r, extra = ref.step(runs)
    gp, gl = dev_u32(eng, "d_path", (S, 16))[: len(runs)], dev_u32(eng, "d_path_len", (S,))[: len(runs)]
    e = check_sampled(res.ids, res.logits, ids_r, logits_r, sample_rows_of(ref, extra), "tree step",
                      [16 * j for j in range(len(runs))], gp, gl, extra["path"], extra["path_len"])
    print(f"  {len(ids_r)} draws, {e.size} across a CDF edge; emitted {list(em_r)}", flush=True)
    assert e.size == 0, f"draws {e} moved across a CDF edge (rerun with another seed)"
    assert (em_r >= 4).all(), "the planted path root -> 2 -> 7 -> 15 is accepted"
    assert np.array_equal(res.emitted, em_r)
    assert np.array_equal(dev_u32(eng, "d_path", (S, 16))[: len(runs)], extra["path"])
    assert np.array_equal(dev_u32(eng, "d_lens", (S,)), ref.lens)
    for s in slots:
        assert eng.seq_len(s) == ref.seq_len[s] and eng.seq_pages(s) == ref.pool.pages(s)
    kd, vd = eng.kv_cache()
    got = oracle.bf16_to_f32(vd.view(torch.int16).cpu().numpy().view(np.uint16))
    want = oracle.bf16_to_f32(ref.v)
    assert (np.abs(got - want) <= 2 ** -7 * np.abs(want) + 1e-4).all(), "V cache after kv_compact"
    eng.close()


def test_trees_32_streams_full_layer(gpu):
    """configs[4]'s step shape at one layer: 32 streams x the 16-node tree (512 verify rows: the
    GEMM launch shapes and attention grid configs[4] uses), 4096 cached tokens each on shuffled
    pages, random node ids, T = 0.7 sample-and-match, compaction where a path is accepted.
    Draws (CDF-edge rows counted), emitted counts, paths, lengths and page tables against the
    oracle; logits within 2e-2 / 1e-2."""
    banner("32 streams x 16-node trees, one full layer")
    shape = ModelShape(n_layers=1, vocab=4096, vocab_real=4096)
    S, ctx = 32, 4096
    model, gm, eng, ref, slots, rng = build_pair(shape, ctx=[ctx] * S, n_seqs=S, seed=17, max_seq_len=ctx + 64,
                                                 shuffle=True, max_head_rows=16 * S, fast_kv=True)
    nodes = tree_nodes(TREE16)
    for i, s in enumerate(slots):
        eng.set_sampling(s, 0.7, 1.0, 500 + i)
        ref.set_sampling(s, 0.7, 1.0, 500 + i)
        t0 = int(rng.integers(0, shape.vocab_real))
        eng.set_feed(s, ctx, t0)
        ref.set_feed(s, ctx, t0)
        ref.feed[s * 16 + 1:s * 16 + 16] = rng.integers(0, shape.vocab_real, 15)
        ref.tree[s * 16:s * 16 + 16] = nodes
    put_u32(eng, "d_feed", ref.feed)
    put_u32(eng, "d_tree", ref.tree)
    runs = [(s, [L.FEED_ROW + i for i in range(16)], True) for s in slots]
    res = eng.step(runs, logits=True)
    assert res.info.n_tokens == 512
    ids_r, logits_r, em_r, extra = ref.step(runs)
    gp, gl = dev_u32(eng, "d_path", (S, 16)), dev_u32(eng, "d_path_len", (S,))
    e = check_sampled(res.ids, res.logits, ids_r, logits_r, sample_rows_of(ref, extra), "trees32",
                      [16 * j for j in range(S)], gp, gl, extra["path"], extra["path_len"])
    print(f"  {len(ids_r)} draws, {e.size} across a CDF edge; emitted {int(em_r.sum())}", flush=True)
    assert e.size <= 1
    ok = np.ones(S, bool)
    ok[[int(extra["meta"][extra["head_rows"][i]][0]) for i in e]] = False
    assert np.array_equal(res.emitted[ok], em_r[ok])
    assert np.array_equal(dev_u32(eng, "d_path", (S, 16))[ok], extra["path"][ok])
    for j, s in enumerate(slots):
        if ok[j]:
            assert eng.seq_len(s) == ref.seq_len[s] and eng.seq_pages(s) == ref.pool.pages(s)
    eng.close()


def test_ddtree_feeds_verify_step(gpu):
    """The draft builder feeding the verify step: drafter logits (random, over a 2048-id draft
    vocabulary mapped into the target's) go through draft_top and draft_tree straight into the
    engine's feed and tree; three streams then verify their trees (8, 5 and 16 rows: best-first
    DDTrees of up to four candidates per row) in one greedy step. Trees, logits, ids, emitted
    counts, lengths and page tables against the oracle engine given the oracle's trees."""
    banner("DDTree -> verify step")
    from violetto import kernels as K

    shape = ModelShape(n_layers=2, vocab=4096, vocab_real=4096)
    model, gm, eng, ref, slots, rng = build_pair(shape, ctx=[300, 77, 650], n_seqs=3, seed=23, max_seq_len=1024,
                                                 shuffle=True, max_head_rows=48)
    for s in slots:
        t = int(rng.integers(0, shape.vocab_real))
        eng.set_feed(s, ref.seq_len[s], t)
        ref.set_feed(s, ref.seq_len[s], t)
    block_rows = [8, 5, 16]
    blocks, tin = [], []
    for s, rows in zip(slots, block_rows):
        blocks.append((len(tin), rows))
        tin += [(s, i) for i in range(rows)]
    blocks, tin = np.array(blocks, np.uint32), np.array(tin, np.uint32)
    nv = 2048
    logits = rng.normal(0, 2, (len(tin), nv)).astype(np.float32)
    vocab = np.sort(rng.choice(shape.vocab_real, nv, replace=False)).astype(np.uint32)
    cand_r, q_r = oracle.draft_top(logits, vocab, tin, 1.0, 4)
    oracle.draft_tree(blocks, tin, cand_r, q_r, ref.feed, ref.tree, 4)
    cand = torch.zeros(len(tin) * 4, dtype=torch.int32, device="cuda")
    q = torch.zeros(len(tin) * 4, dtype=torch.float32, device="cuda")
    d_tin = torch.from_numpy(tin.view(np.int32)).cuda()
    d_logits, d_vocab = torch.from_numpy(logits).cuda(), torch.from_numpy(vocab.view(np.int32)).cuda()
    d_blocks = torch.from_numpy(blocks.view(np.int32)).cuda()
    torch.cuda.synchronize()  # torch's copies land before the engine's stream reads them
    K.draft_top(d_logits, d_vocab, d_tin, cand, q, len(tin), nv, 1.0, 4, stream=eng.stream)
    K.draft_tree(d_blocks, len(blocks), d_tin, cand, q,
                 eng.view("d_feed", (3 * 16,)), eng.view("d_tree", (3 * 16,)), 4, stream=eng.stream)
    eng.sync()
    assert np.array_equal(dev_u32(eng, "d_feed", (3 * 16,)), ref.feed), "trees' tokens"
    assert np.array_equal(dev_u32(eng, "d_tree", (3 * 16,)), ref.tree), "trees' nodes"
    assert any((ref.tree[s * 16 + i] >> 8) & 0xFF not in (0xFF, i - 1) for s in slots for i in range(1, 16)), \
        "some tree branches (a node whose parent is not the row before)"
    runs = [(s, [L.FEED_ROW + i for i in range(rows)], True) for s, rows in zip(slots, block_rows)]
    res = eng.step(runs, logits=True)
    ids_r, logits_r, em_r, extra_r = ref.step(runs)
    compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots, runs=runs)
    eng.close()


@pytest.mark.parametrize("group", [64, None])
def test_step_from_weight_file(gpu, tmp_path, group):
    """A model served from the reference's weight-file layout (engine/src/weights.rs): a
    two-layer model written as `embed`, `Lnn.{qkv,o,gate_up,down}` (int8 with `.scale`: groups
    of 64 k, the reference's default, or one per row) and `Lnn.scalars`, uploaded and resolved by
    sv_weights_*, verifies three streams' drafts in one step against the oracle engine."""
    banner(f"step from a weight file, group={group}")
    from violetto.weights import VltModel, WeightFile, write_vlt

    shape = ModelShape(n_layers=2, vocab=4096, vocab_real=4000)
    scal = [LayerScalars(0.9, 1.1, 1.0, 0.8, 1.0, 1.2, 1), LayerScalars(1.0, 0.95, 1.1, 1.0, 0.9, 1.0, 1)]
    model = SyntheticModel.generate(shape, seed=29, device="cpu", scalars=scal, group=group)
    tensors = {"embed": model.embed}
    for i, (lay, s) in enumerate(zip(model.layers, model.scalars)):
        for name, (w, sc) in lay.items():
            tensors[f"L{i:02d}.{name}"] = w
            tensors[f"L{i:02d}.{name}.scale"] = sc
        tensors[f"L{i:02d}.scalars"] = torch.tensor([s.qkv_scale, s.o_scale, s.resid_attn, s.post_attn, s.resid_mlp,
                                                     s.post_mlp, 0.0, 0.0])
    path = tmp_path / "model.vlt"
    write_vlt(path, tensors)
    wf = WeightFile(path)
    wf.upload()
    vm = VltModel(wf, shape)
    freq = rope_freq(500000.0, shape.head_dim)
    eng = Engine(shape, max_seqs=3, max_step_tokens=48, max_seq_len=1024, max_head_rows=48, kv_tokens=3 * 1024,
                 attn_scale=0.125, freq=freq)
    eng.set_model(vm)
    emb, lay, sc = oracle.host_weights(model)
    ref = oracle.OracleEngine(L, shape, emb, lay, sc, max_seqs=3, max_seq_len=1024, kv_tokens=3 * 1024, attn_scale=0.125,
                              freq=freq)
    rng = np.random.default_rng(31)
    slots = []
    for c in (200, 513, 64):
        s = eng.new_seq()
        assert s == ref.new_seq()
        eng.bench_fill(s, c)
        ref.bench_fill(s, c)
        slots.append(s)
    kd, vd = eng.kv_cache()
    bits = rng.integers(0x3C00, 0x4000, (2,) + tuple(kd.shape), dtype=np.uint16) | \
        (rng.integers(0, 2, (2,) + tuple(kd.shape), dtype=np.uint16) << np.uint16(15))
    ref.k[...], ref.v[...] = bits[0], bits[1]
    kd.copy_(torch.from_numpy(bits[0].view(np.int16)).cuda().view(torch.bfloat16))
    vd.copy_(torch.from_numpy(bits[1].view(np.int16)).cuda().view(torch.bfloat16))
    for s in slots:
        t = int(rng.integers(0, shape.vocab_real))
        eng.set_feed(s, ref.seq_len[s], t)
        ref.set_feed(s, ref.seq_len[s], t)
    runs = [(s, [L.FEED_ROW] + [int(x) for x in rng.integers(0, shape.vocab_real, k)], True)
            for s, k in zip(slots, (4, 2, 4))]
    res = eng.step(runs, logits=True)
    ids_r, logits_r, em_r, extra_r = ref.step(runs)
    compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots, runs=runs)
    eng.close()
    wf.close()


def test_prompt_chunks_then_verify(gpu):
    """The chunk path (encode.rs:300-355): three streams on shuffled pages with 100, 37 and 500
    cached tokens each take a prompt chunk of 40, 100 and 23 tokens in one step (attention in
    runs of 16 rows after every new K/V row is written), then a verify step of drafts. Last-row
    logits and greedy ids, lengths, page tables and both caches (within one bf16 step) against
    the oracle engine."""
    banner("prompt chunks, then verify")
    shape = ModelShape(n_layers=2, vocab=4096, vocab_real=4000)
    model, gm, eng, ref, slots, rng = build_pair(shape, ctx=[100, 37, 500], n_seqs=3, seed=41, max_seq_len=1024,
                                                 shuffle=True, max_head_rows=48)
    eng.close()
    freq = rope_freq(500000.0, shape.head_dim)
    eng = Engine(shape, max_seqs=3, max_step_tokens=256, max_seq_len=1024, max_head_rows=48, kv_tokens=3 * 1024,
                 attn_scale=0.125, freq=freq)
    eng.set_model(gm)
    ref2 = oracle.OracleEngine(L, shape, *oracle.host_weights(model), max_seqs=3, max_seq_len=1024,
                               kv_tokens=3 * 1024, attn_scale=0.125, freq=freq)
    for s, c in zip(slots, [100, 37, 500]):
        assert eng.new_seq() == ref2.new_seq() == s
    left = dict(zip(slots, [100, 37, 500]))
    while left:  # shuffled page tables, the same on both sides
        s = int(rng.choice(list(left)))
        k = min(16, left[s])
        eng.bench_fill(s, k)
        ref2.bench_fill(s, k)
        left[s] -= k
        if not left[s]:
            del left[s]
    kd, vd = eng.kv_cache()
    bits = rng.integers(0x3C00, 0x4000, (2,) + tuple(kd.shape), dtype=np.uint16) | \
        (rng.integers(0, 2, (2,) + tuple(kd.shape), dtype=np.uint16) << np.uint16(15))
    ref2.k[...], ref2.v[...] = bits[0], bits[1]
    kd.copy_(torch.from_numpy(bits[0].view(np.int16)).cuda().view(torch.bfloat16))
    vd.copy_(torch.from_numpy(bits[1].view(np.int16)).cuda().view(torch.bfloat16))
    torch.cuda.synchronize()
    ref = ref2
    chunks = [(s, [int(x) for x in rng.integers(0, shape.vocab_real, k)], False, 1) for s, k in zip(slots, [40, 100, 23])]
    res = eng.step(chunks, logits=True)
    ids_r, logits_r, em_r, extra_r = ref.step(chunks)
    assert res.info.n_tokens == 163 and res.info.n_head == 3
    compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots, runs=chunks)
    assert np.array_equal(res.ids, ids_r)
    for s, c in zip(slots, [140, 137, 523]):
        assert eng.seq_len(s) == ref.seq_len[s] == c
    got_k = oracle.bf16_to_f32(kd.view(torch.int16).cpu().numpy().view(np.uint16))
    got_v = oracle.bf16_to_f32(vd.view(torch.int16).cpu().numpy().view(np.uint16))
    for got, want, what in ((got_k, oracle.bf16_to_f32(ref.k), "K"), (got_v, oracle.bf16_to_f32(ref.v), "V")):
        bad = np.abs(got - want) > 2 ** -7 * np.abs(want) + 1e-4
        assert not bad.any(), f"{what} cache differs at {int(bad.sum())} elements"
    # the fed tokens, then a verify step of four drafts per stream on top of the chunks
    for s in slots:
        t = int(ids_r[slots.index(s)])
        assert int(dev_u32(eng, "d_feed", (3 * 16,))[s * 16]) == t
    runs = [(s, [L.FEED_ROW] + [int(x) for x in rng.integers(0, shape.vocab_real, 4)], True) for s in slots]
    res = eng.step(runs, logits=True)
    ids_r, logits_r, em_r, extra_r = ref.step(runs)
    compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots, runs=runs)
    eng.close()


@pytest.mark.parametrize("n_seqs", [1, 8])
def test_config3_long_context_bf16(gpu, n_seqs):
    """configs[3] end to end: unquantised bf16 weights (N(0, 0.02)) over two layers, 1 or 8
    streams each with 65536 cached tokens (random bf16 K/V), two greedy verify steps of k = 4
    linear drafts, the split-KV attention at the engine's own split choice, against the oracle
    engine: logits, greedy ids, emitted counts, lengths and page tables at the step bar."""
    banner(f"configs[3] end to end, {n_seqs} stream(s) x 65536")
    shape = ModelShape(n_layers=2)
    model, gm, eng, ref, slots, rng = build_pair(shape, ctx=65536, n_seqs=n_seqs, seed=31, int8=False,
                                                 max_seq_len=65536 + 64, fast_kv=True, max_head_rows=16 * n_seqs)
    for s in slots:
        t = int(rng.integers(0, shape.vocab_real))
        eng.set_feed(s, 65536, t)
        ref.set_feed(s, 65536, t)
    for step in range(2):
        runs = [(s, [L.FEED_ROW] + [int(x) for x in rng.integers(0, shape.vocab_real, 4)], True) for s in slots]
        ids_r, logits_r, em_r, extra_r = ref.step(runs)
        res = eng.step(runs, logits=True)
        print(f"  step {step}: split {res.info.split} keys, {res.info.max_splits} splits", flush=True)
        compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots, runs=runs)
    eng.close()
