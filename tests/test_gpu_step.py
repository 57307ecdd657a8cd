"""End-to-end verify steps on the GPU engine against the oracle engine (BASELINE.json
configs[0] and smaller variants), through the C ABI.

Bar (north star): logits within 2e-2 max-abs / 1e-2 relative; greedy ids equal wherever the
oracle's top-1 margin exceeds 2e-2; accepted counts, emitted ids, paths, lengths and page
tables bit-exact."""
from __future__ import annotations

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
               max_seq_len=1024, scalars=None, shuffle=False, step_kernel=True, split_keys=0, max_head_rows=16):
    model = SyntheticModel.generate(shape, int8=int8, seed=seed, device="cpu", scalars=scalars)
    freq = rope_freq(500000.0, shape.head_dim)
    eng = Engine(shape, max_seqs=n_seqs, max_step_tokens=16 * n_seqs, max_seq_len=max_seq_len, max_head_rows=max_head_rows,
                 kv_tokens=n_seqs * max_seq_len, page_shift=page_shift, attn_scale=0.125, freq=freq,
                 step_kernel=step_kernel, split_keys=split_keys)
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
    if shuffle:  # take pages in a shuffled order: reserve/release scratch sequences
        pass
    ctxs = [ctx] * n_seqs if np.isscalar(ctx) else list(ctx)
    for s, c in zip(slots, ctxs):
        eng.bench_fill(s, c)
        ref.bench_fill(s, c)
        assert eng.seq_pages(s) == ref.pool.pages(s), "page tables differ"
    # cached K/V ~ N(0, 1) bf16 at every reserved page (same values on both sides)
    kd, vd = eng.kv_cache()
    kv_host = rng.normal(0, 1, (2,) + tuple(kd.shape)).astype(np.float32)
    bits = oracle.np.asarray(kv_host.view(np.uint32) + 0x7FFF + ((kv_host.view(np.uint32) >> 16) & 1), np.uint32) >> 16
    bits = bits.astype(np.uint16)
    ref.k[...] = bits[0]
    ref.v[...] = bits[1]
    kd.copy_(torch.from_numpy(bits[0].view(np.int16)).cuda().view(torch.bfloat16))
    vd.copy_(torch.from_numpy(bits[1].view(np.int16)).cuda().view(torch.bfloat16))
    torch.cuda.synchronize()
    return model, gm, eng, ref, slots, rng


def compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots):
    close(res.logits, logits_r, LOGIT_ATOL, LOGIT_RTOL, "logits")
    err = np.abs(res.logits.astype(np.float64) - logits_r)
    print(f"  logits max-abs err {err[np.isfinite(err)].max():.3e}", flush=True)
    greedy_ids_match(res.ids, ids_r, logits_r)
    if np.array_equal(res.ids, ids_r):
        assert np.array_equal(res.emitted, em_r), f"emitted {res.emitted} != {em_r}"
        for s in slots:
            assert eng.seq_len(s) == ref.seq_len[s]
            assert eng.seq_pages(s) == ref.pool.pages(s)


@pytest.mark.parametrize("persistent", [True, False])
def test_config0_step(gpu, persistent):
    """one layer + head, 512 cached tokens, k = 4 uniform drafts, greedy, seed 0;
    the layers as one persistent launch and as separate launches."""
    banner(f"config0 step persistent={persistent}")
    shape = ModelShape(n_layers=1)
    model, gm, eng, ref, slots, rng = build_pair(shape, ctx=512, seed=0, step_kernel=persistent)
    s = slots[0]
    tok0 = int(rng.integers(0, shape.vocab))
    eng.set_feed(s, 512, tok0)
    ref.set_feed(s, 512, tok0)
    drafts = [int(x) for x in rng.integers(0, shape.vocab, 4)]
    run = (s, [L.FEED_ROW] + drafts, True)
    res = eng.step([run], logits=True)
    assert res.info.persistent == int(persistent)
    ids_r, logits_r, em_r, extra_r = ref.step([run])
    compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots)


@pytest.mark.parametrize("persistent", [True, False])
@pytest.mark.parametrize("scalars", [LayerScalars(), LayerScalars(0.8, 1.2, 0.9, 1.1, 0.95, 0.7, 1),
                                     LayerScalars(1.1, 0.9, 1.0, 0.5, 1.0, 1.3, 0)])
def test_two_layer_steps_with_replayed_drafts(gpu, scalars, persistent):
    """Two layers, two sequences, three steps: drafts copied from the oracle's own greedy
    continuation (some right, some wrong), so acceptance, emitted counts, lengths and the
    next step's inputs are exercised; KV of rejected rows is overwritten later."""
    banner(f"two-layer steps {scalars} persistent={persistent}")
    shape = ModelShape(n_layers=2, vocab=4096, vocab_real=4000)
    model, gm, eng, ref, slots, rng = build_pair(shape, ctx=[300, 77], n_seqs=2, seed=3, scalars=scalars,
                                                 step_kernel=persistent)
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
        assert res.info.persistent == int(persistent)
        compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots)
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
                                                 step_kernel=False, split_keys=128, max_head_rows=64)
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
        compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots)
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
    compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots)
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
