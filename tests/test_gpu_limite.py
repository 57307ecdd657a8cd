"""The Limite layer extras on the GPU against the oracle, through the C ABI: sliding-window
layers over their ring caches, value embeddings, XSA, the attention gate (sv_attn_verify with
sv_attn_extras), the MUDD mix (sv_mudd), and whole verify steps of Limite-layout models
(engine/src/model.rs:49-127, kernels.metal:738-747, 808-811, 1316-1407, kv.rs:26-32,
encode.rs:107-160), including the reference's own shape (48 layers, 1280 hidden, 10 query heads
over 2 kv heads of 128 dims, vocabulary 151680).

Bars: attention outputs within 2e-4 (abs and relative), cached K and V within one bf16 step
(value embeddings are added in fp32 here, in double in the oracle); MUDD within 1e-5; steps as
the other step tests (logits within 2e-2 / 1e-2, greedy ids equal wherever the oracle's margin
exceeds 2e-2, emitted counts, lengths, paths and pages bit-exact)."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

import oracle
from conftest import banner
from helpers import bf16_bits, close, greedy_ids_match, to_dev
from test_gpu_step import dev_u32, put_u32, tree_nodes
from violetto import _lib as L
from violetto import kernels as K
from violetto.engine import Engine
from violetto.model import REFERENCE_SHAPE, ModelShape, SyntheticModel, generate_extras, rope_freq

pytestmark = pytest.mark.gpu

LOGIT_ATOL, LOGIT_RTOL = 2e-2, 1e-2
CFG = ModelShape(hidden=2048, n_heads=32, n_kv_heads=8, head_dim=64, ffn=8192, vocab=4096, vocab_real=4096, n_layers=1)
REF1 = ModelShape(hidden=1280, n_heads=10, n_kv_heads=2, head_dim=128, ffn=3328, vocab=4096, vocab_real=4096,
                  n_layers=1)


def rand_bits(rng, shape) -> np.ndarray:
    """Random bf16 bits of magnitude [2^-7, 2) with random sign."""
    return (rng.integers(0x3C00, 0x4000, shape, dtype=np.uint16) |
            (rng.integers(0, 2, shape, dtype=np.uint16) << np.uint16(15)))


def tree_parents(rng, n):
    return [None] + [int(rng.integers(0, r)) for r in range(1, n)]


def vis_and_depth(parents):
    nodes = tree_nodes(parents)
    return (nodes >> 16).astype(np.uint32), (nodes & 0xFF).astype(np.uint32)


# ---------------------------------------------------------------------------- attention
@pytest.mark.parametrize("which,runs_T,p0s,split", [
    ("cfg", [5, 16, 3], [2500, 300, 1030], 256),
    ("ref", [5, 12, 3], [2500, 300, 1030], 512),
    ("ref", [5], [5000], 128),
    ("cfg", [1, 16], [4000, 1100], 128),
])
def test_window_attention_with_extras(gpu, which, runs_T, p0s, split):
    """A sliding-window layer (window 1024) over rings of 68 pages through a cyclic page table,
    with value embeddings, XSA and the gate on: runs past the window with the ring wrapped
    (2500, 5000), inside it (300) and across its start (1030); chains and random trees; splits
    of 128-512 keys, so the merge adds several splits per output before XSA and the gate."""
    sh = CFG if which == "cfg" else REF1
    banner(f"window attention {which} runs={runs_T} p0={p0s} split={split}")
    rng = np.random.default_rng(sum(p0s) + split)
    D, NQ, NKV, H = sh.head_dim, sh.n_heads, sh.n_kv_heads, sh.hidden
    W = (NQ + 2 * NKV) * D
    window, page = 1024, 16
    ring_pages = -(-(window + 64) // page)
    S = len(runs_T)
    max_pages = -(-(max(p0s) + 32) // page)
    table = np.array([[s * ring_pages + p % ring_pages for p in range(max_pages)] for s in range(S)], np.uint32)
    n_pages = S * ring_pages
    k = rand_bits(rng, (1, n_pages, NKV, page, D))
    v = rand_bits(rng, (1, n_pages, NKV, page, D))
    n = sum(runs_T)
    meta = np.zeros((n, 2), np.uint32)
    vis = np.zeros(n, np.uint32)
    runs = []
    t = 0
    for s, (T, p0) in enumerate(zip(runs_T, p0s)):
        if T > 5:
            vv, dd = vis_and_depth(tree_parents(rng, T))
        else:
            vv, dd = np.array([(2 << i) - 1 for i in range(T)], np.uint32), np.arange(T, dtype=np.uint32)
        meta[t:t + T, 0] = s
        meta[t:t + T, 1] = p0 + dd
        vis[t:t + T] = vv
        runs += [t, T]
        t += T
    runs = np.array(runs, np.uint32)
    qkv = rng.normal(0, 1, (n, W)).astype(np.float32)
    x = rng.normal(0, 1, (n, H)).astype(np.float32)
    inv = (1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(1) + L.RMS_EPS)).astype(np.float32)
    ex = dict(x=x, inv=inv, tokens=rng.integers(0, sh.vocab, n).astype(np.uint32),
              value_embed=rand_bits(rng, (sh.vocab, NKV * D)),
              ve_gate=(rng.normal(0, 0.3, (NKV, 12))).astype(np.float32),
              attn_gate=(rng.normal(0, 0.3, (NQ, D))).astype(np.float32),
              xsa=rng.random(NQ).astype(np.float32))
    rope_tab = oracle.rope_table(rope_freq(500000.0, 64), max(p0s) + 32)
    kv = L.KvArgs(0, 0, ring_pages * page, S, 4, n_pages, max_pages, window)
    max_splits = -(-(window + 31) // split) + 1
    args = L.AttnArgs(split, max_splits, D ** -0.5 * 1.4426950408889634, 1, 0, 0, 0, 0, 0)
    k_ref, v_ref = k.copy(), v.copy()
    ref = oracle.attn_verify(L, sh, qkv, meta.reshape(-1).copy(), k_ref, v_ref, table, rope_tab, kv, args, runs, vis,
                             extras=ex)
    kd, vd = to_dev(k), to_dev(v)
    dex = {name: to_dev(a) for name, a in ex.items()}
    dex["vdir"] = torch.zeros(n, NKV, D, device="cuda")
    out = torch.zeros(n, NQ * D, device="cuda")
    K.attn_verify(sh, to_dev(qkv), to_dev(meta), kd, vd, to_dev(table), to_dev(rope_tab), kv, args, to_dev(runs), S,
                  max(runs_T), to_dev(vis), out, extras=dex)
    torch.cuda.synchronize()
    close(out.cpu().numpy(), ref, atol=2e-4, rtol=2e-4, what="attention output")
    for name, got, want in (("K", kd.cpu().numpy(), k_ref), ("V", vd.cpu().numpy(), v_ref)):
        d = np.abs(oracle.bf16_to_f32(got) - oracle.bf16_to_f32(want))
        assert (d <= 2 ** -7 * np.abs(oracle.bf16_to_f32(want)) + 1e-30).all(), f"{name} cache off by more than one step"


def test_window_attention_refuses_bad_extras(gpu):
    """An extra without its inputs, or a sliding-window layer with window 0, is refused before
    any launch."""
    sh = CFG
    one = torch.zeros(16, device="cuda")
    kv = L.KvArgs(0, 0, 64, 1, 4, 4, 4, 0)
    args = L.AttnArgs(128, 2, 0.18, 1, 0, 0, 0, 0, 0)
    with pytest.raises(L.SvError, match="window 0"):
        K.attn_verify(sh, one, one, one, one, one, one, kv, args, one, 1, 5, one, one)
    kv.window = 64
    with pytest.raises(L.SvError, match="without its inputs"):
        K.attn_verify(sh, one, one, one, one, one, one, kv, args, one, 1, 5, one, one, extras={"xsa": one})


# -------------------------------------------------------------------------------- MUDD
@pytest.mark.parametrize("n,hidden", [(5, 1280), (160, 2048), (1, 256)])
def test_mudd_kernel(gpu, n, hidden):
    banner(f"mudd n={n} hidden={hidden}")
    rng = np.random.default_rng(n + hidden)
    cur, tap0, tap1 = (rng.normal(0, 1, (n, hidden)).astype(np.float32) for _ in range(3))
    dense1 = rng.normal(0, 0.05, (32, hidden)).astype(np.float32)
    mix = rng.normal(0, 0.3, (2, 3, 33)).astype(np.float32)
    ra, rb = oracle.mudd(cur, tap0, tap1, dense1, mix)
    oa = torch.zeros(n, hidden, device="cuda")
    ob = torch.zeros(n, hidden, device="cuda")
    K.mudd(to_dev(cur), to_dev(tap0), to_dev(tap1), to_dev(dense1), to_dev(mix), oa, ob)
    torch.cuda.synchronize()
    close(oa.cpu().numpy(), ra, 1e-5, 1e-5, "out_attn")
    close(ob.cpu().numpy(), rb, 1e-5, 1e-5, "out_base")


# ------------------------------------------------------------------------- whole steps
def build_limite_pair(shape, *, window, ctx, n_seqs=1, seed=0, max_seq_len=512, std=0.02, group=None,
                      max_step_tokens=64, max_head_rows=16):
    model = SyntheticModel.generate(shape, seed=seed, device="cpu", std=std, group=group)
    model = model.with_extras(generate_extras(shape, seed=seed + 7, window=window))
    freq = rope_freq(500000.0, shape.head_dim)
    eng = Engine(shape, max_seqs=n_seqs, max_step_tokens=max_step_tokens, max_seq_len=max_seq_len,
                 max_head_rows=max_head_rows, kv_tokens=n_seqs * max_seq_len, page_shift=4, attn_scale=0.125, freq=freq,
                 local=model.extras.local, window=window)
    gm = model.to("cuda")
    eng.set_model(gm)
    emb, lay, sc = oracle.host_weights(model)
    ref = oracle.OracleEngine(L, shape, emb, lay, sc, max_seqs=n_seqs, max_seq_len=max_seq_len,
                              kv_tokens=n_seqs * max_seq_len, page_shift=4, attn_scale=0.125, freq=freq,
                              extras=oracle.host_extras(model), max_step_tokens=max_step_tokens)
    assert eng.buf.ring_pages == ref.ring_pages and eng.buf.n_local_pages == ref.n_lpages
    kl, vl, tab = eng.local_cache()
    assert np.array_equal(tab.cpu().numpy().view(np.uint32), ref.local_table), "cyclic tables differ"
    rng = np.random.default_rng(seed + 1)
    slots = []
    for _ in range(n_seqs):
        a, b = eng.new_seq(), ref.new_seq()
        assert a == b
        slots.append(a)
    ctxs = [ctx] * n_seqs if np.isscalar(ctx) else list(ctx)
    for s, c in zip(slots, ctxs):
        eng.bench_fill(s, c)
        ref.bench_fill(s, c)
    kd, vd = eng.kv_cache()
    for dev_t, host in ((kd, ref.k), (vd, ref.v), (kl, ref.k_local), (vl, ref.v_local)):
        bits = rand_bits(rng, host.shape)
        host[...] = bits
        dev_t.copy_(torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16))
    torch.cuda.synchronize()
    return model, gm, eng, ref, slots, rng


def caches_close(eng, ref) -> None:
    kd, vd = eng.kv_cache()
    kl, vl, _ = eng.local_cache()
    for name, dev_t, host in (("K", kd, ref.k), ("V", vd, ref.v), ("K local", kl, ref.k_local),
                              ("V local", vl, ref.v_local)):
        got = oracle.bf16_to_f32(dev_t.view(torch.int16).cpu().numpy().view(np.uint16))
        want = oracle.bf16_to_f32(host)
        # one bf16 step, plus what the fp32 matmul upstream leaves on elements small against their
        # row (K rows are rms-normed: |k| ~ 1); a row written at a wrong place is off by O(1)
        bad = ~(np.abs(got - want) <= 2 ** -7 * np.abs(want) + 2e-3)
        if bad.any():
            idx = np.argwhere(bad)
            rows = sorted({tuple(int(v) for v in i[:4]) for i in idx})
            raise AssertionError(f"{name} cache: {bad.sum()} values in {len(rows)} rows (layer, page, head, row) "
                                 f"{rows[:8]}; first {idx[0].tolist()}: {got[tuple(idx[0])]} != {want[tuple(idx[0])]}")


def step_both(eng, ref, runs, slots, what):
    ids_r, logits_r, em_r, extra = ref.step(runs)
    res = eng.step(runs, logits=True)
    close(res.logits, logits_r, LOGIT_ATOL, LOGIT_RTOL, f"{what} logits")
    fin = np.isfinite(logits_r)  # the -inf columns past vocab_real were compared by close()
    err = np.abs(res.logits.astype(np.float64)[fin] - logits_r[fin])
    print(f"  {what}: logits max-abs err {err.max():.3e}", flush=True)
    greedy_ids_match(res.ids, ids_r, logits_r)
    same = np.array_equal(res.ids, ids_r)
    if same:
        assert np.array_equal(res.emitted, em_r), f"emitted {res.emitted} != {em_r}"
        for s in slots:
            assert eng.seq_len(s) == ref.seq_len[s] and eng.seq_pages(s) == ref.pool.pages(s)
    return same, ids_r, em_r, extra


def planted_tree_step(eng, ref, slots, rng, parents, path, vocab_real, what):
    """Drafts of a tree whose path root -> path... is set, level by level, to the oracle's greedy
    ids at the parents (probed on the oracle, then rolled back), so a path that is not a prefix
    of the rows is accepted and kv_compact moves it (global pages and local rings)."""
    nodes = tree_nodes(parents)
    n = len(parents)
    for s in slots:
        ref.feed[s * 16 + 1:s * 16 + n] = rng.integers(0, vocab_real, n - 1)
        ref.tree[s * 16:s * 16 + n] = nodes
    runs = [(s, [L.FEED_ROW + i for i in range(n)], True) for s in slots]
    for parent, child in zip((0,) + tuple(path[:-1]), path):
        saved = (ref.lens.copy(), ref.feed.copy(), ref.tree.copy(), list(ref.seq_len), bytes(ref.gen),
                 ref.k.copy(), ref.v.copy(), ref.k_local.copy(), ref.v_local.copy())
        ids = ref.step(runs)[0]
        ref.lens[:], ref.feed[:], ref.tree[:] = saved[0], saved[1], saved[2]
        ref.seq_len[:] = saved[3]
        C.memmove(ref.gen, saved[4], len(saved[4]))
        ref.k[...], ref.v[...], ref.k_local[...], ref.v_local[...] = saved[5:]
        for j, s in enumerate(slots):
            ref.feed[s * 16 + child] = ids[n * j + parent]
    put_u32(eng, "d_feed", ref.feed)
    put_u32(eng, "d_tree", ref.tree)
    same, ids_r, em_r, extra = step_both(eng, ref, runs, slots, what)
    if same:
        assert np.array_equal(dev_u32(eng, "d_path", (len(slots), 16)), extra["path"][:len(slots)])
        assert np.array_equal(dev_u32(eng, "d_lens", (len(slots),)), ref.lens[:len(slots)])
    return same, em_r


@pytest.mark.parametrize("which", ["cfg", "ref"])
def test_limite_model_steps(gpu, which):
    """An 8-layer Limite-layout model (6 sliding-window layers of 48 keys, value embeddings on
    layers 1, 4, 7, gates and XSA everywhere, MUDD before layers 4 and 7 with taps after 2 and
    3), two sequences past the window (their rings of 112 keys wrapped): a prompt chunk of 24
    rows each (attention runs of 16 or 12 after a kv_write pass), greedy chains with replayed drafts,
    and a tree with a planted non-prefix path (kv_compact over pages and rings)."""
    if which == "cfg":
        shape = ModelShape(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=512, vocab=1024, vocab_real=1000,
                           n_layers=8)
        parents, path = [None, 0, 0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 5, 6, 7, 8], (2, 7, 14)
    else:
        shape = ModelShape(hidden=1280, n_heads=10, n_kv_heads=2, head_dim=128, ffn=1280, vocab=1024,
                           vocab_real=1000, n_layers=8)
        parents, path = [None, 0, 0, 0, 1, 1, 2, 2, 3, 4, 6, 7], (2, 6, 10)
    banner(f"limite model steps {which}")
    model, gm, eng, ref, slots, rng = build_limite_pair(shape, window=48, ctx=[150, 201], n_seqs=2, seed=21,
                                                        max_seq_len=512, max_head_rows=32)
    assert eng.buf.ring_pages == 7
    prompt = [[int(t) for t in rng.integers(0, shape.vocab_real, 24)] for _ in slots]
    same, ids_r, _, _ = step_both(eng, ref, [(s, p, False, 1) for s, p in zip(slots, prompt)], slots, "chunk")
    assert same, "chunk step ids"
    caches_close(eng, ref)
    compared = 1
    for step in range(4):
        runs = []
        for s in slots:
            drafts = [int(x) for x in rng.integers(0, shape.vocab_real, int(rng.integers(1, 5)))]
            runs.append((s, [L.FEED_ROW] + drafts, True))
        same, _, _, _ = step_both(eng, ref, runs, slots, f"chain step {step}")
        if not same:
            break
        compared += 1
        caches_close(eng, ref)
    assert compared >= 3, "too few steps compared"
    if same:
        same, em = planted_tree_step(eng, ref, slots, rng, parents, path, shape.vocab_real, "tree step")
        if same:
            assert (em >= len(path) + 1).all(), "the planted path is accepted"
            caches_close(eng, ref)
    eng.close()


def test_limite_reference_shape_step(gpu):
    """The reference's own model shape (model.rs:6-21: 48 layers, hidden 1280, 10 x 128 query heads
    over 2 kv heads, ffn 3328, vocabulary 151680 with 151667 real, window 1024, MUDD at 24 and 47
    with taps 11 and 22, int8 groups of 64): one sequence 1500 tokens in (rings wrapped), a
    prompt chunk of 24 rows, then a verify chain of 5 rows, against the oracle."""
    banner("limite reference shape")
    model, gm, eng, ref, slots, rng = build_limite_pair(REFERENCE_SHAPE, window=1024, ctx=1500, seed=5,
                                                        max_seq_len=1600, group=64)
    s = slots[0]
    assert (eng.n_local, eng.buf.ring_pages) == (36, 68)
    prompt = [int(t) for t in rng.integers(0, REFERENCE_SHAPE.vocab_real, 24)]
    same, _, _, _ = step_both(eng, ref, [(s, prompt, False, 1)], slots, "chunk")
    if same:
        drafts = [int(x) for x in rng.integers(0, REFERENCE_SHAPE.vocab_real, 4)]
        step_both(eng, ref, [(s, [L.FEED_ROW] + drafts, True)], slots, "verify")
        caches_close(eng, ref)
    eng.close()


@pytest.mark.parametrize("head_group", [64, None])
def test_limite_from_weight_file(gpu, tmp_path, head_group):
    """A Limite-layout model written under the reference's tensor names (tools/convert.py:76-113:
    int8 layers in groups of 64, gates, XSA, value embeddings, MUDD, RoPE frequencies and an int8
    head of its own, groups of 64 or one per row), uploaded and resolved by VltModel (the layer
    pattern of model.rs:116), verifies two streams past the window against the oracle engine
    built from the same tensors."""
    banner(f"limite model from a weight file, head group {head_group}")
    from violetto.weights import VltModel, WeightFile, reference_tensors, write_vlt

    shape = ModelShape(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=512, vocab=1024, vocab_real=1000,
                       n_layers=8)
    window = 48
    model = SyntheticModel.generate(shape, seed=41, device="cpu", group=64)
    model = model.with_extras(generate_extras(shape, seed=42, window=window)).with_head(head_group)
    freq = rope_freq(500000.0, 64)
    path = tmp_path / "limite.vlt"
    write_vlt(path, reference_tensors(model, freq))
    wf = WeightFile(path)
    wf.upload()
    vm = VltModel(wf, shape, window=window)
    assert vm.limite and vm.extras.local == model.extras.local and vm.extras.mudd_layer == (4, 7)
    assert np.array_equal(vm.rope_freq(), freq)
    eng = Engine(shape, max_seqs=2, max_step_tokens=64, max_seq_len=512, max_head_rows=32, kv_tokens=1024,
                 attn_scale=0.125, freq=vm.rope_freq(), local=vm.extras.local, window=window)
    eng.set_model(vm)
    emb, lay, sc = oracle.host_weights(model)
    ref = oracle.OracleEngine(L, shape, emb, lay, sc, max_seqs=2, max_seq_len=512, kv_tokens=1024, attn_scale=0.125,
                              freq=freq, extras=oracle.host_extras(model), max_step_tokens=64,
                              head=oracle.host_head(model))
    rng = np.random.default_rng(43)
    slots = []
    for c in (130, 77):
        s = eng.new_seq()
        assert s == ref.new_seq()
        eng.bench_fill(s, c)
        ref.bench_fill(s, c)
        slots.append(s)
    kd, vd = eng.kv_cache()
    kl, vl, _ = eng.local_cache()
    for dev_t, host in ((kd, ref.k), (vd, ref.v), (kl, ref.k_local), (vl, ref.v_local)):
        bits = rand_bits(rng, host.shape)
        host[...] = bits
        dev_t.copy_(torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16))
    for s in slots:
        t = int(rng.integers(0, shape.vocab_real))
        eng.set_feed(s, ref.seq_len[s], t)
        ref.set_feed(s, ref.seq_len[s], t)
    for step in range(3):
        runs = [(s, [L.FEED_ROW] + [int(x) for x in rng.integers(0, shape.vocab_real, 4)], True) for s in slots]
        same, _, _, _ = step_both(eng, ref, runs, slots, f"step {step}")
        if not same:
            break
    eng.close()
    wf.close()


@pytest.mark.parametrize("group", [8, 32])
def test_head_in_small_groups(gpu, group):
    """The reference converter's default int8 head (groups of 8, tools/convert.py:20; model.rs:98
    accepts 8-256) and groups of 32, with layers in groups of 64 as INT8_DEFAULT writes them:
    the engine serves the head as two exact bf16 matrices hi + lo and a softcap pass. Two
    streams of 5-row verify steps (the one-shot matmul) and of 12-row steps (24 rows: the
    GEMM path) against the oracle engine with the same int8 head."""
    banner(f"int8 head in groups of {group}")
    shape = ModelShape(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=512, vocab=1024, vocab_real=1000,
                       n_layers=2)
    model = SyntheticModel.generate(shape, seed=17, device="cpu", group=64).with_head(group)
    freq = rope_freq(500000.0, 64)
    eng = Engine(shape, max_seqs=2, max_step_tokens=32, max_seq_len=512, max_head_rows=32, kv_tokens=1024,
                 attn_scale=0.125, freq=freq)
    eng.set_model(model.to("cuda"))
    emb, lay, sc = oracle.host_weights(model)
    ref = oracle.OracleEngine(L, shape, emb, lay, sc, max_seqs=2, max_seq_len=512, kv_tokens=1024, attn_scale=0.125,
                              freq=freq, head=oracle.host_head(model))
    rng = np.random.default_rng(group)
    slots = []
    for c in (200, 90):
        s = eng.new_seq()
        assert s == ref.new_seq()
        eng.bench_fill(s, c)
        ref.bench_fill(s, c)
        slots.append(s)
    kd, vd = eng.kv_cache()
    for dev_t, host in ((kd, ref.k), (vd, ref.v)):
        bits = rand_bits(rng, host.shape)
        host[...] = bits
        dev_t.copy_(torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16))
    for s in slots:
        t = int(rng.integers(0, shape.vocab_real))
        eng.set_feed(s, ref.seq_len[s], t)
        ref.set_feed(s, ref.seq_len[s], t)
    for step, rows in enumerate((5, 12, 5)):
        runs = [(s, [L.FEED_ROW] + [int(x) for x in rng.integers(0, shape.vocab_real, rows - 1)], True) for s in slots]
        same, _, _, _ = step_both(eng, ref, runs, slots, f"step {step} ({rows} rows per stream)")
        if not same:
            break
    eng.close()
