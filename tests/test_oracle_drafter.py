"""Pinning the oracle's drafter (CPU only): engine/src/engine/drafter.rs:278-447 and its kernels
(kernels.metal:135-148, 1725-1836) against an independent float64 torch restatement of the
training-time model, tools/spec/drafter.py (Drafter.context / forward, Layer, Conv2, attend,
block_mask), written from that file's algebra: one softmax over the window of context keys
before the block and the whole block, left-to-right two-tap convolutions, the inject of the
context before the block, the final norm into the head. The engine stores keys and values in
bf16 rings, so the restatement rounds k and v to bf16 where the engine stores them; everything
else is float64. A dropped convolution tap, a window off by one, a block row that misses a
later row of its block, or an inject from the wrong position fails these checks."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

import oracle
from violetto import _lib as L
from violetto.drafter import SyntheticDrafter
from violetto.model import ModelShape, rope_freq

O = oracle
SH = ModelShape(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=384, vocab=512, vocab_real=500, n_layers=4)
EPS = L.RMS_EPS


def rms_t(x: torch.Tensor) -> torch.Tensor:
    return x / torch.sqrt((x * x).mean(-1, keepdim=True) + EPS)


def bf16_t(x: torch.Tensor) -> torch.Tensor:
    return x.float().bfloat16().double()


def rope_t(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """drafter.py rope: pairs (2j, 2j + 1) of dims 0..63 -> (c a0 + s a1, c a1 - s a0)."""
    xr = x[..., :64].unflatten(-1, (32, 2))
    a0, a1 = xr[..., 0], xr[..., 1]
    out = torch.stack([cos * a0 + sin * a1, cos * a1 - sin * a0], -1).flatten(-2)
    return torch.cat([out, x[..., 64:]], -1)


def restated_block(d: SyntheticDrafter, taps: list[np.ndarray], ctx_pos: np.ndarray, L0: int, bonus: int,
                   rows: int, embed_bits: np.ndarray, rope: np.ndarray, scale: float) -> torch.Tensor:
    """The raw logits [rows][v] of one block at position L0 (rows L0 .. L0 + rows - 1) whose
    context is every tapped position in ctx_pos (< L0), from drafter.py's forward."""
    s = d.shape
    H, NQ, NKV, D, F = s.hidden, s.n_heads, s.n_kv_heads, s.head_dim, s.ffn
    G = NQ // NKV
    cs = torch.from_numpy(rope.astype(np.float64)).view(-1, 32, 2)
    cos, sin = cs[..., 0], cs[..., 1]
    feats = sum(d.dense(f"fc.{k}") @ torch.from_numpy(taps[k]).double().T for k in range(len(taps))).T  # [C][H]
    ctx = rms_t(feats)
    pos_c = torch.from_numpy(ctx_pos.astype(np.int64))
    pos_b = torch.arange(L0, L0 + rows)
    emb = torch.from_numpy(embed_bits.astype(np.int32)).to(torch.int16).view(torch.bfloat16).double()
    x = torch.cat([rms_t(emb[bonus])[None], d.mask_emb.double().expand(rows - 1, H)])
    if d.inject:
        last = ctx[int(np.nonzero(ctx_pos == L0 - 1)[0][0])]
        x = x + d.dense("inject") @ last
    # Conv2 (drafter.py:52-57): k = base + corr(rms(x)) per 16 channels; out_t = k0 x_t + k1 x_(t-1)
    def conv(li: int, c: int, v: torch.Tensor) -> torch.Tensor:
        key = f"D{li:02d}.conv{c}"
        if key not in d.conv_base:
            return v
        base = d.conv_base[key].double()
        corr = (d.dense(key + ".corr") @ rms_t(v).T).T[:, : H // 8]  # [rows][2 H / 16]
        k = base[None] + corr.unflatten(-1, (2, H // 16)).repeat_interleave(16, -1)
        prev = torch.cat([torch.zeros(1, H, dtype=v.dtype), v[:-1]])
        return k[:, 0] * v + k[:, 1] * prev

    # visibility of the context: row i sees positions [L0 + i - window, L0) (block_mask)
    win = d.window
    vis_c = torch.stack([(pos_c < L0) & (pos_c >= L0 + i - win) for i in range(rows)])  # [rows][C]
    kv_w = d.dense("kv_all")
    for li in range(d.n_layers):
        qkv_w = d.dense(f"D{li:02d}.qkv")
        wq, wk, wv = qkv_w[: NQ * D], qkv_w[NQ * D:(NQ + NKV) * D], qkv_w[(NQ + NKV) * D:]
        # Layer.kv of the context, from kv_all's rows of this layer (export.py: wk, wv per layer)
        kvl = kv_w[li * 2 * NKV * D:(li + 1) * 2 * NKV * D]
        kc = rms_t((ctx @ kvl[: NKV * D].T).unflatten(-1, (NKV, D)))
        kc = bf16_t(rope_t(kc, cos[pos_c][:, None], sin[pos_c][:, None]))
        vc = bf16_t((ctx @ kvl[NKV * D:].T).unflatten(-1, (NKV, D)))
        h = rms_t(conv(li, 0, x))
        q = rope_t(rms_t((h @ wq.T).unflatten(-1, (NQ, D))), cos[pos_b][:, None], sin[pos_b][:, None])
        kb = bf16_t(rope_t(rms_t((h @ wk.T).unflatten(-1, (NKV, D))), cos[pos_b][:, None], sin[pos_b][:, None]))
        vb = bf16_t((h @ wv.T).unflatten(-1, (NKV, D)))
        out = torch.zeros(rows, NQ, D, dtype=torch.float64)
        for hq in range(NQ):
            g = hq // G
            sc = torch.cat([q[:, hq] @ kc[:, g].T, q[:, hq] @ kb[:, g].T], -1) * scale  # [rows][C + rows]
            mask = torch.cat([vis_c, torch.ones(rows, rows, dtype=torch.bool)], -1)
            p = torch.softmax(sc.masked_fill(~mask, float("-inf")), -1)
            out[:, hq] = p @ torch.cat([vc[:, g], vb[:, g]])
        o = out.flatten(-2) @ d.dense(f"D{li:02d}.o").T
        x = x + conv(li, 1, o)
        gu = (rms_t(conv(li, 2, x)) @ d.dense(f"D{li:02d}.gate_up").T).unflatten(-1, (F, 2))
        act = torch.nn.functional.silu(gu[..., 0]) * gu[..., 1]
        x = x + conv(li, 3, act @ d.dense(f"D{li:02d}.down").T)
    return rms_t(x) @ d.dense("head").T


def run_draft(d: SyntheticDrafter, taps, meta, on_path, lens, feed, blocks, tin, vis, embed_bits, rope, scale,
              k_ring=None, v_ring=None, cring=None, page_shift=4, max_seqs=2, max_pages=32, ring_pages=None):
    """orc_draft over one step (context of the tokens in meta, then the blocks)."""
    s = d.shape
    page = 1 << page_shift
    ring_pages = ring_pages or -(-(d.window + 64) // page)
    n_pages = max_seqs * ring_pages
    table = np.array([[sl * ring_pages + p % ring_pages for p in range(max_pages)] for sl in range(max_seqs)], np.uint32)
    if k_ring is None:
        k_ring = np.zeros((d.n_layers, n_pages, s.n_kv_heads, page, s.head_dim), np.uint16)
        v_ring = np.zeros_like(k_ring)
        cring = np.zeros((max_seqs, 64, s.hidden), np.float32)
    dc, keep = O.host_drafter(d)
    n = len(on_path)
    rows = len(vis)
    tap_arr = [np.ascontiguousarray(t, np.float32) for t in taps]
    tp = (C.c_void_p * len(tap_arr))(*[t.ctypes.data for t in tap_arr])
    logits = np.zeros((max(1, rows), d.v), np.float32)
    ctx = np.zeros((max(1, n), s.hidden), np.float32)
    io = O.DraftIO()
    io.n, io.taps, io.meta, io.on_path, io.rope = n, C.cast(tp, C.c_void_p), O.ptr(meta), O.ptr(on_path), O.ptr(rope)
    io.k_ring, io.v_ring, io.table = O.ptr(k_ring), O.ptr(v_ring), O.ptr(table)
    io.kv[:] = [0, 0, ring_pages << page_shift, max_seqs, page_shift, n_pages, max_pages, d.window]
    io.ctx_ring, io.cr = O.ptr(cring), 64 if d.inject else 0
    io.n_blocks, io.rows = len(blocks) // 2, rows
    io.blocks, io.tin, io.vis = O.ptr(blocks), O.ptr(tin), O.ptr(vis)
    io.lens, io.feed = O.ptr(lens), O.ptr(feed)
    tree = np.zeros(max_seqs * 16, np.uint32)
    io.tree = O.ptr(tree)
    io.logits, io.ctx = O.ptr(logits), O.ptr(ctx)
    sh = s.c()
    rc = O.lib().orc_draft(C.byref(sh), O.ptr(embed_bits), C.byref(dc), C.c_float(scale), C.byref(io))
    assert rc == 0
    return logits[:rows], ctx[:n], tree, (k_ring, v_ring, cring)


def make_case(seed=0, convs=True, inject=True, window=24, head_group=8, n_layers=2):
    d = SyntheticDrafter.generate(SH, n_layers=n_layers, taps=(1, 3), v=256, window=window, seed=seed, convs=convs,
                                  inject=inject, head_group=head_group, conv_std=0.2)
    rng = np.random.default_rng(seed)
    embed = torch.randn(SH.vocab, SH.hidden, generator=torch.Generator().manual_seed(seed + 7)) * 0.5
    embed_bits = embed.bfloat16().view(torch.int16).numpy().view(np.uint16).copy()
    rope = O.rope_table(rope_freq(10000.0, SH.head_dim), 256)
    return d, rng, embed_bits, rope


def taps_for(rng, n):
    """Tapped rows as the engine writes them: rms-normed and rounded to bf16."""
    out = []
    for _ in range(2):
        t = rng.normal(0, 1, (n, SH.hidden)).astype(np.float32)
        t = (t / np.sqrt((t.astype(np.float64) ** 2).mean(-1, keepdims=True) + EPS)).astype(np.float32)
        out.append(torch.from_numpy(t).bfloat16().float().numpy())
    return out


@pytest.mark.parametrize("convs,inject,window", [(True, True, 24), (False, False, 24), (True, False, 200),
                                                 (False, True, 5)])
def test_one_step_block_against_drafter_py(convs, inject, window):
    """One step feeding positions 0..39 of slot 1, then a block of 4 rows at position 40:
    the oracle's raw logits against the float64 restatement of drafter.py."""
    d, rng, embed_bits, rope = make_case(convs=convs, inject=inject, window=window)
    n, rows, slot = 40, 4, 1
    taps = taps_for(rng, n)
    meta = np.array([[slot, p] for p in range(n)], np.uint32).reshape(-1)
    on_path = np.ones(n, np.uint32)
    lens = np.array([0, n], np.uint32)
    feed = np.zeros(2 * 16, np.uint32)
    feed[slot * 16] = 123
    blocks = np.array([0, rows], np.uint32)
    tin = np.array([[slot, i] for i in range(rows)], np.uint32).reshape(-1)
    vis = np.full(rows, (1 << rows) - 1, np.uint32)
    scale = 0.1
    got, ctx, tree, _ = run_draft(d, taps, meta, on_path, lens, feed, blocks, tin, vis, embed_bits, rope, scale)
    want = restated_block(d, taps, np.arange(n), n, 123, rows, embed_bits, rope, scale).numpy()
    err = np.abs(got - want).max()
    assert err <= 2e-4 * max(1.0, np.abs(want).max()), err
    # the context: sum over taps of fc[k] tap_k, unnormed
    want_ctx = sum(d.dense(f"fc.{k}").numpy() @ taps[k].astype(np.float64).T for k in range(2)).T
    np.testing.assert_allclose(ctx, want_ctx, rtol=1e-5, atol=1e-5)


def test_off_path_tokens_and_two_steps():
    """Context built over two steps, with the second step's rejected branch (off path) never
    reaching the rings: the block equals the restatement over the on-path positions only. Two
    blocks (slots 0 and 1, 3 and 2 rows) in one pass, each with its own context."""
    d, rng, embed_bits, rope = make_case(seed=3, window=30)
    scale = 0.1
    # step 1: slot 0 positions 0..19, slot 1 positions 0..24
    n1 = 20 + 25
    taps1 = taps_for(rng, n1)
    meta1 = np.array([[0, p] for p in range(20)] + [[1, p] for p in range(25)], np.uint32).reshape(-1)
    lens = np.array([20, 25], np.uint32)
    feed = np.zeros(32, np.uint32)
    empty = np.zeros(1, np.uint32)
    _, _, _, state = run_draft(d, taps1, meta1, np.ones(n1, np.uint32), lens, feed, empty, np.zeros(2, np.uint32),
                               empty, embed_bits, rope, scale)
    # step 2: slot 0 verifies 4 rows at 20..23 of which the path keeps rows 0, 2 (positions 20, 21
    # after compaction the engine reports meta by the row's own position: a branch row shares its
    # position with its sibling), slot 1 feeds 3 tokens at 25..27 all on path
    meta2 = np.array([[0, 20], [0, 21], [0, 21], [0, 22], [1, 25], [1, 26], [1, 27]], np.uint32).reshape(-1)
    on2 = np.array([1, 0, 1, 0, 1, 1, 1], np.uint32)
    taps2 = taps_for(rng, 7)
    lens = np.array([22, 28], np.uint32)
    feed[0], feed[16] = 77, 301
    blocks = np.array([0, 3, 3, 2], np.uint32)
    tin = np.array([[0, 0], [0, 1], [0, 2], [1, 0], [1, 1]], np.uint32).reshape(-1)
    vis = np.array([7, 7, 7, 3, 3], np.uint32)
    got, _, _, _ = run_draft(d, taps2, meta2, on2, lens, feed, blocks, tin, vis, embed_bits, rope, scale, *state)
    for slot, (first, rows, L0, bonus) in enumerate([(0, 3, 22, 77), (3, 2, 28, 301)]):
        if slot == 0:
            tp = [np.concatenate([taps1[k][:20], taps2[k][[0, 2]]]) for k in range(2)]
            pos = np.arange(22)
        else:
            tp = [np.concatenate([taps1[k][20:], taps2[k][4:]]) for k in range(2)]
            pos = np.arange(28)
        want = restated_block(d, tp, pos, L0, bonus, rows, embed_bits, rope, scale).numpy()
        err = np.abs(got[first:first + rows] - want).max()
        assert err <= 2e-4 * max(1.0, np.abs(want).max()), (slot, err)


def test_identity_convolutions_equal_no_convolutions():
    """Conv2 starts as the identity (base (1, 0), zero corrections: drafter.py:47-50): such a
    drafter drafts what the same drafter without convolutions drafts (up to the fp32 rounding
    of the intermediate rows the convolution path stores)."""
    d, rng, embed_bits, rope = make_case(seed=5, convs=True)
    plain = SyntheticDrafter(d.shape, d.n_layers, d.taps, d.window, d.device,
                             {k: v for k, v in d.mats.items() if ".conv" not in k}, {}, d.mask_emb, d.vocab)
    for key in d.conv_base:
        d.conv_base[key] = torch.stack([torch.ones(SH.hidden), torch.zeros(SH.hidden)])
        w, s = d.mats[key + ".corr"]
        d.mats[key + ".corr"] = (torch.zeros_like(w), s)
    n, rows = 12, 3
    taps = taps_for(rng, n)
    args = (np.array([[0, p] for p in range(n)], np.uint32).reshape(-1), np.ones(n, np.uint32),
            np.array([n, 0], np.uint32), np.zeros(32, np.uint32), np.array([0, rows], np.uint32),
            np.array([[0, i] for i in range(rows)], np.uint32).reshape(-1), np.full(rows, 7, np.uint32))
    a, *_ = run_draft(d, taps, *args, embed_bits, rope, 0.1)
    b, *_ = run_draft(plain, taps, *args, embed_bits, rope, 0.1)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6)


def test_tap_rows_is_bf16_of_rms_norm():
    rng = np.random.default_rng(2)
    x = (rng.normal(0, 3, (5, 256))).astype(np.float32)
    out = np.zeros_like(x)
    O.lib().orc_tap_rows(O.ptr(x), O.ptr(out), C.c_uint32(5), C.c_uint32(256))
    t = torch.from_numpy(x).double()
    want = (t / torch.sqrt((t * t).mean(-1, keepdim=True) + EPS)).float().bfloat16().float().numpy()
    # one bf16 step apart at most where the float64 norm sits on a rounding boundary
    assert (np.abs(out - want) <= np.abs(want) * 2.0 ** -8).all()
    assert (out == want).mean() > 0.99


def test_draft_tree_from_block_logits():
    """The block's trees come out of draft_top and draft_tree over the oracle's logits: row 0
    of the feed keeps the bonus token, its drafts are ids of the draft vocabulary, and a block
    of R rows drafts R - 1 nodes."""
    d, rng, embed_bits, rope = make_case(seed=9)
    n, rows, slot = 16, 4, 0
    taps = taps_for(rng, n)
    meta = np.array([[slot, p] for p in range(n)], np.uint32).reshape(-1)
    feed = np.zeros(32, np.uint32)
    feed[0] = 55
    got, _, tree, _ = run_draft(d, taps, meta, np.ones(n, np.uint32), np.array([n, 0], np.uint32), feed,
                                np.array([0, rows], np.uint32),
                                np.array([[slot, i] for i in range(rows)], np.uint32).reshape(-1),
                                np.full(rows, 15, np.uint32), embed_bits, rope, 0.1)
    assert feed[0] == 55
    vocab = set(d.vocab.tolist())
    assert all(int(t) in vocab for t in feed[1:rows])
    # the first draft is the best candidate of row 1 (the row after the bonus token)
    best = d.vocab[int(np.argmax(got[1]))].item()
    assert feed[1] == best
