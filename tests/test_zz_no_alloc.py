"""sv_attn_verify_noalloc, the attention entry point that allocates nothing (its split partials
live in a static array of the library, one per GPU), against sv_attn_verify on the same inputs:
two calls in a row, the second with fewer runs and shorter contexts (the array keeps the first
call's partials), results bit-identical; and the size check that refuses partials larger than
the array before anything runs."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

import oracle
from conftest import banner
from helpers import to_dev
from test_gpu_kernels import SH, make_attn_case
from violetto import _lib as L
from violetto import kernels as K


def test_noalloc_refuses_partials_beyond_its_scratch():
    """Host-side check, no GPU: 64 runs of 16 rows over 65536-key contexts in 128-key splits need
    far more than the array; the call returns SV_ERR_CAPACITY and names the limit."""
    lib = L.lib()
    limit = lib.sv_attn_noalloc_max_bytes()
    assert limit == 32 << 20
    sh = SH.c()
    kv = L.KvArgs(1, 0, 0, 64, 4, 1, 1, 0)
    args = L.AttnArgs(128, 513, 0.18, 1, 0, 0, 0, 0, 0)
    assert lib.sv_attn_workspace_bytes(C.byref(sh), 64, 513, 16) > limit
    one = C.c_void_p(16)
    rc = lib.sv_attn_verify_noalloc(None, C.byref(sh), one, one, one, one, one, one, C.byref(kv), C.byref(args), one,
                                    64, 16, one, one)
    assert rc == 3 and b"scratch" in lib.sv_last_error()


def _call(case, runs_T, p0s, split, noalloc):
    c = case
    freq = (500000.0 ** (-2.0 * np.arange(32) / 64)).astype(np.float32)
    rope_tab = oracle.rope_table(freq, max(p0s) + 20)
    kv = L.KvArgs(1, 0, 0, len(runs_T), c["page_shift"], c["n_pages"], c["max_pages"], 0)
    max_splits = max(-(-p // split) + 1 for p in p0s)
    args = L.AttnArgs(split, max_splits, 0.125 * 1.4426950408889634, 1, 0, 0, 0, 0, 0)
    kd, vd = to_dev(c["k"]), to_dev(c["v"])
    out = torch.full((sum(runs_T), SH.n_heads * SH.head_dim), float("nan"), device="cuda")
    fn = K.attn_verify_noalloc if noalloc else K.attn_verify
    fn(SH, to_dev(c["qkv"]), to_dev(c["meta"]), kd, vd, to_dev(c["page_table"]), to_dev(rope_tab), kv, args,
       to_dev(c["runs"].reshape(-1).copy()), len(runs_T), max(runs_T), to_dev(c["vis"]), out)
    torch.cuda.synchronize()
    return out.cpu().numpy(), kd.cpu().numpy(), vd.cpu().numpy()


@pytest.mark.gpu
def test_noalloc_matches_allocating_entry_point(gpu):
    """configs[2]-like first call (32 runs of 5 rows, contexts 1024-8192, 1152-key splits), then a
    smaller one (3 runs, one with a 16-node tree, 256-key splits): outputs and the new K/V rows
    equal the allocating entry point's bit for bit."""
    rng = np.random.default_rng(5)
    calls = [([5] * 32, [int(x) for x in rng.integers(1024, 8193, 32)], 1152, False),
             ([5, 16, 3], [700, 2100, 33], 256, True)]
    for i, (runs_T, p0s, split, tree) in enumerate(calls):
        banner(f"attn noalloc call {i}: {len(runs_T)} runs, split {split}")
        case = make_attn_case(SH, runs_T, p0s, seed=40 + i, tree=tree)
        want = _call(case, runs_T, p0s, split, noalloc=False)
        got = _call(case, runs_T, p0s, split, noalloc=True)
        assert np.isfinite(got[0]).all()
        for g, w, what in zip(got, want, ("output", "K cache", "V cache")):
            assert np.array_equal(g, w), f"call {i}: {what} differs from sv_attn_verify"


def _window_case(sh, runs_T, p0s, seed):
    """A sliding-window layer (window 1024) over per-slot rings of pages reached through a
    cyclic page table (the layout the engine gives its local layers)."""
    rng = np.random.default_rng(seed)
    D, NQ, NKV = sh.head_dim, sh.n_heads, sh.n_kv_heads
    window, page = 1024, 16
    ring_pages = -(-(window + 64) // page)
    S = len(runs_T)
    max_pages = -(-(max(p0s) + 32) // page)
    table = np.array([[s * ring_pages + p % ring_pages for p in range(max_pages)] for s in range(S)], np.uint32)
    n_pages = S * ring_pages
    bits = lambda: (rng.integers(0x3C00, 0x4000, (1, n_pages, NKV, page, D), dtype=np.uint16) |
                    (rng.integers(0, 2, (1, n_pages, NKV, page, D), dtype=np.uint16) << np.uint16(15)))
    k, v = bits(), bits()
    n = sum(runs_T)
    meta = np.zeros((n, 2), np.uint32)
    vis = np.zeros(n, np.uint32)
    runs, t = [], 0
    for s, (T, p0) in enumerate(zip(runs_T, p0s)):
        meta[t:t + T, 0] = s
        meta[t:t + T, 1] = p0 + np.arange(T)
        vis[t:t + T] = [(2 << i) - 1 for i in range(T)]
        runs += [t, T]
        t += T
    qkv = rng.normal(0, 1, (n, (NQ + 2 * NKV) * D)).astype(np.float32)
    kv = L.KvArgs(0, 0, ring_pages * page, S, 4, n_pages, max_pages, window)
    return dict(qkv=qkv, meta=meta, vis=vis, runs=np.array(runs, np.uint32), k=k, v=v, page_table=table, kv=kv,
                max_splits=-(-(window + 31) // 256) + 1)


def _call_shape(sh, c, runs_T, p0s, split, kv, max_splits, noalloc):
    freq = (500000.0 ** (-2.0 * np.arange(32) / 64)).astype(np.float32)
    rope_tab = oracle.rope_table(freq, max(p0s) + 40)
    args = L.AttnArgs(split, max_splits, sh.head_dim ** -0.5 * 1.4426950408889634, 1, 0, 0, 0, 0, 0)
    kd, vd = to_dev(c["k"]), to_dev(c["v"])
    out = torch.full((sum(runs_T), sh.n_heads * sh.head_dim), float("nan"), device="cuda")
    fn = K.attn_verify_noalloc if noalloc else K.attn_verify
    fn(sh, to_dev(c["qkv"]), to_dev(c["meta"]), kd, vd, to_dev(c["page_table"]), to_dev(rope_tab), kv, args,
       to_dev(c["runs"].reshape(-1).copy()), len(runs_T), max(runs_T), to_dev(c["vis"]), out)
    torch.cuda.synchronize()
    return out.cpu().numpy(), kd.cpu().numpy(), vd.cpu().numpy()


@pytest.mark.gpu
def test_noalloc_window_layer_and_head_dim_128(gpu):
    """The scratch-free entry point on a sliding-window layer (ring caches through a cyclic
    page table, runs past, inside and across the window; the LOCAL kernel variant) and at head
    dim 128 (the reference's shape: 10 query heads over 2 kv heads), each bit-identical to
    sv_attn_verify; the second call is the smaller one."""
    from violetto.model import ModelShape
    ref_sh = ModelShape(hidden=1280, n_heads=10, n_kv_heads=2, head_dim=128, ffn=3328, vocab=4096, vocab_real=4096,
                        n_layers=1)
    banner("attn noalloc: window layer")
    runs_T, p0s = [5, 12, 3], [2500, 300, 1030]
    c = _window_case(SH, runs_T, p0s, seed=61)
    want = _call_shape(SH, c, runs_T, p0s, 256, c["kv"], c["max_splits"], noalloc=False)
    got = _call_shape(SH, c, runs_T, p0s, 256, c["kv"], c["max_splits"], noalloc=True)
    assert np.isfinite(got[0]).all()
    for g, w, what in zip(got, want, ("output", "K cache", "V cache")):
        assert np.array_equal(g, w), f"window layer: {what} differs from sv_attn_verify"
    banner("attn noalloc: head dim 128")
    runs_T, p0s = [5, 3], [3000, 90]
    c = make_attn_case(ref_sh, runs_T, p0s, seed=62)
    kv = L.KvArgs(1, 0, 0, len(runs_T), c["page_shift"], c["n_pages"], c["max_pages"], 0)
    max_splits = max(-(-p // 512) + 1 for p in p0s)
    want = _call_shape(ref_sh, c, runs_T, p0s, 512, kv, max_splits, noalloc=False)
    got = _call_shape(ref_sh, c, runs_T, p0s, 512, kv, max_splits, noalloc=True)
    assert np.isfinite(got[0]).all()
    for g, w, what in zip(got, want, ("output", "K cache", "V cache")):
        assert np.array_equal(g, w), f"head dim 128: {what} differs from sv_attn_verify"
