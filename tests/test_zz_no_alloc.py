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
