"""GPU parity of each kernel group against the oracle, through the C ABI (libsv_verify.so).

Integer and sampling results are compared bit for bit; fp32 results within tolerances stated
per test (fp32 accumulation in a different order, activations as bf16 hi + lo pairs: 16
significant bits per element)."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

import oracle
from conftest import banner
from helpers import bf16_bits, close, to_dev, u16_dev_bf16
from violetto import _lib as L
from violetto import kernels as K
from violetto.model import ModelShape, quantize_rows

pytestmark = pytest.mark.gpu

SH = ModelShape(n_layers=2)  # the configs' layer shapes


# ------------------------------------------------------------------------------- matmul
MM_CASES = [
    # (m, k, fmt)
    (3072, 2048, "i8"),   # qkv
    (2048, 8192, "i8"),   # down: k over 8 workgroups
    (512, 1280, "i8"),    # the reference's k: a partial workgroup of k slices
    (256, 3328, "bf16"),  # the reference's FFN k
    (1024, 2048, "bf16"),
]


@pytest.mark.parametrize("m,k,fmt", MM_CASES)
@pytest.mark.parametrize("n", [1, 5, 16])
@pytest.mark.parametrize("epi", [L.EPI_NORM, L.EPI_RESID, L.EPI_SWIGLU, L.EPI_HEAD, L.EPI_RAW])
@pytest.mark.parametrize("tiled", [False, True])
def test_matmul(gpu, m, k, fmt, n, epi, tiled):
    banner(f"matmul m={m} k={k} {fmt} n={n} epi={epi} tiled={tiled}")
    rng = np.random.default_rng(1000 * n + epi)
    w = torch.from_numpy(rng.normal(0, 0.02, (m, k)).astype(np.float32))
    if fmt == "i8":
        q, s = quantize_rows(w)
        wq, sc = q.numpy(), s.view(torch.int16).numpy().view(np.uint16)
        mat = K.matrix(q.cuda(), s.cuda(), 31)
        host_w, host_s, gs = wq, sc, 31
    else:
        wb = bf16_bits(w.numpy())
        mat = K.matrix(u16_dev_bf16(wb))
        host_w, host_s, gs = wb, None, 0
    if tiled:
        mat = mat.tiled()
    x = (rng.normal(0, 1, (n, k)) * rng.uniform(0.5, 4, (n, 1))).astype(np.float32)
    base = rng.normal(0, 1, (n, m)).astype(np.float32)
    flags = L.FLAG_WRITE_INV if epi == L.EPI_NORM else (L.FLAG_NORM_IN if epi in (L.EPI_HEAD, L.EPI_RAW) else 0)
    if epi == L.EPI_RESID:
        flags = L.FLAG_WRITE_RAW
    scale, ra, rb = 0.75, 0.9, 1.3
    vocab_real = m - 7
    a = L.MatArgs(n, k, m, epi, flags, vocab_real, scale, ra, rb, 1, k, gs)
    out_m = m // 2 if epi == L.EPI_SWIGLU else m
    aux_n = n if epi == L.EPI_NORM else n * m
    aux_ref = np.zeros(aux_n, np.float32)
    ref = oracle.matmul(L, host_w, host_s, gs, x, a, base=base if epi == L.EPI_RESID else None, aux=aux_ref)
    y = torch.zeros(n, out_m, device="cuda")
    aux = torch.zeros(aux_n, device="cuda")
    K.matmul(mat, to_dev(x), y, n=n, epi=epi, flags=flags, scale=scale, ra=ra, rb=rb,
             base=to_dev(base) if epi == L.EPI_RESID else None, aux=aux, vocab_real=vocab_real)
    torch.cuda.synchronize()
    assert C.c_int.in_dll(L.lib(), "_ZN2sv12g_mm_variantE").value == 3, "1-16 rows run the one-shot kernel"
    got = y.cpu().numpy()
    # Tolerance: |error| <= 2e-5 x the norm of the terms summed (hi/lo split: 2^-17 per term).
    mag = float(np.abs(ref[np.isfinite(ref)]).max())
    close(got, ref, atol=5e-5 * max(mag, 1.0), rtol=1e-4, what=f"matmul epi {epi}")
    if epi in (L.EPI_NORM, L.EPI_RESID):
        close(aux.cpu().numpy(), aux_ref, atol=1e-5 * max(1.0, np.abs(aux_ref).max()), rtol=1e-4, what="aux")


@pytest.mark.parametrize("n", [5, 160])
@pytest.mark.parametrize("tiled", [False, True])
def test_matmul_scales_unaligned(gpu, n, tiled):
    """Per-row int8 scales placed 2 bytes past an aligned base (the weight file only promises
    the element's alignment for a `.scale` tensor): every kernel reads them as 16-bit words."""
    banner(f"matmul unaligned scales n={n} tiled={tiled}")
    m, k = 2048, 2048
    rng = np.random.default_rng(77 + n)
    w = torch.from_numpy(rng.normal(0, 0.02, (m, k)).astype(np.float32))
    q, s = quantize_rows(w)
    buf = torch.zeros(m + 8, dtype=s.dtype, device="cuda")
    buf[1:m + 1] = s.cuda().view(-1)
    sd = buf[1:m + 1]
    assert sd.data_ptr() % 8 == 2
    mat = K.matrix(q.cuda(), sd, 31)
    if tiled:
        mat = mat.tiled()
    x = rng.normal(0, 1, (n, k)).astype(np.float32)
    base = rng.normal(0, 1, (n, m)).astype(np.float32)
    a = L.MatArgs(n, k, m, L.EPI_RESID, 0, m, 0.75, 0.9, 1.3, 1, k, 31)
    ref = oracle.matmul(L, q.numpy(), s.view(torch.int16).numpy().view(np.uint16), 31, x, a, base=base)
    y = torch.zeros(n, m, device="cuda")
    K.matmul(mat, to_dev(x), y, n=n, epi=L.EPI_RESID, scale=0.75, ra=0.9, rb=1.3, base=to_dev(base))
    torch.cuda.synchronize()
    close(y.cpu().numpy(), ref, atol=5e-5 * max(float(np.abs(ref).max()), 1.0), rtol=1e-4, what="unaligned scales")


def test_matmul_rows_gather(gpu):
    """x_rows gathers input rows (the head's head_rows)."""
    banner("matmul gather")
    rng = np.random.default_rng(7)
    m, k, n = 512, 2048, 4
    wb = bf16_bits(rng.normal(0, 0.02, (m, k)).astype(np.float32))
    x = rng.normal(0, 1, (9, k)).astype(np.float32)
    rows = np.array([8, 0, 3, 3], np.uint32)
    a = L.MatArgs(n, k, m, L.EPI_HEAD, L.FLAG_NORM_IN, m, 1.0, 0, 0, 1, k, 0)
    ref = oracle.matmul(L, wb, None, 0, x, a, x_rows=rows)
    y = torch.zeros(n, m, device="cuda")
    K.matmul(K.matrix(u16_dev_bf16(wb)), to_dev(x), y, n=n, epi=L.EPI_HEAD, flags=L.FLAG_NORM_IN,
             x_rows=to_dev(rows))
    torch.cuda.synchronize()
    close(y.cpu().numpy(), ref, atol=1e-4, rtol=1e-5, what="gathered head")


def test_matmul_repeat_workspace(gpu):
    """20 calls in a row give identical results (no scheduling-dependent sums)."""
    banner("matmul repeat")
    rng = np.random.default_rng(3)
    m, k, n = 2048, 8192, 5
    q, s = quantize_rows(torch.from_numpy(rng.normal(0, 0.02, (m, k)).astype(np.float32)))
    mat = K.matrix(q.cuda(), s.cuda(), 31)
    x = to_dev(rng.normal(0, 1, (n, k)).astype(np.float32))
    ws = K.Workspace(L.lib().sv_matmul_workspace_bytes(n, m, k))
    outs = []
    for _ in range(20):
        y = torch.zeros(n, m, device="cuda")
        K.matmul(mat, x, y, n=n, epi=L.EPI_RAW, ws=ws)
        outs.append(y)
    torch.cuda.synchronize()
    for y in outs[1:]:
        assert torch.equal(y, outs[0])


def test_matmul_shared_workspace_across_shapes(gpu):
    """Matmuls of different shapes, each with k splits, take turns on one workspace (as in an
    engine step): each finds its hand-off counters at zero and its results match the oracle."""
    banner("matmul shared workspace")
    rng = np.random.default_rng(21)
    n = 5
    qd, sd = quantize_rows(torch.from_numpy(rng.normal(0, 0.02, (2048, 8192)).astype(np.float32)))
    down = K.matrix(qd.cuda(), sd.cuda(), 31)
    wh = bf16_bits(rng.normal(0, 0.02, (32000, 2048)).astype(np.float32))
    head = K.matrix(u16_dev_bf16(wh))
    ws = K.Workspace(max(L.lib().sv_matmul_workspace_bytes(n, 2048, 8192), L.lib().sv_matmul_workspace_bytes(n, 32000, 2048)))
    xd = rng.normal(0, 1, (n, 8192)).astype(np.float32)
    xh = rng.normal(0, 1, (8, 2048)).astype(np.float32)
    rows = np.array([3, 0, 7, 1, 5], np.uint32)
    ad = L.MatArgs(n, 8192, 2048, L.EPI_RAW, 0, 2048, 1.0, 0, 0, 1, 8192, 31)
    ah = L.MatArgs(n, 2048, 32000, L.EPI_HEAD, L.FLAG_NORM_IN, 32000, 1.0, 0, 0, 1, 2048, 0)
    ref_d = oracle.matmul(L, qd.numpy(), sd.view(torch.int16).numpy().view(np.uint16), 31, xd, ad)
    ref_h = oracle.matmul(L, wh, None, 0, xh, ah, x_rows=rows)
    for rep in range(2):
        yd = torch.zeros(n, 2048, device="cuda")
        yh = torch.zeros(n, 32000, device="cuda")
        K.matmul(down, to_dev(xd), yd, n=n, epi=L.EPI_RAW, ws=ws)
        K.matmul(head, to_dev(xh), yh, n=n, epi=L.EPI_HEAD, flags=L.FLAG_NORM_IN, x_rows=to_dev(rows), ws=ws)
        torch.cuda.synchronize()
        close(yd.cpu().numpy(), ref_d, atol=5e-5 * max(1.0, float(np.abs(ref_d).max())), rtol=1e-4, what=f"down {rep}")
        close(yh.cpu().numpy(), ref_h, atol=1e-4, rtol=1e-5, what=f"head {rep}")


@pytest.mark.parametrize("rt,waves,splits", [(1, 8, 2), (1, 4, 8), (2, 8, 4), (4, 4, 2), (2, 16, 1), (1, 16, 2)])
def test_matmul_skinny_launch_shapes(gpu, rt, waves, splits):
    """Every skinny launch shape (row tiles, waves, k splits) gives the oracle's result,
    including the sums of squares carried across splits (EPI_NORM), on two calls that share
    one workspace. The shape is forced through the library's internal override."""
    banner(f"matmul launch shape rt={rt} waves={waves} splits={splits}")
    tune = (C.c_int * 4).in_dll(L.lib(), "_ZN2sv13g_skinny_tuneE")
    rng = np.random.default_rng(rt * 100 + waves * 10 + splits)
    m, k, n = 2048, 8192, 5
    q, s = quantize_rows(torch.from_numpy(rng.normal(0, 0.02, (m, k)).astype(np.float32)))
    mat = K.matrix(q.cuda(), s.cuda(), 31)
    ws = K.Workspace(32 << 20)
    try:
        tune[0], tune[1], tune[2], tune[3] = rt, waves, splits, 1
        for call in range(2):
            x = (rng.normal(0, 1, (n, k)) * rng.uniform(0.5, 4, (n, 1))).astype(np.float32)
            a = L.MatArgs(n, k, m, L.EPI_NORM, L.FLAG_WRITE_INV, m, 0.75, 0, 0, 1, k, 31)
            aux_ref = np.zeros(n, np.float32)
            ref = oracle.matmul(L, q.numpy(), s.view(torch.int16).numpy().view(np.uint16), 31, x, a, aux=aux_ref)
            y = torch.zeros(n, m, device="cuda")
            aux = torch.zeros(n, device="cuda")
            K.matmul(mat, to_dev(x), y, n=n, epi=L.EPI_NORM, flags=L.FLAG_WRITE_INV, scale=0.75, aux=aux, ws=ws)
            torch.cuda.synchronize()
            assert C.c_int.in_dll(L.lib(), "_ZN2sv12g_mm_variantE").value == 1, "skinny kernel not launched"
            close(y.cpu().numpy(), ref, atol=5e-5 * max(float(np.abs(ref).max()), 1.0), rtol=1e-4,
                  what=f"call {call}")
            close(aux.cpu().numpy(), aux_ref, atol=1e-5, rtol=1e-4, what="inv")
    finally:
        tune[0] = tune[1] = tune[2] = tune[3] = 0


@pytest.mark.parametrize("rt,waves,nch,splits", [(1, 8, 1, 1), (2, 8, 1, 1), (4, 8, 1, 1), (1, 8, 2, 1), (2, 8, 2, 1),
                                                (1, 8, 4, 1), (1, 4, 1, 2), (1, 4, 2, 2), (1, 8, 2, 2), (2, 8, 1, 2)])
@pytest.mark.parametrize("n", [3, 5, 12])
def test_matmul_one_shot_launch_shapes(gpu, rt, waves, nch, splits, n):
    """Every one-shot launch shape of the 1-16 row kernel (row tiles, waves, chunks per wave,
    k splits merged by the last split to arrive; chunks past k and token slots past n are read
    and discarded) gives the oracle's result, int8 with the sums of squares of EPI_NORM and
    bf16 with EPI_RESID's base, in both weight layouts, on calls that share one workspace. The
    shape is forced through the library's internal override."""
    banner(f"matmul one-shot rt={rt} waves={waves} nch={nch} splits={splits} n={n}")
    tune = (C.c_int * 5).in_dll(L.lib(), "_ZN2sv13g_skinny_tuneE")
    rng = np.random.default_rng(rt * 100 + waves * 10 + nch + n + 1000 * splits)
    m = 256 * rt
    per_split = waves * nch
    k = 256 * (per_split * (splits - 1) + per_split - (nch > 1))  # the last split's last chunk is past k when nch > 1
    ws = K.Workspace(8 << 20)
    try:
        tune[0], tune[1], tune[2], tune[3], tune[4] = rt, waves, nch, 3, splits
        for fmt in ("i8", "bf16"):
            if fmt == "bf16" and rt * nch > 2:
                continue
            w = torch.from_numpy(rng.normal(0, 0.02, (m, k)).astype(np.float32))
            if fmt == "i8":
                q, s = quantize_rows(w)
                host_w, host_s, gs = q.numpy(), s.view(torch.int16).numpy().view(np.uint16), 31
                mat = K.matrix(q.cuda(), s.cuda(), 31)
                epi, flags = L.EPI_NORM, L.FLAG_WRITE_INV
            else:
                host_w, host_s, gs = bf16_bits(w.numpy()), None, 0
                mat = K.matrix(u16_dev_bf16(host_w))
                epi, flags = L.EPI_RESID, 0
            x = (rng.normal(0, 1, (n, k)) * rng.uniform(0.5, 4, (n, 1))).astype(np.float32)
            base = rng.normal(0, 1, (n, m)).astype(np.float32)
            a = L.MatArgs(n, k, m, epi, flags, m, 0.75, 0.9, 1.3, 1, k, gs)
            aux_ref = np.zeros(n, np.float32)
            ref = oracle.matmul(L, host_w, host_s, gs, x, a, base=base if epi == L.EPI_RESID else None, aux=aux_ref)
            for layout in (mat, mat.tiled()):
                y = torch.zeros(n, m, device="cuda")
                aux = torch.zeros(n, device="cuda")
                K.matmul(layout, to_dev(x), y, n=n, epi=epi, flags=flags, scale=0.75, ra=0.9, rb=1.3,
                         base=to_dev(base) if epi == L.EPI_RESID else None, aux=aux, ws=ws)
                torch.cuda.synchronize()
                assert C.c_int.in_dll(L.lib(), "_ZN2sv12g_mm_variantE").value == 3, "one-shot kernel not launched"
                close(y.cpu().numpy(), ref, atol=5e-5 * max(float(np.abs(ref).max()), 1.0), rtol=1e-4,
                      what=f"{fmt} tiled={layout is not mat}")
                if epi == L.EPI_NORM:
                    close(aux.cpu().numpy(), aux_ref, atol=1e-5, rtol=1e-4, what="inv")
    finally:
        tune[0] = tune[1] = tune[2] = tune[3] = tune[4] = 0


# ---------------------------------------------------------------------------- attention
def make_attn_case(sh: ModelShape, runs_T, p0s, *, seed=0, tree=False, page_shift=4, shuffle=True, fast_kv=False):
    rng = np.random.default_rng(seed)
    D, NQ, NKV = sh.head_dim, sh.n_heads, sh.n_kv_heads
    W = (NQ + 2 * NKV) * D
    n = sum(runs_T)
    page = 1 << page_shift
    max_len = max(p + t for p, t in zip(p0s, runs_T))
    max_pages = -(-max_len // page)
    n_runs = len(runs_T)
    n_pages = n_runs * max_pages + 3
    perm = rng.permutation(n_pages) if shuffle else np.arange(n_pages)
    page_table = perm[: n_runs * max_pages].reshape(n_runs, max_pages).astype(np.uint32)
    if fast_kv:  # long contexts: random bf16 of magnitude [2^-7, 2) and random sign, drawn as bits
        def kv_bits():
            size = (1, n_pages, NKV, page, D)
            return (rng.integers(0x3C00, 0x4000, size, dtype=np.uint16) |
                    (rng.integers(0, 2, size, dtype=np.uint16) << np.uint16(15)))
        k_cache, v_cache = kv_bits(), kv_bits()
    else:
        k_cache = bf16_bits(rng.normal(0, 1, (1, n_pages, NKV, page, D)).astype(np.float32))
        v_cache = bf16_bits(rng.normal(0, 1, (1, n_pages, NKV, page, D)).astype(np.float32))
    qkv = (rng.normal(0, 1, (n, W)) * rng.uniform(0.2, 3, (n, 1))).astype(np.float32)
    meta = np.zeros((n, 2), np.uint32)
    vis = np.zeros(n, np.uint32)
    runs = np.zeros((n_runs, 2), np.uint32)
    t = 0
    for r, (T, p0) in enumerate(zip(runs_T, p0s)):
        runs[r] = (t, T)
        if tree:
            # a random tree over the run's rows: parent of row i is a random earlier row
            parent = [None] + [int(rng.integers(0, i)) for i in range(1, T)]
            depth = [0] * T
            sees = [1] * T
            for i in range(1, T):
                depth[i] = depth[parent[i]] + 1
                sees[i] = sees[parent[i]] | (1 << i)
        else:
            depth = list(range(T))
            sees = [(2 << i) - 1 for i in range(T)]
        for i in range(T):
            meta[t + i] = (r, p0 + depth[i])
            vis[t + i] = sees[i]
        t += T
    return dict(qkv=qkv, meta=meta, vis=vis, runs=runs, k=k_cache, v=v_cache, page_table=page_table,
                n_pages=n_pages, max_pages=max_pages, page_shift=page_shift)


ATTN_CASES = [
    # (run lengths, first positions, split, tree)
    ([5], [512], 128, False),            # config 0's run
    ([5], [8192], 256, False),           # config 1's run
    ([1], [0], 32, False),               # no cached keys
    ([3, 5, 2], [31, 100, 64], 32, False),
    ([16], [300], 64, True),             # a 16-row draft tree
    ([16, 9, 1], [33, 1000, 17], 96, True),
    ([5], [8192], 384, False),           # config 1's split: three batches per wave
    ([5, 4], [1000, 2047], 512, False),  # four batches per wave, a partial last split
    ([2], [700], 160, False),            # five batches: waves with one and two
    ([5, 1, 3, 5, 2, 4], [4000, 0, 17, 9000, 1, 2500], 256, False),  # empty and one-key contexts among long ones
    ([4] * 40, [37 * i for i in range(40)], 128, False),              # 40 runs (not inline), short contexts
]


@pytest.mark.parametrize("runs_T,p0s,split,tree", ATTN_CASES)
@pytest.mark.parametrize("rope", [1, 0])
@pytest.mark.parametrize("allin", [1, 0])
def test_attn_verify(gpu, runs_T, p0s, split, tree, rope, allin):
    """Both cached-key variants (all of a wave's batches in flight, where built: up to 32
    columns per kv head and 512 keys per split; one batch ahead) against the oracle."""
    banner(f"attn runs={runs_T} p0={p0s} split={split} tree={tree} rope={rope} allin={allin}")
    sel = C.c_int.in_dll(L.lib(), "_ZN2sv12g_attn_allinE")
    sel.value = allin
    try:
        _attn_verify_case(runs_T, p0s, split, tree, rope)
    finally:
        sel.value = -1


@pytest.mark.parametrize("runs_T,p0s,split,tree", [([5], [8192], 384, False), ([5], [8192], 256, False),
                                                   ([5, 4], [1000, 2047], 512, False), ([16], [300], 64, True),
                                                   ([3, 5, 2], [31, 100, 64], 32, False),
                                                   ([4] * 40, [37 * i for i in range(40)], 128, False)])
@pytest.mark.parametrize("allin", [1, 0])
def test_attn_fused_merge_bit_identical(gpu, runs_T, p0s, split, tree, allin):
    """The merge by the last split to arrive (attention launch only) adds the splits' partials
    in attn_merge_kernel's order (P parts of every P-th split from zero, then the parts in
    order), so both merges give the same bits: configs[1]'s run (23 splits: four parts; at 33
    splits, eight parts, the separate merge runs), ragged runs, a draft tree, 40 runs read from
    memory; both cached-key variants. The second fused call shares the workspace, so it also
    finds the counters back at zero (graph replays rely on it)."""
    banner(f"attn fused merge runs={runs_T} p0={p0s} split={split} tree={tree} allin={allin}")
    sh = SH
    c = make_attn_case(sh, runs_T, p0s, seed=len(runs_T) * 17 + split, tree=tree)
    freq = oracle.np.asarray((500000.0 ** (-2.0 * np.arange(32) / 64)), np.float32)
    rope_tab = to_dev(oracle.rope_table(freq, max(p0s) + 20))
    kv = L.KvArgs(1, 0, 0, len(runs_T), c["page_shift"], c["n_pages"], c["max_pages"], 0)
    max_splits = max(-(-p // split) + 1 for p in p0s)
    args = L.AttnArgs(split, max_splits, sh.head_dim ** -0.5 * 1.4426950408889634, 1, 0, 0, 0, 0, 0)
    runs = to_dev(c["runs"].reshape(-1).copy())
    qkv, meta, vis, pt = to_dev(c["qkv"]), to_dev(c["meta"]), to_dev(c["vis"]), to_dev(c["page_table"])
    kd, vd = to_dev(c["k"]), to_dev(c["v"])
    sel = C.c_int.in_dll(L.lib(), "_ZN2sv12g_attn_allinE")
    fused = C.c_bool.in_dll(L.lib(), "_ZN2sv18g_attn_fused_mergeE")
    outs = []
    ws = K.Workspace(64 << 20)
    assert L.lib().sv_attn_workspace_bytes(C.byref(sh.c()), len(runs_T), max_splits, max(runs_T)) <= ws.nbytes
    try:
        sel.value = allin
        for f in (False, True, True):
            fused.value = f
            out = torch.full((sum(runs_T), sh.n_heads * sh.head_dim), 7.0, device="cuda")
            K.attn_verify(sh, qkv, meta, kd, vd, pt, rope_tab, kv, args, runs, len(runs_T), max(runs_T), vis, out, ws=ws)
            torch.cuda.synchronize()
            outs.append(out.cpu().numpy())
    finally:
        fused.value = False
        sel.value = -1
    assert np.isfinite(outs[0]).all()
    for i in (1, 2):
        assert np.array_equal(outs[0].view(np.uint32), outs[i].view(np.uint32)), f"fused merge call {i} differs"


@pytest.mark.parametrize("runs_T,p0s,split", [([5], [65536], 1152), ([5] * 8, [65536] * 8, 3584)])
def test_attn_verify_long_context(gpu, runs_T, p0s, split):
    """configs[3]'s attention: 65536 cached keys per stream (1 stream with 1152-key splits, 8
    streams with 3584-key splits, the engine's choices there), rope on, shuffled pages, the
    variant the launch picks by shape."""
    banner(f"attn long context runs={runs_T} split={split}")
    _attn_verify_case(runs_T, p0s, split, False, 1, fast_kv=True)


def _attn_verify_case(runs_T, p0s, split, tree, rope, sh=SH, fast_kv=False):
    c = make_attn_case(sh, runs_T, p0s, seed=len(runs_T) * 31 + split, tree=tree, fast_kv=fast_kv)
    freq = oracle.np.asarray((500000.0 ** (-2.0 * np.arange(32) / 64)), np.float32)
    rope_tab = oracle.rope_table(freq, max(p0s) + 20)
    kv = L.KvArgs(1, 0, 0, len(runs_T), c["page_shift"], c["n_pages"], c["max_pages"], 0)
    max_splits = max(-(-p // split) + 1 for p in p0s)
    args = L.AttnArgs(split, max_splits, sh.head_dim ** -0.5 * 1.4426950408889634, rope, 0, 0, 0, 0, 0)
    runs_flat = c["runs"].reshape(-1).copy()
    k_ref, v_ref = c["k"].copy(), c["v"].copy()
    ref = oracle.attn_verify(L, sh, c["qkv"], c["meta"].reshape(-1).copy(), k_ref, v_ref, c["page_table"], rope_tab,
                             kv, args, runs_flat, c["vis"])
    kd, vd = to_dev(c["k"]), to_dev(c["v"])
    out = torch.zeros(sum(runs_T), sh.n_heads * sh.head_dim, device="cuda")
    K.attn_verify(sh, to_dev(c["qkv"]), to_dev(c["meta"]), kd, vd, to_dev(c["page_table"]), to_dev(rope_tab), kv,
                  args, to_dev(runs_flat), len(runs_T), max(runs_T), to_dev(c["vis"]), out)
    torch.cuda.synchronize()
    close(out.cpu().numpy(), ref, atol=2e-4, rtol=2e-4, what="attention output")
    # The new keys/values in the cache: V bit-exact (a rounding of the same fp32), K within one
    # bf16 step (normed and roped in fp32 here, in double in the oracle).
    kg, vg = kd.cpu().numpy(), vd.cpu().numpy()
    assert np.array_equal(vg, v_ref), "V cache differs"
    dk = np.abs(oracle.bf16_to_f32(kg) - oracle.bf16_to_f32(k_ref))
    assert (dk <= 2 ** -7 * np.abs(oracle.bf16_to_f32(k_ref)) + 1e-30).all(), "K cache off by more than one step"


SH128 = ModelShape(n_layers=2, n_heads=16, n_kv_heads=4, head_dim=128)


@pytest.mark.parametrize("runs_T,p0s,split,tree", [([5], [700], 128, False), ([3, 5, 2], [31, 100, 64], 32, False),
                                                   ([16], [300], 64, True)])
@pytest.mark.parametrize("rope", [1, 0])
def test_attn_verify_head_dim_128(gpu, runs_T, p0s, split, tree, rope):
    """The head_dim 128 instantiations (16 query heads over 4 kv heads: 4 to 64 columns per kv
    head; RoPE on dims 0..63 only, as the table has 32 pairs) against the oracle."""
    banner(f"attn D=128 runs={runs_T} p0={p0s} split={split} tree={tree} rope={rope}")
    _attn_verify_case(runs_T, p0s, split, tree, rope, sh=SH128)


# ------------------------------------------------------------------------------ sampler
def sample_rows(n, temps, top_ps, seed=11, pos0=100):
    rows = []
    for r in range(n):
        s = seed * 7919 + r
        rows.append(L.SampleRow(s & 0xFFFFFFFF, (s >> 32) & 0xFFFFFFFF, pos0 + r, float(temps[r % len(temps)]),
                                float(top_ps[r % len(top_ps)]), L.NO_TOK))
    return rows


@pytest.mark.parametrize("runs_T,p0s,split,tree", [([5], [515], 128, False), ([3, 5, 2], [31, 100, 64], 32, False),
                                                   ([16], [300], 64, True)])
def test_attn_verify_garbage_past_context(gpu, runs_T, p0s, split, tree):
    """Cache slots past each run's context (the rest of its last page, and never-used pages) hold
    NaN bit patterns, as a caller's uninitialised cache may: keys there are read inside their
    page but masked, their V rows zeroed, so the output is finite and matches the oracle."""
    banner(f"attn garbage runs={runs_T} p0={p0s} split={split} tree={tree}")
    sh = SH
    c = make_attn_case(sh, runs_T, p0s, seed=len(runs_T) * 7 + split, tree=tree)
    page = 1 << c["page_shift"]
    nan = np.uint16(0x7FC0)
    used = set()
    for r, p0 in enumerate(p0s):
        for pos in range(c["max_pages"] * page):
            pg = int(c["page_table"][r, pos // page])
            if pos < p0:
                used.add(pg)
            else:
                c["k"][0, pg, :, pos % page, :] = nan
                c["v"][0, pg, :, pos % page, :] = nan
    for pg in range(c["n_pages"]):
        if pg not in used and pg not in set(c["page_table"].reshape(-1).tolist()):
            c["k"][0, pg] = nan
            c["v"][0, pg] = nan
    freq = oracle.np.asarray((500000.0 ** (-2.0 * np.arange(32) / 64)), np.float32)
    rope_tab = oracle.rope_table(freq, max(p0s) + 20)
    kv = L.KvArgs(1, 0, 0, len(runs_T), c["page_shift"], c["n_pages"], c["max_pages"], 0)
    max_splits = max(-(-p // split) + 1 for p in p0s)
    args = L.AttnArgs(split, max_splits, 0.125 * 1.4426950408889634, 1, 0, 0, 0, 0, 0)
    runs_flat = c["runs"].reshape(-1).copy()
    ref = oracle.attn_verify(L, sh, c["qkv"], c["meta"].reshape(-1).copy(), c["k"].copy(), c["v"].copy(),
                             c["page_table"], rope_tab, kv, args, runs_flat, c["vis"])
    assert np.all(np.isfinite(ref))
    out = torch.zeros(sum(runs_T), sh.n_heads * sh.head_dim, device="cuda")
    K.attn_verify(sh, to_dev(c["qkv"]), to_dev(c["meta"]), to_dev(c["k"]), to_dev(c["v"]), to_dev(c["page_table"]),
                  to_dev(rope_tab), kv, args, to_dev(runs_flat), len(runs_T), max(runs_T), to_dev(c["vis"]), out)
    torch.cuda.synchronize()
    close(out.cpu().numpy(), ref, atol=2e-4, rtol=2e-4, what="attention output over garbage")


@pytest.mark.parametrize("vocab", [32000, 257, 1024, 151680])
def test_sample_bit_exact(gpu, vocab):
    banner(f"sample vocab={vocab}")
    rng = np.random.default_rng(vocab)
    n = 24
    logits = (rng.normal(15.4, 0.6, (n, vocab))).astype(np.float32)
    logits[3, :] = 7.0                       # all ties: lowest id wins at T = 0
    logits[4, rng.integers(0, vocab, 5)] = logits[4].max() + 0.5  # tied maxima
    logits[5, vocab // 2:] = -np.inf         # masked tail (vocab_real)
    temps = [0.0, 0.7, 1.0, 0.6, 1.5, 0.3]
    top_ps = [1.0, 1.0, 0.95, 0.9, 0.5, 0.99, 0.7, 1.0]
    rows = sample_rows(n, temps, top_ps)
    ref = oracle.sample(L, logits, rows)
    d_rows = torch.from_numpy(np.frombuffer(bytes((L.SampleRow * n)(*rows)), np.uint8).copy()).cuda()
    out = torch.zeros(n, dtype=torch.int32, device="cuda")
    K.sample(to_dev(logits), d_rows, out, None, n, vocab)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32)
    assert np.array_equal(got, ref), f"ids differ at rows {np.nonzero(got != ref)[0]}"


# --------------------------------------------------------------- accept / compact / replay
def random_runs(rng, n_runs, max_count=16):
    """Random verify runs over random trees, with sampled tokens that match some drafts."""
    runs, tokens, tree, out = [], [], np.zeros(n_runs * 16, np.uint32), []
    first = head0 = 0
    for r in range(n_runs):
        count = int(rng.integers(1, max_count + 1))
        verify = int(count > 1 or rng.integers(0, 2))
        parent = [0xFF] + [int(rng.integers(0, i)) for i in range(1, count)]
        depth = [0] * count
        sees = [1] * count
        for i in range(1, count):
            depth[i] = depth[parent[i]] + 1
            sees[i] = sees[parent[i]] | (1 << i)
        for i in range(count):
            tree[r * 16 + i] = depth[i] | (parent[i] << 8) | (sees[i] << 16)
        toks = [int(x) for x in rng.integers(0, 6, count)]
        samp = [int(x) for x in rng.integers(0, 6, count)]
        nhead = count if verify else int(rng.integers(0, 2))
        runs.append(L.RunIn(r, first, count, head0, nhead, verify))
        tokens += toks
        out += samp[:nhead]
        first += count
        head0 += nhead
    return runs, np.array(tokens, np.uint32), tree, np.array(out, np.uint32)


@pytest.mark.parametrize("seed", range(6))
def test_accept_compact_bit_exact(gpu, seed):
    banner(f"accept/compact seed={seed}")
    rng = np.random.default_rng(seed)
    n_runs = 12
    runs, tokens, tree, out = random_runs(rng, n_runs)
    lens = rng.integers(0, 40, n_runs).astype(np.uint32)
    feed = rng.integers(0, 100, n_runs * 16).astype(np.uint32)
    gen = []
    for r in range(n_runs):
        g = L.GenState()
        g.remaining = int(rng.choice([0xFFFFFFFF, 1, 2, 3, 10]))
        g.done = int(rng.random() < 0.15)
        g.nstop = int(rng.integers(0, 3))
        for j in range(g.nstop):
            g.stop[j] = int(rng.integers(0, 6))
        gen.append(g)
    n_tok = len(tokens)
    o_out, o_lens, o_feed, o_gen, o_em, o_path, o_plen, o_on = oracle.accept(L, runs, tokens, out, lens, feed, gen,
                                                                             tree, n_tok)
    d_runs = torch.from_numpy(np.frombuffer(bytes((L.RunIn * n_runs)(*runs)), np.uint8).copy()).cuda()
    d_gen = torch.from_numpy(np.frombuffer(bytes((L.GenState * n_runs)(*gen)), np.uint8).copy()).cuda()
    d_out, d_lens, d_feed = to_dev(out.copy()), to_dev(lens.copy()), to_dev(feed.copy())
    d_em = torch.zeros(n_runs, dtype=torch.int32, device="cuda")
    d_path = torch.zeros(n_runs * 16, dtype=torch.int32, device="cuda")
    d_plen = torch.zeros(n_runs, dtype=torch.int32, device="cuda")
    d_on = torch.zeros(max(1, n_tok), dtype=torch.int32, device="cuda")
    K.accept(d_runs, to_dev(tokens), d_out, d_lens, d_feed, d_gen, d_em, n_runs, to_dev(tree), d_path, d_plen, d_on)
    torch.cuda.synchronize()
    u = lambda t: t.cpu().numpy().view(np.uint32)  # noqa: E731
    assert np.array_equal(u(d_out), o_out)
    assert np.array_equal(u(d_lens), o_lens)
    assert np.array_equal(u(d_feed), o_feed)
    assert np.array_equal(u(d_em), o_em)
    assert np.array_equal(u(d_path), o_path)
    assert np.array_equal(u(d_plen), o_plen)
    assert np.array_equal(u(d_on)[:n_tok], o_on[:n_tok])
    assert bytes(d_gen.cpu().numpy()) == bytes((L.GenState * n_runs)(*o_gen))

    # kv_compact on the accepted paths (2 layers, shuffled pages).
    sh = ModelShape(n_layers=2)
    page_shift, page = 4, 16
    max_pages = 8
    n_pages = n_runs * max_pages
    perm = rng.permutation(n_pages).astype(np.uint32).reshape(n_runs, max_pages)
    kc = rng.integers(0, 65535, (2, n_pages, sh.n_kv_heads, page, sh.head_dim)).astype(np.uint16)
    vc = rng.integers(0, 65535, kc.shape).astype(np.uint16)
    kv = L.KvArgs(1, 0, 0, n_runs, page_shift, n_pages, max_pages, 0)
    k_ref, v_ref = kc.copy(), vc.copy()
    oracle.kv_compact(L, sh, runs, o_path, o_plen, o_lens, k_ref, v_ref, perm, kv)
    kd, vd = to_dev(kc), to_dev(vc)
    K.kv_compact(sh, d_runs, n_runs, d_path, d_plen, d_lens, kd, vd, to_dev(perm), kv)
    torch.cuda.synchronize()
    assert np.array_equal(kd.cpu().numpy(), k_ref)
    assert np.array_equal(vd.cpu().numpy(), v_ref)

    # replay drafter after accept
    stride = 64
    trace = rng.integers(0, 1000, n_runs * stride).astype(np.uint32)
    trace_len = rng.integers(0, stride, n_runs).astype(np.uint32)
    ra = L.ReplayArgs(stride, 77, 0.35, 1000)
    f_ref, t_ref = o_feed.copy(), tree.copy()
    oracle.replay_draft(L, runs, o_lens, f_ref, trace, trace_len, ra, t_ref)
    d_tree = to_dev(tree.copy())
    K.replay_draft(d_runs, n_runs, d_lens, d_feed, to_dev(trace), to_dev(trace_len), ra, d_tree)
    torch.cuda.synchronize()
    assert np.array_equal(u(d_feed), f_ref)
    assert np.array_equal(u(d_tree), t_ref)


def test_embed(gpu):
    banner("embed")
    rng = np.random.default_rng(5)
    sh = ModelShape(vocab=1000, n_layers=1)
    table = bf16_bits(rng.normal(0, 0.02, (sh.vocab, sh.hidden)).astype(np.float32))
    tokens = np.array([5, L.FEED_ROW + 0, L.FEED_ROW + 2, L.FEED_ROW + 1, 999], np.uint32)
    tin = np.array([[0, 0], [1, 0], [1, 1], [1, 2], [2, 0]], np.uint32)
    lens = np.array([10, 20, 30], np.uint32)
    feed = rng.integers(0, 1000, 3 * 16).astype(np.uint32)
    tree = np.array([(i % 16) | ((i % 16 + 3) << 8) | ((i * 37 % 65536) << 16) for i in range(48)], np.uint32)
    vis = np.array([1, 1, 3, 7, 1], np.uint32)
    o_tok, o_out, o_meta, o_vis = oracle.embed(L, sh, table, tokens, tin, lens, feed, tree, vis)
    d_tok, d_vis = to_dev(tokens.copy()), to_dev(vis.copy())
    d_out = torch.zeros(5, sh.hidden, device="cuda")
    d_meta = torch.zeros(10, dtype=torch.int32, device="cuda")
    K.embed(sh, u16_dev_bf16(table), d_tok, d_out, to_dev(tin), d_meta, to_dev(lens), to_dev(feed), to_dev(tree),
            d_vis, 5)
    torch.cuda.synchronize()
    assert np.array_equal(d_tok.cpu().numpy().view(np.uint32), o_tok)
    assert np.array_equal(d_meta.cpu().numpy().view(np.uint32), o_meta.reshape(-1))
    assert np.array_equal(d_vis.cpu().numpy().view(np.uint32), o_vis)
    close(d_out.cpu().numpy(), o_out, atol=1e-5, rtol=1e-5, what="embed rows")


# --------------------------------------------------------------------- matmul, large n
GEMM_CASES = [
    # (m, k, fmt, group)  group None: one scale per row
    (16384, 2048, "i8", None),  # gate_up at 32 streams
    (2048, 8192, "i8", None),   # down
    (3072, 2048, "i8", None),   # qkv (256-row blocks of the 32-wide kernel)
    (3072, 2048, "i8", 64),     # int8 groups of 64 (the reference's default)
    (1280, 1280, "i8", 128),    # 20 chunks of 64 in 4 k splits: groups straddle splits
    (2048, 2048, "bf16", None),
]


@pytest.mark.parametrize("m,k,fmt,group", GEMM_CASES)
@pytest.mark.parametrize("n", [17, 40, 100, 160, 512])
@pytest.mark.parametrize("epi", [L.EPI_NORM, L.EPI_RESID, L.EPI_SWIGLU, L.EPI_HEAD])
def test_matmul_many_rows(gpu, m, k, fmt, group, n, epi):
    banner(f"gemm m={m} k={k} {fmt} group={group} n={n} epi={epi}")
    rng = np.random.default_rng(17 * n + epi)
    w = rng.normal(0, 0.02, (m, k)).astype(np.float32)
    if fmt == "i8":
        if group is None:
            q, s = quantize_rows(torch.from_numpy(w))
            wq, sc, gs = q.numpy(), s.view(torch.int16).numpy().view(np.uint16), 31
        else:
            wq, sc = oracle.quantize(w, group)
            gs = int(np.log2(group))
        mat = K.matrix(torch.from_numpy(wq).cuda(), torch.from_numpy(sc.view(np.int16)).cuda().view(torch.bfloat16), gs)
        host_w, host_s = wq, sc
    else:
        wb = bf16_bits(w)
        mat = K.matrix(u16_dev_bf16(wb))
        host_w, host_s, gs = wb, None, 0
    x = (rng.normal(0, 1, (n, k)) * rng.uniform(0.5, 4, (n, 1))).astype(np.float32)
    base = rng.normal(0, 1, (n, m)).astype(np.float32)
    flags = {L.EPI_NORM: L.FLAG_WRITE_INV, L.EPI_RESID: L.FLAG_WRITE_RAW, L.EPI_HEAD: L.FLAG_NORM_IN}.get(epi, 0)
    a = L.MatArgs(n, k, m, epi, flags, m - 3, 0.8, 1.1, 0.7, 1, k, gs)
    out_m = m // 2 if epi == L.EPI_SWIGLU else m
    aux_n = n if epi == L.EPI_NORM else n * m
    # The GPU computes every row; at the largest matrices the oracle checks a seeded sample of
    # 48 rows (each output row depends on its input row alone), so gate_up and down at 512 rows
    # run in the launch shape the engine uses for configs[4].
    rows = np.sort(rng.choice(n, 48, replace=False)).astype(np.uint32) if m * k * n > 2048 * 8192 * 160 else None
    nr = n if rows is None else len(rows)
    a_ref = L.MatArgs(nr, k, m, epi, flags, m - 3, 0.8, 1.1, 0.7, 1, k, gs)
    aux_ref = np.zeros(nr if epi == L.EPI_NORM else nr * m, np.float32)
    ref = oracle.matmul(L, host_w, host_s, gs, x, a_ref, x_rows=rows, aux=aux_ref,
                        base=(base if rows is None else np.ascontiguousarray(base[rows])) if epi == L.EPI_RESID else None)
    y = torch.zeros(n, out_m, device="cuda")
    aux = torch.zeros(aux_n, device="cuda")
    K.matmul(mat, to_dev(x), y, n=n, epi=epi, flags=flags, scale=0.8, ra=1.1, rb=0.7,
             base=to_dev(base) if epi == L.EPI_RESID else None, aux=aux, vocab_real=m - 3)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    got_aux = aux.cpu().numpy()
    if rows is not None:
        got = got[rows]
        got_aux = got_aux[rows] if epi == L.EPI_NORM else got_aux.reshape(n, m)[rows].reshape(-1)
    mag = float(np.abs(ref[np.isfinite(ref)]).max())
    close(got, ref, atol=5e-5 * max(mag, 1.0), rtol=1e-4, what=f"gemm epi {epi}")
    if epi in (L.EPI_NORM, L.EPI_RESID):
        close(got_aux, aux_ref, atol=1e-5 * max(1.0, np.abs(aux_ref).max()), rtol=1e-4, what="aux")


def test_matmul_head_many_cells(gpu):
    """The reference model's head at 32 sequences x 8 rows: 151680 rows x 1280 in int8 groups
    of 64 at n = 256 (the GEMM's k-split cells, rows blocks x token blocks, past 16384),
    softcapped with the norm folded in; a seeded sample of 8 rows against the oracle."""
    m, k, n = 151680, 1280, 256
    banner(f"gemm head m={m} k={k} n={n}")
    rng = np.random.default_rng(5)
    w = rng.normal(0, 0.02, (m, k)).astype(np.float32)
    wq, sc = oracle.quantize(w, 64)
    mat = K.matrix(torch.from_numpy(wq).cuda(), torch.from_numpy(sc.view(np.int16)).cuda().view(torch.bfloat16), 6)
    x = rng.normal(0, 1, (n, k)).astype(np.float32)
    rows = np.sort(rng.choice(n, 8, replace=False)).astype(np.uint32)
    a_ref = L.MatArgs(len(rows), k, m, L.EPI_HEAD, L.FLAG_NORM_IN, m - 13, 1.0, 0.0, 0.0, 1, k, 6)
    ref = oracle.matmul(L, wq, sc, 6, x, a_ref, x_rows=rows)
    y = torch.zeros(n, m, device="cuda")
    ws = K.Workspace(L.lib().sv_matmul_workspace_bytes(n, m, k))
    K.matmul(mat, to_dev(x), y, n=n, epi=L.EPI_HEAD, flags=L.FLAG_NORM_IN, vocab_real=m - 13, ws=ws)
    torch.cuda.synchronize()
    got = y.cpu().numpy()[rows]
    close(got, ref, atol=5e-5 * 23, rtol=1e-4, what="head at 256 rows")


@pytest.mark.parametrize("shape", [(1, 2, 1, 4), (2, 2, 2, 4), (2, 2, 4, 8), (1, 3, 2, 8), (2, 3, 1, 4),
                                                  (2, 4, 2, 4), (1, 5, 4, 4), (2, 5, 1, 4), (2, 8, 2, 4), (1, 8, 1, 4),
                                                  (4, 4, 1, 4), (4, 2, 2, 4), (4, 5, 4, 4), (4, 4, 2, 2), (4, 3, 1, 2),
                                                  (4, 2, 4, 2), (4, 2, 1, 2), (2, 2, 4, 2), (1, 2, 2, 2), (2, 5, 1, 2),
                                                  (2, 2, 8, 2), (1, 2, 8, 2), (4, 2, 8, 2),
                                                  # 32 x 32 x 16 tiles (the fifth field: tile width)
                                                  (1, 1, 1, 2, 32), (1, 1, 2, 2, 32), (2, 1, 4, 2, 32), (1, 2, 1, 4, 32),
                                                  (2, 2, 2, 2, 32), (1, 3, 8, 2, 32), (2, 3, 1, 4, 32), (1, 1, 8, 4, 32),
                                                  # eight waves (the sixth field)
                                                  (1, 1, 2, 2, 32, 8), (1, 2, 1, 2, 32, 8), (2, 1, 4, 4, 32, 8),
                                                  (1, 3, 8, 2, 32, 8),
                                                  # two chunks per barrier (the seventh field)
                                                  (1, 1, 2, 4, 32, 8, 2), (2, 1, 1, 4, 32, 4, 2), (1, 2, 8, 4, 32, 8, 2)])
@pytest.mark.parametrize("n", [17, 100, 170])
def test_matmul_gemm_launch_shapes(gpu, shape, n):
    """Every GEMM launch shape (row tiles per wave, token tiles, k splits merged by the last
    split to arrive, chunks in flight) gives the oracle's result: int8 with EPI_NORM (sums of
    squares carried across splits, the inverse norm written once) and bf16 with EPI_RESID in
    the tiled layout, with a row gather, ragged token blocks (17, 100 rows) and a k whose chunk
    count leaves a partial round of zero chunks (k = 1280: 20 chunks; 2560 = 40 chunks for eight
    splits, five each); two calls share one workspace. The shape is forced through the
    library's internal override: 16-wide tiles (mm_gemm) and 32-wide tiles (mm_gemm32) with 4
    or 8 waves and one or two chunks per barrier."""
    rtw, nt, splits, depth, mf, nw, cpi = (tuple(shape) + (16, 4, 1)[len(shape) - 4:])[:7]
    banner(f"gemm launch shape rtw={rtw} nt={nt} splits={splits} depth={depth} tile={mf} waves={nw} "
           f"chunks per barrier={cpi} n={n}")
    tune = (C.c_int * 7).in_dll(L.lib(), "_ZN2sv11g_gemm_tuneE")
    rng = np.random.default_rng(rtw * 1000 + nt * 100 + splits * 10 + depth + n)
    m, k = ({1: 384, 2: 512, 4: 768} if nw == 4 else {1: 512, 2: 1024})[rtw], (2560 if splits == 8 else 1280)
    ws = K.Workspace(16 << 20)
    try:
        tune[0], tune[1], tune[2], tune[3], tune[4], tune[5], tune[6] = rtw, nt, splits, depth, mf, nw, cpi
        w = torch.from_numpy(rng.normal(0, 0.02, (m, k)).astype(np.float32))
        q, s = quantize_rows(w)
        mi8 = K.matrix(q.cuda(), s.cuda(), 31)
        wb = bf16_bits(w.numpy())
        mbf = K.matrix(u16_dev_bf16(wb)).tiled()
        for call in range(2):
            x = (rng.normal(0, 1, (n + 3, k)) * rng.uniform(0.5, 4, (n + 3, 1))).astype(np.float32)
            rows = rng.permutation(n + 3)[:n].astype(np.uint32)
            # int8, EPI_NORM, gathered rows
            a = L.MatArgs(n, k, m, L.EPI_NORM, L.FLAG_WRITE_INV, m, 0.75, 0, 0, 1, k, 31)
            aux_ref = np.zeros(n, np.float32)
            ref = oracle.matmul(L, q.numpy(), s.view(torch.int16).numpy().view(np.uint16), 31, x, a, aux=aux_ref,
                                x_rows=rows)
            y = torch.zeros(n, m, device="cuda")
            aux = torch.zeros(n, device="cuda")
            K.matmul(mi8, to_dev(x), y, n=n, epi=L.EPI_NORM, flags=L.FLAG_WRITE_INV, scale=0.75, aux=aux,
                     x_rows=to_dev(rows), ws=ws)
            torch.cuda.synchronize()
            assert C.c_int.in_dll(L.lib(), "_ZN2sv12g_mm_variantE").value == 2, "GEMM kernel not launched"
            close(y.cpu().numpy(), ref, atol=5e-5 * max(float(np.abs(ref).max()), 1.0), rtol=1e-4,
                  what=f"int8 call {call}")
            close(aux.cpu().numpy(), aux_ref, atol=1e-5, rtol=1e-4, what="inv")
            # bf16 tiled, EPI_RESID
            base = rng.normal(0, 1, (n, m)).astype(np.float32)
            xr = x[:n].copy()
            a = L.MatArgs(n, k, m, L.EPI_RESID, 0, m, 0.5, 1.1, 0.7, 1, k, 0)
            ref = oracle.matmul(L, wb, None, 0, xr, a, base=base)
            y = torch.zeros(n, m, device="cuda")
            K.matmul(mbf, to_dev(xr), y, n=n, epi=L.EPI_RESID, scale=0.5, ra=1.1, rb=0.7, base=to_dev(base), ws=ws)
            torch.cuda.synchronize()
            close(y.cpu().numpy(), ref, atol=5e-5 * max(float(np.abs(ref).max()), 1.0), rtol=1e-4,
                  what=f"bf16 call {call}")
    finally:
        tune[0] = tune[1] = tune[2] = tune[3] = tune[4] = tune[5] = tune[6] = 0


def test_matmul_skinny_groups_of_256(gpu):
    """int8 with groups of 256 on the skinny path (one scale per k chunk)."""
    banner("skinny group 256")
    rng = np.random.default_rng(8)
    m, k, n = 512, 2048, 5
    w = rng.normal(0, 0.02, (m, k)).astype(np.float32)
    wq, sc = oracle.quantize(w, 256)
    mat = K.matrix(torch.from_numpy(wq).cuda(), torch.from_numpy(sc.view(np.int16)).cuda().view(torch.bfloat16), 8)
    x = rng.normal(0, 1, (n, k)).astype(np.float32)
    a = L.MatArgs(n, k, m, L.EPI_RAW, 0, m, 1.0, 0, 0, 1, k, 8)
    ref = oracle.matmul(L, wq, sc, 8, x, a)
    y = torch.zeros(n, m, device="cuda")
    K.matmul(mat, to_dev(x), y, n=n, epi=L.EPI_RAW)
    torch.cuda.synchronize()
    close(y.cpu().numpy(), ref, atol=5e-5 * float(np.abs(ref).max()), rtol=1e-4, what="skinny grouped")


# ------------------------------------------------------------------- DDTree draft builder
def _draft_case(seed, block_rows, nv=16384):
    rng = np.random.default_rng(seed)
    slots = rng.permutation(16)[: len(block_rows)]
    blocks, tin = [], []
    for slot, rows in zip(slots, block_rows):
        blocks.append((len(tin), rows))
        tin += [(int(slot), i) for i in range(rows)]
    n = len(tin)
    logits = rng.normal(0, 3, (n, nv)).astype(np.float32)
    logits[1, rng.integers(0, nv, 3)] = logits[1].max() + 0.25  # tied maxima
    if n > 3:
        logits[3, :] = -np.inf                                    # no candidate at all
        logits[3, 7] = 2.0                                        # ... but one
    vocab = np.sort(rng.choice(151680, nv, replace=False)).astype(np.uint32)
    return (np.array(blocks, np.uint32), np.array(tin, np.uint32), logits, vocab,
            rng.integers(0, 1 << 30, 16 * 16).astype(np.uint32), rng.integers(0, 1 << 30, 16 * 16).astype(np.uint32))


@pytest.mark.parametrize("ncand", [1, 2, 3, 4])
@pytest.mark.parametrize("seed,block_rows", [(1, [5, 8, 1, 16]), (2, [8] * 12), (3, [2, 3, 4, 16, 7])])
def test_draft_builder_bit_exact(gpu, ncand, seed, block_rows):
    """draft_top then draft_tree (kernels.metal:1845-1934) on drafter logits over a 16384-id
    draft vocabulary: candidate ids, their probabilities (bit for bit: the same exp2 and
    summation order), and every slot's feed and tree entries equal the oracle's."""
    banner(f"draft builder ncand={ncand} blocks={block_rows}")
    blocks, tin, logits, vocab, feed0, tree0 = _draft_case(seed * 10 + ncand, block_rows)
    n, nv = logits.shape
    inv_t = 1.0 / 0.6
    cand_r, q_r = oracle.draft_top(logits, vocab, tin, inv_t, ncand)
    feed_r, tree_r = feed0.copy(), tree0.copy()
    oracle.draft_tree(blocks, tin, cand_r, q_r, feed_r, tree_r, ncand)
    cand = torch.zeros(n * 4, dtype=torch.int32, device="cuda")
    q = torch.zeros(n * 4, dtype=torch.float32, device="cuda")
    d_tin, d_blocks = to_dev(tin), to_dev(blocks)
    K.draft_top(to_dev(logits), to_dev(vocab), d_tin, cand, q, n, nv, inv_t, ncand)
    feed, tree = to_dev(feed0.view(np.int32)), to_dev(tree0.view(np.int32))
    K.draft_tree(d_blocks, len(blocks), d_tin, cand, q, feed, tree, ncand)
    torch.cuda.synchronize()
    drafted = tin[:, 1] > 0
    got_c = cand.cpu().numpy().view(np.uint32).reshape(n, 4)
    got_q = q.cpu().numpy().reshape(n, 4)
    assert np.array_equal(got_c[drafted, :ncand], cand_r[drafted, :ncand])
    assert np.array_equal(got_q[drafted, :ncand].view(np.uint32), q_r[drafted, :ncand].view(np.uint32))
    assert np.array_equal(feed.cpu().numpy().view(np.uint32), feed_r)
    assert np.array_equal(tree.cpu().numpy().view(np.uint32), tree_r)
    assert not (feed_r[feed_r != feed0] == L.NO_TOK).any(), "an unfilled candidate became a node"


# --------------------------------------------- int8 scale groups of 64 / 128 (1-16 rows)
@pytest.mark.parametrize("m,k,group", [(3072, 2048, 64), (2048, 8192, 64), (16384, 2048, 128), (2048, 2048, 64),
                                       (512, 1280, 128)])
@pytest.mark.parametrize("n", [1, 5, 16])
@pytest.mark.parametrize("epi", [L.EPI_NORM, L.EPI_RESID, L.EPI_SWIGLU])
@pytest.mark.parametrize("tiled", [False, True])
def test_matmul_int8_groups_one_shot(gpu, m, k, group, n, epi, tiled):
    """The reference's default int8 layer format (tools/convert.py:20: groups of 64 k; 128 as
    well) on the one-shot kernel at 1-16 rows: each group's products summed on their own and
    scaled, against the oracle's dequantised float64 matmul."""
    if k % 256:
        pytest.skip("the one-shot kernel takes k in chunks of 256")
    banner(f"int8 groups m={m} k={k} group={group} n={n} epi={epi} tiled={tiled}")
    rng = np.random.default_rng(m + k + group + 10 * n + epi)
    w = rng.normal(0, 0.02, (m, k)).astype(np.float32)
    w[:, :group] *= 40.0  # the first group of every row 40x larger: scales that differ a lot
    wq, sc = oracle.quantize(w, group)
    gs = int(np.log2(group))
    mat = K.matrix(torch.from_numpy(wq).cuda(), torch.from_numpy(sc.view(np.int16)).cuda().view(torch.bfloat16), gs)
    if tiled:
        mat = mat.tiled()
    x = (rng.normal(0, 1, (n, k)) * rng.uniform(0.5, 4, (n, 1))).astype(np.float32)
    base = rng.normal(0, 1, (n, m)).astype(np.float32)
    flags = {L.EPI_NORM: L.FLAG_WRITE_INV, L.EPI_RESID: L.FLAG_WRITE_RAW}.get(epi, 0)
    a = L.MatArgs(n, k, m, epi, flags, m, 0.8, 1.1, 0.7, 1, k, gs)
    out_m = m // 2 if epi == L.EPI_SWIGLU else m
    aux_n = n if epi == L.EPI_NORM else n * m
    aux_ref = np.zeros(aux_n, np.float32)
    ref = oracle.matmul(L, wq, sc, gs, x, a, base=base if epi == L.EPI_RESID else None, aux=aux_ref)
    y = torch.zeros(n, out_m, device="cuda")
    aux = torch.zeros(aux_n, device="cuda")
    K.matmul(mat, to_dev(x), y, n=n, epi=epi, flags=flags, scale=0.8, ra=1.1, rb=0.7,
             base=to_dev(base) if epi == L.EPI_RESID else None, aux=aux)
    torch.cuda.synchronize()
    assert C.c_int.in_dll(L.lib(), "_ZN2sv12g_mm_variantE").value == 3, "1-16 rows run the one-shot kernel"
    mag = float(np.abs(ref[np.isfinite(ref)]).max())
    close(y.cpu().numpy(), ref, atol=5e-5 * max(mag, 1.0), rtol=1e-4, what=f"grouped epi {epi}")
    if epi in (L.EPI_NORM, L.EPI_RESID):
        close(aux.cpu().numpy(), aux_ref, atol=1e-5 * max(1.0, np.abs(aux_ref).max()), rtol=1e-4, what="aux")


@pytest.mark.parametrize("m,k,n", [(2048, 8192, 512), (2048, 8192, 160), (2048, 2048, 512)])
def test_matmul_gemm_work_orders(gpu, m, k, n):
    """The GEMM's work order (which XCD takes which row blocks, splits and token blocks) changes
    only where operands are cached: the legacy order, each grouping of row blocks and the
    modelled choice give bit-identical outputs, within the bar of the oracle."""
    banner(f"gemm work orders m={m} k={k} n={n}")
    rng = np.random.default_rng(m + k + n)
    w = torch.from_numpy(rng.normal(0, 0.02, (m, k)).astype(np.float32))
    q, s = quantize_rows(w)
    mat = K.matrix(q.cuda(), s.cuda(), 31).tiled()
    x = rng.normal(0, 1, (n, k)).astype(np.float32)
    base = rng.normal(0, 1, (n, m)).astype(np.float32)
    a = L.MatArgs(n, k, m, L.EPI_RESID, 0, m, 0.75, 0.9, 1.3, 1, k, 31)
    ref = oracle.matmul(L, q.numpy(), s.view(torch.int16).numpy().view(np.uint16), 31, x, a, base=base)
    order = C.c_int.in_dll(L.lib(), "_ZN2sv12g_gemm_orderE")
    outs = []
    try:
        for g in (-1, 0, 1, 2, 4, 8):
            order.value = g
            y = torch.zeros(n, m, device="cuda")
            K.matmul(mat, to_dev(x), y, n=n, epi=L.EPI_RESID, scale=0.75, ra=0.9, rb=1.3, base=to_dev(base))
            torch.cuda.synchronize()
            outs.append(y.cpu().numpy())
    finally:
        order.value = -1
    close(outs[0], ref, atol=5e-5 * max(float(np.abs(ref).max()), 1.0), rtol=1e-4, what="gemm")
    for g, o in zip((0, 1, 2, 4, 8), outs[1:]):
        assert np.array_equal(o, outs[0]), f"order {g} differs"
