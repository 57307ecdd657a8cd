"""Pinning the oracle (CPU only): each function is checked against something independent of
its own formula — published known answers, an independent library, closed forms, brute force
or invariants — chosen so a plausible mistake (a dropped term, a wrong sign or index, a
transposed operand) fails one of them. The reference itself (Metal + Rust) cannot be built in
this image, and its repository holds no golden vectors for this path."""
from __future__ import annotations

import ctypes as C
import itertools

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from violetto import _lib as L
from violetto.model import ModelShape

O = oracle


def to_bf_array(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.shape, np.uint16)
    O.lib().orc_to_bf_array(O.ptr(x), O.ptr(out), C.c_size_t(x.size))
    return out


def exp2_array(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.shape, np.float32)
    O.lib().orc_exp2_array(O.ptr(x), O.ptr(out), C.c_size_t(x.size))
    return out


# ------------------------------------------------------------------------ bf16 rounding
def test_bf16_rounding_against_torch_every_finite_pattern_in_strides():
    """kernels.metal:23-27 to_bf vs torch's float32 -> bfloat16 (round to nearest even), over
    every finite float32 bit pattern in a stride-3 sweep of all 2^32 (1.4 G values) plus the
    rounding-boundary patterns (low halves 0x7fff, 0x8000, 0x8001) of every upper half."""
    step = 1 << 25
    for start in range(0, 1 << 32, step):
        u = np.arange(start, start + step, 3, dtype=np.uint64).astype(np.uint32)
        u = u[(u & 0x7F800000) != 0x7F800000]
        f = u.view(np.float32)
        want = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        got = to_bf_array(f)
        fin = np.isfinite(torch.from_numpy(f).to(torch.bfloat16).float().numpy())
        assert np.array_equal(got[fin], want[fin]), f"mismatch near {start:#x}"
    hi = np.arange(0, 1 << 16, dtype=np.uint32)
    hi = hi[(hi & 0x7F80) != 0x7F80]
    for lo in (0x7FFF, 0x8000, 0x8001, 0x0000, 0xFFFF):
        f = ((hi << 16) | lo).view(np.float32)
        want = torch.from_numpy(f).to(torch.bfloat16)
        fin = torch.isfinite(want).numpy()
        assert np.array_equal(to_bf_array(f)[fin], want.view(torch.int16).numpy().view(np.uint16)[fin])


# -------------------------------------------------------------------------------- philox
def test_philox_known_answers():
    """Random123's philox4x32-10 known-answer vectors (kat_vectors)."""
    assert O.philox([0, 0, 0, 0], [0, 0]) == [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    assert O.philox([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2) == [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]
    assert O.philox([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0]) == [
        0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]


def test_uniform01_is_philox_x_top_24_bits():
    for seed, pos, rnd in [(0, 0, 0), (7, 123, 3), (0xFFFFFFFF, 8191, 7)]:
        x = O.philox([pos, rnd, 0, 0], [seed, 0])[0]
        u = O.uniform01(seed, 0, pos, rnd)
        assert u == (x >> 8) / 2.0 ** 24 and 0.0 <= u < 1.0


# ---------------------------------------------------------------------------------- exp2
def test_exp2_accuracy_and_special_points():
    """Every 16th float in [-125, 0) against float64 exp2: at most 2 ulp; exact at integers;
    0 below -125 and at -inf."""
    lo = np.float32(-125.0).view(np.uint32)
    u = np.arange(0x80000001, lo, 16, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    got = exp2_array(x).astype(np.float64)
    want = np.exp2(x.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    err = np.abs(got - want) / ulp
    assert err.max() <= 2.0, f"max error {err.max():.2f} ulp at x = {x[np.argmax(err)]}"
    ints = np.arange(-125, 1, dtype=np.float32)
    assert np.array_equal(exp2_array(ints), np.exp2(ints.astype(np.float64)).astype(np.float32))
    assert exp2_array(np.array([-125.5, -200.0, -np.inf], np.float32)).tolist() == [0.0, 0.0, 0.0]


# ------------------------------------------------------------------------------ quantize
def test_quantize_closed_form_invariants():
    rng = np.random.default_rng(0)
    w = rng.normal(0, 0.02, (64, 512)).astype(np.float32)
    w[3] = 0.0
    for group in (64, 512):
        q, s = O.quantize(w, group)
        g = w.reshape(64, 512 // group, group)
        amax = np.abs(g).max(-1)
        want_s = torch.from_numpy((amax / np.float32(127)).astype(np.float32)).to(torch.bfloat16)
        assert np.array_equal(s, want_s.view(torch.int16).numpy().view(np.uint16)), "scale != bf16(absmax/127)"
        sf = O.bf16_to_f32(s)[..., None]
        qg = q.reshape(64, 512 // group, group).astype(np.float64)
        assert np.abs(q.astype(np.int32)).max() <= 127
        err = np.abs(g - qg * sf)
        # half a step, or the clamp's quarter step when the scale rounded down
        assert (err <= sf * 0.5 + 1e-12).all() or (err <= sf * 0.75 + 1e-12).all()
        assert (q[3] == 0).all()


def test_quantize_ties_round_to_even():
    """w exactly at k + 1/2 steps: q is the even neighbour (torch.round semantics)."""
    s = np.float32(2.0 ** -7)
    row = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 3.0, -126.5], np.float32) * s
    q, sc = O.quantize(row[None, :].repeat(1, 0), 8)
    assert O.bf16_to_f32(sc)[0, 0] == s
    assert q[0].tolist() == [127, 0, 2, 2, 0, -2, 3, -126]


def test_quantize_matches_reference_converter_vectors():
    """orc_quantize against the reference converter's own quantize (tools/convert.py:41-50),
    vectors written by tests/golden/make_quantize_vectors.py: every q and bf16 scale bit for
    bit at groups of 8, 64 and 512, on rows that include exact half steps (ties), groups whose
    scale rounded down (the clamp) and a zero row."""
    f = np.load(Path(__file__).parent / "golden" / "quantize_vectors.npz")
    w = f["w"]
    clamped = ties = 0
    for group in (8, 64, 512):
        q, s = O.quantize(w, group)
        assert np.array_equal(q, f[f"q{group}"]), f"group {group}: q differs"
        assert np.array_equal(s, f[f"s{group}"]), f"group {group}: scales differ"
        sf = O.bf16_to_f32(s).astype(np.float64)
        g = w.reshape(w.shape[0], -1, group).astype(np.float64)
        clamped += int((np.abs(g).max(-1) > 127 * sf).sum())
        ties += int((np.abs(g / np.where(sf > 0, sf, 1)[..., None] % 1 - 0.5) < 1e-12).sum())
    assert clamped > 0 and ties > 0, "the vectors should hold clamped groups and exact half steps"


# -------------------------------------------------------------------------------- matmul
def mat_args(n, k, m, epi, flags=0, scale=1.0, ra=0.0, rb=0.0, vocab_real=None, gshift=31):
    return L.MatArgs(n, k, m, epi, flags, m if vocab_real is None else vocab_real, scale, ra, rb, 1, k, gshift)


@pytest.mark.parametrize("group", [64, 256, 512])
def test_matmul_against_numpy_float64(group):
    rng = np.random.default_rng(group)
    m, k, n = 96, 512, 3
    w = rng.normal(0, 0.05, (m, k)).astype(np.float32)
    q, s = O.quantize(w, group)
    gshift = int(np.log2(group))
    wd = q.astype(np.float64) * np.repeat(O.bf16_to_f32(s).astype(np.float64), group, axis=1)
    x = rng.normal(0, 2, (n, k)).astype(np.float32)
    base = rng.normal(0, 1, (n, m)).astype(np.float32)
    acc = x.astype(np.float64) @ wd.T
    inv = 1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(1) + L.RMS_EPS)
    sig = lambda z: 1 / (1 + np.exp(-z))  # noqa: E731
    aux = np.zeros(n, np.float32)
    y = O.matmul(L, q, s, gshift, x, mat_args(n, k, m, L.EPI_NORM, L.FLAG_WRITE_INV, 0.7, gshift=gshift), aux=aux)
    np.testing.assert_allclose(y, acc * inv[:, None] * 0.7, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(aux, inv, rtol=1e-6)
    raw = np.zeros(n * m, np.float32)
    y = O.matmul(L, q, s, gshift, x, mat_args(n, k, m, L.EPI_RESID, L.FLAG_WRITE_RAW, 0.7, 0.9, 1.3, gshift=gshift),
                 base=base, aux=raw)
    np.testing.assert_allclose(y, 0.9 * base + 1.3 * 0.7 * acc, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(raw.reshape(n, m), 0.7 * acc, rtol=1e-6, atol=1e-7)
    y = O.matmul(L, q, s, gshift, x, mat_args(n, k, m, L.EPI_SWIGLU, scale=1.1, gshift=gshift))
    g, u = acc[:, 0::2] * inv[:, None] * 1.1, acc[:, 1::2] * inv[:, None] * 1.1
    np.testing.assert_allclose(y, g * sig(g) * u, rtol=1e-5, atol=1e-7)
    y = O.matmul(L, q, s, gshift, x, mat_args(n, k, m, L.EPI_HEAD, vocab_real=m - 5, gshift=gshift))
    np.testing.assert_allclose(y[:, : m - 5], 23 * sig((acc[:, : m - 5] + 5) / 7.5), rtol=1e-6)
    assert np.isneginf(y[:, m - 5:]).all()
    y = O.matmul(L, q, s, gshift, x, mat_args(n, k, m, L.EPI_RAW, L.FLAG_NORM_IN, gshift=gshift))
    np.testing.assert_allclose(y, acc * inv[:, None], rtol=1e-6, atol=1e-7)


def test_matmul_identity_and_one_hot():
    """Special cases: bf16 identity weights return the input; a one-hot input picks a column."""
    k = 256
    eye = np.eye(k, dtype=np.float32)
    bits = torch.from_numpy(eye).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    x = np.random.default_rng(1).normal(0, 1, (2, k)).astype(np.float32)
    y = O.matmul(L, bits, None, 0, x, mat_args(2, k, k, L.EPI_RAW))
    assert np.array_equal(y, x)
    w = np.random.default_rng(2).normal(0, 1, (8, k)).astype(np.float32)
    wb = torch.from_numpy(w).to(torch.bfloat16)
    oh = np.zeros((1, k), np.float32)
    oh[0, 77] = 1.0
    y = O.matmul(L, wb.view(torch.int16).numpy().view(np.uint16), None, 0, oh, mat_args(1, k, 8, L.EPI_RAW))
    assert np.array_equal(y[0], wb.float().numpy()[:, 77])


# ----------------------------------------------------------------------------- attention
def textbook_attention(q, K, V, scale):
    """softmax(q . K^T * scale) V with max subtraction, float64 (independent of 2^s sums)."""
    s = (K @ q) * scale
    p = np.exp(s - s.max())
    return (p[:, None] * V).sum(0) / p.sum()


def rotate_pairs(x, cs):
    """RoPE as a complex product, written from the reference's own Python statement of it
    (tools/spec/drafter.py:33-38): dims (2j, 2j + 1) as z_j = x_2j + i x_2j+1 become z_j (cos - i sin),
    i.e. (c a0 + s a1, c a1 - s a0); cs holds (cos, sin) per pair."""
    z = x[0::2].astype(np.complex128) + 1j * x[1::2]
    z = z * (cs[:, 0] - 1j * cs[:, 1])
    out = np.empty_like(x, dtype=np.float64)
    out[0::2], out[1::2] = z.real, z.imag
    return out


@pytest.mark.parametrize("theta", [None, 500000.0])
def test_attention_against_textbook_softmax(theta):
    """Attention against max-subtracted natural-exp softmax in float64, with RoPE off (theta None:
    zero frequencies, the identity) and on (theta 500000: the queries and new keys rotated at
    their own positions as complex products). A wrong pair layout, sign or table row for q or k
    changes the scores and fails this."""
    sh = ModelShape(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=256, vocab=64, vocab_real=64, n_layers=1)
    rng = np.random.default_rng(0)
    D, NQ, NKV = 64, 4, 2
    W = (NQ + 2 * NKV) * D
    page_shift, page = 4, 16
    T, p0 = 3, 40
    n_pages = 4
    table = np.array([[2, 0, 3, 1]], np.uint32)
    k_cache = to_bf_array(rng.normal(0, 1, (1, n_pages, NKV, page, D)))
    v_cache = to_bf_array(rng.normal(0, 1, (1, n_pages, NKV, page, D)))
    qkv = rng.normal(0, 1, (T, W)).astype(np.float32)
    meta = np.array([0, p0, 0, p0 + 1, 0, p0 + 2], np.uint32)
    vis = np.array([1, 3, 5], np.uint32)  # row 2 sees row 0 and itself only
    freq = np.zeros(32, np.float32) if theta is None else (theta ** (-2.0 * np.arange(32) / 64)).astype(np.float32)
    rope = O.rope_table(freq, p0 + 4)
    kv = L.KvArgs(1, 0, 0, 1, page_shift, n_pages, 4, 0)
    scale = 0.125
    args = L.AttnArgs(32, 3, scale * np.log2(np.e), 1, 0, 0, 0, 0, 0)
    kc, vc = k_cache.copy(), v_cache.copy()
    out = O.attn_verify(L, sh, qkv, meta, kc, vc, table, rope, kv, args, np.array([0, T], np.uint32), vis)

    def rms(v):
        return v / np.sqrt((v.astype(np.float64) ** 2).mean() + L.RMS_EPS)

    def roped(v, pos):  # the table (pinned against float64 trig) at the row's own position
        return rotate_pairs(rms(v), rope[pos].reshape(32, 2).astype(np.float64))

    def cached(cache, pos, g):
        page_i = table[0, pos >> page_shift]
        return O.bf16_to_f32(cache[0, page_i, g, pos & (page - 1)]).astype(np.float64)

    new_k = [[O.bf16_to_f32(to_bf_array(roped(qkv[i, NQ * D + g * D: NQ * D + (g + 1) * D], p0 + i).astype(np.float32)))
              for g in range(NKV)] for i in range(T)]
    new_v = [[O.bf16_to_f32(to_bf_array(qkv[i, (NQ + NKV) * D + g * D:(NQ + NKV) * D + (g + 1) * D]))
              for g in range(NKV)] for i in range(T)]
    for i in range(T):
        for h in range(NQ):
            g = h // (NQ // NKV)
            keys = [cached(k_cache, j, g) for j in range(p0)] + [new_k[j][g] for j in range(T) if vis[i] >> j & 1]
            vals = [cached(v_cache, j, g) for j in range(p0)] + [new_v[j][g] for j in range(T) if vis[i] >> j & 1]
            want = textbook_attention(roped(qkv[i, h * D:(h + 1) * D], p0 + i), np.array(keys), np.array(vals), scale)
            np.testing.assert_allclose(out[i, h * D:(h + 1) * D], want, rtol=1e-5, atol=1e-6)
    # the new keys landed at p0 + row, through the page table
    for i in range(T):
        pg = table[0, (p0 + i) >> page_shift]
        assert np.array_equal(O.bf16_to_f32(kc[0, pg, 1, (p0 + i) & 15]), new_k[i][1])
        assert np.array_equal(O.bf16_to_f32(vc[0, pg, 1, (p0 + i) & 15]), new_v[i][1])


def test_attention_uniform_values_and_masking_invariants():
    """Uniform V gives V whatever the scores; keys outside the mask do not matter."""
    sh = ModelShape(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=256, vocab=64, vocab_real=64, n_layers=1)
    rng = np.random.default_rng(3)
    D, NQ, NKV = 64, 4, 2
    W = (NQ + 2 * NKV) * D
    T, p0 = 2, 16
    table = np.array([[0, 1]], np.uint32)
    k_cache = to_bf_array(rng.normal(0, 1, (1, 2, NKV, 16, D)))
    v_cache = to_bf_array(np.full((1, 2, NKV, 16, D), 0.75, np.float32))
    qkv = rng.normal(0, 1, (T, W)).astype(np.float32)
    qkv[:, (NQ + NKV) * D:] = 0.75
    meta = np.array([0, p0, 0, p0 + 1], np.uint32)
    rope = O.rope_table(np.full(32, 0.01, np.float32), 20)
    kv = L.KvArgs(1, 0, 0, 1, 4, 2, 2, 0)
    args = L.AttnArgs(32, 2, 0.18, 1, 0, 0, 0, 0, 0)
    out = O.attn_verify(L, sh, qkv, meta, k_cache.copy(), v_cache.copy(), table, rope, kv, args,
                        np.array([0, T], np.uint32), np.array([1, 3], np.uint32))
    np.testing.assert_allclose(out, 0.75, rtol=1e-12)
    # token 0 sees only row 0: changing row 1's K/V leaves its output alone
    v2 = qkv.copy()
    v2[:, (NQ + NKV) * D:] = rng.normal(0, 1, (T, NKV * D))
    o1 = O.attn_verify(L, sh, v2, meta, k_cache.copy(), v_cache.copy(), table, rope, kv, args,
                       np.array([0, T], np.uint32), np.array([1, 3], np.uint32))
    v3 = v2.copy()
    v3[1, NQ * D:] = rng.normal(0, 5, (2 * NKV * D,))
    o2 = O.attn_verify(L, sh, v3, meta, k_cache.copy(), v_cache.copy(), table, rope, kv, args,
                       np.array([0, T], np.uint32), np.array([1, 3], np.uint32))
    assert np.array_equal(o1[0], o2[0]) and not np.array_equal(o1[1], o2[1])


# ------------------------------------------------------------------------------- sampler
def test_sample_greedy_is_numpy_argmax_lowest_on_ties():
    rng = np.random.default_rng(4)
    logits = rng.normal(0, 1, (6, 3000)).astype(np.float32)
    logits[1, [10, 500, 2999]] = 9.0
    logits[2, :] = -np.inf
    logits[2, 1234] = 0.0
    rows = [L.SampleRow(0, 0, 5, 0.0, 1.0, L.NO_TOK)] * 6
    got = O.sample(L, logits, rows)
    assert got.tolist() == [int(np.argmax(r)) for r in logits]
    assert got[1] == 10


@pytest.mark.parametrize("vocab", [7, 64, 1500])
def test_sample_inverse_cdf_against_float64(vocab):
    """top_p = 1: the draw at u = uniform01(seed, pos, 0) is the token whose float64 CDF
    interval (in the kernel's id order: thread t owns t, t + 1024, ...) holds u; cases within
    1e-5 of an interval edge are skipped (rounding decides them)."""
    rng = np.random.default_rng(vocab)
    T = 0.7
    logits = rng.normal(10, 1.5, (1, vocab)).astype(np.float32)
    order = np.concatenate([np.arange(t, vocab, 1024) for t in range(1024)])
    x = logits[0].astype(np.float64)
    e = np.exp2((x - x.max()) * (np.log2(np.e) / T))
    cdf = np.cumsum(e[order]) / e.sum()
    checked = 0
    for seed in range(400):
        u = O.uniform01(seed, 0, 77, 0)
        j = int(np.searchsorted(cdf, u, side="right"))
        if min(abs(u - cdf[max(j - 1, 0)]), abs(cdf[min(j, vocab - 1)] - u)) < 1e-5:
            continue
        got = O.sample(L, logits, [L.SampleRow(seed, 0, 77, T, 1.0, L.NO_TOK)])[0]
        assert got == order[j], f"seed {seed}: {got} != {order[j]}"
        checked += 1
    assert checked > 300


def test_sample_top_p_set_and_frequencies():
    """With top_p < 1 every draw lies in the top-p set (tokens more likely than it hold less
    than top_p of the mass), and empirical frequencies follow the renormalised top-p
    distribution (chi-square)."""
    vocab, T, top_p = 12, 1.0, 0.8
    logits = np.array([[3.0, 2.5, 2.4, 1.0, 0.5, 0.0, -1, -2, -2, -3, -5, -9]], np.float32)
    x = logits[0].astype(np.float64)
    p = np.exp(x - x.max())
    p /= p.sum()
    above = np.array([p[x > xi].sum() for xi in x])
    in_set = above < top_p
    counts = np.zeros(vocab)
    n = 4000
    for seed in range(n):
        j = O.sample(L, logits, [L.SampleRow(seed, 1, 5, T, top_p, L.NO_TOK)])[0]
        assert in_set[j], f"token {j} outside the top-p set"
        counts[j] += 1
    q = np.where(in_set, p, 0)
    q /= q.sum()
    chi2 = ((counts - n * q) ** 2 / np.maximum(n * q, 1e-9))[in_set].sum()
    assert chi2 < 30, f"chi-square {chi2:.1f}"


# -------------------------------------------------------------------------------- accept
def independent_accept(parent, tokens, out, remaining, stops):
    """Path: from the root, the lowest-index child whose draft equals the parent's sampled
    token; then emission stops after a stop token and at the budget."""
    path, at = [0], 0
    while True:
        kids = [c for c in range(1, len(parent)) if parent[c] == at and tokens[c] == out[at]]
        if not kids:
            break
        at = min(kids)
        path.append(at)
    k = 0
    emitted = []
    for r in path:
        if k >= remaining:
            break
        emitted.append(out[r])
        k += 1
        if out[r] in stops:
            break
    return path[:k], emitted


def all_trees(n):
    """Every parent assignment with parent(c) < c (n <= 5: 24 trees)."""
    return [[0xFF] + list(ps) for ps in itertools.product(*[range(c) for c in range(1, n)])]


def test_accept_brute_force_small_trees():
    checked = 0
    for n in range(1, 6):
        for parent in all_trees(n):
            for tokens in itertools.product(range(2), repeat=n):
                for out in itertools.product(range(2), repeat=n):
                    for remaining, stops in [(0xFFFFFFFF, ()), (2, ()), (0xFFFFFFFF, (1,))]:
                        depth = [0] * n
                        sees = [1] * n
                        for i in range(1, n):
                            depth[i] = depth[parent[i]] + 1
                            sees[i] = sees[parent[i]] | 1 << i
                        tree = np.zeros(16, np.uint32)
                        tree[:n] = [depth[i] | parent[i] << 8 | sees[i] << 16 for i in range(n)]
                        g = L.GenState(remaining, 0, len(stops), 0, (C.c_uint32 * 8)(*stops))
                        run = L.RunIn(0, 0, n, 0, n, 1)
                        o_out, lens, feed, gen, em, path, plen, on = O.accept(
                            L, [run], list(tokens), list(out), [100], [0] * 16, [g], tree, n)
                        want_path, want_em = independent_accept(parent, tokens, out, remaining, stops)
                        assert em[0] == len(want_em) and plen[0] == len(want_path)
                        assert o_out[: em[0]].tolist() == want_em
                        assert path[: plen[0]].tolist() == want_path
                        assert lens[0] == 100 + len(want_em)
                        if want_em:
                            assert feed[0] == want_em[-1]
                        assert on[:n].tolist() == [1 if i in want_path else 0 for i in range(n)]
                        checked += 1
    assert checked > 10000


def test_kv_compact_moves_only_path_rows():
    sh = ModelShape(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=256, vocab=64, vocab_real=64, n_layers=2)
    rng = np.random.default_rng(6)
    kc = rng.integers(0, 65535, (2, 4, 2, 16, 64)).astype(np.uint16)
    vc = rng.integers(0, 65535, kc.shape).astype(np.uint16)
    table = np.array([[3, 1, 0, 2]], np.uint32)
    kv = L.KvArgs(1, 0, 0, 1, 4, 4, 4, 0)
    path = np.zeros(16, np.uint32)
    path[:4] = [0, 2, 5, 9]
    run = L.RunIn(0, 0, 10, 0, 10, 1)
    lens = np.array([30 + 4], np.uint32)  # p0 = 30
    k2, v2 = kc.copy(), vc.copy()
    O.kv_compact(L, sh, [run], path, np.array([4], np.uint32), lens, k2, v2, table, kv)

    def row(c, pos):
        return c[:, table[0, pos >> 4], :, pos & 15]

    for j, frm in enumerate([0, 2, 5, 9]):
        assert np.array_equal(row(k2, 30 + j), row(kc, 30 + frm))
        assert np.array_equal(row(v2, 30 + j), row(vc, 30 + frm))
    moved = {30 + j for j in range(1, 4)}
    for pos in range(64):
        if pos not in moved:
            assert np.array_equal(row(k2, pos), row(kc, pos))


def test_pool_lifo_order():
    p = O.Pool(8, 3, 4, 4)
    assert p.reserve(0, 40) and p.pages(0) == [0, 1, 2]
    assert p.reserve(1, 17) and p.pages(1) == [3, 4]
    p.release(0)
    assert p.reserve(2, 33) and p.pages(2) == [0, 1, 2]
    assert p.reserve(0, 16) and p.pages(0) == [5]
    assert not p.reserve(1, 16 * 4 + 1), "max_pages exceeded or pool exhausted"


# --------------------------------------------------------------- the lossless invariant
def tiny_model(seed=0, n_layers=2):
    from violetto.model import SyntheticModel

    shape = ModelShape(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=300, vocab_real=290,
                       n_layers=n_layers)
    return shape, SyntheticModel.generate(shape, seed=seed, device="cpu", std=0.1)


def test_lossless_speculation_on_the_oracle():
    """bench_spec.rs:119-139: greedy verification with replayed drafts (some wrong) emits
    exactly the tokens plain decoding emits."""
    from violetto.model import rope_freq

    shape, model = tiny_model()
    emb, lay, sc = O.host_weights(model)
    freq = rope_freq(500000.0, 64)

    def engine():
        e = O.OracleEngine(L, shape, emb, lay, sc, max_seqs=1, max_seq_len=256, kv_tokens=256, freq=freq)
        s = e.new_seq()
        rng = np.random.default_rng(11)
        e.bench_fill(s, 40)
        e.k[...] = to_bf_array(rng.normal(0, 1, e.k.shape))
        e.v[...] = to_bf_array(rng.normal(0, 1, e.v.shape))
        e.set_feed(s, 40, 5)
        return e, s

    plain, s = engine()
    trace = [5]
    for _ in range(24):
        ids, _, em, _ = plain.step([(s, [L.FEED_ROW], False)])
        trace.append(int(ids[0]))
    spec, s = engine()
    rng = np.random.default_rng(2)
    got = [5]
    while len(got) < 20:
        pos = len(got) - 1
        drafts = [trace[pos + i] if rng.random() > 0.3 else (trace[pos + i] + 1) % 290 for i in range(1, 5)]
        ids, _, em, extra = spec.step([(s, [L.FEED_ROW] + drafts, True)])
        got += [int(t) for t in ids[: em[0]]]
    assert got[:20] == trace[:20]


# ------------------------------------------------- rope table, embed, rmsnorm_rows, replay
def bf16_round_torch(x: np.ndarray) -> np.ndarray:
    """float -> bf16 (round to nearest even) -> float, by torch (independent of the oracle)."""
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).float().numpy()


def test_rope_freq_closed_form():
    """f_j = theta^(-2 j / 64) (model.rs:81, tools/convert.py:59-61), as float32."""
    from violetto.model import rope_freq

    f = rope_freq(500000.0, 64)
    want = np.array([500000.0 ** (-2.0 * j / 64) for j in range(32)])
    assert f.dtype == np.float32 and f.shape == (32,)
    assert np.all(np.abs(f.astype(np.float64) - want) <= np.spacing(np.float32(want)).astype(np.float64))
    assert f[0] == 1.0 and np.all(np.diff(f) < 0)


def test_rope_table_against_float64_trig():
    """engine.rs:394-421: tab[pos][j] = (bf16(cos th), bf16(sin th)), th = f32(pos) * f_j in
    float32. Pinned against float64 cos/sin of the same float32 angle, rounded to bf16 by
    torch: equal except where the float32 library value and the exact one straddle a bf16
    rounding boundary (then one bf16 step apart, and the exact value within 2^-22 relative of
    that boundary)."""
    from violetto.model import rope_freq

    f = rope_freq(500000.0, 64)
    pos = np.arange(0, 70000, 7, dtype=np.float32)  # every 7th position up to past 65536
    n = int(pos[-1]) + 1
    tab = O.rope_table(f, n)[pos.astype(np.int64)]
    th = (pos[:, None] * f[None, :]).astype(np.float32)  # float32 product, as the reference
    exact = np.stack([np.cos(th.astype(np.float64)), np.sin(th.astype(np.float64))], -1)
    want = bf16_round_torch(exact.astype(np.float32))
    diff = tab != want
    assert tab[0, 0, 0] == 1.0 and tab[0, 0, 1] == 0.0  # pos 0: cos 1, sin 0 (sign convention)
    assert np.all(np.isfinite(tab)) and np.all(np.abs(tab) <= 1.0)
    if diff.any():
        e = exact[diff]
        step = np.abs(np.spacing(bf16_round_torch(e.astype(np.float32)).astype(np.float32))) * 65536.0
        assert np.all(np.abs(tab[diff] - want[diff]) <= step * 1.0001), "off by more than one bf16 step"
        # the exact value sits at a rounding boundary: (value - boundary) tiny relative to the value
        mid = (tab[diff].astype(np.float64) + want[diff].astype(np.float64)) / 2
        assert np.all(np.abs(e - mid) <= 2.0 ** -22 * np.abs(e) + 1e-30)
    assert diff.mean() < 1e-3


def test_embed_resolution_and_norm_properties():
    """kernels.metal:82-114: GPU-fed rows take their id from feed[slot][i] and depth/vis from
    the tree node; meta = (slot, lens[slot] + depth); out = row / rms(row) (no gain, eps
    2^-23): collinear with the bf16 row, mean square 1 / (1 + eps / ms), and for a constant row
    c the closed form c / sqrt(c^2 + eps)."""
    shape = ModelShape(n_layers=1, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=64,
                       vocab_real=64)
    rng = np.random.default_rng(3)
    table = (rng.normal(0, 0.02, (64, 256)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    table[5] = 0x3F40  # a constant row: 0.75
    feed = np.zeros((2, 16), np.uint32)
    tree = np.zeros((2, 16), np.uint32)
    feed[1, :3] = [9, 5, 33]
    # node i: depth | parent << 8 | sees << 16 (kernels.metal:64-72): 0 root, 1 and 2 children of 0
    tree[1, :3] = [0 | (0xFF << 8) | (1 << 16), 1 | (0 << 8) | (0b011 << 16), 1 | (0 << 8) | (0b101 << 16)]
    lens = np.array([40, 100], np.uint32)
    tokens = [7, L.FEED_ROW + 0, L.FEED_ROW + 1, L.FEED_ROW + 2, 5]
    tin = np.array([[0, 0], [1, 0], [1, 1], [1, 2], [0, 1]], np.uint32)
    vis0 = np.array([0xAA, 0, 0, 0, 0xBB], np.uint32)
    tok, out, meta, vis = O.embed(L, shape, table, tokens, tin, lens, feed.reshape(-1), tree.reshape(-1), vis0)
    assert list(tok) == [7, 9, 5, 33, 5]
    assert meta.tolist() == [[0, 40], [1, 100], [1, 101], [1, 101], [0, 41]]
    assert list(vis) == [0xAA, 0b001, 0b011, 0b101, 0xBB]  # CPU rows keep theirs
    rows = (table.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    eps = 2.0 ** -23
    for t, tk in enumerate(tok):
        r = rows[tk]
        o = out[t].astype(np.float64)
        ms = np.mean(r * r)
        assert abs(np.mean(o * o) - 1.0 / (1.0 + eps / ms)) < 1e-5
        cos = np.dot(o, r) / np.linalg.norm(o) / np.linalg.norm(r)
        assert cos > 1 - 1e-12
    assert np.all(out[4] == np.float32(0.75 / np.sqrt(0.75 ** 2 + eps)))


def test_rmsnorm_rows_gather_and_properties():
    """kernels.metal:117-131: out[r] = in[rows[r]] / rms (no gain): gathered in rows' order,
    collinear, mean square 1 / (1 + eps / ms); a zero row stays zero."""
    rng = np.random.default_rng(4)
    x = (rng.normal(0, 1, (6, 128)) * rng.uniform(0.01, 30, (6, 1))).astype(np.float32)
    x[2] = 0.0
    rows = np.array([4, 0, 2, 4], np.uint32)
    out = np.zeros((4, 128), np.float32)
    O.lib().orc_rmsnorm_rows(O.ptr(x), O.ptr(rows), O.ptr(out), C.c_uint32(4), C.c_uint32(128))
    eps = 2.0 ** -23
    for r, src in enumerate(rows):
        v = x[src].astype(np.float64)
        o = out[r].astype(np.float64)
        if not v.any():
            assert not o.any()
            continue
        ms = np.mean(v * v)
        assert abs(np.mean(o * o) - 1.0 / (1.0 + eps / ms)) < 1e-5
        assert np.dot(o, v) / np.linalg.norm(o) / np.linalg.norm(v) > 1 - 1e-12
    assert np.array_equal(out[0], out[3])


def test_replay_draft_rules():
    """kernels.metal:1695-1724: drafts i = 1..15 replay trace[lens + i]; with probability rate
    (Philox4x32-10 of (pos, 0x5eed) under (seed, 0x0dd5), top 24 bits) the id is replaced by
    id + 1 mod vocab; positions past the trace read 0; the tree becomes the chain; runs with
    no head rows are left alone; feed[slot][0] is untouched."""
    stride, vocab = 64, 50
    trace = np.zeros((3, stride), np.uint32)
    trace[0, :40] = np.arange(40) % vocab
    trace[1, :64] = (np.arange(64) * 7 + 3) % vocab
    trace_len = np.array([40, 64, 0], np.uint32)
    lens = np.array([30, 10, 5], np.uint32)
    runs = [L.RunIn(0, 0, 5, 0, 5, 1), L.RunIn(1, 5, 5, 5, 0, 1), L.RunIn(2, 10, 1, 10, 1, 0)]

    def run(rate, seed=11):
        feed = np.full(3 * 16, 777, np.uint32)
        tree = np.full(3 * 16, 0xDEAD, np.uint32)
        O.replay_draft(L, runs, lens, feed, trace.reshape(-1), trace_len, L.ReplayArgs(stride, seed, rate, vocab), tree)
        return feed.reshape(3, 16), tree.reshape(3, 16)

    f0, t0 = run(0.0)
    want = np.array([trace[0, 30 + i] if 30 + i < 40 else 0 for i in range(1, 16)])
    assert np.array_equal(f0[0, 1:], want) and f0[0, 0] == 777
    assert np.all(f0[1] == 777) and np.all(t0[1] == 0xDEAD)  # no head rows: untouched
    assert np.all(f0[2] == 777)  # empty trace: untouched
    for i in range(1, 16):
        assert t0[0, i] == i | ((i - 1) << 8) | (((2 << i) - 1) << 16)
    f1, _ = run(1.0)
    assert np.array_equal(f1[0, 1:], (want + 1) % vocab)
    # an intermediate rate mixes the two, per position, the same way for the same seed
    fa, _ = run(0.5, seed=3)
    fb, _ = run(0.5, seed=3)
    assert np.array_equal(fa, fb)
    assert set(np.nonzero(fa[0, 1:] != want)[0]) == set(np.nonzero(fa[0, 1:] == (want + 1) % vocab)[0])


# ------------------------------------------------------------------- DDTree draft builder
@pytest.mark.parametrize("ncand", [1, 2, 4])
def test_draft_top_against_sort(ncand):
    """draft_top: each drafted row's candidates are its top ids by a float64 sort (value
    descending, ties to the lower id), mapped through the draft vocabulary; their
    probabilities the float64 softmax at temperature 1 / inv_t; the block's row 0 untouched."""
    rng = np.random.default_rng(ncand)
    nv, n, inv_t = 3000, 6, 1.0 / 0.7
    logits = rng.normal(0, 2, (n, nv)).astype(np.float32)
    logits[2, [17, 900, 2999]] = logits[2].max() + 1.0  # tied maxima: lowest ids first
    logits[3, 5:] = logits[3, :5].min() - 50.0          # a peaked row
    vocab = np.sort(rng.choice(100000, nv, replace=False)).astype(np.uint32)
    tin = np.array([[0, i] for i in range(n)], np.uint32)  # one block: row 0 is the bonus token's
    cand, cand_q = O.draft_top(logits, vocab, tin, inv_t, ncand)
    assert (cand[0] == 0).all() and (cand_q[0] == 0).all()
    for r in range(1, n):
        x = logits[r].astype(np.float64)
        order = np.lexsort((np.arange(nv), -x))[:ncand]
        assert np.array_equal(cand[r, :ncand], vocab[order]), f"row {r}"
        p = np.exp((x - x.max()) * inv_t)
        p /= p.sum()
        np.testing.assert_allclose(cand_q[r, :ncand], p[order], rtol=2e-5)


def _tree_brute_force(q, ids, first, rows, ncand):
    """Every candidate path of the block (block row d gives the choices at depth d), scored by
    the fp32 product of q along it, highest first: the first rows - 1 are the tree's nodes."""
    paths = [()]
    frontier = [()]
    for d in range(1, rows):
        frontier = [p + (c,) for p in frontier for c in range(ncand)]
        paths += frontier
    scored = []
    for p in paths[1:]:
        s = np.float32(1.0)
        for d, c in enumerate(p, start=1):
            s = np.float32(s * np.float32(q[first + d, c]))
        scored.append((float(s), p))
    scored.sort(key=lambda e: -e[0])
    top = scored[: rows - 1]
    if len(scored) > rows - 1:
        assert top[-1][0] != scored[rows - 1][0], "tie at the cut (pick another seed)"
    index = {(): 0}
    nodes = []
    sees = {0: 1}
    for n, (_, p) in enumerate(top, start=1):
        parent = index[p[:-1]]
        index[p] = n
        sees[n] = sees[parent] | 1 << n
        nodes.append((int(ids[first + len(p), p[-1]]), len(p) | parent << 8 | sees[n] << 16))
    return nodes


@pytest.mark.parametrize("seed", range(6))
def test_draft_tree_brute_force(seed):
    """draft_tree against a brute force over every candidate path: the nodes, in order, are the
    highest path products (a child never outscores its parent, so best-first order is score
    order); tokens from their block row's candidates; parents, depths and ancestry masks from
    the paths; the rest of each slot's entries dead nodes; slot 0 entries other blocks do not
    own untouched."""
    rng = np.random.default_rng(100 + seed)
    ncand = [1, 2, 3, 4, 2, 2][seed]  # the enumeration has ncand^(rows - 1) leaves
    block_rows = [[1, 2, 5], [8, 3], [6, 8, 2, 4], [5, 8], [16], [12, 1, 9]][seed]
    blocks, tin = [], []
    slots = rng.permutation(8)[: len(block_rows)]
    for slot, rows in zip(slots, block_rows):
        blocks.append((len(tin), rows))
        tin += [(int(slot), i) for i in range(rows)]
    n = len(tin)
    q = np.sort(rng.dirichlet(np.ones(6), n)[:, :4], axis=1)[:, ::-1].astype(np.float32)  # descending, < 1
    ids = rng.integers(0, 50000, (n, 4)).astype(np.uint32)
    feed = rng.integers(0, 50000, 8 * 16).astype(np.uint32)
    tree = rng.integers(0, 1 << 30, 8 * 16).astype(np.uint32)
    feed0, tree0 = feed.copy(), tree.copy()
    O.draft_tree(np.array(blocks, np.uint32), np.array(tin, np.uint32), ids, q, feed, tree, ncand)
    for slot, (first, rows) in zip(slots, blocks):
        nodes = _tree_brute_force(q, ids, first, rows, ncand) if rows > 1 else []
        got_feed = feed[slot * 16: slot * 16 + 16]
        got_tree = tree[slot * 16: slot * 16 + 16]
        assert got_feed[0] == feed0[slot * 16] and got_tree[0] == tree0[slot * 16], "the root entry is the caller's"
        for i, (tok, node) in enumerate(nodes, start=1):
            assert got_feed[i] == tok and got_tree[i] == node, f"slot {slot} node {i}"
        for i in range(len(nodes) + 1, 16):
            assert got_tree[i] == 1 | 0xFF << 8 | (1 | 1 << i) << 16, f"slot {slot} dead node {i}"
            assert got_feed[i] == feed0[slot * 16 + i]
    for s in set(range(8)) - set(int(x) for x in slots):
        assert np.array_equal(feed[s * 16: s * 16 + 16], feed0[s * 16: s * 16 + 16])
        assert np.array_equal(tree[s * 16: s * 16 + 16], tree0[s * 16: s * 16 + 16])


def test_draft_tree_skips_unfilled_candidates():
    """A block row with fewer candidates than ncand (draft_top's SV_NO_TOK: no ordered value
    left) offers only the ones it has: a chain of 4 rows where row 2 has one candidate."""
    q = np.array([[0, 0, 0, 0], [0.6, 0.3, 0, 0], [0.9, 0, 0, 0], [0.5, 0.4, 0, 0]], np.float32)
    ids = np.array([[0, 0, 0, 0], [11, 12, 0, 0], [21, L.NO_TOK, 0, 0], [31, 32, 0, 0]], np.uint32)
    feed = np.zeros(16, np.uint32)
    tree = np.zeros(16, np.uint32)
    O.draft_tree(np.array([0, 4], np.uint32), np.array([[0, i] for i in range(4)], np.uint32), ids, q, feed, tree, 2)
    # best-first: 11 (0.6), 21 under it (0.54), 12 (0.3)... : three nodes, none of them NO_TOK
    assert list(feed[1:4]) == [11, 21, 12]
    assert L.NO_TOK not in feed


# ------------------------------------------------------------------- prompt chunks
def test_chunk_prefill_equals_token_by_token():
    """A prompt chunk (one non-verify run of 40 rows: attention runs of 16, each later one seeing
    the earlier ones' keys as cached) leaves the same KV cache and the same last-row logits as
    feeding the prompt one token per step, bit for bit (the oracle's sums run in position
    order either way), on top of 23 cached tokens."""
    from violetto.model import ModelShape, SyntheticModel

    shape = ModelShape(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=256, vocab=512, vocab_real=500,
                       n_layers=2)
    model = SyntheticModel.generate(shape, seed=5, device="cpu")
    emb, lay, sc = O.host_weights(model)
    freq = (500000.0 ** (-2.0 * np.arange(32) / 64)).astype(np.float32)
    engines = [O.OracleEngine(L, shape, emb, lay, sc, max_seqs=1, max_seq_len=128, kv_tokens=128, freq=freq)
               for _ in range(2)]
    rng = np.random.default_rng(6)
    kv0 = rng.integers(0x3C00, 0x4000, engines[0].k.shape, dtype=np.uint16)
    prompt = [int(x) for x in rng.integers(0, 500, 40)]
    for e in engines:
        s = e.new_seq()
        e.bench_fill(s, 23)
        e.k[...] = kv0
        e.v[...] = kv0 ^ np.uint16(0x8000)
    ids_a, logits_a, _, _ = engines[0].step([(0, prompt, False, 1)])
    for i, t in enumerate(prompt):
        ids_b, logits_b, _, _ = engines[1].step([(0, [t], False, 1)])
    assert engines[0].seq_len[0] == engines[1].seq_len[0] == 63
    assert engines[0].lens[0] == engines[1].lens[0] == 63
    assert np.array_equal(logits_a[-1], logits_b[-1]) and ids_a[-1] == ids_b[-1]
    pages = engines[0].pool.pages(0)
    assert pages == engines[1].pool.pages(0)
    for arr in ("k", "v"):
        a, b = getattr(engines[0], arr), getattr(engines[1], arr)
        assert np.array_equal(a[:, pages], b[:, pages]), f"{arr} cache"
