"""Pinning the oracle's Limite extras (CPU only): sliding-window layers over a ring cache,
value embeddings, XSA, the attention gate and MUDD (engine/src/kernels.metal:738-747, 808-811,
910-942, 1316-1407; kv.rs:26-32; encode.rs:107-160). Each check is independent of the oracle's
own formula: textbook attention over explicit position arrays, special cases that reduce an
extra to the plain path, geometric invariants, one-hot cases against float64 numpy and
math.erf, and whole-step invariants (a prompt chunk equals token-by-token feeding, and greedy
verification with replayed drafts emits the plain-decode tokens)."""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from test_oracle import rotate_pairs, textbook_attention, to_bf_array
from violetto import _lib as L
from violetto.model import ModelShape, SyntheticModel, generate_extras, limite_layout, rope_freq

O = oracle
D, NQ, NKV = 64, 4, 2
W = (NQ + 2 * NKV) * D
SH = ModelShape(hidden=256, n_heads=NQ, n_kv_heads=NKV, head_dim=D, ffn=256, vocab=64, vocab_real=64, n_layers=1)


def rms(v):
    return v / np.sqrt((v.astype(np.float64) ** 2).mean() + L.RMS_EPS)


# ------------------------------------------------------------------- sliding-window layers
def test_window_attention_against_textbook_over_the_ring():
    """A sliding-window layer (window 40) over rings of 4 pages (64 keys) through a cyclic page
    table: each query at pos sees exactly the keys [pos - 40, pos) of its history plus the new
    keys in its vis mask, computed by textbook softmax from position-indexed history arrays
    (no ring). Sequence 0 is past the window (positions 150-152, the ring has wrapped twice);
    sequence 1 (p0 = 20) is inside it. A window off by one, or a ring slot read for the wrong
    position, changes the key set and fails this."""
    rng = np.random.default_rng(1)
    window, ring_pages, page = 40, 4, 16
    max_pages = 16
    table = np.array([[s * ring_pages + p % ring_pages for p in range(max_pages)] for s in range(2)], np.uint32)
    n_pages = 2 * ring_pages
    p0s, T = [150, 20], 3
    hist = {s: (to_bf_array(rng.normal(0, 1, (p0s[s], NKV, D))), to_bf_array(rng.normal(0, 1, (p0s[s], NKV, D))))
            for s in range(2)}
    kc = to_bf_array(rng.normal(0, 1, (1, n_pages, NKV, page, D)))  # slots never written hold noise
    vc = to_bf_array(rng.normal(0, 1, (1, n_pages, NKV, page, D)))
    for s in range(2):
        for pos in range(max(0, p0s[s] - ring_pages * page), p0s[s]):
            pg = table[s, pos >> 4]
            kc[0, pg, :, pos & 15] = hist[s][0][pos]
            vc[0, pg, :, pos & 15] = hist[s][1][pos]
    qkv = rng.normal(0, 1, (2 * T, W)).astype(np.float32)
    meta = np.array([[s, p0s[s] + i] for s in range(2) for i in range(T)], np.uint32).reshape(-1)
    vis = np.array([1, 3, 7] * 2, np.uint32)
    freq = (500000.0 ** (-2.0 * np.arange(32) / 64)).astype(np.float32)
    rope = O.rope_table(freq, 160)
    kv = L.KvArgs(0, 0, ring_pages * page, 2, 4, n_pages, max_pages, window)
    scale = 0.125
    args = L.AttnArgs(32, 8, scale * np.log2(np.e), 1, 0, 0, 0, 0, 0)
    k2, v2 = kc.copy(), vc.copy()
    out = O.attn_verify(L, SH, qkv, meta, k2, v2, table, rope, kv, args, np.array([0, T, T, T], np.uint32), vis)

    def roped(v, pos):
        return rotate_pairs(rms(v), rope[pos].reshape(32, 2).astype(np.float64))

    for s in range(2):
        for i in range(T):
            t, pos = s * T + i, p0s[s] + i
            new_k = [O.bf16_to_f32(to_bf_array(roped(qkv[s * T + j, NQ * D + g * D:NQ * D + (g + 1) * D],
                                                     p0s[s] + j).astype(np.float32))) for j in range(T)
                     for g in range(NKV)]
            for h in range(NQ):
                g = h // (NQ // NKV)
                lo = max(0, pos - window)
                keys = [O.bf16_to_f32(hist[s][0][j, g]) for j in range(lo, p0s[s])]
                vals = [O.bf16_to_f32(hist[s][1][j, g]) for j in range(lo, p0s[s])]
                for j in range(T):
                    if vis[t] >> j & 1:
                        keys.append(new_k[j * NKV + g])
                        vals.append(O.bf16_to_f32(to_bf_array(qkv[s * T + j, (NQ + NKV) * D + g * D:
                                                                   (NQ + NKV) * D + (g + 1) * D])))
                want = textbook_attention(roped(qkv[t, h * D:(h + 1) * D], pos), np.array(keys, np.float64),
                                          np.array(vals, np.float64), scale)
                np.testing.assert_allclose(out[t, h * D:(h + 1) * D], want, rtol=1e-5, atol=1e-6)
    # the new rows went to their ring slots
    for s in range(2):
        for i in range(T):
            pos = p0s[s] + i
            assert np.array_equal(k2[0, table[s, pos >> 4], 0, pos & 15],
                                  to_bf_array(roped(qkv[s * T + i, NQ * D:NQ * D + D], pos).astype(np.float32)))


# ---------------------------------------------------------------------- attention extras
def extras_case(seed=3, T=3, p0=40):
    rng = np.random.default_rng(seed)
    c = dict(T=T, p0=p0)
    c["table"] = np.array([[0, 1, 2, 3]], np.uint32)
    c["k"] = to_bf_array(rng.normal(0, 1, (1, 4, NKV, 16, D)))
    c["v"] = to_bf_array(rng.normal(0, 1, (1, 4, NKV, 16, D)))
    c["qkv"] = rng.normal(0, 1, (T, W)).astype(np.float32)
    c["meta"] = np.array([[0, p0 + i] for i in range(T)], np.uint32).reshape(-1)
    c["vis"] = np.array([(2 << i) - 1 for i in range(T)], np.uint32)
    c["rope"] = O.rope_table((500000.0 ** (-2.0 * np.arange(32) / 64)).astype(np.float32), 64)
    c["kv"] = L.KvArgs(1, 0, 0, 1, 4, 4, 4, 0)
    c["args"] = L.AttnArgs(32, 4, 0.125 * np.log2(np.e), 1, 0, 0, 0, 0, 0)
    c["x"] = rng.normal(0, 1, (T, SH.hidden)).astype(np.float32)
    c["inv"] = (1.0 / np.sqrt((c["x"].astype(np.float64) ** 2).mean(1) + L.RMS_EPS)).astype(np.float32)
    c["tokens"] = rng.integers(0, SH.vocab, T).astype(np.uint32)
    c["value_embed"] = to_bf_array(rng.normal(0, 1, (SH.vocab, NKV * D)))
    return c


def run_case(c, qkv=None, **extras):
    k, v = c["k"].copy(), c["v"].copy()
    ex = None
    if extras:
        ex = dict(x=c["x"], inv=c["inv"], tokens=c["tokens"], value_embed=c["value_embed"], **extras)
    out = O.attn_verify(L, SH, c["qkv"] if qkv is None else qkv, c["meta"], k, v, c["table"], c["rope"], c["kv"],
                        c["args"], np.array([0, c["T"]], np.uint32), c["vis"], extras=ex)
    return out, k, v


def test_value_embedding_reduces_to_shifted_values():
    """With a zero ve_gate the gate is 2 sigmoid(0) = 1, so the layer equals the plain one on
    values V + value_embed[token] (float32 sums); with a one-hot gate (c at input 5 of kv head 1)
    head 1's values get 2 sigmoid(c x[5] / rms(x)) value_embed, head 0's the plain 1x."""
    c = extras_case()
    T, VO = c["T"], (NQ + NKV) * D
    ve_rows = O.bf16_to_f32(c["value_embed"][c["tokens"]])  # [T][NKV * D]
    shifted = c["qkv"].copy()
    shifted[:, VO:] = (shifted[:, VO:] + ve_rows).astype(np.float32)
    plain, k0, v0 = run_case(c, qkv=shifted)
    got, k1, v1 = run_case(c, ve_gate=np.zeros((NKV, 12), np.float32))
    assert np.array_equal(got, plain) and np.array_equal(v1, v0) and np.array_equal(k1, k0)
    gate = np.zeros((NKV, 12), np.float32)
    gate[1, 5] = 1.7
    g1 = 2.0 / (1.0 + np.exp(-(1.7 * c["x"][:, 5].astype(np.float64) * c["inv"])))
    shifted = c["qkv"].copy()
    shifted[:, VO:VO + D] = (c["qkv"][:, VO:VO + D] + ve_rows[:, :D]).astype(np.float32)
    shifted[:, VO + D:] = (c["qkv"][:, VO + D:].astype(np.float64) + g1[:, None] * ve_rows[:, D:]).astype(np.float32)
    plain, _, v0 = run_case(c, qkv=shifted)
    got, _, v1 = run_case(c, ve_gate=gate)
    np.testing.assert_allclose(got, plain, rtol=1e-6, atol=1e-7)
    diff = np.abs(O.bf16_to_f32(v1).astype(np.float64) - O.bf16_to_f32(v0))
    assert diff.max() <= np.abs(O.bf16_to_f32(v0)).max() * 2.0 ** -7  # one bf16 step at most


def test_xsa_removes_the_value_direction():
    """xsa = 1: each head's output is orthogonal to its token's new value row of its kv head
    (head h uses kv head h // 2); xsa = 0 is the plain output; the output is linear in xsa
    and moves only along that direction."""
    c = extras_case(seed=4)
    T, VO = c["T"], (NQ + NKV) * D
    plain, _, _ = run_case(c)
    zero, _, _ = run_case(c, xsa=np.zeros(NQ, np.float32))
    one, _, _ = run_case(c, xsa=np.ones(NQ, np.float32))
    half, _, _ = run_case(c, xsa=np.full(NQ, 0.5, np.float32))
    assert np.array_equal(zero, plain)
    np.testing.assert_allclose(half, (zero.astype(np.float64) + one) / 2, rtol=1e-5, atol=1e-6)
    for t in range(T):
        for h in range(NQ):
            g = h // (NQ // NKV)
            v = c["qkv"][t, VO + g * D:VO + (g + 1) * D].astype(np.float64)
            u = v / np.linalg.norm(v)
            o1 = one[t, h * D:(h + 1) * D].astype(np.float64)
            o0 = plain[t, h * D:(h + 1) * D].astype(np.float64)
            assert abs(o1 @ u) < 1e-5 * (1 + np.linalg.norm(o0))
            np.testing.assert_allclose(o0 - o1, (o0 @ u) * u, rtol=1e-4, atol=1e-6)


def test_attention_gate_scales_each_head():
    """attn_gate row h = c e_50 scales head h's output by 2 sigmoid(c x[50] / rms(x)) (dims of x
    up to head_dim count, so input 50 is beyond the value-embedding gate's 12)."""
    c = extras_case(seed=5)
    plain, _, _ = run_case(c)
    gate = np.zeros((NQ, D), np.float32)
    cs = [0.0, 0.9, -1.3, 2.2]
    for h in range(NQ):
        gate[h, 50] = cs[h]
    got, _, _ = run_case(c, attn_gate=gate)
    for h in range(NQ):
        f = 2.0 / (1.0 + np.exp(-(cs[h] * c["x"][:, 50].astype(np.float64) * c["inv"])))
        np.testing.assert_allclose(got[:, h * D:(h + 1) * D], plain[:, h * D:(h + 1) * D] * f[:, None], rtol=1e-6,
                                   atol=1e-7)


# -------------------------------------------------------------------------------- MUDD
def gelu(x):
    return 0.5 * x * (1.0 + math.erf(x / math.sqrt(2.0)))


def test_mudd_bias_only_and_one_hot_cases():
    """dense1 = 0: inner = gelu(0) = 0, so each mix is its bias: out_attn = b0 tap0 + b1 tap1 +
    b2 cur, out_base = b3 tap0 + b4 tap1 + b5 cur. One-hot dense1 rows (row j = a_j e_k_j) and
    one-hot mix weights (row i takes inner j_i with weight m_i): w_i = m_i gelu(a_j cur[k_j] /
    rms(cur)) + b_i, against math.erf."""
    rng = np.random.default_rng(7)
    n, H = 3, 256
    cur, tap0, tap1 = (rng.normal(0, 1, (n, H)).astype(np.float32) for _ in range(3))
    bias = np.array([0.3, -0.2, 1.1, 0.05, 0.7, 0.9])
    mix = np.zeros((2, 3, 33), np.float32)
    mix.reshape(6, 33)[:, 32] = bias
    oa, ob = O.mudd(cur, tap0, tap1, np.zeros((32, H), np.float32), mix)
    c64 = [a.astype(np.float64) for a in (tap0, tap1, cur)]
    np.testing.assert_allclose(oa, bias[0] * c64[0] + bias[1] * c64[1] + bias[2] * c64[2], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(ob, bias[3] * c64[0] + bias[4] * c64[1] + bias[5] * c64[2], rtol=1e-6, atol=1e-6)
    dense1 = np.zeros((32, H), np.float32)
    ks, a = [3, 77, 200, 5, 128, 255], [1.5, -0.8, 2.0, 0.4, -1.1, 0.9]
    js = [0, 7, 13, 21, 30, 31]
    mw = [0.5, -1.2, 0.8, 2.0, -0.3, 1.0]
    for i in range(6):
        dense1[js[i], ks[i]] = a[i]
        mix.reshape(6, 33)[i, js[i]] = mw[i]
    oa, ob = O.mudd(cur, tap0, tap1, dense1, mix)
    inv = 1.0 / np.sqrt((cur.astype(np.float64) ** 2).mean(1) + L.RMS_EPS)
    for t in range(n):
        w = [mw[i] * gelu(a[i] * cur[t, ks[i]] * inv[t]) + bias[i] for i in range(6)]
        np.testing.assert_allclose(oa[t], w[0] * c64[0][t] + w[1] * c64[1][t] + w[2] * c64[2][t], rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(ob[t], w[3] * c64[0][t] + w[4] * c64[1][t] + w[5] * c64[2][t], rtol=1e-6, atol=1e-6)


# ------------------------------------------------------------------- the whole layer stack
def test_limite_layout_is_the_references():
    local, ve, sites, taps = limite_layout(48)
    assert [i for i in range(48) if not local[i]] == list(range(3, 48, 4))
    assert [i for i in range(48) if ve[i]] == list(range(1, 48, 3))
    assert sites == (24, 47) and taps == (11, 22)


def limite_model(n_layers=8, window=24, seed=9):
    shape = ModelShape(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=256, vocab=512, vocab_real=500,
                       n_layers=n_layers)
    model = SyntheticModel.generate(shape, seed=seed, device="cpu", std=0.1)
    return shape, model.with_extras(generate_extras(shape, seed=seed + 1, window=window))


def oracle_engine(shape, model, *, max_seq_len=256):
    emb, lay, sc = O.host_weights(model)
    return O.OracleEngine(L, shape, emb, lay, sc, max_seqs=1, max_seq_len=max_seq_len, kv_tokens=max_seq_len,
                          freq=rope_freq(500000.0, 64), extras=O.host_extras(model), max_step_tokens=64)


def test_limite_chunk_equals_token_by_token():
    """On a Limite-layout model (8 layers: 6 sliding-window layers of 24 keys, value embeddings
    on layers 1, 4, 7, MUDD before layers 4 and 7 with taps after 2 and 3): a 60-row prompt
    chunk on 23 cached tokens leaves the same caches (global pages and local rings) and the same
    last-row logits as feeding it one token per step; 40 more single-token steps past the ring's
    96 keys (it wraps) stay equal, bit for bit."""
    shape, model = limite_model()
    engines = [oracle_engine(shape, model) for _ in range(2)]
    assert engines[0].ring_pages == 6 and int(engines[0].local.sum()) == 6
    rng = np.random.default_rng(6)
    kg = rng.integers(0x3C00, 0x4000, engines[0].k.shape, dtype=np.uint16)
    kl = rng.integers(0x3C00, 0x4000, engines[0].k_local.shape, dtype=np.uint16)
    prompt = [int(x) for x in rng.integers(0, 500, 60)]
    for e in engines:
        s = e.new_seq()
        e.bench_fill(s, 23)
        e.k[...], e.v[...] = kg, kg ^ np.uint16(0x8000)
        e.k_local[...], e.v_local[...] = kl, kl ^ np.uint16(0x8000)
    ids_a, logits_a, _, _ = engines[0].step([(0, prompt, False, 1)])
    for t in prompt:
        ids_b, logits_b, _, _ = engines[1].step([(0, [t], False, 1)])
    assert np.array_equal(logits_a[-1], logits_b[-1]) and ids_a[-1] == ids_b[-1]
    for _ in range(40):
        nxt = [int(ids_a[-1])]
        ids_a, logits_a, _, _ = engines[0].step([(0, nxt, False, 1)])
        ids_b, logits_b, _, _ = engines[1].step([(0, nxt, False, 1)])
        assert np.array_equal(logits_a, logits_b)
    assert engines[0].seq_len[0] == 123
    for arr in ("k", "v", "k_local", "v_local"):
        assert np.array_equal(getattr(engines[0], arr), getattr(engines[1], arr)), arr


@pytest.mark.parametrize("part", ["window", "mudd", "value_embed", "xsa", "gate"])
def test_limite_each_extra_is_live(part):
    """Each extra changes the logits once the context is past the window (a guard against an
    extra that is read but never applied): the model without it differs by more than 1e-3."""
    shape, model = limite_model()
    x = model.extras
    y = type(x)(list(x.local), x.window, list(x.attn_gate), list(x.ve_gate), list(x.xsa), x.value_embed,
                x.mudd_dense1, x.mudd_mix, x.mudd_layer, x.mudd_tap)
    if part == "window":
        y.local = [0] * len(x.local)
    elif part == "mudd":
        y.mudd_layer, y.mudd_tap = (), ()
    elif part == "value_embed":
        y.ve_gate = [None] * len(x.ve_gate)
    elif part == "xsa":
        y.xsa = [None] * len(x.xsa)
    else:
        y.attn_gate = [None] * len(x.attn_gate)
    rng = np.random.default_rng(3)
    prompt = [int(t) for t in rng.integers(0, 500, 50)]
    outs = []
    for m in (model, model.with_extras(y)):
        e = oracle_engine(shape, m)
        e.new_seq()
        _, lg, _, _ = e.step([(0, prompt, False, 1)])
        outs.append(lg[-1][:500])
    assert np.abs(outs[0] - outs[1]).max() > 1e-3


def test_limite_lossless_speculation():
    """bench_spec.rs:119-139 on the Limite-layout model: greedy verification with replayed drafts
    (30 % wrong) emits exactly the plain-decode tokens, through the window and the ring's wrap."""
    shape, model = limite_model()

    def engine():
        e = oracle_engine(shape, model)
        s = e.new_seq()
        e.step([(s, [int(t) for t in np.random.default_rng(4).integers(0, 500, 30)], False, 0)])
        e.feed[s * 16] = 5
        return e, s

    plain, s = engine()
    trace = [5]
    for _ in range(90):
        ids, _, em, _ = plain.step([(s, [L.FEED_ROW], False)])
        trace.append(int(ids[0]))
    spec, s = engine()
    rng = np.random.default_rng(2)
    got = [5]
    while len(got) < 85:
        pos = len(got) - 1
        drafts = [trace[pos + i] if rng.random() > 0.3 else (trace[pos + i] + 1) % 500 for i in range(1, 5)]
        ids, _, em, _ = spec.step([(s, [L.FEED_ROW] + drafts, True)])
        got += [int(t) for t in ids[: em[0]]]
    assert got[:85] == trace[:85]
