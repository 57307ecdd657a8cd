"""Pinning the oracle's per-layer capture (Engine::step_capture, engine/src/engine.rs:318-355,
LayerCapture :176-188) on the CPU, by relations the model fixes rather than by its own formulas:
rms-norms of the residuals it reports, unit-RMS query and key heads (the norm, then a rotation by
the RoPE table's rounded cos/sin, whose c^2 + s^2 is divided back out),
the residual mixes of encode.rs:172-185 over its raw products (and MUDD's base on the MUDD
layers), the next layer's input and the step's final hidden rows, and a lone first token whose
attention output is its own value rounded to bf16 (one key, weight 1)."""
from __future__ import annotations

import numpy as np

import oracle
from violetto import _lib as L
from violetto.model import LayerScalars, ModelShape, SyntheticModel, generate_extras, rope_freq

O = oracle


def rms(v):
    v = v.astype(np.float64)
    return v / np.sqrt((v ** 2).mean(-1, keepdims=True) + L.RMS_EPS)


def engine(shape, model, extras=None, max_seq_len=256):
    emb, lay, sc = O.host_weights(model)
    return O.OracleEngine(L, shape, emb, lay, sc, max_seqs=1, max_seq_len=max_seq_len, kv_tokens=max_seq_len,
                          freq=rope_freq(500000.0, shape.head_dim), attn_scale=0.125, extras=extras,
                          max_step_tokens=64)


SCAL = [LayerScalars(1.0, 0.9, 0.8, 1.3, 1.1, 0.7), LayerScalars(1.2, 1.1, 1.05, 0.6, 0.95, 1.4),
        LayerScalars(0.8, 1.0, 1.0, 1.0, 0.5, 1.2)]


def unit_rms_before_rope(v, cs, rope):
    """Mean square of each head vector v [n][heads][D] before its rotation: each pair (2j, 2j+1)
    was multiplied by the table's (c, s) at the token's position, which scales its squared norm
    by c^2 + s^2 (not exactly 1: the table holds rounded values)."""
    v = v.astype(np.float64)
    sq = v ** 2
    if rope:
        f = (cs.astype(np.float64) ** 2).sum(-1)  # [n][32]
        pairs = sq[..., :64].reshape(v.shape[0], v.shape[1], 32, 2).sum(-1) / f[:, None, :]
        return (pairs.sum(-1) + sq[..., 64:].sum(-1)) / v.shape[-1]
    return sq.mean(-1)


def check_layers(shape, model, caps, hidden, n, positions, rope_table, mudd_layers=()):
    H, D, NQ, NKV = shape.hidden, shape.head_dim, shape.n_heads, shape.n_kv_heads
    assert len(caps) == shape.n_layers
    for li, c in enumerate(caps):
        s = model.scalars[li]
        for name, w in (("resid_in", H), ("attn_in", H), ("qkv", (NQ + 2 * NKV) * D), ("sdpa_out", NQ * D),
                        ("attn_out", H), ("mlp_in", H), ("mlp_out", H)):
            assert c[name].shape == (n, w), (li, name)
        mudd = li in mudd_layers
        assert (c["resid_base"] is not None) == mudd
        if not mudd:
            np.testing.assert_allclose(c["attn_in"], rms(c["resid_in"]), rtol=1e-5, atol=1e-6)
        q = c["qkv"][:, :NQ * D].reshape(n, NQ, D)
        k = c["qkv"][:, NQ * D:(NQ + NKV) * D].reshape(n, NKV, D)
        cs = rope_table.reshape(-1, 32, 2)[positions]
        for v in (q, k):
            np.testing.assert_allclose(unit_rms_before_rope(v, cs, s.rope), 1.0, rtol=0, atol=1e-5)
        base = c["resid_base"] if mudd else c["resid_in"]
        mixed = s.resid_attn * base.astype(np.float64) + s.post_attn * c["attn_out"]
        np.testing.assert_allclose(c["mlp_in"], rms(mixed), rtol=1e-4, atol=1e-5)
        out = s.resid_mlp * mixed + s.post_mlp * c["mlp_out"]
        nxt = caps[li + 1]["resid_in"] if li + 1 < len(caps) else hidden
        np.testing.assert_allclose(nxt, out, rtol=1e-5, atol=1e-4 * np.abs(out).max())


def test_capture_relations_plain_model():
    """3 layers with distinct residual scalars, a 7-row prompt chunk on 40 cached tokens."""
    shape = ModelShape(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=256, vocab=512, vocab_real=500,
                       n_layers=3)
    model = SyntheticModel.generate(shape, seed=4, device="cpu", std=0.1, scalars=SCAL)
    e = engine(shape, model)
    s = e.new_seq()
    e.bench_fill(s, 40)
    rng = np.random.default_rng(2)
    e.k[...] = rng.integers(0x3C00, 0x4000, e.k.shape, dtype=np.uint16)
    e.v[...] = e.k ^ np.uint16(0x8000)
    toks = [int(t) for t in rng.integers(0, 500, 7)]
    _, _, _, x = e.step([(s, toks, False, 1)], want_hidden=True, capture=True)
    check_layers(shape, model, x["capture"], x["hidden"], 7, np.arange(40, 47), e.rope)


def test_capture_relations_limite_layout():
    """The Limite layout on 8 layers (window layers, value embeddings, XSA, gates, MUDD before
    layers 4 and 7): MUDD layers report their residual base, the others none."""
    shape = ModelShape(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=256, vocab=512, vocab_real=500,
                       n_layers=8)
    model = SyntheticModel.generate(shape, seed=9, device="cpu", std=0.1)
    model = model.with_extras(generate_extras(shape, seed=10, window=24))
    e = engine(shape, model, extras=O.host_extras(model))
    s = e.new_seq()
    rng = np.random.default_rng(5)
    toks = [int(t) for t in rng.integers(0, 500, 30)]
    _, _, _, x = e.step([(s, toks, False, 1)], want_hidden=True, capture=True)
    check_layers(shape, model, x["capture"], x["hidden"], 30, np.arange(30), e.rope,
                 mudd_layers=tuple(model.extras.mudd_layer))


def test_capture_lone_token_attends_to_itself():
    """A fresh sequence's first token sees one key, its own: the attention output of each query
    head is the value row of its kv head, rounded to bf16 as the cache holds it."""
    shape = ModelShape(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=256, vocab=512, vocab_real=500,
                       n_layers=2)
    model = SyntheticModel.generate(shape, seed=7, device="cpu", std=0.1)
    e = engine(shape, model)
    s = e.new_seq()
    _, _, _, x = e.step([(s, [123], False, 1)], capture=True)
    NQ, NKV, D = 4, 2, 64
    for c in x["capture"]:
        v = c["qkv"][0, (NQ + NKV) * D:].reshape(NKV, D)
        vb = O.bf16_to_f32(((v.view(np.uint32) + 0x7FFF + ((v.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16))
        sd = c["sdpa_out"][0].reshape(NQ, D)
        for h in range(NQ):
            np.testing.assert_allclose(sd[h], vb[h // (NQ // NKV)], rtol=1e-6, atol=0)
