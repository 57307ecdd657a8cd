"""sv_step_capture (Engine::step_capture, engine/src/engine.rs:318-355): every layer's
intermediates against the oracle's capture of the same step (plain and Limite-layout models, a
prompt chunk and verify chains), and the capture step itself against sv_step on a twin engine
(ids, logits, emitted counts and lengths bit-identical: capturing only adds reads and writes
beside the step's own kernels)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import banner
from test_gpu_limite import build_limite_pair
from test_gpu_step import build_pair, compare_step
from violetto import _lib as L
from violetto.model import LayerScalars, ModelShape

pytestmark = pytest.mark.gpu

FIELDS = ("resid_in", "attn_in", "qkv", "sdpa_out", "attn_out", "mlp_in", "mlp_out", "resid_base")
# Each field within a fraction of its largest magnitude in the layer. fp32 activations against
# the oracle's float64 math (int8 x bf16 hi + lo products, fp32 sums in another order): observed
# below 1e-4 everywhere but in the attention output and o's product of it, which also carry the
# step's own new keys and values: rounded to bf16 from fp32 where the oracle rounds from float64,
# an element near a rounding boundary lands one ulp apart (observed up to 1.5e-3 and 9.4e-4 over
# 8 Limite layers; the attention kernel alone, on identical cache bits, is within 2e-4).
REL_TOL = {"sdpa_out": 3e-3, "attn_out": 3e-3}
REL_TOL_OTHER = 5e-4
# At the reference model's layer shape (1280 hidden, five query heads of 128 per kv head) those
# one-ulp K/V differences move every field about ten times as much: observed up to 2.6e-3 in the
# attention output and 5.0e-4 in later fields over 8 layers.
REF_TOL_OTHER = 1e-3


def compare_capture(got, want, what, tol_other=REL_TOL_OTHER):
    assert [c.layer for c in got] == list(range(len(want))), f"{what}: layers out of order"
    worst = {}
    bad = []
    for c, w in zip(got, want):
        for name in FIELDS:
            a, b = getattr(c, name), w[name]
            if b is None:
                assert a is None, f"{what} layer {c.layer}: {name} on a layer without MUDD"
                continue
            assert a is not None and a.shape == b.shape, f"{what} layer {c.layer}: {name} shape"
            scale = max(float(np.abs(b).max()), 1e-6)
            err = float(np.abs(a.astype(np.float64) - b).max()) / scale
            worst[name] = max(worst.get(name, 0.0), err)
            if err > REL_TOL.get(name, tol_other):
                bad.append(f"layer {c.layer}: {name} off by {err:.2e} of its scale")
    print(f"  {what}: worst error of scale per field " + ", ".join(f"{k} {v:.1e}" for k, v in worst.items()), flush=True)
    assert not bad, f"{what}: " + "; ".join(bad)


def captured_step(eng, ref, runs, slots, what, tol_other=REL_TOL_OTHER):
    got = []
    res = eng.step_capture(runs, got.append, logits=True)
    ids_r, logits_r, em_r, extra_r = ref.step(runs, capture=True)
    if eng.__dict__.get("_diverged"):
        # an earlier step's id differed where the oracle's margin is within the logits tolerance:
        # the sequences no longer hold the same tokens
        print(f"  {what}: capture not compared (slots {sorted(eng._diverged)} diverged)", flush=True)
    else:
        compare_capture(got, extra_r["capture"], what, tol_other)
    compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots, runs=runs)


def test_capture_against_oracle_plain(gpu):
    """3 layers with distinct residual scalars; two sequences 700 and 1300 tokens in: a prompt
    chunk of 20 rows on one beside a 5-row verify run on the other, then two verify steps."""
    banner("step_capture vs oracle: plain model")
    shape = ModelShape(n_layers=3, vocab=4096, vocab_real=4000)
    scal = [LayerScalars(1.0, 0.9, 0.8, 1.3, 1.1, 0.7), LayerScalars(1.2, 1.1, 1.05, 0.6, 0.95, 1.4),
            LayerScalars(0.8, 1.0, 1.0, 1.0, 0.5, 1.2)]
    model, gm, eng, ref, slots, rng = build_pair(shape, ctx=[700, 1300], n_seqs=2, seed=31, scalars=scal,
                                                 max_seq_len=1400)
    for s in slots:
        t = int(rng.integers(0, shape.vocab_real))
        eng.set_feed(s, ref.seq_len[s], t)
        ref.set_feed(s, ref.seq_len[s], t)
    prompt = [int(t) for t in rng.integers(0, shape.vocab_real, 20)]
    drafts = [int(t) for t in rng.integers(0, shape.vocab_real, 4)]
    captured_step(eng, ref, [(slots[0], prompt, False, 1), (slots[1], [L.FEED_ROW] + drafts, True)], slots, "mixed step")
    for step in range(2):
        runs = [(s, [L.FEED_ROW] + [int(t) for t in rng.integers(0, shape.vocab_real, 4)], True) for s in slots]
        captured_step(eng, ref, runs, slots, f"verify step {step}")
    eng.close()


def test_capture_against_oracle_limite(gpu):
    """The Limite layout (8 layers: window layers of 48 keys, value embeddings, gates, XSA, MUDD
    before layers 4 and 7, which report their residual base): a 24-row prompt chunk, then a
    verify step."""
    banner("step_capture vs oracle: Limite layout")
    shape = ModelShape(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=512, vocab=1024, vocab_real=1000,
                       n_layers=8)
    model, gm, eng, ref, slots, rng = build_limite_pair(shape, window=48, ctx=[150], seed=23, max_seq_len=512)
    s = slots[0]
    prompt = [int(t) for t in rng.integers(0, shape.vocab_real, 24)]
    captured_step(eng, ref, [(s, prompt, False, 1)], slots, "chunk")
    runs = [(s, [L.FEED_ROW] + [int(t) for t in rng.integers(0, shape.vocab_real, 4)], True)]
    captured_step(eng, ref, runs, slots, "verify step")
    eng.close()


def test_capture_against_oracle_reference_shape(gpu):
    """The reference model's own layer shape (hidden 1280, 10 query heads of 128 over 2 kv heads,
    ffn 3328) in the Limite layout over 8 layers: the capture's head_dim 128 kernels, five query
    heads per kv head (a 20-row prompt chunk runs as attention runs of 12 rows), then a verify
    step."""
    banner("step_capture vs oracle: reference layer shape")
    shape = ModelShape(hidden=1280, n_heads=10, n_kv_heads=2, head_dim=128, ffn=3328, vocab=1024, vocab_real=1000,
                       n_layers=8)
    model, gm, eng, ref, slots, rng = build_limite_pair(shape, window=48, ctx=[150], seed=29, max_seq_len=512)
    s = slots[0]
    prompt = [int(t) for t in rng.integers(0, shape.vocab_real, 20)]
    captured_step(eng, ref, [(s, prompt, False, 1)], slots, "chunk", tol_other=REF_TOL_OTHER)
    runs = [(s, [L.FEED_ROW] + [int(t) for t in rng.integers(0, shape.vocab_real, 4)], True)]
    captured_step(eng, ref, runs, slots, "verify step", tol_other=REF_TOL_OTHER)
    eng.close()


@pytest.mark.parametrize("options", [0, L.OPT_LAYERS_KERNEL])
def test_capture_step_equals_step(gpu, options):
    """Twin engines (same model, cache and feed): sv_step on one, sv_step_capture on the other,
    four 5-row verify steps: ids, logits, emitted counts and lengths bit-identical. With
    SV_OPT_LAYERS_KERNEL the capture engine runs the launch chain (the twin runs sv_step without
    the option)."""
    banner(f"step_capture equals step (options {options})")
    shape = ModelShape(n_layers=4, vocab=4096, vocab_real=4000)
    _, _, a, _, slots, rng = build_pair(shape, ctx=[1500], seed=12, max_seq_len=1600)
    _, _, b, _, _, _ = build_pair(shape, ctx=[1500], seed=12, max_seq_len=1600, options=options)
    s = slots[0]
    for e in (a, b):
        e.set_feed(s, 1500, 17)
    for step in range(4):
        run = [(s, [L.FEED_ROW] + [int(x) for x in rng.integers(0, shape.vocab_real, 4)], True)]
        layers = []
        ra, rb = a.step(run, logits=True), b.step_capture(run, layers.append, logits=True)
        assert len(layers) == shape.n_layers and all(c.n == 5 for c in layers)
        assert np.array_equal(ra.ids, rb.ids) and np.array_equal(ra.emitted, rb.emitted), f"step {step}"
        assert np.array_equal(ra.logits, rb.logits, equal_nan=True), f"step {step}: logits differ"
        assert a.seq_len(s) == b.seq_len(s)
    a.close()
    b.close()
