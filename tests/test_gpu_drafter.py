"""GPU parity of the drafter's pass (engine/src/engine/drafter.rs:278-447 with kernels.metal:135-148,
1725-1934) against the oracle (orc_draft, pinned against a float64 restatement of
tools/spec/drafter.py in test_oracle_drafter.py).

Each step runs on the GPU first; the oracle then runs the same step on the GPU's tapped rows (so
the drafter is checked on its own inputs, the target's taps separately), and:
  - the target's logits and ids, and the taps (bf16 of the normed layer outputs), agree;
  - the drafter's raw logits agree within the logit tolerance;
  - the candidates and their probabilities equal draft_top over the GPU's own logits, and the
    slots' next feed and tree equal draft_tree over those (integer and fp32-compare work:
    bit-exact);
  - the drafter's rings (context keys and values of every on-path token, cyclic pages) agree.
The oracle then takes the GPU's trees, so the next step verifies the same drafts on both sides.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from conftest import banner
from helpers import bf16_bits, close, greedy_ids_match
from test_gpu_limite import LOGIT_ATOL, LOGIT_RTOL, build_limite_pair
from test_gpu_step import dev_u32, put_u32
from violetto import _lib as L
from violetto.drafter import SyntheticDrafter
from violetto.model import ModelShape

pytestmark = pytest.mark.gpu


def ring_close(eng, ref) -> None:
    kd, vd, tab = eng.draft_rings()
    assert np.array_equal(tab.cpu().numpy().view(np.uint32), ref.d_table), "drafter tables differ"
    for name, dev_t, host in (("K", kd, ref.dk), ("V", vd, ref.dv)):
        got = oracle.bf16_to_f32(dev_t.view(torch.int16).cpu().numpy().view(np.uint16))
        want = oracle.bf16_to_f32(host)
        bad = ~(np.abs(got - want) <= 2 ** -7 * np.abs(want) + 2e-3)
        if bad.any():
            idx = np.argwhere(bad)
            raise AssertionError(f"drafter ring {name}: {bad.sum()} values off; first {idx[0].tolist()}: "
                                 f"{got[tuple(idx[0])]} != {want[tuple(idx[0])]}")


def draft_step(eng, ref, d, runs, slots, what, flags=L.STEP_DRAFT):
    res = eng.step(runs, flags=flags, logits=True)
    n = res.info.n_tokens
    gpu_taps = [t.cpu().numpy().copy() for t in eng.draft_taps(n)]
    ids_r, logits_r, em_r, extra = ref.step(runs, draft=bool(flags & L.STEP_DRAFT), taps=gpu_taps)
    close(res.logits, logits_r, LOGIT_ATOL, LOGIT_RTOL, f"{what} target logits")
    greedy_ids_match(res.ids, ids_r, logits_r)
    same = np.array_equal(res.ids, ids_r)
    for k, (g, w) in enumerate(zip(gpu_taps, extra["taps"])):
        bad = ~(np.abs(g - w) <= 2 ** -7 * np.abs(w) + 2e-3)
        assert not bad.any(), f"{what} tap {k}: {bad.sum()} values off"
    close(eng.draft_context(n).cpu().numpy(), extra["ctx"], 2e-3, 2e-3, f"{what} context")
    blocks, tin = extra["blocks"], extra["draft_tin"]
    rows = len(tin) if len(blocks) else 0
    if rows:
        got = eng.draft_logits(rows).cpu().numpy()
        close(got, extra["draft_logits"], LOGIT_ATOL, LOGIT_RTOL, f"{what} draft logits")
        err = np.abs(got.astype(np.float64) - extra["draft_logits"]).max()
        print(f"  {what}: {len(blocks)} blocks, {rows} rows, draft logits max-abs err {err:.3e}", flush=True)
        ncand = min(L.DRAFT_CANDS, int(blocks[:, 1].max()) - 1)
        if ncand > 0:
            cand, cand_q = (t.cpu().numpy() for t in eng.draft_candidates(rows))
            cand = cand.view(np.uint32)
            want_c, want_q = oracle.draft_top(got, d.vocab.cpu().numpy().astype(np.uint32), tin.reshape(-1), d.inv_temperature,
                                              ncand)
            drafted = tin[:, 1] > 0
            assert np.array_equal(cand[drafted, :ncand], want_c[drafted, :ncand]), f"{what} candidates"
            assert np.array_equal(cand_q[drafted, :ncand], want_q[drafted, :ncand]), f"{what} candidate probabilities"
            feed, tree = ref.feed.copy(), ref.tree.copy()
            oracle.draft_tree(blocks.reshape(-1), tin.reshape(-1), want_c, want_q, feed, tree, ncand)
            S = ref.max_seqs
            gfeed, gtree = dev_u32(eng, "d_feed", (S * 16,)), dev_u32(eng, "d_tree", (S * 16,))
            for s in {int(x) for x in tin[:, 0]}:
                r = blocks[[int(tin[int(b[0]), 0]) == s for b in blocks]][0][1]
                assert gfeed[s * 16] == ref.feed[s * 16], f"{what} slot {s} bonus token"
                assert np.array_equal(gfeed[s * 16:s * 16 + r], feed[s * 16:s * 16 + r]), f"{what} slot {s} feed"
                assert np.array_equal(gtree[s * 16:s * 16 + r], tree[s * 16:s * 16 + r]), f"{what} slot {s} tree"
            # the next step verifies the GPU's drafts on both sides
            ref.feed[:], ref.tree[:] = gfeed, gtree
    if same:
        assert np.array_equal(res.emitted, em_r), f"{what} emitted {res.emitted} != {em_r}"
        ring_close(eng, ref)
    return same, res


@pytest.mark.parametrize("which", ["cfg", "ref"])
def test_drafter_steps(gpu, which):
    """A Limite-layout target of 8 layers, two sequences 150 and 201 tokens in, and a 2-layer
    drafter (convolutions, inject, a head in int8 groups of 8 as export.py writes it, window
    48 so its rings of 112 positions wrap) tapping layers 2 and 7: a prompt chunk of 24 rows per
    sequence that drafts blocks of 4 and 3 rows, then verify steps of those trees that draft
    again. cfg: hidden 512, 8 query heads of 64 over 2 kv heads (runs of 16 rows); ref: the
    reference's head layout, 10 query heads of 128 over 2 (runs of 12)."""
    if which == "cfg":
        shape = ModelShape(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=512, vocab=1024, vocab_real=1000,
                           n_layers=8)
    else:
        shape = ModelShape(hidden=1280, n_heads=10, n_kv_heads=2, head_dim=128, ffn=1280, vocab=1024,
                           vocab_real=1000, n_layers=8)
    banner(f"drafter steps {which}")
    model, gm, eng, ref, slots, rng = build_limite_pair(shape, window=48, ctx=[150, 201], n_seqs=2, seed=31,
                                                        max_seq_len=512, max_head_rows=32)
    d = SyntheticDrafter.generate(shape, n_layers=2, taps=(2, 7), v=512, window=48, seed=4, device="cpu")
    eng.set_drafter(d.to("cuda"))
    ref.set_drafter(d, max_step_tokens=eng.cfg.max_step_tokens)
    rows = {slots[0]: 4, slots[1]: 3}
    for s, r in rows.items():
        eng.set_draft_rows(s, r)
        ref.draft_rows[s] = r
    prompt = [[int(t) for t in rng.integers(0, shape.vocab_real, 24)] for _ in slots]
    same, _ = draft_step(eng, ref, d, [(s, p, False, 1) for s, p in zip(slots, prompt)], slots, "chunk")
    assert same, "chunk step ids"
    compared = 1
    for step in range(5):
        runs = [(s, [L.FEED_ROW + i for i in range(rows[s])], True) for s in slots]
        same, res = draft_step(eng, ref, d, runs, slots, f"verify step {step}")
        if not same:
            break
        compared += 1
    assert compared >= 3, "too few steps compared"
    eng.close()


def test_drafter_context_without_blocks_and_refusals(gpu):
    """Without STEP_DRAFT the context still reaches the rings (so a later drafted step sees it);
    a slot without draft rows gets no block; more rows than an attention run, a tap past the
    target's layers, and a drafter matrix in int8 groups of 8 are refused."""
    shape = ModelShape(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=512, vocab=1024, vocab_real=1000,
                       n_layers=4)
    banner("drafter context and refusals")
    model, gm, eng, ref, slots, rng = build_limite_pair(shape, window=48, ctx=[40, 60], n_seqs=2, seed=8,
                                                        max_seq_len=256, max_head_rows=32)
    bad = SyntheticDrafter.generate(shape, n_layers=1, taps=(1, 4), v=256, window=48, seed=1, device="cuda")
    with pytest.raises(L.SvError):
        eng.set_drafter(bad)
    bad = SyntheticDrafter.generate(shape, n_layers=1, taps=(1, 2), v=256, window=48, seed=1, device="cuda", group=8)
    with pytest.raises(L.SvError):
        eng.set_drafter(bad)
    d = SyntheticDrafter.generate(shape, n_layers=1, taps=(1, 2), v=256, window=48, seed=2, device="cpu",
                                  convs=False, inject=False, head_group=None)
    eng.set_drafter(d.to("cuda"))
    ref.set_drafter(d, max_step_tokens=eng.cfg.max_step_tokens)
    with pytest.raises(L.SvError):
        eng.set_draft_rows(slots[0], 17)
    prompt = [[int(t) for t in rng.integers(0, shape.vocab_real, 10)] for _ in slots]
    same, _ = draft_step(eng, ref, d, [(s, p, False, 1) for s, p in zip(slots, prompt)], slots, "context only", flags=0)
    assert same
    eng.set_draft_rows(slots[1], 5)
    ref.draft_rows[slots[1]] = 5
    runs = [(s, [L.FEED_ROW], False, 1) for s in slots]
    same, _ = draft_step(eng, ref, d, runs, slots, "one slot drafted")
    assert same
    eng.close()


@pytest.mark.parametrize("hidden,rows", [(512, 7), (1280, 12)])
def test_draft_conv_and_tap_rows_kernels(gpu, hidden, rows):
    """sv_draft_conv (kernels.metal:1820-1836, the corrections given) and sv_tap_rows
    (kernels.metal:135-148) through the C ABI against the oracle: two blocks (rows 0..2 and
    3..rows-1), with and without the residual."""
    import ctypes as C

    banner(f"draft_conv / tap_rows kernels hidden {hidden}")
    rng = np.random.default_rng(hidden + rows)
    cw = -(-(hidden // 8) // 64) * 64
    x = rng.normal(0, 1, (rows, hidden)).astype(np.float32)
    corr = rng.normal(0, 0.1, (rows, cw)).astype(np.float32)
    base = np.stack([1 + rng.normal(0, 0.1, hidden), rng.normal(0, 0.1, hidden)]).astype(np.float32)
    resid = rng.normal(0, 1, (rows, hidden)).astype(np.float32)
    tin = np.array([[0, i] for i in range(3)] + [[1, i] for i in range(rows - 3)], np.uint32)
    lib = L.lib()
    dev = {k: torch.from_numpy(v.view(np.int32) if v.dtype == np.uint32 else v).cuda()
           for k, v in dict(x=x, corr=corr, base=base, resid=resid, tin=tin).items()}
    for with_resid in (False, True):
        out = torch.zeros_like(dev["x"])
        L.check(lib.sv_draft_conv(None, dev["x"].data_ptr(), dev["corr"].data_ptr(), cw, dev["base"].data_ptr(),
                                  dev["tin"].data_ptr(), dev["resid"].data_ptr() if with_resid else None,
                                  out.data_ptr(), rows, hidden))
        torch.cuda.synchronize()
        want = np.zeros_like(x)
        O = oracle
        O.lib().orc_draft_conv(O.ptr(x), O.ptr(corr), C.c_uint32(cw), O.ptr(base), O.ptr(tin),
                               O.ptr(resid) if with_resid else None, O.ptr(want), C.c_uint32(rows), C.c_uint32(hidden))
        close(out.cpu().numpy(), want, 1e-5, 1e-5, f"draft_conv resid={with_resid}")
    taps = torch.zeros_like(dev["x"])
    L.check(lib.sv_tap_rows(None, dev["x"].data_ptr(), taps.data_ptr(), rows, hidden))
    torch.cuda.synchronize()
    want = np.zeros_like(x)
    oracle.lib().orc_tap_rows(oracle.ptr(x), oracle.ptr(want), C.c_uint32(rows), C.c_uint32(hidden))
    got = taps.cpu().numpy()
    # bf16 values: equal, or one bf16 step apart where fp32 and float64 norms round differently
    assert (np.abs(got - want) <= np.abs(want) * 2.0 ** -8).all()
    assert (got == want).mean() > 0.99


def test_drafter_from_weight_file(gpu, tmp_path):
    """The same drafter served from its weight file (export.py's names, uploaded through
    sv_weights_*; VltDrafter) and from memory drafts the same blocks: raw logits, candidates and
    trees bit-identical over a prompt step and two verify steps."""
    from violetto.drafter import VltDrafter, drafter_tensors
    from violetto.weights import WeightFile, write_vlt

    shape = ModelShape(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=512, vocab=1024, vocab_real=1000,
                       n_layers=4)
    banner("drafter from weight file")
    d = SyntheticDrafter.generate(shape, n_layers=2, taps=(1, 3), v=256, window=48, seed=6, device="cpu")
    path = tmp_path / "drafter.vlt"
    write_vlt(path, drafter_tensors(d))
    wf = WeightFile(path)
    wf.upload()
    results = []
    for source in ("memory", "file"):
        model, gm, eng, ref, slots, rng = build_limite_pair(shape, window=48, ctx=[40, 60], n_seqs=2, seed=12,
                                                            max_seq_len=256, max_head_rows=32)
        eng.set_drafter(d.to("cuda") if source == "memory" else VltDrafter(wf, shape))
        for s in slots:
            eng.set_draft_rows(s, 4)
        out = []
        prompt = [[int(t) for t in rng.integers(0, shape.vocab_real, 10)] for _ in slots]
        eng.step([(s, p, False, 1) for s, p in zip(slots, prompt)], flags=L.STEP_DRAFT)
        out.append(eng.draft_logits(8).cpu().numpy().copy())
        for _ in range(2):
            eng.step([(s, [L.FEED_ROW + i for i in range(4)], True) for s in slots], flags=L.STEP_DRAFT)
            out.append(eng.draft_logits(8).cpu().numpy().copy())
            out.append(dev_u32(eng, "d_feed", (2 * 16,)))
            out.append(dev_u32(eng, "d_tree", (2 * 16,)))
        results.append(out)
        eng.close()
    for a, b in zip(*results):
        np.testing.assert_array_equal(a, b)


def test_drafter_reference_shape(gpu):
    """The reference drafter's own shape (tools/spec/drafter.py: hidden 1280, 10 x 128 query heads
    over 2 kv heads, ffn 3328, 2 layers, window 1024, blocks of 8 rows; export.py: int8 groups of
    64, a 16384-id head in groups of 8) on a 4-layer target of the reference's dimensions
    (vocabulary 151680), two sequences 1500 and 1100 tokens in with the drafter's rings filled
    (1088 positions a slot: wrapped) and the window crossing them: a prompt step and three verify
    steps of the drafter's trees, against the oracle as in test_drafter_steps."""
    import dataclasses

    from violetto.model import REFERENCE_SHAPE

    shape = dataclasses.replace(REFERENCE_SHAPE, n_layers=4)
    banner("drafter at the reference shape")
    model, gm, eng, ref, slots, rng = build_limite_pair(shape, window=1024, ctx=[1500, 1100], n_seqs=2, seed=41,
                                                        max_seq_len=1700, max_head_rows=32, group=64)
    d = SyntheticDrafter.generate(shape, n_layers=2, taps=(1, 3), v=16384, window=1024, seed=9, device="cpu")
    eng.set_drafter(d.to("cuda"))
    ref.set_drafter(d, max_step_tokens=eng.cfg.max_step_tokens)
    kd, vd, _ = eng.draft_rings()
    assert kd.shape == ref.dk.shape
    for dev_t, host in ((kd, ref.dk), (vd, ref.dv)):
        bits = bf16_bits(rng.normal(0, 1, host.shape).astype(np.float32))
        host[...] = bits
        dev_t.copy_(torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16))
    torch.cuda.synchronize()
    for s in slots:
        eng.set_draft_rows(s, 8)
        ref.draft_rows[s] = 8
    prompt = [[int(t) for t in rng.integers(0, shape.vocab_real, 6)] for _ in slots]
    same, _ = draft_step(eng, ref, d, [(s, p, False, 1) for s, p in zip(slots, prompt)], slots, "prompt")
    assert same, "prompt step ids"
    compared = 1
    for step in range(3):
        runs = [(s, [L.FEED_ROW + i for i in range(8)], True) for s in slots]
        same, _ = draft_step(eng, ref, d, runs, slots, f"verify step {step}")
        if not same:
            break
        compared += 1
    assert compared >= 3, "too few steps compared"
    eng.close()
