"""The persistent layer kernel (silicon-violetto_amd/csrc/layers.hip): every decoder layer of a
1-8 row step in one launch. Checked against the oracle engine at the step bar (logits within
2e-2 / 1e-2, greedy ids where the margin allows, emitted counts, lengths and page tables
bit-exact), against the launch-per-kernel path on the same inputs, under graph replay, and its
bounded waits (a barrier forced from the host never to complete: every workgroup exits, the
step reports the error, the next step runs)."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

from conftest import banner
from test_gpu_step import build_pair, compare_step, dev_u32
from violetto import _lib as L
from violetto.model import ModelShape

pytestmark = pytest.mark.gpu


def layer_launches(eng) -> tuple[int, int]:
    """(layer kernel launches, qkv matmul launches) of one more profiled step of the plan."""
    prof = eng.profile_step(0, 1)
    return prof["layers"][1], prof["qkv"][1]


@pytest.mark.parametrize("n_layers,ctxs,rows", [
    (2, [1000], 5),       # 5 token slots, 2 column tiles (the configs[1] variant)
    (2, [2500], 1),       # plain decode: 4 token slots, 1 column tile, 21 splits
    (3, [700], 3),
    (2, [300, 900], 4),   # two runs, 8 rows
    (2, [600], 8),        # 8 rows, 32 columns per kv head
    (16, [8192], 5),      # configs[1]'s depth and context
])
def test_layers_kernel_steps(gpu, n_layers, ctxs, rows):
    banner(f"layer kernel steps: {n_layers} layers, contexts {ctxs}, {rows} rows per run")
    shape = ModelShape(n_layers=n_layers, vocab=4096, vocab_real=4000)
    model, gm, eng, ref, slots, rng = build_pair(shape, ctx=ctxs, n_seqs=len(ctxs), seed=21 + rows,
                                                 max_seq_len=max(ctxs) + 64, options=L.OPT_LAYERS_KERNEL)
    for s in slots:
        t = int(rng.integers(0, shape.vocab_real))
        eng.set_feed(s, ref.seq_len[s], t)
        ref.set_feed(s, ref.seq_len[s], t)
    for step in range(2 if n_layers > 8 else 3):
        runs = [(s, [L.FEED_ROW] + [int(x) for x in rng.integers(0, shape.vocab_real, rows - 1)], True) for s in slots]
        ids_r, logits_r, em_r, extra_r = ref.step(runs)
        res = eng.step(runs, logits=True)
        compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots, runs=runs)
    eng.plan(runs)
    assert layer_launches(eng) == (1, 0), "the step did not run on the persistent layer kernel"
    eng.close()


def test_layers_kernel_equals_launch_chain(gpu):
    """The same model and cache in two engines, one with the layer kernel and one with a launch
    per kernel (the default, without SV_OPT_LAYERS_KERNEL): four steps of 5 rows give logits within 1e-4 of each
    other, equal ids, emitted counts and lengths, and caches within one bf16 step."""
    banner("layer kernel vs launch chain")
    shape = ModelShape(n_layers=4, vocab=4096, vocab_real=4000)
    _, _, a, ref, slots, rng = build_pair(shape, ctx=[1500], seed=5, max_seq_len=1600, options=L.OPT_LAYERS_KERNEL)
    _, _, b, _, _, _ = build_pair(shape, ctx=[1500], seed=5, max_seq_len=1600)
    s = slots[0]
    for e in (a, b):
        e.set_feed(s, 1500, 17)
    for step in range(4):
        run = (s, [L.FEED_ROW] + [int(x) for x in rng.integers(0, shape.vocab_real, 4)], True)
        ra, rb = a.step([run], logits=True), b.step([run], logits=True)
        fin = np.isfinite(rb.logits)
        assert np.array_equal(fin, np.isfinite(ra.logits)), "-inf columns differ"
        d = float(np.abs(ra.logits[fin] - rb.logits[fin]).max())
        print(f"  step {step}: max |logits difference| {d:.2e}", flush=True)
        assert d <= 1e-4
        assert np.array_equal(ra.ids, rb.ids) and np.array_equal(ra.emitted, rb.emitted)
        assert a.seq_len(s) == b.seq_len(s)
    for (ka, va), (kb, vb) in ((a.kv_cache(), b.kv_cache()),):
        for x, y, what in ((ka, kb, "K"), (va, vb, "V")):
            xf, yf = x.float().cpu().numpy(), y.float().cpu().numpy()
            # one bf16 step of the value, or of 1/4 where RoPE's rotation cancels towards zero
            # (K rows are rms-normed: magnitude ~1)
            bad = np.abs(xf - yf) > 2 ** -7 * np.maximum(np.abs(yf), 0.25)
            assert not bad.any(), f"{what} caches differ at {np.argwhere(bad)[:4].tolist()}: {xf[bad][:4]} vs {yf[bad][:4]}"
    a.plan([run])
    b.plan([run])
    assert layer_launches(a) == (1, 0) and layer_launches(b)[0] == 0
    a.close()
    b.close()


def test_layers_kernel_graph_replay(gpu):
    """Captured once and replayed (as bench.py times it): a plain decode of 8 replays, then
    greedy verify steps drafted by the replay drafter (35% wrong) over the engine's own
    continuation, 5 replays; the same on an engine without the layer kernel. After every replay
    both engines' lengths, feeds and emitted counts are equal, and the verify steps reproduce
    the recorded continuation (the lossless property)."""
    banner("layer kernel graph replay")
    shape = ModelShape(n_layers=3, vocab=4096, vocab_real=4000)
    S, k, trace_n, steps, max_len = 1, 4, 8, 5, 1400
    _, _, a, _, slots, rng = build_pair(shape, ctx=[1100], seed=9, max_seq_len=max_len, options=L.OPT_LAYERS_KERNEL)
    _, _, b, _, _, _ = build_pair(shape, ctx=[1100], seed=9, max_seq_len=max_len)
    s = slots[0]
    engines = (a, b)
    for e in engines:
        e.set_feed(s, 1100, 33)
    runs1 = [(s, [L.FEED_ROW], False, 1)]
    trace = [33]
    for e in engines:
        e.plan(runs1, extra_keys=trace_n + 8)
        e.graph_capture(0)
    for i in range(trace_n):
        got = []
        for e in engines:
            e.graph_replay(1)
            e.sync()
            got.append((dev_u32(e, "d_lens", (1,)).copy(), dev_u32(e, "d_feed", (16,)).copy()))
        assert np.array_equal(got[0][0], got[1][0]) and np.array_equal(got[0][1], got[1][1]), f"decode {i}"
        trace.append(int(got[0][1][0]))
    tr = np.zeros((1, max_len), np.uint32)
    tr[0, 1100:1100 + len(trace)] = trace
    for e in engines:
        e.view("d_trace", tr.shape).copy_(torch.from_numpy(tr.view(np.int32)).cuda())
        e.view("d_trace_len", (1,)).copy_(torch.tensor([1100 + len(trace)], dtype=torch.int32).cuda())
        torch.cuda.synchronize()
        e.set_feed(s, 1100, 33)
        e.set_replay(77, 0.35)
    runs2 = [(s, [L.FEED_ROW + i for i in range(k + 1)], True)]
    for e in engines:
        e.plan(runs2, extra_keys=(k + 1) * steps + 8)
        e.graph_capture(L.STEP_REPLAY)
    for i in range(steps):
        got = []
        for e in engines:
            e.graph_replay(1)
            e.sync()
            got.append((dev_u32(e, "d_lens", (1,)).copy(), dev_u32(e, "d_feed", (16,)).copy(),
                        dev_u32(e, "d_emitted", (1,)).copy()))
        for x, y, what in zip(got[0], got[1], ("lengths", "feed", "emitted")):
            assert np.array_equal(x, y), f"verify {i}: {what} differ"
        n = int(got[0][0][0])
        if n - 1100 < len(trace):
            assert got[0][1][0] == trace[n - 1100], f"verify {i}: left the continuation"
    assert layer_launches(a)[0] == 1
    a.close()
    b.close()


def test_layers_kernel_abort_recovers(gpu):
    """A barrier forced never to complete (one producer more than exist, set from the host) with
    a short poll limit: every workgroup gives up and exits, the step reports the error, the
    counters are cleared, and the next step runs at the bar again."""
    banner("layer kernel abort path")
    lib = L.lib()
    spin = C.c_uint32.in_dll(lib, "_ZN2sv13g_layers_spinE")
    extra = C.c_uint32.in_dll(lib, "_ZN2sv14g_layers_extraE")
    shape = ModelShape(n_layers=2, vocab=4096, vocab_real=4000)
    model, gm, eng, ref, slots, rng = build_pair(shape, ctx=[400], seed=2, max_seq_len=512, options=L.OPT_LAYERS_KERNEL)
    s = slots[0]
    eng.set_feed(s, 400, 5)
    ref.set_feed(s, 400, 5)
    run = (s, [L.FEED_ROW, 1, 2, 3, 4], True)
    spin.value, extra.value = 2000, 1
    try:
        with pytest.raises(L.SvError, match="gave up waiting"):
            eng.step([run], logits=True)
    finally:
        spin.value, extra.value = 0, 0
    eng.close()
    # a fresh engine pair: the aborted step left its sequence state undefined
    model, gm, eng, ref, slots, rng = build_pair(shape, ctx=[400], seed=2, max_seq_len=512, options=L.OPT_LAYERS_KERNEL)
    eng.set_feed(s, 400, 5)
    ref.set_feed(s, 400, 5)
    ids_r, logits_r, em_r, extra_r = ref.step([run])
    res = eng.step([run], logits=True)
    compare_step(res, ids_r, logits_r, em_r, extra_r, eng, ref, slots, runs=[run])
    eng.close()
