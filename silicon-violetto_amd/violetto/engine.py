"""The engine (include/sv_verify.h sv_engine_*): the reference's Engine API over the C ABI."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib as L
from .model import ModelShape, SyntheticModel, rope_freq


def device_view(ptr: int, shape: tuple, dtype: torch.dtype) -> torch.Tensor:
    """A torch tensor over device memory the engine owns (no copy)."""
    typestr = {torch.uint16: "<u2", torch.int16: "<i2", torch.uint32: "<u4", torch.int32: "<i4",
               torch.float32: "<f4", torch.bfloat16: "<u2"}[dtype]

    class _Holder:
        __cuda_array_interface__ = {"shape": tuple(int(s) for s in shape), "typestr": typestr,
                                    "data": (int(ptr), False), "version": 2}

    t = torch.as_tensor(_Holder(), device="cuda")
    if dtype == torch.bfloat16:
        t = t.view(torch.bfloat16)
    return t


@dataclass
class StepResult:
    ids: np.ndarray
    logits: np.ndarray | None
    emitted: np.ndarray
    info: L.PlanInfo


@dataclass
class LayerCapture:
    """One layer's intermediates over a capture step (LayerCapture, engine.rs:176-188), [n][width]
    fp32 each: the layer's input residual, rms_norm of the attention input, q | k | v after the
    norms, RoPE and value embeddings, the attention output before XSA and the gate, o's product
    before the residual, rms_norm of the MLP input, down's product before the residual, and
    MUDD's residual base (None on other layers)."""
    layer: int
    n: int
    resid_in: np.ndarray
    attn_in: np.ndarray
    qkv: np.ndarray
    sdpa_out: np.ndarray
    attn_out: np.ndarray
    mlp_in: np.ndarray
    mlp_out: np.ndarray
    resid_base: np.ndarray | None


class Engine:
    def __init__(self, shape: ModelShape, *, max_seqs: int = 8, max_step_tokens: int = 64, max_seq_len: int = 8192,
                 max_head_rows: int = 16, kv_tokens: int | None = None, page_shift: int = 4, attn_scale: float = 0.125,
                 split_keys: int = 0, freq: np.ndarray | None = None, local: list[int] | None = None,
                 window: int = 0, options: int = 0):
        """local: per layer 1 for a sliding-window layer of `window` keys (model.rs:16-17,116);
        options: SV_OPT_* bits (OPT_LAYERS_KERNEL: the persistent layer kernel where it applies)."""
        self.shape = shape
        self.lib = L.lib()
        self._local = None if local is None else (C.c_uint8 * shape.n_layers)(*[int(x) for x in local])
        cfg = L.EngineConfig(shape.c(), max_seqs, max_step_tokens, max_seq_len, max_head_rows,
                             kv_tokens if kv_tokens is not None else max_seqs * max_seq_len, page_shift, attn_scale,
                             split_keys, options, window, 0,
                             C.cast(self._local, C.c_void_p) if self._local is not None else None)
        self.cfg = cfg
        f = np.ascontiguousarray(freq if freq is not None else rope_freq(500000.0, shape.head_dim), dtype=np.float32)
        self.freq = f
        h = C.c_void_p()
        L.check(self.lib.sv_engine_create(C.byref(cfg), f.ctypes.data_as(C.POINTER(C.c_float)), C.byref(h)))
        self.h = h
        self.model: SyntheticModel | None = None
        b = L.EngineBuffers()
        L.check(self.lib.sv_engine_get_buffers(self.h, C.byref(b)))
        self.buf = b

    def close(self) -> None:
        if self.h:
            self.lib.sv_engine_destroy(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- model
    def set_model(self, model) -> None:
        """A SyntheticModel on the GPU or a weights.VltModel (anything with embed_ptr() and
        c_layer(i) over device memory)."""
        assert getattr(model, "device", torch.device("cuda")).type == "cuda", "the engine reads weights from device memory"
        self.model = model
        L.check(self.lib.sv_engine_set_embed(self.h, model.embed_ptr()))
        for i in range(model.shape.n_layers):
            lay = model.c_layer(i)
            L.check(self.lib.sv_engine_set_layer(self.h, i, C.byref(lay)))
        head = model.c_head() if hasattr(model, "c_head") else None
        L.check(self.lib.sv_engine_set_head(self.h, C.byref(head) if head is not None else None))
        if getattr(model, "extras", None) is not None:
            ex = model.extras.c()
            L.check(self.lib.sv_engine_set_extras(self.h, C.byref(ex)))

    # -- the drafter (drafter.rs)
    def set_drafter(self, drafter) -> None:
        """A SyntheticDrafter on the GPU: the engine taps its layers on every step and, with
        STEP_DRAFT, drafts each slot's next block after the step."""
        assert drafter.device.type == "cuda", "the engine reads weights from device memory"
        self.drafter = drafter
        self._dc = drafter.c()
        L.check(self.lib.sv_engine_set_drafter(self.h, C.byref(self._dc)))
        b = L.DraftBuffers()
        L.check(self.lib.sv_engine_draft_buffers(self.h, C.byref(b)))
        self.dbuf = b

    def set_draft_rows(self, slot: int, rows: int) -> None:
        L.check(self.lib.sv_set_draft_rows(self.h, slot, rows))

    def draft_logits(self, rows: int) -> torch.Tensor:
        return device_view(self.dbuf.d_logits, (rows, self.drafter.v), torch.float32)

    def draft_candidates(self, rows: int) -> tuple[torch.Tensor, torch.Tensor]:
        return (device_view(self.dbuf.d_cand, (rows, L.DRAFT_CANDS), torch.int32),
                device_view(self.dbuf.d_cand_q, (rows, L.DRAFT_CANDS), torch.float32))

    def draft_taps(self, n: int) -> list[torch.Tensor]:
        return [device_view(self.dbuf.d_taps[k], (n, self.shape.hidden), torch.float32)
                for k in range(len(self.drafter.taps))]

    def draft_context(self, n: int) -> torch.Tensor:
        return device_view(self.dbuf.d_ctx, (n, self.shape.hidden), torch.float32)

    def draft_rings(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """The drafter's K, V [n_layers][n_pages][NKV][page][D] and their cyclic table."""
        s, b = self.shape, self.dbuf
        shape = (self.drafter.n_layers, b.n_pages, s.n_kv_heads, 1 << self.cfg.page_shift, s.head_dim)
        return (device_view(b.d_k_ring, shape, torch.bfloat16), device_view(b.d_v_ring, shape, torch.bfloat16),
                device_view(b.d_table, (self.cfg.max_seqs, b.max_pages), torch.int32))

    # -- views of engine-owned device memory
    @property
    def n_local(self) -> int:
        return 0 if self._local is None else sum(self._local)

    def kv_cache(self) -> tuple[torch.Tensor, torch.Tensor]:
        """The global (paged) layers' K and V: [n_global][n_pages][NKV][page][D]."""
        s = self.shape
        shape = (s.n_layers - self.n_local, self.buf.n_pages, s.n_kv_heads, 1 << self.cfg.page_shift, s.head_dim)
        return (device_view(self.buf.d_k_cache, shape, torch.bfloat16), device_view(self.buf.d_v_cache, shape, torch.bfloat16))

    def local_cache(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """The sliding-window layers' K, V [n_local][max_seqs * ring_pages][NKV][page][D] and
        their cyclic page table [max_seqs][max_pages]."""
        s = self.shape
        shape = (self.n_local, self.buf.n_local_pages, s.n_kv_heads, 1 << self.cfg.page_shift, s.head_dim)
        tab = device_view(self.buf.d_local_table, (self.cfg.max_seqs, self.buf.max_pages), torch.int32)
        return (device_view(self.buf.d_k_local, shape, torch.bfloat16), device_view(self.buf.d_v_local, shape, torch.bfloat16),
                tab)

    def view(self, name: str, shape: tuple, dtype=torch.int32) -> torch.Tensor:
        return device_view(getattr(self.buf, name), shape, dtype)

    # -- sequences
    def new_seq(self) -> int:
        s = C.c_uint32()
        L.check(self.lib.sv_new_seq(self.h, C.byref(s)))
        return s.value

    def free_seq(self, slot: int) -> None:
        L.check(self.lib.sv_free_seq(self.h, slot))

    def seq_len(self, slot: int) -> int:
        n = C.c_uint32()
        L.check(self.lib.sv_seq_len(self.h, slot, C.byref(n)))
        return n.value

    def seq_pages(self, slot: int) -> list[int]:
        n = C.c_uint32()
        L.check(self.lib.sv_seq_pages(self.h, slot, None, 0, C.byref(n)))
        arr = (C.c_uint32 * max(1, n.value))()
        L.check(self.lib.sv_seq_pages(self.h, slot, arr, n.value, C.byref(n)))
        return list(arr)[: n.value]

    def set_sampling(self, slot: int, temperature: float = 0.0, top_p: float = 1.0, seed: int = 0) -> None:
        L.check(self.lib.sv_set_sampling(self.h, slot, temperature, top_p, seed))

    def set_gen(self, slot: int, remaining: int = 0xFFFFFFFF, stop: tuple[int, ...] = (), done: int = 0) -> None:
        g = L.GenState(remaining, done, len(stop), 0, (C.c_uint32 * L.MAX_STOP)(*stop))
        L.check(self.lib.sv_set_gen(self.h, slot, C.byref(g)))

    def bench_fill(self, slot: int, n: int) -> None:
        L.check(self.lib.sv_bench_fill(self.h, slot, n))

    def settle(self, slot: int, unused: int) -> None:
        L.check(self.lib.sv_settle(self.h, slot, unused))

    def set_feed(self, slot: int, length: int, token: int) -> None:
        L.check(self.lib.sv_set_feed(self.h, slot, length, token))

    def set_replay(self, seed: int, rate: float) -> None:
        L.check(self.lib.sv_set_replay(self.h, seed, rate))

    # -- steps
    @staticmethod
    def _runs(runs: list[tuple]) -> tuple:
        """runs: (slot, tokens, verify[, head]) -> (sv_run array, keep-alive buffers)."""
        arr = (L.Run * len(runs))()
        keep = []
        for i, r in enumerate(runs):
            slot, toks, verify = r[0], r[1], r[2]
            head = r[3] if len(r) > 3 else 1
            t = (C.c_uint32 * len(toks))(*[int(x) for x in toks])
            keep.append(t)
            arr[i] = L.Run(slot, len(toks), C.cast(t, C.POINTER(C.c_uint32)), 1 if verify else 0, head)
        return arr, keep

    def plan(self, runs: list[tuple], extra_keys: int = 0) -> L.PlanInfo:
        torch.cuda.synchronize()  # writes torch made to engine buffers land first
        arr, keep = self._runs(runs)
        info = L.PlanInfo()
        L.check(self.lib.sv_plan(self.h, arr, len(runs), extra_keys, C.byref(info)))
        return info

    def encode(self, flags: int = 0) -> None:
        L.check(self.lib.sv_encode(self.h, flags))

    def graph_capture(self, flags: int = 0) -> None:
        torch.cuda.synchronize()
        L.check(self.lib.sv_graph_capture(self.h, flags))

    def graph_replay(self, count: int = 1) -> None:
        L.check(self.lib.sv_graph_replay(self.h, count))

    def sync(self) -> None:
        L.check(self.lib.sv_sync(self.h))

    @property
    def stream(self) -> int:
        return self.lib.sv_engine_stream(self.h)

    def step(self, runs: list[tuple], flags: int = 0, logits: bool = False) -> StepResult:
        torch.cuda.synchronize()  # writes torch made to engine buffers land first
        arr, keep = self._runs(runs)
        n_head = sum(len(r[1]) if r[2] else (r[3] if len(r) > 3 else 1) for r in runs)
        ids = (C.c_uint32 * max(1, n_head))()
        em = (C.c_uint32 * len(runs))()
        lg = np.zeros((n_head, self.shape.vocab), np.float32) if logits else None
        info = L.PlanInfo()
        L.check(self.lib.sv_step(self.h, arr, len(runs), flags, ids,
                                 lg.ctypes.data_as(C.POINTER(C.c_float)) if lg is not None else None, em, C.byref(info)))
        return StepResult(np.array(ids[:n_head], np.uint32), lg, np.array(em[:], np.uint32), info)

    def step_capture(self, runs: list[tuple], f, flags: int = 0, logits: bool = False) -> StepResult:
        """Engine::step_capture (engine.rs:318-355): the step run layer by layer; f(LayerCapture)
        is called for each layer in order (its arrays are copies), then the head and tail run as
        in step(), whose result this returns."""
        torch.cuda.synchronize()
        arr, keep = self._runs(runs)
        n_head = sum(len(r[1]) if r[2] else (r[3] if len(r) > 3 else 1) for r in runs)
        ids = (C.c_uint32 * max(1, n_head))()
        em = (C.c_uint32 * len(runs))()
        lg = np.zeros((n_head, self.shape.vocab), np.float32) if logits else None
        info = L.PlanInfo()
        errors = []

        def cb(cp, _user):
            if errors:
                return
            try:
                c = cp.contents
                rows = lambda p, w: np.ctypeslib.as_array(p, shape=(c.n, w)).copy() if p else None
                f(LayerCapture(c.layer, c.n, rows(c.resid_in, c.hidden), rows(c.attn_in, c.hidden),
                               rows(c.qkv, c.qkv_width), rows(c.sdpa_out, c.sdpa_width), rows(c.attn_out, c.hidden),
                               rows(c.mlp_in, c.hidden), rows(c.mlp_out, c.hidden), rows(c.resid_base, c.hidden)))
            except BaseException as e:  # raised again after the step (a callback cannot raise through C)
                errors.append(e)

        fn = L.CAPTURE_FN(cb)
        L.check(self.lib.sv_step_capture(self.h, arr, len(runs), flags, fn, None, ids,
                                         lg.ctypes.data_as(C.POINTER(C.c_float)) if lg is not None else None, em,
                                         C.byref(info)))
        if errors:
            raise errors[0]
        return StepResult(np.array(ids[:n_head], np.uint32), lg, np.array(em[:], np.uint32), info)

    def profile_step(self, flags: int = 0, reps: int = 1) -> dict[str, tuple[float, int]]:
        """kind -> (total ms, launches) over `reps` encoded steps with an event pair per kernel."""
        torch.cuda.synchronize()
        ms = (C.c_float * len(L.KINDS))()
        n = (C.c_uint32 * len(L.KINDS))()
        L.check(self.lib.sv_profile_step(self.h, flags, reps, ms, n))
        return {k: (ms[i], n[i]) for i, k in enumerate(L.KINDS)}

    def sample_logits(self, logits: np.ndarray, temperature, top_p, seed, pos) -> np.ndarray:
        logits = np.ascontiguousarray(logits, np.float32)
        rows = logits.shape[0]
        t = np.ascontiguousarray(np.broadcast_to(np.asarray(temperature, np.float32), (rows,)))
        p = np.ascontiguousarray(np.broadcast_to(np.asarray(top_p, np.float32), (rows,)))
        s = np.ascontiguousarray(np.broadcast_to(np.asarray(seed, np.uint64), (rows,)))
        q = np.ascontiguousarray(np.broadcast_to(np.asarray(pos, np.uint32), (rows,)))
        out = np.zeros(rows, np.uint32)
        L.check(self.lib.sv_sample_logits(self.h, logits.ctypes.data_as(C.POINTER(C.c_float)), rows,
                                          t.ctypes.data_as(C.POINTER(C.c_float)), p.ctypes.data_as(C.POINTER(C.c_float)),
                                          s.ctypes.data_as(C.POINTER(C.c_uint64)), q.ctypes.data_as(C.POINTER(C.c_uint32)),
                                          out.ctypes.data_as(C.POINTER(C.c_uint32))))
        return out
