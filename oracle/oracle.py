"""ctypes binding of the CPU oracle (liboracle.so). TEST INFRASTRUCTURE ONLY: imported by
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product."""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

u32 = C.c_uint32
f32 = C.c_float
vp = C.c_void_p

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        L.orc_bf.restype = f32
        L.orc_bf.argtypes = [C.c_uint16]
        L.orc_to_bf.restype = C.c_uint16
        L.orc_to_bf.argtypes = [f32]
        L.orc_round_bf16.restype = f32
        L.orc_round_bf16.argtypes = [f32]
        L.orc_uniform01.restype = f32
        L.orc_uniform01.argtypes = [u32, u32, u32, u32]
        L.orc_exp2.restype = f32
        L.orc_exp2.argtypes = [f32]
        L.orc_pool_reserve.restype = C.c_int
        L.orc_plan.restype = C.c_int
        L.orc_step.restype = C.c_int
        L.orc_draft.restype = C.c_int
        _lib = L
    return _lib


def ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(vp)


def struct_ptr(s):
    return C.byref(s) if s is not None else None


# -- scalars / formats ------------------------------------------------------------------------
def philox(ctr, key) -> list[int]:
    c = (u32 * 4)(*ctr)
    k = (u32 * 2)(*key)
    lib().orc_philox(c, k)
    return list(c)


def exp2(x: float) -> float:
    return lib().orc_exp2(x)


def uniform01(seed_lo: int, seed_hi: int, pos: int, rnd: int) -> float:
    return lib().orc_uniform01(seed_lo, seed_hi, pos, rnd)


def quantize(w: np.ndarray, group: int) -> tuple[np.ndarray, np.ndarray]:
    w = np.ascontiguousarray(w, np.float32)
    m, k = w.shape
    q = np.zeros((m, k), np.int8)
    s = np.zeros((m, k // group), np.uint16)
    lib().orc_quantize(ptr(w), m, k, group, ptr(q), ptr(s))
    return q, s


def rope_table(freq: np.ndarray, n_pos: int) -> np.ndarray:
    f = np.ascontiguousarray(freq, np.float32)
    tab = np.zeros((n_pos, 32, 2), np.float32)
    lib().orc_rope_table(ptr(f), n_pos, ptr(tab))
    return tab


def bf16_to_f32(u: np.ndarray) -> np.ndarray:
    return (np.asarray(u, np.uint16).astype(np.uint32) << 16).view(np.float32)


# -- kernels ----------------------------------------------------------------------------------
def matmul(L, mat_w: np.ndarray, scales: np.ndarray | None, gshift: int, x: np.ndarray, a, *,
           base: np.ndarray | None = None, x_rows: np.ndarray | None = None, aux: np.ndarray | None = None
           ) -> np.ndarray:
    """y = epilogue(W x) as the reference's matmul group. L is violetto._lib (struct types)."""
    m, k = mat_w.shape
    fmt = 1 if mat_w.dtype == np.int8 else 0
    w = np.ascontiguousarray(mat_w)
    sc = np.ascontiguousarray(scales) if scales is not None else None
    mat = L.Matrix(w.ctypes.data, sc.ctypes.data if sc is not None else None, m, k, fmt, gshift)
    out_m = m // 2 if a.epi == 3 else m
    y = np.zeros((a.n, out_m), np.float32)
    lib().orc_matmul(C.byref(mat), ptr(np.ascontiguousarray(x, np.float32)),
                     ptr(x_rows), ptr(y), ptr(base), ptr(aux), C.byref(a))
    return y


def attn_extras(L, shape, extras: dict | None):
    """sv_attn_extras over host arrays (x, inv, tokens, value_embed, ve_gate, attn_gate, xsa), or None."""
    if not extras:
        return None, []
    keep = {k: np.ascontiguousarray(v) for k, v in extras.items() if v is not None}
    g = lambda k: ptr(keep.get(k))  # noqa: E731
    return L.AttnExtras(g("x"), g("inv"), g("tokens"), g("value_embed"), g("ve_gate"), g("attn_gate"), g("xsa"),
                        None, shape.hidden, 0), keep


def attn_verify(L, shape, qkv, meta, k_cache, v_cache, page_table, rope, kv, args, runs, vis,
                extras: dict | None = None) -> np.ndarray:
    sh = shape.c()
    n = qkv.shape[0]
    out = np.zeros((n, shape.n_heads * shape.head_dim), np.float32)
    ex, keep = attn_extras(L, shape, extras)
    lib().orc_attn_verify(C.byref(sh), ptr(qkv), ptr(meta), ptr(k_cache), ptr(v_cache), ptr(page_table), ptr(rope),
                          C.byref(kv), C.byref(args), ptr(runs), u32(len(runs) // 2), ptr(vis), ptr(out),
                          C.byref(ex) if ex is not None else None)
    return out


def mudd(cur, tap0, tap1, dense1, mix) -> tuple[np.ndarray, np.ndarray]:
    """orc_mudd over [n][hidden] rows; mix is one site's [2][3][33]."""
    c = [np.ascontiguousarray(a, np.float32) for a in (cur, tap0, tap1, dense1, mix)]
    n, hidden = c[0].shape
    oa = np.zeros((n, hidden), np.float32)
    ob = np.zeros((n, hidden), np.float32)
    lib().orc_mudd(*[ptr(a) for a in c], ptr(oa), ptr(ob), u32(n), u32(hidden))
    return oa, ob


def sample(L, logits: np.ndarray, rows, meta: np.ndarray | None = None) -> np.ndarray:
    logits = np.ascontiguousarray(logits, np.float32)
    n, vocab = logits.shape
    arr = (L.SampleRow * n)(*rows)
    out = np.zeros(n, np.uint32)
    lib().orc_sample(ptr(logits), arr, ptr(out), ptr(meta), u32(n), u32(vocab))
    return out


def accept(L, runs, tokens, out, lens, feed, gen, tree, n_tokens: int):
    """Returns (out, lens, feed, gen, emitted, path, path_len, on_path) after accept."""
    nr = len(runs)
    runs_a = (L.RunIn * nr)(*runs)
    gen_a = (L.GenState * len(gen))(*gen)
    out = np.array(out, np.uint32)
    lens = np.array(lens, np.uint32)
    feed = np.array(feed, np.uint32)
    emitted = np.zeros(nr, np.uint32)
    path = np.zeros(nr * 16, np.uint32)
    path_len = np.zeros(nr, np.uint32)
    on_path = np.zeros(max(1, n_tokens), np.uint32)
    lib().orc_accept(runs_a, ptr(np.ascontiguousarray(tokens, np.uint32)), ptr(out), ptr(lens), ptr(feed), gen_a,
                     ptr(emitted), u32(nr), ptr(np.ascontiguousarray(tree, np.uint32)), ptr(path), ptr(path_len),
                     ptr(on_path))
    return out, lens, feed, list(gen_a), emitted, path, path_len, on_path


def kv_compact(L, shape, runs, path, path_len, lens, k_cache, v_cache, page_table, kv):
    sh = shape.c()
    runs_a = (L.RunIn * len(runs))(*runs)
    lib().orc_kv_compact(C.byref(sh), runs_a, u32(len(runs)), ptr(path), ptr(path_len), ptr(lens), ptr(k_cache),
                         ptr(v_cache), ptr(page_table), C.byref(kv))


def replay_draft(L, runs, lens, feed, trace, trace_len, ra, tree):
    runs_a = (L.RunIn * len(runs))(*runs)
    lib().orc_replay_draft(runs_a, u32(len(runs)), ptr(lens), ptr(feed), ptr(trace), ptr(trace_len), C.byref(ra),
                           ptr(tree))


def draft_top(logits: np.ndarray, vocab: np.ndarray, tin: np.ndarray, inv_t: float, ncand: int):
    """kernels.metal:1845-1891 draft_top: (cand [rows][4] target ids, cand_q [rows][4])."""
    logits = np.ascontiguousarray(logits, np.float32)
    n, nv = logits.shape
    cand = np.zeros((n, 4), np.uint32)
    cand_q = np.zeros((n, 4), np.float32)
    lib().orc_draft_top(ptr(logits), ptr(np.ascontiguousarray(vocab, np.uint32)), ptr(np.ascontiguousarray(tin, np.uint32)),
                        ptr(cand), ptr(cand_q), u32(n), u32(nv), f32(inv_t), u32(ncand))
    return cand, cand_q


def draft_tree(blocks: np.ndarray, tin: np.ndarray, cand: np.ndarray, cand_q: np.ndarray, feed: np.ndarray,
               tree: np.ndarray, ncand: int) -> None:
    """kernels.metal:1893-1934 draft_tree, writing feed/tree [slots * 16] in place."""
    b = np.ascontiguousarray(blocks, np.uint32)
    lib().orc_draft_tree(ptr(b), u32(b.size // 2), ptr(np.ascontiguousarray(tin, np.uint32)),
                         ptr(np.ascontiguousarray(cand, np.uint32)), ptr(np.ascontiguousarray(cand_q, np.float32)),
                         ptr(feed), ptr(tree), u32(ncand))


def embed(L, shape, table, tokens, tin, lens, feed, tree, vis):
    sh = shape.c()
    n = len(tokens)
    tokens = np.array(tokens, np.uint32)
    out = np.zeros((n, shape.hidden), np.float32)
    meta = np.zeros((n, 2), np.uint32)
    vis = np.array(vis, np.uint32)
    lib().orc_embed(C.byref(sh), ptr(table), ptr(tokens), ptr(out), ptr(np.ascontiguousarray(tin, np.uint32)),
                    ptr(meta), ptr(np.ascontiguousarray(lens, np.uint32)), ptr(np.ascontiguousarray(feed, np.uint32)),
                    ptr(np.ascontiguousarray(tree, np.uint32)), ptr(vis), u32(n))
    return tokens, out, meta, vis


class Pool:
    """kv.rs page pool (LIFO free list)."""

    class _S(C.Structure):
        _fields_ = [("free_list", vp), ("n_free", u32), ("n_pages", u32), ("max_pages", u32), ("page_shift", u32),
                    ("page_table", vp), ("seq_pages", vp)]

    def __init__(self, n_pages: int, max_seqs: int, max_pages: int, page_shift: int):
        self.free = np.zeros(n_pages, np.uint32)
        self.table = np.zeros((max_seqs, max_pages), np.uint32)
        self.held = np.zeros(max_seqs, np.uint32)
        self.s = Pool._S()
        lib().orc_pool_init(C.byref(self.s), u32(n_pages), u32(max_seqs), u32(max_pages), u32(page_shift),
                            ptr(self.free), ptr(self.table), ptr(self.held))

    def reserve(self, slot: int, length: int) -> bool:
        return lib().orc_pool_reserve(C.byref(self.s), u32(slot), u32(length)) == 0

    def release(self, slot: int) -> None:
        lib().orc_pool_release(C.byref(self.s), u32(slot))

    def pages(self, slot: int) -> list[int]:
        return [int(x) for x in self.table[slot, : self.held[slot]]]


class StepIO(C.Structure):
    _fields_ = [("n", u32), ("n_head", u32), ("n_runs", u32), ("tokens", vp), ("tin", vp), ("vis", vp),
                ("head_rows", vp), ("samples", vp), ("runs", vp), ("attn_runs", vp), ("compact", u32),
                ("lens", vp), ("feed", vp), ("tree", vp), ("gen", vp), ("k_cache", vp), ("v_cache", vp),
                ("page_table", vp), ("kv", C.c_uint32 * 8), ("rope", vp), ("meta", vp), ("logits", vp),
                ("out", vp), ("emitted", vp), ("path", vp), ("path_len", vp), ("on_path", vp), ("hidden", vp),
                ("n_attn", u32), ("extras", vp), ("local", vp), ("k_local", vp), ("v_local", vp), ("local_table", vp),
                ("kv_local", C.c_uint32 * 8), ("head", vp), ("n_taps", u32), ("tap_layers", vp), ("tap_out", vp),
                ("cap", vp)]


class DraftIO(C.Structure):
    _fields_ = [("n", u32), ("taps", vp), ("meta", vp), ("on_path", vp), ("rope", vp), ("k_ring", vp), ("v_ring", vp),
                ("table", vp), ("kv", C.c_uint32 * 8), ("ctx_ring", vp), ("cr", u32), ("n_blocks", u32), ("rows", u32),
                ("blocks", vp), ("tin", vp), ("vis", vp), ("lens", vp), ("feed", vp), ("tree", vp), ("logits", vp),
                ("ctx", vp)]


def host_drafter(drafter):
    """(sv_drafter over host copies, the arrays it points into) of a SyntheticDrafter."""
    import torch

    keep = []

    def hp(t):
        if t.dtype == torch.bfloat16:
            a = t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
        else:
            a = t.detach().cpu().contiguous().numpy()
        a = np.ascontiguousarray(a)
        keep.append(a)
        return a.ctypes.data

    return drafter.c(hp), keep


def _chain(row: int) -> int:
    return row | ((0xFF if row == 0 else row - 1) << 8) | (((2 << row) - 1) << 16)


class OracleEngine:
    """The engine on host memory: page pool, sequence state, plan and step (orc_plan, orc_step).

    `weights`: per layer a dict name -> (w, scales) numpy (int8 + uint16 [m][1], or bf16 bits as
    uint16 [m][k] with scales None); `embed` uint16 [vocab][hidden]; `scalars` per layer
    (qkv_scale, o_scale, resid_attn, post_attn, resid_mlp, post_mlp, rope).
    """

    def __init__(self, L, shape, embed, weights, scalars, *, max_seqs=8, max_seq_len=8192, kv_tokens=None,
                 page_shift=4, attn_scale=0.125, freq=None, extras=None, max_step_tokens=64, head=None):
        """extras: host_extras() of a model with the Limite extras (sliding-window layers with
        rings laid out as the engine's, for max_step_tokens rows per step)."""
        self.L, self.shape = L, shape
        self.arun = min(16, 64 // (shape.n_heads // shape.n_kv_heads))
        self.page_shift = page_shift
        page = 1 << page_shift
        kv_tokens = kv_tokens if kv_tokens is not None else max_seqs * max_seq_len
        self.n_pages = -(-kv_tokens // page)
        self.max_pages = -(-max_seq_len // page)
        self.max_seqs, self.max_seq_len = max_seqs, max_seq_len
        s = shape
        self.hx = extras
        self.local = np.array(extras["local"] if extras else [0] * s.n_layers, np.uint8)
        n_local = int(self.local.sum())
        self.window = extras["window"] if extras else 0
        self.ring_pages = -(-(self.window + max_step_tokens) // page) if n_local else 0
        self.n_lpages = max_seqs * self.ring_pages
        self.k = np.zeros((s.n_layers - n_local, self.n_pages, s.n_kv_heads, page, s.head_dim), np.uint16)
        self.v = np.zeros_like(self.k)
        self.k_local = np.zeros((n_local, max(1, self.n_lpages), s.n_kv_heads, page, s.head_dim), np.uint16)
        self.v_local = np.zeros_like(self.k_local)
        self.local_table = np.array([[slot * self.ring_pages + p % max(1, self.ring_pages) for p in range(self.max_pages)]
                                     for slot in range(max_seqs)], np.uint32)
        self._mx = None
        self._mudd_layers = tuple(extras["mudd_layer"]) if extras else ()
        if extras:
            n = len(extras["mudd_layer"])
            self._mx = L.ModelExtras(ptr(extras["value_embed"]), ptr(extras["mudd_dense1"]), ptr(extras["mudd_mix"]), n,
                                     (u32 * 2)(*(list(extras["mudd_layer"]) + [0] * (2 - n))),
                                     (u32 * 2)(*(list(extras["mudd_tap"]) + [0] * (2 - n))), 0)
        self.pool = Pool(self.n_pages, max_seqs, self.max_pages, page_shift)
        self.lens = np.zeros(max_seqs, np.uint32)
        self.feed = np.zeros(max_seqs * 16, np.uint32)
        self.tree = np.array([_chain(i % 16) for i in range(max_seqs * 16)], np.uint32)
        self.gen = (L.GenState * max_seqs)()
        for g in self.gen:
            g.remaining = 0xFFFFFFFF
        self.seq_len = [0] * max_seqs
        self.used = [False] * max_seqs
        self.sampling = [L.SampleRow(0, 0, 0, 0.0, 1.0, 0xFFFFFFFF) for _ in range(max_seqs)]
        self.attn_scale = attn_scale
        self.rope = rope_table(freq, max_seq_len + 16)
        self.embed = np.ascontiguousarray(embed, np.uint16)
        self._keep = []
        layers = (L.Layer * s.n_layers)()
        for i, (lay, sc) in enumerate(zip(weights, scalars)):
            mats = []
            for name in ("qkv", "o", "gate_up", "down"):
                w, scl = lay[name]
                w = np.ascontiguousarray(w)
                self._keep.append(w)
                if scl is not None:
                    scl = np.ascontiguousarray(scl, np.uint16)
                    self._keep.append(scl)
                m, k = w.shape
                gshift = 0 if scl is None else (31 if scl.shape[1] == 1 else int(k // scl.shape[1]).bit_length() - 1)
                mats.append(L.Matrix(w.ctypes.data, scl.ctypes.data if scl is not None else None, m, k,
                                     1 if w.dtype == np.int8 else 0, gshift))
            ex = [ptr(extras[k][i]) if extras and extras[k][i] is not None else None
                  for k in ("attn_gate", "ve_gate", "xsa")]
            layers[i] = L.Layer(*mats, *sc[:6], int(sc[6]), 0, *ex)
        self.layers = layers
        self._head = None  # its own head: (int8 q [vocab][hidden], bf16 scales bits) as host_head gives
        if head is not None:
            q, scl = (np.ascontiguousarray(head[0]), np.ascontiguousarray(head[1], np.uint16))
            self._keep += [q, scl]
            m, k = q.shape
            gshift = 31 if scl.shape[1] == 1 else int(k // scl.shape[1]).bit_length() - 1
            self._head = L.Matrix(q.ctypes.data, scl.ctypes.data, m, k, 1, gshift)

    # the drafter
    def set_drafter(self, drafter, max_step_tokens=64) -> None:
        """A SyntheticDrafter: its rings laid out as the engine's (cyclic pages of the window plus
        a step's or a block's rows), the context ring with inject."""
        self.dr = drafter
        self._dc, self._dkeep = host_drafter(drafter)
        s, page = self.shape, 1 << self.page_shift
        span = drafter.window + max(max_step_tokens, self.arun)
        self.d_ring_pages = -(-span // page)
        self.d_n_pages = self.max_seqs * self.d_ring_pages
        self.d_max_pages = -(-(self.max_seq_len + self.arun) // page)
        self.dk = np.zeros((drafter.n_layers, self.d_n_pages, s.n_kv_heads, page, s.head_dim), np.uint16)
        self.dv = np.zeros_like(self.dk)
        self.d_table = np.array([[slot * self.d_ring_pages + p % self.d_ring_pages for p in range(self.d_max_pages)]
                                 for slot in range(self.max_seqs)], np.uint32)
        self.d_cr = max_step_tokens if drafter.inject else 0
        self.d_cring = np.zeros((self.max_seqs, max(1, self.d_cr), s.hidden), np.float32)
        self.draft_rows = [0] * self.max_seqs

    def _draft(self, runs, n, meta, on_path, taps, blocks_on):
        """drafter.rs:278-447 after orc_step: the context of the step's n tokens; with blocks_on,
        a block per run that draws and whose slot has draft rows."""
        d, H = self.dr, self.shape.hidden
        blocks, tin, vis = [], [], []
        if blocks_on:
            for r in runs:
                rows = self.draft_rows[r[0]]
                head = r[3] if len(r) > 3 else 1
                if rows == 0 or not (r[2] or head):
                    continue
                blocks += [len(vis), rows]
                for i in range(rows):
                    tin += [r[0], i]
                    vis.append((1 << rows) - 1)
        rows = len(vis)
        blocks = np.array(blocks or [0], np.uint32)
        tin = np.array(tin or [0, 0], np.uint32)
        vis = np.array(vis or [0], np.uint32)
        logits = np.zeros((max(1, rows), d.v), np.float32)
        ctx = np.zeros((max(1, n), H), np.float32)
        tap_arr = [np.ascontiguousarray(t, np.float32) for t in taps]
        tap_ptrs = (vp * len(tap_arr))(*[t.ctypes.data for t in tap_arr])
        io = DraftIO()
        io.n, io.taps, io.meta, io.on_path, io.rope = n, C.cast(tap_ptrs, vp), ptr(meta), ptr(on_path), ptr(self.rope)
        io.k_ring, io.v_ring, io.table = ptr(self.dk), ptr(self.dv), ptr(self.d_table)
        io.kv[:] = [0, 0, self.d_ring_pages << self.page_shift, self.max_seqs, self.page_shift, self.d_n_pages,
                    self.d_max_pages, d.window]
        io.ctx_ring, io.cr = ptr(self.d_cring), self.d_cr
        io.n_blocks, io.rows = len(blocks) // 2 if rows else 0, rows
        io.blocks, io.tin, io.vis = ptr(blocks), ptr(tin), ptr(vis)
        io.lens, io.feed, io.tree = ptr(self.lens), ptr(self.feed), ptr(self.tree)
        io.logits, io.ctx = ptr(logits), ptr(ctx)
        sh = self.shape.c()
        rc = lib().orc_draft(C.byref(sh), ptr(self.embed), C.byref(self._dc), f32(self.attn_scale), C.byref(io))
        assert rc == 0
        return dict(draft_logits=logits[:rows], ctx=ctx[:n], blocks=blocks[: 2 * io.n_blocks].reshape(-1, 2),
                    draft_tin=tin[: 2 * rows].reshape(-1, 2))

    # sequences
    def new_seq(self) -> int:
        slot = self.used.index(False)
        self.used[slot] = True
        self.seq_len[slot] = 0
        self.lens[slot] = 0
        g = self.gen[slot]
        g.remaining, g.done, g.nstop = 0xFFFFFFFF, 0, 0
        return slot

    def set_sampling(self, slot, temperature=0.0, top_p=1.0, seed=0):
        self.sampling[slot] = self.L.SampleRow(seed & 0xFFFFFFFF, seed >> 32, 0, temperature, top_p, 0xFFFFFFFF)

    def set_gen(self, slot, remaining=0xFFFFFFFF, stop=(), done=0):
        g = self.gen[slot]
        g.remaining, g.done, g.nstop = remaining, done, len(stop)
        for i, t in enumerate(stop):
            g.stop[i] = t

    def set_feed(self, slot, length, token):
        assert self.pool.reserve(slot, length)
        self.seq_len[slot] = length
        self.lens[slot] = length
        self.feed[slot * 16] = token

    def bench_fill(self, slot, n):
        self.seq_len[slot] += n
        assert self.pool.reserve(slot, self.seq_len[slot])
        self.lens[slot] = self.seq_len[slot]

    def step(self, runs, compact=None, want_hidden=False, draft=False, taps=None, capture=False):
        """runs: (slot, tokens, verify[, head]). Returns (ids, logits, emitted, extra). With a
        drafter set: its context pass, and with draft=True its blocks; `taps` replaces the
        oracle's own tapped rows as the drafter's input (to check the drafter alone). With
        capture: extra["capture"], per layer a dict of its intermediates (Engine::step_capture,
        engine.rs:318-355): resid_in, attn_in, qkv, sdpa_out, attn_out, mlp_in, mlp_out,
        resid_base (None off the MUDD layers), [n][width] each."""
        L = self.L
        n_runs = len(runs)
        in_runs = np.zeros((n_runs, 4), np.uint32)
        toks = []
        for i, r in enumerate(runs):
            in_runs[i] = (r[0], len(r[1]), 1 if r[2] else 0, r[3] if len(r) > 3 else 1)
            toks += [int(t) for t in r[1]]
        n = len(toks)
        for r in runs:
            assert self.pool.reserve(r[0], self.seq_len[r[0]] + len(r[1]))
        in_tokens = np.array(toks, np.uint32)
        tokens = np.zeros(n, np.uint32)
        tin = np.zeros(2 * n, np.uint32)
        vis = np.zeros(n, np.uint32)
        head_rows = np.zeros(n, np.uint32)
        samples = (L.SampleRow * max(1, n))()
        run_in = (L.RunIn * n_runs)()
        seq_len = np.array(self.seq_len, np.uint32)
        samp = (L.SampleRow * self.max_seqs)(*self.sampling)
        n_head = lib().orc_plan(ptr(in_runs), u32(n_runs), ptr(in_tokens), ptr(seq_len), samp, ptr(tokens), ptr(tin),
                                ptr(vis), ptr(head_rows), samples, run_in, u32(self.arun))
        assert n_head >= 0, "plan rejected"
        # attention runs of at most arun rows: a prompt chunk's later rows see its earlier ones as
        # cached keys (written by the earlier runs)
        a = self.arun
        attn_runs = np.array([[ri.first + j, min(a, ri.count - j)] for ri in run_in for j in range(0, ri.count, a)],
                             np.uint32).reshape(-1)
        branches = any(r[2] and len(r[1]) > 2 for r in runs)
        meta = np.zeros(2 * n, np.uint32)
        logits = np.zeros((max(1, n_head), self.shape.vocab), np.float32)
        out = np.zeros(max(1, n_head), np.uint32)
        emitted = np.zeros(n_runs, np.uint32)
        path = np.zeros(n_runs * 16, np.uint32)
        path_len = np.zeros(n_runs, np.uint32)
        on_path = np.zeros(n, np.uint32)
        hidden = np.zeros((n, self.shape.hidden), np.float32) if want_hidden else None
        io = StepIO()
        io.n, io.n_head, io.n_runs = n, n_head, n_runs
        io.tokens, io.tin, io.vis, io.head_rows = ptr(tokens), ptr(tin), ptr(vis), ptr(head_rows)
        io.samples = C.cast(samples, vp)
        io.runs = C.cast(run_in, vp)
        io.attn_runs = ptr(attn_runs)
        io.compact = int(branches if compact is None else compact)
        io.n_attn = attn_runs.size // 2
        io.lens, io.feed, io.tree = ptr(self.lens), ptr(self.feed), ptr(self.tree)
        io.gen = C.cast(self.gen, vp)
        io.k_cache, io.v_cache, io.page_table = ptr(self.k), ptr(self.v), ptr(self.pool.table)
        io.kv[:] = [1, 0, 0, self.max_seqs, self.page_shift, self.n_pages, self.max_pages, 0]
        io.rope = ptr(self.rope)
        io.meta, io.logits, io.out = ptr(meta), ptr(logits), ptr(out)
        io.emitted, io.path, io.path_len, io.on_path = ptr(emitted), ptr(path), ptr(path_len), ptr(on_path)
        io.hidden = ptr(hidden)
        io.extras = C.cast(C.pointer(self._mx), vp) if self._mx is not None else None
        io.head = C.cast(C.pointer(self._head), vp) if self._head is not None else None
        io.local = ptr(self.local)
        io.k_local, io.v_local, io.local_table = ptr(self.k_local), ptr(self.v_local), ptr(self.local_table)
        io.kv_local[:] = [0, 0, self.ring_pages * page_of(self.page_shift), self.max_seqs, self.page_shift,
                          max(1, self.n_lpages), self.max_pages, self.window]
        dr = getattr(self, "dr", None)
        tap_out = [np.zeros((n, self.shape.hidden), np.float32) for _ in (dr.taps if dr else ())]
        if dr is not None:
            tl = np.array(dr.taps, np.uint32)
            tp = (vp * len(tap_out))(*[t.ctypes.data for t in tap_out])
            io.n_taps, io.tap_layers, io.tap_out = len(tap_out), ptr(tl), C.cast(tp, vp)
        H, D = self.shape.hidden, self.shape.head_dim
        NQD, W = self.shape.n_heads * D, (self.shape.n_heads + 2 * self.shape.n_kv_heads) * D
        widths = [("resid_in", H), ("attn_in", H), ("qkv", W), ("sdpa_out", NQD), ("attn_out", H), ("mlp_in", H),
                  ("mlp_out", H), ("resid_base", H)]
        cap = np.zeros((self.shape.n_layers, n * sum(w for _, w in widths)), np.float32) if capture else None
        io.cap = ptr(cap)
        sh = self.shape.c()
        rc = lib().orc_step(C.byref(sh), ptr(self.embed), self.layers, f32(self.attn_scale), C.byref(io))
        assert rc == 0
        dx = {}
        if dr is not None:
            dx = self._draft(runs, n, meta, on_path, tap_out if taps is None else taps, draft)
            dx["taps"] = tap_out
        for i, r in enumerate(runs):
            self.seq_len[r[0]] += len(r[1])
            if r[2]:
                self.seq_len[r[0]] -= len(r[1]) - min(int(emitted[i]), len(r[1]))
        extra = dict(tokens=tokens, meta=meta.reshape(n, 2), vis=vis, path=path.reshape(n_runs, 16),
                     path_len=path_len, on_path=on_path, hidden=hidden, head_rows=head_rows[:n_head], **dx)
        if capture:
            mudd_layers = set(self._mudd_layers)
            layers = []
            for li in range(self.shape.n_layers):
                d, o = {}, 0
                for name, w in widths:
                    d[name] = cap[li, o:o + n * w].reshape(n, w).copy()
                    o += n * w
                if li not in mudd_layers:
                    d["resid_base"] = None
                layers.append(d)
            extra["capture"] = layers
        return out[:n_head].copy(), logits[:n_head].copy(), emitted, extra


def page_of(shift: int) -> int:
    return 1 << shift


def host_extras(model) -> dict | None:
    """The model's Limite extras as host arrays (OracleEngine's `extras`), or None."""
    import torch

    x = getattr(model, "extras", None)
    if x is None:
        return None

    def f32(t):
        return None if t is None else np.ascontiguousarray(t.detach().float().cpu().numpy())

    return dict(local=list(x.local), window=x.window, attn_gate=[f32(t) for t in x.attn_gate],
                ve_gate=[f32(t) for t in x.ve_gate], xsa=[f32(t) for t in x.xsa],
                value_embed=None if x.value_embed is None else
                np.ascontiguousarray(x.value_embed.detach().cpu().view(torch.int16).numpy().view(np.uint16)),
                mudd_dense1=f32(x.mudd_dense1), mudd_mix=f32(x.mudd_mix), mudd_layer=tuple(x.mudd_layer),
                mudd_tap=tuple(x.mudd_tap))


def host_head(model):
    """The model's own head as (int8 q, bf16 scale bits) host arrays, or None (tied)."""
    import torch

    if getattr(model, "head", None) is None:
        return None
    q, s = model.head
    return (q.detach().cpu().numpy(), s.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16))


def host_weights(model) -> tuple[np.ndarray, list, list]:
    """(embed, per-layer weights, per-layer scalars) of a violetto SyntheticModel as numpy."""
    import torch

    def bits(t):
        return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)

    embed = bits(model.embed)
    layers = []
    for lay in model.layers:
        d = {}
        for name, (w, s) in lay.items():
            if s is None:
                d[name] = (bits(w), None)
            else:
                d[name] = (w.detach().cpu().numpy(), bits(s))
        layers.append(d)
    scal = [(s.qkv_scale, s.o_scale, s.resid_attn, s.post_attn, s.resid_mlp, s.post_mlp, s.rope)
            for s in model.scalars]
    return embed, layers, scal
