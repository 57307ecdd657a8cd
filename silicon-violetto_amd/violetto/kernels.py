"""Kernel-level calls of include/sv_verify.h on torch device tensors (one call per pipeline
group of the reference's forward pass). Every call is asynchronous on the given stream
(default: torch's current stream)."""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib as L
from .model import ModelShape


def _p(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    assert t.is_cuda and t.is_contiguous(), "device tensors must be contiguous CUDA tensors"
    return t.data_ptr()


def _stream(stream: int | None) -> int:
    return stream if stream is not None else torch.cuda.current_stream().cuda_stream


class Workspace:
    """Zero-filled device workspace (the kernels keep its counters at zero between calls)."""

    def __init__(self, nbytes: int):
        self.t = torch.zeros(max(1, (nbytes + 3) // 4), dtype=torch.int32, device="cuda")

    @property
    def nbytes(self) -> int:
        return self.t.numel() * 4

    def grow(self, nbytes: int) -> "Workspace":
        return self if nbytes <= self.nbytes else Workspace(nbytes)


class Mat:
    """A weight matrix on the device and its sv_matrix (the tensors stay referenced here)."""

    def __init__(self, w: torch.Tensor, scales: torch.Tensor | None = None, gshift: int = 31):
        self.w, self.scales = w, scales
        m, k = w.shape
        if w.dtype == torch.int8:
            assert scales is not None
            self.c = L.Matrix(_p(w), _p(scales), m, k, L.FMT_I8, gshift)
        else:
            assert w.dtype == torch.bfloat16
            self.c = L.Matrix(_p(w), None, m, k, L.FMT_BF16, 0)

    def tiled(self, stream: int | None = None) -> "Mat":
        """The same matrix in the tiled layout (SV_FMT_TILED), packed on the device."""
        out = Mat.__new__(Mat)
        out.w, out.scales = torch.empty_like(self.w), self.scales
        out.c = L.Matrix()
        L.check(L.lib().sv_pack_matrix(_stream(stream), C.byref(self.c), _p(out.w), C.byref(out.c)))
        return out

    @property
    def m(self) -> int:
        return self.c.m

    @property
    def k(self) -> int:
        return self.c.k

    @property
    def gshift(self) -> int:
        return self.c.gshift


def matrix(w: torch.Tensor, scales: torch.Tensor | None = None, gshift: int = 31) -> Mat:
    return Mat(w, scales, gshift)


def matmul(mat: Mat, x: torch.Tensor, y: torch.Tensor, *, n: int, epi: int, flags: int = 0, scale: float = 1.0,
           ra: float = 0.0, rb: float = 0.0, base: torch.Tensor | None = None, aux: torch.Tensor | None = None,
           x_rows: torch.Tensor | None = None, vocab_real: int | None = None, ws: Workspace | None = None,
           stream: int | None = None) -> None:
    a = L.MatArgs(n, mat.k, mat.m, epi, flags, vocab_real if vocab_real is not None else mat.m, scale, ra, rb, 1,
                  mat.k, mat.gshift)
    need = L.lib().sv_matmul_workspace_bytes(n, mat.m, mat.k)
    ws = ws.grow(need) if ws is not None else Workspace(need)
    L.check(L.lib().sv_matmul(_stream(stream), C.byref(mat.c), _p(x), _p(x_rows), _p(y), _p(base), _p(aux), C.byref(a),
                              _p(ws.t), ws.nbytes))


def attn_verify(shape: ModelShape, qkv: torch.Tensor, meta: torch.Tensor, k_cache: torch.Tensor,
                v_cache: torch.Tensor, page_table: torch.Tensor, rope: torch.Tensor, kv: L.KvArgs, args: L.AttnArgs,
                runs: torch.Tensor, n_runs: int, max_run: int, vis: torch.Tensor, out: torch.Tensor,
                ws: Workspace | None = None, stream: int | None = None, extras: dict | None = None) -> None:
    """extras: the layer's extras (sv_attn_extras) as tensors: x, inv, tokens, value_embed, ve_gate,
    attn_gate, xsa, vdir (absent: off)."""
    sh = shape.c()
    need = L.lib().sv_attn_workspace_bytes(C.byref(sh), n_runs, args.max_splits, max_run)
    ws = ws.grow(need) if ws is not None else Workspace(need)
    ex = None
    if extras:
        g = lambda k: _p(extras.get(k))  # noqa: E731
        ex = L.AttnExtras(g("x"), g("inv"), g("tokens"), g("value_embed"), g("ve_gate"), g("attn_gate"), g("xsa"),
                          g("vdir"), shape.hidden, 0)
    L.check(L.lib().sv_attn_verify(_stream(stream), C.byref(sh), _p(qkv), _p(meta), _p(k_cache), _p(v_cache),
                                   _p(page_table), _p(rope), C.byref(kv), C.byref(args), _p(runs), n_runs, max_run,
                                   _p(vis), _p(out), _p(ws.t), ws.nbytes, C.byref(ex) if ex is not None else None))


def mudd(cur: torch.Tensor, tap0: torch.Tensor, tap1: torch.Tensor, dense1: torch.Tensor, mix: torch.Tensor,
         out_attn: torch.Tensor, out_base: torch.Tensor, stream: int | None = None) -> None:
    """sv_mudd: the MUDD mixes of [n][hidden] rows (mix: one site's [2][3][33])."""
    n, hidden = cur.shape
    L.check(L.lib().sv_mudd(_stream(stream), _p(cur), _p(tap0), _p(tap1), _p(dense1), _p(mix), _p(out_attn),
                            _p(out_base), n, hidden))


def attn_verify_noalloc(shape: ModelShape, qkv: torch.Tensor, meta: torch.Tensor, k_cache: torch.Tensor,
                        v_cache: torch.Tensor, page_table: torch.Tensor, rope: torch.Tensor, kv: L.KvArgs,
                        args: L.AttnArgs, runs: torch.Tensor, n_runs: int, max_run: int, vis: torch.Tensor,
                        out: torch.Tensor, stream: int | None = None) -> None:
    """sv_attn_verify_noalloc: attn_verify with the library's static scratch (no allocation)."""
    sh = shape.c()
    L.check(L.lib().sv_attn_verify_noalloc(_stream(stream), C.byref(sh), _p(qkv), _p(meta), _p(k_cache), _p(v_cache),
                                           _p(page_table), _p(rope), C.byref(kv), C.byref(args), _p(runs), n_runs,
                                           max_run, _p(vis), _p(out)))


def draft_top(logits, vocab, tin, cand, cand_q, n_rows: int, nv: int, inv_t: float, ncand: int, stream=None) -> None:
    """sv_draft_top: each drafted block row's ncand best candidates and their probabilities."""
    L.check(L.lib().sv_draft_top(_stream(stream), _p(logits), _p(vocab), _p(tin), _p(cand), _p(cand_q), n_rows, nv,
                                 inv_t, ncand))


def draft_tree(blocks, nblocks: int, tin, cand, cand_q, feed, tree, ncand: int, stream=None) -> None:
    """sv_draft_tree: each block's DDTree into its slot's feed / tree entries."""
    L.check(L.lib().sv_draft_tree(_stream(stream), _p(blocks), nblocks, _p(tin), _p(cand), _p(cand_q), _p(feed),
                                  _p(tree), ncand))


def embed(shape: ModelShape, table, tokens, out, tin, meta, lens, feed, tree, vis, n: int, stream=None) -> None:
    sh = shape.c()
    L.check(L.lib().sv_embed(_stream(stream), C.byref(sh), _p(table), _p(tokens), _p(out), _p(tin), _p(meta), _p(lens),
                             _p(feed), _p(tree), _p(vis), n))


def rmsnorm_rows(x, rows, out, n: int, hidden: int, stream=None) -> None:
    L.check(L.lib().sv_rmsnorm_rows(_stream(stream), _p(x), _p(rows), _p(out), n, hidden))


def sample(logits, rows, out, meta, n_rows: int, vocab: int, stream=None) -> None:
    L.check(L.lib().sv_sample(_stream(stream), _p(logits), _p(rows), _p(out), _p(meta), n_rows, vocab))


def accept(runs, tokens, out, lens, feed, gen, emitted, nruns: int, tree, path, path_len, on_path, stream=None) -> None:
    L.check(L.lib().sv_accept(_stream(stream), _p(runs), _p(tokens), _p(out), _p(lens), _p(feed), _p(gen), _p(emitted),
                              nruns, _p(tree), _p(path), _p(path_len), _p(on_path)))


def kv_compact(shape: ModelShape, runs, nruns: int, path, path_len, lens, k_cache, v_cache, page_table,
               kv: L.KvArgs, stream=None) -> None:
    sh = shape.c()
    L.check(L.lib().sv_kv_compact(_stream(stream), C.byref(sh), _p(runs), nruns, _p(path), _p(path_len), _p(lens),
                                  _p(k_cache), _p(v_cache), _p(page_table), C.byref(kv)))


def replay_draft(runs, nruns: int, lens, feed, trace, trace_len, ra: L.ReplayArgs, tree, stream=None) -> None:
    L.check(L.lib().sv_replay_draft(_stream(stream), _p(runs), nruns, _p(lens), _p(feed), _p(trace), _p(trace_len),
                                    C.byref(ra), _p(tree)))
