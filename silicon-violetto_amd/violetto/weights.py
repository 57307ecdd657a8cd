"""The weight file of the reference engine (engine/src/weights.rs:38-74; the layout
tools/convert.py:117-150 documents), through include/sv_verify.h's sv_weights_* calls, and a
writer of the same layout for synthetic models.

Layout (little endian): "VIOLETTO", u32 version 1, u32 tensor count, u64 data-region offset
(16 KiB aligned), two reserved u32; then one 128-byte record per tensor (name[64] NUL padded,
u32 dtype 0 f32 / 1 bf16 / 2 int8, u32 ndim, u32 shape[4], u64 offset from the data region,
u64 bytes, 24 reserved); tensors 256-byte aligned in the data region.
"""
from __future__ import annotations

import ctypes as C
import struct
from pathlib import Path

import numpy as np
import torch

from . import _lib as L
from .model import LayerScalars, ModelShape

DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.int8: 2}
DATA_ALIGN, TENSOR_ALIGN = 16384, 256


def write_vlt(path: str | Path, tensors: dict[str, torch.Tensor]) -> None:
    """Writes `tensors` (f32, bf16 or int8, at most 4 dimensions, names under 64 bytes)."""
    records, blobs, off = [], [], 0
    for name, t in tensors.items():
        t = t.detach().cpu().contiguous()
        assert t.dtype in DTYPES and t.dim() <= 4 and len(name.encode()) < 64, name
        off = -(-off // TENSOR_ALIGN) * TENSOR_ALIGN
        raw = t.view(torch.uint8).numpy().tobytes() if t.numel() else b""
        shape = list(t.shape) + [0] * (4 - t.dim())
        records.append(struct.pack("<64sII4IQQ24x", name.encode(), DTYPES[t.dtype], t.dim(), *shape, off, len(raw)))
        blobs.append((off, raw))
        off += len(raw)
    data_offset = -(-(32 + 128 * len(records)) // DATA_ALIGN) * DATA_ALIGN
    with open(path, "wb") as fh:
        fh.write(struct.pack("<8sIIQII", b"VIOLETTO", 1, len(records), data_offset, 0, 0))
        fh.writelines(records)
        for o, raw in blobs:
            fh.seek(data_offset + o)
            fh.write(raw)
        fh.truncate(data_offset + -(-off // DATA_ALIGN) * DATA_ALIGN)


class WeightFile:
    """sv_weights_*: records checked on open; upload() puts every tensor in one device buffer."""

    def __init__(self, path: str | Path):
        self.lib = L.lib()
        h = C.c_void_p()
        L.check(self.lib.sv_weights_open(str(path).encode(), C.byref(h)))
        self.h = h

    def close(self) -> None:
        if self.h:
            self.lib.sv_weights_close(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        return self.lib.sv_weights_count(self.h)

    def info(self, i: int) -> L.TensorInfo:
        t = L.TensorInfo()
        L.check(self.lib.sv_weights_info(self.h, i, C.byref(t)))
        return t

    def find(self, name: str) -> L.TensorInfo:
        t = L.TensorInfo()
        L.check(self.lib.sv_weights_find(self.h, name.encode(), C.byref(t)))
        return t

    def read(self, name: str) -> np.ndarray:
        """A tensor's bytes from the file, as numpy (f32, uint16 bf16 bits or int8)."""
        t = self.find(name)
        dt = {0: np.float32, 1: np.uint16, 2: np.int8}[t.dtype]
        out = np.zeros(tuple(t.shape[: t.ndim]), dt)
        L.check(self.lib.sv_weights_read(self.h, name.encode(), out.ctypes.data, out.nbytes))
        return out

    def upload(self, stream: int | None = None) -> None:
        L.check(self.lib.sv_weights_upload(self.h, stream if stream is not None else torch.cuda.current_stream().cuda_stream))

    def device_ptr(self, name: str) -> int:
        p = C.c_void_p()
        L.check(self.lib.sv_weights_device(self.h, name.encode(), C.byref(p)))
        return p.value

    def has(self, name: str) -> bool:
        t = L.TensorInfo()
        return self.lib.sv_weights_find(self.h, name.encode(), C.byref(t)) == 0

    def check(self, name: str, dtype: int, shape: tuple) -> None:
        """Raises unless `name` has this dtype (0 f32, 1 bf16, 2 int8) and shape (model.rs get)."""
        t = self.find(name)
        got = tuple(t.shape[: t.ndim])
        if t.dtype != dtype or got != tuple(shape):
            raise ValueError(f"{name}: dtype {t.dtype} shape {got}, expected dtype {dtype} shape {tuple(shape)}")

    def matrix(self, name: str, m: int, k: int) -> L.Matrix:
        out = L.Matrix()
        L.check(self.lib.sv_weights_matrix(self.h, name.encode(), m, k, C.byref(out)))
        return out


class _FileExtras:
    """The Limite extras of a weight file, as the engine takes them (device pointers into the
    uploaded file)."""

    def __init__(self, wf: "WeightFile", local: list[int], window: int, sites: tuple, taps: tuple):
        self.local, self.window = local, window
        self.mudd_layer, self.mudd_tap = sites, taps
        self._ptrs = (wf.device_ptr("value_embed") if wf.has("value_embed") else None,
                      wf.device_ptr("mudd.dense1") if sites else None, wf.device_ptr("mudd.mix") if sites else None)

    def c(self) -> L.ModelExtras:
        n = len(self.mudd_layer)
        pad = [0] * (L.MUDD_SITES - n)
        return L.ModelExtras(*self._ptrs, n, (L.u32 * L.MUDD_SITES)(*(list(self.mudd_layer) + pad)),
                             (L.u32 * L.MUDD_SITES)(*(list(self.mudd_tap) + pad)), 0)


class VltModel:
    """A model served from an uploaded weight file with the reference's tensor names
    (engine/src/model.rs:109-141, tools/convert.py:76-113): `embed` (bf16 [vocab][hidden]), per
    layer `Lnn.qkv`, `.o`, `.gate_up`, `.down` (bf16, or int8 with `.scale`) and `Lnn.scalars`
    (f32 [8]: qkv_scale, o_scale, resid_attn, post_attn, resid_mlp, post_mlp, ...), and `head`
    (its own, usually int8) when the file has one.

    A file with the Limite tensors (`Lnn.attn_gate` f32 [n_heads][head_dim], `Lnn.xsa` f32
    [n_heads], `Lnn.ve_gate` f32 [n_kv_heads][12] on the layers with value embeddings,
    `value_embed` bf16 [vocab][n_kv_heads head_dim], `mudd.dense1` f32 [32][hidden], `mudd.mix` f32
    [2][2][3][33], `rope_freq` f32 [32]) gets the reference's layer pattern (model.rs:116: every
    fourth layer global, the others sliding-window layers of `window` keys with RoPE; MUDD sites
    and taps as limite_layout gives them); otherwise every layer is global with RoPE."""

    def __init__(self, wf: WeightFile, shape: ModelShape, window: int = 1024):
        from .model import limite_layout

        self.wf, self.shape = wf, shape
        H, F, NQ, NKV, D = shape.hidden, shape.ffn, shape.n_heads, shape.n_kv_heads, shape.head_dim
        self.limite = wf.has("L00.attn_gate")
        local, _, sites, taps = limite_layout(shape.n_layers)
        if not self.limite:
            local = [0] * shape.n_layers
        elif not wf.has("mudd.dense1"):
            sites, taps = (), ()
        self.mats, self.scalars, self.ex_ptrs = [], [], []
        for i in range(shape.n_layers):
            n = f"L{i:02d}."
            self.mats.append([wf.matrix(n + "qkv", shape.qkv_width, H), wf.matrix(n + "o", H, NQ * D),
                              wf.matrix(n + "gate_up", 2 * F, H), wf.matrix(n + "down", H, F)])
            s = wf.read(n + "scalars")
            self.scalars.append(LayerScalars(*[float(x) for x in s[:6]], rope=0 if self.limite and not local[i] else 1))
            ptrs = [None, None, None]
            if self.limite:
                wf.check(n + "attn_gate", 0, (NQ, D))
                wf.check(n + "xsa", 0, (NQ,))
                ptrs[0], ptrs[2] = wf.device_ptr(n + "attn_gate"), wf.device_ptr(n + "xsa")
                if wf.has(n + "ve_gate"):
                    wf.check(n + "ve_gate", 0, (NKV, L.VE_GATE_W))
                    ptrs[1] = wf.device_ptr(n + "ve_gate")
            self.ex_ptrs.append(ptrs)
        wf.check("embed", 1, (shape.vocab, H))
        self._embed = wf.device_ptr("embed")
        self.extras = None
        if self.limite:
            if any(p[1] for p in self.ex_ptrs):
                wf.check("value_embed", 1, (shape.vocab, NKV * D))
            if sites:
                wf.check("mudd.dense1", 0, (L.MUDD_INNER, H))
                wf.check("mudd.mix", 0, (2, 2, 3, L.MUDD_INNER + 1))
            self.extras = _FileExtras(wf, local, window, tuple(sites), tuple(taps))
        self._head = wf.matrix("head", shape.vocab, H) if wf.has("head") else None

    def rope_freq(self) -> np.ndarray | None:
        """The file's RoPE frequencies (f32 [32], tools/convert.py:59-61), if it has them."""
        return self.wf.read("rope_freq") if self.wf.has("rope_freq") else None

    def embed_ptr(self) -> int:
        return self._embed

    def c_head(self) -> L.Matrix | None:
        return self._head

    def c_layer(self, i: int) -> L.Layer:
        s = self.scalars[i]
        return L.Layer(*self.mats[i], s.qkv_scale, s.o_scale, s.resid_attn, s.post_attn, s.resid_mlp, s.post_mlp,
                       s.rope, 0, *self.ex_ptrs[i])


def reference_tensors(model, rope_freq: np.ndarray | None = None) -> dict[str, torch.Tensor]:
    """The tensors tools/convert.py:76-113 writes, under its names, for a SyntheticModel (with
    its Limite extras, its own head and RoPE frequencies when given): the writer side of
    VltModel."""
    out = {"embed": model.embed}
    if rope_freq is not None:
        out["rope_freq"] = torch.from_numpy(np.ascontiguousarray(rope_freq, np.float32))
    x = model.extras
    if x is not None:
        if x.value_embed is not None:
            out["value_embed"] = x.value_embed
        if x.mudd_dense1 is not None:
            out["mudd.dense1"] = x.mudd_dense1.float()
            mix = torch.zeros(2, 2, 3, L.MUDD_INNER + 1)
            mix[: x.mudd_mix.shape[0]] = x.mudd_mix.float().cpu()
            out["mudd.mix"] = mix
    for i, (lay, s) in enumerate(zip(model.layers, model.scalars)):
        n = f"L{i:02d}."
        for name, (w, sc) in lay.items():
            out[n + name] = w
            if sc is not None:
                out[n + name + ".scale"] = sc
        if x is not None:
            out[n + "attn_gate"] = x.attn_gate[i].float()
            if x.ve_gate[i] is not None:
                out[n + "ve_gate"] = x.ve_gate[i].float()
            out[n + "xsa"] = x.xsa[i].float()
        out[n + "scalars"] = torch.tensor([s.qkv_scale, s.o_scale, s.resid_attn, s.post_attn, s.resid_mlp, s.post_mlp,
                                           0.0, 0.0])
    if getattr(model, "head", None) is not None:
        out["head"], out["head.scale"] = model.head
    return out
