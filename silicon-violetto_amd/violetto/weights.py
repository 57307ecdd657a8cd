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

    def matrix(self, name: str, m: int, k: int) -> L.Matrix:
        out = L.Matrix()
        L.check(self.lib.sv_weights_matrix(self.h, name.encode(), m, k, C.byref(out)))
        return out


class VltModel:
    """A model served from an uploaded weight file with the reference's tensor names
    (engine/src/model.rs:109-141): `embed` (bf16 [vocab][hidden]), per layer `Lnn.qkv`, `.o`,
    `.gate_up`, `.down` (bf16, or int8 with `.scale`) and `Lnn.scalars` (f32 [8]: qkv_scale,
    o_scale, resid_attn, post_attn, resid_mlp, post_mlp, ...). RoPE on every layer."""

    def __init__(self, wf: WeightFile, shape: ModelShape):
        self.wf, self.shape = wf, shape
        H, F = shape.hidden, shape.ffn
        self.mats, self.scalars = [], []
        for i in range(shape.n_layers):
            n = f"L{i:02d}."
            self.mats.append([wf.matrix(n + "qkv", shape.qkv_width, H), wf.matrix(n + "o", H, shape.n_heads * shape.head_dim),
                              wf.matrix(n + "gate_up", 2 * F, H), wf.matrix(n + "down", H, F)])
            s = wf.read(n + "scalars")
            self.scalars.append(LayerScalars(*[float(x) for x in s[:6]]))
        t = wf.find("embed")
        assert t.dtype == 1 and tuple(t.shape[:2]) == (shape.vocab, H), "embed: bf16 [vocab][hidden]"
        self._embed = wf.device_ptr("embed")

    def embed_ptr(self) -> int:
        return self._embed

    def c_layer(self, i: int) -> L.Layer:
        s = self.scalars[i]
        return L.Layer(*self.mats[i], s.qkv_scale, s.o_scale, s.resid_attn, s.post_attn, s.resid_mlp, s.post_mlp,
                       s.rope, 0)
