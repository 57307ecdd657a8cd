"""The drafter (engine/src/engine/drafter.rs; its model tools/spec/drafter.py, its file
tools/spec/export.py): a few layers of the target's shape that read the target's tapped
layers, and draft a block of rows per slot after each step.

SyntheticDrafter holds random weights laid out as export.py writes them: per tap an fc
[hidden][hidden] (the columns of fc.weight for that tap), kv_all (every layer's wk, wv
stacked), inject, per layer qkv (wq | wk | wv), o, gate_up (gate/up rows interleaved), down and
four two-tap convolutions (base [2][hidden], corrections [corr_rows][hidden] with rows past
hidden / 8 zero), the head with the final norm's gain folded in, mask_emb and the draft
vocabulary (target ids, ascending). Matrices are int8 in groups of 64 (export.py's default)
or bf16; the head in groups of `head_group` (export.py: 8).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib as L
from .model import ModelShape, gshift_of, quantize_groups, quantize_rows

TRAIN_TEMPERATURE = 0.6  # drafter.rs:19 TRAIN_TEMPERATURE: draft_top scores at 1 / 0.6


def corr_rows(hidden: int) -> int:
    """export.py:14 CONV_ROWS: the corrections' hidden / 8 rows padded to 64-row tiles."""
    return -(-(hidden // 8) // 64) * 64


@dataclass
class SyntheticDrafter:
    shape: ModelShape
    n_layers: int
    taps: tuple
    window: int
    device: torch.device
    mats: dict = field(default_factory=dict)      # name -> (w, scales or None)
    conv_base: dict = field(default_factory=dict)  # "D{i}.conv{c}" -> f32 [2][hidden]
    mask_emb: torch.Tensor | None = None           # f32 [hidden]
    vocab: torch.Tensor | None = None              # int32 [v]
    inv_temperature: float = 1.0 / TRAIN_TEMPERATURE

    @property
    def v(self) -> int:
        return int(self.vocab.numel())

    @property
    def convs(self) -> bool:
        return bool(self.conv_base)

    @property
    def inject(self) -> bool:
        return "inject" in self.mats

    @staticmethod
    def generate(shape: ModelShape, *, n_layers: int = 2, taps: tuple = (0, 1), v: int = 4096, window: int = 1024,
                 seed: int = 0, device: str | torch.device = "cpu", int8: bool = True, group: int = 64,
                 head_group: int | None = 8, convs: bool = True, inject: bool = True, std: float = 0.02,
                 head_std: float = 0.1, conv_std: float = 0.1) -> "SyntheticDrafter":
        """Random weights; convolutions near the identity (base (1, 0) plus noise, small
        corrections), as Conv2 starts (drafter.py:47-50) and drifts in training."""
        dev = torch.device(device)
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        H, F, NKV, D = shape.hidden, shape.ffn, shape.n_kv_heads, shape.head_dim

        def normal(*size, s=std) -> torch.Tensor:
            return torch.randn(*size, generator=g, device=dev, dtype=torch.float32) * s

        def mat(w: torch.Tensor, grp: int | None = group):
            if not int8:
                return (w.to(torch.bfloat16), None)
            return quantize_rows(w) if grp is None or grp >= w.shape[1] else quantize_groups(w, grp)

        d = SyntheticDrafter(shape, n_layers, tuple(taps), window, dev)
        for k in range(len(taps)):
            d.mats[f"fc.{k}"] = mat(normal(H, H))
        d.mats["kv_all"] = mat(normal(n_layers * 2 * NKV * D, H))
        if inject:
            d.mats["inject"] = mat(normal(H, H))
        d.mats["head"] = mat(normal(v, H, s=head_std), head_group)
        cr = corr_rows(H)
        for i in range(n_layers):
            p = f"D{i:02d}."
            d.mats[p + "qkv"] = mat(normal(shape.qkv_width, H))
            d.mats[p + "o"] = mat(normal(H, shape.n_heads * D))
            d.mats[p + "gate_up"] = mat(normal(2 * F, H))
            d.mats[p + "down"] = mat(normal(H, F))
            if convs:
                for c in range(4):
                    base = torch.stack([1.0 + normal(H, s=conv_std), normal(H, s=conv_std)]).contiguous()
                    d.conv_base[f"{p}conv{c}"] = base
                    corr = torch.cat([normal(H // 8, H), torch.zeros(cr - H // 8, H, device=dev)])
                    d.mats[f"{p}conv{c}.corr"] = mat(corr)
        d.mask_emb = normal(H)
        perm = torch.randperm(shape.vocab_real, generator=g, device=dev)[:v]
        d.vocab = perm.sort().values.to(torch.int32).contiguous()
        return d

    def to(self, device: str | torch.device) -> "SyntheticDrafter":
        dev = torch.device(device)
        mv = lambda t: None if t is None else t.to(dev)  # noqa: E731
        return SyntheticDrafter(self.shape, self.n_layers, self.taps, self.window, dev,
                                {k: (mv(w), mv(s)) for k, (w, s) in self.mats.items()},
                                {k: mv(t) for k, t in self.conv_base.items()}, mv(self.mask_emb), mv(self.vocab),
                                self.inv_temperature)

    # -- the C struct (device pointers when on the GPU, host pointers for the oracle)
    def _matrix(self, name: str, ptr) -> L.Matrix:
        if name not in self.mats:
            return L.Matrix(None, None, 0, 0, 0, 0)
        w, s = self.mats[name]
        m, k = w.shape
        if s is None:
            return L.Matrix(ptr(w), None, m, k, L.FMT_BF16, 0)
        return L.Matrix(ptr(w), ptr(s), m, k, L.FMT_I8, gshift_of(k, s))

    def c(self, ptr=None) -> L.Drafter:
        """The sv_drafter; `ptr` maps a tensor to its address (default: data_ptr()). The
        returned struct keeps its layer array alive."""
        ptr = ptr or (lambda t: t.data_ptr())
        layers = (L.DraftLayer * self.n_layers)()
        for i in range(self.n_layers):
            p = f"D{i:02d}."
            lay = layers[i]
            lay.qkv, lay.o = self._matrix(p + "qkv", ptr), self._matrix(p + "o", ptr)
            lay.gate_up, lay.down = self._matrix(p + "gate_up", ptr), self._matrix(p + "down", ptr)
            for c in range(4):
                key = f"{p}conv{c}"
                lay.conv_base[c] = ptr(self.conv_base[key]) if key in self.conv_base else None
                lay.conv_corr[c] = self._matrix(key + ".corr", ptr)
        d = L.Drafter()
        d.n_layers, d.n_taps, d.v = self.n_layers, len(self.taps), self.v
        for k, t in enumerate(self.taps):
            d.taps[k] = t
            d.fc[k] = self._matrix(f"fc.{k}", ptr)
        d.kv_all = self._matrix("kv_all", ptr)
        d.inject = self._matrix("inject", ptr)
        d.head = self._matrix("head", ptr)
        d.mask_emb = ptr(self.mask_emb)
        d.vocab = ptr(self.vocab)
        d.layers = C.cast(layers, C.POINTER(L.DraftLayer))
        d.inv_temperature = self.inv_temperature
        d.window = self.window
        d._layers = layers  # keep alive
        return d

    # -- dequantised float64 weights (for independent restatements in tests)
    def dense(self, name: str) -> torch.Tensor:
        w, s = self.mats[name]
        if s is None:
            return w.double()
        m, k = w.shape
        grp = k // s.shape[1]
        return (w.double().reshape(m, s.shape[1], grp) * s.double().unsqueeze(-1)).reshape(m, k)


BLOCK = 8  # tools/spec/drafter.py BLOCK: the meta tensor's block size (rows are set per slot here)


def drafter_tensors(d: SyntheticDrafter) -> dict[str, torch.Tensor]:
    """The tensors tools/spec/export.py:28-60 writes, under its names, for a SyntheticDrafter:
    int8 matrices as `<name>` + `<name>.scale`, convolution bases f32 [2][hidden], `mask_emb`,
    `vocab` (f32 ids) and `meta` (f32: layers, taps, block, window, vocabulary, the taps)."""
    out: dict[str, torch.Tensor] = {}
    for name, (w, s) in d.mats.items():
        out[name] = w
        if s is not None:
            out[name + ".scale"] = s
    for key, base in d.conv_base.items():
        out[key + ".base"] = base.float()
    out["mask_emb"] = d.mask_emb.float()
    out["vocab"] = d.vocab.float()
    out["meta"] = torch.tensor([d.n_layers, len(d.taps), BLOCK, d.window, d.v, *d.taps], dtype=torch.float32)
    return out


class VltDrafter:
    """A drafter served from an uploaded weight file with export.py's tensor names (the reader
    side of drafter.rs:145-241 `Drafter::load`): `meta`, `fc.k`, `kv_all`, `inject` (optional),
    `D{i}.qkv/o/gate_up/down`, `D{i}.conv{c}.base/.corr` (optional, all four or none), `head`,
    `mask_emb`, `vocab`. Shapes are checked as the reference checks them; the window is the
    file's (the reference also requires it to equal its engine's WINDOW)."""

    def __init__(self, wf, shape: ModelShape, inv_temperature: float = 1.0 / TRAIN_TEMPERATURE):
        self.wf, self.shape, self.device = wf, shape, torch.device("cuda")
        meta = wf.read("meta")
        if meta.size < 5:
            raise ValueError(f"meta {meta.tolist()}")
        n_layers, n_taps, window, v = int(meta[0]), int(meta[1]), int(meta[3]), int(meta[4])
        if meta.size != 5 + n_taps:
            raise ValueError(f"window {window}, meta {meta.tolist()}")
        self.n_layers, self.window, self.taps = n_layers, window, tuple(int(t) for t in meta[5:])
        self.inv_temperature = inv_temperature
        H, F, NKV, D = shape.hidden, shape.ffn, shape.n_kv_heads, shape.head_dim
        self.fc = [wf.matrix(f"fc.{k}", H, H) for k in range(n_taps)]
        self.kv_all = wf.matrix("kv_all", n_layers * 2 * NKV * D, H)
        self.inject = wf.matrix("inject", H, H) if wf.has("inject") else None
        self.head = wf.matrix("head", v, H)
        self.layers = []
        for i in range(n_layers):
            p = f"D{i:02d}."
            lay = dict(qkv=wf.matrix(p + "qkv", shape.qkv_width, H), o=wf.matrix(p + "o", H, shape.n_heads * D),
                       gate_up=wf.matrix(p + "gate_up", 2 * F, H), down=wf.matrix(p + "down", H, F), convs=None)
            if wf.has(p + "conv0.base"):
                convs = []
                for c in range(4):
                    wf.check(f"{p}conv{c}.base", 0, (2, H))
                    corr = wf.find(f"{p}conv{c}.corr")
                    convs.append((wf.device_ptr(f"{p}conv{c}.base"), wf.matrix(f"{p}conv{c}.corr", corr.shape[0], H)))
                lay["convs"] = convs
            self.layers.append(lay)
        wf.check("mask_emb", 0, (H,))
        self.mask_emb = wf.device_ptr("mask_emb")
        wf.check("vocab", 0, (v,))
        ids = wf.read("vocab")
        if not np.array_equal(ids, np.round(ids)) or ids.min() < 0 or ids.max() >= shape.vocab_real:
            raise ValueError("vocab: the draft vocabulary's ids must be target ids")
        self.vocab = torch.from_numpy(ids.astype(np.int32)).to(self.device)
        self.v = v

    @property
    def convs(self) -> bool:
        return self.layers[0]["convs"] is not None

    def c(self) -> L.Drafter:
        layers = (L.DraftLayer * self.n_layers)()
        for i, lay in enumerate(self.layers):
            dl = layers[i]
            dl.qkv, dl.o, dl.gate_up, dl.down = lay["qkv"], lay["o"], lay["gate_up"], lay["down"]
            for c in range(4):
                if lay["convs"] is not None:
                    dl.conv_base[c], dl.conv_corr[c] = lay["convs"][c]
        d = L.Drafter()
        d.n_layers, d.n_taps, d.v = self.n_layers, len(self.taps), self.v
        for k, t in enumerate(self.taps):
            d.taps[k] = t
            d.fc[k] = self.fc[k]
        d.kv_all = self.kv_all
        d.inject = self.inject if self.inject is not None else L.Matrix(None, None, 0, 0, 0, 0)
        d.head = self.head
        d.mask_emb = self.mask_emb
        d.vocab = self.vocab.data_ptr()
        d.layers = C.cast(layers, C.POINTER(L.DraftLayer))
        d.inv_temperature = self.inv_temperature
        d.window = self.window
        d._layers = layers
        return d
