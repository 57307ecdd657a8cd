"""Synthetic models of the benchmark configurations: shapes, int8/bf16 weights, RoPE.

Weights are random (there is no checkpoint offline): N(0, 0.02), int8 symmetric per output
channel with bf16 scales (tools/convert.py:41-50 `quantize` with group = k) or bf16, and a
tied bf16 embedding / head. Generation runs on the given torch device (the GPU for the
16-layer benchmark, the CPU for parity fixtures).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib as L


@dataclass(frozen=True)
class ModelShape:
    hidden: int = 2048
    n_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = 64
    ffn: int = 8192
    vocab: int = 32000
    vocab_real: int = 32000
    n_layers: int = 16

    @property
    def qkv_width(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim

    def c(self) -> L.Shape:
        return L.Shape(self.hidden, self.n_heads, self.n_kv_heads, self.head_dim, self.ffn, self.vocab,
                       self.vocab_real, self.n_layers)

    def weight_bytes(self, int8: bool = True) -> int:
        """Bytes one pass over every matrix reads (model.rs:41-46 Matrix::bytes), head included."""
        H, F = self.hidden, self.ffn
        mats = [(self.qkv_width, H), (H, self.n_heads * self.head_dim), (2 * F, H), (H, F)]
        per = sum(m * k + 2 * m for m, k in mats) if int8 else sum(2 * m * k for m, k in mats)
        return self.n_layers * per + 2 * self.vocab * H


# BASELINE.json configs[0..4] shapes; REFERENCE_SHAPE is the reference's own model
# (engine/src/model.rs:6-18), kept as a second parity shape.
CONFIG_SHAPE = ModelShape()
REFERENCE_SHAPE = ModelShape(hidden=1280, n_heads=10, n_kv_heads=2, head_dim=128, ffn=3328, vocab=151680,
                             vocab_real=151667, n_layers=48)


def rope_freq(theta: float = 500000.0, head_dim: int = 64) -> np.ndarray:
    """f_j = theta^(-2j / head_dim), j < 32: the 32 pairs of dims 0..63 the kernels rotate."""
    j = np.arange(L.ROPE_PAIRS, dtype=np.float64)
    return (theta ** (-2.0 * j / head_dim)).astype(np.float32)


def quantize_rows(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """int8 per output channel (tools/convert.py:41-50 with group = k): s = bf16(absmax / 127),
    q = clamp(round_half_even(w / s), -127, 127). Returns (q int8 [m][k], s bf16 [m][1])."""
    wf = w.float()
    s = (wf.abs().amax(-1, keepdim=True) / 127).to(torch.bfloat16)
    sf = s.float()
    q = torch.where(sf > 0, wf / sf, torch.zeros((), device=w.device)).round().clamp(-127, 127).to(torch.int8)
    return q, s


def quantize_groups(w: torch.Tensor, group: int) -> tuple[torch.Tensor, torch.Tensor]:
    """int8 over groups of `group` consecutive k (tools/convert.py:41-50): per group s =
    bf16(absmax / 127), q = clamp(round_half_even(w / s), -127, 127). Returns (q int8 [m][k],
    s bf16 [m][k / group])."""
    m, k = w.shape
    g = w.float().reshape(m, k // group, group)
    s = (g.abs().amax(-1) / 127).to(torch.bfloat16)
    sf = s.float().unsqueeze(-1)
    q = torch.where(sf > 0, g / sf, torch.zeros((), device=w.device)).round().clamp(-127, 127).to(torch.int8)
    return q.reshape(m, k), s


def gshift_of(k: int, scales: torch.Tensor) -> int:
    """sv_matrix.gshift of int8 scales [m][groups]: 31 for one per row, else log2(k / groups)."""
    groups = scales.shape[1]
    return 31 if groups == 1 else int(k // groups).bit_length() - 1


@dataclass
class LayerScalars:
    qkv_scale: float = 1.0
    o_scale: float = 1.0
    resid_attn: float = 1.0
    post_attn: float = 1.0
    resid_mlp: float = 1.0
    post_mlp: float = 1.0
    rope: int = 1


@dataclass
class Extras:
    """The Limite model's extras (engine/src/model.rs:49-99, kernels.metal:738-747,1316-1407):
    sliding-window layers, attention gates, value embeddings, XSA and the MUDD mixes. Per-layer
    lists hold None where a layer lacks the part."""
    local: list[int]                           # 1: sliding-window layer
    window: int
    attn_gate: list                            # f32 [n_heads][head_dim] or None
    ve_gate: list                              # f32 [n_kv_heads][12] or None
    xsa: list                                  # f32 [n_heads] or None
    value_embed: torch.Tensor | None = None    # bf16 [vocab][n_kv_heads * head_dim]
    mudd_dense1: torch.Tensor | None = None    # f32 [32][hidden]
    mudd_mix: torch.Tensor | None = None       # f32 [sites][2][3][33]
    mudd_layer: tuple = ()
    mudd_tap: tuple = ()

    def to(self, dev) -> "Extras":
        mv = lambda t: None if t is None else t.to(dev)  # noqa: E731
        return Extras(list(self.local), self.window, [mv(t) for t in self.attn_gate], [mv(t) for t in self.ve_gate],
                      [mv(t) for t in self.xsa], mv(self.value_embed), mv(self.mudd_dense1), mv(self.mudd_mix),
                      tuple(self.mudd_layer), tuple(self.mudd_tap))

    def c(self) -> L.ModelExtras:
        n = len(self.mudd_layer)
        ml = (L.u32 * L.MUDD_SITES)(*(list(self.mudd_layer) + [0] * (L.MUDD_SITES - n)))
        mt = (L.u32 * L.MUDD_SITES)(*(list(self.mudd_tap) + [0] * (L.MUDD_SITES - n)))
        ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        return L.ModelExtras(ptr(self.value_embed), ptr(self.mudd_dense1), ptr(self.mudd_mix), n, ml, mt, 0)


def limite_layout(n_layers: int) -> tuple[list[int], list[int], tuple, tuple]:
    """(local, has value embeddings, MUDD sites, their taps) of the reference's layer pattern
    (model.rs:21,116-127; encode.rs:107-122): global every fourth layer (i % 4 == 3), value
    embeddings on i % 3 == 1, MUDD before layers 24 and 47 with taps after 11 and 22; for
    other depths the sites sit at the middle and the last layer, the taps a quarter and half way."""
    local = [0 if i % 4 == 3 else 1 for i in range(n_layers)]
    ve = [1 if i % 3 == 1 else 0 for i in range(n_layers)]
    if n_layers == 48:
        return local, ve, (24, 47), (11, 22)
    if n_layers < 4:
        return local, ve, (), ()
    return local, ve, (n_layers // 2, n_layers - 1), (n_layers // 4, n_layers // 2 - 1)


def generate_extras(shape: ModelShape, *, seed: int = 1, device="cpu", window: int = 1024,
                    mudd: bool = True) -> Extras:
    """Random extras of the reference's layout (limite_layout): gates N(0, 0.05) (gates near 1),
    value embeddings N(0, 1) bf16, xsa U[0, 1), MUDD dense1 N(0, 0.05) and mixes around
    (attention input, residual base) = (0.1 tap0 + 0.1 tap1 + cur)."""
    dev = torch.device(device)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    rn = lambda *sz: torch.randn(*sz, generator=g, device=dev, dtype=torch.float32)  # noqa: E731
    local, ve, sites, taps = limite_layout(shape.n_layers)
    if not mudd:
        sites, taps = (), ()
    NQ, NKV, D = shape.n_heads, shape.n_kv_heads, shape.head_dim
    attn_gate = [rn(NQ, D) * 0.05 for _ in range(shape.n_layers)]
    ve_gate = [rn(NKV, L.VE_GATE_W) * 0.3 if v else None for v in ve]
    xsa = [torch.rand(NQ, generator=g, device=dev) for _ in range(shape.n_layers)]
    value_embed = rn(shape.vocab, NKV * D).to(torch.bfloat16) if any(ve) else None
    dense1 = mix = None
    if sites:
        dense1 = rn(L.MUDD_INNER, shape.hidden) * 0.05
        mix = rn(len(sites), 2, 3, L.MUDD_INNER + 1) * 0.02
        base = torch.tensor([0.1, 0.1, 1.0], device=dev)
        mix[:, :, :, L.MUDD_INNER] += base
    return Extras(local, window, attn_gate, ve_gate, xsa, value_embed, dense1, mix, tuple(sites), tuple(taps))


@dataclass
class SyntheticModel:
    shape: ModelShape
    int8: bool
    device: torch.device
    embed: torch.Tensor                       # bf16 [vocab][hidden]
    layers: list[dict] = field(default_factory=list)  # name -> (w, scales or None)
    scalars: list[LayerScalars] = field(default_factory=list)
    extras: Extras | None = None
    head: tuple | None = None                 # its own head (int8 q, scales) or None: the tied embedding

    @staticmethod
    def generate(shape: ModelShape, *, int8: bool = True, seed: int = 0, device: str | torch.device = "cpu",
                 scalars: LayerScalars | list[LayerScalars] | None = None, std: float = 0.02,
                 group: int | None = None) -> "SyntheticModel":
        """group: int8 scale groups of `group` k (the reference's default is 64); None: one per row."""
        dev = torch.device(device)
        g = torch.Generator(device=dev)
        g.manual_seed(seed)

        def normal(m: int, k: int) -> torch.Tensor:
            return torch.randn(m, k, generator=g, device=dev, dtype=torch.float32) * std

        H, F = shape.hidden, shape.ffn
        embed = normal(shape.vocab, H).to(torch.bfloat16)
        layers = []
        for _ in range(shape.n_layers):
            lay = {}
            for name, (m, k) in (("qkv", (shape.qkv_width, H)), ("o", (H, shape.n_heads * shape.head_dim)),
                                 ("gate_up", (2 * F, H)), ("down", (H, F))):
                w = normal(m, k)
                if not int8:
                    lay[name] = (w.to(torch.bfloat16), None)
                else:
                    lay[name] = quantize_rows(w) if group is None else quantize_groups(w, group)
                del w
            layers.append(lay)
        if scalars is None:
            sc = [LayerScalars() for _ in range(shape.n_layers)]
        elif isinstance(scalars, LayerScalars):
            sc = [scalars for _ in range(shape.n_layers)]
        else:
            sc = list(scalars)
        return SyntheticModel(shape, int8, dev, embed, layers, sc)

    def to(self, device: str | torch.device) -> "SyntheticModel":
        dev = torch.device(device)
        layers = [{k: (w.to(dev), None if s is None else s.to(dev)) for k, (w, s) in lay.items()} for lay in self.layers]
        return SyntheticModel(self.shape, self.int8, dev, self.embed.to(dev), layers, self.scalars,
                              None if self.extras is None else self.extras.to(dev),
                              None if self.head is None else tuple(t.to(dev) for t in self.head))

    def with_head(self, group: int | None) -> "SyntheticModel":
        """This model with an int8 head quantized from the embedding (tools/convert.py:111-112,
        `matrix("head", "head", embed)`): groups of `group` k, or one scale per row."""
        w = self.embed.float()
        q = quantize_rows(w) if group is None else quantize_groups(w, group)
        return SyntheticModel(self.shape, self.int8, self.device, self.embed, self.layers, self.scalars, self.extras, q)

    def c_head(self) -> L.Matrix | None:
        if self.head is None:
            return None
        q, s = self.head
        return L.Matrix(q.data_ptr(), s.data_ptr(), q.shape[0], q.shape[1], L.FMT_I8, gshift_of(q.shape[1], s))

    def with_extras(self, extras: Extras) -> "SyntheticModel":
        """This model with the Limite extras; RoPE on the sliding-window layers only
        (encode.rs:237 rope = !global)."""
        sc = [LayerScalars(s.qkv_scale, s.o_scale, s.resid_attn, s.post_attn, s.resid_mlp, s.post_mlp, int(loc))
              for s, loc in zip(self.scalars, extras.local)]
        return SyntheticModel(self.shape, self.int8, self.device, self.embed, self.layers, sc, extras.to(self.device),
                              self.head)

    def embed_ptr(self) -> int:
        return self.embed.data_ptr()

    def c_layer(self, i: int) -> L.Layer:
        """The sv_layer of layer i (device pointers: the model must live on the GPU)."""
        lay, s = self.layers[i], self.scalars[i]

        def mat(name: str) -> L.Matrix:
            w, sc = lay[name]
            m, k = w.shape
            if sc is None:
                return L.Matrix(w.data_ptr(), None, m, k, L.FMT_BF16, 0)
            return L.Matrix(w.data_ptr(), sc.data_ptr(), m, k, L.FMT_I8, gshift_of(k, sc))

        x = self.extras
        ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        return L.Layer(mat("qkv"), mat("o"), mat("gate_up"), mat("down"), s.qkv_scale, s.o_scale, s.resid_attn,
                       s.post_attn, s.resid_mlp, s.post_mlp, s.rope, 0, ptr(x.attn_gate[i]) if x else None,
                       ptr(x.ve_gate[i]) if x else None, ptr(x.xsa[i]) if x else None)
