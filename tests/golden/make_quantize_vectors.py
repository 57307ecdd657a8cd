"""Writes quantize_vectors.npz: inputs and outputs of the reference converter's int8
quantisation (tools/convert.py:41-50 `quantize`), imported from a checkout of the reference,
for tests/test_oracle.py to compare orc_quantize with bit for bit. Run in a container that has
the reference (default /root/reference; argument 1 overrides it); the tests read only the .npz.

Inputs (seed 7): Gaussian rows at the configs' scale (N(0, 0.02)) and at large and tiny scales,
a zero row, rows of exact half steps of a power-of-two scale (ties), rows whose absmax / 127
rounds down in bf16 (the clamp case), signed outliers; groups of 8, 64 and 512 (one scale per
row at k = 512)."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
sys.path.insert(0, str(ref / "tools"))
from convert import quantize  # noqa: E402

rng = np.random.default_rng(7)
k = 512
rows = [rng.normal(0, 0.02, k), rng.normal(0, 0.02, k), rng.normal(0, 3.0, k), rng.normal(0, 1e-5, k), np.zeros(k)]
s = 2.0 ** -7
rows.append(np.tile(np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 3.0, -126.5]), k // 8) * s)
clamp = rng.normal(0, 0.02, k)
clamp[::8] = 0.0999  # absmax / 127 rounds down in bf16 for many groups
rows.append(clamp)
out = rng.normal(0, 0.02, k)
out[5], out[300] = 0.9, -1.3
rows.append(out)
w = np.stack(rows).astype(np.float32)
arrays = {"w": w}
for group in (8, 64, 512):
    q, sc = quantize(torch.from_numpy(w), group)
    arrays[f"q{group}"] = q.numpy()
    arrays[f"s{group}"] = sc.view(torch.int16).numpy().view(np.uint16)
np.savez(Path(__file__).with_name("quantize_vectors.npz"), **arrays)
print({k: v.shape for k, v in arrays.items()})
