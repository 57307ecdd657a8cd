"""Shared helpers of the parity tests: seeded inputs, the oracle, tolerance checks."""
from __future__ import annotations

import numpy as np
import torch

import oracle
import violetto
from violetto import _lib as L


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def to_dev(a: np.ndarray, dtype=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


def u16_dev_bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.uint16).view(np.int16)).cuda().view(torch.bfloat16)


def close(got: np.ndarray, want: np.ndarray, atol: float, rtol: float, what: str) -> None:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin), f"{what}: non-finite mismatch"
    err = np.abs(got[fin] - want[fin])
    lim = atol + rtol * np.abs(want[fin])
    bad = err > lim
    if bad.any():
        i = int(np.argmax(err - lim))
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside tol; worst |{got[fin][i]} - {want[fin][i]}| "
                             f"= {err[i]:.3e} > {lim[i]:.3e}")


def greedy_ids_match(ids_gpu, ids_ref, logits_ref, tol=2e-2) -> int:
    """Greedy ids must match wherever the reference's top-1 margin exceeds tol; returns the
    number of rows compared."""
    checked = 0
    for r in range(len(ids_ref)):
        row = np.sort(logits_ref[r][np.isfinite(logits_ref[r])])
        margin = row[-1] - row[-2] if row.size > 1 else np.inf
        if margin > tol:
            assert ids_gpu[r] == ids_ref[r], f"row {r}: id {ids_gpu[r]} != {ids_ref[r]} (margin {margin:.4f})"
            checked += 1
    return checked
