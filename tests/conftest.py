"""Test setup: the product package (silicon-violetto_amd/violetto) and the oracle binding
(oracle/oracle.py) on sys.path; the `gpu` marker for tests that need an MI355X."""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "silicon-violetto_amd"))
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libsv_verify.so on cuda:0)")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import violetto

    violetto.lib()  # loud failure if the library was not built
    return torch.device("cuda:0")


def banner(msg: str) -> None:
    """Name the case on stdout before a GPU step (a fault may end the box before pytest reports)."""
    print(f"[case] {msg}", flush=True)
    os.sync() if hasattr(os, "sync") else None
