"""bench.py's output contract on the GPU: one JSON line with the metric of BASELINE.json, the
measured value, the roofline and CPU-baseline objects; run as a child process with a tiny
configs[1] workload, a short configs[2] leg, the other configs off."""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

from conftest import banner

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parent.parent


def test_bench_json_contract(gpu):
    banner("bench.py contract (configs[1], 3 steps)")
    cmd = [sys.executable, str(ROOT / "bench.py"), "--steps", "3", "--warmup", "1", "--streams32-steps", "3",
           "--long-steps", "0", "--tree-steps", "0", "--cpu-steps", "1", "--cpu-streams", "1", "--profile-reps", "1"]
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=115, cwd=ROOT)
    assert out.returncode == 0, out.stderr[-2000:]
    lines = [ln for ln in out.stdout.splitlines() if ln.startswith("{")]
    assert len(lines) == 1, out.stdout[-2000:]
    d = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
                "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in d, key
    assert d["n_gpus"] == 1 and d["steps"] == 3 and d["warmup"] == 1 and d["higher_is_better"] is True
    assert d["value"] > 0 and d["ms_per_step"] > 0 and d["vs_baseline"] is None
    assert d["config"]["workload"].startswith("configs[1]")
    r = d["roofline"]
    assert r["bound"] in ("hbm", "mfma") and r["peak"] > 0 and 0 < r["frac"] <= 1.0
    assert abs(r["frac"] - r["achieved"] / r["peak"]) < 1e-3
    c = d["cpu_baseline"]
    assert c["value"] > 0 and c["cores"] >= 1 and c["kind"] in ("port", "reference") and c["sample"]
    # The measured steps are correct: configs[1]'s greedy verify steps reproduce the plain decode,
    # and the oracle's steps on the CPU emit the GPU's tokens.
    assert d["lossless_trace_check"] is True
    assert c["matches_gpu"] is True
    # configs[2] (32 streams, T = 0.7, nearly flat distributions over 32000 ids): a stream leaves
    # its sampled plain decode only where the decode (32 rows) and the verify (160 rows), whose
    # fp32 sums round differently, put a CDF edge on different sides of the shared uniform: the
    # drawn id is then the recorded id's neighbour in the sampler's order. Every stream that
    # leaves its trace, in the checked warm-up steps or in the timed ones (re-run one at a time
    # from the same device state, which reproduces the timed run's tokens), is such a neighbour.
    s32 = d["streams32"]
    assert s32["config"]["rows_per_step"] == 160 and s32["value"] > 0
    div = s32["divergences"]
    assert all(x["order_distance"] == 1 for x in div), div
    assert s32["rerun_emitted"] == s32["emitted"], s32
    assert s32["lossless_streams"] >= 32 - len(div), s32
    assert s32["cpu_baseline"]["value"] > 0 and s32["cpu_baseline"]["kind"] == "port"
