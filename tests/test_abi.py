"""The C ABI (CPU only, no compute): libsv_verify.so loads and exports every entry point that
include/sv_verify.h declares; the ctypes structs match the C layouts; host-side argument
checks reject bad calls with the documented status codes before touching the GPU."""
from __future__ import annotations

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from violetto import _lib as L

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "sv_verify.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sv_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_what_binding_binds():
    assert declared_functions() == sorted(L.PROTOS), "header and ctypes binding disagree"


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} not exported"
    out = subprocess.run(["nm", "-D", "--defined-only", str(L.LIB_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (sv_[a-z0-9_]+)$", out, flags=re.M))
    assert set(declared_functions()) <= exported


STRUCTS = ["sv_shape", "sv_matrix", "sv_mat_args", "sv_kv_args", "sv_attn_args", "sv_sample_row", "sv_run_in",
           "sv_gen_state", "sv_replay_args", "sv_engine_config", "sv_layer", "sv_engine_buffers", "sv_run",
           "sv_plan_info", "sv_tensor_info", "sv_model_extras", "sv_attn_extras", "sv_draft_layer", "sv_drafter",
           "sv_draft_buffers", "sv_layer_capture"]
PY = {"sv_shape": L.Shape, "sv_matrix": L.Matrix, "sv_mat_args": L.MatArgs, "sv_kv_args": L.KvArgs,
      "sv_attn_args": L.AttnArgs, "sv_sample_row": L.SampleRow, "sv_run_in": L.RunIn, "sv_gen_state": L.GenState,
      "sv_replay_args": L.ReplayArgs, "sv_engine_config": L.EngineConfig, "sv_layer": L.Layer,
      "sv_engine_buffers": L.EngineBuffers, "sv_run": L.Run, "sv_plan_info": L.PlanInfo,
      "sv_tensor_info": L.TensorInfo, "sv_model_extras": L.ModelExtras, "sv_attn_extras": L.AttnExtras,
      "sv_draft_layer": L.DraftLayer, "sv_drafter": L.Drafter, "sv_draft_buffers": L.DraftBuffers,
      "sv_layer_capture": L.LayerCapture}


def test_struct_layouts_match_c(tmp_path):
    src = tmp_path / "sizes.c"
    src.write_text('#include <stdio.h>\n#include "sv_verify.h"\nint main(void){\n' +
                   "".join(f'printf("{s} %zu\\n", sizeof({s}));\n' for s in STRUCTS) + "return 0;}\n")
    exe = tmp_path / "sizes"
    subprocess.run(["gcc", "-std=c11", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    sizes = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True).stdout.split("\n")
                 if line)
    for s in STRUCTS:
        assert int(sizes[s]) == C.sizeof(PY[s]), f"{s}: C {sizes[s]} != ctypes {C.sizeof(PY[s])}"
    # The reference's #[repr(C)] structs (kernels.rs:36-136) keep their sizes.
    assert C.sizeof(L.MatArgs) == 48 and C.sizeof(L.KvArgs) == 32 and C.sizeof(L.AttnArgs) == 36
    assert C.sizeof(L.SampleRow) == 24 and C.sizeof(L.RunIn) == 24 and C.sizeof(L.GenState) == 48
    assert C.sizeof(L.ReplayArgs) == 16


def test_argument_checks_without_gpu():
    """Calls that fail validation return before any HIP call."""
    lib = L.lib()
    m = L.Matrix(None, None, 16, 256, L.FMT_I8, 31)
    a = L.MatArgs(1, 256, 16, L.EPI_RAW, 0, 16, 1.0, 0, 0, 1, 256, 31)
    assert lib.sv_matmul(None, C.byref(m), None, None, None, None, None, C.byref(a), None, 0) == 1
    assert b"null" in lib.sv_last_error()
    sh = L.Shape(2048, 32, 8, 96, 8192, 32000, 32000, 1)
    kv = L.KvArgs(1, 0, 0, 1, 4, 1, 1, 0)
    args = L.AttnArgs(128, 2, 0.18, 1, 0, 0, 0, 0, 0)
    one = C.c_void_p(16)
    rc = lib.sv_attn_verify(None, C.byref(sh), one, one, one, one, one, one, C.byref(kv), C.byref(args), one, 1, 5,
                            one, one, one, 1 << 20, None)
    assert rc == 4 and b"head_dim 96" in lib.sv_last_error()
    cfg = L.EngineConfig(L.Shape(2048, 32, 8, 64, 8192, 32000, 32000, 16), 1, 16, 1024, 16, 1024, 3, 0.125, 0)
    h = C.c_void_p()
    assert lib.sv_engine_create(C.byref(cfg), (C.c_float * 32)(), C.byref(h)) == 1  # page_shift 3
    assert lib.sv_new_seq(None, C.byref(C.c_uint32())) == 1


def test_workspace_sizes_grow_with_work():
    lib = L.lib()
    # split-k partials: the 1-16 row kernel with few row tiles and long k, and the GEMM path
    # (17+ rows) for narrow matrices
    assert lib.sv_matmul_workspace_bytes(5, 2048, 8192) > 0
    assert lib.sv_matmul_workspace_bytes(160, 2048, 8192) > 0
    assert lib.sv_matmul_workspace_bytes(600, 2048, 8192) > 0
    assert lib.sv_matmul_workspace_bytes(0, 2048, 8192) == 0
    sh = L.Shape(2048, 32, 8, 64, 8192, 32000, 32000, 16)
    assert lib.sv_attn_workspace_bytes(C.byref(sh), 32, 64, 16) > lib.sv_attn_workspace_bytes(C.byref(sh), 1, 64, 5)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus 2 exits with status 2 and says so (before any GPU work)."""
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parent.parent
    out = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=60, cwd=root)
    assert out.returncode == 2
    assert "one GPU" in out.stderr
