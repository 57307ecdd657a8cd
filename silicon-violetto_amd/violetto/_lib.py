"""ctypes binding of libsv_verify.so (include/sv_verify.h).

The library is built in-tree (`make -C silicon-violetto_amd`, or __graft_entry__.build());
loading fails loudly when it is missing: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

# torch ships its own HIP runtime (libamdhip64.so.7); importing it first makes the library's
# dependency on that soname resolve to the same runtime, so both share one HIP context.
import torch  # noqa: F401

PKG_DIR = Path(__file__).resolve().parent.parent
LIB_PATH = PKG_DIR / "libsv_verify.so"

FEED_ROW = 0xFFFF0000
FEED_W = 16
NO_TOK = 0xFFFFFFFF
NO_PARENT = 0xFF
MAX_STOP = 8
MAX_RUN = 16
SAMPLE_THREADS = 1024
RMS_EPS = 1.1920928955078125e-07
ROPE_PAIRS = 32
VE_GATE_W = 12
MUDD_INNER = 32
MUDD_SITES = 2
MAX_COLS = 64
DRAFT_TAPS = 4
DRAFT_LAYERS = 8
DRAFT_CANDS = 4

EPI_NORM, EPI_RESID, EPI_SWIGLU, EPI_HEAD, EPI_RAW = 1, 2, 3, 4, 5
FLAG_WRITE_INV, FLAG_WRITE_RAW, FLAG_NORM_IN = 1, 2, 4
FMT_BF16, FMT_I8 = 0, 1
FMT_TILED = 0x10  # layout flag: 16-row tiles in matrix-core lane order (sv_pack_matrix)
STEP_REPLAY, STEP_COMPACT, STEP_NO_COMPACT, STEP_DRAFT = 1, 2, 4, 8
KINDS = ("embed", "qkv", "attn", "o", "gate_up", "down", "head", "sample", "accept", "compact", "replay", "attn_merge", "kv_write",
         "mudd", "draft", "layers")
OPT_LAYERS_KERNEL = 1

STATUS = {0: "OK", 1: "ERR_ARG", 2: "ERR_HIP", 3: "ERR_CAPACITY", 4: "ERR_UNSUPPORTED", 5: "ERR_STATE"}

u32 = C.c_uint32
f32 = C.c_float
vp = C.c_void_p


class Shape(C.Structure):
    _fields_ = [(n, u32) for n in ("hidden", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab", "vocab_real", "n_layers")]


class Matrix(C.Structure):
    _fields_ = [("d_w", vp), ("d_scales", vp), ("m", u32), ("k", u32), ("format", u32), ("gshift", u32)]


class MatArgs(C.Structure):
    _fields_ = [("n", u32), ("k", u32), ("m", u32), ("epi", u32), ("flags", u32), ("vocab_real", u32),
                ("scale", f32), ("ra", f32), ("rb", f32), ("ksplit", u32), ("kchunk", u32), ("gshift", u32)]


class KvArgs(C.Structure):
    _fields_ = [(n, u32) for n in ("is_global", "kv_layer", "ring", "max_seqs", "page_shift", "n_pages", "max_pages", "window")]


class AttnArgs(C.Structure):
    _fields_ = [("split", u32), ("max_splits", u32), ("scale_log2", f32), ("rope", u32), ("ve", u32),
                ("capture", u32), ("fixed_splits", u32), ("col_sets", u32), ("one_round", u32)]


class SampleRow(C.Structure):
    _fields_ = [("seed_lo", u32), ("seed_hi", u32), ("pos", u32), ("temperature", f32), ("top_p", f32), ("tok", u32)]


class RunIn(C.Structure):
    _fields_ = [(n, u32) for n in ("slot", "first", "count", "head0", "nhead", "verify")]


class GenState(C.Structure):
    _fields_ = [("remaining", u32), ("done", u32), ("nstop", u32), ("pad", u32), ("stop", u32 * MAX_STOP)]


class ReplayArgs(C.Structure):
    _fields_ = [("stride", u32), ("seed", u32), ("rate", f32), ("vocab", u32)]


class EngineConfig(C.Structure):
    _fields_ = [("shape", Shape), ("max_seqs", u32), ("max_step_tokens", u32), ("max_seq_len", u32),
                ("max_head_rows", u32), ("kv_tokens", u32), ("page_shift", u32), ("attn_scale", f32),
                ("split_keys", u32), ("options", u32), ("window", u32), ("pad", u32), ("local", vp)]


class Layer(C.Structure):
    _fields_ = [("qkv", Matrix), ("o", Matrix), ("gate_up", Matrix), ("down", Matrix), ("qkv_scale", f32),
                ("o_scale", f32), ("resid_attn", f32), ("post_attn", f32), ("resid_mlp", f32), ("post_mlp", f32),
                ("rope", u32), ("pad", u32), ("attn_gate", vp), ("ve_gate", vp), ("xsa", vp)]


class ModelExtras(C.Structure):
    _fields_ = [("value_embed", vp), ("mudd_dense1", vp), ("mudd_mix", vp), ("n_mudd", u32),
                ("mudd_layer", u32 * MUDD_SITES), ("mudd_tap", u32 * MUDD_SITES), ("pad", u32)]


class AttnExtras(C.Structure):
    _fields_ = [(n, vp) for n in ("d_x", "d_inv", "d_tokens", "d_value_embed", "d_ve_gate", "d_attn_gate", "d_xsa",
                                  "d_vdir")] + [("hidden", u32), ("pad", u32)]


class EngineBuffers(C.Structure):
    _fields_ = [(n, vp) for n in ("d_k_cache", "d_v_cache", "d_page_table", "d_lens", "d_feed", "d_tree", "d_gen",
                                  "d_trace", "d_trace_len", "d_logits", "d_rope", "d_out_ids", "d_emitted", "d_path",
                                  "d_path_len")] + [("n_pages", u32), ("max_pages", u32), ("kv_bytes", C.c_size_t),
                                                    ("d_k_local", vp), ("d_v_local", vp), ("d_local_table", vp),
                                                    ("n_local_pages", u32), ("ring_pages", u32),
                                                    ("local_bytes", C.c_size_t)]


class DraftLayer(C.Structure):
    _fields_ = [("qkv", Matrix), ("o", Matrix), ("gate_up", Matrix), ("down", Matrix), ("conv_base", vp * 4),
                ("conv_corr", Matrix * 4)]


class Drafter(C.Structure):
    _fields_ = [("n_layers", u32), ("n_taps", u32), ("v", u32), ("taps", u32 * DRAFT_TAPS), ("fc", Matrix * DRAFT_TAPS),
                ("kv_all", Matrix), ("inject", Matrix), ("head", Matrix), ("mask_emb", vp), ("vocab", vp),
                ("layers", C.POINTER(DraftLayer)), ("inv_temperature", f32), ("window", u32)]


class DraftBuffers(C.Structure):
    _fields_ = [("d_logits", vp), ("d_cand", vp), ("d_cand_q", vp), ("d_ctx", vp), ("d_taps", vp * DRAFT_TAPS),
                ("d_k_ring", vp), ("d_v_ring", vp), ("d_table", vp), ("ring_pages", u32), ("n_pages", u32),
                ("max_pages", u32), ("pad", u32)]


class Run(C.Structure):
    _fields_ = [("slot", u32), ("count", u32), ("tokens", C.POINTER(u32)), ("verify", u32), ("head", u32)]


class TensorInfo(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("dtype", u32), ("ndim", u32), ("shape", u32 * 4), ("offset", C.c_uint64),
                ("nbytes", C.c_uint64)]


class PlanInfo(C.Structure):
    _fields_ = [(n, u32) for n in ("n_tokens", "n_head", "n_runs", "branches", "max_run", "split", "max_splits")]


class LayerCapture(C.Structure):
    _fields_ = ([(n, u32) for n in ("layer", "n", "hidden", "qkv_width", "sdpa_width", "pad")] +
                [(n, C.POINTER(C.c_float)) for n in ("resid_in", "attn_in", "qkv", "sdpa_out", "attn_out", "mlp_in",
                                                     "mlp_out", "resid_base")])


CAPTURE_FN = C.CFUNCTYPE(None, C.POINTER(LayerCapture), C.c_void_p)

P = C.POINTER
# name -> (restype, argtypes): every entry point include/sv_verify.h declares.
PROTOS = {
    "sv_last_error": (C.c_char_p, []),
    "sv_embed": (C.c_int, [vp, P(Shape), vp, vp, vp, vp, vp, vp, vp, vp, vp, u32]),
    "sv_rmsnorm_rows": (C.c_int, [vp, vp, vp, vp, u32, u32]),
    "sv_matmul_workspace_bytes": (C.c_size_t, [u32, u32, u32]),
    "sv_matmul": (C.c_int, [vp, P(Matrix), vp, vp, vp, vp, vp, P(MatArgs), vp, C.c_size_t]),
    "sv_pack_matrix": (C.c_int, [vp, P(Matrix), vp, P(Matrix)]),
    "sv_attn_workspace_bytes": (C.c_size_t, [P(Shape), u32, u32, u32]),
    "sv_attn_verify": (C.c_int, [vp, P(Shape), vp, vp, vp, vp, vp, vp, P(KvArgs), P(AttnArgs), vp, u32, u32, vp, vp,
                                 vp, C.c_size_t, P(AttnExtras)]),
    "sv_mudd": (C.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, u32, u32]),
    "sv_attn_noalloc_max_bytes": (C.c_size_t, []),
    "sv_attn_verify_noalloc": (C.c_int, [vp, P(Shape), vp, vp, vp, vp, vp, vp, P(KvArgs), P(AttnArgs), vp, u32, u32,
                                         vp, vp]),
    "sv_sample": (C.c_int, [vp, vp, vp, vp, vp, u32, u32]),
    "sv_accept": (C.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, u32, vp, vp, vp, vp]),
    "sv_kv_compact": (C.c_int, [vp, P(Shape), vp, u32, vp, vp, vp, vp, vp, vp, P(KvArgs)]),
    "sv_draft_top": (C.c_int, [vp, vp, vp, vp, vp, vp, u32, u32, f32, u32]),
    "sv_draft_tree": (C.c_int, [vp, vp, u32, vp, vp, vp, vp, vp, u32]),
    "sv_tap_rows": (C.c_int, [vp, vp, vp, u32, u32]),
    "sv_draft_kv": (C.c_int, [vp, P(Shape), vp, vp, vp, vp, vp, vp, vp, P(KvArgs), u32, u32]),
    "sv_draft_ctx": (C.c_int, [vp, vp, vp, vp, vp, vp, u32, u32, u32]),
    "sv_draft_embed": (C.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, u32, u32, u32]),
    "sv_draft_conv": (C.c_int, [vp, vp, vp, u32, vp, vp, vp, vp, u32, u32]),
    "sv_weights_open": (C.c_int, [C.c_char_p, P(vp)]),
    "sv_weights_count": (u32, [vp]),
    "sv_weights_info": (C.c_int, [vp, u32, P(TensorInfo)]),
    "sv_weights_find": (C.c_int, [vp, C.c_char_p, P(TensorInfo)]),
    "sv_weights_read": (C.c_int, [vp, C.c_char_p, vp, C.c_size_t]),
    "sv_weights_upload": (C.c_int, [vp, vp]),
    "sv_weights_device": (C.c_int, [vp, C.c_char_p, P(vp)]),
    "sv_weights_matrix": (C.c_int, [vp, C.c_char_p, u32, u32, P(Matrix)]),
    "sv_weights_close": (None, [vp]),
    "sv_replay_draft": (C.c_int, [vp, vp, u32, vp, vp, vp, vp, P(ReplayArgs), vp]),
    "sv_engine_create": (C.c_int, [P(EngineConfig), P(f32), P(vp)]),
    "sv_engine_destroy": (None, [vp]),
    "sv_engine_set_embed": (C.c_int, [vp, vp]),
    "sv_engine_set_layer": (C.c_int, [vp, u32, P(Layer)]),
    "sv_engine_set_extras": (C.c_int, [vp, P(ModelExtras)]),
    "sv_engine_set_head": (C.c_int, [vp, P(Matrix)]),
    "sv_engine_set_drafter": (C.c_int, [vp, P(Drafter)]),
    "sv_set_draft_rows": (C.c_int, [vp, u32, u32]),
    "sv_engine_draft_buffers": (C.c_int, [vp, P(DraftBuffers)]),
    "sv_engine_stream": (vp, [vp]),
    "sv_engine_get_buffers": (C.c_int, [vp, P(EngineBuffers)]),
    "sv_new_seq": (C.c_int, [vp, P(u32)]),
    "sv_free_seq": (C.c_int, [vp, u32]),
    "sv_seq_len": (C.c_int, [vp, u32, P(u32)]),
    "sv_seq_pages": (C.c_int, [vp, u32, P(u32), u32, P(u32)]),
    "sv_set_sampling": (C.c_int, [vp, u32, f32, f32, C.c_uint64]),
    "sv_set_gen": (C.c_int, [vp, u32, P(GenState)]),
    "sv_bench_fill": (C.c_int, [vp, u32, u32]),
    "sv_settle": (C.c_int, [vp, u32, u32]),
    "sv_set_feed": (C.c_int, [vp, u32, u32, u32]),
    "sv_plan": (C.c_int, [vp, P(Run), u32, u32, P(PlanInfo)]),
    "sv_encode": (C.c_int, [vp, u32]),
    "sv_graph_capture": (C.c_int, [vp, u32]),
    "sv_graph_replay": (C.c_int, [vp, u32]),
    "sv_sync": (C.c_int, [vp]),
    "sv_set_replay": (C.c_int, [vp, u32, f32]),
    "sv_step": (C.c_int, [vp, P(Run), u32, u32, P(u32), P(f32), P(u32), P(PlanInfo)]),
    "sv_step_capture": (C.c_int, [vp, P(Run), u32, u32, CAPTURE_FN, vp, P(u32), P(f32), P(u32), P(PlanInfo)]),
    "sv_profile_step": (C.c_int, [vp, u32, u32, P(f32), P(u32)]),
    "sv_sample_logits": (C.c_int, [vp, P(f32), u32, P(f32), P(f32), P(C.c_uint64), P(u32), P(u32)]),
}


class SvError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status


_lib = None


def lib() -> C.CDLL:
    """The loaded library; raises if it was not built (no fallback exists)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"{LIB_PATH} is not built: run `make -C {PKG_DIR}` or __graft_entry__.build()")
        L = C.CDLL(os.fspath(LIB_PATH))
        for name, (res, args) in PROTOS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != 0:
        raise SvError(status, lib().sv_last_error().decode())
