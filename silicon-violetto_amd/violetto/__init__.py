"""violetto — Python binding of the MI355X verify path (libsv_verify.so, include/sv_verify.h).

Kernel-level calls live in `kernels`, the engine (the reference's Engine: sequences, the paged
KV cache, plan/encode/step, graph replay) in `engine`, synthetic benchmark models in `model`, the drafter's in `drafter`.
"""
from . import _lib
from ._lib import SvError, lib
from .engine import Engine
from .drafter import SyntheticDrafter
from .model import CONFIG_SHAPE, REFERENCE_SHAPE, LayerScalars, ModelShape, SyntheticModel, quantize_rows, rope_freq

__all__ = ["_lib", "SvError", "lib", "Engine", "CONFIG_SHAPE", "REFERENCE_SHAPE", "LayerScalars", "ModelShape",
           "SyntheticModel", "SyntheticDrafter", "quantize_rows", "rope_freq"]
