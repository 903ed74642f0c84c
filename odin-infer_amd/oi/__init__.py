"""Python mirror of the odin-infer Engine API over the gfx950 HIP library.

The reference's host API is Odin (infer/engine.odin:7-60, ggml/quant.odin);
this package exposes the same procedures (engine_load, engine_forward,
engine_destroy, engine_config; dequant_row, row_byte_size) through ctypes on
the C ABI of include/oi.h.  Nothing here computes: every call goes to
liboi_hip.so, and importing a compute entry point without that library raises.
"""
from . import ggml, infer, synth  # noqa: F401
