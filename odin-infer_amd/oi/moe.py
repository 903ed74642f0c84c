"""Routed-expert FFN on the device (oi_moe_ffn): router top-k and the chosen
experts' SwiGLU for one token."""
import ctypes

import numpy as np

from . import _native
from ._native import check


def moe_ffn(n_experts, top_k, dim, inter, norm_topk_prob, router_type, router_blocks, expert_type, gate_blocks,
            up_blocks, down_blocks, x):
    """Returns (y [dim], ids [top_k], weights [top_k])."""
    d = _native.MoeDims(n_experts, top_k, dim, inter, int(bool(norm_topk_prob)))
    b = lambda a: np.ascontiguousarray(a, np.uint8)
    rb, gb, ub, db = b(router_blocks), b(gate_blocks), b(up_blocks), b(down_blocks)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(dim, np.float32)
    ids = np.empty(top_k, np.int32)
    w = np.empty(top_k, np.float32)
    check(_native.hip().oi_moe_ffn(ctypes.byref(d), int(router_type), rb.ctypes.data, int(expert_type),
                                   gb.ctypes.data, ub.ctypes.data, db.ctypes.data, x.ctypes.data, y.ctypes.data,
                                   ids.ctypes.data, w.ctypes.data))
    return y, ids, w
