"""ctypes bindings of the CPU oracle for the GPT-2 ops around attention (test
infrastructure only: tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg use it; the product package ``gpt_amd`` never does).

Two implementations of each op, same arguments as the IGPTBackend methods
(reference src/backend/backend_interface.h:26-237), numpy arrays in place of
device pointers:
  * ``impl="oracle"``: ``oracle/liboracle_ops.so``, our C restatement
    (oracle/ops_oracle.c);
  * ``impl="ref"``: the reference's own CPUBackend methods
    (src/backend/cpu/cpu_backend.cpp:65-287, 439-557) compiled from
    /root/reference into ``oracle/_ref/libref_cpu_attn.so`` with the same
    flags; ``impl="ref_fast"`` the same sources at -O3 (CPU baseline).
Every function works in place on the arrays it is given, as the reference
does on its buffers (accumulating outputs are added to; inputs such as the
LayerNorm x may be modified exactly where the reference modifies them).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from .pyoracle import LIBDIR, REF_FAST_SO, REF_SO, _load

OPS_SO = os.path.join(LIBDIR, "liboracle_ops.so")

_NAMES = {
    "embedding_forward": "embedding_forward",
    "unembedding_forward": "unembedding_forward",
    "embedding_backward": "embedding_backward",
    "unembedding_backward": "unembedding_backward",
    "layernorm_forward": "layernorm_forward",
    "layernorm_backward": "layernorm_backward",
    "linear_forward": "linear_forward",
    "linear_backward": "linear_backward",
    "activation_backward": "activation_backward",
    "softmax_forward": "softmax_forward",
    "ce_backward": "ce_backward",
    "ce_loss": "ce_loss",
    "adamw": "adamw",
    "scale_clip": "scale_clip",
}


def _fn(op: str, impl: str):
    if impl == "oracle":
        return getattr(_load(OPS_SO), "ops_oracle_" + _NAMES[op])
    if impl == "ref":
        return getattr(_load(REF_SO), "ref_op_" + _NAMES[op])
    if impl == "ref_fast":
        return getattr(_load(REF_FAST_SO), "ref_op_" + _NAMES[op])
    raise ValueError(impl)


def _f(a):
    if a is None:
        return ctypes.c_void_p(0)
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return ctypes.c_void_p(a.ctypes.data)


def _i(a):
    assert a.dtype == np.int32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return ctypes.c_void_p(a.ctypes.data)


_F = ctypes.c_float


def embedding_forward(y, wte, wpe, tok, B, T, C, impl="oracle"):
    _fn("embedding_forward", impl)(_f(y), _f(wte), _f(wpe), _i(tok), B, T, C)


def unembedding_forward(y, x, wte, B, T, C, Vp, impl="oracle"):
    _fn("unembedding_forward", impl)(_f(y), _f(x), _f(wte), B, T, C, Vp)


def embedding_backward(gwte, gwpe, gy, tok, B, T, C, impl="oracle"):
    _fn("embedding_backward", impl)(_f(gwte), _f(gwpe), _f(gy), _i(tok), B, T, C)


def unembedding_backward(gx, gwte, gy, x, wte, B, T, C, Vp, impl="oracle"):
    _fn("unembedding_backward", impl)(_f(gx), _f(gwte), _f(gy), _f(x), _f(wte), B, T, C, Vp)


def layernorm_forward(y, means, vars_, x, res, gamma, beta, B, T, C, impl="oracle"):
    _fn("layernorm_forward", impl)(_f(y), _f(means), _f(vars_), _f(x), _f(res), _f(gamma), _f(beta), B, T, C)


def layernorm_backward(gx, ggamma, gbeta, gy, gres, x, means, vars_, gamma, B, T, C, impl="oracle"):
    _fn("layernorm_backward", impl)(_f(gx), _f(ggamma), _f(gbeta), _f(gy), _f(gres), _f(x), _f(means), _f(vars_),
                                    _f(gamma), B, T, C)


def linear_forward(y, act, x, w, b, activation, B, T, n_in, n_out, impl="oracle"):
    _fn("linear_forward", impl)(_f(y), _f(act), _f(x), _f(w), _f(b), 1 if activation else 0, B, T, n_in, n_out)


def linear_backward(gx, gw, gb, gy, x, w, B, T, n_in, n_out, impl="oracle"):
    _fn("linear_backward", impl)(_f(gx), _f(gw), _f(gb), _f(gy), _f(x), _f(w), B, T, n_in, n_out)


def activation_backward(gx, gy, x, B, T, n, impl="oracle"):
    _fn("activation_backward", impl)(_f(gx), _f(gy), _f(x), B, T, n)


def softmax_forward(y, x, B, T, V, Vp, impl="oracle"):
    _fn("softmax_forward", impl)(_f(y), _f(x), B, T, V, Vp)


def ce_backward(gx, y, labels, B, T, V, Vp, impl="oracle"):
    _fn("ce_backward", impl)(_f(gx), _f(y), _i(labels), B, T, V, Vp)


def ce_loss(y, labels, B, T, Vp, impl="oracle") -> float:
    out = np.zeros(1, np.float32)
    _fn("ce_loss", impl)(_f(out), _f(y), _i(labels), B, T, Vp)
    return float(out[0])


def adamw(p, g, m, v, n, lr, beta1, beta2, eps, wd, step, impl="oracle"):
    _fn("adamw", impl)(_f(p), _f(g), _f(m), _f(v), n, _F(lr), _F(beta1), _F(beta2), _F(eps), _F(wd), step)


def scale_clip(g, n, max_norm, accum, impl="oracle"):
    _fn("scale_clip", impl)(_f(g), n, _F(max_norm), accum)
