"""Host-side mirror of the reference's other GPT-2 op methods.

Each function has the name, argument order and meaning of one virtual method
of the reference's op interface IGPTBackend (src/backend/backend_interface.h:
26-237), plus an optional stream, and calls the gfx950 library
``gpt_amd/libgpt_hip_ops.so`` (C ABI in include/gpt_hip_ops.h) through
ctypes. Tensors are torch device (HIP) tensors, contiguous, float32 (token
ids int32), or raw device addresses as ints. Where the reference aborts on a
device error (src/backend/cuda/utils/cuda_utils.cuh:21-34), these raise
``HipOpsError`` with the library's message. There is no CPU fallback: if the
library is missing, loading it raises.

Two entry points take one argument the reference's methods lack:
``device_embedding_forward`` / ``device_embedding_backward`` accept
``vocab_rows`` (rows of wte; token ids are checked against it on the device;
0 = unchecked, the reference's behaviour).
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

from .attention import Ptr, _stream

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_NAME = "libgpt_hip_ops.so"

_lib = None


class HipOpsError(RuntimeError):
    """Non-zero status from the gfx950 ops library."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


def lib_path() -> str:
    return os.path.join(_HERE, _LIB_NAME)


# name -> argument kinds: p pointer, i int, f float, z size_t, u unsigned long long, s stream
_SIGS = {
    "gpt_hip_embedding_forward_f32": "ppppiiiis",
    "gpt_hip_embedding_backward_f32": "ppppiiiis",
    "gpt_hip_unembedding_forward_f32": "pppiiiis",
    "gpt_hip_unembedding_backward_f32": "pppppiiiis",
    "gpt_hip_layernorm_residual_forward_f32": "pppppppiiis",
    "gpt_hip_layernorm_residual_backward_f32": "pppppppppiiis",
    "gpt_hip_linear_activation_forward_f32": "pppppiiiiis",
    "gpt_hip_linear_backward_f32": "ppppppiiiis",
    "gpt_hip_activation_backward_f32": "pppiiis",
    "gpt_hip_softmax_forward_f32": "ppiiiis",
    "gpt_hip_cross_entropy_softmax_backward_f32": "pppiiiis",
    "gpt_hip_cross_entropy_loss_f32": "pppiiis",
    "gpt_hip_adamw_step_f32": "ppppifffffis",
    "gpt_hip_scale_and_clip_grad_f32": "pifis",
    "gpt_hip_fill_normal_f32": "pffzus",
    "gpt_hip_fill_const_f32": "pfzs",
}
_CT = {"p": ctypes.c_void_p, "i": ctypes.c_int, "f": ctypes.c_float, "z": ctypes.c_size_t,
       "u": ctypes.c_ulonglong, "s": ctypes.c_void_p}


def load_library():
    """Load ``libgpt_hip_ops.so`` (built by ``make -C gpt_amd``)."""
    global _lib
    if _lib is None:
        path = lib_path()
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is missing: build it with __graft_entry__.build() or `make -C gpt_amd`")
        lib = ctypes.CDLL(path)
        for name, sig in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = [_CT[c] for c in sig]
            fn.restype = ctypes.c_int
        lib.gpt_hip_ops_last_error.argtypes = []
        lib.gpt_hip_ops_last_error.restype = ctypes.c_char_p
        lib.gpt_hip_ops_gemm_info.argtypes = [ctypes.POINTER(ctypes.c_int)] * 3
        lib.gpt_hip_ops_gemm_info.restype = ctypes.c_int
        _lib = lib
    return _lib


def _addr(x: Ptr, name: str, tokens: bool = False) -> Optional[int]:
    if x is None or isinstance(x, int):
        return x
    import torch

    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name}: expected a torch tensor or an int address, got {type(x)}")
    want = torch.int32 if tokens else torch.float32
    if x.dtype != want:
        raise TypeError(f"{name}: expected {want}, got {x.dtype}")
    if not x.is_cuda:
        raise ValueError(f"{name}: expected a device (HIP) tensor")
    if not x.is_contiguous():
        raise ValueError(f"{name}: expected a contiguous tensor")
    return x.data_ptr()


def _call(name: str, *args) -> None:
    rc = getattr(load_library(), name)(*args)
    if rc != 0:
        raise HipOpsError(rc, load_library().gpt_hip_ops_last_error().decode(errors="replace"))


def device_embedding_forward(y, wte, wpe, input_tokens, batch_size, seq_len, hidden_size, vocab_rows=0,
                             stream=None):
    _call("gpt_hip_embedding_forward_f32", _addr(y, "y"), _addr(wte, "wte"), _addr(wpe, "wpe"),
          _addr(input_tokens, "input_tokens", True), batch_size, seq_len, hidden_size, vocab_rows, _stream(stream))


def device_embedding_backward(grad_wte, grad_wpe, grad_y, input_tokens, batch_size, seq_len, hidden_size,
                              vocab_rows=0, stream=None):
    _call("gpt_hip_embedding_backward_f32", _addr(grad_wte, "grad_wte"), _addr(grad_wpe, "grad_wpe"),
          _addr(grad_y, "grad_y"), _addr(input_tokens, "input_tokens", True), batch_size, seq_len, hidden_size,
          vocab_rows, _stream(stream))


def device_unembedding_forward(y, x, wte, batch_size, seq_len, hidden_size, vocab_size_padded, stream=None):
    _call("gpt_hip_unembedding_forward_f32", _addr(y, "y"), _addr(x, "x"), _addr(wte, "wte"), batch_size,
          seq_len, hidden_size, vocab_size_padded, _stream(stream))


def device_unembedding_backward(grad_x, grad_wte, grad_y, x, wte, batch_size, seq_len, hidden_size,
                                vocab_size_padded, stream=None):
    _call("gpt_hip_unembedding_backward_f32", _addr(grad_x, "grad_x"), _addr(grad_wte, "grad_wte"),
          _addr(grad_y, "grad_y"), _addr(x, "x"), _addr(wte, "wte"), batch_size, seq_len, hidden_size,
          vocab_size_padded, _stream(stream))


def device_layernorm_residual_fused_forward(y, means, vars, x, residual, gamma, beta, batch_size, seq_len,
                                            hidden_size, stream=None):
    _call("gpt_hip_layernorm_residual_forward_f32", _addr(y, "y"), _addr(means, "means"), _addr(vars, "vars"),
          _addr(x, "x"), _addr(residual, "residual"), _addr(gamma, "gamma"), _addr(beta, "beta"), batch_size,
          seq_len, hidden_size, _stream(stream))


def device_layernorm_residual_fused_backward(grad_x, grad_gamma, grad_beta, grad_y, grad_residual, x, means, vars,
                                             gamma, batch_size, seq_len, hidden_size, stream=None):
    _call("gpt_hip_layernorm_residual_backward_f32", _addr(grad_x, "grad_x"), _addr(grad_gamma, "grad_gamma"),
          _addr(grad_beta, "grad_beta"), _addr(grad_y, "grad_y"), _addr(grad_residual, "grad_residual"),
          _addr(x, "x"), _addr(means, "means"), _addr(vars, "vars"), _addr(gamma, "gamma"), batch_size, seq_len,
          hidden_size, _stream(stream))


def device_linear_activation_fused_forward(y, act, x, w, b, activation, batch_size, seq_len, input_size,
                                           output_size, stream=None):
    _call("gpt_hip_linear_activation_forward_f32", _addr(y, "y"), _addr(act, "act"), _addr(x, "x"),
          _addr(w, "w"), _addr(b, "b"), 1 if activation else 0, batch_size, seq_len, input_size, output_size,
          _stream(stream))


def device_linear_backward(grad_x, grad_w, grad_b, grad_y, x, w, batch_size, seq_len, input_size, output_size,
                           stream=None):
    _call("gpt_hip_linear_backward_f32", _addr(grad_x, "grad_x"), _addr(grad_w, "grad_w"), _addr(grad_b, "grad_b"),
          _addr(grad_y, "grad_y"), _addr(x, "x"), _addr(w, "w"), batch_size, seq_len, input_size, output_size,
          _stream(stream))


def device_activation_backward(grad_x, grad_y, x, batch_size, seq_len, output_size, stream=None):
    _call("gpt_hip_activation_backward_f32", _addr(grad_x, "grad_x"), _addr(grad_y, "grad_y"), _addr(x, "x"),
          batch_size, seq_len, output_size, _stream(stream))


def device_softmax_forward(y, x, batch_size, seq_len, vocab_size, vocab_size_padded, stream=None):
    _call("gpt_hip_softmax_forward_f32", _addr(y, "y"), _addr(x, "x"), batch_size, seq_len, vocab_size,
          vocab_size_padded, _stream(stream))


def device_cross_entropy_softmax_fused_backward(grad_x, y_softmax, tokens_labels, batch_size, seq_len, vocab_size,
                                                vocab_size_padded, stream=None):
    _call("gpt_hip_cross_entropy_softmax_backward_f32", _addr(grad_x, "grad_x"), _addr(y_softmax, "y_softmax"),
          _addr(tokens_labels, "tokens_labels", True), batch_size, seq_len, vocab_size, vocab_size_padded,
          _stream(stream))


def device_cross_entropy_loss(loss, y_softmax, tokens_labels, batch_size, seq_len, vocab_size_padded,
                              stream=None):
    _call("gpt_hip_cross_entropy_loss_f32", _addr(loss, "loss"), _addr(y_softmax, "y_softmax"),
          _addr(tokens_labels, "tokens_labels", True), batch_size, seq_len, vocab_size_padded, _stream(stream))


def device_adamw_step(params, g, m, v, size, lr, beta1, beta2, eps, weight_decay, step, stream=None):
    _call("gpt_hip_adamw_step_f32", _addr(params, "params"), _addr(g, "g"), _addr(m, "m"), _addr(v, "v"), size,
          lr, beta1, beta2, eps, weight_decay, step, _stream(stream))


def device_scale_and_clip_grad(g, size, max_norm, accum_steps, stream=None):
    _call("gpt_hip_scale_and_clip_grad_f32", _addr(g, "g"), size, max_norm, accum_steps, _stream(stream))


def device_fill_normal(ptr, mean, stddev, size, seed=0, stream=None):
    _call("gpt_hip_fill_normal_f32", _addr(ptr, "ptr"), mean, stddev, size, seed, _stream(stream))


def device_fill_const(ptr, value, size, stream=None):
    _call("gpt_hip_fill_const_f32", _addr(ptr, "ptr"), value, size, _stream(stream))


def gemm_info() -> dict:
    """{"plans", "tuned", "blaslt_version"}: the hipBLASLt GEMM plans this
    process has made, how many of them run the tuning table's kernel for
    their shape, and the loaded hipBLASLt's version (0 before any plan)."""
    lib = load_library()
    vals = [ctypes.c_int(0) for _ in range(3)]
    rc = lib.gpt_hip_ops_gemm_info(*[ctypes.byref(v) for v in vals])
    if rc != 0:
        raise HipOpsError(rc, lib.gpt_hip_ops_last_error().decode(errors="replace"))
    return {"plans": vals[0].value, "tuned": vals[1].value, "blaslt_version": vals[2].value}
