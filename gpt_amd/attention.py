"""Host-side mirror of the reference's attention operator interface.

Reference interface (src/backend/backend_interface.h:161-184):

    void device_flash_attention_forward(float *y, float *logsumexp,
        const float *qkv, int batch_size, int seq_len, int hidden_size,
        int num_heads);
    void device_flash_attention_backward(float *grad_x, float *D_cache,
        const float *logsumexp, const float *grad_y, const float *y,
        const float *qkv, int batch_size, int seq_len, int hidden_size,
        int num_heads);

The functions here take the same arguments in the same order. Tensors are
torch CUDA (HIP) tensors, fp32 and contiguous, or raw device addresses as
ints. Where the reference aborts on a device error
(src/backend/cuda/utils/cuda_utils.cuh:21-34), these raise
``HipAttentionError`` with the library's message. There is no CPU fallback:
if the HIP library is missing, loading it raises.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Union

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_NAME = "libgpt_hip_attn.so"

_lib = None


class HipAttentionError(RuntimeError):
    """Non-zero status from the gfx950 attention library."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


def lib_path() -> str:
    return os.path.join(_HERE, _LIB_NAME)


def load_library():
    """Load ``libgpt_hip_attn.so`` (built by ``make -C gpt_amd``)."""
    global _lib
    if _lib is None:
        path = lib_path()
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is missing: build it with __graft_entry__.build() or `make -C gpt_amd`")
        lib = ctypes.CDLL(path)
        i, p, vp = ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p
        lib.gpt_hip_attn_fwd_f32.argtypes = [p, p, p, i, i, i, i, vp]
        lib.gpt_hip_attn_fwd_f32.restype = i
        lib.gpt_hip_attn_bwd_f32.argtypes = [p, p, p, p, p, p, i, i, i, i, vp]
        lib.gpt_hip_attn_bwd_f32.restype = i
        lib.gpt_hip_attn_bwd_f32_noalloc.argtypes = [p, p, p, p, p, p, i, i, i, i, vp]
        lib.gpt_hip_attn_bwd_f32_noalloc.restype = i
        lib.gpt_hip_attn_last_error.argtypes = []
        lib.gpt_hip_attn_last_error.restype = ctypes.c_char_p
        lib.gpt_hip_attn_device_ok.argtypes = []
        lib.gpt_hip_attn_device_ok.restype = i
        lib.gpt_hip_attn_wait_timeouts.argtypes = []
        lib.gpt_hip_attn_wait_timeouts.restype = i
        lib.gpt_hip_attn_release_workspaces.argtypes = []
        lib.gpt_hip_attn_release_workspaces.restype = i
        lib.gpt_hip_attn_set_path.argtypes = [i]
        lib.gpt_hip_attn_set_path.restype = i
        lib.gpt_hip_attn_set_wait_limit.argtypes = [ctypes.c_longlong, i]
        lib.gpt_hip_attn_set_wait_limit.restype = i
        lib.gpt_hip_attn_timing_enable.argtypes = [i]
        lib.gpt_hip_attn_timing_enable.restype = i
        lib.gpt_hip_attn_timing_read.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int), i]
        lib.gpt_hip_attn_timing_read.restype = i
        _lib = lib
    return _lib


Ptr = Union[int, None, "torch.Tensor"]  # noqa: F821


def _addr(x: Ptr, name: str) -> Optional[int]:
    if x is None or isinstance(x, int):
        return x
    import torch

    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name}: expected a torch tensor or an int address, got {type(x)}")
    if x.dtype != torch.float32:
        raise TypeError(f"{name}: expected float32, got {x.dtype}")
    if not x.is_cuda:
        raise ValueError(f"{name}: expected a device (HIP) tensor")
    if not x.is_contiguous():
        raise ValueError(f"{name}: expected a contiguous tensor")
    return x.data_ptr()


def _stream(stream) -> Optional[int]:
    if stream is None or isinstance(stream, int):
        return stream
    return stream.cuda_stream  # torch.cuda.Stream


def _check(rc: int) -> None:
    if rc != 0:
        msg = load_library().gpt_hip_attn_last_error().decode(errors="replace")
        raise HipAttentionError(rc, msg)


def device_flash_attention_forward(y: Ptr, logsumexp: Ptr, qkv: Ptr, batch_size: int, seq_len: int,
                                   hidden_size: int, num_heads: int, stream=None) -> None:
    """y [B,T,C] and logsumexp [B,T,H] from qkv [B,T,3C] (causal, scale 1/sqrt(d))."""
    rc = load_library().gpt_hip_attn_fwd_f32(
        _addr(y, "y"), _addr(logsumexp, "logsumexp"), _addr(qkv, "qkv"),
        batch_size, seq_len, hidden_size, num_heads, _stream(stream))
    _check(rc)


def device_flash_attention_backward(grad_x: Ptr, D_cache: Ptr, logsumexp: Ptr, grad_y: Ptr, y: Ptr,
                                    qkv: Ptr, batch_size: int, seq_len: int, hidden_size: int,
                                    num_heads: int, stream=None) -> None:
    """Overwrites grad_x [B,T,3C] with dQ|dK|dV and writes D_cache [B,T,H]."""
    rc = load_library().gpt_hip_attn_bwd_f32(
        _addr(grad_x, "grad_x"), _addr(D_cache, "D_cache"), _addr(logsumexp, "logsumexp"),
        _addr(grad_y, "grad_y"), _addr(y, "y"), _addr(qkv, "qkv"),
        batch_size, seq_len, hidden_size, num_heads, _stream(stream))
    _check(rc)


def device_flash_attention_backward_noalloc(grad_x: Ptr, D_cache: Ptr, logsumexp: Ptr, grad_y: Ptr, y: Ptr,
                                            qkv: Ptr, batch_size: int, seq_len: int, hidden_size: int,
                                            num_heads: int, stream=None) -> None:
    """As device_flash_attention_backward, but the library allocates no device
    memory: its dS tiles live in a fixed per-device scratch array (head_dim 64
    up to T = 5760; longer rows raise). Calls overlapping on one device race."""
    rc = load_library().gpt_hip_attn_bwd_f32_noalloc(
        _addr(grad_x, "grad_x"), _addr(D_cache, "D_cache"), _addr(logsumexp, "logsumexp"),
        _addr(grad_y, "grad_y"), _addr(y, "y"), _addr(qkv, "qkv"),
        batch_size, seq_len, hidden_size, num_heads, _stream(stream))
    _check(rc)


def attention_forward(qkv, num_heads: int, stream=None):
    """Allocating convenience wrapper: returns (y, logsumexp) for qkv [B,T,3C]."""
    import torch

    B, T, W = qkv.shape
    C = W // 3
    y = torch.empty((B, T, C), dtype=torch.float32, device=qkv.device)
    lse = torch.empty((B, T, num_heads), dtype=torch.float32, device=qkv.device)
    device_flash_attention_forward(y, lse, qkv, B, T, C, num_heads, stream)
    return y, lse


def attention_backward(qkv, y, lse, grad_y, num_heads: int, stream=None):
    """Allocating convenience wrapper: returns (grad_x, D_cache)."""
    import torch

    B, T, W = qkv.shape
    C = W // 3
    grad_x = torch.empty((B, T, W), dtype=torch.float32, device=qkv.device)
    D = torch.empty((B, T, num_heads), dtype=torch.float32, device=qkv.device)
    device_flash_attention_backward(grad_x, D, lse, grad_y, y, qkv, B, T, C, num_heads, stream)
    return grad_x, D


def device_ok() -> bool:
    return bool(load_library().gpt_hip_attn_device_ok())


KERNEL_KINDS = ("fwd", "bwd_rowdot", "bwd_dkdv", "bwd_dq", "other", "bwd_fused")


def timing_enable(on: bool = True) -> None:
    """Start (or stop) recording a HIP event pair around every kernel launch."""
    _check(load_library().gpt_hip_attn_timing_enable(1 if on else 0))


def timing_read() -> dict:
    """Wait for the recorded launches; return {kind: (total_ms, launches)} and
    forget them. Kinds are KERNEL_KINDS."""
    n = len(KERNEL_KINDS)
    ms = (ctypes.c_double * n)()
    cnt = (ctypes.c_int * n)()
    rc = load_library().gpt_hip_attn_timing_read(ms, cnt, n)
    if rc < 0:
        _check(rc)
    return {k: (ms[i], cnt[i]) for i, k in enumerate(KERNEL_KINDS)}


def wait_timeouts() -> int:
    """Waits for the device, then returns (and clears) how many dQ waits of
    the one-launch backward reached their time limit since the last call (0
    in every correct run)."""
    rc = load_library().gpt_hip_attn_wait_timeouts()
    if rc < 0:
        _check(rc)
    return rc


def set_wait_limit(microseconds: int = -1, extra_need: int = 0) -> None:
    """Test hook for the one-launch backward's dQ waits: the owners' wait
    before they hand an item to the orphan runners (default 50 us) and the
    runners' safety limit for an item's counts (default one second), both set
    to `microseconds` (negative restores the defaults), and a count added to
    every awaited count (extra_need > 0 makes every owner hand its item over
    and every runner's wait expire). Process-wide; read at each launch."""
    _check(load_library().gpt_hip_attn_set_wait_limit(int(microseconds), int(extra_need)))


def release_workspaces() -> None:
    """Frees the backward's per-stream dS workspaces on the current device
    after waiting for its queued work; the next backward call allocates again."""
    _check(load_library().gpt_hip_attn_release_workspaces())


def set_path(path: int) -> int:
    """0 = automatic (MFMA kernels for head_dim 64, deterministic backward:
    one fused launch for T <= 256, dK/dV then dQ beyond), 1 = general-d
    kernels only, 2 = as 0 but with the fp32-atomic dQ backward, 3 = as 0 but
    the two-launch backward at every T.
    Returns the previous setting. Test and tuning hook; process-wide."""
    rc = load_library().gpt_hip_attn_set_path(path)
    if rc < 0:
        _check(rc)
    return rc
