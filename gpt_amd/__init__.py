"""gpt_amd: MI355X (gfx950) causal self-attention backend for Filipeak/gpt.

The product is the C-ABI shared library ``gpt_amd/libgpt_hip_attn.so``
(entry points declared in ``include/gpt_hip_attn.h``). This package is the
Python host-side mirror of the reference's attention op pair
(``IGPTBackend::device_flash_attention_forward`` / ``..._backward``,
reference src/backend/backend_interface.h:161-184), calling that library
through ctypes with device pointers taken from torch tensors.
"""
from .attention import (  # noqa: F401
    HipAttentionError,
    attention_backward,
    attention_forward,
    device_flash_attention_backward,
    device_flash_attention_backward_noalloc,
    device_flash_attention_forward,
    device_ok,
    lib_path,
    load_library,
    release_workspaces,
    set_path,
    set_wait_limit,
    timing_enable,
    timing_read,
    wait_timeouts,
)
