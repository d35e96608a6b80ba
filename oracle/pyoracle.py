"""ctypes bindings for the CPU oracle (test infrastructure only).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
import this module. The product path (package ``gpt_amd``) never does.

Three libraries:
  * ``oracle/liboracle_attn.so``            our C restatement of the reference
    CPU backend's attention (src/backend/cpu/cpu_backend.cpp:289-437), in fp32
    and fp64;
  * ``oracle/_ref/libref_cpu_attn.so``      the reference's own CPUBackend
    compiled from /root/reference with the same flags (built in the dev
    container only; travels with the tree);
  * ``oracle/_ref/libref_cpu_attn_fast.so`` the same sources at -O3, timed as
    the CPU baseline.
All arrays are C-contiguous numpy arrays in the reference layouts:
qkv [B,T,3C], y [B,T,C], lse / D [B,T,H], grad_x [B,T,3C].
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# GPT_ORACLE_LIBDIR selects another build of the same libraries, e.g.
# oracle/_san (make -C oracle sanitize: AddressSanitizer + UBSan)
LIBDIR = os.environ.get("GPT_ORACLE_LIBDIR", _HERE)
ORACLE_SO = os.path.join(LIBDIR, "liboracle_attn.so")
REF_SO = os.path.join(LIBDIR, "_ref", "libref_cpu_attn.so")
REF_FAST_SO = os.path.join(LIBDIR, "_ref", "libref_cpu_attn_fast.so")

_libs: dict = {}


def _load(path: str):
    if path not in _libs:
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is not built; run __graft_entry__.build() (make -C oracle)")
        _libs[path] = ctypes.CDLL(path)
    return _libs[path]


def ref_available(fast: bool = False) -> bool:
    return os.path.exists(REF_FAST_SO if fast else REF_SO)


def _p(a: np.ndarray, dtype) -> ctypes.c_void_p:
    assert a.dtype == dtype and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return ctypes.c_void_p(a.ctypes.data)


def _shape(qkv: np.ndarray, H: int):
    B, T, W = qkv.shape
    assert W % 3 == 0
    C = W // 3
    assert C % H == 0
    return B, T, C


def forward(qkv: np.ndarray, H: int, impl: str = "oracle"):
    """Causal attention forward. ``impl`` is "oracle" (fp32 restatement),
    "oracle64" (fp64 restatement; qkv cast to fp64), "ref" (reference
    CPUBackend, exact flags) or "ref_fast" (reference CPUBackend, -O3).
    Returns (y [B,T,C], lse [B,T,H])."""
    B, T, C = _shape(qkv, H)
    if impl == "oracle64":
        x = np.ascontiguousarray(qkv, dtype=np.float64)
        y = np.empty((B, T, C), np.float64)
        lse = np.empty((B, T, H), np.float64)
        _load(ORACLE_SO).oracle_attn_forward_f64(_p(y, np.float64), _p(lse, np.float64),
                                                 _p(x, np.float64), B, T, C, H)
        return y, lse
    x = np.ascontiguousarray(qkv, dtype=np.float32)
    y = np.empty((B, T, C), np.float32)
    lse = np.empty((B, T, H), np.float32)
    if impl == "oracle":
        fn = _load(ORACLE_SO).oracle_attn_forward_f32
    elif impl == "ref":
        fn = _load(REF_SO).ref_attn_forward_f32
    elif impl == "ref_fast":
        fn = _load(REF_FAST_SO).ref_attn_forward_f32
    else:
        raise ValueError(impl)
    fn(_p(y, np.float32), _p(lse, np.float32), _p(x, np.float32), B, T, C, H)
    return y, lse


def backward(qkv: np.ndarray, y: np.ndarray, lse: np.ndarray, dy: np.ndarray, H: int,
             impl: str = "oracle"):
    """Causal attention backward. Returns (grad_x [B,T,3C], D [B,T,H])."""
    B, T, C = _shape(qkv, H)
    if impl == "oracle64":
        f = np.float64
        x, yy, ll, gg = (np.ascontiguousarray(a, dtype=f) for a in (qkv, y, lse, dy))
        gx = np.empty((B, T, 3 * C), f)
        D = np.empty((B, T, H), f)
        _load(ORACLE_SO).oracle_attn_backward_f64(_p(gx, f), _p(D, f), _p(ll, f), _p(gg, f),
                                                  _p(yy, f), _p(x, f), B, T, C, H)
        return gx, D
    f = np.float32
    x, yy, ll, gg = (np.ascontiguousarray(a, dtype=f) for a in (qkv, y, lse, dy))
    gx = np.empty((B, T, 3 * C), f)
    D = np.empty((B, T, H), f)
    if impl == "oracle":
        fn = _load(ORACLE_SO).oracle_attn_backward_f32
    elif impl == "ref":
        fn = _load(REF_SO).ref_attn_backward_f32
    elif impl == "ref_fast":
        fn = _load(REF_FAST_SO).ref_attn_backward_f32
    else:
        raise ValueError(impl)
    fn(_p(gx, f), _p(D, f), _p(ll, f), _p(gg, f), _p(yy, f), _p(x, f), B, T, C, H)
    return gx, D
