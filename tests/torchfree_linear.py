"""The GPT-2 124M linear layers at the training step's 4096 rows through the
ops library in a process that never imports PyTorch, so that the library
binds ROCm's own hipBLASLt (the one the reference-side trainer and generator
load), not the copy PyTorch bundles: the tuning table's kernels for that
build are the ones exercised. Run by tests/test_ops_gpu.py in a subprocess;
device memory comes from the HIP runtime through ctypes. Checks y = x w + b
(and GELU), grad_x, grad_w accumulated onto a nonzero start and grad_b
against float64 numpy at 1e-5 norm-wise, and that the tuned kernels were
taken. Exit status 0 on success."""
import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from gpt_amd import ops  # noqa: E402  (imports no torch)

RTOL = 1e-5
hip = ctypes.CDLL("libamdhip64.so")
hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
hip.hipFree.argtypes = [ctypes.c_void_p]
H2D, D2H = 1, 2


def dev(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    p = ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(p), max(a.nbytes, 4)) == 0
    assert hip.hipMemcpy(p, a.ctypes.data, a.nbytes, H2D) == 0
    return p.value


def empty(n):
    p = ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(p), n * 4) == 0
    return p.value


def host(p, shape):
    out = np.empty(shape, np.float32)
    assert hip.hipDeviceSynchronize() == 0
    assert hip.hipMemcpy(out.ctypes.data, ctypes.c_void_p(p), out.nbytes, D2H) == 0
    return out


def rel(x, r):
    return float(np.abs(x.astype(np.float64) - r).max() / np.abs(r).max())


def main():
    assert "torch" not in sys.modules
    B, T = 16, 256
    worst = 0.0
    for n_in, n_out, act in ((768, 2304, False), (768, 768, False), (768, 3072, True), (3072, 768, False)):
        r = np.random.default_rng(7 + n_in + n_out)
        x = r.standard_normal((B, T, n_in)).astype(np.float32)
        w = (r.standard_normal((n_in, n_out)) / np.sqrt(n_in)).astype(np.float32)
        b = (0.1 * r.standard_normal(n_out)).astype(np.float32)
        gy = r.standard_normal((B, T, n_out)).astype(np.float32)
        gw0 = r.standard_normal((n_in, n_out)).astype(np.float32)
        gb0 = r.standard_normal(n_out).astype(np.float32)
        x64, w64, gy64 = (a.astype(np.float64).reshape(-1, a.shape[-1]) for a in (x, w, gy))
        dx, dw, db, dgy = dev(x), dev(w), dev(b), dev(gy)
        y, a = empty(B * T * n_out), empty(B * T * n_out)
        ops.device_linear_activation_fused_forward(y, a if act else None, dx, dw, db, act, B, T, n_in, n_out)
        yh = host(y, (B * T, n_out))
        errs = {"y": rel(yh, x64 @ w64 + b.astype(np.float64))}
        if act:
            ys = yh.astype(np.float64)
            errs["gelu"] = rel(host(a, (B * T, n_out)), 0.5 * ys * (1.0 + np.tanh(0.79788456 * (ys + 0.044715 * ys ** 3))))
        gx, dgw, dgb = empty(B * T * n_in), dev(gw0), dev(gb0)
        ops.device_linear_backward(gx, dgw, dgb, dgy, dx, dw, B, T, n_in, n_out)
        errs["grad_x"] = rel(host(gx, (B * T, n_in)), gy64 @ w64.T)
        errs["grad_w"] = rel(host(dgw, (n_in, n_out)), gw0.astype(np.float64) + x64.T @ gy64)
        errs["grad_b"] = rel(host(dgb, (n_out,)), gb0.astype(np.float64) + gy64.sum(0))
        print(f"linear {n_in}x{n_out}{' +GELU' if act else ''}: " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()),
              flush=True)
        worst = max(worst, max(errs.values()))
        for p in (dx, dw, db, dgy, y, a, gx, dgw, dgb):
            hip.hipFree(ctypes.c_void_p(p))
    info = ops.gemm_info()
    print("gemm plans:", info, "torch loaded:", "torch" in sys.modules, flush=True)
    assert "torch" not in sys.modules
    assert worst <= RTOL, worst
    assert info["tuned"] >= 1, info
    return 0


if __name__ == "__main__":
    sys.exit(main())
