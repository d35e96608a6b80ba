"""Pins the CPU oracle (oracle/attn_oracle.c) before it is trusted as the
checker of the HIP kernels. CPU only.

Each check is chosen so that a plausible mistake in the oracle fails it:
  * bit-exact agreement with the reference's own CPUBackend compiled from
    /root/reference (oracle/_ref; cpu_backend.cpp:289-437)
  * closed forms: T = 1 and identical keys (uniform causal weights)
  * invariants: shift of K, causality, sum_j dK_j = 0, sum_j dV_j = sum_i dO_i
  * an independent dense fp64 numpy restatement (masked softmax)
  * fp64 central finite differences of <O, dO> (catches sign, scale and
    transposition errors in the backward)
  * torch.nn.functional.scaled_dot_product_attention(is_causal=True) with
    autograd in fp64 (a library, not the reference)
"""
import numpy as np
import pytest

from gpt_amd import synth
from oracle import pyoracle
from tests import dense64

SHAPES = [
    # B, T, C, H
    (1, 1, 16, 2),
    (2, 5, 16, 2),     # d = 8
    (1, 64, 32, 4),    # the gpt_test shape (d = 8)
    (2, 37, 128, 2),   # d = 64, ragged T
    (1, 70, 192, 3),   # d = 64
    (1, 9, 60, 4),     # d = 15
]


def _inputs(B, T, C, H, seed=7):
    x = synth.qkv(B, T, C, seed)
    g = synth.grad_out(B, T, C, seed, std=1.0)
    return x, g


dense_forward64 = dense64.forward_np
dense_backward64 = dense64.backward_np


@pytest.mark.parametrize("B,T,C,H", [(1, 1, 64, 1), (2, 37, 128, 2), (1, 70, 192, 3), (3, 64, 32, 4)])
def test_dense64_torch_matches_numpy(B, T, C, H):
    """The torch float64 restatement the GPU tests run on the device (whole
    configurations) computes what the numpy one (pinned above and below)
    does, on the CPU, to float64 rounding; with a chunk smaller than B * H the
    (b, h) chunking is exercised too."""
    import torch

    x, g = _inputs(B, T, C, H, seed=19)
    yr, lr = dense_forward64(x, H)
    gr, Dr = dense_backward64(x, g, H)
    y, lse, gx, D = dense64.fwd_bwd_torch(torch.from_numpy(x), torch.from_numpy(g), H, chunk=max(1, B * H // 2))
    for a, r in ((y, yr), (lse, lr), (gx, gr), (D, Dr)):
        a = a.numpy()
        assert a.shape == r.shape
        assert np.abs(a - r).max() <= 1e-12 * max(1.0, np.abs(r).max())


@pytest.mark.parametrize("B,T,C,H", SHAPES)
def test_oracle_bitexact_vs_reference_cpu_backend(B, T, C, H):
    if not pyoracle.ref_available():
        pytest.skip("oracle/_ref not built (needs /root/reference at build time)")
    x, g = _inputs(B, T, C, H)
    y0, l0 = pyoracle.forward(x, H, "oracle")
    y1, l1 = pyoracle.forward(x, H, "ref")
    assert np.array_equal(y0, y1) and np.array_equal(l0, l1)
    gx0, D0 = pyoracle.backward(x, y0, l0, g, H, "oracle")
    gx1, D1 = pyoracle.backward(x, y1, l1, g, H, "ref")
    assert np.array_equal(gx0, gx1) and np.array_equal(D0, D1)


@pytest.mark.parametrize("B,T,C,H", SHAPES)
def test_oracle_matches_dense_fp64(B, T, C, H):
    x, g = _inputs(B, T, C, H)
    y, lse = pyoracle.forward(x, H, "oracle64")
    yr, lr = dense_forward64(x, H)
    np.testing.assert_allclose(y, yr, rtol=0, atol=1e-12 * max(1.0, np.abs(yr).max()))
    np.testing.assert_allclose(lse, lr, rtol=0, atol=1e-12 * max(1.0, np.abs(lr).max()))
    gx, D = pyoracle.backward(x, y, lse, g, H, "oracle64")
    gr, Dr = dense_backward64(x, g, H)
    np.testing.assert_allclose(gx, gr, rtol=0, atol=1e-11 * max(1.0, np.abs(gr).max()))
    np.testing.assert_allclose(D, Dr, rtol=0, atol=1e-11 * max(1.0, np.abs(Dr).max()))
    # fp32 oracle stays within fp32 rounding of the fp64 answer
    y32, l32 = pyoracle.forward(x, H, "oracle")
    assert np.abs(y32 - yr).max() <= 1e-5 * np.abs(yr).max()
    assert np.abs(l32 - lr).max() <= 1e-5 * np.abs(lr).max()


def test_oracle_T1_closed_form():
    B, T, C, H = 3, 1, 128, 2
    d = C // H
    x, g = _inputs(B, T, C, H)
    y, lse = pyoracle.forward(x, H, "oracle")
    # one visible key: O = V_0 and LSE = q.k / sqrt(d)
    assert np.array_equal(y, x[:, :, 2 * C:])
    q = x[:, :, :C].reshape(B, H, d).astype(np.float64)
    k = x[:, :, C:2 * C].reshape(B, H, d).astype(np.float64)
    np.testing.assert_allclose(lse.reshape(B, H), (q * k).sum(-1) / np.sqrt(d), rtol=1e-6, atol=1e-6)
    gx, D = pyoracle.backward(x, y, lse, g, H, "oracle")
    # p == 1 exactly, dP == D exactly: dQ = dK = 0, dV = dO
    assert np.all(gx[:, :, :2 * C] == 0)
    assert np.array_equal(gx[:, :, 2 * C:], g)


def test_oracle_identical_keys_prefix_mean():
    B, T, C, H = 1, 40, 128, 2
    d = C // H
    x, _ = _inputs(B, T, C, H)
    x[:, :, C:2 * C] = x[:, :1, C:2 * C]  # every key equals key 0
    y, lse = pyoracle.forward(x, H, "oracle64")
    v = x[0, :, 2 * C:].astype(np.float64)
    prefix_mean = np.cumsum(v, axis=0) / np.arange(1, T + 1)[:, None]
    np.testing.assert_allclose(y[0], prefix_mean, rtol=0, atol=1e-12)
    q = x[0, :, :C].reshape(T, H, d).astype(np.float64)
    k0 = x[0, 0, C:2 * C].reshape(H, d).astype(np.float64)
    c = (q * k0).sum(-1) / np.sqrt(d)
    np.testing.assert_allclose(lse[0], c + np.log(np.arange(1, T + 1))[:, None], rtol=0, atol=1e-12)


def test_oracle_shift_invariance_and_causality():
    B, T, C, H = 2, 33, 128, 2
    d = C // H
    x, _ = _inputs(B, T, C, H)
    y, lse = pyoracle.forward(x, H, "oracle64")
    u = synth.normal(99, (C,)).astype(np.float64)
    xs = x.astype(np.float64).copy()
    xs[:, :, C:2 * C] += u
    ys, lses = pyoracle.forward(xs, H, "oracle64")
    np.testing.assert_allclose(ys, y, rtol=0, atol=1e-12)
    qu = (x[:, :, :C].astype(np.float64).reshape(B, T, H, d) * u.reshape(H, d)).sum(-1) / np.sqrt(d)
    np.testing.assert_allclose(lses, lse + qu, rtol=0, atol=1e-11)
    # perturbing keys/values after position i leaves rows <= i bit-identical
    i = 17
    y32, l32 = pyoracle.forward(x, H, "oracle")
    xp = x.copy()
    xp[:, i + 1:, C:] += 1.0
    yp, lp = pyoracle.forward(xp, H, "oracle")
    assert np.array_equal(yp[:, :i + 1], y32[:, :i + 1]) and np.array_equal(lp[:, :i + 1], l32[:, :i + 1])
    assert not np.array_equal(yp[:, i + 1:], y32[:, i + 1:])


def test_oracle_backward_invariants():
    B, T, C, H = 2, 29, 128, 2
    d = C // H
    x, g = _inputs(B, T, C, H)
    y, lse = pyoracle.forward(x, H, "oracle64")
    gx, _ = pyoracle.backward(x, y, lse, g, H, "oracle64")
    dk = gx[:, :, C:2 * C].reshape(B, T, H, d)
    dv = gx[:, :, 2 * C:].reshape(B, T, H, d)
    # rows of dS sum to zero, so sum_j dK_j = 0; rows of P sum to one, so
    # sum_j dV_j = sum_i dO_i
    assert np.abs(dk.sum(1)).max() <= 1e-12 * np.abs(dk).max() * T
    np.testing.assert_allclose(dv.sum(1), g.astype(np.float64).reshape(B, T, H, d).sum(1), rtol=0, atol=1e-12)


def test_oracle_backward_finite_differences():
    B, T, C, H = 1, 6, 16, 2
    x, g = _inputs(B, T, C, H, seed=3)
    x = x.astype(np.float64)
    g = g.astype(np.float64)
    y, lse = pyoracle.forward(x, H, "oracle64")
    gx, _ = pyoracle.backward(x, y, lse, g, H, "oracle64")
    eps = 1e-6
    fd = np.zeros_like(x)
    flat = x.reshape(-1)
    for idx in range(flat.size):
        xp = flat.copy()
        xp[idx] += eps
        xm = flat.copy()
        xm[idx] -= eps
        fp = (pyoracle.forward(xp.reshape(x.shape), H, "oracle64")[0] * g).sum()
        fm = (pyoracle.forward(xm.reshape(x.shape), H, "oracle64")[0] * g).sum()
        fd.reshape(-1)[idx] = (fp - fm) / (2 * eps)
    np.testing.assert_allclose(gx, fd, rtol=0, atol=1e-7 * np.abs(fd).max())


def test_oracle_matches_torch_sdpa_fp64():
    torch = pytest.importorskip("torch")
    F = torch.nn.functional
    B, T, C, H = 2, 23, 128, 2
    d = C // H
    x, g = _inputs(B, T, C, H)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    q, k, v = xt.view(B, T, 3, H, d).permute(2, 0, 3, 1, 4)
    o = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    o = o.transpose(1, 2).reshape(B, T, C)
    o.backward(torch.tensor(g, dtype=torch.float64))
    y, lse = pyoracle.forward(x, H, "oracle64")
    gx, _ = pyoracle.backward(x, y, lse, g, H, "oracle64")
    np.testing.assert_allclose(y, o.detach().numpy(), rtol=0, atol=1e-12)
    np.testing.assert_allclose(gx, xt.grad.numpy(), rtol=0, atol=1e-11)
