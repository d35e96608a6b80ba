"""Parity of the gfx950 attention kernels against the CPU oracle.

Every call goes through the C ABI (gpt_amd -> libgpt_hip_attn.so). The oracle
(oracle/attn_oracle.c, bit-exact with the reference CPU backend,
src/backend/cpu/cpu_backend.cpp:289-437) is run on the same seeded inputs.
Tolerances (tests/tolerances.py): norm-wise relative error <= 1e-5 for O and
LSE, <= 1e-4 for dQ, dK, dV and D, and the elementwise gate
|x - r| <= rtol |r| + 0.1 rtol max|r|; every comparison prints both numbers.

Large configurations (C3's 12 layers, C4, C5a) are checked against the oracle
on whole (b, h) slices (attention is independent per (b, h)), on every slice
through size-independent invariants (sum_j dK_j = 0 and sum_j dV_j = sum_i
dO_i per (b, h), finiteness), and in full, every (b, h), against the dense
float64 restatement of tests/dense64.py (pinned to the oracle by
tests/test_oracle.py), run with torch in float64 on the device.
"""
import numpy as np
import pytest

import gpt_amd
from gpt_amd import synth
from oracle import pyoracle
from tests.tolerances import BWD_RTOL, ELEM_ATOL_FRAC, FWD_RTOL, assert_close, rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def no_wait_timeouts(dev):
    """After every test: no dQ wait of the one-launch backward gave up at its
    spin limit (each would have read incomplete dS tiles)."""
    gpt_amd.wait_timeouts()
    yield
    assert gpt_amd.wait_timeouts() == 0


def _to(dev, a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def gpu_fwd(dev, x, H):
    import torch

    y, lse = gpt_amd.attention_forward(_to(dev, x), H)
    torch.cuda.synchronize()
    return y.cpu().numpy(), lse.cpu().numpy()


def gpu_bwd(dev, x, y, lse, g, H):
    import torch

    gx, D = gpt_amd.attention_backward(_to(dev, x), _to(dev, y), _to(dev, lse), _to(dev, g), H)
    torch.cuda.synchronize()
    return gx.cpu().numpy(), D.cpu().numpy()


def qkv_slice(x, b, h, H):
    C = x.shape[-1] // 3
    d = C // H
    cols = np.r_[h * d:(h + 1) * d, C + h * d:C + (h + 1) * d, 2 * C + h * d:2 * C + (h + 1) * d]
    return np.ascontiguousarray(x[b:b + 1, :, cols])


def row_slice(a, b, h, H):
    d = a.shape[-1] // H
    return np.ascontiguousarray(a[b:b + 1, :, h * d:(h + 1) * d])


def check_fwd_bwd(dev, x, g, H, check_bwd=True, tag="", elem_frac=ELEM_ATOL_FRAC):
    y, lse = gpu_fwd(dev, x, H)
    yr, lr = pyoracle.forward(x, H)
    e_y = assert_close(f"{tag} O", y, yr, FWD_RTOL, elem_frac=elem_frac)
    e_l = assert_close(f"{tag} LSE", lse, lr, FWD_RTOL, elem_frac=elem_frac)
    errs = {"O": e_y, "LSE": e_l}
    if check_bwd:
        # backward from the oracle's forward outputs, as the reference test does
        gx, D = gpu_bwd(dev, x, yr, lr, g, H)
        gr, Dr = pyoracle.backward(x, yr, lr, g, H)
        C = x.shape[-1] // 3
        for name, sl in (("dQ", slice(0, C)), ("dK", slice(C, 2 * C)), ("dV", slice(2 * C, 3 * C))):
            errs[name] = assert_close(f"{tag} {name}", gx[..., sl], gr[..., sl], BWD_RTOL, elem_frac=elem_frac)
        errs["D"] = assert_close(f"{tag} D", D, Dr, BWD_RTOL, elem_frac=elem_frac)
    return errs


def test_config1_forward_B1_T256(dev):
    x = synth.qkv(1, 256, 768, seed=1235)
    check_fwd_bwd(dev, x, None, 12, check_bwd=False, tag="C1")


def test_config2_fwd_bwd_B8_T256(dev):
    x = synth.qkv(8, 256, 768, seed=1236)
    g = synth.grad_out(8, 256, 768, seed=1236)
    errs = check_fwd_bwd(dev, x, g, 12, tag="C2")
    print("C2 errors", errs)


@pytest.mark.parametrize("B,T,C,H", [(6, 256, 768, 12), (10, 256, 768, 12), (16, 200, 512, 8), (24, 128, 512, 8),
                                     (16, 160, 512, 8)])
def test_paired_grids_fwd_bwd(dev, B, T, C, H):
    """Grids of 1 to 2 workgroups per CU (on 256 CUs: 288, 480, 512 and 384
    workgroups of 4, 4, 4, 2 and 3 item classes) take the paired layout
    (paired_item: the heaviest items alone on their CUs, the others paired
    heavy with light), in the forward and in the one-launch backward: every
    output against the oracle, which fails if an item were lost or run
    twice."""
    x = synth.qkv(B, T, C, seed=700 + B + T)
    g = synth.grad_out(B, T, C, seed=700 + B + T)
    check_fwd_bwd(dev, x, g, H, tag=f"paired B={B} T={T} H={H}")


@pytest.mark.parametrize("T", [1, 2, 3, 31, 32, 33, 63, 64, 65, 95, 127, 128, 129, 191, 255, 257, 300])
def test_ragged_T_fwd_bwd(dev, T):
    B, C, H = 2, 192, 3
    x = synth.qkv(B, T, C, seed=100 + T)
    g = synth.grad_out(B, T, C, seed=100 + T, std=1.0)
    check_fwd_bwd(dev, x, g, H, tag=f"T={T}")


@pytest.mark.parametrize("T", [256, 300])
def test_growing_scores_fwd_bwd(dev, T):
    """Scores that step up by 50 (about 9 in log2 units, past the forward's
    lazy-rescale margin of 8) at several keys, block-aligned in head 0 and
    not in head 1, so the running max rises after the first key block and
    the kernels must rescale O mid-row; head 2 keeps random scores."""
    B, C, H, d = 2, 192, 3, 64
    x = synth.qkv(B, T, C, seed=4242 + T)
    g = synth.grad_out(B, T, C, seed=4242 + T, std=1.0)
    rng = np.random.default_rng(17)
    for h, steps in ((0, (64, 128, 192, 256)), (1, (40, 100, 170, 230, 290))):
        u = rng.standard_normal(d).astype(np.float32)
        u /= np.linalg.norm(u)
        level = np.zeros(T, np.float32)
        for s in steps:
            level[s:] += 6.25  # q . k steps by 8 * 6.25 = 50
        for b in range(B):
            x[b, :, h * d:(h + 1) * d] = 8.0 * u
            x[b, :, C + h * d:C + (h + 1) * d] = (level[:, None] * u[None, :]
                                                  + 0.1 * rng.standard_normal((T, d)).astype(np.float32))
    # score jumps of 50 give P a dynamic range of e^50 within a row: near-zero
    # dQ entries carry up to 2.6e-5 max|r| of difference between the two fp32
    # summation orders (measured), so the elementwise term is 0.5 rtol here
    check_fwd_bwd(dev, x, g, H, tag=f"growing T={T}", elem_frac=0.5)


@pytest.mark.parametrize("B,T", [(1, 256), (2, 512), (8, 256), (1, 512), (2, 1024), (1, 2048)])
def test_forward_kernel_choice(dev, B, T):
    """One shape per head_dim-64 forward kernel the launcher picks by size:
    split-key (B=1 T=256, B=1 T=512: at most 512 16-query groups; B=2
    T=1024, B=1 T=2048: long rows, 256..511 64-query groups), heavy/light pair
    (B=2 T=512), Q-stationary (B=8 T=256: at least 256 64-query groups); O and
    LSE against the oracle, the backward at the same shapes too (its D rows
    inside the dK/dV kernel up to T = 256, from the separate D-row kernel
    beyond)."""
    C, H = 768, 12
    x = synth.qkv(B, T, C, seed=5000 + B * T)
    g = synth.grad_out(B, T, C, seed=5000 + B * T)
    check_fwd_bwd(dev, x, g, H, tag=f"B={B} T={T}")


@pytest.mark.parametrize("B,T,H", [(2, 96, 1), (2, 70, 20), (1, 64, 33), (4, 256, 20), (2, 256, 33)])
def test_head_counts_d64(dev, B, T, H):
    """head_dim 64 with 1, 20 and 33 heads (C = 64, 1280, 2112): the
    per-(b, h) index math of every kernel away from H = 12 (the last two
    shapes take the Q-stationary forward, B*H = 66 not a multiple of 8), and
    the D-row kernel's rows of more than 256 float4s (it takes a row in
    chunks of 4 x 64 float4s)."""
    C = 64 * H
    x = synth.qkv(B, T, C, seed=7000 + H)
    g = synth.grad_out(B, T, C, seed=7000 + H, std=1.0)
    check_fwd_bwd(dev, x, g, H, tag=f"H={H}")


def test_config5b_prefix_sweep_T1_to_256(dev):
    """Forward at B=1 for every prefix length 1..256, as autoregressive
    generation without a KV cache does."""
    C, H = 768, 12
    x = synth.qkv(1, 256, C, seed=1239)
    worst = (0.0, 0.0)
    for T in range(1, 257):
        xt = np.ascontiguousarray(x[:, :T])
        y, lse = gpu_fwd(dev, xt, H)
        yr, lr = pyoracle.forward(xt, H)
        e = (rel_err(y, yr), rel_err(lse, lr))
        assert e[0] <= FWD_RTOL and e[1] <= FWD_RTOL, (T, e)
        worst = (max(worst[0], e[0]), max(worst[1], e[1]))
    print("C5b worst O/LSE rel err", worst)


def test_backward_sweep_T1_to_256(dev):
    """Backward at B=1 (12 heads) for every T = 1..256 against the oracle: every
    query-block count and ragged tail of the one-launch backward (1 to 4 key
    groups, odd and even block counts, rows past T in the last block), with
    one workspace growing call by call; the two-launch form (path 3) on every
    fifth T. Inputs are the prefixes of one B=1, T=256 draw, as generation
    would see them; dO is drawn at unit scale so that every row matters."""
    C, H = 768, 12
    x = synth.qkv(1, 256, C, seed=1240)
    g = synth.grad_out(1, 256, C, seed=1240, std=1.0)
    worst = {}
    for T in range(1, 257):
        xt, gt = np.ascontiguousarray(x[:, :T]), np.ascontiguousarray(g[:, :T])
        yr, lr = pyoracle.forward(xt, H)
        gr, Dr = pyoracle.backward(xt, yr, lr, gt, H)
        paths = (0, 3) if T % 5 == 0 else (0,)
        for path in paths:
            prev = gpt_amd.set_path(path)
            try:
                gx, D = gpu_bwd(dev, xt, yr, lr, gt, H)
            finally:
                gpt_amd.set_path(prev)
            for name, a, r in (("dQ", gx[..., :C], gr[..., :C]), ("dK", gx[..., C:2 * C], gr[..., C:2 * C]),
                               ("dV", gx[..., 2 * C:], gr[..., 2 * C:]), ("D", D, Dr)):
                e = rel_err(a, r)
                assert e <= BWD_RTOL, (T, path, name, e)
                worst[name] = max(worst.get(name, 0.0), e)
    print("backward sweep T=1..256 worst rel err", worst)


@pytest.mark.parametrize("B,T,C,H", [(1, 64, 32, 4), (2, 50, 64, 4), (1, 40, 60, 4), (1, 33, 96, 3),
                                     (1, 70, 256, 2), (2, 17, 24, 3)])
def test_general_head_dim(dev, B, T, C, H):
    """head_dim != 64 runs the general-d kernels (d = 8 is the gpt_test model)."""
    x = synth.qkv(B, T, C, seed=5)
    g = synth.grad_out(B, T, C, seed=5, std=1.0)
    check_fwd_bwd(dev, x, g, H, tag=f"d={C // H}")


@pytest.mark.parametrize("B,T", [(8, 256), (2, 97), (1, 33)])
def test_atomic_dq_path_parity(dev, B, T):
    """The fp32-atomic dQ backward (path 2) against the oracle."""
    C, H = 768, 12
    x = synth.qkv(B, T, C, seed=77 + T)
    g = synth.grad_out(B, T, C, seed=77 + T)
    prev = gpt_amd.set_path(2)
    try:
        check_fwd_bwd(dev, x, g, H, tag=f"atomic T={T}")
    finally:
        gpt_amd.set_path(prev)


@pytest.mark.parametrize("B,T,C,H", [(16, 256, 768, 12), (3, 255, 768, 12), (5, 257, 768, 12), (1, 1, 64, 1),
                                     (2, 64, 128, 2), (7, 129, 192, 3), (1, 33, 768, 12)])
def test_fused_backward_matches_two_launch_backward(dev, B, T, C, H):
    """The default backward takes one fused launch for T <= 256 (dK/dV work
    items store the dS tiles, dQ items start on a query block once its
    completion counter is full) and the two-launch form beyond; path 3 forces
    the two-launch form. Both against the oracle on (b, h) slices, and against
    each other on the whole tensor (other summation orders of dK and dV:
    fp32 rounding only). T = 257 is past the fused kernel's limit (both paths
    then run the same kernels, bit for bit)."""
    x = synth.qkv(B, T, C, seed=300 + T)
    g = synth.grad_out(B, T, C, seed=300 + T)
    y, lse = gpu_fwd(dev, x, H)
    gx, D = gpu_bwd(dev, x, y, lse, g, H)
    prev = gpt_amd.set_path(3)
    try:
        gx3, D3 = gpu_bwd(dev, x, y, lse, g, H)
    finally:
        gpt_amd.set_path(prev)
    assert np.isfinite(gx).all() and np.isfinite(D).all()
    for name, sl in (("dQ", slice(0, C)), ("dK", slice(C, 2 * C)), ("dV", slice(2 * C, 3 * C))):
        assert_close(f"fused vs two-launch {name} T={T}", gx[..., sl], gx3[..., sl], BWD_RTOL)
    assert np.array_equal(D, D3)
    if T > 256:
        assert np.array_equal(gx.view(np.uint32), gx3.view(np.uint32))
    for (b, h) in {(0, 0), (B - 1, H - 1)}:
        xs = qkv_slice(x, b, h, H)
        gr, _ = pyoracle.backward(xs, row_slice(y, b, h, H), np.ascontiguousarray(lse[b:b + 1, :, h:h + 1]),
                                  row_slice(g, b, h, H), 1)
        d = C // H
        cols = np.r_[h * d:(h + 1) * d, C + h * d:C + (h + 1) * d, 2 * C + h * d:2 * C + (h + 1) * d]
        assert_close(f"fused T={T} (b,h)=({b},{h})", gx[b:b + 1, :, cols], gr, BWD_RTOL)


def test_fused_backward_repeatable_across_shapes(dev):
    """The fused backward's control block is all zeros between launches (every
    completion counter is reset by the dQ item that used it): interleaving
    shapes that lay out their counters differently changes nothing, bit for
    bit, and a dQ item never reads a tile before it is complete."""
    import torch

    shapes = [(16, 256, 768, 12), (3, 100, 768, 12), (1, 200, 64, 1), (8, 256, 768, 12)]
    data = {}
    for (B, T, C, H) in shapes:
        x = _to(dev, synth.qkv(B, T, C, seed=400 + B))
        g = _to(dev, synth.grad_out(B, T, C, seed=400 + B))
        y, lse = gpt_amd.attention_forward(x, H)
        data[(B, T, C, H)] = (x, g, y, lse)
    first = {}
    for rnd in range(4):
        for key in (shapes if rnd % 2 == 0 else shapes[::-1]):
            B, T, C, H = key
            x, g, y, lse = data[key]
            gx = torch.full((B, T, 3 * C), float("nan"), device=dev)
            D = torch.full((B, T, H), float("nan"), device=dev)
            gpt_amd.device_flash_attention_backward(gx, D, lse, g, y, x, B, T, C, H)
            torch.cuda.synchronize()
            if key not in first:
                assert torch.isfinite(gx).all()
                first[key] = gx.clone()
            else:
                assert torch.equal(first[key], gx), f"run {rnd} differs at {key}"


def test_general_path_agrees_with_mfma_path(dev):
    B, T, C, H = 2, 200, 256, 4
    x = synth.qkv(B, T, C, seed=11)
    g = synth.grad_out(B, T, C, seed=11)
    y, lse = gpu_fwd(dev, x, H)
    gx, D = gpu_bwd(dev, x, y, lse, g, H)
    prev = gpt_amd.set_path(1)
    try:
        y1, l1 = gpu_fwd(dev, x, H)
        gx1, D1 = gpu_bwd(dev, x, y, lse, g, H)
    finally:
        gpt_amd.set_path(prev)
    assert rel_err(y, y1) <= FWD_RTOL and rel_err(lse, l1) <= FWD_RTOL
    assert rel_err(gx, gx1) <= BWD_RTOL and rel_err(D, D1) <= BWD_RTOL


def _slices_and_invariants(dev, x, g, H, slices, tag):
    B, T, W = x.shape
    C = W // 3
    d = C // H
    y, lse = gpu_fwd(dev, x, H)
    gx, D = gpu_bwd(dev, x, y, lse, g, H)
    assert np.all(np.isfinite(y)) and np.all(np.isfinite(lse)) and np.all(np.isfinite(gx))
    for b, h in slices:
        xs = qkv_slice(x, b, h, H)
        yr, lr = pyoracle.forward(xs, 1)
        assert_close(f"{tag} O[{b},{h}]", row_slice(y, b, h, H), yr, FWD_RTOL)
        assert_close(f"{tag} LSE[{b},{h}]", lse[b:b + 1, :, h:h + 1], lr, FWD_RTOL)
        gr, Dr = pyoracle.backward(xs, yr, lr, row_slice(g, b, h, H), 1)
        gs = qkv_slice(gx, b, h, H)
        for name, sl in (("dQ", slice(0, d)), ("dK", slice(d, 2 * d)), ("dV", slice(2 * d, 3 * d))):
            assert_close(f"{tag} {name}[{b},{h}]", gs[..., sl], gr[..., sl], BWD_RTOL)
        assert_close(f"{tag} D[{b},{h}]", D[b:b + 1, :, h:h + 1], Dr, BWD_RTOL)
    # invariants on every (b, h)
    dk = gx[..., C:2 * C].astype(np.float64).reshape(B, T, H, d)
    dv = gx[..., 2 * C:].astype(np.float64).reshape(B, T, H, d)
    go = g.astype(np.float64).reshape(B, T, H, d)
    assert np.abs(dk.sum(1)).max() <= 1e-4 * np.abs(dk).max() * np.sqrt(T)
    assert rel_err(dv.sum(1), go.sum(1)) <= 1e-4
    return y, lse, gx, D


def _whole_config_fp64(dev, x, g, H, outs, tag):
    """Every (b, h) of a configuration against the dense float64 restatement
    (tests/dense64.py, pinned to the oracle by tests/test_oracle.py), computed
    with torch in float64 on the device: O and LSE of the forward; dQ, dK, dV
    and D of the backward (which ran from the kernels' own O and LSE, checked
    first), norm-wise and elementwise (tests/tolerances.py)."""
    from tests import dense64

    y, lse, gx, D = outs
    C = x.shape[-1] // 3
    y64, l64, g64, D64 = (t.cpu().numpy() for t in dense64.fwd_bwd_torch(_to(dev, x), _to(dev, g), H))
    assert_close(f"{tag} O (all b,h, fp64)", y, y64, FWD_RTOL)
    assert_close(f"{tag} LSE (all b,h, fp64)", lse, l64, FWD_RTOL)
    for name, sl in (("dQ", slice(0, C)), ("dK", slice(C, 2 * C)), ("dV", slice(2 * C, 3 * C))):
        assert_close(f"{tag} {name} (all b,h, fp64)", gx[..., sl], g64[..., sl], BWD_RTOL)
    assert_close(f"{tag} D (all b,h, fp64)", D, D64, BWD_RTOL)


def test_config3_layers_B16_T256(dev):
    """12 layers of B=16, T=256 with per-layer scale U[0.5, 2]: layer 0 and 11
    in full against the oracle, the others on (b, h) slices against the oracle
    and invariants; every layer in full (all 192 (b, h)) against the dense
    float64 restatement."""
    B, T, C, H = 16, 256, 768, 12
    scales = synth.layer_scales(12, 1237)
    for layer in range(12):
        seed = 1237 + layer
        x = synth.qkv(B, T, C, seed, scale=float(scales[layer]))
        g = synth.grad_out(B, T, C, seed)
        if layer in (0, 11):
            check_fwd_bwd(dev, x, g, H, tag=f"C3 layer {layer}")
        outs = _slices_and_invariants(dev, x, g, H, [(0, 0), (B - 1, H - 1)], f"C3 layer {layer}")
        _whole_config_fp64(dev, x, g, H, outs, f"C3 layer {layer}")


def test_config4_B8_T1024(dev):
    """B=8 T=1024: (b, h) slices against the oracle, invariants, and all 96
    (b, h) against the dense float64 restatement."""
    B, T, C, H = 8, 1024, 768, 12
    x = synth.qkv(B, T, C, 1238)
    g = synth.grad_out(B, T, C, 1238)
    outs = _slices_and_invariants(dev, x, g, H, [(0, 0), (3, 5), (7, 11)], "C4")
    _whole_config_fp64(dev, x, g, H, outs, "C4")


def test_config5a_B2_T4096(dev):
    """B=2 T=4096: (b, h) slices against the oracle, invariants, and all 24
    (b, h) against the dense float64 restatement."""
    B, T, C, H = 2, 4096, 768, 12
    x = synth.qkv(B, T, C, 1239)
    g = synth.grad_out(B, T, C, 1239)
    outs = _slices_and_invariants(dev, x, g, H, [(0, 0), (1, 11)], "C5a")
    _whole_config_fp64(dev, x, g, H, outs, "C5a")


@pytest.mark.parametrize("T", [32736, 32800])
def test_longest_rows_single_head(dev, T):
    """Maximum sequence length of the head_dim-64 backward: at T = 32736 one
    (b, h)'s dS tiles (523776 x 4 KiB) stay just below the 2^31-byte buffer
    range the dQ kernel reads them through; at T = 32800 the call takes the
    general-d kernels. B=1, H=1, d=64 (the oracle would take hours here):
    O, LSE and dQ at sampled rows, dK and dV at keys 0 and T - 1 and D
    everywhere against float64 numpy (dQ, dK_0 and dV_0 from the kernels' own
    LSE and D, which are checked first), plus the size-independent invariants."""
    B, C, H, d = 1, 64, 1, 64
    x = synth.qkv(B, T, C, seed=777)
    g = synth.grad_out(B, T, C, seed=777)
    gpt_amd.timing_enable(True)
    try:
        y, lse = gpu_fwd(dev, x, H)
        gx, D = gpu_bwd(dev, x, y, lse, g, H)
        t = gpt_amd.timing_read()
    finally:
        gpt_amd.timing_enable(False)
    assert t["bwd_dkdv"][1] == (1 if T <= 32736 else 0), t
    assert t["other"][1] == (0 if T <= 32736 else 1), t  # the forward stays on the MFMA kernels
    assert np.all(np.isfinite(y)) and np.all(np.isfinite(lse)) and np.all(np.isfinite(gx))
    q, k, v = (x[0, :, i * C:(i + 1) * C].astype(np.float64) for i in range(3))
    go = g[0].astype(np.float64)
    sc = 1.0 / np.sqrt(d)
    L = lse[0, :, 0].astype(np.float64)
    rows = (0, 1, 4095, T // 2, T - 2, T - 1)
    dq, dq_ref = [], []
    for i in rows:
        s = q[i] @ k[:i + 1].T * sc
        lr = np.logaddexp.reduce(s)
        p = np.exp(s - lr)
        # a single 64-element output row formed from up to 32800 terms, against
        # float64: up to 2.7e-6 max|r| of elementwise excess measured, so the
        # elementwise term is 0.5 rtol here
        assert_close(f"T={T} O[{i}]", y[0, i], p @ v[:i + 1], FWD_RTOL, elem_frac=0.5)
        assert abs(L[i] - lr) <= FWD_RTOL * max(1.0, abs(lr)), (i, L[i], lr)
        pk = np.exp(s - L[i])
        ds = pk * (go[i] @ v[:i + 1].T - D[0, i, 0]) * sc
        dq.append(gx[0, i, :C])
        dq_ref.append(ds @ k[:i + 1])
    # row-wise norms: dQ_0 is zero up to rounding (dS_00 = dO_0 . v_0 - D_0 = 0)
    assert_close(f"T={T} dQ{rows}", np.stack(dq), np.stack(dq_ref), BWD_RTOL)
    assert_close(f"T={T} D", D[0, :, 0], np.sum(go * y[0].astype(np.float64), axis=1), BWD_RTOL)
    # key 0 sees every query, key T - 1 only the last
    p0 = np.exp(q @ k[0] * sc - L)
    assert_close(f"T={T} dV[0]", gx[0, 0, 2 * C:], p0 @ go, BWD_RTOL)
    ds0 = p0 * (go @ v[0] - D[0, :, 0].astype(np.float64)) * sc
    assert_close(f"T={T} dK[0]", gx[0, 0, C:2 * C], ds0 @ q, BWD_RTOL)
    pl = np.exp(q[T - 1] @ k[T - 1] * sc - L[T - 1])
    assert_close(f"T={T} dV[T-1]", gx[0, T - 1, 2 * C:], pl * go[T - 1], BWD_RTOL)
    dsl = pl * (go[T - 1] @ v[T - 1] - D[0, T - 1, 0]) * sc
    assert_close(f"T={T} dK[T-1]", gx[0, T - 1, C:2 * C], dsl * q[T - 1], BWD_RTOL)
    dk = gx[0, :, C:2 * C].astype(np.float64)
    assert np.abs(dk.sum(0)).max() <= 1e-4 * np.abs(dk).max() * np.sqrt(T)
    assert rel_err(gx[0, :, 2 * C:].astype(np.float64).sum(0), go.sum(0)) <= 1e-4


def test_backward_overwrites_grad_x_and_is_repeatable(dev):
    import torch

    B, T, C, H = 2, 160, 768, 12
    x = _to(dev, synth.qkv(B, T, C, 21))
    g = _to(dev, synth.grad_out(B, T, C, 21))
    y, lse = gpt_amd.attention_forward(x, H)
    gx = torch.full((B, T, 3 * C), float("nan"), device=dev)
    D = torch.full((B, T, H), float("nan"), device=dev)
    gpt_amd.device_flash_attention_backward(gx, D, lse, g, y, x, B, T, C, H)
    first = gx.clone()
    gpt_amd.device_flash_attention_backward(gx, D, lse, g, y, x, B, T, C, H)
    torch.cuda.synchronize()
    assert torch.isfinite(first).all()
    # no atomics on the default path: bit-identical run to run
    assert torch.equal(first, gx)
    # the atomic-dQ path (another kernel, other summation orders) overwrites
    # grad_x too and agrees within fp32 rounding
    prev = gpt_amd.set_path(2)
    try:
        gx.fill_(float("nan"))
        gpt_amd.device_flash_attention_backward(gx, D, lse, g, y, x, B, T, C, H)
        torch.cuda.synchronize()
    finally:
        gpt_amd.set_path(prev)
    assert torch.isfinite(gx).all()
    for sl in (slice(0, C), slice(C, 2 * C), slice(2 * C, 3 * C)):
        assert rel_err(gx[..., sl].cpu().numpy(), first[..., sl].cpu().numpy()) <= 1e-6


@pytest.mark.parametrize("T", [256, 300])
def test_release_workspaces_then_backward_again(dev, T):
    """gpt_hip_attn_release_workspaces frees the per-stream dS workspace; the
    next backward allocates a new one (its control block zeroed again) and
    gives the same bits, on the fused (T <= 256) and the two-launch form.
    Releasing with nothing allocated is a no-op."""
    import torch

    B, C, H = 3, 768, 12
    x = _to(dev, synth.qkv(B, T, C, 500 + T))
    g = _to(dev, synth.grad_out(B, T, C, 500 + T))
    y, lse = gpt_amd.attention_forward(x, H)
    first, D0 = gpt_amd.attention_backward(x, y, lse, g, H)
    gpt_amd.release_workspaces()
    gpt_amd.release_workspaces()
    again, D1 = gpt_amd.attention_backward(x, y, lse, g, H)
    torch.cuda.synchronize()
    assert torch.isfinite(first).all()
    assert torch.equal(first, again) and torch.equal(D0, D1)


def test_inputs_untouched_and_side_stream(dev):
    import torch

    B, T, C, H = 2, 96, 768, 12
    x = _to(dev, synth.qkv(B, T, C, 31))
    g = _to(dev, synth.grad_out(B, T, C, 31))
    x0, g0 = x.clone(), g.clone()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        y, lse = gpt_amd.attention_forward(x, H, stream=s)
        gx, D = gpt_amd.attention_backward(x, y, lse, g, H, stream=s)
    s.synchronize()
    assert torch.equal(x, x0) and torch.equal(g, g0)
    yr, lr = pyoracle.forward(x.cpu().numpy(), H)
    assert rel_err(y.cpu().numpy(), yr) <= FWD_RTOL


def test_concurrent_streams_get_separate_workspaces(dev):
    """Backward calls queued on two streams at once (each with its own dS
    workspace, allocated on first use per stream) give the single-stream
    results bit for bit, at two sizes so one stream's workspace grows."""
    import torch

    C, H = 768, 12
    shapes = [(4, 256), (2, 512)]
    data = []
    for B, T in shapes:
        x = _to(dev, synth.qkv(B, T, C, 77 + T))
        g = _to(dev, synth.grad_out(B, T, C, 77 + T))
        y, lse = gpt_amd.attention_forward(x, H)
        ref_gx, ref_D = gpt_amd.attention_backward(x, y, lse, g, H)
        data.append((x, g, y, lse, ref_gx, ref_D))
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    for rep in range(2):
        for k, st in ((0, s1), (1, s2), (1, s1), (0, s2)):
            x, g, y, lse, _, _ = data[k]
            with torch.cuda.stream(st):
                outs.append((k,) + gpt_amd.attention_backward(x, y, lse, g, H, stream=st))
    torch.cuda.synchronize()
    for k, gx, D in outs:
        assert torch.equal(gx, data[k][4]) and torch.equal(D, data[k][5])


def test_batch_slices_are_independent(dev):
    """Running (b, h) slices one at a time gives the batched result."""
    B, T, C, H = 3, 130, 768, 12
    x = synth.qkv(B, T, C, 41)
    y, lse = gpu_fwd(dev, x, H)
    for b in range(B):
        yb, lb = gpu_fwd(dev, np.ascontiguousarray(x[b:b + 1]), H)
        assert np.array_equal(yb, y[b:b + 1]) and np.array_equal(lb, lse[b:b + 1])


@pytest.mark.parametrize("T", [100, 300])
def test_launch_timer_counts_each_kernel(dev, T):
    """One launch per kernel: up to T = 256 the backward is the one fused
    kernel (D rows, dK/dV, dS tiles and dQ); longer rows take the D-row
    kernel, the dK/dV kernel and the dQ kernel."""
    import torch

    B, C, H = 2, 768, 12
    x = _to(dev, synth.qkv(B, T, C, 51))
    g = _to(dev, synth.grad_out(B, T, C, 51))
    gpt_amd.timing_enable(True)
    try:
        y, lse = gpt_amd.attention_forward(x, H)
        gpt_amd.attention_backward(x, y, lse, g, H)
        torch.cuda.synchronize()
        t = gpt_amd.timing_read()
    finally:
        gpt_amd.timing_enable(False)
    kinds = ("fwd", "bwd_fused") if T <= 256 else ("fwd", "bwd_rowdot", "bwd_dkdv", "bwd_dq")
    for k in kinds:
        ms, n = t[k]
        assert n == 1 and ms > 0, (k, t[k])
    for k in set(gpt_amd.attention.KERNEL_KINDS) - set(kinds):
        assert t[k] == (0.0, 0), (k, t[k])
    assert gpt_amd.timing_read()["fwd"] == (0.0, 0)  # read forgets


@pytest.mark.parametrize("B,T", [(16, 255), (16, 200), (3, 257), (1, 100)])
def test_outputs_stay_in_their_buffers(dev, B, T):
    """Every output written only inside its tensor: y, lse, grad_x and D are
    views into buffers with 1024-float guard bands on both sides, filled with
    a bit pattern no kernel writes; after the forward and the backward the
    guards are unchanged and the outputs match the oracle. The shapes take
    the Q-stationary forward with ragged rows and the one-launch backward
    (B = 16), and the smaller-grid forwards and the two-launch backward."""
    import torch

    C, H, G = 768, 12, 1024
    x = synth.qkv(B, T, C, 61)
    g = synth.grad_out(B, T, C, 61)
    xd, gd = _to(dev, x), _to(dev, g)
    pat = -12345.678

    def guarded(n):
        buf = torch.full((G + n + G,), pat, dtype=torch.float32, device=dev)
        return buf, buf[G:G + n]

    ybuf, y = guarded(B * T * C)
    lbuf, lse = guarded(B * T * H)
    gbuf, gx = guarded(B * T * 3 * C)
    dbuf, D = guarded(B * T * H)
    gpt_amd.attention.device_flash_attention_forward(y, lse, xd, B, T, C, H)
    gpt_amd.attention.device_flash_attention_backward(gx, D, lse, gd, y, xd, B, T, C, H)
    torch.cuda.synchronize()
    for name, buf in (("y", ybuf), ("lse", lbuf), ("grad_x", gbuf), ("D", dbuf)):
        guards = torch.cat([buf[:G], buf[-G:]])
        assert bool(torch.all(guards == pat)), f"{name}: a guard band was written"
    yr, lr = pyoracle.forward(x, H)
    assert_close(f"B={B} T={T} O", y.view(B, T, C).cpu().numpy(), yr, FWD_RTOL)
    assert_close(f"B={B} T={T} LSE", lse.view(B, T, H).cpu().numpy(), lr, FWD_RTOL)
    gr, Dr = pyoracle.backward(x, y.view(B, T, C).cpu().numpy(), lse.view(B, T, H).cpu().numpy(), g, H)
    assert_close(f"B={B} T={T} dQKV", gx.view(B, T, 3 * C).cpu().numpy(), gr, BWD_RTOL)
    assert_close(f"B={B} T={T} D", D.view(B, T, H).cpu().numpy(), Dr, BWD_RTOL)
