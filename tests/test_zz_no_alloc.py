"""The backward entry point that allocates nothing
(gpt_hip_attn_bwd_f32_noalloc, include/gpt_hip_attn.h) against the default
one (gpt_hip_attn_bwd_f32): both run the same kernels, so the results must be
identical bit for bit. Two calls in a row, the second smaller than the first
(its dS tiles reuse the scratch array the first call left filled), then the
largest row length the scratch array holds, and the first length past it,
which must be refused before anything is launched. Every call goes through
the C ABI."""
import numpy as np
import pytest

import gpt_amd
from gpt_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def no_wait_timeouts(dev):
    """The scratch array's control block records no timed-out dQ wait."""
    gpt_amd.wait_timeouts()
    yield
    assert gpt_amd.wait_timeouts() == 0

ERANGE = -6


def _run(dev, B, T, C, H, seed, noalloc):
    import torch

    x = torch.from_numpy(synth.qkv(B, T, C, seed=seed)).to(dev)
    g = torch.from_numpy(synth.grad_out(B, T, C, seed=seed)).to(dev)
    y, lse = gpt_amd.attention_forward(x, H)
    gx = torch.full((B, T, 3 * C), float("nan"), device=dev)
    D = torch.full((B, T, H), float("nan"), device=dev)
    fn = (gpt_amd.device_flash_attention_backward_noalloc if noalloc
          else gpt_amd.device_flash_attention_backward)
    fn(gx, D, lse, g, y, x, B, T, C, H)
    torch.cuda.synchronize()
    return gx.cpu().numpy(), D.cpu().numpy()


def _same(a, b):
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("shapes", [[(4, 300, 768, 12), (2, 100, 768, 12)]])
def test_noalloc_matches_default_two_calls(dev, shapes):
    for k, (B, T, C, H) in enumerate(shapes):
        print(f"noalloc call {k}: B={B} T={T} C={C} H={H}", flush=True)
        ref = _run(dev, B, T, C, H, 4100 + k, noalloc=False)
        got = _run(dev, B, T, C, H, 4100 + k, noalloc=True)
        assert np.isfinite(got[0]).all() and np.isfinite(got[1]).all()
        assert _same(got[0], ref[0]), f"grad_x differs at B={B} T={T}"
        assert _same(got[1], ref[1]), f"D differs at B={B} T={T}"


def test_noalloc_longest_rows_and_refusal(dev):
    import torch

    # T = 5760: 180 query blocks, 16290 dS tiles = 63.6 MiB, the largest that fits
    B, T, C, H = 1, 5760, 64, 1
    print(f"noalloc at the limit: B={B} T={T} C={C} H={H}", flush=True)
    ref = _run(dev, B, T, C, H, 4200, noalloc=False)
    got = _run(dev, B, T, C, H, 4200, noalloc=True)
    assert _same(got[0], ref[0]) and _same(got[1], ref[1])
    # T = 5761: 181 query blocks, 64.3 MiB of dS tiles: refused, outputs untouched
    T = 5761
    x = torch.zeros((B, T, 3 * C), device=dev)
    y = torch.zeros((B, T, C), device=dev)
    lse = torch.zeros((B, T, H), device=dev)
    gx = torch.full((B, T, 3 * C), 7.0, device=dev)
    D = torch.full((B, T, H), 7.0, device=dev)
    lib = gpt_amd.load_library()
    rc = lib.gpt_hip_attn_bwd_f32_noalloc(gx.data_ptr(), D.data_ptr(), lse.data_ptr(), y.data_ptr(),
                                          y.data_ptr(), x.data_ptr(), B, T, C, H, None)
    assert rc == ERANGE, rc
    assert b"scratch" in lib.gpt_hip_attn_last_error()
    torch.cuda.synchronize()
    assert (gx == 7.0).all().item() and (D == 7.0).all().item()
