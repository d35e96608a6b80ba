"""The one-launch backward (T <= 256) without whole-grid residency, and its
wait time limits.

The owner of a dQ item waits a bounded time for its dS tiles, then hands the
item to extra workgroups at the end of the grid, which run it once every
main workgroup has decided (gpt_amd/csrc/attn_bwd_fused_kernel.h). These tests run
it (1) with its waits forced to their limits from the host, then again
normally, and (2) while another stream's kernel holds half of the compute
units, so that only part of the grid is resident at a time. Every call goes
through the C ABI. The CPU model of the same protocol is
tests/test_dq_handoff_model.py.
"""
import ctypes
import os
import time

import pytest

import gpt_amd
from gpt_amd import synth

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
C, H, T = 768, 12, 256


def _inputs(dev, B, seed):
    import torch

    x = torch.from_numpy(synth.qkv(B, T, C, seed)).to(dev)
    g = torch.from_numpy(synth.grad_out(B, T, C, seed)).to(dev)
    y, lse = gpt_amd.attention_forward(x, H)
    return x, g, y, lse


def _bwd(entry, x, g, y, lse, B, stream=None):
    import torch

    gx = torch.empty(B, T, 3 * C, device=x.device)
    D = torch.empty(B, T, H, device=x.device)
    entry(gx, D, lse, g, y, x, B, T, C, H, stream)
    return gx, D


ENTRIES = {
    "default": gpt_amd.device_flash_attention_backward,
    "noalloc": gpt_amd.device_flash_attention_backward_noalloc,
}


@pytest.mark.parametrize("entry", sorted(ENTRIES))
@pytest.mark.parametrize("B", [8, 16])
def test_wait_timeouts_are_counted_and_the_next_call_is_clean(dev, B, entry):
    """With every awaited count raised by one (a count that never arrives)
    and zero time limits, every owner of a dQ item of key groups 1..3 hands
    its item over and the wait of the workgroup that takes it reaches its
    limit: B * H * 3 expired waits, reported by gpt_hip_attn_wait_timeouts.
    A call made right after with the defaults, before the count is read (and
    the control block cleared), already gives the clean call's bits: the
    timed-out launch left its counters at 0. B = 8 takes the kernel's
    half-grid instantiation, B = 16 the full-grid one."""
    import torch

    fn = ENTRIES[entry]
    x, g, y, lse = _inputs(dev, B, 9100 + B)
    gpt_amd.wait_timeouts()
    clean, D0 = _bwd(fn, x, g, y, lse, B)
    torch.cuda.synchronize()
    assert gpt_amd.wait_timeouts() == 0
    try:
        gpt_amd.set_wait_limit(0, 1)
        _bwd(fn, x, g, y, lse, B)
    finally:
        gpt_amd.set_wait_limit(-1, 0)
    again, D1 = _bwd(fn, x, g, y, lse, B)
    torch.cuda.synchronize()
    assert torch.equal(again, clean) and torch.equal(D1, D0)
    n = gpt_amd.wait_timeouts()
    print(f"B={B} {entry}: {n} expired waits with the forced limit", flush=True)
    assert n == B * H * 3
    third, D2 = _bwd(fn, x, g, y, lse, B)
    torch.cuda.synchronize()
    assert gpt_amd.wait_timeouts() == 0
    assert torch.equal(third, clean) and torch.equal(D2, D0)


def _occupier():
    path = os.path.join(ROOT, "tests", "libgpt_test_occupy.so")
    assert os.path.exists(path), f"{path} is missing: build it with __graft_entry__.build()"
    lib = ctypes.CDLL(path)
    lib.gpt_test_occupy.argtypes = [ctypes.c_int, ctypes.c_longlong, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_void_p]
    lib.gpt_test_occupy.restype = ctypes.c_int
    return lib


@pytest.mark.parametrize("entry", sorted(ENTRIES))
def test_backward_with_half_the_cus_held_by_another_stream(dev, entry):
    """While a kernel on another stream holds half of the CUs (one workgroup
    with 128 KiB of LDS per CU, for 300 ms), the C3-sized backward (768
    workgroups, 3 per CU when all CUs are free) has at most half of its grid
    resident at a time. It must finish while the CUs are still held, give the
    solo run's bits, and record no wait timeout. Two streams overlap only if
    the runtime gave them different hardware queues; a pair that shares one
    runs the two kernels in turn (still checked bit for bit), and the next
    pair of streams is taken, up to four pairs."""
    import torch

    props = torch.cuda.get_device_properties(dev)
    n_cu = props.multi_processor_count
    B = 16
    x, g, y, lse = _inputs(dev, B, 9300)
    fn = ENTRIES[entry]
    solo, D0 = _bwd(fn, x, g, y, lse, B)
    torch.cuda.synchronize()
    assert gpt_amd.wait_timeouts() == 0

    occ = _occupier()
    hold = n_cu // 2
    overlapped = False
    for attempt in range(4):
        started = torch.zeros(1, dtype=torch.int32, device=dev)
        sink = torch.zeros(1, dtype=torch.float32, device=dev)
        s_occ, s_bwd = torch.cuda.Stream(), torch.cuda.Stream()
        ev = {k: torch.cuda.Event(enable_timing=True) for k in ("occ0", "occ1", "bwd1")}
        gx = torch.empty(B, T, 3 * C, device=dev)
        D = torch.empty(B, T, H, device=dev)
        torch.cuda.synchronize()
        print(f"{entry}: holding {hold} of {n_cu} CUs for 300 ms (stream pair {attempt})", flush=True)
        ev["occ0"].record(s_occ)
        assert occ.gpt_test_occupy(hold, 300000, started.data_ptr(), sink.data_ptr(), s_occ.cuda_stream) == 0
        ev["occ1"].record(s_occ)
        time.sleep(0.05)  # the holding workgroups are resident long before they end
        fn(gx, D, lse, g, y, x, B, T, C, H, s_bwd)
        ev["bwd1"].record(s_bwd)
        torch.cuda.synchronize()
        t_bwd = ev["occ0"].elapsed_time(ev["bwd1"])
        t_occ = ev["occ0"].elapsed_time(ev["occ1"])
        print(f"{entry}: backward done {t_bwd:.2f} ms, holder done {t_occ:.2f} ms after the holder's start; "
              f"holder workgroups {int(started.item())}", flush=True)
        assert int(started.item()) == hold
        assert gpt_amd.wait_timeouts() == 0
        assert torch.equal(gx, solo) and torch.equal(D, D0)
        if t_bwd < t_occ:
            overlapped = True
            break
    assert overlapped, "the backward never ran while the CUs were held (every stream pair serialised)"


def test_shapes_change_between_calls_on_one_control_block(dev):
    """Calls of different shapes in a row on one stream share its control
    block. Each must give the bits it gives on a freshly zeroed block (a
    layout that moved with the shape once read an earlier call's start marks
    as counters: T = 65 after T = 64 gave wrong dQ)."""
    import torch

    shapes = [(2, 64, 3), (2, 65, 3), (3, 256, 12), (1, 129, 12), (8, 256, 12), (2, 65, 3)]
    fresh = []
    for k, (B, Tk, Hk) in enumerate(shapes):
        Ck = 64 * Hk
        x = torch.from_numpy(synth.qkv(B, Tk, Ck, 9500 + k)).to(dev)
        g = torch.from_numpy(synth.grad_out(B, Tk, Ck, 9500 + k)).to(dev)
        y, lse = gpt_amd.attention_forward(x, Hk)
        gpt_amd.release_workspaces()
        gx, D = gpt_amd.attention_backward(x, y, lse, g, Hk)
        torch.cuda.synchronize()
        fresh.append((x, g, y, lse, Hk, gx, D))
    for rep in range(2):
        for x, g, y, lse, Hk, gx0, D0 in fresh:
            gx, D = gpt_amd.attention_backward(x, y, lse, g, Hk)
            torch.cuda.synchronize()
            assert torch.equal(gx, gx0) and torch.equal(D, D0)
    assert gpt_amd.wait_timeouts() == 0
