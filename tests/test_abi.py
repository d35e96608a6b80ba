"""The C-ABI library loads, exports exactly what include/gpt_hip_attn.h
declares, and validates arguments before touching a device. CPU only: no
compute call is made here."""
import ctypes
import os
import re

import pytest

import gpt_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gpt_hip_attn.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gpt_hip_attn_\w+)\s*\(", text)))


def test_header_declares_the_op_pair():
    names = declared_functions()
    assert "gpt_hip_attn_fwd_f32" in names and "gpt_hip_attn_bwd_f32" in names


def test_library_exports_every_declared_symbol():
    lib = gpt_amd.load_library()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in include/gpt_hip_attn.h but not exported"


def test_library_has_no_oracle_dependency():
    """The product library never links the CPU oracle."""
    data = open(gpt_amd.lib_path(), "rb").read()
    assert b"oracle_attn" not in data and b"ref_attn_" not in data


def _fwd(*args):
    lib = gpt_amd.load_library()
    return lib.gpt_hip_attn_fwd_f32(*args)


def _bwd(*args):
    lib = gpt_amd.load_library()
    return lib.gpt_hip_attn_bwd_f32(*args)


def _err():
    return gpt_amd.load_library().gpt_hip_attn_last_error().decode()


EINVAL, ENULL, EHEADDIM, ENODEV = -1, -2, -3, -4
P = 4096  # a non-null address that is never dereferenced by these calls


@pytest.mark.parametrize("B,T,C,H", [(-1, 4, 64, 1), (1, -2, 64, 1), (1, 4, 0, 1), (1, 4, 64, 0),
                                     (1, 4, 64, -3), (1, 4, 100, 3)])
def test_invalid_shapes_are_rejected(B, T, C, H):
    assert _fwd(P, P, P, B, T, C, H, None) == EINVAL
    assert "gpt_hip_attn_fwd_f32" in _err()
    assert _bwd(P, P, P, P, P, P, B, T, C, H, None) == EINVAL


def test_unsupported_head_dim():
    assert _fwd(P, P, P, 1, 4, 4 * 300, 4, None) == EHEADDIM
    assert "head_dim 300" in _err()


def test_empty_batch_or_sequence_is_a_noop():
    assert _fwd(None, None, None, 0, 10, 64, 1, None) == 0
    assert _bwd(None, None, None, None, None, None, 3, 0, 64, 1, None) == 0


def test_null_pointers_are_rejected():
    assert _fwd(None, P, P, 1, 4, 64, 1, None) == ENULL
    assert _bwd(P, P, P, None, P, P, 1, 4, 64, 1, None) == ENULL


def test_no_device_is_reported():
    if gpt_amd.device_ok():
        pytest.skip("a HIP device is present")
    assert _fwd(P, P, P, 1, 4, 64, 1, None) == ENODEV
    with pytest.raises(gpt_amd.HipAttentionError) as ei:
        gpt_amd.device_flash_attention_forward(P, P, P, 1, 4, 64, 1)
    assert ei.value.code == ENODEV


def test_release_workspaces_without_device_is_an_error():
    if gpt_amd.device_ok():
        pytest.skip("a HIP device is present")
    assert gpt_amd.load_library().gpt_hip_attn_release_workspaces() == ENODEV
    assert gpt_amd.load_library().gpt_hip_attn_wait_timeouts() == ENODEV


def test_set_path_roundtrip():
    assert gpt_amd.set_path(1) == 0
    assert gpt_amd.set_path(0) == 1
    with pytest.raises(gpt_amd.HipAttentionError):
        gpt_amd.set_path(7)


def test_python_wrapper_rejects_host_tensors():
    torch = pytest.importorskip("torch")
    x = torch.zeros(1, 4, 192)
    with pytest.raises(ValueError):
        gpt_amd.attention_forward(x, 3)


def test_timing_without_device_is_an_error():
    if gpt_amd.device_ok():
        pytest.skip("a HIP device is present")
    assert gpt_amd.load_library().gpt_hip_attn_timing_enable(1) == ENODEV
    assert gpt_amd.timing_read() == {k: (0.0, 0) for k in gpt_amd.attention.KERNEL_KINDS}
