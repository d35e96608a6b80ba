"""The GPT-2 ops library (gpt_amd/libgpt_hip_ops.so) loads, exports exactly
what include/gpt_hip_ops.h declares, does not link the CPU oracle, and
validates arguments before touching a device. CPU only: no compute call is
made here."""
import os
import re

import pytest

from gpt_amd import ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gpt_hip_ops.h")

EINVAL, ENULL, ENODEV = -1, -2, -4
P = 4096  # a non-null address that is never dereferenced by these calls


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    return sorted(set(re.findall(r"\b(gpt_hip_\w+)\s*\(", text)))


def test_header_covers_every_reference_compute_method():
    """One entry point per IGPTBackend compute method other than attention
    (backend_interface.h:26-237), plus the two fill initialisers."""
    names = declared_functions()
    for stem in ("embedding_forward", "embedding_backward", "unembedding_forward", "unembedding_backward",
                 "layernorm_residual_forward", "layernorm_residual_backward", "linear_activation_forward",
                 "linear_backward", "activation_backward", "softmax_forward", "cross_entropy_softmax_backward",
                 "cross_entropy_loss", "adamw_step", "scale_and_clip_grad", "fill_normal", "fill_const"):
        assert f"gpt_hip_{stem}_f32" in names, stem
    assert "gpt_hip_ops_last_error" in names


def test_library_exports_every_declared_symbol():
    lib = ops.load_library()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in include/gpt_hip_ops.h but not exported"


def test_python_binding_declares_every_symbol():
    assert sorted(ops._SIGS) == sorted(n for n in declared_functions()
                                       if n not in ("gpt_hip_ops_last_error", "gpt_hip_ops_gemm_info"))


def test_library_has_no_oracle_dependency():
    data = open(ops.lib_path(), "rb").read()
    assert b"ops_oracle" not in data and b"ref_op_" not in data


def _err():
    return ops.load_library().gpt_hip_ops_last_error().decode()


def test_invalid_arguments_are_rejected_before_any_device_call():
    lib = ops.load_library()
    assert lib.gpt_hip_embedding_forward_f32(P, P, P, P, -1, 4, 8, 0, None) == EINVAL
    assert "gpt_hip_embedding_forward_f32" in _err()
    assert lib.gpt_hip_softmax_forward_f32(P, P, 1, 1, 20, 16, None) == EINVAL
    assert lib.gpt_hip_linear_backward_f32(P, P, P, P, P, P, 1, 1, 0, 4, None) == EINVAL
    assert lib.gpt_hip_scale_and_clip_grad_f32(P, 16, 1.0, 0, None) == EINVAL
    assert lib.gpt_hip_adamw_step_f32(P, P, P, P, -5, 1e-3, 0.9, 0.95, 1e-8, 0.0, 1, None) == EINVAL


def test_null_pointers_are_rejected():
    lib = ops.load_library()
    assert lib.gpt_hip_layernorm_residual_forward_f32(P, None, P, P, None, P, P, 1, 2, 8, None) == ENULL
    assert lib.gpt_hip_linear_activation_forward_f32(P, None, P, P, P, 1, 1, 2, 4, 4, None) == ENULL
    assert lib.gpt_hip_cross_entropy_loss_f32(None, P, P, 1, 1, 4, None) == ENULL


def test_empty_shapes_are_noops():
    lib = ops.load_library()
    assert lib.gpt_hip_embedding_forward_f32(None, None, None, None, 0, 5, 8, 0, None) == 0
    assert lib.gpt_hip_linear_backward_f32(None, None, None, None, None, None, 2, 0, 4, 4, None) == 0
    assert lib.gpt_hip_adamw_step_f32(None, None, None, None, 0, 1e-3, 0.9, 0.95, 1e-8, 0.0, 1, None) == 0
    assert lib.gpt_hip_fill_const_f32(None, 1.0, 0, None) == 0


def test_no_device_is_reported():
    import gpt_amd

    if gpt_amd.device_ok():
        pytest.skip("a HIP device is present")
    lib = ops.load_library()
    assert lib.gpt_hip_fill_const_f32(P, 1.0, 4, None) == ENODEV
    with pytest.raises(ops.HipOpsError) as ei:
        ops.device_fill_const(P, 1.0, 4)
    assert ei.value.code == ENODEV
