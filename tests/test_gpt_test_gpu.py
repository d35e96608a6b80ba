"""The reference's own whole-model gradient test, run against the HIP backend.

oracle/_ref/gpt_test is the reference's src/model/gpt_test.cpp, gpt.cpp and
cpu_backend.cpp compiled unchanged, linked with gpt_amd/adapter (its
"CUDABackend" is the HIP attention adapter: attention on the GPU through the
C ABI, every other op on the reference CPU backend). It computes the 16
weight-gradient tensors on the CPU backend and on the adapter and compares
CPU vs GPU, then GPU vs the fixture gradients (tests/golden/gpt_test), each
with |a - b| <= 1e-5 (reference src/model/gpt_test.cpp:12, 257-269). The
config has head_dim 8, T = 64, B = 1, so this exercises the general-d kernels.

oracle/_ref/gpt_test_full is the same test with its "CUDABackend" the all-GPU
HipBackend (gpt_amd/adapter/hip_backend.*): every op of the model, forward,
backward and loss, runs on the GPU through libgpt_hip_attn.so and
libgpt_hip_ops.so, and the weight gradients must match the reference CPU
backend and the fixture gradients at the test's own 1e-5.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "oracle", "_ref", "gpt_test")
BIN_FULL = os.path.join(ROOT, "oracle", "_ref", "gpt_test_full")
GOLD = os.path.join(ROOT, "tests", "golden", "gpt_test")

pytestmark = pytest.mark.gpu


def _run_gpt_test(binary, tmp_path):
    if not os.path.exists(binary):
        pytest.skip(f"{binary} not built (needs /root/reference at build time)")
    data = tmp_path / "data"
    data.mkdir()
    for f in os.listdir(GOLD):
        shutil.copy(os.path.join(GOLD, f), data / f)
    r = subprocess.run([binary], cwd=tmp_path, capture_output=True, text=True, timeout=600)
    print(r.stdout[-4000:])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    tallies = re.findall(r"--- (\d+) passed, (\d+) failed ---", r.stdout)
    assert tallies == [("16", "0"), ("16", "0")], tallies


def test_reference_gpt_test_passes_on_hip_backend(tmp_path, dev):
    _run_gpt_test(BIN, tmp_path)


def test_reference_gpt_test_passes_with_every_op_on_the_gpu(tmp_path, dev):
    _run_gpt_test(BIN_FULL, tmp_path)
