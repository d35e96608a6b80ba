"""The gpt_test fixtures (tests/golden/gpt_test/) and the model they pin. CPU only.

* make_gpt_fixtures.py regenerates the committed files byte for byte.
* The reference GPT model on the reference CPU backend (oracle/_ref/
  gpt_cpu_grads, built from /root/reference/src/model/gpt.cpp and
  src/backend/cpu/cpu_backend.cpp) reproduces the committed gradients within
  gpt_test's own criterion, |a - b| <= 1e-5 (reference
  src/model/gpt_test.cpp:12, 27-41): the fixture's independent float64 torch
  restatement of the model and the reference model agree.
* A planted mistake in the restatement (GELU without its cubic term) breaks
  that agreement, so the comparison is sensitive to the model's math.
"""
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden", "gpt_test")
CPU_GRADS = os.path.join(ROOT, "oracle", "_ref", "gpt_cpu_grads")
FILES = ("gpt_dummy_tokens.bin", "gpt_dummy_weights.bin", "gpt_dummy_ref_gradients.bin")

sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
import make_gpt_fixtures as mk  # noqa: E402


def test_fixtures_regenerate_bytewise(tmp_path):
    mk.main(str(tmp_path))
    for f in FILES:
        assert open(os.path.join(GOLD, f), "rb").read() == open(tmp_path / f, "rb").read(), f


def test_fixture_sizes():
    assert os.path.getsize(os.path.join(GOLD, FILES[0])) == 65 * 4
    assert os.path.getsize(os.path.join(GOLD, FILES[1])) == mk.N_PARAMS * 4 == 102592 * 4
    assert os.path.getsize(os.path.join(GOLD, FILES[2])) == 102592 * 4


def _reference_cpu_grads(tmp_path, weights=None):
    if not os.path.exists(CPU_GRADS):
        pytest.skip("oracle/_ref/gpt_cpu_grads not built (needs /root/reference at build time)")
    wpath = os.path.join(GOLD, FILES[1])
    if weights is not None:
        wpath = str(tmp_path / "w.bin")
        weights.astype(np.float32).tofile(wpath)
    out = tmp_path / "g.bin"
    subprocess.run([CPU_GRADS, os.path.join(GOLD, FILES[0]), wpath, str(out)], check=True,
                   capture_output=True)
    return np.fromfile(out, np.float32)


def test_reference_cpu_model_matches_fixture_gradients(tmp_path):
    ref = np.fromfile(os.path.join(GOLD, FILES[2]), np.float32)
    cpu = _reference_cpu_grads(tmp_path)
    d = np.abs(cpu - ref)
    assert np.all(np.isfinite(cpu))
    assert d.max() <= 1e-5, d.max()
    assert np.abs(ref).max() > 1e-2  # the gradients are not trivially small


def test_planted_gelu_mistake_is_caught(tmp_path, monkeypatch):
    """A restatement that drops GELU's cubic term disagrees with the reference."""
    pytest.importorskip("torch")
    cpu = _reference_cpu_grads(tmp_path)
    monkeypatch.setattr(mk, "GELU_CUBIC", 0.0)
    _, g_bad = mk.gradients(mk.make_weights(), mk.make_tokens())
    assert np.abs(g_bad - cpu).max() > 1e-5


def test_d64_gradient_fixture_pins_the_restatement():
    """tests/golden/gpt_d64/meta.json (written by make_gpt_d64_fixture.py from
    the reference's own CPU backend and the float64 restatement at head_dim
    64) holds every tensor's CPU-vs-float64 error at fp32 round-off level: the
    restatement, which the head_dim-64 GPU check compares against, is the
    reference model at that config too."""
    import json

    meta = json.load(open(os.path.join(ROOT, "tests", "golden", "gpt_d64", "meta.json")))
    assert len(meta["tensors"]) == 16
    for rec in meta["tensors"]:
        assert 0 < rec["cpu_rel_err"] < 1e-5, rec
    assert abs(meta["cpu_loss"] - meta["fp64_loss"]) < 1e-4
    n = sum(r["size"] for r in meta["tensors"])
    assert os.path.getsize(os.path.join(ROOT, "tests", "golden", "gpt_d64", "cpu_sample.bin")) == 4 * sum(
        min(meta["sample"], r["size"]) for r in meta["tensors"])
    assert n == 15160320
