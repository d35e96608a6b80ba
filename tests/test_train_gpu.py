"""The reference's own trainer (src/train/train.cpp with its data loader, LR
schedule and GPT model, compiled unchanged into oracle/_ref/train_full) on the
all-GPU HipBackend: GPT-2 124M (12 layers, d_model 768, vocab 50257, context
256, reference train.cpp:63-70), batch 16, on a synthetic uint16 token file in
the reference's data format (data_loader.cpp:55-110). Every optimizer step's
loss must be finite and the loss must fall; the per-step times the trainer
prints (forward + backward + loss, host clock, train.cpp:121-126) are
reported."""
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "oracle", "_ref", "train_full")

pytestmark = pytest.mark.gpu


def token_file(path, n_tokens, seed=5):
    """A learnable stream: a fixed random 97-token phrase repeated, ids < 50257."""
    phrase = np.random.default_rng(seed).integers(0, 50257, size=97)
    np.resize(phrase, n_tokens).astype(np.uint16).tofile(path)


def test_reference_trainer_runs_gpt2_124m_on_the_gpu(tmp_path, dev):
    if not os.path.exists(BIN):
        pytest.skip("oracle/_ref/train_full not built (needs /root/reference at build time)")
    batch, steps, seq = 16, 12, 256
    data = tmp_path / "tokens.bin"
    token_file(data, (batch * steps + 2) * seq)
    out = tmp_path / "ckpt.bin"
    r = subprocess.run([BIN, "--epochs", "1", "--batch-size", str(batch), "--batch-accum-steps", "1",
                        "--output", str(out), "--data", str(data), "--seed", "7"],
                       cwd=tmp_path, capture_output=True, text=True, timeout=600)
    print(r.stdout[-3000:])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    rows = re.findall(r"Avg Loss: ([-+0-9.eEnaif]+)\s+\|\s+Avg Time: ([0-9.]+) ms", r.stdout)
    assert len(rows) >= steps - 1, rows
    loss = np.array([float(a) for a, _ in rows])
    ms = np.array([float(b) for _, b in rows])
    assert np.all(np.isfinite(loss)), loss
    assert 10.0 < loss[0] < 11.5  # ~ln(50257) at initialisation
    assert loss[-1] < loss[0] - 0.05, loss
    print(f"GPT-2 124M B={batch} T={seq}: loss {loss[0]:.4f} -> {loss[-1]:.4f}; "
          f"forward+backward+loss {np.median(ms[2:]):.2f} ms median (steps 3..{len(ms)})")
    assert os.path.getsize(out) == 4 * (50304 * 768 + 256 * 768 + 12 * (2 * 768 + 768 * 2304 + 2304 + 768 * 768
                                                                        + 768 + 2 * 768 + 2 * 768 * 3072 + 3072
                                                                        + 768) + 2 * 768)
