"""The reference's own generation program (src/infer/infer.cpp with its data
manager, token sampler and GPT model, compiled unchanged into
oracle/_ref/infer_full) on the all-GPU HipBackend: GPT-2 124M from a
checkpoint file in the reference's format (16 tensors of raw fp32 in
gpt_weights order, gpt.cpp:38-84, 327-397), a uint16 prompt, 48 sampled
tokens; every step re-runs the causal forward over the whole prefix (no KV
cache, infer.cpp:117-124), so the prefix grows through T = 33..80 at B = 1 and
takes the split-key small-call attention kernel. The output file must hold the
prompt followed by 48 valid token ids; the timings the program prints are
reported."""
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "oracle", "_ref", "infer_full")
N_PARAMS = (50304 * 768 + 256 * 768 + 12 * (2 * 768 + 768 * 2304 + 2304 + 768 * 768 + 768 + 2 * 768
                                          + 2 * 768 * 3072 + 3072 + 768) + 2 * 768)

pytestmark = pytest.mark.gpu


def test_reference_generator_runs_gpt2_124m_on_the_gpu(tmp_path, dev):
    if not os.path.exists(BIN):
        pytest.skip("oracle/_ref/infer_full not built (needs /root/reference at build time)")
    rng = np.random.default_rng(11)
    ckpt = tmp_path / "model.bin"
    w = (rng.standard_normal(N_PARAMS, dtype=np.float32) * 0.02).astype(np.float32)
    w.tofile(ckpt)
    del w
    prompt = rng.integers(0, 50257, size=32).astype(np.uint16)
    prompt.tofile(tmp_path / "prompt.bin")
    n_new = 48
    r = subprocess.run([BIN, "--model", str(ckpt), "--input", str(tmp_path / "prompt.bin"), "--output",
                        str(tmp_path / "out.bin"), "--max-tokens", str(n_new), "--seed", "3"],
                       cwd=tmp_path, capture_output=True, text=True, timeout=600)
    print(r.stdout[-1500:])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    out = np.fromfile(tmp_path / "out.bin", dtype=np.uint16)
    assert out.size == prompt.size + n_new
    np.testing.assert_array_equal(out[:prompt.size], prompt)
    assert np.all(out < 50257)
    fwd = re.search(r"Average forward pass time: ([0-9.]+) ms", r.stdout)
    assert fwd, r.stdout[-1000:]
    # the program's own per-step scopes (infer.cpp:116-124): Preparation is
    # gpt.set_size (every activation freed and allocated again for the new
    # prefix length), ForwardPass the forward plus the copy of the last row of
    # logits; the averages cover every step, the 5 warm-up steps included
    prep = [float(v) for v in re.findall(r"Preparation took ([0-9.]+) ms", r.stdout)]
    fp = [float(v) for v in re.findall(r"ForwardPass took ([0-9.]+) ms", r.stdout)]
    assert prep and fp and len(prep) == len(fp)
    print(f"GPT-2 124M generation, prefix 33..80: average forward pass {float(fwd.group(1)):.2f} ms; "
          f"per step (all {len(fp)} steps): Preparation {np.mean(prep):.3f} ms (median {np.median(prep):.3f}), "
          f"ForwardPass {np.mean(fp):.3f} ms (median {np.median(fp):.3f})")
