"""Writes tests/golden/gpt_d64/: what the head_dim-64 gradient check
(tests/test_gpt_grads_d64_gpu.py) needs from the reference CPU backend, which
takes about two minutes at this size and so is run here once, not on the GPU
box.

Config: the reference GPT model (src/model/gpt.cpp, unchanged) with d_model
768, 12 heads (head_dim 64, the hot path's MFMA kernels), 2 layers, d_ffn
3072, vocab 1024, B = 2, T = 256 (max_seq_len 256). Weights and tokens come
from tests/golden/make_gpt_fixtures.py (splitmix64, seed SEED), so the test
regenerates them byte for byte.

Steps: oracle/_ref/gpt_grad_check cpu runs the reference model on its own
CPUBackend (zero_grad, forward, backward, loss, as gpt_test does); the float64
restatement make_gpt_fixtures.gradients gives the exact gradients. Written:

  meta.json       config, seed, both losses, and per weight tensor (gpt_weights
                  packing order): size, max |g64|, and the reference CPU
                  backend's own fp32 error max|g_cpu - g64|, absolute and
                  relative to max|g64| (the scale of error the check allows)
  cpu_sample.bin  float32 CPU-backend gradients at SAMPLE indices per tensor
                  (numpy default_rng(SEED), sorted), for gpt_test-style
                  CPU-vs-GPU comparisons

Usage: python tests/golden/make_gpt_d64_fixture.py   (needs oracle/_ref built)
"""
import json
import os
import re
import subprocess
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from tests.golden import make_gpt_fixtures as fx  # noqa: E402

CONFIG = dict(S=256, V=1024, VP=1024, L=2, H=12, D=768, F=3072)
B, T = 2, 256
SEED = 6464
SAMPLE = 2048
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gpt_d64")
DRIVER = os.path.join(ROOT, "oracle", "_ref", "gpt_grad_check")


def inputs():
    return fx.make_weights(CONFIG, seed=SEED), fx.make_tokens(CONFIG, n=B * T + 1, seed=SEED)


def driver_args(mode, tokens_path, weights_path, prefix):
    c = CONFIG
    return [DRIVER, mode, str(c["V"]), str(c["VP"]), str(c["L"]), str(c["H"]), str(c["D"]), str(c["F"]),
            str(c["S"]), str(B), str(T), tokens_path, weights_path, prefix]


def sample_indices(size):
    rng = np.random.default_rng(SEED)
    k = min(SAMPLE, size)
    return np.sort(rng.choice(size, size=k, replace=False))


def tensors(flat):
    off = 0
    for name, shape in fx.layout(CONFIG):
        n = int(np.prod(shape))
        yield name, flat[off:off + n]
        off += n


def main():
    w, t = inputs()
    with tempfile.TemporaryDirectory() as d:
        tp, wp = os.path.join(d, "tokens.bin"), os.path.join(d, "weights.bin")
        t.astype(np.int32).tofile(tp)
        w.astype(np.float32).tofile(wp)
        r = subprocess.run(driver_args("cpu", tp, wp, os.path.join(d, "")), capture_output=True, text=True,
                           check=True)
        cpu_loss = float(re.search(r"^cpu loss (\S+)", r.stdout, re.M).group(1))
        cpu = np.fromfile(os.path.join(d, "cpu.bin"), dtype=np.float32)
    loss64, g64 = fx.gradients(w, t, CONFIG, B, T, as_float64=True)
    assert cpu.size == g64.size
    meta = {"config": CONFIG, "B": B, "T": T, "seed": SEED, "sample": SAMPLE,
            "cpu_loss": cpu_loss, "fp64_loss": loss64, "tensors": []}
    samples = []
    for (name, gc), (_, gr) in zip(tensors(cpu.astype(np.float64)), tensors(g64)):
        scale = float(np.abs(gr).max())
        diff = float(np.abs(gc - gr).max())
        meta["tensors"].append({"name": name, "size": int(gr.size), "max_abs_fp64": scale,
                                "cpu_max_abs_diff": diff, "cpu_rel_err": diff / scale if scale > 0 else 0.0})
        samples.append(gc[sample_indices(gr.size)].astype(np.float32))
    os.makedirs(OUT, exist_ok=True)
    np.concatenate(samples).tofile(os.path.join(OUT, "cpu_sample.bin"))
    with open(os.path.join(OUT, "meta.json"), "w") as f:
        json.dump(meta, f, indent=1)
    for e in meta["tensors"]:
        print(f"{e['name']:12s} size {e['size']:9d} max|g| {e['max_abs_fp64']:.3e} "
              f"cpu err {e['cpu_max_abs_diff']:.3e} ({e['cpu_rel_err']:.2e})")
    print(f"loss cpu {cpu_loss:.7f} fp64 {loss64:.7f}")


if __name__ == "__main__":
    main()
