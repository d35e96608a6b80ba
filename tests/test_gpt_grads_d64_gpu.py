"""Whole-model weight gradients at head_dim 64, through the reference's own
GPT model (src/model/gpt.cpp forward and backward, unchanged), with the
attention on the hot path's MFMA kernels.

The reference's gpt_test (tests/test_gpt_test_gpu.py) checks the 16 weight
gradients at head_dim 8, which takes the general-d kernels. Here
oracle/_ref/gpt_grad_check runs the same model sequence as gpt_test
(src/model/gpt_test.cpp:148-164) at d_model 768, 12 heads, 2 layers, d_ffn
3072, vocab 1024, B = 2, T = 256 on HipAttnBackend (attention through
libgpt_hip_attn.so, every other op the reference CPU backend's) and on
HipBackend (every op on the GPU). Its gradients are compared per tensor, in
gpt_weights order:

* with the float64 restatement of the model (tests/golden/make_gpt_fixtures.py):
  max|g - g64| / max|g64| must stay within 4 times the reference CPU backend's
  own fp32 error at this size (recorded in tests/golden/gpt_d64/meta.json by
  tests/golden/make_gpt_d64_fixture.py: 0.9e-6 to 2.7e-6), i.e. the GPU model
  is as accurate as the reference's own;
* with the reference CPU backend's gradients at 2048 sampled entries per
  tensor (tests/golden/gpt_d64/cpu_sample.bin), as gpt_test compares CPU and
  GPU: |g_gpu - g_cpu| <= 1e-5 (gpt_test.cpp:12).
"""
import json
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden", "gpt_d64")
GPT_TEST_EPS = 1e-5
FP32_ERR_FACTOR = 4.0

pytestmark = pytest.mark.gpu


def test_weight_gradients_at_head_dim_64(tmp_path):
    from tests.golden import make_gpt_d64_fixture as fxd
    from tests.golden import make_gpt_fixtures as fx

    if not os.path.exists(fxd.DRIVER):
        pytest.skip(f"{fxd.DRIVER} not built (needs /root/reference at build time)")
    meta = json.load(open(os.path.join(GOLD, "meta.json")))
    assert meta["config"] == fxd.CONFIG and (meta["B"], meta["T"], meta["seed"]) == (fxd.B, fxd.T, fxd.SEED)
    w, t = fxd.inputs()
    tp, wp = str(tmp_path / "tokens.bin"), str(tmp_path / "weights.bin")
    t.astype(np.int32).tofile(tp)
    w.astype(np.float32).tofile(wp)
    r = subprocess.run(fxd.driver_args("gpu", tp, wp, str(tmp_path) + "/"), capture_output=True, text=True,
                       timeout=600)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stderr[-2000:]
    losses = {m.group(1): float(m.group(2)) for m in re.finditer(r"^(attn|full) loss (\S+)", r.stdout, re.M)}
    loss64, g64 = fx.gradients(w, t, fxd.CONFIG, fxd.B, fxd.T, as_float64=True)
    print(f"loss: fp64 {loss64:.7f}, reference CPU {meta['cpu_loss']:.7f}, "
          + ", ".join(f"{k} {v:.7f}" for k, v in losses.items()), flush=True)
    for v in losses.values():
        assert abs(v - loss64) <= 4 * max(abs(meta["cpu_loss"] - loss64), 1e-6)

    cpu_sample = np.fromfile(os.path.join(GOLD, "cpu_sample.bin"), dtype=np.float32)
    bad = []
    for backend in ("attn", "full"):
        g = np.fromfile(str(tmp_path / f"{backend}.bin"), dtype=np.float32)
        assert g.size == g64.size
        off = soff = 0
        for (name, shape), rec in zip(fx.layout(fxd.CONFIG), meta["tensors"]):
            n = int(np.prod(shape))
            assert rec["name"] == name and rec["size"] == n
            gg, rr = g[off:off + n].astype(np.float64), g64[off:off + n]
            rel = float(np.abs(gg - rr).max() / np.abs(rr).max())
            idx = fxd.sample_indices(n)
            cs = cpu_sample[soff:soff + idx.size]
            dcpu = float(np.abs(g[off:off + n][idx] - cs).max())
            limit = FP32_ERR_FACTOR * rec["cpu_rel_err"]
            ok = rel <= limit and dcpu <= GPT_TEST_EPS and np.isfinite(gg).all()
            print(f"[{'PASS' if ok else 'FAIL'}] {backend:4s} {name:12s} rel err vs fp64 {rel:.2e} "
                  f"(reference CPU {rec['cpu_rel_err']:.2e}, limit {limit:.2e}), "
                  f"max|gpu - cpu| on {idx.size} entries {dcpu:.2e}", flush=True)
            if not ok:
                bad.append((backend, name))
            off += n
            soff += idx.size
    assert not bad, bad
