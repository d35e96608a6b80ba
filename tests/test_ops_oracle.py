"""Pins the CPU oracle of the GPT-2 ops around attention (oracle/ops_oracle.c)
before it is trusted as the checker of the HIP ops library. CPU only.

  * bit-exact agreement, op by op, with the reference's own CPUBackend
    methods compiled from /root/reference (oracle/_ref, cpu_backend.cpp:
    65-287, 439-557), on random inputs including ragged widths, repeated
    tokens, NULL residuals and the clipping threshold on both sides;
  * independent fp64 numpy restatements and closed forms (a dropped term, a
    wrong sign or a transposed weight fails these even where the oracle and
    the reference agree): matrix products against numpy, LayerNorm output
    statistics and its gradient against fp64 finite differences, softmax rows
    summing to 1, the loss of a uniform softmax = log V, the first AdamW step
    = lr * g / (|g| + eps), the clipped gradient norm = max_norm.
"""
import numpy as np
import pytest

from oracle import pyoracle, pyops

pytestmark = pytest.mark.skipif(not pyoracle.ref_available(), reason="oracle/_ref not built (needs /root/reference)")


def rng(seed):
    return np.random.default_rng(seed)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def both(fn, arrays, *args):
    """Run fn on the oracle and on the reference, each on its own copies of
    `arrays` (a dict of arrays the op reads or updates); return both dicts."""
    out = {}
    for impl in ("oracle", "ref"):
        a = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in arrays.items()}
        fn(a, impl)
        out[impl] = a
    return out["oracle"], out["ref"]


SHAPES = [(2, 5, 12), (1, 7, 30), (3, 4, 64)]  # B, T, C (C = 30: not a multiple of 4)


@pytest.mark.parametrize("B,T,C", SHAPES)
def test_embedding_matches_reference(B, T, C):
    r = rng(1)
    V = 11
    tok = r.integers(0, V, size=B * T).astype(np.int32)
    tok[: min(4, B * T)] = 3  # repeated token
    a = dict(y=np.zeros((B, T, C), np.float32), wte=f32(r.standard_normal((V, C))), wpe=f32(r.standard_normal((T, C))),
             gwte=f32(r.standard_normal((V, C))), gwpe=f32(r.standard_normal((T, C))),
             gy=f32(r.standard_normal((B, T, C))))

    def run(d, impl):
        pyops.embedding_forward(d["y"], d["wte"], d["wpe"], tok, B, T, C, impl)
        pyops.embedding_backward(d["gwte"], d["gwpe"], d["gy"], tok, B, T, C, impl)

    o, f = both(run, a)
    for k in ("y", "gwte", "gwpe"):
        assert same_bits(o[k], f[k]), k
    np.testing.assert_array_equal(o["y"], a["wte"][tok].reshape(B, T, C) + a["wpe"][None])
    gw = a["gwte"].astype(np.float64)
    np.add.at(gw, tok, a["gy"].reshape(B * T, C).astype(np.float64))
    np.testing.assert_allclose(o["gwte"], gw, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(o["gwpe"], a["gwpe"] + a["gy"].astype(np.float64).sum(0), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("B,T,C", SHAPES)
def test_unembedding_matches_reference(B, T, C):
    r = rng(2)
    Vp = 24
    a = dict(y=np.zeros((B, T, Vp), np.float32), x=f32(r.standard_normal((B, T, C))),
             wte=f32(r.standard_normal((Vp, C))), gx=np.zeros((B, T, C), np.float32),
             gwte=f32(r.standard_normal((Vp, C))), gy=f32(r.standard_normal((B, T, Vp))))

    def run(d, impl):
        pyops.unembedding_forward(d["y"], d["x"], d["wte"], B, T, C, Vp, impl)
        pyops.unembedding_backward(d["gx"], d["gwte"], d["gy"], d["x"], d["wte"], B, T, C, Vp, impl)

    o, f = both(run, a)
    for k in ("y", "gx", "gwte"):
        assert same_bits(o[k], f[k]), k
    x64, w64, g64 = (a[k].astype(np.float64) for k in ("x", "wte", "gy"))
    np.testing.assert_allclose(o["y"], x64 @ w64.T, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(o["gx"], g64 @ w64, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(o["gwte"], a["gwte"] + g64.reshape(-1, Vp).T @ x64.reshape(-1, C), rtol=1e-5,
                               atol=1e-4)


@pytest.mark.parametrize("B,T,C", SHAPES)
@pytest.mark.parametrize("with_res", [True, False])
def test_layernorm_matches_reference(B, T, C, with_res):
    r = rng(3)
    a = dict(y=np.zeros((B, T, C), np.float32), m=np.zeros((B, T), np.float32), v=np.zeros((B, T), np.float32),
             x=f32(r.standard_normal((B, T, C)) * 2 + 0.5), res=f32(r.standard_normal((B, T, C))) if with_res else None,
             g=f32(1 + 0.1 * r.standard_normal(C)), b=f32(0.1 * r.standard_normal(C)),
             gx=np.zeros((B, T, C), np.float32), gg=f32(r.standard_normal(C)), gb=f32(r.standard_normal(C)),
             gy=f32(r.standard_normal((B, T, C))), gres=f32(r.standard_normal((B, T, C))) if with_res else None)

    def run(d, impl):
        pyops.layernorm_forward(d["y"], d["m"], d["v"], d["x"], d["res"], d["g"], d["b"], B, T, C, impl)
        pyops.layernorm_backward(d["gx"], d["gg"], d["gb"], d["gy"], d["gres"], d["x"], d["m"], d["v"], d["g"], B, T,
                                 C, impl)

    o, f = both(run, a)
    for k in ("y", "m", "v", "x", "gx", "gg", "gb"):
        assert same_bits(o[k], f[k]), k
    # fp64 restatement of the forward, and of the backward by finite differences
    x = a["x"].astype(np.float64) + (a["res"] if with_res else 0)
    np.testing.assert_allclose(o["x"], x, rtol=1e-6)
    mu, var = x.mean(-1), x.var(-1)
    np.testing.assert_allclose(o["m"], mu, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(o["v"], var, rtol=1e-5)
    g, bb = a["g"].astype(np.float64), a["b"].astype(np.float64)

    def ln(z):
        m_, v_ = z.mean(-1, keepdims=True), z.var(-1, keepdims=True)
        return (z - m_) / np.sqrt(v_ + 1e-5) * g + bb

    np.testing.assert_allclose(o["y"], ln(x), rtol=1e-5, atol=1e-5)
    gy = a["gy"].astype(np.float64)
    h = 1e-6
    num = np.zeros_like(x)
    it = np.nditer(x[:1, :2], flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        xp, xm = x.copy(), x.copy()
        xp[i] += h
        xm[i] -= h
        num[i] = ((ln(xp) - ln(xm)) * gy).sum() / (2 * h)
    exp = num[:1, :2] + (a["gres"][:1, :2] if with_res else 0)
    np.testing.assert_allclose(o["gx"][:1, :2], exp, rtol=1e-3, atol=1e-4)
    xh = (x - mu[..., None]) / np.sqrt(var[..., None] + 1e-5)
    np.testing.assert_allclose(o["gg"], a["gg"] + (gy * xh).sum((0, 1)), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(o["gb"], a["gb"] + gy.sum((0, 1)), rtol=1e-5, atol=1e-5)


def gelu64(s):
    return 0.5 * s * (1 + np.tanh(np.sqrt(2 / np.pi) * (s + 0.044715 * s ** 3)))


@pytest.mark.parametrize("B,T,n_in,n_out", [(2, 3, 12, 20), (1, 5, 7, 9)])
@pytest.mark.parametrize("activation", [False, True])
def test_linear_matches_reference(B, T, n_in, n_out, activation):
    r = rng(4)
    a = dict(y=np.zeros((B, T, n_out), np.float32), act=np.zeros((B, T, n_out), np.float32),
             x=f32(r.standard_normal((B, T, n_in))), w=f32(r.standard_normal((n_in, n_out)) * 0.3),
             b=f32(r.standard_normal(n_out)), gx=np.zeros((B, T, n_in), np.float32),
             gw=f32(r.standard_normal((n_in, n_out))), gb=f32(r.standard_normal(n_out)),
             gy=f32(r.standard_normal((B, T, n_out))), ga=np.zeros((B, T, n_out), np.float32))

    def run(d, impl):
        pyops.linear_forward(d["y"], d["act"], d["x"], d["w"], d["b"], activation, B, T, n_in, n_out, impl)
        pyops.linear_backward(d["gx"], d["gw"], d["gb"], d["gy"], d["x"], d["w"], B, T, n_in, n_out, impl)
        pyops.activation_backward(d["ga"], d["gy"], d["y"], B, T, n_out, impl)

    o, f = both(run, a)
    for k in ("y", "act", "gx", "gw", "gb", "ga"):
        assert same_bits(o[k], f[k]), k
    x, w, gy = (a[k].astype(np.float64) for k in ("x", "w", "gy"))
    y = x @ w + a["b"]
    np.testing.assert_allclose(o["y"], y, rtol=1e-5, atol=1e-5)
    if activation:
        np.testing.assert_allclose(o["act"], gelu64(y), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(o["gx"], gy @ w.T, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(o["gw"], a["gw"] + x.reshape(-1, n_in).T @ gy.reshape(-1, n_out), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(o["gb"], a["gb"] + gy.sum((0, 1)), rtol=1e-5, atol=1e-5)
    hh = 1e-6
    yy = o["y"].astype(np.float64)
    np.testing.assert_allclose(o["ga"], gy * (gelu64(yy + hh) - gelu64(yy - hh)) / (2 * hh), rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("B,T,V,Vp", [(2, 3, 17, 20), (1, 4, 50, 64)])
def test_softmax_and_cross_entropy_match_reference(B, T, V, Vp):
    r = rng(5)
    x = f32(r.standard_normal((B, T, Vp)) * 3)
    labels = r.integers(0, V, size=B * T).astype(np.int32)
    a = dict(y=np.full((B, T, Vp), 7.0, np.float32), x=x, gx=np.full((B, T, Vp), 5.0, np.float32))
    res = {}

    def run(d, impl):
        pyops.softmax_forward(d["y"], d["x"], B, T, V, Vp, impl)
        pyops.ce_backward(d["gx"], d["y"], labels, B, T, V, Vp, impl)
        res[impl] = pyops.ce_loss(d["y"], labels, B, T, Vp, impl)

    o, f = both(run, a)
    for k in ("y", "gx"):
        assert same_bits(o[k], f[k]), k
    assert np.float32(res["oracle"]).view(np.uint32) == np.float32(res["ref"]).view(np.uint32)
    x64 = x[..., :V].astype(np.float64)
    p = np.exp(x64 - x64.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(o["y"][..., :V], p, rtol=1e-5, atol=1e-7)
    assert np.all(o["y"][..., V:] == 0)
    np.testing.assert_allclose(o["y"][..., :V].sum(-1), 1.0, rtol=1e-5)
    oh = np.zeros_like(p).reshape(-1, V)
    oh[np.arange(B * T), labels] = 1
    np.testing.assert_allclose(o["gx"][..., :V], (p - oh.reshape(p.shape)) / (B * T), rtol=1e-5, atol=1e-7)
    assert np.all(o["gx"][..., V:] == 5.0)  # padding columns untouched
    np.testing.assert_allclose(res["oracle"], -np.log(p.reshape(-1, V)[np.arange(B * T), labels] + 1e-8).mean(),
                               rtol=1e-5)
    # uniform softmax: loss = log V
    yu = np.zeros((B, T, Vp), np.float32)
    pyops.softmax_forward(yu, np.zeros((B, T, Vp), np.float32), B, T, V, Vp, "oracle")
    np.testing.assert_allclose(pyops.ce_loss(yu, labels, B, T, Vp, "oracle"), np.log(V), rtol=1e-5)


@pytest.mark.parametrize("step,wd", [(1, 0.0), (3, 0.1)])
def test_adamw_matches_reference(step, wd):
    r = rng(6)
    n = 37
    a = dict(p=f32(r.standard_normal(n)), g=f32(r.standard_normal(n)), m=f32(0.1 * r.standard_normal(n) * (step > 1)),
             v=f32(np.abs(0.1 * r.standard_normal(n)) * (step > 1)))
    lr, b1, b2, eps = 3e-4, 0.9, 0.95, 1e-8

    def run(d, impl):
        pyops.adamw(d["p"], d["g"], d["m"], d["v"], n, lr, b1, b2, eps, wd, step, impl)

    o, f = both(run, a)
    for k in ("p", "m", "v"):
        assert same_bits(o[k], f[k]), k
    if step == 1:  # m_hat = g, v_hat = g^2
        g = a["g"].astype(np.float64)
        np.testing.assert_allclose(o["p"], a["p"] - lr * g / (np.abs(g) + eps), rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("max_norm", [1e9, 0.5])
@pytest.mark.parametrize("accum", [1, 4])
def test_scale_clip_matches_reference(max_norm, accum):
    r = rng(7)
    n = 101
    a = dict(g=f32(r.standard_normal(n)))

    def run(d, impl):
        pyops.scale_clip(d["g"], n, max_norm, accum, impl)

    o, f = both(run, a)
    assert same_bits(o["g"], f["g"])
    s = a["g"].astype(np.float64) / accum
    if np.linalg.norm(s) > max_norm:
        np.testing.assert_allclose(np.linalg.norm(o["g"].astype(np.float64)), max_norm, rtol=1e-5)
    else:
        np.testing.assert_array_equal(o["g"], (a["g"] / np.float32(accum)).astype(np.float32))
