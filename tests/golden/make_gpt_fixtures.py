"""Writes the three fixture files the reference's gpt_test reads
(reference src/model/gpt_test.cpp:9-11):

  gpt_dummy_tokens.bin         65 int32 tokens (inputs = [0:64], labels = [1:65])
  gpt_dummy_weights.bin        102,592 fp32 weights in gpt_weights packing order
                               (reference src/model/gpt.cpp:40-96)
  gpt_dummy_ref_gradients.bin  102,592 fp32 gradients of the mean cross-entropy
                               loss w.r.t. those weights, same order

The reference produces these with its own PyTorch model (tools/prep_grad.py),
which is not imported here. This script restates the reference C++ model
(src/model/gpt.cpp:426-642 with the CPU ops of src/backend/cpu/cpu_backend.cpp)
in float64 torch from scratch: pre-LayerNorm GPT-2 blocks with in-place
residual adds, LayerNorm eps 1e-5 with the biased variance, tanh-GELU with the
reference's 0.79788456 constant, causal softmax attention with scale
1/sqrt(d), unembedding tied to wte over all padded rows, softmax / loss over
the first vocab_size logits, loss = mean over the B*T positions. Weights and
tokens come from gpt_amd.synth (splitmix64), not from torch's RNG, so the files
are reproducible byte for byte on any host.

Config = the gpt_test config (src/model/gpt_test.cpp:168-178): max_seq_len 64,
vocab 507 (padded 512), 4 layers, 4 heads, d_model 32, d_ffn 256, B=1, T=64.

Usage: python tests/golden/make_gpt_fixtures.py [out_dir]
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from gpt_amd import synth  # noqa: E402

S, V, VP, L, H, D, F = 64, 507, 512, 4, 4, 32, 256
SEED = 4242
# the gpt_test config as a mapping; the functions below take any such config
GPT_TEST = dict(S=S, V=V, VP=VP, L=L, H=H, D=D, F=F)
GELU_SQRT_2_OVER_PI = 0.79788456  # reference src/backend/cpu/cpu_backend.cpp:234
GELU_CUBIC = 0.044715

def layout(cfg):
    """(name, shape) in gpt_weights packing order."""
    S_, VP_, L_, D_, F_ = cfg["S"], cfg["VP"], cfg["L"], cfg["D"], cfg["F"]
    return [
        ("wte", (VP_, D_)), ("wpe", (S_, D_)),
        ("ln_1_w", (L_, D_)), ("ln_1_b", (L_, D_)),
        ("qkv_proj_w", (L_, D_, 3 * D_)), ("qkv_proj_b", (L_, 3 * D_)),
        ("attn_proj_w", (L_, D_, D_)), ("attn_proj_b", (L_, D_)),
        ("ln_2_w", (L_, D_)), ("ln_2_b", (L_, D_)),
        ("ffn_up_w", (L_, D_, F_)), ("ffn_up_b", (L_, F_)),
        ("ffn_down_w", (L_, F_, D_)), ("ffn_down_b", (L_, D_)),
        ("ln_f_w", (D_,)), ("ln_f_b", (D_,)),
    ]


LAYOUT = layout(GPT_TEST)
N_PARAMS = sum(int(np.prod(s)) for _, s in LAYOUT)


def make_weights(cfg=GPT_TEST, seed=SEED) -> np.ndarray:
    """N(0, 0.02) everywhere, LayerNorm gains 1 + N(0, 0.1), so that every
    parameter (biases included) carries a gradient path that depends on it."""
    lay = layout(cfg)
    n_params = sum(int(np.prod(s)) for _, s in lay)
    flat = synth.normal(seed, (n_params,), std=0.02)
    gains = synth.normal(seed + 1, (n_params,), std=0.1)
    off = 0
    for name, shape in lay:
        n = int(np.prod(shape))
        if name in ("ln_1_w", "ln_2_w", "ln_f_w"):
            flat[off:off + n] = (1.0 + gains[off:off + n]).astype(np.float32)
        off += n
    return flat


def make_tokens(cfg=GPT_TEST, n=S + 1, seed=SEED) -> np.ndarray:
    u = synth.uniform(seed + 2, n)
    return np.minimum((u * cfg["V"]).astype(np.int32), cfg["V"] - 1)


def unpack(flat, torch, cfg=GPT_TEST):
    out, off = {}, 0
    for name, shape in layout(cfg):
        n = int(np.prod(shape))
        out[name] = torch.tensor(flat[off:off + n].reshape(shape), dtype=torch.float64, requires_grad=True)
        off += n
    return out


def loss_fn(w, tokens, torch, cfg=GPT_TEST, B=1, T=S):
    """Mean cross-entropy over the B*T positions; inputs tokens[0:B*T] as B
    rows of T, labels tokens[1:B*T+1] (the reference's gpt_test shift)."""
    F_ = torch.nn.functional
    V_, L_, H_, D_ = cfg["V"], cfg["L"], cfg["H"], cfg["D"]
    inp = torch.tensor(tokens[:B * T], dtype=torch.long).reshape(B, T)
    lbl = torch.tensor(tokens[1:B * T + 1], dtype=torch.long)
    d = D_ // H_

    def ln(x, g, b):
        mean = x.mean(-1, keepdim=True)
        var = ((x - mean) ** 2).mean(-1, keepdim=True)
        return (x - mean) / torch.sqrt(var + 1e-5) * g + b

    def gelu(u):
        return 0.5 * u * (1.0 + torch.tanh(GELU_SQRT_2_OVER_PI * (u + GELU_CUBIC * u ** 3)))

    mask = torch.triu(torch.ones(T, T, dtype=torch.bool), 1)
    h = w["wte"][inp] + w["wpe"][:T]
    for l in range(L_):
        qkv = ln(h, w["ln_1_w"][l], w["ln_1_b"][l]) @ w["qkv_proj_w"][l] + w["qkv_proj_b"][l]
        q, k, v = (qkv[..., i * D_:(i + 1) * D_].reshape(B, T, H_, d).transpose(1, 2) for i in range(3))
        sc = (q @ k.transpose(-1, -2)) / np.sqrt(d)
        p = torch.softmax(sc.masked_fill(mask, float("-inf")), -1)
        att = (p @ v).transpose(1, 2).reshape(B, T, D_)
        h = h + att @ w["attn_proj_w"][l] + w["attn_proj_b"][l]
        u = ln(h, w["ln_2_w"][l], w["ln_2_b"][l]) @ w["ffn_up_w"][l] + w["ffn_up_b"][l]
        h = h + gelu(u) @ w["ffn_down_w"][l] + w["ffn_down_b"][l]
    logits = ln(h, w["ln_f_w"], w["ln_f_b"]) @ w["wte"].t()
    return F_.cross_entropy(logits[..., :V_].reshape(B * T, V_), lbl)


def gradients(flat: np.ndarray, tokens: np.ndarray, cfg=GPT_TEST, B=1, T=S, as_float64=False):
    import torch

    w = unpack(flat, torch, cfg)
    loss = loss_fn(w, tokens, torch, cfg, B, T)
    loss.backward()
    g = np.concatenate([w[name].grad.numpy().reshape(-1) for name, _ in layout(cfg)])
    return float(loss.detach()), (g if as_float64 else g.astype(np.float32))


def main(out_dir: str) -> None:
    os.makedirs(out_dir, exist_ok=True)
    flat, tokens = make_weights(), make_tokens()
    loss, grads = gradients(flat, tokens)
    tokens.astype(np.int32).tofile(os.path.join(out_dir, "gpt_dummy_tokens.bin"))
    flat.astype(np.float32).tofile(os.path.join(out_dir, "gpt_dummy_weights.bin"))
    grads.tofile(os.path.join(out_dir, "gpt_dummy_ref_gradients.bin"))
    print(f"loss {loss:.6f}; wrote {tokens.size} tokens, {flat.size} weights, {grads.size} gradients to {out_dir}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else os.path.join(os.path.dirname(os.path.abspath(__file__)), "gpt_test"))
