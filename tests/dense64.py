"""Dense float64 restatement of causal attention, forward and backward (test
infrastructure only).

Independent of the C oracle: a masked softmax over the whole [T, T] score
matrix per (b, h), in float64. Two backends with the same formulas:
  * numpy (CPU), pinned to the oracle and to the reference CPU backend by
    tests/test_oracle.py;
  * torch float64 on any device, pinned to the numpy one by
    tests/test_oracle.py::test_dense64_torch_matches_numpy, and used by the
    GPU tests to compare whole configurations (every (b, h)) in float64 on
    the device, a chunk of (b, h) at a time.
Layouts are the reference's (src/backend/backend_interface.h:161-184):
qkv [B, T, 3C], y [B, T, C], lse / D [B, T, H], grad_x [B, T, 3C].
"""
import numpy as np


def forward_np(qkv, H):
    """(y [B,T,C], lse [B,T,H]) in float64."""
    B, T, W = qkv.shape
    C = W // 3
    d = C // H
    x = qkv.astype(np.float64).reshape(B, T, 3, H, d).transpose(2, 0, 3, 1, 4)  # 3,B,H,T,d
    q, k, v = x
    s = q @ k.transpose(0, 1, 3, 2) / np.sqrt(d)
    mask = np.triu(np.ones((T, T), bool), 1)
    s = np.where(mask, -np.inf, s)
    m = s.max(-1, keepdims=True)
    p = np.exp(s - m)
    z = p.sum(-1, keepdims=True)
    o = (p / z) @ v
    lse = (m + np.log(z))[..., 0]  # B,H,T
    return o.transpose(0, 2, 1, 3).reshape(B, T, C), lse.transpose(0, 2, 1)


def backward_np(qkv, dy, H):
    """(grad_x [B,T,3C], D [B,T,H]) in float64, from the float64 forward."""
    B, T, W = qkv.shape
    C = W // 3
    d = C // H
    x = qkv.astype(np.float64).reshape(B, T, 3, H, d).transpose(2, 0, 3, 1, 4)
    q, k, v = x
    do = dy.astype(np.float64).reshape(B, T, H, d).transpose(0, 2, 1, 3)
    s = q @ k.transpose(0, 1, 3, 2) / np.sqrt(d)
    s = np.where(np.triu(np.ones((T, T), bool), 1), -np.inf, s)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    o = p @ v
    dv = p.transpose(0, 1, 3, 2) @ do
    dp = do @ v.transpose(0, 1, 3, 2)
    Dr = (do * o).sum(-1, keepdims=True)
    ds = p * (dp - Dr) / np.sqrt(d)
    dq = ds @ k
    dk = ds.transpose(0, 1, 3, 2) @ q
    g = np.stack([dq, dk, dv])  # 3,B,H,T,d
    return g.transpose(1, 3, 0, 2, 4).reshape(B, T, 3 * C), Dr[..., 0].transpose(0, 2, 1)


def _heads(t, B, T, n, H, d):
    """[B, T, n*H*d] -> [n, B*H, T, d] (contiguous)."""
    import torch

    return t.reshape(B, T, n, H, d).permute(2, 0, 3, 1, 4).reshape(n, B * H, T, d).contiguous()


def fwd_bwd_torch(qkv, dy, H, chunk=48):
    """Forward and backward in float64 with torch, on qkv's device; qkv
    [B,T,3C] and dy [B,T,C] are torch tensors (any float dtype). Returns
    (y, lse, grad_x, D) as float64 tensors in the reference layouts. The (b, h)
    pairs are processed `chunk` at a time ([chunk, T, T] score matrices)."""
    import torch

    B, T, W = qkv.shape
    C = W // 3
    d = C // H
    x = _heads(qkv.to(torch.float64), B, T, 3, H, d)  # 3, BH, T, d
    do_all = _heads(dy.to(torch.float64), B, T, 1, H, d)[0]
    mask = torch.triu(torch.ones(T, T, dtype=torch.bool, device=qkv.device), 1)
    scale = 1.0 / np.sqrt(d)
    o_all = torch.empty(B * H, T, d, dtype=torch.float64, device=qkv.device)
    lse_all = torch.empty(B * H, T, dtype=torch.float64, device=qkv.device)
    g_all = torch.empty(3, B * H, T, d, dtype=torch.float64, device=qkv.device)
    D_all = torch.empty(B * H, T, dtype=torch.float64, device=qkv.device)
    for c0 in range(0, B * H, chunk):
        sl = slice(c0, min(c0 + chunk, B * H))
        q, k, v, do = x[0, sl], x[1, sl], x[2, sl], do_all[sl]
        kt = k.transpose(1, 2).contiguous()
        s = torch.matmul(q, kt) * scale
        s = s.masked_fill(mask, float("-inf"))
        m = s.amax(-1, keepdim=True)
        p = torch.exp(s - m)
        z = p.sum(-1, keepdim=True)
        p = p / z
        o = torch.matmul(p, v)
        o_all[sl] = o
        lse_all[sl] = (m + torch.log(z))[..., 0]
        pt = p.transpose(1, 2).contiguous()
        vt = v.transpose(1, 2).contiguous()
        dv = torch.matmul(pt, do)
        dp = torch.matmul(do, vt)
        Dr = (do * o).sum(-1, keepdim=True)
        ds = p * (dp - Dr) * scale
        dst = ds.transpose(1, 2).contiguous()
        g_all[0, sl] = torch.matmul(ds, k)
        g_all[1, sl] = torch.matmul(dst, q)
        g_all[2, sl] = dv
        D_all[sl] = Dr[..., 0]
    y = o_all.reshape(B, H, T, d).permute(0, 2, 1, 3).reshape(B, T, C)
    lse = lse_all.reshape(B, H, T).permute(0, 2, 1)
    gx = g_all.reshape(3, B, H, T, d).permute(1, 3, 0, 2, 4).reshape(B, T, 3 * C)
    D = D_all.reshape(B, H, T).permute(0, 2, 1)
    return y, lse, gx, D
