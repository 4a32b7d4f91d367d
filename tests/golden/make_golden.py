"""Writes tests/golden/attention_small.npz: a small causal + window + softcap
+ bias + ALiBi + GQA attention case and its gradients computed with torch
float64 autograd (independent of oracle/attention.py).  Run once; the output
is committed."""

import math
import os

import numpy as np
import torch


def main():
    g = np.random.default_rng(7)
    q = g.standard_normal((1, 4, 9, 8))
    k = g.standard_normal((1, 2, 12, 8))
    v = g.standard_normal((1, 2, 12, 8))
    dout = g.standard_normal((1, 4, 9, 8))
    bias = g.standard_normal((1, 1, 9, 12))
    alibi = np.array([2.0 ** (-2 * (i + 1)) for i in range(4)])
    scale, softcap, left = 0.35, 6.0, 5
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    kk, vv = tk.repeat_interleave(2, 1), tv.repeat_interleave(2, 1)
    s = torch.einsum("bhid,bhjd->bhij", tq, kk) * scale
    s = softcap * torch.tanh(s / softcap) + torch.tensor(bias)
    qi = torch.arange(9)[:, None] + 3
    kj = torch.arange(12)[None, :]
    s = s - torch.tensor(alibi)[None, :, None, None] * (kj - qi).abs()
    keep = (kj <= qi) & (kj >= qi - left)
    s = s.masked_fill(~keep, float("-inf"))
    out = torch.softmax(s, -1) @ vv
    lse = torch.logsumexp(s, -1)
    (out * torch.tensor(dout)).sum().backward()
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "attention_small.npz")
    np.savez(path, q=q, k=k, v=v, dout=dout, bias=bias, alibi=alibi, scale=scale, softcap=softcap,
             out=out.detach().numpy(), lse=lse.detach().numpy(), dq=tq.grad.numpy(), dk=tk.grad.numpy(),
             dv=tv.grad.numpy())


if __name__ == "__main__":
    main()
