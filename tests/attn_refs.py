"""Torch fp32/fp64 attention references shared by the GPU tests.

The references keep the input dtype for the matmuls and run the softmax in
fp32: passed fp32 inputs they are the exact answer, passed fp16/bf16 inputs
they are the "naive" same-precision baseline that the error-ratio checks
(kernel error <= 2 x naive error + slack) compare against.
"""

import math

import torch


def keep_mask(sq, sk, causal, window, device):
    left, right = window
    i = torch.arange(sq, device=device)[:, None] + (sk - sq)
    j = torch.arange(sk, device=device)[None, :]
    keep = torch.ones(sq, sk, dtype=torch.bool, device=device)
    if causal:
        keep &= j <= i
    if left >= 0:
        keep &= j >= i - left
    if right >= 0:
        keep &= j <= i + right
    return keep


def attention(query, key, value, causal=False, scale=None, window=(-1, -1), softcap=0.0,
              bias=None, alibi=None):
    """(B,H,S,D) reference with GQA, bottom-right causal, window, softcap,
    bias and ALiBi; rows with no visible key produce zeros."""
    group = query.shape[1] // key.shape[1]
    if group > 1:
        key = key.repeat_interleave(group, dim=1)
        value = value.repeat_interleave(group, dim=1)
    scale = 1.0 / math.sqrt(query.shape[-1]) if scale is None else scale
    acc = torch.promote_types(query.dtype, torch.float32)  # fp32 softmax, fp64 kept for CPU pins
    logits = (torch.matmul(query, key.transpose(-1, -2)) * scale).to(acc)
    sq, sk = logits.shape[-2:]
    if softcap > 0:
        logits = softcap * torch.tanh(logits / softcap)
    if bias is not None:
        logits = logits + bias.to(acc)
    if alibi is not None:
        i = torch.arange(sq, device=logits.device)[:, None]
        j = torch.arange(sk, device=logits.device)[None, :]
        logits = logits - alibi.to(acc).view(1, -1, 1, 1) * (j - i - (sk - sq)).abs().to(acc)
    keep = keep_mask(sq, sk, causal, window, logits.device)
    logits = logits.masked_fill(~keep, float("-inf"))
    valid = torch.isfinite(logits).any(dim=-1, keepdim=True)
    logits = torch.where(valid, logits, torch.zeros_like(logits))
    probs = torch.where(valid, torch.softmax(logits, dim=-1), 0.0)
    return torch.matmul(probs.to(value.dtype), value)


def varlen_attention(query, key, value, lengths_q, lengths_k, **kw):
    """Packed (T,H,D) reference: dense attention per sequence."""
    outs, qs, ks = [], 0, 0
    for lq, lk in zip(lengths_q, lengths_k):
        q = query[qs:qs + lq].transpose(0, 1)[None]
        k = key[ks:ks + lk].transpose(0, 1)[None]
        v = value[ks:ks + lk].transpose(0, 1)[None]
        outs.append(attention(q, k, v, **kw)[0].transpose(0, 1))
        qs += lq
        ks += lk
    return torch.cat(outs, dim=0)


def grads(fn, query, key, value, dout):
    q = query.detach().clone().requires_grad_(True)
    k = key.detach().clone().requires_grad_(True)
    v = value.detach().clone().requires_grad_(True)
    fn(q, k, v).backward(dout)
    return q.grad, k.grad, v.grad


def max_err(a, b):
    return (a.float() - b.float()).abs().max().item()


def assert_ratio(kernel, naive, exact, slack=1e-3, name=""):
    """Kernel error must stay within twice the same-precision naive error."""
    ke, ne = max_err(kernel, exact), max_err(naive, exact)
    assert ke <= 2.0 * ne + slack, f"{name}: kernel_err={ke:.3e} naive_err={ne:.3e}"


def check_grads(fn_kernel, fn_ref, q, k, v, dout, slack=1e-3):
    kernel = grads(fn_kernel, q, k, v, dout)
    exact = grads(fn_ref, q.float(), k.float(), v.float(), dout.float())
    naive = grads(fn_ref, q, k, v, dout)
    for kg, ng, eg, name in zip(kernel, naive, exact, ("dq", "dk", "dv")):
        assert kg.shape == eg.shape
        assert_ratio(kg, ng, eg, slack, name)


def cu_seqlens(lengths, device="cuda"):
    vals = [0]
    for n in lengths:
        vals.append(vals[-1] + n)
    return torch.tensor(vals, dtype=torch.int32, device=device)
