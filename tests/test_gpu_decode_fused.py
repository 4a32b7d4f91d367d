"""The split merge done inside the split launch (last-arriving workgroup,
zero-reset arrival counters) against the two-launch merge and the oracle.

The reference merges split partials with a second launch
(interface.py:458/:471 and :704/:720); both forms must give the same rows."""

import math

import numpy as np
import pytest
import torch

from fa_rdna3 import _native, flash_attention_decode, flash_attention_decode_paged
from oracle import attention as oracle

pytestmark = pytest.mark.gpu
DEVICE = "cuda"


def _both(fn):
    saved = _native.FUSED_SPLIT_MERGE
    try:
        _native.FUSED_SPLIT_MERGE = False
        two = fn()
        _native.FUSED_SPLIT_MERGE = True
        fused = fn()
    finally:
        _native.FUSED_SPLIT_MERGE = saved
    return fused, two


def _ulp_close(a, b):
    # The in-launch merge may split the keys differently (proportional
    # shares), so the two differ by rounding: about one unit in the last
    # place of the output type.
    rel = 2.0 ** -9 if a.dtype == torch.float16 else 2.0 ** -7
    bound = rel * b.float().abs().clamp_min(2.0 ** -4)
    assert torch.all((a.float() - b.float()).abs() <= bound), (a.float() - b.float()).abs().max().item()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("seqlen_q,head_dim", [(1, 128), (3, 64), (9, 32)])
def test_fused_merge_matches_two_launch_and_oracle(dtype, seqlen_q, head_dim):
    g = torch.Generator().manual_seed(seqlen_q * 100 + head_dim)
    q = torch.randn(3, 16, seqlen_q, head_dim, generator=g).to(dtype)
    k = torch.randn(3, 4, 5000, head_dim, generator=g).to(dtype)
    v = torch.randn(3, 4, 5000, head_dim, generator=g).to(dtype)
    lens = torch.tensor([4999, 0, 1234], dtype=torch.int32)
    dq, dk, dv, dl = (t.to(DEVICE) for t in (q, k, v, lens))
    with torch.no_grad():
        fused, two = _both(lambda: flash_attention_decode(dq, dk, dv, cache_seqlens=dl))
    _ulp_close(fused, two)
    ref = oracle.decode(q.float().numpy(), k.float().numpy(), v.float().numpy(), 1 / math.sqrt(head_dim),
                        lens.numpy())
    tol = 2e-3 if dtype == torch.float16 else 1e-2
    assert np.abs(fused.float().cpu().numpy() - ref).max() <= tol


def test_fused_merge_repeated_calls_and_changing_split_counts():
    # The counters are reset by each call's last workgroup: back-to-back calls
    # with different grids (split counts, batch sizes) on one stream reuse them.
    torch.manual_seed(5)
    outs = []
    for n, b in ((8192, 4), (700, 2), (16384, 1), (8192, 4)):
        q = torch.randn(b, 32, 1, 128, device=DEVICE, dtype=torch.float16)
        k = torch.randn(b, 8, n, 128, device=DEVICE, dtype=torch.float16)
        v = torch.randn_like(k)
        with torch.no_grad():
            fused, two = _both(lambda: flash_attention_decode(q, k, v))
            again = flash_attention_decode(q, k, v)
        _ulp_close(fused, two)
        torch.testing.assert_close(again, fused, atol=0, rtol=0)
        outs.append(fused)


def test_fused_merge_on_two_streams():
    torch.manual_seed(6)
    q = torch.randn(2, 32, 1, 128, device=DEVICE, dtype=torch.float16)
    k = torch.randn(2, 8, 9000, 128, device=DEVICE, dtype=torch.float16)
    v = torch.randn_like(k)
    with torch.no_grad():
        ref = flash_attention_decode(q, k, v)
        s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
        torch.cuda.synchronize()
        with torch.cuda.stream(s1):
            a = [flash_attention_decode(q, k, v) for _ in range(4)]
        with torch.cuda.stream(s2):
            b = [flash_attention_decode(q, k, v) for _ in range(4)]
        torch.cuda.synchronize()
    for t in a + b:
        torch.testing.assert_close(t, ref, atol=0, rtol=0)


@pytest.mark.parametrize("block_size,num_splits", [(16, 5), (64, 16), (8, 7), (4, 3)])
def test_fused_merge_paged(block_size, num_splits):
    torch.manual_seed(block_size + num_splits)
    ctx = torch.tensor([0, 33, 700, 2048], device=DEVICE, dtype=torch.int32)
    nblk = 2048 // block_size
    q = torch.randn(4, 8, 128, device=DEVICE, dtype=torch.float16)
    kc = torch.randn(4 * nblk, block_size, 2, 128, device=DEVICE, dtype=torch.float16)
    vc = torch.randn_like(kc)
    bt = torch.randperm(4 * nblk, device=DEVICE, dtype=torch.int32).reshape(4, nblk)
    with torch.no_grad():
        fused, two = _both(lambda: flash_attention_decode_paged(q, kc, vc, bt, ctx, num_splits=num_splits))
    _ulp_close(fused, two)
    ref = oracle.paged_decode(q.float().cpu().numpy(), kc.float().cpu().numpy(), vc.float().cpu().numpy(),
                              bt.cpu().numpy(), ctx.cpu().numpy(), 1 / math.sqrt(128))
    assert np.abs(fused.float().cpu().numpy() - ref).max() <= 2e-3


@pytest.mark.parametrize("lens", [
    [1, 20000, 3, 0, 700],            # one long sequence among short and empty ones
    [0, 0, 0],                         # nothing to attend: zero rows
    [17] * 64,                         # 64 sequences: the balanced partition's largest batch
    [33 * (i % 7) for i in range(70)],  # 70 sequences: per-sequence splits, merged in-launch
])
def test_fused_merge_ragged_lengths(lens):
    torch.manual_seed(len(lens))
    b, sk = len(lens), max(max(lens), 1)
    q = torch.randn(b, 8, 2, 64, device=DEVICE, dtype=torch.float16)
    k = torch.randn(b, 2, sk, 64, device=DEVICE, dtype=torch.float16)
    v = torch.randn_like(k)
    cl = torch.tensor(lens, device=DEVICE, dtype=torch.int32)
    with torch.no_grad():
        fused, two = _both(lambda: flash_attention_decode(q, k, v, cache_seqlens=cl))
    _ulp_close(fused, two)
    ref = oracle.decode(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(), 0.125,
                        np.array(lens))
    assert np.abs(fused.float().cpu().numpy() - ref).max() <= 2e-3
