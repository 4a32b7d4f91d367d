"""Packed variable-length attention (behaviour contract of the reference
tests test_varlen.py and test_varlen_mods.py)."""

import pytest
import torch

from attn_refs import check_grads, cu_seqlens, max_err, varlen_attention, assert_ratio
from fa_rdna3 import alibi_slopes, flash_attention, flash_attention_varlen

pytestmark = pytest.mark.gpu
DEVICE = "cuda"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("q_heads,kv_heads", [(8, 8), (8, 2)])
def test_varlen_forward(dtype, causal, q_heads, kv_heads):
    torch.manual_seed(q_heads + kv_heads + int(causal))
    lengths = [128, 57, 300, 1]
    total = sum(lengths)
    q = torch.randn(total, q_heads, 64, device=DEVICE, dtype=dtype)
    k = torch.randn(total, kv_heads, 64, device=DEVICE, dtype=dtype)
    v = torch.randn_like(k)
    cu = cu_seqlens(lengths)
    out = flash_attention_varlen(q, k, v, cu, cu, max(lengths), max(lengths), causal=causal)
    exact = varlen_attention(q.float(), k.float(), v.float(), lengths, lengths, causal=causal)
    naive = varlen_attention(q, k, v, lengths, lengths, causal=causal)
    assert_ratio(out, naive, exact)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("q_heads,kv_heads", [(8, 8), (8, 2)])
def test_varlen_backward(causal, q_heads, kv_heads):
    torch.manual_seed(q_heads + kv_heads + int(causal))
    lengths = [200, 64, 129]
    total = sum(lengths)
    cu = cu_seqlens(lengths)
    q = torch.randn(total, q_heads, 64, device=DEVICE, dtype=torch.float16)
    k = torch.randn(total, kv_heads, 64, device=DEVICE, dtype=torch.float16)
    v = torch.randn_like(k)
    do = torch.randn_like(q)
    check_grads(lambda a, b, c: flash_attention_varlen(a, b, c, cu, cu, 200, 200, causal),
                lambda a, b, c: varlen_attention(a, b, c, lengths, lengths, causal=causal), q, k, v, do)


@pytest.mark.parametrize("causal", [False, True])
def test_varlen_backward_long_bf16(causal):
    torch.manual_seed(41 + int(causal))
    lengths = [600, 129]
    total = sum(lengths)
    cu = cu_seqlens(lengths)
    q = torch.randn(total, 4, 128, device=DEVICE, dtype=torch.bfloat16)
    k = torch.randn(total, 2, 128, device=DEVICE, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    do = torch.randn_like(q)
    check_grads(lambda a, b, c: flash_attention_varlen(a, b, c, cu, cu, 600, 600, causal),
                lambda a, b, c: varlen_attention(a, b, c, lengths, lengths, causal=causal), q, k, v, do)


def test_varlen_intervals_bounded_to_storage():
    torch.manual_seed(53)
    q = torch.randn(128, 2, 64, device=DEVICE, dtype=torch.float16)
    k, v = torch.randn_like(q), torch.randn_like(q)
    valid = torch.tensor([0, 128], device=DEVICE, dtype=torch.int32)
    oob = torch.tensor([-32, 160], device=DEVICE, dtype=torch.int32)
    torch.testing.assert_close(flash_attention_varlen(q, k, v, oob, oob, 128, 128),
                               flash_attention_varlen(q, k, v, valid, valid, 128, 128))


def test_varlen_matches_batched():
    torch.manual_seed(7)
    q, k, v = (torch.randn(3, 8, 128, 64, device=DEVICE, dtype=torch.float16) for _ in range(3))
    batched = flash_attention(q, k, v, causal=True)
    pack = lambda t: t.transpose(1, 2).reshape(3 * 128, 8, 64)
    cu = cu_seqlens([128] * 3)
    out = flash_attention_varlen(pack(q), pack(k), pack(v), cu, cu, 128, 128, causal=True)
    out = out.reshape(3, 128, 8, 64).transpose(1, 2)
    torch.testing.assert_close(out.float(), batched.float(), atol=2e-3, rtol=2e-3)


@pytest.mark.parametrize("causal", [False, True])
def test_varlen_cross_attention(causal):
    torch.manual_seed(29 + int(causal))
    lq, lk = [65, 129], [200, 80]
    cq, ck = cu_seqlens(lq), cu_seqlens(lk)
    q = torch.randn(sum(lq), 4, 64, device=DEVICE, dtype=torch.float16)
    k = torch.randn(sum(lk), 2, 64, device=DEVICE, dtype=torch.float16)
    v = torch.randn_like(k)
    do = torch.randn_like(q)
    check_grads(lambda a, b, c: flash_attention_varlen(a, b, c, cq, ck, 129, 200, causal),
                lambda a, b, c: varlen_attention(a, b, c, lq, lk, causal=causal), q, k, v, do)


CASES = [
    dict(causal=True, window=(31, 0), softcap=0.0, use_alibi=False),
    dict(causal=False, window=(-1, -1), softcap=30.0, use_alibi=False),
    dict(causal=True, window=(-1, -1), softcap=0.0, use_alibi=True),
    dict(causal=True, window=(100, -1), softcap=50.0, use_alibi=False),
]


@pytest.mark.parametrize("case", CASES, ids=str)
def test_varlen_modifiers(case):
    torch.manual_seed(len(str(case)))
    lengths = [128, 65, 200]
    total = sum(lengths)
    cu = cu_seqlens(lengths)
    slopes = alibi_slopes(8, device=DEVICE) if case["use_alibi"] else None
    q, k, v, do = (torch.randn(total, 8, 64, device=DEVICE, dtype=torch.float16) for _ in range(4))
    kw = dict(causal=case["causal"], window=case["window"], softcap=case["softcap"], alibi=slopes)
    fn = lambda a, b, c: flash_attention_varlen(a, b, c, cu, cu, 200, 200, causal=case["causal"],
                                                window_size=case["window"], softcap=case["softcap"],
                                                alibi_slopes=slopes)
    ref = lambda a, b, c: varlen_attention(a, b, c, lengths, lengths, **kw)
    assert_ratio(fn(q, k, v), ref(q, k, v), ref(q.float(), k.float(), v.float()), slack=2e-3)
    check_grads(fn, ref, q, k, v, do, slack=2e-3)
