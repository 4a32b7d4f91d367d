"""fa_decode_splitk_noalloc (static per-GPU scratch, no allocation) against
fa_decode_splitk with a caller workspace, both called through the C ABI.

Two calls in a row, the second on a smaller input, each checked bit for bit
against the allocating entry point (same kernels, same partition, same
merge), and against the oracle within the fp16 tolerance.  Oversized calls
are rejected with a clear message."""

import ctypes
import math

import numpy as np
import pytest
import torch

from fa_rdna3 import _native
from fa_rdna3.interface import _streaming_decode_splits
from oracle import attention as oracle

pytestmark = pytest.mark.gpu
DEVICE = "cuda"


def _params(q, k, v, out, lens, num_splits):
    p = _native.DecodeParams()
    p.abi_version = _native.ABI_VERSION
    p.dtype = _native.DTYPE_CODE[q.dtype]
    p.q, p.k, p.v, p.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    for name, t in (("q_stride", q), ("k_stride", k), ("v_stride", v), ("out_stride", out)):
        getattr(p, name)[:] = _native.strides(t)
    p.batch, p.heads_q, p.seqlen_q, p.head_dim = q.shape
    p.heads_kv, p.seqlen_k = k.shape[1], k.shape[2]
    p.cache_seqlens = lens.data_ptr()
    p.cache_seqlens_stride = 1
    p.softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    p.num_splits = num_splits
    p.k_scale = p.v_scale = 1.0
    return p


def _call(name, p):
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = getattr(_native.lib(), name)(ctypes.byref(p), stream)
    return rc, _native.lib().fa_last_error_string().decode()


def _run_pair(b, hq, hk, sq, sk, lens, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, sq, 128, generator=g).half()
    k = torch.randn(b, hk, sk, 128, generator=g).half()
    v = torch.randn(b, hk, sk, 128, generator=g).half()
    lt = torch.tensor(lens, dtype=torch.int32)
    dq, dk, dv, dl = (t.to(DEVICE) for t in (q, k, v, lt))
    splits = _streaming_decode_splits(b, hk, (hq // hk) * sq, sk, torch.cuda.get_device_properties(0).multi_processor_count)
    ref_out = torch.empty_like(dq)
    ws = torch.empty(_native.decode_workspace_bytes(b, hq, sq, 128, splits), dtype=torch.uint8, device=DEVICE)
    tickets = torch.zeros(b * hq * sq, dtype=torch.int32, device=DEVICE)
    p = _params(dq, dk, dv, ref_out, dl, splits)
    p.workspace, p.tickets = ws.data_ptr(), tickets.data_ptr()
    assert _call("fa_decode_splitk", p)[0] == 0
    out = torch.empty_like(dq)
    pn = _params(dq, dk, dv, out, dl, splits)
    rc, msg = _call("fa_decode_splitk_noalloc", pn)
    assert rc == 0, msg
    torch.cuda.synchronize()
    print(f"noalloc b={b} hq={hq} sq={sq} sk={sk} splits={splits}", flush=True)
    torch.testing.assert_close(out, ref_out, atol=0, rtol=0)
    want = oracle.decode(q.float().numpy(), k.float().numpy(), v.float().numpy(), 1 / math.sqrt(128), lt.numpy())
    assert np.abs(out.float().cpu().numpy() - want).max() <= 2e-3
    return out


def test_noalloc_matches_allocating_entry_point_twice():
    # First call: 4 sequences of up to 8192 keys; second: a smaller problem
    # on the same scratch (its counters must have been left at zero).
    _run_pair(4, 32, 8, 1, 8192, [5713, 6857, 7358, 8192], seed=1)
    _run_pair(2, 16, 4, 2, 3000, [2999, 17], seed=2)


def test_noalloc_rejects_oversized_calls():
    q = torch.zeros(64, 64, 16, 128, dtype=torch.float16, device=DEVICE)
    k = torch.zeros(64, 8, 64, 128, dtype=torch.float16, device=DEVICE)
    lens = torch.full((64,), 64, dtype=torch.int32, device=DEVICE)
    p = _params(q, k, k, torch.empty_like(q), lens, 64)
    rc, msg = _call("fa_decode_splitk_noalloc", p)
    assert rc != 0 and "static scratch" in msg


def test_noalloc_replays_under_hip_graph_capture():
    # The entry point's purpose: a call recorded in a HIP graph (no
    # allocation, no memset node) replays correctly, with eager work and
    # synchronisations between the replays, against the eager result.
    g = torch.Generator().manual_seed(9)
    q = torch.randn(2, 32, 1, 128, generator=g).half().to(DEVICE)
    k = torch.randn(2, 8, 4096, 128, generator=g).half().to(DEVICE)
    v = torch.randn(2, 8, 4096, 128, generator=g).half().to(DEVICE)
    lens = torch.tensor([4000, 1500], dtype=torch.int32, device=DEVICE)
    splits = 8
    eager = torch.empty_like(q)
    assert _call("fa_decode_splitk_noalloc", _params(q, k, v, eager, lens, splits))[0] == 0
    torch.cuda.synchronize()
    out = torch.zeros_like(q)
    p = _params(q, k, v, out, lens, splits)
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        rc, msg = _call("fa_decode_splitk_noalloc", p)
    assert rc == 0, msg
    for i in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(out, eager, atol=0, rtol=0)
        _ = (k[:, :, :64].float() * (i + 1)).sum().item()  # eager work between replays


def test_noalloc_calls_on_two_streams_are_ordered():
    # Calls on different streams share the static scratch; the entry point
    # orders each call after the previous one on the device (an event wait),
    # so back-to-back calls on two streams without any caller
    # synchronisation both give the allocating entry point's bits.
    g = torch.Generator().manual_seed(11)
    cases = []
    for i, (b, sk) in enumerate(((4, 8192), (2, 3000), (4, 6000), (1, 8192), (3, 2048), (4, 8192))):
        q = torch.randn(b, 32, 1, 128, generator=g).half().to(DEVICE)
        k = torch.randn(b, 8, sk, 128, generator=g).half().to(DEVICE)
        v = torch.randn(b, 8, sk, 128, generator=g).half().to(DEVICE)
        lens = torch.randint(1, sk + 1, (b,), generator=g).to(torch.int32).to(DEVICE)
        splits = 8
        ref = torch.empty_like(q)
        ws = torch.empty(_native.decode_workspace_bytes(b, 32, 1, 128, splits), dtype=torch.uint8, device=DEVICE)
        tickets = torch.zeros(b * 32, dtype=torch.int32, device=DEVICE)
        p = _params(q, k, v, ref, lens, splits)
        p.workspace, p.tickets = ws.data_ptr(), tickets.data_ptr()
        assert _call("fa_decode_splitk", p)[0] == 0
        out = torch.full_like(q, float("nan"))
        # The params hold raw pointers: keep the tensors alive with them.
        cases.append((_params(q, k, v, out, lens, splits), out, ref, (q, k, v, lens)))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    # A long matrix product ahead of the first call keeps stream 0 busy, so
    # the calls queued behind it on both streams would otherwise overlap.
    big = torch.randn(4096, 4096, device=DEVICE, dtype=torch.float16)
    with torch.cuda.stream(streams[0]):
        for _ in range(4):
            big = big @ big
            big = big / big.abs().amax().clamp(min=1)
    for i, (p, out, _, _) in enumerate(cases):
        with torch.cuda.stream(streams[i % 2]):
            rc, msg = _call("fa_decode_splitk_noalloc", p)
        assert rc == 0, msg
    torch.cuda.synchronize()
    print("noalloc two streams: 6 calls", flush=True)
    for p, out, ref, _ in cases:
        torch.testing.assert_close(out, ref, atol=0, rtol=0)
