"""Split-K and paged decode recorded in HIP graphs, replayed between eager
calls on the same stream and beside a second graph captured on that stream.

The in-launch merge of the split partials counts arrivals in a per-stream
counter buffer that every call leaves at zero.  A call captured before its
stream has such a buffer records the two-launch merge instead (a buffer made
during capture would never be zeroed); later captures on the stream use the
buffer eager calls created.  Every replay is checked against the eager
result, with eager work and synchronisations between replays."""

import pytest
import torch

from fa_rdna3 import flash_attention_decode, flash_attention_decode_paged

pytestmark = pytest.mark.gpu
DEVICE = "cuda"


def _inputs():
    g = torch.Generator().manual_seed(7)
    q = torch.randn(3, 16, 1, 128, generator=g).half().to(DEVICE)
    k = torch.randn(3, 4, 3000, 128, generator=g).half().to(DEVICE)
    v = torch.randn(3, 4, 3000, 128, generator=g).half().to(DEVICE)
    lens = torch.tensor([2999, 1500, 37], dtype=torch.int32, device=DEVICE)
    qp = torch.randn(2, 16, 128, generator=g).half().to(DEVICE)
    kc = torch.randn(300, 16, 4, 128, generator=g).half().to(DEVICE)
    vc = torch.randn(300, 16, 4, 128, generator=g).half().to(DEVICE)
    bt = torch.randperm(300, generator=g)[:256].to(torch.int32).reshape(2, 128).to(DEVICE)
    ctx = torch.tensor([2048, 777], dtype=torch.int32, device=DEVICE)
    return (q, k, v, lens), (qp, kc, vc, bt, ctx)


def test_decode_graphs_with_eager_calls_between_replays():
    (q, k, v, lens), (qp, kc, vc, bt, ctx) = _inputs()
    dense = lambda: flash_attention_decode(q, k, v, cache_seqlens=lens)
    paged = lambda: flash_attention_decode_paged(qp, kc, vc, bt, ctx, max_context_len=2048)
    ref_d, ref_p = dense(), paged()
    torch.cuda.synchronize()

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    g1 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1, stream=stream):  # fresh stream: no counter buffer yet
        out1d, out1p = dense(), paged()
    with torch.cuda.stream(stream):  # eager calls on the capture stream create the buffer
        e_d, e_p = dense(), paged()
    stream.synchronize()
    torch.testing.assert_close(e_d, ref_d, atol=0, rtol=0)
    torch.testing.assert_close(e_p, ref_p, atol=0, rtol=0)
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=stream):  # records the fused merge on that buffer
        out2d, out2p = dense(), paged()

    for it in range(4):
        # g2 runs the same fused merge as the eager calls (bit-identical); g1
        # merges in a second launch, whose summation order differs.
        for graph, od, op, tol in ((g2, out2d, out2p, 0.0), (g1, out1d, out1p, 1e-3)):
            od.zero_()
            op.zero_()
            graph.replay()
            torch.cuda.synchronize()
            torch.testing.assert_close(od, ref_d, atol=tol, rtol=0, msg=f"dense replay {it}")
            torch.testing.assert_close(op, ref_p, atol=tol, rtol=0, msg=f"paged replay {it}")
            with torch.cuda.stream(stream):
                e_d, e_p = dense(), paged()
            stream.synchronize()
            torch.testing.assert_close(e_d, ref_d, atol=0, rtol=0, msg=f"eager after replay {it}")
            torch.testing.assert_close(e_p, ref_p, atol=0, rtol=0, msg=f"eager after replay {it}")
