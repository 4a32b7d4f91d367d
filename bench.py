#!/usr/bin/env python3
"""Benchmark of the MI355X FlashAttention path (one JSON line on stdout).

Metric: causal fwd+bwd TFLOP/s at 2x16x2048x128 fp16
(config 2), with the decode KV-read GB/s of configs 3 (split-K GQA decode)
and 4 (paged decode) reported beside it.  A "step" is one forward + backward
of config 2 on synthetic N(0,1) inputs already resident in HBM.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]

FLOP convention (reference bench/benchmark.py:32-36, :123): forward
4*B*H*S^2*D / 2 under causal masking, backward 2.5x forward.  Decode bytes
count every K/V byte of the visible keys once per KV head (+ q and out).

The JSON line carries `roofline` for the dominant kernel (the dK/dV backward
kernel, timed alone with HIP events on the launch stream) and `cpu_baseline`
(the reference's CPU path, torch math SDPA in fp32, on config 2 or a
slice of its heads).
"""

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "flash-attention-rdna3_amd"))

import torch  # noqa: E402

# MI355X published peaks.
PEAK_FP16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0

# HBM bytes moved per dkdv16_kernel<f16,128,0> launch at config 2, from
# rocprofv3 FETCH_SIZE / WRITE_SIZE runs scaled by a 256 MiB copy
# (profiles/cfg2_hbm_traffic.md).  The bench cannot read counters itself;
# re-measure when the kernel changes.
DKDV_TRAFFIC_BYTES = 318.6e6

CFG2 = dict(batch=2, heads=16, seqlen=2048, head_dim=128, causal=True, dtype=torch.float16)


# ---------------------------------------------------------------------------
# Seeded workloads of BASELINE.json (inputs drawn on the CPU with
# torch.Generator().manual_seed(0), cast, then moved to the device).
# ---------------------------------------------------------------------------

def _gen(seed=0):
    return torch.Generator().manual_seed(seed)


def workload_cfg1(device="cpu"):
    g = _gen()
    q, k, v = (torch.randn(1, 16, 1024, 64, generator=g).half().float().to(device) for _ in range(3))
    return q, k, v, 1.0 / 8.0


def workload_cfg2(device="cuda", dtype=torch.float16):
    g = _gen()
    shape = (CFG2["batch"], CFG2["heads"], CFG2["seqlen"], CFG2["head_dim"])
    q, k, v, do = (torch.randn(shape, generator=g).to(dtype).to(device) for _ in range(4))
    return q, k, v, do, 1.0 / math.sqrt(128)


def workload_cfg3(device="cuda"):
    g = _gen()
    q = torch.randn(4, 32, 1, 128, generator=g).half()
    k = torch.randn(4, 8, 8192, 128, generator=g).half()
    v = torch.randn(4, 8, 8192, 128, generator=g).half()
    lens = torch.randint(1024, 8193, (4,), generator=_gen()).to(torch.int32)
    return q.to(device), k.to(device), v.to(device), lens.to(device)


def workload_cfg4(device="cuda"):
    g = _gen()
    q = torch.randn(4, 32, 128, generator=g).half()
    kc = torch.randn(4096, 16, 8, 128, generator=g).half()
    vc = torch.randn(4096, 16, 8, 128, generator=g).half()
    bt = torch.randperm(4096, generator=_gen()).to(torch.int32).reshape(4, 1024)
    ctx = torch.full((4,), 16384, dtype=torch.int32)
    return q.to(device), kc.to(device), vc.to(device), bt.to(device), ctx.to(device)


def workload_cfg5(device="cuda"):
    lengths = torch.randint(128, 2049, (16,), generator=_gen()).tolist()
    total = sum(lengths)
    g = _gen()
    q = torch.randn(total, 32, 128, generator=g).bfloat16()
    k = torch.randn(total, 8, 128, generator=g).bfloat16()
    v = torch.randn(total, 8, 128, generator=g).bfloat16()
    do = torch.randn(total, 32, 128, generator=g).bfloat16()
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)), dtype=torch.int32)
    return lengths, q.to(device), k.to(device), v.to(device), do.to(device), cu.to(device)


def cfg2_flops():
    c = CFG2
    fwd = 4.0 * c["batch"] * c["heads"] * c["seqlen"] ** 2 * c["head_dim"] / 2
    return fwd, 2.5 * fwd


def cfg3_bytes(lens):
    return sum(int(n) for n in lens) * 8 * 128 * 2 * 2 + 2 * 4 * 32 * 128 * 2


def kvcache_bytes(lens, snew=4):
    """cfg3's cache read at lengths len_b + snew, the appended rows written
    (and read from the inputs), q and out (Sq = snew)."""
    return (sum(int(n) + snew for n in lens) * 8 * 128 * 2 * 2 + 2 * 4 * 8 * snew * 128 * 2 * 2
            + 2 * 4 * 32 * snew * 128 * 2)


def cfg4_bytes():
    return 4 * 16384 * 8 * 128 * 2 * 2 + 4 * 1024 * 4 + 2 * 4 * 32 * 128 * 2


def cfg5_flops(lengths, window_left=1024):
    pairs = sum(min(i + 1, window_left + 1) for n in lengths for i in range(n))
    fwd = 4.0 * 32 * 128 * pairs
    return fwd, 2.5 * fwd


# ---------------------------------------------------------------------------
# GPU timing helpers
# ---------------------------------------------------------------------------

def _event_time(fn, iters, stream):
    """Average ms per call of fn() measured with HIP events on `stream`."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / iters


def _flush_buffer(device):
    """512 MiB (twice the 256 MiB MALL) whose full read evicts the caches.

    The flush reads instead of writing: zero-filling it would leave the MALL
    full of dirty lines whose write-back then competes with the kernel being
    timed, which charges the kernel for the flush.
    """
    return torch.ones(128 * 1024 * 1024, dtype=torch.int32, device=device)


def _flush(buf):
    buf.max()


# Warm-up continues past the requested step count until this much wall time
# of steps has run: the first ~0.1 s of back-to-back steps on a fresh box run
# up to 20 % slower than the steady state (shader clock still ramping).
MIN_WARMUP_S = 1.0


def run_cfg2(steps, warmup):
    from fa_rdna3 import flash_attention

    q, k, v, do, scale = workload_cfg2()
    q.requires_grad_(True)
    k.requires_grad_(True)
    v.requires_grad_(True)

    def step():
        # As after optimizer.zero_grad(set_to_none=True): the gradients are
        # written, not added into earlier ones (no extra elementwise kernels).
        q.grad = k.grad = v.grad = None
        out = flash_attention(q, k, v, causal=True, softmax_scale=scale)
        out.backward(do)

    t_warm = time.perf_counter()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    while time.perf_counter() - t_warm < MIN_WARMUP_S:
        for _ in range(10):
            step()
        torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    return dt, (q, k, v, do, scale)


def gemm_ceiling(n=8192, iters=10):
    """The MFMA rate a library GEMM reaches on this GPU: torch.matmul
    (hipBLASLt) on n x n x n fp16, HIP events, after warm-up.  Context for the
    attention kernels' fraction of the 2.5 PF/s datasheet peak."""
    a = torch.randn(n, n, device="cuda", dtype=torch.float16)
    b = torch.randn(n, n, device="cuda", dtype=torch.float16)
    for _ in range(3):
        torch.matmul(a, b)
    ms = _event_time(lambda: torch.matmul(a, b), iters, torch.cuda.current_stream())
    return 2.0 * n ** 3 / (ms * 1e-3) / 1e12


def dkdv_roofline(tensors, iters=100):
    """Time the dK/dV kernel (fa_bwd phase 1) with HIP events, in the order
    of a training step: each of `iters` rounds runs the delta phase, the
    dK/dV phase between two events, then dQ from the stored dS, so dK/dV
    meets the cache state it has inside the step (a loop of dK/dV alone
    runs each launch behind the previous one's 143 MB of dS writes and
    measured 6-10 % slower).  `avg_us` is the mean over the rounds of the
    bracketed dK/dV launch; `avg_us_back_to_back` the dK/dV-only loop."""
    from fa_rdna3 import interface as I

    q, k, v, do, scale = tensors
    stream = torch.cuda.current_stream()
    with torch.no_grad():
        out, lse = I._forward(q.detach(), k.detach(), v.detach(), True, scale, (-1, -1), 0.0, None, None, 0.0, 0)
        launch = I._backward_launcher(do, q.detach(), k.detach(), v.detach(), out, lse, True, scale,
                                      (-1, -1), 0.0, None, None, 0.0, 0)
        launch(0)  # delta, needed by the dK/dV phase
        for _ in range(5):
            launch(1)
        ms_b2b = _event_time(lambda: launch(1), iters, stream)
        for _ in range(5):
            launch(0), launch(1), launch(2)
        pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
        for e0, e1 in pairs:
            launch(0)
            e0.record(stream)
            launch(1)
            e1.record(stream)
            launch(2)
        pairs[-1][1].synchronize()
        ms = sum(e0.elapsed_time(e1) for e0, e1 in pairs) / iters
    fwd, _ = cfg2_flops()
    flops = 2.0 * fwd  # S recompute, dP, dV, dK: 4 of the 5 algorithmic backward GEMMs
    achieved = flops / (ms * 1e-3) / 1e12
    return {"kernel": "dkdv16_kernel<f16,128,0>", "bound": "mfma", "achieved": round(achieved, 2),
            "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP16_TFLOPS, 4),
            "traffic": DKDV_TRAFFIC_BYTES, "avg_us": round(ms * 1e3, 2), "flops_per_launch": flops,
            "avg_us_back_to_back": round(ms_b2b * 1e3, 2),
            "how": "HIP events around each dK/dV launch in delta -> dK/dV -> dQ rounds on the launch stream"}


def step_kernel_times(tensors, iters=50):
    """Each kernel of the config-2 step alone, HIP events over `iters`
    launches on the current stream: forward, delta, dK/dV (stores dS) and
    dQ from that dS, with the algorithmic TFLOP/s of the three products
    (forward 4·D, dK/dV 8·D, dQ 2·D flops per visible pair)."""
    from fa_rdna3 import interface as I

    q, k, v, do, scale = tensors
    stream = torch.cuda.current_stream()
    fwd, _ = cfg2_flops()
    with torch.no_grad():
        qd, kd, vd = q.detach(), k.detach(), v.detach()
        run_fwd = lambda: I._forward(qd, kd, vd, True, scale, (-1, -1), 0.0, None, None, 0.0, 0)
        out, lse = run_fwd()
        launch = I._backward_launcher(do, qd, kd, vd, out, lse, True, scale, (-1, -1), 0.0, None, None, 0.0, 0)
        res = {}
        for name, fn, flops in (("forward", run_fwd, fwd), ("delta", lambda: launch(0), 0.0),
                                ("dkdv", lambda: launch(1), 2.0 * fwd), ("dq", lambda: launch(2), 0.5 * fwd)):
            for _ in range(3):
                fn()
            ms = _event_time(fn, iters, stream)
            res[name] = {"us": round(ms * 1e3, 2)}
            if flops:
                res[name]["TFLOP/s"] = round(flops / (ms * 1e-3) / 1e12, 1)
    return res


def run_decode_configs(iters=100):
    from fa_rdna3 import (flash_attention_decode, flash_attention_decode_paged, flash_attention_decode_paged_multi,
                          flash_attention_with_kvcache)

    res = {}
    stream = torch.cuda.current_stream()
    flush = _flush_buffer("cuda")
    with torch.no_grad():
        q, k, v, lens = workload_cfg3()
        f3 = lambda: flash_attention_decode(q, k, v, cache_seqlens=lens)
        for _ in range(5):
            f3()
        tot = 0.0
        for _ in range(iters):
            _flush(flush)
            tot += _event_time(f3, 1, stream)
        ms = tot / iters
        gb = cfg3_bytes(lens.tolist()) / (ms * 1e-3) / 1e9
        res["cfg3_splitk_decode"] = {"us": round(ms * 1e3, 2), "GB/s": round(gb, 1),
                                     "frac_hbm": round(gb / PEAK_HBM_GBS, 4), "caches_flushed": "read of 512 MiB"}
        # The cfg3 cache stored as fp8 (OCP e4m3, per-tensor scale 1): half
        # the bytes of the fp16 cache.
        k8, v8 = k.to(torch.float8_e4m3fn), v.to(torch.float8_e4m3fn)
        f8 = lambda: flash_attention_decode(q, k8, v8, cache_seqlens=lens)
        for _ in range(5):
            f8()
        tot = 0.0
        for _ in range(iters):
            _flush(flush)
            tot += _event_time(f8, 1, stream)
        ms = tot / iters
        b8 = sum(int(n) for n in lens.tolist()) * 8 * 128 * 1 * 2 + 2 * 4 * 32 * 128 * 2
        gb = b8 / (ms * 1e-3) / 1e9
        res["cfg3_fp8_kv_decode"] = {"us": round(ms * 1e3, 2), "GB/s": round(gb, 1),
                                     "frac_hbm": round(gb / PEAK_HBM_GBS, 4), "caches_flushed": "read of 512 MiB",
                                     "bytes": b8}
        del k8, v8
        # KV-cache entry point on the cfg3 cache: 4 new tokens per sequence
        # appended in place at the cfg3 lengths, then 4 query rows attend
        # bottom-right causally (speculative / chunked decode step).
        g = _gen(1)
        q4 = torch.randn(4, 32, 4, 128, generator=g).half().cuda()
        kn = torch.randn(4, 8, 4, 128, generator=g).half().cuda()
        vn = torch.randn(4, 8, 4, 128, generator=g).half().cuda()
        fk = lambda: flash_attention_with_kvcache(q4, k, v, kn, vn, cache_seqlens=lens, causal=True)
        for _ in range(5):
            fk()
        tot = 0.0
        for _ in range(iters):
            _flush(flush)
            tot += _event_time(fk, 1, stream)
        ms = tot / iters
        gb = kvcache_bytes(lens.tolist()) / (ms * 1e-3) / 1e9
        res["kvcache_append_decode"] = {"us": round(ms * 1e3, 2), "GB/s": round(gb, 1),
                                        "frac_hbm": round(gb / PEAK_HBM_GBS, 4), "caches_flushed": "read of 512 MiB",
                                        "shape": "cfg3 cache, Sq = Snew = 4, causal"}
        del q, k, v
        q, kc, vc, bt, ctx = workload_cfg4()
        f4 = lambda: flash_attention_decode_paged(q, kc, vc, bt, ctx, max_context_len=16384)
        for _ in range(5):
            f4()
        tot = 0.0
        for _ in range(iters):
            _flush(flush)
            tot += _event_time(f4, 1, stream)
        ms = tot / iters
        gb = cfg4_bytes() / (ms * 1e-3) / 1e9
        res["cfg4_paged_decode"] = {"us": round(ms * 1e3, 2), "GB/s": round(gb, 1),
                                    "frac_hbm": round(gb / PEAK_HBM_GBS, 4), "caches_flushed": "read of 512 MiB"}
        # The cfg4 cache stored as fp8 (OCP e4m3, scale 1).
        kc8, vc8 = kc.to(torch.float8_e4m3fn), vc.to(torch.float8_e4m3fn)
        f48 = lambda: flash_attention_decode_paged(q, kc8, vc8, bt, ctx, max_context_len=16384)
        for _ in range(5):
            f48()
        tot = 0.0
        for _ in range(iters):
            _flush(flush)
            tot += _event_time(f48, 1, stream)
        ms = tot / iters
        b8 = 4 * 16384 * 8 * 128 * 1 * 2 + 4 * 1024 * 4 + 2 * 4 * 32 * 128 * 2
        gb = b8 / (ms * 1e-3) / 1e9
        res["cfg4_fp8_paged_decode"] = {"us": round(ms * 1e3, 2), "GB/s": round(gb, 1),
                                        "frac_hbm": round(gb / PEAK_HBM_GBS, 4),
                                        "caches_flushed": "read of 512 MiB", "bytes": b8}
        del kc8, vc8
        # Several query rows per sequence over the cfg4 cache (speculative /
        # chunked decode): 4 rows, bottom-right causal.
        q4 = torch.randn(4, 32, 4, 128, generator=_gen(2)).half().cuda()
        fm = lambda: flash_attention_decode_paged_multi(q4, kc, vc, bt, ctx, causal=True, max_context_len=16384)
        for _ in range(5):
            fm()
        tot = 0.0
        for _ in range(iters):
            _flush(flush)
            tot += _event_time(fm, 1, stream)
        ms = tot / iters
        gb = (cfg4_bytes() + 2 * 4 * 32 * 3 * 128 * 2) / (ms * 1e-3) / 1e9
        res["paged_multi_decode"] = {"us": round(ms * 1e3, 2), "GB/s": round(gb, 1),
                                     "frac_hbm": round(gb / PEAK_HBM_GBS, 4), "caches_flushed": "read of 512 MiB",
                                     "shape": "cfg4 cache, Sq = 4, causal"}
        del q4
        # A ragged serving batch: 16 sequences from 64 to 32768 keys in one
        # contiguous cache (GQA 32/8, D 128).  The split kernel shares its
        # workgroups out by sequence length, so the long sequences do not
        # leave the CUs of the short ones idle.
        rl = [32768, 512, 1024, 300, 2048, 128, 4096, 700, 16384, 64, 900, 1500, 256, 8000, 100, 3000]
        gr = _gen(3)
        qr = torch.randn(16, 32, 1, 128, generator=gr).half().cuda()
        kr = torch.randn(16, 8, 32768, 128, dtype=torch.float16, device="cuda")
        vr = torch.randn_like(kr)
        lr = torch.tensor(rl, dtype=torch.int32, device="cuda")
        fr = lambda: flash_attention_decode(qr, kr, vr, cache_seqlens=lr)
        for _ in range(5):
            fr()
        tot = 0.0
        for _ in range(iters):
            _flush(flush)
            tot += _event_time(fr, 1, stream)
        ms = tot / iters
        br = sum(rl) * 8 * 128 * 2 * 2 + 2 * 16 * 32 * 128 * 2
        gb = br / (ms * 1e-3) / 1e9
        res["ragged_decode"] = {"us": round(ms * 1e3, 2), "GB/s": round(gb, 1), "frac_hbm": round(gb / PEAK_HBM_GBS, 4),
                                "caches_flushed": "read of 512 MiB", "bytes": br,
                                "shape": "B=16 lengths 64..32768 (sum 71780), Hq 32, Hkv 8, D 128, fp16"}
        del qr, kr, vr
        res["hbm_read_ceiling"] = hbm_read_ceiling(
            {"cfg3_bytes": cfg3_bytes(lens.tolist()), "cfg4_bytes": cfg4_bytes()}, flush, iters)
        for name, key in (("cfg3_splitk_decode", "cfg3_bytes"), ("cfg4_paged_decode", "cfg4_bytes")):
            res[name]["frac_of_read_ceiling"] = round(res["hbm_read_ceiling"][key]["us"] / res[name]["us"], 4)
    return res


def hbm_read_ceiling(sizes, flush, iters=50):
    """The HBM read rate a plain hand-written streaming kernel reaches for
    each byte count (fa_hbm_read_probe: every 16-byte piece read once, U
    loads per lane in flight), caches flushed before every timed call; the
    best of the probe's variants (block size, loads in flight, nontemporal,
    one-pass or persistent grid) is the ceiling."""
    from fa_rdna3 import _native

    stream = torch.cuda.current_stream()
    sink = torch.zeros(1024, dtype=torch.int32, device="cuda")
    names = _native.hbm_read_probe_variants()
    out = {}
    for key, nbytes in sizes.items():
        x = torch.ones((nbytes + 15) // 16 * 4, dtype=torch.int32, device="cuda")
        best = None
        for vi in range(len(names)):
            fn = lambda: _native.hbm_read_probe(x, sink, vi)
            for _ in range(3):
                fn()
            tot = 0.0
            for _ in range(iters):
                _flush(flush)
                tot += _event_time(fn, 1, stream)
            us = tot / iters * 1e3
            if best is None or us < best[0]:
                best = (us, vi)
        us, vi = best
        out[key] = {"bytes": nbytes, "us": round(us, 2), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
                    "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4), "variant": names[vi]}
        del x
    out["how"] = ("fa_hbm_read_probe (csrc/fa_hbm_read.hip), best of its variants, HIP events, "
                  "512 MiB read before every call")
    return out


def run_cfg5(iters=20):
    from fa_rdna3 import flash_attention_varlen

    lengths, q, k, v, do, cu = workload_cfg5()
    q.requires_grad_(True)
    k.requires_grad_(True)
    v.requires_grad_(True)
    mx = max(lengths)

    def step():
        q.grad = k.grad = v.grad = None
        out = flash_attention_varlen(q, k, v, cu, cu, mx, mx, causal=True, window_size=(1024, -1), softcap=50.0)
        out.backward(do)

    t_warm = time.perf_counter()
    step()
    torch.cuda.synchronize()
    while time.perf_counter() - t_warm < MIN_WARMUP_S:
        step()
        torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / iters
    fwd, bwd = cfg5_flops(lengths)
    return {"ms": round(dt * 1e3, 3), "TFLOP/s": round((fwd + bwd) / dt / 1e12, 1)}


def run_varlen_many(iters=20):
    """Many short packed sequences: 400 of 64-192 tokens (seed 3), Hq=32,
    Hkv=8, D=128 fp16 causal fwd + bwd, warmed up, then `iters` steps; GFLOP
    by the cfg2 convention (fwd 4*D*Hq*pairs, fwd + bwd 3.5x that)."""
    from fa_rdna3 import flash_attention_varlen

    g = torch.Generator().manual_seed(3)
    lengths = torch.randint(64, 193, (400,), generator=g).tolist()
    total = sum(lengths)
    q, do = (torch.randn(total, 32, 128, generator=g).half().cuda() for _ in range(2))
    k, v = (torch.randn(total, 8, 128, generator=g).half().cuda() for _ in range(2))
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)), dtype=torch.int32).cuda()
    mx = max(lengths)
    for t in (q, k, v):
        t.requires_grad_(True)

    def step():
        q.grad = k.grad = v.grad = None
        flash_attention_varlen(q, k, v, cu, cu, mx, mx, causal=True).backward(do)

    for _ in range(5):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / iters
    fwd = 4.0 * 32 * 128 * sum(n * (n + 1) // 2 for n in lengths)
    return {"ms": round(dt * 1e3, 3), "TFLOP/s": round(3.5 * fwd / dt / 1e12, 1),
            "shape": "400 sequences of 64-192 tokens, Hq=32 Hkv=8 D=128 fp16 causal fwd+bwd"}


def run_long_causal(iters=5):
    """A long causal sequence: B=1, H=32, S=16384, D=128 fp16 fwd + bwd
    (7.70 TFLOP by the cfg2 convention), warmed up, then `iters` steps."""
    from fa_rdna3 import flash_attention

    g = _gen(4)
    shape = (1, 32, 16384, 128)
    q, k, v, do = (torch.randn(shape, generator=g).half().cuda() for _ in range(4))
    for t in (q, k, v):
        t.requires_grad_(True)

    def step():
        q.grad = k.grad = v.grad = None
        flash_attention(q, k, v, causal=True).backward(do)

    step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / iters
    fwd = 4.0 * 32 * 16384 ** 2 * 128 / 2
    return {"ms": round(dt * 1e3, 3), "TFLOP/s": round(3.5 * fwd / dt / 1e12, 1),
            "shape": "B=1 H=32 S=16384 D=128 fp16 causal fwd+bwd"}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(budget_s=20.0):
    """The reference's CPU path: PyTorch math SDPA in fp32 (reference
    bench/benchmark.py:69,116 and README.md:20-28), forward + autograd
    backward of config 2 on the host cores, median of >= 5 timed runs after
    3 warm-ups.  When one full run would not fit the budget the sample is a
    leading slice of the heads (same B, S, D, causal), and the rate is that
    slice's flops over its time."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    threads = torch.get_num_threads()  # OMP_NUM_THREADS on the GPU box: its CPU share
    S, D, B, H = CFG2["seqlen"], CFG2["head_dim"], CFG2["batch"], CFG2["heads"]
    g = _gen()
    full = [torch.randn(B, H, S, D, generator=g).half().float() for _ in range(4)]

    def run(heads):
        q, k, v = (t[:, :heads].clone().requires_grad_(True) for t in full[:3])
        with sdpa_kernel([SDPBackend.MATH]):
            out = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True,
                                                                   scale=1.0 / math.sqrt(D))
        out.backward(full[3][:, :heads])

    run(1)  # first call pays one-time set-up
    t0 = time.perf_counter()
    run(1)
    one = time.perf_counter() - t0
    # 8 runs (3 warm-up + 5 timed) inside the budget
    heads = max(1, min(H, int(budget_s / 8 / max(one, 1e-3))))
    for _ in range(3):
        run(heads)
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        run(heads)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    fwd = 4.0 * B * heads * S * S * D / 2
    return {"value": round(3.5 * fwd / med / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "reference",
            "sample": f"torch math SDPA fp32 (SDPBackend.MATH) causal fwd+autograd bwd, B={B} H={heads} of {H} "
                      f"S={S} D={D}; median of 5 runs after 3 warm-ups, {med * 1e3:.0f} ms per run",
            "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count(), "torch_threads": threads}


def _cpu_median(run, budget_s):
    """Median wall time of run() over 5 timed calls after 3 warm-ups (one
    untimed call first pays one-time set-up)."""
    run()
    times = []
    for i in range(8):
        t0 = time.perf_counter()
        run()
        if i >= 3:
            times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def _cpu_attention(q, k, v, scale, causal=False, window_left=-1, softcap=0.0):
    """fp32 math attention on the host, (H, Sq, D) x (Hkv, Sk, D), GQA by
    head groups, bottom-right causal, left window, tanh softcap: the
    matmul -> softmax -> matmul path of the reference's CPU comparison.
    Returns (out, lse)."""
    hq, sq, d = q.shape
    hk, sk = k.shape[0], k.shape[1]
    qg = q.reshape(hk, (hq // hk) * sq, d)
    s = torch.matmul(qg, k.transpose(-1, -2)).reshape(hq, sq, sk) * scale
    if softcap > 0:
        s = softcap * torch.tanh(s / softcap)
    if causal or window_left >= 0:
        i = torch.arange(sq)[:, None] + (sk - sq)
        j = torch.arange(sk)[None, :]
        keep = torch.ones(sq, sk, dtype=torch.bool)
        if causal:
            keep &= j <= i
        if window_left >= 0:
            keep &= j >= i - window_left
        s = s.masked_fill(~keep, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.exp(s - lse[..., None])
    out = torch.matmul(p.reshape(hk, (hq // hk) * sq, sk), v).reshape(hq, sq, d)
    return out, lse


def cpu_baseline_configs(budget_s=8.0):
    """The reference's CPU path (fp32 math attention, reference
    bench/benchmark.py:69,116 and bench/decode_benchmark.py:56-57) on the
    other BASELINE configurations, on the host cores, inputs already in fp32
    host memory:
      cfg1  forward with out + LSE (the configuration that is the CPU path);
      cfg3  split-K GQA decode: per sequence, the first cache_seqlens keys;
      cfg4  paged decode: the block table's pages gathered, then attended
            (the gather is inside the timed region);
      cfg5  varlen causal fwd + autograd bwd with window 1024 and softcap 50,
            on a leading slice of the sequences sized to the budget.
    Rates use the GPU bench's algorithmic units (GFLOP/s; GB/s of the fp16
    K/V bytes of the workload, whatever width the CPU reads)."""
    res = {}
    torch.manual_seed(0)
    # cfg1
    q, k, v, scale = workload_cfg1()
    q, k, v = q[0], k[0], v[0]
    with torch.no_grad():
        t = _cpu_median(lambda: _cpu_attention(q, k, v, scale), budget_s)
    flops = 4.0 * 16 * 1024 * 1024 * 64
    res["cfg1_fwd"] = {"value": round(flops / t / 1e9, 2), "unit": "GFLOP/s", "ms": round(t * 1e3, 2),
                       "sample": "full cfg1: B=1 H=16 S=1024 D=64 fp32, non-causal, out + LSE"}
    # cfg3
    q, k, v, lens = workload_cfg3("cpu")
    q, k, v = q.float(), k.float(), v.float()
    lens = lens.tolist()

    def dec3():
        for b, n in enumerate(lens):
            _cpu_attention(q[b], k[b, :, :n], v[b, :, :n], 1.0 / math.sqrt(128))

    with torch.no_grad():
        t = _cpu_median(dec3, budget_s)
    res["cfg3_decode"] = {"value": round(cfg3_bytes(lens) / t / 1e9, 2), "unit": "GB/s", "ms": round(t * 1e3, 2),
                          "sample": "full cfg3: 4 sequences, Hq 32 / Hkv 8, cache_seqlens [5713, 6857, 7358, 7415], "
                                    "fp32 cache in host memory"}
    del q, k, v
    # cfg4
    q, kc, vc, bt, ctx = workload_cfg4("cpu")
    q, kc, vc = q.float(), kc.float(), vc.float()

    def dec4():
        for b in range(4):
            pages = bt[b].long()
            kk = kc.index_select(0, pages).reshape(-1, 8, 128)[: int(ctx[b])].transpose(0, 1)
            vv = vc.index_select(0, pages).reshape(-1, 8, 128)[: int(ctx[b])].transpose(0, 1)
            _cpu_attention(q[b][:, None], kk, vv, 1.0 / math.sqrt(128))

    with torch.no_grad():
        t = _cpu_median(dec4, budget_s)
    res["cfg4_paged_decode"] = {"value": round(cfg4_bytes() / t / 1e9, 2), "unit": "GB/s", "ms": round(t * 1e3, 2),
                                "sample": "full cfg4: 4 x 16384 keys in 16-key pages, Hq 32 / Hkv 8, gather + attend, "
                                          "fp32 cache in host memory"}
    del q, kc, vc
    # cfg5: the first sequence, on as many KV-head groups (4 query heads
    # each) as fit the budget
    lengths, q, k, v, do, cu = workload_cfg5("cpu")
    q, k, v, do = q.float(), k.float(), v.float(), do.float()
    n0 = lengths[0]

    def varlen(hk):
        qs = q[:n0, :4 * hk].transpose(0, 1).clone().requires_grad_(True)
        ks = k[:n0, :hk].transpose(0, 1).clone().requires_grad_(True)
        vs = v[:n0, :hk].transpose(0, 1).clone().requires_grad_(True)
        out, _ = _cpu_attention(qs, ks, vs, 1.0 / math.sqrt(128), causal=True, window_left=1024, softcap=50.0)
        out.backward(do[:n0, :4 * hk].transpose(0, 1))

    varlen(1)
    t0 = time.perf_counter()
    varlen(1)
    one = time.perf_counter() - t0
    hk = max(1, min(8, int(budget_s / 6 / max(one, 1e-3))))
    times = []
    for i in range(4):
        t0 = time.perf_counter()
        varlen(hk)
        if i >= 1:
            times.append(time.perf_counter() - t0)
    t = sorted(times)[1]
    fwd, bwd = cfg5_flops(lengths[:1])
    frac = hk / 8
    res["cfg5_varlen_fwd_bwd"] = {"value": round((fwd + bwd) * frac / t / 1e9, 2), "unit": "GFLOP/s",
                                  "ms": round(t * 1e3, 2),
                                  "sample": f"first cfg5 sequence ({n0} tokens), {4 * hk} of 32 query heads "
                                            f"({hk} of 8 KV heads), D 128 fp32, causal, window 1024, softcap 50, "
                                            "fwd + autograd bwd; median of 3 after 1 warm-up"}
    for r in res.values():
        r["cores"] = torch.get_num_threads()
        r["kind"] = "reference"
    return res


def pmc_summary(dirs):
    """Markdown table of rocprofv3 --pmc results (one directory per counter
    pass, each holding run_results.db): per kernel and grid, the average per
    dispatch of every counter, plus the derived MFMA figures."""
    import glob
    import sqlite3
    from collections import defaultdict

    acc = defaultdict(lambda: defaultdict(list))
    dur = defaultdict(list)
    for d in dirs:
        for db in glob.glob(os.path.join(d, "**", "*results.db"), recursive=True):
            con = sqlite3.connect(db)
            q = "select dispatch_id, kernel_name, grid_size, counter_name, value, duration from counters_collection"
            for disp, name, grid, cname, value, duration in con.execute(q):
                if "fa::" not in name:
                    continue
                key = (name.split("(")[0].replace("void fa::", ""), int(grid))
                acc[key][cname].append(float(value))
                dur[key].append(float(duration))
    simds = 256 * 4
    rows = []
    for key in sorted(acc, key=lambda k: -sum(dur[k]) / len(dur[k])):
        c = {n: sum(v) / len(v) for n, v in acc[key].items()}
        us = sum(dur[key]) / len(dur[key]) / 1e3
        mops = c.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0) + c.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0)
        tf = mops * 512 / (us * 1e-6) / 1e12 if us else 0.0
        # GRBM_GUI_ACTIVE counts GPU-busy cycles of the dispatch (summed over
        # the 8 XCDs): cycles per XCD = value / 8.
        cyc = c.get("GRBM_GUI_ACTIVE", 0.0) / 8
        busy = c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (cyc * simds) if cyc else 0.0
        mf = c.get("SQ_INSTS_MFMA", 0.0)
        rows.append((key, us, cyc / us / 1e3 if us else 0.0, tf, busy, c.get("SQ_INSTS_LDS", 0.0) / mf if mf else 0.0,
                     c.get("SQ_INSTS_VALU", 0.0) / mf if mf else 0.0, c))
    print("| kernel | grid | avg us | clock GHz | MFMA TFLOP/s (MOPS x 512) | MFMA busy | LDS / MFMA inst | VALU / MFMA inst |")
    print("|---|---|---|---|---|---|---|---|")
    for (name, grid), us, ghz, tf, busy, lpm, vpm, _ in rows:
        print(f"| `{name}` | {grid} | {us:.1f} | {ghz:.2f} | {tf:.0f} | {busy * 100:.1f} % | {lpm:.2f} | {vpm:.2f} |")
    print()
    names = sorted({n for *_, c in rows for n in c})
    print("| kernel | grid | " + " | ".join(names) + " |")
    print("|---|---|" + "---|" * len(names))
    for (name, grid), *_, c in rows:
        print(f"| `{name}` | {grid} | " + " | ".join(f"{c[n]:.4g}" if n in c else "" for n in names) + " |")


def stats_summary(d):
    """Markdown table of a rocprofv3 --kernel-trace --stats run
    (--output-format csv): calls, average and total time per kernel.  With
    the run's kernel_trace.csv present, one row per (kernel, grid size), so
    launches of one kernel on different workloads are averaged apart."""
    import csv
    import glob

    def short(name):
        return name if len(name) <= 100 else name[:100] + "…"

    traces = glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)
    if traces:
        groups = {}
        for r in csv.DictReader(open(traces[0])):
            grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
            ns = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            g = groups.setdefault((r["Kernel_Name"], grid), [0, 0])
            g[0] += 1
            g[1] += ns
        total = sum(v[1] for v in groups.values()) or 1
        print("| kernel | grid (threads) | calls | avg us | total us | % |")
        print("|---|---|---|---|---|---|")
        for (name, grid), (n, ns) in sorted(groups.items(), key=lambda kv: -kv[1][1]):
            print(f"| `{short(name)}` | {grid} | {n} | {ns / n / 1e3:.2f} | {ns / 1e3:.1f} | {100.0 * ns / total:.1f} |")
        return
    f = glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True)[0]
    rows = list(csv.DictReader(open(f)))
    print("| kernel | calls | avg us | total us | % |")
    print("|---|---|---|---|---|")
    for r in rows:
        print(f"| `{short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
              f"{float(r['TotalDurationNs']) / 1e3:.1f} | {float(r['Percentage']):.1f} |")


def traffic_summary(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir, copy_mib=256):
    """Markdown table of HBM bytes per dispatch from rocprofv3 --pmc
    FETCH_SIZE and WRITE_SIZE runs (--output-format csv), one directory per
    counter, each scaled by what the same counter reads for a device copy of
    copy_mib MiB (bench.py --copy-calibration)."""
    import csv
    import glob
    from collections import defaultdict

    def means(d, only_fa=True):
        acc = defaultdict(list)
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                name = r["Kernel_Name"]
                if only_fa and "fa::" not in name:
                    continue
                key = (name.split("(")[0].replace("void fa::", "").replace("fa::", ""), int(r.get("Grid_Size", 0)))
                acc[key].append(float(r["Counter_Value"]))
        return {k: sum(v) / len(v) for k, v in acc.items()}

    def copy_kib(d):
        vals = [v for (n, _), v in means(d, only_fa=False).items() if "copyBuffer" in n or "copy" in n.lower()]
        return max(vals) if vals else None

    n = copy_mib * 1024 * 1024
    cf, cw = copy_kib(copy_fetch_dir), copy_kib(copy_write_dir)
    fs, ws = n / (cf * 1024), n / (cw * 1024)
    fetch, write = means(fetch_dir), means(write_dir)
    print(f"Calibration, {copy_mib} MiB device copy: FETCH_SIZE {cf:.0f} KiB per dispatch -> x{fs:.2f} to bytes read; "
          f"WRITE_SIZE {cw:.0f} KiB -> x{ws:.2f} to bytes written.")
    print()
    print("| kernel | grid | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM read MB | HBM write MB | total MB |")
    print("|---|---|---|---|---|---|---|")
    for key in sorted(set(fetch) | set(write), key=lambda k: -fetch.get(k, 0.0)):
        f, w = fetch.get(key, 0.0), write.get(key, 0.0)
        rd, wr = f * 1024 * fs / 1e6, w * 1024 * ws / 1e6
        print(f"| `{key[0]}` | {key[1]} | {f:.0f} | {w:.0f} | {rd:.1f} | {wr:.1f} | {rd + wr:.1f} |")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip decode/varlen side measurements")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 10 device copies of MIB MiB (scales rocprofv3 FETCH/WRITE_SIZE)")
    ap.add_argument("--pmc-summary", nargs="+", metavar="DIR",
                    help="only summarise rocprofv3 --pmc result directories as markdown")
    ap.add_argument("--traffic-summary", nargs=4, metavar=("FETCH", "WRITE", "COPY_FETCH", "COPY_WRITE"),
                    help="only summarise rocprofv3 FETCH_SIZE / WRITE_SIZE csv directories as HBM bytes")
    ap.add_argument("--stats-summary", metavar="DIR",
                    help="only summarise a rocprofv3 --kernel-trace --stats csv directory as markdown")
    ap.add_argument("--decode-only", action="store_true",
                    help="only run the decode measurements (a few calls each) and print them")
    args = ap.parse_args()
    if args.pmc_summary:
        pmc_summary(args.pmc_summary)
        return
    if args.stats_summary:
        stats_summary(args.stats_summary)
        return
    if args.traffic_summary:
        traffic_summary(*args.traffic_summary)
        return
    if args.decode_only:
        print(json.dumps(run_decode_configs(iters=max(1, args.steps))), flush=True)
        return
    if args.copy_calibration:
        n = args.copy_calibration * 1024 * 1024
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "copies": 10}))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: the attention path is single-GPU in this build "
              "(multi-GPU sharding is design-only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    dt, tensors = run_cfg2(args.steps, args.warmup)
    fwd, bwd = cfg2_flops()
    value = (fwd + bwd) / dt / 1e12
    line = {
        "metric": "fwd+bwd TFLOP/s (2x16x2048x128 causal fp16); decode KV-read GB/s",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_min_s": MIN_WARMUP_S,
        "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic N(0,1), seed 0",
        "config": {"workload": "cfg2: causal fwd+bwd B=2 H=16 S=2048 D=128 fp16, bottom-right causal",
                   "global_batch": 2, "seq_len": 2048, "parallelism": "none (1 GPU)"},
        "frac_of_peak": round(value / PEAK_FP16_TFLOPS, 4),
    }
    line["roofline"] = dkdv_roofline(tensors)
    line["cfg2_kernels"] = step_kernel_times(tensors)
    if not args.no_extras:
        ceil = gemm_ceiling()
        line["mfma_gemm_ceiling"] = {
            "value": round(ceil, 1), "unit": "TFLOP/s", "how": "torch.matmul fp16 8192^3 (hipBLASLt)",
            "step_frac": round(value / ceil, 4), "dkdv_frac": round(line["roofline"]["achieved"] / ceil, 4)}
        line["decode"] = run_decode_configs()
        line["cfg5_varlen"] = run_cfg5()
        line["long_causal"] = run_long_causal()
        line["varlen_many"] = run_varlen_many()
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
        line["cpu_baseline_configs"] = cpu_baseline_configs()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
