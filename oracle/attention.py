"""CPU oracle for the fa_rdna3 attention path (TEST INFRASTRUCTURE ONLY).

A plain numpy (float64) restatement of what the reference computes, used
solely as the checker by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``.  Nothing in the product imports it.

Each function names the reference code it restates
(chelokot/flash-attention-rdna3, paths relative to the repository root):

* ``attention_forward``   - kernels/forward.py:28-164 with the inner loop
  kernels/_common.py:233-345: scores s = q.k * scale, then softcap
  (cap * tanh(s / cap)), additive bias, ALiBi (-slope * |j - i - (Sk - Sq)|),
  then the bottom-right causal / sliding-window mask; softmax per row with
  rows that keep no key giving out = 0 and lse = -inf (forward.py:154-164).
* ``attention_backward``  - kernels/backward.py:18-322 and
  _common.py:347-508: delta = rowsum(O * dO), dP = dO V^T,
  dS = P (dP - delta) * (1 - tanh^2) under softcap, dQ = scale dS K,
  dK = scale dS^T Q, dV = P^T dO (GQA heads summed into their KV head).
* ``varlen_forward`` / ``varlen_backward`` - kernels/varlen.py:21-421:
  the dense functions per sequence of cu_seqlens, with the interval bounded
  to the tensor (varlen.py:21-27).
* ``decode`` - kernels/decode.py:9-125 (non-causal attention of a few query
  rows over a cache), plus the ``cache_seqlens`` key limit of this build.
* ``kvcache_attention`` - no counterpart in the reference (the
  flash_attn_with_kvcache pattern of FlashAttention-2):
  new rows written into a copy of the cache at [len_b, len_b + Snew) below
  the cache size, then ``attention_forward`` of each sequence over its first
  len_b + Snew rows (bottom-right causal when asked).  Pinned by reduction to
  ``decode`` (no new rows, non-causal) and to ``attention_forward`` (full
  cache, causal), each checked against its own vectors.
* ``paged_decode`` - kernels/paged.py:16-89: block-table gather, context
  clamped to table capacity, invalid physical ids contribute nothing.
* ``paged_attention`` - no counterpart in the reference (paged decode of
  several query rows): ``paged_decode`` for Sq query rows per sequence, keys kept at
  their cache positions, bottom-right causal when asked.  Pinned by its
  reduction to ``paged_decode`` (Sq = 1) and to ``kvcache_attention`` over
  the gathered contiguous cache.
* ``decode_num_splits`` / ``paged_num_splits`` / ``alibi_slopes`` -
  interface.py:53-58, :61-77, :136-151.
* ``split_combine`` - decode.py:79-125: LSE-weighted merge of split partials.

Pins (tests/test_oracle.py, tests/test_refs_pin.py): torch float64
autograd, central finite differences, closed forms, the committed golden
vectors and the reference's known answers.  ``varlen_backward`` is pinned by
torch float64 autograd of ragged packed cases, by finite differences of
``varlen_forward`` (out-of-range cu_seqlens included) and by its reduction to
``attention_backward``; ``attention_flops`` by known answers of the
reference's bench convention.

Dropout is not restated (its Philox bitstream is implementation-defined);
tests check it statistically and by finite differences instead.
"""

import math

import numpy as np

NEG_INF = -np.inf


def _f64(x):
    return None if x is None else np.asarray(x, dtype=np.float64)


def _keep_mask(sq, sk, causal, window):
    """Boolean (sq, sk) of kept (query, key) pairs, bottom-right aligned."""
    left, right = window
    i = np.arange(sq)[:, None] + (sk - sq)
    j = np.arange(sk)[None, :]
    keep = np.ones((sq, sk), dtype=bool)
    if causal:
        keep &= j <= i
    if left >= 0:
        keep &= j >= i - left
    if right >= 0:
        keep &= j <= i + right
    return keep


def _logits(q, k, scale, softcap, bias, slope, keep):
    """Modified logits (natural-log domain) of one head; masked = -inf.
    Returns (logits, tanh_term or None)."""
    s = (q @ k.T) * scale
    t = None
    if softcap > 0:
        t = np.tanh(s / softcap)
        s = softcap * t
    if bias is not None:
        s = s + bias
    if slope is not None:
        sq, sk = s.shape
        i = np.arange(sq)[:, None]
        j = np.arange(sk)[None, :]
        s = s - slope * np.abs(j - i - (sk - sq))
    s = np.where(keep, s, NEG_INF)
    return s, t


def _softmax_rows(s):
    """Row softmax with empty rows (all -inf) -> zero probabilities, lse -inf."""
    m = np.max(s, axis=-1, keepdims=True)
    empty = ~np.isfinite(m)
    m_safe = np.where(empty, 0.0, m)
    e = np.exp(s - m_safe)
    e = np.where(np.isneginf(s), 0.0, e)
    den = e.sum(axis=-1, keepdims=True)
    p = np.where(den > 0, e / np.where(den > 0, den, 1.0), 0.0)
    with np.errstate(divide="ignore"):
        lse = np.where(den[..., 0] > 0, m_safe[..., 0] + np.log(np.where(den[..., 0] > 0, den[..., 0], 1.0)),
                       NEG_INF)
    return p, lse


def attention_forward(q, k, v, causal=False, scale=None, window=(-1, -1), softcap=0.0,
                      bias=None, alibi=None):
    """q (B,Hq,Sq,D), k/v (B,Hkv,Sk,D) -> out (B,Hq,Sq,D), lse (B,Hq,Sq)."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    B, Hq, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    g = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    bias = None if bias is None else np.broadcast_to(_f64(bias), (B, Hq, Sq, Sk))
    alibi = _f64(alibi)
    keep = _keep_mask(Sq, Sk, causal, window)
    out = np.zeros((B, Hq, Sq, v.shape[-1]))
    lse = np.zeros((B, Hq, Sq))
    for b in range(B):
        for h in range(Hq):
            s, _ = _logits(q[b, h], k[b, h // g], scale, softcap,
                           None if bias is None else bias[b, h],
                           None if alibi is None else alibi[h], keep)
            p, lse[b, h] = _softmax_rows(s)
            out[b, h] = p @ v[b, h // g]
    return out, lse


def attention_backward(q, k, v, dout, causal=False, scale=None, window=(-1, -1), softcap=0.0,
                       bias=None, alibi=None):
    """Analytic gradients (dq, dk, dv) of sum(out * dout)."""
    q, k, v, dout = _f64(q), _f64(k), _f64(v), _f64(dout)
    B, Hq, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    g = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    bias = None if bias is None else np.broadcast_to(_f64(bias), (B, Hq, Sq, Sk))
    alibi = _f64(alibi)
    keep = _keep_mask(Sq, Sk, causal, window)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    for b in range(B):
        for h in range(Hq):
            kh, vh = k[b, h // g], v[b, h // g]
            s, t = _logits(q[b, h], kh, scale, softcap,
                           None if bias is None else bias[b, h],
                           None if alibi is None else alibi[h], keep)
            p, _ = _softmax_rows(s)
            o = p @ vh
            do = dout[b, h]
            delta = np.sum(o * do, axis=-1, keepdims=True)
            dp = do @ vh.T
            ds = p * (dp - delta)
            if t is not None:
                ds = ds * (1.0 - t * t)
            dq[b, h] = scale * (ds @ kh)
            dk[b, h // g] += scale * (ds.T @ q[b, h])
            dv[b, h // g] += p.T @ do
    return dq, dk, dv


def bounded_intervals(cu, total):
    """(start, length) per sequence, clamped to [0, total] (varlen.py:21-27)."""
    cu = np.asarray(cu, dtype=np.int64)
    out = []
    for i in range(len(cu) - 1):
        s = min(max(int(cu[i]), 0), total)
        e = min(max(int(cu[i + 1]), 0), total)
        out.append((s, max(e - s, 0)))
    return out


def varlen_forward(q, k, v, cu_q, cu_k, causal=False, scale=None, window=(-1, -1), softcap=0.0,
                   alibi=None):
    """q (Tq,Hq,D), k/v (Tk,Hkv,D) -> out (Tq,Hq,D), lse (Hq,Tq).  Rows of no
    sequence are left at zero (the kernels do not write them)."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    out = np.zeros(q.shape[:2] + (v.shape[2],))
    lse = np.full((q.shape[1], q.shape[0]), NEG_INF)
    for (qs, lq), (ks, lk) in zip(bounded_intervals(cu_q, q.shape[0]), bounded_intervals(cu_k, k.shape[0])):
        if lq == 0:
            continue
        qq = q[qs:qs + lq].transpose(1, 0, 2)[None]
        kk = k[ks:ks + lk].transpose(1, 0, 2)[None]
        vv = v[ks:ks + lk].transpose(1, 0, 2)[None]
        if lk == 0:
            continue
        o, l = attention_forward(qq, kk, vv, causal, scale, window, softcap, None, alibi)
        out[qs:qs + lq] = o[0].transpose(1, 0, 2)
        lse[:, qs:qs + lq] = l[0]
    return out, lse


def varlen_backward(q, k, v, dout, cu_q, cu_k, causal=False, scale=None, window=(-1, -1), softcap=0.0,
                    alibi=None):
    """(dq, dk, dv) of sum(out * dout) for packed sequences: the dense
    backward per bounded interval (varlen.py:186-421, dK/dV :193-317 and dQ
    :325-421); rows of no sequence get zero gradient."""
    q, k, v, dout = _f64(q), _f64(k), _f64(v), _f64(dout)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    for (qs, lq), (ks, lk) in zip(bounded_intervals(cu_q, q.shape[0]), bounded_intervals(cu_k, k.shape[0])):
        if lq == 0 or lk == 0:
            continue
        t = lambda x, s, n: x[s:s + n].transpose(1, 0, 2)[None]
        gq, gk, gv = attention_backward(t(q, qs, lq), t(k, ks, lk), t(v, ks, lk), t(dout, qs, lq),
                                        causal, scale, window, softcap, None, alibi)
        dq[qs:qs + lq] += gq[0].transpose(1, 0, 2)
        dk[ks:ks + lk] += gk[0].transpose(1, 0, 2)
        dv[ks:ks + lk] += gv[0].transpose(1, 0, 2)
    return dq, dk, dv


def decode(q, k, v, scale=None, cache_seqlens=None):
    """Non-causal attention of q (B,Hq,Sq,D) over k/v (B,Hkv,Sk,D); sequence b
    sees keys [0, cache_seqlens[b]) when given (a zero-length cache gives 0)."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    B = q.shape[0]
    out = np.zeros(q.shape[:3] + (v.shape[-1],))
    for b in range(B):
        n = k.shape[2] if cache_seqlens is None else min(max(int(cache_seqlens[b]), 0), k.shape[2])
        if n == 0:
            continue
        out[b] = attention_forward(q[b:b + 1], k[b:b + 1, :, :n], v[b:b + 1, :, :n], scale=scale)[0][0]
    return out


def kvcache_attention(q, k_cache, v_cache, k_new=None, v_new=None, cache_seqlens=None, causal=False,
                      scale=None):
    """q (B,Hq,Sq,D); caches (B,Hkv,Sc,D); k_new/v_new (B,Hkv,Snew,D) or None;
    cache_seqlens (B,) or None.  Returns (out, k_cache', v_cache')."""
    q, kc, vc = _f64(q), _f64(k_cache).copy(), _f64(v_cache).copy()
    B, Sc = q.shape[0], kc.shape[2]
    snew = 0 if k_new is None else k_new.shape[2]
    base = np.full(B, Sc) if cache_seqlens is None else np.asarray(cache_seqlens, dtype=np.int64)
    for b in range(B):
        for s in range(snew):
            pos = int(base[b]) + s
            if 0 <= pos < Sc:
                kc[b, :, pos] = _f64(k_new)[b, :, s]
                vc[b, :, pos] = _f64(v_new)[b, :, s]
    out = np.zeros(q.shape[:3] + (vc.shape[-1],))
    for b in range(B):
        n = min(max(int(base[b]) + snew, 0), Sc)
        if n == 0:
            continue
        out[b] = attention_forward(q[b:b + 1], kc[b:b + 1, :, :n], vc[b:b + 1, :, :n], causal=causal,
                                   scale=scale)[0][0]
    return out, kc, vc


def paged_decode(q, k_cache, v_cache, block_table, context_lens, scale=None):
    """q (B,Hq,D); caches (NB,P,Hkv,D); block_table (B,M) int; context_lens (B,)."""
    q, kc, vc = _f64(q), _f64(k_cache), _f64(v_cache)
    bt = np.asarray(block_table, dtype=np.int64)
    B, Hq, D = q.shape
    NB, P, Hkv, _ = kc.shape
    g = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    out = np.zeros((B, Hq, vc.shape[-1]))
    for b in range(B):
        ctx = min(max(int(context_lens[b]), 0), bt.shape[1] * P)
        keys, vals = [], []
        for n in range(ctx):
            phys = int(bt[b, n // P])
            if 0 <= phys < NB:
                keys.append(kc[phys, n % P])
                vals.append(vc[phys, n % P])
        if not keys:
            continue
        kk = np.stack(keys, 0)  # (n, Hkv, D)
        vv = np.stack(vals, 0)
        for h in range(Hq):
            s = (kk[:, h // g] @ q[b, h]) * scale
            p = np.exp(s - s.max())
            p /= p.sum()
            out[b, h] = p @ vv[:, h // g]
    return out


def paged_attention(q, k_cache, v_cache, block_table, context_lens, causal=False, scale=None):
    """q (B,Hq,Sq,D); caches (NB,P,Hkv,D); block_table (B,M); context_lens (B,).
    Key n of sequence b is page block_table[b, n // P], row n % P; keys on
    invalid pages contribute nothing but keep their positions."""
    q, kc, vc = _f64(q), _f64(k_cache), _f64(v_cache)
    bt = np.asarray(block_table, dtype=np.int64)
    B, Hq, Sq, D = q.shape
    NB, P, Hkv, _ = kc.shape
    g = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    out = np.zeros((B, Hq, Sq, vc.shape[-1]))
    for b in range(B):
        ctx = min(max(int(context_lens[b]), 0), bt.shape[1] * P)
        if ctx == 0:
            continue
        phys = bt[b, np.arange(ctx) // P]
        ok = (phys >= 0) & (phys < NB)
        rows = np.arange(ctx) % P
        kk = np.zeros((ctx, Hkv, D))
        vv = np.zeros((ctx, Hkv, vc.shape[-1]))
        kk[ok] = kc[phys[ok], rows[ok]]
        vv[ok] = vc[phys[ok], rows[ok]]
        keep = np.broadcast_to(ok[None, :], (Sq, ctx)).copy()
        if causal:
            keep &= np.arange(ctx)[None, :] <= np.arange(Sq)[:, None] + (ctx - Sq)
        for h in range(Hq):
            s = np.where(keep, (q[b, h] @ kk[:, h // g].T) * scale, NEG_INF)
            p, _ = _softmax_rows(s)
            out[b, h] = p @ vv[:, h // g]
    return out


def split_combine(o_parts, lse_parts):
    """Merge split partials: o_parts (S, ..., D), lse_parts (S, ...)."""
    o_parts, lse_parts = _f64(o_parts), _f64(lse_parts)
    m = np.max(lse_parts, axis=0)
    m_safe = np.where(np.isfinite(m), m, 0.0)
    w = np.where(np.isneginf(lse_parts), 0.0, np.exp(lse_parts - m_safe))
    den = w.sum(axis=0)
    num = (w[..., None] * o_parts).sum(axis=0)
    return num / np.where(den == 0, 1.0, den)[..., None]


def decode_num_splits(batch, heads, seqlen_q, seqlen_k, target_programs=192):
    base = batch * heads * (-(-seqlen_q // 16))
    wanted = -(-target_programs // base)
    return max(1, min(32, wanted, -(-seqlen_k // 64)))


def paged_num_splits(batch, heads, block_size, max_blocks, target_programs,
                     max_context_len=None, requested_splits=None):
    if requested_splits is not None:
        return requested_splits
    if max_context_len is None:
        active_blocks, active_tokens = max_blocks, max_blocks * block_size
    else:
        active_blocks = min(max_blocks, -(-max_context_len // block_size))
        active_tokens = min(max_blocks * block_size, max_context_len)
    if active_tokens <= 64:
        return 1
    cap = min(16, active_blocks, target_programs)
    occupancy = -(-5 * target_programs // (batch * heads))
    work = min(16, -(-active_tokens // 256))
    return min(cap, max(occupancy, work))


def alibi_slopes(n):
    """Press et al. (2021): for n = 2^k, slopes 2^(-8 i / n), i = 1..n."""
    def pow2(m):
        return [2.0 ** (-8.0 * (i + 1) / m) for i in range(m)]
    if n & (n - 1) == 0:
        return np.array(pow2(n))
    lo = 1 << (n.bit_length() - 1)
    return np.array(pow2(lo) + pow2(2 * lo)[0::2][: n - lo])


def attention_flops(batch, heads, seqlen_q, seqlen_k, head_dim, causal):
    """Forward FLOPs by the reference benchmark convention (bench/benchmark.py:32-36)."""
    f = 4.0 * batch * heads * seqlen_q * seqlen_k * head_dim
    return f / 2 if causal else f
