"""CPU oracle for the FlashAttention-2 forward and backward (test infrastructure).

This module is TEST INFRASTRUCTURE ONLY. It is imported by `tests/`, by
`__graft_entry__.smoke()` (as the checker) and by `bench.py`'s `cpu_baseline`
leg (as the timed CPU restatement). The product path (`fa_p100.flash_attn`, the
torch extension and the C-ABI library) never imports or calls it.

It restates the reference's algorithm in numpy, in float64 by default:

  forward   O = softmax(Q K^T * scale) V, scale = 1/sqrt(D), causal mask col > row
            (fa_p100.py:65-75, attention.cu:72-102); LSE = logsumexp of the
            SCALED logits per row, natural log (flash_fwd.cuh:321-329)
  GQA       query head h reads key/value head h // (Hq/Hkv), i.e.
            repeat_interleave over the head axis (fa_p100.py:58-62,
            flash_fwd.cuh:90)
  preprocess Dv = rowsum(dO * O) (flash_bwd.cuh:65-78)
  backward  P = exp(S*scale - LSE), dV = P^T dO, dP = dO V^T,
            dS = P (dP - Dv), dQ = dS K * scale, dK = dS^T Q * scale
            (bwd.cu:20-69, flash_bwd.cuh:11-16, 267-282, 434-463);
            GQA dK/dV sum over the query heads of a group
  loss      sum(dO * O), whose gradient is exactly the backward above
            (bwd.cu:73-105); used by the finite-difference pin
  metrics   rel = max|got-ref| / RMS(ref) (test_fa_p100.py:35-37), relative
            L2, max-abs

How each function is pinned (tests/test_oracle.py): the backward against
central finite differences of `loss` (bwd.cu:136-160); forward and backward
against torch's own scaled_dot_product_attention + autograd in float64 (an
independent library routine); closed forms (N=1 gives O=V, causal row 0 gives
V_0, Q=0 gives the (prefix) mean of V and LSE=log(count)); GQA equals MHA on
repeat_interleave'd K/V with group-summed dK/dV; permutation equivariance over
heads and key-permutation invariance (dense); causal tail independence.

Block-sparse layouts (an extension; the reference raises on them,
README.md:72-75) are element masks: block_layout_mask expands one into the
`mask` argument, and block_lists restates the int32 lists the kernels step
over (pinned in tests/test_oracle.py against per-element loops and the
lists' own invariants).
"""
import math

import numpy as np

__all__ = [
    "expand_kv", "attention_fwd", "bwd_preprocess", "attention_bwd",
    "attention_loss", "rel_max_rms", "rel_l2", "max_abs", "fwd_flops",
    "bwd_flops", "lowbias32", "dropout_threshold", "dropout_keep",
    "block_layout_mask", "block_lists", "SPARSE_BLOCK",
]


def expand_kv(k, n_head):
    """Repeat each K/V head across the query heads sharing it (fa_p100.py:58-62)."""
    hkv = k.shape[1]
    if hkv == n_head:
        return k
    if n_head % hkv:
        raise ValueError("query heads must be a multiple of kv heads")
    return np.repeat(k, n_head // hkv, axis=1)


def _group_sum(g, hkv):
    """Sum gradients over the query heads that share one K/V head."""
    b, hq, n, d = g.shape
    if hq == hkv:
        return g
    return g.reshape(b, hkv, hq // hkv, n, d).sum(axis=2)


def _scores(q, k, causal, dtype, kv_len=None, window=None, alibi=None, segments=None,
            scale=None, mask=None, bias=None):
    """Scaled logits S*scale with the causal upper triangle set to -inf.

    The scale is applied to the logit after the product, never to Q
    (flash_fwd.cuh:94-101, 220-224). Causal is top-left aligned with
    q_len == kv_len: key col is masked for query row when col > row
    (flash_fwd.cuh:239). With `kv_len` (B ints, an extension: the reference
    has no padding masks) key col is also masked for batch entry b when
    col >= kv_len[b], clamped to [1, N] as the kernels do. With `window` W
    (causal only, another extension) key col is also masked for row when
    col <= row - W: each row sees its last W keys. With `alibi` (Hq slopes,
    another extension) query head h adds -alibi[h] * |row - col| to every
    scaled logit before the masks. With `segments` (B x N ids, another
    extension: packed sequences) each maximal run of equal ids is one
    sequence and key col is masked for row unless both lie in the same run.
    With `mask` (a boolean array broadcastable to (B, Hq, N, N), another
    extension) key col is also masked for row wherever mask[b, h, row, col]
    is False, as torch's scaled_dot_product_attention reads a boolean
    attn_mask. With `bias` (a float array broadcastable to (B, Hq, N, N),
    another extension) it is added to the scaled logits before the masks, as
    SDPA reads a float attn_mask.

    K may hold nk rows where Q holds n (another extension: the reference
    needs q_len == kv_len, fa_p100_hf.py:100-105). The causal diagonal is
    then bottom-right aligned, key col is masked for row when
    col > row + nk - n, and the window and ALiBi distances count from that
    diagonal (row + nk - n against col); key lengths clamp to [1, nk].
    Segments, masks and biases need nk == n.
    """
    d = q.shape[-1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    s = np.matmul(q.astype(dtype), np.swapaxes(k.astype(dtype), -1, -2)) * dtype(scale)
    n, nk = q.shape[-2], k.shape[-2]
    kofs = nk - n
    if kofs and (segments is not None or mask is not None or bias is not None):
        raise ValueError("segments, masks and biases need as many key rows as query rows")
    if alibi is not None:
        slopes = np.asarray(alibi, dtype=np.float64).reshape(-1)
        if slopes.size != q.shape[1]:
            raise ValueError("alibi needs one slope per query head")
        dist = np.abs(np.arange(n)[:, None] + kofs - np.arange(nk)[None, :]).astype(np.float64)
        s = (s - (slopes[:, None, None] * dist[None]).astype(dtype)[None]).astype(dtype)
    if bias is not None:
        s = (s + np.broadcast_to(np.asarray(bias, dtype=np.float64), s.shape)).astype(dtype)
    if causal:
        above = np.triu(np.ones((n, nk), dtype=bool), 1 + kofs)
        s = np.where(above, -np.inf, s).astype(dtype)
    if window is not None:
        if not causal:
            raise ValueError("a sliding window needs causal masking")
        outside = np.tril(np.ones((n, nk), dtype=bool), kofs - int(window))
        s = np.where(outside, -np.inf, s).astype(dtype)
    if segments is not None:
        seg = np.asarray(segments).reshape(q.shape[0], n)
        run = np.concatenate([np.zeros((seg.shape[0], 1), dtype=np.int64),
                              np.cumsum(seg[:, 1:] != seg[:, :-1], axis=1)], axis=1)
        other = run[:, :, None] != run[:, None, :]  # (B, N, N): different sequences
        s = np.where(other[:, None], -np.inf, s).astype(dtype)
    if kv_len is not None:
        lens = np.clip(np.asarray(kv_len).reshape(-1), 1, nk)
        cols = np.arange(nk)[None, :] >= lens[:, None]  # (B, Nk) masked key columns
        s = np.where(cols[:, None, None, :], -np.inf, s).astype(dtype)
    if mask is not None:
        m = np.broadcast_to(np.asarray(mask, dtype=bool), s.shape)
        s = np.where(m, s, -np.inf).astype(dtype)
    return s


def lowbias32(x):
    """C. Wellons' 32-bit integer hash (hash-prospector's `lowbias32`), on
    uint32 arrays with wrap-around multiplies."""
    m32 = np.uint64(0xFFFFFFFF)
    x = np.asarray(x, dtype=np.uint32).astype(np.uint64)
    x = x ^ (x >> np.uint64(16))
    x = (x * np.uint64(0x7FEB352D)) & m32
    x = x ^ (x >> np.uint64(15))
    x = (x * np.uint64(0x846CA68B)) & m32
    return (x ^ (x >> np.uint64(16))).astype(np.uint32)


def dropout_threshold(p):
    """16-bit keep threshold of a drop probability p (a float32, as the C ABI
    takes it): draws >= t are kept; the drop rate is t / 65536."""
    t = np.rint(np.float64(np.float32(p)) * 65536.0)
    return int(min(max(t, 0.0), 65535.0))


def dropout_keep(seed, p, planes, n, causal=False):
    """Keep mask (planes, n, n) of attention dropout, restating the draw that
    include/fa_mi355x.h states for fa_dropout_bits (an extension: the
    reference has no dropout, fa_p100_hf.py:83-85): row key
    r = h(h(h(h(lo) ^ hi) ^ plane) ^ row) of the seed's 32-bit halves, key j
    draws the low (j even) or high (j odd) 16 bits of h(r ^ (j // 2)), and
    is kept iff the draw >= dropout_threshold(p). causal: fa_dropout_bits_causal,
    the same draw with keys j > i of row i cleared. Returns (keep, scale), the
    scale 65536 / (65536 - t) of the kept probabilities."""
    t = dropout_threshold(p)
    seed = int(seed) % (1 << 64)
    lo, hi = np.uint32(seed & 0xFFFFFFFF), np.uint32(seed >> 32)
    base = lowbias32(lowbias32(lowbias32(lo) ^ hi) ^ np.arange(planes, dtype=np.uint32))
    rows = lowbias32(base[:, None] ^ np.arange(n, dtype=np.uint32)[None, :])
    u = lowbias32(rows[:, :, None] ^ np.arange((n + 1) // 2, dtype=np.uint32)[None, None, :])
    draws = np.stack([u & np.uint32(0xFFFF), u >> np.uint32(16)], axis=-1).reshape(planes, n, -1)
    keep = draws[:, :, :n] >= t
    if causal:
        keep &= np.tril(np.ones((n, n), dtype=bool))
    return keep, 65536.0 / (65536 - t)


def _drop_factor(dropout, shape):
    """Z / (1 - p) over (B, Hq, N, N) from dropout = (keep (B*Hq, N, N) or
    broadcastable to (B, Hq, N, N), scale)."""
    keep, zs = dropout
    keep = np.asarray(keep, dtype=bool)
    if keep.ndim == 3:
        keep = keep.reshape(shape)
    return np.broadcast_to(keep, shape) * np.float64(zs)


def attention_fwd(q, k, v, causal=False, dtype=np.float64, kv_len=None, window=None,
                  alibi=None, segments=None, scale=None, mask=None, dropout=None, bias=None):
    """Forward: returns (O, LSE) computed in `dtype`.

    q: (B,Hq,N,D); k, v: (B,Hkv,N,D). O is (B,Hq,N,D) and LSE is (B,Hq,N),
    both in `dtype`. LSE is in natural-log units of the scaled logits
    (flash_fwd.cuh:324-329). `kv_len`, `window`, `alibi`, `segments`, `mask`:
    optional per-entry key lengths, sliding window, ALiBi slopes, packed
    sequence ids, boolean mask and float bias (see _scores). `dropout` = (keep, scale)
    (an extension): O = (P * keep * scale) V with P the softmax over every
    key; LSE is that softmax's, unchanged by dropout.
    """
    hq = q.shape[1]
    k = expand_kv(np.asarray(k), hq)
    v = expand_kv(np.asarray(v), hq)
    s = _scores(np.asarray(q), k, causal, dtype, kv_len, window, alibi, segments, scale, mask,
                bias)
    m = s.max(axis=-1, keepdims=True)
    # A row that sees no key at all (key lengths with a window: pad rows more
    # than W past their entry's length; or a mask row without a set bit) gets
    # O = 0 and LSE = +inf, so that the backward's P = exp(S - LSE) is 0 there
    # too.
    empty = m == -np.inf
    m = np.where(empty, 0, m)
    p = np.exp(s - m)
    l = p.sum(axis=-1, keepdims=True)
    pn = p / np.where(empty, 1, l)
    if dropout is not None:
        pn = pn * _drop_factor(dropout, pn.shape)
    o = np.matmul(pn, v.astype(dtype))
    lse = np.where(empty, np.inf, m + np.log(np.where(empty, 1, l)))[..., 0]
    return o, lse


def bwd_preprocess(o, do, dtype=np.float64):
    """Dv = rowsum(dO * O) per query row (flash_bwd.cuh:65-78)."""
    return (np.asarray(o).astype(dtype) * np.asarray(do).astype(dtype)).sum(axis=-1)


def attention_bwd(q, k, v, do, causal=False, o=None, lse=None, dtype=np.float64, kv_len=None,
                  window=None, alibi=None, segments=None, scale=None, mask=None, dropout=None,
                  bias=None, dbias=False):
    """Analytic backward: returns (dQ, dK, dV) in `dtype`.

    When `o`/`lse` are given they are used as the saved forward state (as the
    kernels do, flash_bwd.cuh:278); otherwise they are recomputed here.
    dK and dQ carry the scale; dV does not (flash_bwd.cuh:442, 457).
    With `dropout` = (keep, scale), F = keep * scale: dV = (P F)^T dO,
    dP = (dO V^T) F, dS = P (dP - rowsum(dO O)) with O the dropped output.
    With dbias=True a fourth result is dS (B, Hq, N, N), the gradient of
    the scaled logits and hence of an additive `bias`.
    """
    q = np.asarray(q)
    hq, hkv = q.shape[1], np.asarray(k).shape[1]
    d = q.shape[-1]
    sc = dtype(1.0 / math.sqrt(d) if scale is None else scale)
    ke = expand_kv(np.asarray(k), hq).astype(dtype)
    ve = expand_kv(np.asarray(v), hq).astype(dtype)
    qd = q.astype(dtype)
    dod = np.asarray(do).astype(dtype)
    if o is None or lse is None:
        o, lse = attention_fwd(q, k, v, causal, dtype, kv_len, window, alibi, segments, scale,
                               mask, dropout, bias)
    s = _scores(q, ke, causal, dtype, kv_len, window, alibi, segments, scale, mask, bias)
    p = np.exp(s - np.asarray(lse).astype(dtype)[..., None])
    f = 1.0 if dropout is None else _drop_factor(dropout, p.shape)
    dv = np.matmul(np.swapaxes(p * f, -1, -2), dod)
    dp = np.matmul(dod, np.swapaxes(ve, -1, -2)) * f
    dvec = bwd_preprocess(o, dod, dtype)
    ds = p * (dp - dvec[..., None])
    dq = np.matmul(ds, ke) * sc
    dk = np.matmul(np.swapaxes(ds, -1, -2), qd) * sc
    if dbias:
        return dq, _group_sum(dk, hkv), _group_sum(dv, hkv), ds
    return dq, _group_sum(dk, hkv), _group_sum(dv, hkv)


def attention_loss(q, k, v, do, causal=False, dtype=np.float64, kv_len=None, window=None,
                   alibi=None, segments=None, scale=None, mask=None, dropout=None, bias=None):
    """Scalar loss sum(dO * O) whose gradient is attention_bwd (bwd.cu:73-105)."""
    o, _ = attention_fwd(q, k, v, causal, dtype, kv_len, window, alibi, segments, scale, mask,
                         dropout, bias)
    return float((o * np.asarray(do).astype(dtype)).sum())


def rel_max_rms(got, ref):
    """max|got - ref| / RMS(ref), the reference suite's metric (test_fa_p100.py:35-37)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(got - ref).max() / math.sqrt(float((ref * ref).mean())))


def rel_l2(got, ref):
    """||got - ref||_2 / ||ref||_2."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm((got - ref).ravel()) / np.linalg.norm(ref.ravel()))


def max_abs(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(got - ref).max())


def fwd_flops(b, hq, n, d, causal):
    """Algorithmic forward FLOPs 4*B*Hq*N^2*D, halved for causal (attention.cu:219)."""
    f = 4.0 * b * hq * n * n * d
    return f / 2 if causal else f


def bwd_flops(b, hq, n, d, causal):
    """Backward FLOPs = 2.5x the forward (bwd.cu:246)."""
    return 2.5 * fwd_flops(b, hq, n, d, causal)


SPARSE_BLOCK = 128  # rows and keys per block of a block-sparse layout


def block_layout_mask(layout, n, block=SPARSE_BLOCK):
    """Element mask (..., n, n) of a block layout (..., nb, nb): query row i
    may attend key j iff layout[..., i // block, j // block] (flash_attn's
    block_mask; pass the result as `mask`)."""
    lay = np.asarray(layout, dtype=bool)
    idx = np.arange(n) // block
    return lay[..., idx[:, None], idx[None, :]]


def block_lists(layout, batch, heads, kv_heads, n, causal=False, block=SPARSE_BLOCK):
    """(rows, cols) of a block layout (B|1, H|1, nb, nb), as int32 arrays
    (batch, heads, nb, nb + 1) and (batch, kv_heads, nb, G*nb + 1), G =
    heads // kv_heads. rows[b, h, r] = [count, visible key blocks of query
    block r ascending, then the last of them repeated (0 if none)];
    cols[b, g, c] = [count, the (query head, query block) pairs that see key
    block c as hg * nb + r (query head g * G + hg) ascending, then the last
    repeated]. causal drops blocks above the diagonal (key block >
    query block) from both."""
    nb = (n + block - 1) // block
    lay = np.broadcast_to(np.asarray(layout, dtype=bool), (batch, heads, nb, nb))
    G = heads // kv_heads
    rows = np.zeros((batch, heads, nb, nb + 1), dtype=np.int32)
    cols = np.zeros((batch, kv_heads, nb, G * nb + 1), dtype=np.int32)
    for b in range(batch):
        for h in range(heads):
            for r in range(nb):
                vis = [c for c in range(nb) if lay[b, h, r, c] and (not causal or c <= r)]
                rows[b, h, r, 0] = len(vis)
                rows[b, h, r, 1:] = (vis + [vis[-1] if vis else 0] * nb)[:nb]
        for g in range(kv_heads):
            for c in range(nb):
                vis = [hg * nb + r for hg in range(G) for r in range(nb)
                       if lay[b, g * G + hg, r, c] and (not causal or c <= r)]
                cols[b, g, c, 0] = len(vis)
                cols[b, g, c, 1:] = (vis + [vis[-1] if vis else 0] * (G * nb))[:G * nb]
    return rows, cols
