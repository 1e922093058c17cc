"""Pins the CPU oracle (oracle/attention.py) before anything is checked against it.

Each check is chosen so a plausible slip in the restatement fails it:
  * finite differences of loss = sum(dO*O) against the analytic backward
    (bwd.cu:136-160) catch a wrong formula, sign, missing scale or a swapped
    dK/dQ;
  * torch's scaled_dot_product_attention + autograd in float64 (an independent
    library implementation) catches a wrong scale, mask orientation, GQA head
    map or LSE convention;
  * closed forms (N=1, causal row 0, Q=0, LSE=log(count)) and invariants
    (GQA == MHA on repeat_interleave'd K/V with group-summed grads, head
    permutation equivariance, key permutation invariance, causal tail
    independence) catch indexing slips that happen to cancel elsewhere.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as ora


def rnd(rng, *shape, scale=1.0):
    return rng.standard_normal(shape) * scale


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("hq,hkv", [(2, 2), (4, 2), (3, 1)])
def test_backward_matches_finite_differences(causal, hq, hkv):
    # bwd.cu:136-160: central differences with h = 1e-4, 12 probes cycling
    # over Q, K, V, pass if the relative error is < 1e-4 (published 4e-10).
    rng = np.random.default_rng(4242)
    n, d = 19, 16
    q, do = rnd(rng, 1, hq, n, d), rnd(rng, 1, hq, n, d)
    k, v = rnd(rng, 1, hkv, n, d), rnd(rng, 1, hkv, n, d)
    grads = ora.attention_bwd(q, k, v, do, causal)
    h, worst = 1e-4, 0.0
    for trial in range(12):
        which = trial % 3
        base = [q, k, v]
        idx = int(rng.integers(base[which].size))
        plus = [t.copy() for t in base]
        minus = [t.copy() for t in base]
        plus[which].flat[idx] += h
        minus[which].flat[idx] -= h
        fd = (ora.attention_loss(*plus, do, causal) - ora.attention_loss(*minus, do, causal)) / (2 * h)
        an = grads[which].flat[idx]
        worst = max(worst, abs(fd - an) / max(abs(an), 1e-3))
    assert worst < 1e-4, worst


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("b,hq,hkv,n,d", [(1, 2, 2, 1, 64), (2, 4, 2, 37, 64),
                                          (1, 4, 1, 65, 128), (1, 3, 3, 130, 32)])
def test_matches_torch_sdpa_float64(causal, b, hq, hkv, n, d):
    rng = np.random.default_rng(7)
    q, do = rnd(rng, b, hq, n, d), rnd(rng, b, hq, n, d)
    k, v = rnd(rng, b, hkv, n, d), rnd(rng, b, hkv, n, d)
    o, lse = ora.attention_fwd(q, k, v, causal)
    dq, dk, dv = ora.attention_bwd(q, k, v, do, causal)

    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    to = F.scaled_dot_product_attention(tq, tk, tv, is_causal=causal, enable_gqa=hq != hkv)
    to.backward(torch.tensor(do))
    assert np.allclose(o, to.detach().numpy(), atol=1e-12, rtol=1e-10)
    for mine, theirs in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad)):
        assert np.allclose(mine, theirs.numpy(), atol=1e-11, rtol=1e-9)

    # LSE: natural-log logsumexp of the scaled logits, computed independently.
    ke = np.repeat(k, hq // hkv, axis=1)
    s = torch.tensor(q @ np.swapaxes(ke, -1, -2) / math.sqrt(d))
    if causal:
        s = s.masked_fill(torch.triu(torch.ones(n, n, dtype=torch.bool), 1), float("-inf"))
    assert np.allclose(lse, torch.logsumexp(s, -1).numpy(), atol=1e-12)


def test_closed_forms():
    rng = np.random.default_rng(1)
    d = 64
    # N = 1: the only key is the row itself, O = V and LSE = q.k * scale.
    q, k, v = rnd(rng, 1, 2, 1, d), rnd(rng, 1, 2, 1, d), rnd(rng, 1, 2, 1, d)
    for causal in (False, True):
        o, lse = ora.attention_fwd(q, k, v, causal)
        assert np.allclose(o, v)
        assert np.allclose(lse, (q * k).sum(-1) / math.sqrt(d))
    # Causal row 0 sees only key 0.
    n = 9
    q, k, v = rnd(rng, 1, 2, n, d), rnd(rng, 1, 2, n, d), rnd(rng, 1, 2, n, d)
    o, _ = ora.attention_fwd(q, k, v, True)
    assert np.allclose(o[:, :, 0], v[:, :, 0])
    # Q = 0: uniform weights, O = (prefix) mean of V, LSE = log(count).
    z = np.zeros_like(q)
    o, lse = ora.attention_fwd(z, k, v, False)
    assert np.allclose(o, np.broadcast_to(v.mean(axis=2, keepdims=True), o.shape))
    assert np.allclose(lse, math.log(n))
    o, lse = ora.attention_fwd(z, k, v, True)
    counts = np.arange(1, n + 1)
    assert np.allclose(o, np.cumsum(v, axis=2) / counts[:, None])
    assert np.allclose(lse, np.log(counts))


@pytest.mark.parametrize("causal", [False, True])
def test_gqa_equals_mha_on_expanded_kv(causal):
    rng = np.random.default_rng(3)
    b, hq, hkv, n, d = 2, 6, 2, 23, 64
    q, do = rnd(rng, b, hq, n, d), rnd(rng, b, hq, n, d)
    k, v = rnd(rng, b, hkv, n, d), rnd(rng, b, hkv, n, d)
    ke, ve = np.repeat(k, 3, axis=1), np.repeat(v, 3, axis=1)
    o1, l1 = ora.attention_fwd(q, k, v, causal)
    o2, l2 = ora.attention_fwd(q, ke, ve, causal)
    assert np.allclose(o1, o2) and np.allclose(l1, l2)
    dq1, dk1, dv1 = ora.attention_bwd(q, k, v, do, causal)
    dq2, dk2, dv2 = ora.attention_bwd(q, ke, ve, do, causal)
    assert np.allclose(dq1, dq2)
    assert np.allclose(dk1, dk2.reshape(b, hkv, 3, n, d).sum(2))
    assert np.allclose(dv1, dv2.reshape(b, hkv, 3, n, d).sum(2))
    # head h uses kv head h // 3 (repeat_interleave), not h % hkv
    o_h4, _ = ora.attention_fwd(q[:, 4:5], k[:, 1:2], v[:, 1:2], causal)
    assert np.allclose(o1[:, 4:5], o_h4)


def test_permutations_and_tail_independence():
    rng = np.random.default_rng(5)
    b, h, n, d = 1, 3, 17, 64
    q, k, v, do = (rnd(rng, b, h, n, d) for _ in range(4))
    # Head permutation equivariance.
    perm = np.array([2, 0, 1])
    o, _ = ora.attention_fwd(q, k, v, True)
    op, _ = ora.attention_fwd(q[:, perm], k[:, perm], v[:, perm], True)
    assert np.allclose(op, o[:, perm])
    # Dense attention is invariant to permuting keys together with values;
    # dK/dV permute along.
    kp = rng.permutation(n)
    o, _ = ora.attention_fwd(q, k, v, False)
    o2, _ = ora.attention_fwd(q, k[:, :, kp], v[:, :, kp], False)
    assert np.allclose(o, o2)
    _, dk, dv = ora.attention_bwd(q, k, v, do, False)
    _, dk2, dv2 = ora.attention_bwd(q, k[:, :, kp], v[:, :, kp], do, False)
    assert np.allclose(dk[:, :, kp], dk2) and np.allclose(dv[:, :, kp], dv2)
    # Causal: rows < m do not depend on anything at positions >= m.
    m = 11
    o_full, l_full = ora.attention_fwd(q, k, v, True)
    o_cut, l_cut = ora.attention_fwd(q[:, :, :m], k[:, :, :m], v[:, :, :m], True)
    assert np.allclose(o_full[:, :, :m], o_cut) and np.allclose(l_full[:, :, :m], l_cut)


def test_preprocess_and_metrics():
    rng = np.random.default_rng(9)
    o, do = rnd(rng, 1, 2, 5, 8), rnd(rng, 1, 2, 5, 8)
    assert np.allclose(ora.bwd_preprocess(o, do), np.einsum("bhnd,bhnd->bhn", o, do))
    ref = np.array([3.0, -4.0])                   # RMS = sqrt(12.5)
    got = np.array([3.5, -4.0])
    assert ora.rel_max_rms(got, ref) == pytest.approx(0.5 / math.sqrt(12.5))
    assert ora.rel_l2(got, ref) == pytest.approx(0.5 / 5.0)
    assert ora.max_abs(got, ref) == pytest.approx(0.5)
    # FLOP convention (attention.cu:219, bwd.cu:246) at the headline shape.
    assert ora.fwd_flops(1, 8, 4096, 128, True) == pytest.approx(34.36e9, rel=1e-3)
    assert ora.bwd_flops(1, 8, 4096, 128, True) == pytest.approx(85.90e9, rel=1e-3)


def test_planted_mistakes_are_caught():
    """A wrong scale placement or a transposed GQA map must fail the pins above."""
    rng = np.random.default_rng(11)
    b, hq, hkv, n, d = 1, 4, 2, 12, 64
    q, k, v = rnd(rng, b, hq, n, d), rnd(rng, b, hkv, n, d), rnd(rng, b, hkv, n, d)
    tq, tk, tv = (torch.tensor(x) for x in (q, k, v))
    good = F.scaled_dot_product_attention(tq, tk, tv, is_causal=True, enable_gqa=True).numpy()
    o, _ = ora.attention_fwd(q, k, v, True)
    assert np.allclose(o, good)
    # Planted: kv head chosen by h % hkv (tile) instead of h // G (interleave).
    bad_k, bad_v = np.tile(k, (1, 2, 1, 1)), np.tile(v, (1, 2, 1, 1))
    bad, _ = ora.attention_fwd(q, bad_k, bad_v, True)
    assert not np.allclose(bad, good)
    # Planted: mask orientation flipped (future visible, past hidden).
    bad, _ = ora.attention_fwd(q[:, :, ::-1], k[:, :, ::-1], v[:, :, ::-1], True)
    assert not np.allclose(bad[:, :, ::-1], good)


# ---------------------------------------------------------------------------
# Key lengths (right padding; an extension beyond the reference, which raises
# on padding masks).
@pytest.mark.parametrize("causal", [False, True])
def test_kv_len_pins(causal):
    rng = np.random.default_rng(31)
    b, hq, hkv, n, d = 3, 4, 2, 23, 16
    q, do = rnd(rng, b, hq, n, d), rnd(rng, b, hq, n, d)
    k, v = rnd(rng, b, hkv, n, d), rnd(rng, b, hkv, n, d)
    lens = np.array([n, 9, 1])
    o, lse = ora.attention_fwd(q, k, v, causal, kv_len=lens)
    dq, dk, dv = ora.attention_bwd(q, k, v, do, causal, kv_len=lens)
    # Full length: identical to no key lengths; out-of-range lengths clamp.
    o_full, _ = ora.attention_fwd(q, k, v, causal)
    assert np.array_equal(o[0], o_full[0])
    o_clamp, _ = ora.attention_fwd(q, k, v, causal, kv_len=np.array([n + 5, 9, 0]))
    assert np.array_equal(o_clamp, o)
    for i, L in enumerate(lens):
        # Against attention over the truncated keys, as an independent
        # float64 library routine with explicit masks.
        qb, kb, vb = (torch.tensor(x[i:i + 1]) for x in (q, k, v))
        ke = kb.repeat_interleave(hq // hkv, dim=1)[:, :, :L]
        ve = vb.repeat_interleave(hq // hkv, dim=1)[:, :, :L]
        mask = torch.ones(n, L, dtype=torch.bool)
        if causal:  # key j < L visible to row i when j <= i
            mask = torch.tril(torch.ones(n, n, dtype=torch.bool))[:, :L]
        ref = F.scaled_dot_product_attention(qb, ke, ve, attn_mask=mask)
        assert np.allclose(o[i:i + 1], ref.numpy(), atol=1e-12)
        # Keys past the length get exactly zero gradient.
        assert not np.any(dk[i, :, L:]) and not np.any(dv[i, :, L:])
    # The backward is the gradient of the loss with the same lengths.
    h = 1e-4
    for which, g in ((0, dq), (1, dk), (2, dv)):
        for _ in range(4):
            base = [q, k, v]
            idx = int(rng.integers(base[which].size))
            plus = [t.copy() for t in base]
            minus = [t.copy() for t in base]
            plus[which].flat[idx] += h
            minus[which].flat[idx] -= h
            fd = (ora.attention_loss(*plus, do, causal, kv_len=lens)
                  - ora.attention_loss(*minus, do, causal, kv_len=lens)) / (2 * h)
            assert abs(fd - g.flat[idx]) < 1e-6 * max(1.0, abs(fd))


@pytest.mark.parametrize("window", [1, 5, 23, 40])
def test_sliding_window_pins(window):
    """Sliding window W (causal; an extension): row i sees keys (i - W, i].
    Pinned against torch SDPA with an explicit band mask, W >= N equal to
    plain causal, W = 1 giving O = V row by row, and finite differences."""
    rng = np.random.default_rng(window)
    b, hq, hkv, n, d = 2, 4, 2, 23, 16
    q, do = rnd(rng, b, hq, n, d), rnd(rng, b, hq, n, d)
    k, v = rnd(rng, b, hkv, n, d), rnd(rng, b, hkv, n, d)
    lens = np.array([n, 11])
    o, _ = ora.attention_fwd(q, k, v, True, kv_len=lens, window=window)
    grads = ora.attention_bwd(q, k, v, do, True, kv_len=lens, window=window)
    i, j = np.arange(n)[:, None], np.arange(n)[None, :]
    for e, L in enumerate(lens):
        band = (j <= i) & (j > i - window) & (j < L)
        ke = torch.tensor(np.repeat(k[e:e + 1], hq // hkv, axis=1))
        ve = torch.tensor(np.repeat(v[e:e + 1], hq // hkv, axis=1))
        ref = F.scaled_dot_product_attention(torch.tensor(q[e:e + 1]), ke, ve,
                                             attn_mask=torch.tensor(band)).numpy()
        seen = band.any(axis=1)  # rows with no key at all: O = 0, zero gradients
        assert np.allclose(o[e][:, seen], ref[0][:, seen], atol=1e-12)
        assert not np.any(o[e][:, ~seen]) and not np.any(grads[0][e][:, ~seen])
    if window >= n:
        assert np.array_equal(o, ora.attention_fwd(q, k, v, True, kv_len=lens)[0])
    if window == 1:  # each row sees only itself (entry 0 has every key)
        assert np.allclose(o[0], np.repeat(v, hq // hkv, axis=1)[0], atol=1e-12)
    h = 1e-4
    for which, g in enumerate(grads):
        for _ in range(4):
            base = [q, k, v]
            idx = int(rng.integers(base[which].size))
            plus = [t.copy() for t in base]
            minus = [t.copy() for t in base]
            plus[which].flat[idx] += h
            minus[which].flat[idx] -= h
            fd = (ora.attention_loss(*plus, do, True, kv_len=lens, window=window)
                  - ora.attention_loss(*minus, do, True, kv_len=lens, window=window)) / (2 * h)
            assert abs(fd - g.flat[idx]) < 1e-6 * max(1.0, abs(fd))
    with pytest.raises(ValueError):
        ora.attention_fwd(q, k, v, False, window=window)


def alibi_slopes(h):
    """The ALiBi paper's geometric slopes 2^(-8 i / h), i = 1 .. h."""
    return np.array([2.0 ** (-8.0 * (i + 1) / h) for i in range(h)])


@pytest.mark.parametrize("causal", [False, True])
def test_alibi_pins(causal):
    """ALiBi slopes (an extension): head h adds -slope[h] * |i - j| to every
    scaled logit. Pinned against torch SDPA + autograd in float64 with the
    bias as a float mask, against the causal identity -slope (i - j) ==
    +slope j up to a per-row constant (so a per-key bias gives the same O),
    slope 0 equal to no ALiBi, a huge slope giving O = V row by row (a sign
    slip would pick the farthest key), and finite differences."""
    rng = np.random.default_rng(7 + causal)
    b, hq, hkv, n, d = 2, 4, 2, 21, 16
    q, do = rnd(rng, b, hq, n, d), rnd(rng, b, hq, n, d)
    k, v = rnd(rng, b, hkv, n, d), rnd(rng, b, hkv, n, d)
    slopes = alibi_slopes(hq) * 4  # steep enough that the bias matters at n = 21
    lens = np.array([n, 13])
    o, lse = ora.attention_fwd(q, k, v, causal, kv_len=lens, alibi=slopes)
    grads = ora.attention_bwd(q, k, v, do, causal, kv_len=lens, alibi=slopes)

    i, j = np.arange(n)[:, None], np.arange(n)[None, :]
    tq = torch.tensor(q, requires_grad=True)
    tk = torch.tensor(k, requires_grad=True)
    tv = torch.tensor(v, requires_grad=True)
    bias = -torch.tensor(slopes)[:, None, None] * torch.tensor(np.abs(i - j), dtype=torch.float64)
    keep = torch.tensor(j < lens[:, None, None])[:, None]  # (B, 1, 1, N) key lengths
    if causal:
        keep = keep & torch.tensor(j <= i)
    mask = torch.where(keep, bias[None], torch.tensor(-math.inf, dtype=torch.float64))
    ref = F.scaled_dot_product_attention(tq, tk.repeat_interleave(hq // hkv, 1),
                                         tv.repeat_interleave(hq // hkv, 1), attn_mask=mask)
    ref.backward(torch.tensor(do))
    assert np.allclose(o, ref.detach().numpy(), atol=1e-12)
    for got, t in zip(grads, (tq, tk, tv)):
        assert np.allclose(got, t.grad.numpy(), atol=1e-10)
    ref_lse = torch.logsumexp(
        (tq.detach() @ tk.detach().repeat_interleave(hq // hkv, 1).transpose(-1, -2))
        / math.sqrt(d) + mask, dim=-1).numpy()
    assert np.allclose(lse, ref_lse, atol=1e-12)
    # Planted: a flipped sign or the slopes in reversed head order fail that check.
    for bad_slopes in (-slopes, slopes[::-1].copy()):
        bad, _ = ora.attention_fwd(q, k, v, causal, kv_len=lens, alibi=bad_slopes)
        assert not np.allclose(bad, ref.detach().numpy(), atol=1e-6)

    if causal:  # per-key bias +slope j: same O, LSE shifted by -slope i
        per_key = torch.where(keep, torch.tensor(slopes)[:, None, None]
                              * torch.tensor(j, dtype=torch.float64)[None],
                              torch.tensor(-math.inf, dtype=torch.float64))
        alt = F.scaled_dot_product_attention(
            torch.tensor(q), torch.tensor(k).repeat_interleave(hq // hkv, 1),
            torch.tensor(v).repeat_interleave(hq // hkv, 1), attn_mask=per_key)
        assert np.allclose(o, alt.numpy(), atol=1e-12)
    assert np.array_equal(ora.attention_fwd(q, k, v, causal, kv_len=lens, alibi=np.zeros(hq))[0],
                          ora.attention_fwd(q, k, v, causal, kv_len=lens)[0])
    # Huge slopes: each row keeps its own key only, so O = V (GQA-expanded)
    # and LSE = scaled q_i . k_i.
    o_big, lse_big = ora.attention_fwd(q, k, v, causal, alibi=np.full(hq, 1e4))
    ve = np.repeat(v, hq // hkv, axis=1)
    ke = np.repeat(k, hq // hkv, axis=1)
    assert np.allclose(o_big, ve, atol=1e-12)
    assert np.allclose(lse_big, (q * ke).sum(-1) / math.sqrt(d), atol=1e-12)

    h = 1e-4
    for which, g in enumerate(grads):
        for _ in range(4):
            base = [q, k, v]
            idx = int(rng.integers(base[which].size))
            plus = [t.copy() for t in base]
            minus = [t.copy() for t in base]
            plus[which].flat[idx] += h
            minus[which].flat[idx] -= h
            fd = (ora.attention_loss(*plus, do, causal, kv_len=lens, alibi=slopes)
                  - ora.attention_loss(*minus, do, causal, kv_len=lens, alibi=slopes)) / (2 * h)
            assert abs(fd - g.flat[idx]) < 1e-6 * max(1.0, abs(fd))
    with pytest.raises(ValueError):
        ora.attention_fwd(q, k, v, causal, alibi=slopes[:2])


def test_alibi_with_window_matches_sdpa():
    """ALiBi combined with a sliding window and key lengths, against SDPA."""
    rng = np.random.default_rng(99)
    b, hq, hkv, n, d, w = 2, 2, 1, 17, 8, 6
    q, k, v = rnd(rng, b, hq, n, d), rnd(rng, b, hkv, n, d), rnd(rng, b, hkv, n, d)
    slopes, lens = np.array([0.5, 0.125]), np.array([17, 9])
    o, _ = ora.attention_fwd(q, k, v, True, kv_len=lens, window=w, alibi=slopes)
    i, j = np.arange(n)[:, None], np.arange(n)[None, :]
    for e, L in enumerate(lens):
        band = (j <= i) & (j > i - w) & (j < L)
        seen = band.any(axis=1)
        bias = -slopes[:, None, None] * np.abs(i - j)[None]
        mask = torch.tensor(np.where(band[None], bias, -np.inf))
        ref = F.scaled_dot_product_attention(
            torch.tensor(q[e:e + 1]), torch.tensor(np.repeat(k[e:e + 1], hq, 1)),
            torch.tensor(np.repeat(v[e:e + 1], hq, 1)), attn_mask=mask[None]).numpy()
        assert np.allclose(o[e][:, seen], ref[0][:, seen], atol=1e-12)
        assert not np.any(o[e][:, ~seen])


# ---------------------------------------------------------------------------
# Packed sequences (an extension): several causal sequences in one row.
def test_packed_sequence_pins():
    """Each maximal run of equal segment ids attends within itself only
    (causal and not).
    Pinned by running every sequence alone through the plain causal oracle
    (outputs, LSE and gradients must match row for row), against torch SDPA
    with the block-diagonal causal mask, one run equal to plain causal, the
    run definition (ids need not be sorted: a repeated id after a change is a
    new sequence), with key lengths and a window, and finite differences."""
    rng = np.random.default_rng(31)
    b, hq, hkv, n, d = 2, 4, 2, 23, 16
    q, do = rnd(rng, b, hq, n, d), rnd(rng, b, hq, n, d)
    k, v = rnd(rng, b, hkv, n, d), rnd(rng, b, hkv, n, d)
    seg = np.array([[0] * 5 + [1] * 1 + [2] * 9 + [3] * 8,
                    [7] * 10 + [3] * 6 + [7] * 7])  # entry 1: ids 7, 3, 7 = three runs
    o, lse = ora.attention_fwd(q, k, v, True, segments=seg)
    grads = ora.attention_bwd(q, k, v, do, True, segments=seg)
    runs = {0: [(0, 5), (5, 6), (6, 15), (15, 23)], 1: [(0, 10), (10, 16), (16, 23)]}
    for e, spans in runs.items():
        for a, z in spans:
            sl = (slice(e, e + 1), slice(None), slice(a, z))
            o1, l1 = ora.attention_fwd(q[sl], k[sl], v[sl], True)
            g1 = ora.attention_bwd(q[sl], k[sl], v[sl], do[sl], True)
            assert np.allclose(o[sl], o1, atol=1e-12) and np.allclose(lse[sl], l1, atol=1e-12)
            for got, ref in zip(grads, g1):
                assert np.allclose(got[sl], ref, atol=1e-12)
        i, j = np.arange(n)[:, None], np.arange(n)[None, :]
        run = np.concatenate([[0], np.cumsum(seg[e, 1:] != seg[e, :-1])])
        mask = (j <= i) & (run[:, None] == run[None, :])
        ref = F.scaled_dot_product_attention(
            torch.tensor(q[e:e + 1]), torch.tensor(np.repeat(k[e:e + 1], hq // hkv, 1)),
            torch.tensor(np.repeat(v[e:e + 1], hq // hkv, 1)), attn_mask=torch.tensor(mask))
        assert np.allclose(o[e], ref[0].numpy(), atol=1e-12)
    one = np.zeros((b, n), dtype=np.int64)
    assert np.array_equal(ora.attention_fwd(q, k, v, True, segments=one)[0],
                          ora.attention_fwd(q, k, v, True)[0])
    # Planted: ignoring the packing attends across sequences.
    assert not np.allclose(ora.attention_fwd(q, k, v, True)[0], o, atol=1e-6)
    # With key lengths and a window too: each sequence alone, keys cut at the
    # entry's length and at the window.
    lens = np.array([n, 12])
    o2, _ = ora.attention_fwd(q, k, v, True, kv_len=lens, window=4, segments=seg)
    for e, spans in runs.items():
        for a, z in spans:
            zz = min(z, lens[e]) if a < lens[e] else a
            if zz <= a:
                continue
            sl = (slice(e, e + 1), slice(None), slice(a, zz))
            o1, _ = ora.attention_fwd(q[sl], k[sl], v[sl], True, window=4)
            assert np.allclose(o2[sl], o1, atol=1e-12)
    h = 1e-4
    for which, g in enumerate(grads):
        for _ in range(4):
            base = [q, k, v]
            idx = int(rng.integers(base[which].size))
            plus = [t.copy() for t in base]
            minus = [t.copy() for t in base]
            plus[which].flat[idx] += h
            minus[which].flat[idx] -= h
            fd = (ora.attention_loss(*plus, do, True, segments=seg)
                  - ora.attention_loss(*minus, do, True, segments=seg)) / (2 * h)
            assert abs(fd - g.flat[idx]) < 1e-6 * max(1.0, abs(fd))
    # Without causal masking: each sequence alone, bidirectional, and SDPA
    # with the block-diagonal mask.
    o_nc, lse_nc = ora.attention_fwd(q, k, v, False, segments=seg)
    g_nc = ora.attention_bwd(q, k, v, do, False, segments=seg)
    for e, spans in runs.items():
        for a, z in spans:
            sl = (slice(e, e + 1), slice(None), slice(a, z))
            o1, l1 = ora.attention_fwd(q[sl], k[sl], v[sl], False)
            g1 = ora.attention_bwd(q[sl], k[sl], v[sl], do[sl], False)
            assert np.allclose(o_nc[sl], o1, atol=1e-12) and np.allclose(lse_nc[sl], l1, atol=1e-12)
            for got, ref in zip(g_nc, g1):
                assert np.allclose(got[sl], ref, atol=1e-12)
        run = np.concatenate([[0], np.cumsum(seg[e, 1:] != seg[e, :-1])])
        ref = F.scaled_dot_product_attention(
            torch.tensor(q[e:e + 1]), torch.tensor(np.repeat(k[e:e + 1], hq // hkv, 1)),
            torch.tensor(np.repeat(v[e:e + 1], hq // hkv, 1)),
            attn_mask=torch.tensor(run[:, None] == run[None, :]))
        assert np.allclose(o_nc[e], ref[0].numpy(), atol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_softmax_scale_pins(causal):
    """A softmax scale other than 1/sqrt(D) (an extension): against torch SDPA
    with its own `scale` argument and autograd in float64, the default scale
    equal to no argument, and finite differences (dq, dk carry the scale)."""
    rng = np.random.default_rng(5 + causal)
    b, hq, hkv, n, d, sc = 1, 4, 2, 19, 16, 0.37
    q, do = rnd(rng, b, hq, n, d), rnd(rng, b, hq, n, d)
    k, v = rnd(rng, b, hkv, n, d), rnd(rng, b, hkv, n, d)
    o, lse = ora.attention_fwd(q, k, v, causal, scale=sc)
    grads = ora.attention_bwd(q, k, v, do, causal, scale=sc)
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    ref = F.scaled_dot_product_attention(tq, tk.repeat_interleave(hq // hkv, 1),
                                         tv.repeat_interleave(hq // hkv, 1), is_causal=causal,
                                         scale=sc)
    ref.backward(torch.tensor(do))
    assert np.allclose(o, ref.detach().numpy(), atol=1e-12)
    for got, t in zip(grads, (tq, tk, tv)):
        assert np.allclose(got, t.grad.numpy(), atol=1e-10)
    assert np.array_equal(ora.attention_fwd(q, k, v, causal, scale=1 / math.sqrt(d))[0],
                          ora.attention_fwd(q, k, v, causal)[0])
    assert not np.allclose(ora.attention_fwd(q, k, v, causal)[0], o, atol=1e-6)
    h = 1e-4
    for which, g in enumerate(grads):
        for _ in range(3):
            base = [q, k, v]
            idx = int(rng.integers(base[which].size))
            plus = [t.copy() for t in base]
            minus = [t.copy() for t in base]
            plus[which].flat[idx] += h
            minus[which].flat[idx] -= h
            fd = (ora.attention_loss(*plus, do, causal, scale=sc)
                  - ora.attention_loss(*minus, do, causal, scale=sc)) / (2 * h)
            assert abs(fd - g.flat[idx]) < 1e-6 * max(1.0, abs(fd))


def _fd_check(rng, grads, q, k, v, do, causal, probes=3, **opts):
    h = 1e-4
    for which, g in enumerate(grads):
        for _ in range(probes):
            base = [q, k, v]
            idx = int(rng.integers(base[which].size))
            plus = [t.copy() for t in base]
            minus = [t.copy() for t in base]
            plus[which].flat[idx] += h
            minus[which].flat[idx] -= h
            fd = (ora.attention_loss(*plus, do, causal, **opts)
                  - ora.attention_loss(*minus, do, causal, **opts)) / (2 * h)
            assert abs(fd - g.flat[idx]) < 1e-6 * max(1.0, abs(fd))


@pytest.mark.parametrize("causal", [False, True])
def test_mask_pins(causal):
    """An arbitrary boolean mask (an extension: the reference takes none,
    fa_p100_hf.py:64-70). Pinned against torch SDPA with the same boolean
    attn_mask and autograd in float64 (per-head and head-shared masks); the
    special masks that reduce to features pinned above (lower triangle =
    causal, key columns = kv_len, block diagonal = packed sequences); an
    empty row (o = 0, lse = +inf, no gradient through it); finite
    differences; and a planted transposed mask that SDPA rejects."""
    rng = np.random.default_rng(61 + causal)
    b, hq, hkv, n, d = 2, 4, 2, 21, 16
    q, do = rnd(rng, b, hq, n, d), rnd(rng, b, hq, n, d)
    k, v = rnd(rng, b, hkv, n, d), rnd(rng, b, hkv, n, d)
    i, j = np.arange(n)[:, None], np.arange(n)[None, :]
    mask = rng.random((b, hq, n, n)) < 0.4
    mask |= (i == j)[None, None]  # every row keeps a key (causal too)
    o, lse = ora.attention_fwd(q, k, v, causal, mask=mask)
    grads = ora.attention_bwd(q, k, v, do, causal, mask=mask)
    allowed = mask & (j <= i) if causal else mask
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    ref = F.scaled_dot_product_attention(tq, tk.repeat_interleave(hq // hkv, 1),
                                         tv.repeat_interleave(hq // hkv, 1),
                                         attn_mask=torch.tensor(allowed))
    ref.backward(torch.tensor(do))
    assert np.allclose(o, ref.detach().numpy(), atol=1e-12)
    for got, t in zip(grads, (tq, tk, tv)):
        assert np.allclose(got, t.grad.numpy(), atol=1e-10)
    s = np.matmul(q, np.swapaxes(np.repeat(k, hq // hkv, 1), -1, -2)) / math.sqrt(d)
    s = np.where(allowed, s, -np.inf)
    assert np.allclose(lse, np.log(np.exp(s - s.max(-1, keepdims=True)).sum(-1))
                       + s.max(-1), atol=1e-12)
    _fd_check(rng, grads, q, k, v, do, causal, mask=mask)
    # Planted: the transposed mask gives other values.
    assert not np.allclose(ora.attention_fwd(q, k, v, causal, mask=np.swapaxes(mask, -1, -2))[0],
                           o, atol=1e-6)
    # One plane shared by every head == that plane repeated per head.
    shared = mask[:, :1]
    assert np.array_equal(ora.attention_fwd(q, k, v, causal, mask=shared)[0],
                          ora.attention_fwd(q, k, v, causal,
                                            mask=np.repeat(shared, hq, 1))[0])
    # Special masks: the lower triangle is causal; key columns below kv_len
    # are kv_len; the block diagonal of runs is packed sequences.
    tril = np.broadcast_to(j <= i, (b, 1, n, n))
    for got, want in zip(ora.attention_bwd(q, k, v, do, False, mask=tril),
                         ora.attention_bwd(q, k, v, do, True)):
        assert np.allclose(got, want, atol=1e-12)
    lens = np.array([n, 9])
    cols = (j[None] < lens[:, None, None])[:, None]  # (B, 1, 1, N)
    assert np.allclose(ora.attention_fwd(q, k, v, causal, mask=cols)[0],
                       ora.attention_fwd(q, k, v, causal, kv_len=lens)[0], atol=1e-12)
    seg = np.array([[0] * 6 + [1] * 15, [2] * 13 + [5] * 8])
    block = (seg[:, :, None] == seg[:, None, :])[:, None]
    assert np.allclose(ora.attention_fwd(q, k, v, causal, mask=block)[0],
                       ora.attention_fwd(q, k, v, causal, segments=seg)[0], atol=1e-12)
    # An empty row: o = 0, lse = +inf; the gradients equal those of a run in
    # which that row attends everywhere but receives no upstream gradient.
    e_mask = mask.copy()
    e_mask[1, 2, 7] = False
    o_e, lse_e = ora.attention_fwd(q, k, v, causal, mask=e_mask)
    assert np.all(o_e[1, 2, 7] == 0) and np.isinf(lse_e[1, 2, 7]) and lse_e[1, 2, 7] > 0
    g_e = ora.attention_bwd(q, k, v, do, causal, mask=e_mask)
    f_mask, f_do = mask.copy(), do.copy()
    f_mask[1, 2, 7] = True
    f_do[1, 2, 7] = 0
    g_f = ora.attention_bwd(q, k, v, f_do, causal, mask=f_mask)
    assert np.all(g_e[0][1, 2, 7] == 0)
    for got, want in zip(g_e, g_f):
        assert np.allclose(got, want, atol=1e-12)


def _h32(x):
    """lowbias32 on Python integers (mod 2^32), written out independently."""
    x &= 0xFFFFFFFF
    x ^= x >> 16
    x = (x * 0x7FEB352D) & 0xFFFFFFFF
    x ^= x >> 15
    x = (x * 0x846CA68B) & 0xFFFFFFFF
    return x ^ (x >> 16)


def test_dropout_draw_pins():
    """The dropout keep-bit draw (an extension; the reference has no
    dropout, fa_p100_hf.py:83-85). The vectorised hash equals plain integer
    arithmetic; it avalanches (each input bit flips each output bit about
    half the time); the row keys and draws follow the stated recipe on a few
    hand-computed entries; keep rates match 1 - t/65536 within 5 sigma; and
    neighbouring keys, rows, planes and seeds are uncorrelated."""
    rng = np.random.default_rng(8)
    xs = rng.integers(0, 1 << 32, 4000, dtype=np.uint64).astype(np.uint32)
    got = ora.lowbias32(xs)
    assert all(int(g) == _h32(int(x)) for g, x in zip(got[:500], xs[:500]))
    for bit in range(32):
        flipped = ora.lowbias32(xs ^ np.uint32(1 << bit)) ^ got
        frac = np.unpackbits(flipped.view(np.uint8)).reshape(-1, 32).mean(axis=0)
        assert np.all((frac > 0.4) & (frac < 0.6)), (bit, frac.min(), frac.max())
    # Hand-computed entries of the recipe.
    seed, p, planes, n = 0x0123456789ABCDEF, 0.3, 3, 37
    keep, zs = ora.dropout_keep(seed, p, planes, n)
    t = ora.dropout_threshold(p)
    assert t == round(float(np.float32(0.3)) * 65536) and zs == 65536 / (65536 - t)
    for plane, i, j in [(0, 0, 0), (2, 36, 36), (1, 5, 17), (2, 11, 2)]:
        r = _h32(_h32(_h32(_h32(seed & 0xFFFFFFFF) ^ (seed >> 32)) ^ plane) ^ i)
        u = _h32(r ^ (j // 2))
        draw = (u >> 16) if j % 2 else (u & 0xFFFF)
        assert keep[plane, i, j] == (draw >= t)
    # The causal draw (fa_dropout_bits_causal): keys at or left of the
    # diagonal draw as above, keys past it are cleared.
    kc, _ = ora.dropout_keep(seed, p, planes, n, causal=True)
    for plane, i, j in [(0, 0, 0), (2, 36, 36), (1, 17, 5), (2, 11, 2), (1, 5, 17), (0, 0, 36)]:
        r = _h32(_h32(_h32(_h32(seed & 0xFFFFFFFF) ^ (seed >> 32)) ^ plane) ^ i)
        u = _h32(r ^ (j // 2))
        draw = (u >> 16) if j % 2 else (u & 0xFFFF)
        assert kc[plane, i, j] == (j <= i and draw >= t)
    assert ora.dropout_threshold(0.0) == 0 and ora.dropout_threshold(0.9999999) == 65535
    # Statistics over ~1M draws per rate.
    for p in (0.1, 0.5, 0.9):
        keep, _ = ora.dropout_keep(99, p, 4, 512)
        q_keep = 1 - ora.dropout_threshold(p) / 65536
        n_all = keep.size
        assert abs(keep.mean() - q_keep) < 5 * math.sqrt(q_keep * (1 - q_keep) / n_all)
        z = keep.astype(np.float64) - keep.mean()
        lim = 5 / math.sqrt(n_all / 2)
        for a, b in ((z[:, :, 1:], z[:, :, :-1]), (z[:, 1:], z[:, :-1]), (z[1:], z[:-1])):
            corr = (a * b).mean() / z.var()
            assert abs(corr) < lim, (p, corr)
    k1, _ = ora.dropout_keep(1, 0.5, 2, 256)
    k2, _ = ora.dropout_keep(2, 0.5, 2, 256)
    agree = (k1 == k2).mean()
    assert abs(agree - 0.5) < 0.01


@pytest.mark.parametrize("causal", [False, True])
def test_dropout_attention_pins(causal):
    """Attention with a fixed dropout keep mask: forward and backward
    against torch autograd through o = (softmax(S) * Z * s) V in float64
    (the backward formula of attention_bwd is derived by hand; autograd
    derives its own), GQA included; keep-all with scale 1 equals no
    dropout; finite differences; and a planted slip (dP not dropped) fails."""
    rng = np.random.default_rng(13 + causal)
    b, hq, hkv, n, d = 2, 4, 2, 19, 16
    q, do = rnd(rng, b, hq, n, d), rnd(rng, b, hq, n, d)
    k, v = rnd(rng, b, hkv, n, d), rnd(rng, b, hkv, n, d)
    keep, zs = ora.dropout_keep(2024, 0.25, b * hq, n)
    drop = (keep, zs)
    o, lse = ora.attention_fwd(q, k, v, causal, dropout=drop)
    grads = ora.attention_bwd(q, k, v, do, causal, dropout=drop)
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    s = tq @ tk.repeat_interleave(hq // hkv, 1).transpose(-1, -2) / math.sqrt(d)
    if causal:
        s = s.masked_fill(torch.triu(torch.ones(n, n, dtype=torch.bool), 1), float("-inf"))
    pt = torch.softmax(s, -1)
    ref = (pt * torch.tensor(keep.reshape(b, hq, n, n)) * zs) @ tv.repeat_interleave(hq // hkv, 1)
    ref.backward(torch.tensor(do))
    assert np.allclose(o, ref.detach().numpy(), atol=1e-12)
    assert np.allclose(lse, torch.logsumexp(s, -1).detach().numpy(), atol=1e-12)
    for got, t in zip(grads, (tq, tk, tv)):
        assert np.allclose(got, t.grad.numpy(), atol=1e-10)
    ones = (np.ones_like(keep), 1.0)
    for got, want in zip(ora.attention_bwd(q, k, v, do, causal, dropout=ones),
                         ora.attention_bwd(q, k, v, do, causal)):
        assert np.allclose(got, want, atol=1e-13)
    _fd_check(rng, grads, q, k, v, do, causal, dropout=drop)
    # Planted: dS from the undropped dP misses autograd's dQ.
    p = np.exp(ora._scores(q, ora.expand_kv(k, hq), causal, np.float64) - lse[..., None])
    dp = do @ np.swapaxes(ora.expand_kv(v, hq), -1, -2)
    ds = p * (dp - (o * do).sum(-1)[..., None])
    wrong_dq = ds @ ora.expand_kv(k, hq) / math.sqrt(d)
    assert not np.allclose(wrong_dq, tq.grad.numpy(), atol=1e-6)


@pytest.mark.parametrize("causal", [False, True])
def test_bias_pins(causal):
    """An additive attention bias (an extension; the reference has no bias
    input, HANDOFF.md:281): against torch SDPA with the same float attn_mask
    and autograd in float64, the bias's own gradient included (per-head and
    shared planes, with a boolean mask and ALiBi beside it); a zero bias
    equals none; a bias of -slope |i - j| equals ALiBi; finite differences in
    the bias; and a planted transposed bias fails."""
    rng = np.random.default_rng(71 + causal)
    b, hq, hkv, n, d = 2, 4, 2, 17, 16
    q, do = rnd(rng, b, hq, n, d), rnd(rng, b, hq, n, d)
    k, v = rnd(rng, b, hkv, n, d), rnd(rng, b, hkv, n, d)
    i, j = np.arange(n)[:, None], np.arange(n)[None, :]
    for shape in ((b, hq, n, n), (1, hq, n, n), (b, 1, n, n)):
        bias = rnd(rng, *shape, scale=2.0)
        mask = rng.random((b, 1, n, n)) < 0.8
        mask |= (i == j)[None, None]
        o, lse = ora.attention_fwd(q, k, v, causal, bias=bias, mask=mask)
        dq, dk, dv, ds = ora.attention_bwd(q, k, v, do, causal, bias=bias, mask=mask, dbias=True)
        tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
        tb = torch.tensor(bias, requires_grad=True)
        allowed = torch.tensor(mask & (j <= i) if causal else mask)
        fb = tb.masked_fill(~allowed, float("-inf"))
        ref = F.scaled_dot_product_attention(tq, tk.repeat_interleave(hq // hkv, 1),
                                             tv.repeat_interleave(hq // hkv, 1), attn_mask=fb)
        ref.backward(torch.tensor(do))
        assert np.allclose(o, ref.detach().numpy(), atol=1e-12)
        for got, t in zip((dq, dk, dv), (tq, tk, tv)):
            assert np.allclose(got, t.grad.numpy(), atol=1e-10)
        red = ds.sum(axis=tuple(a for a in (0, 1) if shape[a] == 1), keepdims=True)
        assert np.allclose(red, tb.grad.numpy(), atol=1e-10), shape
    zero = np.zeros((1, 1, n, n))
    assert np.array_equal(ora.attention_fwd(q, k, v, causal, bias=zero)[0],
                          ora.attention_fwd(q, k, v, causal)[0])
    slopes = np.array([0.3, 0.1, 0.05, 0.02])
    as_bias = -slopes[None, :, None, None] * np.abs(i - j)[None, None]
    assert np.allclose(ora.attention_fwd(q, k, v, causal, bias=as_bias)[0],
                       ora.attention_fwd(q, k, v, causal, alibi=slopes)[0], atol=1e-12)
    bias = rnd(rng, b, hq, n, n)
    _, _, _, ds = ora.attention_bwd(q, k, v, do, causal, bias=bias, dbias=True)
    h = 1e-5
    for _ in range(6):
        idx = tuple(int(rng.integers(x)) for x in bias.shape)
        plus, minus = bias.copy(), bias.copy()
        plus[idx] += h
        minus[idx] -= h
        fd = (ora.attention_loss(q, k, v, do, causal, bias=plus)
              - ora.attention_loss(q, k, v, do, causal, bias=minus)) / (2 * h)
        assert abs(fd - ds[idx]) < 1e-6 * max(1.0, abs(fd))
    assert not np.allclose(ora.attention_fwd(q, k, v, causal, bias=np.swapaxes(bias, -1, -2))[0],
                           ora.attention_fwd(q, k, v, causal, bias=bias)[0], atol=1e-6)


def _fd_kv(rng, q, k, v, do, grads, loss_kw, probes=4, tol=1e-6):
    h = 1e-4
    for which, g in enumerate(grads):
        for _ in range(probes):
            base = [q, k, v]
            idx = int(rng.integers(base[which].size))
            plus = [t.copy() for t in base]
            minus = [t.copy() for t in base]
            plus[which].flat[idx] += h
            minus[which].flat[idx] -= h
            fd = (ora.attention_loss(*plus, do, **loss_kw)
                  - ora.attention_loss(*minus, do, **loss_kw)) / (2 * h)
            assert abs(fd - g.flat[idx]) < tol * max(1.0, abs(fd)), (which, fd, g.flat[idx])


@pytest.mark.parametrize("n,nk", [(1, 37), (5, 37), (19, 40), (37, 37), (40, 19), (3, 1)])
def test_kv_rows_pins(n, nk):
    """K/V with nk rows where Q has n (an extension; the reference needs
    q_len == kv_len): causal masking is aligned at the bottom right, as torch
    defines it in torch.nn.attention.bias.causal_lower_right (an independent
    library definition), dense attention ignores the row counts; finite
    differences pin the backward; rows above the first key (n > nk) see
    nothing and get O = 0, LSE = +inf and zero gradients; decoding one row
    is dense attention of that row; a chunk of the last n rows equals those
    rows of the square causal attention over all nk rows, and so do its dK,
    dV when the earlier rows carry no output gradient."""
    from torch.nn.attention.bias import causal_lower_right
    rng = np.random.default_rng(100 * n + nk)
    b, hq, hkv, d = 2, 4, 2, 16
    q, do = rnd(rng, b, hq, n, d), rnd(rng, b, hq, n, d)
    k, v = rnd(rng, b, hkv, nk, d), rnd(rng, b, hkv, nk, d)
    for causal in (False, True):
        o, lse = ora.attention_fwd(q, k, v, causal)
        grads = ora.attention_bwd(q, k, v, do, causal)
        tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
        ke = tk.repeat_interleave(hq // hkv, dim=1)
        ve = tv.repeat_interleave(hq // hkv, dim=1)
        if causal:
            seen = (np.arange(nk)[None, :] <= np.arange(n)[:, None] + nk - n).any(axis=1)
            mask = causal_lower_right(n, nk)
        else:
            seen, mask = np.ones(n, dtype=bool), None
        to = F.scaled_dot_product_attention(tq, ke, ve, attn_mask=mask)
        (to[:, :, torch.tensor(seen)] * torch.tensor(do)[:, :, torch.tensor(seen)]).sum().backward()
        assert np.allclose(o[:, :, seen], to.detach().numpy()[:, :, seen], atol=1e-12)
        assert not np.any(o[:, :, ~seen]) and np.all(lse[:, :, ~seen] == np.inf)
        assert not np.any(grads[0][:, :, ~seen])
        for mine, theirs in zip(grads, (tq.grad, tk.grad, tv.grad)):
            assert np.allclose(mine, theirs.numpy(), atol=1e-11, rtol=1e-9)
        _fd_kv(rng, q, k, v, do, grads, {"causal": causal})
    if n == 1:  # the one row sees every key
        assert np.allclose(ora.attention_fwd(q, k, v, True)[0], ora.attention_fwd(q, k, v, False)[0],
                           atol=1e-14)
    if n <= nk:
        qf = rnd(rng, b, hq, nk, d)
        qf[:, :, nk - n:] = q
        dof = np.zeros((b, hq, nk, d))
        dof[:, :, nk - n:] = do
        of, _ = ora.attention_fwd(qf, k, v, True)
        assert np.allclose(ora.attention_fwd(q, k, v, True)[0], of[:, :, nk - n:], atol=1e-13)
        _, dkf, dvf = ora.attention_bwd(qf, k, v, dof, True)
        _, dk, dv = ora.attention_bwd(q, k, v, do, True)
        assert np.allclose(dk, dkf, atol=1e-12) and np.allclose(dv, dvf, atol=1e-12)


@pytest.mark.parametrize("window", [1, 4, 9])
def test_kv_rows_with_window_alibi_and_key_lengths(window):
    """With nk != n the window and ALiBi count from the bottom-right diagonal
    (row i's diagonal key is i + nk - n) and key lengths clamp to [1, nk]:
    pinned against SDPA with the explicit band and bias built from that
    diagonal, and by finite differences."""
    rng = np.random.default_rng(window)
    b, hq, hkv, n, nk, d = 2, 2, 1, 6, 17, 16
    q, do = rnd(rng, b, hq, n, d), rnd(rng, b, hq, n, d)
    k, v = rnd(rng, b, hkv, nk, d), rnd(rng, b, hkv, nk, d)
    lens, slopes = np.array([nk, 13]), alibi_slopes(hq)
    kw = dict(causal=True, kv_len=lens, window=window, alibi=slopes)
    o, _ = ora.attention_fwd(q, k, v, **kw)
    grads = ora.attention_bwd(q, k, v, do, **kw)
    i, j = np.arange(n)[:, None] + nk - n, np.arange(nk)[None, :]
    for e, L in enumerate(lens):
        band = (j <= i) & (j > i - window) & (j < L)
        bias = -slopes[:, None, None] * np.abs(i - j)[None]
        allowed = np.where(band[None], bias, -np.inf)
        ke = torch.tensor(np.repeat(k[e:e + 1], hq // hkv, axis=1))
        ve = torch.tensor(np.repeat(v[e:e + 1], hq // hkv, axis=1))
        ref = F.scaled_dot_product_attention(torch.tensor(q[e:e + 1]), ke, ve,
                                             attn_mask=torch.tensor(allowed)[None]).numpy()
        seen = band.any(axis=1)
        assert np.allclose(o[e][:, seen], ref[0][:, seen], atol=1e-12)
        assert not np.any(o[e][:, ~seen])
    _fd_kv(rng, q, k, v, do, grads, kw)
    with pytest.raises(ValueError):
        ora.attention_fwd(q, k, v, True, segments=np.zeros((b, n), dtype=np.int64))


# ---------------------------------------------------------------------------
# Block-sparse layouts (an extension; the reference raises on them,
# README.md:72-75).

def test_block_layout_mask_is_the_per_element_rule():
    """Element (i, j) of the expanded mask is the layout's block
    (i // 128, j // 128), checked element by element on a ragged N."""
    rng = np.random.default_rng(5)
    n = 300
    nb = (n + 127) // 128
    lay = rng.random((2, 3, nb, nb)) < 0.5
    m = ora.block_layout_mask(lay, n)
    assert m.shape == (2, 3, n, n)
    for i in range(0, n, 7):
        for j in range(0, n, 5):
            assert (m[:, :, i, j] == lay[:, :, i // 128, j // 128]).all()


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("lb,lh", [(1, 1), (2, 1), (2, 4)])
def test_block_lists_invariants(lb, lh, causal):
    """The lists hold exactly the visible blocks (np.flatnonzero of the
    layout, cut at the diagonal when causal), ascending, padded with valid
    indices; the by-key lists are the transpose of the by-row ones."""
    rng = np.random.default_rng(lb * 10 + lh + causal)
    B, H, Hkv, n = 2, 4, 2, 700
    nb = (n + 127) // 128
    lay = rng.random((lb, lh, nb, nb)) < 0.4
    lay[..., 2, :] = False  # an empty block row
    rows, cols = ora.block_lists(lay, B, H, Hkv, n, causal)
    full = np.broadcast_to(lay, (B, H, nb, nb)) & (
        np.tril(np.ones((nb, nb), dtype=bool)) if causal else True)
    G = H // Hkv
    for b in range(B):
        for h in range(H):
            for r in range(nb):
                want = np.flatnonzero(full[b, h, r])
                c = rows[b, h, r, 0]
                assert c == len(want) and np.array_equal(rows[b, h, r, 1:1 + c], want)
                assert ((rows[b, h, r, 1:] >= 0) & (rows[b, h, r, 1:] < nb)).all()
        for g in range(Hkv):
            for c in range(nb):
                cnt = cols[b, g, c, 0]
                got = cols[b, g, c, 1:1 + cnt]
                assert (np.diff(got) > 0).all()
                pairs = {(f // nb, f % nb) for f in got}
                want = {(hg, r) for hg in range(G) for r in range(nb)
                        if c in rows[b, g * G + hg, r, 1:1 + rows[b, g * G + hg, r, 0]]}
                assert pairs == want
                assert ((cols[b, g, c, 1:] >= 0) & (cols[b, g, c, 1:] < G * nb)).all()
    assert rows[:, :, 2, 0].sum() == 0


def test_block_sparse_attention_is_softmax_over_visible_keys():
    """Forward with an expanded layout equals a per-row softmax over the keys
    the block rule leaves (computed row by row); a row whose block row is
    empty gets o = 0 and lse = +inf."""
    rng = np.random.default_rng(11)
    b, h, n, d = 1, 2, 260, 8
    nb = (n + 127) // 128
    lay = np.array([[[[True, False, True], [False, False, False], [True, True, False]],
                     [[False, True, False], [True, False, True], [False, False, True]]]])
    assert lay.shape == (b, h, nb, nb)
    q, k, v = rnd(rng, b, h, n, d), rnd(rng, b, h, n, d), rnd(rng, b, h, n, d)
    for causal in (False, True):
        o, lse = ora.attention_fwd(q, k, v, causal, mask=ora.block_layout_mask(lay, n))
        for hh in range(h):
            for i in range(0, n, 3):
                keys = [j for j in range(n)
                        if lay[0, hh, i // 128, j // 128] and (not causal or j <= i)]
                if not keys:
                    assert not o[0, hh, i].any() and np.isinf(lse[0, hh, i])
                    continue
                s = q[0, hh, i] @ k[0, hh, keys].T / math.sqrt(d)
                w = np.exp(s - s.max())
                assert np.allclose(o[0, hh, i], (w / w.sum()) @ v[0, hh, keys], atol=1e-12)
                assert math.isclose(lse[0, hh, i], s.max() + math.log(w.sum()), abs_tol=1e-12)
