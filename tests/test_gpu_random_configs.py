"""Seeded random configurations that cross every option at once.

The other GPU tests cover each option on its own and in hand-picked sets;
here 560 seeded draws combine them: batch 1-2, MHA/GQA/MQA, N from 1 to 320,
any head dim that is a multiple of 8 up to 128, causal or not, fp16 or bf16,
dense (B, H, N, D) tensors or views of (B, N, H, D) storage, and a random
subset of key lengths, a sliding window (causal only), ALiBi, a softmax
scale, packed sequences, a boolean mask (shared or per head), dropout and an
additive bias with its gradient. Each is checked against the float64 oracle
(its options pinned in test_oracle.py) to the fp16 bars of helpers.py or
the bf16 bars of test_gpu_bf16.py: o, LSE, dQ, dK, dV and dbias."""
import numpy as np
import pytest
import torch

from helpers import FWD_MAX_ABS, GRAD_REL_L2, LSE_MAX_ABS, REF_REL, np64
from oracle import attention as ora
from test_gpu_bf16 import BF_ELEM_REL, BF_FWD_MAX_ABS, BF_GRAD_REL_L2, BF_LSE_MAX_ABS, rel_elem

pytestmark = pytest.mark.gpu

DEV = "cuda"
N_CASES = 560
OPTIONS = ("kv_len", "window", "alibi", "scale", "segments", "mask", "dropout", "bias")


def config(i):
    rng = np.random.default_rng(1000 + i)
    hkv = int(rng.choice([1, 2]))
    causal = bool(rng.random() < 0.6)
    opts = [o for o in OPTIONS if rng.random() < 0.35 and (o != "window" or causal)]
    return dict(B=int(rng.integers(1, 3)), Hq=hkv * int(rng.choice([1, 2, 4])), Hkv=hkv,
                N=int(rng.integers(1, 321)), D=8 * int(rng.integers(1, 17)), causal=causal,
                bf16=bool(rng.random() < 0.3), bnhd=bool(rng.random() < 0.3), opts=opts)


def as_bnhd(t):
    return t.transpose(1, 2).contiguous().transpose(1, 2)


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_configuration_matches_oracle(i):
    import fa_p100
    c = config(i)
    B, Hq, Hkv, N, D, causal, opts = (c[k] for k in ("B", "Hq", "Hkv", "N", "D", "causal", "opts"))
    what = f"case {i}: {c}"
    rng = np.random.default_rng(2000 + i)
    g = torch.Generator().manual_seed(i)
    dt = torch.bfloat16 if c["bf16"] else torch.float16
    shapes = ((B, Hq, N, D), (B, Hkv, N, D), (B, Hkv, N, D), (B, Hq, N, D))
    q, k, v, do = (torch.randn(*s, generator=g).to(dt) for s in shapes)

    kw, lse_kw, ora_kw, zs = {}, {}, {}, 1.0
    if "kv_len" in opts:
        lens = [int(rng.integers(1, N + 1)) for _ in range(B)]
        kw["kv_len"] = lse_kw["kv_len"] = torch.tensor(lens, dtype=torch.int32, device=DEV)
        ora_kw["kv_len"] = lens
    if "window" in opts:
        w = int(rng.integers(1, N + 1))
        kw["sliding_window"], lse_kw["window"], ora_kw["window"] = w, w, w
    if "alibi" in opts:
        slopes = np.float32(rng.uniform(0.01, 0.5, Hq))
        kw["alibi_slopes"] = lse_kw["alibi_slopes"] = torch.tensor(slopes, device=DEV)
        ora_kw["alibi"] = slopes.astype(np.float64)
    if "scale" in opts:
        s = float(rng.uniform(0.03, 0.3))
        kw["softmax_scale"], lse_kw["scale"] = s, s
        ora_kw["scale"] = np.float32(s).item()
    if "segments" in opts:
        ids = np.sort(rng.integers(0, 4, (B, N)), axis=1)  # up to four packed sequences
        sid = torch.tensor(ids, device=DEV)
        kw["segment_ids"] = sid
        lse_kw["seg_start"], lse_kw["seg_end"] = fa_p100.segment_bounds(sid)
        ora_kw["segments"] = ids
    if "mask" in opts:
        heads = Hq if rng.random() < 0.5 else 1
        mask = rng.random((B, heads, N, N)) < 0.85
        kw["attn_mask"] = torch.tensor(mask, device=DEV)
        lse_kw["mask"] = fa_p100.pack_mask(kw["attn_mask"], B, Hq)[0]
        ora_kw["mask"] = mask
    if "dropout" in opts:
        p, seed = float(rng.choice([0.1, 0.3])), int(rng.integers(0, 2 ** 62))
        kw.update(dropout_p=p, dropout_seed=seed)
        ora_kw["dropout"] = ora.dropout_keep(seed, p, B * Hq, N)
        zs = ora_kw["dropout"][1]
    bias = bg = None
    if "bias" in opts:
        shape = [(1, Hq, N, N), (B, 1, N, N), (N, N)][int(rng.integers(0, 3))]
        bias = torch.randn(*shape, generator=g)
        b4 = bias.reshape((1, 1, N, N)) if bias.dim() == 2 else bias
        bg = bias.to(DEV).requires_grad_(True)
        lse_kw["bias"] = b4.to(DEV)
        ora_kw["bias"] = b4.double().numpy()

    lay = as_bnhd if c["bnhd"] else (lambda t: t)
    leaves = [lay(t.to(DEV)).detach().requires_grad_(True) for t in (q, k, v)]
    o = fa_p100.flash_attn(*leaves, causal, attn_bias=bg, **kw)
    o.backward(lay(do.to(DEV)))
    _, lse = fa_p100._ext.forward_dt(q.to(DEV), k.to(DEV), v.to(DEV), causal, **lse_kw)
    torch.cuda.synchronize()

    f = lambda t: t.float().numpy()
    ref_o, ref_lse = ora.attention_fwd(f(q), f(k), f(v), causal, **ora_kw)
    got_o = np64(o)
    seen = np.isfinite(ref_lse)
    if c["bf16"]:
        assert ora.max_abs(got_o, ref_o) <= BF_FWD_MAX_ABS * zs, what
        assert ora.max_abs(np64(lse)[seen], ref_lse[seen]) <= BF_LSE_MAX_ABS, what
    else:
        assert ora.max_abs(got_o, ref_o) <= FWD_MAX_ABS * zs, what
        assert ora.rel_max_rms(got_o, ref_o) < REF_REL, what
        assert ora.max_abs(np64(lse)[seen], ref_lse[seen]) <= LSE_MAX_ABS, what
    # The backward consumes the forward's saved o and LSE, as the kernels do.
    ref = ora.attention_bwd(f(q), f(k), f(v), f(do), causal, o=got_o, lse=np64(lse),
                            dbias=bias is not None, **ora_kw)
    got = [t.grad for t in leaves]
    want = list(ref[:3])
    if bias is not None:
        ds = ref[3]
        red = ds.sum(axis=tuple(a for a in (0, 1) if b4.shape[a] == 1), keepdims=True)
        got.append(bg.grad)
        want.append(red.reshape(tuple(bias.shape)))
    for label, gt, r in zip(("dQ", "dK", "dV", "dbias"), got, want):
        gt = np64(gt)
        assert gt.shape == r.shape, (what, label)
        assert np.isfinite(gt).all(), (what, label)
        if not np.any(r):
            # An exact-zero reference: every row masked away, or (dQ, dbias)
            # every row left with one key, where dS = P (dP - Dv) cancels
            # exactly in float64 and to fp32 rounding in the kernels (dP and
            # Dv are the same dot product summed in different orders).
            # Wrong gradients are of order one here.
            assert ora.max_abs(gt, r) <= 1e-4, (what, label, ora.max_abs(gt, r))
            continue
        l2 = ora.rel_l2(gt, r)
        if c["bf16"]:
            assert l2 <= BF_GRAD_REL_L2 and rel_elem(gt, r) <= BF_ELEM_REL, (what, label, l2)
        else:
            rr = ora.rel_max_rms(gt, r)
            assert l2 <= GRAD_REL_L2 and rr < REF_REL, (what, label, l2, rr)
