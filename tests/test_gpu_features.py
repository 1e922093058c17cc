"""Every set of optional per-score inputs on every kernel width.

The kernels keep one copy per set of those inputs (a bit-packed mask,
dropout keep bits, both, or an additive bias with the other two as run-time
options) and compile each at the widths 32, 64, 96 and 128. Each copy reads
its operands its own way: the backward's feature copies read K from LDS, and
the bias forward stages Q through LDS. Here each set runs at head dims 24,
64, 80 and 128 (widths 32, 64, 96, 128; 24 and 80 with padded columns),
causal or not, with GQA and a ragged N, against the float64 oracle (its
mask, dropout and bias pinned in test_oracle.py): o, LSE, dQ, dK, dV and
dbias, to the fp16 bars of helpers.py."""
import numpy as np
import pytest
import torch

from helpers import FWD_MAX_ABS, GRAD_REL_L2, LSE_MAX_ABS, REF_REL, make_inputs, np64
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"
SETS = {"mask": ("mask",), "dropout": ("drop",), "mask+dropout": ("mask", "drop"),
        "bias+mask+dropout": ("bias", "mask", "drop"), "bias": ("bias",)}


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D", [24, 64, 80, 128])
@pytest.mark.parametrize("name", list(SETS))
def test_option_set_at_every_width(name, D, causal):
    import fa_p100
    feats = SETS[name]
    B, Hq, Hkv, N = 2, 4, 2, 203
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=D + 3 * causal + len(name))
    rng = np.random.default_rng(D + len(name))
    kw, opts, zs = {}, {}, 1.0
    if "mask" in feats:
        mask = rng.random((B, 1, N, N)) < 0.8
        mask[0, 0, 5] = False  # a row with no key
        kw["attn_mask"] = torch.tensor(mask, device=DEV)
        opts["mask"] = mask
    if "drop" in feats:
        p, seed = 0.2, 11 + D
        kw.update(dropout_p=p, dropout_seed=seed)
        opts["dropout"] = ora.dropout_keep(seed, p, B * Hq, N)
        zs = opts["dropout"][1]
    bias = bg = None
    if "bias" in feats:
        bias = torch.randn(1, Hq, N, N, generator=torch.Generator().manual_seed(D)) * 1.5
        bg = bias.to(DEV).requires_grad_(True)
        opts["bias"] = bias.double().numpy()
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal, attn_bias=bg, **kw)
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    # The LSE (which dropout leaves unchanged) from the forward with the same
    # mask and bias.
    lkw = {}
    if "mask" in feats:
        lkw["mask"] = fa_p100.pack_mask(kw["attn_mask"], B, Hq)[0]
    if bias is not None:
        lkw["bias"] = bias.to(DEV)
    _, lse = fa_p100._ext.forward_dt(q.to(DEV), k.to(DEV), v.to(DEV), causal, **lkw)

    what = f"{name} D{D} causal={causal}"
    qn, kn, vn, dn = (t.float().numpy() for t in (q, k, v, do))
    ref_o, ref_lse = ora.attention_fwd(qn, kn, vn, causal, **opts)
    assert ora.max_abs(np64(o), ref_o) <= FWD_MAX_ABS * zs, what
    assert ora.rel_max_rms(np64(o), ref_o) < REF_REL, what
    seen = np.isfinite(ref_lse)
    assert ora.max_abs(np64(lse)[seen], ref_lse[seen]) <= LSE_MAX_ABS, what
    # The backward consumes the forward's saved state (the fp16-rounded o in
    # Dv = rowsum(dO o)), as the kernels and the reference do
    # (flash_bwd.cuh:65-78).
    ref = ora.attention_bwd(qn, kn, vn, dn, causal, o=np64(o), lse=np64(lse),
                            dbias=bias is not None, **opts)
    got = [qg.grad, kg.grad, vg.grad]
    want = list(ref[:3])
    if bias is not None:
        got.append(bg.grad)
        want.append(ref[3].sum(axis=0, keepdims=True))
    for label, g, r in zip(("dQ", "dK", "dV", "dbias"), got, want):
        g = np64(g)
        assert g.shape == r.shape, (what, label)
        assert np.isfinite(g).all(), (what, label)
        l2, rr = ora.rel_l2(g, r), ora.rel_max_rms(g, r)
        assert l2 <= GRAD_REL_L2 and rr < REF_REL, (what, label, l2, rr)
