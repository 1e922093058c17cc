"""A softmax scale other than 1/sqrt(D) (beyond the reference, which fixes
1/sqrt(D), fa_p100_ext.cu:71, 117, and whose hook raised on any other
scaling): flash_attn(..., softmax_scale=s) against the float64 oracle with
the same scale (pinned in test_oracle.py against torch SDPA's own `scale`
argument and finite differences), and a Qwen3 with a non-default attention
scaling through the hook against eager. Bars: the fp16 ones (helpers.py)."""
import numpy as np
import pytest
import torch

from helpers import FWD_MAX_ABS, GRAD_REL_L2, LSE_MAX_ABS, REF_REL, make_inputs, np64
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D,scale", [(64, 0.05), (128, 0.3)])
def test_softmax_scale_matches_oracle(D, scale, causal):
    """A softmax scale other than 1/sqrt(D) (the reference fixes 1/sqrt(D))."""
    import fa_p100
    B, Hq, Hkv, N = 2, 4, 2, 333
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=D + causal)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal, softmax_scale=scale)
    o.backward(do.to(DEV))
    _, lse = fa_p100._ext.forward_dt(qg.detach(), kg.detach(), vg.detach(), causal, None, 0,
                                     None, None, None, scale)
    torch.cuda.synchronize()
    qn, kn, vn, dn = (t.float().numpy() for t in (q, k, v, do))
    ref_o, ref_lse = ora.attention_fwd(qn, kn, vn, causal, scale=np.float32(scale).item())
    assert ora.max_abs(np64(o), ref_o) <= FWD_MAX_ABS
    assert ora.max_abs(np64(lse), ref_lse) <= LSE_MAX_ABS
    ref = ora.attention_bwd(qn, kn, vn, dn, causal, scale=np.float32(scale).item())
    for name, g, r in zip(("dQ", "dK", "dV"), (qg.grad, kg.grad, vg.grad), ref):
        l2, rr = ora.rel_l2(np64(g), r), ora.rel_max_rms(np64(g), r)
        assert l2 <= GRAD_REL_L2 and rr < REF_REL, (name, l2, rr)
    with pytest.raises(ValueError, match="softmax_scale"):
        fa_p100.flash_attn(qg, kg, vg, causal, softmax_scale=-1.0)


def test_hf_hook_custom_scaling_matches_eager():
    """A model whose attention scale is not 1/sqrt(D) (the reference's hook
    raised): Qwen3 with every attention module's scaling set to 0.05, logits
    within the eager-vs-sdpa envelope of eager."""
    import fa_p100_hf
    from test_gpu_hf import qwen3
    ids = torch.randint(0, 1000, (2, 260), device=DEV, generator=torch.Generator(DEV).manual_seed(12))
    model = qwen3(2, 512, 8, 2, 64, 1024, 1000).eval()
    for m in model.modules():
        if hasattr(m, "scaling"):
            m.scaling = 0.05

    def logits(impl):
        model.config._attn_implementation = impl
        with torch.no_grad(), torch.autocast("cuda", torch.float16):
            return model(ids).logits.float()

    eager, sdpa = logits("eager"), logits("sdpa")
    fa_p100_hf.enable_fa_p100(model)
    fa = logits("fa_p100")
    env, gap = (sdpa - eager).abs(), (fa - eager).abs()
    assert gap.mean() <= 2 * env.mean() + 1e-4, (gap.mean().item(), env.mean().item())


def _check_all(o, lse, grads, q, k, v, do, causal, scale, what, **opts):
    qn, kn, vn, dn = (t.float().numpy() for t in (q, k, v, do))
    sc = np.float32(scale).item()
    ref_o, ref_lse = ora.attention_fwd(qn, kn, vn, causal, scale=sc, **opts)
    assert ora.max_abs(np64(o), ref_o) <= FWD_MAX_ABS, what
    assert ora.rel_max_rms(np64(o), ref_o) < REF_REL, what
    assert ora.max_abs(np64(lse), ref_lse) <= LSE_MAX_ABS, what
    ref = ora.attention_bwd(qn, kn, vn, dn, causal, scale=sc, **opts)
    for name, g, r in zip(("dQ", "dK", "dV"), grads, ref):
        l2, rr = ora.rel_l2(np64(g), r), ora.rel_max_rms(np64(g), r)
        assert l2 <= GRAD_REL_L2 and rr < REF_REL, (what, name, l2, rr)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D,scale", [(64, 0.07), (128, 0.2)])
def test_softmax_scale_with_alibi_matches_oracle(D, scale, causal):
    """A custom softmax scale together with ALiBi slopes: the kernels divide
    each slope by the scale to subtract the bias from the raw score, so a
    wrong pairing of the two (bias in raw units, or scaled twice) shows here.
    Forward, LSE and gradients against the float64 oracle (whose ALiBi is in
    units of the scaled logits, pinned against SDPA with a float mask)."""
    import fa_p100
    B, Hq, Hkv, N = 2, 4, 2, 301
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=7 * D + causal)
    slopes = np.array([2.0 ** (-8.0 * (i + 1) / Hq) for i in range(Hq)]) * 4.0
    al = torch.tensor(slopes, dtype=torch.float32, device=DEV)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal, alibi_slopes=al, softmax_scale=scale)
    o.backward(do.to(DEV))
    _, lse = fa_p100._ext.forward_dt(qg.detach(), kg.detach(), vg.detach(), causal, None, 0, al,
                                     None, None, scale)
    torch.cuda.synchronize()
    _check_all(o, lse, (qg.grad, kg.grad, vg.grad), q, k, v, do, causal, scale,
               f"scale+alibi D={D} causal={causal}",
               alibi=np.float32(slopes).astype(np.float64))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D,scale", [(64, 0.3), (128, 0.06)])
def test_softmax_scale_with_packed_sequences_matches_oracle(D, scale, causal):
    """A custom softmax scale on packed sequences (block-diagonal masking,
    causal within each sequence or not), against the float64 oracle."""
    import fa_p100
    B, Hq, Hkv, N = 2, 4, 1, 400
    lengths = [130, 1, 64, 205]
    seg = np.concatenate([np.full(n, i) for i, n in enumerate(lengths)])
    seg = np.stack([seg, seg[::-1].copy()])
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=11 * D + causal)
    sid = torch.tensor(seg, device=DEV)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal, segment_ids=sid, softmax_scale=scale)
    o.backward(do.to(DEV))
    s0, s1 = fa_p100.segment_bounds(sid)
    _, lse = fa_p100._ext.forward_dt(qg.detach(), kg.detach(), vg.detach(), causal, None, 0,
                                     None, s0, s1, scale)
    torch.cuda.synchronize()
    _check_all(o, lse, (qg.grad, kg.grad, vg.grad), q, k, v, do, causal, scale,
               f"scale+packed D={D} causal={causal}", segments=seg)
