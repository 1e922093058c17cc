"""Key lengths (right padding), beyond the reference, which raises on padding
masks (README.md:72-75, fa_p100_hf.py:64-70): flash_attn(..., kv_len) against
the float64 oracle with the same lengths (oracle pinned in test_oracle.py
against masked torch SDPA and finite differences), bit-identities, and the HF
hook on a right-padded batch against eager attention with the same mask.
Bars are the fp16 ones (helpers.py) and the bf16 ones of test_gpu_bf16.py."""
import numpy as np
import pytest
import torch

from helpers import FWD_MAX_ABS, GRAD_REL_L2, LSE_MAX_ABS, REF_REL, make_inputs, np64
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"


def run(q, k, v, do, causal, lens):
    import fa_p100
    kv_len = torch.tensor(lens, dtype=torch.int32, device=DEV)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal, kv_len=kv_len)
    o.backward(do.to(DEV))
    _, lse = fa_p100._ext.forward_dt(qg.detach(), kg.detach(), vg.detach(), causal, kv_len)
    torch.cuda.synchronize()
    return o, lse, qg.grad, kg.grad, vg.grad


CASES = [(B, Hq, Hkv, N, lens, causal)
         for B, Hq, Hkv, N, lens in [(2, 4, 4, 300, [300, 77]), (3, 8, 2, 1000, [1000, 513, 1]),
                                     (3, 2, 1, 129, [1, 64, 129])]
         for causal in (False, True)] + [(1, 4, 2, 4096, [2049], True)]


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("B,Hq,Hkv,N,lens,causal", CASES)
def test_kv_len_matches_oracle(D, B, Hq, Hkv, N, lens, causal):
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + D + causal)
    o, lse, dq, dk, dv = run(q, k, v, do, causal, lens)
    qn, kn, vn, dn = (t.numpy() for t in (q, k, v, do))
    ref_o, ref_lse = ora.attention_fwd(qn, kn, vn, causal, kv_len=lens)
    what = f"kv_len D{D} {B},{Hq}/{Hkv},N{N} {lens} causal={causal}"
    assert ora.max_abs(np64(o), ref_o) <= FWD_MAX_ABS, what
    assert ora.rel_max_rms(np64(o), ref_o) < REF_REL, what
    assert ora.max_abs(np64(lse), ref_lse) <= LSE_MAX_ABS, what
    ref = ora.attention_bwd(qn, kn, vn, dn, causal, kv_len=lens)
    for name, g, r in zip(("dQ", "dK", "dV"), (dq, dk, dv), ref):
        g = np64(g)
        assert np.isfinite(g).all(), (what, name)
        assert ora.rel_l2(g, r) <= GRAD_REL_L2 and ora.rel_max_rms(g, r) < REF_REL, (what, name)
    for b, L in enumerate(lens):  # keys past the length: exactly zero gradient
        assert not dk[b, :, L:].any() and not dv[b, :, L:].any(), (what, b)


def test_full_lengths_equal_no_lengths_and_bnhd_views_match():
    import fa_p100
    B, Hq, Hkv, N, D = 2, 8, 2, 512, 128
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=5))
    full = torch.full((B,), N, dtype=torch.int32, device=DEV)
    a = fa_p100._ext.forward_dt(q, k, v, True, full)
    b = fa_p100._ext.forward_dt(q, k, v, True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    # (B, N, H, D) views with key lengths: bit-identical to the dense tensors.
    lens = torch.tensor([300, 17], dtype=torch.int32, device=DEV)
    as_bnhd = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)
    dense = [t.clone().requires_grad_(True) for t in (q, k, v)]
    views = [as_bnhd(t).detach().requires_grad_(True) for t in (q, k, v)]
    o1 = fa_p100.flash_attn(*dense, True, kv_len=lens)
    o2 = fa_p100.flash_attn(*views, True, kv_len=lens)
    o1.backward(do)
    o2.backward(as_bnhd(do))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    for x, y in zip(dense, views):
        assert torch.equal(x.grad, y.grad)


def test_kv_len_bf16():
    import fa_p100
    from test_gpu_bf16 import bf16_inputs, check
    lens = [700, 1]
    q, k, v, do = bf16_inputs(2, 4, 2, 700, 128, seed=8)
    kv_len = torch.tensor(lens, dtype=torch.int32, device=DEV)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, True, kv_len=kv_len)
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    # check() compares with the unpadded oracle, so compare entry 0 (full
    # length) there and entry 1 against its own oracle call below.
    check(o[:1], (qg.grad[:1], kg.grad[:1], vg.grad[:1]), None, q[:1], k[:1], v[:1], do[:1],
          True, "bf16 kv_len entry 0")
    f = lambda t: t.detach().float().cpu().double().numpy()
    ref_o, _ = ora.attention_fwd(f(q), f(k), f(v), True, kv_len=lens)
    assert ora.max_abs(f(o)[1], ref_o[1]) <= 2.5e-2


def test_hf_hook_right_padding_matches_eager_with_mask():
    """A right-padded batch through the hook: logits (every position) within
    the eager-vs-sdpa envelope of eager with the same mask, and a training
    step's loss and attention-weight gradients against eager."""
    import fa_p100_hf
    from test_gpu_hf import qwen3
    lens = [384, 250, 37]
    ids = torch.randint(0, 1000, (3, 384), device=DEV, generator=torch.Generator(DEV).manual_seed(4))
    mask = (torch.arange(384, device=DEV)[None, :] < torch.tensor(lens, device=DEV)[:, None]).long()

    def logits(model, impl):
        model.config._attn_implementation = impl
        with torch.no_grad(), torch.autocast("cuda", torch.float16):
            return model(ids, attention_mask=mask).logits.float()

    model = qwen3(2, 512, 8, 2, 64, 1024, 1000).eval()
    eager = logits(model, "eager")
    sdpa = logits(model, "sdpa")
    fa_p100_hf.enable_fa_p100(model)
    fa = logits(model, "fa_p100")
    env, gap = (sdpa - eager).abs(), (fa - eager).abs()
    for b, L in enumerate(lens):  # real positions, then everything
        assert gap[b, :L].mean() <= 2 * env[b, :L].mean() + 1e-4, (b, gap[b, :L].mean().item())
    assert gap.mean() <= 2 * env.mean() + 1e-4
    assert (fa.argmax(-1) == eager.argmax(-1)).float().mean() >= \
        (sdpa.argmax(-1) == eager.argmax(-1)).float().mean() - 0.01

    labels = ids.masked_fill(mask == 0, -100)
    losses, grads = {}, {}
    for impl in ("eager", "fa_p100"):
        m = qwen3(2, 256, 4, 2, 64, 512, 1000, seed=3)
        if impl == "fa_p100":
            fa_p100_hf.enable_fa_p100(m)
        else:
            m.config._attn_implementation = "eager"
        with torch.autocast("cuda", torch.float16):
            out = m(ids % 1000, attention_mask=mask, labels=labels)
        out.loss.backward()
        losses[impl] = out.loss.item()
        grads[impl] = {n: p.grad.float().clone() for n, p in m.named_parameters()
                       if "self_attn" in n and p.grad is not None}
    assert abs(losses["fa_p100"] - losses["eager"]) <= 1e-3 * abs(losses["eager"])
    for n, g in grads["eager"].items():
        rel = ((grads["fa_p100"][n] - g).norm() / g.norm()).item()
        assert rel < 5e-2, (n, rel)


def test_hf_hook_left_and_both_sided_padding_match_eager_with_mask():
    """Left- and both-sided-padded rows through the hook (the pads become a
    packed sequence of their own): logits at every real position within the
    eager-vs-sdpa envelope of eager with the same mask (pad rows, which
    nothing reads, are not compared), with generate()-style position ids
    too, and a training step's loss and attention gradients against eager
    (the loss over real rows only)."""
    import fa_p100_hf
    from test_gpu_hf import qwen3
    N = 320
    spans = [(0, 320), (70, 320), (5, 200), (100, 101)]  # (first, end) of the real tokens
    idx = torch.arange(N, device=DEV)[None, :]
    first = torch.tensor([a for a, _ in spans], device=DEV)[:, None]
    end = torch.tensor([z for _, z in spans], device=DEV)[:, None]
    mask = ((idx >= first) & (idx < end)).long()
    ids = torch.randint(0, 1000, (len(spans), N), device=DEV,
                        generator=torch.Generator(DEV).manual_seed(9))
    gen_pos = (mask.cumsum(-1) - 1).masked_fill(mask == 0, 1)  # what generate() passes

    def logits(model, impl, **kw):
        model.config._attn_implementation = impl
        with torch.no_grad(), torch.autocast("cuda", torch.float16):
            return model(ids, attention_mask=mask, **kw).logits.float()

    model = qwen3(2, 512, 8, 2, 64, 1024, 1000).eval()
    for kw in ({}, {"position_ids": gen_pos}):
        eager, sdpa = logits(model, "eager", **kw), logits(model, "sdpa", **kw)
        fa_p100_hf.enable_fa_p100(model)
        fa = logits(model, "fa_p100", **kw)
        real = mask.bool()
        env, gap = (sdpa - eager).abs()[real], (fa - eager).abs()[real]
        assert gap.mean() <= 2 * env.mean() + 1e-4, (kw.keys(), gap.mean().item())
        for b, (a, z) in enumerate(spans):
            g = (fa - eager).abs()[b, a:z].mean().item()
            e = (sdpa - eager).abs()[b, a:z].mean().item()
            assert g <= 2 * e + 1e-4, (b, g, e)

    # With HF's label shift the last left pad would predict the first real
    # token, putting a pad row (whose output every implementation defines
    # differently: eager lets it see all keys) into the loss; mask that label
    # so the loss reads real rows only.
    labels = ids.masked_fill(mask == 0, -100)
    labels[torch.arange(len(spans), device=DEV), first[:, 0]] = -100
    losses, grads = {}, {}
    for impl in ("eager", "sdpa", "fa_p100"):
        m = qwen3(2, 256, 4, 2, 64, 512, 1000, seed=3)
        if impl == "fa_p100":
            fa_p100_hf.enable_fa_p100(m)
        else:
            m.config._attn_implementation = impl
        with torch.autocast("cuda", torch.float16):
            out = m(ids, attention_mask=mask, labels=labels)
        out.loss.backward()
        losses[impl] = out.loss.item()
        grads[impl] = {n: p.grad.float().clone() for n, p in m.named_parameters()
                       if "self_attn" in n and p.grad is not None}
    assert abs(losses["fa_p100"] - losses["eager"]) <= 1e-3 * abs(losses["eager"])
    for n, g in grads["eager"].items():
        rel = ((grads["fa_p100"][n] - g).norm() / g.norm()).item()
        env_g = ((grads["sdpa"][n] - g).norm() / g.norm()).item()
        assert rel <= max(5e-2, 2 * env_g), (n, rel, env_g)


@pytest.mark.parametrize("padding", ["right", "left"])
def test_hf_hook_padding_under_gradient_checkpointing_matches_eager(padding):
    """Gradient checkpointing re-runs each decoder layer inside backward, after
    the model call has returned; the hook must then see the batch's padding
    again (key lengths for right padding, packed-sequence bounds for left
    padding), or the recomputed layers attend to pad keys and the gradients
    belong to another forward than the loss. Loss and attention-weight
    gradients of a checkpointed training step through the hook against eager
    with the same mask (also checkpointed)."""
    import fa_p100_hf
    from test_gpu_hf import qwen3
    N = 256
    spans = [(0, 256), (0, 131), (40, 256), (9, 200)] if padding == "left" else \
        [(0, 256), (0, 131), (0, 17), (0, 200)]
    idx = torch.arange(N, device=DEV)[None, :]
    first = torch.tensor([a for a, _ in spans], device=DEV)[:, None]
    end = torch.tensor([z for _, z in spans], device=DEV)[:, None]
    mask = ((idx >= first) & (idx < end)).long()
    ids = torch.randint(0, 1000, (len(spans), N), device=DEV,
                        generator=torch.Generator(DEV).manual_seed(21))
    labels = ids.masked_fill(mask == 0, -100)
    labels[torch.arange(len(spans), device=DEV), first[:, 0]] = -100  # see the left-padding test
    losses, grads = {}, {}
    for impl in ("eager", "sdpa", "fa_p100"):
        m = qwen3(2, 256, 4, 2, 64, 512, 1000, seed=5)
        if impl == "fa_p100":
            fa_p100_hf.enable_fa_p100(m)
        else:
            m.config._attn_implementation = impl
        m.gradient_checkpointing_enable()
        m.train()
        with torch.autocast("cuda", torch.float16):
            out = m(ids, attention_mask=mask, labels=labels)
        out.loss.backward()
        losses[impl] = out.loss.item()
        grads[impl] = {n: p.grad.float().clone() for n, p in m.named_parameters()
                       if "self_attn" in n and p.grad is not None}
    assert abs(losses["fa_p100"] - losses["eager"]) <= 1e-3 * abs(losses["eager"])
    for n, g in grads["eager"].items():
        rel = ((grads["fa_p100"][n] - g).norm() / g.norm()).item()
        env_g = ((grads["sdpa"][n] - g).norm() / g.norm()).item()
        assert rel <= max(5e-2, 2 * env_g), (n, rel, env_g)
