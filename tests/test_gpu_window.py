"""Causal sliding windows (beyond the reference, which raises on them,
README.md:72-75, fa_p100_hf.py:78-82): row i attends to keys (i - W, i].
flash_attn(..., sliding_window=W) against the float64 oracle with the same
window (pinned in test_oracle.py against torch SDPA with a band mask and
finite differences), with key lengths too (rows that see no key give zeros),
in bf16, and a Qwen3 model with sliding-window layers through the hook
against eager attention. Bars: the fp16 ones (helpers.py)."""
import numpy as np
import pytest
import torch

from helpers import FWD_MAX_ABS, GRAD_REL_L2, LSE_MAX_ABS, REF_REL, make_inputs, np64
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"


def run(q, k, v, do, window, lens=None):
    import fa_p100
    kv_len = None if lens is None else torch.tensor(lens, dtype=torch.int32, device=DEV)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, True, kv_len=kv_len, sliding_window=window)
    o.backward(do.to(DEV))
    _, lse = fa_p100._ext.forward_dt(qg.detach(), kg.detach(), vg.detach(), True, kv_len, window)
    torch.cuda.synchronize()
    return o, lse, qg.grad, kg.grad, vg.grad


def check(got, q, k, v, do, window, lens, what):
    o, lse, dq, dk, dv = got
    qn, kn, vn, dn = (t.float().numpy() for t in (q, k, v, do))
    ref_o, ref_lse = ora.attention_fwd(qn, kn, vn, True, kv_len=lens, window=window)
    assert ora.max_abs(np64(o), ref_o) <= FWD_MAX_ABS, what
    assert ora.rel_max_rms(np64(o), ref_o) < REF_REL, what
    seen = np.isfinite(ref_lse)  # rows with no key: lse +inf in both
    assert np.array_equal(np.isfinite(np64(lse)), seen), what
    assert ora.max_abs(np64(lse)[seen], ref_lse[seen]) <= LSE_MAX_ABS, what
    ref = ora.attention_bwd(qn, kn, vn, dn, True, kv_len=lens, window=window)
    for name, g, r in zip(("dQ", "dK", "dV"), (dq, dk, dv), ref):
        g = np64(g)
        assert np.isfinite(g).all(), (what, name)
        if not np.any(r):
            # W = 1: each row sees one key, so dQ = dK = 0 exactly; the kernels
            # get dP - Dv (two fp32 sums of D products of size ~1 that differ
            # only in order) to ~1e-6.
            assert np.abs(g).max() <= 1e-5, (what, name)
            continue
        assert ora.rel_l2(g, r) <= GRAD_REL_L2 and ora.rel_max_rms(g, r) < REF_REL, (what, name)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("B,Hq,Hkv,N,window", [(2, 4, 4, 300, 1), (2, 4, 4, 300, 37),
                                               (2, 4, 4, 300, 128), (2, 4, 4, 300, 1000),
                                               (1, 8, 2, 1000, 257), (1, 4, 2, 4096, 1024),
                                               (1, 2, 1, 129, 64)])
def test_window_matches_oracle(D, B, Hq, Hkv, N, window):
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + D + window)
    got = run(q, k, v, do, window)
    check(got, q, k, v, do, window, None, f"W{window} D{D} {B},{Hq}/{Hkv},N{N}")


@pytest.mark.parametrize("D", [64, 128])
def test_window_with_key_lengths(D):
    """Pad rows more than W past their entry's length see no key: o = 0,
    lse = +inf, zero gradients (the oracle's convention)."""
    B, Hq, Hkv, N, window, lens = 3, 4, 2, 700, 100, [700, 300, 5]
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=D)
    got = run(q, k, v, do, window, lens)
    check(got, q, k, v, do, window, lens, f"W{window} lens {lens} D{D}")
    o = got[0]
    assert not o[2, :, 5 + window:].any() and not o[1, :, 300 + window:].any()


def test_window_bf16_and_rejections():
    import fa_p100
    from test_gpu_bf16 import bf16_inputs
    q, k, v, do = (t.to(DEV) for t in bf16_inputs(1, 4, 2, 600, 128, seed=2))
    o = fa_p100.flash_attn(q, k, v, True, sliding_window=150)
    f = lambda t: t.float().cpu().double().numpy()
    ref_o, _ = ora.attention_fwd(f(q), f(k), f(v), True, window=150)
    assert ora.max_abs(f(o), ref_o) <= 2.5e-2
    with pytest.raises(ValueError, match="causal"):
        fa_p100.flash_attn(q, k, v, False, sliding_window=150)
    with pytest.raises(RuntimeError, match="sliding window"):
        fa_p100._ext.forward_dt(q, k, v, False, None, 150)


def test_hf_hook_sliding_window_layers_match_eager():
    """Qwen3 with sliding-window layers (use_sliding_window, window 96,
    layers >= 1 sliding): logits within the eager-vs-sdpa envelope, and a
    training step's loss and attention-weight gradients against eager."""
    import fa_p100_hf
    from transformers import Qwen3Config, Qwen3ForCausalLM

    def model(seed=0):
        cfg = Qwen3Config(vocab_size=1000, hidden_size=512, intermediate_size=1024,
                          num_hidden_layers=3, num_attention_heads=8, num_key_value_heads=2,
                          head_dim=64, max_position_embeddings=1024, use_cache=False,
                          use_sliding_window=True, sliding_window=96, max_window_layers=1)
        assert cfg.layer_types == ["full_attention", "sliding_attention", "sliding_attention"]
        torch.manual_seed(seed)
        with torch.device(DEV):
            return Qwen3ForCausalLM(cfg)

    ids = torch.randint(0, 1000, (2, 400), device=DEV, generator=torch.Generator(DEV).manual_seed(6))

    def logits(m, impl):
        m.config._attn_implementation = impl
        with torch.no_grad(), torch.autocast("cuda", torch.float16):
            return m(ids).logits.float()

    m = model().eval()
    eager, sdpa = logits(m, "eager"), logits(m, "sdpa")
    fa_p100_hf.enable_fa_p100(m)
    fa = logits(m, "fa_p100")
    env, gap = (sdpa - eager).abs(), (fa - eager).abs()
    assert gap.mean() <= 2 * env.mean() + 1e-4, (gap.mean().item(), env.mean().item())
    assert (fa.argmax(-1) == eager.argmax(-1)).float().mean() >= \
        (sdpa.argmax(-1) == eager.argmax(-1)).float().mean() - 0.01

    # Gradients: within 5e-2 of eager, or within twice sdpa's own distance
    # from eager (fp16 autocast noise in the small norm-weight reductions).
    losses, grads = {}, {}
    for impl in ("eager", "sdpa", "fa_p100"):
        mm = model(seed=3)
        if impl == "fa_p100":
            fa_p100_hf.enable_fa_p100(mm)
        else:
            mm.config._attn_implementation = impl
        with torch.autocast("cuda", torch.float16):
            out = mm(ids, labels=ids)
        out.loss.backward()
        losses[impl] = out.loss.item()
        grads[impl] = {n: p.grad.float().clone() for n, p in mm.named_parameters()
                       if "self_attn" in n and p.grad is not None}
    assert abs(losses["fa_p100"] - losses["eager"]) <= 1e-3 * abs(losses["eager"])
    for n, g in grads["eager"].items():
        rel = ((grads["fa_p100"][n] - g).norm() / g.norm()).item()
        env = ((grads["sdpa"][n] - g).norm() / g.norm()).item()
        assert rel < max(5e-2, 2 * env), (n, rel, env)
