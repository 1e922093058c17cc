"""Packed sequences (beyond the reference, whose hook ignored position_ids and
so attended across packed sequences): flash_attn(..., segment_ids=s), causal,
each maximal run of equal ids one sequence. Against the float64 oracle with
the same ids (pinned in test_oracle.py by running each sequence alone,
against torch SDPA with the block-diagonal mask, and finite differences),
against the kernels run on each sequence alone, with key lengths and a
window, in bf16, the (B, N, H, D) views, the C ABI, and a packed Qwen3 batch
through the hook against eager attention with the same position_ids.
Bars: the fp16 ones (helpers.py)."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import (FWD_MAX_ABS, GRAD_REL_L2, LSE_MAX_ABS, REF_REL, fa_opts, load_capi,
                     make_inputs, np64)
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"


def ids_from_lengths(lengths):
    return np.concatenate([np.full(n, i) for i, n in enumerate(lengths)])


def run(q, k, v, do, seg, lens=None, window=None, causal=True):
    import fa_p100
    kv_len = None if lens is None else torch.tensor(lens, dtype=torch.int32, device=DEV)
    sid = torch.tensor(seg, device=DEV)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal, kv_len=kv_len, sliding_window=window,
                           segment_ids=sid)
    o.backward(do.to(DEV))
    s0, s1 = fa_p100.segment_bounds(sid)
    _, lse = fa_p100._ext.forward_dt(qg.detach(), kg.detach(), vg.detach(), causal, kv_len,
                                     window or 0, None, s0, s1)
    torch.cuda.synchronize()
    return o, lse, qg.grad, kg.grad, vg.grad


def check(got, q, k, v, do, seg, what, lens=None, window=None, causal=True):
    o, lse, dq, dk, dv = got
    qn, kn, vn, dn = (t.float().numpy() for t in (q, k, v, do))
    ref_o, ref_lse = ora.attention_fwd(qn, kn, vn, causal, kv_len=lens, window=window,
                                       segments=seg)
    assert ora.max_abs(np64(o), ref_o) <= FWD_MAX_ABS, what
    assert ora.rel_max_rms(np64(o), ref_o) < REF_REL, what
    seen = np.isfinite(ref_lse)
    assert np.array_equal(np.isfinite(np64(lse)), seen), what
    assert ora.max_abs(np64(lse)[seen], ref_lse[seen]) <= LSE_MAX_ABS, what
    ref = ora.attention_bwd(qn, kn, vn, dn, causal, kv_len=lens, window=window, segments=seg)
    for name, g, r in zip(("dQ", "dK", "dV"), (dq, dk, dv), ref):
        g = np64(g)
        assert np.isfinite(g).all(), (what, name)
        l2, rr = ora.rel_l2(g, r), ora.rel_max_rms(g, r)
        assert l2 <= GRAD_REL_L2 and rr < REF_REL, (what, name, l2, rr)


# Sequence lengths: boundaries inside and on tile edges (64 forward, 128
# backward), single tokens, one sequence filling the row, many short ones.
CASES = [
    (1, 4, 4, 1000, [[300, 1, 1, 128, 570]]),
    (2, 8, 2, 777, [[64, 64, 128, 521], [777]]),
    (1, 4, 1, 2048, [[37] * 55 + [13]]),
    (1, 2, 2, 4096, [[1000, 2000, 1, 1095]]),
    (2, 4, 2, 129, [[128, 1], [1, 128]]),
]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("B,Hq,Hkv,N,lengths", CASES)
def test_packed_matches_oracle(D, B, Hq, Hkv, N, lengths, causal):
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + D + B)
    seg = np.stack([ids_from_lengths(l) for l in lengths])
    got = run(q, k, v, do, seg, causal=causal)
    check(got, q, k, v, do, seg, f"packed {lengths} D{D} {B},{Hq}/{Hkv},N{N} causal={causal}",
          causal=causal)


def test_packed_non_causal_with_key_lengths():
    B, Hq, Hkv, N, D = 2, 4, 2, 700, 128
    seg = np.stack([ids_from_lengths([250, 50, 400]), ids_from_lengths([100, 600])])
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=77)
    check(run(q, k, v, do, seg, lens=[700, 420], causal=False), q, k, v, do, seg,
          "packed non-causal lens", lens=[700, 420], causal=False)


def test_packed_equals_each_sequence_alone():
    """The kernels on a packed row give, sequence by sequence, what they give
    on each sequence alone (to fp16 rounding: tiles fall differently)."""
    import fa_p100
    D, Hq, Hkv, lengths = 128, 4, 2, [200, 77, 1, 600, 146]
    N = sum(lengths)
    q, k, v, do = (t.to(DEV) for t in make_inputs(1, Hq, Hkv, N, D, seed=5))
    sid = torch.tensor(ids_from_lengths(lengths), device=DEV)[None]
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
    o = fa_p100.flash_attn(*leaves, True, segment_ids=sid)
    o.backward(do)
    a = 0
    for n in lengths:
        parts = [t[:, :, a:a + n].clone().requires_grad_(True) for t in (q, k, v)]
        o1 = fa_p100.flash_attn(*parts, True)
        o1.backward(do[:, :, a:a + n])
        assert (o[:, :, a:a + n].float() - o1.float()).abs().max().item() <= 4e-3
        for full, part in zip(leaves, parts):
            g, g1 = full.grad[:, :, a:a + n].float(), part.grad.float()
            assert ((g - g1).norm() / g1.norm().clamp_min(1e-6)).item() <= 1e-2
        a += n


@pytest.mark.parametrize("D", [64, 128])
def test_packed_with_key_lengths_and_window(D):
    B, Hq, Hkv, N = 2, 4, 2, 700
    lengths = [[250, 50, 400], [100, 600]]
    seg = np.stack([ids_from_lengths(l) for l in lengths])
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=2 * D)
    check(run(q, k, v, do, seg, lens=[700, 420]), q, k, v, do, seg, f"packed lens D{D}",
          lens=[700, 420])
    check(run(q, k, v, do, seg, window=96), q, k, v, do, seg, f"packed W96 D{D}", window=96)


def test_packed_bf16_bnhd_and_capi():
    """bf16 against the oracle; (B,N,H,D) views bit-identical to dense; the C
    ABI with seg_start/seg_end bit-identical to the op; bad inputs raise."""
    import fa_p100
    from test_gpu_bf16 import BF_FWD_MAX_ABS, BF_GRAD_REL_L2, bf16_inputs
    B, Hq, Hkv, N, D = 2, 8, 2, 500, 128
    seg = np.stack([ids_from_lengths([120, 8, 372]), ids_from_lengths([499, 1])])
    sid = torch.tensor(seg, device=DEV)
    q, k, v, do = (t.to(DEV) for t in bf16_inputs(B, Hq, Hkv, N, D, seed=13))
    as_bnhd = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)
    dense = [t.clone().requires_grad_(True) for t in (q, k, v)]
    views = [as_bnhd(t).detach().requires_grad_(True) for t in (q, k, v)]
    o1 = fa_p100.flash_attn(*dense, True, segment_ids=sid)
    o2 = fa_p100.flash_attn(*views, True, segment_ids=sid)
    o1.backward(do)
    o2.backward(as_bnhd(do))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    for a, b in zip(dense, views):
        assert torch.equal(a.grad, b.grad)
    f = lambda t: t.detach().float().cpu().double().numpy()
    ref_o, _ = ora.attention_fwd(f(q), f(k), f(v), True, segments=seg)
    assert ora.max_abs(f(o1), ref_o) <= BF_FWD_MAX_ABS
    ref = ora.attention_bwd(f(q), f(k), f(v), f(do), True, segments=seg)
    for t, r in zip(dense, ref):
        assert ora.rel_l2(f(t.grad), r) <= BF_GRAD_REL_L2

    lib = load_capi()
    s0, s1 = fa_p100.segment_bounds(sid)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    opts = fa_opts(dtype=1, seg_start=s0, seg_end=s1)
    o, lse = torch.empty_like(q), torch.empty(B, Hq, N, device=DEV)
    assert lib.fa_fwd_ex(p(q), p(k), p(v), p(o), p(lse), B, Hq, Hkv, N, D, 1, opts, s) == 0
    ws_bytes = lib.fa_bwd_workspace_bytes(B, Hq, Hkv, N, D)
    ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    rc = lib.fa_bwd_ex(p(q), p(k), p(v), p(do), p(o), p(lse), p(dq), p(dk), p(dv), p(ws),
                       ws_bytes, B, Hq, Hkv, N, D, 1, opts, s)
    assert rc == 0, lib.fa_error_string(rc)
    torch.cuda.synchronize()
    o_op, lse_op = fa_p100._ext.forward_dt(q, k, v, True, None, 0, None, s0, s1)
    dq_op, dk_op, dv_op = fa_p100._ext.backward_dt(q, k, v, do, o_op, lse_op, True, None, 0,
                                                   None, s0, s1)
    for a, b in ((o, o_op), (lse, lse_op), (dq, dq_op), (dk, dk_op), (dv, dv_op)):
        assert torch.equal(a, b)
    with pytest.raises(ValueError, match="segment_ids must have shape"):
        fa_p100.flash_attn(q, k, v, True, segment_ids=sid[:, :10])
    with pytest.raises(RuntimeError, match="seg_start must be int32"):
        fa_p100._ext.forward_dt(q, k, v, True, None, 0, None, s0.long(), s1)
    with pytest.raises(RuntimeError, match="packed sequences need both"):
        fa_p100._ext.forward_dt(q, k, v, True, None, 0, None, s0, None)


def test_hf_hook_packed_batch_matches_eager():
    """A Qwen3 batch of three sequences packed into one row (position_ids
    restarting at each), as DataCollatorWithFlattening makes it: logits within
    the eager-vs-sdpa envelope of eager attention with the same position_ids
    (transformers masks across the packed sequences for eager), the packed
    logits of each sequence equal to that sequence alone, and a training
    step's loss and attention gradients against eager."""
    import fa_p100_hf
    from transformers import Qwen3Config, Qwen3ForCausalLM

    def model(seed=0):
        cfg = Qwen3Config(vocab_size=1000, hidden_size=512, intermediate_size=1024,
                          num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2,
                          head_dim=64, max_position_embeddings=1024, use_cache=False)
        torch.manual_seed(seed)
        with torch.device(DEV):
            return Qwen3ForCausalLM(cfg)

    lengths = [150, 260, 90]
    N = sum(lengths)
    g = torch.Generator(DEV).manual_seed(8)
    ids = torch.randint(0, 1000, (1, N), device=DEV, generator=g)
    pos = torch.cat([torch.arange(n, device=DEV) for n in lengths])[None]

    def logits(m, impl, **kw):
        m.config._attn_implementation = impl
        with torch.no_grad(), torch.autocast("cuda", torch.float16):
            return m(ids, position_ids=pos, **kw).logits.float()

    m = model().eval()
    eager, sdpa = logits(m, "eager"), logits(m, "sdpa")
    fa_p100_hf.enable_fa_p100(m)
    fa = logits(m, "fa_p100")
    env, gap = (sdpa - eager).abs(), (fa - eager).abs()
    assert gap.mean() <= 2 * env.mean() + 1e-4, (gap.mean().item(), env.mean().item())
    # Each sequence alone through the hook gives the same logits.
    a = 0
    for n in lengths:
        with torch.no_grad(), torch.autocast("cuda", torch.float16):
            alone = m(ids[:, a:a + n]).logits.float()
        assert (alone - fa[:, a:a + n]).abs().max().item() <= 5e-2
        a += n
    # Cross-sequence attention would be far outside the envelope.
    m.config._attn_implementation = "eager"
    with torch.no_grad(), torch.autocast("cuda", torch.float16):
        unpacked = m(ids).logits.float()
    assert (unpacked - eager).abs().mean() > 10 * gap.mean()

    losses, grads = {}, {}
    for impl in ("eager", "sdpa", "fa_p100"):
        mm = model(seed=3)
        if impl == "fa_p100":
            fa_p100_hf.enable_fa_p100(mm)
        else:
            mm.config._attn_implementation = impl
        with torch.autocast("cuda", torch.float16):
            out = mm(ids, position_ids=pos, labels=ids)
        out.loss.backward()
        losses[impl] = out.loss.item()
        grads[impl] = {n: p.grad.float().clone() for n, p in mm.named_parameters()
                       if "self_attn" in n and p.grad is not None}
    assert abs(losses["fa_p100"] - losses["eager"]) <= 1e-3 * abs(losses["eager"])
    for n, gr in grads["eager"].items():
        rel = ((grads["fa_p100"][n] - gr).norm() / gr.norm()).item()
        env_g = ((grads["sdpa"][n] - gr).norm() / gr.norm()).item()
        assert rel <= max(5e-2, 2 * env_g), (n, rel, env_g)


def test_packed_with_alibi_matches_oracle():
    """Packed sequences and ALiBi slopes together (both ride on the masked
    instantiation): against the oracle with the same ids and slopes."""
    import fa_p100
    B, Hq, Hkv, N, D = 2, 4, 2, 600, 128
    seg = np.stack([ids_from_lengths([200, 1, 399]), ids_from_lengths([64, 536])])
    slopes = np.array([2.0 ** (-8.0 * (i + 1) / Hq) for i in range(Hq)], dtype=np.float32)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=21)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    al = torch.tensor(slopes, device=DEV)
    o = fa_p100.flash_attn(qg, kg, vg, True, alibi_slopes=al,
                           segment_ids=torch.tensor(seg, device=DEV))
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    qn, kn, vn, dn = (t.float().numpy() for t in (q, k, v, do))
    sl = slopes.astype(np.float64)
    ref_o, _ = ora.attention_fwd(qn, kn, vn, True, alibi=sl, segments=seg)
    assert ora.max_abs(np64(o), ref_o) <= FWD_MAX_ABS
    ref = ora.attention_bwd(qn, kn, vn, dn, True, alibi=sl, segments=seg)
    for name, g, r in zip(("dQ", "dK", "dV"), (qg.grad, kg.grad, vg.grad), ref):
        l2, rr = ora.rel_l2(np64(g), r), ora.rel_max_rms(np64(g), r)
        assert l2 <= GRAD_REL_L2 and rr < REF_REL, (name, l2, rr)

