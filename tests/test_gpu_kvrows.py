"""K/V with a different number of rows than Q (q_len != kv_len), beyond the
reference, which raises on it (fa_p100_hf.py:100-105, README.md:72-75): KV-cache
decoding (one query row), chunked prefill (a chunk of rows after cached ones)
and more query rows than keys. Causal masking is aligned at the bottom right,
the last query row against the last key, as torch's causal_lower_right defines
it (the oracle is pinned against it in test_oracle.py). flash_attn and the C
ABI (fa_options.kv_rows) against the float64 oracle, bit-identities between
layouts and entry points, chunked prefill against the square causal
attention, and greedy generation with a KV cache through the HF hook against
eager attention with the same cache."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import FWD_MAX_ABS, GRAD_REL_L2, LSE_MAX_ABS, REF_REL, fa_opts, load_capi, np64
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"


def inputs(B, Hq, Hkv, N, Nk, D, seed, dtype=torch.half):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, N, D, generator=g)
    k = torch.randn(B, Hkv, Nk, D, generator=g)
    v = torch.randn(B, Hkv, Nk, D, generator=g)
    do = torch.randn(B, Hq, N, D, generator=g)
    return [t.to(dtype) for t in (q, k, v, do)]


def run(q, k, v, do, causal, **kw):
    import fa_p100
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal, **kw)
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    return o.detach(), qg.grad, kg.grad, vg.grad


def elementwise(got, ref):
    """max |got - ref| / (|ref| + RMS(ref)), the bf16 suite's elementwise bar
    (test_gpu_bf16.py): bf16's 8x coarser rounding of the largest elements
    would dominate the reference's max|err| / RMS."""
    rms = float(np.sqrt(np.mean(ref * ref)))
    return float(np.max(np.abs(got - ref) / (np.abs(ref) + rms)))


def check(what, got, ref, fwd_tol=FWD_MAX_ABS, grad_tol=GRAD_REL_L2, rel_tol=REF_REL,
          bf16=False):
    o, dq, dk, dv = (np64(t) for t in got)
    ref_o, grads = ref
    rel = elementwise if bf16 else ora.rel_max_rms
    assert ora.max_abs(o, ref_o) <= fwd_tol, what
    assert rel(o, ref_o) < rel_tol, what
    for name, g, r in zip(("dQ", "dK", "dV"), (dq, dk, dv), grads):
        assert np.isfinite(g).all(), (what, name)
        if not np.any(r):
            assert not np.any(g), (what, name)
            continue
        assert ora.rel_l2(g, r) <= grad_tol and rel(g, r) < rel_tol, (what, name)


CASES = [
    # B, Hq, Hkv, N, Nk, D, causal
    (2, 4, 2, 1, 700, 128, True),     # decoding one token against a cache
    (2, 4, 2, 1, 700, 64, False),
    (1, 8, 8, 5, 333, 128, True),     # a short chunk
    (2, 4, 1, 128, 640, 64, True),    # chunked prefill, tile-aligned
    (1, 4, 4, 190, 577, 128, True),   # chunked prefill, ragged
    (2, 2, 2, 300, 70, 128, True),    # more query rows than keys
    (1, 4, 2, 257, 129, 64, False),
    (1, 2, 2, 100, 1000, 96, False),
    (1, 4, 2, 64, 4096, 128, True),   # a long cache
    (1, 2, 1, 33, 512, 40, True),     # a head dim below its tile width
]


@pytest.mark.parametrize("B,Hq,Hkv,N,Nk,D,causal", CASES)
def test_kv_rows_match_oracle(B, Hq, Hkv, N, Nk, D, causal):
    import fa_p100
    q, k, v, do = inputs(B, Hq, Hkv, N, Nk, D, seed=N + Nk + D)
    got = run(q, k, v, do, causal)
    qn, kn, vn, dn = (t.double().numpy() for t in (q, k, v, do))
    ref_o, ref_lse = ora.attention_fwd(qn, kn, vn, causal)
    grads = ora.attention_bwd(qn, kn, vn, dn, causal)
    what = f"{B},{Hq}/{Hkv},N{N},Nk{Nk},D{D},causal={causal}"
    check(what, got, (ref_o, grads))
    _, lse = fa_p100._ext.forward_dt(q.to(DEV), k.to(DEV), v.to(DEV), causal)
    lse = np64(lse)
    fin = np.isfinite(ref_lse)
    assert np.array_equal(np.isfinite(lse), fin), what  # rows with no key: +inf
    assert ora.max_abs(lse[fin], ref_lse[fin]) <= LSE_MAX_ABS, what
    if causal and N > Nk:  # rows above the first key: exactly zero output and dq
        dead = N - Nk
        assert not got[0][:, :, :dead].any() and not got[1][:, :, :dead].any(), what


@pytest.mark.parametrize("dtype", [torch.half, torch.bfloat16])
def test_kv_rows_with_window_alibi_and_key_lengths(dtype):
    """Windows and ALiBi count from the bottom-right diagonal; key lengths
    clamp to the key rows; bf16 with its bars (test_gpu_bf16.py)."""
    B, Hq, Hkv, N, Nk, D = 2, 4, 2, 96, 500, 128
    q, k, v, do = inputs(B, Hq, Hkv, N, Nk, D, seed=77, dtype=dtype)
    lens = [500, 271]
    slopes = torch.tensor([2.0 ** (-8.0 * (i + 1) / Hq) for i in range(Hq)])
    kw = dict(kv_len=torch.tensor(lens, dtype=torch.int32, device=DEV), sliding_window=150,
              alibi_slopes=slopes.to(DEV))
    got = run(q, k, v, do, True, **kw)
    qn, kn, vn, dn = (t.double().numpy() for t in (q, k, v, do))
    okw = dict(kv_len=lens, window=150, alibi=slopes.double().numpy())
    ref = (ora.attention_fwd(qn, kn, vn, True, **okw)[0], ora.attention_bwd(qn, kn, vn, dn, True, **okw))
    bf = dtype == torch.bfloat16
    check(f"kv_rows options {dtype}", got, ref, fwd_tol=2.5e-2 if bf else FWD_MAX_ABS,
          grad_tol=2e-2 if bf else GRAD_REL_L2, bf16=bf)
    for b, L in enumerate(lens):  # keys past the length: exactly zero gradient
        assert not got[2][b, :, L:].any() and not got[3][b, :, L:].any()


def test_kv_rows_bnhd_views_and_capi_are_bit_identical():
    """(B, N, H, D) views of dense (B, N, H, D) storage give the dense
    results bit for bit, and the C ABI with fa_options.kv_rows gives the
    op's."""
    import fa_p100
    B, Hq, Hkv, N, Nk, D = 2, 8, 2, 77, 300, 128
    q, k, v, do = (t.to(DEV) for t in inputs(B, Hq, Hkv, N, Nk, D, seed=9))
    as_bnhd = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)
    dense = [t.clone().requires_grad_(True) for t in (q, k, v)]
    views = [as_bnhd(t).detach().requires_grad_(True) for t in (q, k, v)]
    o1 = fa_p100.flash_attn(*dense, True)
    o2 = fa_p100.flash_attn(*views, True)
    o1.backward(do)
    o2.backward(as_bnhd(do))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    for x, y in zip(dense, views):
        assert torch.equal(x.grad, y.grad)

    lib = load_capi()
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    o = torch.empty_like(q)
    lse = torch.empty(B, Hq, N, dtype=torch.float32, device=DEV)
    op = fa_opts(kv_rows=Nk)
    assert lib.fa_fwd_ex(ptr(q), ptr(k), ptr(v), ptr(o), ptr(lse), B, Hq, Hkv, N, D, 1, op, s) == 0
    ws_bytes = lib.fa_bwd_workspace_bytes(B, Hq, Hkv, N, D)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    assert lib.fa_bwd_ex(ptr(q), ptr(k), ptr(v), ptr(do), ptr(o), ptr(lse), ptr(dq), ptr(dk),
                         ptr(dv), ptr(ws), ws_bytes, B, Hq, Hkv, N, D, 1, op, s) == 0
    torch.cuda.synchronize()
    assert torch.equal(o, o1.detach())
    for x, y in zip((dq, dk, dv), dense):
        assert torch.equal(x, y.grad)
    # kv_rows with a mask is refused before any launch
    bits = torch.zeros(1, dtype=torch.int32, device=DEV)
    bad = fa_opts(kv_rows=Nk, mask=bits, mask_t=bits, mask_heads=1)
    assert lib.fa_fwd_ex(ptr(q), ptr(k), ptr(v), ptr(o), ptr(lse), B, Hq, Hkv, N, D, 1, bad, s) \
        == 10017


def test_chunked_prefill_equals_the_square_causal_attention():
    """A prompt run in chunks against the growing cache gives each chunk's
    rows of the one-shot causal attention over the whole prompt, and the
    chunks' dK, dV sum to the one-shot ones (each chunk's loss covers its own
    rows)."""
    import fa_p100
    B, Hq, Hkv, N, D = 1, 8, 2, 1000, 128
    q, k, v, do = (t.to(DEV) for t in inputs(B, Hq, Hkv, N, N, D, seed=3))
    full = [t.clone().requires_grad_(True) for t in (q, k, v)]
    o_full = fa_p100.flash_attn(*full, True)
    o_full.backward(do)
    kc, vc = k.clone().requires_grad_(True), v.clone().requires_grad_(True)
    start, outs = 0, []
    for size in (1, 300, 129, 570):
        end = start + size
        qc = q[:, :, start:end].clone().requires_grad_(True)
        oc = fa_p100.flash_attn(qc, kc[:, :, :end], vc[:, :, :end], True)
        oc.backward(do[:, :, start:end])
        outs.append((start, end, oc.detach(), qc.grad))
        start = end
    torch.cuda.synchronize()
    for a, b, oc, dqc in outs:
        assert (oc - o_full[:, :, a:b].detach()).abs().max().item() <= FWD_MAX_ABS, (a, b)
        ref = full[0].grad[:, :, a:b].float()
        assert ((dqc.float() - ref).norm() / ref.norm()).item() <= GRAD_REL_L2, (a, b)
    for g, ref in ((kc.grad, full[1].grad), (vc.grad, full[2].grad)):
        assert ((g.float() - ref.float()).norm() / ref.float().norm()).item() <= GRAD_REL_L2


def test_flash_attn_refuses_row_counts_with_masks():
    import fa_p100
    q, k, v, _ = (t.to(DEV) for t in inputs(1, 2, 2, 4, 9, 64, seed=1))
    with pytest.raises(ValueError, match="q_len == kv_len"):
        fa_p100.flash_attn(q, k, v, True, attn_mask=torch.ones(4, 4, dtype=torch.bool,
                                                               device=DEV))
    with pytest.raises(ValueError, match="q_len == kv_len"):
        fa_p100.flash_attn(q, k, v, True, dropout_p=0.1, dropout_seed=1)


def test_hook_generates_with_a_kv_cache_like_eager():
    """Generation with transformers' KV cache through the hook (the reference
    turned the cache off and raised on it): the prompt's prefill (q_len ==
    kv_len) and every decoding step (q_len 1 against the growing cache),
    teacher-forced on eager's greedy tokens, give logits within the
    eager-vs-sdpa envelope at every step and the same argmax as often as
    sdpa does; a chunked prefill (the prompt's second half against the cached
    first half, q_len 20 against kv_len 40) too."""
    import fa_p100_hf
    from test_gpu_hf import qwen3
    model = qwen3(2, 512, 8, 2, 128, 1024, 1000, seed=11).eval()
    ids = torch.randint(0, 1000, (1, 40), device=DEV,
                        generator=torch.Generator(DEV).manual_seed(5))
    steps = 12

    def use(impl):
        if impl == "fa_p100":
            fa_p100_hf.enable_fa_p100(model, use_cache=True)
        else:
            model.config._attn_implementation = impl

    def decode(impl, forced=None):
        use(impl)
        toks, logits, cache, step_in = [], [], None, ids
        with torch.no_grad(), torch.autocast("cuda", torch.float16):
            for i in range(steps):
                r = model(step_in, past_key_values=cache, use_cache=True)
                cache = r.past_key_values
                logits.append(r.logits[:, -1].float())
                nxt = logits[-1].argmax(-1, keepdim=True) if forced is None else forced[i]
                toks.append(nxt)
                step_in = nxt
        return toks, torch.stack(logits)

    toks_e, log_e = decode("eager")
    _, log_s = decode("sdpa", toks_e)
    _, log_f = decode("fa_p100", toks_e)
    env = (log_s - log_e).abs().amax(dim=(1, 2))
    gap = (log_f - log_e).abs().amax(dim=(1, 2))
    assert bool((gap <= 4 * env + 1e-3).all()), (gap.tolist(), env.tolist())
    agree_f = (log_f.argmax(-1) == log_e.argmax(-1)).float().mean()
    agree_s = (log_s.argmax(-1) == log_e.argmax(-1)).float().mean()
    assert agree_f >= agree_s - 1e-6

    def chunked(impl):
        use(impl)
        with torch.no_grad(), torch.autocast("cuda", torch.float16):
            r = model(ids[:, :20], use_cache=True)
            r = model(ids[:, 20:], past_key_values=r.past_key_values, use_cache=True)
        return r.logits.float()

    ce, cs, cf = chunked("eager"), chunked("sdpa"), chunked("fa_p100")
    assert (cf - ce).abs().max().item() <= 4 * (cs - ce).abs().max().item() + 1e-3
