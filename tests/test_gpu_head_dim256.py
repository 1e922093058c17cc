"""Head dims 136 .. 256, beyond the reference's 64 and 128 (fa_p100_ext.cu:59,
111). They run at tile width 256, whose kernels are shaped differently from
the narrower ones: the forward has 4 waves (2 row blocks x 2 key halves of a
64-key stage), the backward 4 waves of one 32-row block each, K operands
loaded from global memory into registers, 32-row streamed tiles and no
causal split of key tiles. Here: every such width class against the float64
oracle; long rows; every option (key lengths, window, ALiBi, packed
sequences, a mask, softmax scale); dropout; q_len != kv_len; bf16, the
(B, N, H, D) views and the C ABI bit-identical to the op; the bias refused;
and Qwen3 with head_dim 256 through the hook. Bars: the fp16 ones
(helpers.py), bf16's from test_gpu_bf16.py."""
import numpy as np
import pytest
import torch

from helpers import make_inputs
from oracle import attention as ora
from test_gpu_dropout import check as _dropout_check
from test_gpu_dropout import lse_of as _dropout_lse
from test_gpu_dropout import run as _dropout_run
from test_gpu_head_dims import check
from test_gpu_head_dims import test_d96_bf16_bnhd_and_capi as _bf16_bnhd_capi
from test_gpu_head_dims import test_d96_every_option_matches_oracle as _every_option
from test_gpu_kvrows import check as _kv_check
from test_gpu_kvrows import inputs as _kv_inputs
from test_gpu_kvrows import run as _kv_run

pytestmark = pytest.mark.gpu

DEV = "cuda"


def run_and_check(B, Hq, Hkv, N, D, causal, seed):
    import fa_p100
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=seed)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal)
    o.backward(do.to(DEV))
    _, lse = fa_p100._ext.forward(qg.detach(), kg.detach(), vg.detach(), causal, False)
    torch.cuda.synchronize()
    assert o.shape == q.shape and qg.grad.shape == q.shape and kg.grad.shape == k.shape
    check(o, lse, (qg.grad, kg.grad, vg.grad), q, k, v, do, causal,
          f"{B},{Hq}/{Hkv},N{N},D{D} causal={causal}")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D", [136, 160, 192, 200, 224, 248, 256])
def test_wide_head_dims_match_oracle(D, causal):
    """Ragged N with GQA; two key tiles per workgroup."""
    run_and_check(2, 4, 2, 397, D, causal, seed=D + causal)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,Hq,Hkv,N", [(1, 4, 4, 2048), (2, 4, 2, 1000), (1, 2, 1, 4096)])
def test_d256_long_rows_match_oracle(B, Hq, Hkv, N, causal):
    """Many key tiles per workgroup (the causal pairing of query tiles in the
    forward), GQA and MQA."""
    run_and_check(B, Hq, Hkv, N, 256, causal, seed=N + Hkv + causal)


@pytest.mark.parametrize("D", [256, 200])
@pytest.mark.parametrize("causal", [True, False])
def test_d256_every_option_matches_oracle(causal, D):
    _every_option(causal, D)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,Hq,Hkv,N,p", [(2, 4, 2, 333, 0.1), (1, 2, 1, 1024, 0.5)])
def test_d256_dropout_matches_oracle(B, Hq, Hkv, N, p, causal):
    D = 256
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + D + causal)
    seed = 2000 + N
    got = _dropout_run(q, k, v, do, causal, p, seed)
    _dropout_check(got, _dropout_lse(q, k, v, causal), q, k, v, do, causal, p, seed,
                   f"dropout p={p} {B},{Hq}/{Hkv},N{N} D{D} causal={causal}")


@pytest.mark.parametrize("B,Hq,Hkv,N,Nk,causal", [
    (2, 4, 2, 1, 700, True),     # decoding one token against a cache
    (1, 4, 4, 190, 577, True),   # chunked prefill, ragged
    (2, 2, 2, 300, 70, True),    # more query rows than keys
    (1, 2, 2, 100, 1000, False),
])
def test_d256_kv_rows_match_oracle(B, Hq, Hkv, N, Nk, causal):
    D = 256
    q, k, v, do = _kv_inputs(B, Hq, Hkv, N, Nk, D, seed=N + Nk)
    got = _kv_run(q, k, v, do, causal)
    qn, kn, vn, dn = (t.double().numpy() for t in (q, k, v, do))
    ref_o, _ = ora.attention_fwd(qn, kn, vn, causal)
    grads = ora.attention_bwd(qn, kn, vn, dn, causal)
    _kv_check(f"{B},{Hq}/{Hkv},N{N},Nk{Nk},D{D},causal={causal}", got, (ref_o, grads))


@pytest.mark.parametrize("D", [256, 168])
def test_d256_bf16_bnhd_and_capi(D):
    _bf16_bnhd_capi(D)


def test_d256_refuses_a_bias():
    """The width-256 kernels take no attention bias: flash_attn raises before
    any launch, and the binding reports the C ABI's error."""
    import fa_p100
    q, k, v, _ = (t.to(DEV) for t in make_inputs(1, 2, 2, 64, 256, seed=1))
    bias = torch.zeros(64, 64, device=DEV)
    with pytest.raises(ValueError, match="head dim up to 128, got 256"):
        fa_p100.flash_attn(q, k, v, True, attn_bias=bias)
    with pytest.raises(RuntimeError, match="head dim up to 128"):
        fa_p100._ext.forward_dt(q, k, v, True, bias=bias[None, None])


def test_hf_hook_head_dim_256_matches_eager():
    """Qwen3 with head_dim 256 through the hook: logits within the
    eager-vs-sdpa envelope."""
    import fa_p100_hf
    from test_gpu_hf import logits_with, qwen3
    model = qwen3(2, 512, 4, 2, 256, 1024, 1000).eval()
    ids = torch.randint(0, 1000, (2, 300), device=DEV,
                        generator=torch.Generator(DEV).manual_seed(3))
    eager, sdpa = logits_with(model, "eager", ids), logits_with(model, "sdpa", ids)
    fa_p100_hf.enable_fa_p100(model)
    fa = logits_with(model, "fa_p100", ids)
    env, gap = (sdpa - eager).abs(), (fa - eager).abs()
    assert gap.mean() <= 2 * env.mean() + 1e-4, (gap.mean().item(), env.mean().item())
    assert np.isfinite(fa.cpu().numpy()).all()
