"""The HF hook's raise-on-unsupported guards (fa_p100_hf.py:64-105, 186-206).

All guards fire before any kernel runs, so they are checked on the CPU with
host tensors and a stub module; registration and enable_fa_p100 are checked on
a tiny random-init Qwen3 built on the CPU.
"""
import types
import warnings

import pytest
import torch

import fa_p100_hf as hf


def qkv(n=4, d=64, hq=4, hkv=2, dtype=torch.half, kv_len=None):
    kv_len = n if kv_len is None else kv_len
    return (torch.zeros(1, hq, n, d, dtype=dtype), torch.zeros(1, hkv, kv_len, d, dtype=dtype),
            torch.zeros(1, hkv, kv_len, d, dtype=dtype))


MOD = types.SimpleNamespace(is_causal=True)


@pytest.mark.parametrize("kwargs,match", [
    (dict(attention_mask=torch.ones(1, 3, 4, 4, dtype=torch.bool)), "4-D attention mask"),
    (dict(attention_mask=torch.ones(1, 1, 4, 4, dtype=torch.int32)), "boolean or floating"),
    (dict(attention_mask=None, output_attentions=True), "output_attentions"),
    (dict(attention_mask=None, head_mask=torch.ones(4)), "head_mask"),
    (dict(attention_mask=None, sliding_window=128, is_causal=False), "a window of 128"),
    (dict(attention_mask=None, sliding_window=0), "a window of 0"),
    (dict(attention_mask=None, s_aux=torch.zeros(4)), "attention sinks"),
    (dict(attention_mask=None, softcap=50.0), "soft-capping"),
])
def test_unsupported_requests_raise(kwargs, match):
    q, k, v = qkv()
    with pytest.raises(NotImplementedError, match=match):
        hf.fa_p100_attention_forward(MOD, q, k, v, **kwargs)


def test_dropout_reaches_the_kernel():
    """Attention dropout passes the hook (the reference raised,
    fa_p100_hf.py:83-85); host tensors then stop at the device check."""
    q, k, v = qkv()
    with pytest.raises(RuntimeError, match="q must be a CUDA tensor"):
        hf.fa_p100_attention_forward(MOD, q, k, v, None, dropout=0.1)


def test_head_dim_scale_and_kv_len_guards():
    q, k, v = qkv(d=100)
    with pytest.raises(NotImplementedError, match="multiples of 8 up to 256, got 100"):
        hf.fa_p100_attention_forward(MOD, q, k, v, None)
    with pytest.raises(NotImplementedError, match="multiples of 8 up to 256, got 264"):
        hf.fa_p100_attention_forward(MOD, *qkv(d=264), None)
    # head_dim 256 passes the guards (host tensors stop at the device check),
    # but not with an additive float mask, which would be a bias
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        hf.fa_p100_attention_forward(MOD, *qkv(d=256), None)
    soft = torch.zeros(1, 1, 4, 4)
    soft[..., 0] = -0.5
    with pytest.raises(NotImplementedError, match="up to head_dim 128, got 256"):
        hf.fa_p100_attention_forward(MOD, *qkv(d=256), soft)
    q, k, v = qkv(d=128)
    # Another scale passes the guards now (the host tensors then stop at the
    # binding's device check); the reference raised here.
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        hf.fa_p100_attention_forward(MOD, q, k, v, None, scaling=0.1)
    # q_len != kv_len (a KV cache) passes to the kernels now (the reference
    # raised); host tensors stop at the binding's device check. A cached step
    # with a padding bound raises.
    q, k, v = qkv(n=1, kv_len=9)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        hf.fa_p100_attention_forward(MOD, q, k, v, None)
    with pytest.raises(NotImplementedError, match="KV cache"):
        hf.fa_p100_attention_forward(MOD, q, k, v, None,
                                     fa_p100_bounds=(torch.tensor([5], dtype=torch.int32),
                                                     hf._NOT_PACKED, None))


def test_valid_call_reaches_the_kernel_and_casts_with_one_warning():
    # Host tensors pass every hook guard and are stopped by the binding's
    # device check, i.e. the call really goes to the kernel (no CPU fallback).
    hf._warned_cast = False
    q, k, v = qkv(dtype=torch.float32)
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
            hf.fa_p100_attention_forward(MOD, q, k, v, None, scaling=64 ** -0.5)
        with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
            hf.fa_p100_attention_forward(MOD, q, k, v, None)
    assert sum("casts" in str(x.message) for x in w) == 1


def _tiny_qwen3():
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=128, hidden_size=128, intermediate_size=256,
                      num_hidden_layers=2, num_attention_heads=2, num_key_value_heads=1,
                      head_dim=64, max_position_embeddings=256)
    torch.manual_seed(0)
    return Qwen3ForCausalLM(cfg)


def test_register_and_enable():
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    assert hf.register() == "fa_p100"
    assert ALL_ATTENTION_FUNCTIONS.get_interface("fa_p100", None) is hf.fa_p100_attention_forward
    model = _tiny_qwen3()
    hf.enable_fa_p100(model, full_precision=True)
    assert model.config._attn_implementation == "fa_p100"
    assert model.config.use_cache is False
    assert all(getattr(m, "_fa_p100_full_precision") is True for m in model.modules())
    other = _tiny_qwen3()
    other.config.use_cache = True
    hf.enable_fa_p100(other, use_cache=True)  # leaves the cache setting alone
    assert other.config.use_cache is True
    inner = model.forward
    hf.enable_fa_p100(model)          # idempotent: the guard wraps once
    assert model.forward is inner

    ids = torch.zeros(1, 6, dtype=torch.long)
    # Holes and all-zero rows go to the kernels as key bit masks; right, left
    # and both-sided padding as key lengths / sequence bounds
    # (tests/test_gpu_kvlen.py and test_gpu_mask.py run them against eager
    # with the mask). Host tensors stop at the binding's device check.
    for mask in ([[1, 1, 0, 1, 1, 1]], [[0, 0, 0, 0, 0, 0]], [[0, 1, 0, 1, 1, 0]]):
        with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
            model(ids, attention_mask=torch.tensor(mask))
    # A 4-D mask is packed once in the wrapper (the packer's device check
    # stops host tensors).
    with pytest.raises(RuntimeError, match="mask must be a CUDA tensor"):
        model(ids, attention_mask=torch.ones(1, 1, 6, 6, dtype=torch.bool).tril())
    assert hf.right_padding_lengths(torch.tensor([[1, 1, 1, 1, 0, 0], [1] * 6])).tolist() == [4, 6]
    assert hf.right_padding_lengths(torch.tensor([[1, 0, 1, 0, 0, 0]])) is None
    first, end = hf.padding_spans(torch.tensor([[0, 0, 1, 1, 1, 1], [1, 1, 1, 0, 0, 0],
                                                [0, 1, 1, 1, 0, 0]]))
    assert first.tolist() == [2, 0, 1] and end.tolist() == [6, 3, 4]
    assert hf.padding_spans(torch.tensor([[1, 0, 1, 1, 1, 1]])) is None
    assert hf._left_padding_segments(first, 6).tolist() == [
        [0, 0, 1, 1, 1, 1], [1, 1, 1, 1, 1, 1], [0, 1, 1, 1, 1, 1]]
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        model(ids, attention_mask=torch.tensor([[1, 1, 1, 1, 0, 0]]))
    # A cached call is served (the reference raised on use_cache); host
    # tensors then stop at the binding's device check.
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        model(ids, use_cache=True)
    # An all-ones mask passes the guard; the attention hook then receives no
    # mask (transformers' early exit) and the call reaches the binding, whose
    # device check stops host tensors.
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        model(ids, attention_mask=torch.ones(1, 6, dtype=torch.long))


def test_packed_position_ids_become_segment_bounds():
    """Restarting position_ids mark packed sequences exactly as transformers'
    find_packed_sequence_indices does; one sequence per row gives None; the
    bounds are each token's [start, end) run; a packed batch on a
    non-causal call raises."""
    from fa_p100 import segment_bounds
    pos = torch.tensor([[0, 1, 2, 0, 1, 0, 1, 2, 3]])
    ids = hf.packed_segment_ids(pos, 1)
    assert ids.tolist() == [[0, 0, 0, 1, 1, 2, 2, 2, 2]]
    from transformers.masking_utils import find_packed_sequence_indices
    assert torch.equal(ids, find_packed_sequence_indices(pos))
    assert hf.packed_segment_ids(torch.arange(9)[None], 1) is None
    assert hf.packed_segment_ids(torch.arange(9)[None] + 5, 2) is None  # offset, one sequence
    assert hf.packed_segment_ids(pos, 3).shape == (3, 9)  # broadcast over the batch
    start, end = segment_bounds(ids)
    assert start.tolist() == [[0, 0, 0, 3, 3, 5, 5, 5, 5]]
    assert end.tolist() == [[3, 3, 3, 5, 5, 9, 9, 9, 9]]
    q, k, v = qkv(n=9)
    # A packed non-causal call passes the guards (the host tensors then stop
    # at the binding's device check).
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        hf.fa_p100_attention_forward(types.SimpleNamespace(is_causal=False), q, k, v, None,
                                     position_ids=pos)


def test_checkpointed_layers_see_the_padding_in_their_recompute(monkeypatch):
    """With gradient checkpointing every decoder layer runs its forward a
    second time inside backward, after the model call has returned. The
    padding (key lengths) and packing (sequence bounds) that enable_fa_p100's
    wrapper derived from the mask must reach that recompute too: the bounds
    ride on the model call's kwargs, which checkpointing replays. A spy
    stands in for the kernel call (CPU) and records what each call got."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    seen = []

    def spy(q, k, v, causal=False, full_precision=False, kv_len=None, sliding_window=None,
            segment_ids=None, softmax_scale=None, attn_mask=None, dropout_p=None,
            attn_bias=None):
        seen.append((torch.is_grad_enabled(),
                     None if kv_len is None else kv_len.tolist(),
                     None if segment_ids is None else segment_ids[0].tolist(),
                     None if attn_mask is None else attn_mask[0][:, 0, 0].tolist()))
        g = q.size(1) // k.size(1)
        return torch.nn.functional.scaled_dot_product_attention(
            q.float(), k.float().repeat_interleave(g, 1), v.float().repeat_interleave(g, 1),
            is_causal=causal).to(q.dtype)

    monkeypatch.setattr(hf, "flash_attn", spy)
    cfg = Qwen3Config(vocab_size=64, hidden_size=64, intermediate_size=64, num_hidden_layers=2,
                      num_attention_heads=2, num_key_value_heads=1, head_dim=64,
                      use_cache=False)
    torch.manual_seed(0)
    model = Qwen3ForCausalLM(cfg)
    hf.enable_fa_p100(model)
    model.gradient_checkpointing_enable()
    model.train()
    ids = torch.randint(0, 64, (2, 6))
    for mask, kv_len, seg_start, words in (
            (torch.tensor([[1, 1, 1, 1, 0, 0], [1, 1, 1, 1, 1, 1]]), [4, 6], None, None),  # right
            (torch.tensor([[0, 0, 1, 1, 1, 1], [1, 1, 1, 1, 1, 1]]), [6, 6],               # left
             [[0, 0, 2, 2, 2, 2], [0, 0, 0, 0, 0, 0]], None),
            (torch.tensor([[1, 0, 1, 1, 0, 1], [1, 1, 1, 1, 1, 1]]), None, None,          # holes
             [[0b101101], [0b111111]])):
        seen.clear()
        loss = model(ids, attention_mask=mask, labels=ids).loss
        first = list(seen)
        loss.backward()
        recompute = seen[len(first):]
        assert len(first) == len(recompute) == 2  # one call per layer, each replayed
        for _, kl, ss, wd in first + recompute:
            assert kl == kv_len and ss == seg_start and wd == words


def test_mask_words_match_a_dense_packing():
    """key_mask_bits (2-D padding masks with holes) against the bits of the
    dense mask it stands for, packed on the host with numpy (bit j % 32 of
    word j // 32, little-endian bit order), and its transpose."""
    import numpy as np
    rng = np.random.default_rng(3)
    for n in (1, 5, 32, 33, 70):
        m = torch.tensor(rng.random((3, n)) < 0.6)
        bits, bits_t = hf.key_mask_bits(m)
        dense = np.broadcast_to(m.numpy()[:, None, None, :], (3, 1, n, n))
        w = (n + 31) // 32

        def words(a):
            pad = np.zeros(a.shape[:-1] + (w * 32,), dtype=bool)
            pad[..., :n] = a
            packed = np.packbits(pad, axis=-1, bitorder="little")
            return packed.view("<u4").astype(np.int64)

        got = bits.numpy().astype(np.int64) & 0xFFFFFFFF
        got_t = bits_t.numpy().astype(np.int64) & 0xFFFFFFFF
        assert bits.shape == bits_t.shape == (3, 1, n, w)
        assert np.array_equal(got, words(dense))
        assert np.array_equal(got_t, words(np.swapaxes(dense, -1, -2)))


def test_dense_mask_checks_on_the_host():
    """4-D masks: boolean, or additive with 0 / blocking values only; the
    causal flag survives only when nothing above the diagonal is allowed.
    Host tensors pass the checks and stop at the packer's device check."""
    n = 6
    tril = torch.ones(n, n, dtype=torch.bool).tril()[None, None]
    additive = torch.zeros(1, 1, n, n).masked_fill(~tril, float("-inf"))
    finfo_min = torch.zeros(1, 1, n, n).masked_fill(~tril, torch.finfo(torch.float32).min)
    for m in (tril, additive, finfo_min, tril.expand(2, 4, n, n)):
        with pytest.raises(RuntimeError, match="mask must be a CUDA tensor"):
            hf.dense_mask_bits(m, 2, 4)
    # An additive mask with other values is a bias: no bits, the fp32 values.
    bits, bits_t, causal, bias = hf.dense_mask_bits(additive + 0.5 * tril, 2, 4)
    assert bits is None and causal and bias.dtype == torch.float32
    assert torch.equal(bias, additive + 0.5 * tril)
    _, _, causal, _ = hf.dense_mask_bits(torch.full((1, 1, n, n), 0.25), 2, 4)
    assert not causal
    with pytest.raises(NotImplementedError, match="4-D attention mask"):
        hf.dense_mask_bits(tril.expand(3, 1, n, n), 2, 4)
