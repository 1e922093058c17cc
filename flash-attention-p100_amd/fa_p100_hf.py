"""HuggingFace transformers attention hook for the gfx950 FlashAttention kernels.

Drop-in for the reference module of the same name (fa_p100_hf.py): registers
the kernels under the attention-implementation name "fa_p100", so a supported
model (Qwen3, Llama-style decoders) runs on them with

    from fa_p100_hf import enable_fa_p100
    model = AutoModelForCausalLM.from_config(cfg).half().cuda()
    enable_fa_p100(model)

Checked against transformers 5.15: `ALL_ATTENTION_FUNCTIONS` is a mapping whose
`__setitem__` registers a local implementation, `config._attn_implementation`
is a recursive setter, and masking_utils returns no mask at all for an
implementation that is not in the mask registry (masking_utils.py:819-820).
That last point is relied on: the kernel applies causality itself, so no
(B, H, N, N) mask is ever built. The price is that a padding mask would be
dropped without a word, which is why `enable_fa_p100` wraps `model.forward`
to look at it first (fa_p100_hf.py:13-22, 183-211). Beyond the reference,
which rejects every padding mask, a right-padded 2-D mask (each row ones, then
zeros) is served exactly: its row sums go to the kernels as per-entry key
lengths, so every position attends to the real keys only, as with eager
attention and the same mask. Left (and both-sided) padding is served on
causal layers too: the pads form a packed sequence of their own (below), so
every real token attends to the real keys only, as with eager; only the pad
rows' outputs, which nothing reads, differ. Any other 2-D mask (holes inside
a row) goes to the kernels as a bit mask over the keys, on top of the layer's
causal mask and window, as eager combines them; a query row left with no key
gets a zero output where eager's is arbitrary.

A 4-D mask handed to the model (boolean, True = attend, or additive) reaches
every layer as it is (masking_utils returns 4-D masks unchanged); as with
eager and sdpa it alone decides which keys each query sees. Boolean masks and
additive ones with only 0 and blocking values (<= -1e4 or -inf) go to the
kernels as a bit mask; any other additive mask is an attention bias and goes
to them as such (fp32), added to the scaled scores as eager adds it. The
causal flag is kept only when the mask allows no key above the diagonal,
where it changes nothing but the tiles skipped.

Also beyond the reference, a causal layer's sliding window (Qwen3's and
Mistral-style `sliding_window`) runs in the kernels: row i sees keys
(i - W, i], as transformers' own sliding-window mask; and packed sequences
(several sequences in one row, marked by `position_ids` that restart, as
transformers' DataCollatorWithFlattening produces them) attend within their
own sequence only, as transformers' packed-sequence mask does for eager and
sdpa (masking_utils.find_packed_sequence_indices) when the model gets no
attention mask. The reference, which ignores position_ids, attended across the
packed sequences.

The kernels run in the autocast dtype (fp16 or bf16; bf16 inputs without
autocast stay bf16); the reference cast everything to fp16.

Attention dropout (a layer's `attention_dropout` in training), which the
reference rejects (fa_p100_hf.py:83-85), runs in the kernels with keep bits
drawn per call from torch's default generator (fa_p100.dropout_bits).

KV-cache steps (q_len != kv_len: decoding one token, or a chunk of the
prompt after cached ones), which the reference rejects (fa_p100_hf.py:100-105),
run in the kernels with the causal diagonal aligned at the bottom right (the
last query row against the last key), without a padding mask.

Every other unsupported request raises NotImplementedError instead of
degrading (fa_p100_hf.py:24-32): output_attentions,
head_mask, attention sinks (s_aux) and logit soft-capping (softcap), which
other models pass to the attention interface, a window on non-causal
attention, a head_dim that is not a multiple of 8 up to 256 (up to 128 with
an additive float mask, which goes to the kernels as a bias), a cached step
with padding or a mask. A scale other than 1/sqrt(D),
which the reference rejected, goes to the kernels.
"""
import warnings

import torch

from fa_p100 import flash_attn, pack_mask, segment_bounds

_IMPL_NAME = "fa_p100"
_warned_cast = False
# enable_fa_p100's forward wrapper hands every attention call of a model call
# the batch's padding, packing and mask as one keyword argument,
# (kv_len, segs, mask):
#   kv_len: key lengths, int32 (B,) on the model's device, of a padded batch,
#           or None;
#   segs:   packed-sequence bounds (seg_start, seg_end), or _NOT_PACKED once
#           the call's position_ids were found to hold one sequence per row;
#   mask:   None, or (bits, bits_t, causal, bias): the packed words of a
#           mask (pack_mask's layout; None for a bias), for a 4-D mask
#           whether the causal flag may stay on (None for a 2-D padding mask,
#           which the layer's causal mask and window apply on top of), and
#           an additive 4-D mask that carries a bias (fp32), or None.
# The mask is packed once per model call rather than once per layer.
# transformers passes a model's **kwargs down to each decoder layer and from
# there to the attention interface, and gradient checkpointing replays a
# layer with the same kwargs, so a layer recomputed in the backward pass sees
# the same bounds as its first forward (state kept beside the call, such as a
# context variable, is gone by then).
_BOUNDS_KW = "fa_p100_bounds"
_NOT_PACKED = ()


def packed_segment_ids(position_ids, batch):
    """Sequence ids of packed rows, as transformers derives them: a new
    sequence starts wherever a position id is not its predecessor's plus one
    (masking_utils.find_packed_sequence_indices). Returns (batch, N) ids, or
    None when every row holds one sequence. Synchronises with the device."""
    pos = position_ids
    if pos.dim() == 1:
        pos = pos[None]
    first = pos[:, :1] - 1
    ids = (torch.diff(pos, prepend=first, dim=-1) != 1).cumsum(-1)
    if not bool((ids[:, -1] != 0).any()):
        return None
    if ids.size(0) != batch:
        ids = ids.expand(batch, -1)
    return ids


def _packed_bounds(position_ids, batch):
    ids = packed_segment_ids(position_ids, batch)
    return _NOT_PACKED if ids is None else segment_bounds(ids)


def right_padding_lengths(mask):
    """Row sums of a right-padded 2-D mask (each row: ones, then zeros, at
    least one one) as int32, or None for any other mask."""
    if mask.dim() != 2:
        return None
    m = mask != 0
    lens = m.sum(dim=1)
    ref = torch.arange(m.size(1), device=m.device)[None, :] < lens[:, None]
    if not bool(torch.equal(m, ref)) or not bool((lens > 0).all()):
        return None
    return lens.to(torch.int32)


def padding_spans(mask):
    """(first, end) int32 (B,) of a 2-D mask whose ones form one contiguous,
    non-empty run per row (left, right or both-sided padding), or None for
    any other mask."""
    if mask.dim() != 2:
        return None
    m = mask != 0
    lens = m.sum(dim=1)
    first = m.int().argmax(dim=1)  # first one (0 for an all-zero row, caught below)
    idx = torch.arange(m.size(1), device=m.device)[None, :]
    ref = (idx >= first[:, None]) & (idx < (first + lens)[:, None])
    if not bool(torch.equal(m, ref)) or not bool((lens > 0).all()):
        return None
    return first.to(torch.int32), (first + lens).to(torch.int32)


def _left_padding_segments(first, n):
    """Sequence ids (B, n) that put each row's left pads in a sequence of
    their own (0) and the rest in another (1), so that causal real tokens
    see real keys only."""
    idx = torch.arange(n, device=first.device)[None, :]
    return (idx >= first[:, None].long()).to(torch.int32)


# Additive mask values at or below this block a key: exp(s - 1e4) is exactly
# 0 in fp32 next to any allowed key's logit.
_BLOCKED = -1.0e4


def key_mask_bits(mask):
    """(bits, bits_t), int32 (B, 1, N, ceil(N/32)) each, of a 2-D padding
    mask: every query row may attend key j of entry b iff mask[b, j] != 0.
    Built from the (B, N) mask with a few device ops, without an N x N
    boolean tensor."""
    m = mask != 0
    b, n = m.shape
    w = (n + 31) // 32
    flat = torch.zeros(b, w * 32, dtype=torch.int64, device=m.device)
    flat[:, :n] = m.long()
    shifts = torch.arange(32, dtype=torch.int64, device=m.device)
    words = (flat.view(b, w, 32) << shifts).sum(-1)  # in [0, 2^32)
    bits = _as_int32(words)[:, None, None, :].expand(b, 1, n, w).contiguous()
    # Transposed: key j's words over the query rows, all set (rows past N
    # clear) for a real key, none for a pad.
    full = torch.full((w,), (1 << 32) - 1, dtype=torch.int64, device=m.device)
    full[-1] = (1 << (n - 32 * (w - 1))) - 1
    rows = _as_int32(full)
    bits_t = torch.where(m[:, None, :, None], rows, torch.zeros_like(rows)).contiguous()
    return bits, bits_t


def _as_int32(words):
    """int64 values in [0, 2^32) as the int32 with the same 32 bits."""
    return torch.where(words >= (1 << 31), words - (1 << 32), words).to(torch.int32)


def dense_mask_bits(mask, batch, heads):
    """(bits, bits_t, causal, bias) of a 4-D attention mask (B or 1, 1 or
    heads, N, N) as transformers hands it to the attention interface:
    boolean (True = attend), or additive. An additive mask whose values are
    only 0 (attend) and blocking ones (-inf, or <= -1e4) becomes bits like a
    boolean one (bias None); any other additive mask is a bias: it goes to
    the kernels as fp32 `attn_bias` (bits None), blocking values included
    (exp underflows to exactly 0 there). `causal` tells whether the mask
    allows no key above the diagonal."""
    if mask.dim() != 4 or mask.size(-1) != mask.size(-2) or mask.size(0) not in (1, batch) \
            or mask.size(1) not in (1, heads):
        raise NotImplementedError(
            f"fa_p100 takes a 4-D attention mask of shape ({batch} or 1, 1 or {heads}, N, N); "
            f"got {tuple(mask.shape)}.")
    bias = None
    if mask.dtype == torch.bool:
        allowed = mask
    elif mask.is_floating_point():
        allowed = mask > _BLOCKED
        if not bool((mask[allowed] == 0).all()):
            bias = mask.float()
    else:
        raise NotImplementedError(
            f"fa_p100 takes a boolean or floating attention mask, got {mask.dtype}.")
    causal = not bool(torch.triu(allowed, diagonal=1).any())
    if bias is not None:
        return None, None, causal, bias
    bits, bits_t = pack_mask(allowed, batch, heads)
    return bits, bits_t, causal, None


def fa_p100_attention_forward(module, query, key, value, attention_mask, dropout=0.0,
                              scaling=None, is_causal=None, **kwargs):
    """transformers attention-interface entry point (fa_p100_hf.py:46-142).

    query is (B, Hq, N, D) and key/value (B, Hkv, N, D); returns
    (out (B, N, Hq, D) in query's dtype, None), the contract of
    transformers' sdpa_attention_forward.
    """
    global _warned_cast

    if kwargs.get("output_attentions", False):
        raise NotImplementedError(
            "fa_p100 never forms the attention probabilities, so "
            "output_attentions=True is not available; use attn_implementation='eager'.")
    if kwargs.get("head_mask") is not None:
        raise NotImplementedError("fa_p100 does not support head_mask.")
    # Terms of other models' attention that the kernels do not compute:
    # learnable attention sinks (gpt-oss and others pass them as s_aux, an
    # extra logit per head in the softmax denominator) and logit soft-capping
    # (Gemma 2: softcap * tanh(s / softcap)). Ignoring either would change the
    # output without an error.
    if kwargs.get("s_aux") is not None:
        raise NotImplementedError(
            "fa_p100 does not support attention sinks (s_aux); use attn_implementation='eager'.")
    if kwargs.get("softcap") is not None:
        raise NotImplementedError(
            "fa_p100 does not support logit soft-capping (softcap); "
            "use attn_implementation='eager'.")

    head_dim = query.size(-1)
    if not (8 <= head_dim <= 256 and head_dim % 8 == 0):
        raise NotImplementedError(
            f"fa_p100 supports head_dim multiples of 8 up to 256, got {head_dim}.")
    # The reference fixed scale = 1/sqrt(D) and raised on anything else; the
    # kernels take the model's scale (softmax_scale) when it differs.
    softmax_scale = None
    if scaling is not None and abs(scaling - head_dim ** -0.5) > 1e-6:
        softmax_scale = float(scaling)
    # q_len != kv_len: a KV cache (decoding, chunked prefill). The kernels
    # align the causal diagonal at the bottom right, the last query row with
    # the last key row, as the cached positions require (the reference
    # raised, fa_p100_hf.py:100-105).
    cached = key.size(2) != query.size(2)

    if is_causal is None:
        is_causal = getattr(module, "is_causal", True) and query.size(2) > 1
    # Padding, packing and mask of the model call (enable_fa_p100's wrapper).
    kv_len, segs, mask = kwargs.pop(_BOUNDS_KW, None) or (None, None, None)
    if attention_mask is not None and mask is None:  # a 4-D mask, no wrapper
        mask = dense_mask_bits(attention_mask, query.size(0), query.size(1))
    if mask is not None and mask[3] is not None and head_dim > 128:
        raise NotImplementedError(
            f"fa_p100 takes an additive float mask (an attention bias) up to head_dim 128, "
            f"got {head_dim}; use a boolean mask or attn_implementation='eager'.")
    sliding_window = kwargs.get("sliding_window")
    if mask is not None and mask[2] is not None:
        # A 4-D mask alone decides which keys each query sees (eager adds it
        # to the logits, sdpa passes it with is_causal=False).
        is_causal, sliding_window, kv_len, segs = mask[2], None, None, _NOT_PACKED
    if cached and (mask is not None or kv_len is not None
                   or (segs is not None and segs is not _NOT_PACKED)):
        raise NotImplementedError(
            f"fa_p100 serves q_len != kv_len (q={query.size(2)}, kv={key.size(2)}: a KV cache) "
            "without padding, packing or an attention mask; run the cached steps unpadded.")
    if sliding_window is not None and (not is_causal or sliding_window <= 0):
        raise NotImplementedError(
            f"fa_p100 serves sliding windows on causal attention only; this layer asks for "
            f"a window of {sliding_window} with is_causal={is_causal}.")

    # The kernels take fp16 or bf16. Under autocast, Qwen3's fp32 q_norm/k_norm
    # weights and rotary tables hand q and k over in fp32 while v is in the
    # autocast dtype, so casting to that dtype is the normal path. Without
    # autocast, bf16 inputs stay bf16 and anything else goes to fp16 (the
    # reference's only format), with one warning.
    orig_dtype = query.dtype
    autocast_dt = (torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda")
                   else None)
    if autocast_dt in (torch.float16, torch.bfloat16):
        target = autocast_dt
    elif query.dtype == key.dtype == value.dtype == torch.bfloat16:
        target = torch.bfloat16
    else:
        target = torch.float16
    if query.dtype != target or key.dtype != target or value.dtype != target:
        if autocast_dt != target and not _warned_cast:
            warnings.warn(
                f"fa_p100 casts q={query.dtype} k={key.dtype} v={value.dtype} to {target} "
                "outside fp16/bf16 autocast; the kernels take fp16 or bf16. Run the step "
                "under torch.autocast('cuda', torch.float16) or torch.bfloat16.",
                stacklevel=2)
            _warned_cast = True
        query, key, value = query.to(target), key.to(target), value.to(target)

    # Without the wrapper, packed sequences come from position_ids here.
    position_ids = kwargs.get("position_ids")
    if segs is None and position_ids is not None:
        segs = _packed_bounds(position_ids, query.size(0))
    if segs is _NOT_PACKED or segs is None:
        segs = None
    else:
        if tuple(segs[0].shape) != (query.size(0), query.size(2)) \
                or segs[0].device != query.device:
            raise NotImplementedError(
                "fa_p100: the packed position_ids given to the model do not match this "
                "attention call's batch and length.")

    # GQA/MQA go to the kernel as they are: no repeat_kv copies.
    full_precision = getattr(module, "_fa_p100_full_precision", False)
    if kv_len is not None:
        if kv_len.numel() != query.size(0) or kv_len.device != query.device:
            raise NotImplementedError(
                "fa_p100: the padding mask given to the model does not match this "
                "attention call's batch.")
    # transformers passes the layer's attention_dropout in training, 0 in eval.
    out = flash_attn(query, key, value, causal=bool(is_causal), full_precision=full_precision,
                     kv_len=kv_len, sliding_window=sliding_window, segment_ids=segs,
                     softmax_scale=softmax_scale,
                     attn_mask=None if mask is None or mask[0] is None else mask[:2],
                     attn_bias=None if mask is None else mask[3],
                     dropout_p=float(dropout) if dropout else None)
    return out.transpose(1, 2).contiguous().to(orig_dtype), None


def register():
    """Add "fa_p100" to transformers' attention registry (idempotent)."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    ALL_ATTENTION_FUNCTIONS[_IMPL_NAME] = fa_p100_attention_forward
    return _IMPL_NAME


def _set_impl(config, name):
    config._attn_implementation = name
    for sub in getattr(config, "sub_configs", {}) or {}:
        child = getattr(config, sub, None)
        if child is not None:
            _set_impl(child, name)


def enable_fa_p100(model, full_precision=False, use_cache=False):
    """Switch `model` onto the kernels and guard the paths they cannot serve.

    Mirrors fa_p100_hf.py:161-213: registers the implementation, points every
    config at it, records `full_precision` on every module, turns the KV cache
    off (unless use_cache=True), and wraps `model.forward` once so that the
    attention mask, which transformers would drop before the attention
    interface, reaches the kernels: a right-padded mask as per-entry key
    lengths, a left-padded one (causal layers) as packed-sequence bounds, any
    other 2-D mask as a key bit mask, and a 4-D mask as a bit mask of its
    own, each prepared once per model call.

    The reference raised on use_cache (its kernels needed q_len == kv_len);
    here cached steps run with the causal diagonal aligned at the bottom
    right, so a call may pass use_cache=True (and enable_fa_p100(model,
    use_cache=True) leaves the model's cache setting alone). Cached steps take
    no padding mask: a padded batch raises there.
    """
    register()
    _set_impl(model.config, _IMPL_NAME)
    for mod in model.modules():
        if hasattr(mod, "config") and hasattr(mod.config, "_attn_implementation"):
            _set_impl(mod.config, _IMPL_NAME)
        mod._fa_p100_full_precision = full_precision

    # As the reference: training needs no cache. Cached steps (q_len !=
    # kv_len) are served when a caller asks for them.
    if not use_cache:
        model.config.use_cache = False
        if getattr(model, "generation_config", None) is not None:
            model.generation_config.use_cache = False

    if not getattr(model, "_fa_p100_guarded", False):
        inner = model.forward

        def guarded(*args, attention_mask=None, use_cache=None, **kwargs):
            # transformers drops a 2-D mask before the attention interface sees
            # it for unregistered implementations: this is the last place to
            # catch it. A 4-D mask reaches every layer; it is packed here once.
            kv_len, left, mask = None, None, None
            ref = kwargs.get("input_ids")
            if ref is None:
                ref = kwargs.get("inputs_embeds")
            if ref is None and args:
                ref = args[0]
            if attention_mask is not None and attention_mask.dim() == 4:
                batch = ref.size(0) if ref is not None else attention_mask.size(0)
                mask = dense_mask_bits(attention_mask, batch, attention_mask.size(1))
            elif attention_mask is not None and not bool(attention_mask.all()):
                spans = padding_spans(attention_mask)
                if spans is None:
                    mask = key_mask_bits(attention_mask) + (None, None)
                else:
                    first, end = spans
                    kv_len = end  # keys past the run exist for no row
                    if bool((first > 0).any()):
                        left = first
            # Packed sequences: restarting position_ids (checked once per call)
            # when the model gets no mask, as transformers' mask creation does.
            # Left padding rides on the same bounds: the pads form a sequence
            # of their own, so real tokens (causal) see real keys only.
            segs = _NOT_PACKED
            position_ids = kwargs.get("position_ids")
            if left is not None:
                # Position ids of the pads are arbitrary (generate() sets them to
                # 1); a restart between two real tokens would mean packing too.
                # kv_len is each row's end of real tokens.
                if position_ids is not None:
                    pos = position_ids if position_ids.dim() == 2 else position_ids[None]
                    idx = torch.arange(1, pos.size(-1), device=pos.device)[None, :]
                    real_pair = (idx > left[:, None].long()) & (idx < kv_len[:, None].long())
                    restart = (torch.diff(pos, dim=-1) != 1) & real_pair
                    if bool(restart.any()):
                        raise NotImplementedError(
                            "fa_p100 does not serve left padding and packed sequences "
                            "together.")
                segs = segment_bounds(_left_padding_segments(left, attention_mask.size(1)))
            elif position_ids is not None and attention_mask is None:
                batch = ref.size(0) if ref is not None else position_ids.size(0)
                segs = _packed_bounds(position_ids, batch)
            kwargs[_BOUNDS_KW] = (kv_len, segs, mask)
            return inner(*args, attention_mask=attention_mask, use_cache=use_cache, **kwargs)

        model.forward = guarded
        model._fa_p100_guarded = True

    return model
