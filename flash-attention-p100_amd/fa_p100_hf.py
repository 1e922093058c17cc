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
rows' outputs, which nothing reads, differ.

Also beyond the reference, a causal layer's sliding window (Qwen3's and
Mistral-style `sliding_window`) runs in the kernels: row i sees keys
(i - W, i], as transformers' own sliding-window mask; and packed sequences
(several sequences in one row, marked by `position_ids` that restart, as
transformers' DataCollatorWithFlattening produces them) attend within their
own sequence only, as transformers' packed-sequence mask does for eager and
sdpa (masking_utils.find_packed_sequence_indices). The reference, which
ignores position_ids, attended across the packed sequences.

The kernels run in the autocast dtype (fp16 or bf16; bf16 inputs without
autocast stay bf16); the reference cast everything to fp16.

Every other unsupported request raises NotImplementedError instead of
degrading (fa_p100_hf.py:24-32): other attention / padding masks,
output_attentions, head_mask, a window on non-causal attention, dropout,
head_dim other than 64/128, q_len != kv_len (KV-cache decoding). A scale other
than 1/sqrt(D), which the reference rejected, goes to the kernels.
"""
import warnings

import torch

from fa_p100 import flash_attn, segment_bounds

_IMPL_NAME = "fa_p100"
_warned_cast = False
# enable_fa_p100's forward wrapper hands every attention call of a model call
# the batch's padding and packing as one keyword argument, (kv_len, segs):
#   kv_len: key lengths, int32 (B,) on the model's device, of a padded batch,
#           or None;
#   segs:   packed-sequence bounds (seg_start, seg_end), or _NOT_PACKED once
#           the call's position_ids were found to hold one sequence per row.
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


def fa_p100_attention_forward(module, query, key, value, attention_mask, dropout=0.0,
                              scaling=None, is_causal=None, **kwargs):
    """transformers attention-interface entry point (fa_p100_hf.py:46-142).

    query is (B, Hq, N, D) and key/value (B, Hkv, N, D); returns
    (out (B, N, Hq, D) in query's dtype, None), the contract of
    transformers' sdpa_attention_forward.
    """
    global _warned_cast

    if attention_mask is not None:
        raise NotImplementedError(
            "fa_p100 got an attention mask, but the kernel has no mask input. "
            "Pack sequences to one fixed length so no padding is needed.")
    if kwargs.get("output_attentions", False):
        raise NotImplementedError(
            "fa_p100 never forms the attention probabilities, so "
            "output_attentions=True is not available; use attn_implementation='eager'.")
    if kwargs.get("head_mask") is not None:
        raise NotImplementedError("fa_p100 does not support head_mask.")
    if dropout:
        raise NotImplementedError(f"fa_p100 has no attention dropout (got {dropout}).")

    head_dim = query.size(-1)
    if head_dim not in (64, 128):
        raise NotImplementedError(f"fa_p100 supports head_dim 64 or 128, got {head_dim}.")
    # The reference fixed scale = 1/sqrt(D) and raised on anything else; the
    # kernels take the model's scale (softmax_scale) when it differs.
    softmax_scale = None
    if scaling is not None and abs(scaling - head_dim ** -0.5) > 1e-6:
        softmax_scale = float(scaling)
    if key.size(2) != query.size(2):
        raise NotImplementedError(
            f"fa_p100 needs q_len == kv_len (got q={query.size(2)}, kv={key.size(2)}); "
            "incremental decoding with a KV cache is not supported.")

    if is_causal is None:
        is_causal = getattr(module, "is_causal", True) and query.size(2) > 1
    sliding_window = kwargs.get("sliding_window")
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

    # Padding and packing of the model call (enable_fa_p100's wrapper); when
    # the hook runs without it, packed sequences come from position_ids here.
    kv_len, segs = kwargs.pop(_BOUNDS_KW, None) or (None, None)
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
    out = flash_attn(query, key, value, causal=bool(is_causal), full_precision=full_precision,
                     kv_len=kv_len, sliding_window=sliding_window, segment_ids=segs,
                     softmax_scale=softmax_scale)
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


def enable_fa_p100(model, full_precision=False):
    """Switch `model` onto the kernels and guard the paths they cannot serve.

    Mirrors fa_p100_hf.py:161-213: registers the implementation, points every
    config at it, records `full_precision` on every module, turns the KV cache
    off, and wraps `model.forward` once so that use_cache=True and any
    padding mask other than right padding raise instead of being silently
    ignored; a right-padded mask is served through per-entry key lengths and
    a left-padded one (causal layers) through packed-sequence bounds.
    """
    register()
    _set_impl(model.config, _IMPL_NAME)
    for mod in model.modules():
        if hasattr(mod, "config") and hasattr(mod.config, "_attn_implementation"):
            _set_impl(mod.config, _IMPL_NAME)
        mod._fa_p100_full_precision = full_precision

    # q_len must equal kv_len, so a cache could never be used.
    model.config.use_cache = False
    if getattr(model, "generation_config", None) is not None:
        model.generation_config.use_cache = False

    if not getattr(model, "_fa_p100_guarded", False):
        inner = model.forward

        def guarded(*args, attention_mask=None, use_cache=None, **kwargs):
            # transformers drops the mask before the attention interface sees it
            # for unregistered implementations: this is the last place to catch it.
            kv_len, left = None, None
            if attention_mask is not None and not bool(attention_mask.all()):
                spans = padding_spans(attention_mask)
                if spans is None:
                    raise NotImplementedError(
                        "fa_p100 serves only padding masks whose ones form one run per row "
                        "(right, left or both-sided padding); this mask would be discarded "
                        "silently. Pad at the ends or pack the batch so every position is "
                        "real.")
                first, end = spans
                kv_len = end  # keys past the run exist for no row
                if bool((first > 0).any()):
                    left = first
            # Rejected up front rather than at the first decode step, after a
            # prefill that would have succeeded.
            if use_cache:
                raise NotImplementedError(
                    "fa_p100 needs q_len == kv_len, so it cannot serve a KV cache; it "
                    "is a training kernel. Set generation_config.use_cache = False for "
                    "cache-free generation.")
            # Packed sequences: restarting position_ids (checked once per call).
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
            elif position_ids is not None:
                ref = kwargs.get("input_ids")
                if ref is None:
                    ref = kwargs.get("inputs_embeds")
                if ref is None and args:
                    ref = args[0]
                batch = ref.size(0) if ref is not None else position_ids.size(0)
                segs = _packed_bounds(position_ids, batch)
            kwargs[_BOUNDS_KW] = (kv_len, segs)
            return inner(*args, attention_mask=attention_mask, use_cache=use_cache, **kwargs)

        model.forward = guarded
        model._fa_p100_guarded = True

    return model
