"""FlashAttention-2 for the AMD Instinct MI355X (gfx950) as a torch autograd Function.

Drop-in for the reference module of the same name (fa_p100.py): same public
names, arguments and return values.

    from fa_p100 import flash_attn
    o = flash_attn(q, k, v, causal=True)   # q: (B, Hq, N, D) fp16 on the GPU
                                           # k, v: (B, Hkv, N, D), Hq % Hkv == 0

D is any multiple of 8 up to 256 (the reference: 64 or 128); N is arbitrary; Hkv == Hq is
multi-head, Hkv == 1 multi-query, anything between grouped-query. The kernels
are hand-written HIP for gfx950 (fp16 MFMA with fp32 accumulation), built
in-tree by build.py into libfa_mi355x.so, and reached through the
`fa_p100_ext` torch binding. Unlike
the reference (fa_p100.py:21-28), importing does not compile anything: the
binding must already be built, and importing fails loudly if it is not.

`full_precision` is accepted for API compatibility (fa_p100.py:48). The
reference used it to switch its forward from fp16 to fp32 multiply-adds; on
MFMA every fp16 product is exact in the fp32 accumulator, so both settings run
the same kernel.
"""
import importlib.machinery
import importlib.util
import math
import os
import sysconfig

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_EXT_NAME = "fa_p100_ext"


def _load_ext():
    """Load the in-tree torch binding; raise ImportError if it is not built."""
    path = os.path.join(_HERE, _EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is not built. Run `python {os.path.join(_HERE, 'build.py')}` "
            "(or __graft_entry__.build()) first; there is no fallback path.")
    loader = importlib.machinery.ExtensionFileLoader(_EXT_NAME, path)
    spec = importlib.util.spec_from_file_location(_EXT_NAME, path, loader=loader)
    mod = importlib.util.module_from_spec(spec)
    loader.exec_module(mod)
    return mod


_ext = _load_ext()

# Rows and keys per block of a block-sparse layout (flash_attn's block_mask).
BLOCK_SIZE = 128


def _bnhd_storage(t):
    """The dense (B, N, H, D) tensor a (B, H, N, D) view `t` is a transpose of,
    or None."""
    tt = t.transpose(1, 2)
    return tt if tt.is_contiguous() else None


class _FlashAttnP100(torch.autograd.Function):
    """Autograd wrapper; same saved state and return types as fa_p100.py:31-45.

    When q, k and v are all (B, H, N, D) views of dense (B, N, H, D) storage
    (the projections' layout, which the HF hook passes), the kernels read and
    write that layout directly: no copies in, and o and the gradients come
    back as (B, H, N, D) views of (B, N, H, D) tensors. Results are
    bit-identical to the dense path.
    """

    @staticmethod
    def forward(ctx, q, k, v, causal, full_precision, kv_len=None, window=0, alibi=None,
                segs=None, scale=0.0, mask=None, drop=None, bias=None, blocks=None):
        # (B, N, H, D) path when q is not dense (B, H, N, D) but is dense
        # (B, N, H, D), and k, v are dense (B, N, H, D) too (with one kv head
        # they are dense in both layouts).
        qb = None if q.is_contiguous() else _bnhd_storage(q)
        kb, vb = _bnhd_storage(k), _bnhd_storage(v)
        ctx.causal = causal
        ctx.kv_len = kv_len
        ctx.window = window
        ctx.alibi = alibi
        ctx.segs = segs
        ctx.scale = scale
        ctx.mask = mask
        # drop: (seed, p, scale). Only the seed is kept for the backward, which
        # draws the keep bits again (the draw is a pure function of the seed):
        # keeping the forward's bit planes would hold B*Hq*N*ceil(N/32)*4 bytes
        # per call from the forward to the backward.
        ctx.drop = drop
        # bias: fp32 (B|1, Hq|1, N, N) view with dense rows (see flash_attn).
        ctx.bias = bias.detach() if bias is not None else None
        # blocks: the block-sparse lists (block_rows, block_cols) of pack_blocks.
        ctx.blocks = blocks
        b_rows, b_cols = blocks if blocks is not None else (None, None)
        seg_start, seg_end = segs if segs is not None else (None, None)
        bits, bits_t = mask if mask is not None else (None, None)
        z, z_scale = None, 1.0
        if drop is not None:
            z, _, z_scale = dropout_bits(drop[0], drop[1], q.size(0), q.size(1), q.size(2),
                                         q.device, transposed=False, causal=causal)
        ctx.bnhd = qb is not None and kb is not None and vb is not None
        if ctx.bnhd:
            ob, lse = _ext.forward_bnhd(qb, kb, vb, causal, kv_len, window, alibi, seg_start,
                                        seg_end, scale, bits, drop=z, drop_scale=z_scale,
                                        bias=ctx.bias, block_rows=b_rows)
            ctx.save_for_backward(qb, kb, vb, ob, lse)
            return ob.transpose(1, 2)
        if (q.dtype == torch.bfloat16 or kv_len is not None or window or alibi is not None
                or segs is not None or scale or mask is not None or drop is not None
                or bias is not None or blocks is not None or k.size(2) != q.size(2)):
            o, lse = _ext.forward_dt(q, k, v, causal, kv_len, window, alibi, seg_start, seg_end,
                                     scale, bits, drop=z, drop_scale=z_scale, bias=ctx.bias,
                                     block_rows=b_rows)
        else:
            o, lse = _ext.forward(q, k, v, causal, full_precision)
        ctx.save_for_backward(q, k, v, o, lse)
        return o

    @staticmethod
    def backward(ctx, grad_o):
        seg_start, seg_end = ctx.segs if ctx.segs is not None else (None, None)
        bits, bits_t = ctx.mask if ctx.mask is not None else (None, None)
        b_rows, b_cols = ctx.blocks if ctx.blocks is not None else (None, None)
        z, z_t, z_scale = None, None, 1.0
        if ctx.drop is not None:  # the forward's keep bits, drawn again from its seed
            z, z_t, z_scale = dropout_bits(ctx.drop[0], ctx.drop[1], grad_o.size(0),
                                           grad_o.size(1), grad_o.size(2), grad_o.device,
                                           causal=ctx.causal)
        dbias = None
        if ctx.bias is not None and ctx.needs_input_grad[12]:  # bias is input 12
            B, H, N = grad_o.size(0), grad_o.size(1), grad_o.size(2)
            dbias = torch.zeros(B, H, N, N, dtype=torch.float32, device=grad_o.device)
        if ctx.bnhd:
            qb, kb, vb, ob, lse = ctx.saved_tensors
            gb = grad_o.transpose(1, 2).contiguous()
            dq, dk, dv = _ext.backward_bnhd(qb, kb, vb, gb, ob, lse, ctx.causal, ctx.kv_len,
                                            ctx.window, ctx.alibi, seg_start, seg_end, ctx.scale,
                                            bits, bits_t, z, z_t, z_scale, ctx.bias, dbias,
                                            b_rows, b_cols)
            return (dq.transpose(1, 2), dk.transpose(1, 2), dv.transpose(1, 2),
                    None, None, None, None, None, None, None, None, None,
                    _reduce_bias_grad(dbias, ctx.bias), None)
        q, k, v, o, lse = ctx.saved_tensors
        # dq is accumulated in fp32 and handed back in q's dtype (fa_p100.py:45);
        # backward_half_dq rounds it to fp16 in the kernel (bit-identical to
        # `_ext.backward(...)[0].to(torch.float16)`) instead of a separate cast,
        # and backward_dt to bf16 for bf16 inputs.
        g = grad_o.contiguous()
        if (q.dtype == torch.bfloat16 or ctx.kv_len is not None or ctx.window
                or ctx.alibi is not None or ctx.segs is not None or ctx.scale
                or ctx.mask is not None or ctx.drop is not None or ctx.bias is not None
                or ctx.blocks is not None or k.size(2) != q.size(2)):
            dq, dk, dv = _ext.backward_dt(q, k, v, g, o, lse, ctx.causal, ctx.kv_len, ctx.window,
                                          ctx.alibi, seg_start, seg_end, ctx.scale, bits, bits_t,
                                          z, z_t, z_scale, ctx.bias, dbias, b_rows, b_cols)
        else:
            dq, dk, dv = _ext.backward_half_dq(q, k, v, g, o, lse, ctx.causal)
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), None, None, None, None, None,
                None, None, None, None, _reduce_bias_grad(dbias, ctx.bias), None)


def _reduce_bias_grad(dbias, bias):
    """The full (B, Hq, N, N) gradient summed over the dimensions the bias
    shares (size 1), in the bias's shape."""
    if dbias is None:
        return None
    dims = [d for d in (0, 1) if bias.size(d) == 1 and dbias.size(d) != 1]
    return dbias.sum(dim=dims, keepdim=True) if dims else dbias


def flash_attn(q, k, v, causal=False, full_precision=False, kv_len=None, sliding_window=None,
               alibi_slopes=None, segment_ids=None, softmax_scale=None, attn_mask=None,
               dropout_p=None, dropout_seed=None, attn_bias=None, block_mask=None):
    """Attention over fp16 GPU tensors (fa_p100.py:48-55).

    q is (B, Hq, N, D); k and v are (B, Hkv, N, D) with Hq a multiple of Hkv
    and D a multiple of 8 up to 256 (the reference: 64 or 128; attn_bias only
    up to 128). scale = 1/sqrt(D).
    Causal masking is top-left aligned (key j is hidden from query i when
    j > i).

    k and v may also hold a different number of rows Nk than q's N (the
    reference requires N == Nk): KV-cache decoding (N = 1) and chunked
    prefill (N < Nk). Causal masking then aligns the last query row with the
    last key row (key j is hidden from query i when j > i + Nk - N; with
    N > Nk the first N - Nk rows see no key and get o = 0 and zero
    gradients), and sliding windows and ALiBi count from that diagonal. Not
    with segment_ids, attn_mask, dropout_p, attn_bias or block_mask.

    Beyond the reference (which raises on anything but fp16 and on padding
    masks, README.md:72-75):
      * q, k and v may also all be bf16: the products then run on the bf16
        MFMA with fp32 accumulation, and o and the gradients come back in bf16;
      * kv_len, an int32 tensor (B,) on q's device, gives each batch entry's
        key length (right padding): entry b has keys [0, kv_len[b]) (values
        clamped to [1, N]); every query row, pad rows included, attends to
        those keys only, and the gradients of k, v past kv_len[b] are zero;
      * sliding_window W (causal only): query row i attends to keys
        (i - W, i]. A row that then sees no key at all (only possible with
        kv_len: a pad row more than W past its entry's length) gets o = 0 and
        zero gradients;
      * alibi_slopes, a float32 tensor (Hq,) on q's device: query head h adds
        the bias -alibi_slopes[h] * |i - j| to its scaled score of key j
        (ALiBi, in the symmetric form that also serves non-causal attention;
        under causal masking j <= i, so it is -slope * (i - j)). The slopes
        are constants: no gradient flows to them;
      * segment_ids, an integer tensor (B, N) on q's device: several
        sequences packed into each batch entry. Each maximal run of equal ids
        is one sequence, and a token attends to the keys of its own sequence
        only (causal within it when causal=True), as if each sequence had been
        run alone. Also accepted: the (seg_start, seg_end) pair segment_bounds()
        makes from such ids, for callers that reuse one packing across calls;
      * softmax_scale: a positive float used in place of 1/sqrt(D) (the
        reference fixes 1/sqrt(D), fa_p100_ext.cu:71); the returned LSE is in
        units of the scaled logits;
      * attn_mask, a boolean tensor on q's device of shape (N, N), (B, N, N)
        or (B or 1, 1 or Hq, N, N): key j is hidden from query i wherever it
        is False (torch scaled_dot_product_attention's boolean attn_mask),
        on top of every other mask, causal included. A row left with no key
        gets o = 0 and zero gradients. Also accepted: the (bits, bits_t)
        pair pack_mask() makes, for callers that reuse one mask across calls.
        The mask is a constant: no gradient flows to it;
      * dropout_p in [0, 1): attention dropout. Each probability of the
        softmax (normalised over every key) is dropped with that
        probability and the kept ones are scaled by 1 / (1 - p); the
        returned o is (P * Z / (1 - p)) V and the gradients are those of
        that o. The keep bits Z come from a counter-based hash of
        dropout_seed (64-bit; drawn from torch's default CPU generator when
        None, so torch.manual_seed makes runs repeat, and checkpoint
        recomputation, which replays that generator, draws the same seed)
        through dropout_bits(). The backward draws the same bits again
        from the seed rather than keeping the forward's, so no bit planes
        are held between the passes. Under HIP graph capture the seed must
        be given (a seed drawn on the host at capture time would be
        replayed unchanged by every replay): every replay then uses that
        seed's bits. The drawn rate is p rounded to a multiple of 1/65536,
        and the scale matches it exactly;
      * attn_bias, a floating tensor of shape (N, N), (B, N, N) or
        (B|1, Hq|1, N, N) on q's device: added to the scaled scores before
        the masks and the softmax (torch scaled_dot_product_attention's
        float attn_mask), in fp32. When it requires grad its gradient (the
        gradient of the scaled scores, summed over the dimensions it
        shares) comes back in its own shape and dtype;
      * block_mask, a boolean block-sparse layout on q's device of shape
        (nb, nb), (B, nb, nb) or (B or 1, Hq or 1, nb, nb), nb =
        ceil(N / BLOCK_SIZE): query i may attend key j only if block
        (i // BLOCK_SIZE, j // BLOCK_SIZE) is True, on top of the causal and
        other masks. The kernels step over the visible blocks only, so the
        time scales with their number. A row with no visible key gets o = 0
        and zero gradients. Also accepted: the (block_rows, block_cols) pair
        pack_blocks() makes, for callers that reuse one layout across calls.
        Not with attn_mask or attn_bias.
    """
    if k.size(2) != q.size(2) and (segment_ids is not None or attn_mask is not None
                                   or dropout_p or attn_bias is not None
                                   or block_mask is not None):
        raise ValueError(
            f"q has {q.size(2)} rows and k, v {k.size(2)}: segment_ids, attn_mask, dropout_p, "
            "attn_bias and block_mask need q_len == kv_len")
    if block_mask is not None and (attn_mask is not None or attn_bias is not None):
        raise ValueError("block_mask does not combine with attn_mask or attn_bias")
    if attn_bias is not None and q.size(-1) > 128:
        raise ValueError(f"attn_bias needs a head dim up to 128, got {q.size(-1)}")
    window = 0
    if sliding_window is not None:
        window = int(sliding_window)
        if window <= 0 or not causal:
            raise ValueError("sliding_window must be positive and needs causal=True")
    if alibi_slopes is not None:
        if alibi_slopes.dim() != 1 or alibi_slopes.numel() != q.size(1):
            raise ValueError(f"alibi_slopes must have shape ({q.size(1)},), got "
                             f"{tuple(alibi_slopes.shape)}")
        alibi_slopes = alibi_slopes.detach().float().contiguous()
    segs = None
    if segment_ids is not None:
        pair = isinstance(segment_ids, (tuple, list))
        shape = tuple(segment_ids[0].shape) if pair else tuple(segment_ids.shape)
        if shape != (q.size(0), q.size(2)):
            raise ValueError(f"segment_ids must have shape ({q.size(0)}, {q.size(2)}), got "
                             f"{shape}")
        segs = tuple(segment_ids) if pair else segment_bounds(segment_ids)
    scale = 0.0
    if softmax_scale is not None:
        scale = float(softmax_scale)
        if not (scale > 0.0 and math.isfinite(scale)):
            raise ValueError(f"softmax_scale must be positive and finite, got {softmax_scale}")
    mask = None
    if attn_mask is not None:
        if isinstance(attn_mask, (tuple, list)):
            mask = tuple(attn_mask)
            want = (q.size(0), q.size(2), (q.size(2) + 31) // 32)
            got = tuple(mask[0].shape)
            if (len(mask) != 2 or len(got) != 4 or (got[0], got[2], got[3]) != want
                    or got[1] not in (1, q.size(1)) or tuple(mask[1].shape) != got):
                raise ValueError(f"packed attn_mask must be two ({want[0]}, 1 or {q.size(1)}, "
                                 f"{want[1]}, {want[2]}) tensors from pack_mask, got "
                                 f"{[tuple(t.shape) for t in mask]}")
        else:
            mask = pack_mask(attn_mask, q.size(0), q.size(1))
    drop = None
    if dropout_p:
        p = float(dropout_p)
        if not 0.0 <= p < 1.0:
            raise ValueError(f"dropout_p must lie in [0, 1), got {dropout_p}")
        if not q.is_cuda:  # the binding's own check and message, before any drawing
            raise RuntimeError("q must be a CUDA tensor")
        if dropout_seed is None:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    "dropout under HIP graph capture needs an explicit dropout_seed: a seed "
                    "drawn on the host now would repeat in every replay")
            dropout_seed = int(torch.randint(0, 2 ** 63 - 1, (), dtype=torch.int64))
        drop = (int(dropout_seed), p, _ext.dropout_scale(p))
    bias = None
    if attn_bias is not None:
        bias = attn_bias
        if not bias.is_floating_point():
            raise ValueError(f"attn_bias must be a floating tensor, got {bias.dtype}")
        if bias.dim() == 2:
            bias = bias[None, None]
        elif bias.dim() == 3:
            bias = bias[:, None]
        n = q.size(2)
        if bias.dim() != 4 or tuple(bias.shape[2:]) != (n, n) \
                or bias.size(0) not in (1, q.size(0)) or bias.size(1) not in (1, q.size(1)):
            raise ValueError(f"attn_bias must be (N, N), (B, N, N) or (B|1, Hq|1, N, N) with "
                             f"N = {n}, got {tuple(attn_bias.shape)}")
        bias = bias.float()
        if bias.stride(-1) != 1 or bias.stride(-2) != n:
            bias = bias.contiguous()
    blocks = None
    if block_mask is not None:
        if isinstance(block_mask, (tuple, list)):
            blocks = tuple(block_mask)
            nb = (q.size(2) + BLOCK_SIZE - 1) // BLOCK_SIZE
            want = [(q.size(0), q.size(1), nb, nb + 1),
                    (q.size(0), k.size(1), nb, (q.size(1) // k.size(1)) * nb + 1)]
            if len(blocks) != 2 or [tuple(t.shape) for t in blocks] != want:
                raise ValueError(f"packed block_mask must be the two int32 tensors of "
                                 f"pack_blocks, shaped {want}, got "
                                 f"{[tuple(t.shape) for t in blocks]}")
        else:
            blocks = pack_blocks(block_mask, q.size(0), q.size(1), k.size(1), q.size(2), causal)
    return _FlashAttnP100.apply(q, k, v, causal, full_precision, kv_len, window, alibi_slopes,
                                segs, scale, mask, drop, bias, blocks)


def dropout_bits(seed, p, batch, heads, n, device, transposed=True, causal=False):
    """(bits, bits_t, scale) of attention dropout: int32 keep bits
    (batch, heads, n, ceil(n/32)) in the mask layout and its transpose (bit
    set = keep; None when `transposed` is False), drawn by one HIP kernel from
    the 64-bit `seed` with drop probability p (fa_dropout_bits in the C ABI
    states the draw), and the scale 1 / (1 - drawn rate) of the kept
    probabilities. With `causal` the bits of keys j > i (row i) are cleared
    and not drawn (fa_dropout_bits_causal): causal attention over n keys
    never reads them, so its results do not change, and the draw does about
    half the work."""
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError(f"dropout bits are drawn on the GPU, got device {device}")
    index = device.index if device.index is not None else torch.cuda.current_device()
    seed = int(seed) % (1 << 64)
    if seed >= 1 << 63:  # the binding takes a signed 64-bit value with the same bits
        seed -= 1 << 64
    bits, bits_t = _ext.dropout_bits(seed, float(p), batch, heads, n, index, bool(transposed),
                                     bool(causal))
    return bits, bits_t, _ext.dropout_scale(float(p))


def pack_blocks(block_mask, batch, heads, kv_heads, n, causal=False):
    """(block_rows, block_cols) of a block-sparse layout: the int32 lists the
    kernels step over (fa_options.block_rows / block_cols in the C ABI), built
    by one HIP kernel on the layout's device.

    block_mask is boolean, (nb, nb), (B, nb, nb) or (B or 1, heads or 1, nb,
    nb) with nb = ceil(n / BLOCK_SIZE): query row i may attend key j only if
    block_mask[..., i // BLOCK_SIZE, j // BLOCK_SIZE] is True. With causal,
    blocks above the diagonal are left out (a causal call never reads them).
    Packing once and passing the pair as flash_attn's block_mask saves the
    packing in every call with the same layout.
    """
    m = block_mask
    if m.dtype != torch.bool:
        raise ValueError(f"block_mask must be a boolean tensor (True = visible), got {m.dtype}")
    if m.dim() == 2:
        m = m[None, None]
    elif m.dim() == 3:
        m = m[:, None]
    nb = (n + BLOCK_SIZE - 1) // BLOCK_SIZE
    if m.dim() != 4 or tuple(m.shape[2:]) != (nb, nb) or m.size(0) not in (1, batch) \
            or m.size(1) not in (1, heads):
        raise ValueError(f"block_mask must be ({nb}, {nb}), ({batch}, {nb}, {nb}) or ({batch} "
                         f"or 1, {heads} or 1, {nb}, {nb}) for N = {n} (blocks of "
                         f"{BLOCK_SIZE}), got {tuple(block_mask.shape)}")
    rows, cols = _ext.pack_blocks(m, batch, heads, kv_heads, n, bool(causal))
    return rows, cols


def pack_mask(attn_mask, batch, heads):
    """(bits, bits_t), int32 (batch, 1 or heads, N, ceil(N/32)) each, of a
    boolean mask (N, N), (B, N, N) or (B or 1, 1 or heads, N, N).

    Bit j % 32 of bits[b, h, i, j // 32] is set iff query i may attend key j
    (attn_mask True); bits_t holds the transpose (bit i % 32 of
    bits_t[b, h, j, i // 32]), which the backward reads. These are the words
    the kernels take (fa_options.mask / mask_t in the C ABI); one HIP kernel
    packs them on the mask's device.
    """
    m = attn_mask
    if m.dtype != torch.bool:
        raise ValueError(f"attn_mask must be a boolean tensor (True = attend), got {m.dtype}")
    if m.dim() == 2:
        m = m[None, None]
    elif m.dim() == 3:
        m = m[:, None]
    if m.dim() != 4 or m.size(-1) != m.size(-2) or m.size(0) not in (1, batch) \
            or m.size(1) not in (1, heads):
        raise ValueError(f"attn_mask must be (N, N), ({batch}, N, N) or ({batch} or 1, 1 or "
                         f"{heads}, N, N), got {tuple(attn_mask.shape)}")
    bits, bits_t = _ext.pack_mask(m, True)
    if bits.size(0) != batch:  # one plane set shared by the batch
        shape = (batch,) + tuple(bits.shape[1:])
        bits, bits_t = bits.expand(shape).contiguous(), bits_t.expand(shape).contiguous()
    return bits, bits_t


def segment_bounds(segment_ids):
    """(seg_start, seg_end), int32 (B, N) each, of packed sequences.

    A sequence is a maximal run of equal ids along a row: token i belongs to
    the run [seg_start[b, i], seg_end[b, i]). These are the bounds the kernels
    take (fa_options.seg_start / seg_end in the C ABI). Computed with a few
    device-side scans; nothing is copied to the host.
    """
    s = segment_ids
    B, N = s.shape
    idx = torch.arange(N, device=s.device, dtype=torch.int64).expand(B, N)
    change = s[:, 1:] != s[:, :-1]  # a new run starts at i + 1
    starts = torch.ones(B, N, dtype=torch.bool, device=s.device)
    starts[:, 1:] = change
    ends = torch.ones(B, N, dtype=torch.bool, device=s.device)  # a run ends after i
    ends[:, :-1] = change
    seg_start = torch.where(starts, idx, torch.zeros_like(idx)).cummax(dim=1).values
    seg_end = torch.where(ends, idx + 1, torch.full_like(idx, N)).flip(1).cummin(dim=1).values.flip(1)
    return seg_start.to(torch.int32).contiguous(), seg_end.to(torch.int32).contiguous()


def _expand_kv(k, n_head):
    """Repeat each K/V head across the query heads that share it (fa_p100.py:58-62)."""
    if k.size(1) == n_head:
        return k
    return k.repeat_interleave(n_head // k.size(1), dim=1)


def reference(q, k, v, causal=False):
    """Plain-torch attention for comparison, as the reference ships (fa_p100.py:65-75).

    A helper for users' own checks; `flash_attn` never calls it.
    """
    k = _expand_kv(k, q.size(1))
    v = _expand_kv(v, q.size(1))
    scale = 1.0 / math.sqrt(q.size(-1))
    s = (q.float() @ k.float().transpose(-1, -2).contiguous()) * scale
    if causal:
        n = q.size(-2)
        mask = torch.triu(torch.ones(n, n, device=q.device, dtype=torch.bool), 1)
        s = s.masked_fill(mask, float("-inf"))
    return (s.softmax(-1) @ v.float()).to(q.dtype)
