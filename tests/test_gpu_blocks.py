"""Block-sparse layouts, beyond the reference, which raises on block-sparse
patterns (README.md:72-75). A layout of 128 x 128 blocks hides whole blocks;
the kernels step over the visible blocks only. Checked: the GPU packer
against the oracle's lists (bit-exact, integer work); flash_attn with a
block_mask against the float64 oracle with the expanded element mask, over
random, local+global and empty-row layouts, causal or not, GQA, head dims of
every tile width, ragged N, bf16, with dropout and with the run-time options;
the block path bit-identical to the same pattern given as an element mask
(skipping a hidden block only drops exact zeros); (B, N, H, D) views and the
C ABI bit-identical to the op; and a quarter of the blocks running in well
under the time of all of them."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import (FWD_MAX_ABS, GRAD_REL_L2, LSE_MAX_ABS, REF_REL, fa_opts, load_capi,
                     make_inputs, np64)
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"
BS = 128


def nblocks(n):
    return (n + BS - 1) // BS


def random_layout(rng, lb, lh, n, density):
    nb = nblocks(n)
    return rng.random((lb, lh, nb, nb)) < density


def local_global(n, width=1):
    """Each block row sees its own block, `width` blocks either side and
    block column 0 (a BigBird-style local + global pattern)."""
    nb = nblocks(n)
    r, c = np.arange(nb)[:, None], np.arange(nb)[None, :]
    return ((np.abs(r - c) <= width) | (c == 0))[None, None]


def run(q, k, v, do, causal, **kw):
    import fa_p100
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal, **kw)
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    return o.detach(), qg.grad, kg.grad, vg.grad


def check(what, got, q, k, v, do, causal, lse=None, **opts):
    o, dq, dk, dv = (np64(t) for t in got)
    qn, kn, vn, dn = (t.double().numpy() for t in (q, k, v, do))
    ref_o, ref_lse = ora.attention_fwd(qn, kn, vn, causal, **opts)
    assert ora.max_abs(o, ref_o) <= FWD_MAX_ABS, what
    assert ora.rel_max_rms(o, ref_o) < REF_REL, what
    if lse is not None:
        lse = np64(lse)
        fin = np.isfinite(ref_lse)
        assert np.array_equal(np.isfinite(lse), fin), what
        assert ora.max_abs(lse[fin], ref_lse[fin]) <= LSE_MAX_ABS, what
    for name, g, r in zip(("dQ", "dK", "dV"), (dq, dk, dv),
                          ora.attention_bwd(qn, kn, vn, dn, causal, **opts)):
        assert np.isfinite(g).all(), (what, name)
        if not np.any(r):
            assert not np.any(g), (what, name)
            continue
        l2, rr = ora.rel_l2(g, r), ora.rel_max_rms(g, r)
        assert l2 <= GRAD_REL_L2 and rr < REF_REL, (what, name, l2, rr)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("lb,lh,B,Hq,Hkv,N", [(1, 1, 2, 4, 2, 700), (2, 1, 2, 2, 2, 300),
                                              (2, 4, 2, 4, 1, 1000), (1, 8, 1, 8, 4, 128)])
def test_packer_matches_oracle_lists(lb, lh, B, Hq, Hkv, N, causal):
    import fa_p100
    rng = np.random.default_rng(N + lb + lh + causal)
    lay = random_layout(rng, lb, lh, N, 0.4)
    lay[..., 0, :] = False  # an empty block row
    rows, cols = fa_p100.pack_blocks(torch.tensor(lay, device=DEV), B, Hq, Hkv, N, causal)
    ref_rows, ref_cols = ora.block_lists(lay, B, Hq, Hkv, N, causal)
    assert np.array_equal(rows.cpu().numpy(), ref_rows)
    assert np.array_equal(cols.cpu().numpy(), ref_cols)


LAYOUTS = ["random", "local_global", "empty_rows", "all"]


def layout_of(kind, rng, n, lb=1, lh=1):
    if kind == "random":
        return random_layout(rng, lb, lh, n, 0.45)
    if kind == "local_global":
        return local_global(n)
    lay = np.ones((lb, lh, nblocks(n), nblocks(n)), dtype=bool)
    if kind == "empty_rows":  # block rows 1 and 3 see nothing; key block 2 is never seen
        lay[..., [1, 3], :] = False
        lay[..., :, 2] = False
    return lay


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("kind", LAYOUTS)
@pytest.mark.parametrize("B,Hq,Hkv,N,D", [(2, 4, 2, 777, 128), (1, 4, 4, 1024, 64),
                                          (1, 2, 1, 640, 96)])
def test_block_mask_matches_oracle(B, Hq, Hkv, N, D, kind, causal):
    import fa_p100
    rng = np.random.default_rng(N + D + causal)
    lay = layout_of(kind, rng, N, 1, Hq if kind == "random" else 1)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + D)
    bm = torch.tensor(lay, device=DEV)
    got = run(q, k, v, do, causal, block_mask=bm)
    rows, _ = fa_p100.pack_blocks(bm, B, Hq, Hkv, N, causal)
    _, lse = fa_p100._ext.forward_dt(q.to(DEV), k.to(DEV), v.to(DEV), causal, block_rows=rows)
    check(f"{kind} {B},{Hq}/{Hkv},N{N},D{D},causal={causal}", got, q, k, v, do, causal, lse=lse,
          mask=ora.block_layout_mask(lay, N))


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("D", [256, 40])
def test_block_mask_other_widths(D, causal):
    """Width 256 (32-row streamed tiles in the backward: four per block) and
    a head dim below its tile width."""
    rng = np.random.default_rng(D + causal)
    B, Hq, Hkv, N = 2, 4, 2, 600
    lay = random_layout(rng, 2, 1, N, 0.5)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=D)
    got = run(q, k, v, do, causal, block_mask=torch.tensor(lay, device=DEV))
    check(f"D{D} causal={causal}", got, q, k, v, do, causal, mask=ora.block_layout_mask(lay, N))


@pytest.mark.parametrize("causal", [False, True])
def test_block_mask_with_dropout_and_runtime_options(causal):
    """Dropout (its own instantiation), key lengths, ALiBi, a scale, packed
    sequences and, when causal, a window, all with one layout."""
    rng = np.random.default_rng(40 + causal)
    B, Hq, Hkv, N, D = 2, 4, 2, 900, 64
    lay = random_layout(rng, 1, Hq, N, 0.6)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=77)
    p, seed = 0.2, 1234
    lens = [900, 640]
    slopes = np.array([2.0 ** (-8.0 * (h + 1) / Hq) for h in range(Hq)])
    seg = np.stack([np.repeat([0, 1], [500, 400]), np.repeat([3, 4, 5], [100, 300, 500])])
    kw = dict(kv_len=torch.tensor(lens, dtype=torch.int32, device=DEV),
              alibi_slopes=torch.tensor(slopes, dtype=torch.float32, device=DEV),
              softmax_scale=0.1, segment_ids=torch.tensor(seg, device=DEV))
    opts = dict(kv_len=lens, alibi=np.float32(slopes).astype(np.float64),
                scale=np.float32(0.1).item(), segments=seg)
    if causal:
        kw["sliding_window"] = opts["window"] = 300
    bm = torch.tensor(lay, device=DEV)
    got = run(q, k, v, do, causal, block_mask=bm, dropout_p=p, dropout_seed=seed, **kw)
    keep, zs = ora.dropout_keep(seed, p, B * Hq, N)
    mask = ora.block_layout_mask(lay, N)
    check(f"dropout+options causal={causal}", got, q, k, v, do, causal,
          mask=mask, dropout=(keep, zs), **opts)
    # without dropout: the block instantiation alone, against the oracle
    got = run(q, k, v, do, causal, block_mask=bm, **kw)
    check(f"options causal={causal}", got, q, k, v, do, causal, mask=mask, **opts)


@pytest.mark.parametrize("causal", [False, True])
def test_block_mask_equals_element_mask_bit_for_bit(causal):
    """The same pattern as a block layout and as an element mask: hidden
    blocks contribute exact zeros, so skipping them changes no bit. (Causal
    dK/dV: the element-mask path splits a long key tile's dK/dV sum between
    two workgroups and adds the two halves, the block path does not, so
    there they agree to rounding, not bit for bit.)"""
    rng = np.random.default_rng(9 + causal)
    B, Hq, Hkv, N, D = 2, 4, 2, 1000, 128
    lay = random_layout(rng, 1, Hq, N, 0.5)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=5)
    a = run(q, k, v, do, causal, block_mask=torch.tensor(lay, device=DEV))
    m = torch.tensor(ora.block_layout_mask(lay, N), device=DEV)
    b = run(q, k, v, do, causal, attn_mask=m)
    for name, x, y in zip(("o", "dq", "dk", "dv"), a, b):
        if causal and name in ("dk", "dv"):
            assert ora.rel_l2(np64(x), np64(y)) <= 1e-3, name
        else:
            assert torch.equal(x, y), name


def test_block_mask_bf16_bnhd_and_capi():
    """bf16 against the oracle; (B, N, H, D) views bit-identical to dense;
    fa_fwd_ex / fa_bwd_ex with the packed lists bit-identical to the op."""
    import fa_p100
    from test_gpu_bf16 import BF_FWD_MAX_ABS, BF_GRAD_REL_L2, bf16_inputs
    rng = np.random.default_rng(3)
    B, Hq, Hkv, N, D = 2, 8, 2, 555, 128
    lay = torch.tensor(random_layout(rng, B, 1, N, 0.5), device=DEV)
    q, k, v, do = (t.to(DEV) for t in bf16_inputs(B, Hq, Hkv, N, D, seed=19))
    as_bnhd = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)
    dense = [t.clone().requires_grad_(True) for t in (q, k, v)]
    views = [as_bnhd(t).detach().requires_grad_(True) for t in (q, k, v)]
    o1 = fa_p100.flash_attn(*dense, True, block_mask=lay)
    o2 = fa_p100.flash_attn(*views, True, block_mask=lay)
    o1.backward(do)
    o2.backward(as_bnhd(do))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    for x, y in zip(dense, views):
        assert torch.equal(x.grad, y.grad)
    f = lambda t: t.detach().float().cpu().double().numpy()
    mask = ora.block_layout_mask(lay.cpu().numpy(), N)
    ref_o, _ = ora.attention_fwd(f(q), f(k), f(v), True, mask=mask)
    assert ora.max_abs(f(o1), ref_o) <= BF_FWD_MAX_ABS
    for t, r in zip(dense, ora.attention_bwd(f(q), f(k), f(v), f(do), True, mask=mask)):
        assert ora.rel_l2(f(t.grad), r) <= BF_GRAD_REL_L2

    lib = load_capi()
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rows, cols = fa_p100.pack_blocks(lay, B, Hq, Hkv, N, True)
    opts = fa_opts(dtype=1, block_rows=rows, block_cols=cols)
    o, lse = torch.empty_like(q), torch.empty(B, Hq, N, device=DEV)
    assert lib.fa_fwd_ex(p(q), p(k), p(v), p(o), p(lse), B, Hq, Hkv, N, D, 1, opts, s) == 0
    ws_bytes = lib.fa_bwd_workspace_bytes(B, Hq, Hkv, N, D)
    ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    rc = lib.fa_bwd_ex(p(q), p(k), p(v), p(do), p(o), p(lse), p(dq), p(dk), p(dv), p(ws),
                       ws_bytes, B, Hq, Hkv, N, D, 1, opts, s)
    assert rc == 0, lib.fa_error_string(rc)
    torch.cuda.synchronize()
    assert torch.equal(o, o1)
    for got, t in zip((dq, dk, dv), dense):
        assert torch.equal(got, t.grad)
    # the backward without block_cols is refused
    rc = lib.fa_bwd_ex(p(q), p(k), p(v), p(do), p(o), p(lse), p(dq), p(dk), p(dv), p(ws),
                       ws_bytes, B, Hq, Hkv, N, D, 1, fa_opts(dtype=1, block_rows=rows), s)
    assert rc == 10018


def test_block_mask_argument_errors():
    import fa_p100
    q, k, v, _ = (t.to(DEV) for t in make_inputs(1, 2, 2, 256, 64, seed=1))
    with pytest.raises(ValueError, match="block_mask must be"):
        fa_p100.flash_attn(q, k, v, block_mask=torch.ones(3, 3, dtype=torch.bool, device=DEV))
    with pytest.raises(ValueError, match="boolean"):
        fa_p100.flash_attn(q, k, v, block_mask=torch.ones(2, 2, device=DEV))
    with pytest.raises(ValueError, match="does not combine"):
        fa_p100.flash_attn(q, k, v, block_mask=torch.ones(2, 2, dtype=torch.bool, device=DEV),
                           attn_mask=torch.ones(256, 256, dtype=torch.bool, device=DEV))
    with pytest.raises(ValueError, match="packed block_mask"):
        fa_p100.flash_attn(q, k, v, block_mask=(torch.zeros(1, dtype=torch.int32, device=DEV),
                                                torch.zeros(1, dtype=torch.int32, device=DEV)))


def test_sparse_layout_runs_faster_than_dense():
    """A quarter of the blocks visible (local band, non-causal) at B=1 H=8
    N=8192 D=128: fwd+bwd in under half the time of the all-visible layout,
    which itself stays within 10% of the plain op."""
    import fa_p100
    B, H, N, D = 1, 8, 8192, 128
    nb = nblocks(N)
    r, c = np.arange(nb)[:, None], np.arange(nb)[None, :]
    band = torch.tensor((np.abs(r - c) < nb // 8)[None, None], device=DEV)
    full = torch.ones(1, 1, nb, nb, dtype=torch.bool, device=DEV)
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, H, H, N, D, seed=2))
    qg, kg, vg = (t.requires_grad_(True) for t in (q, k, v))

    def ms(**kw):
        blocks = None
        if "block_mask" in kw:
            blocks = fa_p100.pack_blocks(kw.pop("block_mask"), B, H, H, N, False)
        for _ in range(3):
            fa_p100.flash_attn(qg, kg, vg, False, block_mask=blocks).backward(do)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            fa_p100.flash_attn(qg, kg, vg, False, block_mask=blocks).backward(do)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 10

    plain, dense, sparse = ms(), ms(block_mask=full), ms(block_mask=band)
    frac = float(band.float().mean())
    print(f"plain {plain:.3f} ms, all blocks {dense:.3f} ms, {frac:.0%} of blocks {sparse:.3f} ms")
    assert sparse < 0.5 * dense and dense < 1.1 * plain
