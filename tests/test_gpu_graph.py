"""Forward + backward captured in a HIP graph (torch.cuda.CUDAGraph) and
replayed: the launches take torch's current stream, allocate through the
caching allocator only (no memset: the backward's split-tile counters are
cleared by its own preprocess kernel), so a captured step replays exactly.

Each replay follows eager work on the same buffers (the graph's outputs
overwritten with NaN, an unrelated eager step, a synchronisation) and is
checked bit for bit against the eager results on the same inputs; new input
values copied into the captured input buffers give the new eager results.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
CASES = {
    "causal MHA D128": dict(B=1, Hq=4, Hkv=4, N=1024, D=128, causal=True, mask=False),
    "GQA D64 dense": dict(B=2, Hq=8, Hkv=2, N=640, D=64, causal=False, mask=False),
    "causal D128 with a mask": dict(B=1, Hq=2, Hkv=2, N=512, D=128, causal=True, mask=True),
}


def step(ext, q, k, v, do, causal, opts):
    o, lse = ext.forward_dt(q, k, v, causal, **opts["fwd"])
    dq, dk, dv = ext.backward_dt(q, k, v, do, o, lse, causal, **opts["bwd"])
    return o, lse, dq, dk, dv


@pytest.mark.parametrize("name", list(CASES))
def test_captured_step_replays_exactly(name):
    import fa_p100
    ext = fa_p100._ext
    c = CASES[name]
    print(name, flush=True)
    g = torch.Generator(device=DEV).manual_seed(5)
    B, Hq, Hkv, N, D = (c[x] for x in ("B", "Hq", "Hkv", "N", "D"))

    def rand(h):
        return torch.randn(B, h, N, D, generator=g, device=DEV).half()

    q, k, v, do = rand(Hq), rand(Hkv), rand(Hkv), rand(Hq)
    opts = {"fwd": {}, "bwd": {}}
    if c["mask"]:
        allowed = torch.rand(B, Hq, N, N, generator=g, device=DEV) < 0.8
        bits, bits_t = fa_p100.pack_mask(allowed, B, Hq)
        opts = {"fwd": {"mask": bits}, "bwd": {"mask": bits, "mask_t": bits_t}}
    ref = [t.clone() for t in step(ext, q, k, v, do, c["causal"], opts)]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up before capture, as torch requires
        for _ in range(2):
            step(ext, q, k, v, do, c["causal"], opts)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step(ext, q, k, v, do, c["causal"], opts)

    other = [rand(Hq), rand(Hkv), rand(Hkv), rand(Hq)]
    for rep in range(4):
        for t in outs:
            t.fill_(float("nan"))
        step(ext, *other, c["causal"], {"fwd": {}, "bwd": {}})  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for label, got, want in zip(("o", "lse", "dq", "dk", "dv"), outs, ref):
            assert torch.equal(got, want), (name, rep, label)

    # New values in the captured input buffers.
    for t in (q, k, v, do):
        t.copy_(torch.randn(t.shape, generator=g, device=DEV).half())
    ref2 = [t.clone() for t in step(ext, q, k, v, do, c["causal"], opts)]
    graph.replay()
    torch.cuda.synchronize()
    for label, got, want in zip(("o", "lse", "dq", "dk", "dv"), outs, ref2):
        assert torch.equal(got, want), (name, "new inputs", label)
    assert not torch.equal(ref2[0], ref[0])
