"""Benchmark: fwd+bwd attention TFLOPS and % of MI355X fp16 dense MFMA peak.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C3] [--no-cpu]
    python bench.py --config C5 --steps 5 --warmup 2   (Qwen3-shaped training step)

Workload (BASELINE.json metric, quoted on the headline shape): config C3,
causal MHA, B=1, Hq=Hkv=8, N=4096, D=128, fp16 inputs from one seeded CPU
generator (q, k, v, dO in that order, N(0,1)), resident in HBM before timing.

One step = the hot path through the C ABI on torch's current stream:
fa_fwd, then fa_bwd_preprocess (Dv), then fa_bwd_main (dK, dV, dQ), into
preallocated buffers. K steps are timed between two device synchronisations;
HIP events recorded on the same stream between the launches give each
kernel's average duration. The same step through the public autograd op
(`flash_attn(...).backward(g)`, which adds output and workspace allocation;
its backward writes dQ as fp16) is timed as `api_ms_per_step`, in short runs
alternating with the C-ABI step (`abi_interleaved_ms_per_step`), so that the
two compare at one clock state; torch's own GPU
scaled_dot_product_attention (flash and memory-efficient backends, fp16,
same inputs) as `torch_sdpa_gpu`, for comparison.

FLOPs follow the reference's convention (attention.cu:219, bwd.cu:246):
fwd = 4*B*Hq*N^2*D, halved for causal; bwd = 2.5x fwd.

Beside the headline, the metric's D=64 leg (causal B=1 Hq=Hkv=16 N=4096
D=64, the reference's BENCH.log:268 shape) is timed the same way under "d64".

Before the W warmup steps the step runs untimed for about half a second, so
that the GPU has left its idle clocks whatever W is (W=5 steps are ~1 ms of
work); the timed region is exactly K steps either way.

roofline: the dominant kernel (fa_bwd_main) at its algorithmic FLOPs (the
bwd count above) over its average duration, measured with HIP events on the
launch stream in a second pass of K steps; the peak is the fp16 dense MFMA
rate, 2.4 GHz x 256 CUs x 4 SIMDs x 1024 FLOP/clk = 2516.6 TFLOP/s (AMD's
published 2.5 PFLOP/s). profiles/ holds rocprofv3 kernel-trace summaries of
this same command, whose bwd_main average agrees with the event time.

cpu_baseline (BASELINE.md's CPU plan): torch's CPU
scaled_dot_product_attention fwd+bwd in fp32 on the whole headline workload
(same inputs as the GPU), 2 warmups then the median of 5 timed iterations, on
the host threads of the GPU box's CPU share; the float64-pinned oracle's
float32 numpy restatement (the "port") is timed beside it on one
(batch, head) slice.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "flash-attention-p100_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

# MI355X dense fp16 MFMA rate: 2.4 GHz x 256 CUs x 4 SIMDs x 1024 FLOP/clk
# (AMD publishes 2.5 PFLOP/s dense, no sparsity).
PEAK_FP16_TFLOPS = 2.4e9 * 256 * 4 * 1024 / 1e12  # 2516.58
P100_HEADLINE_TFLOPS = 120.259e9 / 45.485e-3 / 1e12  # 45.485 ms on P100

CONFIGS = {
    "C2": dict(B=1, Hq=16, Hkv=16, N=2048, D=64, causal=True, s=1.0,
               desc="causal MHA fwd+bwd fp16 B=1 Hq=Hkv=16 N=2048 D=64"),
    "C3": dict(B=1, Hq=8, Hkv=8, N=4096, D=128, causal=True, s=1.0,
               desc="causal MHA fwd+bwd fp16 B=1 Hq=Hkv=8 N=4096 D=128 (headline)"),
    "C4": dict(B=2, Hq=32, Hkv=8, N=3001, D=128, causal=False, s=0.5,
               desc="non-causal GQA fwd+bwd fp16 B=2 Hq=32 Hkv=8 N=3001 D=128"),
    "D64": dict(B=1, Hq=16, Hkv=16, N=4096, D=64, causal=True, s=1.0,
                desc="causal MHA fwd+bwd fp16 B=1 Hq=Hkv=16 N=4096 D=64 (the metric's D=64 leg)"),
}
SPIN_UP_S = 0.5  # untimed running before the warmup steps (clock ramp)


QWEN3_C5 = dict(layers=28, hidden=1024, heads=16, kv_heads=8, head_dim=128, inter=3072,
                vocab=151936, seq=8192)


def qwen3_bench(steps, warmup, impls=("fa_p100", "sdpa")):
    """a random-init Qwen3-0.6B-shaped decoder, B=1, seq
    8192, token ids uniform over the vocabulary, one forward + backward
    (fp16 autocast) per step, attention through the HF hook ("fa_p100"), and
    the same step with transformers' "sdpa" attention on the same weights
    (`impls` picks which of the two run, for kernel traces of one)."""
    import torch
    from transformers import Qwen3Config, Qwen3ForCausalLM
    import fa_p100_hf

    q = QWEN3_C5
    cfg = Qwen3Config(vocab_size=q["vocab"], hidden_size=q["hidden"],
                      intermediate_size=q["inter"], num_hidden_layers=q["layers"],
                      num_attention_heads=q["heads"], num_key_value_heads=q["kv_heads"],
                      head_dim=q["head_dim"], max_position_embeddings=q["seq"], use_cache=False)
    torch.manual_seed(0)
    with torch.device("cuda"):
        model = Qwen3ForCausalLM(cfg)
    model.train()
    g = torch.Generator("cuda").manual_seed(0)
    ids = torch.randint(0, q["vocab"], (1, q["seq"]), device="cuda", generator=g)

    def step():
        model.zero_grad(set_to_none=True)
        with torch.autocast("cuda", torch.float16):
            loss = model(ids, labels=ids).loss
        loss.backward()
        return loss

    out = {}
    for impl in impls:
        if impl == "fa_p100":
            fa_p100_hf.enable_fa_p100(model)
        else:
            model.config._attn_implementation = "sdpa"
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            loss = step()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        out[impl] = {"ms_per_step": round(ms, 2),
                     "tokens_per_s": round(q["seq"] / (ms * 1e-3), 1),
                     "loss": round(loss.item(), 4)}
    return out


def flops(c):
    f = 4.0 * c["B"] * c["Hq"] * c["N"] ** 2 * c["D"]
    if c["causal"]:
        f /= 2
    return f, 2.5 * f


def make_inputs(c, torch):
    g = torch.Generator().manual_seed(0)
    shp_q = (c["B"], c["Hq"], c["N"], c["D"])
    shp_k = (c["B"], c["Hkv"], c["N"], c["D"])
    out = []
    for shp in (shp_q, shp_k, shp_k, shp_q):
        out.append((torch.randn(*shp, generator=g) * c["s"]).half())
    return out


def load_capi():
    lib = ctypes.CDLL(os.path.join(PKG, "libfa_mi355x.so"))
    vp, i, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    lib.fa_fwd.argtypes = [vp] * 5 + [i] * 7 + [vp]
    lib.fa_bwd_preprocess.argtypes = [vp] * 4 + [sz] + [i] * 4 + [vp]
    lib.fa_bwd_main.argtypes = [vp] * 5 + [sz] + [vp] * 3 + [i] * 6 + [vp]
    lib.fa_bwd_workspace_bytes.argtypes = [i] * 5
    lib.fa_bwd_workspace_bytes.restype = sz
    lib.fa_error_string.restype = ctypes.c_char_p
    return lib


class FaOptions(ctypes.Structure):
    """struct fa_options of include/fa_mi355x.h (same field order and types)."""
    _fields_ = [("dtype", ctypes.c_int), ("layout", ctypes.c_int),
                ("kv_len", ctypes.c_void_p), ("window", ctypes.c_int),
                ("alibi_slopes", ctypes.c_void_p), ("seg_start", ctypes.c_void_p),
                ("seg_end", ctypes.c_void_p), ("scale", ctypes.c_float),
                ("mask", ctypes.c_void_p), ("mask_t", ctypes.c_void_p),
                ("mask_heads", ctypes.c_int), ("drop", ctypes.c_void_p),
                ("drop_t", ctypes.c_void_p), ("drop_scale", ctypes.c_float),
                ("bias", ctypes.c_void_p), ("bias_stride_b", ctypes.c_longlong),
                ("bias_stride_h", ctypes.c_longlong), ("dbias", ctypes.c_void_p),
                ("kv_rows", ctypes.c_int), ("block_rows", ctypes.c_void_p),
                ("block_cols", ctypes.c_void_p)]


def feature_paths(c, steps, warmup):
    """fwd+bwd ms per step through the general pair (fa_fwd_ex, fa_bwd_ex) on
    the same inputs, with each optional input the reference lacks: the step
    as timed above but with options (plain, for comparison), an all-true
    boolean mask packed once (the packing is per model call, not per layer),
    dropout 0.1 with its keep bits drawn in every step (as in training:
    fa_dropout_bits_causal for a causal workload, as flash_attn draws them
    there, else fa_dropout_bits), both, and an fp32 (1, Hq, N, N) bias with
    and without its gradient (dbias zeroed in every step). Back-to-back
    steps on one stream, wall clock. The block runs after the headline and
    D=64 measurements, whose load lowers the clock a little, so the cases run
    in rounds (each case a short run per round) and `vs_plain` gives each
    case's time over plain_ex's, measured in the same rounds."""
    import torch
    lib = load_capi()
    vp, i, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    opts_t = ctypes.POINTER(FaOptions)
    lib.fa_fwd_ex.argtypes = [vp] * 5 + [i] * 6 + [opts_t, vp]
    lib.fa_bwd_ex.argtypes = [vp] * 10 + [sz] + [i] * 6 + [opts_t, vp]
    lib.fa_pack_mask.argtypes = [vp, i, i, vp, vp, vp]
    lib.fa_dropout_bits.argtypes = [ctypes.c_uint64, ctypes.c_float, i, i, vp, vp, vp]
    lib.fa_dropout_bits_causal.argtypes = lib.fa_dropout_bits.argtypes
    lib.fa_dropout_scale.argtypes = [ctypes.c_float]
    lib.fa_dropout_scale.restype = ctypes.c_float
    dev = torch.device("cuda:0")
    B, Hq, Hkv, N, D, causal = c["B"], c["Hq"], c["Hkv"], c["N"], c["D"], int(c["causal"])
    q, k, v, do = (t.to(dev) for t in make_inputs(c, torch))
    o, lse = torch.empty_like(q), torch.empty(B, Hq, N, device=dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws_bytes = lib.fa_bwd_workspace_bytes(B, Hq, Hkv, N, D)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    W = (N + 31) // 32
    mask = torch.ones(B, N, N, dtype=torch.uint8, device=dev)
    m, m_t = (torch.empty(B, N, W, dtype=torch.int32, device=dev) for _ in range(2))
    z, z_t = (torch.empty(B * Hq, N, W, dtype=torch.int32, device=dev) for _ in range(2))
    bias = torch.randn(1, Hq, N, N, device=dev)
    dbias = torch.empty(B, Hq, N, N, device=dev)
    stream = torch.cuda.current_stream(dev)
    s = ctypes.c_void_p(stream.cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())

    def check(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {lib.fa_error_string(rc).decode()}")

    check(lib.fa_pack_mask(P(mask), B, N, P(m), P(m_t), s), "fa_pack_mask")
    zs = lib.fa_dropout_scale(0.1)

    def opts(with_mask=False, with_drop=False, with_bias=False, grad=False):
        f = FaOptions()
        if with_mask:
            f.mask, f.mask_t, f.mask_heads = m.data_ptr(), m_t.data_ptr(), 1
        if with_drop:
            f.drop, f.drop_t, f.drop_scale = z.data_ptr(), z_t.data_ptr(), zs
        if with_bias:
            f.bias, f.bias_stride_b, f.bias_stride_h = bias.data_ptr(), 0, N * N
            if grad:
                f.dbias = dbias.data_ptr()
        return f

    cases = {"plain_ex": opts(), "mask_all_true": opts(with_mask=True),
             "dropout_0.1": opts(with_drop=True),
             "mask_and_dropout": opts(with_mask=True, with_drop=True),
             "bias": opts(with_bias=True), "bias_with_grad": opts(with_bias=True, grad=True)}
    out = {}
    # Arguments built once, so that the host stays well ahead of the GPU.
    pz, pzt = P(z), P(z_t)
    fwd_args = (P(q), P(k), P(v), P(o), P(lse), B, Hq, Hkv, N, D, causal)
    bwd_args = (P(q), P(k), P(v), P(do), P(o), P(lse), P(dq), P(dk), P(dv), P(ws), ws_bytes,
                B, Hq, Hkv, N, D, causal)
    drawer = lib.fa_dropout_bits_causal if causal else lib.fa_dropout_bits

    def make_step(f):
        fp = ctypes.pointer(f)
        draw, zero = bool(f.drop), bool(f.dbias)

        def step(seed):
            if draw:
                check(drawer(seed, 0.1, B * Hq, N, pz, pzt, s), "dropout draw")
            if zero:
                dbias.zero_()
            check(lib.fa_fwd_ex(*fwd_args, fp, s), "fa_fwd_ex")
            check(lib.fa_bwd_ex(*bwd_args, fp, s), "fa_bwd_ex")
        return step

    runs = {name: make_step(f) for name, f in cases.items()}
    for name, step in runs.items():
        for n in range(warmup):
            step(n)
    # Every case runs once per round, in short runs, so that clock drift over
    # the block reaches all cases alike; each case's time is its total over
    # the rounds, and `vs_plain` its ratio to plain_ex's.
    rounds = 5
    per = max(1, steps // rounds)
    tot = {name: 0.0 for name in runs}
    seed = warmup
    for _ in range(rounds):
        for name, step in runs.items():
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(per):
                step(seed)
                seed += 1
            torch.cuda.synchronize()
            tot[name] += time.perf_counter() - t0
    for name in runs:
        out[name + "_ms"] = round(tot[name] * 1e3 / (rounds * per), 4)
    out["vs_plain"] = {name: round(tot[name] / tot["plain_ex"], 3)
                       for name in runs if name != "plain_ex"}
    return out


def gpu_bench(c, steps, warmup, copy_mib=0, compare=True):
    import torch
    import fa_p100  # noqa: F401  (fails loudly if the binding is not built)

    lib = load_capi()
    dev = torch.device("cuda:0")
    if copy_mib:
        # A plain device copy of known size, so a counter run (FETCH_SIZE,
        # WRITE_SIZE) of this same command can calibrate the counters' scale.
        src = torch.ones(copy_mib * 2**20 // 4, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    q, k, v, do = (t.to(dev) for t in make_inputs(c, torch))
    B, Hq, Hkv, N, D, causal = c["B"], c["Hq"], c["Hkv"], c["N"], c["D"], int(c["causal"])
    o = torch.empty_like(q)
    lse = torch.empty(B, Hq, N, device=dev)
    ws_bytes = lib.fa_bwd_workspace_bytes(B, Hq, Hkv, N, D)
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    dq = torch.empty(B, Hq, N, D, device=dev)
    dk, dv = torch.empty_like(k), torch.empty_like(v)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    pq, pk, pv, pdo, po, plse, pws, pdq, pdk, pdv = map(P, (q, k, v, do, o, lse, ws, dq, dk, dv))
    stream = torch.cuda.current_stream(dev)
    s = ctypes.c_void_p(stream.cuda_stream)

    def check(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {lib.fa_error_string(rc).decode()}")

    def step(ev=None):
        if ev is not None:
            ev[0].record(stream)
        check(lib.fa_fwd(pq, pk, pv, po, plse, B, Hq, Hkv, N, D, causal, 0, s), "fa_fwd")
        if ev is not None:
            ev[1].record(stream)
        check(lib.fa_bwd_preprocess(pdo, po, plse, pws, ws_bytes, B, Hq, N, D, s),
              "fa_bwd_preprocess")
        if ev is not None:
            ev[2].record(stream)
        check(lib.fa_bwd_main(pq, pk, pv, pdo, pws, ws_bytes, pdq, pdk, pdv, B, Hq, Hkv, N, D,
                              causal, s), "fa_bwd_main")
        if ev is not None:
            ev[3].record(stream)

    t_spin = time.perf_counter()
    while time.perf_counter() - t_spin < SPIN_UP_S:
        for _ in range(10):
            step()
        torch.cuda.synchronize()
    for _ in range(warmup):
        step()
    # The timed steps run back to back with nothing else on the stream; a
    # second pass with events between the kernels gives the per-kernel split
    # (event records between kernels add gaps, so that pass is not the one
    # the step time comes from).
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    torch.cuda.synchronize()
    for i in range(steps):
        step(evs[i])
    torch.cuda.synchronize()
    fwd_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / steps
    pre_ms = sum(e[1].elapsed_time(e[2]) for e in evs) / steps
    main_ms = sum(e[2].elapsed_time(e[3]) for e in evs) / steps

    out = dict(wall_ms=wall_ms, fwd_ms=fwd_ms, pre_ms=pre_ms, main_ms=main_ms,
               device=torch.cuda.get_device_name(0))
    if not compare:
        return out
    # Same step through the public autograd op.
    import fa_p100 as fa
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))

    def api_step():
        for t in (qa, ka, va):
            t.grad = None
        fa.flash_attn(qa, ka, va, bool(causal)).backward(do)

    for _ in range(warmup):
        api_step()
    # Interleaved with the C-ABI step in short alternating runs, so that both
    # see the same clock state (run after the headline, a block of either
    # alone would read the GPU at a different clock).
    rounds = 4
    per = max(1, steps // rounds)
    t_api = t_abi = 0.0
    for _ in range(rounds):
        for fn, is_api in ((step, False), (api_step, True)):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(per):
                fn()
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
            if is_api:
                t_api += dt
            else:
                t_abi += dt
    api_ms = t_api * 1e3 / (rounds * per)
    abi_ms = t_abi * 1e3 / (rounds * per)
    out.update(api_ms=api_ms, abi_interleaved_ms=abi_ms,
               sdpa=gpu_sdpa(c, q, k, v, do, steps, warmup))
    return out


def gpu_sdpa(c, q, k, v, do, steps, warmup):
    """torch's own GPU scaled_dot_product_attention fwd+bwd on the same inputs
    (fp16), each fused backend that accepts them, for comparison only."""
    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = {}
    for name, be in (("flash", SDPBackend.FLASH_ATTENTION),
                     ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
        def sd():
            for t in (qa, ka, va):
                t.grad = None
            with sdpa_kernel([be]):
                torch.nn.functional.scaled_dot_product_attention(
                    qa, ka, va, is_causal=c["causal"],
                    enable_gqa=c["Hq"] != c["Hkv"]).backward(do)
        try:
            for _ in range(max(warmup, 1)):
                sd()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                sd()
            torch.cuda.synchronize()
            ms = (time.perf_counter() - t0) * 1e3 / steps
            f_fwd, f_bwd = flops(c)
            out[name] = {"ms_per_step": round(ms, 4),
                         "tflops": round((f_fwd + f_bwd) / (ms * 1e-3) / 1e12, 2)}
        except RuntimeError as ex:
            out[name] = {"unavailable": str(ex).splitlines()[0][:160]}
    return out


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads():
    """Host threads of this job's CPU share: OMP_NUM_THREADS when the box
    sets it (16 per GPU on the MI355X pool), else every CPU."""
    try:
        return max(1, int(os.environ["OMP_NUM_THREADS"]))
    except (KeyError, ValueError):
        return os.cpu_count() or 1


def cpu_baseline(c, port_budget_s=10.0):
    """BASELINE.md's CPU plan: torch's CPU scaled_dot_product_attention
    fwd+bwd, fp32, on the whole workload (the GPU's inputs, in fp32), 2
    warmups then the median of 5 timed iterations. The oracle's numpy fp32
    restatement (the "port") is timed beside it on one (batch, head) slice."""
    import numpy as np
    import torch
    from oracle import attention as ora

    threads = cpu_threads()
    torch.set_num_threads(threads)
    f_fwd, f_bwd = flops(c)
    q, k, v, do = make_inputs(c, torch)
    tq, tk, tv = (t.float().requires_grad_(True) for t in (q, k, v))
    tdo = do.float()

    def sdpa():
        for t in (tq, tk, tv):
            t.grad = None
        torch.nn.functional.scaled_dot_product_attention(
            tq, tk, tv, is_causal=c["causal"], enable_gqa=c["Hq"] != c["Hkv"]).backward(tdo)

    for _ in range(2):
        sdpa()
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        sdpa()
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    value = (f_fwd + f_bwd) / med / 1e12

    # The port on one (batch, head) slice, repeated within a budget.
    one = dict(c, B=1, Hq=1, Hkv=1)
    qs, ks, vs, dos = make_inputs(one, torch)
    qn, kn, vn, don = (t.float().numpy() for t in (qs, ks, vs, dos))
    p_fwd, p_bwd = flops(one)

    def run():
        o, lse = ora.attention_fwd(qn, kn, vn, c["causal"], dtype=np.float32)
        ora.attention_bwd(qn, kn, vn, don, c["causal"], o=o, lse=lse, dtype=np.float32)

    run()
    reps, t_tot = 0, 0.0
    while t_tot < port_budget_s and reps < 500:
        t0 = time.perf_counter()
        run()
        t_tot += time.perf_counter() - t0
        reps += 1
    return {
        "value": round(value, 4), "unit": "TFLOPS", "cores": threads, "kind": "port",
        "impl": "torch.nn.functional.scaled_dot_product_attention fwd+bwd, fp32, CPU",
        "cpu_model": cpu_model(),
        "ms_per_step": round(med * 1e3, 1),
        "sample": (f"the whole workload ({c['desc']}) in fp32 on the same inputs; 2 warmups, "
                   f"median of 5 ({', '.join(f'{t * 1e3:.0f}' for t in times)} ms); "
                   "FLOPs by the same convention"),
        "oracle_port_numpy_fp32": {
            "value": round((p_fwd + p_bwd) * reps / t_tot / 1e12, 4),
            "unit": "TFLOPS", "threads": "numpy's BLAS pool",
            "sample": f"1 of {c['B'] * c['Hq']} (batch, head) slices, x{reps} in {t_tot:.1f} s"},
    }


def read_traffic(workload):
    path = os.path.join(ROOT, "profiles", f"traffic_bwd_main_{workload}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_dispatch")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="C3", choices=sorted(CONFIGS) + ["C5"],
                    help="C5: the Qwen3-0.6B-shaped training step (hook vs sdpa) instead")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="first run one device copy of MIB MiB (counter calibration)")
    ap.add_argument("--no-features", action="store_true",
                    help="skip the optional-input timings (feature_paths)")
    ap.add_argument("--no-d64", action="store_true",
                    help="skip the D=64 leg beside the headline (C3) line")
    ap.add_argument("--c5-impl", default="both", choices=["both", "fa_p100", "sdpa"],
                    help="C5: run only the hook's step or only sdpa's (kernel traces)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures one GPU "
              "(the attention kernel at its single-GPU shape); run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    if args.config == "C5":
        import torch
        impls = ("fa_p100", "sdpa") if args.c5_impl == "both" else (args.c5_impl,)
        r = qwen3_bench(args.steps, args.warmup, impls)
        if args.c5_impl != "both":
            print(json.dumps({"c5_impl": args.c5_impl, **r[args.c5_impl]}), flush=True)
            return
        fa, sd = r["fa_p100"], r["sdpa"]
        print(json.dumps({
            "metric": "Qwen3-0.6B-shaped training step (fwd+bwd), attention through the HF hook",
            "value": fa["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": fa["ms_per_step"], "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
            "config": {"workload": "C5: random-init Qwen3-0.6B shape (28 layers, hidden 1024, "
                       "16/8 heads, D=128, SwiGLU 3072, vocab 151936), B=1, seq 8192, "
                       "fp16 autocast", **QWEN3_C5},
            "loss": fa["loss"], "sdpa": sd,
            "speedup_vs_sdpa": round(sd["ms_per_step"] / fa["ms_per_step"], 3),
            "device": torch.cuda.get_device_name(0)}), flush=True)
        return

    c = CONFIGS[args.config]
    f_fwd, f_bwd = flops(c)
    r = gpu_bench(c, args.steps, args.warmup, args.copy_calibration)
    step_ms = r["wall_ms"]
    value = (f_fwd + f_bwd) / (step_ms * 1e-3) / 1e12
    main_tf = f_bwd / (r["main_ms"] * 1e-3) / 1e12
    traffic = read_traffic(args.config)
    out = {
        "metric": "fwd+bwd attention TFLOPS & % fp16 MFMA peak, causal N=4096 D=64/128",
        "value": round(value, 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / P100_HEADLINE_TFLOPS, 1) if args.config == "C3" else None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": f"{args.config}: {c['desc']}", "B": c["B"], "Hq": c["Hq"],
                   "Hkv": c["Hkv"], "N": c["N"], "D": c["D"], "causal": c["causal"]},
        "pct_peak": round(100 * value / PEAK_FP16_TFLOPS, 2),
        "fwd_tflops": round(f_fwd / (r["fwd_ms"] * 1e-3) / 1e12, 2),
        "bwd_tflops": round(f_bwd / ((r["pre_ms"] + r["main_ms"]) * 1e-3) / 1e12, 2),
        "kernel_ms": {"fwd": round(r["fwd_ms"], 4), "bwd_preprocess": round(r["pre_ms"], 4),
                      "bwd_main": round(r["main_ms"], 4)},
        "api_ms_per_step": round(r["api_ms"], 4),
        "abi_interleaved_ms_per_step": round(r["abi_interleaved_ms"], 4),
        "torch_sdpa_gpu": r["sdpa"],
        "device": r["device"],
        "roofline": {"kernel": "bwd_main (fa_bwd_main)", "bound": "mfma",
                     "achieved": round(main_tf, 2), "peak": round(PEAK_FP16_TFLOPS, 1),
                     "unit": "TFLOP/s", "frac": round(main_tf / PEAK_FP16_TFLOPS, 4),
                     "traffic": traffic,
                     "time_source": "HIP events on the launch stream, second pass of K steps",
                     "kernel_ms": round(r["main_ms"], 4),
                     "algorithmic_gflop": round(f_bwd / 1e9, 3)},
    }
    if args.config == "C3" and not args.no_d64:
        d = CONFIGS["D64"]
        d_fwd, d_bwd = flops(d)
        rd = gpu_bench(d, args.steps, args.warmup, compare=False)
        d_val = (d_fwd + d_bwd) / (rd["wall_ms"] * 1e-3) / 1e12
        out["d64"] = {
            "workload": f"D64: {d['desc']}", "value": round(d_val, 2), "unit": "TFLOPS",
            "ms_per_step": round(rd["wall_ms"], 4),
            "pct_peak": round(100 * d_val / PEAK_FP16_TFLOPS, 2),
            "fwd_tflops": round(d_fwd / (rd["fwd_ms"] * 1e-3) / 1e12, 2),
            "bwd_tflops": round(d_bwd / ((rd["pre_ms"] + rd["main_ms"]) * 1e-3) / 1e12, 2),
            "kernel_ms": {"fwd": round(rd["fwd_ms"], 4), "bwd_preprocess": round(rd["pre_ms"], 4),
                          "bwd_main": round(rd["main_ms"], 4)},
            "p100_reference_ms": 29.596}
    if args.config == "C3" and not args.no_features:
        out["feature_paths"] = {"workload": "C3 shape through fa_fwd_ex + fa_bwd_ex (dq in fp16)",
                                **feature_paths(c, min(args.steps, 50), 20)}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(c)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
