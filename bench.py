#!/usr/bin/env python3
"""MLA latent-cache decode benchmark on one MI355X.

Workload: one MLA layer geometry (n_embd 1024, 16
heads, kv_lora_rank 256, rope 64, nope 128, v 128), bf16, batch 32, every
sequence pre-filled to 4096 cached tokens by the append path on N(0,1)
hidden states, then K decode steps through the drop-in
``swamla_amd.MLA.forward``, captured as one HIP graph per step: four HIP
launches (stacked input product, one-token append + decode attention, split
merge + W_uv read-out, wo).

One layer's cache (86.5 MB) fits MI355X's 256 MB Infinity Cache, so a single
layer decoded back to back would be served from there, not from HBM.  The
bench therefore rotates ``--layers`` independent layers (own weights, own
cache: 8 x 86.5 MB by default), like a decoder stack, and counts each token
once per layer it passes: value = batch * steps * layers / seconds
("layer-token decodes per second").

roofline: the step's attention launch (mla_decode_attn_append: the decode
kernel with the one-token append folded in, split-KV), timed with HIP events
on its stream around back-to-back launches rotating over the layers' caches
(each launch does its full work; the same launches replayed from a HIP graph
and the stand-alone split merge are timed too and reported beside it);
achieved = algorithmic bytes per launch /
average launch duration, with bytes = sum_b L_b*(R+P)*2 (latent + rope
cache) + B*H*(R+P)*2 (queries) + B*H*R*2 (latent outputs) + the append's
B*(R+P)*2 read and B*(R+P)*2 written (+ LayerNorm parameters).

Ceiling legs beside it (measurement kernels, not the product path):
roofline.ceiling_gbs is the plain HBM read rate of the GPU
(mla_probe_read over 1 GiB per launch, regions alternated so the Infinity
Cache serves nothing, best of four grid sizes), and roofline.stream_only_us the same decode launches'
cache stream with the arithmetic left out (mla_probe_cache_stream), timed the
same way as avg_launch_us.  step_account.empty_launch_us is the cost of one
kernel node that does nothing, graph-replayed back to back: the floor each of
the decode step's four launches pays before its work.

Every figure is the median of 5 timed repetitions.  ms_per_step is per
graph replay of the whole stack (ms_per_step x steps = the timed region);
us_per_layer_step divides it by the layers.

cpu_baseline: the oracle's op-for-op CPU restatement of the reference MLA
(oracle/mla_ref.py, which re-projects the cache and runs SDPA exactly as
models/mla.py does) on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
R, P, H = 256, 64, 16
TIMING_REPS = 5  # every figure is the median of this many timed repetitions


CONFIGS = {
    # BASELINE.json configs[1..4]; config 1 is the CPU-runnable fp32 case (a parity test)
    2: dict(batch=32, ctx=4096, dim=1024, steps=128, warmup=8, layers=8, cache="bf16", ragged=False),
    3: dict(batch=64, ctx=16384, dim=1024, steps=32, warmup=4, layers=2, cache="bf16", ragged=True),
    4: dict(batch=8, ctx=131072, dim=1536, steps=32, warmup=4, layers=1, cache="bf16", ragged=False),
    5: dict(batch=128, ctx=8192, dim=1024, steps=64, warmup=4, layers=6, cache="fp8", ragged=False),
}
WORKLOADS = {
    2: "BASELINE config 2: MLA decode, batch 32, prefill 4096 then append+attention steps",
    3: "BASELINE config 3: ragged batch of 64 sequences, cache lengths U[256, 16384] (seed 0), per-sequence start_pos",
    4: "BASELINE config 4: long-context split-KV, n_embd 1536, batch 8, cache length 131072",
    5: "BASELINE config 5: 6-layer decode stack, fp8-e4m3 latent cache, batch 128, cache length 8192",
}


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS),
                   help="BASELINE configuration (2 = the headline metric)")
    p.add_argument("--steps", type=int, default=None)
    p.add_argument("--warmup", type=int, default=None)
    p.add_argument("--layers", type=int, default=None, help="independent layers rotated per step")
    p.add_argument("--batch", type=int, default=None)
    p.add_argument("--ctx", type=int, default=None, help="prefilled context (the maximum for the ragged config)")
    p.add_argument("--dim", type=int, default=None)
    p.add_argument("--cache", choices=["bf16", "fp8"], default=None)
    p.add_argument("--heads", type=int, default=16, choices=[16, 32],
                   help="query heads (32: the xl preset's count, one attention launch of two head groups)")
    p.add_argument("--kernel-reps", type=int, default=50, help="roofline launches per layer")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    p.add_argument("--cpu-batch", type=int, default=4)
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run plain device copies of known size (calibrates FETCH_SIZE / WRITE_SIZE)")
    p.add_argument("--prefill", type=int, default=0, metavar="T",
                   help="only time the prompt pass: MLA.forward over T tokens per sequence at start_pos 0 "
                        "(its own JSON line; the profiling workload for the prefill-side products)")
    p.add_argument("--prefill-batch", type=int, default=4)
    p.add_argument("--rank-sweep", type=str, default="", metavar="R1,R2,...",
                   help="only time the drop-in decode step at config 2's shape (batch, ctx, dim, heads) for "
                        "each kv_lora_rank listed, graph-replayed over --layers layers (one JSON line per rank; "
                        "the profiling workload for ranks above 512)")
    args = p.parse_args()
    preset = CONFIGS[args.config]
    for k, v in preset.items():
        if getattr(args, k, None) is None:
            setattr(args, k, v)
    # The roofline launch is timed at the configuration's own end length
    # (config 2: ctx 4096 + 128 decode steps = 4224), whatever --steps is, so
    # its shape matches the committed traffic counters.
    args.canonical_steps = preset["steps"]
    if args.config != 2:
        args.no_cpu_baseline = True  # the CPU leg samples the headline workload only
    return args


def start_lengths(args, torch):
    """Per-sequence prefilled lengths: all ctx, or U[256, ctx] from seed 0."""
    if not args.ragged:
        return torch.full((args.batch,), args.ctx, dtype=torch.int32)
    g = torch.Generator().manual_seed(0)
    return torch.randint(256, args.ctx + 1, (args.batch,), generator=g, dtype=torch.int32)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# the decode kernel's translation unit (its traffic summary is keyed by these)
KERNEL_SOURCES = [os.path.join(ROOT, "swamla_amd", "csrc", f)
                  for f in ("mla_decode.hip", "mla_fused.h", "mla_kernels.hip", "mla_device.h", "mla_plan.h",
                            "mla_args.h", "numerics.h")]


def kernel_source_hash() -> str:
    import hashlib

    h = hashlib.sha256()
    for path in KERNEL_SOURCES:
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def measured_traffic(B: int, L: int, cache: str, heads: int = H):
    """HBM bytes per decode launch from a committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (profiles/*_traffic.md) taken on this kernel source at
    this launch shape, else None (counters cannot be read from inside this
    process).  Returns (bytes, summary file name)."""
    import glob

    try:
        src = kernel_source_hash()
    except OSError:
        return None, None
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*_traffic.md"))):
        fields = {}
        for line in open(path).read().splitlines():
            key, sep, val = line.partition(": ")
            if sep and key.isidentifier():
                fields[key] = val.strip()
        launch = f"B={B} L={L} cache={cache}" + (f" heads={heads}" if heads != H else "")
        if fields.get("kernel_source_sha256_16") == src and fields.get("launch") == launch:
            try:
                return int(fields["traffic_bytes_per_launch"]), os.path.relpath(path, ROOT)
            except (KeyError, ValueError):
                pass
    return None, None


def attention_bytes(B: int, L: int, fp8: bool, heads: int = H) -> int:
    per_tok = R * (1 if fp8 else 2) + P * 2 + (4 if fp8 else 0)
    return B * L * per_tok + B * heads * (R + P) * 2 + B * heads * R * 2


def attention_bytes_rows(lens, fp8: bool, heads: int = H) -> int:
    """Algorithmic bytes of one decode launch over rows of lengths ``lens``."""
    per_tok = R * (1 if fp8 else 2) + P * 2 + (4 if fp8 else 0)
    B = int(lens.numel())
    return int(lens.sum()) * per_tok + B * heads * (R + P) * 2 + B * heads * R * 2


def append_bytes(B: int, fp8: bool) -> int:
    """Algorithmic bytes of a one-token append of B rows: the wkv_a rows and
    LayerNorm parameters read, the cache tokens (and e4m3 scales) written."""
    return B * ((R + P) * 2 + R * (1 if fp8 else 2) + P * 2 + (4 if fp8 else 0)) + 2 * R * 2


def init_linear_weights(module, seed: int, torch) -> None:
    """N(0, 0.02) Linear weights in parameter order from a CPU generator and
    zero biases; LayerNorm stays at weight 1 / bias 0, as the reference model
    initialises it (models/swa_mla_model.py:314-320)."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in module.named_parameters():
            if name.startswith(("wq", "wkv_a", "wkv_b", "wo")) and name.endswith("weight"):
                p.copy_(torch.randn(p.shape, generator=g) * 0.02)
            elif name.endswith("bias") and not name.startswith(("kv_norm", "q_norm")):
                p.zero_()


def build_layers(args, dev, torch):
    from swamla_amd import MLA, MLAConfig

    max_seq = (args.ctx + max(args.steps + args.warmup, args.canonical_steps) + 63) // 64 * 64
    cfg = MLAConfig(n_embd=args.dim, n_head=args.heads, max_batch_size=args.batch, max_seq_len=max_seq)
    layers = []
    g = torch.Generator(device=dev).manual_seed(1234)
    for i in range(args.layers):
        m = MLA(cfg, cache_dtype="fp8_e4m3" if args.cache == "fp8" else None)
        init_linear_weights(m, 100 + i, torch)
        m.eval().to(torch.bfloat16).to(dev)
        m.set_inference_mode(True)
        # The start_pos tensor only lets the replayed graph advance the
        # position; a uniform batch gets the plan the reference's int
        # start_pos gets (each row cut by its own length).  The ragged batch
        # balances its rows' splits over the CUs on the device.
        m.split_plan = "auto" if args.ragged else "static"
        with torch.no_grad():
            x = torch.randn(args.batch, args.ctx, args.dim, generator=g, device=dev, dtype=torch.bfloat16)
            m.prefill_cache(x, 0)  # append path over the whole prompt (RoPE positions 0..ctx-1)
            del x
        layers.append(m)
    torch.cuda.synchronize()
    return layers


def run_rank_sweep(args, dev, torch) -> int:
    """The drop-in decode step at config 2's shape for each listed
    kv_lora_rank: every sequence prefilled to ctx through the append path,
    one step of MLA.forward over the layers captured as a HIP graph, K timed
    replays (median of the repetitions).  Ranks above 512 take the unfused
    step (ATen query projection, append, channel-split decode attention,
    merge, ATen W_uv and wo).  `attention_bytes` is the decode launch's
    algorithmic bytes at the mean timed length."""
    from swamla_amd import MLA, MLAConfig

    ranks = [int(x) for x in args.rank_sweep.split(",") if x]
    nl = min(args.layers, 4)
    for rank in ranks:
        cfg = MLAConfig(n_embd=args.dim, n_head=args.heads, kv_lora_rank=rank, max_batch_size=args.batch,
                        max_seq_len=(args.ctx + args.steps + args.warmup + 63) // 64 * 64)
        g = torch.Generator(device=dev).manual_seed(1234)
        layers = []
        for i in range(nl):
            m = MLA(cfg, cache_dtype="fp8_e4m3" if args.cache == "fp8" else None)
            init_linear_weights(m, 100 + i, torch)
            m.eval().to(torch.bfloat16).to(dev)
            m.set_inference_mode(True)
            m.split_plan = "static"
            with torch.no_grad():
                m.prefill_cache(torch.randn(args.batch, args.ctx, args.dim, generator=g, device=dev,
                                            dtype=torch.bfloat16), 0)
            layers.append(m)
        xs = [torch.randn(args.batch, 1, args.dim, generator=g, device=dev, dtype=torch.bfloat16) for _ in layers]
        sp0 = torch.full((args.batch,), args.ctx, dtype=torch.int32, device=dev)
        sp = sp0.clone()
        layers[-1].advance_positions = True
        outs = [None] * nl

        def stack_step():
            for i, m in enumerate(layers):
                outs[i] = m(xs[i], sp)

        with torch.no_grad():
            side = torch.cuda.Stream(dev)
            side.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(side):
                stack_step()
            torch.cuda.current_stream(dev).wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                stack_step()
            sp.copy_(sp0)
            for _ in range(args.warmup):
                graph.replay()
            reps = []
            for _ in range(TIMING_REPS):
                sp.copy_(sp0)
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for _ in range(args.steps):
                    graph.replay()
                torch.cuda.synchronize()
                reps.append(time.perf_counter() - t0)
        for m in layers:
            m.check_cache_errors()
        us = median(reps) / (args.steps * nl) * 1e6
        mid = args.ctx + (args.steps + 1) // 2
        rp = (rank + 63) // 64 * 64
        fp8 = args.cache == "fp8"
        abytes = (args.batch * mid * (rp * (1 if fp8 else 2) + P * 2 + (4 if fp8 else 0))
                  + args.batch * args.heads * (2 * rp + P) * 2)
        print(json.dumps({
            "metric": "MLA decode layer-step time at config 2's shape, by kv_lora_rank",
            "kv_lora_rank": rank, "us_per_layer_step": us, "value": args.batch / (us * 1e-6), "unit": "tok/s",
            "layers_rotated": nl, "steps": args.steps, "timed_reps": TIMING_REPS,
            "attention_bytes": abytes, "finite": all(bool(torch.isfinite(o).all()) for o in outs),
            "config": {"batch": args.batch, "ctx": args.ctx, "n_embd": args.dim, "heads": args.heads,
                       "cache": args.cache},
        }), flush=True)
        del layers, graph, outs
        torch.cuda.empty_cache()
    return 0


def time_decode_kernel(layers, xs, lens, args, dev, torch):
    """Average duration of one decode-attention launch from HIP events
    recorded on its stream around back-to-back launches that rotate over the
    layers' caches ("cold": the working set exceeds the MALL) or repeat on one
    layer ("warm": served from the MALL).  The cold launches are timed twice:
    replayed from a HIP graph, the launch mode of the decode step (the
    roofline figure), and issued one by one on the stream.  The merge kernel
    is timed on the stream."""
    from swamla_amd import _abi, kernels

    lib = _abi.lib()
    stream = torch.cuda.current_stream(dev)
    h = stream.cuda_stream
    preps = []
    with torch.no_grad():
        for m, x in zip(layers, xs):
            B = x.shape[0]
            NH = args.heads
            q = m.wq(x).view(B, NH, -1)
            w_uk, _ = m.absorbed_weights()
            q_abs = torch.bmm(q[:, :, :128].transpose(0, 1).contiguous(), w_uk)  # [H, B, R]
            kv = m.wkv_a(x).view(B, -1)  # the step's new tokens (wkv_a output rows)
            cache = m.latent_cache()
            L = int(lens.max())
            sp = (lens - 1).to(device=dev, dtype=torch.int32)  # row b attends [0, lens[b])
            # the plan MLA.forward uses for a start_pos tensor
            n_splits, min_chunk, balance = m._decode_plan(B, L, dev, True)
            ws = kernels.DecodeWorkspace.allocate(B, n_splits, dev, heads=NH)
            plan = _abi.ptr(ws.plan if balance else None)
            o_lat = torch.empty(NH, B, R, dtype=torch.bfloat16, device=dev)
            cos, sin = m.rope.half_tables()
            qa, qp, ol = q_abs.transpose(0, 1), q[:, :, 128:], o_lat.transpose(0, 1)
            # the step's attention launch: one-token append folded into decode
            dargs = (
                kv.data_ptr(), kv.stride(0), m.kv_norm.weight.data_ptr(), m.kv_norm.bias.data_ptr(),
                float(m.kv_norm.eps), None,
                qa.data_ptr(), qa.stride(0), qa.stride(1), qp.data_ptr(), qp.stride(0), qp.stride(1),
                cos.data_ptr(), sin.data_ptr(), cos.shape[0],
                cache.ckv.data_ptr(), cache.kpe.data_ptr(), _abi.ptr(cache.scale),
                cache.ckv.shape[0], cache.ckv.shape[1], sp.data_ptr(), 0,
                B, NH, R, P, float(m.softmax_scale), n_splits, min_chunk, balance, plan,
                ws.o_part.data_ptr(), ws.lse_part.data_ptr(),
                ol.data_ptr(), ol.stride(0), ol.stride(1), None, _abi.DTYPE_BF16, cache.cache_code, h,
            )
            margs = (ws.o_part.data_ptr(), ws.lse_part.data_ptr(), None, None, sp.data_ptr(), 1,
                     cache.ckv.shape[0], cache.ckv.shape[1], B, NH, R, n_splits, min_chunk, plan,
                     ol.data_ptr(), ol.stride(0), ol.stride(1), None, _abi.DTYPE_BF16, h)
            preps.append((dargs, (q, q_abs, kv, sp, ws, o_lat, cos, sin), L, B, n_splits, margs, balance))

    def run(indices, reps, which=0):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            for i in indices:
                if which == 0:
                    _abi.check(lib.mla_decode_attn_append(*preps[i][0]))
                else:
                    _abi.check(lib.mla_merge(*preps[i][5]))
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * len(indices))  # us

    def run_graph(launch_one, indices, reps):
        """Launches captured once in a HIP graph (as the decode step runs
        them) and replayed: no host launch work between them.  Median over
        TIMING_REPS timed repetitions of ``reps`` replays."""
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            hc = torch.cuda.current_stream(dev).cuda_stream
            for i in indices:
                launch_one(i, hc)
        graph.replay()
        torch.cuda.synchronize()
        times = []
        for _ in range(TIMING_REPS):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                graph.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) * 1e3 / (reps * len(indices)))  # us
        return median(times)

    def attn(i, hc):
        _abi.check(lib.mla_decode_attn_append(*(preps[i][0][:-1] + (hc,))))

    # the stream probe: the same launches' cache stream with no arithmetic
    sinks = [torch.empty(p[4] * p[3] * 256, dtype=torch.int32, device=dev) for p in preps]

    def probe(i, hc):
        cache = layers[i].latent_cache()
        dargs = preps[i][0]
        _abi.check(lib.mla_probe_cache_stream(
            cache.ckv.data_ptr(), cache.kpe.data_ptr(), _abi.ptr(cache.scale), cache.ckv.shape[0],
            cache.ckv.shape[1], preps[i][1][3].data_ptr(), preps[i][3], R, preps[i][4], dargs[28],
            cache.cache_code, sinks[i].data_ptr(), hc))

    run(range(len(preps)), 3)  # warm-up
    cold_us = median([run(range(len(preps)), args.kernel_reps) for _ in range(TIMING_REPS)])
    graph_us = run_graph(attn, range(len(preps)), args.kernel_reps)
    stream_us = None
    if max(p[6] for p in preps) == 0:  # the probe runs the static plan only
        stream_us = run_graph(probe, range(len(preps)), args.kernel_reps)
    warm_us = median([run([0], args.kernel_reps * len(preps)) for _ in range(TIMING_REPS)])
    merge_us = median([run(range(len(preps)), args.kernel_reps, which=1) for _ in range(TIMING_REPS)])
    L, B, n_splits = preps[0][2], preps[0][3], preps[0][4]
    return cold_us, graph_us, warm_us, merge_us, L, B, n_splits, preps[0][6], stream_us


def median(xs):
    xs = sorted(xs)
    n = len(xs)
    return xs[n // 2] if n % 2 else 0.5 * (xs[n // 2 - 1] + xs[n // 2])


CEILING_GRIDS = (256, 512, 1024, 2048)


def launch_floor(dev, torch, n: int = 64) -> float:
    """Cost of one kernel node with no work in a replayed HIP graph: n
    back-to-back mla_probe_read launches of 256 workgroups that read nothing
    (each thread stores one word), replayed from a graph and timed with HIP
    events; returns the median us per launch over TIMING_REPS repetitions.
    Every launch of the decode step pays at least this."""
    from swamla_amd import _abi

    lib = _abi.lib()
    sink = torch.empty(256 * 256, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        hc = torch.cuda.current_stream(dev).cuda_stream
        for _ in range(n):
            _abi.check(lib.mla_probe_read(sink.data_ptr(), 0, sink.data_ptr(), 256, hc))
    graph.replay()
    torch.cuda.synchronize()
    per = []
    for _ in range(TIMING_REPS):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(4):
            graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) * 1e3 / (4 * n))
    del graph
    return median(per)


def read_ceiling(dev, torch, gib: int = 1):
    """HBM read ceiling of this GPU: mla_probe_read streaming ``gib`` GiB per
    launch with 16-byte non-temporal loads, alternating between two disjoint
    regions (each far above the 256 MB Infinity Cache), replayed from a HIP
    graph, at each grid size of CEILING_GRIDS (256-thread workgroups).  How
    many bytes are in flight changes the rate on this GPU, so the ceiling is
    the best grid's median GB/s over TIMING_REPS repetitions; returns
    (ceiling, {grid: median GB/s})."""
    from swamla_amd import _abi

    lib = _abi.lib()
    nbytes = gib << 30
    buf = torch.empty(2 * nbytes, dtype=torch.uint8, device=dev)
    buf.view(torch.int32).random_(0, 1 << 30)
    sink = torch.empty(max(CEILING_GRIDS) * 256, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    by_grid = {}
    for grid in CEILING_GRIDS:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            hc = torch.cuda.current_stream(dev).cuda_stream
            for i in range(2):
                _abi.check(lib.mla_probe_read(buf.data_ptr() + i * nbytes, nbytes, sink.data_ptr(), grid, hc))
        graph.replay()
        torch.cuda.synchronize()
        rates = []
        reps = 2
        for _ in range(TIMING_REPS):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                graph.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            rates.append(2 * reps * nbytes / (e0.elapsed_time(e1) * 1e-3) / 1e9)
        by_grid[grid] = median(rates)
        del graph
    del buf
    return max(by_grid.values()), by_grid


def cpu_baseline(args, torch):
    """Op-for-op restatement of the reference on the host: a bounded sample
    of decode steps over a bf16 cache of length ctx."""
    from oracle.mla_ref import MLAConfig, RefMLA, enable_cache, init_weights

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    B = args.cpu_batch
    cfg = MLAConfig(n_embd=args.dim, max_batch_size=B, max_seq_len=args.ctx + 1024)
    m = RefMLA(cfg)
    init_weights(m, 7)
    m.eval()
    enable_cache(m)
    m.to(torch.bfloat16)
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        m.kv_cache[:, : args.ctx] = torch.randn(B, args.ctx, R, generator=g).to(torch.bfloat16)
        m.pe_cache[:, : args.ctx] = torch.randn(B, args.ctx, P, generator=g).to(torch.bfloat16)
        x = torch.randn(B, 1, args.dim, generator=g).to(torch.bfloat16)
        m(x, args.ctx)  # untimed warm-up step
        steps, t0 = 0, time.perf_counter()
        while True:
            m(x, args.ctx + 1 + steps)
            steps += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds or steps >= 1000:
                break
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": B * steps / el,
        "unit": "tok/s",
        "cores": threads,
        "kind": "port",
        "sample": (
            f"{B} sequences x {steps} decode steps at ctx {args.ctx + 1}-{args.ctx + steps}, bf16, "
            f"oracle/mla_ref.RefMLA (op-for-op restatement of models/mla.py absorb branch: cache "
            f"re-projection einsums + SDPA) on {el:.1f} s of CPU time; per-token cost is independent "
            f"of batch, so the rate stands for batch {args.batch}"
        ),
        "cpu": cpu_model,
        "nproc": os.cpu_count(),
        "capability": torch.backends.cpu.get_cpu_capability(),
    }


def run_prefill(args, dev, torch) -> int:
    """One layer's prompt pass: the drop-in MLA.forward over args.prefill
    tokens per sequence at start_pos 0, i.e. the input products and the
    query absorption (ATen GEMMs above 128 rows), the append of every token,
    causal attention over the latent cache (mla_prefill_attn), the W_uv
    read-out and wo; timed over a few forwards after one warm-up."""
    from swamla_amd import MLA, MLAConfig

    B, T, reps = args.prefill_batch, args.prefill, 5
    cfg = MLAConfig(n_embd=args.dim, max_batch_size=B, max_seq_len=(T + 63) // 64 * 64)
    m = MLA(cfg, cache_dtype="fp8_e4m3" if args.cache == "fp8" else None)
    init_linear_weights(m, 100, torch)
    m.eval().to(torch.bfloat16).to(dev)
    m.set_inference_mode(True)
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn(B, T, args.dim, generator=g, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        y = m(x, 0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            y = m(x, 0)
        torch.cuda.synchronize()
        el = time.perf_counter() - t0
    pairs = B * T * (T + 1) // 2  # causal (query, cached token) pairs
    attn_flop = pairs * H * (2 * (R + P) + 2 * R)
    attn_us = time_prefill_attention(m, B, T, dev, torch)
    print(json.dumps({
        "metric": "MLA prefill: prompt tokens/s through the drop-in MLA.forward at start_pos 0",
        "value": B * T * reps / el, "unit": "tok/s", "n_gpus": 1, "higher_is_better": True,
        "ms_per_forward": el / reps * 1e3, "dtype": "bf16" if args.cache == "bf16" else "bf16+e4m3-cache",
        "data": "synthetic: N(0,1) hidden states, N(0,0.02) random-init weights (no checkpoint)",
        "config": {"workload": f"prompt pass, batch {B}, {T} tokens per sequence", "batch": B, "tokens": T,
                   "n_embd": args.dim, "heads": H, "kv_lora_rank": R, "rope_dim": P, "cache": args.cache},
        "attention_flop_per_forward": attn_flop, "finite": bool(torch.isfinite(y).all()),
        "attention_kernel": {
            "kernel": "mla_prefill_attn (causal, eight query tokens per workgroup) on the forward's cache",
            "avg_launch_us": attn_us, "tflops": attn_flop / (attn_us * 1e-6) / 1e12,
            "peak_tflops": 2500.0, "frac": attn_flop / (attn_us * 1e-6) / 1e12 / 2500.0,
            "timing": "HIP events around back-to-back launches, median of 5 repetitions",
        },
    }), flush=True)
    return 0


def time_prefill_attention(m, B: int, T: int, dev, torch) -> float:
    """The prompt pass's attention launch alone (kernels.prefill_attention over
    the module's filled cache, N(0, 0.3) bf16 queries), HIP events around
    back-to-back launches on the current stream; median us per launch over
    TIMING_REPS repetitions."""
    from swamla_amd import kernels
    from swamla_amd.rope import rope_tables

    cache = m.latent_cache()
    g = torch.Generator(device=dev).manual_seed(11)
    q_abs = (0.3 * torch.randn(B * T, H, R, generator=g, device=dev)).to(torch.bfloat16)
    q_pe = (0.3 * torch.randn(B * T, H, P, generator=g, device=dev)).to(torch.bfloat16)
    cos, sin = rope_tables(P, cache.ckv.shape[1])
    cos = cos.to(torch.bfloat16)[0, 0, :, :P // 2].contiguous().to(dev)
    sin = sin.to(torch.bfloat16)[0, 0, :, :P // 2].contiguous().to(dev)
    sp = torch.zeros(B, dtype=torch.int32, device=dev)
    out = torch.empty(B * T, H, R, dtype=torch.bfloat16, device=dev)

    def launch():
        kernels.prefill_attention(q_abs, q_pe, cos, sin, cache, (128 + P) ** -0.5, start_pos=sp, rows_per_seq=T, out=out)

    launch()
    torch.cuda.synchronize()
    times = []
    reps = 5
    for _ in range(TIMING_REPS):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            launch()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) * 1e3 / reps)
    return median(times)


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(
            f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); the decode "
            "path shards by sequence with no exchange, so the one-GPU figure is per-GPU throughput",
            file=sys.stderr,
        )
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        # 256 MiB bf16 -> 256 MiB: each copy reads and writes exactly 268435456 B.
        src = torch.randn(128 << 20, device=dev, dtype=torch.float32).to(torch.bfloat16)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 2, "copy_bytes_written": dst.numel() * 2, "copies": 5}))
        return 0
    if args.prefill:
        return run_prefill(args, dev, torch)
    if args.rank_sweep:
        return run_rank_sweep(args, dev, torch)
    fp8 = args.cache == "fp8"
    log(f"building {args.layers} layers, batch {args.batch}, prefill {args.ctx} ({args.cache} cache)")
    layers = build_layers(args, dev, torch)
    g = torch.Generator(device=dev).manual_seed(99)
    xs = [torch.randn(args.batch, 1, args.dim, generator=g, device=dev, dtype=torch.bfloat16) for _ in layers]
    # one start-position tensor for the whole stack, advanced once per step
    # (every layer of a decoder sees the same positions): the last layer adds
    # 1 after its kernels have read them, inside its last launch
    lens0 = start_lengths(args, torch)
    sp0 = lens0.to(dev)
    sp = sp0.clone()
    outs = [None] * len(layers)
    layers[-1].advance_positions = True

    def stack_step():
        for i, m in enumerate(layers):
            outs[i] = m(xs[i], sp)

    # eager warm-up (allocates workspaces), then capture one stack step
    with torch.no_grad():
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            stack_step()
        torch.cuda.current_stream(dev).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            stack_step()
        sp.copy_(sp0)
        for _ in range(args.warmup):
            graph.replay()
        log("timing")
        dist = torch.distributed.is_available() and torch.distributed.is_initialized()
        elapsed_reps = []
        for _ in range(TIMING_REPS):
            sp.copy_(sp0)  # each repetition decodes positions start .. start+K-1
            if dist:
                torch.distributed.barrier()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(args.steps):
                graph.replay()
            torch.cuda.synchronize()
            elapsed_reps.append(time.perf_counter() - t0)
            if dist:
                torch.distributed.barrier()
        elapsed = median(elapsed_reps)
        ok = all(bool(torch.isfinite(o).all()) for o in outs)

    layer_steps = args.steps * len(layers)
    value = args.batch * layer_steps / elapsed
    ms_per_step = elapsed / args.steps * 1e3  # one stack step: every layer once
    us_per_layer_step = elapsed / layer_steps * 1e6
    log(f"decode: {value:.0f} layer-token/s, {us_per_layer_step:.2f} us per layer-step, finite={ok}")

    lens = lens0 + args.canonical_steps  # the configuration's end lengths (config 2: 4224)
    cold_us, graph_us, warm_us, merge_us, L, B, n_splits, balance, stream_us = time_decode_kernel(
        layers, xs, lens, args, dev, torch)
    ceiling, ceiling_by_grid = read_ceiling(dev, torch)
    floor_us = launch_floor(dev, torch)
    log(f"empty graph-node launch {floor_us:.2f} us")
    log(f"read ceiling {ceiling:.0f} GB/s; cache stream alone "
        + (f"{stream_us:.2f} us" if stream_us is not None else "n/a (balanced plan)"))
    abytes = attention_bytes_rows(lens, fp8, args.heads) + append_bytes(B, fp8)
    stream_bytes = int(lens.sum()) * (R * (1 if fp8 else 2) + P * 2 + (4 if fp8 else 0))
    traffic, traffic_src = measured_traffic(B, L, args.cache, args.heads) if not args.ragged else (None, None)
    achieved = abytes / (graph_us * 1e-6) / 1e9
    warm = abytes / (warm_us * 1e-6) / 1e9
    log(f"decode kernel: {graph_us:.2f} us cold, graph-replayed ({achieved:.0f} GB/s), {cold_us:.2f} us cold on the "
        f"stream, {warm_us:.2f} us warm ({warm:.0f} GB/s); merge {merge_us:.2f} us")
    # algorithmic bytes of one full layer-step (attention + append + weights), mean context
    w_bytes = sum(p.numel() * p.element_size() for p in layers[0].parameters())
    mid = lens0 + (args.steps + 1) // 2
    step_bytes = attention_bytes_rows(mid, fp8, args.heads) + w_bytes + append_bytes(args.batch, fp8)

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        cpu = cpu_baseline(args, torch)
        log(f"cpu: {cpu['value']:.2f} tok/s on {cpu['cores']} threads")

    line = {
        "metric": ("MLA decode tok/s + achieved HBM GB/s (% peak), bs=32 ctx=4096 bf16"
                   if args.config == 2 and args.heads == H
                   else f"MLA decode tok/s + achieved HBM GB/s (% peak), config {args.config}"
                        + (f", {args.heads} heads" if args.heads != H else "")),
        "value": value,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "us_per_layer_step": us_per_layer_step,
        "timed_reps": TIMING_REPS,
        "elapsed_s_reps": elapsed_reps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if not fp8 else "bf16+e4m3-cache",
        "data": "synthetic: N(0,1) hidden states, N(0,0.02) random-init weights (no checkpoint)",
        "config": {
            "workload": WORKLOADS[args.config],
            "batch": args.batch, "ctx": args.ctx, "decode_steps": args.steps, "n_embd": args.dim,
            "heads": args.heads, "kv_lora_rank": R, "rope_dim": P, "cache": args.cache,
            "layers_rotated": len(layers),
            "value_counts": "tokens x layers per second (each token counted once per MLA layer)",
            "step_unit": (f"one step = one graph replay of the {len(layers)}-layer stack (ms_per_step x steps = "
                          f"the timed region; us_per_layer_step = ms_per_step / {len(layers)}); figures are "
                          f"medians of {TIMING_REPS} timed repetitions of the K steps"),
            "step": "full drop-in MLA.forward as one HIP graph per layer-step: stacked input product "
                    "(wq with W_uk absorbed, wkv_a), append + decode attention, split merge + W_uv, wo "
                    "(four launches)",
        },
        # one layer's algorithmic bytes over one layer-step's time
        "hbm_gbs_step": step_bytes / (us_per_layer_step * 1e-6) / 1e9,
        "roofline": {
            "kernel": "mla_decode_dma, fused-append instance (mla_decode_attn_append: one-token append + "
                      "split-KV decode attention)",
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "traffic_source": (f"rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated: {traffic_src}" if traffic
                               else "no committed PMC summary for this kernel source and launch shape"),
            "bytes_per_launch": abytes,
            "avg_launch_us": graph_us,
            "timing": ("HIP events on the launch stream around back-to-back launches, one per layer in turn "
                       "(caches rotated), replayed from a HIP graph as the decode step runs them; "
                       "avg_launch_us_stream: the same launches issued one by one on the stream"),
            "avg_launch_us_stream": cold_us,
            "launch": (f"B={B} L={L} splits<={n_splits}, caches rotated over {len(layers)} layers" if not args.ragged
                       else f"B={B} ragged L in [{int(lens.min())}, {L}] (sum {int(lens.sum())}), "
                            + (f"splits balanced over {balance} workgroups (per-row cap {n_splits})" if balance
                               else f"splits<={n_splits}")
                            + f", caches rotated over {len(layers)} layers"),
            "ceiling_gbs": ceiling,
            "ceiling_source": ("mla_probe_read: 1 GiB per launch with 16-byte non-temporal loads, alternating "
                               "over two disjoint 1 GiB regions, graph-replayed, best of the grid sizes in "
                               "ceiling_by_grid (the plain HBM read rate of this GPU)"),
            "ceiling_by_grid": {str(g): r for g, r in ceiling_by_grid.items()},
            "frac_of_ceiling": achieved / ceiling,
            "stream_only_us": stream_us,
            "stream_only_gbs": (stream_bytes / (stream_us * 1e-6) / 1e9) if stream_us else None,
            "stream_only_source": ("mla_probe_cache_stream: this launch's cache stream alone (same grid, split "
                                   "plan, LDS ring, DMA instructions and waits; no query, arithmetic or epilogue), "
                                   f"{stream_bytes} cache bytes, timed as avg_launch_us"),
            "above_stream_only_us": (graph_us - stream_us) if stream_us else None,
            "warm_mall_achieved": warm,
            "warm_mall_avg_launch_us": warm_us,
            "merge_avg_launch_us": merge_us,
            "attention_achieved_with_merge": abytes / ((graph_us + merge_us) * 1e-6) / 1e9,
        },
        "step_account": {
            "launches_per_layer_step": 4,
            "empty_launch_us": floor_us,
            "launch_floor_us": 4 * floor_us,
            "source": ("launch_floor: 64 back-to-back kernel nodes of 256 workgroups that read nothing "
                       "(mla_probe_read, 0 bytes), graph-replayed, HIP events; the decode step's four launches "
                       "(input product, append + attention, merge + W_uv, wo) each pay at least empty_launch_us "
                       "before any of their work"),
        },
        "cpu_baseline": cpu,
        "host": platform.node(),
        "gpu": torch.cuda.get_device_name(dev),
    }
    print(json.dumps(line), flush=True)
    return 0 if ok else 3


if __name__ == "__main__":
    sys.exit(main())
