"""Benchmark of the MI355X attention hot path on one GPU.

Headline (`value`): config 1 -- Gated DeltaNet chunked prefill, one layer,
batch 1, T = 4096, chunk 64 -- in tokens/s, inputs resident in HBM. The same
JSON line carries every other configuration under "configs", each with its
own roofline block; the top-level `roofline` is the headline's dominant
kernel (timed live with HIP events on the launch stream through
qff_profile_*) on its share of the workload's canonical flops, MFMA-bound as
the workload defines it. `cpu_baseline`: the reference's CPU algorithms
(oracle/cpu_baseline.c, built for this host with gcc -O3 -march=native) on a
bounded sample, one thread and all cores.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu] [--only c0,c1,...]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen-fieldfare_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA

# Canonical work per unit of each workload (algorithmic bytes and flops)
C0_BYTES = 4_424_448           # DeltaNet decode, one layer-step at B=1
C0_FLOPS = 3_670_016
C1_FLOPS = 23_622_320_128      # DeltaNet chunked prefill T=4096
C1_BYTES = 137_428_992
# Config 1 per kernel, per launch (64 chunks x 32 heads, C = 64, d = 128),
# the canonical terms split by the kernel that computes them: the state pass
# forms K S^T, the state update K^T U and Q S^T (3 * 2Cd^2 per chunk and
# head) and T Y, P U (2 * 2C^2 d); the chunk-local pass the Gram products
# K K^T, Q K^T and T = (I + A)^-1, credited with the remaining 3 * 2C^2 d of
# the canonical count; the two sum to C1_FLOPS (the norm pass does no matrix
# work).
C1_KERNEL_FLOPS = {
    "dn_chunk_local": 2048 * 3 * 2 * 64 * 64 * 128,
    "dn_chunk_state": 2048 * (3 * 2 * 64 * 128 * 128 + 2 * 2 * 64 * 64 * 128),
}
assert sum(C1_KERNEL_FLOPS.values()) == 23_622_320_128
C3_ATTN_FLOPS = 549_822_922_752   # GQA causal prefill T=8192: 32 D T (T + 1)
C3_PROJ_FLOPS = 309_237_645_312   # 2 T 2048 (8192 + 512 + 512)
COPY_PROBE_BYTES = 256 << 20   # --copy-probe: one D2D copy of this size (counter calibration)


def hbm_roof(nbytes, ms, basis):
    """HBM roofline block: algorithmic bytes over a measured time."""
    gbps = nbytes / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": gbps, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbps / HBM_PEAK_GBS,
            "bytes": nbytes, "ms": ms, "basis": basis}


def mfma_roof(flops, ms, basis):
    """bf16 MFMA roofline block: algorithmic flops over a measured time."""
    tf = flops / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": tf, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": tf / BF16_PEAK_TFLOPS, "flops": flops, "ms": ms, "basis": basis}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _ctypes_profile(ctx, enable):
    from qff._lib import check, lib
    check("qff_profile_enable", lib().qff_profile_enable(ctx.handle, int(enable)))


def _profile_read(ctx):
    import ctypes
    from qff._lib import check, lib
    cap = 4096
    names = (ctypes.c_char_p * cap)()
    ms = (ctypes.c_float * cap)()
    n = ctypes.c_int()
    check("qff_profile_read", lib().qff_profile_read(ctx.handle, names, ms, cap, ctypes.byref(n)))
    out = {}
    for i in range(n.value):
        out.setdefault(names[i].decode(), []).append(ms[i])
    return out


def timed(fn, steps, warmup, stream):
    import torch
    for _ in range(warmup):
        fn(0)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        fn(i)
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def timed_graph(fn, unroll, steps, warmup):
    """Per-step time of `unroll` consecutive steps (fn(0) .. fn(unroll - 1),
    each on its own rotating input set) captured in one HIP graph and
    replayed: the GPU time of back-to-back steps, as a serving loop that
    replays graphs sees it, without Python's per-call launch cost."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(unroll):
            fn(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(unroll):
            fn(i)
    reps = max(3, steps // unroll)
    ms = timed(lambda i: graph.replay(), reps, max(1, warmup // unroll), torch.cuda.current_stream())
    return ms / unroll


def kernel_times(ctx, fn, steps):
    """Per-kernel average durations (ms) over `steps` calls, from the
    library's own hipEvent brackets on the launch stream."""
    import torch
    torch.cuda.synchronize()
    _ctypes_profile(ctx, True)
    for i in range(steps):
        fn(i)
    torch.cuda.synchronize()
    rec = _profile_read(ctx)
    _ctypes_profile(ctx, False)
    return {k: sum(v) / len(v) for k, v in rec.items()}, {k: len(v) for k, v in rec.items()}


def bf16_randn(shape, gen, std=1.0):
    import torch
    return (torch.randn(shape, generator=gen, device="cuda") * std).to(torch.bfloat16)


# ------------------------------------------------------------------ configs
def bench_c1(ctx, steps, warmup, sets=6):
    """Config 1: DeltaNet prefill T=4096 from zero state. Steps rotate over
    `sets` distinct input sets (qkv, z, a, b: 101 MB each, 606 MB in all,
    over twice the 256 MB MALL), so each step's inputs come from HBM; a
    step zeroes its set's conv and recurrent state (the workload starts
    from zero state) and runs the prefill. Timed as back-to-back steps
    replayed from one HIP graph (`ms_per_step`), and one Python call per
    step (`ms_per_step_eager`)."""
    import torch
    import qff
    from qff import synth
    T = 4096
    g = torch.Generator(device="cuda").manual_seed(1)
    p = {k: torch.from_numpy(v).cuda() for k, v in synth.deltanet_params().items()}
    qkv = bf16_randn((sets, T, 8192), g)
    z = bf16_randn((sets, T, 4096), g)
    a = torch.randn(sets, T, 32, generator=g, device="cuda")
    b = torch.randn(sets, T, 32, generator=g, device="cuda")
    conv = torch.zeros(sets, 8192, 4, device="cuda")
    ssm = torch.zeros(sets, 32, 128, 128, device="cuda")
    out = torch.empty(sets, T, 4096, dtype=torch.bfloat16, device="cuda")

    def step(i):
        j = i % sets
        # every step starts from zero state, as the workload defines
        conv[j].zero_()
        ssm[j].zero_()
        qff.deltanet_prefill(ctx, p, qkv[j], z[j], a[j], b[j], conv[j], ssm[j], out=out[j])

    stream = torch.cuda.current_stream()
    ms_eager = timed(step, steps, warmup, stream)
    ms = timed_graph(step, sets, steps, warmup)
    kt, _ = kernel_times(ctx, step, max(3, min(steps, 12)))
    return {"ms_per_step": ms, "ms_per_step_eager": ms_eager, "tokens_per_s": T / (ms * 1e-3),
            "input_sets": sets, "kernels_ms": kt,
            "roofline": mfma_roof(C1_FLOPS, ms, "whole step, canonical flops"),
            "roofline_hbm": hbm_roof(C1_BYTES, ms, "whole step, canonical bytes")}


def bench_c0(ctx, steps, warmup, sets=128):
    """Config 0: DeltaNet decode B=1, one layer-step, rotating over `sets`
    distinct state/input sets so the 4.4 MB working set comes from HBM."""
    import torch
    import qff
    from qff import synth
    g = torch.Generator(device="cuda").manual_seed(0)
    p = {k: torch.from_numpy(v).cuda() for k, v in synth.deltanet_params().items()}
    qkv = bf16_randn((sets, 1, 8192), g)
    z = bf16_randn((sets, 1, 4096), g)
    a = torch.randn(sets, 1, 32, generator=g, device="cuda")
    b = torch.randn(sets, 1, 32, generator=g, device="cuda")
    conv = torch.randn(sets, 1, 8192, 4, generator=g, device="cuda")
    ssm = torch.randn(sets, 1, 32, 128, 128, generator=g, device="cuda") * 0.02
    out = torch.empty(sets, 1, 4096, dtype=torch.bfloat16, device="cuda")

    def step(i):
        j = i % sets
        qff.deltanet_decode(ctx, p, qkv[j], z[j], a[j], b[j], conv[j], ssm[j], out=out[j])

    stream = torch.cuda.current_stream()
    ms_eager = timed(step, steps, warmup, stream)
    ms = timed_graph(step, sets, steps, warmup)
    kt, _ = kernel_times(ctx, step, min(steps, 256))
    return {"ms_per_step": ms, "ms_per_step_eager": ms_eager, "tokens_per_s": 1.0 / (ms * 1e-3),
            "kernels_us_event": {k_: v * 1e3 for k_, v in kt.items()},
            "roofline": hbm_roof(C0_BYTES, ms, "graph-replayed step (kernels + launch gaps)")}


def bench_dn_decode_batch(ctx, B, steps, warmup):
    """DeltaNet decode at batch B (the config-4 decode shape), one layer."""
    import torch
    import qff
    from qff import synth
    sets = max(1, 256 // B)
    g = torch.Generator(device="cuda").manual_seed(B)
    p = {k: torch.from_numpy(v).cuda() for k, v in synth.deltanet_params().items()}
    qkv = bf16_randn((sets, B, 8192), g)
    z = bf16_randn((sets, B, 4096), g)
    a = torch.randn(sets, B, 32, generator=g, device="cuda")
    b = torch.randn(sets, B, 32, generator=g, device="cuda")
    conv = torch.randn(sets, B, 8192, 4, generator=g, device="cuda")
    ssm = torch.randn(sets, B, 32, 128, 128, generator=g, device="cuda") * 0.02
    out = torch.empty(sets, B, 4096, dtype=torch.bfloat16, device="cuda")

    def step(i):
        j = i % sets
        qff.deltanet_decode(ctx, p, qkv[j], z[j], a[j], b[j], conv[j], ssm[j], out=out[j])

    ms_eager = timed(step, steps, warmup, torch.cuda.current_stream())
    ms = timed_graph(step, sets, steps, warmup)
    kt, _ = kernel_times(ctx, step, min(steps, 64))
    return {"ms_per_step": ms, "ms_per_step_eager": ms_eager, "tokens_per_s": B / (ms * 1e-3),
            "kernels_us_event": {k_: v * 1e3 for k_, v in kt.items()},
            "roofline": hbm_roof(B * C0_BYTES, ms, "graph-replayed step (kernels + launch gaps)")}


def bench_c2(ctx, B, steps, warmup, max_ctx=8192):
    """Config 2: GQA decode at batch B, context 8192, random lengths."""
    import numpy as np
    import torch
    import qff
    from qff import synth
    pools = max(2, 64 // B)
    rng = np.random.default_rng(1000 + B)
    lengths = rng.integers(1, max_ctx + 1, B)
    g = torch.Generator(device="cuda").manual_seed(B)
    p = {k: torch.from_numpy(v).cuda() for k, v in synth.gqa_params().items()}
    kc = [bf16_randn((B, max_ctx, 2, 256), g) for _ in range(pools)]
    vc = [bf16_randn((B, max_ctx, 2, 256), g) for _ in range(pools)]
    qg = bf16_randn((B, 16, 512), g)
    kn = bf16_randn((B, 2, 256), g)
    vn = bf16_randn((B, 2, 256), g)
    pos = torch.from_numpy((lengths - 1).astype(np.int32)).cuda()
    out = torch.empty(B, 16, 256, dtype=torch.bfloat16, device="cuda")

    def step(i):
        j = i % pools
        qff.gqa_decode(ctx, p, qg, kn, vn, kc[j], vc[j], pos, out=out)

    ms_eager = timed(step, steps, warmup, torch.cuda.current_stream())
    ms = timed_graph(step, pools, steps, warmup)
    kt, _ = kernel_times(ctx, step, min(steps, 64))
    nbytes = int(np.sum(2048 * lengths.astype(np.int64) + 29_696))
    flops = int(np.sum(16_384 * lengths.astype(np.int64)))
    return {"ms_per_step": ms, "ms_per_step_eager": ms_eager, "tokens_per_s": B / (ms * 1e-3),
            "mean_len": float(lengths.mean()),
            "kernels_us_event": {k: v * 1e3 for k, v in kt.items()},
            "roofline": hbm_roof(nbytes, ms, "graph-replayed step (kernels + launch gaps)"),
            "TFLOPs": flops / (ms * 1e-3) / 1e12}


def bench_c3(ctx, steps, warmup):
    """Config 3: GQA causal prefill, T = 8192, with the q|gate, k and v
    affine-Q4 projections from hidden 2048 (three Q4 GEMMs, then attention)."""
    import numpy as np
    import torch
    import qff
    from qff import synth
    T, H = 8192, 2048
    g = torch.Generator(device="cuda").manual_seed(3)
    p = {k: torch.from_numpy(v).cuda() for k, v in synth.gqa_params().items()}
    X = bf16_randn((T, H), g)
    wts = []
    for i, rows in enumerate((8192, 512, 512)):
        w, sc, bi = synth.q4_weight(rows, H, seed=300 + i)
        wts.append((torch.from_numpy(w.view(np.int32)).cuda(),
                    torch.from_numpy(sc.view(np.int16)).view(torch.float16).cuda(),
                    torch.from_numpy(bi.view(np.int16)).view(torch.float16).cuda()))
    qg = torch.empty(T, 8192, dtype=torch.bfloat16, device="cuda")
    k = torch.empty(T, 512, dtype=torch.bfloat16, device="cuda")
    v = torch.empty(T, 512, dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros(T, 2, 256, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros(T, 2, 256, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(T, 16, 256, dtype=torch.bfloat16, device="cuda")

    def step(i):
        # q|gate, k and v share X: one multi-part product (one x16 pass, one
        # tiled launch over the three parts' row tiles)
        qff.q4_matmul_parts(ctx, wts, X, outs=(qg, k, v))
        qff.gqa_prefill(ctx, p, qg.view(T, 16, 512), k.view(T, 2, 256), v.view(T, 2, 256), kc, vc, 0, out=out)

    # the step captured once in a HIP graph and replayed back-to-back, as the
    # DeltaNet prefill and the 40-layer stack are timed (a prefill server
    # replays captured steps); the eager one-call-per-launch time rides beside
    ms_eager = timed(step, steps, warmup, torch.cuda.current_stream())
    ms = timed_graph(step, 1, steps, warmup)
    kt, cnt = kernel_times(ctx, step, max(2, min(steps, 5)))
    # one x16 pass and one GEMM launch per step
    proj_ms = sum(v for k_, v in kt.items() if k_.startswith("q4_"))
    attn_ms = sum(v for k_, v in kt.items() if k_.startswith("gqa_prefill"))
    return {"ms_per_step": ms, "ms_per_step_eager": ms_eager, "tokens_per_s": T / (ms * 1e-3), "kernels_ms": kt,
            "roofline": mfma_roof(C3_ATTN_FLOPS + C3_PROJ_FLOPS, ms, "whole step, canonical flops"),
            "roofline_attention": mfma_roof(C3_ATTN_FLOPS, attn_ms, "attention kernels (event-timed)"),
            "roofline_projections": mfma_roof(C3_PROJ_FLOPS, proj_ms, "Q4 projection kernels (event-timed)")}


C4_BYTES = {(16, 32768): 13_535_395_840, (1, 65536): 2_193_735_680}


def bench_c4(B, L, steps, warmup):
    """Config 4: attention-only stack of the 40-layer pattern (3 Gated DeltaNet
    + 1 GQA) x 10, hidden 2048, every projection affine-Q4 group 64, MoE
    replaced by identity: one decode step of B sequences at context L,
    through qff.stack.AttentionStack (the per-layer schedule the parity tests
    check layer by layer): fp32 residual stream and intermediates, input
    RMSNorm fused into the in-projections, the out-projections adding into
    the stream in place. The step is captured once in a HIP graph and
    replayed (the serving loop's shape), so the timing is GPU time, not
    Python launch time."""
    import torch
    import qff
    from qff import stack as S
    from qff import synth
    g = torch.Generator(device="cuda").manual_seed(40 + B)
    ctx = qff.Context(max_batch=B, max_ctx=L, max_prefill_tokens=64)
    dnp = {k: torch.from_numpy(v).cuda() for k, v in synth.deltanet_params().items()}
    gqp = {k: torch.from_numpy(v).cuda() for k, v in synth.gqa_params().items()}
    st = S.AttentionStack(ctx, S.random_layers(40, g, dnp, gqp), B, L)
    for kind, s_ in zip(st.kinds, st.states):
        if kind == "dn":
            s_["conv_state"].normal_(generator=g)
            s_["ssm_state"].normal_(generator=g).mul_(0.02)
        else:
            for key in ("k_cache", "v_cache"):
                s_[key].copy_(torch.randn(s_[key].shape, device="cuda", generator=g).to(torch.bfloat16))
    x = torch.randn(B, 2048, generator=g, device="cuda")   # the residual stream (fp32)
    pos = torch.full((B,), L - 1, dtype=torch.int32, device="cuda")

    def step(i):
        st.decode_step(x, pos)

    kt, cnt = kernel_times(ctx, step, 2)
    per_step_kernel_ms = {k: v * cnt[k] / 2 for k, v in kt.items()}
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step(0)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(0)
    ms = timed(lambda i: graph.replay(), steps, warmup, torch.cuda.current_stream())
    nbytes = C4_BYTES.get((B, L))
    del graph
    ctx.close()
    return {"ms_per_step": ms, "tokens_per_s": B / (ms * 1e-3), "batch": B, "context": L,
            "kernel_ms_per_step_event": per_step_kernel_ms,
            "roofline": hbm_roof(nbytes, ms, "graph-replayed 40-layer step") if nbytes else None}


def bench_router(ctx, B, steps, warmup, sets=64):
    """MoE router of B tokens (the reference's decode step: 256 experts,
    hidden 2048, Q8 weights): logits and top-8. Rotates over weight sets so
    the 0.56 MB of weights come from HBM."""
    import numpy as np
    import torch
    import qff
    from qff import synth
    ws = []
    for i in range(sets):
        w, sc, bi = synth.q8_weight(256, 2048, seed=500 + i) if i < 2 else (ws[i % 2][3], None, None)
        if i < 2:
            ws.append((torch.from_numpy(w.view(np.int32)).cuda(),
                       torch.from_numpy(sc.view(np.int16)).view(torch.bfloat16).cuda(),
                       torch.from_numpy(bi.view(np.int16)).view(torch.bfloat16).cuda(), w))
        else:
            src = ws[i % 2]
            ws.append((src[0].clone(), src[1].clone(), src[2].clone(), src[3]))
    g = torch.Generator(device="cuda").manual_seed(B)
    x = torch.randn(B, 2048, generator=g, device="cuda")
    lg = torch.empty(B, 256, device="cuda")
    idx = torch.empty(B, 8, dtype=torch.int32, device="cuda")
    scr = torch.empty(B, 8, device="cuda")

    def step(i):
        w, sc, bi, _ = ws[i % sets]
        qff.router_top8(ctx, w, sc, bi, x, logits=lg, indices=idx, scores=scr)

    ms_eager = timed(step, steps, warmup, torch.cuda.current_stream())
    ms = timed_graph(step, sets, steps, warmup)
    kt, _ = kernel_times(ctx, step, min(steps, 64))
    nbytes = 256 * 2048 + 2 * 256 * 32 * 2 + B * 2048 * 4
    return {"ms_per_step": ms, "ms_per_step_eager": ms_eager, "tokens_per_s": B / (ms * 1e-3),
            "kernels_us_event": {k_: v * 1e3 for k_, v in kt.items()},
            "roofline": hbm_roof(nbytes, ms, "graph-replayed step (kernels + launch gaps)")}


def _median_time(fn, reps=10, warm=3):
    import statistics
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _host_info():
    import platform
    model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"host_cores": len(os.sched_getaffinity(0)), "nproc": os.cpu_count(), "cpu_model": model}


def _filled(shape, rng):
    """fp32 array of `shape` filled with a repeated random block (timing data:
    the baselines have no data-dependent control flow, and drawing GBs of
    normals would cost more than the timed work)."""
    import numpy as np
    a = np.empty(shape, np.float32)
    flat = a.reshape(-1)
    blk = rng.standard_normal(1 << 16).astype(np.float32)
    for o in range(0, flat.size, blk.size):
        n = min(blk.size, flat.size - o)
        flat[o:o + n] = blk[:n]
    return a


def cpu_baselines():
    """The reference's CPU algorithms (oracle/cpu_baseline.c: the oracle's
    fp32 functions in the reference's loop order with OpenMP drivers, equal
    to the oracle bit for bit, tests/test_oracle_deltanet.py and
    tests/test_oracle_cpu_baseline.py), compiled here with gcc -O3
    -march=native, one thread and all cores, 3 warm-ups then the median of
    10 runs (3 for the multi-second samples). Per configuration:
      c0  one DeltaNet decode step (the config-0 inputs);
      c1  the 4096-token sequence (all cores) and its first 1024 tokens (one
          thread), token by token;
      c2  split-KV decode attention at batch 1, 8 and 32, context 8192 with
          random lengths (attention.metal:134-224, 342-377);
      c3  the reference's token-by-token prefill of the full-attention layer
          (Q4 projections, norms, RoPE, attention over 0..t, gate) on tokens
          4064-4095 of the 8192-token sequence, whose cost is the sequence's
          average per token (attention grows linearly with the position);
      c4  one DeltaNet layer and one full-attention layer of the stack
          (input norm, Q4 in-projection, core, Q4 out-projection +
          residual) at the step's batch and context, composed as 30 + 10
          layers.
    Returns {config key: baseline}."""
    import numpy as np
    from oracle import cpu_baseline as CB
    from oracle import oracle as O
    from qff import synth
    import tempfile
    path = CB.build_native(os.path.join(tempfile.gettempdir(), "qff_cpu_baseline"))
    L = CB.load(path)
    build = "gcc -O3 -march=native -fopenmp -ffp-contract=off" if path else "portable build (-march=x86-64-v2)"
    info = _host_info()
    threads = min(info["host_cores"], int(os.environ.get("OMP_NUM_THREADS", info["host_cores"]) or 1))
    med = "median of 10 after 3 warm-ups"
    out = {}
    p = synth.deltanet_params()

    # config 1 and config 0
    inp = synth.deltanet_prefill_inputs(4096)
    qkv, z = O.bf16_to_f32(inp["qkv"]), O.bf16_to_f32(inp["z"])

    def dn(T, th):
        return lambda: CB.deltanet_prefill(L, qkv[:T], z[:T], inp["a"][:T], inp["b"][:T], p, inp["conv_state"],
                                           inp["ssm_state"], threads=th)
    t1 = _median_time(dn(1024, 1))
    tn = _median_time(dn(4096, threads))
    c1 = {"value": 4096 / tn, "unit": "tokens/s", "cores": threads, "kind": "port",
          "sample": f"config 1, the 4096-token sequence from zero state through the DeltaNet layer core "
                    f"(oracle/cpu_baseline.c, {build}), {threads} threads; {med}",
          "single_thread": {"value": 1024 / t1, "unit": "tokens/s", "cores": 1,
                            "sample": "the first 1024 tokens of the same sequence, 1 thread"}}
    c1.update(info)
    out["c1_deltanet_prefill_t4096"] = c1
    d0 = synth.deltanet_decode_inputs(1)
    q0, z0 = O.bf16_to_f32(d0["qkv"]), O.bf16_to_f32(d0["z"])

    def dn0(th):
        return lambda: CB.deltanet_prefill(L, q0, z0, d0["a"], d0["b"], p, d0["conv_state"][0], d0["ssm_state"][0],
                                           threads=th)
    out["c0_deltanet_decode_b1"] = {
        "value": 1.0 / _median_time(dn0(threads)), "unit": "tokens/s", "cores": threads, "kind": "port",
        "sample": f"config 0, one DeltaNet decode step (batch 1), {threads} threads; {med}",
        "single_thread": {"value": 1.0 / _median_time(dn0(1)), "unit": "tokens/s", "cores": 1}}

    # config 2
    rng = np.random.default_rng(1008)
    ctxlen = 8192
    for B in (1, 8, 32):
        lengths = rng.integers(1, ctxlen + 1, B).astype(np.int32)
        q = rng.standard_normal((B, 16, 256)).astype(np.float32)
        K = _filled((B, ctxlen, 2, 256), rng)
        V = _filled((B, ctxlen, 2, 256), rng)
        a1 = _median_time(lambda: CB.attention_decode(L, q, K, V, lengths, threads=1))
        an = _median_time(lambda: CB.attention_decode(L, q, K, V, lengths, threads=threads))
        out[f"c2_gqa_decode_b{B}"] = {
            "value": B / an, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"config 2 batch {B}, context 8192, lengths "
                      f"{lengths.tolist() if B <= 8 else 'U[1, 8192]'}: split-KV decode attention of 16 q heads "
                      f"per sequence, {threads} threads; {med}",
            "single_thread": {"value": B / a1, "unit": "tokens/s", "cores": 1}}
        del K, V

    # config 3: token-by-token prefill sample at mid-sequence
    T, t0, t1_ = 8192, 4064, 4096
    x = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((t1_, 2048)).astype(np.float32)))
    parts = []
    for i, rows in enumerate((8192, 512, 512)):
        w, sc, bi = synth.q4_weight(rows, 2048, seed=300 + i)
        parts.append((w, O.f16_to_f32(sc), O.f16_to_f32(bi)))
    w, sc, bi = CB.q4_stack(parts)
    gp = synth.gqa_params()
    K = _filled((T, 2, 256), rng)
    V = _filled((T, 2, 256), rng)
    att = np.zeros((t1_, 16, 256), np.float32)
    t3 = _median_time(lambda: CB.gqa_prefill_tokens(L, t0, t1_, x, w, sc, bi, gp["q_norm_w"], gp["k_norm_w"], K, V,
                                                    att, threads=threads), reps=3, warm=1)
    v3 = (t1_ - t0) / t3
    out["c3_gqa_prefill_t8192"] = {
        "value": v3, "unit": "tokens/s", "cores": threads, "kind": "port",
        "sample": f"config 3, tokens {t0}-{t1_ - 1} of the 8192-token sequence through the full-attention layer "
                  f"token by token as the reference prefills (Q4 q|gate/k/v projections from hidden 2048, norms, "
                  f"RoPE, attention over positions 0..t, gate), {threads} threads; median of 3 after 1 warm-up; "
                  f"the whole 8192-token prefill at this average rate: {T / v3:.1f} s"}

    # config 4: one layer of each kind, composed as 30 DeltaNet + 10 full attention
    dn_in = CB.q4_stack([(w_, O.f16_to_f32(s_), O.f16_to_f32(b_)) for w_, s_, b_ in
                         (synth.q4_weight(r, 2048, seed=500 + i) for i, r in enumerate((8192, 4096, 32, 32)))])
    outp = synth.q4_weight(2048, 4096, seed=510)
    dn_out = CB.q4_stack([(outp[0], O.f16_to_f32(outp[1]), O.f16_to_f32(outp[2]))])
    norm_w = np.ones(2048, np.float32)
    g_in = CB.q4_stack(parts)
    for B, Lc in ((16, 32768), (1, 65536)):
        xs = rng.standard_normal((B, 2048)).astype(np.float32)
        conv = rng.standard_normal((B, 8192, 4)).astype(np.float32)
        ssm = (rng.standard_normal((B, 32, 128, 128)) * 0.02).astype(np.float32)
        Kc = _filled((B, Lc, 2, 256), rng)
        Vc = _filled((B, Lc, 2, 256), rng)
        pos = np.full(B, Lc - 1, np.int32)
        t_dn = _median_time(lambda: CB.dn_layer_decode(L, xs, norm_w, dn_in, dn_out, p, conv, ssm, threads=threads),
                            reps=3, warm=1)
        t_gq = _median_time(lambda: CB.gqa_layer_decode(L, xs, norm_w, g_in, dn_out, gp["q_norm_w"],
                                                        gp["k_norm_w"], Kc, Vc, pos, threads=threads), reps=3, warm=1)
        step = 30 * t_dn + 10 * t_gq
        out[f"c4_stack_b{B}_l{Lc}"] = {
            "value": B / step, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"config 4 at batch {B}, context {Lc}: one Gated DeltaNet layer ({t_dn * 1e3:.2f} ms) and one "
                      f"full-attention layer ({t_gq * 1e3:.2f} ms) of the stack's attention blocks, {threads} "
                      f"threads, median of 3 after 1 warm-up, composed as 30 + 10 layers: {step * 1e3:.1f} ms "
                      f"per step"}
        del Kc, Vc
    return out


def measured_peaks():
    """What this MI355X delivers, measured with the probes of
    qwen-fieldfare_amd/probe/peaks.hip (lib/libqff_probe.so): an MFMA loop
    (16,384 waves, each with two independent v_mfma_f32_32x32x16_bf16
    chains, then each with sixteen v_mfma_f32_16x16x32_bf16 chains) and a grid-stride 16-byte streaming read of 2 GiB, copy of 1 GiB
    and in-place scale of 1 GiB (read + write of the same bytes, the traffic
    of an in-place state update), each timed with HIP events on the launch
    stream over 5 launches after 2 warm-ups. Reported beside the datasheet peaks the rooflines use
    (BASELINE: the builder re-measures them)."""
    import ctypes
    import torch
    L = ctypes.CDLL(os.path.join(ROOT, "qwen-fieldfare_amd", "lib", "libqff_probe.so"))
    vp, i32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    L.qffp_mfma_bf16.argtypes = [vp, i32, i32, i32, vp]
    L.qffp_stream_read.argtypes = [vp, vp, sz, i32, vp]
    L.qffp_stream_copy.argtypes = [vp, vp, vp, sz, i32]
    L.qffp_stream_rmw.argtypes = [vp, vp, sz, i32]
    st = torch.cuda.current_stream()
    sv = ctypes.c_void_p(st.cuda_stream)

    def time_launch(fn, reps=5, warm=2):
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(reps):
            fn()
        e1.record(st)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e-3

    blocks, iters = 4096, 2000
    sink = torch.empty(max(blocks * 4, 8192 * 256), device="cuda")
    mfma_tf = {}
    # flops per wave and iteration: two 32x32x16 (32,768 each), sixteen 16x16x32 (16,384 each)
    for shape, name, per_it in ((0, "32x32x16", 2 * 32768), (1, "16x16x32", 16 * 16384)):
        t = time_launch(lambda: L.qffp_mfma_bf16(sv, shape, blocks, iters, ctypes.c_void_p(sink.data_ptr())))
        mfma_tf[name] = blocks * 4 * iters * per_it / t / 1e12
    nbytes = 2 << 30
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    dst = torch.empty(nbytes // 2, dtype=torch.uint8, device="cuda")
    rd = {}
    for nb in (2048, 8192):
        tr = time_launch(lambda: L.qffp_stream_read(sv, ctypes.c_void_p(src.data_ptr()), nbytes, nb,
                                                    ctypes.c_void_p(sink.data_ptr())))
        rd[nb] = nbytes / tr / 1e9
    tc = time_launch(lambda: L.qffp_stream_copy(sv, ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()),
                                                nbytes // 2, 8192))
    tw = time_launch(lambda: L.qffp_stream_rmw(sv, ctypes.c_void_p(dst.data_ptr()), nbytes // 2, 8192))
    del src, dst, sink
    torch.cuda.empty_cache()
    best = max(mfma_tf.values())
    return {"mfma_bf16_TFLOPs": best, "mfma_bf16_TFLOPs_by_shape": mfma_tf,
            "mfma_frac_of_datasheet": best / BF16_PEAK_TFLOPS,
            "hbm_read_GBps": max(rd.values()), "hbm_read_GBps_by_grid": rd,
            "hbm_copy_GBps": nbytes / tc / 1e9, "hbm_inplace_rmw_GBps": nbytes / tw / 1e9,
            "hbm_read_frac_of_datasheet": max(rd.values()) / HBM_PEAK_GBS,
            "basis": "probe kernels of qwen-fieldfare_amd/probe/peaks.hip, HIP events, 5 launches after 2 warm-ups; "
                     "copy and in-place count bytes read + written"}


def copy_probe():
    """One elementwise pass (dst = -src, fp32) that reads and writes
    COPY_PROBE_BYTES each, for scaling the FETCH_SIZE / WRITE_SIZE counters
    of a profiling run to bytes. An elementwise kernel spreads over every CU
    like the kernels it calibrates; a runtime blit copy does not always."""
    import torch
    src = torch.ones(COPY_PROBE_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.neg(src, out=dst)
    torch.cuda.synchronize()


COUNTERS_JSON = os.path.join(ROOT, "profiles", "counters.json")


def traffic_for(kernel, workload="c1"):
    """HBM bytes per launch of `kernel` in `workload` from the committed
    counter summary (profiles/counters.json: FETCH_SIZE + WRITE_SIZE scaled
    by the copy probe), or None when it holds no figure for that kernel."""
    try:
        with open(COUNTERS_JSON) as f:
            W = json.load(f)["workloads"][workload]
        hits = [r for k, r in W.items() if k.split("@")[0] == kernel and "traffic_bytes" in r]
        return hits[0]["traffic_bytes"] if len(hits) == 1 else None
    except (OSError, KeyError, ValueError, TypeError):
        return None


def _kernel_key(name):
    """qff::dn_chunk_state_kernel<...>(...) -> dn_chunk_state; torch's
    elementwise negation (the copy probe) -> copy_probe; other kernels keep
    the first 60 characters of their name."""
    if "qff::" in name:
        n = name.split("qff::", 1)[1].split("(")[0].split("<")[0].strip()
        return n[:-len("_kernel")] if n.endswith("_kernel") else n
    if "neg" in name and "elementwise" in name:
        return "copy_probe"
    return name[:60]


def _geometry(gx, gy, gz, wx, wy, wz):
    """'workgroups x.y.z / threads' of a dispatch (rocprofv3 grid sizes
    count work-items)."""
    g = [a // b if b and a % b == 0 else a for a, b in ((gx, wx), (gy, wy), (gz, wz))]
    return f"{g[0]}.{g[1]}.{g[2]}/{wx * wy * wz}"


def summarize_trace(db, out_md, title, command):
    """Kernel-trace summary of one rocprofv3 --kernel-trace database as a
    markdown table: one row per (kernel, launch geometry), calls and
    dispatch durations in microseconds, sorted by total time."""
    import sqlite3
    con = sqlite3.connect(db)
    rows = {}
    for name, start, end, gx, gy, gz, wx, wy, wz in con.execute(
            "select S.display_name, K.start, K.end, K.grid_size_x, K.grid_size_y, K.grid_size_z,"
            " K.workgroup_size_x, K.workgroup_size_y, K.workgroup_size_z from rocpd_kernel_dispatch K"
            " join rocpd_info_kernel_symbol S on S.id = K.kernel_id and S.guid = K.guid"):
        short = name.split("(")[0].replace("void ", "").strip()
        key = (short, _geometry(gx, gy, gz, wx, wy, wz))
        rows.setdefault(key, []).append((end - start) / 1000.0)
    con.close()
    total = sum(sum(v) for v in rows.values()) or 1.0
    lines = [f"# {title}", "", "Command:", "", "    " + command, "",
             "One row per kernel and launch geometry (workgroups x.y.z / threads per workgroup); "
             "durations are rocprofv3 dispatch times in microseconds.", "",
             "| kernel | geometry | calls | avg us | min us | max us | % of kernel time |",
             "|---|---|---:|---:|---:|---:|---:|"]
    for (k, g), v in sorted(rows.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| {k} | {g} | {len(v)} | {sum(v) / len(v):.1f} | {min(v):.1f} | {max(v):.1f} | "
                     f"{100.0 * sum(v) / total:.1f} |")
    with open(out_md, "w") as fh:
        fh.write("\n".join(lines) + "\n")


def summarize_pmc(root, out_json):
    """Per-kernel means of the counter passes under `root` (one rocprofv3
    --pmc output directory per pass, named <pass>_<workload>, pass one of
    mfma / fetch / write) into `out_json`. FETCH_SIZE and WRITE_SIZE are
    scaled to bytes by what the same counter reads for the copy probe of the
    same run (COPY_PROBE_BYTES read and written); MFMA flops are the MOPS
    counters x 512; MFMA utilisation is busy cycles over GUI-active cycles of
    every SIMD."""
    import glob
    import sqlite3
    res = {"copy_probe_bytes": COPY_PROBE_BYTES, "factors": {}, "workloads": {}}
    for d in sorted(glob.glob(os.path.join(root, "*_*"))):
        if not os.path.isdir(d):
            continue
        kind, wl = os.path.basename(d).split("_", 1)
        dbs = glob.glob(os.path.join(d, "**", "*.db"), recursive=True)
        if not dbs:
            continue
        sums, disp = {}, {}
        for db in dbs:
            con = sqlite3.connect(db)
            for did, kname, cname, val, gx, gy, gz, wx, wy, wz in con.execute(
                    "select dispatch_id, kernel_name, counter_name, value, grid_size_x, grid_size_y, grid_size_z,"
                    " workgroup_size_x, workgroup_size_y, workgroup_size_z from counters_collection"):
                k = _kernel_key(kname)
                if k != "copy_probe":
                    k += "@" + _geometry(gx, gy, gz, wx, wy, wz)
                sums[(k, cname)] = sums.get((k, cname), 0.0) + float(val)
                disp.setdefault((k, cname), set()).add((db, did))
            con.close()
        mean = {key: v / len(disp[key]) for key, v in sums.items()}
        W = res["workloads"].setdefault(wl, {})
        for (k, cname), v in mean.items():
            rec = W.setdefault(k, {})
            rec[cname] = v
            rec.setdefault("dispatches", {})[kind] = len(disp[(k, cname)])
        if kind in ("fetch", "write"):
            cname = "FETCH_SIZE" if kind == "fetch" else "WRITE_SIZE"
            probe = [v for (k, c), v in mean.items() if c == cname and k == "copy_probe"]
            if probe:
                res["factors"].setdefault(wl, {})[cname] = COPY_PROBE_BYTES / 1024.0 / probe[0]
    for wl, W in res["workloads"].items():
        f = res["factors"].get(wl, {})
        for k, rec in W.items():
            if "FETCH_SIZE" in rec and "FETCH_SIZE" in f:
                rec["read_bytes"] = rec["FETCH_SIZE"] * 1024.0 * f["FETCH_SIZE"]
            if "WRITE_SIZE" in rec and "WRITE_SIZE" in f:
                rec["write_bytes"] = rec["WRITE_SIZE"] * 1024.0 * f["WRITE_SIZE"]
            if "read_bytes" in rec and "write_bytes" in rec:
                rec["traffic_bytes"] = rec["read_bytes"] + rec["write_bytes"]
            mops = sum(rec.get(c, 0.0) for c in ("SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_INSTS_VALU_MFMA_MOPS_F16",
                                                   "SQ_INSTS_VALU_MFMA_MOPS_F32"))
            if mops:
                rec["mfma_flops"] = mops * 512.0
            if "MfmaUtil" in rec:
                rec["mfma_util_pct"] = rec["MfmaUtil"]
    with open(out_json, "w") as fh:
        json.dump(res, fh, indent=1, sort_keys=True)
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--only", default="", help="comma list of c0,c1,c2,c3,c4,dnb,rt")
    ap.add_argument("--copy-probe", action="store_true", help="also run one copy of known size "
                    "(calibrates FETCH_SIZE / WRITE_SIZE in a counter run)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("DIR", "OUT_JSON"),
                    help="summarise rocprofv3 --pmc pass directories DIR/<pass>_<workload> into OUT_JSON "
                    "and exit (no GPU work)")
    ap.add_argument("--summarize-trace", nargs=4, metavar=("DB", "OUT_MD", "TITLE", "COMMAND"),
                    help="summarise a rocprofv3 --kernel-trace database into a markdown table and exit")
    args = ap.parse_args()
    if args.summarize_pmc:
        summarize_pmc(args.summarize_pmc[0], args.summarize_pmc[1])
        return
    if args.summarize_trace:
        summarize_trace(*args.summarize_trace)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1"}))
        sys.exit(2)

    import torch
    import qff
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    only = set(args.only.split(",")) if args.only else {"c0", "c1", "c2", "c3", "c4", "dnb", "rt"}
    ctx = qff.Context(max_batch=32, max_ctx=8192, max_prefill_tokens=8192)
    configs = {}
    if "c0" in only:
        log("config 0: DeltaNet decode B=1")
        configs["c0_deltanet_decode_b1"] = bench_c0(ctx, max(args.steps * 50, 500), args.warmup * 10)
    if "dnb" in only:
        for B in (16, 32):
            log(f"DeltaNet decode B={B}")
            configs[f"deltanet_decode_b{B}"] = bench_dn_decode_batch(ctx, B, max(args.steps * 5, 100), args.warmup)
    if "rt" in only:
        for B in (1, 16):
            log(f"MoE router B={B}")
            configs[f"router_top8_b{B}"] = bench_router(ctx, B, max(args.steps * 10, 200), args.warmup)
    if "c2" in only:
        for B in (1, 8, 32):
            log(f"config 2: GQA decode B={B}")
            configs[f"c2_gqa_decode_b{B}"] = bench_c2(ctx, B, max(args.steps * 10, 200), args.warmup)
    if "c3" in only:
        log("config 3: GQA prefill T=8192 + Q4 projections")
        configs["c3_gqa_prefill_t8192"] = bench_c3(ctx, max(5, args.steps // 2), 3)
    if "c4" in only:
        for B, L in ((16, 32768), (1, 65536)):
            log(f"config 4: 40-layer stack decode B={B} L={L}")
            configs[f"c4_stack_b{B}_l{L}"] = bench_c4(B, L, max(5, args.steps // 2), 2)
            import torch
            torch.cuda.empty_cache()
    c1 = None
    if "c1" in only:
        log("config 1: DeltaNet prefill T=4096")
        c1 = bench_c1(ctx, args.steps, args.warmup)
        configs["c1_deltanet_prefill_t4096"] = c1
    cpu = None
    if not args.skip_cpu and c1 is not None:
        log("cpu baselines (oracle/cpu_baseline.c)")
        for key, base in cpu_baselines().items():
            if key == "c1_deltanet_prefill_t4096":
                cpu = base
            elif key in configs:
                configs[key]["cpu_baseline"] = base

    if args.copy_probe:
        log("copy probe")
        copy_probe()
    peaks = None
    if c1 is not None:
        log("measured peaks (MFMA loop, streaming read / copy)")
        peaks = measured_peaks()

    roof = None
    if c1 is not None:
        # The workload is MFMA-bound by definition (canonical flops / bytes
        # ~172 flop/B): the dominant kernel's share of the canonical flops
        # over its event-timed duration is the roofline; HBM on the
        # canonical bytes of the whole step rides along.
        kt = c1["kernels_ms"]
        dom = max((k for k in kt if k in C1_KERNEL_FLOPS), key=kt.get)
        roof = mfma_roof(C1_KERNEL_FLOPS[dom], kt[dom], "dominant kernel, event-timed")
        roof.update({"traffic": traffic_for(dom), "kernel": dom, "kernel_ms": kt[dom],
                     "flops_per_launch": C1_KERNEL_FLOPS[dom],
                     "path": {"TFLOPs": c1["roofline"]["achieved"], "mfma_frac": c1["roofline"]["frac"],
                              "hbm_GBps": c1["roofline_hbm"]["achieved"], "hbm_frac": c1["roofline_hbm"]["frac"]}})
    value = c1["tokens_per_s"] if c1 else None
    line = {
        "metric": "attn tokens/s: DeltaNet+GQA decode (B=1..32) & 8K prefill; % HBM/MFMA roofline",
        "value": value, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": c1["ms_per_step"] if c1 else None, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 in/out, fp32 state+accum", "data": "synthetic",
        "config": {"workload": "config 1: Gated DeltaNet chunked prefill, 1 layer, B=1, T=4096, C=64",
                   "global_batch": 1, "seq_len": 4096, "parallelism": "none (1 GPU)"},
        "roofline": roof, "cpu_baseline": cpu, "measured_peaks": peaks, "configs": configs,
    }
    # leave nothing behind on the GPU: the context's workspace and torch's
    # cached blocks are released before the line is printed and the
    # process exits
    torch.cuda.synchronize()
    ctx.close()
    torch.cuda.empty_cache()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
