#!/usr/bin/env python3
"""Benchmark of the MI355X HIP backend on Clove's hot path.

One "step" is one pass of the fused elementwise chain y = gelu(a*b + c) * d
over the four 16,777,216-element f32 inputs of configuration 2 (the workload
the headline metric is quoted on), with every input already resident in HBM.
Consecutive steps of every HBM-bound part cycle through identical copies of
its inputs: at least --sets (default 3), and as many as cover --in-mib
(default 512 MiB, twice MI355X's 256 MB last-level cache, the MALL).  With
fewer, the MALL still holds a step's inputs from the steps before: three
64 MiB copies all fit in it, and a kernel reading 64 MiB in 128-byte column
strips then measured 66% of HBM peak where HBM gave it 43%.
Likewise each step's outputs stay alive for as many steps as cover --out-mib
(default 512 MiB), so consecutive steps write different blocks: one output
block rewritten every step stays partly in the MALL (the config 2 chain reads
~7% faster so).
Rank 0 prints ONE JSON line on stdout:

  value        whole-job algorithmic HBM GB/s of the step (5 x 64 MiB per step)
  roofline     the chain kernel: algorithmic bytes / mean launch duration
               (two HIP events on the library's stream bracketing the K
               back-to-back launches of the timed region) vs the 8 TB/s HBM3E
               peak; `traffic` is the measured HBM bytes per launch from the
               rocprof FETCH_SIZE / WRITE_SIZE summary in profiles/
  cpu_baseline the CPU restatement of Clove's Rayon kernels (oracle/), four
               unfused passes as Clove's eager CPU path runs them, timed on
               this host's cores; every CPU leg runs after all GPU timings
  parts        the other configurations measured in the same run: the
               broadcast chain, softmax and layer norm (GB/s), 4096^3 (plain
               and with the planner's fused bias + GELU epilogue) and skinny
               matmul (TFLOP/s), paged decode (tokens/s and GB/s; config 5
               at D = 128 and the same shape at D = 96, the general kernel), the
               MLP plan (us per forward) and the backward passes and losses
               (GB/s; the matmul backward in TFLOP/s), attention prefill
               (TFLOP/s) and RoPE (GB/s), each with its roofline fraction and
               a CPU baseline over the full workload (the attention prefill's
               on sampled query rows: the full one is ~20 s of host time),
               with the host CPU model; an HBM-bound part's `traffic` is the
               measured bytes per step of its kernels from the same summary.
  parity_checked  true when every checked part's output (one more launch
               of its first input set after all timings, the timed steps'
               bits: the kernels are deterministic) is within its parity
               bound of the oracle's output, computed by its CPU leg (AdamW:
               one step from zero moments on copies, bit for bit; attention:
               the leg's sampled query rows); else the failing parts, and
               the exit status is 1.  parity_parts names the parts checked.
Everything else goes to stderr.  This backend runs on one GPU: --gpus > 1
exits with a message.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, AMD published
FP32_MFMA_PEAK_TFS = 157.3   # MI355X dense FP32 matrix, AMD published
METRIC = "fused-op HBM GB/s (% of peak); f32 GEMM TFLOP/s; paged-decode tokens/s"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Timing:
    """wall: host ms per step over the timed region (device synchronised on
    both sides); kernel: device ms per launch from the two HIP events that
    bracket the launches on the library's stream."""

    def __init__(self, wall, kernel):
        self.wall, self.kernel = wall, kernel

    def mean(self):
        return self.kernel


# Bytes of outputs held across steps (--out-mib) and the least bytes of
# inputs a part's rotation covers (--in-mib): set by main().
OUT_HOLD_BYTES = 512 << 20
IN_ROT_BYTES = 512 << 20


def input_sets(args, bytes_per_set):
    """Copies of a part's inputs its steps cycle through: --sets, or more, so
    that the copies cover IN_ROT_BYTES (twice the 256 MB MALL by default):
    three 64 MiB copies would all fit in the MALL and be read from there."""
    return max(args.sets, -(-IN_ROT_BYTES // bytes_per_set))


def output_tensors(r):
    """The tensors a launch returned (one, a list or tuple of them, or none)."""
    if isinstance(r, (list, tuple)):
        return [t for t in r if hasattr(t, "numel")]
    return [r] if hasattr(r, "numel") else []


def timed(ca, launch, steps, warmup):
    """Runs `launch` warmup + steps times back to back.  Each step's outputs
    stay alive for the next `hold` steps, enough steps that the held outputs
    cover OUT_HOLD_BYTES (twice the 256 MB MALL by default): consecutive steps
    then write different blocks, as they read different input sets, instead of
    rewriting one block the MALL keeps absorbing (a 64 MiB output rewritten
    in place reads ~7% faster than HBM takes it).  Every block is allocated
    during the warmup, so no hipMalloc happens in the timed region; no event
    sits between two launches."""
    r = launch()
    out_bytes = sum(4 * int(t.numel) for t in output_tensors(r))
    hold = 1
    if out_bytes >= (1 << 20) and OUT_HOLD_BYTES > 0:  # outputs the MALL could keep
        hold = min(64, max(1, -(-OUT_HOLD_BYTES // out_bytes)))
    # `hold` blocks rotate: a step releases the oldest outputs, then launches
    # (with --out-mib 0, every step gets the block the step before released)
    ring = [None] * hold
    ring[0] = r
    del r
    i = 1
    for _ in range(max(warmup, hold)):
        ring[i % hold] = None
        ring[i % hold] = launch()
        i += 1
    ca.synchronize()
    ca.event_reset()
    t0 = time.perf_counter()
    e0 = ca.event_record()
    for _ in range(steps):
        ring[i % hold] = None
        ring[i % hold] = launch()
        i += 1
    e1 = ca.event_record()
    ca.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    ring.clear()
    return wall, Timing(wall, ca.event_elapsed(e0, e1) / steps)


def rotating(launches):
    """One launch callable per input set; each call of the result runs the
    next set's, so consecutive steps read different copies of the inputs."""
    i = [0]

    def run():
        f = launches[i[0] % len(launches)]
        i[0] += 1
        return f()
    return run


# CPU baseline legs, run after every GPU timing has finished: run in between,
# they changed the GPU times of the parts timed after them (the cross-entropy
# steps by up to 4 us).
CPU_LEGS = []


def defer(leg):
    CPU_LEGS.append(leg)


def cpu_time(fn, reps=3, keep=None):
    """Median seconds of `reps` runs of fn; the last run's result is appended
    to `keep` when a list is given."""
    best = []
    for _ in range(reps):
        t0 = time.perf_counter()
        r = fn()
        best.append(time.perf_counter() - t0)
    if keep is not None:
        keep.append(r)
    return float(np.median(best))


# Output parity of the timed parts: after every GPU timing, each checked part
# runs once more on its first input set (the bytes its timed steps read; every
# kernel here is deterministic, so these are the timed steps' output bits)
# and is compared with the oracle's output, which its CPU leg computes anyway,
# at the bound its parity tests use: |g - c| <= atol + rtol |c|.
PARITY = {}


def check_parity(name, got, want, rtol, atol):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    if got.shape != want.shape:
        PARITY[name] = f"shape {got.shape} != {want.shape}"
        return
    err = np.abs(got - want)
    bad = ~(err <= atol + rtol * np.abs(want))
    PARITY[name] = "ok" if not bad.any() else \
        f"{int(bad.sum())} of {err.size} elements out of bound (max abs err {err.max():.3e})"
    log(f"parity {name}: {PARITY[name]}")


def gemm_atol(want):
    return 1e-4 * float(np.abs(want).max() or 1.0)


def cpu_model():
    """The host CPU's model name from /proc/cpuinfo (the baseline's hardware)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_record(oracle, value, unit, sample):
    """A cpu_baseline object: the oracle (a restatement of Clove's Rayon
    kernels, kind "port") on `oracle.threads()` host threads."""
    return {"value": value, "unit": unit, "cores": oracle.threads(), "kind": "port",
            "cpu_model": cpu_model(), "sample": sample}


def roofline(bound, achieved, peak, unit, traffic=None):
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


# ---------------------------------------------------------------------------
# parts
# ---------------------------------------------------------------------------

CHAIN = [("mul", -1, -2), ("add", 0, -3), ("gelu", 1), ("mul", 2, -4)]


def bench_chain(ca, args, broadcast=False):
    n = 4096 * 4096
    sets = []
    for _ in range(input_sets(args, 4 * n * (3 if broadcast else 4))):  # identical copies
        ins = [ca.empty((4096, 4096)).fill_normal(1 + i) for i in range(4)]
        if broadcast:
            ins[2] = ca.empty((4096,)).fill_normal(3)
        sets.append(ins)
    nbytes = 4 * n * 5 if not broadcast else 4 * n * 4 + 4 * 4096
    wall, per = timed(ca, rotating([ca.FusedChain(CHAIN, ins) for ins in sets]), args.steps,
                      args.warmup)
    return sets[0], nbytes, wall, per


def cpu_chain(oracle, ins_host):
    a, b, c, d = ins_host
    return lambda: oracle.mul(oracle.gelu(oracle.add(oracle.mul(a, b), c)), d)


def bench_rows(ca, oracle, args, out):
    g = np.random.Generator(np.random.PCG64(2))
    xs_sets = [ca.empty((8192, 4096)).fill_normal(2, 0.0, 2.0)
               for _ in range(input_sets(args, 4 * 8192 * 4096))]
    x = xs_sets[0]
    gam = ca.tensor(g.uniform(0.5, 1.5, 4096).astype(np.float32))
    bet = ca.tensor(g.uniform(-0.1, 0.1, 4096).astype(np.float32))
    n = 8192 * 4096
    for name, launch, nbytes in (
            ("softmax", rotating([lambda x=x: ca.softmax(x) for x in xs_sets]), 2 * 4 * n),
            ("layer_norm", rotating([lambda x=x: ca.layer_norm(x, gam, bet) for x in xs_sets]),
             2 * 4 * n + 2 * 4 * 4096)):
        wall, per = timed(ca, launch, args.steps, args.warmup)
        gbs = nbytes / (per.mean() * 1e-3) / 1e9
        part = {"value": round(gbs, 1), "unit": "GB/s", "ms": round(per.mean(), 4),
                "bytes": nbytes, "roofline": roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s")}
        if not args.no_cpu:
            def leg(name=name, part=part, nbytes=nbytes):
                xs = x.numpy()
                gh, bh = gam.numpy(), bet.numpy()
                fn = (lambda: oracle.softmax(xs)) if name == "softmax" else \
                    (lambda: oracle.layer_norm(xs, gh, bh))
                want = []
                t = cpu_time(fn, keep=want)
                part["cpu_baseline"] = cpu_record(oracle, round(nbytes / t / 1e9, 2), "GB/s",
                                                  "full [8192, 4096] workload, median of 3")
                if name == "softmax":
                    check_parity(name, ca.softmax(x).numpy(), want[0], 1e-4, 1e-9)
                else:
                    check_parity(name, ca.layer_norm(x, gam, bet).numpy(), want[0], 1e-4, 1e-5)
            defer(leg)
        out[name] = part
        log(f"{name}: {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of HBM peak), {per.mean() * 1e3:.1f} us")


def bench_matmul(ca, oracle, args, out, skinny_only=False):
    K = 4096
    a = ca.empty((4096, K)).fill_normal(3, 0.0, 1 / 64)
    b = ca.empty((K, 4096)).fill_normal(33, 0.0, 1 / 64)
    a32 = ca.empty((32, K)).fill_normal(333, 0.0, 1 / 64)
    if skinny_only:
        bench_skinny(ca, oracle, args, out, a32, b)
        return
    steps = max(5, args.steps // 10)
    # 30 untimed launches (~30 ms) bring the clocks from the HBM-bound parts
    # before to their steady MFMA level (10 left the first timed launches
    # ~5% slow)
    wall, per = timed(ca, lambda: ca.matmul(a, b), steps, max(30, args.warmup))
    flops = 2.0 * 4096 ** 3
    tf = flops / (per.mean() * 1e-3) / 1e12
    part = {"value": round(tf, 2), "unit": "TFLOP/s", "ms": round(per.mean(), 4),
            "roofline": roofline("mfma", tf, FP32_MFMA_PEAK_TFS, "TFLOP/s")}
    if not args.no_cpu:
        def leg():
            ah, bh = a.numpy(), b.numpy()
            want = []
            t = cpu_time(lambda: oracle.matmul(ah, bh), reps=1, keep=want)
            part["cpu_baseline"] = cpu_record(oracle, round(flops / t / 1e12, 5), "TFLOP/s",
                                              "full 4096^3 product (B transpose included), "
                                              "one run")
            check_parity("matmul_4096", ca.matmul(a, b).numpy(), want[0], 2e-3,
                         gemm_atol(want[0]))
            ah32 = a32.numpy()
            want = []
            t = cpu_time(lambda: oracle.matmul(ah32, bh), reps=3, keep=want)
            out["matmul_skinny_32"]["cpu_baseline"] = cpu_record(
                oracle, round(2.0 * 32 * K * 4096 / t / 1e12, 5), "TFLOP/s",
                "full 32x4096x4096 product (B transpose included), median of 3")
            check_parity("matmul_skinny_32", ca.matmul(a32, b).numpy(), want[0], 2e-3,
                         gemm_atol(want[0]))
        defer(leg)
    out["matmul_4096"] = part
    log(f"matmul 4096^3: {tf:.1f} TFLOP/s ({tf / FP32_MFMA_PEAK_TFS:.1%} of FP32 MFMA peak), "
        f"{per.mean():.3f} ms")
    # the planner's GEMM with a fused bias + GELU epilogue (one step)
    bias = ca.empty((4096,)).fill_normal(7)
    g = ca.Graph()
    x, w, bi = g.input("4096,4096"), g.input("4096,4096"), g.input("4096")
    model = g.compile([g.op("gelu", g.op("add", g.op("matmul", x, w), bi))])
    assert model.num_steps == 1, model.describe()
    wall, per = timed(ca, lambda: model.execute([a, b, bias])[0], steps, args.warmup)
    tf = flops / (per.mean() * 1e-3) / 1e12
    epart = {"value": round(tf, 2), "unit": "TFLOP/s", "ms": round(per.mean(), 4),
             "roofline": roofline("mfma", tf, FP32_MFMA_PEAK_TFS, "TFLOP/s")}
    if not args.no_cpu:
        def eleg():
            ah, bh, biash = a.numpy(), b.numpy(), bias.numpy()
            want = []
            t = cpu_time(lambda: oracle.gelu(oracle.add(oracle.matmul(ah, bh), biash)), reps=1,
                         keep=want)
            epart["cpu_baseline"] = cpu_record(oracle, round(flops / t / 1e12, 5), "TFLOP/s",
                                               "full 4096^3 product, bias and GELU, one run")
            check_parity("matmul_4096_bias_gelu", model.execute([a, b, bias])[0].numpy(),
                         want[0], 2e-3, gemm_atol(want[0]))
        defer(eleg)
    out["matmul_4096_bias_gelu"] = epart
    log(f"matmul 4096^3 + bias + GELU (fused): {tf:.1f} TFLOP/s, {per.mean():.3f} ms")
    bench_skinny(ca, oracle, args, out, a32, b)


def bench_skinny(ca, oracle, args, out, a32, b):
    K = 4096
    # B (64 MiB) is what the skinny product streams: one copy per input set
    bs = [b] + [ca.empty((K, 4096)).fill_normal(33, 0.0, 1 / 64)
                for _ in range(input_sets(args, 4 * K * 4096) - 1)]
    wall, per = timed(ca, rotating([lambda bb=bb: ca.matmul(a32, bb) for bb in bs]), args.steps,
                      args.warmup)
    del bs[1:]
    nbytes = 4 * (32 * K + K * 4096 + 32 * 4096)
    gbs = nbytes / (per.mean() * 1e-3) / 1e9
    tfs = 2.0 * 32 * K * 4096 / (per.mean() * 1e-3) / 1e12
    out["matmul_skinny_32"] = {"value": round(tfs, 2), "unit": "TFLOP/s", "ms": round(per.mean(), 4),
                               "gbs": round(gbs, 1),
                               "roofline": roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s")}
    log(f"matmul 32x4096x4096: {tfs:.2f} TFLOP/s, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%}), "
        f"{per.mean() * 1e3:.1f} us")


def bench_paged(ca, oracle, args, out):
    """Config 5 (D = 128, the fixed-shape kernel), and the same shape at
    D = 96, a head dim only the general kernel runs (a 3072-wide model with
    32 heads)."""
    from clove_amd import workloads

    for D, name in ((workloads.PAGED["head_dim"], "paged_decode"), (96, "paged_decode_d96")):
        paged_case(ca, oracle, args, out, D, name)


def paged_case(ca, oracle, args, out, D, name):
    from clove_amd import workloads

    P = workloads.PAGED
    B, H, bs, nb = P["num_seqs"], P["num_heads"], P["block_size"], P["pool_blocks"]
    ctx, bt = workloads.paged_layout(4)
    kv = ca.empty((2, nb, bs, H, D)).fill_normal(4)
    q = ca.tensor(np.random.Generator(np.random.PCG64(4)).standard_normal((B, H * D), dtype=np.float32))
    tbt, tcl = ca.tensor(bt), ca.tensor(ctx)
    wall, per = timed(ca, lambda: ca.paged_attention(q, None, None, kv, tbt, tcl), args.steps,
                      args.warmup)
    nbytes = workloads.paged_bytes(ctx, H, D, bs)
    sec = per.mean() * 1e-3
    gbs = nbytes / sec / 1e9
    part = {"value": round(B / sec, 1), "unit": "tokens/s", "ms": round(per.mean(), 4),
            "gbs": round(gbs, 1), "bytes": nbytes, "context_tokens": int(ctx.sum()),
            "head_dim": D, "roofline": roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s")}
    if not args.no_cpu:
        def leg():
            seqs = list(range(B))
            plane, blk = nb * bs * H * D, bs * H * D
            # the blocks the 32 sequences use, renumbered: the same rows the
            # decode reads from the full pool
            pool, sbt, scl = workloads.compact_pool(
                lambda p, b: kv.read(p * plane + b * blk, blk).reshape(bs, H, D), bt, ctx, seqs,
                bs)
            qh = q.numpy()
            want = []
            t = cpu_time(lambda: oracle.paged_attention(qh, None, None, pool, sbt, scl),
                         keep=want)
            part["cpu_baseline"] = cpu_record(oracle, round(B / t, 2), "tokens/s",
                                              f"full config 5 decode at D={D} (32 sequences, "
                                              "all heads) on the blocks it reads, median of 3")
            got = ca.paged_attention(q, None, None, kv, tbt, tcl).numpy()
            check_parity(name, got, want[0].reshape(got.shape), 2e-3, 1e-5)
            kv.free()
        defer(leg)
    else:
        kv.free()
    out[name] = part
    log(f"{name} (D={D}): {B / sec:.0f} tokens/s, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of "
        f"HBM), {per.mean() * 1e3:.1f} us")


def bench_mlp(ca, oracle, args, out):
    from clove_amd import workloads

    x, w1, b1, w2, b2 = workloads.mlp_inputs(0)
    g = ca.Graph()
    ids = [g.input("64,784"), g.input("784,128"), g.input("1,128"), g.input("128,10"),
           g.input("1,10")]
    h = g.op("relu", g.op("add", g.op("matmul", ids[0], ids[1]), ids[2]))
    y = g.op("softmax", g.op("add", g.op("matmul", h, ids[3]), ids[4]))
    model = g.compile([y])
    ins = [ca.tensor(v) for v in (x, w1, b1, w2, b2)]
    wall, per = timed(ca, lambda: model.execute(ins), args.steps, args.warmup)
    part = {"value": round(wall * 1e3, 2), "unit": "us/forward (wall, plan of "
            f"{model.num_steps} steps)", "gpu_us": round(per.mean() * 1e3, 2)}
    if not args.no_cpu:
        def leg():
            want = []
            t = cpu_time(lambda: oracle.mlp_forward(x, w1, b1, w2, b2), reps=5, keep=want)
            part["cpu_baseline"] = cpu_record(oracle, round(t * 1e6, 1), "us/forward",
                                              "full config 1 forward, median of 5")
            check_parity("mlp_forward", model.execute(ins)[0].numpy(), want[0], 1e-4, 1e-7)
        defer(leg)
    out["mlp_forward"] = part
    log(f"mlp plan: {wall * 1e3:.1f} us/forward wall, {per.mean() * 1e3:.1f} us GPU")


def bench_backward(ca, oracle, args, out):
    """The backward row: each op at a config-sized shape, HBM roofline (the
    matmul backward: FP32 MFMA), CPU baseline on a bounded sample."""
    g = np.random.Generator(np.random.PCG64(7))
    R, Cc, N = 8192, 4096, 4096 * 4096
    targets = ca.tensor(g.integers(0, Cc, R).astype(np.float32))
    one = ca.tensor(np.ones(1, np.float32))
    sets = []
    # identical copies (same seeds), enough for the smallest input (64 MiB)
    for _ in range(input_sets(args, 4 * N)):
        x = ca.empty((R, Cc)).fill_normal(2, 0.0, 2.0)
        sets.append({"x": x, "y": ca.softmax(x), "dy": ca.empty((R, Cc)).fill_normal(21),
                     "a": ca.empty((4096, 4096)).fill_normal(5),
                     "b": ca.empty((4096, 4096)).fill_normal(6)})
    x, y, dy, a, b = (sets[0][k] for k in ("x", "y", "dy", "a", "b"))

    def each(f):
        return rotating([lambda t=t: f(t) for t in sets])
    cases = [
        ("softmax_backward", each(lambda t: ca.softmax_backward(t["y"], t["dy"])), 3 * 4 * R * Cc),
        ("gelu_backward", each(lambda t: ca.gelu_backward(t["a"], t["b"])), 3 * 4 * N),
        ("broadcast_grad", each(lambda t: ca.broadcast_grad(t["a"], 4096)), 4 * N + 4 * 4096),
        ("cross_entropy", each(lambda t: ca.cross_entropy(t["x"], targets)), 4 * R * Cc + 4 * R),
        ("cross_entropy_backward", each(lambda t: ca.cross_entropy_backward(t["x"], targets, one)),
         2 * 4 * R * Cc + 4 * R),
        ("mse", each(lambda t: ca.mse(t["a"], t["b"])), 2 * 4 * N),
        ("mse_backward", each(lambda t: ca.mse_backward(t["a"], t["b"], one)), 3 * 4 * N),
    ]
    for name, launch, nbytes in cases:
        wall, per = timed(ca, launch, args.steps, args.warmup)
        gbs = nbytes / (per.mean() * 1e-3) / 1e9
        part = {"value": round(gbs, 1), "unit": "GB/s", "ms": round(per.mean(), 4),
                "bytes": nbytes, "roofline": roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s")}
        if oracle is not None:
            def leg(name=name, part=part, nbytes=nbytes):
                part["cpu_baseline"], want = cpu_backward(oracle, name, y, dy, x, targets, a, b,
                                                          nbytes)
                backward_parity(ca, name, want, y, dy, x, targets, one, a, b)
            defer(leg)
        out[name] = part
        log(f"{name}: {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of HBM peak), "
            f"{per.mean() * 1e3:.1f} us")
    del sets[1:]
    # AdamW on a 4096x4096 parameter: reads w, g, m, v, writes w, m, v; the
    # steps cycle through copies of (w, g, m, v) as the other parts cycle
    # through input sets (each copy is updated in place)
    copies = []
    for _ in range(input_sets(args, 4 * 4 * N)):
        copies.append((ca.empty((4096, 4096)).fill_normal(11),
                       ca.empty((4096, 4096)).fill_normal(12, 0.0, 65536.0),
                       ca.tensor(np.zeros(N, np.float32)), ca.tensor(np.zeros(N, np.float32))))
    w, gw = copies[0][0], copies[0][1]
    step = [0]

    def adamw_once():
        k = step[0]
        step[0] += 1
        c = copies[k % len(copies)]
        ca.adamw_step([c[0]], [c[1]], [c[2]], [c[3]], k // len(copies) + 1)
    wall, per = timed(ca, adamw_once, args.steps, args.warmup)
    nbytes = 28 * N
    gbs = nbytes / (per.mean() * 1e-3) / 1e9
    part = {"value": round(gbs, 1), "unit": "GB/s", "ms": round(per.mean(), 4), "bytes": nbytes,
            "roofline": roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s")}
    if oracle is not None:
        def leg(part=part, nbytes=nbytes):
            wh, gh = w.numpy(), gw.numpy()
            zh = np.zeros(N, np.float32)
            want = []
            t = cpu_time(lambda: oracle.adamw(wh, gh, zh, zh, 1), keep=want)
            # one more step, from zero moments on fresh copies of the
            # parameter and gradient the oracle stepped, bit for bit
            tw, tm, tv = ca.tensor(wh), ca.tensor(zh), ca.tensor(zh)
            ca.adamw_step([tw], [ca.tensor(gh)], [tm], [tv], 1)
            check_parity("adamw_4096x4096",
                         np.concatenate([t_.numpy().ravel() for t_ in (tw, tm, tv)]),
                         np.concatenate([h.ravel() for h in want[0]]), 0.0, 0.0)
            part["cpu_baseline"] = cpu_record(oracle, round(nbytes / t / 1e9, 2), "GB/s",
                                              "full 16.7M-element parameter, one step, "
                                              "median of 3")
        defer(leg)
    out["adamw_4096x4096"] = part
    log(f"adamw 4096x4096: {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of HBM peak), "
        f"{per.mean() * 1e3:.1f} us")
    # AdamW over the MLP's four parameters in one launch (latency-bound)
    from clove_amd import workloads
    mlp = [ca.tensor(p) for p in workloads.mlp_inputs(0)[1:]]
    mlp_g = [ca.tensor(np.full(p.numel, 100.0, np.float32)) for p in mlp]
    mlp_m = [ca.tensor(np.zeros(p.numel, np.float32)) for p in mlp]
    mlp_v = [ca.tensor(np.zeros(p.numel, np.float32)) for p in mlp]
    step2 = [0]

    def adamw_mlp():
        step2[0] += 1
        ca.adamw_step(mlp, mlp_g, mlp_m, mlp_v, step2[0])
    wall, per = timed(ca, adamw_mlp, args.steps, args.warmup)
    out["adamw_mlp_params"] = {"value": round(wall * 1e3, 2),
                               "unit": "us/step (wall, 4 tensors, 1 launch)",
                               "gpu_us": round(per.mean() * 1e3, 2)}
    log(f"adamw MLP parameters: {wall * 1e3:.1f} us/step wall")
    # matmul backward at 4096^3: grad_a and grad_b, two GEMMs and two transposes
    dc = ca.empty((4096, 4096)).fill_normal(8)
    steps = max(5, args.steps // 10)
    wall, per = timed(ca, lambda: ca.matmul_backward(a, b, dc), steps, max(15, args.warmup // 2))
    flops = 4.0 * 4096 ** 3
    tf = flops / (per.mean() * 1e-3) / 1e12
    part = {"value": round(tf, 2), "unit": "TFLOP/s", "ms": round(per.mean(), 4),
            "roofline": roofline("mfma", tf, FP32_MFMA_PEAK_TFS, "TFLOP/s")}
    if oracle is not None:
        def leg(part=part):
            ah, bh, dch = a.numpy(), b.numpy(), dc.numpy()
            want = []
            t = cpu_time(lambda: oracle.matmul_backward(ah, bh, dch), reps=1, keep=want)
            da, db = ca.matmul_backward(a, b, dc)
            check_parity("matmul_backward_4096", np.stack([da.numpy(), db.numpy()]),
                         np.stack(want[0]), 2e-3, gemm_atol(np.stack(want[0])))
            part["cpu_baseline"] = cpu_record(oracle, round(flops / t / 1e12, 5), "TFLOP/s",
                                              "full grad_a and grad_b at 4096^3, one run")
        defer(leg)
    out["matmul_backward_4096"] = part
    log(f"matmul backward 4096^3: {tf:.1f} TFLOP/s ({tf / FP32_MFMA_PEAK_TFS:.1%} of FP32 MFMA "
        f"peak), {per.mean():.3f} ms")


def backward_parity(ca, name, want, y, dy, x, targets, one, a, b):
    """The first input set's output of a backward part against the oracle's,
    at the bound of that op's parity test."""
    if name == "softmax_backward":
        got = ca.softmax_backward(y, dy).numpy()
        # the row sum s (summed in another order) reaches dx as y * ds
        yh, dyh = y.numpy(), dy.numpy()
        ds = 1e-5 * np.sum(np.abs(dyh * yh), axis=-1, keepdims=True)
        err = np.abs(got.astype(np.float64) - want)
        bad = ~(err <= 1e-4 * np.abs(want) + yh * ds + 1e-12)
        PARITY[name] = "ok" if not bad.any() else f"{int(bad.sum())} elements out of bound"
        log(f"parity {name}: {PARITY[name]}")
        return
    if name == "mse":
        # Clove's sequential f32 fold over 16.7M terms of ~2 ends ~3% low (its
        # running sum's ulp reaches 2), so the loss is held to float64, as in
        # its parity test; the oracle's output stays the CPU leg's workload
        got = ca.mse(a, b).numpy()
        ah, bh = a.numpy().astype(np.float64), b.numpy()
        exact = np.mean((ah - bh) ** 2)
        check_parity(name, got, np.full(got.shape, exact), 1e-4, 0.0)
        return
    got, rtol, atol = {
        "gelu_backward": (lambda: ca.gelu_backward(a, b), 1e-5, 2e-6),
        # sums of 4096 unit normals, in another order than the oracle's
        "broadcast_grad": (lambda: ca.broadcast_grad(a, 4096), 1e-4, np.sqrt(4096) * 1e-5),
        "cross_entropy": (lambda: ca.cross_entropy(x, targets), 1e-4, 0.0),
        "cross_entropy_backward": (lambda: ca.cross_entropy_backward(x, targets, one), 1e-4,
                                   1e-10),
        "mse_backward": (lambda: ca.mse_backward(a, b, one), 1e-6, 1e-30),
    }[name]
    got = got().numpy()
    check_parity(name, got, np.asarray(want).reshape(got.shape), rtol, atol)


def cpu_backward(oracle, name, y, dy, x, targets, a, b, nbytes):
    """(cpu_baseline record, the oracle's output) of one backward part."""
    if name in ("softmax_backward", "cross_entropy", "cross_entropy_backward"):
        th = targets.numpy()
        if name == "softmax_backward":
            ys, dys = y.numpy(), dy.numpy()
            fn = lambda: oracle.softmax_backward(ys, dys)
        else:
            xs = x.numpy()
            fn = (lambda: oracle.cross_entropy(xs, th)) if name == "cross_entropy" else \
                (lambda: oracle.cross_entropy_backward(xs, th, 1.0))
        want = []
        t = cpu_time(fn, keep=want)
        sample = "full [8192, 4096] workload, median of 3"
    else:
        ah, bh = a.numpy(), b.numpy()
        fn = {"gelu_backward": lambda: oracle.gelu_backward(ah, bh),
              "broadcast_grad": lambda: oracle.bias_grad(ah, 4096),
              "mse": lambda: oracle.mse(ah, bh),
              "mse_backward": lambda: oracle.mse_backward(ah, bh, 1.0)}[name]
        want = []
        t = cpu_time(fn, keep=want)
        sample = "full [4096, 4096] workload, median of 3"
    return cpu_record(oracle, round(nbytes / t / 1e9, 2), "GB/s", sample), want[0]


def bench_attention(ca, oracle, args, out):
    """Attention prefill (the fused FlashAttention step): B=1, S=4096, H=32,
    D=128, causal + RoPE; algorithmic FLOPs 4*D*H*S(S+1)/2 (QK^T and PV over
    the visible keys); FP32 MFMA roofline.  Also RoPE alone (HBM)."""
    B, S, H, D = 1, 4096, 32, 128
    q = ca.empty((B, S, H * D)).fill_normal(31)
    k = ca.empty((B, S, H * D)).fill_normal(32)
    v = ca.empty((B, S, H * D)).fill_normal(33)
    steps = max(5, args.steps // 10)
    wall, per = timed(ca, lambda: ca.flash_attention(q, k, v, H), steps, max(10, args.warmup // 2))
    flops = 4.0 * D * H * S * (S + 1) / 2
    tf = flops / (per.mean() * 1e-3) / 1e12
    part = {"value": round(tf, 2), "unit": "TFLOP/s", "ms": round(per.mean(), 4),
            "roofline": roofline("mfma", tf, FP32_MFMA_PEAK_TFS, "TFLOP/s")}
    if oracle is not None:
        def leg():
            qh, kh, vh = q.numpy(), k.numpy(), v.numpy()
            rows = [255 + 256 * i for i in range(16)]  # mean visible keys ~ S/2, as over all rows
            t_rope = cpu_time(lambda: oracle.attention(qh, kh, vh, H, rows=(0, 0)), reps=1)
            t_rows = 0.0
            want = []
            for r in rows:
                t_rows += cpu_time(lambda: oracle.attention(qh, kh, vh, H, rows=(r, r + 1)),
                                   reps=1, keep=want)
            got = ca.flash_attention(q, k, v, H).numpy()
            check_parity("flash_attention_4096", np.stack([got[:, r] for r in rows]),
                         np.stack([w[:, r] for w, r in zip(want, rows)]), 2e-3, 1e-5)
            t_rows = max(t_rows - len(rows) * t_rope, 0.0)
            t = t_rope + t_rows * S / len(rows)
            part["cpu_baseline"] = cpu_record(oracle, round(flops / t / 1e12, 5), "TFLOP/s",
                                              f"{len(rows)} of {S} query rows (all heads) plus "
                                              "the full RoPE of q and k, row time scaled (the "
                                              "full prefill is about 20 s of host time)")
        defer(leg)
    out["flash_attention_4096"] = part
    log(f"attention prefill S=4096 H=32 D=128 causal+rope: {tf:.1f} TFLOP/s "
        f"({tf / FP32_MFMA_PEAK_TFS:.1%} of FP32 MFMA peak), {per.mean():.3f} ms")
    xs_sets = [ca.empty((1, S, H * D)).fill_normal(34)
               for _ in range(input_sets(args, 4 * S * H * D))]
    x = xs_sets[0]
    wall, per = timed(ca, rotating([lambda x=x: ca.rope(x, D) for x in xs_sets]), args.steps,
                      args.warmup)
    del xs_sets[1:]
    nbytes = 2 * 4 * S * H * D
    gbs = nbytes / (per.mean() * 1e-3) / 1e9
    out["rope"] = {"value": round(gbs, 1), "unit": "GB/s", "ms": round(per.mean(), 4),
                   "bytes": nbytes, "roofline": roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s")}
    if oracle is not None:
        def leg2():
            xs = x.numpy()
            want = []
            t = cpu_time(lambda: oracle.rope(xs, D), keep=want)
            check_parity("rope", ca.rope(x, D).numpy(), want[0], 1e-5, 1e-6 * S / 64)
            out["rope"]["cpu_baseline"] = cpu_record(oracle, round(nbytes / t / 1e9, 2), "GB/s",
                                                     f"full [{S}, {H * D}] workload, median of 3")
        defer(leg2)
    log(f"rope [4096, 4096]: {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%}), {per.mean() * 1e3:.1f} us")


# The kernels one step of each HBM-bound part launches, as the rocprof summary
# names them: a part's roofline.traffic is the measured HBM bytes per step when
# every one of its kernels was in the FETCH_SIZE / WRITE_SIZE passes.
PART_KERNELS = {
    "copy_reference": ["clove_chain_flatten_b0"],
    "chain_broadcast": ["clove_chain_mul_add_gelu_mul_b0020"],
    "softmax": ["softmax_block_kernel<2>"],
    "layer_norm": ["layer_norm_wave_kernel<16>"],
    "matmul_skinny_32": ["gemm_skinny_kernel<1, 4, 4, 8>", "gemm_splitk_reduce"],
    "paged_decode": ["paged_heads_kernel<128, 16, 4>", "paged_merge_kernel"],
    "paged_decode_d96": ["paged_general_kernel<8, 3, true, 1>", "paged_merge_kernel"],
    "softmax_backward": ["softmax_bw_block_kernel<2>"],
    "gelu_backward": ["clove_chain_gelugrad_b00"],
    "broadcast_grad": ["bcast_grad_cols4_kernel", "bcast_grad_final_kernel"],
    "cross_entropy": ["cross_entropy_rows2_kernel<2>", "ordered_sum_kernel"],
    "cross_entropy_backward": ["cross_entropy_block_kernel<2, 1>"],
    "mse": ["sq_diff_partial_kernel<true>", "ordered_sum_kernel"],
    "mse_backward": ["mse_backward_kernel<true>"],
    "rope": ["rope_rows_kernel<true>"],
    # the 4096x4096 parameter's launches (the MLP's small ones run the same
    # kernel at a smaller grid and are summarised apart)
    "adamw_4096x4096": ["adamw_kernel (4096x4096)"],
}


def add_part_traffic(out, path):
    if not path or not os.path.exists(path):
        return
    with open(path) as f:
        kernels = json.load(f).get("kernels", {})
    for name, part in out.items():
        names = PART_KERNELS.get(name)
        roof = part.get("roofline")
        if not names or not roof or roof.get("bound") != "hbm":
            continue
        if all(k in kernels for k in names):
            roof["traffic"] = int(sum(kernels[k]["bytes_per_launch"] for k in names))


# ---------------------------------------------------------------------------

def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--parts", default="all",
                    help="comma list of copy,bcast,rows,matmul,paged,mlp,backward,attention "
                         "(skinny: only matmul's 32x4096x4096 product) or "
                         "'all' / "
                         "'none' "
                         "(the config 2 chain always runs)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--sets", type=int, default=3,
                    help="identical copies of each HBM-bound part's inputs that consecutive "
                         "steps cycle through, so that no step finds its inputs in the 256 MB "
                         "last-level cache (MALL) from the step before")
    ap.add_argument("--in-mib", type=int, default=512,
                    help="least MiB of inputs each HBM-bound part's input copies cover "
                         "(more copies than --sets where a copy is small), so that the "
                         "MALL cannot hold all of them")
    ap.add_argument("--out-mib", type=int, default=512,
                    help="MiB of outputs kept alive across consecutive steps, so that steps "
                         "write different blocks and the MALL cannot absorb rewrites of one "
                         "(0: every step reuses one output block)")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "hbm_traffic.json"),
                    help="JSON summary of the rocprof FETCH_SIZE/WRITE_SIZE passes "
                         "(bytes per launch of the chain kernel)")
    args = ap.parse_args()

    if args.sets < 1:
        ap.error("--sets must be at least 1")
    if args.out_mib < 0:
        ap.error("--out-mib must be at least 0")
    if args.in_mib < 0:
        ap.error("--in-mib must be at least 0")
    global OUT_HOLD_BYTES, IN_ROT_BYTES
    OUT_HOLD_BYTES = args.out_mib << 20
    IN_ROT_BYTES = args.in_mib << 20
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this backend runs on one GPU; multi-GPU runs are not part of this "
              "build (the decode path would shard by sequence and head, the rest by rows)",
              file=sys.stderr)
        sys.exit(2)

    import clove_amd as ca

    ca.init(0)
    parts = {"copy", "bcast", "rows", "matmul", "paged", "mlp", "backward", "attention"} \
        if args.parts == "all" else \
        set() if args.parts == "none" else set(args.parts.split(","))
    oracle = None
    if not args.no_cpu:
        import oracle as oracle_mod
        oracle = oracle_mod

    # --- the headline step: config 2 chain ---
    ins, nbytes, wall, per = bench_chain(ca, args)
    kernel_ms = float(per.mean())
    value = nbytes / (wall * 1e-3) / 1e9
    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    traffic = None
    if args.traffic and os.path.exists(args.traffic):
        with open(args.traffic) as f:
            traffic = json.load(f).get("bytes_per_launch")
    log(f"chain gelu(a*b+c)*d: {value:.0f} GB/s wall, kernel {kernel_ms * 1e3:.1f} us -> "
        f"{achieved:.0f} GB/s ({achieved / HBM_PEAK_GBS:.1%} of peak)")
    result = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (splitmix64 normal(0,1) streams, seeds 1-4)",
        "config": {"workload": "config 2: fused chain y = gelu(a*b+c)*d, 4 x [4096,4096] f32",
                   "elements": 4096 * 4096, "bytes_per_step": nbytes,
                   "input_sets": input_sets(args, 4 * 4 * 4096 * 4096),
                   "input_rotation_min_mib": args.in_mib, "output_hold_mib": args.out_mib},
        "roofline": roofline("hbm", achieved, HBM_PEAK_GBS, "GB/s", traffic),
    }
    if oracle is not None:
        def leg():
            host = [ins[i].numpy() for i in range(4)]
            want = []
            t = cpu_time(cpu_chain(oracle, host), keep=want)
            result["cpu_baseline"] = cpu_record(oracle, round(nbytes / t / 1e9, 2), "GB/s",
                                                "full config 2 workload, 4 unfused passes "
                                                "(Clove's eager CPU path), median of 3")
            check_parity("chain", ca.FusedChain(CHAIN, ins)()[0].numpy(), want[0], 1e-5, 1e-6)
        defer(leg)

    out = {}
    if "copy" in parts:
        # A plain copy through the same chain kernel (one Flatten op): the
        # practical streaming ceiling of this box, and the known-size kernel
        # that calibrates the HBM byte counters.
        srcs = [ca.empty((4096, 4096)).fill_normal(9)
                for _ in range(input_sets(args, 4 * 4096 * 4096))]
        cwall, cper = timed(ca, rotating([ca.FusedChain([("flatten", -1)], [src])
                                          for src in srcs]), args.steps, args.warmup)
        src = srcs[0]
        del srcs
        cbytes = 2 * 4 * 4096 * 4096
        gbs = cbytes / (cper.mean() * 1e-3) / 1e9
        out["copy_reference"] = {"value": round(gbs, 1), "unit": "GB/s", "ms": round(cper.mean(), 4),
                                 "bytes": cbytes,
                                 "roofline": roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s")}
        log(f"copy reference: {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%})")
        del src
    if "bcast" in parts:
        bins, bbytes, bwall, bper = bench_chain(ca, args, broadcast=True)
        gbs = bbytes / (bper.mean() * 1e-3) / 1e9
        out["chain_broadcast"] = {"value": round(gbs, 1), "unit": "GB/s",
                                  "ms": round(bper.mean(), 4), "bytes": bbytes,
                                  "roofline": roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s")}
        log(f"chain broadcast: {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%})")
        if oracle is not None:
            def bleg(bins=bins, part=out["chain_broadcast"], bbytes=bbytes):
                host = [bins[i].numpy() for i in range(4)]
                want = []
                t = cpu_time(cpu_chain(oracle, host), keep=want)
                part["cpu_baseline"] = cpu_record(oracle, round(bbytes / t / 1e9, 2), "GB/s",
                                                  "full broadcast workload, 4 unfused passes, "
                                                  "median of 3")
                check_parity("chain_broadcast", ca.FusedChain(CHAIN, bins)()[0].numpy(), want[0],
                             1e-5, 1e-6)
            defer(bleg)
        del bins
    if "rows" in parts:
        bench_rows(ca, oracle, args, out)
    if "matmul" in parts:
        bench_matmul(ca, oracle, args, out)
    elif "skinny" in parts:
        bench_matmul(ca, None, args, out, skinny_only=True)
    if "paged" in parts:
        bench_paged(ca, oracle, args, out)
    if "mlp" in parts:
        bench_mlp(ca, oracle, args, out)
    if "backward" in parts:
        bench_backward(ca, oracle, args, out)
    if "attention" in parts:
        bench_attention(ca, oracle, args, out)
    ca.synchronize()
    for leg in CPU_LEGS:
        leg()
    CPU_LEGS.clear()
    if out:
        add_part_traffic(out, args.traffic)
        result["parts"] = out
    ca.synchronize()
    failed = sorted(k for k, v in PARITY.items() if v != "ok")
    if oracle is None:
        result["parity_checked"] = False
    elif failed:
        result["parity_checked"] = {"failed": {k: PARITY[k] for k in failed},
                                    "passed": sorted(k for k in PARITY if k not in failed)}
    else:
        result["parity_checked"] = True
        result["parity_parts"] = sorted(PARITY)
    print(json.dumps(result), flush=True)
    if failed:
        log("bench.py: outputs out of their parity bound: " + ", ".join(failed))
        sys.exit(1)


if __name__ == "__main__":
    main()
