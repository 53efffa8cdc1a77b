"""Benchmark of the gfx950 INT4 quantized-matmul + Omni INT4 MoE hot path.

Metric: INT4 GEMM TOPS (% of the int8 MFMA peak) + MoE-layer tokens/s at
M=4096 on one MI355X.

  value        TOPS of the INT4 GEMM M=4096 K=4096 N=12288 (the gate projection
               of the 4096-token INT4-MLP block), prepacked operands resident in
               HBM, timed over --steps launches. TOPS = 2*M*N*K / time. The
               INT4 codes run as bf6 (e3m2 holds every code -8..7 exactly) on
               the fp6 MFMA; the output equals the INT4-operand GEMM's bit for
               bit (checked in the run), which is reported beside it
               (int4_operand_gemm).
  rotating_weights  the same projection in both forms with the weight cycled
               through copies that exceed the 256 MB last-level cache (INT4 14
               x 25 MB, bf6 10 x 38 MB), each with its own output, so every
               call streams its weight from HBM.
  moe_*        Omni INT4 MoE layer, 4096 tokens, hidden 2048, 128 experts,
               top-8, expert intermediate 768: route -> group -> expert GEMMs
               -> SwiGLU -> combine, timed over --steps layer calls.
  mlp_*        INT4-MLP dense block, 4096 x 4096 input, gate|up 24576 x 4096,
               down 4096 x 12288: quantize -> gate|up GEMM with SwiGLU in its
               epilogue -> quantize -> GEMM (bf6 form of the codes, checked
               against the INT4 block).
  int8_gemm_*  the INT8 x INT8 projection at the GEMM's shape.
  small_m_*    M = 1, 16, 64 on the GEMM's weight (K4096 N12288): GPU time per
               call (HIP graph replay) and HBM GB/s of the bytes the call moves,
               cycling through more weight copies than the last-level cache
               holds; us_cached repeats one weight (cache-resident).
  linear_m512_k2048_n2048  the single INT4 linear M512 K2048 N2048: GPU time
               per call (graph replay), TOPS and HBM GB/s.
  attn_proj_*  INT4 attention projections at M=16384 (Q, K, V, O + residual)
               on a prepared activation (bf6 form, checked against INT4).
  moe_skewed_t65536  the MoE layer at 65536 tokens with skewed routing (a few
               experts take most rows, eight none).
  moe_small_t  the MoE layer at 1, 16 and 256 tokens: GPU time per layer by
               graph replay (weights from HBM, and cache-resident), and the
               HBM rate of the skinny expert GEMMs over the routed experts'
               codes.
  roofline     the GEMM kernel against the peak of the MFMA it runs on (fp6
               dense, 10.1 POP/s); pct_int8_peak is the metric's own ratio.
  cpu_baseline the CPU oracle (quantize + i32 matmul + epilogue; MoE layer) on
               a bounded sample, timed on this host's cores.

Inputs are synthetic: X ~ N(0,1) bf16, weights ~ N(0,0.02) bf16 packed by the
library's own quantizer, router logits ~ N(0,1) bf16, all seeded.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "clef-hrx_amd"))
sys.path.insert(0, ROOT)

INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POP/s
FP6_PEAK_TOPS = 10100.0  # MI355X dense fp6 / fp4 MFMA, 10.1 PFLOP/s
HBM_PEAK_GBS = 8000.0
# HBM bytes moved per launch of the M4096 K4096 N12288 bf6 GEMM kernel:
# rocprofv3 FETCH_SIZE and WRITE_SIZE passes over `bench.py --only gemm`, each
# scaled by the reading for a plain 512 MiB copy (x2.000 fetch, x1.000 write);
# the runs and raw readings are in profiles/int4_gemm_m4096_k4096_n12288.txt.
GEMM_TRAFFIC_BYTES = 332.66e6
# HBM bytes moved per MoE layer call at 4096 tokens: the same two counter
# passes over `bench.py --only moe`, summed over the layer's eight kernels
# (read 628.1 MB + written 235.3 MB; per kernel in
# profiles/omni_int4_moe_t4096.txt).
MOE_TRAFFIC_BYTES = 863.4e6


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    # The board's power management settles within ~0.1 s of sustained MFMA
    # load (the first ~100 launches run up to 25 % slower); the default warmup
    # runs well past that so the timed steps measure the sustained rate.
    p.add_argument("--steps", type=int, default=400)
    p.add_argument("--warmup", type=int, default=600)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--moe-tokens", type=int, default=4096,
                   help="tokens of the MoE leg (4096 is the benchmark workload; small counts show the "
                        "decode-sized path)")
    p.add_argument("--only", choices=["gemm", "moe", "moe65536", "moesmall", "mlp", "attn", "i8", "smallm", "copy",
                                      "peaks"],
                   default=None,
                   help="run one leg; 'copy' is a plain 512 MiB device copy, the known-size "
                        "kernel that scales HBM byte counters")
    return p.parse_args()


def device_warmup(seconds=0.25):
    """Brings the board to its sustained clock before the first leg: an idle
    MI355X needs ~0.1 s of MFMA load before its power management settles (the
    first ~100 GEMM launches run up to 25 % slower), which a leg's own few
    warmup calls do not cover. Runs the library's INT4 GEMM, untimed; every
    leg still does its --warmup calls and times exactly --steps calls."""
    import torch

    import clef_i4

    x = bf16_randn((4096, 4096), 1.0, 7)
    w = clef_i4.load_quantized_weight(bf16_randn((4096, 4096), 0.02, 8))
    a = clef_i4.prepare(x)
    out = torch.empty((4096, 4096), dtype=torch.bfloat16, device="cuda")
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            clef_i4.project_prepared(a, w, out=out)
        torch.cuda.synchronize()


def timed(fn, steps, warmup):
    """Average ms per call of fn over `steps` calls on the current stream."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def bf16_randn(shape, std, seed):
    import torch

    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda", dtype=torch.float32) * std).to(torch.bfloat16)


def gemm_leg(args):
    """The INT4 projection M4096 K4096 N12288 two ways, both on the same
    quantized operands: the bf6 GEMM (codes re-encoded as e3m2, exact; weight
    re-encoded once at load, activation quantized straight into bf6) -- the
    headline -- and the GEMM on the reference's packed INT4 operands. The two
    outputs must be identical bit for bit."""
    import torch

    import clef_i4

    m, k, n = 4096, 4096, 12288
    x = bf16_randn((m, k), 1.0, 1002 * 16 + 0)
    w = bf16_randn((n, k), 0.02, 1002 * 16 + 1)
    qw = clef_i4.load_quantized_weight(w)
    fw = clef_i4.f6_weight(qw)
    a = clef_i4.prepare(x)
    af = clef_i4.prepare_f6(x)

    out = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    out_i4 = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    i4_ms = timed(lambda: clef_i4.project_prepared(a, qw, out=out_i4), args.steps, args.warmup)
    i4_prep_ms = timed(lambda: clef_i4.prepare(x, out=a.storage), args.steps, args.warmup)
    prep_ms = timed(lambda: clef_i4.prepare_f6(x, out=af.storage), args.steps, args.warmup)
    ms = timed(lambda: clef_i4.project_f6(af, fw, out=out), args.steps, args.warmup)
    torch.cuda.synchronize()
    if not torch.equal(out.view(torch.int16), out_i4.view(torch.int16)):
        raise SystemExit("bf6 GEMM output differs from the INT4 GEMM's")
    ops = 2.0 * m * n * k
    # operands read once (codes + f32 scales) and the bf16 output written once
    nbytes = m * k * 3 // 4 + 4 * m + n * k * 3 // 4 + 4 * n + 2 * m * n
    i4_bytes = m * k // 2 + 4 * m + n * k // 2 + 4 * n + 2 * m * n
    rot = rotating_gemm(args, a, af, qw, fw, out_i4, out)
    return {"m": m, "n": n, "k": k, "ms": ms, "tops": ops / ms / 1e9, "prepare_ms": prep_ms,
            "ops": ops, "bytes": nbytes, "rotating": rot,
            "int4": {"ms": i4_ms, "tops": ops / i4_ms / 1e9, "prepare_ms": i4_prep_ms, "bytes": i4_bytes}}


def rotating_gemm(args, a, af, qw, fw, out_i4, out_f6):
    """The headline projection with its weight cycled through copies that
    together exceed the 256 MB last-level cache (as the reference's paired
    integer benchmark keeps rotating weight copies, src/benchmarking.rs:318-381),
    each copy with its own output: every call then streams its weight from
    HBM instead of the cache that holds a repeated one. Both weight forms, each
    copy's output checked against the resident run's."""
    import torch

    import clef_i4

    ops = 2.0 * a.rows * qw.rows * qw.cols
    res = {}
    for form, copies, make, run, want in (
            ("int4", 14, lambda: clef_i4.QuantizedWeight(qw.codes.clone(), qw.scales.clone(), qw.rows, qw.cols,
                                                         qw.stride, qw.bits),
             lambda w, o: clef_i4.project_prepared(a, w, out=o), out_i4),
            ("bf6", 10, lambda: clef_i4.F6Weight(fw.codes.clone(), fw.scales.clone(), fw.rows, fw.cols),
             lambda w, o: clef_i4.project_f6(af, w, out=o), out_f6)):
        ws = [make() for _ in range(copies)]
        outs = [torch.empty_like(want) for _ in range(copies)]
        turn = [0]

        def call():
            i = turn[0] = (turn[0] + 1) % copies
            run(ws[i], outs[i])

        # whole rounds of the copies, at least as many calls as the resident timing
        steps = max(copies, (args.steps + copies - 1) // copies * copies)
        ms = timed(call, steps, max(copies, args.warmup // copies * copies))
        torch.cuda.synchronize()
        for o in outs:
            if not torch.equal(o.view(torch.int16), want.view(torch.int16)):
                raise SystemExit(f"rotating {form} GEMM output differs from the resident run's")
        res[form] = {"ms": ms, "tops": ops / ms / 1e9, "copies": copies,
                     "weight_mb_cycled": round(copies * (ws[0].codes.numel() * ws[0].codes.element_size()
                                                         + 4 * qw.rows) / 1e6, 1)}
        del ws, outs
        torch.cuda.empty_cache()
    return res


def graph_timed(fn, calls=50, replays=8):
    """GPU-side ms per call of fn: `calls` calls captured in one HIP graph,
    replayed `replays` times. For kernels of a few microseconds, where the
    host's per-call launch cost would otherwise be what is measured."""
    import torch

    for _ in range(20):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (calls * replays)


def small_m_leg(args):
    """Decode-sized projections on the headline weight (K4096 N12288): the
    weight stream is the whole cost, so the figure of merit is HBM GB/s
    (weight codes and scales, activation, output). Two figures per M: `us`
    cycles the calls through 14 copies of the weight (352 MB, more than the
    256 MB last-level cache, as a multi-layer decode does), so every call
    streams its weight from HBM; `us_cached` repeats one weight, which then
    stays in the last-level cache."""
    import torch

    import clef_i4

    k, n = 4096, 12288
    w = bf16_randn((n, k), 0.02, 1002 * 16 + 1)
    qws = [clef_i4.load_quantized_weight(w) for _ in range(14)]
    del w
    res = {}
    for m in (1, 16, 64):
        a = clef_i4.prepare(bf16_randn((m, k), 1.0, 1002 * 16 + 0))
        out = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        turn = [0]

        def rotating():
            turn[0] = (turn[0] + 1) % len(qws)
            clef_i4.project_prepared(a, qws[turn[0]], out=out)

        ms = graph_timed(rotating, calls=56)
        ms_cached = graph_timed(lambda: clef_i4.project_prepared(a, qws[0], out=out))
        nbytes = n * k // 2 + 4 * n + m * (k // 2 + 4) + 2 * m * n
        res[m] = {"us": ms * 1e3, "gbs": nbytes / ms / 1e6, "us_cached": ms_cached * 1e3}
    return res


def moe_skewed_leg(args):
    """Omni INT4 MoE layer at 65536 tokens with skewed routing: router logits
    N(0,1) + bias_e, bias_e = -1.1 * 0.57 * ln(1 + rank(e)) for a seeded rank
    permutation (seed 55), the eight lowest-ranked experts at -30 (never
    chosen)."""
    import numpy as np
    import torch

    import clef_i4

    t, d, inter = 65536, 2048, 768
    rank = np.random.default_rng(55).permutation(128)
    bias = -1.1 * 0.57 * np.log1p(rank)
    bias[rank >= 120] = -30.0
    g = torch.Generator(device="cuda").manual_seed(1005 * 16 + 1)
    z = torch.randn((t, 128), generator=g, device="cuda", dtype=torch.float32)
    logits = (z + torch.from_numpy(bias.astype(np.float32)).cuda()).to(torch.bfloat16)
    x = bf16_randn((t, d), 1.0, 1005 * 16 + 0)
    gate = clef_i4.load_quantized_weight(bf16_randn((128 * inter, d), 0.02, 1005 * 16 + 2))
    up = clef_i4.load_quantized_weight(bf16_randn((128 * inter, d), 0.02, 1005 * 16 + 3))
    down = clef_i4.load_quantized_weight(bf16_randn((128 * d, inter), 0.02, 1005 * 16 + 4))
    layer = clef_i4.MoeLayer(gate, up, down)
    out = torch.empty((t, d), dtype=torch.bfloat16, device="cuda")
    ms = timed(lambda: layer(x, logits, out=out), args.steps, max(1, args.warmup // 20))
    ops = 8.0 * t * 2 * (2 * inter * d + d * inter)
    return {"tokens": t, "ms": ms, "tokens_per_s": t / ms * 1e3, "tops": ops / ms / 1e9}


def linear_c1_leg(args):
    """Single INT4 linear M512 K2048 N2048 (the reference's CPU-path shape):
    latency-bound, so GPU time per call by graph replay, with TOPS and the HBM
    rate of the bytes the call moves."""
    import torch

    import clef_i4

    m, k, n = 512, 2048, 2048
    qw = clef_i4.load_quantized_weight(bf16_randn((n, k), 0.02, 1001 * 16 + 1))
    a = clef_i4.prepare(bf16_randn((m, k), 1.0, 1001 * 16 + 0))
    out = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    ms = graph_timed(lambda: clef_i4.project_prepared(a, qw, out=out))
    nbytes = n * k // 2 + 4 * n + m * (k // 2 + 4) + 2 * m * n
    return {"us": ms * 1e3, "tops": 2.0 * m * n * k / ms / 1e9, "gbs": nbytes / ms / 1e6}


def attention_leg(args):
    """INT4 attention projections at M=16384: Q 4096->4096, K and V 4096->1024
    on one shared quantized activation, and O 4096->4096 with the residual
    (fed the same activation here: its real input, the attention output, has
    the same shape). Run on the bf6 form of the codes (weights re-encoded
    once, the activation quantized straight into bf6); the outputs are
    checked against the INT4-operand projections bit for bit."""
    import torch

    import clef_i4

    m, d, kv = 16384, 4096, 1024
    x = bf16_randn((m, d), 1.0, 1003 * 16 + 0)
    ws = [clef_i4.load_quantized_weight(bf16_randn((n, d), 0.02, 1003 * 16 + 1 + i))
          for i, n in enumerate((d, kv, kv, d))]
    fws = [clef_i4.f6_weight(w) for w in ws]
    res = bf16_randn((m, d), 1.0, 1003 * 16 + 5)
    ax = clef_i4.prepare_f6(x)
    outs = [torch.empty((m, n), dtype=torch.bfloat16, device="cuda") for n in (d, kv, kv, d)]

    def step():
        for i in range(4):
            clef_i4.project_f6(ax, fws[i], residual=res if i == 3 else None, out=outs[i])

    ms = timed(step, args.steps, max(1, args.warmup // 4))
    a4 = clef_i4.prepare(x)
    for i in range(4):
        want = clef_i4.project_prepared(a4, ws[i], residual=res if i == 3 else None)
        if not torch.equal(want.view(torch.int16), outs[i].view(torch.int16)):
            raise SystemExit("bf6 attention projection differs from the INT4 one")
    ops = 2.0 * m * d * (d + kv + kv + d)
    return {"ms": ms, "tops": ops / ms / 1e9}


def i8_leg(args):
    """INT8 x INT8 projection at the headline shape (h3_gemm_i8_256 path)."""
    import torch

    import clef_i4

    m, k, n = 4096, 4096, 12288
    x = bf16_randn((m, k), 1.0, 1002 * 16 + 0)
    w = bf16_randn((n, k), 0.02, 1002 * 16 + 1)
    qw = clef_i4.load_quantized_weight(w, bits=8)
    a = clef_i4.prepare(x, bits=8)
    out = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    ms = timed(lambda: clef_i4.project_prepared(a, qw, out=out), args.steps, max(1, args.warmup // 4))
    return {"ms": ms, "tops": 2.0 * m * n * k / ms / 1e9}


def mlp_leg(args):
    """The INT4-MLP block M4096 D4096 F12288 on the bf6 form of the codes:
    Q1(x) -> gate and up projections with SwiGLU in one GEMM (h written once)
    -> Q1(h) -> down projection, each quantizer writing bf6, the weights
    re-encoded once. The output is checked bit for bit against the same block
    on INT4 operands (separate gate, up and SwiGLU-fused Q1)."""
    import torch

    import clef_i4

    m, d, f = 4096, 4096, 12288
    x = bf16_randn((m, d), 1.0, 1002 * 16 + 0)
    wg = clef_i4.load_quantized_weight(bf16_randn((f, d), 0.02, 1002 * 16 + 2))
    wu = clef_i4.load_quantized_weight(bf16_randn((f, d), 0.02, 1002 * 16 + 3))
    wd = clef_i4.load_quantized_weight(bf16_randn((d, f), 0.02, 1002 * 16 + 4))
    fg, fu, fd = clef_i4.f6_weight(wg), clef_i4.f6_weight(wu), clef_i4.f6_weight(wd)
    hb = torch.empty((m, f), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((m, d), dtype=torch.bfloat16, device="cuda")
    a = clef_i4.prepare_f6(x)
    h = clef_i4.prepare_f6(hb)

    def block():
        clef_i4.prepare_f6(x, out=a.storage)
        clef_i4.project_gate_up_f6(a, fg, fu, out=hb)
        clef_i4.prepare_f6(hb, out=h.storage)
        clef_i4.project_f6(h, fd, out=y)

    ms = timed(block, args.steps, max(1, args.warmup // 2))
    a4 = clef_i4.prepare(x)
    h4 = clef_i4.prepare_swiglu(clef_i4.project_prepared(a4, wg), clef_i4.project_prepared(a4, wu))
    if not torch.equal(clef_i4.project_prepared(h4, wd).view(torch.int16), y.view(torch.int16)):
        raise SystemExit("bf6 MLP block differs from the INT4 one")
    ops = 2.0 * m * (2 * f) * d + 2.0 * m * d * f
    return {"ms": ms, "tops": ops / ms / 1e9}


def moe_leg(args):
    import torch

    import clef_i4

    t, d, inter = args.moe_tokens, 2048, 768
    x = bf16_randn((t, d), 1.0, 1004 * 16 + 0)
    logits = bf16_randn((t, 128), 1.0, 1004 * 16 + 1)
    gate = clef_i4.load_quantized_weight(bf16_randn((128 * inter, d), 0.02, 1004 * 16 + 2))
    up = clef_i4.load_quantized_weight(bf16_randn((128 * inter, d), 0.02, 1004 * 16 + 3))
    down = clef_i4.load_quantized_weight(bf16_randn((128 * d, inter), 0.02, 1004 * 16 + 4))
    layer = clef_i4.MoeLayer(gate, up, down)
    out = torch.empty((t, d), dtype=torch.bfloat16, device="cuda")
    ms = timed(lambda: layer(x, logits, out=out), args.steps, args.warmup)
    ops = 8.0 * t * 2 * (2 * inter * d + d * inter)
    # Minimum HBM bytes: the codes and scales of every expert with a route (all
    # 128 at 4096 tokens), x and the logits read once, the output written once.
    nbytes = 128 * (3 * inter * d // 2 + 4 * (2 * inter + d)) + t * (2 * d + 2 * 128) + 2 * t * d
    return {"tokens": t, "ms": ms, "tokens_per_s": t / ms * 1e3, "tops": ops / ms / 1e9, "ops": ops,
            "bytes": nbytes}


def moe_small_leg(args):
    """The Omni MoE layer at decode-sized token counts (1, 16 and 256 tokens;
    hidden 2048, 128 experts, top-8, intermediate 768): GPU time per layer by
    HIP graph replay, and the HBM rate of the two expert GEMMs alone (the
    skinny 32-slot kernels; each call also runs its small tile-schedule
    kernel), over the codes and scales of the experts the tokens route to.
    `us` and the GEMM figures cycle through 14 copies of the layer's packed
    weights, so each call reads its experts from HBM as a multi-layer decode
    does; `us_cached` repeats one copy (the touched experts stay in the
    last-level cache)."""
    import ctypes

    import torch

    import clef_i4

    d, inter, copies = 2048, 768, 14
    base = [clef_i4.load_quantized_weight(bf16_randn((128 * inter, d), 0.02, 1004 * 16 + 2)),
            clef_i4.load_quantized_weight(bf16_randn((128 * inter, d), 0.02, 1004 * 16 + 3)),
            clef_i4.load_quantized_weight(bf16_randn((128 * d, inter), 0.02, 1004 * 16 + 4))]
    layers = [[clef_i4.QuantizedWeight(w.codes.clone(), w.scales.clone(), w.rows, w.cols, w.stride, w.bits)
               for w in base] for _ in range(copies)]
    lib = clef_i4.lib()
    P = ctypes.c_void_p
    res = {}
    for t in (1, 16, 256):
        x = bf16_randn((t, d), 1.0, 1004 * 16 + 0)
        logits = bf16_randn((t, 128), 1.0, 1004 * 16 + 1)
        out = torch.empty((t, d), dtype=torch.bfloat16, device="cuda")
        mods = [clef_i4.MoeLayer(*ws) for ws in layers]
        turn = [0]

        def layer_rotating():
            i = turn[0] = (turn[0] + 1) % copies
            mods[i](x, logits, out=out)

        us = graph_timed(layer_rotating, calls=56) * 1e3
        us_cached = graph_timed(lambda: mods[0](x, logits, out=out)) * 1e3

        # the expert GEMMs alone on this call's routing, through the C ABI
        routes = clef_i4.omni_route(logits, 8)
        groups, _ = clef_i4.omni_group_routes(routes)
        active = int((groups[:, 0] > 0).sum().item())
        ax = clef_i4.prepare(x)
        h = clef_i4.omni_gate_up(ax, base[0], base[1], groups, t, 8)
        ah = clef_i4.prepare(h)
        v = torch.empty((t * 8, d), dtype=torch.bfloat16, device="cuda")
        wsb = int(lib.clef_moe_expert_workspace_bytes(t, 8))
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")

        def gate_up():
            i = turn[0] = (turn[0] + 1) % copies
            g, u = layers[i][0], layers[i][1]
            clef_i4._check(lib.clef_moe_expert_gate_up_i4(
                P(ax.storage.data_ptr()), ax.stride, P(ax.scales.data_ptr()), P(g.codes.data_ptr()),
                P(g.scales.data_ptr()), P(u.codes.data_ptr()), P(u.scales.data_ptr()), P(groups.data_ptr()), t, 8, d,
                inter, P(h.data_ptr()), P(ws.data_ptr()), wsb, P(torch.cuda.current_stream().cuda_stream)))

        def down():
            i = turn[0] = (turn[0] + 1) % copies
            w = layers[i][2]
            clef_i4._check(lib.clef_moe_expert_i4(
                P(ah.storage.data_ptr()), ah.stride, P(ah.scales.data_ptr()), P(w.codes.data_ptr()),
                P(w.scales.data_ptr()), P(groups.data_ptr()), t, 8, inter, d, 1, P(v.data_ptr()), P(ws.data_ptr()),
                wsb, P(torch.cuda.current_stream().cuda_stream)))

        gu_us = graph_timed(gate_up, calls=56) * 1e3
        dn_us = graph_timed(down, calls=56) * 1e3
        gu_bytes = active * (2 * inter * d // 2 + 2 * 4 * inter)  # gate and up codes + scales
        dn_bytes = active * (d * inter // 2 + 4 * d)
        res[t] = {"us": us, "us_cached": us_cached, "tokens_per_s": t / us * 1e6, "active_experts": active,
                  "gate_up_us": gu_us, "gate_up_hbm_gbs": gu_bytes / gu_us / 1e3,
                  "down_us": dn_us, "down_hbm_gbs": dn_bytes / dn_us / 1e3}
        del mods
    return res


def copy_leg(args):
    """Plain device-to-device copy of 512 MiB: read and written bytes are known
    exactly, so a counter run over it gives the factor between the FETCH_SIZE /
    WRITE_SIZE readings and bytes."""
    import torch

    nbytes = 512 << 20
    src = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    ms = timed(lambda: dst.copy_(src), args.steps, args.warmup)
    return {"bytes": nbytes, "ms": ms, "gbs": 2 * nbytes / ms / 1e6}


def cpu_leg():
    """The oracle on the GEMM and MoE workloads, timed on this host's cores.

    Timing does not depend on the weight values, so weights are random packed
    codes with unit scales; activations are N(0,1) bf16 quantized inside the
    timed region (the reference's CPU path is quantize -> i32 dot -> scale).
    """
    import numpy as np

    import oracle

    rng = np.random.default_rng(1002)
    threads = oracle.threads()

    def codes(words):
        return rng.integers(0, 1 << 32, size=words, dtype=np.uint64).astype(np.uint32)

    m, n, k = 4096, 12288, 4096
    x = oracle.f32_to_bf16(rng.standard_normal((m, k)).astype(np.float32))
    w_tiled, w_scales = codes(n * k // 8), np.full(n, 1e-3, dtype=np.float32)
    t0 = time.perf_counter()
    a_codes, a_scales, _ = oracle.prepare(x, oracle.activation_stride(k))
    oracle.gemm(a_codes, a_scales, w_tiled, w_scales, n, k)
    gemm_s = time.perf_counter() - t0

    # c1, the single linear M512 K2048 N2048 (quantize + GEMM), repeated so
    # the sample is long enough to time.
    m1, n1, k1, reps = 512, 2048, 2048, 20
    x1 = oracle.f32_to_bf16(rng.standard_normal((m1, k1)).astype(np.float32))
    w1 = codes(n1 * k1 // 8), np.full(n1, 1e-3, dtype=np.float32)
    t0 = time.perf_counter()
    for _ in range(reps):
        c1_codes, c1_scales, _ = oracle.prepare(x1, oracle.activation_stride(k1))
        oracle.gemm(c1_codes, c1_scales, w1[0], w1[1], n1, k1)
    c1_s = (time.perf_counter() - t0) / reps

    t, d, inter = 4096, 2048, 768
    xs = oracle.f32_to_bf16(rng.standard_normal((t, d)).astype(np.float32))
    lg = oracle.f32_to_bf16(rng.standard_normal((t, 128)).astype(np.float32))
    g = (codes(128 * inter * d // 8), np.full(128 * inter, 1e-3, dtype=np.float32))
    u = (codes(128 * inter * d // 8), np.full(128 * inter, 1e-3, dtype=np.float32))
    dn = (codes(128 * d * inter // 8), np.full(128 * d, 1e-3, dtype=np.float32))
    t0 = time.perf_counter()
    oracle.moe_layer(xs, lg, g, u, dn)
    moe_s = time.perf_counter() - t0
    return {
        "value": round(2.0 * m * n * k / gemm_s / 1e12, 4),
        "unit": "TOPS",
        "cores": threads,
        "kind": "port",
        "sample": f"full INT4 GEMM M{m} N{n} K{k} incl. activation quantize ({gemm_s:.2f} s); "
                  f"{reps} x the M{m1} K{k1} N{n1} linear incl. quantize ({c1_s * 1e3:.1f} ms each); "
                  f"full MoE layer T{t} D{d} I{inter} ({moe_s:.2f} s)",
        "c1_tops": round(2.0 * m1 * n1 * k1 / c1_s / 1e12, 4),
        "moe_tokens_per_s": round(t / moe_s, 1),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the multi-GPU "
              "sharding of this path is a design note, not a measured configuration.", file=sys.stderr)
        sys.exit(2)
    import torch

    import clef_i4

    clef_i4.lib()
    torch.cuda.init()
    if args.only not in ("copy", "peaks"):
        device_warmup()
    res = {}
    if args.only in (None, "mlp"):
        res["mlp"] = mlp_leg(args)
    if args.only in (None, "i8"):
        res["i8"] = i8_leg(args)
    if args.only in (None, "smallm"):
        res["smallm"] = small_m_leg(args)
        res["c1"] = linear_c1_leg(args)
    if args.only in (None, "attn"):
        res["attn"] = attention_leg(args)
    if args.only in (None, "moe65536"):
        res["moe65536"] = moe_skewed_leg(args)
    if args.only in (None, "moesmall"):
        res["moesmall"] = moe_small_leg(args)
    # The MoE layer and the headline GEMM run last: the other legs keep the
    # device busy before them, so their timed calls see the sustained clock of
    # a loaded device rather than the ramp of an idle one (the first ~100
    # calls on an idle board run up to 25 % slower).
    if args.only in (None, "moe"):
        res["moe"] = moe_leg(args)
    if args.only in (None, "gemm"):
        res["gemm"] = gemm_leg(args)
    if args.only == "peaks":
        import subprocess
        probe = os.path.join(ROOT, "clef-hrx_amd", "lib", "peaks")
        proc = subprocess.run([probe], check=True, capture_output=True, text=True)
        print(proc.stdout.strip())
        return
    if args.only == "copy":
        c = copy_leg(args)
        print(json.dumps({"copy_bytes": c["bytes"], "copy_ms": round(c["ms"], 4),
                          "copy_gbs": round(c["gbs"], 1)}))
        return
    cpu = None if args.no_cpu or args.only else cpu_leg()

    g = res.get("gemm")
    line = {
        "metric": "INT4 GEMM TOPS (% int8 MFMA peak) + MoE-layer tokens/s at M=4096, 1 MI355X",
        "value": round(g["tops"], 1) if g else None,
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms"], 4) if g else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 codes as bf6 (e3m2, exact) -> f32 (fp6 MFMA), bf16 out",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights, packed by the library)",
        "config": {"workload": "int4_gemm M4096 K4096 N12288 prepacked + omni_int4_moe T4096 "
                               "D2048 E128 top8 I768 + int4_mlp M4096 D4096 F12288",
                   "parallelism": "single GPU"},
    }
    if g:
        line["pct_int8_peak"] = round(100.0 * g["tops"] / INT8_PEAK_TOPS, 2)
        line["prepare_ms"] = round(g["prepare_ms"], 4)
        line["roofline"] = {"bound": "mfma", "achieved": round(g["tops"], 1), "peak": FP6_PEAK_TOPS,
                            "unit": "TOPS", "frac": round(g["tops"] / FP6_PEAK_TOPS, 4),
                            "mfma": "v_mfma_scale_f32_32x32x64_f8f6f4 (bf6 x bf6)",
                            "traffic": GEMM_TRAFFIC_BYTES,
                            "traffic_source": "profiles/int4_gemm_m4096_k4096_n12288.txt (FETCH_SIZE, WRITE_SIZE)",
                            "algorithmic_bytes": g["bytes"]}
        i4 = g["int4"]
        line["int4_operand_gemm"] = {"ms": round(i4["ms"], 4), "tops": round(i4["tops"], 1),
                                     "pct_int8_peak": round(100.0 * i4["tops"] / INT8_PEAK_TOPS, 2),
                                     "prepare_ms": round(i4["prepare_ms"], 4)}
        line["rotating_weights"] = {f: {"ms": round(v["ms"], 4), "tops": round(v["tops"], 1),
                                        "pct_int8_peak": round(100.0 * v["tops"] / INT8_PEAK_TOPS, 2),
                                        "copies": v["copies"], "weight_mb_cycled": v["weight_mb_cycled"]}
                                    for f, v in g["rotating"].items()}
    if "moe" in res:
        if res["moe"]["tokens"] != 4096:
            line["moe_tokens"] = res["moe"]["tokens"]
        line["moe_tokens_per_s"] = round(res["moe"]["tokens_per_s"], 1)
        line["moe_layer_ms"] = round(res["moe"]["ms"], 4)
        line["moe_tops"] = round(res["moe"]["tops"], 1)
        m = res["moe"]
        # The layer is MFMA-bound (3.09e11 ops at 5.0 POP/s = 61.8 us against
        # 0.34 GB at 8 TB/s = 42 us).
        line["moe_roofline"] = {"bound": "mfma", "achieved": round(m["tops"], 1), "peak": INT8_PEAK_TOPS,
                                "unit": "TOPS", "frac": round(m["tops"] / INT8_PEAK_TOPS, 4),
                                "roofline_us": round(max(m["ops"] / INT8_PEAK_TOPS / 1e6,
                                                         m["bytes"] / HBM_PEAK_GBS / 1e3), 1),
                                "hbm_gbs": round(m["bytes"] / m["ms"] / 1e6, 1),
                                "algorithmic_bytes": m["bytes"]}
        # The counter readings were taken at 4096 tokens; other token counts
        # carry no traffic figure here.
        if m["tokens"] == 4096:
            line["moe_roofline"].update({"traffic": MOE_TRAFFIC_BYTES,
                                         "traffic_source": "profiles/omni_int4_moe_t4096.txt (FETCH_SIZE, WRITE_SIZE)"})
        else:
            line["moe_roofline"]["traffic"] = None
    if "mlp" in res:
        line["mlp_block_ms"] = round(res["mlp"]["ms"], 4)
        line["mlp_tops"] = round(res["mlp"]["tops"], 1)
    if "i8" in res:
        line["int8_gemm_ms"] = round(res["i8"]["ms"], 4)
        line["int8_gemm_tops"] = round(res["i8"]["tops"], 1)
    if "c1" in res:
        line["linear_m512_k2048_n2048"] = {"us": round(res["c1"]["us"], 2), "tops": round(res["c1"]["tops"], 1),
                                           "hbm_gbs": round(res["c1"]["gbs"], 1)}
    if "moe65536" in res:
        line["moe_skewed_t65536"] = {"ms": round(res["moe65536"]["ms"], 3),
                                     "tokens_per_s": round(res["moe65536"]["tokens_per_s"], 1),
                                     "tops": round(res["moe65536"]["tops"], 1)}
    if "attn" in res:
        line["attn_proj_m16384_ms"] = round(res["attn"]["ms"], 4)
        line["attn_proj_tops"] = round(res["attn"]["tops"], 1)
    if "moesmall" in res:
        line["moe_small_t"] = {f"t{t}": {"us": round(v["us"], 2), "us_cached": round(v["us_cached"], 2),
                                         "tokens_per_s": round(v["tokens_per_s"], 1),
                                         "active_experts": v["active_experts"],
                                         "gate_up_us": round(v["gate_up_us"], 2),
                                         "gate_up_hbm_gbs": round(v["gate_up_hbm_gbs"], 1),
                                         "down_us": round(v["down_us"], 2),
                                         "down_hbm_gbs": round(v["down_hbm_gbs"], 1)}
                               for t, v in res["moesmall"].items()}
    if "smallm" in res:
        line["small_m_k4096_n12288"] = {f"m{m}": {"us": round(v["us"], 2), "hbm_gbs": round(v["gbs"], 1),
                                                  "us_cached": round(v["us_cached"], 2)}
                                        for m, v in res["smallm"].items()}
    if cpu:
        line["cpu_baseline"] = cpu
        if "moe" in res:
            line["moe_vs_cpu"] = round(res["moe"]["tokens_per_s"] / cpu["moe_tokens_per_s"], 1)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
