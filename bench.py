#!/usr/bin/env python3
"""Benchmark of the MI355X W8A8 linear-layer path (one GPU).

Headline (`value`): BASELINE configs[1] -- decode GEMV, M=1 token, g256, the
four linears of a Qwen3-4B-class DualAR layer (qkv K=2560 N=6144, o K=4096
N=2560, gate_up K=2560 N=19456, down K=9728 N=2560), each through the drop-in
entry point fa_w8a8_gemm (dynamic per-(token, group) activation quant + int8
GEMV + fp32 dequant-sum + fp16 out).  One step = those four linears for each
of 36 layers with distinct weights (3.6 GB), so weights stream from HBM and
not from the 256 MB last-level cache; the step is replayed from a HIP graph.
value = algorithmic bytes (int8 W + fp16 scales + fp16 x + fp16 y) / time.

Extra objects on the same JSON line: roofline of the dominant kernel (the
gate_up GEMV, timed with HIP events on its own stream), the CPU baseline (the
scalar C oracle with OpenMP on this host), and secondary figures for configs
[2] (M=8 g64), [3] (prefill M=512/2048 int8 TOPS) and [4] (36-layer decode
stack with fused prologues).
"""
import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "fish-audio-cpp_amd"))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
FP16_PEAK_TFLOPS = 2500.0   # dense fp16 MFMA
METRIC = "decode GEMV HBM GB/s + prefill INT8 TOPS (% of MI355X peak), g256/g64"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(stack, torch, budget_s):
    """configs[1] on the host: the C oracle (scalar C restatement of the
    reference's W8A8 math, OpenMP over output rows) for one layer's four
    linears at M=1 g256; median over repetitions within budget_s."""
    from oracle import ref
    from fish_amd.synth import LAYER_SHAPES
    march = ref.use_baseline_build()
    model = ref.host_cpu_id()
    lay = stack.layers[0]
    host = {}
    nbytes = 0
    for name, (K, N) in LAYER_SHAPES.items():
        L = lay[name]
        host[name] = (L.W.cpu().numpy(), L.scale.cpu().numpy(),
                      stack.x_in[name].cpu().numpy())
        nbytes += L.algo_bytes + 2 * (K + N)
    threads = ref.num_threads()

    def one():
        for name, (W, S, X) in host.items():
            ref.w8a8_gemm(W, S, stack.g, X)

    one()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "cpu_model": model, "build": "gcc -O3 -fopenmp -march=%s" % march,
            "sample": "one layer's 4 linears (qkv/o/gate_up/down) at M=1 g256, "
                      "%d reps, median %.2f ms" % (len(times), med * 1e3)}


def cpu_baseline_prefill(budget_s):
    """configs[3] on the host: the C oracle (the reference's W8A8 math:
    per-token, per-group activation quantization, int32 group partials,
    the group-ordered fp32 chain, fp16 out; OpenMP over output rows) for
    one layer's four linears at 512 and 2048 tokens, g256, the whole layer
    (no row sampling), on the same synthetic distributions as the GPU
    figures.  Reports int8 TOP/s (2*M*N*K per linear) for the median
    repetition; at least one repetition, more while budget_s lasts."""
    from oracle import ref
    from fish_amd import synth
    from fish_amd.synth import LAYER_SHAPES
    march = ref.use_baseline_build()
    g = 256
    wts = {name: ref.quantize_weights(synth.weights_f16(N, K, seed=31 + i), g)
           for i, (name, (K, N)) in enumerate(LAYER_SHAPES.items())}
    res = {"unit": "TOP/s", "cores": ref.num_threads(), "kind": "port",
           "cpu_model": ref.host_cpu_id(), "build": "gcc -O3 -fopenmp -march=%s" % march}
    for M in (512, 2048):
        xs = {name: synth.activations_f16(M, K, seed=M + i)
              for i, (name, (K, N)) in enumerate(LAYER_SHAPES.items())}
        ops_layer = sum(2.0 * M * N * K for K, N in LAYER_SHAPES.values())
        times = []
        t_end = time.perf_counter() + budget_s / 2
        while not times or (time.perf_counter() < t_end and len(times) < 5):
            t0 = time.perf_counter()
            for name, (q, sc) in wts.items():
                ref.w8a8_gemm(q, sc, g, xs[name])
            times.append(time.perf_counter() - t0)
        med = statistics.median(times)
        res["m%d_g256_layer_TOPS" % M] = round(ops_layer / med / 1e12, 4)
        res["m%d_g256_layer_ms" % M] = round(med * 1e3, 1)
        res["m%d_reps" % M] = len(times)
    res["value"] = res["m2048_g256_layer_TOPS"]
    res["sample"] = ("one layer's 4 linears (qkv/o/gate_up/down), full size, at 512 and "
                     "2048 tokens, g256, fa_w8a8_gemm semantics incl. activation "
                     "quantization; value = the 2048-token layer")
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--cpu-prefill-budget", type=float, default=20.0)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the gate_up GEMV event timing (for rocprofv3 runs)")
    ap.add_argument("--stack-only", action="store_true",
                    help="only the configs[4] four-launch stack, graph-replayed 13 times "
                         "(for rocprofv3 runs)")
    ap.add_argument("--chain-only", action="store_true",
                    help="only the experimental configs[4] decode chain, 20 runs (for rocprofv3 runs)")
    ap.add_argument("--attn-only", action="store_true",
                    help="only the T=2048 prefill attention side (for rocprofv3 runs)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the configs[3] g256 prefill GEMMs at --prefill-tokens "
                         "(for rocprofv3 runs)")
    ap.add_argument("--prefill-tokens", type=int, default=2048)
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(--gpus %d requested)" % args.gpus, file=sys.stderr)
        sys.exit(2)

    import torch
    from fish_amd import ops
    from fish_amd.decode_stack import DecodeStack
    from fish_amd.synth import LAYER_SHAPES

    torch.cuda.init()
    if args.attn_only:
        print(json.dumps(attention_side(torch, ops)), flush=True)
        return
    if args.prefill_only:
        print(json.dumps(prefill_tops(torch, ops, [(256, args.prefill_tokens)])), flush=True)
        return
    log("building 36-layer g256 weight set ...")
    st = DecodeStack(n_layers=args.layers, g=256, tokens=1, seed=0)
    torch.cuda.synchronize()

    if args.stack_only:
        st.h.copy_(st.h0)
        g_stack = st.capture(lambda: st.run_stack())
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(13):
            g_stack.replay()
        torch.cuda.synchronize()
        print(json.dumps({"stack_step_ms_mean": round((time.perf_counter() - t0) / 13 * 1e3, 4)}),
              flush=True)
        return

    if args.chain_only:
        st.build_chain()
        t = []
        for _ in range(20):
            t0 = time.perf_counter()
            st.run_chain(check=False)
            torch.cuda.synchronize()
            t.append(time.perf_counter() - t0)
        print(json.dumps({"chain_step_ms_median": round(statistics.median(t) * 1e3, 4),
                          "complete": st.chain.status() == 0}), flush=True)
        st.chain.close()
        return

    if args.roofline_only:
        # The gate_up GEMV, then a plain 64 MiB device copy whose known byte
        # count calibrates the FETCH_SIZE / WRITE_SIZE counters.
        r = roofline_gate_up(torch, ops, st, LAYER_SHAPES)
        del st
        torch.cuda.empty_cache()
        rp = roofline_prefill(torch, ops)
        a = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"roofline": r, "roofline_prefill": rp,
                          "calibration_copy_bytes": 64 << 20}), flush=True)
        return

    # ---- headline: configs[1] linears, graph-replayed --------------------
    graph = st.capture(lambda: st.run_linears())
    eager_y = {k: v.clone() for k, v in st.y.items()}
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    for k in st.y:   # graph replays reproduce the eager result
        assert torch.equal(st.y[k], eager_y[k]), k
    ms_per_step = dt / args.steps * 1e3
    step_bytes = st.linears_bytes()
    value = step_bytes / (dt / args.steps) / 1e9

    roofline = roofline_gate_up(torch, ops, st, LAYER_SHAPES)
    roofline_pf = None

    secondary = {}
    if not args.no_secondary:
        secondary = run_secondary(torch, ops, st, args)

    cpu = cpu_baseline(st, torch, args.cpu_budget)
    del st
    torch.cuda.empty_cache()
    roofline_pf = roofline_prefill(torch, ops)
    try:
        cpu_pf = cpu_baseline_prefill(args.cpu_prefill_budget)
    except Exception as e:   # noqa: BLE001 -- reported in the JSON line
        cpu_pf = {"error": "%s: %s" % (type(e).__name__, str(e)[:160])}

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "configs[1]: decode M=1 g256, qkv/o/gate_up/down via "
                               "fa_w8a8_gemm (quant + GEMV), 36 layers of distinct weights "
                               "per step, HIP-graph replay",
                   "tokens": 1, "group_size": 256, "layers_per_step": args.layers,
                   "bytes_per_step": step_bytes, "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4)},
        "roofline": roofline,
        "roofline_prefill": roofline_pf,
        "cpu_baseline": cpu,
        "cpu_baseline_prefill": cpu_pf,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)


def graph_us_per_call(torch, calls, reps=10, rounds=5):
    """Duration per call of `calls` (a list of closures launching one kernel
    each on torch's current stream), captured back to back in one HIP graph:
    after three warm-up replays, `rounds` rounds of `reps` replays are timed
    with events on that stream, and the median round is reported."""
    for c in calls:
        c()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in calls:
            c()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    per = []
    for _ in range(rounds):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            g.replay()
        e.record()
        e.synchronize()
        per.append(s.elapsed_time(e) * 1e3 / (reps * len(calls)))
    return statistics.median(per)


def _traffic(key):
    """HBM bytes per launch of `key` from the calibrated rocprofv3
    FETCH_SIZE / WRITE_SIZE runs committed under profiles/ (or None)."""
    tpath = os.path.join(REPO, "profiles", "traffic.json")
    if os.path.exists(tpath):
        rec = json.load(open(tpath)).get(key)
        if rec:
            return rec["bytes_per_launch"]
    return None


GATE_UP_QX_KEY = "gemv_dot_kernel QX gate_up K=2560 N=19456 m1 g256"
PREFILL_KEY = "gemm_tile_kernel gate_up K=2560 N=19456 M=2048 g256"


def roofline_gate_up(torch, ops, st, LAYER_SHAPES):
    """Dominant kernel of the headline: the gate_up linear exactly as the
    headline runs it -- fa_w8a8_gemm at one token, i.e. gemv_dot_kernel with
    in-kernel activation quantization (K=2560 N=19456, g256) -- one launch
    per layer's weights so every launch streams its 50 MB from HBM, timed
    with HIP events on the stream the launches go to (torch's current
    stream).  Algorithmic bytes per launch: int8 W + fp16 scales + fp16 x
    in + fp16 y out."""
    x = st.x_in["gate_up"]
    out = st.y["gate_up"]
    calls = [(lambda L=lay["gate_up"]: ops.w8a8_gemm(L.W, L.scale, x, 256, out=out))
             for lay in st.layers]
    us = graph_us_per_call(torch, calls)
    K, N = LAYER_SHAPES["gate_up"]
    kbytes = st.layers[0]["gate_up"].algo_bytes + 2 * (K + N)
    achieved = kbytes / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": _traffic(GATE_UP_QX_KEY),
            "kernel": "gemv_dot_kernel, in-kernel quantization (fa_w8a8_gemm: gate_up, "
                      "K=2560 N=19456, 1 token, g256)",
            "avg_launch_us": round(us, 3), "bytes_per_launch": kbytes}


def roofline_prefill(torch, ops):
    """Dominant kernel of the metric's prefill half: the gate_up GEMM at
    2048 tokens, g256, through fa_w8a8_gemm_quantized
    (gemm_tile_kernel; the call also runs the small scale-table launch,
    which the timing includes).  Algorithmic work per call: 2*M*N*K int8
    ops.  Random operands (the matrix units' clock depends on the data)."""
    from fish_amd.synth import LAYER_SHAPES
    K, N = LAYER_SHAPES["gate_up"]
    M, g = 2048, 256
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    w = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
    W, S = ops.quantize_weights_groupwise(w, g)
    del w
    x = torch.randn((M, K), generator=gen, device="cuda").half()
    xq, xs = ops.quantize_activations(x, g)
    y = torch.empty((M, N), device="cuda", dtype=torch.float16)
    us = graph_us_per_call(torch, [lambda: ops.w8a8_gemm_quantized(W, S, g, xq, xs, out=y)] * 8,
                           reps=5)
    o = 2.0 * M * N * K
    tops = o / (us * 1e-6) / 1e12
    return {"bound": "mfma", "achieved": round(tops, 1), "peak": INT8_PEAK_TOPS,
            "unit": "TOP/s", "frac": round(tops / INT8_PEAK_TOPS, 4),
            "traffic": _traffic(PREFILL_KEY),
            "kernel": "gemm_tile_kernel (gate_up, K=2560 N=19456, 2048 tokens, g256), "
                      "+ scale-table launch",
            "avg_launch_us": round(us, 3), "ops_per_launch": o}


def run_secondary(torch, ops, st, args):
    from fish_amd.decode_stack import DecodeStack
    from fish_amd.synth import LAYER_SHAPES
    out = {}
    # full decode-step linear stack with fused prologues (g256)
    st.h.copy_(st.h0)
    g_stack = st.capture(lambda: st.run_stack())
    for _ in range(2):
        g_stack.replay()
    torch.cuda.synchronize()
    reps = 10
    t0 = time.perf_counter()
    for _ in range(reps):
        g_stack.replay()
    torch.cuda.synchronize()
    t = (time.perf_counter() - t0) / reps
    out["cfg4_stack_g256_m1"] = {"step_ms": round(t * 1e3, 4),
                                 "GB/s": round(st.stack_bytes() / t / 1e9, 1)}
    # configs[4] with the calibrated (AWQ) layout a real dual_ar.bin carries:
    # wqkv / w1 / w3 with their own smooth_inv, w1 and w3 separate weights
    # (four launches per layer: w1 and w3 in one fa_w8a8_gemm_swiglu_sep)
    sa = DecodeStack(n_layers=args.layers, g=256, tokens=1, seed=7, awq=True)
    sa.h.copy_(sa.h0)
    g_awq = sa.capture(lambda: sa.run_stack_awq())
    for _ in range(2):
        g_awq.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        g_awq.replay()
    torch.cuda.synchronize()
    t = (time.perf_counter() - t0) / reps
    out["cfg4_awq_stack_g256_m1"] = {"step_ms": round(t * 1e3, 4),
                                     "GB/s": round(sa.awq_stack_bytes() / t / 1e9, 1)}
    # ... and as the reference's separate calls (w1, w3, silu_mul: five launches)
    sa.h.copy_(sa.h0)
    g_awq5 = sa.capture(lambda: sa.run_stack_awq_unfused())
    for _ in range(2):
        g_awq5.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        g_awq5.replay()
    torch.cuda.synchronize()
    t = (time.perf_counter() - t0) / reps
    out["cfg4_awq_stack_unfused_g256_m1"] = {"step_ms": round(t * 1e3, 4),
                                             "GB/s": round(sa.awq_stack_bytes() / t / 1e9, 1)}
    del sa, g_awq, g_awq5
    torch.cuda.empty_cache()
    # configs[2] as a whole decode step: 8 tokens, g64, the 36-layer stack
    # with every prologue (RMSNorm + quant, SiLU * mul) as the entry points
    # run it at more than one token
    s8 = DecodeStack(n_layers=args.layers, g=64, tokens=8, seed=13)
    s8.h.copy_(s8.h0)
    g_8 = s8.capture(lambda: s8.run_stack())
    for _ in range(2):
        g_8.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        g_8.replay()
    torch.cuda.synchronize()
    t = (time.perf_counter() - t0) / reps
    out["cfg2_stack_g64_m8"] = {"step_ms": round(t * 1e3, 4),
                                "GB/s": round(s8.stack_bytes() / t / 1e9, 1)}
    del s8, g_8
    torch.cuda.empty_cache()
    # configs[4] at g64 (4x the scale bytes)
    s64 = DecodeStack(n_layers=args.layers, g=64, tokens=1, seed=9)
    s64.h.copy_(s64.h0)
    g_64 = s64.capture(lambda: s64.run_stack())
    for _ in range(2):
        g_64.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        g_64.replay()
    torch.cuda.synchronize()
    t = (time.perf_counter() - t0) / reps
    out["cfg4_stack_g64_m1"] = {"step_ms": round(t * 1e3, 4),
                                "GB/s": round(s64.stack_bytes() / t / 1e9, 1)}
    del s64, g_64
    torch.cuda.empty_cache()
    # the fast (codebook) decoder: 4 layers + int8 head (4096 x 2560), 10
    # passes per frame over the same ~0.4 GB of weights
    from fish_amd.decode_stack import FastDecoder, NUM_CODEBOOKS
    fd = FastDecoder(g=256, seed=11)
    g_fd = fd.capture(lambda: fd.run_frame())
    for _ in range(2):
        g_fd.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        g_fd.replay()
    torch.cuda.synchronize()
    t = (time.perf_counter() - t0) / reps
    out["fast_decoder_frame_g256"] = {"frame_ms": round(t * 1e3, 4), "passes": NUM_CODEBOOKS,
                                      "GB/s": round(NUM_CODEBOOKS * fd.pass_bytes() / t / 1e9, 1)}
    del fd, g_fd
    torch.cuda.empty_cache()
    # configs[1] per-linear GEMV time (graph of one launch per layer, cold weights)
    for name, (K, N) in LAYER_SHAPES.items():
        xq, xs = ops.quantize_activations(st.x_in[name], 256)
        y = st.y[name]
        calls = [(lambda L=lay[name]: ops.w8a8_gemm_quantized(L.W, L.scale, 256, xq, xs, out=y))
                 for lay in st.layers]
        us = graph_us_per_call(torch, calls)
        b = st.layers[0][name].algo_bytes + 2 * (K + N)
        out["cfg1_gemv_%s_us" % name] = round(us, 2)
        out["cfg1_gemv_%s_GBs" % name] = round(b / (us * 1e-6) / 1e9, 1)
    del st
    torch.cuda.empty_cache()

    # the fp16 tied-embedding logits head (155776 x 2560, 0.8 GB), one token;
    # two weight copies alternate so each launch reads from HBM
    Wl = [(torch.randn(155776, 2560, device="cuda") * 0.02).half() for _ in range(2)]
    xl = torch.randn(1, 2560, device="cuda").half()
    yl = torch.empty(1, 155776, device="cuda", dtype=torch.float16)
    us = graph_us_per_call(torch, [(lambda W=W: ops.gemm_fp16(W, xl, out=yl)) for W in Wl] * 4,
                           reps=5)
    lb = 155776 * 2560 * 2 + 2 * (2560 + 155776)
    out["logits_fp16_m1_us"] = round(us, 2)
    out["logits_fp16_m1_GBs"] = round(lb / (us * 1e-6) / 1e9, 1)
    del Wl
    torch.cuda.empty_cache()

    # M=8, g64 (smaller layer count keeps the bench short)
    st8 = DecodeStack(n_layers=12, g=64, tokens=8, seed=1)
    for name, (K, N) in LAYER_SHAPES.items():
        xq, xs = ops.quantize_activations(st8.x_in[name], 64)
        y = st8.y[name]
        calls = [(lambda L=lay[name]: ops.w8a8_gemm_quantized(L.W, L.scale, 64, xq, xs, out=y))
                 for lay in st8.layers]
        us = graph_us_per_call(torch, calls)
        b = st8.layers[0][name].algo_bytes + 2 * 8 * (K + N)
        out["cfg2_gemv_m8_g64_%s_us" % name] = round(us, 2)
        out["cfg2_gemv_m8_g64_%s_GBs" % name] = round(b / (us * 1e-6) / 1e9, 1)
    del st8
    torch.cuda.empty_cache()

    # prefill, M=512 / 2048, g256 (and g64 at 2048), int8 TOPS
    out.update(prefill_tops(torch, ops, [(256, 512), (256, 2048), (64, 2048)]))
    # (a failure in one of these lines is recorded, not fatal to the bench line)
    for name, fn in (("prefill_k_split", prefill_k_split), ("tp8_shards", tp_shard_lines)):
        try:
            out.update(fn(torch, ops))
        except Exception as e:   # noqa: BLE001 -- reported in the JSON line
            out[name + "_error"] = "%s: %s" % (type(e).__name__, str(e)[:160])
            torch.cuda.synchronize()
    out.update(vendor_int8_gemm(torch))
    out.update(attention_side(torch, ops))
    return out


def attention_side(torch, ops):
    """The prefill attention side at the DualAR shape (n_q 32, n_kv 8, D 128,
    dual_ar_config.h:11-15), T = 2048: fused QKV split, causal attention,
    head merge.  Attention FLOPs count the causal half only:
    4 D n_q T (T + 1) / 2 (QK^T and PV, 2 flops per multiply-add)."""
    T, n_q, n_kv, D = 2048, 32, 8, 128
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    qkv = torch.randn((T, (n_q + 2 * n_kv) * D), generator=gen, device="cuda").half()
    q, k, v = ops.qkv_split_heads_gqa(qkv, n_q, n_kv, D)
    o = torch.empty_like(q)
    m = torch.empty((T, n_q * D), device="cuda", dtype=torch.float16)
    sc = 1.0 / D ** 0.5
    out = {}
    us = graph_us_per_call(torch, [lambda: ops.prefill_attention(q, k, v, sc, out=o)] * 4, reps=5)
    fl = 4.0 * D * n_q * T * (T + 1) / 2
    out["prefill_attn_t2048_us"] = round(us, 2)
    out["prefill_attn_t2048_TFLOPs"] = round(fl / (us * 1e-6) / 1e12, 1)
    out["prefill_attn_t2048_frac_fp16_peak"] = round(fl / (us * 1e-6) / 1e12 / FP16_PEAK_TFLOPS, 4)
    mt = torch.empty((T, n_q * D), device="cuda", dtype=torch.float16)
    us = graph_us_per_call(
        torch, [lambda: ops.prefill_attention_merged(q, k, v, sc, out=mt)] * 4, reps=5)
    out["prefill_attn_merged_t2048_us"] = round(us, 2)
    # the any-shape kernel (taken for head dims that are not a multiple of 8
    # or above 128, non-positive scales, or buffers not 16-byte aligned) on
    # the same shape, here reached through a negative scale
    us = graph_us_per_call(
        torch, [lambda: ops.prefill_attention(q, k, v, -sc, out=o)], reps=1, rounds=3)
    out["prefill_attn_anyshape_t2048_us"] = round(us, 1)
    us = graph_us_per_call(torch, [lambda: ops.qkv_split_heads_gqa(qkv, n_q, n_kv, D)] * 4)
    out["qkv_split_t2048_us"] = round(us, 2)
    out["qkv_split_t2048_GBs"] = round(2 * qkv.numel() * 2 / (us * 1e-6) / 1e9, 1)
    us = graph_us_per_call(torch, [lambda: ops.merge_heads(o, out=m)] * 4)
    out["merge_heads_t2048_us"] = round(us, 2)
    out["merge_heads_t2048_GBs"] = round(2 * o.numel() * 2 / (us * 1e-6) / 1e9, 1)
    return out


def vendor_int8_gemm(torch):
    """Context for configs[3]: the vendor library's plain int8 GEMM
    (torch._int_mm, int8 x int8 -> int32, no group scales, no epilogue) on
    the same four layer shapes at 2048 tokens, random operands, timed the
    same way.  Not part of the product; a yardstick for the MFMA roofline
    these shapes reach on this device."""
    from fish_amd.synth import LAYER_SHAPES
    out = {}
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4)
    M = 2048
    tot_ops, tot_us = 0.0, 0.0
    for name, (K, N) in LAYER_SHAPES.items():
        a = torch.randint(-127, 128, (M, K), generator=gen, device="cuda", dtype=torch.int8)
        b = torch.randint(-127, 128, (N, K), generator=gen, device="cuda", dtype=torch.int8)
        bt = b.t()
        try:
            us = graph_us_per_call(torch, [lambda: torch._int_mm(a, bt)] * 8, reps=5)
        except Exception as e:   # the library may not take a shape
            out["vendor_int8_mm_m2048_%s" % name] = "unavailable: %s" % str(e)[:80]
            continue
        o = 2.0 * M * N * K
        tot_ops += o
        tot_us += us
        out["vendor_int8_mm_m2048_%s_TOPS" % name] = round(o / (us * 1e-6) / 1e12, 1)
    if tot_us > 0:
        out["vendor_int8_mm_m2048_layer_TOPS"] = round(tot_ops / (tot_us * 1e-6) / 1e12, 1)
    return out


# One GPU's share of each linear under 8-way tensor parallelism: qkv and
# gate_up split their output rows, o and down their K (on group boundaries
# where g divides the share; down's 1216 leaves a short last group at g256).
TP8_SHAPES = {"qkv": (2560, 768), "o": (512, 2560), "gate_up": (2560, 2432),
              "down": (1216, 2560)}


def tp_shard_lines(torch, ops, layers=36, g=256):
    """The TP=8 shard shapes on one GPU: decode (1 token, fa_w8a8_gemm with
    in-kernel quantization, `layers` distinct weight copies per graph so
    every launch reads from HBM) in GB/s of algorithmic bytes, and prefill
    (2048 tokens, fa_w8a8_gemm_quantized) in int8 TOP/s."""
    out = {}
    gen = torch.Generator(device="cuda")
    gen.manual_seed(21)
    for name, (K, N) in TP8_SHAPES.items():
        G = (K + g - 1) // g
        ws = []
        for _ in range(layers):
            w = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
            ws.append(ops.quantize_weights_groupwise(w, g))
        x = torch.randn((1, K), generator=gen, device="cuda").half()
        y = torch.empty((1, N), device="cuda", dtype=torch.float16)
        us = graph_us_per_call(torch, [(lambda W=W, S=S: ops.w8a8_gemm(W, S, x, g, out=y))
                                       for W, S in ws])
        b = N * K + 2 * N * G + 2 * (K + N)
        out["tp8_gemv_m1_g256_%s_us" % name] = round(us, 2)
        out["tp8_gemv_m1_g256_%s_GBs" % name] = round(b / (us * 1e-6) / 1e9, 1)
        M = 2048
        xp = torch.randn((M, K), generator=gen, device="cuda").half()
        xq, xs = ops.quantize_activations(xp, g)
        yp = torch.empty((M, N), device="cuda", dtype=torch.float16)
        W, S = ws[0]
        us = graph_us_per_call(torch, [lambda: ops.w8a8_gemm_quantized(W, S, g, xq, xs, out=yp)]
                               * 8, reps=5)
        out["tp8_gemm_m2048_g256_%s_us" % name] = round(us, 2)
        out["tp8_gemm_m2048_g256_%s_TOPS" % name] = round(2.0 * M * N * K / (us * 1e-6) / 1e12, 1)
        del ws, xp, xq, xs, yp
        torch.cuda.empty_cache()
    return out


def prefill_k_split(torch, ops):
    """o and down at 512 tokens, g256, with the opt-in K split
    (fa_w8a8_set_k_split(8): partial chains added in split order, within
    1 ulp / rtol 1e-3 of the reference's chain rather than bit-exact) --
    beside the default exact figures of prefill_tops."""
    from fish_amd.synth import LAYER_SHAPES
    out = {}
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    M, g = 512, 256
    for name in ("o", "down"):
        K, N = LAYER_SHAPES[name]
        w = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
        W, S = ops.quantize_weights_groupwise(w, g)
        x = torch.randn((M, K), generator=gen, device="cuda").half()
        xq, xs = ops.quantize_activations(x, g)
        y = torch.empty((M, N), device="cuda", dtype=torch.float16)
        with ops.k_split(8):
            us = graph_us_per_call(torch, [lambda: ops.w8a8_gemm_quantized(W, S, g, xq, xs, out=y)]
                                   * 8, reps=5)
            out["cfg3_gemm_m512_g256_%s_ksplit%d_us" % (name, ops.k_splits(N, M, K, g))] = \
                round(us, 2)
    return out


def prefill_tops(torch, ops, cases):
    """int8 TOPS of w8a8_gemm_quantized (scale-table launch + GEMM)
    on the four layer shapes, for each (group size, tokens) case; random
    weights and activations (the MFMA clock depends on the data)."""
    from fish_amd.synth import LAYER_SHAPES
    out = {}
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    for g, M in cases:
        tot_ops, tot_ms = 0.0, 0.0
        for name, (K, N) in LAYER_SHAPES.items():
            w = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
            W, S = ops.quantize_weights_groupwise(w, g)
            del w
            x = torch.randn((M, K), generator=gen, device="cuda").half()
            xq, xs = ops.quantize_activations(x, g)
            y = torch.empty((M, N), device="cuda", dtype=torch.float16)
            f = lambda: ops.w8a8_gemm_quantized(W, S, g, xq, xs, out=y)
            # both launches of the call (scale tables + GEMM), 8 calls per
            # graph, so host launch overhead stays out of the GPU time
            ms = graph_us_per_call(torch, [f] * 8, reps=5) * 1e-3
            o = 2.0 * M * N * K
            tot_ops += o
            tot_ms += ms
            out["cfg3_gemm_m%d_g%d_%s_TOPS" % (M, g, name)] = round(o / (ms * 1e-3) / 1e12, 1)
            out["cfg3_gemm_m%d_g%d_%s_us" % (M, g, name)] = round(ms * 1e3, 2)
        tops = tot_ops / (tot_ms * 1e-3) / 1e12
        out["cfg3_gemm_m%d_g%d_layer_TOPS" % (M, g)] = round(tops, 1)
        out["cfg3_gemm_m%d_g%d_frac_int8_peak" % (M, g)] = round(tops / INT8_PEAK_TOPS, 4)
    return out


if __name__ == "__main__":
    main()
