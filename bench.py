"""Benchmark of the MoE expert path on one MI355X: the headline configuration (config
3), the Qwen3-30B-A3B-shaped MXFP8 routed-experts layer, forward and backward.

A step is one forward and backward of the layer (``bux_amd.moe.experts_forward`` then
``experts_backward``) on synthetic inputs already resident in HBM, captured in a HIP
graph and replayed (eager steps, timed too, give the per-op breakdown): the sort by
expert, 12 MXFP8 quantizations, 6 grouped GEMMs, the activation and its gradient, and
the token sums. `value` is the six GEMMs' algorithmic FLOP (2 M K N each, M = the picks)
per second of the whole step. One JSON line on stdout; with `roofline` for the
dominant kernel (per-op HIP events over the timed steps) and `cpu_baseline` (the CPU
oracle on a bounded sample of the same layer, on this host's cores).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
    python bench.py --config-forward N   # config N's forward alone (1, 2, 4 or 5)
"""

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "MXFP8 grouped-GEMM TFLOP/s + % of MFMA peak, Qwen3-30B-A3B MoE layer fwd+bwd"
PEAK_MXFP8_TFLOPS = 5000.0  # MI355X dense MXFP8 MFMA
PEAK_HBM_GBS = 8000.0
# Config 3 (and its sample for the CPU baseline): tokens, width, experts, picks, units.
T, D, E, K, F = 16384, 2048, 128, 8, 768
SEED = 1  # configs 2 and 3


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def inputs(t, d, e, k, f, device, seed=SEED):
    """Config 3's synthetic inputs: activations bf16 N(0,1) with 0.1% outliers x100,
    router logits N(0,1) -> softmax -> top-k, normalised; kernels bf16 N(0, 0.02);
    upstream grads bf16 N(0, 1e-2)."""
    g = torch.Generator(device=device).manual_seed(seed)
    z = torch.randn(t, d, generator=g, device=device)
    outliers = torch.randperm(t * d, generator=g, device=device)[: max(1, t * d // 1000)]
    z.view(-1)[outliers] *= 100
    logits = torch.randn(t, e, generator=g, device=device)
    probs = torch.softmax(logits, -1)
    weights, idx = torch.topk(probs, k, -1)
    weights = weights / weights.sum(-1, keepdim=True)
    up = torch.randn(e, d, f, 2, generator=g, device=device) * 0.02
    down = torch.randn(e, f, d, generator=g, device=device) * 0.02
    dy = torch.randn(t, d, generator=g, device=device) * 1e-2
    bf = torch.bfloat16
    return (z.to(bf), idx.to(torch.int32).contiguous(), weights.to(bf), up.to(bf), down.to(bf),
            dy.to(bf))


def zipf_picks(t, e, k, seed, s=1.2, empty=0.2):
    """Config 5's picks, built from their loads: Zipf(s) shares over a seeded permutation
    of the experts, the last `empty` fraction of the ranks given none; each expert's
    load is its share of the t k picks, capped at t (a token picks k distinct experts,
    so no expert holds more than 1/k of them: 12.5% at k = 8), the cut spread over the
    others by their shares, rounded by largest remainders to sum to t k. The picks are
    laid out expert after expert and dealt to tokens round-robin (pick j to token j mod
    t), which gives every token k distinct experts since no load exceeds t; the tokens
    are then shuffled. Returns idx (t, k) int32 and the loads (e,)."""
    rng = np.random.default_rng(seed)
    ranked = rng.permutation(e)
    live = e - int(round(e * empty))
    share = np.zeros(e)
    share[ranked[:live]] = np.arange(1, live + 1, dtype=np.float64) ** -s
    total, capped = t * k, np.zeros(e, bool)
    while True:  # cap the experts whose share of what is left passes t; repeat
        scale = (total - t * capped.sum()) / share[~capped].sum()
        over = ~capped & (share * scale > t)
        if not over.any():
            break
        capped |= over
    want = np.where(capped, float(t), share * scale)
    loads = np.floor(want).astype(np.int64)
    short = total - int(loads.sum())
    loads[np.argsort(-(want - loads), kind="stable")[:short]] += 1
    assert loads.sum() == total and loads.max() <= t
    seq = np.repeat(np.arange(e), loads)
    idx = np.empty((t, k), np.int64)
    idx[np.arange(total) % t, np.arange(total) // t] = seq
    idx = idx[rng.permutation(t)]
    return idx.astype(np.int32), loads


def gemm_flops(m, d, f):
    """The six GEMMs' algorithmic FLOP of one fwd+bwd: 2 M K N each."""
    up = 2 * m * d * 2 * f
    down = 2 * m * f * d
    return {"up fprop": up, "down fprop": down, "down dgrad": down, "up dgrad": up,
            "down wgrad": down, "up wgrad": up}


def gemm_bytes(m, d, f, e):
    """Algorithmic HBM bytes of each GEMM: both MXFP8 operands (a code and 1/32 of a
    scale byte an element) read once and the bfloat16 output written once."""
    q = 1 + 1 / 32
    rows = {"up fprop": (m * d, e * 2 * f * d, m * 2 * f), "down fprop": (m * f, e * d * f, m * d),
            "down dgrad": (m * d, e * f * d, m * f), "up dgrad": (m * 2 * f, e * d * 2 * f, m * d),
            "down wgrad": (m * d, m * f, e * d * f), "up wgrad": (m * 2 * f, m * d, e * 2 * f * d)}
    return {name: (a + b) * q + 2 * c for name, (a, b, c) in rows.items()}


def op_bytes(t, m, d, f, e):
    """Algorithmic HBM bytes of the streaming ops: unique input bytes + output bytes."""
    q = 1 + 1 / 32  # an E4M3 code and its share of a scale byte
    return {
        "quantize x": t * d * 2 + 2 * m * d * q,
        "quantize W_up": e * d * 2 * f * 2 + 2 * e * d * 2 * f * q,
        # the activation (projected and the row weights in) and both copies of h out
        "activation + quantize h": m * 2 * f * 2 + m * 2 + 2 * m * f * q,
        "quantize W_down": e * f * d * 2 + 2 * e * f * d * q,
        "quantize dy": t * d * 2 + 2 * m * d * q,
        # its gradient: projected, dh and the weights in; both copies of d projected
        # and the row weights' gradient out
        "activation backward + quantize dp": m * 2 * f * 2 + m * f * 2 + m * 2
                                             + 2 * m * 2 * f * q + m * 2,
        "combine": m * d * 2 + t * d * 2,
        "combine dx": m * d * 2 + t * d * 2,
    }


def measured_traffic(op):
    """HBM bytes (read + written) of one launch of `op`, as rocprofv3's FETCH_SIZE and
    WRITE_SIZE counters measured it (scaled by a plain copy of known size), from the
    summary committed under profiles/; None when that summary has no row for `op`."""
    path = os.path.join(ROOT, "profiles", "c3_layer_step_hbm_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 7 and cells[0] == op:
            try:
                return round((float(cells[2]) + float(cells[5])) * 2**20)
            except ValueError:
                return None
    return None


def step(z, idx, w, up, down, dy):
    from bux_amd import moe

    out, saved = moe.experts_forward(z, idx, w, up, down)
    grads = moe.experts_backward(saved, dy, up, down)
    return out, grads


def graph_step_ms(z, idx, w, up, down, dy, steps, warmup):
    """The step captured once in a HIP graph (torch.cuda.CUDAGraph: the same kernels on
    the same stream, launched without the host in between) and replayed: `warmup`
    untimed replays, then `steps` timed between two synchronisations. Returns (ms a
    step, how it was launched); (None, why) if the capture fails, and the eager time
    stands."""
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step(z, idx, w, up, down, dy)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step(z, idx, w, up, down, dy)
        for _ in range(warmup):
            graph.replay()
        torch.cuda.synchronize()
        start = time.perf_counter()
        for _ in range(steps):
            graph.replay()
        torch.cuda.synchronize()
        seconds = time.perf_counter() - start
        log(f"timed {steps} graph replays in {seconds:.3f} s")
        return seconds * 1e3 / steps, "hip graph of the whole step (per-op times: eager, HIP events)"
    except RuntimeError as err:  # no capture here: the eager steps' time stands
        log(f"graph capture failed ({err}); eager time stands")
        return None, f"eager (graph capture failed: {str(err)[:120]})"


def timed(fn, reps=20):
    """Average milliseconds of `fn()` over `reps` calls after 3 untimed ones: HIP events
    on the current stream, which the library's kernels run on."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(s)
    for _ in range(reps):
        fn()
    end.record(s)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def feed_ops(z, idx, e, k):
    """Time the ops either side of the layer, and the mxfp8_2d recipe's weight
    quantizer, outside the timed step (they are not part of its GEMM FLOP): the router (bux_amd.router.route: logits, softmax, top-k,
    weights) on the step's tokens with a random-init Qwen3 router kernel (d x E,
    N(0, 0.02)), W_up's two copies with a scale per 32 x 32 tile, and an expert-parallel dispatch's MXFP8 rows (bux_amd.dispatch: the
    picks' rows packed from the tokens, then unpacked to bfloat16). Each with its
    algorithmic bytes (inputs read once, outputs written once) and HBM fraction."""
    from bux_amd import dispatch, moe, router

    g = torch.Generator(device=z.device).manual_seed(SEED + 1)
    kernel = (torch.randn(z.shape[1], e, generator=g, device=z.device) * 0.02).to(torch.bfloat16)
    t, d = z.shape
    m = t * k
    row = d + d // 32
    order = moe.sort_by_expert(idx, e).order
    packed = dispatch.picked_in_mxfp8(z, order, k)
    from bux_amd import grouped_mxfp8

    up = (torch.randn(e, d, 2 * F, generator=g, device=z.device) * 0.02).to(torch.bfloat16)
    q = 1 + 1 / 32
    ops = {
        "router": (lambda: router.route(z, kernel, top_k=k), t * d * 2 + d * e * 2 + t * k * 6),
        "quantize W_up (mxfp8_2d: 32x32 tiles)": (
            lambda: grouped_mxfp8.quantized_twice(up, tiles=True), up.numel() * (2 + 2 * q)),
        "dispatch pack": (lambda: dispatch.picked_in_mxfp8(z, order, k), t * d * 2 + m * 4 + m * row),
        "dispatch unpack": (lambda: dispatch.from_mxfp8(packed, d), m * row + m * d * 2),
    }
    out = {}
    for name, (fn, nbytes) in ops.items():
        ms = timed(fn)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"ms": round(ms, 4), "bytes": nbytes, "gbs": round(gbs, 1),
                     "frac_of_hbm": round(gbs / PEAK_HBM_GBS, 4)}
    return out


def fused_up(z, idx, w, up, e, k):
    """Time the up GEMM with the activation and h's two MXFP8 copies in its epilogue
    (grouped_mxfp8.activated, one GEMM kernel and a small fix-up) against the step's
    unfused pair (the rows GEMM, then the activation's quantizer) on the step's own
    operands: the two give the same bits, so the faster one belongs in the step."""
    from bux_amd import grouped_mxfp8, moe

    t, d = z.shape
    m = t * k
    f = up.shape[2]
    s = moe.sort_by_expert(idx, e)
    height = grouped_mxfp8.whole(m)
    x_k, _ = grouped_mxfp8.quantized_twice(z, s.filled, False, s.order, k, height)
    _, up_k = grouped_mxfp8.quantized_twice(up.reshape(e, d, 2 * f))
    row_weights = moe.picked_weights(w, s.order)
    ffn = moe.Ffn()

    def unfused():
        projected = grouped_mxfp8.rows(x_k, up_k, s.sizes, height=m)
        return moe.weighted_units_quantized(ffn, projected.view(m, f, 2), row_weights, s.filled,
                                            height)

    def fused():
        return grouped_mxfp8.activated(x_k, up_k, s.sizes, row_weights, ffn.struct(True), m)

    return {"fused_ms": round(timed(fused), 4), "unfused_ms": round(timed(unfused), 4),
            "used_in_step": "unfused"}


def fused_down(z, idx, w, up, down, dy, e, k):
    """Time the down dgrad with the activation's gradient and d projected's two MXFP8
    copies in its epilogue (grouped_mxfp8.activation_grad: one GEMM kernel, a small
    fix-up and the weights' sums) against the step's unfused pair (the rows GEMM into dh,
    then the quantizing activation backward) on the step's own operands: the two give the
    same bits."""
    from bux_amd import grouped_mxfp8, moe

    t, d = z.shape
    m = t * k
    f = up.shape[2]
    _, saved = moe.experts_forward(z, idx, w, up, down)
    s = saved.sorted
    height = grouped_mxfp8.whole(m)
    dy_n, _ = grouped_mxfp8.quantized_twice(dy, s.filled, False, s.order, k, height)
    ffn = moe.Ffn()

    def unfused():
        dh = grouped_mxfp8.rows(dy_n, saved.down_n, s.sizes, height=m)
        return moe.weighted_units_backward_quantized(ffn, saved.projected.view(m, f, 2),
                                                     saved.row_weights, dh, s.filled, height)

    def fused():
        return grouped_mxfp8.activation_grad(dy_n, saved.down_n, s.sizes, saved.projected,
                                             saved.row_weights, ffn.struct(True), m)

    return {"fused_ms": round(timed(fused), 4), "unfused_ms": round(timed(unfused), 4),
            "used_in_step": "unfused"}


PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bfloat16 MFMA


def compute_step(z, idx, w, up, down, dy, reps=5):
    """The same layer step with every pass in bfloat16 (fmt "compute": the bfloat16
    grouped GEMMs), its ops timed by spans (HIP events around each), over `reps` steps
    after two untimed ones."""
    from bux_amd import moe
    from bux_amd.spans import Spans

    def run():
        _, saved = moe.experts_forward(z, idx, w, up, down, fmt="compute")
        moe.experts_backward(saved, dy, up, down, fmt="compute")

    for _ in range(2):
        run()
    torch.cuda.synchronize()
    with Spans() as spans:
        for _ in range(reps):
            run()
        torch.cuda.synchronize()
    ms = {name: float(np.mean(v)) for name, v in spans.milliseconds().items()}
    flops = gemm_flops(z.shape[0] * idx.shape[1], z.shape[1], up.shape[2])
    gemms = {}
    for name, fl in flops.items():
        tf = fl / (ms[name] * 1e-3) / 1e12
        gemms[name] = {"ms": round(ms[name], 4), "tflops": round(tf, 1),
                       "frac_of_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4)}
    return {"ms_per_step_spans": round(sum(ms.values()), 4), "gemms": gemms}

# The other configs of BASELINE.json, forward only there: (tokens, width, experts, picks,
# units, activation (kind, limit, up offset), seed, router skew, format, the CPU
# oracle's sample (tokens, experts): None for the whole config).
OTHER_CONFIGS = {
    "config 1: tiny bf16 layer forward": (
        4096, 256, 8, 2, 512, ("swish", None, 0.0), 0, None, "compute", None),
    "config 2: Qwen3-30B-A3B layer forward": (
        16384, 2048, 128, 8, 768, ("swish", None, 0.0), 1, None, "mxfp8", (1024, 8)),
    "config 4: gpt-oss-120b layer forward (clamped SwiGLU)": (
        8192, 2880, 128, 4, 2880, ("quick_gelu", 7.0, 1.0), 2, "bias", "mxfp8", (256, 4)),
    "config 5: DeepSeek-V3 layer forward (Zipf loads)": (
        8192, 7168, 256, 8, 2048, ("swish", None, 0.0), 3, "zipf", "mxfp8", (128, 8)),
}


def other_config(t, d, e, k, f, act, seed, skew, fmt, sample, device, reps=10):
    """One config's MXFP8 forward (the layer as training runs it: x^T and h^T quantized
    for the wgrad too), timed as HIP graph replays, with the weights quantized inside
    (`ms`) and given already in MXFP8 (`ms_weights_given`: the reference's `quantized`,
    quantized once an optimizer step); and with only the fprop pass in MXFP8
    (`ms_fprop_pass_only`: one MXFP8 copy of each operand, the weights quantized inside,
    what the bfloat16 dgrad and wgrad take kept in bfloat16). Router logits N(0,1), plus a
    per-expert bias N(0, 0.5) (config 4), softmax, top-k, normalised; config 5's picks
    built from Zipf(1.2) loads (`zipf_picks`), each token's k weights a softmax of
    N(0, 1) draws."""
    from bux_amd import moe

    g = torch.Generator(device=device).manual_seed(seed)
    z = torch.randn(t, d, generator=g, device=device)
    outliers = torch.randperm(t * d, generator=g, device=device)[: max(1, t * d // 1000)]
    z.view(-1)[outliers] *= 100
    if skew == "zipf":
        picks, _ = zipf_picks(t, e, k, seed)
        idx = torch.from_numpy(picks).to(device)
        weights = torch.softmax(torch.randn(t, k, generator=g, device=device), -1)
    else:
        logits = torch.randn(t, e, generator=g, device=device)
        if skew == "bias":
            logits += torch.randn(e, generator=g, device=device) * 0.5
        weights, idx = torch.topk(torch.softmax(logits, -1), k, -1)
        weights = weights / weights.sum(-1, keepdim=True)
        del logits
    weights = weights.to(torch.bfloat16)
    idx = idx.to(torch.int32).contiguous()
    up = (torch.randn(e, d, f, 2, generator=g, device=device) * 0.02).to(torch.bfloat16)
    down = (torch.randn(e, f, d, generator=g, device=device) * 0.02).to(torch.bfloat16)
    z = z.to(torch.bfloat16)
    ffn = moe.Ffn(*act)

    def graph_ms(forward):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            forward()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            forward()
        graph.replay()
        torch.cuda.synchronize()
        start = time.perf_counter()
        for _ in range(reps):
            graph.replay()
        torch.cuda.synchronize()
        return (time.perf_counter() - start) * 1e3 / reps

    ms = graph_ms(lambda: moe.experts_forward(z, idx, weights, up, down, ffn, fmt))
    loads = torch.bincount(idx.view(-1).long(), minlength=e)
    m = t * k
    flops = 2 * m * d * 2 * f + 2 * m * f * d
    peak = PEAK_MXFP8_TFLOPS if fmt != "compute" else PEAK_BF16_TFLOPS
    out = {"format": fmt, "ms": round(ms, 4), "gemm_tflop": round(flops / 1e12, 4),
           "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
           "frac_of_peak": round(flops / (ms * 1e-3) / 1e12 / peak, 4), "peak_tflops": peak}
    if fmt != "compute":
        given = moe.in_mxfp8(up, down)
        ms_given = graph_ms(lambda: moe.experts_forward(z, idx, weights, up, down, ffn, fmt,
                                                        quantized=given))
        out.update(ms_weights_given=round(ms_given, 4),
                   tflops_weights_given=round(flops / (ms_given * 1e-3) / 1e12, 1))
        # only the fprop pass in MXFP8 (passes=("fprop",), grouped_blockscaled.py:180-183):
        # one MXFP8 copy each of x, W and h, along the GEMMs' K; x's rows and h kept in
        # bfloat16 for the dgrad and wgrad, which then multiply in bfloat16
        ms_fprop = graph_ms(lambda: moe.experts_forward(z, idx, weights, up, down, ffn, fmt,
                                                        passes=("fprop",)))
        out.update(ms_fprop_pass_only=round(ms_fprop, 4),
                   tflops_fprop_pass_only=round(flops / (ms_fprop * 1e-3) / 1e12, 1))
    out.update(largest_group_share=round(float(loads.max()) / m, 4),
               empty_experts=int((loads == 0).sum()))
    return out


def other_configs(device):
    """BASELINE.json's other MXFP8 configs, each timed on its own (an error is recorded,
    not raised: the headline line stands)."""
    out = {}
    for name, cfg in OTHER_CONFIGS.items():
        try:
            out[name] = other_config(*cfg, device)
            log(f"{name}: {out[name]}")
        except (RuntimeError, torch.OutOfMemoryError) as err:
            out[name] = {"error": str(err)[:200]}
        torch.cuda.empty_cache()
    return out


def config_cpu_baselines():
    """The CPU oracle's forward on each other config: the whole of config 1, and for the
    others a bounded sample of the same per-expert shape (a few experts, their share of
    the tokens), timed on this host's cores."""
    from oracle import bf16, moe as omoe

    out = {}
    for name, (t, d, e, k, f, act, seed, _, fmt, sample) in OTHER_CONFIGS.items():
        ts, es = (t, e) if sample is None else sample
        rng = np.random.default_rng(seed)

        def bits(shape, scale):
            return bf16.to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))

        z, up, down = bits((ts, d), 1.0), bits((es, d, f, 2), 0.02), bits((es, f, d), 0.02)
        idx = np.stack([rng.choice(es, k, replace=False) for _ in range(ts)]).astype(np.int32)
        w = bf16.to_bf16((rng.random((ts, k)) / k).astype(np.float32))
        start = time.perf_counter()
        omoe.layer_forward(z, idx, w, up, down, omoe.Ffn(*act), fmt)
        seconds = time.perf_counter() - start
        m = ts * k
        flops = 2 * m * d * 2 * f + 2 * m * f * d
        out[name] = {"value": round(flops / seconds / 1e12, 5), "unit": "TFLOP/s",
                     "cores": len(os.sched_getaffinity(0)), "kind": "port",
                     "sample": ("the whole config" if sample is None else
                                f"{ts} tokens x top-{k} over {es} experts of d={d} f={f}")
                               + f", oracle forward ({fmt}), {flops / 1e9:.1f} GFLOP in "
                                 f"{seconds:.2f} s"}
        log(f"cpu {name}: {out[name]}")
    return out


def cpu_baseline():
    """The CPU oracle (numpy: float64/float32 quantizer, BLAS float32 GEMMs) on a bounded
    sample of config 3: 8 of its 128 experts with the same per-expert shape (1024
    tokens x top-8 = 8192 picks, ~1024 rows an expert, d=2048, f=768)."""
    from oracle import bf16, moe as omoe

    t, e = 1024, 8
    rng = np.random.default_rng(SEED)

    def bits(shape, scale):
        return bf16.to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))

    z, up, down, dy = bits((t, D), 1.0), bits((e, D, F, 2), 0.02), bits((e, F, D), 0.02), bits((t, D), 1e-2)
    idx = np.stack([rng.choice(e, K, replace=False) for _ in range(t)]).astype(np.int32)
    w = bf16.to_bf16((rng.random((t, K)) / K).astype(np.float32))
    start = time.perf_counter()
    _, saved = omoe.layer_forward(z, idx, w, up, down)
    omoe.layer_backward(saved, dy, z, up, down, K)
    seconds = time.perf_counter() - start
    flops = sum(gemm_flops(t * K, D, F).values())
    cores = len(os.sched_getaffinity(0))
    return {
        "value": flops / seconds / 1e12,
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": f"oracle layer fwd+bwd, {t} tokens x top-{K}, {e} experts of d={D} f={F} "
                  f"({flops / 1e12:.3f} TFLOP in {seconds:.1f} s); BLAS GEMMs on up to "
                  f"{cores} threads, numpy quantizer single-threaded",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the forward timings of configs 2, 4 and 5")
    ap.add_argument("--config-forward", type=int, default=0, metavar="N",
                    help="run only config N's forward timing (1, 2, 4 or 5; as other_configs "
                         "reports it) and print its JSON: the command a per-config kernel "
                         "trace profiles")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="run only a plain device-to-device copy of MIB MiB, 10 times: the "
                         "kernel of known traffic that scales rocprofv3's FETCH_SIZE and "
                         "WRITE_SIZE counters to bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py runs on one GPU: this build has no multi-GPU path (the MoE expert "
              "path would shard by expert over an RCCL all-to-all of MXFP8 rows)", file=sys.stderr)
        sys.exit(2)

    from bux_amd import kernels
    from bux_amd.spans import Spans

    if not kernels.runs():
        raise SystemExit("bench.py needs a gfx950 GPU and the built library (python -m bux_amd.build)")
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.ones(n, dtype=torch.uint8, device=device)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": n, "copies": 10}), flush=True)
        return
    if args.config_forward:
        names = [n for n in OTHER_CONFIGS if n.startswith(f"config {args.config_forward}:")]
        if not names:
            raise SystemExit(f"no config {args.config_forward} among {list(OTHER_CONFIGS)}")
        name = names[0]
        out = other_config(*OTHER_CONFIGS[name], device)
        print(json.dumps({"config": name, **out}), flush=True)
        return
    log(f"inputs: config 3, T={T} d={D} E={E} k={K} f={F}")
    z, idx, w, up, down, dy = inputs(T, D, E, K, F, device)
    torch.cuda.synchronize()
    for i in range(args.warmup):
        step(z, idx, w, up, down, dy)
        torch.cuda.synchronize()
        log(f"warmup step {i} done")
    torch.cuda.synchronize()
    with Spans() as spans:
        start = time.perf_counter()
        for _ in range(args.steps):
            step(z, idx, w, up, down, dy)
        torch.cuda.synchronize()
        seconds = time.perf_counter() - start
    log(f"timed {args.steps} eager steps in {seconds:.3f} s")
    ms = {name: float(np.mean(v)) for name, v in spans.milliseconds().items()}
    m = T * K
    flops = gemm_flops(m, D, F)
    total_flops = sum(flops.values())
    eager_ms = seconds * 1e3 / args.steps
    graph_ms, launch = graph_step_ms(z, idx, w, up, down, dy, args.steps, args.warmup)
    ms_per_step = graph_ms if graph_ms is not None else eager_ms
    value = total_flops / (ms_per_step * 1e-3) / 1e12
    gemms = {name: {"ms": ms[name], "tflops": flops[name] / (ms[name] * 1e-3) / 1e12,
                    "frac_of_peak": flops[name] / (ms[name] * 1e-3) / 1e12 / PEAK_MXFP8_TFLOPS}
             for name in flops}
    dominant = max(gemms, key=lambda n: gemms[n]["ms"])
    nbytes = op_bytes(T, m, D, F, E)
    streams = {name: {"ms": ms[name], "gbs": nbytes[name] / (ms[name] * 1e-3) / 1e9,
                      "frac_of_peak": nbytes[name] / (ms[name] * 1e-3) / 1e9 / PEAK_HBM_GBS}
               for name in nbytes if name in ms}
    other = {name: {"ms": v} for name, v in ms.items() if name not in gemms and name not in streams}
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "launch": launch,
        "ms_per_step_eager": round(eager_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp8 (e4m3 x e4m3, e8m0 1x32 scales, f32 accumulate, bf16 out)",
        "data": "synthetic (seeded: bf16 N(0,1) tokens with 0.1% x100 outliers, softmax top-8 of "
                "N(0,1) logits, kernels N(0,0.02), grads N(0,1e-2)); random-init weights",
        "config": {"workload": "config 3: Qwen3-30B-A3B MoE experts layer fwd+bwd, MXFP8",
                   "tokens": T, "d_model": D, "experts": E, "top_k": K, "moe_intermediate": F,
                   "gemm_tflop_per_step": total_flops / 1e12, "parallelism": "single GPU"},
        "roofline": {
            "bound": "mfma",
            "kernel": f"{dominant} ({'contract_kernel' if 'wgrad' in dominant else 'rows_kernel'})",
            "achieved": round(gemms[dominant]["tflops"], 2),
            "peak": PEAK_MXFP8_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(gemms[dominant]["frac_of_peak"], 4),
            "traffic": measured_traffic(dominant),
            "traffic_source": "profiles/c3_layer_step_hbm_traffic.md (rocprofv3 --pmc "
                              "FETCH_SIZE, WRITE_SIZE; bytes a launch)",
            "algorithmic_bytes": round(gemm_bytes(m, D, F, E)[dominant]),
        },
        "gemms": {n: {k2: round(v2, 4) for k2, v2 in g.items()} for n, g in gemms.items()},
        "streaming": {n: {k2: round(v2, 4) for k2, v2 in g.items()} for n, g in streams.items()},
        "other_ms": {n: round(g["ms"], 4) for n, g in other.items()},
        "gemm_ms_per_step": round(sum(g["ms"] for g in gemms.values()), 4),
    }
    result["feed"] = feed_ops(z, idx, E, K)
    result["fused_up_gemm"] = fused_up(z, idx, w, up, E, K)
    result["fused_down_dgrad"] = fused_down(z, idx, w, up, down, dy, E, K)
    result["compute_step"] = compute_step(z, idx, w, up, down, dy)
    if not args.no_other_configs:
        result["other_configs"] = other_configs(device)
    if not args.no_cpu_baseline:
        log("cpu baseline: oracle on a sample of config 3 ...")
        result["cpu_baseline"] = cpu_baseline()
        if "other_configs" in result:
            for name, cpu in config_cpu_baselines().items():
                result["other_configs"][name]["cpu_baseline"] = cpu
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
