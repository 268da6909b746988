"""Benchmark of the MI355X DiT hot path: Q8_0 x bf16 products at M = 22
and the 10-step CFG DiT patch.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

A step is one pass over the product sweep's four weight shapes
(K, N) in {(1024, 3072), (1024, 8192), (2048, 2048), (2048, 16384)} with
22 bf16 activation rows: four launches, each on the next of the rotating
weight copies that keep at least 1 GiB per shape in HBM (beyond the 256 MB
Infinity Cache), the launches replayed from one HIP graph. `value` is the
weight bytes (N K 34 / 32 per product, read once) of the K timed steps over
their wall time. Beside it the line reports every (M, K, N) of the sweep,
a plain-read probe, the whole 12-block 10-step CFG patch (MALL-warm and
MALL-cold), and the CPU oracle on the host's cores.

Prints progress to stderr and one JSON line to stdout.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
SWEEP_SHAPES = [(1024, 3072), (1024, 8192), (2048, 2048), (2048, 16384)]
# The single product of the CPU-runnable configuration (M = 22, K = 1024,
# N = 4096): timed beside the sweep, not part of `value`.
SINGLE_SHAPE = (1024, 4096)
SWEEP_ROWS = [1, 2, 22, 44, 128]
ROWS = 22
# Runs of the CPU oracle's whole patch (the median is reported).
CPU_PATCH_RUNS = 5
ROTATION_BYTES = 1.1e9
BF16_PEAK_TFLOPS = 2500.0
# MFMA utilisation read from rocprofv3 counters for the prefill kernel
# (SQ_VALU_MFMA_BUSY_CYCLES over the SIMDs' cycles), next to the
# wall-clock mfma_frac of each prefill row; profiles/q8_gemm_prefill.md.
PREFILL_MFMA_BUSY = {"source": "profiles/q8_gemm_prefill.md (rocprofv3 --pmc "
                               "SQ_VALU_MFMA_BUSY_CYCLES, GRBM_GUI_ACTIVE)",
                     "m512_n16384": 0.309, "m1024_n16384": 0.413}
# HBM bytes per launch of the M=22 sweep kernels from two rocprofv3 PMC runs
# (profiles/q8_skinny_m22_traffic.md): FETCH_SIZE KiB (scaled by 2.0, its
# reading of a 256 MiB copy of known size) + WRITE_SIZE KiB (scale 1.0).
# Measured, not computed: re-measure when the product kernel changes. Last
# measured on the build of commit TRAFFIC_BUILD (the summary names it).
FETCH_SCALE = 262144 / 131083.5
TRAFFIC_BUILD = "6605d9d"
TRAFFIC_KIB = {(1024, 3072): (1831.5, 264.0), (1024, 8192): (4545.5, 704.0),
               (2048, 2048): (2547.5, 176.0), (2048, 16384): (17802.0, 1408.0)}
# The decode steps' products (tools/bench/gemm_bench.cpp:34-38): the base and
# residual LMs (hidden 2048, 16 + 2 x 2 heads of 128, MLP 6144) and the
# local encoder/DiT shapes, at one row (an LM step) and five (the encoder's
# patch + special row).
LM_SHAPES = [("lm qkv", 2048, 2560), ("lm o", 2048, 2048), ("lm gate_up", 2048, 12288),
             ("lm down", 6144, 2048), ("local qkv", 1024, 2560), ("local o", 2048, 1024),
             ("local gate_up", 1024, 8192), ("local down", 4096, 1024)]
LM_ROWS = [1, 5]
PREFILL_M = [129, 256, 512, 1024]
PREFILL_N = [2048, 6144, 16384]
PREFILL_K = 2048
METRIC = "Q8_0 GEMM GB/s (% HBM peak) at M=22; us per 10-step CFG DiT patch"


def log(message: str) -> None:
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def q8_bytes(k: int, n: int) -> int:
    return n * k * 34 // 32


class Product:
    """One sweep shape on the GPU: a pool of rotating weight copies."""

    def __init__(self, ops, synth, torch, device, k: int, n: int, seed: int,
                 rows=SWEEP_ROWS):
        self.k, self.n = k, n
        rng = synth.Rng(seed, k * 31 + n)
        blocks = torch.from_numpy(synth.q8_blocks(rng, n, k)).to(device)
        packed = ops.q8_pack(blocks, n, k)
        self.bytes = packed.numel()
        assert self.bytes == q8_bytes(k, n)
        self.copies = max(8, int(np.ceil(ROTATION_BYTES / self.bytes)))
        self.pool = packed.repeat(self.copies).view(self.copies, -1)
        self.inputs = {}
        self.outputs_bf16 = {}
        for m in rows:
            x = synth.activations(rng, m, k)
            self.inputs[m] = (
                torch.from_numpy(x.view(np.int16)).to(device).view(torch.bfloat16),
                torch.empty((m, n), dtype=torch.float32, device=device))
            self.outputs_bf16[m] = torch.empty((m, n), dtype=torch.bfloat16, device=device)
        self.launches = 0

    def launch(self, ops, scratch, m: int) -> None:
        x, y = self.inputs[m]
        ops.q8_linear(x, self.pool[self.launches % self.copies], self.n, y=y,
                      scratch=scratch)
        self.launches += 1

    def launch_bf16(self, ops, scratch, m: int) -> None:
        """The same product with its bf16 output (vx_q8_linear_bf16)."""
        x, _ = self.inputs[m]
        ops.q8_linear_bf16(x, self.pool[self.launches % self.copies], self.n,
                           y=self.outputs_bf16[m], scratch=scratch)
        self.launches += 1


def graph_of(torch, stream, body, count: int):
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(count):
            body(i)
    return graph


def time_graph(torch, stream, graph, repeats: int = 1, warm_seconds: float = 0.0) -> float:
    """Seconds of one replay (the median of `repeats`), events on the replay
    stream, after replaying for `warm_seconds` untimed."""
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    begin = time.perf_counter()
    while time.perf_counter() - begin < warm_seconds:
        graph.replay()
        stream.synchronize()
    times = []
    for _ in range(repeats):
        stream.synchronize()
        start.record(stream)
        graph.replay()
        stop.record(stream)
        stop.synchronize()
        times.append(start.elapsed_time(stop) / 1e3)
    return float(np.median(times))


def read_probe(torch, device, stream) -> float:
    """GB/s of torch's sum over 2 GiB of int64 (a read-bound pass)."""
    data = torch.ones(1 << 28, dtype=torch.int64, device=device)
    for _ in range(2):
        data.sum()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(5):
        data.sum()
    stop.record(stream)
    stop.synchronize()
    seconds = start.elapsed_time(stop) / 1e3 / 5
    return data.numel() * 8 / seconds / 1e9


def gpu_launch_floor(torch, ops, device, stream):
    """The per-launch costs every kernel of a HIP graph pays, measured with
    the kernels' own launch pattern (vx_handoff, replayed from a graph,
    events on the launch stream): an empty launch of one workgroup and of
    the products' grid (256 workgroups of 1024 threads), and a chain of
    dependent launches in which every workgroup reads the whole block the
    previous launch wrote (1, 45 and 64 KB: the DiT's activation blocks
    are 45-64 KB of bf16 per workgroup)."""
    sink = torch.zeros(4, dtype=torch.int32, device=device)
    buffers = [torch.zeros(1 << 18, dtype=torch.int32, device=device) for _ in range(2)]
    count = 400
    result = {}
    for name, workgroups, threads, nbytes in [
            ("empty_1x64", 1, 64, 0), ("empty_256x1024", 256, 1024, 0),
            ("dependent_1KB", 256, 1024, 1024), ("dependent_45KB", 256, 1024, 45056),
            ("dependent_64KB", 256, 1024, 65536)]:
        g = graph_of(torch, stream,
                     lambda i, w=workgroups, t=threads, b=nbytes: ops.handoff(
                         buffers[i % 2], buffers[(i + 1) % 2], b, w, t, sink), count)
        g.replay()
        result[name] = round(time_graph(torch, stream, g, repeats=5) / count * 1e6, 3)
        del g
    log(f"launch floor: {result}")
    return {"launch_floor_us": result["empty_256x1024"],
            "dependent_launch_us": result["dependent_64KB"],
            "us": result,
            "method": "vx_handoff launches replayed 400 at a time from one HIP graph, "
                      "median of five replays"}


def gpu_products(args, torch, ops, synth, device, stream):
    scratch = ops.Scratch(128, 16384)
    log("building weight pools")
    products = [Product(ops, synth, torch, device, k, n, seed=0) for k, n in SWEEP_SHAPES]
    single = Product(ops, synth, torch, device, *SINGLE_SHAPE, seed=0, rows=[ROWS])

    def step(_):
        for p in products:
            p.launch(ops, scratch, ROWS)

    for _ in range(args.warmup):
        step(0)
    stream.synchronize()
    timed = graph_of(torch, stream, step, args.steps)
    warm = graph_of(torch, stream, step, max(1, args.warmup))
    warm.replay()
    torch.cuda.synchronize()
    seconds = time_graph(torch, stream, timed)
    torch.cuda.synchronize()
    step_bytes = sum(p.bytes for p in products)
    value = step_bytes * args.steps / seconds / 1e9
    log(f"M=22 sweep: {value:.0f} GB/s over {args.steps} steps, "
        f"{seconds / args.steps * 1e6:.2f} us per step")

    sweep = []
    for p in products:
        for m in SWEEP_ROWS:
            count = max(p.copies, 64)
            g = graph_of(torch, stream, lambda _i, p=p, m=m: p.launch(ops, scratch, m), count)
            g.replay()
            s = time_graph(torch, stream, g)
            us = s / count * 1e6
            sweep.append({"m": m, "k": p.k, "n": p.n, "us": round(us, 3),
                          "gbs": round(p.bytes / us / 1e3, 1),
                          "hbm_frac": round(p.bytes / us / 1e3 / HBM_PEAK_GBS, 4),
                          "tflops": round(2 * m * p.k * p.n / us / 1e6, 2)})
            del g
    for row in sweep:
        if row["m"] == ROWS:
            log(f"  M=22 K={row['k']} N={row['n']}: {row['us']} us, {row['gbs']} GB/s")
    # The CPU-runnable configuration's product: bf16 output [22][4096] as
    # that configuration states it (vx_q8_linear_bf16), and beside it the
    # float32 output of the sweep's launches.
    count = max(single.copies, 64)
    g = graph_of(torch, stream, lambda _i: single.launch_bf16(ops, scratch, ROWS), count)
    g.replay()
    us = time_graph(torch, stream, g) / count * 1e6
    del g
    g = graph_of(torch, stream, lambda _i: single.launch(ops, scratch, ROWS), count)
    g.replay()
    us_f32 = time_graph(torch, stream, g) / count * 1e6
    del g
    single_row = {"m": ROWS, "k": single.k, "n": single.n, "output": "bf16",
                  "us": round(us, 3),
                  "gbs": round(single.bytes / us / 1e3, 1),
                  "hbm_frac": round(single.bytes / us / 1e3 / HBM_PEAK_GBS, 4),
                  "us_f32_output": round(us_f32, 3)}
    log(f"  single product M=22 K={single.k} N={single.n}, bf16 output: {us:.3f} us, "
        f"{single.bytes / us / 1e3:.1f} GB/s (float32 output {us_f32:.3f} us)")
    del single
    # The per-launch read ceiling: each shape's bytes, rotated and replayed
    # from a HIP graph the same way, read once with no arithmetic
    # (vx_stream_read): what one launch of that size can reach on this GPU.
    sink = torch.zeros(1, dtype=torch.int32, device=device)
    ceiling = []
    for p in products:
        count = max(p.copies, 64)
        g = graph_of(torch, stream,
                     lambda i, p=p: ops.stream_read(p.pool[i % p.copies], sink), count)
        g.replay()
        us = time_graph(torch, stream, g) / count * 1e6
        ceiling.append({"k": p.k, "n": p.n, "us": round(us, 3),
                        "gbs": round(p.bytes / us / 1e3, 1)})
        log(f"  read ceiling K={p.k} N={p.n}: {us:.3f} us, {p.bytes / us / 1e3:.1f} GB/s")
        del g
    launches = 4 * args.steps
    result = {
        "value": value,
        "seconds": seconds,
        "step_bytes": step_bytes,
        "launch_bytes": step_bytes / 4,
        "launch_us": seconds / launches * 1e6,
        "sweep": sweep,
        "single": single_row,
        "ceiling": ceiling,
    }
    del products
    torch.cuda.empty_cache()
    return result


def gpu_lm(args, torch, ops, synth, device, stream):
    """The decode shapes at 1 and 5 rows, MALL-cold (rotated copies),
    graph-replayed like the sweep; beside each the plain-read ceiling."""
    scratch = ops.Scratch(128, 16384)
    sink = torch.zeros(1, dtype=torch.int32, device=device)
    rows_out = []
    for name, k, n in LM_SHAPES:
        p = Product(ops, synth, torch, device, k, n, seed=1, rows=LM_ROWS)
        count = max(p.copies, 64)
        g = graph_of(torch, stream,
                     lambda i, p=p: ops.stream_read(p.pool[i % p.copies], sink), count)
        g.replay()
        read_us = time_graph(torch, stream, g) / count * 1e6
        del g
        for m in LM_ROWS:
            g = graph_of(torch, stream, lambda _i, p=p, m=m: p.launch(ops, scratch, m), count)
            g.replay()
            us = time_graph(torch, stream, g) / count * 1e6
            del g
            rows_out.append({"name": name, "m": m, "k": k, "n": n, "us": round(us, 3),
                             "gbs": round(p.bytes / us / 1e3, 1),
                             "hbm_frac": round(p.bytes / us / 1e3 / HBM_PEAK_GBS, 4),
                             "read_ceiling_us": round(read_us, 3)})
            log(f"  {name} M={m}: {us:.3f} us, {p.bytes / us / 1e3:.1f} GB/s "
                f"(read ceiling {read_us:.3f} us)")
        del p
        torch.cuda.empty_cache()
    # Product time of one base-LM step (28 layers) and one residual-LM step
    # (8 layers) at one row, from the per-shape figures.
    layer_us = sum(r["us"] for r in rows_out if r["m"] == 1 and r["name"].startswith("lm "))
    layer_bytes = sum(q8_bytes(k, n) for name, k, n in LM_SHAPES if name.startswith("lm "))
    return {"shapes": rows_out, "lm_layer_us_m1": round(layer_us, 3),
            "lm_layer_gbs_m1": round(layer_bytes / layer_us / 1e3, 1),
            "base_lm_products_us_m1": round(28 * layer_us, 1),
            "residual_lm_products_us_m1": round(8 * layer_us, 1)}


def device_stack_weights(torch, synth, config, device, seed: int):
    """Random weights of a stack's shape made on the device (GGML Q8_0
    blocks: int8 uniform in [-127, 127], float16 scales |N(0, 0.02)| / 127;
    norms bf16(1 + N(0, 0.02))): the decode benchmark's 28 distinct layers
    (1.4 GB) without host generation."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)

    def blocks(n, k):
        kb = k // 32
        q = torch.randint(-127, 128, (n, kb, 32), dtype=torch.int8, device=device,
                          generator=gen)
        scale = (torch.randn((n, kb), device=device, generator=gen).abs() * (0.02 / 127))
        out = torch.empty((n, kb, 34), dtype=torch.uint8, device=device)
        out[..., :2] = scale.to(torch.float16).view(torch.uint8).view(n, kb, 2)
        out[..., 2:] = q.view(torch.uint8)
        return out

    def norm(width):
        values = 1.0 + 0.02 * torch.randn(width, device=device, generator=gen)
        return values.to(torch.bfloat16).view(torch.int16)

    h = config.hidden
    layers = [{"input_norm": norm(h), "qkv": blocks(config.qkv_width, h),
               "o": blocks(h, config.q_width), "post_norm": norm(h),
               "gate_up": blocks(2 * config.ffn, h), "down": blocks(h, config.ffn)}
              for _ in range(config.layers)]
    return synth.StackWeightsHost(config, layers, norm(h))


def stack_bytes(config, rows_keys: int) -> int:
    """Algorithmic bytes of one forward: every layer's Q8_0 weights read
    once, plus the float32 keys and values the rows attend to."""
    layer = (q8_bytes(config.hidden, config.qkv_width) + q8_bytes(config.q_width, config.hidden)
             + q8_bytes(config.hidden, 2 * config.ffn) + q8_bytes(config.ffn, config.hidden))
    cache = 2 * config.kv_heads * rows_keys * config.head_dim * 4
    return config.layers * (layer + cache)


def gpu_lm_step(args, torch, ops, synth, device, stream):
    """One decode step of VoxCPM2's base LM (28 layers, one row at `past`
    cached positions), of the residual LM (8 layers, no rotary embedding)
    and one encoder call (12 layers, one 5-row patch), each on its fused and
    per-kernel paths; eager launches, inputs and caches resident."""
    from voxcpm_amd import _lib
    rope = ops.rope_table(10000.0, 128, synth.VOXCPM2_SHORT_FACTORS, 1.0, 8192)
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    out = {}
    cases = [("base_lm", synth.VOXCPM2_BASE_LM, 1, [128, 1024, 4096]),
             ("residual_lm", synth.VOXCPM2_RESIDUAL_LM, 1, [1024]),
             ("encoder", synth.VOXCPM2_ENCODER, 5, [0])]
    for name, config, rows, pasts in cases:
        weights = device_stack_weights(torch, synth, config, device, 7)
        stack = ops.Stack(weights, rope if config.rope else None, device, stream)
        del weights
        capacity = max(pasts) + rows + 1
        k, v = stack.cache(capacity)
        k.normal_()
        v.normal_()
        hidden0 = torch.randn((rows, config.hidden), dtype=torch.float32, device=device)
        hidden = hidden0.clone()
        output = torch.empty_like(hidden)
        entry = {}
        for past in pasts:
            causal = rows == 1
            positions = torch.arange(past, past + rows, dtype=torch.int32, device=device) \
                if causal else torch.arange(rows, dtype=torch.int32, device=device)
            for path_name, path in (("fused", _lib.STACK_PATH_AUTO),
                                    ("unfused", _lib.STACK_PATH_UNFUSED)):
                stack.set_path(path)

                def once():
                    hidden.copy_(hidden0)
                    stack.forward(hidden, output, positions, positions, rows, rows, past,
                                  causal, k, v, stream)

                for _ in range(3):
                    once()
                torch.cuda.synchronize()
                steps = max(10, args.steps // 2)
                start.record(stream)
                for _ in range(steps):
                    once()
                stop.record(stream)
                stop.synchronize()
                us = start.elapsed_time(stop) * 1e3 / steps
                keys = past + (1 if causal else rows)
                nbytes = stack_bytes(config, rows * keys)
                entry[f"{path_name}_past{past}"] = {
                    "us": round(us, 1), "bytes": nbytes,
                    "gbs": round(nbytes / us / 1e3, 1),
                    "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
                log(f"  {name} rows {rows} past {past} {path_name}: {us:.1f} us "
                    f"({nbytes / us / 1e3:.0f} GB/s of weights + cache)")
        out[name] = {"layers": config.layers, "rows": rows, **entry}
        stack.close()
        del stack, k, v
        torch.cuda.empty_cache()
    return out


def device_vae_weights(torch, synth, config, device, seed: int):
    """AudioVAE decoder weights of `config` made on the device with the
    scales of synth.vae_weights (1/sqrt(fan-in) products, Snake alphas
    near 1)."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)

    def normal(shape, std):
        return torch.randn(shape, device=device, generator=gen) * std

    def alpha(c):
        return (1.0 + normal((c,), 0.1)).abs() + 0.05

    t = {"in_depthwise": normal((config.latent, 7), 7 ** -0.5),
         "in_depthwise_bias": normal((config.latent,), 0.02),
         "in_pointwise": normal((config.decoder_dim, config.latent), config.latent ** -0.5),
         "in_pointwise_bias": normal((config.decoder_dim,), 0.02), "blocks": []}
    for b, s in enumerate(config.rates):
        c_in, c_out = config.channels(b)
        units = [{"alpha_in": alpha(c_out), "depthwise": normal((c_out, 7), 7 ** -0.5),
                  "depthwise_bias": normal((c_out,), 0.02), "alpha_out": alpha(c_out),
                  "pointwise": normal((c_out, c_out), 0.5 * c_out ** -0.5),
                  "pointwise_bias": normal((c_out,), 0.02)} for _ in range(3)]
        t["blocks"].append({"stride": s, "scale": 1.0 + normal((c_in,), 0.05),
                            "bias": normal((c_in,), 0.05), "alpha": alpha(c_in),
                            "up": normal((c_in, c_out, 2 * s), (2 * c_in) ** -0.5),
                            "up_bias": normal((c_out,), 0.02), "units": units})
    c_last = config.channels(len(config.rates) - 1)[1]
    t["out_alpha"] = alpha(c_last)
    t["out_conv"] = normal((c_last, 7), (7 * c_last) ** -0.5)
    t["out_bias"] = 0.01
    return synth.VaeWeightsHost(config, t)


def vae_weight_bytes(config) -> int:
    """float32 weight bytes one chunk reads: every matrix once (the
    transposed convolutions as their repacked [s out][2 in] products)."""
    total = config.latent * 7 + config.decoder_dim * config.latent
    for b, s in enumerate(config.rates):
        c_in, c_out = config.channels(b)
        total += s * c_out * 2 * c_in + 3 * (c_out * c_out + c_out * 7)
    return 4 * total


def gpu_vae(args, torch, ops, synth, device, stream):
    """AudioVAE V2's decoder on each patch's 4 latent frames (VoxCPM2's
    shape: 2048 channels, rates 8 6 5 2 2 2: 7680 samples at 48 kHz per
    patch), the same chunk buffers replayed as one graph."""
    config = synth.VOXCPM2_VAE
    weights = device_vae_weights(torch, synth, config, device, 11)
    vae = ops.Vae(weights, device, stream)
    chunk = torch.randn((4, config.latent), dtype=torch.float32, device=device)
    samples = torch.empty(4 * config.hop, dtype=torch.float32, device=device)
    # 0.2 s of untimed decodes first, as for the prefill replays: the
    # shader clock ramps up over the first milliseconds of work.
    begin = time.perf_counter()
    while time.perf_counter() - begin < 0.2:
        for _ in range(10):
            vae.decode(chunk, samples, stream)
        torch.cuda.synchronize()
    patches = max(10, args.steps)
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(patches):
        vae.decode(chunk, samples, stream)
    stop.record(stream)
    stop.synchronize()
    us = start.elapsed_time(stop) * 1e3 / patches
    nbytes = vae_weight_bytes(config)
    log(f"AudioVAE decode of one patch (4 frames, {4 * config.hop} samples): {us:.1f} us, "
        f"{nbytes / 1e6:.1f} MB of float32 weights, {nbytes / us / 1e3:.0f} GB/s")
    vae.close()
    return {"us_per_patch": round(us, 1), "frames": 4, "samples": 4 * config.hop,
            "weight_bytes": nbytes, "gbs": round(nbytes / us / 1e3, 1),
            "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
            "realtime_factor": round(4 * config.hop / 48000 / (us * 1e-6), 1)}


def gpu_bf16(args, torch, ops, synth, device, stream):
    """The sweep shapes at M=22 on bf16 weights (2 N K bytes): panels
    (vx_bf16_linear) and rows as they come (vx_bf16_linear_rows), rotated
    over >= 1 GiB per shape and replayed from HIP graphs."""
    scratch = ops.Scratch(128, 16384)
    rows = []
    for k, n in SWEEP_SHAPES:
        rng = synth.Rng(2, k * 31 + n)
        w = torch.from_numpy(synth.bf16_bits(rng.normal(n * k).astype(np.float32))
                             .view(np.int16).reshape(n, k)).to(device).view(torch.bfloat16)
        x = torch.from_numpy(synth.activations(rng, ROWS, k).view(np.int16)).to(device) \
            .view(torch.bfloat16)
        y = torch.empty((ROWS, n), dtype=torch.float32, device=device)
        weight_bytes = 2 * n * k
        copies = max(8, int(np.ceil(ROTATION_BYTES / weight_bytes)))
        entry = {"m": ROWS, "k": k, "n": n, "bytes": weight_bytes}
        packed = ops.bf16_pack(w)
        for name, pool, call in (
                ("panels", packed.repeat(copies).view(copies, -1),
                 lambda i, pool: ops.bf16_linear(x, pool[i % copies], n, y=y, scratch=scratch)),
                ("rows", w.repeat(copies, 1).view(copies, n, k),
                 lambda i, pool: ops.bf16_linear_rows(x, pool[i % copies], y=y))):
            count = max(copies, 64)
            g = graph_of(torch, stream, lambda i, pool=pool, call=call: call(i, pool), count)
            g.replay()
            us = time_graph(torch, stream, g) / count * 1e6
            entry[f"us_{name}"] = round(us, 3)
            entry[f"gbs_{name}"] = round(weight_bytes / us / 1e3, 1)
            del g, pool
            torch.cuda.empty_cache()
        log(f"  bf16 M=22 K={k} N={n}: panels {entry['us_panels']} us "
            f"({entry['gbs_panels']} GB/s), rows {entry['us_rows']} us "
            f"({entry['gbs_rows']} GB/s)")
        rows.append(entry)
    return rows


def gpu_prefill(args, torch, ops, synth, device, stream):
    """Prefill-sized Q8_0 products (m > 128, matrix-core bound): TFLOP/s of
    2 m n k per launch, launches replayed from a HIP graph over a few
    rotating weight copies."""
    import ctypes

    from voxcpm_amd import _lib

    def prefill_kernel(m: int, k: int, n: int, scratch) -> str:
        """The kernel vx_q8_linear's dispatch picks (vx_q8_prefill_plan)."""
        plan = (ctypes.c_int32 * 4)()
        _lib.check(_lib.lib().vx_q8_prefill_plan(m, k, n, scratch.handle, plan))
        names = {0: "TiledKernel (q8_tiled.hip)", 1: "GemmKernel (q8_gemm.hip)",
                 2: "EngineKernel in blocks of 64 rows (q8_tile.hpp)"}
        split = f", k split {plan[3]} ways" if plan[3] > 1 else ""
        return names[plan[0]] + split

    rows = []
    k = PREFILL_K
    # The product scratch (as the reference's Bf16Gemm owns its workspace):
    # small grids split k into its partial-sum area.
    scratch = ops.Scratch(128, 16384)
    for n in PREFILL_N:
        rng = synth.Rng(7, n)
        blocks = torch.from_numpy(synth.q8_blocks(rng, n, k)).to(device)
        packed = ops.q8_pack(blocks, n, k)
        copies = 4
        pool = packed.repeat(copies).view(copies, -1)
        del blocks
        for m in PREFILL_M:
            x = torch.from_numpy(synth.activations(rng, m, k).view(np.int16)).to(
                device).view(torch.bfloat16)
            y = torch.empty((m, n), dtype=torch.float32, device=device)
            ops.q8_linear(x, pool[0], n, y=y, scratch=scratch)
            count = 20
            g = graph_of(torch, stream,
                         lambda i: ops.q8_linear(x, pool[i % copies], n, y=y, scratch=scratch),
                         count)
            # Median of five replays after 0.2 s of untimed ones: the
            # products follow seconds of host-side weight generation, and
            # the first milliseconds of matrix-core work after an idle GPU
            # run slower than a prefill's steady state.
            seconds = time_graph(torch, stream, g, repeats=5, warm_seconds=0.2) / count
            tflops = 2.0 * m * n * k / seconds / 1e12
            rows.append({"m": m, "k": k, "n": n, "us": round(seconds * 1e6, 2),
                         "tflops": round(tflops, 1),
                         "mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                         "kernel": prefill_kernel(m, k, n, scratch)})
            log(f"  prefill M={m} K={k} N={n}: {seconds * 1e6:.1f} us, {tflops:.1f} TFLOP/s")
            del g
        del pool, packed
    torch.cuda.empty_cache()
    return rows


def prefill_workload(torch, ops, synth, device, stream) -> None:
    """Eager launches for counter runs of the prefill kernel: five products
    each at m = 512 and 1024 rows, k 2048, n 16384 (the MFMA-bound end of
    the prefill sweep), weights rotated over four copies."""
    k, n = PREFILL_K, 16384
    rng = synth.Rng(7, n)
    packed = ops.q8_pack(torch.from_numpy(synth.q8_blocks(rng, n, k)).to(device), n, k)
    pool = packed.repeat(4).view(4, -1)
    scratch = ops.Scratch(128, 16384)
    for m in (512, 1024):
        x = torch.from_numpy(synth.activations(rng, m, k).view(np.int16)).to(
            device).view(torch.bfloat16)
        y = torch.empty((m, n), dtype=torch.float32, device=device)
        for i in range(5):
            ops.q8_linear(x, pool[i % 4], n, y=y, scratch=scratch)
        torch.cuda.synchronize()
        log(f"prefill workload M={m} K={k} N={n}: 5 launches")


def pmc_workload(torch, ops, synth, device, stream) -> None:
    """Eager launches for counter runs: a plain 256 MiB device copy (the
    calibration of FETCH_SIZE / WRITE_SIZE against known bytes), then 20
    launches of each M=22 sweep shape on rotating copies."""
    src = torch.ones(1 << 25, dtype=torch.int64, device=device)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    scratch = ops.Scratch(128, 16384)
    products = [Product(ops, synth, torch, device, k, n, seed=0) for k, n in SWEEP_SHAPES]
    for p in products:
        for _ in range(20):
            p.launch(ops, scratch, ROWS)
    torch.cuda.synchronize()
    log("pmc workload done: 5 copies of 256 MiB, 20 launches per sweep shape")


def gpu_patch(args, torch, ops, synth, device, stream):
    config = synth.SYNTHETIC_DIT
    log("building the synthetic DiT (12 blocks, 214 MB of Q8_0)")
    rope = ops.rope_table(config.rope_theta, config.head_dim, config.rope_factors,
                          config.rope_scaling, 3 + 2 * config.patch)
    weights = synth.dit_weights(config, 3, rope)
    dit = ops.Dit(weights, device, stream)
    inputs = synth.patch_inputs(config, 4)
    t, dt, evaluate = ops.euler_schedule(config.steps, config.sway, config.skip)
    mu = torch.from_numpy(inputs.mu).to(device)
    cond = torch.from_numpy(inputs.cond_latent).to(device)
    x = torch.from_numpy(inputs.noise).to(device)
    for _ in range(max(2, args.warmup)):
        dit.patch(mu, cond, x, t, dt, evaluate, config.cfg, config.zero_star)
    torch.cuda.synchronize()
    patches = max(5, args.steps)
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(patches):
        dit.patch(mu, cond, x, t, dt, evaluate, config.cfg, config.zero_star)
    stop.record(stream)
    stop.synchronize()
    warm_us = start.elapsed_time(stop) * 1e3 / patches
    # MALL-cold: a 1 GiB read between patches evicts the weights.
    flush = torch.ones(1 << 27, dtype=torch.int64, device=device)
    cold = []
    for _ in range(5):
        flush.sum()
        start.record(stream)
        dit.patch(mu, cond, x, t, dt, evaluate, config.cfg, config.zero_star)
        stop.record(stream)
        stop.synchronize()
        cold.append(start.elapsed_time(stop) * 1e3)
    cold_us = float(np.median(cold))
    # The persistent evaluation (one launch per Euler step, grid barriers
    # between the layer's phases), selected explicitly.
    from voxcpm_amd import _lib
    default_path = dit.path
    dit.set_path(_lib.DIT_PATH_PERSISTENT)
    for _ in range(2):
        dit.patch(mu, cond, x, t, dt, evaluate, config.cfg, config.zero_star)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(patches):
        dit.patch(mu, cond, x, t, dt, evaluate, config.cfg, config.zero_star)
    stop.record(stream)
    stop.synchronize()
    dit.status()
    persistent_us = start.elapsed_time(stop) * 1e3 / patches
    # The per-kernel evaluation (the reference's launch sequence and norm
    # rounding order), selected explicitly.
    dit.set_path(_lib.DIT_PATH_UNFUSED)
    for _ in range(2):
        dit.patch(mu, cond, x, t, dt, evaluate, config.cfg, config.zero_star)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(patches):
        dit.patch(mu, cond, x, t, dt, evaluate, config.cfg, config.zero_star)
    stop.record(stream)
    stop.synchronize()
    unfused_us = start.elapsed_time(stop) * 1e3 / patches
    # The fused kernels in the reference's norm rounding order.
    dit.set_path(_lib.DIT_PATH_FUSED_REFERENCE_ORDER)
    for _ in range(2):
        dit.patch(mu, cond, x, t, dt, evaluate, config.cfg, config.zero_star)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(patches):
        dit.patch(mu, cond, x, t, dt, evaluate, config.cfg, config.zero_star)
    stop.record(stream)
    stop.synchronize()
    reference_order_us = start.elapsed_time(stop) * 1e3 / patches
    dit.set_path(_lib.DIT_PATH_AUTO)
    dit.close()
    # The same DiT on bf16 weights (bf16(scale q) panels, twice the bytes).
    dit_bf16 = ops.Dit(weights, device, stream, bf16_weights=True)
    for _ in range(2):
        dit_bf16.patch(mu, cond, x, t, dt, evaluate, config.cfg, config.zero_star)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(patches):
        dit_bf16.patch(mu, cond, x, t, dt, evaluate, config.cfg, config.zero_star)
    stop.record(stream)
    stop.synchronize()
    dit_bf16.status()
    bf16_us = start.elapsed_time(stop) * 1e3 / patches
    dit_bf16.close()
    # Algorithmic bytes of a patch: 10 evaluations x 12 blocks of weights,
    # in/out projections per evaluation and cond_proj once; the time MLP is
    # cached per t and not counted.
    block = (q8_bytes(config.hidden, config.qkv_width) + q8_bytes(config.q_width, config.hidden)
             + q8_bytes(config.hidden, 2 * config.ffn) + q8_bytes(config.ffn, config.hidden))
    io = q8_bytes(config.feat, config.hidden) + q8_bytes(config.hidden, config.feat)
    evaluations = int(np.sum(evaluate))
    patch_bytes = evaluations * (config.layers * block + io) + q8_bytes(config.feat, config.hidden)
    log(f"patch: {warm_us:.1f} us warm, {cold_us:.1f} us cold "
        f"({patch_bytes / 1e6:.1f} MB of weights per patch); "
        f"persistent evaluation {persistent_us:.1f} us; per-kernel {unfused_us:.1f} us; "
        f"fused in the reference's norm order {reference_order_us:.1f} us; "
        f"bf16 weights {bf16_us:.1f} us warm")
    gpu_patch.weights = weights
    return {"us_warm": round(warm_us, 2), "us_cold": round(cold_us, 2),
            "us_warm_persistent": round(persistent_us, 2),
            "us_warm_per_kernel": round(unfused_us, 2),
            "us_warm_fused_reference_order": round(reference_order_us, 2),
            "us_warm_bf16_weights": round(bf16_us, 2),
            "patches_timed": patches, "evaluations": evaluations,
            "bytes": patch_bytes,
            "gbs_warm": round(patch_bytes / warm_us / 1e3, 1),
            "gbs_cold": round(patch_bytes / cold_us / 1e3, 1),
            "roofline_us": round(patch_bytes / HBM_PEAK_GBS / 1e3, 1),
            "hbm_frac_cold": round(patch_bytes / cold_us / 1e3 / HBM_PEAK_GBS, 4),
            "workload": "12 blocks hidden 1024, 16 heads x 64, SwiGLU 4096, "
                        "22 rows (CFG pair x 11), 10 uniform Euler steps, CFG 2.0",
            "path": "us_warm and us_cold: the default (AUTO) path, "
                    f"{PATH_NAMES[default_path]}; us_warm_persistent, us_warm_per_kernel and "
                    "us_warm_fused_reference_order the other paths, selected explicitly"}


PATH_NAMES = {
    1: "PERSISTENT (one launch per evaluation, grid barriers between the phases)",
    2: "FUSED (five launches per layer: qkv from the producers' norm operand, "
       "attention, o + residual, gate_up + SwiGLU, down + residual)",
    3: "UNFUSED (the reference's launch sequence)",
    4: "FUSED_REFERENCE_ORDER (the fused launches with the norms before the products' "
       "bf16 rounding)",
}


def dit_workload(torch, ops, synth, device, stream) -> None:
    """Eager launches for counter runs of the DiT's fused kernels: twenty
    evaluations of the synthetic 12-block DiT on the default path (the
    weights stay in the 256 MB MALL across evaluations, as within a
    patch), after five untimed ones."""
    config = synth.SYNTHETIC_DIT
    rope = ops.rope_table(config.rope_theta, config.head_dim, config.rope_factors,
                          config.rope_scaling, 3 + 2 * config.patch)
    weights = synth.dit_weights(config, 3, rope)
    dit = ops.Dit(weights, device, stream)
    inputs = synth.patch_inputs(config, 4)
    mu = torch.from_numpy(inputs.mu).to(device)
    cond = torch.from_numpy(inputs.cond_latent).to(device)
    x = torch.from_numpy(inputs.noise).to(device)
    for _ in range(25):
        dit.velocity(mu, cond, x, 0.63)
    torch.cuda.synchronize()
    log(f"DiT workload done: 25 evaluations on path {dit.path}")
    dit.close()


def dit_trace(torch, ops, synth, device, stream) -> None:
    """The persistent evaluation's per-phase timeline (vx_dit_set_trace):
    one traced evaluation of the synthetic 12-block DiT after warm-up; per
    phase kind, the mean over layers of the workgroups' times from leaving
    the previous barrier to their products done (mean and latest workgroup)
    and to their stores done (latest), the phase's critical time (first
    workgroup out of the previous barrier to the last one in at the next),
    and the barrier's own time (last arrival to first and last exit).
    Printed as a table to stderr."""
    from voxcpm_amd import _lib
    config = synth.SYNTHETIC_DIT
    rope = ops.rope_table(config.rope_theta, config.head_dim, config.rope_factors,
                          config.rope_scaling, 3 + 2 * config.patch)
    weights = synth.dit_weights(config, 3, rope)
    dit = ops.Dit(weights, device, stream)
    inputs = synth.patch_inputs(config, 4)
    mu = torch.from_numpy(inputs.mu).to(device)
    cond = torch.from_numpy(inputs.cond_latent).to(device)
    x = torch.from_numpy(inputs.noise).to(device)
    dit.set_path(_lib.DIT_PATH_PERSISTENT)
    for _ in range(5):
        dit.velocity(mu, cond, x, 0.63)
    torch.cuda.synchronize()
    trace = dit.set_trace(True)
    for _ in range(3):
        dit.velocity(mu, cond, x, 0.63)
        torch.cuda.synchronize()
    dit.status()
    layers = config.layers
    barriers = 1 + 5 * layers
    tr = trace.cpu().numpy().astype(np.float64)
    grid = tr.size // (4 * (barriers + 1))
    tr = tr.reshape(grid, barriers + 1, 4) / 100.0  # 100 MHz ticks -> us
    start = tr[:, 0, 0].min()
    span = tr[:, 0, 1].max() - start
    kinds = ["qkv", "attention", "o", "gate_up", "down"]
    rows = {name: [] for name in ["input assembly"] + kinds}
    for b in range(1, barriers + 1):
        arrive, leave, products, stores = (tr[:, b, i] for i in range(4))
        previous = tr[:, b - 1, 1] if b > 1 else tr[:, 0, 0]
        kind = "input assembly" if b == 1 else kinds[(b - 2) % 5]
        rows[kind].append(((products - previous).mean(), (products - previous).max(),
                           (stores - previous).max(), arrive.max() - previous.min(),
                           leave.min() - arrive.max(), leave.max() - arrive.max()))
    log(f"persistent evaluation: {grid} workgroups, {span:.2f} us per evaluation, "
        f"{span / layers:.2f} us per layer")
    log("| phase | products done, mean (us) | products done, latest | stores done, latest | "
        "critical | barrier to first exit | barrier to last exit |")
    log("|---|---|---|---|---|---|---|")
    total = 0.0
    for name, values in rows.items():
        mean = np.mean(np.array(values), axis=0)
        if name != "input assembly":
            total += mean[3] + mean[4]
        log(f"| {name} | " + " | ".join(f"{v:.2f}" for v in mean) + " |")
    log(f"per layer, critical + barrier summed over the five phases: {total:.2f} us")
    dit.close()


def host_cores() -> int:
    """The cores this process may run on (its CPU affinity: the host's share
    given to this job), every one of which the CPU legs use."""
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:
        return max(1, os.cpu_count() or 1)


def cpu_baseline(synth):
    """The oracle's scalar products on the host's cores: a bounded sample
    (about 10 s) of the same M=22 workload."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib
    threads = host_cores()
    inputs = []
    for k, n in SWEEP_SHAPES:
        rng = synth.Rng(0, k * 31 + n)
        inputs.append((k, n, synth.q8_blocks(rng, n, k), synth.activations(rng, ROWS, k)))

    def rate(thread_count, seconds_per_shape, max_repeats):
        total_bytes = 0
        total_seconds = 0.0
        repeats = {}
        for k, n, blocks, x in inputs:
            count = 0
            start = time.perf_counter()
            while True:
                oracle_lib.q8_linear(x, blocks, n, threads=thread_count)
                count += 1
                elapsed = time.perf_counter() - start
                if elapsed > seconds_per_shape or count >= max_repeats:
                    break
            total_seconds += elapsed
            total_bytes += count * q8_bytes(k, n)
            repeats[f"{k}x{n}"] = count
        return total_bytes / total_seconds / 1e9, repeats, total_seconds

    value, repeats, seconds = rate(threads, 3.0, 400)
    log(f"CPU oracle: {value:.2f} GB/s on {threads} threads")
    single, single_repeats, single_seconds = rate(1, 2.0, 40)
    log(f"CPU oracle: {single:.3f} GB/s on 1 thread")
    return {"value": round(value, 3), "unit": "GB/s", "cores": threads,
            "host_cpu_count": os.cpu_count(), "kind": "port",
            "sample": "oracle Q8_0 x bf16 products, M=22, the four sweep shapes, "
                      f"repeats {repeats}, {seconds:.1f} s",
            "value_1_thread": round(single, 4),
            "sample_1_thread": f"the same shapes on one thread, repeats {single_repeats}, "
                               f"{single_seconds:.1f} s"}


def cpu_patch(synth):
    """One whole 10-step CFG patch of the oracle (the synthetic 12-block
    DiT: ten evaluations and their Euler steps, vo_dit_patch) on every host
    core, timed as one call."""
    import oracle_lib
    config = synth.SYNTHETIC_DIT
    threads = host_cores()
    weights = getattr(gpu_patch, "weights", None)
    if weights is None:
        rope = oracle_lib.rope_table(config.rope_theta, config.head_dim, None, 1.0, 11)
        weights = synth.dit_weights(config, 3, rope)
    dit = oracle_lib.OracleDit(weights, threads=threads)
    inputs = synth.patch_inputs(config, 4)
    t, dt, evaluate = oracle_lib.euler_schedule(config.steps, config.sway, config.skip)
    times = []
    for _ in range(CPU_PATCH_RUNS):
        start = time.perf_counter()
        dit.patch(inputs.mu, inputs.cond_latent, inputs.noise, t, dt, evaluate, config.cfg,
                  config.zero_star)
        times.append(time.perf_counter() - start)
    seconds = float(np.median(times))
    log(f"CPU oracle: one 10-step patch {seconds * 1e3:.0f} ms on {threads} threads "
        f"(median of {len(times)})")
    return {"us_per_patch": round(seconds * 1e6, 1), "cores": threads,
            "runs_us": [round(x * 1e6, 1) for x in times],
            "sample": f"one whole patch ({int(np.sum(evaluate))} evaluations), the median "
                      f"of {len(times)} runs"}


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--no-cpu", action="store_true",
                        help="skip the CPU baseline")
    parser.add_argument("--no-patch", action="store_true",
                        help="skip the DiT patch measurement")
    parser.add_argument("--no-bf16", action="store_true",
                        help="skip the bf16-weight products")
    parser.add_argument("--no-lm", action="store_true",
                        help="skip the LM decode shapes and steps and the AudioVAE")
    parser.add_argument("--no-prefill", action="store_true",
                        help="skip the prefill-sized products")
    parser.add_argument("--pmc-workload", action="store_true",
                        help="only run the eager launches that counter runs read")
    parser.add_argument("--prefill-workload", action="store_true",
                        help="only run eager prefill products (for counter runs)")
    parser.add_argument("--dit-workload", action="store_true",
                        help="only run eager DiT evaluations (for counter runs)")
    parser.add_argument("--dit-trace", action="store_true",
                        help="only print the persistent DiT evaluation's per-phase timeline")
    parser.add_argument("--lm-step-workload", action="store_true",
                        help="only run the stacks' decode steps and the AudioVAE "
                             "(for kernel traces)")
    parser.add_argument("--vae-workload", action="store_true",
                        help="only run the AudioVAE's patch decodes (for counter runs)")
    args = parser.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the DiT hot path runs one patch per "
              "GPU and this build has no multi-GPU path; run with --gpus 1.",
              file=sys.stderr)
        return 2

    import torch
    from voxcpm_amd import ops, synth

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    device = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=device)
    torch.cuda.set_stream(stream)
    log(f"device {torch.cuda.get_device_properties(0).gcnArchName}")
    if args.pmc_workload:
        pmc_workload(torch, ops, synth, device, stream)
        return 0
    if args.prefill_workload:
        prefill_workload(torch, ops, synth, device, stream)
        return 0
    if args.dit_trace:
        dit_trace(torch, ops, synth, device, stream)
        return 0
    if args.dit_workload:
        dit_workload(torch, ops, synth, device, stream)
        return 0
    if args.lm_step_workload:
        gpu_lm_step(args, torch, ops, synth, device, stream)
        gpu_vae(args, torch, ops, synth, device, stream)
        return 0
    if args.vae_workload:
        gpu_vae(args, torch, ops, synth, device, stream)
        return 0

    probe = read_probe(torch, device, stream)
    log(f"read probe {probe:.0f} GB/s")
    floor = gpu_launch_floor(torch, ops, device, stream)
    products = gpu_products(args, torch, ops, synth, device, stream)
    lm = None if args.no_lm else gpu_lm(args, torch, ops, synth, device, stream)
    if lm is not None:
        lm["steps"] = gpu_lm_step(args, torch, ops, synth, device, stream)
    vae = None if args.no_lm else gpu_vae(args, torch, ops, synth, device, stream)
    bf16 = None if args.no_bf16 else gpu_bf16(args, torch, ops, synth, device, stream)
    prefill = None if args.no_prefill else gpu_prefill(args, torch, ops, synth, device, stream)
    patch = None if args.no_patch else gpu_patch(args, torch, ops, synth, device, stream)
    baseline = None
    if not args.no_cpu:
        baseline = cpu_baseline(synth)
        if patch is not None:
            patch["cpu"] = cpu_patch(synth)

    value = products["value"]
    ceiling_gbs = products["step_bytes"] / sum(c["us"] for c in products["ceiling"]) / 1e3
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(products["seconds"] / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "Q8_0 x bf16 skinny products, M=22, (K,N) in "
                        "{(1024,3072),(1024,8192),(2048,2048),(2048,16384)}, "
                        "weights rotated over >= 1 GiB per shape, HIP-graph launches",
            "m": ROWS,
            "shapes": SWEEP_SHAPES,
            "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(products["launch_bytes"] / products["launch_us"] / 1e3, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(products["launch_bytes"] / products["launch_us"] / 1e3
                          / HBM_PEAK_GBS, 4),
            "traffic": round(sum(f * FETCH_SCALE + w for f, w in TRAFFIC_KIB.values())
                             * 1024 / len(TRAFFIC_KIB)),
            "traffic_source": "profiles/q8_skinny_m22_traffic.md, rocprofv3 PMC on the "
                              f"build of commit {TRAFFIC_BUILD}",
            "kernel": "EngineKernel<2, RG, kRowMajor, kStore, 1, 3> "
                      "(voxcpm_amd/csrc/q8_tile.hpp) via vx_q8_linear",
            "launch_bytes": products["launch_bytes"],
            "launch_us": round(products["launch_us"], 3),
            # The same bytes per launch read with no arithmetic, launched the
            # same way: the achievable per-launch ceiling (launch and memory
            # latency included) against which `value` is also quoted.
            "read_ceiling_gbs": round(ceiling_gbs, 1),
            "frac_of_read_ceiling": round(value / ceiling_gbs, 4),
            "read_ceiling": products["ceiling"],
        },
        "cpu_baseline": baseline,
        "read_probe_gbs": round(probe, 1),
        "launch_floor_us": floor["launch_floor_us"],
        "dependent_launch_us": floor["dependent_launch_us"],
        "launch_costs": floor,
        "sweep": products["sweep"],
        "single_product": products["single"],
        "lm_decode": lm,
        "vae_decode": vae,
        "bf16_weights": bf16,
        "prefill": prefill,
        "prefill_mfma_busy_counters": PREFILL_MFMA_BUSY,
        "patch": patch,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
