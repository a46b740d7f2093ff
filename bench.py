#!/usr/bin/env python3
"""Benchmark of the fovi hot path on one MI355X.

Primary line (``value``): the C3 large kNN-conv layer forward -- B=64,
16384 log-polar points in and out, k=25 (5x5 ref grid), 256 -> 256 channels,
bf16 operands with fp32 accumulation -- in TFLOP/s of algorithmic work
2*B*N_out*C_out*C_in*V, with its bf16-MFMA roofline fraction.

Alongside, in the same JSON line: the C4 foveated sampler (128 images
3x512x512 bf16, 4 fixations each = 512 views of 16384 points) in algorithmic
GB/s against HBM peak, and the CPU baseline (the oracle's torch-CPU
restatement of the reference op sequence on a bounded batch slice).

Inputs are synthetic (seeded) and resident in HBM before timing starts.
Timing: ``warmup`` untimed steps, then ``steps`` steps between HIP events on
the stream the kernels are launched on, bracketed by device synchronisation.
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0
PEAK_FP8_TFLOPS = 5000.0
PEAK_HBM_GBS = 8000.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def time_steps(fn, steps, warmup):
    """Median ms per step: ``warmup`` untimed steps, then ``steps`` steps, each between two HIP
    events recorded on torch's current stream (the stream every C-ABI call here is enqueued on),
    the whole timed region bracketed by device synchronisation (as fovi/utils/flops.py:279-417
    times GPU work: events around each iteration, median)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    times = sorted(a.elapsed_time(b) for a, b in ev)
    return times[len(times) // 2]


def cpu_randn(shape, seed, dtype=None, dev=None):
    """Seeded CPU normal draws moved to the device (portable across boxes)."""
    import torch
    t = torch.randn(*shape, generator=torch.Generator().manual_seed(seed))
    if dtype is not None:
        t = t.to(dtype)
    return t if dev is None else t.to(dev)


def cpu_rand(shape, seed, dtype=None, dev=None):
    """Seeded CPU uniform [0, 1) draws moved to the device."""
    import torch
    t = torch.rand(*shape, generator=torch.Generator().manual_seed(seed))
    if dtype is not None:
        t = t.to(dtype)
    return t if dev is None else t.to(dev)


def bench_c3(steps, warmup, dev):
    import torch
    from fovi_amd.arch.knn import KNNConvLayer
    from fovi_amd.sensing.coords import SamplingCoords
    B, C, K, RES = 64, 256, 25, 128
    t0 = time.time()
    coords = SamplingCoords(16, 2.78, RES, style="logpolar")
    layer = KNNConvLayer(C, C, K, coords, coords, device=dev)
    torch.cuda.synchronize()
    t_tables = time.time() - t0
    # the same layer once more: the per-layer cost without the process's first-use set-up
    # (library and kernel-module loads, the torch ops' first calls)
    t0 = time.time()
    KNNConvLayer(C, C, K, coords, coords, device=dev)
    torch.cuda.synchronize()
    t_warm = time.time() - t0
    log(f"[c3] layer and tables built in {t_tables:.2f}s first, {t_warm:.3f}s again (kNN search and ref slots "
        f"on the GPU: {layer._gpu_tables(RES * RES)}, {getattr(layer, 'slots_recomputed', None)} points' slots "
        f"recomputed on the host)")
    with torch.no_grad():
        layer.weight.copy_(cpu_randn(layer.weight.shape, 1, dev=dev) * (1.0 / (C * K)) ** 0.5)
    # channels-last storage [B, N, C], handed to the layer as the [B, C, N] view
    x = cpu_randn((B, RES * RES, C), 0, torch.bfloat16, dev).transpose(1, 2)
    with torch.no_grad():
        ms = time_steps(lambda: layer(x), steps, warmup)
    flops = 2.0 * B * RES * RES * C * C * layer.ref_coords.shape[0]
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"[c3] {ms:.3f} ms/step  {tflops:.1f} TFLOP/s  ({100 * tflops / PEAK_BF16_TFLOPS:.1f}% of bf16 peak)")
    return dict(ms=ms, flops=flops, tflops=tflops, layer=layer, x=x, table_s=t_tables, table_warm_s=t_warm)


def bench_c3_backward(c3, steps, warmup):
    """Backward of the C3 layer (input and weight gradients, bf16): dx as a kNN-conv forward
    over the inverse neighbour table (the wide-layer kernel), dW by the pair-list kernel
    (fovi_knnconv_dw, no slot-sum matrix). Reported against the two products' flops (2x the
    forward's)."""
    import torch
    layer, x = c3["layer"], c3["x"]
    n = layer.out_coords.shape[0]
    dy = cpu_randn((x.shape[0], n, layer.out_channels), 5, torch.bfloat16, x.device).transpose(1, 2)
    layer._inverse_tables(x.device)
    ms = time_steps(lambda: layer._backward(x, layer.weight, dy, True, True), steps, warmup)
    flops = 2.0 * c3["flops"]
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"[c3 backward] {ms:.3f} ms/step  {tflops:.1f} TFLOP/s over the two GEMMs "
        f"({100 * tflops / PEAK_BF16_TFLOPS:.1f}% of bf16 peak)")
    return dict(ms=ms, tflops=tflops)


def bench_c5(c3, steps, warmup):
    """C5: the C3 layer with e4m3 activations (per-tensor scale) and weights
    (per-output-channel scales), fp32 accumulation, bf16 output. The input is
    quantized once before timing (the layer's producer would emit e4m3); the
    quantizer is timed on its own."""
    import torch
    layer, x = c3["layer"], c3["x"]
    with torch.no_grad():
        xq = layer.quantize_input(x)
        ms = time_steps(lambda: layer(xq), steps, warmup)
        ms_q = time_steps(lambda: layer.quantize_input(x), steps, warmup)
    tflops = c3["flops"] / (ms * 1e-3) / 1e12
    # per-layer cosine of the bf16 output against the unquantized fp32 layer (the fp32 kernel at
    # B=64), for the layer's scale amax * headroom / 448 and the plain amax / 448
    from fovi_amd.arch.fp8 import quantize_e4m3

    def cos(a, b):
        a, b = a.double().flatten(), b.double().flatten()
        return (a @ b / (a.norm() * b.norm())).item()
    with torch.no_grad():
        y32 = layer(x.float())
        cos_layer = cos(layer(xq).float(), y32)
        cos_plain = cos(layer(quantize_e4m3(x, 1.0)).float(), y32)
        del y32
    # quantizer: amax pass reads x, quantize pass reads x and writes e4m3
    q_bytes = 2 * x.numel() * x.element_size() + x.numel()
    q_gbs = q_bytes / (ms_q * 1e-3) / 1e9
    log(f"[c5] {ms:.3f} ms/step  {tflops:.1f} TFLOP/s  ({100 * tflops / PEAK_FP8_TFLOPS:.1f}% of fp8 peak); "
        f"quantize {ms_q:.3f} ms ({q_gbs:.0f} GB/s); cosine vs fp32 {cos_layer:.6f} (headroom "
        f"{layer.fp8_headroom:g}), {cos_plain:.6f} (amax/448)")
    return dict(ms=ms, tflops=tflops, ms_q=ms_q, q_gbs=q_gbs, cos=cos_layer, cos_plain=cos_plain,
                headroom=layer.fp8_headroom)


def sampler_algorithmic_bytes(sampler, img, fix, sizes, vmap, mode):
    """Output bytes + sum over views of distinct in-bounds tap pixels x C x element size."""
    import torch
    _, grid = sampler.sample_views(img, fix, sizes, view_image=vmap, return_grid=True)
    n_img, C, H, W = img.shape
    ix = (grid[..., 0] + 1.0) * (W * 0.5) - 0.5
    iy = (grid[..., 1] + 1.0) * (H * 0.5) - 0.5
    taps = []
    if mode == "nearest":
        taps.append((torch.round(ix), torch.round(iy)))
    else:
        fx, fy = torch.floor(ix), torch.floor(iy)
        taps += [(fx, fy), (fx + 1, fy), (fx, fy + 1), (fx + 1, fy + 1)]
    V = grid.shape[0]
    view = torch.arange(V, device=grid.device).view(V, 1)
    keys = []
    for tx, ty in taps:
        ok = (tx >= 0) & (tx < W) & (ty >= 0) & (ty < H)
        k = view * (H * W) + ty.long() * W + tx.long()
        keys.append(k[ok])
    distinct = torch.unique(torch.cat(keys)).numel()
    es = img.element_size()
    out_bytes = V * C * grid.shape[1] * es
    return out_bytes + distinct * C * es, out_bytes, distinct


def bench_c4_sampler(steps, warmup, dev, mode="nearest", channels_last=False):
    """C4 sampler; ``channels_last``: the same images in torch's channels-last memory format
    (the layout image decoders produce), whose taps read all channels of a pixel at once."""
    import numpy as np
    import torch
    from fovi_amd.sensing.samplers import GridSampler
    B, Fx, RES, S = 128, 4, 128, 512
    # two image sets (2 x 201 MB) rotated so the 256 MB MALL cannot hold the input
    imgs = [cpu_rand((B, 3, S, S), i, torch.bfloat16, dev) for i in range(2)]
    if channels_last:
        imgs = [x.contiguous(memory_format=torch.channels_last) for x in imgs]
    gf = torch.Generator().manual_seed(2)
    fix = 0.25 + 0.5 * torch.rand(B * Fx, 2, generator=gf)
    sizes = np.array([[S, S]] * (B * Fx))
    vmap = torch.arange(B).repeat_interleave(Fx)
    sampler = GridSampler(16, 2.78, RES, device=dev, mode=mode, style="logpolar")
    out = torch.empty(B * Fx, 3, RES * RES, device=dev, dtype=torch.bfloat16)
    state = {"i": 0}
    fix_d = fix.to(dev)
    views = sampler.prepare_views(fix_d, sizes, B, dev, view_image=vmap)

    def step():
        sampler.sample_views(imgs[state["i"] & 1], out=out, views=views)
        state["i"] += 1

    with torch.no_grad():
        ms = time_steps(step, steps, warmup)
        nbytes, out_bytes, distinct = sampler_algorithmic_bytes(sampler, imgs[0], fix_d, sizes, vmap, mode)
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"[c4 sampler {mode}{' channels-last' if channels_last else ''}] {ms:.3f} ms/step  {gbs:.0f} GB/s algorithmic "
        f"({100 * gbs / PEAK_HBM_GBS:.1f}% of HBM peak); bytes {nbytes / 1e6:.1f} MB "
        f"(out {out_bytes / 1e6:.1f} MB, {distinct} distinct taps)")
    return dict(ms=ms, bytes=nbytes, gbs=gbs, images_per_s=B / (ms * 1e-3))


def _init_weights(layers, dev, seed):
    """N(0, 1 / (C_in k)) weights (layer i drawn with seed + i), zero bias."""
    import torch
    with torch.no_grad():
        for i, c in enumerate(layers):
            c.weight.copy_(cpu_randn(c.weight.shape, seed + i, dev=dev) * (1.0 / (c.in_channels * c._k)) ** 0.5)
            if c.bias is not None:
                c.bias.zero_()


def bench_pool(steps, warmup, dev):
    """kNN max pooling of the reference AlexNet (pool after a conv block, knnalexnet.py:90-101):
    256 images, 64 channels on 1024 log-polar points -> 256 points, k=9, bf16 channels-last.
    Algorithmic bytes: every input row once (all are neighbours) plus the output."""
    import torch
    from fovi_amd.arch.knn import KNNPoolingLayer
    from fovi_amd.sensing.coords import SamplingCoords
    B, C = 256, 64
    ci = SamplingCoords(16, 2.78, 32, style="logpolar")
    co = SamplingCoords(16, 2.78, 16, style="logpolar")
    layer = KNNPoolingLayer(9, ci, co, mode="max", device=dev)
    x = cpu_randn((B, ci.shape[0], C), 3, torch.bfloat16, dev).transpose(1, 2)
    with torch.no_grad():
        ms = time_steps(lambda: layer(x), steps, warmup)
    nbytes = B * C * (ci.shape[0] + co.shape[0]) * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"[pool] {ms:.4f} ms/step  {gbs:.0f} GB/s algorithmic ({100 * gbs / PEAK_HBM_GBS:.1f}% of HBM peak); "
        f"bytes {nbytes / 1e6:.1f} MB")
    return dict(ms=ms, gbs=gbs, bytes=nbytes)


def bench_c2(steps, warmup, dev):
    """C2: 256 images 3x224x224 fp32 -> bilinear sampler (4096 log-polar points, bf16 out) ->
    5 kNN-conv layers 64/192/384/256/256, k=49/25/9/9/9, strides 2,2,1,1,1, ReLU between."""
    import numpy as np
    import torch
    from fovi_amd.arch.knnalexnet import KNNAlexNet
    from fovi_amd.sensing.samplers import GridSampler
    B, S = 256, 224
    t0 = time.time()
    net = KNNAlexNet(64, 3, [64, 192, 384, 256, 256], [2, 2, 1, 1, 1], [], [49, 25, 9, 9, 9], style="logpolar",
                     norm_type="none", fov=16, cmf_a=2.78, device=dev, final_activation=False)
    _init_weights([blk.conv for blk in net.layers], dev, 3)
    sampler = GridSampler(16, 2.78, 64, device=dev, mode="bilinear", style="logpolar")
    log(f"[c2] model built in {time.time() - t0:.1f}s")
    imgs = [cpu_rand((B, 3, S, S), i, dev=dev) for i in range(2)]
    views = sampler.prepare_views(torch.full((B, 2), 0.5), np.array([[S, S]] * B), B, dev)
    # the sampler writes the first layer's input rows padded to 4 channels, view-major (the rows
    # of one sensor point for all images adjacent): the layout its view-major kernel reads
    _, feats = net.layers[0].conv.padded_input(B, view_major=True)
    state = {"i": 0}

    def step():
        sampler.sample_views(imgs[state["i"] & 1], out=feats, views=views)
        state["i"] += 1
        return net(feats)

    with torch.no_grad():
        ms = time_steps(step, steps, warmup)
    flops = 0.0
    for blk in net.layers:
        c = blk.conv
        flops += 2.0 * B * c.out_coords.shape[0] * c.out_channels * c.in_channels * c.ref_coords.shape[0]
    ips = B / (ms * 1e-3)
    log(f"[c2] {ms:.3f} ms/step  {ips:.0f} images/s  ({flops / 1e9:.1f} GFLOP/batch, "
        f"{flops / (ms * 1e-3) / 1e12:.1f} TFLOP/s)")
    return dict(ms=ms, images_per_s=ips, gflop=flops / 1e9, tflops=flops / (ms * 1e-3) / 1e12)


def bench_c4_frontend(steps, warmup, dev):
    """C4: 128 images 3x512x512 bf16, 4 fixations each -> nearest sampler (16384 points) ->
    kNN patch embedding 3 -> 384 (k=256, 16x16 ref grid) onto 256 tokens, bias."""
    import numpy as np
    import torch
    from fovi_amd.arch.knnvit import KNNPatchEmbedding
    from fovi_amd.sensing.samplers import GridSampler
    B, Fx, S = 128, 4, 512
    t0 = time.time()
    pe = KNNPatchEmbedding(3, 384, 128, 16, 2.78, style="logpolar", auto_match_cart_resources=0,
                           cart_patch_size=16, patch_overlap_factor=2, new_parameterization=True, transposed=True,
                           sample_cortex=True, ref_frame_side_length=16, device=dev, bias=True)
    _init_weights([pe], dev, 4)
    sampler = GridSampler(16, 2.78, 128, device=dev, mode="nearest", style="logpolar")
    log(f"[c4] model built in {time.time() - t0:.1f}s")
    imgs = [cpu_rand((B, 3, S, S), i, torch.bfloat16, dev) for i in range(2)]
    gf = torch.Generator().manual_seed(2)
    fix = 0.25 + 0.5 * torch.rand(B * Fx, 2, generator=gf)
    views = sampler.prepare_views(fix, np.array([[S, S]] * (B * Fx)), B, dev,
                                  view_image=torch.arange(B).repeat_interleave(Fx))
    # the sampler writes the patch embedding's input view-major (the layout of its view-major
    # kernel); the point-major layout ([views, points, 4], the point-tile kernel) is timed too
    _, feats = pe.padded_input(B * Fx, view_major=True)
    _, feats_pm = pe.padded_input(B * Fx)
    state = {"i": 0}

    def step():
        sampler.sample_views(imgs[state["i"] & 1], out=feats, views=views)
        state["i"] += 1
        return pe(feats)

    def step_pm():
        sampler.sample_views(imgs[state["i"] & 1], out=feats_pm, views=views)
        state["i"] += 1
        return pe(feats_pm)

    # the drop-in policy path: near-centre fixations drawn on the host (numpy, the reference's
    # draw order), all B x F views sampled in one launch
    from fovi_amd.sensing.policies import MultiRandomSaccadePolicy
    from fovi_amd.sensing.retina import RetinalTransform
    rt = RetinalTransform(128, start_res=S, fov=16, cmf_a=2.78, style="logpolar", sampler="grid_nn", device=dev,
                          dtype=torch.bfloat16, auto_match_cart_resources=0)
    pol = MultiRandomSaccadePolicy(rt, n_fixations=Fx, norm_dist_from_center=0.25).eval()
    np.random.seed(2)

    def policy_step():
        out = pol(imgs[state["i"] & 1])
        state["i"] += 1
        return out

    with torch.no_grad():
        ms = time_steps(step, steps, warmup)
        ms_pe = time_steps(lambda: pe(feats), steps, warmup)
        ms_pm = time_steps(step_pm, steps, warmup)
        ms_pe_pm = time_steps(lambda: pe(feats_pm), steps, warmup)
        ms_pol = time_steps(policy_step, steps, warmup)
    flops = 2.0 * B * Fx * 256 * 384 * 3 * 256
    log(f"[c4] {ms:.3f} ms/step  {B / (ms * 1e-3):.0f} images/s  (patch embed alone {ms_pe:.3f} ms = "
        f"{flops / (ms_pe * 1e-3) / 1e12:.1f} TFLOP/s; point-major input {ms_pm:.3f} ms, patch embed "
        f"{ms_pe_pm:.3f} ms; policy draws + fused views {ms_pol:.3f} ms)")
    return dict(ms=ms, images_per_s=B / (ms * 1e-3), ms_patch_embed=ms_pe,
                patch_embed_tflops=flops / (ms_pe * 1e-3) / 1e12, ms_policy=ms_pol,
                ms_point_major=ms_pm, ms_patch_embed_point_major=ms_pe_pm)


def copy_probe(dev, mib=256, reps=3):
    """A plain device copy of known size (``mib`` MiB read + written per launch):
    the calibration kernel for rocprofv3 FETCH_SIZE / WRITE_SIZE counters."""
    import torch
    x = torch.empty(mib << 20, dtype=torch.uint8, device=dev)
    y = torch.empty_like(x)
    for _ in range(reps):
        y.copy_(x)
    torch.cuda.synchronize()
    log(f"[copy] {reps} copies of {mib} MiB")


def measured_traffic(kernel_prefix):
    """HBM bytes per launch of the named kernel from the committed rocprofv3
    counter summary (profiles/hbm_traffic.json), or None."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    k = rec.get("kernels", {}).get(kernel_prefix)
    return None if k is None else int(k["fetch_bytes"] + k["write_bytes"])


def _host_cores():
    """(cores this process may run on, os.cpu_count(), the CPU model)."""
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 1
    model = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return avail, os.cpu_count(), model


def cpu_baseline_c3(c3, runs=5, warmup=1):
    """The oracle (torch-CPU fp32 restatement of knn.py:484-557) on a B=1 slice of C3: ``warmup``
    untimed runs, then ``runs`` timed ones, median, scaled linearly to the batch. Threads: every
    core the process may run on."""
    import torch
    from oracle import knnconv_ref
    avail, total, model = _host_cores()
    torch.set_num_threads(avail)
    layer = c3["layer"]
    bs = 1
    x = c3["x"][:bs].float().cpu().contiguous()
    idx = layer.knn_indices.cpu()
    rf = layer.local_rf.cpu()
    w = layer.weight.detach().float().cpu()
    n_in = layer.in_coords.shape[0]
    for _ in range(warmup):
        knnconv_ref.knnconv_forward(x, idx, n_in, rf, w)
    times = []
    for _ in range(runs):
        t = time.time()
        knnconv_ref.knnconv_forward(x, idx, n_in, rf, w)
        times.append(time.time() - t)
    times.sort()
    med = times[len(times) // 2]
    flops = c3["flops"] * bs / 64
    log(f"[cpu] C3 slice B={bs}: runs {', '.join(f'{t:.2f}' for t in times)} s on {torch.get_num_threads()} "
        f"threads")
    return {"value": flops / med / 1e12, "unit": "TFLOP/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"C3 slice B={bs} of 64 (fp32 torch-CPU restatement of the reference op sequence, "
                      f"knn.py:484-557), {warmup} warmup + {runs} timed runs, median {med:.2f} s, scaled "
                      f"linearly in B; host {model}, {avail} cores available of os.cpu_count()={total}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-sampler", action="store_true")
    ap.add_argument("--no-e2e", action="store_true", help="skip the C2/C4 end-to-end legs")
    ap.add_argument("--no-fp8", action="store_true", help="skip the C5 fp8 leg")
    ap.add_argument("--only", default="", help="comma list of legs to run (c3,c5,bwd,sampler,pool,c2,c4,cpu,copy); "
                                                "for profiling runs, the JSON line then holds only those legs")
    args = ap.parse_args()
    if args.only:
        legs = set(args.only.split(","))
        unknown = legs - {"c3", "c5", "bwd", "sampler", "pool", "c2", "c4", "cpu", "copy"}
        if unknown:
            ap.error(f"unknown legs {sorted(unknown)}")
        if legs & {"c5", "cpu", "bwd"}:
            legs.add("c3")
        args.no_fp8 = "c5" not in legs
        args.no_sampler = "sampler" not in legs
        args.no_e2e = not (legs & {"c2", "c4"})
        args.no_cpu_baseline = "cpu" not in legs
    else:
        legs = {"c3", "c5", "bwd", "sampler", "pool", "c2", "c4", "cpu"}
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              f"(the forward would shard over the batch with no communication)", file=sys.stderr)
        sys.exit(2)
    import torch
    dev = torch.device("cuda:0")
    c3 = bench_c3(args.steps, args.warmup, dev) if "c3" in legs else None
    c5 = None if args.no_fp8 else bench_c5(c3, args.steps, args.warmup)
    bwd = bench_c3_backward(c3, args.steps, args.warmup) if "bwd" in legs else None
    c4 = None if args.no_sampler else bench_c4_sampler(args.steps, args.warmup, dev, "nearest")
    c4b = None if args.no_sampler else bench_c4_sampler(args.steps, args.warmup, dev, "bilinear")
    c4cl = None if args.no_sampler else bench_c4_sampler(args.steps, args.warmup, dev, "nearest", True)
    c4bcl = None if args.no_sampler else bench_c4_sampler(args.steps, args.warmup, dev, "bilinear", True)
    pool = bench_pool(args.steps, args.warmup, dev) if "pool" in legs else None
    c2 = None if args.no_e2e or "c2" not in legs else bench_c2(args.steps, args.warmup, dev)
    c4e = None if args.no_e2e or "c4" not in legs else bench_c4_frontend(args.steps, args.warmup, dev)
    cpu = None if args.no_cpu_baseline else cpu_baseline_c3(c3)
    if "copy" in legs and args.only:
        copy_probe(dev)
    if c3 is None:
        c3 = {"tflops": float("nan"), "ms": float("nan")}
    line = {
        "metric": "kNN-conv fwd TFLOP/s + sampler GB/s (% of MI355X roofline); images/sec",
        "value": round(c3["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c3["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded randn activations, N(0,1/(C_in*k)) weights)",
        "config": {"workload": "C3 large kNN-conv layer: B=64, N_in=N_out=16384 log-polar (a=2.78), "
                               "k=25, V=25, C_in=C_out=256, bf16 in/out, fp32 accumulate",
                   "batch": 64, "points": 16384, "k": 25, "c_in": 256, "c_out": 256},
        "roofline": {"bound": "mfma", "achieved": round(c3["tflops"], 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(c3["tflops"] / PEAK_BF16_TFLOPS, 4),
                     "traffic": measured_traffic("knnconv_bf16_v5_kernel")},
        "cpu_baseline": cpu,
    }
    if "table_s" in c3:
        line["c3_layer_build_s"] = {"first": round(c3["table_s"], 3), "again": round(c3["table_warm_s"], 3)}
    if c5 is not None:
        line["c5_fp8"] = {"workload": "C5: C3 layer with OCP e4m3 activations (per-tensor scale) and weights "
                                      "(per-output-channel scales), fp32 accumulate, bf16 out",
                          "TFLOP/s": round(c5["tflops"], 2), "ms": round(c5["ms"], 4),
                          "roofline": {"bound": "mfma", "peak": PEAK_FP8_TFLOPS, "unit": "TFLOP/s",
                                       "frac": round(c5["tflops"] / PEAK_FP8_TFLOPS, 4)},
                          "quantize_ms": round(c5["ms_q"], 4), "quantize_GB/s": round(c5["q_gbs"], 1),
                          "cosine_vs_fp32": {f"amax*{c5['headroom']:g}/448 (layer scale)": round(c5["cos"], 6),
                                             "amax/448": round(c5["cos_plain"], 6),
                                             "reference": "unquantized fp32 layer (fp32 kernel), B=64"}}
    if bwd is not None:
        line["c3_backward"] = {"workload": "C3 layer backward, bf16: input gradient (kNN-conv forward over the "
                                           "inverse table) and weight gradient (per-slot pair-list MFMA kernel)",
                               "ms": round(bwd["ms"], 4), "TFLOP/s": round(bwd["tflops"], 2)}
    def traffic_frac(kernel, ms):
        """HBM bytes per launch from the counter record, over the launch time, as a fraction of peak."""
        t = measured_traffic(kernel)
        return None if t is None else round(t / (ms * 1e-3) / (PEAK_HBM_GBS * 1e9), 4)

    if c4 is not None:
        line["sampler_c4"] = {
            "workload": "C4 sampler: 128 images 3x512x512 bf16, 4 fixations each (512 views), "
                        "16384 log-polar points, bf16 out",
            "nearest": {"GB/s": round(c4["gbs"], 1), "frac": round(c4["gbs"] / PEAK_HBM_GBS, 4),
                        "traffic_frac": traffic_frac("sampler_rings_kernel<bf16,nearest>", c4["ms"]),
                        "ms": round(c4["ms"], 4), "images/s": round(c4["images_per_s"], 1)},
            "bilinear": {"GB/s": round(c4b["gbs"], 1), "frac": round(c4b["gbs"] / PEAK_HBM_GBS, 4),
                         "traffic_frac": traffic_frac("sampler_rings_kernel<bf16,bilinear>", c4b["ms"]),
                         "ms": round(c4b["ms"], 4), "images/s": round(c4b["images_per_s"], 1)},
            "channels_last_images": {
                "nearest": {"GB/s": round(c4cl["gbs"], 1), "frac": round(c4cl["gbs"] / PEAK_HBM_GBS, 4),
                            "traffic_frac": traffic_frac("sampler_rings_kernel<bf16,nearest,channels_last>",
                                                         c4cl["ms"]),
                            "ms": round(c4cl["ms"], 4)},
                "bilinear": {"GB/s": round(c4bcl["gbs"], 1), "frac": round(c4bcl["gbs"] / PEAK_HBM_GBS, 4),
                             "traffic_frac": traffic_frac("sampler_rings_kernel<bf16,bilinear,channels_last>",
                                                          c4bcl["ms"]),
                             "ms": round(c4bcl["ms"], 4)}},
            "roofline": {"bound": "hbm", "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "traffic": {"nearest": measured_traffic("sampler_rings_kernel<bf16,nearest>"),
                                     "bilinear": measured_traffic("sampler_rings_kernel<bf16,bilinear>"),
                                     "channels_last_nearest":
                                         measured_traffic("sampler_rings_kernel<bf16,nearest,channels_last>"),
                                     "channels_last_bilinear":
                                         measured_traffic("sampler_rings_kernel<bf16,bilinear,channels_last>")},
                         "note": "frac: algorithmic bytes (distinct in-bounds tap pixels + output) per launch "
                                 "time; traffic_frac: HBM bytes the counters read per launch (fetch + write) "
                                 "per launch time, both against 8 TB/s"},
        }
    if pool is not None:
        line["knn_pool"] = {"workload": "kNN max pooling (AlexNet block): 256 images, 64 channels, 1024 -> 256 "
                                        "log-polar points, k=9, bf16 channels-last",
                            "GB/s": round(pool["gbs"], 1), "ms": round(pool["ms"], 4),
                            "roofline": {"bound": "hbm", "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                         "frac": round(pool["gbs"] / PEAK_HBM_GBS, 4)}}
    if c2 is not None:
        line["c2_alexnet"] = {"workload": "C2: 256 images 3x224x224 -> bilinear sampler (4096 pts) -> 5 kNN-conv "
                                          "layers 64/192/384/256/256, k=49/25/9/9/9, ReLU between, bf16",
                              "images/s": round(c2["images_per_s"], 1), "ms": round(c2["ms"], 4),
                              "GFLOP/batch": round(c2["gflop"], 2), "TFLOP/s": round(c2["tflops"], 1)}
    if c4e is not None:
        line["c4_frontend"] = {"workload": "C4: 128 images 3x512x512 bf16 x 4 fixations -> nearest sampler "
                                           "(16384 pts) -> kNN patch embed 3->384, k=256, 256 tokens; "
                                           "sampler output view-major, the patch embedding's view-major kernel",
                               "images/s": round(c4e["images_per_s"], 1), "ms": round(c4e["ms"], 4),
                               "patch_embed_ms": round(c4e["ms_patch_embed"], 4),
                               "patch_embed_TFLOP/s": round(c4e["patch_embed_tflops"], 1),
                               "point_major_ms": round(c4e["ms_point_major"], 4),
                               "point_major_patch_embed_ms": round(c4e["ms_patch_embed_point_major"], 4),
                               "patch_embed_traffic": measured_traffic("knnconv_fewc_vm_kernel<c4>"),
                               "policy_ms": round(c4e["ms_policy"], 4),
                               "policy_note": "MultiRandomSaccadePolicy (near-centre 0.25, eval) forward: host "
                                              "draws + one sampler launch for the 512 views, bf16 out"}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
