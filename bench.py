#!/usr/bin/env python3
"""bench.py -- throughput of the neural-field hot path on one MI355X.

Workload ("C2"): the image-fit training step.
  * 2D multiresolution hash grid: 16 levels x 2 features, T = 2^15 entries per
    level, base resolution 16, per-level scale 1.5, fp32 table;
  * MLP 32 -> 64 -> 64 -> 3, ReLU hidden, no output activation, fp16 MFMA
    operands with fp32 accumulation and fp32 master parameters;
  * RelativeL2 loss against a seeded procedural 1024x1024 RGB image
    (8 random-frequency sinusoids + a 32-px checkerboard, in [0, 1]) sampled
    bilinearly at 2^18 uniform random coordinates per step;
  * full backward through the MLP and the hash table (int32 fixed-point
    scatter), then the fused Adam pass (lr 1e-2, b1 0.9, b2 0.99, eps 1e-15).
One step = Morton sort (a second stream, overlapping the previous step) ->
hash-grid encode kernel -> MLP train kernel (forward, loss, backward, dW, and
the hash-grid backward of each tile: int32 atomics and visit flags) ->
finish kernel (dW / loss reductions, Adam, weight image for the next step),
on the library's HIP streams, inputs resident in HBM before the timed region
starts.

Inside the timed region the library brackets the phases of a few sampled
steps with timing-only HIP events on its own stream (`profile_every`: two
sampled steps for K < 100, five from K = 100); those sampled steps give the
per-kernel durations behind the roofline fractions (`kernel_rooflines`, the
slowest kernel is `roofline`) and `phase_us_per_step`. The events of a
sampled step cost ~13.4 us of stream time (measured: 107.3 us/step with
events on every step, 93.9 us without), so the samples add 1.3 us per step
at K = 20 and 0.3 us at K = 200 (`profile_overhead_us_per_step`).

Also reported: inference samples/s on configs[0] ("C1": the same field shape,
fp32, 2^16 points per call) and the CPU restatement of the reference math
timed on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2|c3|c4|c5]

--workload c3/c4/c5 time the other BASELINE training configs (synthetic
inputs as described in BASELINE.json; the training step and a forward-only
pass over the same batch, timed separately) and print one JSON line for them;
the default, c2, is the headline line above.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "tiny-metal-nn_amd"))

METRIC = "train samples/s (hash-grid+64w MLP, B=2^18); infer samples/s; % roofline"
B_TRAIN = 1 << 18
B_INFER = 1 << 16
IMG = 1024
HBM_PEAK_GBS = 8000.0
EVENT_COST_US = 13.4  # stream time of one sampled step's phase events (measured)


def profile_every(steps: int) -> int:
    """Phase events on one timed step in this many: two sampled steps below
    100 timed steps, five from 100."""
    return max(1, steps // (2 if steps < 100 else 5))
MFMA_F16_PEAK_TFLOPS = 2500.0

C2_CONFIG = {
    "encoding": {"otype": "HashGrid", "n_levels": 16, "n_features_per_level": 2,
                 "log2_hashmap_size": 15, "base_resolution": 16.0, "per_level_scale": 1.5},
    "network": {"otype": "FullyFusedMLP", "n_neurons": 64, "n_hidden_layers": 2,
                "activation": "ReLU", "output_activation": "None"},
    "loss": {"otype": "RelativeL2"},
    "optimizer": {"otype": "Adam", "learning_rate": 1e-2, "beta1": 0.9, "beta2": 0.99,
                  "epsilon": 1e-15},
    "weight_init": {"seed": 42, "hash_grid_range": 1e-4},
    "batch_size": B_TRAIN,
    "mi355x": {"precision": "fp16", "hash_adam": "lazy", "morton_sort": True},
}


def kernel_models(d: int = 2, levels: int = 16, feats: int = 2, n_out: int = 3,
                  inp: int = 32, hidden: int = 64, n_hidden: int = 2,
                  hash_params: int = 16 << 16, mlp_params: int = 6467) -> dict:
    """Algorithmic work of one step's kernels (per point, or per step for
    Adam):
      encode   -- position read, 2^D corner gathers of every level (fp32
                  features), the X tile write (fp32, padded input width);
      mlp      -- 3 x the forward FLOPs 2 * sum(in * out) (forward, delta chain,
                  weight gradients; the split-fp16 forward's extra products and
                  the transposes are overhead, not algorithmic work);
      scatter  -- position and dx row reads, one F-float int32 update per
                  corner and level;
      adam     -- 28 B per parameter (param, m, v read+write, gradient read),
                  the dense figure; the lazy pass reads a flag per table entry
                  on top. The kernel that runs it (finish_step_kernel) also
                  reduces the MLP kernel's per-block dW rows and writes the
                  weight image: overhead, not counted."""
    corners = 1 << d
    flops = 2 * (inp * hidden + (n_hidden - 1) * hidden * hidden + hidden * n_out)
    return {
        "encode": {"bound": "hbm", "per_point": 4 * d + corners * levels * feats * 4 + inp * 4},
        "mlp": {"bound": "mfma", "per_point": 3 * flops},
        "scatter": {"bound": "hbm", "per_point": 4 * d + levels * feats * 4 + corners * levels * feats * 4},
        "adam": {"bound": "hbm", "per_step": 28 * (hash_params + mlp_params) + hash_params // feats},
        # the hash-grid backward run inside the MLP kernel's tiles: position
        # read and the int32 update of every corner and level (dx stays in
        # registers)
        "scatter_fused": {"bound": "hbm", "per_point": 4 * d + corners * levels * feats * 4},
    }


KERNELS = {  # model key -> (step-profile phase, kernel name in rocprof traces)
    "encode": ("gpu_encode_us", "encode_features_kernel<2, 2>"),
    "mlp": ("gpu_fwd_bwd_us", "mlp_train_kernel<64, 32, 2, 8>"),
    "scatter": ("gpu_scatter_us", "hash_scatter_kernel<2, 2>"),
    "adam": ("gpu_adam_us", "finish_step_kernel<2>"),
}
# the C2 kernel when the hash-grid backward runs in its tiles (tile_scatter.hpp)
MLP_FUSED_NAME = "mlp_train_kernel<64, 32, 2, 8, 2, 2>"


def kernel_rooflines(prof: dict, fused_scatter: bool = False, models: dict | None = None,
                     names: dict | None = None, n: int = B_TRAIN) -> list[dict]:
    """Per-kernel roofline fractions from the sampled phase durations. With
    the scatter fused into the MLP kernel, that kernel carries both the MLP's
    FLOPs and the hash backward's bytes; its roofline time is max(FLOPs / MFMA
    peak, bytes / HBM peak), and the entry's bound, achieved, peak and frac
    are those of the larger term (the HBM bytes at every BASELINE shape), with
    the other in "mfma" (FLOP rate) and both times in "fused_scatter"; there
    is no separate scatter kernel then. models / names / n default to the C2
    step (kernel_models(), KERNELS, B_TRAIN)."""
    steps = max(1, prof["steps"])
    models = models or kernel_models()
    out = []
    for key, model in models.items():
        if key == "scatter_fused" or (key == "scatter" and fused_scatter):
            continue
        phase, name = KERNELS[key]
        if names:
            name = names[key]
        elif key == "mlp" and fused_scatter:
            name = MLP_FUSED_NAME
        us = prof[phase] / steps
        work = model.get("per_point", 0) * n + model.get("per_step", 0)
        if model["bound"] == "mfma":
            achieved = work / (us * 1e-6) / 1e12
            r = {"bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                 "unit": "TFLOP/s", "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4)}
        else:
            achieved = work / (us * 1e-6) / 1e9
            r = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                 "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4)}
        r.update({"traffic": traffic_from_profiles(key) if not names else None, "kernel": name,
                  "kernel_avg_us": round(us, 2), "work_per_launch": work})
        if key == "mlp" and fused_scatter:
            sb = models["scatter_fused"]["per_point"] * n
            t_mfma = work / (MFMA_F16_PEAK_TFLOPS * 1e12) * 1e6
            t_hbm = sb / (HBM_PEAK_GBS * 1e9) * 1e6
            r["fused_scatter"] = {
                "bytes_per_launch": sb, "achieved_GBps": round(sb / (us * 1e-6) / 1e9, 1),
                "peak_GBps": HBM_PEAK_GBS, "t_mfma_us": round(t_mfma, 2),
                "t_hbm_us": round(t_hbm, 2),
                "frac_of_roofline_time": round(max(t_mfma, t_hbm) / us, 4)}
            if t_hbm > t_mfma:  # the bytes bound the kernel: report them up front
                r["mfma"] = {k: r[k] for k in ("achieved", "peak", "unit", "frac")}
                gbs = sb / (us * 1e-6) / 1e9
                r.update({"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                          "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                          "work_per_launch": sb, "flops_per_launch": work})
        out.append(r)
    return out


FP32_MFMA_PEAK_TFLOPS = 157.3


def infer_roofline(prof: dict) -> dict | None:
    """C1 forward kernel (field_forward_kernel, fp32 MFMA, inline encode):
    algorithmic FLOPs 2 * (32*64 + 64*64 + 64*3) = 12,672 per point against
    the fp32 dense MFMA peak, and algorithmic bytes per point (position 8 B,
    4 corners x 16 levels x 2 features x 4 B of gathers, 12 B of outputs =
    532 B) against the HBM peak, per launch of 2^16 points over the sampled
    calls' average kernel duration."""
    if not prof.get("infer_calls"):
        return None
    us = prof["gpu_infer_us"] / prof["infer_calls"]
    flops = 2 * (32 * 64 + 64 * 64 + 64 * 3) * B_INFER
    bytes_ = (8 + 4 * 16 * 2 * 4 + 12) * B_INFER
    tf = flops / (us * 1e-6) / 1e12
    gbs = bytes_ / (us * 1e-6) / 1e9
    return {"bound": "mfma", "achieved": round(tf, 2), "peak": FP32_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4),
            "traffic": None, "kernel": "field_forward_kernel<64, 32, false, 18>",
            "kernel_avg_us": round(us, 2), "work_per_launch": flops,
            "gather_GBps": round(gbs, 1), "gather_frac_of_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "sampled_calls": int(prof["infer_calls"])}


OTHER_WORKLOADS = {
    # D, levels, feats, log2T, base, scale, hidden, hidden layers, outputs, loss, batch
    "c3": (3, 16, 2, 19, 16.0, 1.381913, 64, 1, 16, "L2", 1 << 20),
    "c4": (3, 16, 4, 21, 16.0, 1.5, 64, 3, 1, "L1", 1 << 19),
    "c5": (4, 16, 2, 22, 8.0, 1.4, 128, 4, 4, "L2", 1 << 20),
}


def workload_batch(torch, which: str, n: int, gen, dev):
    """Synthetic batch of BASELINE configs[2..4] (seeded):
    c3 -- 70% of the points from 64 Gaussian blobs (sigma 0.02), 30% uniform in
          [0,1)^3; target = sum of the blob Gaussians in output 0, zeros in the
          other 15 (the reference's loss sums every output, so a 16-wide target
          with the density in channel 0 is the faithful reading);
    c4 -- 50% within +-0.01 of the union of 8 spheres (r 0.05-0.25), 50% uniform;
          target = the analytic SDF of the union (L1);
    c5 -- uniform in [0,1)^4; output c = sum of 16 seeded 4D sinusoids."""
    g = torch.Generator(device=dev).manual_seed(11)
    if which == "c3":
        centers = torch.rand(64, 3, device=dev, generator=g)
        nb = int(0.7 * n)
        idx = torch.randint(0, 64, (nb,), device=dev, generator=gen)
        blob = centers[idx] + 0.02 * torch.randn(nb, 3, device=dev, generator=gen)
        pos = torch.cat([blob, torch.rand(n - nb, 3, device=dev, generator=gen)]).clamp(0.0, 0.999999)
        d2 = ((pos[:, None, :] - centers[None, :, :]) ** 2).sum(-1)
        dens = torch.exp(-d2 / (2 * 0.02 ** 2)).sum(1, keepdim=True)
        tgt = torch.cat([dens, torch.zeros(n, 15, device=dev)], 1)
    elif which == "c4":
        centers = 0.25 + 0.5 * torch.rand(8, 3, device=dev, generator=g)
        radii = 0.05 + 0.2 * torch.rand(8, device=dev, generator=g)
        nb = n // 2
        k = torch.randint(0, 8, (nb,), device=dev, generator=gen)
        dirs = torch.nn.functional.normalize(torch.randn(nb, 3, device=dev, generator=gen), dim=1)
        shell = centers[k] + dirs * (radii[k] + 0.02 * torch.rand(nb, 1, device=dev, generator=gen).squeeze(1) - 0.01)[:, None]
        pos = torch.cat([shell, torch.rand(n - nb, 3, device=dev, generator=gen)]).clamp(0.0, 0.999999)
        sdf = ((pos[:, None, :] - centers[None]).norm(dim=-1) - radii[None]).amin(1, keepdim=True)
        tgt = sdf
    else:
        pos = torch.rand(n, 4, device=dev, generator=gen)
        freq = torch.rand(4, 16, 4, device=dev, generator=g) * 8.0 - 4.0
        phase = torch.rand(4, 16, device=dev, generator=g) * 2 * math.pi
        tgt = torch.sin(2 * math.pi * torch.einsum("nd,ckd->nck", pos, freq) + phase[None]).sum(-1) / 4.0
    return pos.contiguous().float(), tgt.contiguous().float()


def run_other_workload(args, which: str) -> int:
    import torch
    from tiny_metal_nn import Trainer
    d, levels, feats, log2t, base, scale, hidden, nhl, m, loss, n = OTHER_WORKLOADS[which]
    dev = torch.device("cuda:0")
    cfg = {"encoding": {"otype": "HashGrid", "n_levels": levels, "n_features_per_level": feats,
                        "log2_hashmap_size": log2t, "base_resolution": base,
                        "per_level_scale": scale},
           "network": {"otype": "FullyFusedMLP", "n_neurons": hidden, "n_hidden_layers": nhl},
           "loss": {"otype": loss},
           "optimizer": {"otype": "Adam", "learning_rate": 1e-2, "beta1": 0.9, "beta2": 0.99,
                         "epsilon": 1e-15},
           "weight_init": {"seed": 42}, "batch_size": n,
           "mi355x": {"precision": "fp16", "hash_adam": "lazy", "morton_sort": True}}
    gen = torch.Generator(device=dev).manual_seed(7)
    batches = [workload_batch(torch, which, n, gen, dev) for _ in range(2)]
    loss_dev = torch.zeros(args.steps + args.warmup + 1, device=dev)
    tr = Trainer.from_config(cfg, n_input=d, n_output=m)
    for i in range(args.warmup):
        x, y = batches[i % 2]
        tr.training_step_device(x.data_ptr(), y.data_ptr(), n, loss_dev[i].data_ptr())
    tr.synchronize()
    # timed steps, phase events on one in `every` (as the C2 line)
    every = profile_every(args.steps)
    tr.set_training_step_profiling(True, every)
    t0 = time.perf_counter()
    for i in range(args.steps):
        x, y = batches[i % 2]
        tr.training_step_device(x.data_ptr(), y.data_ptr(), n,
                                loss_dev[args.warmup + i].data_ptr())
    tr.synchronize()
    el = time.perf_counter() - t0
    prof = tr.training_step_profile()
    tr.set_training_step_profiling(False)
    out = torch.empty(n, m, device=dev)
    x = batches[0][0]
    for _ in range(3):
        tr.inference_device(x.data_ptr(), out.data_ptr(), n)
    tr.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        tr.inference_device(x.data_ptr(), out.data_ptr(), n)
    tr.synchronize()
    fwd = (time.perf_counter() - t1) / args.steps
    # reference rates at this shape over a batch in the step's Morton order
    rates = tr.debug_hash_rates(batches[0][0].data_ptr(), n, sorted=True, reps=5)
    losses = loss_dev.cpu().numpy()
    fused = bool(tr.inspect_runtime().get("train_fused_scatter"))
    tr.close()
    steps_prof = max(1, prof["steps"])
    inp = 32 if levels * feats <= 32 else 64
    mlp_params = (levels * feats * hidden + hidden + (nhl - 1) * (hidden * hidden + hidden)
                  + hidden * m + m)
    models = kernel_models(d, levels, feats, m, inp, hidden, nhl, levels * feats << log2t,
                           mlp_params)
    mlp_name = {"c3": "mlp_train_kernel<64, 32, 1, 8, 3, 2>" if fused else
                      "mlp_train_kernel<64, 32, 1, 8, 0, 0>",
                "c4": "mlp_train_kernel<64, 64, 3, 4, 0, 0>", "c5": "wide_train_kernel<4>"}[which]
    names = {"encode": f"encode_level_kernel<{d}, {feats}>", "mlp": mlp_name,
             "scatter": f"hash_scatter_level_kernel<{d}, {feats}>",
             "adam": f"finish_step_kernel<{feats}>"}
    per_kernel = kernel_rooflines(prof, fused, models, names, n) if prof["steps"] else []
    attach_achievable(per_kernel, rates)
    print(json.dumps({
        "metric": f"train samples/s ({which}); forward-only samples/s", "value": round(n * args.steps / el, 1),
        "unit": "samples/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(el * 1e3 / args.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16 MFMA / f32 encode+Adam / i32 hash grads",
        "data": "synthetic (see workload_batch)",
        "config": {"workload": which, "batch": n, "encoding": f"{d}D L{levels} F{feats} T2^{log2t}",
                   "mlp": f"{hidden}x{nhl}->{m}", "loss": loss},
        "forward_samples_per_s": round(n / fwd, 1), "forward_ms": round(fwd * 1e3, 4),
        "phase_us_per_step": {k: round(prof[k] / steps_prof, 2) for k in prof if k.startswith("gpu_")},
        "kernel_rooflines": per_kernel,
        "loss_first_last": [round(float(losses[0]), 6),
                            round(float(losses[args.warmup + args.steps - 1]), 6)]}), flush=True)
    return 0


def attach_achievable(per_kernel: list, rates: dict) -> None:
    """Adds the reference-rate kernels' times (tmnn_debug_hash_rates at the
    trainer's shape, over the step's Morton-ordered batch, walking the levels
    as the kernel they stand for does) to the encode and scatter entries."""
    for r in per_kernel:
        if r["kernel"].startswith("encode"):
            r["achievable"] = {"reference": "gather-only kernel (the encode's corner loads)",
                               "us": round(rates["gather_us"], 2),
                               "frac_of_achievable": round(rates["gather_us"] / r["kernel_avg_us"], 4)}
        elif r["kernel"].startswith("hash_scatter") or "fused_scatter" in r:
            r["achievable"] = {"reference": "flag-store-only and atomic-only kernels (the "
                                            "scatter's memory operations: one per run of "
                                            "lanes on the same entry, every corner and level)",
                               "flag_us": round(rates["flag_us"], 2),
                               "atomic_us": round(rates["atomic_us"], 2)}


def make_image(torch, seed: int, device):
    """Seeded procedural RGB image in [0, 1]: 8 random-frequency sinusoids per
    channel plus a 32-pixel checkerboard, min-max normalised per channel."""
    g = torch.Generator().manual_seed(seed)
    v, u = torch.meshgrid(torch.arange(IMG, dtype=torch.float64) / IMG,
                          torch.arange(IMG, dtype=torch.float64) / IMG, indexing="ij")
    chans = []
    for _ in range(3):
        acc = torch.zeros(IMG, IMG, dtype=torch.float64)
        for _ in range(8):
            amp = 0.5 + 0.5 * torch.rand((), generator=g, dtype=torch.float64)
            fx, fy = (torch.rand(2, generator=g, dtype=torch.float64) * 80.0 - 40.0)
            ph = torch.rand((), generator=g, dtype=torch.float64) * 2 * math.pi
            acc += amp * torch.sin(2 * math.pi * (fx * u + fy * v) + ph)
        chans.append(acc)
    img = torch.stack(chans, 0)
    iy = torch.arange(IMG).view(IMG, 1) // 32
    ix = torch.arange(IMG).view(1, IMG) // 32
    img = img + 2.0 * ((ix + iy) % 2).to(torch.float64)
    lo = img.amin(dim=(1, 2), keepdim=True)
    hi = img.amax(dim=(1, 2), keepdim=True)
    img = (img - lo) / (hi - lo)
    return img.to(torch.float32).to(device)  # [3][H][W]


def sample_bilinear(torch, img, pos):
    """Bilinear image sample at pos in [0,1)^2 (pixel-centre convention)."""
    grid = (pos * 2.0 - 1.0).view(1, 1, -1, 2)
    out = torch.nn.functional.grid_sample(img.unsqueeze(0), grid, mode="bilinear",
                                          padding_mode="border", align_corners=False)
    return out.view(3, -1).t().contiguous()


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(seconds: float = 12.0) -> dict:
    """The CPU restatement of the reference math (oracle/, compiled -O3,
    OpenMP over points) running the same C2 training step (B = 2^18, the GPU
    line's batch) on this host's cores, on a bounded sample: all threads for
    about `seconds` * 2/3 of steps, then one thread for the rest (the 1-core
    figure); each leg runs at least one whole step."""
    sys.path.insert(0, str(REPO / "tests"))
    from oracle_binding import Oracle  # the checker's binding; CPU baseline only

    o = Oracle()
    nproc = os.cpu_count() or 1
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or nproc
    threads = max(1, min(threads, nproc))
    e = C2_CONFIG["encoding"]
    m = o.model(2, e["n_levels"], e["n_features_per_level"], e["log2_hashmap_size"],
                e["base_resolution"], e["per_level_scale"], 64, 2, 3, "RelativeL2")
    adam = o.adam(1e-2, 1e-2)
    hw, mw = o.init_params(m, 42, 1e-4)
    params = np.concatenate([hw, mw])
    m1, m2 = np.zeros_like(params), np.zeros_like(params)
    rng = np.random.default_rng(0)
    n = B_TRAIN
    pos = rng.random((n, 2), dtype=np.float32)
    tgt = rng.random((n, 3), dtype=np.float32)
    step = 0

    def leg(nthreads: int, budget: float):
        nonlocal step
        steps, t0 = 0, time.perf_counter()
        while True:
            o.training_step(m, adam, step, params, m1, m2, pos, tgt, threads=nthreads)
            step += 1
            steps += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return steps, el

    o.training_step(m, adam, step, params, m1, m2, pos, tgt, threads=threads)  # warm
    step += 1
    s_all, t_all = leg(threads, seconds * 2 / 3)
    s_one, t_one = leg(1, seconds / 3)
    return {"value": n * s_all / t_all, "unit": "samples/s", "cores": threads, "kind": "port",
            "one_core_value": n * s_one / t_one, "cpu_model": _cpu_model(), "nproc": nproc,
            "batch": n,
            "sample": f"C2 training steps of 2^18 points (the GPU line's batch): {s_all} in "
                      f"{t_all:.1f} s on {threads} threads, {s_one} in {t_one:.1f} s on 1 thread "
                      f"(oracle/, -O3, OpenMP over points; {_cpu_model()}, nproc {nproc})"}


def traffic_from_profiles(key: str) -> float | None:
    """HBM bytes per launch of one kernel of the C2 step, from the committed
    rocprofv3 PMC summary profiles/c2_step_kernels.md (FETCH_SIZE + WRITE_SIZE
    per dispatch, each scaled by the same counter's reading for a plain copy
    of known size)."""
    f = REPO / "profiles" / "c2_step_kernels.md"
    if not f.exists():
        return None
    tag = f"traffic_bytes_per_launch[{key}]:"
    for line in f.read_text().splitlines():
        if line.startswith(tag):
            try:
                return float(line.split(":", 1)[1])
            except ValueError:
                return None
    return None


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--workload", default="c2", choices=["c2", "c3", "c4", "c5"])
    ap.add_argument("--profile-every", type=int, default=None, metavar="K",
                    help="phase events on one timed step in K (0: none)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (5 launches): the "
                         "known-size reference for FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n * 4, "launches": 5}))
        return 0
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures one "
              "MI355X (the hot path runs on a single GPU: samples are data parallel, a "
              "multi-GPU step would shard the batch and all-reduce the gradients)",
              file=sys.stderr)
        return 2

    import torch
    from tiny_metal_nn import Trainer

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    if args.workload != "c2":
        return run_other_workload(args, args.workload)
    dev = torch.device("cuda:0")
    img = make_image(torch, 1234, dev)
    gen = torch.Generator(device=dev).manual_seed(7)
    nb = 4
    xs = [torch.rand(B_TRAIN, 2, device=dev, generator=gen) for _ in range(nb)]
    ys = [sample_bilinear(torch, img, x) for x in xs]
    loss_dev = torch.zeros(args.steps + args.warmup + 1, device=dev)
    torch.cuda.synchronize()

    tr = Trainer.from_config(C2_CONFIG, n_input=2, n_output=3)
    ins = tr.inspect_runtime()
    print(f"# trainer: {ins}", file=sys.stderr, flush=True)

    def step(i: int) -> None:
        tr.training_step_device(xs[i % nb].data_ptr(), ys[i % nb].data_ptr(), B_TRAIN,
                                loss_dev[i].data_ptr())

    for i in range(args.warmup):
        step(i)
    tr.synchronize()
    torch.cuda.synchronize()
    print(f"# warmup done ({args.warmup} steps)", file=sys.stderr, flush=True)

    # timed region: phase events on one step in `every` (the kernel durations),
    # the rest run exactly as a caller runs them
    every = profile_every(args.steps) if args.profile_every is None else args.profile_every
    tr.set_training_step_profiling(every > 0, max(every, 1))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(args.warmup + i)
    tr.synchronize()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    elapsed = t1 - t0
    prof = tr.training_step_profile()
    tr.set_training_step_profiling(False)
    losses = loss_dev.cpu().numpy()
    first_loss = float(losses[0])
    last_loss = float(losses[args.warmup + args.steps - 1])
    if not (math.isfinite(last_loss) and last_loss < first_loss):
        print(f"bench.py: training did not progress (loss {first_loss} -> {last_loss})",
              file=sys.stderr)
        return 1
    train_sps = B_TRAIN * args.steps / elapsed
    print(f"# timed {args.steps} steps in {elapsed * 1e3:.1f} ms; loss {first_loss:.5f} -> "
          f"{last_loss:.5f}; profile {prof}", file=sys.stderr, flush=True)

    # reference rates at this shape over a batch in the step's Morton order:
    # gather-only (the encode's loads), atomic-only and flag-store-only (the
    # scatter's memory operations) -- the achievable denominators
    rates = tr.debug_hash_rates(xs[0].data_ptr(), B_TRAIN, sorted=True, reps=20)

    # inference on the C1 shape (same field, fp32, 2^16 points per call)
    xi = torch.rand(B_INFER, 2, device=dev, generator=gen)
    yi = torch.empty(B_INFER, 3, device=dev)
    for _ in range(10):
        tr.inference_device(xi.data_ptr(), yi.data_ptr(), B_INFER)
    tr.synchronize()
    torch.cuda.synchronize()
    iters = max(50, args.steps)
    # five calls of the timed loop carry an event pair around the kernel
    tr.set_training_step_profiling(True, max(1, iters // 5))
    t2 = time.perf_counter()
    for _ in range(iters):
        tr.inference_device(xi.data_ptr(), yi.data_ptr(), B_INFER)
    tr.synchronize()
    torch.cuda.synchronize()
    infer_sps = B_INFER * iters / (time.perf_counter() - t2)
    iprof = tr.training_step_profile()
    tr.set_training_step_profiling(False)
    tr.close()
    infer_roof = infer_roofline(iprof)

    steps_prof = max(1, prof["steps"])
    fused = bool(ins.get("train_fused_scatter"))
    per_kernel = kernel_rooflines(prof, fused) if prof["steps"] else []
    attach_achievable(per_kernel, rates)
    roofline = max(per_kernel, key=lambda r: r["kernel_avg_us"]) if per_kernel else None
    phases = {k: round(prof[k] / steps_prof, 2) for k in
              ("gpu_sort_us", "gpu_encode_us", "gpu_fwd_bwd_us", "gpu_scatter_us", "gpu_reduce_us",
               "gpu_adam_us", "gpu_total_us")}

    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": round(train_sps, 1),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 MFMA (fp32 accumulate) / f32 encode+Adam / i32 hash grads",
        "data": "synthetic: seeded procedural 1024x1024 RGB image (8 sinusoids + 32-px "
                "checkerboard) sampled bilinearly at uniform random coords; Philox-seeded "
                "weights; inputs resident in HBM",
        "config": {"workload": "C2 image-fit training step (configs[1])",
                   "batch": B_TRAIN, "encoding": "2D hash grid L16 F2 T2^15 base16 x1.5",
                   "mlp": "32-64-64-3 ReLU", "loss": "RelativeL2",
                   "optimizer": "Adam lr1e-2 (lazy hash + dense MLP)",
                   "parallelism": "single GPU"},
        "infer_samples_per_s": round(infer_sps, 1),
        "infer_config": "C1 (configs[0]): same field, fp32, 2^16 points per call",
        "infer_roofline": infer_roof,
        "phase_us_per_step": phases,
        "profile_every": every,
        "profiled_steps": int(prof["steps"]),
        "profile_overhead_us_per_step": round(EVENT_COST_US * prof["steps"] / args.steps, 2),
        "loss_first_last": [round(first_loss, 6), round(last_loss, 6)],
        "roofline": roofline,
        "kernel_rooflines": per_kernel,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
