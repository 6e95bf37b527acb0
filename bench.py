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

The timed region runs the K steps exactly as a caller runs them (no
profiling events). After it, PROFILED_STEPS more steps run with timing-only
HIP events around every phase of every step and start / stop events recorded
by the main kernels' own dispatches (tmnn_get_step_profile_samples); the
MEDIAN of those per-step kernel durations is each kernel's duration behind
`phase_us_median`, the roofline fractions (`kernel_rooflines`) and
`roofline` (the MLP training kernel: max(FLOPs / fp16 MFMA peak, LDS bytes /
LDS peak) over its duration, the LDS peak measured in the same run by
tmnn_debug_lds_rate). The same statistic over the same kernel's dispatches
in a rocprofv3 kernel trace of this command is what `--trace-summary`
prints.

Also reported: inference samples/s on configs[0] ("C1": the same field shape,
fp32, 2^16 points per call), the C2 step in fp32 (the reference's own
training precision), the other BASELINE training configs C3-C5 (training
step and forward-only pass over the same batch, timed separately) and three
layer-wise (Tiled family) shapes under `workloads`, and the CPU restatement
of the reference math timed on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2|c3|c4|c5|tiled_*]
       python bench.py --trace-summary KERNEL_TRACE_CSV

--workload c3/c4/c5 print the one JSON line of that config alone; the
default, c2, is the headline line above with every config under
`workloads`. --workload tiled_h512_2d / tiled_w128_fp32_4d / tiled_h256_3d
time a layer-wise (Tiled family) shape at 2^16 points: shapes no fused
kernel instantiates, outside the BASELINE configs.
"""
from __future__ import annotations

import argparse
import json
import math
import statistics
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
MFMA_F16_PEAK_TFLOPS = 2500.0
PROFILED_STEPS = 40  # steps after the timed region with every phase timed (medians)

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

# ---------------------------------------------------------------- LDS model --
# LDS bytes of the MLP training kernels, counted from their code: every LDS
# instruction of these kernels moves 16 bytes per lane (ds_read_b128 /
# ds_write_b128 of weight fragments, bias rows and parked operands; 1 KiB
# per wave-wide instruction), and the width-128 kernel's direct
# global-to-LDS weight stages write 16 bytes per lane as well. The counts are
# per 32-point wave tile (64-wide kernel) or per 128-point block round
# (width-128 kernel); the end-of-launch reductions (a few KB per block) and
# the fused hash-grid backward's resolution-table reads (4 bytes per point
# and level) are left out.

def mlp_lds_bytes_per_tile(inp: int, nhl: int, waves: int) -> int:
    """mlp_train_kernel<64, INP, NHL, W>: HT = 4 unit tiles, HS = 2 K steps per
    hidden layer, KT0 = INP / 16 input tiles, XS = KT0 / 2.
      forward A fragments, hi + lo: 2 XS HT (layer 0) + 2 HS HT per further
        hidden layer + 2 HS (output);
      bias rows: HT per hidden layer + 1;
      backward A fragments: HT (output) + HS HT per further hidden layer +
        HS KT0 (the input-feature gradient);
      parked transposed operands: KT0 inputs + HT per hidden layer's
        activations + HT per delta (+1 output gradient in 4-wave blocks);
      dW_out: 8-wave blocks read their own HT parked tiles; 4-wave blocks run
        HT owner jobs per round of W tiles, 2 W operands each: 2 HT per tile;
      owner jobs: HT^2 dW tiles per further hidden layer and KT0 HT for dW_0,
        each reading 2 W parked operands per round of W tiles: 2 per tile."""
    HT, HS, KT0, XS = 4, 2, inp // 16, inp // 32
    fwd = 2 * XS * HT + (nhl - 1) * 2 * HS * HT + 2 * HS
    bias = nhl * HT + 1
    bwd = HT + (nhl - 1) * HS * HT + HS * KT0
    park = KT0 + 2 * nhl * HT + (0 if waves == 8 else 1)
    dwout = HT if waves == 8 else 2 * HT
    owners = (nhl - 1) * 2 * HT * HT + 2 * KT0 * HT
    return 1024 * (fwd + bias + bwd + park + dwout + owners)


def wide_lds_bytes_per_round(nhl: int) -> int:
    """wide_train_kernel<NHL> (hidden width 128, 32 inputs, four waves, one
    32-point tile each per round): HT = 8, HS = 4, KT0 = 2, XS = 1.
    Per wave: forward hi + lo fragments 2 XS HT + 2 HS HT per further hidden
    layer + 2 HS; bias rows HT per hidden layer + 1; backward fragments HT +
    HS HT per further hidden layer + HS KT0; parks 1 (output gradient) + HT
    (last hidden layer) + 2 HT per further hidden layer (delta, layer input) +
    HT + KT0 (delta_0, inputs); owner jobs 2 W operands each: HT^2 / W per
    further hidden layer, HT KT0 / W for dW_0, HT / W for dW_out, with the
    bias sums' parked-tile reads (2 W per layer) and the dW_0 / dW_out
    accumulator slots (load + store). Per block: the weight stages written
    into LDS, the image's forward hi + lo and backward fragments."""
    HT, HS, KT0, XS, W = 8, 4, 2, 1, 4
    fwd = 2 * XS * HT + (nhl - 1) * 2 * HS * HT + 2 * HS
    bias = nhl * HT + 1
    bwd = HT + (nhl - 1) * HS * HT + HS * KT0
    park = 1 + HT + 2 * HT * (nhl - 1) + HT + KT0
    owners = (2 * W * (HT * HT // W) * (nhl - 1) + 2 * W * (HT * KT0 // W) + 2 * W * (HT // W)
              + 2 * W * nhl + 2 * (HT * KT0 // W + HT // W))
    per_wave = fwd + bias + bwd + park + owners
    stages = 2 * 32 * 128 * 2 + (nhl - 1) * 2 * 128 * 128 * 2 + 2 * 128 * 16 * 2 \
        + 128 * 32 * 2 + (nhl - 1) * 128 * 128 * 2 + 32 * 128 * 2
    return 1024 * W * per_wave + stages


def lds_bytes_per_launch(kernel: str, n: int, inp: int, nhl: int, waves: int) -> int:
    if kernel.startswith("wide_train_kernel"):
        return wide_lds_bytes_per_round(nhl) * ((n + 127) // 128)
    return mlp_lds_bytes_per_tile(inp, nhl, waves) * ((n + 31) // 32)


def median_phases(samples) -> dict:
    """Per-column medians of the per-step samples (rows = steps): the step's
    phases and its main kernels' own durations."""
    from tiny_metal_nn._lib import PROFILE_PHASES
    if len(samples) == 0:
        return {k: 0.0 for k in PROFILE_PHASES}
    med = np.median(np.asarray(samples, np.float64), axis=0)
    return {k: float(v) for k, v in zip(PROFILE_PHASES, med)}


def kernel_rooflines(phase_us: dict, models: dict, names: dict, n: int, fused_scatter: bool,
                     mlp_shape: tuple, lds_peak_gbs: float, rates: dict | None,
                     traffic: dict | None = None, fp32: bool = False) -> list[dict]:
    """Roofline entries of one training step's kernels from the kernels'
    median durations (phase_us): encode and finish (Adam) against the HBM
    peak (the encode also against its gather-only reference kernel); the MLP
    training kernel against max(FLOPs / MFMA peak, LDS bytes / LDS peak)
    (bound "mfma" or "lds", whichever term is larger), with the hash-grid
    backward it runs in its tiles (fused_scatter) rated against the
    flag-store-only reference kernel at the same shape; a separate scatter
    kernel against its flag and atomic references. mlp_shape = (kernel's
    input width, hidden layers, waves per block)."""
    out = []
    mfma_peak = FP32_MFMA_PEAK_TFLOPS if fp32 else MFMA_F16_PEAK_TFLOPS
    for key, phase, kern in (("encode", "gpu_encode_us", "gpu_encode_kernel_us"),
                             ("mlp", "gpu_fwd_bwd_us", "gpu_train_kernel_us"),
                             ("scatter", "gpu_scatter_us", "gpu_scatter_kernel_us"),
                             ("adam", "gpu_adam_us", "gpu_finish_kernel_us")):
        if key == "scatter" and fused_scatter:
            continue
        # the kernel's own duration (dispatch timestamps); the phase (which
        # also holds the launch gap) where the step runs several kernels
        us = phase_us.get(kern, 0.0) or phase_us[phase]
        if us <= 0:
            continue
        model = models[key]
        work = model.get("per_point", 0) * n + model.get("per_step", 0)
        r = {"kernel": names[key], "kernel_us": round(us, 2),
             "traffic": (traffic or {}).get(key)}
        if key == "mlp":
            tf = work / (us * 1e-6) / 1e12
            t_mfma = work / (mfma_peak * 1e12) * 1e6
            mfma = {"achieved": round(tf, 1), "peak": mfma_peak, "unit": "TFLOP/s",
                    "frac": round(tf / mfma_peak, 4), "flops_per_launch": work,
                    "t_us": round(t_mfma, 2)}
            r["mfma"] = mfma
            if fp32:  # the fp32 training kernels: no LDS model, fp32 MFMA peak
                r.update({"bound": "mfma", "achieved": mfma["achieved"], "peak": mfma_peak,
                          "unit": "TFLOP/s", "frac": mfma["frac"]})
                r["roofline_us"] = round(t_mfma, 2)
            else:
                lb = lds_bytes_per_launch(names[key], n, *mlp_shape)
                t_lds = lb / (lds_peak_gbs * 1e9) * 1e6
                lgbs = lb / (us * 1e-6) / 1e9
                r["lds"] = {"bytes_per_launch": lb, "achieved": round(lgbs, 1),
                            "peak": round(lds_peak_gbs, 1), "unit": "GB/s",
                            "frac": round(lgbs / lds_peak_gbs, 4), "t_us": round(t_lds, 2)}
                if t_lds >= t_mfma:
                    r.update({"bound": "lds", "achieved": round(lgbs, 1),
                              "peak": round(lds_peak_gbs, 1), "unit": "GB/s",
                              "frac": round(t_lds / us, 4)})
                else:
                    r.update({"bound": "mfma", "achieved": mfma["achieved"], "peak": mfma_peak,
                              "unit": "TFLOP/s", "frac": round(t_mfma / us, 4)})
                r["roofline_us"] = round(max(t_mfma, t_lds), 2)
            if fused_scatter and rates:
                sb = models["scatter_fused"]["per_point"] * n
                t_ref = rates["flag_us"]
                r["fused_scatter"] = {
                    "bytes_per_launch": sb,
                    "reference": "flag-store-only kernel at this shape (one flag store per run of "
                                 "lanes on an entry, every corner and level; a converging batch's "
                                 "hash-grid backward stores flags only for 90-99% of its groups)",
                    "flag_ref_us": round(t_ref, 2), "atomic_ref_us": round(rates["atomic_us"], 2),
                    "frac_with_scatter": round(max(r.get("roofline_us", 0.0), t_ref) / us, 4)}
        else:
            gbs = work / (us * 1e-6) / 1e9
            r.update({"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                      "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                      "bytes_per_launch": work})
            if rates and key == "encode":
                r["achievable"] = {"reference": "gather-only kernel (the encode's corner loads)",
                                   "us": round(rates["gather_us"], 2),
                                   "frac_of_achievable": round(rates["gather_us"] / us, 4)}
            if rates and key == "scatter":
                r["achievable"] = {"reference": "flag-store-only and atomic-only kernels",
                                   "flag_us": round(rates["flag_us"], 2),
                                   "atomic_us": round(rates["atomic_us"], 2)}
        out.append(r)
    return out


FP32_MFMA_PEAK_TFLOPS = 157.3


def infer_roofline(groups: list, gather_ref_us: float | None = None) -> dict | None:
    """C1 forward kernel (field_forward_kernel, fp32 MFMA, inline encode):
    algorithmic FLOPs 2 * (32*64 + 64*64 + 64*3) = 12,672 per point against
    the fp32 dense MFMA peak, and algorithmic bytes per point (position 8 B,
    4 corners x 16 levels x 2 features x 4 B of gathers, 12 B of outputs =
    532 B) against the HBM peak, per launch of 2^16 points over the sampled
    calls' kernel duration: the median over groups of calls of each group's
    average (`groups`: the sampled-call profiles). `achievable`: the
    gather-only reference kernel over the same unsorted 2^16 points (every
    corner of every level, one thread per point), measured in the same run --
    the time the kernel's gathers alone take."""
    per = [g["gpu_infer_us"] / g["infer_calls"] for g in groups if g.get("infer_calls")]
    if not per:
        return None
    us = statistics.median(per)
    calls = sum(int(g["infer_calls"]) for g in groups if g.get("infer_calls"))
    flops = 2 * (32 * 64 + 64 * 64 + 64 * 3) * B_INFER
    bytes_ = (8 + 4 * 16 * 2 * 4 + 12) * B_INFER
    tf = flops / (us * 1e-6) / 1e12
    gbs = bytes_ / (us * 1e-6) / 1e9
    return {"bound": "mfma", "achieved": round(tf, 2), "peak": FP32_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4),
            "traffic": None, "kernel": "field_forward_kernel<64, 32, false, 18>",
            "kernel_avg_us": round(us, 2), "work_per_launch": flops,
            "gather_GBps": round(gbs, 1), "gather_frac_of_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "sampled_calls": calls,
            "statistic": f"median over {len(per)} groups of {calls // len(per)} calls of the group's "
                         "average kernel duration (event pair around each kernel)",
            "achievable": None if gather_ref_us is None else {
                "reference": "gather-only kernel over the same unsorted points",
                "us": round(gather_ref_us, 2),
                "frac_of_achievable": round(gather_ref_us / us, 4)}}


OTHER_WORKLOADS = {
    # D, levels, feats, log2T, base, scale, hidden, hidden layers, outputs, loss, batch
    "c3": (3, 16, 2, 19, 16.0, 1.381913, 64, 1, 16, "L2", 1 << 20),
    "c4": (3, 16, 4, 21, 16.0, 1.5, 64, 3, 1, "L1", 1 << 19),
    "c5": (4, 16, 2, 22, 8.0, 1.4, 128, 4, 4, "L2", 1 << 20),
}


TILED_WORKLOADS = {
    # Layer-wise (Tiled family) shapes, the ones no fused kernel instantiates:
    # D, levels, feats, log2T, base, scale, hidden, hidden layers, outputs
    # (fp32 training, L2 loss, B_TILED points)
    "tiled_h512_2d": (2, 16, 2, 14, 16.0, 1.5, 512, 1, 3),
    "tiled_w128_fp32_4d": (4, 16, 2, 16, 8.0, 1.4, 128, 4, 4),
    "tiled_h256_3d": (3, 8, 2, 14, 8.0, 2.0, 256, 2, 4),
}
B_TILED = 1 << 16


def run_tiled(torch, which: str, steps: int, warmup: int) -> dict:
    """A layer-wise (Tiled family) shape: `steps` timed fp32 training steps over
    B_TILED seeded uniform random points with uniform random targets in [0,1)
    (after `warmup` untimed ones), then forward-only passes over the same batch,
    timed separately. Exits if the planner does not select the Tiled family."""
    from tiny_metal_nn import Trainer
    d, levels, feats, log2t, base, scale, hidden, nhl, m = TILED_WORKLOADS[which]
    n = B_TILED
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(7)
    x = torch.rand(n, d, device=dev, generator=gen)
    y = torch.rand(n, m, device=dev, generator=gen)
    loss_dev = torch.zeros(steps + warmup, device=dev)
    torch.cuda.synchronize()
    tr = Trainer.from_config(_config(d, levels, feats, log2t, base, scale, hidden, nhl, "L2", n, "fp32"),
                             n_input=d, n_output=m)
    family = tr.inspect_runtime()["family_name"]
    if family != "Tiled":
        tr.close()
        raise SystemExit(f"bench.py: {which} planned as {family}, not Tiled")
    for i in range(warmup):
        tr.training_step_device(x.data_ptr(), y.data_ptr(), n, loss_dev[i].data_ptr())
    tr.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        tr.training_step_device(x.data_ptr(), y.data_ptr(), n, loss_dev[warmup + i].data_ptr())
    tr.synchronize()
    el = time.perf_counter() - t0
    out = torch.empty(n, m, device=dev)
    for _ in range(3):
        tr.inference_device(x.data_ptr(), out.data_ptr(), n)
    tr.synchronize()
    fwd_iters = max(5, steps)
    t1 = time.perf_counter()
    for _ in range(fwd_iters):
        tr.inference_device(x.data_ptr(), out.data_ptr(), n)
    tr.synchronize()
    fwd = (time.perf_counter() - t1) / fwd_iters
    losses = loss_dev.cpu().numpy()
    tr.close()
    return {"workload": which, "family": family, "precision": "fp32", "batch": n,
            "encoding": f"{d}D L{levels} F{feats} T2^{log2t} base{base:g} x{scale:g}",
            "mlp": f"{levels * feats}->{hidden}x{nhl}->{m}", "loss": "L2",
            "train_samples_per_s": round(n * steps / el, 1), "ms_per_step": round(el * 1e3 / steps, 4),
            "forward_samples_per_s": round(n / fwd, 1), "forward_ms": round(fwd * 1e3, 4),
            "loss_first_last": [round(float(losses[0]), 6), round(float(losses[-1]), 6)]}


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

def _config(d, levels, feats, log2t, base, scale, hidden, nhl, loss, n, precision):
    return {"encoding": {"otype": "HashGrid", "n_levels": levels, "n_features_per_level": feats,
                         "log2_hashmap_size": log2t, "base_resolution": base,
                         "per_level_scale": scale},
            "network": {"otype": "FullyFusedMLP", "n_neurons": hidden, "n_hidden_layers": nhl},
            "loss": {"otype": loss},
            "optimizer": {"otype": "Adam", "learning_rate": 1e-2, "beta1": 0.9, "beta2": 0.99,
                          "epsilon": 1e-15},
            "weight_init": {"seed": 42, "hash_grid_range": 1e-4}, "batch_size": n,
            "mi355x": {"precision": precision, "hash_adam": "lazy", "morton_sort": True}}


def mlp_kernel_name(which: str, fused: bool, precision: str) -> str:
    if precision == "fp32":
        return {"c2": "field_train_kernel<64, 32, false, 2, 2, 2>" if fused else
                      "field_train_kernel<64, 32, false, 2, 0, 0>"}.get(which, "field_train_kernel")
    return {"c2": "mlp_train_kernel<64, 32, 2, 8, 2, 2>" if fused else
                  "mlp_train_kernel<64, 32, 2, 8, 0, 0>",
            "c3": "mlp_train_kernel<64, 32, 1, 8, 3, 2>" if fused else
                  "mlp_train_kernel<64, 32, 1, 8, 0, 0>",
            "c4": "mlp_train_kernel<64, 64, 3, 4, 0, 0>", "c5": "wide_train_kernel<4>"}[which]


def run_workload(torch, which: str, steps: int, warmup: int, lds_peak_gbs: float,
                 precision: str = "fp16", batches=None, profiled: int = 10) -> dict:
    """One BASELINE training config on device-resident synthetic batches:
    `steps` timed training steps (no profiling events), then `profiled` steps
    with every phase timed (medians per kernel), then forward-only passes over
    the same batch, timed separately, and the reference-rate kernels."""
    from tiny_metal_nn import Trainer
    if which == "c2":
        d, levels, feats, log2t, base, scale, hidden, nhl, m, loss, n = (
            2, 16, 2, 15, 16.0, 1.5, 64, 2, 3, "RelativeL2", B_TRAIN)
    else:
        d, levels, feats, log2t, base, scale, hidden, nhl, m, loss, n = OTHER_WORKLOADS[which]
    dev = torch.device("cuda:0")
    cfg = _config(d, levels, feats, log2t, base, scale, hidden, nhl, loss, n, precision)
    if batches is None:
        gen = torch.Generator(device=dev).manual_seed(7)
        batches = [workload_batch(torch, which, n, gen, dev) for _ in range(2)]
    loss_dev = torch.zeros(steps + warmup + profiled + 1, device=dev)
    tr = Trainer.from_config(cfg, n_input=d, n_output=m)
    ins = tr.inspect_runtime()

    def step(i):
        x, y = batches[i % len(batches)]
        tr.training_step_device(x.data_ptr(), y.data_ptr(), n, loss_dev[i].data_ptr())

    for i in range(warmup):
        step(i)
    tr.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(warmup + i)
    tr.synchronize()
    el = time.perf_counter() - t0
    tr.set_training_step_profiling(True, 1)
    for i in range(profiled):
        step(warmup + steps + i)
    samples = tr.training_step_profile_samples()
    tr.set_training_step_profiling(False)
    out = torch.empty(n, m, device=dev)
    x = batches[0][0]
    for _ in range(3):
        tr.inference_device(x.data_ptr(), out.data_ptr(), n)
    tr.synchronize()
    fwd_iters = max(5, steps)
    t1 = time.perf_counter()
    for _ in range(fwd_iters):
        tr.inference_device(x.data_ptr(), out.data_ptr(), n)
    tr.synchronize()
    fwd = (time.perf_counter() - t1) / fwd_iters
    rates = tr.debug_hash_rates(x.data_ptr(), n, sorted=True, reps=5)
    losses = loss_dev.cpu().numpy()
    tr.close()
    fused = bool(ins.get("train_fused_scatter"))
    inp = 32 if levels * feats <= 32 else 64
    mlp_params = (levels * feats * hidden + hidden + (nhl - 1) * (hidden * hidden + hidden)
                  + hidden * m + m)
    models = kernel_models(d, levels, feats, m, inp, hidden, nhl, levels * feats << log2t,
                           mlp_params)
    lm = which in ("c3", "c4", "c5")
    names = {"encode": f"encode_level_kernel<{d}, {feats}>" if lm
             else f"encode_features_kernel<{d}, {feats}>",
             "mlp": mlp_kernel_name(which, fused, precision),
             "scatter": f"hash_scatter_level_kernel<{d}, {feats}>" if lm
             else f"hash_scatter_kernel<{d}, {feats}>",
             "adam": f"finish_step_kernel<{feats}, false>"}
    ph = median_phases(samples)
    per_kernel = kernel_rooflines(ph, models, names, n, fused, (inp, nhl, ins["waves_per_block_train"]),
                                  lds_peak_gbs, rates, fp32=precision == "fp32")
    return {"workload": which, "precision": precision, "batch": n,
            "encoding": f"{d}D L{levels} F{feats} T2^{log2t} base{base:g} x{scale:g}",
            "mlp": f"{inp}->{hidden}x{nhl}->{m}", "loss": loss,
            "train_samples_per_s": round(n * steps / el, 1), "ms_per_step": round(el * 1e3 / steps, 4),
            "steps": steps, "warmup": warmup,
            "forward_samples_per_s": round(n / fwd, 1), "forward_ms": round(fwd * 1e3, 4),
            "phase_us_median": {k: round(v, 2) for k, v in ph.items()},
            "profiled_steps": int(len(samples)),
            "kernel_rooflines": per_kernel,
            "loss_first_last": [round(float(losses[0]), 6),
                                round(float(losses[warmup + steps + profiled - 1]), 6)]}


def trace_summary(path: str) -> int:
    """Per-kernel duration statistics of a rocprofv3 kernel trace CSV
    (--kernel-trace --output-format csv): dispatch count, mean, median, min,
    max in microseconds, and the median over the dispatches after each
    kernel's first 20 (the warmup steps of a bench run)."""
    import csv
    rows = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            name = r.get("Kernel_Name") or r.get("KernelName") or r.get("kernel_name")
            t0 = int(r.get("Start_Timestamp") or r.get("BeginNs") or 0)
            t1 = int(r.get("End_Timestamp") or r.get("EndNs") or 0)
            rows.setdefault(name, []).append((t0, (t1 - t0) / 1e3))
    print(f"# {path}")
    print("| kernel | dispatches | mean us | median us | min us | max us | median us after first 20 |")
    print("|---|---|---|---|---|---|---|")
    for name, v in sorted(rows.items(), key=lambda kv: -sum(x for _, x in kv[1])):
        v.sort()
        us = np.array([x for _, x in v])
        steady = us[20:] if len(us) > 20 else us
        short = name if len(name) < 110 else name[:107] + "..."
        print(f"| `{short}` | {len(us)} | {us.mean():.2f} | {np.median(us):.2f} | {us.min():.2f} | "
              f"{us.max():.2f} | {np.median(steady):.2f} |")
    return 0



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
    ap.add_argument("--workload", default="c2", choices=["c2", "c3", "c4", "c5", *TILED_WORKLOADS])
    ap.add_argument("--no-workloads", action="store_true",
                    help="skip the C2-fp32, C3-C5 and Tiled entries of the default line")
    ap.add_argument("--trace-summary", metavar="CSV", default=None,
                    help="print per-kernel duration statistics of a rocprofv3 kernel trace")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (5 launches): the "
                         "known-size reference for FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.trace_summary:
        return trace_summary(args.trace_summary)
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
    dev = torch.device("cuda:0")
    if args.workload in TILED_WORKLOADS:
        r = run_tiled(torch, args.workload, args.steps, args.warmup)
        print(json.dumps({
            "metric": f"train samples/s ({args.workload}); forward-only samples/s",
            "value": r["train_samples_per_s"], "unit": "samples/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": r["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "f32 MFMA (fp32 accumulate) / f32 encode+Adam / i32 hash grads",
            "data": "synthetic (see run_tiled)", "config": {"workload": args.workload}, **r}),
            flush=True)
        return 0
    if args.workload != "c2":
        probe = Trainer.from_config(C2_CONFIG, n_input=2, n_output=3)
        lds_peak = probe.debug_lds_rate(10) / 1e9
        probe.close()
        r = run_workload(torch, args.workload, args.steps, args.warmup, lds_peak)
        print(json.dumps({
            "metric": f"train samples/s ({args.workload}); forward-only samples/s",
            "value": r["train_samples_per_s"], "unit": "samples/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": r["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "f16 MFMA / f32 encode+Adam / i32 hash grads",
            "data": "synthetic (see workload_batch)", "config": {"workload": args.workload},
            "lds_peak_GBps": round(lds_peak, 1), **r}), flush=True)
        return 0
    img = make_image(torch, 1234, dev)
    gen = torch.Generator(device=dev).manual_seed(7)
    nb = 4
    xs = [torch.rand(B_TRAIN, 2, device=dev, generator=gen) for _ in range(nb)]
    ys = [sample_bilinear(torch, img, x) for x in xs]
    loss_dev = torch.zeros(args.steps + args.warmup + PROFILED_STEPS + 1, device=dev)
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

    # timed region: the K steps exactly as a caller runs them
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(args.warmup + i)
    tr.synchronize()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    train_sps = B_TRAIN * args.steps / elapsed
    # kernel durations: PROFILED_STEPS more steps with every phase timed
    tr.set_training_step_profiling(True, 1)
    for i in range(PROFILED_STEPS):
        step(args.warmup + args.steps + i)
    samples = tr.training_step_profile_samples()
    tr.set_training_step_profiling(False)
    losses = loss_dev.cpu().numpy()
    first_loss = float(losses[0])
    last_loss = float(losses[args.warmup + args.steps + PROFILED_STEPS - 1])
    if not (math.isfinite(last_loss) and last_loss < first_loss):
        print(f"bench.py: training did not progress (loss {first_loss} -> {last_loss})",
              file=sys.stderr)
        return 1
    print(f"# timed {args.steps} steps in {elapsed * 1e3:.1f} ms; loss {first_loss:.5f} -> "
          f"{last_loss:.5f}", file=sys.stderr, flush=True)

    # reference rates at this shape over a batch in the step's Morton order:
    # gather-only (the encode's loads), atomic-only and flag-store-only (the
    # scatter's memory operations) -- the achievable denominators; the LDS
    # read rate (the MLP kernel's LDS peak)
    rates = tr.debug_hash_rates(xs[0].data_ptr(), B_TRAIN, sorted=True, reps=20)
    lds_peak = tr.debug_lds_rate(10) / 1e9

    # inference on the C1 shape (same field, fp32, 2^16 points per call)
    xi = torch.rand(B_INFER, 2, device=dev, generator=gen)
    yi = torch.empty(B_INFER, 3, device=dev)
    for _ in range(10):
        tr.inference_device(xi.data_ptr(), yi.data_ptr(), B_INFER)
    tr.synchronize()
    torch.cuda.synchronize()
    iters = max(50, args.steps)
    t2 = time.perf_counter()
    for _ in range(iters):
        tr.inference_device(xi.data_ptr(), yi.data_ptr(), B_INFER)
    tr.synchronize()
    torch.cuda.synchronize()
    infer_sps = B_INFER * iters / (time.perf_counter() - t2)
    # five groups of five more calls with an event pair around the kernel
    igroups = []
    for _ in range(5):
        tr.set_training_step_profiling(True, 1)
        for _ in range(5):
            tr.inference_device(xi.data_ptr(), yi.data_ptr(), B_INFER)
        igroups.append(tr.training_step_profile())
        tr.set_training_step_profiling(False)
    infer_gather = tr.debug_hash_rates(xi.data_ptr(), B_INFER, sorted=False, reps=20)["gather_us"]
    tr.close()
    infer_roof = infer_roofline(igroups, infer_gather)

    fused = bool(ins.get("train_fused_scatter"))
    ph = median_phases(samples)
    names = {"encode": "encode_features_kernel<2, 2>", "mlp": mlp_kernel_name("c2", fused, "fp16"),
             "scatter": "hash_scatter_kernel<2, 2>", "adam": "finish_step_kernel<2, false>"}
    traffic = {k: traffic_from_profiles(k) for k in ("encode", "mlp", "adam")}
    per_kernel = kernel_rooflines(ph, kernel_models(), names, B_TRAIN, fused,
                                  (32, 2, ins["waves_per_block_train"]), lds_peak, rates, traffic)
    roofline = next((r for r in per_kernel if r["kernel"] == names["mlp"]), None)
    if roofline is not None:
        roofline = dict(roofline, statistic=f"median kernel duration over {len(samples)} profiled "
                                            "steady-state steps after the timed region")

    workloads = {}
    if not args.no_workloads:
        for which, prec in (("c2", "fp32"), ("c3", "fp16"), ("c4", "fp16"), ("c5", "fp16")):
            batches = [(xs[k], ys[k]) for k in range(2)] if which == "c2" else None
            key = which + ("_fp32" if prec == "fp32" else "")
            workloads[key] = run_workload(torch, which, 20, 5, lds_peak, prec, batches)
            print(f"# {key}: {workloads[key]['ms_per_step']} ms/step", file=sys.stderr, flush=True)
        for which in TILED_WORKLOADS:
            workloads[which] = run_tiled(torch, which, 50, 5)
            print(f"# {which}: {workloads[which]['ms_per_step']} ms/step", file=sys.stderr, flush=True)

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
        "phase_us_median": {k: round(v, 2) for k, v in ph.items()},
        "profiled_steps": int(len(samples)),
        "lds_peak_GBps": round(lds_peak, 1),
        "loss_first_last": [round(first_loss, 6), round(last_loss, 6)],
        "roofline": roofline,
        "kernel_rooflines": per_kernel,
        "workloads": workloads,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
