"""GPU parity over seeded random shapes beyond the named geometries: spatial
dims 2-4, levels x features 4-64, table sizes 2^10-2^19, hidden widths 32-256
with one to four hidden layers, 1-20 outputs, fp32 and fp16 precision, three
losses and batches of 1 to 70001 points. Each shape runs whichever family the
planner picks (fused kernels or the layer-wise path) and is checked against
the oracle on identical seeded inputs: inference within 1e-5 (element-wise,
against |ref| + rms) and the loss of one training step within 1e-5 (fp32) or
3e-3 (fp16, split-fp16 forward) relative. Marked gpu."""
from __future__ import annotations

import random
import sys

import numpy as np
import pytest

from test_gpu_parity import make_trainer, omodel

pytestmark = pytest.mark.gpu


def _shapes(seed: int, count: int) -> list[tuple]:
    rng = random.Random(seed)
    out = []
    while len(out) < count:
        d = rng.choice([2, 3, 4])
        F, L = rng.choice([(2, 16), (2, 8), (4, 16), (4, 8), (1, 16), (2, 4), (1, 4), (4, 2)])
        log2T = rng.randint(10, 19)
        base = rng.choice([2.0, 4.0, 8.0, 16.0])
        scale = rng.choice([1.3, 1.5, 2.0])
        H = rng.choice([32, 48, 64, 64, 96, 128, 256])
        NHL = rng.randint(1, 4)
        M = rng.randint(1, 20)
        prec = rng.choice(["fp32", "fp16"])
        loss = rng.choice(["L2", "L1", "RelativeL2"])
        n = rng.choice([1, 33, 5003, 70001])
        out.append((d, L, F, log2T, base, scale, H, NHL, M, prec, loss, n))
    return out


SHAPES = _shapes(20261202, 24)


@pytest.mark.parametrize("idx", range(len(SHAPES)))
def test_random_shape_inference_and_step_loss(oracle, idx):
    d, L, F, log2T, base, scale, H, NHL, M, prec, loss, n = SHAPES[idx]
    print(f"shape {idx}: d{d} L{L} F{F} T2^{log2T} H{H}x{NHL} M{M} {prec} {loss} n{n}", flush=True)
    sys.stdout.flush()
    enc = dict(n_levels=L, n_features_per_level=F, log2_hashmap_size=log2T,
               base_resolution=base, per_level_scale=scale)
    net = dict(n_neurons=H, n_hidden_layers=NHL)
    prng = np.random.default_rng(idx)
    with make_trainer(d, M, enc, net, loss=loss, precision=prec, batch=max(n, 1024),
                      hash_range=0.5) as tr:
        pos = prng.random((n, d), dtype=np.float32)
        hw, mw = tr.get_weights()
        out = tr.inference(pos)
        ref = oracle.forward(omodel(oracle, tr), hw, mw, pos)
        tol = 1e-5 * (np.abs(ref) + np.sqrt((ref.astype(np.float64) ** 2).mean()))
        assert np.all(np.abs(out - ref) <= tol), float(np.abs(out - ref).max())
        tgt = prng.random((n, M), dtype=np.float32)
        params = np.concatenate([hw, mw])
        m1, m2 = np.zeros_like(params), np.zeros_like(params)
        lg = tr.training_step(pos, tgt)
        lo = oracle.training_step(omodel(oracle, tr), oracle.adam(1e-2, 1e-2), 0, params, m1, m2,
                                  pos, tgt)
        assert lg == pytest.approx(lo, rel=1e-5 if prec == "fp32" else 3e-3), (lg, lo)


STEP_SHAPES = _shapes(7027, 8)


@pytest.mark.parametrize("idx", range(len(STEP_SHAPES)))
def test_random_shape_three_steps_track_oracle(oracle, idx):
    """Three fused training steps (Adam in between) on random shapes: each
    step's loss against the oracle's step on the same batch and state, within
    1e-4 (fp32) or 1e-2 (fp16) relative."""
    d, L, F, log2T, base, scale, H, NHL, M, prec, loss, n = STEP_SHAPES[idx]
    n = max(n, 33)
    print(f"steps {idx}: d{d} L{L} F{F} T2^{log2T} H{H}x{NHL} M{M} {prec} {loss} n{n}", flush=True)
    sys.stdout.flush()
    enc = dict(n_levels=L, n_features_per_level=F, log2_hashmap_size=log2T,
               base_resolution=base, per_level_scale=scale)
    net = dict(n_neurons=H, n_hidden_layers=NHL)
    prng = np.random.default_rng(100 + idx)
    with make_trainer(d, M, enc, net, loss=loss, precision=prec, batch=max(n, 1024),
                      hash_range=0.5) as tr:
        hw, mw = tr.get_weights()
        m = omodel(oracle, tr)
        a = oracle.adam(1e-2, 1e-2)
        params = np.concatenate([hw, mw])
        m1, m2 = np.zeros_like(params), np.zeros_like(params)
        for step in range(3):
            pos = prng.random((n, d), dtype=np.float32)
            tgt = prng.random((n, M), dtype=np.float32)
            lg = tr.training_step(pos, tgt)
            lo = oracle.training_step(m, a, step, params, m1, m2, pos, tgt)
            assert lg == pytest.approx(lo, rel=1e-4 if prec == "fp32" else 1e-2), (step, lg, lo)
