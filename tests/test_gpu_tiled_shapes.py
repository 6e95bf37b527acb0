"""GPU parity of the layer-wise (Tiled) path: the KernelSpec shapes no fused
kernel instantiates (kernel_spec.cpp:12-44: hidden widths up to 512, up to
32 levels x 4 features = 128 inputs, any number of outputs, fp32 training at
width 128) run one fp32 matrix product per layer (layer_kernels.hpp); each
is checked against the oracle on identical seeded inputs. Marked gpu.

Tolerances: fp32 outputs 1e-5 relative (element-wise, against |ref| + rms);
fp32 MLP gradients 1e-5 of the tensor's max; int32 hash gradients exact on
>= 99% of entries (95% for the 8-layer shape) and within 16 units elsewhere;
visited set exact; loss after N Adam steps within 1%.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from test_gpu_parity import make_trainer, omodel, rel_tensor

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


LW_GEOMS = {
    # name: (dims, encoding, network, outputs, precision)
    "h256_3d": (3, dict(n_levels=8, n_features_per_level=2, log2_hashmap_size=14,
                        base_resolution=8.0, per_level_scale=2.0),
                dict(n_neurons=256, n_hidden_layers=2), 4, "fp32"),
    "h512_2d": (2, dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=14,
                        base_resolution=16.0, per_level_scale=1.5),
                dict(n_neurons=512, n_hidden_layers=1), 3, "fp32"),
    "in128_2d": (2, dict(n_levels=32, n_features_per_level=4, log2_hashmap_size=12,
                         base_resolution=4.0, per_level_scale=1.3),
                 dict(n_neurons=64, n_hidden_layers=2), 3, "fp32"),
    "m32_3d": (3, dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=14,
                       base_resolution=16.0, per_level_scale=1.5),
               dict(n_neurons=64, n_hidden_layers=1), 32, "fp32"),
    "w128_fp32_4d": (4, dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=16,
                             base_resolution=8.0, per_level_scale=1.4),
                     dict(n_neurons=128, n_hidden_layers=4), 4, "fp32"),
    "w128_in64_fp16": (3, dict(n_levels=16, n_features_per_level=4, log2_hashmap_size=14,
                               base_resolution=16.0, per_level_scale=1.5),
                       dict(n_neurons=128, n_hidden_layers=2), 2, "fp16"),
    "h96_8layers": (3, dict(n_levels=4, n_features_per_level=1, log2_hashmap_size=10,
                            base_resolution=4.0, per_level_scale=2.0),
                    dict(n_neurons=96, n_hidden_layers=8), 1, "fp32"),
    # a width that is not a multiple of 4: rows unaligned for 16-byte access,
    # so the output layer's products take the tile kernel, not the narrow ones
    "h98_2d": (2, dict(n_levels=8, n_features_per_level=2, log2_hashmap_size=12,
                       base_resolution=8.0, per_level_scale=1.5),
               dict(n_neurons=98, n_hidden_layers=2), 3, "fp32"),
    # the output layer at the narrow kernels' limit (16 outputs) and one past
    # it (17: the tile kernel)
    "m16_h96_2d": (2, dict(n_levels=8, n_features_per_level=2, log2_hashmap_size=12,
                           base_resolution=8.0, per_level_scale=1.5),
                   dict(n_neurons=96, n_hidden_layers=1), 16, "fp32"),
    "m17_h96_2d": (2, dict(n_levels=8, n_features_per_level=2, log2_hashmap_size=12,
                           base_resolution=8.0, per_level_scale=1.5),
                   dict(n_neurons=96, n_hidden_layers=1), 17, "fp32"),
}


def _trainer(name, **kw):
    d, enc, net, m_out, prec = LW_GEOMS[name]
    kw.setdefault("precision", prec)
    return make_trainer(d, m_out, enc, net, **kw)


@pytest.mark.parametrize("name", list(LW_GEOMS))
def test_tiled_plan_and_inference(oracle, name):
    _say(f"tiled inference {name}")
    d, _, _, m_out, _ = LW_GEOMS[name]
    rng = np.random.default_rng(3)
    with _trainer(name, hash_range=0.5) as tr:
        assert tr.network_plan()["selected_family"] == "Tiled"
        assert tr.inspect_runtime()["family_name"] == "Tiled"
        hw, mw = tr.get_weights()
        oh, om = oracle.init_params(omodel(oracle, tr), 42, 0.5)
        assert np.array_equal(hw, oh) and np.array_equal(mw, om)
        for n in (1, 70, 3001):
            pos = rng.random((n, d), dtype=np.float32)
            out = tr.inference(pos)
            ref = oracle.forward(omodel(oracle, tr), hw, mw, pos)
            tol = 1e-5 * (np.abs(ref) + np.sqrt((ref.astype(np.float64) ** 2).mean()))
            assert np.all(np.abs(out - ref) <= tol), (n, float(np.abs(out - ref).max()))
        # forward_for_training: caller's point order through the Morton sort
        a = tr.forward_for_training(pos)
        tol = 1e-5 * (np.abs(ref) + np.sqrt((ref.astype(np.float64) ** 2).mean()))
        assert np.all(np.abs(a - ref) <= tol)


def test_tiled_inference_beyond_one_forward_chunk(oracle):
    """A forward pass over more points than one layer-wise forward chunk
    (2^18 points, two ping-pong activation buffers): the second chunk's
    outputs land in the right rows (bit-identical to separate calls over the
    same two ranges, which run the same kernels on the same points) and a
    random sample matches the oracle within 1e-5."""
    name = "in128_2d"
    _say(f"tiled inference beyond one chunk {name}")
    d = LW_GEOMS[name][0]
    rng = np.random.default_rng(17)
    n = (1 << 18) + 3001
    with _trainer(name, hash_range=0.5) as tr:
        pos = rng.random((n, d), dtype=np.float32)
        out = tr.inference(pos)
        first = tr.inference(pos[: 1 << 18])
        rest = tr.inference(pos[1 << 18:])
        assert np.array_equal(out, np.concatenate([first, rest]))
        hw, mw = tr.get_weights()
        idx = np.sort(rng.choice(n, 2048, replace=False))
        ref = oracle.forward(omodel(oracle, tr), hw, mw, pos[idx])
        tol = 1e-5 * (np.abs(ref) + np.sqrt((ref.astype(np.float64) ** 2).mean()))
        assert np.all(np.abs(out[idx] - ref) <= tol)


@pytest.mark.parametrize("name", list(LW_GEOMS))
def test_tiled_backward_matches_oracle(oracle, name):
    _say(f"tiled backward {name}")
    d, _, _, m_out, _ = LW_GEOMS[name]
    rng = np.random.default_rng(5)
    with _trainer(name, hash_range=0.5, batch=1 << 16) as tr:
        hw, mw = tr.get_weights()
        pos = rng.random((2503, d), dtype=np.float32)
        g = rng.normal(0, 1.0, (2503, m_out)).astype(np.float32)
        tr.zero_gradients()
        tr.backward_accumulate(pos, g)
        gh, gm = tr.debug_gradients()
        mask = tr.debug_active_mask()
        ogh, ogm, omask, _, _ = oracle.forward_backward(omodel(oracle, tr), hw, mw, pos, d_out=g)
        assert np.array_equal(mask, omask)
        assert rel_tensor(gm, ogm) <= 1e-5
        diff = np.abs(gh.astype(np.int64) - ogh.astype(np.int64))
        # int32 truncation: an fp32 ulp of d_feat may flip one unit. Eight
        # fp32 layers reassociated (tiled products vs the oracle's sequential
        # sums) move d_feat by a few ulps, and the 4096-entry table of
        # h96_8layers sums ~10 contributions per entry
        exact = 0.95 if name == "h96_8layers" else 0.99
        assert (diff == 0).mean() > exact and diff.max() <= 16, int(diff.max())


@pytest.mark.parametrize("name", ["h256_3d", "in128_2d", "m32_3d", "w128_fp32_4d", "h96_8layers",
                                  "h98_2d"])
@pytest.mark.parametrize("loss", ["L2", "L1"])
def test_tiled_training_loss_tracks_oracle(oracle, name, loss):
    _say(f"tiled training {name} {loss}")
    d, _, _, m_out, _ = LW_GEOMS[name]
    rng = np.random.default_rng(7)
    n, steps = 4096, 6
    with _trainer(name, loss=loss, batch=n) as tr:
        hw, mw = tr.get_weights()
        m = omodel(oracle, tr)
        a = oracle.adam(1e-2, 1e-2)
        params = np.concatenate([hw, mw])
        m1, m2 = np.zeros_like(params), np.zeros_like(params)
        for step in range(steps):
            pos = rng.random((n, d), dtype=np.float32)
            tgt = np.sin(3 * pos[:, :1] + np.arange(m_out, dtype=np.float32)[None] * 0.3 +
                         step).astype(np.float32)
            lg = tr.training_step(pos, tgt)
            lo = oracle.training_step(m, a, step, params, m1, m2, pos, tgt)
            assert lg == pytest.approx(lo, rel=0.01), (step, lg, lo)
        _, mw2 = tr.get_weights()
        assert rel_tensor(mw2, params[len(hw):]) <= 1e-3


@pytest.mark.parametrize("name", ["h256_3d", "w128_fp32_4d", "in128_2d"])
def test_tiled_evaluate_with_gradient(oracle, name):
    _say(f"tiled evaluate_with_gradient {name}")
    d, _, _, m_out, _ = LW_GEOMS[name]
    rng = np.random.default_rng(9)
    with _trainer(name, hash_range=0.5) as tr:
        hw, mw = tr.get_weights()
        pos = rng.random((555, d), dtype=np.float32)
        out, jac = tr.evaluate_with_gradient(pos)
        oout, ojac = oracle.evaluate_with_gradient(omodel(oracle, tr), hw, mw, pos)
        for got, ref in ((out, oout), (jac, ojac)):
            tol = 1e-5 * (np.abs(ref) + np.sqrt((ref.astype(np.float64) ** 2).mean()))
            assert np.all(np.abs(got - ref) <= tol), float(np.abs(got - ref).max())


def test_tiled_fused_step_matches_oracle(oracle):
    """The fused step on the layer-wise path (partial rows reduced and Adam
    applied by finish_step_kernel) against the oracle's step: loss within
    1e-5, MLP weights within fp32 tolerance."""
    _say("tiled fused vs oracle one step")
    d, _, _, m_out, _ = LW_GEOMS["h512_2d"]
    rng = np.random.default_rng(13)
    with _trainer("h512_2d", hash_range=0.5, batch=3000) as tr:
        hw, mw = tr.get_weights()
        params = np.concatenate([hw, mw])
        m1, m2 = np.zeros_like(params), np.zeros_like(params)
        pos = rng.random((3000, d), dtype=np.float32)
        tgt = rng.random((3000, m_out), dtype=np.float32)
        lg = tr.training_step(pos, tgt)
        lo = oracle.training_step(omodel(oracle, tr), oracle.adam(1e-2, 1e-2), 0, params, m1, m2,
                                  pos, tgt)
        assert lg == pytest.approx(lo, rel=1e-5)
        _, mw2 = tr.get_weights()
        dp = np.abs(mw2.astype(np.float64) - params[len(hw):])
        assert (dp <= 1e-5 * np.abs(params[len(hw):]) + 1e-7).mean() > 0.999
