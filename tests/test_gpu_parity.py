"""GPU parity: the HIP path through the C-ABI vs the CPU oracle on identical
seeded inputs (marked gpu; run on an MI355X with `pytest -m gpu`).

Tolerances (north_star):
  * hash indices, corner weights, Philox init, active-hash mask: bit-exact;
  * fp32 encodings: bit-exact (no FMA contraction on either side);
  * fp32 outputs: |gpu - oracle| <= 1e-5 * (|oracle| + rms(oracle));
  * fp16-compute MLP outputs / gradients: per-tensor max error <= 2e-3 of the
    tensor's max magnitude;
  * loss after N Adam steps: within 1% of the oracle.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def make_trainer(n_input, n_output, enc, net, loss="L2", lr=1e-2, batch=1 << 16,
                 precision="fp32", hash_adam="lazy", morton=True, seed=42, hash_range=1e-4,
                 huber_delta=None, family="auto"):
    from tiny_metal_nn import Trainer
    lo = {"otype": loss}
    if huber_delta is not None:
        lo["huber_delta"] = huber_delta
    cfg = {"encoding": dict(otype="HashGrid", **enc), "network": dict(otype="FullyFusedMLP", **net),
           "loss": lo, "optimizer": {"otype": "Adam", "learning_rate": lr},
           "weight_init": {"seed": seed, "hash_grid_range": hash_range},
           "batch_size": batch,
           "mi355x": {"precision": precision, "hash_adam": hash_adam, "morton_sort": morton,
                      "family": family}}
    return Trainer.from_config(cfg, n_input=n_input, n_output=n_output)


def omodel(oracle, tr):
    c = tr.config
    e, n = c["encoding"], c["network"]
    return oracle.model(e["n_input_dims"], e["n_levels"], e["n_features_per_level"],
                        e["log2_hashmap_size"], e["base_resolution"], e["per_level_scale"],
                        n["n_neurons"], n["n_hidden_layers"], n["n_output_dims"],
                        c["loss"]["otype"], c["loss"].get("huber_delta", 1.0))


def rel_tensor(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    scale = np.abs(b).max()
    return float(np.abs(a - b).max() / scale) if scale > 0 else float(np.abs(a).max())


C2_ENC = dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=15, base_resolution=16.0,
              per_level_scale=1.5)
C2_NET = dict(n_neurons=64, n_hidden_layers=2)

GEOMS = {
    "2d_f2": (2, dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=15,
                      base_resolution=16.0, per_level_scale=1.5), dict(n_neurons=64, n_hidden_layers=2), 3),
    "3d_f2": (3, dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=19,
                      base_resolution=16.0, per_level_scale=128 ** (1 / 15)),
              dict(n_neurons=64, n_hidden_layers=1), 16),
    "3d_f4": (3, dict(n_levels=16, n_features_per_level=4, log2_hashmap_size=16,
                      base_resolution=16.0, per_level_scale=1.5), dict(n_neurons=64, n_hidden_layers=3), 1),
    "3d_f1": (3, dict(n_levels=8, n_features_per_level=1, log2_hashmap_size=12,
                      base_resolution=4.0, per_level_scale=2.0), dict(n_neurons=32, n_hidden_layers=1), 2),
    "4d_f2": (4, dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=16,
                      base_resolution=8.0, per_level_scale=1.4), dict(n_neurons=64, n_hidden_layers=2), 4),
    "small": (3, dict(n_levels=2, n_features_per_level=2, log2_hashmap_size=10,
                      base_resolution=4.0, per_level_scale=2.0), dict(n_neurons=8, n_hidden_layers=1), 1),
    # 16 MB per level: the hash-grid backward runs level-major (large tables)
    "3d_bigT": (3, dict(n_levels=4, n_features_per_level=2, log2_hashmap_size=21,
                        base_resolution=16.0, per_level_scale=2.0), dict(n_neurons=64, n_hidden_layers=1), 1),
    "4d_bigT": (4, dict(n_levels=4, n_features_per_level=2, log2_hashmap_size=21,
                        base_resolution=8.0, per_level_scale=1.4), dict(n_neurons=64, n_hidden_layers=2), 4),
}


# ------------------------------------------------------------ init / RNG --

def test_philox_golden_on_gpu():
    from tiny_metal_nn import philox_uniform
    _say("philox golden")
    g = json.loads((GOLDEN / "philox_seed42_golden.json").read_text())
    out = philox_uniform(g["seed"], g["counter_base"], g["count"], g["low"], g["high"])
    assert np.array_equal(out[:8].view(np.uint32),
                          np.array(g["first8"], np.float32).view(np.uint32))


@pytest.mark.parametrize("name", list(GEOMS))
def test_seeded_init_matches_oracle(oracle, name):
    _say(f"init {name}")
    d, enc, net, m_out = GEOMS[name]
    with make_trainer(d, m_out, enc, net, seed=1234, hash_range=1e-4) as tr:
        hw, mw = tr.get_weights()
        oh, om = oracle.init_params(omodel(oracle, tr), 1234, 1e-4)
        assert np.array_equal(hw, oh) and np.array_equal(mw, om)
        assert np.array_equal(tr.debug_resolutions(), oracle.resolutions(omodel(oracle, tr)))


# ---------------------------------------------------------------- encode --

@pytest.mark.parametrize("name", list(GEOMS))
def test_encode_bit_exact(oracle, name):
    _say(f"encode {name}")
    d, enc, net, m_out = GEOMS[name]
    rng = np.random.default_rng(7)
    with make_trainer(d, m_out, enc, net, hash_range=0.5) as tr:
        hw, _ = tr.get_weights()
        pos = rng.random((1000, d), dtype=np.float32)
        pos[:3] = 0.0
        pos[3:6] = np.float32(0.999999)
        feats, idx, w = tr.debug_encode(pos, with_corners=True)
        of, oi, ow = oracle.encode(omodel(oracle, tr), hw, pos, with_corners=True)
        C = 1 << d
        assert np.array_equal(idx, oi[:, :, :C])
        assert np.array_equal(w.view(np.uint32), ow[:, :, :C].view(np.uint32))
        if d == 2:
            assert np.all(ow[:, :, 4:] == 0.0)
        assert np.array_equal(feats.view(np.uint32), of.view(np.uint32))


# ------------------------------------------------------------- inference --

@pytest.mark.parametrize("name", list(GEOMS))
@pytest.mark.parametrize("n", [1, 33, 4099])
def test_inference_fp32_matches_oracle(oracle, name, n):
    _say(f"inference {name} n={n}")
    d, enc, net, m_out = GEOMS[name]
    rng = np.random.default_rng(n)
    with make_trainer(d, m_out, enc, net, hash_range=0.5) as tr:
        hw, mw = tr.get_weights()
        pos = rng.random((n, d), dtype=np.float32)
        out = tr.inference(pos)
        ref = oracle.forward(omodel(oracle, tr), hw, mw, pos)
        tol = 1e-5 * (np.abs(ref) + np.sqrt((ref.astype(np.float64) ** 2).mean()))
        assert np.all(np.abs(out - ref) <= tol), float(np.abs(out - ref).max())


def test_inference_empty_and_errors():
    from tiny_metal_nn import DTypeError
    d, enc, net, m_out = GEOMS["small"]
    with make_trainer(d, m_out, enc, net) as tr:
        assert tr.inference(np.zeros((0, 3), np.float32)).shape == (0, 1)
        with pytest.raises(DTypeError):
            tr.inference(np.zeros((4, 3), np.float64))
        with pytest.raises(ValueError):
            tr.training_step(np.zeros((0, 3), np.float32), np.zeros((0, 1), np.float32))


# ------------------------------------------------------------- gradients --

def _grads_vs_oracle(oracle, name, precision, n, seed, family="auto"):
    d, enc, net, m_out = GEOMS[name]
    rng = np.random.default_rng(seed)
    with make_trainer(d, m_out, enc, net, precision=precision, hash_range=0.5,
                      batch=1 << 20, family=family) as tr:
        hw, mw = tr.get_weights()
        pos = rng.random((n, d), dtype=np.float32)
        if precision == "fp16":
            # the fp16 forward is not the oracle's fp32 one: keep ReLU masks
            # decidable (see away_from_relu_kinks)
            pos = away_from_relu_kinks(oracle, tr, hw, mw, pos)
            assert len(pos) > 0.95 * n
        g = rng.normal(0, 1.0, (len(pos), m_out)).astype(np.float32)
        tr.zero_gradients()
        tr.backward_accumulate(pos, g)
        gh, gm = tr.debug_gradients()
        mask = tr.debug_active_mask()
        ogh, ogm, omask, _, _ = oracle.forward_backward(omodel(oracle, tr), hw, mw, pos, d_out=g)
        return gh, gm, mask, ogh, ogm, omask, tr.config


@pytest.mark.parametrize("name", ["2d_f2", "3d_f2", "3d_f4", "3d_f1", "4d_f2", "small", "3d_bigT",
                                  "4d_bigT"])
def test_backward_fp32_matches_oracle(oracle, name):
    _say(f"backward fp32 {name}")
    gh, gm, mask, ogh, ogm, omask, _ = _grads_vs_oracle(oracle, name, "fp32", 2051, 3)
    assert np.array_equal(mask, omask)           # visited set: exact
    assert rel_tensor(gm, ogm) <= 1e-5
    diff = np.abs(gh.astype(np.int64) - ogh.astype(np.int64))
    # int32 fixed point: an fp32 ulp in d_feat may flip one truncation
    assert (diff == 0).mean() > 0.99 and diff.max() <= 16, int(diff.max())


@pytest.mark.parametrize("name", ["2d_f2", "3d_f2", "3d_f4", "4d_f2", "3d_bigT", "4d_bigT"])
def test_backward_fp16_matches_oracle(oracle, name):
    _say(f"backward fp16 {name}")
    gh, gm, mask, ogh, ogm, omask, _ = _grads_vs_oracle(oracle, name, "fp16", 4096, 4)
    assert np.array_equal(mask, omask)
    assert rel_tensor(gm, ogm) <= 2e-3
    assert rel_tensor(gh, ogh) <= 2e-3


@pytest.mark.parametrize("family,precision", [("Tiled", "fp16"), ("Tiled", "fp32"),
                                              ("SafeDebug", "fp16")])
def test_planner_families_match_oracle(oracle, family, precision):
    """Every family the planner can select runs the same math: the generic
    (Tiled) kernels, and SafeDebug (generic, fp32, input order)."""
    _say(f"family {family} {precision}")
    gh, gm, mask, ogh, ogm, omask, _ = _grads_vs_oracle(oracle, "2d_f2", precision, 3000, 6,
                                                        family=family)
    assert np.array_equal(mask, omask)
    exact = family == "SafeDebug" or precision == "fp32"
    assert rel_tensor(gm, ogm) <= (1e-5 if exact else 2e-3)
    if exact:
        diff = np.abs(gh.astype(np.int64) - ogh.astype(np.int64))
        assert (diff == 0).mean() > 0.99 and diff.max() <= 16
    else:
        assert rel_tensor(gh, ogh) <= 2e-3
    d, enc, net, m_out = GEOMS["2d_f2"]
    with make_trainer(d, m_out, enc, net, precision=precision, family=family) as tr:
        ins = tr.inspect_runtime()
        assert ins["family_name"] == family
        assert tr.network_plan()["selected_family"] == family
        if family == "SafeDebug":
            assert ins["precision"] == 0
        rng = np.random.default_rng(1)
        pos = rng.random((4096, 2), dtype=np.float32)
        tgt = rng.random((4096, m_out), dtype=np.float32)
        l0 = tr.training_step(pos, tgt)
        for _ in range(5):
            l1 = tr.training_step(pos, tgt)
        assert np.isfinite(l1) and l1 < l0


def test_default_plan_is_fully_fused_for_the_image_fit():
    d, enc, net, m_out = GEOMS["2d_f2"]
    with make_trainer(d, m_out, enc, net, precision="fp16") as tr:
        p = tr.network_plan()
        assert p["selected_family"] == "FullyFused" and p["fused_train"]
        assert tr.inspect_runtime()["waves_per_block_train"] == p["train_waves_per_block"]


def test_int_hash_gradients_are_deterministic():
    d, enc, net, m_out = GEOMS["2d_f2"]
    rng = np.random.default_rng(5)
    pos = rng.random((8192, 2), dtype=np.float32)
    g = rng.normal(0, 1.0, (8192, 3)).astype(np.float32)
    with make_trainer(d, m_out, enc, net, hash_range=0.5, batch=1 << 20) as tr:
        tr.zero_gradients()
        tr.backward_accumulate(pos, g)
        a, _ = tr.debug_gradients()
        tr.zero_gradients()
        tr.backward_accumulate(pos, g)
        b, _ = tr.debug_gradients()
        assert np.array_equal(a, b)


def test_accumulate_is_linear():
    """AccumGradientLinearityFourCalls: 4 accumulations of g == 4 * g once
    (MLP grads; hash ints within truncation)."""
    d, enc, net, m_out = GEOMS["3d_f2"]
    rng = np.random.default_rng(8)
    pos = rng.random((3000, 3), dtype=np.float32)
    g = rng.normal(0, 1.0, (3000, m_out)).astype(np.float32)
    with make_trainer(d, m_out, enc, net, hash_range=0.5, batch=1 << 20) as tr:
        tr.zero_gradients()
        for _ in range(4):
            tr.backward_accumulate(pos, g)
        gh4, gm4 = tr.debug_gradients()
        tr.zero_gradients()
        tr.backward_accumulate(pos, 4 * g)
        gh1, gm1 = tr.debug_gradients()
        assert rel_tensor(gm4, gm1) <= 1e-5
        assert np.abs(gh4.astype(np.int64) - gh1.astype(np.int64)).max() <= 4 * 64


# -------------------------------------------------------------- training --

def test_sphere_sdf_trajectory_on_gpu():
    """The reference's published Metal loss curve (examples/sphere_sdf)."""
    torch = pytest.importorskip("torch")
    _say("sphere_sdf trajectory")
    from tiny_metal_nn import Trainer
    g = json.loads((GOLDEN / "sphere_sdf_reference_metrics.json").read_text())
    losses = []
    torch.manual_seed(42)
    with Trainer.from_config(g["config"], n_input=3, n_output=1) as tr:
        for _ in range(50):
            pos = torch.rand(4096, 3, dtype=torch.float32)
            tgt = ((pos - 0.5).norm(dim=1, keepdim=True) - 0.5).to(torch.float32)
            losses.append(tr.training_step(pos.numpy(), tgt.numpy()))
        assert tr.step() == 50
    for k, v in g["convergence"].items():
        assert losses[int(k)] == pytest.approx(v, rel=0.02), (k, losses[int(k)], v)


@pytest.mark.parametrize("precision", ["fp32", "fp16"])
@pytest.mark.parametrize("loss", ["L2", "RelativeL2"])
def test_training_loss_tracks_oracle(oracle, precision, loss):
    """C2-shaped image fit (2D, 16x2, T=2^15, 64x2 MLP, 3 outputs): loss after
    N Adam steps within 1% of the oracle (N = 8192 points, 15 steps)."""
    _say(f"training {precision} {loss}")
    d, enc, net, m_out = GEOMS["2d_f2"]
    rng = np.random.default_rng(17)
    n, steps = 8192, 15
    with make_trainer(d, m_out, enc, net, loss=loss, precision=precision, batch=n) as tr:
        hw, mw = tr.get_weights()
        m = omodel(oracle, tr)
        a = oracle.adam(1e-2, 1e-2)
        params = np.concatenate([hw, mw])
        m1, m2 = np.zeros_like(params), np.zeros_like(params)
        for step in range(steps):
            pos = rng.random((n, 2), dtype=np.float32)
            tgt = np.stack([np.sin(6 * pos[:, 0]), np.cos(5 * pos[:, 1]),
                            pos[:, 0] * pos[:, 1]], 1).astype(np.float32) * 0.5 + 0.5
            lg = tr.training_step(pos, tgt)
            lo = oracle.training_step(m, a, step, params, m1, m2, pos, tgt)
            assert lg == pytest.approx(lo, rel=0.01), (step, lg, lo)
        hw2, mw2 = tr.get_weights()
        tol = 2e-3 if precision == "fp16" else 1e-4
        assert rel_tensor(mw2, params[len(hw):]) <= max(tol, 1e-4) * 50


def test_batch_cap_truncates():
    d, enc, net, m_out = GEOMS["small"]
    from tiny_metal_nn import _lib
    import ctypes
    with make_trainer(d, m_out, enc, net, batch=100) as tr:
        pos = np.random.default_rng(0).random((250, 3), dtype=np.float32)
        tgt = np.zeros((250, 1), np.float32)
        res = _lib.StepResult()
        x = np.ascontiguousarray(pos)
        y = np.ascontiguousarray(tgt)
        _lib.check(tr._lib.tmnn_training_step(tr._h, x.ctypes.data_as(ctypes.c_void_p),
                                              y.ctypes.data_as(ctypes.c_void_p), 250,
                                              ctypes.byref(res)))
        assert res.batch_n == 100 and res.step == 1


# ------------------------------------------------------ split path / state --

def test_forward_for_training_matches_inference_and_order():
    d, enc, net, m_out = GEOMS["3d_f2"]
    rng = np.random.default_rng(10)
    pos = rng.random((5000, 3), dtype=np.float32)
    with make_trainer(d, m_out, enc, net, hash_range=0.5, batch=1 << 20) as tr:
        a = tr.forward_for_training(pos)
        b = tr.inference(pos)
        tol = 1e-5 * (np.abs(b) + np.sqrt((b.astype(np.float64) ** 2).mean()))
        assert np.all(np.abs(a - b) <= tol)


def test_optimizer_blob_round_trip_and_continuity():
    """OracleOptimizerBlobPreservesTrainingContinuity (1e-5 rel)."""
    d, enc, net, m_out = GEOMS["small"]
    rng = np.random.default_rng(12)
    batches = [(rng.random((512, 3), dtype=np.float32),
                rng.random((512, 1), dtype=np.float32)) for _ in range(6)]
    with make_trainer(d, m_out, enc, net) as a, make_trainer(d, m_out, enc, net) as b:
        for x, y in batches[:3]:
            a.training_step(x, y)
        blob = a.export_optimizer_state()
        assert blob.version == 1 and blob.step == 3
        nh, nm = a.hash_param_count, a.mlp_param_count
        assert len(blob.payload) == 16 + 8 * (nh + nm)
        hw, mw = a.get_weights()
        b.set_initial_weights(hw, mw)
        assert b.step() == 0
        b.import_optimizer_state(blob)
        assert b.step() == 3
        for x, y in batches[3:]:
            la, lb = a.training_step(x, y), b.training_step(x, y)
            assert la == pytest.approx(lb, rel=1e-5)
        bad = type(blob)(blob.version, blob.step, blob.payload[:-1])
        with pytest.raises(Exception, match="truncated|mismatch|trailing"):
            b.import_optimizer_state(bad)
        with pytest.raises(Exception, match="version"):
            b.import_optimizer_state(type(blob)(2, blob.step, blob.payload))


def test_set_initial_weights_size_mismatch():
    d, enc, net, m_out = GEOMS["small"]
    with make_trainer(d, m_out, enc, net) as tr:
        with pytest.raises(Exception, match="count mismatch"):
            tr.set_initial_weights(np.zeros(5, np.float32), None)


# ------------------------------------------------------------ Morton sort --

def _compact_2d(code3):
    """x/y interleave of a lifted (x, y, 0) 3D Morton code (the z bits are the
    same on every point, so dropping them keeps the order)."""
    out = np.zeros_like(code3)
    for b in range(10):
        out |= ((code3 >> (3 * b)) & 1) << (2 * b)
        out |= ((code3 >> (3 * b + 1)) & 1) << (2 * b + 1)
    return out


@pytest.mark.parametrize("d,n,span", [(2, 1, 1.0), (2, 2, 1.0), (2, 1536, 1.0), (2, 1537, 1.0),
                                      (2, 2048, 1.0), (2, 2049, 1.0), (2, 3073, 1.0),
                                      (2, 4097, 1.0), (2, 70000, 1.0), (2, 1 << 18, 1.0),
                                      (2, 1 << 18, 0.5), (2, 1 << 18, 0.35), (3, 12345, 1.0),
                                      (3, 1 << 20, 1.0), (4, 9000, 1.0), (4, 300001, 1.0)])
def test_morton_sort_matches_oracle_codes_and_stable_order(oracle, d, n, span):
    """morton_sort.h: same codes as the oracle (the reference's quantisation),
    and the permutation is the stable argsort of those codes. 2D sorts each
    top-10-bit bucket in one block; positions in [0, span)^2 set the bucket
    sizes: span 1 ~n/1024 per bucket (up to 512: ranked by comparison), 0.5
    ~n/256 (513-1536: one chunk), 0.35 ~n/125 (several chunks), and the
    quarter of the points tied at one position make one bucket of n/4."""
    _say(f"morton sort d={d} n={n} span={span}")
    name = {2: "2d_f2", 3: "3d_f2", 4: "4d_f2"}[d]
    _, enc, net, m_out = GEOMS[name]
    rng = np.random.default_rng(n)
    pos = rng.random((n, d), dtype=np.float32) * np.float32(span)
    pos[: n // 4] = pos[0]  # ties
    with make_trainer(d, m_out, enc, net, batch=1 << 20) as tr:
        codes, perm = tr.debug_morton_sort(pos)
    want = oracle.morton_codes(pos, d)
    if d == 2:
        # the lifted z = 0 quantises to 512 on every point: a constant bit 29
        assert np.all(((want >> 2) & 0o1111111111) == (1 << 27))
        want = _compact_2d(want)
    assert np.array_equal(codes, want)
    assert np.array_equal(perm, np.argsort(want, kind="stable").astype(np.uint32))


# ------------------------------------------------- evaluate_with_gradient --

@pytest.mark.parametrize("name", list(GEOMS))
def test_evaluate_with_gradient_matches_oracle(oracle, name):
    """FieldEvaluator::evaluate_with_gradient: outputs and the position
    Jacobian [N][M][D] against the oracle's restatement of the reference's
    analytic gradient kernel (fp32, same tolerance as outputs)."""
    _say(f"evaluate_with_gradient {name}")
    d, enc, net, m_out = GEOMS[name]
    rng = np.random.default_rng(31)
    with make_trainer(d, m_out, enc, net, hash_range=0.5, precision="fp16") as tr:
        hw, mw = tr.get_weights()
        pos = rng.random((777, d), dtype=np.float32)
        out, jac = tr.evaluate_with_gradient(pos)
        oout, ojac = oracle.evaluate_with_gradient(omodel(oracle, tr), hw, mw, pos)
        assert jac.shape == (777, m_out, d)
        for got, ref in ((out, oout), (jac, ojac)):
            tol = 1e-5 * (np.abs(ref) + np.sqrt((ref.astype(np.float64) ** 2).mean()))
            assert np.all(np.abs(got - ref) <= tol), float(np.abs(got - ref).max())
        e_out, e_jac = tr.evaluate_with_gradient(np.zeros((0, d), np.float32))
        assert e_out.shape == (0, m_out) and e_jac.shape == (0, m_out, d)


# ------------------------------------------------------- hidden width 128 --

WIDE_GEOMS = {
    # BASELINE config 5 shape (4D, 16x2, base 8, scale 1.4, 32 -> 128 x4 -> 4), smaller table
    "4d_w128": (4, dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=16,
                        base_resolution=8.0, per_level_scale=1.4),
                dict(n_neurons=128, n_hidden_layers=4), 4),
    "3d_w128": (3, dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=14,
                        base_resolution=16.0, per_level_scale=1.5),
                dict(n_neurons=128, n_hidden_layers=2), 2),
}


@pytest.mark.parametrize("name", list(WIDE_GEOMS))
def test_wide_inference_and_position_gradient(oracle, name):
    _say(f"wide inference {name}")
    d, enc, net, m_out = WIDE_GEOMS[name]
    rng = np.random.default_rng(41)
    with make_trainer(d, m_out, enc, net, hash_range=0.5, precision="fp16") as tr:
        hw, mw = tr.get_weights()
        m = omodel(oracle, tr)
        pos = rng.random((3001, d), dtype=np.float32)
        out = tr.inference(pos)
        ref = oracle.forward(m, hw, mw, pos)
        tol = 1e-5 * (np.abs(ref) + np.sqrt((ref.astype(np.float64) ** 2).mean()))
        assert np.all(np.abs(out - ref) <= tol), float(np.abs(out - ref).max())
        out2, jac = tr.evaluate_with_gradient(pos[:500])
        oout, ojac = oracle.evaluate_with_gradient(m, hw, mw, pos[:500])
        for got, want in ((out2, oout), (jac, ojac)):
            tol = 1e-5 * (np.abs(want) + np.sqrt((want.astype(np.float64) ** 2).mean()))
            assert np.all(np.abs(got - want) <= tol), float(np.abs(got - want).max())
        a = tr.forward_for_training(pos)
        assert rel_tensor(a, ref) <= 2e-3


def away_from_relu_kinks(oracle, tr, hw, mw, pos, margin=1e-5):
    """Rows of `pos` whose hidden pre-activations all lie at least `margin`
    from zero, judged by a float64 forward over the oracle's encoding.

    A pre-activation within fp32 rounding of zero has a ReLU mask that the
    summation order decides; one flipped mask moves a weight-gradient element
    by that point's whole contribution, which says nothing about the kernel.
    With 4 x 128 hidden units about one point in 30 sits within 1e-5 of a
    kink; the gradient comparisons below run on the rest."""
    c = tr.config
    m = omodel(oracle, tr)
    IN = c["encoding"]["n_levels"] * c["encoding"]["n_features_per_level"]
    H, NHL = c["network"]["n_neurons"], c["network"]["n_hidden_layers"]
    a = oracle.encode(m, hw, pos).astype(np.float64)
    off, keep, kin = 0, np.ones(len(pos), bool), IN
    for _ in range(NHL):
        W = mw[off:off + kin * H].astype(np.float64).reshape(kin, H)
        b = mw[off + kin * H:off + kin * H + H].astype(np.float64)
        off += kin * H + H
        z = a @ W + b
        keep &= (np.abs(z) >= margin).all(axis=1)
        a, kin = np.maximum(z, 0.0), H
    return pos[keep]


@pytest.mark.parametrize("name", list(WIDE_GEOMS))
def test_wide_backward_fp16_matches_oracle(oracle, name):
    _say(f"wide backward {name}")
    d, enc, net, m_out = WIDE_GEOMS[name]
    rng = np.random.default_rng(43)
    with make_trainer(d, m_out, enc, net, precision="fp16", hash_range=0.5,
                      batch=1 << 20) as tr:
        hw, mw = tr.get_weights()
        pos = away_from_relu_kinks(oracle, tr, hw, mw, rng.random((4133, d), dtype=np.float32))
        assert len(pos) > 3500
        g = rng.normal(0, 1.0, (len(pos), m_out)).astype(np.float32)
        tr.zero_gradients()
        tr.backward_accumulate(pos, g)
        gh, gm = tr.debug_gradients()
        mask = tr.debug_active_mask()
        ogh, ogm, omask, _, _ = oracle.forward_backward(omodel(oracle, tr), hw, mw, pos, d_out=g)
        assert np.array_equal(mask, omask)
        assert rel_tensor(gm, ogm) <= 2e-3
        assert rel_tensor(gh, ogh) <= 2e-3


def test_wide_training_loss_tracks_oracle(oracle):
    _say("wide training")
    d, enc, net, m_out = WIDE_GEOMS["4d_w128"]
    rng = np.random.default_rng(47)
    n, steps = 4096, 8
    with make_trainer(d, m_out, enc, net, loss="L2", precision="fp16", batch=n) as tr:
        hw, mw = tr.get_weights()
        m = omodel(oracle, tr)
        a = oracle.adam(1e-2, 1e-2)
        params = np.concatenate([hw, mw])
        m1, m2 = np.zeros_like(params), np.zeros_like(params)
        for step in range(steps):
            pos = rng.random((n, d), dtype=np.float32)
            tgt = np.sin(3 * pos[:, :m_out] + step).astype(np.float32)
            lg = tr.training_step(pos, tgt)
            lo = oracle.training_step(m, a, step, params, m1, m2, pos, tgt)
            assert lg == pytest.approx(lo, rel=0.01), (step, lg, lo)


# ------------------------------------------------------ fused step image --

@pytest.mark.parametrize("name,precision", [("2d_f2", "fp16"), ("3d_f4", "fp16"), ("3d_f2", "fp16"),
                                            ("2d_f2", "fp32"), ("small", "fp32"),
                                            ("4d_w128", "fp16")])
def test_fused_step_keeps_the_training_image_current(name, precision):
    """The fused end of a training step writes every updated MLP weight into
    the training plan's packed LDS image (forward hi/lo and backward
    fragments, biases): after several steps it equals a repack from the
    parameters, byte for byte."""
    _say(f"fused step image {name} {precision}")
    d, enc, net, m_out = GEOMS[name] if name in GEOMS else WIDE_GEOMS[name]
    rng = np.random.default_rng(5)
    with make_trainer(d, m_out, enc, net, precision=precision, hash_range=0.1) as tr:
        for _ in range(3):
            pos = rng.random((5000, d), dtype=np.float32)
            tgt = rng.random((5000, m_out), dtype=np.float32)
            tr.training_step(pos, tgt)
        cur, rep = tr.debug_train_image()
    assert cur.size > 0
    assert np.array_equal(cur, rep)


def test_step_profiling_samples_one_step_in_k():
    """TrainingStepProfile with an interval: one training step in k carries
    the phase events (the first after enabling, then every k-th); 1 is every
    step, 0 off; a negative interval is an argument error."""
    _say("step profiling interval")
    d, enc, net, m_out = GEOMS["small"]
    rng = np.random.default_rng(9)
    pos = rng.random((3000, d), dtype=np.float32)
    tgt = rng.random((3000, m_out), dtype=np.float32)
    with make_trainer(d, m_out, enc, net) as tr:
        for every, steps, want in ((3, 7, 3), (1, 4, 4), (5, 5, 1)):
            tr.set_training_step_profiling(True, every)
            for _ in range(steps):
                tr.training_step(pos, tgt)
            prof = tr.training_step_profile()
            assert prof["steps"] == want, (every, prof)
            assert prof["gpu_total_us"] > 0.0
        tr.set_training_step_profiling(False)
        tr.training_step(pos, tgt)
        assert tr.training_step_profile()["steps"] == 0
        with pytest.raises(ValueError):
            tr.set_training_step_profiling(True, 0)
