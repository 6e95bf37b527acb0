"""GPU parity, second part: the kernels the training step itself runs at every
BASELINE geometry, every loss kind, every Adam variant, the state after one
fused step, and loss-after-N at the BASELINE batch sizes. Marked gpu; every
comparison is against the CPU oracle on identical seeded inputs.

Tolerances (north_star): hash indices / corner weights / fp32 encodings
bit-exact; fp32 outputs and gradients 1e-5 relative; fp16 2e-3; loss after N
Adam steps within 1%. Adam fed with the GPU's own gradients is compared bit
for bit (same fp32 operations in the same order on both sides).
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from test_gpu_parity import (GEOMS, away_from_relu_kinks, make_trainer, omodel,
                             rel_tensor)

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


# The BASELINE.json configs' hash-grid and MLP geometries (tables at full
# size): C1/C2 image fit, C3 NeRF density, C4 SDF, C5 4D wide field.
BASELINE = {
    "c2": (2, dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=15, base_resolution=16.0,
                   per_level_scale=1.5), dict(n_neurons=64, n_hidden_layers=2), 3, "RelativeL2"),
    "c3": (3, dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=19, base_resolution=16.0,
                   per_level_scale=1.381913), dict(n_neurons=64, n_hidden_layers=1), 16, "L2"),
    "c4": (3, dict(n_levels=16, n_features_per_level=4, log2_hashmap_size=21, base_resolution=16.0,
                   per_level_scale=1.5), dict(n_neurons=64, n_hidden_layers=3), 1, "L1"),
    "c5": (4, dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=22, base_resolution=8.0,
                   per_level_scale=1.4), dict(n_neurons=128, n_hidden_layers=4), 4, "L2"),
}


def parse_optimizer_blob(payload: bytes, nh: int, nm: int):
    """OptimizerStateBlob v1 payload (default_trainer.cpp:1656-1661,83-88):
    four [u32 LE byte_len][fp32 ...] sections m_hash, v_hash, m_mlp, v_mlp."""
    out, off = [], 0
    for count in (nh, nh, nm, nm):
        ln = int.from_bytes(payload[off:off + 4], "little")
        off += 4
        assert ln == 4 * count, (ln, count)
        out.append(np.frombuffer(payload[off:off + ln], np.float32).copy())
        off += ln
    assert off == len(payload)
    return out


def _edge_positions(rng, n, d):
    pos = rng.random((n, d), dtype=np.float32)
    pos[:3] = 0.0
    pos[3:6] = np.float32(0.999999)
    pos[6:8] = np.float32(0.5)
    pos[8: n // 5] = pos[8]  # ties for the sort (a fifth of the batch on one code)
    return pos


# ------------------------------------------------------ production encode --

@pytest.mark.parametrize("name", ["c2", "c3", "c4", "c5", "3d_f2", "3d_f4", "3d_f1", "4d_f2"])
@pytest.mark.parametrize("sorted_", [True, False])
def test_training_encode_kernels_bit_exact(oracle, name, sorted_):
    """The feature tiles the training step's encode kernels write
    (encode_features_kernel point-major, encode_level_kernel for table slices
    over 2 MB per level: C3, C4, C5), read through the step's Morton
    permutation: every feature bit-identical to the oracle's encode of the
    same point, the positions handed to the scatter equal, padding zero."""
    if name in BASELINE:
        d, enc, net, m_out, _ = BASELINE[name]
    else:
        d, enc, net, m_out = GEOMS[name]
    _say(f"training encode {name} sorted={sorted_}")
    rng = np.random.default_rng(11)
    prec = "fp16" if net["n_neurons"] > 64 else "fp32"
    with make_trainer(d, m_out, enc, net, hash_range=0.5, precision=prec, batch=1 << 16) as tr:
        hw, _ = tr.get_weights()
        for n in (1, 31, 4133):
            pos = _edge_positions(rng, n, d) if n > 10 else rng.random((n, d), dtype=np.float32)
            feats, perm, spos, pad = tr.debug_encode_tiles(pos, sorted=sorted_)
            assert pad == 0
            assert np.array_equal(np.sort(perm), np.arange(n, dtype=np.uint32))
            if not sorted_:
                assert np.array_equal(perm, np.arange(n, dtype=np.uint32))
            assert np.array_equal(spos, pos[perm])
            want = oracle.encode(omodel(oracle, tr), hw, pos[perm])
            assert np.array_equal(feats.view(np.uint32), want.view(np.uint32)), n


def _identity_mlp(IN, H, NHL, M, first):
    """MLP weights (reference layout) whose forward copies input features
    first .. first+M-1 to the outputs: W0 = [I 0], hidden W = I, WO selects
    the units, all biases 0."""
    parts = []
    W0 = np.zeros((IN, H), np.float32)
    W0[np.arange(IN), np.arange(IN)] = 1.0
    parts += [W0.ravel(), np.zeros(H, np.float32)]
    for _ in range(NHL - 1):
        parts += [np.eye(H, dtype=np.float32).ravel(), np.zeros(H, np.float32)]
    WO = np.zeros((H, M), np.float32)
    for m in range(M):
        if first + m < IN:
            WO[first + m, m] = 1.0
    parts += [WO.ravel(), np.zeros(M, np.float32)]
    return np.concatenate(parts)


@pytest.mark.parametrize("name", ["2d_f2", "3d_f2", "3d_f4"])
@pytest.mark.parametrize("family", ["auto", "Tiled"])
def test_inference_inline_encode_bit_exact(oracle, name, family):
    """The encode of the fp32 inference path (inline in field_forward_kernel,
    specialised per geometry under FullyFused, generic under Tiled; for F <= 2
    tables with level slices over 2 MB, 3d_f2 here, encode_level_kernel's X
    tiles read by field_forward_x_kernel), read
    through an MLP that copies features to outputs: with a positive table
    the features are >= 0, ReLU passes them, and each output is
    1.0 * feature + exact zeros, so every output equals the oracle's feature
    bit for bit."""
    d, enc, _, _ = GEOMS[name]
    IN = enc["n_levels"] * enc["n_features_per_level"]
    H, NHL, M = 64, 2, 16
    _say(f"inline encode {name} {family}")
    rng = np.random.default_rng(12)
    with make_trainer(d, M, enc, dict(n_neurons=H, n_hidden_layers=NHL), hash_range=0.5,
                      family=family) as tr:
        hw, _ = tr.get_weights()
        hw = np.abs(hw) + np.float32(1e-3)
        pos = _edge_positions(rng, 3001, d)
        want = oracle.encode(omodel(oracle, tr), hw, pos)
        for first in range(0, IN, M):
            tr.set_initial_weights(hw, _identity_mlp(IN, H, NHL, M, first))
            out = tr.inference(pos)
            k = min(M, IN - first)
            assert np.array_equal(out[:, :k].view(np.uint32),
                                  want[:, first:first + k].view(np.uint32)), first


# ------------------------------------------------------------ loss kinds --

@pytest.mark.parametrize("name", ["2d_f2", "3d_f2"])
@pytest.mark.parametrize("precision", ["fp32", "fp16"])
@pytest.mark.parametrize("loss,delta", [("L1", None), ("Huber", 0.05), ("Cosine", None)])
def test_loss_kinds_track_oracle(oracle, name, precision, loss, delta):
    """L1, Huber (delta != 1) and Cosine (M >= 2) through the fused training
    step: loss after each of N Adam steps within 1% of the oracle
    (emitLoss, mlp_kernel_emitter.cpp:562-670; detail/{l1,huber,cosine}_loss.h)."""
    _say(f"loss {loss} {name} {precision}")
    d, enc, net, m_out = GEOMS[name]
    rng = np.random.default_rng(19)
    n, steps = 4096, 8
    with make_trainer(d, m_out, enc, net, loss=loss, huber_delta=delta, precision=precision,
                      batch=n) as tr:
        hw, mw = tr.get_weights()
        m = omodel(oracle, tr)
        a = oracle.adam(1e-2, 1e-2)
        params = np.concatenate([hw, mw])
        m1, m2 = np.zeros_like(params), np.zeros_like(params)
        for step in range(steps):
            pos = rng.random((n, d), dtype=np.float32)
            tgt = np.sin(4 * pos[:, :1] + np.arange(m_out, dtype=np.float32)[None] * 0.7 +
                         pos[:, -1:]).astype(np.float32) * 0.5
            lg = tr.training_step(pos, tgt)
            lo = oracle.training_step(m, a, step, params, m1, m2, pos, tgt)
            assert lg == pytest.approx(lo, rel=0.01), (step, lg, lo)


# --------------------------------------------- state after one fused step --

def _int_tol_compare(gpu, want, scale, what):
    """Hash-part comparison: the int32 gradients agree except where an fp32
    ulp of d_feat flips a truncation (<= 16 units), so the moments agree
    exactly on >= 99% of entries and within that bound elsewhere."""
    diff = np.abs(gpu.astype(np.float64) - want.astype(np.float64))
    assert (diff == 0).mean() > 0.99, (what, (diff == 0).mean())
    assert diff.max() <= scale, (what, diff.max(), scale)


@pytest.mark.parametrize("name,loss,delta", [("2d_f2", "L2", None), ("2d_f2", "RelativeL2", None),
                                             ("2d_f2", "Huber", 0.05), ("3d_f2", "L1", None),
                                             ("3d_f2", "Cosine", None), ("3d_f4", "L2", None),
                                             ("4d_f2", "L2", None)])
@pytest.mark.parametrize("hash_adam", ["lazy", "dense"])
def test_one_fused_step_state_matches_oracle(oracle, name, loss, delta, hash_adam):
    """After one fp32 fused training step: MLP params, m and v within fp32
    tolerance of the oracle's step; hash-table m and v exact on >= 99% of
    entries (the int32 gradients agree up to truncation flips); the set of
    entries Adam touched (m != 0) equal; the optimizer blob's sections parse
    in the reference order m_hash, v_hash, m_mlp, v_mlp."""
    _say(f"one step {name} {loss} {hash_adam}")
    d, enc, net, m_out = GEOMS[name]
    rng = np.random.default_rng(23)
    n = 3000
    beta1, beta2, lr = 0.9, 0.99, 1e-2
    with make_trainer(d, m_out, enc, net, loss=loss, huber_delta=delta, hash_adam=hash_adam,
                      hash_range=0.5, batch=n) as tr:
        hw, mw = tr.get_weights()
        m = omodel(oracle, tr)
        params = np.concatenate([hw, mw])
        m1, m2 = np.zeros_like(params), np.zeros_like(params)
        pos = rng.random((n, d), dtype=np.float32)
        tgt = rng.random((n, m_out), dtype=np.float32)
        lg = tr.training_step(pos, tgt)
        lo = oracle.training_step(m, oracle.adam(lr, lr, beta1, beta2), 0, params, m1, m2, pos,
                                  tgt, dense_hash=hash_adam == "dense")
        assert lg == pytest.approx(lo, rel=1e-5)
        nh, nm = tr.hash_param_count, tr.mlp_param_count
        blob = tr.export_optimizer_state()
        mh, vh, mm, vm = parse_optimizer_blob(blob.payload, nh, nm)
        gh2, gm2 = tr.get_weights()
        # MLP: fp32 gradients within 1e-5 (v carries g^2: 2e-5)
        assert rel_tensor(mm, m1[nh:]) <= 1e-5
        assert rel_tensor(vm, m2[nh:]) <= 2e-5
        dp = np.abs(gm2.astype(np.float64) - params[nh:])
        assert (dp <= 1e-5 * np.abs(params[nh:]) + 1e-7).mean() > 0.999
        assert dp.max() <= 2.05 * lr
        # hash: m = (1 - beta1) g, v = (1 - beta2) g^2 with g = int / 65536
        g_ulp = 16.0 / 65536.0
        gmax = float(np.abs(m1[:nh]).max()) / (1 - beta1)
        _int_tol_compare(mh, m1[:nh], (1 - beta1) * g_ulp * 1.01, "m_hash")
        _int_tol_compare(vh, m2[:nh], (1 - beta2) * (2 * gmax + g_ulp) * g_ulp * 1.01, "v_hash")
        touched_gpu, touched_orc = mh != 0, m1[:nh] != 0
        assert (touched_gpu == touched_orc).mean() > 0.999
        # entries whose moments agree were updated by the same fp32 operations
        same = (mh == m1[:nh]) & (vh == m2[:nh])
        assert np.array_equal(gh2[same].view(np.uint32),
                              params[:nh][same].astype(np.float32).view(np.uint32))
        if hash_adam == "lazy":
            # untouched entries keep their weights bit for bit
            assert np.array_equal(gh2[~touched_orc & ~touched_gpu], hw[~touched_orc & ~touched_gpu])


# ------------------------------------------- split-path Adam, every variant --

ADAM_VARIANTS = {
    "plain": {},
    "clip": {"grad_clip": 2e-4},
    "l2": {"l2_reg": 1e-3},
    "l1": {"l1_reg": 1e-4},        # forces the dense hash update (default_trainer.cpp:1868-1876)
    "wd": {"weight_decay": 1e-2},  # AdamW: decay first, no L1/L2
    "all": {"grad_clip": 2e-4, "l1_reg": 1e-4, "l2_reg": 1e-3},
}


@pytest.mark.parametrize("name", ["2d_f2", "3d_f4", "3d_f1"])
@pytest.mark.parametrize("hash_adam", ["lazy", "dense"])
@pytest.mark.parametrize("variant", list(ADAM_VARIANTS))
def test_split_adam_step_bit_exact(oracle, name, hash_adam, variant):
    """adam_step (split path, adam_kernel) fed with the GPU's own accumulated
    gradients and visit mask: params, m and v bit-identical to the oracle's
    Adam (adam_kernel_msl.h:37-203 -- dense unified kernel, lazy sparse hash +
    dense MLP kernels; clip, L1 hash / L2 MLP regularisation, AdamW decay;
    bias corrections in fp32 on the host, adam_params.h:33-52). Two Adam
    steps, so the moments carry history into the second."""
    _say(f"split adam {name} {hash_adam} {variant}")
    d, enc, net, m_out = GEOMS[name]
    opts = ADAM_VARIANTS[variant]
    from tiny_metal_nn import Trainer
    cfg = {"encoding": dict(otype="HashGrid", **enc), "network": dict(otype="FullyFusedMLP", **net),
           "loss": {"otype": "L2"},
           "optimizer": {"otype": "Adam", "learning_rate": 1e-2,
                         "l1_reg": opts.get("l1_reg", 0.0), "l2_reg": opts.get("l2_reg", 0.0)},
           "weight_init": {"seed": 7, "hash_grid_range": 0.5}, "batch_size": 1 << 16,
           "mi355x": {"precision": "fp32", "hash_adam": hash_adam,
                      "grad_clip": opts.get("grad_clip", 0.0),
                      "weight_decay": opts.get("weight_decay", 0.0)}}
    a = oracle.adam(1e-2, 1e-2, 0.9, 0.99, 1e-15, opts.get("l1_reg", 0.0), opts.get("l2_reg", 0.0),
                    opts.get("grad_clip", 0.0), opts.get("weight_decay", 0.0))
    rng = np.random.default_rng(29)
    with Trainer.from_config(cfg, n_input=d, n_output=m_out) as tr:
        m = omodel(oracle, tr)
        nh, nm = tr.hash_param_count, tr.mlp_param_count
        hw, mw = tr.get_weights()
        params = np.concatenate([hw, mw])
        m1, m2 = np.zeros_like(params), np.zeros_like(params)
        for step in range(2):
            pos = rng.random((2500, d), dtype=np.float32)
            g = rng.normal(0, 1.0, (2500, m_out)).astype(np.float32)
            tr.zero_gradients()
            tr.backward_accumulate(pos, g)
            gh, gm = tr.debug_gradients()
            mask = tr.debug_active_mask()
            tr.adam_step()
            assert tr.step() == step + 1
            dense = hash_adam == "dense" or opts.get("l1_reg", 0.0) != 0.0
            oracle.adam_step(m, a, step, params, m1, m2, gh, gm, None if dense else mask)
            ghw, gmw = tr.get_weights()
            mh, vh, mm, vm = parse_optimizer_blob(tr.export_optimizer_state().payload, nh, nm)
            for got, want, what in ((ghw, params[:nh], "hash w"), (gmw, params[nh:], "mlp w"),
                                    (mh, m1[:nh], "m hash"), (vh, m2[:nh], "v hash"),
                                    (mm, m1[nh:], "m mlp"), (vm, m2[nh:], "v mlp")):
                bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
                assert bad.size == 0, (what, step, bad[:5], got[bad[:5]], want[bad[:5]])
            # the split path keeps the gradients until zero_gradients
            gh_after, gm_after = tr.debug_gradients()
            assert np.array_equal(gh_after, gh) and np.array_equal(gm_after, gm)


# --------------------------------------------------- C4 at its real shape --

def test_c4_backward_fp16_matches_oracle(oracle):
    """C4: 3D, 16 levels x 4 features, T = 2^21 (32 MB
    per level: the encode and the scatter run level-major,
    encode_level_kernel<3,4> / hash_scatter_level_kernel<3,4>), MLP
    64 -> 64^3 -> 1 in fp16: gradients within 2e-3 of the oracle, visited
    set exact."""
    _say("c4 backward fp16")
    d, enc, net, m_out, _ = BASELINE["c4"]
    rng = np.random.default_rng(37)
    with make_trainer(d, m_out, enc, net, precision="fp16", hash_range=0.5, batch=1 << 16) as tr:
        hw, mw = tr.get_weights()
        pos = away_from_relu_kinks(oracle, tr, hw, mw, rng.random((8192, d), dtype=np.float32))
        assert len(pos) > 0.95 * 8192
        g = rng.normal(0, 1.0, (len(pos), m_out)).astype(np.float32)
        tr.zero_gradients()
        tr.backward_accumulate(pos, g)
        gh, gm = tr.debug_gradients()
        mask = tr.debug_active_mask()
        ogh, ogm, omask, _, _ = oracle.forward_backward(omodel(oracle, tr), hw, mw, pos, d_out=g)
        assert np.array_equal(mask, omask)
        assert rel_tensor(gm, ogm) <= 2e-3
        assert rel_tensor(gh, ogh) <= 2e-3


@pytest.mark.parametrize("name", ["c2", "c3", "c4"])
@pytest.mark.parametrize("mix", ["tiny", "mixed"])
@pytest.mark.parametrize("precision", ["fp32", "fp16"])
def test_scatter_vanishing_levels_match_oracle(oracle, name, mix, precision):
    """The hash-grid backward at the gradient sizes of a converging batch
    (|d_out| ~ 1/N): a wave whose contributions at a level all truncate to 0
    only marks that level's corners. "tiny": every point's gradient vanishes,
    so the int32 table stays all zero while the visited set is the oracle's;
    "mixed": 2% of the points carry large gradients, so lanes of both kinds
    run in one launch. fp32 runs hash_scatter_kernel (point-major at C2/C3,
    level-major at C4's T = 2^21); fp16 at C2/C3 runs the backward fused into
    the MLP kernel's tiles (tile_scatter.hpp), at C4 the level-major kernel."""
    _say(f"scatter vanishing levels {name} {mix} {precision}")
    d, enc, net, m_out, _ = BASELINE[name]
    rng = np.random.default_rng(41)
    with make_trainer(d, m_out, enc, net, precision=precision, hash_range=0.5,
                      batch=1 << 16) as tr:
        hw, mw = tr.get_weights()
        pos = rng.random((8192, d), dtype=np.float32)
        if precision == "fp16":
            pos = away_from_relu_kinks(oracle, tr, hw, mw, pos)
        g = rng.normal(0, 1.0, (len(pos), m_out)).astype(np.float32)
        scale = np.full((len(pos), 1), 1e-9, np.float32)
        if mix == "mixed":
            scale[rng.random(len(pos)) < 0.02] = 1.0
        g = (g * scale).astype(np.float32)
        tr.zero_gradients()
        tr.backward_accumulate(pos, g)
        gh, gm = tr.debug_gradients()
        mask = tr.debug_active_mask()
        ogh, ogm, omask, _, _ = oracle.forward_backward(omodel(oracle, tr), hw, mw, pos, d_out=g)
        assert np.array_equal(mask, omask)
        # fp16 "tiny": d_out ~ 1e-9 times the loss scale (~N) is below fp16's
        # normal range, so the fp16 MLP gradients are not compared there; the
        # table and the visited set are what this case checks
        if precision == "fp32":
            assert rel_tensor(gm, ogm) <= 1e-5
        elif mix == "mixed":
            assert rel_tensor(gm, ogm) <= 2e-3
        if mix == "tiny":
            assert not ogh.any() and not gh.any()
        elif precision == "fp32":
            assert ogh.any()
            diff = np.abs(gh.astype(np.int64) - ogh.astype(np.int64))
            assert (diff == 0).mean() > 0.99 and diff.max() <= 16, int(diff.max())
        else:
            assert ogh.any()
            assert rel_tensor(gh, ogh) <= 2e-3


def _sdf_batch(rng, n, centers, radii):
    """C4 inputs: half within +-0.01 of a union of spheres, half uniform;
    target = the analytic SDF of the union."""
    k = n // 2
    idx = rng.integers(0, len(centers), k)
    v = rng.normal(size=(k, 3))
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    shell = centers[idx] + v * (radii[idx, None] + rng.uniform(-0.01, 0.01, (k, 1)))
    pos = np.concatenate([shell, rng.random((n - k, 3))]).astype(np.float32)
    pos = np.clip(pos, 0.0, np.float32(0.999999))
    dist = np.linalg.norm(pos[:, None, :] - centers[None], axis=2) - radii[None]
    return pos, dist.min(axis=1, keepdims=True).astype(np.float32)


@pytest.mark.parametrize("precision", ["fp16", "fp32"])
def test_c4_training_loss_tracks_oracle(oracle, precision):
    """C4's training step (L1 against the analytic SDF of 8 spheres, fused
    Adam): loss after each of N steps within 1% of the oracle."""
    _say(f"c4 training {precision}")
    d, enc, net, m_out, loss = BASELINE["c4"]
    rng = np.random.default_rng(41)
    centers = rng.uniform(0.25, 0.75, (8, 3))
    radii = rng.uniform(0.05, 0.25, 8)
    n, steps = 16384, 6
    with make_trainer(d, m_out, enc, net, loss=loss, precision=precision, batch=n) as tr:
        hw, mw = tr.get_weights()
        m = omodel(oracle, tr)
        a = oracle.adam(1e-2, 1e-2)
        params = np.concatenate([hw, mw])
        del hw
        m1, m2 = np.zeros_like(params), np.zeros_like(params)
        for step in range(steps):
            pos, tgt = _sdf_batch(rng, n, centers, radii)
            lg = tr.training_step(pos, tgt)
            lo = oracle.training_step(m, a, step, params, m1, m2, pos, tgt)
            assert lg == pytest.approx(lo, rel=0.01), (step, lg, lo)


# ------------------------------------- loss after N at the BASELINE batch --

def _image(rng, size=256):
    """Seeded procedural RGB image: 8 random sinusoids + a checkerboard, in [0, 1]."""
    yy, xx = np.mgrid[0:size, 0:size].astype(np.float32) / size
    img = np.zeros((size, size, 3), np.float32)
    for _ in range(8):
        f = rng.uniform(1, 12, 2)
        ph = rng.uniform(0, 2 * np.pi)
        img += np.sin(2 * np.pi * (f[0] * xx + f[1] * yy) + ph)[..., None] * rng.uniform(0, 1, 3)
    img += ((np.floor(xx * size / 8) + np.floor(yy * size / 8)) % 2)[..., None]
    img -= img.min()
    return img / img.max()


@pytest.mark.parametrize("batch", [1024, 65536, 1 << 18])
def test_c2_loss_after_n_at_baseline_batches(oracle, batch):
    """C2 (fp16, RelativeL2, lr 1e-2, beta 0.9 / 0.99, eps 1e-15) at the batch
    sizes the reference caps at and the BASELINE batch: loss after each of N
    steps within 1% of the oracle."""
    _say(f"c2 loss after N batch={batch}")
    d, enc, net, m_out, loss = BASELINE["c2"]
    rng = np.random.default_rng(batch)
    img = _image(rng)
    steps = 5 if batch >= 1 << 18 else 8
    with make_trainer(d, m_out, enc, net, loss=loss, precision="fp16", batch=batch) as tr:
        hw, mw = tr.get_weights()
        m = omodel(oracle, tr)
        a = oracle.adam(1e-2, 1e-2)
        params = np.concatenate([hw, mw])
        m1, m2 = np.zeros_like(params), np.zeros_like(params)
        for step in range(steps):
            pos = rng.random((batch, 2), dtype=np.float32)
            ij = np.minimum((pos * img.shape[0]).astype(np.int64), img.shape[0] - 1)
            tgt = np.ascontiguousarray(img[ij[:, 1], ij[:, 0]])
            lg = tr.training_step(pos, tgt)
            lo = oracle.training_step(m, a, step, params, m1, m2, pos, tgt)
            assert lg == pytest.approx(lo, rel=0.01), (step, lg, lo)


# ------------------------------------------------------ runtime authority --

def test_runtime_authority_views_and_batch_plan():
    """RuntimeAuthority::buffer(role) device ranges hold what the
    download entry points return; ParameterLayout / TrainerBatchPlan /
    RuntimeStoragePolicy describe the trainer (runtime_authority.h:33-119)."""
    _say("runtime authority")
    d, enc, net, m_out = GEOMS["2d_f2"]
    rng = np.random.default_rng(3)
    with make_trainer(d, m_out, enc, net, precision="fp16", batch=5000) as tr:
        pos = rng.random((5000, 2), dtype=np.float32)
        tgt = rng.random((5000, 3), dtype=np.float32)
        tr.training_step(pos, tgt)
        tr.synchronize()
        nh, nm = tr.hash_param_count, tr.mlp_param_count
        hw, mw = tr.get_weights()
        mh, vh, mm, vm = parse_optimizer_blob(tr.export_optimizer_state().payload, nh, nm)

        def read(view, dtype):
            assert view["valid"] and view["device_ptr"] == view["gpu_buffer"] + view["offset"]
            host = np.empty(view["bytes"] // np.dtype(dtype).itemsize, dtype)
            _hip_to_host(host, view["device_ptr"], view["bytes"])
            return host

        assert np.array_equal(read(tr.runtime_buffer("HashWeights"), np.float32), hw)
        assert np.array_equal(read(tr.runtime_buffer("MlpWeights"), np.float32), mw)
        fused = read(tr.runtime_buffer("FusedWeights"), np.float32)
        assert np.array_equal(fused, np.concatenate([hw, mw]))
        assert np.array_equal(read(tr.runtime_buffer("FusedFirstMoment"), np.float32),
                              np.concatenate([mh, mm]))
        assert np.array_equal(read(tr.runtime_buffer("FusedSecondMoment"), np.float32),
                              np.concatenate([vh, vm]))
        gview = tr.runtime_buffer("GradHash")
        assert gview["element_kind"] == "i32_packed_pair" and gview["bytes"] == 4 * nh
        assert not np.any(read(gview, np.int32))  # a fused step consumes its gradients
        for role in ("TrainParams", "AdamParams"):
            v = tr.runtime_buffer(role)
            assert not v["valid"] and v["bytes"] == 0
        cw = tr.runtime_buffer("ConfigWeights")
        cur, _ = tr.debug_train_image()
        assert cw["bytes"] == cur.size and cw["element_kind"] == "opaque"
        lay = tr.parameter_layout()
        assert lay["hash_grid_float_count"] == nh and lay["mlp_weight_float_count"] == nm
        assert lay["target_dims"] == 3 and lay["fused_adam"] == 1
        bp = tr.batch_plan()
        assert bp["max_batch_size"] == 5000 and bp["input_dims"] == 2 and bp["target_dims"] == 3
        assert bp["positions_bytes_per_lane"] == 5000 * 2 * 4
        assert bp["targets_bytes_per_lane"] == 5000 * 3 * 4
        ins = tr.inspect_runtime()
        assert bp["threadgroup_size"] == 64 * ins["waves_per_block_train"]
        assert bp["points_per_threadgroup"] == 32 * ins["waves_per_block_train"]
        sp = tr.storage_policy()
        assert sp["parameter_weights"] == "GpuOnly" and sp["requires_staging_uploads"]
        with pytest.raises(ValueError):
            tr.runtime_buffer("Nope")


def _hip_to_host(host: np.ndarray, src: int, nbytes: int) -> None:
    """Synchronous device-to-host hipMemcpy (kind 2) through the HIP runtime
    the library is linked against."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.restype = ctypes.c_int
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert host.nbytes == nbytes
    rc = hip.hipMemcpy(host.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(src), nbytes, 2)
    assert rc == 0, rc


@pytest.mark.parametrize("name", ["2d_f2", "3d_bigT", "4d_bigT"])
def test_hash_rate_reference_kernels_leave_the_trainer_alone(name):
    """tmnn_debug_hash_rates (the gather / atomic / flag reference kernels)
    returns positive per-launch times and touches no trainer state, with the
    point-major kernels (2d_f2) and the level-major ones (16 MB level slices
    of the bigT tables)."""
    torch = pytest.importorskip("torch")
    _say(f"hash rates {name}")
    d, enc, net, m_out = GEOMS[name]
    with make_trainer(d, m_out, enc, net, precision="fp16", batch=1 << 16) as tr:
        x = torch.rand(1 << 16, d, device="cuda:0")
        y = torch.rand(1 << 16, m_out, device="cuda:0")
        torch.cuda.synchronize()
        tr.training_step_device(x.data_ptr(), y.data_ptr(), 1 << 16)
        tr.synchronize()
        hw, mw = tr.get_weights()
        gh, gm = tr.debug_gradients()
        mask = tr.debug_active_mask()
        r = tr.debug_hash_rates(x.data_ptr(), 1 << 16, sorted=True, reps=3)
        assert all(v > 0.0 for v in r.values()), r
        hw2, mw2 = tr.get_weights()
        gh2, gm2 = tr.debug_gradients()
        assert np.array_equal(hw, hw2) and np.array_equal(mw, mw2)
        assert np.array_equal(gh, gh2) and np.array_equal(gm, gm2)
        assert np.array_equal(mask, tr.debug_active_mask())


def test_fused_step_profile_phases():
    """Phase events of the fused device step at the C2 shape (hash-grid
    backward inside the MLP kernel, reduction inside the finish kernel): the
    scatter and reduce phases have no work and no boundary events, so they
    read exactly 0; every other phase is positive and the phases add up to
    the step total."""
    torch = pytest.importorskip("torch")
    _say("fused step profile phases")
    d, enc, net, m_out, loss = BASELINE["c2"]
    n = 1 << 14
    with make_trainer(d, m_out, enc, net, loss=loss, precision="fp16", batch=n) as tr:
        assert tr.inspect_runtime()["train_fused_scatter"] == 1
        x = torch.rand(n, d, device="cuda:0")
        y = torch.rand(n, m_out, device="cuda:0")
        torch.cuda.synchronize()
        tr.training_step_device(x.data_ptr(), y.data_ptr(), n)
        tr.synchronize()
        tr.set_training_step_profiling(True, 1)
        for _ in range(3):
            tr.training_step_device(x.data_ptr(), y.data_ptr(), n)
        tr.synchronize()
        prof = tr.training_step_profile()
        tr.set_training_step_profiling(False)
        assert prof["steps"] == 3, prof
        assert prof["gpu_scatter_us"] == 0.0 and prof["gpu_reduce_us"] == 0.0, prof
        for k in ("gpu_sort_us", "gpu_encode_us", "gpu_fwd_bwd_us", "gpu_adam_us"):
            assert prof[k] > 0.0, (k, prof)
        parts = sum(prof[k] for k in ("gpu_sort_us", "gpu_encode_us", "gpu_fwd_bwd_us",
                                      "gpu_scatter_us", "gpu_reduce_us", "gpu_adam_us"))
        assert abs(parts - prof["gpu_total_us"]) <= 1e-3 * prof["gpu_total_us"], prof
        # the main kernels' own durations (dispatch timestamps): positive, no
        # scatter kernel, and each within its phase (which adds the launch gap)
        assert prof["gpu_scatter_kernel_us"] == 0.0, prof
        for kern, phase in (("gpu_encode_kernel_us", "gpu_encode_us"),
                            ("gpu_train_kernel_us", "gpu_fwd_bwd_us"),
                            ("gpu_finish_kernel_us", "gpu_adam_us")):
            assert 0.0 < prof[kern] <= prof[phase] * 1.001, (kern, phase, prof)


def test_profile_samples_add_up_to_the_profile_and_lds_rate_is_sane():
    """tmnn_get_step_profile_samples: one row per profiled step, in the
    columns of PROFILE_PHASES, whose column sums are the aggregate profile
    (tmnn_get_step_profile) and whose phases add up to each row's total;
    reading keeps them, switching profiling off drops them.
    tmnn_debug_lds_rate: between 1 TB/s and 1 PB/s (a few hundred CUs
    reading at most a few hundred bytes per clock each)."""
    torch = pytest.importorskip("torch")
    from tiny_metal_nn._lib import PROFILE_PHASES
    _say("profile samples, lds rate")
    d, enc, net, m_out, loss = BASELINE["c2"]
    n = 1 << 14
    with make_trainer(d, m_out, enc, net, loss=loss, precision="fp16", batch=n) as tr:
        x = torch.rand(n, d, device="cuda:0")
        y = torch.rand(n, m_out, device="cuda:0")
        torch.cuda.synchronize()
        tr.training_step_device(x.data_ptr(), y.data_ptr(), n)
        tr.synchronize()
        tr.set_training_step_profiling(True, 1)
        for _ in range(4):
            tr.training_step_device(x.data_ptr(), y.data_ptr(), n)
        tr.synchronize()
        rows = tr.training_step_profile_samples()
        assert rows.shape == (4, len(PROFILE_PHASES)), rows.shape
        col = {k: i for i, k in enumerate(PROFILE_PHASES)}
        phases = ("gpu_sort_us", "gpu_encode_us", "gpu_fwd_bwd_us", "gpu_scatter_us",
                  "gpu_reduce_us", "gpu_adam_us")
        for r in rows:
            total = r[col["gpu_total_us"]]
            assert total > 0.0
            assert abs(sum(r[col[k]] for k in phases) - total) <= 1e-3 * total, r
            assert 0.0 < r[col["gpu_train_kernel_us"]] <= r[col["gpu_fwd_bwd_us"]] * 1.001, r
        prof = tr.training_step_profile()
        assert prof["steps"] == 4, prof
        for k in PROFILE_PHASES:
            assert abs(float(rows[:, col[k]].sum()) - prof[k]) <= 1e-3 * max(1.0, prof[k]), (k, prof)
        assert np.array_equal(tr.training_step_profile_samples(), rows)
        tr.set_training_step_profiling(False)
        assert tr.training_step_profile_samples().shape[0] == 0
        rate = tr.debug_lds_rate(3)
        assert 1e12 < rate < 1e15, rate
