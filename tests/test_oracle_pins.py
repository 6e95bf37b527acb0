"""Pins of the CPU oracle (oracle/tmnn_oracle.cpp) -- CPU only.

Each test checks the oracle against something other than itself: the
reference's golden vectors and published trajectory, the reference's own
compiled host code and generated MSL text (oracle/_ref), closed forms, and
finite differences.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
PY, PZ, PW = 2654435761, 805459861, 56711039


# ---------------------------------------------------------------- Philox --

def test_philox_seed42_golden_is_bit_exact(oracle):
    g = json.loads((GOLDEN / "philox_seed42_golden.json").read_text())
    out = oracle.philox_uniform(g["seed"], g["counter_base"], g["count"], g["low"], g["high"])
    gold = np.array(g["first8"], np.float32)
    assert np.array_equal(out[:8].view(np.uint32), gold.view(np.uint32))


def test_philox_counter_base_offsets_the_stream(oracle):
    a = oracle.philox_uniform(7, 0, 64, 0.0, 1.0)
    b = oracle.philox_uniform(7, 4, 48, 0.0, 1.0)  # counter 4 -> element 16
    assert np.array_equal(a[16:], b)
    assert 0.0 <= a.min() and a.max() < 1.0


# ------------------------------------------------------- end-to-end pins --

def test_sphere_sdf_trajectory_matches_reference(oracle):
    """examples/sphere_sdf: the reference's published Metal loss curve."""
    torch = pytest.importorskip("torch")
    g = json.loads((GOLDEN / "sphere_sdf_reference_metrics.json").read_text())
    m = oracle.model(3, 4, 2, 14, 16.0, 1.5, 16, 1, 1, "L2")
    assert oracle.counts(m)[:2] == (g["params"]["encoding"], g["params"]["network"])
    a = oracle.adam(1e-2, 1e-2)
    h, w = oracle.init_params(m, 42, 1e-4)
    params = np.concatenate([h, w])
    m1, m2 = np.zeros_like(params), np.zeros_like(params)
    torch.manual_seed(42)
    losses = []
    for step in range(50):
        pos = torch.rand(4096, 3, dtype=torch.float32)
        tgt = ((pos - 0.5).norm(dim=1, keepdim=True) - 0.5).to(torch.float32)
        losses.append(oracle.training_step(m, a, step, params, m1, m2, pos.numpy(), tgt.numpy()))
    ref = {int(k): v for k, v in g["convergence"].items()}
    # step 0 is a forward pass on the seeded init: fast-math ulps only
    assert losses[0] == pytest.approx(ref[0], rel=1e-5)
    # later steps go through Adam and the int32 gradient truncation
    for k, v in ref.items():
        assert losses[k] == pytest.approx(v, rel=0.02), (k, losses[k], v)


def test_closed_form_034(oracle):
    """test_default_trainer.cpp:2260-2336: constant table 0.5, weights 0.1."""
    m = oracle.model(3, 2, 2, 10, 4.0, 2.0, 8, 1, 1, "L2")
    nh, nm, _ = oracle.counts(m)
    assert nm == 49
    table = np.full(nh, 0.5, np.float32)
    mlp = np.full(nm, 0.1, np.float32)
    pos = np.array([[0.5, 0.5, 0.5]], np.float32)
    assert np.all(oracle.encode(m, table, pos) == 0.5)
    out = oracle.forward(m, table, mlp, pos)
    assert out[0, 0] == pytest.approx(0.34, abs=1e-4)


# ------------------------------------------- reference host code (_ref) --

@pytest.mark.parametrize("geom", [(32, 64, 2, 3), (32, 64, 2, 1), (32, 64, 1, 16),
                                  (64, 64, 3, 1), (32, 128, 4, 4), (4, 8, 1, 1),
                                  (8, 16, 1, 1)])
def test_mlp_weight_count_matches_reference(oracle, reflib, geom):
    inp, hd, nhl, nout = geom
    F = 2 if inp % 2 == 0 else 1
    m = oracle.model(3, inp // F, F, 12, 16.0, 1.5, hd, nhl, nout)
    assert oracle.counts(m)[1] == reflib.lib.ref_mlp_weight_count(inp, hd, nhl, nout)


def test_morton_codes_match_reference(oracle, reflib):
    rng = np.random.default_rng(3)
    p3 = rng.uniform(-1.3, 1.3, (2000, 3)).astype(np.float32)
    p3[:5] = [[-1, -1, -1], [1, 1, 1], [0, 0, 0], [0.999, -0.999, 0.5], [2, -2, 0]]
    got = oracle.morton_codes(p3, 3)
    ref = np.array([reflib.lib.ref_morton_code_3d(*map(float, p)) for p in p3], np.uint32)
    assert np.array_equal(got, ref)
    p4 = rng.uniform(-1.3, 1.3, (2000, 4)).astype(np.float32)
    got4 = oracle.morton_codes(p4, 4)
    ref4 = np.array([reflib.lib.ref_morton_code_4d(*map(float, p)) for p in p4], np.uint32)
    assert np.array_equal(got4, ref4)
    # 2D points are lifted to (x, y, 0)
    p2 = p3[:, :2].copy()
    lifted = np.concatenate([p2, np.zeros((len(p2), 1), np.float32)], 1)
    assert np.array_equal(oracle.morton_codes(p2, 2), oracle.morton_codes(lifted, 3))


def test_morton_sort_order_matches_reference(oracle, reflib):
    rng = np.random.default_rng(4)
    pos = rng.random((5000, 3), dtype=np.float32)
    tgt = rng.random((5000, 2), dtype=np.float32)
    sp, st, idx = reflib.morton_sort_batch(pos, tgt)
    codes = oracle.morton_codes(pos, 3)
    stable = np.argsort(codes, kind="stable")
    # same key sequence; ties may be permuted by the reference's std::sort
    assert np.array_equal(codes[stable], codes[idx])
    assert np.array_equal(sp, pos[idx]) and np.array_equal(st, tgt[idx])


@pytest.mark.parametrize("kind,name", [(0, "L2"), (1, "L1"), (2, "Huber")])
def test_elementwise_losses_match_reference_cpu_losses(oracle, reflib, kind, name):
    """loss = (sum over points and outputs) / N, vs the reference's
    detail/{l2,l1,huber}_loss.h evaluate_cpu (mean over elements)."""
    rng = np.random.default_rng(kind)
    m = oracle.model(3, 2, 2, 10, 4.0, 2.0, 16, 1, 3, name, huber_delta=0.05)
    h, w = oracle.init_params(m, 5, 0.5)
    pos = rng.random((257, 3), dtype=np.float32)
    tgt = rng.normal(0, 0.2, (257, 3)).astype(np.float32)
    _, _, _, loss_sum, out = oracle.forward_backward(m, h, w, pos, target=tgt)
    ref = reflib.loss_evaluate_cpu(kind, out, tgt, delta=0.05)
    assert loss_sum / 257 == pytest.approx(ref * 3, rel=1e-5)


def test_cosine_loss_matches_reference_cpu_loss(oracle, reflib):
    rng = np.random.default_rng(9)
    m = oracle.model(3, 2, 2, 10, 4.0, 2.0, 16, 1, 4, "Cosine")
    h, w = oracle.init_params(m, 6, 0.5)
    pos = rng.random((129, 3), dtype=np.float32)
    tgt = rng.normal(0, 1.0, (129, 4)).astype(np.float32)
    _, _, _, loss_sum, out = oracle.forward_backward(m, h, w, pos, target=tgt)
    ref = reflib.loss_evaluate_cpu(3, out, tgt, output_dims=4)
    assert loss_sum / 129 == pytest.approx(ref, rel=1e-5)


def test_kernel_spec_bounds_match_reference(reflib):
    ok = reflib.lib.ref_kernel_spec_validate
    assert ok(16, 2, 19, 64, 2, 3) == 0
    assert ok(16, 3, 19, 64, 2, 3) == 1      # F must be 1, 2, 4
    assert ok(33, 2, 19, 64, 2, 3) == 1      # L <= 32
    assert ok(16, 2, 25, 64, 2, 3) == 1      # log2T <= 24
    assert ok(16, 2, 19, 64, 9, 3) == 1      # nhl <= 8
    assert ok(16, 2, 19, 64, 2, 2) == 1      # the reference has no native 2D


# ------------------------------------ the reference's generated MSL text --

def test_emitted_msl_has_the_oracles_hash_and_gradient_forms(reflib):
    """The restated formulas appear verbatim in the reference's emitted
    kernels (mlp_kernel_emitter.cpp): primes, fixed-point scale, the float2
    scatter association, both resolution formulas and the 6-decimal baking."""
    src = reflib.emit_kernel_source(0, 3, 16, 2, 19, 16.0, 1.3819128799, 64, 2, 3, 0)
    assert f"uint(coords.y) * {PY}u" in src and f"uint(coords.z) * {PZ}u" in src
    assert "#define GRAD_SCALE 65536.0f" in src
    assert "int(d_feat2.x * w * GRAD_SCALE)" in src
    assert "float w=wx*wy*wz;" in src
    assert "BASE_RESOLUTION * pow(PER_LEVEL_SCALE, float(l))" in src
    assert "constant float PER_LEVEL_SCALE = 1.381913f;" in src
    assert "d_out[m] = 2.0f * residual * inv_N;" in src
    assert "uint entry_idx = grid_off >> 1u;" in src
    src4 = reflib.emit_kernel_source(0, 4, 16, 2, 19, 8.0, 1.4, 128, 4, 4, 0)
    assert f"uint(coords.w) * {PW}u" in src4
    assert "int(d_feat * wx * wy * wz * wt * GRAD_SCALE)" in src4
    src1 = reflib.emit_kernel_source(0, 3, 8, 1, 14, 16.0, 1.5, 32, 1, 1, 0)
    assert "int(d_feat * wx * wy * wz * GRAD_SCALE)" in src1
    ev = reflib.emit_kernel_source(1, 3, 16, 2, 19, 16.0, 1.5, 64, 2, 3, 0)
    assert "resolution *= PER_LEVEL_SCALE;" in ev


# --------------------------------------------------- closed forms / math --

def test_resolution_table(oracle):
    m = oracle.model(3, 16, 2, 15, 16.0, 1.5)
    r = oracle.resolutions(m)
    # 16 * 1.5^l = 3^l * 2^(4-l) is exact in fp32 for l < 16
    assert np.array_equal(r, np.array([16 * 1.5 ** l for l in range(16)], np.float32))
    m3 = oracle.model(3, 16, 2, 19, 16.0, 128 ** (1 / 15))
    r3 = oracle.resolutions(m3)
    assert r3[-1] == pytest.approx(2048.0, rel=2e-5)
    assert r3[1] == np.float32(16.0) * np.float32(1.381913)


def test_hash_indices_closed_form(oracle):
    """Corner 0 of a level is floor(p*r); its index is x ^ y*PY ^ z*PZ mod T.
    Points placed on lattice coordinates make every corner known."""
    m = oracle.model(3, 3, 2, 12, 4.0, 2.0)
    T = 1 << 12
    table = np.zeros(oracle.counts(m)[0], np.float32)
    ijk = np.array([[0, 0, 0], [1, 0, 0], [0, 1, 0], [0, 0, 1], [3, 2, 1], [7, 5, 6]])
    pos = (ijk / 8.0 + 1e-3).astype(np.float32)  # level 1 has r = 8
    _, idx, w = oracle.encode(m, table, pos, with_corners=True)

    def h(x, y, z):
        return ((x * 1) ^ ((y * PY) & 0xFFFFFFFF) ^ ((z * PZ) & 0xFFFFFFFF)) % T

    for n, (i, j, k) in enumerate(ijk):
        for c in range(8):
            dx, dy, dz = c & 1, (c >> 1) & 1, (c >> 2) & 1
            assert idx[n, 1, c] == h(i + dx, j + dy, k + dz)
    assert idx[0, 1, 0] == 0 and idx[1, 1, 0] == 1 and idx[2, 1, 0] == PY % T
    assert np.allclose(w.sum(-1), 1.0, atol=1e-6)


def test_2d_is_the_lifted_3d(oracle):
    rng = np.random.default_rng(11)
    m2 = oracle.model(2, 16, 2, 15, 16.0, 1.5, 64, 2, 3)
    m3 = oracle.model(3, 16, 2, 15, 16.0, 1.5, 64, 2, 3)
    h, w = oracle.init_params(m2, 1, 0.1)
    p2 = rng.random((300, 2), dtype=np.float32)
    p3 = np.concatenate([p2, np.zeros((300, 1), np.float32)], 1)
    f2, i2, w2 = oracle.encode(m2, h, p2, with_corners=True)
    f3, i3, w3 = oracle.encode(m3, h, p3, with_corners=True)
    assert np.array_equal(f2, f3) and np.array_equal(i2, i3)
    assert np.all(w2[:, :, 4:] == 0.0)  # the z = 1 plane has weight 0


def test_trilinear_reproduces_linear_tables(oracle):
    """A table that is linear in the lattice coordinates interpolates to the
    same linear function (checked away from hash collisions: tiny grid)."""
    m = oracle.model(3, 1, 1, 16, 8.0, 2.0)
    T = 1 << 16
    table = np.zeros(T, np.float32)
    for x in range(10):
        for y in range(10):
            for z in range(10):
                hh = (x ^ ((y * PY) & 0xFFFFFFFF) ^ ((z * PZ) & 0xFFFFFFFF)) % T
                table[hh] = 0.5 * x - 0.25 * y + 0.125 * z
    rng = np.random.default_rng(2)
    pos = rng.random((500, 3), dtype=np.float32)
    f = oracle.encode(m, table, pos)[:, 0]
    s = pos.astype(np.float64) * 8.0
    want = 0.5 * s[:, 0] - 0.25 * s[:, 1] + 0.125 * s[:, 2]
    assert np.allclose(f, want, atol=1e-5)


def _zero_mlp_with_bias(oracle, m, bias_out):
    nh, nm, _ = oracle.counts(m)
    w = np.zeros(nm, np.float32)
    w[nm - m.num_outputs:] = bias_out
    return np.zeros(nh, np.float32), w


@pytest.mark.parametrize("loss,y,t,lval,dval", [
    ("L2", 0.75, 0.25, 0.25, 1.0),
    ("L1", 0.75, 0.25, 0.5, 1.0),
    ("L1", -0.5, 0.25, 0.75, -1.0),
    ("Huber", 0.75, 0.25, 0.25 * (0.5 - 0.125), 0.25),   # delta 0.25, |r| > delta
    ("Huber", 0.3, 0.25, 0.5 * 0.05 ** 2, 0.05),         # |r| <= delta
    ("RelativeL2", 1.0, 0.0, 1 / 1.01, 2 / 1.01),
    ("RelativeL2", 0.1, 0.0, 0.5, 10.0),
])
def test_loss_closed_forms(oracle, loss, y, t, lval, dval):
    """Output = bias exactly (zero weights); loss/N and dL/dbias are closed
    form. RelativeL2 follows tcnn: r^2/(y^2+0.01), denominator constant in
    the gradient."""
    m = oracle.model(3, 2, 2, 10, 4.0, 2.0, 8, 1, 1, loss, huber_delta=0.25)
    h, w = _zero_mlp_with_bias(oracle, m, y)
    n = 64
    pos = np.random.default_rng(0).random((n, 3), dtype=np.float32)
    tgt = np.full((n, 1), t, np.float32)
    _, gm, _, lsum, out = oracle.forward_backward(m, h, w, pos, target=tgt)
    assert np.all(out == np.float32(y))
    assert lsum / n == pytest.approx(lval, rel=1e-5)
    assert gm[-1] == pytest.approx(dval, rel=1e-5)  # sum_i d_out_i = N * (dval / N)


def _total_loss(oracle, m, h, w, pos, tgt):
    _, _, _, lsum, _ = oracle.forward_backward(m, h, w, pos, target=tgt)
    return lsum


@pytest.mark.parametrize("loss,nhl", [("L2", 2), ("L1", 1), ("Huber", 2), ("Cosine", 1)])
def test_mlp_gradients_match_finite_differences(oracle, loss, nhl):
    rng = np.random.default_rng(21)
    m = oracle.model(3, 2, 2, 10, 4.0, 2.0, 16, nhl, 3, loss, huber_delta=0.1)
    h, w = oracle.init_params(m, 3, 0.5)
    pos = rng.random((64, 3), dtype=np.float32)
    tgt = rng.normal(0, 0.5, (64, 3)).astype(np.float32)
    _, gm, _, _, _ = oracle.forward_backward(m, h, w, pos, target=tgt)
    n = 64
    checked = 0
    for k in rng.choice(len(w), 40, replace=False):
        if abs(gm[k]) < 1e-3:
            continue
        eps = 1e-3
        wp, wm = w.copy(), w.copy()
        wp[k] += eps
        wm[k] -= eps
        fd = (_total_loss(oracle, m, h, wp, pos, tgt) - _total_loss(oracle, m, h, wm, pos, tgt))
        fd /= (wp[k] - wm[k]) * n  # the gradient carries 1/N
        assert gm[k] == pytest.approx(fd, rel=3e-2, abs=2e-4), k
        checked += 1
    assert checked >= 8


def test_hash_gradients_match_finite_differences(oracle):
    """With an external output gradient g, d(sum g*y)/d table = grad_hash/65536."""
    rng = np.random.default_rng(5)
    m = oracle.model(3, 2, 2, 10, 4.0, 2.0, 16, 1, 2, "L2")
    h, w = oracle.init_params(m, 8, 0.5)
    pos = rng.random((8, 3), dtype=np.float32)
    g = rng.normal(0, 1.0, (8, 2)).astype(np.float32)
    gh, _, mask, _, _ = oracle.forward_backward(m, h, w, pos, d_out=g)
    touched = np.flatnonzero(gh)
    assert len(touched) > 20
    for k in rng.choice(touched, 20, replace=False):
        eps = 1e-2
        hp, hm = h.copy(), h.copy()
        hp[k] += eps
        hm[k] -= eps
        fp = float((oracle.forward(m, hp, w, pos) * g).sum())
        fm = float((oracle.forward(m, hm, w, pos) * g).sum())
        fd = (fp - fm) / (hp[k] - hm[k])
        assert gh[k] / 65536.0 == pytest.approx(fd, rel=2e-2, abs=2e-3), k
        slot = k >> 1
        assert (mask[slot >> 5] >> (slot & 31)) & 1


def test_gradients_are_linear_in_the_output_gradient(oracle):
    """AccumGradientLinearityFourCalls (test_default_trainer.cpp:2754-2818)."""
    rng = np.random.default_rng(6)
    m = oracle.model(3, 4, 2, 12, 8.0, 1.5, 32, 2, 3)
    h, w = oracle.init_params(m, 9, 0.2)
    pos = rng.random((200, 3), dtype=np.float32)
    g = rng.normal(0, 1.0, (200, 3)).astype(np.float32)
    gh1, gm1, _, _, _ = oracle.forward_backward(m, h, w, pos, d_out=g)
    gh4, gm4, _, _, _ = oracle.forward_backward(m, h, w, pos, d_out=4 * g)
    assert np.array_equal(gm4, 4 * gm1)  # 4*x is exact in fp32
    # int32 truncation per contribution: |int(4v) - 4 int(v)| < 4 per term
    assert np.abs(gh4.astype(np.int64) - 4 * gh1.astype(np.int64)).max() <= 4 * 200


def test_adam_first_step_closed_form(oracle):
    """Step 0: m_hat = g, v_hat = g^2, so w moves by lr*sign(g) (eps ~ 0)."""
    m = oracle.model(3, 1, 2, 10, 4.0, 2.0, 8, 1, 1)
    nh, nm, nw = oracle.counts(m)
    a = oracle.adam(0.01, 0.001)
    params = np.full(nh + nm, 0.5, np.float32)
    m1, m2 = np.zeros_like(params), np.zeros_like(params)
    gh = np.zeros(nh, np.int32)
    gh[:4] = [65536, -65536, 3, 0]
    gm = np.zeros(nm, np.float32)
    gm[:2] = [0.25, -1e-3]
    oracle.adam_step(m, a, 0, params, m1, m2, gh, gm, mask=None)
    assert params[0] == pytest.approx(0.49, abs=1e-7)
    assert params[1] == pytest.approx(0.51, abs=1e-7)
    assert params[2] == pytest.approx(0.49, abs=1e-7)   # g = 3/65536 > 0
    assert params[3] == 0.5                               # g = 0, m = v = 0
    assert params[nh] == pytest.approx(0.499, abs=1e-7)
    assert params[nh + 1] == pytest.approx(0.501, abs=1e-7)
    b1, b2 = oracle.bias_corrections(0.9, 0.99, 0)
    assert b1 == np.float32(1) - np.float32(0.9) and b2 == np.float32(1) - np.float32(0.99)


def _two_adam_steps(oracle, a, w0, gh_steps, gm_steps, mask=None):
    """Two Adam steps of the oracle on a 1-level model with every parameter
    starting at w0 (hash w0[0] for entries 0..3, MLP w0[1] for all MLP
    parameters unless w0 has more entries); returns the parameters after each
    step."""
    m = oracle.model(3, 1, 2, 10, 4.0, 2.0, 8, 1, 1)
    nh, nm, _ = oracle.counts(m)
    params = np.full(nh + nm, 0.5, np.float32)
    for i, w in enumerate(w0):
        params[i if i < 4 else nh + i - 4] = w
    m1, m2 = np.zeros_like(params), np.zeros_like(params)
    out = []
    for step, (gh_vals, gm_vals) in enumerate(zip(gh_steps, gm_steps)):
        gh = np.zeros(nh, np.int32)
        gh[:len(gh_vals)] = gh_vals
        gm = np.zeros(nm, np.float32)
        gm[:len(gm_vals)] = gm_vals
        oracle.adam_step(m, a, step, params, m1, m2, gh, gm, mask=mask)
        out.append((params[:4].astype(np.float64).copy(), params[nh:nh + 4].astype(np.float64).copy()))
    return out


def _adam2(g1, g2, lr):
    """Hand-evaluated second Adam step from zero moments (beta 0.9 / 0.99):
    m = 0.09 g1 + 0.1 g2, v = 0.0099 g1^2 + 0.01 g2^2, bias corrections
    0.19 and 0.0199; returns the two steps' moves (lr * m_hat / sqrt(v_hat))."""
    d1 = lr * np.sign(g1) if g1 != 0 else 0.0
    m = 0.09 * g1 + 0.1 * g2
    v = 0.0099 * g1 * g1 + 0.01 * g2 * g2
    return d1, lr * (m / 0.19) / np.sqrt(v / 0.0199)


def test_adam_gradient_clip_two_steps(oracle):
    """grad_clip (adam_kernel_msl.h:81-82): clamp(g, -c, c) before the
    moments. A first gradient above the clip and a second below it make the
    clip visible in the second step: with c = 0.5, hash g = 5 then 0.125 and
    MLP g = -2 then 0.25 move like 0.5 then 0.125 and -0.5 then 0.25 (and not
    like the raw values, whose second step differs by 17% and 60%)."""
    a = oracle.adam(0.01, 0.01, grad_clip=0.5)
    out = _two_adam_steps(oracle, a, [], [[5 * 65536], [8192]], [[-2.0], [0.25]])
    dh1, dh2 = _adam2(0.5, 0.125, 0.01)
    dm1, dm2 = _adam2(-0.5, 0.25, 0.01)
    assert out[0][0][0] == pytest.approx(0.5 - dh1, abs=2e-7)
    assert out[1][0][0] == pytest.approx(0.5 - dh1 - dh2, abs=2e-7)
    assert out[0][1][0] == pytest.approx(0.5 - dm1, abs=2e-7)
    assert out[1][1][0] == pytest.approx(0.5 - dm1 - dm2, abs=2e-7)
    _, raw2 = _adam2(5.0, 0.125, 0.01)
    assert abs(raw2 - dh2) > 0.1 * dh2  # the clip changed the second step


def test_adam_l1_hash_regularisation_two_steps(oracle):
    """l1_reg (adam_kernel_msl.h:89-92): g += l1 * sign(w) on hash entries
    only, with the sign of the weight before the step. Zero gradients, l1 =
    0.01, lr = 0.01: w = 0.5 and -0.5 each move lr toward 0, w = 0 stays; w =
    0.005 crosses zero in step 1 (to -0.005), so step 2 sees g = -0.01:
    m = 0.09 * 0.01 - 0.1 * 0.01, v = 0.0099e-4 + 0.01e-4, and w ends at
    -0.005 + 0.01 * (1e-4 / 0.19) / sqrt(1.99e-6 / 0.0199). MLP parameters get
    no L1 term (zero gradient, zero moments: unchanged)."""
    a = oracle.adam(0.01, 0.01, l1_reg=0.01)
    out = _two_adam_steps(oracle, a, [0.5, -0.5, 0.0, 0.005], [[], []], [[], []])
    h1, m1_ = out[0]
    h2, m2_ = out[1]
    assert h1[0] == pytest.approx(0.49, abs=1e-7) and h1[1] == pytest.approx(-0.49, abs=1e-7)
    assert h1[2] == 0.0 and h2[2] == 0.0
    assert h1[3] == pytest.approx(-0.005, abs=1e-8)
    want = -0.005 + 0.01 * (1e-4 / 0.19) / np.sqrt(1.99e-6 / 0.0199)
    assert h2[3] == pytest.approx(want, abs=2e-8)
    assert np.all(m1_ == np.float32(0.5)) and np.all(m2_ == np.float32(0.5))


def test_adam_l2_mlp_regularisation_two_steps(oracle):
    """l2_reg (adam_kernel_msl.h:93-95): g += l2 * w on MLP parameters only.
    Zero gradients, l2 = 0.1, lr = 0.01, w = 0.5: step 1 sees g = 0.05 and
    moves lr; step 2 sees g = 0.049 (w = 0.49): m = 0.0045 + 0.0049,
    v = 0.0099 * 0.05^2 + 0.01 * 0.049^2, w = 0.49 - 0.01 * m_hat /
    sqrt(v_hat). Hash entries get no L2 term (unchanged)."""
    a = oracle.adam(0.01, 0.01, l2_reg=0.1)
    out = _two_adam_steps(oracle, a, [], [[], []], [[], []])
    m = 0.09 * 0.05 + 0.1 * 0.049
    v = 0.0099 * 0.05 ** 2 + 0.01 * 0.049 ** 2
    assert out[0][1][0] == pytest.approx(0.49, abs=1e-7)
    assert out[1][1][0] == pytest.approx(0.49 - 0.01 * (m / 0.19) / np.sqrt(v / 0.0199), abs=2e-7)
    assert np.all(out[1][0] == np.float32(0.5))


def test_adamw_decay_first_and_suppresses_l1_l2(oracle):
    """weight_decay (adam_kernel_msl.h:84-88): w -= lr * wd * w before the
    Adam move, and L1/L2 are then not applied. wd = 0.1, lr = 0.01, l1 = l2 =
    0.1 set as well: a hash entry with g = 0.25 goes 0.5 -> 0.4995 - 0.01; an
    MLP parameter with g = 0 only decays (0.5 -> 0.4995, no L2 move); step 2
    decays again before its move."""
    a = oracle.adam(0.01, 0.01, l1_reg=0.1, l2_reg=0.1, weight_decay=0.1)
    out = _two_adam_steps(oracle, a, [], [[16384], [16384]], [[], []])
    assert out[0][0][0] == pytest.approx(0.4995 - 0.01, abs=1e-7)
    assert out[0][1][0] == pytest.approx(0.4995, abs=1e-7)
    w1 = 0.4995 - 0.01
    assert out[1][0][0] == pytest.approx(w1 * (1 - 0.001) - 0.01, abs=2e-7)
    assert out[1][1][0] == pytest.approx(0.4995 * (1 - 0.001), abs=1e-7)
    # a zero-gradient hash entry decays only
    assert out[0][0][1] == pytest.approx(0.4995, abs=1e-7)


def test_lazy_adam_branches_match_dense_on_marked_entries(oracle):
    """The sparse hash kernel (adam_kernel_msl.h:120-164) applies clip and
    AdamW like the unified one: on marked entries the lazy and dense updates
    agree bit for bit."""
    a = oracle.adam(0.01, 0.01, grad_clip=0.5, weight_decay=0.05)
    m = oracle.model(3, 1, 2, 10, 4.0, 2.0, 8, 1, 1)
    nh, nm, nw = oracle.counts(m)
    mask = np.zeros(nw, np.uint32)
    mask[0] = 0b11  # slots 0 and 1 -> elements 0..3
    dense = _two_adam_steps(oracle, a, [0.3, -0.2, 0.1, 0.0], [[5 * 65536, -8192, 3], [8192, 1, 0]],
                            [[], []])
    lazy = _two_adam_steps(oracle, a, [0.3, -0.2, 0.1, 0.0], [[5 * 65536, -8192, 3], [8192, 1, 0]],
                           [[], []], mask=mask)
    for (hd, _), (hl, _) in zip(dense, lazy):
        assert np.array_equal(hd, hl)


def test_lazy_adam_updates_only_marked_entries(oracle):
    """neural_sdf_adam_hash_sparse: unmarked entries keep w, m, v; marked
    entries with g = 0 still move by their momentum."""
    m = oracle.model(3, 1, 2, 10, 4.0, 2.0, 8, 1, 1)
    nh, nm, nw = oracle.counts(m)
    a = oracle.adam()
    params = np.full(nh + nm, 0.5, np.float32)
    m1 = np.full_like(params, 0.1)
    m2 = np.full_like(params, 0.01)
    mask = np.zeros(nw, np.uint32)
    mask[0] = 0b101  # slots 0 and 2 -> elements 0,1 and 4,5
    gh = np.zeros(nh, np.int32)
    gh[0] = 65536
    oracle.adam_step(m, a, 3, params, m1, m2, gh, np.zeros(nm, np.float32), mask=mask)
    moved = np.flatnonzero(params[:nh] != 0.5)
    assert set(moved) == {0, 1, 4, 5}
    assert np.all(m1[2:4] == np.float32(0.1)) and np.all(m2[6:nh] == np.float32(0.01))


def test_training_step_reports_sum_over_outputs_over_n(oracle):
    """ParameterStore::finalize_async_step: loss = sum(partials) / N, each
    point contributing the sum over its outputs (finding 13)."""
    m = oracle.model(3, 2, 2, 10, 4.0, 2.0, 8, 1, 3, "L2")
    h, w = _zero_mlp_with_bias(oracle, m, [0.5, 0.25, -0.5])
    params = np.concatenate([h, w])
    m1, m2 = np.zeros_like(params), np.zeros_like(params)
    pos = np.random.default_rng(1).random((100, 3), dtype=np.float32)
    tgt = np.zeros((100, 3), np.float32)
    loss = oracle.training_step(m, oracle.adam(), 0, params, m1, m2, pos, tgt)
    assert loss == pytest.approx(0.25 + 0.0625 + 0.25, rel=1e-6)


@pytest.mark.parametrize("d,f,nhl,m_out", [(3, 2, 2, 1), (2, 2, 1, 3), (4, 2, 1, 2), (3, 4, 1, 1),
                                           (3, 1, 2, 2)])
def test_position_gradient_matches_finite_differences(oracle, d, f, nhl, m_out):
    """evaluate_with_gradient (mlp_kernel_emitter.cpp:1865-2090): the analytic
    Jacobian equals central differences of the oracle's own forward, and its
    output equals orc_forward exactly. Points are kept away from cell faces so
    the +-eps steps stay in one cell at every level (ReLU kinks may still lie
    inside a step)."""
    m = oracle.model(d, 4, f, 12, 4.0, 2.0, 16, nhl, m_out, "L2")
    h, w = oracle.init_params(m, 5, 0.5)
    rng = np.random.default_rng(d * 10 + f)
    res = oracle.resolutions(m).astype(np.float64)
    pts = []
    while len(pts) < 24:
        p = rng.random(d) * 0.8 + 0.1
        fr = (p[None, :] * res[:, None]) % 1.0
        if np.all((fr > 0.05) & (fr < 0.95)):
            pts.append(p)
    pos = np.array(pts, np.float32)
    out, jac = oracle.evaluate_with_gradient(m, h, w, pos)
    assert np.array_equal(out, oracle.forward(m, h, w, pos))
    eps = 1e-4
    for a in range(d):
        pp, pm = pos.astype(np.float64).copy(), pos.astype(np.float64).copy()
        pp[:, a] += eps
        pm[:, a] -= eps
        fd = (oracle.forward(m, h, w, pp.astype(np.float32)).astype(np.float64)
              - oracle.forward(m, h, w, pm.astype(np.float32)).astype(np.float64))
        fd /= (pp[:, a].astype(np.float32).astype(np.float64)
               - pm[:, a].astype(np.float32).astype(np.float64))[:, None]
        # a ReLU kink inside +-eps spoils the difference at a few points;
        # a wrong term or sign would spoil nearly all of them
        err = np.abs(jac[:, :, a] - fd) / np.abs(jac).max()
        assert (err <= 2e-3).mean() >= 0.85, (a, np.sort(err.ravel())[-5:])
