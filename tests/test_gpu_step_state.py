"""GPU parity, third part: the state one fused fp16 step leaves behind with
the kernels the benchmark times (the 64-wide fp16 training kernel with the
hash-grid backward fused per tile, then the finish kernel: dW reduction,
loss, Adam), the C5 shape at its BASELINE table size, the numerics report of
the step result, and device steps ordered after a caller's stream. Marked
gpu; every comparison is against the CPU oracle on identical seeded inputs
or against the library's own synchronous path.

Tolerances (north_star): fp16-compute outputs and gradients within 2e-3 of
the tensor's largest magnitude; loss after N Adam steps within 1%.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from test_gpu_coverage import BASELINE, parse_optimizer_blob
from test_gpu_parity import away_from_relu_kinks, make_trainer, omodel, rel_tensor

pytestmark = pytest.mark.gpu

LR, BETA1, BETA2 = 1e-2, 0.9, 0.99


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


# Hash-table gradients are sums of int32(trunc(d * w * 65536)) per corner
# contribution: besides the fp16 bar on d (2e-3 of the largest gradient),
# each contribution whose fp32 and fp16 values straddle an integer truncates
# differently, one unit of 2^-16 each; the fp32 fused-step test allows 16 such
# units per entry and so does this one.
G_ULP = 16.0 / 65536.0


def _update_check(got, before, g, lr, what, slack=0.0):
    """One Adam step from zero moments moves each parameter by lr * g / |g|
    (up to fp32 rounding): where the oracle's gradient is larger than the
    fp16 tolerance (2e-3 max|g| + slack), so that the GPU's cannot have the
    other sign or be zero, the new parameter equals the oracle's within 1e-6;
    elsewhere the step is still at most lr."""
    big = np.abs(g) > 2e-3 * np.abs(g).max() + slack
    d = np.abs(got.astype(np.float64) - (before.astype(np.float64) - lr * np.sign(g)))
    assert d[big].max() <= 1e-6, (what, d[big].max())
    step = np.abs(got.astype(np.float64) - before.astype(np.float64))
    assert step.max() <= lr * 1.0001, (what, step.max())


@pytest.mark.parametrize("name", ["c2", "c3"])
def test_one_fused_fp16_step_state_matches_oracle(oracle, name):
    """One fused fp16 step at the C2 (2D, T = 2^15, 64x2 -> 3, RelativeL2) and
    C3 (3D, T = 2^19, 64 -> 16, L2) geometries, whose training kernel runs the
    hash-grid backward of each tile itself: the training kernel's forward
    outputs, the loss, the MLP and hash-table first and second moments within
    2e-3 of each tensor's largest magnitude; the parameters the single Adam
    step produced per element (_update_check); the entries Adam touched equal
    except where both sides' moment is within 2e-3 of the tensor's largest
    (an fp16 gradient of a tiny entry truncating to zero on one side); and
    the step's numerics report against the same quantities."""
    d, enc, net, m_out, loss = BASELINE[name]
    n = 65536 if name == "c2" else 16384
    _say(f"fp16 step state {name} n={n}")
    rng = np.random.default_rng(31)
    with make_trainer(d, m_out, enc, net, loss=loss, precision="fp16", hash_range=0.5,
                      batch=n) as tr:
        ins = tr.inspect_runtime()
        assert ins["train_fused_scatter"] == 1 and ins["precision"] == 1
        hw, mw = tr.get_weights()
        pos = away_from_relu_kinks(oracle, tr, hw, mw, rng.random((n, d), dtype=np.float32))
        assert len(pos) > 0.95 * n
        tgt = rng.random((len(pos), m_out), dtype=np.float32)
        out, res = tr.debug_step_outputs(pos, tgt)
        m = omodel(oracle, tr)
        want_out = oracle.forward(m, hw, mw, pos)
        params = np.concatenate([hw, mw])
        m1, m2 = np.zeros_like(params), np.zeros_like(params)
        lo = oracle.training_step(m, oracle.adam(LR, LR, BETA1, BETA2), 0, params, m1, m2, pos, tgt)
        nh, nm = tr.hash_param_count, tr.mlp_param_count
        assert rel_tensor(out, want_out) <= 2e-3
        assert res["loss"] == pytest.approx(lo, rel=2e-3)
        mh, vh, mm, vm = parse_optimizer_blob(tr.export_optimizer_state().payload, nh, nm)
        hw1, mw1 = tr.get_weights()
        assert rel_tensor(mm, m1[nh:]) <= 2e-3
        assert rel_tensor(vm, m2[nh:]) <= 2e-3
        g = m1 / (1.0 - BETA1)  # the oracle's gradients (first step: m = (1 - beta1) g)
        gh_max = float(np.abs(g[:nh]).max())
        delta = 2e-3 * gh_max + G_ULP  # per-entry hash gradient bound
        dm = np.abs(mh.astype(np.float64) - m1[:nh])
        dv = np.abs(vh.astype(np.float64) - m2[:nh])
        _say(f"  hash m: max|diff| {dm.max() / (1 - BETA1) * 65536:.2f} units of 2^-16 "
             f"(largest gradient {gh_max * 65536:.1f} units), exact on {(dm == 0).mean():.6f}")
        assert dm.max() <= (1 - BETA1) * delta * 1.01
        assert dv.max() <= (1 - BETA2) * delta * (2 * gh_max + delta) * 1.01
        _update_check(mw1, mw, g[nh:], LR, "mlp")
        _update_check(hw1, hw, g[:nh], LR, "hash", G_ULP)
        touched_gpu, touched_orc = mh != 0, m1[:nh] != 0
        differ = touched_gpu != touched_orc
        tiny = np.maximum(np.abs(mh), np.abs(m1[:nh])) <= (1 - BETA1) * delta * 1.01
        assert not (differ & ~tiny).any()
        _say(f"  touched sets agree on {1.0 - differ.mean():.6f} of {nh} entries")
        assert 1.0 - differ.mean() >= 0.999
        # untouched entries keep their weights bit for bit (lazy hash Adam)
        keep = ~touched_gpu & ~touched_orc
        assert np.array_equal(hw1[keep], hw[keep])
        # numerics report of the step (step 1 is sampled)
        nr = res["numerics"]
        assert res["numerics_reported"] and not res["has_numerics_anomaly"]
        assert nr["finite_forward"] and nr["finite_backward"] and nr["finite_update"]
        assert nr["max_abs_activation"] == np.abs(out).max()
        du = np.abs(np.concatenate([hw, mw]) - np.concatenate([hw1, mw1]))
        assert nr["max_abs_update"] == du.max()
        # the report's gradient terms are those of the gradients the step
        # applied, which its first moments hold (m = (1 - beta1) g on step 1)
        g_gpu = np.concatenate([mh, mm]).astype(np.float64) / (1.0 - BETA1)
        assert nr["max_abs_gradient"] == pytest.approx(np.abs(g_gpu).max(), rel=1e-5)
        assert res["grad_norm"] == pytest.approx(np.sqrt((g_gpu ** 2).sum()), rel=1e-4)


def test_c5_step_at_baseline_geometry(oracle):
    """C5 at its real shape: 4D, 16 levels x 2
    features, T = 2^22 (32 MB per level: level-major encode and scatter),
    base 8, scale 1.4, MLP 32 -> 128^4 -> 4 in fp16 (wide_train_kernel<4>),
    L2. The backward (split path, the training kernel in external-gradient
    mode) within 2e-3 of the oracle with the visited set exact, then the loss
    of each fused step within 1% over four steps."""
    d, enc, net, m_out, loss = BASELINE["c5"]
    n = 4096
    _say("c5 geometry step")
    rng = np.random.default_rng(41)
    with make_trainer(d, m_out, enc, net, loss=loss, precision="fp16", batch=n) as tr:
        assert tr.hash_param_count == 16 * 2 * (1 << 22)
        hw, mw = tr.get_weights()
        m = omodel(oracle, tr)
        pos = away_from_relu_kinks(oracle, tr, hw, mw, rng.random((n, d), dtype=np.float32))
        assert len(pos) > 0.9 * n
        gout = rng.normal(0, 1.0, (len(pos), m_out)).astype(np.float32)
        tr.zero_gradients()
        tr.backward_accumulate(pos, gout)
        gh, gm = tr.debug_gradients()
        mask = tr.debug_active_mask()
        ogh, ogm, omask, _, _ = oracle.forward_backward(m, hw, mw, pos, d_out=gout)
        assert np.array_equal(mask, omask)
        assert rel_tensor(gm, ogm) <= 2e-3
        assert rel_tensor(gh, ogh) <= 2e-3
        del gh, ogh
        tr.zero_gradients()
        params = np.concatenate([hw, mw])
        m1, m2 = np.zeros_like(params), np.zeros_like(params)
        a = oracle.adam(LR, LR, BETA1, BETA2)
        freq = rng.normal(0, 3.0, (16, 4)).astype(np.float32)
        phase = rng.uniform(0, 6.28, (16, 4)).astype(np.float32)
        for step in range(4):
            p = rng.random((n, d), dtype=np.float32)
            t = np.stack([np.sin(p @ freq[4 * k:4 * k + 4].T + phase[4 * k:4 * k + 4, 0]).sum(1)
                          for k in range(m_out)], 1).astype(np.float32) * 0.25
            lg = tr.training_step(p, t)
            lo = oracle.training_step(m, a, step, params, m1, m2, p, t)
            _say(f"  step {step}: gpu {lg:.6f} oracle {lo:.6f}")
            assert lg == pytest.approx(lo, rel=0.01), (step, lg, lo)


# ------------------------------------------------------------- numerics --

def test_numerics_report_flags_a_nan_batch():
    """A batch with one NaN target: the loss is not finite, so the step is
    reported even with sampling disabled (the reference's forced probe), with
    the forward, backward (NaN MLP gradients) and update non-finite; the next
    step is sampled because the previous one was anomalous."""
    _say("numerics nan")
    d, enc, net, m_out, _ = BASELINE["c2"]
    rng = np.random.default_rng(3)
    n = 4096
    with make_trainer(d, m_out, enc, net, precision="fp16", batch=n) as tr:
        tr.set_numerics_sampling("Disabled")
        pos = rng.random((n, d), dtype=np.float32)
        tgt = rng.random((n, m_out), dtype=np.float32)
        r = tr.training_step_result(pos, tgt)
        assert np.isfinite(r["loss"]) and not r["numerics_reported"]
        bad = tgt.copy()
        bad[17, 1] = np.nan
        r = tr.training_step_result(pos, bad)
        assert not np.isfinite(r["loss"])
        assert r["numerics_reported"] and r["has_numerics_anomaly"]
        nr = r["numerics"]
        assert not nr["finite_forward"] and not nr["finite_backward"] and not nr["finite_update"]
    # L1 against an infinite target: the loss is infinite but the gradients
    # (sign / N) stay finite, so the weights do too and only that step is
    # anomalous
    with make_trainer(d, m_out, enc, net, loss="L1", precision="fp32", batch=n) as tr:
        tr.set_numerics_sampling("Sampled", 1000)
        steps = []
        for k in range(4):
            t = tgt.copy()
            if k == 1:
                t[3, 0] = np.inf
            steps.append(tr.training_step_result(pos, t))
        # step 1 (bootstrap), step 2 (forced: infinite loss), step 3 (after an
        # anomaly), step 4 not sampled
        assert [s["numerics_reported"] for s in steps] == [True, True, True, False]
        assert steps[0]["numerics"]["finite_forward"] and not steps[0]["has_numerics_anomaly"]
        nr = steps[1]["numerics"]
        assert steps[1]["has_numerics_anomaly"] and not nr["finite_forward"]
        assert nr["finite_backward"] and nr["finite_update"]
        assert not steps[2]["has_numerics_anomaly"] and np.isfinite(steps[3]["loss"])


@pytest.mark.parametrize("mode,interval,want", [
    ("Sampled", 4, [1, 4, 8]), ("Periodic", 3, [3, 6, 9]),
    ("FullPerStep", 1, list(range(1, 10))), ("Disabled", 1, [])])
def test_numerics_sampling_policy(mode, interval, want):
    """NumericsGuard::should_sample (numerics_guard.cpp:12-36) on the step
    counter after the update, for clean batches: which of steps 1..9 carry a
    report; every report is finite with positive gradient and update terms."""
    _say(f"numerics policy {mode}")
    d, enc, net, m_out, _ = BASELINE["c2"]
    rng = np.random.default_rng(5)
    n = 2048
    with make_trainer(d, m_out, enc, net, precision="fp16", batch=n) as tr:
        tr.set_numerics_sampling(mode, interval)
        got = []
        for _ in range(9):
            r = tr.training_step_result(rng.random((n, d), dtype=np.float32),
                                        rng.random((n, m_out), dtype=np.float32))
            if r["numerics_reported"]:
                got.append(r["step"])
                nr = r["numerics"]
                assert nr["finite_forward"] and nr["finite_backward"] and nr["finite_update"]
                assert nr["max_abs_gradient"] > 0 and nr["max_abs_update"] > 0
                assert r["grad_norm"] >= nr["max_abs_gradient"]
        assert got == want


def test_device_step_numerics_read_on_demand():
    """Device steps compute the report on their sampled steps and read
    nothing back; last_numerics returns the last such step's report, with its
    loss equal to the loss the step wrote to device memory."""
    torch = pytest.importorskip("torch")
    _say("numerics device")
    d, enc, net, m_out, _ = BASELINE["c2"]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(9)
    n = 8192
    with make_trainer(d, m_out, enc, net, precision="fp16", batch=n) as tr:
        assert tr.last_numerics()["numerics_reported"] is False
        tr.set_numerics_sampling("Sampled", 2)
        losses = torch.zeros(3, device=dev)
        for k in range(3):
            x = torch.rand(n, d, device=dev, generator=g)
            y = torch.rand(n, m_out, device=dev, generator=g)
            torch.cuda.synchronize()
            tr.training_step_device(x.data_ptr(), y.data_ptr(), n, losses[k].data_ptr())
        r = tr.last_numerics()  # steps 1 and 2 are sampled: the report is step 2's
        assert r["numerics_reported"] and r["step"] == 2 and r["batch_n"] == n
        assert r["loss"] == losses[1].item()
        assert r["numerics"]["finite_backward"] and r["numerics"]["max_abs_update"] > 0


# ------------------------------------------- device steps after an event --

def test_device_calls_ordered_after_a_producer_stream():
    """Inputs written by a torch stream that is still busy when the library
    is called: training_step_device_after / inference_device_after wait for
    the producer's event on every stream that reads the batch (the sort's and
    the step's), and record_event hands the results to a consumer stream; no
    host synchronization in between. Losses, weights and inference outputs
    are bit-identical to a trainer fed host-synchronized copies."""
    torch = pytest.importorskip("torch")
    _say("device after event")
    d, enc, net, m_out, _ = BASELINE["c2"]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(13)
    n = 1 << 16
    producer, consumer = torch.cuda.Stream(), torch.cuda.Stream()
    with make_trainer(d, m_out, enc, net, precision="fp16", batch=n) as ref, \
            make_trainer(d, m_out, enc, net, precision="fp16", batch=n) as tr:
        for k in range(3):
            bx = torch.rand(n, d, device=dev, generator=g)
            by = torch.rand(n, m_out, device=dev, generator=g)
            torch.cuda.synchronize()
            loss_ref = torch.zeros(1, device=dev)
            ref.training_step_device(bx.data_ptr(), by.data_ptr(), n, loss_ref.data_ptr())
            ref.synchronize()
            with torch.cuda.stream(producer):
                # a long chain of exact identities: the copy is complete only
                # when the whole chain has run
                x, y = bx.clone(), by.clone()
                for _ in range(200):
                    x = x * 1.0
                    y = y + 0.0
                ready = torch.cuda.Event()
                ready.record(producer)
            loss = torch.zeros(1, device=dev)
            tr.training_step_device_after(x.data_ptr(), y.data_ptr(), n, ready, loss.data_ptr())
            done = torch.cuda.Event()
            done.record(consumer)  # creates the event; re-recorded on the trainer's stream
            tr.record_event(done)
            with torch.cuda.stream(consumer):
                consumer.wait_event(done)
                got = loss.clone()
            torch.cuda.synchronize()
            assert got.item() == loss_ref.item(), k
            hr, mr = ref.get_weights()
            ht, mt = tr.get_weights()
            assert np.array_equal(mr, mt) and np.array_equal(hr, ht), k
        q = torch.rand(n, d, device=dev, generator=g)
        torch.cuda.synchronize()
        want = ref.inference(q.cpu().numpy())
        with torch.cuda.stream(producer):
            qq = q.clone()
            for _ in range(200):
                qq = qq * 1.0
            ready = torch.cuda.Event()
            ready.record(producer)
        out = torch.empty(n, m_out, device=dev)
        tr.inference_device_after(qq.data_ptr(), out.data_ptr(), n, ready)
        done = torch.cuda.Event()
        done.record(consumer)
        tr.record_event(done)
        with torch.cuda.stream(consumer):
            consumer.wait_event(done)
            res = out.clone()
        torch.cuda.synchronize()
        assert np.array_equal(res.cpu().numpy(), want)
