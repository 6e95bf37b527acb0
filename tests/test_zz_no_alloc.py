"""The allocation-free training step (tmnn_training_step_device_noalloc)
against the existing device entry point (tmnn_training_step_device) through
the C-ABI: two trainers from the same seed take the same batches, one
through each entry point, two calls in a row (the second with a smaller
batch); losses and every parameter are bit-identical (the kernels and their
order are the same), except for the Tiled family's generic kernel, whose
LDS weight-gradient accumulator adds with atomics in arrival order (loss and
weights within 1e-6 there). A second case alternates the two entry points on
one trainer, which also meets the regular step's side-stream sort sets.
Marked gpu."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from test_gpu_parity import GEOMS, make_trainer, rel_tensor

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


CASES = {
    # name: (geometry, precision, family, batch sizes of the two calls)
    "c2_fp16": ("2d_f2", "fp16", "auto", (1 << 18, 5000)),
    "3d_fp32": ("3d_f2", "fp32", "auto", (20000, 777)),
    "3d_f4_fp16": ("3d_f4", "fp16", "auto", (9000, 4100)),
    "2d_tiled": ("2d_f2", "fp16", "Tiled", (6000, 3001)),
}


@pytest.mark.parametrize("case", list(CASES))
def test_noalloc_step_matches_device_step(case):
    torch = pytest.importorskip("torch")
    name, precision, family, sizes = CASES[case]
    d, enc, net, m_out = GEOMS[name]
    _say(f"noalloc {case}")
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(5)
    batch = max(sizes)
    with make_trainer(d, m_out, enc, net, precision=precision, family=family, batch=batch,
                      hash_range=0.1) as ref, \
            make_trainer(d, m_out, enc, net, precision=precision, family=family, batch=batch,
                         hash_range=0.1) as tr:
        loss_ref = torch.zeros(len(sizes), device=dev)
        loss_na = torch.zeros(len(sizes), device=dev)
        for i, n in enumerate(sizes):
            x = torch.rand(n, d, device=dev, generator=g)
            y = torch.rand(n, m_out, device=dev, generator=g)
            torch.cuda.synchronize()
            ref.training_step_device(x.data_ptr(), y.data_ptr(), n, loss_ref[i].data_ptr())
            tr.training_step_device_noalloc(x.data_ptr(), y.data_ptr(), n, loss_na[i].data_ptr())
            ref.synchronize()
            tr.synchronize()
            a, b = loss_ref[i].item(), loss_na[i].item()
            hr, mr = ref.get_weights()
            hn, mn = tr.get_weights()
            if family == "Tiled":  # order-dependent LDS atomics in the dW accumulator
                assert np.isfinite(a) and b == pytest.approx(a, rel=1e-6, abs=0.0), (i, a, b)
                assert rel_tensor(mn, mr) <= 1e-6 and rel_tensor(hn, hr) <= 1e-6, i
            else:
                assert np.isfinite(a) and a == b, (i, a, b)
                assert np.array_equal(mn, mr) and np.array_equal(hn, hr), (
                    i, rel_tensor(mn, mr), rel_tensor(hn, hr))
            assert tr.step() == ref.step() == i + 1
            _say(f"  call {i} n={n}: loss {a:.6f} / {b:.6f}, weights bit-identical "
                 f"{np.array_equal(mn, mr) and np.array_equal(hn, hr)}")


def test_noalloc_alternating_with_regular_steps_on_one_trainer():
    """Regular, allocation-free, regular, allocation-free steps on one trainer
    (the regular steps sort on the side stream into their buffer sets, the
    allocation-free ones on the main stream into the scratch, lending and
    restoring the trainer's batch buffers) against a trainer that takes only
    regular steps: losses and weights bit-identical after every step."""
    torch = pytest.importorskip("torch")
    d, enc, net, m_out = GEOMS["2d_f2"]
    _say("noalloc alternating")
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(21)
    sizes = (20000, 8192, 20000, 3001, 12345, 20000)
    with make_trainer(d, m_out, enc, net, precision="fp16", batch=20000, hash_range=0.1) as ref, \
            make_trainer(d, m_out, enc, net, precision="fp16", batch=20000, hash_range=0.1) as tr:
        for i, n in enumerate(sizes):
            x = torch.rand(n, d, device=dev, generator=g)
            y = torch.rand(n, m_out, device=dev, generator=g)
            lr_, lt = torch.zeros(1, device=dev), torch.zeros(1, device=dev)
            torch.cuda.synchronize()
            ref.training_step_device(x.data_ptr(), y.data_ptr(), n, lr_.data_ptr())
            if i % 2:
                tr.training_step_device_noalloc(x.data_ptr(), y.data_ptr(), n, lt.data_ptr())
            else:
                tr.training_step_device(x.data_ptr(), y.data_ptr(), n, lt.data_ptr())
            ref.synchronize()
            tr.synchronize()
            assert lr_.item() == lt.item(), (i, lr_.item(), lt.item())
            hr, mr = ref.get_weights()
            hn, mn = tr.get_weights()
            assert np.array_equal(mn, mr) and np.array_equal(hn, hr), i
            _say(f"  step {i} n={n} {'noalloc' if i % 2 else 'regular'}: bit-identical")


def test_noalloc_rejects_oversize_and_wide_without_running():
    """A batch above the scratch and a width-128 model are refused with an
    error before anything is enqueued; the trainer keeps working."""
    torch = pytest.importorskip("torch")
    from tiny_metal_nn._lib import TmnnError
    _say("noalloc limits")
    dev = torch.device("cuda:0")
    d, enc, net, m_out = GEOMS["2d_f2"]
    n = 1 << 19  # ~149 MB of scratch at this shape
    with make_trainer(d, m_out, enc, net, precision="fp16", batch=n) as tr:
        x = torch.rand(n, d, device=dev)
        y = torch.rand(n, m_out, device=dev)
        with pytest.raises(ValueError, match="scratch"):
            tr.training_step_device_noalloc(x.data_ptr(), y.data_ptr(), n)
        assert tr.step() == 0
        tr.training_step_device_noalloc(x.data_ptr(), y.data_ptr(), 4096)
        tr.synchronize()
        assert tr.step() == 1
    wenc = dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=14, base_resolution=16.0,
                per_level_scale=1.5)
    with make_trainer(3, 2, wenc, dict(n_neurons=128, n_hidden_layers=2), precision="fp16",
                      batch=4096) as tr:
        x = torch.rand(4096, 3, device=dev)
        y = torch.rand(4096, 2, device=dev)
        with pytest.raises(TmnnError, match="width 128"):
            tr.training_step_device_noalloc(x.data_ptr(), y.data_ptr(), 4096)
