"""C-ABI library checks that need no GPU: the library loads, exports every
symbol include/tmnn_hip.h declares, and the struct layouts agree; JSON config
canonicalization follows the reference's rules (factory_json_detail.h)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "tmnn_hip.h"


def declared_symbols() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(tmnn_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for must in ("tmnn_training_step", "tmnn_inference", "tmnn_forward_for_training",
                 "tmnn_zero_gradients", "tmnn_backward_accumulate", "tmnn_adam_step",
                 "tmnn_export_optimizer_state", "tmnn_import_optimizer_state",
                 "tmnn_set_initial_weights", "tmnn_get_weights", "tmnn_last_error"):
        assert must in syms


def test_library_exports_every_declared_symbol():
    from tiny_metal_nn import _lib
    lib = _lib.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert set(declared_symbols()) == set(_lib.SIGNATURES)
    assert lib.tmnn_abi_version() == 3


def test_desc_defaults_and_struct_size():
    from tiny_metal_nn import _lib
    d = _lib.ModelDesc()
    _lib.load().tmnn_model_desc_init(ctypes.byref(d))
    assert d.struct_size == ctypes.sizeof(_lib.ModelDesc)
    # HashGridEncoding / FullyFusedMLP / TrainerConfig / WeightInitConfig defaults
    assert (d.num_levels, d.features_per_level, d.log2_hashmap_size) == (16, 2, 19)
    assert d.base_resolution == 16.0 and d.per_level_scale == pytest.approx(1.447)
    assert (d.hidden_dim, d.num_hidden_layers, d.batch_size) == (64, 2, 1024)
    assert d.lr_encoding == pytest.approx(1e-2) and d.lr_network == pytest.approx(1e-3)
    assert d.beta1 == pytest.approx(0.9) and d.beta2 == pytest.approx(0.99)
    assert d.epsilon == pytest.approx(1e-15) and d.seed == 42
    assert d.hash_init_range == pytest.approx(1e-4)


def test_null_handles_are_rejected_without_a_gpu():
    from tiny_metal_nn import _lib
    lib = _lib.load()
    assert lib.tmnn_training_step(None, None, None, 4, None) == _lib.TMNN_ERR_INVALID_ARGUMENT
    assert b"null" in lib.tmnn_last_error()
    assert lib.tmnn_adam_step(None) == _lib.TMNN_ERR_INVALID_ARGUMENT
    assert lib.tmnn_trainer_destroy(None) == 0


def test_canonicalize_defaults():
    from tiny_metal_nn import canonicalize_model_config
    c = canonicalize_model_config(3, 1, {})
    assert c["encoding"] == {"otype": "HashGrid", "n_input_dims": 3, "n_levels": 16,
                             "n_features_per_level": 2, "log2_hashmap_size": 19,
                             "base_resolution": 16.0, "per_level_scale": 1.447,
                             "interpolation": "Linear"}
    assert c["network"]["n_neurons"] == 64 and c["network"]["n_hidden_layers"] == 2
    assert c["network"]["n_input_dims"] == 32
    assert c["loss"] == {"otype": "L2"}
    assert c["optimizer"]["learning_rate"] == pytest.approx(1e-3)
    assert c["batch_size"] == 1024


@pytest.mark.parametrize("bad,frag", [
    ({"network": {"otype": "TiledMLP"}}, "TiledMLP"),
    ({"network": {"activation": "Tanh"}}, "ReLU"),
    ({"loss": {"otype": "MSE"}}, "unsupported loss"),
    ({"loss": {"otype": "Huber", "huber_delta": -1.0}}, "huber_delta"),
    ({"loss": {"otype": "Cosine", "output_dims": 1}}, "output_dims"),
    ({"optimizer": {"otype": "SGD"}}, "optimizer"),
    ({"optimizer": {"learning_rate": 0.0}}, "learning_rate"),
    ({"encoding": {"interpolation": "Nearest"}}, "Linear"),
    ({"encoding": {"n_levels": "many"}}, "n_levels"),
    ({"bogus": 1}, "bogus"),
    ({"mi355x": {"weight_decay": -1.0}}, "weight_decay"),
    ({"mi355x": {"grad_clip": -0.5}}, "grad_clip"),
])
def test_canonicalize_rejects(bad, frag):
    from tiny_metal_nn import ConfigError, canonicalize_model_config
    with pytest.raises(ConfigError, match=frag):
        canonicalize_model_config(3, 1, bad)


def test_canonicalize_aliases_and_extensions():
    from tiny_metal_nn import canonicalize_model_config
    c = canonicalize_model_config(2, 3, {
        "encoding": {"otype": "MultiresolutionHashGrid", "n_levels": 16},
        "network": {"output_activation": "Linear"},
        "loss": {"otype": "RelativeL2"},
        "mi355x": {"precision": "fp16"}})
    assert c["encoding"]["otype"] == "HashGrid"
    assert c["network"]["output_activation"] == "None"
    assert c["loss"]["otype"] == "RelativeL2"
    assert c["mi355x"]["precision"] == "fp16"


def test_model_desc_from_config():
    from tiny_metal_nn import _lib, canonicalize_model_config
    from tiny_metal_nn.config import model_desc
    c = canonicalize_model_config(2, 3, {
        "encoding": {"n_levels": 16, "log2_hashmap_size": 15, "per_level_scale": 1.5},
        "optimizer": {"learning_rate": 1e-2, "beta2": 0.99, "epsilon": 1e-15},
        "loss": {"otype": "RelativeL2"}, "batch_size": 262144,
        "mi355x": {"precision": "fp16", "hash_adam": "dense"}})
    d = model_desc(c)
    assert (d.spatial_dims, d.num_outputs, d.log2_hashmap_size) == (2, 3, 15)
    assert d.lr_encoding == pytest.approx(1e-2) and d.lr_network == pytest.approx(1e-2)
    assert d.loss_kind == _lib.LOSS_RELATIVE_L2 and d.batch_size == 262144
    assert d.precision == _lib.PRECISION_FP16 and d.hash_adam_mode == _lib.HASH_ADAM_DENSE
    c = canonicalize_model_config(3, 1, {"optimizer": {"l1_reg": 1e-4, "l2_reg": 1e-3},
                                         "mi355x": {"grad_clip": 0.5, "weight_decay": 0.01}})
    d = model_desc(c)
    assert d.l1_reg == pytest.approx(1e-4) and d.l2_reg == pytest.approx(1e-3)
    assert d.grad_clip == pytest.approx(0.5) and d.weight_decay == pytest.approx(0.01)


def test_struct_layouts_match_the_header(tmp_path):
    """Every descriptor struct of include/tmnn_hip.h has the size and field
    offsets the ctypes binding assumes (compiled with the host C compiler)."""
    import shutil
    import subprocess
    from tiny_metal_nn import _lib
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no host C compiler")
    structs = {"tmnn_model_desc": _lib.ModelDesc, "tmnn_device_caps": _lib.DeviceCaps,
               "tmnn_network_plan": _lib.NetworkPlan, "tmnn_step_result": _lib.StepResult,
               "tmnn_numerics_report": _lib.NumericsReport,
               "tmnn_inspection": _lib.Inspection, "tmnn_step_profile": _lib.StepProfile,
               "tmnn_buffer_view": _lib.BufferView, "tmnn_parameter_layout_t": _lib.ParameterLayout,
               "tmnn_batch_plan_t": _lib.BatchPlan, "tmnn_storage_policy_t": _lib.StoragePolicy}
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "tmnn_hip.h"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'printf("{cname}.{field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run([cc, "-I", str(HEADER.parent), str(src), "-o", str(exe)], check=True)
    got = dict(l.rsplit(" ", 1) for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                         check=True).stdout.splitlines())
    for cname, cls in structs.items():
        assert int(got[cname]) == ctypes.sizeof(cls), cname
        for field, _ in cls._fields_:
            assert int(got[f"{cname}.{field}"]) == getattr(cls, field).offset, (cname, field)


def test_call_guard_releases_and_rejects_concurrent_entry():
    """The single-caller guard (tmnn_pybind.cpp:366-375) is released after each
    call and a second entry while held raises instead of blocking."""
    import threading

    from tiny_metal_nn import ConcurrentTrainingStepError, Trainer
    tr = object.__new__(Trainer)
    tr._busy = threading.Lock()
    tr._closed = False
    for _ in range(3):
        with tr._enter("training_step"):
            with pytest.raises(ConcurrentTrainingStepError):
                with tr._enter("inference"):
                    pass
    assert not tr._busy.locked()
    with pytest.raises(RuntimeError):
        with tr._enter("training_step"):
            raise RuntimeError("boom")
    assert not tr._busy.locked()
    tr._closed = True
