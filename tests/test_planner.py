"""Network planner (plan_network, network_planning.h:160-190;
network_planner.cpp:132-300) on nominal MI355X capabilities: no GPU needed.

Family eligibility comes from the kernels the library instantiates and
their LDS plans against the capabilities; the reasons use the reference's
PlannerFallbackReason names."""
from __future__ import annotations

import copy
import sys
from pathlib import Path

import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "tiny-metal-nn_amd"))

from tiny_metal_nn import ConfigError, plan_network  # noqa: E402

C2 = {"encoding": {"otype": "HashGrid", "n_levels": 16, "n_features_per_level": 2,
                   "log2_hashmap_size": 15, "base_resolution": 16.0, "per_level_scale": 1.5},
      "network": {"otype": "FullyFusedMLP", "n_neurons": 64, "n_hidden_layers": 2},
      "loss": {"otype": "RelativeL2"},
      "mi355x": {"precision": "fp16"}}


def cfg(**kw):
    c = copy.deepcopy(C2)
    for path, v in kw.items():
        sec, key = path.split("__")
        c[sec][key] = v
    return c


def test_image_fit_is_fully_fused():
    p = plan_network(C2, 2, 3)
    assert p["selected_family"] == "FullyFused"
    assert p["fused_train"] and p["fused_eval"]
    assert p["candidate_families"] == ["FullyFused", "Tiled", "SafeDebug"]
    assert p["reasons"] == []
    assert p["train_waves_per_block"] == 8          # mlp_train_kernel: 2 waves per SIMD
    assert 0 < p["train_lds_bytes"] <= 160 * 1024


def test_sdf_shape_runs_four_waves():
    # 16x4 features into 64x3: the weight image leaves LDS for four waves' parking
    c = cfg(encoding__n_features_per_level=4, network__n_hidden_layers=3)
    p = plan_network(c, 3, 1)
    assert p["selected_family"] == "FullyFused" and p["fused_train"]
    assert p["train_waves_per_block"] == 4
    assert 0 < p["train_lds_bytes"] <= 160 * 1024


def test_unspecialised_depth_falls_back_to_tiled():
    p = plan_network(cfg(network__n_hidden_layers=4), 2, 3)
    assert p["selected_family"] == "Tiled"
    assert not p["fused_train"]
    assert "NoFusedInstance" in p["reasons"]
    assert "FullyFused" not in p["candidate_families"]


def test_narrow_hidden_is_tiled():
    p = plan_network(cfg(network__n_neurons=32), 2, 3)
    assert p["selected_family"] == "Tiled" and "NoFusedInstance" in p["reasons"]


@pytest.mark.parametrize("family,reason", [("Tiled", "ForcedTiled"), ("SafeDebug", "ForcedSafeDebug")])
def test_forced_family(family, reason):
    p = plan_network(cfg(mi355x__family=family), 2, 3)
    assert p["selected_family"] == family
    assert reason in p["reasons"]
    assert not p["fused_train"] and not p["fused_eval"]


def test_forced_fully_fused_is_the_default_choice():
    assert plan_network(cfg(mi355x__family="FullyFused"), 2, 3)["selected_family"] == "FullyFused"


def test_lds_limit_moves_to_tiled():
    p = plan_network(C2, 2, 3, {"lds_bytes_per_cu": 64 * 1024})
    assert p["selected_family"] == "Tiled"
    assert "ThreadgroupMemoryExceeded" in p["reasons"]
    assert p["train_lds_bytes"] <= 64 * 1024


def test_no_gpu_context():
    p = plan_network(C2, 2, 3, {"gpu_available": 0})
    assert p["selected_family"] is None and p["reasons"] == ["NoGPUContext"]


def test_width_128_fused_or_layerwise_tiled():
    """Width 128: the instantiated fp16 shapes run fully fused; Tiled (forced,
    or for fp32 whose operands exceed one CU's LDS) runs the layer-wise path."""
    c = cfg(network__n_neurons=128, network__n_hidden_layers=4,
            encoding__base_resolution=8.0, encoding__per_level_scale=1.4)
    assert plan_network(c, 4, 4)["selected_family"] == "FullyFused"
    p = plan_network(copy.deepcopy(c) | {"mi355x": {"precision": "fp16", "family": "Tiled"}}, 4, 4)
    assert p["selected_family"] == "Tiled" and "ForcedTiled" in p["reasons"]
    p = plan_network(copy.deepcopy(c) | {"mi355x": {"precision": "fp32"}}, 4, 4)
    assert p["selected_family"] == "Tiled" and not p["fused_train"]
    assert "ThreadgroupMemoryExceeded" in p["reasons"]


@pytest.mark.parametrize("n_in,neurons,layers,levels,feats,n_out,reason", [
    (3, 256, 2, 16, 2, 1, "HiddenDimUnsupported"),
    (3, 512, 8, 16, 2, 4, "HiddenDimUnsupported"),
    (2, 64, 2, 32, 4, 3, "NoFusedInstance"),      # 128 input features
    (3, 64, 2, 16, 2, 32, "UnsupportedOutputDims"),
    (3, 128, 2, 16, 4, 2, "NoFusedInstance"),     # width 128 with 64 input features
])
def test_every_kernel_spec_shape_has_a_tiled_plan(n_in, neurons, layers, levels, feats, n_out,
                                                  reason):
    """KernelSpec bounds (kernel_spec.cpp:12-44: hidden <= 512, <= 8 layers,
    <= 32 levels x <= 4 features, any outputs): shapes no fused kernel holds
    fall back to Tiled (the layer-wise path) with the reason recorded."""
    c = cfg(network__n_neurons=neurons, network__n_hidden_layers=layers, encoding__n_levels=levels,
            encoding__n_features_per_level=feats)
    p = plan_network(c, n_in, n_out)
    assert p["selected_family"] == "Tiled" and not p["fused_train"]
    assert reason in p["reasons"]
    assert "Tiled" in p["candidate_families"] and "SafeDebug" in p["candidate_families"]


def test_fingerprint_tracks_the_shape():
    a = plan_network(C2, 2, 3)["planner_fingerprint"]
    assert a == plan_network(copy.deepcopy(C2), 2, 3)["planner_fingerprint"]
    assert a != plan_network(cfg(network__n_hidden_layers=1), 2, 3)["planner_fingerprint"]
    assert a != plan_network(cfg(mi355x__precision="fp32"), 2, 3)["planner_fingerprint"]


def test_unknown_family_is_a_config_error():
    with pytest.raises(ConfigError):
        plan_network(cfg(mi355x__family="Scalar"), 2, 3)
