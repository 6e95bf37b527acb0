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


def test_width_128_only_fully_fused():
    c = cfg(network__n_neurons=128, network__n_hidden_layers=4,
            encoding__base_resolution=8.0, encoding__per_level_scale=1.4)
    assert plan_network(c, 4, 4)["selected_family"] == "FullyFused"
    p = plan_network(copy.deepcopy(c) | {"mi355x": {"precision": "fp16", "family": "Tiled"}}, 4, 4)
    assert p["selected_family"] is None and "HiddenDimUnsupported" in p["reasons"]
    p = plan_network(copy.deepcopy(c) | {"mi355x": {"precision": "fp32"}}, 4, 4)
    assert p["selected_family"] is None and "HiddenDimUnsupported" in p["reasons"]


def test_fingerprint_tracks_the_shape():
    a = plan_network(C2, 2, 3)["planner_fingerprint"]
    assert a == plan_network(copy.deepcopy(C2), 2, 3)["planner_fingerprint"]
    assert a != plan_network(cfg(network__n_hidden_layers=1), 2, 3)["planner_fingerprint"]
    assert a != plan_network(cfg(mi355x__precision="fp32"), 2, 3)["planner_fingerprint"]


def test_unknown_family_is_a_config_error():
    with pytest.raises(ConfigError):
        plan_network(cfg(mi355x__family="Scalar"), 2, 3)
