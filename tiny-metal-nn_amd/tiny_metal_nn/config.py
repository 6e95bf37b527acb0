"""JSON-shaped config -> canonical config -> C-ABI model descriptor.

Mirrors the reference's canonicalization (include/tiny-metal-nn/detail/
factory_json_detail.h): the same keys, defaults and rejections for the
"encoding" (:159-219), "network" (:221-290), "loss" (:367-406), "optimizer"
(:408-462) and "weight_init" (:542-624) sections and "batch_size". Two
additions: loss otype "RelativeL2" (absent from the reference, which accepts
only L2/L1/Huber/Cosine) and an optional "mi355x" section for this build's
runtime choices (precision, hash-Adam mode, Morton sort, gradient clip).
"""
from __future__ import annotations

import copy
from typing import Any

from . import _lib


class ConfigError(ValueError):
    """A config field failed validation (the reference's ConfigError)."""


_TOP_KEYS = {"encoding", "network", "loss", "optimizer", "weight_init", "batch_size",
             "training", "mi355x"}


def _known(cfg: dict, keys: set, where: str, errors: list) -> None:
    for k in cfg:
        if k not in keys:
            errors.append(f"{where}.{k}: unknown key")


def _get(cfg: dict, key: str, default, kind, where: str, errors: list):
    if key not in cfg:
        return default
    v = cfg[key]
    try:
        if kind is int:
            if isinstance(v, bool) or (isinstance(v, float) and not v.is_integer()):
                raise TypeError
            return int(v)
        if kind is float:
            if isinstance(v, bool):
                raise TypeError
            return float(v)
        if kind is str:
            if not isinstance(v, str):
                raise TypeError
            return v
        if kind is bool:
            if not isinstance(v, bool):
                raise TypeError
            return v
    except (TypeError, ValueError):
        errors.append(f"{where}.{key}: expected {kind.__name__}")
        return default
    return v


def _pos(v, path, errors):
    if not (v > 0):
        errors.append(f"{path}: must be > 0")


def canonicalize_model_config(n_input: int, n_output: int, config: dict) -> dict:
    """Canonical copy of `config` with every default filled in.

    Raises ConfigError listing every error found (factory_json.h:21-37).
    """
    if not isinstance(config, dict):
        raise ConfigError("config must be a dict")
    errors: list[str] = []
    _known(config, _TOP_KEYS, "config", errors)
    if n_input < 1:
        errors.append("n_input: must be >= 1")
    if n_output < 1:
        errors.append("n_output: must be >= 1")

    enc = config.get("encoding", {}) or {}
    _known(enc, {"otype", "n_levels", "n_features_per_level", "log2_hashmap_size",
                 "base_resolution", "per_level_scale", "interpolation"}, "encoding", errors)
    otype = _get(enc, "otype", "HashGrid", str, "encoding", errors)
    if otype in ("RotatedMHE", "RotatedMultiresHashGrid"):
        errors.append("encoding.otype: RotatedMHE is not built in this library")
    elif otype not in ("HashGrid", "MultiresolutionHashGrid"):
        errors.append(f"encoding.otype: unsupported encoding otype '{otype}'")
    e = {
        "otype": "HashGrid",
        "n_input_dims": n_input,
        "n_levels": _get(enc, "n_levels", 16, int, "encoding", errors),
        "n_features_per_level": _get(enc, "n_features_per_level", 2, int, "encoding", errors),
        "log2_hashmap_size": _get(enc, "log2_hashmap_size", 19, int, "encoding", errors),
        "base_resolution": _get(enc, "base_resolution", 16.0, float, "encoding", errors),
        "per_level_scale": _get(enc, "per_level_scale", 1.447, float, "encoding", errors),
        "interpolation": _get(enc, "interpolation", "Linear", str, "encoding", errors),
    }
    for k in ("n_levels", "n_features_per_level", "log2_hashmap_size", "base_resolution",
              "per_level_scale"):
        _pos(e[k], f"encoding.{k}", errors)
    if e["interpolation"] != "Linear":
        errors.append("encoding.interpolation: only 'Linear' interpolation is supported")

    net = config.get("network", {}) or {}
    _known(net, {"otype", "n_neurons", "n_hidden_layers", "activation", "output_activation",
                 "training"}, "network", errors)
    notype = _get(net, "otype", "FullyFusedMLP", str, "network", errors)
    if notype == "TiledMLP":
        errors.append("network.otype: TiledMLP JSON canonicalization is reserved")
    elif notype != "FullyFusedMLP":
        errors.append(f"network.otype: unsupported network otype '{notype}'")
    out_act = _get(net, "output_activation", "None", str, "network", errors)
    if out_act == "Linear":
        out_act = "None"
    elif out_act != "None":
        errors.append("network.output_activation: only 'None' output activation is supported")
    act = _get(net, "activation", "ReLU", str, "network", errors)
    if act != "ReLU":
        errors.append("network.activation: only 'ReLU' activation is supported")
    n = {
        "otype": "FullyFusedMLP",
        "n_input_dims": e["n_levels"] * e["n_features_per_level"],
        "n_output_dims": n_output,
        "n_neurons": _get(net, "n_neurons", 64, int, "network", errors),
        "n_hidden_layers": _get(net, "n_hidden_layers", 2, int, "network", errors),
        "activation": "ReLU",
        "output_activation": out_act,
    }
    _pos(n["n_neurons"], "network.n_neurons", errors)
    _pos(n["n_hidden_layers"], "network.n_hidden_layers", errors)

    loss = config.get("loss", {}) or {}
    lotype = _get(loss, "otype", "L2", str, "loss", errors)
    if lotype not in ("L2", "L1", "Huber", "Cosine", "RelativeL2"):
        errors.append(f"loss.otype: unsupported loss otype '{lotype}'")
    lo: dict[str, Any] = {"otype": lotype}
    if lotype == "Huber":
        _known(loss, {"otype", "huber_delta"}, "loss", errors)
        lo["huber_delta"] = _get(loss, "huber_delta", 1.0, float, "loss", errors)
        _pos(lo["huber_delta"], "loss.huber_delta", errors)
    elif lotype == "Cosine":
        _known(loss, {"otype", "output_dims"}, "loss", errors)
        if "output_dims" in loss:
            od = _get(loss, "output_dims", 0, int, "loss", errors)
            if od < 2:
                errors.append("loss.output_dims: must be >= 2 when provided")
            lo["output_dims"] = od
    else:
        _known(loss, {"otype"}, "loss", errors)

    opt = config.get("optimizer", {}) or {}
    _known(opt, {"otype", "learning_rate", "beta1", "beta2", "epsilon", "l1_reg", "l2_reg"},
           "optimizer", errors)
    ootype = _get(opt, "otype", "Adam", str, "optimizer", errors)
    if ootype != "Adam":
        errors.append(f"optimizer.otype: unsupported optimizer otype '{ootype}'")
    o = {
        "otype": "Adam",
        "learning_rate": _get(opt, "learning_rate", 1e-3, float, "optimizer", errors),
        "beta1": _get(opt, "beta1", 0.9, float, "optimizer", errors),
        "beta2": _get(opt, "beta2", 0.99, float, "optimizer", errors),
        "epsilon": _get(opt, "epsilon", 1e-15, float, "optimizer", errors),
        "l1_reg": _get(opt, "l1_reg", 0.0, float, "optimizer", errors),
        "l2_reg": _get(opt, "l2_reg", 0.0, float, "optimizer", errors),
    }
    for k in ("learning_rate", "beta1", "beta2", "epsilon"):
        _pos(o[k], f"optimizer.{k}", errors)
    for k in ("l1_reg", "l2_reg"):
        if o[k] < 0:
            errors.append(f"optimizer.{k}: must be >= 0")

    wi = config.get("weight_init", {}) or {}
    _known(wi, {"hash_grid_init", "hash_grid_range", "mlp_init", "mlp_nonlinearity",
                "mlp_uniform_range", "mlp_normal_stddev", "mlp_kaiming_a", "seed"},
           "weight_init", errors)
    w = {
        "hash_grid_init": _get(wi, "hash_grid_init", "Uniform", str, "weight_init", errors),
        "hash_grid_range": _get(wi, "hash_grid_range", 1e-4, float, "weight_init", errors),
        "mlp_init": _get(wi, "mlp_init", "KaimingUniform", str, "weight_init", errors),
        "mlp_nonlinearity": _get(wi, "mlp_nonlinearity", "ReLU", str, "weight_init", errors),
        "seed": _get(wi, "seed", 42, int, "weight_init", errors),
    }
    if w["hash_grid_init"] != "Uniform":
        errors.append("weight_init.hash_grid_init: only 'Uniform' is built in this library")
    if w["mlp_init"] != "KaimingUniform" or w["mlp_nonlinearity"] != "ReLU":
        errors.append("weight_init.mlp_init: only KaimingUniform/ReLU is built in this library")
    _pos(w["hash_grid_range"], "weight_init.hash_grid_range", errors)
    if not (0 <= w["seed"] < 2 ** 64):
        errors.append("weight_init.seed: must fit in uint64")

    batch = _get(config, "batch_size", 1024, int, "config", errors)
    if batch < 1:
        errors.append("batch_size: must be >= 1")

    mi = config.get("mi355x", {}) or {}
    _known(mi, {"precision", "hash_adam", "morton_sort", "grad_clip", "weight_decay", "family"},
           "mi355x", errors)
    m = {
        "precision": _get(mi, "precision", "fp32", str, "mi355x", errors),
        "hash_adam": _get(mi, "hash_adam", "lazy", str, "mi355x", errors),
        "morton_sort": _get(mi, "morton_sort", True, bool, "mi355x", errors),
        "grad_clip": _get(mi, "grad_clip", 0.0, float, "mi355x", errors),
        # decoupled (AdamW) decay of the adapters' training configs
        # (extension/training_adapter.h:43; adam_kernel_msl.h:85-88)
        "weight_decay": _get(mi, "weight_decay", 0.0, float, "mi355x", errors),
        # NetworkFactoryOptions::forced_family (network_planning.h:146-158)
        "family": _get(mi, "family", "auto", str, "mi355x", errors),
    }
    if m["family"] not in _lib.FAMILY_CODES:
        errors.append("mi355x.family: must be one of " + ", ".join(sorted(_lib.FAMILY_CODES)))
    if m["precision"] not in ("fp32", "fp16"):
        errors.append("mi355x.precision: must be 'fp32' or 'fp16'")
    if m["hash_adam"] not in ("lazy", "dense"):
        errors.append("mi355x.hash_adam: must be 'lazy' or 'dense'")
    for k in ("grad_clip", "weight_decay"):
        if isinstance(m[k], float) and m[k] < 0.0:
            errors.append(f"mi355x.{k}: must be >= 0")

    if errors:
        raise ConfigError("; ".join(errors))
    return {"encoding": e, "network": n, "loss": lo, "optimizer": o, "weight_init": w,
            "batch_size": batch, "mi355x": m}


_LOSS = {"L2": _lib.LOSS_L2, "L1": _lib.LOSS_L1, "Huber": _lib.LOSS_HUBER,
         "Cosine": _lib.LOSS_COSINE, "RelativeL2": _lib.LOSS_RELATIVE_L2}


def model_desc(canonical: dict) -> _lib.ModelDesc:
    """Fill the C-ABI descriptor from a canonical config."""
    c = copy.deepcopy(canonical)
    d = _lib.ModelDesc()
    _lib.load().tmnn_model_desc_init(d)
    e, n, lo, o, w, m = (c["encoding"], c["network"], c["loss"], c["optimizer"],
                         c["weight_init"], c["mi355x"])
    d.spatial_dims = e["n_input_dims"]
    d.num_levels = e["n_levels"]
    d.features_per_level = e["n_features_per_level"]
    d.log2_hashmap_size = e["log2_hashmap_size"]
    d.base_resolution = e["base_resolution"]
    d.per_level_scale = e["per_level_scale"]
    d.hidden_dim = n["n_neurons"]
    d.num_hidden_layers = n["n_hidden_layers"]
    d.num_outputs = n["n_output_dims"]
    d.loss_kind = _LOSS[lo["otype"]]
    d.huber_delta = lo.get("huber_delta", 1.0)
    # trainer_config_from_optimizer_config (factory_json_detail.h:464-499):
    # JSON learning_rate sets both the encoding and the network rate.
    d.lr_encoding = o["learning_rate"]
    d.lr_network = o["learning_rate"]
    d.beta1 = o["beta1"]
    d.beta2 = o["beta2"]
    d.epsilon = o["epsilon"]
    d.l1_reg = o["l1_reg"]
    d.l2_reg = o["l2_reg"]
    d.grad_clip = m["grad_clip"]
    d.weight_decay = m.get("weight_decay", 0.0)
    d.batch_size = c["batch_size"]
    d.precision = _lib.PRECISION_FP16 if m["precision"] == "fp16" else _lib.PRECISION_FP32
    d.hash_adam_mode = _lib.HASH_ADAM_DENSE if m["hash_adam"] == "dense" else _lib.HASH_ADAM_LAZY
    d.morton_sort = 1 if m["morton_sort"] else 0
    d.seed = w["seed"]
    d.hash_init_range = w["hash_grid_range"]
    d.forced_family = _lib.FAMILY_CODES[m.get("family", "auto")]
    return d
