"""ctypes binding of libtmnn_hip.so (the C-ABI declared in include/tmnn_hip.h).

The shared library is built in-tree by tiny-metal-nn_amd/build.py. There is
no fallback: if the library is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent.parent
LIB_PATH = Path(os.environ.get("TMNN_HIP_LIB", PKG_ROOT / "libtmnn_hip.so"))

TMNN_OK = 0
TMNN_ERR_INVALID_ARGUMENT = -1
TMNN_ERR_RUNTIME = -2
TMNN_ERR_GPU = -3
TMNN_ERR_UNSUPPORTED = -4

LOSS_L2, LOSS_L1, LOSS_HUBER, LOSS_COSINE, LOSS_RELATIVE_L2 = range(5)
PRECISION_FP32, PRECISION_FP16 = 0, 1
HASH_ADAM_LAZY, HASH_ADAM_DENSE = 0, 1

c_float_p = ctypes.POINTER(ctypes.c_float)


class ModelDesc(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("spatial_dims", ctypes.c_int32),
        ("num_levels", ctypes.c_int32),
        ("features_per_level", ctypes.c_int32),
        ("log2_hashmap_size", ctypes.c_int32),
        ("base_resolution", ctypes.c_float),
        ("per_level_scale", ctypes.c_float),
        ("hidden_dim", ctypes.c_int32),
        ("num_hidden_layers", ctypes.c_int32),
        ("num_outputs", ctypes.c_int32),
        ("loss_kind", ctypes.c_int32),
        ("huber_delta", ctypes.c_float),
        ("lr_encoding", ctypes.c_float),
        ("lr_network", ctypes.c_float),
        ("beta1", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("epsilon", ctypes.c_float),
        ("l1_reg", ctypes.c_float),
        ("l2_reg", ctypes.c_float),
        ("grad_clip", ctypes.c_float),
        ("weight_decay", ctypes.c_float),
        ("batch_size", ctypes.c_int32),
        ("precision", ctypes.c_int32),
        ("hash_adam_mode", ctypes.c_int32),
        ("morton_sort", ctypes.c_int32),
        ("seed", ctypes.c_uint64),
        ("hash_init_range", ctypes.c_float),
        ("forced_family", ctypes.c_int32),
    ]


class DeviceCaps(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("gpu_available", ctypes.c_int32),
        ("cu_count", ctypes.c_int32),
        ("lds_bytes_per_cu", ctypes.c_int32),
        ("wave_size", ctypes.c_int32),
        ("has_mfma_f16", ctypes.c_int32),
        ("global_mem_bytes", ctypes.c_uint64),
    ]


class NetworkPlan(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("selected_family", ctypes.c_int32),
        ("fused_eval", ctypes.c_int32),
        ("fused_train", ctypes.c_int32),
        ("planner_fingerprint", ctypes.c_uint64),
        ("candidate_families", ctypes.c_uint32),
        ("reasons", ctypes.c_uint32),
        ("train_lds_bytes", ctypes.c_int32),
        ("train_waves_per_block", ctypes.c_int32),
        ("capabilities", DeviceCaps),
    ]


# NetworkFamily / PlannerFallbackReason names (network_planning.h:29-58)
FAMILIES = {0: "FullyFused", 1: "Tiled", 2: "SafeDebug"}
FAMILY_CODES = {"auto": -1, "FullyFused": 0, "Tiled": 1, "SafeDebug": 2}
PLAN_REASONS = {1: "NoGPUContext", 4: "ThreadgroupMemoryExceeded", 6: "UnsupportedInputDims",
                7: "UnsupportedOutputDims", 9: "HiddenDimUnsupported", 10: "ForcedTiled",
                11: "ForcedSafeDebug", 13: "NoFusedInstance"}


class NumericsReport(ctypes.Structure):
    """NumericsReport (detail/runtime_stats.h:32-40)."""
    _fields_ = [
        ("finite_forward", ctypes.c_int32),
        ("finite_backward", ctypes.c_int32),
        ("finite_update", ctypes.c_int32),
        ("max_abs_activation", ctypes.c_float),
        ("max_abs_gradient", ctypes.c_float),
        ("max_abs_update", ctypes.c_float),
        ("first_bad_layer", ctypes.c_uint32),
    ]


class StepResult(ctypes.Structure):
    """TrainingStepResult (common.h:97-110); struct_size is set on creation."""
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("loss", ctypes.c_float),
        ("step", ctypes.c_uint32),
        ("batch_n", ctypes.c_uint32),
        ("grad_norm", ctypes.c_float),
        ("numerics_reported", ctypes.c_int32),
        ("has_numerics_anomaly", ctypes.c_int32),
        ("numerics", NumericsReport),
    ]

    def __init__(self, *args, **kw):
        super().__init__(*args, **kw)
        self.struct_size = ctypes.sizeof(StepResult)

    def to_dict(self) -> dict:
        out = {k: getattr(self, k) for k, _ in self._fields_ if k not in ("struct_size", "numerics")}
        out["numerics"] = {k: getattr(self.numerics, k) for k, _ in NumericsReport._fields_}
        for k in ("finite_forward", "finite_backward", "finite_update"):
            out["numerics"][k] = bool(out["numerics"][k])
        out["numerics_reported"] = bool(out["numerics_reported"])
        out["has_numerics_anomaly"] = bool(out["has_numerics_anomaly"])
        return out


# NumericsSamplingMode (runtime_policy.h:13-18), same numbering
NUMERICS_MODES = {"Sampled": 0, "Periodic": 1, "FullPerStep": 2, "Disabled": 3}


class Inspection(ctypes.Structure):
    _fields_ = [
        ("family", ctypes.c_int32),
        ("precision", ctypes.c_int32),
        ("hidden_padded", ctypes.c_int32),
        ("input_padded", ctypes.c_int32),
        ("points_per_wave_tile", ctypes.c_int32),
        ("waves_per_block_train", ctypes.c_int32),
        ("blocks_train", ctypes.c_int32),
        ("lds_bytes_train", ctypes.c_int32),
        ("lds_bytes_infer", ctypes.c_int32),
        ("cu_count", ctypes.c_int32),
        ("hash_param_count", ctypes.c_uint32),
        ("mlp_param_count", ctypes.c_uint32),
        ("batch_size", ctypes.c_uint32),
        ("train_fused_scatter", ctypes.c_int32),
    ]


class StepProfile(ctypes.Structure):
    _fields_ = [
        ("steps", ctypes.c_uint32),
        ("batch_size", ctypes.c_uint32),
        ("gpu_sort_us", ctypes.c_double),
        ("gpu_fwd_bwd_us", ctypes.c_double),
        ("gpu_scatter_us", ctypes.c_double),
        ("gpu_reduce_us", ctypes.c_double),
        ("gpu_adam_us", ctypes.c_double),
        ("gpu_total_us", ctypes.c_double),
        ("gpu_encode_us", ctypes.c_double),
        ("infer_calls", ctypes.c_uint32),
        ("gpu_infer_us", ctypes.c_double),
        ("gpu_encode_kernel_us", ctypes.c_double),
        ("gpu_train_kernel_us", ctypes.c_double),
        ("gpu_scatter_kernel_us", ctypes.c_double),
        ("gpu_finish_kernel_us", ctypes.c_double),
    ]


# columns of tmnn_get_step_profile_samples (TMNN_PROFILE_*)
PROFILE_PHASES = ("gpu_sort_us", "gpu_encode_us", "gpu_fwd_bwd_us", "gpu_scatter_us",
                  "gpu_reduce_us", "gpu_adam_us", "gpu_total_us", "gpu_encode_kernel_us",
                  "gpu_train_kernel_us", "gpu_scatter_kernel_us", "gpu_finish_kernel_us")

# RuntimeBufferRole (runtime_authority.h:68-79), same numbering
BUFFER_ROLES = {"ConfigWeights": 0, "HashWeights": 1, "MlpWeights": 2, "GradHash": 3,
                "GradMlp": 4, "TrainParams": 5, "AdamParams": 6, "FusedWeights": 7,
                "FusedFirstMoment": 8, "FusedSecondMoment": 9}
ELEMENT_KINDS = {0: "f32", 1: "i32", 2: "i32_packed_pair", 3: "opaque"}
STORAGE = {0: "CpuVisible", 1: "GpuOnly"}
LIFETIMES = {0: "Persistent", 1: "Transient", 2: "Staging"}


class BufferView(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("role", ctypes.c_int32),
        ("gpu_buffer", ctypes.c_void_p),
        ("offset", ctypes.c_uint64),
        ("bytes", ctypes.c_uint64),
        ("device_ptr", ctypes.c_void_p),
        ("element_kind", ctypes.c_int32),
        ("visibility", ctypes.c_int32),
        ("lifetime", ctypes.c_int32),
    ]


class ParameterLayout(ctypes.Structure):
    _fields_ = [(k, ctypes.c_uint32) for k in (
        "struct_size", "hash_grid_float_count", "mlp_weight_float_count",
        "train_params_float_count", "train_params_idx_n", "train_params_idx_unsigned_mode",
        "train_params_idx_loss_scale", "train_params_idx_num_active_levels",
        "adam_params_float_count", "config_header_float_count", "config_tail_float_count",
        "target_dims", "reduction_terms")] + [("fused_adam", ctypes.c_int32)]


class BatchPlan(ctypes.Structure):
    _fields_ = [(k, ctypes.c_uint32) for k in (
        "struct_size", "max_batch_size", "lane_count", "input_dims", "target_dims",
        "reduction_terms")] + [(k, ctypes.c_uint64) for k in (
            "positions_bytes_per_lane", "targets_bytes_per_lane", "reduction_bytes_per_lane")] + [
        (k, ctypes.c_uint32) for k in ("threadgroup_size", "points_per_threadgroup")]


class StoragePolicy(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32)] + [(k, ctypes.c_int32) for k in (
        "parameter_weights", "gradients", "optimizer_state", "control_buffers", "step_inputs",
        "step_targets", "step_reduction", "requires_staging_uploads")]


_V = ctypes.c_void_p
_I32 = ctypes.c_int32
_U32 = ctypes.c_uint32
_SZ = ctypes.c_size_t
_F = ctypes.c_float

# name -> (restype, argtypes); every symbol include/tmnn_hip.h declares.
SIGNATURES = {
    "tmnn_last_error": (ctypes.c_char_p, []),
    "tmnn_abi_version": (_U32, []),
    "tmnn_context_create": (ctypes.c_int, [_I32, ctypes.POINTER(_V)]),
    "tmnn_context_destroy": (ctypes.c_int, [_V]),
    "tmnn_context_device_info": (ctypes.c_int, [_V, ctypes.POINTER(_I32),
                                                ctypes.POINTER(ctypes.c_uint64),
                                                ctypes.c_char_p, _SZ]),
    "tmnn_model_desc_init": (None, [ctypes.POINTER(ModelDesc)]),
    "tmnn_trainer_create": (ctypes.c_int, [_V, ctypes.POINTER(ModelDesc), ctypes.POINTER(_V)]),
    "tmnn_trainer_destroy": (ctypes.c_int, [_V]),
    "tmnn_trainer_param_counts": (ctypes.c_int, [_V, ctypes.POINTER(_U32), ctypes.POINTER(_U32)]),
    "tmnn_trainer_inspect": (ctypes.c_int, [_V, ctypes.POINTER(Inspection)]),
    "tmnn_trainer_get_plan": (ctypes.c_int, [_V, ctypes.POINTER(NetworkPlan)]),
    "tmnn_context_caps": (ctypes.c_int, [_V, ctypes.POINTER(DeviceCaps)]),
    "tmnn_device_caps_init": (None, [ctypes.POINTER(DeviceCaps)]),
    "tmnn_plan_network": (ctypes.c_int, [ctypes.POINTER(DeviceCaps), ctypes.POINTER(ModelDesc),
                                         ctypes.POINTER(NetworkPlan)]),
    "tmnn_training_step": (ctypes.c_int, [_V, _V, _V, _I32, ctypes.POINTER(StepResult)]),
    "tmnn_training_step_device": (ctypes.c_int, [_V, _V, _V, _I32, _V]),
    "tmnn_training_step_device_after": (ctypes.c_int, [_V, _V, _V, _I32, _V, _V]),
    "tmnn_record_event": (ctypes.c_int, [_V, _V]),
    "tmnn_set_numerics_sampling": (ctypes.c_int, [_V, _I32, _U32]),
    "tmnn_get_last_numerics": (ctypes.c_int, [_V, ctypes.POINTER(StepResult)]),
    "tmnn_training_step_device_noalloc": (ctypes.c_int, [_V, _V, _V, _I32, _V]),
    "tmnn_inference": (ctypes.c_int, [_V, _V, _V, _I32]),
    "tmnn_inference_device": (ctypes.c_int, [_V, _V, _V, _I32]),
    "tmnn_inference_device_after": (ctypes.c_int, [_V, _V, _V, _I32, _V]),
    "tmnn_evaluate_with_gradient": (ctypes.c_int, [_V, _V, _V, _V, _I32]),
    "tmnn_forward_for_training": (ctypes.c_int, [_V, _V, _V, _I32, ctypes.POINTER(_U32)]),
    "tmnn_zero_gradients": (ctypes.c_int, [_V]),
    "tmnn_backward_accumulate": (ctypes.c_int, [_V, _V, _V, _I32]),
    "tmnn_adam_step": (ctypes.c_int, [_V]),
    "tmnn_synchronize": (ctypes.c_int, [_V]),
    "tmnn_get_step": (ctypes.c_int, [_V, ctypes.POINTER(_U32)]),
    "tmnn_get_weights": (ctypes.c_int, [_V, _V, _SZ, _V, _SZ]),
    "tmnn_set_initial_weights": (ctypes.c_int, [_V, _V, _SZ, _V, _SZ]),
    "tmnn_export_optimizer_state": (ctypes.c_int, [_V, ctypes.POINTER(_U32), ctypes.POINTER(_U32),
                                                   _V, _SZ, ctypes.POINTER(_SZ)]),
    "tmnn_import_optimizer_state": (ctypes.c_int, [_V, _U32, _U32, _V, _SZ]),
    "tmnn_reset_optimizer": (ctypes.c_int, [_V]),
    "tmnn_set_learning_rate": (ctypes.c_int, [_V, _F, _F]),
    "tmnn_set_step_profiling": (ctypes.c_int, [_V, _I32]),
    "tmnn_get_step_profile": (ctypes.c_int, [_V, ctypes.POINTER(StepProfile)]),
    "tmnn_get_step_profile_samples": (ctypes.c_int, [_V, _V, _U32, ctypes.POINTER(_U32)]),
    "tmnn_debug_lds_rate": (ctypes.c_int, [_V, _I32, ctypes.POINTER(ctypes.c_double)]),
    "tmnn_runtime_buffer": (ctypes.c_int, [_V, _I32, ctypes.POINTER(BufferView)]),
    "tmnn_parameter_layout": (ctypes.c_int, [_V, ctypes.POINTER(ParameterLayout)]),
    "tmnn_storage_policy": (ctypes.c_int, [_V, ctypes.POINTER(StoragePolicy)]),
    "tmnn_batch_plan": (ctypes.c_int, [_V, ctypes.POINTER(BatchPlan)]),
    "tmnn_debug_encode": (ctypes.c_int, [_V, _V, _I32, _V, _V, _V]),
    "tmnn_debug_encode_tiles": (ctypes.c_int, [_V, _V, _I32, _I32, _V, _V, _V,
                                               ctypes.POINTER(ctypes.c_uint64)]),
    "tmnn_debug_hash_rates": (ctypes.c_int, [_V, _V, _I32, _I32, _I32,
                                             ctypes.POINTER(ctypes.c_double),
                                             ctypes.POINTER(ctypes.c_double),
                                             ctypes.POINTER(ctypes.c_double)]),
    "tmnn_debug_step_outputs": (ctypes.c_int, [_V, _V, _V, _I32, _V, ctypes.POINTER(StepResult)]),
    "tmnn_debug_get_gradients": (ctypes.c_int, [_V, _V, _SZ, _V, _SZ]),
    "tmnn_debug_get_active_mask": (ctypes.c_int, [_V, _V, _SZ]),
    "tmnn_debug_morton_sort": (ctypes.c_int, [_V, _V, _I32, _V, _V]),
    "tmnn_debug_get_resolutions": (ctypes.c_int, [_V, _V, _I32]),
    "tmnn_debug_train_image": (ctypes.c_int, [_V, _V, _V, ctypes.POINTER(ctypes.c_uint64)]),
    "tmnn_debug_philox_uniform": (ctypes.c_int, [_V, ctypes.c_uint64, _U32, _U32, _F, _F, _V]),
}


class TmnnError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


_lib = None


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python tiny-metal-nn_amd/build.py`")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != TMNN_OK:
        msg = load().tmnn_last_error().decode(errors="replace")
        if rc == TMNN_ERR_INVALID_ARGUMENT:
            raise ValueError(msg)
        raise TmnnError(rc, msg)
