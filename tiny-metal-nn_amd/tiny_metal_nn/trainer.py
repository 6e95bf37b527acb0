"""Trainer: the reference's Python surface (src/python/tmnn_pybind.cpp:274-600)
over the MI355X C-ABI.

Same construction (`Trainer.from_config(config, n_input=, n_output=)`), same
calls (`training_step`, `inference`, `step`, `close`, context manager), same
errors (ConfigError, DTypeError, ClosedError, ConcurrentTrainingStepError),
plus the split/accumulate API and checkpoint calls of the C++ Trainer
(include/tiny-metal-nn/trainer.h) and device-pointer entry points for
callers whose batches already live in GPU memory.
"""
from __future__ import annotations

import contextlib
import ctypes
import threading
from dataclasses import dataclass

import numpy as np

from . import _lib
from .config import ConfigError, canonicalize_model_config, model_desc


class DTypeError(TypeError):
    """An input array is not float32 (the reference's DTypeError)."""


class ClosedError(RuntimeError):
    """The trainer was already closed."""


class ConcurrentTrainingStepError(RuntimeError):
    """A second thread entered the single-threaded trainer."""


@dataclass
class OptimizerStateBlob:
    """OptimizerStateBlob v1 (include/tiny-metal-nn/detail/runtime_authority.h)."""

    version: int
    step: int
    payload: bytes


def _as_f32_2d(x, name: str, cols: int | None = None) -> np.ndarray:
    arr = np.asarray(x)
    if arr.dtype != np.float32:
        raise DTypeError(f"{name} must be float32, got {arr.dtype}")
    if arr.ndim != 2:
        raise ValueError(f"{name} must be 2D (batch_size, dims)")
    if not arr.flags["C_CONTIGUOUS"]:
        raise ValueError(f"{name} must be C-contiguous")
    if cols is not None and arr.shape[1] != cols:
        raise ValueError(f"{name} must have {cols} columns, got {arr.shape[1]}")
    return arr


def _event_arg(event):
    """A HIP event argument: None, an int address, or an object exposing a
    ctypes `_as_parameter_` (torch.cuda.Event, once recorded)."""
    if event is None:
        return None
    if isinstance(event, int):
        return ctypes.c_void_p(event)
    p = getattr(event, "_as_parameter_", None)
    if p is None:
        raise TypeError("event must be None, an address or an object with _as_parameter_")
    return p if isinstance(p, ctypes.c_void_p) else ctypes.c_void_p(int(p))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


class _Context:
    """One HIP device + stream shared by trainers (MetalContext analogue)."""

    _lock = threading.Lock()
    _by_device: dict[int, "_Context"] = {}

    def __init__(self, device: int):
        lib = _lib.load()
        h = ctypes.c_void_p()
        _lib.check(lib.tmnn_context_create(device, ctypes.byref(h)))
        self.handle = h
        self.device = device

    @classmethod
    def get(cls, device: int = 0) -> "_Context":
        with cls._lock:
            ctx = cls._by_device.get(device)
            if ctx is None:
                ctx = cls._by_device[device] = _Context(device)
            return ctx


class Trainer:
    """The single object for training and inference on hash-grid + MLP."""

    def __init__(self, canonical: dict, device: int = 0):
        self._lib = _lib.load()
        self.config = canonical
        self.n_input = canonical["encoding"]["n_input_dims"]
        self.n_output = canonical["network"]["n_output_dims"]
        self._ctx = _Context.get(device)
        h = ctypes.c_void_p()
        desc = model_desc(canonical)
        _lib.check(self._lib.tmnn_trainer_create(self._ctx.handle, ctypes.byref(desc),
                                                 ctypes.byref(h)))
        self._h = h
        hc, mc = ctypes.c_uint32(), ctypes.c_uint32()
        _lib.check(self._lib.tmnn_trainer_param_counts(h, ctypes.byref(hc), ctypes.byref(mc)))
        self.hash_param_count = hc.value
        self.mlp_param_count = mc.value
        self._busy = threading.Lock()
        self._closed = False

    # ---- construction ---------------------------------------------------
    @classmethod
    def from_config(cls, config: dict, *, n_input: int, n_output: int,
                    device: int = 0) -> "Trainer":
        """Construct from a JSON-shaped dict (try_create_from_config)."""
        canonical = canonicalize_model_config(int(n_input), int(n_output), config)
        return cls(canonical, device=device)

    # ---- lifetime ---------------------------------------------------------
    def close(self) -> None:
        if not self._closed:
            self._closed = True
            self._lib.tmnn_trainer_destroy(self._h)
            self._h = None

    @property
    def closed(self) -> bool:
        return self._closed

    def __enter__(self) -> "Trainer":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __repr__(self) -> str:
        if self._closed:
            return "<tmnn.Trainer closed>"
        return (f"<tmnn.Trainer n_input={self.n_input} n_output={self.n_output} "
                f"step={self.step()}>")

    def _check_open(self) -> None:
        if self._closed:
            raise ClosedError("Trainer is closed")

    @contextlib.contextmanager
    def _enter(self, what: str):
        """Hold the single-caller guard for one call (tmnn_pybind.cpp:366-375):
        a second thread entering meanwhile gets ConcurrentTrainingStepError."""
        self._check_open()
        if not self._busy.acquire(blocking=False):
            raise ConcurrentTrainingStepError(
                f"{what} is already in progress on another thread. tmnn.Trainer is "
                "single-threaded; use one Trainer per thread.")
        try:
            yield
        finally:
            self._busy.release()

    # ---- accessors ----------------------------------------------------------
    def step(self) -> int:
        self._check_open()
        s = ctypes.c_uint32()
        _lib.check(self._lib.tmnn_get_step(self._h, ctypes.byref(s)))
        return s.value

    def is_gpu_available(self) -> bool:
        self._check_open()
        return True

    def inspect_runtime(self) -> dict:
        self._check_open()
        ins = _lib.Inspection()
        _lib.check(self._lib.tmnn_trainer_inspect(self._h, ctypes.byref(ins)))
        out = {k: getattr(ins, k) for k, _ in _lib.Inspection._fields_}
        out["family_name"] = _lib.FAMILIES.get(out["family"], "Unknown")
        return out

    def network_plan(self) -> dict:
        """The NetworkPlan this trainer's kernels were chosen from."""
        self._check_open()
        p = _lib.NetworkPlan()
        _lib.check(self._lib.tmnn_trainer_get_plan(self._h, ctypes.byref(p)))
        return plan_to_dict(p)

    # ---- fused path -----------------------------------------------------------
    def training_step(self, input, target) -> float:
        """One fused step (forward + backward + Adam); returns the loss."""
        x = _as_f32_2d(input, "input", self.n_input)
        y = _as_f32_2d(target, "target", self.n_output)
        if x.shape[0] != y.shape[0]:
            raise ValueError("input and target must have matching batch_size")
        return self.training_step_result(x, y)["loss"]

    def training_step_result(self, input, target) -> dict:
        """One fused step; returns the C++ API's TrainingStepResult as a dict
        (loss, step, batch_n, grad_norm, numerics_reported,
        has_numerics_anomaly, numerics{finite_forward, finite_backward,
        finite_update, max_abs_activation, max_abs_gradient, max_abs_update,
        first_bad_layer}); the numerics are filled on sampled steps
        (set_numerics_sampling) and whenever the loss is not finite."""
        x = _as_f32_2d(input, "input", self.n_input)
        y = _as_f32_2d(target, "target", self.n_output)
        if x.shape[0] != y.shape[0]:
            raise ValueError("input and target must have matching batch_size")
        with self._enter("training_step"):
            res = _lib.StepResult()
            _lib.check(self._lib.tmnn_training_step(self._h, _ptr(x), _ptr(y), x.shape[0],
                                                    ctypes.byref(res)))
            return res.to_dict()

    def set_numerics_sampling(self, mode: str = "Sampled", interval: int = 128) -> None:
        """NumericsSamplingMode ("Sampled", "Periodic", "FullPerStep",
        "Disabled") and sample interval (runtime_policy.h:13-38)."""
        if mode not in _lib.NUMERICS_MODES:
            raise ValueError(f"unknown numerics sampling mode {mode!r}")
        with self._enter("set_numerics_sampling"):
            _lib.check(self._lib.tmnn_set_numerics_sampling(self._h, _lib.NUMERICS_MODES[mode],
                                                            int(interval)))

    def last_numerics(self) -> dict:
        """Report of the last step whose numerics were computed (waits for the
        trainer's stream): every host-pointer step, sampled device steps."""
        with self._enter("last_numerics"):
            res = _lib.StepResult()
            _lib.check(self._lib.tmnn_get_last_numerics(self._h, ctypes.byref(res)))
            return res.to_dict()

    def debug_step_outputs(self, input, target) -> tuple[np.ndarray, dict]:
        """A regular fused step that also returns the outputs its training
        kernel computed ((N, n_output), caller row order) and the step result."""
        x = _as_f32_2d(input, "input", self.n_input)
        y = _as_f32_2d(target, "target", self.n_output)
        n = min(x.shape[0], self.config["batch_size"])
        out = np.empty((n, self.n_output), np.float32)
        with self._enter("debug_step_outputs"):
            res = _lib.StepResult()
            _lib.check(self._lib.tmnn_debug_step_outputs(self._h, _ptr(x), _ptr(y), x.shape[0],
                                                         _ptr(out), ctypes.byref(res)))
            return out, res.to_dict()

    def training_step_device_after(self, input_ptr: int, target_ptr: int, n: int,
                                   wait_event=None, loss_ptr: int = 0) -> None:
        """training_step_device ordered after a caller's HIP event (an object
        with a ctypes `_as_parameter_`, e.g. torch.cuda.Event, or a raw
        pointer); the trainer's streams wait for it before reading the batch."""
        with self._enter("training_step_device_after"):
            _lib.check(self._lib.tmnn_training_step_device_after(
                self._h, ctypes.c_void_p(input_ptr), ctypes.c_void_p(target_ptr), int(n),
                ctypes.c_void_p(loss_ptr) if loss_ptr else None, _event_arg(wait_event)))

    def inference_device_after(self, input_ptr: int, output_ptr: int, n: int,
                               wait_event=None) -> None:
        with self._enter("inference_device_after"):
            _lib.check(self._lib.tmnn_inference_device_after(
                self._h, ctypes.c_void_p(input_ptr), ctypes.c_void_p(output_ptr), int(n),
                _event_arg(wait_event)))

    def record_event(self, event) -> None:
        """Record a caller's HIP event on the trainer's stream after every call
        enqueued so far (outputs of *_device calls are complete when it is)."""
        with self._enter("record_event"):
            _lib.check(self._lib.tmnn_record_event(self._h, _event_arg(event)))

    def training_step_device(self, input_ptr: int, target_ptr: int, n: int,
                             loss_ptr: int = 0) -> None:
        """Enqueue one step on device-resident data (no host synchronization)."""
        with self._enter("training_step_device"):
            _lib.check(self._lib.tmnn_training_step_device(
                self._h, ctypes.c_void_p(input_ptr), ctypes.c_void_p(target_ptr), int(n),
                ctypes.c_void_p(loss_ptr) if loss_ptr else None))

    def training_step_device_noalloc(self, input_ptr: int, target_ptr: int, n: int,
                                     loss_ptr: int = 0) -> None:
        """training_step_device without any device allocation: the step's
        batch buffers live in the library's fixed per-GPU scratch (batches up
        to its size; calls overlapping on one GPU race)."""
        with self._enter("training_step_device_noalloc"):
            _lib.check(self._lib.tmnn_training_step_device_noalloc(
                self._h, ctypes.c_void_p(input_ptr), ctypes.c_void_p(target_ptr), int(n),
                ctypes.c_void_p(loss_ptr) if loss_ptr else None))

    def inference(self, input) -> np.ndarray:
        """Evaluate at N positions; returns a fresh (N, n_output) float32 array."""
        x = _as_f32_2d(input, "input", self.n_input)
        out = np.empty((x.shape[0], self.n_output), np.float32)
        with self._enter("inference"):
            if x.shape[0]:
                _lib.check(self._lib.tmnn_inference(self._h, _ptr(x), _ptr(out), x.shape[0]))
        return out

    evaluate = inference

    def evaluate_with_gradient(self, input) -> tuple[np.ndarray, np.ndarray]:
        """(outputs (N, n_output), Jacobian (N, n_output, n_input)) in fp32."""
        x = _as_f32_2d(input, "input", self.n_input)
        n = x.shape[0]
        out = np.empty((n, self.n_output), np.float32)
        jac = np.empty((n, self.n_output, self.n_input), np.float32)
        with self._enter("evaluate_with_gradient"):
            if n:
                _lib.check(self._lib.tmnn_evaluate_with_gradient(self._h, _ptr(x), _ptr(out),
                                                                 _ptr(jac), n))
        return out, jac

    def inference_device(self, input_ptr: int, output_ptr: int, n: int) -> None:
        with self._enter("inference_device"):
            _lib.check(self._lib.tmnn_inference_device(
                self._h, ctypes.c_void_p(input_ptr), ctypes.c_void_p(output_ptr), int(n)))

    def synchronize(self) -> None:
        with self._enter("synchronize"):
            _lib.check(self._lib.tmnn_synchronize(self._h))

    # ---- split / accumulate path -------------------------------------------
    def forward_for_training(self, input) -> np.ndarray:
        x = _as_f32_2d(input, "input", self.n_input)
        out = np.empty((x.shape[0], self.n_output), np.float32)
        written = ctypes.c_uint32()
        with self._enter("forward_for_training"):
            _lib.check(self._lib.tmnn_forward_for_training(self._h, _ptr(x), _ptr(out),
                                                           x.shape[0], ctypes.byref(written)))
        return out[: written.value // self.n_output]

    def zero_gradients(self) -> None:
        with self._enter("zero_gradients"):
            _lib.check(self._lib.tmnn_zero_gradients(self._h))

    def backward_accumulate(self, input, d_output) -> None:
        x = _as_f32_2d(input, "input", self.n_input)
        g = _as_f32_2d(d_output, "d_output", self.n_output)
        if x.shape[0] != g.shape[0]:
            raise ValueError("input and d_output must have matching batch_size")
        with self._enter("backward_accumulate"):
            _lib.check(self._lib.tmnn_backward_accumulate(self._h, _ptr(x), _ptr(g), x.shape[0]))

    def adam_step(self) -> None:
        with self._enter("adam_step"):
            _lib.check(self._lib.tmnn_adam_step(self._h))

    # ---- state ---------------------------------------------------------------
    def get_weights(self) -> tuple[np.ndarray, np.ndarray]:
        hw = np.empty(self.hash_param_count, np.float32)
        mw = np.empty(self.mlp_param_count, np.float32)
        with self._enter("get_weights"):
            _lib.check(self._lib.tmnn_get_weights(self._h, _ptr(hw), hw.size, _ptr(mw), mw.size))
        return hw, mw

    def set_initial_weights(self, hash_weights=None, mlp_weights=None) -> None:
        hp, hn, mp, mn = None, 0, None, 0
        if hash_weights is not None:
            hash_weights = np.ascontiguousarray(hash_weights, np.float32).ravel()
            hp, hn = _ptr(hash_weights), hash_weights.size
        if mlp_weights is not None:
            mlp_weights = np.ascontiguousarray(mlp_weights, np.float32).ravel()
            mp, mn = _ptr(mlp_weights), mlp_weights.size
        with self._enter("set_initial_weights"):
            _lib.check(self._lib.tmnn_set_initial_weights(self._h, hp, hn, mp, mn))

    def export_optimizer_state(self) -> OptimizerStateBlob:
        n = ctypes.c_size_t()
        ver, st = ctypes.c_uint32(), ctypes.c_uint32()
        with self._enter("export_optimizer_state"):
            _lib.check(self._lib.tmnn_export_optimizer_state(self._h, ctypes.byref(ver),
                                                             ctypes.byref(st), None, 0,
                                                             ctypes.byref(n)))
            buf = (ctypes.c_uint8 * n.value)()
            _lib.check(self._lib.tmnn_export_optimizer_state(self._h, ctypes.byref(ver),
                                                             ctypes.byref(st), buf, n.value,
                                                             ctypes.byref(n)))
        return OptimizerStateBlob(ver.value, st.value, bytes(buf))

    def import_optimizer_state(self, blob: OptimizerStateBlob) -> None:
        data = (ctypes.c_uint8 * len(blob.payload)).from_buffer_copy(blob.payload)
        with self._enter("import_optimizer_state"):
            _lib.check(self._lib.tmnn_import_optimizer_state(self._h, blob.version, blob.step,
                                                             data, len(blob.payload)))

    def reset_optimizer(self) -> None:
        with self._enter("reset_optimizer"):
            _lib.check(self._lib.tmnn_reset_optimizer(self._h))

    def set_learning_rate(self, lr: float) -> None:
        with self._enter("set_learning_rate"):
            _lib.check(self._lib.tmnn_set_learning_rate(self._h, float(lr), float(lr)))

    # ---- step profiling (TrainingStepProfile GPU timestamps) -------------------
    def set_training_step_profiling(self, enabled: bool, every: int = 1) -> None:
        """Enable/disable per-phase GPU event timing of fused steps (one step in
        `every` when enabled); resets the sums."""
        if every < 1:
            raise ValueError("every must be >= 1")
        with self._enter("set_training_step_profiling"):
            _lib.check(self._lib.tmnn_set_step_profiling(self._h, int(every) if enabled else 0))

    def training_step_profile(self) -> dict:
        """Per-phase GPU microseconds summed over the profiled steps."""
        p = _lib.StepProfile()
        with self._enter("training_step_profile"):
            _lib.check(self._lib.tmnn_get_step_profile(self._h, ctypes.byref(p)))
        return {k: getattr(p, k) for k, _ in _lib.StepProfile._fields_}

    def training_step_profile_samples(self) -> np.ndarray:
        """Per profiled step (rows, step order) the phase GPU microseconds,
        columns as _lib.PROFILE_PHASES."""
        with self._enter("training_step_profile_samples"):
            cnt = ctypes.c_uint32()
            _lib.check(self._lib.tmnn_get_step_profile_samples(self._h, None, 0, ctypes.byref(cnt)))
            out = np.zeros((cnt.value, len(_lib.PROFILE_PHASES)), np.float32)
            if cnt.value:
                _lib.check(self._lib.tmnn_get_step_profile_samples(self._h, _ptr(out), cnt.value,
                                                                   ctypes.byref(cnt)))
        return out

    def debug_lds_rate(self, reps: int = 10) -> float:
        """LDS read bandwidth of this trainer's device, bytes/s
        (tmnn_debug_lds_rate)."""
        b = ctypes.c_double()
        with self._enter("debug_lds_rate"):
            _lib.check(self._lib.tmnn_debug_lds_rate(self._ctx.handle, int(reps), ctypes.byref(b)))
        return b.value

    # ---- runtime authority (RuntimeAuthority / batch_plan) ----------------------
    def runtime_buffer(self, role: str) -> dict:
        """RuntimeAuthority::buffer(role): the device range of a buffer role
        (pointer, offset, bytes, element kind); bytes == 0 for roles this
        library passes as launch arguments."""
        self._check_open()
        if role not in _lib.BUFFER_ROLES:
            raise ValueError(f"unknown RuntimeBufferRole {role!r}")
        v = _lib.BufferView()
        v.struct_size = ctypes.sizeof(v)
        _lib.check(self._lib.tmnn_runtime_buffer(self._h, _lib.BUFFER_ROLES[role], ctypes.byref(v)))
        return {"role": role, "gpu_buffer": v.gpu_buffer or 0, "offset": v.offset,
                "bytes": v.bytes, "device_ptr": v.device_ptr or 0,
                "element_kind": _lib.ELEMENT_KINDS[v.element_kind],
                "visibility": _lib.STORAGE[v.visibility],
                "lifetime": _lib.LIFETIMES[v.lifetime], "valid": bool(v.gpu_buffer and v.bytes)}

    def parameter_layout(self) -> dict:
        """RuntimeAuthority::parameter_layout."""
        self._check_open()
        p = _lib.ParameterLayout()
        p.struct_size = ctypes.sizeof(p)
        _lib.check(self._lib.tmnn_parameter_layout(self._h, ctypes.byref(p)))
        return {k: getattr(p, k) for k, _ in _lib.ParameterLayout._fields_ if k != "struct_size"}

    def storage_policy(self) -> dict:
        """RuntimeAuthority::storage_policy."""
        self._check_open()
        p = _lib.StoragePolicy()
        p.struct_size = ctypes.sizeof(p)
        _lib.check(self._lib.tmnn_storage_policy(self._h, ctypes.byref(p)))
        out = {k: getattr(p, k) for k, _ in _lib.StoragePolicy._fields_ if k != "struct_size"}
        for k in ("parameter_weights", "gradients", "optimizer_state", "control_buffers"):
            out[k] = _lib.STORAGE[out[k]]
        for k in ("step_inputs", "step_targets", "step_reduction"):
            out[k] = _lib.LIFETIMES[out[k]]
        out["requires_staging_uploads"] = bool(out["requires_staging_uploads"])
        return out

    def batch_plan(self) -> dict:
        """ITrainerRuntime::batch_plan (TrainerBatchPlan)."""
        self._check_open()
        p = _lib.BatchPlan()
        p.struct_size = ctypes.sizeof(p)
        _lib.check(self._lib.tmnn_batch_plan(self._h, ctypes.byref(p)))
        return {k: getattr(p, k) for k, _ in _lib.BatchPlan._fields_ if k != "struct_size"}

    # ---- inspection hooks (parity tests) --------------------------------------
    def debug_encode(self, positions, with_corners: bool = False):
        x = _as_f32_2d(positions, "positions", self.n_input)
        e = self.config["encoding"]
        L, F = e["n_levels"], e["n_features_per_level"]
        C = 1 << self.n_input
        n = x.shape[0]
        feats = np.empty((n, L * F), np.float32)
        idx = np.empty((n, L, C), np.uint32) if with_corners else None
        w = np.empty((n, L, C), np.float32) if with_corners else None
        _lib.check(self._lib.tmnn_debug_encode(
            self._h, _ptr(x), n, _ptr(feats), _ptr(idx) if with_corners else None,
            _ptr(w) if with_corners else None))
        return (feats, idx, w) if with_corners else feats

    def debug_encode_tiles(self, positions, sorted: bool = True):
        """The training step's own encode kernels: (features [N][L*F] in the
        step's point order, perm (row j is input row perm[j]), the sorted
        positions the encode wrote, count of nonzero padding floats)."""
        x = _as_f32_2d(positions, "positions", self.n_input)
        e = self.config["encoding"]
        n = x.shape[0]
        feats = np.empty((n, e["n_levels"] * e["n_features_per_level"]), np.float32)
        perm = np.empty(n, np.uint32)
        spos = np.empty((n, self.n_input), np.float32)
        pad = ctypes.c_uint64(0)
        with self._enter("debug_encode_tiles"):
            _lib.check(self._lib.tmnn_debug_encode_tiles(self._h, _ptr(x), n, 1 if sorted else 0,
                                                         _ptr(feats), _ptr(perm), _ptr(spos),
                                                         ctypes.byref(pad)))
        return feats, perm, spos, pad.value

    def debug_hash_rates(self, positions_ptr: int, n: int, sorted: bool = True,
                         reps: int = 20) -> dict:
        """GPU microseconds per launch of the gather / atomic / flag-store
        reference kernels over n device-resident positions at this trainer's
        hash-grid shape (tmnn_debug_hash_rates)."""
        g, a, f = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        with self._enter("debug_hash_rates"):
            _lib.check(self._lib.tmnn_debug_hash_rates(
                self._h, ctypes.c_void_p(positions_ptr), int(n), 1 if sorted else 0, int(reps),
                ctypes.byref(g), ctypes.byref(a), ctypes.byref(f)))
        return {"gather_us": g.value, "atomic_us": a.value, "flag_us": f.value}

    def debug_gradients(self) -> tuple[np.ndarray, np.ndarray]:
        self._check_open()
        gh = np.empty(self.hash_param_count, np.int32)
        gm = np.empty(self.mlp_param_count, np.float32)
        _lib.check(self._lib.tmnn_debug_get_gradients(self._h, _ptr(gh), gh.size, _ptr(gm),
                                                      gm.size))
        return gh, gm

    def debug_active_mask(self) -> np.ndarray:
        self._check_open()
        F = self.config["encoding"]["n_features_per_level"]
        width = 2 if F == 2 else 1
        words = (self.hash_param_count // width + 31) // 32
        out = np.empty(words, np.uint32)
        _lib.check(self._lib.tmnn_debug_get_active_mask(self._h, _ptr(out), words))
        return out

    def debug_morton_sort(self, positions) -> tuple[np.ndarray, np.ndarray]:
        """(Morton codes, stable sort permutation) the step applies to a batch."""
        x = _as_f32_2d(positions, "positions", self.n_input)
        n = x.shape[0]
        codes = np.empty(n, np.uint32)
        perm = np.empty(n, np.uint32)
        if n:
            _lib.check(self._lib.tmnn_debug_morton_sort(self._h, _ptr(x), n, _ptr(codes),
                                                        _ptr(perm)))
        return codes, perm

    def debug_train_image(self) -> tuple[np.ndarray, np.ndarray]:
        """(current, repacked) bytes of the training plan's packed weight image."""
        self._check_open()
        nbytes = ctypes.c_uint64(0)
        _lib.check(self._lib.tmnn_debug_train_image(self._h, None, None, ctypes.byref(nbytes)))
        cur = np.empty(nbytes.value, np.uint8)
        rep = np.empty(nbytes.value, np.uint8)
        _lib.check(self._lib.tmnn_debug_train_image(self._h, _ptr(cur), _ptr(rep),
                                                    ctypes.byref(nbytes)))
        return cur, rep

    def debug_resolutions(self) -> np.ndarray:
        self._check_open()
        L = self.config["encoding"]["n_levels"]
        out = np.empty(L, np.float32)
        _lib.check(self._lib.tmnn_debug_get_resolutions(self._h, _ptr(out), L))
        return out


def philox_uniform(seed: int, counter_base: int, count: int, low: float, high: float,
                   device: int = 0) -> np.ndarray:
    """The GPU's seeded Philox-4x32-10 uniform fill (weight-init stream)."""
    ctx = _Context.get(device)
    out = np.empty(count, np.float32)
    _lib.check(_lib.load().tmnn_debug_philox_uniform(ctx.handle, seed, counter_base, count,
                                                     low, high, _ptr(out)))
    return out


__all__ = ["Trainer", "ConfigError", "DTypeError", "ClosedError",
           "ConcurrentTrainingStepError", "OptimizerStateBlob", "philox_uniform"]


def plan_to_dict(p) -> dict:
    caps = {k: getattr(p.capabilities, k) for k, _ in _lib.DeviceCaps._fields_ if k != "struct_size"}
    return {
        "selected_family": _lib.FAMILIES.get(p.selected_family) if p.selected_family >= 0 else None,
        "fused_eval": bool(p.fused_eval),
        "fused_train": bool(p.fused_train),
        "planner_fingerprint": p.planner_fingerprint,
        "candidate_families": [n for f, n in _lib.FAMILIES.items() if p.candidate_families >> f & 1],
        "reasons": [n for r, n in sorted(_lib.PLAN_REASONS.items()) if p.reasons >> r & 1],
        "train_lds_bytes": p.train_lds_bytes,
        "train_waves_per_block": p.train_waves_per_block,
        "capabilities": caps,
    }


def plan_network(config: dict, n_input: int, n_output: int, capabilities: dict | None = None) -> dict:
    """plan_network(model, capabilities) (network_planning.h:176-190): the
    family this library would run `config` with on a device of the given
    capabilities (default: a nominal MI355X; runs without a GPU)."""
    from .config import canonicalize_model_config, model_desc
    canon = canonicalize_model_config(int(n_input), int(n_output), config)
    d = model_desc(canon)
    lib = _lib.load()
    caps = _lib.DeviceCaps()
    lib.tmnn_device_caps_init(caps)
    for k, v in (capabilities or {}).items():
        if k == "struct_size" or not hasattr(caps, k):
            raise ValueError(f"unknown capability {k!r}")
        setattr(caps, k, v)
    p = _lib.NetworkPlan()
    _lib.check(lib.tmnn_plan_network(ctypes.byref(caps), ctypes.byref(d), ctypes.byref(p)))
    return plan_to_dict(p)

