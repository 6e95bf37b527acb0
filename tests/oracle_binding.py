"""ctypes binding of the CPU oracle (oracle/libtmnn_oracle.so) and of the
reference-source build (oracle/_ref/libtmnn_ref.so) for the tests.

Test infrastructure only: the product (tiny-metal-nn_amd/) never loads these.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent.parent
ORACLE_SO = REPO / "oracle" / "libtmnn_oracle.so"
REF_SO = REPO / "oracle" / "_ref" / "libtmnn_ref.so"

L2, L1, HUBER, COSINE, RELATIVE_L2 = range(5)
_LOSS_NAMES = {"L2": L2, "L1": L1, "Huber": HUBER, "Cosine": COSINE, "RelativeL2": RELATIVE_L2}


class OrcModel(ctypes.Structure):
    _fields_ = [
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
    ]


class OrcAdam(ctypes.Structure):
    _fields_ = [(k, ctypes.c_float) for k in (
        "lr_encoding", "lr_network", "beta1", "beta2", "epsilon", "l1_reg", "l2_reg",
        "grad_clip", "weight_decay")]


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


_V = ctypes.c_void_p


class Oracle:
    def __init__(self, path: Path = ORACLE_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        lib = ctypes.CDLL(str(path))
        M = ctypes.POINTER(OrcModel)
        A = ctypes.POINTER(OrcAdam)
        sig = {
            "orc_hash_param_count": (ctypes.c_uint32, [M]),
            "orc_mlp_param_count": (ctypes.c_uint32, [M]),
            "orc_mask_word_count": (ctypes.c_uint32, [M]),
            "orc_resolutions": (None, [M, _V]),
            "orc_philox_uniform": (None, [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                                          ctypes.c_float, ctypes.c_float, _V]),
            "orc_init_params": (None, [M, ctypes.c_uint64, ctypes.c_float, _V, _V]),
            "orc_encode": (None, [M, _V, _V, ctypes.c_int32, _V, _V, _V]),
            "orc_forward": (None, [M, _V, _V, _V, ctypes.c_int32, _V]),
            "orc_forward_backward": (None, [M, _V, _V, _V, ctypes.c_int32, _V, _V, _V, _V, _V,
                                            _V, _V, ctypes.c_int32]),
            "orc_adam_bias_corrections": (None, [ctypes.c_float, ctypes.c_float, ctypes.c_uint32,
                                                 _V, _V]),
            "orc_adam_step": (None, [M, A, ctypes.c_uint32, _V, _V, _V, _V, _V, _V,
                                     ctypes.c_int32]),
            "orc_morton_codes": (None, [_V, ctypes.c_int32, ctypes.c_int32, _V]),
            "orc_evaluate_with_gradient": (None, [M, _V, _V, _V, ctypes.c_int32, _V, _V]),
            "orc_training_step": (ctypes.c_float, [M, A, ctypes.c_uint32, _V, _V, _V, _V, _V,
                                                   ctypes.c_int32, ctypes.c_int32,
                                                   ctypes.c_int32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        self.lib = lib

    # ---- model helpers ----------------------------------------------------
    @staticmethod
    def model(spatial_dims=3, num_levels=16, features_per_level=2, log2_hashmap_size=19,
              base_resolution=16.0, per_level_scale=1.447, hidden_dim=64,
              num_hidden_layers=2, num_outputs=1, loss="L2", huber_delta=1.0) -> OrcModel:
        return OrcModel(spatial_dims, num_levels, features_per_level, log2_hashmap_size,
                        base_resolution, per_level_scale, hidden_dim, num_hidden_layers,
                        num_outputs, _LOSS_NAMES[loss] if isinstance(loss, str) else loss,
                        huber_delta)

    @staticmethod
    def adam(lr_encoding=1e-2, lr_network=1e-2, beta1=0.9, beta2=0.99, epsilon=1e-15,
             l1_reg=0.0, l2_reg=0.0, grad_clip=0.0, weight_decay=0.0) -> OrcAdam:
        return OrcAdam(lr_encoding, lr_network, beta1, beta2, epsilon, l1_reg, l2_reg,
                       grad_clip, weight_decay)

    def counts(self, m):
        return (self.lib.orc_hash_param_count(m), self.lib.orc_mlp_param_count(m),
                self.lib.orc_mask_word_count(m))

    def resolutions(self, m) -> np.ndarray:
        out = np.empty(m.num_levels, np.float32)
        self.lib.orc_resolutions(m, _p(out))
        return out

    def philox_uniform(self, seed, counter_base, count, low, high) -> np.ndarray:
        out = np.empty(count, np.float32)
        self.lib.orc_philox_uniform(seed, counter_base, count, low, high, _p(out))
        return out

    def init_params(self, m, seed=42, hash_range=1e-4):
        nh, nm, _ = self.counts(m)
        h = np.empty(nh, np.float32)
        w = np.empty(nm, np.float32)
        self.lib.orc_init_params(m, seed, hash_range, _p(h), _p(w))
        return h, w

    def encode(self, m, table, pos, with_corners=False):
        pos = np.ascontiguousarray(pos, np.float32)
        n = pos.shape[0]
        L, F = m.num_levels, m.features_per_level
        D = 3 if m.spatial_dims == 2 else m.spatial_dims
        C = 1 << D
        feats = np.empty((n, L * F), np.float32)
        idx = np.empty((n, L, C), np.uint32) if with_corners else None
        w = np.empty((n, L, C), np.float32) if with_corners else None
        self.lib.orc_encode(m, _p(table), _p(pos), n, _p(feats), _p(idx), _p(w))
        return (feats, idx, w) if with_corners else feats

    def forward(self, m, table, mlp, pos) -> np.ndarray:
        pos = np.ascontiguousarray(pos, np.float32)
        out = np.empty((pos.shape[0], m.num_outputs), np.float32)
        self.lib.orc_forward(m, _p(table), _p(mlp), _p(pos), pos.shape[0], _p(out))
        return out

    def evaluate_with_gradient(self, m, table, mlp, pos):
        """(out [N][M], Jacobian [N][M][D]) of the evaluator's gradient kernel."""
        pos = np.ascontiguousarray(pos, np.float32)
        n = pos.shape[0]
        out = np.empty((n, m.num_outputs), np.float32)
        grads = np.empty((n, m.num_outputs, m.spatial_dims), np.float32)
        self.lib.orc_evaluate_with_gradient(m, _p(table), _p(mlp), _p(pos), n, _p(out),
                                            _p(grads))
        return out, grads

    def forward_backward(self, m, table, mlp, pos, target=None, d_out=None, threads=8):
        """Returns (grad_hash int32, grad_mlp float64, mask uint32, loss_sum, outputs)."""
        pos = np.ascontiguousarray(pos, np.float32)
        n = pos.shape[0]
        nh, nm, nw = self.counts(m)
        gh = np.zeros(nh, np.int32)
        gm = np.zeros(nm, np.float64)
        mask = np.zeros(nw, np.uint32)
        loss = ctypes.c_double(0.0)
        out = np.empty((n, m.num_outputs), np.float32)
        tgt = None if target is None else np.ascontiguousarray(target, np.float32)
        dout = None if d_out is None else np.ascontiguousarray(d_out, np.float32)
        self.lib.orc_forward_backward(m, _p(table), _p(mlp), _p(pos), n, _p(tgt), _p(dout),
                                      _p(gh), _p(gm), _p(mask), ctypes.byref(loss), _p(out),
                                      threads)
        return gh, gm, mask, loss.value, out

    def bias_corrections(self, beta1, beta2, step):
        b1, b2 = ctypes.c_float(), ctypes.c_float()
        self.lib.orc_adam_bias_corrections(beta1, beta2, step, ctypes.byref(b1),
                                           ctypes.byref(b2))
        return b1.value, b2.value

    def adam_step(self, m, a, step, params, m1, m2, grad_hash, grad_mlp, mask=None, threads=8):
        gm32 = np.ascontiguousarray(grad_mlp, np.float32)
        self.lib.orc_adam_step(m, a, step, _p(params), _p(m1), _p(m2),
                               _p(np.ascontiguousarray(grad_hash, np.int32)), _p(gm32),
                               _p(mask), threads)

    def morton_codes(self, pos, dims) -> np.ndarray:
        pos = np.ascontiguousarray(pos, np.float32)
        out = np.empty(pos.shape[0], np.uint32)
        self.lib.orc_morton_codes(_p(pos), pos.shape[0], dims, _p(out))
        return out

    def training_step(self, m, a, step, params, m1, m2, pos, target, dense_hash=False,
                      threads=8) -> float:
        pos = np.ascontiguousarray(pos, np.float32)
        tgt = np.ascontiguousarray(target, np.float32)
        return self.lib.orc_training_step(m, a, step, _p(params), _p(m1), _p(m2), _p(pos),
                                          _p(tgt), pos.shape[0], 1 if dense_hash else 0,
                                          threads)


class RefLib:
    """C entry points over the reference's own host sources (oracle/ref_shim.cpp)."""

    def __init__(self, path: Path = REF_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} missing (reference checkout absent at build)")
        lib = ctypes.CDLL(str(path))
        sig = {
            "ref_morton_code_3d": (ctypes.c_uint32, [ctypes.c_float] * 3),
            "ref_morton_code_4d": (ctypes.c_uint32, [ctypes.c_float] * 4),
            "ref_morton_sort_batch": (ctypes.c_int, [_V, _V, ctypes.c_int, ctypes.c_uint32,
                                                     ctypes.c_uint32, _V, _V, _V]),
            "ref_mlp_weight_count": (ctypes.c_int, [ctypes.c_int] * 4),
            "ref_kernel_spec_validate": (ctypes.c_int, [ctypes.c_int] * 6),
            "ref_loss_evaluate_cpu": (ctypes.c_float, [ctypes.c_int, _V, _V, ctypes.c_int,
                                                       ctypes.c_float, ctypes.c_uint32]),
            "ref_emit_kernel_source": (ctypes.c_long, [ctypes.c_int] * 5 + [ctypes.c_float] * 2
                                       + [ctypes.c_int] * 4 + [ctypes.c_char_p,
                                                               ctypes.c_size_t]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        self.lib = lib

    def morton_sort_batch(self, pos, tgt):
        pos = np.ascontiguousarray(pos, np.float32)
        tgt = np.ascontiguousarray(tgt, np.float32)
        n, di = pos.shape
        dt = tgt.shape[1]
        sp = np.empty_like(pos)
        st = np.empty_like(tgt)
        idx = np.empty(n, np.uint32)
        rc = self.lib.ref_morton_sort_batch(_p(pos), _p(tgt), n, di, dt, _p(sp), _p(st), _p(idx))
        if rc != 0:
            raise ValueError("ref_morton_sort_batch failed")
        return sp, st, idx

    def loss_evaluate_cpu(self, kind, pred, target, delta=1.0, output_dims=0):
        pred = np.ascontiguousarray(pred, np.float32).ravel()
        target = np.ascontiguousarray(target, np.float32).ravel()
        return self.lib.ref_loss_evaluate_cpu(kind, _p(pred), _p(target), pred.size, delta,
                                              output_dims)

    def emit_kernel_source(self, kind, spatial_dims=3, num_levels=16, features_per_level=2,
                           log2_hashmap_size=19, base_resolution=16.0, per_level_scale=1.447,
                           hidden_dim=64, num_hidden_layers=2, num_outputs=1, loss=0) -> str:
        """The reference's generated MSL text (kind 0: scalar train, 1: eval)."""
        args = (kind, spatial_dims, num_levels, features_per_level, log2_hashmap_size,
                base_resolution, per_level_scale, hidden_dim, num_hidden_layers, num_outputs,
                loss)
        n = self.lib.ref_emit_kernel_source(*args, None, 0)
        if n < 0:
            raise ValueError("reference emitter rejected the spec")
        buf = ctypes.create_string_buffer(n + 1)
        self.lib.ref_emit_kernel_source(*args, buf, n + 1)
        return buf.value.decode()
