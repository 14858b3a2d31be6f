"""ctypes binding of ``libpack3d_hip.so`` (declared in ``include/pack3d_hip.h``).

Loading fails loudly: there is no CPU or PyTorch fallback for any entry point.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

# The in-tree build; PACK3D_HIP_LIB may name another build of the same ABI.
LIB_PATH = os.environ.get("PACK3D_HIP_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                             "libpack3d_hip.so")

c_int32, c_int64, c_float, c_void_p = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p

P3D_F32, P3D_F16, P3D_BF16 = 0, 1, 2
P3D_EUNSUPPORTED = 3  # enum p3d_status
DTYPES = {torch.float32: P3D_F32, torch.float16: P3D_F16, torch.bfloat16: P3D_BF16}


class View(ctypes.Structure):
    _fields_ = [("data", c_void_p), ("sb", c_int64), ("sh", c_int64), ("sn", c_int64)]


ABI_VERSION = 19  # P3D_ABI_VERSION in include/pack3d_hip.h


class Rope(ctypes.Structure):
    _fields_ = [("table", c_void_p), ("pairs", c_void_p), ("coords", c_void_p),
                ("packed", c_int32), ("table_entries", c_int32)]


class PoolArgs(ctypes.Structure):
    _fields_ = [("batch", c_int32), ("kv_heads", c_int32), ("tokens", c_int32), ("head_dim", c_int32),
                ("dtype", c_int32), ("fine_blocks", c_int32), ("slots", c_int32), ("pool_size", c_int32),
                ("summaries", c_int32), ("temperature", c_float), ("key_scale", c_float),
                ("kg", View), ("vg", View),
                ("blocks", c_void_p), ("weight", c_void_p), ("bias", c_void_p), ("rope", Rope),
                ("sk", c_void_p), ("svt", c_void_p), ("sk_norm_max", c_void_p), ("norms_cleared", c_int32)]


class AttnArgs(ctypes.Structure):
    _fields_ = [("batch", c_int32), ("heads", c_int32), ("kv_heads", c_int32), ("tokens", c_int32),
                ("head_dim", c_int32), ("dtype", c_int32), ("summaries", c_int32), ("gate_dtype", c_int32),
                ("q", View), ("kl", View), ("vl", View), ("gate", View),
                ("local_scale", c_void_p), ("global_scale", c_void_p), ("sk", c_void_p), ("svt", c_void_p),
                ("sk_norm_max", c_void_p),
                ("rope", Rope), ("grid", c_int32 * 3), ("radius", c_int32 * 3),
                ("raster_to_packed", c_void_p), ("o_local_in", c_void_p), ("y", View),
                ("lse_local", c_void_p), ("lse_global", c_void_p), ("o_local", c_void_p),
                ("o_global", c_void_p), ("kl_rotated", c_int32)]


class BwdArgs(ctypes.Structure):
    _fields_ = [("batch", c_int32), ("heads", c_int32), ("kv_heads", c_int32), ("tokens", c_int32),
                ("head_dim", c_int32), ("dtype", c_int32), ("summaries", c_int32), ("gate_dtype", c_int32),
                ("parts", c_int32), ("splits", c_int32),
                ("q", View), ("kl", View), ("vl", View), ("gate", View),
                ("local_scale", c_void_p), ("global_scale", c_void_p), ("sk", c_void_p), ("svt", c_void_p),
                ("key_scale", c_float), ("pad_", c_int32),
                ("o_local", c_void_p), ("o_global", c_void_p), ("lse_local", c_void_p), ("lse_global", c_void_p),
                ("dy", View), ("dol", c_void_p), ("dog", c_void_p), ("delta_local", c_void_p),
                ("delta_global", c_void_p), ("dgate", c_void_p), ("dsl_part", c_void_p), ("dsg_part", c_void_p),
                ("sv_rows", c_void_p), ("skt", c_void_p), ("dq_local", c_void_p), ("dq_global", c_void_p),
                ("dk_local", c_void_p), ("dv_local", View), ("dsk_part", c_void_p), ("dsv_part", c_void_p),
                ("q_t", c_void_p), ("dog_t", c_void_p)]


class ProjectArgs(ctypes.Structure):
    _fields_ = [("x", c_void_p), ("ln_weight", c_void_p), ("ln_bias", c_void_p), ("wq", c_void_p),
                ("wkv", c_void_p), ("wg", c_void_p), ("gate_bias", c_void_p), ("q", c_void_p), ("kv", c_void_p),
                ("gate", c_void_p), ("rows", c_int64), ("dim", c_int32), ("q_out", c_int32), ("kv_out", c_int32),
                ("heads", c_int32), ("dtype", c_int32), ("ln_dtype", c_int32), ("gate_bias_dtype", c_int32),
                ("eps", c_float)]


_P = c_void_p
SIGNATURES = {
    "p3d_last_error": ([], ctypes.c_char_p),
    "p3d_abi_version": ([], c_int32),
    "p3d_build_layout": ([_P, _P, _P, c_int32, _P, _P, _P, _P, _P, _P], c_int32),
    "p3d_geometry_check": ([_P, c_int32, c_int64, c_int32, _P, c_int32, c_int64, c_int32, c_int32,
                            _P, _P, _P, _P, _P, _P], c_int32),
    "p3d_reverse_adjacency": ([_P, c_int64, c_int32, _P, _P, c_int32, _P], c_int32),
    "p3d_repack": ([_P, c_int64, _P, c_int32, _P, c_int64, c_int32, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                    _P, _P], c_int32),
    "p3d_check_layout": ([_P, _P, _P, _P, _P, _P], c_int32),
    "p3d_stencil_match": ([_P, _P, _P, _P, c_int32, _P, _P, _P], c_int32),
    "p3d_pool_fwd": ([ctypes.POINTER(PoolArgs), _P], c_int32),
    "p3d_attn_fwd_grid": ([ctypes.POINTER(AttnArgs), _P], c_int32),
    "p3d_attn_fwd_rows": ([ctypes.POINTER(AttnArgs), _P], c_int32),
    "p3d_attn_fwd_grid_noalloc": ([ctypes.POINTER(PoolArgs), ctypes.POINTER(AttnArgs), _P], c_int32),
    "p3d_local_fwd_indexed": ([ctypes.POINTER(AttnArgs), _P, c_int32, _P], c_int32),
    "p3d_selftest_mfma": ([c_int32, _P, _P, _P, _P], c_int32),
    "p3d_struct_sizes": ([_P], c_int32),
    "p3d_rotate": ([View, View, c_int32, c_int32, c_int32, c_int32, c_int32, ctypes.POINTER(Rope), c_int32, _P],
                   c_int32),
    "p3d_layer_norm": ([_P, _P, _P, c_int32, _P, c_int64, c_int32, c_int32, c_float, _P], c_int32),
    "p3d_project": ([ctypes.POINTER(ProjectArgs), _P], c_int32),
    "p3d_project_linear": ([ctypes.POINTER(ProjectArgs), _P], c_int32),
    "p3d_project_pool": ([ctypes.POINTER(ProjectArgs), ctypes.POINTER(PoolArgs), c_int32, _P], c_int32),
    "p3d_out_residual": ([_P, _P, _P, _P, c_int64, c_int32, c_int32, c_int32, c_int32, _P], c_int32),
    "p3d_layer_norm_train": ([_P, _P, _P, c_int32, _P, _P, _P, _P, c_int64, c_int32, c_int32, c_int32, c_float,
                              _P], c_int32),
    "p3d_layer_norm_bwd": ([_P, _P, _P, _P, c_int32, _P, _P, _P, _P, c_int64, c_int32, c_int32, c_int32, c_int32,
                            c_int32, _P], c_int32),
    "p3d_copy_rows": ([View, View, c_int64, c_int32, c_int64, c_int32, c_int32, _P], c_int32),
    "p3d_input_grad": ([_P, c_int64, c_int32, _P, c_int64, c_int32, _P, c_int64, c_int32, _P, c_int32, _P, c_int64,
                        c_int32, c_int32, _P], c_int32),
    "p3d_weight_grad3": ([_P, c_int64, c_int32, _P, c_int64, c_int32, _P, c_int64, c_int32, _P, c_int64, _P, _P,
                          c_int64, c_int32, c_int32, c_int32, _P], c_int32),
    "p3d_weight_grad": ([_P, c_int64, _P, c_int64, _P, _P, c_int64, c_int32, c_int32, c_int32, c_int32, _P], c_int32),
    "p3d_mix_bwd": ([ctypes.POINTER(BwdArgs), _P], c_int32),
    "p3d_local_bwd_indexed": ([ctypes.POINTER(BwdArgs), _P, c_int32, _P, c_int32, _P], c_int32),
    "p3d_local_bwd_grid": ([ctypes.POINTER(BwdArgs), _P, _P, _P, _P], c_int32),
    "p3d_global_bwd": ([ctypes.POINTER(BwdArgs), _P], c_int32),
    "p3d_global_bwd_dq": ([ctypes.POINTER(BwdArgs), _P], c_int32),
    "p3d_global_bwd_dkv": ([ctypes.POINTER(BwdArgs), _P], c_int32),
    "p3d_transpose_rows": ([View, _P, c_int32, c_int32, c_int32, c_int32, c_int32, _P], c_int32),
    "p3d_finish_bwd": ([ctypes.POINTER(BwdArgs), ctypes.POINTER(Rope), View, View, _P], c_int32),
    "p3d_pool_bwd": ([ctypes.POINTER(PoolArgs), _P, _P, c_int32, View, View, _P, _P, _P], c_int32),
}

_lock = threading.Lock()
_lib = None


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(f"pack3d_amd HIP library missing at {LIB_PATH}; "
                                       "build it with `python -m pack3d_amd.build`")
                handle = ctypes.CDLL(LIB_PATH)
                for name, (args, res) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.argtypes = args
                    fn.restype = res
                if handle.p3d_abi_version() != ABI_VERSION:
                    raise RuntimeError("pack3d_amd HIP library ABI mismatch; rebuild it")
                _lib = handle
    return _lib


PROBE_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libpack3d_probe.so")
_probe = None


def probe_lib():
    """The measurement library (``include/pack3d_probe.h``): the issue-rate
    probe behind ``bench.py --probe-rates``.  Not part of the product
    library; loaded only when asked for."""
    global _probe
    if _probe is None:
        with _lock:
            if _probe is None:
                if not os.path.exists(PROBE_PATH):
                    raise RuntimeError(f"probe library missing at {PROBE_PATH}; build it with "
                                       "`python -m pack3d_amd.build`")
                handle = ctypes.CDLL(PROBE_PATH)
                handle.p3d_probe_issue_rates.argtypes = [c_int32, c_int64, c_int32, _P, _P]
                handle.p3d_probe_issue_rates.restype = c_int32
                handle.p3d_last_error.argtypes = []
                handle.p3d_last_error.restype = ctypes.c_char_p
                _probe = handle
    return _probe


def call(name, *args):
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().p3d_last_error().decode()
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def stream_of(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t):
    return None if t is None else t.data_ptr()


def i64x3(values):
    return (c_int64 * 3)(*[int(v) for v in values])


def i32x3(values):
    return (c_int32 * 3)(*[int(v) for v in values])


def view(t: torch.Tensor) -> View:
    """A [B, H, N, C] tensor with unit channel stride as a p3d_view."""
    sb, sh, sn, sc = t.stride()
    assert sc == 1 or t.shape[3] == 1
    return View(t.data_ptr(), sb, sh, sn)


def view3(t: torch.Tensor) -> View:
    """A [B, H, N] tensor (the gate) as a p3d_view."""
    sb, sh, sn = t.stride()
    return View(t.data_ptr(), sb, sh, sn)


def require_device(t: torch.Tensor, what="tensor"):
    if t.device.type != "cuda":
        raise ValueError(f"the hip backend requires {what} on a HIP device; no CPU fallback exists")
