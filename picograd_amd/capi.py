"""ctypes binding of the picograd C ABI.

The same prototypes describe libpicograd_amd.so (device-resident tensors)
and any library that exports the reference ABI (autograd.h, jit.h, sgd.h,
tensor.h, backend.h).  `PgLib.device` says whether tensor data must be
fetched with pg_tensor_copy_to_host (this build) or read from t->data.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

PG_MAX_NDIM = 8
F32, F16, BF16 = 0, 1, 2
_NP_OF = {F32: np.float32, F16: np.uint16, BF16: np.uint16}


class PgTensor(C.Structure):
    """Leading fields shared by the reference pg_tensor and this build's."""
    _fields_ = [
        ("ndim", C.c_size_t),
        ("shape", C.c_size_t * PG_MAX_NDIM),
        ("stride", C.c_size_t * PG_MAX_NDIM),
        ("numel", C.c_size_t),
        ("data", C.c_void_p),
        ("data_ref", C.c_void_p),
        ("is_view", C.c_bool),
        ("view_parent", C.c_void_p),
        ("dtype", C.c_int),
        ("elem_size", C.c_size_t),
    ]


class PgTensorAmd(C.Structure):
    _fields_ = PgTensor._fields_ + [("dev", C.c_void_p), ("pg_flags", C.c_uint)]


class PgNode(C.Structure):
    _fields_ = [
        ("value", C.c_void_p),
        ("grad", C.c_void_p),
        ("nparents", C.c_size_t),
        ("parents", C.c_void_p),
        ("ctx", C.c_void_p),
        ("backward", C.c_void_p),
        ("ag_op", C.c_int),
        ("requires_grad", C.c_bool),
        ("refs", C.c_uint),
        ("mark", C.c_ubyte),
    ]


class SgdCfg(C.Structure):
    _fields_ = [("lr", C.c_float), ("momentum", C.c_float), ("dampening", C.c_float),
                ("weight_decay", C.c_float), ("nesterov", C.c_bool)]


class AdamCfg(C.Structure):
    _fields_ = [("lr", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float), ("eps", C.c_float),
                ("weight_decay", C.c_float), ("amsgrad", C.c_bool), ("decoupled_wd", C.c_bool)]


vp, sz, fl, bo, ip = C.c_void_p, C.c_size_t, C.c_float, C.c_bool, C.c_int
SZP = C.POINTER(C.c_size_t)

_PROTOS = {
    # tensor.h
    "pg_seed": (None, [C.c_ulonglong]),
    "pg_tensor_from_data": (vp, [sz, SZP, vp]),
    "pg_tensor_from_data_dtype": (vp, [ip, sz, SZP, vp]),
    "pg_tensor_zeros": (vp, [sz, SZP]),
    "pg_tensor_full": (vp, [sz, SZP, fl]),
    "pg_tensor_uniform": (vp, [sz, SZP, fl, fl]),
    "pg_tensor_normal": (vp, [sz, SZP, fl, fl]),
    "pg_tensor_free": (None, [vp]),
    "pg_tensor_fill": (None, [vp, fl]),
    "pg_tensor_save": (bo, [vp, C.c_char_p]),
    "pg_tensor_load": (vp, [C.c_char_p]),
    # autograd.h
    "pg_var_from_data": (vp, [sz, SZP, vp, bo]),
    "pg_var_from_tensor": (vp, [vp, bo]),
    "pg_var_zeros": (vp, [sz, SZP, bo]),
    "pg_var_full": (vp, [sz, SZP, fl, bo]),
    "pg_var_uniform": (vp, [sz, SZP, fl, fl, bo]),
    "pg_var_normal": (vp, [sz, SZP, fl, fl, bo]),
    "pg_var_scalar": (vp, [fl, bo]),
    "pg_node_retain": (vp, [vp]),
    "pg_node_free": (None, [vp]),
    "pg_ag_matmul": (vp, [vp, vp]),
    "pg_ag_sum": (vp, [vp, sz, bo]),
    "pg_ag_mean": (vp, [vp, sz, bo]),
    "pg_ag_sum_all": (vp, [vp]),
    "pg_ag_mean_all": (vp, [vp]),
    "pg_ag_mse": (vp, [vp, vp, bo]),
    "pg_ag_leaky_relu": (vp, [vp, fl]),
    "pg_ag_clamp": (vp, [vp, fl, fl]),
    "pg_backward": (None, [vp]),
    "pg_backward_jit": (bo, [vp]),
    "pg_autograd_set_jit": (None, [bo]),
    "pg_autograd_is_jit_enabled": (bo, []),
    "pg_autograd_last_error": (C.c_char_p, []),
    "pg_autograd_last_was_jit": (bo, []),
    "pg_autograd_jit_hits": (sz, []),
    "pg_autograd_jit_fallbacks": (sz, []),
    "pg_no_grad_push": (None, []),
    "pg_no_grad_pop": (None, []),
    # sgd.h
    "pg_sgd_cfg_default": (SgdCfg, []),
    "pg_sgd_new": (vp, [C.POINTER(SgdCfg)]),
    "pg_sgd_free": (None, [vp]),
    "pg_sgd_add_param": (ip, [vp, vp]),
    "pg_sgd_num_params": (sz, [vp]),
    "pg_sgd_zero_grad": (None, [vp]),
    "pg_sgd_step": (None, [vp]),
    # adam.h
    "pg_adam_cfg_default": (AdamCfg, []),
    "pg_adam_new": (vp, [C.POINTER(AdamCfg)]),
    "pg_adam_free": (None, [vp]),
    "pg_adam_add_param": (ip, [vp, vp]),
    "pg_adam_add_param_lr": (ip, [vp, vp, fl, fl]),
    "pg_adam_num_params": (sz, [vp]),
    "pg_adam_set_lr": (None, [vp, fl]),
    "pg_adam_get_lr": (fl, [vp]),
    "pg_adam_set_param_lr": (None, [vp, sz, fl]),
    "pg_adam_set_param_wd": (None, [vp, sz, fl]),
    "pg_adam_zero_grad": (None, [vp]),
    "pg_adam_step": (None, [vp]),
    "pg_adam_set_step": (None, [vp, C.c_ulonglong]),
    "pg_adam_get_step": (C.c_ulonglong, [vp]),
    # clip.h
    "pg_clip_grad_norm": (fl, [C.POINTER(vp), sz, fl, fl]),
    "pg_clip_grad_value": (None, [C.POINTER(vp), sz, fl]),
    "pg_grad_norm": (fl, [C.POINTER(vp), sz]),
    # backend.h
    "pg_gemm": (None, [sz, sz, sz, vp, sz, vp, sz, vp, sz]),
    "pg_gemm_ex": (None, [ip, sz, sz, sz, vp, sz, vp, sz, vp, sz]),
    "pg_hgemm": (None, [sz, sz, sz, vp, sz, vp, sz, vp, sz]),
    "pg_bgemm": (None, [sz, sz, sz, vp, sz, vp, sz, vp, sz]),
    # jit.h
    "pg_jit_graph_new": (vp, []),
    "pg_jit_graph_free": (None, [vp]),
    "pg_jit_add_input": (ip, [vp, sz, SZP]),
    "pg_jit_add_const": (ip, [vp, fl]),
    "pg_jit_add_op": (ip, [vp, ip, C.POINTER(C.c_int), sz]),
    "pg_jit_mark_output": (None, [vp, ip]),
    "pg_jit_num_inputs": (sz, [vp]),
    "pg_jit_num_outputs": (sz, [vp]),
    "pg_jit_num_nodes": (sz, [vp]),
    "pg_jit_compile": (vp, [vp]),
    "pg_jit_exe_free": (None, [vp]),
    "pg_jit_run": (bo, [vp, C.POINTER(vp), sz, C.POINTER(vp), sz]),
    "pg_jit_run_single": (vp, [vp, C.POINTER(vp), sz]),
    "pg_jit_last_error": (C.c_char_p, []),
    "pg_jit_cache_size": (sz, []),
    "pg_jit_cache_clear": (None, []),
    "pg_jit_graph_hash": (C.c_uint64, [vp]),
    "pg_jit_set_cache_enabled": (None, [bo]),
}
for _op in ("add", "sub", "mul", "div"):
    _PROTOS[f"pg_ag_{_op}"] = (vp, [vp, vp])
for _op in ("neg", "exp", "log", "sqrt", "sin", "cos", "relu", "sigmoid", "tanh", "gelu", "erf", "abs"):
    _PROTOS[f"pg_ag_{_op}"] = (vp, [vp])
for _op in ("add", "sub", "mul", "div"):
    _PROTOS[f"pg_jit_{_op}"] = (ip, [vp, ip, ip])
for _op in ("neg", "exp", "log", "sqrt", "sin", "cos", "abs", "relu", "sigmoid", "tanh", "gelu", "erf", "step"):
    _PROTOS[f"pg_jit_{_op}"] = (ip, [vp, ip])

_AMD_PROTOS = {
    "pg_amd_init": (ip, []),
    "pg_amd_stream": (vp, []),
    "pg_amd_sync": (ip, []),
    "pg_amd_last_error": (C.c_char_p, []),
    "pg_amd_bytes_in_use": (sz, []),
    "pg_amd_bytes_cached": (sz, []),
    "pg_amd_release_cached": (None, []),
    "pg_amd_backward_from": (None, [vp, vp]),
    "pg_amd_ag_matmul16": (vp, [vp, vp, ip]),
    "pg_amd_ag_linear16": (vp, [vp, vp, vp, ip, ip]),
    "pg_amd_linear16_preact": (vp, [vp]),
    "pg_amd_linear16_keep_dz": (None, [bo]),
    "pg_amd_linear16_narrow": (None, [bo]),
    "pg_amd_jit_copies16": (None, [bo]),
    "pg_amd_linear16_dz": (vp, [vp]),
    "pg_amd_tensor_modified": (None, [vp]),
    "pg_amd_tensor_refresh16": (bo, [vp]),
    "pg_amd_tensor_to_dtype": (vp, [vp, ip]),
    "pg_amd_gemm_ex_noalloc": (ip, [ip, sz, sz, sz, vp, sz, vp, sz, vp, sz]),
    "pg_amd_sgd_buffer": (vp, [vp, sz]),
    "pg_tensor_clone": (vp, [vp]),
    "pg_tensor_view": (vp, [vp]),
    "pg_tensor_copy_from": (None, [vp, vp]),
    "pg_amd_jit_compiles": (sz, []),
    "pg_amd_jit_cache_hits": (sz, []),
    "pg_tensor_sync_host": (bo, [vp]),
    "pg_tensor_sync_device": (bo, [vp]),
    "pg_tensor_copy_to_host": (bo, [vp, vp]),
    "pg_tensor_copy_from_host": (bo, [vp, vp]),
    "pg_tensor_empty_dtype": (vp, [ip, sz, SZP]),
    "pg_tensor_full_dtype": (vp, [ip, sz, SZP, fl]),
    "pg_amd_timer_enable": (None, [ip]),
    "pg_amd_mfma_probe": (C.c_double, [ip]),
    "pg_amd_gemm16_plan": (ip, [ip, ip, sz, sz, sz, sz, ip, C.POINTER(C.c_int), C.POINTER(C.c_double)]),
    "pg_amd_timer_read": (C.c_double, [ip, C.POINTER(C.c_size_t)]),
    "pg_amd_timer_reset": (None, []),
    "pg_amd_params_save": (bo, [C.POINTER(vp), sz, C.c_char_p]),
    "pg_amd_params_load_into": (bo, [C.POINTER(vp), sz, C.c_char_p]),
    "pg_amd_sgd_save": (bo, [vp, C.c_char_p]),
    "pg_amd_sgd_load_into": (bo, [vp, C.c_char_p]),
    "pg_amd_adam_save": (bo, [vp, C.c_char_p]),
    "pg_amd_adam_load_into": (bo, [vp, C.c_char_p]),
}


def shape_arg(shape) -> tuple[int, C.Array]:
    shape = tuple(int(s) for s in shape)
    return len(shape), (C.c_size_t * max(1, len(shape)))(*shape)


class PgLib:
    """Typed handle on a library exporting the picograd ABI."""

    def __init__(self, path: str | Path, device: bool):
        self.path = str(path)
        self.device = device
        self.lib = C.CDLL(self.path)
        protos = dict(_PROTOS)
        if device:
            protos.update(_AMD_PROTOS)
        for name, (res, args) in protos.items():
            fn = getattr(self.lib, name)
            fn.restype = res
            fn.argtypes = args
            setattr(self, name, fn)
        self._tensor_t = PgTensorAmd if device else PgTensor

    # ---- tensors
    def tinfo(self, t: int) -> PgTensor:
        if not t:
            raise ValueError("null tensor")
        return self._tensor_t.from_address(t)

    def shape(self, t: int) -> tuple[int, ...]:
        ti = self.tinfo(t)
        return tuple(ti.shape[i] for i in range(ti.ndim))

    def read(self, t: int) -> np.ndarray:
        """Copy of a tensor's elements (f32, or uint16 bits for f16/bf16)."""
        ti = self.tinfo(t)
        dt = _NP_OF[ti.dtype]
        shape = tuple(ti.shape[i] for i in range(ti.ndim))
        out = np.empty(shape, dtype=dt)
        if self.device:
            if not self.pg_tensor_copy_to_host(t, out.ctypes.data):
                raise RuntimeError(f"pg_tensor_copy_to_host: {self.pg_amd_last_error().decode()}")
        else:
            C.memmove(out.ctypes.data, ti.data, out.nbytes)
        return out

    def tensor(self, arr: np.ndarray, dtype: int = F32) -> int:
        arr = np.ascontiguousarray(arr, dtype=_NP_OF[dtype])
        nd, sh = shape_arg(arr.shape if arr.ndim else (1,))
        t = self.pg_tensor_from_data_dtype(dtype, nd, sh, arr.ctypes.data)
        if not t:
            raise RuntimeError("pg_tensor_from_data_dtype failed")
        return t

    # ---- nodes
    def node(self, n: int) -> PgNode:
        if not n:
            raise ValueError(f"null node: {self.pg_autograd_last_error().decode()}")
        return PgNode.from_address(n)

    def var(self, arr: np.ndarray, requires_grad: bool = True, dtype: int = F32) -> int:
        """Leaf node holding `arr` (uint16 bits for f16/bf16)."""
        if dtype == F32:
            arr = np.ascontiguousarray(arr, dtype=np.float32)
            nd, sh = shape_arg(arr.shape)
            n = self.pg_var_from_data(nd, sh, arr.ctypes.data, requires_grad)
            return self._check(n)
        t = self.tensor(arr, dtype)
        if self.device:
            n = self.pg_var_from_tensor(t, requires_grad)
            self.pg_tensor_free(t)
            return self._check(n)
        # the reference has no 16-bit leaf constructor: swap a zeros leaf's value
        nd, sh = shape_arg(arr.shape)
        n = self._check(self.pg_var_zeros(nd, sh, requires_grad))
        node = PgNode.from_address(n)
        old = node.value
        node.value = t
        self.pg_tensor_free(old)
        return n

    def _check(self, n: int) -> int:
        if not n:
            raise RuntimeError(f"picograd call failed: {self.pg_autograd_last_error().decode()}")
        return n

    def value(self, n: int) -> np.ndarray:
        return self.read(self.node(n).value)

    def grad(self, n: int) -> np.ndarray | None:
        g = self.node(n).grad
        return None if not g else self.read(g)

    def op(self, name: str, *args) -> int:
        return self._check(getattr(self, f"pg_ag_{name}")(*args))

    def sync(self) -> None:
        if self.device and self.pg_amd_sync() != 0:
            raise RuntimeError(f"device sync failed: {self.pg_amd_last_error().decode()}")


_DEFAULT_LIB = Path(__file__).resolve().parent / "lib" / "libpicograd_amd.so"


def load(path: str | Path | None = None) -> PgLib:
    """The MI355X library.  Raises if it has not been built: nothing falls
    back to a CPU path."""
    p = Path(path) if path else _DEFAULT_LIB
    if not p.exists():
        raise FileNotFoundError(f"{p} is missing: run `python -m picograd_amd.build` first")
    return PgLib(p, device=True)
