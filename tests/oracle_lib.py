"""ctypes handle on the CPU oracle (oracle/liboracle.so) -- the checker.

Test infrastructure only: tests, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use it; the product library never does.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_SO = ROOT / "oracle" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libpicograd_ref.so"
REF_CONVERT_SO = ROOT / "oracle" / "_ref" / "libref_convert.so"

_vp, _sz, _fl, _ip = C.c_void_p, C.c_size_t, C.c_float, C.c_int


class Oracle:
    def __init__(self, path: Path = ORACLE_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = C.CDLL(str(path))
        protos = {
            "orc_seed": (None, [C.c_ulonglong]),
            "orc_uniform": (None, [_vp, _sz, _fl, _fl]),
            "orc_normal": (None, [_vp, _sz, _fl, _fl]),
            "orc_f32_to_bf16": (C.c_uint16, [_fl]),
            "orc_bf16_to_f32": (_fl, [C.c_uint16]),
            "orc_f32_to_f16": (C.c_uint16, [_fl]),
            "orc_f16_to_f32": (_fl, [C.c_uint16]),
            "orc_cast_f32": (None, [_ip, _vp, _vp, _sz]),
            "orc_round_f32": (None, [_ip, _vp, _sz]),
            "orc_sgd_step": (None, [_vp, _vp, _vp, _sz, _fl, _fl, _fl, _fl, C.c_bool]),
            "orc_adam_bias_correction": (_fl, [_fl, C.c_ulonglong]),
            "orc_adam_step": (None, [_vp, _vp, _vp, _vp, _vp, _sz, _fl, _fl, _fl, _fl, _fl, C.c_bool, C.c_bool,
                                     C.c_ulonglong]),
            "orc_grad_norm": (_fl, [C.POINTER(_vp), C.POINTER(_sz), _sz]),
            "orc_clip_grad_norm": (_fl, [C.POINTER(_vp), C.POINTER(_sz), _sz, _fl, _fl]),
            "orc_clip_grad_value": (None, [C.POINTER(_vp), C.POINTER(_sz), _sz, _fl]),
            "orc_pgt1_write": (_sz, [_ip, _sz, C.POINTER(_sz), _vp, _vp, _sz]),
            "orc_pgt1_check": (_sz, [_vp, _sz]),
            "orc_gemm_acc32": (None, [_ip, _ip, _ip, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _ip, _ip]),
            "orc_gemm_acc64": (None, [_ip, _ip, _ip, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _ip]),
            "orc_chain1_backward": (None, [_vp, _vp, _vp, _sz, _vp, _vp, _vp]),
            "orc_chain2_backward": (None, [_vp, _vp, _vp, _sz, _sz, _vp, _vp, _vp, _vp]),
            "orc_gelu": (_fl, [_fl]),
            "orc_gelu_backward": (None, [_vp, _vp, _vp, _sz]),
            "orc_sigmoid": (_fl, [_fl]),
            "orc_mse_grad_scale": (_fl, [_sz, C.POINTER(_sz), C.c_bool]),
            "orc_mlp_step": (None, [_ip, _sz, C.POINTER(_sz), _sz, _vp, _vp, C.POINTER(_vp), C.POINTER(_vp),
                                    C.POINTER(_vp), C.POINTER(_vp), C.POINTER(_vp), C.POINTER(_vp), _fl, _fl,
                                    _fl, _fl, C.c_bool, C.POINTER(_fl), _ip]),
        }
        for name, (res, args) in protos.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
            setattr(self, name, fn)
        self.lib = L

    # ---- numpy conveniences
    def uniform(self, n: int, lo: float, hi: float) -> np.ndarray:
        out = np.empty(n, np.float32)
        self.orc_uniform(out.ctypes.data, n, lo, hi)
        return out

    def normal(self, n: int, mean: float, sd: float) -> np.ndarray:
        out = np.empty(n, np.float32)
        self.orc_normal(out.ctypes.data, n, mean, sd)
        return out

    def cast16(self, dtype: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.shape, np.uint16)
        self.orc_cast_f32(dtype, x.ctypes.data, out.ctypes.data, x.size)
        return out

    def gemm(self, dtype: int, a: np.ndarray, b: np.ndarray, ta=False, tb=False, f64=False,
             threads: int = 8) -> np.ndarray:
        """C = op(A) . op(B) with f32 (or f64) accumulation of upcast operands."""
        a = np.ascontiguousarray(a)
        b = np.ascontiguousarray(b)
        m = a.shape[1] if ta else a.shape[0]
        k = a.shape[0] if ta else a.shape[1]
        n = b.shape[0] if tb else b.shape[1]
        c = np.zeros((m, n), np.float64 if f64 else np.float32)
        if f64:
            self.orc_gemm_acc64(dtype, int(ta), int(tb), m, n, k, a.ctypes.data, a.shape[1],
                                b.ctypes.data, b.shape[1], c.ctypes.data, n, threads)
        else:
            self.orc_gemm_acc32(dtype, int(ta), int(tb), m, n, k, a.ctypes.data, a.shape[1],
                                b.ctypes.data, b.shape[1], c.ctypes.data, n, 0, threads)
        return c

    def sgd_step(self, p, g, buf, lr, mu, damp, wd, nesterov) -> None:
        self.orc_sgd_step(p.ctypes.data, g.ctypes.data, buf.ctypes.data if buf is not None else None,
                          p.size, lr, mu, damp, wd, nesterov)

    def adam_step(self, p, g, m, v, vmax, lr, beta1, beta2, eps, wd, amsgrad, decoupled, step) -> None:
        """One orc_adam_step over f32 arrays, in place (vmax may be None unless amsgrad)."""
        for a in (p, g, m, v) + ((vmax,) if vmax is not None else ()):
            assert a.dtype == np.float32 and a.flags.c_contiguous and a.size == p.size
        self.orc_adam_step(p.ctypes.data, g.ctypes.data, m.ctypes.data, v.ctypes.data,
                           vmax.ctypes.data if vmax is not None else None, p.size, lr, beta1, beta2, eps, wd,
                           bool(amsgrad), bool(decoupled), int(step))

    @staticmethod
    def _grad_list(gs):
        for g in gs:
            assert g is None or (g.dtype == np.float32 and g.flags.c_contiguous)
        ptrs = (C.c_void_p * len(gs))(*[g.ctypes.data if g is not None else None for g in gs])
        ns = (C.c_size_t * len(gs))(*[g.size if g is not None else 0 for g in gs])
        return ptrs, ns

    def grad_norm(self, gs) -> float:
        ptrs, ns = self._grad_list(gs)
        return self.orc_grad_norm(ptrs, ns, len(gs))

    def clip_grad_norm(self, gs, max_norm, eps) -> float:
        """In place over the arrays of gs (None entries skipped); returns the norm."""
        ptrs, ns = self._grad_list(gs)
        return self.orc_clip_grad_norm(ptrs, ns, len(gs), max_norm, eps)

    def clip_grad_value(self, gs, c) -> None:
        ptrs, ns = self._grad_list(gs)
        self.orc_clip_grad_value(ptrs, ns, len(gs), c)

    def pgt1_bytes(self, dtype: int, arr: np.ndarray) -> bytes:
        """The PGT1 record of arr (f32, or uint16 bits for f16/bf16)."""
        arr = np.ascontiguousarray(arr)
        shape = (C.c_size_t * max(1, arr.ndim))(*arr.shape)
        n = self.orc_pgt1_write(dtype, arr.ndim, shape, arr.ctypes.data, None, 0)
        out = (C.c_ubyte * n)()
        self.orc_pgt1_write(dtype, arr.ndim, shape, arr.ctypes.data, out, n)
        return bytes(out)

    def pgt1_check(self, blob: bytes) -> int:
        buf = (C.c_ubyte * max(1, len(blob))).from_buffer_copy(blob + b"\0" * (len(blob) == 0))
        return self.orc_pgt1_check(buf, len(blob))

    def gelu_backward(self, z, g):
        """g * gelu'(z) elementwise (f32 arrays of one shape)."""
        z = np.ascontiguousarray(z, np.float32)
        g = np.ascontiguousarray(g, np.float32)
        assert z.shape == g.shape
        out = np.empty_like(z)
        self.orc_gelu_backward(z.ctypes.data, g.ctypes.data, out.ctypes.data, z.size)
        return out

    def chain1(self, a, b, c):
        da, db, dc = (np.empty_like(a) for _ in range(3))
        self.orc_chain1_backward(a.ctypes.data, b.ctypes.data, c.ctypes.data, a.size,
                                 da.ctypes.data, db.ctypes.data, dc.ctypes.data)
        return da, db, dc

    def chain2(self, x, bias, g):
        R, Cc = x.shape
        dx, dg = np.empty_like(x), np.empty_like(g)
        db = np.empty(Cc, np.float32)
        db64 = np.empty(Cc, np.float64)
        self.orc_chain2_backward(x.ctypes.data, bias.ctypes.data, g.ctypes.data, R, Cc,
                                 dx.ctypes.data, dg.ctypes.data, db.ctypes.data, db64.ctypes.data)
        return dx, dg, db, db64

    def mlp_step(self, dtype: int, x, target, Ws, bs, Wbufs, bbufs, lr, mu, damp, wd, nesterov,
                 threads: int = 8):
        """One orc_mlp_step: updates Ws, bs, Wbufs, bbufs in place (f32 contiguous
        arrays); returns (loss, dWs, dbs)."""
        L = len(Ws)
        dims = [Ws[0].shape[0]] + [w.shape[1] for w in Ws]
        dWs = [np.empty_like(w) for w in Ws]
        dbs = [np.empty_like(b) for b in bs]
        arrs = [Ws, bs, Wbufs, bbufs, dWs, dbs]
        for group in arrs:
            for a in group:
                assert a.dtype == np.float32 and a.flags.c_contiguous
        ptrs = [(C.c_void_p * L)(*[a.ctypes.data for a in group]) for group in arrs]
        loss = C.c_float()
        self.orc_mlp_step(dtype, L, (C.c_size_t * (L + 1))(*dims), x.shape[0], x.ctypes.data,
                          target.ctypes.data, *ptrs, lr, mu, damp, wd, nesterov, C.byref(loss), threads)
        return loss.value, dWs, dbs


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    return h.view(np.float16).astype(np.float32)


def rel_fro(x: np.ndarray, ref: np.ndarray) -> float:
    x = x.astype(np.float64)
    ref = ref.astype(np.float64)
    return float(np.linalg.norm(x - ref) / max(np.linalg.norm(ref), 1e-300))


def pure_rel(x: np.ndarray, ref: np.ndarray) -> dict:
    """The unfloored elementwise relative error |x - ref| / |ref| over the
    elements with ref != 0: its maximum, 99.9th percentile and median, and
    the number of exact zeros of ref left out.  Reported beside max_rel: near
    a zero of GELU' or tanh' the pure measure is ~eps * 0.5 / |ref| for any
    f32 evaluation, so its maximum says where the zeros are rather than how
    good the kernel is; the percentiles show the bulk."""
    x = x.astype(np.float64).ravel()
    ref = ref.astype(np.float64).ravel()
    nz = ref != 0
    r = np.abs(x[nz] - ref[nz]) / np.abs(ref[nz])
    return {"max": float(r.max()) if r.size else 0.0, "p999": float(np.quantile(r, 0.999)) if r.size else 0.0,
            "median": float(np.median(r)) if r.size else 0.0, "zeros_left_out": int((~nz).sum())}


def max_rel(x: np.ndarray, ref: np.ndarray, floor_frac: float = 1e-2) -> float:
    """max |x - ref| / (|ref| + floor), floor = floor_frac * max|ref|.

    The elementwise relative error used for the f32 grads.  The floor keeps
    the measure meaningful where a grad passes through zero: GELU' and tanh'
    cancel terms of size ~0.5 there, so any f32 evaluation (the reference's
    included) carries ~eps * 0.5 absolute error that a pure relative measure
    would blow up.  With the 1e-5 bar this allows 1e-7 * max|ref| (about two
    f32 ulps of the largest grad) on elements below 1% of the largest, and
    1e-5 relative on the rest."""
    x = x.astype(np.float64)
    ref = ref.astype(np.float64)
    floor = floor_frac * max(float(np.abs(ref).max()), 1e-30)
    return float((np.abs(x - ref) / (np.abs(ref) + floor)).max())
