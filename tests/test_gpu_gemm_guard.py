"""Writes past C: the MFMA GEMM launches with guard rows and slack columns
around the output, as the reference's tests/test_gemm.c:95-189 checks its
CPU kernels (ld slack and canaries around C).

Each case calls the kernel layer (pgk_gemm16_cu, pgk_gemm16_pair_dw: the
launches every matmul grad and pg_gemm_ex go through) with C placed inside
a larger buffer: GUARD rows above and below, and ldc = n + SLACK columns.
The whole buffer starts as a NaN sentinel; afterwards the guard rows and
slack columns must hold the sentinel bit for bit, and every element of C
must match the f64 product of the same operands within the f32 summation
bound (gemm_check.check_product).  Shapes: the ragged M = 4097 with
N = 10 and 33 (the skinny kernel for at most 16 columns, split-K outputs
summed one element per thread past that) and N = 3000, the skinny kernel at
widths 1 to 16 and reductions from 8 to 9000, every operand layout
(forward, dgrad, wgrad), K % 64 != 0 and
K % 8 != 0 (the zero-page tail and the padded k-slab launch), beta 0 and
beta 1, the whole chip and a CU budget, and the paired dgrad + wgrad launch
(split between CUs, and whole-chip).
"""
import ctypes as C

import numpy as np
import pytest

from gemm_check import check_product
from oracle_lib import bf16_to_f32, f16_to_f32
from picograd_amd.capi import BF16, F16

pytestmark = pytest.mark.gpu

GUARD, SLACK = 5, 7
SENTINEL = np.array([0x7FC0DEAD], np.uint32).view(np.float32)[0]  # a quiet NaN


class GemmDesc(C.Structure):
    _fields_ = [("m", C.c_size_t), ("n", C.c_size_t), ("k", C.c_size_t),
                ("a", C.c_void_p), ("lda", C.c_size_t), ("stride_a", C.c_size_t), ("a_extent", C.c_size_t),
                ("b", C.c_void_p), ("ldb", C.c_size_t), ("stride_b", C.c_size_t), ("b_extent", C.c_size_t),
                ("c", C.c_void_p), ("ldc", C.c_size_t), ("stride_c", C.c_size_t), ("batch", C.c_size_t),
                ("beta", C.c_int)]


@pytest.fixture(scope="module")
def k(lib):
    L = lib.lib
    L.pgd_malloc.restype, L.pgd_malloc.argtypes = C.c_void_p, [C.c_size_t]
    L.pgd_free.restype, L.pgd_free.argtypes = None, [C.c_void_p, C.c_size_t]
    L.pgd_h2d.restype, L.pgd_h2d.argtypes = C.c_bool, [C.c_void_p, C.c_void_p, C.c_size_t]
    L.pgd_d2h.restype, L.pgd_d2h.argtypes = C.c_bool, [C.c_void_p, C.c_void_p, C.c_size_t]
    L.pgd_stream.restype, L.pgd_stream.argtypes = C.c_void_p, []
    sz, vp = C.c_size_t, C.c_void_p
    L.pgk_gemm16_cu.restype = C.c_int
    L.pgk_gemm16_cu.argtypes = [C.c_int, C.c_int, C.c_int, sz, sz, sz, vp, sz, sz, sz, vp, sz, sz, sz, vp, sz, sz,
                                sz, C.c_int, vp, vp, C.c_int, vp]
    L.pgk_gemm16_workspace_cu.restype = sz
    L.pgk_gemm16_workspace_cu.argtypes = [C.c_int, C.c_int, sz, sz, sz, sz, C.c_int]
    L.pgk_gemm16_time.restype = C.c_double
    L.pgk_gemm16_time.argtypes = [C.c_int, C.c_int, sz, sz, sz, sz, C.c_int]
    L.pgk_gemm16_plan.restype = C.c_int
    L.pgk_gemm16_plan.argtypes = [C.c_int, C.c_int, sz, sz, sz, sz, C.c_int, C.POINTER(C.c_int)]
    L.pgk_gemm16_pair_dw.restype = C.c_int
    L.pgk_gemm16_pair_dw.argtypes = [C.c_int, C.POINTER(GemmDesc), C.POINTER(GemmDesc), C.c_int, vp, vp]
    L.pgk_gemm16_pair_dw_workspace.restype = sz
    L.pgk_gemm16_pair_dw_workspace.argtypes = [C.POINTER(GemmDesc), C.POINTER(GemmDesc), C.c_int,
                                               C.POINTER(C.c_size_t)]
    return L


class Dev:
    """Device buffers from the library allocator, freed together."""

    def __init__(self, L):
        self.L, self.bufs = L, []

    def put(self, arr: np.ndarray) -> int:
        arr = np.ascontiguousarray(arr)
        p = self.alloc(arr.nbytes)
        assert self.L.pgd_h2d(p, arr.ctypes.data, arr.nbytes)
        return p

    def alloc(self, nbytes: int) -> int:
        p = self.L.pgd_malloc(max(nbytes, 1))
        assert p, "pgd_malloc failed"
        self.bufs.append((p, max(nbytes, 1)))
        return p

    def get(self, p: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert self.L.pgd_d2h(out.ctypes.data, p, out.nbytes)
        return out

    def free(self):
        for p, n in self.bufs:
            self.L.pgd_free(p, n)
        self.bufs = []


def _up8(x):
    return (x + 7) // 8 * 8


def _operands(oracle, rng, dt, ta, tb, m, n, kk):
    """Logical A [m, kk], B [kk, n] (16-bit bits), and their stored forms
    (layout ta / tb, leading dims padded past the minimum) with the extents
    the kernel may read."""
    cast = lambda x: oracle.cast16(dt, x)  # noqa: E731
    A = cast(rng.standard_normal((m, kk)).astype(np.float32))
    B = cast((0.05 * rng.standard_normal((kk, n))).astype(np.float32))
    if ta:  # a[p * lda + i], extent a multiple of 8 >= m
        lda = _up8(m) + 8
        a_st = np.zeros((kk, lda), np.uint16)
        a_st[:, :m] = A.T
        a_ext = _up8(m)
    else:
        lda = _up8(kk) + 16
        a_st = np.zeros((m, lda), np.uint16)
        a_st[:, :kk] = A
        a_ext = m
    if tb:  # b[p * ldb + j]
        ldb = _up8(n) + 8
        b_st = np.zeros((kk, ldb), np.uint16)
        b_st[:, :n] = B
        b_ext = _up8(n)
    else:  # b[j * ldb + p]
        ldb = _up8(kk) + 8
        b_st = np.zeros((n, ldb), np.uint16)
        b_st[:, :kk] = B.T
        b_ext = n
    return A, B, a_st, lda, a_ext, b_st, ldb, b_ext


def _f32(dt, h):
    return f16_to_f32(h) if dt == F16 else bf16_to_f32(h)


def _c_buffer(rng, m, n, beta):
    ldc = n + SLACK
    buf = np.full((GUARD + m + GUARD, ldc), SENTINEL, np.float32)
    c0 = rng.standard_normal((m, n)).astype(np.float32) if beta else None
    if beta:
        buf[GUARD:GUARD + m, :n] = c0
    return buf, ldc, c0


def _check_guards(buf_after, m, n, what):
    u = buf_after.view(np.uint32)
    s = np.array([SENTINEL], np.float32).view(np.uint32)[0]
    assert (u[:GUARD] == s).all(), f"{what}: guard rows above C written"
    assert (u[GUARD + m:] == s).all(), f"{what}: guard rows below C written"
    assert (u[GUARD:GUARD + m, n:] == s).all(), f"{what}: slack columns past n written"


CASES = [
    # dt, ta, tb, m, n, k, beta, cus
    (BF16, 0, 1, 4097, 10, 4096, 0, 0),
    (BF16, 0, 1, 4097, 33, 4096, 1, 0),
    (F16, 0, 0, 4097, 10, 1000, 0, 0),
    (F16, 0, 0, 4097, 33, 1004, 1, 0),
    (BF16, 1, 1, 1000, 33, 4097, 0, 0),
    (F16, 1, 1, 1000, 10, 4097, 1, 0),
    (F16, 0, 0, 4097, 3000, 1000, 0, 0),
    (F16, 1, 1, 1000, 3000, 4097, 1, 96),
    (BF16, 0, 1, 4097, 3000, 1004, 0, 160),
    # the skinny kernel (n <= 16, B MN-contiguous, 64 or more 16-row
    # blocks; the 1000-row cases above take split-K): widths 1, 8 and 16, a
    # reduction shorter than one chunk, one ending mid-chunk, a long one,
    # config 5's 10-wide weight grad, beta 1
    (F16, 0, 1, 1040, 16, 136, 1, 0),
    (BF16, 0, 1, 2048, 1, 8, 0, 0),
    (BF16, 1, 1, 4096, 10, 4096, 0, 0),
    (F16, 1, 1, 1032, 8, 77, 0, 0),
    (BF16, 1, 1, 1024, 16, 9000, 1, 0),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "dt%d-ta%d-tb%d-%dx%dx%d-beta%d-cus%d" % c)
def test_gemm_guards(lib, oracle, k, case):
    dt, ta, tb, m, n, kk, beta, cus = case
    what = "gemm dt=%d ta=%d tb=%d %dx%dx%d beta=%d cus=%d" % case
    print(what, flush=True)
    rng = np.random.default_rng(abs(hash(case)) % 2**32)
    A, B, a_st, lda, a_ext, b_st, ldb, b_ext = _operands(oracle, rng, dt, ta, tb, m, n, kk)
    buf, ldc, c0 = _c_buffer(rng, m, n, beta)
    d = Dev(k)
    try:
        pa, pb, pc = d.put(a_st), d.put(b_st), d.put(buf)
        wsz = k.pgk_gemm16_workspace_cu(ta, tb, m, n, kk, 1, cus)
        ws = d.alloc(wsz) if wsz else None
        rc = k.pgk_gemm16_cu(dt, ta, tb, m, n, kk, pa, lda, 0, a_ext, pb, ldb, 0, b_ext, pc + GUARD * ldc * 4, ldc,
                             0, 1, beta, None, ws, cus, k.pgd_stream())
        assert rc == 0, rc
        after = d.get(pc, buf.shape, np.float32)
    finally:
        d.free()
    _check_guards(after, m, n, what)
    check_product(after[GUARD:GUARD + m, :n], [(_f32(dt, A), _f32(dt, B))], what, add=c0)


@pytest.mark.parametrize("dt", [F16, BF16])
@pytest.mark.parametrize("shape", [(4097, 1000, 3000, 1), (4096, 4096, 4096, 0)], ids=["cu-split", "whole-chip"])
def test_pair_guards(lib, oracle, k, dt, shape):
    """The paired dgrad + wgrad launch of one matmul C = X.W, X [M, K],
    W [K, N]: dX = G.W^T (dgrad: both operands K-contiguous, reduction N)
    and dW = X^T.G (wgrad: both MN-contiguous, reduction M), each into a
    guarded output, the second accumulating (beta 1)."""
    M, K, N, cu_d = shape
    what = f"pair dt={dt} M={M} K={K} N={N} cu_d={cu_d}"
    print(what, flush=True)
    rng = np.random.default_rng(M + dt)
    X = oracle.cast16(dt, rng.standard_normal((M, K)).astype(np.float32))
    W = oracle.cast16(dt, (0.05 * rng.standard_normal((K, N))).astype(np.float32))
    G = oracle.cast16(dt, rng.standard_normal((M, N)).astype(np.float32))
    if cu_d:  # the CU split the library's matmul backward picks (its time model)
        best = None
        for cd in range(32, 225, 32):
            t = max(k.pgk_gemm16_time(0, 0, M, K, N, 1, cd), k.pgk_gemm16_time(1, 1, K, N, M, 1, 256 - cd))
            if best is None or t < best[0]:
                best = (t, cd)
        cu_d = best[1]
    sp = C.c_int(0)
    assert k.pgk_gemm16_plan(0, 0, M, K, N, 1, cu_d, C.byref(sp)) == \
        k.pgk_gemm16_plan(1, 1, K, N, M, 1, 256 - cu_d if cu_d else 0, C.byref(sp)), "plans on different tiles"
    bx, ldx, _ = _c_buffer(rng, M, K, 0)
    bw, ldw, c0w = _c_buffer(rng, K, N, 1)
    d = Dev(k)
    try:
        pg, pw, px = d.put(G), d.put(W), d.put(X)
        cx, cw = d.put(bx), d.put(bw)
        dd = GemmDesc(M, K, N, pg, N, 0, M, pw, N, 0, K, cx + GUARD * ldx * 4, ldx, 0, 1, 0)
        dwd = GemmDesc(K, N, M, px, K, 0, K, pg, N, 0, N, cw + GUARD * ldw * 4, ldw, 0, 1, 1)
        off = C.c_size_t(0)
        wsz = k.pgk_gemm16_pair_dw_workspace(C.byref(dd), C.byref(dwd), cu_d, C.byref(off))
        ws = d.alloc(wsz) if wsz else None
        rc = k.pgk_gemm16_pair_dw(dt, C.byref(dd), C.byref(dwd), cu_d, ws, k.pgd_stream())
        assert rc == 0, rc
        ax = d.get(cx, bx.shape, np.float32)
        aw = d.get(cw, bw.shape, np.float32)
    finally:
        d.free()
    _check_guards(ax, M, K, what + " dX")
    _check_guards(aw, K, N, what + " dW")
    f = lambda h: _f32(dt, h)  # noqa: E731
    check_product(ax[GUARD:GUARD + M, :K], [(f(G), f(W).T)], what + " dX")
    check_product(aw[GUARD:GUARD + K, :N], [(f(X).T, f(G))], what + " dW", add=c0w)
