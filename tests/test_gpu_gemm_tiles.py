"""The 256 x 256-tile MFMA GEMM path (eight waves, global -> LDS ring) in
each operand layout the autograd uses, at shapes large enough that the
launch plan picks it (at least 128 such tiles, no split-K), with ragged
edges in every dim:

- forward C = A . W (A K-contiguous, W MN-contiguous): M = 2900 rows (a
  partial last tile row), K = 3000 (a partial last k-tile, K % 8 == 0);
- dgrad dA = dC . W^T (both K-contiguous): K = 3080;
- wgrad dW = A^T . dC (both MN-contiguous): K = 2900, K % 8 == 4, the
  last k-tile reading zero rows past K;
- the fused bias + GELU epilogue on the forward layout (pg_amd_ag_linear16).

The oracle checks sampled rows and columns (each against the
f32-accumulating product of the same 16-bit operands, relative Frobenius
<= 1e-5: identical operands, summation order only); exact linearity in the
upstream grad and bit-for-bit determinism cover the rest.
"""
import ctypes as C

import numpy as np
import pytest

from oracle_lib import bf16_to_f32, f16_to_f32, rel_fro
from picograd_amd.capi import BF16, F16, F32

pytestmark = pytest.mark.gpu

M, K, N = 2900, 3000, 3080


def _to_f32(dt, h):
    return f16_to_f32(h) if dt == F16 else bf16_to_f32(h)


def _backward(lib, dt, a16, w16, g16, scale=1.0):
    na, nw = lib.var(a16, dtype=dt), lib.var(w16, dtype=dt)
    c = lib.op("matmul", na, nw)
    out = lib.value(c)
    seed = lib.tensor(_to_f32(dt, g16) * np.float32(scale))
    lib.pg_amd_backward_from(c, seed)
    da, dw = lib.grad(na), lib.grad(nw)
    lib.pg_tensor_free(seed)
    for n in (c, na, nw):
        lib.pg_node_free(n)
    return out, da, dw


@pytest.mark.parametrize("dt", [BF16, F16])
def test_big_tile_matmul_all_layouts(lib, oracle, dt):
    print(f"gemm 256-tile matmul fwd/bwd dt={dt} {M}x{K}x{N}", flush=True)
    oracle.orc_seed(50 + dt)
    a = oracle.cast16(dt, oracle.normal(M * K, 0.0, 1.0).reshape(M, K))
    w = oracle.cast16(dt, oracle.normal(K * N, 0.0, 0.02).reshape(K, N))
    g = oracle.cast16(dt, oracle.normal(M * N, 0.0, 1.0).reshape(M, N))
    out, da, dw = _backward(lib, dt, a, w, g)
    assert out.shape == (M, N) and da.shape == (M, K) and dw.shape == (K, N)
    rng = np.random.default_rng(dt)
    rows = np.unique(np.concatenate([rng.choice(M, 40, replace=False), [0, 255, 256, 2815, 2816, M - 1]]))
    # forward rows: C[r, :] = A[r, :] . W
    ref = oracle.gemm(dt, np.ascontiguousarray(a[rows]), w, threads=16)
    assert rel_fro(out[rows], ref) <= 1e-5
    # dgrad rows: dA[r, :] = dC[r, :] . W^T
    ref = oracle.gemm(dt, np.ascontiguousarray(g[rows]), w, tb=True, threads=16)
    assert rel_fro(da[rows], ref) <= 1e-5
    # wgrad rows: dW[k, :] = A[:, k]^T . dC
    ks = np.unique(np.concatenate([rng.choice(K, 24, replace=False), [0, 2815, 2816, K - 1]]))
    ref = oracle.gemm(dt, np.ascontiguousarray(a[:, ks]), g, ta=True, threads=16)
    assert rel_fro(dw[ks], ref) <= 1e-5
    # columns at tile edges, all rows
    js = np.array([0, 255, 256, 3071, 3072, N - 1])
    ref = oracle.gemm(dt, a, np.ascontiguousarray(w[:, js]), threads=16)
    assert rel_fro(out[:, js], ref) <= 1e-5
    ref = oracle.gemm(dt, a, np.ascontiguousarray(g[:, js]), ta=True, threads=16)
    assert rel_fro(dw[:, js], ref) <= 1e-5
    # exact linearity in the upstream grad, and determinism
    _, da2, dw2 = _backward(lib, dt, a, w, g, scale=2.0)
    assert np.array_equal(da2, 2 * da) and np.array_equal(dw2, 2 * dw)
    out3, da3, dw3 = _backward(lib, dt, a, w, g)
    assert np.array_equal(out3, out) and np.array_equal(da3, da) and np.array_equal(dw3, dw)


@pytest.mark.parametrize("dt", [BF16, F16])
def test_big_tile_fused_epilogue(lib, oracle, dt):
    """out = gelu(q(x) . q(W) + b) from one launch with the epilogue fused
    (K = 520: no k-tail, no split)."""
    kk = 520
    print(f"gemm 256-tile linear16 gelu dt={dt} {M}x{kk}x{N}", flush=True)
    rng = np.random.default_rng(60 + dt)
    x = rng.standard_normal((M, kk)).astype(np.float32)
    wt = (rng.standard_normal((kk, N)) / np.sqrt(kk)).astype(np.float32)
    b = (0.3 * rng.standard_normal(N)).astype(np.float32)
    nx, nw, nb = lib.var(x), lib.var(wt), lib.var(b)
    out = lib._check(lib.pg_amd_ag_linear16(nx, nw, nb, 2, dt))
    got = lib.value(out)
    rows = np.unique(np.concatenate([rng.choice(M, 32, replace=False), [0, 2815, 2816, M - 1]]))
    qx = _to_f32(dt, oracle.cast16(dt, np.ascontiguousarray(x[rows])))
    qw = _to_f32(dt, oracle.cast16(dt, wt))
    z = oracle.gemm(F32, qx, qw).astype(np.float64) + b
    from math import erf
    want = 0.5 * z * (1.0 + np.vectorize(erf)(z / np.sqrt(2.0)))
    assert rel_fro(got[rows], want) <= 1e-5
    for n in (out, nx, nw, nb):
        lib.pg_node_free(n)


@pytest.mark.parametrize("dt", [BF16, F16])
def test_whole_chip_pair_accumulates(lib, oracle, dt):
    """A matmul whose dgrad and wgrad each fill the chip (4096^3 bf16 or f16: 256
    tiles of 256 x 256 each) runs both as one paired launch; used twice with
    two upstream grads, the second backward accumulates into both grads
    (beta = 1).  dX = q(G1).W^T + q(G2).W^T and dW = X^T.q(G1) + X^T.q(G2)
    against the oracle on sampled rows and columns; a repeat reproduces every
    bit."""
    n = 4096
    print(f"whole-chip dgrad + wgrad pair, 4096^3 dt={dt}, used twice (beta = 1)", flush=True)
    rng = np.random.default_rng(4096)
    x16 = oracle.cast16(dt, rng.standard_normal((n, n)).astype(np.float32))
    w16 = oracle.cast16(dt, (0.02 * rng.standard_normal((n, n))).astype(np.float32))
    g1 = oracle.cast16(dt, rng.standard_normal((n, n)).astype(np.float32))
    g2 = oracle.cast16(dt, rng.standard_normal((n, n)).astype(np.float32))
    for ta in (0, 1):  # both plan 256 x 256 tiles without split-K: the pair launch
        sp, sec = C.c_int(0), C.c_double(0.0)
        assert lib.pg_amd_gemm16_plan(ta, ta, n, n, n, 1, 0, C.byref(sp), C.byref(sec)) == 2 and sp.value == 1

    def run():
        nx, nw = lib.var(x16, dtype=dt), lib.var(w16, dtype=dt)
        c1, c2 = lib.op("matmul", nx, nw), lib.op("matmul", nx, nw)
        ng1 = lib.var(_to_f32(dt, g1), requires_grad=False)
        ng2 = lib.var(_to_f32(dt, g2), requires_grad=False)
        p1, p2 = lib.op("mul", c1, ng1), lib.op("mul", c2, ng2)
        s1, s2 = lib.op("sum_all", p1), lib.op("sum_all", p2)
        loss = lib.op("add", s1, s2)
        lib.pg_backward(loss)
        dx, dw = lib.grad(nx), lib.grad(nw)
        for node in (loss, s2, s1, p2, p1, ng2, ng1, c2, c1, nw, nx):
            lib.pg_node_free(node)
        return dx, dw

    dx, dw = run()
    rows = np.array([0, 1, 255, 256, 2047, 2048, 4095])
    cols = np.array([0, 255, 256, 3000, 4095])
    gx = lambda g, r: oracle.gemm(dt, np.ascontiguousarray(g[r]), w16, tb=True, threads=16)  # noqa: E731
    assert rel_fro(dx[rows], gx(g1, rows) + gx(g2, rows)) <= 1e-5
    gw = lambda g, k: oracle.gemm(dt, np.ascontiguousarray(x16[:, k]), g, ta=True, threads=16)  # noqa: E731
    assert rel_fro(dw[rows], gw(g1, rows) + gw(g2, rows)) <= 1e-5
    gwc = lambda g: oracle.gemm(dt, x16, np.ascontiguousarray(g[:, cols]), ta=True, threads=16)  # noqa: E731
    assert rel_fro(dw[:, cols], gwc(g1) + gwc(g2)) <= 1e-5
    dx2, dw2 = run()
    assert np.array_equal(dx2, dx) and np.array_equal(dw2, dw)
