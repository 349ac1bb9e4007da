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

Every element of every output is checked against the f64 product of the
same 16-bit operands within the f32 summation bound (gemm_check), with the
relative Frobenius error held to 1e-5 (identical operands, summation order
only); exact linearity in the upstream grad and bit-for-bit determinism
are checked as well.
"""
import ctypes as C

import numpy as np
import pytest

from gemm_check import check_linear, check_product
from oracle_lib import bf16_to_f32, f16_to_f32
from picograd_amd.capi import BF16, F16

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
    fa, fw, fg = _to_f32(dt, a), _to_f32(dt, w), _to_f32(dt, g)
    check_product(out, [(fa, fw)], "forward A.W")
    check_product(da, [(fg, fw.T)], "dgrad dC.W^T")
    check_product(dw, [(fa.T, fg)], "wgrad A^T.dC")
    del fa, fw, fg
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
    z = lib.read(lib.pg_amd_linear16_preact(out))
    qx, qw = _to_f32(dt, oracle.cast16(dt, x)), _to_f32(dt, oracle.cast16(dt, wt))
    check_linear(got, z, [(qx, qw)], b, 2, "linear16 gelu epilogue")
    for n in (out, nx, nw, nb):
        lib.pg_node_free(n)


@pytest.mark.parametrize("dt", [BF16, F16])
def test_whole_chip_pair_accumulates(lib, oracle, dt):
    """A matmul whose dgrad and wgrad each fill the chip (4096^3 bf16 or f16: 256
    tiles of 256 x 256 each) runs both as one paired launch; used twice with
    two upstream grads, the second backward accumulates into both grads
    (beta = 1).  dX = q(G1).W^T + q(G2).W^T and dW = X^T.q(G1) + X^T.q(G2),
    every element; a repeat reproduces every bit."""
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
    fx, fw, f1, f2 = (_to_f32(dt, h) for h in (x16, w16, g1, g2))
    check_product(dx, [(f1, fw.T), (f2, fw.T)], "pair dX = G1.W^T + G2.W^T")
    check_product(dw, [(fx.T, f1), (fx.T, f2)], "pair dW = X^T.G1 + X^T.G2")
    del fx, fw, f1, f2
    dx2, dw2 = run()
    assert np.array_equal(dx2, dx) and np.array_equal(dw2, dw)
