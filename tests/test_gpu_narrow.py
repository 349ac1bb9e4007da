"""Products with a narrow output (n <= 16 columns, as config 5's 10-wide
layer): with rows enough for 32 blocks of 32 the skinny kernel (one launch,
the epilogue applied per element after the waves' partial sums), else
split-K over 128 x 128 MFMA tiles with the epilogue applied by the summing
launch.  Each output against the f32-accumulating product of the same
16-bit operands (identical operands, only the summation order differs:
relative Frobenius <= 1e-5), through pg_amd_ag_linear16 (bias + GELU
epilogue, the pre-activation kept for the backward, whose bias grad must
match, and the weight grad over the dz the backward formed) and through
matmul16 (no epilogue), at ragged row counts, k not a multiple of the
k-tile, and widths 1, 10 and 16; a repeat reproduces every bit.
"""
from math import erf

import numpy as np
import pytest

from oracle_lib import bf16_to_f32, f16_to_f32, rel_fro
from picograd_amd.capi import BF16, F16, F32

pytestmark = pytest.mark.gpu


def _q(oracle, dt, x):
    h = oracle.cast16(dt, np.ascontiguousarray(x))
    return f16_to_f32(h) if dt == F16 else bf16_to_f32(h)


def _f32q(dt, h):
    return f16_to_f32(h) if dt == F16 else bf16_to_f32(h)


def _gelu(z):
    return 0.5 * z * (1.0 + np.vectorize(erf)(z / np.sqrt(2.0)))


@pytest.mark.parametrize("dt", [BF16, F16])
@pytest.mark.parametrize("M,K,N", [(4096, 4096, 10), (1037, 1544, 16), (70, 24, 1)])
def test_narrow_linear16_forward_and_grads(lib, oracle, dt, M, K, N):
    print(f"narrow linear16 gelu dt={dt} {M}x{K}x{N}", flush=True)
    rng = np.random.default_rng(M + N + dt)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    b = (0.3 * rng.standard_normal(N)).astype(np.float32)
    g = rng.standard_normal((M, N)).astype(np.float32)
    nx, nw, nb = lib.var(x), lib.var(w), lib.var(b)
    out = lib._check(lib.pg_amd_ag_linear16(nx, nw, nb, 2, dt))
    got = lib.value(out)
    qx, qw = _q(oracle, dt, x), _q(oracle, dt, w)
    z = oracle.gemm(F32, qx, qw, threads=16).astype(np.float64) + b
    assert rel_fro(got, _gelu(z)) <= 1e-5
    # the backward reads the kept pre-activation: db = sum of dz over rows;
    # dW = q(x)^T . dz over the 16-bit dz the backward formed (read back)
    seed = lib.tensor(g)
    lib.pg_amd_linear16_keep_dz(True)
    try:
        lib.pg_amd_backward_from(out, seed)
        dz = _f32q(dt, lib.read(lib.pg_amd_linear16_dz(out)))[:, :N]
    finally:
        lib.pg_amd_linear16_keep_dz(False)
    db = lib.grad(nb)
    dgelu = 0.5 * (1.0 + np.vectorize(erf)(z / np.sqrt(2.0))) + z * np.exp(-0.5 * z * z) / np.sqrt(2.0 * np.pi)
    assert rel_fro(db, (g * dgelu).sum(axis=0)) <= 1e-4
    dw = lib.grad(nw)
    assert rel_fro(dw, oracle.gemm(F32, np.ascontiguousarray(qx.T), np.ascontiguousarray(dz), threads=16)) <= 1e-5
    lib.pg_tensor_free(seed)
    for n in (out, nx, nw, nb):
        lib.pg_node_free(n)


@pytest.mark.parametrize("dt", [BF16, F16])
def test_narrow_matmul16_accumulates(lib, oracle, dt):
    """y = q(X1).q(W) and q(X2).q(W) with W [K, 10] (one padded 16-bit copy
    of W serves both); a repeat reproduces every bit."""
    M, K, N = 3000, 2056, 10
    print(f"narrow matmul16 dt={dt} {M}x{K}x{N}", flush=True)
    rng = np.random.default_rng(7 + dt)
    x1 = rng.standard_normal((M, K)).astype(np.float32)
    x2 = rng.standard_normal((M, K)).astype(np.float32)
    w = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    n1, n2, nw = lib.var(x1, requires_grad=False), lib.var(x2, requires_grad=False), lib.var(w)

    def run():
        c1 = lib._check(lib.pg_amd_ag_matmul16(n1, nw, dt))
        c2 = lib._check(lib.pg_amd_ag_matmul16(n2, nw, dt))
        v1, v2 = lib.value(c1), lib.value(c2)
        for n in (c2, c1):
            lib.pg_node_free(n)
        return v1, v2

    v1, v2 = run()
    qw = _q(oracle, dt, w)
    assert rel_fro(v1, oracle.gemm(F32, _q(oracle, dt, x1), qw, threads=16)) <= 1e-5
    assert rel_fro(v2, oracle.gemm(F32, _q(oracle, dt, x2), qw, threads=16)) <= 1e-5
    r1, r2 = run()
    assert np.array_equal(r1, v1) and np.array_equal(r2, v2)
    for n in (nw, n2, n1):
        lib.pg_node_free(n)
