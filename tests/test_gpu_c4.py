"""Config 4 at its full shapes on the MI355X: the ragged f16 matmul backward
(M=4097, K=1000, N=3000) and the attention-style bmm backward
(32 x [512,128] . [128,512]), inputs drawn from the library RNG with the
reference's seed order (seed 45: A, B, dC, Q, K^T, dS).

The oracle checks sampled rows and columns of every grad (the full products
would take the CPU too long for a test), each against the f32-accumulating
product of the same f16 operands (relative Frobenius <= 1e-3 on the sample,
BASELINE.json north_star).  Size-independent properties cover the rest:
doubling the upstream grad doubles every grad bit for bit (scaling by 2 is
exact through the f16 rounding and the f32 accumulation), and a repeated
backward reproduces the grads bit for bit (the kernels are deterministic).
"""
import numpy as np
import pytest

from oracle_lib import f16_to_f32, rel_fro
from picograd_amd.capi import F16

pytestmark = pytest.mark.gpu

GEMM_TOL = 1e-3


@pytest.fixture(scope="module")
def c4(lib, oracle):
    oracle.orc_seed(45)
    M, K, N = 4097, 1000, 3000
    a = oracle.cast16(F16, oracle.normal(M * K, 0.0, 1.0).reshape(M, K))
    b = oracle.cast16(F16, oracle.normal(K * N, 0.0, 1.0).reshape(K, N))
    dc = oracle.cast16(F16, oracle.normal(M * N, 0.0, 1.0).reshape(M, N))
    sd = float(1.0 / np.sqrt(128.0))
    q = oracle.cast16(F16, oracle.normal(32 * 512 * 128, 0.0, sd).reshape(32, 512, 128))
    kt = oracle.cast16(F16, oracle.normal(32 * 128 * 512, 0.0, sd).reshape(32, 128, 512))
    ds = oracle.cast16(F16, oracle.normal(32 * 512 * 512, 0.0, 1.0).reshape(32, 512, 512))
    return dict(a=a, b=b, dc=dc, q=q, kt=kt, ds=ds)


def _backward(lib, x16, w16, g16, scale=1.0):
    nx, nw = lib.var(x16, dtype=F16), lib.var(w16, dtype=F16)
    c = lib.op("matmul", nx, nw)
    seed = lib.tensor(f16_to_f32(g16) * np.float32(scale))
    lib.pg_amd_backward_from(c, seed)
    dx, dw = lib.grad(nx), lib.grad(nw)
    lib.pg_tensor_free(seed)
    for n in (c, nx, nw):
        lib.pg_node_free(n)
    return dx, dw


def test_ragged_matmul_backward(lib, oracle, c4):
    a, b, dc = c4["a"], c4["b"], c4["dc"]
    print("c4 ragged f16 matmul 4097x1000x3000", flush=True)
    dA, dB = _backward(lib, a, b, dc)
    assert dA.shape == (4097, 1000) and dB.shape == (1000, 3000)
    rng = np.random.default_rng(4)
    rows = np.unique(np.concatenate([rng.choice(4097, 48, replace=False), [0, 4095, 4096]]))
    # dA[r, :] = dC[r, :] . B^T
    ref = oracle.gemm(F16, np.ascontiguousarray(dc[rows]), b, tb=True, threads=16)
    assert rel_fro(dA[rows], ref) <= GEMM_TOL
    assert rel_fro(dA[rows], ref) <= 1e-5  # identical operands: summation order only
    # dB[k, :] = A[:, k]^T . dC for sampled k
    ks = np.unique(np.concatenate([rng.choice(1000, 24, replace=False), [0, 999]]))
    ref = oracle.gemm(F16, np.ascontiguousarray(a[:, ks]), dc, ta=True, threads=16)
    assert rel_fro(dB[ks], ref) <= 1e-5
    # columns near the ragged edges, all rows: dB[:, j] = A^T . dC[:, j]
    js = np.array([0, 1, 2047, 2048, 2999])
    ref = oracle.gemm(F16, a, np.ascontiguousarray(dc[:, js]), ta=True, threads=16)
    assert rel_fro(dB[:, js], ref) <= 1e-5
    # linearity (exact) and determinism at the full shape
    dA2, dB2 = _backward(lib, a, b, dc, scale=2.0)
    assert np.array_equal(dA2, 2 * dA) and np.array_equal(dB2, 2 * dB)
    dA3, dB3 = _backward(lib, a, b, dc)
    assert np.array_equal(dA3, dA) and np.array_equal(dB3, dB)


def test_bmm_backward(lib, oracle, c4):
    q, kt, ds = c4["q"], c4["kt"], c4["ds"]
    print("c4 bmm f16 32x[512,128].[128,512]", flush=True)
    dQ, dKt = _backward(lib, q, kt, ds)
    assert dQ.shape == (32, 512, 128) and dKt.shape == (32, 128, 512)
    for z in (0, 13, 31):
        assert rel_fro(dQ[z], oracle.gemm(F16, ds[z], kt[z], tb=True, threads=16)) <= 1e-5
        assert rel_fro(dKt[z], oracle.gemm(F16, q[z], ds[z], ta=True, threads=16)) <= 1e-5
    dQ2, dKt2 = _backward(lib, q, kt, ds, scale=2.0)
    assert np.array_equal(dQ2, 2 * dQ) and np.array_equal(dKt2, 2 * dKt)
