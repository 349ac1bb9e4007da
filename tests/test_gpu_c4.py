"""Config 4 at its full shapes on the MI355X: the ragged f16 matmul backward
(M=4097, K=1000, N=3000) and the attention-style bmm backward
(32 x [512,128] . [128,512]), inputs drawn from the library RNG with the
reference's seed order (seed 45: A, B, dC, Q, K^T, dS).

Every element of every grad is checked against the f64 product of the same
f16 operands, within the f32 summation bound gamma(K) sum |A B|, and the
relative Frobenius error over each whole grad is held to 1e-5 (north star:
1e-3) -- gemm_check.check_product, which also shows that a skipped,
misplaced or doubled tile fails it.  Doubling the upstream grad doubles
every grad bit for bit (scaling by 2 is exact through the f16 rounding and
the f32 accumulation), and a repeated backward reproduces the grads bit for
bit (the kernels are deterministic).
"""
import numpy as np
import pytest

from gemm_check import check_product
from oracle_lib import f16_to_f32
from picograd_amd.capi import F16

pytestmark = pytest.mark.gpu


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
    fa, fb, fdc = f16_to_f32(a), f16_to_f32(b), f16_to_f32(dc)
    check_product(dA, [(fdc, fb.T)], "c4 dA = dC.B^T")
    check_product(dB, [(fa.T, fdc)], "c4 dB = A^T.dC")
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
    fq, fk, fs = f16_to_f32(q), f16_to_f32(kt), f16_to_f32(ds)
    check_product(dQ, [(fs, fk.transpose(0, 2, 1))], "c4 dQ = dS.Kt^T")
    check_product(dKt, [(fq.transpose(0, 2, 1), fs)], "c4 dKt = Q^T.dS")
    dQ2, dKt2 = _backward(lib, q, kt, ds, scale=2.0)
    assert np.array_equal(dQ2, 2 * dQ) and np.array_equal(dKt2, 2 * dKt)
