"""The 128 x 256-tile MFMA GEMM (eight waves of 64 x 64; tile 3 of the
launch plan) in each operand layout the autograd uses, at shapes where the
plan picks it, with ragged edges in every dim:

- one matmul whose forward (A K-contiguous, W MN-contiguous), dgrad (both
  K-contiguous, k-tiles of 64 in three stages) and wgrad (both
  MN-contiguous, k = 2201 rows, the last k-tile reading zero rows past k)
  each plan tile 3 without split-K, and whose dgrad and wgrad run one after
  the other (each fills the chip alone);
- the fused bias + GELU epilogue on the forward layout;
- a matmul whose dgrad and wgrad run side by side in ONE launch on tile 3,
  each split along k (3 and 5 slices) and summed by one more launch;
- config 4's ragged shape, whose pair takes tile 3 without split-K, is
  checked at full size by test_gpu_c4.py.

The oracle checks sampled rows and columns, or whole grads where the
product is small, each against the f32-accumulating product of the same
16-bit operands (relative Frobenius <= 1e-5: identical operands, summation
order only); exact linearity in the upstream grad and bit-for-bit
determinism cover the rest.
"""
import ctypes as C
from math import erf

import numpy as np
import pytest

from oracle_lib import bf16_to_f32, f16_to_f32, rel_fro
from picograd_amd.capi import BF16, F16, F32

pytestmark = pytest.mark.gpu

T_GEMM16 = 2  # pg_amd_timer_read kind of the MFMA GEMMs


def _plan(lib, ta, tb, m, n, k, batch=1):
    sp = C.c_int(0)
    tile = lib.pg_amd_gemm16_plan(ta, tb, m, n, k, batch, 0, C.byref(sp), None)
    return tile, sp.value


def _to_f32(dt, h):
    return f16_to_f32(h) if dt == F16 else bf16_to_f32(h)


def _backward(lib, dt, a16, w16, g16, scale=1.0):
    """matmul forward + backward; also the number of GEMM intervals the
    library timed (a dgrad + wgrad pair counts once)."""
    lib.pg_amd_timer_reset()
    lib.pg_amd_timer_enable(1)
    na, nw = lib.var(a16, dtype=dt), lib.var(w16, dtype=dt)
    c = lib.op("matmul", na, nw)
    out = lib.value(c)
    seed = lib.tensor(_to_f32(dt, g16) * np.float32(scale))
    lib.pg_amd_backward_from(c, seed)
    da, dw = lib.grad(na), lib.grad(nw)
    cnt = C.c_size_t(0)
    lib.pg_amd_timer_read(T_GEMM16, C.byref(cnt))
    lib.pg_amd_timer_enable(0)
    lib.pg_amd_timer_reset()
    lib.pg_tensor_free(seed)
    for n in (c, na, nw):
        lib.pg_node_free(n)
    return out, da, dw, cnt.value


def _operands(oracle, dt, seed, M, K, N):
    oracle.orc_seed(seed)
    a = oracle.cast16(dt, oracle.normal(M * K, 0.0, 1.0).reshape(M, K))
    w = oracle.cast16(dt, oracle.normal(K * N, 0.0, 0.02).reshape(K, N))
    g = oracle.cast16(dt, oracle.normal(M * N, 0.0, 1.0).reshape(M, N))
    return a, w, g


@pytest.mark.parametrize("dt", [BF16, F16])
def test_wide_tile_matmul_all_layouts(lib, oracle, dt):
    M, K, N = 2201, 1808, 2208
    print(f"gemm 128x256-tile matmul fwd/bwd dt={dt} {M}x{K}x{N}", flush=True)
    assert _plan(lib, 0, 1, M, N, K) == (3, 1)  # forward
    assert _plan(lib, 0, 0, M, K, N) == (3, 1)  # dgrad
    assert _plan(lib, 1, 1, K, N, M) == (3, 1)  # wgrad
    a, w, g = _operands(oracle, dt, 70 + dt, M, K, N)
    out, da, dw, launches = _backward(lib, dt, a, w, g)
    assert launches == 3  # forward, dgrad, wgrad: no pair
    rng = np.random.default_rng(dt)
    rows = np.unique(np.concatenate([rng.choice(M, 40, replace=False), [0, 127, 128, 2175, 2176, M - 1]]))
    ref = oracle.gemm(dt, np.ascontiguousarray(a[rows]), w, threads=16)
    assert rel_fro(out[rows], ref) <= 1e-5
    ref = oracle.gemm(dt, np.ascontiguousarray(g[rows]), w, tb=True, threads=16)
    assert rel_fro(da[rows], ref) <= 1e-5
    ks = np.unique(np.concatenate([rng.choice(K, 24, replace=False), [0, 127, 128, 1791, 1792, K - 1]]))
    ref = oracle.gemm(dt, np.ascontiguousarray(a[:, ks]), g, ta=True, threads=16)
    assert rel_fro(dw[ks], ref) <= 1e-5
    # columns at tile edges (256-wide column tiles), all rows
    js = np.array([0, 255, 256, 2047, 2048, N - 1])
    ref = oracle.gemm(dt, a, np.ascontiguousarray(w[:, js]), threads=16)
    assert rel_fro(out[:, js], ref) <= 1e-5
    ref = oracle.gemm(dt, a, np.ascontiguousarray(g[:, js]), ta=True, threads=16)
    assert rel_fro(dw[:, js], ref) <= 1e-5
    cs = np.array([0, 255, 256, 1535, 1536, K - 1])
    ref = oracle.gemm(dt, g, np.ascontiguousarray(w[cs]), tb=True, threads=16)
    assert rel_fro(da[:, cs], ref) <= 1e-5
    _, da2, dw2, _ = _backward(lib, dt, a, w, g, scale=2.0)
    assert np.array_equal(da2, 2 * da) and np.array_equal(dw2, 2 * dw)
    out3, da3, dw3, _ = _backward(lib, dt, a, w, g)
    assert np.array_equal(out3, out) and np.array_equal(da3, da) and np.array_equal(dw3, dw)


@pytest.mark.parametrize("dt", [BF16, F16])
def test_wide_tile_fused_epilogue(lib, oracle, dt):
    """out = gelu(q(x) . q(W) + b) from one tile-3 launch with the epilogue
    fused, and its 16-bit copy."""
    M, K, N = 2201, 1808, 2208
    assert _plan(lib, 0, 1, M, N, K) == (3, 1)
    print(f"gemm 128x256-tile linear16 gelu dt={dt} {M}x{K}x{N}", flush=True)
    rng = np.random.default_rng(80 + dt)
    x = rng.standard_normal((M, K)).astype(np.float32)
    wt = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    b = (0.3 * rng.standard_normal(N)).astype(np.float32)
    nx, nw, nb = lib.var(x), lib.var(wt), lib.var(b)
    out = lib._check(lib.pg_amd_ag_linear16(nx, nw, nb, 2, dt))
    got = lib.value(out)
    rows = np.unique(np.concatenate([rng.choice(M, 32, replace=False), [0, 127, 128, 2175, 2176, M - 1]]))
    qx = _to_f32(dt, oracle.cast16(dt, np.ascontiguousarray(x[rows])))
    qw = _to_f32(dt, oracle.cast16(dt, wt))
    z = oracle.gemm(F32, qx, qw).astype(np.float64) + b
    want = 0.5 * z * (1.0 + np.vectorize(erf)(z / np.sqrt(2.0)))
    assert rel_fro(got[rows], want) <= 1e-5
    for n in (out, nx, nw, nb):
        lib.pg_node_free(n)


@pytest.mark.parametrize("dt", [BF16, F16])
def test_wide_tile_pair_split(lib, oracle, dt):
    """dgrad and wgrad side by side in one launch, both on tile 3 and both
    split along k; whole grads against the oracle."""
    M, K, N = 1537, 504, 1496
    print(f"gemm 128x256-tile dgrad+wgrad pair, split-K dt={dt} {M}x{K}x{N}", flush=True)
    a, w, g = _operands(oracle, dt, 90 + dt, M, K, N)
    out, da, dw, launches = _backward(lib, dt, a, w, g)
    assert launches == 2  # forward, then the pair as one interval
    ref = oracle.gemm(dt, g, w, tb=True, threads=16)
    assert rel_fro(da, ref) <= 1e-5
    ref = oracle.gemm(dt, a, g, ta=True, threads=16)
    assert rel_fro(dw, ref) <= 1e-5
    _, da2, dw2, _ = _backward(lib, dt, a, w, g, scale=2.0)
    assert np.array_equal(da2, 2 * da) and np.array_equal(dw2, 2 * dw)
    _, da3, dw3, _ = _backward(lib, dt, a, w, g)
    assert np.array_equal(da3, da) and np.array_equal(dw3, dw)
