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
    fa, fw, fg = _to_f32(dt, a), _to_f32(dt, w), _to_f32(dt, g)
    check_product(out, [(fa, fw)], "tile-3 forward A.W")
    check_product(da, [(fg, fw.T)], "tile-3 dgrad dC.W^T")
    check_product(dw, [(fa.T, fg)], "tile-3 wgrad A^T.dC")
    del fa, fw, fg
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
    z = lib.read(lib.pg_amd_linear16_preact(out))
    qx, qw = _to_f32(dt, oracle.cast16(dt, x)), _to_f32(dt, oracle.cast16(dt, wt))
    check_linear(got, z, [(qx, qw)], b, 2, "tile-3 linear16 gelu epilogue")
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
    fa, fw, fg = _to_f32(dt, a), _to_f32(dt, w), _to_f32(dt, g)
    check_product(da, [(fg, fw.T)], "split pair dgrad")
    check_product(dw, [(fa.T, fg)], "split pair wgrad")
    _, da2, dw2, _ = _backward(lib, dt, a, w, g, scale=2.0)
    assert np.array_equal(da2, 2 * da) and np.array_equal(dw2, 2 * dw)
    _, da3, dw3, _ = _backward(lib, dt, a, w, g)
    assert np.array_equal(da3, da) and np.array_equal(dw3, dw)
