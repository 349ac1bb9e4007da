"""Matmul backward when both operands are one tensor.

- pg_ag_matmul(x, x): one node on both sides, so dgrad and wgrad write ONE
  grad, dx = G.x^T + x^T.G (autograd.c:561-706 adds both into x's grad in
  turn).  At 4096^2 the two would otherwise run as one whole-chip paired
  launch, at 512^2 side by side on a CU split: in either, wgrad's blocks
  would add to the grad while dgrad's write it.
- pg_amd_ag_linear16(x, x): the same for the fused layer (one grad, one
  kept 16-bit copy).
- linear16 and matmul16 of two nodes whose values share one storage with
  different shapes (x [12, 20] and a [20, 12] view of it): each operand's
  16-bit copy has its own row pitch, so taking the second remakes the
  first; the first GEMM must be queued before that happens.

Every element is checked against the f64 products of the device's own
16-bit operands (gemm_check).
"""
import ctypes as C

import numpy as np
import pytest

from gemm_check import check_product
from oracle_lib import bf16_to_f32, f16_to_f32
from picograd_amd.capi import BF16, F16, shape_arg

pytestmark = pytest.mark.gpu


def _f32(dt, h):
    return f16_to_f32(h) if dt == F16 else bf16_to_f32(h)


@pytest.mark.parametrize("n", [4096, 512])
def test_matmul_x_times_x(lib, oracle, n):
    dt = BF16
    print(f"alias: matmul(x, x) bf16 {n}^2", flush=True)
    rng = np.random.default_rng(n)
    x16 = oracle.cast16(dt, (0.05 * rng.standard_normal((n, n))).astype(np.float32))
    g = _f32(dt, oracle.cast16(dt, rng.standard_normal((n, n)).astype(np.float32)))
    nx = lib.var(x16, dtype=dt)
    c = lib.op("matmul", nx, nx)
    seed = lib.tensor(g)
    lib.pg_amd_backward_from(c, seed)
    dx = lib.grad(nx)
    lib.pg_tensor_free(seed)
    lib.pg_node_free(c)
    lib.pg_node_free(nx)
    fx = _f32(dt, x16)
    check_product(dx, [(g, fx.T), (fx.T, g)], f"matmul(x, x) {n}^2: dx = G.x^T + x^T.G")


@pytest.mark.parametrize("n", [4096, 512])
def test_linear16_x_x(lib, oracle, n):
    dt = BF16
    print(f"alias: linear16(x, x) gelu bf16 {n}^2", flush=True)
    rng = np.random.default_rng(n + 1)
    x = (rng.standard_normal((n, n)) / np.sqrt(n)).astype(np.float32)
    g = rng.standard_normal((n, n)).astype(np.float32)
    nx = lib.var(x)
    lib.pg_amd_linear16_keep_dz(True)
    try:
        out = lib._check(lib.pg_amd_ag_linear16(nx, nx, None, 2, dt))
        seed = lib.tensor(g)
        lib.pg_amd_backward_from(out, seed)
        dx = lib.grad(nx)
        dz = _f32(dt, lib.read(lib.pg_amd_linear16_dz(out)))
    finally:
        lib.pg_amd_linear16_keep_dz(False)
    lib.pg_tensor_free(seed)
    lib.pg_node_free(out)
    lib.pg_node_free(nx)
    qx = _f32(dt, oracle.cast16(dt, x))
    check_product(dx, [(dz, qx.T), (qx.T, dz)], f"linear16(x, x) {n}^2: dx = dz.q(x)^T + q(x)^T.dz")


def _shared_pair(lib, x):
    """Nodes a (x, [12, 20]) and b (a [20, 12] view of a's storage)."""
    na = lib.var(x)
    nd, sh = shape_arg((x.shape[1], x.shape[0]))
    nb = lib._check(lib.pg_var_zeros(nd, sh, True))
    node = lib.node(nb)
    view = lib.lib.pg_tensor_reshape_view(lib.node(na).value, nd, sh)
    assert view
    old = node.value
    node.value = view
    lib.pg_tensor_free(old)
    return na, nb


@pytest.mark.parametrize("fused", [True, False])
def test_shared_storage_different_pitch(lib, oracle, fused):
    dt = BF16
    print(f"alias: shared storage x [12, 20] and its [20, 12] view, fused={fused}", flush=True)
    lib.lib.pg_tensor_reshape_view.restype = C.c_void_p
    lib.lib.pg_tensor_reshape_view.argtypes = [C.c_void_p, C.c_size_t, C.POINTER(C.c_size_t)]
    rng = np.random.default_rng(1220)
    x = rng.standard_normal((12, 20)).astype(np.float32)
    g = rng.standard_normal((12, 12)).astype(np.float32)
    na, nb = _shared_pair(lib, x)
    if fused:
        lib.pg_amd_linear16_keep_dz(True)
    try:
        out = lib._check(lib.pg_amd_ag_linear16(na, nb, None, 0, dt) if fused
                         else lib.pg_amd_ag_matmul16(na, nb, dt))
        seed = lib.tensor(g)
        lib.pg_amd_backward_from(out, seed)
        da, db = lib.grad(na), lib.grad(nb)
        dz = _f32(dt, lib.read(lib.pg_amd_linear16_dz(out)))[:, :12] if fused else None
    finally:
        lib.pg_amd_linear16_keep_dz(False)
    lib.pg_tensor_free(seed)
    for n in (out, nb, na):
        lib.pg_node_free(n)
    qa = _f32(dt, oracle.cast16(dt, x))
    qb = np.ascontiguousarray(qa.reshape(20, 12))
    qg = _f32(dt, oracle.cast16(dt, g))
    if fused:
        assert np.array_equal(dz, qg)  # act NONE: dz = q(dout)
    check_product(da, [(qg, qb.T)], "shared storage: da = q(G).q(b)^T", planted=False)
    check_product(db, [(qa.T, qg)], "shared storage: db = q(a)^T.q(G)", planted=False)
