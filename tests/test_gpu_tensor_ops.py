"""Tensor-level ops (ops/elementwise.h, activations.h, matmul.h) and the
tensor utilities of core/tensor.h on the MI355X, through the C ABI.

- Every tensor op equals its pg_ag_* op bit for bit (the same kernels), with
  the JIT's deferred execution on and off, on broadcast operands and on a
  transposed view.
- pg_matmul / pg_bmm against the f32-accumulating oracle.
- arange / linspace against the reference's f32 formulas
  (tensor.c:276-357), get / set with strides and RNE, allclose's rule,
  print's text, the pool.
- A transposed view saved with pg_tensor_save is written in logical
  row-major order, byte for byte the PGT1 record the reference writes for
  it (tensor.c:628-647; the oracle's writer is pinned to the reference's
  files).
"""
import ctypes as C
import os

import numpy as np
import pytest

from oracle_lib import rel_fro
from picograd_amd.capi import BF16, F16, F32

pytestmark = pytest.mark.gpu

UNARY = ["neg", "abs", "sqrt", "exp", "log", "sin", "cos", "erf", "relu", "sigmoid", "tanh", "gelu"]
BINARY = ["add", "sub", "mul", "div"]


def _proto(lib, name, res, args):
    fn = getattr(lib.lib, name)
    fn.restype, fn.argtypes = res, args
    return fn


@pytest.fixture(scope="module")
def ops(lib):
    vp, fl, sz = C.c_void_p, C.c_float, C.c_size_t
    SZP = C.POINTER(C.c_size_t)
    o = {n: _proto(lib, f"pg_{n}", vp, [vp]) for n in UNARY}
    o.update({n: _proto(lib, f"pg_{n}", vp, [vp, vp]) for n in BINARY + ["matmul", "bmm"]})
    o["clamp"] = _proto(lib, "pg_clamp", vp, [vp, fl, fl])
    o["leaky_relu"] = _proto(lib, "pg_leaky_relu", vp, [vp, fl])
    o["arange"] = _proto(lib, "pg_tensor_arange", vp, [fl, fl, fl])
    o["linspace"] = _proto(lib, "pg_tensor_linspace", vp, [fl, fl, sz])
    o["eye"] = _proto(lib, "pg_tensor_eye", vp, [sz])
    o["get"] = _proto(lib, "pg_tensor_get", fl, [vp, SZP])
    o["set"] = _proto(lib, "pg_tensor_set", None, [vp, SZP, fl])
    o["allclose"] = _proto(lib, "pg_tensor_allclose", C.c_bool, [vp, vp, fl, fl])
    o["permute"] = _proto(lib, "pg_tensor_permute_view", vp, [vp, SZP])
    o["pool_size"] = _proto(lib, "pg_tensor_pool_size", sz, [])
    o["pool_bytes"] = _proto(lib, "pg_tensor_pool_bytes", sz, [])
    o["pool_clear"] = _proto(lib, "pg_tensor_pool_clear", None, [])
    return o


def _idx(*i):
    return (C.c_size_t * len(i))(*i)


@pytest.mark.parametrize("jit", [True, False])
def test_tensor_ops_equal_the_autograd_ops(lib, ops, jit):
    rng = np.random.default_rng(11)
    a = rng.uniform(0.2, 2.0, (33, 70)).astype(np.float32) * rng.choice([-1, 1], (33, 70)).astype(np.float32)
    b = rng.uniform(0.5, 1.5, (70,)).astype(np.float32)
    ta, tb = lib.tensor(a), lib.tensor(b)
    na, nb = lib.var(a), lib.var(b)
    lib.pg_autograd_set_jit(jit)
    try:
        for name in UNARY:
            src = lib.tensor(np.abs(a)) if name in ("sqrt", "log") else ta
            nsrc = lib.var(np.abs(a)) if name in ("sqrt", "log") else na
            y = ops[name](src)
            ny = lib.op(name, nsrc)
            assert y, name
            assert np.array_equal(lib.read(y).view(np.uint32), lib.value(ny).view(np.uint32)), name
            lib.pg_tensor_free(y)
            lib.pg_node_free(ny)
            if src != ta:
                lib.pg_tensor_free(src)
                lib.pg_node_free(nsrc)
        for name in BINARY:
            y = ops[name](ta, tb)
            ny = lib.op(name, na, nb)
            assert lib.shape(y) == (33, 70)
            assert np.array_equal(lib.read(y).view(np.uint32), lib.value(ny).view(np.uint32)), name
            lib.pg_tensor_free(y)
            lib.pg_node_free(ny)
        y = ops["clamp"](ta, -0.5, 0.75)
        assert np.array_equal(lib.read(y), np.clip(a, -0.5, 0.75))
        lib.pg_tensor_free(y)
        assert not ops["clamp"](ta, 1.0, -1.0)
        y = ops["leaky_relu"](ta, 0.1)
        ny = lib.op("leaky_relu", na, 0.1)
        assert np.array_equal(lib.read(y), lib.value(ny))
        lib.pg_tensor_free(y)
        lib.pg_node_free(ny)
        # a transposed view is read in logical order
        tv = ops["permute"](ta, _idx(1, 0))
        y = ops["add"](tv, lib.tensor(np.zeros(33, np.float32)))
        assert np.array_equal(lib.read(y), a.T + np.float32(0))
        lib.pg_tensor_free(y)
        lib.pg_tensor_free(tv)
        # incompatible broadcast shapes
        assert not ops["add"](ta, lib.tensor(np.ones(69, np.float32)))
    finally:
        lib.pg_autograd_set_jit(True)
    for t in (ta, tb):
        lib.pg_tensor_free(t)
    for n in (na, nb):
        lib.pg_node_free(n)


@pytest.mark.parametrize("dt", [F32, BF16, F16])
def test_matmul_and_bmm_match_the_oracle(lib, ops, oracle, dt):
    rng = np.random.default_rng(3 + dt)
    a = rng.standard_normal((4, 37, 64)).astype(np.float32)
    b = rng.standard_normal((4, 64, 24)).astype(np.float32)
    if dt != F32:
        a16, b16 = oracle.cast16(dt, a), oracle.cast16(dt, b)
        ta, tb = lib.tensor(a16, dt), lib.tensor(b16, dt)
    else:
        a16, b16 = a, b
        ta, tb = lib.tensor(a), lib.tensor(b)
    y = ops["bmm"](ta, tb)
    assert y and lib.shape(y) == (4, 37, 24)
    got = lib.read(y)
    for z in range(4):
        assert rel_fro(got[z], oracle.gemm(dt, a16[z], b16[z])) <= 1e-5
    m = ops["matmul"](ta, tb)
    assert np.array_equal(lib.read(m), got)
    assert not ops["bmm"](ta, ta)
    for t in (y, m, ta, tb):
        lib.pg_tensor_free(t)


def test_tensor_utilities(lib, ops):
    t = ops["arange"](0.25, 4.0, 0.7)
    n = int(np.ceil(np.float32(4.0 - 0.25) / np.float32(0.7)))
    want = np.float32(0.25) + np.float32(0.7) * np.arange(n, dtype=np.float32)
    assert np.array_equal(lib.read(t), want)
    lib.pg_tensor_free(t)
    assert not ops["arange"](1.0, 0.0, 1.0) and not ops["arange"](0.0, 1.0, 0.0)
    t = ops["linspace"](-2.0, 3.0, 7)
    step = np.float32(5.0) / np.float32(6.0)
    want = np.float32(-2.0) + step * np.arange(7, dtype=np.float32)
    want[-1] = 3.0
    assert np.array_equal(lib.read(t), want)
    lib.pg_tensor_free(t)
    t = ops["eye"](5)
    assert np.array_equal(lib.read(t), np.eye(5, dtype=np.float32))
    ops["set"](t, _idx(2, 4), 9.5)
    assert ops["get"](t, _idx(2, 4)) == 9.5 and ops["get"](t, _idx(4, 2)) == 0.0
    tv = ops["permute"](t, _idx(1, 0))
    assert ops["get"](tv, _idx(4, 2)) == 9.5
    e2 = lib.tensor(np.eye(5, dtype=np.float32))
    assert not ops["allclose"](t, e2, 0.0, 0.0)
    assert ops["allclose"](t, e2, 0.0, 9.5) and not ops["allclose"](t, e2, 0.0, 9.4)
    for x in (tv, t, e2):
        lib.pg_tensor_free(x)
    # f16 set rounds to nearest even
    h = lib.pg_tensor_full_dtype(F16, 1, (C.c_size_t * 1)(3), 0.0)
    ops["set"](h, _idx(1), 1.0 + 2.0 ** -11)  # halfway between 1 and 1 + 2^-10: even is 1
    ops["set"](h, _idx(2), 1.0 + 3 * 2.0 ** -11)  # halfway: rounds up to 1 + 2^-9
    assert list(lib.read(h).view(np.float16)) == [0.0, 1.0, 1.0 + 2.0 ** -9]
    lib.pg_tensor_free(h)
    # the pool is the allocator's cache of freed blocks
    assert ops["pool_bytes"]() == lib.pg_amd_bytes_cached()
    ops["pool_clear"]()
    assert ops["pool_size"]() == 0 and ops["pool_bytes"]() == 0


def test_print_matches_the_reference_text(lib, tmp_path):
    libc = C.CDLL(None)
    libc.fopen.restype, libc.fopen.argtypes = C.c_void_p, [C.c_char_p, C.c_char_p]
    libc.fclose.argtypes = [C.c_void_p]
    pr = _proto(lib, "pg_tensor_print", None, [C.c_void_p, C.c_void_p])
    x = np.arange(12, dtype=np.float32).reshape(2, 2, 3) / 4
    t = lib.tensor(x)
    path = tmp_path / "p.txt"
    f = libc.fopen(str(path).encode(), b"w")
    pr(t, f)
    libc.fclose(f)
    lib.pg_tensor_free(t)
    # print_rec (tensor.c:522-545): %g elements, rows after the first on a new
    # line indented by their depth
    assert path.read_text() == ("[[[0, 0.25, 0.5],\n  [0.75, 1, 1.25]],\n [[1.5, 1.75, 2],\n  [2.25, 2.5, 2.75]]]\n")


def test_save_of_a_transposed_view_is_the_reference_record(lib, ops, oracle, tmp_path):
    x = np.arange(24, dtype=np.float32).reshape(4, 6) * 0.5 - 3.0
    t = lib.tensor(x)
    tv = ops["permute"](t, _idx(1, 0))
    path = tmp_path / "v.pgt"
    assert lib.pg_tensor_save(tv, str(path).encode())
    assert path.read_bytes() == oracle.pgt1_bytes(F32, np.ascontiguousarray(x.T))
    back = lib.pg_tensor_load(str(path).encode())
    assert np.array_equal(lib.read(back), x.T)
    for z in (back, tv, t):
        lib.pg_tensor_free(z)
    os.remove(path)
