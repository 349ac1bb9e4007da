"""Small host-to-device copies, which the library batches into one scatter
kernel reading a pinned staging ring (device.c): every tensor must hold
exactly the bytes it was created from, whatever the batching."""
from __future__ import annotations

import numpy as np
import pytest

from picograd_amd.capi import F16

pytestmark = pytest.mark.gpu


def test_many_small_tensors_round_trip(lib):
    """1500 tensors of 1 B to 200 KB (odd sizes, f32 and f16): batches of
    32 entries, slot changes and wrap-arounds of the 16 MiB ring; each
    read back equals its source."""
    rng = np.random.default_rng(0)
    made = []
    for i in range(1500):
        n = int(rng.integers(1, 50000)) if i % 7 else int(rng.integers(1, 8))
        if i % 3 == 0:
            arr = rng.integers(0, 65536, n, dtype=np.uint16)
            made.append((lib.tensor(arr, F16), arr))
        else:
            arr = rng.standard_normal(n).astype(np.float32)
            made.append((lib.tensor(arr), arr))
    for t, arr in made:
        assert np.array_equal(lib.read(t), arr)
        lib.pg_tensor_free(t)


def test_ordering_with_rewrites_frees_and_kernels(lib):
    """A second upload to the same tensor wins; a freed destination reused
    by the next allocation gets the new bytes; uploads between kernels are
    seen by the kernels that follow them."""
    a1 = np.arange(1000, dtype=np.float32)
    a2 = -a1
    t = lib.tensor(a1)
    assert lib.pg_tensor_copy_from_host(t, a2.ctypes.data)
    assert np.array_equal(lib.read(t), a2)
    for _ in range(50):
        x = lib.tensor(np.full(4096, 3.0, np.float32))
        lib.pg_tensor_free(x)
        y = lib.tensor(np.full(4096, 5.0, np.float32))
        assert np.all(lib.read(y) == 5.0)
        lib.pg_tensor_free(y)
    lib.pg_tensor_free(t)
    rng = np.random.default_rng(1)
    xs = [rng.standard_normal(777).astype(np.float32) for _ in range(40)]
    nodes = [lib.var(x) for x in xs]
    acc = nodes[0]
    made = []
    for n in nodes[1:]:
        acc = lib.op("add", acc, n)  # a kernel between each pair of uploads
        made.append(acc)
    want = np.sum(np.stack(xs).astype(np.float64), axis=0)
    assert np.allclose(lib.value(acc), want, rtol=1e-5, atol=1e-5)
    for n in reversed(made):
        lib.pg_node_free(n)
    for n in nodes:
        lib.pg_node_free(n)


def test_chain_loop_grads_stay_exact(lib, oracle):
    """The config-1 loop (three fresh leaves per iteration, then the fused
    backward) for 300 iterations with new values each time: every grad
    equals the oracle's."""
    import ctypes as C
    shp = (C.c_size_t * 2)(64, 64)
    oracle.orc_seed(7)
    for it in range(300):
        a, b, c = (oracle.uniform(4096, -1.0, 1.0).reshape(64, 64) for _ in range(3))
        na = lib.pg_var_from_data(2, shp, a.ctypes.data, True)
        nb = lib.pg_var_from_data(2, shp, b.ctypes.data, True)
        nc = lib.pg_var_from_data(2, shp, c.ctypes.data, True)
        t0 = lib.pg_ag_add(na, nb)
        t1 = lib.pg_ag_mul(t0, nc)
        t2 = lib.pg_ag_relu(t1)
        t3 = lib.pg_ag_tanh(t2)
        loss = lib.pg_ag_sum_all(t3)
        lib.pg_backward(loss)
        if it % 50 == 0 or it == 299:
            da, db, dc = oracle.chain1(a.ravel(), b.ravel(), c.ravel())
            for n, want in ((na, da), (nb, db), (nc, dc)):
                got = lib.grad(n).ravel()
                assert np.max(np.abs(got - want)) <= 1e-5 * max(1.0, float(np.max(np.abs(want)))), it
        for n in (loss, t3, t2, t1, t0, na, nb, nc):
            lib.pg_node_free(n)


def test_large_uploads_in_pieces(lib):
    """Copies above one staging slot (256 KiB) up to 4 MiB go through the
    ring as slot-sized pieces; larger ones through a pageable copy.  Odd
    sizes around the piece and batch boundaries, interleaved with small
    uploads, a rewrite of a large tensor, and a kernel reading one: every
    read back equals its source."""
    rng = np.random.default_rng(7)
    sizes = [65536, 65537, 65536 * 3 + 5, 262143, 262144, 1048576, 1048577 - 4, 1000003, 4 << 18, (4 << 18) + 1]
    made = []
    for n in sizes:
        arr = rng.standard_normal(n).astype(np.float32)
        made.append((lib.tensor(arr), arr))
        small = rng.standard_normal(int(rng.integers(1, 5000))).astype(np.float32)
        made.append((lib.tensor(small), small))
    for t, arr in made:
        assert np.array_equal(lib.read(t), arr), arr.size
    t, arr = made[10]  # 1,048,573 floats
    arr2 = -arr
    assert lib.pg_tensor_copy_from_host(t, arr2.ctypes.data)
    x = lib.var(arr2)
    y = lib.op("add", x, x)
    assert np.array_equal(lib.value(y), arr2 + arr2)
    assert np.array_equal(lib.read(t), arr2)
    for n in (y, x):
        lib.pg_node_free(n)
    for t, _ in made:
        lib.pg_tensor_free(t)
