"""Deferred elementwise forward ops: with the JIT on, runs of elementwise ops
execute as one fused kernel when their values are first needed.  Every value
must equal what the eager kernels (JIT off) compute, bit for bit, whatever
the run looks like and whatever happens to its operands meanwhile."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

UNARY = ["neg", "exp", "log", "sqrt", "sin", "cos", "relu", "sigmoid", "tanh", "gelu", "erf", "abs"]
BINARY = ["add", "sub", "mul", "div"]


def bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def run_both(lib, build):
    """build(lib) -> (nodes_to_read, nodes_to_free); values with the JIT on
    (deferred) and off (eager)."""
    out = {}
    for jit in (True, False):
        lib.pg_autograd_set_jit(jit)
        try:
            read, made = build(lib)
            out[jit] = [lib.value(n) for n in read]
            for n in reversed(made):
                lib.pg_node_free(n)
        finally:
            lib.pg_autograd_set_jit(True)
    return out[True], out[False]


@pytest.mark.parametrize("op", UNARY)
def test_unary_deferred_equals_eager(lib, op):
    rng = np.random.default_rng(UNARY.index(op))
    x = rng.uniform(0.1, 3.0, 5000).astype(np.float32) if op in ("log", "sqrt") else \
        rng.standard_normal(5000).astype(np.float32) * 3

    def build(L):
        a = L.var(x)
        y = L.op(op, a)
        z = L.op(op, y) if op not in ("log", "sqrt") else L.op("abs", y)  # a run of two
        return [y, z], [a, y, z]

    d, e = run_both(lib, build)
    for u, v in zip(d, e):
        assert np.array_equal(bits(u), bits(v))


@pytest.mark.parametrize("op", BINARY)
def test_binary_broadcast_deferred_equals_eager(lib, op):
    rng = np.random.default_rng(10 + BINARY.index(op))
    x = rng.standard_normal((37, 64)).astype(np.float32)
    b = rng.uniform(0.5, 2.0, 64).astype(np.float32)
    c = rng.uniform(0.5, 2.0, (37, 1)).astype(np.float32)

    def build(L):
        nx, nb, nc = L.var(x), L.var(b), L.var(c)
        y = L.op(op, nx, nb)   # row broadcast
        z = L.op(op, y, nc)    # column broadcast
        w = L.op(op, z, z)     # the same operand twice
        return [y, z, w], [nx, nb, nc, y, z, w]

    d, e = run_both(lib, build)
    for u, v in zip(d, e):
        assert np.array_equal(bits(u), bits(v))


def test_config_chains_deferred_equal_eager(lib):
    """Config 1's chain, config 2's forward, an mse tail and a 40-op chain
    over 20 leaves (runs of at most 16 ops and 16 inputs), read back at the
    end and once in the middle."""
    rng = np.random.default_rng(3)
    a, b, c = (rng.uniform(-1, 1, (64, 64)).astype(np.float32) for _ in range(3))
    x = rng.standard_normal((96, 160)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(160)).astype(np.float32)
    g = rng.standard_normal((96, 160)).astype(np.float32)
    leaves = [rng.uniform(0.5, 1.5, (33, 7)).astype(np.float32) for _ in range(20)]

    def build(L):
        made = []
        na, nb, nc = (L.var(v) for v in (a, b, c))
        t = L.op("tanh", L.op("relu", L.op("mul", L.op("add", na, nb), nc)))
        made += [na, nb, nc]
        nx, nbias, ng = L.var(x), L.var(bias), L.var(g)
        z = L.op("add", nx, nbias)
        mid = L.value(z)  # a read in the middle of a run
        y = L.op("mul", L.op("gelu", z), L.op("sigmoid", ng))
        d = L.op("sub", y, nx)
        sq = L.op("mul", d, d)
        made += [nx, nbias, ng]
        ls = [L.var(v) for v in leaves]
        acc = ls[0]
        for i in range(1, 40):
            acc = L.op("mul" if i % 2 else "add", acc, ls[i % 20])
            acc = L.op("sigmoid", acc) if i % 5 == 0 else acc
        made += ls
        return [t, z, y, sq, acc], made + [t, z, y, d, sq, acc]

    d, e = run_both(lib, build)
    for u, v in zip(d, e):
        assert np.array_equal(bits(u), bits(v))


def test_operand_changes_after_recording(lib):
    """An op recorded before its operand is overwritten (copy_from_host,
    fill) or freed computes from the operand as it was, as the eager op
    would; storage freed while a run is pending is not recycled into it."""
    lib.pg_autograd_set_jit(True)
    x0 = np.arange(1, 1001, dtype=np.float32)
    nx = lib.var(x0)
    y = lib.op("mul", nx, nx)
    assert lib.pg_tensor_copy_from_host(lib.node(nx).value, (-x0).ctypes.data)
    z = lib.op("add", nx, nx)
    assert np.array_equal(lib.value(y), x0 * x0)
    assert np.array_equal(lib.value(z), -2 * x0)
    w = lib.op("exp", nx)
    lib.pg_tensor_fill(lib.node(nx).value, 0.0)
    assert np.array_equal(bits(lib.value(w)), bits(np.exp(-x0.astype(np.float64)).astype(np.float32))) or \
        np.allclose(lib.value(w), np.exp(-x0), rtol=1e-6)
    for n in (y, z, w, nx):
        lib.pg_node_free(n)
    vals = []
    for i in range(30):
        a = lib.var(np.full(4096, float(i), np.float32))
        b = lib.op("add", a, a)
        lib.pg_node_free(a)     # the run still needs a's storage
        c = lib.var(np.full(4096, 100.0 + i, np.float32))  # may not land on a's block
        d = lib.op("mul", b, c)
        vals.append((b, c, d, i))
    for b, c, d, i in vals:
        assert np.all(lib.value(b) == 2.0 * i) and np.all(lib.value(d) == 2.0 * i * (100.0 + i))
        for n in (d, c, b):
            lib.pg_node_free(n)


def test_backward_through_deferred_values(lib, oracle):
    """pg_backward right after deferred ops: the fused backward reads the
    run's inputs and its grads equal the oracle's (config 1 chain)."""
    import ctypes as C
    lib.pg_autograd_set_jit(True)
    oracle.orc_seed(11)
    a, b, c = (oracle.uniform(4096, -1.0, 1.0).reshape(64, 64) for _ in range(3))
    na, nb, nc = lib.var(a), lib.var(b), lib.var(c)
    t3 = lib.op("tanh", lib.op("relu", lib.op("mul", lib.op("add", na, nb), nc)))
    loss = lib.op("sum_all", t3)
    lib.pg_backward(loss)
    da, db, dc = oracle.chain1(a.ravel(), b.ravel(), c.ravel())
    for n, want in ((na, da), (nb, db), (nc, dc)):
        assert np.max(np.abs(lib.grad(n).ravel() - want)) <= 1e-6
    want_loss = np.tanh(np.maximum((a.astype(np.float64) + b) * c, 0)).sum()
    assert abs(float(lib.value(loss)[0]) - want_loss) <= 1e-3
    for n in (loss, t3, na, nb, nc):
        lib.pg_node_free(n)


@pytest.mark.parametrize("shape", [(64, 64), (37, 63), (127, 127), (1, 100), (100, 1), (130, 64)])
@pytest.mark.parametrize("mean", [False, True])
def test_small_runs_fold_uploads_and_reduce_all(lib, shape, mean):
    """A small run ending in sum_all / mean_all (config 1's loop): with the
    JIT on, one block performs the leaves' uploads, the run and both
    reduction stages; the values equal the eager path's (JIT off: upload
    scatter, one kernel per op, pgk_sum_all2_f32) bit for bit.  (37, 63)
    has leaves that are not whole 16-byte pieces, (127, 127) the largest
    folded reduction, (130, 64) a reduction that does not fold (its row
    axis is reduced in two stages)."""
    rng = np.random.default_rng(shape[0] * 1000 + shape[1])
    a, b, c = (rng.uniform(-1, 1, shape).astype(np.float32) for _ in range(3))
    red = "mean_all" if mean else "sum_all"

    def build(L):
        na, nb, nc = L.var(a), L.var(b), L.var(c)
        t = L.op("tanh", L.op("relu", L.op("mul", L.op("add", na, nb), nc)))
        loss = L.op(red, t)
        direct = L.op(red, nc)  # a leaf: no run to fold into
        return [loss, t, direct], [na, nb, nc, t, loss, direct]

    d, e = run_both(lib, build)
    for u, v in zip(d, e):
        assert np.array_equal(bits(u), bits(v))


@pytest.mark.parametrize("nleaves,side", [(5, 32), (4, 127)])
def test_small_run_with_uploads_it_cannot_fold(lib, nleaves, side):
    """More pending uploads than the one-block kernel takes (5 > 4), or more
    bytes (4 x 127 x 127 floats > 256 KiB): the uploads go back to the batch
    in order and the run still equals the eager path, as does the mse
    tail's mean_all and the grads of a backward through it."""
    rng = np.random.default_rng(nleaves * side)
    leaves = [rng.standard_normal((side, side)).astype(np.float32) for _ in range(nleaves)]
    target = rng.standard_normal((side, side)).astype(np.float32)

    grads = {}

    def build(L):
        ns = [L.var(v) for v in leaves]
        acc = ns[0]
        made = list(ns)
        for n in ns[1:]:
            m = L.op("mul", acc, n)
            acc = L.op("add", m, n)
            made += [m, acc]
        nt = L.var(target, requires_grad=False)
        loss = L.op("mse", acc, nt, True)
        L.pg_backward(loss)
        grads[bool(L.pg_autograd_is_jit_enabled())] = [L.grad(n) for n in ns]
        return [loss, acc], made + [nt, loss]

    d, e = run_both(lib, build)
    for u, v in zip(d, e):
        assert np.array_equal(bits(u), bits(v))
    for u, v in zip(grads[True], grads[False]):  # fused backward against eager: f32 reassociation only
        assert np.max(np.abs(u - v)) <= 1e-5 * max(1.0, float(np.max(np.abs(v))))


@pytest.mark.parametrize("shape", [(4096, 10), (4097, 7), (2000, 17), (65536, 1)])
@pytest.mark.parametrize("mean", [False, True])
def test_sliced_reduce_all_in_one_launch(lib, shape, mean):
    """sum_all / mean_all over [rows, cols] whose column sums are sliced
    (config 5's mse over [4096, 10]): one launch gives the values of the
    pg_ag_sum(axis 0) -> pg_ag_sum / pg_ag_mean chain (three launches) bit
    for bit, and the same grads; the values are within f32 summation error
    of the f64 sums."""
    rng = np.random.default_rng(shape[0] + shape[1])
    x = rng.standard_normal(shape).astype(np.float32)
    na = lib.var(x)
    one = lib.op("mean_all" if mean else "sum_all", na)
    s0 = lib.op("sum", na, 0, False)
    chain = lib.op("mean" if mean else "sum", s0, 0, False)
    v1, v2 = lib.value(one), lib.value(chain)
    assert np.array_equal(bits(v1), bits(v2))
    col = x.astype(np.float64).sum(axis=0)
    want = col.mean() if mean else col.sum()
    assert abs(float(v1[0]) - want) <= 1e-5 * np.abs(x).astype(np.float64).sum() / (shape[1] if mean else 1)
    lib.pg_backward(one)
    g1 = lib.grad(na).copy()
    lib.pg_node_free(one)
    nb = lib.var(x)
    s1 = lib.op("sum", nb, 0, False)
    chain2 = lib.op("mean" if mean else "sum", s1, 0, False)
    lib.pg_backward(chain2)
    assert np.array_equal(bits(g1), bits(lib.grad(nb)))
    for n in (chain2, s1, nb, chain, s0, na):
        lib.pg_node_free(n)


@pytest.mark.parametrize("shape", [(64, 64), (37, 63), (127, 127), (1, 100)])
@pytest.mark.parametrize("reuse", [False, True])
def test_backward_joins_the_small_run(lib, oracle, shape, reuse):
    """Config 1's iteration -- three fresh leaves, a deferred forward run
    ending in sum_all, pg_backward -- takes ONE JIT launch with the JIT on:
    the fused backward region joins the pending run's one-block kernel
    (uploads, forward values, both reduction stages, grads; leaves that are
    not whole 16-byte pieces, (37, 63) and (127, 127), are uploaded by one
    k_upload ahead of it).  The forward
    values and the loss equal the eager path's bit for bit, and the grads
    agree with the eager backward to 1e-6 (both evaluate the same chain
    rule; the joined body is compiled without FMA contraction).  `reuse`
    feeds leaf a into two ops (its grad sums two contributions)."""
    import ctypes as C
    rng = np.random.default_rng(shape[0] * 7 + shape[1] + reuse)
    a, b, c = (rng.uniform(-1, 1, shape).astype(np.float32) for _ in range(3))

    def build(L):
        na, nb, nc = L.var(a), L.var(b), L.var(c)
        t0 = L.op("add", na, nb)
        t1 = L.op("mul", t0, na if reuse else nc)
        t2 = L.op("tanh", L.op("relu", t1))
        loss = L.op("sum_all", t2)
        return (na, nb, nc, t2, loss), [na, nb, nc, t0, t1, t2, loss]

    got = {}
    for jit in (True, False):
        lib.pg_autograd_set_jit(jit)
        try:
            (na, nb, nc, t2, loss), made = build(lib)
            lib.pg_amd_timer_reset()
            lib.pg_amd_timer_enable(1)
            lib.pg_backward(loss)
            cnt = C.c_size_t(0)
            lib.pg_amd_timer_read(0, C.byref(cnt))  # JIT kernel launches (PGD_T_JIT_MAIN)
            lib.pg_amd_timer_enable(0)
            lib.pg_amd_timer_reset()
            got[jit] = dict(vals=[lib.value(t2), lib.value(loss)], grads=[lib.grad(n) for n in (na, nb, nc)],
                            launches=cnt.value)
            for n in reversed(made):
                lib.pg_node_free(n)
        finally:
            lib.pg_autograd_set_jit(True)
    assert got[True]["launches"] == 1, got[True]["launches"]
    for u, v in zip(got[True]["vals"], got[False]["vals"]):
        assert np.array_equal(bits(u), bits(v))
    for i, (g1, g0) in enumerate(zip(got[True]["grads"], got[False]["grads"])):
        if reuse and i == 2:  # c is not in the graph
            assert g1 is None and g0 is None
            continue
        assert np.max(np.abs(g1 - g0)) <= 1e-6 * max(1.0, float(np.abs(g0).max()))
    if not reuse and shape == (64, 64):
        da, db, dc = oracle.chain1(a.ravel(), b.ravel(), c.ravel())
        for g, want in zip(got[True]["grads"], (da, db, dc)):
            assert np.max(np.abs(g.ravel() - want)) <= 1e-6


def test_broadcast_grad_keeps_the_run_and_region_apart(lib):
    """A run whose backward region reduces a grad onto a broadcast leaf
    (tanh(x + b), b [cols]) cannot share the one-block kernel (the region's
    column reduction needs the main kernel): the run and the region launch
    separately and the grads equal the eager path's within 1e-6."""
    import ctypes as C
    rng = np.random.default_rng(77)
    x = rng.uniform(-1, 1, (64, 64)).astype(np.float32)
    b = rng.uniform(-1, 1, 64).astype(np.float32)
    got = {}
    for jit in (True, False):
        lib.pg_autograd_set_jit(jit)
        try:
            nx, nb = lib.var(x), lib.var(b)
            y = lib.op("tanh", lib.op("add", nx, nb))
            loss = lib.op("sum_all", y)
            lib.pg_amd_timer_reset()
            lib.pg_amd_timer_enable(1)
            lib.pg_backward(loss)
            cnt = C.c_size_t(0)
            lib.pg_amd_timer_read(0, C.byref(cnt))
            lib.pg_amd_timer_enable(0)
            lib.pg_amd_timer_reset()
            got[jit] = (lib.grad(nx), lib.grad(nb), cnt.value)
            for n in (loss, y, nb, nx):
                lib.pg_node_free(n)
        finally:
            lib.pg_autograd_set_jit(True)
    assert got[True][2] == 2  # the run's block, then the region's main kernel
    for g1, g0 in zip(got[True][:2], got[False][:2]):
        assert np.max(np.abs(g1 - g0)) <= 1e-6 * max(1.0, float(np.abs(g0).max()))
