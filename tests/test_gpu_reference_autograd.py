"""The reference's own autograd test suite (tests/test_autograd.c) run
against the MI355X library through the C ABI.

Each case builds the same graph on the same inputs as test_autograd.c and
checks the device grads the way the reference does: against central
differences of the loss (numcheck, h = 1e-2, |g - num| <= 2e-2 (1 + |num|)
+ 1e-3, test_autograd.c:28-99), or against closed forms (closef, 1e-4
relative, :24-26).  Every numcheck case runs with the fused JIT on and off.
"""
import ctypes as C

import numpy as np
import pytest

from picograd_amd.capi import shape_arg

pytestmark = pytest.mark.gpu


def close_num(x, y):
    return abs(x - y) <= 2e-2 * (1.0 + abs(y)) + 1e-3


def numcheck(lib, build, leaves):
    """leaves: list of (node, host array); build(nodes) -> loss node."""
    nodes = [n for n, _ in leaves]
    loss = build(nodes)
    assert lib.shape(lib.node(loss).value) in ((1,), ())
    lib.pg_backward(loss)
    grads = [lib.grad(n) for n in nodes]
    lib.pg_node_free(loss)
    h = np.float32(1e-2)
    for k, (n, arr) in enumerate(leaves):
        assert grads[k] is not None, f"leaf {k} has no grad"
        t = lib.node(n).value
        flat = arr.reshape(-1)
        for i in range(flat.size):
            old = flat[i]
            vals = []
            for d in (h, -h):
                flat[i] = old + d
                assert lib.pg_tensor_copy_from_host(t, arr.ctypes.data)
                lp = build(nodes)
                vals.append(float(lib.value(lp).reshape(-1)[0]))
                lib.pg_node_free(lp)
            flat[i] = old
            assert lib.pg_tensor_copy_from_host(t, arr.ctypes.data)
            num = (vals[0] - vals[1]) / (2.0 * float(h))
            g = float(grads[k].reshape(-1)[i])
            assert close_num(g, num), f"leaf{k}[{i}] grad={g} numeric={num}"


def leaf(lib, data, rg=True):
    arr = np.ascontiguousarray(np.asarray(data, np.float32))
    return lib.var(arr, requires_grad=rg), arr


def uniform_leaf(lib, shape, lo, hi, rg=True):
    nd, sh = shape_arg(shape)
    n = lib._check(lib.pg_var_uniform(nd, sh, lo, hi, rg))
    return n, lib.value(n).copy()


def owned(lib, fn, t):
    loss = lib.op(fn, t)
    lib.pg_node_free(t)
    return loss


@pytest.fixture(params=[True, False], ids=["jit", "eager"])
def jit(lib, request):
    lib.pg_autograd_set_jit(request.param)
    yield request.param
    lib.pg_autograd_set_jit(True)


def free(lib, leaves):
    for n, _ in leaves:
        lib.pg_node_free(n)


def test_lifecycle(lib):
    """test_autograd.c:106-160"""
    a = lib.var(np.array([1, -2, 3, -4], np.float32))
    node = lib.node(a)
    assert node.refs == 1 and node.requires_grad and not node.grad
    assert lib.value(a)[2] == 3.0
    b = lib.pg_node_retain(a)
    c = lib.op("neg", a)
    assert lib.node(c).nparents == 1 and lib.node(c).requires_grad
    assert lib.value(c)[1] == 2.0
    lib.pg_node_free(a)
    assert lib.value(b)[0] == 1.0
    lib.pg_node_free(c)
    assert lib.value(b)[2] == 3.0
    lib.pg_node_free(b)
    lib.pg_node_free(None)
    ng = lib._check(lib.pg_var_scalar(5.0, False))
    loss = lib.op("sum_all", ng)
    lib.pg_backward(loss)
    assert not lib.node(ng).grad and not lib.node(loss).grad
    lib.pg_node_free(loss)
    lib.pg_node_free(ng)
    lib.pg_backward(None)


@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
def test_arithmetic(lib, jit, op):
    """test_autograd.c:162-214: same-shape operands"""
    lv = [leaf(lib, [[1.0, -2.0, 3.0], [0.5, -1.5, 2.5]]), leaf(lib, [[2.0, 0.5, 4.0], [-1.0, 3.0, -2.5]])]
    numcheck(lib, lambda xs: owned(lib, "sum_all", lib.op(op, xs[0], xs[1])), lv)
    free(lib, lv)


@pytest.mark.parametrize("case", ["add-bcast-scalar", "mul-bcast-row", "div-bcast-col"])
def test_arithmetic_broadcast(lib, jit, case):
    """test_autograd.c:190-213: scalar, row and column broadcasts"""
    c = [[1, 2, 3], [4, 5, 6]]
    if case == "add-bcast-scalar":
        lv, op = [leaf(lib, c), leaf(lib, [0.5])], "add"
    elif case == "mul-bcast-row":
        lv, op = [leaf(lib, c), leaf(lib, [1.0, 2.0, 3.0])], "mul"
    else:
        lv, op = [leaf(lib, [[10.0], [20.0]]), leaf(lib, c)], "div"
    numcheck(lib, lambda xs: owned(lib, "sum_all", lib.op(op, xs[0], xs[1])), lv)
    free(lib, lv)


@pytest.mark.parametrize("op", ["exp", "log", "sqrt", "sin", "cos", "neg", "relu", "sigmoid", "tanh"])
def test_unary(lib, jit, op):
    """test_autograd.c:256-286: mean_all of each unary op"""
    data = [0.5, 1.5, 2.5, 4.0] if op in ("log", "sqrt") else [-1.2, 0.7, 1.9, -0.4]
    lv = [leaf(lib, data)]
    numcheck(lib, lambda xs: owned(lib, "mean_all", lib.op(op, xs[0])), lv)
    free(lib, lv)


A_RAW = [[0.5, -1.0, 2.0, 0.3], [-0.7, 1.1, 0.2, -0.4], [0.9, 1.5, -2.0, 0.6]]
B_RAW = [[1.0, -0.5], [2.0, 0.25], [-1.5, 0.75], [0.1, -0.2]]
V_RAW = [0.5, -1.0, 2.0, 0.3]


@pytest.mark.parametrize("case", ["2d2d", "v2d", "2dv", "vv"])
def test_matmul(lib, jit, case):
    """test_autograd.c:288-324: matrix and vector operands"""
    a = {"2d2d": A_RAW, "v2d": V_RAW, "2dv": A_RAW, "vv": V_RAW}[case]
    b = {"2d2d": B_RAW, "v2d": B_RAW, "2dv": V_RAW, "vv": [1.0, 0.5, -0.5, 2.0]}[case]
    lv = [leaf(lib, a), leaf(lib, b)]
    numcheck(lib, lambda xs: owned(lib, "sum_all", lib.op("matmul", xs[0], xs[1])), lv)
    free(lib, lv)


@pytest.mark.parametrize("bshape", [(2, 4, 5), (4, 5)], ids=["bmm", "bcast-batch"])
def test_matmul_batched(lib, jit, bshape):
    """test_autograd.c:326-343 (seed 11)"""
    lib.pg_seed(11)
    lv = [uniform_leaf(lib, (2, 3, 4), -1.0, 1.0), uniform_leaf(lib, bshape, -1.0, 1.0)]
    numcheck(lib, lambda xs: owned(lib, "sum_all", lib.op("matmul", xs[0], xs[1])), lv)
    free(lib, lv)


@pytest.mark.parametrize("case", ["sum-axis1", "mean-axis0-keepdim", "mean-axis2"])
def test_reduce(lib, jit, case):
    """test_autograd.c:345-379 (seed 21)"""
    lib.pg_seed(21)
    lv = [uniform_leaf(lib, (2, 3, 4), -2.0, 2.0)]

    def build(xs):
        if case == "sum-axis1":
            s = lib._check(lib.pg_ag_sum(xs[0], 1, False))
        elif case == "mean-axis0-keepdim":
            s = lib._check(lib.pg_ag_mean(xs[0], 0, True))
        else:
            s = lib._check(lib.pg_ag_mean(xs[0], 2, False))
        return owned(lib, "sum_all", s)

    numcheck(lib, build, lv)
    free(lib, lv)


def test_mlp(lib, jit):
    """test_autograd.c:408-437 (seed 55): matmul + bias + sigmoid, twice"""
    lib.pg_seed(55)
    x = uniform_leaf(lib, (2, 3), -1.0, 1.0)
    w1 = uniform_leaf(lib, (3, 8), -0.5, 0.5)
    b1 = leaf(lib, np.zeros(8))
    w2 = uniform_leaf(lib, (8, 2), -0.5, 0.5)
    b2 = leaf(lib, np.zeros(2))
    lv = [x, w1, b1, w2, b2]

    def build(xs):
        mm1 = lib.op("matmul", xs[0], xs[1])
        z1 = lib.op("add", mm1, xs[2])
        h = lib.op("sigmoid", z1)
        mm2 = lib.op("matmul", h, xs[3])
        y = lib.op("add", mm2, xs[4])
        for n in (mm1, z1, h, mm2):
            lib.pg_node_free(n)
        return owned(lib, "mean_all", y)

    numcheck(lib, build, lv)
    free(lib, lv)


def test_analytic(lib, jit):
    """test_autograd.c:439-470: x*x and x*x + x, the second backward twice
    into the same grad tensor"""
    raw = np.array([0.5, -1.0, 2.0, -0.25], np.float32)
    x = lib.var(raw)
    loss = owned(lib, "sum_all", lib.op("mul", x, x))
    lib.pg_backward(loss)
    np.testing.assert_allclose(lib.grad(x), 2 * raw, rtol=1e-4, atol=1e-4)
    lib.pg_node_free(loss)
    lib.pg_node_free(x)
    y = lib.var(raw)
    sq = lib.op("mul", y, y)
    s = lib.op("add", sq, y)
    lib.pg_node_free(sq)
    loss2 = owned(lib, "sum_all", s)
    lib.pg_backward(loss2)
    g2 = lib.node(y).grad
    np.testing.assert_allclose(lib.grad(y), 2 * raw + 1, rtol=1e-4, atol=1e-4)
    lib.pg_backward(loss2)
    assert lib.node(y).grad == g2
    np.testing.assert_allclose(lib.grad(y), 2 * raw + 1, rtol=1e-4, atol=1e-4)
    lib.pg_node_free(loss2)
    lib.pg_node_free(y)
