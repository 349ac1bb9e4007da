"""GPU parity of the MI355X path against the CPU oracle, through the C ABI.

Tolerances: f32 elementwise grads max relative
error <= 1e-5 (oracle_lib.max_rel: elements below 1% of max|ref| are held
to 1e-7 * max|ref| absolute, where grads pass through zero); f16/bf16 GEMM
grads relative Frobenius <= 1e-3 against the f32-accumulating oracle on the
same 16-bit operands; SGD weights <= 1e-6 relative, and in fact bit-exact.
"""
import ctypes as C

import numpy as np
import pytest

from oracle_lib import bf16_to_f32, f16_to_f32, max_rel, rel_fro
from picograd_amd.capi import BF16, F16, F32, SgdCfg

pytestmark = pytest.mark.gpu

ELEM_TOL = 1e-5
GEMM_TOL = 1e-3
SGD_TOL = 1e-6


def _shape(*s):
    return len(s), (C.c_size_t * len(s))(*s)


# ---------------------------------------------------------------- SGD

@pytest.mark.parametrize("cfg", [
    dict(lr=0.01, momentum=0.9, dampening=0.0, weight_decay=1e-4, nesterov=True),
    dict(lr=0.1, momentum=0.5, dampening=0.3, weight_decay=0.01, nesterov=False),
    dict(lr=0.05, momentum=0.0, dampening=0.0, weight_decay=0.0, nesterov=False),
])
def test_sgd_multi_tensor_matches_oracle(lib, oracle, cfg):
    rng = np.random.default_rng(7)
    shapes = [(257,), (64, 33), (1000,), (3,)]
    ps = [rng.standard_normal(s).astype(np.float32) for s in shapes]
    nodes = [lib.var(p) for p in ps]
    opt = lib.pg_sgd_new(C.byref(SgdCfg(**cfg)))
    for n in nodes:
        assert lib.pg_sgd_add_param(opt, n) == 0
    ref_p = [p.copy() for p in ps]
    ref_buf = [np.zeros_like(p) for p in ps]
    for step in range(3):
        gs = [rng.standard_normal(s).astype(np.float32) for s in shapes]
        lib.pg_sgd_zero_grad(opt)
        for n, g in zip(nodes, gs):
            # loss = sum(p * G) makes dL/dp = G exactly
            gn = lib.var(g, requires_grad=False)
            prod = lib.op("mul", n, gn)
            loss = lib.op("sum_all", prod)
            lib.pg_backward(loss)
            for x in (loss, prod, gn):
                lib.pg_node_free(x)
        lib.pg_sgd_step(opt)
        for i, g in enumerate(gs):
            oracle.sgd_step(ref_p[i], g, ref_buf[i] if cfg["momentum"] else None, cfg["lr"],
                            cfg["momentum"], cfg["dampening"], cfg["weight_decay"], cfg["nesterov"])
        for n, rp in zip(nodes, ref_p):
            got = lib.value(n)
            err = np.abs(got - rp) / np.maximum(np.abs(rp), 1e-30)
            assert err.max() <= SGD_TOL, f"step {step}: max rel {err.max():.3e}"
            # neither side fuses multiply-adds: the weights agree bit for bit
            assert np.array_equal(got.view(np.uint32), rp.view(np.uint32)), f"step {step}"
    lib.pg_sgd_free(opt)
    for n in nodes:
        lib.pg_node_free(n)


def _sgd_scalar(lib, cfg, steps, loss_fn):
    x = lib.var(np.array([1.0], np.float32))
    opt = lib.pg_sgd_new(C.byref(cfg))
    lib.pg_sgd_add_param(opt, x)
    vals = []
    for _ in range(steps):
        lib.pg_sgd_zero_grad(opt)
        loss_fn(x)
        lib.pg_sgd_step(opt)
        vals.append(float(lib.value(x)[0]))
    lib.pg_sgd_free(opt)
    lib.pg_node_free(x)
    return vals


def test_sgd_reference_known_answers(lib):
    """The trajectories of the reference's test_opt.c:48-138."""
    def loss_sq_minus_2(x):  # loss = (x - 2)^2 -> grad 2(x - 2)
        two = lib.var(np.array([2.0], np.float32), requires_grad=False)
        d = lib.op("sub", x, two)
        sq = lib.op("mul", d, d)
        l = lib.op("sum_all", sq)
        lib.pg_backward(l)
        for n in (l, sq, d, two):
            lib.pg_node_free(n)

    def loss_sq(x):
        sq = lib.op("mul", x, x)
        l = lib.op("sum_all", sq)
        lib.pg_backward(l)
        lib.pg_node_free(l)
        lib.pg_node_free(sq)

    cfg = lib.pg_sgd_cfg_default()
    cfg.lr = 0.1
    assert np.allclose(_sgd_scalar(lib, cfg, 2, loss_sq_minus_2), [1.2, 1.36], atol=1e-5)
    cfg.momentum = 0.9
    assert np.allclose(_sgd_scalar(lib, cfg, 2, loss_sq_minus_2), [1.2, 1.54], atol=1e-5)
    cfg = lib.pg_sgd_cfg_default()
    cfg.lr, cfg.weight_decay = 0.1, 0.5
    assert np.allclose(_sgd_scalar(lib, cfg, 1, loss_sq), [0.75], atol=1e-5)
    cfg = lib.pg_sgd_cfg_default()
    cfg.lr, cfg.momentum, cfg.nesterov = 0.1, 0.5, True
    assert np.allclose(_sgd_scalar(lib, cfg, 2, loss_sq_minus_2), [1.3, 1.56], atol=1e-5)


# ---------------------------------------------------------------- elementwise chains

def _chain1(lib, a, b, c):
    na, nb, nc = lib.var(a), lib.var(b), lib.var(c)
    t0 = lib.op("add", na, nb)
    t1 = lib.op("mul", t0, nc)
    t2 = lib.op("relu", t1)
    t3 = lib.op("tanh", t2)
    loss = lib.op("sum_all", t3)
    lib.pg_backward(loss)
    out = [lib.grad(n) for n in (na, nb, nc)]
    for n in (loss, t3, t2, t1, t0, na, nb, nc):
        lib.pg_node_free(n)
    return out


@pytest.mark.parametrize("shape", [(64, 64), (7, 13), (3, 5, 8)])
@pytest.mark.parametrize("jit", [True, False])
def test_chain1_grads_match_oracle(lib, oracle, shape, jit):
    """Config 1: loss = sum_all(tanh(relu((a + b) * c))), a, b, c ~ U[-1, 1]."""
    oracle.orc_seed(42)
    n = int(np.prod(shape))
    a, b, c = (oracle.uniform(n, -1.0, 1.0).reshape(shape) for _ in range(3))
    lib.pg_autograd_set_jit(jit)
    try:
        got = _chain1(lib, a, b, c)
        if jit:
            assert lib.pg_autograd_last_was_jit(), lib.pg_autograd_last_error().decode()
    finally:
        lib.pg_autograd_set_jit(True)
    ref = oracle.chain1(a.ravel().copy(), b.ravel().copy(), c.ravel().copy())
    for g, r in zip(got, ref):
        assert g.shape == shape
        assert max_rel(g.ravel(), r) <= ELEM_TOL


def _chain2(lib, x, bias, g):
    nx, nb, ng = lib.var(x), lib.var(bias), lib.var(g)
    t0 = lib.op("add", nx, nb)
    t1 = lib.op("gelu", t0)
    t2 = lib.op("sigmoid", ng)
    y = lib.op("mul", t1, t2)
    loss = lib.op("sum_all", y)
    lib.pg_backward(loss)
    out = [lib.grad(n) for n in (nx, ng, nb)]
    lv = float(lib.value(loss)[0])
    for n in (loss, y, t2, t1, t0, nx, nb, ng):
        lib.pg_node_free(n)
    return out, lv


def dbias_bound(rdx: np.ndarray, depth: int = 128) -> np.ndarray:
    """How far a device column sum of dx may sit from the f64 sum of the
    oracle's addends: the f32 rounding of a sum tree of depth <= 128,
    depth * 2^-24 * sum|dx| (the fused kernel's depth for loops up to
    [16384, 4096] is at most 88: 4 rows per lane, 4 row lanes, up to 64
    partial rows per finisher lane, 16 finisher lanes), plus the elementwise
    tolerance of the addends.  A dropped 16-row band moves a column by
    ~16 / R of sum|dx|, about 1e-3 at R = 16384, well outside it."""
    absum = np.abs(rdx.astype(np.float64)).sum(axis=0)
    return (ELEM_TOL + depth * 2.0 ** -24) * absum + 1e-30


@pytest.mark.parametrize("R,Cc", [(512, 1024), (37, 515), (1, 8), (1000, 4), (4096, 64), (4000, 64),
                                  (3000, 63), (24000, 64), (33001, 63)])
@pytest.mark.parametrize("jit", [True, False])
def test_chain2_broadcast_grads_match_oracle(lib, oracle, R, Cc, jit):
    """Config 2 at reduced size: y = gelu(x + bias) * sigmoid(g), dbias is a
    column sum over R rows fused into the backward kernel.  The narrow
    shapes leave one column block, so the fused kernel writes one partial
    row per 16-row band: 256, 250 and 188 rows take only the finisher's
    one-row loop (each of its 128 block lanes adds every 128th row); 1500
    and 2063 rows also take its eight-deep loop (once or twice per lane, then
    the one-row loop), as config 2's full shape does (1024 rows, eight per
    lane); (33001, 63) also ends on a partial band."""
    oracle.orc_seed(43)
    x = oracle.normal(R * Cc, 0.0, 1.0).reshape(R, Cc)
    bias = oracle.normal(Cc, 0.0, 0.1)
    g = oracle.normal(R * Cc, 0.0, 1.0).reshape(R, Cc)
    lib.pg_autograd_set_jit(jit)
    try:
        (dx, dg, db), _ = _chain2(lib, x, bias, g)
        if jit:
            assert lib.pg_autograd_last_was_jit(), lib.pg_autograd_last_error().decode()
    finally:
        lib.pg_autograd_set_jit(True)
    rdx, rdg, rdb, rdb64 = oracle.chain2(x, bias, g)
    assert max_rel(dx, rdx) <= ELEM_TOL
    assert max_rel(dg, rdg) <= ELEM_TOL
    # dbias against the f64 sum of the oracle's addends (the eager path adds
    # the R rows serially, as the reference does); the oracle's own serial
    # f32 sum within its summation bound
    assert np.all(np.abs(db - rdb64) <= dbias_bound(rdx, 128 if jit else max(R, 128)))
    absum = np.abs(rdx.astype(np.float64)).sum(axis=0)
    assert np.all(np.abs(rdb - rdb64) <= R * 2.0 ** -24 * absum + 1e-30)


# ---------------------------------------------------------------- GEMM

@pytest.mark.parametrize("dtype", [BF16, F16])
@pytest.mark.parametrize("m,n,k", [(129, 96, 40), (64, 64, 64), (1, 1, 8), (17, 33, 9), (300, 260, 1000)])
def test_gemm_ex_matches_oracle(lib, oracle, dtype, m, n, k):
    rng = np.random.default_rng(m * 1000 + n + k)
    a16 = oracle.cast16(dtype, rng.standard_normal((m, k)).astype(np.float32))
    b16 = oracle.cast16(dtype, rng.standard_normal((k, n)).astype(np.float32))
    ta, tb = lib.tensor(a16, dtype), lib.tensor(b16, dtype)
    nd, sh = _shape(m, n)
    tc = lib.pg_tensor_empty_dtype(F32, nd, sh)
    ti = lib.tinfo
    lib.pg_gemm_ex(dtype, m, n, k, ti(ta).dev, k, ti(tb).dev, n, ti(tc).dev, n)
    got = lib.read(tc)
    ref = oracle.gemm(dtype, a16, b16)
    assert rel_fro(got, ref) <= 1e-5
    for t in (ta, tb, tc):
        lib.pg_tensor_free(t)


@pytest.mark.parametrize("dtype", [BF16, F16])
@pytest.mark.parametrize("M,K,N", [(256, 192, 320), (129, 40, 96), (65, 1000, 33)])
def test_matmul_backward_16bit_matches_oracle(lib, oracle, dtype, M, K, N):
    """dA = dC . W^T and dW = A^T . dC with 16-bit operands, f32 grads."""
    rng = np.random.default_rng(M + K + N)
    a16 = oracle.cast16(dtype, rng.standard_normal((M, K)).astype(np.float32))
    w16 = oracle.cast16(dtype, (0.02 * rng.standard_normal((K, N))).astype(np.float32))
    dc = rng.standard_normal((M, N)).astype(np.float32)
    na, nw = lib.var(a16, dtype=dtype), lib.var(w16, dtype=dtype)
    c = lib.op("matmul", na, nw)
    seed = lib.tensor(dc)
    lib.pg_amd_backward_from(c, seed)
    dA, dW = lib.grad(na), lib.grad(nw)
    dc16 = oracle.cast16(dtype, dc)
    ref_dA = oracle.gemm(dtype, dc16, w16, tb=True)
    ref_dW = oracle.gemm(dtype, a16, dc16, ta=True)
    assert rel_fro(dA, ref_dA) <= GEMM_TOL
    assert rel_fro(dW, ref_dW) <= GEMM_TOL
    # same operands, so the only difference is summation order
    assert rel_fro(dA, ref_dA) <= 1e-5 and rel_fro(dW, ref_dW) <= 1e-5
    lib.pg_tensor_free(seed)
    for n in (c, na, nw):
        lib.pg_node_free(n)


@pytest.mark.parametrize("dtype", [BF16, F16])
@pytest.mark.parametrize("abat,wbat", [(True, True), (True, False), (False, True)])
def test_matmul_backward_batched_matches_oracle(lib, oracle, dtype, abat, wbat):
    """Batched 16-bit matmul backward (autograd.c:592-610): both operands
    batched; only A batched (the batch folds into the wgrad reduction);
    only W batched (dA accumulates over the batch).  K and N ragged, so the
    k-tail and padding paths run."""
    Bt, M, K, N = 3, 72, 40, 100
    rng = np.random.default_rng(Bt * 100 + abat * 10 + wbat)
    ash = (Bt, M, K) if abat else (M, K)
    wsh = (Bt, K, N) if wbat else (K, N)
    a16 = oracle.cast16(dtype, rng.standard_normal(ash).astype(np.float32))
    w16 = oracle.cast16(dtype, (0.05 * rng.standard_normal(wsh)).astype(np.float32))
    dc = rng.standard_normal((Bt, M, N)).astype(np.float32)
    na, nw = lib.var(a16, dtype=dtype), lib.var(w16, dtype=dtype)
    c = lib.op("matmul", na, nw)
    assert lib.shape(lib.node(c).value) == (Bt, M, N)
    seed = lib.tensor(dc)
    lib.pg_amd_backward_from(c, seed)
    dA, dW = lib.grad(na), lib.grad(nw)
    dc16 = oracle.cast16(dtype, dc)
    ra = [oracle.gemm(dtype, dc16[z], w16[z] if wbat else w16, tb=True, f64=True) for z in range(Bt)]
    rw = [oracle.gemm(dtype, a16[z] if abat else a16, dc16[z], ta=True, f64=True) for z in range(Bt)]
    ref_dA = np.stack(ra) if abat else np.sum(ra, axis=0)
    ref_dW = np.stack(rw) if wbat else np.sum(rw, axis=0)
    assert rel_fro(dA, ref_dA) <= 1e-5
    assert rel_fro(dW, ref_dW) <= 1e-5
    lib.pg_tensor_free(seed)
    for n in (c, na, nw):
        lib.pg_node_free(n)


@pytest.mark.parametrize("dtype", [BF16, F16])
@pytest.mark.parametrize("M,K,N", [(520, 256, 264), (300, 200, 10), (8, 64, 8), (1, 8, 1)])
def test_matmul_forward_16bit_matches_oracle(lib, oracle, dtype, M, K, N):
    """pg_matmul on 16-bit operands (matmul.c:186-284): f32 output of
    f32-accumulated products; tiles of both sizes, padded N (the 10-wide
    output layer of config 5) and single-element edges."""
    rng = np.random.default_rng(M + K + N)
    a16 = oracle.cast16(dtype, rng.standard_normal((M, K)).astype(np.float32))
    w16 = oracle.cast16(dtype, rng.standard_normal((K, N)).astype(np.float32))
    na, nw = lib.var(a16, dtype=dtype), lib.var(w16, dtype=dtype)
    c = lib.op("matmul", na, nw)
    assert rel_fro(lib.value(c), oracle.gemm(dtype, a16, w16, f64=True)) <= 1e-5
    for n in (c, na, nw):
        lib.pg_node_free(n)


# ---------------------------------------------------------------- JIT API

def _jit_run(lib, build, inputs):
    g = lib.pg_jit_graph_new()
    out_id = build(g)
    lib.pg_jit_mark_output(g, out_id)
    exe = lib.pg_jit_compile(g)
    assert exe, lib.pg_jit_last_error().decode()
    ts = [lib.tensor(x) for x in inputs]
    arr = (C.c_void_p * len(ts))(*ts)
    out = lib.pg_jit_run_single(exe, arr, len(ts))
    assert out, lib.pg_jit_last_error().decode()
    res = lib.read(out)
    for t in ts + [out]:
        lib.pg_tensor_free(t)
    lib.pg_jit_exe_free(exe)
    lib.pg_jit_graph_free(g)
    return res


def test_jit_reference_known_answers(lib):
    """Expected vectors of the reference's test_jit.c:17-62."""
    def fused(g):
        s23 = _shape(2, 3)
        a, b, c = (lib.pg_jit_add_input(g, *s23) for _ in range(3))
        return lib.pg_jit_relu(g, lib.pg_jit_mul(g, lib.pg_jit_add(g, a, b), c))

    got = _jit_run(lib, fused, [np.array([[1, -2, 3], [4, -5, 6]], np.float32),
                                np.array([[6, 5, 4], [3, 2, 1]], np.float32),
                                np.ones((2, 3), np.float32)])
    assert np.array_equal(got.ravel(), [7, 3, 7, 7, 0, 7])

    def bcast(g):
        a = lib.pg_jit_add_input(g, *_shape(2, 4))
        b = lib.pg_jit_add_input(g, *_shape(4))
        return lib.pg_jit_relu(g, lib.pg_jit_add(g, a, b))

    got = _jit_run(lib, bcast, [np.array([[-1, 2, -3, 4], [-5, 6, -7, 8]], np.float32),
                                np.array([10, 20, 30, 40], np.float32)])
    assert np.array_equal(got.ravel(), [9, 22, 27, 44, 5, 26, 23, 48])


def test_repeat_backward_same_grad_tensor(lib):
    """d(x^2 + x)/dx = 2x + 1; a second backward on the same graph returns
    the same grad tensor with the same values (test_autograd.c:439-470)."""
    x0 = np.array([1.5, -2.0, 0.25], np.float32)
    x = lib.var(x0)
    sq = lib.op("mul", x, x)
    s = lib.op("add", sq, x)
    loss = lib.op("sum_all", s)
    lib.pg_backward(loss)
    g1 = lib.node(x).grad
    v1 = lib.grad(x)
    lib.pg_backward(loss)
    assert lib.node(x).grad == g1
    assert np.allclose(lib.grad(x), v1)
    assert np.allclose(v1, 2 * x0 + 1, rtol=1e-6)
    for n in (loss, s, sq, x):
        lib.pg_node_free(n)
