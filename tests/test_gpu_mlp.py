"""Config 5 on the MI355X through the C ABI: the mixed-precision matmul
(pg_amd_ag_matmul16) and the full MLP training step against the CPU oracle
and the reference's own golden f32 run.

Tolerances: GEMM grads relative Frobenius <= 1e-3 against the oracle on the
same 16-bit operands; f32 grads of the golden
run 1e-5 relative Frobenius; updated weights 1e-6 relative (f32 run) or the
update itself within 1e-3 relative Frobenius (16-bit runs, where the grads
carry the GEMM tolerance).
"""
import ctypes as C

import numpy as np
import pytest

from oracle_lib import bf16_to_f32, f16_to_f32, rel_fro
from picograd_amd.capi import BF16, F16, F32
from picograd_amd.mlp import Mlp

pytestmark = pytest.mark.gpu

GEMM_TOL = 1e-3


def golden(name):
    from pathlib import Path
    with np.load(Path(__file__).resolve().parent / "golden" / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _round(oracle, dt, x):
    h = oracle.cast16(dt, x)
    return bf16_to_f32(h) if dt == BF16 else f16_to_f32(h)


# ---------------------------------------------------------------- matmul16

@pytest.mark.parametrize("dt", [BF16, F16])
@pytest.mark.parametrize("M,K,N", [(128, 192, 256), (70, 50, 10), (33, 64, 72), (256, 1024, 8)])
def test_matmul16_forward_backward(lib, oracle, dt, M, K, N):
    """C = q(A).q(B), dA = q(G).q(B)^T, dB = q(A)^T.q(G) with G = dL/dC
    (loss = sum_all(C * G)); K or N off a multiple of 8 take the padded
    copies, the rest the kept 16-bit copies."""
    print(f"matmul16 dt={dt} M={M} K={K} N={N}", flush=True)
    rng = np.random.default_rng(M * 7 + K + N)
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    g = rng.standard_normal((M, N)).astype(np.float32)
    na, nb = lib.var(a), lib.var(b)
    c = lib._check(lib.pg_amd_ag_matmul16(na, nb, dt))
    ng = lib.var(g, requires_grad=False)
    prod = lib.op("mul", c, ng)
    loss = lib.op("sum_all", prod)
    lib.pg_backward(loss)
    qa, qb, qg = _round(oracle, dt, a), _round(oracle, dt, b), _round(oracle, dt, g)
    assert rel_fro(lib.value(c), oracle.gemm(F32, qa, qb)) < GEMM_TOL
    assert rel_fro(lib.grad(na), oracle.gemm(F32, qg, qb, tb=True)) < GEMM_TOL
    assert rel_fro(lib.grad(nb), oracle.gemm(F32, qa, qg, ta=True)) < GEMM_TOL
    for n in (loss, prod, ng, c, na, nb):
        lib.pg_node_free(n)


def test_matmul16_rejects_bad_input(lib):
    a = lib.var(np.ones((4, 8), np.float32))
    b = lib.var(np.ones((6, 8), np.float32))
    assert not lib.pg_amd_ag_matmul16(a, b, BF16)  # inner dims differ
    assert b"matmul16" in lib.pg_autograd_last_error()
    c = lib.var(np.ones((8, 8), np.float32))
    assert not lib.pg_amd_ag_matmul16(a, c, F32)  # not a 16-bit dtype
    for n in (a, b, c):
        lib.pg_node_free(n)


def test_matmul16_kept_copy_follows_writes(lib, oracle):
    """The 16-bit copy of an operand is remade after writes to its tensor
    (fill, copy from host, a JIT output, a raw write reported with
    pg_amd_tensor_modified) and rewritten by pg_sgd_step: with A = I the
    product returns q(B) exactly."""
    from picograd_amd.capi import SgdCfg
    K = 64
    eye = lib.var(np.eye(K, dtype=np.float32), requires_grad=False)
    rng = np.random.default_rng(3)
    w0 = rng.standard_normal((K, K)).astype(np.float32)
    w = lib.var(w0)

    def qw():
        c = lib._check(lib.pg_amd_ag_matmul16(eye, w, BF16))
        v = lib.value(c)
        lib.pg_node_free(c)
        return v

    assert np.array_equal(qw(), _round(oracle, BF16, w0))
    wt = lib.node(w).value
    lib.pg_tensor_fill(wt, 0.3)
    assert np.array_equal(qw(), _round(oracle, BF16, np.full((K, K), 0.3, np.float32)))
    w1 = rng.standard_normal((K, K)).astype(np.float32)
    assert lib.pg_tensor_copy_from_host(wt, w1.ctypes.data)
    assert np.array_equal(qw(), _round(oracle, BF16, w1))
    # an SGD step rewrites the copy from the updated weights
    opt = lib.pg_sgd_new(C.byref(SgdCfg(0.1, 0.9, 0.0, 1e-4, True)))
    assert lib.pg_sgd_add_param(opt, w) == 0
    c = lib._check(lib.pg_amd_ag_matmul16(eye, w, BF16))
    loss = lib.op("sum_all", c)
    lib.pg_backward(loss)
    lib.pg_sgd_step(opt)
    lib.pg_node_free(loss)
    lib.pg_node_free(c)
    w2 = lib.value(w)
    assert not np.array_equal(w2, w1)
    assert np.array_equal(qw(), _round(oracle, BF16, w2))
    # a fused-JIT kernel writing the tensor as an output
    g = lib.pg_jit_graph_new()
    shp = (C.c_size_t * 2)(K, K)
    xin = lib.pg_jit_add_input(g, 2, shp)
    y = lib.pg_jit_mul(g, xin, lib.pg_jit_add_const(g, 2.0))
    lib.pg_jit_mark_output(g, y)
    exe = lib.pg_jit_compile(g)
    assert exe, lib.pg_jit_last_error()
    src = lib.tensor(w0)
    ins = (C.c_void_p * 1)(src)
    outs = (C.c_void_p * 1)(wt)
    assert lib.pg_jit_run(exe, ins, 1, outs, 1), lib.pg_jit_last_error()
    assert np.array_equal(qw(), _round(oracle, BF16, 2 * w0))
    lib.pg_jit_exe_free(exe)
    lib.pg_jit_graph_free(g)
    lib.pg_tensor_free(src)
    # a raw-pointer write (pg_gemm_ex into the tensor's storage), reported
    # with pg_amd_tensor_modified
    a16 = oracle.cast16(BF16, np.eye(K, dtype=np.float32))
    b16 = oracle.cast16(BF16, w1)
    ta, tb = lib.tensor(a16, BF16), lib.tensor(b16, BF16)
    lib.pg_gemm_ex(BF16, K, K, K, lib.tinfo(ta).dev, K, lib.tinfo(tb).dev, K, lib.tinfo(wt).dev, K)
    lib.pg_amd_tensor_modified(wt)
    assert np.array_equal(qw(), _round(oracle, BF16, w1))
    lib.pg_tensor_free(ta)
    lib.pg_tensor_free(tb)
    lib.pg_sgd_free(opt)
    lib.pg_node_free(w)
    lib.pg_node_free(eye)


# ---------------------------------------------------------------- linear16

def _act_np(act, z):
    from scipy.special import erf
    z = z.astype(np.float64)
    if act == 1:
        return np.maximum(z, 0.0), (z > 0).astype(np.float64)
    if act == 2:
        cdf = 0.5 * (1.0 + erf(z / np.sqrt(2.0)))
        return z * cdf, cdf + z * np.exp(-0.5 * z * z) / np.sqrt(2.0 * np.pi)
    return z, np.ones_like(z)


@pytest.mark.parametrize("dt", [BF16, F16])
@pytest.mark.parametrize("act", [0, 1, 2])
@pytest.mark.parametrize("M,K,N,bias", [(256, 192, 256, True), (70, 50, 10, True), (64, 128, 72, False),
                                        (512, 4096, 16, True)])
def test_linear16_matches_oracle(lib, oracle, dt, act, M, K, N, bias):
    """out = act(q(x).q(W) + b) and its grads: dz = dout * act'(z),
    db = sum_rows dz, dx = q(dz).q(W)^T, dW = q(x)^T.q(dz).  The shapes
    cover the fused GEMM epilogue (one launch), the epilogue pass after a
    k-tail (K = 50) or split-K (K = 4096, N = 16), and padded N = 10."""
    print(f"linear16 dt={dt} act={act} M={M} K={K} N={N} bias={bias}", flush=True)
    rng = np.random.default_rng(M + 3 * K + 7 * N + act)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    b = (0.3 * rng.standard_normal(N)).astype(np.float32)
    g = rng.standard_normal((M, N)).astype(np.float32)
    nx, nw = lib.var(x), lib.var(w)
    nb = lib.var(b) if bias else None
    out = lib._check(lib.pg_amd_ag_linear16(nx, nw, nb, act, dt))
    ng = lib.var(g, requires_grad=False)
    prod = lib.op("mul", out, ng)
    loss = lib.op("sum_all", prod)
    lib.pg_backward(loss)
    qx, qw = _round(oracle, dt, x), _round(oracle, dt, w)
    z = oracle.gemm(F32, qx, qw).astype(np.float64) + (b if bias else 0.0)
    o, d = _act_np(act, z)
    got = lib.value(out)
    assert rel_fro(got, o) < GEMM_TOL
    if act == 1:
        # ReLU' is a step: where z is within rounding of 0 the device's sign
        # decides, and out > 0 exactly when its z > 0
        d = (got > 0).astype(np.float64)
    dz = g.astype(np.float64) * d
    qdz = _round(oracle, dt, dz.astype(np.float32))
    assert rel_fro(lib.grad(nx), oracle.gemm(F32, qdz, qw, tb=True)) < GEMM_TOL
    assert rel_fro(lib.grad(nw), oracle.gemm(F32, qx, qdz, ta=True)) < GEMM_TOL
    if bias:
        assert rel_fro(lib.grad(nb), dz.sum(axis=0)) < GEMM_TOL
    for n in (loss, prod, ng, out, nx, nw) + ((nb,) if bias else ()):
        lib.pg_node_free(n)


def test_linear16_output_feeds_next_layer(lib, oracle):
    """Two stacked layers: the second reads the first's 16-bit output copy
    written by the GEMM epilogue; the result equals rounding the first
    layer's f32 output."""
    rng = np.random.default_rng(21)
    x = rng.standard_normal((128, 64)).astype(np.float32)
    w1 = (rng.standard_normal((64, 96)) / 8).astype(np.float32)
    w2 = (rng.standard_normal((96, 40)) / 10).astype(np.float32)
    nx, n1, n2 = lib.var(x, requires_grad=False), lib.var(w1), lib.var(w2)
    h = lib._check(lib.pg_amd_ag_linear16(nx, n1, None, 2, BF16))
    y = lib._check(lib.pg_amd_ag_linear16(h, n2, None, 0, BF16))
    want = oracle.gemm(F32, _round(oracle, BF16, lib.value(h)), _round(oracle, BF16, w2))
    assert rel_fro(lib.value(y), want) < 1e-5
    for n in (y, h, nx, n1, n2):
        lib.pg_node_free(n)


def test_linear16_rejects_bad_input(lib):
    a = lib.var(np.ones((4, 8), np.float32))
    w = lib.var(np.ones((8, 6), np.float32))
    b = lib.var(np.ones(5, np.float32))
    assert not lib.pg_amd_ag_linear16(a, w, b, 0, BF16)  # bias length
    assert not lib.pg_amd_ag_linear16(a, w, None, 3, BF16)  # act code
    assert not lib.pg_amd_ag_linear16(a, w, None, 0, F32)  # dtype
    for n in (a, w, b):
        lib.pg_node_free(n)


# ---------------------------------------------------------------- MLP step

def _read_params(lib, mlp):
    return [lib.value(n) for n in mlp.Ws], [lib.value(n) for n in mlp.bs]


def _read_grads(lib, mlp):
    return [lib.grad(n) for n in mlp.Ws], [lib.grad(n) for n in mlp.bs]


def test_mlp_f32_matches_reference_golden(lib):
    """The f32 graph (pg_ag_matmul) reproduces two training steps of the
    reference's own MLP run: loss, every grad, the updated parameters."""
    g = golden("mlp")
    L = len(g["dims"]) - 1
    mlp = Mlp.from_arrays(lib, [g[f"W{i}_0"] for i in range(L)], [g[f"b{i}_0"] for i in range(L)], F32)
    x, t = lib.var(g["x"], requires_grad=False), lib.var(g["t"], requires_grad=False)
    for s in (1, 2):
        loss = mlp.step(x, t, keep_loss=True)
        assert abs(lib.value(loss)[0] - g[f"loss_{s}"][0]) <= 1e-6 * abs(g[f"loss_{s}"][0])
        lib.pg_node_free(loss)
        dW, db = _read_grads(lib, mlp)
        Ws, bs = _read_params(lib, mlp)
        for i in range(L):
            assert rel_fro(dW[i], g[f"dW{i}_{s}"]) < 1e-5, (s, i)
            assert rel_fro(db[i], g[f"db{i}_{s}"]) < 1e-5, (s, i)
            for got, key in ((Ws[i], f"W{i}_{s}"), (bs[i], f"b{i}_{s}")):
                assert np.abs(got - g[key]).max() <= 1e-6 * np.abs(g[key]).max(), (s, key)
    mlp.free()
    lib.pg_node_free(x)
    lib.pg_node_free(t)


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("dt", [BF16, F16])
@pytest.mark.parametrize("dims,batch", [((96, 128, 128, 128, 10), 64), ((50, 96, 72, 10), 40)])
def test_mlp_16bit_matches_oracle(lib, oracle, dt, dims, batch, fused):
    """Two steps of the 16-bit network (matmul16 + add + gelu nodes, or one
    linear16 node per layer) against orc_mlp_step on the same inputs.
    Step 2 reads the weight copies pg_sgd_step wrote in step 1."""
    print(f"mlp dt={dt} dims={dims} batch={batch} fused={fused}", flush=True)
    rng = np.random.default_rng(sum(dims) + batch)
    Ws = [(rng.uniform(-1, 1, (dims[i], dims[i + 1])) / np.sqrt(dims[i])).astype(np.float32)
          for i in range(len(dims) - 1)]
    bs = [(0.1 * rng.standard_normal(dims[i + 1])).astype(np.float32) for i in range(len(dims) - 1)]
    x = rng.standard_normal((batch, dims[0])).astype(np.float32)
    t = rng.standard_normal((batch, dims[-1])).astype(np.float32)
    mlp = Mlp.from_arrays(lib, Ws, bs, dt, fused=fused)
    nx, nt = lib.var(x, requires_grad=False), lib.var(t, requires_grad=False)
    rW, rb = [w.copy() for w in Ws], [b.copy() for b in bs]
    rWb, rbb = [np.zeros_like(w) for w in Ws], [np.zeros_like(b) for b in bs]
    for s in (1, 2):
        prevW, prevb = _read_params(lib, mlp)
        loss = mlp.step(nx, nt, keep_loss=True)
        rloss, rdW, rdb = oracle.mlp_step(dt, x, t, rW, rb, rWb, rbb, 0.01, 0.9, 0.0, 1e-4, True)
        assert abs(lib.value(loss)[0] - rloss) <= 1e-4 * abs(rloss), s
        lib.pg_node_free(loss)
        dW, db = _read_grads(lib, mlp)
        Wn, bn = _read_params(lib, mlp)
        for i in range(len(Ws)):
            assert rel_fro(dW[i], rdW[i]) < GEMM_TOL, (s, "dW", i, rel_fro(dW[i], rdW[i]))
            assert rel_fro(db[i], rdb[i]) < GEMM_TOL, (s, "db", i, rel_fro(db[i], rdb[i]))
            # the update applied, against the oracle's update from the same start
            assert rel_fro(Wn[i] - prevW[i], rW[i] - prevW[i]) < GEMM_TOL, (s, "W", i)
            assert rel_fro(bn[i] - prevb[i], rb[i] - prevb[i]) < GEMM_TOL, (s, "b", i)
        # continue the oracle from the device's parameters so step 2 compares
        # grads of identical inputs
        for i in range(len(Ws)):
            rW[i][...] = Wn[i]
            rb[i][...] = bn[i]
    mlp.free()
    lib.pg_node_free(nx)
    lib.pg_node_free(nt)
