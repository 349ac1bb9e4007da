"""Narrow dgrads of linear16 layers: dx = q(dz).q(W)^T for a layer of at
most 16 outputs is formed by a pass that runs the GEMM's own MFMA sequence
(pgk_act_bwd16n), so dx must have the bits of the GEMM path that
pg_amd_linear16_narrow(false) restores, and both must hold the f32
summation bound against the f64 product of the same 16-bit operands (dz
read back from the node, W rounded here).

Fused (x is another linear16 node, whose activation pass forms dx and
derives its own dz from it in the same pass; dx is written when read):
  - dx and that node's dz bit for bit as with the narrow path off (GEMM,
    then the activation pass reading dx back);
  - ReLU: dz = q(dx * (z > 0)) bit for bit, computed here from the read-back
    dx and pre-activation z; GELU (bf16): within one bf16 ulp of
    q(orc_gelu_backward(z, dx));
  - db within the summation bound of the f64 column sums of dz.
Cases: ragged rows (a last partial 32-row step), widths with n % 16 != 0
(a lane's columns partly past n) and n % 4 != 0 (the lane-scalar path),
layer widths 1, 10 and 16 (k of 8 and 16), both 16-bit types.

Formed alone (x a leaf): the same bits as the GEMM.  With two narrow
consumers of one linear16 output, the second consumer's grad write forms
the first's pending product before adding its own (the walk's order), so
x's grad is the sum of both products.

In the fused case x's grad is not written by the backward at all: it stays
pending, over the dz of the narrow layer and a copy of its weights, until
read.  Read after an SGD step has rewritten those weights (and their
16-bit copy), it must still be the product of the weights the backward
used; a second backward drops the first's pending product.
"""
import ctypes as C

import numpy as np
import pytest

from gemm_check import check_product
from oracle_lib import bf16_to_f32, f16_to_f32
from picograd_amd.capi import BF16, F16, SgdCfg
from test_gpu_full_shapes import _dz_within_one_ulp
from test_gpu_parity import dbias_bound

pytestmark = pytest.mark.gpu

RELU, GELU, NONE = 1, 2, 0


def _dec(dt, bits):
    return f16_to_f32(bits) if dt == F16 else bf16_to_f32(bits)


def _q(oracle, dt, x):
    return _dec(dt, oracle.cast16(dt, np.ascontiguousarray(x, dtype=np.float32)))


def _kept_dz(lib, node, n):
    kept = lib.pg_amd_linear16_dz(node)
    assert kept, "linear16 backward kept no dz"
    bits = lib.read(kept)
    assert not bits[:, n:].any(), "dz pad columns not zero"
    return np.ascontiguousarray(bits[:, :n])


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.fixture
def keep_dz(lib):
    lib.pg_amd_linear16_keep_dz(True)
    yield
    lib.pg_amd_linear16_keep_dz(False)
    lib.pg_amd_linear16_narrow(True)


def _two_layers(lib, arrays, act, dt, narrow):
    """h = act(x W1 + b1), out = h W2 + b2, backward from out with seed g;
    returns h's grad, dz and pre-activation, b1's and W1's grads and the
    narrow layer's dz (bits)"""
    x, w1, b1, w2, b2, g = arrays
    lib.pg_amd_linear16_narrow(narrow)
    nx, n1w, n1b, n2w, n2b = (lib.var(v) for v in (x, w1, b1, w2, b2))
    h = lib._check(lib.pg_amd_ag_linear16(nx, n1w, n1b, act, dt))
    out = lib._check(lib.pg_amd_ag_linear16(h, n2w, n2b, NONE, dt))
    seed = lib.tensor(g)
    lib.pg_amd_backward_from(out, seed)
    H, N = w1.shape[1], w2.shape[1]
    res = {"dh": lib.grad(h), "dz1": _kept_dz(lib, h, H), "z1": lib.read(lib.pg_amd_linear16_preact(h)),
           "db1": lib.grad(n1b), "dw1": lib.grad(n1w), "dz2": _kept_dz(lib, out, N)}
    lib.pg_tensor_free(seed)
    for n in (out, h, nx, n1w, n1b, n2w, n2b):
        lib.pg_node_free(n)
    return res


@pytest.mark.parametrize(
    "M,F,H,N,act,dt",
    [
        (1037, 96, 300, 10, RELU, BF16),
        (1037, 96, 300, 10, GELU, BF16),
        (700, 64, 301, 16, RELU, F16),
        (259, 40, 130, 1, GELU, BF16),
        (4096, 256, 4096, 10, GELU, BF16),
    ],
)
def test_fused_narrow_dgrad(lib, oracle, keep_dz, M, F, H, N, act, dt):
    print(f"fused narrow dgrad M={M} F={F} H={H} N={N} act={act} dt={dt}", flush=True)
    rng = np.random.default_rng(M + H + N + act)
    arrays = (rng.standard_normal((M, F)).astype(np.float32),
              (rng.standard_normal((F, H)) / np.sqrt(F)).astype(np.float32),
              (0.1 * rng.standard_normal(H)).astype(np.float32),
              (rng.standard_normal((H, N)) / np.sqrt(H)).astype(np.float32),
              (0.1 * rng.standard_normal(N)).astype(np.float32),
              rng.standard_normal((M, N)).astype(np.float32))
    on = _two_layers(lib, arrays, act, dt, True)
    off = _two_layers(lib, arrays, act, dt, False)
    # the narrow layer's dz is q(g) either way; dh is the GEMM's, bit for bit
    assert np.array_equal(on["dz2"], oracle.cast16(dt, arrays[5]))
    assert np.array_equal(on["dz2"], off["dz2"])
    assert np.array_equal(_bits(on["dh"]), _bits(off["dh"])), "fused dh differs from the GEMM's"
    check_product(on["dh"], [(_dec(dt, on["dz2"]), _q(oracle, dt, arrays[3]).T)], "fused narrow: dh",
                  planted=False)
    # h's own dz, formed from dh in the same pass: the activation pass's bits
    assert np.array_equal(on["dz1"], off["dz1"]), "fused dz differs from the activation pass's"
    dh, z1, dz1 = on["dh"], on["z1"], on["dz1"]
    if act == RELU:
        d = dh * (z1 > 0).astype(np.float32)
        assert np.array_equal(dz1, oracle.cast16(dt, d))
    else:
        d = oracle.gelu_backward(z1, dh)
        frac = _dz_within_one_ulp(dz1, oracle.cast16(BF16, d), z1, dh)
        assert frac <= 1e-3, frac
    # db: the fused pass's own column-sum order, within the summation bound
    for res in (on, off):
        assert np.all(np.abs(res["db1"] - d.astype(np.float64).sum(axis=0)) <= dbias_bound(d, 128))
    assert np.array_equal(_bits(on["dw1"]), _bits(off["dw1"]))


@pytest.mark.parametrize("dt", [BF16, F16])
@pytest.mark.parametrize("N", [10, 4])
def test_narrow_dgrad_of_a_leaf(lib, oracle, keep_dz, dt, N):
    """x a leaf: the narrow dgrad is formed at once, the GEMM's bits"""
    print(f"narrow dgrad of a leaf dt={dt} N={N}", flush=True)
    rng = np.random.default_rng(11 + dt + N)
    M, K = 777, 515
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    g = rng.standard_normal((M, N)).astype(np.float32)
    grads = []
    for narrow in (True, False):
        lib.pg_amd_linear16_narrow(narrow)
        nx, nw = lib.var(x), lib.var(w)
        out = lib._check(lib.pg_amd_ag_linear16(nx, nw, None, NONE, dt))
        seed = lib.tensor(g)
        lib.pg_amd_backward_from(out, seed)
        dz = _dec(dt, _kept_dz(lib, out, N))
        dx = lib.grad(nx)
        check_product(dx, [(dz, _q(oracle, dt, w).T)], f"narrow dgrad, narrow={narrow}", planted=False)
        grads.append(dx)
        lib.pg_tensor_free(seed)
        for n in (out, nx, nw):
            lib.pg_node_free(n)
    assert np.array_equal(_bits(grads[0]), _bits(grads[1]))


def test_two_narrow_consumers(lib, oracle, keep_dz):
    """h feeds two narrow layers; loss = mse(a, ta) + mse(b, tb).  The first
    narrow consumer leaves its product pending on h's grad, the second's
    grad write forms it before adding its own, and h's backward then reads
    the sum: the same bits as with the narrow path off."""
    print("two narrow consumers of one linear16 output", flush=True)
    rng = np.random.default_rng(23)
    M, F, H = 513, 72, 200
    dt = BF16
    x = rng.standard_normal((M, F)).astype(np.float32)
    w1 = (rng.standard_normal((F, H)) / np.sqrt(F)).astype(np.float32)
    wa = (rng.standard_normal((H, 10)) / np.sqrt(H)).astype(np.float32)
    wb = (rng.standard_normal((H, 5)) / np.sqrt(H)).astype(np.float32)
    ta = rng.standard_normal((M, 10)).astype(np.float32)
    tb = rng.standard_normal((M, 5)).astype(np.float32)
    got = []
    for narrow in (True, False):
        lib.pg_amd_linear16_narrow(narrow)
        nx, n1w, naw, nbw = (lib.var(v) for v in (x, w1, wa, wb))
        nta, ntb = lib.var(ta, requires_grad=False), lib.var(tb, requires_grad=False)
        h = lib._check(lib.pg_amd_ag_linear16(nx, n1w, None, GELU, dt))
        a = lib._check(lib.pg_amd_ag_linear16(h, naw, None, NONE, dt))
        b = lib._check(lib.pg_amd_ag_linear16(h, nbw, None, NONE, dt))
        la = lib._check(lib.pg_ag_mse(a, nta, True))
        lb = lib._check(lib.pg_ag_mse(b, ntb, True))
        loss = lib._check(lib.op("add", la, lb))
        lib.pg_backward(loss)
        dza = _dec(dt, _kept_dz(lib, a, 10))
        dzb = _dec(dt, _kept_dz(lib, b, 5))
        dh = lib.grad(h)
        check_product(dh, [(dza, _q(oracle, dt, wa).T), (dzb, _q(oracle, dt, wb).T)],
                      f"two narrow consumers: dh, narrow={narrow}", planted=False)
        z1 = lib.read(lib.pg_amd_linear16_preact(h))
        dz1 = _kept_dz(lib, h, H)
        frac = _dz_within_one_ulp(dz1, oracle.cast16(BF16, oracle.gelu_backward(z1, dh)), z1, dh)
        assert frac <= 1e-3, frac
        got.append((dh, dz1))
        for n in (loss, la, lb, a, b, h, nx, n1w, naw, nbw, nta, ntb):
            lib.pg_node_free(n)
    assert np.array_equal(_bits(got[0][0]), _bits(got[1][0]))
    assert np.array_equal(got[0][1], got[1][1])


def test_pending_grad_keeps_the_weights_it_was_formed_with(lib, oracle, keep_dz):
    print("pending narrow grad read after an SGD step and after a second backward", flush=True)
    rng = np.random.default_rng(31)
    M, F, H, N = 600, 48, 160, 10
    dt = BF16
    x = rng.standard_normal((M, F)).astype(np.float32)
    w1 = (rng.standard_normal((F, H)) / np.sqrt(F)).astype(np.float32)
    w2 = (rng.standard_normal((H, N)) / np.sqrt(H)).astype(np.float32)
    g = rng.standard_normal((M, N)).astype(np.float32)
    want = {}
    for narrow in (False, True):
        lib.pg_amd_linear16_narrow(narrow)
        nx, n1w, n2w = lib.var(x), lib.var(w1), lib.var(w2)
        h = lib._check(lib.pg_amd_ag_linear16(nx, n1w, None, GELU, dt))
        out = lib._check(lib.pg_amd_ag_linear16(h, n2w, None, NONE, dt))
        seed = lib.tensor(g)
        lib.pg_amd_backward_from(out, seed)
        if not narrow:
            want["dh"] = lib.grad(h)
            want["dz1"] = _kept_dz(lib, h, H)
        else:
            # the step rewrites W2 and its 16-bit copy before dh is read
            opt = lib.pg_sgd_new(C.byref(SgdCfg(0.5, 0.0, 0.0, 0.0, False)))
            assert lib.pg_sgd_add_param(opt, n2w) == 0
            lib.pg_sgd_step(opt)
            assert not np.array_equal(lib.value(n2w), w2)
            assert np.array_equal(_bits(lib.grad(h)), _bits(want["dh"])), "pending dh read the updated weights"
            assert np.array_equal(_kept_dz(lib, h, H), want["dz1"])
            # a second backward (new weights) replaces it
            lib.pg_amd_backward_from(out, seed)
            dz2 = _dec(dt, _kept_dz(lib, out, N))
            check_product(lib.grad(h), [(dz2, _q(oracle, dt, lib.value(n2w)).T)], "second backward: dh",
                          planted=False)
            lib.pg_sgd_free(opt)
        lib.pg_tensor_free(seed)
        for n in (out, h, nx, n1w, n2w):
            lib.pg_node_free(n)


@pytest.mark.parametrize("M,N,act", [(2730, 20, RELU), (4096, 16, NONE), (1, 3, RELU), (257, 1000, RELU),
                                     (4096, 10, GELU), (3000, 4096, GELU), (1100, 640, RELU), (2050, 200, GELU)])
def test_small_activation_pass(lib, oracle, keep_dz, M, N, act):
    """The activation pass at narrow and ragged widths (ldd 8 to 1000, one
    row up to 4096) and at wide ones whose row blocks take an odd number of
    row pairs (3000 x 4096: 96 rows per block), one pair (1100 x 640), or
    pairs and then single rows beside a partial column block (2050 x 200):
    dz bit for bit (ReLU, none), within one ulp (GELU), db within the
    summation bound."""
    print(f"small activation pass M={M} N={N} act={act}", flush=True)
    rng = np.random.default_rng(M * 7 + N)
    dt = BF16
    K = 24
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    b = (0.1 * rng.standard_normal(N)).astype(np.float32)
    g = rng.standard_normal((M, N)).astype(np.float32)
    nx, nw, nb = lib.var(x), lib.var(w), lib.var(b)
    out = lib._check(lib.pg_amd_ag_linear16(nx, nw, nb, act, dt))
    seed = lib.tensor(g)
    lib.pg_amd_backward_from(out, seed)
    dz = _kept_dz(lib, out, N)
    if act == NONE:
        d = g
        assert np.array_equal(dz, oracle.cast16(dt, d))
    else:
        z = lib.read(lib.pg_amd_linear16_preact(out))
        if act == RELU:
            d = g * (z > 0).astype(np.float32)
            assert np.array_equal(dz, oracle.cast16(dt, d))
        else:
            d = oracle.gelu_backward(z, g)
            assert _dz_within_one_ulp(dz, oracle.cast16(BF16, d), z, g) <= 1e-3
    assert np.all(np.abs(lib.grad(nb) - d.astype(np.float64).sum(axis=0)) <= dbias_bound(d, 128))
    lib.pg_tensor_free(seed)
    for n in (out, nx, nw, nb):
        lib.pg_node_free(n)
