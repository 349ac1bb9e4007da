"""Adam / AdamW and gradient clipping on the MI355X, through the C ABI.

The device kernels evaluate adam.c and clip.c in the order the reference's
-ffast-math build does, with IEEE sqrt and division, exactly as the oracle
(oracle/oracle.c) restates them: against the oracle the weights, moments and
clipped grads must agree bit for bit.  Against the reference's own golden
trajectories (tests/golden/adam.npz, clip.npz) the bar is the oracle's:
bit for bit where the reference computes with IEEE arithmetic, within one
ulp plus 2^-21 of the update where its 8-wide loop uses reciprocal
estimates.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from picograd_amd.capi import BF16, AdamCfg

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
ADAM_SKIP = 3


def golden(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bits(x) -> np.ndarray:
    return np.asarray(x, np.float32).view(np.uint32)


def set_grad(lib, n: int, arr: np.ndarray) -> None:
    """node->grad = a device tensor holding arr (as test_training.c:256-257
    assigns grads); the node owns it from here."""
    node = lib.node(n)
    if node.grad:
        lib.pg_tensor_free(node.grad)
    node.grad = lib.tensor(np.ascontiguousarray(arr, np.float32))


def params_arg(nodes):
    return (C.c_void_p * len(nodes))(*[n if n else None for n in nodes])


class OracleAdam:
    """The oracle driven like pg_adam: per-parameter overrides
    (adam.c:136-138), lazily zeroed moments, a step counter."""

    def __init__(self, oracle, cfg, overrides, ps):
        self.o, self.cfg = oracle, cfg
        lr, _, _, _, wd, ams, _ = cfg
        self.lr = [o[0] if o[0] > 0 else lr for o in overrides]
        self.wd = [o[1] if o[1] >= 0 else wd for o in overrides]
        self.p = [np.ascontiguousarray(p, np.float32).reshape(-1).copy() for p in ps]
        self.mom = [[np.zeros(p.size, np.float32) for _ in range(3)] for p in self.p]
        self.step = 0

    def run(self, grads):
        lr, b1, b2, eps, wd, ams, dec = self.cfg
        self.step += 1
        for k, g in enumerate(grads):
            if g is None:
                continue
            m, v, vm = self.mom[k]
            self.o.adam_step(self.p[k], np.ascontiguousarray(g, np.float32).reshape(-1), m, v,
                             vm if ams else None, self.lr[k], b1, b2, eps, self.wd[k], ams, dec, self.step)


def make_adam(lib, cfg, nodes, overrides, step0=0):
    opt = lib.pg_adam_new(C.byref(AdamCfg(*cfg)))
    assert opt
    for n, (lr, wd) in zip(nodes, overrides):
        assert lib.pg_adam_add_param_lr(opt, n, lr, wd) == 0
    if step0:
        lib.pg_adam_set_step(opt, step0)
    return opt


@pytest.mark.parametrize("ci", range(5))
def test_adam_matches_reference_and_oracle(lib, oracle, ci):
    """The golden configurations (L2, AdamW, amsgrad, per-parameter
    overrides, a parameter without a grad, a counter set by
    pg_adam_set_step): six device steps equal the oracle's bit for bit and
    stay in the oracle's band around the reference's weights."""
    g = golden("adam")
    lr, b1, b2, eps, wd, ams, dec, lr1, wd1, step0 = (float(x) for x in g["cfgs"][ci])
    cfg = (lr, b1, b2, eps, wd, bool(ams), bool(dec))
    ps = [g[f"p0_{ci}"], g[f"p1_{ci}"]]
    nodes = [lib.var(p) for p in ps]
    opt = make_adam(lib, cfg, nodes, [(0.0, -1.0), (lr1, wd1)], int(step0))
    ref = OracleAdam(oracle, cfg, [(0.0, -1.0), (lr1, wd1)], ps)
    ref.step = int(step0)
    try:
        for s in range(6):
            lib.pg_adam_zero_grad(opt)
            grads = [g[f"g0_{ci}"][s], None if s == ADAM_SKIP else g[f"g1_{ci}"][s]]
            for n, gr in zip(nodes, grads):
                if gr is not None:
                    set_grad(lib, n, gr)
            lib.pg_adam_step(opt)
            ref.run(grads)
            for k in range(2):
                dev = lib.value(nodes[k]).reshape(-1)
                assert np.array_equal(bits(dev), bits(ref.p[k])), (s, k)
                gold = g[f"traj{k}_{ci}"][s].reshape(-1)
                assert np.all(np.abs(dev - gold) <= 2.0 ** -22 * np.maximum(1.0, np.abs(gold))), (s, k)
                t = gold.size - gold.size % 8  # the reference's IEEE remainder loop
                assert np.array_equal(bits(dev[t:]), bits(gold[t:])), (s, k)
        assert lib.pg_adam_get_step(opt) == int(g[f"final_step_{ci}"])
    finally:
        lib.pg_adam_free(opt)
        for n in nodes:
            lib.pg_node_free(n)


SIZES = [1, 3, 5, 8, 31, 2047, 2048, 2049, 4099, 8191, 65536 + 5, 300001]


@pytest.mark.parametrize("ams,dec,wd", [(False, True, 0.01), (True, False, 0.05), (True, True, 0.0)])
def test_adam_many_tensors_bit_exact(lib, oracle, ams, dec, wd):
    """40 tensors of ragged sizes (two launches of the 32-tensor table,
    chunk edges, 1-3 element tails), per-parameter overrides, grads missing
    in some steps: weights equal the oracle's bit for bit."""
    rng = np.random.default_rng(int(ams) * 2 + int(dec))
    sizes = [SIZES[i % len(SIZES)] for i in range(40)]
    ps = [rng.standard_normal(n).astype(np.float32) for n in sizes]
    overrides = [((0.003 if i % 3 == 0 else 0.0), (0.2 if i % 4 == 1 else -1.0)) for i in range(40)]
    cfg = (0.01, 0.9, 0.999, 1e-8, wd, ams, dec)
    nodes = [lib.var(p) for p in ps]
    opt = make_adam(lib, cfg, nodes, overrides)
    ref = OracleAdam(oracle, cfg, overrides, ps)
    try:
        for s in range(3):
            lib.pg_adam_zero_grad(opt)
            grads = []
            for i, n in enumerate(nodes):
                if (i + s) % 7 == 3:
                    grads.append(None)
                    continue
                gr = (rng.standard_normal(sizes[i]) * (1 + 10 * (i % 2))).astype(np.float32)
                gr[::17] = 0.0
                set_grad(lib, n, gr)
                grads.append(gr)
            lib.pg_adam_step(opt)
            ref.run(grads)
        for i, n in enumerate(nodes):
            assert np.array_equal(bits(lib.value(n)), bits(ref.p[i])), (i, sizes[i])
    finally:
        lib.pg_adam_free(opt)
        for n in nodes:
            lib.pg_node_free(n)


def test_adam_rewrites_the_16bit_copy(lib):
    """A weight used by matmul16 keeps a bf16 copy; pg_adam_step rewrites
    it in its update pass, so the next product uses the updated weight."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((64, 96)).astype(np.float32)
    w = rng.standard_normal((96, 128)).astype(np.float32)
    nx, nw = lib.var(x, requires_grad=False), lib.var(w)
    y0 = lib.pg_amd_ag_matmul16(nx, nw, BF16)  # makes the copy
    lib.pg_node_free(y0)
    opt = make_adam(lib, (0.05, 0.9, 0.999, 1e-8, 0.0, False, True), [nw], [(0.0, -1.0)])
    try:
        set_grad(lib, nw, rng.standard_normal(w.shape).astype(np.float32))
        lib.pg_adam_step(opt)
        y1 = lib.pg_amd_ag_matmul16(nx, nw, BF16)
        fresh = lib.var(lib.value(nw))
        y2 = lib.pg_amd_ag_matmul16(nx, fresh, BF16)
        assert not np.array_equal(lib.value(nw), w)
        assert np.array_equal(lib.value(y1), lib.value(y2))
        lib.pg_node_free(y1)
        lib.pg_node_free(y2)
        lib.pg_node_free(fresh)
    finally:
        lib.pg_adam_free(opt)
        lib.pg_node_free(nx)
        lib.pg_node_free(nw)


def test_adam_api_and_reference_known_answer(lib):
    """adam.c:27-111: defaults, lr get/set, counts, the step counter,
    zero_grad freeing grads; test_training.c:237-268: with grads of 1, a
    parameter given lr 0.01 moves less than one at the optimiser's 0.1."""
    d = lib.pg_adam_cfg_default()
    assert (round(d.lr, 6), round(d.beta1, 6), round(d.beta2, 6), d.amsgrad, d.decoupled_wd) == \
        (0.001, 0.9, 0.999, False, True)
    cfg = lib.pg_adam_cfg_default()
    cfg.lr = 0.1
    opt = lib.pg_adam_new(C.byref(cfg))
    x = lib.var(np.ones(1, np.float32))
    y = lib.var(np.ones(1, np.float32))
    try:
        assert lib.pg_adam_add_param(opt, x) == 0 and lib.pg_adam_add_param(opt, y) == 0
        assert lib.pg_adam_num_params(opt) == 2
        lib.pg_adam_set_param_lr(opt, 0, 0.01)
        assert abs(lib.pg_adam_get_lr(opt) - 0.1) < 1e-7
        set_grad(lib, x, np.ones(1, np.float32))
        set_grad(lib, y, np.ones(1, np.float32))
        lib.pg_adam_step(opt)
        dx = 1.0 - float(lib.value(x)[0])
        dy = 1.0 - float(lib.value(y)[0])
        assert dy > dx and abs(dx - 0.01) < 1e-6 and abs(dy - 0.1) < 1e-6
        assert lib.pg_adam_get_step(opt) == 1
        lib.pg_adam_zero_grad(opt)
        assert not lib.node(x).grad and not lib.node(y).grad
        lib.pg_adam_step(opt)  # no grads: nothing moves, the counter still advances
        assert lib.pg_adam_get_step(opt) == 2 and float(lib.value(x)[0]) == 1.0 - dx
        lib.pg_adam_set_step(opt, 41)
        assert lib.pg_adam_get_step(opt) == 41
        lib.pg_adam_set_lr(opt, 0.5)
        assert lib.pg_adam_get_lr(opt) == 0.5
    finally:
        lib.pg_adam_free(opt)
        lib.pg_node_free(x)
        lib.pg_node_free(y)


# ---------------------------------------------------------------- clipping

def _clip_case(lib, g, case):
    shapes = [(100,), (6, 7), (1,)]
    nodes = [lib.var(np.zeros(sh, np.float32)) for sh in shapes]
    for i, n in enumerate(nodes):
        set_grad(lib, n, g[f"g{i}_{case}"])
    nograd = lib.var(np.ones(3, np.float32))
    return nodes, nograd


def test_clip_matches_reference(lib):
    """The golden clip cases through pg_grad_norm / pg_clip_grad_norm /
    pg_clip_grad_value on device grads: norms and clipped grads bit for bit,
    with NULL entries and grad-less nodes skipped, no change within
    max_norm, eps < 0 as 1e-6, a grad listed twice scaled twice."""
    g = golden("clip")
    for case in range(5):
        nodes, nograd = _clip_case(lib, g, case)
        lst = [nodes[0], None, nodes[1], nograd, nodes[2]]
        pa = params_arg(lst)
        if case == 0:
            assert bits(lib.pg_grad_norm(pa, len(lst))) == bits(g["norm_0"])
        elif case == 1:
            assert bits(lib.pg_clip_grad_norm(pa, len(lst), float(g["max_norm_1"]), 1e-6)) == bits(g["ret_1"])
        elif case == 2:
            assert bits(lib.pg_clip_grad_norm(pa, len(lst), float(g["max_norm_2a"]), 1e-6)) == bits(g["ret_2a"])
            assert bits(lib.pg_clip_grad_norm(pa, len(lst), float(g["max_norm_2b"]), -1.0)) == bits(g["ret_2b"])
        elif case == 3:
            dup = [nodes[0], nodes[0], nodes[1]]
            assert bits(lib.pg_clip_grad_norm(params_arg(dup), 3, 1.0, 1e-6)) == bits(g["ret_3"])
        else:
            lib.pg_clip_grad_value(pa, len(lst), float(g["clip_value_4"]))
        for i, n in enumerate(nodes):
            assert np.array_equal(bits(lib.grad(n)), bits(g[f"after{i}_{case}"])), (case, i)
        assert not lib.node(nograd).grad
        for n in nodes + [nograd]:
            lib.pg_node_free(n)
    big = lib.var(np.zeros(g["big_g"].size, np.float32))
    set_grad(lib, big, g["big_g"])
    assert bits(lib.pg_grad_norm(params_arg([big]), 1)) == bits(g["big_norm"])
    assert lib.pg_clip_grad_norm(params_arg([big]), 1, 0.0, 1e-6) == -1.0
    assert lib.pg_grad_norm(None, 0) == 0.0
    lib.pg_node_free(big)


def test_clip_many_grads_and_large_norm(lib, oracle):
    """70 grads (two launches of the 64-tensor table, ragged sizes) clipped
    by norm then by value: equal to the oracle bit for bit; the norm of a
    40M-element grad within one f32 ulp of numpy's f64 sum, the same bits on
    a second call."""
    rng = np.random.default_rng(9)
    sizes = [SIZES[i % len(SIZES)] for i in range(70)]
    gs = [(rng.standard_normal(n) * 3).astype(np.float32) for n in sizes]
    nodes = [lib.var(np.zeros(n, np.float32)) for n in sizes]
    for n, gr in zip(nodes, gs):
        set_grad(lib, n, gr)
    ref = [x.copy() for x in gs]
    want = oracle.clip_grad_norm(ref, 7.0, 1e-6)
    got = lib.pg_clip_grad_norm(params_arg(nodes), len(nodes), 7.0, 1e-6)
    assert abs(got - want) <= np.spacing(np.float32(want))
    if bits(got) == bits(want):
        for i, n in enumerate(nodes):
            assert np.array_equal(bits(lib.grad(n)), bits(ref[i])), i
    oracle.clip_grad_value(ref, 0.01)
    lib.pg_clip_grad_value(params_arg(nodes), len(nodes), 0.01)
    for i, n in enumerate(nodes):
        dev = lib.grad(n)
        assert np.all(np.abs(dev) <= np.float32(0.01)), i
        if bits(got) == bits(want):
            assert np.array_equal(bits(dev), bits(ref[i])), i
    for n in nodes:
        lib.pg_node_free(n)
    big = (rng.standard_normal(40_000_003) * 2).astype(np.float32)
    nb = lib.var(np.zeros(big.size, np.float32))
    set_grad(lib, nb, big)
    n1 = lib.pg_grad_norm(params_arg([nb]), 1)
    n2 = lib.pg_grad_norm(params_arg([nb]), 1)
    exact = float(np.sqrt(np.dot(big.astype(np.float64), big.astype(np.float64))))
    assert bits(n1) == bits(n2)
    assert abs(n1 - exact) <= np.spacing(np.float32(exact))
    lib.pg_node_free(nb)


@pytest.mark.parametrize("opt_kind", ["adamw", "sgd"])
def test_clip_scale_applied_by_the_step(lib, oracle, opt_kind):
    """pg_clip_grad_norm leaves its scale pending on the grads' storage and
    the optimiser applies it as it reads them: clip then step equals the
    oracle's clip (grads scaled in place) then step, bit for bit, with no
    read of the grads in between; a second step with the same grads scales
    them again as the reference's still-scaled grads would; reading the
    grads, a second clip, or a backward writing them sees the scaled values
    (or none, when they are overwritten).  Ragged sizes over two launches of
    the 32-tensor table."""
    rng = np.random.default_rng(31 + (opt_kind == "sgd"))
    sizes = [SIZES[i % len(SIZES)] for i in range(36)]
    ps = [rng.standard_normal(n).astype(np.float32) for n in sizes]
    gs = [(rng.standard_normal(n) * 2).astype(np.float32) for n in sizes]
    nodes = [lib.var(p) for p in ps]
    for n, g in zip(nodes, gs):
        set_grad(lib, n, g)
    pa = params_arg(nodes)
    ref_g = [g.copy() for g in gs]
    want_norm = oracle.clip_grad_norm(ref_g, 5.0, 1e-6)
    if opt_kind == "adamw":
        cfg = (1e-3, 0.9, 0.999, 1e-8, 0.01, False, True)
        opt = make_adam(lib, cfg, nodes, [(0.0, -1.0)] * len(nodes))
        ref = OracleAdam(oracle, cfg, [(0.0, -1.0)] * len(nodes), ps)
        step, free = lib.pg_adam_step, lib.pg_adam_free
        ref_params = lambda: ref.p  # noqa: E731
    else:
        from picograd_amd.capi import SgdCfg
        opt = lib.pg_sgd_new(C.byref(SgdCfg(0.01, 0.9, 0.0, 1e-4, True)))
        for n in nodes:
            assert lib.pg_sgd_add_param(opt, n) == 0
        rp = [p.copy() for p in ps]
        rb = [np.zeros_like(p) for p in ps]

        class _R:
            def run(self, grads):
                for k, g in enumerate(grads):
                    oracle.sgd_step(rp[k], g, rb[k], 0.01, 0.9, 0.0, 1e-4, True)
        ref = _R()
        step, free = lib.pg_sgd_step, lib.pg_sgd_free
        ref_params = lambda: rp  # noqa: E731
    try:
        got_norm = lib.pg_clip_grad_norm(pa, len(nodes), 5.0, 1e-6)
        assert bits(got_norm) == bits(want_norm)
        for s in range(2):  # the same (clipped) grads twice
            step(opt)
            ref.run(ref_g)
            for k, n in enumerate(nodes):
                assert np.array_equal(bits(lib.value(n)).reshape(-1), bits(ref_params()[k]).reshape(-1)), (s, k)
        # a reader sees the scaled grads
        for k, n in enumerate(nodes):
            assert np.array_equal(bits(lib.grad(n)), bits(ref_g[k])), k
        # a second clip reads the scaled values
        want2 = oracle.clip_grad_norm(ref_g, 1.0, 1e-6)
        assert bits(lib.pg_clip_grad_norm(pa, len(nodes), 1.0, 1e-6)) == bits(want2)
        step(opt)
        ref.run(ref_g)
        for k, n in enumerate(nodes):
            assert np.array_equal(bits(lib.value(n)).reshape(-1), bits(ref_params()[k]).reshape(-1)), k
        for k, n in enumerate(nodes):
            assert np.array_equal(bits(lib.grad(n)), bits(ref_g[k])), k
    finally:
        free(opt)
        for n in nodes:
            lib.pg_node_free(n)


def test_clip_scale_pending_then_backward_overwrites(lib, oracle):
    """A grad clipped (scale pending) and then written by a backward: the
    backward's grads replace the values (the pending scale is dropped, not
    applied to the new grads), as the reference's zeroing of grads at the
    start of pg_backward (autograd.c:2490-2492) does."""
    x = np.linspace(-2, 2, 4096, dtype=np.float32).reshape(64, 64)
    nx = lib.var(x)
    set_grad(lib, nx, np.full((64, 64), 100.0, np.float32))
    assert lib.pg_clip_grad_norm(params_arg([nx]), 1, 1.0, 1e-6) > 1.0
    y = lib.op("tanh", nx)
    loss = lib.op("sum_all", y)
    lib.pg_backward(loss)
    want = 1.0 - np.tanh(x.astype(np.float64)) ** 2
    assert np.max(np.abs(lib.grad(nx) - want)) <= 1e-6
    for n in (loss, y, nx):
        lib.pg_node_free(n)
