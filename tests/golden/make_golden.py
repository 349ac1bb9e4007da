"""Writes the golden vectors under tests/golden/ from the reference's own
CPU path.

The reference is C11: oracle/ref.mk compiles its CPU sources, where they lie
in the reference checkout, into oracle/_ref/libpicograd_ref.so (and its
header-only converters into oracle/_ref/libref_convert.so).  This script
calls that build through the reference's public C ABI and stores inputs and
outputs as small .npz files (no pickles).  The committed fixtures are data
only; the tests compare the oracle (oracle/liboracle.so) and, on the GPU,
the MI355X library against them.

    python tests/golden/make_golden.py [case ...]   # needs oracle/_ref built

Every case names the reference code it exercises.
"""
from __future__ import annotations

import ctypes as C
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

from oracle_lib import REF_CONVERT_SO, REF_SO  # noqa: E402
from picograd_amd.capi import BF16, F16, F32, AdamCfg, PgLib, SgdCfg, shape_arg  # noqa: E402


def ref_lib() -> PgLib:
    if not REF_SO.exists():
        raise SystemExit(f"{REF_SO} missing: build it with `make -C oracle ref`")
    return PgLib(REF_SO, device=False)


def rng_streams(R: PgLib) -> dict:
    """pg_seed + pg_tensor_uniform/normal (core/tensor.c:289-339)."""
    out = {}
    for seed in (42, 43, 44, 45, 46, 0):
        R.pg_seed(seed)
        nd, sh = shape_arg((1000,))
        t = R.pg_tensor_uniform(nd, sh, -1.0, 1.0)
        out[f"uniform_{seed}"] = R.read(t)
        R.pg_tensor_free(t)
        t = R.pg_tensor_normal(nd, sh, 0.0, 1.0)
        out[f"normal_{seed}"] = R.read(t)
        R.pg_tensor_free(t)
        t = R.pg_tensor_normal(nd, sh, 0.5, 0.02)
        out[f"normal_sd002_{seed}"] = R.read(t)
        R.pg_tensor_free(t)
    return out


def conversions() -> dict:
    """convert.h:15-104 RNE converters: every 16-bit pattern decoded, and a
    set of f32 inputs (specials, halfway cases, subnormals, random bits)
    encoded."""
    L = C.CDLL(str(REF_CONVERT_SO))
    L.ref_f32_to_f16.restype = C.c_uint16
    L.ref_f32_to_f16.argtypes = [C.c_float]
    L.ref_f32_to_bf16.restype = C.c_uint16
    L.ref_f32_to_bf16.argtypes = [C.c_float]
    L.ref_f16_to_f32.restype = C.c_float
    L.ref_f16_to_f32.argtypes = [C.c_uint16]
    L.ref_bf16_to_f32.restype = C.c_float
    L.ref_bf16_to_f32.argtypes = [C.c_uint16]
    rng = np.random.default_rng(2024)
    special = np.array([0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00001,
                        0x7F800001, 0x7FBFFFFF, 0x00000001, 0x007FFFFF, 0x33000000, 0x33000001,
                        0x387FC000, 0x38800000, 0x477FE000, 0x477FF000, 0x477FEFFF, 0x7F7FFFFF,
                        0x3F808000, 0x3F818000, 0x3F808001, 0x3F7FFFFF, 0x3F800000, 0xBF808000,
                        0x33800000, 0x337FFFFF, 0x387FE000, 0x387FF000, 0x38000000, 0x37800000],
                       dtype=np.uint32)
    rand_bits = rng.integers(0, 2**32, size=20000, dtype=np.uint64).astype(np.uint32)
    # values around the f16 range and subnormal boundary, as floats
    rand_vals = np.concatenate([rng.standard_normal(4000), rng.uniform(-70000, 70000, 2000),
                                rng.uniform(-1e-4, 1e-4, 2000), rng.uniform(-7e-8, 7e-8, 1000)])
    enc_in = np.concatenate([special, rand_bits, rand_vals.astype(np.float32).view(np.uint32)])
    f = enc_in.view(np.float32)
    to_f16 = np.array([L.ref_f32_to_f16(float(v)) for v in f], np.uint16)
    to_bf16 = np.array([L.ref_f32_to_bf16(float(v)) for v in f], np.uint16)
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    # ctypes returns Python floats: go through f32 bit patterns explicitly
    f16_dec = np.array([L.ref_f16_to_f32(int(h)) for h in allh], np.float32).view(np.uint32)
    bf16_dec = np.array([L.ref_bf16_to_f32(int(h)) for h in allh], np.float32).view(np.uint32)
    return {"enc_in_bits": enc_in, "to_f16": to_f16, "to_bf16": to_bf16, "f16_dec_bits": f16_dec,
            "bf16_dec_bits": bf16_dec}


def _free(R, *nodes):
    for n in nodes:
        R.pg_node_free(n)


def sgd_trajectories(R: PgLib) -> dict:
    """pg_sgd_step (opt/sgd.c:111-162), three steps per configuration, the
    grads set exactly through loss = sum_all(p * G)."""
    cfgs = [(0.01, 0.9, 0.0, 1e-4, True), (0.1, 0.5, 0.3, 0.01, False), (0.05, 0.0, 0.0, 0.0, False),
            (0.2, 0.7, 0.0, 0.05, True)]
    rng = np.random.default_rng(11)
    out = {"cfgs": np.array([c[:4] + (float(c[4]),) for c in cfgs], np.float32)}
    for ci, (lr, mu, d, wd, nest) in enumerate(cfgs):
        p0 = rng.standard_normal(257).astype(np.float32)
        gs = rng.standard_normal((3, 257)).astype(np.float32)
        p = R.var(p0)
        opt = R.pg_sgd_new(C.byref(SgdCfg(lr, mu, d, wd, nest)))
        R.pg_sgd_add_param(opt, p)
        traj = []
        for s in range(3):
            R.pg_sgd_zero_grad(opt)
            gn = R.var(gs[s], requires_grad=False)
            prod = R.op("mul", p, gn)
            loss = R.op("sum_all", prod)
            R.pg_backward(loss)
            _free(R, loss, prod, gn)
            R.pg_sgd_step(opt)
            traj.append(R.value(p))
        R.pg_sgd_free(opt)
        _free(R, p)
        out[f"p0_{ci}"] = p0
        out[f"g_{ci}"] = gs
        out[f"traj_{ci}"] = np.stack(traj)
    return out


def chain1(R: PgLib) -> dict:
    """Config 1 chain through the reference pg_backward, JIT on and off
    (autograd.c:2483-2533; the fused loop of jit.c:399-583)."""
    out = {}
    R.pg_seed(42)
    nd, sh = shape_arg((64, 64))
    ts = [R.pg_tensor_uniform(nd, sh, -1.0, 1.0) for _ in range(3)]
    a, b, c = (R.read(t) for t in ts)
    for t in ts:
        R.pg_tensor_free(t)
    out.update(a=a, b=b, c=c)
    for jit in (True, False):
        R.pg_autograd_set_jit(jit)
        na, nb, nc = R.var(a), R.var(b), R.var(c)
        t0 = R.op("add", na, nb)
        t1 = R.op("mul", t0, nc)
        t2 = R.op("relu", t1)
        t3 = R.op("tanh", t2)
        loss = R.op("sum_all", t3)
        R.pg_backward(loss)
        tag = "jit" if jit else "eager"
        # last_was_jit is only updated while the JIT is enabled (autograd.c:2499-2519)
        assert not jit or R.pg_autograd_last_was_jit(), R.pg_autograd_last_error()
        out[f"da_{tag}"], out[f"db_{tag}"], out[f"dc_{tag}"] = (R.grad(n) for n in (na, nb, nc))
        out[f"loss_{tag}"] = R.value(loss)
        _free(R, loss, t3, t2, t1, t0, na, nb, nc)
    R.pg_autograd_set_jit(True)
    return out


def chain2(R: PgLib, rows=96, cols=160) -> dict:
    """Config 2 chain at a reduced shape: hybrid JIT (mul, sigmoid) + eager
    GELU' + serial broadcast reduction for dbias (autograd.c:364-387)."""
    out = {}
    R.pg_seed(43)
    nd, sh = shape_arg((rows, cols))
    tx = R.pg_tensor_normal(nd, sh, 0.0, 1.0)
    x = R.read(tx)
    ndb, shb = shape_arg((cols,))
    tb = R.pg_tensor_normal(ndb, shb, 0.0, 0.1)
    bias = R.read(tb)
    tg = R.pg_tensor_normal(nd, sh, 0.0, 1.0)
    g = R.read(tg)
    for t in (tx, tb, tg):
        R.pg_tensor_free(t)
    out.update(x=x, bias=bias, g=g)
    for jit in (True, False):
        R.pg_autograd_set_jit(jit)
        nx, nb, ng = R.var(x), R.var(bias), R.var(g)
        t0 = R.op("add", nx, nb)
        t1 = R.op("gelu", t0)
        t2 = R.op("sigmoid", ng)
        y = R.op("mul", t1, t2)
        loss = R.op("sum_all", y)
        R.pg_backward(loss)
        tag = "jit" if jit else "eager"
        out[f"dx_{tag}"], out[f"dg_{tag}"], out[f"dbias_{tag}"] = (R.grad(n) for n in (nx, ng, nb))
        out[f"loss_{tag}"] = R.value(loss)
        out[f"was_jit_{tag}"] = np.array(bool(R.pg_autograd_last_was_jit()))
        _free(R, loss, y, t2, t1, t0, nx, nb, ng)
    R.pg_autograd_set_jit(True)
    return out


GEMM_SHAPES = [(129, 96, 40), (17, 33, 9), (1, 1, 8), (64, 64, 64), (33, 70, 257)]


def gemms(R: PgLib) -> dict:
    """pg_gemm_ex / pg_hgemm / pg_bgemm (backend.c:150-192 -> gemm.c:575-629):
    C = A.B from 16-bit operands with f32 accumulation, C overwritten."""
    out = {}
    rng = np.random.default_rng(5)
    for dt, name in ((F16, "f16"), (BF16, "bf16")):
        for (m, n, k) in GEMM_SHAPES:
            a = rng.standard_normal((m, k)).astype(np.float32)
            b = rng.standard_normal((k, n)).astype(np.float32)
            if dt == F16:
                a16 = a.astype(np.float16).view(np.uint16)
                b16 = b.astype(np.float16).view(np.uint16)
            else:  # RNE to bf16 on the bits (finite inputs)
                a16 = _bf16(a)
                b16 = _bf16(b)
            c = np.full((m, n), np.nan, np.float32)
            R.pg_gemm_ex(dt, m, n, k, a16.ctypes.data, k, b16.ctypes.data, n, c.ctypes.data, n)
            key = f"{name}_{m}_{n}_{k}"
            out[f"{key}_a"], out[f"{key}_b"], out[f"{key}_c"] = a16, b16, c
    f = rng.standard_normal((7, 5)).astype(np.float32), rng.standard_normal((5, 3)).astype(np.float32)
    c = np.zeros((7, 3), np.float32)
    R.pg_gemm(7, 3, 5, f[0].ctypes.data, 5, f[1].ctypes.data, 3, c.ctypes.data, 3)
    out.update(f32_a=f[0], f32_b=f[1], f32_c=c)
    # which f16 micro the reference picked (gemm.c:277-284): AVX512-FP16
    # hosts run hgemm_avx512fp16_micro, which drops the accumulator of the
    # first 16 columns of each 32-column strip between KC=256 k-blocks
    flags = Path("/proc/cpuinfo").read_text()
    out["host_avx512fp16"] = np.array("avx512_fp16" in flags)
    return out


def _bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


MM_SHAPES = [(65, 40, 33), (8, 16, 24), (130, 72, 20)]


def matmul_backward(R: PgLib) -> dict:
    """bwd_matmul (autograd.c:561-706) with bf16 and f16 leaves: loss =
    sum_all(matmul(A, W) * G) makes dC = G.  G is chosen exactly
    representable in the operand dtype, so rounding dC to the operand dtype
    is the identity and the grads are exact products accumulated in f32."""
    out = {}
    rng = np.random.default_rng(9)
    for dt, name in ((F16, "f16"), (BF16, "bf16")):
        for (M, K, N) in MM_SHAPES:
            a = rng.standard_normal((M, K)).astype(np.float32)
            w = (0.02 * rng.standard_normal((K, N))).astype(np.float32)
            g = rng.standard_normal((M, N)).astype(np.float32)
            if dt == F16:
                a16, w16 = a.astype(np.float16).view(np.uint16), w.astype(np.float16).view(np.uint16)
                g = g.astype(np.float16).astype(np.float32)
            else:
                a16, w16 = _bf16(a), _bf16(w)
                g = (_bf16(g).astype(np.uint32) << 16).view(np.float32)
            R.pg_autograd_set_jit(False)
            na, nw = R.var(a16, dtype=dt), R.var(w16, dtype=dt)
            c = R.op("matmul", na, nw)
            ng = R.var(g, requires_grad=False)
            prod = R.op("mul", c, ng)
            loss = R.op("sum_all", prod)
            R.pg_backward(loss)
            key = f"{name}_{M}_{K}_{N}"
            out[f"{key}_a"], out[f"{key}_w"], out[f"{key}_g"] = a16, w16, g
            out[f"{key}_c"] = R.value(c)
            out[f"{key}_da"], out[f"{key}_dw"] = R.grad(na), R.grad(nw)
            _free(R, loss, prod, ng, c, na, nw)
            R.pg_autograd_set_jit(True)
    # batched f32: bmm-style [B, M, K] . [B, K, N]
    a = rng.standard_normal((3, 9, 7)).astype(np.float32)
    w = rng.standard_normal((3, 7, 5)).astype(np.float32)
    g = rng.standard_normal((3, 9, 5)).astype(np.float32)
    na, nw = R.var(a), R.var(w)
    c = R.op("matmul", na, nw)
    ng = R.var(g, requires_grad=False)
    prod = R.op("mul", c, ng)
    loss = R.op("sum_all", prod)
    R.pg_backward(loss)
    out.update(bmm_a=a, bmm_w=w, bmm_g=g, bmm_c=R.value(c), bmm_da=R.grad(na), bmm_dw=R.grad(nw))
    _free(R, loss, prod, ng, c, na, nw)
    return out


def mse(R: PgLib) -> dict:
    """pg_ag_mse(pred, target, mean) (autograd.c:1758-1771) over a [6, 10]
    prediction: the mean divides by the last axis only (reduce_all,
    autograd.c:1018-1043)."""
    rng = np.random.default_rng(3)
    pred = rng.standard_normal((6, 10)).astype(np.float32)
    tgt = rng.standard_normal((6, 10)).astype(np.float32)
    out = {"pred": pred, "tgt": tgt}
    for mean in (True, False):
        npd, nt = R.var(pred), R.var(tgt, requires_grad=False)
        loss = R.pg_ag_mse(npd, nt, mean)
        R.pg_backward(loss)
        tag = "mean" if mean else "sum"
        out[f"loss_{tag}"] = R.value(loss)
        out[f"dpred_{tag}"] = R.grad(npd)
        _free(R, loss, npd, nt)
    return out


MLP_DIMS = (48, 64, 64, 64, 10)
MLP_BATCH = 32
MLP_SGD = (0.01, 0.9, 0.0, 1e-4, True)


def mlp(R: PgLib) -> dict:
    """Config 5 in f32 at a reduced shape: two training steps of
    linear(nn.c:117-125: matmul then broadcast bias add) + gelu layers, mse
    (mean) loss, pg_backward (JIT on) and a Nesterov pg_sgd_step
    (opt/sgd.c:111-162) with the config-5 hyper-parameters."""
    rng = np.random.default_rng(5)
    dims, B = MLP_DIMS, MLP_BATCH
    out = {"dims": np.array(dims, np.int64)}
    x = rng.standard_normal((B, dims[0])).astype(np.float32)
    t = rng.standard_normal((B, dims[-1])).astype(np.float32)
    out.update(x=x, t=t)
    Ws, bs = [], []
    for i in range(len(dims) - 1):
        lim = 1.0 / np.sqrt(dims[i])
        Ws.append(rng.uniform(-lim, lim, (dims[i], dims[i + 1])).astype(np.float32))
        bs.append((0.1 * rng.standard_normal(dims[i + 1])).astype(np.float32))
        out[f"W{i}_0"], out[f"b{i}_0"] = Ws[-1], bs[-1]
    nW = [R.var(w) for w in Ws]
    nb = [R.var(b) for b in bs]
    opt = R.pg_sgd_new(C.byref(SgdCfg(*MLP_SGD)))
    for w, b in zip(nW, nb):
        R.pg_sgd_add_param(opt, w)
        R.pg_sgd_add_param(opt, b)
    nx, nt = R.var(x, requires_grad=False), R.var(t, requires_grad=False)
    for step in (1, 2):
        R.pg_sgd_zero_grad(opt)
        h, made = nx, []
        for i in range(len(Ws)):
            mm = R.op("matmul", h, nW[i])
            z = R.op("add", mm, nb[i])
            made += [mm, z]
            if i + 1 < len(Ws):
                h = R.op("gelu", z)
                made.append(h)
            else:
                h = z
        loss = R.pg_ag_mse(h, nt, True)
        R.pg_backward(loss)
        out[f"loss_{step}"] = R.value(loss)
        for i in range(len(Ws)):
            out[f"dW{i}_{step}"], out[f"db{i}_{step}"] = R.grad(nW[i]), R.grad(nb[i])
        R.pg_sgd_step(opt)
        for i in range(len(Ws)):
            out[f"W{i}_{step}"], out[f"b{i}_{step}"] = R.value(nW[i]), R.value(nb[i])
        _free(R, loss, *reversed(made))
    R.pg_sgd_free(opt)
    _free(R, nx, nt, *nW, *nb)
    return out


# (lr, beta1, beta2, eps, weight_decay, amsgrad, decoupled_wd), the second
# parameter's (lr, wd) override for pg_adam_add_param_lr, and the step
# counter set before the first step (pg_adam_set_step; 0 = untouched)
ADAM_CFGS = [
    ((1e-3, 0.9, 0.999, 1e-8, 0.0, False, True), (0.0, -1.0), 0),
    ((0.01, 0.9, 0.999, 1e-8, 0.01, False, True), (0.003, 0.0), 0),
    ((0.02, 0.85, 0.99, 1e-6, 0.05, False, False), (0.0, 0.2), 100),
    ((0.005, 0.9, 0.99, 1e-8, 0.01, True, True), (0.02, -1.0), 0),
    ((0.01, 0.5, 0.9, 1e-3, 0.1, True, False), (0.0, -1.0), 0),
]
ADAM_STEPS = 6
ADAM_SKIP = 3  # the step at which the second parameter has no grad


def adam_trajectories(R: PgLib) -> dict:
    """pg_adam_step (opt/adam.c:113-181): two parameters per configuration,
    one registered with per-parameter overrides (adam.c:136-138), six steps
    with grads set exactly through loss = sum_all(p0 * G0) + sum_all(p1 * G1);
    at step ADAM_SKIP the second parameter is left out of the loss, so it has
    no grad and is skipped while the step counter still advances.  Grads mix
    normal values, exact zeros and a few large entries."""
    rng = np.random.default_rng(17)
    out = {"cfgs": np.array([c + o + (s,) for c, o, s in ADAM_CFGS], np.float64)}
    for ci, (cfg, (lr1, wd1), step0) in enumerate(ADAM_CFGS):
        p0 = rng.standard_normal(257).astype(np.float32)
        p1 = rng.standard_normal((5, 7)).astype(np.float32)
        g0 = rng.standard_normal((ADAM_STEPS, 257)).astype(np.float32)
        g1 = rng.standard_normal((ADAM_STEPS, 5, 7)).astype(np.float32)
        g0[:, ::13] = 0.0
        g0[:, 5::37] *= 100.0
        g1[:, 0, :] *= 0.01
        n0, n1 = R.var(p0), R.var(p1)
        opt = R.pg_adam_new(C.byref(AdamCfg(*cfg)))
        R.pg_adam_add_param(opt, n0)
        R.pg_adam_add_param_lr(opt, n1, lr1, wd1)
        if step0:
            R.pg_adam_set_step(opt, step0)
        t0, t1 = [], []
        for s in range(ADAM_STEPS):
            R.pg_adam_zero_grad(opt)
            a = R.var(g0[s], requires_grad=False)
            pa = R.op("mul", n0, a)
            la = R.op("sum_all", pa)
            made = [la, pa, a]
            loss = la
            if s != ADAM_SKIP:
                b = R.var(g1[s], requires_grad=False)
                pb = R.op("mul", n1, b)
                lb = R.op("sum_all", pb)
                loss = R.op("add", la, lb)
                made = [loss, lb, pb, b] + made
            R.pg_backward(loss)
            _free(R, *made)
            R.pg_adam_step(opt)
            t0.append(R.value(n0))
            t1.append(R.value(n1))
        out[f"final_step_{ci}"] = np.array(R.pg_adam_get_step(opt), np.int64)
        R.pg_adam_free(opt)
        _free(R, n0, n1)
        out.update({f"p0_{ci}": p0, f"p1_{ci}": p1, f"g0_{ci}": g0, f"g1_{ci}": g1,
                    f"traj0_{ci}": np.stack(t0), f"traj1_{ci}": np.stack(t1)})
    return out


def _params(nodes):
    return (C.c_void_p * len(nodes))(*[n if n else None for n in nodes])


def clip(R: PgLib) -> dict:
    """pg_grad_norm / pg_clip_grad_norm / pg_clip_grad_value (opt/clip.c):
    three grads (set exactly through sum_all(p * G)), a NULL entry and a node
    without a grad in the list; the norm, clipping below and above the norm,
    the default eps (eps < 0), a grad listed twice, value clipping, and the
    norm of one large grad (f64 accumulation)."""
    rng = np.random.default_rng(23)
    shapes = [(100,), (6, 7), (1,)]
    out = {}

    def setup(gs, scale=1.0):
        ps = [R.var(rng.standard_normal(sh).astype(np.float32)) for sh in shapes]
        terms, made = [], []
        for p, g in zip(ps, gs):
            gn = R.var(g, requires_grad=False)
            pr = R.op("mul", p, gn)
            sm = R.op("sum_all", pr)
            made += [sm, pr, gn]
            terms.append(sm)
        loss = terms[0]
        for t in terms[1:]:
            loss = R.op("add", loss, t)
            made.insert(0, loss)
        R.pg_backward(loss)
        _free(R, *made)
        return ps

    for case in range(5):
        gs = [(rng.standard_normal(sh) * (1 + 3 * case)).astype(np.float32) for sh in shapes]
        for i, g in enumerate(gs):
            out[f"g{i}_{case}"] = g
        ps = setup(gs)
        nograd = R.var(np.ones(3, np.float32))
        lst = [ps[0], None, ps[1], nograd, ps[2]]
        if case == 0:
            out["norm_0"] = np.float32(R.pg_grad_norm(_params(lst), len(lst)))
        elif case == 1:  # clip below the norm
            n = R.pg_grad_norm(_params(lst), len(lst))
            out["max_norm_1"] = np.float32(0.5 * n)
            out["ret_1"] = np.float32(R.pg_clip_grad_norm(_params(lst), len(lst), out["max_norm_1"], 1e-6))
        elif case == 2:  # above the norm: untouched; then default eps
            n = R.pg_grad_norm(_params(lst), len(lst))
            out["max_norm_2a"] = np.float32(2.0 * n)
            out["ret_2a"] = np.float32(R.pg_clip_grad_norm(_params(lst), len(lst), out["max_norm_2a"], 1e-6))
            out["max_norm_2b"] = np.float32(0.25 * n)
            out["ret_2b"] = np.float32(R.pg_clip_grad_norm(_params(lst), len(lst), out["max_norm_2b"], -1.0))
        elif case == 3:  # a grad listed twice
            lst = [ps[0], ps[0], ps[1]]
            out["max_norm_3"] = np.float32(1.0)
            out["ret_3"] = np.float32(R.pg_clip_grad_norm(_params(lst), len(lst), 1.0, 1e-6))
        else:  # value clipping
            out["clip_value_4"] = np.float32(2.5)
            R.pg_clip_grad_value(_params(lst), len(lst), 2.5)
        for i, p in enumerate(ps):
            out[f"after{i}_{case}"] = R.grad(p)
        _free(R, nograd, *ps)
    big = (10.0 * rng.standard_normal(30011)).astype(np.float32)
    out["big_g"] = big
    (pb,) = [R.var(np.zeros_like(big))]
    gn = R.var(big, requires_grad=False)
    pr = R.op("mul", pb, gn)
    sm = R.op("sum_all", pr)
    R.pg_backward(sm)
    out["big_norm"] = np.float32(R.pg_grad_norm(_params([pb]), 1))
    _free(R, sm, pr, gn, pb)
    return out


def _pgt1_header(dtype, shape, numel=None, elem=None, magic=b"PGT1", ver=1, ndim=None):
    import struct
    nd = len(shape) if ndim is None else ndim
    h = magic + struct.pack("<III", ver, dtype, nd) + b"".join(struct.pack("<Q", d) for d in shape)
    n = int(np.prod(shape)) if numel is None else numel
    es = (4 if dtype == F32 else 2) if elem is None else elem
    return h + struct.pack("<QQ", n, es)


# crafted PGT1 byte strings and whether the reference's pg_tensor_load takes
# them (tensor.c:655-702); the data after each header is zeros
CKPT_CRAFTED = [
    ("ok_f32", _pgt1_header(F32, (2, 3)) + bytes(24)),
    ("ok_bf16", _pgt1_header(BF16, (5,)) + bytes(10)),
    ("bad_magic", _pgt1_header(F32, (2,), magic=b"PGT2") + bytes(8)),
    ("bad_version", _pgt1_header(F32, (2,), ver=2) + bytes(8)),
    ("bad_dtype", _pgt1_header(3, (2,), elem=4) + bytes(8)),
    ("ndim_zero", _pgt1_header(F32, (), ndim=0) + bytes(4)),
    ("ndim_nine", _pgt1_header(F32, (1,) * 9) + bytes(4)),
    ("dim_zero", _pgt1_header(F32, (3, 0), numel=0) + bytes(0)),
    ("dim_too_big", _pgt1_header(F32, (10000001,)) + bytes(16)),
    ("dim_at_bound", _pgt1_header(F16, (10000000,)) + bytes(20000000)),
    ("numel_mismatch", _pgt1_header(F32, (2, 3), numel=5) + bytes(24)),
    ("elem_mismatch", _pgt1_header(F32, (2, 3), elem=2) + bytes(24)),
    ("truncated_data", _pgt1_header(F32, (2, 3)) + bytes(20)),
    ("truncated_header", _pgt1_header(F32, (2, 3))[:20]),
]


def checkpoint_files(R: PgLib) -> dict:
    """pg_tensor_save / pg_tensor_load (core/tensor.c:604-711) and
    pg_module_save (nn/module.c:91-104): the bytes the reference writes for
    f32, f16 and bf16 tensors of several ranks and for a three-parameter
    module, and its loader's verdict on crafted headers."""
    import os
    import tempfile
    rng = np.random.default_rng(31)
    out = {}
    arrays = {
        "t0": (F32, rng.standard_normal((3, 5)).astype(np.float32)),
        "t1": (F16, rng.standard_normal((2, 3, 4)).astype(np.float16).view(np.uint16)),
        "t2": (BF16, (rng.standard_normal(7).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)),
        "t3": (F32, np.array([42.5], np.float32)),
        "t4": (F32, rng.standard_normal((2, 1, 3, 1, 2, 1, 1, 2)).astype(np.float32)),
    }
    with tempfile.TemporaryDirectory() as d:
        for name, (dt, arr) in arrays.items():
            t = R.tensor(arr, dt)
            path = os.path.join(d, name + ".pgt")
            assert R.lib.pg_tensor_save(C.c_void_p(t), path.encode())
            R.pg_tensor_free(t)
            out[f"{name}_dtype"] = np.array(dt, np.int64)
            out[f"{name}_data"] = arr
            out[f"{name}_bytes"] = np.frombuffer(open(path, "rb").read(), np.uint8)
        L = R.lib
        L.pg_module_new.restype = C.c_void_p
        L.pg_module_register.argtypes = [C.c_void_p, C.c_void_p]
        L.pg_module_save.argtypes = [C.c_void_p, C.c_char_p]
        L.pg_module_free.argtypes = [C.c_void_p]
        L.pg_tensor_load.restype = C.c_void_p
        L.pg_tensor_load.argtypes = [C.c_char_p]
        m = L.pg_module_new()
        nodes = [R.var(rng.standard_normal(sh).astype(np.float32)) for sh in ((4, 6), (6,), (6, 2))]
        for i, n in enumerate(nodes):
            L.pg_module_register(C.c_void_p(m), C.c_void_p(n))
            out[f"mod_p{i}"] = R.value(n)
        path = os.path.join(d, "mod.pgmd")
        assert L.pg_module_save(C.c_void_p(m), path.encode())
        out["mod_bytes"] = np.frombuffer(open(path, "rb").read(), np.uint8)
        L.pg_module_free(C.c_void_p(m))
        _free(R, *nodes)
        names, verdicts = [], []
        for i, (name, blob) in enumerate(CKPT_CRAFTED):
            out[f"crafted_{i}"] = np.frombuffer(blob, np.uint8)
            path = os.path.join(d, name + ".pgt")
            open(path, "wb").write(blob)
            t = L.pg_tensor_load(path.encode())
            verdicts.append(bool(t))
            if t:
                R.pg_tensor_free(t)
            names.append(name)
        out["crafted_names"] = np.array(names)
        out["crafted_loads"] = np.array(verdicts)
    return out


# pg_jit op codes (jit.h)
JADD, JSUB, JMUL, JDIV, JNEG, JEXP, JLOG, JSQRT, JSIN, JCOS, JABS, JRELU, JSIGMOID, JTANH, JGELU, JERF, JSTEP = range(17)


def _jit_specs():
    """Forward graphs of the reference's test_jit.c and jit_demo.c, with
    the inputs fed to them: nodes are ["in", shape], ["const", value] or
    ["op", code, [ids]]; ids count every node in order."""
    rng = np.random.default_rng(41)
    u = lambda shape, lo, hi: rng.uniform(lo, hi, shape).astype(np.float32)
    specs = []
    chain = [["in", [64, 64]], ["in", [64, 64]], ["in", [64, 64]], ["op", JADD, [0, 1]], ["op", JMUL, [3, 2]],
             ["op", JRELU, [4]], ["op", JTANH, [5]]]
    specs.append(("basic", [["in", [2, 3]]] * 3 + [["op", JADD, [0, 1]], ["op", JMUL, [3, 2]], ["op", JRELU, [4]]],
                  [5], [np.array([[1, -2, 3], [4, -5, 6]], np.float32), np.array([[6, 5, 4], [3, 2, 1]], np.float32),
                        np.ones((2, 3), np.float32)]))
    specs.append(("bcast", [["in", [2, 4]], ["in", [4]], ["op", JADD, [0, 1]], ["op", JRELU, [2]]], [3],
                  [np.array([[-1, 2, -3, 4], [-5, 6, -7, 8]], np.float32), np.array([10, 20, 30, 40], np.float32)]))
    specs.append(("bcast3d", [["in", [2, 3, 4]], ["in", [3, 4]], ["in", [4]], ["op", JADD, [0, 1]], ["op", JMUL, [3, 2]]],
                  [4], [u((2, 3, 4), -2, 2), u((3, 4), -2, 2), u((4,), -2, 2)]))
    for code, name in ((JNEG, "neg"), (JEXP, "exp"), (JLOG, "log"), (JSQRT, "sqrt"), (JSIN, "sin"), (JCOS, "cos"),
                       (JABS, "abs"), (JRELU, "relu"), (JSIGMOID, "sigmoid"), (JTANH, "tanh"), (JGELU, "gelu"),
                       (JERF, "erf"), (JSTEP, "step")):
        lo, hi = (0.5, 2.0) if code in (JLOG, JSQRT) else (-4.0, 4.0)
        x = u((1031,), lo, hi)
        if code not in (JLOG, JSQRT):
            x[:8] = [0.0, -0.0, 1e-3, -1e-3, 3.9, -3.9, 1e-30, 9.5]
        specs.append((f"unary_{name}", [["in", [1031]], ["op", code, [0]]], [1], [x]))
    for code, name in ((JADD, "add"), (JSUB, "sub"), (JMUL, "mul"), (JDIV, "div")):
        specs.append((f"binary_{name}", [["in", [19, 53]], ["in", [19, 53]], ["op", code, [0, 1]]], [2],
                      [u((19, 53), -2, 2), u((19, 53), 0.5, 2)]))
    specs.append(("const", [["in", [2, 4]], ["const", 2.5], ["op", JMUL, [0, 1]], ["op", JRELU, [2]]], [3],
                  [u((2, 4), -2, 2)]))
    specs.append(("complex", [["in", [4, 8]], ["in", [8]], ["in", [4, 8]], ["const", 0.5], ["op", JADD, [0, 1]],
                              ["op", JMUL, [4, 2]], ["op", JADD, [5, 3]], ["op", JTANH, [6]]], [7],
                  [u((4, 8), -1, 1), u((8,), -0.5, 0.5), u((4, 8), -1, 1)]))
    specs.append(("multi", [["in", [4]], ["in", [4]], ["op", JADD, [0, 1]], ["op", JMUL, [0, 1]]], [2, 3],
                  [np.array([1, 2, 3, 4], np.float32), np.array([5, 6, 7, 8], np.float32)]))
    specs.append(("demo64", chain, [6], [u((64, 64), -1, 1) for _ in range(3)]))
    specs.append(("gelu_rowbias", [["in", [96, 160]], ["in", [160]], ["in", [96, 160]], ["op", JADD, [0, 1]],
                                   ["op", JGELU, [3]], ["op", JSIGMOID, [2]], ["op", JMUL, [4, 5]]], [6],
                  [rng.standard_normal((96, 160)).astype(np.float32),
                   (0.1 * rng.standard_normal(160)).astype(np.float32),
                   rng.standard_normal((96, 160)).astype(np.float32)]))
    return specs


def jit_forward(R: PgLib) -> dict:
    """Forward graphs through the reference's JIT (jit.c:644-806; it
    compiles each with the system C compiler): test_jit.c's graphs (basic
    fusion, 2-D and 3-D broadcast, every unary and binary op, a constant,
    a complex fused chain, two outputs) on larger inputs, and jit_demo.c's
    (a+b)*c -> relu -> tanh at [64,64]."""
    import json
    out, meta = {}, []
    for name, nodes, outs, inputs in _jit_specs():
        g = R.pg_jit_graph_new()
        for nd in nodes:
            if nd[0] == "in":
                k, sh = shape_arg(nd[1])
                assert R.pg_jit_add_input(g, k, sh) >= 0
            elif nd[0] == "const":
                assert R.pg_jit_add_const(g, nd[1]) >= 0
            else:
                ids = (C.c_int * len(nd[2]))(*nd[2])
                assert R.pg_jit_add_op(g, nd[1], ids, len(nd[2])) >= 0
        for o in outs:
            R.pg_jit_mark_output(g, o)
        exe = R.pg_jit_compile(g)
        assert exe, R.pg_jit_last_error()
        ts = [R.tensor(x) for x in inputs]
        outs_t = []
        shapes = _jit_out_shapes(nodes)
        for o in outs:
            k, sh = shape_arg(shapes[o])
            outs_t.append(R.pg_tensor_zeros(k, sh))
        assert R.pg_jit_run(exe, (C.c_void_p * len(ts))(*ts), len(ts), (C.c_void_p * len(outs_t))(*outs_t),
                            len(outs_t))
        for i, x in enumerate(inputs):
            out[f"{name}_in{i}"] = x
        for i, t in enumerate(outs_t):
            out[f"{name}_out{i}"] = R.read(t)
        for t in ts + outs_t:
            R.pg_tensor_free(t)
        R.pg_jit_exe_free(exe)
        R.pg_jit_graph_free(g)
        meta.append({"name": name, "nodes": nodes, "outputs": outs, "ninputs": len(inputs)})
    out["specs"] = np.array(json.dumps(meta))
    return out


def _jit_out_shapes(nodes):
    """NumPy broadcast shape of every node (consts are scalars)."""
    shapes = []
    for nd in nodes:
        if nd[0] == "in":
            shapes.append(tuple(nd[1]))
        elif nd[0] == "const":
            shapes.append(())
        else:
            shapes.append(tuple(np.broadcast_shapes(*[shapes[i] for i in nd[2]])))
    return shapes


CASES = {
    "rng": rng_streams,
    "convert": lambda R: conversions(),
    "sgd": sgd_trajectories,
    "chain1": chain1,
    "chain2": chain2,
    "gemm": gemms,
    "matmul_bwd": matmul_backward,
    "mse": mse,
    "mlp": mlp,
    "adam": adam_trajectories,
    "clip": clip,
    "ckpt": checkpoint_files,
    "jit_fwd": jit_forward,
}


def main(argv: list[str]) -> int:
    """Writes every case, or only the ones named on the command line."""
    R = ref_lib()
    names = argv or list(CASES)
    for name in names:
        arrays = CASES[name](R)
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **arrays)
        print(f"wrote {path.relative_to(ROOT)} ({path.stat().st_size} bytes)")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
