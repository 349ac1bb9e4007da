"""The CPU oracle pinned against the reference's own outputs (CPU only).

tests/golden/*.npz were written by tests/golden/make_golden.py from the
reference's CPU path compiled from its sources (oracle/_ref).  Each test
below checks one oracle function against those vectors, against the
reference's known answers, or against what the mathematics fixes, and
some plant a plausible mistake in a copy of the oracle's arithmetic to show
the check would catch it.
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest

from oracle_lib import bf16_to_f32, max_rel, rel_fro

GOLDEN = Path(__file__).resolve().parent / "golden"
F16, BF16 = 1, 2


def golden(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ---------------------------------------------------------------- RNG

@pytest.mark.parametrize("seed", [42, 43, 44, 45, 46, 0])
def test_rng_streams_bit_exact(oracle, seed):
    """splitmix64 + Box-Muller (tensor.c:289-339) reproduce the reference's
    streams bit for bit, seeds of every config and the zero-seed default."""
    g = golden("rng")
    oracle.orc_seed(seed)
    u = oracle.uniform(1000, -1.0, 1.0)
    n = oracle.normal(1000, 0.0, 1.0)
    n2 = oracle.normal(1000, 0.5, 0.02)
    assert np.array_equal(u.view(np.uint32), g[f"uniform_{seed}"].view(np.uint32))
    assert np.array_equal(n.view(np.uint32), g[f"normal_{seed}"].view(np.uint32))
    assert np.array_equal(n2.view(np.uint32), g[f"normal_sd002_{seed}"].view(np.uint32))


def test_rng_moments(oracle):
    oracle.orc_seed(7)
    u = oracle.uniform(200000, -1.0, 1.0)
    n = oracle.normal(200000, 0.0, 1.0)
    assert u.min() >= -1.0 and u.max() < 1.0
    assert abs(u.mean()) < 0.01 and abs(n.mean()) < 0.01 and abs(n.std() - 1.0) < 0.01


# ---------------------------------------------------------------- conversions

def test_decode_every_16bit_pattern(oracle):
    g = golden("convert")
    lib = oracle.lib
    h = np.arange(65536, dtype=np.uint32)
    f16 = np.array([oracle.orc_f16_to_f32(int(x)) for x in h], np.float32).view(np.uint32)
    bf = np.array([oracle.orc_bf16_to_f32(int(x)) for x in h], np.float32).view(np.uint32)
    assert np.array_equal(f16, g["f16_dec_bits"])
    assert np.array_equal(bf, g["bf16_dec_bits"])
    # finite f16 decode agrees with numpy's IEEE half
    fin = (h & 0x7C00) != 0x7C00
    ref = h.astype(np.uint16).view(np.float16).astype(np.float32).view(np.uint32)
    assert np.array_equal(f16[fin], ref[fin])
    del lib


def test_encode_matches_reference(oracle):
    g = golden("convert")
    f = g["enc_in_bits"].view(np.float32)
    to16 = np.empty(f.size, np.uint16)
    tob = np.empty(f.size, np.uint16)
    oracle.orc_cast_f32(F16, f.ctypes.data, to16.ctypes.data, f.size)
    oracle.orc_cast_f32(BF16, f.ctypes.data, tob.ctypes.data, f.size)
    # bf16: bit-exact for every non-NaN input.  The reference source maps a
    # NaN to the quiet NaN 0x7FC0 | bit 16 (convert.h:89-92) and the oracle
    # does so too; the reference's own -ffast-math build folds that test
    # away (finite-math) and rounds NaN bits like numbers instead.
    nan = np.isnan(f)
    assert np.array_equal(tob[~nan], g["to_bf16"][~nan])
    assert np.all(tob[nan] == (0x7FC0 | ((g["enc_in_bits"][nan] >> 16) & 1)))
    # f16: the reference's subnormal branch (convert.h:31-42) shifts the
    # 24-bit significand by 1-e instead of 1-e+13, so its results for
    # 2^-25 <= |x| < 2^-14 are not f16 values of x.  The oracle (and the
    # device cast) round those IEEE-correctly; everywhere else they agree
    # with the reference bit for bit.
    ex = (g["enc_in_bits"] >> 23) & 0xFF
    sub = (ex >= 127 - 25) & (ex <= 127 - 15)
    keep = ~sub & ~nan  # NaN payloads: the same finite-math caveat as bf16
    assert np.array_equal(to16[keep], g["to_f16"][keep])
    assert sub.sum() > 100 and not np.array_equal(to16[sub], g["to_f16"][sub])
    # finite values that stay finite: IEEE round-to-nearest-even (numpy) agrees
    fin = np.isfinite(f) & (np.abs(f) < 65504.0)
    assert np.array_equal(to16[fin], f[fin].astype(np.float16).view(np.uint16))


def test_bf16_rounding_planted_mistake_is_caught():
    """Truncation instead of RNE (a plausible slip) disagrees with the
    reference on the fixture's halfway and random inputs."""
    g = golden("convert")
    bits = g["enc_in_bits"]
    fin = (bits & 0x7F800000) != 0x7F800000
    trunc = (bits >> 16).astype(np.uint16)
    assert not np.array_equal(trunc[fin], g["to_bf16"][fin])


# ---------------------------------------------------------------- SGD

def test_sgd_trajectories_bit_exact(oracle):
    """Three steps of pg_sgd_step (sgd.c:111-162) under four configurations
    reproduce the reference's weights exactly."""
    g = golden("sgd")
    for ci, (lr, mu, d, wd, nest) in enumerate(g["cfgs"]):
        p = g[f"p0_{ci}"].copy()
        buf = np.zeros_like(p)
        for s in range(3):
            oracle.sgd_step(p, g[f"g_{ci}"][s].copy(), buf if mu else None, lr, mu, d, wd, bool(nest))
            assert np.array_equal(p.view(np.uint32), g[f"traj_{ci}"][s].view(np.uint32)), (ci, s)


def test_sgd_known_answers(oracle):
    """test_opt.c:48-138: plain, momentum, weight decay and Nesterov runs."""
    def run(lr, mu, d, wd, nest, steps, grad):
        p = np.array([1.0], np.float32)
        buf = np.zeros(1, np.float32)
        out = []
        for _ in range(steps):
            oracle.sgd_step(p, np.array([grad(p[0])], np.float32), buf if mu else None, lr, mu, d, wd, nest)
            out.append(float(p[0]))
        return out
    g2 = lambda x: 2.0 * (x - 2.0)
    assert np.allclose(run(0.1, 0, 0, 0, False, 2, g2), [1.2, 1.36], atol=1e-5)
    assert np.allclose(run(0.1, 0.9, 0, 0, False, 2, g2), [1.2, 1.54], atol=1e-5)
    assert np.allclose(run(0.1, 0, 0, 0.5, False, 1, lambda x: 2.0 * x), [0.75], atol=1e-5)
    assert np.allclose(run(0.1, 0.5, 0, 0, True, 2, g2), [1.3, 1.56], atol=1e-5)


def test_sgd_planted_mistake_is_caught():
    """Nesterov with buf alone (dropping the g' term) misses the fixture."""
    g = golden("sgd")
    lr, mu, d, wd, _ = g["cfgs"][0]
    p = g["p0_0"].astype(np.float32)
    gj = g["g_0"][0] + np.float32(wd) * p
    buf = np.float32(1 - d) * gj
    wrong = p - np.float32(lr) * (np.float32(mu) * buf)
    assert np.abs(wrong - g["traj_0"][0]).max() > 1e-5


# ---------------------------------------------------------------- Adam

# The reference's 8-wide loop takes sqrt and the quotient through x86
# reciprocal estimates plus one Newton step; its remainder loop (the last
# n % 8 elements of a tensor) uses IEEE sqrt and division, as the oracle does.
ADAM_UPDATE_TOL = 2.0 ** -21  # relative to the update, beyond one ulp of the weight
ADAM_SKIP = 3  # tests/golden/make_golden.py: the second parameter has no grad at this step


def _adam_cfg(g, ci):
    lr, b1, b2, eps, wd, ams, dec, lr1, wd1, step0 = (float(x) for x in g["cfgs"][ci])
    lrs = [lr, lr1 if lr1 > 0 else lr]  # adam.c:136-138
    wds = [wd, wd1 if wd1 >= 0 else wd]
    return lrs, wds, b1, b2, eps, bool(ams), bool(dec), int(step0)


def _adam_stepwise(oracle, g, ci, step_fn=None):
    """Runs configuration ci, each step starting from the reference's
    weights of the previous step (the moments are the run's own).  Returns
    the worst update error beyond one ulp of the weight, relative to the
    reference's update, and whether every remainder-loop element matched
    bit for bit."""
    lrs, wds, b1, b2, eps, ams, dec, step = _adam_cfg(g, ci)
    prev = [g[f"p0_{ci}"].reshape(-1).copy(), g[f"p1_{ci}"].reshape(-1).copy()]
    mom = [[np.zeros(p.size, np.float32) for _ in range(3)] for p in prev]
    worst, tails = 0.0, True
    for s in range(6):
        step += 1
        for k in range(2):
            ref = g[f"traj{k}_{ci}"][s].reshape(-1)
            if k == 1 and s == ADAM_SKIP:
                assert np.array_equal(ref, prev[k]), "a parameter without a grad must not move"
                continue
            p = prev[k].copy()
            gr = g[f"g{k}_{ci}"][s].reshape(-1).astype(np.float32)
            m, v, vm = mom[k]
            (step_fn or oracle.adam_step)(p, gr, m, v, vm if ams else None, lrs[k], b1, b2, eps, wds[k], ams,
                                          dec, step)
            r = ref.astype(np.float64)
            u = np.abs(prev[k].astype(np.float64) - r)
            beyond = np.maximum(np.abs(p.astype(np.float64) - r) - np.spacing(np.abs(ref)), 0.0)
            worst = max(worst, float((beyond / np.maximum(u, 1e-30)).max()))
            t = ref.size - ref.size % 8
            tails &= bool(np.array_equal(p[t:].view(np.uint32), ref[t:].view(np.uint32)))
            prev[k] = ref.copy()
    assert step == int(g[f"final_step_{ci}"])
    return worst, tails


@pytest.mark.parametrize("ci", range(5))
def test_adam_matches_reference(oracle, ci):
    """Six steps of pg_adam_step (adam.c:113-181) per configuration: Adam
    with L2 decay, AdamW, amsgrad, per-parameter lr / wd overrides, a
    parameter without a grad (skipped while the step counter advances) and
    a counter set by pg_adam_set_step.  Step by step from the reference's
    weights, the elements its build computes with IEEE arithmetic match bit
    for bit and the rest within one ulp plus 2^-21 of the update; run freely
    for six steps the weights stay within 2^-23 * max(1, |p|) * 2."""
    g = golden("adam")
    worst, tails = _adam_stepwise(oracle, g, ci)
    assert tails and worst <= ADAM_UPDATE_TOL, (tails, worst)
    lrs, wds, b1, b2, eps, ams, dec, step = _adam_cfg(g, ci)
    ps = [g[f"p0_{ci}"].reshape(-1).copy(), g[f"p1_{ci}"].reshape(-1).copy()]
    mom = [[np.zeros(p.size, np.float32) for _ in range(3)] for p in ps]
    for s in range(6):
        step += 1
        for k in range(2):
            if k == 1 and s == ADAM_SKIP:
                continue
            m, v, vm = mom[k]
            oracle.adam_step(ps[k], g[f"g{k}_{ci}"][s].reshape(-1).astype(np.float32), m, v,
                             vm if ams else None, lrs[k], b1, b2, eps, wds[k], ams, dec, step)
    for k in range(2):
        ref = g[f"traj{k}_{ci}"][5].reshape(-1)
        assert np.all(np.abs(ps[k] - ref) <= 2.0 ** -22 * np.maximum(1.0, np.abs(ref))), k


def test_adam_source_order_misses_reference(oracle):
    """Why the oracle follows the build's evaluation order: adam.c:167-176
    evaluated as written (b2*v + (1 - b2)*g*g, m / bc1, v / bc2) leaves the
    reference's weights by up to ~4e-5 of the update at beta2 = 0.999 (the
    reassociated v = g^2 + b2*(v - g^2) cancels), far outside the band."""
    f = np.float32
    g = golden("adam")

    def as_written(p, gr, m, v, vm, lr, b1, b2, eps, wd, ams, dec, step):
        bc1 = max(f(1) - np.power(f(b1), f(step)), f(1e-12))
        bc2 = max(f(1) - np.power(f(b2), f(step)), f(1e-12))
        if wd != 0 and dec:
            p[:] = p - f(lr) * f(wd) * p
        if wd != 0 and not dec:
            gr = gr + f(wd) * p
        m[:] = f(b1) * m + (f(1) - f(b1)) * gr
        v[:] = f(b2) * v + (f(1) - f(b2)) * gr * gr
        vv = v
        if ams:
            vm[:] = np.maximum(vm, v)
            vv = vm
        p[:] = p - f(lr) * (m / bc1) / (np.sqrt(vv / bc2) + f(eps))

    worst, _ = _adam_stepwise(oracle, g, 1, as_written)
    assert worst > 20 * ADAM_UPDATE_TOL


def test_adam_known_answers(oracle):
    """Closed forms.  Step 1 moves every weight with g != 0 by lr * sign(g)
    (the bias corrections cancel the moment scales), leaves g == 0 weights
    alone, and AdamW first shrinks by lr*wd.  test_training.c:237-268: with
    grads of 1, a parameter with lr 0.1 moves 0.1 and one with 0.01 moves
    0.01."""
    p0 = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    gr = np.array([0.3, -5.0, 0.0, 1e-3], np.float32)
    p = p0.copy()
    z = [np.zeros(4, np.float32) for _ in range(3)]
    oracle.adam_step(p, gr, z[0], z[1], None, 0.01, 0.9, 0.999, 1e-8, 0.0, False, True, 1)
    want = p0 - 0.01 * np.sign(gr)
    assert np.allclose(p, want, rtol=0, atol=2e-6) and p[2] == p0[2]
    p = p0.copy()
    z = [np.zeros(4, np.float32) for _ in range(3)]
    oracle.adam_step(p, np.zeros(4, np.float32), z[0], z[1], None, 0.1, 0.9, 0.999, 1e-8, 0.5, False, True, 1)
    assert np.array_equal(p, p0 - np.float32(0.1 * 0.5) * p0)
    for lr in (0.1, 0.01):
        x = np.ones(1, np.float32)
        z = [np.zeros(1, np.float32) for _ in range(3)]
        oracle.adam_step(x, np.ones(1, np.float32), z[0], z[1], None, lr, 0.9, 0.999, 1e-8, 0.0, False, True, 1)
        assert abs((1.0 - x[0]) - lr) < 1e-6
    # amsgrad keeps the running maximum of v: a smaller second grad moves
    # the weight less than plain Adam does
    outs = []
    for ams in (False, True):
        x = np.zeros(1, np.float32)
        m, v, vm = (np.zeros(1, np.float32) for _ in range(3))
        for t, gv in enumerate((10.0, 0.1), start=1):
            oracle.adam_step(x, np.array([gv], np.float32), m, v, vm, 0.01, 0.9, 0.999, 1e-8, 0.0, ams, True, t)
        outs.append(float(x[0]))
        if ams:
            assert vm[0] >= v[0] > 0
    assert abs(outs[1]) < abs(outs[0])


def test_adam_planted_mistakes_are_caught(oracle):
    """A bias correction one step off, L2 decay applied as AdamW, or the
    betas swapped each leave the tolerance band."""
    g = golden("adam")

    def off_by_one(p, gr, m, v, vm, lr, b1, b2, eps, wd, ams, dec, step):
        oracle.adam_step(p, gr, m, v, vm, lr, b1, b2, eps, wd, ams, dec, step + 1)

    def decay_kind(p, gr, m, v, vm, lr, b1, b2, eps, wd, ams, dec, step):
        oracle.adam_step(p, gr, m, v, vm, lr, b1, b2, eps, wd, ams, not dec, step)

    def swapped(p, gr, m, v, vm, lr, b1, b2, eps, wd, ams, dec, step):
        oracle.adam_step(p, gr, m, v, vm, lr, b2, b1, eps, wd, ams, dec, step)

    for fn, ci in ((off_by_one, 0), (decay_kind, 2), (swapped, 3)):
        worst, _ = _adam_stepwise(oracle, g, ci, fn)
        assert worst > 100 * ADAM_UPDATE_TOL, fn.__name__


# ---------------------------------------------------------------- gradient clipping

def test_clip_matches_reference(oracle):
    """pg_grad_norm / pg_clip_grad_norm / pg_clip_grad_value (clip.c:5-61):
    the norm (f64 sum, f32 result) and every clipped grad bit for bit, with
    NULL entries and grad-less nodes skipped, no change when the norm is
    within max_norm, eps < 0 taken as 1e-6, and a grad listed twice counted
    and scaled twice."""
    g = golden("clip")
    gs = lambda c: [g[f"g{i}_{c}"].copy() for i in range(3)]
    with_gaps = lambda a: [a[0], None, a[1], None, a[2]]
    bits = lambda x: np.asarray(x, np.float32).view(np.uint32)

    a = gs(0)
    assert bits(oracle.grad_norm(with_gaps(a))) == bits(g["norm_0"])
    a = gs(1)
    assert bits(oracle.clip_grad_norm(with_gaps(a), float(g["max_norm_1"]), 1e-6)) == bits(g["ret_1"])
    for i in range(3):
        assert np.array_equal(bits(a[i]), bits(g[f"after{i}_1"])), i
    a = gs(2)
    assert bits(oracle.clip_grad_norm(with_gaps(a), float(g["max_norm_2a"]), 1e-6)) == bits(g["ret_2a"])
    assert bits(oracle.clip_grad_norm(with_gaps(a), float(g["max_norm_2b"]), -1.0)) == bits(g["ret_2b"])
    for i in range(3):
        assert np.array_equal(bits(a[i]), bits(g[f"after{i}_2"])), i
    a = gs(3)
    assert bits(oracle.clip_grad_norm([a[0], a[0], a[1]], 1.0, 1e-6)) == bits(g["ret_3"])
    for i in range(3):
        assert np.array_equal(bits(a[i]), bits(g[f"after{i}_3"])), i
    a = gs(4)
    oracle.clip_grad_value(with_gaps(a), float(g["clip_value_4"]))
    for i in range(3):
        assert np.array_equal(bits(a[i]), bits(g[f"after{i}_4"])), i
    assert bits(oracle.grad_norm([g["big_g"].copy()])) == bits(g["big_norm"])
    assert oracle.clip_grad_norm([a[0]], 0.0, 1e-6) == -1.0


def test_clip_closed_forms_and_planted_mistake(oracle):
    """The norm of a 3-4-12 vector is 13; clipping to 6.5 halves it up to
    eps; a norm summed in f32 instead of f64 misses the reference on the
    large fixture."""
    v = np.array([3.0, 4.0, 12.0], np.float32)
    assert oracle.grad_norm([v.copy()]) == 13.0
    w = v.copy()
    assert oracle.clip_grad_norm([w], 6.5, 0.0) == 13.0
    assert np.array_equal(w, v * np.float32(0.5))
    g = golden("clip")
    big = g["big_g"]
    f32_sum = np.float32(0)
    for x in big:  # serial f32 accumulation
        f32_sum = np.float32(f32_sum + x * x)
    assert np.float32(np.sqrt(f32_sum)) != g["big_norm"]
    assert abs(float(np.sqrt(np.sum(big.astype(np.float64) ** 2))) - float(g["big_norm"])) <= np.spacing(g["big_norm"])


# ---------------------------------------------------------------- checkpoint bytes

def test_pgt1_bytes_match_reference(oracle):
    """pg_tensor_save (tensor.c:607-650) and pg_module_save (module.c:91-104):
    the oracle's records equal the files the reference wrote, for f32, f16
    and bf16 tensors of ranks 1 to 8 and a three-parameter module."""
    import struct
    g = golden("ckpt")
    for i in range(5):
        dt, arr = int(g[f"t{i}_dtype"]), g[f"t{i}_data"]
        assert oracle.pgt1_bytes(dt, arr) == g[f"t{i}_bytes"].tobytes(), i
        assert oracle.pgt1_check(g[f"t{i}_bytes"].tobytes()) == g[f"t{i}_bytes"].size
    mod = b"PGMD" + struct.pack("<IQ", 1, 3) + b"".join(oracle.pgt1_bytes(0, g[f"mod_p{i}"]) for i in range(3))
    assert mod == g["mod_bytes"].tobytes()


def test_pgt1_loader_checks_match_reference(oracle):
    """pg_tensor_load's verdict (tensor.c:655-702) on crafted records: bad
    magic, version, dtype, ndim 0 or 9, a zero or oversized dimension (the
    10,000,000 bound is inclusive), numel or element size disagreeing, and
    truncation."""
    g = golden("ckpt")
    for i, (name, ok) in enumerate(zip(g["crafted_names"], g["crafted_loads"])):
        assert bool(oracle.pgt1_check(g[f"crafted_{i}"].tobytes())) == bool(ok), name


def test_pgt1_planted_mistakes_are_caught(oracle):
    """A shape written as u32 or a big-endian header would not be the
    reference's file."""
    import struct
    g = golden("ckpt")
    arr = g["t0_data"]
    ref = g["t0_bytes"].tobytes()
    as_u32 = b"PGT1" + struct.pack("<III", 1, 0, 2) + struct.pack("<II", *arr.shape) + struct.pack(
        "<QQ", arr.size, 4) + arr.tobytes()
    big = b"PGT1" + struct.pack(">III", 1, 0, 2) + struct.pack(">QQ", *arr.shape) + struct.pack(
        ">QQ", arr.size, 4) + arr.tobytes()
    assert as_u32 != ref and big != ref
    assert oracle.pgt1_check(as_u32) == 0 and oracle.pgt1_check(big) == 0


# ---------------------------------------------------------------- elementwise chains

def test_chain1_matches_reference(oracle):
    g = golden("chain1")
    da, db, dc = oracle.chain1(g["a"].ravel().copy(), g["b"].ravel().copy(), g["c"].ravel().copy())
    for tag in ("jit", "eager"):
        assert max_rel(da, g[f"da_{tag}"].ravel()) <= 1e-6
        assert max_rel(db, g[f"db_{tag}"].ravel()) <= 1e-6
        assert max_rel(dc, g[f"dc_{tag}"].ravel()) <= 1e-6


def test_chain1_closed_form_and_planted_mistake(oracle):
    """tanh' = 1 - tanh^2 against d/dx tanh = sech^2 in f64; a tanh' that
    forgets the square fails the 1e-5 bar."""
    g = golden("chain1")
    a, b, c = (g[k].astype(np.float64).ravel() for k in "abc")
    t0 = a + b
    t1 = t0 * c
    step = (t1 > 0).astype(np.float64)
    sech2 = 1.0 / np.cosh(np.maximum(t1, 0)) ** 2
    dc64 = sech2 * step * t0
    da64 = sech2 * step * c
    da, db, dc = oracle.chain1(g["a"].ravel().copy(), g["b"].ravel().copy(), g["c"].ravel().copy())
    assert max_rel(da, da64) <= 1e-5 and max_rel(dc, dc64) <= 1e-5
    wrong = (1.0 - np.tanh(np.maximum(t1, 0))) * step * c
    assert max_rel(wrong, g["da_jit"].ravel()) > 1e-2


def test_chain2_matches_reference(oracle):
    g = golden("chain2")
    x, bias, gg = g["x"], g["bias"], g["g"]
    R, Cc = x.shape
    dx, dg, db, db64 = oracle.chain2(x.copy(), bias.copy(), gg.copy())
    for tag in ("jit", "eager"):
        assert max_rel(dx, g[f"dx_{tag}"]) <= 1e-5
        assert max_rel(dg, g[f"dg_{tag}"]) <= 1e-5
        bound = 4 * R * np.finfo(np.float32).eps * np.abs(dx).sum(axis=0) + 1e-30
        assert np.all(np.abs(g[f"dbias_{tag}"] - db64) <= bound)
    assert np.all(np.abs(db - db64) <= 4 * R * np.finfo(np.float32).eps * np.abs(dx).sum(axis=0))


def test_chain2_gelu_grad_closed_form_and_planted_mistake(oracle):
    """GELU'(x) = Phi(x) + x phi(x) in f64; dropping the x phi(x) term (a
    plausible slip) fails the bar."""
    g = golden("chain2")
    x, bias, gg = (g[k].astype(np.float64) for k in ("x", "bias", "g"))
    t0 = x + bias
    Phi = 0.5 * (1.0 + np.vectorize(math.erf)(t0 / math.sqrt(2.0)))
    phi = np.exp(-0.5 * t0 * t0) / math.sqrt(2.0 * math.pi)
    s = 1.0 / (1.0 + np.exp(-gg))
    dx64 = s * (Phi + t0 * phi)
    dg64 = t0 * Phi * s * (1.0 - s)
    dx, dg, _, _ = oracle.chain2(g["x"].copy(), g["bias"].copy(), g["g"].copy())
    assert max_rel(dx, dx64) <= 1e-5 and max_rel(dg, dg64) <= 1e-5
    assert max_rel(s * Phi, g["dx_jit"]) > 1e-3


def test_gelu_backward_matches_reference_eager_grad(oracle):
    """orc_gelu_backward(z, g) = g * gelu'(z): the reference's eager chain-2
    backward computes dx = sigmoid(g) * grad_gelu(x + bias) with exactly this
    call (autograd.c:519-559, :794-801), so its golden dx_eager is reproduced
    to f32 rounding; the f64 closed form Phi + x phi agrees, and dropping the
    x phi term fails."""
    g = golden("chain2")
    t0 = (g["x"] + g["bias"]).astype(np.float32)
    s = (1.0 / (1.0 + np.exp(-g["g"].astype(np.float64)))).astype(np.float32)
    got = oracle.gelu_backward(t0, s)
    assert max_rel(got, g["dx_eager"]) <= 1e-5
    t = t0.astype(np.float64)
    Phi = 0.5 * (1.0 + np.vectorize(math.erf)(t / math.sqrt(2.0)))
    phi = np.exp(-0.5 * t * t) / math.sqrt(2.0 * math.pi)
    assert max_rel(got, s * (Phi + t * phi)) <= 1e-5
    assert max_rel(s * Phi, got) > 1e-3


# ---------------------------------------------------------------- GEMM

def _gemm_keys(g):
    return sorted({k.rsplit("_", 1)[0] for k in g if k[:3] in ("f16", "bf1")})


def test_gemm_ex_matches_reference(oracle):
    """pg_gemm_ex / hgemm / bgemm (gemm.c:575-629): the oracle's f32
    accumulation of upcast operands agrees with the reference up to
    summation order, and both sit within f32 bounds of an f64 sum."""
    g = golden("gemm")
    for key in _gemm_keys(g):
        dt = F16 if key.startswith("f16") else BF16
        a, b, c = g[f"{key}_a"], g[f"{key}_b"], g[f"{key}_c"]
        mine = oracle.gemm(dt, a, b)
        ref64 = oracle.gemm(dt, a, b, f64=True)
        k = a.shape[1]
        if dt == F16 and k > 256 and bool(g["host_avx512fp16"]):
            # the reference's AVX512-FP16 micro (hgemm_avx512fp16.c:22-34)
            # resets the accumulator of columns 0-15 of every 32-column
            # strip at each KC=256 block, so those columns hold only the
            # last block's products; the other columns are the full sum.
            # Hosts without AVX512-FP16 run the scalar micro, which is right.
            lo = (np.arange(c.shape[1]) % 32) < 16
            kk = (k - 1) // 256 * 256
            last = oracle.gemm(dt, np.ascontiguousarray(a[:, kk:]), np.ascontiguousarray(b[kk:, :]))
            assert rel_fro(last[:, lo], c[:, lo]) <= 1e-6, key
            assert rel_fro(mine[:, ~lo], c[:, ~lo]) <= 1e-6, key
            continue
        assert rel_fro(mine, c) <= 1e-6, key
        assert rel_fro(c, ref64) <= 2 * k * 6e-8 + 1e-7, key
        assert rel_fro(mine, ref64) <= 2 * k * 6e-8 + 1e-7, key
    a, b = g["f32_a"], g["f32_b"]
    assert np.allclose(oracle.gemm(0, a, b), g["f32_c"], rtol=1e-6, atol=1e-6)


def test_gemm_brute_force_and_transpose_flags(oracle):
    """op(A)op(B) with the transpose flags against numpy f64 on ragged
    shapes; a transposed operand would fail."""
    rng = np.random.default_rng(1)
    for (m, n, k) in [(5, 7, 3), (1, 9, 17), (13, 1, 4)]:
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        a16, b16 = oracle.cast16(BF16, a), oracle.cast16(BF16, b)
        af, bf = bf16_to_f32(a16).astype(np.float64), bf16_to_f32(b16).astype(np.float64)
        want = af @ bf
        assert rel_fro(oracle.gemm(BF16, a16, b16), want) <= 1e-6
        assert rel_fro(oracle.gemm(BF16, np.ascontiguousarray(a16.T), b16, ta=True), want) <= 1e-6
        assert rel_fro(oracle.gemm(BF16, a16, np.ascontiguousarray(b16.T), tb=True), want) <= 1e-6
        if m == n == k:
            assert rel_fro(oracle.gemm(BF16, a16, b16, ta=True), want) > 1e-2


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_gemm_acc32_is_the_serial_dot_product(oracle, ta, tb):
    """orc_gemm_acc32 computes each output as acc = acc + a*b over k in order,
    every product and sum rounded to f32: numpy float32 arithmetic over the
    whole output at once does the same per element, so the two agree bit for
    bit (ragged m, n; beta = 1 adds the sum to the old C after the loop)."""
    rng = np.random.default_rng(5)
    m, n, k = 7, 37, 300
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    a16, b16 = oracle.cast16(BF16, a), oracle.cast16(BF16, b)
    af, bf = bf16_to_f32(a16), bf16_to_f32(b16)
    acc = np.zeros((m, n), np.float32)
    for p in range(k):
        acc = acc + np.outer(af[:, p], bf[p, :]).astype(np.float32)
    A = np.ascontiguousarray(a16.T) if ta else a16
    B = np.ascontiguousarray(b16.T) if tb else b16
    got = oracle.gemm(BF16, A, B, ta=bool(ta), tb=bool(tb), threads=3)
    assert np.array_equal(got.view(np.uint32), acc.view(np.uint32))
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    c = c0.copy()
    oracle.orc_gemm_acc32(BF16, ta, tb, m, n, k, A.ctypes.data, A.shape[1], B.ctypes.data, B.shape[1],
                          c.ctypes.data, n, 1, 2)
    assert np.array_equal(c.view(np.uint32), (c0 + acc).view(np.uint32))


def test_matmul_backward_matches_reference(oracle):
    """bwd_matmul (autograd.c:561-706) on 16-bit leaves with dC exactly
    representable: dA = dC.W^T and dW = A^T.dC from the oracle agree with
    the reference up to summation order."""
    g = golden("matmul_bwd")
    keys = sorted({k.rsplit("_", 1)[0] for k in g if k.startswith(("f16", "bf16"))})
    for key in keys:
        dt = F16 if key.startswith("f16") else BF16
        a, w, gr = g[f"{key}_a"], g[f"{key}_w"], g[f"{key}_g"]
        g16 = oracle.cast16(dt, gr)
        da = oracle.gemm(dt, g16, w, tb=True)
        dw = oracle.gemm(dt, a, g16, ta=True)
        assert rel_fro(da, g[f"{key}_da"]) <= 1e-6, key
        assert rel_fro(dw, g[f"{key}_dw"]) <= 1e-6, key
        assert rel_fro(oracle.gemm(dt, a, w), g[f"{key}_c"]) <= 1e-6, key
    a, w, gr = g["bmm_a"], g["bmm_w"], g["bmm_g"]
    da = np.einsum("bmn,bkn->bmk", gr.astype(np.float64), w.astype(np.float64))
    dw = np.einsum("bmk,bmn->bkn", a.astype(np.float64), gr.astype(np.float64))
    assert rel_fro(g["bmm_da"], da) <= 1e-6 and rel_fro(g["bmm_dw"], dw) <= 1e-6


# ---------------------------------------------------------------- losses

def test_mse_scale_matches_reference(oracle):
    """mean_all divides by the last axis only: mse grad = 2 (p - t) / 10
    on [6, 10] (autograd.c:1018-1043, :1758-1771)."""
    import ctypes as C
    g = golden("mse")
    d = g["pred"] - g["tgt"]
    shape = (C.c_size_t * 2)(6, 10)
    s_mean = oracle.orc_mse_grad_scale(2, shape, True)
    s_sum = oracle.orc_mse_grad_scale(2, shape, False)
    assert np.allclose(s_mean * d, g["dpred_mean"], rtol=1e-6, atol=0)
    assert np.allclose(s_sum * d, g["dpred_sum"], rtol=1e-6, atol=0)
    assert np.allclose(g["loss_mean"], (d.astype(np.float64) ** 2).sum() / 10, rtol=1e-5)
    assert not np.allclose(2.0 / 60 * d, g["dpred_mean"], rtol=1e-3)


# ---------------------------------------------------------------- MLP step

def _mlp_run(oracle, g, dtype, steps=2, nesterov=True):
    L = len(g["dims"]) - 1
    Ws = [g[f"W{i}_0"].copy() for i in range(L)]
    bs = [g[f"b{i}_0"].copy() for i in range(L)]
    Wb = [np.zeros_like(w) for w in Ws]
    bb = [np.zeros_like(b) for b in bs]
    hist = []
    for _ in range(steps):
        loss, dW, db = oracle.mlp_step(dtype, g["x"], g["t"], Ws, bs, Wb, bb, 0.01, 0.9, 0.0, 1e-4, nesterov)
        hist.append((loss, dW, db, [w.copy() for w in Ws], [b.copy() for b in bs]))
    return hist


def _mlp_errors(g, hist):
    """(loss rel, worst grad rel-Frobenius, worst updated-param max rel)"""
    L = len(g["dims"]) - 1
    el, eg, ep = 0.0, 0.0, 0.0
    for s, (loss, dW, db, Ws, bs) in enumerate(hist, start=1):
        ref = float(g[f"loss_{s}"][0])
        el = max(el, abs(loss - ref) / abs(ref))
        for i in range(L):
            eg = max(eg, rel_fro(dW[i], g[f"dW{i}_{s}"]), rel_fro(db[i], g[f"db{i}_{s}"]))
            for got, key in ((Ws[i], f"W{i}_{s}"), (bs[i], f"b{i}_{s}")):
                want = g[key].astype(np.float64)
                ep = max(ep, float(np.abs(got - want).max() / np.abs(want).max()))
    return el, eg, ep


def test_mlp_step_matches_reference(oracle):
    """orc_mlp_step in f32 reproduces two training steps of the reference's
    own MLP (linear + gelu layers, mse, pg_backward, Nesterov pg_sgd_step):
    loss, every weight and bias grad, and the updated parameters.  The
    remaining differences come from the GEMM summation order (the reference
    blocks k by 256 with AVX-512 partial sums, the oracle sums in k order)."""
    g = golden("mlp")
    el, eg, ep = _mlp_errors(g, _mlp_run(oracle, g, 0))
    assert el < 1e-6, el
    assert eg < 2e-6, eg
    assert ep < 1e-6, ep


def test_mlp_step_planted_mistakes_are_caught(oracle):
    """The same comparison rejects plausible mistakes: GEMM operands rounded
    where the reference keeps f32, and the update without Nesterov."""
    g = golden("mlp")
    _, eg, _ = _mlp_errors(g, _mlp_run(oracle, g, BF16, steps=1))
    assert eg > 1e-3, eg
    _, _, ep = _mlp_errors(g, _mlp_run(oracle, g, 0, steps=1, nesterov=False))
    assert ep > 1e-5, ep


def test_mlp_step_bf16_close_to_f32(oracle):
    """The 16-bit mode differs from the f32 step by operand rounding only:
    grads stay within a few bf16 ulps (rel Frobenius < 2e-2) of the f32 run,
    and the f16 mode, with 3 more mantissa bits, lands 8x closer."""
    g = golden("mlp")
    ref = _mlp_run(oracle, g, 0, steps=1)[0]
    errs = {}
    for dt in (F16, BF16):
        run = _mlp_run(oracle, g, dt, steps=1)[0]
        errs[dt] = max(rel_fro(a, b) for a, b in zip(run[1] + run[2], ref[1] + ref[2]))
    assert errs[BF16] < 2e-2, errs
    assert errs[F16] < errs[BF16] / 4, errs
