"""The device's RNE conversions against the reference's own (convert.h:15-104),
through every path that rounds on the device: the cast kernel
(pg_amd_tensor_to_dtype, also what makes the kept 16-bit operand copies and
rounds upstream grads), the linear16 GEMM epilogue's 16-bit output copy, and
pg_sgd_step's rewrite of a weight's 16-bit copy.

tests/golden/convert.npz holds the reference's encodings of 29,030 f32
inputs (specials, ties, subnormals, random bits) and its decodings of every
16-bit pattern.  Agreement is bit for bit, except for NaN decodings (see
test_cast_kernel_decodes_every_pattern) and where the oracle tests document
the reference build as wrong: NaN inputs to the bf16 encoder (its
-ffast-math build folds the NaN test away; the source's rule 0x7FC0 | bit 16
is kept) and f16 subnormal results (its encoder shifts by 1-e instead of
1-e+13; IEEE round-to-nearest-even is kept, checked against the oracle and
numpy's IEEE half).
"""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from oracle_lib import rel_fro
from picograd_amd.capi import BF16, F16, F32
from picograd_amd.mlp import ACT_NONE

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def golden():
    with np.load(GOLDEN / "convert.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _expected(g, dt):
    """The golden encodings with the documented exceptions replaced by the
    source rule (bf16 NaN) or IEEE (f16 subnormal results)."""
    bits = g["enc_in_bits"]
    f = bits.view(np.float32)
    nan = np.isnan(f)
    if dt == BF16:
        want = g["to_bf16"].copy()
        want[nan] = (0x7FC0 | ((bits[nan] >> 16) & 1)).astype(np.uint16)
        return want
    want = g["to_f16"].copy()
    ex = (bits >> 23) & 0xFF
    sub = (ex >= 127 - 25) & (ex <= 127 - 15)
    with np.errstate(over="ignore"):
        want[sub] = f[sub].astype(np.float16).view(np.uint16)
    return want


def _f16_nan_rule(bits):
    """NaN -> quiet NaN keeping the top payload bits (convert.h:22-28)."""
    man = bits & 0x7FFFFF
    q = ((bits >> 16) & 0x8000) | 0x7C00 | (man >> 13)
    q = np.where((q & 0x3FF) == 0, q | 1, q)
    return (q | 0x200).astype(np.uint16)


@pytest.mark.parametrize("dt", [BF16, F16])
def test_cast_kernel_encodes_like_the_reference(lib, oracle, dt):
    g = golden()
    bits = g["enc_in_bits"]
    f = bits.view(np.float32)
    t = lib.tensor(f)
    h = lib._check(lib.pg_amd_tensor_to_dtype(t, dt))
    got = lib.read(h)
    want = _expected(g, dt)
    nan = np.isnan(f)
    if dt == F16:
        want[nan] = _f16_nan_rule(bits[nan])
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(hex(bits[i]), hex(got[i]), hex(want[i])) for i in bad[:8]]
    # the oracle's encoder is the same function
    ref = oracle.cast16(dt, f)
    assert np.array_equal(got, ref)
    lib.pg_tensor_free(t)
    lib.pg_tensor_free(h)


@pytest.mark.parametrize("dt", [BF16, F16])
def test_cast_kernel_decodes_every_pattern(lib, dt):
    g = golden()
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    t = lib.tensor(pats, dt)
    y = lib._check(lib.pg_amd_tensor_to_dtype(t, F32))
    got = lib.read(y).view(np.uint32)
    want = (g["bf16_dec_bits"] if dt == BF16 else g["f16_dec_bits"]).copy()
    # NaN patterns: the decoders keep the payload as it is (convert.h:71-72,
    # :99-104: f16 sign | 0x7F800000 | man << 13, bf16 h << 16).  The golden
    # file's NaN entries came back from the reference through a Python
    # float, which sets the quiet bit of a signalling NaN; they equal the
    # source rule with that bit set.
    p32 = pats.astype(np.uint32)
    rule = p32 << 16 if dt == BF16 else ((p32 & 0x8000) << 16) | 0x7F800000 | ((p32 & 0x3FF) << 13)
    nan = np.isnan(want.view(np.float32))
    assert np.array_equal(want[nan], rule[nan] | 0x400000)
    want[nan] = rule[nan]
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (bad.size, [(hex(i), hex(got[i]), hex(want[i])) for i in bad[:12]])
    # and back: every non-NaN pattern survives f32 and returns to itself
    back = lib._check(lib.pg_amd_tensor_to_dtype(y, dt))
    rb = lib.read(back)
    f = got.view(np.float32)
    assert np.array_equal(rb[~np.isnan(f)], pats[~np.isnan(f)])
    for x in (t, y, back):
        lib.pg_tensor_free(x)


class _DataRef(C.Structure):
    _fields_ = [("ptr", C.c_void_p), ("nbytes", C.c_size_t), ("refs", C.c_int), ("shadow", C.c_void_p),
                ("shadow_dtype", C.c_int), ("shadow_stale", C.c_bool), ("shadow_cols", C.c_size_t),
                ("shadow_ld", C.c_size_t), ("shadow_bytes", C.c_size_t)]


def _read_kept16(lib, t, rows, cols, dt):
    """The kept 16-bit copy of f32 tensor t [rows, cols], decoded exactly:
    pg_gemm_ex(copy [rows, cols] . I [cols, cols]) puts each element into
    C as its one nonzero product with 1.0, summed with zeros in f32 (so the
    copy must hold no infinities or NaNs, and a -0 reads as +0)."""
    ref = _DataRef.from_address(lib.tinfo(t).data_ref)
    assert ref.shadow and not ref.shadow_stale and ref.shadow_dtype == dt
    e32 = lib.tensor(np.eye(cols, dtype=np.float32))
    te = lib._check(lib.pg_amd_tensor_to_dtype(e32, dt))
    tc = lib.pg_tensor_empty_dtype(F32, 2, (C.c_size_t * 2)(rows, cols))
    lib.pg_gemm_ex(dt, rows, cols, cols, ref.shadow, cols, lib.tinfo(te).dev, cols, lib.tinfo(tc).dev, cols)
    out = lib.read(tc)
    for x in (e32, te, tc):
        lib.pg_tensor_free(x)
    return out


def _decoded(oracle, dt, x):
    """The oracle's encoding of x, decoded, with -0 as +0 (what the identity
    GEMM reads back for a -0 in the copy; the cast-kernel tests pin zero
    signs bit for bit)."""
    h = oracle.cast16(dt, x)
    f = (h.astype(np.uint32) << 16).view(np.float32) if dt == BF16 else h.view(np.float16).astype(np.float32)
    return np.where(f == 0.0, np.float32(0.0), f)


def _inputs(g, n, dt):
    """Golden encoder inputs that stay finite in dt (the identity GEMM that
    reads a copy back cannot carry an infinity) and are not -0 (0 + -0 is
    +0 in the epilogue's sum)."""
    bits = g["enc_in_bits"]
    f = bits.view(np.float32)
    keep = np.isfinite(f) & (np.abs(f) < (65504.0 if dt == F16 else 1e30)) & (bits != 0x80000000)
    out = f[keep][:n]
    assert out.size == n
    return out


@pytest.mark.parametrize("dt", [BF16, F16])
def test_linear16_epilogue_rounds_like_the_reference(lib, oracle, dt):
    """out = 0 . W + b with b = golden inputs: the epilogue writes out and
    its 16-bit copy; the copy must be the reference's encoding of b."""
    g = golden()
    N = 4096
    b = _inputs(g, N, dt)
    R, K = 64, 64
    x = np.zeros((R, K), np.float32)
    w = np.zeros((K, N), np.float32)
    nx, nw, nb = lib.var(x), lib.var(w), lib.var(b)
    out = lib._check(lib.pg_amd_ag_linear16(nx, nw, nb, ACT_NONE, dt))
    vals = lib.value(out)
    assert np.array_equal(vals, np.broadcast_to(b, (R, N)))
    kept = _read_kept16(lib, lib.node(out).value, R, N, dt)
    want = np.broadcast_to(_decoded(oracle, dt, b), (R, N))
    assert np.array_equal(kept.view(np.uint32), want.view(np.uint32))
    for n in (out, nx, nw, nb):
        lib.pg_node_free(n)


@pytest.mark.parametrize("dt", [BF16, F16])
def test_sgd_rewrites_the_kept_copy_like_the_reference(lib, oracle, dt):
    """A weight with a kept 16-bit copy, stepped by pg_sgd_step with a zero
    grad and lr 0 (the values stay): the update pass rewrites the copy, which
    must be the reference's encoding of the weight."""
    from picograd_amd.capi import SgdCfg
    g = golden()
    K, N = 64, 256
    w = _inputs(g, K * N, dt).reshape(K, N)
    nw = lib.var(w)
    x = lib.var(np.zeros((8, K), np.float32), requires_grad=False)
    y = lib._check(lib.pg_amd_ag_matmul16(x, nw, dt))  # makes W's kept copy
    loss = lib.op("sum_all", y)
    opt = lib.pg_sgd_new(C.byref(SgdCfg(0.0, 0.0, 0.0, 0.0, False)))
    assert lib.pg_sgd_add_param(opt, nw) == 0
    lib.pg_backward(loss)
    # a write marks the copy stale; the step must remake it in its pass
    lib.pg_amd_tensor_modified(lib.node(nw).value)
    lib.pg_sgd_step(opt)
    kept = _read_kept16(lib, lib.node(nw).value, K, N, dt)
    assert np.array_equal(kept.view(np.uint32), _decoded(oracle, dt, w).view(np.uint32))
    lib.pg_sgd_free(opt)
    for n in (loss, y, x, nw):
        lib.pg_node_free(n)


@pytest.mark.parametrize("opt_kind", ["sgd", "adam"])
@pytest.mark.parametrize("dt", [BF16, F16])
def test_pitched_kept_copy_of_a_narrow_weight(lib, oracle, dt, opt_kind):
    """A weight [64, 10] (rows not whole 16-byte pieces) used as a GEMM
    operand keeps its 16-bit copy as rows at a pitch of 16 with zeros
    between (no padded copy per call); the optimiser's update pass rewrites
    it in that layout.  After a real step the copy must be the reference's
    encoding of the updated weight, and the pad columns zero."""
    from picograd_amd.capi import SgdCfg
    K, N, LD = 64, 10, 16
    rng = np.random.default_rng(dt * 7 + len(opt_kind))
    w = (rng.standard_normal((K, N)) * 0.5).astype(np.float32)
    nw = lib.var(w)
    x = lib.var(rng.standard_normal((8, K)).astype(np.float32), requires_grad=False)
    y = lib._check(lib.pg_amd_ag_matmul16(x, nw, dt))
    ref = _DataRef.from_address(lib.tinfo(lib.node(nw).value).data_ref)
    assert ref.shadow and ref.shadow_cols == N and ref.shadow_ld == LD and ref.shadow_bytes == K * LD * 2
    loss = lib.op("sum_all", y)
    if opt_kind == "sgd":
        opt = lib.pg_sgd_new(C.byref(SgdCfg(0.05, 0.9, 0.0, 0.0, True)))
        assert lib.pg_sgd_add_param(opt, nw) == 0
    else:
        cfg = lib.pg_adam_cfg_default()
        cfg.lr = 0.05
        opt = lib.pg_adam_new(C.byref(cfg))
        assert lib.pg_adam_add_param(opt, nw) == 0
    lib.pg_backward(loss)
    (lib.pg_sgd_step if opt_kind == "sgd" else lib.pg_adam_step)(opt)
    w1 = lib.value(nw)
    assert not np.array_equal(w1, w)
    ref = _DataRef.from_address(lib.tinfo(lib.node(nw).value).data_ref)
    assert ref.shadow and not ref.shadow_stale and ref.shadow_cols == N and ref.shadow_ld == LD
    # decode the [64, 16] pitched copy through an identity GEMM
    e32 = lib.tensor(np.eye(LD, dtype=np.float32))
    te = lib._check(lib.pg_amd_tensor_to_dtype(e32, dt))
    tc = lib.pg_tensor_empty_dtype(F32, 2, (C.c_size_t * 2)(K, LD))
    lib.pg_gemm_ex(dt, K, LD, LD, ref.shadow, LD, lib.tinfo(te).dev, LD, lib.tinfo(tc).dev, LD)
    kept = lib.read(tc)
    assert np.array_equal(kept[:, :N].view(np.uint32), _decoded(oracle, dt, w1).view(np.uint32))
    assert np.all(kept[:, N:] == 0.0)
    # the next forward reads the kept copy: it equals the oracle's product
    y2 = lib._check(lib.pg_amd_ag_matmul16(x, nw, dt))
    want = oracle.gemm(dt, oracle.cast16(dt, lib.value(x)), oracle.cast16(dt, w1))
    assert rel_fro(lib.value(y2), want) <= 1e-5
    for t in (e32, te, tc):
        lib.pg_tensor_free(t)
    (lib.pg_sgd_free if opt_kind == "sgd" else lib.pg_adam_free)(opt)
    for n in (y2, loss, y, x, nw):
        lib.pg_node_free(n)
