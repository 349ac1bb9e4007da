"""16-bit operand copies written by the fused elementwise kernels
(pg_amd_jit_copies16): a deferred forward run whose output a matmul16 node
takes as its operand stores that output's f16/bf16 copy beside its f32
elements, and a fused backward region that writes a matmul16 node's grad
whole stores the grad's copy; the matmul16 forward and backward read those
copies instead of running a cast pass.  Each copy must be what the cast
kernel (k_cast_to16, the rounding held to the reference's convert.h by
test_gpu_convert.py) makes of the same f32 values, so every result is the
same bit for bit with the copies on and off, for NaN, infinities, f32 and
f16 subnormals, rounding halfway cases and f16 overflow alike; and with an
identity weight the product is the copy itself.  A grad the region wrote
and a later GEMM then accumulated into is read through a fresh cast.
"""
import numpy as np
import pytest

from oracle_lib import bf16_to_f32, f16_to_f32
from picograd_amd.capi import BF16, F16

pytestmark = pytest.mark.gpu


def bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def _specials(rng, shape, finite_only):
    """Normal values with edge cases planted: f32 and f16 subnormals, bf16
    and f16 rounding halfway points (both parities), values past f16's
    range, signed zeros, and (unless finite_only) NaNs and infinities."""
    x = rng.standard_normal(shape).astype(np.float32)
    flat = x.reshape(-1)
    u = flat.view(np.uint32)
    n = flat.size
    idx = rng.permutation(n)
    k = 0

    def plant(vals):
        nonlocal k
        for v in vals:
            flat[idx[k]] = v
            k += 1

    plant([1e-40, -3e-42, 1.5e-45, 6e-8, -5.9e-8, 3e-5, -6.1e-5, 0.0, -0.0])
    # bf16 halfway: low 16 bits exactly 0x8000, even and odd upper halves
    for hi in (0x3F80, 0x3F81, 0xBF82, 0x4003, 0x0001):
        flat[idx[k]] = np.array([(hi << 16) | 0x8000], np.uint32).view(np.float32)[0]
        k += 1
    # f16 halfway: 1 + 2^-11 (ties to even: 1.0), 1 + 3 * 2^-11 (to 1 + 2^-9)
    plant([1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, -(2.0 + 2.0 ** -10)])
    if not finite_only:
        plant([70000.0, -1e6, 65520.0, np.inf, -np.inf, np.nan])
        u[idx[k]] = 0x7F800001  # signalling-pattern NaN
        k += 1
    return x


@pytest.mark.parametrize("dt", [BF16, F16])
@pytest.mark.parametrize("chain", ["add", "gelu"])
def test_forward_copy_same_bits(lib, dt, chain):
    """c = matmul16(op(x + b), W) with the run's copy and with the cast."""
    print(f"jit16 forward dt={dt} chain={chain}", flush=True)
    rng = np.random.default_rng(11 + dt)
    M, K, N = 1024, 512, 256
    x = _specials(rng, (M, K), finite_only=False)
    b = (0.1 * rng.standard_normal(K)).astype(np.float32)
    w = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    out = {}
    for on in (True, False):
        lib.pg_amd_jit_copies16(on)
        try:
            nx, nb, nw = lib.var(x, requires_grad=False), lib.var(b, requires_grad=False), lib.var(w)
            s = lib.op("add", nx, nb)
            h = lib.op("gelu", s) if chain == "gelu" else s
            c = lib._check(lib.pg_amd_ag_matmul16(h, nw, dt))
            out[on] = lib.value(c)
            nodes = [c, h] + ([s] if chain == "gelu" else []) + [nw, nb, nx]
            for n in nodes:
                lib.pg_node_free(n)
        finally:
            lib.pg_amd_jit_copies16(True)
    assert np.array_equal(bits(out[True]), bits(out[False])), f"dt={dt} {chain}: results differ"


@pytest.mark.parametrize("dt", [BF16, F16])
def test_forward_copy_is_the_cast(lib, dt):
    """With W the identity, matmul16(x + b, W) is the run output's 16-bit
    copy, element by element: equal to the cast kernel's rounding of the
    run's f32 output (finite values: a NaN or infinity would spread over
    the row through the products with zeros).  Normal values bit for bit; a
    16-bit subnormal may reach the product flushed to zero by the matrix
    unit (the same with the cast's copy: the test above)."""
    print(f"jit16 identity dt={dt}", flush=True)
    rng = np.random.default_rng(29 + dt)
    M, K = 1024, 256
    x = _specials(rng, (M, K), finite_only=True)
    b = np.zeros(K, np.float32)
    nx, nb, nw = lib.var(x, requires_grad=False), lib.var(b, requires_grad=False), lib.var(np.eye(K, dtype=np.float32))
    s = lib.op("add", nx, nb)
    c = lib._check(lib.pg_amd_ag_matmul16(s, nw, dt))
    got = lib.value(c)
    t16 = lib.pg_amd_tensor_to_dtype(lib.node(s).value, dt)
    assert t16
    h = lib.read(t16)
    lib.pg_tensor_free(t16)
    want = f16_to_f32(h) if dt == F16 else bf16_to_f32(h)
    tiny = 2.0 ** -14 if dt == F16 else 2.0 ** -126
    normal = np.abs(want) >= tiny
    ok = np.where(normal, bits(got) == bits(want), (got == want) | (got == 0))
    bad = np.argwhere(~ok)
    assert bad.size == 0, [(tuple(i), float(want[tuple(i)]), float(got[tuple(i)])) for i in bad[:8]]
    for n in (c, s, nw, nb, nx):
        lib.pg_node_free(n)


def _mlp_grads(lib, dt, x, w1, b1, w2, g, shared):
    """y = matmul16(gelu(matmul16(x, W1) + b1), W2), loss = sum(y * g); with
    `shared`, z = matmul16(x, W1) also feeds a second matmul16 whose output
    joins the loss, so z's grad is written by the fused region and by a
    GEMM.  Returns the leaves' grads."""
    leaves = [lib.var(x), lib.var(w1), lib.var(b1), lib.var(w2)]
    nx, n1, nb, n2 = leaves
    ng = lib.var(g, requires_grad=False)
    made = [ng]
    z = lib._check(lib.pg_amd_ag_matmul16(nx, n1, dt))
    made.append(z)
    made.append(lib.op("add", z, nb))
    made.append(lib.op("gelu", made[-1]))
    made.append(lib._check(lib.pg_amd_ag_matmul16(made[-1], n2, dt)))
    made.append(lib.op("mul", made[-1], ng))
    made.append(lib.op("sum_all", made[-1]))
    loss = made[-1]
    if shared:
        made.append(lib._check(lib.pg_amd_ag_matmul16(z, n2, dt)))
        made.append(lib.op("mul", made[-1], ng))
        made.append(lib.op("sum_all", made[-1]))
        made.append(lib.op("add", loss, made[-1]))
        loss = made[-1]
    lib.pg_backward(loss)
    grads = [lib.grad(n).copy() for n in leaves]
    for n in made[::-1] + leaves[::-1]:
        lib.pg_node_free(n)
    return grads


@pytest.mark.parametrize("dt", [BF16, F16])
@pytest.mark.parametrize("shared", [False, True], ids=["one-consumer", "region-and-gemm"])
def test_backward_copy_same_bits(lib, dt, shared):
    """Every leaf grad of the two-layer graph is the same bit for bit with
    the region's copy of the first matmul16's grad and with the cast."""
    print(f"jit16 backward dt={dt} shared={shared}", flush=True)
    rng = np.random.default_rng(41 + dt + 2 * shared)
    M, K, H, N = 1024, 256, 512, 512 if shared else 128
    x = rng.standard_normal((M, K)).astype(np.float32)
    w1 = (rng.standard_normal((K, H)) / np.sqrt(K)).astype(np.float32)
    b1 = (0.1 * rng.standard_normal(H)).astype(np.float32)
    if shared:  # z [M, H] also goes through W2 [H, N] with N == H
        w2 = (rng.standard_normal((H, H)) / np.sqrt(H)).astype(np.float32)
        g = rng.standard_normal((M, H)).astype(np.float32)
    else:
        w2 = (rng.standard_normal((H, N)) / np.sqrt(H)).astype(np.float32)
        g = rng.standard_normal((M, N)).astype(np.float32)
    res = {}
    for on in (True, False):
        lib.pg_amd_jit_copies16(on)
        try:
            res[on] = _mlp_grads(lib, dt, x, w1, b1, w2, g, shared)
        finally:
            lib.pg_amd_jit_copies16(True)
    for name, a, b in zip(("dx", "dW1", "db1", "dW2"), res[True], res[False]):
        assert np.array_equal(bits(a), bits(b)), f"{name} differs (dt={dt}, shared={shared})"
