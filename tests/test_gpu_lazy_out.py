"""A linear16 layer's output written only when something reads it.

With grads enabled and an activation, the layer's GEMM writes the kept
pre-activation z and out's 16-bit copy but not out's f32 elements; they are
pending as act(z) and written by one pass with the epilogue's arithmetic
when first read (the next layer reads the 16-bit copy, the backward reads
z, so in training they are never written).  Every way of reading out must
give the bits the GEMM epilogue writes when it does write out (grads off:
no z is kept, so out is written at once), and a write of the whole of out
must drop the pending state.
"""
import ctypes as C

import numpy as np
import pytest

from picograd_amd.capi import BF16, F16

pytestmark = pytest.mark.gpu

ACT_RELU, ACT_GELU = 1, 2


def _layer(lib, x, w, b, act, dt, grad):
    if not grad:
        lib.pg_no_grad_push()
    try:
        nx, nw, nb = lib.var(x), lib.var(w), lib.var(b)
        out = lib._check(lib.pg_amd_ag_linear16(nx, nw, nb, act, dt))
    finally:
        if not grad:
            lib.pg_no_grad_pop()
    return out, (nx, nw, nb)


@pytest.mark.parametrize("act", [ACT_RELU, ACT_GELU])
@pytest.mark.parametrize("dt", [BF16, F16])
def test_pending_output_equals_the_written_one(lib, act, dt):
    print(f"lazy linear16 output act={act} dt={dt}", flush=True)
    rng = np.random.default_rng(act * 10 + dt)
    x = rng.standard_normal((300, 256)).astype(np.float32)
    w = (rng.standard_normal((256, 512)) / 16).astype(np.float32)
    b = (0.1 * rng.standard_normal(512)).astype(np.float32)
    eager, leaves_e = _layer(lib, x, w, b, act, dt, grad=False)
    want = lib.value(eager)
    lazy, leaves_l = _layer(lib, x, w, b, act, dt, grad=True)
    assert lib.pg_amd_linear16_preact(lazy)  # z kept: out is pending
    got = lib.value(lazy)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # a second layer reads the first's 16-bit copy: the same bits either way
    w2 = (rng.standard_normal((512, 64)) / 16).astype(np.float32)
    nw2 = lib.var(w2)
    y_e = lib._check(lib.pg_amd_ag_linear16(eager, nw2, None, 0, dt))
    lazy2, leaves_l2 = _layer(lib, x, w, b, act, dt, grad=True)
    y_l = lib._check(lib.pg_amd_ag_linear16(lazy2, nw2, None, 0, dt))
    assert np.array_equal(lib.value(y_l).view(np.uint32), lib.value(y_e).view(np.uint32))
    assert np.array_equal(lib.value(lazy2).view(np.uint32), want.view(np.uint32))
    for n in (y_l, y_e, nw2, lazy2, *leaves_l2, lazy, *leaves_l, eager, *leaves_e):
        lib.pg_node_free(n)


def test_pending_output_outlives_its_node_and_is_dropped_by_a_write(lib):
    """A view of the output read after the layer's node (and with it z) was
    freed still reads act(z): the pending state holds z's storage.  A fill
    of the whole output drops the pending state instead of applying it."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((128, 64)).astype(np.float32)
    w = (rng.standard_normal((64, 96)) / 8).astype(np.float32)
    b = np.zeros(96, np.float32)
    eager, leaves_e = _layer(lib, x, w, b, ACT_GELU, BF16, grad=False)
    want = lib.value(eager)
    lazy, leaves_l = _layer(lib, x, w, b, ACT_GELU, BF16, grad=True)
    lib.lib.pg_tensor_view.restype = C.c_void_p
    lib.lib.pg_tensor_view.argtypes = [C.c_void_p]
    view = lib.lib.pg_tensor_view(lib.node(lazy).value)
    assert view
    lib.pg_node_free(lazy)  # frees the node's value tensor and its z
    assert np.array_equal(lib.read(view).view(np.uint32), want.view(np.uint32))
    lib.pg_tensor_free(view)
    lazy2, leaves_l2 = _layer(lib, x, w, b, ACT_GELU, BF16, grad=True)
    lib.pg_tensor_fill(lib.node(lazy2).value, 3.0)
    assert np.all(lib.value(lazy2) == 3.0)
    for n in (lazy2, *leaves_l2, *leaves_l, eager, *leaves_e):
        lib.pg_node_free(n)
