"""Bias grads of linear16 layers: each activation pass writes the row-block
partials of its bias grad, and the last step (adding them per column, the
row blocks in order) runs in the NEXT activation pass's launch, or at the
end of the backward walk, or before that grad is taken for writing again.
Where it runs must not change a bit:
  - a chain of layers: every bias grad equals the f64 column sums of the
    layer's f32 dz (the oracle's dout * gelu'(z) on the device's own dout
    and pre-activation; the seed for the last, linear layer), within the
    f32 summation bound, and a repeat of the backward reproduces every bit;
  - one bias shared by two layers: its grad is the first layer's sums,
    then the second's added to them (the second pass takes the grad for
    writing, which runs the first's deferred sums before it), so it equals,
    bit for bit, the f32 sum of the two grads of the same graph with two
    separate biases of the same values.
"""
import numpy as np
import pytest

from picograd_amd.capi import BF16
from test_gpu_parity import dbias_bound

pytestmark = pytest.mark.gpu

GELU, NONE = 2, 0


def test_chain_bias_grads(lib, oracle):
    """Three GELU layers and a linear one: four bias grads, three of them
    finished by the next layer's activation pass, the last by the walk."""
    print("bias sums: chain", flush=True)
    rng = np.random.default_rng(71)
    M, widths = 1537, [96, 512, 384, 640, 200]
    x = rng.standard_normal((M, widths[0])).astype(np.float32)
    ws = [(rng.standard_normal((a, b)) / np.sqrt(a)).astype(np.float32) for a, b in zip(widths, widths[1:])]
    bs = [(0.1 * rng.standard_normal(b)).astype(np.float32) for b in widths[1:]]
    g = rng.standard_normal((M, widths[-1])).astype(np.float32)
    runs = []
    for _ in range(2):
        nodes = [lib.var(x)]
        params = []
        h = nodes[0]
        for i, (w, b) in enumerate(zip(ws, bs)):
            nw, nb = lib.var(w), lib.var(b)
            params += [nw, nb]
            h = lib._check(lib.pg_amd_ag_linear16(h, nw, nb, NONE if i == len(ws) - 1 else GELU, BF16))
            nodes.append(h)
        seed = lib.tensor(g)
        lib.pg_amd_backward_from(h, seed)
        dbs = [lib.grad(nb).copy() for nb in params[1::2]]
        dzs = [oracle.gelu_backward(lib.read(lib.pg_amd_linear16_preact(n)), lib.grad(n))
               for n in nodes[1:-1]] + [g]
        runs.append(dbs)
        for i, (db, dz) in enumerate(zip(dbs, dzs)):
            bad = np.abs(db - dz.astype(np.float64).sum(axis=0)) > dbias_bound(dz, 128)
            assert not bad.any(), f"layer {i}: {int(bad.sum())} bias grad columns off"
        lib.pg_tensor_free(seed)
        for n in nodes[::-1] + params:
            lib.pg_node_free(n)
    for a, b in zip(*runs):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "bias grads differ between repeats"


def _two_layers(lib, x, w1, w2, b1, b2, g, shared):
    nx, n1, n2 = lib.var(x), lib.var(w1), lib.var(w2)
    nb1 = lib.var(b1)
    nb2 = nb1 if shared else lib.var(b2)
    h = lib._check(lib.pg_amd_ag_linear16(nx, n1, nb1, GELU, BF16))
    out = lib._check(lib.pg_amd_ag_linear16(h, n2, nb2, NONE, BF16))
    seed = lib.tensor(g)
    lib.pg_amd_backward_from(out, seed)
    res = [lib.grad(nb1).copy()] + ([] if shared else [lib.grad(nb2).copy()])
    lib.pg_tensor_free(seed)
    for n in [out, h, nx, n1, n2, nb1] + ([] if shared else [nb2]):
        lib.pg_node_free(n)
    return res


def test_shared_bias(lib):
    """db of a bias used by two layers = f32 sum of the two separate grads:
    the out layer's sums (deferred, then run when the first layer's pass
    takes the grad for writing) plus the first layer's."""
    print("bias sums: shared bias", flush=True)
    rng = np.random.default_rng(72)
    M, K, H = 2049, 128, 384
    x = rng.standard_normal((M, K)).astype(np.float32)
    w1 = (rng.standard_normal((K, H)) / np.sqrt(K)).astype(np.float32)
    w2 = (rng.standard_normal((H, H)) / np.sqrt(H)).astype(np.float32)
    b = (0.1 * rng.standard_normal(H)).astype(np.float32)
    g = rng.standard_normal((M, H)).astype(np.float32)
    db1, db2 = _two_layers(lib, x, w1, w2, b, b, g, shared=False)
    (db,) = _two_layers(lib, x, w1, w2, b, b, g, shared=True)
    # the out layer's grad is written first (beta 0), the first layer's added
    want = (db2 + db1).astype(np.float32)
    assert np.array_equal(db.view(np.uint32), want.view(np.uint32))
