"""Forward elementwise graphs through the device JIT (pg_jit_*).

tests/golden/jit_fwd.npz holds the graphs of the reference's test_jit.c and
jit_demo.c with their inputs, and what the reference's own JIT (C compiled
by the system compiler, jit.c:589-806) returned for them.  The device JIT
must return the same: bit for bit where the arithmetic is exact in f32
(add, sub, mul, neg, abs, relu, step, constants, broadcasts), within the
path's elementwise tolerance (max relative error 1e-5, oracle_lib.max_rel)
for the transcendental ops, and within a few ulps of the f64 value of the
mathematics on every op.
"""
from __future__ import annotations

import ctypes as C
import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle_lib import max_rel

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
with np.load(GOLDEN / "jit_fwd.npz", allow_pickle=False) as _z:
    G = {k: _z[k] for k in _z.files}
SPECS = {m["name"]: m for m in json.loads(str(G["specs"]))}

EXACT = {"basic", "bcast", "bcast3d", "unary_neg", "unary_abs", "unary_relu", "unary_step", "binary_add",
         "binary_sub", "binary_mul", "const", "multi"}
_erf = np.vectorize(math.erf, otypes=[np.float64])


def f64_eval(code, args):
    """The mathematics of each pg_jit op in f64 (jit.c:320-342 op_to_expr)."""
    a = [np.asarray(x, np.float64) for x in args]
    x = a[0]
    return {0: lambda: a[0] + a[1], 1: lambda: a[0] - a[1], 2: lambda: a[0] * a[1], 3: lambda: a[0] / a[1],
            4: lambda: -x, 5: lambda: np.exp(x), 6: lambda: np.log(x), 7: lambda: np.sqrt(x),
            8: lambda: np.sin(x), 9: lambda: np.cos(x), 10: lambda: np.abs(x), 11: lambda: np.maximum(x, 0),
            12: lambda: 1 / (1 + np.exp(-x)), 13: lambda: np.tanh(x),
            14: lambda: 0.5 * x * (1 + _erf(x / math.sqrt(2))), 15: lambda: _erf(x),
            16: lambda: (x > 0).astype(np.float64)}[code]()


def run_spec(lib, spec, inputs, single=False):
    """Builds the graph on the device library and runs it: pg_jit_run_single
    for one output when `single`, else pg_jit_run into zeroed outputs."""
    g = lib.pg_jit_graph_new()
    shapes = []
    for nd in spec["nodes"]:
        if nd[0] == "in":
            sh = (C.c_size_t * len(nd[1]))(*nd[1])
            assert lib.pg_jit_add_input(g, len(nd[1]), sh) >= 0
            shapes.append(tuple(nd[1]))
        elif nd[0] == "const":
            assert lib.pg_jit_add_const(g, nd[1]) >= 0
            shapes.append(())
        else:
            ids = (C.c_int * len(nd[2]))(*nd[2])
            assert lib.pg_jit_add_op(g, nd[1], ids, len(nd[2])) >= 0
            shapes.append(tuple(np.broadcast_shapes(*[shapes[i] for i in nd[2]])))
    for o in spec["outputs"]:
        lib.pg_jit_mark_output(g, o)
    exe = lib.pg_jit_compile(g)
    assert exe, lib.pg_jit_last_error()
    ts = [lib.tensor(x) for x in inputs]
    ins = (C.c_void_p * len(ts))(*ts)
    if single:
        outs = [lib.pg_jit_run_single(exe, ins, len(ts))]
        assert outs[0], lib.pg_jit_last_error()
    else:
        outs = [lib.tensor(np.zeros(shapes[o], np.float32)) for o in spec["outputs"]]
        assert lib.pg_jit_run(exe, ins, len(ts), (C.c_void_p * len(outs))(*outs), len(outs)), lib.pg_jit_last_error()
    res = [lib.read(t) for t in outs]
    for t in ts + outs:
        lib.pg_tensor_free(t)
    lib.pg_jit_exe_free(exe)
    lib.pg_jit_graph_free(g)
    return res


def f64_spec(spec, inputs):
    vals = []
    it = iter(inputs)
    for nd in spec["nodes"]:
        if nd[0] == "in":
            vals.append(np.asarray(next(it), np.float64))
        elif nd[0] == "const":
            vals.append(np.float64(np.float32(nd[1])))
        else:
            vals.append(f64_eval(nd[1], [vals[i] for i in nd[2]]))
    return [vals[o] for o in spec["outputs"]]


@pytest.mark.parametrize("name", sorted(SPECS))
def test_forward_graph_matches_reference(lib, name):
    spec = SPECS[name]
    inputs = [G[f"{name}_in{i}"] for i in range(spec["ninputs"])]
    got = run_spec(lib, spec, inputs, single=len(spec["outputs"]) == 1 and name != "basic")
    exact = f64_spec(spec, inputs)
    for k, y in enumerate(got):
        ref = G[f"{name}_out{k}"]
        assert y.shape == ref.shape
        if name in EXACT:
            assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), k
        else:
            assert max_rel(y, ref) <= 1e-5, (k, max_rel(y, ref))
        # against the mathematics: 4 ulps of f32 (relative 4.8e-7) above the
        # max_rel floor
        assert max_rel(y.astype(np.float64), exact[k]) <= 4.8e-7, (k, max_rel(y.astype(np.float64), exact[k]))


@pytest.mark.parametrize("shape", [(512, 512), (2048, 4096)])
def test_demo_chain_at_size(lib, oracle, shape):
    """jit_demo.c's (a+b)*c -> relu -> tanh (the reference benchmarks it at
    [64,64] and [512,512]) at larger sizes, inputs from the reference's RNG
    (seed 42, uniform(-1, 1)), against the f64 value."""
    spec = SPECS["demo64"]
    spec = dict(spec, nodes=[[n[0], list(shape)] if n[0] == "in" else n for n in spec["nodes"]])
    oracle.orc_seed(42)
    n = shape[0] * shape[1]
    inputs = [oracle.uniform(n, -1.0, 1.0).reshape(shape) for _ in range(3)]
    (y,) = run_spec(lib, spec, inputs, single=True)
    (ref,) = f64_spec(spec, inputs)
    assert max_rel(y.astype(np.float64), ref) <= 4.8e-7


def test_cache_and_run_errors(lib):
    """test_jit.c:228-292: a second compile of the same graph is a cache
    hit; a run with a wrong input shape fails."""
    g = lib.pg_jit_graph_new()
    sh = (C.c_size_t * 1)(4)
    a = lib.pg_jit_add_input(g, 1, sh)
    b = lib.pg_jit_add_input(g, 1, sh)
    lib.pg_jit_mark_output(g, lib.pg_jit_add(g, a, b))
    before = lib.pg_jit_cache_size()
    e1 = lib.pg_jit_compile(g)
    mid = lib.pg_jit_cache_size()
    e2 = lib.pg_jit_compile(g)
    assert e1 and e2 and mid <= before + 1 and lib.pg_jit_cache_size() == mid
    wrong = lib.tensor(np.zeros(5, np.float32))
    ok_in = lib.tensor(np.zeros(4, np.float32))
    out = lib.tensor(np.zeros(4, np.float32))
    assert not lib.pg_jit_run(e1, (C.c_void_p * 2)(wrong, ok_in), 2, (C.c_void_p * 1)(out), 1)
    for t in (wrong, ok_in, out):
        lib.pg_tensor_free(t)
    lib.pg_jit_exe_free(e1)
    lib.pg_jit_exe_free(e2)
    lib.pg_jit_graph_free(g)
