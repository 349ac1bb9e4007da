"""The JIT's compile-failure path through pg_backward (the reference's
autograd.c:2514-2519: when the fused suffix cannot be compiled, the backward
falls back to the eager per-node path, counts a fallback, records the error,
and still produces the grads).

PG_JIT_FORCE_COMPILE_ERROR=1 makes every hiprtc compile fail.  It runs in a
fresh process with an empty code-object cache directory, so no kernel is
loaded from memory or disk: configs 1 and 2 (at reduced size) go through
pg_backward there, and the grads it writes come back here to be checked
against the oracle at the north star's 1e-5.
"""
import json
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from oracle_lib import max_rel
from test_gpu_parity import dbias_bound

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent

CHILD = r'''
import json, sys
import numpy as np
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[1] + "/tests")
import picograd_amd
from oracle_lib import Oracle
L = picograd_amd.load()
assert L.pg_amd_init() == 0, L.pg_amd_last_error().decode()
o = Oracle()
out, res = {}, {}
fb0, hit0 = L.pg_autograd_jit_fallbacks(), L.pg_autograd_jit_hits()
# config 1 chain
o.orc_seed(42)
a, b, c = (o.uniform(4096, -1.0, 1.0).reshape(64, 64) for _ in range(3))
na, nb, nc = L.var(a), L.var(b), L.var(c)
t0 = L.op("add", na, nb); t1 = L.op("mul", t0, nc); t2 = L.op("relu", t1); t3 = L.op("tanh", t2)
loss = L.op("sum_all", t3)
L.pg_backward(loss)
res["c1_was_jit"] = bool(L.pg_autograd_last_was_jit())
res["c1_error"] = L.pg_autograd_last_error().decode()
res["jit_error"] = L.pg_jit_last_error().decode()
for k, n in (("da", na), ("db", nb), ("dc", nc)):
    out[k] = L.grad(n)
for n in (loss, t3, t2, t1, t0, na, nb, nc):
    L.pg_node_free(n)
res["fallbacks_after_c1"] = L.pg_autograd_jit_fallbacks() - fb0
# config 2 chain with the broadcast bias
o.orc_seed(43)
R, C = 300, 520
x = o.normal(R * C, 0.0, 1.0).reshape(R, C); bias = o.normal(C, 0.0, 0.1); g = o.normal(R * C, 0.0, 1.0).reshape(R, C)
nx, nbias, ng = L.var(x), L.var(bias), L.var(g)
t0 = L.op("add", nx, nbias); t1 = L.op("gelu", t0); t2 = L.op("sigmoid", ng); y = L.op("mul", t1, t2)
loss = L.op("sum_all", y)
L.pg_backward(loss)
res["c2_was_jit"] = bool(L.pg_autograd_last_was_jit())
for k, n in (("dx", nx), ("dg", ng), ("dbias", nbias)):
    out[k] = L.grad(n)
for n in (loss, y, t2, t1, t0, nx, nbias, ng):
    L.pg_node_free(n)
res["fallbacks"] = L.pg_autograd_jit_fallbacks() - fb0
res["hits"] = L.pg_autograd_jit_hits() - hit0
res["compiles"] = L.pg_amd_jit_compiles()
np.savez(sys.argv[2], **out)
print(json.dumps(res), flush=True)
'''


def test_compile_failure_falls_back_to_eager_with_correct_grads(oracle, tmp_path):
    env = dict(os.environ, PG_JIT_FORCE_COMPILE_ERROR="1", PG_JIT_CACHE_DIR=str(tmp_path / "jitcache"))
    npz = tmp_path / "grads.npz"
    print("jit fallback child: PG_JIT_FORCE_COMPILE_ERROR=1, fresh cache", flush=True)
    res = subprocess.run([sys.executable, "-c", CHILD, str(ROOT), str(npz)], env=env, capture_output=True,
                         text=True, timeout=180)
    assert res.returncode == 0, res.stdout + res.stderr
    info = json.loads(res.stdout.strip().splitlines()[-1])
    print(info)
    # both backwards fell back: not JIT, counted, with the compile error kept
    assert info["c1_was_jit"] is False and info["c2_was_jit"] is False
    assert info["fallbacks_after_c1"] == 1 and info["fallbacks"] == 2 and info["hits"] == 0
    assert info["jit_error"], "the JIT's last error should name the failed compile"
    assert info["compiles"] == 0
    with np.load(npz, allow_pickle=False) as z:
        got = {k: z[k] for k in z.files}
    oracle.orc_seed(42)
    a, b, c = (oracle.uniform(4096, -1.0, 1.0) for _ in range(3))
    rda, rdb, rdc = oracle.chain1(a, b, c)
    for k, r in (("da", rda), ("db", rdb), ("dc", rdc)):
        assert max_rel(got[k].ravel(), r) <= 1e-5, k
    oracle.orc_seed(43)
    R, Cc = 300, 520
    x = oracle.normal(R * Cc, 0.0, 1.0).reshape(R, Cc)
    bias = oracle.normal(Cc, 0.0, 0.1)
    g = oracle.normal(R * Cc, 0.0, 1.0).reshape(R, Cc)
    rdx, rdg, _, rdb64 = oracle.chain2(x, bias, g)
    assert max_rel(got["dx"], rdx) <= 1e-5 and max_rel(got["dg"], rdg) <= 1e-5
    # the eager path sums dbias serially over the rows, as the reference does
    assert np.all(np.abs(got["dbias"] - rdb64) <= dbias_bound(rdx, R))
