"""pg_amd_gemm_ex_noalloc against pg_gemm_ex, through the C ABI.

The no-alloc entry point runs pg_gemm_ex's kernels with its buffers taken
from a fixed per-device workspace, so on the same inputs it must write the
same bits.  Two calls in a row, the second with a smaller input (the
workspace keeps the first call's contents), each checked against
pg_gemm_ex and against the f32-accumulating oracle; the library's allocator
must see no allocation during the calls; a GEMM whose split-K partials need
more than the workspace is refused with an error and leaves C untouched.
"""
import ctypes as C

import numpy as np
import pytest

from oracle_lib import rel_fro
from picograd_amd.capi import BF16, F16, F32

pytestmark = pytest.mark.gpu


def _shape(*s):
    return len(s), (C.c_size_t * len(s))(*s)


class _Case:
    def __init__(self, lib, oracle, dt, m, n, k, seed):
        rng = np.random.default_rng(seed)
        self.m, self.n, self.k, self.dt = m, n, k, dt
        self.a16 = oracle.cast16(dt, rng.standard_normal((m, k)).astype(np.float32))
        self.b16 = oracle.cast16(dt, rng.standard_normal((k, n)).astype(np.float32))
        self.ta, self.tb = lib.tensor(self.a16, dt), lib.tensor(self.b16, dt)
        nd, sh = _shape(m, n)
        self.c_ref = lib.pg_tensor_empty_dtype(F32, nd, sh)
        self.c_new = lib.pg_tensor_full(nd, sh, 7.0)

    def run_ref(self, lib):
        ti = lib.tinfo
        lib.pg_gemm_ex(self.dt, self.m, self.n, self.k, ti(self.ta).dev, self.k, ti(self.tb).dev, self.n,
                       ti(self.c_ref).dev, self.n)

    def run_new(self, lib):
        ti = lib.tinfo
        return lib.pg_amd_gemm_ex_noalloc(self.dt, self.m, self.n, self.k, ti(self.ta).dev, self.k,
                                          ti(self.tb).dev, self.n, ti(self.c_new).dev, self.n)

    def free(self, lib):
        for t in (self.ta, self.tb, self.c_ref, self.c_new):
            lib.pg_tensor_free(t)


def test_noalloc_gemm_matches_pg_gemm_ex_twice(lib, oracle):
    # call 1: bf16, operands read in place, split-K partials in the
    # workspace; call 2: smaller, n % 8 != 0 so both operands are padded into
    # the workspace, with split-K partials behind them
    cases = [_Case(lib, oracle, BF16, 2048, 40, 4096, 1), _Case(lib, oracle, BF16, 1000, 10, 2048, 2)]
    for cs in cases:
        cs.run_ref(lib)
    lib.sync()
    used, cached = lib.pg_amd_bytes_in_use(), lib.pg_amd_bytes_cached()
    for i, cs in enumerate(cases):
        print(f"no-alloc gemm call {i + 1}: dt={cs.dt} m={cs.m} n={cs.n} k={cs.k}", flush=True)
        assert cs.run_new(lib) == 0, lib.pg_amd_last_error().decode()
    lib.sync()
    assert (lib.pg_amd_bytes_in_use(), lib.pg_amd_bytes_cached()) == (used, cached)
    for cs in cases:
        got, want = lib.read(cs.c_new), lib.read(cs.c_ref)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        ref = oracle.gemm(cs.dt, cs.a16, cs.b16, threads=16)
        assert rel_fro(got, ref) <= 1e-5
        cs.free(lib)


@pytest.mark.parametrize("dt,m,n,k", [(F16, 300, 64, 1000), (F16, 77, 33, 1003), (F32, 65, 70, 90),
                                      (BF16, 129, 96, 40)])
def test_noalloc_gemm_other_shapes(lib, oracle, dt, m, n, k):
    """f16, a ragged k (the padded path), the f32 kernel, and a GEMM too
    small to split, each bit for bit against pg_gemm_ex."""
    print(f"no-alloc gemm dt={dt} m={m} n={n} k={k}", flush=True)
    if dt == F32:
        rng = np.random.default_rng(m + n + k)
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        ta, tb = lib.tensor(a), lib.tensor(b)
        nd, sh = _shape(m, n)
        c1, c2 = lib.pg_tensor_empty_dtype(F32, nd, sh), lib.pg_tensor_empty_dtype(F32, nd, sh)
        ti = lib.tinfo
        lib.pg_gemm_ex(F32, m, n, k, ti(ta).dev, k, ti(tb).dev, n, ti(c1).dev, n)
        assert lib.pg_amd_gemm_ex_noalloc(F32, m, n, k, ti(ta).dev, k, ti(tb).dev, n, ti(c2).dev, n) == 0
        assert np.array_equal(lib.read(c1), lib.read(c2))
        for t in (ta, tb, c1, c2):
            lib.pg_tensor_free(t)
        return
    cs = _Case(lib, oracle, dt, m, n, k, m * n)
    cs.run_ref(lib)
    assert cs.run_new(lib) == 0, lib.pg_amd_last_error().decode()
    got, want = lib.read(cs.c_new), lib.read(cs.c_ref)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert rel_fro(got, oracle.gemm(dt, cs.a16, cs.b16)) <= 1e-5
    cs.free(lib)


def test_noalloc_gemm_refuses_beyond_the_workspace(lib):
    """2048 x 2048 x 16384 splits its reduction in four: 64 MiB of
    partials, above the 32 MiB workspace.  The call is refused and C is not
    written."""
    m, n, k = 2048, 2048, 16384
    sp = C.c_int(0)
    lib.pg_amd_gemm16_plan(0, 1, m, n, k, 1, 0, C.byref(sp), None)
    assert sp.value * m * n * 4 > (32 << 20), "the planner no longer splits this shape"
    print(f"no-alloc gemm refusal m={m} n={n} k={k}", flush=True)
    nd, sh = _shape(m, k)
    ta = lib.pg_tensor_full_dtype(BF16, nd, sh, 1.0)
    nd, sh = _shape(k, n)
    tb = lib.pg_tensor_full_dtype(BF16, nd, sh, 1.0)
    nd, sh = _shape(m, n)
    tc = lib.pg_tensor_full(nd, sh, 3.0)
    ti = lib.tinfo
    rc = lib.pg_amd_gemm_ex_noalloc(BF16, m, n, k, ti(ta).dev, k, ti(tb).dev, n, ti(tc).dev, n)
    assert rc == -1
    msg = lib.pg_amd_last_error().decode()
    assert "no-alloc maximum" in msg and str(32 << 20) in msg, msg
    assert np.all(lib.read(tc) == 3.0)
    # bad arguments are refused before anything is queued
    assert lib.pg_amd_gemm_ex_noalloc(BF16, m, n, k, None, k, ti(tb).dev, n, ti(tc).dev, n) == -1
    assert lib.pg_amd_gemm_ex_noalloc(7, m, n, k, ti(ta).dev, k, ti(tb).dev, n, ti(tc).dev, n) == -1
    for t in (ta, tb, tc):
        lib.pg_tensor_free(t)


def test_noalloc_gemm_refuses_pending_work(lib, oracle):
    """With an upload still waiting to be queued (a leaf made from host
    data), the call is refused instead of queueing it (which may wait on a
    staging slot); after pg_amd_sync() the same call runs and matches
    pg_gemm_ex bit for bit."""
    print("no-alloc gemm with a pending upload", flush=True)
    cs = _Case(lib, oracle, BF16, 256, 64, 512, 7)
    cs.run_ref(lib)
    lib.sync()
    pending = lib.tensor(np.ones((64, 64), np.float32))  # a small upload: batched, not yet queued
    assert cs.run_new(lib) == -1
    assert "pending" in lib.pg_amd_last_error().decode()
    assert np.all(lib.read(cs.c_new) == 7.0)  # C untouched (the read queues the upload)
    lib.sync()
    assert cs.run_new(lib) == 0, lib.pg_amd_last_error().decode()
    assert np.array_equal(lib.read(cs.c_new).view(np.uint32), lib.read(cs.c_ref).view(np.uint32))
    assert np.all(lib.read(pending) == 1.0)
    lib.pg_tensor_free(pending)
    cs.free(lib)
