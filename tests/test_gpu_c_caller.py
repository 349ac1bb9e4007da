"""The reference-style C caller (tests/c_callers/xor_jit_ops.c) run on the
MI355X: test_jit.c's fused-vs-eager checks and known answers,
train_xor_jit.c's XOR training and eager-vs-JIT inference, and the tensor
utilities, all through the C ABI from a C program linked against
include/picograd and libpicograd_amd.so."""
import subprocess

import pytest

from picograd_amd.build import C_CALLERS, build_c_callers

pytestmark = pytest.mark.gpu


def test_c_caller_runs_clean():
    exe = C_CALLERS / "bin" / "xor_jit_ops"
    if not exe.exists():
        build_c_callers()
    print(f"running {exe}", flush=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "0 failed" in res.stdout and "FAIL" not in res.stdout


def test_chain_loop_c_program():
    """Config 1's timed C loop (tests/c_callers/chain_loop.c) over this
    build: 500 iterations with the JIT on and off, the last iteration's
    grads against the chain rule in double precision (the program's exit
    status)."""
    import json
    from picograd_amd.capi import _DEFAULT_LIB
    exe = C_CALLERS / "bin" / "chain_loop"
    if not exe.exists():
        build_c_callers()
    for jit in ("1", "0"):
        print(f"running {exe} jit={jit}", flush=True)
        res = subprocess.run([str(exe), str(_DEFAULT_LIB), "500", jit], capture_output=True, text=True, timeout=120)
        assert res.returncode == 0, res.stdout + res.stderr
        out = json.loads(res.stdout.strip().splitlines()[-1])
        assert out["iters"] == 500 and out["max_err"] <= 1e-5 and out["us_per_iter"] > 0
