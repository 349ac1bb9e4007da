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
