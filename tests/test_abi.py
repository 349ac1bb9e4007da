"""The C-ABI library on the CPU: it loads, exports every function the public
headers declare, links nothing of the oracle, and its host-only logic
(JIT graph building, hashing, codegen + hiprtc compile) works without a
GPU.  No test here launches device work."""
from __future__ import annotations

import ctypes as C
import os
import re
import subprocess
from pathlib import Path

import pytest

import picograd_amd
from picograd_amd.capi import shape_arg

ROOT = Path(__file__).resolve().parent.parent
INCLUDE = ROOT / "include" / "picograd"
LIB = ROOT / "picograd_amd" / "lib" / "libpicograd_amd.so"

_DECL = re.compile(r"^(?!\s*(?:static|typedef|#|\*|/))[A-Za-z_][\w\s\*]*?\b(pg_\w+)\s*\(", re.M)


def declared_functions() -> dict[str, list[str]]:
    out = {}
    for h in sorted(INCLUDE.glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        names = sorted(set(_DECL.findall(text)))
        out[h.name] = names
    return out


def test_headers_declare_the_reference_abi():
    decl = declared_functions()
    every = {n for v in decl.values() for n in v}
    # the reference entry points the drop-in must keep (autograd.h, jit.h,
    # sgd.h, backend.h, tensor.h of the reference)
    for name in ("pg_backward", "pg_backward_jit", "pg_ag_add", "pg_ag_matmul", "pg_ag_mse", "pg_ag_gelu",
                 "pg_jit_compile", "pg_jit_run", "pg_jit_run_single", "pg_jit_graph_hash",
                 "pg_sgd_new", "pg_sgd_step", "pg_sgd_zero_grad", "pg_gemm", "pg_gemm_ex", "pg_hgemm",
                 "pg_bgemm", "pg_seed", "pg_tensor_uniform", "pg_tensor_normal", "pg_var_from_data"):
        assert name in every, name
    assert len(every) > 100


def test_library_exports_every_declared_function():
    lib = C.CDLL(str(LIB))
    missing = [(h, n) for h, names in declared_functions().items() for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_library_does_not_link_the_oracle():
    syms = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], capture_output=True, text=True,
                          check=True).stdout
    assert "orc_" not in syms
    deps = subprocess.run(["ldd", str(LIB)], capture_output=True, text=True).stdout
    assert "oracle" not in deps and "picograd_ref" not in deps
    assert "libamdhip64" in deps and "libhiprtc" in deps


def test_kernels_are_built_for_gfx950_only(tmp_path):
    """The fat binary embedded in the library carries gfx950 code objects
    and no other GPU target."""
    fatbin = tmp_path / "fatbin"
    r = subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", str(LIB), str(fatbin)],
                       capture_output=True, text=True)
    if r.returncode != 0 or not fatbin.exists():
        pytest.skip("objcopy unavailable")
    data = fatbin.read_bytes()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx\w+)", data))
    assert targets == {b"gfx950"}, targets


@pytest.fixture(scope="module")
def host_lib(tmp_path_factory):
    os.environ["PG_JIT_CACHE_DIR"] = str(tmp_path_factory.mktemp("jitcache"))
    return picograd_amd.load()


def _graph(L, build):
    g = L.pg_jit_graph_new()
    out = build(g)
    if out is not None:
        L.pg_jit_mark_output(g, out)
    return g


def test_jit_graph_building_and_errors(host_lib):
    """test_jit.c:270-296: invalid ids fail with -1, a graph without
    outputs does not compile, broadcasting follows numpy rules."""
    L = host_lib
    g = L.pg_jit_graph_new()
    assert L.pg_jit_add(g, 999, 1000) == -1
    assert L.pg_jit_compile(g) is None
    a = L.pg_jit_add_input(g, *shape_arg((2, 4)))
    b = L.pg_jit_add_input(g, *shape_arg((4,)))
    c = L.pg_jit_add_input(g, *shape_arg((3,)))
    assert L.pg_jit_add(g, a, b) >= 0
    assert L.pg_jit_add(g, a, c) == -1  # 4 vs 3 does not broadcast
    assert L.pg_jit_num_inputs(g) == 3 and L.pg_jit_num_nodes(g) == 4
    ins = (C.c_int * 1)(a)
    assert L.pg_jit_add_op(g, 0, ins, 1) == -1  # binary op with one input
    L.pg_jit_graph_free(g)


def test_jit_hash_is_structural(host_lib):
    L = host_lib

    def build(shape, op):
        def f(g):
            a = L.pg_jit_add_input(g, *shape_arg(shape))
            b = L.pg_jit_add_input(g, *shape_arg(shape))
            return op(g, a, b)
        return f
    g1 = _graph(L, build((4, 4), L.pg_jit_add))
    g2 = _graph(L, build((4, 4), L.pg_jit_add))
    g3 = _graph(L, build((4, 4), L.pg_jit_mul))
    g4 = _graph(L, build((4, 5), L.pg_jit_add))
    h = [L.pg_jit_graph_hash(g) for g in (g1, g2, g3, g4)]
    assert h[0] == h[1] and len(set(h)) == 3
    for g in (g1, g2, g3, g4):
        L.pg_jit_graph_free(g)


def test_jit_codegen_compiles_for_gfx950_without_a_gpu(host_lib):
    """pg_jit_compile generates HIP source and compiles it with hiprtc for
    gfx950 before it needs the device: on this CPU-only host it stops at
    the module load, after writing the code object to the cache."""
    L = host_lib
    cache = Path(os.environ["PG_JIT_CACHE_DIR"])
    before = set(cache.glob("*.hsaco"))

    def chain(g):  # the config-1 chain plus a broadcast bias, every op kind
        a = L.pg_jit_add_input(g, *shape_arg((64, 64)))
        b = L.pg_jit_add_input(g, *shape_arg((64,)))
        x = L.pg_jit_relu(g, L.pg_jit_mul(g, L.pg_jit_add(g, a, b), a))
        for op in (L.pg_jit_tanh, L.pg_jit_gelu, L.pg_jit_sigmoid, L.pg_jit_erf, L.pg_jit_exp, L.pg_jit_abs,
                   L.pg_jit_sin, L.pg_jit_cos, L.pg_jit_neg, L.pg_jit_step):
            x = op(g, x)
        x = L.pg_jit_div(g, L.pg_jit_sub(g, x, L.pg_jit_add_const(g, 0.5)), L.pg_jit_add_const(g, 3.0))
        return L.pg_jit_sqrt(g, L.pg_jit_log(g, L.pg_jit_add(g, L.pg_jit_abs(g, x),
                                                               L.pg_jit_add_const(g, 1.0))))
    g = _graph(L, chain)
    exe = L.pg_jit_compile(g)
    if exe is None:
        err = L.pg_jit_last_error().decode()
        assert "no device" in err, err
        assert set(cache.glob("*.hsaco")) - before, "no code object was written"
    else:  # a GPU is present
        L.pg_jit_exe_free(exe)
    L.pg_jit_graph_free(g)
    # a compile error surfaces as NULL plus the hiprtc log
    os.environ["PG_JIT_FORCE_COMPILE_ERROR"] = "1"
    try:
        g = _graph(L, lambda g: L.pg_jit_neg(g, L.pg_jit_add_input(g, *shape_arg((5,)))))
        assert L.pg_jit_compile(g) is None
        assert "hiprtc compile failed" in L.pg_jit_last_error().decode()
        L.pg_jit_graph_free(g)
    finally:
        del os.environ["PG_JIT_FORCE_COMPILE_ERROR"]


def test_reference_style_c_caller_compiles_and_links(tmp_path):
    """tests/c_callers/*.c, written against include/picograd the way the
    reference's tests and examples are (C11, the reference's entry points by
    name), compile warning-free and link against the library alone; the
    timing loop (chain_loop.c) loads the library it times with dlopen and
    links against nothing of either build."""
    from picograd_amd.build import C_CALLERS, DLOPEN_CALLERS, LIBDIR
    srcs = sorted(C_CALLERS.glob("*.c"))
    assert srcs
    for src in srcs:
        exe = tmp_path / src.stem
        dl = src.stem in DLOPEN_CALLERS
        link = ["-ldl", "-lm"] if dl else [f"-L{LIBDIR}", "-lpicograd_amd", "-lm", f"-Wl,-rpath,{LIBDIR}"]
        res = subprocess.run(["gcc", "-std=c11", "-O2", "-Wall", "-Wextra", "-Werror", f"-I{ROOT / 'include'}",
                              str(src), "-o", str(exe), *link], capture_output=True, text=True)
        assert res.returncode == 0, res.stdout + res.stderr
        deps = subprocess.run(["ldd", str(exe)], capture_output=True, text=True).stdout
        assert "not found" not in deps
        assert ("libpicograd" in deps) != dl, deps


def test_tensor_and_ops_abi_is_complete():
    """The tensor utilities (core/tensor.h:52-95) and the tensor-level ops of
    ops/elementwise.h, activations.h and matmul.h that the configs' own
    callers use are declared and exported."""
    every = {n for v in declared_functions().values() for n in v}
    lib = C.CDLL(str(LIB))
    for name in ("pg_tensor_allclose", "pg_tensor_arange", "pg_tensor_linspace", "pg_tensor_eye",
                 "pg_tensor_get", "pg_tensor_set", "pg_tensor_print", "pg_tensor_permute_view",
                 "pg_tensor_pool_clear", "pg_tensor_pool_size", "pg_tensor_pool_bytes",
                 "pg_add", "pg_sub", "pg_mul", "pg_div", "pg_neg", "pg_exp", "pg_log", "pg_sqrt", "pg_sin",
                 "pg_cos", "pg_erf", "pg_abs", "pg_clamp", "pg_relu", "pg_leaky_relu", "pg_sigmoid", "pg_tanh",
                 "pg_gelu", "pg_matmul", "pg_bmm"):
        assert name in every and hasattr(lib, name), name


def _plan(lib, ta, tb, m, n, k, batch=1, cus=0):
    sp, sec = C.c_int(0), C.c_double(0.0)
    tile = lib.pg_amd_gemm16_plan(ta, tb, m, n, k, batch, cus, C.byref(sp), C.byref(sec))
    assert sec.value > 0.0
    return tile, sp.value


def test_gemm_launch_plans_of_the_configs():
    """The MFMA GEMM planner's choices for the configs' GEMMs (host logic):
    256 x 256 tiles where they fill the chip (config 3, config 5's 4096-wide
    layers: their dgrad and wgrad then pair in one launch), the 128 x 256 tile for config 4's ragged grads on their shares
    of the chip (160 CUs for dgrad, 96 for wgrad: both then run without
    split-K, in one launch), 128 x 256 tiles split two ways for config 5's
    first-layer wgrad and the skinny kernel (one launch, no split) for its
    10-wide layer's forward and wgrad."""
    lib = picograd_amd.load()
    assert _plan(lib, 0, 0, 8192, 4096, 4096) == (2, 1)    # config 3 dgrad
    assert _plan(lib, 1, 1, 4096, 4096, 8192) == (2, 1)    # config 3 wgrad
    assert _plan(lib, 0, 1, 4096, 4096, 4096) == (2, 1)    # config 5 forward
    # config 5's 4096-wide dgrad and wgrad: both 256 x 256 without split-K,
    # so the backward runs them as one whole-chip paired launch (as config 3)
    assert _plan(lib, 0, 0, 4096, 4096, 4096) == (2, 1)
    assert _plan(lib, 1, 1, 4096, 4096, 4096) == (2, 1)
    assert _plan(lib, 1, 1, 1024, 4096, 4096) == (3, 2)    # config 5 first-layer wgrad
    assert _plan(lib, 0, 1, 4096, 10, 4096) == (4, 1)      # config 5 10-wide forward: skinny kernel
    assert _plan(lib, 1, 1, 4096, 10, 4096) == (4, 1)      # config 5 10-wide wgrad: skinny kernel
    assert _plan(lib, 0, 1, 512, 10, 4096) == (1, 8)       # too few rows for it: split-K
    assert _plan(lib, 0, 0, 4097, 1000, 3000, cus=160) == (3, 1)  # config 4 dgrad
    assert _plan(lib, 1, 1, 1000, 3000, 4097, cus=96) == (3, 1)   # config 4 wgrad
    assert _plan(lib, 0, 0, 512, 128, 512, batch=32, cus=128) == (1, 1)  # config 4 bmm grads
    # a budget of fewer CUs never makes the estimate faster
    t_all, t_half = C.c_double(), C.c_double()
    sp = C.c_int()
    lib.pg_amd_gemm16_plan(0, 0, 4097, 1000, 3000, 1, 0, C.byref(sp), C.byref(t_all))
    lib.pg_amd_gemm16_plan(0, 0, 4097, 1000, 3000, 1, 128, C.byref(sp), C.byref(t_half))
    assert t_half.value >= t_all.value
