"""Benchmark of the MI355X picograd backward path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only c2,c3,c4,c1,c5,opt,ckpt,jit]

Headline (the JSON `value`): config 2 of BASELINE.json -- the fused
broadcasting elementwise backward of y = gelu(x + bias) * sigmoid(g),
x, g f32 [16384, 4096], bias [4096], loss = sum_all(y).  One step is one
pg_backward() over the resident graph: the fused kernel reads x, g and bias
and writes dx, dg and dbias (the column sum over 16384 rows) in one pass.
value = algorithmic bytes (16 B/element + 32 KiB) / measured step time.

Also reported in `extra`: config 3 (bf16 dgrad + wgrad, TFLOP/s), config 4
(ragged f16 matmul + bmm backward, TFLOP/s), config 1 (the [64, 64] chain,
µs per iteration of leaves + forward + backward), config 5 (the MLP
training step, steps/s), the optimiser leg (AdamW + clipping by the
global grad norm over config 5's 37.8M parameters, GB/s) and the
checkpoint leg (config 5's parameters and SGD momentum saved and loaded in
the reference's PGT1/PGMD formats, GB/s) and jit_demo.c's workloads
(µs per iteration, beside the reference's published figures).

Timing: HIP events on the library stream around K steps (after W warmup
steps, with stream synchronisation on both sides); per-kernel durations
come from the library's kernel timer (HIP events around each launch of
the dominant kernel on the same stream).  The CPU baseline is the
reference's own CPU path (oracle/_ref, built from the reference sources)
timed on this host over a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import csv
import ctypes as C
import json
import math
import os
import shutil
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0  # dense MFMA, MI355X
T_JIT_MAIN, T_JIT_FIN, T_GEMM16, T_SGD, T_STAGE, T_ADAM, T_CLIP = 0, 1, 2, 3, 4, 5, 6


class HipEvents:
    """hipEvent timing on an explicit stream (the library stream)."""

    def __init__(self, stream: int):
        self.hip = C.CDLL("libamdhip64.so")
        self.stream = C.c_void_p(stream)
        for fn, args in (("hipEventCreate", [C.POINTER(C.c_void_p)]),
                         ("hipEventRecord", [C.c_void_p, C.c_void_p]),
                         ("hipEventSynchronize", [C.c_void_p]),
                         ("hipEventElapsedTime", [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]),
                         ("hipEventDestroy", [C.c_void_p])):
            getattr(self.hip, fn).argtypes = args
            getattr(self.hip, fn).restype = C.c_int

    def time_segments(self, segments) -> float:
        """segments: (prepare, fn, n) triples, run in order on the stream:
        prepare() untimed, then fn() n times between two events.  Nothing
        waits in between, so the host keeps enqueueing ahead of the device.
        Returns the summed milliseconds of the timed parts."""
        evs = []
        for prepare, fn, n in segments:
            a, b = C.c_void_p(), C.c_void_p()
            self.hip.hipEventCreate(C.byref(a))
            self.hip.hipEventCreate(C.byref(b))
            prepare()
            self.hip.hipEventRecord(a, self.stream)
            for _ in range(n):
                fn()
            self.hip.hipEventRecord(b, self.stream)
            evs.append((a, b))
        total = 0.0
        for a, b in evs:
            self.hip.hipEventSynchronize(b)
            ms = C.c_float()
            self.hip.hipEventElapsedTime(C.byref(ms), a, b)
            total += ms.value
            self.hip.hipEventDestroy(a)
            self.hip.hipEventDestroy(b)
        return total

    def time(self, fn, steps: int) -> float:
        a, b = C.c_void_p(), C.c_void_p()
        self.hip.hipEventCreate(C.byref(a))
        self.hip.hipEventCreate(C.byref(b))
        self.hip.hipEventRecord(a, self.stream)
        for _ in range(steps):
            fn()
        self.hip.hipEventRecord(b, self.stream)
        self.hip.hipEventSynchronize(b)
        ms = C.c_float()
        self.hip.hipEventElapsedTime(C.byref(ms), a, b)
        self.hip.hipEventDestroy(a)
        self.hip.hipEventDestroy(b)
        return ms.value


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def warm(L, step, min_steps, min_seconds=0.1):
    """Untimed warmup: at least min_steps steps and min_seconds of device
    work.  Under sustained MFMA load the chip settles at a higher clock
    after some tens of milliseconds than in the first few (the GEMMs run
    ~10 % slower during the first ~20 ms), so the GEMM legs warm up by
    time, not by a step count alone."""
    t0, n = time.perf_counter(), 0
    while n < min_steps or time.perf_counter() - t0 < min_seconds:
        step()
        n += 1
        if n % 8 == 0:
            L.sync()
    L.sync()
    return n


def timer_ms(lib, kind):
    cnt = C.c_size_t()
    total = lib.pg_amd_timer_read(kind, C.byref(cnt))
    return total, cnt.value


# ---------------------------------------------------------------- counter calibration

CALIB_ROWS, CALIB_COLS = 16384, 4096


def calibrate_copy(L, reps=3):
    """pg_ag_neg over an f32 [16384, 4096] leaf: the k_unary kernel reads
    256 MiB and writes 256 MiB, a copy of known size whose FETCH_SIZE and
    WRITE_SIZE readings scale the fused kernel's."""
    shp = (C.c_size_t * 2)(CALIB_ROWS, CALIB_COLS)
    x = L.pg_var_full(2, shp, 1.5, False)
    jit = L.pg_autograd_is_jit_enabled()
    L.pg_autograd_set_jit(False)  # the eager kernel, not a deferred fused run
    for _ in range(reps):
        y = L.pg_ag_neg(x)
        L.sync()
        L.pg_node_free(y)
    L.pg_autograd_set_jit(jit)
    L.sync()
    L.pg_node_free(x)
    log(f"[calib] k_unary copy of {CALIB_ROWS * CALIB_COLS * 4} B read + write, {reps} launches")


# ---------------------------------------------------------------- HBM traffic (rocprofv3 --pmc)

def _pmc_pass(counter: str, outdir: Path) -> dict[str, list[float]] | None:
    """One rocprofv3 counter pass over `bench.py --pmc-child`; returns the
    per-dispatch counter values (KiB) by kernel name."""
    cmd = ["rocprofv3", "--pmc", counter, "-d", str(outdir), "-o", "run", "--output-format", "csv", "--",
           sys.executable, str(Path(__file__).resolve()), "--pmc-child"]
    env = dict(os.environ, TMPDIR="/tmp")
    try:
        subprocess.run(cmd, timeout=150, env=env, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL,
                       check=False)
    except subprocess.TimeoutExpired:
        return None
    files = list(outdir.rglob("run_counter_collection.csv"))
    if not files:
        return None
    out: dict[str, list[float]] = {}
    with open(files[0]) as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"].replace("(anonymous namespace)::", "").split("(")[0]
            out.setdefault(f"{name}@{r['Grid_Size']}", []).append(float(r["Counter_Value"]))
    return out


def measure_traffic() -> dict | None:
    """HBM bytes per pgjit_main launch from FETCH_SIZE and WRITE_SIZE, each
    scaled by what the same counter reads for the calibration copy
    (k_unary reading and writing 256 MiB).  Runs before this process
    touches the GPU, as two child processes under rocprofv3."""
    if not shutil.which("rocprofv3"):
        return None
    calib_grid = "2097152"  # k_unary over 16384 x 4096 f32: 8192 blocks x 256
    calib_kib = CALIB_ROWS * CALIB_COLS * 4 / 1024
    res = {}
    with tempfile.TemporaryDirectory(dir="/tmp") as td:
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            got = _pmc_pass(counter, Path(td) / counter)
            if not got:
                return None
            cal = got.get(f"k_unary@{calib_grid}")
            # the fused backward is the pgjit_main dispatched three times (the
            # forward run of the graph is a pgjit_main dispatched once)
            main = sorted((v for k, v in got.items() if k.startswith("pgjit_main@")), key=len)
            if not cal or not main:
                return None
            cal_kib = sum(cal) / len(cal)
            main_kib = sum(main[-1]) / len(main[-1])
            res[counter] = {"kib_per_dispatch": round(main_kib, 1), "calib_kib": round(cal_kib, 1),
                            "factor": round(calib_kib / cal_kib, 4)}
    total = sum(v["kib_per_dispatch"] * v["factor"] * 1024 for v in res.values())
    return {"bytes": int(total), "counters": res}


def pmc_child() -> int:
    """The workload the counter passes profile: the calibration copy, then
    three backward steps of config 2."""
    import picograd_amd
    L = picograd_amd.load()
    if L.pg_amd_init() != 0:
        return 1
    calibrate_copy(L)
    x, bias, g = c2_inputs(16384, 4096)
    loss, nodes = c2_graph(L, x, bias, g)
    for _ in range(3):
        L.pg_backward(loss)
    L.sync()
    for n in nodes:
        L.pg_node_free(n)
    L.sync()
    return 0


# ---------------------------------------------------------------- config 2

def c2_inputs(R, Cc, seed=43):
    from oracle_lib import Oracle
    o = Oracle()
    o.orc_seed(seed)
    x = o.normal(R * Cc, 0.0, 1.0).reshape(R, Cc)
    bias = o.normal(Cc, 0.0, 0.1)
    g = o.normal(R * Cc, 0.0, 1.0).reshape(R, Cc)
    return x, bias, g


def c2_graph(L, x, bias, g):
    nx, nb, ng = L.var(x), L.var(bias), L.var(g)
    t0 = L.op("add", nx, nb)
    t1 = L.op("gelu", t0)
    t2 = L.op("sigmoid", ng)
    y = L.op("mul", t1, t2)
    loss = L.op("sum_all", y)
    return loss, [loss, y, t2, t1, t0, nx, nb, ng]


def bench_c2(L, ev, steps, warmup, R=16384, Cc=4096):
    log(f"[c2] inputs {R}x{Cc}")
    x, bias, g = c2_inputs(R, Cc)
    loss, nodes = c2_graph(L, x, bias, g)
    del x, g
    L.sync()
    step = lambda: L.pg_backward(loss)
    for _ in range(warmup):
        step()
    L.sync()
    assert L.pg_autograd_last_was_jit(), L.pg_autograd_last_error().decode()
    L.pg_amd_timer_reset()
    L.pg_amd_timer_enable(1)
    ms = ev.time(step, steps)
    L.pg_amd_timer_enable(0)
    main_ms, main_n = timer_ms(L, T_JIT_MAIN)
    fin_ms, fin_n = timer_ms(L, T_JIT_FIN)
    L.pg_amd_timer_reset()
    # untimed re-run without the timer events for the step time
    ms = ev.time(step, steps)
    nbytes = 16 * R * Cc + 8 * Cc  # read x, g; write dx, dg (+ bias in, dbias out)
    step_ms = ms / steps
    kern_ms = main_ms / max(main_n, 1)
    for n in nodes:
        L.pg_node_free(n)
    L.sync()
    return {
        "step_ms": step_ms,
        "gbs": nbytes / (step_ms * 1e-3) / 1e9,
        "kernel_ms": kern_ms,
        "kernel_gbs": nbytes / (kern_ms * 1e-3) / 1e9,
        "fin_ms": fin_ms / max(fin_n, 1),
        "bytes": nbytes,
        "launches": main_n,
    }


def _ref_threads() -> int:
    """Threads of the reference's pool: PICOGRAD_THREADS, else the online
    CPU count capped at 64 (thread/pool.c:59, :99-141)."""
    env = os.environ.get("PICOGRAD_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return min(int(env), 64)
    return min(os.cpu_count() or 1, 64)


def host_info() -> dict:
    """What the CPU figures were measured on: CPU model, the ISA extensions
    that decide which reference micro-kernels run (backend/cpu/gemm.c:259-360),
    logical CPUs available, glibc, and the compiler and flags of the
    reference build in oracle/_ref."""
    model, flags, ident = None, set(), {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key = line.split(":", 1)[0].strip()
                if key == "model name" and model is None:
                    model = line.split(":", 1)[1].strip()
                elif key == "flags" and not flags:
                    flags = set(line.split(":", 1)[1].split())
                elif key in ("vendor_id", "cpu family", "model", "stepping", "cache size") and key not in ident:
                    ident[key] = line.split(":", 1)[1].strip()
    except OSError:
        pass
    # a virtualised host may name only the product line ("AMD EPYC"): the
    # family / model / stepping numbers identify the part (family 26: Zen 5)
    if model and ident:
        model = (f"{model} (vendor {ident.get('vendor_id')}, family {ident.get('cpu family')}, "
                 f"model {ident.get('model')}, stepping {ident.get('stepping')}, cache {ident.get('cache size')})")
    isa = {k: k in flags for k in ("avx2", "fma", "f16c", "avx512f", "avx512_bf16", "avx512_fp16",
                                   "amx_bf16", "amx_tile")}
    try:
        cpus = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        cpus = os.cpu_count()
    build = None
    info = ROOT / "oracle" / "_ref" / "build_info.txt"
    if info.exists():
        build = info.read_text().strip().splitlines()
    try:
        glibc = os.confstr("CS_GNU_LIBC_VERSION")
    except (ValueError, OSError):
        glibc = None
    return {"cpu_model": model, "isa": isa, "logical_cpus": cpus, "glibc": glibc,
            "reference_build": build, "reference_pool_threads": _ref_threads()}


def cpu_c2(rows=2048, Cc=4096, budget_s=20.0):
    """The reference CPU path (oracle/_ref) on a row sample of config 2."""
    from oracle_lib import REF_SO
    from picograd_amd.capi import PgLib
    if not REF_SO.exists():
        return None
    R = PgLib(REF_SO, device=False)
    x, bias, g = c2_inputs(rows, Cc)
    loss, nodes = c2_graph(R, x, bias, g)
    t0 = time.perf_counter()
    R.pg_backward(loss)  # warmup: absorbs the reference JIT's compile
    times = []
    while len(times) < 5 and time.perf_counter() - t0 < budget_s:
        s = time.perf_counter()
        R.pg_backward(loss)
        times.append(time.perf_counter() - s)
    for n in nodes:
        R.pg_node_free(n)
    t = float(np.median(times))
    nbytes = 16 * rows * Cc + 8 * Cc
    return {"value": nbytes / t / 1e9, "unit": "GB/s", "cores": _ref_threads(), "kind": "reference",
            "sample": f"config 2 at [{rows},{Cc}] (of [16384,{Cc}]), reference pg_backward "
                      f"(hybrid JIT + eager, the pool capped at 64 threads; the JIT loop, "
                      f"GELU' and dbias loops are single-threaded), median of {len(times)}",
            "ms_per_step": t * 1e3}


# ---------------------------------------------------------------- config 3

def bench_c3(L, ev, steps, warmup, M=8192, K=4096, N=4096):
    from oracle_lib import Oracle
    from picograd_amd.capi import BF16
    log(f"[c3] A {M}x{K}, W {K}x{N}")
    o = Oracle()
    o.orc_seed(44)
    a16 = o.cast16(BF16, o.normal(M * K, 0.0, 1.0).reshape(M, K))
    w16 = o.cast16(BF16, o.normal(K * N, 0.0, 0.02).reshape(K, N))
    dc = o.normal(M * N, 0.0, 1.0).reshape(M, N)
    na, nw = L.var(a16, dtype=BF16), L.var(w16, dtype=BF16)
    c = L.op("matmul", na, nw)
    seed = L.tensor(dc)
    del a16, w16, dc
    L.sync()
    step = lambda: L.pg_amd_backward_from(c, seed)
    warm(L, step, warmup)
    L.pg_amd_timer_reset()
    L.pg_amd_timer_enable(1)
    ev.time(step, steps)
    L.pg_amd_timer_enable(0)
    g_ms, g_n = timer_ms(L, T_GEMM16)
    L.pg_amd_timer_reset()
    ms = ev.time(step, steps)
    flops = 2 * 2 * M * N * K
    step_ms = ms / steps
    # per GEMM: dgrad and wgrad run as one timed interval when they pair
    kern_ms = g_ms / (2 * steps)
    L.pg_tensor_free(seed)
    for n in (c, na, nw):
        L.pg_node_free(n)
    L.sync()
    # the attainable MFMA rate on this chip: pseudo-random bf16 operands from
    # registers, and fed from LDS as in the GEMM's inner loop
    probe_reg, probe_lds = L.pg_amd_mfma_probe(0), L.pg_amd_mfma_probe(1)
    gemm_tf = (flops / 2) / (kern_ms * 1e-3) / 1e12
    return {"step_ms": step_ms, "tflops": flops / (step_ms * 1e-3) / 1e12,
            "gemm_ms": kern_ms, "gemm_tflops": gemm_tf, "gemm_frac_of_2p5": gemm_tf / BF16_PEAK_TFLOPS,
            "flops": flops, "gemm_launches": g_n,
            "mfma_probe_tflops": {"registers": probe_reg, "lds_fed": probe_lds},
            "gemm_frac_of_lds_fed_probe": gemm_tf / probe_lds if probe_lds > 0 else None}


def cpu_c3(M=1024, K=4096, N=4096, budget_s=20.0):
    """Reference bwd_matmul (bf16 upcast + transpose + f32 sgemm) on a row
    sample of config 3."""
    from oracle_lib import REF_SO, Oracle
    from picograd_amd.capi import BF16, PgLib
    if not REF_SO.exists():
        return None
    R = PgLib(REF_SO, device=False)
    o = Oracle()
    o.orc_seed(44)
    a16 = o.cast16(BF16, o.normal(M * K, 0.0, 1.0).reshape(M, K))
    w16 = o.cast16(BF16, o.normal(K * N, 0.0, 0.02).reshape(K, N))
    w = o.normal(M * N, 0.0, 1.0).reshape(M, N)
    na, nw = R.var(a16, dtype=BF16), R.var(w16, dtype=BF16)
    c = R.op("matmul", na, nw)
    gw = R.var(w, requires_grad=False)
    prod = R.op("mul", c, gw)
    loss = R.op("sum_all", prod)
    R.pg_autograd_set_jit(False)
    t0 = time.perf_counter()
    times = []
    while len(times) < 3 and time.perf_counter() - t0 < budget_s:
        s = time.perf_counter()
        R.pg_backward(loss)
        times.append(time.perf_counter() - s)
    R.pg_autograd_set_jit(True)
    for n in (loss, prod, gw, c, na, nw):
        R.pg_node_free(n)
    t = float(np.median(times))
    flops = 2 * 2 * M * N * K
    return {"value": flops / t / 1e12, "unit": "TFLOP/s", "cores": _ref_threads(), "kind": "reference",
            "sample": f"bwd_matmul at M={M} of 8192 (bf16 upcast, transposes, the pool's f32 sgemm), "
                      f"median of {len(times)}", "ms": t * 1e3}


# ---------------------------------------------------------------- config 4

def bench_c4(L, ev, steps, warmup):
    """Config 4: the ragged f16 matmul backward (4097 x 1000 x 3000) and the
    bmm backward (32 x [512,128] . [128,512]) in one step; inputs from the
    library RNG, seed 45, in the reference's draw order."""
    from oracle_lib import Oracle
    from picograd_amd.capi import F16
    log("[c4] f16 4097x1000x3000 + bmm 32x512x128x512")
    o = Oracle()
    o.orc_seed(45)
    M, K, N = 4097, 1000, 3000
    a = o.cast16(F16, o.normal(M * K, 0.0, 1.0).reshape(M, K))
    b = o.cast16(F16, o.normal(K * N, 0.0, 1.0).reshape(K, N))
    dc = o.normal(M * N, 0.0, 1.0).reshape(M, N)
    sd = float(1.0 / np.sqrt(128.0))
    q = o.cast16(F16, o.normal(32 * 512 * 128, 0.0, sd).reshape(32, 512, 128))
    kt = o.cast16(F16, o.normal(32 * 128 * 512, 0.0, sd).reshape(32, 128, 512))
    ds = o.normal(32 * 512 * 512, 0.0, 1.0).reshape(32, 512, 512)
    na, nb, nq, nk = (L.var(x, dtype=F16) for x in (a, b, q, kt))
    c = L.op("matmul", na, nb)
    s = L.op("matmul", nq, nk)
    # upstream grads: f16 values (the cast in the backward is then exact)
    dc_t = L.tensor(o.cast16(F16, dc).view(np.float16).astype(np.float32))
    ds_t = L.tensor(o.cast16(F16, ds).view(np.float16).astype(np.float32))
    L.sync()

    def step():
        L.pg_amd_backward_from(c, dc_t)
        L.pg_amd_backward_from(s, ds_t)

    warm(L, step, warmup)
    L.pg_amd_timer_reset()
    L.pg_amd_timer_enable(1)
    ev.time(step, steps)
    L.pg_amd_timer_enable(0)
    g_ms, g_n = timer_ms(L, T_GEMM16)
    L.pg_amd_timer_reset()
    ms = ev.time(step, steps)
    for t in (dc_t, ds_t):
        L.pg_tensor_free(t)
    for n in (c, s, na, nb, nq, nk):
        L.pg_node_free(n)
    L.sync()
    flops = 2 * 2 * M * N * K + 2 * 2 * 32 * 512 * 512 * 128
    step_ms = ms / steps
    return {"step_ms": step_ms, "tflops": flops / (step_ms * 1e-3) / 1e12, "flops": flops,
            "gemm_ms_per_step": g_ms / steps, "gemm_tflops": flops / (g_ms / steps * 1e-3) / 1e12,
            "gemm_launches_per_step": g_n / steps, "peak_frac": flops / (step_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS}


# ---------------------------------------------------------------- config 5

C5_DIMS = (1024, 4096, 4096, 4096, 10)
C5_BATCH = 4096


def c5_counts(dims=C5_DIMS, batch=C5_BATCH):
    """GEMM FLOP per step (forward, wgrad of every layer, dgrad of layers
    2..L) and SGD bytes (p, buf read + write, g read = 20 B per parameter,
    plus the 2 B bf16 weight copy written for each weight the GEMMs read
    unpadded).  The last layer's dgrad (0.34 GFLOP of 894) is formed inside
    the activation pass of the layer before it, so its time falls in
    act_bwd_ms_per_step, not in gemm_ms_per_step."""
    kn = [dims[i] * dims[i + 1] for i in range(len(dims) - 1)]
    fwd = 2 * batch * sum(kn)
    bwd = 2 * batch * sum(kn) + 2 * batch * sum(kn[1:])
    params = sum(kn) + sum(dims[1:])
    shadow = sum(k for k, i in zip(kn, range(len(kn))) if dims[i] % 8 == 0 and dims[i + 1] % 8 == 0)
    return fwd, bwd, params, 20 * params + 2 * shadow


C5_CHUNK = 3  # steps between restores of the initial state


def bench_c5(L, ev, steps, warmup, dims=C5_DIMS, batch=C5_BATCH, fused=True):
    """Config 5: forward + pg_backward + pg_sgd_step of the bf16-GEMM MLP,
    layers as pg_amd_ag_linear16 nodes (fused) or matmul16 + add + gelu.

    The reference's mean_all makes this loss a sum over the batch, so at
    lr 0.01 it diverges (inf by step 4, NaN by step 5, in the reference as
    here).  Every run of C5_CHUNK steps therefore starts from the initial
    state: parameters copied back on the device from a snapshot, momentum
    buffers zeroed (as before the first step) and the bf16 weight copies
    remade, all enqueued outside the timed events.  Each timed step is one of
    steps 1-3 of the same trajectory, and every timed step's loss is checked
    finite."""
    from picograd_amd.capi import BF16, shape_arg
    from picograd_amd.mlp import Mlp
    log(f"[c5] MLP {dims}, batch {batch}, bf16 GEMM operands, f32 masters, fused={fused}")
    L.pg_seed(46)
    nd, sh = shape_arg((batch, dims[0]))
    x = L._check(L.pg_var_normal(nd, sh, 0.0, 1.0, False))
    nd, sh = shape_arg((batch, dims[-1]))
    t = L._check(L.pg_var_normal(nd, sh, 0.0, 1.0, False))
    mlp = Mlp.seeded(L, dims, BF16, fused=fused)
    params = [L.node(n).value for n in mlp.Ws + mlp.bs]
    snap = [L.pg_tensor_clone(p) for p in params]
    losses = []

    def one():
        n = mlp.step(x, t, keep_loss=True)
        losses.append(L.pg_tensor_view(L.node(n).value))  # keeps the 4 bytes, not the graph
        L.pg_node_free(n)

    one()  # creates the momentum buffers
    bufs = [L.pg_amd_sgd_buffer(mlp.opt, i) for i in range(len(params))]
    assert all(bufs), "momentum buffers missing after the first step"

    def restore():
        for p, s0 in zip(params, snap):
            L.pg_tensor_copy_from(p, s0)
        for b in bufs:
            L.pg_tensor_fill(b, 0.0)
        for p in params:
            L.pg_amd_tensor_refresh16(p)

    def segments(n):
        out = []
        while n > 0:
            k = min(C5_CHUNK, n)
            out.append((restore, one, k))
            n -= k
        return out

    t0 = time.perf_counter()
    while True:  # warm up by time as well (see warm)
        ev.time_segments(segments(max(warmup, C5_CHUNK)))
        if time.perf_counter() - t0 >= 0.1:
            break
    L.pg_amd_timer_reset()
    L.pg_amd_timer_enable(1)
    ev.time_segments(segments(steps))
    L.pg_amd_timer_enable(0)
    g_ms, g_n = timer_ms(L, T_GEMM16)
    s_ms, s_n = timer_ms(L, T_SGD)
    j_ms, j_n = timer_ms(L, T_JIT_MAIN)
    f_ms, f_n = timer_ms(L, T_JIT_FIN)
    a_ms, a_n = timer_ms(L, T_STAGE)
    L.pg_amd_timer_reset()
    n_before = len(losses)
    ms = ev.time_segments(segments(steps))
    vals = [float(L.read(v)[0]) for v in losses]
    timed = vals[n_before:]
    for v in losses:
        L.pg_tensor_free(v)
    for s0 in snap:
        L.pg_tensor_free(s0)
    mlp.free()
    L.pg_node_free(x)
    L.pg_node_free(t)
    L.sync()
    if not all(math.isfinite(v) for v in vals):
        raise RuntimeError(f"config 5: a non-finite loss among the measured steps: {vals}")
    fwd, bwd, params_n, sgd_bytes = c5_counts(dims, batch)
    step_ms = ms / steps
    gemm_ms = g_ms / steps
    sgd_ms = s_ms / max(s_n, 1)
    return {"steps_per_s": 1e3 / step_ms, "step_ms": step_ms, "gemm_flop": fwd + bwd,
            "step_tflops": (fwd + bwd) / (step_ms * 1e-3) / 1e12,
            "gemm_ms_per_step": gemm_ms, "gemm_tflops": (fwd + bwd) / (gemm_ms * 1e-3) / 1e12,
            "gemm_launches_per_step": g_n / steps,
            "sgd_ms": sgd_ms, "sgd_gbs": sgd_bytes / (sgd_ms * 1e-3) / 1e9, "sgd_bytes": sgd_bytes,
            "params": params_n, "fused_bwd_ms_per_step": (j_ms + f_ms) / steps,
            "act_bwd_ms_per_step": a_ms / steps,
            "restore_every": C5_CHUNK,
            "loss_first": vals[0], "loss_last": timed[-1],
            "losses_timed": sorted(set(round(v, 3) for v in timed)),
            "steps_run": len(vals)}


def cpu_c5(dims=C5_DIMS, batch=C5_BATCH, budget_s=40.0):
    """The reference's CPU path for config 5 at full shape in f32 (its matmul
    cannot take bf16 weights with f32 activations): pg_ag_matmul + add +
    gelu layers, mse, pg_backward, pg_sgd_step, timed per step."""
    from oracle_lib import REF_SO
    from picograd_amd.capi import F32, PgLib, shape_arg
    from picograd_amd.mlp import Mlp
    if not REF_SO.exists():
        return None
    R = PgLib(REF_SO, device=False)
    R.pg_seed(46)
    nd, sh = shape_arg((batch, dims[0]))
    x = R._check(R.pg_var_normal(nd, sh, 0.0, 1.0, False))
    nd, sh = shape_arg((batch, dims[-1]))
    t = R._check(R.pg_var_normal(nd, sh, 0.0, 1.0, False))
    mlp = Mlp.seeded(R, dims, F32)
    times = []
    t0 = time.perf_counter()
    # another step only while it fits the budget (one step is ~10-20 s)
    while len(times) < 3 and (not times or time.perf_counter() - t0 + times[-1] < budget_s):
        s = time.perf_counter()
        mlp.step(x, t)
        times.append(time.perf_counter() - s)
    mlp.free()
    R.pg_node_free(x)
    R.pg_node_free(t)
    # the first step also pays the reference's first allocations of every
    # buffer: left out of the median whenever a later step fits the budget
    timed = times[1:] if len(times) > 1 else times
    sec = float(np.median(timed))
    return {"value": 1.0 / sec, "unit": "steps/s", "cores": _ref_threads(),
            "kind": "reference",
            "sample": (f"median of {len(timed)} full config-5 steps in f32 after a first step"
                       if len(times) > 1 else "one full config-5 step in f32 (the only one within the budget)"),
            "ms": sec * 1e3, "steps_s": times}


# ---------------------------------------------------------------- optimiser leg

ADAM_CFG = (1e-3, 0.9, 0.999, 1e-8, 0.01, False, True)  # AdamW, weight decay 0.01


def c5_param_shapes(dims=C5_DIMS):
    """Config 5's parameters in registration order: W [in, out], b [out]."""
    out = []
    for i in range(len(dims) - 1):
        out += [(dims[i], dims[i + 1]), (dims[i + 1],)]
    return out


def _opt_setup(X, seed, dims):
    """Leaves of config 5's parameter shapes with N(0, 1) grads attached
    (node->grad assigned, as the reference's tests do), and the AdamW
    optimiser over them."""
    from picograd_amd.capi import AdamCfg, shape_arg
    X.pg_seed(seed)
    params = []
    for shp in c5_param_shapes(dims):
        nd, sh = shape_arg(shp)
        p = X._check(X.pg_var_normal(nd, sh, 0.0, 0.02, True))
        X.node(p).grad = X.pg_tensor_normal(nd, sh, 0.0, 1.0)
        params.append(p)
    opt = X.pg_adam_new(C.byref(AdamCfg(*ADAM_CFG)))
    for p in params:
        X.pg_adam_add_param(opt, p)
    arr = (C.c_void_p * len(params))(*params)
    return params, opt, arr


def bench_opt(L, ev, steps, warmup, dims=C5_DIMS):
    """One optimiser step = pg_clip_grad_norm (f64 norm pass, finisher, one
    host read of the norm; the scale is left pending on the grads) +
    pg_adam_step (one fused multi-tensor launch that applies the pending
    scale as it reads each grad) over config 5's 8 parameter tensors.
    Before each step the grads are rewritten from a snapshot on the device
    (untimed), as a backward writes them in training: without it the loop
    would re-clip the same grads, and each clip would first have to write
    the previous step's pending scale.  max_norm is 0.9 x the grads' norm,
    so every step scales.
    Algorithmic bytes per parameter: Adam 28 (read p, g, m, v; write p, m,
    v), the norm 4 (read g)."""
    params, opt, arr = _opt_setup(L, 48, dims)
    n = sum(int(np.prod(s)) for s in c5_param_shapes(dims))
    snaps = [L.pg_tensor_clone(L.node(p).grad) for p in params]

    def refresh():
        for p, snap in zip(params, snaps):
            L.pg_tensor_copy_from(L.node(p).grad, snap)

    norm0 = L.pg_grad_norm(arr, len(params))
    mx = 0.9 * norm0
    state = {"norm": norm0}

    def step():
        state["norm"] = L.pg_clip_grad_norm(arr, len(params), mx, 1e-6)
        L.pg_adam_step(opt)

    for _ in range(max(1, warmup)):
        refresh()
        step()
    L.sync()
    L.pg_amd_timer_reset()
    L.pg_amd_timer_enable(1)
    ev.time_segments([(refresh, step, 1)] * steps)
    L.pg_amd_timer_enable(0)
    a_ms, a_n = timer_ms(L, T_ADAM)
    c_ms, c_n = timer_ms(L, T_CLIP)
    L.pg_amd_timer_reset()
    ms = ev.time_segments([(refresh, step, 1)] * steps)
    L.pg_adam_free(opt)
    for p in params:
        L.pg_node_free(p)
    for snap in snaps:
        L.pg_tensor_free(snap)
    L.sync()
    adam_ms, clip_ms, step_ms = a_ms / max(a_n, 1), c_ms / max(c_n, 1), ms / steps
    return {"params": n, "step_ms": step_ms, "steps_per_s": 1e3 / step_ms,
            "step_gbs": 32 * n / (step_ms * 1e-3) / 1e9,
            "adam_ms": adam_ms, "adam_bytes": 28 * n, "adam_gbs": 28 * n / (adam_ms * 1e-3) / 1e9,
            "clip_ms": clip_ms, "clip_bytes": 4 * n, "clip_gbs": 4 * n / (clip_ms * 1e-3) / 1e9,
            "norm": norm0, "norm_clipped_to": mx, "grads": "rewritten from a snapshot before each step (untimed)",
            "optimizer": "AdamW lr 1e-3 wd 0.01 + clip by norm"}


def cpu_opt(dims=C5_DIMS, budget_s=15.0):
    """The reference's CPU pg_clip_grad_norm + pg_adam_step over the same
    parameter set (its loops are single-threaded)."""
    from oracle_lib import REF_SO
    from picograd_amd.capi import PgLib
    if not REF_SO.exists():
        return None
    R = PgLib(REF_SO, device=False)
    params, opt, arr = _opt_setup(R, 48, dims)
    n = sum(int(np.prod(s)) for s in c5_param_shapes(dims))
    norm, times = float("inf"), []
    t0 = time.perf_counter()
    while len(times) < 6 and time.perf_counter() - t0 < budget_s:
        s = time.perf_counter()
        mx = 0.9 * norm if math.isfinite(norm) else 1e30
        norm = min(R.pg_clip_grad_norm(arr, len(params), mx, 1e-6), mx)
        R.pg_adam_step(opt)
        times.append(time.perf_counter() - s)
    R.pg_adam_free(opt)
    for p in params:
        R.pg_node_free(p)
    sec = float(np.median(times))
    return {"value": 40 * n / sec / 1e9, "unit": "GB/s", "cores": 1, "kind": "reference",
            "sample": f"{len(times)} clip + AdamW steps over config 5's {n} parameters", "ms": sec * 1e3}


# ---------------------------------------------------------------- checkpoint leg

def _ckpt_dir() -> str:
    """A memory-backed directory when there is one, so the file system's
    disk speed is not what is measured."""
    import tempfile
    return "/dev/shm" if os.access("/dev/shm", os.W_OK) else tempfile.gettempdir()


def bench_ckpt(L, reps=3, dims=C5_DIMS):
    """pg_amd_params_save (PGMD, the reference's module format) +
    pg_amd_sgd_save (momentum) of config 5's parameters after one SGD step,
    then pg_amd_params_load_into + pg_amd_sgd_load_into back; best of
    `reps`.  Bytes = both files."""
    from picograd_amd.capi import SgdCfg, shape_arg
    L.pg_seed(49)
    params = []
    for shp in c5_param_shapes(dims):
        nd, sh = shape_arg(shp)
        p = L._check(L.pg_var_normal(nd, sh, 0.0, 0.02, True))
        L.node(p).grad = L.pg_tensor_normal(nd, sh, 0.0, 1.0)
        params.append(p)
    opt = L.pg_sgd_new(C.byref(SgdCfg(0.01, 0.9, 0.0, 1e-4, True)))
    for p in params:
        L.pg_sgd_add_param(opt, p)
    L.pg_sgd_step(opt)
    arr = (C.c_void_p * len(params))(*params)
    d = _ckpt_dir()
    pf, sf = os.path.join(d, f"pg_bench_{os.getpid()}.pgmd"), os.path.join(d, f"pg_bench_{os.getpid()}.pgsg")
    save, load = [], []
    try:
        for _ in range(reps):
            L.sync()
            t0 = time.perf_counter()
            ok = L.pg_amd_params_save(arr, len(params), pf.encode()) and L.pg_amd_sgd_save(opt, sf.encode())
            save.append(time.perf_counter() - t0)
            assert ok, L.pg_amd_last_error()
            t0 = time.perf_counter()
            ok = L.pg_amd_params_load_into(arr, len(params), pf.encode()) and L.pg_amd_sgd_load_into(opt, sf.encode())
            L.sync()
            load.append(time.perf_counter() - t0)
            assert ok, L.pg_amd_last_error()
        nbytes = os.path.getsize(pf) + os.path.getsize(sf)
    finally:
        for f in (pf, sf):
            if os.path.exists(f):
                os.remove(f)
        L.pg_sgd_free(opt)
        for p in params:
            L.pg_node_free(p)
    return {"bytes": nbytes, "dir": d, "save_ms": min(save) * 1e3, "load_ms": min(load) * 1e3,
            "save_gbs": nbytes / min(save) / 1e9, "load_gbs": nbytes / min(load) / 1e9}


def cpu_ckpt(reps=3, dims=C5_DIMS):
    """The reference's pg_module_save of the same parameter list from host
    memory (it has no optimiser-state format), and pg_module_load_into."""
    from oracle_lib import REF_SO
    from picograd_amd.capi import PgLib, shape_arg
    if not REF_SO.exists():
        return None
    R = PgLib(REF_SO, device=False)
    lib = R.lib
    lib.pg_module_new.restype = C.c_void_p
    lib.pg_module_register.argtypes = [C.c_void_p, C.c_void_p]
    lib.pg_module_save.argtypes = [C.c_void_p, C.c_char_p]
    lib.pg_module_load_into.argtypes = [C.c_void_p, C.c_char_p]
    lib.pg_module_free.argtypes = [C.c_void_p]
    R.pg_seed(49)
    m = lib.pg_module_new()
    nodes = []
    for shp in c5_param_shapes(dims):
        nd, sh = shape_arg(shp)
        n = R._check(R.pg_var_normal(nd, sh, 0.0, 0.02, True))
        lib.pg_module_register(C.c_void_p(m), C.c_void_p(n))
        nodes.append(n)
    f = os.path.join(_ckpt_dir(), f"pg_bench_ref_{os.getpid()}.pgmd")
    save, load = [], []
    try:
        for _ in range(reps):
            t0 = time.perf_counter()
            assert lib.pg_module_save(C.c_void_p(m), f.encode())
            save.append(time.perf_counter() - t0)
            t0 = time.perf_counter()
            assert lib.pg_module_load_into(C.c_void_p(m), f.encode())
            load.append(time.perf_counter() - t0)
        nbytes = os.path.getsize(f)
    finally:
        if os.path.exists(f):
            os.remove(f)
        lib.pg_module_free(C.c_void_p(m))
        for n in nodes:
            R.pg_node_free(n)
    return {"value": nbytes / min(save) / 1e9, "unit": "GB/s", "cores": 1, "kind": "reference",
            "sample": f"pg_module_save of config 5's parameters ({nbytes} B) from host memory",
            "load_gbs": nbytes / min(load) / 1e9}


# ---------------------------------------------------------------- forward JIT leg

def _demo_graph(X, shape):
    """jit_demo.c's graph: (a + b) * c -> relu -> tanh over `shape`."""
    from picograd_amd.capi import shape_arg
    g = X.pg_jit_graph_new()
    ids = []
    for _ in range(3):
        nd, sh = shape_arg(shape)
        ids.append(X.pg_jit_add_input(g, nd, sh))
    t = X.pg_jit_add(g, ids[0], ids[1])
    t = X.pg_jit_mul(g, t, ids[2])
    t = X.pg_jit_add_op(g, 11, (C.c_int * 1)(t), 1)  # PG_JIT_RELU
    t = X.pg_jit_add_op(g, 13, (C.c_int * 1)(t), 1)  # PG_JIT_TANH
    X.pg_jit_mark_output(g, t)
    exe = X.pg_jit_compile(g)
    assert exe, X.pg_jit_last_error()
    return g, exe


def _demo_inputs(X, shape):
    from picograd_amd.capi import shape_arg
    X.pg_seed(42)
    nd, sh = shape_arg(shape)
    return [X.pg_tensor_uniform(nd, sh, -1.0, 1.0) for _ in range(3)]


def jit_forward_loop(X, shape, iters):
    """jit_demo.c's timed loop: y = pg_jit_run_single(exe, ins, 3);
    pg_tensor_free(y), `iters` times; microseconds per iteration (the
    device library's result waited for at the end)."""
    g, exe = _demo_graph(X, shape)
    ts = _demo_inputs(X, shape)
    ins = (C.c_void_p * 3)(*ts)
    for _ in range(min(iters, 50)):
        X.pg_tensor_free(X.pg_jit_run_single(exe, ins, 3))
    if X.device:
        X.sync()
    t0 = time.perf_counter()
    for _ in range(iters):
        X.pg_tensor_free(X.pg_jit_run_single(exe, ins, 3))
    if X.device:
        X.sync()
    us = (time.perf_counter() - t0) / iters * 1e6
    for t in ts:
        X.pg_tensor_free(t)
    X.pg_jit_exe_free(exe)
    X.pg_jit_graph_free(g)
    return us


def chain_backward_loop(X, shape, iters):
    """The config-1 loop (leaves, add, mul, relu, tanh, sum_all,
    pg_backward) at `shape`: the README's "large [512,512]" backward case."""
    from oracle_lib import Oracle
    o = Oracle()
    o.orc_seed(42)
    n = shape[0] * shape[1]
    a, b, c = (o.uniform(n, -1.0, 1.0).reshape(shape) for _ in range(3))
    shp = (C.c_size_t * 2)(*shape)

    def one():
        na = X.pg_var_from_data(2, shp, a.ctypes.data, True)
        nb = X.pg_var_from_data(2, shp, b.ctypes.data, True)
        nc = X.pg_var_from_data(2, shp, c.ctypes.data, True)
        t0 = X.pg_ag_add(na, nb)
        t1 = X.pg_ag_mul(t0, nc)
        t2 = X.pg_ag_relu(t1)
        t3 = X.pg_ag_tanh(t2)
        loss = X.pg_ag_sum_all(t3)
        X.pg_backward(loss)
        for nn in (loss, t3, t2, t1, t0, na, nb, nc):
            X.pg_node_free(nn)

    for _ in range(min(iters, 10)):
        one()
    if X.device:
        X.sync()
    t0 = time.perf_counter()
    for _ in range(iters):
        one()
    if X.device:
        X.sync()
    return (time.perf_counter() - t0) / iters * 1e6


def cpu_c1():
    """The reference's own config-1 loop (oracle/_ref) on this host, with
    its JIT on and off (it runs single-threaded)."""
    from oracle_lib import REF_SO
    from picograd_amd.capi import PgLib
    if not REF_SO.exists():
        return None
    c_jit, c_eager = run_chain_loop(REF_SO, 10000, True), run_chain_loop(REF_SO, 10000, False)
    R = PgLib(REF_SO, device=False)
    jit = chain_backward_loop(R, (64, 64), 10000)
    R.pg_autograd_set_jit(False)
    eager = chain_backward_loop(R, (64, 64), 10000)
    R.pg_autograd_set_jit(True)
    out = {"value": c_jit["us_per_iter"] if c_jit else jit, "unit": "us/iter",
           "eager_us_per_iter": c_eager["us_per_iter"] if c_eager else eager,
           "python_ctypes_us_per_iter": jit, "python_ctypes_eager_us_per_iter": eager, "cores": 1,
           "kind": "reference", "loop": "C (tests/c_callers/chain_loop.c)" if c_jit else "Python ctypes",
           "sample": "10,000 iterations of the config-1 loop, JIT on (value) and off"}
    return out


def bench_jit(L):
    """jit_demo.c's workloads on the device: the fused forward at [64,64]
    (10,000 iterations, as the demo) and [512,512], and the chain's
    forward + backward at [512,512]."""
    return {"fwd_64x64_us_per_iter": jit_forward_loop(L, (64, 64), 10000),
            "fwd_512x512_us_per_iter": jit_forward_loop(L, (512, 512), 2000),
            "fwd_bwd_512x512_us_per_iter": chain_backward_loop(L, (512, 512), 1000),
            "reference_published_us_per_iter": {"fwd_64x64_jit": 14.0, "fwd_64x64_eager": 90.0,
                                                "bwd_512x512_jit": 500.0, "bwd_512x512_eager": 970.0,
                                                "source": "README.md:126-130, 10,000 iterations"}}


def cpu_jit():
    """The reference's own JIT (oracle/_ref; it compiles the graph with the
    system C compiler) on the same loops, on this host."""
    from oracle_lib import REF_SO
    from picograd_amd.capi import PgLib
    if not REF_SO.exists():
        return None
    R = PgLib(REF_SO, device=False)
    return {"fwd_64x64_us_per_iter": jit_forward_loop(R, (64, 64), 10000),
            "fwd_512x512_us_per_iter": jit_forward_loop(R, (512, 512), 200),
            "fwd_bwd_512x512_us_per_iter": chain_backward_loop(R, (512, 512), 100),
            "cores": 1, "kind": "reference"}


# ---------------------------------------------------------------- config 1

def bench_c1(L, iters=10000):
    from oracle_lib import Oracle
    o = Oracle()
    o.orc_seed(42)
    a, b, c = (o.uniform(4096, -1.0, 1.0).reshape(64, 64) for _ in range(3))
    shp = (C.c_size_t * 2)(64, 64)

    def one():
        na = L.pg_var_from_data(2, shp, a.ctypes.data, True)
        nb = L.pg_var_from_data(2, shp, b.ctypes.data, True)
        nc = L.pg_var_from_data(2, shp, c.ctypes.data, True)
        t0 = L.pg_ag_add(na, nb)
        t1 = L.pg_ag_mul(t0, nc)
        t2 = L.pg_ag_relu(t1)
        t3 = L.pg_ag_tanh(t2)
        loss = L.pg_ag_sum_all(t3)
        L.pg_backward(loss)
        for n in (loss, t3, t2, t1, t0, na, nb, nc):
            L.pg_node_free(n)

    for _ in range(20):
        one()
    L.sync()
    s = time.perf_counter()
    for _ in range(iters):
        one()
    L.sync()
    py_us = (time.perf_counter() - s) / iters * 1e6
    c_loop = run_chain_loop(picograd_amd_lib_path(), iters)
    out = {"us_per_iter": c_loop["us_per_iter"] if c_loop else py_us, "iters": iters,
           "loop": "C (tests/c_callers/chain_loop.c)" if c_loop else "Python ctypes",
           "us_per_iter_python_ctypes": py_us, "reference_published_us_per_iter": 114.0}
    if c_loop:
        out["c_loop_max_grad_err"] = c_loop["max_err"]
    return out


CHAIN_LOOP = ROOT / "tests" / "c_callers" / "bin" / "chain_loop"


def picograd_amd_lib_path():
    from picograd_amd.capi import _DEFAULT_LIB
    return _DEFAULT_LIB


def run_chain_loop(lib_path, iters, jit=True):
    """Config 1's loop as a C program (the reference's benchmark is a C
    loop, examples/train_xor_jit.c:200-214) over `lib_path`, run as a child
    process: {"us_per_iter", "iters", "max_err"}, or None when the program
    is not built or fails."""
    if not CHAIN_LOOP.exists():
        return None
    r = subprocess.run([str(CHAIN_LOOP), str(lib_path), str(iters), "1" if jit else "0"], capture_output=True,
                       text=True, timeout=600)
    if r.returncode != 0:
        log(f"[c1] chain_loop failed ({r.returncode}): {r.stderr.strip()[-300:]}")
        return None
    return json.loads(r.stdout.strip().splitlines()[-1])


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="c2,c3,c4,c1,c5,opt,ckpt,jit")
    ap.add_argument("--calib", action="store_true",
                    help="first run a plain copy kernel of known size (the HBM counter calibration)")
    ap.add_argument("--no-traffic", action="store_true", help="skip the two rocprofv3 counter passes")
    ap.add_argument("--pmc-child", action="store_true", help=argparse.SUPPRESS)
    a = ap.parse_args(argv)
    if a.pmc_child:
        return pmc_child()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (every box here has one); --gpus {a.gpus} is not supported",
              file=sys.stderr)
        return 2
    traffic = None
    if not a.no_traffic:
        log("[traffic] rocprofv3 FETCH_SIZE / WRITE_SIZE passes (child processes)")
        traffic = measure_traffic()
        log(f"[traffic] {traffic}")
    import picograd_amd
    L = picograd_amd.load()
    if L.pg_amd_init() != 0:
        raise SystemExit(f"no device: {L.pg_amd_last_error().decode()}")
    ev = HipEvents(L.pg_amd_stream())
    only = set(a.only.split(","))
    extra = {}
    if a.calib:
        calibrate_copy(L)
    c2 = bench_c2(L, ev, a.steps, a.warmup)
    log(f"[c2] {c2}")
    if "c3" in only:
        extra["c3_bf16_dgrad_wgrad"] = bench_c3(L, ev, max(3, a.steps // 2), a.warmup)
        log(f"[c3] {extra['c3_bf16_dgrad_wgrad']}")
    if "c4" in only:
        extra["c4_f16_ragged_and_bmm"] = bench_c4(L, ev, max(3, a.steps // 2), a.warmup)
        log(f"[c4] {extra['c4_f16_ragged_and_bmm']}")
    if "c1" in only:
        extra["c1_chain_64x64"] = bench_c1(L)
        log(f"[c1] {extra['c1_chain_64x64']}")
    if "c5" in only:
        c5 = bench_c5(L, ev, max(3, a.steps // 2), a.warmup, fused=True)
        c5["unfused_graph"] = bench_c5(L, ev, max(3, a.steps // 2), a.warmup, fused=False)
        extra["c5_mlp_train_step"] = c5
        log(f"[c5] {extra['c5_mlp_train_step']}")
    if "opt" in only:
        extra["opt_adamw_clip_c5_params"] = bench_opt(L, ev, max(3, a.steps), a.warmup)
        log(f"[opt] {extra['opt_adamw_clip_c5_params']}")
    if "jit" in only:
        extra["jit_demo"] = bench_jit(L)
        log(f"[jit] {extra['jit_demo']}")
    if "ckpt" in only:
        extra["ckpt_c5_params_and_momentum"] = bench_ckpt(L)
        log(f"[ckpt] {extra['ckpt_c5_params_and_momentum']}")
    cpu = None
    if not a.no_cpu:
        log("[cpu] reference CPU path, config 2 sample")
        cpu = cpu_c2()
        if cpu is not None:
            cpu["host"] = host_info()
        if "c3" in only and cpu is not None:
            log("[cpu] reference CPU path, config 3 sample")
            c3cpu = cpu_c3()
            if c3cpu:
                extra.setdefault("c3_bf16_dgrad_wgrad", {})["cpu_reference"] = c3cpu
        if "c5" in only and cpu is not None:
            log("[cpu] reference CPU path, config 5 (f32)")
            c5cpu = cpu_c5()
            if c5cpu:
                extra.setdefault("c5_mlp_train_step", {})["cpu_reference"] = c5cpu
        if "opt" in only and cpu is not None:
            log("[cpu] reference CPU path, clip + AdamW over config 5's parameters")
            ocpu = cpu_opt()
            if ocpu:
                extra.setdefault("opt_adamw_clip_c5_params", {})["cpu_reference"] = ocpu
        if "ckpt" in only and cpu is not None:
            log("[cpu] reference CPU path, pg_module_save of config 5's parameters")
            kcpu = cpu_ckpt()
            if kcpu:
                extra.setdefault("ckpt_c5_params_and_momentum", {})["cpu_reference"] = kcpu
        if "c1" in only and cpu is not None:
            log("[cpu] reference CPU path, config 1 loop")
            c1cpu = cpu_c1()
            if c1cpu:
                extra.setdefault("c1_chain_64x64", {})["cpu_reference"] = c1cpu
        if "jit" in only and cpu is not None:
            log("[cpu] reference JIT on jit_demo.c's loops")
            jcpu = cpu_jit()
            if jcpu:
                extra.setdefault("jit_demo", {})["cpu_reference"] = jcpu
    out = {
        "metric": "fused-bwd HBM GB/s",
        "value": round(c2["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(c2["step_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (splitmix64 seed 43, the reference's RNG)",
        "config": {"workload": "config 2: fused broadcasting elementwise backward, "
                               "y = gelu(x + bias) * sigmoid(g), x, g f32 [16384, 4096], bias [4096]",
                   "rows": 16384, "cols": 4096},
        "roofline": {"bound": "hbm", "achieved": round(c2["kernel_gbs"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(c2["kernel_gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic["bytes"] if traffic else None,
                     "traffic_counters": traffic["counters"] if traffic else None,
                     "kernel": "pgjit_main (fused backward)", "kernel_ms": round(c2["kernel_ms"], 5),
                     "finisher_ms": round(c2["fin_ms"], 5)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out, allow_nan=False), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
