"""Checkpoints of device tensors, parameter lists and optimiser state.

PGT1 / PGMD files written here must be the reference's bytes for the same
tensors (tests/golden/ckpt.npz holds the files the reference wrote), files
the reference wrote must load, and crafted headers must be refused exactly
where the reference's loader refuses them.  Optimiser state (which the
reference cannot save) must resume a run bit for bit.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from picograd_amd.capi import AdamCfg, SgdCfg

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def golden(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def plist(nodes):
    return (C.c_void_p * len(nodes))(*nodes)


def test_save_writes_the_reference_bytes(lib, tmp_path):
    """pg_tensor_save of device tensors (f32, f16, bf16; ranks 1 to 8)
    writes the reference's file byte for byte."""
    g = golden("ckpt")
    for i in range(5):
        dt, arr = int(g[f"t{i}_dtype"]), g[f"t{i}_data"]
        t = lib.tensor(arr, dt)
        path = tmp_path / f"t{i}.pgt"
        assert lib.pg_tensor_save(t, str(path).encode()), lib.pg_amd_last_error()
        lib.pg_tensor_free(t)
        assert path.read_bytes() == g[f"t{i}_bytes"].tobytes(), i


def test_load_reads_the_reference_files(lib, tmp_path):
    """pg_tensor_load of the reference's files gives device tensors with
    the same dtype, shape and elements."""
    g = golden("ckpt")
    for i in range(5):
        path = tmp_path / f"r{i}.pgt"
        path.write_bytes(g[f"t{i}_bytes"].tobytes())
        t = lib.pg_tensor_load(str(path).encode())
        assert t, i
        arr = g[f"t{i}_data"]
        ti = lib.tinfo(t)
        assert ti.dtype == int(g[f"t{i}_dtype"]) and lib.shape(t) == arr.shape
        assert np.array_equal(lib.read(t), arr), i
        lib.pg_tensor_free(t)


def test_loader_refuses_what_the_reference_refuses(lib, tmp_path):
    """Crafted records: the device loader accepts exactly those the
    reference's pg_tensor_load accepted (tensor.c:655-702)."""
    g = golden("ckpt")
    for i, (name, ok) in enumerate(zip(g["crafted_names"], g["crafted_loads"])):
        path = tmp_path / f"c{i}.pgt"
        path.write_bytes(g[f"crafted_{i}"].tobytes())
        t = lib.pg_tensor_load(str(path).encode())
        assert bool(t) == bool(ok), name
        if t:
            lib.pg_tensor_free(t)
    assert not lib.pg_tensor_load(str(tmp_path / "missing.pgt").encode())


def test_large_round_trip_through_the_pipeline(lib, oracle, tmp_path):
    """A 100 MB f32 tensor and a 27 MB bf16 tensor (several 8 MiB chunks
    and a ragged last one) save to the oracle's PGT1 bytes and load back
    bit for bit."""
    rng = np.random.default_rng(5)
    for dt, arr in ((0, rng.standard_normal((5003, 4999)).astype(np.float32)),
                    (2, rng.integers(0, 65536, (3, 4500, 1003), dtype=np.uint16))):
        t = lib.tensor(arr, dt)
        path = tmp_path / "big.pgt"
        assert lib.pg_tensor_save(t, str(path).encode())
        lib.pg_tensor_free(t)
        blob = path.read_bytes()
        assert blob == oracle.pgt1_bytes(dt, arr)
        t2 = lib.pg_tensor_load(str(path).encode())
        assert t2 and np.array_equal(lib.read(t2), arr)
        lib.pg_tensor_free(t2)


def test_params_in_the_reference_module_format(lib, tmp_path):
    """pg_amd_params_load_into reads the reference's pg_module_save file
    into device parameters; pg_amd_params_save writes it back byte for
    byte.  A count or shape mismatch is refused; a refused record leaves
    its parameter unchanged."""
    g = golden("ckpt")
    ref = tmp_path / "ref.pgmd"
    ref.write_bytes(g["mod_bytes"].tobytes())
    shapes = [g[f"mod_p{i}"].shape for i in range(3)]
    nodes = [lib.var(np.zeros(s, np.float32)) for s in shapes]
    assert lib.pg_amd_params_load_into(plist(nodes), 3, str(ref).encode())
    for i, n in enumerate(nodes):
        assert np.array_equal(lib.value(n), g[f"mod_p{i}"])
    out = tmp_path / "out.pgmd"
    assert lib.pg_amd_params_save(plist(nodes), 3, str(out).encode())
    assert out.read_bytes() == g["mod_bytes"].tobytes()
    assert not lib.pg_amd_params_load_into(plist(nodes[:2]), 2, str(ref).encode())
    wrong = [lib.var(np.zeros(shapes[0], np.float32)), lib.var(np.full((3, 2), 7.0, np.float32)),
             lib.var(np.zeros(shapes[2], np.float32))]
    assert not lib.pg_amd_params_load_into(plist(wrong), 3, str(ref).encode())
    assert np.array_equal(lib.value(wrong[0]), g["mod_p0"])  # loaded before the mismatch
    assert np.array_equal(lib.value(wrong[1]), np.full((3, 2), 7.0, np.float32))
    for n in nodes + wrong:
        lib.pg_node_free(n)


def _set_grad(lib, n, arr):
    node = lib.node(n)
    if node.grad:
        lib.pg_tensor_free(node.grad)
    node.grad = lib.tensor(arr)


SHAPES = [(64, 48), (48,), (48, 10), (10,)]


def _run(lib, nodes, opt, step_fn, zero_fn, grads):
    for gs in grads:
        zero_fn(opt)
        for n, gr in zip(nodes, gs):
            if gr is not None:
                _set_grad(lib, n, gr)
        step_fn(opt)


def _grads(seed, steps, skip_last_bias=False):
    rng = np.random.default_rng(seed)
    out = []
    for s in range(steps):
        gs = [rng.standard_normal(sh).astype(np.float32) for sh in SHAPES]
        if skip_last_bias:
            gs[3] = None  # that parameter has no state yet at the checkpoint
        out.append(gs)
    return out


@pytest.mark.parametrize("kind", ["sgd", "adam"])
def test_optimiser_state_resumes_bit_for_bit(lib, tmp_path, kind):
    """Three steps, a checkpoint of the parameters (PGMD) and the optimiser
    state (PGSG / PGAD, with the Adam step counter), two more steps; a
    fresh run restored from the checkpoint and given the same two grads
    ends on the same weights bit for bit.  Without the state it does not."""
    rng = np.random.default_rng(8)
    init = [rng.standard_normal(s).astype(np.float32) for s in SHAPES]
    before, after = _grads(1, 3, skip_last_bias=True), _grads(2, 2)
    if kind == "sgd":
        cfg = SgdCfg(0.05, 0.9, 0.0, 1e-3, True)
        new = lambda: lib.pg_sgd_new(C.byref(cfg))
        add, step, zero, free = lib.pg_sgd_add_param, lib.pg_sgd_step, lib.pg_sgd_zero_grad, lib.pg_sgd_free
        save, load = lib.pg_amd_sgd_save, lib.pg_amd_sgd_load_into
    else:
        cfg = AdamCfg(0.01, 0.9, 0.99, 1e-8, 0.01, True, True)
        new = lambda: lib.pg_adam_new(C.byref(cfg))
        add, step, zero, free = lib.pg_adam_add_param, lib.pg_adam_step, lib.pg_adam_zero_grad, lib.pg_adam_free
        save, load = lib.pg_amd_adam_save, lib.pg_amd_adam_load_into

    def fresh():
        nodes = [lib.var(a) for a in init]
        opt = new()
        for n in nodes:
            assert add(opt, n) == 0
        return nodes, opt

    nodes, opt = fresh()
    _run(lib, nodes, opt, step, zero, before)
    pfile, sfile = tmp_path / "p.pgmd", tmp_path / "s.state"
    assert lib.pg_amd_params_save(plist(nodes), len(nodes), str(pfile).encode())
    assert save(opt, str(sfile).encode())
    _run(lib, nodes, opt, step, zero, after)
    want = [lib.value(n) for n in nodes]
    if kind == "adam":
        assert lib.pg_adam_get_step(opt) == 5
    free(opt)

    results = {}
    for restore_state in (True, False):
        nodes2, opt2 = fresh()
        assert lib.pg_amd_params_load_into(plist(nodes2), len(nodes2), str(pfile).encode())
        if restore_state:
            assert load(opt2, str(sfile).encode())
            if kind == "adam":
                assert lib.pg_adam_get_step(opt2) == 3
        _run(lib, nodes2, opt2, step, zero, after)
        results[restore_state] = [lib.value(n) for n in nodes2]
        free(opt2)
        for n in nodes2:
            lib.pg_node_free(n)
    for a, b in zip(want, results[True]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert not all(np.array_equal(a, b) for a, b in zip(want, results[False]))
    for n in nodes:
        lib.pg_node_free(n)


def test_optimiser_state_mismatch_is_refused(lib, tmp_path):
    """A state file for a different parameter count or shape is refused."""
    a = [lib.var(np.ones((4, 3), np.float32)), lib.var(np.ones(3, np.float32))]
    opt = lib.pg_sgd_new(C.byref(SgdCfg(0.1, 0.9, 0.0, 0.0, False)))
    for n in a:
        lib.pg_sgd_add_param(opt, n)
        _set_grad(lib, n, np.ones(lib.shape(lib.node(n).value), np.float32))
    lib.pg_sgd_step(opt)
    f = tmp_path / "s.pgsg"
    assert lib.pg_amd_sgd_save(opt, str(f).encode())
    other = lib.pg_sgd_new(C.byref(SgdCfg(0.1, 0.9, 0.0, 0.0, False)))
    b = [lib.var(np.ones((4, 3), np.float32))]
    lib.pg_sgd_add_param(other, b[0])
    assert not lib.pg_amd_sgd_load_into(other, str(f).encode())  # count
    c = [lib.var(np.ones((3, 4), np.float32)), lib.var(np.ones(3, np.float32))]
    third = lib.pg_sgd_new(C.byref(SgdCfg(0.1, 0.9, 0.0, 0.0, False)))
    for n in c:
        lib.pg_sgd_add_param(third, n)
    assert not lib.pg_amd_sgd_load_into(third, str(f).encode())  # shape
    adam = lib.pg_adam_new(None)
    assert not lib.pg_amd_adam_load_into(adam, str(f).encode())  # an SGD file
    lib.pg_adam_free(adam)
    for o in (opt, other, third):
        lib.pg_sgd_free(o)
    for n in a + b + c:
        lib.pg_node_free(n)
