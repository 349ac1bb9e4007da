"""The device math helpers (picograd_amd/csrc/kernels/pgmath.h) compiled for
the host and checked against f64 references on dense grids (CPU only).

The device build swaps exp2f / division for v_exp_f32 / v_rcp_f32 (both
within 1 ulp); the GPU tests check the device results against the
reference's grads.
"""
from __future__ import annotations

import ctypes as C
import math
import subprocess
from pathlib import Path

import numpy as np
import pytest
from scipy.special import ndtr

ROOT = Path(__file__).resolve().parent.parent
HDR = ROOT / "picograd_amd" / "csrc" / "kernels"

SRC = r"""
#include "pgmath.h"
#include <stddef.h>
void eval(const float *z, float *gelu, float *ggrad, float *sig, float *tail, size_t n)
{
    for (size_t i = 0; i < n; i++) {
        float d;
        gelu[i] = pgm_gelu(z[i]);
        ggrad[i] = pgm_gelu_grad(z[i]);
        sig[i] = pgm_sigmoid(z[i]);
        tail[i] = pgm_phi_tail(z[i], &d);
    }
}
"""


@pytest.fixture(scope="module")
def pgm(tmp_path_factory):
    d = tmp_path_factory.mktemp("pgmath")
    (d / "t.c").write_text(SRC)
    so = d / "t.so"
    subprocess.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fPIC", "-shared", f"-I{HDR}",
                    str(d / "t.c"), "-o", str(so), "-lm"], check=True)
    L = C.CDLL(str(so))
    L.eval.argtypes = [C.c_void_p] * 5 + [C.c_size_t]

    def run(z):
        z = np.ascontiguousarray(z, np.float32)
        outs = [np.empty_like(z) for _ in range(4)]
        L.eval(z.ctypes.data, *(o.ctypes.data for o in outs), z.size)
        return outs
    return run


def test_phi_tail_relative_accuracy(pgm):
    z = np.linspace(-12.0, 12.0, 400001).astype(np.float32)
    _, _, _, tail = pgm(z)
    exact = ndtr(-np.abs(z.astype(np.float64)))
    rel = np.abs(tail - exact) / exact
    # f32 evaluation: the exponent z^2/2 is rounded once (|z|^2 2^-24 relative)
    bound = 2e-6 + (z.astype(np.float64) ** 2) * 2 ** -24
    assert np.all(rel <= bound)
    assert rel[np.abs(z) <= 4].max() <= 1.5e-6


def test_gelu_and_grad_against_f64(pgm):
    z = np.linspace(-10.0, 10.0, 200001).astype(np.float32)
    gelu, ggrad, _, _ = pgm(z)
    z64 = z.astype(np.float64)
    Phi = ndtr(z64)
    phi = np.exp(-0.5 * z64 * z64) / math.sqrt(2 * math.pi)
    g64 = z64 * Phi
    d64 = Phi + z64 * phi
    # gelu: relative accuracy everywhere (the tail bound for z < 0)
    nz = g64 != 0
    rel = np.abs(gelu[nz] - g64[nz]) / np.abs(g64[nz])
    assert np.all(rel <= 2e-6 + z64[nz] ** 2 * 2 ** -24)
    assert np.all(gelu[~nz] == 0)
    # gelu': within 8 f32 ulps of the terms that cancel (P(t) near t = 1, and
    # Phi + z phi near the zero at z ~ -0.75): 50x inside the 1e-5 bar
    assert np.all(np.abs(ggrad - d64) <= 5e-7 * np.maximum(np.abs(d64), 0.5))


def test_sigmoid_against_f64(pgm):
    z = np.linspace(-40.0, 40.0, 200001).astype(np.float32)
    _, _, sig, _ = pgm(z)
    exact = 1.0 / (1.0 + np.exp(-z.astype(np.float64)))
    assert np.all(np.abs(sig - exact) <= 4e-7 * exact + 1e-30 + (np.abs(z) * 2 ** -24 * exact))


def test_planted_mistake_in_the_fit_is_caught(pgm):
    """A sign slip in one coefficient of the tail polynomial (a plausible
    transcription error) breaks the accuracy bound by orders of magnitude."""
    z = np.linspace(0.0, 4.0, 4001)
    t = 1.0 / (1.0 + 0.263464875 * z)
    c = [0.263531536, 0.262051702, 0.258060277, 0.142426163, 0.367844224, -0.325497687, 0.579365075,
         -0.372467279, 0.0780001506]
    phi = np.exp(-0.5 * z * z) / math.sqrt(2 * math.pi)
    good = phi * t * np.polyval(c[::-1], t)
    c[5] = -c[5]
    bad = phi * t * np.polyval(c[::-1], t)
    exact = ndtr(-z)
    assert (np.abs(good - exact) / exact).max() < 1e-7
    assert (np.abs(bad - exact) / exact).max() > 1e-2
