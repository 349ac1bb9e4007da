"""Whole-output checks of the MFMA GEMM results (test infrastructure).

Every element of a device GEMM output is compared with the exact product of
the same 16-bit operands, computed in f64 on the host (numpy's BLAS: an
8192 x 4096 x 4096 product takes about a second), against the worst-case
bound of f32 summation:

    |got[i, j] - sum_p A[i, p] B[p, j]|  <=  gamma(K) * sum_p |A[i, p] B[p, j]|

gamma(K) = K u / (1 - K u) holds for any order of K rounded additions
(Higham, Accuracy and Stability of Numerical Algorithms, 2nd ed., eq. 3.5),
and bf16 x bf16 or f16 x f16 products are exact in f32 (8- or 11-bit
significands), so the bound covers every kernel whatever its tiling,
split-K order or MFMA-internal order.  u is taken as 2^-23, which also
covers additions that truncate instead of rounding to nearest.  On the
configs' data |ref| is ~sqrt(K) times smaller than sum |A B| while the bound
is ~K u times it, so the bound sits 100-1000x below a typical element: a
tile left at zero, written with another tile's values, or written twice
fails in nearly every element.  `check_product` proves that on each call by
planting such mistakes in a copy of the reference on the CPU.

The relative Frobenius error over the whole output is held to 1e-5 as well
(identical operands, summation order only; the north star's GEMM bar is
1e-3).
"""
from __future__ import annotations

import numpy as np

U = 2.0 ** -23
FRO_TOL = 1e-5


def gamma(k: int) -> float:
    return k * U / (1.0 - k * U)


def _f64(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float64)


def product_ref(terms, add=None):
    """(ref, S, K) for add + sum_t A_t @ B_t: the f64 value, |add| +
    sum |A_t| @ |B_t| and the total number of additions (batched operands:
    leading batch dims)."""
    ref = S = None
    k = 0
    for A, B in terms:
        A, B = _f64(A), _f64(B)
        r, s = A @ B, np.abs(A) @ np.abs(B)
        ref = r if ref is None else ref + r
        S = s if S is None else S + s
        k += A.shape[-1]
    if add is not None:
        ref = ref + _f64(add)
        S = S + np.abs(_f64(add))
        k += 1
    return ref, S, k


def _bad_tiles(bad: np.ndarray, tile: int) -> list:
    m, n = bad.shape[-2:]
    b = bad.reshape(-1, m, n).any(axis=0)
    out = []
    for i in range(0, m, tile):
        for j in range(0, n, tile):
            if b[i:i + tile, j:j + tile].any():
                out.append((i // tile, j // tile))
    return out


def check_product(got: np.ndarray, terms, what: str, tile: int = 128, planted: bool = True, add=None) -> dict:
    """Every element of `got` (f32, [..., M, N]) against add + sum_t A_t @ B_t.

    terms: list of (A, B) as upcast 16-bit operands ([..., M, K] and
    [..., K, N]); more than one term, or `add` (the f32 C a beta = 1 launch
    added to), for a grad that accumulates.  Returns the measured figures.
    With `planted`, also shows on the CPU that the same check rejects the
    reference with one tile zeroed, one tile replaced by another's values
    and one tile doubled."""
    ref, S, k = product_ref(terms, add)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    # the bound, plus f32 rounding of the stored result and an absolute
    # floor at the f32 subnormal scale
    bound = gamma(k + 1) * S + 2.0 ** -126
    err = np.abs(got.astype(np.float64) - ref)
    bad = err > bound
    fro = float(np.linalg.norm(err) / max(np.linalg.norm(ref), 1e-300))
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements outside gamma(K) sum|AB| "
                           f"(K = {k}); 128-tiles {_bad_tiles(bad, tile)[:16]}")
    assert fro <= FRO_TOL, f"{what}: relative Frobenius {fro:.3e} > {FRO_TOL}"
    m, n = ref.shape[-2:]
    ntiles = ((m + tile - 1) // tile) * ((n + tile - 1) // tile) * (ref.size // (m * n))
    out = {"elements": int(ref.size), "tiles128": ntiles, "rel_fro": fro,
           "max_err_over_bound": float((err / bound).max())}
    if planted and m >= 2 * tile and n >= tile:
        out["planted_rejected"] = _planted(ref, bound, tile)
    print(f"  {what}: every element of {ref.shape} within gamma({k}) sum|AB| "
          f"(max err/bound {out['max_err_over_bound']:.2e}), rel_fro {fro:.2e}", flush=True)
    return out


def _planted(ref: np.ndarray, bound: np.ndarray, tile: int) -> int:
    """Plants three mistakes into a copy of the reference's first matrix and
    checks that the element test rejects each one in most of the tile."""
    r2 = ref.reshape(-1, *ref.shape[-2:])[0]
    b2 = bound.reshape(-1, *bound.shape[-2:])[0]
    m, n = r2.shape
    i0, j0 = (m // tile - 1) * tile, (n // tile - 1) * tile  # last whole tile
    sl = (slice(i0, i0 + tile), slice(j0, j0 + tile))
    other = (slice(0, tile), slice(0, tile))
    rejected = 0
    for bad_val in (np.zeros((tile, tile)), r2[other], 2.0 * r2[sl]):
        frac = float((np.abs(bad_val - r2[sl]) > b2[sl]).mean())
        assert frac > 0.9, f"planted mistake caught in only {frac:.2%} of the tile"
        rejected += 1
    return rejected




def check_linear(got_out: np.ndarray, got_z, terms, bias, act: int, what: str) -> dict:
    """The fused epilogue out = act(z), z = sum_t A_t @ B_t + bias, every
    element: z within gamma(K + 1) (sum |A B| + |bias|) of its f64 value
    (got_z, the kept pre-activation, may be None), and out within the same
    bound carried through act (ReLU and GELU are Lipschitz with constants 1
    and 1.13) plus the f32 evaluation of act (GELU: relative 2e-6 + z^2 2^-24,
    the accuracy pgmath.h's GELU is held to in test_pgmath.py)."""
    from scipy.special import erf
    ref, S, k = product_ref(terms)
    b = _f64(bias) if bias is not None else 0.0
    z = ref + b
    bz = gamma(k + 1) * (S + np.abs(b)) + 2.0 ** -126
    if got_z is not None:
        ez = np.abs(got_z.astype(np.float64) - z)
        assert (ez <= bz).all(), f"{what}: {int((ez > bz).sum())} pre-activations outside the bound"
    if act == 2:
        o, lip = 0.5 * z * (1.0 + erf(z / np.sqrt(2.0))), 1.13
        ev = (2e-6 + z * z * 2.0 ** -24) * np.abs(o)
    elif act == 1:
        o, lip, ev = np.maximum(z, 0.0), 1.0, 0.0
    else:
        o, lip, ev = z, 1.0, 0.0
    bound = lip * bz + ev + 2.0 ** -24 * np.abs(o) + 2.0 ** -126
    err = np.abs(got_out.astype(np.float64) - o)
    assert (err <= bound).all(), (f"{what}: {int((err > bound).sum())} outputs outside the bound; "
                                  f"128-tiles {_bad_tiles(err > bound, 128)[:16]}")
    fro = float(np.linalg.norm(err) / max(np.linalg.norm(o), 1e-300))
    assert fro <= FRO_TOL, f"{what}: relative Frobenius {fro:.3e}"
    print(f"  {what}: every element of {o.shape} within the epilogue bound, rel_fro {fro:.2e}", flush=True)
    return {"rel_fro": fro}
