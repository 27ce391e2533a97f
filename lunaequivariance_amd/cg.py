"""Real-basis Clebsch-Gordan (Wigner-3j) coefficients in e3nn's convention.

The reference obtains its coefficients from e3nn 0.6.0's construction
(``src/lunatp/utils/cg.py:99-180``): complex SU(2) Clebsch-Gordan
coefficients from the Racah formula, a change of basis from complex to real
spherical harmonics for each of the three degrees, and Frobenius
normalisation.  The construction is restated here from that mathematics;
the sign and ordering conventions must agree exactly because every output
of the convolution depends on them.

``sparse_terms`` mirrors ``build_cg_terms`` (``cg.py:31-41``): the non-zero
entries in ``(i, j, k)`` row-major order, scaled by the path weight, with
``|c| > 1e-12`` kept.
"""

from __future__ import annotations

import functools
from fractions import Fraction
from math import factorial, sqrt

import numpy as np
import torch

CG_THRESHOLD = 1.0e-12


def _racah(j1: int, m1: int, j2: int, m2: int, j3: int, m3: int) -> float:
    """<j1 m1 j2 m2 | j3 m3> for integer degrees (Condon-Shortley phase)."""
    if m1 + m2 != m3 or abs(m3) > j3:
        return 0.0
    if not abs(j1 - j2) <= j3 <= j1 + j2:
        return 0.0
    f = factorial
    prefactor = Fraction(
        (2 * j3 + 1) * f(j3 + j1 - j2) * f(j3 - j1 + j2) * f(j1 + j2 - j3)
        * f(j3 + m3) * f(j3 - m3),
        f(j1 + j2 + j3 + 1) * f(j1 - m1) * f(j1 + m1) * f(j2 - m2) * f(j2 + m2),
    )
    total = Fraction(0)
    low = max(-j1 + j2 + m3, -j1 + m1, 0)
    high = min(j2 + j3 + m1, j3 - j1 + j2, j3 + m3)
    for v in range(low, high + 1):
        sign = -1 if (v + j2 + m2) % 2 else 1
        total += sign * Fraction(
            f(j2 + j3 + m1 - v) * f(j1 - m1 + v),
            f(v) * f(j3 - j1 + j2 - v) * f(j3 + m3 - v) * f(v + j1 - j2 - m3),
        )
    return float(prefactor) ** 0.5 * float(total)


def su2_clebsch_gordan(l1: int, l2: int, l3: int) -> np.ndarray:
    """Complex-basis coefficients indexed ``[l1+m1, l2+m2, l3+m3]``."""
    out = np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1))
    for m1 in range(-l1, l1 + 1):
        for m2 in range(-l2, l2 + 1):
            m3 = m1 + m2
            if abs(m3) <= l3:
                out[l1 + m1, l2 + m2, l3 + m3] = _racah(l1, m1, l2, m2, l3, m3)
    return out


def real_to_complex(l: int) -> np.ndarray:
    """Unitary ``Q`` with complex harmonic ``m`` = sum over real index of ``Q[m, r]``.

    Real index ``r = l + m`` holds the ``sin``-type harmonic for ``m < 0`` and
    the ``cos``-type one for ``m > 0``; the global factor ``(-i)^l`` makes the
    resulting coupling coefficients real (e3nn's convention).
    """
    q = np.zeros((2 * l + 1, 2 * l + 1), dtype=np.complex128)
    half = 1.0 / sqrt(2.0)
    q[l, l] = 1.0
    for m in range(1, l + 1):
        sign = -1.0 if m % 2 else 1.0
        q[l - m, l + m] = half
        q[l - m, l - m] = -1j * half
        q[l + m, l + m] = sign * half
        q[l + m, l - m] = 1j * sign * half
    return ((-1j) ** l) * q


@functools.lru_cache(maxsize=None)
def _wigner_3j_np(l1: int, l2: int, l3: int) -> np.ndarray:
    if not (abs(l1 - l2) <= l3 <= l1 + l2):
        raise ValueError(f"({l1}, {l2}, {l3}) violates the triangle inequality")
    c = su2_clebsch_gordan(l1, l2, l3).astype(np.complex128)
    q1, q2, q3 = real_to_complex(l1), real_to_complex(l2), real_to_complex(l3)
    # Real coefficient [a, b, c] = sum_{m1 m2 m3} Q1[m1,a] Q2[m2,b] conj(Q3[m3,c]) C[m1,m2,m3]
    real = np.einsum("ia,jb,kc,ijk->abc", q1, q2, np.conj(q3), c)
    if np.abs(real.imag).max(initial=0.0) >= 1e-5:
        raise AssertionError("basis change left an imaginary part")
    real = real.real
    real = real / np.linalg.norm(real)
    real.setflags(write=False)
    return real


def wigner_3j(l1: int, l2: int, l3: int, dtype=None, device=None) -> torch.Tensor:
    """Real coupling tensor of shape ``(2l1+1, 2l2+1, 2l3+1)`` with unit Frobenius norm."""
    for value in (l1, l2, l3):
        if not isinstance(value, int):
            raise TypeError("degrees must be int")
    dtype = torch.get_default_dtype() if dtype is None else dtype
    return torch.tensor(_wigner_3j_np(l1, l2, l3), dtype=dtype, device=device)


def sparse_terms(l1: int, l2: int, l3: int, scale: float = 1.0):
    """Non-zero ``(i, j, k, c*scale)`` in row-major order (``cg.py:31-41``)."""
    dense = _wigner_3j_np(l1, l2, l3)
    terms = []
    for i in range(dense.shape[0]):
        for j in range(dense.shape[1]):
            for k in range(dense.shape[2]):
                value = float(dense[i, j, k]) * scale
                if abs(value) > CG_THRESHOLD:
                    terms.append((i, j, k, value))
    return terms


__all__ = ["wigner_3j", "sparse_terms", "su2_clebsch_gordan", "real_to_complex", "CG_THRESHOLD"]
