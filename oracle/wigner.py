"""Real-basis Wigner-3j coefficients, restated for the oracle.

Follows e3nn 0.6.0 as restated by the reference
(``src/lunatp/utils/cg.py:99-180``): complex Clebsch-Gordan coefficients from
the Racah formula (``su2_clebsch_gordan``, ``cg.py:148-180``), a unitary
change of basis to real harmonics per degree (``change_basis_real_to_complex``,
``cg.py:103-118``) and Frobenius normalisation (``so3_clebsch_gordan``,
``cg.py:132-141``).  Written with explicit loops, independently of the
package's vectorised version, so the two can be compared.

Pinned by tests/test_oracle_pins.py: textbook Clebsch-Gordan values and the
stretched-state closed form, unitarity of the basis change, the closed forms
C(0,l,l) = C(l,0,l)-type identities and C(1,1,0) = delta/sqrt(3)
(``examples/basic_uvu_conv.py:33-41``), equivariance under Wigner-D matrices
built from the reference's spherical-harmonic polynomials, and agreement of
C(l1,l2,l3) contracted with those harmonics with the harmonics of degree l3.
"""

from __future__ import annotations

import math
from functools import lru_cache

import numpy as np


def racah_cg(j1: int, m1: int, j2: int, m2: int, j3: int, m3: int) -> float:
    """<j1 m1; j2 m2 | j3 m3> with the Condon-Shortley phase (integer degrees)."""
    if m1 + m2 != m3 or abs(m1) > j1 or abs(m2) > j2 or abs(m3) > j3:
        return 0.0
    if j3 < abs(j1 - j2) or j3 > j1 + j2:
        return 0.0
    f = math.factorial
    norm = (2 * j3 + 1) * f(j3 + j1 - j2) * f(j3 - j1 + j2) * f(j1 + j2 - j3) / f(j1 + j2 + j3 + 1)
    norm *= f(j3 + m3) * f(j3 - m3) / (f(j1 - m1) * f(j1 + m1) * f(j2 - m2) * f(j2 + m2))
    total = 0.0
    for v in range(0, j1 + j2 + j3 + 1):
        denominators = (v, j3 - j1 + j2 - v, j3 + m3 - v, v + j1 - j2 - m3)
        numerators = (j2 + j3 + m1 - v, j1 - m1 + v)
        if min(denominators) < 0 or min(numerators) < 0:
            continue
        term = f(numerators[0]) * f(numerators[1])
        term /= f(denominators[0]) * f(denominators[1]) * f(denominators[2]) * f(denominators[3])
        total += (-1) ** (v + j2 + m2) * term
    return math.sqrt(norm) * total


def basis_change(l: int) -> np.ndarray:
    """Q[m + l, r]: complex harmonic m in terms of real harmonics r (e3nn convention)."""
    q = np.zeros((2 * l + 1, 2 * l + 1), dtype=complex)
    s = 1 / math.sqrt(2)
    for m in range(-l, l + 1):
        if m < 0:
            q[l + m, l + abs(m)] = s
            q[l + m, l - abs(m)] = -1j * s
        elif m == 0:
            q[l, l] = 1
        else:
            q[l + m, l + m] = (-1) ** m * s
            q[l + m, l - m] = 1j * (-1) ** m * s
    return (-1j) ** l * q


@lru_cache(maxsize=None)
def wigner_3j(l1: int, l2: int, l3: int) -> np.ndarray:
    q1, q2, q3 = basis_change(l1), basis_change(l2), basis_change(l3)
    out = np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1), dtype=complex)
    for a in range(2 * l1 + 1):
        for b in range(2 * l2 + 1):
            for c in range(2 * l3 + 1):
                acc = 0j
                for m1 in range(-l1, l1 + 1):
                    for m2 in range(-l2, l2 + 1):
                        m3 = m1 + m2
                        if abs(m3) > l3:
                            continue
                        coupling = racah_cg(l1, m1, l2, m2, l3, m3)
                        if coupling == 0.0:
                            continue
                        acc += q1[l1 + m1, a] * q2[l2 + m2, b] * np.conj(q3[l3 + m3, c]) * coupling
                out[a, b, c] = acc
    assert np.abs(out.imag).max() < 1e-5
    real = out.real
    return real / np.sqrt((real ** 2).sum())
