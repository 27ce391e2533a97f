"""Pins of the CPU oracle's Clebsch-Gordan coefficients (no GPU).

The oracle's real-basis coefficients are built from two ingredients
(``oracle/wigner.py``): complex Clebsch-Gordan coefficients (Racah formula)
and the complex-to-real basis change.  Each is checked against facts that do
not come from the same code: textbook values and the stretched-state closed
form for the first; unitarity and agreement with the reference's own
spherical-harmonic polynomials for the second.  The products are then
checked for closed forms, normalisation, equivariance and consistency with
those harmonics.
"""

import math

import numpy as np
import pytest

from oracle.sh import spherical_harmonics
from oracle.wigner import basis_change, racah_cg, wigner_3j


@pytest.mark.parametrize("args,value", [
    ((1, 1, 1, 1, 2, 2), 1.0),
    ((1, 1, 1, -1, 1, 0), 1 / math.sqrt(2)),
    ((1, -1, 1, 1, 1, 0), -1 / math.sqrt(2)),
    ((1, 1, 1, -1, 0, 0), 1 / math.sqrt(3)),
    ((1, 0, 1, 0, 0, 0), -1 / math.sqrt(3)),
    ((1, 0, 1, 0, 2, 0), 2 / math.sqrt(6)),
    ((1, 0, 1, 0, 1, 0), 0.0),
    ((2, 2, 1, -1, 2, 1), math.sqrt(1 / 3)),   # <j m+1; 1 -1|j m> = sqrt((j-m)(j+m+1)/(2j(j+1)))
    ((2, 1, 1, 0, 2, 1), math.sqrt(1 / 6)),    # <j m; 1 0|j m> = m/sqrt(j(j+1))
    ((2, 0, 1, 1, 2, 1), -math.sqrt(1 / 2)),   # <j m-1; 1 1|j m> = -sqrt((j+m)(j-m+1)/(2j(j+1)))
])
def test_racah_textbook_values(args, value):
    """Condon-Shortley values from the standard 1x1 and j x 1 coupling tables."""
    assert racah_cg(*args) == pytest.approx(value, abs=1e-14)


@pytest.mark.parametrize("j1,j2", [(1, 1), (2, 1), (2, 3), (3, 3)])
def test_racah_stretched_and_orthonormal(j1, j2):
    J = j1 + j2
    comb = math.comb
    for m1 in range(-j1, j1 + 1):
        for m2 in range(-j2, j2 + 1):
            expected = math.sqrt(comb(2 * j1, j1 + m1) * comb(2 * j2, j2 + m2) / comb(2 * J, J + m1 + m2))
            assert racah_cg(j1, m1, j2, m2, J, m1 + m2) == pytest.approx(expected, abs=1e-13)
    rows = []
    for j3 in range(abs(j1 - j2), j1 + j2 + 1):
        for m3 in range(-j3, j3 + 1):
            rows.append([racah_cg(j1, m1, j2, m2, j3, m3) for m1 in range(-j1, j1 + 1)
                         for m2 in range(-j2, j2 + 1)])
    rows = np.array(rows)
    assert np.allclose(rows @ rows.T, np.eye(len(rows)), atol=1e-12)


@pytest.mark.parametrize("l", range(6))
def test_basis_change_unitary(l):
    q = basis_change(l)
    assert np.allclose(q @ q.conj().T, np.eye(2 * l + 1), atol=1e-14)


def triples(lmax):
    return [(a, b, c) for a in range(lmax + 1) for b in range(lmax + 1)
            for c in range(abs(a - b), min(a + b, lmax) + 1)]


@pytest.mark.parametrize("l", range(5))
def test_closed_forms(l):
    d = 2 * l + 1
    assert np.allclose(wigner_3j(0, l, l)[0], np.eye(d) / math.sqrt(d), atol=1e-14)
    assert np.allclose(wigner_3j(l, 0, l)[:, 0, :], np.eye(d) / math.sqrt(d), atol=1e-14)
    assert np.allclose(wigner_3j(l, l, 0)[:, :, 0], np.eye(d) / math.sqrt(d), atol=1e-14)


def test_vector_products():
    """C(1,1,0) = delta/sqrt(3) (examples/basic_uvu_conv.py:33-41) and C(1,1,1) = +epsilon/sqrt(6)."""
    assert np.allclose(wigner_3j(1, 1, 0)[:, :, 0], np.eye(3) / math.sqrt(3), atol=1e-15)
    eps = np.zeros((3, 3, 3))
    for i, j, k in ((0, 1, 2), (1, 2, 0), (2, 0, 1)):
        eps[i, j, k], eps[j, i, k] = 1, -1
    assert np.allclose(wigner_3j(1, 1, 1), eps / math.sqrt(6), atol=1e-15)


@pytest.mark.parametrize("l1,l2,l3", triples(4))
def test_unit_norm(l1, l2, l3):
    assert np.linalg.norm(wigner_3j(l1, l2, l3)) == pytest.approx(1.0, abs=1e-14)


def test_harmonics_couple_with_positive_weight():
    """sum_ij C_ijk Y^l1_i(v) Y^l2_j(v) = alpha Y^l3_k(v) with alpha > 0 when
    l1 + l2 + l3 is even, and 0 when odd, for the reference's harmonics
    (src/o3/spherical_harmonics/kernels/forward.py:21-57).  This fixes the
    real basis, its ordering and the sign of every even triple."""
    rng = np.random.default_rng(0)
    v = rng.normal(size=(64, 3))
    Y = spherical_harmonics(4, v)
    for l1, l2, l3 in triples(4):
        if l1 + l2 > 4 and l3 > 4:
            continue
        z = np.einsum("ijk,ni,nj->nk", wigner_3j(l1, l2, l3), Y[l1], Y[l2])
        if (l1 + l2 + l3) % 2:
            assert np.abs(z).max() < 1e-12
            continue
        alpha = (z * Y[l3]).sum() / (Y[l3] ** 2).sum()
        assert alpha > 0.1, (l1, l2, l3, alpha)
        assert np.abs(z - alpha * Y[l3]).max() < 1e-12


def random_rotation(rng):
    q, r = np.linalg.qr(rng.normal(size=(3, 3)))
    q = q @ np.diag(np.sign(np.diag(r)))
    return q if np.linalg.det(q) > 0 else -q


def wigner_d(l, R, rng):
    """D^l with Y^l(R v) = D^l Y^l(v), fitted from the reference harmonics."""
    v = rng.normal(size=(200, 3))
    A = spherical_harmonics(4, v)[l]
    B = spherical_harmonics(4, v @ R.T)[l]
    D, *_ = np.linalg.lstsq(A, B, rcond=None)
    return D.T


@pytest.mark.parametrize("seed", [0, 1])
def test_equivariance_all_triples(seed):
    """C is an intertwiner: C contracted with D1 (x) D2 equals D3 applied to C.
    Odd triples are included (their sign follows from the pinned ingredients)."""
    rng = np.random.default_rng(seed)
    R = random_rotation(rng)
    D = [wigner_d(l, R, rng) for l in range(4)]
    for l in range(4):
        assert np.allclose(D[l] @ D[l].T, np.eye(2 * l + 1), atol=1e-10)
    for l1, l2, l3 in triples(3):
        C = wigner_3j(l1, l2, l3)
        left = np.einsum("ijk,ia,jb->abk", C, D[l1], D[l2])
        right = np.einsum("abq,kq->abk", C, D[l3])
        assert np.allclose(left, right, atol=1e-10), (l1, l2, l3)


@pytest.mark.parametrize("l1,l2,l3", triples(4))
def test_package_coefficients_match_oracle(l1, l2, l3):
    from lunaequivariance_amd.cg import wigner_3j as package_w3j
    import torch

    assert np.allclose(package_w3j(l1, l2, l3, dtype=torch.float64).numpy(), wigner_3j(l1, l2, l3), atol=1e-15)
