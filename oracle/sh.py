"""e3nn real spherical harmonics (component normalisation), degrees 0-4.

The polynomials are the Cartesian forms the reference uses
(``src/o3/spherical_harmonics/kernels/forward.py:21-57``), evaluated on
``(x, y, z)`` exactly as written there; ``|Y_l|^2 = 2l + 1`` on unit vectors.
"""

from __future__ import annotations

import math

import numpy as np


def spherical_harmonics(lmax: int, vectors: np.ndarray) -> list[np.ndarray]:
    """List over l of arrays [n, 2l+1] for the unit-normalised input vectors."""
    v = np.asarray(vectors, dtype=np.float64)
    v = v / np.linalg.norm(v, axis=-1, keepdims=True)
    x, y, z = v[..., 0], v[..., 1], v[..., 2]
    r = math.sqrt
    out = [np.ones_like(x)[..., None]]
    sh1 = [r(3.0) * x, r(3.0) * y, r(3.0) * z]
    out.append(np.stack(sh1, -1))
    y2 = y ** 2
    x2z2 = x ** 2 + z ** 2
    sh2 = [r(15.0) * x * z, r(15.0) * x * y, r(5.0) * (y2 - 0.5 * x2z2), r(15.0) * y * z,
           0.5 * r(15.0) * (z ** 2 - x ** 2)]
    out.append(np.stack(sh2, -1))
    rad2 = x2z2 + y2
    sh3 = [
        r(7.0 / 6.0) * (sh2[0] * z + sh2[4] * x),
        r(7.0) * y * sh2[0],
        r(35.0 / 8.0) * y * sh2[1] - r(21.0 / 24.0) * rad2 * sh1[0],
        r(35.0 / 9.0) * y * sh2[2] - r(28.0 / 27.0) * rad2 * sh1[1],
        r(35.0 / 8.0) * y * sh2[3] - r(21.0 / 24.0) * rad2 * sh1[2],
        r(7.0) * y * sh2[4],
        r(7.0 / 6.0) * (sh2[4] * z - sh2[0] * x),
    ]
    out.append(np.stack(sh3, -1))
    sh4 = [
        r(9.0 / 8.0) * (sh3[0] * z + sh3[6] * x),
        r(9.0) * y * sh3[0],
        r(63.0 / 12.0) * y * sh3[1] - r(45.0 / 60.0) * rad2 * sh2[0],
        r(63.0 / 15.0) * y * sh3[2] - r(72.0 / 75.0) * rad2 * sh2[1],
        r(63.0 / 16.0) * y * sh3[3] - r(81.0 / 80.0) * rad2 * sh2[2],
        r(63.0 / 15.0) * y * sh3[4] - r(72.0 / 75.0) * rad2 * sh2[3],
        r(63.0 / 12.0) * y * sh3[5] - r(45.0 / 60.0) * rad2 * sh2[4],
        r(9.0) * y * sh3[6],
        r(9.0 / 8.0) * (sh3[6] * z - sh3[0] * x),
    ]
    out.append(np.stack(sh4, -1))
    return out[: lmax + 1]
