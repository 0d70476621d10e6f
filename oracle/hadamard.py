"""Walsh-Hadamard incoherent processing, restated on the CPU (test oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

The reference names ``generate_hadamard_signs()`` and ``hadamard_transform()``
(``README.md:68-71``, ``:77``) but has no code for them, so the algorithm is
fixed by the build: ``R = diag(s) H_d / sqrt(d)`` with the Sylvester matrix
``H_d[i, j] = (-1)^popcount(i & j)`` and seeded signs ``s``.  The rotated row
is ``x' = x R``.  Evaluated in fp32 in a fixed order so the device result can
be compared bit for bit:

1. ``y = x * s`` (exact: sign flips),
2. butterflies for ``h = 1, 2, 4, ..., d/2``: for each i with ``i & h == 0``
   ``(y[i], y[i+h]) <- (y[i] + y[i+h], y[i] - y[i+h])`` (each fp32-rounded),
3. ``y * fp32(1/sqrt(d))``, then a single rounding to the output dtype.

The inverse (used for gradients) is ``g R^T``: butterflies first, then the
scale, then the signs.
"""
from __future__ import annotations

import numpy as np


def sylvester(d: int) -> np.ndarray:
    i = np.arange(d)
    pc = np.vectorize(lambda x: bin(x).count("1"))(i[:, None] & i[None, :])
    return np.where(pc % 2 == 0, 1.0, -1.0)


def _butterflies(y: np.ndarray) -> np.ndarray:
    d = y.shape[-1]
    y = y.copy()
    h = 1
    while h < d:
        yr = y.reshape(*y.shape[:-1], d // (2 * h), 2, h)
        a = yr[..., 0, :].copy()
        b = yr[..., 1, :].copy()
        yr[..., 0, :] = a + b
        yr[..., 1, :] = a - b
        y = yr.reshape(*y.shape)
        h *= 2
    return y


def rotate_fp32(x: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """``x R`` evaluated in fp32 in the fixed order described above."""
    d = x.shape[-1]
    y = x.astype(np.float32) * signs.astype(np.float32)
    y = _butterflies(y)
    return (y * np.float32(1.0 / np.sqrt(np.float64(d)))).astype(np.float32)


def unrotate_fp32(g: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """``g R^T`` in fp32: butterflies, scale, then signs."""
    d = g.shape[-1]
    y = _butterflies(g.astype(np.float32))
    y = y * np.float32(1.0 / np.sqrt(np.float64(d)))
    return (y * signs.astype(np.float32)).astype(np.float32)


def rotation_matrix(signs: np.ndarray) -> np.ndarray:
    """Dense fp64 ``R = diag(s) H / sqrt(d)``."""
    d = signs.shape[0]
    return (signs.astype(np.float64)[:, None] * sylvester(d)) / np.sqrt(d)
