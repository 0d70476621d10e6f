"""Exhaustive tile classification of a dense mask (test oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

The reference has no tile map: every kernel re-evaluates the mask formula on
every visited tile (``original_kernel.py:424-517``).  The tile map is the
build's own structure; this module defines it from the dense mask by brute
reduction so the device classifier can be checked bit-exactly.

Class codes: 0 = EMPTY (no allowed entry), 1 = PARTIAL, 2 = FULL (every entry
allowed).  Entries outside ``[0, T)`` count as not allowed, so a tile that
crosses T is never FULL.  Block lists join ``R`` consecutive base tiles; a base
tile index past the end counts as EMPTY.
"""
from __future__ import annotations

import numpy as np

EMPTY, PARTIAL, FULL = 0, 1, 2


def classify(mask: np.ndarray, tile: int = 64) -> np.ndarray:
    """``[B, nT, nT]`` uint8 class map of a boolean ``[B, T, T]`` mask."""
    B, T, _ = mask.shape
    n = -(-T // tile)
    pad = np.zeros((B, n * tile, n * tile), dtype=bool)
    pad[:, :T, :T] = mask
    tiles = pad.reshape(B, n, tile, n, tile)
    cnt = tiles.sum(axis=(2, 4))
    out = np.full((B, n, n), PARTIAL, dtype=np.uint8)
    out[cnt == 0] = EMPTY
    out[cnt == tile * tile] = FULL
    return out


def _combine(classes: np.ndarray) -> np.ndarray:
    """Class of the union of base tiles along the last axis."""
    anyne = (classes != EMPTY).any(axis=-1)
    allfull = (classes == FULL).all(axis=-1)
    out = np.where(anyne, PARTIAL, EMPTY).astype(np.uint8)
    out[allfull] = FULL
    return out


def q_lists(cls: np.ndarray, rq: int):
    """Per q-block (``rq`` base q-tiles) list of non-empty base k-tiles.

    Returns ``(entries [B, nQB, nK] uint32, counts [B, nQB] int32)``; entry =
    ``(k_tile << 8) | sum_r class(q-tile rq*block + r, k_tile) << 2r`` in
    ascending k order, zero padded; a member past the last tile is EMPTY.
    """
    B, nQ, nK = cls.shape
    nqb = -(-nQ // rq)
    pad = np.full((B, nqb * rq, nK), EMPTY, dtype=np.uint8)
    pad[:, :nQ] = cls
    grp = pad.reshape(B, nqb, rq, nK).transpose(0, 1, 3, 2)  # [B, nqb, nK, rq]
    comb = _combine(grp)
    members = np.zeros((B, nqb, nK), dtype=np.uint32)
    for r in range(rq):
        members |= grp[..., r].astype(np.uint32) << (2 * r)
    entries = np.zeros((B, nqb, nK), dtype=np.uint32)
    counts = np.zeros((B, nqb), dtype=np.int32)
    for b in range(B):
        for q in range(nqb):
            ks = np.nonzero(comb[b, q] != EMPTY)[0]
            counts[b, q] = len(ks)
            entries[b, q, :len(ks)] = (ks.astype(np.uint32) << 8) | members[b, q, ks]
    return entries, counts


def k_lists(cls: np.ndarray, rk: int):
    """Per k-block (``rk`` base k-tiles) list of non-empty base q-tiles.

    Returns ``(entries [B, nKB, nQ] uint32, counts [B, nKB] int32)``; entry =
    ``(q_tile << 8) | sum_r class(q_tile, k-tile rk*block + r) << 2r``.
    """
    return q_lists(np.ascontiguousarray(cls.transpose(0, 2, 1)), rk)


def tile_bits(mask: np.ndarray, tile: int = 64):
    """Row and column bit masks of every 64x64 tile of a ``[B, T, T]`` mask.

    Returns ``(qbits, kbits)``, both ``[B, nT, nT, 64]`` uint64: ``qbits[b, qt,
    kt, r]`` has bit ``j`` set iff query ``64 qt + r`` may see key ``64 kt + j``;
    ``kbits[b, qt, kt, r]`` has bit ``i`` set iff query ``64 qt + i`` may see key
    ``64 kt + r``.  Entries past T are not allowed.
    """
    B, T, _ = mask.shape
    n = -(-T // tile)
    pad = np.zeros((B, n * tile, n * tile), dtype=bool)
    pad[:, :T, :T] = mask
    tiles = pad.reshape(B, n, tile, n, tile).transpose(0, 1, 3, 2, 4)  # [B, qt, kt, row, col]
    weights = np.left_shift(np.uint64(1), np.arange(tile, dtype=np.uint64))
    qbits = (tiles.astype(np.uint64) * weights).sum(axis=-1, dtype=np.uint64)
    kbits = (tiles.transpose(0, 1, 2, 4, 3).astype(np.uint64) * weights).sum(axis=-1, dtype=np.uint64)
    return qbits, kbits


def useful_entries(mask: np.ndarray) -> int:
    """Number of allowed (i, j) entries over the batch (per head)."""
    return int(mask.sum())
