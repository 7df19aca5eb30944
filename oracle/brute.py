"""Brute-force edge set straight from the definition -- TEST INFRASTRUCTURE ONLY.

Edge set (the contract of the build; the reference's cell list enumerates the same set,
dynamis_state/src/csrc/graph/radius_graph_kernels.cu:18-141 + 197-258):

    {(i, j, S) : S in Z^3,  1e-8 < |p_i + S.C - p_j|^2 <= r^2,
                 S_d = floor(f_j,d) - floor(f_i,d) on every non-periodic axis d}

where f = p . C^-1 are fractional coordinates (the reference wraps every axis, periodic or
not, radius_graph_kernels.cu:603-605, so on a non-periodic axis only the wrapped images
can meet).  i is the source (edge_index[0]), j the target (edge_index[1]).

This uses numpy's own matrix inverse and plain (non-fused) float64 arithmetic, so it is
independent of the oracle's fixed fma order; pairs within ``amb`` of the cutoff (or of
the self-exclusion threshold) are reported separately as ambiguous instead of being
decided.
"""
from __future__ import annotations

import itertools
import math

import numpy as np

SELF_THR = float(np.float32(1e-8))


def brute_edges(pos, cell, pbc, radius, target_indices=None, amb=1e-9):
    pos = np.asarray(pos, dtype=np.float64)
    cell = np.asarray(cell, dtype=np.float64).reshape(3, 3)
    pbc = np.asarray(pbc, dtype=bool).reshape(3)
    n = pos.shape[0]
    tg = np.arange(n) if target_indices is None else np.asarray(target_indices, np.int64)
    r2 = float(radius) ** 2
    inv = np.linalg.inv(cell)
    frac = pos @ inv
    flo = np.floor(frac).astype(np.int64)
    # heights between lattice planes -> max |S_d| that can matter
    vol = abs(np.linalg.det(cell))
    rng = []
    for d in range(3):
        a, b = cell[(d + 1) % 3], cell[(d + 2) % 3]
        h = vol / np.linalg.norm(np.cross(a, b))
        k = int(math.ceil(radius / h)) + 1
        rng.append(range(-k, k + 1) if pbc[d] else [None])
    edges = set()
    ambiguous = set()
    for S0 in itertools.product(*rng):
        for t_slot, j in enumerate(tg):
            S = np.empty((n, 3), np.int64)
            for d in range(3):
                S[:, d] = S0[d] if pbc[d] else flo[j, d] - flo[:, d]
            v = pos + S @ cell - pos[j]
            d2 = np.einsum("ij,ij->i", v, v)
            inside = (d2 <= r2) & (d2 > SELF_THR)
            near = (np.abs(d2 - r2) < amb * max(1.0, r2)) | (np.abs(d2 - SELF_THR) < amb)
            for i in np.nonzero(inside & ~near)[0]:
                edges.add((int(i), int(j), int(S[i, 0]), int(S[i, 1]), int(S[i, 2])))
            for i in np.nonzero(near)[0]:
                ambiguous.add((int(i), int(j), int(S[i, 0]), int(S[i, 1]), int(S[i, 2])))
    return edges, ambiguous


def edge_set(src, dst, shift):
    shift = np.asarray(shift).astype(np.int64)
    return set(zip(np.asarray(src).tolist(), np.asarray(dst).tolist(),
                   shift[:, 0].tolist(), shift[:, 1].tolist(), shift[:, 2].tolist()))
