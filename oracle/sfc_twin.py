"""Second restatement of the SFC keys (TEST INFRASTRUCTURE ONLY), following the
reference's CPU fallback dynamis_state/src/csrc/partition/sfc_partitioner.cpp:21-92
(torch.where chains over bit planes) rather than the CUDA kernel that oracle/graph_oracle.c
follows (sfc_kernels.cu:19-109).  Vectorised numpy over quantised grid coordinates; used to
pin the oracle's (and the GPU's) keys exhaustively over all 128^3 "Hilbert" cells and a
sample of Morton cells."""
from __future__ import annotations

import numpy as np


def hilbert_from_grid(x, y, z, order: int = 7):
    """sfc_partitioner.cpp:66-90 on integer grid coordinates in [0, 2^order)."""
    x = np.asarray(x, np.int64)
    y = np.asarray(y, np.int64)
    z = np.asarray(z, np.int64)
    out = np.zeros(x.shape, np.int64)
    for i in range(order):
        xb, yb, zb = (x >> i) & 1, (y >> i) & 1, (z >> i) & 1
        if i == 0:
            bx, by, bz = xb, yb, zb
        else:
            xm, ym, zm = xb.astype(bool), yb.astype(bool), zb.astype(bool)
            bx = np.where(xm, zb, xb)
            by = np.where(xm, yb, np.where(ym, zb, yb))
            bz = np.where(xm, yb, np.where(ym, xb, np.where(zm, yb, zb)))
        out |= (bx << (3 * i)) | (by << (3 * i + 1)) | (bz << (3 * i + 2))
    return out


def morton_from_grid(x, y, z, bits: int = 21):
    """sfc_partitioner.cpp:21-45: bit i of x/y/z goes to bit 3i / 3i+1 / 3i+2."""
    x = np.asarray(x, np.int64)
    y = np.asarray(y, np.int64)
    z = np.asarray(z, np.int64)
    out = np.zeros(x.shape, np.int64)
    for i in range(bits):
        out |= (((x >> i) & 1) << (3 * i)) | (((y >> i) & 1) << (3 * i + 1)) | (((z >> i) & 1) << (3 * i + 2))
    return out


def grid_positions(n: int, scale: float):
    """fp32 positions whose keys quantise to the integer grid cells (x, y, z), 0 <= x < n:
    cell centres (x + 0.5) * scale plus the two bounding corners 0 and (n - 1) * scale, so
    that the data's min is 0 and its range is (n - 1) * scale (the quantisation multiplies
    by 2^order - 1 = n - 1 for "Hilbert")."""
    g = np.arange(n, dtype=np.int64)
    X, Y, Z = np.meshgrid(g, g, g, indexing="ij")
    X, Y, Z = X.ravel(), Y.ravel(), Z.ravel()
    pos = np.stack([X, Y, Z], 1).astype(np.float64) + 0.5
    pos = np.concatenate([pos, np.zeros((1, 3)), np.full((1, 3), float(n - 1))]) * scale
    return pos.astype(np.float32), X, Y, Z
