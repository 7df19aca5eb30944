"""Writes the golden edge lists in this folder (graph_*.npz).

Each case is a small periodic system; its expected edges come from the definition of the
edge set alone -- every atom pair and every integer image shift S on the periodic axes
with |S_d| <= ceil(r / d_face_d) + 1, v = p_src + S . C - p_dst in fp64, edge iff
1e-8 < |v|^2 <= r^2 (atoms inside the cell, so S_d = 0 on non-periodic axes) -- with no
cell list, no oracle and no library code.  Systems are drawn until no pair lies within
1e-6 A^2 of the cutoff, so the fp64 summation order cannot matter.  The reference's own
known answer (one atom in a 5 A box, r = 6 -> the 6 face images; test_radius_graph_pbc_
cuda.py:270-288) is the first case.

    python tests/golden/make_golden.py
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def definition_edges(frac, cell, pbc, r):
    pos = frac @ cell
    n = len(pos)
    inv = np.linalg.inv(cell)
    dface = 1.0 / np.linalg.norm(inv, axis=0)
    m = [int(np.ceil(r / dface[d])) + 1 if pbc[d] else 0 for d in range(3)]
    rng = [np.arange(-m[d], m[d] + 1) for d in range(3)]
    S = np.stack(np.meshgrid(*rng, indexing="ij"), -1).reshape(-1, 3)
    out, near = [], 0
    for i in range(n):  # i = source, j = target
        v = pos[i][None, None, :] + (S @ cell)[None, :, :] - pos[:, None, :]  # [j, S, 3]
        d2 = np.sum(v * v, axis=-1)
        near += int(np.sum(np.abs(d2 - r * r) < 1e-6))
        jj, ss = np.nonzero((d2 > 1e-8) & (d2 <= r * r))
        for j, s in zip(jj, ss):
            out.append((i, j, *S[s]))
    e = np.array(out, np.int64).reshape(-1, 5)
    order = np.lexsort((e[:, 4], e[:, 3], e[:, 2], e[:, 0], e[:, 1]))
    return e[order], near


def case(name, cell, pbc, r, n, seed, frac=None):
    rng = np.random.default_rng(seed)
    for attempt in range(100):
        f = frac if frac is not None else rng.uniform(0.0, 1.0, (n, 3))
        e, near = definition_edges(f, np.asarray(cell, float), pbc, r)
        if near == 0:
            break
        assert frac is None, "fixed frac has a pair on the cutoff"
    pos = f @ np.asarray(cell, float)
    np.savez(os.path.join(HERE, f"graph_{name}.npz"), pos=pos, cell=np.asarray(cell, float),
             pbc=np.asarray(pbc, np.int8), radius=np.float64(r), src=e[:, 0], dst=e[:, 1],
             shift=e[:, 2:])
    print(f"{name}: {len(pos)} atoms, {len(e)} edges")


if __name__ == "__main__":
    case("single_atom_box5", np.eye(3) * 5.0, (1, 1, 1), 6.0, 1, 0, frac=np.full((1, 3), 0.5))
    case("triclinic_lowtri", [[9.0, 0, 0], [2.0, 8.5, 0], [-1.0, 1.5, 10.0]], (1, 1, 1), 4.25, 40, 1)
    case("triclinic_general", [[7.0, 1.0, 0.5], [-0.8, 8.0, 1.2], [0.6, -1.1, 9.0]], (1, 1, 1), 3.75, 30, 2)
    case("partial_pbc", np.diag([8.0, 9.0, 7.0]), (1, 0, 1), 3.5, 30, 3)
    case("small_box_many_images", np.eye(3) * 3.2, (1, 1, 1), 5.5, 6, 4)
    case("no_pbc", np.diag([10.0, 11.0, 9.0]), (0, 0, 0), 4.0, 40, 5)
