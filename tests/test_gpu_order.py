"""Output order of the build where a bin or a tile bucket is too large for the LDS orderings:
a tile bucket of more than 2048 entries (tile-level sort), a bin of more than 128 atoms or
targets (per-bin sort, used above 36000 tiles).  Those segments are sorted in global memory
(dg_segsort.hpp), so the order of the output is a function of the input alone: atoms in a bin
by id, explicit targets in a bin by their position in the caller's list.  (Bins sorted in LDS
order the atoms of a lower-triangular cell by their offset along the a axis in the bin
first, then by id.)

Each case puts a clump of atoms, scattered over the atom ids, inside one bin of a uniform
box.  The clump's atoms then share one bin, so their first appearances as targets in
edge_index[1] must follow that order.  Each case is also checked against the oracle as an
edge set, and built twice with byte-identical results.
"""
import numpy as np
import pytest
import torch

import oracle
from dynamis_amd.dynamis_state import dynamis_state_impl as impl

pytestmark = pytest.mark.gpu


def _clump_box(n, L, r, n_clump, width, seed):
    """n atoms uniform in a cube of side L; n_clump of them (random ids) moved into a cube
    of side `width` around the centre of one bin (bins as the planner lays them out for a
    cube: floor(2 L / r) per axis, asserted to stay below its bin cap)."""
    nb = int(np.floor(2.0 * L / r * (1.0 - 1e-6)))
    assert nb ** 3 <= max(4 * n, 4096)
    h = L / nb
    assert width < 0.5 * h
    rng = np.random.default_rng(seed)
    pos = rng.uniform(0.0, L, (n, 3))
    ids = np.sort(rng.choice(n, n_clump, replace=False))
    centre = (np.array([nb // 3, nb // 2, (2 * nb) // 3]) + 0.5) * h
    pos[ids] = centre + rng.uniform(-0.5 * width, 0.5 * width, (n_clump, 3))
    return pos.astype(np.float32), np.eye(3) * L, ids


def _first_appearances(dst):
    return dst[np.r_[True, dst[1:] != dst[:-1]]] if len(dst) else dst


def _build(dev, pos, cell, r, targets):
    p = torch.from_numpy(pos).to(dev)
    t = None if targets is None else torch.from_numpy(targets).to(dev)
    return impl.radius_graph_pbc_ex(p, torch.from_numpy(cell), torch.tensor([True] * 3), r, 0, False, t)


def _check(dev, pos, cell, r, clump, targets=None):
    ei, co, nn, cnt = _build(dev, pos, cell, r, targets)
    ei2, co2, _, cnt2 = _build(dev, pos, cell, r, targets)
    assert torch.equal(ei, ei2) and torch.equal(co, co2) and torch.equal(cnt, cnt2)
    src, dst = ei[0].cpu().numpy(), ei[1].cpu().numpy()
    sh = co.cpu().numpy()
    o = oracle.radius_graph(pos, cell, (1, 1, 1), float(np.float32(r)), target_indices=targets)
    assert np.array_equal(cnt.cpu().numpy(), o["counts"])
    g = oracle.canonical_sort(src, dst, sh.astype(np.int64))
    w = oracle.canonical_sort(o["src"], o["dst"], o["shift"])
    assert all(np.array_equal(a, b) for a, b in zip(g, w))
    # order inside the clump's bin
    got = _first_appearances(dst)
    got = got[np.isin(got, clump)]
    if targets is None:
        want = clump  # by atom id
    else:
        want = _first_appearances(targets[np.isin(targets, clump)])  # by caller position
    assert np.array_equal(got, want)


def _targets(n, clump, seed):
    rng = np.random.default_rng(seed)
    others = rng.choice(np.setdiff1d(np.arange(n), clump), 2000, replace=False)
    t = np.concatenate([clump, clump[::3], others])
    return t[rng.permutation(len(t))].astype(np.int64)


def test_oversized_tile_bucket(cuda):
    """51200 atoms at 0.1 A^-3, r = 5, 3000 of them in a 0.3 A cube: the clump's tile
    bucket holds more than 2048 entries."""
    pos, cell, clump = _clump_box(51200, 80.0, 5.0, 3000, 0.3, seed=61)
    print("\n[case] oversized tile bucket, 3000-atom clump", flush=True)
    _check(cuda, pos, cell, 5.0, clump)


def test_oversized_tile_bucket_targets(cuda):
    """The same box with explicit targets: the clump's atoms (a third of them twice) and
    2000 others, in random order."""
    pos, cell, clump = _clump_box(51200, 80.0, 5.0, 3000, 0.3, seed=62)
    tg = _targets(len(pos), clump, seed=63)
    print(f"\n[case] oversized tile bucket, {len(tg)} explicit targets", flush=True)
    _check(cuda, pos, cell, 5.0, clump, tg)


def test_big_bin_per_bin_sort(cuda):
    """1.3M atoms at 1 A^-3, r = 1.28 (170^3 bins, 39304 tiles: the per-bin sort), 600 of
    them in a 0.2 A cube: a bin of more than 128 atoms."""
    pos, cell, clump = _clump_box(1_300_000, 1_300_000 ** (1 / 3), 1.28, 600, 0.2, seed=64)
    print("\n[case] per-bin sort, 600-atom bin", flush=True)
    _check(cuda, pos, cell, 1.28, clump)


def test_big_bin_per_bin_sort_targets(cuda):
    """The same with explicit targets: a bin of 800 targets."""
    pos, cell, clump = _clump_box(1_300_000, 1_300_000 ** (1 / 3), 1.28, 600, 0.2, seed=65)
    tg = _targets(len(pos), clump, seed=66)
    print(f"\n[case] per-bin sort, {len(tg)} explicit targets", flush=True)
    _check(cuda, pos, cell, 1.28, clump, tg)
