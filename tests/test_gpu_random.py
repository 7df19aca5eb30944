"""Seeded random sweep of the HIP build against the CPU oracle (bit-exact edge sets and
per-target counts after the canonical sort): random cells (cubic, orthorhombic,
lower-triangular, general, thin slabs), PBC patterns, radii from below one bin to several
cell widths, fp32 and fp64 positions, positions inside and outside the cell, atom counts
from 1 to tens of thousands, with and without explicit targets (prefix, random subsets
with duplicates); edge vectors and distances on a quarter of the cases.  Each case prints
its parameters before it runs."""
import numpy as np
import pytest
import torch

import oracle
from dynamis_amd.dynamis_state import dynamis_state_impl as impl

pytestmark = pytest.mark.gpu


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    kind = ["cubic", "ortho", "lowtri", "general", "slab"][seed % 5]
    L = rng.uniform(8.0, 60.0)
    if kind == "cubic":
        cell = np.eye(3) * L
    elif kind == "ortho":
        cell = np.diag(rng.uniform(0.5, 1.5, 3) * L)
    elif kind == "lowtri":
        cell = np.diag(rng.uniform(0.7, 1.3, 3) * L)
        cell[1, 0], cell[2, 0], cell[2, 1] = rng.uniform(-0.4, 0.4, 3) * L
    elif kind == "general":
        cell = np.eye(3) * L + rng.uniform(-0.3, 0.3, (3, 3)) * L
    else:
        cell = np.diag([L, L, rng.uniform(0.1, 0.3) * L])
    vol = abs(np.linalg.det(cell))
    n = int(min(max(1, rng.uniform(0.005, 0.12) * vol), 40000))
    pbc = tuple(bool(b) for b in rng.integers(0, 2, 3)) if seed % 3 else (True, True, True)
    dmin = vol / max(np.linalg.norm(np.cross(cell[1], cell[2])), np.linalg.norm(np.cross(cell[2], cell[0])),
                     np.linalg.norm(np.cross(cell[0], cell[1])))
    r = float(rng.choice([rng.uniform(0.5, 3.0), rng.uniform(3.0, 7.0), rng.uniform(0.5, 2.5) * dmin]))
    # keep the edge count modest (the oracle's lists are compared element by element)
    while n * (4.0 / 3.0 * np.pi * r ** 3 * n / vol) > 3e6 and n > 1:
        n = max(1, n // 2)
    lo, hi = (0.0, 1.0) if seed % 4 else (-1.5, 2.5)
    frac = rng.uniform(lo, hi, (n, 3))
    dtype = np.float64 if seed % 2 else np.float32
    pos = (frac @ cell).astype(dtype)
    tg = None
    if seed % 7 == 3:
        tg = np.arange(max(1, n // 2), dtype=np.int64)  # a prefix: the partition path
    elif seed % 7 == 5:
        tg = rng.integers(0, n, max(1, n // 3)).astype(np.int64)  # random, with duplicates
    return kind, cell, pbc, r, pos, tg


@pytest.mark.parametrize("seed", range(160))
def test_random_case(cuda, seed):
    kind, cell, pbc, r, pos, tg = _case(seed)
    print(f"\n[case] random seed={seed} kind={kind} n={len(pos)} dtype={pos.dtype} pbc={pbc} r={r:.3f} "
          f"targets={None if tg is None else len(tg)}", flush=True)
    pt = torch.from_numpy(np.ascontiguousarray(pos)).to(cuda)
    tt = None if tg is None else torch.from_numpy(tg).to(cuda)
    ei, co, nn, cnt = impl.radius_graph_pbc_ex(pt, torch.from_numpy(cell), torch.tensor(pbc), r, 0, False, tt)
    cell_used = np.asarray(cell, np.float64).astype(pos.dtype).astype(np.float64)
    o = oracle.radius_graph(pos, cell_used, pbc, float(np.float32(r)), target_indices=tg)
    assert ei.shape[1] == len(o["src"]) == int(nn.item())
    assert np.array_equal(cnt.cpu().numpy(), o["counts"])
    got = oracle.canonical_sort(ei[0].cpu().numpy(), ei[1].cpu().numpy(), co.cpu().numpy().astype(np.int64))
    want = oracle.canonical_sort(o["src"], o["dst"], o["shift"])
    for a, b in zip(got, want):
        assert np.array_equal(a, b)


def _brute_case(seed):
    """Cells much smaller than the radius (the all-pairs kernel): r = 4.5 - 7 times the
    thinnest cell width, positions inside or up to three cells outside the cell."""
    rng = np.random.default_rng(5000 + seed)
    L = rng.uniform(2.0, 5.0)
    cell = np.eye(3) * L
    if seed % 3 == 1:
        cell[1, 0], cell[2, 0], cell[2, 1] = rng.uniform(-0.3, 0.3, 3) * L
    elif seed % 3 == 2:
        cell = cell + rng.uniform(-0.25, 0.25, (3, 3)) * L
    vol = abs(np.linalg.det(cell))
    dmin = vol / max(np.linalg.norm(np.cross(cell[1], cell[2])), np.linalg.norm(np.cross(cell[2], cell[0])),
                     np.linalg.norm(np.cross(cell[0], cell[1])))
    r = float(rng.uniform(4.5, 7.0) * dmin)
    n = int(rng.integers(1, 40))
    pbc = (True, True, True) if seed % 2 else tuple(bool(b) for b in rng.integers(0, 2, 3))
    lo, hi = (0.0, 1.0) if seed % 4 == 0 else (-3.0, 4.0)
    pos = (rng.uniform(lo, hi, (n, 3)) @ cell).astype(np.float64 if seed % 2 else np.float32)
    tg = rng.integers(0, n, max(1, n // 2)).astype(np.int64) if seed % 5 == 4 else None
    return cell, pbc, r, pos, tg


@pytest.mark.parametrize("seed", range(24))
def test_random_all_pairs(cuda, seed):
    cell, pbc, r, pos, tg = _brute_case(seed)
    print(f"\n[case] random all-pairs seed={seed} n={len(pos)} dtype={pos.dtype} pbc={pbc} r={r:.3f} "
          f"targets={None if tg is None else len(tg)}", flush=True)
    pt = torch.from_numpy(np.ascontiguousarray(pos)).to(cuda)
    tt = None if tg is None else torch.from_numpy(tg).to(cuda)
    ei, co, nn, cnt = impl.radius_graph_pbc_ex(pt, torch.from_numpy(cell), torch.tensor(pbc), r, 0, False, tt)
    cell_used = np.asarray(cell, np.float64).astype(pos.dtype).astype(np.float64)
    o = oracle.radius_graph(pos, cell_used, pbc, float(np.float32(r)), target_indices=tg)
    assert ei.shape[1] == len(o["src"]) == int(nn.item())
    assert np.array_equal(cnt.cpu().numpy(), o["counts"])
    got = oracle.canonical_sort(ei[0].cpu().numpy(), ei[1].cpu().numpy(), co.cpu().numpy().astype(np.int64))
    want = oracle.canonical_sort(o["src"], o["dst"], o["shift"])
    for a, b in zip(got, want):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("seed", range(40))
def test_random_vectors(cuda, seed):
    """Edge vectors and distances on the sweep's cases (every fourth seed, so every cell
    kind, PBC pattern, target kind and position dtype comes up), fp32 and fp64 vectors in
    turn: fp64 bit-identical to the canonical formula, fp32 its rounding, distances within
    1e-15 relative (fp64) or 2 ulp (fp32) of the oracle's."""
    kind, cell, pbc, r, pos, tg = _case(4 * seed + seed % 4)
    vdt = torch.float64 if seed % 2 else torch.float32
    print(f"\n[case] random vectors seed={seed} kind={kind} n={len(pos)} dtype={pos.dtype} pbc={pbc} "
          f"r={r:.3f} targets={None if tg is None else len(tg)} vectors={vdt}", flush=True)
    pt = torch.from_numpy(np.ascontiguousarray(pos)).to(cuda)
    tt = None if tg is None else torch.from_numpy(tg).to(cuda)
    ei, co, nn, cnt, vec, dist = impl.radius_graph_pbc_vectors(pt, torch.from_numpy(cell), torch.tensor(pbc), r,
                                                               tt, vector_dtype=vdt)
    cell_used = np.asarray(cell, np.float64).astype(pos.dtype).astype(np.float64)
    o = oracle.radius_graph(pos, cell_used, pbc, float(np.float32(r)), target_indices=tg, vectors=True)
    assert ei.shape[1] == len(o["src"]) == int(nn.item())
    assert np.array_equal(cnt.cpu().numpy(), o["counts"])
    got = oracle.canonical_sort(ei[0].cpu().numpy(), ei[1].cpu().numpy(), co.cpu().numpy().astype(np.int64),
                                vec.cpu().numpy(), dist.cpu().numpy())
    want = oracle.canonical_sort(o["src"], o["dst"], o["shift"], o["vec"], np.sqrt(o["d2"]))
    for a, b in zip(got[:3], want[:3]):
        assert np.array_equal(a, b)
    if vdt == torch.float64:
        assert np.array_equal(got[3], want[3])
        assert np.allclose(got[4], want[4], rtol=1e-15, atol=0)
    else:
        assert np.array_equal(got[3], want[3].astype(np.float32))
        ulp = np.spacing(want[4].astype(np.float32))
        assert np.all(np.abs(got[4].astype(np.float64) - want[4]) <= 2 * ulp)
