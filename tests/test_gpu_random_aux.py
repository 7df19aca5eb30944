"""Seeded random sweeps of the paths beside the graph build, each against the CPU oracle:

* filter_edges_to_radius: random boxes (cubic, lower-triangular and general cells, full and
  partial PBC, fp32 and fp64 positions), random radius and skin, every shift dtype the API
  takes; the kept mask must equal the oracle's canonical-predicate mask edge for edge (so
  the output is the input's kept rows in order, shifts bit-equal), and the kept set must be
  the build at the smaller radius.
* SFC keys, order and partition labels: random point clouds (uniform, clustered,
  degenerate and huge-range axes, negative coordinates, duplicated points), both curves;
  keys bit-exact, the order a stable argsort of the oracle's keys, labels the oracle's.
"""
import numpy as np
import pytest
import torch

import oracle
from dynamis_amd.dynamis_state import dynamis_state_impl as impl

pytestmark = pytest.mark.gpu

SHIFT_DTYPES = [torch.float32, torch.float64, torch.int64, torch.int32, torch.float16, torch.bfloat16]


def _cell(rng, kind, L):
    if kind == "cubic":
        return np.eye(3) * L
    if kind == "lowtri":
        c = np.diag(L * rng.uniform(0.8, 1.2, 3))
        c[1, 0], c[2, 0], c[2, 1] = L * rng.uniform(-0.3, 0.3, 3)
        return c
    c = np.diag(L * rng.uniform(0.8, 1.2, 3)) + L * rng.uniform(-0.25, 0.25, (3, 3))
    return c


def _filter_case(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(300, 9000))
    rho = rng.uniform(0.03, 0.15)
    kind = ["cubic", "lowtri", "general"][seed % 3]
    L = (n / rho) ** (1.0 / 3.0)
    cell = _cell(rng, kind, L)
    pdt = np.float64 if seed % 4 == 1 else np.float32
    pos = (rng.uniform(-0.1, 1.1, (n, 3)) @ cell).astype(pdt)
    pbc = [(1, 1, 1), (1, 0, 1), (0, 0, 0), (1, 1, 0)][seed % 4]
    r = float(np.float32(rng.uniform(2.5, 7.0)))
    skin = float(np.float32(rng.uniform(0.1, 1.5)))
    sdt = SHIFT_DTYPES[seed % len(SHIFT_DTYPES)]
    return pos, cell, pbc, r, skin, sdt, kind


@pytest.mark.parametrize("seed", range(30))
def test_filter_random(cuda, seed):
    pos, cell, pbc, r, skin, sdt, kind = _filter_case(seed)
    print(f"\n[case] filter seed={seed} n={len(pos)} {kind} pbc={pbc} {pos.dtype} r={r} skin={skin} "
          f"shifts={sdt}", flush=True)
    p = torch.from_numpy(pos).to(cuda)
    c = torch.from_numpy(cell)
    b = torch.tensor([bool(x) for x in pbc])
    ei, co, _ = impl.radius_graph_pbc(p, c, b, r + skin, 0, False)
    sh = co.to(sdt)
    ef, cf = impl.filter_edges_to_radius(ei, sh, p, c, r)
    cell_used = cell.astype(pos.dtype).astype(np.float64)
    keep = oracle.filter_edges(pos, cell_used, r, ei[0].cpu().numpy(), ei[1].cpu().numpy(),
                               co.cpu().numpy().astype(np.int32))
    assert np.array_equal(ef.cpu().numpy(), ei.cpu().numpy()[:, keep])
    kt = torch.from_numpy(np.nonzero(keep)[0]).to(cuda)
    assert cf.dtype == sdt and torch.equal(cf, sh.index_select(0, kt))
    e2, c2, _ = impl.radius_graph_pbc(p, c, b, r, 0, False)
    g = oracle.canonical_sort(ef[0].cpu().numpy(), ef[1].cpu().numpy(), cf.float().cpu().numpy().astype(np.int64))
    w = oracle.canonical_sort(e2[0].cpu().numpy(), e2[1].cpu().numpy(), c2.cpu().numpy().astype(np.int64))
    assert all(np.array_equal(x, y) for x, y in zip(g, w))


def _cloud(seed):
    rng = np.random.default_rng(1000 + seed)
    n = int(rng.choice([1, 2, 3, 64, 1000, 4097, 30000, 120000]))
    kind = seed % 6
    if kind == 0:
        p = rng.uniform(-50, 80, (n, 3))
    elif kind == 1:  # clusters
        centres = rng.uniform(-100, 100, (7, 3))
        p = centres[rng.integers(0, 7, n)] + rng.normal(0, 2.0, (n, 3))
    elif kind == 2:  # a degenerate axis
        p = rng.uniform(0, 30, (n, 3))
        p[:, seed % 3] = -4.75
    elif kind == 3:  # huge range on one axis, tiny on another
        p = rng.uniform(0, 1, (n, 3)) * [1e5, 1e-3, 10.0]
    elif kind == 4:  # many duplicated points
        base = rng.uniform(-20, 20, (max(1, n // 50), 3))
        p = base[rng.integers(0, len(base), n)]
    else:  # a lattice (exact quantisation boundaries)
        k = int(np.ceil(n ** (1 / 3)))
        g = np.stack(np.meshgrid(np.arange(k), np.arange(k), np.arange(k), indexing="ij"), -1).reshape(-1, 3)
        p = g[:n] * 1.25
    return p.astype(np.float32)


@pytest.mark.parametrize("seed", range(24))
def test_sfc_random(cuda, seed):
    p = _cloud(seed)
    n = len(p)
    print(f"\n[case] sfc seed={seed} n={n}", flush=True)
    pt = torch.from_numpy(p).to(cuda)
    for curve in (0, 1):
        k = impl.sfc_keys(pt, curve).cpu().numpy()
        want = oracle.morton_keys(p) if curve == 0 else oracle.hilbert_keys(p)
        assert np.array_equal(k, want)
        perm = np.argsort(want, kind="stable")
        assert np.array_equal(impl.sfc_order(torch.from_numpy(want).to(cuda)).cpu().numpy(), perm)
        W = int(np.random.default_rng(seed).integers(1, 17))
        lab = impl.sfc_partition_cuda(pt, None, W, curve).cpu().numpy()
        assert np.array_equal(lab, oracle.sfc_labels(perm, W))
        w = np.random.default_rng(seed + 5).integers(0, 1000, n)
        labw = impl.sfc_partition_cuda(pt, torch.from_numpy(w).to(cuda), W, curve).cpu().numpy()
        assert np.array_equal(labw, oracle.sfc_labels(perm, W, w))
