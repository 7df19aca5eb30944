"""Pins the CPU oracle (oracle/graph_oracle.c) before it is trusted as the checker.

Each check is independent of the oracle's own formula: brute force from the definition
(numpy inverse, unfused fp64), scipy's cKDTree, closed-form lattice counts, the known
answers of the reference's own tests (dynamis_state/tests/test_radius_graph_pbc_cuda.py),
and invariants (symmetry, filter consistency)."""
import numpy as np
import pytest

import oracle
from oracle.brute import brute_edges, edge_set
from dynamis_amd import configs


def _rand_case(rng, kind):
    n = int(rng.integers(4, 45))
    L = rng.uniform(5.0, 16.0)
    cell = np.eye(3) * L * rng.uniform(0.8, 1.2, 3)
    if kind in ("tri", "tri_partial"):
        cell = cell + np.tril(rng.uniform(-0.3, 0.3, (3, 3)) * L, -1)
    pbc = {"ortho": (1, 1, 1), "tri": (1, 1, 1), "partial": (1, 1, 0), "tri_partial": (0, 1, 1),
           "none": (0, 0, 0)}[kind]
    frac = rng.uniform(-0.3, 1.3, (n, 3))  # some atoms outside the cell: exercises the wrap
    pos = frac @ cell
    r = rng.uniform(1.5, 8.0)
    return pos, cell, pbc, r


@pytest.mark.parametrize("kind", ["ortho", "tri", "partial", "tri_partial", "none"])
@pytest.mark.parametrize("seed", range(4))
def test_oracle_matches_brute_force(kind, seed):
    rng = np.random.default_rng(100 * seed + ["ortho", "tri", "partial", "tri_partial", "none"].index(kind))
    pos, cell, pbc, r = _rand_case(rng, kind)
    for dt in (np.float64, np.float32):
        p = pos.astype(dt)
        o = oracle.radius_graph(p, cell.astype(dt).astype(np.float64), pbc, r)
        want, amb = brute_edges(p, cell.astype(dt), pbc, r)
        got = edge_set(o["src"], o["dst"], o["shift"])
        assert got - amb == want
        assert len(o["src"]) == int(o["counts"].sum())


def test_oracle_target_subset_matches_brute_force():
    rng = np.random.default_rng(7)
    pos, cell, pbc, r = _rand_case(rng, "tri")
    tg = rng.choice(pos.shape[0], size=pos.shape[0] // 2, replace=False)
    o = oracle.radius_graph(pos, cell, pbc, r, target_indices=tg)
    want, amb = brute_edges(pos, cell, pbc, r, target_indices=tg)
    assert edge_set(o["src"], o["dst"], o["shift"]) - amb == want
    # counts in target_indices order
    for t, a in enumerate(tg):
        assert o["counts"][t] == int(np.sum(o["dst"] == a))


def test_reference_known_answers():
    # test_radius_graph_pbc_cuda.py:270-288: one atom, box 5, r 6 -> exactly 6 edges
    o = oracle.radius_graph(np.array([[2.5, 2.5, 2.5]], np.float32), np.eye(3) * 5.0, (1, 1, 1), 6.0)
    assert len(o["src"]) == 6
    assert np.all(o["src"] == 0) and np.all(o["dst"] == 0)
    assert not np.any(np.all(o["shift"] == 0, axis=1))
    assert sorted(map(tuple, o["shift"].tolist())) == sorted(
        [(1, 0, 0), (-1, 0, 0), (0, 1, 0), (0, -1, 0), (0, 0, 1), (0, 0, -1)])
    # :290-297 single atom without PBC -> 0 edges
    o = oracle.radius_graph(np.array([[5.0, 5.0, 5.0]], np.float32), np.eye(3) * 10.0, (0, 0, 0), 5.0)
    assert len(o["src"]) == 0
    # :260-268 empty
    o = oracle.radius_graph(np.zeros((0, 3), np.float32), np.eye(3), (1, 1, 1), 5.0)
    assert len(o["src"]) == 0


def test_fcc_closed_form():
    # perfect FCC a=3.6, r=6: shells 12+6+24+12+24 = 78 neighbours (next shell 6.235 A)
    box = configs.fcc(jitter=0.0)
    o = oracle.radius_graph(box.pos, box.cell, box.pbc, box.radius)
    assert len(o["src"]) == 864 * 78
    assert np.all(o["counts"] == 78)
    _, d2 = oracle.edge_vectors(box.pos, box.cell, o["src"], o["dst"], o["shift"])
    shells = np.unique(np.round(np.sqrt(d2), 6))
    assert np.allclose(shells, 3.6 * np.sqrt([0.5, 1.0, 1.5, 2.0, 2.5]), atol=1e-9)


def test_exact_cutoff_lattice():
    # simple cubic spacing 2, r = 4: |n|^2 <= 4 -> 6 + 12 + 8 + 6 = 32 neighbours; the
    # (+-2,0,0) shell sits exactly on the cutoff and must be included (d2 <= r^2)
    g = np.stack(np.meshgrid(*[np.arange(6)] * 3, indexing="ij"), -1).reshape(-1, 3) * 2.0
    for dt in (np.float32, np.float64):
        o = oracle.radius_graph(g.astype(dt), np.eye(3) * 12.0, (1, 1, 1), 4.0)
        assert np.all(o["counts"] == 32)


def test_cross_check_ckdtree():
    from scipy.spatial import cKDTree

    box = configs.uniform(3000, seed=11, dtype=np.float64)
    L = box.cell[0, 0]
    o = oracle.radius_graph(box.pos, box.cell, box.pbc, box.radius)
    t = cKDTree(box.pos, boxsize=L)
    pairs = t.query_pairs(box.radius, output_type="ndarray")
    assert len(o["src"]) == 2 * len(pairs)
    got = set(zip(o["src"].tolist(), o["dst"].tolist()))
    for i, j in pairs[:2000]:
        assert (int(i), int(j)) in got and (int(j), int(i)) in got


def test_symmetry_and_vectors():
    box = configs.c4(scale=0.25)
    o = oracle.radius_graph(box.pos, box.cell, box.pbc, box.radius, vectors=True)
    fwd = edge_set(o["src"], o["dst"], o["shift"])
    rev = edge_set(o["dst"], o["src"], -o["shift"])
    assert fwd == rev
    assert np.all(o["d2"] <= box.radius ** 2) and np.all(o["d2"] > 1e-8)
    # vector closed form: v = pos[src] + S.cell - pos[dst]
    v = box.pos[o["src"]] + o["shift"] @ box.cell - box.pos[o["dst"]]
    assert np.allclose(v, o["vec"], rtol=0, atol=1e-10)


def test_filter_consistency():
    box = configs.uniform(2000, seed=5, dtype=np.float32)
    big = oracle.radius_graph(box.pos, box.cell, box.pbc, 6.5)
    small = oracle.radius_graph(box.pos, box.cell, box.pbc, 6.0)
    keep = oracle.filter_edges(box.pos, box.cell, 6.0, big["src"], big["dst"], big["shift"])
    a = edge_set(big["src"][keep], big["dst"][keep], big["shift"][keep])
    assert a == edge_set(small["src"], small["dst"], small["shift"])


def _decode_morton(k):
    x = y = z = 0
    for i in range(21):
        x |= ((k >> (3 * i)) & 1) << i
        y |= ((k >> (3 * i + 1)) & 1) << i
        z |= ((k >> (3 * i + 2)) & 1) << i
    return x, y, z


def test_morton_keys_pins():
    rng = np.random.default_rng(3)
    pos = rng.uniform(-50, 50, (2000, 3)).astype(np.float32)
    mn, rg = oracle.sfc_bounds(pos)
    assert np.array_equal(mn, pos.min(0)) and np.allclose(rg, pos.max(0) - pos.min(0))
    keys = oracle.morton_keys(pos, mn, rg)
    gm = np.float32(2 ** 21 - 1)
    q = np.minimum((((pos - mn) / rg) * gm).astype(np.uint32), 2 ** 21 - 1)
    for i in range(0, 2000, 7):
        assert _decode_morton(int(keys[i])) == tuple(int(v) for v in q[i])
    # corners: min -> 0, max -> all 63 bits set
    assert keys[np.argmin(pos.sum(1))] >= 0
    corner = np.array([[0, 0, 0], [1, 1, 1]], np.float32)
    k2 = oracle.morton_keys(corner)
    assert k2[0] == 0 and k2[1] == (1 << 63) - 1


def test_hilbert_keys_properties():
    rng = np.random.default_rng(4)
    pos = rng.uniform(0, 10, (5000, 3)).astype(np.float32)
    k = oracle.hilbert_keys(pos)
    assert k.min() >= 0 and k.max() < 2 ** 21
    # bit level 0 passes the quantised coordinates' low bits straight through
    mn, rg = oracle.sfc_bounds(pos)
    q = np.clip((((pos - mn) / rg) * np.float32(127)).astype(np.int64), 0, 127)
    assert np.array_equal(k & 7, (q[:, 0] & 1) | ((q[:, 1] & 1) << 1) | ((q[:, 2] & 1) << 2))


def test_sfc_labels_closed_form():
    n, W = 103, 4
    perm = np.random.default_rng(0).permutation(n)
    lab = oracle.sfc_labels(perm, W)
    counts = np.bincount(lab, minlength=W)
    assert counts.tolist() == [26, 26, 26, 25]
    # sorted position i gets partition of i
    assert np.all(np.diff(lab[perm]) >= 0)
    # weighted: exact integer cut floor(cumsum * W / total)
    w = np.ones(n, np.int64)
    w[perm[:3]] = 100
    lw = oracle.sfc_labels(perm, W, w)
    cs = np.cumsum(w[perm])
    assert np.array_equal(lw[perm], np.minimum(cs * W // cs[-1], W - 1))


def test_hilbert_exhaustive_vs_cpu_twin():
    """Every one of the 128^3 quantised cells: the oracle (restating the CUDA kernel,
    sfc_kernels.cu:62-109) equals the restatement of the reference's CPU twin
    (sfc_partitioner.cpp:50-92)."""
    from oracle import sfc_twin

    pos, X, Y, Z = sfc_twin.grid_positions(128, 1.0)
    k = oracle.hilbert_keys(pos)[:-2]
    assert np.array_equal(k, sfc_twin.hilbert_from_grid(X, Y, Z))
    assert len(np.unique(k)) < len(k)  # the transform is not injective; equality is the pin


def test_morton_grid_vs_cpu_twin():
    from oracle import sfc_twin

    # Morton quantises by 2^21 - 1: a 2^21-1 wide box makes cell centres land on integers
    rng = np.random.default_rng(2)
    cells = rng.integers(0, 2 ** 21 - 1, (20000, 3))
    pos = np.concatenate([(cells + 0.5), np.zeros((1, 3)), np.full((1, 3), 2 ** 21 - 1.0)])
    # fp32 cannot hold 2^21 + 0.5 exactly; quantise in double on the CPU-twin side instead
    p32 = pos.astype(np.float32)
    mn, rg = oracle.sfc_bounds(p32)
    q = np.clip(((p32.astype(np.float32) - mn) / rg * np.float32(2 ** 21 - 1)).astype(np.float32)
                .astype(np.int64), 0, 2 ** 21 - 1)
    k = oracle.morton_keys(p32)
    assert np.array_equal(k, sfc_twin.morton_from_grid(q[:, 0], q[:, 1], q[:, 2]))
