"""GPU parity of the radius graph: HIP path (through the C ABI) vs the pinned CPU oracle.

Integer outputs (src, dst, integer shifts, per-target counts) must be bit-identical after
the canonical (src, dst, shift) sort; edge vectors fp64 bit-identical (same canonical
formula), fp32 = fp64 correctly rounded, distances within 1 ulp.  Cases follow the
reference's own tests (dynamis_state/tests/test_radius_graph_pbc_cuda.py) plus the
benchmark configurations and the corner cases of this design (multi-chunk regions,
oversized targets, the all-pairs fallback, wrapped positions, explicit targets).
"""
import numpy as np
import pytest
import torch

import oracle
from dynamis_amd import configs
from dynamis_amd.dynamis_state import dynamis_state_impl as impl
from dynamis_amd.dynamis_state import radius_graph_pbc_cuda

pytestmark = pytest.mark.gpu


def _announce(name):
    print(f"\n[case] {name}", flush=True)


def _gpu_build(pos, cell, pbc, r, targets, dev, vectors=False, vdt=None):
    pt = torch.from_numpy(np.ascontiguousarray(pos)).to(dev)
    ct = torch.from_numpy(np.asarray(cell, np.float64))
    bt = torch.tensor([bool(x) for x in pbc])
    tt = None if targets is None else torch.from_numpy(np.asarray(targets, np.int64)).to(dev)
    if vectors:
        return impl.radius_graph_pbc_vectors(pt, ct, bt, r, tt, vector_dtype=vdt)
    return impl.radius_graph_pbc_ex(pt, ct, bt, r, 0, False, tt)


def check_parity(pos, cell, pbc, r, dev, targets=None, name=""):
    _announce(f"{name} N={len(pos)} dtype={pos.dtype} pbc={pbc} r={r}")
    r32 = float(np.float32(r))
    ei, co, nn, cnt = _gpu_build(pos, cell, pbc, r, targets, dev)
    torch.cuda.synchronize()
    cell_used = np.asarray(cell, np.float64).astype(pos.dtype).astype(np.float64)
    o = oracle.radius_graph(pos, cell_used, pbc, r32, target_indices=targets)
    E = ei.shape[1]
    assert E == len(o["src"]), f"edge count {E} vs oracle {len(o['src'])}"
    assert int(nn.item()) == E
    assert np.array_equal(cnt.cpu().numpy(), o["counts"])
    src, dst = ei[0].cpu().numpy(), ei[1].cpu().numpy()
    sh = co.cpu().numpy()
    assert np.array_equal(sh, np.round(sh))
    g = oracle.canonical_sort(src, dst, sh.astype(np.int64))
    w = oracle.canonical_sort(o["src"], o["dst"], o["shift"])
    for a, b in zip(g, w):
        assert np.array_equal(a, b)
    return ei, co, cnt, o


def _rand(n, L, seed, dtype=np.float32, lo=0.0, hi=1.0, cell=None):
    rng = np.random.default_rng(seed)
    c = np.eye(3) * L if cell is None else np.asarray(cell, float)
    return (rng.uniform(lo, hi, (n, 3)) @ c).astype(dtype), c


# ---- reference test cases (test_radius_graph_pbc_cuda.py:113-393) ----------------------
@pytest.mark.parametrize("n,L,r,seed", [(8, 10.0, 3.0, 42), (100, 20.0, 5.0, 123), (10, 8.0, 6.0, 7),
                                        (20, 10.0, 4.0, 42), (1000, 30.0, 5.0, 2024), (50, 15.0, 4.0, 42)])
def test_reference_cubic_cases(cuda, n, L, r, seed):
    pos, cell = _rand(n, L, seed)
    check_parity(pos, cell, (1, 1, 1), r, cuda, name="cubic")


def test_reference_triclinic(cuda):
    cell = np.array([[15.0, 0.0, 0.0], [3.0, 14.0, 0.0], [1.0, 2.0, 13.0]])
    pos, _ = _rand(20, 1.0, 99, cell=cell)
    check_parity(pos, cell, (1, 1, 1), 5.0, cuda, name="triclinic")


def test_reference_partial_and_no_pbc(cuda):
    pos, cell = _rand(30, 15.0, 55)
    check_parity(pos, cell, (1, 1, 0), 4.0, cuda, name="pbc xy")
    pos, cell = _rand(25, 20.0, 77)
    check_parity(pos, cell, (0, 0, 0), 5.0, cuda, name="no pbc")


def test_reference_edge_cases(cuda):
    _announce("empty / single atom")
    ei, co, nn = impl.radius_graph_pbc(torch.empty(0, 3, device=cuda), torch.eye(3),
                                       torch.tensor([True] * 3), 5.0, 100, False)
    assert ei.shape == (2, 0) and co.shape == (0, 3)
    pos = torch.tensor([[2.5, 2.5, 2.5]], device=cuda)
    ei, co, nn = impl.radius_graph_pbc(pos, torch.eye(3) * 5.0, torch.tensor([True] * 3), 6.0, 100, False)
    assert ei.size(1) == 6 and torch.all(ei == 0)
    assert not torch.any(co.abs().sum(1) == 0)
    pos = torch.tensor([[5.0, 5.0, 5.0]], device=cuda)
    ei, co, nn = impl.radius_graph_pbc(pos, torch.eye(3) * 10.0, torch.tensor([False] * 3), 5.0, 100, False)
    assert ei.size(1) == 0
    # indices in range (test_source_count_less_than_full)
    p, c = _rand(100, 50.0, 42)
    ei, co, nn = impl.radius_graph_pbc(torch.from_numpy(p).to(cuda), torch.from_numpy(c),
                                       torch.tensor([True] * 3), 6.0, 1000, False)
    assert ei.size(1) > 0 and int(ei.min()) >= 0 and int(ei.max()) < 100


def test_wrapper_batch(cuda):
    _announce("wrapper batch of 2")
    p1, c1 = _rand(40, 12.0, 1)
    p2, c2 = _rand(30, 10.0, 2)

    class D:
        pass

    d = D()
    d.pos = torch.from_numpy(np.concatenate([p1, p2])).to(cuda)
    d.cell = torch.from_numpy(np.stack([c1, c2]).astype(np.float32)).to(cuda)
    d.natoms = torch.tensor([40, 30])
    d.pbc = torch.tensor([[True, True, True], [True, True, True]])
    ei, co, nn = radius_graph_pbc_cuda(d, 4.0, 0)
    o1 = oracle.radius_graph(p1, c1, (1, 1, 1), 4.0)
    o2 = oracle.radius_graph(p2, c2, (1, 1, 1), 4.0)
    assert nn.tolist() == [len(o1["src"]), len(o2["src"])]
    want = oracle.canonical_sort(np.r_[o1["src"], o2["src"] + 40], np.r_[o1["dst"], o2["dst"] + 40],
                                 np.r_[o1["shift"], o2["shift"]])
    got = oracle.canonical_sort(ei[0].cpu().numpy(), ei[1].cpu().numpy(), co.cpu().numpy().astype(np.int64))
    for a, b in zip(got, want):
        assert np.array_equal(a, b)


# ---- benchmark configurations -----------------------------------------------------
def test_c1_fcc(cuda):
    box = configs.fcc()
    check_parity(box.pos, box.cell, box.pbc, box.radius, cuda, name="C1 fcc jitter")
    box = configs.fcc(jitter=0.0)
    ei, co, cnt, o = check_parity(box.pos, box.cell, box.pbc, box.radius, cuda, name="C1 fcc perfect")
    assert torch.all(cnt == 78)


def test_exact_cutoff_lattice(cuda):
    g = np.stack(np.meshgrid(*[np.arange(6)] * 3, indexing="ij"), -1).reshape(-1, 3) * 2.0
    for dt in (np.float32, np.float64):
        _, _, cnt, _ = check_parity(g.astype(dt), np.eye(3) * 12.0, (1, 1, 1), 4.0, cuda, name="sc r=4 exact")
        assert torch.all(cnt == 32)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_c2_uniform_100k(cuda, dtype):
    box = configs.c2(dtype)
    check_parity(box.pos, box.cell, box.pbc, box.radius, cuda, name="C2")


def test_c4_triclinic_slab(cuda):
    box = configs.c4()
    check_parity(box.pos, box.cell, box.pbc, box.radius, cuda, name="C4")


def test_c5_partition_small(cuda):
    box = configs.c5(n_owned=30_000, side=66.9)
    check_parity(box.pos, box.cell, box.pbc, box.radius, cuda, targets=box.targets, name="C5 small")


def test_c5_full_size_counts(cuda):
    """C5 at full size (4.4M atoms, 4M owned targets): 21600 tiles, past the 16000 of one
    64 KiB LDS histogram, so the tile-level sort runs with its larger LDS.  Per-target
    degrees against the oracle's (counts only: the 3.6e8 edges would not fit the oracle's
    memory), and the edge count equals their sum."""
    box = configs.c5()
    _announce(f"C5 full N={len(box.pos)} targets={len(box.targets)}")
    pt = torch.from_numpy(box.pos).to(cuda)
    tt = torch.from_numpy(box.targets).to(cuda)
    c = torch.from_numpy(np.asarray(box.cell, np.float64))
    b = torch.tensor(list(box.pbc))
    cnt = impl.radius_graph_pbc_counts_ex(pt, c, b, box.radius, tt)
    want, wtot = oracle.radius_graph_counts(box.pos, np.asarray(box.cell, np.float64), box.pbc,
                                            float(np.float32(box.radius)), target_indices=box.targets)
    assert np.array_equal(cnt.cpu().numpy(), want)
    assert int(wtot) == int(want.sum()) > 3e8


def test_c3_full_size(cuda):
    """The headline workload at full size (1M atoms, ~9.05e7 edges), through properties
    that need no full oracle edge list: per-target degrees equal the oracle's (C, exact
    canonical predicate), dst-degrees of the edge list equal them, every edge is within the
    cutoff in fp64, and the set is symmetric: (i, j, S) is an edge iff (j, i, -S) is."""
    box = configs.c3()
    N = len(box.pos)
    _announce(f"C3 full N={N}")
    cell = np.asarray(box.cell, np.float64)
    ei, co, nn, cnt = _gpu_build(box.pos, cell, box.pbc, box.radius, None, cuda)
    # the predicate sees the cell rounded to the position dtype, as the API passes it on
    # (at C3 one pair lies between the two cells' cutoff spheres)
    cell = cell.astype(box.pos.dtype).astype(np.float64)
    E = ei.shape[1]
    r32 = float(np.float32(box.radius))
    want, wtot = oracle.radius_graph_counts(box.pos, cell, box.pbc, r32)
    assert np.array_equal(cnt.cpu().numpy(), want)
    assert E == int(wtot) == int(nn.sum()) > 9e7
    src, dst = ei[0], ei[1]
    assert torch.equal(torch.bincount(dst, minlength=N).to(torch.int32), cnt)
    S = co.to(torch.int64)
    assert torch.equal(co, S.to(co.dtype)) and int(S.abs().max()) <= 8  # integer-valued shifts
    p64 = torch.from_numpy(box.pos).to(cuda).to(torch.float64)
    vec = p64[src] + S.to(torch.float64) @ torch.from_numpy(cell).to(cuda) - p64[dst]
    d2 = (vec * vec).sum(1)
    del vec
    assert float(d2.max()) <= r32 * r32 * (1 + 1e-12) and float(d2.min()) > 0.0
    del d2, p64
    sk = (S[:, 0] + 8) * 289 + (S[:, 1] + 8) * 17 + (S[:, 2] + 8)
    fwd = (src * N + dst) * 4913 + sk
    rev = (dst * N + src) * 4913 + (4912 - sk)  # -S in the same 17-radix digits
    assert torch.equal(torch.sort(fwd).values, torch.sort(rev).values)


# ---- design corner cases ----------------------------------------------------------
def test_wrapped_and_far_positions(cuda):
    cell = np.array([[11.0, 0, 0], [2.0, 12.0, 0], [-1.5, 1.0, 10.0]])
    pos, _ = _rand(300, 1.0, 5, dtype=np.float64, lo=-3.0, hi=4.0, cell=cell)
    for pbc in [(1, 1, 1), (1, 0, 1), (0, 0, 0)]:
        check_parity(pos, cell, pbc, 4.5, cuda, name="wrapped")


def test_all_pairs_fallback(cuda):
    # r >> cell: at r = 10 in a 3 A cell the stencil is 9^3 copies of one bin (the largest
    # region the tiled path takes); at r = 13 it would exceed that -> all-pairs kernel
    pos, cell = _rand(7, 3.0, 9)
    check_parity(pos, cell, (1, 1, 1), 13.0, cuda, name="all-pairs r=13")
    check_parity(pos, cell, (1, 1, 1), 10.0, cuda, name="all-pairs")
    check_parity(pos, cell, (1, 0, 1), 10.0, cuda, name="all-pairs partial")


def test_all_pairs_far_positions(cuda):
    """The all-pairs kernel with atoms up to three cell lengths outside the cell: an edge's
    shift is its image plus the difference of the two atoms' floors, so the image range
    must be taken around that difference (cubic and triclinic, full and partial PBC)."""
    pos, cell = _rand(12, 3.0, 34, lo=-3.0, hi=4.0)
    check_parity(pos, cell, (1, 1, 1), 13.0, cuda, name="all-pairs far positions")
    check_parity(pos, cell, (1, 0, 1), 13.0, cuda, name="all-pairs far positions partial")
    tri = np.array([[3.0, 0.0, 0.0], [0.8, 2.8, 0.0], [-0.5, 0.4, 3.1]])
    pos, _ = _rand(10, 1.0, 35, dtype=np.float64, lo=-2.5, hi=3.5, cell=tri)
    check_parity(pos, tri, (1, 1, 0), 13.0, cuda, name="all-pairs far positions triclinic")


def test_all_pairs_fallback_many_atoms(cuda):
    """The all-pairs kernel (a stencil of more than 768 bins: r > 4 cell widths) on tens of
    atoms with tens of thousands of periodic-image neighbours each, orthorhombic and
    triclinic, full and partial PBC; and the many-chunk sweep just below that limit (r = 10
    in a 6 A cell: one bin, a 5x5x5 stencil of its periodic copies)."""
    pos, cell = _rand(60, 3.0, 31)
    _, _, cnt, _ = check_parity(pos, cell, (1, 1, 1), 13.0, cuda, name="all-pairs 60")
    assert int(cnt.min()) > 15000
    tri = np.array([[3.0, 0.0, 0.0], [0.8, 2.8, 0.0], [-0.5, 0.4, 3.1]])
    pos, _ = _rand(40, 1.0, 32, dtype=np.float64, cell=tri)
    check_parity(pos, tri, (1, 0, 1), 13.0, cuda, name="all-pairs triclinic partial pbc")
    pos, cell = _rand(300, 6.0, 33)
    _, _, cnt, _ = check_parity(pos, cell, (1, 1, 1), 10.0, cuda, name="one bin, 125 copies")
    assert int(cnt.min()) > 3000


def test_dense_multichunk_and_oversized_targets(cuda):
    # 1500 atoms in an 8 A box, r=6: region >> LDS chunk, degree > staging capacity
    pos, cell = _rand(1500, 8.0, 13)
    _, _, cnt, _ = check_parity(pos, cell, (1, 1, 1), 6.0, cuda, name="dense")
    assert int(cnt.max()) > 2560


def test_explicit_targets_with_duplicates(cuda):
    box = configs.uniform(5000, seed=21, dtype=np.float32)
    rng = np.random.default_rng(0)
    tg = rng.choice(5000, 1200, replace=False)
    tg = np.r_[tg, tg[:50]]  # duplicates are separate targets
    check_parity(box.pos, box.cell, box.pbc, box.radius, cuda, targets=tg, name="targets")


def test_prefix_targets(cuda):
    """Explicit targets 0 .. nt - 1 (the local atoms of a partition) take the count over
    every atom of a tile with the ghosts' lanes idle, instead of a target sort.  With
    nt = n the result is byte-identical to the build without targets; with nt < n it
    equals the same target set given in another order (the sorted path), edge set and
    per-target counts."""
    _announce("prefix targets")
    box = configs.uniform(30000, seed=26, dtype=np.float32)
    p = torch.from_numpy(box.pos).to(cuda)
    c = torch.from_numpy(box.cell)
    b = torch.tensor([True] * 3)
    n = len(box.pos)
    full = impl.radius_graph_pbc_ex(p, c, b, box.radius, 0, False)
    pref = impl.radius_graph_pbc_ex(p, c, b, box.radius, 0, False, torch.arange(n, device=cuda))
    for x, y in zip(full, pref):
        assert torch.equal(x, y)
    box = configs.c5(n_owned=30_000, side=66.9)
    p = torch.from_numpy(box.pos).to(cuda)
    c = torch.from_numpy(np.asarray(box.cell, np.float64))
    b = torch.tensor(list(box.pbc))
    nt = len(box.targets)
    t1 = torch.arange(nt, device=cuda)
    t2 = t1.clone()
    t2[[0, nt - 1]] = t2[[nt - 1, 0]]  # not the prefix: the sorted-target path
    e1, s1, _, c1 = impl.radius_graph_pbc_ex(p, c, b, box.radius, 0, False, t1)
    e2, s2, _, c2 = impl.radius_graph_pbc_ex(p, c, b, box.radius, 0, False, t2)
    c2 = c2.clone()
    c2[[0, nt - 1]] = c2[[nt - 1, 0]]
    assert torch.equal(c1, c2)
    g1 = oracle.canonical_sort(e1[0].cpu().numpy(), e1[1].cpu().numpy(), s1.cpu().numpy().astype(np.int64))
    g2 = oracle.canonical_sort(e2[0].cpu().numpy(), e2[1].cpu().numpy(), s2.cpu().numpy().astype(np.int64))
    for x, y in zip(g1, g2):
        assert np.array_equal(x, y)
    # and nt = 0 .. a few: tiny prefixes
    for k in (1, 7):
        _, _, _, ck = impl.radius_graph_pbc_ex(p, c, b, box.radius, 0, False, torch.arange(k, device=cuda))
        assert torch.equal(ck, c1[:k])


def test_counts_only_matches(cuda):
    box = configs.uniform(20000, seed=3, dtype=np.float32)
    p = torch.from_numpy(box.pos).to(cuda)
    c = torch.from_numpy(box.cell)
    b = torch.tensor([True] * 3)
    cnt = impl.radius_graph_pbc_counts_ex(p, c, b, 6.0)
    _, _, nn, cnt2 = impl.radius_graph_pbc_ex(p, c, b, 6.0, 0, False)
    assert torch.equal(cnt, cnt2) and int(cnt.sum()) == int(nn.item())


def test_deterministic_bytes(cuda):
    box = configs.uniform(50000, seed=8, dtype=np.float32)
    p = torch.from_numpy(box.pos).to(cuda)
    c = torch.from_numpy(box.cell)
    b = torch.tensor([True] * 3)
    a = impl.radius_graph_pbc(p, c, b, 6.0, 0, False)
    z = impl.radius_graph_pbc(p, c, b, 6.0, 0, False)
    assert torch.equal(a[0], z[0]) and torch.equal(a[1], z[1])


def _two_phase_box():
    class B:
        pass
    b = B()
    b.pos, b.cell = _two_phase(50.0, 0.3, 0.01, 5)
    b.pbc, b.radius = (1, 1, 1), 5.0
    return b


@pytest.mark.parametrize("which", ["c4", "two-phase"])
def test_edge_vectors(cuda, which):
    """Edge vectors and distances (fp64 bit-identical to the canonical formula, fp32 the
    correctly rounded values); the two-phase box has two-chunk tiles, whose edges come from
    the fix-up kernel's expansion."""
    box = configs.c4(scale=0.4) if which == "c4" else _two_phase_box()
    r = box.radius
    o = oracle.radius_graph(box.pos, box.cell, box.pbc, r, vectors=True)
    want = oracle.canonical_sort(o["src"], o["dst"], o["shift"], o["vec"], np.sqrt(o["d2"]))
    for vdt in (torch.float64, torch.float32):
        _announce(f"edge vectors {vdt}")
        ei, co, nn, cnt, vec, dist = _gpu_build(box.pos, box.cell, box.pbc, r, None, cuda, True, vdt)
        got = oracle.canonical_sort(ei[0].cpu().numpy(), ei[1].cpu().numpy(), co.cpu().numpy(),
                                    vec.cpu().numpy(), dist.cpu().numpy())
        for a, b in zip(got[:3], want[:3]):
            assert np.array_equal(a, b)
        if vdt == torch.float64:
            assert np.array_equal(got[3], want[3])  # same canonical formula: bit-identical
            assert np.allclose(got[4], want[4], rtol=1e-15, atol=0)
        else:
            assert np.array_equal(got[3], want[3].astype(np.float32))
            ulp = np.spacing(want[4].astype(np.float32))
            assert np.all(np.abs(got[4].astype(np.float64) - want[4]) <= 2 * ulp)


def _filter_case(cuda, n, seed, r_big, r, dtype):
    box = configs.uniform(n, seed=seed, dtype=np.float32)
    p = torch.from_numpy(box.pos).to(cuda)
    c = torch.from_numpy(box.cell)
    b = torch.tensor([True] * 3)
    ei, co, _ = impl.radius_graph_pbc(p, c, b, r_big, 0, False)
    sh = co.to(dtype)
    ef, cf = impl.filter_edges_to_radius(ei, sh, p, c, r)
    e6, c6, _ = impl.radius_graph_pbc(p, c, b, r, 0, False)
    got = oracle.canonical_sort(ef[0].cpu().numpy(), ef[1].cpu().numpy(), cf.float().cpu().numpy().astype(np.int64))
    want = oracle.canonical_sort(e6[0].cpu().numpy(), e6[1].cpu().numpy(), c6.cpu().numpy().astype(np.int64))
    for a, bb in zip(got, want):
        assert np.array_equal(a, bb)
    # order preserving: kept edges appear in their original relative order, and the kept
    # shifts are the input rows bit for bit, in the input dtype
    keep = oracle.filter_edges(box.pos, box.cell, r, ei[0].cpu().numpy(), ei[1].cpu().numpy(),
                               co.cpu().numpy().astype(np.int32))
    kt = torch.from_numpy(np.nonzero(keep)[0]).to(cuda)
    assert np.array_equal(ef.cpu().numpy(), ei.cpu().numpy()[:, keep])
    assert cf.dtype == sh.dtype and torch.equal(cf, sh.index_select(0, kt))
    return ei.shape[1]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.int64, torch.int32,
                                   torch.float16, torch.bfloat16])
def test_filter_edges_to_radius(cuda, dtype):
    _announce(f"filter, shifts {dtype}")
    _filter_case(cuda, 8000, 17, 6.5, 6.0, dtype)


def test_filter_large_list(cuda):
    """More than 2.1M edges: hundreds of look-back tiles of 4096 edges (offsets passed
    through many predecessors' status words), the last tile partial."""
    _announce("filter, large list")
    E = _filter_case(cuda, 30000, 18, 6.5, 6.0, torch.float32)
    assert E > 2_100_000 and E % 4096 != 0


def test_filter_rejects_out_of_range_atoms(cuda):
    _announce("filter, out-of-range atom index")
    box = configs.uniform(2000, seed=19, dtype=np.float32)
    p = torch.from_numpy(box.pos).to(cuda)
    c = torch.from_numpy(box.cell)
    ei, co, _ = impl.radius_graph_pbc(p, c, torch.tensor([True] * 3), 6.0, 0, False)
    for bad in (2000, -1):
        e2 = ei.clone()
        e2[0, 17] = bad
        with pytest.raises(RuntimeError, match="outside"):
            impl.filter_edges_to_radius(e2, co, p, c, 5.0)


def test_vectors_round_radius_like_the_build(cuda):
    """radius_graph_pbc_vectors rounds the radius to fp32 as radius_graph_pbc_ex does, so
    both return the same edge set at a radius fp32 cannot hold exactly."""
    _announce("vectors radius rounding")
    box = configs.uniform(20000, seed=23, dtype=np.float32)
    p = torch.from_numpy(box.pos).to(cuda)
    c = torch.from_numpy(box.cell)
    b = torch.tensor([True] * 3)
    r = 5.3
    assert float(np.float32(r)) != r
    e1, s1, _, n1 = impl.radius_graph_pbc_ex(p, c, b, r, 0, False)
    e2, s2, _, n2, vec, dist = impl.radius_graph_pbc_vectors(p, c, b, r)
    assert torch.equal(e1, e2) and torch.equal(s1, s2) and torch.equal(n1, n2)
    assert float(dist.max()) <= float(np.float32(r))


def test_far_atom_is_rejected(cuda):
    """An atom more than 255 cell lengths outside the cell (along a lattice vector) is
    refused with an error naming the limit; 250 cell lengths are accepted."""
    _announce("far atom")
    box = configs.uniform(500, seed=24, dtype=np.float64, radius=5.0)
    c = torch.from_numpy(box.cell)
    b = torch.tensor([True] * 3)
    L = float(box.cell[0, 0])
    pos = box.pos.copy()
    pos[7, 1] += 250.0 * L
    check_parity(pos, box.cell, box.pbc, 5.0, cuda, name="250 cells out")
    pos[7, 1] += 10.0 * L
    with pytest.raises(RuntimeError, match="255 cell lengths"):
        impl.radius_graph_pbc(torch.from_numpy(pos).to(cuda), c, b, 5.0, 0, False)


def test_stage_timer(cuda, capfd, monkeypatch):
    """RADIUS_PBC_PROFILE (as the reference's radius_graph_kernels.cu:444-465) prints the
    time of every stage of a build to stderr; unset, nothing is printed."""
    _announce("stage timer")
    box = configs.uniform(20000, seed=25, dtype=np.float32)
    p = torch.from_numpy(box.pos).to(cuda)
    c = torch.from_numpy(box.cell)
    b = torch.tensor([True] * 3)
    impl.radius_graph_pbc(p, c, b, 6.0, 0, False)
    torch.cuda.synchronize()
    assert "[radius_graph_pbc profile]" not in capfd.readouterr().err
    monkeypatch.setenv("RADIUS_PBC_PROFILE", "1")
    impl.radius_graph_pbc(p, c, b, 6.0, 0, False)
    err = capfd.readouterr().err
    for stage in ("dg_graph_count", "sfc reorder + sort", "count", "dg_graph_write",
                  "write (slot expansion)", "write (fix-up)", "total"):
        assert stage in err, err


# ---- prefilter band: pairs within a few ulp of the cutoff ---------------------------
def _near_cutoff_box(cell, r, n_anchor, seed, dtype):
    """Anchors spread over the cell (many near its faces, so pairs cross the periodic
    boundary), each with partners at r (1 + eps) in random directions, eps down to the
    fp32 rounding of the coordinates: every such pair sits in or next to the fp32
    prefilter band, where only the exact canonical test may decide."""
    rng = np.random.default_rng(seed)
    cell = np.asarray(cell, np.float64)
    f = rng.uniform(0, 1, (n_anchor, 3))
    h = n_anchor // 2  # these get one fractional coordinate within 2 % of a face
    axis = rng.integers(0, 3, h)
    f[np.arange(h), axis] = np.where(rng.uniform(size=h) < 0.5, rng.uniform(0, 0.02, h), rng.uniform(0.98, 1.0, h))
    anchors = f @ cell
    eps = np.array([-3e-6, -1e-6, -3e-7, -1e-7, 0.0, 1e-7, 3e-7, 1e-6, 3e-6])
    d = rng.normal(size=(n_anchor, len(eps), 3))
    d /= np.linalg.norm(d, axis=-1, keepdims=True)
    partners = anchors[:, None, :] + d * (r * (1.0 + eps))[None, :, None]
    return np.concatenate([anchors, partners.reshape(-1, 3)]).astype(dtype)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape", ["cubic", "lowtri", "general"])
def test_near_cutoff_pairs(cuda, dtype, shape):
    cell = {"cubic": np.eye(3) * 215.443,
            "lowtri": np.array([[120.0, 0, 0], [30.0, 110.0, 0], [-20.0, 25.0, 100.0]]),
            "general": np.array([[110.0, 8.0, -5.0], [20.0, 105.0, 6.0], [-10.0, 15.0, 98.0]])}[shape]
    pos = _near_cutoff_box(cell, 6.0, 1500, 17, dtype)
    _, _, cnt, o = check_parity(pos, cell, (1, 1, 1), 6.0, cuda, name=f"near-cutoff {shape}")
    assert len(o["src"]) > 1500 * 4  # the inside half of every anchor's partners at least


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape", ["cubic", "lowtri"])
def test_near_cutoff_pairs_along_x(cuda, dtype, shape):
    """Pairs within a few ulp of the cutoff, mostly along x, in a background at C3's density
    (0.1 per cubic angstrom, so bins hold a few atoms each).  The count pass starts and ends
    each stencil row at quarter-bin x boundaries of its end bins (bins ordered by x): every
    partner here sits near the far x end of some anchor's rows, where a cut one quarter too
    deep would drop it."""
    cell = {"cubic": np.eye(3) * 48.0,
            "lowtri": np.array([[48.0, 0, 0], [12.0, 46.0, 0], [-8.0, 10.0, 45.0]])}[shape]
    r = 6.0
    rng = np.random.default_rng(31)
    vol = abs(np.linalg.det(cell))
    bg = rng.uniform(0, 1, (int(0.1 * vol), 3)) @ cell
    anchors = rng.uniform(0, 1, (600, 3)) @ cell
    eps = np.array([-3e-6, -1e-6, -1e-7, 0.0, 1e-7, 1e-6, 3e-6])
    n_e = len(eps)
    # y, z offsets up to 3 A (the rows of the anchor's bin and its neighbours), x from the
    # distance; both x directions
    yz = rng.uniform(-3.0, 3.0, (len(anchors), n_e, 2))
    dist = r * (1.0 + eps)[None, :]
    dx = np.sqrt(dist ** 2 - (yz ** 2).sum(-1))
    sgn = np.where(rng.uniform(size=dx.shape) < 0.5, -1.0, 1.0)
    off = np.concatenate([(sgn * dx)[..., None], yz], axis=-1)
    partners = anchors[:, None, :] + off
    pos = np.concatenate([bg, anchors, partners.reshape(-1, 3)]).astype(dtype)
    _, _, cnt, o = check_parity(pos, cell, (1, 1, 1), r, cuda, name=f"near-cutoff along x {shape}")
    assert len(o["src"]) > 0.1 * vol * 30


@pytest.mark.parametrize("shape", ["cubic", "lowtri"])
def test_crowded_bins_in_sparse_rows(cuda, shape):
    """Bins of 16 to 80 atoms (spread over the whole bin) in a background at C3's density,
    each tile still one LDS chunk: the count's quarter-bin prefix counts saturate at 15 in
    these bins, and rows that start or end in them must fall back to the whole bin on the
    saturated side."""
    cell = {"cubic": np.eye(3) * 45.0,
            "lowtri": np.array([[45.0, 0, 0], [10.0, 44.0, 0], [-6.0, 8.0, 43.0]])}[shape]
    r = 6.0
    rng = np.random.default_rng(37)
    vol = abs(np.linalg.det(cell))
    bg = rng.uniform(0, 1, (int(0.1 * vol), 3))
    nb = {"cubic": 15, "lowtri": 14}[shape]  # bins per axis: the planner's floor(2 d_face / r)
    crowds = []
    for k, m in enumerate([16, 24, 40, 80]):
        b = rng.integers(0, nb, 3)
        crowds.append((b + rng.uniform(0.0, 1.0, (m, 3))) / nb)  # inside one bin, in fractions
    frac = np.concatenate([bg] + crowds)
    pos = (frac @ cell).astype(np.float32)
    _, _, cnt, o = check_parity(pos, cell, (1, 1, 1), r, cuda, name=f"crowded bins {shape}")
    assert len(o["src"]) > 0


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape", ["cubic", "general"])
def test_near_coincident_atoms(cuda, dtype, shape):
    """Distinct atoms at or near the same place: exact duplicates (d2 = 0, never an edge)
    and partners at distances around 1e-4 A, where the canonical d2 > 1e-8 threshold
    decides; some anchors sit on periodic faces, so the duplicate is an image."""
    cell = {"cubic": np.eye(3) * 60.0,
            "general": np.array([[60.0, 4.0, -3.0], [10.0, 58.0, 3.0], [-5.0, 7.0, 55.0]])}[shape]
    rng = np.random.default_rng(29)
    n = 400
    f = rng.uniform(0, 1, (n, 3))
    f[: n // 4, 0] = 0.0  # on a face: partners across it are periodic images
    anchors = f @ cell
    dist = np.array([0.0, 0.0, 5e-5, 9e-5, 9.9e-5, 1e-4, 1.01e-4, 1.1e-4, 2e-4, 1e-3])
    d = rng.normal(size=(n, len(dist), 3))
    d /= np.linalg.norm(d, axis=-1, keepdims=True)
    partners = anchors[:, None, :] + d * dist[None, :, None]
    pos = np.concatenate([anchors, partners.reshape(-1, 3)]).astype(dtype)
    _, _, _, o = check_parity(pos, cell, (1, 1, 1), 5.0, cuda, name=f"near-coincident {shape}")
    c = np.asarray(cell, np.float64).astype(dtype).astype(np.float64)
    _, d2 = oracle.edge_vectors(pos, c, o["src"], o["dst"], o["shift"])
    # thousands of pairs within 3 % above the threshold (1e-8 rounded to fp32, as the
    # reference writes it), none at or below it
    thr = float(np.float32(1e-8))
    assert np.all(d2 > thr) and np.sum(d2 < 1.03 * thr) > 1000


def _two_phase(side, rho_lo, rho_hi, seed):
    rng = np.random.default_rng(seed)
    cell = np.eye(3) * side
    vol = side ** 3
    f_lo = rng.uniform(0, 1, (int(rho_lo * vol / 2), 3)) * [1, 1, 0.5]
    f_hi = rng.uniform(0, 1, (int(rho_hi * vol / 2), 3)) * [1, 1, 0.5] + [0, 0, 0.5]
    return (np.concatenate([f_lo, f_hi]) @ cell).astype(np.float32), cell


@pytest.mark.parametrize("side,rho_lo,rho_hi,r", [(60.0, 0.2, 0.02, 6.0), (50.0, 0.3, 0.01, 5.0)])
def test_two_phase_dense_tiles(cuda, side, rho_lo, rho_hi, r):
    """A two-phase box: tiles are planned for the mean density, so in the dense phase the
    region needs two LDS chunks (slots over both chunks, expanded by the fix-up kernel) and
    many targets exceed the slot capacity (their edges k >= K swept again across both
    chunks)."""
    pos, cell = _two_phase(side, rho_lo, rho_hi, 5)
    check_parity(pos, cell, (1, 1, 1), r, cuda, name=f"two-phase {side} {rho_lo}/{rho_hi}")


@pytest.mark.parametrize("side,cube,rho_bg,rho_c", [(60.0, 24.0, 0.005, 0.5), (64.0, 26.0, 0.004, 0.45)])
def test_dense_cube_in_sparse_box(cuda, side, cube, rho_bg, rho_c):
    """A dense cube in a sparse periodic box, r = 5: tiles are planned for the mean
    density, so around the cube regions need two, three or four LDS chunks, and the cube's
    targets have several times the slot capacity K.  Covers every fix-up path: targets past
    K in one- and two-chunk regions (slots, then a second sweep across the chunks) and in
    regions of more than two chunks (written directly, chunk by chunk)."""
    rng = np.random.default_rng(11)
    bg = rng.uniform(0, side, (int(rho_bg * side ** 3), 3))
    cl = rng.uniform(0, cube, (int(rho_c * cube ** 3), 3)) + (side - cube) / 2
    pos = np.concatenate([bg, cl]).astype(np.float32)
    check_parity(pos, np.eye(3) * side, (1, 1, 1), 5.0, cuda, name=f"dense cube {cube} in {side}")


@pytest.mark.parametrize("which", ["left-handed", "negative diagonal", "permuted rows", "tiny skewed"])
def test_unusual_cells(cuda, which):
    """Cells the lower-triangular fast path does not take: a left-handed cell (negative
    determinant), a diagonal with negative entries, the rows of a triclinic cell permuted,
    and a strongly skewed small cell (all-pairs range); parity with the oracle, full and
    partial PBC, atoms inside and outside the cell."""
    base = np.array([[14.0, 0.0, 0.0], [3.0, 13.0, 0.0], [-2.0, 1.5, 12.0]])
    r = 5.0
    if which == "left-handed":
        cell = base.copy()
        cell[2] *= -1.0
    elif which == "negative diagonal":
        cell = np.diag([-13.0, 12.0, -14.0])
    elif which == "permuted rows":
        cell = base[[2, 0, 1]]
    else:
        cell = np.array([[3.0, 0.0, 0.0], [2.6, 1.5, 0.0], [1.0, 1.2, 2.8]])
        r = 9.0
    pos, _ = _rand(200 if which != "tiny skewed" else 20, 1.0, 91, dtype=np.float64, lo=-1.2, hi=2.2, cell=cell)
    for pbc in [(1, 1, 1), (1, 0, 1)]:
        check_parity(pos, cell, pbc, r, cuda, name=f"{which} pbc={pbc}")


def test_errors_are_raised(cuda):
    """Non-finite positions and explicit targets outside [0, N) raise RuntimeError (the
    reference has no check; here the build reports them instead of producing garbage)."""
    p, c = _rand(500, 20.0, 92)
    pt = torch.from_numpy(p).to(cuda)
    bad = pt.clone()
    bad[17, 1] = float("nan")
    with pytest.raises(RuntimeError, match="non-finite"):
        impl.radius_graph_pbc(bad, torch.from_numpy(c), torch.tensor([True] * 3), 5.0, 0, False)
    for t in (500, -1):
        tg = torch.tensor([0, 3, t], dtype=torch.int64, device=cuda)
        with pytest.raises(RuntimeError, match="target"):
            impl.radius_graph_pbc_ex(pt, torch.from_numpy(c), torch.tensor([True] * 3), 5.0, 0, False, tg)
    # and a good build right after still works
    check_parity(p, c, (1, 1, 1), 5.0, cuda, name="after errors")
