"""Full-size parity of the HIP build against the CPU oracle, edge set by edge set.

Every edge (src, dst, S) of a build is packed into one int64 key (src, then dst, then
the three shift components, each field wide enough for the case); the GPU's keys and the
oracle's keys are sorted on the device and compared element by element, which is the
canonical (src, dst, shift) sort of the whole edge list.  Strictly increasing sorted keys
also show that the build emits no edge twice.

Cases: the headline C3 box (1M atoms, ~9.05e7 edges); C4 at its stated 500k atoms (the
triclinic cell scaled by 1.3934); the C5 random walk of the benchmark (degrees at full
size on frames 1, 50 and 99; every edge on a reduced box over 10 frames); and the sort
paths no benchmark configuration reaches: more tiles than the tile-level sort takes (the
per-bin fallback), with more than 2^24 atoms, 64-bit tile-bucket entries (more than
2^24 targets), and a slot array past 4 GiB (64-bit slot addresses).
"""
import itertools

import numpy as np
import pytest
import torch

import oracle
from dynamis_amd import configs
from dynamis_amd.dynamis_state import dynamis_state_impl as impl

pytestmark = pytest.mark.gpu


def _announce(name):
    print(f"\n[case] {name}", flush=True)


def _layout(n, smax):
    """Bits of the atom fields and of each shift field of an edge key for n atoms."""
    nb = max(1, (int(n) - 1).bit_length())
    sb = (63 - 2 * nb) // 3
    assert sb >= 3 and smax < (1 << (sb - 1)), (n, smax)
    return nb, sb


def _keys_torch(src, dst, S, nb, sb):
    off = 1 << (sb - 1)
    k = (src << nb) | dst
    for c in range(3):
        k = (k << sb) | (S[:, c] + off)
    return k


def _keys_numpy(src, dst, S, nb, sb):
    off = np.int64(1 << (sb - 1))
    k = (src.astype(np.int64) << np.int64(nb)) | dst.astype(np.int64)
    for c in range(3):
        k = (k << np.int64(sb)) | (S[:, c].astype(np.int64) + off)
    return k


def _cell_used(box):
    # the API rounds the cell to the position dtype (radius_graph.cpp:24)
    return np.asarray(box.cell, np.float64).astype(box.pos.dtype).astype(np.float64)


def check_edge_set(dev, pos_np, box, targets=None, pos_t=None):
    """GPU build vs oracle: sorted edge keys equal, no duplicates, degrees equal."""
    n = len(pos_np)
    pt = torch.from_numpy(pos_np).to(dev) if pos_t is None else pos_t
    tt = None if targets is None else torch.from_numpy(targets).to(dev)
    ei, co, nn, cnt = impl.radius_graph_pbc_ex(pt, torch.from_numpy(np.asarray(box.cell, np.float64)),
                                               torch.tensor([bool(x) for x in box.pbc]), box.radius,
                                               0, False, tt)
    S = co.to(torch.int64)
    assert torch.equal(S.to(co.dtype), co)  # integer-valued shifts
    o = oracle.radius_graph(pos_np, _cell_used(box), box.pbc, float(np.float32(box.radius)),
                            target_indices=targets)
    E = ei.shape[1]
    assert E == len(o["src"]) == int(nn.item())
    assert np.array_equal(cnt.cpu().numpy(), o["counts"])
    smax = max(int(S.abs().max()) if E else 0, int(np.abs(o["shift"]).max()) if E else 0)
    nb, sb = _layout(n, smax)
    got = torch.sort(_keys_torch(ei[0], ei[1], S, nb, sb)).values
    del ei, co, S
    want = torch.from_numpy(_keys_numpy(o["src"], o["dst"], o["shift"], nb, sb)).to(dev)
    del o
    want = torch.sort(want).values
    assert torch.equal(got, want)
    if E > 1:
        assert bool((got[1:] > got[:-1]).all())  # no edge twice
    return E


def test_c3_full_edge_set(cuda):
    """C3 (1M atoms, fp32, r = 6): all ~9.05e7 edges equal the oracle's."""
    box = configs.c3()
    _announce(f"C3 full edge set N={len(box.pos)}")
    E = check_edge_set(cuda, box.pos, box)
    assert E > 9e7


def test_c3_vectors_full_size(cuda):
    """C3 with edge vectors and distances at full size.  The write stage splits its waves'
    output ranges at 32-edge offsets or at 4-edge ones, chosen from the edge total and the
    outputs' width; at C3 the plain build takes the first and the build with fp32 vectors
    the second, so equal edge lists (byte for byte, same order) check the two against each
    other.  The vectors are pos[src] + S.cell - pos[dst] evaluated in fp64 and rounded to
    fp32 (compared with torch's fp64 evaluation within one fp32 rounding), the distances
    their norms."""
    box = configs.c3()
    _announce(f"C3 vectors full size N={len(box.pos)}")
    p = torch.from_numpy(box.pos).to(cuda)
    cell = torch.from_numpy(np.asarray(box.cell, np.float64))
    pbc = torch.tensor([bool(x) for x in box.pbc])
    ei, co, nn, cnt = impl.radius_graph_pbc_ex(p, cell, pbc, box.radius, 0, False, None)
    ei2, co2, nn2, cnt2, vec, dist = impl.radius_graph_pbc_vectors(p, cell, pbc, box.radius,
                                                                   vector_dtype=torch.float32)
    assert ei.shape[1] > 9e7
    assert torch.equal(ei2, ei) and torch.equal(co2, co) and torch.equal(cnt2, cnt)
    c64 = cell.to(torch.float32).to(torch.float64).to(cuda)  # the cell the fp32 build uses
    p64 = p.to(torch.float64)
    v64 = p64[ei[0]] + co.to(torch.float64) @ c64 - p64[ei[1]]
    # one fp32 rounding, plus 1e-12 A for fp64 evaluation-order differences near zero
    tol = torch.finfo(torch.float32).eps * v64.abs() + 1e-12
    assert bool(((vec.to(torch.float64) - v64).abs() <= tol).all())
    d64 = v64.norm(dim=1)
    del v64
    assert bool(((dist.to(torch.float64) - d64).abs() <= torch.finfo(torch.float32).eps * d64).all())


def test_c4_at_500k_atoms(cuda):
    """C4 at the stated 500,000 atoms: the triclinic cell scaled by 1.3934 at the stated
    densities (fp64, r = 5, two-phase slab)."""
    box = configs.c4(scale=1.3934)
    _announce(f"C4 x1.3934 N={len(box.pos)}")
    assert 495_000 < len(box.pos) < 505_000
    check_edge_set(cuda, box.pos, box)


def test_c5_walk_full_size_degrees(cuda):
    """The benchmark's C5 trajectory (4.44M atoms, 4M owned targets, no PBC, Gaussian
    0.01 A per coordinate per frame, generated on the device as bench.py does): per-target
    degrees equal the oracle's on frames 1, 50 and 99."""
    box = configs.c5()
    pt = torch.from_numpy(box.pos).to(cuda)
    tt = torch.from_numpy(box.targets).to(cuda)
    c = torch.from_numpy(np.asarray(box.cell, np.float64))
    b = torch.tensor(list(box.pbc))
    want_frames = {1, 50, 99}
    for k, fr in enumerate(itertools.islice(configs.walk(pt, 0.01, seed=7), 100)):
        if k not in want_frames:
            continue
        _announce(f"C5 walk frame {k}")
        cnt = impl.radius_graph_pbc_counts_ex(fr, c, b, box.radius, tt)
        p_np = fr.cpu().numpy()
        want, wtot = oracle.radius_graph_counts(p_np, _cell_used(box), box.pbc,
                                                float(np.float32(box.radius)), target_indices=box.targets)
        assert np.array_equal(cnt.cpu().numpy(), want)
        assert wtot > 3.5e8


def test_c5_walk_reduced_edge_sets(cuda):
    """C5's shape at 30k owned atoms (same density, shell, indexing and no PBC): every edge
    of 10 consecutive frames of the walk equals the oracle's."""
    box = configs.c5(n_owned=30_000, side=66.9)
    pt = torch.from_numpy(box.pos).to(cuda)
    for k, fr in enumerate(itertools.islice(configs.walk(pt, 0.01, seed=7), 10)):
        _announce(f"C5 reduced walk frame {k}")
        check_edge_set(cuda, fr.cpu().numpy(), box, targets=box.targets, pos_t=fr)


def test_sort_fallback_many_tiles(cuda):
    """50653 tiles (1.5M atoms at 1.5 A^-3, r = 1): more than the tile-level sort takes,
    so the per-bin atomic counting sort builds the cell list.  Every edge checked."""
    box = configs.uniform(1_500_000, density=1.5, seed=42, dtype=np.float32, radius=1.0)
    _announce("sort fallback, 50653 tiles")
    E = check_edge_set(cuda, box.pos, box)
    assert E > 9e6


def test_more_than_2_24_atoms(cuda):
    """17M atoms (past 2^24) at 1 A^-3, r = 1 (551368 tiles: the per-bin sort): per-target
    degrees equal the oracle's, and the written edge list has exactly those degrees."""
    box = configs.uniform(17_000_000, density=1.0, seed=41, dtype=np.float32, radius=1.0)
    n = len(box.pos)
    assert n > (1 << 24)
    _announce(f"N={n} > 2^24")
    pt = torch.from_numpy(box.pos).to(cuda)
    c = torch.from_numpy(box.cell)
    b = torch.tensor([True] * 3)
    ei, co, nn, cnt = impl.radius_graph_pbc_ex(pt, c, b, box.radius, 0, False)
    want, wtot = oracle.radius_graph_counts(box.pos, _cell_used(box), box.pbc, box.radius)
    assert np.array_equal(cnt.cpu().numpy(), want)
    assert ei.shape[1] == int(wtot) > 5e7
    assert torch.equal(torch.bincount(ei[1], minlength=n).to(torch.int32), cnt)
    assert int(ei.min()) >= 0 and int(ei.max()) < n


def test_more_than_2_24_targets(cuda):
    """17M explicit targets (duplicates of 6064 atoms; r = 3 in a 49.5 A box, 21952
    one-bin tiles): past 2^24 targets, the tile-level sort keeps 64-bit bucket entries.
    Each target's degree equals the oracle's degree of its atom."""
    box = configs.uniform(6064, density=0.05, seed=43, dtype=np.float32, radius=3.0)
    rng = np.random.default_rng(44)
    tg = rng.integers(0, 6064, 17_000_000, dtype=np.int64)
    _announce(f"{len(tg)} targets > 2^24")
    cnt = impl.radius_graph_pbc_counts_ex(torch.from_numpy(box.pos).to(cuda), torch.from_numpy(box.cell),
                                          torch.tensor([True] * 3), box.radius,
                                          torch.from_numpy(tg).to(cuda))
    deg, _ = oracle.radius_graph_counts(box.pos, _cell_used(box), box.pbc, box.radius)
    assert np.array_equal(cnt.cpu().numpy(), deg[tg])


def test_slots_past_4_gib(cuda):
    """12M atoms at C3's density and radius (1.09e9 edges): the count pass's slot array
    (2 bytes x 184 entries x 12M targets) is larger than 4 GiB, so slot addresses need 64
    bits.  Checks without the oracle (whose run would take minutes here): the written edges
    have exactly the degrees the count pass reports, each satisfies the predicate (fp64,
    canonical form), none appears twice, and the set is symmetric under
    (i, j, S) <-> (j, i, -S)."""
    n = 12_000_000
    box = configs.uniform(n, density=0.1, seed=45, dtype=np.float32)
    _announce(f"N={n}: slots past 4 GiB")
    p = torch.from_numpy(box.pos).to(cuda)
    c = torch.from_numpy(box.cell)
    b = torch.tensor([True] * 3)
    assert 2 * 184 * n > 2 ** 32
    ei, co, nn, cnt = impl.radius_graph_pbc_ex(p, c, b, box.radius, 0, False)
    E = ei.shape[1]
    assert E > 1.0e9 and int(nn.item()) == E
    assert torch.equal(torch.bincount(ei[1], minlength=n).to(torch.int32), cnt)
    cell = torch.from_numpy(np.asarray(box.cell, np.float32).astype(np.float64)).to(cuda)
    p64 = p.double()
    r2 = float(np.float32(box.radius)) ** 2
    step = 100_000_000
    for e0 in range(0, E, step):
        s_, d_ = ei[0, e0:e0 + step], ei[1, e0:e0 + step]
        v = p64[s_] + co[e0:e0 + step].double() @ cell - p64[d_]
        d2 = (v * v).sum(1)
        assert bool((d2 <= r2 * (1 + 1e-12)).all()) and bool((d2 > 1e-8).all())
        del v, d2
    nb, sb = _layout(n, 1)
    S = co.to(torch.int64)
    fwd = torch.sort(_keys_torch(ei[0], ei[1], S, nb, sb)).values
    assert bool((fwd[1:] > fwd[:-1]).all())  # no edge twice
    rev = torch.sort(_keys_torch(ei[1], ei[0], -S, nb, sb)).values
    assert torch.equal(fwd, rev)
