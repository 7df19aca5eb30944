"""Pins the halo-plan oracle (oracle/halo.py) before it is trusted as the checker: a
hand-worked case, the agreement of its two restatements (per-rank edges vs the full-graph
needed_by map, as dynamis_state/tests/test_dist_graph_builder.py:199-271 asserts for the
reference), and the send/recv mirror identity between ranks."""
import numpy as np
import pytest

import oracle
from oracle import halo


def _line_case():
    # 5 atoms at x = 0..4, no PBC, r = 1.1: bonds 0-1, 1-2, 2-3, 3-4 in both directions.
    pos = np.zeros((5, 3))
    pos[:, 0] = np.arange(5)
    o = oracle.radius_graph(pos, np.eye(3) * 10.0, (0, 0, 0), 1.1)
    return o["src"], o["dst"], np.array([0, 0, 1, 1, 0])


def test_hand_worked_line():
    src, dst, pid = _line_case()
    assert len(src) == 8
    # rank 0 owns {0, 1, 4}: needs 2 (for 1) and 3 (for 4) from rank 1, sends 1 and 4
    m = np.isin(dst, [0, 1, 4])  # the rank's edges: dst owned by it
    so, sl, ro, rg, im, ra = halo.extract_halo_info(src[m], dst[m], pid, [0, 1, 4], 0, 2, 5)
    assert so.tolist() == [0, 0, 2] and sl.tolist() == [1, 2]
    assert ro.tolist() == [0, 0, 2] and ra.tolist() == [2, 3] and rg.tolist() == [3, 4]
    assert im.tolist() == [True, False, False]
    # rank 1 owns {2, 3}: needs 1 and 4 from rank 0, sends both its atoms
    m = np.isin(dst, [2, 3])
    so, sl, ro, rg, im, ra = halo.extract_halo_info(src[m], dst[m], pid, [2, 3], 1, 2, 5)
    assert so.tolist() == [0, 2, 2] and sl.tolist() == [0, 1]
    assert ro.tolist() == [0, 2, 2] and ra.tolist() == [1, 4] and rg.tolist() == [2, 3]
    assert im.tolist() == [False, False]


def _box(seed, n=600, L=18.0):
    rng = np.random.default_rng(seed)
    return rng.uniform(0, L, (n, 3)), np.eye(3) * L


@pytest.mark.parametrize("W,part", [(2, "slab"), (4, "slab"), (3, "random"), (70, "random")])
def test_two_restatements_agree(W, part):
    pos, cell = _box(7 + W)
    N = pos.shape[0]
    rng = np.random.default_rng(W)
    if part == "slab":
        pid = np.clip(np.floor(pos[:, 0] / cell[0, 0] * W).astype(np.int64), 0, W - 1)
    else:
        pid = rng.integers(0, W, N)
    r = 3.5
    full = oracle.radius_graph(pos, cell, (1, 1, 1), r)
    total_send = 0
    for R in range(W):
        my = np.nonzero(pid == R)[0]
        per = oracle.radius_graph(pos, cell, (1, 1, 1), r, target_indices=my)
        a = halo.extract_halo_info(per["src"], per["dst"], pid, my, R, W, N)
        b = halo.build_halo_maps(full["src"], full["dst"], pid, R, W, N)
        for k in range(6):
            assert np.array_equal(a[k], b[k]), (R, k)
        total_send += a[1].size
    assert total_send > 0


def test_mirror_identity():
    W = 4
    pos, cell = _box(3)
    N = pos.shape[0]
    pid = np.random.default_rng(5).integers(0, W, N)
    full = oracle.radius_graph(pos, cell, (1, 1, 1), 3.0)
    plans = {}
    for R in range(W):
        my = np.nonzero(pid == R)[0]
        mask = np.isin(full["dst"], my)
        plans[R] = (my, halo.extract_halo_info(full["src"][mask], full["dst"][mask], pid, my, R, W, N))
    for p in range(W):
        for q in range(W):
            if p == q:
                continue
            my_p, (so, sl, _, _, _, _) = plans[p]
            _, (_, _, ro, _, _, ra) = plans[q]
            sent = my_p[sl[so[q]:so[q + 1]]]
            recv = ra[ro[p]:ro[p + 1]]
            assert np.array_equal(sent, recv), (p, q)
