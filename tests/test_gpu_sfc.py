"""GPU parity of the SFC keys, the stable order and the partition labels vs the oracle
(sfc_kernels.cu:19-173 restated in oracle/graph_oracle.c)."""
import numpy as np
import pytest
import torch

import oracle
from dynamis_amd.dynamis_state import dynamis_state_impl as impl

pytestmark = pytest.mark.gpu


def _pos(n, seed, lo=-40.0, hi=60.0):
    return np.random.default_rng(seed).uniform(lo, hi, (n, 3)).astype(np.float32)


@pytest.mark.parametrize("curve", [0, 1])
@pytest.mark.parametrize("n", [1, 17, 100_000])
def test_keys_bit_exact(cuda, curve, n):
    print(f"\n[case] sfc keys curve={curve} n={n}", flush=True)
    p = _pos(n, n + curve)
    k = impl.sfc_keys(torch.from_numpy(p).to(cuda), curve).cpu().numpy()
    want = oracle.morton_keys(p) if curve == 0 else oracle.hilbert_keys(p)
    assert np.array_equal(k, want)


def test_keys_degenerate_axis(cuda):
    p = _pos(1000, 5)
    p[:, 1] = 3.25  # zero range -> 1
    for curve in (0, 1):
        k = impl.sfc_keys(torch.from_numpy(p).to(cuda), curve).cpu().numpy()
        want = oracle.morton_keys(p) if curve == 0 else oracle.hilbert_keys(p)
        assert np.array_equal(k, want)


@pytest.mark.parametrize("n", [1, 4095, 4096, 4097, 65536 * 3 + 17])
@pytest.mark.parametrize("kind", ["one byte", "two far bytes", "sign", "top byte", "all bytes"])
def test_order_varying_bytes(cuda, n, kind):
    # keys that vary in chosen bytes only: the device-side pass plan skips the others
    print(f"\n[case] sfc order bytes n={n} {kind}", flush=True)
    rng = np.random.default_rng(n + len(kind))
    if kind == "one byte":
        keys = rng.integers(0, 256, n) << 16
    elif kind == "two far bytes":
        keys = (rng.integers(0, 256, n) << 8) | (rng.integers(0, 4, n) << 48) | (123 << 24)
    elif kind == "sign":
        keys = rng.integers(-3, 3, n)
    elif kind == "top byte":
        keys = rng.integers(-128, 127, n) << 56
    else:
        keys = rng.integers(-2 ** 63, 2 ** 63 - 1, n, dtype=np.int64)
    keys = np.asarray(keys, np.int64)
    perm = impl.sfc_order(torch.from_numpy(keys).to(cuda)).cpu().numpy()
    assert np.array_equal(perm, np.argsort(keys, kind="stable"))


@pytest.mark.parametrize("n", [1, 1000, 300_001, 1_000_000, 2_200_001])
def test_order_is_stable_argsort(cuda, n):
    print(f"\n[case] sfc order n={n}", flush=True)
    rng = np.random.default_rng(n)
    keys = rng.integers(-2 ** 40, 2 ** 40, n) // 1000  # plenty of ties
    keys[: n // 3] = rng.integers(0, 5, n // 3)
    perm = impl.sfc_order(torch.from_numpy(keys).to(cuda)).cpu().numpy()
    assert np.array_equal(perm, np.argsort(keys, kind="stable"))
    same = np.full(n, 7, np.int64)
    assert np.array_equal(impl.sfc_order(torch.from_numpy(same).to(cuda)).cpu().numpy(), np.arange(n))


@pytest.mark.parametrize("curve", [0, 1])
@pytest.mark.parametrize("W", [1, 3, 8])
def test_partition_labels(cuda, curve, W):
    p = _pos(50_000, 9)
    pt = torch.from_numpy(p).to(cuda)
    lab = impl.sfc_partition_cuda(pt, None, W, curve).cpu().numpy()
    keys = oracle.morton_keys(p) if curve == 0 else oracle.hilbert_keys(p)
    perm = np.argsort(keys, kind="stable")
    assert np.array_equal(lab, oracle.sfc_labels(perm, W))
    w = np.random.default_rng(1).integers(0, 200, 50_000)
    labw = impl.sfc_partition_cuda(pt, torch.from_numpy(w).to(cuda), W, curve).cpu().numpy()
    assert np.array_equal(labw, oracle.sfc_labels(perm, W, w))


def test_hilbert_keys_exhaustive_grid(cuda):
    """All 128^3 quantised cells (plus the two bounding corners): GPU "Hilbert" keys equal
    the restatement of the reference's CPU twin (sfc_partitioner.cpp:50-92) cell by cell."""
    from oracle import sfc_twin

    print("\n[case] hilbert keys, exhaustive 128^3 grid", flush=True)
    pos, X, Y, Z = sfc_twin.grid_positions(128, 1.0)
    k = impl.sfc_keys(torch.from_numpy(pos).to(cuda), 1).cpu().numpy()
    assert np.array_equal(k[:-2], sfc_twin.hilbert_from_grid(X, Y, Z))
    assert np.array_equal(k, oracle.hilbert_keys(pos))


@pytest.mark.parametrize("name", ["C2-like 60k fp32", "C4 triclinic fp64"])
def test_build_after_sfc_permutation(cuda, name):
    """The reference API's SFC reorder followed by the build (what bench.py's
    sfc_permuted_rebuild times): Morton keys, stable order, positions gathered into that
    order on the device, then radius_graph_pbc_ex.  Mapped back through the permutation,
    the edge set and the per-atom degrees must be the build's on the original order."""
    from dynamis_amd import configs

    box = configs.uniform(60_000, seed=71, dtype=np.float32) if name.startswith("C2") else configs.c4(scale=0.6)
    print(f"\n[case] build after sfc permutation {name} N={len(box.pos)}", flush=True)
    pos = torch.from_numpy(box.pos).to(cuda)
    cell = torch.from_numpy(np.asarray(box.cell, np.float64))
    pbc = torch.tensor(list(box.pbc))
    keys = impl.sfc_keys(pos.float(), 0)
    perm = impl.sfc_order(keys)
    assert np.array_equal(perm.cpu().numpy(), np.argsort(keys.cpu().numpy(), kind="stable"))
    ppos = torch.index_select(pos, 0, perm)
    e0, s0, n0, c0 = impl.radius_graph_pbc_ex(pos, cell, pbc, box.radius, 0, False)
    e1, s1, n1, c1 = impl.radius_graph_pbc_ex(ppos, cell, pbc, box.radius, 0, False)
    p = perm.cpu().numpy()
    assert int(n0.item()) == int(n1.item()) > 0
    # degrees: atom p[i] of the original is atom i of the permuted build
    deg = np.empty(len(p), np.int32)
    deg[p] = c1.cpu().numpy()
    assert np.array_equal(deg, c0.cpu().numpy())
    got = oracle.canonical_sort(p[e1[0].cpu().numpy()], p[e1[1].cpu().numpy()], s1.cpu().numpy().astype(np.int64))
    want = oracle.canonical_sort(e0[0].cpu().numpy(), e0[1].cpu().numpy(), s0.cpu().numpy().astype(np.int64))
    for a, b in zip(got, want):
        assert np.array_equal(a, b)
