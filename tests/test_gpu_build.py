"""GPU tests of the one-call build (dg_graph_build, C ABI): it must produce exactly the
bytes of the two-stage build (dg_graph_count + dg_graph_write, itself checked against
the oracle in test_gpu_graph.py) -- same edges in the same order, same counts -- on the
cases that exercise every path of the fused kernel (slot expansion, targets past the slot
capacity, chunked dense regions, explicit targets, edge vectors), and report the edge
count with DG_ERR_CAPACITY when the preallocated buffers are too small."""
import numpy as np
import pytest
import torch

from dynamis_amd import _lib as L
from dynamis_amd import configs
from dynamis_amd.dynamis_state import dynamis_state_impl as impl

pytestmark = pytest.mark.gpu


def _one_call(pos, cell, pbc, r, targets, capacity, vdt=None, vec_offset=0):
    lib = L.lib()
    d = impl._desc(pos, cell, pbc, impl._r32(r), targets)
    dev = pos.device
    wsb = lib.dg_graph_workspace_size(d)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    nt = pos.shape[0] if targets is None else targets.shape[0]
    cnt = torch.empty(nt, dtype=torch.int32, device=dev)
    ei = torch.full((2, capacity), -7, dtype=torch.int64, device=dev)
    sh = torch.full((capacity, 3), -7.0, dtype=torch.float32, device=dev)
    vec = dist = None
    if vdt is not None:
        # vec_offset elements in: outputs off the 16-byte alignment the grouped stores need
        vec = torch.empty(3 * capacity + vec_offset, dtype=vdt, device=dev)[vec_offset:].view(capacity, 3)
        dist = torch.empty(capacity + vec_offset, dtype=vdt, device=dev)[vec_offset:]
    s = L.stream_of(dev)
    st = lib.dg_graph_build(d, L.ptr(pos), L.ptr(targets), L.ptr(ws), wsb, capacity, L.ptr(cnt),
                            L.ctypes.c_void_p(ei.data_ptr()),
                            L.ctypes.c_void_p(ei.data_ptr() + 8 * capacity), L.ptr(sh), L.ptr(vec),
                            L.ptr(dist), L.DG_F64 if vdt == torch.float64 else L.DG_F32, s)
    L.check(st, "dg_graph_build")
    E, fl = L._i64(0), L._i64(0)
    st = lib.dg_graph_read_totals(d, L.ptr(ws), E, fl, s)
    return st, int(E.value), ei, sh, cnt, vec, dist


def _cases():
    out = []
    b = configs.uniform(60000, seed=31, dtype=np.float32)
    out.append(("uniform", b.pos, b.cell, b.pbc, b.radius, None))
    b = configs.c4(scale=0.4)
    out.append(("c4", b.pos, b.cell, b.pbc, b.radius, None))
    rng = np.random.default_rng(13)
    out.append(("dense", (rng.uniform(0, 1, (1500, 3)) * 8.0).astype(np.float32), np.eye(3) * 8.0,
                (True, True, True), 6.0, None))
    # a clump: targets far past the slot capacity, in a tile whose region fits LDS
    p = rng.uniform(0, 40.0, (6000, 3))
    p[:400] = 20.0 + rng.uniform(-1.2, 1.2, (400, 3))
    out.append(("clump", p.astype(np.float32), np.eye(3) * 40.0, (True, True, True), 5.0, None))
    b = configs.uniform(8000, seed=21, dtype=np.float32)
    tg = rng.choice(8000, 1500, replace=False)
    out.append(("targets", b.pos, b.cell, b.pbc, b.radius, np.r_[tg, tg[:40]]))
    out.append(("partial", b.pos, b.cell, (True, False, True), b.radius, None))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: c[0])
def test_matches_two_stage_bytes(cuda, case):
    name, pos, cell, pbc, r, tg = case
    print(f"\n[case] one-call build {name} N={len(pos)}", flush=True)
    p = torch.from_numpy(np.ascontiguousarray(pos)).to(cuda)
    c = torch.from_numpy(np.asarray(cell, np.float64))
    b = torch.tensor([bool(x) for x in pbc])
    t = None if tg is None else torch.from_numpy(np.asarray(tg, np.int64)).to(cuda)
    ei, co, nn, cnt = impl.radius_graph_pbc_ex(p, c, b, r, 0, False, t)
    E = ei.shape[1]
    for rep in range(2):  # the second call reuses nothing but must agree again
        st, E1, ei1, sh1, cnt1, _, _ = _one_call(p, c, b, r, t, E + 5)
        assert st == L.DG_OK and E1 == E
        assert torch.equal(cnt1, cnt)
        assert torch.equal(ei1[:, :E], ei) and torch.equal(sh1[:E], co)
        assert bool((ei1[:, E:] == -7).all()) and bool((sh1[E:] == -7.0).all())  # untouched


def test_vectors_match(cuda):
    b = configs.uniform(20000, seed=5, dtype=np.float32)
    p = torch.from_numpy(b.pos).to(cuda)
    c = torch.from_numpy(b.cell)
    bb = torch.tensor([True] * 3)
    ei, co, nn, cnt, vec, dist = impl.radius_graph_pbc_vectors(p, c, bb, b.radius, None,
                                                               vector_dtype=torch.float64)
    E = ei.shape[1]
    st, E1, ei1, sh1, _, vec1, dist1 = _one_call(p, c, bb, b.radius, None, E, torch.float64)
    assert st == L.DG_OK and E1 == E
    assert torch.equal(ei1, ei) and torch.equal(sh1, co)
    assert torch.equal(vec1, vec) and torch.equal(dist1, dist)


def test_capacity_too_small_reports_count(cuda):
    b = configs.uniform(30000, seed=9, dtype=np.float32)
    p = torch.from_numpy(b.pos).to(cuda)
    c = torch.from_numpy(b.cell)
    bb = torch.tensor([True] * 3)
    _, _, nn, _ = impl.radius_graph_pbc_ex(p, c, bb, b.radius, 0, False, None)
    E = int(nn.item())
    st, E1, ei1, _, _, _, _ = _one_call(p, c, bb, b.radius, None, E // 2)
    assert st == L.DG_ERR_CAPACITY and E1 == E
    assert "capacity" in L.lib().dg_last_error().decode()


@pytest.mark.parametrize("case", _cases(), ids=lambda c: c[0])
def test_vectors_grouped_equal_per_lane(cuda, case):
    """Edge vectors and distances written in 16-byte groups (outputs aligned to 16 bytes)
    must be the bytes the per-lane writer gives (outputs one element off that alignment),
    for fp32 and fp64 vectors, with the edges themselves unchanged."""
    name, pos, cell, pbc, r, tg = case
    p = torch.from_numpy(np.ascontiguousarray(pos)).to(cuda)
    c = torch.from_numpy(np.asarray(cell, np.float64))
    b = torch.tensor([bool(x) for x in pbc])
    t = None if tg is None else torch.from_numpy(np.asarray(tg, np.int64)).to(cuda)
    ei, co, nn, cnt = impl.radius_graph_pbc_ex(p, c, b, r, 0, False, t)
    E = ei.shape[1]
    for vdt in (torch.float32, torch.float64):
        print(f"\n[case] vectors {name} N={len(pos)} {vdt}", flush=True)
        st, E1, ei1, sh1, _, vec1, dist1 = _one_call(p, c, b, r, t, E + 3, vdt)
        st2, E2, ei2, sh2, _, vec2, dist2 = _one_call(p, c, b, r, t, E + 3, vdt, vec_offset=1)
        assert st == st2 == L.DG_OK and E1 == E2 == E
        assert vec1.data_ptr() % 16 == 0 and vec2.data_ptr() % 16 != 0
        assert torch.equal(ei1[:, :E], ei) and torch.equal(sh1[:E], co)
        assert torch.equal(ei2[:, :E], ei) and torch.equal(sh2[:E], co)
        assert torch.equal(vec1[:E], vec2[:E]) and torch.equal(dist1[:E], dist2[:E])
        # and the vectors are the edges' own (|v| = dist, |v| <= r)
        assert torch.allclose(vec1[:E].double().norm(dim=1), dist1[:E].double(), rtol=1e-6, atol=0)
        assert float(dist1[:E].max()) <= float(np.float32(r)) * (1 + 1e-6)


def _write(pos, cell, pbc, r, targets, cap, out_ids, vdt=None, vec_offset=0):
    lib = L.lib()
    d = impl._desc(pos, cell, pbc, impl._r32(r), targets)
    dev = pos.device
    wsb = lib.dg_graph_workspace_size(d)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    nt = pos.shape[0] if targets is None else targets.shape[0]
    cnt = torch.empty(nt, dtype=torch.int32, device=dev)
    s = L.stream_of(dev)
    L.check(lib.dg_graph_count(d, L.ptr(pos), L.ptr(targets), L.ptr(ws), wsb, L.ptr(cnt), s), "count")
    ei = torch.full((2, cap), -1, dtype=torch.int64, device=dev)
    sh = torch.full((cap, 3), -1.0, dtype=torch.float32, device=dev)
    vec = dist = None
    if vdt is not None:
        vec = torch.empty(3 * cap + vec_offset, dtype=vdt, device=dev)[vec_offset:].view(cap, 3)
        dist = torch.empty(cap + vec_offset, dtype=vdt, device=dev)[vec_offset:]
    L.check(lib.dg_graph_write_ids(d, L.ptr(pos), L.ptr(targets), L.ptr(ws), wsb, cap, L.ptr(out_ids),
                                   L.ctypes.c_void_p(ei.data_ptr()), L.ctypes.c_void_p(ei.data_ptr() + 8 * cap),
                                   L.ptr(sh), L.ptr(vec), L.ptr(dist),
                                   L.DG_F64 if vdt == torch.float64 else L.DG_F32, s), "write_ids")
    E, fl = L._i64(0), L._i64(0)
    L.check(lib.dg_graph_read_totals(d, L.ptr(ws), E, fl, s), "totals")
    return int(E.value), ei, sh, vec, dist


def _ids_cases():
    out = list(_cases())
    rng = np.random.default_rng(17)
    small = np.eye(3) * 3.0  # the radius spans several cells: the all-pairs kernel
    out.append(("all-pairs", (rng.uniform(0, 1, (40, 3)) @ small).astype(np.float32), small, (True, True, True),
                7.0, None))
    return out


@pytest.mark.parametrize("case", _ids_cases(), ids=lambda c: c[0])
def test_write_ids_is_the_remapped_write(cuda, case):
    """dg_graph_write_ids (the ids written for the atoms mapped, as DistGraphBuilder's steady
    step needs) gives the plain write's edges with src and dst replaced by out_ids[src],
    out_ids[dst], and the same shifts, vectors and distances -- on every path: the grouped
    expansion, the fix-up pass (dense and clumped cases), grouped and per-lane vectors, and
    the all-pairs kernel."""
    name, pos, cell, pbc, r, tg = case
    p = torch.from_numpy(np.ascontiguousarray(pos)).to(cuda)
    c = torch.from_numpy(np.asarray(cell, np.float64))
    b = torch.tensor([bool(x) for x in pbc])
    t = None if tg is None else torch.from_numpy(np.asarray(tg, np.int64)).to(cuda)
    n = p.shape[0]
    ids = torch.from_numpy(np.random.default_rng(3).choice(2_000_000_000, n, replace=False)).to(cuda)
    ei0, co0, _, _ = impl.radius_graph_pbc_ex(p, c, b, r, 0, False, t)
    E0 = ei0.shape[1]
    for vdt, off in ((None, 0), (torch.float32, 0), (torch.float32, 1), (torch.float64, 0)):
        print(f"\n[case] write_ids {name} N={n} vectors={vdt} offset={off}", flush=True)
        E1, ei1, sh1, v1, d1 = _write(p, c, b, r, t, E0 + 4, None, vdt, off)
        E2, ei2, sh2, v2, d2 = _write(p, c, b, r, t, E0 + 4, ids, vdt, off)
        assert E1 == E2 == E0
        assert torch.equal(ei2[:, :E0], ids[ei1[:, :E0]])
        assert torch.equal(sh2[:E0], sh1[:E0])
        if vdt is not None:
            assert torch.equal(v2[:E0], v1[:E0]) and torch.equal(d2[:E0], d1[:E0])


@pytest.mark.parametrize("case", _cases(), ids=lambda c: c[0])
def test_counts_only(cuda, case):
    """dg_graph_counts (no neighbour lists recorded) gives dg_graph_count's per-target counts
    and edge total, and a write after it (every tile then from the fix-up pass) still gives
    the bytes of the ordinary two-stage build."""
    name, pos, cell, pbc, r, tg = case
    print(f"\n[case] counts only {name} N={len(pos)}", flush=True)
    p = torch.from_numpy(np.ascontiguousarray(pos)).to(cuda)
    c = torch.from_numpy(np.asarray(cell, np.float64))
    b = torch.tensor([bool(x) for x in pbc])
    t = None if tg is None else torch.from_numpy(np.asarray(tg, np.int64)).to(cuda)
    ei, co, nn, cnt = impl.radius_graph_pbc_ex(p, c, b, r, 0, False, t)
    cnt2 = impl.radius_graph_pbc_counts_ex(p, c, b, r, t)
    assert torch.equal(cnt2, cnt)
    lib = L.lib()
    d = impl._desc(p, c, b, impl._r32(r), t)
    wsb = lib.dg_graph_workspace_size(d)
    ws = torch.empty(wsb, dtype=torch.uint8, device=cuda)
    s = L.stream_of(cuda)
    cnt3 = torch.empty_like(cnt)
    L.check(lib.dg_graph_counts(d, L.ptr(p), L.ptr(t), L.ptr(ws), wsb, L.ptr(cnt3), s), "counts")
    E, fl = L._i64(0), L._i64(0)
    L.check(lib.dg_graph_read_totals(d, L.ptr(ws), E, fl, s), "totals")
    assert int(E.value) == ei.shape[1] and torch.equal(cnt3, cnt)
    E = ei.shape[1]
    ei4 = torch.full((2, E), -1, dtype=torch.int64, device=cuda)
    sh4 = torch.full((E, 3), -1.0, dtype=torch.float32, device=cuda)
    L.check(lib.dg_graph_write(d, L.ptr(p), L.ptr(t), L.ptr(ws), wsb, E, L.ctypes.c_void_p(ei4.data_ptr()),
                               L.ctypes.c_void_p(ei4.data_ptr() + 8 * E), L.ptr(sh4), None, None, L.DG_F32, s),
            "write")
    torch.cuda.synchronize()
    assert torch.equal(ei4, ei) and torch.equal(sh4, co)
