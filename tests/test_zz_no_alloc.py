"""dg_graph_build_noalloc (the allocation-free build, C ABI) against dg_graph_build with a
caller workspace: byte-identical edges, shifts, counts (and edge vectors and distances),
and the same {edge count, flags}, on two calls in a row -- the second on a smaller input,
so stale contents of the shared static scratch from the first call would show -- and a
build too large for the scratch is refused before anything runs."""
import numpy as np
import pytest
import torch

from dynamis_amd import _lib as L
from dynamis_amd import configs
from dynamis_amd.dynamis_state import dynamis_state_impl as impl

pytestmark = pytest.mark.gpu


def _desc(box, dev):
    pos = torch.from_numpy(box.pos).to(dev)
    tgt = None if box.targets is None else torch.from_numpy(box.targets).to(dev)
    d = impl._desc(pos, torch.from_numpy(np.asarray(box.cell, np.float64)),
                   torch.tensor([bool(x) for x in box.pbc]), impl._r32(box.radius), tgt)
    return d, pos, tgt


def _outputs(cap, nt, dev):
    ei = torch.full((2, cap), -7, dtype=torch.int64, device=dev)
    sh = torch.full((cap, 3), -7.0, dtype=torch.float32, device=dev)
    cnt = torch.full((nt,), -7, dtype=torch.int32, device=dev)
    return ei, sh, cnt


def _vec_outputs(cap, dev, vectors):
    if not vectors:
        return None, None
    return (torch.full((cap, 3), -7.0, dtype=torch.float32, device=dev),
            torch.full((cap,), -7.0, dtype=torch.float32, device=dev))


def _with_workspace(box, dev, cap, vectors=False):
    lib = L.lib()
    d, pos, tgt = _desc(box, dev)
    wsb = lib.dg_graph_workspace_size(d)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    ei, sh, cnt = _outputs(cap, pos.shape[0] if tgt is None else tgt.shape[0], dev)
    vec, dist = _vec_outputs(cap, dev, vectors)
    s = L.stream_of(dev)
    L.check(lib.dg_graph_build(d, L.ptr(pos), L.ptr(tgt), L.ptr(ws), wsb, cap, L.ptr(cnt),
                               L.ctypes.c_void_p(ei.data_ptr()), L.ctypes.c_void_p(ei.data_ptr() + 8 * cap),
                               L.ptr(sh), L.ptr(vec), L.ptr(dist), L.DG_F32, s), "dg_graph_build")
    E, fl = L._i64(0), L._i64(0)
    L.check(lib.dg_graph_read_totals(d, L.ptr(ws), E, fl, s), "totals")
    if vectors:
        return int(E.value), int(fl.value), ei, sh, cnt, vec, dist
    return int(E.value), int(fl.value), ei, sh, cnt


def _no_alloc(box, dev, cap, vectors=False):
    lib = L.lib()
    d, pos, tgt = _desc(box, dev)
    ei, sh, cnt = _outputs(cap, pos.shape[0] if tgt is None else tgt.shape[0], dev)
    vec, dist = _vec_outputs(cap, dev, vectors)
    tot = torch.full((2,), -7, dtype=torch.int64, device=dev)
    s = L.stream_of(dev)
    L.check(lib.dg_graph_build_noalloc(d, L.ptr(pos), L.ptr(tgt), cap, L.ptr(cnt),
                                       L.ctypes.c_void_p(ei.data_ptr()),
                                       L.ctypes.c_void_p(ei.data_ptr() + 8 * cap), L.ptr(sh), L.ptr(vec),
                                       L.ptr(dist), L.DG_F32, L.ptr(tot), s), "dg_graph_build_noalloc")
    torch.cuda.synchronize()
    t = tot.cpu().tolist()
    if vectors:
        return int(t[0]), int(t[1]), ei, sh, cnt, vec, dist
    return int(t[0]), int(t[1]), ei, sh, cnt


def test_no_alloc_matches_workspace_build(cuda):
    # two calls in a row on the shared scratch, the second on a smaller input
    boxes = [("uniform 60000", configs.uniform(60000, seed=31, dtype=np.float32)),
             ("uniform 9000", configs.uniform(9000, seed=32, dtype=np.float32)),
             ("C5 small, explicit targets", configs.c5(n_owned=12_000, side=49.3))]
    for name, box in boxes:
        print(f"\n[case] noalloc {name} N={len(box.pos)}", flush=True)
        E, fl, ei, sh, cnt = _with_workspace(box, cuda, int(len(box.pos) * 100))
        cap = E + 64
        E, fl, ei, sh, cnt = _with_workspace(box, cuda, cap)
        E2, fl2, ei2, sh2, cnt2 = _no_alloc(box, cuda, cap)
        assert (E2, fl2) == (E, fl) and E > 0
        assert torch.equal(cnt2, cnt)
        assert torch.equal(ei2[:, :E], ei[:, :E])
        assert torch.equal(sh2[:E], sh[:E])
        assert bool((ei2[:, E:] == -7).all())  # nothing written past the edges


def test_no_alloc_vectors(cuda):
    # edge vectors and distances too (their cell-ordered positions live in the scratch):
    # two calls in a row, the second smaller
    for name, box in [("uniform 40000", configs.uniform(40000, seed=33, dtype=np.float32)),
                      ("uniform 7000", configs.uniform(7000, seed=34, dtype=np.float32))]:
        print(f"\n[case] noalloc vectors {name} N={len(box.pos)}", flush=True)
        E, *_ = _with_workspace(box, cuda, int(len(box.pos) * 100))
        cap = E + 64
        E, fl, ei, sh, cnt, vec, dist = _with_workspace(box, cuda, cap, vectors=True)
        E2, fl2, ei2, sh2, cnt2, vec2, dist2 = _no_alloc(box, cuda, cap, vectors=True)
        assert (E2, fl2) == (E, fl) and E > 0
        assert torch.equal(cnt2, cnt) and torch.equal(ei2[:, :E], ei[:, :E]) and torch.equal(sh2[:E], sh[:E])
        assert torch.equal(vec2[:E], vec[:E]) and torch.equal(dist2[:E], dist[:E])
        assert bool((vec2[E:] == -7.0).all()) and bool((dist2[E:] == -7.0).all())


def test_no_alloc_capacity_and_limit(cuda):
    lib = L.lib()
    box = configs.uniform(9000, seed=32, dtype=np.float32)
    E, fl, *_ = _with_workspace(box, cuda, 9000 * 100)
    print("\n[case] noalloc capacity", flush=True)
    E2, fl2, *_ = _no_alloc(box, cuda, E // 2)
    assert E2 == E and (fl2 & 4)  # DG_FLAG_CAPACITY
    # a build whose workspace exceeds the static scratch is refused before any launch
    big = configs.uniform(400_000, seed=1, dtype=np.float32)
    d, pos, tgt = _desc(big, cuda)
    assert lib.dg_graph_workspace_size(d) > (64 << 20)
    tot = torch.zeros(2, dtype=torch.int64, device=cuda)
    st = lib.dg_graph_build_noalloc(d, L.ptr(pos), None, 16, None, L.ptr(tot), L.ptr(tot), L.ptr(tot),
                                    None, None, L.DG_F32, L.ptr(tot), L.stream_of(cuda))
    assert st == L.DG_ERR_WORKSPACE
    assert b"static scratch" in lib.dg_last_error()


def test_no_alloc_at_the_scratch_limit(cuda):
    # the largest uniform box whose workspace still fits the 64 MiB scratch, byte for byte
    lib = L.lib()

    def box_of(n):
        return configs.uniform(n, seed=35, dtype=np.float32)

    def wsb(n):
        d, *_ = _desc(box_of(n), torch.device("cpu"))
        return lib.dg_graph_workspace_size(d)

    lo, hi = 50_000, 400_000
    while hi - lo > 1:
        m = (lo + hi) // 2
        lo, hi = (m, hi) if wsb(m) <= (64 << 20) else (lo, m)
    assert (64 << 20) - wsb(lo) < (1 << 20) < wsb(lo + 1) - (64 << 20) + (1 << 20)
    box = box_of(lo)
    print(f"\n[case] noalloc at the limit N={lo} workspace={wsb(lo)}", flush=True)
    E, *_ = _with_workspace(box, cuda, int(lo * 100))
    cap = E + 64
    E, fl, ei, sh, cnt = _with_workspace(box, cuda, cap)
    E2, fl2, ei2, sh2, cnt2 = _no_alloc(box, cuda, cap)
    assert (E2, fl2) == (E, fl) and E > 0
    assert torch.equal(cnt2, cnt) and torch.equal(ei2, ei) and torch.equal(sh2, sh)
    # one atom more does not fit
    d, pos, _ = _desc(box_of(lo + 1), cuda)
    tot = torch.zeros(2, dtype=torch.int64, device=cuda)
    st = lib.dg_graph_build_noalloc(d, L.ptr(pos), None, 16, None, L.ptr(tot), L.ptr(tot), L.ptr(tot),
                                    None, None, L.DG_F32, L.ptr(tot), L.stream_of(cuda))
    assert st == L.DG_ERR_WORKSPACE


def test_no_alloc_explicit_targets_with_vectors(cuda):
    # random explicit targets (the target sort path) with edge vectors: two calls, the
    # second smaller
    rng = np.random.default_rng(36)
    for n, nt in [(30000, 11000), (8000, 900)]:
        box = configs.uniform(n, seed=37 + n, dtype=np.float32)
        box.targets = rng.permutation(rng.choice(n, nt, replace=False)).astype(np.int64)
        print(f"\n[case] noalloc targets + vectors N={n} nt={nt}", flush=True)
        E, *_ = _with_workspace(box, cuda, int(nt * 100))
        cap = E + 64
        E, fl, ei, sh, cnt, vec, dist = _with_workspace(box, cuda, cap, vectors=True)
        E2, fl2, ei2, sh2, cnt2, vec2, dist2 = _no_alloc(box, cuda, cap, vectors=True)
        assert (E2, fl2) == (E, fl) and E > 0
        assert torch.equal(cnt2, cnt) and torch.equal(ei2, ei) and torch.equal(sh2, sh)
        assert torch.equal(vec2, vec) and torch.equal(dist2, dist)


def test_no_alloc_refuses_an_overlapping_call(cuda):
    # a call on stream B while the previous call's work on stream A is still pending
    # (held back behind a bounded spin kernel) is refused; once A has drained, B may call
    lib = L.lib()
    box = configs.uniform(9000, seed=32, dtype=np.float32)
    E, *_ = _with_workspace(box, cuda, 9000 * 100)
    d, pos, _ = _desc(box, cuda)
    ei, sh, cnt = _outputs(E + 64, len(box.pos), cuda)
    tot = torch.zeros(2, dtype=torch.int64, device=cuda)
    a, b = torch.cuda.Stream(cuda), torch.cuda.Stream(cuda)
    torch.cuda.synchronize()

    def call(stream):
        s = L.ctypes.c_void_p(stream.cuda_stream)
        return lib.dg_graph_build_noalloc(d, L.ptr(pos), None, E + 64, L.ptr(cnt),
                                          L.ctypes.c_void_p(ei.data_ptr()),
                                          L.ctypes.c_void_p(ei.data_ptr() + 8 * (E + 64)), L.ptr(sh),
                                          None, None, L.DG_F32, L.ptr(tot), s)

    print("\n[case] noalloc overlap guard", flush=True)
    with torch.cuda.stream(a):
        torch.cuda._sleep(200_000_000)  # ~0.1 s of spinning on stream A
    assert call(a) == L.DG_OK
    assert call(a) == L.DG_OK  # the same stream is ordered: allowed
    assert call(b) == L.DG_ERR_INVALID
    assert b"has not completed" in lib.dg_last_error()
    torch.cuda.synchronize()
    assert call(b) == L.DG_OK
    torch.cuda.synchronize()
    assert int(tot[0]) == E
