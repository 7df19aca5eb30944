"""One build (dg_graph_build, C ABI, caller-owned buffers) captured in a HIP graph and
replayed: it records no memset and no host synchronisation, so a molecular-dynamics loop
can capture it once and replay it every step.  The graph is replayed several times with
eager work (positions moved in place) and synchronisations between the replays, and every
replay must give the bytes of an eager build of the same positions, edge count included."""
import numpy as np
import pytest
import torch

from dynamis_amd import _lib as L
from dynamis_amd import configs
from dynamis_amd.dynamis_state import dynamis_state_impl as impl

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["uniform fp32", "c4 fp64"])
def test_build_replays_in_a_graph(cuda, name):
    box = configs.uniform(30000, seed=41, dtype=np.float32) if name == "uniform fp32" else configs.c4(scale=0.5)
    print(f"\n[case] graph capture {name} N={len(box.pos)}", flush=True)
    lib = L.lib()
    pos = torch.from_numpy(np.ascontiguousarray(box.pos)).to(cuda)
    cell = torch.from_numpy(np.asarray(box.cell, np.float64))
    pbc = torch.tensor([bool(x) for x in box.pbc])
    d = impl._desc(pos, cell, pbc, impl._r32(box.radius), None)
    n = pos.shape[0]
    wsb = lib.dg_graph_workspace_size(d)
    E0 = impl.radius_graph_pbc_ex(pos, cell, pbc, box.radius, 0, False, None)[0].shape[1]
    cap = int(E0 * 1.2) + 1024

    def buffers():
        return (torch.empty(wsb, dtype=torch.uint8, device=cuda), torch.empty(n, dtype=torch.int32, device=cuda),
                torch.full((2, cap), -1, dtype=torch.int64, device=cuda),
                torch.full((cap, 3), -1.0, dtype=torch.float32, device=cuda))

    def build(ws, cnt, ei, sh, stream):
        L.check(lib.dg_graph_build(d, L.ptr(pos), None, L.ptr(ws), wsb, cap, L.ptr(cnt),
                                   L.ctypes.c_void_p(ei.data_ptr()), L.ctypes.c_void_p(ei.data_ptr() + 8 * cap),
                                   L.ptr(sh), None, None, L.DG_F32, stream), "dg_graph_build")

    def total(ws):
        E, fl = L._i64(0), L._i64(0)
        L.check(lib.dg_graph_read_totals(d, L.ptr(ws), E, fl, L.stream_of(cuda)), "totals")
        return int(E.value)

    g_ws, g_cnt, g_ei, g_sh = buffers()
    side = torch.cuda.Stream(device=cuda)
    side.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(side):  # a warm-up on the capture stream (library initialisation)
        build(g_ws, g_cnt, g_ei, g_sh, L.stream_of(cuda))
    torch.cuda.current_stream(cuda).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        build(g_ws, g_cnt, g_ei, g_sh, L.stream_of(cuda))
    torch.cuda.synchronize()
    gen = torch.Generator(device=cuda).manual_seed(5)
    e_ws, e_cnt, e_ei, e_sh = buffers()
    for rep in range(5):
        # eager work between the replays: the positions move in place
        pos.add_(torch.randn(pos.shape, device=cuda, dtype=pos.dtype, generator=gen) * 0.02)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        Eg = total(g_ws)
        build(e_ws, e_cnt, e_ei, e_sh, L.stream_of(cuda))
        Ee = total(e_ws)
        assert Eg == Ee and 0 < Eg <= cap, (rep, Eg, Ee)
        assert torch.equal(g_cnt, e_cnt)
        assert torch.equal(g_ei[:, :Eg], e_ei[:, :Ee]) and torch.equal(g_sh[:Eg], e_sh[:Ee])


def test_sfc_order_replays_in_a_graph(cuda):
    """dg_sfc_order (keys -> stable permutation) captured once and replayed over new keys
    written in place between the replays: it has no host synchronisation (the passes it
    needs are chosen on the device), so every replay must equal the eager order and a
    stable argsort, including replays whose keys vary in other bytes than the captured
    call's keys did."""
    lib = L.lib()
    n = 250_003
    rng = np.random.default_rng(77)
    keys = torch.from_numpy(rng.integers(0, 2 ** 21, n).astype(np.int64)).to(cuda)
    wsb = lib.dg_sfc_workspace_size(n)
    g_ws = torch.empty(wsb, dtype=torch.uint8, device=cuda)
    g_perm = torch.full((n,), -1, dtype=torch.int64, device=cuda)

    def order(ws, perm):
        L.check(lib.dg_sfc_order(L.ptr(keys), n, L.ptr(perm), L.ptr(ws), wsb, L.stream_of(cuda)), "dg_sfc_order")

    side = torch.cuda.Stream(device=cuda)
    side.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(side):
        order(g_ws, g_perm)
    torch.cuda.current_stream(cuda).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        order(g_ws, g_perm)
    torch.cuda.synchronize()
    e_ws = torch.empty(wsb, dtype=torch.uint8, device=cuda)
    e_perm = torch.empty(n, dtype=torch.int64, device=cuda)
    cases = [rng.integers(0, 2 ** 21, n), rng.integers(-2 ** 62, 2 ** 62, n), np.full(n, -5),
             rng.integers(0, 3, n) << 40, rng.integers(-2 ** 20, 2 ** 20, n) * 7]
    for rep, k in enumerate(cases):
        print(f"\n[case] sfc order graph replay {rep}", flush=True)
        keys.copy_(torch.from_numpy(np.asarray(k, np.int64)))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        order(e_ws, e_perm)
        torch.cuda.synchronize()
        want = np.argsort(np.asarray(k, np.int64), kind="stable")
        assert np.array_equal(g_perm.cpu().numpy(), want), rep
        assert torch.equal(g_perm, e_perm)
