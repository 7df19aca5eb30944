"""One rank of the multi-process DistGraphBuilder tests (run as a subprocess, one per rank,
gloo over 127.0.0.1; on a one-GPU box every rank shares cuda:0).

    python tests/dist_worker.py --mode reduce|builder --rank R --world W --port P [...]

Exit status 0 = every check on this rank passed.  Mirrors the reference's torchrun
runner scripts (dynamis_state/tests/test_dist_graph_builder.py:275-653).
"""
import argparse
import datetime
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402
import torch  # noqa: E402
import torch.distributed as dist  # noqa: E402


def _canon(src, dst, shift):
    key = np.lexsort((shift[:, 2], shift[:, 1], shift[:, 0], src, dst))
    return src[key], dst[key], shift[key]


def reduce_mode(a):
    from dynamis_amd.dynamis_state.dist_graph_builder import _all_reduce_degrees

    N = 50
    mine = torch.arange(a.rank, N, a.world, dtype=torch.int64)
    deg = (mine * 3 + 1).to(torch.int32)
    full = _all_reduce_degrees(deg, mine, N)
    want = torch.arange(N, dtype=torch.int32) * 3 + 1
    return ([] if torch.equal(full, want) else [f"reduce: {full.tolist()} != {want.tolist()}"]), None


def builder_mode(a):
    import oracle
    from oracle import halo
    from dynamis_amd.dynamis_state import dynamis_state_impl as impl
    from dynamis_amd.dynamis_state.dist_graph_builder import BuildMode, DistGraphBuilder

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    R, W = a.rank, a.world
    g = torch.Generator().manual_seed(a.seed)
    N, L, r, skin = a.n, a.box, a.cutoff, 0.5
    pos = (torch.rand(N, 3, generator=g) * L).to(dev)
    cell = torch.eye(3, dtype=torch.float32) * L
    pbc = torch.tensor([True, True, True])
    env = impl.DistEnvironment()
    env.global_rank, env.world_size, env.local_rank = R, W, 0
    env.gpus_per_node, env.num_nodes = W, 1
    b = DistGraphBuilder(cell, pbc, cutoff=r, ghost_buffer=skin, env=env, refresh_interval=100)
    errs = []
    res = b.build(pos)
    if res.mode != BuildMode.REFRESH:
        errs.append("first build is not a refresh")
    pos_w = b._pbc_wrap(pos).cpu().numpy()
    c64 = np.eye(3) * L
    r32 = float(np.float32(r))
    rs32 = float(np.float32(r + skin))
    # degrees and partition
    deg, _ = oracle.radius_graph_counts(pos_w, c64, (1, 1, 1), r32)
    if not np.array_equal(res.full_degrees.cpu().numpy(), deg):
        errs.append("full_degrees differ from the oracle's r-degrees")
    keys = oracle.morton_keys(pos_w)
    perm = np.argsort(keys, kind="stable")
    pid = oracle.sfc_labels(perm, W, deg.astype(np.int64))
    if not np.array_equal(res.pid_outer.cpu().numpy(), pid):
        errs.append("pid_outer differs from the oracle's weighted SFC cut")
    my = np.nonzero(pid == R)[0]
    if not np.array_equal(res.my_outer_atoms.cpu().numpy(), my):
        errs.append("my_outer_atoms")
    # mode A edges = the graph at r restricted to my targets

    def same_edges(resx, pw, tag):
        e = resx.edges_outer.cpu().numpy()
        s = resx.cell_shifts_outer.cpu().numpy()
        w = oracle.radius_graph(pw, c64, (1, 1, 1), r32, target_indices=my)
        got = _canon(e[0], e[1], s.astype(np.int64))
        exp = _canon(w["src"], w["dst"], w["shift"].astype(np.int64))
        if not all(np.array_equal(x, y) for x, y in zip(got, exp)):
            errs.append(f"{tag}: edges differ ({e.shape[1]} vs {len(w['src'])})")
        return e.shape[1]

    same_edges(res, pos_w, "mode A")
    # halo = serial full-graph map at r + skin
    full = oracle.radius_graph(pos_w, c64, (1, 1, 1), rs32)
    hm = halo.build_halo_maps(full["src"], full["dst"], pid, R, W, N)
    info = res.halo_info
    got = [info.send_offsets, info.send_local_indices, info.recv_offsets, info.recv_ghost_indices,
           info.interior_mask, res.halo_recv_global_ids]
    for k, name in enumerate(["send_offsets", "send_local_indices", "recv_offsets",
                              "recv_ghost_indices", "interior_mask", "halo_recv_global_ids"]):
        if not np.array_equal(got[k].cpu().numpy(), hm[k]):
            errs.append(f"halo {name}")
    # send / recv lists in global ids, compared across ranks in main()
    so, sl = info.send_offsets.cpu(), info.send_local_indices.cpu()
    ro, ra = info.recv_offsets.cpu(), res.halo_recv_global_ids.cpu()
    mo = res.my_outer_atoms.cpu()
    lists = {"send": {q: mo[sl[so[q]:so[q + 1]]].tolist() for q in range(W)},
             "recv": {p: ra[ro[p]:ro[p + 1]].tolist() for p in range(W)}}
    # mode B at the same positions = mode A's edges
    res_b = b.build(pos)
    if res_b.mode != BuildMode.STEADY:
        errs.append("second build is not steady")
    same_edges(res_b, pos_w, "mode B same pos")
    # small drift: steady, and still the exact graph at r of the drifted positions
    d = (torch.rand(N, 3, generator=g) - 0.5) * 0.2
    pos2 = pos + d.to(dev)
    res_c = b.build(pos2)
    if res_c.mode != BuildMode.STEADY:
        errs.append("small drift refreshed")
    same_edges(res_c, b._pbc_wrap(pos2).cpu().numpy(), "mode B drifted")
    # large drift: refresh
    res_d = b.build(pos + 1.0)
    if res_d.mode != BuildMode.REFRESH:
        errs.append("large drift did not refresh")
    return errs, lists


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--mode", default="builder")
    ap.add_argument("--rank", type=int)
    ap.add_argument("--world", type=int)
    ap.add_argument("--port", type=int)
    ap.add_argument("--seed", type=int, default=12345)
    ap.add_argument("--n", type=int, default=500)
    ap.add_argument("--box", type=float, default=30.0)
    ap.add_argument("--cutoff", type=float, default=4.0)
    a = ap.parse_args()
    dist.init_process_group("gloo", init_method=f"tcp://127.0.0.1:{a.port}", rank=a.rank,
                            world_size=a.world, timeout=datetime.timedelta(seconds=90))
    lists = None
    try:
        errs, lists = reduce_mode(a) if a.mode == "reduce" else builder_mode(a)
    except Exception as e:  # report, then fail this rank
        errs = [f"exception: {type(e).__name__}: {e}"]
    # mirror symmetry: what rank p sends to q is what q receives from p
    every = [None] * a.world
    dist.all_gather_object(every, lists)
    if a.mode == "builder" and all(x is not None for x in every):
        for p in range(a.world):
            if p != a.rank and every[p]["send"][a.rank] != every[a.rank]["recv"][p]:
                errs.append(f"mirror {p}->{a.rank}")
    for e in errs:
        print(f"[rank {a.rank}] ERROR {e}", flush=True)
    bad = torch.tensor([len(errs)], dtype=torch.int64)
    dist.all_reduce(bad)
    print(f"[rank {a.rank}] errors here {len(errs)}, all ranks {int(bad.item())}", flush=True)
    dist.destroy_process_group()
    sys.exit(0 if int(bad.item()) == 0 else 1)


if __name__ == "__main__":
    main()
