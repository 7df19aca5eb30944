"""Benchmark: full PBC radius-graph rebuild (SFC reorder + cell-list sort + count + write)
of the 1M-atom, r_cut = 6 A uniform box (config C3) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C3] [--no-cpu]

One step = one full rebuild through the C ABI (dg_graph_build, issued as its two calls
dg_graph_count + dg_graph_write) into preallocated output buffers, positions already
resident in HBM, no host sync inside the step.  Prints ONE JSON line.  `roofline` is for
the dominant kernel, the edge expansion of the write stage (expand_kernel, followed by the
search_kernel<1> fix-up pass, which exits at once on tiles without fix-up work), timed
with HIP events on the stream it runs on.  `cpu_baseline` times the CPU oracle (a restatement of the
reference algorithm) on the same box on this host.
"""
from __future__ import annotations

import argparse
import ctypes
import itertools
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
WRITE_BYTES_PER_EDGE = 28   # edge_index int64 x2 + cell shift fp32 x3
VECTOR_BYTES_PER_EDGE = 16  # with --vectors: edge vector fp32 x3 + distance fp32
METRIC = "Gedges/s and ms per full rebuild, 1M atoms r_cut=6 Å, 1 GPU; % HBM peak"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="C3")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--trajectory", type=int, default=-1,
                    help="rebuild from this many position frames, each the previous one displaced "
                         "by Gaussian --sigma per coordinate, cycled over the steps (all resident in "
                         "HBM before the timed region); 0 = the same positions every step.  "
                         "Default: 100 for C5 (its stated 100 rebuilds at 0.01 A per step), else 0")
    ap.add_argument("--sigma", type=float, default=0.01)
    ap.add_argument("--vectors", action="store_true",
                    help="graph path: also emit the edge vectors (fp32 [E,3]) and distances "
                         "(fp32 [E]) in the write stage: 44 bytes per edge instead of 28")
    ap.add_argument("--path", default="graph", choices=["graph", "halo", "filter", "batch", "sfc", "dist"],
                    help="graph: the headline full rebuild; halo: extract_halo_info of one rank "
                         "of an 8-way SFC partition of the same box (edges at r + 0.5); filter: "
                         "filter_edges_to_radius of the box's edges at r + 0.5 down to r; batch: "
                         "radius_graph_pbc_cuda on batches of small structures, batched against "
                         "the per-structure loop; sfc: the SFC partition of the box's atoms "
                         "(keys, stable order, labels); dist: DistGraphBuilder on one rank "
                         "(refresh and steady steps)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 1 GiB device-to-device copy (5 times): the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch

        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda:0").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": 1 << 30, "repeats": 5}))
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the "
              "graph build shards by space (each rank builds its own atoms' graph with a ghost shell), with no "
              "collective inside it.",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from dynamis_amd import _lib as L
    from dynamis_amd import configs

    if args.path == "halo":
        return bench_halo(args)
    if args.path == "filter":
        return bench_filter(args)
    if args.path == "batch":
        return bench_batch(args)
    if args.path == "sfc":
        return bench_sfc(args)
    if args.path == "dist":
        return bench_dist(args)

    box = {"C1": configs.fcc, "C2": configs.c2, "C3": configs.c3, "C4": configs.c4,
           "C4-500k": lambda: configs.c4(scale=1.3934), "C5": configs.c5}[args.config]()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = L.lib()
    pos = torch.from_numpy(box.pos).to(dev)
    tgt = None if box.targets is None else torch.from_numpy(box.targets).to(dev)
    n = pos.shape[0]

    from dynamis_amd.dynamis_state import dynamis_state_impl as impl

    # the cell is rounded to the position dtype and the radius to fp32, as the reference
    # binding does (radius_graph.cpp:7,24)
    d = impl._desc(pos, torch.from_numpy(np.asarray(box.cell, np.float64)),
                   torch.tensor([bool(x) for x in box.pbc]), impl._r32(box.radius), tgt)
    nt = n if tgt is None else tgt.shape[0]

    wsb = lib.dg_graph_workspace_size(d)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    counts = torch.empty(nt, dtype=torch.int32, device=dev)
    s = L.stream_of(dev)
    stream = torch.cuda.current_stream(dev)

    # size the preallocated edge buffers once (5 % headroom)
    L.check(lib.dg_graph_count(d, L.ptr(pos), L.ptr(tgt), L.ptr(ws), wsb, L.ptr(counts), s), "count")
    E0 = L._i64(0)
    fl = L._i64(0)
    L.check(lib.dg_graph_read_totals(d, L.ptr(ws), E0, fl, s), "totals")
    cap = int(E0.value * 1.05) + 1024
    src = torch.empty(cap, dtype=torch.int64, device=dev)
    dst = torch.empty(cap, dtype=torch.int64, device=dev)
    shift = torch.empty((cap, 3), dtype=torch.float32, device=dev)
    vec = dist = None
    if args.vectors:
        vec = torch.empty((cap, 3), dtype=torch.float32, device=dev)
        dist = torch.empty(cap, dtype=torch.float32, device=dev)
    bpe = WRITE_BYTES_PER_EDGE + (VECTOR_BYTES_PER_EDGE if args.vectors else 0)

    # position frames: a random walk of sigma per coordinate per frame (seeded), generated
    # on the device before any timing
    nframes = args.trajectory if args.trajectory >= 0 else (100 if args.config == "C5" else 0)
    frames = [pos]
    if nframes > 1:
        frames = list(itertools.islice(configs.walk(pos, args.sigma, seed=7), nframes))
    torch.cuda.synchronize()

    def step(ev=None, k=0):
        # one full rebuild = dg_graph_build: the count stage (SFC reorder, degrees, tile
        # offsets) then the write stage, back to back, no host sync
        p = frames[k % len(frames)]
        L.check(lib.dg_graph_count(d, L.ptr(p), L.ptr(tgt), L.ptr(ws), wsb, L.ptr(counts), s), "count")
        if ev is not None:
            ev[0].record(stream)
        L.check(lib.dg_graph_write(d, L.ptr(p), L.ptr(tgt), L.ptr(ws), wsb, cap, L.ptr(src), L.ptr(dst),
                                   L.ptr(shift), L.ptr(vec), L.ptr(dist), 0, s), "write")
        if ev is not None:
            ev[1].record(stream)

    for w in range(args.warmup):
        step(k=w)
    torch.cuda.synchronize()
    kev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for k in range(args.steps):
        step(kev[k], k)
    t1.record(stream)
    torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    write_ms = float(np.mean([a.elapsed_time(b) for a, b in kev]))
    E = L._i64(0)
    L.check(lib.dg_graph_read_totals(d, L.ptr(ws), E, fl, s), "totals")
    E = int(E.value)  # of the last frame built
    if len(frames) > 1:
        # edges per rebuild over the frames timed (they differ slightly along the walk)
        Es = []
        for k in range(args.steps):
            step(None, k)
            Ek = L._i64(0)
            L.check(lib.dg_graph_read_totals(d, L.ptr(ws), Ek, fl, s), "totals")
            Es.append(int(Ek.value))
        E = int(round(float(np.mean(Es))))
    ms = total_ms / args.steps

    # The same rebuild (dg_graph_build: both stages, no host synchronisation) captured once
    # in a HIP graph and replayed: what a molecular-dynamics loop that keeps its buffers
    # gets without the per-kernel launch cost.  (Positions frame 0; not the headline.)
    graph_ms = None
    if not args.vectors:
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(stream)

        def build_on_current():
            L.check(lib.dg_graph_build(d, L.ptr(pos), L.ptr(tgt), L.ptr(ws), wsb, cap, L.ptr(counts),
                                       L.ptr(src), L.ptr(dst), L.ptr(shift), None, None, 0, L.stream_of(dev)),
                    "build")

        with torch.cuda.stream(side):
            build_on_current()
        stream.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            build_on_current()
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        ga, gb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ga.record(stream)
        for _ in range(args.steps):
            graph.replay()
        gb.record(stream)
        torch.cuda.synchronize()
        graph_ms = ga.elapsed_time(gb) / args.steps
        del graph

    # The rebuild preceded by the reference API's own SFC reorder of the atoms
    # (sfc_kernels.cu:178-224: Morton keys, stable order) and the gather of the positions
    # into that order, all on the device with no host sync, as one step: what a caller that
    # applies the SFC permutation before every build pays.  (Positions frame 0.)
    sfc_leg = None
    if tgt is None and pos.dtype == torch.float32 and not args.vectors:
        swsb = lib.dg_sfc_workspace_size(n)
        sws = torch.empty(swsb, dtype=torch.uint8, device=dev)
        keys = torch.empty(n, dtype=torch.int64, device=dev)
        perm = torch.empty(n, dtype=torch.int64, device=dev)
        ppos = torch.empty_like(pos)

        def sfc_step():
            L.check(lib.dg_sfc_keys(L.ptr(pos), n, 0, L.ptr(keys), L.ptr(sws), swsb, s), "sfc_keys")
            L.check(lib.dg_sfc_order(L.ptr(keys), n, L.ptr(perm), L.ptr(sws), swsb, s), "sfc_order")
            torch.index_select(pos, 0, perm, out=ppos)
            L.check(lib.dg_graph_count(d, L.ptr(ppos), None, L.ptr(ws), wsb, L.ptr(counts), s), "count")
            L.check(lib.dg_graph_write(d, L.ptr(ppos), None, L.ptr(ws), wsb, cap, L.ptr(src), L.ptr(dst),
                                       L.ptr(shift), None, None, 0, s), "write")

        for _ in range(max(2, args.warmup)):
            sfc_step()
        torch.cuda.synchronize()
        sa, sb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        sa.record(stream)
        for _ in range(args.steps):
            sfc_step()
        sb.record(stream)
        torch.cuda.synchronize()
        sfc_ms = sa.elapsed_time(sb) / args.steps
        Ep = L._i64(0)
        L.check(lib.dg_graph_read_totals(d, L.ptr(ws), Ep, fl, s), "totals")
        Ep = int(Ep.value)
        # + keys (read positions 12, write 8), order (read keys 8, write the permutation 8),
        # gather (read the permutation 8 and positions 12, write positions 12): 68 B per atom
        sfc_bytes = (12 * n + 16 * n + 24 * n + WRITE_BYTES_PER_EDGE * Ep) + 68 * n
        sfc_leg = {"ms_per_rebuild": round(sfc_ms, 4), "value": round(Ep / (sfc_ms * 1e-3) / 1e9, 3),
                   "unit": "Gedges/s", "edges": Ep, "algorithmic_bytes": sfc_bytes,
                   "hbm_frac": round(sfc_bytes / (sfc_ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
                   "steps": "dg_sfc_keys (Morton) + dg_sfc_order + gather of the positions + "
                            "dg_graph_count + dg_graph_write on the permuted positions"}
        del sws, keys, perm, ppos

    # drop-in Python API (exact-size outputs, one host sync per build)

    cell_t = torch.from_numpy(np.asarray(box.cell))
    pbc_t = torch.tensor(list(box.pbc))
    def api_call():
        if args.vectors:
            impl.radius_graph_pbc_vectors(pos, cell_t, pbc_t, box.radius, tgt, torch.float32)
        else:
            impl.radius_graph_pbc_ex(pos, cell_t, pbc_t, box.radius, 0, False, tgt)

    for _ in range(2):
        api_call()
    torch.cuda.synchronize()
    ta = time.perf_counter()
    api_steps = max(3, args.steps // 4)
    for _ in range(api_steps):
        api_call()
    torch.cuda.synchronize()
    api_ms = (time.perf_counter() - ta) * 1e3 / api_steps

    pos_bytes = 24 if pos.dtype == torch.float64 else 12
    # Full-rebuild algorithmic bytes: read positions, keys write+read, reordered positions
    # write+read, the edge outputs (28 B per edge: int64 src, int64 dst, 3 x fp32 shift).
    rebuild_bytes = pos_bytes * n + 16 * n + 24 * n + bpe * E
    # Dominant kernel (the write stage), algorithmic bytes per launch: the edge outputs
    # only.  Everything else it moves (the count pass's slot entries, the cell list, the
    # tile tables) is an intermediate of this design and shows up in `traffic`.
    kbytes = bpe * E
    achieved = kbytes / (write_ms * 1e-3) / 1e9

    # HBM bytes per launch of the write stage measured by rocprofv3 (FETCH_SIZE +
    # WRITE_SIZE, scaled by a plain copy of known size); recorded in profiles/ by the
    # commands written there, for this config.
    traffic = None
    tfile = os.path.join(ROOT, "profiles", f"edge_write_{args.config}{'_vectors' if args.vectors else ''}"
                                           "_traffic.json")
    if os.path.exists(tfile):
        try:
            traffic = json.load(open(tfile)).get("bytes_per_launch")
        except (OSError, ValueError):
            traffic = None

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args, box, n, E)

    out = {
        "metric": METRIC,
        "value": round(E / (ms * 1e-3) / 1e9, 3),
        "unit": "Gedges/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 positions, fp64 predicate, int64 edges",
        "data": "synthetic (seeded numpy uniform box)" + (
            f"; {len(frames)} position frames, each displaced by Gaussian sigma={args.sigma} A per "
            "coordinate from the previous, cycled" if len(frames) > 1 else ""),
        "config": {"workload": f"{args.config}: {box.name} N={n} r_cut={box.radius} "
                               f"pbc={list(box.pbc)}", "atoms": n, "edges": E,
                   "parallelism": "single GPU"},
        "rebuilds_per_s": round(1e3 / ms, 2),
        "hbm_frac_rebuild": round(rebuild_bytes / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
        "hbm_frac_rebuild_target": 0.5,
        "rebuild_algorithmic_bytes": rebuild_bytes,
        "count_ms": round(ms - write_ms, 4),
        "write_ms": round(write_ms, 4),
        "api_ms_per_rebuild": round(api_ms, 3),
        "graph_replay_ms_per_rebuild": None if graph_ms is None else round(graph_ms, 4),
        "sfc_permuted_rebuild": sfc_leg,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_over_algorithmic": round(traffic / kbytes, 3) if traffic else None,
                     "kernel": "expand_kernel (+ search_kernel<1> fix-up): the write stage",
                     "algorithmic_bytes": kbytes, "bytes_per_unit": f"{bpe} per edge",
                     "launch_ms": round(write_ms, 4)},
        "cpu_baseline": cpu,
    }
    if pos.dtype == torch.float64:
        out["dtype"] = "fp64 positions, fp64 predicate, int64 edges"
    if args.vectors:
        out["config"]["outputs"] = "edge_index, cell shifts, fp32 edge vectors and distances"
    print(json.dumps(out), flush=True)


def _host_threads():
    """Threads the CPU baseline may use: the cores this process may run on, capped by
    OMP_NUM_THREADS when the job sets it (the GPU box's CPU share)."""
    cores = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    return (min(cores, int(omp)) if omp.isdigit() and int(omp) > 0 else cores), cores


def cpu_baseline(args, box, n, E_gpu):
    """The C oracle (the reference algorithm with the canonical predicate) on this host:
    the full build of the benchmarked box with all the threads the job may use, median of
    5; a one-thread full build, median of 5, of the same box when it has at most 200k atoms,
    else of C2 (100k atoms: the one-thread build of C3 would take about 18 s per run); and
    the Morton SFC keys of all atoms, with all threads and with one, median of 5."""
    import numpy as np

    import oracle
    from dynamis_amd import configs

    thr, cores = _host_threads()
    if args.cpu_threads:
        thr = args.cpu_threads

    def cell_of(b):
        return np.asarray(b.cell, np.float64).astype(b.pos.dtype).astype(np.float64)

    r32 = float(np.float32(box.radius))

    def timed(fn, reps):
        ts = []
        out = None
        for _ in range(reps):
            t = time.perf_counter()
            out = fn()
            ts.append(time.perf_counter() - t)
        return float(np.median(ts)), out

    full_s, o = timed(lambda: oracle.radius_graph(box.pos, cell_of(box), box.pbc, r32,
                                                  target_indices=box.targets, threads=thr), 5)
    E_cpu = len(o["src"])
    del o
    one_box, one_name = (box, args.config) if n <= 200_000 else (configs.c2(), "C2")
    one_s, oc = timed(lambda: oracle.radius_graph(one_box.pos, cell_of(one_box), one_box.pbc,
                                                  float(np.float32(one_box.radius)),
                                                  target_indices=one_box.targets, threads=1), 5)
    E_one = len(oc["src"])
    del oc
    p32 = box.pos.astype(np.float32)
    keys_s, _ = timed(lambda: oracle.morton_keys(p32, threads=thr), 5)
    keys1_s, _ = timed(lambda: oracle.morton_keys(p32, threads=1), 5)
    cpu = {"value": round(E_cpu / full_s / 1e9, 5), "unit": "Gedges/s", "cores": thr,
           "kind": "port",
           "sample": f"full build of {args.config} ({n} atoms, {E_cpu} edges) by the C oracle "
                     f"(reference algorithm, fp64 predicate), OpenMP {thr} threads "
                     f"({cores} cores in this process's affinity), median of 5: "
                     f"{full_s * 1e3:.0f} ms",
           "ms_per_rebuild": round(full_s * 1e3, 1),
           "host_cores_affinity": cores,
           "one_thread": {"value": round(E_one / one_s / 1e9, 5), "unit": "Gedges/s", "cores": 1,
                          "config": one_name,
                          "sample": f"full build of {one_name} ({len(one_box.pos)} atoms, {E_one} edges), "
                                    f"one thread, median of 5: {one_s * 1e3:.0f} ms",
                          "ms_per_rebuild": round(one_s * 1e3, 1)},
           "sfc_keys": {"ms": round(keys_s * 1e3, 2), "cores": thr, "ms_one_thread": round(keys1_s * 1e3, 2),
                        "sample": f"Morton keys of all {n} atoms, median of 5 each"}}
    if E_cpu != E_gpu:
        cpu["edge_count_mismatch"] = [E_cpu, E_gpu]
    return cpu


def bench_filter(args):
    """filter_edges_to_radius of the whole box's edges at r + 0.5 down to r: one step =
    dg_filter_compact (one pass) into preallocated outputs of the input's size (the Python
    call adds the allocations, one host sync and the move of the target row)."""
    import numpy as np
    import torch

    from dynamis_amd import _lib as L
    from dynamis_amd import configs
    from dynamis_amd.dynamis_state import dynamis_state_impl as impl

    skin = 0.5
    box = {"C2": configs.c2, "C3": configs.c3}[args.config]()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = L.lib()
    pos = torch.from_numpy(box.pos).to(dev)
    n = pos.shape[0]
    cell = torch.from_numpy(np.asarray(box.cell))
    ei, sh, _ = impl.radius_graph_pbc(pos, cell, torch.tensor(list(box.pbc)), box.radius + skin, 0, False)
    E = ei.shape[1]
    r = float(np.float32(box.radius))
    cbuf = (L.ctypes.c_double * 9)(*np.asarray(box.cell, np.float64).astype(np.float32).astype(np.float64).reshape(-1).tolist())
    wsb = lib.dg_filter_compact_workspace_size(E)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    nk = torch.empty(1, dtype=torch.int64, device=dev)
    base = ei.data_ptr()
    fargs = (L.ptr(pos), L.DG_F32, n, cbuf, r, L.ctypes.c_void_p(base), L.ctypes.c_void_p(base + 8 * E),
             L.ptr(sh), L.DG_F32, E)
    s = L.stream_of(dev)
    stream = torch.cuda.current_stream(dev)
    out_src = torch.empty(E, dtype=torch.int64, device=dev)
    out_dst = torch.empty(E, dtype=torch.int64, device=dev)
    out_s = torch.empty((E, 3), dtype=torch.float32, device=dev)

    def step(ev=None):
        if ev is not None:
            ev[0].record(stream)
        L.check(lib.dg_filter_compact(*fargs, L.ptr(out_src), L.ptr(out_dst), L.ptr(out_s), L.ptr(nk),
                                      L.ptr(ws), wsb, s), "filter")
        if ev is not None:
            ev[1].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    K = int(nk.item())
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(args.steps)]
    for k in range(args.steps):
        step(evs[k])
    torch.cuda.synchronize()
    ms = float(np.mean([a.elapsed_time(b) for a, b in evs]))
    # exact-size Python call (one host sync, allocation)
    torch.cuda.synchronize()
    ta = time.perf_counter()
    for _ in range(max(3, args.steps // 4)):
        impl.filter_edges_to_radius(ei, sh, pos, cell, r)
    torch.cuda.synchronize()
    api_ms = (time.perf_counter() - ta) * 1e3 / max(3, args.steps // 4)
    # algorithmic bytes: read the edge list (28 B per edge: src, dst, fp32 shift), write the
    # kept edges (28 B each), read the positions once
    nbytes = 28 * E + 28 * K + 12 * n
    ach = nbytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "filter_edges_to_radius edges/s (edges at r+0.5 filtered to r)",
        "value": round(E / (ms * 1e-3) / 1e9, 3), "unit": "Gedges/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32 positions, fp64 predicate",
        "data": "synthetic (seeded numpy uniform box)",
        "config": {"workload": f"filter, {args.config} N={n}, r={box.radius}+{skin} -> {box.radius}",
                   "edges_in": E, "edges_kept": K},
        "api_ms": round(api_ms, 3),
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "dg_filter_compact (single pass, all kernels)",
                     "algorithmic_bytes": nbytes}}), flush=True)


def bench_batch(args):
    """radius_graph_pbc_cuda on batches of small periodic structures (uniform at 0.08
    atoms/A^3, r = 6 A, fp32): the batched build (one launch sequence per batch) against the
    per-structure loop the reference runs.  One line per (structures, atoms per structure);
    one step = one wrapper call, the host clock around `--steps` calls."""
    import importlib
    import types

    import numpy as np
    import torch

    wrap = importlib.import_module("dynamis_amd.dynamis_state.radius_graph_pbc_cuda")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    rng = np.random.default_rng(1)
    cases = [(B, nat) for B in (8, 32, 128, 512) for nat in (30, 100, 250, 500)]
    cases += [(4, 1000), (16, 1000), (4, 2000), (16, 2000), (4, 5000), (16, 5000)]
    for B, nat in cases:
        natoms = rng.integers(nat // 2, nat + 1, B)
        cells, pos = [], []
        for n in natoms:
            L = (n / 0.08) ** (1 / 3)
            cells.append(np.eye(3) * L)
            pos.append(rng.uniform(0, L, (n, 3)))
        data = types.SimpleNamespace(
            pos=torch.from_numpy(np.concatenate(pos).astype(np.float32)).to(dev),
            cell=torch.from_numpy(np.array(cells)).float().to(dev),
            natoms=torch.from_numpy(natoms).to(dev), pbc=torch.tensor([[True] * 3] * B).to(dev))

        def timed(batched):
            # the wrapper with its choice forced either way
            old = wrap._batch_in_one_pass
            wrap._batch_in_one_pass = lambda natoms, *a: batched
            try:
                for _ in range(max(1, args.warmup)):
                    wrap.radius_graph_pbc_cuda(data, 6.0, 0)
                torch.cuda.synchronize()
                t = time.perf_counter()
                for _ in range(args.steps):
                    out = wrap.radius_graph_pbc_cuda(data, 6.0, 0)
                torch.cuda.synchronize()
                return (time.perf_counter() - t) * 1e3 / args.steps, out
            finally:
                wrap._batch_in_one_pass = old

        chosen = wrap._batch_in_one_pass([int(x) for x in natoms], np.array(cells), [True] * 3, 6.0)
        ms_batch, out = timed(True)
        ms_loop, _ = timed(False)
        print(json.dumps({"metric": "radius_graph_pbc_cuda ms per batch", "structures": B,
                          "atoms_per_structure_max": nat, "atoms": int(natoms.sum()),
                          "edges": int(out[0].shape[1]), "batched_ms": round(ms_batch, 4),
                          "loop_ms": round(ms_loop, 4), "speedup": round(ms_loop / ms_batch, 2),
                          "batched_chosen": chosen, "steps": args.steps}), flush=True)


def bench_halo(args):
    """extract_halo_info on rank 3 of an 8-way Morton partition of the config's box: the
    per-rank edges at r + 0.5 are built once; one step = dg_halo_count + dg_halo_write
    into preallocated outputs."""
    import numpy as np
    import torch

    from dynamis_amd import _lib as L
    from dynamis_amd import configs
    from dynamis_amd.dynamis_state import dynamis_state_impl as impl

    W, R, skin = 8, 3, 0.5
    box = {"C2": configs.c2, "C3": configs.c3}[args.config]()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = L.lib()
    pos = torch.from_numpy(box.pos).to(dev)
    n = pos.shape[0]
    pid = impl.sfc_partition_cuda(pos, None, W, 0)
    my = torch.nonzero(pid.eq(R)).squeeze(-1)
    ei, _, _, _ = impl.radius_graph_pbc_ex(pos, torch.from_numpy(np.asarray(box.cell)),
                                           torch.tensor(list(box.pbc)), box.radius + skin, 0, False, my)
    E = ei.shape[1]
    d = L.HaloDesc()
    d.n_atoms, d.n_edges, d.num_local, d.my_rank, d.world_size = n, E, my.numel(), R, W
    d.pid_dtype = L.DG_I64
    wsb = lib.dg_halo_workspace_size(n, W)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    so = torch.empty(W + 1, dtype=torch.int64, device=dev)
    ro = torch.empty(W + 1, dtype=torch.int64, device=dev)
    im = torch.empty(my.numel(), dtype=torch.bool, device=dev)
    s = L.stream_of(dev)
    stream = torch.cuda.current_stream(dev)
    src_p, dst_p = L.ctypes.c_void_p(ei.data_ptr()), L.ctypes.c_void_p(ei.data_ptr() + 8 * E)

    def count():
        L.check(lib.dg_halo_count(d, src_p, dst_p, L.ptr(pid), L.ptr(my), L.ptr(so), L.ptr(ro),
                                  L.ptr(im), L.ptr(ws), wsb, s), "halo count")

    count()
    ts, tr = L._i64(0), L._i64(0)
    L.check(lib.dg_halo_read_totals(L.ptr(ws), ts, tr, s), "halo totals")
    sl = torch.empty(ts.value, dtype=torch.int64, device=dev)
    rg = torch.empty(tr.value, dtype=torch.int64, device=dev)
    ra = torch.empty(tr.value, dtype=torch.int64, device=dev)

    def step():
        count()
        L.check(lib.dg_halo_write(d, L.ptr(pid), L.ptr(sl), L.ptr(rg), L.ptr(ra), L.ptr(ws), wsb, s),
                "halo write")

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(args.steps):
        step()
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    # algorithmic bytes: edges (src, dst) + pid[src] per edge; per atom the peer word
    # (clear, mark, 2 walks, interior), recv flag and global->local entry; the outputs
    cpu = None
    if not args.no_cpu:
        from oracle import halo as ohalo

        e_np, pid_np, my_np = ei.cpu().numpy(), pid.cpu().numpy(), my.cpu().numpy()
        tc = time.perf_counter()
        ohalo.extract_halo_info(e_np[0], e_np[1], pid_np, my_np, R, W, n)
        cs = time.perf_counter() - tc
        cpu = {"value": round(E / cs / 1e9, 5), "unit": "Gedges/s", "cores": 1, "kind": "port",
               "sample": f"one extract_halo_info of the same {E} edges by the numpy oracle "
                         f"(sorted unique, as the reference), {cs * 1e3:.0f} ms"}
    nbytes = 24 * E + n * (8 * 4 + 3 + 8) + 8 * (ts.value + 2 * tr.value) + 9 * my.numel()
    ach = nbytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "extract_halo_info edges/s (rank 3 of 8, edges at r+0.5)", "value": round(E / ms / 1e6, 3),
        "unit": "Gedges/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int64", "data": "synthetic (seeded numpy uniform box)",
        "config": {"workload": f"halo plan, {args.config} N={n}, W={W}, rank {R}, r={box.radius}+{skin}",
                   "edges": E, "num_local": int(my.numel()), "total_send": ts.value,
                   "total_recv": tr.value},
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "dg_halo_count + dg_halo_write (all kernels)", "algorithmic_bytes": nbytes},
        "cpu_baseline": cpu}), flush=True)


def bench_dist(args):
    """DistGraphBuilder (row f4) on one rank (no communication) over the config's box, with
    the positions moving by Gaussian sigma per coordinate per step (the drift watchdog never
    trips): the refresh step (mode A: degrees, SFC partition, build at r + skin, halo plan,
    filter to r) and the steady steps (mode B: the local build from the cached partition).
    One step = one DistGraphBuilder.build; host clock around synchronised steps."""
    import numpy as np
    import torch

    from dynamis_amd import configs
    from dynamis_amd.dynamis_state import dynamis_state_impl as impl
    from dynamis_amd.dynamis_state.dist_graph_builder import BuildMode, DistGraphBuilder

    box = {"C2": configs.c2, "C3": configs.c3}[args.config]()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    pos = torch.from_numpy(np.ascontiguousarray(box.pos, dtype=np.float32)).to(dev)
    cell = torch.from_numpy(np.asarray(box.cell, np.float32))
    env = impl.DistEnvironment()
    gen = torch.Generator(device=dev).manual_seed(11)
    noise = [torch.randn(pos.shape, device=dev, generator=gen) * args.sigma for _ in range(8)]
    b = DistGraphBuilder(cell, torch.tensor(list(box.pbc)), box.radius, 0.5, env,
                         refresh_interval=10 ** 9)
    refresh, steady = [], []
    for k in range(args.warmup + args.steps + 1):
        if k == 0 or k == args.warmup:
            b.reset()  # this step refreshes
        torch.cuda.synchronize()
        t = time.perf_counter()
        res = b.build(pos)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t) * 1e3
        if k >= args.warmup:
            (refresh if res.mode == BuildMode.REFRESH else steady).append(dt)
        pos.add_(noise[k % len(noise)])
    E = int(res.edges_outer.shape[1])
    ms = float(np.median(steady))
    print(json.dumps({
        "metric": "DistGraphBuilder step (one rank), ms", "value": round(ms, 4), "unit": "ms",
        "n_gpus": 1, "steps": len(steady), "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32 positions, fp64 predicate, int64 edges",
        "data": f"synthetic (seeded numpy uniform box), moved by sigma={args.sigma} A per coordinate per step",
        "config": {"workload": f"DistGraphBuilder W=1, {args.config} N={pos.shape[0]}, r={box.radius}, skin=0.5",
                   "edges": E},
        "refresh_ms": round(float(np.median(refresh)), 4), "steady_ms": round(ms, 4),
        "roofline": None, "cpu_baseline": None}), flush=True)


def bench_sfc(args):
    """The SFC partition path (rows a13, a14, f2) on the config's atoms: one step = Morton
    keys, their stable order and the W = 8 partition labels, through the C ABI into
    preallocated outputs; each stage is timed with HIP events as well.  The dominant kernel
    is the sort, whose algorithmic bytes are 16 per key (keys read, permutation written)."""
    import numpy as np
    import torch

    from dynamis_amd import _lib as L
    from dynamis_amd import configs

    W = 8
    box = {"C2": configs.c2, "C3": configs.c3}[args.config]()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = L.lib()
    pos = torch.from_numpy(np.ascontiguousarray(box.pos, dtype=np.float32)).to(dev)
    n = pos.shape[0]
    wsb = lib.dg_sfc_workspace_size(n)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    keys = torch.empty(n, dtype=torch.int64, device=dev)
    perm = torch.empty(n, dtype=torch.int64, device=dev)
    labels = torch.empty(n, dtype=torch.int64, device=dev)
    weights = torch.from_numpy(np.random.default_rng(3).integers(1, 100, n)).to(dev)
    s = L.stream_of(dev)
    stream = torch.cuda.current_stream(dev)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4 * args.steps + 2)]

    def step(k=None):
        if k is not None:
            ev[4 * k].record(stream)
        L.check(lib.dg_sfc_keys(L.ptr(pos), n, 0, L.ptr(keys), L.ptr(ws), wsb, s), "keys")
        if k is not None:
            ev[4 * k + 1].record(stream)
        L.check(lib.dg_sfc_order(L.ptr(keys), n, L.ptr(perm), L.ptr(ws), wsb, s), "order")
        if k is not None:
            ev[4 * k + 2].record(stream)
        L.check(lib.dg_sfc_labels(L.ptr(perm), n, W, None, L.ptr(labels), L.ptr(ws), wsb, s), "labels")
        if k is not None:
            ev[4 * k + 3].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0, t1 = ev[-2], ev[-1]
    t0.record(stream)
    for k in range(args.steps):
        step(k)
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    st = np.array([[ev[4 * k + j].elapsed_time(ev[4 * k + j + 1]) for j in range(3)] for k in range(args.steps)])
    keys_ms, order_ms, labels_ms = (float(np.mean(st[:, j])) for j in range(3))
    # weighted labels (exact int64 cut), timed apart
    for _ in range(2):
        L.check(lib.dg_sfc_labels(L.ptr(perm), n, W, L.ptr(weights), L.ptr(labels), L.ptr(ws), wsb, s), "w")
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(args.steps):
        L.check(lib.dg_sfc_labels(L.ptr(perm), n, W, L.ptr(weights), L.ptr(labels), L.ptr(ws), wsb, s), "w")
    b.record(stream)
    torch.cuda.synchronize()
    wlabels_ms = a.elapsed_time(b) / args.steps
    kbytes = 16 * n
    ach = kbytes / (order_ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        import oracle

        p_np = np.ascontiguousarray(box.pos, dtype=np.float32)
        tc = time.perf_counter()
        k_np = oracle.morton_keys(p_np, threads=0)
        perm_np = np.argsort(k_np, kind="stable")
        oracle.sfc_labels(perm_np, W)
        cs = time.perf_counter() - tc
        cpu = {"value": round(cs * 1e3, 2), "unit": "ms", "cores": _host_threads()[0], "kind": "port",
               "sample": f"one partition of the same {n} atoms: the C oracle's Morton keys (OpenMP), numpy's "
                         "stable argsort (one thread) and the oracle's labels"}
    print(json.dumps({
        "metric": f"SFC partition of {n} atoms (Morton keys, stable order, W={W} labels), ms per partition",
        "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32 positions, int64 keys", "data": "synthetic (seeded numpy uniform box)",
        "config": {"workload": f"SFC partition, {args.config} N={n}, W={W}"},
        "keys_ms": round(keys_ms, 4), "order_ms": round(order_ms, 4), "labels_ms": round(labels_ms, 4),
        "weighted_labels_ms": round(wlabels_ms, 4),
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "dg_sfc_order (all its kernels)", "algorithmic_bytes": kbytes,
                     "bytes_per_unit": "16 per key"},
        "cpu_baseline": cpu}), flush=True)


if __name__ == "__main__":
    main()
