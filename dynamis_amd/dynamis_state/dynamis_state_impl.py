"""MI355X implementation of the ``dynamis_state_impl`` graph entry points.

Same names, arguments, return tensors and error messages as the reference's pybind11
module (dynamis_state/src/dynamis_state_bindings.cpp:153-163, 241-254; validation in
dynamis_state/src/csrc/graph/radius_graph.cpp:7-127 and dist_graph_ops.cpp:5-35;
stubs dynamis_state/src/dynamis_state/dynamis_state_impl.pyi:213-258), running the
hand-written gfx950 kernels of libdynamis_graph.so.  There is no CPU path: every
function requires device tensors and the built library.

Differences from the reference, all deliberate:
  * the cutoff predicate is the fp64 canonical one (see include/dynamis_graph.h), not
    fp32 -- edge sets agree except for pairs within ~1e-5 A of the cutoff;
  * ``pos`` may also be float64 (the cell is then used in float64);
  * edges come grouped by target in space-filling-curve order (the reference groups
    them by target in cell order); compare edge sets after a canonical sort.
"""
from __future__ import annotations

import enum

import numpy as np
import torch

from .. import _lib as L


class SFCCurveType(enum.IntEnum):
    """dynamis_state/include/dynamis_state/partitioner.hpp:54 (bindings :96-98)."""

    Morton = 0
    Hilbert = 1


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _shape(t: torch.Tensor) -> str:
    return "[" + ", ".join(str(s) for s in t.shape) + "]"


def _validate(pos, cell, pbc, radius, max_num_neighbors=None, target_indices=None):
    """radius_graph.cpp:15-37 and :78-86 (messages kept)."""
    _check(isinstance(pos, torch.Tensor) and pos.is_cuda, "pos must be a CUDA tensor")
    _check(pos.dim() == 2 and pos.size(1) == 3,
           f"pos must have shape [N, 3], got {_shape(pos)}")
    _check(pos.dtype in (torch.float32, torch.float64),
           f"pos must be float32 or float64, got {pos.dtype}")
    cell = torch.as_tensor(cell)
    _check(cell.dim() == 2 and cell.size(0) == 3 and cell.size(1) == 3,
           f"cell must have shape [3, 3], got {_shape(cell)}")
    pbc = torch.as_tensor(pbc)
    _check(pbc.dim() == 1 and pbc.size(0) == 3, f"pbc must have shape [3], got {_shape(pbc)}")
    _check(float(radius) > 0.0, f"radius must be positive, got {float(radius)}")
    if max_num_neighbors is not None:
        _check(int(max_num_neighbors) >= 0,
               f"max_num_neighbors must be non-negative, got {int(max_num_neighbors)}")
    if target_indices is not None:
        ti = target_indices
        _check(isinstance(ti, torch.Tensor), f"target_indices must be a tensor, got {type(ti).__name__}")
        _check(ti.device == pos.device, "target_indices must be on the same device as pos")
        _check(ti.dim() == 1, f"target_indices must be 1-D, got shape {list(ti.shape)}")
        _check(ti.dtype == torch.int64, f"target_indices must be int64, got {ti.dtype}")
        target_indices = ti.contiguous()
    return pos.contiguous(), cell, pbc, target_indices


def _desc(pos, cell, pbc, radius, target_indices):
    d = L.GraphDesc()
    d.n_atoms = pos.size(0)
    d.has_targets = 0 if target_indices is None else 1
    d.n_targets = 0 if target_indices is None else target_indices.size(0)
    d.pos_dtype = L.DG_F64 if pos.dtype == torch.float64 else L.DG_F32
    # The reference casts the cell to float32 (radius_graph.cpp:24); with float64
    # positions the cell is kept in float64.
    c = cell.detach().to(device="cpu", dtype=pos.dtype).to(torch.float64).reshape(-1).tolist()
    for k in range(9):
        d.cell[k] = c[k]
    pb = pbc.detach().to("cpu").to(torch.bool).tolist()
    for k in range(3):
        d.pbc[k] = 1 if pb[k] else 0
    d.radius = float(radius)
    return d


def _empty(device, n_target):
    return (torch.empty((2, 0), dtype=torch.long, device=device),
            torch.empty((0, 3), dtype=torch.float32, device=device),
            torch.zeros(1, dtype=torch.long, device=device),
            torch.zeros(n_target, dtype=torch.int32, device=device))


def build_graph(pos, cell, pbc, radius, target_indices=None, counts_only=False,
                return_vectors=False, vector_dtype=None, out_ids=None):
    """Core build shared by every entry point (validated inputs).

    out_ids (int64 [N] on the device, or None): the ids written into edge_index for the
    atoms (atom i is written as out_ids[i]); DistGraphBuilder's steady step passes the
    global ids of its local atoms, which saves remapping the edges afterwards.

    Returns (edge_index [2,E] int64, cell_shifts [E,3] float32, num_neighbors_image [1]
    int64, neighbor_counts [N_target] int32[, edge_vec [E,3], edge_dist [E]]).
    """
    lib = L.lib()
    dev = pos.device
    n = pos.size(0)
    nt = n if target_indices is None else target_indices.size(0)
    vdt = vector_dtype or pos.dtype
    if n == 0 or nt == 0:
        out = _empty(dev, nt)
        if return_vectors:
            out = out + (torch.empty((0, 3), dtype=vdt, device=dev), torch.empty(0, dtype=vdt, device=dev))
        return out
    d = _desc(pos, cell, pbc, radius, target_indices)
    wsb = lib.dg_graph_workspace_size(d)
    if wsb == 0:
        raise RuntimeError(lib.dg_last_error().decode())
    with torch.cuda.device(dev):
        s = L.stream_of(dev)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        counts = torch.empty(nt, dtype=torch.int32, device=dev)
        count = lib.dg_graph_counts if counts_only else lib.dg_graph_count
        L.check(count(d, L.ptr(pos), L.ptr(target_indices), L.ptr(ws), wsb, L.ptr(counts), s),
                "radius_graph_pbc")
        if counts_only:
            return None, None, None, counts
        E = L._i64(0)
        fl = L._i64(0)
        L.check(lib.dg_graph_read_totals(d, L.ptr(ws), E, fl, s), "radius_graph_pbc")
        E = int(E.value)
        edge_index = torch.empty((2, E), dtype=torch.long, device=dev)
        shifts = torch.empty((E, 3), dtype=torch.float32, device=dev)
        vec = dist = None
        if return_vectors:
            vec = torch.empty((E, 3), dtype=vdt, device=dev)
            dist = torch.empty(E, dtype=vdt, device=dev)
        if E > 0:
            src_ptr = edge_index.data_ptr()
            L.check(lib.dg_graph_write_ids(
                d, L.ptr(pos), L.ptr(target_indices), L.ptr(ws), wsb, E, L.ptr(out_ids),
                L.ctypes.c_void_p(src_ptr), L.ctypes.c_void_p(src_ptr + 8 * E), L.ptr(shifts),
                L.ptr(vec), L.ptr(dist), L.DG_F64 if vdt == torch.float64 else L.DG_F32, s),
                "radius_graph_pbc")
        nn = torch.full((1,), E, dtype=torch.long, device=dev)
        out = (edge_index, shifts, nn, counts)
        if return_vectors:
            out = out + (vec, dist)
        return out


def build_batch(pos, cells, natoms, pbc, radius, max_num_neighbors=0):
    """Graphs of a batch of structures in one launch sequence (dg_batch_*): the batched
    form of radius_graph_pbc_cuda's per-structure loop (radius_graph_pbc_cuda.py:64-110).

    pos [N, 3] (the structures one after another), cells [B, 3, 3], natoms [B], pbc [3]
    shared by the batch.  Returns (edge_index [2, E] with batch atom indices, cell_offsets
    [E, 3] float32, num_neighbors_image [B] int64).  Edges are grouped by target,
    structures in batch order, targets in index order.
    """
    pos, _, pbc, _ = _validate(pos, torch.eye(3), pbc, radius, max_num_neighbors)
    lib = L.lib()
    dev = pos.device
    natoms = torch.as_tensor(natoms)
    _check(natoms.dim() == 1, f"natoms must have shape [B], got {_shape(natoms)}")
    _check(not natoms.is_floating_point() and not natoms.is_complex() and natoms.dtype != torch.bool,
           f"natoms must be integers, got {natoms.dtype}")
    B = int(natoms.numel())
    _check(B >= 1, "the batch is empty")
    cells = torch.as_tensor(cells)
    _check(cells.dim() == 3 and cells.size(0) == B and cells.size(1) == 3 and cells.size(2) == 3,
           f"cell must have shape [{B}, 3, 3], got {_shape(cells)}")
    d = L.BatchDesc()
    d.n_images = B
    d.n_atoms = pos.size(0)
    d.pos_dtype = L.DG_F64 if pos.dtype == torch.float64 else L.DG_F32
    for k in range(3):
        d.pbc[k] = 1 if bool(pbc[k]) else 0
    d.radius = _r32(radius)
    # the cell rounded to the position dtype, as the single-structure binding does
    # (radius_graph.cpp:24)
    c = cells.to(device=dev, dtype=pos.dtype).to(torch.float64).contiguous()
    na = torch.as_tensor(natoms).to(device=dev, dtype=torch.int64).contiguous()
    wsb = lib.dg_batch_workspace_size(d)
    if wsb == 0:
        raise RuntimeError(lib.dg_last_error().decode())
    with torch.cuda.device(dev):
        s = L.stream_of(dev)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        L.check(lib.dg_batch_count(d, L.ptr(pos), L.ptr(na), L.ptr(c), None, L.ptr(ws), wsb, s),
                "radius_graph_pbc_cuda")
        E, fl = L._i64(0), L._i64(0)
        L.check(lib.dg_batch_read_totals(d, L.ptr(ws), E, fl, s), "radius_graph_pbc_cuda")
        E = int(E.value)
        edge_index = torch.empty((2, E), dtype=torch.long, device=dev)
        shifts = torch.empty((E, 3), dtype=torch.float32, device=dev)
        nn = torch.empty(B, dtype=torch.long, device=dev)
        base = edge_index.data_ptr()
        L.check(lib.dg_batch_write(d, L.ptr(pos), L.ptr(ws), wsb, E, L.ctypes.c_void_p(base),
                                   L.ctypes.c_void_p(base + 8 * E), L.ptr(shifts), L.ptr(nn), s),
                "radius_graph_pbc_cuda")
    return edge_index, shifts, nn


def _r32(radius) -> float:
    # the reference binds radius as C++ float (radius_graph.cpp:7)
    return float(np.float32(radius))


def radius_graph_pbc(pos, cell, pbc, radius, max_num_neighbors, enforce_max_strictly):
    """(edge_index [2,E] int64, cell_offsets [E,3] float32, num_neighbors_image [1] int64).

    radius_graph.cpp:7-49.  max_num_neighbors / enforce_max_strictly are validated and
    ignored, exactly as the reference (radius_graph_kernels.cu:771-775).
    """
    pos, cell, pbc, _ = _validate(pos, cell, pbc, radius, max_num_neighbors)
    ei, co, nn, _c = build_graph(pos, cell, pbc, _r32(radius))
    return ei, co, nn


def radius_graph_pbc_ex(pos, cell, pbc, radius, max_num_neighbors, enforce_max_strictly,
                        target_indices=None):
    """(edge_index, cell_shifts, num_neighbors_image, neighbor_counts[N_target] int32).

    radius_graph.cpp:51-92: only ``target_indices`` atoms are targets; sources are all
    atoms; ids are global; neighbor_counts is in target_indices order.
    """
    pos, cell, pbc, ti = _validate(pos, cell, pbc, radius, max_num_neighbors, target_indices)
    return build_graph(pos, cell, pbc, _r32(radius), ti)


def radius_graph_pbc_counts_ex(pos, cell, pbc, radius, target_indices=None):
    """neighbor_counts[N_target] int32 only, no host sync (radius_graph.cpp:94-127)."""
    pos, cell, pbc, ti = _validate(pos, cell, pbc, radius, None, target_indices)
    return build_graph(pos, cell, pbc, _r32(radius), ti, counts_only=True)[3]


def radius_graph_pbc_vectors(pos, cell, pbc, radius, target_indices=None, vector_dtype=None):
    """Extension: also returns the canonical edge vectors v = pos[src] + S.cell - pos[dst]
    and distances |v| (fp64 exact, or fp32 correctly rounded from fp64).

    Returns (edge_index, cell_shifts, num_neighbors_image, neighbor_counts, edge_vec,
    edge_dist).  radius is rounded to fp32, as every other entry point does, so the edge
    set is the one radius_graph_pbc_ex returns at the same radius.
    """
    pos, cell, pbc, ti = _validate(pos, cell, pbc, radius, None, target_indices)
    return build_graph(pos, cell, pbc, _r32(radius), ti, return_vectors=True,
                       vector_dtype=vector_dtype)


def filter_edges_to_radius(edges, cell_shifts, pos, cell, radius):
    """Order-preserving filter to ``radius`` (dist_graph_ops.cpp:5-35, kernels :16-102).

    Keeps edge e iff |pos[src] + cell_shifts[e] @ cell - pos[dst]|^2 <= radius^2 with the
    canonical fp64 evaluation, so filter(build(r + skin), r) == build(r) as edge sets.
    Returns (edges', cell_shifts'), cell_shifts' keeps its dtype.
    """
    _check(isinstance(edges, torch.Tensor) and edges.is_cuda, "edges must be a CUDA tensor")
    _check(edges.dim() == 2 and edges.size(0) == 2,
           f"edges must have shape [2, E], got {list(edges.shape)}")
    _check(edges.dtype == torch.int64, f"edges must be int64, got {edges.dtype}")
    E = edges.size(1)
    _check(cell_shifts.dim() == 2 and cell_shifts.size(1) == 3,
           f"cell_shifts must have shape [E, 3], got {list(cell_shifts.shape)}")
    _check(cell_shifts.size(0) == E,
           f"cell_shifts rows ({cell_shifts.size(0)}) must equal number of edges E ({E})")
    _check(isinstance(pos, torch.Tensor) and pos.is_cuda, "pos must be a CUDA tensor")
    _check(pos.dim() == 2 and pos.size(1) == 3, f"pos must have shape [N, 3], got {list(pos.shape)}")
    _check(pos.dtype in (torch.float32, torch.float64),
           f"pos must be float32 or float64, got {pos.dtype}")
    cell = torch.as_tensor(cell)
    _check(cell.dim() == 2 and cell.size(0) == 3 and cell.size(1) == 3,
           f"cell must have shape [3, 3], got {list(cell.shape)}")
    _check(float(radius) > 0.0, f"radius must be positive, got {float(radius)}")
    if E == 0:
        return edges, cell_shifts
    lib = L.lib()
    dev = pos.device
    edges = edges.contiguous()
    pos = pos.contiguous()
    sh = cell_shifts.contiguous()
    # The kernels read float32, float64, int32 and int64 shifts.  Other dtypes go through
    # one whose values hold theirs exactly (float16 / bfloat16 -> float32, other integer
    # types -> int64) and come back unchanged, so the returned shifts are bit-equal to the
    # input rows, as the reference's compaction of the original tensor gives
    # (dist_graph_ops_kernels.cu:95-100).
    native = {torch.float32: L.DG_F32, torch.float64: L.DG_F64, torch.int64: L.DG_I64,
              torch.int32: L.DG_I32}
    if sh.dtype in native:
        sdt = native[sh.dtype]
    elif sh.is_floating_point():
        sh = sh.to(torch.float32)
        sdt = L.DG_F32
    else:
        sh = sh.to(torch.int64)
        sdt = L.DG_I64
    c = cell.detach().to(device="cpu", dtype=pos.dtype).to(torch.float64).contiguous()
    cbuf = (L.ctypes.c_double * 9)(*c.reshape(-1).tolist())
    pdt = L.DG_F64 if pos.dtype == torch.float64 else L.DG_F32
    base = edges.data_ptr()
    with torch.cuda.device(dev):
        s = L.stream_of(dev)
        wsb = lib.dg_filter_compact_workspace_size(E)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        nk = torch.empty(1, dtype=torch.int64, device=dev)
        # One pass: the kept edges land in order in the first k rows of E-row outputs.  The
        # sources go straight to row 0 of the result, the targets to a scratch row, moved
        # behind them once k is known, so edge_index is [2, k] contiguous.
        buf = torch.empty(2 * E, dtype=torch.int64, device=dev)
        dst_tmp = torch.empty(E, dtype=torch.int64, device=dev)
        out_s = torch.empty((E, 3), dtype=sh.dtype, device=dev)
        L.check(lib.dg_filter_compact(L.ptr(pos), pdt, pos.size(0), cbuf, float(radius),
                                      L.ctypes.c_void_p(base), L.ctypes.c_void_p(base + 8 * E), L.ptr(sh),
                                      sdt, E, L.ptr(buf), L.ptr(dst_tmp), L.ptr(out_s), L.ptr(nk),
                                      L.ptr(ws), wsb, s), "filter_edges_to_radius")
        k = int(nk.item())
        _check(k != -1, f"filter_edges_to_radius: edges hold atom indices outside [0, {pos.size(0)})")
        _check(k >= 0, "filter_edges_to_radius: internal error (a block's wait for its predecessors gave up)")
        buf[k:2 * k].copy_(dst_tmp[:k])
        out_e = buf[:2 * k].view(2, k)
        out_s = out_s[:k]
        if out_s.dtype != cell_shifts.dtype:
            out_s = out_s.to(cell_shifts.dtype)
        return out_e, out_s


def extract_halo_info(edges, pid_outer, my_outer_atoms, my_rank, world_size, N):
    """Halo send/recv CSR and interior mask of one rank from its edges (every dst in
    ``my_outer_atoms``), dist_graph_ops.cpp:38-60 / dist_graph_ops_kernels.cu:104-188.

    Returns (send_offsets [W+1] int64, send_local_indices int64 (positions into
    my_outer_atoms), recv_offsets [W+1] int64, recv_ghost_indices int64
    (arange(num_local, num_local + total_recv)), interior_mask [num_local] bool,
    recv_atom_global int64), both lists grouped by peer rank and sorted by global atom id
    inside a peer.  One host sync (the list sizes).
    """
    _check(isinstance(edges, torch.Tensor) and edges.is_cuda, "edges must be a CUDA tensor")
    _check(edges.dim() == 2 and edges.size(0) == 2,
           f"edges must have shape [2, E], got {list(edges.shape)}")
    _check(edges.dtype == torch.int64, "edges must be int64")
    N = int(N)
    _check(isinstance(pid_outer, torch.Tensor) and pid_outer.is_cuda and pid_outer.dim() == 1,
           "pid_outer must be a 1-D CUDA tensor")
    _check(pid_outer.size(0) == N, f"pid_outer must have length N ({N}), got {pid_outer.size(0)}")
    _check(isinstance(my_outer_atoms, torch.Tensor) and my_outer_atoms.is_cuda
           and my_outer_atoms.dim() == 1 and my_outer_atoms.dtype == torch.int64,
           "my_outer_atoms must be 1-D int64 CUDA")
    W, R = int(world_size), int(my_rank)
    _check(W >= 1, f"world_size must be >= 1, got {W}")
    _check(0 <= R < W, "my_rank must be in [0, world_size)")
    lib = L.lib()
    dev = edges.device
    edges = edges.contiguous()
    if pid_outer.dtype not in (torch.int32, torch.int64):
        pid_outer = pid_outer.to(torch.int64)
    pid = pid_outer.contiguous()
    outer = my_outer_atoms.contiguous()
    E = edges.size(1)
    d = L.HaloDesc()
    d.n_atoms, d.n_edges, d.num_local, d.my_rank, d.world_size = N, E, outer.size(0), R, W
    d.pid_dtype = L.DG_I32 if pid.dtype == torch.int32 else L.DG_I64
    wsb = lib.dg_halo_workspace_size(N, W)
    _check(wsb > 0, f"extract_halo_info: world_size must be <= 4096, got {W}")
    with torch.cuda.device(dev):
        s = L.stream_of(dev)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        send_off = torch.empty(W + 1, dtype=torch.int64, device=dev)
        recv_off = torch.empty(W + 1, dtype=torch.int64, device=dev)
        interior = torch.empty(outer.size(0), dtype=torch.bool, device=dev)
        base = edges.data_ptr()
        L.check(lib.dg_halo_count(d, L.ctypes.c_void_p(base), L.ctypes.c_void_p(base + 8 * E),
                                  L.ptr(pid), L.ptr(outer), L.ptr(send_off), L.ptr(recv_off),
                                  L.ptr(interior), L.ptr(ws), wsb, s), "extract_halo_info")
        ts, tr = L._i64(0), L._i64(0)
        L.check(lib.dg_halo_read_totals(L.ptr(ws), ts, tr, s), "extract_halo_info")
        send_local = torch.empty(ts.value, dtype=torch.int64, device=dev)
        recv_ghost = torch.empty(tr.value, dtype=torch.int64, device=dev)
        recv_atom = torch.empty(tr.value, dtype=torch.int64, device=dev)
        L.check(lib.dg_halo_write(d, L.ptr(pid), L.ptr(send_local), L.ptr(recv_ghost),
                                  L.ptr(recv_atom), L.ptr(ws), wsb, s), "extract_halo_info")
    return send_off, send_local, recv_off, recv_ghost, interior, recv_atom


def sfc_keys(pos, curve_type=SFCCurveType.Morton):
    """SFC keys of every atom, int64 [N] (sfc_kernels.cu:19-109, bounds :196-198)."""
    _check(isinstance(pos, torch.Tensor) and pos.is_cuda, "pos must be a CUDA tensor")
    _check(pos.dim() == 2 and pos.size(1) == 3, f"pos must have shape [N, 3], got {_shape(pos)}")
    _check(pos.dtype == torch.float32, f"pos must be float32, got {pos.dtype}")
    ct = int(curve_type)
    _check(ct in (0, 1), f"curve_type must be 0 (Morton) or 1 (Hilbert), got {ct}")
    lib = L.lib()
    pos = pos.contiguous()
    n = pos.size(0)
    keys = torch.empty(n, dtype=torch.int64, device=pos.device)
    if n == 0:
        return keys
    wsb = lib.dg_sfc_workspace_size(n)
    with torch.cuda.device(pos.device):
        ws = torch.empty(wsb, dtype=torch.uint8, device=pos.device)
        L.check(lib.dg_sfc_keys(L.ptr(pos), n, ct, L.ptr(keys), L.ptr(ws), wsb,
                                L.stream_of(pos.device)), "sfc_keys")
    return keys


def sfc_order(keys):
    """Stable ascending permutation of int64 keys (replaces at::sort, sfc_kernels.cu:224)."""
    _check(keys.is_cuda and keys.dtype == torch.int64 and keys.dim() == 1,
           "keys must be a 1-D int64 CUDA tensor")
    lib = L.lib()
    keys = keys.contiguous()
    n = keys.size(0)
    perm = torch.empty(n, dtype=torch.int64, device=keys.device)
    if n == 0:
        return perm
    wsb = lib.dg_sfc_workspace_size(n)
    with torch.cuda.device(keys.device):
        ws = torch.empty(wsb, dtype=torch.uint8, device=keys.device)
        L.check(lib.dg_sfc_order(L.ptr(keys), n, L.ptr(perm), L.ptr(ws), wsb,
                                 L.stream_of(keys.device)), "sfc_order")
    return perm


def sfc_partition_cuda(pos, weights, W, curve_type):
    """Partition labels int64 [N] (sfc.cpp:9-32 / sfc_kernels.cu:178-251).

    ``weights`` is None (unweighted) or [N] integer-valued; W >= 1; curve_type 0 / 1.
    """
    _check(isinstance(pos, torch.Tensor) and pos.is_cuda, "pos must be a CUDA tensor")
    _check(pos.dim() == 2 and pos.size(1) == 3,
           f"pos must have shape [N, 3], got [{pos.size(0)}, {pos.size(1) if pos.dim() > 1 else 0}]")
    _check(pos.dtype == torch.float32, f"pos must be float32, got {pos.dtype}")
    _check(int(W) >= 1, f"W must be >= 1, got {int(W)}")
    ct = int(curve_type)
    _check(ct in (0, 1), f"curve_type must be 0 (Morton) or 1 (Hilbert), got {ct}")
    n = pos.size(0)
    dev = pos.device
    if weights is not None:
        _check(weights.is_cuda, "weights must be a CUDA tensor")
        _check(weights.dim() == 1 and weights.size(0) == n,
               f"weights must have shape [N], got [{weights.size(0)}]")
        weights = weights.to(torch.int64).contiguous()
    if int(W) == 1:
        return torch.zeros(n, dtype=torch.int64, device=dev)
    keys = sfc_keys(pos, ct)
    perm = sfc_order(keys)
    labels = torch.empty(n, dtype=torch.int64, device=dev)
    if n == 0:
        return labels
    lib = L.lib()
    wsb = lib.dg_sfc_workspace_size(n)
    with torch.cuda.device(dev):
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        L.check(lib.dg_sfc_labels(L.ptr(perm), n, int(W), L.ptr(weights), L.ptr(labels), L.ptr(ws),
                                  wsb, L.stream_of(dev)), "sfc_partition_cuda")
    return labels


# ---------------------------------------------------------------------------------------
# Plain holders of the reference's bound structs that DistGraphBuilder exchanges
# (dynamis_state_impl.pyi:23-29, 64-85), and the SFC partitioner's partition() for device
# tensors (partition/sfc_partitioner.cpp:97-195).
# ---------------------------------------------------------------------------------------


class DistEnvironment:
    """dynamis_state_impl.pyi:23-29."""

    def __init__(self) -> None:
        self.global_rank = 0
        self.world_size = 1
        self.local_rank = 0
        self.gpus_per_node = 1
        self.num_nodes = 1


class MolecularInfo:
    """dynamis_state_impl.pyi:64-72 (the fields the partitioner reads)."""

    def __init__(self) -> None:
        self.num_atoms = 0
        self.atom_positions = None
        self.atom_vertex_numbers = None
        self.edge_counts = None
        self.atom_types = None
        self.atom_velocities = None
        self.atom_forces = None


class PartitionMessagePassingInfo:
    """dynamis_state_impl.pyi:74-85."""

    def __init__(self) -> None:
        self.partition_id = None
        self.partition_indices = None
        self.atom_counts = None
        self.global_send_recv_matrix = None
        self.send_offsets = None
        self.send_local_indices = None
        self.recv_offsets = None
        self.recv_ghost_indices = None
        self.interior_mask = None
        self.edge_index = None
        self.edge_index_halo = None


class SFCPartitioner:
    """SFC partitioner (partition/sfc_partitioner.cpp:97-195), device path only."""

    def __init__(self, curve_type=SFCCurveType.Morton) -> None:
        self.curve_type = SFCCurveType(int(curve_type))

    def partition(self, state: MolecularInfo, env: DistEnvironment) -> PartitionMessagePassingInfo:
        """Unweighted, or weighted by ``state.edge_counts`` when set (:184-195, :97-179)."""
        pos = state.atom_positions
        W, R = int(env.world_size), int(env.global_rank)
        labels = sfc_partition_cuda(pos.to(torch.float32), state.edge_counts, W, self.curve_type)
        info = PartitionMessagePassingInfo()
        info.partition_id = labels
        mine = torch.nonzero(labels.eq(R), as_tuple=False).squeeze(-1)
        info.atom_counts = torch.bincount(labels, minlength=W)
        vn = state.atom_vertex_numbers
        if vn is None:
            vn = torch.arange(int(state.num_atoms), dtype=torch.int64, device=pos.device)
        info.partition_indices = vn.index_select(0, mine)
        info.global_send_recv_matrix = torch.zeros(W, W, dtype=torch.int64, device=pos.device)
        info.global_send_recv_matrix[R, R] = mine.numel()
        return info
