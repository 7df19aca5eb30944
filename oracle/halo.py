"""CPU oracle of the halo send/recv plan (TEST INFRASTRUCTURE ONLY: imported by tests/,
never by the product path).

Two independent restatements of the reference, in numpy:

  extract_halo_info  dist_graph_ops_kernels.cu:104-188 -- per-rank edges (dst in this
                     rank's atoms), boundary = src owned elsewhere, sorted unique of
                     peer * N + atom keys for recv and send, global->local lookup,
                     interior = no boundary edge into the atom.
  build_halo_maps    build_halo_maps.cpp:20-157 -- the serial map from the FULL graph:
                     a needed_by[N, W] matrix (each atom needed by its owner, and by the
                     owner of every dst it is the src of), send = my atoms needed by other
                     ranks, recv = atoms my rank needs but does not own, both ordered by
                     (peer, global id) as tests/test_dist_graph_builder.py:85-113 fixes.

Pinning: the two are different algorithms over different edge sets (per-rank vs full
graph); they agree exactly when the graph is symmetric, which the reference's own test
asserts (test_dist_graph_builder.py:199-271) and tests/test_oracle_halo.py repeats.  A
hand-worked 5-atom case and the send/recv mirror identity (rank p's send list to q is
rank q's recv list from p) pin the orderings.
"""
from __future__ import annotations

import numpy as np


def extract_halo_info(src, dst, pid, my_outer, my_rank, world_size, N):
    """dist_graph_ops_kernels.cu:104-188.  Returns (send_offsets, send_local_indices,
    recv_offsets, recv_ghost_indices, interior_mask, recv_atom_global)."""
    src = np.asarray(src, np.int64)
    dst = np.asarray(dst, np.int64)
    pid = np.asarray(pid, np.int64)
    my_outer = np.asarray(my_outer, np.int64)
    W, R = int(world_size), int(my_rank)
    num_local = my_outer.size
    peer = pid[src]                                   # :46-58
    keep = peer != R
    b_src, b_dst, b_peer = src[keep], dst[keep], peer[keep]
    g2l = np.full(N, -1, np.int64)                    # :140-142
    g2l[my_outer] = np.arange(num_local, dtype=np.int64)
    recv_u = np.unique(b_peer * N + b_src)            # :144-158 (sorted unique)
    recv_peer, recv_atom = recv_u // N, recv_u % N
    recv_off = np.zeros(W + 1, np.int64)
    recv_off[1:] = np.cumsum(np.bincount(recv_peer, minlength=W))
    recv_ghost = np.arange(num_local, num_local + recv_atom.size, dtype=np.int64)
    send_u = np.unique(b_peer * N + b_dst)            # :160-173
    send_peer, send_atom = send_u // N, send_u % N
    send_local = g2l[send_atom]
    send_off = np.zeros(W + 1, np.int64)
    send_off[1:] = np.cumsum(np.bincount(send_peer, minlength=W))
    has_remote = np.zeros(N, bool)                    # :175-182
    has_remote[b_dst] = True
    interior = ~has_remote[my_outer]
    return send_off, send_local, recv_off, recv_ghost, interior, recv_atom


def build_halo_maps(src, dst, pid, my_rank, world_size, N):
    """build_halo_maps.cpp:20-157 over the full graph.  Same 6-tuple (recv atoms last)
    plus my_indices (this rank's atoms, ascending)."""
    src = np.asarray(src, np.int64)
    dst = np.asarray(dst, np.int64)
    pid = np.asarray(pid, np.int64)
    W, R = int(world_size), int(my_rank)
    needed = np.zeros((N, W), bool)                   # :46-53
    needed[np.arange(N), pid] = True
    needed[src, pid[dst]] = True
    my_idx = np.nonzero(pid == R)[0]                  # :56-58
    num_local = my_idx.size
    mine = needed[my_idx].copy()
    mine[:, R] = False
    loc, peer = np.nonzero(mine)                      # row-major: (local, peer)
    order = np.lexsort((my_idx[loc], peer))           # by peer, then global id
    send_local = loc[order].astype(np.int64)
    send_off = np.zeros(W + 1, np.int64)
    send_off[1:] = np.cumsum(np.bincount(peer, minlength=W))
    need = needed[:, R].copy()                        # :99-101
    need[my_idx] = False
    recv = np.nonzero(need)[0]
    recv = recv[np.lexsort((recv, pid[recv]))]
    recv_off = np.zeros(W + 1, np.int64)
    recv_off[1:] = np.cumsum(np.bincount(pid[recv], minlength=W))
    recv_ghost = np.arange(num_local, num_local + recv.size, dtype=np.int64)
    mine_e = pid[dst] == R                            # :126-134
    ghost_src = pid[src[mine_e]] != R
    has_ghost = np.zeros(N, bool)
    has_ghost[dst[mine_e][ghost_src]] = True
    interior = ~has_ghost[my_idx]
    return send_off, send_local, recv_off, recv_ghost, interior, recv.astype(np.int64), my_idx
