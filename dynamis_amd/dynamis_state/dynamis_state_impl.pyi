"""Type stubs of the graph entry points of ``dynamis_state_impl`` as this package exports them.

The signatures follow the reference module's stubs
(dynamis_state/src/dynamis_state/dynamis_state_impl.pyi:213-258 for the graph functions,
:23-29, :64-85 for the holder classes, partitioner.hpp:54 for SFCCurveType); the extra
entry points below (vectors, SFC keys / order / partition, the batched build) have no
counterpart there.
"""
from __future__ import annotations

import enum
import typing

import torch

__all__: list[str] = [
    "DistEnvironment",
    "MolecularInfo",
    "PartitionMessagePassingInfo",
    "SFCCurveType",
    "SFCPartitioner",
    "build_batch",
    "build_graph",
    "extract_halo_info",
    "filter_edges_to_radius",
    "radius_graph_pbc",
    "radius_graph_pbc_counts_ex",
    "radius_graph_pbc_ex",
    "radius_graph_pbc_vectors",
    "sfc_keys",
    "sfc_order",
    "sfc_partition_cuda",
]

class SFCCurveType(enum.IntEnum):
    Morton = 0
    Hilbert = 1

class DistEnvironment:
    global_rank: int
    gpus_per_node: int
    local_rank: int
    num_nodes: int
    world_size: int
    def __init__(self) -> None: ...

class MolecularInfo:
    num_atoms: int
    atom_positions: torch.Tensor | None
    atom_vertex_numbers: torch.Tensor | None
    edge_counts: torch.Tensor | None
    atom_types: torch.Tensor | None
    atom_velocities: torch.Tensor | None
    atom_forces: torch.Tensor | None
    def __init__(self) -> None: ...

class PartitionMessagePassingInfo:
    partition_id: torch.Tensor | None
    partition_indices: torch.Tensor | None
    atom_counts: torch.Tensor | None
    global_send_recv_matrix: torch.Tensor | None
    send_offsets: torch.Tensor | None
    send_local_indices: torch.Tensor | None
    recv_offsets: torch.Tensor | None
    recv_ghost_indices: torch.Tensor | None
    interior_mask: torch.Tensor | None
    edge_index: torch.Tensor | None
    edge_index_halo: torch.Tensor | None
    def __init__(self) -> None: ...

class SFCPartitioner:
    curve_type: SFCCurveType
    def __init__(self, curve_type: SFCCurveType | int = ...) -> None: ...
    def partition(self, state: MolecularInfo, env: DistEnvironment) -> PartitionMessagePassingInfo: ...

def radius_graph_pbc(
    pos: torch.Tensor,
    cell: torch.Tensor,
    pbc: torch.Tensor,
    radius: float,
    max_num_neighbors: int,
    enforce_max_strictly: bool,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(edge_index [2, E] int64, cell_offsets [E, 3] float32, num_neighbors_image [1] int64)."""

def radius_graph_pbc_ex(
    pos: torch.Tensor,
    cell: torch.Tensor,
    pbc: torch.Tensor,
    radius: float,
    max_num_neighbors: int,
    enforce_max_strictly: bool,
    target_indices: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(edge_index, cell_shifts, num_neighbors_image, neighbor_counts [N_target] int32)."""

def radius_graph_pbc_counts_ex(
    pos: torch.Tensor,
    cell: torch.Tensor,
    pbc: torch.Tensor,
    radius: float,
    target_indices: torch.Tensor | None = None,
) -> torch.Tensor:
    """neighbor_counts [N_target] int32, without a host synchronisation."""

def filter_edges_to_radius(
    edges: torch.Tensor,
    cell_shifts: torch.Tensor,
    pos: torch.Tensor,
    cell: torch.Tensor,
    radius: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Order-preserving filter of an edge list down to ``radius`` (edges', cell_shifts')."""

def extract_halo_info(
    edges: torch.Tensor,
    pid_outer: torch.Tensor,
    my_outer_atoms: torch.Tensor,
    my_rank: int,
    world_size: int,
    N: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(send_offsets, send_local_indices, recv_offsets, recv_ghost_indices, interior_mask,
    recv_atom_global)."""

# Extensions of this package (no counterpart in the reference's stubs).

def radius_graph_pbc_vectors(
    pos: torch.Tensor,
    cell: torch.Tensor,
    pbc: torch.Tensor,
    radius: float,
    target_indices: torch.Tensor | None = None,
    vector_dtype: torch.dtype | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(edge_index, cell_shifts, num_neighbors_image, neighbor_counts, edge_vec, edge_dist)."""

def build_graph(
    pos: torch.Tensor,
    cell: torch.Tensor,
    pbc: torch.Tensor,
    radius: float,
    target_indices: torch.Tensor | None = None,
    counts_only: bool = False,
    return_vectors: bool = False,
    vector_dtype: torch.dtype | None = None,
    out_ids: torch.Tensor | None = None,
) -> tuple[typing.Any, ...]: ...

def build_batch(
    pos: torch.Tensor,
    cells: torch.Tensor,
    natoms: typing.Sequence[int] | torch.Tensor,
    pbc: torch.Tensor,
    radius: float,
    max_num_neighbors: int = 0,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]: ...

def sfc_keys(pos: torch.Tensor, curve_type: SFCCurveType | int = ...) -> torch.Tensor: ...
def sfc_order(keys: torch.Tensor) -> torch.Tensor: ...
def sfc_partition_cuda(
    pos: torch.Tensor, weights: torch.Tensor | None, W: int, curve_type: SFCCurveType | int
) -> torch.Tensor: ...
