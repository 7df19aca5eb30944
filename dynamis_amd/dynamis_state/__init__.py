"""MI355X drop-in for the graph surface of ``dynamis_state``.

    from dynamis_amd import dynamis_state
    edge_index, cell_offsets, nn = dynamis_state.radius_graph_pbc_cuda(data, 6.0, 0)

Mirrors dynamis_state/src/dynamis_state/__init__.py:17 (``radius_graph_pbc_cuda``) and the
``dynamis_state_impl`` graph entry points.
"""
from . import dynamis_state_impl
from .dynamis_state_impl import SFCCurveType
from .radius_graph_pbc_cuda import radius_graph_pbc_cuda
from . import dist_graph_builder
from .dist_graph_builder import BuildMode, DistBuildGraphResult, DistGraphBuilder

__all__ = ["dynamis_state_impl", "radius_graph_pbc_cuda", "SFCCurveType", "dist_graph_builder",
           "DistGraphBuilder", "DistBuildGraphResult", "BuildMode"]
