"""dynamis_amd -- MI355X-native (gfx950) build of Dynamis's neighbour-graph hot path:
the periodic radius graph with space-filling-curve reordering, behind the reference's
``dynamis_state`` Python surface (see ``dynamis_amd.dynamis_state``).

Kernels: dynamis_amd/csrc/*.hip -> libdynamis_graph.so (C ABI: include/dynamis_graph.h).
"""
__version__ = "0.1.0"
