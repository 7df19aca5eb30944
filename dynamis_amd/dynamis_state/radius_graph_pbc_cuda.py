"""Python drop-in ``radius_graph_pbc_cuda`` (dynamis_state/src/dynamis_state/
radius_graph_pbc_cuda.py:13-110): resolves PBC flags from ``data.pbc`` and builds one
graph per structure of the batch, offsetting atom indices."""
from __future__ import annotations

import torch

from . import dynamis_state_impl as _impl


def radius_graph_pbc_cuda(data, radius: float, max_num_neighbors_threshold: int,
                          enforce_max_neighbors_strictly: bool = False,
                          pbc: torch.Tensor | None = None):
    """Returns (edge_index [2,E] int64, cell_offsets [E,3] float32,
    num_neighbors_image [batch] int64).

    ``data`` carries pos [N,3], cell [batch,3,3], natoms [batch], pbc [batch,3] or [3].
    Mixed PBC across the batch raises RuntimeError (reference :37-48).
    """
    if pbc is None:
        data_pbc = torch.atleast_2d(data.pbc)
        all_true = torch.all(data_pbc, dim=0)
        all_false = torch.all(~data_pbc, dim=0)
        mixed = ~(all_true | all_false)
        if mixed.any():
            raise RuntimeError(
                "Different structures in the batch have different PBC "
                "configurations. This is not currently supported.")
        pbc_flags = all_true
    else:
        pbc_flags = pbc.to(torch.bool)

    batch_size = len(data.natoms)
    if batch_size == 1:
        return _impl.radius_graph_pbc(data.pos, data.cell[0], pbc_flags, float(radius),
                                      int(max_num_neighbors_threshold),
                                      enforce_max_neighbors_strictly)

    eis, cos, nns = [], [], []
    offset = 0
    for i in range(batch_size):
        n = int(data.natoms[i].item())
        ei, co, nn = _impl.radius_graph_pbc(data.pos[offset:offset + n], data.cell[i], pbc_flags,
                                            float(radius), int(max_num_neighbors_threshold),
                                            enforce_max_neighbors_strictly)
        if ei.size(1) > 0:
            ei = ei + offset
        eis.append(ei)
        cos.append(co)
        nns.append(nn)
        offset += n
    if eis:
        return torch.cat(eis, dim=1), torch.cat(cos, dim=0), torch.cat(nns, dim=0)
    dev = data.pos.device
    return (torch.empty(2, 0, dtype=torch.long, device=dev),
            torch.empty(0, 3, dtype=torch.float, device=dev),
            torch.zeros(batch_size, dtype=torch.long, device=dev))
