"""Python drop-in ``radius_graph_pbc_cuda`` (dynamis_state/src/dynamis_state/
radius_graph_pbc_cuda.py:13-110): resolves PBC flags from ``data.pbc`` and builds the graph
of every structure of the batch, with batch atom indices -- a batch of small structures in
one launch sequence (``dynamis_state_impl.build_batch``), others one structure at a time."""
from __future__ import annotations

import torch

from . import dynamis_state_impl as _impl


# A batch goes through the one-pass batched build (all-pairs within each structure, over
# the periodic images its cell needs) when that is expected to be faster than building the
# structures one by one with the cell-list build, as the reference loop does.  Measured on
# one MI355X (uniform structures at 0.08 atoms/A^3, r = 6 A): the loop costs about 0.19 ms
# per structure; the batched build about 0.22 ms plus 16 ps per atom pair within the
# structures (one wave per atom sweeps its structure's atoms and images), e.g. 128
# structures of up to 250 atoms in 0.35 ms against 23.4 ms, 512 of up to 500 in 1.5 ms
# against 92 ms.  A single structure, and structures above BATCH_MAX_ATOMS, always go
# through the cell-list build.
#
# The batched kernel visits, for every atom pair, the periodic shifts S with
# |frac_t - frac_s - S_d| <= r / d_face on each periodic axis: about prod_d (2 r / d_face + 1)
# of them.  The per-pair cost above was measured at about 6 such images per pair (250-atom
# cubes at r = 6 A: r / d_face = 0.41 per axis), so a structure's pairs are weighted by its
# image count over 6.  A structure needing more than BATCH_MAX_IMAGES images per pair (a
# cell that is small against the cutoff) sends the batch through the loop, whose cell-list
# build handles such cells without visiting every image of every pair.
BATCH_MAX_ATOMS = 8192
BATCH_MAX_IMAGES = 343.0
_LOOP_MS_PER_STRUCTURE = 0.19
_BATCH_MS = 0.22
_BATCH_MS_PER_PAIR = 1.6e-8
_BATCH_IMAGES_MEASURED = 6.0


def _images_per_pair(cell, pbc, radius) -> float:
    """prod over periodic axes of (2 r / d_face + 1) for one cell (rows = lattice vectors)."""
    import numpy as np

    c = np.asarray(cell, dtype=np.float64).reshape(3, 3)
    vol = abs(float(np.dot(c[0], np.cross(c[1], c[2]))))
    img = 1.0
    for d in range(3):
        if not pbc[d]:
            continue
        area = float(np.linalg.norm(np.cross(c[(d + 1) % 3], c[(d + 2) % 3])))
        if vol <= 0.0 or area <= 0.0:
            return float("inf")
        img *= 2.0 * float(radius) / (vol / area) + 1.0
    return img


def _batch_in_one_pass(natoms, cells=None, pbc=(True, True, True), radius=6.0) -> bool:
    """Whether the batched build is expected to beat the per-structure loop.  Without
    ``cells`` every structure is costed at the measured image count."""
    if len(natoms) < 2 or max(natoms) > BATCH_MAX_ATOMS:
        return False
    if cells is None:
        weights = [1.0] * len(natoms)
    else:
        weights = [_images_per_pair(c, pbc, radius) / _BATCH_IMAGES_MEASURED for c in cells]
        if max(weights) * _BATCH_IMAGES_MEASURED > BATCH_MAX_IMAGES:
            return False
    pairs = sum(n * n * w for n, w in zip(natoms, weights))
    return _BATCH_MS + _BATCH_MS_PER_PAIR * pairs < _LOOP_MS_PER_STRUCTURE * len(natoms)


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

    natoms = [int(x) for x in data.natoms.tolist()]
    pbc_list = [bool(x) for x in pbc_flags.tolist()]
    if _batch_in_one_pass(natoms, data.cell.detach().to("cpu", torch.float64).numpy(), pbc_list,
                          float(radius)):
        return _impl.build_batch(data.pos, data.cell, data.natoms, pbc_flags, float(radius),
                                 int(max_num_neighbors_threshold))

    eis, cos, nns = [], [], []
    offset = 0
    for i in range(batch_size):
        n = natoms[i]
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
