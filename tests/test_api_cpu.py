"""The Python mirror of the reference API raises the reference's errors on bad input
(radius_graph.cpp:15-37) without touching a GPU."""
import pytest
import torch

from dynamis_amd.dynamis_state import dynamis_state_impl as impl
from dynamis_amd.dynamis_state import radius_graph_pbc_cuda


def test_pos_must_be_cuda():
    with pytest.raises(RuntimeError, match="pos must be a CUDA tensor"):
        impl.radius_graph_pbc(torch.zeros(4, 3), torch.eye(3), torch.ones(3, dtype=torch.bool), 5.0, 0, False)
    with pytest.raises(RuntimeError, match="pos must be a CUDA tensor"):
        impl.radius_graph_pbc_counts_ex(torch.zeros(4, 3), torch.eye(3), torch.ones(3, dtype=torch.bool), 5.0)
    with pytest.raises(RuntimeError, match="edges must be a CUDA tensor"):
        impl.filter_edges_to_radius(torch.zeros(2, 3, dtype=torch.long), torch.zeros(3, 3),
                                    torch.zeros(4, 3), torch.eye(3), 5.0)


def test_wrapper_rejects_mixed_pbc():
    class D:
        pos = torch.zeros(2, 3)
        cell = torch.eye(3).unsqueeze(0).repeat(2, 1, 1)
        natoms = torch.tensor([1, 1])
        pbc = torch.tensor([[True, True, True], [True, False, True]])

    with pytest.raises(RuntimeError, match="different PBC"):
        radius_graph_pbc_cuda(D(), 5.0, 0)


def test_sfc_curve_enum():
    assert int(impl.SFCCurveType.Morton) == 0 and int(impl.SFCCurveType.Hilbert) == 1
