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


def test_type_stubs_match_the_module():
    """Every name the stub file declares exists in the module, and every function's
    parameter names and defaults' presence match the implementation."""
    import ast
    import inspect
    import os

    path = os.path.join(os.path.dirname(impl.__file__), "dynamis_state_impl.pyi")
    tree = ast.parse(open(path).read())
    names = [n for n in tree.body if isinstance(n, (ast.FunctionDef, ast.ClassDef))]
    assert len(names) >= 15
    for node in names:
        assert hasattr(impl, node.name), node.name
        if isinstance(node, ast.FunctionDef):
            sig = inspect.signature(getattr(impl, node.name))
            stub = [a.arg for a in node.args.args]
            assert stub == list(sig.parameters), (node.name, stub, list(sig.parameters))
            n_def = len(node.args.defaults)
            has_def = [p.default is not inspect.Parameter.empty for p in sig.parameters.values()]
            assert has_def == [False] * (len(stub) - n_def) + [True] * n_def, node.name


def test_batch_cost_model_counts_periodic_images():
    import importlib
    wrap = importlib.import_module("dynamis_amd.dynamis_state.radius_graph_pbc_cuda")
    cube = lambda L: [[L, 0, 0], [0, L, 0], [0, 0, L]]
    # 128 structures of 250 atoms in 14.6 A cubes at r = 6: the batch (the measured case)
    assert abs(wrap._images_per_pair(cube(14.6), [True] * 3, 6.0) - (2 * 6 / 14.6 + 1) ** 3) < 1e-9
    assert wrap._batch_in_one_pass([250] * 128, [cube(14.6)] * 128, [True] * 3, 6.0)
    # the same atoms in 1.5 A cells at r = 6 A: 9^3 images per pair -> the loop
    assert wrap._images_per_pair(cube(1.5), [True] * 3, 6.0) == 9.0 ** 3
    assert not wrap._batch_in_one_pass([250] * 128, [cube(1.5)] * 128, [True] * 3, 6.0)
    # no periodic axis: one image whatever the cell
    assert wrap._images_per_pair(cube(2.0), [False] * 3, 6.0) == 1.0
    assert wrap._batch_in_one_pass([250] * 128, [cube(2.0)] * 128, [False] * 3, 6.0)
    # a singular cell is never batched
    assert not wrap._batch_in_one_pass([10, 10], [[[1, 0, 0], [1, 0, 0], [0, 0, 1]]] * 2, [True] * 3, 6.0)
