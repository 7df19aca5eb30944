"""The C-ABI library loads, exports every symbol include/dynamis_graph.h declares, and
its host-side planning answers without a GPU (no kernel is launched here)."""
import ctypes
import os
import re

import numpy as np

from dynamis_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "dynamis_graph.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(dg_[a-z_0-9]+)\s*\(", src)))


def test_exports_every_declared_symbol():
    lib = L.lib()
    names = _declared()
    assert "dg_graph_count" in names and "dg_graph_write" in names
    raw = ctypes.CDLL(L.LIB_PATH)
    for n in names:
        assert hasattr(raw, n), n
    assert lib.dg_version().startswith(b"dynamis_graph")


def _desc(n, L_box=50.0, r=6.0, pbc=(1, 1, 1), cell=None):
    d = L.GraphDesc()
    d.n_atoms = n
    d.pos_dtype = L.DG_F32
    c = np.eye(3) * L_box if cell is None else np.asarray(cell, float)
    for k, v in enumerate(c.reshape(-1)):
        d.cell[k] = float(v)
    for k in range(3):
        d.pbc[k] = pbc[k]
    d.radius = r
    return d


def test_workspace_size_and_validation():
    lib = L.lib()
    assert lib.dg_graph_workspace_size(_desc(1_000_000, 215.443)) > 16 * 1_000_000
    assert lib.dg_graph_workspace_size(_desc(10, r=-1.0)) == 0
    assert b"radius must be positive" in lib.dg_last_error()
    assert lib.dg_graph_workspace_size(_desc(10, cell=np.zeros((3, 3)))) == 0
    assert b"singular" in lib.dg_last_error()
    # a cell far thinner than the radius (2 r / 1e-7 images per pair on one axis) is refused
    assert lib.dg_graph_workspace_size(_desc(10, cell=np.diag([10.0, 10.0, 1e-7]))) == 0
    assert b"too thin" in lib.dg_last_error()
    # a workspace that is too small is refused before anything is launched
    d = _desc(100)
    st = lib.dg_graph_count(d, ctypes.c_void_p(1), None, ctypes.c_void_p(1), 16, None, None)
    assert st == L.DG_ERR_WORKSPACE
    assert lib.dg_filter_workspace_size(1000) > 4000
    assert lib.dg_sfc_workspace_size(1000) > 8000


def test_write_refuses_null_inputs():
    """dg_graph_write checks its input pointers before anything is launched (no GPU needed)."""
    lib = L.lib()
    d = _desc(100)
    big = 1 << 40
    one = ctypes.c_void_p(16)
    st = lib.dg_graph_write(d, None, None, one, big, 10, one, one, one, None, None, L.DG_F32, None)
    assert st == L.DG_ERR_INVALID and b"pos is NULL" in lib.dg_last_error()
    st = lib.dg_graph_counts(d, None, None, one, big, None, None)
    assert st == L.DG_ERR_INVALID and b"pos is NULL" in lib.dg_last_error()
