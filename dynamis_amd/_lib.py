"""ctypes binding of libdynamis_graph.so (C ABI: include/dynamis_graph.h).

torch is imported first so the library's libamdhip64.so.7 dependency resolves to the HIP
runtime torch already loaded (same soname), giving one runtime, one set of streams.
Loading fails loudly when the library is missing -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the dlopen below)

_HERE = os.path.dirname(os.path.abspath(__file__))
# DYNAMIS_GRAPH_LIB selects another build of the same library (e.g. one compiled with
# different options); the default is the in-tree build.
LIB_PATH = os.environ.get("DYNAMIS_GRAPH_LIB") or os.path.join(_HERE, "libdynamis_graph.so")

DG_F32, DG_F64, DG_I64, DG_I32 = 0, 1, 2, 3
DG_OK, DG_ERR_INVALID, DG_ERR_WORKSPACE, DG_ERR_HIP, DG_ERR_RANGE, DG_ERR_CAPACITY = range(6)


class GraphDesc(ctypes.Structure):
    """dg_graph_desc."""

    _fields_ = [
        ("n_atoms", ctypes.c_int64),
        ("n_targets", ctypes.c_int64),
        ("has_targets", ctypes.c_int32),
        ("pos_dtype", ctypes.c_int32),
        ("cell", ctypes.c_double * 9),
        ("pbc", ctypes.c_uint8 * 3),
        ("pad_", ctypes.c_uint8 * 5),
        ("radius", ctypes.c_double),
    ]


class HaloDesc(ctypes.Structure):
    """dg_halo_desc."""

    _fields_ = [
        ("n_atoms", ctypes.c_int64),
        ("n_edges", ctypes.c_int64),
        ("num_local", ctypes.c_int64),
        ("my_rank", ctypes.c_int64),
        ("world_size", ctypes.c_int64),
        ("pid_dtype", ctypes.c_int32),
        ("pad_", ctypes.c_int32),
    ]


class BatchDesc(ctypes.Structure):
    """dg_batch_desc."""

    _fields_ = [
        ("n_images", ctypes.c_int64),
        ("n_atoms", ctypes.c_int64),
        ("pos_dtype", ctypes.c_int32),
        ("pbc", ctypes.c_uint8 * 3),
        ("pad_", ctypes.c_uint8),
        ("radius", ctypes.c_double),
    ]


_lib = None

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build the HIP library first "
            "(python -m dynamis_amd.build, or __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    D = ctypes.POINTER(GraphDesc)
    sig = {
        "dg_graph_workspace_size": (_sz, [D]),
        "dg_graph_count": (_i32, [D, _p, _p, _p, _sz, _p, _p]),
        "dg_graph_read_totals": (_i32, [D, _p, ctypes.POINTER(_i64), ctypes.POINTER(_i64), _p]),
        "dg_graph_counts": (_i32, [D, _p, _p, _p, _sz, _p, _p]),
        "dg_graph_write": (_i32, [D, _p, _p, _p, _sz, _i64, _p, _p, _p, _p, _p, _i32, _p]),
        "dg_graph_write_ids": (_i32, [D, _p, _p, _p, _sz, _i64, _p, _p, _p, _p, _p, _p, _i32, _p]),
        "dg_graph_build": (_i32, [D, _p, _p, _p, _sz, _i64, _p, _p, _p, _p, _p, _p, _i32, _p]),
        "dg_graph_build_noalloc": (_i32, [D, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _i32, _p, _p]),
        "dg_filter_workspace_size": (_sz, [_i64]),
        "dg_filter_edges_to_radius": (_i32, [_p, _i32, _i64, _p, ctypes.c_double, _p, _p, _p, _i32,
                                             _i64, _p, _p, _p, _sz, _p]),
        "dg_filter2_workspace_size": (_sz, [_i64]),
        "dg_filter_count": (_i32, [_p, _i32, _i64, _p, ctypes.c_double, _p, _p, _p, _i32, _i64, _p,
                                   _p, _sz, _p]),
        "dg_filter_write": (_i32, [_p, _i32, _i64, _p, ctypes.c_double, _p, _p, _p, _i32, _i64, _p,
                                   _sz, _p, _p, _p, _p]),
        "dg_filter_compact_workspace_size": (_sz, [_i64]),
        "dg_filter_compact": (_i32, [_p, _i32, _i64, _p, ctypes.c_double, _p, _p, _p, _i32, _i64, _p,
                                     _p, _p, _p, _p, _sz, _p]),
        "dg_sfc_workspace_size": (_sz, [_i64]),
        "dg_sfc_keys": (_i32, [_p, _i64, _i32, _p, _p, _sz, _p]),
        "dg_sfc_order": (_i32, [_p, _i64, _p, _p, _sz, _p]),
        "dg_sfc_labels": (_i32, [_p, _i64, _i64, _p, _p, _p, _sz, _p]),
        "dg_halo_workspace_size": (_sz, [_i64, _i64]),
        "dg_halo_count": (_i32, [ctypes.POINTER(HaloDesc), _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p]),
        "dg_halo_read_totals": (_i32, [_p, ctypes.POINTER(_i64), ctypes.POINTER(_i64), _p]),
        "dg_halo_write": (_i32, [ctypes.POINTER(HaloDesc), _p, _p, _p, _p, _p, _sz, _p]),
        "dg_batch_workspace_size": (_sz, [ctypes.POINTER(BatchDesc)]),
        "dg_batch_count": (_i32, [ctypes.POINTER(BatchDesc), _p, _p, _p, _p, _p, _sz, _p]),
        "dg_batch_read_totals": (_i32, [ctypes.POINTER(BatchDesc), _p, ctypes.POINTER(_i64), ctypes.POINTER(_i64), _p]),
        "dg_batch_write": (_i32, [ctypes.POINTER(BatchDesc), _p, _p, _sz, _i64, _p, _p, _p, _p, _p]),
        "dg_last_error": (ctypes.c_char_p, []),
        "dg_version": (ctypes.c_char_p, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(status: int, what: str) -> None:
    if status != DG_OK:
        msg = lib().dg_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {msg}")


def stream_of(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)
