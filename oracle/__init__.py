"""CPU oracle for the PBC radius graph and SFC keys -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this package, and only as the checker or the reported CPU baseline.  The product
(``dynamis_amd``) never imports it.

``graph_oracle.c`` restates the reference algorithm (file:line citations there) with the
canonical fp64 cutoff predicate.  ``brute.py`` is an independent O(N^2 * images) checker
written directly from the mathematical definition of the edge set.

Pinning (what checks each function; see tests/test_oracle.py):
  * ``radius_graph``        -- brute force (independent definition, tiny N), scipy cKDTree
                               (orthorhombic, r < L/2), the reference tests' closed-form
                               answers (single atom box 5 r 6 -> 6 edges; no PBC -> 0;
                               empty), FCC closed form (78 neighbours/atom), exact-cutoff
                               lattice (simple cubic spacing 2, r=4 -> 32 neighbours/atom),
                               symmetry (i,j,S) <-> (j,i,-S).
  * ``edge_vectors``        -- closed form on lattices; |v| <= r on every edge.
  * ``filter_edges``        -- filter(build(r+skin), r) == build(r) as sets.
  * ``morton_keys``         -- spread identities, decode(encode) round trip with an
                               independent decoder, magic-number form in the HIP build.
  * ``hilbert_keys``        -- exhaustive over all 128^3 quantised cells against
                               oracle/sfc_twin.py, a second restatement that follows the
                               reference's CPU twin (sfc_partitioner.cpp:50-92) instead of
                               the CUDA kernel this file follows; range, b=0 pass-through.
  * ``morton_keys`` (again) -- against the CPU twin's bit loop (sfc_partitioner.cpp:21-45).
  * ``sfc_labels``          -- closed-form balance (unweighted), exact integer cut rule
                               (weighted) on hand-checked cases.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_dbl = ctypes.c_double


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_graph_count.restype = _p
        L.orc_graph_count.argtypes = [_p, ctypes.c_int, _i64, _p, _p, _dbl, _p, _i64, _p, _p, ctypes.c_int]
        L.orc_graph_write.restype = None
        L.orc_graph_write.argtypes = [_p, _p, _p, _p, _p, _p]
        L.orc_graph_free.argtypes = [_p]
        L.orc_graph_num_images.restype = _i64
        L.orc_graph_num_images.argtypes = [_p]
        L.orc_geometry_export.restype = ctypes.c_int
        L.orc_geometry_export.argtypes = [_p, _p, _dbl, _p, _p, _p]
        L.orc_edge_vectors.argtypes = [_p, ctypes.c_int, _p, _i64, _p, _p, _p, _p, _p]
        L.orc_filter_edges.restype = _i64
        L.orc_filter_edges.argtypes = [_p, ctypes.c_int, _p, _dbl, _i64, _p, _p, _p, _p]
        L.orc_ref32_decide.restype = None
        L.orc_ref32_decide.argtypes = [_p, _i64, _p, _p, _dbl, _i64, _p, _p, _p, _p]
        L.orc_sfc_bounds.argtypes = [_p, _i64, _p, _p]
        L.orc_morton_keys.argtypes = [_p, _i64, _p, _p, _p, ctypes.c_int]
        L.orc_hilbert_keys.argtypes = [_p, _i64, _p, _p, _p]
        L.orc_sfc_labels.argtypes = [_p, _i64, _i64, _p, _p]
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _prep(pos, cell, pbc):
    pos = np.ascontiguousarray(pos)
    if pos.dtype not in (np.float32, np.float64):
        raise TypeError("pos must be float32 or float64")
    cell = np.ascontiguousarray(np.asarray(cell, dtype=np.float64).reshape(3, 3))
    pbc = np.ascontiguousarray(np.asarray(pbc, dtype=np.uint8).reshape(3))
    return pos, cell, pbc


def radius_graph(pos, cell, pbc, radius, target_indices=None, vectors=False, threads=0):
    """Edge list of the canonical predicate, in the reference's emission order.

    Returns dict(src, dst int64 [E], shift int32 [E,3], counts int32 [N_target],
    num_images int, and vec fp64 [E,3], d2 fp64 [E] if ``vectors``).
    """
    L = lib()
    pos, cell, pbc = _prep(pos, cell, pbc)
    n = pos.shape[0]
    tgt = None if target_indices is None else np.ascontiguousarray(target_indices, dtype=np.int64)
    nt = n if tgt is None else tgt.shape[0]
    counts = np.zeros(nt, dtype=np.int32)
    total = np.zeros(1, dtype=np.int64)
    h = L.orc_graph_count(_ptr(pos), int(pos.dtype == np.float64), n, _ptr(cell), _ptr(pbc),
                          float(radius), _ptr(tgt), nt, _ptr(counts), _ptr(total), int(threads))
    if not h:
        raise RuntimeError("oracle: singular cell")
    try:
        E = int(total[0])
        src = np.empty(E, np.int64)
        dst = np.empty(E, np.int64)
        shift = np.empty((E, 3), np.int32)
        vec = np.empty((E, 3), np.float64) if vectors else None
        d2 = np.empty(E, np.float64) if vectors else None
        L.orc_graph_write(h, _ptr(src), _ptr(dst), _ptr(shift), _ptr(vec), _ptr(d2))
        out = dict(src=src, dst=dst, shift=shift, counts=counts, num_images=L.orc_graph_num_images(h))
        if vectors:
            out["vec"] = vec
            out["d2"] = d2
        return out
    finally:
        L.orc_graph_free(h)


def radius_graph_counts(pos, cell, pbc, radius, target_indices=None, threads=0):
    L = lib()
    pos, cell, pbc = _prep(pos, cell, pbc)
    n = pos.shape[0]
    tgt = None if target_indices is None else np.ascontiguousarray(target_indices, dtype=np.int64)
    nt = n if tgt is None else tgt.shape[0]
    counts = np.zeros(nt, dtype=np.int32)
    total = np.zeros(1, dtype=np.int64)
    h = L.orc_graph_count(_ptr(pos), int(pos.dtype == np.float64), n, _ptr(cell), _ptr(pbc),
                          float(radius), _ptr(tgt), nt, _ptr(counts), _ptr(total), int(threads))
    if not h:
        raise RuntimeError("oracle: singular cell")
    L.orc_graph_free(h)
    return counts, int(total[0])


def geometry(cell, pbc, radius):
    L = lib()
    cell = np.ascontiguousarray(np.asarray(cell, dtype=np.float64).reshape(3, 3))
    pbc = np.ascontiguousarray(np.asarray(pbc, dtype=np.uint8).reshape(3))
    cinv = np.zeros(9)
    dface = np.zeros(3)
    rep = np.zeros(3, np.int32)
    if L.orc_geometry_export(_ptr(cell), _ptr(pbc), float(radius), _ptr(cinv), _ptr(dface), _ptr(rep)):
        raise RuntimeError("oracle: singular cell")
    return cinv.reshape(3, 3), dface, rep


def edge_vectors(pos, cell, src, dst, shift):
    L = lib()
    pos = np.ascontiguousarray(pos)
    cell = np.ascontiguousarray(np.asarray(cell, dtype=np.float64).reshape(3, 3))
    src = np.ascontiguousarray(src, np.int64)
    dst = np.ascontiguousarray(dst, np.int64)
    shift = np.ascontiguousarray(shift, np.int32)
    E = src.shape[0]
    vec = np.empty((E, 3), np.float64)
    d2 = np.empty(E, np.float64)
    L.orc_edge_vectors(_ptr(pos), int(pos.dtype == np.float64), _ptr(cell), E, _ptr(src), _ptr(dst),
                       _ptr(shift), _ptr(vec), _ptr(d2))
    return vec, d2


def filter_edges(pos, cell, radius, src, dst, shift):
    L = lib()
    pos = np.ascontiguousarray(pos)
    cell = np.ascontiguousarray(np.asarray(cell, dtype=np.float64).reshape(3, 3))
    src = np.ascontiguousarray(src, np.int64)
    dst = np.ascontiguousarray(dst, np.int64)
    shift = np.ascontiguousarray(shift, np.int32)
    E = src.shape[0]
    keep = np.zeros(E, np.uint8)
    L.orc_filter_edges(_ptr(pos), int(pos.dtype == np.float64), _ptr(cell), float(radius), E,
                       _ptr(src), _ptr(dst), _ptr(shift), _ptr(keep))
    return keep.astype(bool)


def ref32_decide(pos, cell, pbc, radius, src, dst, shift):
    """The reference's fp32 decision (radius_graph_kernels.cu:70-141, 247-250, 515-605)
    for candidate edges (src, dst, S): keep[e] is True iff its arithmetic emits edge e.
    For the fp32-vs-canonical disagreement report (see graph_oracle.c)."""
    L = lib()
    pos = np.ascontiguousarray(pos, np.float32)
    cell = np.ascontiguousarray(np.asarray(cell, dtype=np.float64).reshape(3, 3))
    pbc = np.ascontiguousarray(np.asarray(pbc, dtype=np.uint8).reshape(3))
    src = np.ascontiguousarray(src, np.int64)
    dst = np.ascontiguousarray(dst, np.int64)
    shift = np.ascontiguousarray(shift, np.int32)
    keep = np.zeros(src.shape[0], np.uint8)
    L.orc_ref32_decide(_ptr(pos), pos.shape[0], _ptr(cell), _ptr(pbc), float(radius), src.shape[0],
                       _ptr(src), _ptr(dst), _ptr(shift), _ptr(keep))
    return keep.astype(bool)


def fp32_disagreement(pos, cell, pbc, radius, delta=1e-3):
    """Canonical (fp64) edge set vs the reference's fp32 decisions on the same input.

    Candidates are the canonical edges at radius + delta (the fp32 errors are orders of
    magnitude below delta, so every edge either side can emit is among them).  Returns a
    dict: canonical edge count, the edges only the canonical set holds, the edges only the
    fp32 arithmetic emits, and the largest |d - r| over the differing pairs.
    """
    r = float(np.float32(radius))
    c = np.asarray(cell, np.float64).astype(np.float32).astype(np.float64)
    p32 = np.ascontiguousarray(pos, np.float32)
    o = radius_graph(p32, c, pbc, r + delta, vectors=True)
    canon = o["d2"] <= r * r
    ref = ref32_decide(p32, c, pbc, r, o["src"], o["dst"], o["shift"])
    only_c = canon & ~ref
    only_r = ref & ~canon
    diff = only_c | only_r
    dmax = float(np.max(np.abs(np.sqrt(o["d2"][diff]) - r))) if diff.any() else 0.0
    return {"edges": int(canon.sum()), "canonical_only": int(only_c.sum()),
            "fp32_only": int(only_r.sum()), "max_abs_d_minus_r": dmax}


def sfc_bounds(pos):
    L = lib()
    pos = np.ascontiguousarray(pos, np.float32)
    mn = np.zeros(3, np.float32)
    rg = np.zeros(3, np.float32)
    L.orc_sfc_bounds(_ptr(pos), pos.shape[0], _ptr(mn), _ptr(rg))
    return mn, rg


def morton_keys(pos, mn=None, rg=None, threads=1):
    L = lib()
    pos = np.ascontiguousarray(pos, np.float32)
    if mn is None:
        mn, rg = sfc_bounds(pos)
    keys = np.empty(pos.shape[0], np.int64)
    L.orc_morton_keys(_ptr(pos), pos.shape[0], _ptr(np.ascontiguousarray(mn, np.float32)),
                      _ptr(np.ascontiguousarray(rg, np.float32)), _ptr(keys), int(threads))
    return keys


def hilbert_keys(pos, mn=None, rg=None):
    L = lib()
    pos = np.ascontiguousarray(pos, np.float32)
    if mn is None:
        mn, rg = sfc_bounds(pos)
    keys = np.empty(pos.shape[0], np.int64)
    L.orc_hilbert_keys(_ptr(pos), pos.shape[0], _ptr(np.ascontiguousarray(mn, np.float32)),
                       _ptr(np.ascontiguousarray(rg, np.float32)), _ptr(keys))
    return keys


def sfc_labels(perm, W, weights=None):
    L = lib()
    perm = np.ascontiguousarray(perm, np.int64)
    w = None if weights is None else np.ascontiguousarray(weights, np.int64)
    labels = np.empty(perm.shape[0], np.int64)
    L.orc_sfc_labels(_ptr(perm), perm.shape[0], int(W), _ptr(w), _ptr(labels))
    return labels


def canonical_sort(src, dst, shift, *extra):
    """Lexicographic (src, dst, sx, sy, sz) order -- the canonical edge order."""
    shift = np.asarray(shift).astype(np.int64)
    order = np.lexsort((shift[:, 2], shift[:, 1], shift[:, 0], np.asarray(dst), np.asarray(src)))
    out = [np.asarray(src)[order], np.asarray(dst)[order], shift[order]]
    out += [np.asarray(x)[order] for x in extra]
    return out
