"""Frozen golden edge lists (tests/golden/graph_*.npz, written by tests/golden/
make_golden.py from the definition of the edge set alone): the CPU oracle and the GPU
path must reproduce them exactly after a canonical (dst, src, shift) sort."""
import glob
import os

import numpy as np
import pytest

import oracle

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                       "graph_*.npz")))


def _canon(src, dst, shift):
    e = np.concatenate([np.asarray(src, np.int64)[:, None], np.asarray(dst, np.int64)[:, None],
                        np.asarray(shift).astype(np.int64)], 1)
    return e[np.lexsort((e[:, 4], e[:, 3], e[:, 2], e[:, 0], e[:, 1]))]


def _load(path):
    z = np.load(path)  # allow_pickle stays False: plain arrays written by make_golden.py
    return (z["pos"], z["cell"], tuple(int(x) for x in z["pbc"]), float(z["radius"]),
            _canon(z["src"], z["dst"], z["shift"]))


def test_golden_files_present():
    assert len(GOLDEN) >= 6


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: os.path.basename(p)[6:-4])
def test_oracle_matches_golden(path):
    pos, cell, pbc, r, want = _load(path)
    o = oracle.radius_graph(pos, cell, pbc, r)
    assert np.array_equal(_canon(o["src"], o["dst"], o["shift"]), want)


@pytest.mark.gpu
@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: os.path.basename(p)[6:-4])
def test_gpu_matches_golden(cuda, path):
    import torch

    from dynamis_amd.dynamis_state import dynamis_state_impl as impl

    print(f"\n[case] golden {os.path.basename(path)}", flush=True)
    pos, cell, pbc, r, want = _load(path)
    ei, sh, nn, cnt = impl.radius_graph_pbc_ex(torch.from_numpy(pos).to(cuda), torch.from_numpy(cell),
                                               torch.tensor([bool(x) for x in pbc]), r, 0, False)
    got = _canon(ei[0].cpu().numpy(), ei[1].cpu().numpy(), sh.cpu().numpy())
    assert np.array_equal(got, want)
    assert int(nn.item()) == len(want)
