"""DistGraphBuilder (dist_graph_builder.py:234-495): host logic on the CPU, the W=1
smoke of the reference's tests on the GPU, and multi-rank runs (one process per rank,
gloo over 127.0.0.1, every rank on cuda:0) checked against the oracles: r-degrees, the
weighted SFC cut, mode A / mode B edge sets, the halo plan against the serial full-graph
map, the send/recv mirror identity, and the drift watchdog.  Mirrors
dynamis_state/tests/test_dist_graph_builder.py:160-653."""
import os
import socket
import subprocess
import sys

import numpy as np
import pytest
import torch

from dynamis_amd.dynamis_state import dynamis_state_impl as impl
from dynamis_amd.dynamis_state.dist_graph_builder import (BuildMode, DistGraphBuilder,
                                                          _cell_block_partition)

WORKER = os.path.join(os.path.dirname(os.path.abspath(__file__)), "dist_worker.py")


def _free_port():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _launch(mode, W, extra=(), timeout=240):
    port = _free_port()
    env = dict(os.environ, MASTER_ADDR="127.0.0.1")
    procs = [subprocess.Popen([sys.executable, WORKER, "--mode", mode, "--rank", str(r), "--world",
                               str(W), "--port", str(port), *extra],
                              stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, env=env)
             for r in range(W)]
    outs, codes = [], []
    for p in procs:
        try:
            out, _ = p.communicate(timeout=timeout)
        except subprocess.TimeoutExpired:
            for q in procs:
                q.kill()
            out, _ = p.communicate()
        outs.append(out)
        codes.append(p.returncode)
    text = "\n".join(outs)
    print(text[-4000:])
    assert codes == [0] * W, text[-4000:]


def test_cell_block_partition_covers_and_splits():
    g = torch.Generator().manual_seed(0)
    L = torch.tensor([30.0, 31.0, 29.0])
    pos = torch.rand(2000, 3, generator=g) * L
    for W in (1, 2, 3, 7):
        parts = [_cell_block_partition(pos, L, 4.5, r, W) for r in range(W)]
        allv = torch.cat(parts).sort().values
        assert torch.equal(allv, torch.arange(2000))  # disjoint and complete
    # 6 x 6 x 6 cells of 5 A: rank r of 2 owns cell ids [0,108) / [108,216): z < 15 / z >= 15
    L = torch.tensor([30.0, 30.0, 30.0])
    pos = torch.rand(500, 3, generator=g) * L
    lo = _cell_block_partition(pos, L, 5.0, 0, 2)
    assert torch.equal(lo, torch.nonzero(pos[:, 2] < 15.0).squeeze(-1))


def test_drift_watchdog_minimum_image():
    env = impl.DistEnvironment()
    b = DistGraphBuilder(torch.eye(3) * 10.0, torch.tensor([True] * 3), 3.0, 0.5, env)
    assert b.drift_threshold == 0.25
    p0 = torch.tensor([[9.95, 5.0, 5.0], [1.0, 1.0, 1.0]])
    b._pos_w_at_refresh = b._pbc_wrap(p0)
    assert not b._live_drift_exceeded(b._pbc_wrap(p0 + torch.tensor([0.1, 0.0, 0.0])))  # crosses L
    assert b._live_drift_exceeded(b._pbc_wrap(p0 + torch.tensor([0.0, 0.3, 0.0])))
    assert b.next_is_refresh
    b.reset()
    assert b._pos_w_at_refresh is None and b.next_is_refresh


def test_gloo_degree_sum_two_ranks():
    _launch("reduce", 2, timeout=120)


@pytest.mark.gpu
def test_single_rank_smoke(cuda):
    """Reference test_v5_single_rank_smoke: W=1, everything local, empty halo."""
    torch.manual_seed(42)
    N, L = 200, 30.0
    pos = torch.rand(N, 3, device=cuda) * L
    env = impl.DistEnvironment()
    b = DistGraphBuilder(torch.eye(3) * L, torch.tensor([True] * 3), 4.0, 0.5, env, refresh_interval=100)
    res = b.build(pos)
    assert res.mode == BuildMode.REFRESH
    assert res.my_outer_atoms.numel() == N
    assert res.halo_info.send_offsets[-1].item() == 0
    assert res.halo_info.recv_offsets[-1].item() == 0
    assert bool(res.interior_mask.all().item())
    assert res.halo_recv_global_ids.numel() == 0
    ei, sh, _, _ = impl.radius_graph_pbc_ex(b._pbc_wrap(pos), torch.eye(3) * L, torch.tensor([True] * 3),
                                            4.0, 0, False, None)
    assert res.edges_outer.shape == ei.shape
    res2 = b.build(pos)
    assert res2.mode == BuildMode.STEADY and res2.edges_outer.shape == ei.shape


@pytest.mark.gpu
@pytest.mark.parametrize("W,extra", [(2, ()), (3, ("--n", "6000", "--box", "40", "--cutoff", "5",
                                                     "--seed", "9999"))])
def test_multirank_vs_oracles(cuda, W, extra):
    print(f"\n[case] dist builder W={W} {extra}", flush=True)
    _launch("builder", W, extra)
