"""Seeded synthetic atom boxes of the benchmark configurations (numpy default_rng,
positions generated in fp64, cast at the end).

C1  FCC a=3.6 A, 6^3 unit cells (L=21.6 A), Gaussian jitter 0.1 A, fp64, r=6, PBC.
C2  100,000 atoms uniform at 0.1 A^-3 (L=100 A), r=6, fp32 or fp64.
C3  1,000,000 atoms uniform at 0.1 A^-3 (L=(1e7)^(1/3)=215.443 A), r=6, fp32.  Headline.
C4  triclinic rows a=(160,0,0) b=(40,150,0) c=(30,25,140); lower half along c at 0.1 A^-3,
    upper half at 0.01 A^-3 -> 184,800 atoms; r=5; fp64.
C5  one GPU's partition: 4,000,000 owned atoms uniform in a 342 A cube plus ghosts at
    0.1 A^-3 in the 6 A shell around it; owned first, then ghosts; no PBC; the box is
    translated by +6 A so the 354 A cubic cell contains every atom; targets = owned.

Sizes differing from the benchmark text (100k at 0.1 A^-3 needs L=100 A, not 46.4 A; the
triclinic cell holds 184,800 atoms at the stated densities, not 500,000) follow the
densities, which fix the ~90 neighbours per atom the text also states.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class Box:
    name: str
    pos: np.ndarray
    cell: np.ndarray
    pbc: tuple
    radius: float
    targets: np.ndarray | None = None
    note: str = ""
    extra: dict = field(default_factory=dict)


def fcc(cells=6, a=3.6, jitter=0.1, seed=0, dtype=np.float64):
    rng = np.random.default_rng(seed)
    base = np.array([[0, 0, 0], [0.5, 0.5, 0], [0.5, 0, 0.5], [0, 0.5, 0.5]])
    g = np.stack(np.meshgrid(np.arange(cells), np.arange(cells), np.arange(cells), indexing="ij"), -1)
    pos = ((g.reshape(-1, 1, 3) + base[None]) * a).reshape(-1, 3)
    if jitter:
        pos = pos + rng.normal(0.0, jitter, pos.shape)
    L = cells * a
    return Box("C1", pos.astype(dtype), np.eye(3) * L, (True, True, True), 6.0)


def uniform(n, density=0.1, seed=1, dtype=np.float32, radius=6.0, name="uniform"):
    rng = np.random.default_rng(seed)
    L = (n / density) ** (1.0 / 3.0)
    pos = rng.uniform(0.0, L, (n, 3))
    return Box(name, pos.astype(dtype), np.eye(3) * L, (True, True, True), radius)


def c2(dtype=np.float32):
    return uniform(100_000, seed=1, dtype=dtype, name="C2")


def c3(dtype=np.float32):
    return uniform(1_000_000, seed=2, dtype=dtype, name="C3")


def c4(scale=1.0, dtype=np.float64, seed=3):
    rng = np.random.default_rng(seed)
    cell = np.array([[160.0, 0, 0], [40.0, 150.0, 0], [30.0, 25.0, 140.0]]) * scale
    vol = abs(np.linalg.det(cell))
    n_lo = int(round(0.1 * vol / 2))
    n_hi = int(round(0.01 * vol / 2))
    f_lo = rng.uniform(0, 1, (n_lo, 3)) * [1, 1, 0.5]
    f_hi = rng.uniform(0, 1, (n_hi, 3)) * [1, 1, 0.5] + [0, 0, 0.5]
    frac = np.concatenate([f_lo, f_hi])
    pos = frac @ cell
    return Box("C4", pos.astype(dtype), cell, (True, True, True), 5.0)


def c5(n_owned=4_000_000, side=342.0, shell=6.0, density=0.1, seed=4, dtype=np.float32):
    rng = np.random.default_rng(seed)
    owned = rng.uniform(0.0, side, (n_owned, 3))
    outer = side + 2 * shell
    n_ghost = int(round(density * (outer ** 3 - side ** 3)))
    # rejection-sample the shell in chunks
    ghosts = []
    got = 0
    while got < n_ghost:
        cand = rng.uniform(-shell, side + shell, (max(2 * (n_ghost - got), 1024), 3))
        inside = np.all((cand >= 0.0) & (cand < side), axis=1)
        cand = cand[~inside]
        ghosts.append(cand[: n_ghost - got])
        got += ghosts[-1].shape[0]
    ghost = np.concatenate(ghosts) if ghosts else np.zeros((0, 3))
    pos = np.concatenate([owned, ghost]) + shell
    box = Box("C5", pos.astype(dtype), np.eye(3) * outer, (False, False, False), 6.0,
              targets=np.arange(n_owned, dtype=np.int64))
    box.extra["n_owned"] = n_owned
    return box


def displace(pos, sigma, seed):
    rng = np.random.default_rng(seed)
    return (pos.astype(np.float64) + rng.normal(0.0, sigma, pos.shape)).astype(pos.dtype)


def walk(pos, sigma, seed=7):
    """Position frames of a random walk on the device: frame 0 is ``pos`` (a torch tensor),
    frame k is frame k - 1 displaced by Gaussian ``sigma`` per coordinate (torch generator
    on pos's device, seeded).  The trajectory the benchmark rebuilds from (C5: 100 frames
    at 0.01 A)."""
    import torch

    g = torch.Generator(device=pos.device).manual_seed(seed)
    cur = pos
    while True:
        yield cur
        cur = cur + sigma * torch.randn(pos.shape, generator=g, device=pos.device, dtype=pos.dtype)
