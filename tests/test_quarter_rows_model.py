"""Model check of the count pass's quarter-bin row ends (dg_graph.hip: row_range in
search_tile, bin_xkey).  The row bounds and quarter cuts are evaluated here in fp32 as the
kernel states them (an fma as one rounding), for random orthorhombic and lower-triangular
cells, targets and atoms, with atoms placed on and just below every quarter boundary.
Every atom within the cutoff of the target must survive the cut: it lies in the row's
bins, at or above the first bin's quarter start and below the last bin's quarter end.
The GPU parity tests check the kernel itself against the oracle; this pins the bound's
arithmetic on some 10^5 pairs at no GPU cost."""
import numpy as np

f32 = np.float32


def fma(a, b, c):
    return f32(np.float64(a) * np.float64(b) + np.float64(c))


def _grid(rng, ortho):
    L = rng.uniform(30, 60, 3)
    C = np.diag(L)
    if not ortho:
        C[1, 0], C[2, 0], C[2, 1] = rng.uniform(-0.4, 0.4, 3) * L[[1, 2, 2]]
    r = rng.uniform(3, 7)
    vol = abs(np.linalg.det(C))
    a0, a1, a2 = C
    dface = [vol / np.linalg.norm(np.cross(a1, a2)), vol / np.linalg.norm(np.cross(a2, a0)),
             vol / np.linalg.norm(np.cross(a0, a1))]
    nb = [int(np.floor(2 * d / r * (1 - 1e-6))) for d in dface]
    P = [int(np.ceil(r / d * n * (1 + 1e-9) + 1e-12)) for d, n in zip(dface, nb)]
    return C, r, nb, P


def _rows(C, r, nb, P, ft, ortho):
    """(oy, oz, xlo, xhi, qlo, qhi) of every row the padded cutoff reaches, as the kernel
    computes them for a target at fractions ft inside its bin."""
    hax, hbx, hby = f32(C[0, 0] / nb[0]), f32(C[1, 0] / nb[1]), f32(C[1, 1] / nb[1])
    hcx, hcy, hcz = f32(C[2, 0] / nb[2]), f32(C[2, 1] / nb[2]), f32(C[2, 2] / nb[2])
    inv_hax, inv_hby, inv_hcz = f32(nb[0] / C[0, 0]), f32(nb[1] / C[1, 1]), f32(nb[2] / C[2, 2])
    pm = f32(1e-4 * r + 1e-3)
    rprune2 = f32((r + 2 * pm) ** 2)
    gy_off, gz_off = f32(-hby - pm), f32(-hcz - pm)
    nrx = 2 * P[0] + 1
    hb = _steps(C, nb)
    ut = (ft @ hb).astype(f32)
    Oz = f32(ut[2] * inv_hcz)
    Oy = f32((ut[1] - Oz * hcy) * inv_hby)
    Ox = f32((ut[0] - Oy * hbx - Oz * hcx) * inv_hax)
    Oxp = f32(Ox + P[0])
    Oxp4, inv4 = f32(4 * Oxp), f32(4 * inv_hax)
    out = []
    for oz in range(2 * P[2] + 1):
        for oy in range(2 * P[1] + 1):
            py, pz = f32(f32(oy - P[1]) - Oy), f32(f32(oz - P[2]) - Oz)
            if ortho:
                gy = max(fma(py, hby, -pm), fma(-py, hby, gy_off), f32(0))
                gz = max(fma(pz, hcz, -pm), fma(-pz, hcz, gz_off), f32(0))
                rem2 = fma(-gy, gy, fma(-gz, gz, rprune2))
                if rem2 < 0:
                    continue
                rem = f32(np.sqrt(rem2))
                QL = max(int(np.floor(fma(-rem, inv4, Oxp4))), 0)
                QH = min(int(np.floor(fma(rem, inv4, Oxp4))), 4 * nrx - 1)
            else:
                zl = f32(pz * hcz)
                zh = f32(zl + hcz)
                cyl = min(f32(pz * hcy), f32(f32(pz + 1) * hcy))
                cyh = max(f32(pz * hcy), f32(f32(pz + 1) * hcy))
                yl, yh = f32(f32(py * hby) + cyl), f32(f32(f32(py + 1) * hby) + cyh)
                gy = max(f32(max(yl, -yh, f32(0)) - pm), f32(0))
                gz = max(f32(max(zl, -zh, f32(0)) - pm), f32(0))
                rem2 = f32(f32(rprune2 - f32(gy * gy)) - f32(gz * gz))
                if rem2 < 0:
                    continue
                rem = f32(np.sqrt(rem2))
                sl = f32(min(f32(py * hbx), f32(f32(py + 1) * hbx)) + min(f32(pz * hcx), f32(f32(pz + 1) * hcx)))
                sh = f32(max(f32(py * hbx), f32(f32(py + 1) * hbx)) + max(f32(pz * hcx), f32(f32(pz + 1) * hcx)))
                QL = max(int(np.floor(f32(4 * f32(Ox + f32(f32(-rem - sh) * inv_hax))))) + 4 * P[0], 0)
                QH = min(int(np.floor(f32(4 * f32(Ox + f32(f32(rem - sl) * inv_hax))))) + 4 * P[0], 4 * nrx - 1)
            if (QL >> 2) <= (QH >> 2):
                out.append((oy, oz, QL >> 2, QH >> 2, QL & 3, QH & 3))
    return out


def _steps(C, nb):
    """Bin step vectors (rows): C[d] / nb[d]."""
    return np.array([C[d] / nb[d] for d in range(3)])


def _xkey(e, C, nb):
    """bin_xkey of a cell-list record's offset e inside its bin."""
    hbx, hcx, hcy = f32(C[1, 0] / nb[1]), f32(C[2, 0] / nb[2]), f32(C[2, 1] / nb[2])
    inv_hby, inv_hcz = f32(nb[1] / C[1, 1]), f32(nb[2] / C[2, 2])
    fc = f32(e[2] * inv_hcz)
    fb = f32(fma(-fc, hcy, e[1]) * inv_hby)
    return fma(-fc, hcx, fma(-fb, hbx, e[0]))


def test_quarter_cuts_keep_every_neighbour():
    rng = np.random.default_rng(1)
    checked = missed = 0
    for trial in range(240):
        ortho = trial % 2 == 0
        C, r, nb, P = _grid(rng, ortho)
        if max(P) != 2:
            continue
        hb = _steps(C, nb)
        hax = f32(C[0, 0] / nb[0])
        ft = rng.uniform(0, 1, 3)
        for oy, oz, xlo, xhi, qlo, qhi in _rows(C, r, nb, P, ft, ortho):
            for xr in range(2 * P[0] + 1):
                fr = rng.uniform(0, 1, (40, 3))
                fr[:8, 0] = [0, 0.25, 0.5, 0.75, 1 - 1e-7, 0.25 - 1e-7, 0.5 - 1e-7, 0.75 - 1e-7]
                for f in fr:
                    d = (np.array([xr - P[0], oy - P[1], oz - P[2]]) + f - ft) @ hb
                    if d @ d > r * r:
                        continue
                    checked += 1
                    k = _xkey((f @ hb).astype(f32), C, nb)
                    kept = xlo <= xr <= xhi
                    if kept and xr == xlo and qlo > 0 and k < f32(qlo * 0.25 * hax):
                        kept = False
                    if kept and xr == xhi and qhi < 3 and not k < f32((qhi + 1) * 0.25 * hax):
                        kept = False
                    missed += not kept
    assert checked > 100000
    assert missed == 0
