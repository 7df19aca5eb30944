// dg_plan.hpp -- host-side plan of one radius-graph build: cell geometry, the periodic
// fractional bin grid, the tile decomposition, the fp32 prefilter band and the layout of
// the caller-provided device workspace.
//
// Geometry follows dynamis_state/src/csrc/graph/radius_graph_kernels.cu:515-594
// (plane spacings d_face = |V| / |a_j x a_k|, cutoff_frac = r / d_face, cell^-1 by the
// adjugate), evaluated in fp64.  The grid differs from the reference's Cartesian bounding
// box (:662-692): bins are laid out in FRACTIONAL coordinates, nb_d bins along lattice
// vector d, so a triclinic cell is binned without empty corners and periodic images are
// reached by wrapping the bin index instead of materialising image atoms (:18-141).
#pragma once
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>

namespace dg {

constexpr int kBlock = 256;      // threads per search workgroup (4 x wave64)
#ifndef DG_SORT_CHUNKS
#define DG_SORT_CHUNKS 128
#endif
constexpr int kSortChunks = DG_SORT_CHUNKS;  // atom chunks of the tile-level counting sort
constexpr int kSortTilesMax = 36000;  // tiles it handles (an LDS histogram of ints, < 144 KiB)
constexpr int kMaxRegion = 768;  // region bins staged per tile
constexpr int kMaxReach = 1 << 16;  // bins a cutoff may reach per axis (far past kMaxRegion)
constexpr int kTileTargets = 235; // aim: targets per tile <= this (a 256-lane workgroup)
constexpr int kTileMax = 6;
constexpr int64_t kFewTiles = 1024;       // tiles below one round of workgroups on 256 CUs
constexpr double kFewTileTargets = 192;   // expected targets per tile when tiles are few       // bins per tile along one axis
constexpr int kCap = 1792;        // region entries staged in LDS per chunk

struct Plan {
    int64_t n = 0, nt = 0;  // atoms, targets
    int subset = 0;         // explicit target list
    int f64 = 0;            // positions are fp64
    double C[9], Cinv[9];
    double r = 0, r2 = 0;
    double d_face[3], cf[3];
    int pbc[3];
    int nb[3], P[3], T[3], ntl[3], R[3], mb[3];
    int tb = 0;             // bins per tile
    int64_t ntiles = 0, nbins = 0, ncodes = 0;
    int nregion = 0;
    int brute = 0;          // region too large: all-pairs path
    float hi = 0, lo_in = 0, tiny = 0;
    float toff = 0, hi_off = 0;  // the same bounds on d2 - toff (see plan_grid)
    uint32_t lo_bits = 0;        // bits of the fp32 bound lo_off on d2 - toff
    // workspace layout (byte offsets)
    size_t o_key, o_rank, o_rec, o_bcnt, o_bstart, o_sid, o_spos, o_sflr, o_inv;
    size_t o_cpos;  // write stage, vector outputs: positions in cell-list order (over key .. rec)
    size_t o_arr, o_tor, o_rot;  // o_arr: cell-list ids in arrival order (before the in-bin sort)
    size_t o_tcnt, o_tstart, o_wgb;  // tile-level counting sort: tile totals, starts, chunk bases
    size_t o_tarr;                   // the same sort of explicit targets: their tile buckets
    size_t o_stmp;                   // segment-sort scratch (8 B per atom or target)
    size_t o_tkey, o_trank, o_tbcnt, o_tbstart, o_tslot, o_tsidx, o_tcaller;
    size_t o_cnt, o_ttot, o_tfix, o_tbase, o_part, o_tot, o_slot;
    int K = 0;              // neighbour slot entries per target
    int64_t nrow = 0;       // slot rows (group-major row length)
    size_t ws_bytes = 0;
};

inline size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

// Fills geometry; returns nonzero for a singular / non-finite cell.
inline int plan_geometry(Plan& p, const double* cell, const uint8_t* pbc, double r)
{
    const double *a0 = cell, *a1 = cell + 3, *a2 = cell + 6;
    double c12[3] = {a1[1] * a2[2] - a1[2] * a2[1], a1[2] * a2[0] - a1[0] * a2[2],
                     a1[0] * a2[1] - a1[1] * a2[0]};
    double c20[3] = {a2[1] * a0[2] - a2[2] * a0[1], a2[2] * a0[0] - a2[0] * a0[2],
                     a2[0] * a0[1] - a2[1] * a0[0]};
    double c01[3] = {a0[1] * a1[2] - a0[2] * a1[1], a0[2] * a1[0] - a0[0] * a1[2],
                     a0[0] * a1[1] - a0[1] * a1[0]};
    double vol = a0[0] * c12[0] + a0[1] * c12[1] + a0[2] * c12[2];
    if (!(fabs(vol) > 0.0) || !isfinite(vol)) return 1;
    memcpy(p.C, cell, sizeof p.C);
    const double* cs[3] = {c12, c20, c01};
    double av = fabs(vol);
    for (int d = 0; d < 3; d++) {
        double nrm = sqrt(cs[d][0] * cs[d][0] + cs[d][1] * cs[d][1] + cs[d][2] * cs[d][2]);
        p.d_face[d] = av / nrm;
        p.cf[d] = r / p.d_face[d];
        p.pbc[d] = pbc[d] ? 1 : 0;
    }
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++) p.Cinv[i * 3 + j] = cs[j][i] / vol;
    p.r = r;
    p.r2 = r * r;
    return 0;
}

inline void plan_grid(Plan& p)
{
    // Bins: thickness >= r/2 between bin planes (cf * nb <= 2), capped so that a sparse
    // system does not allocate many more bins than atoms.
    double nbd[3];
    for (int d = 0; d < 3; d++) {
        double v = floor(2.0 / p.cf[d] * (1.0 - 1e-6));
        nbd[d] = std::min(std::max(v, 1.0), 1024.0);
    }
    const double cap = std::max(4.0 * (double)p.n, 4096.0);
    while (nbd[0] * nbd[1] * nbd[2] > cap) {
        double s = cbrt(nbd[0] * nbd[1] * nbd[2] / cap);
        if (s < 1.01) s = 1.01;
        for (int d = 0; d < 3; d++) nbd[d] = std::max(1.0, floor(nbd[d] / s));
    }
    for (int d = 0; d < 3; d++) {
        p.nb[d] = (int)nbd[d];
        // bins the cutoff reaches, capped (in double, before the conversion) far beyond any
        // region the tiled search takes: a cutoff of many cell widths goes all-pairs
        const double reach = ceil(p.cf[d] * p.nb[d] * (1.0 + 1e-9) + 1e-12);
        p.P[d] = (int)std::min(std::max(reach, 1.0), (double)kMaxReach);
    }
    // Tile: as many bins as keep the expected targets of a tile within one 256-lane
    // workgroup, with a region of at most kMaxRegion bins; prefer compact tiles.
    {
        const double bins = (double)p.nb[0] * p.nb[1] * p.nb[2];
        const double per_bin = (double)std::max<int64_t>(p.subset ? p.nt : p.n, 1) / bins;
        const double src_per_bin = (double)std::max<int64_t>(p.n, 1) / bins;
        // max_targets: the expected targets a tile may hold
        auto pick = [&](double max_targets, int* best) {
            double best_score = -1;
            best[0] = best[1] = best[2] = 1;
            for (int a = 1; a <= std::min(kTileMax, p.nb[0]); ++a)
                for (int b = 1; b <= std::min(kTileMax, p.nb[1]); ++b)
                    for (int c = 1; c <= std::min(kTileMax, p.nb[2]); ++c) {
                        const int64_t reg = (int64_t)(a + 2 * p.P[0]) * (b + 2 * p.P[1]) * (c + 2 * p.P[2]);
                        if (reg > kMaxRegion) continue;
                        if (a * b * c * per_bin > max_targets && a * b * c > 1) continue;
                        // the region's atoms fit one LDS chunk with 4 standard deviations to
                        // spare (a chunked tile is written by the slow direct path)
                        const double ra = (double)reg * src_per_bin;
                        if (ra + 4.0 * sqrt(ra) > kCap && a * b * c > 1) continue;
                        // most bins per tile first, then the least halo per bin
                        const double score = a * b * c * 1e6 - (double)reg / (a * b * c);
                        if (score > best_score) { best_score = score; best[0] = a; best[1] = b; best[2] = c; }
                    }
        };
        auto tiles_of = [&](const int* t) {
            return (int64_t)((p.nb[0] + t[0] - 1) / t[0]) * ((p.nb[1] + t[1] - 1) / t[1]) *
                   ((p.nb[2] + t[2] - 1) / t[2]);
        };
        int best[3];
        pick(kTileTargets, best);
        // A grid of fewer tiles than one round of workgroups (four per CU) runs as a single
        // wave of tiles, whose time is one tile's: there, tiles of at most three waves of
        // targets run faster (measured at 100k atoms: 0.199 vs 0.244 ms per build).
        if (tiles_of(best) < kFewTiles && best[0] * best[1] * best[2] * per_bin > kFewTileTargets) {
            int alt[3];
            pick(kFewTileTargets, alt);
            if (tiles_of(alt) <= 2 * kFewTiles)
                for (int d = 0; d < 3; d++) best[d] = alt[d];
        }
        for (int d = 0; d < 3; d++) p.T[d] = best[d];
    }
    auto region = [&]() {
        return (int64_t)(p.T[0] + 2 * p.P[0]) * (p.T[1] + 2 * p.P[1]) * (p.T[2] + 2 * p.P[2]);
    };
    p.brute = region() > kMaxRegion;
    for (int d = 0; d < 3; d++) {
        p.R[d] = p.T[d] + 2 * p.P[d];
        p.ntl[d] = (p.nb[d] + p.T[d] - 1) / p.T[d];
        int b = 0;
        while ((1 << b) < p.ntl[d]) b++;
        p.mb[d] = b;
    }
    p.nregion = p.brute ? 0 : (int)region();  // (the all-pairs path has no region table)
    p.tb = p.T[0] * p.T[1] * p.T[2];
    p.ntiles = (int64_t)p.ntl[0] * p.ntl[1] * p.ntl[2];
    p.nbins = p.ntiles * p.tb;
    p.ncodes = (int64_t)1 << (p.mb[0] + p.mb[1] + p.mb[2]);

    // fp32 prefilter band.  Positions in LDS are fp32 offsets from the tile centre: q =
    // fl(rel + o), rel = (position - bin origin) rounded once, o = (bin origin - tile
    // centre) rounded once; the same for the target t.  Every such offset lies in the box
    // of +-m_d = T_d / 2 + P_d bins along the lattice vectors around the centre, whose
    // largest norm (at a corner) is rmax.  Per component the fp32 difference fl(q - t)
    // then differs from the exact canonical vector by at most
    //   u (|rel_q| + |o_q| + |q| + |rel_t| + |o_t| + |t| + |q - t|)
    //     <= u (2 bin_diag + 4 rmax + rr);
    // delta takes twice that.
    const double u = 1.0 / 16777216.0;  // 2^-24
    double len[3], bin_diag = 0;
    for (int d = 0; d < 3; d++) {
        len[d] = sqrt(p.C[3 * d] * p.C[3 * d] + p.C[3 * d + 1] * p.C[3 * d + 1] +
                      p.C[3 * d + 2] * p.C[3 * d + 2]);
        bin_diag += len[d] / p.nb[d];
    }
    double rmax2 = 0;
    for (int sx = -1; sx <= 1; sx += 2)
        for (int sy = -1; sy <= 1; sy += 2)
            for (int sz = -1; sz <= 1; sz += 2) {
                const int sg[3] = {sx, sy, sz};
                double x[3] = {0, 0, 0};
                for (int d = 0; d < 3; d++) {
                    const double m = 0.5 * p.T[d] + p.P[d];
                    for (int c = 0; c < 3; c++) x[c] += sg[d] * m * p.C[3 * d + c] / p.nb[d];
                }
                rmax2 = std::max(rmax2, x[0] * x[0] + x[1] * x[1] + x[2] * x[2]);
            }
    const double rmax = sqrt(rmax2);
    double delta = 2.0 * u * (2.0 * bin_diag + 4.0 * rmax + p.r + 1.0);
    double rr = p.r + 2.0 * delta;
    double band = 2.0 * (2.0 * sqrt(3.0) * rr * delta + 3.0 * delta * delta + 4.0 * u * rr * rr);
    p.hi = nextafterf((float)(p.r2 + band), INFINITY);
    double lo = p.r2 - band;
    p.lo_in = lo > 0 ? nextafterf((float)lo, 0.0f) : 0.0f;
    double t = sqrt(kSelfThr) + 2.0 * sqrt(3.0) * delta;
    p.tiny = nextafterf((float)(t * t * (1.0 + 1e-3)), INFINITY);
    // The kernels evaluate d2' = fl(dz² + (dy² + (dx² - toff))), the offset folded into the
    // innermost fma: three roundings as for d2, so d2' is within the same band of the
    // exact d2 - toff.  A candidate is an edge without the exact test iff 0 <= d2' <
    // lo_off: one unsigned compare of the bits (a negative d2' has its sign bit set).
    // d2' >= 0 gives d2 >= toff (1 - 6u) > tiny's square-root bound, as d2 > tiny did; the
    // fast upper end and the band end move down by toff, rounded inwards (lo) and
    // outwards (hi), one more fp32 step each.
    p.toff = nextafterf(p.tiny, INFINITY);
    const double lo2 = (double)p.lo_in - (double)p.toff;
    float lo_off = 0.0f;
    if (lo2 > 0) {
        lo_off = (float)lo2;
        if ((double)lo_off > lo2) lo_off = nextafterf(lo_off, 0.0f);
        lo_off = nextafterf(lo_off, 0.0f);
    }
    memcpy(&p.lo_bits, &lo_off, 4);
    const double hi2 = (double)p.hi - (double)p.toff;
    p.hi_off = (float)hi2;
    if ((double)p.hi_off < hi2) p.hi_off = nextafterf(p.hi_off, INFINITY);
    p.hi_off = nextafterf(p.hi_off, INFINITY);

    // Neighbour slot per target: the expected degree at the mean density with ample
    // headroom (targets past it are swept a second time in the write pass).
    const double vol = fabs(p.C[0] * (p.C[4] * p.C[8] - p.C[5] * p.C[7]) -
                            p.C[1] * (p.C[3] * p.C[8] - p.C[5] * p.C[6]) +
                            p.C[2] * (p.C[3] * p.C[7] - p.C[4] * p.C[6]));
    const double deg = (double)p.n / vol * (4.0 / 3.0) * 3.14159265358979 * p.r * p.r * p.r;
    // (1.5x + 48: the headroom also covers a density up to about twice the mean in part
    // of the cell, as in a two-phase slab; unused groups of a slot are never touched)
    double k = 1.5 * deg + 48.0;
    k = std::min(std::max(k, 32.0), 2048.0);
    p.K = ((int)k + 7) & ~7;
}

inline void plan_layout(Plan& p)
{
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t r = o; o = align_up(o + (bytes ? bytes : 1)); return r; };
    const size_t n = (size_t)p.n, nt = (size_t)p.nt, nbins = (size_t)p.nbins;
    const size_t ntl = (size_t)p.ntiles;
    // the build's totals: [0] edges, [1] status flags, [2] explicit targets that are not
    // 0 .. nt - 1, [3] some tile needs the fix-up pass; cleared at the start of a build
    p.o_tot = take(8 * 8);
    p.o_key = take(4 * n);
    p.o_rank = take(4 * n);
    p.o_rec = take(16 * n);
    // key, rank and rec serve the count stage's sort only; the write stage reuses their
    // 24 bytes per atom (or more) for the positions in cell-list order
    p.o_cpos = p.o_key;
    p.o_bcnt = take(4 * nbins);
    p.o_bstart = take(4 * (nbins + 1));
    p.o_sid = take(4 * n);
    p.o_spos = take(16 * n);
    p.o_sflr = take(4 * n);
    p.o_inv = take(p.subset ? 4 * n : 0);
    p.o_arr = take(8 * n);
    p.o_tcnt = take(4 * ntl);
    p.o_tstart = take(4 * (ntl + 1));
    p.o_wgb = take(4 * (size_t)kSortChunks * ntl);
    p.o_tor = take(4 * ntl);
    p.o_rot = take(4 * ntl);
    p.o_tkey = take(p.subset ? 4 * nt : 0);
    p.o_trank = take(p.subset ? 4 * nt : 0);
    p.o_tbcnt = take(p.subset ? 4 * nbins : 0);
    p.o_tbstart = take(p.subset ? 4 * (nbins + 1) : 0);
    p.o_tslot = take(p.subset ? 4 * nt : 0);
    p.o_tarr = take(p.subset ? 8 * nt : 0);
    p.o_tsidx = take(p.subset ? 4 * nt : 0);
    p.o_tcaller = take(p.subset ? 4 * nt : 0);
    // scratch of the segment sort (tile buckets, bins of the per-bin sort): one entry per
    // atom or target
    p.o_stmp = take(8 * std::max(n, nt));
    // per-target counts and slots: one row per target, or per atom when explicit targets
    // turn out to be the atoms 0 .. nt - 1 (the count then runs over every atom of a tile)
    // (rows padded to 256 targets: the group rows of a row length of 2 mod 4 targets, e.g.
    // C5's 4,436,018 atoms, made the expansion 5 % slower, 3.02 against 2.87 ms)
    const size_t nrow = (std::max(n, nt) + 255) / 256 * 256;
    p.nrow = (int64_t)nrow;
    p.o_cnt = take(4 * nrow);
    p.o_slot = take(2 * (size_t)p.K * nrow);
    p.o_ttot = take(4 * std::max(ntl, nt));
    p.o_tfix = take(4 * ntl);
    p.o_tbase = take(8 * (std::max(ntl, nt) + 1));
    // scan partials: one int64 per 2048-item block of the largest scan
    size_t big = std::max(nbins + 1, std::max(ntl, nt) + 1);
    p.o_part = take(8 * (big / 2048 + 2));
    p.ws_bytes = o;
}

}  // namespace dg
