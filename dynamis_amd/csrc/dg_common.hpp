// dg_common.hpp -- shared host/device helpers for the gfx950 neighbour-graph build.
//
// Canonical arithmetic (the build's contract, evaluated identically on the host and on
// the GPU; every file that includes this header is compiled with -ffp-contract=off):
//   frac_j = fma(p2, Cinv[2][j], fma(p1, Cinv[1][j], p0 * Cinv[0][j]))
//   v_a    = (p_src,a - p_tgt,a) + fma(S2, C[2][a], fma(S1, C[1][a], S0 * C[0][a]))
//   d2     = fma(v2, v2, fma(v1, v1, v0 * v0));   edge iff 1e-8f < d2 <= r^2
// The reference evaluates the same predicate in fp32 on wrapped coordinates
// (dynamis_state/src/csrc/graph/radius_graph_kernels.cu:247-250, 399-400) and the
// output shift as image_shift + floor(frac_tgt) - floor(frac_src) (:282-303); the integer
// shift S here is that same quantity.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define DG_HD __host__ __device__ __forceinline__

namespace dg {

constexpr double kSelfThr = (double)1e-8f;  // radius_graph_kernels.cu:250 (1e-8f)
constexpr int kFloorBias = 512;             // packed 10-bit signed fields
constexpr int kFloorMax = 255;              // |floor(frac)| accepted per axis

// status bits written by kernels
constexpr int kStatusRange = 1;     // an atom lies more than kFloorMax cells outside
constexpr int kStatusNonFinite = 2; // NaN / inf position
constexpr int kStatusCapacity = 4;  // edge output capacity exceeded

// Periodic images that one atom pair may have within the cutoff, at most: a cell far
// thinner than the radius is refused (the all-pairs kernels loop over these images per pair;
// the reference materialises n (2 ceil(cf) + 1)^3 image atoms for it and runs out of memory).
constexpr double kMaxPairImages = 16777216.0;  // 2^24

// Upper bound on the images per atom pair: every shift S with |x - S| <= cf on a periodic
// axis (cf = r / face distance), one on the others.
DG_HD double pair_images(const double* cf, const int* pbc)
{
    double m = 1.0;
    for (int d = 0; d < 3; ++d) m *= pbc[d] ? 2.0 * cf[d] + 1.0 : 1.0;
    return m;
}

DG_HD double canon_frac(double p0, double p1, double p2, const double* Cinv, int j)
{
    return fma(p2, Cinv[6 + j], fma(p1, Cinv[3 + j], p0 * Cinv[j]));
}

DG_HD double canon_shift(int S0, int S1, int S2, const double* C, int a)
{
    return fma((double)S2, C[6 + a], fma((double)S1, C[3 + a], (double)S0 * C[a]));
}

// Returns d2; writes v.
DG_HD double canon_d2(const double* ps, const double* pt, int S0, int S1, int S2, const double* C,
                      double* v)
{
    v[0] = (ps[0] - pt[0]) + canon_shift(S0, S1, S2, C, 0);
    v[1] = (ps[1] - pt[1]) + canon_shift(S0, S1, S2, C, 1);
    v[2] = (ps[2] - pt[2]) + canon_shift(S0, S1, S2, C, 2);
    return fma(v[2], v[2], fma(v[1], v[1], v[0] * v[0]));
}

DG_HD uint32_t pack3(int x, int y, int z)
{
    return (uint32_t)(x + kFloorBias) | ((uint32_t)(y + kFloorBias) << 10) |
           ((uint32_t)(z + kFloorBias) << 20);
}
DG_HD int unpack3(uint32_t w, int d) { return (int)((w >> (10 * d)) & 1023u) - kFloorBias; }

DG_HD int floor_div(int a, int b) { return a >= 0 ? a / b : -((-a + b - 1) / b); }

// Compact Morton code over tile coordinates: bit level k interleaves x, y, z (x lowest,
// as in partition/sfc_kernels.cu:19-56) but only for axes that still have bits at level k,
// so anisotropic grids do not waste code space.
DG_HD uint32_t morton_encode(int x, int y, int z, const int* mb)
{
    uint32_t code = 0;
    int pos = 0;
    int top = mb[0] > mb[1] ? mb[0] : mb[1];
    top = top > mb[2] ? top : mb[2];
    for (int k = 0; k < top; ++k) {
        if (k < mb[0]) code |= (uint32_t)((x >> k) & 1) << pos++;
        if (k < mb[1]) code |= (uint32_t)((y >> k) & 1) << pos++;
        if (k < mb[2]) code |= (uint32_t)((z >> k) & 1) << pos++;
    }
    return code;
}
DG_HD void morton_decode(uint32_t code, const int* mb, int* x, int* y, int* z)
{
    int pos = 0, c[3] = {0, 0, 0};
    int top = mb[0] > mb[1] ? mb[0] : mb[1];
    top = top > mb[2] ? top : mb[2];
    for (int k = 0; k < top; ++k)
        for (int d = 0; d < 3; ++d)
            if (k < mb[d]) c[d] |= (int)((code >> pos++) & 1u) << k;
    *x = c[0]; *y = c[1]; *z = c[2];
}

}  // namespace dg
