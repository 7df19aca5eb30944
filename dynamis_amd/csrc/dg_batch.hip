// dg_batch.hip -- the radius graphs of a batch of small structures in one launch sequence.
//
// radius_graph_pbc_cuda (radius_graph_pbc_cuda.py:64-110) builds a batch image by image:
// one full build, and one host synchronisation, per structure.  For the small structures
// of a training batch (tens to a few hundred atoms each) every one of those builds is
// launch-bound.  Here one wave per atom of the whole batch tests every atom of its own
// structure (64 lanes at a time) over the periodic images of that structure's cell, with the canonical fp64
// predicate and shift convention of the single-structure build (an edge's shift is its
// image plus the floor difference of its two atoms, radius_graph_kernels.cu:282-303): a
// count pass, one scan over the batch, a write pass.  Edges come grouped by target, the
// structures in batch order and the targets of a structure in index order.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <string>

#include "../../include/dynamis_graph.h"
#include "dg_common.hpp"
#include "dg_scan.hpp"

namespace dg {
dg_status fail(dg_status st, const std::string& msg);  // dg_graph.hip
}

namespace {

using namespace dg;

inline size_t al(size_t x) { return (x + 255) & ~(size_t)255; }
inline unsigned nblk(int64_t n, int b = 256) { return (unsigned)((n + b - 1) / b); }

// Per structure, set up on the device from its cell: the cell and its inverse, the
// fractional reach of the cutoff per axis (which bounds each pair's periodic images), and
// the structure's atom range.
struct Image {
    double C[9], Cinv[9];
    double cf[3];  // r / face distance: the fractional reach of the cutoff sphere per axis
    int ok;
    int64_t off, n;
};

struct Layout {
    size_t o_tot, o_img, o_off, o_cnt, o_offs, o_part, total;
};

Layout layout(int64_t B, int64_t N)
{
    Layout L;
    size_t o = 0;
    auto take = [&](size_t b) { size_t r = o; o = al(o + (b ? b : 1)); return r; };
    L.o_tot = take(8 * 8);
    L.o_img = take(sizeof(Image) * (size_t)B);
    L.o_off = take(8 * (size_t)(B + 1));
    L.o_cnt = take(4 * (size_t)N);
    L.o_offs = take(8 * (size_t)std::max<int64_t>(N + 1, 8));
    const size_t big = (size_t)std::max<int64_t>(N, B) + 1;
    L.o_part = take(8 * (big / kScanTile + 2));
    L.total = o;
    return L;
}

struct Args {
    const Image* img;
    const int64_t* off;  // [B + 1] first atom of every structure, off[B] = N
    int64_t B, N;
    const void* pos;
    int f64;
    int pbc[3];
    double r2;
    int* cnt;
    int32_t* counts_user;
    const int64_t* offs;  // [N + 1] first edge of every target
    int64_t* out_src;
    int64_t* out_dst;
    float* out_shift;
    int64_t capacity;
    int64_t* totals;
};

__device__ __forceinline__ void load_pos(const void* pos, int f64, int64_t i, double* p)
{
    if (f64) {
        const double* q = (const double*)pos + 3 * i;
        p[0] = q[0]; p[1] = q[1]; p[2] = q[2];
    } else {
        const float* q = (const float*)pos + 3 * i;
        p[0] = q[0]; p[1] = q[1]; p[2] = q[2];
    }
}

__global__ void clear_kernel(int64_t* totals)
{
    if (threadIdx.x < 8) totals[threadIdx.x] = 0;
}

// One thread per structure: the cell's inverse and face distances (the geometry of the
// single-structure plan), its image range, and its atoms' range (off: exclusive scan of the
// atom counts, done before).
__global__ void setup_kernel(int64_t B, int64_t N, const double* __restrict__ cells,
                             const int64_t* __restrict__ natoms, const int64_t* __restrict__ off, int pbc0,
                             int pbc1, int pbc2, double r, Image* __restrict__ img, int64_t* __restrict__ totals)
{
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    if (b == B - 1 && off[B] != N)  // the atom counts must add up to the atoms given
        atomicOr((unsigned long long*)&totals[1], (unsigned long long)kStatusRange);
    Image m;
    const double* a0 = cells + 9 * b;
    const double *a1 = a0 + 3, *a2 = a0 + 6;
    const double c12[3] = {a1[1] * a2[2] - a1[2] * a2[1], a1[2] * a2[0] - a1[0] * a2[2], a1[0] * a2[1] - a1[1] * a2[0]};
    const double c20[3] = {a2[1] * a0[2] - a2[2] * a0[1], a2[2] * a0[0] - a2[0] * a0[2], a2[0] * a0[1] - a2[1] * a0[0]};
    const double c01[3] = {a0[1] * a1[2] - a0[2] * a1[1], a0[2] * a1[0] - a0[0] * a1[2], a0[0] * a1[1] - a0[1] * a1[0]};
    const double vol = a0[0] * c12[0] + a0[1] * c12[1] + a0[2] * c12[2];
    const double* cs[3] = {c12, c20, c01};
    const int pbc[3] = {pbc0, pbc1, pbc2};
    m.ok = fabs(vol) > 0.0 && isfinite(vol);
    for (int k = 0; k < 9; ++k) m.C[k] = a0[k];
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j) m.Cinv[i * 3 + j] = m.ok ? cs[j][i] / vol : 0.0;
    for (int d = 0; d < 3; ++d) {
        const double nrm = sqrt(cs[d][0] * cs[d][0] + cs[d][1] * cs[d][1] + cs[d][2] * cs[d][2]);
        m.cf[d] = m.ok && pbc[d] ? r / (fabs(vol) / nrm) : 0.0;
    }
    m.off = off[b];
    m.n = natoms[b];
    // a cell far thinner than the radius is refused, as by the single-structure plan
    if (m.ok && !(pair_images(m.cf, pbc) <= kMaxPairImages)) m.ok = 0;
    if (!m.ok || m.n < 0) atomicOr((unsigned long long*)&totals[1], (unsigned long long)kStatusRange);
    img[b] = m;
}

__global__ void atom_offsets_kernel(int64_t B, const int64_t* __restrict__ natoms, int64_t* __restrict__ off)
{
    // (B <= a few thousand structures: one workgroup scans them)
    __shared__ int64_t s_w[1024 / 64];
    int64_t carry = 0;
    for (int64_t b0 = 0; b0 <= B; b0 += 1024) {
        const int64_t b = b0 + threadIdx.x;
        const int64_t v = b < B ? natoms[b] : 0;
        int64_t tot;
        const int64_t ex = block_excl_scan<int64_t, 1024>(v, s_w, &tot);
        if (b <= B) off[b] = carry + ex;
        carry += tot;
    }
}

// The shifts S an edge (source at ps, target at fractional frt) can have: on an axis without
// PBC the floor difference (image 0); on a periodic one, every S with |frt - frs - S| <= cf
// (the distance between the source image and the target is at least that fractional
// distance times the face distance), widened by 1e-9 against rounding.
__device__ __forceinline__ void shift_range(const int* pbc, const double* cf, const double* frt,
                                            const double* ps, const double* Cinv, int* lo, int* hi)
{
    for (int d = 0; d < 3; ++d) {
        const double frs = canon_frac(ps[0], ps[1], ps[2], Cinv, d);
        if (pbc[d]) {
            const double x = frt[d] - frs;
            lo[d] = (int)ceil(x - cf[d] - 1e-9);
            hi[d] = (int)floor(x + cf[d] + 1e-9);
        } else {
            lo[d] = hi[d] = (int)floor(frt[d]) - (int)floor(frs);
        }
    }
}

// The structure of atom t: the last b with off[b] <= t (off is nondecreasing).
__device__ __forceinline__ int64_t image_of(const int64_t* off, int64_t B, int64_t t)
{
    int64_t lo = 0, hi = B;  // off[lo] <= t < off[hi]
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (off[mid] <= t) lo = mid; else hi = mid;
    }
    return lo;
}

// One wave per atom t of the batch (the target): its lanes take the sources of t's structure
// 64 at a time, each lane every periodic image of its source that can hold an edge.  The
// count pass adds up the lanes' edges; the write pass places each lane's edges after those
// of the lanes before it (a wave scan per group of 64 sources), so edges come in source
// order and, for one source, in image order (s0, s1, s2 ascending, nested).
template <bool WRITE>
__global__ __launch_bounds__(256) void batch_kernel(Args a)
{
    const int64_t t = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;  // one wave per target
    const int lane = threadIdx.x & 63;
    if (t >= a.N) return;
    const Image& m = a.img[image_of(a.off, a.B, t)];
    double pt[3];
    load_pos(a.pos, a.f64, t, pt);
    const bool finite_t = isfinite(pt[0]) && isfinite(pt[1]) && isfinite(pt[2]);
    const bool good = m.ok && finite_t;
    if (!WRITE && !finite_t && lane == 0)
        atomicOr((unsigned long long*)&a.totals[1], (unsigned long long)kStatusNonFinite);
    int64_t o = 0;
    if (WRITE) {
        o = a.offs[t];
        if (a.offs[t + 1] > a.capacity) {
            if (lane == 0) atomicOr((unsigned long long*)&a.totals[1], (unsigned long long)kStatusCapacity);
            return;
        }
    }
    int found = 0;  // this lane's edges (count pass); edges of the wave so far (write pass)
    if (good) {
        double frt[3];
        for (int d = 0; d < 3; ++d) frt[d] = canon_frac(pt[0], pt[1], pt[2], m.Cinv, d);
        // (clamped to the batch: atom counts that do not add up are flagged by setup_kernel)
        const int64_t jb = max(m.off, (int64_t)0), je = min(m.off + m.n, a.N);
        for (int64_t j0 = jb; j0 < je; j0 += 64) {
            const int64_t j = j0 + lane;
            double ps[3];
            int lo[3] = {0, 0, 0}, hi[3] = {-1, -1, -1};  // (no images for an idle lane)
            if (j < je) {
                load_pos(a.pos, a.f64, j, ps);
                if (isfinite(ps[0]) && isfinite(ps[1]) && isfinite(ps[2]))
                    shift_range(a.pbc, m.cf, frt, ps, m.Cinv, lo, hi);
            }
            auto each_edge = [&](auto&& f) {
                for (int s0 = lo[0]; s0 <= hi[0]; ++s0)
                    for (int s1 = lo[1]; s1 <= hi[1]; ++s1)
                        for (int s2 = lo[2]; s2 <= hi[2]; ++s2) {
                            double v[3];
                            const double d2 = canon_d2(ps, pt, s0, s1, s2, m.C, v);
                            if (d2 > kSelfThr && d2 <= a.r2) f(s0, s1, s2);
                        }
            };
            int mine = 0;
            each_edge([&](int, int, int) { ++mine; });
            if (!WRITE) {
                found += mine;
            } else {
                const int incl = wave_incl_scan<int>(mine);
                int64_t e = o + found + (incl - mine);
                each_edge([&](int s0, int s1, int s2) {
                    a.out_src[e] = j;
                    a.out_dst[e] = t;
                    a.out_shift[3 * e] = (float)s0;
                    a.out_shift[3 * e + 1] = (float)s1;
                    a.out_shift[3 * e + 2] = (float)s2;
                    ++e;
                });
                found += __shfl(incl, 63, 64);
            }
        }
    }
    if (!WRITE) {
        // the wave's total
        for (int sh = 32; sh > 0; sh >>= 1) found += __shfl_xor(found, sh, 64);
        if (lane == 0) {
            a.cnt[t] = found;
            if (a.counts_user) a.counts_user[t] = found;
        }
    }
}

__global__ void per_image_kernel(int64_t B, int64_t N, const int64_t* __restrict__ off,
                                 const int64_t* __restrict__ offs, int64_t* __restrict__ out)
{
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    // (atom counts that do not add up, flagged by setup_kernel, must not index past offs)
    if (b < B) out[b] = offs[min(max(off[b + 1], (int64_t)0), N)] - offs[min(max(off[b], (int64_t)0), N)];
}

dg_status check(const dg_batch_desc* d)
{
    if (!d) return fail(DG_ERR_INVALID, "desc is NULL");
    if (d->n_images < 1 || d->n_images > (1 << 20))
        return fail(DG_ERR_INVALID, "n_images must be in [1, 2^20]");
    if (d->n_atoms < 0 || d->n_atoms > 0x7ffffff0LL) return fail(DG_ERR_INVALID, "n_atoms must be in [0, 2^31)");
    if (d->pos_dtype != DG_F32 && d->pos_dtype != DG_F64) return fail(DG_ERR_INVALID, "pos must be float32 or float64");
    if (!(d->radius > 0.0) || !isfinite(d->radius))
        return fail(DG_ERR_INVALID, "radius must be positive, got " + std::to_string(d->radius));
    return DG_OK;
}

Args make_args(const dg_batch_desc* d, const Layout& L, const void* pos, void* ws)
{
    char* w = (char*)ws;
    Args a;
    memset(&a, 0, sizeof a);
    a.img = (const Image*)(w + L.o_img);
    a.off = (const int64_t*)(w + L.o_off);
    a.B = d->n_images;
    a.N = d->n_atoms;
    a.pos = pos;
    a.f64 = d->pos_dtype == DG_F64;
    for (int k = 0; k < 3; ++k) a.pbc[k] = d->pbc[k] ? 1 : 0;
    a.r2 = d->radius * d->radius;
    a.cnt = (int*)(w + L.o_cnt);
    a.offs = (const int64_t*)(w + L.o_offs);
    a.totals = (int64_t*)(w + L.o_tot);
    return a;
}

dg_status launched(const char* what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(DG_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
    return DG_OK;
}

}  // namespace

extern "C" {

size_t dg_batch_workspace_size(const dg_batch_desc* desc)
{
    if (check(desc) != DG_OK) return 0;
    return layout(desc->n_images, desc->n_atoms).total;
}

dg_status dg_batch_count(const dg_batch_desc* desc, const void* pos, const int64_t* natoms,
                         const double* cells, int32_t* counts_out, void* ws, size_t ws_bytes,
                         hipStream_t s)
{
    dg_status st = check(desc);
    if (st != DG_OK) return st;
    const Layout L = layout(desc->n_images, desc->n_atoms);
    if (!ws || ws_bytes < L.total) return fail(DG_ERR_WORKSPACE, "workspace too small");
    if (!natoms || !cells || (desc->n_atoms > 0 && !pos)) return fail(DG_ERR_INVALID, "inputs are NULL");
    Args a = make_args(desc, L, pos, ws);
    a.counts_user = counts_out;
    char* w = (char*)ws;
    int64_t* off = (int64_t*)(w + L.o_off);
    hipLaunchKernelGGL(clear_kernel, dim3(1), dim3(64), 0, s, a.totals);
    hipLaunchKernelGGL(atom_offsets_kernel, dim3(1), dim3(1024), 0, s, desc->n_images, natoms, off);
    hipLaunchKernelGGL(setup_kernel, dim3(nblk(desc->n_images)), dim3(256), 0, s, desc->n_images, desc->n_atoms,
                       cells, natoms,
                       (const int64_t*)off, (int)a.pbc[0], (int)a.pbc[1], (int)a.pbc[2], desc->radius,
                       (Image*)(w + L.o_img), a.totals);
    if (desc->n_atoms > 0) {
        hipLaunchKernelGGL(batch_kernel<false>, dim3(nblk(64 * desc->n_atoms)), dim3(256), 0, s, a);
        excl_scan<int, int64_t>(a.cnt, desc->n_atoms, (int64_t*)(w + L.o_offs), (int64_t*)(w + L.o_part), s,
                                a.totals);
    } else {
        hipLaunchKernelGGL(clear_kernel, dim3(1), dim3(64), 0, s, (int64_t*)(w + L.o_offs));  // offs[0] = 0
    }
    return launched("dg_batch_count");
}

dg_status dg_batch_read_totals(const dg_batch_desc* desc, const void* ws, int64_t* total_edges,
                               int64_t* flags, hipStream_t s)
{
    dg_status st = check(desc);
    if (st != DG_OK) return st;
    int64_t h[2] = {0, 0};
    hipError_t e = hipMemcpyAsync(h, ws, sizeof h, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail(DG_ERR_HIP, std::string("dg_batch_read_totals: ") + hipGetErrorString(e));
    if (total_edges) *total_edges = h[0];
    if (flags) *flags = h[1];
    if (h[1] & kStatusNonFinite) return fail(DG_ERR_RANGE, "pos contains non-finite values");
    if (h[1] & kStatusRange)
        return fail(DG_ERR_INVALID, "a cell is singular or too thin for the radius (more than 2^24 periodic "
                                    "images per atom pair), or the atom counts are negative or do not add "
                                    "up to n_atoms");
    if (h[1] & kStatusCapacity) return fail(DG_ERR_CAPACITY, "edge capacity exceeded");
    return DG_OK;
}

dg_status dg_batch_write(const dg_batch_desc* desc, const void* pos, void* ws, size_t ws_bytes,
                         int64_t capacity, int64_t* edge_src, int64_t* edge_dst, float* cell_shift,
                         int64_t* edges_per_image, hipStream_t s)
{
    dg_status st = check(desc);
    if (st != DG_OK) return st;
    const Layout L = layout(desc->n_images, desc->n_atoms);
    if (!ws || ws_bytes < L.total) return fail(DG_ERR_WORKSPACE, "workspace too small");
    if (capacity < 0) return fail(DG_ERR_INVALID, "capacity < 0");
    Args a = make_args(desc, L, pos, ws);
    a.out_src = edge_src;
    a.out_dst = edge_dst;
    a.out_shift = cell_shift;
    a.capacity = capacity;
    if (desc->n_atoms > 0 && capacity > 0) {
        if (!edge_src || !edge_dst || !cell_shift) return fail(DG_ERR_INVALID, "edge outputs are NULL");
        hipLaunchKernelGGL(batch_kernel<true>, dim3(nblk(64 * desc->n_atoms)), dim3(256), 0, s, a);
    }
    if (edges_per_image) {
        char* w = (char*)ws;
        hipLaunchKernelGGL(per_image_kernel, dim3(nblk(desc->n_images)), dim3(256), 0, s, desc->n_images,
                           desc->n_atoms, (const int64_t*)(w + L.o_off), (const int64_t*)(w + L.o_offs),
                           edges_per_image);
    }
    return launched("dg_batch_write");
}

}  // extern "C"
