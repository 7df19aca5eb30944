// dg_graph.hip -- PBC radius-graph build for gfx950 (MI355X), C ABI in
// include/dynamis_graph.h.
//
// Pipeline of one build (all on the caller's stream, one host sync in the Python layer
// to size the outputs, none inside this file):
//   1. tile_flags / tile_fill      Morton (SFC) rank of every 4x4x4 tile of bins
//   2. bin_atoms                   fractional coords -> floor (wrap), bin, SFC key, and
//                                  an atomic slot inside the key's bin
//   3. scan                        bin starts (counting sort == single-digit radix sort)
//   4. scatter_atoms               atom id -> sorted slot
//   5. finish_bins                 stable order inside each bin, then the SoA cell list
//                                  (fp32 position relative to the bin origin + id,
//                                  packed floor) in SFC order
//   6. search<false>               per-target degree (one workgroup per tile, region of
//                                  (T+2P)^3 bins staged in LDS, one lane per target)
//   7. scan                        per-tile edge offsets in SFC tile order
//   8. search<true>                edges: lanes stage (src, shift) records in LDS, the
//                                  workgroup then streams them out with coalesced stores
//
// Reference stages replaced (dynamis_state/src/csrc/graph/radius_graph_kernels.cu):
// wrap :596-605, selective images :18-141 (here: periodic bin wrap, no image atoms),
// grid + sort :146-194,662-714, target sort :731-769, count :197-258, write :320-442,
// outputs :925-933.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "../../include/dynamis_graph.h"
#include "dg_common.hpp"
#include "dg_plan.hpp"
#include "dg_scan.hpp"
#include "dg_segsort.hpp"

// The count kernel (search_kernel<0>) is compiled in a translation unit of its own,
// dg_count.hip, which includes this file with DG_COUNT_TU defined: there, only the
// device code the count kernel needs and its launcher are compiled (under another
// instruction-scheduling strategy, see build.py), and everything else is left out.
#ifdef DG_COUNT_TU
#define DG_MAIN_TU 0
#else
#define DG_MAIN_TU 1
#endif

namespace dg {

#if DG_MAIN_TU
thread_local std::string g_last_error;

dg_status fail(dg_status st, const std::string& msg)
{
    g_last_error = msg;
    return st;
}
#endif

constexpr int kRegPerThread = (kMaxRegion + kBlock - 1) / kBlock;
constexpr int kBinSortMax = 128;
constexpr int kExpandIlp = 4;  // 64-edge steps per iteration of the expansion (even)

// Whether a device-wide flag word still reads 0 (a device-scope load, so a flag another
// XCD set is seen): raising flags only then keeps the atomics on one address few.
__device__ __forceinline__ bool flag_clear(int64_t* w)
{
    return __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0;
}

// search_kernel<1> work of a tile, set by the count pass
constexpr int kFixOver = 1;     // a target has more than K neighbours
constexpr int kFixChunked = 2;  // the region needs more than two LDS chunks (or no slots)
constexpr int kFix2 = 4;        // the region needs two LDS chunks (slots hold both)
#ifndef DG_FIXGRID
#define DG_FIXGRID 512
#endif
constexpr int64_t kFixGrid = DG_FIXGRID;  // workgroups of the fix-up pass (it loops over the tiles)

// Value known to be uniform across the wave, moved to a scalar register.
__device__ __forceinline__ int rfl(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ uint32_t rfl(uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); }

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

struct GridArgs {
    double C[9], Cinv[9];
    int nb[3], T[3], ntl[3], mb[3];
    int tb;
};

// Offset of a cell-list record along the cell's a axis inside its bin, as a Cartesian x
// length (lower-triangular cells): x less the b and c shears of its y and z offsets, so the
// key is fa * hax for the record's fraction fa of the bin along a.  The tile sort orders
// bins by it and the count pass counts quarter-bin prefixes of it: both evaluate it with
// these explicit operations on the same inputs, so the counts are prefixes of the order.
struct XKey {
    float hbx, hcx, hcy, inv_hby, inv_hcz;
};
__device__ __forceinline__ float bin_xkey(const float4& e, const XKey& k)
{
    const float fc = e.z * k.inv_hcz;
    const float fb = fmaf(-fc, k.hcy, e.y) * k.inv_hby;
    return fmaf(-fc, k.hcx, fmaf(-fb, k.hbx, e.x));
}

#if DG_MAIN_TU
// ---------------------------------------------------------------- tile SFC ranks
// Rank of every tile in the compact Morton order (morton_encode) among the tiles of the
// grid, computed directly: for each 1 bit of the tile's code, the tiles whose codes share
// the bits above it and have a 0 there all come first; per axis, their coordinate has its
// high bits fixed and f free low bits, so the axis admits clamp(n - lo, 0, 2^f) values.
// Also clears the bin counts (bcnt) for the binning that follows.
__global__ void tile_rank_kernel(GridArgs g, int64_t ntiles, int* __restrict__ tile_of_rank,
                                 int* __restrict__ rank_of_tile, int* __restrict__ bcnt,
                                 int64_t nbins, int64_t* __restrict__ totals)
{
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    if (blockIdx.x == 0 && threadIdx.x < 8) totals[threadIdx.x] = 0;  // the build's totals and flags
    for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < nbins; q += stride) bcnt[q] = 0;
    for (int64_t lin = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; lin < ntiles; lin += stride) {
        const int X[3] = {(int)(lin % g.ntl[0]), (int)((lin / g.ntl[0]) % g.ntl[1]),
                          (int)(lin / ((int64_t)g.ntl[0] * g.ntl[1]))};
        int f[3] = {0, 0, 0};
        int64_t r = 0;
        const int top = max(max(g.mb[0], g.mb[1]), g.mb[2]);
        for (int k = 0; k < top; ++k) {
            for (int dp = 0; dp < 3; ++dp) {
                if (k >= g.mb[dp]) continue;
                if ((X[dp] >> k) & 1) {
                    int64_t cnt = 1;
#pragma unroll
                    for (int d = 0; d < 3; ++d) {
                        const int lo = d == dp ? (X[d] >> (k + 1)) << (k + 1) : (X[d] >> f[d]) << f[d];
                        cnt *= (int64_t)min(max(g.ntl[d] - lo, 0), 1 << f[d]);
                    }
                    r += cnt;
                }
                ++f[dp];
            }
        }
        tile_of_rank[r] = (int)lin;
        rank_of_tile[lin] = (int)r;
    }
}

// ---------------------------------------------------------------- binning
// Canonical wrap of one atom: floor of the fractional coordinate (all axes, as the
// reference, radius_graph_kernels.cu:603-605), wrapped fraction s in [0,1) and bin b.
__device__ __forceinline__ int wrap_atom(const GridArgs& g, const double* p, int* f, double* s,
                                         int* b)
{
    int st = 0;
    double q[3] = {p[0], p[1], p[2]};
    if (!(isfinite(q[0]) && isfinite(q[1]) && isfinite(q[2]))) {
        st |= kStatusNonFinite;
        q[0] = q[1] = q[2] = 0.0;
    }
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        double fr = canon_frac(q[0], q[1], q[2], g.Cinv, j);
        double fl = floor(fr);
        if (!(fabs(fl) <= (double)kFloorMax)) {
            st |= kStatusRange;
            fl = 0.0;
            fr = 0.0;
        }
        f[j] = (int)fl;
        s[j] = fr - fl;
        int bj = (int)(s[j] * (double)g.nb[j]);
        b[j] = bj < 0 ? 0 : (bj >= g.nb[j] ? g.nb[j] - 1 : bj);
    }
    return st;
}

__device__ __forceinline__ uint32_t bin_key(const GridArgs& g, const int* b,
                                            const int* __restrict__ rank_of_tile)
{
    int t0 = b[0] / g.T[0], t1 = b[1] / g.T[1], t2 = b[2] / g.T[2];
    int l0 = b[0] - t0 * g.T[0], l1 = b[1] - t1 * g.T[1], l2 = b[2] - t2 * g.T[2];
    int lin = t0 + g.ntl[0] * (t1 + g.ntl[1] * t2);
    return (uint32_t)rank_of_tile[lin] * (uint32_t)g.tb + (uint32_t)(l0 + g.T[0] * (l1 + g.T[1] * l2));
}

// Per atom: wrap, bin, SFC key and an atomic slot inside the key's bin; and the atom's
// cell-list record (fp32 position relative to its bin origin, packed floor), which
// finish_bins moves to the atom's sorted place.
__global__ void bin_atoms_kernel(GridArgs g, const void* __restrict__ pos, int f64, int64_t n,
                                 const int* __restrict__ rank_of_tile, uint32_t* __restrict__ key,
                                 uint32_t* __restrict__ rank, int* __restrict__ bcnt,
                                 float4* __restrict__ rec, int64_t* __restrict__ totals)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    double p[3], s[3];
    int f[3], b[3];
    load_pos(pos, f64, i, p);
    int st = wrap_atom(g, p, f, s, b);
    if (st) atomicOr((unsigned long long*)&totals[1], (unsigned long long)st);
    uint32_t k = bin_key(g, b, rank_of_tile);
    key[i] = k;
    if (bcnt) rank[i] = (uint32_t)atomicAdd(&bcnt[k], 1);
    // position relative to the bin origin: (s - b/nb) . C
    double o[3];
#pragma unroll
    for (int d = 0; d < 3; ++d) o[d] = s[d] - (double)b[d] / (double)g.nb[d];
    float4 e;
    e.x = (float)fma(o[2], g.C[6], fma(o[1], g.C[3], o[0] * g.C[0]));
    e.y = (float)fma(o[2], g.C[7], fma(o[1], g.C[4], o[0] * g.C[1]));
    e.z = (float)fma(o[2], g.C[8], fma(o[1], g.C[5], o[0] * g.C[2]));
    e.w = __uint_as_float(pack3(f[0], f[1], f[2]));
    rec[i] = e;
}

__global__ void scatter_atoms_kernel(int64_t n, const uint32_t* __restrict__ key,
                                     const uint32_t* __restrict__ rank,
                                     const int* __restrict__ bstart, int* __restrict__ sid)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    sid[bstart[key[i]] + rank[i]] = (int)i;
}

// Insertion sort of a[lo, hi) ascending (bins hold a handful of entries).
__device__ __forceinline__ void small_sort(int* a, int lo, int hi)
{
    for (int j = lo + 1; j < hi; ++j) {
        int v = a[j];
        int k = j - 1;
        while (k >= lo && a[k] > v) {
            a[k + 1] = a[k];
            --k;
        }
        a[k + 1] = v;
    }
}

// Sorts every segment [start[b], start[b + 1]) of v longer than kBinSortMax (by value,
// ascending; ids < 2^31) in place, tmp its scratch: the bins that order_atoms_kernel and
// finish_targets_kernel leave as they are.  Workgroup g scans its own range of segments,
// 256 at a time, and sorts the long ones of each batch in turn.
__global__ __launch_bounds__(kSegSortThreads) void sort_big_bins_kernel(int64_t nseg, const int* __restrict__ start,
                                                                        uint32_t* __restrict__ v,
                                                                        uint32_t* __restrict__ tmp)
{
    __shared__ SegSortLds L;
    __shared__ int big[kSegSortThreads];
    const int64_t per = (nseg + gridDim.x - 1) / gridDim.x;
    const int64_t b0 = (int64_t)blockIdx.x * per, b1 = min(nseg, b0 + per);
    for (int64_t c = b0; c < b1; c += kSegSortThreads) {
        const int64_t b = c + threadIdx.x;
        big[threadIdx.x] = b < b1 && start[b + 1] - start[b] > kBinSortMax;
        __syncthreads();
        for (int k = 0; k < kSegSortThreads; ++k) {
            if (!big[k]) continue;  // (the same for every thread)
            const int lo = start[c + k], hi = start[c + k + 1];
            segment_sort<uint32_t>(v + lo, tmp + lo, hi - lo, 32, L);
        }
        __syncthreads();
    }
}

// One thread per cell-list entry j (in arrival order inside its bin, from scatter_atoms):
// the entry's place in its bin ordered by atom id (the number of smaller ids in the bin),
// then the SoA cell list.  Bins of more than kBinSortMax atoms were put in id order by
// sort_big_bins_kernel already: there the place is j.
__global__ void order_atoms_kernel(int64_t n, const uint32_t* __restrict__ key,
                                   const int* __restrict__ bstart, const int* __restrict__ arr,
                                   const float4* __restrict__ rec, float4* __restrict__ spos,
                                   uint32_t* __restrict__ sflr, int* __restrict__ sid,
                                   int* __restrict__ inv)
{
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    const int i = arr[j];
    const uint32_t b = key[i];
    const int lo = bstart[b], hi = bstart[b + 1];
    int d = (int)j;
    if (hi - lo > 1 && hi - lo <= kBinSortMax) {
        int below = 0;
        for (int m = lo; m < hi; ++m) below += arr[m] < i;
        d = lo + below;
    }
    const float4 r = rec[i];
    spos[d] = make_float4(r.x, r.y, r.z, __int_as_float(i));
    sflr[d] = __float_as_uint(r.w);
    sid[d] = i;
    if (inv) inv[i] = d;
}

// ---------------------------------------------------------------- tile-level counting sort
// Without per-atom device atomics (about 25 G/s on this part, the dominant cost of a
// per-bin counting sort): kSortChunks workgroups each histogram the tiles of one chunk of
// atoms in LDS and reserve their share of every tile with one device atomic per tile;
// the same chunks then place their atoms into tile buckets; one workgroup per tile then
// orders its bucket by (bin, offset along the a axis in the bin for lower-triangular cells,
// atom id) in LDS and writes the bin starts and the cell list.

// Chunk c of the atoms: [c n / G, (c + 1) n / G).
__device__ __forceinline__ void sort_chunk(int64_t n, int64_t* lo, int64_t* hi)
{
    *lo = n * blockIdx.x / gridDim.x;
    *hi = n * (blockIdx.x + 1) / gridDim.x;
}

__global__ __launch_bounds__(1024) void tile_hist_kernel(int64_t n, int tb, int64_t ntiles,
                                                         const uint32_t* __restrict__ key,
                                                         int* __restrict__ tcnt, int* __restrict__ wgb,
                                                         const int64_t* __restrict__ run_if)
{
    if (run_if && *run_if == 0) return;  // (explicit targets that need no sort)
    extern __shared__ int h[];
    for (int64_t r = threadIdx.x; r < ntiles; r += blockDim.x) h[r] = 0;
    __syncthreads();
    int64_t lo, hi;
    sort_chunk(n, &lo, &hi);
    for (int64_t i = lo + threadIdx.x; i < hi; i += blockDim.x) atomicAdd(&h[key[i] / (uint32_t)tb], 1);
    __syncthreads();
    for (int64_t r = threadIdx.x; r < ntiles; r += blockDim.x) {
        const int c = h[r];
        wgb[blockIdx.x * ntiles + r] = c ? atomicAdd(&tcnt[r], c) : 0;
    }
}

// Places every atom of the chunk in its tile's bucket as (atom id, bin inside the tile);
// the atoms are read in order, the scattered side is the 8-byte stores.
// Each workgroup scans the tile totals itself (workgroup 0 also stores the tile starts,
// with tstart[ntiles] = n, for tile_sort_kernel).
// A tile-bucket entry: an id and the bin inside the tile (< 256).  32 bits (24 + 8) when
// every id fits 24 bits, else 64 (32 + 32).
__device__ __forceinline__ uint32_t bk_pack(uint32_t i, uint32_t l, uint32_t*) { return i | (l << 24); }
__device__ __forceinline__ uint64_t bk_pack(uint32_t i, uint32_t l, uint64_t*) { return (uint64_t)i | ((uint64_t)l << 32); }
__device__ __forceinline__ int bk_id(uint32_t w) { return (int)(w & 0xFFFFFFu); }
__device__ __forceinline__ int bk_id(uint64_t w) { return (int)(uint32_t)w; }
__device__ __forceinline__ int bk_bin(uint32_t w) { return (int)(w >> 24); }
__device__ __forceinline__ int bk_bin(uint64_t w) { return (int)(w >> 32); }

template <typename BT>
__global__ __launch_bounds__(1024) void tile_scatter_kernel(int64_t n, int tb, int64_t ntiles,
                                                            const uint32_t* __restrict__ key,
                                                            const int* __restrict__ tcnt,
                                                            int* __restrict__ tstart,
                                                            const int* __restrict__ wgb,
                                                            BT* __restrict__ bucket,
                                                            const int64_t* __restrict__ run_if)
{
    if (run_if && *run_if == 0) return;  // (explicit targets that need no sort)
    extern __shared__ int h[];  // this chunk's next place in every tile's bucket
    __shared__ int s_w[1024 / 64];
    {
        const int per = (int)((ntiles + 1023) / 1024);
        const int64_t r0 = (int64_t)threadIdx.x * per;
        int loc = 0;
        for (int k = 0; k < per; ++k)
            if (r0 + k < ntiles) loc += tcnt[r0 + k];
        int tot;
        int ex = block_excl_scan<int, 1024>(loc, s_w, &tot);
        for (int k = 0; k < per; ++k) {
            const int64_t r = r0 + k;
            if (r < ntiles) {
                h[r] = ex + wgb[blockIdx.x * ntiles + r];
                if (blockIdx.x == 0) tstart[r] = ex;
                ex += tcnt[r];
            }
        }
        if (blockIdx.x == 0 && threadIdx.x == 0) tstart[ntiles] = tot;
    }
    __syncthreads();
    int64_t lo, hi;
    sort_chunk(n, &lo, &hi);
    // four atoms per thread and step, their loads issued together
    for (int64_t i0 = lo + threadIdx.x; i0 < hi; i0 += 4 * (int64_t)blockDim.x) {
        uint32_t k[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t i = i0 + (int64_t)u * blockDim.x;
            k[u] = i < hi ? key[i] : 0u;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t i = i0 + (int64_t)u * blockDim.x;
            if (i < hi) {
                const uint32_t r = k[u] / (uint32_t)tb;
                const int d = atomicAdd(&h[r], 1);
                bucket[d] = bk_pack((uint32_t)i, k[u] - r * (uint32_t)tb, (BT*)nullptr);
            }
        }
    }
}

constexpr int kTileSortCap = 2048;  // bucket entries ordered in LDS (larger: sorted by segment_sort)
constexpr int kTileSortPer = kTileSortCap / 256;
struct TileSortLds {
    union {
        int by[kTileSortCap];  // ids grouped by bin
        SegSortLds seg;        // a larger bucket: sorted in global memory
    };
    uint32_t bx[kTileSortCap];  // atoms: order key of each grouped entry's x in its bin
    int cnt[kTileMax * kTileMax * kTileMax];
    int st[kTileMax * kTileMax * kTileMax + 1];
    int w32[4];
};

// What tile_sort_kernel writes for one sorted entry.  Atoms (TGT false): the cell-list
// record (position in the bin and id, floor, id, and the inverse map); ids are atom ids.
// Explicit targets (TGT true): ids are caller positions t; the caller position and the
// cell-list index of target t's atom.
struct TileSortOut {
    const float4* rec;  // atoms: records by atom id
    float4* spos;
    uint32_t* sflr;
    int* sid;
    int* inv;           // atoms: written when given; targets: read (atom -> cell-list index)
    const int64_t* tgt; // targets: atom of each caller position
    int64_t natoms;
    int* tslot;
    int* tsidx;
    const int64_t* run_if;  // targets: skipped when *run_if == 0 (they need no sort)
    void* stmp;             // scratch for a bucket of more than kTileSortCap entries (one per entry)
    int64_t* xflag;         // atoms: raised when a bucket's bins are left in id order
    int xorder;             // atoms: order bins by (bin_xkey, id) (else by id)
    XKey xk;
};

// Order key of a float: unsigned compare of the keys is the float order (-0 below +0).
__device__ __forceinline__ uint32_t float_order_key(float x)
{
    const uint32_t u = __float_as_uint(x);
    return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
}

// One workgroup per tile: orders its bucket by bin, writes the tile's bin starts and its
// part of the sorted list.  Inside a bin, atoms go by (x relative to the bin origin, id),
// so that the count pass can cut a stencil row's end bins at quarter-bin x boundaries;
// explicit targets go by caller position.  A bucket too large for LDS is ordered by (bin,
// id) and raises *xflag (the count pass then uses whole bins).  Each entry's payload is
// gathered into registers as soon as its id is known, so the gathers overlap the ordering
// in LDS.
template <bool TGT, typename BT>
__global__ __launch_bounds__(256) void tile_sort_kernel(int64_t n, int tb, int64_t ntiles,
                                                        const int* __restrict__ tstart,
                                                        BT* __restrict__ bucket,
                                                        int* __restrict__ bstart, TileSortOut o)
{
    if (o.run_if && *o.run_if == 0) return;
    __shared__ TileSortLds S;
    typedef typename std::conditional<TGT, int, float4>::type Pay;
    auto gather = [&](int i) -> Pay {
        if constexpr (TGT) {
            int64_t at = o.tgt[i];
            at = at < 0 || at >= o.natoms ? 0 : at;  // (out of range: flagged by target_keys_kernel)
            return o.inv[at];
        } else {
            return o.rec[i];
        }
    };
    const int64_t r = blockIdx.x;
    const int base = tstart[r], m = tstart[r + 1] - base;
    const bool fits = m <= kTileSortCap;
    for (int l = threadIdx.x; l < tb; l += 256) S.cnt[l] = 0;
    __syncthreads();
    Pay q[kTileSortPer];
    int qi[kTileSortPer], ql[kTileSortPer];
#pragma unroll
    for (int u = 0; u < kTileSortPer; ++u) {
        const int e = threadIdx.x + 256 * u;
        qi[u] = -1;
        if (fits && e < m) {
            const BT w = bucket[base + e];
            qi[u] = bk_id(w);
            ql[u] = bk_bin(w);
            q[u] = gather(qi[u]);
            atomicAdd(&S.cnt[ql[u]], 1);
        }
    }
    if (!fits)
        for (int e = threadIdx.x; e < m; e += 256) atomicAdd(&S.cnt[bk_bin(bucket[base + e])], 1);
    __syncthreads();
    // bin starts inside the bucket (tb <= 216: one pass of a 256-thread scan)
    {
        const int c = (int)threadIdx.x < tb ? S.cnt[threadIdx.x] : 0;
        int tot;
        const int ex = block_excl_scan<int, 256>(c, S.w32, &tot);
        if ((int)threadIdx.x < tb) {
            S.st[threadIdx.x] = ex;
            S.cnt[threadIdx.x] = ex;  // placement cursors
            bstart[r * tb + threadIdx.x] = base + ex;
        }
        if (threadIdx.x == 0) {
            S.st[tb] = tot;
            if (r == ntiles - 1) bstart[ntiles * tb] = (int)n;
        }
    }
    __syncthreads();
    auto emit = [&](int d, int i, Pay v) {
        if constexpr (TGT) {
            o.tslot[d] = i;
            o.tsidx[d] = v;
        } else {
            o.spos[d] = make_float4(v.x, v.y, v.z, __int_as_float(i));
            o.sflr[d] = __float_as_uint(v.w);
            o.sid[d] = i;
            if (o.inv) o.inv[i] = d;
        }
    };
    if (!fits) {
        // a very dense tile: the bucket sorted by (bin, id) in global memory (an entry's
        // bin sits above its id), then each entry goes to its place
        if constexpr (!TGT)
            if (o.xorder && threadIdx.x == 0 && flag_clear(o.xflag))
                atomicOr((unsigned long long*)o.xflag, 1ull);
        segment_sort<BT>(bucket + base, (BT*)o.stmp + base, m, sizeof(BT) == 4 ? 32 : 40, S.seg);
        for (int e = threadIdx.x; e < m; e += 256) {
            const int i = bk_id(bucket[base + e]);
            emit(base + e, i, gather(i));
        }
        return;
    }
    uint32_t qx[kTileSortPer];
#pragma unroll
    for (int u = 0; u < kTileSortPer; ++u) {
        qx[u] = 0;
        if constexpr (!TGT)
            if (qi[u] >= 0 && o.xorder) qx[u] = float_order_key(bin_xkey(q[u], o.xk));
        if (qi[u] >= 0) {
            const int d = atomicAdd(&S.cnt[ql[u]], 1);
            S.by[d] = qi[u];
            S.bx[d] = qx[u];
        }
    }
    __syncthreads();
    // each entry's place in its bin: the number of entries there with a smaller (x, id)
    // (targets, and atoms without xorder: x keys all 0, so by id)
#pragma unroll
    for (int u = 0; u < kTileSortPer; ++u) {
        if (qi[u] < 0) continue;
        const int i = qi[u], l = ql[u];
        const uint32_t x = qx[u];
        int below = 0;
        for (int k = S.st[l]; k < S.st[l + 1]; ++k) {
            const uint32_t xk = S.bx[k];
            below += (xk < x) | ((xk == x) & (S.by[k] < i));
        }
        emit(base + S.st[l] + below, i, q[u]);
    }
}

// ---------------------------------------------------------------- explicit targets
// Bin key of every target's atom (tile-level sort of the targets); out-of-range targets
// are flagged and take atom 0.  Also clears the tile totals for the targets' histogram.
__global__ void target_keys_kernel(int64_t nt, int64_t n, const int64_t* __restrict__ tgt,
                                   const uint32_t* __restrict__ key, uint32_t* __restrict__ tkey,
                                   int* __restrict__ tcnt, int64_t ntiles, int64_t* __restrict__ totals)
{
    if (totals[2] == 0) return;  // the targets are 0 .. nt - 1: no sort (target_prefix_kernel)
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (int64_t r = i0; r < ntiles; r += stride) tcnt[r] = 0;
    for (int64_t t = i0; t < nt; t += stride) {
        int64_t a = tgt[t];
        if (a < 0 || a >= n) {
            atomicOr((unsigned long long*)&totals[1], (unsigned long long)DG_FLAG_TARGET);
            a = 0;
        }
        tkey[t] = key[a];
    }
}

// Raises totals[2] unless the explicit targets are exactly 0, 1, ..., nt - 1 with nt <= n
// (then the count takes the atoms of each tile with ids < nt as its targets, in cell-list
// order, with no target sort).  totals[2] was cleared by tile_rank_kernel.
__global__ void target_prefix_kernel(int64_t nt, int64_t n, const int64_t* __restrict__ tgt,
                                     int64_t* __restrict__ totals)
{
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    bool other = nt > n;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < nt && !other; t += stride)
        other = tgt[t] != t;
    // one device atomic per workgroup at most, and none once the flag is seen set (atomics
    // on one address serialise: one per wave of a large list costs tens of microseconds)
    __shared__ int s_w[256 / 64];
    if (block_any<256>(other, s_w) && threadIdx.x == 0 && flag_clear(&totals[2]))
        atomicOr((unsigned long long*)&totals[2], 1ull);
}

__global__ void bin_targets_kernel(int64_t nt, int64_t n, const int64_t* __restrict__ tgt,
                                   const uint32_t* __restrict__ key, uint32_t* __restrict__ tkey,
                                   uint32_t* __restrict__ trank, int* __restrict__ tbcnt,
                                   int64_t* __restrict__ totals)
{
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nt) return;
    int64_t a = tgt[t];
    if (a < 0 || a >= n) {
        atomicOr((unsigned long long*)&totals[1], (unsigned long long)DG_FLAG_TARGET);
        a = 0;
    }
    uint32_t k = key[a];
    tkey[t] = k;
    trank[t] = (uint32_t)atomicAdd(&tbcnt[k], 1);
}

__global__ void scatter_targets_kernel(int64_t nt, const uint32_t* __restrict__ tkey,
                                       const uint32_t* __restrict__ trank,
                                       const int* __restrict__ tbstart, int* __restrict__ tslot)
{
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nt) return;
    tslot[tbstart[tkey[t]] + trank[t]] = (int)t;
}

__global__ void finish_targets_kernel(int64_t nbins, int64_t n, const int* __restrict__ tbstart,
                                      int* __restrict__ tslot, const int64_t* __restrict__ tgt,
                                      const int* __restrict__ inv, int* __restrict__ tsidx)
{
    int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= nbins) return;
    int lo = tbstart[q], hi = tbstart[q + 1];
    if (hi - lo > 1 && hi - lo <= kBinSortMax) small_sort(tslot, lo, hi);
    for (int j = lo; j < hi; ++j) {
        int64_t a = tgt[tslot[j]];
        if (a < 0 || a >= n) a = 0;
        tsidx[j] = inv[a];
    }
}

#endif  // DG_MAIN_TU (sort kernels)

// ---------------------------------------------------------------- neighbour search
struct SearchArgs {
    int64_t align_max_edges;  // line-aligned wave ranges in the expansion up to this edge total
    double C[9];
    double Cinv[9];
    double hC[9];  // bin step vectors: row d = C[d] / nb[d]
    double r2;
    int lowtri;    // lower-triangular cell (a along x, b in the xy plane, positive diagonal):
                   // stencil rows are trimmed to the padded cutoff sphere; 2: orthorhombic
    float hax, hbx, hby, hcx, hcy, hcz;  // bin step vectors C[d] / nb[d] (lower triangle)
    float rprune2, pmargin;
    float gy_off, gz_off;             // -hby - pmargin, -hcz - pmargin (orthorhombic rows)
    float inv_hax, inv_hby, inv_hcz;  // reciprocals of the diagonal bin steps
    int nb[3], P[3], T[3], ntl[3], R[3], pbc[3];
    int tb, nregion;
    int64_t ntiles;
    float toff, hi_off;  // d2' = d2 - toff: edge iff bits(d2') < lo_bits, band iff d2' <= hi_off
    uint32_t lo_bits;
    const float4* spos;
    const uint32_t* sflr;
    const int* sid;    // atom id of every cell-list entry
    const void* cpos;  // the positions in cell-list order (pos dtype; set for vector outputs)
    const int* bstart;
    const int* tile_of_rank;
    const int* rank_of_tile;
    const void* pos;
    int f64;
    // explicit targets (subset != 0)
    int subset;
    // Explicit targets that are exactly 0, 1, ..., ntarg - 1 (checked on the device: the
    // local atoms of a partition, DistGraphBuilder's mode B) need no target sort: every atom
    // of a tile is a lane, and atoms with ids >= ntarg (the ghosts) stay idle.  pmis is the
    // device word that is nonzero when the list is not that prefix (null: never masked).
    const int64_t* pmis;
    int64_t ntarg;
    const int* tbstart;
    const int* tsidx;
    const int* tslot;  // caller position of each sorted target
    // count pass
    int* cnt;          // per target, processing order
    int* counts_user;  // per target, caller order (nullable)
    int* ttot;         // per tile (rank order)
    int* tfix;         // per tile: kFix* bits, work left to search_kernel<1>
    // write pass
    int64_t* tbase;
    int64_t* out_src;
    int64_t* out_dst;
    float* out_shift;
    void* out_vec;
    void* out_dist;
    int vout_f64;
    int64_t capacity;
    int64_t* totals;
    const int64_t* out_ids;  // written for atom i: out_ids[i] (null: i); positions use i
    // Per-target neighbour slots (K region indices each), or null.  Entries go in groups
    // of 8 (16 bytes), group-major: group g of target j at slot + 8 * (g * nslot + j), so
    // the groups that neighbouring targets fill at about the same time share cache lines.
    uint16_t* slot;
    int K;
    int64_t nslot;  // targets (group row length)
    int xsplit;     // bins ordered by x unless *xflag (see tile_sort_kernel): quarter-bin row ends
};

// Whether this build's targets are the atoms of the tile with ids < ntarg (see SearchArgs).
__device__ __forceinline__ bool masked_targets(const SearchArgs& a)
{
    return a.subset && a.pmis != nullptr && *a.pmis == 0;
}
// Whether targets come from the explicit (sorted) target list.
__device__ __forceinline__ bool listed_targets(const SearchArgs& a)
{
    return a.subset && !masked_targets(a);
}

// Output order -> tile rank.  Consecutive workgroups go round-robin to the 8 XCDs; the
// Morton order is dealt out to them in runs of kXcdRun tiles (run q to XCD q mod 8), so a
// run of neighbouring tiles shares its halo bins in one L2, and every XCD's share is
// spread over the whole box.  (One contiguous eighth of the Morton order per XCD puts all
// the work of a half-empty box -- a slab, a two-phase cell -- on four XCDs: C4's count
// took 0.317 ms that way against 0.256 ms with runs.)  The output holds the tiles in this
// order; the last ntiles mod (8 kXcdRun) tiles keep their Morton rank.
constexpr int64_t kXcdRun = 16;
__device__ __forceinline__ int64_t xcd_tile_rank(int64_t b, int64_t ntiles)
{
    const int64_t full = ntiles / (8 * kXcdRun) * (8 * kXcdRun);
    if (b >= full) return b;
    const int64_t x = b & 7, j = b >> 3;
    return ((j / kXcdRun) * 8 + x) * kXcdRun + (j % kXcdRun);
}

// LDS of one search workgroup.
//   qbuf   the staged region: float4 (position relative to the tile origin, atom id) per
//          entry while distances are tested; reused as ExpandStage by the expansion;
//   rt/bt  region bin table (rp: first entry of each region bin, rg: its cell-list start)
//          while the region is staged; reused as the batch tables of the expansion.
// The count pass adds the per-lane slot staging (lb) and still fits four workgroups per
// CU; the fix-up write pass adds the per-entry shift table T.
constexpr int kStage = 64 * kExpandIlp;  // edges one wave stages per step
// Edges whose outputs span whole 128-byte lines from a line-aligned start: 32 edges are 256
// bytes of int64 ids, 384 of fp32 shifts (and of fp32 vectors), 128 of fp32 distances.
constexpr int kLineEdges = 32;
// Line-aligned wave ranges pay while the slot array plus a small share of the outputs stay
// under a budget, and cost time past it (a rule fitted to measurements on this part: at
// C3 the write stage takes 0.545 ms aligned against 0.645 ms; with 448 MB of slots, or with
// C3's edge vectors, aligned ranges are 4-10 % slower).
constexpr double kAlignBudget = 564e6;      // bytes
constexpr double kAlignOutShare = 0.065;    // of the output bytes
static_assert(kLineEdges <= 64 * kExpandIlp, "a wave's head is fetched in one step");
// CAP: region entries staged (one LDS chunk, or two for the dense tiles of expand2)
// STG: edges a wave stages per step (64 per unit of the expansion's ILP)
template <int CAP, int STG = kStage>
struct ExpandStageT {
    int2 e[CAP + 1];  // per region entry: source atom id, packed (bin shift - floor)
    int st_src[kBlock / 64][STG];
    int st_dst[kBlock / 64][STG];
    uint32_t st_S[kBlock / 64][STG];
};
typedef ExpandStageT<kCap> ExpandStage;
struct BatchTab {
    int off[kBlock + 1];  // edge offsets of the batch's targets
    int tid[kBlock];
    uint32_t tf[kBlock];
};
constexpr int kQBytes = (int)sizeof(float4) * (kCap + 1);
static_assert(sizeof(ExpandStage) <= (size_t)kQBytes, "expansion view exceeds the region buffer");

constexpr int kRing = 16;  // slot entries a lane stages in LDS (two groups of 8)

// Byte address of ring entry k2 / 2 (mod 16) of the lane whose ring starts at byte lane_off
// (a multiple of 32): lane_off | (k2 & 30) in one VALU op (the compiler emits an and and an
// add for it).
__device__ __forceinline__ uint32_t ring_at(int k2, uint32_t lane_off)
{
    uint32_t r;
    asm("v_and_or_b32 %0, %1, 30, %2" : "=v"(r) : "v"(k2), "v"(lane_off));
    return r;
}
struct SearchLds {
    __align__(16) unsigned char qbuf[kQBytes];
    int tbs[kTileMax * kTileMax * kTileMax + 1];  // bin starts of the tile
    int64_t w64[kBlock / 64];
    int w32[kBlock / 64];
    int64_t bc[2];  // workgroup broadcasts
};
struct CountLds : SearchLds {
    int rp[kMaxRegion + 1];                     // first region entry of each region bin
    __align__(16) uint16_t lb[kBlock][kRing];   // per-lane ring of slot entries
};
struct FixLds : SearchLds {
    int rp[kMaxRegion + 1];
    uint32_t T[kCap + 1];  // packed (bin image shift - source floor) per entry
};
struct ExpandLds : SearchLds {
    BatchTab bt;
};
// The expansion of two-chunk tiles: the same members, a region buffer for 2 kCap entries.
struct Expand2Lds {
    __align__(16) unsigned char qbuf[sizeof(ExpandStageT<2 * kCap>)];
    int tbs[kTileMax * kTileMax * kTileMax + 1];
    int64_t w64[kBlock / 64];
    int w32[kBlock / 64];
    int64_t bc[2];
    BatchTab bt;
};
template <int CAP> struct ExpandLdsOf { typedef ExpandLds type; };
template <> struct ExpandLdsOf<2 * kCap> { typedef Expand2Lds type; };
// Per wave, the edge vectors and distances of one step (STG edges) as the bytes they take
// in the outputs (v: 3 per edge, d: 1 per edge), so 16-byte chunks go out as they are.
template <typename VT, int STG>
struct VecStageT {
    __align__(16) VT v[kBlock / 64][3 * STG];
    __align__(16) VT d[kBlock / 64][STG];
};
// The expansion with edge vectors / distances of type VT, in steps of 64 * kVecIlp edges.
// (Half the steps -- 8 KB less staging, four workgroups per CU for fp32 vectors -- measured
// slower: C3 1.27 vs 1.21 ms.)
constexpr int kVecIlp = kExpandIlp;
template <typename VT>
struct ExpandVLds : ExpandLds {
    VecStageT<VT, 64 * kVecIlp> vs;
};
static_assert(sizeof(CountLds) <= 40960, "count pass must fit four workgroups per CU");
template <int MODE>
struct LdsOf { typedef CountLds type; };
template <>
struct LdsOf<1> { typedef FixLds type; };

// Cartesian offset of region bin (rx, ry, rz) from the centre of its tile: positions in
// LDS are relative to the tile centre, which keeps their magnitudes (and so their
// rounding) small.
__device__ __forceinline__ void region_offset(const SearchArgs& a, int rx, int ry, int rz,
                                              float* o)
{
    const double u0 = (double)(rx - a.P[0]) - 0.5 * a.T[0], u1 = (double)(ry - a.P[1]) - 0.5 * a.T[1],
                 u2 = (double)(rz - a.P[2]) - 0.5 * a.T[2];
#pragma unroll
    for (int c = 0; c < 3; ++c) o[c] = (float)fma(u2, a.hC[6 + c], fma(u1, a.hC[3 + c], u0 * a.hC[c]));
}

// Exact (canonical fp64) decision for a candidate the fp32 prefilter cannot settle: atom
// src as seen from target tgt, (dq0, dq1, dq2) = its fp32 LDS position minus the target's.
// The integer image shift is recovered by rounding: dq - (pos[src] - pos[tgt]) is S.C up
// to the LDS rounding (~1e-5 A), far below half a cell.
__device__ __forceinline__ bool exact_edge(const SearchArgs& a, int src, int tgt, double dq0,
                                        double dq1, double dq2)
{
    double ps[3], pt[3], v[3];
    load_pos(a.pos, a.f64, src, ps);
    load_pos(a.pos, a.f64, tgt, pt);
    const double w0 = dq0 - (ps[0] - pt[0]), w1 = dq1 - (ps[1] - pt[1]), w2 = dq2 - (ps[2] - pt[2]);
    const int S0 = (int)rint(canon_frac(w0, w1, w2, a.Cinv, 0));
    const int S1 = (int)rint(canon_frac(w0, w1, w2, a.Cinv, 1));
    const int S2 = (int)rint(canon_frac(w0, w1, w2, a.Cinv, 2));
    if (src == tgt && S0 == 0 && S1 == 0 && S2 == 0) return false;
    const double d2 = canon_d2(ps, pt, S0, S1, S2, a.C, v);
    return d2 > kSelfThr && d2 <= a.r2;
}

// One edge: edge_index columns, integer cell shift, optional canonical vector / distance.
__device__ __forceinline__ int out_id(const SearchArgs& a, int i)
{
    return a.out_ids ? (int)a.out_ids[i] : i;
}

// src, dst: atom indices (of pos); the ids written go through a.out_ids.
__device__ __forceinline__ void emit_edge(const SearchArgs& a, int64_t o, int src, int dst, int S0,
                                          int S1, int S2)
{
    a.out_src[o] = out_id(a, src);
    a.out_dst[o] = out_id(a, dst);
    *(float3*)(a.out_shift + 3 * o) = make_float3((float)S0, (float)S1, (float)S2);
    if (a.out_vec || a.out_dist) {
        double ps[3], pt[3], vv[3];
        load_pos(a.pos, a.f64, src, ps);
        load_pos(a.pos, a.f64, dst, pt);
        const double dd = canon_d2(ps, pt, S0, S1, S2, a.C, vv);
        if (a.vout_f64) {
            if (a.out_vec) {
                double* ov = (double*)a.out_vec + 3 * o;
                ov[0] = vv[0]; ov[1] = vv[1]; ov[2] = vv[2];
            }
            if (a.out_dist) ((double*)a.out_dist)[o] = sqrt(dd);
        } else {
            if (a.out_vec) {
                float* ov = (float*)a.out_vec + 3 * o;
                ov[0] = (float)vv[0]; ov[1] = (float)vv[1]; ov[2] = (float)vv[2];
            }
            if (a.out_dist) ((float*)a.out_dist)[o] = (float)sqrt(dd);
        }
    }
}

// ---------------------------------------------------------------- region bins
// Bin-list key of region bin rb of the tile at bin g0 (periodic wrap on pbc axes); false
// outside the grid on a non-periodic axis (an empty bin).
__device__ __forceinline__ bool region_bin_key(const SearchArgs& a, const int* g0, int rb,
                                               int64_t* key)
{
    const int R0 = a.R[0], R1 = a.R[1];
    const int r[3] = {rb % R0, (rb / R0) % R1, rb / (R0 * R1)};
    int w[3];
    bool ok = true;
#pragma unroll
    for (int d = 0; d < 3; ++d) {
        const int gg = g0[d] - a.P[d] + r[d];
        if (a.pbc[d]) {
            const int m = gg % a.nb[d];
            w[d] = m < 0 ? m + a.nb[d] : m;
        } else {
            ok = ok && gg >= 0 && gg < a.nb[d];
            w[d] = gg;
        }
    }
    if (!ok) return false;
    const int t0 = w[0] / a.T[0], t1 = w[1] / a.T[1], t2 = w[2] / a.T[2];
    const int l0 = w[0] - t0 * a.T[0], l1 = w[1] - t1 * a.T[1], l2 = w[2] - t2 * a.T[2];
    const int tl = t0 + a.ntl[0] * (t1 + a.ntl[1] * t2);
    *key = (int64_t)a.rank_of_tile[tl] * a.tb + (l0 + a.T[0] * (l1 + a.T[1] * l2));
    return true;
}

// Cell-list start of region bin rb (0 for a bin outside the grid, which is empty).
__device__ __forceinline__ int region_bin_start(const SearchArgs& a, const int* g0, int rb)
{
    int64_t key;
    return region_bin_key(a, g0, rb, &key) ? a.bstart[key] : 0;
}

// Cell-list range of the region bins rb = kRegPerThread * threadIdx.x + h of the tile at
// bin g0; returns the thread's total.
__device__ __forceinline__ int region_bins(const SearchArgs& a, const int* g0, int* rcnt, int* rst)
{
    int sum = 0;
#pragma unroll
    for (int h = 0; h < kRegPerThread; ++h) {
        rcnt[h] = 0;
        rst[h] = 0;
        const int rb = kRegPerThread * threadIdx.x + h;
        int64_t key;
        if (rb < a.nregion && region_bin_key(a, g0, rb, &key)) {
            rst[h] = a.bstart[key];
            rcnt[h] = a.bstart[key + 1] - rst[h];
        }
        sum += rcnt[h];
    }
    return sum;
}

typedef float v3f __attribute__((ext_vector_type(3)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- edge expansion
// Stages the tile's region into ExpandStage::e as (source atom id, packed bin shift -
// floor) pairs -- 8 bytes per entry -- bin by bin from the cell list.  The caller has
// finished every use of the float4 view of the region buffer.
// GIDX: an entry names its source by cell-list index instead of atom id; MAP: by the id
// written for it (a.out_ids), for expansions that need no positions.
template <int CAP, bool GIDX = false, bool MAP = false>
__device__ __forceinline__ void stage_pairs(const SearchArgs& a, typename ExpandLdsOf<CAP>::type& sh,
                                            const int* g0)
{
    ExpandStageT<CAP>& X = *(ExpandStageT<CAP>*)sh.qbuf;
    {
        int rcnt[kRegPerThread], rst[kRegPerThread];
        const int mysum = region_bins(a, g0, rcnt, rst);
        int total;
        int ex = block_excl_scan<int, kBlock>(mysum, sh.w32, &total);
        const int R0 = a.R[0], R1 = a.R[1];
#pragma unroll
        for (int h = 0; h < kRegPerThread; ++h) {
            const int rb = kRegPerThread * threadIdx.x + h;
            if (rcnt[h] > 0) {
                const int r[3] = {rb % R0, (rb / R0) % R1, rb / (R0 * R1)};
                int sb[3];
#pragma unroll
                for (int d = 0; d < 3; ++d) {
                    const int gg = g0[d] - a.P[d] + r[d];
                    sb[d] = a.pbc[d] ? floor_div(gg, a.nb[d]) : 0;
                }
                for (int i = 0; i < rcnt[h]; ++i) {
                    const int gidx = rst[h] + i;
                    const uint32_t fl = a.sflr[gidx];
                    const int src = GIDX ? gidx : (MAP ? out_id(a, a.sid[gidx]) : a.sid[gidx]);
                    X.e[ex + i] = make_int2(src, (int)pack3(sb[0] - unpack3(fl, 0),
                                                                     sb[1] - unpack3(fl, 1),
                                                                     sb[2] - unpack3(fl, 2)));
                }
            }
            ex += rcnt[h];
        }
        if (threadIdx.x == 0) X.e[CAP] = make_int2(0, 0);
    }

}

// Writes edge k < K of every target of the tile from its slot (region entries staged by
// stage_pairs; ebase = output offset of the tile's first edge).  Each batch of up to 256
// targets has its edges split evenly over the waves; a wave walks its range 64 edges at a
// time, lane e finding its target by a short forward walk from the wave's current target.
// Edges k >= K are left to search_kernel<1>.
// PLAIN: edges go out in 16-byte groups staged in LDS; with VT (float or double) the edge
// vectors and distances too, staged in *vsp (a VecStageT<VT>); without PLAIN every edge is
// written by its lane (emit_edge, vectors included).
template <bool PLAIN, int CAP, typename VT = void, int ILP = kExpandIlp>
__device__ __forceinline__ void expand_tile(const SearchArgs& a, typename ExpandLdsOf<CAP>::type& sh,
                                            int tbeg, int ntg, int64_t ebase, void* vsp = nullptr)
{
    static_assert(ILP % 2 == 0, "two edges per 16-byte chunk of sources / targets");
    constexpr int kStg = 64 * ILP;  // edges a wave stages per step
    ExpandStageT<CAP, kStg>& X = *(ExpandStageT<CAP, kStg>*)sh.qbuf;
    BatchTab& B = sh.bt;
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int NWv = kBlock / 64;
    constexpr bool plain = PLAIN;
    constexpr bool kVec = !std::is_void<VT>::value;
    static_assert(PLAIN || !kVec, "the per-lane path writes vectors itself");
    typedef typename std::conditional<kVec, VT, float>::type VTn;  // (a type when VT is void)
    for (int k0 = 0; k0 < ntg; k0 += kBlock) {
        const int nbatch = min(kBlock, ntg - k0);
        const int j = tbeg + k0 + threadIdx.x;
        const bool active = (int)threadIdx.x < nbatch;
        const int mycnt = active ? a.cnt[j] : 0;
        int btot;
        const int ex = block_excl_scan<int, kBlock>(mycnt, sh.w32, &btot);
        if (active) {
            const int sidx = listed_targets(a) ? a.tsidx[j] : j;
            B.off[threadIdx.x] = ex;
            // (the plain path writes B.tid as it is: the id to write; with vectors it also
            // indexes the target's position, and the id is mapped when staged)
            B.tid[threadIdx.x] = (plain && !kVec) ? out_id(a, a.sid[sidx]) : a.sid[sidx];
            B.tf[threadIdx.x] = a.sflr[sidx];
        }
        if (threadIdx.x == 0) B.off[nbatch] = btot;
        __syncthreads();  // region entries and the batch tables visible to all waves

        // the waves' ranges split at output offsets that are multiples of line: with
        // kLineEdges the 16-byte groups of every full step fill whole 128-byte lines of each
        // output (the edge total, from the count stage, decides: see kAlignBudget)
        const int line = a.totals[0] <= a.align_max_edges ? kLineEdges : 4;
        auto split = [&](int ww) {
            if (ww == 0) return 0;
            if (ww == NWv) return btot;
            const int64_t g = ebase + ((int64_t)btot * ww) / NWv;
            const int64_t al = (g + line - 1) & ~(int64_t)(line - 1);
            return (int)min<int64_t>(al - ebase, btot);
        };
        const int E0 = split(w), E1 = split(w + 1);
        int tcur = 0;
        {
            int lo = 0, hi = nbatch;  // target containing E0
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (B.off[mid] <= E0) lo = mid; else hi = mid;
            }
            tcur = rfl(lo);
        }
        const int64_t wbase = ebase + E0;
        const char* __restrict__ sl = (const char*)a.slot + (size_t)16 * (tbeg + k0);
        const uint64_t gstep = 16ull * (uint64_t)a.nslot;  // bytes between a target's groups

        // Edges [b0, b1) of the batch (b1 - b0 <= 64 * ILP), lane-strided: edge
        // b0 + 64u + lane -> source id, target id, packed shift; ok = false past b1 or for
        // k >= K (left to search_kernel<1>).  All slot loads are issued before the first
        // entry is looked up.  Advances tcur to the target of edge b1 - 1.
        // Two halves: locate() finds (target, k) of edges [b0, b1) and issues their slot
        // loads -- unconditionally (edges past b1 or with k >= K load a valid dummy), so all
        // ILP loads are in flight together -- and advances tcur to the target of
        // edge b1 - 1; resolve() turns them into (source id, target id, packed shift).  The
        // plain path locates the next step before storing this one, so the wait on its
        // loads does not also wait on the stores (the memory counter is shared).
        struct Loc {
            int tt[ILP], kk[ILP], raw[ILP];
        };
        auto locate = [&](int b0, int b1, Loc& L) {
            int t = tcur;
#pragma unroll
            for (int u = 0; u < ILP; ++u) {
                const int e = b0 + 64 * u + lane;
                L.kk[u] = a.K;
                L.tt[u] = t;
                if (e < b1) {
                    while (B.off[t + 1] <= e) ++t;
                    L.tt[u] = t;
                    L.kk[u] = e - B.off[t];
                }
            }
#pragma unroll
            for (int u = 0; u < ILP; ++u) {
                const uint64_t at = L.kk[u] < a.K ? (uint64_t)(uint32_t)(L.kk[u] >> 3) * gstep +
                                                        (16u * (uint32_t)L.tt[u] + 2u * (L.kk[u] & 7))
                                                  : 0ull;
                L.raw[u] = (int)*(const uint16_t*)(sl + at);
            }
            // the lane holding edge b1 - 1 has its target in t
            if (b1 > b0) tcur = __builtin_amdgcn_readlane(t, (b1 - 1 - b0) & 63);
        };
        // with vectors, region entries name their source by cell-list index (rg), which
        // also indexes the positions in cell-list order
        int rg[ILP];
        auto resolve = [&](const Loc& L, int* rs, int* rd, uint32_t* rS, bool* rok) {
#pragma unroll
            for (int u = 0; u < ILP; ++u) {
                rok[u] = L.kk[u] < a.K;
                const int2 en = X.e[rok[u] ? min(L.raw[u] >> 4, CAP) : CAP];
                const uint32_t ft = B.tf[L.tt[u]];
                if constexpr (kVec) {
                    rg[u] = en.x;
                    rs[u] = a.sid[en.x];
                } else {
                    rs[u] = en.x;
                }
                rd[u] = B.tid[L.tt[u]];
                rS[u] = pack3(unpack3((uint32_t)en.y, 0) + unpack3(ft, 0),
                              unpack3((uint32_t)en.y, 1) + unpack3(ft, 1),
                              unpack3((uint32_t)en.y, 2) + unpack3(ft, 2));
            }
        };
        auto fetch = [&](int b0, int b1, int* rs, int* rd, uint32_t* rS, bool* rok) {
            Loc L;
            locate(b0, b1, L);
            resolve(L, rs, rd, rS, rok);
        };
        // per-lane stores of the fetched edges (ranges not aligned to 4 edges, and the
        // vector / distance outputs)
        auto store_lanes = [&](int b0, const int* rs, const int* rd, const uint32_t* rS,
                               const bool* rok) {
#pragma unroll
            for (int u = 0; u < ILP; ++u) {
                if (!rok[u]) continue;
                const int64_t o = wbase + (b0 + 64 * u + lane - E0);
                const int S0 = unpack3(rS[u], 0), S1 = unpack3(rS[u], 1), S2 = unpack3(rS[u], 2);
                if constexpr (plain && !kVec) {
                    __builtin_nontemporal_store((int64_t)rs[u], a.out_src + o);
                    __builtin_nontemporal_store((int64_t)rd[u], a.out_dst + o);
                    const v3f sv = {(float)S0, (float)S1, (float)S2};
                    __builtin_nontemporal_store(sv, (v3f*)(a.out_shift + 3 * o));
                } else {
                    emit_edge(a, o, rs[u], rd[u], S0, S1, S2);
                }
            }
        };

        int rs[ILP], rd[ILP];
        uint32_t rS[ILP];
        bool rok[ILP];
        if constexpr (!plain) {
            for (int b0 = E0; b0 < E1; b0 += 64 * ILP) {
                fetch(b0, min(E1, b0 + 64 * ILP), rs, rd, rS, rok);
                store_lanes(b0, rs, rd, rS, rok);
            }
        } else {
            // Groups of 4 edges that start at a multiple of 4 in the output are staged in
            // LDS and written as 16-byte stores: 2 for the 4 sources, 2 for the targets, 3
            // for the shifts, every one 16-byte aligned.  The edges before the first line
            // boundary (up to kLineEdges - 1, only at the start of a batch) and the up-to-3
            // after the last group are stored per lane, so no 16-byte store of this wave
            // touches another wave's edges.  A slot left to search_kernel<1> (k >= K)
            // receives a placeholder here and its edge there, later on the same stream.
            const int head = min((int)((line - (wbase & (line - 1))) & (line - 1)), E1 - E0);
            const int A0 = E0 + head;
            const int A1 = A0 + ((E1 - A0) & ~3);
            if (head > 0) {
                fetch(E0, A0, rs, rd, rS, rok);
                store_lanes(E0, rs, rd, rS, rok);
            }
            int* st_s = X.st_src[w];
            int* st_d = X.st_dst[w];
            uint32_t* st_S = X.st_S[w];
            // with vectors: this lane's edges' canonical vectors and distances (fp64, as
            // emit_edge computes them), and the wave's staging rows for them
            VTn rv[ILP][3], rdd[ILP];
            VTn* st_v = nullptr;
            VTn* st_dd = nullptr;
            if constexpr (kVec) {
                VecStageT<VTn, kStg>& VS = *(VecStageT<VTn, kStg>*)vsp;
                st_v = VS.v[w];
                st_dd = VS.d[w];
            }
            auto vectors = [&]() {
                if constexpr (kVec) {
#pragma unroll
                    for (int u = 0; u < ILP; ++u) {
                        double ps[3], pt[3], vv[3];
                        load_pos(a.cpos, a.f64, rg[u], ps);  // (cell-list order: local)
                        load_pos(a.pos, a.f64, rd[u], pt);
                        const double dd = canon_d2(ps, pt, unpack3(rS[u], 0), unpack3(rS[u], 1),
                                                   unpack3(rS[u], 2), a.C, vv);
                        rv[u][0] = (VTn)vv[0];
                        rv[u][1] = (VTn)vv[1];
                        rv[u][2] = (VTn)vv[2];
                        rdd[u] = (VTn)sqrt(dd);
                    }
                }
            };
            // Full steps of 64 * ILP edges run branch-free: the next step's slot loads
            // are issued before this step's stores and consumed right behind them, in
            // straight-line code, so the wait on the loads leaves the stores in flight (the
            // memory counter is shared by loads and stores).  The last, partial step is
            // masked.
            constexpr int kStep = 64 * ILP;
            const int nfull = (A1 - A0) / kStep;
            auto stage = [&](int n) {
#pragma unroll
                for (int u = 0; u < ILP; ++u) {
                    const int i = 64 * u + lane;
                    if (i < n) {
                        if constexpr (kVec) {
                            st_s[i] = out_id(a, rs[u]);
                            st_d[i] = out_id(a, rd[u]);
                        } else {
                            st_s[i] = rs[u];
                            st_d[i] = rd[u];
                        }
                        st_S[i] = rS[u];
                        if constexpr (kVec) {
                            st_v[3 * i] = rv[u][0];
                            st_v[3 * i + 1] = rv[u][1];
                            st_v[3 * i + 2] = rv[u][2];
                            st_dd[i] = rdd[u];
                        }
                    }
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            };
            // 16-byte stores of n staged edges (n a multiple of 4) starting at output gb
            auto store_groups = [&](int64_t gb, int n, auto full) {
                const int G = n >> 2;
                v4i* __restrict__ os = (v4i*)(a.out_src + gb);
                v4i* __restrict__ od = (v4i*)(a.out_dst + gb);
                v4f* __restrict__ of = (v4f*)(a.out_shift + 3 * gb);
                // chunks of a full step: kStg / 2 of sources (and of targets), 3 kStg / 4
                // of shifts; a loop over them masks the chunks past its count
                constexpr int kChE = kStg / 2, kChS = 3 * kStg / 4;
#pragma unroll
                for (int h = 0; h < (kChE + 63) / 64; ++h) {
                    const int c = 64 * h + lane;  // 16-byte chunk: edges 2c, 2c + 1
                    if (c < (full ? kChE : 2 * G)) {
                        const v4i vs = {st_s[2 * c], 0, st_s[2 * c + 1], 0};
                        const v4i vd = {st_d[2 * c], 0, st_d[2 * c + 1], 0};
                        __builtin_nontemporal_store(vs, os + c);
                        __builtin_nontemporal_store(vd, od + c);
                    }
                }
#pragma unroll
                for (int h = 0; h < (kChS + 63) / 64; ++h) {
                    const int c = 64 * h + lane;  // 16-byte chunk: shift floats 4c .. 4c + 3
                    if (c < (full ? kChS : 3 * G)) {
                        float f[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int fi = 4 * c + i;
                            f[i] = (float)unpack3(st_S[fi / 3], fi % 3);
                        }
                        const v4f vf = {f[0], f[1], f[2], f[3]};
                        __builtin_nontemporal_store(vf, of + c);
                    }
                }
                if constexpr (kVec) {
                    // the staged rows are the outputs' bytes: n edges are 3 n VT of vector
                    // and n VT of distance, whole 16-byte chunks (n is a multiple of 4)
                    constexpr int kPer = 16 / (int)sizeof(VTn);  // VT per chunk
                    constexpr int kChV = 3 * kStg / kPer, kChD = kStg / kPer;
                    if (a.out_vec) {
                        v4i* __restrict__ ov = (v4i*)((VTn*)a.out_vec + 3 * gb);
                        const v4i* sv = (const v4i*)st_v;
#pragma unroll
                        for (int h = 0; h < (kChV + 63) / 64; ++h) {
                            const int c = 64 * h + lane;
                            if (c < (full ? kChV : 3 * n / kPer)) __builtin_nontemporal_store(sv[c], ov + c);
                        }
                    }
                    if (a.out_dist) {
                        v4i* __restrict__ odd = (v4i*)((VTn*)a.out_dist + gb);
                        const v4i* sd = (const v4i*)st_dd;
#pragma unroll
                        for (int h = 0; h < (kChD + 63) / 64; ++h) {
                            const int c = 64 * h + lane;
                            if (c < (full ? kChD : n / kPer)) __builtin_nontemporal_store(sd[c], odd + c);
                        }
                    }
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            };
            if (A0 < A1) {
                fetch(A0, min(A1, A0 + kStep), rs, rd, rS, rok);
                vectors();
            }
            for (int s0 = 0; s0 < nfull; ++s0) {
                const int b0 = A0 + s0 * kStep;
                stage(kStep);
                Loc L;
                locate(b0 + kStep, min(A1, b0 + 2 * kStep), L);  // empty past A1: dummy loads
                store_groups(wbase + (b0 - E0), kStep, std::true_type());
                resolve(L, rs, rd, rS, rok);
                vectors();
            }
            if (nfull * kStep < A1 - A0) {
                const int b0 = A0 + nfull * kStep;
                stage(A1 - b0);
                store_groups(wbase + (b0 - E0), A1 - b0, std::false_type());
            }
            if (A1 < E1) {
                fetch(A1, E1, rs, rd, rS, rok);
                store_lanes(A1, rs, rd, rS, rok);
            }
        }
        ebase += btot;
        __syncthreads();  // before the next batch rewrites the tables
    }
}

// Neighbour search, one tile of bins per workgroup.
//
// The region of (T+2P)^3 bins around the tile is staged in LDS (in chunks if it does
// not fit).  Both passes share the per-target sweep below (one lane per target, rows of
// the stencil trimmed to the cutoff sphere for lower-triangular cells), so they agree on
// every edge and on its order.
//
// MODE 0 (count): per-target degree, per-tile total, and -- for tiles whose region fits
//   in one chunk -- the target's neighbours as 2-byte LDS entry byte offsets in its slot of
//   K entries (written 16 bytes at a time through a per-lane LDS buffer).
// MODE 1 (fix-up write, only tiles the count pass flagged): targets with more than K
//   neighbours get their edges k >= K by a second sweep, tiles with a chunked region are
//   swept again and written directly.  Every other edge is written by expand_kernel.
// What the count of one tile leaves for the publication / expansion of its edges.
struct TileOut {
    int64_t tt;  // edges of the tile
    int fix;     // kFix* bits
    int tbeg, ntg;
    int g0[3];
};

// QS (count pass, cell list ordered by bin_xkey inside bins): the quarter-bin row ends
// described below, for orthorhombic (1) or other lower-triangular cells (2); 0: whole
// bins, any cell.
template <int MODE, int QS = 0>
__device__ __forceinline__ TileOut search_tile(const SearchArgs& a,
                                               typename LdsOf<MODE>::type& sh, int64_t ord)
{
    constexpr bool WRITE = MODE == 1;
    float4* const shq = (float4*)sh.qbuf;
    TileOut out;
    out.tt = 0;
    out.fix = 0;
    // ord: the tile's place in the output (and index of its per-tile records); rank: its
    // Morton rank.  Tiles go to the output in ord order; ord -> rank is xcd_tile_rank.
    const int64_t rank = xcd_tile_rank(ord, a.ntiles);
    const int lin = a.tile_of_rank[rank];
    const int tx = lin % a.ntl[0];
    const int ty = (lin / a.ntl[0]) % a.ntl[1];
    const int tz = lin / (a.ntl[0] * a.ntl[1]);
    const int g0[3] = {tx * a.T[0], ty * a.T[1], tz * a.T[2]};
    const bool listed = listed_targets(a), masked = a.subset && !listed;
    const int* tstart = listed ? a.tbstart : a.bstart;
    const int64_t kb = rank * a.tb;
    const int tbeg = tstart[kb], tend = tstart[kb + a.tb];
    const int ntg = tend - tbeg;
    out.tbeg = tbeg;
    out.ntg = ntg;
    for (int d = 0; d < 3; ++d) out.g0[d] = g0[d];
    if (ntg == 0) {
        if (MODE == 0 && threadIdx.x == 0) {
            a.ttot[ord] = 0;
            a.tfix[ord] = 0;
        }
        return out;
    }
    if (WRITE && (a.tfix[ord] & (kFixOver | kFixChunked)) == 0) return out;  // written by an expansion
    if (!WRITE && masked) {
        // a tile of ghosts only (atoms with ids >= ntarg) has no targets: nothing to count
        bool mine = false;
        for (int k = threadIdx.x; k < ntg; k += kBlock) mine = mine || a.sid[tbeg + k] < a.ntarg;
        if (!block_any<kBlock>(mine, sh.w32)) {
            if (threadIdx.x == 0) {
                a.ttot[ord] = 0;
                a.tfix[ord] = 0;
            }
            return out;
        }
    }
    for (int k = threadIdx.x; k <= a.tb; k += kBlock) sh.tbs[k] = tstart[kb + k];

    int64_t ebase = 0;
    if (WRITE) {
        ebase = a.tbase[ord];
        if (ebase + a.ttot[ord] > a.capacity) {
            if (threadIdx.x == 0)
                atomicOr((unsigned long long*)&a.totals[1], (unsigned long long)kStatusCapacity);
            return out;
        }
    }

    // ---- region table: (T+2P)^3 bins around the tile, periodic wrap on pbc axes
    const int R0 = a.R[0], R1 = a.R[1];
    int rcnt[kRegPerThread], rst[kRegPerThread];
    const int mysum = region_bins(a, g0, rcnt, rst);
    int total;
    int rex[kRegPerThread];  // first region entry of this thread's bins
    {
        int ex = block_excl_scan<int, kBlock>(mysum, sh.w32, &total);
#pragma unroll
        for (int h = 0; h < kRegPerThread; ++h) {
            const int rb = kRegPerThread * threadIdx.x + h;
            rex[h] = ex;
            if (rb < a.nregion) sh.rp[rb] = ex;
            ex += rcnt[h];
        }
        if (threadIdx.x == 0) sh.rp[a.nregion] = total;
    }
    __syncthreads();
    const int nchunks = (total + kCap - 1) / kCap;
    // Quarter-bin row ends (QS: count pass, lower-triangular cell; a one-chunk region whose
    // bins are ordered by bin_xkey): staging packs into each rp word, above its 20-bit first
    // entry, the number of the bin's entries whose key lies below each of its quarter
    // boundaries (3 x 4 bits; 15: 15 or more), and a row then starts at the quarter of its
    // first bin that the cutoff reaches and ends after the quarter of its last.
    // Entries cut off this way lie beyond the padded cutoff along x alone, so they are never
    // edges: every target's edge sequence is unchanged (the fix-up pass, which sweeps whole
    // bins, numbers edges alike).
    static_assert(kCap < (1 << 20), "a one-chunk region's first entries fit the rp word's 20 bits");
    const bool qsplit = QS != 0 && nchunks == 1 && a.totals[4] == 0;
    XKey xkey;
    xkey.hbx = a.hbx; xkey.hcx = a.hcx; xkey.hcy = a.hcy; xkey.inv_hby = a.inv_hby; xkey.inv_hcz = a.inv_hcz;
    const int rpm = qsplit ? 0xFFFFF : -1;  // first-entry bits of an rp word
    const float qb1 = 0.25f * a.hax, qb2 = 0.5f * a.hax, qb3 = 0.75f * a.hax;
    // slots hold up to two chunks' entries (2-byte byte offsets in the region); a larger
    // region is written directly by search_kernel<1>
    // (the write pass follows what the count pass recorded: a tile it flagged as chunked --
    // a region of more than two chunks, or a count that kept no slots -- is swept again)
    const bool slotted = nchunks <= 2 && a.slot != nullptr && !(WRITE && (a.tfix[ord] & kFixChunked));
    int loaded = -1;

    // packed (image shift of region bin rb - floor of cell-list entry gidx)
    auto entry_T = [&](int rb, int gidx) -> uint32_t {
        const uint32_t fl = a.sflr[gidx];
        const int r[3] = {rb % R0, (rb / R0) % R1, rb / (R0 * R1)};
        int sb[3];
#pragma unroll
        for (int d = 0; d < 3; ++d) {
            const int gg = g0[d] - a.P[d] + r[d];
            sb[d] = a.pbc[d] ? floor_div(gg, a.nb[d]) : 0;
        }
        return pack3(sb[0] - unpack3(fl, 0), sb[1] - unpack3(fl, 1), sb[2] - unpack3(fl, 2));
    };
    // every thread copies the entries of its own region bins that fall in chunk c
    auto load_chunk = [&](int c) {
        const int c0 = c * kCap;
        const int c1 = min(total, c0 + kCap);
#pragma unroll
        for (int h = 0; h < kRegPerThread; ++h) {
            const int rb = kRegPerThread * threadIdx.x + h;
            const int b0 = max(rex[h], c0), b1 = min(rex[h] + rcnt[h], c1);
            if (b0 >= b1) continue;
            const int r[3] = {rb % R0, (rb / R0) % R1, rb / (R0 * R1)};
            float o[3];
            region_offset(a, r[0], r[1], r[2], o);
            const int g = rst[h] - rex[h];  // cell-list index minus region index
            int s1 = 0, s2 = 0, s3 = 0;  // entries below the quarter boundaries
            for (int vv = b0; vv < b1; vv += 4) {
                float4 e[4];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (vv + u < b1) e[u] = a.spos[g + vv + u];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (vv + u < b1) {
                        shq[vv + u - c0] = make_float4(e[u].x + o[0], e[u].y + o[1], e[u].z + o[2], e[u].w);
                        if constexpr (WRITE) sh.T[vv + u - c0] = entry_T(rb, g + vv + u);
                        if constexpr (QS != 0) {
                            const float xk = QS == 1 ? e[u].x : bin_xkey(e[u], xkey);
                            s1 += xk < qb1;
                            s2 += xk < qb2;
                            s3 += xk < qb3;
                        }
                    }
            }
            if (QS != 0 && qsplit)  // (one chunk: [b0, b1) is the whole bin)
                sh.rp[rb] = rex[h] | (int)((uint32_t)(min(s1, 15) | (min(s2, 15) << 4) | (min(s3, 15) << 8)) << 20);
        }
    };
    auto ensure_chunk = [&](int c) {  // uniform
        if (loaded != c) {
            __syncthreads();
            load_chunk(c);
            __syncthreads();
            loaded = c;
        }
    };

    const int nrx = 2 * a.P[0] + 1, nry = 2 * a.P[1] + 1, nrz = 2 * a.P[2] + 1;
    int64_t tile_found = 0;
    bool over_any = false;

    for (int k0 = 0; k0 < ntg; k0 += kBlock) {
        const int nbatch = min(kBlock, ntg - k0);
        const int kk = k0 + threadIdx.x;
        const int j = tbeg + kk;
        const bool in_batch = (int)threadIdx.x < nbatch;
        bool active = in_batch;

        // ---- per-lane target state
        int lx = 0, ly = 0, lz = 0, my_id = 0, caller = 0, v_self = -1;
        uint32_t my_f = 0;
        float t0 = 0.f, t1 = 0.f, t2 = 0.f, ux = 0.f, uy = 0.f, uz = 0.f;
        if (active) {
            int lo = 0, hi = a.tb;
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (sh.tbs[mid] <= j) lo = mid; else hi = mid;
            }
            lx = lo % a.T[0];
            ly = (lo / a.T[0]) % a.T[1];
            lz = lo / (a.T[0] * a.T[1]);
            const int sidx = listed ? a.tsidx[j] : j;
            const float4 e = a.spos[sidx];
            my_f = a.sflr[sidx];
            my_id = __float_as_int(e.w);
            caller = listed ? a.tslot[j] : my_id;
            active = !masked || my_id < a.ntarg;  // (masked: a ghost atom's lane idles)
            ux = e.x; uy = e.y; uz = e.z;  // position inside its own bin
            float o[3];
            region_offset(a, lx + a.P[0], ly + a.P[1], lz + a.P[2], o);
            t0 = e.x + o[0]; t1 = e.y + o[1]; t2 = e.z + o[2];
            // the target's own region entry (same atom, zero shift) is never an edge
            const int rb_self = ((lz + a.P[2]) * R1 + (ly + a.P[1])) * R0 + (lx + a.P[0]);
            const int bin_start = listed ? a.bstart[kb + lo] : sh.tbs[lo];
            v_self = (sh.rp[rb_self] & rpm) + (sidx - bin_start);
        }
        const int fx = unpack3(my_f, 0), fy = unpack3(my_f, 1), fz = unpack3(my_f, 2);
        // the target's position inside its bin in bin units (lower-triangular cells)
        // (reciprocals and the hardware square root below: their few-ulp errors are far
        // inside the trimming margin pmargin)
        const float Oz = uz * a.inv_hcz, Oy = (uy - Oz * a.hcy) * a.inv_hby,
                    Ox = (ux - Oy * a.hbx - Oz * a.hcx) * a.inv_hax;
        const float Oxp = Ox + (float)a.P[0];  // (orthorhombic rows: x bins from the region's first)
        const float Oxp4 = 4.f * Oxp, inv_hax4 = 4.f * a.inv_hax;  // in quarter bins (exact scalings)

        // Sweep this lane's target over the resident chunk c, in the fixed order (dz, dy,
        // x, atom) -- ascending region index; on_cand(v, edge, k) receives every candidate's
        // byte offset in the chunk (16 x its chunk-local region index), whether it is an
        // edge, and twice the running neighbour
        // number, k2 = 2 k (k: the edge's number when it is one); on_step(k2) follows every
        // step of two candidates, on_row(k2) every row.
        //
        // Rows are swept with one row of lookahead: the wave stays on row r until every
        // lane has finished its row r, and a lane that finishes early goes on into its row
        // r + 1 meanwhile, so a wave waits for its longest row less often.
        int found2 = 0;  // twice the neighbours found so far
        // (QS 1: rprune2 - gz^2 of the layer oz = gz_oz, kept while the rows of one z
        // layer go by; gz_oz is uniform)
        float gzz = 0.f;
        int gz_oz = -1;
        // candidate range [va, vb) of row ri (oz * nry + oy) of this lane, chunk-local;
        // empty when the padded cutoff sphere misses the row
        auto row_range = [&](int ri, int c0, int c1, int& va, int& vb) {
            const int oz = ri / nry, oy = ri - oz * nry;
            int xlo = 0, xhi = nrx - 1;
            int qlo = 0, qhi = 3;  // first and last quarter of the end bins
            va = vb = 0;
            if (QS == 1 || (QS == 0 && a.lowtri == 2)) {
                // orthorhombic: the row's bins span y in [py, py + 1] hby and z in
                // [pz, pz + 1] hcz around the target; their gaps (less the margin) bound the
                // distance from below, and the x range follows without shear
                const float py = (float)(oy - a.P[1]) - Oy;
                const float gy = fmaxf(fmaxf(fmaf(py, a.hby, -a.pmargin), fmaf(-py, a.hby, a.gy_off)), 0.f);
                float rem2;
                if constexpr (QS == 1) {
                    if (oz != gz_oz) {
                        const float pz = (float)(oz - a.P[2]) - Oz;
                        const float gz = fmaxf(fmaxf(fmaf(pz, a.hcz, -a.pmargin), fmaf(-pz, a.hcz, a.gz_off)), 0.f);
                        gzz = fmaf(-gz, gz, a.rprune2);
                        gz_oz = oz;
                    }
                    rem2 = fmaf(-gy, gy, gzz);
                } else {
                    const float pz = (float)(oz - a.P[2]) - Oz;
                    const float gz = fmaxf(fmaxf(fmaf(pz, a.hcz, -a.pmargin), fmaf(-pz, a.hcz, a.gz_off)), 0.f);
                    rem2 = fmaf(-gz, gz, fmaf(-gy, gy, a.rprune2));
                }
                if (rem2 < 0.f) return;
                const float rem = __builtin_amdgcn_sqrtf(rem2);
                if constexpr (QS == 1) {
                    // (4 floor(u) + quarter = floor(4 u): the bins are those of floor(u))
                    const int QL = max((int)floorf(fmaf(-rem, inv_hax4, Oxp4)), 0);
                    const int QH = min((int)floorf(fmaf(rem, inv_hax4, Oxp4)), 4 * nrx - 1);
                    xlo = QL >> 2;
                    xhi = QH >> 2;
                    if (xlo > xhi) return;
                    if (qsplit) {
                        qlo = QL & 3;
                        qhi = QH & 3;
                    }
                } else {
                    xlo = max((int)floorf(fmaf(-rem, a.inv_hax, Oxp)), 0);
                    xhi = min((int)floorf(fmaf(rem, a.inv_hax, Oxp)), nrx - 1);
                    if (xlo > xhi) return;
                }
            } else if (QS == 2 || (QS == 0 && a.lowtri)) {
                // bounding box of the row (bins py, pz relative to the target's bin, all x)
                // in Cartesian y and z, from the target: its gaps gy, gz bound the distance
                // from below; the x range that the (padded) cutoff sphere can reach then
                // follows from the row's x shear
                const float py = (float)(oy - a.P[1]) - Oy, pz = (float)(oz - a.P[2]) - Oz;
                const float zl = pz * a.hcz, zh = zl + a.hcz;
                const float cyl = fminf(pz * a.hcy, (pz + 1.f) * a.hcy);
                const float cyh = fmaxf(pz * a.hcy, (pz + 1.f) * a.hcy);
                const float yl = py * a.hby + cyl, yh = (py + 1.f) * a.hby + cyh;
                float gy = fmaxf(fmaxf(yl, -yh), 0.f), gz = fmaxf(fmaxf(zl, -zh), 0.f);
                gy = fmaxf(gy - a.pmargin, 0.f);
                gz = fmaxf(gz - a.pmargin, 0.f);
                const float rem2 = a.rprune2 - gy * gy - gz * gz;
                if (rem2 < 0.f) return;
                const float rem = __builtin_amdgcn_sqrtf(rem2);
                const float sl = fminf(py * a.hbx, (py + 1.f) * a.hbx) + fminf(pz * a.hcx, (pz + 1.f) * a.hcx);
                const float sh = fmaxf(py * a.hbx, (py + 1.f) * a.hbx) + fmaxf(pz * a.hcx, (pz + 1.f) * a.hcx);
                if constexpr (QS == 2) {
                    // in quarter bins, as the orthorhombic rows: an entry of the first bin
                    // whose a fraction is below u - xlo lies at least rem below the target
                    // in x (its shear is at most sh), one of the last bin at or above
                    // w - xhi at least rem above it (its shear is at least sl)
                    const int QL = max((int)floorf(4.f * (Ox + (-rem - sh) * a.inv_hax)) + 4 * a.P[0], 0);
                    const int QH = min((int)floorf(4.f * (Ox + (rem - sl) * a.inv_hax)) + 4 * a.P[0], 4 * nrx - 1);
                    xlo = QL >> 2;
                    xhi = QH >> 2;
                    if (xlo > xhi) return;
                    if (qsplit) {
                        qlo = QL & 3;
                        qhi = QH & 3;
                    }
                } else {
                    xlo = max((int)floorf(Ox + (-rem - sh) * a.inv_hax) + a.P[0], 0);
                    xhi = min((int)floorf(Ox + (rem - sl) * a.inv_hax) + a.P[0], nrx - 1);
                    if (xlo > xhi) return;
                }
            }
            const int rb = ((lz + oz) * R1 + (ly + oy)) * R0 + lx;
            int sa, sb;
            if (QS != 0 && qsplit) {  // (wave-uniform)
                // (all three words read unconditionally: a select, not a branch)
                const uint32_t wl = (uint32_t)sh.rp[rb + xlo], wh = (uint32_t)sh.rp[rb + xhi],
                               we = (uint32_t)sh.rp[rb + xhi + 1];
                sa = (int)(wl & 0xFFFFFu) + (int)((wl >> (16 + 4 * qlo)) & (qlo ? 15u : 0u));
                const int ch = (int)((wh >> (20 + 4 * min(qhi, 2))) & 15u);
                sb = (int)((qhi < 3 && ch != 15 ? wh + (uint32_t)ch : we) & 0xFFFFFu);
            } else {
                sa = sh.rp[rb + xlo];
                sb = sh.rp[rb + xhi + 1];
            }
            va = max(sa, c0) - c0;
            vb = min(sb, c1) - c0;
            if (va >= vb) va = vb = 0;
            va <<= 4;  // byte offsets of the 16-byte entries
            vb <<= 4;
        };
        auto sweep = [&](int c, auto&& on_cand, auto&& on_step, auto&& on_row) {
            const int c0 = c * kCap;
            const int c1 = min(total, c0 + kCap);
            const int vs = (v_self - c0) << 4;
            const int nrows = nrz * nry;
            const char* const qb = (const char*)shq;
            // Candidates are addressed by the byte offset of their 16-byte entry in shq.
            // [v, e): this lane's unswept part of its current row; [pv, pe): its next row,
            // pv == pe once the lane has moved on to it (an empty or missing next row is
            // [16, 0) until then).  A lane moves on to its next row the step it finishes its
            // current one, so when the wave leaves row ri every lane is on its row ri + 1.
            int v, e, pv, pe;
            row_range(0, c0, c1, v, e);
            if (!active) v = e = 0;
            for (int ri = 0; ri < nrows; ++ri) {
                pv = 0; pe = 0;
                if (ri + 1 < nrows && active) row_range(ri + 1, c0, c1, pv, pe);
                if (pv == pe) { pv = 16; pe = 0; }
                if (v >= e) { v = pv; e = pe; pv = pe; }  // nothing left of row ri
                // two candidates per step, both loads issued first (the second may be one
                // past the range -- at most the sentinel -- and is then masked); the edge
                // test is branch-free, the rare exact test sits behind a scalar mask test,
                // and on_cand sees every candidate in order
                if (__builtin_amdgcn_ballot_w64(pv != pe) != 0ull) do {
                    const float4 q0 = *(const float4*)(qb + v), q1 = *(const float4*)(qb + v + 16);
                    const bool in0 = v < e, in1 = v + 16 < e;
                    // d2 - toff with the offset in the innermost fma; edge iff its bits are
                    // below lo_bits (0 <= d2' < lo_off), band iff d2' <= hi_off
                    float dx = q0.x - t0, dyv = q0.y - t1, dzv = q0.z - t2;
                    const float d20 = fmaf(dzv, dzv, fmaf(dyv, dyv, fmaf(dx, dx, -a.toff)));
                    dx = q1.x - t0; dyv = q1.y - t1; dzv = q1.z - t2;
                    const float d21 = fmaf(dzv, dzv, fmaf(dyv, dyv, fmaf(dx, dx, -a.toff)));
                    bool e0 = in0 & (__float_as_uint(d20) < a.lo_bits);
                    bool e1 = in1 & (__float_as_uint(d21) < a.lo_bits);
                    const bool b0 = in0 & !e0 & (d20 <= a.hi_off) & (v != vs);
                    const bool b1 = in1 & !e1 & (d21 <= a.hi_off) & (v + 16 != vs);
                    if (__builtin_expect(b0 | b1, 0)) {  // divergent: the mask test is scalar
                        if (b0)
                            e0 = exact_edge(a, __float_as_int(q0.w), my_id, (double)q0.x - t0,
                                            (double)q0.y - t1, (double)q0.z - t2);
                        if (b1)
                            e1 = exact_edge(a, __float_as_int(q1.w), my_id, (double)q1.x - t0,
                                            (double)q1.y - t1, (double)q1.z - t2);
                    }
                    // (a candidate past the range is no edge: k does not advance)
                    on_cand(v, e0, found2);
                    found2 += e0 ? 2 : 0;
                    on_cand(v + 16, e1, found2);
                    found2 += e1 ? 2 : 0;
                    on_step(found2);
                    // range done: from row ri on to the next row, from that one to rest (at
                    // v = e: masked loads of entries e and e + 1, inside LDS)
                    // (a lane already on its next row that finishes it takes [pe, pe): empty)
                    const int nv = v + 32;
                    const bool fin = nv >= e;
                    v = fin ? pv : nv;
                    e = fin ? pe : e;
                    pv = fin ? pe : pv;
                } while (__builtin_amdgcn_ballot_w64(pv != pe) != 0ull);
                on_row(found2);
            }
        };
        auto none = [](int) {};

        if constexpr (!WRITE) {
            // ---------------- count pass
            // Slot entries are staged in a per-lane LDS ring of 16: the entry of slot k is
            // written for every candidate (an edge keeps it: k advances), and full groups
            // of 8 go out to the slot at the end of each row -- or within the row, before
            // the ring could wrap onto a group not yet stored.
            // this lane's ring: byte lane_off of sh.lb (its low five bits clear, so an entry's
            // byte address is lane_off | (k2 & 30), one bitwise VALU)
            static_assert(2 * kRing == 32, "ring of 16 two-byte entries per lane");
            char* const lb0 = (char*)&sh.lb[0][0];
            const uint32_t lane_off = threadIdx.x << 5;
            char* const lbb = lb0 + lane_off;
            const bool slots = slotted;
            char* const slotb = (char*)a.slot;
            const uint64_t gstep = 16ull * (uint64_t)a.nslot;  // bytes between a target's groups
            uint64_t goff = 16ull * (uint64_t)j;                // byte offset of group kf2 / 16
            int kf2 = 0;                                      // 2 x entries stored (or skipped)
            int klim = 2 * kRing - 4;                         // kf2 + 28: the in-row flush mark
            const int K2 = 2 * a.K;
            auto store_group = [&]() {  // the group starting at entry kf2 / 2
                if (kf2 + 16 <= K2) *(uint4*)(slotb + goff) = *(const uint4*)(lbb + (kf2 & 16));
                kf2 += 16;
                klim += 16;
                goff += gstep;
            };
            auto flush = [&](int k2) {  // every full group below entry k2 / 2
                while (kf2 + 16 <= k2) store_group();
            };
            for (int c = 0; c < nchunks; ++c) {
                ensure_chunk(c);
                if (!active) continue;
                if (slots) {
                    auto on_step = [&](int k2) {
                        // k2 - kf2 <= 32 here: at most two groups to store
                        if (k2 > klim) {
                            store_group();
                            if (k2 - kf2 >= 16) store_group();
                        }
                    };
                    auto on_row = [&](int k2) { flush(k2); };
                    // slot entries are byte offsets in the whole region: chunk 1's entries
                    // follow chunk 0's kCap
                    if (c == 0)
                        sweep(c, [&](int v, bool, int k2) {
                                  *(uint16_t*)(lb0 + ring_at(k2, lane_off)) = (uint16_t)v;
                              }, on_step, on_row);
                    else
                        sweep(c, [&](int v, bool, int k2) {
                                  *(uint16_t*)(lb0 + ring_at(k2, lane_off)) = (uint16_t)(v + 16 * kCap);
                              }, on_step, on_row);
                } else {
                    sweep(c, [&](int, bool, int) {}, none, none);
                }
            }
            const int found = found2 >> 1;
            if (active) {
                if (slots) {
                    flush(found2);
                    if ((found & 7) && found < a.K) *(uint4*)(slotb + goff) = *(const uint4*)(lbb + (kf2 & 16));
                }
                a.cnt[j] = found;
                if (a.counts_user) a.counts_user[caller] = found;
                tile_found += found;
                over_any = over_any || found > a.K;
            } else if (in_batch) {
                a.cnt[j] = 0;  // (masked: a ghost, no edges)
            }
            __syncthreads();
            continue;
        }

        if constexpr (WRITE) {
        // ---------------- write pass
        const int mycnt = active ? a.cnt[j] : 0;
        int btot;
        const int ex = block_excl_scan<int, kBlock>(mycnt, sh.w32, &btot);
        if (slotted) {
            // targets with more than K neighbours: the rest by a second sweep (over both
            // chunks of a two-chunk region, k counting on as in the count pass)
            const bool over = active && mycnt > a.K;
            if (block_any<kBlock>(over, sh.w32)) {
                const int64_t base = ebase + ex;
                for (int c = 0; c < nchunks; ++c) {
                    ensure_chunk(c);
                    if (over)
                        sweep(c, [&](int vb, bool e, int k2) {
                            const int k = k2 >> 1, v = vb >> 4;
                            if (e && k >= a.K && k < mycnt) {
                                const uint32_t Tp = sh.T[v];
                                emit_edge(a, base + k, __float_as_int(shq[v].w), my_id,
                                          unpack3(Tp, 0) + fx, unpack3(Tp, 1) + fy, unpack3(Tp, 2) + fz);
                            }
                        }, none, none);
                }
            }
        } else {
            // chunked region (very dense tiles): sweep and write directly
            const int64_t base = ebase + ex;
            for (int c = 0; c < nchunks; ++c) {
                ensure_chunk(c);
                if (!active) continue;
                sweep(c, [&](int vb, bool e, int k2) {
                    const int k = k2 >> 1, v = vb >> 4;
                    if (e && k < mycnt) {
                        const uint32_t Tp = sh.T[v];
                        emit_edge(a, base + k, __float_as_int(shq[v].w), my_id,
                                  unpack3(Tp, 0) + fx, unpack3(Tp, 1) + fy, unpack3(Tp, 2) + fz);
                    }
                }, none, none);
            }
        }
        ebase += btot;
        }
        __syncthreads();
    }

    if (!WRITE) {
        int64_t tt;
        block_excl_scan<int64_t, kBlock>(tile_found, sh.w64, &tt);
        const bool over = block_any<kBlock>(over_any, sh.w32);
        const int fix = (over ? kFixOver : 0) | (slotted ? (nchunks == 2 ? kFix2 : 0) : kFixChunked);
        out.tt = tt;
        out.fix = fix;
        if (MODE == 0 && threadIdx.x == 0) {
            a.ttot[ord] = (int)tt;
            a.tfix[ord] = fix;
            if (fix && flag_clear(&a.totals[3]))  // the fix-up pass has work
                atomicOr((unsigned long long*)&a.totals[3], 1ull);
        }
    }
    return out;
}

// Writes every edge the count pass left in the slots of tile ord (output order), from a
// region staged for up to CAP entries: kCap for most tiles (expand_kernel), 2 kCap for the
// two-chunk tiles (inside search_kernel<1>).
// VT: the type of the edge vectors / distances written in 16-byte groups from *vsp (void:
// none, or written per lane).
template <int CAP, typename VT = void>
__device__ __forceinline__ void expand_one(const SearchArgs& a, typename ExpandLdsOf<CAP>::type& sh,
                                           int64_t ord, void* vsp = nullptr)
{
    const int64_t rank = xcd_tile_rank(ord, a.ntiles);
    const int* tstart = listed_targets(a) ? a.tbstart : a.bstart;
    const int64_t kb = rank * a.tb;
    const int tbeg = tstart[kb], tend = tstart[kb + a.tb];
    const int ntg = tend - tbeg;
    if (ntg == 0 || a.ttot[ord] == 0) return;  // (no edges: nothing to expand)
    const int64_t ebase = a.tbase[ord];
    if (ebase + a.ttot[ord] > a.capacity) {
        if (threadIdx.x == 0)
            atomicOr((unsigned long long*)&a.totals[1], (unsigned long long)kStatusCapacity);
        return;
    }
    const int lin = a.tile_of_rank[rank];
    const int g0[3] = {(lin % a.ntl[0]) * a.T[0], ((lin / a.ntl[0]) % a.ntl[1]) * a.T[1],
                       (lin / (a.ntl[0] * a.ntl[1])) * a.T[2]};
    // region entries: cell-list indices (grouped vectors), the ids to write (the plain
    // path, which needs no positions), or atom indices (the per-lane path)
    if constexpr (!std::is_void<VT>::value) {
        stage_pairs<CAP, true>(a, sh, g0);
        expand_tile<true, CAP, VT, kVecIlp>(a, sh, tbeg, ntg, ebase, vsp);
    } else if (!a.out_vec && !a.out_dist) {
        stage_pairs<CAP, false, true>(a, sh, g0);
        expand_tile<true, CAP>(a, sh, tbeg, ntg, ebase);
    } else {
        stage_pairs<CAP>(a, sh, g0);
        expand_tile<false, CAP>(a, sh, tbeg, ntg, ebase);
    }
}

// MODE 0 (count) and MODE 1 (fix-up write): one tile per workgroup.  The fix-up also
// expands the slots of the two-chunk tiles (their region needs the larger staging buffer).
// QS: the count with quarter-bin row ends (1: orthorhombic cells, 2: other lower-triangular
// cells; cell list ordered by bin_xkey).
template <int MODE, int QS = 0>
__global__ __launch_bounds__(kBlock) void search_kernel(SearchArgs a)
{
    if constexpr (MODE == 0) {
        __shared__ CountLds sh;
        search_tile<0, QS>(a, sh, blockIdx.x);
    } else {
        __shared__ union {
            FixLds f;
            Expand2Lds e;
        } u;
        // a grid of at most DG_FIXGRID workgroups walks the tiles: most have nothing to do,
        // and in most builds no tile has (the count pass raises totals[3] when one does)
        if (a.totals[3] == 0) return;
        for (int64_t ord = blockIdx.x; ord < a.ntiles; ord += gridDim.x) {
            const int fix = a.tfix[ord];
            if (fix == 0) continue;
            if (fix & kFix2) {
                expand_one<2 * kCap>(a, u.e, ord);
                __syncthreads();
            }
            search_tile<1>(a, u.f, ord);
            __syncthreads();  // before the next tile reuses the LDS
        }
    }
}

#if DG_MAIN_TU
// the count kernel's launcher, compiled in dg_count.hip
void launch_count_kernel(const SearchArgs& a, unsigned grid, hipStream_t s);

// Writes every edge held in the count pass's slots, one workgroup per tile (the write
// stage of the two-stage build; tiles whose region needs two LDS chunks are expanded by
// search_kernel<1>, larger ones written by it directly).
// The positions in cell-list order (entry g: atom sid[g]), for the edge vectors: the
// expansion then reads a tile's sources from a few contiguous runs instead of from all
// over the caller's order.
__global__ void cell_pos_kernel(int64_t n, const int* __restrict__ sid, const void* __restrict__ pos,
                                int f64, void* __restrict__ cpos)
{
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n) return;
    const int64_t i = sid[g];
    if (f64) {
        const double* ps = (const double*)pos + 3 * i;
        double* pc = (double*)cpos + 3 * g;
        pc[0] = ps[0]; pc[1] = ps[1]; pc[2] = ps[2];
    } else {
        const float* ps = (const float*)pos + 3 * i;
        float* pc = (float*)cpos + 3 * g;
        pc[0] = ps[0]; pc[1] = ps[1]; pc[2] = ps[2];
    }
}

// VT: void without vector / distance outputs, else their type.
template <typename VT>
__global__ __launch_bounds__(kBlock) void expand_kernel(SearchArgs a)
{
    // Tiles in reverse output order: the count stage wrote the slots in output order, so the
    // last tiles' slots are the likeliest still in the memory-side cache when this kernel
    // starts (C5 write stage 2.78 -> 2.70 ms, a uniform 1.25M-atom box 0.87 -> 0.82 ms).
    // Each tile still writes its own output range.
    const int64_t ord = (int64_t)gridDim.x - 1 - blockIdx.x;
    if (a.tfix[ord] & (kFixChunked | kFix2)) return;
    if constexpr (std::is_void<VT>::value) {
        __shared__ ExpandLds sh;
        expand_one<kCap>(a, sh, ord);
    } else {
        __shared__ ExpandVLds<VT> sh;
        expand_one<kCap, VT>(a, sh, ord, &sh.vs);
    }
}

// ---------------------------------------------------------------- all-pairs fallback
// Used only when the search region of a tile would exceed kMaxRegion bins (cutoff much
// larger than the cell).  One thread per target, every atom, and for each pair every
// periodic shift that can put the source within the cutoff (brute_kernel: the exact
// per-pair range).
struct BruteArgs {
    double C[9], Cinv[9];
    double r2;
    double cf[3];  // r / face distance per axis: the fractional reach of the cutoff sphere
    int pbc[3];
    const void* pos;
    int f64;
    int64_t n, nt;
    const int64_t* tgt;
    int* cnt;
    int* counts_user;
    const int64_t* offs;
    int64_t* out_src;
    int64_t* out_dst;
    float* out_shift;
    void* out_vec;
    void* out_dist;
    int vout_f64;
    int64_t capacity;
    int64_t* totals;
    const int64_t* out_ids;  // written for atom i: out_ids[i] (null: i)
};

template <bool WRITE>
__global__ void brute_kernel(BruteArgs a)
{
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= a.nt) return;
    int64_t tg = a.tgt ? a.tgt[t] : t;
    if (tg < 0 || tg >= a.n) {
        atomicOr((unsigned long long*)&a.totals[1], (unsigned long long)DG_FLAG_TARGET);
        if (!WRITE) { a.cnt[t] = 0; if (a.counts_user) a.counts_user[t] = 0; }
        return;
    }
    double pt[3], frt[3];
    load_pos(a.pos, a.f64, tg, pt);
    for (int d = 0; d < 3; ++d) frt[d] = canon_frac(pt[0], pt[1], pt[2], a.Cinv, d);
    int64_t o = WRITE ? a.offs[t] : 0;
    if (WRITE && a.offs[t + 1] > a.capacity) {
        atomicOr((unsigned long long*)&a.totals[1], (unsigned long long)kStatusCapacity);
        return;
    }
    int found = 0;
    for (int64_t j = 0; j < a.n; ++j) {
        double ps[3];
        load_pos(a.pos, a.f64, j, ps);
        // an edge's shift is its periodic image plus the floor difference of the two atoms
        // (radius_graph_kernels.cu:282-303); on a periodic axis every S with
        // |frt - frs - S| <= cf can be one (the source image is at least that fractional
        // distance times the face distance from the target), widened by 1e-9 against
        // rounding; without PBC only the floor difference
        int lo[3], hi[3];
        for (int d = 0; d < 3; ++d) {
            const double frs = canon_frac(ps[0], ps[1], ps[2], a.Cinv, d);
            if (a.pbc[d]) {
                lo[d] = (int)ceil(frt[d] - frs - a.cf[d] - 1e-9);
                hi[d] = (int)floor(frt[d] - frs + a.cf[d] + 1e-9);
            } else {
                lo[d] = hi[d] = (int)floor(frt[d]) - (int)floor(frs);
            }
        }
        for (int s0 = lo[0]; s0 <= hi[0]; ++s0)
            for (int s1 = lo[1]; s1 <= hi[1]; ++s1)
                for (int s2 = lo[2]; s2 <= hi[2]; ++s2) {
                    double v[3];
                    double d2 = canon_d2(ps, pt, s0, s1, s2, a.C, v);
                    if (!(d2 > kSelfThr && d2 <= a.r2)) continue;
                    if (WRITE) {
                        int64_t e = o + found;
                        a.out_src[e] = a.out_ids ? a.out_ids[j] : j;
                        a.out_dst[e] = a.out_ids ? a.out_ids[tg] : tg;
                        a.out_shift[3 * e] = (float)s0;
                        a.out_shift[3 * e + 1] = (float)s1;
                        a.out_shift[3 * e + 2] = (float)s2;
                        if (a.out_vec) {
                            if (a.vout_f64) {
                                double* ov = (double*)a.out_vec + 3 * e;
                                ov[0] = v[0]; ov[1] = v[1]; ov[2] = v[2];
                            } else {
                                float* ov = (float*)a.out_vec + 3 * e;
                                ov[0] = (float)v[0]; ov[1] = (float)v[1]; ov[2] = (float)v[2];
                            }
                        }
                        if (a.out_dist) {
                            if (a.vout_f64) ((double*)a.out_dist)[e] = sqrt(d2);
                            else ((float*)a.out_dist)[e] = (float)sqrt(d2);
                        }
                    }
                    ++found;
                }
    }
    if (!WRITE) {
        a.cnt[t] = found;
        if (a.counts_user) a.counts_user[t] = found;
    }
}

// ---------------------------------------------------------------- small utilities
__global__ void zero_i32_kernel(int* __restrict__ p, int64_t n)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

__global__ void zero_i64_kernel(int64_t* __restrict__ p, int64_t n)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

inline unsigned nblocks(int64_t n, int b = 256) { return (unsigned)((n + b - 1) / b); }

template <typename T>
inline T* at(void* ws, size_t off)
{
    return (T*)((char*)ws + off);
}

dg_status check_launch(const char* what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail(DG_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
    return DG_OK;
}

// Opt-in stage timer: with RADIUS_PBC_PROFILE set in the environment (the switch of
// radius_graph_kernels.cu:444-465), a count or write call records a HIP event on its
// stream at every stage boundary, waits for the last one and prints each stage's time to
// stderr.  Off (the default) it does nothing: no events, no synchronisation.
struct StageTimer {
    static constexpr int kMax = 8;
    hipEvent_t ev[kMax];
    const char* name[kMax];
    int n = 0;
    bool on;
    hipStream_t s;
    explicit StageTimer(hipStream_t st) : on(getenv("RADIUS_PBC_PROFILE") != nullptr), s(st) {}
    // marks the end of stage `what` (the first mark opens the clock)
    void mark(const char* what)
    {
        if (!on || n >= kMax) return;
        if (hipEventCreate(&ev[n]) != hipSuccess) { on = false; return; }
        (void)hipEventRecord(ev[n], s);
        name[n++] = what;
    }
    void report(const char* call, const Plan& p, int64_t capacity)
    {
        if (!on || n < 2) { release(); return; }
        (void)hipEventSynchronize(ev[n - 1]);
        float total = 0;
        fprintf(stderr, "[radius_graph_pbc profile] %s: N=%lld targets=%lld bins=%dx%dx%d tiles=%lld "
                        "(%dx%dx%d bins) K=%d%s", call, (long long)p.n, (long long)p.nt, p.nb[0], p.nb[1],
                p.nb[2], (long long)p.ntiles, p.T[0], p.T[1], p.T[2], p.K, p.brute ? " all-pairs" : "");
        if (capacity >= 0) fprintf(stderr, " edge capacity=%lld", (long long)capacity);
        fprintf(stderr, "\n");
        for (int i = 1; i < n; ++i) {
            float ms = 0;
            (void)hipEventElapsedTime(&ms, ev[i - 1], ev[i]);
            total += ms;
            fprintf(stderr, "  %-22s %8.3f ms\n", name[i], ms);
        }
        fprintf(stderr, "  %-22s %8.3f ms\n", "total", total);
        release();
    }
    void release()
    {
        for (int i = 0; i < n; ++i) (void)hipEventDestroy(ev[i]);
        n = 0;
    }
    ~StageTimer() { release(); }
};

// Validates the description and builds the plan (host only).
dg_status make_plan(const dg_graph_desc* d, Plan& p)
{
    if (!d) return fail(DG_ERR_INVALID, "desc is NULL");
    if (d->n_atoms < 0 || d->n_atoms > 0x7ffffff0LL)
        return fail(DG_ERR_INVALID, "n_atoms must be in [0, 2^31)");
    if (d->has_targets && (d->n_targets < 0 || d->n_targets > 0x7ffffff0LL))
        return fail(DG_ERR_INVALID, "n_targets must be in [0, 2^31)");
    if (d->pos_dtype != DG_F32 && d->pos_dtype != DG_F64)
        return fail(DG_ERR_INVALID, "pos must be float32 or float64");
    if (!(d->radius > 0.0) || !isfinite(d->radius))
        return fail(DG_ERR_INVALID, "radius must be positive, got " + std::to_string(d->radius));
    for (int k = 0; k < 9; ++k)
        if (!isfinite(d->cell[k])) return fail(DG_ERR_INVALID, "cell must be finite");
    p = Plan();
    p.n = d->n_atoms;
    p.subset = d->has_targets ? 1 : 0;
    p.nt = d->has_targets ? d->n_targets : d->n_atoms;
    p.f64 = d->pos_dtype == DG_F64;
    if (plan_geometry(p, d->cell, d->pbc, d->radius)) return fail(DG_ERR_INVALID, "cell is singular");
    if (!(pair_images(p.cf, p.pbc) <= kMaxPairImages))
        return fail(DG_ERR_INVALID, "cell too thin for the radius: more than 2^24 periodic images per atom pair");
    plan_grid(p);
    plan_layout(p);
    if (p.nbins >= 0x7fffffffLL || p.ncodes >= 0x7fffffffLL)
        return fail(DG_ERR_INVALID, "grid too large");
    return DG_OK;
}

// 2: orthorhombic cell; 1: other lower-triangular cell (a along x, b in the xy plane,
// positive diagonal); 0: any other.
int cell_shape(const Plan& p)
{
    const bool low = p.C[1] == 0.0 && p.C[2] == 0.0 && p.C[5] == 0.0 && p.C[0] > 0.0 && p.C[4] > 0.0 &&
                     p.C[8] > 0.0;
    if (!low) return 0;
    return p.C[3] == 0.0 && p.C[6] == 0.0 && p.C[7] == 0.0 ? 2 : 1;
}

// The bin steps bin_xkey needs, as the search's arguments hold them.
XKey xkey_of(const Plan& p)
{
    XKey k;
    k.hbx = (float)(p.C[3] / p.nb[1]);
    k.hcx = (float)(p.C[6] / p.nb[2]);
    k.hcy = (float)(p.C[7] / p.nb[2]);
    k.inv_hby = (float)(p.nb[1] / p.C[4]);
    k.inv_hcz = (float)(p.nb[2] / p.C[8]);
    return k;
}

GridArgs grid_args(const Plan& p)
{
    GridArgs g;
    memcpy(g.C, p.C, sizeof g.C);
    memcpy(g.Cinv, p.Cinv, sizeof g.Cinv);
    for (int d = 0; d < 3; ++d) {
        g.nb[d] = p.nb[d]; g.T[d] = p.T[d]; g.ntl[d] = p.ntl[d]; g.mb[d] = p.mb[d];
    }
    g.tb = p.tb;
    return g;
}

SearchArgs search_args(const Plan& p, const void* pos, void* ws)
{
    SearchArgs a;
    memset(&a, 0, sizeof a);
    memcpy(a.C, p.C, sizeof a.C);
    memcpy(a.Cinv, p.Cinv, sizeof a.Cinv);
    for (int d = 0; d < 3; ++d)
        for (int c = 0; c < 3; ++c) a.hC[3 * d + c] = p.C[3 * d + c] / (double)p.nb[d];
    a.r2 = p.r2;
    a.lowtri = cell_shape(p);
    a.hax = (float)(p.C[0] / p.nb[0]);
    a.hbx = (float)(p.C[3] / p.nb[1]);
    a.hby = (float)(p.C[4] / p.nb[1]);
    a.hcx = (float)(p.C[6] / p.nb[2]);
    a.hcy = (float)(p.C[7] / p.nb[2]);
    a.hcz = (float)(p.C[8] / p.nb[2]);
    a.inv_hax = (float)(p.nb[0] / p.C[0]);
    a.inv_hby = (float)(p.nb[1] / p.C[4]);
    a.inv_hcz = (float)(p.nb[2] / p.C[8]);
    // row trimming must never drop a candidate the exact test could accept: pad the
    // cutoff by far more than the fp32 position error
    a.pmargin = (float)(1e-4 * p.r + 1e-3);
    a.rprune2 = (float)((p.r + 2.0 * a.pmargin) * (p.r + 2.0 * a.pmargin));
    a.gy_off = -a.hby - a.pmargin;
    a.gz_off = -a.hcz - a.pmargin;
    for (int d = 0; d < 3; ++d) {
        a.nb[d] = p.nb[d]; a.P[d] = p.P[d]; a.T[d] = p.T[d]; a.ntl[d] = p.ntl[d];
        a.R[d] = p.R[d]; a.pbc[d] = p.pbc[d];
    }
    a.tb = p.tb;
    a.nregion = p.nregion;
    a.xsplit = p.ntiles <= kSortTilesMax;  // (the per-bin sort above keeps bins in id order)
    a.ntiles = p.ntiles;
    a.toff = p.toff; a.hi_off = p.hi_off; a.lo_bits = p.lo_bits;
    a.spos = at<float4>(ws, p.o_spos);
    a.sflr = at<uint32_t>(ws, p.o_sflr);
    a.sid = at<int>(ws, p.o_sid);
    a.bstart = at<int>(ws, p.o_bstart);
    a.tile_of_rank = at<int>(ws, p.o_tor);
    a.rank_of_tile = at<int>(ws, p.o_rot);
    a.pos = pos;
    a.f64 = p.f64;
    a.subset = p.subset;
    a.tbstart = at<int>(ws, p.o_tbstart);
    a.tsidx = at<int>(ws, p.o_tsidx);
    a.tslot = at<int>(ws, p.o_tslot);
    a.cnt = at<int>(ws, p.o_cnt);
    a.ttot = at<int>(ws, p.o_ttot);
    a.tfix = at<int>(ws, p.o_tfix);
    a.tbase = at<int64_t>(ws, p.o_tbase);
    a.totals = at<int64_t>(ws, p.o_tot);
    // slot rows: one per target, or per atom when the targets are the atoms with ids < nt
    // (every atom of a tile is then a lane)
    const int64_t nrow = p.nrow;
    a.slot = at<uint16_t>(ws, p.o_slot);
    a.K = p.K;
    a.nslot = nrow;
    a.align_max_edges = -1;  // (set by the write call, which knows the outputs)
    a.ntarg = p.nt;
    // the prefix test runs with the tile-level sort only (the per-bin fallback sorts the
    // explicit targets as listed)
    a.pmis = p.subset && p.ntiles <= kSortTilesMax ? at<int64_t>(ws, p.o_tot) + 2 : nullptr;
    return a;
}

BruteArgs brute_args(const Plan& p, const void* pos, const int64_t* tgt, void* ws)
{
    BruteArgs b;
    memset(&b, 0, sizeof b);
    memcpy(b.C, p.C, sizeof b.C);
    memcpy(b.Cinv, p.Cinv, sizeof b.Cinv);
    b.r2 = p.r2;
    for (int d = 0; d < 3; ++d) { b.pbc[d] = p.pbc[d]; b.cf[d] = p.cf[d]; }
    b.pos = pos;
    b.f64 = p.f64;
    b.n = p.n;
    b.nt = p.nt;
    b.tgt = p.subset ? tgt : nullptr;
    b.cnt = at<int>(ws, p.o_cnt);
    b.offs = at<int64_t>(ws, p.o_tbase);
    b.totals = at<int64_t>(ws, p.o_tot);
    return b;
}

// Dynamic LDS beyond the default 64 KiB for kernel fn (gfx950 allows up to 160 KiB per
// workgroup); the attribute is raised once per kernel and size.
static void allow_dyn_lds(const void* fn, size_t bytes)
{
    if (bytes <= 65536) return;
    static std::mutex mu;
    static std::vector<std::pair<const void*, size_t>> done;
    std::lock_guard<std::mutex> lock(mu);
    for (auto& d : done)
        if (d.first == fn && d.second >= bytes) return;
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) == hipSuccess)
        done.emplace_back(fn, bytes);
}

// Workgroups of sort_big_bins_kernel: about 1024 bins each, at most 2048.
static unsigned big_bins_grid(int64_t nbins)
{
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(2048, (nbins + 1023) / 1024));
}

// Steps 1-5 of a build: Morton tile ranks, counting sort of the atoms (and of the
// explicit targets) into the SFC-ordered cell list.
void launch_sort(const Plan& p, const void* pos, const int64_t* target_idx, void* ws,
                 int64_t* totals, hipStream_t s)
{
    GridArgs g = grid_args(p);
    int* bcnt = at<int>(ws, p.o_bcnt);
    int* bstart = at<int>(ws, p.o_bstart);
    if (p.ntiles <= kSortTilesMax) {
        // 1. Morton rank of the tiles (and cleared tile counts)
        int* tcnt = at<int>(ws, p.o_tcnt);
        int* tstart = at<int>(ws, p.o_tstart);
        int* wgb = at<int>(ws, p.o_wgb);
        hipLaunchKernelGGL(tile_rank_kernel, dim3((unsigned)std::min<int64_t>(nblocks(p.ntiles), 2048)),
                           dim3(256), 0, s, g, p.ntiles, at<int>(ws, p.o_tor), at<int>(ws, p.o_rot), tcnt,
                           p.ntiles, totals);
        // 2. wrap, bin key and cell-list record of every atom
        hipLaunchKernelGGL(bin_atoms_kernel, dim3(nblocks(p.n)), dim3(256), 0, s, g, pos, p.f64, p.n,
                           (const int*)at<int>(ws, p.o_rot), at<uint32_t>(ws, p.o_key),
                           (uint32_t*)nullptr, (int*)nullptr, at<float4>(ws, p.o_rec), totals);
        // 3-5. tile buckets, then each tile's bins in LDS
        const unsigned nch = (unsigned)std::max<int64_t>(1, std::min<int64_t>(kSortChunks, (p.n + 4095) / 4096));
        const size_t hl = 4 * (size_t)p.ntiles;
        allow_dyn_lds((const void*)tile_hist_kernel, hl);
        // 32-bit bucket entries when every id (atom, and target position) fits 24 bits
        const bool narrow = p.n < (1 << 24) && (!p.subset || p.nt < (1 << 24));
        allow_dyn_lds(narrow ? (const void*)tile_scatter_kernel<uint32_t> : (const void*)tile_scatter_kernel<uint64_t>, hl);
        const int64_t* always = nullptr;
        hipLaunchKernelGGL(tile_hist_kernel, dim3(nch), dim3(1024), hl, s, p.n, p.tb, p.ntiles,
                           (const uint32_t*)at<uint32_t>(ws, p.o_key), tcnt, wgb, always);
        if (narrow)
            hipLaunchKernelGGL(tile_scatter_kernel<uint32_t>, dim3(nch), dim3(1024), hl, s, p.n, p.tb, p.ntiles,
                               (const uint32_t*)at<uint32_t>(ws, p.o_key), (const int*)tcnt, tstart,
                               (const int*)wgb, at<uint32_t>(ws, p.o_arr), always);
        else
            hipLaunchKernelGGL(tile_scatter_kernel<uint64_t>, dim3(nch), dim3(1024), hl, s, p.n, p.tb, p.ntiles,
                               (const uint32_t*)at<uint32_t>(ws, p.o_key), (const int*)tcnt, tstart,
                               (const int*)wgb, at<uint64_t>(ws, p.o_arr), always);
        TileSortOut o;
        memset(&o, 0, sizeof o);
        o.rec = at<float4>(ws, p.o_rec);
        o.spos = at<float4>(ws, p.o_spos);
        o.sflr = at<uint32_t>(ws, p.o_sflr);
        o.sid = at<int>(ws, p.o_sid);
        o.inv = p.subset ? at<int>(ws, p.o_inv) : (int*)nullptr;
        o.stmp = at<void>(ws, p.o_stmp);
        o.xflag = totals + 4;
        o.xorder = cell_shape(p) != 0;  // (the count cuts bins by x in lower-triangular cells)
        o.xk = xkey_of(p);
        if (narrow)
            hipLaunchKernelGGL((tile_sort_kernel<false, uint32_t>), dim3((unsigned)p.ntiles), dim3(256), 0, s, p.n,
                               p.tb, p.ntiles, (const int*)tstart, at<uint32_t>(ws, p.o_arr), bstart, o);
        else
            hipLaunchKernelGGL((tile_sort_kernel<false, uint64_t>), dim3((unsigned)p.ntiles), dim3(256), 0, s, p.n,
                               p.tb, p.ntiles, (const int*)tstart, at<uint64_t>(ws, p.o_arr), bstart, o);
        if (p.subset) {
            // the explicit targets through the same tile-level sort: keyed by their atom's
            // bin, ordered by caller position inside a bin -- unless they are exactly
            // 0 .. nt - 1 (target_prefix_kernel leaves totals[2] at 0): then the kernels below
            // exit at once and the count takes the atoms of each tile with ids < nt
            hipLaunchKernelGGL(target_prefix_kernel, dim3((unsigned)std::min<int64_t>(nblocks(p.nt), 2048)), dim3(256),
                               0, s, p.nt, p.n, target_idx, totals);
            const int64_t* listed = totals + 2;
            uint32_t* tkey = at<uint32_t>(ws, p.o_tkey);
            hipLaunchKernelGGL(target_keys_kernel, dim3((unsigned)std::min<int64_t>(nblocks(std::max(p.nt, p.ntiles)), 4096)),
                               dim3(256), 0, s, p.nt, p.n, target_idx, (const uint32_t*)at<uint32_t>(ws, p.o_key),
                               tkey, tcnt, p.ntiles, totals);
            const unsigned tch = (unsigned)std::max<int64_t>(1, std::min<int64_t>(kSortChunks, (p.nt + 4095) / 4096));
            hipLaunchKernelGGL(tile_hist_kernel, dim3(tch), dim3(1024), hl, s, p.nt, p.tb, p.ntiles,
                               (const uint32_t*)tkey, tcnt, wgb, listed);
            if (narrow)
                hipLaunchKernelGGL(tile_scatter_kernel<uint32_t>, dim3(tch), dim3(1024), hl, s, p.nt, p.tb, p.ntiles,
                                   (const uint32_t*)tkey, (const int*)tcnt, tstart, (const int*)wgb,
                                   at<uint32_t>(ws, p.o_tarr), listed);
            else
                hipLaunchKernelGGL(tile_scatter_kernel<uint64_t>, dim3(tch), dim3(1024), hl, s, p.nt, p.tb, p.ntiles,
                                   (const uint32_t*)tkey, (const int*)tcnt, tstart, (const int*)wgb,
                                   at<uint64_t>(ws, p.o_tarr), listed);
            TileSortOut ot;
            memset(&ot, 0, sizeof ot);
            ot.inv = at<int>(ws, p.o_inv);
            ot.tgt = target_idx;
            ot.natoms = p.n;
            ot.tslot = at<int>(ws, p.o_tslot);
            ot.tsidx = at<int>(ws, p.o_tsidx);
            ot.run_if = listed;
            ot.stmp = at<void>(ws, p.o_stmp);
            if (narrow)
                hipLaunchKernelGGL((tile_sort_kernel<true, uint32_t>), dim3((unsigned)p.ntiles), dim3(256), 0, s,
                                   p.nt, p.tb, p.ntiles, (const int*)tstart,
                                   at<uint32_t>(ws, p.o_tarr), at<int>(ws, p.o_tbstart), ot);
            else
                hipLaunchKernelGGL((tile_sort_kernel<true, uint64_t>), dim3((unsigned)p.ntiles), dim3(256), 0, s,
                                   p.nt, p.tb, p.ntiles, (const int*)tstart,
                                   at<uint64_t>(ws, p.o_tarr), at<int>(ws, p.o_tbstart), ot);
        }
        return;
    } else {
    // 1. Morton rank of the tiles (and cleared bin counts)
    hipLaunchKernelGGL(tile_rank_kernel, dim3((unsigned)std::min<int64_t>(nblocks(p.nbins), 2048)), dim3(256),
                       0, s, g, p.ntiles, at<int>(ws, p.o_tor), at<int>(ws, p.o_rot), bcnt, p.nbins, totals);
    // 2-5. counting sort of the atoms into SFC-ordered bins (per-bin device atomics)
    hipLaunchKernelGGL(bin_atoms_kernel, dim3(nblocks(p.n)), dim3(256), 0, s, g, pos, p.f64, p.n,
                       (const int*)at<int>(ws, p.o_rot), at<uint32_t>(ws, p.o_key),
                       at<uint32_t>(ws, p.o_rank), bcnt, at<float4>(ws, p.o_rec), totals);
    device_excl_scan<int, int>(bcnt, p.nbins, bstart, at<int>(ws, p.o_part), s);
    hipLaunchKernelGGL(scatter_atoms_kernel, dim3(nblocks(p.n)), dim3(256), 0, s, p.n,
                       (const uint32_t*)at<uint32_t>(ws, p.o_key),
                       (const uint32_t*)at<uint32_t>(ws, p.o_rank), (const int*)bstart,
                       at<int>(ws, p.o_arr));
    hipLaunchKernelGGL(sort_big_bins_kernel, dim3(big_bins_grid(p.nbins)), dim3(kSegSortThreads), 0, s, p.nbins,
                       (const int*)bstart, at<uint32_t>(ws, p.o_arr), at<uint32_t>(ws, p.o_stmp));
    hipLaunchKernelGGL(order_atoms_kernel, dim3(nblocks(p.n)), dim3(256), 0, s, p.n,
                       (const uint32_t*)at<uint32_t>(ws, p.o_key), (const int*)bstart,
                       (const int*)at<int>(ws, p.o_arr), (const float4*)at<float4>(ws, p.o_rec),
                       at<float4>(ws, p.o_spos), at<uint32_t>(ws, p.o_sflr), at<int>(ws, p.o_sid),
                       p.subset ? at<int>(ws, p.o_inv) : (int*)nullptr);
    }
    if (p.subset) {
        int* tbcnt = at<int>(ws, p.o_tbcnt);
        int* tbstart = at<int>(ws, p.o_tbstart);
        hipLaunchKernelGGL(zero_i32_kernel, dim3(nblocks(p.nbins)), dim3(256), 0, s, tbcnt, p.nbins);
        hipLaunchKernelGGL(bin_targets_kernel, dim3(nblocks(p.nt)), dim3(256), 0, s, p.nt, p.n,
                           target_idx, (const uint32_t*)at<uint32_t>(ws, p.o_key),
                           at<uint32_t>(ws, p.o_tkey), at<uint32_t>(ws, p.o_trank), tbcnt, totals);
        device_excl_scan<int, int>(tbcnt, p.nbins, tbstart, at<int>(ws, p.o_part), s);
        hipLaunchKernelGGL(scatter_targets_kernel, dim3(nblocks(p.nt)), dim3(256), 0, s, p.nt,
                           (const uint32_t*)at<uint32_t>(ws, p.o_tkey),
                           (const uint32_t*)at<uint32_t>(ws, p.o_trank), (const int*)tbstart,
                           at<int>(ws, p.o_tslot));
        hipLaunchKernelGGL(sort_big_bins_kernel, dim3(big_bins_grid(p.nbins)), dim3(kSegSortThreads), 0, s,
                           p.nbins, (const int*)tbstart, at<uint32_t>(ws, p.o_tslot), at<uint32_t>(ws, p.o_stmp));
        hipLaunchKernelGGL(finish_targets_kernel, dim3(nblocks(p.nbins)), dim3(256), 0, s, p.nbins,
                           p.n, (const int*)tbstart, at<int>(ws, p.o_tslot), target_idx,
                           (const int*)at<int>(ws, p.o_inv), at<int>(ws, p.o_tsidx));
    }
}

#else   // DG_COUNT_TU
void launch_count_kernel(const SearchArgs& a, unsigned grid, hipStream_t s)
{
    if (a.lowtri == 2 && a.xsplit)
        hipLaunchKernelGGL((search_kernel<0, 1>), dim3(grid), dim3(kBlock), 0, s, a);
    else if (a.lowtri == 1 && a.xsplit)
        hipLaunchKernelGGL((search_kernel<0, 2>), dim3(grid), dim3(kBlock), 0, s, a);
    else
        hipLaunchKernelGGL((search_kernel<0, 0>), dim3(grid), dim3(kBlock), 0, s, a);
}
#endif  // DG_MAIN_TU

}  // namespace dg

using namespace dg;

#if DG_MAIN_TU
extern "C" {

const char* dg_last_error(void) { return g_last_error.c_str(); }

const char* dg_version(void) { return "dynamis_graph 0.1 gfx950"; }

size_t dg_graph_workspace_size(const dg_graph_desc* desc)
{
    Plan p;
    if (make_plan(desc, p) != DG_OK) return 0;
    return p.ws_bytes;
}

// The count stage; without slots (counts only) the sweep records no neighbour lists, and a
// dg_graph_write that follows writes every tile from its fix-up pass instead.
static dg_status count_stage(const dg_graph_desc* desc, const void* pos, const int64_t* target_idx,
                             void* ws, size_t ws_bytes, int32_t* counts_out, bool slots, hipStream_t s)
{
    Plan p;
    dg_status st = make_plan(desc, p);
    if (st != DG_OK) return st;
    if (!ws || ws_bytes < p.ws_bytes) return fail(DG_ERR_WORKSPACE, "workspace too small");
    if (p.n > 0 && !pos) return fail(DG_ERR_INVALID, "pos is NULL");
    if (p.subset && p.nt > 0 && !target_idx) return fail(DG_ERR_INVALID, "target_idx is NULL");
    g_last_error.clear();
    int64_t* totals = at<int64_t>(ws, p.o_tot);
    if (p.n == 0 || p.nt == 0 || p.brute)  // (else tile_rank_kernel clears them)
        hipLaunchKernelGGL(zero_i64_kernel, dim3(1), dim3(64), 0, s, totals, (int64_t)8);
    if (p.n == 0 || p.nt == 0) {
        if (counts_out && p.nt > 0)
            hipLaunchKernelGGL(zero_i32_kernel, dim3(nblocks(p.nt)), dim3(256), 0, s, counts_out, p.nt);
        return check_launch("dg_graph_count(empty)");
    }
    if (p.brute) {
        BruteArgs b = brute_args(p, pos, target_idx, ws);
        b.counts_user = counts_out;
        hipLaunchKernelGGL(brute_kernel<false>, dim3(nblocks(p.nt, 64)), dim3(64), 0, s, b);
        excl_scan<int, int64_t>(at<int>(ws, p.o_cnt), p.nt, at<int64_t>(ws, p.o_tbase),
                                at<int64_t>(ws, p.o_part), s, totals);
        return check_launch("dg_graph_count(brute)");
    }
    StageTimer clk(s);
    clk.mark("start");
    launch_sort(p, pos, target_idx, ws, totals, s);
    clk.mark("sfc reorder + sort");
    // 6. degrees
    SearchArgs a = search_args(p, pos, ws);
    a.counts_user = counts_out;
    if (!slots) a.slot = nullptr;
    launch_count_kernel(a, (unsigned)p.ntiles, s);
    clk.mark("count");
    // 7. tile offsets in output order, and the total
    excl_scan<int, int64_t>(at<int>(ws, p.o_ttot), p.ntiles, at<int64_t>(ws, p.o_tbase),
                            at<int64_t>(ws, p.o_part), s, totals);
    clk.mark("tile offset scan");
    st = check_launch("dg_graph_count");
    clk.report("dg_graph_count", p, -1);
    return st;
}

dg_status dg_graph_count(const dg_graph_desc* desc, const void* pos, const int64_t* target_idx,
                         void* ws, size_t ws_bytes, int32_t* counts_out, hipStream_t s)
{
    return count_stage(desc, pos, target_idx, ws, ws_bytes, counts_out, true, s);
}

dg_status dg_graph_counts(const dg_graph_desc* desc, const void* pos, const int64_t* target_idx,
                          void* ws, size_t ws_bytes, int32_t* counts_out, hipStream_t s)
{
    return count_stage(desc, pos, target_idx, ws, ws_bytes, counts_out, false, s);
}

dg_status dg_graph_read_totals(const dg_graph_desc* desc, const void* ws, int64_t* total_edges,
                               int64_t* flags, hipStream_t s)
{
    Plan p;
    dg_status st = make_plan(desc, p);
    if (st != DG_OK) return st;
    // a small pinned buffer per host thread (allocated on its first call, kept): the copy
    // then goes straight to it instead of through a pageable staging path
    thread_local int64_t* pinned = nullptr;
    if (!pinned && hipHostMalloc((void**)&pinned, 2 * sizeof(int64_t), hipHostMallocDefault) != hipSuccess) {
        pinned = nullptr;
        (void)hipGetLastError();  // (the pageable fallback below; no stale error for later checks)
    }
    int64_t hbuf[2] = {0, 0};
    int64_t* h = pinned ? pinned : hbuf;
    h[0] = h[1] = 0;
    hipError_t e = hipMemcpyAsync(h, at<int64_t>((void*)ws, p.o_tot), 2 * sizeof(int64_t), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail(DG_ERR_HIP, std::string("read totals: ") + hipGetErrorString(e));
    if (total_edges) *total_edges = h[0];
    if (flags) *flags = h[1];
    if (h[1] & (DG_FLAG_RANGE | DG_FLAG_NONFINITE | DG_FLAG_TARGET)) {
        std::string m;
        if (h[1] & DG_FLAG_NONFINITE) m += "pos contains non-finite values; ";
        if (h[1] & DG_FLAG_RANGE) m += "an atom lies more than 255 cell lengths outside the cell; ";
        if (h[1] & DG_FLAG_TARGET) m += "target_indices out of range [0, N); ";
        return fail(DG_ERR_RANGE, m);
    }
    if (h[1] & DG_FLAG_CAPACITY) return fail(DG_ERR_CAPACITY, "edge capacity exceeded");
    return DG_OK;
}

dg_status dg_graph_write_ids(const dg_graph_desc* desc, const void* pos, const int64_t* target_idx,
                             void* ws, size_t ws_bytes, int64_t capacity, const int64_t* out_ids,
                             int64_t* edge_src, int64_t* edge_dst, float* cell_shift, void* edge_vec,
                             void* edge_dist, int32_t vec_dtype, hipStream_t s)
{
    Plan p;
    dg_status st = make_plan(desc, p);
    if (st != DG_OK) return st;
    if (!ws || ws_bytes < p.ws_bytes) return fail(DG_ERR_WORKSPACE, "workspace too small");
    if (vec_dtype != DG_F32 && vec_dtype != DG_F64) return fail(DG_ERR_INVALID, "vec_dtype");
    if (capacity < 0) return fail(DG_ERR_INVALID, "capacity < 0");
    g_last_error.clear();
    if (p.n == 0 || p.nt == 0 || capacity == 0) return DG_OK;
    if (!edge_src || !edge_dst || !cell_shift) return fail(DG_ERR_INVALID, "edge outputs are NULL");
    if (!pos) return fail(DG_ERR_INVALID, "pos is NULL");
    if (p.subset && !target_idx) return fail(DG_ERR_INVALID, "target_idx is NULL");
    if (p.brute) {
        BruteArgs b = brute_args(p, pos, target_idx, ws);
        b.out_src = edge_src; b.out_dst = edge_dst; b.out_shift = cell_shift;
        b.out_vec = edge_vec; b.out_dist = edge_dist; b.vout_f64 = vec_dtype == DG_F64;
        b.capacity = capacity;
        b.out_ids = out_ids;
        hipLaunchKernelGGL(brute_kernel<true>, dim3(nblocks(p.nt, 64)), dim3(64), 0, s, b);
        return check_launch("dg_graph_write(brute)");
    }
    SearchArgs a = search_args(p, pos, ws);
    a.out_src = edge_src; a.out_dst = edge_dst; a.out_shift = cell_shift;
    a.out_vec = edge_vec; a.out_dist = edge_dist; a.vout_f64 = vec_dtype == DG_F64;
    a.capacity = capacity;
    a.out_ids = out_ids;
    {
        const double slot_bytes = 2.0 * (double)p.K * (double)a.nslot;
        const double bpe = 28.0 + (edge_vec ? (vec_dtype == DG_F64 ? 24.0 : 12.0) : 0.0) +
                           (edge_dist ? (vec_dtype == DG_F64 ? 8.0 : 4.0) : 0.0);
        const double room = kAlignBudget - slot_bytes;
        a.align_max_edges = room > 0 ? (int64_t)(room / (kAlignOutShare * bpe)) : -1;
    }
    StageTimer clk(s);
    clk.mark("start");
    // vectors / distances go out in 16-byte groups from bases aligned to 16 bytes, else
    // every edge is written by its lane
    const bool vec = edge_vec || edge_dist;
    const bool vec16 = vec && (((uintptr_t)edge_vec | (uintptr_t)edge_dist) & 15u) == 0;
    if (vec16) {
        a.cpos = at<char>(ws, p.o_cpos);
        hipLaunchKernelGGL(cell_pos_kernel, dim3(nblocks(p.n, 256)), dim3(256), 0, s, (int64_t)p.n,
                           (const int*)a.sid, pos, p.f64, (void*)a.cpos);
    }
    if (vec16 && a.vout_f64)
        hipLaunchKernelGGL(expand_kernel<double>, dim3((unsigned)p.ntiles), dim3(kBlock), 0, s, a);
    else if (vec16)
        hipLaunchKernelGGL(expand_kernel<float>, dim3((unsigned)p.ntiles), dim3(kBlock), 0, s, a);
    else
        hipLaunchKernelGGL(expand_kernel<void>, dim3((unsigned)p.ntiles), dim3(kBlock), 0, s, a);
    clk.mark("write (slot expansion)");
    hipLaunchKernelGGL(search_kernel<1>, dim3((unsigned)std::min<int64_t>(p.ntiles, kFixGrid)), dim3(kBlock), 0, s, a);
    clk.mark("write (fix-up)");
    st = check_launch("dg_graph_write");
    clk.report("dg_graph_write", p, capacity);
    return st;
}

dg_status dg_graph_write(const dg_graph_desc* desc, const void* pos, const int64_t* target_idx,
                         void* ws, size_t ws_bytes, int64_t capacity, int64_t* edge_src,
                         int64_t* edge_dst, float* cell_shift, void* edge_vec, void* edge_dist,
                         int32_t vec_dtype, hipStream_t s)
{
    return dg_graph_write_ids(desc, pos, target_idx, ws, ws_bytes, capacity, nullptr, edge_src, edge_dst,
                              cell_shift, edge_vec, edge_dist, vec_dtype, s);
}

dg_status dg_graph_build(const dg_graph_desc* desc, const void* pos, const int64_t* target_idx,
                         void* ws, size_t ws_bytes, int64_t capacity, int32_t* counts_out,
                         int64_t* edge_src, int64_t* edge_dst, float* cell_shift, void* edge_vec,
                         void* edge_dist, int32_t vec_dtype, hipStream_t s)
{
    // the write pass reads only device-side results of the count pass (per-tile offsets,
    // slots), so the two run back to back with no host round trip
    dg_status st = dg_graph_count(desc, pos, target_idx, ws, ws_bytes, counts_out, s);
    if (st != DG_OK) return st;
    return dg_graph_write(desc, pos, target_idx, ws, ws_bytes, capacity, edge_src, edge_dst,
                          cell_shift, edge_vec, edge_dist, vec_dtype, s);
}

}  // extern "C"

// ---------------------------------------------------------------- allocation-free build
// A device-resident workspace for dg_graph_build_noalloc: the build's whole workspace
// (cell list, slots, tile tables, totals) lives in this array, one copy per GPU, held from
// the library's load until the process ends.  Host code never names the array itself (its
// host-side symbol is no device address): it uses the address hipGetSymbolAddress
// returns on each device, kept in g_scratch_ptr.
namespace dg {
constexpr size_t kScratchBytes = (size_t)64 << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];
// Overlap guard, per device: the stream of the last call and an event recorded behind it.
// A call on another stream while that event is still pending would share the scratch with
// work in flight, and is refused.  (Created once per device, with the scratch lookup.)
// A call holds its device's array (busy) from the check until its work is enqueued, so two
// host threads cannot both pass the check.
static hipEvent_t g_scratch_done[kMaxDevices];
static hipStream_t g_scratch_stream[kMaxDevices];
static bool g_scratch_used[kMaxDevices];
static bool g_scratch_busy[kMaxDevices];

// The scratch address on the current device, looked up once per device, and the device's
// array taken for this call (*dev_out; give it back with scratch_release).
// The stream must belong to the current device: the address is that device's copy.
static dg_status scratch_on_current_device(hipStream_t s, void** out, int* dev_out)
{
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(DG_ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(DG_ERR_INVALID, "device ordinal out of range");
    if (s != nullptr) {
        hipDevice_t sdev = -1;
        e = hipStreamGetDevice(s, &sdev);
        if (e != hipSuccess) return fail(DG_ERR_HIP, std::string("hipStreamGetDevice: ") + hipGetErrorString(e));
        if (sdev != dev)
            return fail(DG_ERR_INVALID, "dg_graph_build_noalloc: the stream belongs to device " +
                                            std::to_string(sdev) + ", the current device is " + std::to_string(dev));
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(DG_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        e = hipEventCreateWithFlags(&g_scratch_done[dev], hipEventDisableTiming);
        if (e != hipSuccess)
            return fail(DG_ERR_HIP, std::string("hipEventCreateWithFlags: ") + hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    // A stream under capture records no completion to test: such calls are not guarded.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (s != nullptr) {
        e = hipStreamIsCapturing(s, &cap);
        if (e != hipSuccess) return fail(DG_ERR_HIP, std::string("hipStreamIsCapturing: ") + hipGetErrorString(e));
    }
    if (g_scratch_busy[dev])
        return fail(DG_ERR_INVALID, "dg_graph_build_noalloc: another call on this device is being enqueued "
                                    "(calls share the static scratch and must not overlap)");
    if (cap == hipStreamCaptureStatusNone && g_scratch_used[dev] && g_scratch_stream[dev] != s) {
        e = hipEventQuery(g_scratch_done[dev]);
        if (e == hipErrorNotReady)
            return fail(DG_ERR_INVALID, "dg_graph_build_noalloc: the previous call on this device (on another "
                                        "stream) has not completed; calls on different streams share the static "
                                        "scratch and must not overlap");
        if (e != hipSuccess) return fail(DG_ERR_HIP, std::string("hipEventQuery: ") + hipGetErrorString(e));
    }
    g_scratch_busy[dev] = true;
    *out = g_scratch_ptr[dev];
    *dev_out = dev;
    return DG_OK;
}

// Gives back device dev's array after a call on stream s: records the overlap guard's event
// behind whatever the call enqueued (not on a stream under capture).
static dg_status scratch_release(int dev, hipStream_t s)
{
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (s != nullptr && hipStreamIsCapturing(s, &cap) != hipSuccess) cap = hipStreamCaptureStatusActive;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    g_scratch_busy[dev] = false;
    if (cap != hipStreamCaptureStatusNone) return DG_OK;
    const hipError_t e = hipEventRecord(g_scratch_done[dev], s);
    if (e != hipSuccess) return fail(DG_ERR_HIP, std::string("hipEventRecord: ") + hipGetErrorString(e));
    g_scratch_stream[dev] = s;
    g_scratch_used[dev] = true;
    return DG_OK;
}

// Copies the build's {edge count, flags} to the caller's device buffer.
__global__ void copy_totals_kernel(const int64_t* __restrict__ totals, int64_t* __restrict__ out)
{
    if (threadIdx.x < 2) out[threadIdx.x] = totals[threadIdx.x];
}
}  // namespace dg

extern "C" dg_status dg_graph_build_noalloc(const dg_graph_desc* desc, const void* pos,
                                            const int64_t* target_idx, int64_t capacity,
                                            int32_t* counts_out, int64_t* edge_src,
                                            int64_t* edge_dst, float* cell_shift, void* edge_vec,
                                            void* edge_dist, int32_t vec_dtype,
                                            int64_t* totals_out, hipStream_t s)
{
    Plan p;
    dg_status st = make_plan(desc, p);
    if (st != DG_OK) return st;
    if (!totals_out) return fail(DG_ERR_INVALID, "totals_out is NULL");
    if (p.ws_bytes > kScratchBytes)
        return fail(DG_ERR_WORKSPACE, "dg_graph_build_noalloc: this build needs " +
                                          std::to_string(p.ws_bytes) + " bytes of workspace; the static "
                                          "scratch holds " + std::to_string(kScratchBytes) +
                                          " (use dg_graph_build with a caller workspace)");
    void* ws = nullptr;
    int dev = -1;
    st = scratch_on_current_device(s, &ws, &dev);
    if (st != DG_OK) return st;
    st = dg_graph_build(desc, pos, target_idx, ws, kScratchBytes, capacity, counts_out, edge_src,
                        edge_dst, cell_shift, edge_vec, edge_dist, vec_dtype, s);
    if (st == DG_OK) {
        hipLaunchKernelGGL(copy_totals_kernel, dim3(1), dim3(64), 0, s,
                           (const int64_t*)at<int64_t>(ws, p.o_tot), totals_out);
        st = check_launch("dg_graph_build_noalloc");
    }
    // (also after a failed call: whatever it enqueued still uses the array)
    const std::string err = st != DG_OK ? g_last_error : std::string();
    const dg_status rs = scratch_release(dev, s);
    if (st != DG_OK) {
        g_last_error = err;
        return st;
    }
    return rs;
}
#endif  // DG_MAIN_TU
