// dg_sfc.hip -- SFC keys, stable LSD radix sort and partition labels for gfx950, plus the
// order-preserving edge filter.  C ABI in include/dynamis_graph.h.
//
// Keys follow dynamis_state/src/csrc/partition/sfc_kernels.cu:
//   bounds  :196-198   pos_min = min over atoms, range = max - min (0 -> 1), fp32
//   Morton  :32-56     21-bit quantisation (p - min) / range * (2^21 - 1), clamp, interleave
//                      with x at bit 0 (fp32 arithmetic)
//   Hilbert :62-109    order-7 quantisation with the reference's per-bit transform
//   labels  :114-173   unweighted closed form / exact int64 weighted cut
// The sort replaces at::sort (sfc_kernels.cu:224) with a stable 8-bit LSD radix sort that
// skips, on the device, the bytes in which all keys agree.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/dynamis_graph.h"
#include "dg_common.hpp"
#include "dg_lookback.hpp"
#include "dg_scan.hpp"

namespace dg {
dg_status fail(dg_status st, const std::string& msg);
}

namespace {
using namespace dg;


inline size_t al(size_t x) { return (x + 255) & ~(size_t)255; }
inline unsigned nblk(int64_t n, int b = 256) { return (unsigned)((n + b - 1) / b); }

// ------------------------------------------------------------------ bounds
__global__ void bounds_partial_kernel(const float* __restrict__ pos, int64_t n,
                                      float* __restrict__ part)
{
    __shared__ float s_mn[3][256], s_mx[3][256];
    float mn[3] = {INFINITY, INFINITY, INFINITY}, mx[3] = {-INFINITY, -INFINITY, -INFINITY};
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        for (int a = 0; a < 3; ++a) {
            float v = pos[3 * i + a];
            mn[a] = fminf(mn[a], v);
            mx[a] = fmaxf(mx[a], v);
        }
    for (int a = 0; a < 3; ++a) { s_mn[a][threadIdx.x] = mn[a]; s_mx[a][threadIdx.x] = mx[a]; }
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o)
            for (int a = 0; a < 3; ++a) {
                s_mn[a][threadIdx.x] = fminf(s_mn[a][threadIdx.x], s_mn[a][threadIdx.x + o]);
                s_mx[a][threadIdx.x] = fmaxf(s_mx[a][threadIdx.x], s_mx[a][threadIdx.x + o]);
            }
        __syncthreads();
    }
    if (threadIdx.x == 0)
        for (int a = 0; a < 3; ++a) {
            part[6 * blockIdx.x + a] = s_mn[a][0];
            part[6 * blockIdx.x + 3 + a] = s_mx[a][0];
        }
}

// One workgroup of 256 threads folds the nb <= 1024 partial bounds (min and max are exact,
// so the result does not depend on the order).
__global__ __launch_bounds__(256) void bounds_final_kernel(const float* __restrict__ part, int nb,
                                                           float* __restrict__ out)
{
    __shared__ float s_mn[3][256], s_mx[3][256];
    float mn[3] = {INFINITY, INFINITY, INFINITY}, mx[3] = {-INFINITY, -INFINITY, -INFINITY};
    for (int b = threadIdx.x; b < nb; b += 256)
        for (int a = 0; a < 3; ++a) {
            mn[a] = fminf(mn[a], part[6 * b + a]);
            mx[a] = fmaxf(mx[a], part[6 * b + 3 + a]);
        }
    for (int a = 0; a < 3; ++a) { s_mn[a][threadIdx.x] = mn[a]; s_mx[a][threadIdx.x] = mx[a]; }
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o)
            for (int a = 0; a < 3; ++a) {
                s_mn[a][threadIdx.x] = fminf(s_mn[a][threadIdx.x], s_mn[a][threadIdx.x + o]);
                s_mx[a][threadIdx.x] = fmaxf(s_mx[a][threadIdx.x], s_mx[a][threadIdx.x + o]);
            }
        __syncthreads();
    }
    if (threadIdx.x == 0)
        for (int a = 0; a < 3; ++a) {
            const float rg = s_mx[a][0] - s_mn[a][0];
            out[a] = s_mn[a][0];
            out[3 + a] = rg > 0.0f ? rg : 1.0f;
        }
}

// ------------------------------------------------------------------ keys
// Spread the low 21 bits of v to every third bit (standard magic-mask bit interleave).
__device__ __forceinline__ uint64_t spread21(uint32_t v)
{
    uint64_t x = v & 0x1fffffu;
    x = (x | (x << 32)) & 0x001f00000000ffffull;
    x = (x | (x << 16)) & 0x001f0000ff0000ffull;
    x = (x | (x << 8)) & 0x100f00f00f00f00full;
    x = (x | (x << 4)) & 0x10c30c30c30c30c3ull;
    x = (x | (x << 2)) & 0x1249249249249249ull;
    return x;
}

__global__ void keys_kernel(const float* __restrict__ pos, int64_t n, int curve,
                            const float* __restrict__ bnd, int64_t* __restrict__ keys)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float u[3];
    for (int a = 0; a < 3; ++a) u[a] = (pos[3 * i + a] - bnd[a]) / bnd[3 + a];
    if (curve == 0) {
        const uint32_t gm = (1u << 21) - 1;
        uint32_t q[3];
        for (int a = 0; a < 3; ++a) {
            uint32_t t = (uint32_t)(u[a] * (float)gm);
            q[a] = t < gm ? t : gm;
        }
        keys[i] = (int64_t)(spread21(q[0]) | (spread21(q[1]) << 1) | (spread21(q[2]) << 2));
    } else {
        const int gm = 127;
        int c[3];
        for (int a = 0; a < 3; ++a) {
            int t = (int)(u[a] * (float)gm);
            c[a] = t < 0 ? 0 : (t > gm ? gm : t);
        }
        int64_t r = 0;
        for (int b = 0; b < 7; ++b) {
            int xb = (c[0] >> b) & 1, yb = (c[1] >> b) & 1, zb = (c[2] >> b) & 1;
            int nx = xb, ny = yb, nz = zb;
            if (b > 0) {
                // per-bit rule of sfc_kernels.cu:94-101
                nx = xb ? zb : 0;
                ny = xb ? yb : (yb ? zb : 0);
                nz = xb ? yb : (yb ? xb : (zb ? yb : 0));
            }
            r |= ((int64_t)nx << (3 * b)) | ((int64_t)ny << (3 * b + 1)) | ((int64_t)nz << (3 * b + 2));
        }
        keys[i] = r;
    }
}

// ------------------------------------------------------------------ radix sort
// Stable LSD radix sort, 8 bits per pass, with no host synchronisation, so a call is a
// fixed sequence of launches that a HIP graph can capture:
//   rs_span_kernel       the OR and AND of the keys, per workgroup;
//   rs_plan_kernel       one workgroup: the pass plan -- a byte in which every key has the
//                        same digit is skipped (its kernels exit at once), the first pass
//                        that runs reads the caller's keys, the last writes the int64
//                        permutation;
//   per byte q = 0..7:
//     rs_hist_kernel<q>  each tile's digit counts, digit-major (hist[d * ntiles + t]);
//     device scan of hist (digit-major: each tile's output base per digit)
//     rs_pass_kernel<q>  each tile ranks its keys stably by digit (eight ballots per 64
//                        keys and per-wave running counts) and writes each digit's run
//                        contiguously through LDS: keys and int32 positions, or, in the last
//                        pass, the int64 permutation.
// Keys are kept with the sign bit flipped inside the sort (so they order as unsigned).
constexpr int kRsBlock = 256;
// 8 keys per thread (2048-key tiles, about two workgroups per CU at 1M keys): 1M Morton
// keys in 0.205 ms, against 0.216 ms at 4, 0.208 ms at 6 and 0.246 ms at 16 keys per thread
// (the scatter is latency-bound; smaller tiles put more of them in flight)
constexpr int kRsPer = 8;                      // keys per thread
constexpr int kRsTile = kRsBlock * kRsPer;     // keys per tile
constexpr int kRsWaveKeys = 64 * kRsPer;       // a wave's contiguous share of a tile
constexpr int kRsPasses = 8;
constexpr int kRsSpanBlocks = 512;             // workgroups of the key span (at most)

__device__ __forceinline__ uint64_t ukey(int64_t k) { return (uint64_t)k ^ 0x8000000000000000ull; }
__device__ __forceinline__ int digit_of(uint64_t k, int shift) { return (int)((k >> shift) & 0xffu); }

// What pass q does (written by rs_plan_kernel): run = 0 skips it; src / dst: 0 the
// caller's keys, 1 and 2 the two key / position buffers, 3 the permutation.
struct RsPass {
    int run, src, dst, pad;
};
struct RsCtl {
    RsPass pass[kRsPasses];
    int none;  // every key equal: the permutation is the identity
};

// OR and AND of the (sign-flipped) keys: one pair per workgroup.
__global__ __launch_bounds__(256) void rs_span_kernel(const int64_t* __restrict__ keys, int64_t n,
                                                      unsigned long long* __restrict__ part)
{
    unsigned long long o = 0, a = ~0ull;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const unsigned long long k = ukey(keys[i]);
        o |= k;
        a &= k;
    }
    for (int m = 32; m > 0; m >>= 1) {
        o |= (unsigned long long)__shfl_xor((long long)o, m, 64);
        a &= (unsigned long long)__shfl_xor((long long)a, m, 64);
    }
    __shared__ unsigned long long s_o[4], s_a[4];
    if ((threadIdx.x & 63) == 0) {
        s_o[threadIdx.x >> 6] = o;
        s_a[threadIdx.x >> 6] = a;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) {
            o |= s_o[w];
            a &= s_a[w];
        }
        part[2 * blockIdx.x] = o;
        part[2 * blockIdx.x + 1] = a;
    }
}

// One workgroup: folds the span partials and writes the pass plan (a byte in which every
// key has the same digit is skipped).
__global__ __launch_bounds__(256) void rs_plan_kernel(const unsigned long long* __restrict__ part, int nparts,
                                                      RsCtl* __restrict__ ctl)
{
    unsigned long long o = 0, a = ~0ull;
    for (int b = threadIdx.x; b < nparts; b += blockDim.x) {
        o |= part[2 * b];
        a &= part[2 * b + 1];
    }
    for (int m = 32; m > 0; m >>= 1) {
        o |= (unsigned long long)__shfl_xor((long long)o, m, 64);
        a &= (unsigned long long)__shfl_xor((long long)a, m, 64);
    }
    __shared__ unsigned long long s_o[4], s_a[4];
    if ((threadIdx.x & 63) == 0) {
        s_o[threadIdx.x >> 6] = o;
        s_a[threadIdx.x >> 6] = a;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) {
            o |= s_o[w];
            a &= s_a[w];
        }
        const unsigned long long vary = o & ~a;
        int last = -1;
        for (int p = 0; p < kRsPasses; ++p)
            if ((vary >> (8 * p)) & 0xffull) last = p;
        int cur = 0;  // where the data is before the next pass that runs
        for (int p = 0; p < kRsPasses; ++p) {
            RsPass q = {0, 0, 0, 0};
            if ((vary >> (8 * p)) & 0xffull) {
                q.run = 1;
                q.src = cur;
                q.dst = p == last ? 3 : (cur == 1 ? 2 : 1);
                cur = q.dst;
            }
            ctl->pass[p] = q;
        }
        ctl->none = last < 0 ? 1 : 0;
    }
}

// Digit counts of byte Q of every tile of the pass's input, digit-major.
template <int Q>
__global__ __launch_bounds__(kRsBlock) void rs_hist_kernel(const int64_t* __restrict__ ukeys, int64_t n,
                                                           const int64_t* __restrict__ kb1,
                                                           const int64_t* __restrict__ kb2,
                                                           const RsCtl* __restrict__ ctl, int* __restrict__ hist)
{
    const RsPass P = ctl->pass[Q];
    if (!P.run) return;
    __shared__ int h[256];
    h[threadIdx.x] = 0;
    __syncthreads();
    const int64_t* kin = P.src == 1 ? kb1 : kb2;
    const int64_t base = (int64_t)blockIdx.x * kRsTile;
#pragma unroll 4
    for (int u = 0; u < kRsPer; ++u) {
        const int64_t i = base + u * kRsBlock + threadIdx.x;
        if (i < n) {
            const uint64_t k = P.src == 0 ? ukey(ukeys[i]) : (uint64_t)kin[i];
            atomicAdd(&h[digit_of(k, 8 * Q)], 1);
        }
    }
    __syncthreads();
    hist[(int64_t)threadIdx.x * gridDim.x + blockIdx.x] = h[threadIdx.x];
}

struct RsScatterLds {
    union {
        uint64_t k[kRsTile];  // the tile's keys in slot (digit) order
        int32_t v[kRsTile];   // then their positions
    } buf;
    uint8_t dig[kRsTile];      // the digit of every slot
    int glob[256];             // output index of slot 0 of each digit's run, for this tile
    int wc[kRsBlock / 64][256];  // per wave: running count per digit, then its first slot
    int w32[kRsBlock / 64];
};

// Pass over byte Q.  offs: the exclusive scan of this pass's tile counts (digit-major).
template <int Q>
__global__ __launch_bounds__(kRsBlock) void rs_pass_kernel(
    const int64_t* __restrict__ ukeys, int64_t n, int64_t* __restrict__ kb1, int64_t* __restrict__ kb2,
    int32_t* __restrict__ vb1, int32_t* __restrict__ vb2, int64_t* __restrict__ perm,
    const RsCtl* __restrict__ ctl, const int* __restrict__ offs)
{
    constexpr int shift = 8 * Q;
    const RsPass P = ctl->pass[Q];
    if (Q == 0 && ctl->none) {  // every key equal: the identity
        for (int64_t i = (int64_t)blockIdx.x * kRsBlock + threadIdx.x; i < n; i += (int64_t)gridDim.x * kRsBlock)
            perm[i] = i;
        return;
    }
    if (!P.run) return;
    __shared__ RsScatterLds S;
    const bool first = P.src == 0, last = P.dst == 3;
    const int64_t* kin = P.src == 1 ? kb1 : kb2;
    const int32_t* vin = P.src == 1 ? vb1 : vb2;
    int64_t* kout = P.dst == 1 ? kb1 : kb2;
    int32_t* vout = P.dst == 1 ? vb1 : vb2;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int t = blockIdx.x, ntiles = gridDim.x;
    for (int k = 0; k < kRsBlock / 64; ++k) S.wc[k][threadIdx.x] = 0;
    __syncthreads();
    const int64_t base = (int64_t)t * kRsTile;
    const int m = (int)((n - base) < kRsTile ? (n - base) : kRsTile);  // keys in this tile
    uint64_t key[kRsPer];
    int32_t val[kRsPer];
    int rk[kRsPer];
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
    for (int u = 0; u < kRsPer; ++u) {
        const int i = w * kRsWaveKeys + u * 64 + lane;
        const bool valid = i < m;
        key[u] = valid ? (first ? ukey(ukeys[base + i]) : (uint64_t)kin[base + i]) : 0ull;
        val[u] = valid ? (first ? (int32_t)(base + i) : vin[base + i]) : 0;
    }
    // this tile's output base per digit (independent of the ranking below, so its load
    // overlaps it): the keys of lower digits plus this digit's keys in the tiles before
    const int before_t = offs[(int64_t)threadIdx.x * ntiles + t];
#pragma unroll
    for (int u = 0; u < kRsPer; ++u) {
        const int i = w * kRsWaveKeys + u * 64 + lane;
        const bool valid = i < m;
        const int d = digit_of(key[u], shift);
        uint64_t match = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 8; ++bit) {
            const uint64_t b = __ballot(valid && ((d >> bit) & 1));
            match &= ((d >> bit) & 1) ? b : ~b;
        }
        const int inwave = __popcll(match & lt);
        const int before = valid ? S.wc[w][d] : 0;  // the wave's earlier keys of digit d
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (valid && inwave == 0) S.wc[w][d] = before + __popcll(match);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        rk[u] = before + inwave;
    }
    __syncthreads();
    // thread d: the digit's start in the tile, each wave's first slot of it, and where
    // slot 0 of the digit's run lands in the output
    {
        const int d = threadIdx.x;
        int c = 0;
        for (int k = 0; k < kRsBlock / 64; ++k) c += S.wc[k][d];
        int tot;
        const int ex = block_excl_scan<int, kRsBlock>(c, S.w32, &tot);
        int at = ex;
        for (int k = 0; k < kRsBlock / 64; ++k) {
            const int ck = S.wc[k][d];
            S.wc[k][d] = at;
            at += ck;
        }
        S.glob[d] = before_t - ex;
    }
    __syncthreads();
    int slot[kRsPer];
#pragma unroll
    for (int u = 0; u < kRsPer; ++u) {
        const int i = w * kRsWaveKeys + u * 64 + lane;
        slot[u] = -1;
        if (i < m) {
            const int d = digit_of(key[u], shift);
            slot[u] = S.wc[w][d] + rk[u];
            S.buf.k[slot[u]] = key[u];
            S.dig[slot[u]] = (uint8_t)d;
        }
    }
    __syncthreads();
    if (!last)
        for (int sl = threadIdx.x; sl < m; sl += kRsBlock) kout[S.glob[S.dig[sl]] + sl] = (int64_t)S.buf.k[sl];
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kRsPer; ++u)
        if (slot[u] >= 0) S.buf.v[slot[u]] = val[u];
    __syncthreads();
    for (int sl = threadIdx.x; sl < m; sl += kRsBlock) {
        const int64_t dst = S.glob[S.dig[sl]] + sl;
        if (last)
            perm[dst] = (int64_t)S.buf.v[sl];
        else
            vout[dst] = S.buf.v[sl];
    }
}

// ------------------------------------------------------------------ labels
__global__ void labels_unweighted_kernel(const int64_t* __restrict__ perm, int64_t n, int64_t W,
                                         int64_t* __restrict__ labels)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t p = 0;
    if (W > 1) {
        int64_t base = n / W, rem = n % W, thr = rem * (base + 1);
        p = i < thr ? i / (base + 1) : rem + (i - thr) / (base > 0 ? base : 1);
        if (p > W - 1) p = W - 1;
    }
    labels[perm[i]] = p;
}

__global__ void gather_weights_kernel(const int64_t* __restrict__ perm, int64_t n,
                                      const int64_t* __restrict__ w, int64_t* __restrict__ out)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = w[perm[i]];
}

// cs_excl[i+1] is the inclusive prefix of the sorted weights at i.
__global__ void labels_weighted_kernel(const int64_t* __restrict__ perm, int64_t n, int64_t W,
                                       const int64_t* __restrict__ cs_excl,
                                       int64_t* __restrict__ labels)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t total = cs_excl[n];
    int64_t c = cs_excl[i + 1];
    int64_t p = total > 0 ? (c * W) / total : 0;
    if (p < 0) p = 0;
    if (p > W - 1) p = W - 1;
    labels[perm[i]] = p;
}

// ------------------------------------------------------------------ edge filter
__device__ __forceinline__ double shift_at(const void* sh, int dt, int64_t k)
{
    if (dt == DG_F32) return (double)((const float*)sh)[k];
    if (dt == DG_F64) return ((const double*)sh)[k];
    if (dt == DG_I32) return (double)((const int32_t*)sh)[k];
    return (double)((const int64_t*)sh)[k];
}

struct FilterCell {
    double c[9];
};

// keep iff canonical d2 <= r^2 (dist_graph_ops_kernels.cu:16-43 keeps d2 <= r2, no lower bound).
// An edge naming an atom outside [0, n) is dropped, and raises *bad when bad is given.
__device__ __forceinline__ bool filter_keep(const void* __restrict__ pos, int f64, int64_t n,
                                            const FilterCell& C, double r2, int64_t s, int64_t d,
                                            const void* __restrict__ sh, int sdt, int64_t e,
                                            int* __restrict__ bad)
{
    if ((uint64_t)s >= (uint64_t)n || (uint64_t)d >= (uint64_t)n) {
        if (bad) atomicOr(bad, 1);
        return false;
    }
    double ps[3], pt[3];
    if (f64) {
        const double* a = (const double*)pos;
        for (int k = 0; k < 3; ++k) { ps[k] = a[3 * s + k]; pt[k] = a[3 * d + k]; }
    } else {
        const float* a = (const float*)pos;
        for (int k = 0; k < 3; ++k) { ps[k] = a[3 * s + k]; pt[k] = a[3 * d + k]; }
    }
    const double S0 = shift_at(sh, sdt, 3 * e), S1 = shift_at(sh, sdt, 3 * e + 1),
                 S2 = shift_at(sh, sdt, 3 * e + 2);
    double v[3];
    for (int a = 0; a < 3; ++a)
        v[a] = (ps[a] - pt[a]) + fma(S2, C.c[6 + a], fma(S1, C.c[3 + a], S0 * C.c[a]));
    const double d2 = fma(v[2], v[2], fma(v[1], v[1], v[0] * v[0]));
    return d2 <= r2;
}

__global__ void filter_flag_kernel(const void* __restrict__ pos, int f64, int64_t n, FilterCell C,
                                   double r2, const int64_t* __restrict__ src,
                                   const int64_t* __restrict__ dst, const void* __restrict__ sh,
                                   int sdt, int64_t E, int* __restrict__ flag, int* __restrict__ bad)
{
    int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    flag[e] = filter_keep(pos, f64, n, C, r2, src[e], dst[e], sh, sdt, e, bad) ? 1 : 0;
}

__global__ void filter_clear_kernel(int* __restrict__ bad)
{
    if (threadIdx.x == 0) *bad = 0;
}

// n_kept = -1 when an edge named an atom outside [0, n); -2 when a look-back gave up
__global__ void filter_bad_kernel(const int* __restrict__ bad, int64_t* __restrict__ n_kept)
{
    if (threadIdx.x == 0 && *bad) *n_kept = (*bad & 1) ? -1 : -2;
}

__global__ void zero_one_kernel(int64_t* __restrict__ p)
{
    if (threadIdx.x == 0) *p = 0;
}

// Two-pass compaction (count, then write in order): a workgroup of 256 threads takes
// kFilterPer consecutive edges per thread, kFilterTile per workgroup (one edge per thread:
// each edge's pos gathers depend on its src/dst loads, and with four edges per thread the
// C3 filter took 6.7 ms instead of 2.9 ms).  Pass 1 stores the
// workgroup's kept count; pass 2 re-evaluates the predicate and writes the kept edges at
// the workgroup's offset plus their rank inside it.
constexpr int kFilterPer = 1;
constexpr int kFilterTile = 256 * kFilterPer;

__device__ __forceinline__ int filter_tile_flags(const void* pos, int f64, int64_t na,
                                                 const FilterCell& C, double r2, const int64_t* src,
                                                 const int64_t* dst, const void* sh, int sdt, int64_t E,
                                                 int64_t e0, int64_t* s, int64_t* d, bool* keep, int* bad)
{
    int n = 0;
#pragma unroll
    for (int k = 0; k < kFilterPer; ++k) {
        const int64_t e = e0 + k;
        keep[k] = false;
        if (e < E) {
            s[k] = src[e];
            d[k] = dst[e];
            keep[k] = filter_keep(pos, f64, na, C, r2, s[k], d[k], sh, sdt, e, bad);
        }
        n += keep[k] ? 1 : 0;
    }
    return n;
}

__global__ __launch_bounds__(256) void filter_count_kernel(const void* __restrict__ pos, int f64,
                                                           int64_t na, FilterCell C, double r2,
                                                           const int64_t* __restrict__ src,
                                                           const int64_t* __restrict__ dst,
                                                           const void* __restrict__ sh, int sdt,
                                                           int64_t E, int* __restrict__ bcnt,
                                                           int* __restrict__ bad)
{
    __shared__ int s_w[4];
    const int64_t e0 = (int64_t)blockIdx.x * kFilterTile + (int64_t)threadIdx.x * kFilterPer;
    int64_t s[kFilterPer], d[kFilterPer];
    bool keep[kFilterPer];
    const int n = filter_tile_flags(pos, f64, na, C, r2, src, dst, sh, sdt, E, e0, s, d, keep, bad);
    int tot;
    block_excl_scan<int, 256>(n, s_w, &tot);
    if (threadIdx.x == 0) bcnt[blockIdx.x] = tot;
}

template <typename ST>
__global__ __launch_bounds__(256) void filter_write_kernel(const void* __restrict__ pos, int f64,
                                                           int64_t na, FilterCell C, double r2,
                                                           const int64_t* __restrict__ src,
                                                           const int64_t* __restrict__ dst,
                                                           const ST* __restrict__ sh, int sdt,
                                                           int64_t E, const int64_t* __restrict__ boff,
                                                           int64_t* __restrict__ osrc,
                                                           int64_t* __restrict__ odst,
                                                           ST* __restrict__ osh)
{
    __shared__ int s_w[4];
    const int64_t e0 = (int64_t)blockIdx.x * kFilterTile + (int64_t)threadIdx.x * kFilterPer;
    int64_t s[kFilterPer], d[kFilterPer];
    bool keep[kFilterPer];
    const int n = filter_tile_flags(pos, f64, na, C, r2, src, dst, sh, sdt, E, e0, s, d, keep, nullptr);
    int tot;
    int64_t o = boff[blockIdx.x] + block_excl_scan<int, 256>(n, s_w, &tot);
#pragma unroll
    for (int k = 0; k < kFilterPer; ++k) {
        if (!keep[k]) continue;
        osrc[o] = s[k];
        odst[o] = d[k];
        for (int c = 0; c < 3; ++c) osh[3 * o + c] = sh[3 * (e0 + k) + c];
        ++o;
    }
}

// ---- single-pass compaction (decoupled look-back, dg_lookback.hpp)
// A workgroup takes a ticket t (its tile: edges [t kF1Tile, (t + 1) kF1Tile)), evaluates
// the predicate on its kF1Per edges per thread (thread i holds edges i, i + kF1Threads, ...; all
// their loads issued together), publishes its kept count, looks back for the kept count
// of the tiles before it and writes its kept edges there, in order.  One read of the edge
// list, one write of the kept edges.
// 512 threads x 8 edges per tile: measured at C3 (115M edges) against 256 x 4 (2.51 ms),
// 256 x 8 (2.24-2.40), 512 x 4 (2.32), 1024 x 4 (2.71), 1024 x 8 (2.18) and persistent
// workgroups with a prefetched ticket (3.2 ms): 2.10 ms.
constexpr int kF1Per = 8;
constexpr int kF1Threads = 512;
constexpr int kF1Tile = kF1Threads * kF1Per;
constexpr int kF1Groups = kF1Per / 4;
static_assert(kF1Per % 4 == 0, "kept flags are scanned four strides per uint64");

__device__ __forceinline__ uint64_t lb_load(const uint64_t* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void lb_store(uint64_t* p, uint64_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Clears the ticket counter, the error flags and the status words of the tiles.
__global__ void filter1_clear_kernel(uint64_t* __restrict__ status, int64_t ntiles,
                                     unsigned* __restrict__ ticket, int* __restrict__ bad)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < ntiles) status[i] = 0;
    if (i == 0) {
        *ticket = 0u;
        *bad = 0;
    }
}

template <typename ST>
__global__ __launch_bounds__(kF1Threads) void filter1_kernel(const void* __restrict__ pos, int f64,
                                                             int64_t na, FilterCell C, double r2,
                                                             const int64_t* __restrict__ src,
                                                             const int64_t* __restrict__ dst,
                                                             const ST* __restrict__ sh, int sdt,
                                                             int64_t E, int64_t ntiles,
                                                             uint64_t* __restrict__ status,
                                                             unsigned* __restrict__ ticket,
                                                             int* __restrict__ bad,
                                                             int64_t* __restrict__ osrc,
                                                             int64_t* __restrict__ odst,
                                                             ST* __restrict__ osh,
                                                             int64_t* __restrict__ n_kept)
{
    __shared__ unsigned s_t;
    __shared__ uint64_t s_w[kF1Threads / 64];
    __shared__ uint64_t s_win[lookback::kWindow];
    __shared__ int64_t s_excl;
    const int lane = threadIdx.x & 63;
    if (threadIdx.x == 0) s_t = atomicAdd(ticket, 1u);
    __syncthreads();
    const int64_t t = s_t;
    const int64_t e0 = t * kF1Tile + threadIdx.x;
    // wave 0 walks back: every lane runs the same walk on the same window (one status word
    // loaded per lane)
    auto load = [&](int64_t i0, int m, uint64_t* w) {
        __builtin_amdgcn_wave_barrier();  // every lane is done with the last window
        w[lane] = lane < m ? lb_load(&status[i0 - lane]) : 0ull;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    int64_t s[kF1Per], d[kF1Per];
    bool keep[kF1Per];
#pragma unroll
    for (int k = 0; k < kF1Per; ++k) {
        const int64_t e = e0 + kF1Threads * k;
        s[k] = e < E ? src[e] : 0;
        d[k] = e < E ? dst[e] : 0;
    }
    // the first read of the predecessors' words, overlapping this tile's loads (no wait)
    lookback::Walk W = lookback::walk_start(t);
    if (threadIdx.x < 64) lookback::walk_step(W, s_win, load);
    // kept flags of stride k packed as 16-bit fields, four strides per uint64: one scan per
    // group of four yields, for every k, the kept edges of stride k before this thread (at
    // most kF1Threads per field)
    uint64_t packed[kF1Groups];
#pragma unroll
    for (int g = 0; g < kF1Groups; ++g) packed[g] = 0;
#pragma unroll
    for (int k = 0; k < kF1Per; ++k) {
        const int64_t e = e0 + kF1Threads * k;
        keep[k] = e < E && filter_keep(pos, f64, na, C, r2, s[k], d[k], sh, sdt, e, bad);
        packed[k >> 2] |= (uint64_t)(keep[k] ? 1 : 0) << (16 * (k & 3));
    }
    uint64_t ex[kF1Groups], tot[kF1Groups];
#pragma unroll
    for (int g = 0; g < kF1Groups; ++g) ex[g] = block_excl_scan<uint64_t, kF1Threads>(packed[g], s_w, &tot[g]);
    int64_t tile_total = 0;
#pragma unroll
    for (int k = 0; k < kF1Per; ++k) tile_total += (int64_t)((tot[k >> 2] >> (16 * (k & 3))) & 0xFFFFu);

    if (threadIdx.x < 64) {  // wave 0: publish (AGGREGATE first if the walk is not done)
        if (!W.done) {
            if (lane == 0) lb_store(&status[t], lookback::word(lookback::kAggregate, tile_total));
            auto wait = [] { __builtin_amdgcn_s_sleep(1); };
            if (!lookback::walk_finish(W, s_win, load, wait, lookback::kMaxWaitSteps)) {
                if (lane == 0) atomicOr(bad, 2);
            }
        }
        if (lane == 0) {
            lb_store(&status[t], lookback::word(lookback::kInclusive, W.sum + tile_total));
            s_excl = W.sum;
            if (t == ntiles - 1) *n_kept = W.sum + tile_total;
        }
    }
    __syncthreads();
    int64_t o = s_excl;
#pragma unroll
    for (int k = 0; k < kF1Per; ++k) {
        const uint64_t fk = (ex[k >> 2] >> (16 * (k & 3))) & 0xFFFFu;
        if (keep[k]) {
            const int64_t q = o + (int64_t)fk;
            const int64_t e = e0 + kF1Threads * k;
            // non-temporal: the output stream stays out of the caches the gathers use
            // (C3: 2.05 -> 1.99 ms)
            __builtin_nontemporal_store(s[k], &osrc[q]);
            __builtin_nontemporal_store(d[k], &odst[q]);
            for (int c = 0; c < 3; ++c) __builtin_nontemporal_store(sh[3 * e + c], &osh[3 * q + c]);
        }
        o += (int64_t)((tot[k >> 2] >> (16 * (k & 3))) & 0xFFFFu);
    }
}

__global__ void filter_compact_kernel(const int* __restrict__ flag, const int64_t* __restrict__ pre,
                                      int64_t E, int64_t* __restrict__ keep_idx,
                                      int64_t* __restrict__ n_kept)
{
    int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e < E && flag[e]) keep_idx[pre[e]] = e;
    if (e == 0) *n_kept = pre[E];
}

dg_status launch_ok(const char* what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(DG_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
    return DG_OK;
}

struct SortLayout {
    size_t o_k0, o_v0, o_k1, o_v1, o_part, o_ctl, o_hist, o_offs, o_spart, total;
    int nblocks, nparts;
};

SortLayout sort_layout(int64_t n)
{
    SortLayout L;
    size_t o = 0;
    auto take = [&](size_t b) { size_t r = o; o = al(o + (b ? b : 1)); return r; };
    L.nblocks = (int)((n + kRsTile - 1) / kRsTile);
    if (L.nblocks < 1) L.nblocks = 1;
    L.nparts = (int)std::min<int64_t>(kRsSpanBlocks, std::max<int64_t>(1, (n + 255) / 256));
    const size_t nh = (size_t)L.nblocks * 256;
    L.o_k0 = take(8 * n);
    L.o_v0 = take(4 * n);
    L.o_k1 = take(8 * n);
    L.o_v1 = take(4 * n);
    L.o_part = take(16 * (size_t)L.nparts);
    L.o_ctl = take(sizeof(RsCtl));
    L.o_hist = take(4 * nh);
    L.o_offs = take(4 * (nh + 1));
    L.o_spart = take(4 * (nh / kScanTile + 2));
    L.total = o;
    return L;
}

FilterCell filter_cell(const double* cell)
{
    FilterCell C;
    for (int k = 0; k < 9; ++k) C.c[k] = cell[k];
    return C;
}

dg_status filter_check(int32_t pos_dtype, int32_t shift_dtype, double radius, int64_t E,
                       int64_t n_atoms)
{
    if (pos_dtype != DG_F32 && pos_dtype != DG_F64) return fail(DG_ERR_INVALID, "pos dtype");
    if (shift_dtype != DG_F32 && shift_dtype != DG_F64 && shift_dtype != DG_I64 && shift_dtype != DG_I32)
        return fail(DG_ERR_INVALID, "shift dtype");
    if (!(radius > 0.0)) return fail(DG_ERR_INVALID, "radius must be positive");
    if (E < 0 || n_atoms < 0) return fail(DG_ERR_INVALID, "negative size");
    return DG_OK;
}

}  // namespace

extern "C" {

size_t dg_sfc_workspace_size(int64_t n)
{
    if (n < 0) return 0;
    SortLayout L = sort_layout(n);
    size_t bounds = al(6 * 4 * 1024 + 64);
    // keys need the bounds scratch; order needs the sort layout; labels need 8*(2n+2)
    size_t lab = al(8 * (size_t)(n + 1)) * 2 + al(8 * ((size_t)n / kScanTile + 2));
    size_t m = L.total > bounds ? L.total : bounds;
    return m > lab ? m : lab;
}

dg_status dg_sfc_keys(const float* pos, int64_t n, int32_t curve, int64_t* keys, void* ws,
                      size_t ws_bytes, hipStream_t s)
{
    if (n < 0) return fail(DG_ERR_INVALID, "n < 0");
    if (curve != 0 && curve != 1) return fail(DG_ERR_INVALID, "curve must be 0 (Morton) or 1 (Hilbert)");
    if (n == 0) return DG_OK;
    if (ws_bytes < dg_sfc_workspace_size(n)) return fail(DG_ERR_WORKSPACE, "workspace too small");
    float* part = (float*)ws;
    float* bnd = part + 6 * 1024;
    int nb = (int)((n + 255) / 256);
    if (nb > 1024) nb = 1024;
    hipLaunchKernelGGL(bounds_partial_kernel, dim3(nb), dim3(256), 0, s, pos, n, part);
    hipLaunchKernelGGL(bounds_final_kernel, dim3(1), dim3(256), 0, s, (const float*)part, nb, bnd);
    hipLaunchKernelGGL(keys_kernel, dim3(nblk(n)), dim3(256), 0, s, pos, n, (int)curve,
                       (const float*)bnd, keys);
    return launch_ok("dg_sfc_keys");
}

dg_status dg_sfc_order(const int64_t* keys, int64_t n, int64_t* perm, void* ws, size_t ws_bytes,
                       hipStream_t s)
{
    if (n < 0) return fail(DG_ERR_INVALID, "n < 0");
    if (n == 0) return DG_OK;
    if (n > 0x7ffffff0LL) return fail(DG_ERR_INVALID, "n too large");
    if (!keys || !perm) return fail(DG_ERR_INVALID, "keys / perm is NULL");
    SortLayout L = sort_layout(n);
    if (ws_bytes < L.total) return fail(DG_ERR_WORKSPACE, "workspace too small");
    char* w = (char*)ws;
    int64_t* kb1 = (int64_t*)(w + L.o_k0);
    int64_t* kb2 = (int64_t*)(w + L.o_k1);
    int32_t* vb1 = (int32_t*)(w + L.o_v0);
    int32_t* vb2 = (int32_t*)(w + L.o_v1);
    unsigned long long* part = (unsigned long long*)(w + L.o_part);
    RsCtl* ctl = (RsCtl*)(w + L.o_ctl);
    int* hist = (int*)(w + L.o_hist);
    int* offs = (int*)(w + L.o_offs);
    hipLaunchKernelGGL(rs_span_kernel, dim3((unsigned)L.nparts), dim3(256), 0, s, keys, n, part);
    hipLaunchKernelGGL(rs_plan_kernel, dim3(1), dim3(256), 0, s, (const unsigned long long*)part, L.nparts, ctl);
    const dim3 grid((unsigned)L.nblocks), blk(kRsBlock);
    // (a skipped pass's scan runs over stale counts; nothing reads its result)
#define DG_RS_PASS(q)                                                                                  \
    hipLaunchKernelGGL(rs_hist_kernel<q>, grid, blk, 0, s, keys, n, (const int64_t*)kb1, (const int64_t*)kb2, \
                       (const RsCtl*)ctl, hist);                                                         \
    excl_scan<int, int>(hist, (int64_t)L.nblocks * 256, offs, (int*)(w + L.o_spart), s);               \
    hipLaunchKernelGGL(rs_pass_kernel<q>, grid, blk, 0, s, keys, n, kb1, kb2, vb1, vb2, perm,           \
                       (const RsCtl*)ctl, (const int*)offs)
    DG_RS_PASS(0);
    DG_RS_PASS(1);
    DG_RS_PASS(2);
    DG_RS_PASS(3);
    DG_RS_PASS(4);
    DG_RS_PASS(5);
    DG_RS_PASS(6);
    DG_RS_PASS(7);
#undef DG_RS_PASS
    return launch_ok("dg_sfc_order");
}

dg_status dg_sfc_labels(const int64_t* perm, int64_t n, int64_t W, const int64_t* weights,
                        int64_t* labels, void* ws, size_t ws_bytes, hipStream_t s)
{
    if (n < 0 || W < 1) return fail(DG_ERR_INVALID, "need n >= 0 and n_parts >= 1");
    if (n == 0) return DG_OK;
    if (ws_bytes < dg_sfc_workspace_size(n)) return fail(DG_ERR_WORKSPACE, "workspace too small");
    if (!weights || W == 1) {
        hipLaunchKernelGGL(labels_unweighted_kernel, dim3(nblk(n)), dim3(256), 0, s, perm, n,
                           weights ? (int64_t)1 : W, labels);
        return launch_ok("dg_sfc_labels");
    }
    char* w = (char*)ws;
    int64_t* sw = (int64_t*)w;
    int64_t* cs = (int64_t*)(w + al(8 * (size_t)(n + 1)));
    int64_t* part = (int64_t*)(w + 2 * al(8 * (size_t)(n + 1)));
    hipLaunchKernelGGL(gather_weights_kernel, dim3(nblk(n)), dim3(256), 0, s, perm, n, weights, sw);
    device_excl_scan<int64_t, int64_t>(sw, n, cs, part, s);
    hipLaunchKernelGGL(labels_weighted_kernel, dim3(nblk(n)), dim3(256), 0, s, perm, n, W,
                       (const int64_t*)cs, labels);
    return launch_ok("dg_sfc_labels");
}

size_t dg_filter_workspace_size(int64_t E)
{
    if (E < 0) return 0;
    return al(4 * (size_t)E) + al(8 * (size_t)(E + 1)) + al(8 * ((size_t)E / kScanTile + 2)) + al(8);
}

dg_status dg_filter_edges_to_radius(const void* pos, int32_t pos_dtype, int64_t n_atoms,
                                    const double* cell, double radius, const int64_t* src,
                                    const int64_t* dst, const void* shift, int32_t shift_dtype,
                                    int64_t E, int64_t* keep_idx, int64_t* n_kept, void* ws,
                                    size_t ws_bytes, hipStream_t s)
{
    dg_status st = filter_check(pos_dtype, shift_dtype, radius, E, n_atoms);
    if (st != DG_OK) return st;
    if (ws_bytes < dg_filter_workspace_size(E)) return fail(DG_ERR_WORKSPACE, "workspace too small");
    char* w = (char*)ws;
    int* flag = (int*)w;
    int64_t* pre = (int64_t*)(w + al(4 * (size_t)E));
    int64_t* part = (int64_t*)(w + al(4 * (size_t)E) + al(8 * (size_t)(E + 1)));
    int* bad = (int*)(w + al(4 * (size_t)E) + al(8 * (size_t)(E + 1)) + al(8 * ((size_t)E / kScanTile + 2)));
    hipLaunchKernelGGL(filter_clear_kernel, dim3(1), dim3(64), 0, s, bad);
    if (E > 0)
        hipLaunchKernelGGL(filter_flag_kernel, dim3(nblk(E)), dim3(256), 0, s, pos,
                           (int)(pos_dtype == DG_F64), n_atoms, filter_cell(cell), radius * radius, src,
                           dst, shift, (int)shift_dtype, E, flag, bad);
    device_excl_scan<int, int64_t>(flag, E, pre, part, s);
    hipLaunchKernelGGL(filter_compact_kernel, dim3(E > 0 ? nblk(E) : 1), dim3(256), 0, s,
                       (const int*)flag, (const int64_t*)pre, E, keep_idx, n_kept);
    hipLaunchKernelGGL(filter_bad_kernel, dim3(1), dim3(64), 0, s, (const int*)bad, n_kept);
    return launch_ok("dg_filter_edges_to_radius");
}

// Workspace of the count / write pair: per-block kept counts (nb + 1), their offsets
// (nb + 1), scan partials, and the out-of-range flag.
struct Filter2Layout {
    size_t o_bcnt, o_boff, o_part, o_bad, total;
    int64_t nb;
};
static Filter2Layout filter2_layout(int64_t E)
{
    Filter2Layout L;
    L.nb = (E + kFilterTile - 1) / kFilterTile;
    const size_t nb = (size_t)L.nb;
    L.o_bcnt = 0;
    L.o_boff = al(4 * (nb + 1));
    L.o_part = L.o_boff + al(8 * (nb + 1));
    L.o_bad = L.o_part + al(8 * (nb / kScanTile + 2));
    L.total = L.o_bad + al(8);
    return L;
}

// Workspace of the single-pass filter: ticket, error flags, one status word per tile.
static size_t filter1_ws(int64_t E)
{
    const size_t nt = (size_t)((E + kF1Tile - 1) / kF1Tile);
    return 256 + al(8 * (nt + 1));
}

size_t dg_filter_compact_workspace_size(int64_t E)
{
    if (E < 0) return 0;
    return filter1_ws(E);
}

dg_status dg_filter_compact(const void* pos, int32_t pos_dtype, int64_t n_atoms, const double* cell,
                            double radius, const int64_t* src, const int64_t* dst, const void* shift,
                            int32_t shift_dtype, int64_t E, int64_t* out_src, int64_t* out_dst,
                            void* out_shift, int64_t* n_kept, void* ws, size_t ws_bytes,
                            hipStream_t s)
{
    dg_status st = filter_check(pos_dtype, shift_dtype, radius, E, n_atoms);
    if (st != DG_OK) return st;
    if (!n_kept) return fail(DG_ERR_INVALID, "n_kept is NULL");
    if (ws_bytes < filter1_ws(E)) return fail(DG_ERR_WORKSPACE, "workspace too small");
    const int64_t nt = (E + kF1Tile - 1) / kF1Tile;
    char* w = (char*)ws;
    unsigned* ticket = (unsigned*)w;
    int* bad = (int*)(w + 64);
    uint64_t* status = (uint64_t*)(w + 256);
    if (nt > 0x7fffffffLL) return fail(DG_ERR_INVALID, "too many edges");
    hipLaunchKernelGGL(filter1_clear_kernel, dim3(nt > 0 ? nblk(nt) : 1), dim3(256), 0, s, status, nt,
                       ticket, bad);
    if (nt == 0) {
        hipLaunchKernelGGL(zero_one_kernel, dim3(1), dim3(64), 0, s, n_kept);
        return launch_ok("dg_filter_compact");
    }
    const int f64 = (int)(pos_dtype == DG_F64);
    const FilterCell C = filter_cell(cell);
    const double r2 = radius * radius;
#define DG_F1(T)                                                                                       \
    hipLaunchKernelGGL(filter1_kernel<T>, dim3((unsigned)nt), dim3(kF1Threads), 0, s, pos, f64, n_atoms, \
                       C, r2,                                                                          \
                       src, dst, (const T*)shift, (int)shift_dtype, E, nt, status, ticket, bad, out_src,  \
                       out_dst, (T*)out_shift, n_kept)
    if (shift_dtype == DG_F32) DG_F1(float);
    else if (shift_dtype == DG_F64) DG_F1(double);
    else if (shift_dtype == DG_I32) DG_F1(int32_t);
    else DG_F1(int64_t);
#undef DG_F1
    hipLaunchKernelGGL(filter_bad_kernel, dim3(1), dim3(64), 0, s, (const int*)bad, n_kept);
    return launch_ok("dg_filter_compact");
}

size_t dg_filter2_workspace_size(int64_t E)
{
    if (E < 0) return 0;
    return filter2_layout(E).total;
}

dg_status dg_filter_count(const void* pos, int32_t pos_dtype, int64_t n_atoms, const double* cell,
                          double radius, const int64_t* src, const int64_t* dst, const void* shift,
                          int32_t shift_dtype, int64_t E, int64_t* n_kept, void* ws, size_t ws_bytes,
                          hipStream_t s)
{
    dg_status st = filter_check(pos_dtype, shift_dtype, radius, E, n_atoms);
    if (st != DG_OK) return st;
    const Filter2Layout FL = filter2_layout(E);
    if (ws_bytes < FL.total) return fail(DG_ERR_WORKSPACE, "workspace too small");
    const int64_t nb = FL.nb;
    char* w = (char*)ws;
    int* bcnt = (int*)(w + FL.o_bcnt);
    int64_t* boff = (int64_t*)(w + FL.o_boff);
    int64_t* part = (int64_t*)(w + FL.o_part);
    int* bad = (int*)(w + FL.o_bad);
    hipLaunchKernelGGL(filter_clear_kernel, dim3(1), dim3(64), 0, s, bad);
    if (nb > 0)
        hipLaunchKernelGGL(filter_count_kernel, dim3((unsigned)nb), dim3(256), 0, s, pos,
                           (int)(pos_dtype == DG_F64), n_atoms, filter_cell(cell), radius * radius, src,
                           dst, shift, (int)shift_dtype, E, bcnt, bad);
    excl_scan<int, int64_t>(bcnt, nb, boff, part, s, n_kept);
    hipLaunchKernelGGL(filter_bad_kernel, dim3(1), dim3(64), 0, s, (const int*)bad, n_kept);
    return launch_ok("dg_filter_count");
}

dg_status dg_filter_write(const void* pos, int32_t pos_dtype, int64_t n_atoms, const double* cell,
                          double radius, const int64_t* src, const int64_t* dst, const void* shift,
                          int32_t shift_dtype, int64_t E, const void* ws, size_t ws_bytes,
                          int64_t* out_src, int64_t* out_dst, void* out_shift, hipStream_t s)
{
    dg_status st = filter_check(pos_dtype, shift_dtype, radius, E, n_atoms);
    if (st != DG_OK) return st;
    const Filter2Layout FL = filter2_layout(E);
    if (ws_bytes < FL.total) return fail(DG_ERR_WORKSPACE, "workspace too small");
    const int64_t nb = FL.nb;
    if (nb == 0) return DG_OK;
    const int64_t* boff = (const int64_t*)((const char*)ws + FL.o_boff);
    const int f64 = (int)(pos_dtype == DG_F64);
    const FilterCell C = filter_cell(cell);
    const double r2 = radius * radius;
    if (shift_dtype == DG_F32)
        hipLaunchKernelGGL(filter_write_kernel<float>, dim3((unsigned)nb), dim3(256), 0, s, pos, f64,
                           n_atoms, C, r2, src, dst, (const float*)shift, (int)shift_dtype, E, boff,
                           out_src, out_dst, (float*)out_shift);
    else if (shift_dtype == DG_F64)
        hipLaunchKernelGGL(filter_write_kernel<double>, dim3((unsigned)nb), dim3(256), 0, s, pos, f64,
                           n_atoms, C, r2, src, dst, (const double*)shift, (int)shift_dtype, E, boff,
                           out_src, out_dst, (double*)out_shift);
    else if (shift_dtype == DG_I32)
        hipLaunchKernelGGL(filter_write_kernel<int32_t>, dim3((unsigned)nb), dim3(256), 0, s, pos, f64,
                           n_atoms, C, r2, src, dst, (const int32_t*)shift, (int)shift_dtype, E, boff,
                           out_src, out_dst, (int32_t*)out_shift);
    else
        hipLaunchKernelGGL(filter_write_kernel<int64_t>, dim3((unsigned)nb), dim3(256), 0, s, pos, f64,
                           n_atoms, C, r2, src, dst, (const int64_t*)shift, (int)shift_dtype, E, boff,
                           out_src, out_dst, (int64_t*)out_shift);
    return launch_ok("dg_filter_write");
}

}  // extern "C"
