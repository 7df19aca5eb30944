// dg_scan.hpp -- wave64 / workgroup / device-wide exclusive scans used by the graph build.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dg {

constexpr int kScanBlock = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanBlock * kScanItems;  // 2048 items per workgroup
constexpr int kSmallScanBlock = 1024;  // the one-workgroup scan of short arrays
constexpr int64_t kScanSumParts = 1024;  // up to this many tiles the last phase sums the partials

// Inclusive scan across one wave64.
template <typename T>
__device__ __forceinline__ T wave_incl_scan(T x)
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        T y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    return x;
}

// Exclusive scan across a workgroup of NT threads (NT multiple of 64).  s_w holds
// NT/64 values.  Returns the exclusive prefix; *total receives the workgroup sum.
template <typename T, int NT>
__device__ __forceinline__ T block_excl_scan(T v, T* s_w, T* total)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    T x = wave_incl_scan(v);
    if (lane == 63) s_w[w] = x;
    __syncthreads();
    T before = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) {
        T s = s_w[i];
        before += (i < w) ? s : (T)0;
        tot += s;
    }
    __syncthreads();
    *total = tot;
    return before + x - v;
}

// True on every thread when v is true on any thread of the workgroup of NT threads (s_w:
// NT/64 ints of scratch; the runtime's __syncthreads_or would add its own LDS).
template <int NT>
__device__ __forceinline__ bool block_any(bool v, int* s_w)
{
    const int w = threadIdx.x >> 6;
    const bool wv = __builtin_amdgcn_ballot_w64(v) != 0ull;
    if ((threadIdx.x & 63) == 0) s_w[w] = wv;
    __syncthreads();
    int any = 0;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) any |= s_w[i];
    __syncthreads();
    return any != 0;
}

// Phase 1: per-workgroup sums of kScanTile items.
template <typename Tin, typename Tout>
__global__ __launch_bounds__(kScanBlock) void scan_reduce_kernel(const Tin* __restrict__ in,
                                                                 int64_t n, Tout* __restrict__ part)
{
    __shared__ Tout s_w[kScanBlock / 64];
    int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    Tout s = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k)
        if (base + k < n) s += (Tout)in[base + k];
    Tout tot;
    block_excl_scan<Tout, kScanBlock>(s, s_w, &tot);
    if (threadIdx.x == 0) part[blockIdx.x] = tot;
}

// Phase 2: one workgroup scans the partials in place (exclusive), any length.
template <typename Tout>
__global__ __launch_bounds__(kScanBlock) void scan_partials_kernel(Tout* __restrict__ part,
                                                                   int64_t nblk)
{
    __shared__ Tout s_w[kScanBlock / 64];
    Tout carry = 0;
    for (int64_t b0 = 0; b0 < nblk; b0 += kScanBlock) {
        int64_t i = b0 + threadIdx.x;
        Tout v = i < nblk ? part[i] : (Tout)0;
        Tout tot;
        Tout ex = block_excl_scan<Tout, kScanBlock>(v, s_w, &tot);
        if (i < nblk) part[i] = carry + ex;
        carry += tot;
    }
}

// Phase 3: exclusive scan of each tile plus its offset; out has n+1 entries, out[n] = sum.
// SUM_PARTS: part holds the per-tile sums unscanned, and each workgroup adds up those before
// it (few tiles: phase 2's launch saved).
template <typename Tin, typename Tout, bool SUM_PARTS = false>
__global__ __launch_bounds__(kScanBlock) void scan_final_kernel(const Tin* __restrict__ in,
                                                                int64_t n,
                                                                const Tout* __restrict__ part,
                                                                Tout* __restrict__ out)
{
    __shared__ Tout s_w[kScanBlock / 64];
    Tout off;
    if constexpr (SUM_PARTS) {
        Tout p = 0;
        for (int i = threadIdx.x; i < (int)blockIdx.x; i += kScanBlock) p += part[i];
        block_excl_scan<Tout, kScanBlock>(p, s_w, &off);
    } else {
        off = part[blockIdx.x];
    }
    int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    Tout v[kScanItems];
    Tout s = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        v[k] = (base + k < n) ? (Tout)in[base + k] : (Tout)0;
        s += v[k];
    }
    Tout tot;
    Tout ex = block_excl_scan<Tout, kScanBlock>(s, s_w, &tot) + off;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        if (base + k < n) out[base + k] = ex;
        ex += v[k];
    }
    if (blockIdx.x == gridDim.x - 1 && threadIdx.x == kScanBlock - 1) out[n] = ex;
}

// Host helper: exclusive scan of in[0..n) into out[0..n] (out[n] = total).
// part needs n / kScanTile + 1 entries of Tout.
template <typename Tin, typename Tout>
inline void device_excl_scan(const Tin* in, int64_t n, Tout* out, Tout* part, hipStream_t s)
{
    int64_t nblk = n / kScanTile + 1;
    hipLaunchKernelGGL((scan_reduce_kernel<Tin, Tout>), dim3((unsigned)nblk), dim3(kScanBlock), 0,
                       s, in, n, part);
    if (nblk <= kScanSumParts) {
        hipLaunchKernelGGL((scan_final_kernel<Tin, Tout, true>), dim3((unsigned)nblk), dim3(kScanBlock), 0,
                           s, in, n, (const Tout*)part, out);
        return;
    }
    hipLaunchKernelGGL((scan_partials_kernel<Tout>), dim3(1), dim3(kScanBlock), 0, s, part, nblk);
    hipLaunchKernelGGL((scan_final_kernel<Tin, Tout>), dim3((unsigned)nblk), dim3(kScanBlock), 0,
                       s, in, n, part, out);
}

// Exclusive scan of in[0..n) into out[0..n] (out[n] = sum) by one workgroup, for short
// arrays (one launch instead of three); the sum is also stored to *sum_out if given.
template <typename Tin, typename Tout>
__global__ __launch_bounds__(kSmallScanBlock) void small_scan_kernel(const Tin* __restrict__ in,
                                                                     int64_t n, Tout* __restrict__ out,
                                                                     int64_t* __restrict__ sum_out)
{
    __shared__ Tout s_w[kSmallScanBlock / 64];
    Tout carry = 0;
    for (int64_t b0 = 0; b0 < n; b0 += kSmallScanBlock * kScanItems) {
        const int64_t base = b0 + (int64_t)threadIdx.x * kScanItems;
        Tout v[kScanItems], sum = 0;
#pragma unroll
        for (int k = 0; k < kScanItems; ++k) {
            v[k] = base + k < n ? (Tout)in[base + k] : (Tout)0;
            sum += v[k];
        }
        Tout tot;
        Tout ex = block_excl_scan<Tout, kSmallScanBlock>(sum, s_w, &tot) + carry;
#pragma unroll
        for (int k = 0; k < kScanItems; ++k) {
            if (base + k < n) out[base + k] = ex;
            ex += v[k];
        }
        carry += tot;
    }
    if (threadIdx.x == 0) {
        out[n] = carry;
        if (sum_out) *sum_out = (int64_t)carry;
    }
}

template <typename Tout>
__global__ void copy_sum_kernel(const Tout* __restrict__ src, int64_t* __restrict__ dst)
{
    if (threadIdx.x == 0 && blockIdx.x == 0) *dst = (int64_t)*src;
}

constexpr int64_t kSmallScanMax = 8192;  // one pass of the 1024-thread workgroup

// Exclusive scan choosing the one-workgroup kernel for short arrays (it beats three
// launches up to a few thousand items).
template <typename Tin, typename Tout>
inline void excl_scan(const Tin* in, int64_t n, Tout* out, Tout* part, hipStream_t s,
                      int64_t* sum_out = nullptr)
{
    if (n <= kSmallScanMax) {
        hipLaunchKernelGGL((small_scan_kernel<Tin, Tout>), dim3(1), dim3(kSmallScanBlock), 0, s, in, n,
                           out, sum_out);
        return;
    }
    device_excl_scan<Tin, Tout>(in, n, out, part, s);
    if (sum_out)
        hipLaunchKernelGGL((copy_sum_kernel<Tout>), dim3(1), dim3(64), 0, s, (const Tout*)(out + n),
                           sum_out);
}

}  // namespace dg
