// dg_segsort.hpp -- stable LSD radix sort of one array segment by one workgroup of 256
// threads, in global memory.  The cell-list sort uses it for the rare segments too large
// for its LDS orderings: a tile bucket of more than 2048 entries, a bin of more than 128
// atoms (or targets) in the per-bin sort.  With it, every cell list -- and so the order of
// the output -- depends only on the input, never on the order in which atomics landed.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dg_scan.hpp"

namespace dg {

constexpr int kSegSortThreads = 256;

struct SegSortLds {
    int hist[256];   // entries per digit
    int base[256];   // next output place of each digit (stable: grows block by block)
    int wc[4][256];  // entries per digit in each wave of the current block
    int w32[4];
};

template <typename T>
__device__ __forceinline__ uint32_t seg_digit(T v, int sh)
{
    return (uint32_t)(v >> sh) & 255u;
}

// Sorts a[0, m) ascending on the low key_bits bits of each entry, stably, 8 bits per pass
// (least significant first), going back and forth through tmp[0, m); the result is in a.
// A pass whose digit is the same for every entry is skipped.  Called by all 256 threads.
//
// A pass: a digit histogram (LDS atomics -- only the counts matter), its exclusive scan,
// then the entries in blocks of 256 in order: inside a wave, the lanes with a lane's digit
// come from eight ballots (one per digit bit); the lane's place is the digit's base, plus
// the entries of that digit in the block's earlier waves, plus its rank among its peers in
// its own wave.  Every place is a function of the input alone.
template <typename T>
__device__ void segment_sort(T* a, T* tmp, int m, int key_bits, SegSortLds& L)
{
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint64_t below = (1ull << lane) - 1ull;
    if (m <= 1) return;
    T* src = a;
    T* dst = tmp;
    for (int sh = 0; sh < key_bits; sh += 8) {
        L.hist[tid] = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) L.wc[k][tid] = 0;
        __syncthreads();
        for (int e = tid; e < m; e += kSegSortThreads) atomicAdd(&L.hist[seg_digit(src[e], sh)], 1);
        __syncthreads();
        const bool uniform = L.hist[seg_digit(src[0], sh)] == m;
        int tot;
        L.base[tid] = block_excl_scan<int, kSegSortThreads>(L.hist[tid], L.w32, &tot);  // (synchronises)
        if (uniform) continue;  // (the same for every thread)
        __syncthreads();
        for (int b0 = 0; b0 < m; b0 += kSegSortThreads) {
            const int e = b0 + tid;
            const bool valid = e < m;
            const T v = valid ? src[e] : (T)0;
            const uint32_t d = seg_digit(v, sh);
            uint64_t peers = __builtin_amdgcn_ballot_w64(valid);
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const bool bit = (d >> b) & 1u;
                const uint64_t bb = __builtin_amdgcn_ballot_w64(bit);
                peers &= bit ? bb : ~bb;
            }
            const int rank = __popcll(peers & below);
            if (valid && rank == 0) L.wc[w][d] = __popcll(peers);
            __syncthreads();
            if (valid) {
                int off = L.base[d] + rank;
                for (int k = 0; k < w; ++k) off += L.wc[k][d];
                dst[off] = v;
            }
            __syncthreads();
            L.base[tid] += L.wc[0][tid] + L.wc[1][tid] + L.wc[2][tid] + L.wc[3][tid];
#pragma unroll
            for (int k = 0; k < 4; ++k) L.wc[k][tid] = 0;
            __syncthreads();
        }
        T* t = src;
        src = dst;
        dst = t;
    }
    if (src != a) {
        for (int e = tid; e < m; e += kSegSortThreads) a[e] = src[e];
        __syncthreads();
    }
}

}  // namespace dg
