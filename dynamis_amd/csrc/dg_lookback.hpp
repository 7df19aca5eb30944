// dg_lookback.hpp -- the decoupled look-back protocol of the single-pass compactions
// (Merrill & Garland, "Single-pass Parallel Prefix Scan with Decoupled Look-back", 2016),
// shared by the device kernels and the host-threaded model in tests/.
//
// Every tile t of a single-pass compaction owns one 64-bit status word:
//   bits 63..62  0 = not ready, 1 = AGGREGATE (the tile's own count is in the value),
//                2 = INCLUSIVE (the count of tiles 0..t is in the value)
//   bits 61..0   the value
// A tile reads its predecessors' words (nearest first), summing the values, until it meets
// an INCLUSIVE one, and then publishes INCLUSIVE = that sum + its count.  It starts the
// walk before its own count is known, without waiting; if the walk is not complete when
// the count is, it publishes AGGREGATE first (so its successors never wait on its walk),
// then finishes the walk.
//
// Why this cannot deadlock or read stale data:
//   * Tiles are numbered by a ticket (an atomic counter) taken when the workgroup starts,
//     so every predecessor of tile t belongs to a workgroup that was already running when
//     t's was; a predecessor never waits on a later tile.  Each wait therefore ends once
//     the (running) predecessor publishes, and every wait is bounded besides.
//   * The payload travels inside the status word itself, written and read only with
//     device-scope atomic operations: no other data written by one workgroup is read by
//     another, so no cache write-back or invalidation is needed across the XCDs' L2s.
//   * Loop trip counts never come from another tile's data: the look-back walks at most
//     t words, a window at a time, and the edges a tile writes are its own.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define DG_LB_HD __host__ __device__ __forceinline__
#else
#define DG_LB_HD inline
#endif

namespace dg {
namespace lookback {

constexpr uint64_t kAggregate = 1ull << 62;
constexpr uint64_t kInclusive = 2ull << 62;
constexpr uint64_t kValueMask = (1ull << 62) - 1;
constexpr int kWindow = 64;  // predecessor words examined per step (one wave64)
// Steps a look-back may take waiting for a predecessor (each step reads one window) before
// it gives up and reports an error; far above any real wait (about a second).
constexpr int kMaxWaitSteps = 1 << 20;

DG_LB_HD uint64_t word(uint64_t flag, int64_t value) { return flag | ((uint64_t)value & kValueMask); }
DG_LB_HD uint64_t flag_of(uint64_t w) { return w & ~kValueMask; }
DG_LB_HD int64_t value_of(uint64_t w) { return (int64_t)(w & kValueMask); }

// One read of a window of m predecessor words, w[0] the nearest (tile t - 1), w[i] tile
// t - 1 - i: consumes the leading words that are ready, up to and including the nearest
// INCLUSIVE one, adds their values to *sum and returns how many it consumed (0 when the
// nearest word is not ready yet); *done is set when an INCLUSIVE word ended the walk.
DG_LB_HD int window_step(const uint64_t* w, int m, int64_t* sum, bool* done)
{
    int64_t s = 0;
    int i = 0;
    *done = false;
    for (; i < m; ++i) {
        const uint64_t f = flag_of(w[i]);
        if (f == 0) break;
        s += value_of(w[i]);
        if (f == kInclusive) {
            *done = true;
            ++i;
            break;
        }
    }
    *sum += s;
    return i;
}

// The state of one tile's look-back: the nearest predecessor not yet summed, the sum so
// far, and whether the sum is complete (an INCLUSIVE word was reached; tile 0 has nothing
// to sum).
struct Walk {
    int64_t nxt;
    int64_t sum;
    bool done;
};
DG_LB_HD Walk walk_start(int64_t t) { return Walk{t - 1, 0, t <= 0}; }

// Reads the next window once (load(i0, m, w) fills w[0..m) with the status words of tiles
// i0, i0 - 1, ..., i0 - m + 1: atomic loads, on the device one lane per word) and consumes
// what is ready.  Returns false when nothing was ready.  Every bound of the walk comes
// from t and the window size, never from the words read.
template <class Load>
DG_LB_HD bool walk_step(Walk& W, uint64_t* w, Load&& load)
{
    if (W.done) return true;
    const int m = (int)(W.nxt + 1 < kWindow ? W.nxt + 1 : kWindow);
    load(W.nxt, m, w);
    bool done = false;
    const int k = window_step(w, m, &W.sum, &done);
    W.nxt -= k;
    W.done = done || W.nxt < 0;
    return k > 0;
}

// Finishes a walk: reads windows until the sum is complete, running wait() after a read
// that found nothing ready.  Returns false (the sum incomplete) after max_steps such reads.
template <class Load, class Wait>
DG_LB_HD bool walk_finish(Walk& W, uint64_t* w, Load&& load, Wait&& wait, int max_steps)
{
    int idle = 0;
    while (!W.done) {
        if (walk_step(W, w, load)) continue;
        if (++idle > max_steps) return false;
        wait();
    }
    return true;
}

}  // namespace lookback
}  // namespace dg
