// Host-threaded model of the single-pass compaction's decoupled look-back: the same
// protocol code the device kernels run (dynamis_amd/csrc/dg_lookback.hpp), driven by
// std::thread "workgroups" with relaxed std::atomic status words, ticket-ordered tiles
// and randomised delays.  Built and run by tests/test_lookback_model.py.
//
//   lookback_model <threads> <tiles> <seed> <mode>
//   mode 0: every tile publishes (exclusive offsets must equal the serial scan)
//   mode 1: tile tiles/2 publishes nothing (its successor must give up: bounded wait)
// Prints "ok" or the first mismatch; exit status 0 on success.
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <thread>
#include <vector>

#include "../dynamis_amd/csrc/dg_lookback.hpp"

using namespace dg::lookback;

int main(int argc, char** argv)
{
    if (argc < 5) return 2;
    const int W = atoi(argv[1]);
    const int64_t T = atoll(argv[2]);
    const unsigned seed = (unsigned)atoi(argv[3]);
    const int mode = atoi(argv[4]);
    const int64_t stuck = mode == 1 ? T / 2 : -1;
    const int max_steps = mode == 1 ? 2000 : (1 << 30);
    std::vector<std::atomic<uint64_t>> status(T);
    for (auto& s : status) s.store(0, std::memory_order_relaxed);
    std::atomic<int64_t> ticket{0};
    std::vector<int64_t> count(T), excl(T, -7);
    std::mt19937_64 g(seed);
    for (auto& c : count) c = (int64_t)(g() % 1025);
    std::vector<std::thread> th;
    for (int w = 0; w < W; ++w)
        th.emplace_back([&, w] {
            std::mt19937 r(seed * 7919u + (unsigned)w);
            uint64_t win[kWindow];
            for (;;) {
                const int64_t t = ticket.fetch_add(1, std::memory_order_relaxed);
                if (t >= T) return;
                if (r() % 8 == 0) std::this_thread::sleep_for(std::chrono::microseconds(r() % 50));
                if (t == stuck) continue;  // never publishes
                auto load = [&](int64_t i0, int m, uint64_t* wv) {
                    for (int i = 0; i < m; ++i) wv[i] = status[i0 - i].load(std::memory_order_relaxed);
                };
                auto wait = [] { std::this_thread::yield(); };
                // as the kernel: one read before the tile's own count is known, no waiting
                Walk W = walk_start(t);
                walk_step(W, win, load);
                if (r() % 4 == 0) std::this_thread::sleep_for(std::chrono::microseconds(r() % 20));
                bool ok = true;
                if (!W.done) {
                    status[t].store(word(kAggregate, count[t]), std::memory_order_relaxed);
                    if (r() % 4 == 0) std::this_thread::yield();
                    ok = walk_finish(W, win, load, wait, max_steps);
                }
                excl[t] = ok ? W.sum : -1;
                status[t].store(word(kInclusive, (ok ? W.sum : 0) + count[t]), std::memory_order_relaxed);
            }
        });
    for (auto& x : th) x.join();
    int64_t run = 0;
    for (int64_t t = 0; t < T; ++t) {
        if (mode == 1 && t >= stuck) {
            // the tile right behind the silent one can only give up (-1); a tile that gave up
            // publishes a wrong INCLUSIVE word, so later values are unspecified (the device
            // raises the error flag then): only termination is required of them
            if (t == stuck + 1 && excl[t] != -1) {
                printf("mode 1: tile %lld excl %lld (expected -1)\n", (long long)t, (long long)excl[t]);
                return 1;
            }
            continue;
        }
        if (excl[t] != run) {
            printf("tile %lld: excl %lld, serial scan %lld\n", (long long)t, (long long)excl[t], (long long)run);
            return 1;
        }
        run += count[t];
    }
    printf("ok\n");
    return 0;
}
