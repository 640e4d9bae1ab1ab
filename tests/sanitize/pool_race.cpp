// The retired list and pool of libtensomite_hip.so (tmh_pool.h) under
// threads, host only: pusher threads give memory back as finalizers do
// (never waiting; what the list refuses, the pusher frees itself) while
// several threads drain the list into the pool and take from it, as
// tmh_alloc and tmh_sync do on whatever threads call them. Every pointer
// handed in must come back exactly once -- drained, or refused and freed by
// its pusher -- and the pool must never hand one pointer out twice while it
// is taken. Exit status 0 when that holds; the counts otherwise.
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <thread>
#include <vector>

#include "../../tensomite.cr_amd/csrc/tmh_pool.h"

int main(int argc, char** argv) {
    const int pushers = 4, drainers = 3;
    const int per = argc > 1 ? std::atoi(argv[1]) : 200000;
    const uint64_t ids = (uint64_t)pushers * per;
    auto retired = std::make_unique<tmh::Retired>();
    tmh::Pool pool;
    pool.limit = 1ll << 40;
    // per id: times it came back (drained or refused), and whether the pool
    // has it out right now
    std::vector<std::atomic<int>> back(ids + 1), out(ids + 1);
    std::atomic<int> pushing{pushers};
    std::atomic<int64_t> twice{0};

    auto returned = [&](uint64_t id) { back[id].fetch_add(1); };
    std::vector<std::thread> threads;
    for (int t = 0; t < pushers; ++t)
        threads.emplace_back([&, t] {
            for (int i = 0; i < per; ++i) {
                const uint64_t id = (uint64_t)t * per + i + 1;
                if (!retired->push(id, 64u * (1u + id % 4u))) returned(id);
            }
            pushing.fetch_sub(1);
        });
    for (int t = 0; t < drainers; ++t)
        threads.emplace_back([&] {
            while (pushing.load() > 0) {
                retired->drain([&](uint64_t id, uint64_t bytes) {
                    returned(id);
                    // into the pool; out again at once, then back: a pointer
                    // handed out while it is out means it was given twice
                    if (!pool.give(id, bytes)) return;
                    const uint64_t got = pool.take(bytes);
                    if (!got) return;
                    if (out[got].exchange(1) != 0) twice.fetch_add(1);
                    out[got].store(0);
                    if (!pool.give(got, bytes)) return;
                });
            }
        });
    for (auto& th : threads) th.join();
    retired->drain([&](uint64_t id, uint64_t) { returned(id); });

    int64_t lost = 0, repeated = 0;
    for (uint64_t id = 1; id <= ids; ++id) {
        const int n = back[id].load();
        lost += n == 0;
        repeated += n > 1;
    }
    std::printf("pool_race: %llu pointers, %lld lost, %lld back more than once, %lld handed out twice\n",
                (unsigned long long)ids, (long long)lost, (long long)repeated, (long long)twice.load());
    return lost == 0 && repeated == 0 && twice.load() == 0 ? 0 : 1;
}
