// The device-memory pool and the retired list in front of it, host code
// only (no HIP), so that host tests can build them alone. Each device of
// libtensomite_hip.so keeps one of each.
#pragma once

#include <atomic>
#include <cstdint>
#include <mutex>
#include <thread>
#include <unordered_map>
#include <vector>

namespace tmh {

// Exact-size pool of freed device memory, as BufferPool (buffer_pool.cr:12-74):
// `take` and `give` never wait -- while another caller holds the lock, take
// returns nothing and give returns false, and the caller allocates or frees
// instead.
class Pool {
  public:
    // Written and read from any thread (the pool's limit, its counters);
    // changed under the lock.
    std::atomic<int64_t> limit{1ll << 30};
    std::atomic<int64_t> held{0};
    std::atomic<int64_t> hits{0}, misses{0};

    uint64_t take(uint64_t bytes) {
        uint64_t ptr = 0;
        if (lock()) {
            auto it = free_.find(bytes);
            if (it != free_.end() && !it->second.empty()) {
                ptr = it->second.back();
                it->second.pop_back();
                held.fetch_sub((int64_t)bytes);
            }
            unlock();
        }
        (ptr ? hits : misses).fetch_add(1);
        return ptr;
    }

    bool give(uint64_t ptr, uint64_t bytes) {
        if (bytes == 0 || !lock()) return false;
        bool kept = false;
        if (held.load() + (int64_t)bytes <= limit.load()) {
            free_[bytes].push_back(ptr);
            held.fetch_add((int64_t)bytes);
            kept = true;
        }
        unlock();
        return kept;
    }

    // Frees everything held (at process teardown or on request).
    template <typename F>
    void drain_all(F&& free_fn) {
        while (!lock()) std::this_thread::yield();
        for (auto& [bytes, list] : free_)
            for (uint64_t p : list) free_fn(p, bytes);
        free_.clear();
        held.store(0);
        unlock();
    }

  private:
    std::unordered_map<uint64_t, std::vector<uint64_t>> free_;
    std::atomic<bool> lock_{false};
    bool lock() {
        bool expected = false;
        return lock_.compare_exchange_strong(expected, true);
    }
    void unlock() { lock_.store(false); }
};

// Memory given back from any thread, waiting to move into the pool, as
// RetiredList (buffer_pool.cr:87-129): `push` never allocates and never
// waits; it stores into one of two fixed arrays and returns false when busy
// or full. `drain` swaps the arrays, on the device's own calls only.
class Retired {
  public:
    static constexpr int CAPACITY = 16384;
    struct Entry {
        uint64_t ptr, bytes;
    };

    bool push(uint64_t ptr, uint64_t bytes) {
        bool expected = false;
        if (!lock_.compare_exchange_strong(expected, true)) return false;
        bool kept = false;
        const int count = count_.load();
        if (count < CAPACITY) {
            filling_[count] = Entry{ptr, bytes};
            count_.store(count + 1);
            kept = true;
        }
        lock_.store(false);
        return kept;
    }

    // One drain at a time (callers on several threads wait here, never a
    // push): a second drain would swap the array the first is still reading
    // back into use, where pushes would overwrite its entries.
    template <typename F>
    void drain(F&& each) {
        std::lock_guard<std::mutex> one(draining_lock_);
        if (count_.load() == 0) return;
        bool expected = false;
        while (!lock_.compare_exchange_strong(expected, true)) {
            expected = false;
            std::this_thread::yield();
        }
        Entry* full = filling_;
        const int count = count_.load();
        filling_ = draining_;
        draining_ = full;
        count_.store(0);
        lock_.store(false);
        for (int i = 0; i < count; ++i) each(full[i].ptr, full[i].bytes);
    }

  private:
    Entry a_[CAPACITY];
    Entry b_[CAPACITY];
    Entry* filling_ = a_;
    Entry* draining_ = b_;
    std::atomic<int> count_{0};
    std::atomic<bool> lock_{false};
    std::mutex draining_lock_;
};

}  // namespace tmh
