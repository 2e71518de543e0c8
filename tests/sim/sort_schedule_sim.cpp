// CPU model of the radix pass's tile order and decoupled look-back
// (xlog_amd/csrc/sort.hip: chunk_tile, k_onesweep, radix_sort_u64's grid).
//
// Threads play workgroups.  Blocks are dispatched into `cap` slots (a slot
// frees when its block ends), in index order or, in mode "shuffled", in a
// random order; a starting block takes the next ticket b and runs tile
// ((b/8)/chunk*8 + b%8)*chunk + (b/8)%chunk, publishes its aggregate, walks
// back over 4 predecessors per round until an inclusive prefix, and publishes
// its own inclusive prefix.  Checked: every tile runs once, every exclusive
// prefix is exact, and no run deadlocks (watchdog) when cap >= 8*chunk, the
// condition the host sizes chunk for, whatever the dispatch order.  With cap
// below 8*chunk the same model must be able to deadlock, which shows the
// watchdog detects it.
//
// The mode may also name "index": a block runs the tile of its workgroup index
// (the kernel's default order) instead of its start ticket, and "fallback": the
// look-back's bounded wait (k_onesweep's spin_limit, here 2 failed polls), after
// which the waiting tile counts its unpublished predecessor itself (here: takes
// that tile's count) and walks on.  With the fallback, index order in a
// shuffled dispatch with too few slots must never stall and still give exact
// prefixes; without it the same schedule can stall.
//
// usage: sort_schedule_sim <trials> <watchdog_seconds> <mode: ok|tight|shuffled, with index / fallback>
// prints "runs R failures F hangs H"
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <mutex>
#include <random>
#include <thread>
#include <vector>

static const uint32_t ST_AGG = 1u << 30, ST_INC = 2u << 30, ST_VAL = (1u << 30) - 1, NONE = 0xFFFFFFFFu;

struct Run {
    uint32_t tiles, chunk;
    std::vector<std::atomic<uint32_t>> status;
    std::vector<std::atomic<int>> done;
    std::vector<uint32_t> cnt, prefix;
    std::atomic<bool> abort{false};
    int spin_limit = -1;  // >= 0: the bounded wait
    Run(uint32_t t, uint32_t c) : tiles(t), chunk(c), status(t), done(t), cnt(t), prefix(t) {
        for (uint32_t i = 0; i < t; ++i) {
            status[i] = 0;
            done[i] = 0;
            cnt[i] = 1 + (i * 7919u) % 13;
        }
    }
    // the kernel's chunk_tile
    uint32_t tile_of(uint32_t b) const {
        const uint32_t q = b & 7u, j = b >> 3;
        const uint64_t t = ((uint64_t)(j / chunk) * 8 + q) * chunk + j % chunk;
        return t < tiles ? (uint32_t)t : NONE;
    }
    void process(uint32_t t, std::mt19937 &rng) {
        if (rng() % 3 == 0) std::this_thread::sleep_for(std::chrono::microseconds(rng() % 40));
        status[t].store((t == 0 ? ST_INC : ST_AGG) | cnt[t]);
        uint32_t p = 0;
        if (t > 0) {
            int64_t j = (int64_t)t - 1;
            bool fin = false;
            int spins = 0;
            while (!fin) {
                if (abort) return;
                uint32_t st[4];
                for (int z = 0; z < 4; ++z) st[z] = j - z >= 0 ? status[j - z].load() : ST_INC;
                int used = 0;
                for (int z = 0; z < 4; ++z) {
                    const uint32_t f = st[z] & ~ST_VAL;
                    if (f == 0) break;
                    p += st[z] & ST_VAL;
                    used = z + 1;
                    if (f == ST_INC) {
                        fin = true;
                        break;
                    }
                }
                j -= used;
                if (used) {
                    spins = 0;
                } else if (spin_limit >= 0 && ++spins > spin_limit) {  // count tile j here
                    p += cnt[j];
                    j -= 1;
                    spins = 0;
                    fin = j < 0;
                } else {
                    std::this_thread::yield();
                }
            }
            status[t].store(ST_INC | (p + cnt[t]));
        }
        prefix[t] = p;
        done[t].fetch_add(1);
    }
};

int main(int argc, char **argv) {
    const int trials = argc > 1 ? atoi(argv[1]) : 40;
    const int watchdog = argc > 2 ? atoi(argv[2]) : 10;
    const char *mode = argc > 3 ? argv[3] : "ok";
    const bool tight = strstr(mode, "tight") != nullptr;
    const bool shuffled = strstr(mode, "shuffled") != nullptr;
    const bool by_index = strstr(mode, "index") != nullptr;
    const bool fallback = strstr(mode, "fallback") != nullptr;
    std::mt19937 rng(2024);
    int runs = 0, failures = 0, hangs = 0;
    for (int trial = 0; trial < trials; ++trial) {
        const uint32_t tiles = tight ? 300 + rng() % 300 : 1 + rng() % 900;
        // the host's chunk: at most 1/16 of the device's blocks, at most 8,
        // smaller when there are few tiles
        uint32_t cap = tight ? 0 : 8 + rng() % 600;
        uint32_t chunk = cap / 16 < 8 ? (cap / 16 > 0 ? cap / 16 : 1) : 8;
        if (tight) {
            chunk = 8;
            cap = 2 + rng() % 30;  // below 8 * chunk
        }
        if (!tight && tiles / 64 < chunk) chunk = tiles / 64 > 0 ? tiles / 64 : 1;
        if (!tight && cap < 8 * chunk) cap = 8 * chunk;  // what the host guarantees by sizing chunk
        const uint32_t nchunks = (tiles + chunk - 1) / chunk;
        const uint32_t grid = 8 * ((nchunks + 7) / 8) * chunk;
        Run r(tiles, chunk);
        if (fallback) r.spin_limit = 2;
        std::vector<uint32_t> order(grid);  // dispatch order of the block indices
        for (uint32_t b = 0; b < grid; ++b) order[b] = b;
        if (shuffled) std::shuffle(order.begin(), order.end(), rng);
        std::atomic<uint32_t> ticket{0};
        std::mutex mu;
        std::condition_variable cv;
        uint32_t running = 0;
        std::vector<std::thread> th;
        const auto t0 = std::chrono::steady_clock::now();
        bool hung = false;
        for (uint32_t b = 0; b < grid && !hung; ++b) {
            std::unique_lock<std::mutex> lk(mu);
            while (running >= cap) {
                if (cv.wait_for(lk, std::chrono::milliseconds(20)) == std::cv_status::timeout &&
                    std::chrono::steady_clock::now() - t0 > std::chrono::seconds(watchdog)) {
                    hung = true;
                    break;
                }
            }
            if (hung) break;
            ++running;
            lk.unlock();
            th.emplace_back([&, b] {
                std::mt19937 lr(order[b] * 31u + (uint32_t)trial);
                // the kernel's start-order ticket, or the block's own index
                const uint32_t t = r.tile_of(by_index ? order[b] : ticket.fetch_add(1));
                if (t != NONE) r.process(t, lr);
                std::lock_guard<std::mutex> g(mu);
                --running;
                cv.notify_all();
            });
        }
        while (!hung) {  // the last blocks
            int fin = 0;
            for (uint32_t i = 0; i < tiles; ++i) fin += r.done[i].load() > 0;
            if (fin == (int)tiles) break;
            if (std::chrono::steady_clock::now() - t0 > std::chrono::seconds(watchdog)) hung = true;
            else std::this_thread::sleep_for(std::chrono::milliseconds(1));
        }
        if (hung) r.abort = true;
        for (auto &t : th) t.join();
        ++runs;
        if (hung) {
            ++hangs;
            continue;
        }
        uint32_t acc = 0;
        for (uint32_t i = 0; i < tiles; ++i) {
            if (r.done[i].load() != 1 || r.prefix[i] != acc) {
                ++failures;
                printf("trial %d tiles %u chunk %u cap %u: tile %u done %d prefix %u want %u\n", trial, tiles, chunk,
                       cap, i, r.done[i].load(), r.prefix[i], acc);
                break;
            }
            acc += r.cnt[i];
        }
    }
    printf("runs %d failures %d hangs %d\n", runs, failures, hangs);
    return 0;
}
