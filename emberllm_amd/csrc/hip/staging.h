// staging.h — host-side copies into and out of pinned staging slots, split
// over a few threads (the weight upload and the requantizer stream
// hundreds of MB through such slots; one thread copies at about 6 GB/s from
// a mapped file, eight at about 22 GB/s).
#pragma once

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

namespace ehip {

struct CopySpan {
    uint8_t *dst;
    const uint8_t *src;
    size_t len;
};

// Host threads to use for staging copies.
inline int staging_threads() {
    return (int)std::min(8u, std::max(1u, std::thread::hardware_concurrency()));
}

// Perform every span's copy.  The spans' bytes, taken in order, are split
// into up to `threads` equal pieces of at least 1 MiB; each piece is copied by
// its own thread (the first by the calling thread).
inline void parallel_copy(const std::vector<CopySpan> &spans, int threads) {
    size_t total = 0;
    for (const CopySpan &s : spans) total += s.len;
    if (total == 0) return;
    const int nt = (int)std::max<size_t>(1, std::min<size_t>((size_t)threads, total >> 20));
    const size_t piece = (total + nt - 1) / nt;
    auto run = [&spans](size_t lo, size_t hi) {   // bytes [lo, hi) of the concatenation
        size_t at = 0;
        for (const CopySpan &s : spans) {
            const size_t a = std::max(lo, at), b = std::min(hi, at + s.len);
            if (a < b) memcpy(s.dst + (a - at), s.src + (a - at), b - a);
            at += s.len;
            if (at >= hi) break;
        }
    };
    std::vector<std::thread> ts;
    for (int t = 1; t < nt; t++) ts.emplace_back(run, t * piece, std::min(total, (t + 1) * piece));
    run(0, std::min(total, piece));
    for (auto &t : ts) t.join();
}

}  // namespace ehip
