#include "pool.hpp"

#include <limits>
#include <tuple>

namespace mh {

int64_t best_fit(const uint64_t *lens, const uint64_t *caps, int64_t count, uint64_t len) {
    int64_t best = -1;
    std::tuple<int, uint64_t> best_key{3, 0};
    for (int64_t i = 0; i < count; ++i) {
        const uint64_t l = lens[i], cap = caps[i];
        std::tuple<int, uint64_t> key;
        if (l >= len)
            key = {0, l};
        else if (cap >= len)
            key = {1, len - l};
        else
            key = {2, std::numeric_limits<uint64_t>::max() - cap};
        if (best < 0 || key <= best_key) {  // `<=`: later entries win ties
            best = i;
            best_key = key;
        }
    }
    return best;
}

Pool::~Pool() {
    if (!bufs_.empty()) (void)hipStreamSynchronize(ctx_.stream);
    for (auto &b : bufs_) (void)hipFree(b.p);
}

// The idle buffer with the least capacity that holds `count` floats (later
// entries win ties), else a new buffer. The reference's Scratch grows its
// largest idle buffer in place (best_fit, src/engine/mod.rs:104-117); on the
// device that takes a stream synchronisation and a hipFree, which stalled the
// host for 0.3-0.6 ms per growth for several steps, so buffers are never grown
// or freed here: the set only gains buffers until the step's pattern of sizes
// is covered, after which no step allocates.
float *Pool::floats(int64_t count) {
    const uint64_t len = uint64_t(count > 0 ? count : 1);
    Buf *best = nullptr;
    for (auto &b : bufs_)
        if (!b.used && b.cap >= len && (!best || b.cap <= best->cap)) best = &b;
    if (best) {
        best->len = len;
        best->used = true;
        return best->p;
    }
    Buf b{nullptr, len, len, true};
    mh::dev_malloc(&b.p, len * sizeof(float));
    bufs_.push_back(b);
    ++allocations_;
    return b.p;
}

DT Pool::tensor(int n, int h, int w, int c) {
    DT t;
    t.n = n, t.h = h, t.w = w, t.c = c;
    t.p = floats(t.numel());
    return t;
}

void Pool::recycle(float *p) {
    if (!p) return;
    for (auto &b : bufs_)
        if (b.p == p) {
            b.used = false;
            return;
        }
    fail(kInternal, "pool: recycling a buffer it does not own");
}

void Pool::release_below(int64_t min_floats) {
    bool synced = false;
    for (size_t i = 0; i < bufs_.size();) {
        if (!bufs_[i].used && bufs_[i].cap < uint64_t(min_floats)) {
            if (!synced) {
                HIP_CHECK(hipStreamSynchronize(ctx_.stream));
                synced = true;
            }
            HIP_CHECK(hipFree(bufs_[i].p));
            bufs_.erase(bufs_.begin() + int64_t(i));
        } else {
            ++i;
        }
    }
}

size_t Pool::bytes_held() const {
    size_t s = 0;
    for (auto &b : bufs_) s += b.cap * sizeof(float);
    return s;
}

}  // namespace mh
