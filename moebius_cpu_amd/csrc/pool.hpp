// Device activation pool: the HBM analogue of the reference's `Scratch`
// (src/engine/mod.rs:25-117). Buffers are handed out best-fit by size and
// returned after their last use; roles ask for the same sizes in the same order
// every step, so after the first step each role gets its buffer back and
// nothing is allocated again.
#pragma once

#include <cstdint>
#include <vector>

#include "common.hpp"

namespace mh {

// src/engine/mod.rs:104-117: index of the best buffer for `len` among (len, cap)
// pairs: the shortest one already holding `len`, else the one needing the
// least growth within its capacity, else the largest; later entries win ties.
// -1 when there are none.
int64_t best_fit(const uint64_t *lens, const uint64_t *caps, int64_t count, uint64_t len);

struct DT {  // device NHWC f32 tensor view
    float *p = nullptr;
    int n = 0, h = 0, w = 0, c = 0;
    // GroupNorm statistics partials of the values, written by the producer's
    // epilogue (see GnPartials), or null: [px / gn_rows][c][2], pool-owned.
    float *gn = nullptr;
    int gn_rows = 0;
    int64_t px() const { return int64_t(n) * h * w; }
    int64_t numel() const { return px() * c; }
};

class Pool {
  public:
    explicit Pool(Context &ctx) : ctx_(ctx) {}
    ~Pool();
    Pool(const Pool &) = delete;
    Pool &operator=(const Pool &) = delete;
    // A buffer of at least n*h*w*c floats shaped as given (contents unspecified).
    DT tensor(int n, int h, int w, int c);
    float *floats(int64_t count);
    void recycle(const DT &t) {
        recycle(t.p);
        recycle(t.gn);
    }
    void recycle(float *p);
    // Frees every idle buffer smaller than min_floats (src/engine/mod.rs:87-91).
    void release_below(int64_t min_floats);
    size_t bytes_held() const;
    // Device allocations made so far (a step that allocates nothing leaves it unchanged).
    int64_t allocations() const { return allocations_; }

  private:
    struct Buf {
        float *p;
        uint64_t len, cap;  // floats
        bool used;
    };
    Context &ctx_;
    std::vector<Buf> bufs_;
    int64_t allocations_ = 0;
};

}  // namespace mh
