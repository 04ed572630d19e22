// Shared host-side plumbing of the HIP library: errors, the per-device
// context (stream + workspace arena), device helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace mh {

// Status codes of include/moebius_hip.h (the reference's moebius_cpu.h:13-19 values).
enum Status : int32_t {
    kOk = 0,
    kInvalidArgument = 1,
    kWeights = 2,
    kUnsupportedDevice = 3,
    kCancelled = 4,
    kIo = 5,
    kInternal = 6,
    kOutOfMemory = 7,
};

struct Error : std::runtime_error {
    int32_t code;
    Error(int32_t c, const std::string &m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] void fail(int32_t code, const std::string &msg);
[[noreturn]] void hip_fail(hipError_t e, const char *expr, const char *file, int line);

#define MH_REQUIRE(cond, msg)                                         \
    do {                                                              \
        if (!(cond)) ::mh::fail(::mh::kInvalidArgument, (msg));      \
    } while (0)

#define HIP_CHECK(expr)                                                          \
    do {                                                                         \
        hipError_t e_ = (expr);                                                  \
        if (e_ != hipSuccess) ::mh::hip_fail(e_, #expr, __FILE__, __LINE__);     \
    } while (0)

#define MH_LAUNCH_CHECK() HIP_CHECK(hipGetLastError())

enum class Precision : uint32_t { Exact = 0, Fast = 1 };

// A GEMM tiling forced for every GEMM of one shape (Tuning::gemm_shape_plan).
struct ShapePlan {
    int m = 0, n = 0, k = 0;
    int bm = 0, bn = 0, splits = 0, wm = 2, wn = 2, wk = 1, pipe = 0, bk = 32;
};

// Tuning overrides for A/B runs and tests, read once from the environment
// (MOEBIUS_HIP_GEMM_PLAN, _GN_IN_MAXC, _DW_TILED, _TAP_HEADS, _CROSS_HEADS,
// _GN_BLOCKS, _GN_APPLY, _WINO_FUSED, _UP_CONCAT, _LAMBDA_TAPS, _GEMM_LOG,
// _GEMM_WIDE, _LN_FOLD, _TAP_SPLIT, _GEMM_TIME, _TAPS_ROWS, _CROSS_MFMA, _TAP_SLICE,
// _TAP_JQ, _TAP_FUSED, _GEMM_SHAPE_PLAN, _TAPS_R16, _WINO_U16, _WINO_V16, _DW_OUT16)
// when a context is created and changed with set_tuning (mh_context_set_tuning).
// The defaults are the measured choices; nothing on the hot path reads the
// environment.
struct Tuning {
    int gemm_bm = 0, gemm_bn = 0, gemm_splits = 0;  // forced GEMM tiling, 0: the planner's
    int gemm_wm = 2, gemm_wn = 2, gemm_wk = 1;       // and its wave layout (f32 kernel)
    int gemm_pipe = 0;                               // and its main loop (1: pipelined)
    int gemm_bk = 32;                                // and its K per LDS stage
    int gn_in_maxc = -1;   // GroupNorm applied in proj_in's loads up to this width; -1: per precision
    int dw_tiled = 1;      // 0: the register-window depthwise kernel
    int tap_tile = -1;     // tap filter: -1 default; 0 the per-thread kernel; 4 / 8 the tile kernel's heads
    int tap_heads = 0;     // per-thread tap filter heads per thread (0: default)
    int cross_heads = 0;   // cross-lambda heads per thread (0: default)
    int gn_blocks = 512;   // GroupNorm statistics: at most this many partial blocks per launch
    int gn_apply = 0;      // GroupNorm apply pass: 1 walks the map from its end
    int wino_fused = -1;   // Winograd convs in one kernel: -1 where faster, 1 wherever it fits, 0 never
    int up_concat = 0;     // 1: the UNet's up path writes [h | skip] before each resnet (the reference's order)
    int lambda_taps = 1;   // 0: the self-lambda's position coefficients through the general GEMM
    int gemm_log = 0;      // 1: print each GEMM launch's shape and tiling to stderr (launch census)
    int gemm_wide = 1;     // 0: the square tilings only (no wide wave layouts from the planner)
    int ln_fold = 2;       // the transformers' LayerNorms 1 and 3 folded into the GEMMs that read them, with
                           // the row statistics from the producers' partials (2) or summed by the GEMMs
                           // (1); 0: LayerNorm passes of their own
    int tap_split = 0;     // per-thread tap filter: tap rows split over 1, 3 or 5 threads (0: by map size)
    int gemm_time = 0;     // 1: record events around each GEMM launch (Context::gemm_times)
    int taps_rows = 0;     // lambda position coefficients: rows per part (80, 48, 16; 0: by map size)
    int cross_mfma = 1;    // cross-lambda: 1 the content term on the matrix cores (head widths 40, 80, 160)
    int tap_slice = 0;     // tap filter: > 0 the tile kernel on value channel slices of this many quads
    int tap_jq = 1;        // tap filter tile kernel: value channel quads per thread (1 or 2)
    // gemm_shape_plan: "M,N,K,bm,bn,splits[,wm,wn,wk[,pipe[,bk]]]" entries joined by ';'
    // (at most 8), each forcing the tiling of the GEMMs of that shape as gemm_plan does for all
    ShapePlan shape_plans[8];
    int n_shape_plans = 0;
    int tap_fused = 1;     // self-lambda coefficients formed inside the tap filter, per head width:
                           // bit 0 k = 40 (the 64x64 latents), bit 1 k = 80, bit 2 k = 160
    int taps_r16 = 0;      // FAST contexts: 1 the self-lambda position products on f16-rounded operands
                           // (as the FAST GEMMs take them); 0 on the f32 operands (faster)
    int wino_u16 = 1;      // FAST contexts: the UNet's Winograd plane GEMMs read U stored in f16 (0: f32,
                           // rounded on every load; the same products)
    int wino_v16 = 1;      // FAST contexts with an f16 U: the input transform writes V in f16 (0: f32)
    int dw_out16 = 1;      // FAST contexts: depthwise convs read only by an f16 GEMM write f16 (0: f32)
};
// Sets `key` from its text form (the environment variable's syntax); value NULL
// or "" restores the default. False for an unknown key or a malformed value.
bool set_tuning(Tuning &t, const char *key, const char *value);

// Every device allocation the library makes goes through here, so that the
// count of them (device_allocations, mh_device_allocations) shows which calls
// allocate.
void dev_malloc_bytes(void **p, size_t bytes);
template <class T>
inline void dev_malloc(T **p, size_t bytes) {
    void *v = nullptr;
    dev_malloc_bytes(&v, bytes);
    *p = static_cast<T *>(v);
}
uint64_t device_allocations();

// Device arena for kernel scratch (split-K partials, norm partials): grown on
// demand, kept for the context's life, like the reference's `Scratch` panels
// (src/engine/mod.rs:25-34). Growth synchronises the stream first, since
// queued kernels may still read the old block.
class Workspace {
  public:
    Workspace() = default;
    Workspace(const Workspace &) = delete;
    Workspace &operator=(const Workspace &) = delete;
    ~Workspace();
    void *get(size_t bytes, hipStream_t stream);
    // Frees the buffer once the stream has drained; the next get allocates again.
    void release(hipStream_t stream);
    size_t capacity() const { return cap_; }

  private:
    void *ptr_ = nullptr;
    size_t cap_ = 0;
};

struct Context {
    int device = 0;
    hipStream_t stream = nullptr;
    Precision precision = Precision::Exact;
    int cu_count = 0;
    std::string arch;
    Workspace ws;
    // State that outlives single kernels inside one multi-step call (the denoise
    // loop's latents, UNet input, eps and solver history): grow-only like ws,
    // and apart from it, since the kernels of each step draw on ws.
    Workspace state;
    Tuning tune;
    // GEMM launches timed on the device while tune.gemm_time is set: events
    // recorded before and after each launch (its split-K reduce included),
    // keyed by the kernel configuration, read and cleared by the caller.
    struct GemmTime {
        std::string key;
        double flops;
        hipEvent_t start, stop;
    };
    std::vector<GemmTime> gemm_times;
    std::vector<hipEvent_t> spare_events;
    hipEvent_t take_event();

    explicit Context(int dev);
    ~Context();
    Context(const Context &) = delete;
    Context &operator=(const Context &) = delete;
};

// Sets the context's GEMM precision for a scope, then restores it.
struct PrecisionScope {
    Context &ctx;
    Precision saved;
    PrecisionScope(Context &c, Precision p) : ctx(c), saved(c.precision) { c.precision = p; }
    ~PrecisionScope() { ctx.precision = saved; }
    PrecisionScope(const PrecisionScope &) = delete;
    PrecisionScope &operator=(const PrecisionScope &) = delete;
};

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// NULL counts as aligned (an absent optional operand).
inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace mh
