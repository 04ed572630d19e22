// Context, workspace and error plumbing.
#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <sstream>

#include "common.hpp"
#include "kernels.hpp"

namespace mh {

void fail(int32_t code, const std::string &msg) { throw Error(code, msg); }

void hip_fail(hipError_t e, const char *expr, const char *file, int line) {
    std::ostringstream os;
    os << "HIP error " << hipGetErrorName(e) << " (" << hipGetErrorString(e) << ") at " << file << ":" << line
       << ": " << expr;
    throw Error(e == hipErrorOutOfMemory ? kOutOfMemory : kInternal, os.str());
}

namespace {
std::atomic<uint64_t> g_allocations{0};
}

void dev_malloc_bytes(void **p, size_t bytes) {
    HIP_CHECK(hipMalloc(p, bytes ? bytes : 1));
    g_allocations.fetch_add(1, std::memory_order_relaxed);
}

uint64_t device_allocations() { return g_allocations.load(std::memory_order_relaxed); }

Workspace::~Workspace() {
    if (ptr_) (void)hipFree(ptr_);
}

void Workspace::release(hipStream_t stream) {
    if (!ptr_) return;
    HIP_CHECK(hipStreamSynchronize(stream));
    HIP_CHECK(hipFree(ptr_));
    ptr_ = nullptr;
    cap_ = 0;
}

void *Workspace::get(size_t bytes, hipStream_t stream) {
    if (bytes <= cap_) return ptr_;
    HIP_CHECK(hipStreamSynchronize(stream));
    if (ptr_) HIP_CHECK(hipFree(ptr_));
    ptr_ = nullptr;
    cap_ = 0;
    const size_t want = (bytes + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1);
    dev_malloc(&ptr_, want);
    cap_ = want;
    return ptr_;
}

bool set_tuning(Tuning &t, const char *key, const char *value) {
    const std::string k = key ? key : "";
    const bool clear = !value || !*value;
    const std::string v = clear ? "" : value;
    auto to_int = [&](int &dst, int def) {
        if (clear) {
            dst = def;
            return true;
        }
        char *end = nullptr;
        const long x = std::strtol(v.c_str(), &end, 10);
        if (!end || *end) return false;
        dst = int(x);
        return true;
    };
    if (k == "gemm_plan") {  // "bm,bn,splits" or "bm,bn,splits,wm,wn,wk[,pipe[,bk]]"
        t.gemm_wm = 2, t.gemm_wn = 2, t.gemm_wk = 1, t.gemm_pipe = 0, t.gemm_bk = 32;
        if (clear) {
            t.gemm_bm = t.gemm_bn = t.gemm_splits = 0;
            return true;
        }
        int bm = 0, bn = 0, sp = 0, wm = 2, wn = 2, wk = 1, pipe = 0, bk = 32;
        const int got = std::sscanf(v.c_str(), "%d,%d,%d,%d,%d,%d,%d,%d", &bm, &bn, &sp, &wm, &wn, &wk, &pipe, &bk);
        if ((got != 3 && got < 6) || sp < 1 || wm < 1 || wn < 1 || wk < 1 || pipe < 0 || pipe > 1 ||
            (bk != 16 && bk != 32))
            return false;
        t.gemm_bm = bm, t.gemm_bn = bn, t.gemm_splits = sp;
        t.gemm_wm = wm, t.gemm_wn = wn, t.gemm_wk = wk, t.gemm_pipe = pipe, t.gemm_bk = bk;
        return true;
    }
    if (k == "gemm_shape_plan") {
        t.n_shape_plans = 0;
        if (clear) return true;
        size_t pos = 0;
        while (pos <= v.size()) {
            const size_t end = std::min(v.find(';', pos), v.size());
            const std::string e = v.substr(pos, end - pos);
            pos = end + 1;
            if (e.empty()) continue;
            ShapePlan sp;
            const int got = std::sscanf(e.c_str(), "%d,%d,%d,%d,%d,%d,%d,%d,%d,%d,%d", &sp.m, &sp.n, &sp.k, &sp.bm,
                                        &sp.bn, &sp.splits, &sp.wm, &sp.wn, &sp.wk, &sp.pipe, &sp.bk);
            if ((got != 6 && got < 9) || t.n_shape_plans >= 8 || sp.splits < 1 || sp.wm < 1 || sp.wn < 1 ||
                sp.wk < 1 || sp.pipe < 0 || sp.pipe > 1 || (sp.bk != 16 && sp.bk != 32)) {
                t.n_shape_plans = 0;
                return false;
            }
            t.shape_plans[t.n_shape_plans++] = sp;
        }
        return true;
    }
    if (k == "gn_in_maxc") return to_int(t.gn_in_maxc, -1);
    if (k == "dw_tiled") return to_int(t.dw_tiled, 1);
    if (k == "cross_heads") return to_int(t.cross_heads, 0);
    if (k == "gn_blocks") return to_int(t.gn_blocks, 512) && t.gn_blocks >= 64;
    if (k == "gn_apply") return to_int(t.gn_apply, 0) && t.gn_apply >= 0 && t.gn_apply <= 1;
    if (k == "wino_fused") return to_int(t.wino_fused, -1) && t.wino_fused >= -1 && t.wino_fused <= 1;
    if (k == "up_concat") return to_int(t.up_concat, 0) && t.up_concat >= 0 && t.up_concat <= 1;
    if (k == "lambda_taps") return to_int(t.lambda_taps, 1) && t.lambda_taps >= 0 && t.lambda_taps <= 1;
    if (k == "gemm_log") return to_int(t.gemm_log, 0);
    if (k == "tap_fused") return to_int(t.tap_fused, 1) && t.tap_fused >= 0 && t.tap_fused <= 7;
    if (k == "taps_r16") return to_int(t.taps_r16, 0) && t.taps_r16 >= 0 && t.taps_r16 <= 1;
    if (k == "wino_u16") return to_int(t.wino_u16, 1) && t.wino_u16 >= 0 && t.wino_u16 <= 1;
    if (k == "wino_v16") return to_int(t.wino_v16, 1) && t.wino_v16 >= 0 && t.wino_v16 <= 1;
    if (k == "dw_out16") return to_int(t.dw_out16, 1) && t.dw_out16 >= 0 && t.dw_out16 <= 1;
    if (k == "tap_jq") return to_int(t.tap_jq, 1) && (t.tap_jq == 1 || t.tap_jq == 2);
    if (k == "tap_slice") return to_int(t.tap_slice, 0) && t.tap_slice >= 0 && t.tap_slice <= 64;
    if (k == "cross_mfma") return to_int(t.cross_mfma, 1) && t.cross_mfma >= 0 && t.cross_mfma <= 1;
    if (k == "taps_rows")
        return to_int(t.taps_rows, 0) && (t.taps_rows == 0 || t.taps_rows == 80 || t.taps_rows == 48 ||
                                          t.taps_rows == 16);
    if (k == "gemm_time") return to_int(t.gemm_time, 0) && t.gemm_time >= 0 && t.gemm_time <= 1;
    if (k == "gemm_wide") return to_int(t.gemm_wide, 1) && t.gemm_wide >= 0 && t.gemm_wide <= 1;
    if (k == "ln_fold") return to_int(t.ln_fold, 2) && t.ln_fold >= 0 && t.ln_fold <= 2;
    if (k == "tap_split") return to_int(t.tap_split, 0) && (t.tap_split == 0 || t.tap_split == 1 || t.tap_split == 3 ||
                                                            t.tap_split == 5);
    if (k == "tap_heads") {
        if (clear) {
            t.tap_tile = -1, t.tap_heads = 0;
            return true;
        }
        if (v[0] == 't') {
            t.tap_tile = std::atoi(v.c_str() + 1) == 4 ? 4 : 8;
            t.tap_heads = 0;
        } else {
            t.tap_tile = 0;
            if (!to_int(t.tap_heads, 0)) return false;
        }
        return true;
    }
    return false;
}

Context::Context(int dev) : device(dev) {
    static const char *const env_keys[][2] = {{"MOEBIUS_HIP_GEMM_PLAN", "gemm_plan"},
                                              {"MOEBIUS_HIP_GN_IN_MAXC", "gn_in_maxc"},
                                              {"MOEBIUS_HIP_DW_TILED", "dw_tiled"},
                                              {"MOEBIUS_HIP_TAP_HEADS", "tap_heads"},
                                              {"MOEBIUS_HIP_CROSS_HEADS", "cross_heads"},
                                              {"MOEBIUS_HIP_GN_BLOCKS", "gn_blocks"},
                                              {"MOEBIUS_HIP_GN_APPLY", "gn_apply"},
                                              {"MOEBIUS_HIP_WINO_FUSED", "wino_fused"},
                                              {"MOEBIUS_HIP_UP_CONCAT", "up_concat"},
                                              {"MOEBIUS_HIP_LAMBDA_TAPS", "lambda_taps"},
                                              {"MOEBIUS_HIP_GEMM_LOG", "gemm_log"},
                                              {"MOEBIUS_HIP_GEMM_WIDE", "gemm_wide"},
                                              {"MOEBIUS_HIP_GEMM_TIME", "gemm_time"},
                                              {"MOEBIUS_HIP_TAPS_ROWS", "taps_rows"},
                                              {"MOEBIUS_HIP_CROSS_MFMA", "cross_mfma"},
                                              {"MOEBIUS_HIP_TAP_SLICE", "tap_slice"},
                                              {"MOEBIUS_HIP_TAP_JQ", "tap_jq"},
                                              {"MOEBIUS_HIP_TAP_FUSED", "tap_fused"},
                                              {"MOEBIUS_HIP_GEMM_SHAPE_PLAN", "gemm_shape_plan"},
                                              {"MOEBIUS_HIP_TAPS_R16", "taps_r16"},
                                              {"MOEBIUS_HIP_WINO_U16", "wino_u16"},
                                              {"MOEBIUS_HIP_WINO_V16", "wino_v16"},
                                              {"MOEBIUS_HIP_DW_OUT16", "dw_out16"},
                                              {"MOEBIUS_HIP_LN_FOLD", "ln_fold"},
                                              {"MOEBIUS_HIP_TAP_SPLIT", "tap_split"}};
    for (const auto &kv : env_keys)
        if (const char *e = std::getenv(kv[0])) set_tuning(tune, kv[1], e);
    int count = 0;
    HIP_CHECK(hipGetDeviceCount(&count));
    if (dev < 0 || dev >= count) fail(kInvalidArgument, "device ordinal out of range");
    HIP_CHECK(hipSetDevice(dev));
    hipDeviceProp_t prop;
    HIP_CHECK(hipGetDeviceProperties(&prop, dev));
    arch = prop.gcnArchName;
    const std::string base = arch.substr(0, arch.find(':'));
    if (base != "gfx950") {
        fail(kUnsupportedDevice, "this library is built for gfx950 (MI355X) only; device is " + arch);
    }
    cu_count = prop.multiProcessorCount;
    // The no-allocation entry points' fixed scratch: its device address on this GPU.
    noalloc_scratch_setup(dev);
    HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
}

Context::~Context() {
    if (stream) (void)hipStreamSynchronize(stream);
    for (const GemmTime &g : gemm_times) {
        (void)hipEventDestroy(g.start);
        (void)hipEventDestroy(g.stop);
    }
    for (hipEvent_t e : spare_events) (void)hipEventDestroy(e);
    if (stream) (void)hipStreamDestroy(stream);
}

hipEvent_t Context::take_event() {
    if (!spare_events.empty()) {
        hipEvent_t e = spare_events.back();
        spare_events.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    HIP_CHECK(hipEventCreate(&e));
    return e;
}

}  // namespace mh
