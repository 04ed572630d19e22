// Error plumbing shared by the C-ABI translation units: every entry point runs
// its body inside guard(), which turns an mh::Error or any other exception
// into a status code and a thread-local message (the reference's FFI guard,
// src/ffi.rs:90-103, and moebius_last_error, include/moebius_cpu.h:50-51).
#pragma once

#include <exception>
#include <new>
#include <string>

#include "common.hpp"

namespace mh {
namespace capi {

inline thread_local std::string last_error = "no error";

inline int32_t set_error(int32_t code, const std::string &msg) {
    last_error = msg;
    return code;
}

template <typename F>
int32_t guard(F &&f) {
    try {
        f();
        return kOk;
    } catch (const Error &e) {
        return set_error(e.code, e.what());
    } catch (const std::bad_alloc &) {
        return set_error(kOutOfMemory, "host allocation failed");
    } catch (const std::exception &e) {
        return set_error(kInternal, std::string("internal error: ") + e.what());
    } catch (...) {
        return set_error(kInternal, "internal error: unknown exception");
    }
}

inline void need(const void *p, const char *what) {
    if (!p) fail(kInvalidArgument, std::string(what) + " is NULL");
}

}  // namespace capi
}  // namespace mh
