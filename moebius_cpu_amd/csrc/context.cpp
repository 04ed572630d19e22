// Context, workspace and error plumbing.
#include <cstring>
#include <sstream>

#include "common.hpp"

namespace mh {

void fail(int32_t code, const std::string &msg) { throw Error(code, msg); }

void hip_fail(hipError_t e, const char *expr, const char *file, int line) {
    std::ostringstream os;
    os << "HIP error " << hipGetErrorName(e) << " (" << hipGetErrorString(e) << ") at " << file << ":" << line
       << ": " << expr;
    throw Error(e == hipErrorOutOfMemory ? kOutOfMemory : kInternal, os.str());
}

Workspace::~Workspace() {
    if (ptr_) (void)hipFree(ptr_);
}

void *Workspace::get(size_t bytes, hipStream_t stream) {
    if (bytes <= cap_) return ptr_;
    HIP_CHECK(hipStreamSynchronize(stream));
    if (ptr_) HIP_CHECK(hipFree(ptr_));
    ptr_ = nullptr;
    cap_ = 0;
    const size_t want = (bytes + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1);
    HIP_CHECK(hipMalloc(&ptr_, want));
    cap_ = want;
    return ptr_;
}

Context::Context(int dev) : device(dev) {
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
    HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
    HIP_CHECK(hipMalloc(&counters, kCounters * sizeof(unsigned int)));
    HIP_CHECK(hipMemset(counters, 0, kCounters * sizeof(unsigned int)));
    HIP_CHECK(hipDeviceSynchronize());
}

Context::~Context() {
    if (stream) (void)hipStreamSynchronize(stream);
    if (counters) (void)hipFree(counters);
    if (stream) (void)hipStreamDestroy(stream);
}

// Counter slots are handed out round-robin. A slot is only in use while its
// kernel runs, and kernels on the one stream run in order, so reuse is safe as
// long as one launch takes fewer slots than the ring holds.
unsigned int *Context::counter_block(int n) {
    if (n > kCounters) fail(kInternal, "counter request exceeds the counter ring");
    if (next_counter + n > kCounters) next_counter = 0;
    unsigned int *p = counters + next_counter;
    next_counter += n;
    return p;
}

}  // namespace mh
