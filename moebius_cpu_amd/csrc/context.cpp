// Context, workspace and error plumbing.
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
    // The no-allocation entry points' fixed scratch: its device address on this GPU.
    noalloc_scratch_setup(dev);
    HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
}

Context::~Context() {
    if (stream) (void)hipStreamSynchronize(stream);
    if (stream) (void)hipStreamDestroy(stream);
}

}  // namespace mh
