// runtime.hip -- error reporting, device selection and per-thread resources
// of libgllm_hip (the host side of the C ABI in include/gllm_hip.h).
#include <stdarg.h>
#include <stdio.h>

#include <map>
#include <mutex>

#include "gllm_common.h"

namespace gllm {

static thread_local std::string t_error;

void set_error(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_error = buf;
}

int fail(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_error = buf;
    return code;
}

int check(hipError_t e, const char* what) {
    if (e == hipSuccess) return GLLM_OK;
    (void)hipGetLastError();  // clear the sticky non-fatal error state
    return fail(GLLM_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}

namespace {

constexpr int kScratchSlots = 12;

struct ThreadRes {
    int device = -1;
    hipStream_t stream = nullptr;
    void* scratch[kScratchSlots] = {};
    size_t scratch_n[kScratchSlots] = {};
    void* pinned[kScratchSlots] = {};
    size_t pinned_n[kScratchSlots] = {};
};

thread_local ThreadRes t_res;

int current_device() {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess) return 0;
    return d;
}

// Buffers are kept for the thread's lifetime and never freed at exit: the
// HIP runtime may already be torn down when thread_local destructors run.
void reset_if_device_changed() {
    int d = current_device();
    if (t_res.device != d) {
        t_res = ThreadRes();
        t_res.device = d;
    }
}

}  // namespace

// Compute units of the current device (cached per device).
int device_cus() {
    static int cus[64];
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= 64) return 256;
    if (!cus[d]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, d) != hipSuccess || n <= 0)
            n = 256;
        cus[d] = n;
    }
    return cus[d];
}

hipStream_t thread_stream() {
    reset_if_device_changed();
    if (!t_res.stream) {
        if (hipStreamCreateWithFlags(&t_res.stream, hipStreamNonBlocking) != hipSuccess) {
            t_res.stream = nullptr;
            set_error("hipStreamCreateWithFlags failed");
        }
    }
    return t_res.stream;
}

void* thread_scratch(int slot, size_t bytes) {
    reset_if_device_changed();
    if (slot < 0 || slot >= kScratchSlots) return nullptr;
    if (t_res.scratch_n[slot] < bytes) {
        if (t_res.scratch[slot]) {
            // Another stream of this thread may still read the old buffer.
            (void)hipDeviceSynchronize();
            (void)hipFree(t_res.scratch[slot]);
        }
        size_t n = bytes < 4096 ? 4096 : bytes + bytes / 4;
        void* p = nullptr;
        if (hipMalloc(&p, n) != hipSuccess) {
            (void)hipGetLastError();
            t_res.scratch[slot] = nullptr;
            t_res.scratch_n[slot] = 0;
            set_error("hipMalloc(%zu) for scratch failed", n);
            return nullptr;
        }
        t_res.scratch[slot] = p;
        t_res.scratch_n[slot] = n;
    }
    return t_res.scratch[slot];
}

void* thread_pinned(int slot, size_t bytes) {
    reset_if_device_changed();
    if (slot < 0 || slot >= kScratchSlots) return nullptr;
    if (t_res.pinned_n[slot] < bytes) {
        if (t_res.pinned[slot]) (void)hipHostFree(t_res.pinned[slot]);
        size_t n = bytes < 4096 ? 4096 : bytes + bytes / 4;
        void* p = nullptr;
        if (hipHostMalloc(&p, n, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            t_res.pinned[slot] = nullptr;
            t_res.pinned_n[slot] = 0;
            set_error("hipHostMalloc(%zu) failed", n);
            return nullptr;
        }
        t_res.pinned[slot] = p;
        t_res.pinned_n[slot] = n;
    }
    return t_res.pinned[slot];
}

}  // namespace gllm

using namespace gllm;

extern "C" {

int gllm_hip_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        set_error("no HIP device");
        return 0;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, current_device()) != hipSuccess) {
        (void)hipGetLastError();
        set_error("hipGetDeviceProperties failed");
        return 0;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_error("device is %s, this build targets gfx950", prop.gcnArchName);
        return 0;
    }
    return 1;
}

const char* gllm_hip_last_error(void) { return t_error.c_str(); }

int gllm_hip_set_device(int device) {
    GLLM_HIP(hipSetDevice(device));
    return GLLM_OK;
}

const char* gllm_hip_version(void) { return "gopherllm-mi355x 0.1 (gfx950)"; }

}  // extern "C"
