// runtime.hip -- error reporting, device selection and per-thread resources
// of libgllm_hip (the host side of the C ABI in include/gllm_hip.h).
#include <stdarg.h>
#include <stdio.h>

#include <unordered_map>
#include <vector>

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

// Device scratch of one (host thread, stream) pair.  Work enqueued on one
// stream runs in order, so slots keyed by the stream never serve two
// concurrent kernels; two streams of one thread (a Go scheduler thread
// running two Runners) get separate slots.  in_graph: the slot's buffer was
// handed out while the stream was capturing, so a graph may still use it.
struct StreamScratch {
    void* p[kScratchSlots] = {};
    size_t n[kScratchSlots] = {};
    bool in_graph[kScratchSlots] = {};
};

// Resources of one (host thread, device).  A buffer replaced by a larger one
// is freed once its stream has drained, unless a captured graph may hold it
// (then it goes to `retired` and stays allocated: the graph can be replayed
// at any time).  Growth is geometric, so those total at most a few times the
// largest.
struct DeviceRes {
    hipStream_t stream = nullptr;
    std::unordered_map<hipStream_t, StreamScratch> scratch;
    std::vector<void*> retired;
    void* pinned[kScratchSlots] = {};
    size_t pinned_n[kScratchSlots] = {};
};

// Per device, so switching devices keeps (and later reuses) each device's
// buffers instead of dropping them.
thread_local std::unordered_map<int, DeviceRes> t_devs;
thread_local int t_scratch_code = GLLM_ENOMEM;

int current_device() {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess) return 0;
    return d;
}

// Buffers are kept for the thread's lifetime and never freed at exit: the
// HIP runtime may already be torn down when thread_local destructors run.
DeviceRes& res() { return t_devs[current_device()]; }

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
    DeviceRes& r = res();
    if (!r.stream) {
        if (hipStreamCreateWithFlags(&r.stream, hipStreamNonBlocking) != hipSuccess) {
            r.stream = nullptr;
            set_error("hipStreamCreateWithFlags failed");
        }
    }
    return r.stream;
}

void* thread_scratch(int slot, size_t bytes, hipStream_t stream) {
    if (slot < 0 || slot >= kScratchSlots) return nullptr;
    DeviceRes& r = res();
    StreamScratch& sc = r.scratch[stream];
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess) (void)hipGetLastError();
    const bool capturing = cs != hipStreamCaptureStatusNone;
    if (sc.n[slot] < bytes) {
        // Growing allocates; under stream capture that would either fail or
        // leave the captured graph holding a pointer this thread later
        // replaces.  The caller sizes the slot with one uncaptured call first.
        if (capturing) {
            t_scratch_code = GLLM_EUNSUP;
            set_error("scratch slot %d would grow to %zu bytes inside a stream capture; make the "
                      "same call once outside the capture first", slot, bytes);
            return nullptr;
        }
        size_t n = bytes < 4096 ? 4096 : bytes + bytes / 4;
        void* p = nullptr;
        if (hipMalloc(&p, n) != hipSuccess) {
            (void)hipGetLastError();
            t_scratch_code = GLLM_ENOMEM;
            set_error("hipMalloc(%zu) for scratch failed", n);
            return nullptr;
        }
        if (sc.p[slot]) {
            if (sc.in_graph[slot]) {
                r.retired.push_back(sc.p[slot]);
            } else if (hipStreamSynchronize(stream) == hipSuccess) {
                // work already enqueued on this stream was its only user
                (void)hipFree(sc.p[slot]);
            } else {
                (void)hipGetLastError();
                r.retired.push_back(sc.p[slot]);
            }
        }
        sc.p[slot] = p;
        sc.n[slot] = n;
        sc.in_graph[slot] = false;
    }
    if (capturing) sc.in_graph[slot] = true;
    return sc.p[slot];
}

// The caller is done with `stream` (it will not enqueue on it again): its
// scratch buffers are freed after the stream drains, except those a
// captured graph may still use.
int release_stream_scratch(hipStream_t stream) {
    DeviceRes& r = res();
    auto it = r.scratch.find(stream);
    if (it == r.scratch.end()) return GLLM_OK;
    const bool synced = hipStreamSynchronize(stream) == hipSuccess;
    if (!synced) (void)hipGetLastError();
    for (int i = 0; i < kScratchSlots; i++) {
        if (!it->second.p[i]) continue;
        if (it->second.in_graph[i] || !synced) r.retired.push_back(it->second.p[i]);
        else (void)hipFree(it->second.p[i]);
    }
    r.scratch.erase(it);
    return synced ? GLLM_OK : fail(GLLM_EDEVICE, "stream release: synchronisation failed");
}

int scratch_error() { return t_scratch_code; }

void* thread_pinned(int slot, size_t bytes) {
    if (slot < 0 || slot >= kScratchSlots) return nullptr;
    DeviceRes& r = res();
    if (r.pinned_n[slot] < bytes) {
        if (r.pinned[slot]) (void)hipHostFree(r.pinned[slot]);
        size_t n = bytes < 4096 ? 4096 : bytes + bytes / 4;
        void* p = nullptr;
        if (hipHostMalloc(&p, n, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            r.pinned[slot] = nullptr;
            r.pinned_n[slot] = 0;
            set_error("hipHostMalloc(%zu) failed", n);
            return nullptr;
        }
        r.pinned[slot] = p;
        r.pinned_n[slot] = n;
    }
    return r.pinned[slot];
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
    return self_check() == GLLM_OK ? 1 : 0;
}

const char* gllm_hip_last_error(void) { return t_error.c_str(); }

int gllm_hip_set_device(int device) {
    GLLM_HIP(hipSetDevice(device));
    return GLLM_OK;
}

const char* gllm_hip_version(void) { return "gopherllm-mi355x 0.1 (gfx950)"; }

int gllm_hip_stream_release(void* stream) { return release_stream_scratch((hipStream_t)stream); }

}  // extern "C"
