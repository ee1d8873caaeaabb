// noalloc.hip -- gllm_hip_matvec_dev_noalloc: gllm_hip_matvec_dev for callers
// that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc).
//
// The only device memory gllm_hip_matvec_dev needs beyond its inputs and
// outputs is the quantised-activation buffer (Q8K int8 rows, scales and the
// per-32 / per-16 sums, act_bytes(cols, p) bytes), which it takes from the
// per-(thread, stream) scratch and grows with hipMalloc.  This entry point
// takes it from `scratch`, a fixed array in the library's device image: every
// GPU the library runs on holds its own copy until the process ends.
//
// Host code must not use the array's name as an address (in host code it is
// a stand-in symbol, not device memory): the device address of each GPU's
// copy comes from hipGetSymbolAddress, once per device, with that device
// current, and only that address is handed to kernels.
//
// Every call on one GPU shares that GPU's array, and the array keeps the last
// call's contents.  Nothing in it has to start at zero: the quantiser writes
// every byte the row kernels and the matrix-core kernel read (their token
// and row indices are clamped to the rows this call wrote).  Calls that
// overlap on one GPU (two streams, or two host threads, at the same time)
// race on the array; callers serialise them.
#include <mutex>

#include "gllm_common.h"

namespace gllm {
int validate_matvec(int n, gllm_hip_weight* const* ws, int p, const int* strides);
int gemv_f32(int n, gllm_hip_weight* const* ws, const float* d_xs, int p, float* const* outs,
             const int* strides, void* act_buf, hipStream_t s);
}  // namespace gllm

// 4 MiB: up to about 280 activation rows at 4096 columns, about 80 at 14336
// (batches of more than 16 rows also carry the f16 operand tiles).
constexpr size_t kNoAllocScratchBytes = 4u << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch_dev[kMaxDevices];  // device address of `scratch` on each GPU

// Device address of this GPU's copy of `scratch`, looked up once per device
// with it current: by the device's load-time check (noalloc_prepare), which
// runs before its first weight exists, so never inside a caller's capture.
// Null with the error set on failure.
void* device_scratch() {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= kMaxDevices) {
        (void)hipGetLastError();
        gllm::set_error("gllm_hip_matvec_dev_noalloc: no current HIP device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch_dev[d]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            gllm::set_error("gllm_hip_matvec_dev_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                            hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_dev[d] = p;
    }
    return g_scratch_dev[d];
}

}  // namespace

namespace gllm {
// Resolves this device's address of `scratch` (and so loads this file's code
// object) ahead of any call: the device's load-time check calls it.
int noalloc_prepare() { return device_scratch() ? GLLM_OK : GLLM_EDEVICE; }
}  // namespace gllm

using namespace gllm;

extern "C" {

int gllm_hip_matvec_dev_noalloc(gllm_hip_weight* w, const float* d_xs, int p, float* d_outs,
                                int out_stride, void* stream) {
    if (!d_xs || !d_outs) return fail(GLLM_EINVAL, "gllm_hip_matvec_dev_noalloc: null pointer");
    gllm_hip_weight* ws[1] = {w};
    float* outs[1] = {d_outs};
    int strides[1] = {out_stride > 0 ? out_stride : (w ? w->rows : 0)};
    GLLM_TRY(validate_matvec(1, ws, p, strides));
    const size_t need = act_bytes(w->cols, p);
    if (need > kNoAllocScratchBytes)
        return fail(GLLM_EINVAL,
                    "gllm_hip_matvec_dev_noalloc: %d rows of %d columns need %zu bytes of "
                    "scratch; the maximum is %zu", p, w->cols, need, kNoAllocScratchBytes);
    void* sc = device_scratch();
    if (!sc) return GLLM_EDEVICE;
    return gemv_f32(1, ws, d_xs, p, outs, strides, sc, (hipStream_t)stream);
}

}  // extern "C"
