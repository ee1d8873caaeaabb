// Read-only HBM stream probe (measurement only; not part of the C ABI of
// include/gllm_hip.h).  One launch reads `bytes` with 16-byte loads and
// nothing else, so the fastest configuration over grid size, workgroup size,
// loads in flight per thread and access pattern is the ceiling that a
// single streaming launch of that many bytes reaches on this part:
// `bench.py --read-ceiling` compares the batch-1 GEMV against it.
//
// pattern 0: grid-stride, consecutive waves read consecutive kilobytes;
// pattern 1: workgroup w reads the contiguous chunk w of bytes / wgs (as a
//            row kernel's workgroup reads its own rows).
// Every load is kept: the loaded words fold into one value per thread,
// stored only if it matches a constant no input produces in practice.
#include <hip/hip_runtime.h>
#include <cstdint>

namespace {

template <int D, int PATTERN>
__global__ void stream_read_kernel(const uint4* __restrict__ p, size_t n16, uint32_t* __restrict__ sink) {
    uint32_t acc = 0;
    size_t i, stride, end;
    if (PATTERN == 0) {
        stride = (size_t)gridDim.x * blockDim.x;
        i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
        end = n16;
    } else {
        const size_t chunk = (n16 + gridDim.x - 1) / gridDim.x;
        const size_t b = (size_t)blockIdx.x * chunk;
        end = b + chunk < n16 ? b + chunk : n16;
        stride = blockDim.x;
        i = b + threadIdx.x;
    }
    for (; i + (size_t)(D - 1) * stride < end; i += (size_t)D * stride) {
        uint4 v[D];
#pragma unroll
        for (int u = 0; u < D; u++) v[u] = p[i + (size_t)u * stride];
#pragma unroll
        for (int u = 0; u < D; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < end; i += stride) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

template <int D>
int launch(int pattern, const uint4* p, size_t n16, int wgs, int threads, uint32_t* sink,
           hipStream_t s) {
    if (pattern == 0)
        hipLaunchKernelGGL((stream_read_kernel<D, 0>), dim3(wgs), dim3(threads), 0, s, p, n16, sink);
    else
        hipLaunchKernelGGL((stream_read_kernel<D, 1>), dim3(wgs), dim3(threads), 0, s, p, n16, sink);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

// 0 on success, -1 on a launch error, -2 on bad arguments.  src: device
// memory of `bytes` (a multiple of 16); sink: device memory of wgs words.
extern "C" int gllm_probe_stream_read(const void* src, size_t bytes, int wgs, int threads,
                                      int depth, int pattern, uint32_t* sink, void* stream) {
    if (!src || !sink || bytes % 16 || wgs < 1 || threads < 64 || threads > 1024 || threads % 64 ||
        (pattern != 0 && pattern != 1))
        return -2;
    const uint4* p = (const uint4*)src;
    const size_t n16 = bytes / 16;
    hipStream_t s = (hipStream_t)stream;
    switch (depth) {
    case 1: return launch<1>(pattern, p, n16, wgs, threads, sink, s);
    case 2: return launch<2>(pattern, p, n16, wgs, threads, sink, s);
    case 4: return launch<4>(pattern, p, n16, wgs, threads, sink, s);
    case 8: return launch<8>(pattern, p, n16, wgs, threads, sink, s);
    case 16: return launch<16>(pattern, p, n16, wgs, threads, sink, s);
    default: return -2;
    }
}
