// rtn.hip -- round-to-nearest weight encoders on the device, and the
// counter-based normal generator used to build synthetic benchmark tensors.
//
// One thread encodes one super-block (256 values) of one row, evaluating the
// reference encoder's float operations in its order:
//   QuantizeRowQ8_0  quantize_rtn.go:35-59
//   QuantizeRowQ4K   quantize_rtn.go:128-216 (+ packScaleMinK4All :106-114)
//   QuantizeRowQ6K   quantize_rtn.go:331-417 (+ quantizeQ6KCode :419-428)
// roundHalfAwayFromZero (quantize_rtn.go:643) is roundf: half away from zero
// on the float32 value, which float64 represents exactly.
#include <math.h>

#include "gllm_common.h"

namespace gllm {

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
__device__ __forceinline__ float abs32(float v) { return v < 0.0f ? -v : v; }
__device__ __forceinline__ int rint_away(float v) { return (int)roundf(v); }
__device__ __forceinline__ void put_f16(uint8_t* b, float v) {
    const uint16_t h = f32_to_f16_bits(v);
    b[0] = (uint8_t)h;
    b[1] = (uint8_t)(h >> 8);
}

__global__ void quantize_q8_0_kernel(const float* __restrict__ src, int rows, int cols,
                                     uint8_t* __restrict__ dst) {
    const int nb = cols / 32;
    const size_t total = (size_t)rows * nb;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / nb, b = i % nb;
        const float* x = src + r * cols + b * 32;
        float amax = 0.0f;
        for (int l = 0; l < 32; l++) {
            const float a = abs32(x[l]);
            if (a > amax) amax = a;
        }
        const float d = amax / 127.0f;
        float id = 0.0f;
        if (d != 0.0f) id = 1.0f / d;
        uint8_t* o = dst + r * (size_t)(nb * 34) + b * 34;
        put_f16(o, d);
        for (int l = 0; l < 32; l++) o[2 + l] = (uint8_t)(int8_t)clampi(rint_away(x[l] * id), -127, 127);
    }
}

__global__ void quantize_q4k_kernel(const float* __restrict__ src, int rows, int cols,
                                    uint8_t* __restrict__ dst) {
    const int ns = cols / 256;
    const size_t total = (size_t)rows * ns;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / ns, s = i % ns;
        const float* sup = src + r * cols + s * 256;
        float raw_scale[8], raw_min1[8];
        for (int b = 0; b < 8; b++) {
            const float* sub = sup + b * 32;
            float lo = sub[0], hi = sub[0];
            for (int l = 0; l < 32; l++) {
                const float v = sub[l];
                if (v < lo) lo = v;
                if (v > hi) hi = v;
            }
            float sc = 0.0f;
            if (hi > lo) sc = (hi - lo) / 15.0f;
            raw_scale[b] = sc;
            raw_min1[b] = -lo;
        }
        float max_scale = raw_scale[0], max_min1 = raw_min1[0];
        for (int b = 1; b < 8; b++) {
            if (raw_scale[b] > max_scale) max_scale = raw_scale[b];
            if (raw_min1[b] > max_min1) max_min1 = raw_min1[b];
        }
        const float d = max_scale / 63.0f;
        const float dmin = max_min1 / 63.0f;
        float inv_d = 0.0f, inv_dmin = 0.0f;
        if (d != 0.0f) inv_d = 1.0f / d;
        if (dmin != 0.0f) inv_dmin = 1.0f / dmin;
        uint8_t sc[8], m[8];
        for (int b = 0; b < 8; b++) {
            sc[b] = (uint8_t)clampi(rint_away(raw_scale[b] * inv_d), 0, 63);
            m[b] = (uint8_t)clampi(rint_away(raw_min1[b] * inv_dmin), 0, 63);
        }
        uint8_t* o = dst + r * (size_t)(ns * 144) + s * 144;
        put_f16(o, d);
        put_f16(o + 2, dmin);
        for (int q = 0; q < 4; q++) {
            o[4 + q] = (uint8_t)((sc[q] & 0x3f) | (((sc[q + 4] >> 4) & 0x03) << 6));
            o[8 + q] = (uint8_t)((m[q] & 0x3f) | (((m[q + 4] >> 4) & 0x03) << 6));
            o[12 + q] = (uint8_t)((sc[q + 4] & 0x0f) | ((m[q + 4] & 0x0f) << 4));
        }
        for (int pair = 0; pair < 4; pair++) {
            const int i0 = 2 * pair, i1 = 2 * pair + 1;
            const float d1 = d * (float)sc[i0];
            const float min1 = dmin * (float)m[i0];
            const float d2 = d * (float)sc[i1];
            const float min2 = dmin * (float)m[i1];
            float inv_d1 = 0.0f, inv_d2 = 0.0f;
            if (d1 != 0.0f) inv_d1 = 1.0f / d1;
            if (d2 != 0.0f) inv_d2 = 1.0f / d2;
            const float* sub0 = sup + i0 * 32;
            const float* sub1 = sup + i1 * 32;
            for (int l = 0; l < 32; l++) {
                const int lo = clampi(rint_away((sub0[l] + min1) * inv_d1), 0, 15);
                const int hi = clampi(rint_away((sub1[l] + min2) * inv_d2), 0, 15);
                o[16 + pair * 32 + l] = (uint8_t)(lo | (hi << 4));
            }
        }
    }
}

__device__ __forceinline__ int q6k_code(float x, float scale) {
    float inv = 0.0f;
    if (scale != 0.0f) inv = 1.0f / scale;
    return clampi(rint_away(x * inv) + 32, 0, 63);
}

__global__ void quantize_q6k_kernel(const float* __restrict__ src, int rows, int cols,
                                    uint8_t* __restrict__ dst) {
    const int ns = cols / 256;
    const size_t total = (size_t)rows * ns;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / ns, s = i % ns;
        const float* sup = src + r * cols + s * 256;
        float extreme[16];
        float gmax = 0.0f;
        for (int b = 0; b < 16; b++) {
            float a = 0.0f, ex = 0.0f;
            for (int l = 0; l < 16; l++) {
                const float v = sup[b * 16 + l];
                const float mag = abs32(v);
                if (mag > a) {
                    a = mag;
                    ex = v;
                }
            }
            extreme[b] = ex;
            if (a > gmax) gmax = a;
        }
        const float d = gmax / (32.0f * 127.0f);
        float inv_d = 0.0f;
        if (d != 0.0f) inv_d = 1.0f / d;
        int sc8[16];
        for (int b = 0; b < 16; b++) {
            const float target = extreme[b] / -32.0f;
            sc8[b] = clampi(rint_away(target * inv_d), -127, 127);
        }
        uint8_t* o = dst + r * (size_t)(ns * 210) + s * 210;
        for (int b = 0; b < 16; b++) o[192 + b] = (uint8_t)(int8_t)sc8[b];
        put_f16(o + 208, d);
        for (int half = 0; half < 2; half++) {
            const int n = half * 128, so = half * 8;
            for (int l = 0; l < 32; l++) {
                const int is = l / 16 + so;
                const float s1 = d * (float)sc8[is], s2 = d * (float)sc8[is + 2];
                const float s3 = d * (float)sc8[is + 4], s4 = d * (float)sc8[is + 6];
                const int c1 = q6k_code(sup[n + l], s1), c2 = q6k_code(sup[n + 32 + l], s2);
                const int c3 = q6k_code(sup[n + 64 + l], s3), c4 = q6k_code(sup[n + 96 + l], s4);
                o[half * 64 + l] = (uint8_t)((c1 & 0x0f) | ((c3 & 0x0f) << 4));
                o[half * 64 + 32 + l] = (uint8_t)((c2 & 0x0f) | ((c4 & 0x0f) << 4));
                o[128 + half * 32 + l] = (uint8_t)(((c1 >> 4) & 3) | (((c2 >> 4) & 3) << 2) |
                                                   (((c3 >> 4) & 3) << 4) | (((c4 >> 4) & 3) << 6));
            }
        }
    }
}

// SplitMix64 finaliser: a bijective 64-bit mix of (seed, counter).
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// out[i] = std * N(0,1): Box-Muller on two 53-bit uniforms drawn from
// mix64(seed * golden + 2i) and mix64(seed * golden + 2i + 1), in double.
__global__ void fill_normal_kernel(float* __restrict__ out, size_t n, uint64_t seed, float std) {
    const uint64_t base = mix64(seed * 0x9e3779b97f4a7c15ull + 0x632be59bd9b4e019ull);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const uint64_t a = mix64(base + 2 * (uint64_t)i);
        const uint64_t b = mix64(base + 2 * (uint64_t)i + 1);
        const double u1 = ((double)(a >> 11) + 0.5) * 0x1.0p-53;  // (0, 1)
        const double u2 = (double)(b >> 11) * 0x1.0p-53;          // [0, 1)
        const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        out[i] = (float)(z * (double)std);
    }
}

}  // namespace gllm

using namespace gllm;

extern "C" int gllm_hip_quantize_rows_dev(int ggml_type, const float* d_src, int rows, int cols,
                                          void* d_dst, void* stream) {
    if (!d_src || !d_dst || rows <= 0 || cols <= 0)
        return fail(GLLM_EINVAL, "gllm_hip_quantize_rows_dev: bad arguments");
    hipStream_t s = (hipStream_t)stream;
    size_t units;
    if (ggml_type == GLLM_TYPE_Q8_0) {
        if (cols % 32) return fail(GLLM_EINVAL, "Q8_0 needs cols %% 32 == 0");
        units = (size_t)rows * (cols / 32);
    } else if (ggml_type == GLLM_TYPE_Q4_K || ggml_type == GLLM_TYPE_Q6_K) {
        if (cols % 256) return fail(GLLM_EINVAL, "K-quants need cols %% 256 == 0");
        units = (size_t)rows * (cols / 256);
    } else {
        return fail(GLLM_EUNSUP, "no encoder for type %d", ggml_type);
    }
    const int block = 128;
    const int grid = (int)((units + block - 1) / block < 65536 ? (units + block - 1) / block : 65536);
    if (ggml_type == GLLM_TYPE_Q8_0)
        hipLaunchKernelGGL(quantize_q8_0_kernel, dim3(grid), dim3(block), 0, s, d_src, rows, cols, (uint8_t*)d_dst);
    else if (ggml_type == GLLM_TYPE_Q4_K)
        hipLaunchKernelGGL(quantize_q4k_kernel, dim3(grid), dim3(block), 0, s, d_src, rows, cols, (uint8_t*)d_dst);
    else
        hipLaunchKernelGGL(quantize_q6k_kernel, dim3(grid), dim3(block), 0, s, d_src, rows, cols, (uint8_t*)d_dst);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

extern "C" int gllm_hip_fill_normal_dev(float* d_out, size_t n, uint64_t seed, float std,
                                        void* stream) {
    if (!d_out) return fail(GLLM_EINVAL, "gllm_hip_fill_normal_dev: null output");
    if (n == 0) return GLLM_OK;
    const int block = 256;
    const size_t want = (n + block - 1) / block;
    const int grid = (int)(want < 65536 ? want : 65536);
    hipLaunchKernelGGL(fill_normal_kernel, dim3(grid), dim3(block), 0, (hipStream_t)stream, d_out,
                       n, seed, std);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}
