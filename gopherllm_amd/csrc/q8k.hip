// q8k.hip -- Q8K activation quantiser and the exact-float xsums.
//
// One workgroup per (256-element block, activation row).  Reproduces
//   q8kQuantizePortable  quant_q8k_portable.go:36-62 (== kernels_amd64.s:348-436)
//   sumF32Groups32       kernels_amd64.s:208-230  (Q4_K dmin term)
//   sumF32Groups16       kernels_amd64.s:234-254 (Q2_K min term; Q6_K's offset term
//                        applies ScaleF32(xs, 32) where it reads them)
// bit for bit, and writes q8 in the lane-permuted layout the row kernels read
// (q8perm_offset in gllm_common.h).
#include "gllm_common.h"

namespace gllm {

size_t act_bytes(int cols, int p) {
    size_t n = (size_t)cols * p;                   // q8perm
    n += (size_t)(cols / 256) * p * 4;             // xscale
    n = (n + 255) & ~(size_t)255;
    n += (size_t)(cols / 32) * p * 4;              // xs32
    n += (size_t)(cols / 16) * p * 4;              // xs16
    if (p > kTiledMinP) {
        n = (n + 255) & ~(size_t)255;
        n += (size_t)(p + 15) / 16 * 16 * cols * 2;  // b16t
        n += (size_t)(p + 15) / 16 * 16 * (cols / 32) * 4;  // xs32t
    }
    return n + 256;
}

void act_carve(void* base, int cols, int p, ActQ8* a) {
    uint8_t* c = (uint8_t*)base;
    a->q8perm = (int8_t*)c;
    c += (size_t)cols * p;
    a->xscale = (float*)c;
    c += (size_t)(cols / 256) * p * 4;
    c = (uint8_t*)(((uintptr_t)c + 255) & ~(uintptr_t)255);
    a->xs32 = (float*)c;
    c += (size_t)(cols / 32) * p * 4;
    a->xs16 = (float*)c;
    c += (size_t)(cols / 16) * p * 4;
    a->b16t = nullptr;
    a->xs32t = nullptr;
    a->tiles = 0;
    if (p > kTiledMinP) {
        c = (uint8_t*)(((uintptr_t)c + 255) & ~(uintptr_t)255);
        a->tiles = (p + 15) / 16;
        a->b16t = (uint16_t*)c;
        c += (size_t)a->tiles * 16 * cols * 2;
        a->xs32t = (float*)c;
    }
    a->cols = cols;
    a->p = p;
}

// plain == true writes q8 in element order (the debug entry point) instead of
// the lane-permuted order.  With `up` set, the activation is
// siluMulF32(x, up) (the FFN's SwiGLU), evaluated here instead of in a launch
// of its own.
__global__ __launch_bounds__(256) void q8k_prep_kernel(const float* __restrict__ x, int cols,
                                                       ActQ8 a, int8_t* __restrict__ plain_q8,
                                                       float* __restrict__ plain_scale,
                                                       const float* __restrict__ up) {
    const int b = blockIdx.x, t = blockIdx.y, e = threadIdx.x;
    const int nb = cols / 256;
    if (a.b16t && t >= a.p) {  // padding tokens of the last f16 tile (uniform per workgroup)
        const int kappa = q8perm_offset(e);
        a.b16t[((size_t)b * a.tiles + (t >> 4)) * 4096 + ((kappa >> 3) * 16 + (t & 15)) * 8 +
               (kappa & 7)] = 0;
        if (e < 8) a.xs32t[(((size_t)b * a.tiles + (t >> 4)) * 8 + e) * 16 + (t & 15)] = 0.0f;
        return;
    }
    __shared__ float sx[256];
    __shared__ float wmax[4];
    const size_t idx = (size_t)t * cols + (size_t)b * 256 + e;
    const float v = up ? silu_mul(x[idx], up[idx]) : x[idx];
    sx[e] = v;
    // amax over the block; v_max_f32 is IEEE maxNum, so a NaN element is
    // skipped exactly like the reference's `a > amax` scan.
    const float m = wave_max(fabsf(v));
    if ((e & 63) == 0) wmax[e >> 6] = m;
    __syncthreads();
    const float amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    float scale = 0.0f;
    int q = 0;
    if (amax != 0.0f && amax == amax) {
        scale = amax / 127.0f;
        const float inv = 127.0f / amax;
        q = (int)rintf(v * inv);
    }
    if (plain_q8) {
        plain_q8[(size_t)t * cols + (size_t)b * 256 + e] = (int8_t)q;
        if (e == 0) plain_scale[(size_t)t * nb + b] = scale;
        return;
    }
    const int kappa = q8perm_offset(e);
    a.q8perm[(size_t)t * cols + (size_t)b * 256 + kappa] = (int8_t)q;
    if (a.b16t) {
        // kappa = 32 k + 8 g + i -> ((k 4 + g) 16 + c) 8 + i of the tile block
        a.b16t[((size_t)b * a.tiles + (t >> 4)) * 4096 + ((kappa >> 3) * 16 + (t & 15)) * 8 +
               (kappa & 7)] = __builtin_bit_cast(uint16_t, (_Float16)(float)q);
    }
    if (e == 0) a.xscale[(size_t)t * nb + b] = scale;
    if (e < 8) {
        // sumF32Groups32: v_k = ((x[k] + x[8+k]) + x[16+k]) + x[24+k]
        const float* g = sx + 32 * e;
        float s[8];
#pragma unroll
        for (int k = 0; k < 8; k++) s[k] = ((g[k] + g[8 + k]) + g[16 + k]) + g[24 + k];
        const float a0 = s[0] + s[4], a1 = s[1] + s[5], a2 = s[2] + s[6], a3 = s[3] + s[7];
        const float xs = (a0 + a1) + (a2 + a3);
        a.xs32[(size_t)t * (cols / 32) + b * 8 + e] = xs;
        if (a.xs32t) a.xs32t[(((size_t)b * a.tiles + (t >> 4)) * 8 + e) * 16 + (t & 15)] = xs;
    } else if (e >= 64 && e < 80) {
        // sumF32Groups16: v_k = x[k] + x[8+k], then the same tree, then x32
        const int gi = e - 64;
        const float* g = sx + 16 * gi;
        float s[8];
#pragma unroll
        for (int k = 0; k < 8; k++) s[k] = g[k] + g[8 + k];
        const float a0 = s[0] + s[4], a1 = s[1] + s[5], a2 = s[2] + s[6], a3 = s[3] + s[7];
        a.xs16[(size_t)t * (cols / 16) + b * 16 + gi] = (a0 + a1) + (a2 + a3);
    }
}

int launch_q8k_prep(const float* d_x, int cols, int p, const ActQ8& a, hipStream_t s) {
    if (cols <= 0 || cols % 256 || p <= 0) return fail(GLLM_EINVAL, "q8k: cols %d p %d", cols, p);
    dim3 grid(cols / 256, a.b16t ? 16 * a.tiles : p);
    hipLaunchKernelGGL(q8k_prep_kernel, grid, dim3(256), 0, s, d_x, cols, a, (int8_t*)nullptr,
                       (float*)nullptr, (const float*)nullptr);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

int launch_q8k_prep_silu(const float* d_gate, const float* d_up, int cols, int p, const ActQ8& a,
                         hipStream_t s) {
    if (cols <= 0 || cols % 256 || p <= 0) return fail(GLLM_EINVAL, "q8k: cols %d p %d", cols, p);
    dim3 grid(cols / 256, a.b16t ? 16 * a.tiles : p);
    hipLaunchKernelGGL(q8k_prep_kernel, grid, dim3(256), 0, s, d_gate, cols, a, (int8_t*)nullptr,
                       (float*)nullptr, d_up);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

}  // namespace gllm

using namespace gllm;

extern "C" int gllm_hip_q8k_quantize_dev(const float* d_x, int cols, int p, int8_t* d_q8,
                                         float* d_scales, void* stream) {
    if (!d_x || !d_q8 || !d_scales || cols <= 0 || cols % 256 || p <= 0)
        return fail(GLLM_EINVAL, "gllm_hip_q8k_quantize_dev: bad arguments");
    ActQ8 a{};
    dim3 grid(cols / 256, p);
    hipLaunchKernelGGL(q8k_prep_kernel, grid, dim3(256), 0, (hipStream_t)stream, d_x, cols, a,
                       d_q8, d_scales, (const float*)nullptr);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}
