// rows.hip -- Weight.RowInto on the device (model.go:1034-1100,
// raw_scalar.go:130-161): rows of a weight dequantised to f32, the token
// embedding lookup of every weight type.  Each element is the reference's
// DequantRow*Into expression for it (unfused float32 operations in its
// order), reading the upload-repacked row through repacked_offset.
#include "gllm_common.h"

namespace gllm {

__device__ __forceinline__ uint32_t rw_byte(const uint8_t* row, int type, size_t o, int B) {
    return row[repacked_offset(type, o, B)];
}
__device__ __forceinline__ uint32_t rw_u16(const uint8_t* row, int type, size_t o, int B) {
    return rw_byte(row, type, o, B) | (rw_byte(row, type, o + 1, B) << 8);
}
__device__ __forceinline__ float rw_f16(const uint8_t* row, int type, size_t o, int B) {
    return f16_bits_to_f32(rw_u16(row, type, o, B));
}

// f16ToF32Soft (simd.go:88-109) on the bits: exact for every input, a
// signalling NaN keeping its payload (the hardware conversion would quiet it)
__device__ __forceinline__ float rw_f16_soft(uint32_t h) {
    const uint32_t sign = (h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    if (e == 31) return __uint_as_float(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        const float v = (float)m * 0x1p-24f;  // exact: m < 2^10
        return __uint_as_float(sign | __float_as_uint(v));
    }
    return __uint_as_float(sign | ((e + 112) << 23) | (m << 13));
}

// scaleMinK4 (simd.go:1524-1528): 6-bit scale and min of sub-block j.  The
// bytes j % 4, j % 4 + 4 and j % 4 + 8 of the 12 scale bytes hold both
// cases, so all three are read and the case is a select, not a branch.
__device__ __forceinline__ void rw_scale_min(const uint8_t* row, int type, size_t q, int B, int j,
                                             int* sc, int* m) {
    const int jl = j & 3;
    const uint32_t b0 = rw_byte(row, type, q + jl, B), b4 = rw_byte(row, type, q + jl + 4, B);
    const uint32_t b8 = rw_byte(row, type, q + jl + 8, B);
    *sc = j < 4 ? (int)(b0 & 63) : (int)((b8 & 0x0f) | ((b0 >> 6) << 4));
    *m = j < 4 ? (int)(b4 & 63) : (int)((b8 >> 4) | ((b4 >> 6) << 4));
}

__device__ __forceinline__ float rw_element(const uint8_t* row, int type, int B, int e) {
    switch (type) {
    case GLLM_TYPE_F32: {
        const uint32_t bits = rw_u16(row, type, 4 * (size_t)e, B) |
                              (rw_u16(row, type, 4 * (size_t)e + 2, B) << 16);
        return __uint_as_float(bits);
    }
    case GLLM_TYPE_F16: return rw_f16_soft(rw_u16(row, type, 2 * (size_t)e, B));
    case GLLM_TYPE_BF16: return __uint_as_float(rw_u16(row, type, 2 * (size_t)e, B) << 16);
    case GLLM_TYPE_Q8_0: {  // DequantRowQ8_0Into simd.go:1488-1499
        const size_t base = (size_t)(e / 32) * 34;
        return rw_f16(row, type, base, B) * (float)(int8_t)rw_byte(row, type, base + 2 + e % 32, B);
    }
    case GLLM_TYPE_Q4_0:  // DequantRowQ4_0Into simd.go:1509-1522
    case GLLM_TYPE_Q4_1: {  // DequantRowQ4_1Into quant_extra.go:20-34
        const int bb = type == GLLM_TYPE_Q4_0 ? 18 : 20, hb = bb - 16, i = e % 32;
        const size_t base = (size_t)(e / 32) * bb;
        const uint32_t p = rw_byte(row, type, base + hb + (i & 15), B);
        const int code = (int)(i < 16 ? p & 15 : (p >> 4) & 15);
        const float d = rw_f16(row, type, base, B);
        if (type == GLLM_TYPE_Q4_0) return d * (float)(code - 8);
        return d * (float)code + rw_f16(row, type, base + 2, B);
    }
    case GLLM_TYPE_Q4_K:  // DequantRowQ4KInto simd.go:1530-1557
    case GLLM_TYPE_Q5_K: {  // DequantRowQ5KInto simd.go:1567-1605
        const int bb = type == GLLM_TYPE_Q4_K ? 144 : 176, i = e % 256;
        const size_t base = (size_t)(e / 256) * bb;
        const int chunk = i / 64, l = i % 32, hi = (i / 32) & 1;
        int sc, m;
        rw_scale_min(row, type, base + 4, B, 2 * chunk + hi, &sc, &m);
        const float d1 = rw_f16(row, type, base, B) * (float)sc;
        const float m1 = rw_f16(row, type, base + 2, B) * (float)m;
        const size_t qo = type == GLLM_TYPE_Q4_K ? 16 : 48;
        const uint32_t p = rw_byte(row, type, base + qo + 32 * chunk + l, B);
        int code = (int)(hi ? p >> 4 : p & 15);
        if (type == GLLM_TYPE_Q5_K && ((rw_byte(row, type, base + 16 + l, B) >> (2 * chunk + hi)) & 1))
            code += 16;
        return d1 * (float)code - m1;
    }
    case GLLM_TYPE_Q6_K: {  // DequantRowQ6KInto simd.go:1615-1643
        const int i = e % 256, half = i / 128, g = (i % 128) / 32, l = i % 32;
        const size_t base = (size_t)(e / 256) * 210;
        const uint32_t ql = rw_byte(row, type, base + 64 * half + 32 * (g & 1) + l, B);
        const uint32_t qh = rw_byte(row, type, base + 128 + 32 * half + l, B);
        const int q = (int)(((g < 2 ? ql & 15 : ql >> 4) | (((qh >> (2 * g)) & 3) << 4))) - 32;
        const int sc = (int)(int8_t)rw_byte(row, type, base + 192 + 8 * half + l / 16 + 2 * g, B);
        return rw_f16(row, type, base + 208, B) * (float)sc * (float)q;
    }
    case GLLM_TYPE_Q2_K: {  // DequantRowQ2KInto quant_extra.go:233-263
        const int i = e % 256, is = i / 16, mq = i / 32;
        const size_t base = (size_t)(e / 256) * 84;
        const uint32_t s = rw_byte(row, type, base + is, B);
        const float dl = rw_f16(row, type, base + 80, B) * (float)(s & 15);
        const float ml = rw_f16(row, type, base + 82, B) * (float)(s >> 4);
        const uint32_t q = (rw_byte(row, type, base + 16 + 32 * (mq / 4) + i % 32, B) >> (2 * (mq % 4))) & 3;
        return dl * (float)q - ml;
    }
    case GLLM_TYPE_Q3_K: {  // DequantRowQ3KInto quant_extra.go:336-368
        const int i = e % 256, is = i / 16, mq = i / 32;
        const size_t base = (size_t)(e / 256) * 110;
        const uint32_t lo = (rw_byte(row, type, base + 96 + is % 8, B) >> (4 * (is / 8))) & 15;
        const uint32_t hi = (rw_byte(row, type, base + 104 + is % 4, B) >> (2 * (is / 4))) & 3;
        const float dl = rw_f16(row, type, base + 108, B) * (float)((int)(lo | (hi << 4)) - 32);
        int v = (int)((rw_byte(row, type, base + 32 + 32 * (mq / 4) + i % 32, B) >> (2 * (mq % 4))) & 3);
        if (!((rw_byte(row, type, base + i % 32, B) >> mq) & 1)) v -= 4;
        return dl * (float)v;
    }
    default: {  // MXFP4: DequantRowMXFP4Into simd.go:1653-1670
        const int i = e % 32;
        const size_t base = (size_t)(e / 32) * 17;
        const float scale = ldexpf(1.0f, (int)rw_byte(row, type, base + 16, B) - 127);
        const uint32_t p = rw_byte(row, type, base + i / 2, B);
        const uint32_t code = (i & 1) ? p >> 4 : p & 15;
        const uint32_t c = code & 7;
        const float mag = c < 4 ? 0.5f * (float)c : (float)(2u << ((c - 4) >> 1)) * ((c & 1) ? 1.5f : 1.0f);
        return scale * ((code & 8) ? -mag : mag);
    }
    }
}

// out[t][0..cols) = row ids[t] (clamped to the last row); grid (ceil(cols /
// 256), n), one element per thread.  T >= 0 fixes the type at compile time
// (the element's loads are then straight-line code); T < 0 reads it at run time.
template <int T>
__global__ __launch_bounds__(256) void weight_rows_kernel(const uint8_t* __restrict__ w, size_t rb,
                                                          int type, int B, int rows, int cols,
                                                          const uint32_t* __restrict__ ids,
                                                          float* __restrict__ out) {
    const int t = blockIdx.y, e = blockIdx.x * 256 + threadIdx.x;
    if (e >= cols) return;
    const uint32_t id = min(ids[t], (uint32_t)(rows - 1));
    out[(size_t)t * cols + e] = rw_element(w + (size_t)id * rb, T >= 0 ? T : type, B, e);
}

bool rows_type(int t) {
    return t == GLLM_TYPE_F32 || t == GLLM_TYPE_F16 || t == GLLM_TYPE_BF16 || t == GLLM_TYPE_Q8_0 ||
           t == GLLM_TYPE_Q4_0 || t == GLLM_TYPE_Q4_1 || t == GLLM_TYPE_Q4_K ||
           t == GLLM_TYPE_Q5_K || t == GLLM_TYPE_Q6_K || t == GLLM_TYPE_Q2_K ||
           t == GLLM_TYPE_Q3_K || t == GLLM_TYPE_MXFP4;
}

int launch_weight_rows(const gllm_hip_weight* w, const uint32_t* d_ids, int n, float* d_out,
                       hipStream_t s) {
    if (!rows_type(w->type)) return fail(GLLM_EUNSUP, "weight rows: type %d", w->type);
    if (n <= 0) return n == 0 ? GLLM_OK : fail(GLLM_EINVAL, "weight rows: n = %d", n);
    const dim3 grid((unsigned)((w->cols + 255) / 256), (unsigned)n);
#define GLLM_ROWS(T)                                                                        \
    hipLaunchKernelGGL(weight_rows_kernel<T>, grid, dim3(256), 0, s, w->d_data, w->row_bytes,    \
                       w->type, w->blocks, w->rows, w->cols, d_ids, d_out)
    if (w->type == GLLM_TYPE_Q4_K) GLLM_ROWS(GLLM_TYPE_Q4_K);
    else if (w->type == GLLM_TYPE_Q6_K) GLLM_ROWS(GLLM_TYPE_Q6_K);
    else GLLM_ROWS(-1);
#undef GLLM_ROWS
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

}  // namespace gllm

using namespace gllm;

extern "C" int gllm_hip_weight_rows_dev(const gllm_hip_weight* w, const uint32_t* d_rows, int n,
                                        float* d_out, void* stream) {
    if (!w || !w->d_data || (n > 0 && (!d_rows || !d_out)))
        return fail(GLLM_EINVAL, "gllm_hip_weight_rows_dev: bad arguments");
    return launch_weight_rows(w, d_rows, n, d_out, (hipStream_t)stream);
}
