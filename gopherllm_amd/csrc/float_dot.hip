// float_dot.hip -- float-activation row dots of the reference's same-type
// fused projection groups (matvecSameType2/3Into via sameTypeQuantDot,
// model.go:3213-3283): DotQ8_0F32 (simd.go:646-675), DotQ4_0F32
// (simd.go:677-715), DotQ4_1F32 (quant_extra.go:42-62), DotQ2KF32
// (quant_extra.go:271-302), DotQ3KF32 (quant_extra.go:376-410), DotQ5KF32
// (simd.go:1031-1186) and DotMXFP4F32 (simd.go:1458-1477), on the device
// layouts of the upload repack (read through repacked_offset) and f32
// activations.
//
// Each of these dots adds one term per unit (a 32-element block, a
// 16-element sub-block, for Q5_K a 32-element half of a 64-element step,
// for MXFP4 one element) to a row sum, in unit
// order, and every term depends only on its own unit.  A workgroup computes
// the terms of its rows in parallel into LDS (each term in the reference's
// own operation order, unfused float32 operations as Go evaluates them on
// amd64), then one thread per row adds them up in unit order.
#include <algorithm>

#include "gllm_common.h"

namespace gllm {

constexpr int kFdThreads = 256;
constexpr int kFdLdsTerms = 8192;  // 32 KB of terms per workgroup

__host__ __device__ inline int fd_unit_elems(int type) {
    return type == GLLM_TYPE_MXFP4 ? 1 : (type == GLLM_TYPE_Q2_K || type == GLLM_TYPE_Q3_K) ? 16 : 32;
}

__device__ __forceinline__ uint32_t fd_byte(const uint8_t* row, int type, size_t o, int B) {
    return row[repacked_offset(type, o, B)];
}
__device__ __forceinline__ float fd_f16(const uint8_t* row, int type, size_t o, int B) {
    return f16_bits_to_f32(fd_byte(row, type, o, B) | (fd_byte(row, type, o + 1, B) << 8));
}

// The e2m1 value of a 4-bit code: 0, 0.5, 1, 1.5, 2, 3, 4, 6 and their
// negatives (code 8 is -0), exact in float32.
__device__ __forceinline__ float mxfp4_value(uint32_t code) {
    const uint32_t c = code & 7;
    const float mag = c < 4 ? 0.5f * (float)c : (float)(2u << ((c - 4) >> 1)) * ((c & 1) ? 1.5f : 1.0f);
    return (code & 8) ? -mag : mag;
}

// Q8_0 and Q4_0 terms read their bytes as dwords of the device layout:
// Q8_0 groups of 8 blocks are [8 x f16 d][lane k: the dword of elements
// 4k .. 4k + 3 of blocks q = 0..7 at 16 + 32k + 4q], Q4_0 groups [8 x f16 d]
// [dword kk of blocks g = 0..7 at 16 + 32kk + 4g].  DotQ8_0F32: four lane
// sums over i = 0, 8, 16, 24 of q[i + j] x[i + j] then q[i + 4 + j] x[i + 4 +
// j]; DotQ4_0F32: four lane sums of (lo x[i + j] + hi x[16 + i + j]) over
// i = 0, 4, 8, 12; then scale * ((s0 + s1) + (s2 + s3)), unfused.
struct XSlice {  // the 32 activations of one 32-element unit
    float4 v[8];
};
__device__ __forceinline__ XSlice fd_xslice(const float* __restrict__ x, int u) {
    XSlice r;
    const float4* xb = (const float4*)(x + (size_t)u * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) r.v[i] = xb[i];
    return r;
}

__device__ __forceinline__ float fd_term_q8_0(const uint8_t* row, const XSlice& xsl, int u) {
    const uint8_t* grp = row + (size_t)(u >> 3) * 272;
    const int q = u & 7;
    const float scale = f16_bits_to_f32(*(const uint16_t*)(grp + 2 * q));
    uint32_t dw[8];
#pragma unroll
    for (int k = 0; k < 8; k++) dw[k] = *(const uint32_t*)(grp + 16 + 32 * k + 4 * q);
    const float4* xb = xsl.v;
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int m = 0; m < 4; m++) {
        const float4 xa = xb[2 * m], xc = xb[2 * m + 1];
        const float va[4] = {xa.x, xa.y, xa.z, xa.w}, vc[4] = {xc.x, xc.y, xc.z, xc.w};
#pragma unroll
        for (int jj = 0; jj < 4; jj++) s[jj] = s[jj] + (float)(int8_t)(dw[2 * m] >> (8 * jj)) * va[jj];
#pragma unroll
        for (int jj = 0; jj < 4; jj++) s[jj] = s[jj] + (float)(int8_t)(dw[2 * m + 1] >> (8 * jj)) * vc[jj];
    }
    return scale * ((s[0] + s[1]) + (s[2] + s[3]));
}

__device__ __forceinline__ float fd_term_q4_0(const uint8_t* row, const XSlice& xsl, int u) {
    const uint8_t* grp = row + (size_t)(u >> 3) * 144;
    const int gb = u & 7;
    const float scale = f16_bits_to_f32(*(const uint16_t*)(grp + 2 * gb));
    const float4* xb = xsl.v;
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
        const uint32_t p4 = *(const uint32_t*)(grp + 16 + 32 * kk + 4 * gb);
        const float4 xl = xb[kk], xh = xb[4 + kk];
        const float vl[4] = {xl.x, xl.y, xl.z, xl.w}, vh[4] = {xh.x, xh.y, xh.z, xh.w};
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            const uint32_t p = p4 >> (8 * jj);
            const float lo = (float)((int)(p & 15) - 8), hi = (float)((int)((p >> 4) & 15) - 8);
            s[jj] = s[jj] + (lo * vl[jj] + hi * vh[jj]);
        }
    }
    return scale * ((s[0] + s[1]) + (s[2] + s[3]));
}

// Q5_K unit u = half hf of step st of block b (DotQ5KF32): d1 * qdot -
// min1 * xsum with four lane sums over l = 0, 4, .., 28, k = 0..3.  Device
// block: [16-byte header][lane m: nibble dwords of steps 0..3 at 16 + 16m +
// 4 st][qh bytes at 144 ..].  xsum depends only on x, so the caller passes it.
__device__ __forceinline__ float fd_q5k_xsum(const XSlice& xsl) {
    float xs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const float4 xv = xsl.v[m];
        xs[0] = xs[0] + xv.x;
        xs[1] = xs[1] + xv.y;
        xs[2] = xs[2] + xv.z;
        xs[3] = xs[3] + xv.w;
    }
    return (xs[0] + xs[1]) + (xs[2] + xs[3]);
}

__device__ __forceinline__ float fd_term_q5k(const uint8_t* row, const XSlice& xsl, float xsum, int u) {
    const int b = u >> 3, h = u & 7, st = h >> 1, hf = h & 1, j = h;  // j = 2 st + hf
    const uint8_t* blk = row + (size_t)b * 176;
    const uint4 hd = *(const uint4*)blk;
    const uint32_t hw[4] = {hd.x, hd.y, hd.z, hd.w};
    auto hbyte = [&](int i) { return (hw[i >> 2] >> (8 * (i & 3))) & 0xffu; };
    int sc, mn;
    if (j < 4) {
        sc = (int)(hbyte(4 + j) & 63);
        mn = (int)(hbyte(8 + j) & 63);
    } else {
        const uint32_t a = hbyte(8 + j);
        sc = (int)((a & 0x0f) | ((hbyte(j) >> 6) << 4));
        mn = (int)((a >> 4) | ((hbyte(4 + j) >> 6) << 4));
    }
    const float d1 = f16_bits_to_f32(hd.x & 0xffffu) * (float)sc;
    const float min1 = f16_bits_to_f32(hd.x >> 16) * (float)mn;
    float qd[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const uint32_t nb = *(const uint32_t*)(blk + 16 + 16 * m + 4 * st);
        const uint32_t qh = *(const uint32_t*)(blk + 144 + 4 * m);
        const float4 xv = xsl.v[m];
        const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
        // the four 5-bit codes of elements l .. l + 3, one per byte
        const uint32_t code4 = ((hf ? nb >> 4 : nb) & 0x0f0f0f0fu) | (((qh >> j) & 0x01010101u) << 4);
#pragma unroll
        for (int k = 0; k < 4; k++) qd[k] = qd[k] + (float)((code4 >> (8 * k)) & 0xffu) * xa[k];
    }
    const float qdot = (qd[0] + qd[1]) + (qd[2] + qd[3]);
    return d1 * qdot - min1 * xsum;
}

// The term of unit u of one row (reference offsets o, device row `row`).
__device__ float fd_term(const uint8_t* row, int type, int B, const float* __restrict__ x, int u) {
    if (type == GLLM_TYPE_Q8_0) return fd_term_q8_0(row, fd_xslice(x, u), u);
    if (type == GLLM_TYPE_Q4_0) return fd_term_q4_0(row, fd_xslice(x, u), u);
    if (type == GLLM_TYPE_Q5_K) {
        const XSlice xsl = fd_xslice(x, u);
        return fd_term_q5k(row, xsl, fd_q5k_xsum(xsl), u);
    }
    if (type == GLLM_TYPE_Q4_1) {
        const size_t base = (size_t)u * 20;
        const float d = fd_f16(row, type, base, B), m = fd_f16(row, type, base + 2, B);
        const float* xb = x + (size_t)u * 32;
        float qdot = 0.0f, xsum = 0.0f;
        for (int i = 0; i < 16; i++) {
            const uint32_t p = fd_byte(row, type, base + 4 + i, B);
            qdot = qdot + ((float)(p & 15) * xb[i] + (float)(p >> 4) * xb[16 + i]);
            xsum = xsum + (xb[i] + xb[16 + i]);
        }
        return d * qdot + m * xsum;
    }
    if (type == GLLM_TYPE_Q2_K || type == GLLM_TYPE_Q3_K) {
        const int b = u / 16, is = u % 16;
        const float* xs = x + (size_t)b * 256 + is * 16;
        if (type == GLLM_TYPE_Q2_K) {
            const size_t base = (size_t)b * 84;
            const float d = fd_f16(row, type, base + 80, B), dmin = fd_f16(row, type, base + 82, B);
            const uint32_t sc = fd_byte(row, type, base + is, B);
            const float dl = d * (float)(sc & 15), ml = dmin * (float)(sc >> 4);
            float qdot = 0.0f, xsum = 0.0f;
            for (int l = 0; l < 16; l++) {
                const int e = is * 16 + l, mq = e / 32;
                const uint32_t q = (fd_byte(row, type, base + 16 + 32 * (mq / 4) + e % 32, B) >> (2 * (mq % 4))) & 3;
                qdot = qdot + (float)q * xs[l];
                xsum = xsum + xs[l];
            }
            return dl * qdot - ml * xsum;
        }
        const size_t base = (size_t)b * 110;
        const float d = fd_f16(row, type, base + 108, B);
        // q3KScales: 6-bit scale of sub-block is from the 12 packed bytes
        const uint32_t lo = (fd_byte(row, type, base + 96 + is % 8, B) >> (4 * (is / 8))) & 15;
        const uint32_t hi = (fd_byte(row, type, base + 104 + is % 4, B) >> (2 * (is / 4))) & 3;
        const float dl = d * (float)((int)(lo | (hi << 4)) - 32);
        float acc = 0.0f;
        for (int l = 0; l < 16; l++) {
            const int e = is * 16 + l, mq = e / 32;
            int v = (int)((fd_byte(row, type, base + 32 + 32 * (mq / 4) + e % 32, B) >> (2 * (mq % 4))) & 3);
            if (!((fd_byte(row, type, base + e % 32, B) >> mq) & 1)) v -= 4;
            acc = acc + (float)v * xs[l];
        }
        return dl * acc;
    }
    // MXFP4: unit = one element
    const int b = u / 32, i = u % 32;
    const size_t base = (size_t)b * 17;
    const float scale = ldexpf(1.0f, (int)fd_byte(row, type, base + 16, B) - 127);
    const uint32_t p = fd_byte(row, type, base + i / 2, B);
    const uint32_t code = (i & 1) ? (p >> 4) : (p & 15);
    const float lut = mxfp4_value(code);
    return (lut * scale) * x[(size_t)b * 32 + i];
}

// rows_per_wg rows of one weight per workgroup (grid.y indexes the
// weight); the row's units are taken `chunk` at a time: terms into LDS in
// parallel, then one thread per row adds them to its sum in unit order.
struct FdJob {
    const uint8_t* w[3];
    float* out[3];
    int rows[3];
    int type, cols, B, units, rows_per_wg, chunk;
    size_t rb;
};

__global__ __launch_bounds__(kFdThreads) void float_dot_kernel(FdJob j, const float* __restrict__ x) {
    __shared__ float terms[kFdLdsTerms];
    const int wi = blockIdx.y;
    const int r0 = blockIdx.x * j.rows_per_wg;
    const int nr = min(j.rows_per_wg, j.rows[wi] - r0);
    if (nr <= 0) return;  // uniform
    const uint8_t* w = j.w[wi] + (size_t)r0 * j.rb;
    float sum = 0.0f;
    for (int u0 = 0; u0 < j.units; u0 += j.chunk) {
        const int cu = min(j.chunk, j.units - u0);
        for (int t = threadIdx.x; t < nr * cu; t += kFdThreads) {
            const int rr = t / cu, u = t - rr * cu;
            terms[t] = fd_term(w + (size_t)rr * j.rb, j.type, j.B, x, u0 + u);
        }
        __syncthreads();
        if ((int)threadIdx.x < nr) {
            const float* tr = terms + threadIdx.x * cu;
            for (int u = 0; u < cu; u++) sum = sum + tr[u];
        }
        __syncthreads();
    }
    if ((int)threadIdx.x < nr) j.out[wi][r0 + threadIdx.x] = sum;
}

// Q8_0 / Q4_0 / Q5_K (32-element units): thread (unit u, row subgroup) loads its
// unit's activations once and computes that unit's term for every
// rows-per-workgroup / subgroups-th row; the terms of a row sit kFdPad floats
// apart so the serial per-row sums (thread per row) read distinct banks.
constexpr int kFdPad = 1;

template <int TYPE>
__global__ __launch_bounds__(kFdThreads) void float_dot_u32_kernel(FdJob j, const float* __restrict__ x) {
    __shared__ float terms[kFdLdsTerms];
    const int wi = blockIdx.y, tid = threadIdx.x;
    const int r0 = blockIdx.x * j.rows_per_wg;
    const int nr = min(j.rows_per_wg, j.rows[wi] - r0);
    if (nr <= 0) return;  // uniform
    const uint8_t* w = j.w[wi] + (size_t)r0 * j.rb;
    const int U = j.chunk, ld = U + kFdPad, RG = kFdThreads / U;
    const int u = tid % U, rs = tid / U;
    float sum = 0.0f;
    for (int u0 = 0; u0 < j.units; u0 += U) {
        const int cu = min(U, j.units - u0);
        if (rs < RG && u < cu) {
            const XSlice xsl = fd_xslice(x, u0 + u);
            const float xsum = TYPE == GLLM_TYPE_Q5_K ? fd_q5k_xsum(xsl) : 0.0f;
            for (int rr = rs; rr < nr; rr += RG) {
                const uint8_t* row = w + (size_t)rr * j.rb;
                terms[rr * ld + u] = TYPE == GLLM_TYPE_Q8_0 ? fd_term_q8_0(row, xsl, u0 + u)
                                   : TYPE == GLLM_TYPE_Q4_0 ? fd_term_q4_0(row, xsl, u0 + u)
                                                            : fd_term_q5k(row, xsl, xsum, u0 + u);
            }
        }
        __syncthreads();
        if (tid < nr) {
            const float* tr = terms + tid * ld;
            for (int uu = 0; uu < cu; uu++) sum = sum + tr[uu];
        }
        __syncthreads();
    }
    if (tid < nr) j.out[wi][r0 + tid] = sum;
}

bool float_dot_type(int t) {
    return t == GLLM_TYPE_Q8_0 || t == GLLM_TYPE_Q4_0 || t == GLLM_TYPE_Q4_1 ||
           t == GLLM_TYPE_Q2_K || t == GLLM_TYPE_Q3_K || t == GLLM_TYPE_Q5_K ||
           t == GLLM_TYPE_MXFP4;
}

// n (1..3) weights of one float-dot type and cols against one f32 vector
int launch_float_dot(int n, gllm_hip_weight* const* ws, const float* d_x, float* const* outs,
                     hipStream_t s) {
    if (n < 1 || n > 3) return fail(GLLM_EINVAL, "float row dot: %d weights (1..3)", n);
    FdJob j{};
    j.type = ws[0]->type;
    j.cols = ws[0]->cols;
    j.B = ws[0]->blocks;
    j.rb = ws[0]->row_bytes;
    j.units = j.cols / fd_unit_elems(j.type);
    if (!float_dot_type(j.type)) return fail(GLLM_EUNSUP, "float row dot: type %d", j.type);
    int max_rows = 0, total = 0;
    for (int i = 0; i < n; i++) total += ws[i]->rows;
    // about 1024 workgroups over the group, at most 256 rows each
    j.rows_per_wg = std::max(1, std::min(kFdThreads, (total + 1023) / 1024));
    j.chunk = std::min(j.units, kFdLdsTerms / j.rows_per_wg);
    for (int i = 0; i < n; i++) {
        if (ws[i]->type != j.type || ws[i]->cols != j.cols)
            return fail(GLLM_EINVAL, "float row dot: mixed types or widths");
        j.w[i] = ws[i]->d_data;
        j.out[i] = outs[i];
        j.rows[i] = ws[i]->rows;
        max_rows = std::max(max_rows, ws[i]->rows);
    }
    if (j.type == GLLM_TYPE_Q8_0 || j.type == GLLM_TYPE_Q4_0 || j.type == GLLM_TYPE_Q5_K) {
        // one unit per thread (at most 256 at a time), rows by subgroups
        j.chunk = std::min(j.units, kFdThreads);
        j.rows_per_wg = std::max(1, std::min(kFdLdsTerms / (j.chunk + kFdPad),
                                             (total + 1023) / 1024 * (kFdThreads / j.chunk)));
        const dim3 grid((max_rows + j.rows_per_wg - 1) / j.rows_per_wg, n);
        if (j.type == GLLM_TYPE_Q8_0)
            hipLaunchKernelGGL(float_dot_u32_kernel<GLLM_TYPE_Q8_0>, grid, dim3(kFdThreads), 0, s, j, d_x);
        else if (j.type == GLLM_TYPE_Q4_0)
            hipLaunchKernelGGL(float_dot_u32_kernel<GLLM_TYPE_Q4_0>, grid, dim3(kFdThreads), 0, s, j, d_x);
        else
            hipLaunchKernelGGL(float_dot_u32_kernel<GLLM_TYPE_Q5_K>, grid, dim3(kFdThreads), 0, s, j, d_x);
        GLLM_HIP(hipGetLastError());
        return GLLM_OK;
    }
    const dim3 grid((max_rows + j.rows_per_wg - 1) / j.rows_per_wg, n);
    hipLaunchKernelGGL(float_dot_kernel, grid, dim3(kFdThreads), 0, s, j, d_x);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

}  // namespace gllm
