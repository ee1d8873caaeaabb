// gllm_common.h -- shared device helpers and host plumbing of libgllm_hip.
//
// All HIP sources are compiled with -ffp-contract=off: a fused multiply-add
// appears only where written as fmaf(), matching the VFMADD* sites of the
// reference's amd64 kernels; every other float operation rounds on its own.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <string>

#include "../../include/gllm_hip.h"

namespace gllm {

// ---------------------------------------------------------------------------
// host side: error reporting and per-thread resources
// ---------------------------------------------------------------------------

void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
// Returns GLLM_OK or GLLM_EDEVICE (after recording the message).
int check(hipError_t e, const char* what);

#define GLLM_TRY(expr)                         \
    do {                                       \
        int _rc = (expr);                      \
        if (_rc != GLLM_OK) return _rc;        \
    } while (0)
#define GLLM_HIP(expr) GLLM_TRY(::gllm::check((expr), #expr))

// Per-thread stream used by the blocking host entry points.
hipStream_t thread_stream();
// Compute units of the current device (cached per device).
int device_cus();
// Growable device scratch of the calling thread for work on `stream` (slot
// 0..11).  Null, with the error set, when it cannot grow: allocation failed,
// or the stream is being captured into a graph.
void* thread_scratch(int slot, size_t bytes, hipStream_t stream);
// Status code of the calling thread's last thread_scratch failure
// (GLLM_EUNSUP under capture, GLLM_ENOMEM otherwise).
int scratch_error();
// Load-time known-answer check of the current device (run once per device,
// before its first weight): GLLM_OK, or the failure code with the error set.
int self_check();
// Per-thread pinned host staging buffer.
void* thread_pinned(int slot, size_t bytes);

// Activation buffers produced by the Q8K quantiser for p rows of cols floats.
struct ActQ8 {
    int8_t* q8perm;  // [p][cols] lane-permuted int8 (see q8perm_offset)
    float* xscale;   // [p][cols/256]
    float* xs32;     // [p][cols/32]   per-32 sums (amd64 order)
    float* xs16;     // [p][cols/16]   per-16 sums (amd64 order; Q6_K scales them by 32)
    // Batches of more than kTiledMinP rows also get the q8 values as f16 in
    // the matrix-core operand layout of the batched Q4_K kernel:
    // [block][16-token tile][lane k][group g][token c][8 halves], the eight
    // halves being q8perm's bytes 32 k + 8 g .. + 7 of token 16 tile + c.
    // Tokens p .. 16 tiles - 1 hold zeros.  Null for smaller batches.
    uint16_t* b16t;
    float* xs32t;    // xs32 of the same batches as [block][tile][lane k][token c]
    int tiles;       // ceil(p / 16) when b16t is set
    int cols, p;
};
constexpr int kTiledMinP = 16;
size_t act_bytes(int cols, int p);
void act_carve(void* base, int cols, int p, ActQ8* a);
int launch_q8k_prep(const float* d_x, int cols, int p, const ActQ8& a, hipStream_t s);
// Batched Q4_K x Q8_K on the matrix cores (bit-identical to the row kernel):
// out[t * out_stride + r] for p activation rows.
int launch_q4k_mfma(const uint8_t* d_w, size_t rb, int rows, int blocks, const ActQ8& act, int p,
                    float* out, int out_stride, hipStream_t s);
// Batched Q6_K x Q8_K on the matrix cores, same contract; needs the f16
// tiles (p > kTiledMinP), blocks % 8 == 0 and rows * rb < 4 GiB.
int launch_q6k_tiled(const uint8_t* d_w, size_t rb, int rows, int blocks, const ActQ8& act, int p,
                     float* out, int out_stride, hipStream_t s);
// Batched Q8_0 x Q8_K (vector units, one weight pass per 64 tokens), same
// contract; needs p > kTiledMinP and operands under 4 GiB.
int launch_q8_0_tiled(const uint8_t* d_w, size_t rb, int rows, int blocks, const ActQ8& act, int p,
                      float* out, int out_stride, hipStream_t s);
// Same, for the activation siluMulF32(gate, up) computed on the fly.
int launch_q8k_prep_silu(const float* d_gate, const float* d_up, int cols, int p, const ActQ8& a,
                         hipStream_t s);

struct WeightDesc;  // defined in gemv.hip

}  // namespace gllm

struct gllm_hip_weight {
    int type;
    int rows, cols;
    int blocks;          // cols / 256
    size_t row_bytes;    // reference bytes per row
    uint8_t* d_data;     // device bytes, repacked at upload per type
    int device;
};

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

namespace gllm {

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    // v_cvt_f32_f16: exact widening (subnormals, Inf, NaN preserved) == the
    // reference's f16LUT (simd.go:73-113).
    _Float16 v;
    uint16_t hb = (uint16_t)h;
    __builtin_memcpy(&v, &hb, 2);
    return (float)v;
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    // v_cvt_f16_f32 under the default round-to-nearest-even mode ==
    // F32ToF16 (kv_f16.go:17-49) for every non-NaN input.
    _Float16 v = (_Float16)f;
    uint16_t hb;
    __builtin_memcpy(&hb, &v, 2);
    return hb;
}

// Q4_K device row layout (upload repack; the same 144 bytes per block):
// the row's B block headers (d, dmin, 12 scale bytes; 16 bytes each) first,
// then its B nibble blocks of 128 bytes, in which AVX2 lane k's 16 bytes
// (bytes 4k..4k+3 of each of the four 32-byte chunks) sit at 16k.  Eight
// consecutive blocks' headers are 128 contiguous bytes, so the eight lanes
// of a row fetch them with one 16-byte load each.
__host__ __device__ __forceinline__ size_t q4k_hdr_off(int b) { return (size_t)b * 16; }
__host__ __device__ __forceinline__ size_t q4k_nib_off(int B, int b) {
    return (size_t)B * 16 + (size_t)b * 128;
}

// Offset, in the device row, of byte o of a reference (GGUF) row of B
// blocks: the one-time upload repack of each type (same bytes, block sizes
// unchanged; gllm_hip_weight_download_dev applies it backwards).
__host__ __device__ inline size_t repacked_offset(int type, size_t o, int B) {
    if (type == GLLM_TYPE_Q4_K) {
        // headers to the front of the row (q4k_hdr_off), nibble byte
        // 32s + 4k + j of block b -> q4k_nib_off(B, b) + 16k + 4s + j
        const size_t b = o / 144, e = o % 144;
        if (e < 16) return q4k_hdr_off((int)b) + e;
        const size_t qi = e - 16, s4 = qi / 32, l = qi % 32;
        return q4k_nib_off(B, (int)b) + (l / 4) * 16 + s4 * 4 + (l % 4);
    }
    if (type == GLLM_TYPE_Q6_K) {
        // ql byte 32q + 4k + j -> 16k + 4q + j, qh byte 128 + 32h + 4k + j
        // -> 128 + 8k + 4h + j (lane k's bytes together), scales unchanged,
        // d to the row's tail
        const size_t b = o / 210, e = o % 210;
        if (e < 128) {
            const size_t q = e / 32, l = e % 32;
            return b * 208 + (l / 4) * 16 + q * 4 + (l % 4);
        }
        if (e < 192) {
            const size_t h = (e - 128) / 32, l = (e - 128) % 32;
            return b * 208 + 128 + (l / 4) * 8 + h * 4 + (l % 4);
        }
        if (e < 208) return b * 208 + e;
        return (size_t)B * 208 + b * 2 + (e - 208);
    }
    if (type == GLLM_TYPE_Q8_0) {
        // [d][32 int8] x 8 -> [8 d][lane k: its dword of blocks q = 0..7 at
        // 16 + 32k + 4q]
        const size_t g = o / 272, e = o % 272, q = e / 34, f = e % 34;
        return g * 272 + (f < 2 ? q * 2 + f : 16 + ((f - 2) / 4) * 32 + q * 4 + (f - 2) % 4);
    }
    if (type == GLLM_TYPE_Q5_K) {
        // [header 16][qh 32][nibbles 128] -> [header][lane k: 4 chunk
        // dwords][lane k: qh dword]
        const size_t b = o / 176, e = o % 176;
        if (e < 16) return o;
        if (e < 48) return b * 176 + 144 + (e - 16);
        const size_t qi = e - 48, s4 = qi / 32, l = qi % 32;
        return b * 176 + 16 + (l / 4) * 16 + s4 * 4 + (l % 4);
    }
    if (type == GLLM_TYPE_Q2_K) {
        // [scales 16][qs 64][d][dmin] -> [d][dmin][scales][lane k: qs dwords
        // n = 0, 1]
        const size_t b = o / 84, e = o % 84;
        if (e < 16) return b * 84 + 4 + e;
        if (e < 80) {
            const size_t qi = e - 16, h = qi / 32, l = qi % 32;
            return b * 84 + 20 + (l / 4) * 8 + h * 4 + (l % 4);
        }
        return b * 84 + (e - 80);
    }
    if (type == GLLM_TYPE_Q3_K) {
        // [hmask 32][qs 64][scales 12][d] -> [d][scales][lane k: hmask,
        // qs n = 0, qs n = 1 dwords]
        const size_t b = o / 110, e = o % 110;
        if (e < 32) return b * 110 + 14 + (e / 4) * 12 + (e % 4);
        if (e < 96) {
            const size_t qi = e - 32, h = qi / 32, l = qi % 32;
            return b * 110 + 14 + (l / 4) * 12 + 4 + h * 4 + (l % 4);
        }
        if (e < 108) return b * 110 + 2 + (e - 96);
        return b * 110 + (e - 108);
    }
    if (type == GLLM_TYPE_Q4_0 || type == GLLM_TYPE_Q4_1) {
        // 8 blocks [d (m) | 16 nibble bytes] -> [8 x d (m)][lane group kk:
        // 8 dwords]
        const size_t hb = type == GLLM_TYPE_Q4_0 ? 2 : 4, bb = hb + 16, sb = 8 * bb;
        const size_t S = o / sb, e = o % sb, g = e / bb, f = e % bb;
        return S * sb + (f < hb ? g * hb + f : 8 * hb + ((f - hb) / 4) * 32 + g * 4 + (f - hb) % 4);
    }
    if (type == GLLM_TYPE_MXFP4) {
        // 8 blocks [16 code bytes | e] -> [8 x e][lane k: 8 code ushorts]
        const size_t S = o / 136, e = o % 136, g = e / 17, f = e % 17;
        return S * 136 + (f == 16 ? g : 8 + (f / 2) * 16 + g * 2 + (f % 2));
    }
    return o;  // F32 / F16 / BF16 rows are stored as they are
}

// Byte offset, inside one 256-element block of the lane-permuted Q8K
// activation layout, of element e = 32*m + 4*k + j: lane k of every row
// kernel reads its eight dwords (m = 0..7) as two contiguous 16-byte loads.
__host__ __device__ __forceinline__ int q8perm_offset(int e) {
    int m = e >> 5, k = (e >> 2) & 7, j = e & 3;
    return k * 32 + m * 4 + j;
}

// Exact int8 dot of four byte pairs plus c.  The clamp (saturation at the
// int32 range) never acts on these sums (|dot| <= 4 * 128 * 128 and every
// accumulation stays below 2^24); it selects the VOP3P v_dot4_i32_i8, which
// takes c = 0 as an inline constant where the accumulating v_dot4c form
// needs a v_mov of the zero first.
__device__ __forceinline__ int sdot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, true);
}

// DPP lane moves: a VALU operand modifier, no LDS round trip (a shuffle
// through ds_bpermute waits out an LDS access per step).  CTRL: quad_perm
// 0x00-0xFF, row_shl:n 0x100 + n (lane i of a 16-lane row reads lane i + n;
// lanes past the row end read 0), row_mirror 0x140 (lane i reads 15 - i),
// row_half_mirror 0x141 (lane i reads 7 - i of its 8-lane half).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
constexpr int kQuadXor1 = 0xB1;  // quad_perm [1, 0, 3, 2]
constexpr int kQuadXor2 = 0x4E;  // quad_perm [2, 3, 0, 1]
constexpr int kRowShl4 = 0x104;
constexpr int kRowShl8 = 0x108;
constexpr int kRowMirror = 0x140;
constexpr int kRowHalfMirror = 0x141;

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}

// Maximum of unsigned values over the 64 lanes of a wave (every lane
// active), returned as a wave-uniform value.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t a) {
    a = max(a, dpp_u<0xB1>(a));   // quad_perm [1, 0, 3, 2]
    a = max(a, dpp_u<0x4E>(a));   // quad_perm [2, 3, 0, 1]
    a = max(a, dpp_u<0x141>(a));  // row_half_mirror: 8-lane halves
    a = max(a, dpp_u<0x140>(a));  // row_mirror: 16-lane rows
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)a, 0);
    const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)a, 16);
    const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)a, 32);
    const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)a, 48);
    return max(max(r0, r1), max(r2, r3));
}

__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Maximum over the 64 lanes of a wave (every lane active), in every lane.
// v_max_f32 is IEEE maxNum: a NaN operand is skipped, and the result does
// not depend on the order of the comparisons.
__device__ __forceinline__ float wave_max(float a) {
    a = fmaxf(a, dpp_f<kQuadXor1>(a));
    a = fmaxf(a, dpp_f<kQuadXor2>(a));
    a = fmaxf(a, dpp_f<kRowHalfMirror>(a));  // 8-lane halves
    a = fmaxf(a, dpp_f<kRowMirror>(a));      // 16-lane rows
    return fmaxf(fmaxf(readlane_f(a, 0), readlane_f(a, 16)),
                 fmaxf(readlane_f(a, 32), readlane_f(a, 48)));
}

// 8-lane horizontal tree of the reference's VEXTRACTF128 / VADDPS /
// VHADDPS / VHADDPS sequence: a_k = v_k + v_{k+4}; (a0 + a1) + (a2 + a3).
// Lanes k = 0..7 must be 8 consecutive lanes starting at a multiple of 8;
// lane k == 0 ends with the sum (lanes k = 1..3 hold partial sums, k >= 4
// garbage).  DPP: k reads k + 4 (row_shl:4), then k ^ 1 and k ^ 2 (quad
// permutes); the operands meet in exactly the reference's order.
__device__ __forceinline__ float tree8(float v) {
    v = v + dpp_f<kRowShl4>(v);
    v = v + dpp_f<kQuadXor1>(v);
    v = v + dpp_f<kQuadXor2>(v);
    return v;
}

// siluMulF32AVX2 (kernels_amd64.s:1630-1700) for one element, lane for lane:
// the Cephes exp of -|g| with the reference's constants, then
// (g * (g < 0 ? e : 1) / (1 + e)) * up.
// rmsNormInto's scale over the n floats xs[] (LDS; n % 8 == 0): the
// sum of squares in dotF32AVX2's order (kernels_amd64.s:28-93: 4 x 8 fma
// accumulators over 32-element strides, then the 32 -> 8 -> tree reduction)
// and scale = float32(1 / sqrt(float64(ss / n + eps))) (model.go:2986-3011).
// Threads 0..31 run the accumulator chains; every thread of the block calls
// it and receives the scale.  part[32] and *s_scale are LDS scratch.
__device__ inline float rms_scale_lds(const float* xs, int n, float eps, float* part,
                                      float* s_scale) {
    const int tid = threadIdx.x;
    const int n32 = n & ~31, n8 = n & ~7;
    if (tid < 32) {
        float y = 0.0f;
        int i = 0;
        for (; i + 16 * 32 <= n32; i += 16 * 32) {
            float xb[16];
#pragma unroll
            for (int u = 0; u < 16; u++) xb[u] = xs[i + 32 * u + tid];
#pragma unroll
            for (int u = 0; u < 16; u++) y = fmaf(xb[u], xb[u], y);
        }
        for (; i < n32; i += 32) y = fmaf(xs[i + tid], xs[i + tid], y);
        part[tid] = y;
    }
    __syncthreads();
    if (tid < 8) {
        float acc = (part[tid] + part[8 + tid]) + (part[16 + tid] + part[24 + tid]);
        for (int i = n32; i < n8; i += 8) acc = fmaf(xs[i + tid], xs[i + tid], acc);
        part[tid] = acc;
    }
    __syncthreads();
    if (tid == 0) {
        const float a0 = part[0] + part[4], a1 = part[1] + part[5];
        const float a2 = part[2] + part[6], a3 = part[3] + part[7];
        float ss = (a0 + a1) + (a2 + a3);
        for (int i = n8; i < n; i++) ss = ss + xs[i] * xs[i];
        *s_scale = (float)(1.0 / sqrt((double)(ss / (float)n + eps)));
    }
    __syncthreads();
    return *s_scale;
}

__device__ __forceinline__ float silu_mul(float g, float up) {
    const float lo_clamp = __uint_as_float(0xc2b0c0a5u);  // -88.376
    const float log2e = __uint_as_float(0x3fb8aa3bu);
    const float c1 = __uint_as_float(0x3f318000u);        // 0.693359375
    const float c2 = __uint_as_float(0xb95e8083u);        // -2.12194440e-4
    const float fx_lo = __uint_as_float(0xc2fc0000u);     // -126
    const float a = __uint_as_float(__float_as_uint(g) | 0x80000000u);  // -|g|
    // VMAXPS returns its second source when either operand is NaN
    const float ac = (a != a) ? lo_clamp : (a > lo_clamp ? a : lo_clamp);
    float fx = rintf(ac * log2e);                                       // VROUNDPS $0
    fx = (fx != fx) ? fx_lo : (fx > fx_lo ? fx : fx_lo);
    float r = fmaf(-fx, c1, ac);
    r = fmaf(-fx, c2, r);
    float y = fmaf(__uint_as_float(0x39506967u), r, __uint_as_float(0x3ab743ceu));
    y = fmaf(y, r, __uint_as_float(0x3c088908u));
    y = fmaf(y, r, __uint_as_float(0x3d2aa9c1u));
    y = fmaf(y, r, __uint_as_float(0x3e2aaaaau));
    y = fmaf(y, r, __uint_as_float(0x3f000000u));
    const float r2 = r * r;
    y = fmaf(y, r2, r);
    y = y + 1.0f;
    float e = y * __uint_as_float((uint32_t)((int)fx + 127) << 23);
    if (a < lo_clamp) e = 0.0f;
    const float num = (__float_as_uint(g) & 0x80000000u) ? e : 1.0f;
    const float s = num / (1.0f + e);
    return (g * s) * up;
}

// siluMulF32(gate, up) of 256-element block b of one activation row,
// quantised into a (q8kQuantizePortable, quant_q8k_portable.go:36-62, with
// sumF32Groups32 / sumF32Groups16, kernels_amd64.s:208-254): the work of
// q8k_prep_kernel's workgroup for that block, run by threads 0..255 of the
// calling workgroup (every thread of it calls this; sx: 256 floats and
// wmax: 4 floats of LDS).  SYS: read gate / up with system-scope loads
// (written by other workgroups of the same launch).
template <bool SYS = false>
__device__ inline void silu_q8_block(const float* gate, const float* up, int b, const ActQ8& a,
                                     float* sx, float* wmax) {
    const int e = threadIdx.x;
    const bool on = e < 256;
    const int nb = a.cols / 256;
    float v = 0.0f;
    if (on) {
        const size_t idx = (size_t)b * 256 + e;
        float gv, uv;
        if constexpr (SYS) {
            gv = __hip_atomic_load(gate + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            uv = __hip_atomic_load(up + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        } else {
            gv = gate[idx];
            uv = up[idx];
        }
        v = silu_mul(gv, uv);
        sx[e] = v;
        const float m = wave_max(fabsf(v));
        if ((e & 63) == 0) wmax[e >> 6] = m;
    }
    __syncthreads();
    if (!on) return;  // no barrier follows
    const float amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    float scale = 0.0f;
    int q = 0;
    if (amax != 0.0f && amax == amax) {
        scale = amax / 127.0f;
        const float inv = 127.0f / amax;
        q = (int)rintf(v * inv);
    }
    a.q8perm[(size_t)b * 256 + q8perm_offset(e)] = (int8_t)q;
    if (e == 0) a.xscale[b] = scale;
    if (e < 8) {
        const float* g = sx + 32 * e;
        float s8[8];
#pragma unroll
        for (int k = 0; k < 8; k++) s8[k] = ((g[k] + g[8 + k]) + g[16 + k]) + g[24 + k];
        const float a0 = s8[0] + s8[4], a1 = s8[1] + s8[5], a2 = s8[2] + s8[6], a3 = s8[3] + s8[7];
        a.xs32[(size_t)b * 8 + e] = (a0 + a1) + (a2 + a3);
    } else if (e >= 64 && e < 80) {
        const int gi = e - 64;
        const float* g = sx + 16 * gi;
        float s8[8];
#pragma unroll
        for (int k = 0; k < 8; k++) s8[k] = g[k] + g[8 + k];
        const float a0 = s8[0] + s8[4], a1 = s8[1] + s8[5], a2 = s8[2] + s8[6], a3 = s8[3] + s8[7];
        a.xs16[(size_t)b * 16 + gi] = (a0 + a1) + (a2 + a3);
    }
    (void)nb;
}

// Direct global->LDS copies issued from inline assembly.  The compiler does
// not see them as outstanding vector-memory operations, which is the point:
// they are issued before the weight prefetch and retire first (in order), so
// its vmcnt waits for the weight registers stay exact, and the kernel waits
// for the copies itself (vmcnt <= number of weight loads) before s_barrier.
// M0 holds the wave's LDS destination; lane i writes M0 + 16*i (4*i).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

__device__ __forceinline__ void lds_copy16(const void* gsrc, uint32_t lds_dst) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(gsrc), "s"(lds_dst)
                 : "memory", "m0");
}

__device__ __forceinline__ void lds_copy4(const void* gsrc, uint32_t lds_dst) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off"
                 :
                 : "v"(gsrc), "s"(lds_dst)
                 : "memory", "m0");
}

// s_waitcnt vmcnt(N) for a compile-time N (gfx9 encoding: vmcnt bits [3:0]
// and [15:14], expcnt [6:4] and lgkmcnt [11:8] left unconstrained).
template <int N>
__device__ __forceinline__ void wait_vmem_le() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// s_waitcnt lgkmcnt(0) with vmcnt and expcnt unconstrained.
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Workgroup barrier for LDS data that leaves outstanding global loads in
// flight: the caller has waited for its own LDS traffic; the empty asm
// statements keep the compiler from moving memory operations across it (a
// memory fence would drain the weight prefetch as well).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
}

}  // namespace gllm
