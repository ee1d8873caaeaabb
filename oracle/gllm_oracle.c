/*
 * gllm_oracle.c -- scalar CPU restatement of GopherLLM's quantized matvec,
 * RTN encoders, F16 KV attention and llama decode arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the checker and the CPU baseline); the product in
 * gopherllm_amd/ never links or loads it.  Build with -ffp-contract=off: every
 * fused multiply-add below is an explicit fmaf() placed where the reference's
 * AVX2 code issues VFMADD*, every other float operation rounds on its own,
 * exactly as Go's amd64 compiler (GOAMD64=v1) evaluates the portable code.
 *
 * Parity pins (see tests/test_oracle.py):
 *   f16 conversions    exhaustive round trip + the RNE table of kv_f16_test.go:31-54
 *   q8k quantizer      closed forms, degenerate blocks, the tie list of
 *                      quant_q8k_portable_amd64_test.go:75-81, brute force
 *   row dots           closed-form extremes of q4k_q8_amd64_audit_test.go:18-89
 *                      and q8_0_q8_amd64_test.go:64-98, integer sums vs brute force
 *                      on dequantised codes, generic vs amd64 order at 1e-3,
 *                      int8 path vs float dequant path (cosine >= 0.999)
 *   RTN encoders       known values of quantize_rtn_test.go, decode(encode) error
 *                      bounds, packScaleMinK4All round trip
 *   attention          two-pass == textbook softmax (float64) at 1e-5,
 *                      fastExp vs libm at 2e-6 (attention_fastmath_test.go:11-53)
 *   rope / rmsnorm     textbook float64 forms at 1e-6
 * Parity unpinned: the float32 bits of RoPE tables depend on Go's math.Pow /
 * math.Sincos versus glibc (model.go:1744, 3044); the product computes the
 * same tables with the same host libm, so the GPU and this oracle agree by
 * construction, but agreement with the Go binary itself is unproven.
 */
#include "gllm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------- */
/* f16                                                                        */
/* ------------------------------------------------------------------------- */

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline uint16_t le16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* simd.go:88-109 f16ToF32Soft: exact widening, subnormals normalised. */
float ref_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    uint32_t e = (uint32_t)(h >> 10) & 0x1fu;
    uint32_t mant = (uint32_t)h & 0x3ffu;
    if (e == 0) {
        if (mant == 0) return bits_f32(sign << 31);
        uint32_t shift = 0, m = mant;
        while ((m & 0x400u) == 0) { m <<= 1; shift++; }
        m &= 0x3ffu;
        return bits_f32((sign << 31) | ((127u - 15u + 1u - shift) << 23) | (m << 13));
    }
    if (e == 31) return bits_f32((sign << 31) | (0xffu << 23) | (mant << 13));
    return bits_f32((sign << 31) | ((e + 127u - 15u) << 23) | (mant << 13));
}

/* kv_f16.go:17-49 F32ToF16: round to nearest even, overflow -> Inf,
 * NaN -> sign|0x7e00. */
uint16_t ref_f32_to_f16(float f) {
    uint32_t bits = f32_bits(f);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    int32_t e = (int32_t)((bits >> 23) & 0xffu) - 127 + 15;
    uint32_t mant = bits & 0x7fffffu;
    if (e >= 0x1f) {
        if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
        return (uint16_t)(sign | 0x7c00u);
    }
    if (e <= 0) {
        if (e < -10) return sign;
        mant |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint16_t half = (uint16_t)(mant >> shift);
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t mid = 1u << (shift - 1u);
        if (rem > mid || (rem == mid && (half & 1u))) half++;
        return (uint16_t)(sign | half);
    }
    uint16_t half = (uint16_t)(sign | ((uint32_t)e << 10) | (mant >> 13));
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;
    return half;
}

void ref_f16_to_f32_row(const uint16_t* src, float* dst, long n) {
    for (long i = 0; i < n; i++) dst[i] = ref_f16_to_f32(src[i]);
}

/* kernels_amd64.go:120-127 f32ToF16Row (VCVTPS2PH $0 == F32ToF16). */
void ref_f32_to_f16_row(const float* src, uint16_t* dst, long n) {
    for (long i = 0; i < n; i++) dst[i] = ref_f32_to_f16(src[i]);
}

/* ------------------------------------------------------------------------- */
/* Q8K activation quantiser                                                   */
/* ------------------------------------------------------------------------- */

static inline float abs_f32(float v) { return bits_f32(f32_bits(v) & 0x7fffffffu); }

/* quant_q8k_portable.go:90-94 roundToEvenF32: add/sub 2^23 on the magnitude,
 * reapply the sign bit. */
float ref_round_to_even_f32(float v) {
    const float magic = 8388608.0f;
    float r = (abs_f32(v) + magic) - magic;
    return bits_f32(f32_bits(r) | (f32_bits(v) & 0x80000000u));
}

/* quant_q8k_portable.go:36-62 q8kQuantizePortable (== kernels_amd64.s:348-436
 * for NaN-free input): amax skips NaN, scale = amax/127, inv = 127/amax,
 * q = RNE(x*inv); zero or NaN amax -> scale 0, q 0. */
void ref_q8k_quantize(const float* x, int8_t* q8, float* scales, int blocks) {
    for (int b = 0; b < blocks; b++) {
        const float* xb = x + (long)b * 256;
        float amax = 0.0f;
        for (int i = 0; i < 256; i++) {
            float a = abs_f32(xb[i]);
            if (a > amax) amax = a;
        }
        if (amax == 0.0f || amax != amax) {
            scales[b] = 0.0f;
            memset(q8 + (long)b * 256, 0, 256);
            continue;
        }
        scales[b] = amax / 127.0f;
        float inv = 127.0f / amax;
        for (int i = 0; i < 256; i++)
            q8[(long)b * 256 + i] = (int8_t)(int)ref_round_to_even_f32(xb[i] * inv);
    }
}

/* Horizontal 8-lane tree of VEXTRACTF128/VADDPS/VHADDPS/VHADDPS:
 * a_k = v_k + v_{k+4}; (a0+a1) + (a2+a3). */
static inline float tree8(const float v[8]) {
    float a0 = v[0] + v[4], a1 = v[1] + v[5], a2 = v[2] + v[6], a3 = v[3] + v[7];
    return (a0 + a1) + (a2 + a3);
}

/* kernels_amd64.s:208-230 sumF32Groups32 (amd64) / simd.go:843-860 (generic). */
void ref_xsums32(const float* x, float* out, int groups, int order) {
    for (int g = 0; g < groups; g++) {
        const float* xg = x + (long)g * 32;
        if (order == REF_ORDER_AMD64) {
            float v[8];
            for (int k = 0; k < 8; k++) v[k] = ((xg[k] + xg[8 + k]) + xg[16 + k]) + xg[24 + k];
            out[g] = tree8(v);
        } else {
            float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
            for (int i = 0; i < 32; i += 8) {
                s0 += xg[i] + xg[i + 4];
                s1 += xg[i + 1] + xg[i + 5];
                s2 += xg[i + 2] + xg[i + 6];
                s3 += xg[i + 3] + xg[i + 7];
            }
            out[g] = (s0 + s1) + (s2 + s3);
        }
    }
}

/* kernels_amd64.s:234-254 sumF32Groups16 (amd64) / simd.go:558-575 (generic),
 * then ScaleF32(xs, 32) (simd.go:417). */
void ref_xsums16(const float* x, float* out, int groups, int order, int scale32) {
    for (int g = 0; g < groups; g++) {
        const float* xg = x + (long)g * 16;
        float r;
        if (order == REF_ORDER_AMD64) {
            float v[8];
            for (int k = 0; k < 8; k++) v[k] = xg[k] + xg[8 + k];
            r = tree8(v);
        } else {
            float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
            for (int i = 0; i < 16; i += 4) {
                s0 += xg[i];
                s1 += xg[i + 1];
                s2 += xg[i + 2];
                s3 += xg[i + 3];
            }
            r = (s0 + s1) + (s2 + s3);
        }
        out[g] = scale32 ? r * 32.0f : r;
    }
}

/* ------------------------------------------------------------------------- */
/* Block formats                                                              */
/* ------------------------------------------------------------------------- */

long ref_row_bytes(int type, int cols) {
    switch (type) {
    case REF_Q4_K: return (long)(cols / 256) * 144;
    case REF_Q6_K: return (long)(cols / 256) * 210;
    case REF_Q8_0: return (long)(cols / 32) * 34;
    case REF_Q4_0: return (long)(cols / 32) * 18;
    case REF_Q4_1: return (long)(cols / 32) * 20;
    case REF_MXFP4: return (long)(cols / 32) * 17;
    case REF_Q2_K: return (long)(cols / 256) * 84;
    case REF_Q3_K: return (long)(cols / 256) * 110;
    case REF_Q5_K: return (long)(cols / 256) * 176;
    case REF_F32: return (long)cols * 4;
    case REF_F16: return (long)cols * 2;
    case REF_BF16: return (long)cols * 2;
    default: return -1;
    }
}

/* simd.go:1672-1677 getScaleMinK4 */
static inline void scale_min_k4(int j, const uint8_t* q, int* sc, int* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* Q6_K code of value 128h + 32c + e (simd.go:1615-1643 layout). */
static inline int q6_code(const uint8_t* blk, int h, int c, int e) {
    const uint8_t* ql = blk + 64 * h + ((c & 1) ? 32 : 0);
    const uint8_t* qh = blk + 128 + 32 * h;
    int lo = (c < 2) ? (ql[e] & 0x0f) : (ql[e] >> 4);
    int hi = (qh[e] >> (2 * c)) & 3;
    return lo | (hi << 4);
}

/* ------------------------------------------------------------------------- */
/* Row dots                                                                   */
/* ------------------------------------------------------------------------- */

/* quant_q8k_portable.go:99-128 q4kDotQ8KRowPortable */
static float q4k_dot_generic(const uint8_t* row, const int8_t* q8, const float* xscale,
                             const float* xsums, int blocks) {
    float sum = 0.0f;
    for (int b = 0; b < blocks; b++) {
        const uint8_t* blk = row + (long)b * 144;
        float d = ref_f16_to_f32(le16(blk)), dmin = ref_f16_to_f32(le16(blk + 2));
        const uint8_t* scales = blk + 4;
        const uint8_t* q = blk + 16;
        int32_t block_int = 0;
        for (int s = 0; s < 4; s++) {
            int sc1, sc2, mm;
            scale_min_k4(2 * s, scales, &sc1, &mm);
            scale_min_k4(2 * s + 1, scales, &sc2, &mm);
            int32_t lo = 0, hi = 0;
            for (int l = 0; l < 32; l++) {
                uint8_t qv = q[s * 32 + l];
                lo += (int32_t)(qv & 0x0f) * (int32_t)q8[(long)b * 256 + s * 64 + l];
                hi += (int32_t)(qv >> 4) * (int32_t)q8[(long)b * 256 + s * 64 + 32 + l];
            }
            block_int += sc1 * lo + sc2 * hi;
        }
        sum += (d * xscale[b]) * (float)block_int;
        float min_term = 0.0f;
        for (int j = 0; j < 8; j++) {
            int sc, m;
            scale_min_k4(j, scales, &sc, &m);
            min_term += (float)m * xsums[b * 8 + j];
        }
        sum -= dmin * min_term;
    }
    return sum;
}

/* Integer lanes of kernels_amd64.s:443-455 Q4KQ8CHUNK over one block:
 * lane k collects bytes 4k..4k+3 of every 32-byte nibble chunk s (VPMADDUBSW
 * pairs, VPMADDWD by the sub-block scale). */
static void q4k_lane_ints(const uint8_t* blk, const int8_t* q8b, int32_t acc[8]) {
    const uint8_t* scales = blk + 4;
    const uint8_t* q = blk + 16;
    int sc[8], mm;
    for (int j = 0; j < 8; j++) scale_min_k4(j, scales, &sc[j], &mm);
    for (int k = 0; k < 8; k++) acc[k] = 0;
    for (int s = 0; s < 4; s++) {
        for (int k = 0; k < 8; k++) {
            int32_t lo = 0, hi = 0;
            for (int e = 4 * k; e < 4 * k + 4; e++) {
                uint8_t qv = q[32 * s + e];
                lo += (int32_t)(qv & 0x0f) * (int32_t)q8b[64 * s + e];
                hi += (int32_t)(qv >> 4) * (int32_t)q8b[64 * s + 32 + e];
            }
            acc[k] += sc[2 * s] * lo + sc[2 * s + 1] * hi;
        }
    }
}

/* kernels_amd64.s:465-543 q4kDotQ8KRow */
static float q4k_dot_amd64(const uint8_t* row, const int8_t* q8, const float* xscale,
                           const float* xsums, int blocks) {
    float accF[8] = {0}, accM[8] = {0};
    for (int b = 0; b < blocks; b++) {
        const uint8_t* blk = row + (long)b * 144;
        float d = ref_f16_to_f32(le16(blk)), dmin = ref_f16_to_f32(le16(blk + 2));
        for (int k = 0; k < 8; k++) {
            int sc, m;
            scale_min_k4(k, blk + 4, &sc, &m);
            float mx = (float)m * xsums[b * 8 + k];           /* VMULPS */
            accM[k] = fmaf(dmin, mx, accM[k]);                  /* VFMADD231PS */
        }
        int32_t acc[8];
        q4k_lane_ints(blk, q8 + (long)b * 256, acc);
        float dxs = d * xscale[b];                              /* VMULSS */
        for (int k = 0; k < 8; k++) accF[k] = fmaf((float)acc[k], dxs, accF[k]);
    }
    float t[8];
    for (int k = 0; k < 8; k++) t[k] = accF[k] - accM[k];     /* VSUBPS */
    return tree8(t);
}

/* quant_q8k_portable.go:169-204 q6kDotQ8KRowPortable */
static float q6k_dot_generic(const uint8_t* row, const int8_t* q8, const float* xscale,
                             const float* xsums, int blocks) {
    float sum = 0.0f;
    for (int b = 0; b < blocks; b++) {
        const uint8_t* blk = row + (long)b * 210;
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const int8_t* sc = (const int8_t*)(blk + 192);
        float d = ref_f16_to_f32(le16(blk + 208));
        const int8_t* q8b = q8 + (long)b * 256;
        int32_t block_int = 0;
        for (int half = 0; half < 2; half++) {
            const uint8_t* qlh = ql + half * 64;
            const uint8_t* qhh = qh + half * 32;
            const int8_t* sch = sc + half * 8;
            const int8_t* q8h = q8b + half * 128;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int32_t q1 = (qlh[l] & 0x0f) | ((qhh[l] & 0x03) << 4);
                int32_t q2 = (qlh[l + 32] & 0x0f) | (((qhh[l] >> 2) & 0x03) << 4);
                int32_t q3 = (qlh[l] >> 4) | (((qhh[l] >> 4) & 0x03) << 4);
                int32_t q4 = (qlh[l + 32] >> 4) | (((qhh[l] >> 6) & 0x03) << 4);
                block_int += (int32_t)sch[is] * q1 * (int32_t)q8h[l] +
                             (int32_t)sch[is + 2] * q2 * (int32_t)q8h[32 + l] +
                             (int32_t)sch[is + 4] * q3 * (int32_t)q8h[64 + l] +
                             (int32_t)sch[is + 6] * q4 * (int32_t)q8h[96 + l];
            }
        }
        sum += (d * xscale[b]) * (float)block_int;
        float off_term = 0.0f;
        for (int i = 0; i < 16; i++) off_term += (float)sc[i] * xsums[b * 16 + i];
        sum -= d * off_term;
    }
    return sum;
}

/* Integer lanes of kernels_amd64.s:1130-1142 Q6KQ8QUAD over one block:
 * quad (h, c) covers values 128h+32c+0..31; lanes 0-3 take scale
 * sc[8h+2c], lanes 4-7 sc[8h+2c+1] (VINSERTI128 split). */
static void q6k_lane_ints(const uint8_t* blk, const int8_t* q8b, int32_t acc[8]) {
    const int8_t* sc = (const int8_t*)(blk + 192);
    for (int k = 0; k < 8; k++) acc[k] = 0;
    for (int h = 0; h < 2; h++)
        for (int c = 0; c < 4; c++)
            for (int k = 0; k < 8; k++) {
                int32_t s4 = 0;
                for (int e = 4 * k; e < 4 * k + 4; e++)
                    s4 += q6_code(blk, h, c, e) * (int32_t)q8b[128 * h + 32 * c + e];
                acc[k] += (int32_t)sc[8 * h + 2 * c + (k >= 4)] * s4;
            }
}

/* kernels_amd64.s:1150-1220 q6kDotQ8KRow */
static float q6k_dot_amd64(const uint8_t* row, const int8_t* q8, const float* xscale,
                           const float* xsums, int blocks) {
    float accF[8] = {0}, accM[8] = {0};
    for (int b = 0; b < blocks; b++) {
        const uint8_t* blk = row + (long)b * 210;
        const int8_t* sc = (const int8_t*)(blk + 192);
        float d = ref_f16_to_f32(le16(blk + 208));
        for (int k = 0; k < 8; k++) {
            float t = (float)sc[k] * xsums[b * 16 + k];               /* VMULPS */
            t = fmaf((float)sc[8 + k], xsums[b * 16 + 8 + k], t);   /* VFMADD231PS */
            accM[k] = fmaf(d, t, accM[k]);                           /* VFMADD231PS */
        }
        int32_t acc[8];
        q6k_lane_ints(blk, q8 + (long)b * 256, acc);
        float dxs = d * xscale[b];
        for (int k = 0; k < 8; k++) accF[k] = fmaf((float)acc[k], dxs, accF[k]);
    }
    float t[8];
    for (int k = 0; k < 8; k++) t[k] = accF[k] - accM[k];
    return tree8(t);
}

/* quant_q8k_portable.go:209-228 q8_0DotQ8KRowPortable */
static float q8_0_dot_generic(const uint8_t* row, const int8_t* q8, const float* xscale,
                              int blocks) {
    float sum = 0.0f;
    for (int b = 0; b < blocks; b++) {
        long base = (long)b * 272;
        float block_sum = 0.0f;
        for (int j = 0; j < 8; j++) {
            const uint8_t* blk = row + base + j * 34;
            float d = ref_f16_to_f32(le16(blk));
            const int8_t* w = (const int8_t*)(blk + 2);
            const int8_t* q8b = q8 + (long)b * 256 + j * 32;
            int32_t dot = 0;
            for (int l = 0; l < 32; l++) dot += (int32_t)w[l] * (int32_t)q8b[l];
            block_sum += d * (float)dot;
        }
        sum += xscale[b] * block_sum;
    }
    return sum;
}

/* kernels_amd64.s:1333-1391 q8_0DotQ8KRow: per 32-block j, lane k holds the
 * exact 4-element dot; acc12 = fma(float(p), d_j, acc12); then
 * acc11 = fma(acc12, xs_b, acc11); tree. */
static float q8_0_dot_amd64(const uint8_t* row, const int8_t* q8, const float* xscale,
                            int blocks) {
    float acc11[8] = {0};
    for (int b = 0; b < blocks; b++) {
        float acc12[8] = {0};
        for (int j = 0; j < 8; j++) {
            const uint8_t* blk = row + (long)b * 272 + j * 34;
            float d = ref_f16_to_f32(le16(blk));
            const int8_t* w = (const int8_t*)(blk + 2);
            const int8_t* q8b = q8 + (long)b * 256 + j * 32;
            for (int k = 0; k < 8; k++) {
                int32_t p = 0;
                for (int e = 4 * k; e < 4 * k + 4; e++) p += (int32_t)w[e] * (int32_t)q8b[e];
                acc12[k] = fmaf((float)p, d, acc12[k]);
            }
        }
        for (int k = 0; k < 8; k++) acc11[k] = fmaf(acc12[k], xscale[b], acc11[k]);
    }
    return tree8(acc11);
}

/* ---- Q5_K: Q4_K plus a fifth bit from the 32-byte qh plane ------------- */

/* quant_q8k_portable.go:132-167 q5kDotQ8KRowPortable */
static float q5k_dot_generic(const uint8_t* row, const int8_t* q8, const float* xscale,
                             const float* xsums, int blocks) {
    float sum = 0.0f;
    for (int b = 0; b < blocks; b++) {
        const uint8_t* blk = row + (long)b * 176;
        float d = ref_f16_to_f32(le16(blk)), dmin = ref_f16_to_f32(le16(blk + 2));
        const uint8_t* qh = blk + 16;
        const uint8_t* q = blk + 48;
        int32_t block_int = 0;
        for (int s = 0; s < 4; s++) {
            int sc1, sc2, mm;
            scale_min_k4(2 * s, blk + 4, &sc1, &mm);
            scale_min_k4(2 * s + 1, blk + 4, &sc2, &mm);
            int32_t lo = 0, hi = 0;
            for (int l = 0; l < 32; l++) {
                int qv = q[s * 32 + l];
                int h1 = (qh[l] >> (2 * s)) & 1, h2 = (qh[l] >> (2 * s + 1)) & 1;
                lo += ((qv & 0x0f) + h1 * 16) * (int32_t)q8[b * 256 + s * 64 + l];
                hi += ((qv >> 4) + h2 * 16) * (int32_t)q8[b * 256 + s * 64 + 32 + l];
            }
            block_int += sc1 * lo + sc2 * hi;
        }
        sum += d * xscale[b] * (float)block_int;
        float min_term = 0.0f;
        for (int j = 0; j < 8; j++) {
            int sc, m;
            scale_min_k4(j, blk + 4, &sc, &m);
            min_term += (float)m * xsums[b * 8 + j];
        }
        sum -= dmin * min_term;
    }
    return sum;
}

/* kernels_amd64.s:550-570 Q5KQ8CHUNK lanes: Q4_K's, with bit 2s (low
 * nibbles) / 2s+1 (high nibbles) of qh[e] ORed in as bit 4. */
static void q5k_lane_ints(const uint8_t* blk, const int8_t* q8b, int32_t acc[8]) {
    const uint8_t* qh = blk + 16;
    const uint8_t* q = blk + 48;
    int sc[8], mm;
    for (int j = 0; j < 8; j++) scale_min_k4(j, blk + 4, &sc[j], &mm);
    for (int k = 0; k < 8; k++) acc[k] = 0;
    for (int s = 0; s < 4; s++)
        for (int k = 0; k < 8; k++) {
            int32_t lo = 0, hi = 0;
            for (int e = 4 * k; e < 4 * k + 4; e++) {
                int qv = q[32 * s + e];
                lo += ((qv & 0x0f) | (((qh[e] >> (2 * s)) & 1) << 4)) * (int32_t)q8b[64 * s + e];
                hi += ((qv >> 4) | (((qh[e] >> (2 * s + 1)) & 1) << 4)) * (int32_t)q8b[64 * s + 32 + e];
            }
            acc[k] += sc[2 * s] * lo + sc[2 * s + 1] * hi;
        }
}

/* kernels_amd64.s:578-663 q5kDotQ8KRow (q4kDotQ8KRow's float order) */
static float q5k_dot_amd64(const uint8_t* row, const int8_t* q8, const float* xscale,
                           const float* xsums, int blocks) {
    float accF[8] = {0}, accM[8] = {0};
    for (int b = 0; b < blocks; b++) {
        const uint8_t* blk = row + (long)b * 176;
        float d = ref_f16_to_f32(le16(blk)), dmin = ref_f16_to_f32(le16(blk + 2));
        for (int k = 0; k < 8; k++) {
            int sc, m;
            scale_min_k4(k, blk + 4, &sc, &m);
            float mx = (float)m * xsums[b * 8 + k];           /* VMULPS */
            accM[k] = fmaf(dmin, mx, accM[k]);                  /* VFMADD231PS */
        }
        int32_t acc[8];
        q5k_lane_ints(blk, q8 + (long)b * 256, acc);
        float dxs = d * xscale[b];                              /* VMULSS */
        for (int k = 0; k < 8; k++) accF[k] = fmaf((float)acc[k], dxs, accF[k]);
    }
    float t[8];
    for (int k = 0; k < 8; k++) t[k] = accF[k] - accM[k];     /* VSUBPS */
    return tree8(t);
}

/* ---- Q4_0 / Q4_1: legacy 32-element blocks, 8 per Q8K block ------------ */

/* code of element e (0..31) of a 16-byte nibble block: low nibbles are
 * elements 0..15, high nibbles 16..31 */
static inline int nib32(const uint8_t* nib, int e) { return e < 16 ? nib[e] & 0x0f : nib[e - 16] >> 4; }

/* quant_q8k_portable.go:233-249 q4_0DotQ8KRowPortable */
static float q4_0_dot_generic(const uint8_t* row, const int8_t* q8, const float* xscale,
                              const float* xsums, int blocks) {
    float sum = 0.0f;
    for (int g = 0; g < blocks * 8; g++) {
        const uint8_t* blk = row + (long)g * 18;
        float d = ref_f16_to_f32(le16(blk));
        int32_t intdot = 0;
        for (int i = 0; i < 16; i++) {
            intdot += (blk[2 + i] & 0x0f) * (int32_t)q8[g * 32 + i];
            intdot += (blk[2 + i] >> 4) * (int32_t)q8[g * 32 + 16 + i];
        }
        sum += d * (xscale[g / 8] * (float)intdot - 8.0f * xsums[g]);
    }
    return sum;
}

/* quant_q8k_portable.go:251-271 q4_1DotQ8KRowPortable */
static float q4_1_dot_generic(const uint8_t* row, const int8_t* q8, const float* xscale,
                              const float* xsums, int blocks) {
    float sum = 0.0f;
    for (int g = 0; g < blocks * 8; g++) {
        const uint8_t* blk = row + (long)g * 20;
        float d = ref_f16_to_f32(le16(blk)), m = ref_f16_to_f32(le16(blk + 2));
        int32_t intdot = 0;
        for (int i = 0; i < 16; i++) {
            intdot += (blk[4 + i] & 0x0f) * (int32_t)q8[g * 32 + i];
            intdot += (blk[4 + i] >> 4) * (int32_t)q8[g * 32 + 16 + i];
        }
        sum += d * xscale[g / 8] * (float)intdot + m * xsums[g];
    }
    return sum;
}

/* kernels_amd64.s:679-732 q4_0DotQ8KRow / 734-793 q4_1DotQ8KRow: per
 * 32-block g, lane k holds the unsigned-code dot of elements 4k..4k+3
 * (Q40Q41EXPAND puts low nibbles in lanes 0-3, high in 4-7);
 * accF_k = fma(d*xs, float(I_k), accF_k); a scalar chain carries the offset:
 * Q4_0 fma(-8, d*xsum_g, s), Q4_1 s + m*xsum_g; result tree8(accF) + s. */
static float q4_01_dot_amd64(int type, const uint8_t* row, const int8_t* q8,
                             const float* xscale, const float* xsums, int blocks) {
    const int bb = type == REF_Q4_0 ? 18 : 20, no = type == REF_Q4_0 ? 2 : 4;
    float accF[8] = {0}, accS = 0.0f;
    for (int b = 0; b < blocks; b++) {
        const float xs = xscale[b];
        for (int g = 0; g < 8; g++) {
            const uint8_t* blk = row + (long)(b * 8 + g) * bb;
            const int8_t* q8g = q8 + (long)b * 256 + g * 32;
            float d = ref_f16_to_f32(le16(blk));
            float dxs = d * xs;                                 /* VMULSS X9, X0 */
            for (int k = 0; k < 8; k++) {
                int32_t I = 0;
                for (int e = 4 * k; e < 4 * k + 4; e++) I += nib32(blk + no, e) * (int32_t)q8g[e];
                accF[k] = fmaf(dxs, (float)I, accF[k]);         /* VFMADD231PS */
            }
            if (type == REF_Q4_0) {
                float t = d * xsums[b * 8 + g];                 /* VMULSS (R9), X0 */
                accS = fmaf(-8.0f, t, accS);                    /* VFMADD231SS */
            } else {
                float m = ref_f16_to_f32(le16(blk + 2));
                float t = m * xsums[b * 8 + g];                 /* VMULSS (R9), X6 */
                accS = accS + t;                                /* VADDSS */
            }
        }
    }
    return tree8(accF) + accS;                                  /* VADDSS X10, X11 */
}

/* ---- MXFP4: 17-byte blocks, e2m1 codes, E8M0 scale --------------------- */

/* quant_q8k_portable.go:271-274 mxfp4DoubledLUT: twice the e2m1 value */
static const int mxfp4_dbl[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

static inline int mxfp4_code(const uint8_t* blk, int e) {
    return (e & 1) ? blk[e >> 1] >> 4 : blk[e >> 1] & 0x0f;
}

/* quant_q8k_portable.go:274-303 mxfp4DotQ8KRowPortable */
static float mxfp4_dot_generic(const uint8_t* row, const int8_t* q8, const float* xscale,
                               int blocks) {
    float sum = 0.0f;
    for (int g = 0; g < blocks * 8; g++) {
        const uint8_t* blk = row + (long)g * 17;
        uint32_t e = blk[16];
        float scale = e > 0 ? bits_f32(e << 23) : 0.0f;
        int32_t intdot = 0;
        for (int i = 0; i < 32; i++) intdot += mxfp4_dbl[mxfp4_code(blk, i)] * (int32_t)q8[g * 32 + i];
        sum += scale * 0.5f * xscale[g / 8] * (float)intdot;
    }
    return sum;
}

/* kernels_amd64.s:1065-1128 mxfp4DotQ8KRow: lane k holds elements 4k..4k+3
 * (VPUNPCK restores element order); hx = 0.5*xs per Q8K block, then
 * accF_k = fma(bits(e << 23) * hx, float(I_k), accF_k); tree8. */
static float mxfp4_dot_amd64(const uint8_t* row, const int8_t* q8, const float* xscale,
                             int blocks) {
    float accF[8] = {0};
    for (int b = 0; b < blocks; b++) {
        float hx = 0.5f * xscale[b];                             /* VMULSS (R8), X7 */
        for (int g = 0; g < 8; g++) {
            const uint8_t* blk = row + (long)(b * 8 + g) * 17;
            const int8_t* q8g = q8 + (long)b * 256 + g * 32;
            float sc = bits_f32((uint32_t)blk[16] << 23) * hx; /* VMULSS X10, X0 */
            for (int k = 0; k < 8; k++) {
                int32_t I = 0;
                for (int e = 4 * k; e < 4 * k + 4; e++)
                    I += mxfp4_dbl[mxfp4_code(blk, e)] * (int32_t)q8g[e];
                accF[k] = fmaf(sc, (float)I, accF[k]);          /* VFMADD231PS */
            }
        }
    }
    return tree8(accF);
}

/* ---- Q2_K: 16 sub-blocks of 16, 2-bit codes, 4-bit scale / min -------- */

/* element e (0..255) of a Q2_K / Q3_K block: 32-element group m = e / 32
 * reads qs byte 32 * (m / 4) + e % 32 at shift 2 * (m % 4) */
static inline int q2_code(const uint8_t* qs, int e) {
    const int m = e / 32;
    return (qs[32 * (m / 4) + e % 32] >> (2 * (m % 4))) & 3;
}

/* quant_q8k_portable.go:305-347 q2kDotQ8KRowPortable */
static float q2k_dot_generic(const uint8_t* row, const int8_t* q8, const float* xscale,
                             const float* xsums16, int blocks) {
    float sum = 0.0f;
    for (int b = 0; b < blocks; b++) {
        const uint8_t* blk = row + (long)b * 84;
        float d = ref_f16_to_f32(le16(blk + 80)), dmin = ref_f16_to_f32(le16(blk + 82));
        int32_t block_int = 0;
        float min_term = 0.0f;
        for (int is = 0; is < 16; is++) {
            int32_t qdot = 0;
            for (int l = 0; l < 16; l++)
                qdot += q2_code(blk + 16, is * 16 + l) * (int32_t)q8[b * 256 + is * 16 + l];
            block_int += (blk[is] & 0x0f) * qdot;
            min_term += (float)(blk[is] >> 4) * xsums16[b * 16 + is];
        }
        sum += d * xscale[b] * (float)block_int - dmin * min_term;
    }
    return sum;
}

/* Q2KQ8CHUNK lanes (kernels_amd64.s:795-803): group m, lane k = elements
 * 32m + 4k..+3, weighted by the d-scale nibble of sub-block 2m + k/4. */
static void q2k_lane_ints(const uint8_t* blk, const int8_t* q8b, int32_t acc[8]) {
    for (int k = 0; k < 8; k++) acc[k] = 0;
    for (int m = 0; m < 8; m++)
        for (int k = 0; k < 8; k++) {
            int32_t I = 0;
            for (int e = 32 * m + 4 * k; e < 32 * m + 4 * k + 4; e++)
                I += q2_code(blk + 16, e) * (int32_t)q8b[e];
            acc[k] += (blk[2 * m + k / 4] & 0x0f) * I;
        }
}

/* kernels_amd64.s:816-887 q2kDotQ8KRow: lane k's min term pairs sub-blocks
 * k and 8 + k: t = fma(min_{8+k}, xsum_{8+k}, min_k * xsum_k),
 * accM_k = fma(dmin, t, accM_k); accF as Q4_K; tree8(accF - accM). */
static float q2k_dot_amd64(const uint8_t* row, const int8_t* q8, const float* xscale,
                           const float* xsums16, int blocks) {
    float accF[8] = {0}, accM[8] = {0};
    for (int b = 0; b < blocks; b++) {
        const uint8_t* blk = row + (long)b * 84;
        float d = ref_f16_to_f32(le16(blk + 80)), dmin = ref_f16_to_f32(le16(blk + 82));
        for (int k = 0; k < 8; k++) {
            float t = (float)(blk[k] >> 4) * xsums16[b * 16 + k];               /* VMULPS */
            t = fmaf((float)(blk[8 + k] >> 4), xsums16[b * 16 + 8 + k], t);      /* VFMADD231PS */
            accM[k] = fmaf(dmin, t, accM[k]);                                    /* VFMADD231PS */
        }
        int32_t acc[8];
        q2k_lane_ints(blk, q8 + (long)b * 256, acc);
        float dxs = d * xscale[b];
        for (int k = 0; k < 8; k++) accF[k] = fmaf(dxs, (float)acc[k], accF[k]);
    }
    float t[8];
    for (int k = 0; k < 8; k++) t[k] = accF[k] - accM[k];
    return tree8(t);
}

/* ---- Q3_K: 2-bit codes with a high-bit mask, 6-bit signed scales ------- */

/* quant_extra.go:315-334 q3KScales: 16 six-bit scales from 12 bytes */
static void q3k_scales(const uint8_t* p, int out[16]) {
    uint32_t a0, a1, tmp;
    memcpy(&a0, p, 4);
    memcpy(&a1, p + 4, 4);
    memcpy(&tmp, p + 8, 4);
    uint32_t aux[4];
    aux[2] = ((a0 >> 4) & 0x0f0f0f0fu) | (((tmp >> 4) & 0x03030303u) << 4);
    aux[3] = ((a1 >> 4) & 0x0f0f0f0fu) | (((tmp >> 6) & 0x03030303u) << 4);
    aux[0] = (a0 & 0x0f0f0f0fu) | (((tmp >> 0) & 0x03030303u) << 4);
    aux[1] = (a1 & 0x0f0f0f0fu) | (((tmp >> 2) & 0x03030303u) << 4);
    for (int i = 0; i < 16; i++) out[i] = (int)((aux[i / 4] >> (8 * (i % 4))) & 0xff);
}

/* signed Q3_K value of element e: code - 4 unless hmask bit m = e / 32 of
 * byte e % 32 is set */
static inline int q3_value(const uint8_t* blk, int e) {
    const int h = (blk[e % 32] >> (e / 32)) & 1;
    return q2_code(blk + 32, e) - (h ? 0 : 4);
}

/* quant_q8k_portable.go:349-390 q3kDotQ8KRowPortable */
static float q3k_dot_generic(const uint8_t* row, const int8_t* q8, const float* xscale,
                             int blocks) {
    float sum = 0.0f;
    for (int b = 0; b < blocks; b++) {
        const uint8_t* blk = row + (long)b * 110;
        int sc[16];
        q3k_scales(blk + 96, sc);
        float d = ref_f16_to_f32(le16(blk + 108));
        int32_t block_int = 0;
        for (int is = 0; is < 16; is++) {
            int32_t qdot = 0;
            for (int l = 0; l < 16; l++)
                qdot += q3_value(blk, is * 16 + l) * (int32_t)q8[b * 256 + is * 16 + l];
            block_int += (sc[is] - 32) * qdot;
        }
        sum += d * xscale[b] * (float)block_int;
    }
    return sum;
}

/* Q3KQ8CHUNK lanes (kernels_amd64.s:915-943): w = code + 4h, pair sums
 * w.a - 4.(sum a) (== the signed value times a), weighted by dl = sc - 32 of
 * sub-block 2m + k/4. */
static void q3k_lane_ints(const uint8_t* blk, const int8_t* q8b, int32_t acc[8]) {
    int sc[16];
    q3k_scales(blk + 96, sc);
    for (int k = 0; k < 8; k++) acc[k] = 0;
    for (int m = 0; m < 8; m++)
        for (int k = 0; k < 8; k++) {
            int32_t I = 0;
            for (int e = 32 * m + 4 * k; e < 32 * m + 4 * k + 4; e++)
                I += q3_value(blk, e) * (int32_t)q8b[e];
            acc[k] += (sc[2 * m + k / 4] - 32) * I;
        }
}

/* kernels_amd64.s:945-1063 q3kDotQ8KRow: accF_k = fma(d*xs, float(I_k),
 * accF_k); tree8 (no min term). */
static float q3k_dot_amd64(const uint8_t* row, const int8_t* q8, const float* xscale,
                           int blocks) {
    float accF[8] = {0};
    for (int b = 0; b < blocks; b++) {
        const uint8_t* blk = row + (long)b * 110;
        int32_t acc[8];
        q3k_lane_ints(blk, q8 + (long)b * 256, acc);
        float dxs = ref_f16_to_f32(le16(blk + 108)) * xscale[b];
        for (int k = 0; k < 8; k++) accF[k] = fmaf(dxs, (float)acc[k], accF[k]);
    }
    return tree8(accF);
}

float ref_q4k_dot(const uint8_t* row, const int8_t* q8, const float* xscale,
                  const float* xsums32, int blocks, int order) {
    return order == REF_ORDER_AMD64 ? q4k_dot_amd64(row, q8, xscale, xsums32, blocks)
                                    : q4k_dot_generic(row, q8, xscale, xsums32, blocks);
}
float ref_q6k_dot(const uint8_t* row, const int8_t* q8, const float* xscale,
                  const float* xsums16x32, int blocks, int order) {
    return order == REF_ORDER_AMD64 ? q6k_dot_amd64(row, q8, xscale, xsums16x32, blocks)
                                    : q6k_dot_generic(row, q8, xscale, xsums16x32, blocks);
}
float ref_q8_0_dot(const uint8_t* row, const int8_t* q8, const float* xscale, int blocks,
                   int order) {
    return order == REF_ORDER_AMD64 ? q8_0_dot_amd64(row, q8, xscale, blocks)
                                    : q8_0_dot_generic(row, q8, xscale, blocks);
}

void ref_lane_ints(int type, const uint8_t* row, const int8_t* q8, int blocks, int32_t* out) {
    for (int b = 0; b < blocks; b++) {
        int32_t acc[8];
        if (type == REF_Q4_K) {
            q4k_lane_ints(row + (long)b * 144, q8 + (long)b * 256, acc);
        } else if (type == REF_Q5_K) {
            q5k_lane_ints(row + (long)b * 176, q8 + (long)b * 256, acc);
        } else if (type == REF_Q2_K) {
            q2k_lane_ints(row + (long)b * 84, q8 + (long)b * 256, acc);
        } else if (type == REF_Q3_K) {
            q3k_lane_ints(row + (long)b * 110, q8 + (long)b * 256, acc);
        } else if (type == REF_Q4_0 || type == REF_Q4_1 || type == REF_MXFP4) {
            /* per 32-block pieces, summed over the 8 blocks per lane (exact) */
            const int bb = type == REF_Q4_0 ? 18 : type == REF_Q4_1 ? 20 : 17;
            for (int k = 0; k < 8; k++) acc[k] = 0;
            for (int g = 0; g < 8; g++) {
                const uint8_t* blk = row + (long)(b * 8 + g) * bb;
                const int8_t* q8g = q8 + (long)b * 256 + g * 32;
                for (int k = 0; k < 8; k++)
                    for (int e = 4 * k; e < 4 * k + 4; e++) {
                        const int c = type == REF_MXFP4 ? mxfp4_dbl[mxfp4_code(blk, e)]
                                                        : nib32(blk + (type == REF_Q4_0 ? 2 : 4), e);
                        acc[k] += c * (int32_t)q8g[e];
                    }
            }
        } else if (type == REF_Q6_K) {
            q6k_lane_ints(row + (long)b * 210, q8 + (long)b * 256, acc);
        } else {
            /* Q8_0: the integer pieces are per 32-block; report their sum over
             * the 8 sub-blocks per lane (exact). */
            for (int k = 0; k < 8; k++) acc[k] = 0;
            for (int j = 0; j < 8; j++) {
                const int8_t* w = (const int8_t*)(row + (long)b * 272 + j * 34 + 2);
                const int8_t* q8b = q8 + (long)b * 256 + j * 32;
                for (int k = 0; k < 8; k++)
                    for (int e = 4 * k; e < 4 * k + 4; e++) acc[k] += (int32_t)w[e] * q8b[e];
            }
        }
        memcpy(out + (long)b * 8, acc, sizeof acc);
    }
}

/* ------------------------------------------------------------------------- */
/* Matvec orchestration                                                       */
/* ------------------------------------------------------------------------- */

int ref_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

typedef struct {
    int8_t* q8;
    float* xscale;
    float* xsums; /* 32-group sums (Q4_K) or 16-group sums x32 (Q6_K) */
} act_q8;

/* acquireQ8 + fillQ4KXSums / fillQ6KXSums16+ScaleF32 (kernels_amd64.go:246,
 * simd.go:261-288, 413-441). */
static void prepare_act(int type, const float* x, int cols, int order, act_q8* a) {
    int blocks = cols / 256;
    ref_q8k_quantize(x, a->q8, a->xscale, blocks);
    if (type == REF_Q4_K || type == REF_Q5_K || type == REF_Q4_0 || type == REF_Q4_1)
        ref_xsums32(x, a->xsums, cols / 32, order);  /* fillQ4KXSums */
    else if (type == REF_Q6_K) ref_xsums16(x, a->xsums, cols / 16, order, 1);
    else if (type == REF_Q2_K) ref_xsums16(x, a->xsums, cols / 16, order, 0); /* unscaled */
}

float ref_row_dot_any(int type, const uint8_t* row, const int8_t* q8, const float* xscale,
                      const float* xsums, int blocks, int order) {
    const int amd = order == REF_ORDER_AMD64;
    switch (type) {
    case REF_Q4_K: return ref_q4k_dot(row, q8, xscale, xsums, blocks, order);
    case REF_Q6_K: return ref_q6k_dot(row, q8, xscale, xsums, blocks, order);
    case REF_Q8_0: return ref_q8_0_dot(row, q8, xscale, blocks, order);
    case REF_Q5_K: return amd ? q5k_dot_amd64(row, q8, xscale, xsums, blocks)
                              : q5k_dot_generic(row, q8, xscale, xsums, blocks);
    case REF_Q4_0: return amd ? q4_01_dot_amd64(REF_Q4_0, row, q8, xscale, xsums, blocks)
                              : q4_0_dot_generic(row, q8, xscale, xsums, blocks);
    case REF_Q4_1: return amd ? q4_01_dot_amd64(REF_Q4_1, row, q8, xscale, xsums, blocks)
                              : q4_1_dot_generic(row, q8, xscale, xsums, blocks);
    case REF_MXFP4: return amd ? mxfp4_dot_amd64(row, q8, xscale, blocks)
                               : mxfp4_dot_generic(row, q8, xscale, blocks);
    case REF_Q2_K: return amd ? q2k_dot_amd64(row, q8, xscale, xsums, blocks)
                              : q2k_dot_generic(row, q8, xscale, xsums, blocks);
    case REF_Q3_K: return amd ? q3k_dot_amd64(row, q8, xscale, blocks)
                              : q3k_dot_generic(row, q8, xscale, blocks);
    default: return 0.0f;
    }
}

static float row_dot(int type, const uint8_t* row, const act_q8* a, int blocks, int order) {
    return ref_row_dot_any(type, row, a->q8, a->xscale, a->xsums, blocks, order);
}

int ref_type_supported(int type) {
    return type == REF_Q4_K || type == REF_Q6_K || type == REF_Q8_0 || type == REF_Q5_K ||
           type == REF_Q4_0 || type == REF_Q4_1 || type == REF_MXFP4 || type == REF_Q2_K ||
           type == REF_Q3_K;
}

static int act_alloc(act_q8* a, int cols) {
    a->q8 = (int8_t*)malloc((size_t)cols);
    a->xscale = (float*)malloc(sizeof(float) * (size_t)(cols / 256 + 1));
    a->xsums = (float*)malloc(sizeof(float) * (size_t)(cols / 16 + 1));
    return a->q8 && a->xscale && a->xsums;
}
static void act_free(act_q8* a) { free(a->q8); free(a->xscale); free(a->xsums); }

int ref_matvec_batch(int type, const uint8_t* data, const float* xs, int p, int rows,
                     int cols, float* outs, int order, int threads) {
    if (cols <= 0 || cols % 256 || rows < 0 || p <= 0) return -1;
    if (!ref_type_supported(type)) return -1;
    int blocks = cols / 256;
    long rb = ref_row_bytes(type, cols);
    act_q8* acts = (act_q8*)calloc((size_t)p, sizeof(act_q8));
    for (int t = 0; t < p; t++) {
        act_alloc(&acts[t], cols);
        prepare_act(type, xs + (long)t * cols, cols, order, &acts[t]);
    }
    if (threads <= 0) threads = ref_num_threads();
    (void)threads;
#pragma omp parallel for schedule(static) num_threads(threads) if (rows >= 64)
    for (int r = 0; r < rows; r++)
        for (int t = 0; t < p; t++)
            outs[(long)t * rows + r] = row_dot(type, data + (long)r * rb, &acts[t], blocks, order);
    for (int t = 0; t < p; t++) act_free(&acts[t]);
    free(acts);
    return 0;
}

int ref_matvec(int type, const uint8_t* data, const float* x, int rows, int cols, float* out,
               int order, int threads) {
    return ref_matvec_batch(type, data, x, 1, rows, cols, out, order, threads);
}

/* sampling.go:385 finiteLogit */
static inline int finite_logit(float v) { return (f32_bits(v) & 0x7f800000u) != 0x7f800000u; }

/* sampling.go:399-418 argmaxFiniteToken (without mutating the input) */
uint32_t ref_argmax_finite(const float* logits, long n) {
    long best = 0;
    float best_v = -INFINITY;
    if (n <= 0) return 0;
    if (finite_logit(logits[0])) best_v = logits[0];
    for (long i = 1; i < n; i++) {
        float v = finite_logit(logits[i]) ? logits[i] : -INFINITY;
        if (v > best_v) { best = i; best_v = v; }
    }
    return (uint32_t)best;
}

/* sampling.go:136-153 applyRepeatPenalty, in place: walk the window in order;
 * an id inside the vocabulary turns a non-finite logit into -inf, divides a
 * positive one by the penalty and multiplies any other by it (a repeated id
 * applies the rule again).  penalty 1 leaves the logits untouched. */
void ref_apply_repeat_penalty(float* logits, long n, const uint32_t* recent, int n_recent,
                              float penalty) {
    if (penalty == 1.0f) return;
    for (int i = 0; i < n_recent; i++) {
        uint32_t tok = recent[i];
        if ((long)tok >= n) continue;
        float v = logits[tok];
        if (!finite_logit(v)) logits[tok] = -INFINITY;
        else if (v > 0) logits[tok] = v / penalty;
        else logits[tok] = v * penalty;
    }
}

/* kernels_amd64.go:294-331 argmaxQ6KRowsQ8 (and the Q4_K / Q8_0 twins):
 * skip non-finite, strict >, lowest row on ties, 0 if nothing finite. */
uint32_t ref_argmax_matvec(int type, const uint8_t* data, const float* x, int rows, int cols,
                           int order, int threads) {
    float* logits = (float*)malloc(sizeof(float) * (size_t)rows);
    ref_matvec(type, data, x, rows, cols, logits, order, threads);
    uint32_t tok = 0;
    float best = 0.0f;
    int found = 0;
    for (int r = 0; r < rows; r++) {
        float v = logits[r];
        if (finite_logit(v) && (!found || v > best)) { tok = (uint32_t)r; best = v; found = 1; }
    }
    free(logits);
    return tok;
}

/* ------------------------------------------------------------------------- */
/* RTN encoders (quantize_rtn.go) and decoders (simd.go)                      */
/* ------------------------------------------------------------------------- */

static inline int clamp_int(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
/* quantize_rtn.go:643-645 roundHalfAwayFromZero: float32(math.Round(float64)) */
static inline float round_half_away(float v) { return (float)round((double)v); }
/* quantize_rtn.go:632-637 abs32 */
static inline float abs32(float v) { return v < 0 ? -v : v; }
static inline void put_f16(uint8_t* b, float v) {
    uint16_t h = ref_f32_to_f16(v);
    b[0] = (uint8_t)h;
    b[1] = (uint8_t)(h >> 8);
}
/* Go int(float32) truncates toward zero; the encoders only feed it finite,
 * small values. */
static inline int go_int(float v) { return (int)v; }

/* quantize_rtn.go:35-59 QuantizeRowQ8_0 */
static void quantize_row_q8_0(const float* row, int cols, uint8_t* out) {
    int nb = cols / 32;
    for (int b = 0; b < nb; b++) {
        const float* x = row + (long)b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) {
            float a = abs32(x[i]);
            if (a > amax) amax = a;
        }
        float d = amax / 127.0f;
        float id = 0.0f;
        if (d != 0.0f) id = 1.0f / d;
        uint8_t* o = out + (long)b * 34;
        put_f16(o, d);
        for (int i = 0; i < 32; i++) {
            int q = clamp_int(go_int(round_half_away(x[i] * id)), -127, 127);
            o[2 + i] = (uint8_t)(int8_t)q;
        }
    }
}

/* quantize_rtn.go:106-114 packScaleMinK4All */
static void pack_scale_min_k4(const uint8_t sc[8], const uint8_t m[8], uint8_t q[12]) {
    for (int i = 0; i < 4; i++) {
        q[i] = (uint8_t)((sc[i] & 0x3f) | (((sc[i + 4] >> 4) & 0x03) << 6));
        q[i + 4] = (uint8_t)((m[i] & 0x3f) | (((m[i + 4] >> 4) & 0x03) << 6));
        q[i + 8] = (uint8_t)((sc[i + 4] & 0x0f) | ((m[i + 4] & 0x0f) << 4));
    }
}

/* quantize_rtn.go:128-216 QuantizeRowQ4K */
static void quantize_row_q4k(const float* row, int cols, uint8_t* out) {
    int ns = cols / 256;
    for (int s = 0; s < ns; s++) {
        const float* sup = row + (long)s * 256;
        float raw_scale[8], raw_min1[8];
        for (int i = 0; i < 8; i++) {
            const float* sub = sup + i * 32;
            float lo = sub[0], hi = sub[0];
            for (int l = 0; l < 32; l++) {
                if (sub[l] < lo) lo = sub[l];
                if (sub[l] > hi) hi = sub[l];
            }
            float sc = 0.0f;
            if (hi > lo) sc = (hi - lo) / 15.0f;
            raw_scale[i] = sc;
            raw_min1[i] = -lo;
        }
        float max_scale = raw_scale[0], max_min1 = raw_min1[0];
        for (int i = 1; i < 8; i++) {
            if (raw_scale[i] > max_scale) max_scale = raw_scale[i];
            if (raw_min1[i] > max_min1) max_min1 = raw_min1[i];
        }
        float d = max_scale / 63.0f;
        float dmin = max_min1 / 63.0f;
        float inv_d = 0.0f, inv_dmin = 0.0f;
        if (d != 0.0f) inv_d = 1.0f / d;
        if (dmin != 0.0f) inv_dmin = 1.0f / dmin;
        uint8_t sc[8], m[8], packed[12];
        for (int i = 0; i < 8; i++) {
            sc[i] = (uint8_t)clamp_int(go_int(round_half_away(raw_scale[i] * inv_d)), 0, 63);
            m[i] = (uint8_t)clamp_int(go_int(round_half_away(raw_min1[i] * inv_dmin)), 0, 63);
        }
        pack_scale_min_k4(sc, m, packed);
        uint8_t* o = out + (long)s * 144;
        put_f16(o, d);
        put_f16(o + 2, dmin);
        memcpy(o + 4, packed, 12);
        uint8_t* q = o + 16;
        for (int pair = 0; pair < 4; pair++) {
            int i0 = pair * 2, i1 = pair * 2 + 1;
            float d1 = d * (float)sc[i0];
            float min1 = dmin * (float)m[i0];
            float d2 = d * (float)sc[i1];
            float min2 = dmin * (float)m[i1];
            float inv_d1 = 0.0f, inv_d2 = 0.0f;
            if (d1 != 0.0f) inv_d1 = 1.0f / d1;
            if (d2 != 0.0f) inv_d2 = 1.0f / d2;
            const float* sub0 = sup + i0 * 32;
            const float* sub1 = sup + i1 * 32;
            for (int l = 0; l < 32; l++) {
                int lo = clamp_int(go_int(round_half_away((sub0[l] + min1) * inv_d1)), 0, 15);
                int hi = clamp_int(go_int(round_half_away((sub1[l] + min2) * inv_d2)), 0, 15);
                q[pair * 32 + l] = (uint8_t)(lo | (hi << 4));
            }
        }
    }
}

/* quantize_rtn.go:419-428 quantizeQ6KCode */
static inline uint8_t q6k_code(float x, float scale) {
    float inv = 0.0f;
    if (scale != 0.0f) inv = 1.0f / scale;
    return (uint8_t)clamp_int(go_int(round_half_away(x * inv)) + 32, 0, 63);
}

/* quantize_rtn.go:325-417 QuantizeRowQ6K */
static void quantize_row_q6k(const float* row, int cols, uint8_t* out) {
    int ns = cols / 256;
    for (int s = 0; s < ns; s++) {
        const float* sup = row + (long)s * 256;
        float extreme[16] = {0};
        float gmax = 0.0f;
        for (int i = 0; i < 16; i++) {
            const float* sub = sup + i * 16;
            float a = 0.0f;
            for (int l = 0; l < 16; l++) {
                float m = abs32(sub[l]);
                if (m > a) { a = m; extreme[i] = sub[l]; }
            }
            if (a > gmax) gmax = a;
        }
        float d = gmax / (32.0f * 127.0f);
        float inv_d = 0.0f;
        if (d != 0.0f) inv_d = 1.0f / d;
        int8_t sc8[16];
        for (int i = 0; i < 16; i++) {
            float target = extreme[i] / -32.0f;
            sc8[i] = (int8_t)clamp_int(go_int(round_half_away(target * inv_d)), -127, 127);
        }
        uint8_t* o = out + (long)s * 210;
        memset(o, 0, 210);
        uint8_t* ql = o;
        uint8_t* qh = o + 128;
        for (int i = 0; i < 16; i++) o[192 + i] = (uint8_t)sc8[i];
        put_f16(o + 208, d);
        for (int half = 0; half < 2; half++) {
            int n = half * 128, sc_off = half * 8;
            uint8_t* qlh = ql + half * 64;
            uint8_t* qhh = qh + half * 32;
            for (int l = 0; l < 32; l++) {
                int is = l / 16 + sc_off;
                float s1 = d * (float)sc8[is], s2 = d * (float)sc8[is + 2];
                float s3 = d * (float)sc8[is + 4], s4 = d * (float)sc8[is + 6];
                uint8_t c1 = q6k_code(sup[n + l], s1), c2 = q6k_code(sup[n + 32 + l], s2);
                uint8_t c3 = q6k_code(sup[n + 64 + l], s3), c4 = q6k_code(sup[n + 96 + l], s4);
                qlh[l] |= c1 & 0x0f;
                qlh[l + 32] |= c2 & 0x0f;
                qlh[l] |= (uint8_t)((c3 & 0x0f) << 4);
                qlh[l + 32] |= (uint8_t)((c4 & 0x0f) << 4);
                qhh[l] |= (c1 >> 4) & 0x03;
                qhh[l] |= (uint8_t)(((c2 >> 4) & 0x03) << 2);
                qhh[l] |= (uint8_t)(((c3 >> 4) & 0x03) << 4);
                qhh[l] |= (uint8_t)(((c4 >> 4) & 0x03) << 6);
            }
        }
    }
}

void ref_quantize_rows(int type, const float* src, long rows, int cols, uint8_t* dst,
                       int threads) {
    long rb = ref_row_bytes(type, cols);
    if (threads <= 0) threads = ref_num_threads();
    (void)threads;
#pragma omp parallel for schedule(static) num_threads(threads) if (rows >= 64)
    for (long r = 0; r < rows; r++) {
        const float* row = src + r * cols;
        uint8_t* o = dst + r * rb;
        if (type == REF_Q4_K) quantize_row_q4k(row, cols, o);
        else if (type == REF_Q6_K) quantize_row_q6k(row, cols, o);
        else if (type == REF_Q8_0) quantize_row_q8_0(row, cols, o);
    }
}

/* simd.go:1488-1502 DequantRowQ8_0Into, 1530-1557 DequantRowQ4KInto,
 * 1615-1643 DequantRowQ6KInto */
void ref_dequant_row(int type, const uint8_t* row, int cols, float* out) {
    if (type == REF_Q8_0) {
        for (int b = 0; b < cols / 32; b++) {
            float scale = ref_f16_to_f32(le16(row + (long)b * 34));
            for (int i = 0; i < 32; i++)
                out[b * 32 + i] = scale * (float)(int8_t)row[(long)b * 34 + 2 + i];
        }
    } else if (type == REF_Q4_K) {
        for (int b = 0; b < cols / 256; b++) {
            const uint8_t* blk = row + (long)b * 144;
            float d = ref_f16_to_f32(le16(blk)), dmin = ref_f16_to_f32(le16(blk + 2));
            const uint8_t* q = blk + 16;
            int is = 0;
            for (int j = 0; j < 256; j += 64) {
                int sc1, m1, sc2, m2;
                scale_min_k4(is, blk + 4, &sc1, &m1);
                scale_min_k4(is + 1, blk + 4, &sc2, &m2);
                float d1 = d * (float)sc1, d2 = d * (float)sc2;
                float min1 = dmin * (float)m1, min2 = dmin * (float)m2;
                for (int l = 0; l < 32; l++) {
                    out[b * 256 + j + l] = d1 * (float)(q[l] & 0x0f) - min1;
                    out[b * 256 + j + 32 + l] = d2 * (float)(q[l] >> 4) - min2;
                }
                q += 32;
                is += 2;
            }
        }
    } else if (type == REF_Q6_K) {
        for (int b = 0; b < cols / 256; b++) {
            const uint8_t* blk = row + (long)b * 210;
            float d = ref_f16_to_f32(le16(blk + 208));
            const uint8_t* ql = blk;
            const uint8_t* qh = blk + 128;
            const int8_t* sc = (const int8_t*)(blk + 192);
            for (int n = 0; n < 256; n += 128) {
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    float q1 = (float)(((ql[l] & 0x0f) | ((qh[l] & 0x03) << 4)) - 32);
                    float q2 = (float)(((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 0x03) << 4)) - 32);
                    float q3 = (float)(((ql[l] >> 4) | (((qh[l] >> 4) & 0x03) << 4)) - 32);
                    float q4 = (float)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 0x03) << 4)) - 32);
                    out[b * 256 + n + l] = d * (float)sc[is] * q1;
                    out[b * 256 + n + 32 + l] = d * (float)sc[is + 2] * q2;
                    out[b * 256 + n + 64 + l] = d * (float)sc[is + 4] * q3;
                    out[b * 256 + n + 96 + l] = d * (float)sc[is + 6] * q4;
                }
                ql += 64;
                qh += 32;
                sc += 8;
            }
        }
    } else if (type == REF_Q5_K) {
        /* simd.go:1567-1605 DequantRowQ5KInto */
        for (int b = 0; b < cols / 256; b++) {
            const uint8_t* blk = row + (long)b * 176;
            float d = ref_f16_to_f32(le16(blk)), dmin = ref_f16_to_f32(le16(blk + 2));
            const uint8_t* qh = blk + 16;
            const uint8_t* q = blk + 48;
            int is = 0, u1 = 1, u2 = 2;
            for (int j = 0; j < 256; j += 64) {
                int sc1, m1, sc2, m2;
                scale_min_k4(is, blk + 4, &sc1, &m1);
                scale_min_k4(is + 1, blk + 4, &sc2, &m2);
                float d1 = d * (float)sc1, d2 = d * (float)sc2;
                float min1 = dmin * (float)m1, min2 = dmin * (float)m2;
                for (int l = 0; l < 32; l++) {
                    int hi1 = (qh[l] & u1) ? 16 : 0, hi2 = (qh[l] & u2) ? 16 : 0;
                    out[b * 256 + j + l] = d1 * (float)((q[l] & 0x0f) + hi1) - min1;
                    out[b * 256 + j + 32 + l] = d2 * (float)((q[l] >> 4) + hi2) - min2;
                }
                q += 32;
                is += 2;
                u1 <<= 2;
                u2 <<= 2;
            }
        }
    } else if (type == REF_Q4_0 || type == REF_Q4_1) {
        /* simd.go:1509-1522 DequantRowQ4_0Into, quant_extra.go:20-34 Q4_1 */
        const int bb = type == REF_Q4_0 ? 18 : 20;
        for (int b = 0; b < cols / 32; b++) {
            const uint8_t* blk = row + (long)b * bb;
            float d = ref_f16_to_f32(le16(blk));
            for (int i = 0; i < 16; i++) {
                if (type == REF_Q4_0) {
                    out[b * 32 + i] = d * (float)((blk[2 + i] & 0x0f) - 8);
                    out[b * 32 + 16 + i] = d * (float)(((blk[2 + i] >> 4) & 0x0f) - 8);
                } else {
                    float m = ref_f16_to_f32(le16(blk + 2));
                    out[b * 32 + i] = d * (float)(blk[4 + i] & 0x0f) + m;
                    out[b * 32 + 16 + i] = d * (float)(blk[4 + i] >> 4) + m;
                }
            }
        }
    } else if (type == REF_MXFP4) {
        /* simd.go:1653-1670 DequantRowMXFP4Into: 2^(e-127) * e2m1 value */
        static const float lut[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                                      -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
        for (int b = 0; b < cols / 32; b++) {
            const uint8_t* blk = row + (long)b * 17;
            float scale = (float)ldexp(1.0, (int)blk[16] - 127);
            for (int i = 0; i < 16; i++) {
                out[b * 32 + 2 * i] = scale * lut[blk[i] & 0x0f];
                out[b * 32 + 2 * i + 1] = scale * lut[blk[i] >> 4];
            }
        }
    } else if (type == REF_Q2_K) {
        /* quant_extra.go:233-263 DequantRowQ2KInto */
        for (int b = 0; b < cols / 256; b++) {
            const uint8_t* blk = row + (long)b * 84;
            float d = ref_f16_to_f32(le16(blk + 80)), dmin = ref_f16_to_f32(le16(blk + 82));
            for (int is = 0; is < 16; is++) {
                float dl = d * (float)(blk[is] & 0x0f), ml = dmin * (float)(blk[is] >> 4);
                for (int l = 0; l < 16; l++)
                    out[b * 256 + is * 16 + l] = dl * (float)q2_code(blk + 16, is * 16 + l) - ml;
            }
        }
    } else if (type == REF_Q3_K) {
        /* quant_extra.go:336-368 DequantRowQ3KInto */
        for (int b = 0; b < cols / 256; b++) {
            const uint8_t* blk = row + (long)b * 110;
            int sc[16];
            q3k_scales(blk + 96, sc);
            float d = ref_f16_to_f32(le16(blk + 108));
            for (int is = 0; is < 16; is++) {
                float dl = d * (float)(sc[is] - 32);
                for (int l = 0; l < 16; l++)
                    out[b * 256 + is * 16 + l] = dl * (float)q3_value(blk, is * 16 + l);
            }
        }
    } else if (type == REF_F32) {
        memcpy(out, row, sizeof(float) * (size_t)cols);
    } else if (type == REF_F16) {
        /* raw_scalar.go:145-148: F16ToF32 of each little-endian half */
        for (int i = 0; i < cols; i++) out[i] = ref_f16_to_f32(le16(row + 2L * i));
    } else if (type == REF_BF16) {
        /* raw_scalar.go:149-152: the half's bits as the top of a float32 */
        for (int i = 0; i < cols; i++) {
            const uint32_t bits = (uint32_t)le16(row + 2L * i) << 16;
            memcpy(out + i, &bits, 4);
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Float-activation row dots of the reference's same-type fused groups        */
/* (matvecSameType2/3Into via sameTypeQuantDot, model.go:3213-3283).  Go does */
/* not contract float32 expressions on amd64 (GOAMD64=v1), so every product  */
/* and sum below is rounded on its own, in the Go evaluation order.          */
/* ------------------------------------------------------------------------- */

/* simd.go:646-675 DotQ8_0F32: per block four accumulators over elements
 * i, i+4, ... (s_j gets elements j, 4+j, ..., 28+j in order), then
 * sum += scale * ((s0 + s1) + (s2 + s3)). */
static float float_dot_q8_0(const uint8_t* row, const float* x, int cols) {
    float sum = 0.0f;
    for (int b = 0; b < cols / 32; b++) {
        const uint8_t* blk = row + (long)b * 34;
        const float scale = ref_f16_to_f32(le16(blk));
        const int8_t* r = (const int8_t*)(blk + 2);
        const float* xb = x + (long)b * 32;
        float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int i = 0; i < 32; i += 8) {
            for (int j = 0; j < 4; j++) s[j] = s[j] + (float)r[i + j] * xb[i + j];
            for (int j = 0; j < 4; j++) s[j] = s[j] + (float)r[i + 4 + j] * xb[i + 4 + j];
        }
        sum = sum + scale * ((s[0] + s[1]) + (s[2] + s[3]));
    }
    return sum;
}

/* simd.go:677-715 DotQ4_0F32: s_j += lo*x[i+j] + hi*x[16+i+j] for
 * i = 0, 4, 8, 12 (codes q - 8), sum += scale * ((s0 + s1) + (s2 + s3)). */
static float float_dot_q4_0(const uint8_t* row, const float* x, int cols) {
    float sum = 0.0f;
    for (int b = 0; b < cols / 32; b++) {
        const uint8_t* blk = row + (long)b * 18;
        const float scale = ref_f16_to_f32(le16(blk));
        const uint8_t* r = blk + 2;
        const float* xb = x + (long)b * 32;
        float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int i = 0; i < 16; i += 4)
            for (int j = 0; j < 4; j++) {
                const float lo = (float)((int)(r[i + j] & 0x0f) - 8);
                const float hi = (float)((int)((r[i + j] >> 4) & 0x0f) - 8);
                s[j] = s[j] + (lo * xb[i + j] + hi * xb[16 + i + j]);
            }
        sum = sum + scale * ((s[0] + s[1]) + (s[2] + s[3]));
    }
    return sum;
}

/* quant_extra.go:42-62 DotQ4_1F32: qdot += q_lo*x[i] + q_hi*x[16+i],
 * xsum += x[i] + x[16+i] for i = 0..15, sum += d*qdot + m*xsum. */
static float float_dot_q4_1(const uint8_t* row, const float* x, int cols) {
    float sum = 0.0f;
    for (int b = 0; b < cols / 32; b++) {
        const uint8_t* blk = row + (long)b * 20;
        const float d = ref_f16_to_f32(le16(blk)), m = ref_f16_to_f32(le16(blk + 2));
        const float* xb = x + (long)b * 32;
        float qdot = 0.0f, xsum = 0.0f;
        for (int i = 0; i < 16; i++) {
            const uint8_t pk = blk[4 + i];
            qdot = qdot + ((float)(pk & 0x0f) * xb[i] + (float)(pk >> 4) * xb[16 + i]);
            xsum = xsum + (xb[i] + xb[16 + i]);
        }
        sum = sum + (d * qdot + m * xsum);
    }
    return sum;
}

/* quant_extra.go:271-302 DotQ2KF32: per 16-element sub-block is (scale byte
 * is: low nibble scale, high nibble min) qdot += code*x, xsum += x in
 * element order, sum += dl*qdot - ml*xsum. */
static float float_dot_q2k(const uint8_t* row, const float* x, int cols) {
    float sum = 0.0f;
    for (int b = 0; b < cols / 256; b++) {
        const uint8_t* blk = row + (long)b * 84;
        const float d = ref_f16_to_f32(le16(blk + 80)), dmin = ref_f16_to_f32(le16(blk + 82));
        const float* xb = x + (long)b * 256;
        for (int is = 0; is < 16; is++) {
            const float dl = d * (float)(blk[is] & 0x0f), ml = dmin * (float)(blk[is] >> 4);
            float qdot = 0.0f, xsum = 0.0f;
            for (int l = 0; l < 16; l++) {
                const float xv = xb[is * 16 + l];
                qdot = qdot + (float)q2_code(blk + 16, is * 16 + l) * xv;
                xsum = xsum + xv;
            }
            sum = sum + (dl * qdot - ml * xsum);
        }
    }
    return sum;
}

/* quant_extra.go:376-410 DotQ3KF32: acc += v*x over each 16-element
 * sub-block (v = code - 4 where the hmask bit is clear), sum += dl*acc with
 * dl = d*(scale - 32). */
static float float_dot_q3k(const uint8_t* row, const float* x, int cols) {
    float sum = 0.0f;
    for (int b = 0; b < cols / 256; b++) {
        const uint8_t* blk = row + (long)b * 110;
        int sc[16];
        q3k_scales(blk + 96, sc);
        const float d = ref_f16_to_f32(le16(blk + 108));
        const float* xb = x + (long)b * 256;
        for (int is = 0; is < 16; is++) {
            const float dl = d * (float)(sc[is] - 32);
            float acc = 0.0f;
            for (int l = 0; l < 16; l++)
                acc = acc + (float)q3_value(blk, is * 16 + l) * xb[is * 16 + l];
            sum = sum + dl * acc;
        }
    }
    return sum;
}

/* simd.go:1031-1186 DotQ5KF32: per 64-element step s of a block, lane
 * accumulators j = l % 4 over l = 0..31 of qd1_j += code1*x1, qd2_j +=
 * code2*x2, xs1_j += x1, xs2_j += x2 (code = nibble + 16 * qh bit 2s / 2s+1),
 * then sum += d1*qdot1 - min1*xsum1 and sum += d2*qdot2 - min2*xsum2 with
 * qdot = (a0 + a1) + (a2 + a3). */
static float float_dot_q5k(const uint8_t* row, const float* x, int cols) {
    float sum = 0.0f;
    for (int b = 0; b < cols / 256; b++) {
        const uint8_t* blk = row + (long)b * 176;
        const float d = ref_f16_to_f32(le16(blk)), dmin = ref_f16_to_f32(le16(blk + 2));
        const uint8_t* qh = blk + 16;
        const float* xb = x + (long)b * 256;
        for (int st = 0; st < 4; st++) {
            int sc1, m1, sc2, m2;
            scale_min_k4(2 * st, blk + 4, &sc1, &m1);
            scale_min_k4(2 * st + 1, blk + 4, &sc2, &m2);
            const float d1 = d * (float)sc1, d2 = d * (float)sc2;
            const float min1 = dmin * (float)m1, min2 = dmin * (float)m2;
            const uint8_t* q = blk + 48 + 32 * st;
            const float* x1 = xb + 64 * st;
            const float* x2 = x1 + 32;
            float qd1[4] = {0}, qd2[4] = {0}, xs1[4] = {0}, xs2[4] = {0};
            for (int l = 0; l < 32; l += 4)
                for (int j = 0; j < 4; j++) {
                    const int h1 = (qh[l + j] >> (2 * st)) & 1, h2 = (qh[l + j] >> (2 * st + 1)) & 1;
                    qd1[j] = qd1[j] + (float)((q[l + j] & 0x0f) + 16 * h1) * x1[l + j];
                    qd2[j] = qd2[j] + (float)((q[l + j] >> 4) + 16 * h2) * x2[l + j];
                    xs1[j] = xs1[j] + x1[l + j];
                    xs2[j] = xs2[j] + x2[l + j];
                }
            const float qdot1 = (qd1[0] + qd1[1]) + (qd1[2] + qd1[3]);
            const float qdot2 = (qd2[0] + qd2[1]) + (qd2[2] + qd2[3]);
            const float xsum1 = (xs1[0] + xs1[1]) + (xs1[2] + xs1[3]);
            const float xsum2 = (xs2[0] + xs2[1]) + (xs2[2] + xs2[3]);
            sum = sum + (d1 * qdot1 - min1 * xsum1);
            sum = sum + (d2 * qdot2 - min2 * xsum2);
        }
    }
    return sum;
}

/* simd.go:1458-1477 DotMXFP4F32: sum += (lut[code] * scale) * x for every
 * element in order, scale = float32(2^(e - 127)). */
static float float_dot_mxfp4(const uint8_t* row, const float* x, int cols) {
    static const float lut[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                                  -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
    float sum = 0.0f;
    for (int b = 0; b < cols / 32; b++) {
        const uint8_t* blk = row + (long)b * 17;
        const float scale = (float)ldexp(1.0, (int)blk[16] - 127);
        const float* xb = x + (long)b * 32;
        for (int i = 0; i < 16; i++) {
            sum = sum + (lut[blk[i] & 0x0f] * scale) * xb[2 * i];
            sum = sum + (lut[blk[i] >> 4] * scale) * xb[2 * i + 1];
        }
    }
    return sum;
}

int ref_float_dot_supported(int type) {
    return type == REF_Q8_0 || type == REF_Q4_0 || type == REF_Q4_1 || type == REF_Q2_K ||
           type == REF_Q3_K || type == REF_Q5_K || type == REF_MXFP4;
}

float ref_float_dot(int type, const uint8_t* row, const float* x, int cols) {
    switch (type) {
    case REF_Q8_0: return float_dot_q8_0(row, x, cols);
    case REF_Q4_0: return float_dot_q4_0(row, x, cols);
    case REF_Q4_1: return float_dot_q4_1(row, x, cols);
    case REF_Q2_K: return float_dot_q2k(row, x, cols);
    case REF_Q3_K: return float_dot_q3k(row, x, cols);
    case REF_Q5_K: return float_dot_q5k(row, x, cols);
    case REF_MXFP4: return float_dot_mxfp4(row, x, cols);
    default: return NAN;
    }
}

/* matvecDotRows over all rows (model.go:3213-3256; rows are independent) */
int ref_matvec_float(int type, const uint8_t* data, const float* x, int rows, int cols,
                     float* out, int threads) {
    if (!ref_float_dot_supported(type)) return -1;
    const long rb = ref_row_bytes(type, cols);
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : ref_num_threads())
    for (int r = 0; r < rows; r++) out[r] = ref_float_dot(type, data + (long)r * rb, x, cols);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* Vector helpers (kernels_amd64.s)                                           */
/* ------------------------------------------------------------------------- */

/* kernels_amd64.s:28-93 dotF32AVX2 */
float ref_dot_f32(const float* a, const float* b, long n) {
    float y[4][8];
    memset(y, 0, sizeof y);
    long i = 0, n32 = n & ~31L, n8 = n & ~7L;
    for (; i < n32; i += 32)
        for (int r = 0; r < 4; r++)
            for (int k = 0; k < 8; k++) y[r][k] = fmaf(a[i + 8 * r + k], b[i + 8 * r + k], y[r][k]);
    float acc[8];
    for (int k = 0; k < 8; k++) acc[k] = (y[0][k] + y[1][k]) + (y[2][k] + y[3][k]);
    for (; i < n8; i += 8)
        for (int k = 0; k < 8; k++) acc[k] = fmaf(a[i + k], b[i + k], acc[k]);
    float s = tree8(acc);
    for (; i < n; i++) s = s + a[i] * b[i];
    return s;
}

/* kernels_amd64.s:104-129 dotF32F16AVX2 + the Go scalar tail
 * (kernels_amd64.go:94-100, kv_f16.go:51-58). */
float ref_dot_f32_f16(const float* a, const uint16_t* b, long n) {
    float acc[8] = {0};
    long i = 0, n8 = n & ~7L;
    for (; i < n8; i += 8)
        for (int k = 0; k < 8; k++) acc[k] = fmaf(ref_f16_to_f32(b[i + k]), a[i + k], acc[k]);
    float s = tree8(acc);
    float tail = 0.0f;
    for (; i < n; i++) tail += a[i] * ref_f16_to_f32(b[i]);
    return s + tail;
}

/* fastmath.go:47-77 fastExpF32 */
float ref_fast_exp(float x) {
    if (x > 88.02969f) return INFINITY;
    if (x < -87.33654f) return 0.0f;
    float t = x * (float)1.4426950408889634;
    int32_t k;
    if (t >= 0) k = (int32_t)(t + 0.5f);
    else k = (int32_t)(t - 0.5f);
    float r = (float)((double)x - (double)k * 0.6931471805599453);
    float p = 1.0f + r * (1.0f + r * (0.5f + r * ((float)(1.0 / 6) +
              r * ((float)(1.0 / 24) + r * ((float)(1.0 / 120) + r * (float)(1.0 / 720))))));
    return p * bits_f32((uint32_t)(127 + k) << 23);
}

/* kernels_amd64.s:1630-1700 siluMulF32AVX2 (Cephes exp, stable sigmoid) */
static float silu_mul_one(float g, float up) {
    const float lo_clamp = bits_f32(0xc2b0c0a5u);   /* -88.376 */
    const float log2e = bits_f32(0x3fb8aa3bu);
    const float c1 = bits_f32(0x3f318000u);         /* 0.693359375 */
    const float c2 = bits_f32(0xb95e8083u);         /* -2.12194440e-4 */
    const float p0 = bits_f32(0x39506967u), p1 = bits_f32(0x3ab743ceu);
    const float p2 = bits_f32(0x3c088908u), p3 = bits_f32(0x3d2aa9c1u);
    const float p4 = bits_f32(0x3e2aaaaau), p5 = bits_f32(0x3f000000u);
    const float fx_lo = bits_f32(0xc2fc0000u);       /* -126 */
    float a = bits_f32(f32_bits(g) | 0x80000000u);  /* -|g| */
    float a_unclamped = a;
    float ac = (a != a) ? lo_clamp : (a > lo_clamp ? a : lo_clamp); /* VMAXPS, NaN -> 2nd */
    float fx = ref_round_to_even_f32(ac * log2e);  /* VROUNDPS $0 (|fx| < 2^22) */
    fx = (fx != fx) ? fx_lo : (fx > fx_lo ? fx : fx_lo);
    float r = fmaf(-fx, c1, ac);
    r = fmaf(-fx, c2, r);
    float y = fmaf(p0, r, p1);
    y = fmaf(y, r, p2);
    y = fmaf(y, r, p3);
    y = fmaf(y, r, p4);
    y = fmaf(y, r, p5);
    float r2 = r * r;
    y = fmaf(y, r2, r);
    y = y + 1.0f;
    int32_t fi = (int32_t)fx;                       /* VCVTPS2DQ of an integral value */
    float e = y * bits_f32((uint32_t)(fi + 127) << 23);
    if (a_unclamped < lo_clamp) e = 0.0f;           /* VCMPPS LT_OS + VPANDN */
    float num = (f32_bits(g) & 0x80000000u) ? e : 1.0f;
    float s = num / (1.0f + e);
    return (g * s) * up;
}

void ref_silu_mul(const float* gate, const float* up, float* out, long n) {
    /* n % 8 == 0 on the model shapes; the scalar tail (simd.go fastSigmoidF32)
     * is not restated. */
    for (long i = 0; i < n; i++) out[i] = silu_mul_one(gate[i], up[i]);
}

/* model.go:2986-3011 rmsNormInto with mulScaleF32AVX2 (kernels_amd64.s:1488-1525) */
void ref_rmsnorm(const float* x, const float* w, float eps, long n, float* out) {
    float ss = ref_dot_f32(x, x, n);
    float scale = (float)(1.0 / sqrt((double)(ss / (float)n + eps)));
    for (long i = 0; i < n; i++) out[i] = (x[i] * w[i]) * scale;
}

/* model.go:1728-1756 buildRopeInvFreq (no scaling factors, ropeDim = hd) */
void ref_rope_inv_freq(float theta, int head_dim, float* inv) {
    int pairs = head_dim / 2;
    for (int pair = 0; pair < pairs; pair++) {
        float i = (float)(pair * 2);
        float base = (float)pow((double)theta, (double)(i / (float)head_dim));
        float factor = 1.0f;
        inv[pair] = 1.0f / (factor * base);
    }
}

/* model.go:3020-3049 prepareRopeScratch (mscale 1) */
void ref_rope_sincos(int pos, const float* inv, int pairs, float* sinv, float* cosv) {
    for (int i = 0; i < pairs; i++) {
        double angle = (double)((float)pos * inv[i]);
        sinv[i] = (float)sin(angle) * 1.0f;
        cosv[i] = (float)cos(angle) * 1.0f;
    }
}

/* model.go:3051-3082 applyPreparedRope, interleaved (llama, model.go:3084-3093) */
void ref_rope_apply(float* vec, int head_dim, int n_heads, int pairs, const float* sinv,
                    const float* cosv) {
    for (int h = 0; h < n_heads; h++) {
        float* sub = vec + (long)h * head_dim;
        for (int i = 0; i < pairs; i++) {
            float s = sinv[i], c = cosv[i];
            float v0 = sub[2 * i], v1 = sub[2 * i + 1];
            sub[2 * i] = v0 * c - v1 * s;
            sub[2 * i + 1] = v0 * s + v1 * c;
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Attention (model.go:3527-3588 onlineAttentionGroup4F16; 3761-3787         */
/* attentionWeightsInPlace; the per-head path kv_f16.go:88-111 +              */
/* model.go:3801-3855 performs the same operations)                           */
/* ------------------------------------------------------------------------- */

void ref_attend_group_f16(const float* q, const uint16_t* keys, const uint16_t* values,
                          int q_heads, long kstride, long vstride, int hd, int vd, int start,
                          int end, float scale, float* out) {
    int span = end - start + 1;
    if (span <= 0) return;
    float* scores = (float*)malloc(sizeof(float) * (size_t)span * (size_t)q_heads);
    for (int h = 0; h < q_heads; h++) {
        float* sc = scores + (long)h * span;
        for (int t = start; t <= end; t++)
            sc[t - start] = ref_dot_f32_f16(q + (long)h * hd, keys + (long)t * kstride, hd) * scale;
        float mx = sc[0];
        for (int i = 1; i < span; i++)
            if (sc[i] > mx) mx = sc[i];
        float denom = 0.0f;
        for (int i = 0; i < span; i++) {
            float w = ref_fast_exp(sc[i] - mx);
            sc[i] = w;
            denom += w;
        }
        float* o = out + (long)h * vd;
        for (int d = 0; d < vd; d++) o[d] = 0.0f;
        for (int i = 0; i < span; i++) {
            const uint16_t* v = values + (long)(start + i) * vstride;
            long n8 = vd & ~7L;
            for (long d = 0; d < n8; d++) o[d] = fmaf(sc[i], ref_f16_to_f32(v[d]), o[d]);
            for (long d = n8; d < vd; d++) o[d] += sc[i] * ref_f16_to_f32(v[d]);
        }
        if (denom > 0) {
            float inv = 1.0f / denom;
            for (int d = 0; d < vd; d++) o[d] = o[d] * inv;
        }
    }
    free(scores);
}

/* ------------------------------------------------------------------------- */
/* llama decoder                                                              */
/* ------------------------------------------------------------------------- */

struct ref_llama_state {
    ref_llama m;
    int threads;
    int fast; /* row dots through the AVX2 port (bit-identical to the amd64 order) */
    uint16_t** kc;
    uint16_t** vc;
    float* inv_freq;
    float *x, *xn, *q, *k, *v, *attn, *proj, *gate, *up, *hidden, *logits, *sinv, *cosv;
    /* repeat penalty and the trailing token window it reads (runtime.go:
     * recentTokenWindowInto 1225-1228, appended per emitted token 1089-1093) */
    float penalty;
    int window, n_recent;
    uint32_t* recent;
};

/* append to the window, keeping its last `window` ids in order */
static void llama_push_recent(ref_llama_state* s, uint32_t tok) {
    if (s->window <= 0) return;
    if (s->n_recent == s->window) {
        memmove(s->recent, s->recent + 1, sizeof(uint32_t) * (size_t)(s->window - 1));
        s->n_recent--;
    }
    s->recent[s->n_recent++] = tok;
}

void ref_llama_set_repeat_penalty(ref_llama_state* s, float penalty, int window) {
    free(s->recent);
    s->penalty = penalty;
    s->window = window > 0 ? window : 0;
    s->n_recent = 0;
    s->recent = (uint32_t*)calloc((size_t)(s->window > 0 ? s->window : 1), sizeof(uint32_t));
}

ref_llama_state* ref_llama_state_new(const ref_llama* m, int threads) {
    ref_llama_state* s = (ref_llama_state*)calloc(1, sizeof *s);
    s->m = *m;
    s->threads = threads;
    s->penalty = 1.0f;
    int kvd = m->n_kv_heads * m->head_dim;
    s->kc = (uint16_t**)calloc((size_t)m->n_layers, sizeof(uint16_t*));
    s->vc = (uint16_t**)calloc((size_t)m->n_layers, sizeof(uint16_t*));
    for (int l = 0; l < m->n_layers; l++) {
        s->kc[l] = (uint16_t*)calloc((size_t)m->max_len * kvd, 2);
        s->vc[l] = (uint16_t*)calloc((size_t)m->max_len * kvd, 2);
    }
    s->inv_freq = (float*)malloc(sizeof(float) * (size_t)(m->head_dim / 2));
    ref_rope_inv_freq(m->rope_theta, m->head_dim, s->inv_freq);
    int qd = m->n_heads * m->head_dim;
    s->x = (float*)malloc(sizeof(float) * m->dim);
    s->xn = (float*)malloc(sizeof(float) * m->dim);
    s->q = (float*)malloc(sizeof(float) * qd);
    s->k = (float*)malloc(sizeof(float) * kvd);
    s->v = (float*)malloc(sizeof(float) * kvd);
    s->attn = (float*)malloc(sizeof(float) * qd);
    s->proj = (float*)malloc(sizeof(float) * m->dim);
    s->gate = (float*)malloc(sizeof(float) * m->hidden);
    s->up = (float*)malloc(sizeof(float) * m->hidden);
    s->hidden = (float*)malloc(sizeof(float) * m->hidden);
    s->logits = (float*)malloc(sizeof(float) * m->vocab);
    s->sinv = (float*)malloc(sizeof(float) * (m->head_dim / 2));
    s->cosv = (float*)malloc(sizeof(float) * (m->head_dim / 2));
    return s;
}

void ref_llama_state_free(ref_llama_state* s) {
    if (!s) return;
    for (int l = 0; l < s->m.n_layers; l++) { free(s->kc[l]); free(s->vc[l]); }
    free(s->kc); free(s->vc); free(s->inv_freq);
    free(s->x); free(s->xn); free(s->q); free(s->k); free(s->v); free(s->attn);
    free(s->proj); free(s->gate); free(s->up); free(s->hidden); free(s->logits);
    free(s->sinv); free(s->cosv); free(s->recent);
    free(s);
}

const uint16_t* ref_llama_kcache(ref_llama_state* s, int l) { return s->kc[l]; }
const uint16_t* ref_llama_vcache(ref_llama_state* s, int l) { return s->vc[l]; }

void ref_llama_set_fast(ref_llama_state* s, int on) { s->fast = on && ref_has_avx2(); }

/* W.x in the amd64 order: the lane-level restatement, or its AVX2 port when
 * s->fast is set (the two are bit-identical; the port is only faster). */
static void llama_matvec(ref_llama_state* s, int type, const uint8_t* w, const float* x, int rows,
                         int cols, float* out) {
    if (s->fast && ref_matvec_batch_fast(type, w, x, 1, rows, cols, out, s->threads) == 0) return;
    ref_matvec(type, w, x, rows, cols, out, REF_ORDER_AMD64, s->threads);
}

/* type of matrix `slot` (0..6: wq wk wv wo w1 w2 w3) of layer l */
static int llama_type(const ref_llama* m, int l, int slot) {
    return m->types ? m->types[l * 7 + slot] : m->layer_type;
}

/* W.x through the float kernels of a same-type fused group
 * (matvecSameType2/3Into, model.go:3213-3256) */
static void llama_matvec_float(ref_llama_state* s, int type, const uint8_t* w, const float* x,
                               int rows, int cols, float* out) {
    ref_matvec_float(type, w, x, rows, cols, out, s->threads);
}

/* The fused-group routing of one decode step.  tryMatvec2Into
 * (model.go:3186-3206): a same-type pair of Q4_K or Q6_K runs the int8 row
 * dots (which give each projection the same values as its own MatvecInto),
 * any other same-type pair the float kernels; different types are no pair. */
static int pair_float(int ta, int tb) { return ta == tb && ta != REF_Q4_K && ta != REF_Q6_K; }

/* tryMatvecAttentionInto (model.go:3157-3184) for Q, K, V of layer l: all
 * three of one type -> tryMatvec3Into (int8 for Q4_K / Q6_K, float kernels
 * otherwise); Q4_K/Q4_K/Q6_K -> int8; else the first same-type pair of
 * (q,k), (q,v), (k,v) fused and the third on its own; else each on its own
 * (MatvecInto, int8).  fl[i] = 1 marks the projections that run the float
 * kernels. */
static void qkv_routing(const ref_llama* m, int l, int fl[3]) {
    const int tq = llama_type(m, l, 0), tk = llama_type(m, l, 1), tv = llama_type(m, l, 2);
    fl[0] = fl[1] = fl[2] = 0;
    if (tq == tk && tq == tv) {
        if (pair_float(tq, tq)) fl[0] = fl[1] = fl[2] = 1;
        return;
    }
    if (tq == REF_Q4_K && tk == REF_Q4_K && tv == REF_Q6_K) return;
    if (tq == tk) fl[0] = fl[1] = pair_float(tq, tk);
    else if (tq == tv) fl[0] = fl[2] = pair_float(tq, tv);
    else if (tk == tv) fl[1] = fl[2] = pair_float(tk, tv);
}

/* ForwardBodyInto (model.go:2622-2820) for the plain llama graph; leaves the
 * output-normed hidden state in s->xn.  decode != 0 is the generation step
 * (fused-group routing, qkv_routing / tryMatvec2Into for gate and up);
 * decode == 0 is a prompt token of the batched prefill, where every
 * projection runs matvecBatchQ8's int8 row dots on its own
 * (forward_batch.go:108-204, matvecBatch3/2 forward_batch.go:210-233). */
static void llama_body(ref_llama_state* s, uint32_t token, int pos, int decode) {
    const ref_llama* m = &s->m;
    int dim = m->dim, hd = m->head_dim, kvd = m->n_kv_heads * hd;
    int kvmul = m->n_heads / m->n_kv_heads;
    long er = ref_row_bytes(m->emb_type, dim);
    ref_dequant_row(m->emb_type, m->tok_embd + (long)token * er, dim, s->x);
    ref_rope_sincos(pos, s->inv_freq, hd / 2, s->sinv, s->cosv);
    float scale = m->attn_scale != 0.0f ? m->attn_scale : (float)(1.0 / sqrt((double)hd));
    for (int l = 0; l < m->n_layers; l++) {
        ref_rmsnorm(s->x, m->attn_norm[l], m->rms_eps, dim, s->xn);
        int fl[3] = {0, 0, 0};
        if (decode) qkv_routing(m, l, fl);
        (fl[0] ? llama_matvec_float : llama_matvec)(s, llama_type(m, l, 0), m->wq[l], s->xn,
                                                    m->n_heads * hd, dim, s->q);
        (fl[1] ? llama_matvec_float : llama_matvec)(s, llama_type(m, l, 1), m->wk[l], s->xn, kvd,
                                                    dim, s->k);
        (fl[2] ? llama_matvec_float : llama_matvec)(s, llama_type(m, l, 2), m->wv[l], s->xn, kvd,
                                                    dim, s->v);
        ref_rope_apply(s->q, hd, m->n_heads, hd / 2, s->sinv, s->cosv);
        ref_rope_apply(s->k, hd, m->n_kv_heads, hd / 2, s->sinv, s->cosv);
        ref_f32_to_f16_row(s->k, s->kc[l] + (long)pos * kvd, kvd);
        ref_f32_to_f16_row(s->v, s->vc[l] + (long)pos * kvd, kvd);
        /* kv groups are independent; each keeps its own sequential order */
#pragma omp parallel for schedule(static) num_threads(s->threads > 0 ? s->threads : ref_num_threads()) if (pos >= 64)
        for (int g = 0; g < m->n_kv_heads; g++)
            ref_attend_group_f16(s->q + (long)g * kvmul * hd, s->kc[l] + (long)g * hd,
                                 s->vc[l] + (long)g * hd, kvmul, kvd, kvd, hd, hd, 0, pos, scale,
                                 s->attn + (long)g * kvmul * hd);
        llama_matvec(s, llama_type(m, l, 3), m->wo[l], s->attn, dim, m->n_heads * hd, s->proj);
        for (int i = 0; i < dim; i++) s->x[i] = fmaf(s->proj[i], 1.0f, s->x[i]);
        ref_rmsnorm(s->x, m->ffn_norm[l], m->rms_eps, dim, s->xn);
        const int gu_float = decode && pair_float(llama_type(m, l, 4), llama_type(m, l, 6));
        (gu_float ? llama_matvec_float : llama_matvec)(s, llama_type(m, l, 4), m->w1[l], s->xn,
                                                       m->hidden, dim, s->gate);
        (gu_float ? llama_matvec_float : llama_matvec)(s, llama_type(m, l, 6), m->w3[l], s->xn,
                                                       m->hidden, dim, s->up);
        ref_silu_mul(s->gate, s->up, s->hidden, m->hidden);
        llama_matvec(s, llama_type(m, l, 5), m->w2[l], s->hidden, dim, m->hidden, s->proj);
        for (int i = 0; i < dim; i++) s->x[i] = fmaf(s->proj[i], 1.0f, s->x[i]);
    }
    ref_rmsnorm(s->x, m->out_norm, m->rms_eps, dim, s->xn);
}

/* ForwardBodyInto + ArgmaxMatvec (runtime.go:1607-1656, model.go:2574-2610) */
uint32_t ref_llama_decode(ref_llama_state* s, uint32_t token, int pos, float* hidden_out) {
    llama_body(s, token, pos, 1);
    if (hidden_out) memcpy(hidden_out, s->xn, sizeof(float) * s->m.dim);
    llama_push_recent(s, token);  /* emitToken appends before the next choice */
    if (s->penalty != 1.0f) {
        /* forwardGreedyToken with penalty != 1: ProjectLogitsInto, then
         * SampleWithScratch's greedy branch (sampling.go:86-89) */
        llama_matvec(s, s->m.out_type, s->m.output, s->xn, s->m.vocab, s->m.dim, s->logits);
        ref_apply_repeat_penalty(s->logits, s->m.vocab, s->recent, s->n_recent, s->penalty);
        return ref_argmax_finite(s->logits, s->m.vocab);
    }
    if (s->fast) {
        /* argmax(W.x) over finite logits, lowest index on ties, equals
         * argmaxQ6KRowsQ8's result (kernels_amd64.go:294-331) */
        llama_matvec(s, s->m.out_type, s->m.output, s->xn, s->m.vocab, s->m.dim, s->logits);
        return ref_argmax_finite(s->logits, s->m.vocab);
    }
    return ref_argmax_matvec(s->m.out_type, s->m.output, s->xn, s->m.vocab, s->m.dim,
                             REF_ORDER_AMD64, s->threads);
}

/* prefillBatchedAt (runtime.go:1715-1726) -> ForwardBatchInto
 * (forward_batch.go:336-613).  The batched row kernels produce per-token
 * results identical to the per-token path (same row kernel, same q8 and
 * xsums per token), so the chunk is evaluated token by token; chunking only
 * decides which position's logits are materialised. */
uint32_t ref_llama_prefill(ref_llama_state* s, const uint32_t* tokens, int n, int start_pos,
                           int chunk, float* logits_out) {
    (void)chunk;
    for (int t = 0; t < n; t++) {
        llama_body(s, tokens[t], start_pos + t, 0);
        llama_push_recent(s, tokens[t]);
    }
    llama_matvec(s, s->m.out_type, s->m.output, s->xn, s->m.vocab, s->m.dim, s->logits);
    if (logits_out) memcpy(logits_out, s->logits, sizeof(float) * s->m.vocab);
    /* the first generated token: SampleWithScratch over the prompt window */
    ref_apply_repeat_penalty(s->logits, s->m.vocab, s->recent, s->n_recent, s->penalty);
    return ref_argmax_finite(s->logits, s->m.vocab);
}

/* Greedy decode loop (runtime.go:1129-1170): the first token comes from the
 * prefill logits, each later token from ForwardBodyInto + ArgmaxMatvec. */
void ref_llama_generate(ref_llama_state* s, const uint32_t* prompt, int n_prompt, int n_gen,
                        int chunk, uint32_t* out_tokens) {
    if (n_gen <= 0) return;
    uint32_t tok = ref_llama_prefill(s, prompt, n_prompt, 0, chunk, NULL);
    out_tokens[0] = tok;
    for (int i = 1; i < n_gen; i++) {
        tok = ref_llama_decode(s, tok, n_prompt + i - 1, NULL);
        out_tokens[i] = tok;
    }
}

int ref_has_avx2(void) {
#if defined(__x86_64__)
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") &&
           __builtin_cpu_supports("f16c");
#else
    return 0;
#endif
}
