/*
 * gllm_oracle_avx2.c -- AVX2 port of the reference's amd64 row kernels, used
 * as the timed CPU baseline.  TEST INFRASTRUCTURE ONLY.
 *
 * Each kernel issues the same vector operations in the same order as
 * kernels_amd64.s (VPMADDUBSW pair sums, VPMADDWD by the sub-block scale,
 * VCVTDQ2PS, VFMADD231PS accumulation, 8->4->2->1 tree), so its results are
 * bit-identical to the scalar lane emulation in gllm_oracle.c; the tests
 * assert that equality.  Rows are split across threads with the reference's
 * parallelRows partition (simd.go:1683-1757: threads = min(nproc, rows), run
 * inline below 8 rows per thread).
 */
#include "gllm_oracle.h"

#include <immintrin.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float hsum8(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    lo = _mm_add_ps(lo, hi);
    lo = _mm_hadd_ps(lo, lo);
    lo = _mm_hadd_ps(lo, lo);
    return _mm_cvtss_f32(lo);
}

static inline float f16_scalar(uint16_t h) {
    return _mm_cvtss_f32(_mm_cvtph_ps(_mm_cvtsi32_si128(h)));
}

/* kernels_amd64.s:465-543 */
float ref_q4k_dot_avx2(const uint8_t* q, const int8_t* q8, const float* xscales,
                       const float* xsums, int blocks) {
    const __m256i m4 = _mm256_set1_epi8(0x0f);
    __m256 accF = _mm256_setzero_ps(), accM = _mm256_setzero_ps();
    for (int b = 0; b < blocks; b++, q += 144, q8 += 256) {
        uint32_t A, B, C;
        memcpy(&A, q + 4, 4);
        memcpy(&B, q + 8, 4);
        memcpy(&C, q + 12, 4);
        uint32_t sc03 = A & 0x3f3f3f3fu;
        uint32_t sc47 = (C & 0x0f0f0f0fu) | ((A >> 2) & 0x30303030u);
        uint32_t m03 = B & 0x3f3f3f3fu;
        uint32_t m47 = ((C >> 4) & 0x0f0f0f0fu) | ((B >> 2) & 0x30303030u);
        uint8_t sc[8], mm[8];
        memcpy(sc, &sc03, 4);
        memcpy(sc + 4, &sc47, 4);
        memcpy(mm, &m03, 4);
        memcpy(mm + 4, &m47, 4);
        float d = f16_scalar((uint16_t)(q[0] | (q[1] << 8)));
        float dmin = f16_scalar((uint16_t)(q[2] | (q[3] << 8)));
        __m256 mins = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*)mm)));
        mins = _mm256_mul_ps(mins, _mm256_loadu_ps(xsums + 8 * b));
        accM = _mm256_fmadd_ps(_mm256_set1_ps(dmin), mins, accM);
        __m256i acc = _mm256_setzero_si256();
        for (int s = 0; s < 4; s++) {
            __m256i w = _mm256_loadu_si256((const __m256i*)(q + 16 + 32 * s));
            __m256i lo = _mm256_and_si256(w, m4);
            __m256i hi = _mm256_and_si256(_mm256_srli_epi16(w, 4), m4);
            __m256i plo = _mm256_maddubs_epi16(lo, _mm256_loadu_si256((const __m256i*)(q8 + 64 * s)));
            plo = _mm256_madd_epi16(plo, _mm256_set1_epi16(sc[2 * s]));
            acc = _mm256_add_epi32(acc, plo);
            __m256i phi = _mm256_maddubs_epi16(hi, _mm256_loadu_si256((const __m256i*)(q8 + 64 * s + 32)));
            phi = _mm256_madd_epi16(phi, _mm256_set1_epi16(sc[2 * s + 1]));
            acc = _mm256_add_epi32(acc, phi);
        }
        float dxs = d * xscales[b];
        accF = _mm256_fmadd_ps(_mm256_set1_ps(dxs), _mm256_cvtepi32_ps(acc), accF);
    }
    return hsum8(_mm256_sub_ps(accF, accM));
}

/* kernels_amd64.s:1150-1220 */
float ref_q6k_dot_avx2(const uint8_t* row, const int8_t* q8, const float* xscales,
                       const float* xsums, int blocks) {
    const __m256i m4 = _mm256_set1_epi8(0x0f), m2 = _mm256_set1_epi8(0x03);
    __m256 accF = _mm256_setzero_ps(), accM = _mm256_setzero_ps();
    for (int b = 0; b < blocks; b++, row += 210, q8 += 256) {
        float d = f16_scalar((uint16_t)(row[208] | (row[209] << 8)));
        int16_t sc16[16];
        for (int i = 0; i < 16; i++) sc16[i] = (int8_t)row[192 + i];
        __m256 s_lo = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)(row + 192))));
        __m256 s_hi = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)(row + 200))));
        __m256 t = _mm256_mul_ps(s_lo, _mm256_loadu_ps(xsums + 16 * b));
        t = _mm256_fmadd_ps(s_hi, _mm256_loadu_ps(xsums + 16 * b + 8), t);
        accM = _mm256_fmadd_ps(_mm256_set1_ps(d), t, accM);
        __m256i acc = _mm256_setzero_si256();
        for (int h = 0; h < 2; h++) {
            __m256i y0 = _mm256_loadu_si256((const __m256i*)(row + 64 * h));
            __m256i y1 = _mm256_loadu_si256((const __m256i*)(row + 64 * h + 32));
            __m256i y2 = _mm256_loadu_si256((const __m256i*)(row + 128 + 32 * h));
            for (int c = 0; c < 4; c++) {
                __m256i ql = (c & 1) ? y1 : y0;
                __m256i v = (c < 2) ? ql : _mm256_srli_epi16(ql, 4);
                v = _mm256_and_si256(v, m4);
                __m256i hb = _mm256_and_si256(_mm256_srli_epi16(y2, 2 * c), m2);
                v = _mm256_or_si256(v, _mm256_slli_epi16(hb, 4));
                __m256i p = _mm256_maddubs_epi16(v, _mm256_loadu_si256((const __m256i*)(q8 + 128 * h + 32 * c)));
                __m256i scv = _mm256_set_m128i(_mm_set1_epi16(sc16[8 * h + 2 * c + 1]),
                                               _mm_set1_epi16(sc16[8 * h + 2 * c]));
                acc = _mm256_add_epi32(acc, _mm256_madd_epi16(p, scv));
            }
        }
        float dxs = d * xscales[b];
        accF = _mm256_fmadd_ps(_mm256_set1_ps(dxs), _mm256_cvtepi32_ps(acc), accF);
    }
    return hsum8(_mm256_sub_ps(accF, accM));
}

/* kernels_amd64.s:1333-1391 */
float ref_q8_0_dot_avx2(const uint8_t* row, const int8_t* q8, const float* xscales, int blocks) {
    const __m256i ones = _mm256_set1_epi16(1);
    __m256 acc11 = _mm256_setzero_ps();
    for (int b = 0; b < blocks; b++, row += 272, q8 += 256) {
        __m256 acc12 = _mm256_setzero_ps();
        for (int j = 0; j < 8; j++) {
            const uint8_t* blk = row + 34 * j;
            __m256 d = _mm256_set1_ps(f16_scalar((uint16_t)(blk[0] | (blk[1] << 8))));
            __m256i w = _mm256_loadu_si256((const __m256i*)(blk + 2));
            __m256i x = _mm256_loadu_si256((const __m256i*)(q8 + 32 * j));
            __m256i p = _mm256_maddubs_epi16(_mm256_abs_epi8(w), _mm256_sign_epi8(x, w));
            p = _mm256_madd_epi16(p, ones);
            acc12 = _mm256_fmadd_ps(d, _mm256_cvtepi32_ps(p), acc12);
        }
        acc11 = _mm256_fmadd_ps(_mm256_set1_ps(xscales[b]), acc12, acc11);
    }
    return hsum8(acc11);
}

/* kernels_amd64.s:208-230 / 234-254 */
static void xsums32_avx2(const float* x, float* out, int groups) {
    for (int g = 0; g < groups; g++, x += 32) {
        __m256 v = _mm256_loadu_ps(x);
        v = _mm256_add_ps(v, _mm256_loadu_ps(x + 8));
        v = _mm256_add_ps(v, _mm256_loadu_ps(x + 16));
        v = _mm256_add_ps(v, _mm256_loadu_ps(x + 24));
        out[g] = hsum8(v);
    }
}
static void xsums16x32_avx2(const float* x, float* out, int groups) {
    for (int g = 0; g < groups; g++, x += 16)
        out[g] = hsum8(_mm256_add_ps(_mm256_loadu_ps(x), _mm256_loadu_ps(x + 8))) * 32.0f;
}

/* Fast driver: quantise once per activation vector, then the parallelRows
 * partition over rows (simd.go:1683-1757).  Returns 0 on success, -1 when the
 * host lacks AVX2/FMA/F16C or the shape is unsupported. */
int ref_matvec_batch_fast(int type, const uint8_t* data, const float* xs, int p, int rows,
                          int cols, float* outs, int threads) {
    if (!ref_has_avx2() || cols <= 0 || cols % 256 || p <= 0) return -1;
    if (type != REF_Q4_K && type != REF_Q6_K && type != REF_Q8_0) return -1;
    int blocks = cols / 256;
    long rb = ref_row_bytes(type, cols);
    int8_t* q8 = (int8_t*)malloc((size_t)p * cols);
    float* xsc = (float*)malloc(sizeof(float) * (size_t)p * blocks);
    int per = cols / 16;
    float* xsum = (float*)malloc(sizeof(float) * (size_t)p * per);
    for (int t = 0; t < p; t++) {
        const float* x = xs + (long)t * cols;
        ref_q8k_quantize(x, q8 + (long)t * cols, xsc + (long)t * blocks, blocks);
        if (type == REF_Q4_K) xsums32_avx2(x, xsum + (long)t * per, cols / 32);
        else if (type == REF_Q6_K) xsums16x32_avx2(x, xsum + (long)t * per, cols / 16);
    }
    if (threads <= 0) threads = ref_num_threads();
    if (threads > rows) threads = rows;
    if (threads < 1 || rows < threads * 8) threads = 1;
#pragma omp parallel num_threads(threads)
    {
        int nt = 1, id = 0;
#ifdef _OPENMP
        nt = omp_get_num_threads();
        id = omp_get_thread_num();
#endif
        int start = (int)((long)rows * id / nt), end = (int)((long)rows * (id + 1) / nt);
        /* matvecBatchQ8's 16-row tiles (kernels_amd64.go:565-578) */
        for (int t0 = start; t0 < end; t0 += 16) {
            int t1 = t0 + 16 < end ? t0 + 16 : end;
            for (int t = 0; t < p; t++) {
                const int8_t* q8t = q8 + (long)t * cols;
                const float* xst = xsc + (long)t * blocks;
                const float* sums = xsum + (long)t * per;
                float* out = outs + (long)t * rows;
                for (int r = t0; r < t1; r++) {
                    const uint8_t* w = data + (long)r * rb;
                    if (type == REF_Q4_K) out[r] = ref_q4k_dot_avx2(w, q8t, xst, sums, blocks);
                    else if (type == REF_Q6_K) out[r] = ref_q6k_dot_avx2(w, q8t, xst, sums, blocks);
                    else out[r] = ref_q8_0_dot_avx2(w, q8t, xst, blocks);
                }
            }
        }
    }
    free(q8);
    free(xsc);
    free(xsum);
    return 0;
}
