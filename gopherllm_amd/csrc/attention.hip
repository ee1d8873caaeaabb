// attention.hip -- HBM-resident F16 KV cache and GQA decode attention.
//
// Exact path (GLLM_ATTN_EXACT) evaluates the reference's two-pass attention
// in its float order (onlineAttentionGroup4F16 model.go:3527-3588 and the
// per-head onlineAttentionF16WithSink kv_f16.go:88-111, which perform the
// same operations):
//   s_t   = dotF32F16(q, k_t) * scale     8 fma lanes + tree (kernels_amd64.s:104-129)
//   M     = max_t s_t
//   w_t   = fastExpF32(s_t - M)           fastmath.go:47-77
//   denom = sum_t w_t                     sequential in t
//   out   = sum_t fma(w_t, v_t, out)      sequential in t (axpyF16, kernels_amd64.s:132-155)
//   out  *= 1/denom                       ScaleF32
// Split-K path (GLLM_ATTN_SPLITK) streams K/V tiles per (kv head, chunk)
// with an online-softmax merge; it agrees with the exact path to float
// rounding (not bitwise) and is the long-context fast path.
#include <algorithm>
#include <cstdlib>

#include "gllm_common.h"

namespace gllm {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// fastExpF32 (fastmath.go:47-77), operation for operation, without
// branches: the two range checks select the result, so a thread's several
// exps interleave instead of running one exec-masked block after another.
// Inside the range |t| < 128, so the clamp only keeps the int conversion
// defined for inputs the selects discard (a NaN still gives NaN).  The
// empty asm keeps the compiler from turning the first select back into a
// branch around the polynomial.
__device__ __forceinline__ float fast_exp(float x) {
    const float t = x * 1.44269502f;  // float32(1.4426950408889634)
    const float tc = fminf(fmaxf(t, -256.0f), 256.0f);
    const int k = (int)(tc + (tc >= 0.0f ? 0.5f : -0.5f));
    const float r = (float)((double)x - (double)k * 0.6931471805599453);
    const float p = 1.0f + r * (1.0f + r * (0.5f + r * ((float)(1.0 / 6) +
                    r * ((float)(1.0 / 24) + r * ((float)(1.0 / 120) + r * (float)(1.0 / 720))))));
    float v = p * __uint_as_float((uint32_t)(127 + k) << 23);
    asm volatile("" : "+v"(v));  // computed unconditionally: the selects stay selects
    return x > 88.02969f ? __int_as_float(0x7f800000) : x < -87.33654f ? 0.0f : v;
}

// fast_exp of N independent values, step by step across all of them so
// their dependent chains interleave (one wave per SIMD hides no latency
// otherwise); each value sees exactly fast_exp's operations.
template <int N>
__device__ __forceinline__ void fast_exp_n(const float (&x)[N], float (&y)[N]) {
    int k[N];
    float r[N];
#pragma unroll
    for (int i = 0; i < N; i++) {
        const float t = x[i] * 1.44269502f;
        const float tc = fminf(fmaxf(t, -256.0f), 256.0f);
        k[i] = (int)(tc + (tc >= 0.0f ? 0.5f : -0.5f));
    }
#pragma unroll
    for (int i = 0; i < N; i++) r[i] = (float)((double)x[i] - (double)k[i] * 0.6931471805599453);
#pragma unroll
    for (int i = 0; i < N; i++) {
        const float p = 1.0f + r[i] * (1.0f + r[i] * (0.5f + r[i] * ((float)(1.0 / 6) +
                        r[i] * ((float)(1.0 / 24) + r[i] * ((float)(1.0 / 120) + r[i] * (float)(1.0 / 720))))));
        y[i] = p * __uint_as_float((uint32_t)(127 + k[i]) << 23);
    }
#pragma unroll
    for (int i = 0; i < N; i++) asm volatile("" : "+v"(y[i]));
#pragma unroll
    for (int i = 0; i < N; i++)
        y[i] = x[i] > 88.02969f ? __int_as_float(0x7f800000) : x[i] < -87.33654f ? 0.0f : y[i];
}

// row[t] = fast_exp(row[t] - mx) for t = first, first + stride, ... < span,
// N positions at a time so that their chains interleave.
template <int N>
__device__ __forceinline__ void exp_row(float* row, int first, int stride, int span, float mx) {
    for (int t0 = first; t0 < span; t0 += N * stride) {
        float xv[N], ev[N];
#pragma unroll
        for (int i = 0; i < N; i++) xv[i] = row[min(t0 + i * stride, span - 1)] - mx;
        fast_exp_n(xv, ev);
#pragma unroll
        for (int i = 0; i < N; i++)
            if (t0 + i * stride < span) row[t0 + i * stride] = ev[i];
    }
}

}  // namespace gllm

struct gllm_hip_kv {
    int layers, kv_dim_k, kv_dim_v, max_len;
    uint16_t** k;  // host array of device pointers
    uint16_t** v;
    int device;
};

namespace gllm {

__global__ void kv_store_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                uint16_t* __restrict__ kd, uint16_t* __restrict__ vd, int nk,
                                int nv) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < nk) kd[i] = f32_to_f16_bits(k[i]);
    if (i < nv) vd[i] = f32_to_f16_bits(v[i]);
}

// --- exact path ------------------------------------------------------------

// Scores: one 8-lane group per (position, kv head); lane j owns elements
// 8i + j (i = 0..hd/8-1), the AVX2 lane j of dotF32F16AVX2, and computes the
// dots of all `kvmul` query heads sharing the row.  hd % 8 == 0, kvmul <= 8.
// blockIdx.y indexes the query token: token t attends start .. end0 + t
// (span0 + t positions), so one launch serves a whole causal prefill chunk.
__global__ __launch_bounds__(256) void attn_scores_kernel(const float* __restrict__ q,
                                                          const uint16_t* __restrict__ K,
                                                          int kv_dim, int n_kv, int kvmul, int hd,
                                                          int start, int span0, int span_max,
                                                          float scale, float* __restrict__ scores) {
    const int tok = blockIdx.y;
    const int span = span0 + tok;
    const int j = threadIdx.x & 7;
    const int item = blockIdx.x * 32 + (threadIdx.x >> 3);  // (t, g)
    if (item >= span * n_kv) return;
    const int g = item % n_kv, ti = item / n_kv;
    const int n_heads = n_kv * kvmul;
    const float* qt = q + (size_t)tok * n_heads * hd;
    float* st = scores + (size_t)tok * n_heads * span_max;
    const uint16_t* krow = K + (size_t)(start + ti) * kv_dim + g * hd;
    float acc[8];
    for (int h = 0; h < kvmul; h++) acc[h] = 0.0f;
    for (int i = 0; i < hd / 8; i++) {
        const float kv = f16_bits_to_f32(krow[8 * i + j]);
        for (int h = 0; h < kvmul; h++)
            acc[h] = fmaf(kv, qt[(size_t)(g * kvmul + h) * hd + 8 * i + j], acc[h]);
    }
    for (int h = 0; h < kvmul; h++) {
        const float sc = tree8(acc[h]);
        if (j == 0) st[(size_t)(g * kvmul + h) * span_max + ti] = sc * scale;
    }
}

// Softmax weights in place and the sequential denominator, one workgroup per
// (head, token).  Max and exp are order-free; the sum runs in position order.
__global__ __launch_bounds__(256) void attn_softmax_kernel(float* __restrict__ scores, int span0,
                                                           int span_max, float* __restrict__ inv_denom) {
    const int tok = blockIdx.y, h = blockIdx.x, n_heads = gridDim.x;
    const int span = span0 + tok;
    float* s = scores + ((size_t)tok * n_heads + h) * span_max;
    float m = -__int_as_float(0x7f800000);
    for (int i = threadIdx.x; i < span; i += 256) m = fmaxf(m, s[i]);
    // reference: first score then strict >; for NaN-free scores, the maximum
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    __shared__ float wm[4];
    if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
    __syncthreads();
    const float mx = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
    exp_row<8>(s, threadIdx.x, 256, span, mx);
    __syncthreads();
    if (threadIdx.x == 0) {
        float denom = 0.0f;
        for (int i = 0; i < span; i++) denom += s[i];
        // ScaleF32(out, 1/denom); the per-head path's `denom > 0` guard never
        // triggers since the largest weight is exactly 1.
        inv_denom[(size_t)tok * n_heads + h] = denom > 0.0f ? 1.0f / denom : 1.0f;
    }
}

// Values: one lane per (head, element) and token; out = fma(w_t, v_t, out)
// in position order, then out *= 1/denom.
__global__ __launch_bounds__(128) void attn_values_kernel(const float* __restrict__ weights,
                                                          const float* __restrict__ inv_denom,
                                                          const uint16_t* __restrict__ V,
                                                          int kv_dim, int kvmul, int vd, int start,
                                                          int span0, int span_max,
                                                          float* __restrict__ out) {
    const int h = blockIdx.x, tok = blockIdx.y, n_heads = gridDim.x;
    const int d = threadIdx.x;
    if (d >= vd) return;
    const int span = span0 + tok;
    const int g = h / kvmul;
    const float* w = weights + ((size_t)tok * n_heads + h) * span_max;
    const uint16_t* vcol = V + (size_t)start * kv_dim + g * vd + d;
    float acc = 0.0f;
    int t = 0;
    for (; t + 4 <= span; t += 4) {
        const float v0 = f16_bits_to_f32(vcol[(size_t)t * kv_dim]);
        const float v1 = f16_bits_to_f32(vcol[(size_t)(t + 1) * kv_dim]);
        const float v2 = f16_bits_to_f32(vcol[(size_t)(t + 2) * kv_dim]);
        const float v3 = f16_bits_to_f32(vcol[(size_t)(t + 3) * kv_dim]);
        acc = fmaf(w[t], v0, acc);
        acc = fmaf(w[t + 1], v1, acc);
        acc = fmaf(w[t + 2], v2, acc);
        acc = fmaf(w[t + 3], v3, acc);
    }
    for (; t < span; t++) acc = fmaf(w[t], f16_bits_to_f32(vcol[(size_t)t * kv_dim]), acc);
    out[((size_t)tok * n_heads + h) * vd + d] = acc * inv_denom[(size_t)tok * n_heads + h];
}

// Exact path for head_dim 128 in two launches that keep the three-kernel
// arithmetic (and so its results) while spreading the work over many CUs:
//   attn_scores128_kernel  one workgroup per (kv head, 32-position chunk,
//       query token); the eight lanes of dotF32F16AVX2 (sequential fma
//       chains over elements 8i + j) of a (head, position) run in two
//       threads, lanes 0-3 and 4-7, which then join for the 8->4->2->1
//       tree, then * scale.  Scores go to a global scratch row per
//       (token, head).
//   attn_softmax_values_kernel  one workgroup per (query head, token): the
//       row is read into LDS, max, fastExpF32(s - max), the denominator
//       summed in position order by one thread, then one thread per element
//       runs out = fma(w_t, v_t, out) in position order over V tiles staged
//       through LDS (prefetched from kernel entry), and * 1/denom.
constexpr int kFusedHD = 128;
constexpr int kScoreChunk = 32;   // positions per scores workgroup
constexpr int kVTile = 64;        // positions per staged V tile (16 KB)
constexpr int kVPrefetch = 4;     // tiles in flight per thread (registers)
constexpr int kSmaxSpan = 6144;   // longest span the softmax/values kernel keeps in LDS, several tokens
// One token (four workgroups per head, 32-element slices): the score row and
// two V tiles fit the 160 KB of LDS a gfx950 workgroup may use up to here.
constexpr int kSmaxSpan1 = 36864;

// RoPE for one decode token folded into the scores launch (rope != null,
// one token, position `end` read from d_end): applyPreparedRope on q
// (model.go:3051-3093, interleaved pairs, same operations as rope_kv_kernel)
// as each workgroup stages its query heads, and the workgroup whose chunk holds
// the new position rotates the raw k row, rounds it to f16 and stores it and
// the v row in the cache, using the stored f16 values for its own dot.
struct AttnRope {
    const float* sin_tab;  // [max_len][hd/2]
    const float* cos_tab;
    const float* k;        // raw (unrotated) k of the token, n_kv * hd
    const float* v;
    uint16_t* kc;          // this layer's caches
    uint16_t* vc;
    const float* cur;      // optional: the current position's sin row then cos row
};

constexpr int kEagerRows = 2048;  // rows loaded before a device-side position is read
// CM: also write each chunk's maximum per head to cmax (the long-span values
// kernel's input; the other values kernels take the maximum themselves)
template <bool CM>
__global__ __launch_bounds__(256) void attn_scores128_kernel(
    const float* __restrict__ q, const uint16_t* K, const uint16_t* V, int kv_dim, int n_kv,
    int kvmul, int start, int span0, int span_max, float scale, float* __restrict__ scores,
    const int* __restrict__ d_end, AttnRope rope, int touch, float* __restrict__ cmax) {
    constexpr int pairs = kFusedHD / 2;
    __shared__ __align__(16) float qs[4 * kFusedHD];
    __shared__ __align__(16) uint16_t kcur[kFusedHD];
    // the chunk's K rows, [16-byte piece][row]: copied once per workgroup
    // (two 1 KB copies per wave), read by every head's threads of a row
    __shared__ __align__(16) uint8_t kst[kFusedHD / 8][kScoreChunk][16];
    const int g = blockIdx.x, chunk = blockIdx.y, tok = blockIdx.z;
    // A captured step's launch covers the whole span cap: chunks past the
    // first kEagerRows positions read the position first and leave before
    // loading anything when they lie past the span.
    // (near chunks wait for no argument load: the empty asm keeps the
    // compiler from folding the pointer test into one flag ahead of the
    // branch)
    if (chunk * kScoreChunk >= kEagerRows) {  // uniform
        const int* de = d_end;
        asm volatile("" : "+s"(de));
        if (de && chunk * kScoreChunk >= __builtin_amdgcn_readfirstlane(*de) - start + 1 + tok)
            return;  // the whole workgroup
    }
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n_heads = n_kv * kvmul;
    const float* qg = q + ((size_t)tok * n_heads + (size_t)g * kvmul) * kFusedHD;
    // Everything that does not need the position goes out before it is read:
    // the K copies (wave wv, copy u: lane l copies row l % 32 of piece
    // 4 wv + 2 u + l / 32, rows clamped to span_max - 1, inside the cache;
    // rows past the span are copied and never read), then this thread's q
    // pair and, when the caller uploads them, the current RoPE rows.
    {
        const int row = min(chunk * kScoreChunk + (lane & 31), span_max - 1);
        const uint16_t* krow = K + (size_t)(start + row) * kv_dim + (size_t)g * kFusedHD + 8 * (lane >> 5);
#pragma unroll
        for (int u = 0; u < 2; u++)
            lds_copy16(krow + 8 * (4 * wv + 2 * u), lds_addr(&kst[4 * wv + 2 * u][0][0]));
    }
    // one dword of each 128-byte line of the chunk's V rows of this kv head
    // (lane l: row l / 2, line l % 2; the four waves touch the same lines):
    // workgroup (g, chunk) runs on XCD g % 8, as do the values launch's
    // workgroups of kv head g, which then find these lines in that XCD's L2.
    // touch == 0 (spans whose K and V pass through more than an L2): every
    // lane reads the chunk's first line, which the K copies fetch anyway.
    uint32_t vtouch;
    {
        const int row = min(chunk * kScoreChunk + (touch ? lane >> 1 : 0), span_max - 1);
        vtouch = *(const uint32_t*)((touch ? V : K) + (size_t)(start + row) * kv_dim +
                                    (size_t)g * kFusedHD + (touch ? 64 * (lane & 1) : 0));
    }
    // (unconditional loads, clamped or from a dummy row: a load under a
    // branch is waited for at the branch's end, behind the copies)
    const bool qthr = tid < kvmul * pairs;  // kvmul <= 4: one q pair per thread
    const int pr = tid % pairs;
    const float2 qv = *(const float2*)(qg + 2 * (qthr ? tid : 0));
    const float* rc = rope.cur ? rope.cur : qg;
    float sn = rc[pr], cs = rc[pairs + pr];
    if (d_end) span0 = *d_end - start + 1;  // position read on the device (graph replay)
    const int span = span0 + tok;
    if (chunk * kScoreChunk >= span) {  // uniform
        wait_vmem_le<0>();  // the copies land before the workgroup's LDS is released
        return;
    }
    const int tcur = span - 1;  // the new position (rope mode: one token)
    const bool has_cur = rope.sin_tab && tcur / kScoreChunk == chunk;
    if (rope.sin_tab) {
        // applyPreparedRope on q; the workgroup holding the new position
        // also rotates its k row (kept in kcur) and stores it and the v row
        const int pos = start + tcur;
        if (!rope.cur) {
            sn = rope.sin_tab[(size_t)pos * pairs + pr];
            cs = rope.cos_tab[(size_t)pos * pairs + pr];
        }
        if (qthr) {
            qs[2 * tid] = qv.x * cs - qv.y * sn;
            qs[2 * tid + 1] = qv.x * sn + qv.y * cs;
        }
        if (has_cur && tid < pairs) {
            const float* e = rope.k + (size_t)g * kFusedHD + 2 * tid;
            const float v0 = e[0], v1 = e[1];
            const uint16_t r0 = f32_to_f16_bits(v0 * cs - v1 * sn);
            const uint16_t r1 = f32_to_f16_bits(v0 * sn + v1 * cs);
            kcur[2 * tid] = r0;
            kcur[2 * tid + 1] = r1;
            uint16_t* kc = rope.kc + (size_t)pos * kv_dim + (size_t)g * kFusedHD + 2 * tid;
            kc[0] = r0;
            kc[1] = r1;
        } else if (has_cur && tid < 2 * pairs) {
            const int i = tid - pairs;
            const float* vr = rope.v + (size_t)g * kFusedHD + 2 * i;
            uint16_t* vc = rope.vc + (size_t)pos * kv_dim + (size_t)g * kFusedHD + 2 * i;
            vc[0] = f32_to_f16_bits(vr[0]);
            vc[1] = f32_to_f16_bits(vr[1]);
        }
    } else {
        for (int i = tid; i < kvmul * kFusedHD; i += 256) qs[i] = qg[i];
    }
    wait_vmem_le<0>();  // this wave's K copies (and the V touch) have landed
    __syncthreads();
    if (span < 0) scores[vtouch & 0xffu] = 0.0f;  // keeps the V touch (span > 0 here)
    // wave h = query head h of the group; lanes l and l + 32 share position
    // l and run the chains j = 0..3 and 4..7 (elements 8c + j, c in order)
    const int h = wv, half = lane >> 5, t = chunk * kScoreChunk + (lane & 31);
    if (h >= kvmul) return;  // uniform
    // the new position's row comes from kcur: one stride per lane
    const bool cur = has_cur && t == tcur;
    const uint8_t* kb = cur ? (const uint8_t*)kcur + 8 * half : &kst[0][lane & 31][8 * half];
    const int kstride = cur ? 16 : kScoreChunk * 16;
    uint2 kr[kFusedHD / 8];
#pragma unroll
    for (int c = 0; c < kFusedHD / 8; c++) kr[c] = *(const uint2*)(kb + c * kstride);
    const float* qh = qs + h * kFusedHD + 4 * half;
    float acc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) acc[j] = 0.0f;
#pragma unroll
    for (int c = 0; c < kFusedHD / 8; c++) {
        const float4 qa = *(const float4*)(qh + 8 * c);
        acc[0] = fmaf(f16_bits_to_f32(kr[c].x & 0xffffu), qa.x, acc[0]);
        acc[1] = fmaf(f16_bits_to_f32(kr[c].x >> 16), qa.y, acc[1]);
        acc[2] = fmaf(f16_bits_to_f32(kr[c].y & 0xffffu), qa.z, acc[2]);
        acc[3] = fmaf(f16_bits_to_f32(kr[c].y >> 16), qa.w, acc[3]);
    }
    // chains 4..7 from the partner lane: (y0 + y4, ...), then the tree
    float o[4];
#pragma unroll
    for (int j = 0; j < 4; j++) o[j] = __shfl_xor(acc[j], 32);
    float sv = -__int_as_float(0x7f800000);
    if (half == 0 && t < span) {
        const float a0 = acc[0] + o[0], a1 = acc[1] + o[1];
        const float a2 = acc[2] + o[2], a3 = acc[3] + o[3];
        sv = ((a0 + a1) + (a2 + a3)) * scale;
        scores[((size_t)tok * n_heads + (size_t)g * kvmul + h) * span_max + t] = sv;
    }
    // the chunk's maximum per head, for the long-span values kernel (fmaxf
    // over the same values: the row's maximum is the chunks' maximum)
    if (CM) {
        const float mc = wave_max(sv);
        if (lane == 0) cmax[((size_t)tok * n_heads + (size_t)g * kvmul + h) * gridDim.y + chunk] = mc;
    }
}

// DS workgroups share one (query head, token): workgroup slice c runs the
// value chains of elements c*DW .. c*DW+DW-1 (DW = 128 / DS) and stages only
// that slice of each V row, so a decode token spreads its V stream over
// n_heads * DS compute units.  Every slice recomputes the same max, weights
// and sequential denominator, so each chain sees the same operands in the
// same position order whatever DS is.
// (four waves per SIMD are plenty: the 128-VGPR budget keeps the V prefetch
// registers out of scratch)
template <int DS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 4))) void attn_softmax_values_kernel(
    const float* __restrict__ scores, const uint16_t* __restrict__ V, int kv_dim, int kvmul,
    int start, int span0, int span_max, float* __restrict__ out, const int* __restrict__ d_end) {
    static_assert(DS == 1 || DS == 2 || DS == 4, "slices of 128, 64 or 32 elements");
    constexpr int DW = kFusedHD / DS;   // elements per workgroup
    constexpr int U = 4 / DS;           // 16-byte pieces per thread per tile row
    constexpr int P = DS == 1 ? kVPrefetch : 8;  // tiles in flight (P * U <= 16 registers of 16 bytes)
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int h = blockIdx.x / DS, slice = blockIdx.x % DS, tok = blockIdx.y;
    const int n_heads = gridDim.x / DS;
    const int tid = threadIdx.x;
    const int g = h / kvmul;
    const int wlen = (span_max + 3) & ~3;             // keeps the V tiles 16-byte aligned
    float* w = lds;                                   // [wlen]
    float* red = w + wlen;                            // [8]
    uint16_t* vt = (uint16_t*)(red + 8);              // [2][kVTile][DW] f16
    // V prefetch first: thread (position lp, piece lc) owns U * 16 bytes of
    // the slice of a tile row, P tiles ahead.  Loads are unconditional and
    // clamped to span_max - 1 (rows start .. start + span_max - 1 lie inside
    // the cache), so they neither wait for the device-side position nor sit
    // under a branch (which would make the compiler's vmcnt waits drain the
    // prefetch); rows past the span are never read from LDS.
    const uint16_t* Vg = V + (size_t)start * kv_dim + (size_t)g * kFusedHD + slice * DW;
    const int lp = tid >> 2, lc = tid & 3;
    u32x4 pre[P][U];
    auto fetch = [&](int i, u32x4 (&pr)[U]) __attribute__((always_inline)) {
        const u32x4* src = (const u32x4*)(Vg + (size_t)min(i * kVTile + lp, span_max - 1) * kv_dim + 8 * U * lc);
#pragma unroll
        for (int u = 0; u < U; u++) pr[u] = src[u];
    };
#pragma unroll
    for (int q = 0; q < P; q++) fetch(q, pre[q]);
    if (d_end) span0 = *d_end - start + 1;
    const int span = span0 + tok;
    const int ntiles = (span + kVTile - 1) / kVTile;
    const float* srow = scores + ((size_t)tok * n_heads + h) * span_max;
    float m = -__int_as_float(0x7f800000);
    for (int t = tid; t < span; t += 256) {
        const float v = srow[t];
        w[t] = v;
        m = fmaxf(m, v);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    const float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    exp_row<8>(w, tid, 256, span, mx);
    // (the first tile barrier orders the exp writes before their readers)
    // values: threads 0..DW-1 own one element each; the first thread of the
    // next wave (a wave that otherwise only stages V) sums the denominator
    // tile by tile, in position order
    constexpr int kSummer = (DW + 63) / 64 * 64;
    const int d = tid;
    const bool chain = tid < DW;
    const bool summer = tid == kSummer;
    float acc = 0.0f, denom = 0.0f;
    // one V tile: stage it from registers, refill those registers P tiles
    // ahead, then run the chains over it
    auto tile = [&](int it, u32x4 (&pr)[U]) __attribute__((always_inline)) {
        uint16_t* buf = vt + (size_t)(it & 1) * kVTile * DW;
        u32x4* dst = (u32x4*)(buf + lp * DW + 8 * U * lc);
#pragma unroll
        for (int u = 0; u < U; u++) dst[u] = pr[u];
        fetch(it + P, pr);
        wait_lgkm0();
        lds_barrier();
        const int base = it * kVTile;
        const int n = max(0, min(kVTile, span - base));
        if (chain) {
            if (n == kVTile) {
                // the whole tile's operands first (one LDS round trip), then
                // the chain: w four positions per broadcast read
                uint16_t vb[kVTile];
                float4 wq[kVTile / 4];
#pragma unroll
                for (int u = 0; u < kVTile / 4; u++) wq[u] = *(const float4*)&w[base + 4 * u];
#pragma unroll
                for (int u = 0; u < kVTile; u++) vb[u] = buf[u * DW + d];
#pragma unroll
                for (int u = 0; u < kVTile / 4; u++) {
                    acc = fmaf(wq[u].x, f16_bits_to_f32(vb[4 * u]), acc);
                    acc = fmaf(wq[u].y, f16_bits_to_f32(vb[4 * u + 1]), acc);
                    acc = fmaf(wq[u].z, f16_bits_to_f32(vb[4 * u + 2]), acc);
                    acc = fmaf(wq[u].w, f16_bits_to_f32(vb[4 * u + 3]), acc);
                }
            } else {
                for (int p = 0; p < n; p++)
                    acc = fmaf(w[base + p], f16_bits_to_f32(buf[p * DW + d]), acc);
            }
        } else if (summer) {
            int p = 0;
            for (; p + 16 <= n; p += 16) {
                float wb[16];
#pragma unroll
                for (int u = 0; u < 16; u++) wb[u] = w[base + p + u];
#pragma unroll
                for (int u = 0; u < 16; u++) denom = denom + wb[u];
            }
            for (; p < n; p++) denom = denom + w[base + p];
        }
    };
    // whole groups of P tiles, unconditionally (a branch around a tile makes
    // the compiler's vmcnt waits drain the prefetch): tiles past the span
    // stage clamped rows nobody reads and run no chain steps
    for (int it0 = 0; it0 < ntiles; it0 += P) {
#pragma unroll
        for (int q = 0; q < P; q++) tile(it0 + q, pre[q]);
    }
    if (summer) red[4] = denom > 0.0f ? 1.0f / denom : 1.0f;
    __syncthreads();
    if (chain) out[((size_t)tok * n_heads + h) * kFusedHD + slice * DW + d] = acc * red[4];
}


// One decode token over a long span (past what attn_values_dec_kernel keeps
// in LDS, up to kLongSpan): the arithmetic of attn_softmax_values_kernel<4>
// (so the same bits), with V staged transposed.  Workgroup = (query head,
// 32-element slice).  The score row sits in LDS; its maximum is taken
// before the first step, and each step's 128 weights are exponentiated in
// place by the staging waves (lanes 0-31, one position each) just before
// the step's barrier, so the chains start once the maximum is known.  V
// streams in steps of two 64-position tiles, kLongP steps in flight.  A
// staging lane (waves 1, 2, 3, 5) loads one element pair of eight positions
// (eight dwords), splits them into the two elements' eight-position runs
// (v_perm) and writes each run with one ds_write_b128, element-major
// (vt[e][t], rows padded to 72 halves; two pairs of tiles alternate, one
// barrier per step).  Wave 0 only runs the chains, eight positions of its
// element per ds_read_b128 and the weights as broadcast quads, three groups
// of eight positions ahead: lanes 0-31 the 32 value chains, lane 32 the
// denominator, as fma(w, 1.0, denom) over a row of ones that every tile
// carries (w * 1 is exact, so each step rounds as denom + w does).  Wave 4,
// placed on wave 0's SIMD, only streams the raw score row (two loads and two
// LDS writes a step): heavier work there slows the chain.
constexpr int kLongThreads = 384;  // wave 0: the chains; waves 1-3, 5: staging
constexpr int kLongP = 8;        // steps (two tiles each) in flight per staging lane
constexpr int kLongRow = 72;     // halves per element row of a staged tile (64 + 8 padding)
constexpr int kLongRows = 33;    // rows per staged tile: 32 elements and the row of ones
constexpr int kLongSpan = 32768;
constexpr int kTouchSpan = 8192;  // longest span whose V the scores launch touches
static size_t long_lds_bytes(int span_max) {
    return ((size_t)((span_max + 3) & ~3) + 8) * 4 + 4 * (size_t)kLongRows * kLongRow * 2;
}

__global__ __launch_bounds__(kLongThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void attn_values_long_kernel(
    const float* __restrict__ scores, const float* __restrict__ cmax, const uint16_t* __restrict__ V,
    int kv_dim, int kvmul, int start, int span0, int span_max, float* __restrict__ out,
    const int* __restrict__ d_end) {
    constexpr int DW = 32, T = kVTile, P = kLongP, TR = kLongRows * kLongRow;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    // Workgroup b runs on XCD b % 8.  The (kv head g, pair of quarters, q
    // head of the group, quarter) items go out in runs of gridDim.x / 8 per
    // XCD, so the 2 * kvmul workgroups that read one 128-byte V line share
    // an L2, and kv head g lands on XCD g, where the scores launch touched
    // its lines.
    const int nb = gridDim.x, b = blockIdx.x;
    const int item = nb % 8 == 0 ? (b % 8) * (nb / 8) + b / 8 : b;
    const int gp = (item >> 1) / kvmul;
    const int g = gp >> 1, slice = 2 * (gp & 1) + (item & 1);
    const int h = g * kvmul + (item >> 1) % kvmul;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wlen = (span_max + 3) & ~3;
    float* w = lds;                          // [wlen]
    float* red = w + wlen;                   // [8]: the six waves' maxima
    uint16_t* vt = (uint16_t*)(red + 8);     // [4 tiles][kLongRows][kLongRow]
    // staging lane: stager si covers positions 32 si .. 32 si + 31 of a step,
    // lane (position group pg, element pair c) eight of them, rows clamped to
    // span_max - 1 (inside the cache)
    const bool stager = wave != 0 && wave != 4;
    const int si = wave < 4 ? wave - 1 : 3;
    const int c = lane & 15, pg = lane >> 4;
    const uint16_t* Vg = V + (size_t)start * kv_dim + (size_t)g * kFusedHD + slice * DW + 2 * c;
    const int sp0 = 32 * si + 8 * pg;  // first position of the lane's run within a step
    uint32_t pre[P][8];
    auto fetch = [&](int st, uint32_t (&r)[8]) __attribute__((always_inline)) {
        const int p0 = 2 * st * T + sp0;
#pragma unroll
        for (int j = 0; j < 8; j++)
            r[j] = *(const uint32_t*)(Vg + (size_t)min(p0 + j, span_max - 1) * kv_dim);
    };
    if (stager) {
#pragma unroll
        for (int q = 0; q < P; q++) fetch(q, pre[q]);
    }
    // wave 4 streams the raw score row into LDS one step ahead of the exps:
    // lane l holds positions 2l and 2l + 1 of a step, P steps in flight
    // (spre[k] holds the steps st == k mod P; rows clamped to span_max - 1)
    const float* srow = scores + (size_t)h * span_max;
    float spre[P][2];
    auto sfetch = [&](int st, float (&r)[2]) __attribute__((always_inline)) {
        const int p0 = 2 * st * T + 2 * lane;
        r[0] = srow[min(p0, span_max - 1)];
        r[1] = srow[min(p0 + 1, span_max - 1)];
    };
    if (wave == 4) {
#pragma unroll
        for (int q = 0; q < P; q++) sfetch(q, spre[q]);
    }
    if (d_end) span0 = *d_end - start + 1;
    const int span = min(span0, span_max);
    const int nsteps = (span + 2 * T - 1) / (2 * T);
    auto sput = [&](int st, const float (&r)[2]) __attribute__((always_inline)) {
        const int p0 = 2 * st * T + 2 * lane;
        if (p0 < span) w[p0] = r[0];
        if (p0 + 1 < span) w[p0 + 1] = r[1];
    };
    // the row's maximum from the scores launch's chunk maxima, read by waves
    // 0 and 4 (no V prefetch queued ahead of their loads; chunks clamped to
    // the span's last: the duplicates leave the maximum unchanged)
    float m = -__int_as_float(0x7f800000);
    if (wave == 0 || wave == 4) {
        const int nck = (span + kScoreChunk - 1) / kScoreChunk;
        const float* crow = cmax + (size_t)h * ((span_max + kScoreChunk - 1) / kScoreChunk);
        for (int c0 = (wave == 0 ? 0 : 64) + lane; c0 < nck; c0 += 128 * 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = crow[min(c0 + u * 128, nck - 1)];
#pragma unroll
            for (int u = 0; u < 8; u++) m = fmaxf(m, v[u]);
        }
        m = wave_max(m);
    }
    if (lane == 0) red[wave] = m;
    if (wave == 4) {  // the row of ones in each of the four tiles; step 0's scores
#pragma unroll
        for (int k = 0; k < 4; k++) vt[k * TR + DW * kLongRow + lane] = (uint16_t)0x3C00;
        sput(0, spre[0]);
        sfetch(P, spre[0]);
    }
    __syncthreads();
    const float mx = fmaxf(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])), fmaxf(red[4], red[5]));
    // (a step's barrier orders its exp writes before the chain's reads)
    if (wave == 0) {
        // lanes 0-31 the value chains, lane 32 the denominator; lanes 33-63
        // repeat lane 32's row so the wave runs one uniform path
        const uint16_t* vrow0 = vt + min(tid, DW) * kLongRow;
        float acc = 0.0f;
        // The chains in position order, groups of eight positions read three
        // groups ahead in one ring over every whole step (two tiles,
        // positions 128 st .. 128 st + 127): two groups before a step's
        // end the wave waits for its reads, takes the next step's barrier
        // (the staging waves may then refill this step's pair) and reads
        // the next step's first groups under this step's last 24 FMAs.  As
        // many barriers as the staging waves take (nsteps rounded up to
        // whole groups of P); a partial last step runs position by position.
        const int nbar = (nsteps + P - 1) / P * P;
        const int nfull = span / (2 * T);
        constexpr int NG = 2 * T / 8;  // groups of eight positions per step
        struct Grp {
            u32x4 v;
            float4 a, b;
        };
        auto ld = [&](Grp& r, int st, int u) __attribute__((always_inline)) {
            const uint16_t* vrow = vrow0 + (size_t)(st & 1) * 2 * TR;
            const int base = 2 * st * T;
            r.v = *(const u32x4*)(vrow + (u >> 3) * TR + 8 * (u & 7));
            r.a = *(const float4*)&w[base + 8 * u];
            r.b = *(const float4*)&w[base + 8 * u + 4];
        };
        auto run = [&](const Grp& r) __attribute__((always_inline)) {
            acc = fmaf(r.a.x, f16_bits_to_f32(r.v.x & 0xffffu), acc);
            acc = fmaf(r.a.y, f16_bits_to_f32(r.v.x >> 16), acc);
            acc = fmaf(r.a.z, f16_bits_to_f32(r.v.y & 0xffffu), acc);
            acc = fmaf(r.a.w, f16_bits_to_f32(r.v.y >> 16), acc);
            acc = fmaf(r.b.x, f16_bits_to_f32(r.v.z & 0xffffu), acc);
            acc = fmaf(r.b.y, f16_bits_to_f32(r.v.z >> 16), acc);
            acc = fmaf(r.b.z, f16_bits_to_f32(r.v.w & 0xffffu), acc);
            acc = fmaf(r.b.w, f16_bits_to_f32(r.v.w >> 16), acc);
        };
        Grp ring[4];
        // one whole step; the last one takes no barrier inside and reads
        // nothing ahead (no branch inside a step: the compiler would sink
        // the chain below it and issue every read first)
        auto whole = [&](int st, const bool last) __attribute__((always_inline)) {
#pragma unroll
            for (int u = 0; u < NG; u++) {
                if (u + 3 < NG) ld(ring[(u + 3) & 3], st, u + 3);
                if (u == NG - 2 && !last) {
                    wait_lgkm0();
                    lds_barrier();  // barrier st + 1
                    ld(ring[0], st + 1, 0);
                    ld(ring[1], st + 1, 1);
                }
                if (u == NG - 1 && !last) ld(ring[2], st + 1, 2);
                __builtin_amdgcn_sched_barrier(0);
                run(ring[u & 3]);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        if (nbar > 0) lds_barrier();  // barrier 0: step 0 staged
        if (nfull > 0) {
            ld(ring[0], 0, 0);
            ld(ring[1], 0, 1);
            ld(ring[2], 0, 2);
            for (int st = 0; st < nfull - 1; st++) whole(st, false);
            whole(nfull - 1, true);
            if (nfull < nbar) lds_barrier();  // barrier nfull
        }
        if (nfull < nsteps) {  // the partial last step (its barrier is taken)
            const uint16_t* vrow = vrow0 + (size_t)(nfull & 1) * 2 * TR;
            const int base = 2 * nfull * T;
            for (int p = 0; p < span - base; p++)
                acc = fmaf(w[base + p], f16_bits_to_f32(vrow[(p / T) * TR + p % T]), acc);
        }
        for (int b = min(nfull + 1, nbar); b < nbar; b++) lds_barrier();
        const float denom = __shfl(acc, DW);
        const float inv = denom > 0.0f ? 1.0f / denom : 1.0f;
        if (tid < DW) out[(size_t)h * kFusedHD + slice * DW + tid] = acc * inv;
    } else if (stager) {
        // one step: split the eight dwords into the two elements' runs, write
        // them, refill the registers P steps ahead, exponentiate the step's
        // weights (lane l < 32 of stager si: position 32 si + l of the step,
        // fast_exp as exp_row applies it), barrier; whole groups of
        // P steps (a branch around a step would make the compiler's vmcnt
        // waits drain the prefetch): steps past the span stage clamped rows
        // that no chain reads
        uint16_t* dst0 = vt + ((sp0 >> 6) * kLongRows + 2 * c) * kLongRow + (sp0 & 63);
        auto step = [&](int st, uint32_t (&r)[8]) __attribute__((always_inline)) {
            uint16_t* dst = dst0 + (size_t)(st & 1) * 2 * TR;
            const int pw = 2 * st * T + 32 * si + (lane & 31);
            const float sv = w[min(pw, span - 1)];
            uint4 lo, hi;
            lo.x = __builtin_amdgcn_perm(r[1], r[0], 0x05040100u);
            lo.y = __builtin_amdgcn_perm(r[3], r[2], 0x05040100u);
            lo.z = __builtin_amdgcn_perm(r[5], r[4], 0x05040100u);
            lo.w = __builtin_amdgcn_perm(r[7], r[6], 0x05040100u);
            hi.x = __builtin_amdgcn_perm(r[1], r[0], 0x07060302u);
            hi.y = __builtin_amdgcn_perm(r[3], r[2], 0x07060302u);
            hi.z = __builtin_amdgcn_perm(r[5], r[4], 0x07060302u);
            hi.w = __builtin_amdgcn_perm(r[7], r[6], 0x07060302u);
            *(uint4*)dst = lo;
            *(uint4*)(dst + kLongRow) = hi;
            fetch(st + P, r);
            const float e = fast_exp(sv - mx);
            if (lane < 32 && pw < span) w[pw] = e;
            wait_lgkm0();
            lds_barrier();
        };
        for (int s0 = 0; s0 < nsteps; s0 += P) {
#pragma unroll
            for (int q = 0; q < P; q++) step(s0 + q, pre[q]);
        }
    } else {
        // wave 4: before barrier st, step st + 1's raw scores into LDS (the
        // staging waves exponentiate them after barrier st), then the
        // registers refilled P steps ahead; whole groups of P steps, as the
        // staging waves run
        for (int s0 = 0; s0 < nsteps; s0 += P) {
#pragma unroll
            for (int q = 0; q < P; q++) {
                sput(s0 + q + 1, spre[(q + 1) % P]);
                sfetch(s0 + q + 1 + P, spre[(q + 1) % P]);
                wait_lgkm0();
                lds_barrier();
            }
        }
    }
}

template <int DS>
static size_t smax_lds_bytes(int span_max) {
    return ((size_t)((span_max + 3) & ~3) + 8) * 4 + 2 * (size_t)kVTile * (kFusedHD / DS) * 2;
}

// The value chain of one element over a staged span: out = fma(w_t, v_t,
// out) in position order from 0, eight positions per ds_read_b128 of the
// element's vt row and two of the weight row, in a ring of four groups read
// three ahead (reads past the span stay inside the rows: they hold at least
// span + 56 positions).
__device__ __forceinline__ float dec_value_chain(const uint16_t* vrow, const float* wrow, int span) {
    float acc = 0.0f;
    struct Grp {
        uint4 v;
        float4 a, b;
    };
    auto ld = [&](Grp& r, int t) __attribute__((always_inline)) {
        r.v = *(const uint4*)(vrow + t);
        r.a = *(const float4*)(wrow + t);
        r.b = *(const float4*)(wrow + t + 4);
    };
    auto run = [&](const Grp& r) __attribute__((always_inline)) {
        acc = fmaf(r.a.x, f16_bits_to_f32(r.v.x & 0xffffu), acc);
        acc = fmaf(r.a.y, f16_bits_to_f32(r.v.x >> 16), acc);
        acc = fmaf(r.a.z, f16_bits_to_f32(r.v.y & 0xffffu), acc);
        acc = fmaf(r.a.w, f16_bits_to_f32(r.v.y >> 16), acc);
        acc = fmaf(r.b.x, f16_bits_to_f32(r.v.z & 0xffffu), acc);
        acc = fmaf(r.b.y, f16_bits_to_f32(r.v.z >> 16), acc);
        acc = fmaf(r.b.z, f16_bits_to_f32(r.v.w & 0xffffu), acc);
        acc = fmaf(r.b.w, f16_bits_to_f32(r.v.w >> 16), acc);
    };
    Grp r0, r1, r2, r3;
    int t0 = 0;
    ld(r0, 0);
    ld(r1, 8);
    ld(r2, 16);
    for (; t0 + 32 <= span; t0 += 32) {
        ld(r3, t0 + 24);
        __builtin_amdgcn_sched_barrier(0);
        run(r0);
        __builtin_amdgcn_sched_barrier(0);
        ld(r0, t0 + 32);
        __builtin_amdgcn_sched_barrier(0);
        run(r1);
        __builtin_amdgcn_sched_barrier(0);
        ld(r1, t0 + 40);
        __builtin_amdgcn_sched_barrier(0);
        run(r2);
        __builtin_amdgcn_sched_barrier(0);
        ld(r2, t0 + 48);
        __builtin_amdgcn_sched_barrier(0);
        run(r3);
        __builtin_amdgcn_sched_barrier(0);
    }
    // r0, r1, r2 hold groups t0, t0 + 8, t0 + 16
    if (t0 + 8 <= span) {
        run(r0);
        t0 += 8;
        if (t0 + 8 <= span) {
            run(r1);
            t0 += 8;
            if (t0 + 8 <= span) {
                run(r2);
                t0 += 8;
            }
        }
    }
    for (int t = t0; t < span; t++) acc = fmaf(wrow[t], f16_bits_to_f32(vrow[t]), acc);
    return acc;
}

// The softmax denominator of one weight row: denom + w_t in position order
// from 0, with the value chain's ring (two quads per group, three groups
// ahead), so that it keeps pace with the chains.
__device__ __forceinline__ float dec_denominator(const float* wrow, int span) {
    float den = 0.0f;
    struct Grp {
        float4 a, b;
    };
    auto ld = [&](Grp& r, int t) __attribute__((always_inline)) {
        r.a = *(const float4*)(wrow + t);
        r.b = *(const float4*)(wrow + t + 4);
    };
    auto run = [&](const Grp& r) __attribute__((always_inline)) {
        den = den + r.a.x;
        den = den + r.a.y;
        den = den + r.a.z;
        den = den + r.a.w;
        den = den + r.b.x;
        den = den + r.b.y;
        den = den + r.b.z;
        den = den + r.b.w;
    };
    Grp r0, r1, r2, r3;
    int t0 = 0;
    ld(r0, 0);
    ld(r1, 8);
    ld(r2, 16);
    for (; t0 + 32 <= span; t0 += 32) {
        ld(r3, t0 + 24);
        __builtin_amdgcn_sched_barrier(0);
        run(r0);
        __builtin_amdgcn_sched_barrier(0);
        ld(r0, t0 + 32);
        __builtin_amdgcn_sched_barrier(0);
        run(r1);
        __builtin_amdgcn_sched_barrier(0);
        ld(r1, t0 + 40);
        __builtin_amdgcn_sched_barrier(0);
        run(r2);
        __builtin_amdgcn_sched_barrier(0);
        ld(r2, t0 + 48);
        __builtin_amdgcn_sched_barrier(0);
        run(r3);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (t0 + 8 <= span) {
        run(r0);
        t0 += 8;
        if (t0 + 8 <= span) {
            run(r1);
            t0 += 8;
            if (t0 + 8 <= span) {
                run(r2);
                t0 += 8;
            }
        }
    }
    for (int t = t0; t < span; t++) den = den + wrow[t];
    return den;
}

// wave_max of N values, each DPP step taken for all of them before the next
// (N independent chains interleave); the same comparisons as wave_max.
template <int N>
__device__ __forceinline__ void wave_max_n(float (&a)[N]) {
#pragma unroll
    for (int i = 0; i < N; i++) a[i] = fmaxf(a[i], dpp_f<kQuadXor1>(a[i]));
#pragma unroll
    for (int i = 0; i < N; i++) a[i] = fmaxf(a[i], dpp_f<kQuadXor2>(a[i]));
#pragma unroll
    for (int i = 0; i < N; i++) a[i] = fmaxf(a[i], dpp_f<kRowHalfMirror>(a[i]));
#pragma unroll
    for (int i = 0; i < N; i++) a[i] = fmaxf(a[i], dpp_f<kRowMirror>(a[i]));
#pragma unroll
    for (int i = 0; i < N; i++)
        a[i] = fmaxf(fmaxf(readlane_f(a[i], 0), readlane_f(a[i], 16)),
                     fmaxf(readlane_f(a[i], 32), readlane_f(a[i], 48)));
}

// Softmax + values for one decode token, head_dim 128, KVMUL query heads per
// kv head (the arithmetic of attn_softmax_values_kernel, so the same bits).
// Workgroup = (kv head g, slice c of DW = 64 / KVMUL elements), kVDecThreads threads:
//   * every thread stages part of the slice's V rows into LDS transposed,
//     vt[e][t] (element-major, two positions per 32-bit store), and part of
//     the KVMUL score rows into w[hh][t];
//   * wave hh (< KVMUL) takes row hh's max (order-free) and replaces the row
//     by fastExpF32(s - max);
//   * wave 0 runs the KVMUL * DW value chains, lane (hh, e):
//     out = fma(w_t, v_t, out) in position order (dec_value_chain); wave 1's
//     lanes (hh, e) sum row hh's denominator in position order meanwhile
//     (dec_denominator); then out *= 1 / denom.
// One workgroup holds the whole span: vt and w take (2 * DW + 4 * KVMUL)
// bytes per position (vdec_lds_bytes).  The kv head's V rows are read by
// 2 * KVMUL workgroups, each its own slice, once.
constexpr int kVDecThreads = 512;  // two waves per SIMD: the exps of one fill the other's stalls
constexpr int kVDecCh = 3;  // V items (two 16-byte loads each) per thread per chunk
constexpr int kVDecSc = 2;  // score positions per thread and head per chunk
__host__ __device__ constexpr int vdec_pad(int span_max) {
    // rows of vt / w: at least span_max + 64 positions (the value chains read
    // up to 56 past the span), 8 mod 128 so the 16 lanes' ds_read_b128 of
    // one step fall on distinct banks
    return (span_max + 56 + 127) / 128 * 128 + 8;
}
static size_t vdec_lds_bytes(int kvmul, int span_max) {
    const size_t pad = (size_t)vdec_pad(span_max);
    // then 1 / denom per head and the waves' maxima per head ((1 + 8) kvmul floats)
    return pad * (size_t)(2 * (64 / kvmul) + 4 * kvmul) + 160;
}
template <int KVMUL>
__global__ __launch_bounds__(kVDecThreads) void attn_values_dec_kernel(
    const float* __restrict__ scores, const uint16_t* __restrict__ V, int kv_dim, int start,
    int span0, int span_max, float* __restrict__ out, const int* __restrict__ d_end) {
    static_assert(KVMUL == 1 || KVMUL == 2 || KVMUL == 4, "1, 2 or 4 query heads per kv head");
    constexpr int DW = 64 / KVMUL;    // elements per workgroup
    constexpr int NP = DW / 8;        // 16-byte pieces per V row slice
    constexpr int NS = kFusedHD / DW;  // slices per kv head
    constexpr int NW = kVDecThreads / 64;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    // kv head g = workgroup % n_kv: workgroups go to the eight XCDs in turn,
    // so with n_kv = 8 all slices of a head share one XCD's L2, which reads
    // the head's V lines from memory once for all of them
    const int n_kv = gridDim.x / NS;
    const int g = blockIdx.x % n_kv, c = blockIdx.x / n_kv;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pad = vdec_pad(span_max);
    uint16_t* vt = (uint16_t*)lds;                  // [DW][pad] f16
    float* w = lds + (size_t)DW * pad / 2;          // [KVMUL][pad]
    float* red = w + (size_t)KVMUL * pad;           // [KVMUL] 1 / denom, then [NW][KVMUL] maxima
    // V slice, two positions per item: rows 2tp and 2tp + 1 of piece pc.
    // Loads go out in unrolled chunks of kVDecCh items per thread, every
    // address clamped to a cache row, so a chunk's loads are all in flight
    // before the first one is used; the first chunk (and the score rows) is
    // issued before the device-side position is read, clamped to span_max.
    const uint16_t* Vg = V + (size_t)start * kv_dim + (size_t)g * kFusedHD + c * DW;
    constexpr int CH = kVDecCh;
    uint4 va[CH], vb[CH];
    auto vload = [&](int base, int last) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < CH; k++) {
            const int i = base + tid + k * kVDecThreads;
            const int tp = i / NP, pc = i % NP;
            const int t0 = min(2 * tp, last), t1 = min(2 * tp + 1, last);
            va[k] = *(const uint4*)(Vg + (size_t)t0 * kv_dim + 8 * pc);
            vb[k] = *(const uint4*)(Vg + (size_t)t1 * kv_dim + 8 * pc);
        }
    };
    auto vstore = [&](int base, int nitems) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < CH; k++) {
            const int i = base + tid + k * kVDecThreads;
            if (i < nitems) {
                const int tp = i / NP, pc = i % NP;
                const uint32_t av[4] = {va[k].x, va[k].y, va[k].z, va[k].w};
                const uint32_t bv[4] = {vb[k].x, vb[k].y, vb[k].z, vb[k].w};
                uint32_t* col = (uint32_t*)(vt + (size_t)(8 * pc) * pad + 2 * tp);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const uint32_t lo = (av[j >> 1] >> (16 * (j & 1))) & 0xffffu;
                    const uint32_t hi = (bv[j >> 1] >> (16 * (j & 1))) & 0xffffu;
                    col[(size_t)j * pad / 2] = lo | (hi << 16);
                }
            }
        }
    };
    // score rows: kVDecSc positions per thread and head per chunk
    constexpr int SC = kVDecSc;
    const float* srow = scores + (size_t)g * KVMUL * span_max;
    float sv[KVMUL][SC];
    auto sload = [&](int base) __attribute__((always_inline)) {
#pragma unroll
        for (int hh = 0; hh < KVMUL; hh++)
#pragma unroll
            for (int k = 0; k < SC; k++)
                sv[hh][k] = srow[(size_t)hh * span_max +
                                 min(base + tid + k * kVDecThreads, span_max - 1)];
    };
    auto sstore = [&](int base, int n) __attribute__((always_inline)) {
#pragma unroll
        for (int hh = 0; hh < KVMUL; hh++)
#pragma unroll
            for (int k = 0; k < SC; k++) {
                const int t = base + tid + k * kVDecThreads;
                if (t < n) w[(size_t)hh * pad + t] = sv[hh][k];
            }
    };
    vload(0, span_max - 1);
    sload(0);
    // (clamped to the rows the LDS image was sized for)
    const int span = min(d_end ? *d_end - start + 1 : span0, span_max);
    const int nitems = ((span + 1) >> 1) * NP;
    vstore(0, nitems);
    for (int base = CH * kVDecThreads; base < nitems; base += CH * kVDecThreads) {
        vload(base, span - 1);
        vstore(base, nitems);
    }
    if (span <= SC * kVDecThreads) {  // uniform: the whole score rows are in registers
        // each head's maximum (order-free: DPP within the waves, LDS across
        // them), then fastExpF32(s - max) on the registers, stored as w
        float* wm = red + KVMUL;  // [NW waves][KVMUL]
        {
            // the heads' cross-lane maxima step by step together (their DPP
            // chains interleave)
            float m[KVMUL];
#pragma unroll
            for (int hh = 0; hh < KVMUL; hh++) {
                m[hh] = -__int_as_float(0x7f800000);
#pragma unroll
                for (int k = 0; k < SC; k++)
                    if (tid + k * kVDecThreads < span) m[hh] = fmaxf(m[hh], sv[hh][k]);
            }
            wave_max_n(m);
            if (lane == 0) {
#pragma unroll
                for (int hh = 0; hh < KVMUL; hh++) wm[wave * KVMUL + hh] = m[hh];
            }
        }
        __syncthreads();
        // the exps of every position set and head in one interleaved pass,
        // computed before the guarded stores: the compiler would otherwise
        // sink each one into its store's branch and run them one after
        // another (sets past the span compute values nobody stores)
        float mx[KVMUL];
#pragma unroll
        for (int hh = 0; hh < KVMUL; hh++) {
            float m = wm[hh];
#pragma unroll
            for (int v = 1; v < NW; v++) m = fmaxf(m, wm[v * KVMUL + hh]);
            mx[hh] = m;
        }
        float xv[SC * KVMUL], ev[SC * KVMUL];
#pragma unroll
        for (int k = 0; k < SC; k++)
#pragma unroll
            for (int hh = 0; hh < KVMUL; hh++) xv[k * KVMUL + hh] = sv[hh][k] - mx[hh];
        fast_exp_n(xv, ev);
#pragma unroll
        for (int k = 0; k < SC; k++) {
            const int t = tid + k * kVDecThreads;
            if (t < span) {
#pragma unroll
                for (int hh = 0; hh < KVMUL; hh++) w[(size_t)hh * pad + t] = ev[k * KVMUL + hh];
            }
        }
        __syncthreads();
    } else {
        sstore(0, span);
        for (int base = SC * kVDecThreads; base < span; base += SC * kVDecThreads) {
            sload(base);
            sstore(base, span);
        }
        __syncthreads();
        if (wave < KVMUL) {
            float* wr = w + (size_t)wave * pad;
            float m = -__int_as_float(0x7f800000);
            for (int t = lane; t < span; t += 64) m = fmaxf(m, wr[t]);
            m = wave_max(m);
            exp_row<8>(wr, lane, 64, span, m);
        }
        __syncthreads();
    }
    const int hh = lane / DW, e = lane % DW;
    float acc = 0.0f;
    if (wave == 0) {
        acc = dec_value_chain(vt + (size_t)e * pad, w + (size_t)hh * pad, span);
    } else if (wave == 1) {  // lanes (hh, e): row hh's denominator, every e the same
        const float den = dec_denominator(w + (size_t)hh * pad, span);
        if (e == 0) red[hh] = den > 0.0f ? 1.0f / den : 1.0f;
    }
    __syncthreads();
    if (wave == 0) out[(size_t)(g * KVMUL + hh) * kFusedHD + c * DW + e] = acc * red[hh];
}

// --- split-K path ------------------------------------------------------------

constexpr int kSplitTile = 64;  // positions per tile

// One workgroup per (kv head, chunk of positions): all `kvmul` query heads of
// the group share each K/V tile.  Writes per-head (max, sum, unnormalised out).
template <int HD>
__global__ __launch_bounds__(256) void attn_splitk_kernel(const float* __restrict__ q,
                                                          const uint16_t* __restrict__ K,
                                                          const uint16_t* __restrict__ V,
                                                          int kv_dim, int n_kv, int kvmul,
                                                          int start, int span, int chunk,
                                                          float scale, float* __restrict__ part_m,
                                                          float* __restrict__ part_l,
                                                          float* __restrict__ part_o) {
    const int g = blockIdx.y;
    const int c = blockIdx.x;
    const int nchunks = gridDim.x;
    const int t0 = c * chunk;
    const int t1 = min(span, t0 + chunk);
    __shared__ float qs[8][HD];
    __shared__ float w[8][kSplitTile];
    __shared__ float red[8][4];
    const int tid = threadIdx.x;
    for (int i = tid; i < kvmul * HD; i += 256) qs[i / HD][i % HD] = q[(size_t)g * kvmul * HD + i];
    // running state per head (replicated in every thread that needs it)
    float m_run[8], l_run[8];
    for (int h = 0; h < 8; h++) {
        m_run[h] = -__int_as_float(0x7f800000);
        l_run[h] = 0.0f;
    }
    // output accumulators: thread owns (head, element) pairs tid, tid+256, ...
    constexpr int kOutPer = (8 * HD + 255) / 256;
    float o_acc[kOutPer];
    for (int i = 0; i < kOutPer; i++) o_acc[i] = 0.0f;
    __syncthreads();
    for (int tt = t0; tt < t1; tt += kSplitTile) {
        const int nt = min(kSplitTile, t1 - tt);
        // scores: thread (p, h) for p < nt, h < kvmul; 256 threads = 64 x 4
        for (int item = tid; item < nt * kvmul; item += 256) {
            const int p = item / kvmul, h = item % kvmul;
            const uint16_t* krow = K + (size_t)(start + tt + p) * kv_dim + g * HD;
            float acc = 0.0f;
#pragma unroll 8
            for (int e = 0; e < HD; e += 2) {
                const uint32_t two = *(const uint32_t*)(krow + e);
                acc = fmaf(f16_bits_to_f32(two & 0xffffu), qs[h][e], acc);
                acc = fmaf(f16_bits_to_f32(two >> 16), qs[h][e + 1], acc);
            }
            w[h][p] = acc * scale;
        }
        __syncthreads();
        // per-head tile max and new running max (every thread computes the
        // same values from LDS)
        float alpha[8];
        for (int h = 0; h < kvmul; h++) {
            float mt = m_run[h];
            for (int p = 0; p < nt; p++) mt = fmaxf(mt, w[h][p]);
            alpha[h] = fast_exp(m_run[h] - mt);
            if (m_run[h] == -__int_as_float(0x7f800000)) alpha[h] = 0.0f;
            m_run[h] = mt;
        }
        __syncthreads();
        for (int item = tid; item < nt * kvmul; item += 256) {
            const int p = item / kvmul, h = item % kvmul;
            w[h][p] = fast_exp(w[h][p] - m_run[h]);
        }
        __syncthreads();
        for (int h = 0; h < kvmul; h++) {
            float sum = 0.0f;
            for (int p = 0; p < nt; p++) sum += w[h][p];
            l_run[h] = l_run[h] * alpha[h] + sum;
        }
        for (int i = 0; i < kOutPer; i++) {
            const int idx = tid + 256 * i;
            if (idx < kvmul * HD) {
                const int h = idx / HD, d = idx % HD;
                float acc = o_acc[i] * alpha[h];
                const uint16_t* vcol = V + (size_t)(start + tt) * kv_dim + g * HD + d;
                for (int p = 0; p < nt; p++)
                    acc = fmaf(w[h][p], f16_bits_to_f32(vcol[(size_t)p * kv_dim]), acc);
                o_acc[i] = acc;
            }
        }
        __syncthreads();
    }
    (void)red;
    for (int i = 0; i < kOutPer; i++) {
        const int idx = tid + 256 * i;
        if (idx < kvmul * HD) {
            const int h = idx / HD;
            part_o[(((size_t)g * kvmul + h) * nchunks + c) * HD + idx % HD] = o_acc[i];
        }
    }
    if (tid < kvmul) {
        part_m[((size_t)g * kvmul + tid) * nchunks + c] = m_run[tid];
        part_l[((size_t)g * kvmul + tid) * nchunks + c] = l_run[tid];
    }
}

// Split-K kernel for head_dim 128 and 4 query heads per kv head (Llama-3
// GQA).  Workgroup = 4 waves on one (kv head g, chunk of positions); each wave
// streams its own contiguous run of 16-position tiles:
//   lane = 16*rg + seg: rows rg, rg+4, rg+8, rg+12 of a tile, dims 8*seg..+7
//   (one 16-byte load per row, a 256-byte K or V row per 16 lanes), with the
//   next tile's K and V loads in flight while the current one is used;
//   q for the lane's 8 dims and 4 heads stays in registers;
//   the 16 (row, head) partial dots of a lane are transpose-reduced over its
//   16-lane row group with DPP (ror 8, half mirror, quad perms), leaving lane
//   seg with the score of row 4*(seg>>2)+rg, head seg&3;
//   online softmax per head, weights broadcast to the row group through LDS;
//   o[4 heads][8 dims] accumulated per lane, reduced over rg at the end.
// The 4 waves' (max, sum, o) are merged in LDS into one partial per chunk.
constexpr int kSkTile = 16;
constexpr int kSkWaves = 4;

__device__ __forceinline__ void f16x8_to_f32(const uint4 r, float* f) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
        f[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
    }
}

// one halving step of the 16-lane transpose-reduce: lanes whose `bit` is set
// keep the upper half of v, the DPP partner (which has the bit clear) the
// lower half
template <int N, int CTRL>
__device__ __forceinline__ void tr_step(float* v, bool upper) {
#pragma unroll
    for (int j = 0; j < N / 2; j++) {
        const float keep = upper ? v[j + N / 2] : v[j];
        const float send = upper ? v[j] : v[j + N / 2];
        v[j] = keep + dpp_f<CTRL>(send);
    }
}

__device__ __forceinline__ float wave_head_max(float x) {
    x = fmaxf(x, dpp_f<0x124>(x));  // row_ror:4
    x = fmaxf(x, dpp_f<0x128>(x));  // row_ror:8
    x = fmaxf(x, __shfl_xor(x, 16));
    return fmaxf(x, __shfl_xor(x, 32));
}

__device__ __forceinline__ float wave_head_sum(float x) {
    x += dpp_f<0x124>(x);
    x += dpp_f<0x128>(x);
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
}

__global__ __launch_bounds__(256) void attn_splitk_g4_kernel(
    const float* __restrict__ q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    int kv_dim, int start, int span, int chunk, float scale, float* __restrict__ part_m,
    float* __restrict__ part_l, float* __restrict__ part_o) {
    constexpr int HD = 128, KM = 4;
    const float ninf = -__int_as_float(0x7f800000);
    const int g = blockIdx.y, c = blockIdx.x, nchunks = gridDim.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rg = lane >> 4, seg = lane & 15;
    const int wspan = chunk / kSkWaves;
    const int p0 = c * chunk + wave * wspan;  // relative to start
    const int p1 = min(span, p0 + wspan);
    __shared__ __align__(16) float wl[kSkWaves][64];
    __shared__ float sm[kSkWaves][KM], sl[kSkWaves][KM];
    __shared__ __align__(16) float so[kSkWaves][KM][HD];

    float qv[KM][8];
#pragma unroll
    for (int h = 0; h < KM; h++) {
        const float4* qp = (const float4*)(q + ((size_t)g * KM + h) * HD + 8 * seg);
        const float4 a = qp[0], b = qp[1];
        qv[h][0] = a.x; qv[h][1] = a.y; qv[h][2] = a.z; qv[h][3] = a.w;
        qv[h][4] = b.x; qv[h][5] = b.y; qv[h][6] = b.z; qv[h][7] = b.w;
    }
    float o[KM][8];
#pragma unroll
    for (int h = 0; h < KM; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) o[h][e] = 0.0f;
    float m_run = ninf, l_run = 0.0f;  // head seg & 3

    const size_t col = (size_t)g * HD + 8 * seg;
    auto load_tile = [&](int pb, uint4* kr, uint4* vr) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int pos = pb + 4 * i + rg;
            const size_t row = (size_t)start + (pos < p1 ? pos : p0);
            kr[i] = *(const uint4*)(K + row * kv_dim + col);
            vr[i] = *(const uint4*)(V + row * kv_dim + col);
        }
    };
    if (p0 < p1) {
        uint4 kc[4], vc[4];
        load_tile(p0, kc, vc);
        for (int pb = p0; pb < p1; pb += kSkTile) {
            uint4 kn[4], vn[4];
            const bool more = pb + kSkTile < p1;
            if (more) load_tile(pb + kSkTile, kn, vn);
            // partial dots: v[4*i + h] = sum over this lane's 8 dims
            float v[16];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float kf[8];
                f16x8_to_f32(kc[i], kf);
#pragma unroll
                for (int h = 0; h < KM; h++) {
                    float acc = qv[h][0] * kf[0];
#pragma unroll
                    for (int e = 1; e < 8; e++) acc = fmaf(qv[h][e], kf[e], acc);
                    v[4 * i + h] = acc;
                }
            }
            tr_step<16, 0x128>(v, seg & 8);  // row_ror:8       (partner seg ^ 8)
            tr_step<8, 0x141>(v, seg & 4);   // row_half_mirror (partner seg ^ 7)
            tr_step<4, 0x1B>(v, seg & 2);    // quad_perm 3210  (partner seg ^ 3)
            tr_step<2, 0xB1>(v, seg & 1);    // quad_perm 1032  (partner seg ^ 1)
            const int pos = pb + 4 * (seg >> 2) + rg;
            const float sc = pos < p1 ? v[0] * scale : ninf;
            const float m_new = fmaxf(m_run, wave_head_max(sc));
            const float alpha = m_run == ninf ? 0.0f : fast_exp(m_run - m_new);
            const float w = m_new == ninf ? 0.0f : fast_exp(sc - m_new);
            l_run = fmaf(l_run, alpha, wave_head_sum(w));
            m_run = m_new;
            // lane h (rg 0, seg h) holds head h's rescale factor
            float al[KM];
#pragma unroll
            for (int h = 0; h < KM; h++)
                al[h] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), h));
            if (!(al[0] == 1.0f && al[1] == 1.0f && al[2] == 1.0f && al[3] == 1.0f)) {
#pragma unroll
                for (int h = 0; h < KM; h++)
#pragma unroll
                    for (int e = 0; e < 8; e++) o[h][e] *= al[h];
            }
            wl[wave][lane] = w;
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 wi = *(const float4*)&wl[wave][16 * rg + 4 * i];
                const float wh[KM] = {wi.x, wi.y, wi.z, wi.w};
                float vf[8];
                f16x8_to_f32(vc[i], vf);
#pragma unroll
                for (int h = 0; h < KM; h++)
#pragma unroll
                    for (int e = 0; e < 8; e++) o[h][e] = fmaf(wh[h], vf[e], o[h][e]);
            }
            __builtin_amdgcn_wave_barrier();
            if (more) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    kc[i] = kn[i];
                    vc[i] = vn[i];
                }
            }
        }
    }
    // reduce o over the four row groups
#pragma unroll
    for (int h = 0; h < KM; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float x = o[h][e];
            x += __shfl_xor(x, 16);
            x += __shfl_xor(x, 32);
            o[h][e] = x;
        }
    if (rg == 0) {
#pragma unroll
        for (int h = 0; h < KM; h++) {
            *(float4*)&so[wave][h][8 * seg] = make_float4(o[h][0], o[h][1], o[h][2], o[h][3]);
            *(float4*)&so[wave][h][8 * seg + 4] = make_float4(o[h][4], o[h][5], o[h][6], o[h][7]);
        }
    }
    if (lane < KM) {
        sm[wave][lane] = m_run;
        sl[wave][lane] = l_run;
    }
    __syncthreads();
    const int t = threadIdx.x;
    const int h = t >> 6, d = 2 * (t & 63);
    float M = ninf;
#pragma unroll
    for (int w = 0; w < kSkWaves; w++) M = fmaxf(M, sm[w][h]);
    float L = 0.0f, O0 = 0.0f, O1 = 0.0f;
#pragma unroll
    for (int w = 0; w < kSkWaves; w++) {
        const float f = sl[w][h] > 0.0f ? fast_exp(sm[w][h] - M) : 0.0f;
        L = fmaf(sl[w][h], f, L);
        O0 = fmaf(so[w][h][d], f, O0);
        O1 = fmaf(so[w][h][d + 1], f, O1);
    }
    const size_t hc = ((size_t)g * KM + h) * nchunks + c;
    *(float2*)&part_o[hc * HD + d] = make_float2(O0, O1);
    if ((t & 63) == 0) {
        part_m[hc] = M;
        part_l[hc] = L;
    }
}

__global__ __launch_bounds__(128) void attn_merge_kernel(const float* __restrict__ part_m,
                                                         const float* __restrict__ part_l,
                                                         const float* __restrict__ part_o,
                                                         int nchunks, int hd,
                                                         float* __restrict__ out) {
    const int h = blockIdx.x, d = threadIdx.x;
    if (d >= hd) return;
    const float* pm = part_m + (size_t)h * nchunks;
    const float* pl = part_l + (size_t)h * nchunks;
    float M = -__int_as_float(0x7f800000);
    for (int c = 0; c < nchunks; c++) M = fmaxf(M, pm[c]);
    float L = 0.0f, O = 0.0f;
    for (int c = 0; c < nchunks; c++) {
        if (pl[c] == 0.0f) continue;
        const float a = fast_exp(pm[c] - M);
        L = fmaf(pl[c], a, L);
        O = fmaf(part_o[((size_t)h * nchunks + c) * hd + d], a, O);
    }
    out[(size_t)h * hd + d] = O * (1.0f / L);
}

// Merge of split-K partials, one workgroup per (head, 32-dim quarter): the
// chunk factors exp(m_c - M) are computed once into LDS, then 8 thread groups
// each sum every 8th chunk (independent loads in flight) and are combined.
constexpr int kMergeMaxChunks = 2048;

__global__ __launch_bounds__(256) void attn_merge2_kernel(const float* __restrict__ part_m,
                                                          const float* __restrict__ part_l,
                                                          const float* __restrict__ part_o,
                                                          int nchunks, int hd,
                                                          float* __restrict__ out) {
    const float ninf = -__int_as_float(0x7f800000);
    const int h = blockIdx.x, t = threadIdx.x;
    const float* pm = part_m + (size_t)h * nchunks;
    const float* pl = part_l + (size_t)h * nchunks;
    __shared__ float f[kMergeMaxChunks];
    __shared__ float red[8];
    __shared__ float acc[8][32];
    float m = ninf;
    for (int c = t; c < nchunks; c += 256) m = fmaxf(m, pm[c]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((t & 63) == 0) red[t >> 6] = m;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float lsum = 0.0f;
    for (int c = t; c < nchunks; c += 256) {
        const float l = pl[c];
        const float fc = l > 0.0f ? fast_exp(pm[c] - M) : 0.0f;
        f[c] = fc;
        lsum = fmaf(l, fc, lsum);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) lsum += __shfl_xor(lsum, off);
    __syncthreads();
    if ((t & 63) == 0) red[4 + (t >> 6)] = lsum;
    __syncthreads();
    const float L = (red[4] + red[5]) + (red[6] + red[7]);
    const int d = blockIdx.y * 32 + (t & 31), cg = t >> 5;
    float o = 0.0f;
    if (d < hd) {
        const float* po = part_o + (size_t)h * nchunks * hd + d;
#pragma unroll 8
        for (int c = cg; c < nchunks; c += 8) o = fmaf(po[(size_t)c * hd], f[c], o);
    }
    acc[cg][t & 31] = o;
    __syncthreads();
    if (t < 32 && d < hd) {
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) sum += acc[j][t];
        out[(size_t)h * hd + d] = sum * (1.0f / L);
    }
}

// The one-token values kernel applies when its LDS image of the whole span
// fits a workgroup (attn_softmax_values_kernel otherwise; both give the
// same bits).
static bool vdec_usable(int kvmul, int span_max) {
    if (kvmul != 1 && kvmul != 2 && kvmul != 4) return false;
    const size_t bytes = vdec_lds_bytes(kvmul, span_max);
    if (bytes <= 65536) return true;
    static const bool big_ok = [] {
        const int cap = 160 * 1024;
        return hipFuncSetAttribute((const void*)attn_values_dec_kernel<4>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, cap) == hipSuccess &&
               hipFuncSetAttribute((const void*)attn_values_dec_kernel<2>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, cap) == hipSuccess &&
               hipFuncSetAttribute((const void*)attn_values_dec_kernel<1>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, cap) == hipSuccess;
    }();
    if (!big_ok) (void)hipGetLastError();
    return big_ok && bytes <= 160 * 1024;
}

// Exact attention for p consecutive query tokens: token t attends
// start .. end0 + t.  d_q / d_out: [p][n_heads][hd].
bool attend_exact_graphable(const gllm_hip_kv* kv, int n_heads, int n_kv, int hd, int span_cap) {
    return hd == kFusedHD && n_heads / n_kv <= 4 && kv->kv_dim_k == kv->kv_dim_v &&
           span_cap <= kSmaxSpan1;
}

// scratch: p * n_heads * (span_max + 1) + n_heads * ceil(span_max / 32) + 64
// floats of device memory, or null for the calling thread's scratch.  d_end (with p == 1): the end position is read
// on the device and span_cap bounds the span, so the launches do not depend
// on the position (a captured decode step replays for every position).
int attend_exact(const gllm_hip_kv* kv, int l, const float* d_q, int n_heads, int n_kv, int hd,
                 int start, int end0, int p, float scale, float* d_out, hipStream_t s,
                 float* scratch, const int* d_end, int span_cap, const float* rope_sin,
                 const float* rope_cos, const float* d_knew, const float* d_vnew,
                 const float* rope_cur) {
    const int span0 = end0 - start + 1;
    const int span_max = d_end ? span_cap : span0 + p - 1;
    const int kvmul = n_heads / n_kv;
    // the kernels load rows up to start + span_max - 1 before they know the span
    if (start < 0 || span_max < 1 || start + span_max > kv->max_len)
        return fail(GLLM_EINVAL, "attend: rows %d..%d outside the cache (%d)", start,
                    start + span_max - 1, kv->max_len);
    if (d_end && (p != 1 || !attend_exact_graphable(kv, n_heads, n_kv, hd, span_cap)))
        return fail(GLLM_EUNSUP, "attend: device-side positions need the head_dim 128 path");
    if (rope_sin && (!d_end || !d_knew || !d_vnew))
        return fail(GLLM_EINVAL, "attend: RoPE folding needs one token and its raw k / v rows");
    const AttnRope rope{rope_sin, rope_cos, d_knew, d_vnew, kv->k[l], kv->v[l], rope_cur};
    if (hd == kFusedHD && kvmul <= 4 && kv->kv_dim_k == kv->kv_dim_v &&
        span_max <= (p == 1 ? kSmaxSpan1 : kSmaxSpan)) {
        const int nchunk = (span_max + kScoreChunk - 1) / kScoreChunk;
        // the long-span values kernel takes the row's maximum from per-chunk
        // maxima that the scores launch writes after the score rows
        const bool long_path = p == 1 && !vdec_usable(kvmul, span_max) && span_max <= kLongSpan;
        const size_t sc_floats = (size_t)p * n_heads * span_max + (long_path ? (size_t)n_heads * nchunk : 0);
        float* sc = scratch ? scratch : (float*)thread_scratch(5, sc_floats * 4 + 256, s);
        if (!sc) return scratch_error();
        float* cmax = long_path ? sc + (size_t)n_heads * span_max : nullptr;
        // the V touch pays while one kv head's K and V rows fit an XCD's
        // 4 MB L2 (256 bytes each per position), and not ahead of the
        // long-span kernel, whose deep V prefetch measured faster untouched
        const int touch = span_max <= kTouchSpan && !long_path;
        if (long_path)
            hipLaunchKernelGGL(attn_scores128_kernel<true>, dim3(n_kv, nchunk, p), dim3(256), 0, s,
                               d_q, kv->k[l], kv->v[l], kv->kv_dim_k, n_kv, kvmul, start, span0,
                               span_max, scale, sc, d_end, rope, touch, cmax);
        else
            hipLaunchKernelGGL(attn_scores128_kernel<false>, dim3(n_kv, nchunk, p), dim3(256), 0, s,
                               d_q, kv->k[l], kv->v[l], kv->kv_dim_k, n_kv, kvmul, start, span0,
                               span_max, scale, sc, d_end, rope, touch, cmax);
        GLLM_HIP(hipGetLastError());
        // one token: four workgroups per head (a quarter of each V row apiece);
        // prefill tokens already give n_heads * p workgroups
        if (p == 1 && vdec_usable(kvmul, span_max)) {
            const dim3 grid(n_kv * (kFusedHD / (64 / kvmul)));
            const size_t lds = vdec_lds_bytes(kvmul, span_max);
            if (kvmul == 4)
                hipLaunchKernelGGL(attn_values_dec_kernel<4>, grid, dim3(kVDecThreads), lds, s, sc,
                                   kv->v[l], kv->kv_dim_v, start, span0, span_max, d_out, d_end);
            else if (kvmul == 2)
                hipLaunchKernelGGL(attn_values_dec_kernel<2>, grid, dim3(kVDecThreads), lds, s, sc,
                                   kv->v[l], kv->kv_dim_v, start, span0, span_max, d_out, d_end);
            else
                hipLaunchKernelGGL(attn_values_dec_kernel<1>, grid, dim3(kVDecThreads), lds, s, sc,
                                   kv->v[l], kv->kv_dim_v, start, span0, span_max, d_out, d_end);
        } else if (p == 1 && span_max <= kLongSpan) {
            static const bool lds_ok = [] {
                // dynamic LDS beyond 64 KB for long rows
                return hipFuncSetAttribute((const void*)attn_values_long_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)long_lds_bytes(kLongSpan)) == hipSuccess;
            }();
            if (!lds_ok) {
                (void)hipGetLastError();
                if (long_lds_bytes(span_max) > 65536)
                    return fail(GLLM_EDEVICE, "attend: %zu bytes of LDS not available",
                                long_lds_bytes(span_max));
            }
            hipLaunchKernelGGL(attn_values_long_kernel, dim3(n_heads * 4), dim3(kLongThreads),
                               long_lds_bytes(span_max), s, sc, cmax, kv->v[l], kv->kv_dim_v,
                               kvmul, start, span0, span_max, d_out, d_end);
        } else if (p == 1) {
            static const bool lds_ok = [] {
                // dynamic LDS beyond 64 KB for long rows
                return hipFuncSetAttribute((const void*)attn_softmax_values_kernel<4>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)smax_lds_bytes<4>(kSmaxSpan1)) == hipSuccess;
            }();
            if (!lds_ok) {
                (void)hipGetLastError();
                if (smax_lds_bytes<4>(span_max) > 65536)
                    return fail(GLLM_EDEVICE, "attend: %zu bytes of LDS not available",
                                smax_lds_bytes<4>(span_max));
            }
            hipLaunchKernelGGL(attn_softmax_values_kernel<4>, dim3(n_heads * 4, p), dim3(256),
                               smax_lds_bytes<4>(span_max), s, sc, kv->v[l], kv->kv_dim_v, kvmul,
                               start, span0, span_max, d_out, d_end);
        } else {
            hipLaunchKernelGGL(attn_softmax_values_kernel<1>, dim3(n_heads, p), dim3(256),
                               smax_lds_bytes<1>(span_max), s, sc, kv->v[l], kv->kv_dim_v, kvmul,
                               start, span0, span_max, d_out, d_end);
        }
        GLLM_HIP(hipGetLastError());
        return GLLM_OK;
    }
    float* scr = scratch ? scratch
                         : (float*)thread_scratch(5, ((size_t)p * n_heads * (span_max + 1) + 64) * 4, s);
    if (!scr) return scratch_error();
    float* scores = scr;
    float* inv = scr + (size_t)p * n_heads * span_max;
    const int items = span_max * n_kv;
    hipLaunchKernelGGL(attn_scores_kernel, dim3((items + 31) / 32, p), dim3(256), 0, s, d_q,
                       kv->k[l], kv->kv_dim_k, n_kv, kvmul, hd, start, span0, span_max, scale,
                       scores);
    GLLM_HIP(hipGetLastError());
    hipLaunchKernelGGL(attn_softmax_kernel, dim3(n_heads, p), dim3(256), 0, s, scores, span0,
                       span_max, inv);
    GLLM_HIP(hipGetLastError());
    hipLaunchKernelGGL(attn_values_kernel, dim3(n_heads, p), dim3(128), 0, s, scores, inv,
                       kv->v[l], kv->kv_dim_v, kvmul, hd, start, span0, span_max, d_out);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

int attend_splitk(const gllm_hip_kv* kv, int l, const float* d_q, int n_heads, int n_kv, int hd,
                  int start, int end, float scale, float* d_out, hipStream_t s) {
    if (hd != 128) return fail(GLLM_EUNSUP, "split-K attention is built for head_dim 128");
    const int span = end - start + 1;
    const int kvmul = n_heads / n_kv;
    if (kvmul == 4 && kv->kv_dim_k == kv->kv_dim_v) {
        // one round of resident workgroups (no ragged second round), chunks a
        // multiple of 4 waves x 16 rows
        static int per_cu = 0;
        if (!per_cu) {
            int n = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, attn_splitk_g4_kernel, 256, 0) !=
                    hipSuccess || n <= 0)
                n = 2;
            per_cu = n;
        }
        const int quantum = kSkWaves * kSkTile;
        const int target =
            std::min(kMergeMaxChunks, std::max(1, per_cu * device_cus() / n_kv));
        int chunk = (span + target - 1) / target;
        chunk = std::max(quantum, (chunk + quantum - 1) / quantum * quantum);
        const int nchunks = (span + chunk - 1) / chunk;  // <= target <= kMergeMaxChunks
        const size_t nh = (size_t)n_heads;
        float* scr = (float*)thread_scratch(6, (nh * nchunks * (2 + hd) + 64) * 4, s);
        if (!scr) return scratch_error();
        float* pm = scr;
        float* pl = pm + nh * nchunks;
        float* po = pl + nh * nchunks;
        hipLaunchKernelGGL(attn_splitk_g4_kernel, dim3(nchunks, n_kv), dim3(256), 0, s, d_q,
                           kv->k[l], kv->v[l], kv->kv_dim_k, start, span, chunk, scale, pm, pl, po);
        GLLM_HIP(hipGetLastError());
        hipLaunchKernelGGL(attn_merge2_kernel, dim3(n_heads, (hd + 31) / 32), dim3(256), 0, s, pm,
                           pl, po, nchunks, hd, d_out);
        GLLM_HIP(hipGetLastError());
        return GLLM_OK;
    }
    // chunk so that n_kv * nchunks covers the device several times over
    int nchunks = std::max(1, std::min(512 / std::max(1, n_kv), (span + kSplitTile - 1) / kSplitTile));
    int chunk = (span + nchunks - 1) / nchunks;
    chunk = (chunk + kSplitTile - 1) / kSplitTile * kSplitTile;
    nchunks = (span + chunk - 1) / chunk;
    const size_t nh = (size_t)n_heads;
    float* scr = (float*)thread_scratch(6, (nh * nchunks * (2 + hd) + 64) * 4, s);
    if (!scr) return scratch_error();
    float* pm = scr;
    float* pl = pm + nh * nchunks;
    float* po = pl + nh * nchunks;
    hipLaunchKernelGGL(attn_splitk_kernel<128>, dim3(nchunks, n_kv), dim3(256), 0, s, d_q, kv->k[l],
                       kv->v[l], kv->kv_dim_k, n_kv, kvmul, start, span, chunk, scale, pm, pl, po);
    GLLM_HIP(hipGetLastError());
    hipLaunchKernelGGL(attn_merge_kernel, dim3(n_heads), dim3(128), 0, s, pm, pl, po, nchunks, hd,
                       d_out);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

int attend_dev_impl(gllm_hip_kv* kv, int l, const float* d_q, int n_heads, int n_kv, int hd,
                    int start, int end, float scale, int mode, float* d_out, hipStream_t s) {
    if (!kv || !d_q || !d_out) return fail(GLLM_EINVAL, "attend: null pointer");
    if (l < 0 || l >= kv->layers) return fail(GLLM_EINVAL, "attend: layer %d out of range", l);
    if (n_kv <= 0 || n_heads % n_kv || n_heads / n_kv > 8 || hd % 8 || hd > 128 ||
        n_kv * hd > kv->kv_dim_k || n_kv * hd > kv->kv_dim_v)
        return fail(GLLM_EINVAL, "attend: heads %d/%d hd %d do not fit the cache", n_heads, n_kv, hd);
    if (start < 0 || end < start || end >= kv->max_len)
        return fail(GLLM_EINVAL, "attend: positions %d..%d outside 0..%d", start, end, kv->max_len - 1);
    if (mode == GLLM_ATTN_SPLITK)
        return attend_splitk(kv, l, d_q, n_heads, n_kv, hd, start, end, scale, d_out, s);
    return attend_exact(kv, l, d_q, n_heads, n_kv, hd, start, end, 1, scale, d_out, s, nullptr,
                        nullptr, 0, nullptr, nullptr, nullptr, nullptr, nullptr);
}

int kv_store_dev_impl(gllm_hip_kv* kv, int l, int pos, const float* d_k, const float* d_v,
                      hipStream_t s) {
    if (!kv || !d_k || !d_v) return fail(GLLM_EINVAL, "kv_store: null pointer");
    if (l < 0 || l >= kv->layers || pos < 0 || pos >= kv->max_len)
        return fail(GLLM_EINVAL, "kv_store: layer %d pos %d out of range", l, pos);
    const int n = std::max(kv->kv_dim_k, kv->kv_dim_v);
    hipLaunchKernelGGL(kv_store_kernel, dim3((n + 255) / 256), dim3(256), 0, s, d_k, d_v,
                       kv->k[l] + (size_t)pos * kv->kv_dim_k, kv->v[l] + (size_t)pos * kv->kv_dim_v,
                       kv->kv_dim_k, kv->kv_dim_v);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

}  // namespace gllm

using namespace gllm;

extern "C" {

gllm_hip_kv* gllm_hip_kv_new(int layers, int kv_dim_k, int kv_dim_v, int max_len) {
    if (layers <= 0 || kv_dim_k <= 0 || kv_dim_v <= 0 || max_len <= 0) {
        fail(GLLM_EINVAL, "gllm_hip_kv_new: bad shape");
        return nullptr;
    }
    gllm_hip_kv* kv = new gllm_hip_kv();
    kv->layers = layers;
    kv->kv_dim_k = kv_dim_k;
    kv->kv_dim_v = kv_dim_v;
    kv->max_len = max_len;
    kv->k = new uint16_t*[layers]();
    kv->v = new uint16_t*[layers]();
    if (hipGetDevice(&kv->device) != hipSuccess) kv->device = 0;
    for (int l = 0; l < layers; l++) {
        if (hipMalloc(&kv->k[l], (size_t)max_len * kv_dim_k * 2) != hipSuccess ||
            hipMalloc(&kv->v[l], (size_t)max_len * kv_dim_v * 2) != hipSuccess) {
            (void)hipGetLastError();
            fail(GLLM_ENOMEM, "gllm_hip_kv_new: out of device memory");
            gllm_hip_kv_release(kv);
            return nullptr;
        }
        // zeroed rows, like make([]uint16, ...) in NewKVCacheF16
        if (hipMemset(kv->k[l], 0, (size_t)max_len * kv_dim_k * 2) != hipSuccess ||
            hipMemset(kv->v[l], 0, (size_t)max_len * kv_dim_v * 2) != hipSuccess) {
            (void)hipGetLastError();
            fail(GLLM_EDEVICE, "gllm_hip_kv_new: hipMemset failed");
            gllm_hip_kv_release(kv);
            return nullptr;
        }
    }
    return kv;
}

void gllm_hip_kv_release(gllm_hip_kv* kv) {
    if (!kv) return;
    for (int l = 0; l < kv->layers; l++) {
        if (kv->k[l]) (void)hipFree(kv->k[l]);
        if (kv->v[l]) (void)hipFree(kv->v[l]);
    }
    delete[] kv->k;
    delete[] kv->v;
    delete kv;
}

uint16_t* gllm_hip_kv_k_dev(gllm_hip_kv* kv, int l) {
    if (!kv || l < 0 || l >= kv->layers) {
        fail(GLLM_EINVAL, "gllm_hip_kv_k_dev: bad layer");
        return nullptr;
    }
    return kv->k[l];
}

uint16_t* gllm_hip_kv_v_dev(gllm_hip_kv* kv, int l) {
    if (!kv || l < 0 || l >= kv->layers) {
        fail(GLLM_EINVAL, "gllm_hip_kv_v_dev: bad layer");
        return nullptr;
    }
    return kv->v[l];
}

int gllm_hip_kv_read(gllm_hip_kv* kv, int l, int pos0, int n, uint16_t* k_out, uint16_t* v_out) {
    if (!kv || l < 0 || l >= kv->layers || pos0 < 0 || n < 0 || pos0 + n > kv->max_len)
        return fail(GLLM_EINVAL, "gllm_hip_kv_read: bad range");
    // rows may have been written on another stream (the decoder's): drain the
    // device first, then copy synchronously
    GLLM_HIP(hipDeviceSynchronize());
    if (k_out)
        GLLM_HIP(hipMemcpy(k_out, kv->k[l] + (size_t)pos0 * kv->kv_dim_k,
                           (size_t)n * kv->kv_dim_k * 2, hipMemcpyDeviceToHost));
    if (v_out)
        GLLM_HIP(hipMemcpy(v_out, kv->v[l] + (size_t)pos0 * kv->kv_dim_v,
                           (size_t)n * kv->kv_dim_v * 2, hipMemcpyDeviceToHost));
    return GLLM_OK;
}

int gllm_hip_kv_store_dev(gllm_hip_kv* kv, int l, int pos, const float* d_k, const float* d_v,
                          void* stream) {
    return kv_store_dev_impl(kv, l, pos, d_k, d_v, (hipStream_t)stream);
}

int gllm_hip_kv_store(gllm_hip_kv* kv, int l, int pos, const float* k, const float* v) {
    if (!kv || !k || !v) return fail(GLLM_EINVAL, "gllm_hip_kv_store: null pointer");
    hipStream_t s = thread_stream();
    if (!s) return GLLM_EDEVICE;
    float* d = (float*)thread_scratch(1, (size_t)(kv->kv_dim_k + kv->kv_dim_v) * 4, s);
    if (!d) return scratch_error();
    GLLM_HIP(hipMemcpyAsync(d, k, (size_t)kv->kv_dim_k * 4, hipMemcpyHostToDevice, s));
    GLLM_HIP(hipMemcpyAsync(d + kv->kv_dim_k, v, (size_t)kv->kv_dim_v * 4, hipMemcpyHostToDevice, s));
    GLLM_TRY(kv_store_dev_impl(kv, l, pos, d, d + kv->kv_dim_k, s));
    GLLM_HIP(hipStreamSynchronize(s));
    return GLLM_OK;
}

int gllm_hip_attend_dev(gllm_hip_kv* kv, int l, const float* d_q, int n_heads, int n_kv_heads,
                        int hd, int start, int end, float scale, int mode, float* d_out,
                        void* stream) {
    return attend_dev_impl(kv, l, d_q, n_heads, n_kv_heads, hd, start, end, scale, mode, d_out,
                           (hipStream_t)stream);
}

// attendHeadGroup for one kv head: q_heads queries (host) -> out (host).
int gllm_hip_attend_group(gllm_hip_kv* kv, int l, int kvh, const float* q, int q_heads, int hd,
                          int vd, int start, int end, float scale, float softcap, float* out) {
    if (!kv || !q || !out) return fail(GLLM_EINVAL, "gllm_hip_attend_group: null pointer");
    if (softcap != 0.0f) return fail(GLLM_EUNSUP, "attention softcap is not on this path");
    if (hd != vd) return fail(GLLM_EUNSUP, "key and value head dims must match");
    if (l < 0 || l >= kv->layers || kvh < 0 || hd <= 0 || hd % 8 || hd > 128 ||
        (size_t)(kvh + 1) * hd > (size_t)kv->kv_dim_k || (size_t)(kvh + 1) * vd > (size_t)kv->kv_dim_v ||
        q_heads < 1 || q_heads > 8)
        return fail(GLLM_EINVAL, "gllm_hip_attend_group: bad head arguments");
    if (start < 0 || end < start || end >= kv->max_len)
        return fail(GLLM_EINVAL, "gllm_hip_attend_group: positions %d..%d outside 0..%d", start,
                    end, kv->max_len - 1);
    hipStream_t s = thread_stream();
    if (!s) return GLLM_EDEVICE;
    float* d = (float*)thread_scratch(1, (size_t)q_heads * hd * 2 * 4, s);
    if (!d) return scratch_error();
    GLLM_HIP(hipMemcpyAsync(d, q, (size_t)q_heads * hd * 4, hipMemcpyHostToDevice, s));
    // Present the group as a one-kv-head cache view starting at head kvh.
    gllm_hip_kv view = *kv;
    uint16_t* kp[1] = {kv->k[l] + (size_t)kvh * hd};
    uint16_t* vp[1] = {kv->v[l] + (size_t)kvh * vd};
    view.k = kp;
    view.v = vp;
    view.layers = 1;
    GLLM_TRY(attend_exact(&view, 0, d, q_heads, 1, hd, start, end, 1, scale,
                          d + (size_t)q_heads * hd, s, nullptr, nullptr, 0, nullptr, nullptr,
                          nullptr, nullptr, nullptr));
    GLLM_HIP(hipMemcpyAsync(out, d + (size_t)q_heads * hd, (size_t)q_heads * vd * 4,
                            hipMemcpyDeviceToHost, s));
    GLLM_HIP(hipStreamSynchronize(s));
    return GLLM_OK;
}

}  // extern "C"
