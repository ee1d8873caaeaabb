// gemv.hip -- Q4_K / Q6_K / Q8_0 x Q8K row kernels for gfx950, weight
// handles, and the matvec / argmax entry points of the C ABI.
//
// Lane mapping: eight consecutive lanes own one weight row; lane k plays the
// role of int32 lane k of the reference's 256-bit AVX2 accumulators
// (kernels_amd64.s:437-543, 1123-1220, 1321-1391).  For every 256-element
// block it loads the four (Q4_K), six (Q6_K) or eight (Q8_0) weight dwords
// whose bytes land in that AVX2 lane, forms the same exact int32 partial with
// v_dot4_i32_i8, and advances the same per-lane fp32 chains with fmaf in
// block order; the row ends with the reference's 8->4->2->1 tree.  The
// result is therefore bit-identical to the amd64 kernels.
#include <algorithm>
#include <mutex>
#include <string>
#include <vector>


#include <cstdlib>

#include "gllm_common.h"

namespace gllm {

constexpr int kRowsPerWG = 32;  // 256 threads / 8 lanes per row
constexpr int kMaxTok = 8;      // activation rows per launch
// Q4_K batches from this many activation rows run on the matrix cores (both
// paths give the same bits)
constexpr int kMfmaMinTok = 8;

bool float_dot_type(int t);
int launch_float_dot(int n, gllm_hip_weight* const* ws, const float* d_x, float* const* outs,
                     hipStream_t s);

struct ArgmaxOut {
    unsigned long long* keys;  // null: no argmax epilogue
    const uint32_t* recent;
    int n_recent;
    float penalty;
};

struct GemvJob {
    const uint8_t* w[3];
    float* out[3];
    int rows[3];
    int out_stride[3];
    int wg_begin[4];
    int n;
    int blocks;
    int cols;
    size_t rb;
    ActQ8 act;        // pre-quantised activations (unfused kernels)
    const float* xf;  // f32 activations when the kernel quantises them itself
    int rows_per_wg;  // rows per workgroup: blockDim.x / (8 * G)
    int tok0;         // first activation row of this launch
    int ntok;         // activation rows in this launch (<= NT)
    int sa;           // batch Q6_K / Q8_0: the launch's activations are staged in dynamic LDS
    // RMSNorm prologue (batch-1 Q4_K with xf): x = rmsNormInto(fma(res, 1,
    // xf), nw) computed in the kernel; res may be null; workgroup 0 writes
    // fma(res, 1, xf) to xout when xout is set
    const float* nw;
    const float* res;
    float* xout;
    float eps;
    // SwiGLU epilogue (gate/up group, batch 1): workgroups count finished
    // 256-row blocks in sq_cnt; the last of a block's 2 * 256 / rows_per_wg
    // workgroups quantises siluMulF32(out[0], out[1]) of the block into sq_act
    int* sq_cnt;
    ActQ8 sq_act;
    // greedy argmax epilogue (batch-1 Q6_K, one weight): keys[gridDim.x]
    // and the repeat-penalty window
    ArgmaxOut am;
};

__device__ __forceinline__ int sbyte(uint32_t w, int i) { return (int)(int8_t)(w >> (8 * i)); }
__device__ __forceinline__ int ubyte(uint32_t w, int i) { return (int)((w >> (8 * i)) & 0xffu); }

// Blocks per lane in flight in the Q6_K / Q8_0 row kernels.  Batch 1 keeps
// four for Q6_K (its activation operands ride in the same registers) and
// three for Q8_0; larger batches read the activations per token and keep
// two, which holds the VGPR count at the occupancy the memory stream needs.
// A batch-1 Q6_K launch of many workgroups or long rows takes three
// (gemv_q6k_kernel DQ = 3: 157 instead of 201 VGPRs, three waves per SIMD
// instead of two).  Measured in A/B runs on one box: the 128256 x 4096 head
// of the decode step 602.6 -> 605.0 tok/s, 4096 x 14336 22.6 -> 21.9 us;
// 14336 x 4096 (448 workgroups) 14.3 against 14.8 us keeps four.  Q8_0 at
// three: 4096 x 14336 17.6 -> 17.1 us, 14336 x 4096 unchanged.
template <int NT>
constexpr int kQ6Depth = NT == 1 ? 4 : 2;
template <int NT>
constexpr int kQ8Depth = NT == 1 ? 3 : 2;

__device__ __forceinline__ int locate(const GemvJob& j, int wg, int* wi) {
    int i = 0;
    while (i + 1 < j.n && wg >= j.wg_begin[i + 1]) i++;
    *wi = i;
    return (wg - j.wg_begin[i]) * j.rows_per_wg;
}

// ---------------------------------------------------------------------------
// Q4_K: 144-byte blocks [d f16][dmin f16][12 B 6-bit scales/mins][128 B
// nibbles] (simd.go:1530-1557).  AVX2 lane k covers bytes 4k..4k+3 of each of
// the four 32-byte nibble chunks (Q4KQ8CHUNK, kernels_amd64.s:443-455).  The
// upload repack stores those 16 bytes contiguously (nibble byte 32s + 4k + j
// moves to 16k + 4s + j) and moves the row's headers in front of its nibble
// blocks (q4k_hdr_off / q4k_nib_off; block size unchanged), so a lane reads
// its share of a block with one 16-byte load and the headers of eight blocks
// with another.
//
// G lanes share one AVX2 lane k of one row: lane g takes blocks g, g+G, ...
// and every round of G blocks advances the sequential fp32 chains through
// the G lanes with a quad-permute rotation (lane g adds its block to the
// value lane g-1 produced a step earlier), so the chains see the blocks in
// exactly the reference's order.
// ---------------------------------------------------------------------------

// rotate a value one lane up inside groups of G lanes (lane g receives g-1);
// quad_perm covers every lane, so no "old" value is needed
template <int G>
__device__ __forceinline__ float rot_prev(float v) {
    if constexpr (G == 1) {
        return v;
    } else if constexpr (G == 2) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
    } else {
        static_assert(G == 4, "G must be 1, 2 or 4");
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x93, 0xF, 0xF, false));
    }
}

// Value of lane GG of this lane's G-lane group (adjacent lanes; G = 2 or 4
// fits one DPP quad): quad_perm broadcast.
template <int G, int GG>
__device__ __forceinline__ float slot_bcast(float v) {
    if constexpr (G == 1) {
        return v;
    } else if constexpr (G == 2) {
        return __int_as_float(
            __builtin_amdgcn_mov_dpp(__float_as_int(v), GG == 0 ? 0xA0 : 0xF5, 0xF, 0xF, false));
    } else {
        static_assert(G == 4, "G must be 1, 2 or 4");
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), GG * 0x55, 0xF, 0xF, false));
    }
}

// One round of G blocks of the two sequential fp32 chains: lane g of a group
// holds block i*G + g's operands; every lane gathers the G lanes' operands
// (independent DPP reads, off the dependency chain) and advances its own copy
// of the chains through them in block order, so all G lanes end the round
// with the reference's chain values.
template <int G>
__device__ __forceinline__ void chain_gather(float iv, float dxs, float dmin, float mx,
                                             float& accF, float& accM) {
    if constexpr (G == 1) {
        accF = fmaf(iv, dxs, accF);
        accM = fmaf(dmin, mx, accM);
    } else {
        float a[G], b[G], c[G], e[G];
        a[0] = slot_bcast<G, 0>(iv); b[0] = slot_bcast<G, 0>(dxs);
        c[0] = slot_bcast<G, 0>(dmin); e[0] = slot_bcast<G, 0>(mx);
        a[1] = slot_bcast<G, 1>(iv); b[1] = slot_bcast<G, 1>(dxs);
        c[1] = slot_bcast<G, 1>(dmin); e[1] = slot_bcast<G, 1>(mx);
        if constexpr (G == 4) {
            a[2] = slot_bcast<G, 2>(iv); b[2] = slot_bcast<G, 2>(dxs);
            c[2] = slot_bcast<G, 2>(dmin); e[2] = slot_bcast<G, 2>(mx);
            a[3] = slot_bcast<G, 3>(iv); b[3] = slot_bcast<G, 3>(dxs);
            c[3] = slot_bcast<G, 3>(dmin); e[3] = slot_bcast<G, 3>(mx);
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            accF = fmaf(a[g], b[g], accF);
            accM = fmaf(c[g], e[g], accM);
        }
    }
}

// 8-lane tree across k when the k lanes of a row sit G lanes apart.
template <int G>
__device__ __forceinline__ float tree8_strided(float v) {
    if constexpr (G == 1) {
        return tree8(v);
    } else if constexpr (G == 2) {
        // lane (k, gi) = 2 k + gi of a 16-lane row; lane gi = 1 (k = 0) ends
        // with the sum: k reads k + 4 (row_shl:8), k ^ 1 (quad xor 2), k ^ 2
        // (row_shl:4); every operand lane lies inside the row
        v = v + dpp_f<kRowShl8>(v);
        v = v + dpp_f<kQuadXor2>(v);
        v = v + dpp_f<kRowShl4>(v);
        return v;
    } else {
        v = v + __shfl_xor(v, 4 * G, 8 * G);
        v = v + __shfl_xor(v, 1 * G, 8 * G);
        v = v + __shfl_xor(v, 2 * G, 8 * G);
        return v;
    }
}

__device__ __forceinline__ int mad24(int a, int b, int c) { return __mul24(a, b) + c; }

// Exact int8 dot of four byte pairs with a zero accumulator.  With clamp the
// compiler selects the VOP3P v_dot4_i32_i8 with an inline 0 (without it, the
// accumulating v_dot4c_i32_i8 behind a v_mov of the zero: one more VALU
// instruction per dot); the clamp never acts, as |dot| <= 4 * 15 * 127 or
// 4 * 127 * 127 at most.  VALU instructions are left to the compiler, which
// tracks the wait states a dot result needs before another VALU reads it;
// hand-written ones in inline assembly would bypass that.
__device__ __forceinline__ int dot4z(int a, int b) { return __builtin_amdgcn_sdot4(a, b, 0, true); }

// a * (byte N of s): a is a 14-bit signed dot and s holds 6-bit scales, so
// the 24-bit multiply (v_mul_i32_i24, full rate) is exact.
template <int N>
__device__ __forceinline__ int mul_byte(int a, uint32_t s) {
    return __mul24(a, (int)((s >> (8 * N)) & 0xffu));
}

// Q4_K lane sum sum_j sc_j * t_j from the eight dot4 results t_j: each
// |t_j| <= 4 * 15 * 127 = 7620 and each sc_j <= 63 fit signed 16 bits, so
// pairs (t_j, t_j+1) and (sc_j, sc_j+1) go through v_dot2_i32_i16 (exact
// int32, like the AVX2 VPMADDWD it replaces) instead of eight 24-bit
// multiplies of extracted scale bytes.
typedef short s16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ s16x2 pack16(int lo, int hi) {
    return __builtin_bit_cast(s16x2, __builtin_amdgcn_perm((uint32_t)hi, (uint32_t)lo, 0x05040100u));
}
// scale bytes (0, 1) or (2, 3) of s as two 16-bit halves
template <int N>
__device__ __forceinline__ s16x2 sc_pair(uint32_t s) {
    return __builtin_bit_cast(s16x2, __builtin_amdgcn_perm(0u, s, N == 0 ? 0x0c010c00u : 0x0c030c02u));
}
__device__ __forceinline__ int q4k_lane_sum(int t0, int t1, int t2, int t3, int t4, int t5, int t6,
                                            int t7, uint32_t sc03, uint32_t sc47) {
    // one accumulator chain (the integer sum is exact in any order; the first
    // step clamps only to take the VOP3P form with an inline zero, and
    // |sum| <= 8 * 7620 * 63 never saturates)
    int acc = __builtin_amdgcn_sdot2(pack16(t0, t1), sc_pair<0>(sc03), 0, true);
    acc = __builtin_amdgcn_sdot2(pack16(t2, t3), sc_pair<1>(sc03), acc, false);
    acc = __builtin_amdgcn_sdot2(pack16(t4, t5), sc_pair<0>(sc47), acc, false);
    return __builtin_amdgcn_sdot2(pack16(t6, t7), sc_pair<1>(sc47), acc, false);
}

__device__ __forceinline__ uint32_t ubfe(uint32_t v, uint32_t off, uint32_t width) {
    return __builtin_amdgcn_ubfe(v, off, width);
}

// Per-lane constants that extract m_k, the 6-bit min of sub-block k
// (getScaleMinK4, simd.go:1672-1677), from header dwords z = scales[4..7]
// and w = scales[8..11]:
//   k < 4:  m = z.byte(k) & 63
//   k >= 4: m = (w.byte(k-4) >> 4) | ((z.byte(k-4) >> 6) << 4)
// as m = bfe(k < 4 ? z : w, sa, wa) | (bfe(z, sb, wb) << 4) (width 0 gives 0).
struct MinSel {
    bool lo;
    uint32_t sa, wa, sb, wb;
    __device__ explicit MinSel(int k)
        : lo(k < 4),
          sa(k < 4 ? 8u * k : 8u * (k - 4) + 4u),
          wa(k < 4 ? 6u : 4u),
          sb(k < 4 ? 0u : 8u * (k - 4) + 6u),
          wb(k < 4 ? 0u : 2u) {}
    __device__ __forceinline__ uint32_t get(uint32_t z, uint32_t w) const {
        return ubfe(lo ? z : w, sa, wa) | (ubfe(z, sb, wb) << 4);
    }
};

typedef __attribute__((address_space(3))) void lds_void;

// Stage this launch's activations (q8, xs32, xscale of ntok tokens) into LDS
// with lds_copy16 / lds_copy4.  Layout: [NT*cols q8][NT*cols/32 xs32][NT*B
// xscale].  Every byte range is a multiple of the copy width.
template <int NT>
__device__ __forceinline__ void stage_act_asm(const GemvJob& j, uint8_t* smem) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nw = blockDim.x >> 6;
    const int cols = j.cols, B = j.blocks, nt = j.ntok;
    const uint8_t* gq = (const uint8_t*)(j.act.q8perm + (size_t)j.tok0 * cols);
    const int qbytes = nt * cols;
    for (int base = wave * 1024; base < qbytes; base += nw * 1024)
        if (base + lane * 16 < qbytes) lds_copy16(gq + base + lane * 16, lds_addr(smem + base));
    const uint8_t* gx = (const uint8_t*)(j.act.xs32 + (size_t)j.tok0 * (cols / 32));
    uint8_t* sx = smem + (size_t)NT * cols;
    const int xbytes = nt * (cols / 8);
    for (int base = wave * 1024; base < xbytes; base += nw * 1024)
        if (base + lane * 16 < xbytes) lds_copy16(gx + base + lane * 16, lds_addr(sx + base));
    const uint8_t* gs = (const uint8_t*)(j.act.xscale + (size_t)j.tok0 * B);
    uint8_t* ss = sx + (size_t)NT * (cols / 8);
    const int sbytes = nt * B * 4;
    for (int base = wave * 256; base < sbytes; base += nw * 256)
        if (base + lane * 4 < sbytes) lds_copy4(gs + base + lane * 4, lds_addr(ss + base));
}

// ---------------------------------------------------------------------------
// Q8K quantisation fused into a row kernel (batch 1): every workgroup turns
// the f32 activation into the LDS layout the row loop reads, evaluating
// q8kQuantize (quant_q8k_portable.go:36-62 == kernels_amd64.s:348-436) and
// sumF32Groups32 / sumF32Groups16 (kernels_amd64.s:208-254) exactly as
// q8k_prep_kernel does.  With nw waves (at least 4), wave w handles blocks
// w, w+nw, ...; in a block, lane
// (m = lane/8, kk = lane%8) holds x[32m + kk + 8i] for i = 0..3, i.e. the four
// addends of the reference's v_kk for 32-group m in their summation order.
// ---------------------------------------------------------------------------
template <int QB>  // blocks per wave, compile-time so the loads stay in registers
struct XRegs {
    float v[QB][4];
};

template <int QB, bool SKIP = false>
__device__ __forceinline__ void xq_load(const float* __restrict__ x, int B, XRegs<QB>& xr,
                                        int nw = -1) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (nw < 0) nw = blockDim.x >> 6;
    const int m = lane >> 3, kk = lane & 7;
#pragma unroll
    for (int i = 0; i < QB; i++) {
        const int b = wave + nw * i;
        // QB assumes four waves; wider workgroups own fewer blocks per wave.
        // SKIP: blocks past the end are not loaded (a wave-uniform branch
        // ahead of the weight prefetch, so the vmcnt waits stay exact; taken
        // by the norm prologue, which loads three rows: decode 473 -> 480
        // tok/s in a same-box A/B, and by eight-wave G = 4 launches such as
        // the attention output projection: 482 -> 487 tok/s); otherwise they
        // re-read the last block (the seven-wave batch-1 kernel of 14336 x
        // 4096 measured 1.5 % faster that way)
        if (SKIP && b >= B) break;
        const int bb = b < B ? b : B - 1;  // results of b >= B are not stored
        const float* g = x + (size_t)bb * 256 + 32 * m + kk;
#pragma unroll
        for (int e = 0; e < 4; e++) xr.v[i][e] = g[8 * e];
    }
}

// Quantise one 256-element block b held as x[32m + kk + 8e] = v[e] by lane
// (m = lane / 8, kk = lane % 8) into LDS: q8 (lane-permuted), xs32 and, for
// Q6_K / Q2_K (XS16), the per-16 sums xs16 at the given LDS arrays.
template <bool XS16>
__device__ __forceinline__ void xq_block(const float* xv, int b, int8_t* q8, float* xs32,
                                         float* xs16, float* xsc) {
    const int lane = threadIdx.x & 63;
    const int m = lane >> 3, kk = lane & 7;
    const float x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
    // amax, NaN skipped like the reference's `a > amax` scan: v_max_f32 is
    // IEEE maxNum, so the lane's max over |x| and 0 drops NaNs and is a
    // non-negative float, whose bits order like its value; the cross-lane
    // maximum then runs on the bits (integer max, no NaN canonicalisation).
    // A block of NaNs and zeros ends at 0, as the reference's amax does.
    const float a = fmaxf(fmaxf(fmaxf(fabsf(x0), fabsf(x1)), fmaxf(fabsf(x2), fabsf(x3))), 0.0f);
    const float amax = __uint_as_float(wave_max_u32(__float_as_uint(a)));
    const bool nz = amax != 0.0f;
    // scale = amax / 127 and inv = 127 / amax, both IEEE-rounded, in one
    // division: even lanes divide amax by 127, odd lanes 127 by amax
    const bool odd = lane & 1;
    const float quo = (odd ? 127.0f : amax) / (odd ? amax : 127.0f);
    const float scale = nz ? readlane_f(quo, 0) : 0.0f;
    const float inv = nz ? readlane_f(quo, 1) : 0.0f;
    // inv = 0 makes every q 0 (x * 0 is +-0, or NaN, which converts to 0)
    int8_t* qb = q8 + (size_t)b * 256 + 4 * m + (kk & 3) + 32 * (kk >> 2);
    qb[0] = (int8_t)(int)rintf(x0 * inv);
    qb[64] = (int8_t)(int)rintf(x1 * inv);
    qb[128] = (int8_t)(int)rintf(x2 * inv);
    qb[192] = (int8_t)(int)rintf(x3 * inv);
    if (lane == 0) xsc[b] = scale;
    // v_kk = ((x[kk] + x[8+kk]) + x[16+kk]) + x[24+kk]; a_k = v_k + v_{k+4};
    // r = (a0 + a1) + (a2 + a3): the 8 lanes kk of group m are lanes 8m..8m+7
    const float v = tree8(((x0 + x1) + x2) + x3);
    if (kk == 0) xs32[b * 8 + m] = v;
    if constexpr (XS16) {
        // 16-groups 2m (x0, x1) and 2m+1 (x2, x3): v_k = x[k] + x[8+k]
        const float u = tree8(x0 + x1), w = tree8(x2 + x3);
        if (kk == 0) {
            xs16[b * 16 + 2 * m] = u;
            xs16[b * 16 + 2 * m + 1] = w;
        }
    }
}

// Quantise the blocks held in xr (wave w holds blocks w, w + nw, ...).
template <int QB, bool XS16>
__device__ __forceinline__ void xq_store(const XRegs<QB>& xr, int B, int8_t* q8, float* xs32,
                                         float* xs16, float* xsc, int nw = -1) {
    const int wave = threadIdx.x >> 6;
    if (nw < 0) nw = blockDim.x >> 6;
#pragma unroll
    for (int i = 0; i < QB; i++) {
        const int b = wave + nw * i;
        if (b >= B) break;  // wave-uniform
        xq_block<XS16>(xr.v[i], b, q8, xs32, xs16, xsc);
    }
}

// LDS image of one quantised activation row for the batch-1 Q6_K, Q8_0 and
// other-format row kernels when they quantise x themselves (256-thread
// workgroups, cols <= kFuseCols: four waves of four blocks each).
constexpr int kFuseCols = 4096;
struct FusedAct {
    int8_t q8[kFuseCols];  // lane-permuted, as q8perm
    float xs32[kFuseCols / 32];
    float xs16[kFuseCols / 16];  // unscaled per-16 sums
    float xsc[kFuseCols / 256];
};
constexpr int kFuseQB = kFuseCols / 256 / 4;

// Fused prologue, part 2 (part 1 is xq_load<kFuseQB>, issued before the
// weight prefetch so its registers retire first): quantise into fa and make
// it visible to the workgroup without waiting for the weight loads.
template <bool XS16>
__device__ __forceinline__ void fused_act_store(const XRegs<kFuseQB>& xr, int B, FusedAct& fa) {
    xq_store<kFuseQB, XS16>(xr, B, fa.q8, fa.xs32, fa.xs16, fa.xsc);
    wait_lgkm0();
    lds_barrier();
}

// rmsNormInto (model.go:2986-3011) of x' = fma(res, 1, x) (addInPlace,
// model.go:3857) on an activation held in the xq_load layout (lane (m, kk)
// of the wave owning block b has x[256b + 32m + kk + 8e] in v[e]): x' is
// staged in LDS (xs: cols floats, then 48 floats of scratch), threads 0..31
// run the dotF32AVX2 accumulator chains (kernels_amd64.s:28-93: chain
// 8r + k over elements 32c + 8r + k, c in order), lanes 0..7 of wave 0
// join them as (y0 + y1) + (y2 + y3) and lane 0 runs the 8 -> 1 tree and
// float32(1 / sqrt(float64(ss / n + eps))), through cross-lane reads (one
// workgroup barrier for the scale instead of three); then
// v = (x' * w) * scale.
// Barriers are LDS-only, so the caller's weight prefetch stays in flight.
// xout (workgroup 0 only) receives x'.
template <int QB, bool RES>
__device__ __forceinline__ void norm_regs(XRegs<QB>& xr, const XRegs<QB>& wr,
                                          const XRegs<QB>& rr, int B, float eps, float* xout,
                                          float* xs) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
    const int m = lane >> 3, kk = lane & 7;
    const int n = B * 256;
#pragma unroll
    for (int i = 0; i < QB; i++) {
        const int b = wave + nw * i;
        if (b >= B) break;  // wave-uniform
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float v = xr.v[i][e];
            if constexpr (RES) v = fmaf(rr.v[i][e], 1.0f, v);
            xr.v[i][e] = v;
            const int idx = b * 256 + 32 * m + kk + 8 * e;
            xs[idx] = v;
            if (xout) xout[idx] = v;
        }
    }
    float* part = xs + n;
    wait_lgkm0();
    lds_barrier();
    if (tid < 32) {
        // chain 8r + k over elements 32c + 8r + k in c order, sixteen
        // elements per batch, the next batch's reads in flight meanwhile
        float y = 0.0f;
        float xa[16], xb[16];
        if (n % 512) {  // other sizes: the same chain, one element at a time
            for (int e = tid; e < n; e += 32) y = fmaf(xs[e], xs[e], y);
        } else {
#pragma unroll
            for (int u = 0; u < 16; u++) xa[u] = xs[32 * u + tid];
            int c = 0;
            for (; c + 1024 <= n; c += 1024) {
#pragma unroll
                for (int u = 0; u < 16; u++) xb[u] = xs[c + 512 + 32 * u + tid];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int u = 0; u < 16; u++) y = fmaf(xa[u], xa[u], y);
                __builtin_amdgcn_sched_barrier(0);
                if (c + 1024 < n) {
#pragma unroll
                    for (int u = 0; u < 16; u++) xa[u] = xs[c + 1024 + 32 * u + tid];
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int u = 0; u < 16; u++) y = fmaf(xb[u], xb[u], y);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (c < n) {  // an odd number of 512-element batches: xa holds the last
#pragma unroll
                for (int u = 0; u < 16; u++) y = fmaf(xa[u], xa[u], y);
            }
        }
        // the joins inside wave 0 (lanes 0..31 hold the chains), the same
        // additions in the same order: z_k = (y_k + y_8+k) + (y_16+k + y_24+k),
        // a_i = z_i + z_i+4, ss = (a_0 + a_1) + (a_2 + a_3)
        const float z = (y + __shfl_down(y, 8)) + (__shfl_down(y, 16) + __shfl_down(y, 24));
        const float a = z + __shfl_down(z, 4);
        const float hsum = a + __shfl_down(a, 1);
        const float ss = hsum + __shfl_down(hsum, 2);
        if (tid == 0) part[40] = (float)(1.0 / sqrt((double)(ss / (float)n + eps)));
    }
    wait_lgkm0();
    lds_barrier();
    const float scale = part[40];
#pragma unroll
    for (int i = 0; i < QB; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) xr.v[i][e] = (xr.v[i][e] * wr.v[i][e]) * scale;
}
constexpr size_t kNormLds = 48 * 4;  // norm scratch after the cols floats
// LDS offset of the norm's x' (after the quantised activation, 16-aligned)
__host__ __device__ constexpr size_t q4k_norm_off(int cols) {
    return ((size_t)cols + (size_t)(cols / 32) * 4 + (size_t)(cols / 256) * 4 + 15) & ~(size_t)15;
}

#include "gemv_formats.h"

// One Q4_K block of one AVX2 lane for NT tokens: exact int32 lane sum
//   accI_k = sum_j sc_j * dot4(nibbles of sub-block j in lane k, q8)
// then the fp32 chain steps (G-lane rotation when G > 1):
//   accF = fma(float(accI), d*xs, accF)          VMULSS + VFMADD231PS
//   accM = fma(dmin, m_k*xsum_k, accM)           VMULPS + VFMADD231PS
// Lane k's 32 nibbles of a block as eight dwords of four 4-bit values:
// n[2c] the low and n[2c + 1] the high nibbles of its chunk-c dword.
struct Nib8 {
    int n[8];
    __device__ __forceinline__ explicit Nib8(const uint4 q) {
        n[0] = (int)(q.x & 0x0f0f0f0fu); n[1] = (int)((q.x >> 4) & 0x0f0f0f0fu);
        n[2] = (int)(q.y & 0x0f0f0f0fu); n[3] = (int)((q.y >> 4) & 0x0f0f0f0fu);
        n[4] = (int)(q.z & 0x0f0f0f0fu); n[5] = (int)((q.z >> 4) & 0x0f0f0f0fu);
        n[6] = (int)(q.w & 0x0f0f0f0fu); n[7] = (int)((q.w >> 4) & 0x0f0f0f0fu);
    }
};

// The exact int32 lane sum of lane k's nibbles against its 32 q8 bytes at qp
// (two 16-byte LDS reads), with the block's 6-bit scales sc03 / sc47.
__device__ __forceinline__ int q4k_lane_int(const Nib8& w, const int8_t* qp, uint32_t sc03,
                                            uint32_t sc47) {
    const int4 qa = *(const int4*)qp;
    const int4 qb = *(const int4*)(qp + 16);
    return q4k_lane_sum(dot4z(w.n[0], qa.x), dot4z(w.n[1], qa.y), dot4z(w.n[2], qa.z),
                        dot4z(w.n[3], qa.w), dot4z(w.n[4], qb.x), dot4z(w.n[5], qb.y),
                        dot4z(w.n[6], qb.z), dot4z(w.n[7], qb.w), sc03, sc47);
}

__device__ __forceinline__ uint32_t q4k_sc03(const uint4 h) { return h.y & 0x3f3f3f3fu; }
__device__ __forceinline__ uint32_t q4k_sc47(const uint4 h) {
    return (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
}

template <int NT, int G>
__device__ __forceinline__ void q4k_block(const uint4 h, const uint4 q, int b, int k,
                                          const MinSel& ms, int ntok, const int8_t* q8b,
                                          const float* xs32b, const float* xscb, int cols, int B,
                                          float* accF, float* accM) {
    const float d = f16_bits_to_f32(h.x & 0xffffu);
    const float dmin = f16_bits_to_f32(h.x >> 16);
    const uint32_t sc03 = q4k_sc03(h), sc47 = q4k_sc47(h);
    const float mkf = (float)ms.get(h.z, h.w);
    const Nib8 w(q);
#pragma unroll
    for (int t = 0; t < NT; t++) {
        if (NT == 1 || t < ntok) {
            const int acc = q4k_lane_int(w, q8b + (size_t)t * cols + b * 256 + k * 32, sc03, sc47);
            const float iv = (float)acc;
            const float dxs = d * xscb[(size_t)t * B + b];
            const float mx = mkf * xs32b[(size_t)t * (cols / 32) + b * 8 + k];
            chain_gather<G>(iv, dxs, dmin, mx, accF[t], accM[t]);
        }
    }
}

// Header of lane-local block J (mod 8) of this lane's row and G-slot: the
// eight k-lanes of a (row, gi) group, G lanes apart, each loaded one block's
// header; ds_swizzle (bit mode, inside 32-lane halves) reads lane k = J of
// the group: and-mask keeps the row and gi bits, or-mask sets k.
template <int G>
constexpr int log2g() {
    return G == 1 ? 0 : G == 2 ? 1 : 2;
}
template <int G, int J>
__device__ __forceinline__ uint32_t hdr_bcast1(uint32_t v) {
    constexpr int lg = log2g<G>();
    constexpr int and_mask = 0x1f & ~(7 << lg);
    constexpr int or_mask = J << lg;
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, and_mask | (or_mask << 5));
}
template <int G, int J>
__device__ __forceinline__ uint4 hdr_bcast(uint4 v) {
    return make_uint4(hdr_bcast1<G, J>(v.x), hdr_bcast1<G, J>(v.y), hdr_bcast1<G, J>(v.z),
                      hdr_bcast1<G, J>(v.w));
}
template <int G>
__device__ __forceinline__ uint4 hdr_of(uint4 v, int j) {  // j: compile-time after unrolling
    switch (j & 7) {
    case 0: return hdr_bcast<G, 0>(v);
    case 1: return hdr_bcast<G, 1>(v);
    case 2: return hdr_bcast<G, 2>(v);
    case 3: return hdr_bcast<G, 3>(v);
    case 4: return hdr_bcast<G, 4>(v);
    case 5: return hdr_bcast<G, 5>(v);
    case 6: return hdr_bcast<G, 6>(v);
    default: return hdr_bcast<G, 7>(v);
    }
}

// Row kernel for compile-time blocks per lane NL (B = NL * G) and prefetch
// depth D (NL % D == 0): every weight load is unconditional straight-line
// code, D blocks per lane in flight.  A lane's block headers come from the
// row's header plane (q4k_hdr_off): lane k loads the header of its
// (8h + k)-th block for h = 0..NL/8, one 16-byte load per eight blocks, and
// the loop broadcasts block i's header from lane i % 8 of its group; the
// only per-block weight load is the lane's 16 nibble bytes.
//
// FUSE (batch 1 only): the workgroup quantises the f32 activation itself.
// Its x loads are issued first, the header and nibble prefetch second, so
// the compiler's in-order vmcnt waits hand the x registers to the quantiser
// while the weights are still streaming.  Otherwise the pre-quantised
// activations are copied to LDS with direct global->LDS loads issued before
// the prefetch.  FUSE = 2 (3 with a residual) puts the RMSNorm in front of
// the quantiser (norm_regs): the norm weights (and residual) are loaded with
// x, the LDS for x' follows the quantised activation.
template <int NT, int G, int NL, int D, int FUSE, bool SQ = false>
__global__ __launch_bounds__(FUSE || NL <= 8 ? 1024 : 512) void gemv_q4k_kernel(GemvJob j) {
    static_assert(NL % D == 0, "prefetch depth must divide the blocks per lane");
    static_assert(!FUSE || NT == 1, "fused quantisation is batch 1 only");
    constexpr bool NORM = FUSE >= 2;
    constexpr int B = NL * G;
    constexpr int NH = (NL + 7) / 8;  // header loads per lane
    constexpr int QB = FUSE ? (B + 3) / 4 : 1;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x;
    const int cols = B * 256;
    const int gi = tid % G, k = (tid / G) & 7, rl = tid / (8 * G);
    int wi = 0;
    while (wi + 1 < j.n && (int)blockIdx.x >= j.wg_begin[wi + 1]) wi++;
    const int r = ((int)blockIdx.x - j.wg_begin[wi]) * j.rows_per_wg + rl;
    const bool live = r < j.rows[wi];
    const int rr = live ? r : j.rows[wi] - 1;  // dead lanes read a valid row, write nothing
    const uint8_t* row = j.w[wi] + (size_t)rr * j.rb;
    const uint8_t* lane_nib = row + q4k_nib_off(B, gi) + 16 * k;  // block i: + i * G * 128
    int8_t* q8b = (int8_t*)smem;
    float* xs32b = (float*)(smem + (size_t)NT * cols);
    float* xscb = xs32b + (size_t)NT * (cols / 32);
    XRegs<QB> xr;
    XRegs<NORM ? QB : 1> wr, resr;
    if constexpr (FUSE) {
        xq_load<QB, NORM || G == 4>(j.xf + (size_t)j.tok0 * cols, B, xr);
        if constexpr (NORM) xq_load<QB, true>(j.nw, B, wr);
        if constexpr (FUSE == 3) xq_load<QB, true>(j.res, B, resr);
    } else {
        stage_act_asm<NT>(j, smem);
    }
    __builtin_amdgcn_sched_barrier(0);
    uint4 HG[NH];
#pragma unroll
    for (int h = 0; h < NH; h++) {
        const int i = 8 * h + k < NL ? 8 * h + k : NL - 1;  // clamped lanes are never read
        HG[h] = *(const uint4*)(row + q4k_hdr_off(i * G + gi));
    }
    __builtin_amdgcn_sched_barrier(0);
    // nibble loads pinned in block order: vmcnt retires in issue order, so
    // block i is usable as soon as its own data is in
    uint4 Q[D];
#pragma unroll
    for (int i = 0; i < D; i++) {
        Q[i] = *(const uint4*)(lane_nib + (size_t)i * G * 128);
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (FUSE) {
        if constexpr (NORM)
            norm_regs<QB, FUSE == 3>(xr, wr, resr, B, j.eps, blockIdx.x == 0 ? j.xout : nullptr,
                                     (float*)(smem + q4k_norm_off(cols)));
        xq_store<QB, false>(xr, B, q8b, xs32b, nullptr, xscb);
        wait_lgkm0();
    } else {
        wait_vmem_le<NH + D>();
    }
    lds_barrier();
    const MinSel ms(k);
    float accF[NT], accM[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) accF[t] = accM[t] = 0.0f;
#pragma unroll
    for (int i0 = 0; i0 < NL; i0 += D) {
#pragma unroll
        for (int ii = 0; ii < D; ii++) {
            const int i = i0 + ii;
            const uint4 q = Q[ii];
            const uint4 h = hdr_of<G>(HG[i / 8], i);
            if (i0 + D < NL) Q[ii] = *(const uint4*)(lane_nib + (size_t)(i + D) * G * 128);
            q4k_block<NT, G>(h, q, i * G + gi, k, ms, j.ntok, q8b, xs32b, xscb, cols, B, accF,
                             accM);
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const float v = tree8_strided<G>(accF[t] - accM[t]);  // VSUBPS + tree
        if (live && k == 0 && gi == G - 1 && t < j.ntok) {
            float* o = &j.out[wi][(size_t)(j.tok0 + t) * j.out_stride[wi] + r];
            if constexpr (SQ) __hip_atomic_store(o, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            else *o = v;
        }
    }
    if constexpr (SQ) {
        // the FFN's SwiGLU + Q8K for the down projection (q8k_prep_kernel's
        // work) by the last workgroup to finish each 256-row block: stores
        // made visible device-wide, then one counter increment per workgroup
        __shared__ int s_last;
        __shared__ float sq_x[256];
        __shared__ float sq_max[4];
        // The outputs above are system-scope stores (written through past
        // the XCD's L2); every thread waits for its stores to complete before
        // the barrier, then one system-scope counter increment per
        // workgroup; the last workgroup reads the block with system-scope
        // loads.  No cache-wide writeback or invalidate is needed.
        //
        // Memory model.  In HIP terms the counter is a relaxed atomic, which
        // orders nothing; the handoff rests on what gfx950 does with these
        // instructions instead:
        //  * a system-scope relaxed store is a global_store with sc0 sc1:
        //    it writes through the XCD's L2 to memory (MALL / HBM), and its
        //    vmcnt decrement means memory has acknowledged it;
        //  * s_waitcnt vmcnt(0) in every thread, then s_barrier, so the
        //    counter's atomic (issued after the barrier) leaves the CU only
        //    once all 256 rows of this workgroup's stores are in memory;
        //  * the system-scope atomic add executes at memory, so the workgroup
        //    that reads total - 1 from it does so after every other
        //    workgroup's rows were acknowledged there;
        //  * that workgroup's system-scope loads (sc0 sc1) miss the
        //    non-coherent L2 copies and read memory.
        // A release / acquire pair at agent scope would give the same order
        // through the HIP model, but on this part it writes back (release)
        // and invalidates (acquire) the whole XCD L2: 36 us per launch
        // against 18.4 us for this form.  The decode parity tests
        // (tests/test_gpu_model.py, the SwiGLU epilogue cases) exercise it.
        const int blk = (((int)blockIdx.x - j.wg_begin[wi]) * j.rows_per_wg) / 256;
        wait_vmem_le<0>();  // this thread's output stores have completed
        __syncthreads();
        if (threadIdx.x == 0) {
            const int total = 2 * (256 / j.rows_per_wg);
            s_last = __hip_atomic_fetch_add(&j.sq_cnt[blk], 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_SYSTEM) == total - 1;
        }
        __syncthreads();
        if (s_last) {
            silu_q8_block<true>(j.out[0], j.out[1], blk, j.sq_act, sq_x, sq_max);
            if (threadIdx.x == 0)  // ready for the next step
                __hip_atomic_store(&j.sq_cnt[blk], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

// Any block count (B % G == 0): runtime trip count, activations read from
// global memory.  Used for shapes without a compiled NL.
template <int NT, int G>
__global__ __launch_bounds__(256) void gemv_q4k_any_kernel(GemvJob j) {
    const int tid = threadIdx.x;
    const int B = j.blocks, cols = j.cols;
    const int gi = tid % G, k = (tid / G) & 7, rl = tid / (8 * G);
    int wi = 0;
    while (wi + 1 < j.n && (int)blockIdx.x >= j.wg_begin[wi + 1]) wi++;
    const int r = ((int)blockIdx.x - j.wg_begin[wi]) * (32 / G) + rl;
    if (r >= j.rows[wi]) return;
    const uint8_t* row = j.w[wi] + (size_t)r * j.rb;
    const int8_t* q8b = j.act.q8perm + (size_t)j.tok0 * cols;
    const float* xs32b = j.act.xs32 + (size_t)j.tok0 * (cols / 32);
    const float* xscb = j.act.xscale + (size_t)j.tok0 * B;
    const MinSel ms(k);
    float accF[NT], accM[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) accF[t] = accM[t] = 0.0f;
    for (int i = 0; i < B / G; i++) {
        const int b = i * G + gi;
        q4k_block<NT, G>(*(const uint4*)(row + q4k_hdr_off(b)),
                         *(const uint4*)(row + q4k_nib_off(B, b) + 16 * k), b, k, ms, j.ntok, q8b,
                         xs32b, xscb, cols, B, accF, accM);
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const float v = tree8_strided<G>(accF[t] - accM[t]);
        if (k == 0 && gi == G - 1 && t < j.ntok)
            j.out[wi][(size_t)(j.tok0 + t) * j.out_stride[wi] + r] = v;
    }
}
// ---------------------------------------------------------------------------
// Block-parallel batch-1 Q4_K row kernel.  Of a row dot, only the two fp32
// chains per AVX2 lane k (accF, accM: one step per block, in block order)
// and the final 8->4->2->1 tree are sequential; the four chain operands of a
// block -- float(exact int32 lane sum), d * xscale, dmin and m_k * xs32 --
// depend on that block alone.  NS slices of eight lanes therefore share a
// row: slice s forms the operands of blocks s, s + NS, s + 2 NS, ... (its NB
// = B / NS nibble loads all issued at entry, headers broadcast from the
// 16-byte header plane as in gemv_q4k_kernel) and stores them to LDS at
// X[row][block][k]; after one barrier thread (row, k) runs the two chains
// over the row's B blocks in block order and the tree.  The operands, the
// chains and the tree are the row kernel's, so the bits are the same; the
// slices give a compute unit NS times the waves over the same rows, with the
// whole weight slice in flight from the start.
//
// FUSE = 1: the workgroup quantises x itself (xq_load issued before the
// weight loads, as in gemv_q4k_kernel); FUSE = 2 (3 with a residual): the
// RMSNorm runs in front of the quantiser (norm_regs, as in gemv_q4k_kernel);
// FUSE = 0: pre-quantised activations copied to LDS with direct global->LDS
// loads.
// ---------------------------------------------------------------------------
// Rows per workgroup of a launch shape: NTH / (8 NS) row groups, RP rows
// per lane.
__host__ __device__ constexpr int q4k_bp_rows(int ns, int nth, int rp) { return nth / (8 * ns) * rp; }
// float4 stride of one row of the exchange: B blocks x 8 lanes, padded by 8
// so the chain pass's reads (two rows per 16 lanes) fall in distinct banks
__host__ __device__ constexpr int q4k_bp_xstride(int B) { return B * 8 + 8; }
// LDS: the activation image, then the exchange X[rows][xstride] of float4
__host__ __device__ constexpr size_t q4k_bp_lds(int B, int ns, int nth, int rp) {
    return q4k_norm_off(B * 256) + (size_t)q4k_bp_rows(ns, nth, rp) * q4k_bp_xstride(B) * 16;
}

// Decoded header of one Q4_K block for AVX2 lane k: d, dmin, the eight
// 6-bit scales as two byte-packed dwords and m_k (getScaleMinK4).
struct Q4KHdr {
    float d, dmin, mk;
    uint32_t sc03, sc47;
    __device__ __forceinline__ Q4KHdr() = default;
    __device__ __forceinline__ Q4KHdr(const uint4 h, const MinSel& ms)
        : d(f16_bits_to_f32(h.x & 0xffffu)),
          dmin(f16_bits_to_f32(h.x >> 16)),
          mk((float)ms.get(h.z, h.w)),
          sc03(q4k_sc03(h)),
          sc47(q4k_sc47(h)) {}
};

// Lane (row group g, slice s, k) owns rows r0 + g + R p (p < RP) and, of
// each, blocks s, s + NS, ..., s + NS (NB - 1).  Load order: the headers,
// then x (or the staged activations), then P blocks per row; the wave then
// waits for its own x and issues the rest of its weights before quantising.
// Every wave's x request thus enters the memory system ahead of any weight
// flood but the P blocks (an x read queued behind a full flood arrives
// microseconds late), and the weight stream starts as soon as x is in,
// not after the workgroup's quantiser barrier.
template <int B, int NS, int NTH, int RP, int FUSE, int P>
__global__ __launch_bounds__(NTH) void gemv_q4k_bp_kernel(GemvJob j) {
    constexpr int NB = B / NS;
    static_assert(B % NS == 0 && NTH % (8 * NS) == 0 && NTH % 64 == 0, "launch shape");
    static_assert(NB <= 8, "one header load per lane and row");
    static_assert(P >= 0 && P <= NB, "blocks before the quantiser");
    constexpr int R = NTH / (8 * NS);
    constexpr int RW = R * RP;
    constexpr int NW = NTH / 64;
    constexpr int QB = FUSE ? (B + NW - 1) / NW : 1;
    constexpr bool NORM = FUSE >= 2;
    constexpr int cols = B * 256;
    constexpr int XS = q4k_bp_xstride(B);
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x;
    const int k = tid & 7, u = tid >> 3, s = u % NS, g = u / NS;
    // the launch's weights' rows laid end to end (a workgroup may straddle
    // two of them): Q, K and V of 4096 + 1024 + 1024 rows fill 256
    // workgroups of 24 rows where per-weight workgroups would need 257
    const int r0 = (int)blockIdx.x * RW;
    const int n1 = j.rows[0], n2 = j.n > 1 ? n1 + j.rows[1] : n1;
    const int nrows = j.n > 2 ? n2 + j.rows[2] : n2;
    const uint8_t* rowp[RP];
#pragma unroll
    for (int p = 0; p < RP; p++) {
        int r = r0 + g + R * p;
        r = r < nrows ? r : nrows - 1;  // dead rows read a valid row
        rowp[p] = r < n1 ? j.w[0] + (size_t)r * j.rb
                : r < n2 ? j.w[1] + (size_t)(r - n1) * j.rb
                         : j.w[2] + (size_t)(r - n2) * j.rb;
    }
    int8_t* q8b = (int8_t*)smem;
    float* xs32b = (float*)(smem + cols);
    float* xscb = xs32b + cols / 32;
    float4* X = (float4*)(smem + q4k_norm_off(cols));
    uint4 H[RP];
#pragma unroll
    for (int p = 0; p < RP; p++)
        H[p] = *(const uint4*)(rowp[p] + q4k_hdr_off(NS * (k < NB ? k : NB - 1) + s));
    __builtin_amdgcn_sched_barrier(0);
    XRegs<QB> xr;
    XRegs<NORM ? QB : 1> wr, resr;
    if constexpr (FUSE) {
        xq_load<QB, true>(j.xf, B, xr);
        if constexpr (NORM) xq_load<QB, true>(j.nw, B, wr);
        if constexpr (FUSE == 3) xq_load<QB, true>(j.res, B, resr);
    } else {
        stage_act_asm<1>(j, smem);
    }
    __builtin_amdgcn_sched_barrier(0);
    uint4 Q[NB][RP];
    const size_t nib0 = q4k_nib_off(B, s) + 16 * k;  // block NS i + s at + NS i 128
#pragma unroll
    for (int i = 0; i < P; i++)
#pragma unroll
        for (int p = 0; p < RP; p++) {
            Q[i][p] = *(const uint4*)(rowp[p] + nib0 + (size_t)i * NS * 128);
            __builtin_amdgcn_sched_barrier(0);
        }
    wait_vmem_le<P * RP>();  // this wave's headers and x, norm weights, residual (or staged activations)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = P; i < NB; i++)
#pragma unroll
        for (int p = 0; p < RP; p++) {
            Q[i][p] = *(const uint4*)(rowp[p] + nib0 + (size_t)i * NS * 128);
            __builtin_amdgcn_sched_barrier(0);
        }
    const MinSel ms(k);
    Q4KHdr hd[NB][RP];
#pragma unroll
    for (int i = 0; i < NB; i++)
#pragma unroll
        for (int p = 0; p < RP; p++) hd[i][p] = Q4KHdr(hdr_of<1>(H[p], i), ms);
    if constexpr (NORM)  // x' staged over the exchange, which is written after the barrier below
        norm_regs<QB, FUSE == 3>(xr, wr, resr, B, j.eps, blockIdx.x == 0 ? j.xout : nullptr,
                                 (float*)X);
    if constexpr (FUSE) xq_store<QB, false>(xr, B, q8b, xs32b, nullptr, xscb);
    wait_lgkm0();
    lds_barrier();
    // this lane's operands: block NS i + s at a compile-time offset from here
    const int8_t* q8s = q8b + s * 256 + k * 32;
    const float* x32s = xs32b + s * 8 + k;
    const float* xscs = xscb + s;
    float4* xo = X + (size_t)g * XS + s * 8 + k;
#pragma unroll
    for (int i = 0; i < NB; i++)
#pragma unroll
        for (int p = 0; p < RP; p++) {
            const Nib8 w(Q[i][p]);
            const Q4KHdr& h = hd[i][p];
            const int acc = q4k_lane_int(w, q8s + i * NS * 256, h.sc03, h.sc47);
            xo[(size_t)R * p * XS + i * NS * 8] =
                make_float4((float)acc, h.d * xscs[i * NS], h.dmin, h.mk * x32s[i * NS * 8]);
        }
    __syncthreads();
#pragma unroll
    for (int t0 = 0; t0 < 8 * RW; t0 += NTH) {
        const int t = t0 + tid;
        if (t0 + NTH <= 8 * RW || t < 8 * RW) {
            const int cr = t >> 3;
            const float4* xp = X + (size_t)cr * XS + k;
            float accF = 0.0f, accM = 0.0f;
#pragma unroll
            for (int b = 0; b < B; b++) {
                const float4 v = xp[b * 8];
                accF = fmaf(v.x, v.y, accF);  // VMULSS + VFMADD231PS
                accM = fmaf(v.z, v.w, accM);  // VMULPS + VFMADD231PS
            }
            const float v = tree8(accF - accM);  // VSUBPS + tree
            const int r = r0 + cr;
            if (k == 0 && r < nrows) {
                float* o = r < n1 ? j.out[0] + r : r < n2 ? j.out[1] + (r - n1) : j.out[2] + (r - n2);
                *o = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Wave-specialised batch-1 Q4_K row kernel.  A workgroup owns R rows (one
// workgroup per compute unit at the configs' shapes).  Its last NLD waves
// are loaders: they copy the rows' header planes and nibble blocks straight
// from HBM into LDS (global_load_lds_dwordx4, no registers held) and set a
// per-block flag in LDS once a block's copies have landed (an exact vmcnt
// wait: copies retire in issue order).  The other waves compute, eight lanes
// per row as in gemv_q4k_kernel (AVX2 lane k, chains in block order, the
// 8->4->2->1 tree), so the bits are that kernel's: they quantise x, then
// walk the blocks as they land, reading nibbles, headers and activations
// from LDS.  With NS = 2 a row's lanes come in two slices: slice 1 forms
// the chain operands of the second half of the blocks while slice 0 runs
// the chains over the first half, then continues them from slice 0's values
// (handed over through LDS), so the chains still see every block in order.
//
// Only the loaders ever wait on HBM: a wave issuing a compute unit's whole
// weight slice stalls on issue once the memory queues fill, which here
// never holds up the arithmetic.  The compute waves' x reads are issued at
// entry, ahead of the copies in the compute unit's queue.
//
// LDS: activations (q8 | xs32 | xscale), headers [R][B + 1][16 B] (one
// padding slot per row keeps two rows' broadcast reads in distinct banks),
// nibbles [B][R][k][16 B], B block flags, the compute barrier's counter and
// the chain handover [R][k][2] floats.
// ---------------------------------------------------------------------------
template <int B, int R>
struct Q4KWsLayout {
    static constexpr int cols = B * 256;
    static constexpr int hslots = R * (B + 1);  // header slots, 16 B each
    static constexpr size_t hdr = q4k_norm_off(cols);
    static constexpr size_t nib = hdr + ((size_t)hslots * 16 + 1023) / 1024 * 1024;
    static constexpr size_t flags = nib + (size_t)B * R * 128;
    static constexpr size_t count = flags + (size_t)B * 4;
    static constexpr size_t hand = count + 64;
    static constexpr size_t bytes = hand + (size_t)R * 8 * 8;
};

// Copy order of the blocks: with two slices the halves interleave (0,
// B/2, 1, B/2 + 1, ...) so both slices are fed from the start (slice 0's
// blocks first measured 9.03 against 8.80 us at 14336 x 4096).
template <int B, int NS>
__device__ __forceinline__ constexpr int ws_block(int pos) {
    return NS == 1 ? pos : (pos & 1) ? B / 2 + pos / 2 : pos / 2;
}

// Loader LW copies the header slots n = LW, LW + NLD, ... (1 KB each), then
// the blocks at copy positions LW, LW + NLD, ... (R / 8 copies each), and
// sets a block's flag once its copies have completed, keeping up to D
// blocks in flight before it waits.  Its one workgroup barrier comes after
// its first D blocks' copies, before its first flag store.
template <int B, int R, int NS, int NLD, int D, int LW, int I>
__device__ __forceinline__ void ws_loader_blocks(const uint8_t* __restrict__ w, size_t rb, int r0,
                                                 int nrows, uint8_t* smem) {
    using L = Q4KWsLayout<B, R>;
    constexpr int PER = R / 8;
    constexpr int NBW = (B - LW + NLD - 1) / NLD;
    if constexpr (I < NBW + D) {
        const int lane = threadIdx.x & 63, rl = lane >> 3, k = lane & 7;
        if constexpr (I < NBW) {
            constexpr int b = ws_block<B, NS>(LW + NLD * I);
#pragma unroll
            for (int c = 0; c < PER; c++) {
                const int r = r0 + 8 * c + rl;
                const uint8_t* g =
                    w + (size_t)(r < nrows ? r : nrows - 1) * rb + q4k_nib_off(B, b) + 16 * k;
                lds_copy16(g, lds_addr(smem + L::nib + ((size_t)b * R + 8 * c) * 128));
            }
        }
        if constexpr (I >= D) {
            // the workgroup barrier that orders the flag clears before any
            // flag store: a loader takes it here, after its first copies
            if constexpr (I == D) lds_barrier();
            // block I - D is complete once at most the copies issued after it remain
            constexpr int after = (I < NBW ? I : NBW - 1) - (I - D);
            wait_vmem_le<after * PER>();
            asm volatile("" ::: "memory");
            if (lane == 0) {
                int* flag = (int*)(smem + L::flags) + ws_block<B, NS>(LW + NLD * (I - D));
                __hip_atomic_store(flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
        ws_loader_blocks<B, R, NS, NLD, D, LW, I + 1>(w, rb, r0, nrows, smem);
    }
}

template <int B, int R, int NS, int NLD, int D, int LW>
__device__ __forceinline__ void q4k_ws_loader(const uint8_t* __restrict__ w, size_t rb, int r0,
                                              int nrows, uint8_t* smem) {
    using L = Q4KWsLayout<B, R>;
    constexpr int HI = (L::hslots + 63) / 64;
    const int lane = threadIdx.x & 63;
    // header slot t = r (B + 1) + b: row r's header b (b == B: padding)
#pragma unroll
    for (int n = LW; n < HI; n += NLD) {
        const int t = n * 64 + lane;
        const int r = t / (B + 1), b = t % (B + 1);
        const int rr = r0 + r < nrows ? r0 + r : nrows - 1;
        const uint8_t* g = w + (size_t)rr * rb + q4k_hdr_off(b < B ? b : 0);
        if (t < L::hslots) lds_copy16(g, lds_addr(smem + L::hdr + (size_t)n * 1024));
    }
    // copies retire in issue order: the flag of this loader's first block
    // also covers its header copies
    ws_loader_blocks<B, R, NS, NLD, D, LW, 0>(w, rb, r0, nrows, smem);
}

// One weight, plain arguments (the command processor can preload them into
// SGPRs, where a GemvJob by value is read with scalar loads first): the
// rows' weights w (row bytes rb), f32 x, out[nrows].
template <int B, int R, int NS, int NLD, int D>
__global__ __launch_bounds__(R * 8 * NS + NLD * 64) void gemv_q4k_ws_kernel(
    const uint8_t* __restrict__ w, const float* __restrict__ xf, float* __restrict__ out, int nrows,
    int rb) {
    using L = Q4KWsLayout<B, R>;
    constexpr int NCW = R * NS / 8;  // compute waves
    constexpr int QB = (B + NCW - 1) / NCW;
    constexpr int cols = B * 256;
    constexpr int BS = B / NS;  // blocks per slice
    static_assert(R % 8 == 0 && B % NS == 0 && (NS == 1 || NS == 2), "workgroup shape");
    static_assert(L::bytes <= 160 * 1024 - 64, "LDS");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r0 = (int)blockIdx.x * R;
    int* flags = (int*)(smem + L::flags);
    int* count = (int*)(smem + L::count);  // [0]: compute barrier, [1 + w]: handover of wave w
    XRegs<QB> xr;
    if (wave < NCW) xq_load<QB, true>(xf, B, xr, NCW);  // x first, ahead of every copy
    // LDS holds whatever an earlier workgroup left: clear the flags and the
    // counters before anyone sets or reads them
    if (tid < B) __hip_atomic_store(flags + tid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (tid < 16) __hip_atomic_store(count + tid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    // the loaders' copies go out at once (the copies touch neither the flags
    // nor the counters); each loader takes the barrier below inside its
    // block loop, before its first flag store
    if (wave >= NCW) {
        if constexpr (NLD > 0) if (wave == NCW + 0) q4k_ws_loader<B, R, NS, NLD, D, 0>(w, rb, r0, nrows, smem);
        if constexpr (NLD > 1) if (wave == NCW + 1) q4k_ws_loader<B, R, NS, NLD, D, 1>(w, rb, r0, nrows, smem);
        if constexpr (NLD > 2) if (wave == NCW + 2) q4k_ws_loader<B, R, NS, NLD, D, 2>(w, rb, r0, nrows, smem);
        if constexpr (NLD > 3) if (wave == NCW + 3) q4k_ws_loader<B, R, NS, NLD, D, 3>(w, rb, r0, nrows, smem);
        return;
    }
    wait_lgkm0();
    lds_barrier();
    int8_t* q8b = (int8_t*)smem;
    float* xs32b = (float*)(smem + cols);
    float* xscb = xs32b + cols / 32;
    xq_store<QB, false>(xr, B, q8b, xs32b, nullptr, xscb, NCW);
    // barrier of the compute waves only (the loaders never wait for them)
    wait_lgkm0();
    if ((tid & 63) == 0) __hip_atomic_fetch_add(count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    while (__hip_atomic_load(count, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < NCW)
        __builtin_amdgcn_s_sleep(1);
    const int sl = NS == 1 ? 0 : tid / (R * 8);  // slice
    const int rl = (tid >> 3) % R, k = tid & 7;
    const MinSel ms(k);
    const uint8_t* hrow = smem + L::hdr + (size_t)rl * (B + 1) * 16;
    const uint8_t* nrow = smem + L::nib + (size_t)rl * 128 + 16 * k;
    auto ready = [&](int b) {
        while (__hip_atomic_load(flags + b, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == 0)
            __builtin_amdgcn_s_sleep(1);
    };
    // every loader's headers: the first block each of them flags
#pragma unroll
    for (int l = 0; l < NLD; l++) ready(ws_block<B, NS>(l));
    const int b0 = sl * BS;
    float accF = 0.0f, accM = 0.0f;
    // chain operands of slice 1's blocks, held until slice 0's chains arrive
    float oI[NS == 2 ? BS : 1], oD[NS == 2 ? BS : 1], oN[NS == 2 ? BS : 1], oX[NS == 2 ? BS : 1];
    // the LDS operands of one block, read a block ahead of their use
    struct Ops {
        uint4 h, q;
        int4 qa, qb;
        float xsc, x32;
    };
    auto fetch = [&](int b) {
        Ops o;
        o.h = *(const uint4*)(hrow + b * 16);
        o.q = *(const uint4*)(nrow + (size_t)b * R * 128);
        const int8_t* qp = q8b + b * 256 + k * 32;
        o.qa = *(const int4*)qp;
        o.qb = *(const int4*)(qp + 16);
        o.xsc = xscb[b];
        o.x32 = xs32b[b * 8 + k];
        return o;
    };
    ready(b0);
    Ops cur = fetch(b0);
#pragma unroll
    for (int i = 0; i < BS; i++) {
        const int b = b0 + i;
        Ops nxt = cur;
        if (i + 1 < BS) {
            ready(b + 1);
            nxt = fetch(b + 1);
        }
        const Q4KHdr hd(cur.h, ms);
        const Nib8 wn(cur.q);
        const int acc = q4k_lane_sum(dot4z(wn.n[0], cur.qa.x), dot4z(wn.n[1], cur.qa.y),
                                     dot4z(wn.n[2], cur.qa.z), dot4z(wn.n[3], cur.qa.w),
                                     dot4z(wn.n[4], cur.qb.x), dot4z(wn.n[5], cur.qb.y),
                                     dot4z(wn.n[6], cur.qb.z), dot4z(wn.n[7], cur.qb.w), hd.sc03,
                                     hd.sc47);
        const float iv = (float)acc, dxs = hd.d * cur.xsc, mx = hd.mk * cur.x32;
        if (NS == 1 || sl == 0) {
            accF = fmaf(iv, dxs, accF);      // VMULSS + VFMADD231PS
            accM = fmaf(hd.dmin, mx, accM);  // VMULPS + VFMADD231PS
        } else {
            oI[NS == 2 ? i : 0] = iv;
            oD[NS == 2 ? i : 0] = dxs;
            oN[NS == 2 ? i : 0] = hd.dmin;
            oX[NS == 2 ? i : 0] = mx;
        }
        cur = nxt;
    }
    if constexpr (NS == 2) {
        float2* hand = (float2*)(smem + L::hand) + rl * 8 + k;
        const int hw = 1 + (wave % (NCW / 2));  // the slice-0 wave over the same rows
        if (sl == 0) {
            *hand = make_float2(accF, accM);
            wait_lgkm0();
            if ((tid & 63) == 0)
                __hip_atomic_store(count + hw, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            return;
        }
        while (__hip_atomic_load(count + hw, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == 0)
            __builtin_amdgcn_s_sleep(1);
        const float2 a = *hand;
        accF = a.x;
        accM = a.y;
#pragma unroll
        for (int i = 0; i < BS; i++) {
            accF = fmaf(oI[i], oD[i], accF);  // VMULSS + VFMADD231PS
            accM = fmaf(oN[i], oX[i], accM);  // VMULPS + VFMADD231PS
        }
    }
    const float v = tree8(accF - accM);  // VSUBPS + tree
    if (k == 0 && r0 + rl < nrows) out[r0 + rl] = v;
}

// Batch launches of the Q6_K / Q8_0 row kernels (j.sa): the launch's ntok
// activation rows (q8, xscale and, for Q6_K, xs16) are copied into dynamic
// LDS once per workgroup, so the per-token operands of every block come from
// LDS instead of ntok rounds of global loads per block.  Layout: q8 [ntok][cols],
// then xscale [ntok][B], then xs16 [ntok][cols / 16], each 16-byte aligned.
struct StagedAct {
    const int8_t* q8;
    const float* xsc;
    const float* xs16;
};

__host__ __device__ inline size_t staged_act_bytes(int ntok, int cols, bool xs16) {
    const size_t q = (size_t)ntok * cols, x = ((size_t)ntok * (cols / 256) * 4 + 15) & ~(size_t)15;
    return q + x + (xs16 ? (size_t)ntok * (cols / 16) * 4 : 0);
}

__device__ __forceinline__ StagedAct stage_act(const GemvJob& j, uint8_t* lds, bool xs16) {
    const int B = j.blocks, nt = j.ntok, tid = threadIdx.x;
    const size_t nq = (size_t)nt * j.cols, nx = ((size_t)nt * B * 4 + 15) & ~(size_t)15;
    const uint4* q = (const uint4*)(j.act.q8perm + (size_t)j.tok0 * j.cols);
    for (size_t i = tid; i < nq / 16; i += 256) ((uint4*)lds)[i] = q[i];
    const float* xsc = j.act.xscale + (size_t)j.tok0 * B;
    for (int i = tid; i < nt * B; i += 256) ((float*)(lds + nq))[i] = xsc[i];
    if (xs16) {
        const uint4* x = (const uint4*)(j.act.xs16 + (size_t)j.tok0 * (j.cols / 16));
        for (int i = tid; i < nt * j.cols / 64; i += 256) ((uint4*)(lds + nq + nx))[i] = x[i];
    }
    __syncthreads();
    return StagedAct{(const int8_t*)lds, (const float*)(lds + nq), (const float*)(lds + nq + nx)};
}

// ---------------------------------------------------------------------------
// Q6_K, repacked at upload: per row, B blocks of 208 bytes
// [ql 128][qh 64][int8 scales 16] followed by B f16 d values.  AVX2 lane k
// covers bytes 4k..4k+3 of each 32-byte quad (Q6KQ8QUAD,
// kernels_amd64.s:1130-1142); lanes 0-3 use scale 8h+2c, lanes 4-7 8h+2c+1.
// The repack stores lane k's four ql dwords together at 16k and its two qh
// dwords at 128 + 8k, so a lane reads its share of a block in four loads.
// ---------------------------------------------------------------------------
// Greedy argmax over a logits vector: finite values only, strict >, lowest
// index on ties, 0 when nothing is finite (argmaxQ6KRowsQ8,
// kernels_amd64.go:294-331; finiteLogit sampling.go:385).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool finite_logit(float v) {
    return (__float_as_uint(v) & 0x7f800000u) != 0x7f800000u;
}

// Packs (value, row) so that a larger key is a larger value, or the same
// value at a lower row; 0 means "nothing finite seen".
__device__ __forceinline__ unsigned long long argmax_key(float v, int r) {
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xffffffffu - (uint32_t)r);
}

__device__ __forceinline__ unsigned long long wg_max_key(unsigned long long best) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const unsigned long long o = __shfl_xor(best, off);
        best = o > best ? o : best;
    }
    __shared__ unsigned long long wbest[16];
    const int nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
    __syncthreads();
    unsigned long long b = 0;
    for (int i = 0; i < nw; i++) b = wbest[i] > b ? wbest[i] : b;
    return b;
}

// applyRepeatPenalty (sampling.go:136-153) on logit i, whose id appears
// `count` times in the recent window: every occurrence applies the rule once
// more, to the value the previous one left (non-finite -> -inf, positive /=
// penalty, else *= penalty).  The rule reads only logit i, so applying it
// count times equals the reference's in-order walk over the window.
__device__ __forceinline__ float repeat_penalty(float v, int count, float penalty) {
    for (int c = 0; c < count; c++) {
        if (!finite_logit(v)) v = -INFINITY;
        else if (v > 0.0f) v = v / penalty;
        else v = v * penalty;
    }
    return v;
}


// Greedy argmax fused into the batch-1 epilogue of a row kernel (the decode
// step's vocabulary head; ArgmaxMatvec model.go:754 -> argmaxQ6KRowsQ8,
// kernels_amd64.go:294-331, keeps a running argmax while it dots the rows).
// Every workgroup penalises its rows' logits and reduces them to one key,
// stored at keys[blockIdx.x]; argmax_final_kernel reduces the keys.  Keys
// order by value, then by lower row, so the result is the lowest-index
// finite maximum whatever the reduction order (argmax_partial_kernel's keys).
// Lanes own rows in groups of span = 8 * G lanes, ascending with the lane.
// id0: recent[lane] (all ones past the window), loaded by the caller before
// its weight stream so the window's latency hides behind it.  Each wave
// counts its rows' window hits by ballot, takes the maximum of the keys'
// upper words (the order-preserving image of the value, 0 for non-finite)
// by DPP, then the lowest lane holding it by ballot; one barrier joins the
// four wave keys.
template <int G>
__device__ inline void argmax_epilogue(const GemvJob& j, int r, float v, bool own, uint32_t id0) {
    constexpr int span = 8 * G;
    const ArgmaxOut& am = j.am;
    const int lane = threadIdx.x & 63;
    float x = v;
    if (am.n_recent > 0 && am.penalty != 1.0f) {  // uniform
        int hits = 0;
        for (int c = 0; c < am.n_recent; c += 64) {
            const uint32_t id = c == 0 ? id0
                              : c + lane < am.n_recent ? am.recent[c + lane] : 0xffffffffu;
#pragma unroll
            for (int g = 0; g < 64 / span; g++) {
                const int h = __popcll(__ballot(id == (uint32_t)__builtin_amdgcn_readlane(r, g * span)));
                hits += lane / span == g ? h : 0;
            }
        }
        x = repeat_penalty(v, hits, am.penalty);
    }
    const uint32_t u = own && finite_logit(x) ? (uint32_t)(argmax_key(x, r) >> 32) : 0u;
    const uint32_t umax = wave_max_u32(u);
    const unsigned long long hit = __ballot(own && u == umax);
    const int rmin = __builtin_amdgcn_readlane(r, hit ? __builtin_ctzll(hit) : 0);
    __shared__ unsigned long long wkey[4];
    if (lane == 0)
        wkey[threadIdx.x >> 6] =
            umax ? ((unsigned long long)umax << 32) | (unsigned long long)(0xffffffffu - (uint32_t)rmin)
                 : 0ull;
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned long long a = wkey[0] > wkey[1] ? wkey[0] : wkey[1];
        const unsigned long long b = wkey[2] > wkey[3] ? wkey[2] : wkey[3];
        am.keys[blockIdx.x] = a > b ? a : b;
    }
}

// ---------------------------------------------------------------------------
//
// G lanes share one AVX2 lane (G = 2, 4 for short matrices, so that a launch
// still fills the chip): lane gi takes blocks gi, gi + G, ... and the
// reference's sequential per-lane chain visits the G lanes in block order
// through rot_prev, ending in lane gi = G - 1 after every group of G blocks.
//
// FUSE (batch 1, cols <= kFuseCols): the workgroup quantises the f32
// activation into LDS itself (x loads first, weight prefetch second), so the
// matvec is one launch; lanes past the last row then compute a clamped row
// and store nothing, since the whole workgroup takes part in the barrier.
template <int NT, int G, bool FUSE = false, int DQ = 0>
__global__ __launch_bounds__(256) void gemv_q6k_kernel(GemvJob j) {
    static_assert(!FUSE || NT == 1, "fused quantisation is batch 1 only");
    constexpr int D = DQ ? DQ : kQ6Depth<NT>;
    __shared__ __attribute__((aligned(16))) uint8_t fa_raw[FUSE ? sizeof(FusedAct) : 16];
    FusedAct& fa = *(FusedAct*)fa_raw;
    extern __shared__ __attribute__((aligned(16))) uint8_t dyn_lds[];
    int wi;
    const int tid = threadIdx.x;
    const int gi = tid % G, k = (tid / G) & 7;
    const int r = locate(j, blockIdx.x, &wi) + tid / (8 * G);
    const bool sa = NT > 1 && j.sa;  // uniform
    if (!FUSE && !sa && r >= j.rows[wi]) return;  // whole rows: the rotation and tree stay inside one row
    StagedAct st{};
    if (sa) st = stage_act(j, dyn_lds, true);  // every thread, then lanes past the last row idle
    const bool live = r < j.rows[wi];
    const int B = j.blocks, NB = B / G;
    const uint8_t* row = j.w[wi] + (size_t)(live ? r : j.rows[wi] - 1) * j.rb;
    const uint16_t* dv = (const uint16_t*)(row + (size_t)B * 208);
    const int hk = k >> 2;
    float accF[NT], accM[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) accF[t] = accM[t] = 0.0f;
    const int8_t* q8 = j.act.q8perm + (size_t)j.tok0 * j.cols + k * 32;
    const float* xsc = j.act.xscale + (size_t)j.tok0 * B;
    const float* xs16 = j.act.xs16 + (size_t)j.tok0 * (j.cols / 16) + k;
    // D blocks of this lane's bytes in flight, loaded in block order; the
    // loads are unconditional (clamped to the lane's last block) so the
    // compiler's vmcnt waits never drain the ring.  At batch 1 the block's
    // activation operands ride in the ring too: loaded later than the
    // weights, they would make every wait a full drain.
    struct Blk {
        uint32_t ql[4], qh[2];
        uint4 sv;
        uint32_t d;
        int4 qa, qb;
        float x0, x8, xs;
    };
    auto load_w = [&](int i, Blk& o) __attribute__((always_inline)) {
        const int bb = min(i, NB - 1) * G + gi;
        const uint8_t* blk = row + (size_t)bb * 208;
        const uint4 l4 = *(const uint4*)(blk + 16 * k);   // lane k's ql dwords q = 0..3
        const uint2 h2 = *(const uint2*)(blk + 128 + 8 * k);  // its qh dwords h = 0, 1
        o.ql[0] = l4.x;
        o.ql[1] = l4.y;
        o.ql[2] = l4.z;
        o.ql[3] = l4.w;
        o.qh[0] = h2.x;
        o.qh[1] = h2.y;
        o.sv = *(const uint4*)(blk + 192);
        o.d = dv[bb];
    };
    auto load_a = [&](int i, Blk& o) __attribute__((always_inline)) {
        const int bb = min(i, NB - 1) * G + gi;
        if constexpr (FUSE) {
            o.qa = *(const int4*)(fa.q8 + bb * 256 + k * 32);
            o.qb = *(const int4*)(fa.q8 + bb * 256 + k * 32 + 16);
            o.x0 = fa.xs16[bb * 16 + k] * 32.0f;  // ScaleF32(xs, 32)
            o.x8 = fa.xs16[bb * 16 + 8 + k] * 32.0f;
            o.xs = fa.xsc[bb];
        } else if constexpr (NT == 1) {
            o.qa = *(const int4*)(q8 + bb * 256);
            o.qb = *(const int4*)(q8 + bb * 256 + 16);
            o.x0 = xs16[bb * 16] * 32.0f;      // ScaleF32(xs, 32)
            o.x8 = xs16[bb * 16 + 8] * 32.0f;
            o.xs = xsc[bb];
        }
    };
    auto load = [&](int i, Blk& o) __attribute__((always_inline)) {
        load_w(i, o);
        load_a(i, o);
    };
    auto compute = [&](int i, const Blk& o) __attribute__((always_inline)) {
        const int b = i * G + gi;
        const float d = f16_bits_to_f32(o.d);
        // codes of quad (h, c), c = 0..3 (m = 4h + c)
        int code[8];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t y0 = h ? o.ql[2] : o.ql[0], y1 = h ? o.ql[3] : o.ql[1], qh = o.qh[h];
            code[4 * h + 0] = (int)((y0 & 0x0f0f0f0fu) | ((qh & 0x03030303u) << 4));
            code[4 * h + 1] = (int)((y1 & 0x0f0f0f0fu) | (((qh >> 2) & 0x03030303u) << 4));
            code[4 * h + 2] = (int)(((y0 >> 4) & 0x0f0f0f0fu) | (((qh >> 4) & 0x03030303u) << 4));
            code[4 * h + 3] = (int)(((y1 >> 4) & 0x0f0f0f0fu) | (((qh >> 6) & 0x03030303u) << 4));
        }
        // scale of quad m: byte 8h + 2c + hk of the 16 scale bytes
        const uint32_t sw[4] = {o.sv.x, o.sv.y, o.sv.z, o.sv.w};
        int scl[8];
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const int idx = 2 * m + hk;  // = 8h + 2c + hk
            scl[m] = sbyte(sw[idx >> 2], idx & 3);
        }
        const float sk = (float)sbyte(sw[k >> 2], k & 3);
        const float sk8 = (float)sbyte(sw[2 + (k >> 2)], k & 3);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (NT == 1 || t < j.ntok) {
                const int8_t* q8t = sa ? st.q8 + (size_t)t * j.cols + b * 256 + k * 32
                                       : q8 + (size_t)t * j.cols + b * 256;
                const int4 qa = NT == 1 ? o.qa : *(const int4*)q8t;
                const int4 qb = NT == 1 ? o.qb : *(const int4*)(q8t + 16);
                int acc = scl[0] * sdot4(code[0], qa.x, 0);
                acc += scl[1] * sdot4(code[1], qa.y, 0);
                acc += scl[2] * sdot4(code[2], qa.z, 0);
                acc += scl[3] * sdot4(code[3], qa.w, 0);
                acc += scl[4] * sdot4(code[4], qb.x, 0);
                acc += scl[5] * sdot4(code[5], qb.y, 0);
                acc += scl[6] * sdot4(code[6], qb.z, 0);
                acc += scl[7] * sdot4(code[7], qb.w, 0);
                const float* xs = sa ? st.xs16 + (size_t)t * (j.cols / 16) + b * 16 + k
                                     : xs16 + (size_t)t * (j.cols / 16) + b * 16;
                float o2 = sk * (NT == 1 ? o.x0 : xs[0] * 32.0f);       // VMULPS
                o2 = fmaf(sk8, NT == 1 ? o.x8 : xs[8] * 32.0f, o2);     // VFMADD231PS
                const float xv = sa ? st.xsc[t * B + b] : xsc[(size_t)t * B + b];
                const float dxs = d * (NT == 1 ? o.xs : xv);  // VMULSS
                const float iv = (float)acc;
#pragma unroll
                for (int step = 0; step < G; step++) {
                    accM[t] = fmaf(d, o2, rot_prev<G>(accM[t]));        // VFMADD231PS
                    accF[t] = fmaf(iv, dxs, rot_prev<G>(accF[t]));      // VFMADD231PS
                }
            }
        }
    };
    Blk ring[D];
    XRegs<kFuseQB> xr;
    uint32_t id0 = 0xffffffffu;  // the argmax epilogue's first 64 window ids
    if constexpr (NT == 1) {
        if (j.am.keys && (tid & 63) < j.am.n_recent) id0 = j.am.recent[tid & 63];
    }
    if constexpr (FUSE) {
        xq_load<kFuseQB>(j.xf, B, xr);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < D; i++) {
        if constexpr (FUSE) {
            load_w(i, ring[i]);
        } else {
            load(i, ring[i]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (FUSE) {
        fused_act_store<true>(xr, B, fa);
#pragma unroll
        for (int i = 0; i < D; i++) load_a(i, ring[i]);
    }
    // whole groups straight-line (a guarded compute would turn the waits
    // at its join into drains), then the tail
    int i0 = 0;
    for (; i0 + D <= NB; i0 += D) {
#pragma unroll
        for (int ii = 0; ii < D; ii++) {
            compute(i0 + ii, ring[ii]);
            __builtin_amdgcn_sched_barrier(0);  // keep the loads in block order
            load(i0 + ii + D, ring[ii]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int ii = 0; ii < D - 1; ii++)
        if (i0 + ii < NB) compute(i0 + ii, ring[ii]);  // uniform
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const float v = tree8_strided<G>(accF[t] - accM[t]);  // VSUBPS + tree
        if (live && k == 0 && gi == G - 1 && t < j.ntok)
            j.out[wi][(size_t)(j.tok0 + t) * j.out_stride[wi] + r] = v;
        if constexpr (NT == 1) {
            if (j.am.keys)  // uniform
                argmax_epilogue<G>(j, r, v, live && k == 0 && gi == G - 1, id0);
        }
    }
}

// ---------------------------------------------------------------------------
// Q8_0, repacked at upload: per 256-element group, [8 x f16 d] then lane k's
// dwords of the eight 32-value blocks together at 16 + 32k (272 bytes,
// 16-byte aligned).  AVX2 lane k covers bytes 4k..4k+3 of each 32-value block
// (Q80CHUNK, kernels_amd64.s:1321-1345), read here in two 16-byte loads.
// ---------------------------------------------------------------------------
// G lanes per AVX2 lane and FUSE as in gemv_q6k_kernel.
template <int NT, int G, bool FUSE = false>
__global__ __launch_bounds__(256) void gemv_q8_0_kernel(GemvJob j) {
    static_assert(!FUSE || NT == 1, "fused quantisation is batch 1 only");
    constexpr int D = kQ8Depth<NT>;
    __shared__ __attribute__((aligned(16))) uint8_t fa_raw[FUSE ? sizeof(FusedAct) : 16];
    FusedAct& fa = *(FusedAct*)fa_raw;
    extern __shared__ __attribute__((aligned(16))) uint8_t dyn_lds[];
    int wi;
    const int tid = threadIdx.x;
    const int gi = tid % G, k = (tid / G) & 7;
    const int r = locate(j, blockIdx.x, &wi) + tid / (8 * G);
    const bool sa = NT > 1 && j.sa;  // uniform
    if (!FUSE && !sa && r >= j.rows[wi]) return;  // whole rows: the rotation and tree stay inside one row
    StagedAct st{};
    if (sa) st = stage_act(j, dyn_lds, false);  // every thread, then lanes past the last row idle
    const bool live = r < j.rows[wi];
    const int B = j.blocks, NB = B / G;
    const uint8_t* row = j.w[wi] + (size_t)(live ? r : j.rows[wi] - 1) * j.rb;
    float acc11[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc11[t] = 0.0f;
    const int8_t* q8 = j.act.q8perm + (size_t)j.tok0 * j.cols + k * 32;
    const float* xsc = j.act.xscale + (size_t)j.tok0 * B;
    // D blocks of this lane's bytes in flight (see gemv_q6k_kernel)
    struct Blk {
        uint4 dh;
        int wv[8];
        int4 qa, qb;
        float xs;
    };
    auto load_w = [&](int i, Blk& o) __attribute__((always_inline)) {
        const int bb = min(i, NB - 1) * G + gi;
        const uint8_t* blk = row + (size_t)bb * 272;
        o.dh = *(const uint4*)blk;
        const uint4 w0 = *(const uint4*)(blk + 16 + 32 * k);  // lane k's dwords, blocks 0..3
        const uint4 w1 = *(const uint4*)(blk + 32 + 32 * k);  // blocks 4..7
        o.wv[0] = (int)w0.x;
        o.wv[1] = (int)w0.y;
        o.wv[2] = (int)w0.z;
        o.wv[3] = (int)w0.w;
        o.wv[4] = (int)w1.x;
        o.wv[5] = (int)w1.y;
        o.wv[6] = (int)w1.z;
        o.wv[7] = (int)w1.w;
    };
    auto load_a = [&](int i, Blk& o) __attribute__((always_inline)) {
        const int bb = min(i, NB - 1) * G + gi;
        if constexpr (FUSE) {
            o.qa = *(const int4*)(fa.q8 + bb * 256 + k * 32);
            o.qb = *(const int4*)(fa.q8 + bb * 256 + k * 32 + 16);
            o.xs = fa.xsc[bb];
        } else if constexpr (NT == 1) {
            o.qa = *(const int4*)(q8 + bb * 256);
            o.qb = *(const int4*)(q8 + bb * 256 + 16);
            o.xs = xsc[bb];
        }
    };
    auto load = [&](int i, Blk& o) __attribute__((always_inline)) {
        load_w(i, o);
        load_a(i, o);
    };
    auto compute = [&](int i, const Blk& o) __attribute__((always_inline)) {
        const int b = i * G + gi;
        float dj[8];
        const uint32_t dw[4] = {o.dh.x, o.dh.y, o.dh.z, o.dh.w};
#pragma unroll
        for (int q = 0; q < 8; q++) dj[q] = f16_bits_to_f32((dw[q >> 1] >> (16 * (q & 1))) & 0xffffu);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (NT == 1 || t < j.ntok) {
                const int8_t* q8t = sa ? st.q8 + (size_t)t * j.cols + b * 256 + k * 32
                                       : q8 + (size_t)t * j.cols + b * 256;
                const int4 qa = NT == 1 ? o.qa : *(const int4*)q8t;
                const int4 qb = NT == 1 ? o.qb : *(const int4*)(q8t + 16);
                const int xq[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
                float acc12 = 0.0f;
#pragma unroll
                for (int q = 0; q < 8; q++) acc12 = fmaf((float)sdot4(o.wv[q], xq[q], 0), dj[q], acc12);
                const float xs = NT == 1 ? o.xs : sa ? st.xsc[t * B + b] : xsc[(size_t)t * B + b];
#pragma unroll
                for (int step = 0; step < G; step++) acc11[t] = fmaf(acc12, xs, rot_prev<G>(acc11[t]));
            }
        }
    };
    Blk ring[D];
    XRegs<kFuseQB> xr;
    if constexpr (FUSE) {
        xq_load<kFuseQB>(j.xf, B, xr);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < D; i++) {
        if constexpr (FUSE) {
            load_w(i, ring[i]);
        } else {
            load(i, ring[i]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (FUSE) {
        fused_act_store<false>(xr, B, fa);
#pragma unroll
        for (int i = 0; i < D; i++) load_a(i, ring[i]);
    }
    int i0 = 0;
    for (; i0 + D <= NB; i0 += D) {
#pragma unroll
        for (int ii = 0; ii < D; ii++) {
            compute(i0 + ii, ring[ii]);
            __builtin_amdgcn_sched_barrier(0);  // keep the loads in block order
            load(i0 + ii + D, ring[ii]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int ii = 0; ii < D - 1; ii++)
        if (i0 + ii < NB) compute(i0 + ii, ring[ii]);  // uniform
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const float v = tree8_strided<G>(acc11[t]);
        if (live && k == 0 && gi == G - 1 && t < j.ntok)
            j.out[wi][(size_t)(j.tok0 + t) * j.out_stride[wi] + r] = v;
    }
}

// Debug: the exact int32 lane sums of every (row, block).
__global__ __launch_bounds__(256) void lane_ints_kernel(const uint8_t* __restrict__ w, int type,
                                                        int rows, int B, size_t rb, ActQ8 act,
                                                        int32_t* __restrict__ out) {
    const int r = blockIdx.x * kRowsPerWG + (threadIdx.x >> 3);
    const int k = threadIdx.x & 7;
    if (r >= rows) return;
    const uint8_t* row = w + (size_t)r * rb;
    const int8_t* q8 = act.q8perm + k * 32;
    for (int b = 0; b < B; b++) {
        const int4 qa = *(const int4*)(q8 + b * 256);
        const int4 qb = *(const int4*)(q8 + b * 256 + 16);
        const int xq[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        int acc = 0;
        if (type == GLLM_TYPE_Q4_K) {
            const uint4 h = *(const uint4*)(row + q4k_hdr_off(b));
            const uint8_t* nib = row + q4k_nib_off(B, b);
            const uint32_t sc03 = h.y & 0x3f3f3f3fu;
            const uint32_t sc47 = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
            for (int s = 0; s < 4; s++) {
                const uint32_t wd = *(const uint32_t*)(nib + 16 * k + 4 * s);  // repacked
                const uint32_t sc = s < 2 ? sc03 : sc47;
                acc += ubyte(sc, (2 * s) & 3) * sdot4((int)(wd & 0x0f0f0f0fu), xq[2 * s], 0);
                acc += ubyte(sc, (2 * s + 1) & 3) * sdot4((int)((wd >> 4) & 0x0f0f0f0fu), xq[2 * s + 1], 0);
            }
        } else if (type == GLLM_TYPE_Q6_K) {
            const uint8_t* blk = row + (size_t)b * 208;
            const int8_t* sc = (const int8_t*)(blk + 192);
            for (int m = 0; m < 8; m++) {
                const int h = m >> 2, c = m & 3;
                const uint32_t y = *(const uint32_t*)(blk + 16 * k + 4 * (2 * h + (c & 1)));  // repacked
                const uint32_t qh = *(const uint32_t*)(blk + 128 + 8 * k + 4 * h);
                const uint32_t code = ((y >> (4 * (c >> 1))) & 0x0f0f0f0fu) |
                                      (((qh >> (2 * c)) & 0x03030303u) << 4);
                acc += (int)sc[8 * h + 2 * c + (k >> 2)] * sdot4((int)code, xq[m], 0);
            }
        } else {
            const uint8_t* blk = row + (size_t)b * 272;
            for (int q = 0; q < 8; q++) acc += sdot4(*(const int*)(blk + 16 + 32 * k + 4 * q), xq[q], 0);
        }
        out[((size_t)r * B + b) * 8 + k] = acc;
    }
}

// Two stages: 256-thread workgroups each reduce kArgmaxChunk logits to one
// key, then one workgroup reduces the keys.  Keys compare larger for a
// larger finite value, or the same value at a lower row, so the result is
// the lowest-index maximum regardless of the reduction order.
constexpr int kArgmaxChunk = 1024;  // four logits per thread, all loads in flight together

// First stage; with n_recent > 0 and penalty != 1 the workgroup counts the
// window's ids that fall in its chunk (ids >= n are ignored, as in the
// reference) and penalises those logits before the finite-argmax rule.
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ logits,
                                                             int n,
                                                             unsigned long long* __restrict__ keys,
                                                             const uint32_t* __restrict__ recent,
                                                             int n_recent, float penalty) {
    __shared__ int hits[kArgmaxChunk];
    const int lo = blockIdx.x * kArgmaxChunk;
    const int hi = min(n, lo + kArgmaxChunk);
    const bool pen = n_recent > 0 && penalty != 1.0f;
    if (pen) {
        for (int i = threadIdx.x; i < kArgmaxChunk; i += 256) hits[i] = 0;
        __syncthreads();
        for (int i = threadIdx.x; i < n_recent; i += 256) {
            const uint32_t id = recent[i];
            if (id >= (uint32_t)lo && id < (uint32_t)hi) atomicAdd(&hits[id - lo], 1);
        }
        __syncthreads();
    }
    constexpr int PER = kArgmaxChunk / 256;
    float lv[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int i = lo + threadIdx.x + k * 256;
        lv[k] = i < hi ? logits[i] : 0.0f;
    }
    unsigned long long best = 0;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int i = lo + threadIdx.x + k * 256;
        if (i >= hi) break;
        float v = lv[k];
        if (pen) v = repeat_penalty(v, hits[i - lo], penalty);
        if (finite_logit(v)) {
            const unsigned long long key = argmax_key(v, i);
            best = key > best ? key : best;
        }
    }
    best = wg_max_key(best);
    if (threadIdx.x == 0) keys[blockIdx.x] = best;
}

__global__ __launch_bounds__(1024) void argmax_final_kernel(const unsigned long long* __restrict__ keys,
                                                            int nk, uint32_t* __restrict__ token) {
    unsigned long long best = 0;
    for (int i0 = 0; i0 < nk; i0 += 8 * 1024) {
        unsigned long long kv[8];  // all eight loads in flight together
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int i = i0 + threadIdx.x + k * 1024;
            kv[k] = i < nk ? keys[i] : 0ull;
        }
#pragma unroll
        for (int k = 0; k < 8; k++) best = kv[k] > best ? kv[k] : best;
    }
    best = wg_max_key(best);
    if (threadIdx.x == 0) *token = best ? 0xffffffffu - (uint32_t)(best & 0xffffffffu) : 0u;
}

__global__ void silu_mul_rows_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                     float* __restrict__ out, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = silu_mul(gate[i], up[i]);
}

size_t argmax_keys(int n) { return (size_t)(n + kArgmaxChunk - 1) / kArgmaxChunk; }

// keys: device scratch of argmax_keys(n) entries; recent: n_recent device
// token ids for the repeat penalty (none when n_recent == 0 or penalty == 1).
int launch_argmax(const float* logits, int n, uint32_t* token, unsigned long long* keys,
                  hipStream_t s, const uint32_t* recent, int n_recent, float penalty) {
    if (n_recent < 0 || (n_recent > 0 && !recent))
        return fail(GLLM_EINVAL, "argmax: bad recent-token window (%d ids)", n_recent);
    if (!(penalty > 0.0f) || penalty == INFINITY)
        return fail(GLLM_EINVAL, "argmax: repeat penalty must be finite and positive");
    const int nk = (int)argmax_keys(n);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(nk), dim3(256), 0, s, logits, n, keys, recent,
                       n_recent, penalty);
    GLLM_HIP(hipGetLastError());
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(1024), 0, s, keys, nk, token);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

// ---------------------------------------------------------------------------
// Upload-time repacks (same bytes, 16-byte aligned blocks) and their inverse.
// ---------------------------------------------------------------------------
__global__ void repack_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int type,
                              int rows, int B, size_t rb, int inverse) {
    const size_t total = (size_t)rows * rb;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / rb, o = i % rb;  // o: offset in the reference row
        const size_t n = repacked_offset(type, o, B);
        if (inverse) dst[r * rb + o] = src[r * rb + n];
        else dst[r * rb + n] = src[r * rb + o];
    }
}

int launch_repack(const uint8_t* src, uint8_t* dst, int type, int rows, int B, size_t rb,
                  int inverse, hipStream_t s) {
    const size_t total = (size_t)rows * rb;
    int grid = (int)std::min<size_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(repack_kernel, dim3(grid), dim3(256), 0, s, src, dst, type, rows, B, rb,
                       inverse);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

// Types with a row kernel.
bool row_kernel_type(int t) {
    return t == GLLM_TYPE_Q4_K || t == GLLM_TYPE_Q6_K || t == GLLM_TYPE_Q8_0 || t == GLLM_TYPE_Q5_K ||
           t == GLLM_TYPE_Q2_K || t == GLLM_TYPE_Q3_K || t == GLLM_TYPE_Q4_0 || t == GLLM_TYPE_Q4_1 ||
           t == GLLM_TYPE_MXFP4;
}

size_t ref_row_bytes(int type, int cols) {
    switch (type) {
    case GLLM_TYPE_Q4_K: return (size_t)(cols / 256) * 144;
    case GLLM_TYPE_Q6_K: return (size_t)(cols / 256) * 210;
    case GLLM_TYPE_Q8_0: return (size_t)(cols / 32) * 34;
    case GLLM_TYPE_Q5_K: return (size_t)(cols / 256) * 176;
    case GLLM_TYPE_Q2_K: return (size_t)(cols / 256) * 84;
    case GLLM_TYPE_Q3_K: return (size_t)(cols / 256) * 110;
    case GLLM_TYPE_Q4_0: return (size_t)(cols / 32) * 18;
    case GLLM_TYPE_Q4_1: return (size_t)(cols / 32) * 20;
    case GLLM_TYPE_MXFP4: return (size_t)(cols / 32) * 17;
    case GLLM_TYPE_F32: return (size_t)cols * 4;
    case GLLM_TYPE_F16: case GLLM_TYPE_BF16: return (size_t)cols * 2;
    default: return 0;
    }
}

// ---------------------------------------------------------------------------
// launch helpers
// ---------------------------------------------------------------------------

// Activation bytes one Q4_K workgroup stages in LDS for NT tokens.
static size_t q4k_stage_bytes(int nt, int cols) {
    return (size_t)nt * ((size_t)cols + (size_t)(cols / 32) * 4 + (size_t)(cols / 256) * 4);
}
constexpr size_t kMaxStage = 48 << 10;

template <int NT, int G, int NL, int D>
static void launch_q4k_nl(const GemvJob& j, dim3 grid, dim3 block, size_t stage, hipStream_t s) {
    if constexpr (NT == 1 && NL * G * 256 <= kFuseCols) {
        if (j.xf && j.nw) {
            const size_t lds = q4k_norm_off(j.cols) + (size_t)j.cols * 4 + kNormLds;
            if (j.res && j.sq_cnt)
                hipLaunchKernelGGL((gemv_q4k_kernel<1, G, NL, D, 3, true>), grid, block, lds, s, j);
            else if (j.res) hipLaunchKernelGGL((gemv_q4k_kernel<1, G, NL, D, 3>), grid, block, lds, s, j);
            else hipLaunchKernelGGL((gemv_q4k_kernel<1, G, NL, D, 2>), grid, block, lds, s, j);
            return;
        }
        if (j.xf) {
            hipLaunchKernelGGL((gemv_q4k_kernel<1, G, NL, D, 1>), grid, block, stage, s, j);
            return;
        }
    }
    hipLaunchKernelGGL((gemv_q4k_kernel<NT, G, NL, D, 0>), grid, block, stage, s, j);
}

// Blocks per lane with a compiled row kernel (and its prefetch depth).
static bool q4k_has_nl(int nl) { return nl == 4 || nl == 8 || nl == 14 || nl == 16 || nl == 28; }

// Launch shape of the Q4_K row kernel: one workgroup per compute unit up to
// the row cap below, so a CU's activation staging is the first memory
// traffic it issues (a second workgroup's small activation reads would queue
// behind the first one's weight stream).  G lanes share an AVX2 lane when the
// rows alone give fewer than four waves per workgroup.
struct Q4KShape {
    int g, rows_per_wg, threads;
};
// Smallest workgroup the shape search accepts before trying a larger G
// (every G gives the same bits; at 14336x4096, 896 threads measured 11.8 us
// against 9.7 us).
constexpr int kQ4KMinThreads = 448;
// Largest workgroup in rows at G = 1, and in lanes (rows x 8 x G) at any G:
// 64 rows, 512 threads.  Matrices with more rows than that per compute unit
// (the decode step's fused gate/up, 28672 rows) take several workgroups per
// CU instead of one large one; measured on the 8B decode step, 438 tok/s at
// 64 rows against 434 at 128 (1024 threads), 425 at 72, 414 at 80 and 56,
// 404 at 96; every shape gives the same bits.
constexpr int kQ4KMaxRows = 64;
constexpr int kQ4KMaxThreads = 512;
static Q4KShape q4k_shape(int total_rows, int blocks) {
    const int ncu = device_cus();
    Q4KShape best{0, 0, 0};
    for (int g = 1; g <= 4; g *= 2) {
        if (blocks % g) continue;
        const int unit = 8 / g;  // rows per wave
        int rpw = (total_rows + ncu - 1) / ncu;
        rpw = (rpw + unit - 1) / unit * unit;
        rpw = std::min(rpw, std::max(unit, kQ4KMaxRows / g));
        rpw = std::min(rpw, std::max(unit, kQ4KMaxThreads / (8 * g) / unit * unit));
        const Q4KShape sh{g, rpw, rpw * 8 * g};
        if (!q4k_has_nl(blocks / g) && best.g) continue;
        best = sh;
        if (sh.threads >= kQ4KMinThreads && q4k_has_nl(blocks / g)) break;
    }
    return best;
}

template <int NT, int G>
int launch_q4k(GemvJob& j, const int* rows, int n, const Q4KShape& sh, hipStream_t s) {
    const int nl = j.blocks / G;
    const size_t stage = q4k_stage_bytes(NT, j.cols);
    const bool compiled = stage <= kMaxStage && q4k_has_nl(nl) && sh.threads >= 256;
    if (j.xf && (NT != 1 || !compiled || j.cols > kFuseCols))
        return fail(GLLM_EINVAL, "gemv: fused quantisation needs batch 1 and a compiled shape");
    // the generic kernel keeps 256-thread workgroups of 32 / G rows
    j.rows_per_wg = compiled ? sh.rows_per_wg : 32 / G;
    int wg = 0;
    for (int i = 0; i < n; i++) {
        j.wg_begin[i] = wg;
        wg += (rows[i] + j.rows_per_wg - 1) / j.rows_per_wg;
    }
    j.wg_begin[n] = wg;
    const dim3 grid(wg), block(compiled ? sh.threads : 256);
    if (!compiled) {
        hipLaunchKernelGGL((gemv_q4k_any_kernel<NT, G>), grid, block, 0, s, j);
    } else if (nl == 4) {
        launch_q4k_nl<NT, G, 4, 4>(j, grid, block, stage, s);
    } else if (nl == 8) {
        launch_q4k_nl<NT, G, 8, 8>(j, grid, block, stage, s);
    } else if (nl == 14) {
        launch_q4k_nl<NT, G, 14, 7>(j, grid, block, stage, s);
    } else if (nl == 16) {
        launch_q4k_nl<NT, G, 16, 4>(j, grid, block, stage, s);
    } else {
        launch_q4k_nl<NT, G, 28, 7>(j, grid, block, stage, s);
    }
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

// Lanes per AVX2 lane (G) of the Q6_K / Q8_0 row kernels (G divides the
// block count).  Batch 1 splits a row only while the launch has fewer
// workgroups than the device has compute units: with every CU busy the G-step
// rotation costs more than extra workgroups bring (Q6_K 14336x4096 measured
// 16.7 / 21.2 / 29.5 us at G = 1 / 2 / 4), with half of them idle it is the
// other way round (Q6_K 4096x14336: 44.9 / 27.8 / 24.8 us).  Q6_K, the
// heaviest lane step, also splits while a lane would walk more than 16
// blocks and the launch has fewer than two workgroups per CU (4096x14336 at
// G = 4); the other formats measured faster at G = 2
// there (Q5_K 16.4 / 18.7 us, Q3_K 18.8 / 20.7 us at G = 2 / 4).  Batches (per-token
// activation reads make each block several times longer) take the largest G
// that keeps the launch at one workgroup per compute unit or fewer.
// Every G gives the same bits.
static int row_lanes_g(int total_rows, int blocks, int ntok, int type) {
    const int ncu = device_cus();
    auto wgs = [&](int g) { return (total_rows * g + kRowsPerWG - 1) / kRowsPerWG; };
    int g = 1;
    if (ntok == 1) {
        const bool long_q6k = type == GLLM_TYPE_Q6_K;
        while (g < 4 && blocks % (2 * g) == 0 &&
               (wgs(g) < ncu || (long_q6k && blocks / g > 16 && wgs(g) < 2 * ncu)))
            g *= 2;
    } else {
        // one workgroup per CU at most: at batch 8, 4096x14336 Q6_K 80.2 / 60.4 us
        // and Q8_0 68.1 / 57.4 us at G = 4 (two per CU) / G = 2 (one per CU)
        while (g < 4 && blocks % (2 * g) == 0 && wgs(2 * g) <= ncu) g *= 2;
    }
    return g;
}

template <int NT>
static void (*pick_g(int g, void (*k1)(GemvJob), void (*k2)(GemvJob), void (*k4)(GemvJob)))(GemvJob) {
    return g == 1 ? k1 : g == 2 ? k2 : k4;
}
template <class F, int NT, bool FUSE>
static void (*fmt_kernel(int g))(GemvJob) {
    return pick_g<NT>(g, gemv_fmt_kernel<F, NT, 1, FUSE>, gemv_fmt_kernel<F, NT, 2, FUSE>,
                      gemv_fmt_kernel<F, NT, 4, FUSE>);
}

// Dynamic LDS of the staged batch activations: up to the 160 KB a gfx950
// workgroup may use, after a one-time opt-in per kernel.
constexpr size_t kStagedActMax = 160 * 1024 - 64;
static bool lds_opt_in(const void* kern) {
    static std::mutex mu;
    static std::vector<const void*> done;
    std::lock_guard<std::mutex> lock(mu);
    for (const void* d : done)
        if (d == kern) return true;
    if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kStagedActMax) !=
        hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    done.push_back(kern);
    return true;
}

// The Q6_K, Q8_0 and other-format row kernel for this type, batch tile NT
// and G; FUSE selects the variant that quantises x itself; shallow: the
// batch-1 Q6_K ring of three blocks (kQ6Depth).
template <int NT, bool FUSE>
static void (*row_kernel(int type, int g, bool shallow))(GemvJob) {
    switch (type) {
    case GLLM_TYPE_Q6_K:
        if (NT == 1 && shallow)
            return pick_g<NT>(g, gemv_q6k_kernel<NT, 1, FUSE, 3>, gemv_q6k_kernel<NT, 2, FUSE, 3>,
                              gemv_q6k_kernel<NT, 4, FUSE, 3>);
        return pick_g<NT>(g, gemv_q6k_kernel<NT, 1, FUSE>, gemv_q6k_kernel<NT, 2, FUSE>,
                          gemv_q6k_kernel<NT, 4, FUSE>);
    case GLLM_TYPE_Q8_0:
        return pick_g<NT>(g, gemv_q8_0_kernel<NT, 1, FUSE>, gemv_q8_0_kernel<NT, 2, FUSE>,
                          gemv_q8_0_kernel<NT, 4, FUSE>);
    case GLLM_TYPE_Q5_K: return fmt_kernel<fmt::Q5K, NT, FUSE>(g);
    case GLLM_TYPE_Q2_K: return fmt_kernel<fmt::Q2K, NT, FUSE>(g);
    case GLLM_TYPE_Q3_K: return fmt_kernel<fmt::Q3K, NT, FUSE>(g);
    case GLLM_TYPE_Q4_0: return fmt_kernel<fmt::Q401<false>, NT, FUSE>(g);
    case GLLM_TYPE_Q4_1: return fmt_kernel<fmt::Q401<true>, NT, FUSE>(g);
    default: return fmt_kernel<fmt::MXFP4, NT, FUSE>(g);
    }
}

// Launch shape of the block-parallel batch-1 Q4_K kernel: NS slices per row,
// NTH threads per workgroup, RP rows per lane, P blocks per lane issued
// before the wave waits for its x.  ns == 0: not taken.  Measured on one
// box against gemv_q4k_kernel (three alternations): 4096 x 4096, 4.59
// against 4.98 us per step; 4096 x 14336 (pre-quantised
// activations), 11.88 against 12.75 us.  Other shapes keep the row kernels.
struct Q4KBpShape {
    int ns, nth, rp, p;
};
static Q4KBpShape q4k_bp_pick(int total_rows, int B) {
    const bool rows4k = total_rows >= 3584 && total_rows <= 4608;
    if (B == 16 && rows4k) return {8, 1024, 1, 1};
    if (B == 16 && total_rows == 6144) return {4, 768, 1, 1};  // Q/K/V at 8B: 256 x 24 rows
    if (B == 56 && rows4k) return {14, 896, 1, 2};
    return {0, 0, 0, 0};
}

template <int B, int NS, int NTH, int RP, int P>
static int launch_q4k_bp_inst(GemvJob& j, const int* rows, hipStream_t s) {
    constexpr int RW = q4k_bp_rows(NS, NTH, RP);
    j.rows_per_wg = RW;
    int total = 0;
    for (int i = 0; i < j.n; i++) total += rows[i];
    const int wg = (total + RW - 1) / RW;  // rows of all weights end to end
    constexpr size_t cols = (size_t)B * 256;
    constexpr size_t lds_x = q4k_bp_lds(B, NS, NTH, RP);
    constexpr size_t lds_n = q4k_norm_off(cols) + cols * 4 + kNormLds;  // x' over the exchange
    constexpr size_t lds = lds_x > lds_n ? lds_x : lds_n;
    static_assert(lds <= kStagedActMax, "block-parallel LDS");
    void (*kern)(GemvJob) = gemv_q4k_bp_kernel<B, NS, NTH, RP, 0, P>;
    if constexpr (B * 256 <= kFuseCols) {
        if (j.xf && j.nw) kern = j.res ? gemv_q4k_bp_kernel<B, NS, NTH, RP, 3, P>
                                       : gemv_q4k_bp_kernel<B, NS, NTH, RP, 2, P>;
        else if (j.xf) kern = gemv_q4k_bp_kernel<B, NS, NTH, RP, 1, P>;
    }
    if (lds > 64 * 1024 && !lds_opt_in((const void*)kern))
        return fail(GLLM_EDEVICE, "gemv: %zu B of LDS refused", lds);
    hipLaunchKernelGGL(kern, dim3(wg), dim3(NTH), lds, s, j);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

// Batch-1 Q4_K through the block-parallel kernel when this row length has an
// instance; *done = false otherwise (the row kernels take it).
static int launch_q4k_bp(GemvJob& j, const int* rows, hipStream_t s, bool* done) {
    int total = 0;
    for (int i = 0; i < j.n; i++) total += rows[i];
    const Q4KBpShape sh = q4k_bp_pick(total, j.blocks);
    *done = sh.ns != 0 && (!j.xf || j.cols <= kFuseCols) && (!j.nw || j.xf) && !j.sq_cnt;
    if (!*done) return GLLM_OK;
#define GLLM_BP_INST(b_, ns_, nth_, rp_, p_)                                               \
    if (j.blocks == b_ && sh.ns == ns_ && sh.nth == nth_ && sh.rp == rp_ && sh.p == p_) \
        return launch_q4k_bp_inst<b_, ns_, nth_, rp_, p_>(j, rows, s);
    GLLM_BP_INST(16, 8, 1024, 1, 1)
    GLLM_BP_INST(16, 4, 768, 1, 1)
    GLLM_BP_INST(56, 14, 896, 1, 2)
#undef GLLM_BP_INST
    return fail(GLLM_EINVAL, "gemv: no block-parallel instance (%d, %d, %d, %d, %d)", j.blocks, sh.ns,
                sh.nth, sh.rp, sh.p);
}

// Wave-specialised launch: R rows per workgroup, NS slices, NLD loader
// waves, D blocks in flight per loader before it waits.  r == 0: not taken.
// One weight with at least 230 workgroups of 56 rows (14336 x 4096, one
// workgroup per CU): 8.61 against 8.91 us per step for gemv_q4k_kernel
// (same box, three alternations); the block-parallel kernel took 8.85 there.
// Measured alternatives: D = 2 / 4, 8.93 / 9.58 us; 16-row workgroups 10.4.
struct Q4KWsShape {
    int r, ns, nld, d;
};
static Q4KWsShape q4k_ws_pick(int total_rows, int B) {
    if (B == 16 && total_rows >= 230 * 56) return {56, 2, 2, 1};
    return {0, 0, 0, 0};
}

template <int B, int R, int NS, int NLD, int D>
static int launch_q4k_ws_inst(GemvJob& j, const int* rows, hipStream_t s) {
    constexpr size_t lds = Q4KWsLayout<B, R>::bytes;
    auto kern = gemv_q4k_ws_kernel<B, R, NS, NLD, D>;
    if (lds > 64 * 1024 && !lds_opt_in((const void*)kern))
        return fail(GLLM_EDEVICE, "gemv: %zu B of LDS refused", lds);
    hipLaunchKernelGGL(kern, dim3((rows[0] + R - 1) / R), dim3(R * 8 * NS + NLD * 64), lds, s,
                       j.w[0], j.xf, j.out[0], rows[0], (int)j.rb);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

// Batch-1 Q4_K of one weight that quantises x itself through the
// wave-specialised kernel when the shape has an instance; *done = false
// otherwise.
static int launch_q4k_ws(GemvJob& j, const int* rows, hipStream_t s, bool* done) {
    const Q4KWsShape sh = q4k_ws_pick(rows[0], j.blocks);
    *done = sh.r != 0 && j.n == 1 && j.xf && j.cols <= kFuseCols && !j.nw && j.tok0 == 0;
    if (!*done) return GLLM_OK;
#define GLLM_WS_INST(b_, r_, ns_, nld_, d_)                                                \
    if (j.blocks == b_ && sh.r == r_ && sh.ns == ns_ && sh.nld == nld_ && sh.d == d_) \
        return launch_q4k_ws_inst<b_, r_, ns_, nld_, d_>(j, rows, s);
    GLLM_WS_INST(16, 56, 2, 2, 1)
#undef GLLM_WS_INST
    return fail(GLLM_EINVAL, "gemv: no wave-specialised instance (%d, %d, %d, %d, %d)", j.blocks, sh.r,
                sh.ns, sh.nld, sh.d);
}

template <int NT>
int launch_gemv_nt(GemvJob& j, int type, int grid, const int* rows, hipStream_t s) {
    if (NT == 1 && type == GLLM_TYPE_Q4_K && j.ntok == 1) {
        bool done = false;
        GLLM_TRY(launch_q4k_ws(j, rows, s, &done));
        if (done) return GLLM_OK;
        GLLM_TRY(launch_q4k_bp(j, rows, s, &done));
        if (done) return GLLM_OK;
    }
    if (type == GLLM_TYPE_Q4_K) {
        int total = 0;
        for (int i = 0; i < j.n; i++) total += rows[i];
        const Q4KShape sh = q4k_shape(total, j.blocks);
        return sh.g == 1 ? launch_q4k<NT, 1>(j, rows, j.n, sh, s)
             : sh.g == 2 ? launch_q4k<NT, 2>(j, rows, j.n, sh, s)
                         : launch_q4k<NT, 4>(j, rows, j.n, sh, s);
    }
    if (!row_kernel_type(type)) return fail(GLLM_EUNSUP, "gemv: unsupported type %d", type);
    if (j.xf && (NT != 1 || j.cols > kFuseCols))
        return fail(GLLM_EINVAL, "gemv: fused quantisation needs batch 1 and cols <= %d", kFuseCols);
    int total = 0;
    for (int i = 0; i < j.n; i++) total += rows[i];
    const int g = row_lanes_g(total, j.blocks, j.ntok, type);
    j.rows_per_wg = kRowsPerWG / g;
    int wg = 0;
    for (int i = 0; i < j.n; i++) {
        j.wg_begin[i] = wg;
        wg += (rows[i] + j.rows_per_wg - 1) / j.rows_per_wg;
    }
    j.wg_begin[j.n] = wg;
    // many workgroups (two or more per CU) or long rows: occupancy over depth
    const bool shallow = wg >= 2 * device_cus() || j.blocks >= 32;
    void (*kern)(GemvJob) = row_kernel<NT, false>(type, g, shallow);
    if constexpr (NT == 1) {
        if (j.xf) kern = row_kernel<1, true>(type, g, shallow);
    }
    size_t lds = 0;
    j.sa = 0;
    if (NT > 1 && (type == GLLM_TYPE_Q6_K || type == GLLM_TYPE_Q8_0)) {
        lds = staged_act_bytes(j.ntok, j.cols, type == GLLM_TYPE_Q6_K);
        if (lds <= kStagedActMax && lds_opt_in((const void*)kern)) {
            j.sa = 1;
        } else {
            lds = 0;
        }
    }
    hipLaunchKernelGGL(kern, dim3(wg), dim3(256), lds, s, j);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

int validate_weight(const gllm_hip_weight* w) {
    if (!w || !w->d_data) return fail(GLLM_EINVAL, "null weight handle");
    if (!row_kernel_type(w->type))
        return fail(GLLM_EUNSUP, "weight type %d has no row kernel", w->type);
    return GLLM_OK;
}

// Row kernels for n weights against p activation rows already quantised
// into `act` (activation rows tok0 .. tok0+p-1 of act).
// RMSNorm prologue arguments (GemvJob::nw .. eps) and the optional SwiGLU
// epilogue (GemvJob::sq_cnt, sq_act)
struct NormIn {
    const float* w;
    const float* res;
    float* xout;
    float eps;
    int* sq_cnt;
    ActQ8 sq_act;
};

// The batched Q6_K matrix-core kernel applies (launch_q6k_tiled).
static bool q6k_tiled_fits(const ActQ8& act, int p, const gllm_hip_weight* w) {
    return p > kTiledMinP && act.b16t && w->blocks % 8 == 0 &&
           (size_t)w->rows * w->row_bytes < ((size_t)1 << 32);
}

int run_gemv(int n, gllm_hip_weight* const* ws, const ActQ8& act, int p, float* const* outs,
             const int* strides, hipStream_t s, const float* xf, const NormIn* ni = nullptr,
             const ArgmaxOut* am = nullptr) {
    if (n < 1 || n > 3) return fail(GLLM_EINVAL, "gemv: %d weights (1..3 supported)", n);
    if (xf && p != 1) return fail(GLLM_EINVAL, "gemv: fused quantisation is batch 1 only");
    GemvJob j{};
    j.n = n;
    j.xf = xf;
    if (am) {
        if (n != 1 || !xf || ws[0]->type != GLLM_TYPE_Q6_K)
            return fail(GLLM_EINVAL, "gemv: the argmax epilogue needs one fused Q6_K launch");
        j.am = *am;
    }
    if (ni) {
        if (!xf || ws[0]->type != GLLM_TYPE_Q4_K)
            return fail(GLLM_EINVAL, "gemv: the RMSNorm prologue needs a fused Q4_K launch");
        j.nw = ni->w;
        j.res = ni->res;
        j.xout = ni->xout;
        j.eps = ni->eps;
        j.sq_cnt = ni->sq_cnt;
        j.sq_act = ni->sq_act;
        if (j.sq_cnt && (n != 2 || !j.res))
            return fail(GLLM_EINVAL, "gemv: the SwiGLU epilogue needs the gate/up pair and a residual");
    }
    const gllm_hip_weight* w0 = ws[0];
    j.blocks = w0->blocks;
    j.cols = w0->cols;
    j.rb = w0->row_bytes;
    j.act = act;
    int wg = 0;
    for (int i = 0; i < n; i++) {
        j.w[i] = ws[i]->d_data;
        j.out[i] = outs[i];
        j.rows[i] = ws[i]->rows;
        j.out_stride[i] = strides ? strides[i] : ws[i]->rows;
        j.wg_begin[i] = wg;
        wg += (ws[i]->rows + kRowsPerWG - 1) / kRowsPerWG;
    }
    j.wg_begin[n] = wg;
    if (wg == 0) return GLLM_OK;
    if (w0->type == GLLM_TYPE_Q4_K && p >= kMfmaMinTok) {
        // batched prefill: matrix-core products, same bits as the row kernel
        for (int i = 0; i < n; i++)
            GLLM_TRY(launch_q4k_mfma(ws[i]->d_data, ws[i]->row_bytes, ws[i]->rows, ws[i]->blocks,
                                     act, p, outs[i], j.out_stride[i], s));
        return GLLM_OK;
    }
    if (w0->type == GLLM_TYPE_Q8_0 && p > kTiledMinP && (size_t)w0->rows * w0->row_bytes < ((size_t)1 << 32) &&
        (size_t)p * w0->cols < ((size_t)1 << 32)) {
        for (int i = 0; i < n; i++)
            GLLM_TRY(launch_q8_0_tiled(ws[i]->d_data, ws[i]->row_bytes, ws[i]->rows, ws[i]->blocks,
                                       act, p, outs[i], j.out_stride[i], s));
        return GLLM_OK;
    }
    if (w0->type == GLLM_TYPE_Q6_K && q6k_tiled_fits(act, p, w0)) {
        for (int i = 0; i < n; i++)
            GLLM_TRY(launch_q6k_tiled(ws[i]->d_data, ws[i]->row_bytes, ws[i]->rows, ws[i]->blocks,
                                      act, p, outs[i], j.out_stride[i], s));
        return GLLM_OK;
    }
    for (int t0 = 0; t0 < p; t0 += kMaxTok) {
        j.tok0 = t0;
        j.ntok = std::min(kMaxTok, p - t0);
        int rc = j.ntok == 1 ? launch_gemv_nt<1>(j, w0->type, wg, j.rows, s)
               : j.ntok <= 4 ? launch_gemv_nt<4>(j, w0->type, wg, j.rows, s)
                             : launch_gemv_nt<8>(j, w0->type, wg, j.rows, s);
        GLLM_TRY(rc);
    }
    return GLLM_OK;
}

// True when the batch-1 row kernels for these weights quantise x themselves.
bool fused_quant(int n, gllm_hip_weight* const* ws) {
    // every workgroup quantises the whole of x: worth it for rows up to 4096
    // wide (one launch instead of two); wider rows pay more in-kernel work
    // than the separate launch costs
    if (ws[0]->cols > kFuseCols) return false;
    if (ws[0]->type != GLLM_TYPE_Q4_K) return true;
    int total = 0;
    for (int i = 0; i < n; i++) total += ws[i]->rows;
    const Q4KShape sh = q4k_shape(total, ws[0]->blocks);
    return sh.threads >= 256 && q4k_has_nl(ws[0]->blocks / sh.g) &&
           q4k_stage_bytes(1, ws[0]->cols) <= kMaxStage;
}

// W.x for p rows of f32 activations and n weights of one cols: each run of
// consecutive weights of one type is one row-kernel launch (the run's
// kernel quantises x itself at batch 1 when its shape allows), and every run
// that reads pre-quantised activations shares one q8kQuantize + xsums into
// `act` (act_bytes(cols, p) bytes of device scratch).  Runs of different
// types are what the reference's mixed groups compute: one int8 row dot per
// projection (tryMatvecAttentionInto, model.go:3156-3190;
// matvecBatchQ8Fused, kernels_portable_tunables.go:304-408).
int gemv_f32(int n, gllm_hip_weight* const* ws, const float* d_xs, int p, float* const* outs,
             const int* strides, void* act_buf, hipStream_t s) {
    const int cols = ws[0]->cols;
    ActQ8 act{};
    bool quantised = false;
    for (int i = 0; i < n;) {
        int e = i + 1;
        while (e < n && ws[e]->type == ws[i]->type) e++;
        const int m = e - i;
        const int* st = strides ? strides + i : nullptr;
        if (p == 1 && fused_quant(m, ws + i)) {
            ActQ8 none{};
            GLLM_TRY(run_gemv(m, ws + i, none, 1, outs + i, st, s, d_xs));
        } else {
            if (!quantised) {
                act_carve(act_buf, cols, p, &act);
                GLLM_TRY(launch_q8k_prep(d_xs, cols, p, act, s));
                quantised = true;
            }
            GLLM_TRY(run_gemv(m, ws + i, act, p, outs + i, st, s, nullptr));
        }
        i = e;
    }
    return GLLM_OK;
}

// True when W.x and its greedy argmax can run as one launch
// (argmax_epilogue): a Q6_K weight whose batch-1 kernel quantises x itself.
bool argmax_fusable(const gllm_hip_weight* w) {
    gllm_hip_weight* ws[1] = {const_cast<gllm_hip_weight*>(w)};
    return w->type == GLLM_TYPE_Q6_K && fused_quant(1, ws);
}

// Entries of the key buffer the argmax epilogue needs for w: one per
// workgroup of its batch-1 launch (32 / G rows each).
size_t argmax_epilogue_keys(const gllm_hip_weight* w) {
    const int g = row_lanes_g(w->rows, w->blocks, 1, w->type);
    return (size_t)(w->rows + kRowsPerWG / g - 1) / (kRowsPerWG / g);
}

// logits = W.x (batch 1) and, in the same launch, the workgroups' argmax
// keys of the logits after the repeat penalty over recent[0 .. n_recent); then
// argmax_final_kernel reduces the keys into *token.  keys: device memory of
// argmax_epilogue_keys(w) entries.
int gemv_argmax_f32(gllm_hip_weight* w, const float* x, float* logits, unsigned long long* keys,
                    uint32_t* token, const uint32_t* recent, int n_recent, float penalty,
                    hipStream_t s) {
    if (!argmax_fusable(w)) return fail(GLLM_EUNSUP, "gemv: no argmax epilogue for this weight");
    if (n_recent < 0 || (n_recent > 0 && !recent))
        return fail(GLLM_EINVAL, "argmax: bad recent-token window (%d ids)", n_recent);
    if (!(penalty > 0.0f) || penalty == INFINITY)
        return fail(GLLM_EINVAL, "argmax: repeat penalty must be finite and positive");
    const ArgmaxOut am{keys, recent, n_recent, penalty};
    gllm_hip_weight* ws[1] = {w};
    float* outs[1] = {logits};
    ActQ8 none{};
    GLLM_TRY(run_gemv(1, ws, none, 1, outs, nullptr, s, x, nullptr, &am));
    const int nk = (int)argmax_epilogue_keys(w);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(1024), 0, s, keys, nk, token);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

// True when a batch-1 group can take the RMSNorm prologue: Q4_K row kernels
// of one cols that quantise x themselves.
bool norm_fusable(int n, gllm_hip_weight* const* ws) {
    for (int i = 0; i < n; i++)
        if (ws[i]->type != GLLM_TYPE_Q4_K || ws[i]->cols != ws[0]->cols) return false;
    return fused_quant(n, ws);
}

// W.rmsNormInto(fma(res, 1, x), nw) for a batch-1 Q4_K group in one launch:
// ForwardBodyInto's addInPlace + rmsNormInto in front of the layer's fused
// projections (model.go:2686-2790); res may be null; xout (optional)
// receives fma(res, 1, x), the updated residual stream.
int gemv_norm_f32(int n, gllm_hip_weight* const* ws, const float* x, const float* res,
                  const float* nw, float eps, float* xout, float* const* outs, hipStream_t s) {
    if (!norm_fusable(n, ws)) return fail(GLLM_EUNSUP, "gemv: no RMSNorm prologue for this group");
    const NormIn ni{nw, res, xout, eps, nullptr, ActQ8{}};
    ActQ8 none{};
    return run_gemv(n, ws, none, 1, outs, nullptr, s, x, &ni);
}

// The decode step's FFN with the SwiGLU in the gate/up launch: gate/up =
// W1/W3 . rmsNormInto(fma(res, 1, x), nw) (one launch, norm prologue), whose
// last workgroup per 256-row block evaluates siluMulF32 for the block and
// quantises it into act_buf (the work of q8k_prep_silu); then down . act in
// the row kernel that reads pre-quantised activations.  Needs the gate/up
// shape to cover each 256-row block with whole workgroups and a down
// projection that does not quantise x itself (swiglu_epi_ok); cnt: hidden /
// 256 ints, zero between calls (each block's last workgroup resets its own).
bool swiglu_epi_ok(gllm_hip_weight* const* gu, const gllm_hip_weight* down) {
    if (!norm_fusable(2, gu) || gu[0]->rows != gu[1]->rows || gu[0]->rows % 256 ||
        down->cols != gu[0]->rows || !row_kernel_type(down->type))
        return false;
    gllm_hip_weight* dw[1] = {const_cast<gllm_hip_weight*>(down)};
    if (fused_quant(1, dw)) return false;
    const Q4KShape sh = q4k_shape(2 * gu[0]->rows, gu[0]->blocks);
    return sh.rows_per_wg > 0 && 256 % sh.rows_per_wg == 0;
}

int gemv_norm_swiglu_f32(gllm_hip_weight* const* gu, gllm_hip_weight* down, const float* x,
                         const float* res, const float* nw, float eps, float* xout, float* gate,
                         float* up, float* out, void* act_buf, int* cnt, hipStream_t s) {
    if (!swiglu_epi_ok(gu, down)) return fail(GLLM_EUNSUP, "gemv: no SwiGLU epilogue for this FFN");
    ActQ8 act;
    act_carve(act_buf, down->cols, 1, &act);
    const NormIn ni{nw, res, xout, eps, cnt, act};
    float* outs[2] = {gate, up};
    ActQ8 none{};
    GLLM_TRY(run_gemv(2, gu, none, 1, outs, nullptr, s, x, &ni));
    gllm_hip_weight* dw[1] = {down};
    float* dout[1] = {out};
    return run_gemv(1, dw, act, 1, dout, nullptr, s, nullptr);
}

// W.siluMulF32(gate, up) for p rows (the FFN down projection): the SwiGLU is
// evaluated inside the Q8K quantiser when the row kernel takes pre-quantised
// activations; a fused-quantisation shape gets it materialised in `hidden`
// first.
int gemv_silu_f32(gllm_hip_weight* w, const float* gate, const float* up, int p, float* out,
                  void* act_buf, float* hidden, hipStream_t s) {
    gllm_hip_weight* ws[1] = {w};
    float* outs[1] = {out};
    if (p == 1 && fused_quant(1, ws)) {
        const size_t n = (size_t)w->cols;
        hipLaunchKernelGGL(silu_mul_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                           gate, up, hidden, n);
        GLLM_HIP(hipGetLastError());
        return gemv_f32(1, ws, hidden, 1, outs, nullptr, act_buf, s);
    }
    ActQ8 act;
    act_carve(act_buf, w->cols, p, &act);
    GLLM_TRY(launch_q8k_prep_silu(gate, up, w->cols, p, act, s));
    return run_gemv(1, ws, act, p, outs, nullptr, s, nullptr);
}

// Argument checks shared by every device matvec entry point.
int validate_matvec(int n, gllm_hip_weight* const* ws, int p, const int* strides) {
    for (int i = 0; i < n; i++) GLLM_TRY(validate_weight(ws[i]));
    for (int i = 1; i < n; i++)
        if (ws[i]->cols != ws[0]->cols)
            return fail(GLLM_EINVAL, "fused matvec needs one cols (%d vs %d)", ws[i]->cols,
                        ws[0]->cols);
    if (p <= 0) return fail(GLLM_EINVAL, "p = %d", p);
    for (int i = 0; i < n; i++)
        if (strides && strides[i] < ws[i]->rows) return fail(GLLM_EINVAL, "out stride < rows");
    return GLLM_OK;
}

// Fused batch-1 groups (tryMatvec2Into model.go:3186-3206 for two weights,
// tryMatvecAttentionInto model.go:3157-3184 for three): a same-type pair or
// triple of Q4_K or Q6_K, or Q4_K/Q4_K/Q6_K, runs the int8 row dots, which
// give each projection the value its own MatvecInto gives; a same-type pair
// or triple of another format runs the float kernels (matvecSameType2/3Into);
// for three weights without a same-type triple the first same-type pair of
// (0,1), (0,2), (1,2) is the fused one and the third runs on its own.
// fl[i] = 1 marks the weights that take the float kernels.
static bool pair_float(int ta, int tb) {
    return ta == tb && ta != GLLM_TYPE_Q4_K && ta != GLLM_TYPE_Q6_K;
}
int group_routing(int n, gllm_hip_weight* const* ws, int* fl) {
    for (int i = 0; i < n; i++) fl[i] = 0;
    if (n == 2) {
        fl[0] = fl[1] = pair_float(ws[0]->type, ws[1]->type);
    } else if (n == 3) {
        const int t0 = ws[0]->type, t1 = ws[1]->type, t2 = ws[2]->type;
        if (t0 == t1 && t0 == t2) {
            fl[0] = fl[1] = fl[2] = pair_float(t0, t0);
        } else if (!(t0 == GLLM_TYPE_Q4_K && t1 == GLLM_TYPE_Q4_K && t2 == GLLM_TYPE_Q6_K)) {
            if (t0 == t1) fl[0] = fl[1] = pair_float(t0, t1);
            else if (t0 == t2) fl[0] = fl[2] = pair_float(t0, t2);
            else if (t1 == t2) fl[1] = fl[2] = pair_float(t1, t2);
        }
    }
    for (int i = 0; i < n; i++)
        if (fl[i] && !float_dot_type(ws[i]->type))
            return fail(GLLM_EUNSUP, "fused batch-1 group of type %d: the reference's float "
                                     "kernel for it (sameTypeQuantDot, model.go:3258-3283) "
                                     "is not restated here", ws[i]->type);
    return GLLM_OK;
}

// W.x for a batch-1 fused group: the float-kernel members in one launch,
// the others through gemv_f32's int8 row kernels.
int gemv_group(int n, gllm_hip_weight* const* ws, const float* d_x, float* const* outs,
               const int* strides, void* act_buf, hipStream_t s) {
    int fl[3];
    GLLM_TRY(group_routing(n, ws, fl));
    gllm_hip_weight* fw[3];
    gllm_hip_weight* iw[3];
    float* fo[3];
    float* io[3];
    int is[3];
    int nf = 0, ni = 0;
    for (int i = 0; i < n; i++) {
        if (fl[i]) {
            fw[nf] = ws[i];
            fo[nf++] = outs[i];
        } else {
            iw[ni] = ws[i];
            is[ni] = strides ? strides[i] : ws[i]->rows;
            io[ni++] = outs[i];
        }
    }
    if (nf) GLLM_TRY(launch_float_dot(nf, fw, d_x, fo, s));
    if (ni) GLLM_TRY(gemv_f32(ni, iw, d_x, 1, io, is, act_buf, s));
    return GLLM_OK;
}

int matvec_multi(int n, gllm_hip_weight* const* ws, const float* d_xs, int p, float* const* outs,
                 const int* strides, hipStream_t s, int scratch_slot) {
    GLLM_TRY(validate_matvec(n, ws, p, strides));
    void* sc = thread_scratch(scratch_slot, act_bytes(ws[0]->cols, p), s);
    if (!sc) return scratch_error();
    if (n > 1 && p == 1) return gemv_group(n, ws, d_xs, outs, strides, sc, s);
    return gemv_f32(n, ws, d_xs, p, outs, strides, sc, s);
}

}  // namespace gllm

using namespace gllm;

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {
static gllm_hip_weight* weight_upload(const void* data, size_t len, int ggml_type, int rows,
                                      int cols);
static int matvec_host(int n, gllm_hip_weight* const* ws, const float* x, int p,
                       float* const* outs);


// F32 / F16 / BF16 weights hold rows for gllm_hip_weight_rows_dev (any
// cols); the block formats need whole 256-element super-blocks per row.
static gllm_hip_weight* weight_alloc(int ggml_type, int rows, int cols, size_t len) {
    const bool scalar = ggml_type == GLLM_TYPE_F32 || ggml_type == GLLM_TYPE_F16 ||
                        ggml_type == GLLM_TYPE_BF16;
    if (!row_kernel_type(ggml_type) && !scalar) {
        fail(GLLM_EUNSUP, "weight type %d not supported", ggml_type);
        return nullptr;
    }
    if (rows <= 0 || cols <= 0 || (!scalar && cols % 256)) {
        fail(GLLM_EINVAL, "weight shape %dx%d (cols must be a positive multiple of 256)", rows, cols);
        return nullptr;
    }
    const size_t rb = ref_row_bytes(ggml_type, cols);
    if (len < rb * (size_t)rows) {
        fail(GLLM_EINVAL, "weight bytes %zu < rows*row_bytes %zu", len, rb * (size_t)rows);
        return nullptr;
    }
    gllm_hip_weight* w = new gllm_hip_weight();
    w->type = ggml_type;
    w->rows = rows;
    w->cols = cols;
    w->blocks = cols / 256;
    w->row_bytes = rb;
    if (hipGetDevice(&w->device) != hipSuccess) w->device = 0;
    if (hipMalloc(&w->d_data, rb * (size_t)rows) != hipSuccess) {
        (void)hipGetLastError();
        fail(GLLM_ENOMEM, "hipMalloc(%zu) for weight failed", rb * (size_t)rows);
        delete w;
        return nullptr;
    }
    return w;
}

static gllm_hip_weight* weight_finish(gllm_hip_weight* w, const uint8_t* d_src, hipStream_t s) {
    int rc = launch_repack(d_src, w->d_data, w->type, w->rows, w->blocks, w->row_bytes, 0, s);
    if (rc == GLLM_OK) rc = check(hipStreamSynchronize(s), "weight upload");
    if (rc != GLLM_OK) {
        (void)hipFree(w->d_data);
        delete w;
        return nullptr;
    }
    return w;
}

static gllm_hip_weight* weight_upload(const void* data, size_t len, int ggml_type, int rows,
                                      int cols) {
    gllm_hip_weight* w = weight_alloc(ggml_type, rows, cols, len);
    if (!w) return nullptr;
    hipStream_t s = thread_stream();
    const size_t bytes = w->row_bytes * (size_t)rows;
    void* tmp = nullptr;
    if (hipMalloc(&tmp, bytes) != hipSuccess) {
        (void)hipGetLastError();
        fail(GLLM_ENOMEM, "hipMalloc(%zu) for weight staging failed", bytes);
        (void)hipFree(w->d_data);
        delete w;
        return nullptr;
    }
    if (check(hipMemcpy(tmp, data, bytes, hipMemcpyHostToDevice), "upload weight") != GLLM_OK) {
        (void)hipFree(tmp);
        (void)hipFree(w->d_data);
        delete w;
        return nullptr;
    }
    gllm_hip_weight* out = weight_finish(w, (const uint8_t*)tmp, s);
    (void)hipFree(tmp);
    return out;
}

gllm_hip_weight* gllm_hip_weight_new(const void* data, size_t len, int ggml_type, int rows,
                                     int cols) {
    if (!data) {
        fail(GLLM_EINVAL, "gllm_hip_weight_new: null data");
        return nullptr;
    }
    if (self_check() != GLLM_OK) return nullptr;
    return weight_upload(data, len, ggml_type, rows, cols);
}

gllm_hip_weight* gllm_hip_weight_from_device(const void* d_data, size_t len, int ggml_type,
                                             int rows, int cols, void* stream) {
    if (!d_data) {
        fail(GLLM_EINVAL, "gllm_hip_weight_from_device: null data");
        return nullptr;
    }
    if (self_check() != GLLM_OK) return nullptr;
    gllm_hip_weight* w = weight_alloc(ggml_type, rows, cols, len);
    if (!w) return nullptr;
    // NULL is the legacy default stream, as for every _dev entry point: the
    // repack must be ordered after whatever produced d_data on that stream.
    return weight_finish(w, (const uint8_t*)d_data, (hipStream_t)stream);
}

void gllm_hip_weight_release(gllm_hip_weight* w) {
    if (!w) return;
    if (w->d_data) (void)hipFree(w->d_data);
    delete w;
}

int gllm_hip_weight_shape(const gllm_hip_weight* w, int* ggml_type, int* rows, int* cols) {
    if (!w) return fail(GLLM_EINVAL, "null weight handle");
    if (ggml_type) *ggml_type = w->type;
    if (rows) *rows = w->rows;
    if (cols) *cols = w->cols;
    return GLLM_OK;
}

int gllm_hip_weight_download_dev(const gllm_hip_weight* w, void* d_dst, void* stream) {
    if (!w || !d_dst) return fail(GLLM_EINVAL, "gllm_hip_weight_download_dev: bad arguments");
    hipStream_t s = (hipStream_t)stream;
    return launch_repack(w->d_data, (uint8_t*)d_dst, w->type, w->rows, w->blocks, w->row_bytes, 1, s);
}

int gllm_hip_matvec_dev(gllm_hip_weight* w, const float* d_xs, int p, float* d_outs,
                        int out_stride, void* stream) {
    if (!d_xs || !d_outs) return fail(GLLM_EINVAL, "gllm_hip_matvec_dev: null pointer");
    gllm_hip_weight* ws[1] = {w};
    float* outs[1] = {d_outs};
    int strides[1] = {out_stride > 0 ? out_stride : (w ? w->rows : 0)};
    return matvec_multi(1, ws, d_xs, p, outs, strides, (hipStream_t)stream, 0);
}

int gllm_hip_matvec_multi_dev(int n, gllm_hip_weight* const* ws, const float* d_xs, int p,
                              float* const* d_outs, const int* out_strides, void* stream) {
    if (!ws || !d_xs || !d_outs || n < 1 || n > 3)
        return fail(GLLM_EINVAL, "gllm_hip_matvec_multi_dev: bad arguments");
    for (int i = 0; i < n; i++)
        if (!d_outs[i]) return fail(GLLM_EINVAL, "gllm_hip_matvec_multi_dev: null output");
    return matvec_multi(n, ws, d_xs, p, d_outs, out_strides, (hipStream_t)stream, 0);
}

int gllm_hip_swiglu_down_dev(gllm_hip_weight* gate, gllm_hip_weight* up, gllm_hip_weight* down,
                             const float* d_x, float* d_out, void* stream) {
    if (!d_x || !d_out) return fail(GLLM_EINVAL, "gllm_hip_swiglu_down_dev: null pointer");
    gllm_hip_weight* ws[2] = {gate, up};
    GLLM_TRY(validate_matvec(2, ws, 1, nullptr));
    GLLM_TRY(validate_weight(down));
    if (gate->rows != up->rows || down->cols != gate->rows)
        return fail(GLLM_EINVAL, "gllm_hip_swiglu_down_dev: gate/up rows %d/%d, down cols %d",
                    gate->rows, up->rows, down->cols);
    hipStream_t s = (hipStream_t)stream;
    const int hidden = gate->rows;
    float* buf = (float*)thread_scratch(9, (size_t)hidden * 3 * 4, s);
    void* act = thread_scratch(0, act_bytes(std::max(gate->cols, hidden), 1), s);
    if (!buf || !act) return scratch_error();
    float* outs[2] = {buf, buf + hidden};
    GLLM_TRY(gemv_group(2, ws, d_x, outs, nullptr, act, s));
    return gemv_silu_f32(down, buf, buf + hidden, 1, d_out, act, buf + 2 * (size_t)hidden, s);
}

size_t gllm_hip_act_bytes(int cols, int p) {
    if (cols <= 0 || cols % 256 || p <= 0) return 0;
    return act_bytes(cols, p);
}

int gllm_hip_q8k_prepare_dev(const float* d_xs, int cols, int p, void* d_act, void* stream) {
    if (!d_xs || !d_act || cols <= 0 || cols % 256 || p <= 0)
        return fail(GLLM_EINVAL, "gllm_hip_q8k_prepare_dev: bad arguments");
    ActQ8 act;
    act_carve(d_act, cols, p, &act);
    return launch_q8k_prep(d_xs, cols, p, act, (hipStream_t)stream);
}

int gllm_hip_matvec_q8_dev(gllm_hip_weight* w, const void* d_act, int p, float* d_outs,
                           int out_stride, void* stream) {
    GLLM_TRY(validate_weight(w));
    if (!d_act || !d_outs || p <= 0) return fail(GLLM_EINVAL, "gllm_hip_matvec_q8_dev: bad arguments");
    if (out_stride <= 0) out_stride = w->rows;
    if (out_stride < w->rows) return fail(GLLM_EINVAL, "out stride < rows");
    ActQ8 act;
    act_carve((void*)d_act, w->cols, p, &act);
    gllm_hip_weight* ws[1] = {w};
    float* outs[1] = {d_outs};
    int strides[1] = {out_stride};
    return run_gemv(1, ws, act, p, outs, strides, (hipStream_t)stream, nullptr);
}

// Host-pointer forms: stage through pinned memory on the thread's stream.
static int matvec_host(int n, gllm_hip_weight* const* ws, const float* x, int p, float* const* outs) {
    for (int i = 0; i < n; i++) GLLM_TRY(validate_weight(ws[i]));
    if (!x || p <= 0) return fail(GLLM_EINVAL, "matvec: bad input");
    hipStream_t s = thread_stream();
    if (!s) return GLLM_EDEVICE;
    const int cols = ws[0]->cols;
    size_t out_total = 0;
    for (int i = 0; i < n; i++) out_total += (size_t)ws[i]->rows * p;
    float* d_x = (float*)thread_scratch(1, (size_t)cols * p * 4, s);
    float* d_out = (float*)thread_scratch(2, out_total * 4, s);
    if (!d_x || !d_out) return scratch_error();
    GLLM_HIP(hipMemcpyAsync(d_x, x, (size_t)cols * p * 4, hipMemcpyHostToDevice, s));
    float* douts[3];
    int strides[3];
    size_t off = 0;
    for (int i = 0; i < n; i++) {
        douts[i] = d_out + off;
        strides[i] = ws[i]->rows;
        off += (size_t)ws[i]->rows * p;
    }
    GLLM_TRY(matvec_multi(n, ws, d_x, p, douts, strides, s, 0));
    for (int i = 0; i < n; i++)
        GLLM_HIP(hipMemcpyAsync(outs[i], douts[i], (size_t)ws[i]->rows * p * 4,
                                hipMemcpyDeviceToHost, s));
    GLLM_HIP(hipStreamSynchronize(s));
    return GLLM_OK;
}

int gllm_hip_matvec(gllm_hip_weight* w, const float* x, float* out) {
    if (!out) return fail(GLLM_EINVAL, "gllm_hip_matvec: null out");
    gllm_hip_weight* ws[1] = {w};
    float* outs[1] = {out};
    return matvec_host(1, ws, x, 1, outs);
}

int gllm_hip_matvec2(gllm_hip_weight* a, gllm_hip_weight* b, const float* x, float* out_a,
                     float* out_b) {
    if (!out_a || !out_b) return fail(GLLM_EINVAL, "gllm_hip_matvec2: null out");
    gllm_hip_weight* ws[2] = {a, b};
    float* outs[2] = {out_a, out_b};
    return matvec_host(2, ws, x, 1, outs);
}

int gllm_hip_matvec3(gllm_hip_weight* a, gllm_hip_weight* b, gllm_hip_weight* c, const float* x,
                     float* out_a, float* out_b, float* out_c) {
    if (!out_a || !out_b || !out_c) return fail(GLLM_EINVAL, "gllm_hip_matvec3: null out");
    gllm_hip_weight* ws[3] = {a, b, c};
    float* outs[3] = {out_a, out_b, out_c};
    return matvec_host(3, ws, x, 1, outs);
}

int gllm_hip_matvec_batch(gllm_hip_weight* w, const float* xs, int p, float* outs) {
    if (!outs) return fail(GLLM_EINVAL, "gllm_hip_matvec_batch: null out");
    gllm_hip_weight* ws[1] = {w};
    float* o[1] = {outs};
    return matvec_host(1, ws, xs, p, o);
}

int gllm_hip_argmax_penalized_dev(gllm_hip_weight* w, const float* d_x, const uint32_t* d_recent,
                                  int n_recent, float penalty, uint32_t* d_token, void* stream) {
    GLLM_TRY(validate_weight(w));
    if (!d_x || !d_token) return fail(GLLM_EINVAL, "gllm_hip_argmax_dev: null pointer");
    hipStream_t s = (hipStream_t)stream;
    float* logits = (float*)thread_scratch(3, (size_t)w->rows * 4, s);
    if (!logits) return scratch_error();
    gllm_hip_weight* ws[1] = {w};
    float* outs[1] = {logits};
    int strides[1] = {w->rows};
    GLLM_TRY(matvec_multi(1, ws, d_x, 1, outs, strides, s, 0));
    auto* keys = (unsigned long long*)thread_scratch(7, argmax_keys(w->rows) * 8, s);
    if (!keys) return scratch_error();
    return launch_argmax(logits, w->rows, d_token, keys, s, d_recent, n_recent, penalty);
}

int gllm_hip_argmax_dev(gllm_hip_weight* w, const float* d_x, uint32_t* d_token, void* stream) {
    return gllm_hip_argmax_penalized_dev(w, d_x, nullptr, 0, 1.0f, d_token, stream);
}

int gllm_hip_argmax_penalized(gllm_hip_weight* w, const float* x, const uint32_t* recent,
                              int n_recent, float penalty, uint32_t* token) {
    GLLM_TRY(validate_weight(w));
    if (!x || !token) return fail(GLLM_EINVAL, "gllm_hip_argmax: null pointer");
    if (n_recent < 0 || (n_recent > 0 && !recent))
        return fail(GLLM_EINVAL, "gllm_hip_argmax_penalized: bad recent-token window");
    hipStream_t s = thread_stream();
    if (!s) return GLLM_EDEVICE;
    float* d_x = (float*)thread_scratch(1, (size_t)w->cols * 4, s);
    uint32_t* d_tok = (uint32_t*)thread_scratch(4, 64, s);
    uint32_t* h_tok = (uint32_t*)thread_pinned(0, 64);
    if (!d_x || !d_tok || !h_tok) return GLLM_ENOMEM;
    uint32_t* d_recent = nullptr;
    if (n_recent > 0) {
        d_recent = (uint32_t*)thread_scratch(8, (size_t)n_recent * 4, s);
        if (!d_recent) return scratch_error();
        GLLM_HIP(hipMemcpyAsync(d_recent, recent, (size_t)n_recent * 4, hipMemcpyHostToDevice, s));
    }
    GLLM_HIP(hipMemcpyAsync(d_x, x, (size_t)w->cols * 4, hipMemcpyHostToDevice, s));
    GLLM_TRY(gllm_hip_argmax_penalized_dev(w, d_x, d_recent, n_recent, penalty, d_tok, s));
    GLLM_HIP(hipMemcpyAsync(h_tok, d_tok, 4, hipMemcpyDeviceToHost, s));
    GLLM_HIP(hipStreamSynchronize(s));
    *token = *h_tok;
    return GLLM_OK;
}

int gllm_hip_argmax(gllm_hip_weight* w, const float* x, uint32_t* token) {
    return gllm_hip_argmax_penalized(w, x, nullptr, 0, 1.0f, token);
}

int gllm_hip_lane_ints_dev(gllm_hip_weight* w, const float* d_x, int32_t* d_ints, void* stream) {
    GLLM_TRY(validate_weight(w));
    if (!d_x || !d_ints) return fail(GLLM_EINVAL, "gllm_hip_lane_ints_dev: null pointer");
    hipStream_t s = (hipStream_t)stream;
    void* sc = thread_scratch(0, act_bytes(w->cols, 1), s);
    if (!sc) return scratch_error();
    ActQ8 act;
    act_carve(sc, w->cols, 1, &act);
    GLLM_TRY(launch_q8k_prep(d_x, w->cols, 1, act, s));
    const int grid = (w->rows + kRowsPerWG - 1) / kRowsPerWG;
    hipLaunchKernelGGL(lane_ints_kernel, dim3(grid), dim3(256), 0, s, w->d_data, w->type, w->rows,
                       w->blocks, w->row_bytes, act, d_ints);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Load-time known-answer check (the reference's q8kSelfCheck,
// q8k_dot_arm64.go:146-228, which disables a kernel whose integer dots
// disagree with a restated answer).  Once per device, before the first weight
// is created, small Q4_K, Q6_K and Q8_0 matrices go through the same matvec
// path every caller uses (upload and repack, Q8K quantisation, row kernel,
// float chains, lane tree).  The inputs are chosen so that the answer is an
// integer the float path must hit exactly:
//   * x holds integers in [-3, 3] with one 127 per 256-block, so the Q8K
//     scale is exactly 1 and q8 == x (kernels_amd64.s:348-436);
//   * every f16 d / dmin is 1.0, so each row dot is sum_e w_e * x_e with the
//     integer weight w_e = sc*q - m (Q4_K), sc*(q - 32) (Q6_K) or q (Q8_0);
//   * pattern rows keep sum_e (|A_e| + |B_e|) |x_e| below 2^24 (A, B: the
//     scale chain's and the min / offset chain's integer terms), so every
//     partial sum of every lane chain and of the lane tree is exact;
//   * the Q4_K all-0xff row with x = 127 everywhere (TestAuditQ4KDotExtremes,
//     q4k_q8_amd64_audit_test.go:18-52) gives 28,675,584 per block:
//     all lanes hold equal even values, so each tree addition is exact too.
// On a mismatch no weight can be created on that device and every weight
// constructor fails with GLLM_EUNSUP, which sends the Go seam to its CPU
// kernels.  GLLM_SELF_CHECK_PLANT=1 adds one to a host-side expected value
// (a planted mistake on the CPU), so the refusal path can be tested.
// ---------------------------------------------------------------------------
namespace gllm {
namespace {

// 8192 rows take the fused-quantiser row kernels of every format at batch
// 1, as a full-size matrix does
constexpr int kCheckRows = 8192;

uint8_t check_byte(int i, int mul, int add) { return (uint8_t)(i * mul + add); }

// getScaleMinK4 (simd.go:1672-1677)
void scale_min_k4(int j, const uint8_t* q, int* sc, int* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// Integer terms of element e of a block (GGUF layout, d = dmin = 1): the
// scale chain's term A and the min / offset chain's term B, weight A - B.
void check_terms(int type, const uint8_t* blk, int e, int* A, int* B) {
    if (type == GLLM_TYPE_Q4_K) {
        int sc, m;
        scale_min_k4(e / 32, blk + 4, &sc, &m);
        const int s = e / 64, l = e % 32;
        const uint8_t qb = blk[16 + 32 * s + l];
        *A = sc * ((e / 32) % 2 ? qb >> 4 : qb & 15);
        *B = m;
        return;
    }
    if (type == GLLM_TYPE_Q6_K) {
        const int h = e / 128, r = e % 128, l = r % 32, quad = r / 32;
        const uint8_t* ql = blk + 64 * h;
        const uint8_t qh = blk[128 + 32 * h + l];
        const int lo = quad & 1 ? ql[l + 32] : ql[l];
        const int q = (quad < 2 ? lo & 15 : lo >> 4) | (((qh >> (2 * quad)) & 3) << 4);
        const int sc = (int)(int8_t)blk[192 + 8 * h + l / 16 + 2 * quad];
        *A = sc * q;
        *B = 32 * sc;
        return;
    }
    *A = (int)(int8_t)blk[(e / 32) * 34 + 2 + e % 32];  // Q8_0
    *B = 0;
}

// One format: kCheckRows rows of pattern bytes against a pattern x of
// integers in [-xr, xr] (one 127 per block), and for Q4_K the all-0xff row
// against x = 127.  Returns GLLM_OK, or GLLM_EUNSUP on a wrong answer.
int check_format(int type, int cols, int xr, bool plant) {
    const size_t rb = ref_row_bytes(type, cols);
    const size_t bb = rb / (cols / 256);  // bytes per 256 elements
    std::vector<uint8_t> w(rb * kCheckRows);
    for (int r = 0; r < kCheckRows; r++)
        for (size_t i = 0; i < rb; i++) w[r * rb + i] = check_byte((int)i, 7 + 6 * r + type, 3 * r + 1);
    for (int r = 0; r < kCheckRows; r++)
        for (int b = 0; b < cols / 256; b++) {
            uint8_t* blk = &w[r * rb + b * bb];
            if (type == GLLM_TYPE_Q4_K) {
                blk[0] = 0x00, blk[1] = 0x3c, blk[2] = 0x00, blk[3] = 0x3c;  // d = dmin = 1
            } else if (type == GLLM_TYPE_Q6_K) {
                blk[208] = 0x00, blk[209] = 0x3c;
            } else {
                for (int j = 0; j < 8; j++) blk[34 * j] = 0x00, blk[34 * j + 1] = 0x3c;
            }
        }
    std::vector<float> x(cols);
    for (int i = 0; i < cols; i++) x[i] = (float)((i * 37 + 11) % (2 * xr + 1) - xr);
    for (int b = 0; b < cols / 256; b++) x[b * 256 + (b * 41) % 256] = 127.0f;
    std::vector<float> want(kCheckRows);
    for (int r = 0; r < kCheckRows; r++) {
        long long acc = 0, mag = 0;
        for (int e = 0; e < cols; e++) {
            int A, B;
            check_terms(type, &w[r * rb + (e / 256) * bb], e % 256, &A, &B);
            const long long xe = (long long)x[e];
            acc += (long long)(A - B) * xe;
            mag += (long long)((A < 0 ? -A : A) + (B < 0 ? -B : B)) * (xe < 0 ? -xe : xe);
        }
        // every partial sum of either chain, and of the lane tree, is bounded
        // by mag: below 2^24 they are all exact in float
        if (mag >= (1LL << 24)) return fail(GLLM_EUNSUP, "self-check pattern out of range");
        want[r] = (float)acc;
    }
    if (plant) want[1] += 1.0f;
    gllm_hip_weight* h = weight_upload(w.data(), w.size(), type, kCheckRows, cols);
    if (!h) return GLLM_EDEVICE;
    std::vector<float> got(kCheckRows);
    gllm_hip_weight* ws[1] = {h};
    float* outs[1] = {got.data()};
    int rc = matvec_host(1, ws, x.data(), 1, outs);
    gllm_hip_weight_release(h);
    GLLM_TRY(rc);
    for (int r = 0; r < kCheckRows; r++)
        if (got[r] != want[r])
            return fail(GLLM_EUNSUP, "self-check: type %d row %d gave %.9g, known answer %.9g", type,
                        r, got[r], want[r]);
    if (type == GLLM_TYPE_Q4_K) {
        std::vector<uint8_t> ext(rb, 0xff);
        for (int b = 0; b < cols / 256; b++)
            ext[b * bb] = 0x00, ext[b * bb + 1] = 0x3c, ext[b * bb + 2] = 0x00, ext[b * bb + 3] = 0x3c;
        std::vector<float> x127(cols, 127.0f);
        gllm_hip_weight* he = weight_upload(ext.data(), ext.size(), type, 1, cols);
        if (!he) return GLLM_EDEVICE;
        float g = 0.0f;
        gllm_hip_weight* we[1] = {he};
        float* oe[1] = {&g};
        rc = matvec_host(1, we, x127.data(), 1, oe);
        gllm_hip_weight_release(he);
        GLLM_TRY(rc);
        // (63*15*127*256 - 8*63*32*127) per block
        const float ew = 28675584.0f * (float)(cols / 256);
        if (g != ew)
            return fail(GLLM_EUNSUP, "self-check: Q4_K extremes gave %.9g, known answer %.9g", g, ew);
    }
    return GLLM_OK;
}

std::mutex g_check_mu;
int g_check_state[64];  // per device: 0 not run, 1 passed, <0 the failure code
std::string g_check_msg[64];

}  // namespace

int noalloc_prepare();

int self_check() {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= 64) {
        (void)hipGetLastError();
        return fail(GLLM_EDEVICE, "no HIP device");
    }
    std::lock_guard<std::mutex> lock(g_check_mu);
    if (g_check_state[d] == 0) {
        const char* e = getenv("GLLM_SELF_CHECK_PLANT");
        const bool plant = e && atoi(e) == 1;
        int rc = GLLM_OK;
        // Q6_K's chains carry |sc| * 95 per unit of x, so it takes two blocks
        // of x in [-1, 1] to stay below 2^24
        if (rc == GLLM_OK) rc = check_format(GLLM_TYPE_Q4_K, 1024, 3, plant);
        if (rc == GLLM_OK) rc = check_format(GLLM_TYPE_Q6_K, 512, 1, plant);
        if (rc == GLLM_OK) rc = check_format(GLLM_TYPE_Q8_0, 1024, 3, plant);
        // the allocation-free entry point's device scratch, looked up now,
        // outside any capture a caller may start later
        if (rc == GLLM_OK) rc = noalloc_prepare();
        if (rc == GLLM_OK) {
            g_check_state[d] = 1;
        } else {
            g_check_state[d] = rc == GLLM_EDEVICE ? 0 : rc;  // a device error is retried
            g_check_msg[d] = gllm_hip_last_error();
            return rc;
        }
    }
    if (g_check_state[d] < 0)
        return fail(g_check_state[d], "device %d failed the load-time known-answer check (%s)", d,
                    g_check_msg[d].c_str());
    return GLLM_OK;
}

}  // namespace gllm
