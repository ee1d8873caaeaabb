// prefill.hip -- batched Q4_K x Q8_K products on the matrix cores.
//
// matvecBatchQ8 (kernels_amd64.go:470-581) runs the batch-1 row kernel
// q4kDotQ8KRow (kernels_amd64.s:437-543) once per (row, token), so a batched
// result must equal the per-token one bit for bit.  That kernel keeps eight
// AVX2 lanes per row; lane k owns the 32 elements {32j + 4k + i : j < 8,
// i < 4} of every 256-element block b and runs two float chains over b:
//   accF[k] = fma(float(I_bk), d_b * xscale_b, accF[k])
//   accM[k] = fma(dmin_b, float(m_bk) * xsum_bk, accM[k])
// with the exact integer I_bk = sum over its 32 elements of sc_j * q4 * q8,
// and ends with tree8(accF - accM).
//
// Here I_bk comes from v_mfma_f32_16x16x32_f16: the A operand holds
// sc_j * q4 (<= 63 * 15 = 945, exact in f16), the B operand q8 (exact in
// f16), and every partial sum of 32 products stays below 2^24, so the fp32
// accumulation is exact in any order and equals the int32 lane sum.  The
// float chains then run per (row, token, lane) in VALU registers in the
// reference's order.
//
// K order: lane k's elements are numbered kappa = 4j + i, which is the order
// of the lane-permuted Q8K activations (q8perm_offset) and, for the weights,
// of the upload repack: lane k's 16 nibble bytes sit at 16 + 16k, byte
// 4s + i holding elements kappa = 8s + i (low nibble, sub-block 2s) and
// 8s + 4 + i (high nibble, sub-block 2s + 1).  MFMA lane L supplies
// kappa = 8(L/16) .. 8(L/16) + 7 of both operands, i.e. one weight dword.
//
// Workgroup: RW x TW waves over 16 RW weight rows x 16 TW tokens; wave w
// owns the 16x16 tile of rows 16 (w % RW) .. + 15 and tokens
// 16 (w / RW) .. + 15.  Per block the workgroup
// stages the 32 tokens' q8 (as f16), xsums and xscales and the 64 rows'
// decoded scales/mins and nibble bytes in LDS (double-buffered, loaded one
// block ahead).
#include <cstdlib>

#include "gllm_common.h"

namespace gllm {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

constexpr int kPfBStride = 528;  // bytes per token row of the f16 q8 tile: 512 + 16 (no bank conflicts)
constexpr int kPfWStride = 36;   // dwords per row of the staged weight nibbles: 32 + 4

// One block's staged operands for a workgroup of RW 16-row groups x TW
// 16-token columns.
template <int RW, int TW>
struct PfStage {
    static constexpr int kRows = 16 * RW, kTok = 16 * TW;
    uint8_t b16[kTok * kPfBStride];
    float xsum[8][kTok];        // [lane k][token]
    float xsc[kTok];
    uint32_t sch[8][kRows];     // [sub-block j][row] half2(sc_j, sc_j)
    uint32_t scn[8][kRows];     // [sub-block j][row] half2(-1024 sc_j, -1024 sc_j)
    float m[8][kRows];          // [lane k][row]
    float d[kRows];
    float dmin[kRows];
    // nibble dwords per row as [group s][lane k] (lane (g, c) of a wave reads
    // its 8 dwords as 32 contiguous bytes); 36-dword rows keep the 16 rows'
    // 16-byte reads on distinct banks
    uint32_t wa[kRows][kPfWStride];
};

// four signed bytes -> two half2 words holding the same integers
__device__ __forceinline__ void i8x4_to_h(uint32_t w, uint32_t& lo, uint32_t& hi) {
    const uint32_t u = w ^ 0x80808080u;  // c + 128, as unsigned bytes
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x05010400u);  // 1024 + u0, 1024 + u1
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x05030402u);  // 1024 + u2, 1024 + u3
    typedef _Float16 h2v __attribute__((ext_vector_type(2)));
    const h2v bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    h2v ha = __builtin_bit_cast(h2v, a) + bias;  // exact: integers below 2048
    h2v hb = __builtin_bit_cast(h2v, b) + bias;
    lo = __builtin_bit_cast(uint32_t, ha);
    hi = __builtin_bit_cast(uint32_t, hb);
}

// one weight dword (4 nibble bytes of one lane and sub-block pair) -> the
// 8 f16 A values sc_lo * low nibbles, sc_hi * high nibbles
__device__ __forceinline__ h8v dequant_a(uint32_t w, uint32_t sch_lo, uint32_t scn_lo,
                                         uint32_t sch_hi, uint32_t scn_hi) {
    typedef _Float16 h2v __attribute__((ext_vector_type(2)));
    const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
    const h2v p0 = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, lo, 0x05010400u));
    const h2v p1 = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, lo, 0x05030402u));
    const h2v p2 = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, hi, 0x05010400u));
    const h2v p3 = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, hi, 0x05030402u));
    const h2v sl = __builtin_bit_cast(h2v, sch_lo), nl = __builtin_bit_cast(h2v, scn_lo);
    const h2v sh = __builtin_bit_cast(h2v, sch_hi), nh = __builtin_bit_cast(h2v, scn_hi);
    // (1024 + q) * sc - 1024 * sc == q * sc exactly: one rounding of an exact
    // value below 2048
    const h2v a0 = __builtin_elementwise_fma(p0, sl, nl);
    const h2v a1 = __builtin_elementwise_fma(p1, sl, nl);
    const h2v a2 = __builtin_elementwise_fma(p2, sh, nh);
    const h2v a3 = __builtin_elementwise_fma(p3, sh, nh);
    h8v r;
    r[0] = a0[0]; r[1] = a0[1]; r[2] = a1[0]; r[3] = a1[1];
    r[4] = a2[0]; r[5] = a2[1]; r[6] = a3[0]; r[7] = a3[1];
    return r;
}

struct PfArgs {
    const uint8_t* w;  // repacked Q4_K rows
    size_t rb;         // bytes per row
    int rows, blocks;
    ActQ8 act;         // p tokens of Q8K activations
    int p;
    float* out;        // out[t * out_stride + r]
    int out_stride;
};

// Staging registers of one block for T = 64 RW TW threads, mapped so that
// every LDS store of a wave hits distinct banks:
//   q8: unit u = (token u/16, part u%16), units tid, tid + T, ...: q8 bytes
//       8 part .. + 7 and 128 + 8 part .. + 7, written as f16 at 16 part and
//       256 + 16 part of the token's row;
//   threads 0 .. 2 kTok - 1 one xsum quad, threads 0 .. kTok - 1 one xscale;
//   unit u = (sub-block j = u / kRows, row u % kRows): the row's block header
//   and the 16 nibble bytes of lane k = j.
template <int RW, int TW>
struct PfRegs {
    static constexpr int T = 64 * RW * TW;
    static constexpr int NQ = 16 * 16 * TW / T;  // q8 units per thread
    static constexpr int NH = 8 * 16 * RW / T;   // header units per thread
    uint32_t q[NQ][4];
    f4v xs;
    float xc;
    u4v h[NH];
    u4v w[NH];
};

template <int RW, int TW>
__device__ __forceinline__ void pf_load(const PfArgs& a, int row0, int tok0, int b,
                                        PfRegs<RW, TW>& r) {
    using R = PfRegs<RW, TW>;
    constexpr int kRows = 16 * RW, kTok = 16 * TW;
    const int tid = threadIdx.x;
    const int cols = a.blocks * 256;
#pragma unroll
    for (int i = 0; i < R::NQ; i++) {
        const int u = tid + R::T * i;
        const int t = min(tok0 + (u >> 4), a.p - 1);
        const int8_t* src = a.act.q8perm + (size_t)t * cols + (size_t)b * 256 + 8 * (u & 15);
        const uint2 lo = *(const uint2*)src, hi = *(const uint2*)(src + 128);
        r.q[i][0] = lo.x; r.q[i][1] = lo.y; r.q[i][2] = hi.x; r.q[i][3] = hi.y;
    }
    if (tid < 2 * kTok) {
        const int t = min(tok0 + (tid >> 1), a.p - 1);
        r.xs = *(const f4v*)(a.act.xs32 + (size_t)t * (cols / 32) + b * 8 + 4 * (tid & 1));
    }
    if (tid < kTok) r.xc = a.act.xscale[(size_t)min(tok0 + tid, a.p - 1) * a.blocks + b];
#pragma unroll
    for (int i = 0; i < R::NH; i++) {
        const int u = tid + R::T * i;
        const int row = min(row0 + u % kRows, a.rows - 1);
        const uint8_t* rp = a.w + (size_t)row * a.rb;
        r.h[i] = *(const u4v*)(rp + q4k_hdr_off(b));
        r.w[i] = *(const u4v*)(rp + q4k_nib_off(a.blocks, b) + 16 * (u / kRows));
    }
}

template <int RW, int TW>
__device__ __forceinline__ void pf_store(const PfRegs<RW, TW>& r, PfStage<RW, TW>& st) {
    using R = PfRegs<RW, TW>;
    constexpr int kRows = 16 * RW, kTok = 16 * TW;
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < R::NQ; i++) {
        const int u = tid + R::T * i;
        uint32_t v[8];
        i8x4_to_h(r.q[i][0], v[0], v[1]);
        i8x4_to_h(r.q[i][1], v[2], v[3]);
        i8x4_to_h(r.q[i][2], v[4], v[5]);
        i8x4_to_h(r.q[i][3], v[6], v[7]);
        uint8_t* row = st.b16 + (u >> 4) * kPfBStride + 16 * (u & 15);
        *(u4v*)row = u4v{v[0], v[1], v[2], v[3]};
        *(u4v*)(row + 256) = u4v{v[4], v[5], v[6], v[7]};
    }
    if (tid < 2 * kTok) {
        const int t = tid >> 1, k0 = 4 * (tid & 1);
        st.xsum[k0][t] = r.xs.x;
        st.xsum[k0 + 1][t] = r.xs.y;
        st.xsum[k0 + 2][t] = r.xs.z;
        st.xsum[k0 + 3][t] = r.xs.w;
    }
    if (tid < kTok) st.xsc[tid] = r.xc;
#pragma unroll
    for (int i = 0; i < R::NH; i++) {
        // getScaleMinK4 (simd.go:1672-1677) for sub-block j
        const int u = tid + R::T * i;
        const int row = u % kRows, j = u / kRows;
        const uint32_t s03 = r.h[i].y, s47 = r.h[i].z, s811 = r.h[i].w;
        uint32_t sc, mn;
        if (j < 4) {
            sc = (s03 >> (8 * j)) & 63u;
            mn = (s47 >> (8 * j)) & 63u;
        } else {
            const int jj = j - 4;
            const uint32_t b8 = (s811 >> (8 * jj)) & 0xffu;
            sc = (b8 & 15u) | (((s03 >> (8 * jj + 6)) & 3u) << 4);
            mn = (b8 >> 4) | (((s47 >> (8 * jj + 6)) & 3u) << 4);
        }
        const _Float16 hs = (_Float16)(float)sc, hn = (_Float16)(-1024.0f * (float)sc);
        const uint32_t bs = __builtin_bit_cast(uint16_t, hs), bn = __builtin_bit_cast(uint16_t, hn);
        st.sch[j][row] = bs | (bs << 16);
        st.scn[j][row] = bn | (bn << 16);
        st.m[j][row] = (float)mn;
        if (j == 0) {
            st.d[row] = f16_bits_to_f32(r.h[i].x & 0xffffu);
            st.dmin[row] = f16_bits_to_f32(r.h[i].x >> 16);
        }
        // lane k = j's dwords for groups s = 0..3
        st.wa[row][0 * 8 + j] = r.w[i].x;
        st.wa[row][1 * 8 + j] = r.w[i].y;
        st.wa[row][2 * 8 + j] = r.w[i].z;
        st.wa[row][3 * 8 + j] = r.w[i].w;
    }
}

template <int RW, int TW>
// (two waves per SIMD for multi-wave workgroups; a one-wave workgroup, one
// per CU, may use the whole register file for its deeper staging)
__global__ __launch_bounds__(64 * RW * TW) __attribute__((amdgpu_waves_per_eu(RW * TW > 1 ? 2 : 1)))
void prefill_q4k_mfma_kernel(PfArgs a) {
    using Stage = PfStage<RW, TW>;
    __shared__ __align__(16) Stage stage[2];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int rw = wave % RW, tw = wave / RW;  // 16-row group, 16-token column
    const int row0 = blockIdx.x * Stage::kRows, tok0 = blockIdx.y * Stage::kTok;
    // D layout: rows 4g + i of the wave's 16, token c of its column
    const int lr = 16 * rw + 4 * g;
    const int lt = 16 * tw + c;

    float accF[4][8], accM[4][8];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int k = 0; k < 8; k++) accF[i][k] = accM[i][k] = 0.0f;

    // one block's products from a staged LDS tile
    auto block = [&](const Stage& st) __attribute__((always_inline)) {
        // this lane's A row (MFMA row c of the wave's 16): its 8 nibble dwords
        const u4v wq0 = *(const u4v*)&st.wa[16 * rw + c][8 * g];
        const u4v wq1 = *(const u4v*)&st.wa[16 * rw + c][8 * g + 4];
        const uint32_t wq[8] = {wq0.x, wq0.y, wq0.z, wq0.w, wq1.x, wq1.y, wq1.z, wq1.w};
        const uint32_t sh_lo = st.sch[2 * g][16 * rw + c], sn_lo = st.scn[2 * g][16 * rw + c];
        const uint32_t sh_hi = st.sch[2 * g + 1][16 * rw + c], sn_hi = st.scn[2 * g + 1][16 * rw + c];
        // F chain factors d * xscale per D row
        const f4v dv = *(const f4v*)&st.d[lr];
        const f4v dm = *(const f4v*)&st.dmin[lr];
        const float xc = st.xsc[lt];
        float dxs[4];
#pragma unroll
        for (int i = 0; i < 4; i++) dxs[i] = dv[i] * xc;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const h8v av = dequant_a(wq[k], sh_lo, sn_lo, sh_hi, sn_hi);
            const h8v bv = *(const h8v*)(st.b16 + lt * kPfBStride + 64 * k + 16 * g);
            const f4v z = {0.0f, 0.0f, 0.0f, 0.0f};
            const f4v dI = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, z, 0, 0, 0);
            // M chain operands: mins of the lane's 4 D rows, xsum of its token
            const f4v mk = *(const f4v*)&st.m[k][lr];
            const float xk = st.xsum[k][lt];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                accF[i][k] = fmaf(dI[i], dxs[i], accF[i][k]);
                const float mx = mk[i] * xk;
                accM[i][k] = fmaf(dm[i], mx, accM[i][k]);
            }
        }
    };

    // Two staging register sets: the global loads of block b + 2 are issued
    // while block b is computed and land in LDS after block b + 1 is.  The
    // loads are unconditional (past the end they re-read the last block):
    // under a branch the compiler's vmcnt wait for the older set would also
    // wait for the newer one and cancel the prefetch.
    const int nb = a.blocks;
    PfRegs<RW, TW> r0, r1;
    pf_load(a, row0, tok0, 0, r0);
    pf_store(r0, stage[0]);
    pf_load(a, row0, tok0, min(1, nb - 1), r1);
    __syncthreads();
#pragma unroll 1
    for (int b = 0; b < nb; b += 2) {
        pf_load(a, row0, tok0, min(b + 2, nb - 1), r0);
        block(stage[0]);
        if (b + 1 < nb) pf_store(r1, stage[1]);
        __syncthreads();
        if (b + 1 >= nb) break;
        pf_load(a, row0, tok0, min(b + 3, nb - 1), r1);
        block(stage[1]);
        if (b + 2 < nb) pf_store(r0, stage[0]);
        __syncthreads();
    }
    // tree8 of the reference's horizontal sum, then the (row, token) store
    const int t = tok0 + lt;
    if (t < a.p) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = row0 + lr + i;
            if (r >= a.rows) continue;
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = accF[i][k] - accM[i][k];
            const float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
            a.out[(size_t)t * a.out_stride + r] = (s0 + s1) + (s2 + s3);
        }
    }
}

template <int RW, int TW>
static void launch_pf(const PfArgs& a, hipStream_t s) {
    dim3 grid((a.rows + 16 * RW - 1) / (16 * RW), (a.p + 16 * TW - 1) / (16 * TW));
    hipLaunchKernelGGL((prefill_q4k_mfma_kernel<RW, TW>), grid, dim3(64 * RW * TW), 0, s, a);
}

// One block's per-row and per-token factors of a 16 x 16 tile (rows 0..15,
// tokens 0..15), shared by the waves of the 16-row kernels below.
struct SbParams {  // one block's factors: rows 0..15 and tokens 0..15 of the tile
    float d[16], dmin[16], m[8][16];
    float xs[16], xsum[8][16];
};
// getScaleMinK4 (simd.go:1672-1677): 6-bit scale and min of sub-block j
__device__ __forceinline__ void sb_scale_min(const u4v h, int j, uint32_t& sc, uint32_t& mn) {
    const uint32_t s03 = h.y, s47 = h.z, s811 = h.w;
    if (j < 4) {
        sc = (s03 >> (8 * j)) & 63u;
        mn = (s47 >> (8 * j)) & 63u;
    } else {
        const int jj = j - 4;
        const uint32_t b8 = (s811 >> (8 * jj)) & 0xffu;
        sc = (b8 & 15u) | (((s03 >> (8 * jj + 6)) & 3u) << 4);
        mn = (b8 >> 4) | (((s47 >> (8 * jj + 6)) & 3u) << 4);
    }
}

// --- more than 16 activation rows: operands staged once per workgroup -----
// A workgroup of eight waves covers 64 weight rows x 64 tokens.  Per block it
// stages in LDS, double-buffered:
//   * the 64 rows' A operands, sc_j * q4 as f16, dequantised once for the
//     whole workgroup: wave w copies the nibbles of AVX2 lanes 4 (w % 2) ..
//     + 3 of rows 16 (w / 2) .. + 15, and those rows' headers, into LDS two
//     blocks ahead and dequantises them itself, lane (row, k) the 16 nibble
//     bytes of AVX2 lane k (16 rows per wave keep its LDS writes on distinct
//     banks);
//   * the four 16-token tiles' B operands, q8 as f16 written by the quantiser
//     in this operand layout, copied global -> LDS one block ahead;
//   * the rows' d, dmin and mins and the tokens' xscale and xsums.
// Every global read is a direct global -> LDS copy, so the waits are exact
// vmcnt counts of this wave's own copies.  Both operand tiles are laid out
// [tile][lane k][group g][row or token c][8 halves], so each MFMA operand
// read of a wave is 1 KB of consecutive LDS.  Wave w owns rows 16 (w % 4) ..
// + 15 and the two token tiles 2 (w / 4), 2 (w / 4) + 1, sharing its A
// operand between them; per lane k and tile it runs q4kDotQ8KRow's two chains
// on the exact MFMA lane sums, in block order:
//   accF = fma(I, d * xscale, accF); accM = fma(dmin, m * xsum, accM).
constexpr int kTlRows = 64, kTlTok = 64;

constexpr int kTlMStride = 80;     // floats per sub-block row of m: writes on distinct banks
struct TlStage {
    uint8_t a16[4 * 8 * 4 * 256];  // [row group][lane k][group g][row c][8 halves]
    uint8_t b16[4 * 8 * 4 * 256];  // [token tile][lane k][group g][token c][8 halves]
    float m[8][kTlMStride];        // [sub-block k][row] 6-bit min
    float xsum[4][8][16];          // [token tile][lane k][token c]
    float d[kTlRows], dmin[kTlRows], xs[kTlTok];
};
struct TlRaw {                     // one block of the 64 rows as stored, per wave
    uint8_t nib[8][64][16];        // [wave][lane: row 16 (w / 2) + lane / 4, lane k 4 (w % 2) + lane % 4]
    uint8_t hdr[8][16][16];        // [wave][row 16 (w / 2) + r]: d, dmin, 12 scale bytes
};

// Direct global -> LDS copies addressed by a wave-uniform base and a 32-bit
// per-lane byte offset (the saddr form), so a copy costs one VGPR.
__device__ __forceinline__ void lds_copy16_s(const void* sbase, uint32_t voff, uint32_t lds_dst) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds_dst)
                 : "memory", "m0");
}
__device__ __forceinline__ void lds_copy4_s(const void* sbase, uint32_t voff, uint32_t lds_dst) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds_dst)
                 : "memory", "m0");
}

// Block b's token operands into S: 32 one-KB pieces of B (four per wave),
// the four tiles' xsums (waves 0, 1) and the 64 xscales (wave 2).  Issues 5
// copies on waves 0-2 and 4 on the others.
__device__ __forceinline__ void tl_copy_tokens(const PfArgs& a, int w, int lane, int tile0, int tok0,
                                               int b, TlStage& S) {
    const int cols = a.blocks * 256;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int ch = 4 * w + i, tt = ch >> 3, piece = ch & 7;
        const int gt = min(tile0 + tt, a.act.tiles - 1);
        const uint8_t* base = (const uint8_t*)a.act.b16t + ((size_t)b * a.act.tiles + gt) * 8192 + piece * 1024;
        lds_copy16_s(base, 16 * lane, lds_addr(S.b16 + tt * 8192 + piece * 1024));
    }
    if (w < 2) {
        const int gt = min(tile0 + 2 * w + (lane >> 5), a.act.tiles - 1);
        lds_copy16_s(a.act.xs32t, (uint32_t)(((size_t)b * a.act.tiles + gt) * 512 + 16 * (lane & 31)),
                     lds_addr(&S.xsum[2 * w][0][0]));
    } else if (w == 2) {
        lds_copy4_s(a.act.xscale + b, (uint32_t)min(tok0 + lane, a.p - 1) * a.blocks * 4,
                    lds_addr(&S.xs[0]));
    }
}

// Block b of this wave's rows into R: lane (row 16 (w / 2) + lane / 4, lane
// k = 4 (w % 2) + lane % 4) copies 16 nibble bytes, lanes 0-15 the rows'
// headers.  Two copies.  noff / hoff: this lane's 32-bit offsets of its
// nibble chunk and header row (the launcher checks that rows * rb < 2^32).
__device__ __forceinline__ void tl_copy_raw(const PfArgs& a, int w, int lane, uint32_t noff,
                                            uint32_t hoff, int b, TlRaw& R) {
    lds_copy16_s(a.w + q4k_nib_off(a.blocks, b), noff, lds_addr(&R.nib[w][0][0]));
    if (lane < 16) lds_copy16_s(a.w + q4k_hdr_off(b), hoff, lds_addr(&R.hdr[w][0][0]));
}

// Dequantisation of this wave's part of one block from R into S, in parts
// that the kernel interleaves with the MFMA chains: A operands sc_j * q4
// (f16), the rows' mins (lane k: sub-block k), d and dmin.
struct TlDq {
    u4v nib;
    uint32_t sc03, sc47;
};

__device__ __forceinline__ void tl_dq_begin(int w, int lane, const TlRaw& R, TlDq& q) {
    q.nib = *(const u4v*)&R.nib[w][lane][0];
    const u4v h = *(const u4v*)&R.hdr[w][lane >> 2][0];
    // getScaleMinK4 (simd.go:1672-1677) for all eight sub-blocks at once, one
    // byte each: j < 4 from s03 / s47, j >= 4 from s811 and their top bits
    q.sc03 = h.y & 0x3f3f3f3fu;
    q.sc47 = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
}

// nibble dword sg: sub-blocks 2 sg (low nibbles) and 2 sg + 1 (high nibbles)
__device__ __forceinline__ void tl_dq_part(int w, int lane, int sg, const TlDq& q, TlStage& S) {
    const int c = lane >> 2, k = 4 * (w & 1) + (lane & 3), rg = w >> 1;
    typedef _Float16 h2v __attribute__((ext_vector_type(2)));
    const h2v m1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    // scale bytes 2 (sg & 1) and 2 (sg & 1) + 1 of sc03 / sc47 as (1024 + sc)
    const uint32_t src = sg < 2 ? q.sc03 : q.sc47;
    const uint32_t sel_lo = (sg & 1) ? 0x04020402u : 0x04000400u;
    const uint32_t sel_hi = (sg & 1) ? 0x04030403u : 0x04010401u;
    const h2v pl = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, src, sel_lo));
    const h2v ph = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, src, sel_hi));
    const h2v sl = pl + m1024, sh = ph + m1024;  // exact small integers
    const h2v nl = sl * m1024, nh = sh * m1024;  // exact: at most 64512
    const h8v av = dequant_a(q.nib[sg], __builtin_bit_cast(uint32_t, sl), __builtin_bit_cast(uint32_t, nl),
                             __builtin_bit_cast(uint32_t, sh), __builtin_bit_cast(uint32_t, nh));
    *(h8v*)(S.a16 + ((rg * 8 + k) * 4 + sg) * 256 + c * 16) = av;
}

// the rows' mins (lane k: sub-block k, same packing as the scales), d, dmin;
// the header is read again from R, which the next copies overwrite only
// after the workgroup barrier
__device__ __forceinline__ void tl_dq_end(int w, int lane, const TlRaw& R, TlStage& S) {
    const int c = lane >> 2, k = 4 * (w & 1) + (lane & 3), lr = 16 * (w >> 1) + c;
    const u4v h = *(const u4v*)&R.hdr[w][c][0];
    const uint32_t msrc = k < 4 ? h.z & 0x3f3f3f3fu : ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
    S.m[k][lr] = (float)((msrc >> (8 * (k & 3))) & 63u);
    if (k == 0) S.d[lr] = f16_bits_to_f32(h.x & 0xffffu);
    if (k == 1) S.dmin[lr] = f16_bits_to_f32(h.x >> 16);
}

__device__ __forceinline__ void tl_dequant(int w, int lane, const TlRaw& R, TlStage& S) {
    TlDq q;
    tl_dq_begin(w, lane, R, q);
#pragma unroll
    for (int sg = 0; sg < 4; sg++) tl_dq_part(w, lane, sg, q, S);
    tl_dq_end(w, lane, R, S);
}

// Workgroup -> tile map.  Workgroup i runs on XCD i % 8 (round robin); the
// eight XCDs form an h x v grid, XCD x taking token-tile group x % h and
// row-tile group x / h, so each XCD reads its share of the weights once and
// its (at most four 64-token tiles' worth of) activations stay in its L2
// while the weight rows stream past.  Within an XCD the token tiles of one
// row tile are consecutive, so they read its weights at about the same time.
struct TlMap {
    int row_tiles, tok_tiles;  // whole problem
    int h, v;                  // XCD grid: h token groups x v row groups
    int tg_size, rg_size;      // token / row tiles per group
};

static TlMap tl_map(int rows, int p) {
    TlMap m;
    m.row_tiles = (rows + kTlRows - 1) / kTlRows;
    m.tok_tiles = (p + kTlTok - 1) / kTlTok;
    m.h = 1;
    while (m.h < 8 && (m.tok_tiles + m.h - 1) / m.h > 4) m.h *= 2;
    m.v = 8 / m.h;
    m.tg_size = (m.tok_tiles + m.h - 1) / m.h;
    m.rg_size = (m.row_tiles + m.v - 1) / m.v;
    return m;
}

__global__ __launch_bounds__(512) void prefill_q4k_tiled_kernel(PfArgs a, TlMap mp) {
    __shared__ __align__(16) TlStage st[2];
    __shared__ __align__(16) TlRaw raw[2];
    const int id = blockIdx.x, xcd = id & 7, local = id >> 3;
    const int lt = local % mp.tg_size, lrow = local / mp.tg_size;
    const int ttile = (xcd % mp.h) * mp.tg_size + lt, rtile = (xcd / mp.h) * mp.rg_size + lrow;
    if (lrow >= mp.rg_size || ttile >= mp.tok_tiles || rtile >= mp.row_tiles) return;  // whole workgroup
    const int row0 = rtile * kTlRows, tok0 = ttile * kTlTok, tile0 = tok0 / 16;
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, c = lane & 15;
    const int rg = w & 3, tg = w >> 2;
    const int nb = a.blocks;
    const uint32_t noff = (uint32_t)min(row0 + 16 * (w >> 1) + (lane >> 2), a.rows - 1) * (uint32_t)a.rb +
                          16 * (4 * (w & 1) + (lane & 3));
    const uint32_t hoff = (uint32_t)min(row0 + 16 * (w >> 1) + (lane & 15), a.rows - 1) * (uint32_t)a.rb;

    float accF[2][8][4], accM[2][8][4];
#pragma unroll
    for (int n = 0; n < 2; n++)
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
            for (int i = 0; i < 4; i++) accF[n][k][i] = accM[n][k][i] = 0.0f;

    // prologue: raw blocks 0 and 1, token operands of block 0
    tl_copy_raw(a, w, lane, noff, hoff, 0, raw[0]);
    tl_copy_raw(a, w, lane, noff, hoff, min(1, nb - 1), raw[1]);
    tl_copy_tokens(a, w, lane, tile0, tok0, 0, st[0]);
    wait_vmem_le<0>();
    tl_dequant(w, lane, raw[0], st[0]);
    wait_lgkm0();
    lds_barrier();
#pragma unroll 1
    for (int b = 0; b < nb; b++) {
        // copies stay unconditional (clamped to the last block; the buffers
        // they fill are not read this iteration) so the vmcnt counts below
        // are constants: tokens of b + 1 (5 / 4 copies), raw of b + 2 (2)
        tl_copy_tokens(a, w, lane, tile0, tok0, min(b + 1, nb - 1), st[(b + 1) & 1]);
        tl_copy_raw(a, w, lane, noff, hoff, min(b + 2, nb - 1), raw[b & 1]);
        const TlStage& S = st[b & 1];
        const f4v dv = *(const f4v*)&S.d[16 * rg + 4 * g];
        const f4v dm = *(const f4v*)&S.dmin[16 * rg + 4 * g];
        float dxs[2][4];
#pragma unroll
        for (int n = 0; n < 2; n++) {
            const float xc = S.xs[32 * tg + 16 * n + c];
#pragma unroll
            for (int i = 0; i < 4; i++) dxs[n][i] = dv[i] * xc;
        }
        // raw block b + 1 (copied last iteration) has landed once at most this
        // iteration's copies are outstanding; its dequantisation into the
        // other stage runs in parts between the chain steps below
        if (w < 3) wait_vmem_le<7>();
        else wait_vmem_le<6>();
        asm volatile("" ::: "memory");
        TlDq dq;
        tl_dq_begin(w, lane, raw[(b + 1) & 1], dq);
        // Software pipeline over the lanes k: step k reads lane k + 2's
        // operands, issues lane k + 1's MFMAs and runs lane k's chains on the
        // products issued one step earlier, so neither the LDS latency nor the
        // MFMA latency sits in front of the chains.  The empty asm statements
        // pin that order (lane k's accumulators final and lane k + 2's
        // operands arrived when step k ends); without them the compiler
        // hoists more lanes' operands than two waves per SIMD have registers for.
        struct Ops {
            h8v av, bv[2];
            f4v mk;
            float xk[2];
        };
        auto ops = [&](int k, Ops& o) __attribute__((always_inline)) {
            o.av = *(const h8v*)(S.a16 + ((rg * 8 + k) * 4 + g) * 256 + c * 16);
            o.mk = *(const f4v*)&S.m[k][16 * rg + 4 * g];
#pragma unroll
            for (int n = 0; n < 2; n++) {
                o.bv[n] = *(const h8v*)(S.b16 + (((2 * tg + n) * 8 + k) * 4 + g) * 256 + c * 16);
                o.xk[n] = S.xsum[2 * tg + n][k][c];
            }
        };
        const f4v z = {0.0f, 0.0f, 0.0f, 0.0f};
        Ops o[3];
        f4v dI[2][2];  // [lane k parity][token tile]
        ops(0, o[0]);
        ops(1, o[1]);
        asm volatile("" : "+v"(o[0].av), "+v"(o[0].bv[0]), "+v"(o[0].bv[1]));
#pragma unroll
        for (int n = 0; n < 2; n++) dI[0][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(o[0].av, o[0].bv[n], z, 0, 0, 0);
        asm volatile("" : "+v"(o[1].av), "+v"(o[1].bv[0]), "+v"(o[1].bv[1]), "+v"(o[1].mk), "+v"(o[1].xk[0]),
                     "+v"(o[1].xk[1]));
#pragma unroll
        for (int k = 0; k < 8; k++) {
            if (k < 6) ops(k + 2, o[(k + 2) % 3]);
            if (k < 7) {
                const Ops& nx = o[(k + 1) % 3];
#pragma unroll
                for (int n = 0; n < 2; n++)
                    dI[(k + 1) & 1][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(nx.av, nx.bv[n], z, 0, 0, 0);
            }
            const Ops& cur = o[k % 3];
#pragma unroll
            for (int n = 0; n < 2; n++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    accF[n][k][i] = fmaf(dI[k & 1][n][i], dxs[n][i], accF[n][k][i]);
                    const float mx = cur.mk[i] * cur.xk[n];
                    accM[n][k][i] = fmaf(dm[i], mx, accM[n][k][i]);
                }
            }
            if (k & 1) tl_dq_part(w, lane, k >> 1, dq, st[(b + 1) & 1]);
#pragma unroll
            for (int n = 0; n < 2; n++)
                asm volatile("" : "+v"(accF[n][k][0]), "+v"(accF[n][k][1]), "+v"(accF[n][k][2]),
                             "+v"(accF[n][k][3]), "+v"(accM[n][k][0]), "+v"(accM[n][k][1]),
                             "+v"(accM[n][k][2]), "+v"(accM[n][k][3]));
            if (k < 6) {
                Ops& nx = o[(k + 2) % 3];
                asm volatile("" : "+v"(nx.av), "+v"(nx.bv[0]), "+v"(nx.bv[1]), "+v"(nx.mk),
                             "+v"(nx.xk[0]), "+v"(nx.xk[1]));
            }
        }
        tl_dq_end(w, lane, raw[(b + 1) & 1], st[(b + 1) & 1]);
        wait_vmem_le<2>();  // token operands of b + 1
        wait_lgkm0();
        lds_barrier();
    }
    wait_vmem_le<0>();  // the clamped copies of the last iterations
    // tree8 of the reference's horizontal sum, then the (row, token) stores
#pragma unroll
    for (int n = 0; n < 2; n++) {
        const int t = tok0 + 32 * tg + 16 * n + c;
        if (t >= a.p) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int rr = row0 + 16 * rg + 4 * g + i;
            if (rr >= a.rows) continue;
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = accF[n][k][i] - accM[n][k][i];
            const float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
            a.out[(size_t)t * a.out_stride + rr] = (s0 + s1) + (s2 + s3);
        }
    }
}

// --- Q6_K, more than 16 activation rows: 64 x 64 staged tiles --------------
// q6kDotQ8KRow (kernels_amd64.s Q6KQ8QUAD, the batch-1 row kernel
// gemv_q6k_kernel) per AVX2 lane k of a 256-element block b:
//   I       = sum over the lane's 32 elements of sc(e) * code(e) * q8(e)
//             (int32; code = ql | qh << 4 in 0..63, sc the element's int8 scale)
//   o2      = fma(sc_{8+k}, 32 xs16_{8+k}, sc_k * 32 xs16_k)
//   accM[k] = fma(d_b, o2, accM[k]);  accF[k] = fma(float(I), d_b * xscale_b, accF[k])
// and tree8(accF - accM).  sc * code reaches 128 * 63, past the integers
// f16 holds exactly, so the products split at the code's two fields:
//   I = 16 * (sum sc * (code >> 4) * q8) + sum sc * (code & 15) * q8
// with |sc * (code >> 4)| <= 384 and |sc * (code & 15)| <= 1920 exact in f16
// and every partial sum of 32 products an integer below 2^24, so each of
// the two v_mfma_f32_16x16x32_f16 results is its exact integer sum and
// fma(hi, 16, lo) rounds 16 hi + lo once: float(I).  The chains then run in
// VALU registers in the reference's order.
// Workgroup: 64 rows x 64 tokens, eight waves; wave w owns rows 16 (w & 3)
// .. + 15 and the token tiles 2 (w >> 2), 2 (w >> 2) + 1.  Per block,
// double-buffered in LDS and copied global -> LDS one block ahead: the 64
// rows' block bytes as stored (ql, qh, scales; the A operands are built
// from them by the wave that uses them, lane (g, c) the 8 codes of row c,
// lane k, kappa 8 g .. + 7), the four 16-token B tiles (the quantiser's f16
// layout) and the tokens' xs16 and xscale; the rows' scales and d as floats
// are prepared once per block.  Weights need rows * rb < 4 GiB and
// 16-byte aligned blocks (blocks % 8 == 0).
constexpr int kQ6Rows = 64, kQ6Tok = 64;
constexpr int kQ6RawPieces = 64 * 13;  // 64 rows x 13 pieces of 16 bytes (208-byte blocks)
struct Q6Stage {
    uint8_t q[kQ6RawPieces * 16];  // [row][208]: ql 128, qh 64, scales 16
    uint32_t dw[64];               // [row]: the dword holding d of blocks b & ~1, b | 1
    uint8_t b16[4 * 8 * 4 * 256];  // [token tile][lane k][group g][token c][8 halves]
    float x16[kQ6Tok][16];         // [token][16-group] xs16
    float xs[kQ6Tok];
    float sc[16][kQ6Rows];         // [scale index][row] int8 scale
    float d[kQ6Rows];
};

// Block b's operands into S: the 832 raw pieces (two 1 KB copies on waves
// 0-5, one on wave 6), the rows' d dwords (wave 7), four 1 KB pieces of B
// per wave, the tokens' xs16 (waves 0-3) and xscales (wave 4).
__device__ __forceinline__ void q6_copy(const PfArgs& a, int w, int lane, int row0, int tile0, int tok0,
                                        int b, Q6Stage& S) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
        // pieces 128 w + 64 i + lane of 832: waves 0-5 two each, wave 6 one
        const int pc = 128 * w + 64 * i + lane;
        if (pc < kQ6RawPieces) {  // wave-uniform: 832 = 6.5 x 128
            const int r = pc / 13, off = (pc % 13) * 16;
            const size_t row = (size_t)min(row0 + r, a.rows - 1);
            lds_copy16_s(a.w, (uint32_t)(row * a.rb + (size_t)b * 208 + off), lds_addr(S.q + 16 * (pc - lane)));
        }
    }
    if (w == 7) {
        const size_t row = (size_t)min(row0 + lane, a.rows - 1);
        lds_copy4_s(a.w, (uint32_t)(row * a.rb + (size_t)a.blocks * 208 + (size_t)(b & ~1) * 2),
                    lds_addr(&S.dw[0]));
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int ch = 4 * w + i, tt = ch >> 3, piece = ch & 7;
        const int gt = min(tile0 + tt, a.act.tiles - 1);
        const uint8_t* base = (const uint8_t*)a.act.b16t + ((size_t)b * a.act.tiles + gt) * 8192 + piece * 1024;
        lds_copy16_s(base, 16 * lane, lds_addr(S.b16 + tt * 8192 + piece * 1024));
    }
    if (w < 4) {
        const int t = min(tok0 + 16 * w + (lane >> 2), a.p - 1);
        lds_copy16_s(a.act.xs16, (uint32_t)(((size_t)t * (a.blocks * 16) + (size_t)b * 16) * 4 + 16 * (lane & 3)),
                     lds_addr(&S.x16[16 * w][0]));
    } else if (w == 4) {
        lds_copy4_s(a.act.xscale + b, (uint32_t)min(tok0 + lane, a.p - 1) * a.blocks * 4, lds_addr(&S.xs[0]));
    }
}

// The rows' scales and d of block b as floats: thread t scale index t >> 5
// of rows t & 31 and 32 + (t & 31); threads 0-63 d of row t.
__device__ __forceinline__ void q6_prep(int tid, int b, Q6Stage& S) {
    const int idx = tid >> 5, r = tid & 31;
    S.sc[idx][r] = (float)(int8_t)S.q[r * 208 + 192 + idx];
    S.sc[idx][32 + r] = (float)(int8_t)S.q[(32 + r) * 208 + 192 + idx];
    if (tid < 64) S.d[tid] = f16_bits_to_f32((S.dw[tid] >> (16 * (b & 1))) & 0xffffu);
}

// four bytes (values 0..255, exact) -> two half2 words
__device__ __forceinline__ void u8x4_to_h(uint32_t v, uint32_t& lo, uint32_t& hi) {
    typedef _Float16 h2v __attribute__((ext_vector_type(2)));
    const h2v bias = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    const h2v a = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, v, 0x05010400u)) + bias;
    const h2v c = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, v, 0x05030402u)) + bias;
    lo = __builtin_bit_cast(uint32_t, a);
    hi = __builtin_bit_cast(uint32_t, c);
}

// A operands (low and high code fields) of lane (g, c) for lane k from its
// row's raw bytes: quads m = 2g, 2g + 1 of lane k (ql dwords 2h, 2h + 1 and
// qh dword h of the lane, h = g >> 1, nibble / bit-pair shift 4 (g & 1))
// with scales 8h + 4 (g & 1) + (k >> 2) and + 2.
struct Q6Raw8 {
    uint2 ql;
    uint32_t qh, sc;
};
__device__ __forceinline__ void q6_raw(const uint8_t* row, int k, int g, Q6Raw8& o) {
    const int h = g >> 1;
    o.ql = *(const uint2*)(row + 16 * k + 8 * h);
    o.qh = *(const uint32_t*)(row + 128 + 8 * k + 4 * h);
    o.sc = *(const uint32_t*)(row + 192 + 8 * h + 4 * (g & 1));
}
__device__ __forceinline__ void q6_operands(const Q6Raw8& o, int k, int g, h8v& lo, h8v& hi) {
    typedef _Float16 h2v __attribute__((ext_vector_type(2)));
    const int sh = 4 * (g & 1), hk = k >> 2;
    // scale bytes hk and hk + 2 of o.sc, as exact f16 (byte ^ 0x80 = s + 128)
    const uint32_t sv = o.sc ^ 0x80808080u;
    const h2v m1152 = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const h2v f0 = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, sv, hk ? 0x04010401u : 0x04000400u)) + m1152;
    const h2v f1 = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, sv, hk ? 0x04030403u : 0x04020402u)) + m1152;
    uint32_t l0, l1, l2, l3, h0, h1, h2, h3;
    u8x4_to_h((o.ql.x >> sh) & 0x0f0f0f0fu, l0, l1);
    u8x4_to_h((o.ql.y >> sh) & 0x0f0f0f0fu, l2, l3);
    u8x4_to_h((o.qh >> sh) & 0x03030303u, h0, h1);
    u8x4_to_h((o.qh >> (sh + 2)) & 0x03030303u, h2, h3);
    // exact: products of small integers below 2048
    const h2v a0 = __builtin_bit_cast(h2v, l0) * f0, a1 = __builtin_bit_cast(h2v, l1) * f0;
    const h2v a2 = __builtin_bit_cast(h2v, l2) * f1, a3 = __builtin_bit_cast(h2v, l3) * f1;
    const h2v b0 = __builtin_bit_cast(h2v, h0) * f0, b1 = __builtin_bit_cast(h2v, h1) * f0;
    const h2v b2 = __builtin_bit_cast(h2v, h2) * f1, b3 = __builtin_bit_cast(h2v, h3) * f1;
    lo[0] = a0[0]; lo[1] = a0[1]; lo[2] = a1[0]; lo[3] = a1[1];
    lo[4] = a2[0]; lo[5] = a2[1]; lo[6] = a3[0]; lo[7] = a3[1];
    hi[0] = b0[0]; hi[1] = b0[1]; hi[2] = b1[0]; hi[3] = b1[1];
    hi[4] = b2[0]; hi[5] = b2[1]; hi[6] = b3[0]; hi[7] = b3[1];
}

__global__ __launch_bounds__(512) void prefill_q6k_tiled_kernel(PfArgs a, TlMap mp) {
    __shared__ __align__(16) Q6Stage st[2];
    const int id = blockIdx.x, xcd = id & 7, local = id >> 3;
    const int lt = local % mp.tg_size, lrow = local / mp.tg_size;
    const int ttile = (xcd % mp.h) * mp.tg_size + lt, rtile = (xcd / mp.h) * mp.rg_size + lrow;
    if (lrow >= mp.rg_size || ttile >= mp.tok_tiles || rtile >= mp.row_tiles) return;  // whole workgroup
    const int row0 = rtile * kQ6Rows, tok0 = ttile * kQ6Tok, tile0 = tok0 / 16;
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, c = lane & 15;
    const int rg = w & 3, tg = w >> 2;
    const int nb = a.blocks;

    float accF[2][8][4], accM[2][8][4];
#pragma unroll
    for (int n = 0; n < 2; n++)
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
            for (int i = 0; i < 4; i++) accF[n][k][i] = accM[n][k][i] = 0.0f;

    q6_copy(a, w, lane, row0, tile0, tok0, 0, st[0]);
    wait_vmem_le<0>();
    lds_barrier();
    q6_prep(tid, 0, st[0]);
    wait_lgkm0();
    lds_barrier();
#pragma unroll 1
    for (int b = 0; b < nb; b++) {
        // unconditional copies of block b + 1 (clamped to the last block)
        // into the stage not read this iteration
        q6_copy(a, w, lane, row0, tile0, tok0, min(b + 1, nb - 1), st[(b + 1) & 1]);
        const Q6Stage& S = st[b & 1];
        // per-lane LDS offsets, rebuilt every block behind an empty asm so
        // the compiler keeps one register per operand stream instead of
        // hoisting an address per (lane k, tile) out of the loop
        const int h = g >> 1;
        uint32_t o_ql = (16 * rg + c) * 208 + 8 * h, o_qh = (16 * rg + c) * 208 + 128 + 4 * h;
        uint32_t o_sc = (16 * rg + c) * 208 + 192 + 8 * h + 4 * (g & 1);
        uint32_t o_b = (2 * tg * 8 * 4 + g) * 256 + c * 16, o_x = (32 * tg + c) * 64;
        uint32_t o_k = (16 * rg + 4 * g) * 4;
        asm volatile("" : "+v"(o_ql), "+v"(o_qh), "+v"(o_sc), "+v"(o_b), "+v"(o_x), "+v"(o_k));
        const uint8_t* q = S.q;
        const uint8_t* bt = S.b16;
        const uint8_t* xt = (const uint8_t*)&S.x16[0][0];
        const uint8_t* sct = (const uint8_t*)&S.sc[0][0];
        float dv[4], dxs[2][4];
#pragma unroll
        for (int i = 0; i < 4; i++) dv[i] = S.d[16 * rg + 4 * g + i];
#pragma unroll
        for (int n = 0; n < 2; n++) {
            const float xv = S.xs[32 * tg + 16 * n + c];
#pragma unroll
            for (int i = 0; i < 4; i++) dxs[n][i] = dv[i] * xv;  // VMULSS d * xscale
        }
        const f4v z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < 8; k++) {
            Q6Raw8 raw;
            raw.ql = *(const uint2*)(q + o_ql + 16 * k);
            raw.qh = *(const uint32_t*)(q + o_qh + 8 * k);
            raw.sc = *(const uint32_t*)(q + o_sc);
            h8v bv[2];
            float x0[2], x8[2];
#pragma unroll
            for (int n = 0; n < 2; n++) {
                bv[n] = *(const h8v*)(bt + o_b + n * 8192 + k * 1024);
                x0[n] = *(const float*)(xt + o_x + n * 1024 + 4 * k) * 32.0f;  // ScaleF32(xs, 32)
                x8[n] = *(const float*)(xt + o_x + n * 1024 + 4 * (8 + k)) * 32.0f;
            }
            const f4v sk = *(const f4v*)(sct + o_k + k * 256);
            const f4v sk8 = *(const f4v*)(sct + o_k + (8 + k) * 256);
            h8v alo, ahi;
            q6_operands(raw, k, g, alo, ahi);
#pragma unroll
            for (int n = 0; n < 2; n++) {
                const f4v plo = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bv[n], z, 0, 0, 0);
                const f4v phi = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bv[n], z, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float iv = fmaf(phi[i], 16.0f, plo[i]);  // float(I)
                    float o2 = sk[i] * x0[n];                      // VMULPS
                    o2 = fmaf(sk8[i], x8[n], o2);                  // VFMADD231PS
                    accM[n][k][i] = fmaf(dv[i], o2, accM[n][k][i]);
                    accF[n][k][i] = fmaf(iv, dxs[n][i], accF[n][k][i]);
                }
            }
            // lane k's accumulators final here: without the pin the compiler
            // interleaves the eight lanes' chains past the register file
#pragma unroll
            for (int n = 0; n < 2; n++)
                asm volatile("" : "+v"(accF[n][k][0]), "+v"(accF[n][k][1]), "+v"(accF[n][k][2]),
                             "+v"(accF[n][k][3]), "+v"(accM[n][k][0]), "+v"(accM[n][k][1]),
                             "+v"(accM[n][k][2]), "+v"(accM[n][k][3]));
            __builtin_amdgcn_sched_barrier(0);
        }
        wait_vmem_le<0>();  // block b + 1's copies, issued before this block's products
        lds_barrier();
        q6_prep(tid, min(b + 1, nb - 1), st[(b + 1) & 1]);
        wait_lgkm0();
        lds_barrier();
    }
#pragma unroll
    for (int n = 0; n < 2; n++) {
        const int t = tok0 + 32 * tg + 16 * n + c;
        if (t >= a.p) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int rr = row0 + 16 * rg + 4 * g + i;
            if (rr >= a.rows) continue;
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = accF[n][k][i] - accM[n][k][i];
            const float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
            a.out[(size_t)t * a.out_stride + rr] = (s0 + s1) + (s2 + s3);
        }
    }
}

int launch_q6k_tiled(const uint8_t* d_w, size_t rb, int rows, int blocks, const ActQ8& act, int p,
                     float* out, int out_stride, hipStream_t s) {
    if (rows <= 0 || blocks <= 0 || p <= 0) return GLLM_OK;
    if (!act.b16t || p <= kTiledMinP || blocks % 8 || (size_t)rows * rb >= ((size_t)1 << 32))
        return fail(GLLM_EINVAL, "prefill: Q6_K tiles need > %d tokens, blocks %% 8 == 0, < 4 GiB",
                    kTiledMinP);
    PfArgs a{d_w, rb, rows, blocks, act, p, out, out_stride};
    const TlMap mp = tl_map(rows, p);
    hipLaunchKernelGGL(prefill_q6k_tiled_kernel, dim3(8 * mp.tg_size * mp.rg_size), dim3(512), 0, s, a,
                       mp);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

// --- Q8_0, more than 16 activation rows: 64 x 64 staged tiles ---------------
// q8_0DotQ8KRow (kernels_amd64.s Q80CHUNK) per AVX2 lane k of a 256-element
// group: for its eight 32-value blocks q in order
//   acc12 = fma(d_q, float(I_qk), acc12)   I_qk: the exact dot of the lane's
//                                           4 weight and 4 activation bytes
// then acc11[k] = fma(xscale, acc12, acc11[k]) and tree8(acc11).  The
// per-block float chain sets the cost (25 VALU operations per row, token,
// group and lane with v_dot4_i32_i8 for I), so this kernel stays on the
// vector units and reads every weight byte once per 64 tokens.
// Workgroup: 64 rows x 64 tokens, 512 threads; thread (rp, tq) = (t >> 4,
// t & 15) owns rows 2 rp, 2 rp + 1 and tokens tq + 16 j (j < 4).  Per group,
// double-buffered in LDS: the 64 rows' 272-byte groups as stored (8 f16 d,
// then lane k's 8 dwords at 16 + 32 k) and the 64 tokens' q8perm bytes
// (lane k's 32 at 32 k) in 272-byte rows, both copied global -> LDS one
// group ahead, and the tokens' xscales.
constexpr int kQ80Pieces = 64 * 17;  // 16-byte pieces of 64 rows (or tokens) x 272 bytes
struct Q80Stage {
    uint8_t w[kQ80Pieces * 16];  // [row][272]
    uint8_t q[kQ80Pieces * 16];  // [token][272]: 256 q8perm bytes, 16 unused
    float xs[64];
};

// Group b's operands into S: two 1 KB pieces of the rows and two of the
// tokens per wave, the remaining 64 row pieces on wave 0, 64 token pieces on
// wave 1, the xscales on wave 2: five copies on waves 0-2, four on 3-7.
__device__ __forceinline__ void q80_copy(const PfArgs& a, int w, int lane, int row0, int tok0, int b,
                                         Q80Stage& S) {
    const int cols = a.blocks * 256;
#pragma unroll
    for (int i = 0; i < 3; i++) {
        if (i == 2 && w != 0) break;  // wave-uniform
        const int pc = (i < 2 ? 128 * w + 64 * i : 1024) + lane, r = pc / 17, off = (pc % 17) * 16;
        const size_t row = (size_t)min(row0 + r, a.rows - 1);
        lds_copy16_s(a.w, (uint32_t)(row * a.rb + (size_t)b * 272 + off), lds_addr(S.w + 16 * (pc - lane)));
    }
#pragma unroll
    for (int i = 0; i < 3; i++) {
        if (i == 2 && w != 1) break;  // wave-uniform
        const int pc = (i < 2 ? 128 * w + 64 * i : 1024) + lane, t = pc / 17, off = min((pc % 17) * 16, 240);
        const size_t tok = (size_t)min(tok0 + t, a.p - 1);
        lds_copy16_s(a.act.q8perm, (uint32_t)(tok * cols + (size_t)b * 256 + off), lds_addr(S.q + 16 * (pc - lane)));
    }
    if (w == 2)
        lds_copy4_s(a.act.xscale + b, (uint32_t)min(tok0 + lane, a.p - 1) * a.blocks * 4, lds_addr(&S.xs[0]));
}

__global__ __launch_bounds__(512) void prefill_q8_0_tiled_kernel(PfArgs a, TlMap mp) {
    __shared__ __align__(16) Q80Stage st[2];
    const int id = blockIdx.x, xcd = id & 7, local = id >> 3;
    const int lt = local % mp.tg_size, lrow = local / mp.tg_size;
    const int ttile = (xcd % mp.h) * mp.tg_size + lt, rtile = (xcd / mp.h) * mp.rg_size + lrow;
    if (lrow >= mp.rg_size || ttile >= mp.tok_tiles || rtile >= mp.row_tiles) return;  // whole workgroup
    const int row0 = rtile * kTlRows, tok0 = ttile * kTlTok;
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rp = tid >> 4, tq = tid & 15;
    const int nb = a.blocks;

    float acc11[2][4][8];
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int k = 0; k < 8; k++) acc11[r][j][k] = 0.0f;

    q80_copy(a, w, lane, row0, tok0, 0, st[0]);
    wait_vmem_le<0>();
    lds_barrier();
#pragma unroll 1
    for (int b = 0; b < nb; b++) {
        // unconditional copies (clamped to the last group, into the stage
        // not read this iteration): five on waves 0-2, four on 3-7
        q80_copy(a, w, lane, row0, tok0, min(b + 1, nb - 1), st[(b + 1) & 1]);
        const Q80Stage& S = st[b & 1];
        float d[2][8], xs[4];
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const uint4 dh = *(const uint4*)(S.w + (2 * rp + r) * 272);
            const uint32_t dw[4] = {dh.x, dh.y, dh.z, dh.w};
#pragma unroll
            for (int q = 0; q < 8; q++) d[r][q] = f16_bits_to_f32((dw[q >> 1] >> (16 * (q & 1))) & 0xffffu);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) xs[j] = S.xs[tq + 16 * j];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            int wv[2][8], qv[4][8];
#pragma unroll
            for (int r = 0; r < 2; r++) {
                const int4 lo = *(const int4*)(S.w + (2 * rp + r) * 272 + 16 + 32 * k);
                const int4 hi = *(const int4*)(S.w + (2 * rp + r) * 272 + 32 + 32 * k);
                wv[r][0] = lo.x; wv[r][1] = lo.y; wv[r][2] = lo.z; wv[r][3] = lo.w;
                wv[r][4] = hi.x; wv[r][5] = hi.y; wv[r][6] = hi.z; wv[r][7] = hi.w;
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int4 lo = *(const int4*)(S.q + (tq + 16 * j) * 272 + 32 * k);
                const int4 hi = *(const int4*)(S.q + (tq + 16 * j) * 272 + 32 * k + 16);
                qv[j][0] = lo.x; qv[j][1] = lo.y; qv[j][2] = lo.z; qv[j][3] = lo.w;
                qv[j][4] = hi.x; qv[j][5] = hi.y; qv[j][6] = hi.z; qv[j][7] = hi.w;
            }
#pragma unroll
            for (int r = 0; r < 2; r++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    float acc12 = 0.0f;
#pragma unroll
                    for (int q = 0; q < 8; q++)
                        acc12 = fmaf((float)sdot4(wv[r][q], qv[j][q], 0), d[r][q], acc12);  // VFMADD231PS
                    acc11[r][j][k] = fmaf(acc12, xs[j], acc11[r][j][k]);
                }
            __builtin_amdgcn_sched_barrier(0);
        }
        wait_vmem_le<0>();  // group b + 1's copies, issued before this group's products
        lds_barrier();
    }
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int rr = row0 + 2 * rp + r;
        if (rr >= a.rows) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int t = tok0 + tq + 16 * j;
            if (t >= a.p) continue;
            const float* v = acc11[r][j];
            const float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
            a.out[(size_t)t * a.out_stride + rr] = (s0 + s1) + (s2 + s3);
        }
    }
}

int launch_q8_0_tiled(const uint8_t* d_w, size_t rb, int rows, int blocks, const ActQ8& act, int p,
                      float* out, int out_stride, hipStream_t s) {
    if (rows <= 0 || blocks <= 0 || p <= 0) return GLLM_OK;
    if (p <= kTiledMinP || (size_t)rows * rb >= ((size_t)1 << 32) || (size_t)p * blocks * 256 >= ((size_t)1 << 32))
        return fail(GLLM_EINVAL, "prefill: Q8_0 tiles need > %d tokens and < 4 GiB operands", kTiledMinP);
    PfArgs a{d_w, rb, rows, blocks, act, p, out, out_stride};
    const TlMap mp = tl_map(rows, p);
    hipLaunchKernelGGL(prefill_q8_0_tiled_kernel, dim3(8 * mp.tg_size * mp.rg_size), dim3(512), 0, s,
                       a, mp);
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

// --- at most 16 activation rows, operands through a per-wave LDS ring -----
// One workgroup per 16 weight rows; wave w computes the MFMA products of
// blocks b = w, w + NW, ... (16-row x 16-token tiles, one per AVX2 lane k),
// the waves exchange the exact products through LDS per group of blocks and
// run the float chains in block order (only the integer products are
// block-parallel, so the bits are the row kernel's).  Each wave copies its
// own operands global -> LDS, DEPTH blocks ahead, in layouts that make every
// MFMA operand read of a wave conflict-free:
//   nib [lane k][row c][16 bytes]   (lane (g, c) reads dword g: consecutive)
//   q8  [lane k][token t][32 bytes] (lane (g, c) reads 8 bytes at 8 g)
// The copies are inline-asm global_load_lds, so their vmcnt waits are
// explicit counts: NC copies per block, DEPTH blocks in flight.
template <int PT>  // tokens staged per block (8 or 16)
struct SsSlot {
    uint8_t nib[8][16][16];
    uint8_t hdr[16][16];
    uint8_t q8[8][PT][32];
    float xs32[PT][8];
    float xs[64];  // [token]; copy lanes past the tokens land in the tail
};
template <int PT>
constexpr int ss_copies() { return 2 + 1 + PT / 4 + PT / 8 + 1; }

template <int PT>
__device__ __forceinline__ void ss_copy(const PfArgs& a, int b, uint32_t slot, int lane) {
    typedef SsSlot<PT> S;
    b = min(b, a.blocks - 1);  // past the end: the last block again (never read)
    const int cols = a.blocks * 256;
    const int row0 = blockIdx.x * 16;
#pragma unroll
    for (int i = 0; i < 2; i++) {  // piece 64 i + lane = (k, c)
        const int idx = 64 * i + lane, k = idx >> 4, c = idx & 15;
        const size_t r = (size_t)min(row0 + c, a.rows - 1);
        lds_copy16_s(a.w, (uint32_t)(r * a.rb + q4k_nib_off(a.blocks, b) + 16 * k),
                     slot + offsetof(S, nib) + 1024 * i);
    }
    {
        const size_t r = (size_t)min(row0 + (lane >> 2), a.rows - 1);
        lds_copy4_s(a.w, (uint32_t)(r * a.rb + q4k_hdr_off(b) + 4 * (lane & 3)), slot + offsetof(S, hdr));
    }
#pragma unroll
    for (int i = 0; i < PT / 4; i++) {  // piece 64 i + lane = ((k, t), half)
        const int idx = 64 * i + lane, h = idx & 1, t = (idx >> 1) % PT, k = (idx >> 1) / PT;
        const size_t tok = (size_t)min(t, a.p - 1);
        lds_copy16_s(a.act.q8perm, (uint32_t)(tok * cols + (size_t)b * 256 + 32 * k + 16 * h),
                     slot + offsetof(S, q8) + 1024 * i);
    }
#pragma unroll
    for (int i = 0; i < PT / 8; i++) {  // dword 64 i + lane = (t, k)
        const int idx = 64 * i + lane;
        const size_t t = (size_t)min(idx >> 3, a.p - 1);
        lds_copy4_s(a.act.xs32, (uint32_t)((t * (cols / 32) + (size_t)b * 8 + (idx & 7)) * 4),
                    slot + offsetof(S, xs32) + 256 * i);
    }
    {
        const size_t t = (size_t)min(lane, a.p - 1);
        lds_copy4_s(a.act.xscale, (uint32_t)((t * a.blocks + b) * 4), slot + offsetof(S, xs));
    }
}

template <int NW, int DEPTH, int PT>
constexpr size_t ss_lds_bytes() {
    return sizeof(f4v) * NW * 8 * 64 + sizeof(SbParams) * NW + sizeof(SsSlot<PT>) * NW * DEPTH;
}

template <int NW, int DEPTH, int PT>
__global__ __launch_bounds__(64 * NW) void prefill_q4k_b16s_kernel(PfArgs a) {
    constexpr int KK = 8 / NW;
    constexpr int NC = ss_copies<PT>();
    typedef SsSlot<PT> S;
    extern __shared__ __attribute__((aligned(16))) uint8_t dyn[];
    f4v (*sdI)[8][64] = (f4v (*)[8][64])dyn;                         // [wave][lane k][MFMA lane]
    SbParams* sp = (SbParams*)(dyn + sizeof(f4v) * NW * 8 * 64);      // [wave]
    uint8_t* ring = dyn + sizeof(f4v) * NW * 8 * 64 + sizeof(SbParams) * NW;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, c = lane & 15;
    const int row0 = blockIdx.x * 16;
    const int tc = min(c, a.p - 1);  // B token of this lane
    const int nb = a.blocks;
    const uint32_t ring_w = lds_addr(ring + sizeof(S) * DEPTH * w);
    float accF[KK][4], accM[KK][4];
#pragma unroll
    for (int kk = 0; kk < KK; kk++)
#pragma unroll
        for (int i = 0; i < 4; i++) accF[kk][i] = accM[kk][i] = 0.0f;
#pragma unroll
    for (int d = 0; d < DEPTH; d++) ss_copy<PT>(a, w + NW * d, ring_w + sizeof(S) * d, lane);
    int slot = 0;
#pragma unroll 1
    for (int q0 = 0; q0 < nb; q0 += NW) {
        // this wave's block q0 + w is in `slot` once the later copies alone
        // are outstanding
        wait_vmem_le<(DEPTH - 1) * NC>();
        const S& sl = *(const S*)(ring + sizeof(S) * (DEPTH * w + slot));
        {
            const u4v hdr = *(const u4v*)&sl.hdr[c][0];
            uint32_t sc_lo, sc_hi, mn;
            sb_scale_min(hdr, 2 * g, sc_lo, mn);
            sb_scale_min(hdr, 2 * g + 1, sc_hi, mn);
            const _Float16 hl = (_Float16)(float)sc_lo, nl = (_Float16)(-1024.0f * (float)sc_lo);
            const _Float16 hh = (_Float16)(float)sc_hi, nh = (_Float16)(-1024.0f * (float)sc_hi);
            const uint32_t bl = __builtin_bit_cast(uint16_t, hl), bnl = __builtin_bit_cast(uint16_t, nl);
            const uint32_t bh = __builtin_bit_cast(uint16_t, hh), bnh = __builtin_bit_cast(uint16_t, nh);
            const uint32_t sh_lo = bl | (bl << 16), sn_lo = bnl | (bnl << 16);
            const uint32_t sh_hi = bh | (bh << 16), sn_hi = bnh | (bnh << 16);
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t wd = *(const uint32_t*)&sl.nib[k][c][4 * g];
                const uint2 q8 = *(const uint2*)&sl.q8[k][tc][8 * g];
                const h8v av = dequant_a(wd, sh_lo, sn_lo, sh_hi, sn_hi);
                uint32_t v[4];
                i8x4_to_h(q8.x, v[0], v[1]);
                i8x4_to_h(q8.y, v[2], v[3]);
                const h8v bv = __builtin_bit_cast(h8v, u4v{v[0], v[1], v[2], v[3]});
                const f4v z = {0.0f, 0.0f, 0.0f, 0.0f};
                sdI[w][k][lane] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, z, 0, 0, 0);
            }
            if (g == 0) {
                sp[w].d[c] = f16_bits_to_f32(hdr.x & 0xffffu);
                sp[w].dmin[c] = f16_bits_to_f32(hdr.x >> 16);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    uint32_t scj, mnj;
                    sb_scale_min(hdr, j, scj, mnj);
                    sp[w].m[j][c] = (float)mnj;
                }
            } else if (g == 1) {
                sp[w].xs[c] = sl.xs[tc];
#pragma unroll
                for (int k = 0; k < 8; k++) sp[w].xsum[k][c] = sl.xs32[tc][k];
            }
        }
        // the slot's reads are done: refill it DEPTH groups ahead
        wait_lgkm0();
        ss_copy<PT>(a, q0 + w + NW * DEPTH, ring_w + sizeof(S) * slot, lane);
        slot = slot + 1 == DEPTH ? 0 : slot + 1;
        lds_barrier();
        // the group's blocks in order: chains of lanes k = KK w .. for rows
        // 4g + i and token c (the MFMA D layout of this lane)
#pragma unroll
        for (int u = 0; u < NW; u++) {
            if (q0 + u >= nb) break;  // uniform
            const SbParams& P = sp[u];
            const f4v d4 = *(const f4v*)&P.d[4 * g];
            const f4v dm4 = *(const f4v*)&P.dmin[4 * g];
            const float xs = P.xs[c];
            float dxs[4];
#pragma unroll
            for (int i = 0; i < 4; i++) dxs[i] = d4[i] * xs;
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                const int k = KK * w + kk;
                const f4v dI = sdI[u][k][lane];
                const f4v m4 = *(const f4v*)&P.m[k][4 * g];
                const float xk = P.xsum[k][c];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    accF[kk][i] = fmaf(dI[i], dxs[i], accF[kk][i]);
                    const float mx = m4[i] * xk;
                    accM[kk][i] = fmaf(dm4[i], mx, accM[kk][i]);
                }
            }
        }
        wait_lgkm0();
        lds_barrier();
    }
    wait_vmem_le<0>();  // the last refills (never read) have landed
    // tree8 over the lanes k (held by the waves) through LDS
    float* vb = (float*)dyn;  // [k][MFMA lane][row i]
#pragma unroll
    for (int kk = 0; kk < KK; kk++)
#pragma unroll
        for (int i = 0; i < 4; i++) vb[((KK * w + kk) * 64 + lane) * 4 + i] = accF[kk][i] - accM[kk][i];
    __syncthreads();
    if (w == 0 && c < a.p) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = row0 + 4 * g + i;
            if (r >= a.rows) continue;
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = vb[(k * 64 + lane) * 4 + i];
            const float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
            a.out[(size_t)c * a.out_stride + r] = (s0 + s1) + (s2 + s3);
        }
    }
}

// At most 8 tokens: lane pairs.  Tile m of a block holds AVX2 lanes 2m
// (MFMA columns 0-7, tokens 0-7) and 2m + 1 (columns 8-15): two MFMAs
// accumulate into it, each with the other lane's B columns zero, so every
// column is a real (lane, token) product (the exact integer I, below 2^24,
// whatever the accumulation order).  Eight waves, wave w: the block w of each
// group for the MFMA phase, then the chains of pair w / 2 for rows
// 4g + 2 (w % 2) .. + 1 of each D lane.  Half the products in LDS, half the
// chain steps and B conversions of prefill_q4k_b16s_kernel, and room for a
// ring three blocks deep.
template <int DEPTH>
constexpr size_t sp_lds_bytes() {
    return sizeof(f4v) * 8 * 4 * 64 + sizeof(SbParams) * 8 + sizeof(SsSlot<8>) * 8 * DEPTH;
}
template <int DEPTH>
__global__ __launch_bounds__(512) void prefill_q4k_b16p_kernel(PfArgs a) {
    constexpr int NW = 8;
    constexpr int NC = ss_copies<8>();
    typedef SsSlot<8> S;
    extern __shared__ __attribute__((aligned(16))) uint8_t dyn[];
    f4v (*sdI)[4][64] = (f4v (*)[4][64])dyn;                          // [block][pair][MFMA lane]
    SbParams* sp = (SbParams*)(dyn + sizeof(f4v) * NW * 4 * 64);       // [block]
    uint8_t* ring = dyn + sizeof(f4v) * NW * 4 * 64 + sizeof(SbParams) * NW;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, c = lane & 15;
    const int row0 = blockIdx.x * 16;
    const int odd = c >> 3, t = c & 7;    // this lane's B column: lane parity, token
    const int tb = min(t, a.p - 1);      // token whose q8 this lane supplies
    const int tc = min(c, a.p - 1);      // token of the per-token factors (columns < 8 used)
    const int nb = a.blocks;
    const int pm = w >> 1, ih = w & 1;   // chain phase: pair, row half
    const uint32_t ring_w = lds_addr(ring + sizeof(S) * DEPTH * w);
    float accF[2], accM[2];
    accF[0] = accF[1] = accM[0] = accM[1] = 0.0f;
#pragma unroll
    for (int d = 0; d < DEPTH; d++) ss_copy<8>(a, w + NW * d, ring_w + sizeof(S) * d, lane);
    int slot = 0;
#pragma unroll 1
    for (int q0 = 0; q0 < nb; q0 += NW) {
        wait_vmem_le<(DEPTH - 1) * NC>();
        const S& sl = *(const S*)(ring + sizeof(S) * (DEPTH * w + slot));
        {
            const u4v hdr = *(const u4v*)&sl.hdr[c][0];
            uint32_t sc_lo, sc_hi, mn;
            sb_scale_min(hdr, 2 * g, sc_lo, mn);
            sb_scale_min(hdr, 2 * g + 1, sc_hi, mn);
            const _Float16 hl = (_Float16)(float)sc_lo, nl = (_Float16)(-1024.0f * (float)sc_lo);
            const _Float16 hh = (_Float16)(float)sc_hi, nh = (_Float16)(-1024.0f * (float)sc_hi);
            const uint32_t bl = __builtin_bit_cast(uint16_t, hl), bnl = __builtin_bit_cast(uint16_t, nl);
            const uint32_t bh = __builtin_bit_cast(uint16_t, hh), bnh = __builtin_bit_cast(uint16_t, nh);
            const uint32_t sh_lo = bl | (bl << 16), sn_lo = bnl | (bnl << 16);
            const uint32_t sh_hi = bh | (bh << 16), sn_hi = bnh | (bnh << 16);
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const uint32_t w0 = *(const uint32_t*)&sl.nib[2 * m][c][4 * g];
                const uint32_t w1 = *(const uint32_t*)&sl.nib[2 * m + 1][c][4 * g];
                const uint2 q8 = *(const uint2*)&sl.q8[2 * m + odd][tb][8 * g];
                const h8v a0 = dequant_a(w0, sh_lo, sn_lo, sh_hi, sn_hi);
                const h8v a1 = dequant_a(w1, sh_lo, sn_lo, sh_hi, sn_hi);
                uint32_t v[4];
                i8x4_to_h(q8.x, v[0], v[1]);
                i8x4_to_h(q8.y, v[2], v[3]);
                const u4v zero = {0u, 0u, 0u, 0u};
                const u4v bu = {v[0], v[1], v[2], v[3]};
                const h8v b0 = __builtin_bit_cast(h8v, odd ? zero : bu);
                const h8v b1 = __builtin_bit_cast(h8v, odd ? bu : zero);
                const f4v z = {0.0f, 0.0f, 0.0f, 0.0f};
                f4v dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0, z, 0, 0, 0);
                dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1, dd, 0, 0, 0);
                sdI[w][m][lane] = dd;
            }
            if (g == 0) {
                sp[w].d[c] = f16_bits_to_f32(hdr.x & 0xffffu);
                sp[w].dmin[c] = f16_bits_to_f32(hdr.x >> 16);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    uint32_t scj, mnj;
                    sb_scale_min(hdr, j, scj, mnj);
                    sp[w].m[j][c] = (float)mnj;
                }
            } else if (g == 1) {
                sp[w].xs[c] = sl.xs[tc];
#pragma unroll
                for (int k = 0; k < 8; k++) sp[w].xsum[k][c] = sl.xs32[tc][k];
            }
        }
        wait_lgkm0();
        ss_copy<8>(a, q0 + w + NW * DEPTH, ring_w + sizeof(S) * slot, lane);
        slot = slot + 1 == DEPTH ? 0 : slot + 1;
        lds_barrier();
        // chains of pair pm, rows 4g + 2 ih + ii, lane k = 2 pm + odd, token t
        const int k = 2 * pm + odd;
#pragma unroll
        for (int u = 0; u < NW; u++) {
            if (q0 + u >= nb) break;  // uniform
            const SbParams& P = sp[u];
            const f4v dI = sdI[u][pm][lane];
            const float xs = P.xs[t];
            const float xk = P.xsum[k][t];
#pragma unroll
            for (int ii = 0; ii < 2; ii++) {
                const int i = 2 * ih + ii;
                const float dxs = P.d[4 * g + i] * xs;
                accF[ii] = fmaf(dI[i], dxs, accF[ii]);
                const float mx = P.m[k][4 * g + i] * xk;
                accM[ii] = fmaf(P.dmin[4 * g + i], mx, accM[ii]);
            }
        }
        wait_lgkm0();
        lds_barrier();
    }
    wait_vmem_le<0>();
    // tree8 over the lanes k through LDS: vb[k][row][token]
    float* vb = (float*)dyn;
#pragma unroll
    for (int ii = 0; ii < 2; ii++)
        vb[((2 * pm + odd) * 16 + 4 * g + 2 * ih + ii) * 8 + t] = accF[ii] - accM[ii];
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < 128) {
        const int r = tid >> 3, tt = tid & 7;
        if (tt < a.p && row0 + r < a.rows) {
            float v[8];
#pragma unroll
            for (int kk = 0; kk < 8; kk++) v[kk] = vb[(kk * 16 + r) * 8 + tt];
            const float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
            a.out[(size_t)tt * a.out_stride + row0 + r] = (s0 + s1) + (s2 + s3);
        }
    }
}

template <int DEPTH>
static bool launch_b16p(const PfArgs& a, hipStream_t s) {
    constexpr size_t lds = sp_lds_bytes<DEPTH>();
    static_assert(lds <= 160 * 1024, "LDS");
    static const bool ok = hipFuncSetAttribute((const void*)prefill_q4k_b16p_kernel<DEPTH>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)lds) == hipSuccess;
    if (!ok) {
        (void)hipGetLastError();
        return false;
    }
    hipLaunchKernelGGL((prefill_q4k_b16p_kernel<DEPTH>), dim3((a.rows + 15) / 16), dim3(512), lds,
                       s, a);
    return true;
}

template <int NW, int DEPTH, int PT>
static bool launch_b16s(const PfArgs& a, hipStream_t s) {
    constexpr size_t lds = ss_lds_bytes<NW, DEPTH, PT>();
    static_assert(lds <= 160 * 1024, "LDS");
    static const bool ok = hipFuncSetAttribute((const void*)prefill_q4k_b16s_kernel<NW, DEPTH, PT>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)lds) == hipSuccess;
    if (!ok) {
        (void)hipGetLastError();
        return false;
    }
    hipLaunchKernelGGL((prefill_q4k_b16s_kernel<NW, DEPTH, PT>), dim3((a.rows + 15) / 16),
                       dim3(64 * NW), lds, s, a);
    return true;
}


// Kernel choice.  More than 16 activation rows: the 64 x 64 staged tile
// (prefill_q4k_tiled_kernel).  At most 16 rows (a decode batch): 64 rows x
// 16 tokens (prefill_q4k_mfma_kernel); the per-block staging (q8 to f16,
// scale decoding) is a fixed cost per workgroup, so 64 rows per workgroup
// beat smaller tiles that would fill more CUs (measured at batch 8: 22.8 vs
// 28.4 us for 14336 x 4096), except where 64-row tiles leave a third of the
// CUs idle: there 16-row tiles with block-parallel waves and operands in
// per-wave LDS rings (prefill_q4k_b16p_kernel up to 8 tokens, four-wave
// prefill_q4k_b16s_kernel at 9-16).  The tiled and ring kernels address a
// weight with 32-bit offsets.
int launch_q4k_mfma(const uint8_t* d_w, size_t rb, int rows, int blocks, const ActQ8& act, int p,
                    float* out, int out_stride, hipStream_t s) {
    if (rows <= 0 || blocks <= 0 || p <= 0) return GLLM_OK;
    PfArgs a{d_w, rb, rows, blocks, act, p, out, out_stride};
    const bool fits = (size_t)rows * rb < ((size_t)1 << 32);
    if (p > kTiledMinP) {
        if (!act.b16t || !fits)
            return fail(GLLM_EINVAL, "prefill: %d rows of %zu B need f16 tiles and < 4 GiB", rows, rb);
        const TlMap mp = tl_map(rows, p);
        const int grid = 8 * mp.tg_size * mp.rg_size;
        hipLaunchKernelGGL(prefill_q4k_tiled_kernel, dim3(grid), dim3(512), 0, s, a, mp);
    } else if ((rows + 63) / 64 < 2 * device_cus() / 3) {
        if (!fits) return fail(GLLM_EINVAL, "prefill: weights of %zu B past 4 GiB", (size_t)rows * rb);
        const bool done = p > 8 ? launch_b16s<4, 3, 16>(a, s) : launch_b16p<2>(a, s);
        if (!done) return fail(GLLM_EDEVICE, "prefill: the LDS of the 16-row kernel was refused");
    } else {
        launch_pf<4, 1>(a, s);
    }
    GLLM_HIP(hipGetLastError());
    return GLLM_OK;
}

}  // namespace gllm
