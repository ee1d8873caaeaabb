// gemv_formats.h -- row kernels for Q5_K, Q4_0, Q4_1, MXFP4, Q2_K and Q3_K
// against Q8K activations, bit-exact to kernels_amd64.s:550-1128 (included
// by gemv.hip, which supplies GemvJob, locate, rot_prev, tree8_strided,
// dot4z, q4k_lane_sum, MinSel and the fused-quantisation helpers).
//
// Every format keeps the AVX2 lane structure of its reference kernel: lane k
// of a row owns elements 32m + 4k .. 32m + 4k + 3 of every 32-element group
// m of a 256-element block, which is exactly the lane-permuted q8 layout the
// activations use.  Per block (or per 32-element block for the legacy
// formats) each lane forms its exact int32 and advances its fp32 chains with
// the reference's operations in the reference's order; the row ends with the
// same 8 -> 4 -> 2 -> 1 tree (plus the scalar offset chain of Q4_0 / Q4_1).
//
// Upload repacks (same byte count per 256 elements; see repack_kernel):
//   Q5_K  176 B: [16 header][lane k: 16 nibble bytes at 16+16k][lane k: qh dword at 144+4k]
//   Q2_K   84 B: [d, dmin][16 scale bytes at 4][lane k: qs dwords n=0,1 at 20+8k]
//   Q3_K  110 B: [d][12 scale bytes at 2][lane k: hmask, qs n=0, qs n=1 dwords at 14+12k]
//   Q4_0  144 B per 8 blocks: [8 x f16 d][lane group kk: 8 nibble dwords at 16+32kk]
//   Q4_1  160 B per 8 blocks: [8 x (d, m)][lane group kk: 8 nibble dwords at 32+32kk]
//   MXFP4 136 B per 8 blocks: [8 exponent bytes][lane k: 8 code ushorts at 8+16k]
// Q3_K blocks are only 2-byte aligned, so its lanes read 16-bit halves.

namespace fmt {

// Which activation sums a format reads, and whether its chains exist.
enum Sums { kNone = 0, kX32 = 1, kX16 = 2 };

__device__ __forceinline__ uint32_t ld32(const uint8_t* p) { return *(const uint32_t*)p; }
// two aligned 16-bit halves (p is 2-byte aligned)
__device__ __forceinline__ uint32_t ld32h(const uint8_t* p) {
    const uint16_t* h = (const uint16_t*)p;
    return (uint32_t)h[0] | ((uint32_t)h[1] << 16);
}

// Activation operands of one lane, one token, one 256-element block: the
// q8 bytes, the Q8K scale and the kNX activation sums the format reads
// (Q5_K: x32[k]; Q4_0 / Q4_1: x32[0..7]; Q2_K: x16[k], x16[8 + k]).
struct Act {
    int4 qa, qb;        // groups 0..3 and 4..7, lane k's 4 bytes each
    float xs;           // Q8K scale of the block
    float xv[8];
    __device__ __forceinline__ int q(int m) const {
        const int v[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        return v[m];
    }
};

// Fill a's sums for format F from the block's sums in memory.
template <class F>
__device__ __forceinline__ void load_sums(Act& a, int k, const float* x32, const float* x16) {
    if constexpr (F::kSums == kX32 && F::kNX == 1) {
        a.xv[0] = x32[k];
    } else if constexpr (F::kSums == kX32) {
#pragma unroll
        for (int g = 0; g < 8; g++) a.xv[g] = x32[g];
    } else if constexpr (F::kSums == kX16) {
        a.xv[0] = x16[k];
        a.xv[1] = x16[8 + k];
    }
}

// ---- Q5_K -----------------------------------------------------------------
struct Q5K {
    static constexpr int kBytes = 176, kSums = kX32, kNX = 1;
    static constexpr bool kHasM = true, kHasS = false;
    struct Regs {
        uint4 h, q;
        uint32_t qh;
    };
    __device__ static void load(const uint8_t* blk, int k, Regs& r) {
        r.h = *(const uint4*)blk;
        r.q = *(const uint4*)(blk + 16 + 16 * k);
        r.qh = ld32(blk + 144 + 4 * k);
    }
    // q5kDotQ8KRow (kernels_amd64.s:578-663): Q4_K's chains, codes with the
    // fifth bit of qh ORed in (bit 2s for low nibbles, 2s+1 for high).
    template <int G>
    __device__ static void step(const Regs& r, int k, const Act& a, float& accF, float& accM,
                                float&) {
        const float d = f16_bits_to_f32(r.h.x & 0xffffu);
        const float dmin = f16_bits_to_f32(r.h.x >> 16);
        const uint32_t sc03 = r.h.y & 0x3f3f3f3fu;
        const uint32_t sc47 = (r.h.w & 0x0f0f0f0fu) | ((r.h.y >> 2) & 0x30303030u);
        const float mkf = (float)MinSel(k).get(r.h.z, r.h.w);
        const uint32_t qs[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        int t[8];
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int lo = (int)((qs[s] & 0x0f0f0f0fu) | (((r.qh >> (2 * s)) & 0x01010101u) << 4));
            const int hi = (int)(((qs[s] >> 4) & 0x0f0f0f0fu) | (((r.qh >> (2 * s + 1)) & 0x01010101u) << 4));
            t[2 * s] = dot4z(lo, a.q(2 * s));
            t[2 * s + 1] = dot4z(hi, a.q(2 * s + 1));
        }
        const int acc = q4k_lane_sum(t[0], t[1], t[2], t[3], t[4], t[5], t[6], t[7], sc03, sc47);
        const float iv = (float)acc;
        const float dxs = d * a.xs;                 // VMULSS
        const float mx = mkf * a.xv[0];             // VMULPS
#pragma unroll
        for (int st = 0; st < G; st++) {
            accF = fmaf(iv, dxs, rot_prev<G>(accF));     // VFMADD231PS
            accM = fmaf(dmin, mx, rot_prev<G>(accM));    // VFMADD231PS
        }
    }
};

// ---- Q2_K -----------------------------------------------------------------
struct Q2K {
    static constexpr int kBytes = 84, kSums = kX16, kNX = 2;
    static constexpr bool kHasM = true, kHasS = false;
    struct Regs {
        uint32_t dd, sc[4], q0, q1;
    };
    __device__ static void load(const uint8_t* blk, int k, Regs& r) {
        r.dd = ld32(blk);
#pragma unroll
        for (int i = 0; i < 4; i++) r.sc[i] = ld32(blk + 4 + 4 * i);
        r.q0 = ld32(blk + 20 + 8 * k);
        r.q1 = ld32(blk + 24 + 8 * k);
    }
    // scale byte 4q + (i & 3) where the dword q is fixed at compile time (a
    // runtime index into sc[] would move the whole register ring to scratch)
    __device__ static int byte_of(uint32_t w, int i) { return (int)((w >> (8 * (i & 3))) & 0xffu); }
    // q2kDotQ8KRow (kernels_amd64.s:816-887): group m's codes at shift
    // 2(m%4) of qs dword m/4, weighted by the d-scale nibble of sub-block
    // 2m + k/4; min term t = fma(min_{8+k}, xsum_{8+k}, min_k * xsum_k).
    template <int G>
    __device__ static void step(const Regs& r, int k, const Act& a, float& accF, float& accM,
                                float&) {
        const float d = f16_bits_to_f32(r.dd & 0xffffu);
        const float dmin = f16_bits_to_f32(r.dd >> 16);
        int acc = 0;
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const uint32_t qn = m < 4 ? r.q0 : r.q1;
            const int code = (int)((qn >> (2 * (m & 3))) & 0x03030303u);
            // sub-block 2m + k/4 lies in scale dword m/2
            acc += (byte_of(r.sc[m >> 1], 2 * m + (k >> 2)) & 15) * dot4z(code, a.q(m));
        }
        const int mk = byte_of(k < 4 ? r.sc[0] : r.sc[1], k) >> 4;
        const int mk8 = byte_of(k < 4 ? r.sc[2] : r.sc[3], k) >> 4;
        float t = (float)mk * a.xv[0];                            // VMULPS
        t = fmaf((float)mk8, a.xv[1], t);                         // VFMADD231PS
        const float iv = (float)acc;
        const float dxs = d * a.xs;
#pragma unroll
        for (int st = 0; st < G; st++) {
            accF = fmaf(dxs, iv, rot_prev<G>(accF));
            accM = fmaf(dmin, t, rot_prev<G>(accM));
        }
    }
};

// ---- Q3_K -----------------------------------------------------------------
struct Q3K {
    static constexpr int kBytes = 110, kSums = kNone, kNX = 0;
    static constexpr bool kHasM = false, kHasS = false;
    struct Regs {
        uint32_t d, s0, s1, s2, hm, q0, q1;
    };
    __device__ static void load(const uint8_t* blk, int k, Regs& r) {
        r.d = *(const uint16_t*)blk;
        r.s0 = ld32h(blk + 2);
        r.s1 = ld32h(blk + 6);
        r.s2 = ld32h(blk + 10);
        r.hm = ld32h(blk + 14 + 12 * k);
        r.q0 = ld32h(blk + 18 + 12 * k);
        r.q1 = ld32h(blk + 22 + 12 * k);
    }
    // q3kDotQ8KRow (kernels_amd64.s:945-1063): w = code + 4 * (hmask bit m),
    // lane dot w.a - 4 * sum(a) (== the signed values times a), weighted by
    // dl = scale - 32 of sub-block 2m + k/4 (q3KScales, quant_extra.go:315).
    template <int G>
    __device__ static void step(const Regs& r, int k, const Act& a, float& accF, float&, float&) {
        const uint32_t sc[4] = {
            (r.s0 & 0x0f0f0f0fu) | ((r.s2 << 4) & 0x30303030u),
            (r.s1 & 0x0f0f0f0fu) | ((r.s2 << 2) & 0x30303030u),
            ((r.s0 >> 4) & 0x0f0f0f0fu) | (r.s2 & 0x30303030u),
            ((r.s1 >> 4) & 0x0f0f0f0fu) | ((r.s2 >> 2) & 0x30303030u)};
        int acc = 0;
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const uint32_t qn = m < 4 ? r.q0 : r.q1;
            const uint32_t w = ((qn >> (2 * (m & 3))) & 0x03030303u) + (((r.hm >> m) & 0x01010101u) << 2);
            const int am = a.q(m);
            const int dot = dot4z((int)w, am) - 4 * dot4z(0x01010101, am);
            const int i = 2 * m + (k >> 2);
            const int dl = (int)((sc[i >> 2] >> (8 * (i & 3))) & 0xffu) - 32;
            acc += dl * dot;
        }
        const float iv = (float)acc;
        const float dxs = f16_bits_to_f32(r.d) * a.xs;
#pragma unroll
        for (int st = 0; st < G; st++) accF = fmaf(dxs, iv, rot_prev<G>(accF));
    }
};

// ---- Q4_0 / Q4_1 ------------------------------------------------------------
template <bool Q41>
struct Q401 {
    static constexpr int kBytes = Q41 ? 160 : 144, kSums = kX32, kNX = 8;
    static constexpr bool kHasM = false, kHasS = true;
    struct Regs {
        uint4 h0, h1;  // Q4_0: h0 = 8 f16 d; Q4_1: h0, h1 = 8 (d | m << 16)
        uint4 n0, n1;  // nibble dword of blocks 0..7 for this lane group
    };
    __device__ static void load(const uint8_t* blk, int k, Regs& r) {
        r.h0 = *(const uint4*)blk;
        if constexpr (Q41) r.h1 = *(const uint4*)(blk + 16);
        const uint8_t* nb = blk + (Q41 ? 32 : 16) + 32 * (k & 3);
        r.n0 = *(const uint4*)nb;
        r.n1 = *(const uint4*)(nb + 16);
    }
    // q4_0DotQ8KRow / q4_1DotQ8KRow (kernels_amd64.s:679-793): per 32-block
    // g, lane k's unsigned codes (low nibbles for k < 4, high for k >= 4),
    // accF = fma(d*xs, float(I), accF); the offset chain is
    // fma(-8, d*xsum_g, s) (Q4_0) or s + m*xsum_g (Q4_1).
    template <int G>
    __device__ static void step(const Regs& r, int k, const Act& a, float& accF, float&,
                                float& accS) {
        const uint32_t nib[8] = {r.n0.x, r.n0.y, r.n0.z, r.n0.w, r.n1.x, r.n1.y, r.n1.z, r.n1.w};
        const uint32_t hd[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
        const int sh = 4 * (k >> 2);
        float iv[8], dxs[8], off[8];
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const int code = (int)((nib[g] >> sh) & 0x0f0f0f0fu);
            iv[g] = (float)dot4z(code, a.q(g));
            float d, m = 0.0f;
            if constexpr (Q41) {
                d = f16_bits_to_f32(hd[g] & 0xffffu);
                m = f16_bits_to_f32(hd[g] >> 16);
            } else {
                d = f16_bits_to_f32((hd[g >> 1] >> (16 * (g & 1))) & 0xffffu);
            }
            dxs[g] = d * a.xs;                               // VMULSS X9, X0
            off[g] = (Q41 ? m : d) * a.xv[g];                // VMULSS (R9)
        }
#pragma unroll
        for (int st = 0; st < G; st++) {
            float f = rot_prev<G>(accF), s = rot_prev<G>(accS);
#pragma unroll
            for (int g = 0; g < 8; g++) {
                f = fmaf(dxs[g], iv[g], f);                  // VFMADD231PS
                if constexpr (Q41) s = s + off[g];           // VADDSS
                else s = fmaf(-8.0f, off[g], s);             // VFMADD231SS
            }
            accF = f;
            accS = s;
        }
    }
};

// ---- MXFP4 ------------------------------------------------------------------
struct MXFP4 {
    static constexpr int kBytes = 136, kSums = kNone, kNX = 0;
    static constexpr bool kHasM = false, kHasS = false;
    struct Regs {
        uint2 e;   // exponent bytes of blocks 0..7
        uint4 c;   // code ushort of blocks 0..7 (two per dword)
    };
    __device__ static void load(const uint8_t* blk, int k, Regs& r) {
        r.e = *(const uint2*)blk;
        const uint2 lo = *(const uint2*)(blk + 8 + 16 * k);
        const uint2 hi = *(const uint2*)(blk + 16 + 16 * k);
        r.c = make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
    // Lane dot of one 32-block against mxfp4DoubledLUT values: u holds the
    // lane's four codes (nibbles, element order).  Magnitudes come from one
    // byte permute of the table {0,1,2,3,4,6,8,12}; the sign bit splits the
    // dot into a positive and a negative part (VPSIGNB on the activations
    // gives the same integer), so nothing is negated bytewise.
    __device__ static int lane_dot(uint32_t u, int act) {
        const uint32_t lo = u & 0x0f0fu, hi = (u >> 4) & 0x0f0fu;        // codes 0, 2 | 1, 3
        const uint32_t codes = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // c0 c1 c2 c3
        const uint32_t mag = __builtin_amdgcn_perm(0x0c080604u, 0x03020100u, codes & 0x07070707u);
        const uint32_t neg = ((codes >> 3) & 0x01010101u) * 0xffu;
        return dot4z((int)(mag & ~neg), act) - dot4z((int)(mag & neg), act);
    }
    // mxfp4DotQ8KRow (kernels_amd64.s:1065-1128): hx = 0.5 * xs, then per
    // 32-block accF = fma(bits(e << 23) * hx, float(I), accF).
    template <int G>
    __device__ static void step(const Regs& r, int, const Act& a, float& accF, float&, float&) {
        const uint32_t cw[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
        const float hx = 0.5f * a.xs;                             // VMULSS (R8), X7
        float iv[8], sc[8];
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const uint32_t u = (cw[g >> 1] >> (16 * (g & 1))) & 0xffffu;
            iv[g] = (float)lane_dot(u, a.q(g));
            const uint32_t eb = (g < 4 ? r.e.x >> (8 * g) : r.e.y >> (8 * (g - 4))) & 0xffu;
            sc[g] = __uint_as_float(eb << 23) * hx;                // VMULSS X10, X0
        }
#pragma unroll
        for (int st = 0; st < G; st++) {
            float f = rot_prev<G>(accF);
#pragma unroll
            for (int g = 0; g < 8; g++) f = fmaf(sc[g], iv[g], f);  // VFMADD231PS
            accF = f;
        }
    }
};

}  // namespace fmt

// One row kernel for every format above: lane (k, gi) of row r walks blocks
// gi, gi + G, ... with D blocks of weight bytes in flight, loaded in block
// order and unconditionally (clamped to the lane's last block) so the
// compiler's vmcnt waits never drain the ring.  At batch 1 the block's
// activation operands ride in the ring as well.
template <class F, int NT>
constexpr int fmt_depth() {
    return NT == 1 ? (F::kNX == 8 ? 3 : 4) : 2;
}

//
// FUSE (batch 1, cols <= kFuseCols) quantises x into LDS inside the
// workgroup, as gemv_q6k_kernel does.
template <class F, int NT, int G, bool FUSE = false>
__global__ __launch_bounds__(256) void gemv_fmt_kernel(GemvJob j) {
    static_assert(!FUSE || NT == 1, "fused quantisation is batch 1 only");
    constexpr int D = fmt_depth<F, NT>();
    __shared__ __attribute__((aligned(16))) uint8_t fa_raw[FUSE ? sizeof(FusedAct) : 16];
    FusedAct& fa = *(FusedAct*)fa_raw;
    int wi;
    const int tid = threadIdx.x;
    const int gi = tid % G, k = (tid / G) & 7;
    const int r = locate(j, blockIdx.x, &wi) + tid / (8 * G);
    if (!FUSE && r >= j.rows[wi]) return;  // whole rows: the rotation and tree stay inside one row
    const bool live = r < j.rows[wi];
    const int B = j.blocks, NB = B / G;
    const uint8_t* row = j.w[wi] + (size_t)(live ? r : j.rows[wi] - 1) * j.rb;
    float accF[NT], accM[NT], accS[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) accF[t] = accM[t] = accS[t] = 0.0f;
    struct Slot {
        typename F::Regs w;
        fmt::Act a;  // NT == 1 only
    };
    const size_t tok0 = (size_t)j.tok0;
    auto act_of = [&](size_t tok, int b, fmt::Act& a) __attribute__((always_inline)) {
        if constexpr (FUSE) {
            a.qa = *(const int4*)(fa.q8 + b * 256 + k * 32);
            a.qb = *(const int4*)(fa.q8 + b * 256 + k * 32 + 16);
            a.xs = fa.xsc[b];
            fmt::load_sums<F>(a, k, fa.xs32 + b * 8, fa.xs16 + b * 16);
        } else {
            const int8_t* q8 = j.act.q8perm + tok * j.cols + (size_t)b * 256 + k * 32;
            a.qa = *(const int4*)q8;
            a.qb = *(const int4*)(q8 + 16);
            a.xs = j.act.xscale[tok * B + b];
            fmt::load_sums<F>(a, k, j.act.xs32 + tok * (j.cols / 32) + (size_t)b * 8,
                              j.act.xs16 + tok * (j.cols / 16) + (size_t)b * 16);
        }
    };
    Slot ring[D];
    auto load_w = [&](int i, Slot& o) __attribute__((always_inline)) {
        F::load(row + (size_t)(min(i, NB - 1) * G + gi) * F::kBytes, k, o.w);
    };
    auto load = [&](int i, Slot& o) __attribute__((always_inline)) {
        load_w(i, o);
        if constexpr (NT == 1) act_of(tok0, min(i, NB - 1) * G + gi, o.a);
    };
    auto compute = [&](int i, const Slot& o) __attribute__((always_inline)) {
        if constexpr (NT == 1) {
            F::template step<G>(o.w, k, o.a, accF[0], accM[0], accS[0]);
        } else {
            const int b = i * G + gi;
#pragma unroll
            for (int t = 0; t < NT; t++) {
                if (t < j.ntok) {
                    fmt::Act a;
                    act_of(tok0 + t, b, a);
                    F::template step<G>(o.w, k, a, accF[t], accM[t], accS[t]);
                }
            }
        }
    };
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
        fused_act_store<F::kSums == fmt::kX16>(xr, B, fa);
#pragma unroll
        for (int i = 0; i < D; i++) act_of(tok0, min(i, NB - 1) * G + gi, ring[i].a);
    }
    int i0 = 0;
    for (; i0 + D <= NB; i0 += D) {
#pragma unroll
        for (int ii = 0; ii < D; ii++) {
            compute(i0 + ii, ring[ii]);
            __builtin_amdgcn_sched_barrier(0);
            load(i0 + ii + D, ring[ii]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int ii = 0; ii < D - 1; ii++)
        if (i0 + ii < NB) compute(i0 + ii, ring[ii]);  // uniform
#pragma unroll
    for (int t = 0; t < NT; t++) {
        float v = tree8_strided<G>(F::kHasM ? accF[t] - accM[t] : accF[t]);  // VSUBPS + tree
        if constexpr (F::kHasS) v = v + accS[t];                               // VADDSS
        if (live && k == 0 && gi == G - 1 && t < j.ntok)
            j.out[wi][(size_t)(j.tok0 + t) * j.out_stride[wi] + r] = v;
    }
}
