// decode.hip -- resident llama decoder on one device: the glue kernels of
// ForwardBodyInto (model.go:2622-2820) / ForwardBatchInto
// (forward_batch.go:336-613) in the reference's amd64 float order, and the
// host driver that sequences them around the row kernels and attention.
//
//   embedding      Weight.RowInto model.go:1034-1100 (launch_weight_rows, any type)
//   projections    decode: the fused groups of tryMatvecAttentionInto /
//                  tryMatvec2Into (model.go:3157-3206: int8 row dots, or the
//                  float kernels for same-type groups of the other formats);
//                  prefill: matvecBatchQ8 per matrix (forward_batch.go:108-233)
//   rmsNormInto    model.go:2986-3011: ss = dotF32AVX2(x, x) (kernels_amd64.s:28-93),
//                  scale = float32(1/sqrt(float64(ss/n + eps))), out = (x*w)*scale
//   RoPE           prepareRopeScratch model.go:3020-3049 (host tables, the
//                  same libm calls), applyPreparedRope interleaved :3051-3093
//   storeKV        model.go:1466-1489 (f16 RNE)
//   residual       addInPlace = AxpyF32(dst, 1, src) model.go:3857
//   SwiGLU         siluMulF32AVX2 kernels_amd64.s:1630-1700
//   greedy         ArgmaxMatvec model.go:754 / argmaxFiniteToken sampling.go:399
#include <math.h>

#include <algorithm>
#include <vector>

#include "gllm_common.h"

namespace gllm {
int gemv_f32(int n, gllm_hip_weight* const* ws, const float* d_xs, int p, float* const* outs,
             const int* strides, void* act_buf, hipStream_t s);
int gemv_group(int n, gllm_hip_weight* const* ws, const float* d_x, float* const* outs,
               const int* strides, void* act_buf, hipStream_t s);
int group_routing(int n, gllm_hip_weight* const* ws, int* fl);
bool norm_fusable(int n, gllm_hip_weight* const* ws);
bool swiglu_epi_ok(gllm_hip_weight* const* gu, const gllm_hip_weight* down);
int gemv_norm_swiglu_f32(gllm_hip_weight* const* gu, gllm_hip_weight* down, const float* x,
                         const float* res, const float* nw, float eps, float* xout, float* gate,
                         float* up, float* out, void* act_buf, int* cnt, hipStream_t s);
int gemv_norm_f32(int n, gllm_hip_weight* const* ws, const float* x, const float* res,
                  const float* nw, float eps, float* xout, float* const* outs, hipStream_t s);
bool row_kernel_type(int t);
bool rows_type(int t);
int launch_weight_rows(const gllm_hip_weight* w, const uint32_t* d_ids, int n, float* d_out,
                       hipStream_t s);
int gemv_silu_f32(gllm_hip_weight* w, const float* gate, const float* up, int p, float* out,
                  void* act_buf, float* hidden, hipStream_t s);
int attend_exact(const gllm_hip_kv* kv, int l, const float* d_q, int n_heads, int n_kv, int hd,
                 int start, int end0, int p, float scale, float* d_out, hipStream_t s,
                 float* scratch, const int* d_end, int span_cap, const float* rope_sin,
                 const float* rope_cos, const float* d_knew, const float* d_vnew,
                 const float* rope_cur = nullptr);
bool attend_exact_graphable(const gllm_hip_kv* kv, int n_heads, int n_kv, int hd, int span_cap);
int attend_splitk(const gllm_hip_kv* kv, int l, const float* d_q, int n_heads, int n_kv, int hd,
                  int start, int end, float scale, float* d_out, hipStream_t s);
int kv_store_dev_impl(gllm_hip_kv* kv, int l, int pos, const float* d_k, const float* d_v,
                      hipStream_t s);
int launch_argmax(const float* logits, int n, uint32_t* token, unsigned long long* keys,
                  hipStream_t s, const uint32_t* recent, int n_recent, float penalty);
size_t argmax_keys(int n);
bool argmax_fusable(const gllm_hip_weight* w);
size_t argmax_epilogue_keys(const gllm_hip_weight* w);
int gemv_argmax_f32(gllm_hip_weight* w, const float* x, float* logits, unsigned long long* keys,
                    uint32_t* token, const uint32_t* recent, int n_recent, float penalty,
                    hipStream_t s);
}  // namespace gllm

struct gllm_hip_model {
    gllm_hip_model_config cfg;
    std::vector<gllm_hip_weight*> w;  // [layer * 7 + slot] for slots 0..6
    std::vector<gllm_hip_weight*> owned;  // weights the model releases (loaded from a file)
    gllm_hip_weight* tok_embd = nullptr;
    gllm_hip_weight* output = nullptr;
    float* d_norms = nullptr;  // [2 * n_layers + 1][dim]: attn, ffn per layer, then output
    float* d_sin = nullptr;    // [max_len][head_dim/2]
    float* d_cos = nullptr;
    gllm_hip_kv* kv = nullptr;
    hipStream_t stream = nullptr;
    int max_p = 0;  // capacity of the activation buffers below (tokens)
    float *x = nullptr, *xn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr;
    float* x2 = nullptr;  // second residual-stream buffer (norm-fused launches alternate x / x2)
    int* sq_cnt = nullptr;  // [hidden / 256] block counters of the SwiGLU epilogue (zero at rest)
    float *proj = nullptr, *gate = nullptr, *up = nullptr, *hidden = nullptr, *logits = nullptr;
    uint32_t* d_tokens = nullptr;
    uint32_t* h_tokens = nullptr;  // pinned
    unsigned long long* argmax_keys = nullptr;  // argmax_keys(vocab) entries
    // the head's argmax keys: vocab / 8 + 8 >= argmax_epilogue_keys(output)
    unsigned long long* head_keys = nullptr;
    void* act = nullptr;           // Q8K activation buffers
    size_t act_n = 0;
    float* scores = nullptr;       // attention scores and the long-span kernel's chunk maxima
    int* d_pos = nullptr;          // decode position read by the captured decode step
    int* h_pos = nullptr;          // pinned staging for it
    hipGraphExec_t decode_graph = nullptr;  // one decode step, captured after a first eager step
    int last_p = 0;
    float attn_scale = 0.0f;  // llama.attention.scale; 0 = 1/sqrt(head_dim)
    // repeat penalty over the trailing token window (runtime.go:1035 and
    // 1089-1093): ids of the last `window` tokens seen, oldest first
    float penalty = 1.0f;
    int window = 0;
    std::vector<uint32_t> recent;
    uint32_t* d_recent = nullptr;  // window ids, unused slots 0xffffffff (ignored ids)
    uint32_t* h_recent = nullptr;  // pinned staging for it
};

namespace gllm {

// ---------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------

// addInPlace (x = fma(proj, 1, x): one rounding of x + proj, model.go:3857)
// followed by rmsNormInto (model.go:2986-3011); with proj null, the norm
// alone.  One workgroup per token, 256 threads; every global load (x, proj
// and the norm weights, as float4) is issued up front, and x is staged in
// LDS so lanes 0..31, the 4 x 8 fma accumulators of dotF32AVX2 over
// 32-element strides, run their sequential chains from LDS.  n % 4 == 0 and
// n <= 4 * 256 * kNormVec.
constexpr int kNormVec = 8;  // float4 per thread: n up to 8192

__global__ __launch_bounds__(256) void add_rmsnorm_kernel(float* __restrict__ x,
                                                          const float* __restrict__ proj,
                                                          const float* __restrict__ w, int n,
                                                          float eps, float* __restrict__ out) {
    extern __shared__ float xs[];  // n floats
    __shared__ float part[32];
    __shared__ float s_scale;
    const int t = blockIdx.x, tid = threadIdx.x;
    const int n4 = n >> 2;
    float4* xt = (float4*)(x + (size_t)t * n);
    const float4* pt = proj ? (const float4*)(proj + (size_t)t * n) : nullptr;
    const float4* w4 = (const float4*)w;
    float4 xv[kNormVec], pv[kNormVec], wv[kNormVec];
#pragma unroll
    for (int u = 0; u < kNormVec; u++) {
        const int i = tid + 256 * u;
        if (i < n4) {
            xv[u] = xt[i];
            wv[u] = w4[i];
            if (pt) pv[u] = pt[i];
        }
    }
#pragma unroll
    for (int u = 0; u < kNormVec; u++) {
        const int i = tid + 256 * u;
        if (i < n4) {
            float4 v = xv[u];
            if (pt) {
                v.x = fmaf(pv[u].x, 1.0f, v.x);
                v.y = fmaf(pv[u].y, 1.0f, v.y);
                v.z = fmaf(pv[u].z, 1.0f, v.z);
                v.w = fmaf(pv[u].w, 1.0f, v.w);
                xt[i] = v;
            }
            xv[u] = v;
            ((float4*)xs)[i] = v;
        }
    }
    __syncthreads();
    const float scale = rms_scale_lds(xs, n, eps, part, &s_scale);
    float4* o4 = (float4*)(out + (size_t)t * n);
#pragma unroll
    for (int u = 0; u < kNormVec; u++) {
        const int i = tid + 256 * u;
        if (i < n4) {
            const float4 v = xv[u], ww = wv[u];
            o4[i] = make_float4((v.x * ww.x) * scale, (v.y * ww.y) * scale, (v.z * ww.z) * scale,
                                (v.w * ww.w) * scale);
        }
    }
}

// Interleaved RoPE (applyPreparedRope, model.go:3051-3093) on the q and k
// rows of p tokens at positions pos0 + t, then storeKV (model.go:1466-1489):
// the rotated k and the v row rounded to f16 into the cache.  Thread i owns
// rotation pair i of q and of k and elements 2i, 2i+1 of v.
__global__ void rope_kv_kernel(float* __restrict__ q, float* __restrict__ k,
                               const float* __restrict__ v, int n_heads, int n_kv, int hd, int pos0,
                               const float* __restrict__ sin_tab, const float* __restrict__ cos_tab,
                               uint16_t* __restrict__ kd, uint16_t* __restrict__ vd,
                               const int* __restrict__ d_pos) {
    const int t = blockIdx.y;
    if (d_pos) pos0 = *d_pos;  // position read on the device (graph replay)
    const int pairs = hd / 2, kv_dim = n_kv * hd;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int pos = pos0 + t;
    const int pr = i % pairs;
    const float sn = sin_tab[(size_t)pos * pairs + pr];
    const float cs = cos_tab[(size_t)pos * pairs + pr];
    if (i < n_heads * pairs) {
        float* e = q + (size_t)t * n_heads * hd + 2 * i;
        const float v0 = e[0], v1 = e[1];
        e[0] = v0 * cs - v1 * sn;
        e[1] = v0 * sn + v1 * cs;
    }
    if (i < n_kv * pairs) {
        float* e = k + (size_t)t * kv_dim + 2 * i;
        const float v0 = e[0], v1 = e[1];
        const float r0 = v0 * cs - v1 * sn, r1 = v0 * sn + v1 * cs;
        e[0] = r0;
        e[1] = r1;
        uint16_t* kc = kd + (size_t)pos * kv_dim + 2 * i;
        kc[0] = f32_to_f16_bits(r0);
        kc[1] = f32_to_f16_bits(r1);
        const float* vr = v + (size_t)t * kv_dim + 2 * i;
        uint16_t* vc = vd + (size_t)pos * kv_dim + 2 * i;
        vc[0] = f32_to_f16_bits(vr[0]);
        vc[1] = f32_to_f16_bits(vr[1]);
    }
}

// ---------------------------------------------------------------------------
// host driver
// ---------------------------------------------------------------------------

static inline int grid1(size_t n, int block) { return (int)((n + block - 1) / block); }

// RoPE sin / cos of one position (buildRopeInvFreq model.go:1728-1756,
// prepareRopeScratch model.go:3020-3049): the reference's float64 pow, sin
// and cos on the host, rounded to float32.
static void rope_row(const gllm_hip_model_config& c, int pos, float* sn, float* cs) {
    const int pairs = c.head_dim / 2;
    for (int i = 0; i < pairs; i++) {
        const float fi = (float)(i * 2);
        const float base = (float)pow((double)c.rope_theta, (double)(fi / (float)c.head_dim));
        const float inv = 1.0f / (1.0f * base);
        const double angle = (double)((float)pos * inv);
        sn[i] = (float)sin(angle) * 1.0f;
        cs[i] = (float)cos(angle) * 1.0f;
    }
}

// Decode-step upload: [position][3 pad][sin row][cos row] (floats after the
// first 16 bytes), so the captured step reads the current position's RoPE
// rows without first waiting for the position.
constexpr int kPosHeader = 4;  // 16 bytes: the decode position, the decode token, padding
static size_t pos_bytes(const gllm_hip_model_config& c) {
    return ((size_t)kPosHeader + (size_t)c.head_dim) * 4;
}

constexpr int kMaxRepeatWindow = 4096;  // the reference uses 64 (runtime.go:27)

static void drop_decode_graph(gllm_hip_model* m) {
    if (m->decode_graph) (void)hipGraphExecDestroy(m->decode_graph);
    m->decode_graph = nullptr;
}

static int ensure_buffers(gllm_hip_model* m, int p) {
    if (p <= m->max_p) return GLLM_OK;
    const auto& c = m->cfg;
    float** bufs[] = {&m->x, &m->xn, &m->q, &m->k, &m->v, &m->attn, &m->proj, &m->gate, &m->up,
                      &m->hidden, &m->x2};
    const size_t qd = (size_t)c.n_heads * c.head_dim, kvd = (size_t)c.n_kv_heads * c.head_dim;
    const size_t sizes[] = {(size_t)c.dim, (size_t)c.dim, qd, kvd, kvd, qd, (size_t)c.dim,
                            (size_t)c.hidden, (size_t)c.hidden, (size_t)c.hidden, (size_t)c.dim};
    for (int i = 0; i < 11; i++) {
        if (*bufs[i]) (void)hipFree(*bufs[i]);
        *bufs[i] = nullptr;
        GLLM_HIP(hipMalloc(bufs[i], sizes[i] * p * 4));
    }
    if (m->d_tokens) (void)hipFree(m->d_tokens);
    if (m->h_tokens) (void)hipHostFree(m->h_tokens);
    GLLM_HIP(hipMalloc(&m->d_tokens, (size_t)(p + 4) * 4));
    GLLM_HIP(hipHostMalloc(&m->h_tokens, (size_t)(p + 4) * 4, hipHostMallocDefault));
    const size_t an = act_bytes(std::max(c.dim, c.hidden), p);
    if (m->act) (void)hipFree(m->act);
    GLLM_HIP(hipMalloc(&m->act, an));
    m->act_n = an;
    if (m->scores) (void)hipFree(m->scores);
    // every attention path of a chunk, the long-span one included, works in
    // this buffer (none grows the thread's scratch)
    GLLM_HIP(hipMalloc(&m->scores, ((size_t)p * c.n_heads * (c.max_len + 1) +
                                    (size_t)c.n_heads * ((c.max_len + 31) / 32) + 64) * 4));
    m->max_p = p;
    drop_decode_graph(m);  // it captured the old buffers
    return GLLM_OK;
}

static int matvec(gllm_hip_model* m, int n, gllm_hip_weight* const* ws, const float* x, int p,
                  float* const* outs) {
    return gemv_f32(n, ws, x, p, outs, nullptr, m->act, m->stream);
}

// A layer's fused projections (Q/K/V, gate/up): a generation step routes
// them as one group (ForwardBodyInto's tryMatvecAttentionInto /
// tryMatvec2Into); prompt tokens run each projection on its own
// (matvecBatch3/2 -> matvecBatchQ8, forward_batch.go:210-233).
static int project(gllm_hip_model* m, bool decode, int n, gllm_hip_weight* const* ws,
                   const float* x, int p, float* const* outs) {
    if (decode) return gemv_group(n, ws, x, outs, nullptr, m->act, m->stream);
    return matvec(m, n, ws, x, p, outs);
}

// ForwardBatchInto / ForwardBodyInto for p consecutive tokens already in
// m->d_tokens, at positions pos0 .. pos0+p-1.  Leaves the output-normed
// hidden state of every token in m->xn.  With d_pos (p == 1), the position
// is read on the device instead, so the launches do not depend on it.
// decode (p == 1) is a generation step, otherwise the tokens are prompt
// tokens.
static int forward(gllm_hip_model* m, int pos0, int p, bool decode, const int* d_pos = nullptr,
                   const uint32_t* d_tok = nullptr) {
    const auto& c = m->cfg;
    hipStream_t s = m->stream;
    const int hd = c.head_dim, kvd = c.n_kv_heads * hd;
    // config.AttentionScale, else float32(1/sqrt(headDim)) (model.go:2685-2688)
    const float scale = m->attn_scale != 0.0f ? m->attn_scale : (float)(1.0 / sqrt((double)hd));
    const size_t norm_lds = (size_t)c.dim * 4;
    GLLM_TRY(launch_weight_rows(m->tok_embd, d_tok ? d_tok : m->d_tokens, p, m->x, s));
    // the residual stream: a norm-fused launch reads X[xi] and writes the
    // updated stream to X[xi ^ 1] (its workgroups all read X[xi] first)
    float* X[2] = {m->x, m->x2};
    int xi = 0;
    const bool fuse = decode && p == 1;
    // addInPlace(x, res) + rmsNormInto(x, norm) + the fused projections:
    // inside the projections' launch when their row kernels take the norm
    // prologue, else the add_rmsnorm kernel first
    auto norm_project = [&](int n, gllm_hip_weight* const* ws, const float* res,
                            const float* norm, float* const* outs) -> int {
        if (fuse && norm_fusable(n, ws)) {
            GLLM_TRY(gemv_norm_f32(n, ws, X[xi], res, norm, c.rms_eps, res ? X[xi ^ 1] : nullptr,
                                   outs, s));
            if (res) xi ^= 1;
            return GLLM_OK;
        }
        hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(p), dim3(256), norm_lds, s, X[xi], res, norm,
                           c.dim, c.rms_eps, m->xn);
        GLLM_HIP(hipGetLastError());
        return project(m, decode, n, ws, m->xn, p, outs);
    };
    const float* pending = nullptr;  // FFN output still to be added to the residual
    for (int l = 0; l < c.n_layers; l++) {
        gllm_hip_weight** W = &m->w[(size_t)l * 7];
        {
            gllm_hip_weight* ws[3] = {W[GLLM_T_WQ], W[GLLM_T_WK], W[GLLM_T_WV]};
            float* outs[3] = {m->q, m->k, m->v};
            GLLM_TRY(norm_project(3, ws, pending, m->d_norms + (size_t)(2 * l) * c.dim, outs));
        }
        if (d_pos) {
            // captured decode step: RoPE and the K/V store run inside the
            // attention scores launch
            GLLM_TRY(attend_exact(m->kv, l, m->q, c.n_heads, c.n_kv_heads, hd, 0, pos0, p, scale,
                                  m->attn, s, m->scores, d_pos, c.max_len, m->d_sin, m->d_cos,
                                  m->k, m->v, (const float*)d_pos + kPosHeader));
        } else {
            const int pairs = std::max(c.n_heads, c.n_kv_heads) * (hd / 2);
            hipLaunchKernelGGL(rope_kv_kernel, dim3(grid1((size_t)pairs, 256), p), dim3(256), 0, s,
                               m->q, m->k, m->v, c.n_heads, c.n_kv_heads, hd, pos0, m->d_sin,
                               m->d_cos, gllm_hip_kv_k_dev(m->kv, l), gllm_hip_kv_v_dev(m->kv, l),
                               d_pos);
            GLLM_HIP(hipGetLastError());
            GLLM_TRY(attend_exact(m->kv, l, m->q, c.n_heads, c.n_kv_heads, hd, 0, pos0, p, scale,
                                  m->attn, s, m->scores, d_pos, c.max_len, nullptr, nullptr,
                                  nullptr, nullptr));
        }
        {
            gllm_hip_weight* ws[1] = {W[GLLM_T_WO]};
            float* outs[1] = {m->proj};
            GLLM_TRY(matvec(m, 1, ws, m->attn, p, outs));
        }
        {
            gllm_hip_weight* ws[2] = {W[GLLM_T_W1], W[GLLM_T_W3]};
            const float* ffn_norm = m->d_norms + (size_t)(2 * l + 1) * c.dim;
            if (fuse && swiglu_epi_ok(ws, W[GLLM_T_W2])) {
                // norm in the gate/up launch, SwiGLU + Q8K in its epilogue
                GLLM_TRY(gemv_norm_swiglu_f32(ws, W[GLLM_T_W2], X[xi], m->proj, ffn_norm, c.rms_eps,
                                              X[xi ^ 1], m->gate, m->up, m->proj, m->act,
                                              m->sq_cnt, s));
                xi ^= 1;
            } else {
                float* outs[2] = {m->gate, m->up};
                GLLM_TRY(norm_project(2, ws, m->proj, ffn_norm, outs));
                GLLM_TRY(gemv_silu_f32(W[GLLM_T_W2], m->gate, m->up, p, m->proj, m->act, m->hidden, s));
            }
        }
        pending = m->proj;
    }
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(p), dim3(256), norm_lds, s, X[xi], pending,
                       m->d_norms + (size_t)(2 * c.n_layers) * c.dim, c.dim, c.rms_eps, m->xn);
    GLLM_HIP(hipGetLastError());
    (void)kvd;
    m->last_p = p;
    return GLLM_OK;
}

// The model takes over w: released with the model.
int model_adopt_weight(gllm_hip_model* m, gllm_hip_weight* w) {
    if (!m || !w) return fail(GLLM_EINVAL, "model_adopt_weight: null argument");
    m->owned.push_back(w);
    return GLLM_OK;
}

void model_set_attn_scale(gllm_hip_model* m, float scale) {
    m->attn_scale = scale;
    drop_decode_graph(m);
}

static bool penalty_on(const gllm_hip_model* m) { return m->penalty != 1.0f && m->window > 0; }

// emitToken's window update (runtime.go:1089-1093)
static void push_recent(gllm_hip_model* m, uint32_t tok) {
    if (m->window <= 0) return;
    if ((int)m->recent.size() == m->window) m->recent.erase(m->recent.begin());
    m->recent.push_back(tok);
}

// The window as the argmax reads it: always `window` ids, so a captured
// decode step stays valid while the window fills.
static int upload_recent(gllm_hip_model* m) {
    if (!penalty_on(m)) return GLLM_OK;
    for (int i = 0; i < m->window; i++)
        m->h_recent[i] = i < (int)m->recent.size() ? m->recent[i] : 0xffffffffu;
    GLLM_HIP(hipMemcpyAsync(m->d_recent, m->h_recent, (size_t)m->window * 4, hipMemcpyHostToDevice,
                            m->stream));
    return GLLM_OK;
}

static int model_argmax(gllm_hip_model* m, uint32_t* d_token) {
    const bool on = penalty_on(m);
    return launch_argmax(m->logits, m->cfg.vocab, d_token, m->argmax_keys, m->stream,
                         on ? m->d_recent : nullptr, on ? m->window : 0, m->penalty);
}

// One greedy decode step on the token in d_tokens[0]: forward, the output
// projection (full logits), then the (penalised) argmax into d_tokens[1]:
// in the projection's launch when its kernel allows (argmax_epilogue),
// otherwise as two more launches.
static int decode_step(gllm_hip_model* m, int pos, const int* d_pos) {
    // the token rides in the position buffer's header (word 1): one upload
    GLLM_TRY(forward(m, pos, 1, true, d_pos, (const uint32_t*)m->d_pos + 1));
    if (m->head_keys && argmax_fusable(m->output) &&
        argmax_epilogue_keys(m->output) <= (size_t)m->cfg.vocab / 8 + 8) {
        const bool on = penalty_on(m);
        return gemv_argmax_f32(m->output, m->xn, m->logits, m->head_keys, m->d_tokens + 1,
                               on ? m->d_recent : nullptr, on ? m->window : 0, m->penalty,
                               m->stream);
    }
    gllm_hip_weight* ws[1] = {m->output};
    float* outs[1] = {m->logits};
    GLLM_TRY(matvec(m, 1, ws, m->xn, 1, outs));
    return model_argmax(m, m->d_tokens + 1);
}

// Every weight set, of a type this path runs: any Weight.RowInto type for
// the embedding, a row-kernel type for the projections; a generation step
// (decode) also needs each layer's fused groups to be ones this path
// restates (group_routing refuses same-type groups of a format whose float
// kernel is not restated).
static int check_ready(const gllm_hip_model* m, bool decode) {
    if (!m) return fail(GLLM_EINVAL, "null model");
    if (!m->tok_embd || !m->output) return fail(GLLM_EINVAL, "model: embedding/output not set");
    if (!rows_type(m->tok_embd->type))
        return fail(GLLM_EUNSUP, "model: embedding type %d has no row lookup", m->tok_embd->type);
    if (!row_kernel_type(m->output->type))
        return fail(GLLM_EUNSUP, "model: output type %d has no row kernel", m->output->type);
    for (size_t i = 0; i < m->w.size(); i++) {
        if (!m->w[i]) return fail(GLLM_EINVAL, "model: layer %zu slot %zu not set", i / 7, i % 7);
        if (!row_kernel_type(m->w[i]->type))
            return fail(GLLM_EUNSUP, "model: layer %zu slot %zu has type %d (no row kernel)",
                        i / 7, i % 7, m->w[i]->type);
    }
    if (decode) {
        int fl[3];
        for (int l = 0; l < m->cfg.n_layers; l++) {
            gllm_hip_weight* const* W = &m->w[(size_t)l * 7];
            gllm_hip_weight* qkv[3] = {W[GLLM_T_WQ], W[GLLM_T_WK], W[GLLM_T_WV]};
            gllm_hip_weight* gu[2] = {W[GLLM_T_W1], W[GLLM_T_W3]};
            GLLM_TRY(group_routing(3, qkv, fl));
            GLLM_TRY(group_routing(2, gu, fl));
        }
    }
    return GLLM_OK;
}

}  // namespace gllm

using namespace gllm;

extern "C" {

gllm_hip_model* gllm_hip_model_new(const gllm_hip_model_config* cfg) {
    if (!cfg || cfg->n_layers <= 0 || cfg->dim <= 0 || cfg->dim % 256 || cfg->hidden % 256 ||
        cfg->dim > 4 * 256 * kNormVec ||
        cfg->n_heads <= 0 || cfg->n_kv_heads <= 0 || cfg->n_heads % cfg->n_kv_heads ||
        cfg->head_dim % 8 || cfg->head_dim > 128 || cfg->n_heads / cfg->n_kv_heads > 8 ||
        cfg->n_heads * cfg->head_dim % 256 || cfg->vocab <= 0 || cfg->max_len <= 0) {
        fail(GLLM_EINVAL, "gllm_hip_model_new: unsupported config");
        return nullptr;
    }
    gllm_hip_model* m = new gllm_hip_model();
    m->cfg = *cfg;
    m->w.assign((size_t)cfg->n_layers * 7, nullptr);
    auto bail = [&](const char* what) -> gllm_hip_model* {
        (void)hipGetLastError();
        fail(GLLM_ENOMEM, "gllm_hip_model_new: %s", what);
        gllm_hip_model_release(m);
        return nullptr;
    };
    if (hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess) return bail("stream");
    const size_t nn = (size_t)(2 * cfg->n_layers + 1) * cfg->dim;
    if (hipMalloc(&m->d_norms, nn * 4) != hipSuccess) return bail("norms");
    // RoPE tables (buildRopeInvFreq model.go:1728-1756, prepareRopeScratch
    // model.go:3020-3049), computed on the host with the reference's
    // float64 pow / sin / cos and uploaded once for every position.
    const int pairs = cfg->head_dim / 2;
    std::vector<float> sn((size_t)cfg->max_len * pairs), cs((size_t)cfg->max_len * pairs);
    for (int pos = 0; pos < cfg->max_len; pos++)
        rope_row(*cfg, pos, &sn[(size_t)pos * pairs], &cs[(size_t)pos * pairs]);
    if (hipMalloc(&m->d_sin, sn.size() * 4) != hipSuccess) return bail("rope tables");
    if (hipMalloc(&m->d_cos, cs.size() * 4) != hipSuccess) return bail("rope tables");
    if (hipMemcpy(m->d_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(m->d_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
        return bail("rope upload");
    const int kvd = cfg->n_kv_heads * cfg->head_dim;
    m->kv = gllm_hip_kv_new(cfg->n_layers, kvd, kvd, cfg->max_len);
    if (!m->kv) return bail("kv cache");
    if (ensure_buffers(m, 1) != GLLM_OK) return bail("activation buffers");
    if (hipMalloc(&m->logits, (size_t)cfg->vocab * 4) != hipSuccess) return bail("logits");
    if (hipMalloc(&m->sq_cnt, (size_t)(cfg->hidden / 256) * 4) != hipSuccess ||
        hipMemset(m->sq_cnt, 0, (size_t)(cfg->hidden / 256) * 4) != hipSuccess)
        return bail("SwiGLU counters");
    if (hipMalloc(&m->argmax_keys, argmax_keys(cfg->vocab) * 8) != hipSuccess)
        return bail("argmax keys");
    // one key per workgroup of the head's launch: ceil(vocab / (32 / G)) for
    // G in {1, 2, 4}, at most vocab / 8 + 1
    if (hipMalloc(&m->head_keys, ((size_t)cfg->vocab / 8 + 8) * 8) != hipSuccess)
        return bail("head argmax keys");
    if (hipMalloc(&m->d_pos, pos_bytes(*cfg)) != hipSuccess) return bail("position");
    if (hipHostMalloc(&m->h_pos, pos_bytes(*cfg), hipHostMallocDefault) != hipSuccess)
        return bail("position");
    return m;
}

void gllm_hip_model_release(gllm_hip_model* m) {
    if (!m) return;
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    float* bufs[] = {m->x, m->xn, m->q, m->k, m->v, m->attn, m->proj, m->gate, m->up, m->hidden,
                     m->logits, m->d_norms, m->d_sin, m->d_cos, m->x2};
    for (float* b : bufs)
        if (b) (void)hipFree(b);
    if (m->d_tokens) (void)hipFree(m->d_tokens);
    if (m->h_tokens) (void)hipHostFree(m->h_tokens);
    if (m->act) (void)hipFree(m->act);
    if (m->argmax_keys) (void)hipFree(m->argmax_keys);
    if (m->head_keys) (void)hipFree(m->head_keys);
    drop_decode_graph(m);
    if (m->scores) (void)hipFree(m->scores);
    if (m->d_pos) (void)hipFree(m->d_pos);
    if (m->sq_cnt) (void)hipFree(m->sq_cnt);
    if (m->h_pos) (void)hipHostFree(m->h_pos);
    if (m->kv) gllm_hip_kv_release(m->kv);
    if (m->d_recent) (void)hipFree(m->d_recent);
    if (m->h_recent) (void)hipHostFree(m->h_recent);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    for (gllm_hip_weight* w : m->owned) gllm_hip_weight_release(w);
    delete m;
}

int gllm_hip_model_set_weight(gllm_hip_model* m, int layer, int slot, gllm_hip_weight* w) {
    if (!m || !w) return fail(GLLM_EINVAL, "gllm_hip_model_set_weight: null argument");
    drop_decode_graph(m);
    const auto& c = m->cfg;
    const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
    int rows = 0, cols = 0;
    switch (slot) {
    case GLLM_T_WQ: rows = qd; cols = c.dim; break;
    case GLLM_T_WK: case GLLM_T_WV: rows = kvd; cols = c.dim; break;
    case GLLM_T_WO: rows = c.dim; cols = qd; break;
    case GLLM_T_W1: case GLLM_T_W3: rows = c.hidden; cols = c.dim; break;
    case GLLM_T_W2: rows = c.dim; cols = c.hidden; break;
    case GLLM_T_TOK_EMBD: case GLLM_T_OUTPUT: rows = c.vocab; cols = c.dim; break;
    default: return fail(GLLM_EINVAL, "gllm_hip_model_set_weight: slot %d", slot);
    }
    if (w->rows != rows || w->cols != cols)
        return fail(GLLM_EINVAL, "slot %d expects %dx%d, got %dx%d", slot, rows, cols, w->rows, w->cols);
    if (slot == GLLM_T_TOK_EMBD) {
        m->tok_embd = w;
        return GLLM_OK;
    }
    if (slot == GLLM_T_OUTPUT) {
        m->output = w;
        return GLLM_OK;
    }
    if (layer < 0 || layer >= c.n_layers) return fail(GLLM_EINVAL, "layer %d out of range", layer);
    m->w[(size_t)layer * 7 + slot] = w;
    return GLLM_OK;
}

int gllm_hip_model_set_norm(gllm_hip_model* m, int layer, int slot, const float* w) {
    if (!m || !w) return fail(GLLM_EINVAL, "gllm_hip_model_set_norm: null argument");
    const auto& c = m->cfg;
    size_t idx;
    if (slot == GLLM_T_OUT_NORM) idx = 2 * (size_t)c.n_layers;
    else if ((slot == GLLM_T_ATTN_NORM || slot == GLLM_T_FFN_NORM) && layer >= 0 && layer < c.n_layers)
        idx = 2 * (size_t)layer + (slot == GLLM_T_FFN_NORM);
    else return fail(GLLM_EINVAL, "gllm_hip_model_set_norm: slot %d layer %d", slot, layer);
    GLLM_HIP(hipMemcpy(m->d_norms + idx * c.dim, w, (size_t)c.dim * 4, hipMemcpyHostToDevice));
    return GLLM_OK;
}

int gllm_hip_model_decode(gllm_hip_model* m, uint32_t token, int pos, uint32_t* next) {
    GLLM_TRY(check_ready(m, true));
    if (!next) return fail(GLLM_EINVAL, "gllm_hip_model_decode: null next");
    if (pos < 0 || pos >= m->cfg.max_len) return fail(GLLM_EINVAL, "position %d out of range", pos);
    if (token >= (uint32_t)m->cfg.vocab) return fail(GLLM_EINVAL, "token %u out of range", token);
    hipStream_t s = m->stream;
    push_recent(m, token);
    GLLM_TRY(upload_recent(m));
    // header: position, token; then the position's RoPE rows
    m->h_pos[0] = pos;
    m->h_pos[1] = (int)token;
    {
        float* rows = (float*)m->h_pos + kPosHeader;
        rope_row(m->cfg, pos, rows, rows + m->cfg.head_dim / 2);
    }
    GLLM_HIP(hipMemcpyAsync(m->d_pos, m->h_pos, pos_bytes(m->cfg), hipMemcpyHostToDevice, s));
    if (m->decode_graph) {
        GLLM_HIP(hipGraphLaunch(m->decode_graph, s));
    } else {
        // The first step runs eagerly (and leaves every buffer it needs
        // allocated); the same launches, reading the position on the device,
        // are then captured and replayed for every later step.
        GLLM_TRY(decode_step(m, pos, nullptr));
        const auto& c = m->cfg;
        if (attend_exact_graphable(m->kv, c.n_heads, c.n_kv_heads, c.head_dim, c.max_len)) {
            hipGraph_t g = nullptr;
            GLLM_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
            const int rc = decode_step(m, 0, m->d_pos);
            const hipError_t ec = hipStreamEndCapture(s, &g);
            if (rc != GLLM_OK) {
                if (g) (void)hipGraphDestroy(g);
                return rc;
            }
            GLLM_HIP(ec);
            const hipError_t ei = hipGraphInstantiate(&m->decode_graph, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            if (ei != hipSuccess) m->decode_graph = nullptr;
            GLLM_HIP(ei);
        }
    }
    GLLM_HIP(hipMemcpyAsync(m->h_tokens + 1, m->d_tokens + 1, 4, hipMemcpyDeviceToHost, s));
    GLLM_HIP(hipStreamSynchronize(s));
    *next = m->h_tokens[1];
    return GLLM_OK;
}

int gllm_hip_model_prefill(gllm_hip_model* m, const uint32_t* tokens, int n, int start_pos,
                           uint32_t* first, float* logits) {
    GLLM_TRY(check_ready(m, false));
    if (!tokens || n <= 0 || !first) return fail(GLLM_EINVAL, "gllm_hip_model_prefill: bad arguments");
    if (start_pos < 0 || start_pos + n > m->cfg.max_len)
        return fail(GLLM_EINVAL, "prefill positions %d..%d exceed max_len", start_pos, start_pos + n - 1);
    for (int i = 0; i < n; i++)
        if (tokens[i] >= (uint32_t)m->cfg.vocab) return fail(GLLM_EINVAL, "token %u out of range", tokens[i]);
    // up to 512 prompt tokens per forward: the batched matrix-core products
    // need many token tiles to fill the GPU; the score buffer
    // (tokens x heads x max_len floats) is kept under 1 GiB
    const size_t per_tok = (size_t)m->cfg.n_heads * m->cfg.max_len * 4;
    const int chunk = (int)std::max<size_t>(64, std::min<size_t>(512, ((size_t)1 << 30) / per_tok));
    GLLM_TRY(ensure_buffers(m, std::min(n, chunk)));
    hipStream_t s = m->stream;
    // a prefill from position 0 starts a request: its window is the tail of
    // this prompt (recentTokenWindowInto, runtime.go:1035), not the previous
    // request's tokens; a later start continues the same request's window
    if (start_pos == 0) m->recent.clear();
    for (int i = 0; i < n; i++) push_recent(m, tokens[i]);
    GLLM_TRY(upload_recent(m));
    for (int c0 = 0; c0 < n; c0 += chunk) {
        const int p = std::min(chunk, n - c0);
        memcpy(m->h_tokens, tokens + c0, (size_t)p * 4);
        GLLM_HIP(hipMemcpyAsync(m->d_tokens, m->h_tokens, (size_t)p * 4, hipMemcpyHostToDevice, s));
        GLLM_TRY(forward(m, start_pos + c0, p, false));
        // h_tokens is reused by the next chunk's copy
        GLLM_HIP(hipStreamSynchronize(s));
    }
    // computeLast: full logits of the last position (MatvecQ6KInto), then
    // argmaxFiniteToken.
    const float* last = m->xn + (size_t)(m->last_p - 1) * m->cfg.dim;
    {
        gllm_hip_weight* ws[1] = {m->output};
        float* outs[1] = {m->logits};
        GLLM_TRY(matvec(m, 1, ws, last, 1, outs));
    }
    if (logits)  // the projection, before the penalty
        GLLM_HIP(hipMemcpyAsync(logits, m->logits, (size_t)m->cfg.vocab * 4, hipMemcpyDeviceToHost, s));
    GLLM_TRY(model_argmax(m, m->d_tokens + m->max_p));
    GLLM_HIP(hipMemcpyAsync(m->h_tokens + m->max_p, m->d_tokens + m->max_p, 4, hipMemcpyDeviceToHost, s));
    GLLM_HIP(hipStreamSynchronize(s));
    *first = m->h_tokens[m->max_p];
    // keep the last token's hidden state where gllm_hip_model_hidden reads it
    GLLM_HIP(hipMemcpyAsync(m->xn, last, (size_t)m->cfg.dim * 4, hipMemcpyDeviceToDevice, s));
    GLLM_HIP(hipStreamSynchronize(s));
    m->last_p = 1;
    return GLLM_OK;
}

int gllm_hip_model_hidden(gllm_hip_model* m, float* out) {
    if (!m || !out) return fail(GLLM_EINVAL, "gllm_hip_model_hidden: null argument");
    const float* last = m->xn + (size_t)(std::max(1, m->last_p) - 1) * m->cfg.dim;
    GLLM_HIP(hipMemcpyAsync(out, last, (size_t)m->cfg.dim * 4, hipMemcpyDeviceToHost, m->stream));
    GLLM_HIP(hipStreamSynchronize(m->stream));
    return GLLM_OK;
}

int gllm_hip_model_set_repeat_penalty(gllm_hip_model* m, float penalty, int window) {
    if (!m) return fail(GLLM_EINVAL, "gllm_hip_model_set_repeat_penalty: null model");
    if (!(penalty > 0.0f) || penalty == INFINITY)
        return fail(GLLM_EINVAL, "repeat penalty must be finite and positive");
    if (window < 0 || window > kMaxRepeatWindow)
        return fail(GLLM_EINVAL, "repeat window %d outside 0..%d", window, kMaxRepeatWindow);
    GLLM_HIP(hipStreamSynchronize(m->stream));
    if (m->d_recent) (void)hipFree(m->d_recent);
    if (m->h_recent) (void)hipHostFree(m->h_recent);
    m->d_recent = nullptr;
    m->h_recent = nullptr;
    m->recent.clear();
    m->penalty = 1.0f;
    m->window = 0;
    drop_decode_graph(m);  // it captured the old window arguments
    if (window > 0) {
        GLLM_HIP(hipMalloc(&m->d_recent, (size_t)window * 4));
        GLLM_HIP(hipHostMalloc(&m->h_recent, (size_t)window * 4, hipHostMallocDefault));
    }
    m->penalty = penalty;
    m->window = window;
    return GLLM_OK;
}

gllm_hip_kv* gllm_hip_model_kv(gllm_hip_model* m) { return m ? m->kv : nullptr; }

}  // extern "C"
