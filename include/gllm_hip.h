/*
 * gllm_hip.h -- C ABI of the MI355X (gfx950) quantized-matvec and
 * F16-KV decode-attention path of GopherLLM.
 *
 * The Go engine reaches these through cgo exactly as it reaches its Metal
 * backend today (internal/metal/metal_darwin.go:557-1001): weights are
 * uploaded once at load time and kept as opaque handles on the Weight struct
 * (model.go:2454), every dispatch site tries the device first and falls back
 * to the CPU kernel when the call reports failure (model.go:700-725).
 *
 * Conventions
 *  - Plain C types only; no torch or HIP types.  `stream` arguments are a
 *    hipStream_t passed as void* (NULL = the legacy default stream).
 *  - Every int-returning call returns GLLM_OK (0) on success and a negative
 *    GLLM_E* code on failure, having written nothing to the outputs;
 *    gllm_hip_last_error() then describes the failure (per calling thread).
 *  - "host" entry points take host pointers and block until the result is in
 *    the caller's buffer (the Metal seam's waitUntilCompleted contract);
 *    "_dev" entry points take device pointers and only enqueue on `stream`.
 *  - Shapes follow the reference: cols % 256 == 0 for the Q8K row kernels
 *    (simd.go:264), weights are row-major GGUF tensors with rows = dims[1],
 *    cols = dims[0] (model.go:2393-2396).
 *  - Thread safety: handles may be used from several host threads at once;
 *    host entry points use per-thread streams.  Device scratch (quantised
 *    activations, logits, attention partials) is kept per (host thread,
 *    stream), so two streams driven from one thread never share it.
 *    A KV cache or model handle must not be mutated by two threads at once
 *    (the reference serialises requests per Runner, runtime.go:816-817).
 *  - Graph capture: a "_dev" call may be captured into a caller's HIP graph
 *    once the same call (same shapes, same stream) has run uncaptured: the
 *    scratch it uses then exists, and it stays allocated for the process
 *    lifetime even after a later, larger call on that stream moves to a
 *    bigger buffer.  A call that would have to allocate scratch while its
 *    stream is capturing fails with GLLM_EUNSUP and enqueues nothing.
 *  - Start-up check: before the first weight is created on a device (and in
 *    gllm_hip_available) the library runs a known-answer check of the Q4_K,
 *    Q6_K and Q8_0 matvec path (q8kSelfCheck, q8k_dot_arm64.go:146-228).  On
 *    a mismatch gllm_hip_available() returns 0 and every weight constructor
 *    fails with GLLM_EUNSUP, so the caller keeps its CPU kernels.
 */
#ifndef GLLM_HIP_H
#define GLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML tensor types (gguf.go:27-60).  Every type below except F32, F16 and
 * BF16 has row kernels; F32 / F16 / BF16 weights hold rows for
 * gllm_hip_weight_rows_dev only (token embeddings). */
#define GLLM_TYPE_F32 0
#define GLLM_TYPE_F16 1
#define GLLM_TYPE_BF16 30
#define GLLM_TYPE_Q4_0 2
#define GLLM_TYPE_Q4_1 3
#define GLLM_TYPE_Q8_0 8
#define GLLM_TYPE_Q2_K 10
#define GLLM_TYPE_Q3_K 11
#define GLLM_TYPE_Q4_K 12
#define GLLM_TYPE_Q5_K 13
#define GLLM_TYPE_Q6_K 14
#define GLLM_TYPE_MXFP4 39

#define GLLM_OK 0
#define GLLM_EINVAL (-1)   /* bad argument or shape */
#define GLLM_EDEVICE (-2)  /* HIP runtime error */
#define GLLM_ENOMEM (-3)   /* device allocation failed */
#define GLLM_EUNSUP (-4)   /* type or shape not supported by this path */

/* ---------------------------------------------------------------------- */
/* Runtime                                                                 */
/* ---------------------------------------------------------------------- */

/* 1 when a gfx950 device is usable (replaces gllm_metal_available,
 * internal/metal/metal_darwin.go:396). */
int gllm_hip_available(void);
/* Message of the last failure on the calling thread (replaces
 * gllm_metal_last_error, internal/metal/metal_darwin.go:400). */
const char* gllm_hip_last_error(void);
/* Select the device used by handles created afterwards on this thread. */
int gllm_hip_set_device(int device);
/* Library version string, for logs. */
const char* gllm_hip_version(void);
/* The caller will enqueue no more work on `stream` (a hipStream_t; null is
 * the legacy default stream): the calling thread's scratch buffers for that
 * stream on the current device are freed once the stream drains, except
 * those handed out while the stream was being captured (a captured graph
 * may still be replayed; they stay allocated).  No counterpart in the
 * reference, whose CPU kernels have no streams; for callers that create and
 * destroy many streams, so that their scratch does not accumulate. */
int gllm_hip_stream_release(void* stream);

/* ---------------------------------------------------------------------- */
/* Weights (prepareMetalWeight, model.go:2454; gllm_metal_new_q4k,         */
/* internal/metal/metal_darwin.go:557)                                     */
/* ---------------------------------------------------------------------- */

typedef struct gllm_hip_weight gllm_hip_weight;

/* Upload `len` bytes of a GGUF tensor (rows x cols of ggml_type) from host
 * memory; the host bytes may be released after the call.  Q6_K and Q8_0 rows
 * are repacked once into 16-byte aligned blocks (same size, same values). */
gllm_hip_weight* gllm_hip_weight_new(const void* data, size_t len, int ggml_type, int rows,
                                     int cols);
/* Same, from bytes already in device memory (copied, then repacked). */
gllm_hip_weight* gllm_hip_weight_from_device(const void* d_data, size_t len, int ggml_type,
                                             int rows, int cols, void* stream);
/* replaces gllm_metal_release_weight (internal/metal/metal_darwin.go:1001) */
void gllm_hip_weight_release(gllm_hip_weight* w);
int gllm_hip_weight_shape(const gllm_hip_weight* w, int* ggml_type, int* rows, int* cols);
/* Weight.RowInto (model.go:1034-1100, raw_scalar.go:130-161): out[i][0..cols)
 * = row d_rows[i] dequantised (DequantRow*Into of the weight's type, or the
 * F32 / F16 / BF16 values) for i < n, device pointers, enqueued on stream.
 * Ids must be < rows (an id past the end reads the last row). */
int gllm_hip_weight_rows_dev(const gllm_hip_weight* w, const uint32_t* d_rows, int n,
                             float* d_out, void* stream);
/* Device bytes of the weight in the reference's GGUF layout (undoing the
 * repack); dst is a device buffer of rows*row_bytes. */
int gllm_hip_weight_download_dev(const gllm_hip_weight* w, void* d_dst, void* stream);

/* ---------------------------------------------------------------------- */
/* Matvec (Weight.MatvecInto model.go:670; MatvecQ4KInto simd.go:261,      */
/* MatvecQ6KInto simd.go:413, MatvecQ8_0Into simd.go:204)                  */
/* ---------------------------------------------------------------------- */

/* out[r] = W[r,:] . x.  x: cols floats, out: rows floats.  Quantises x to
 * Q8K (q8kQuantize) and folds the exact-float xsums term, reproducing the
 * reference's amd64 row kernels bit for bit.  (gllm_metal_q4k_matvec,
 * internal/metal/metal_darwin.go:740) */
int gllm_hip_matvec(gllm_hip_weight* w, const float* x, float* out);
/* Two / three weights sharing one activation vector, routed as the
 * reference routes a decode step's fused groups (tryMatvec2Into
 * model.go:3186-3206 for two, tryMatvecAttentionInto model.go:3157-3184 for
 * three): same-type Q4_K or Q6_K groups and Q4_K/Q4_K/Q6_K run the int8 row
 * dots (MatvecQ4K2IntoWithXSums simd.go:295, Q4KMatvec3IntoWithXSums
 * metal.go:14, MatvecQ4K2Q6KIntoWithXSums simd.go:331, MatvecQ6K2Into /
 * MatvecQ6K3Into simd.go:443/483); a same-type pair or triple of Q8_0, Q4_0,
 * Q4_1, Q2_K, Q3_K, Q5_K or MXFP4 runs the float kernels
 * (matvecSameType2/3Into model.go:3213-3256: DotQ8_0F32, DotQ4_0F32,
 * DotQ4_1F32, DotQ2KF32, DotQ3KF32, DotQ5KF32, DotMXFP4F32); a weight
 * outside a fused pair runs its own int8 row dot. */
int gllm_hip_matvec2(gllm_hip_weight* a, gllm_hip_weight* b, const float* x, float* out_a,
                     float* out_b);
int gllm_hip_matvec3(gllm_hip_weight* a, gllm_hip_weight* b, gllm_hip_weight* c,
                     const float* x, float* out_a, float* out_b, float* out_c);
/* p activation rows xs[p][cols] -> outs[p][rows] (matvecBatchQ8,
 * kernels_amd64.go:470); per-row results equal p separate matvecs. */
int gllm_hip_matvec_batch(gllm_hip_weight* w, const float* xs, int p, float* outs);
/* Greedy token: argmax over finite W.x, lowest row on ties
 * (Weight.ArgmaxMatvec model.go:754 -> argmaxQ6KRowsQ8 kernels_amd64.go:294). */
int gllm_hip_argmax(gllm_hip_weight* w, const float* x, uint32_t* token);
/* The same after the repeat penalty (applyRepeatPenalty sampling.go:136-153,
 * as argmaxOutputTokenPenalizedInto model.go:2574-2610 and
 * ArgmaxQ6KPenalized internal/metal/metal_darwin.go:1175-1190 apply it; Metal
 * caps the window at 64 ids, this call takes any length): each of the
 * n_recent ids (duplicates count again, ids >= rows are ignored) divides a
 * positive logit by penalty and multiplies any other by it; non-finite
 * logits drop out.  penalty must be finite and > 0 (GLLM_EINVAL otherwise);
 * penalty 1 is the plain argmax. */
int gllm_hip_argmax_penalized(gllm_hip_weight* w, const float* x, const uint32_t* recent,
                              int n_recent, float penalty, uint32_t* token);

/* Device-pointer forms.  d_xs: p rows of cols floats (row stride cols);
 * d_outs: p rows of out_stride floats (out_stride >= rows). */
int gllm_hip_matvec_dev(gllm_hip_weight* w, const float* d_xs, int p, float* d_outs,
                        int out_stride, void* stream);
/* n weights (same cols) against the same activations; one quantisation of
 * x is shared by the int8 row kernels, runs of one type are one launch.
 * Batches (p > 1) take any mix of the int8 formats (matvecBatch2/3 ->
 * matvecBatchQ8 per weight, forward_batch.go:108-233); batch 1 with n > 1
 * is a fused group, routed as gllm_hip_matvec2 / gllm_hip_matvec3 route it. */
int gllm_hip_matvec_multi_dev(int n, gllm_hip_weight* const* ws, const float* d_xs, int p,
                              float* const* d_outs, const int* out_strides, void* stream);
/* A generation step's SwiGLU FFN (ForwardBodyInto model.go:2780-2800, the
 * path matvecMetalSwiGLUInto metal_darwin.go:161 fuses on Apple GPUs):
 * gate, up = the fused group of tryMatvec2Into (routed as gllm_hip_matvec2),
 * hidden = siluMulF32(gate, up) (kernels_amd64.go:711), d_out =
 * down.MatvecInto(hidden).  Batch 1, device pointers, enqueued on stream;
 * gate / up / hidden live in library scratch of the calling thread. */
int gllm_hip_swiglu_down_dev(gllm_hip_weight* gate, gllm_hip_weight* up, gllm_hip_weight* down,
                             const float* d_x, float* d_out, void* stream);
int gllm_hip_argmax_dev(gllm_hip_weight* w, const float* d_x, uint32_t* d_token, void* stream);
/* d_recent: n_recent device token ids. */
int gllm_hip_argmax_penalized_dev(gllm_hip_weight* w, const float* d_x, const uint32_t* d_recent,
                                  int n_recent, float penalty, uint32_t* d_token, void* stream);

/* gllm_hip_matvec_dev for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, results and
 * errors as gllm_hip_matvec_dev; the quantised activations go to a fixed
 * 4 MiB buffer in the library's device image (one per GPU, held until the
 * process ends) instead of allocated scratch, so the call allocates
 * nothing.  GLLM_EINVAL when gllm_hip_act_bytes(cols, p) exceeds 4 MiB.
 * Every call on one GPU shares that buffer: calls that overlap on one GPU
 * (other streams or host threads) race, and callers serialise them. */
int gllm_hip_matvec_dev_noalloc(gllm_hip_weight* w, const float* d_xs, int p, float* d_outs,
                                int out_stride, void* stream);

/* Split form of the same call, for callers that quantise once and dot many
 * matrices (acquireQ8 + fillQ4KXSums/fillQ6KXSums16, kernels_amd64.go:246,
 * then dotQ4KRowsQ8 / dotQ6KRowsQ8 / dotQ8_0RowsQ8, kernels_amd64.go:268-285,
 * 611-619).  d_act is a caller-owned device buffer of
 * gllm_hip_act_bytes(cols, p) bytes holding the quantised activations. */
size_t gllm_hip_act_bytes(int cols, int p);
int gllm_hip_q8k_prepare_dev(const float* d_xs, int cols, int p, void* d_act, void* stream);
int gllm_hip_matvec_q8_dev(gllm_hip_weight* w, const void* d_act, int p, float* d_outs,
                           int out_stride, void* stream);

/* Q8K activation quantisation alone (q8kQuantize, kernels_amd64.s:348-436):
 * p rows of cols floats -> q8 [p][cols] in element order and scales
 * [p][cols/256]. */
int gllm_hip_q8k_quantize_dev(const float* d_x, int cols, int p, int8_t* d_q8,
                              float* d_scales, void* stream);
/* Debug: the exact integer lane sums of every (row, block): d_ints holds
 * rows*(cols/256)*8 int32 (ref: the int32 lanes of q4kDotQ8KRow /
 * q6kDotQ8KRow / q8_0DotQ8KRow). */
int gllm_hip_lane_ints_dev(gllm_hip_weight* w, const float* d_x, int32_t* d_ints,
                           void* stream);

/* ---------------------------------------------------------------------- */
/* RTN encoders (QuantizeRowQ4K quantize_rtn.go:128, QuantizeRowQ6K :331,  */
/* QuantizeRowQ8_0 :35) run on the device: d_src rows x cols floats ->     */
/* d_dst in the reference's GGUF layout.                                   */
/* ---------------------------------------------------------------------- */
int gllm_hip_quantize_rows_dev(int ggml_type, const float* d_src, int rows, int cols,
                               void* d_dst, void* stream);
/* Deterministic synthetic data: n floats ~ N(0, std^2) from (seed, stream
 * id), counter based; used to build the benchmark models on the device. */
int gllm_hip_fill_normal_dev(float* d_out, size_t n, uint64_t seed, float std, void* stream);

/* ---------------------------------------------------------------------- */
/* F16 KV cache and GQA decode attention (KVCache model.go:1321,           */
/* NewKVCacheF16 :1396, storeKV :1466, attendHeadGroup :1516)              */
/* ---------------------------------------------------------------------- */

typedef struct gllm_hip_kv gllm_hip_kv;

#define GLLM_ATTN_EXACT 0   /* two-pass, the reference's float order */
#define GLLM_ATTN_SPLITK 1  /* split-K online softmax, tolerance-level */

gllm_hip_kv* gllm_hip_kv_new(int layers, int kv_dim_k, int kv_dim_v, int max_len);
void gllm_hip_kv_release(gllm_hip_kv* kv);
/* Device pointer of layer l's K (or V) rows: [max_len][kv_dim] uint16. */
uint16_t* gllm_hip_kv_k_dev(gllm_hip_kv* kv, int l);
uint16_t* gllm_hip_kv_v_dev(gllm_hip_kv* kv, int l);
/* Copy n positions starting at pos0 of layer l to host (f16 bits); either
 * output may be NULL.  (The rows a prefix cache would copy, runtime.go:1334.) */
int gllm_hip_kv_read(gllm_hip_kv* kv, int l, int pos0, int n, uint16_t* k_out, uint16_t* v_out);
/* storeKV: round k, v (host floats) to f16 RNE at position pos. */
int gllm_hip_kv_store(gllm_hip_kv* kv, int l, int pos, const float* k, const float* v);
int gllm_hip_kv_store_dev(gllm_hip_kv* kv, int l, int pos, const float* d_k,
                          const float* d_v, void* stream);
/* attendHeadGroup: q_heads query heads sharing kv head kvh, positions
 * start..end inclusive; out (q_heads*vd floats) is overwritten.  softcap
 * must be 0 (the llama graph). */
int gllm_hip_attend_group(gllm_hip_kv* kv, int l, int kvh, const float* q, int q_heads,
                          int hd, int vd, int start, int end, float scale, float softcap,
                          float* out);
/* All heads of one decode position: d_q [n_heads][hd] -> d_out [n_heads][hd];
 * head h reads kv head h / (n_heads / n_kv_heads). */
int gllm_hip_attend_dev(gllm_hip_kv* kv, int l, const float* d_q, int n_heads, int n_kv_heads,
                        int hd, int start, int end, float scale, int mode, float* d_out,
                        void* stream);

/* ---------------------------------------------------------------------- */
/* Resident llama decoder (ForwardBodyInto model.go:2622,                  */
/* ForwardBatchInto forward_batch.go:316, forwardGreedyToken               */
/* runtime.go:1607)                                                        */
/* ---------------------------------------------------------------------- */

typedef struct gllm_hip_model gllm_hip_model;

typedef struct gllm_hip_model_config {
    int n_layers, dim, hidden, n_heads, n_kv_heads, head_dim, vocab, max_len;
    float rms_eps, rope_theta;
} gllm_hip_model_config;

/* Tensor slots for gllm_hip_model_set_weight / _set_norm. */
#define GLLM_T_WQ 0
#define GLLM_T_WK 1
#define GLLM_T_WV 2
#define GLLM_T_WO 3
#define GLLM_T_W1 4   /* ffn gate */
#define GLLM_T_W2 5   /* ffn down */
#define GLLM_T_W3 6   /* ffn up */
#define GLLM_T_TOK_EMBD 7
#define GLLM_T_OUTPUT 8
#define GLLM_T_ATTN_NORM 9
#define GLLM_T_FFN_NORM 10
#define GLLM_T_OUT_NORM 11

gllm_hip_model* gllm_hip_model_new(const gllm_hip_model_config* cfg);
void gllm_hip_model_release(gllm_hip_model* m);
/* The model borrows the weight handle; it must outlive the model. */
int gllm_hip_model_set_weight(gllm_hip_model* m, int layer, int slot, gllm_hip_weight* w);
/* RMSNorm weights, dim host floats (copied). */
int gllm_hip_model_set_norm(gllm_hip_model* m, int layer, int slot, const float* w);
/* One decode step at position pos; *next = greedy token. */
int gllm_hip_model_decode(gllm_hip_model* m, uint32_t token, int pos, uint32_t* next);
/* Prefill n tokens from start_pos; *first = greedy token from the last
 * position's logits; logits (vocab host floats, the projection before any
 * repeat penalty) may be NULL. */
int gllm_hip_model_prefill(gllm_hip_model* m, const uint32_t* tokens, int n, int start_pos,
                           uint32_t* first, float* logits);
/* Repeat penalty for the greedy choices of prefill and decode
 * (forwardGreedyToken runtime.go:1607 with recent / repeatPenalty): the
 * window holds the last `window` tokens the model has been given (prefill
 * tokens in order, then each decode step's input token, as
 * recentTokenWindowInto runtime.go:1225 and emitToken runtime.go:1089-1093
 * keep it; the reference's window is 64), and every choice applies
 * applyRepeatPenalty (sampling.go:136-153) to the logits before the finite
 * argmax.  penalty must be finite and > 0, window 0..4096; penalty 1 or
 * window 0 turn it off.  Clears the window. */
int gllm_hip_model_set_repeat_penalty(gllm_hip_model* m, float penalty, int window);
/* Normed final hidden state of the last step (dim host floats). */
int gllm_hip_model_hidden(gllm_hip_model* m, float* out);
gllm_hip_kv* gllm_hip_model_kv(gllm_hip_model* m);

/* ---------------------------------------------------------------------- */
/* GGUF files (ParseGGUF gguf.go:493-568, OpenMmap mmap.go:11-14,          */
/* loadWeight model.go:2357-2476, LoadModel model.go:1872-1930)            */
/* ---------------------------------------------------------------------- */

typedef struct gllm_hip_gguf gllm_hip_gguf;

/* Map path read-only (a read copy where mapping fails) and parse its header:
 * metadata, tensor table, DataOffset = aligned end of the header
 * (general.alignment, default 32).  NULL on a malformed or truncated file,
 * with gllm_hip_last_error() naming the problem.  Host-only; no device use. */
gllm_hip_gguf* gllm_hip_gguf_open(const char* path);
/* The same over a caller buffer, which must outlive the handle. */
gllm_hip_gguf* gllm_hip_gguf_parse(const void* data, size_t len);
void gllm_hip_gguf_close(gllm_hip_gguf* g);
uint32_t gllm_hip_gguf_version(const gllm_hip_gguf* g);
size_t gllm_hip_gguf_data_offset(const gllm_hip_gguf* g);
int gllm_hip_gguf_n_tensors(const gllm_hip_gguf* g);
int gllm_hip_gguf_n_metadata(const gllm_hip_gguf* g);
/* Metadata keys in file order (a repeated key keeps its last value). */
const char* gllm_hip_gguf_metadata_key(const gllm_hip_gguf* g, int i);
/* Tensor i: name, dims (GGUF order, dims[0] fastest; up to 8), ggml type id
 * (ids the reference does not know read 255), offset relative to the data
 * offset, and byte size (GGMLType.DataSize, else the gap to the next tensor
 * as inferTensorSizes model.go:2272 derives it).  Outputs may be NULL. */
int gllm_hip_gguf_tensor(const gllm_hip_gguf* g, int i, const char** name, int* n_dims,
                         uint64_t* dims, int* type, uint64_t* offset, uint64_t* bytes);
int gllm_hip_gguf_find_tensor(const gllm_hip_gguf* g, const char* name); /* -1 if absent */
const void* gllm_hip_gguf_tensor_data(const gllm_hip_gguf* g, int i);     /* borrowed */
/* Metadata value kind (GGUF wire kind 0..12); for an array also its element
 * kind and length (elem -1 and count 1 for a scalar). */
int gllm_hip_gguf_meta_kind(const gllm_hip_gguf* g, const char* key, int* kind, int* elem,
                            uint64_t* count);
/* Typed reads of key (idx < 0) or of element idx of the array under key,
 * with MetaValue's conversions (gguf.go:308-350): get_u32 accepts every
 * integer kind (cast to 32 bits), get_f32 f32 and f64.  GLLM_EINVAL when the
 * key is absent or the kind does not convert.  Strings are borrowed from the
 * file and not NUL-terminated. */
int gllm_hip_gguf_get_u32(const gllm_hip_gguf* g, const char* key, int idx, uint32_t* out);
int gllm_hip_gguf_get_u64(const gllm_hip_gguf* g, const char* key, int idx, uint64_t* out);
int gllm_hip_gguf_get_f32(const gllm_hip_gguf* g, const char* key, int idx, float* out);
int gllm_hip_gguf_get_f64(const gllm_hip_gguf* g, const char* key, int idx, double* out);
int gllm_hip_gguf_get_bool(const gllm_hip_gguf* g, const char* key, int idx, int* out);
int gllm_hip_gguf_get_str(const gllm_hip_gguf* g, const char* key, int idx, const char** out,
                          size_t* len);
/* GGMLType.DataSize (gguf.go:241-297): bytes of n elements, 0 if unsized. */
uint64_t gllm_hip_ggml_data_size(int type, uint64_t n);
/* loadWeight for the row-kernel types: tensor name -> device weight with
 * rows = dims[1], cols = dims[0] (model.go:2393-2396), read straight from
 * the mapping; a tensor cut short by the end of the file is zero-padded. */
gllm_hip_weight* gllm_hip_gguf_load_weight(const gllm_hip_gguf* g, const char* name);
/* LoadModel for general.architecture = llama: the llama.* hyperparameters
 * (ConfigFromGGUF model.go:328-420; vocab = token_embd rows), token_embd,
 * output (tied to token_embd when absent), output_norm and blk.N.{attn_q,
 * attn_k, attn_v, attn_output, ffn_gate, ffn_down, ffn_up, attn_norm,
 * ffn_norm}.  The model owns the weights it loads.  max_len <= 0 takes
 * llama.context_length. */
gllm_hip_model* gllm_hip_model_from_gguf(const gllm_hip_gguf* g, int max_len);

#ifdef __cplusplus
}
#endif
#endif
