/*
 * gllm_oracle.h -- CPU restatement of GopherLLM's quantized matvec and
 * decode-attention arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (gopherllm_amd/) links,
 * loads or calls this library.  It is the checker that the HIP kernels are
 * compared against (tests/, __graft_entry__.smoke) and the CPU baseline that
 * bench.py times beside the GPU.
 *
 * Every routine names the reference file:line whose arithmetic it restates.
 * Two evaluation orders exist for the row dots:
 *   - "generic": quant_q8k_portable.go (scalar Go, unfused float ops);
 *   - "amd64":   kernels_amd64.s (eight int32/float32 AVX2 lanes, VFMADD
 *                fused accumulation, fixed 8->4->2->1 horizontal tree).
 * The amd64 order is what the reference executes on x86-64 by default and is
 * the bit-exact target of the GPU decode path.
 */
#ifndef GLLM_ORACLE_H
#define GLLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (gguf.go:27-60). */
enum {
    REF_F32 = 0, REF_F16 = 1, REF_Q4_0 = 2, REF_Q4_1 = 3, REF_Q8_0 = 8, REF_Q2_K = 10,
    REF_Q3_K = 11, REF_Q4_K = 12, REF_Q5_K = 13, REF_Q6_K = 14, REF_BF16 = 30, REF_MXFP4 = 39
};
enum { REF_ORDER_GENERIC = 0, REF_ORDER_AMD64 = 1 };

/* ---- f16 (simd.go:88-109, kv_f16.go:17-49) ---- */
float ref_f16_to_f32(uint16_t h);
uint16_t ref_f32_to_f16(float f);
void ref_f32_to_f16_row(const float* src, uint16_t* dst, long n);
void ref_f16_to_f32_row(const uint16_t* src, float* dst, long n);

/* ---- activation quantisation (quant_q8k_portable.go:36-62) ---- */
void ref_q8k_quantize(const float* x, int8_t* q8, float* scales, int blocks);
float ref_round_to_even_f32(float v);
/* per-32 / per-16 group sums; order selects amd64 (sumF32Groups32/16) or
 * generic (simd.go:836-862 / 551-580).  The 16-group variant multiplies by
 * 32 afterwards (ScaleF32(xs, 32)) when scale32 != 0. */
void ref_xsums32(const float* x, float* out, int groups, int order);
void ref_xsums16(const float* x, float* out, int groups, int order, int scale32);

/* ---- row dots against Q8K activations ---- */
float ref_q4k_dot(const uint8_t* row, const int8_t* q8, const float* xscale,
                  const float* xsums32, int blocks, int order);
float ref_q6k_dot(const uint8_t* row, const int8_t* q8, const float* xscale,
                  const float* xsums16x32, int blocks, int order);
float ref_q8_0_dot(const uint8_t* row, const int8_t* q8, const float* xscale,
                   int blocks, int order);
/* amd64 int32 lane accumulators (the exact integer part) for each block:
 * out[b*8 + k] = accI_k of block b. */
/* Any supported type: one row against prepared activations (xsums as the
 * type needs them: 32-group sums for Q4_K/Q5_K/Q4_0/Q4_1, 16-group sums x32
 * for Q6_K, unscaled 16-group sums for Q2_K, none otherwise). */
float ref_row_dot_any(int type, const uint8_t* row, const int8_t* q8, const float* xscale,
                      const float* xsums, int blocks, int order);
int ref_type_supported(int type);
void ref_lane_ints(int type, const uint8_t* row, const int8_t* q8, int blocks,
                   int32_t* out);

/* ---- float-activation row dots of same-type fused groups ----
 * (sameTypeQuantDot model.go:3258-3283: DotQ8_0F32 simd.go:646, DotQ4_0F32
 * simd.go:677, DotQ4_1F32 quant_extra.go:42, DotQ2KF32 quant_extra.go:271,
 * DotQ3KF32 quant_extra.go:376, DotMXFP4F32 simd.go:1458) on GGUF rows and
 * f32 x; cols % 256 == 0 for the K formats, % 32 otherwise. */
int ref_float_dot_supported(int type);
float ref_float_dot(int type, const uint8_t* row, const float* x, int cols);
int ref_matvec_float(int type, const uint8_t* data, const float* x, int rows, int cols,
                     float* out, int threads);

/* bytes per row for a GGML type */
long ref_row_bytes(int type, int cols);

/* ---- matvec orchestration (simd.go:204/261/413, kernels_amd64.go:470) ----
 * out[r] = W[r,:] . x for r < rows.  x holds cols floats (cols % 256 == 0).
 * threads <= 0 uses all cores. */
int ref_matvec(int type, const uint8_t* data, const float* x, int rows, int cols,
               float* out, int order, int threads);
/* p activation rows, xs row-major [p][cols], outs [p][rows] */
int ref_matvec_batch(int type, const uint8_t* data, const float* xs, int p,
                     int rows, int cols, float* outs, int order, int threads);
/* greedy argmax over finite logits, lowest index on ties
 * (kernels_amd64.go:294-331, sampling.go:385-418) */
uint32_t ref_argmax_matvec(int type, const uint8_t* data, const float* x, int rows,
                           int cols, int order, int threads);
uint32_t ref_argmax_finite(const float* logits, long n);
void ref_apply_repeat_penalty(float* logits, long n, const uint32_t* recent, int n_recent,
                              float penalty);

/* ---- RTN encoders and decoders (quantize_rtn.go, simd.go:1488-1643) ---- */
void ref_quantize_rows(int type, const float* src, long rows, int cols, uint8_t* dst,
                       int threads);
void ref_dequant_row(int type, const uint8_t* row, int cols, float* out);

/* ---- vector helpers, amd64 order (kernels_amd64.s) ---- */
float ref_dot_f32(const float* a, const float* b, long n);
float ref_dot_f32_f16(const float* a, const uint16_t* b, long n);
float ref_fast_exp(float x);
void ref_silu_mul(const float* gate, const float* up, float* out, long n);
void ref_rmsnorm(const float* x, const float* w, float eps, long n, float* out);
void ref_rope_inv_freq(float theta, int head_dim, float* inv);
void ref_rope_sincos(int pos, const float* inv, int pairs, float* sinv, float* cosv);
void ref_rope_apply(float* vec, int head_dim, int n_heads, int pairs,
                    const float* sinv, const float* cosv);

/* ---- attention over an f16 KV cache (model.go:3527-3588, 3761-3787) ----
 * keys/values point at the kv head's first element of position 0; stride is
 * the per-position element stride.  q holds q_heads*hd floats, out
 * q_heads*vd floats (overwritten). */
void ref_attend_group_f16(const float* q, const uint16_t* keys, const uint16_t* values,
                          int q_heads, long kstride, long vstride, int hd, int vd,
                          int start, int end, float scale, float* out);

/* ---- llama decoder (model.go:2622-2820, forward_batch.go:336-613) ---- */
typedef struct ref_llama {
    int n_layers, dim, hidden, n_heads, n_kv_heads, head_dim, vocab, max_len;
    float rms_eps, rope_theta;
    int emb_type, out_type;
    const uint8_t* tok_embd;   /* [vocab][dim] emb_type */
    const uint8_t* output;     /* [vocab][dim] out_type */
    const float* out_norm;     /* [dim] */
    int layer_type;            /* type of every attention/FFN matrix */
    const uint8_t** wq; const uint8_t** wk; const uint8_t** wv; const uint8_t** wo;
    const uint8_t** w1; const uint8_t** w2; const uint8_t** w3;
    const float** attn_norm; const float** ffn_norm;
    /* NULL, or the type of each matrix, n_layers * 7 in the order wq wk wv wo
     * w1 w2 w3 (mixed files such as Q4_K_M, whose attn_v / ffn_down are Q6_K) */
    const int* types;
    /* config.AttentionScale (llama.attention.scale); 0 = 1/sqrt(head_dim)
     * (model.go:2685-2688) */
    float attn_scale;
} ref_llama;

typedef struct ref_llama_state ref_llama_state;
ref_llama_state* ref_llama_state_new(const ref_llama* m, int threads);
void ref_llama_state_free(ref_llama_state* s);
/* route the row dots through the AVX2 port (no-op without AVX2/FMA/F16C) */
void ref_llama_set_fast(ref_llama_state* s, int on);
/* one decode step at position pos; writes the normed final hidden state into
 * hidden_out (dim floats, may be NULL) and returns the greedy token */
uint32_t ref_llama_decode(ref_llama_state* s, uint32_t token, int pos, float* hidden_out);
/* repeat penalty over the last `window` tokens seen by prefill / decode
 * (window 0: none); resets the window */
void ref_llama_set_repeat_penalty(ref_llama_state* s, float penalty, int window);
/* prefill n tokens starting at start_pos in chunks; returns the greedy token
 * from the last position's full logits (logits_out: vocab floats or NULL) */
uint32_t ref_llama_prefill(ref_llama_state* s, const uint32_t* tokens, int n, int start_pos,
                           int chunk, float* logits_out);
/* full greedy run: prefill prompt then decode; writes n_gen tokens */
void ref_llama_generate(ref_llama_state* s, const uint32_t* prompt, int n_prompt,
                        int n_gen, int chunk, uint32_t* out_tokens);
/* access K/V cache rows (f16) of layer l at position pos, for tests */
const uint16_t* ref_llama_kcache(ref_llama_state* s, int l);
const uint16_t* ref_llama_vcache(ref_llama_state* s, int l);

int ref_num_threads(void);
int ref_has_avx2(void);

/* ---- AVX2 port used as the timed CPU baseline (gllm_oracle_avx2.c) ----
 * bit-identical to the amd64-order restatement above */
float ref_q4k_dot_avx2(const uint8_t* row, const int8_t* q8, const float* xscale,
                       const float* xsums32, int blocks);
float ref_q6k_dot_avx2(const uint8_t* row, const int8_t* q8, const float* xscale,
                       const float* xsums16x32, int blocks);
float ref_q8_0_dot_avx2(const uint8_t* row, const int8_t* q8, const float* xscale, int blocks);
int ref_matvec_batch_fast(int type, const uint8_t* data, const float* xs, int p, int rows,
                          int cols, float* outs, int threads);

#ifdef __cplusplus
}
#endif
#endif
