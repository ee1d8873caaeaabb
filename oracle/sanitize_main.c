/* sanitize_main.c -- drives every entry point of the CPU oracle once over
 * deterministic inputs, for the AddressSanitizer / UndefinedBehaviorSanitizer
 * build (`make -C oracle sanitize`, the counterpart of the reference's
 * `make test-race`, Makefile:306).  TEST INFRASTRUCTURE ONLY.
 *
 * Each section exercises one family at small, ragged and edge-case inputs:
 * zero and NaN activation blocks, infinities, every row type in both
 * evaluation orders, the AVX2 port, attention at ragged spans, and a tiny
 * llama decoder with and without the repeat penalty.  Any out-of-bounds
 * access, use after free, leak or undefined operation aborts the run with a
 * sanitizer report; a clean run prints "oracle sanitize: ok" and exits 0. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "gllm_oracle.h"

static uint64_t g_state = 0x9E3779B97F4A7C15ull;

static uint32_t next_u32(void) {
    g_state ^= g_state << 13;
    g_state ^= g_state >> 7;
    g_state ^= g_state << 17;
    return (uint32_t)(g_state >> 16);
}

static float next_normal(float std) {
    /* sum of 12 uniforms - 6: bounded, deterministic, roughly N(0, 1) */
    float s = 0.0f;
    for (int i = 0; i < 12; i++) s += (float)(next_u32() & 0xffffff) / 16777216.0f;
    return (s - 6.0f) * std;
}

static float* normal_vec(long n, float std) {
    float* v = (float*)malloc(sizeof(float) * (size_t)n);
    for (long i = 0; i < n; i++) v[i] = next_normal(std);
    return v;
}

static const int kTypes[] = {REF_Q4_K, REF_Q6_K, REF_Q8_0, REF_Q5_K, REF_Q4_0,
                             REF_Q4_1, REF_MXFP4, REF_Q2_K, REF_Q3_K};

static void check_f16(void) {
    for (uint32_t h = 0; h < 65536; h++) {
        float f = ref_f16_to_f32((uint16_t)h);
        (void)ref_f32_to_f16(f);
    }
    float edge[] = {0.0f, -0.0f, INFINITY, -INFINITY, NAN, 65504.0f, 65520.0f, 1e-8f, -1e-30f};
    uint16_t h[9];
    float back[9];
    ref_f32_to_f16_row(edge, h, 9);
    ref_f16_to_f32_row(h, back, 9);
}

static void check_q8k(void) {
    const int blocks = 4, n = 256 * blocks;
    float* x = normal_vec(n, 1.0f);
    for (int i = 256; i < 512; i++) x[i] = 0.0f;
    for (int i = 512; i < 768; i++) x[i] = NAN;
    x[900] = INFINITY;
    int8_t* q8 = (int8_t*)malloc((size_t)n);
    float sc[4], xs32[32], xs16[64];
    ref_q8k_quantize(x, q8, sc, blocks);
    for (int o = 0; o < 2; o++) {
        ref_xsums32(x, xs32, n / 32, o);
        ref_xsums16(x, xs16, n / 16, o, 1);
        ref_xsums16(x, xs16, n / 16, o, 0);
    }
    (void)ref_round_to_even_f32(2.5f);
    free(x);
    free(q8);
}

static void check_rows(int type, int rows, int cols, int threads) {
    const long rb = ref_row_bytes(type, cols);
    float* w = normal_vec((long)rows * cols, 0.02f);
    for (int c = 0; c < cols; c++) w[c] = 0.0f; /* an all-zero row */
    uint8_t* data = (uint8_t*)malloc((size_t)(rb * rows));
    if (type == REF_Q4_K || type == REF_Q6_K || type == REF_Q8_0) {
        ref_quantize_rows(type, w, rows, cols, data, threads);
    } else {
        /* no RTN encoder on the path for the other formats: random codes
         * with finite f16 scales are valid blocks of every layout */
        for (long i = 0; i < rb * rows; i++) data[i] = (uint8_t)next_u32();
        for (long i = 0; i + 1 < rb * rows; i += 2) data[i + 1] &= 0x3b; /* no inf / nan halves */
    }
    float* row = (float*)malloc(sizeof(float) * (size_t)cols);
    for (int r = 0; r < rows; r++) ref_dequant_row(type, data + (long)r * rb, cols, row);
    const int p = 3;
    float* xs = normal_vec((long)p * cols, 1.0f);
    float* outs = (float*)malloc(sizeof(float) * (size_t)(p * rows));
    for (int o = 0; o < 2; o++) {
        ref_matvec(type, data, xs, rows, cols, outs, o, threads);
        ref_matvec_batch(type, data, xs, p, rows, cols, outs, o, threads);
        (void)ref_argmax_matvec(type, data, xs, rows, cols, o, threads);
    }
    if (ref_has_avx2()) (void)ref_matvec_batch_fast(type, data, xs, p, rows, cols, outs, threads);
    int8_t* q8 = (int8_t*)malloc((size_t)cols);
    float* sc = (float*)malloc(sizeof(float) * (size_t)(cols / 256));
    ref_q8k_quantize(xs, q8, sc, cols / 256);
    int32_t* ints = (int32_t*)malloc(sizeof(int32_t) * (size_t)(cols / 256) * 8);
    if (type == REF_Q4_K || type == REF_Q6_K || type == REF_Q8_0)
        ref_lane_ints(type, data, q8, cols / 256, ints);
    free(ints);
    free(q8);
    free(sc);
    free(outs);
    free(xs);
    free(row);
    free(data);
    free(w);
}

static void check_vectors(void) {
    const int n = 1000; /* not a multiple of 8 or 32: exercises the tails */
    float* a = normal_vec(n, 1.0f);
    float* b = normal_vec(n, 1.0f);
    float* out = (float*)malloc(sizeof(float) * n);
    uint16_t* bh = (uint16_t*)malloc(2 * (size_t)n);
    ref_f32_to_f16_row(b, bh, n);
    (void)ref_dot_f32(a, b, n);
    (void)ref_dot_f32_f16(a, bh, n);
    for (int i = -100; i <= 100; i++) (void)ref_fast_exp((float)i);
    (void)ref_fast_exp(NAN);
    (void)ref_fast_exp(-INFINITY);
    a[3] = NAN;
    a[4] = -200.0f;
    ref_silu_mul(a, b, out, n);
    ref_rmsnorm(b, a, 1e-5f, n, out);
    float inv[32], sn[32], cs[32];
    ref_rope_inv_freq(500000.0f, 64, inv);
    ref_rope_sincos(12345, inv, 32, sn, cs);
    ref_rope_apply(b, 64, 8, 32, sn, cs);
    float logits[7] = {1.0f, NAN, 3.0f, INFINITY, -2.0f, 3.0f, 0.5f};
    uint32_t recent[5] = {2, 2, 99, 5, 0};
    ref_apply_repeat_penalty(logits, 7, recent, 5, 1.3f);
    (void)ref_argmax_finite(logits, 7);
    free(a);
    free(b);
    free(out);
    free(bh);
}

static void check_attention(void) {
    const int kvd = 256, hd = 64, ctx = 77;
    float* k = normal_vec((long)ctx * kvd, 1.0f);
    float* v = normal_vec((long)ctx * kvd, 1.0f);
    uint16_t* kh = (uint16_t*)malloc(2 * (size_t)ctx * kvd);
    uint16_t* vh = (uint16_t*)malloc(2 * (size_t)ctx * kvd);
    ref_f32_to_f16_row(k, kh, (long)ctx * kvd);
    ref_f32_to_f16_row(v, vh, (long)ctx * kvd);
    float* q = normal_vec(4 * hd, 1.0f);
    float out[4 * 64];
    const int spans[][2] = {{0, 0}, {0, 76}, {10, 11}, {76, 76}, {3, 70}};
    for (int g = 0; g < 4; g++)
        for (int s = 0; s < 5; s++)
            ref_attend_group_f16(q, kh + g * hd, vh + g * hd, 4, kvd, kvd, hd, hd, spans[s][0],
                                 spans[s][1], 0.125f, out);
    free(k);
    free(v);
    free(kh);
    free(vh);
    free(q);
}

static uint8_t* quantized(int type, int rows, int cols, float std) {
    float* w = normal_vec((long)rows * cols, std);
    uint8_t* d = (uint8_t*)malloc((size_t)(ref_row_bytes(type, cols) * rows));
    ref_quantize_rows(type, w, rows, cols, d, 1);
    free(w);
    return d;
}

static void check_llama(int fast) {
    ref_llama m;
    memset(&m, 0, sizeof m);
    m.n_layers = 2, m.dim = 256, m.hidden = 512, m.n_heads = 4, m.n_kv_heads = 1;
    m.head_dim = 64, m.vocab = 300, m.max_len = 40;
    m.rms_eps = 1e-5f, m.rope_theta = 500000.0f;
    m.emb_type = REF_Q4_K, m.out_type = REF_Q6_K, m.layer_type = REF_Q4_K;
    const int qd = m.n_heads * m.head_dim, kvd = m.n_kv_heads * m.head_dim;
    uint8_t* emb = quantized(REF_Q4_K, m.vocab, m.dim, 1.0f);
    uint8_t* outw = quantized(REF_Q6_K, m.vocab, m.dim, 0.05f);
    float* onorm = normal_vec(m.dim, 1.0f);
    m.tok_embd = emb, m.output = outw, m.out_norm = onorm;
    const uint8_t *wq[2], *wk[2], *wv[2], *wo[2], *w1[2], *w2[2], *w3[2];
    const float *an[2], *fn[2];
    for (int l = 0; l < 2; l++) {
        wq[l] = quantized(REF_Q4_K, qd, m.dim, 0.05f);
        wk[l] = quantized(REF_Q4_K, kvd, m.dim, 0.05f);
        wv[l] = quantized(REF_Q4_K, kvd, m.dim, 0.05f);
        wo[l] = quantized(REF_Q4_K, m.dim, qd, 0.05f);
        w1[l] = quantized(REF_Q4_K, m.hidden, m.dim, 0.05f);
        w2[l] = quantized(REF_Q4_K, m.dim, m.hidden, 0.05f);
        w3[l] = quantized(REF_Q4_K, m.hidden, m.dim, 0.05f);
        an[l] = normal_vec(m.dim, 1.0f);
        fn[l] = normal_vec(m.dim, 1.0f);
    }
    m.wq = wq, m.wk = wk, m.wv = wv, m.wo = wo, m.w1 = w1, m.w2 = w2, m.w3 = w3;
    m.attn_norm = an, m.ffn_norm = fn;
    uint32_t prompt[9], toks[12];
    for (int i = 0; i < 9; i++) prompt[i] = next_u32() % (uint32_t)m.vocab;
    for (int pen = 0; pen < 2; pen++) {
        ref_llama_state* s = ref_llama_state_new(&m, 2);
        ref_llama_set_fast(s, fast);
        if (pen) ref_llama_set_repeat_penalty(s, 1.7f, 8);
        ref_llama_generate(s, prompt, 9, 12, 4, toks);
        float logits[300], hid[256];
        (void)ref_llama_prefill(s, prompt, 3, 21, 32, logits);
        (void)ref_llama_decode(s, toks[0], 24, hid);
        (void)ref_llama_kcache(s, 1);
        (void)ref_llama_vcache(s, 0);
        ref_llama_state_free(s);
    }
    for (int l = 0; l < 2; l++) {
        free((void*)wq[l]), free((void*)wk[l]), free((void*)wv[l]), free((void*)wo[l]);
        free((void*)w1[l]), free((void*)w2[l]), free((void*)w3[l]);
        free((void*)an[l]), free((void*)fn[l]);
    }
    free(emb);
    free(outw);
    free(onorm);
}

int main(void) {
    check_f16();
    check_q8k();
    check_vectors();
    for (size_t t = 0; t < sizeof kTypes / sizeof kTypes[0]; t++) {
        if (!ref_type_supported(kTypes[t])) continue;
        check_rows(kTypes[t], 37, 512, 1);
        check_rows(kTypes[t], 5, 256, 3);
    }
    check_attention();
    check_llama(0);
    if (ref_has_avx2()) check_llama(1);
    printf("oracle sanitize: ok\n");
    return 0;
}
