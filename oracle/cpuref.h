/*
 * cpuref.h — CPU restatement of llama3pure's quantized forward path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle that the HIP product
 * path is checked against.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product never links it.
 *
 * Every function follows the arithmetic of the reference C engine
 * (llama3pure-c-engine.c, cited as c:LINE) operation for operation, so that a
 * build with -O2 -ffp-contract=off gives the same fp32 bits as the reference
 * built with its own Makefile line (`gcc -O3`, Makefile:7-8).
 */
#ifndef L3P_ORACLE_CPUREF_H
#define L3P_ORACLE_CPUREF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (c:95-113). */
enum {
    L3O_F32 = 0, L3O_F16 = 1, L3O_Q4_0 = 2, L3O_Q4_1 = 3, L3O_Q5_0 = 6, L3O_Q5_1 = 7,
    L3O_Q8_0 = 8, L3O_Q2_K = 10, L3O_Q3_K = 11, L3O_Q4_K = 12, L3O_Q5_K = 13,
    L3O_Q6_K = 14, L3O_IQ4_NL = 20, L3O_BF16 = 29, L3O_BF16_ALT = 30
};

/* ---- scalar conversions ---- */
float    l3o_fp16_to_fp32(uint16_t h);                 /* c:547-582 */
uint16_t l3o_fp32_to_fp16(float f);                    /* c:585-599 (truncating) */
void     l3o_fp16_to_fp32_n(const uint16_t* h, float* f, size_t n);
void     l3o_fp32_to_fp16_n(const float* f, uint16_t* h, size_t n);

/* ---- block formats ---- */
int      l3o_block_elems(int type);                    /* c:1049-1068 */
size_t   l3o_block_bytes(int type);                    /* c:1071-1091 */
size_t   l3o_row_bytes(int type, int cols);            /* c:2076-2080 */
int      l3o_dequant_row(int type, const void* src, float* dst, int n);  /* c:956-1046 */
void     l3o_quantize_q8_0(const float* x, void* dst, int n);            /* c:1508-1528 */

/* ---- GEMV / batched GEMM with the reference's per-type semantics ---- */
/* matmul_quantized (c:2091-2133) with deq_buf/q8_buf allocated as main() does. */
int l3o_matmul(int type, const void* w, int rows, int cols, const float* x, float* y);
/* matmul_quantized_batch (c:2291-2331). */
int l3o_matmul_batch(int type, const void* w, int rows, int cols, const float* x,
                     int batch, int in_stride, float* y, int out_stride);

/* ---- elementwise blocks (c:3089-3186) ---- */
float l3o_fast_expf(float x);
float l3o_fast_tanhf(float x);
void  l3o_rmsnorm(float* o, const float* x, const float* w, int n, float eps);
void  l3o_softmax(float* x, int n);
void  l3o_swiglu(float* hb, const float* hb2, int n);  /* c:3400-3406 */
void  l3o_geglu(float* hb, const float* hb2, int n);   /* c:3391-3398 */

/* ---- sampler (c:4266-4288, c:4803-4907) ---- */
uint32_t l3o_rng_u32(uint64_t* state);
float    l3o_rng_f32(uint64_t* state);
int      l3o_argmax(const float* v, int n);
int      l3o_sample(const float* logits, int n, float temperature, int top_k, float top_p,
                    uint64_t* rng_state);

/* ---- whole model: GGUF in memory -> decode/prefill (c:3190-3680) ---- */
typedef struct l3o_model l3o_model;
/* Parses the GGUF image (kept borrowed; caller keeps it alive) and builds the
 * config exactly as main() does (c:5049-5182).  context_size<=0 keeps the
 * model's own context length.  Returns NULL on error (message via
 * l3o_last_error()). */
l3o_model*  l3o_model_open(const void* gguf, size_t len, int context_size);
void        l3o_model_close(l3o_model* m);
const char* l3o_last_error(void);
/* info: dim hidden n_layers n_heads n_kv_heads vocab seq_len head_dim is_gemma
 *       swa_window swa_pattern */
void  l3o_model_info(const l3o_model* m, int* info11);
int   l3o_forward(l3o_model* m, int token, int pos, int compute_logits, float* logits);
int   l3o_prefill(l3o_model* m, const int* tokens, int start_pos, int batch);
/* Copies one layer's Q8_0 key or value cache ([kv_head][seq][hd/32*34 B]). */
int   l3o_copy_kv(const l3o_model* m, int layer, int which_v, void* dst, size_t cap);
/* Test support (no counterpart in the reference): overwrites one layer's K or
 * V cache with exactly layer_kv bytes in the l3o_copy_kv layout. */
int   l3o_set_kv(l3o_model* m, int layer, int which_v, const void* src, size_t n);
/* Row pos of the RoPE cos/sin tables (c:381-422); swa selects the
 * sliding-window tables of Gemma models. */
int   l3o_rope_row(const l3o_model* m, int swa, int pos, float* cos_out, float* sin_out);
/* Residual stream x after the last forward (dim floats). */
int   l3o_copy_x(const l3o_model* m, float* dst);
/* Load options without a counterpart in the reference: swa_pattern > 0
 * replaces the sliding-window layer pattern (layer l is local when
 * l % p < p - 1; the reference hard-codes 6 for Gemma, c:5100), and
 * attn_softcap > 0 caps every attention score s to cap * tanhf(s / cap). */
int   l3o_set_attention(l3o_model* m, int swa_pattern, float attn_softcap);
/* One head's capped attention over n Q8_0 cache rows (the forward's own). */
void  l3o_attend_head(const uint8_t* q8, const uint8_t* kc, const uint8_t* vc, int n, int hs, float cap,
                      float* att, float* out);

#ifdef __cplusplus
}
#endif
#endif
