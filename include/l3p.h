/*
 * l3p.h — C-ABI of libl3p.so, the MI355X (gfx950) quantized forward path of
 * llama3pure.
 *
 * Plain pointers and sizes only.  Device pointers ("_dev") are HIP device
 * addresses on the context's device; all work is ordered on the context's
 * single HIP stream.  Every call returns L3P_OK (0) or a negative L3P_E_*
 * code, with a message in l3p_last_error(ctx).
 *
 * Each entry point names the reference interface it replaces
 * (llama3pure-c-engine.c "c:LINE", llama3pure-js-engine.js "js:LINE").
 */
#ifndef L3P_H
#define L3P_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define L3P_OK 0
#define L3P_E_INVALID (-1)     /* bad argument or shape                       */
#define L3P_E_UNSUPPORTED (-2) /* tensor type / shape not implemented          */
#define L3P_E_HIP (-3)         /* HIP runtime error                            */
#define L3P_E_NOMEM (-4)       /* device or host allocation failed             */
#define L3P_E_FORMAT (-5)      /* malformed GGUF                               */
#define L3P_E_STATE (-6)       /* call out of order (e.g. no model loaded)     */

/* GGML tensor type ids, identical to the reference's enum ggml_type (c:95-113). */
enum l3p_type {
    L3P_F32 = 0, L3P_F16 = 1, L3P_Q4_0 = 2, L3P_Q4_1 = 3, L3P_Q5_0 = 6, L3P_Q5_1 = 7,
    L3P_Q8_0 = 8, L3P_Q2_K = 10, L3P_Q3_K = 11, L3P_Q4_K = 12, L3P_Q5_K = 13,
    L3P_Q6_K = 14, L3P_IQ4_NL = 20, L3P_BF16 = 29
};

typedef struct l3p_ctx l3p_ctx;

/* ---- context ------------------------------------------------------------ */
/* Opens the GPU `device` and creates the context's stream.  Replaces the
 * process-global engine state of the reference (c:4736-4764, js:205-223). */
int l3p_create(int device, l3p_ctx** out);
void l3p_destroy(l3p_ctx* ctx);
/* Message of the last failed call on ctx (or of l3p_create when ctx is NULL). */
const char* l3p_last_error(const l3p_ctx* ctx);
/* The context's hipStream_t, for callers that time or order work around it. */
void* l3p_stream(l3p_ctx* ctx);
int l3p_synchronize(l3p_ctx* ctx);

/* ---- device memory, for hosts without a GPU runtime of their own -------- */
int l3p_malloc(l3p_ctx* ctx, size_t bytes, void** out_dev);
int l3p_free(l3p_ctx* ctx, void* dev);
int l3p_upload(l3p_ctx* ctx, void* dst_dev, const void* src_host, size_t bytes);
int l3p_download(l3p_ctx* ctx, void* dst_host, const void* src_dev, size_t bytes);

/* ---- quantized ops on device buffers ------------------------------------ */
/* Block bytes of one row of `cols` elements (get_row_size, c:2076-2080). */
size_t l3p_row_bytes(int type, int cols);

/* Dequantize n elements of blocks to fp32, bit-exact with the reference's
 * dequantize_row (c:956-1046; per-type c:611-934).  Types: F32 F16 BF16 Q4_0
 * Q4_1 Q5_0 Q5_1 Q8_0 Q2_K Q3_K Q4_K Q5_K Q6_K IQ4_NL. */
int l3p_dequant(l3p_ctx* ctx, int type, const void* src_dev, int64_t n, float* dst_dev);

/* Quantize n fp32 values (n % 32 == 0) to Q8_0 blocks of 34 bytes, bit-exact
 * with quantize_row_q8_0 (c:1508-1528) and quantize_to_q8_0_cache
 * (c:1535-1570): truncating fp16 scale, roundf quants. */
int l3p_quantize_q8_0(l3p_ctx* ctx, const float* x_dev, int64_t n, void* dst_dev);

/* y[rows] = W[rows x cols] . x[cols] with W in its native block layout.
 * Replaces matmul_quantized (c:2091-2133; js:3107-3142) for F16 BF16 Q4_0
 * Q4_1 Q5_0 Q5_1 Q8_0 Q2_K Q3_K Q4_K Q5_K Q6_K IQ4_NL with cols <= 32768 and
 * F32 with cols <= 16384 (wider: L3P_E_UNSUPPORTED).  Semantics per type
 * follow the reference: Q8_0 and the K-quants use fp32 x (matmul_deq_4row,
 * c:2136-2176), F16/BF16/F32 the float dot (c:1467-1494); Q4_0 Q4_1 Q5_0
 * Q5_1 IQ4_NL quantize x to Q8_0
 * first and use their integer block dots (c:2105-2116, c:1625-1717,
 * c:1994-2011).  Results differ from the reference's only by fp32 summation
 * order.  w_dev and x_dev must be 16-byte aligned (l3p_malloc memory is). */
int l3p_gemv(l3p_ctx* ctx, int type, const void* w_dev, int rows, int cols, const float* x_dev,
             float* y_dev);

/* Batched form for prefill: y[b*out_stride + r] = W[r,:] . x[b*in_stride + :]
 * for b < batch.  Replaces matmul_quantized_batch (c:2291-2331; js:3159-3845).
 * Q8_0, the K-quants, F16, BF16 and F32 run on the fp32-MFMA GEMM (weights
 * dequantized exactly, as matmul_deq_batch_4row, c:2179-2273); Q4_0 Q4_1
 * Q5_0 Q5_1 IQ4_NL on the int8 matrix cores as the reference's
 * Q8_0-activation dots (c:2305-2318): every batch row quantized to Q8_0,
 * exact integer block dots, each output's block terms added in block order.
 * in_stride must be a multiple of 4 and x_dev 16-byte aligned. */
int l3p_gemm(l3p_ctx* ctx, int type, const void* w_dev, int rows, int cols, const float* x_dev,
             int batch, int in_stride, float* y_dev, int out_stride);

/* l3p_gemm without a context and without any allocation.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The work is enqueued on `stream` (a hipStream_t; NULL: the
 * null stream) of the current device.  Split-K partials go to a file-scope
 * device array of 16 MB (4 Mi floats) that each GPU holds for the life of
 * the process; the launch plan is l3p_gemm's, so results are l3p_gemm's, and
 * a shape whose partials would exceed the array returns L3P_E_UNSUPPORTED.
 * (Q4_0 Q4_1 Q5_0 Q5_1 IQ4_NL keep their Q8_0-quantized x rows there
 * instead, as many rows per launch as fit.)
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * race.  Errors: the code, with the message in l3p_last_error(NULL). */
int l3p_gemm_static(int type, const void* w_dev, int rows, int cols, const float* x_dev, int batch,
                    int in_stride, float* y_dev, int out_stride, void* stream);

/* ---- model -------------------------------------------------------------- */
typedef struct {
    int context_size;   /* <=0: the model's context_length (c:5174-5178; js:4335)   */
    /* The two options below have no counterpart in the reference, which
     * hard-codes Gemma's sliding-window pattern to 6 (c:5100) and has no
     * attention score cap; they let Gemma-2 checkpoints run as trained.
     * swa_pattern > 0: Gemma layer l uses the sliding window when
     *   l % swa_pattern < swa_pattern - 1 (2: alternating local/global,
     *   starting local); 0 keeps 6.  No effect on Llama models.
     * attn_softcap > 0: every attention score s becomes
     *   attn_softcap * tanhf(s / attn_softcap) before the softmax (Gemma-2's
     *   attention logit soft-capping); 0: scores as they are.
     * Negative values, an infinite or NaN cap return L3P_E_INVALID. */
    int swa_pattern;
    float attn_softcap;
    int reserved[5];
} l3p_load_opts;

typedef struct {
    int dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len, head_dim;
    int is_gemma, swa_window, swa_pattern, weight_type;
    float rope_theta, rope_theta_swa, rms_eps, final_softcap;
    int64_t device_bytes;   /* HBM held by weights + KV cache + scratch */
    float attn_softcap;     /* the load option in effect (0: none) */
    int reserved;
} l3p_model_info;

/* Parse a GGUF image in host memory and copy every tensor, unchanged, into
 * HBM; allocate the device KV cache for the context length.  Replaces
 * parse_gguf_file + init_weights_from_gguf + malloc_run_state (c:2500-2688,
 * c:2939-3082, c:346-468) and js loadModel/loadWeights/createRunState
 * (js:4288-4584, js:4586-4660).  The host image may be freed after return. */
int l3p_load_gguf(l3p_ctx* ctx, const void* gguf, size_t len, const l3p_load_opts* opts);
int l3p_get_model_info(l3p_ctx* ctx, l3p_model_info* out);

/* One decode position: transformer(token, pos, compute_logits) (c:3190-3435;
 * js:6121-6128).  When compute_logits, logits stay on the device and, if
 * logits_host is non-NULL, vocab_size floats are copied there. */
int l3p_forward(l3p_ctx* ctx, int32_t token, int32_t pos, int compute_logits, float* logits_host);

/* Prefill tokens[0..n) at positions start_pos.. into the KV cache without
 * logits: transformer_prefill (c:3439-3680; js:6130-6136). */
int l3p_prefill(l3p_ctx* ctx, const int32_t* tokens_host, int n, int32_t start_pos);

/* Sampling settings (c:4736-4741; js:218-223).  temperature == 0 -> argmax. */
typedef struct {
    float temperature;
    int top_k;
    float top_p;
    int reserved;
} l3p_sampler;

/* Forward at (token, pos) with logits, then sample on the device; only the
 * token id comes back.  *rng is the xorshift64* state (c:4266-4276),
 * advanced by one draw when temperature != 0.  Replaces generate_token's
 * forward + sampler (c:4766-4907) and js transformer + sample (js:6121,
 * js:6158-6267). */
int l3p_decode(l3p_ctx* ctx, int32_t token, int32_t pos, const l3p_sampler* s, uint64_t* rng,
               int32_t* out_token);

/* Greedy generation: the reference's decode loop (c:5289-5309, each
 * iteration generate_token at temperature 0, c:4766-4813) from (token, pos)
 * for up to max_steps steps, never past the context: step i decodes position
 * pos + i and writes its argmax token to out_tokens[i].  It stops after the
 * first token found in stop_ids[0..n_stop) (the reference's eos/eot checks,
 * c:5296-5303), which is written and counted.  *n_out = tokens written.  The
 * tokens equal those of l3p_decode called step by step with temperature 0;
 * the steps are queued on the device ahead of the host's reads, so no step
 * waits for the host.  The repetition stop (c:4910-4918) is left to the
 * caller, which can cut the returned tokens.  A step already queued behind
 * a stop still runs (the queue is two steps ahead): it writes the K/V rows
 * of position pos + *n_out and leaves its logits (l3p_logits_device) for a
 * token that is not returned. */
int l3p_generate_greedy(l3p_ctx* ctx, int32_t token, int32_t pos, int32_t max_steps, const int32_t* stop_ids,
                        int32_t n_stop, int32_t* out_tokens, int32_t* n_out);

/* Sampled generation: the reference's decode loop (c:5289-5309) with
 * generate_token at temperature > 0 (c:4766-4907) from (token, pos) for up
 * to max_steps steps, never past the context.  Step i decodes position
 * pos + i and writes its sampled token to out_tokens[i]; *rng is the
 * xorshift64* state (c:4266-4276), advanced by one draw per step; it stops
 * after the first token found in stop_ids[0..n_stop), which is written and
 * counted (*n_out = tokens written).  The tokens and the final RNG state equal
 * those of l3p_decode called step by step with the same sampler.  The top-k
 * slots run on the device and the sampler's last part (c:4850-4907: expf,
 * sort, top-p cut, draw) on the host in the reference's arithmetic; the steps
 * are queued on the device ahead of the host, each step's embedding waiting
 * on the device for the token the host hands over through pinned memory, so
 * no launch waits for the host.  A step already queued behind a stop still
 * runs with the stop token (the K/V rows of position pos + *n_out; its
 * logits, l3p_logits_device, belong to no returned token).  temperature must
 * be > 0 (0 is l3p_generate_greedy) and top_k in [1, 1024]. */
int l3p_generate_sampled(l3p_ctx* ctx, int32_t token, int32_t pos, int32_t max_steps, const l3p_sampler* s,
                         uint64_t* rng, const int32_t* stop_ids, int32_t n_stop, int32_t* out_tokens,
                         int32_t* n_out);

/* Sample from vocab logits already on the device (the sampler alone). */
int l3p_sample(l3p_ctx* ctx, const float* logits_dev, int n, const l3p_sampler* s, uint64_t* rng,
               int32_t* out_token);

/* Device pointer of the logits of the last step run (vocab_size floats).
 * After l3p_generate_greedy stopped on a stop id, that is the queued step past
 * the stop, whose token was not returned. */
int l3p_logits_device(l3p_ctx* ctx, const float** out_dev);

/* Copy one layer's K or V cache in the reference layout
 * [kv_head][seq_len][head_dim/32 x 34 B] (c:365-372) to host memory. */
int l3p_copy_kv(l3p_ctx* ctx, int layer, int which_v, void* dst_host, size_t cap);

/* Row `pos` of the RoPE cos/sin tables (head_dim/2 floats each) that the
 * model uses, computed on the host with the reference's expression
 * cosf((float)pos * (1.0f / powf(theta, 2i/head_dim))) (c:381-422); swa
 * selects the sliding-window theta of Gemma models (c:398-416). */
int l3p_rope_row(l3p_ctx* ctx, int swa, int pos, float* cos_host, float* sin_host);

/* GEMV launch timing.  No counterpart in the reference, which only prints
 * whole-token rates (c:5312-5314; tests.js:167-180).  l3p_profile(ctx, 1)
 * clears the statistics and records HIP events on the context stream around
 * every GEMV launch of l3p_forward/l3p_prefill/l3p_decode; l3p_profile(ctx, 0)
 * stops.  l3p_profile_read fills up to cap entries, one per launch class
 * ("<type> gemv <what> <rows>x<cols>"), and sets *n to the number of classes. */
typedef struct {
    char name[64];
    int64_t launches;
    double total_ms;          /* summed event-to-event time of the launches */
    double bytes_per_launch;  /* weight blocks + 4*cols + 4*output rows */
    double p10_ms, p50_ms, p90_ms;   /* percentiles of the launch durations */
} l3p_kernel_stat;
int l3p_profile(l3p_ctx* ctx, int on);
int l3p_profile_read(l3p_ctx* ctx, l3p_kernel_stat* out, int cap, int* n);

/* A plain streaming read of `bytes` (a multiple of 16) from the 16-byte
 * aligned device buffer `buf` on the context stream, timed under l3p_profile
 * as "stream read <bytes>".  No counterpart in the reference: it measures the
 * HBM read ceiling that the GEMVs' weight stream is compared with. */
int l3p_stream_read(l3p_ctx* ctx, const void* buf, size_t bytes);

#ifdef __cplusplus
}
#endif
#endif /* L3P_H */
