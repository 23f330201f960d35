/*
 * ref_harness.c — compiles the UNMODIFIED reference engine where it lies
 * (llama3pure-c-engine.c, path given by -DREF_ENGINE) into one translation
 * unit and exports a few entry points for ctypes, so tests can ask the real
 * reference for its answers.  TEST INFRASTRUCTURE ONLY (the checker of the
 * checker); built into oracle/_ref/ by oracle/Makefile, never shipped.
 *
 * The reference's main() is renamed away with -Dmain=l3p_ref_main.  Apart from
 * that the engine text is compiled as-is, with the flags of its own Makefile.
 */
#include REF_ENGINE

/* ---- scalar and block primitives ---- */
void ref_init(void) { init_fp16_table(); }
float ref_fp16_to_fp32(uint16_t h) { return fp16_to_fp32(h); }
uint16_t ref_fp32_to_fp16(float f) { return fp32_to_fp16(f); }
void ref_fp16_to_fp32_n(const uint16_t* h, float* f, size_t n) { for (size_t i = 0; i < n; i++) f[i] = fp16_to_fp32(h[i]); }
void ref_fp32_to_fp16_n(const float* f, uint16_t* h, size_t n) { for (size_t i = 0; i < n; i++) h[i] = fp32_to_fp16(f[i]); }
void ref_dequant_row(int type, const void* src, float* dst, int n) { dequantize_row(dst, src, n, (enum ggml_type)type); }
void ref_quantize_q8_0(const float* x, void* dst, int n) { quantize_row_q8_0(x, (block_q8_0*)dst, n); }
float ref_fast_expf(float x) { return fast_expf(x); }
float ref_fast_tanhf(float x) { return fast_tanhf(x); }
void ref_rmsnorm(float* o, float* x, float* w, int n, float eps) { rmsnorm(o, x, w, n, 1.0f / (float)n, eps); }
void ref_softmax(float* x, int n) { softmax(x, n); }

/* Size q8_buf/deq_buf the way main() does (c:5186-5201), for inputs up to
 * max_cols wide. */
static int g_buf_cols = 0;
static void ensure_bufs(int max_cols) {
    if (max_cols <= g_buf_cols) return;
    free(q8_buf);
    free(deq_buf);
    q8_buf = (block_q8_0*)calloc((max_cols + QK8_0 - 1) / QK8_0, sizeof(block_q8_0));
    deq_buf_stride = 4 * max_cols;
    deq_buf = (float*)calloc((size_t)omp_get_max_threads() * deq_buf_stride, sizeof(float));
    g_buf_cols = max_cols;
}

/* A QuantizedTensor bound the way load_tensor_quantized() binds one (c:2886-2923). */
static void bind(QuantizedTensor* qt, int type, const void* w, int rows, int cols) {
    qt->data = (void*)w;
    qt->type = (enum ggml_type)type;
    qt->n_elements = rows * cols;
    qt->rows = rows;
    qt->cols = cols;
    qt->row_size = get_row_size(cols, (enum ggml_type)type);
    qt->q8_func = get_vec_dot_q8_func((enum ggml_type)type);
    qt->dot_func = get_vec_dot_func((enum ggml_type)type);
    qt->deq_func = get_deq_row_func((enum ggml_type)type);
}

void ref_matmul(int type, const void* w, int rows, int cols, const float* x, float* y) {
    QuantizedTensor qt;
    ensure_bufs(cols);
    bind(&qt, type, w, rows, cols);
    matmul_quantized(y, x, &qt);
}

void ref_matmul_batch(int type, const void* w, int rows, int cols, const float* x, int batch,
                      int in_stride, float* y, int out_stride) {
    QuantizedTensor qt;
    ensure_bufs(cols);
    bind(&qt, type, w, rows, cols);
    block_q8_0* bq = (block_q8_0*)calloc((size_t)batch * (cols / QK8_0 + 1), sizeof(block_q8_0));
    matmul_quantized_batch(y, x, &qt, batch, in_stride, out_stride, bq, cols / QK8_0 + 1);
    free(bq);
}

/* ---- whole model through the reference's own loader and forward ---- */
/* Builds config exactly as main() does (c:5037-5182) and then allocates what
 * main() allocates (c:5184-5211).  Returns 0 on success. */
int ref_model_open(const char* path, int ctx) {
    init_fp16_table();
    gguf_file = parse_gguf_file(path);
    if (!gguf_file) return -1;
    if (!load_gguf_tokenizer(gguf_file, path)) return -2;
    const char* arch = get_gguf_string(gguf_file, "general.architecture");
    config.is_gemma3 = 0;
    const char* pre = "llama";
    if (arch && (strcmp(arch, "gemma3") == 0 || strcmp(arch, "gemma2") == 0 || strcmp(arch, "gemma") == 0)) {
        config.is_gemma3 = 1;
        use_sentencepiece = 1;
        pre = "gemma3";
        if (get_gguf_int(gguf_file, "gemma3.embedding_length", 0) == 0) {
            if (get_gguf_int(gguf_file, "gemma2.embedding_length", 0) != 0) pre = "gemma2";
            else if (get_gguf_int(gguf_file, "gemma.embedding_length", 0) != 0) pre = "gemma";
        }
    }
    char k[96];
#define K(s) (snprintf(k, sizeof k, "%s." s, pre), k)
    config.swa_window = get_gguf_int(gguf_file, K("attention.sliding_window"), 0);
    config.rope_theta_swa = get_gguf_float(gguf_file, K("rope.freq_base_swa"), 10000.0f);
    config.swa_pattern = 6;
    config.dim = get_gguf_int(gguf_file, K("embedding_length"), 4096);
    config.hidden_dim = get_gguf_int(gguf_file, K("feed_forward_length"), 11008);
    config.n_layers = get_gguf_int(gguf_file, K("block_count"), 32);
    config.n_heads = get_gguf_int(gguf_file, K("attention.head_count"), 32);
    config.n_kv_heads = get_gguf_int(gguf_file, K("attention.head_count_kv"), config.n_heads);
    config.vocab_size = get_gguf_int(gguf_file, K("vocab_size"), 32000);
    config.seq_len = get_gguf_int(gguf_file, K("context_length"), 2048);
    config.rope_theta = get_gguf_float(gguf_file, K("rope.freq_base"), config.is_gemma3 ? 1000000.0f : 500000.0f);
    config.head_dim = get_gguf_int(gguf_file, K("attention.key_length"), config.dim / config.n_heads);
    config.rms_norm_eps = get_gguf_float(gguf_file, K("attention.layer_norm_rms_epsilon"), 1e-6f);
    config.final_logit_softcapping = get_gguf_float(gguf_file, K("final_logit_softcapping"), 0.0f);
#undef K
    if (gguf_file->vocab_size > 0 && (int64_t)config.vocab_size != (int64_t)gguf_file->vocab_size)
        config.vocab_size = (int)gguf_file->vocab_size;
    if (!init_weights_from_gguf(gguf_file, &config, &weights)) return -3;
    if (!init_tokenizer_from_gguf(gguf_file, &config)) return -4;
    if (ctx > 0 && ctx < config.seq_len) config.seq_len = ctx;
    malloc_run_state(&state, &config);
    int hs = config.head_dim > 0 ? config.head_dim : config.dim / config.n_heads;
    int mx = config.dim;
    if (config.n_heads * hs > mx) mx = config.n_heads * hs;
    if (config.hidden_dim > mx) mx = config.hidden_dim;
    ensure_bufs(mx);
    top_k_idx_buf = (int*)calloc(config.vocab_size, sizeof(int));
    top_k_val_buf = (float*)calloc(config.vocab_size, sizeof(float));
    tokenizer.eot_token = config.is_gemma3 ? GEMMA3_END_TURN : LLAMA3_EOT;
    return 0;
}

void ref_forward(int tok, int p, int compute_logits, float* logits) {
    transformer(tok, p, &config, &state, &weights, compute_logits);
    if (compute_logits && logits) memcpy(logits, state.logits, (size_t)config.vocab_size * sizeof(float));
}

void ref_prefill(int* tokens, int start, int bs) {
    transformer_prefill(tokens, start, bs, &config, &state, &weights);
}

int ref_copy_kv(int layer, int which_v, void* dst, size_t cap) {
    size_t n = state.kv_cache_layer_size;
    if (cap < n) return -1;
    memcpy(dst, (which_v ? state.value_cache : state.key_cache) + (size_t)layer * n, n);
    return 0;
}

/* Harness-side test support (the engine has no such entry point): overwrite
 * one layer's K or V cache with exactly kv_cache_layer_size bytes, so a long
 * context written elsewhere can be installed before decode steps. */
int ref_set_kv(int layer, int which_v, const void* src, size_t n) {
    if (layer < 0 || layer >= config.n_layers || n != state.kv_cache_layer_size) return -1;
    memcpy((which_v ? state.value_cache : state.key_cache) + (size_t)layer * n, src, n);
    return 0;
}

void ref_rope_row(int swa, int p, float* c, float* s) {
    int half = state.head_size / 2;
    memcpy(c, (swa ? state.rope_cos_swa_all : state.rope_cos_all) + (size_t)p * half, half * sizeof(float));
    memcpy(s, (swa ? state.rope_sin_swa_all : state.rope_sin_all) + (size_t)p * half, half * sizeof(float));
}

void ref_copy_x(float* dst) { memcpy(dst, state.x, (size_t)config.dim * sizeof(float)); }

/* One call of generate_token() (c:4766-4971) in the sampling phase:
 * forward at (tok, p), then the reference's own sampler with the given
 * settings and xorshift64* state.  Returns the sampled id and the RNG state
 * after the draw. */
int ref_generate_token(int tok, int p, float temp, int topk, float topp, unsigned long long* seed) {
    token = tok;
    pos = p;
    num_prompt_tokens = 1;          /* every position is past the prompt */
    temperature = temp;
    top_k = topk;
    top_p = topp;
    rng_seed = *seed;
    generate_token();
    *seed = rng_seed;
    return next;
}
