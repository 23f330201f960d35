// model.h — device-resident model, run state and the context object.
#pragma once

#include "internal.h"

struct DevBuf {
    void* p = nullptr;
    size_t cap = 0;
    void ensure(size_t n);
    void release();
    ~DevBuf() { release(); }
};

struct Scratch {
    DevBuf xq_buf, gemm_buf;
    XQ8 xq(int cols);
    void release();
};

// One weight matrix in HBM, native GGUF block layout (QuantizedTensor, c:238-249).
struct Mat {
    const uint8_t* w = nullptr;
    int type = 0, rows = 0, cols = 0;
    size_t rb = 0;
};

struct Layer {
    Mat wq, wk, wv, wo, w1, w2, w3;
    float *att_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    float *post_att = nullptr, *post_ffn = nullptr;
};

// Attention launch parameters shared by the attention kernels.
struct AttnArgs {
    const int8_t* qq;      // [n_heads][hs] Q8_0 query quants
    const float* qd;       // [n_heads][hs/32] their scales (fp32 value of the fp16 scale)
    const uint8_t* kc;     // layer base of the K cache [n_kv][seq][hq8]
    const uint8_t* vc;     // layer base of the V cache
    float* att;            // [n_heads][seq] scores, then exp
    float* part_acc;       // [n_heads][max_chunks][hs] chunk outputs
    unsigned* counters;    // [n_heads] combine counters (kept at zero between calls)
    float* out;            // [n_heads][hs]
    int n_heads, kv_mul, hs, hq8, seq, t0, na, n_chunks;
    size_t head_seq;
};

struct Model {
    // config (Config, c:201-219)
    int dim = 0, hidden = 0, n_layers = 0, n_heads = 0, n_kv = 0, vocab = 0, seq_len = 0;
    int hs = 0, kv_dim = 0, q_dim = 0, max_dim = 0, kv_mul = 0, hq8 = 0;
    int is_gemma = 0, swa_window = 0, swa_pattern = 6, weight_type = 0;
    float theta = 0, theta_swa = 0, eps = 0, softcap = 0;
    float attn_scale = 0, embed_scale = 0, inv_dim = 0, inv_hs = 0;
    size_t head_seq = 0, layer_kv = 0;

    std::vector<void*> allocs;
    int64_t device_bytes = 0;

    Mat emb, wcls;
    float* final_norm = nullptr;
    std::vector<Layer> layers;
    uint8_t *kc = nullptr, *vc = nullptr;
    float *cos_d = nullptr, *sin_d = nullptr, *cos_s = nullptr, *sin_s = nullptr;

    // run state (RunState, c:281-343), device resident
    float *x = nullptr, *xb = nullptr, *xb2 = nullptr, *q = nullptr, *k = nullptr, *v = nullptr;
    float *hb = nullptr, *hb2 = nullptr, *logits = nullptr;
    int8_t* qq = nullptr;          // Q8_0 query [n_heads][hs]
    float* qd = nullptr;           // [n_heads][hs/32]
    XQ8 xq{};
    float *att = nullptr, *part_acc = nullptr;
    unsigned* counters = nullptr;
    int max_chunks = 0;
    // sampler scratch
    float* cand_val = nullptr;
    int* cand_idx = nullptr;
    int* out_token = nullptr;      // device
    int* out_token_host = nullptr; // pinned

    void* dalloc(size_t bytes);
    ~Model();
};

struct l3p_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    Scratch scratch;
    Model* model = nullptr;
};

// layers.hip
void launch_embed(const Mat& emb, int token, float* x, hipStream_t s);
void launch_rmsnorm(const float* x_in, float* x_scale_inplace, float scale, const float* w, int n, float inv_n,
                    float eps, float* out, const XQ8* xq, hipStream_t s);
void launch_rmsnorm_add(const float* y, const float* w, int n, float inv_n, float eps, float* x, hipStream_t s);
void launch_rope_kv(const Model& m, int layer, int pos, hipStream_t s);
void launch_attention(const AttnArgs& a, hipStream_t s);
void launch_softcap(float* logits, int n, float cap, hipStream_t s);
void launch_argmax(const float* logits, int n, int* out, hipStream_t s, float* cv, int* ci);
void launch_sample_topk(const float* logits, int n, float temperature, int top_k, float top_p, float r,
                        float* cand_val, int* cand_idx, int* out, hipStream_t s);
int sample_candidates_per_block();
int sample_num_blocks(int n);

// model.cpp
void run_gemm(l3p_ctx* c, int type, const uint8_t* w, int rows, int cols, const float* x, int batch, int in_stride,
              float* y, int out_stride);
