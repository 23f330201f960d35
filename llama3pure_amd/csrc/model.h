// model.h — device-resident model, run state and the context object.
#pragma once

#include "internal.h"

// Floats per attention chunk partial: the chunk's hs outputs, its softmax
// max and sum, padded so that every partial starts 16-byte aligned.
constexpr int attn_part_row(int hs) { return hs + 4; }

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

struct Model {
    // config (Config, c:201-219)
    int dim = 0, hidden = 0, n_layers = 0, n_heads = 0, n_kv = 0, vocab = 0, seq_len = 0;
    int hs = 0, kv_dim = 0, q_dim = 0, max_dim = 0, kv_mul = 0, hq8 = 0;
    int is_gemma = 0, swa_window = 0, swa_pattern = 6, weight_type = 0;
    float theta = 0, theta_swa = 0, eps = 0, softcap = 0;
    float attn_softcap = 0;   // load option: attention score cap (0: none)
    float attn_scale = 0, embed_scale = 0, inv_dim = 0, inv_hs = 0;
    size_t head_seq = 0, layer_kv = 0;

    std::vector<void*> allocs;
    int64_t device_bytes = 0;

    Mat emb, wcls;
    float* final_norm = nullptr;
    std::vector<Layer> layers;
    uint8_t *kc = nullptr, *vc = nullptr;
    float *cos_d = nullptr, *sin_d = nullptr, *cos_s = nullptr, *sin_s = nullptr;
    float* rope_cur = nullptr;     // [cos_d, sin_d, cos_s, sin_s][hs/2]: rows of the decode step's position

    // run state (RunState, c:281-343), device resident
    float *x = nullptr, *x2 = nullptr, *xb = nullptr, *xb2 = nullptr, *q = nullptr, *k = nullptr, *v = nullptr;
    // the residual times the next RMSNorm's weights and the sums of squares of
    // the FFN residual add's workgroups (see layers_impl)
    float *xw = nullptr, *ssp = nullptr;
    float *hb = nullptr, *hb2 = nullptr, *logits = nullptr;
    float* part_acc = nullptr;     // [n_heads][max_chunks][attn_part_row(hs)] attention chunk partials
    int* step = nullptr;           // device {token, pos} of the step being computed
    // prompt-batch rows (transformer_prefill's batch_* arrays, c:326-343),
    // allocated at the first batched prefill for pf_rows tokens
    int pf_rows = 0;
    float *pf_x = nullptr, *pf_xb = nullptr, *pf_xb2 = nullptr, *pf_q = nullptr, *pf_k = nullptr, *pf_v = nullptr;
    float *pf_att = nullptr, *pf_hb = nullptr, *pf_hb2 = nullptr;
    int *pf_tok = nullptr, *pf_steps = nullptr;
    float* pf_part = nullptr;      // attention chunk partials of a batch's tokens
    size_t pf_part_cap = 0;        // floats
    int max_chunks = 0;            // decode attention chunk slots per head
    int dec_tc = 64;               // positions per decode attention chunk
    // sampler scratch
    float* cand_val = nullptr;     // device: group maxima, then top-k slot values
    int* cand_idx = nullptr;       // device: top-k slot indices
    int* out_token = nullptr;      // device
    int* out_token_host = nullptr; // pinned
    float* slot_val_host = nullptr;   // pinned, top-k slot values
    int* slot_idx_host = nullptr;     // pinned, top-k slot indices

    void* dalloc(size_t bytes);
    ~Model();
};

// Per-kernel timing of the GEMV launches of a forward step, with HIP events
// recorded on the launching stream around each launch.
struct Profiler {
    bool on = false;
    struct Stat {
        std::string name;
        int64_t launches = 0;
        double ms = 0.0;
        double bytes = 0.0;   // algorithmic bytes per launch
        std::vector<float> each;   // every launch's duration (ms)
    };
    struct Pending {
        int stat;
        hipEvent_t a, b;
    };
    std::vector<Stat> stats;
    std::vector<Pending> pending;
    std::vector<hipEvent_t> pool;

    hipEvent_t event();
    int stat(const std::string& name, double bytes);
    void reset();                    // drops stats, keeps the event pool
    void collect();                  // after the stream has drained
    void release();
};

// RAII range around one launch: records a start event on construction and an
// end event on destruction when profiling is on.
struct ProfRange {
    Profiler* p = nullptr;
    int st = -1;
    hipEvent_t a{}, b{};
    hipStream_t s{};
    KernelEvents outer;   // the enclosing range's launch events
    ProfRange(Profiler& pr, hipStream_t stream, const std::string& name, double bytes);
    ~ProfRange();
};

struct l3p_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    Model* model = nullptr;
    Profiler prof;
    // the layer stack of one forward step, captured once per variant
    // (index: with logits) and replayed; dropped when the model changes
    // decode graphs by variant: bit 0 logits, bit 1 per-head attention
    hipGraphExec_t graph[4] = {nullptr, nullptr, nullptr, nullptr};
    hipStream_t cap_stream = nullptr;   // idle stream the graphs are captured on (made on first use)
    int graph_runs[4] = {0, 0, 0, 0};
    bool attn_per_head = false;   // the attention of the step being recorded
    // split-K partials of the prefill GEMM (allocated with the context, so
    // no GEMM call allocates)
    float* gemm_ws = nullptr;
    size_t gemm_ws_floats = 0;
    // l3p_generate_greedy: pinned token slots and their events (made on first use)
    static constexpr int kGenSlots = 4;
    int* gen_host = nullptr;
    hipEvent_t gen_ev[kGenSlots] = {};
    // l3p_generate_sampled: coherent pinned memory (made on first use) for
    // the top-k slots each step publishes ([kGenSlots][max k] values and
    // indices, then a sequence word per slot), the tokens the host hands back
    // ((seq << 32) | token per slot) and the device's wait-failure word
    float* smp_v = nullptr;
    int* smp_i = nullptr;
    uint32_t* smp_seq = nullptr;
    uint64_t* smp_tok = nullptr;
    uint32_t* smp_fail = nullptr;
    uint32_t smp_next = 1;   // next sequence number (never 0: the words start at 0)
    void drop_graphs();
};

// y = W . x through the fastest kernel for the type (model.cpp)
void gemv_plain(l3p_ctx* c, int type, const GemvBatch& b, int cols, const float* x);

// layers.hip
// m.x = embedding row of `token` (times Gemma's scale), the device step record
// {token, pos} that the layer kernels read and the RoPE rows of pos (m.rope_cur).
// With dtok the token is read from device memory when the kernel runs.
// With ht.word the token is the host's, waited for on the device (HostToken).
void launch_embed_step(const Model& m, int token, int pos, hipStream_t s, const int* dtok = nullptr,
                       HostToken ht = HostToken{});
// QK-norm, RoPE, the K/V cache write and attention of one layer for the
// step's position (c:3232-3359); out = [n_heads][head_dim].  The first form
// reads the decode step's q, k, v and step record.
struct AttnIO {
    const float *q, *k, *v;   // this token's projections
    const int* step;          // device {token, pos}
    float* out;
};
// per_head: one workgroup per query head (attention_per_head(m, pos) says
// whether the step at pos may take it); else split-position chunks + merge.
bool attention_per_head(const Model& m, int pos);
// positions below which attention_per_head picks the per-head kernel
int attention_head_limit(const Model& m);
void launch_attention(const Model& m, int layer, float* out, bool per_head, hipStream_t s);
void launch_attention(const Model& m, int layer, const AttnIO& io, bool per_head, hipStream_t s);
// Attention of `tokens` consecutive prompt tokens of a batch in three
// launches (K/V rows of all of them, then chunks and merge): io holds token
// 0's rows, token z's are `*_stride` floats further and its step record 2z
// ints further; last_pos is the last token's position.  part holds
// part_cap floats of chunk partials.
int attention_chunks(const Model& m, int layer, int last_pos);
void launch_attention_rows(const Model& m, int layer, const AttnIO& io, int q_stride, int kv_stride, int out_stride,
                           int tokens, int last_pos, float* part, size_t part_cap, hipStream_t s);
// rows of a prompt batch (row strides ld*)
void launch_rmsnorm_add_rows(const float* y, int ldy, const float* w, int n, float inv_n, float eps, float* x,
                             int ldx, int rows, hipStream_t s);
void launch_embed_rows(const Mat& emb, const int* tokens, int rows, int start, float scale, float* x, int ldx,
                       int* steps, hipStream_t s);
void launch_rmsnorm_rows(const float* x, int ldx, const float* w, int n, float inv_n, float eps, float* o, int ldo,
                         int rows, hipStream_t s);
void launch_act_rows(float* h, const float* h2, int64_t n, bool gelu, hipStream_t s);
void launch_softcap(float* logits, int n, float cap, hipStream_t s);
void launch_argmax(const float* logits, int n, int* out, hipStream_t s, float* cv, int* ci);
// with pub.v the slots also go to pinned host memory (HostSlots)
void launch_topk_slots(const float* logits, int n, int k, float* gmax, float* out_v, int* out_i, hipStream_t s,
                       HostSlots pub = HostSlots{});
int sample_groups(int n);
int sample_max_k();

// model.cpp
void run_stream_read(l3p_ctx* c, const void* p, size_t bytes);
void run_gemm(l3p_ctx* c, int type, const uint8_t* w, int rows, int cols, const float* x, int batch, int in_stride,
              float* y, int out_stride);
