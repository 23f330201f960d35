// model.cpp — GGUF upload, the decode/prefill orchestration and the model
// entry points of the C-ABI (include/l3p.h).
//
// Layer order and per-step arithmetic follow transformer() and
// transformer_prefill() of llama3pure-c-engine.c (c:3190-3680); each device
// launch below names the reference lines it replaces.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <initializer_list>
#include <memory>
#include <new>
#include <string>

#include "model.h"

// ---------------------------------------------------------------------------
// Model memory
// ---------------------------------------------------------------------------
void* Model::dalloc(size_t bytes) {
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 16);
    if (e != hipSuccess) (void)hipGetLastError();   // consumed here: later launch checks must not see it
    if (e == hipErrorOutOfMemory) throw L3pError{L3P_E_NOMEM, "model: out of device memory"};
    L3P_HIP(e);
    allocs.push_back(p);
    device_bytes += (int64_t)bytes;
    return p;
}

Model::~Model() {
    for (void* p : allocs) hipFree(p);
    if (out_token_host) hipHostFree(out_token_host);
    if (slot_val_host) hipHostFree(slot_val_host);
    if (slot_idx_host) hipHostFree(slot_idx_host);
}

// ---------------------------------------------------------------------------
// GGUF parsing (format as read by parse_gguf_file, c:2500-2688)
// ---------------------------------------------------------------------------
namespace {

struct Reader {
    const uint8_t* p;
    const uint8_t* end;
    uint64_t u(int n) {
        L3P_REQUIRE(end - p >= n, L3P_E_FORMAT, "GGUF: truncated");
        uint64_t v = 0;
        for (int i = 0; i < n; ++i) v |= (uint64_t)p[i] << (8 * i);
        p += n;
        return v;
    }
    std::string str() {
        uint64_t n = u(8);
        L3P_REQUIRE((uint64_t)(end - p) >= n, L3P_E_FORMAT, "GGUF: truncated string");
        std::string s((const char*)p, n);
        p += n;
        return s;
    }
    void skip(uint32_t type) {
        static const int sz[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
        if (type == 8) { str(); return; }
        if (type == 9) {
            uint32_t at = (uint32_t)u(4);
            uint64_t n = u(8);
            if (at != 8 && at != 9 && at < 13) {
                uint64_t bytes = n * (uint64_t)sz[at];
                L3P_REQUIRE((uint64_t)(end - p) >= bytes, L3P_E_FORMAT, "GGUF: truncated array");
                p += bytes;
                return;
            }
            for (uint64_t i = 0; i < n; ++i) skip(at);
            return;
        }
        L3P_REQUIRE(type < 13 && sz[type] > 0, L3P_E_FORMAT, "GGUF: unknown value type %u", type);
        u(sz[type]);
    }
};

struct KV {
    std::string key;
    uint32_t type;
    const uint8_t* val;
    uint64_t alen = 0;
    uint32_t atype = 0;
};
struct TI {
    std::string name;
    uint32_t ndim;
    uint64_t ne[4];
    uint32_t type;
    uint64_t off;
};

struct Gguf {
    std::vector<KV> kv;
    std::vector<TI> ti;
    const uint8_t* data = nullptr;
    size_t data_len = 0;

    const KV* find(const std::string& k) const {
        for (const auto& e : kv)
            if (e.key == k) return &e;
        return nullptr;
    }
    // get_gguf_int / get_gguf_float / get_gguf_string (c:2447-2497)
    int64_t geti(const std::string& k, int64_t d) const {
        const KV* e = find(k);
        if (!e) return d;
        const uint8_t* v = e->val;
        switch (e->type) {
        case 0: return v[0];
        case 1: return (int8_t)v[0];
        case 2: { uint16_t x; memcpy(&x, v, 2); return x; }
        case 3: { int16_t x; memcpy(&x, v, 2); return x; }
        case 4: { uint32_t x; memcpy(&x, v, 4); return x; }
        case 5: { int32_t x; memcpy(&x, v, 4); return x; }
        case 10: { uint64_t x; memcpy(&x, v, 8); return (int64_t)x; }
        case 11: { int64_t x; memcpy(&x, v, 8); return x; }
        default: return d;
        }
    }
    float getf(const std::string& k, float d) const {
        const KV* e = find(k);
        if (!e) return d;
        if (e->type == 6) { float x; memcpy(&x, e->val, 4); return x; }
        if (e->type == 12) { double x; memcpy(&x, e->val, 8); return (float)x; }
        return d;
    }
    std::string gets(const std::string& k) const {
        const KV* e = find(k);
        if (!e || e->type != 8) return "";
        uint64_t n;
        memcpy(&n, e->val, 8);
        return std::string((const char*)e->val + 8, n);
    }
    const TI* tensor(const std::string& n) const {
        for (const auto& t : ti)
            if (t.name == n) return &t;
        return nullptr;
    }
};

Gguf parse(const void* bytes, size_t len) {
    Gguf g;
    Reader r{(const uint8_t*)bytes, (const uint8_t*)bytes + len};
    L3P_REQUIRE(len >= 24, L3P_E_FORMAT, "GGUF: file too small");
    uint32_t magic = (uint32_t)r.u(4);
    L3P_REQUIRE(magic == 0x46554747u, L3P_E_FORMAT, "Invalid GGUF magic: expected 0x46554747, got 0x%X", magic);
    uint32_t ver = (uint32_t)r.u(4);
    L3P_REQUIRE(ver >= 2 && ver <= 3, L3P_E_FORMAT, "Unsupported GGUF version: %u", ver);
    uint64_t nt = r.u(8), nkv = r.u(8);
    L3P_REQUIRE(nt < (1u << 24) && nkv < (1u << 24), L3P_E_FORMAT, "GGUF: implausible counts");
    g.kv.reserve(nkv);
    for (uint64_t i = 0; i < nkv; ++i) {
        KV e;
        e.key = r.str();
        e.type = (uint32_t)r.u(4);
        e.val = r.p;
        if (e.type == 9) {
            Reader a = r;
            e.atype = (uint32_t)a.u(4);
            e.alen = a.u(8);
        }
        r.skip(e.type);
        g.kv.push_back(std::move(e));
    }
    g.ti.reserve(nt);
    for (uint64_t i = 0; i < nt; ++i) {
        TI t;
        t.name = r.str();
        t.ndim = (uint32_t)r.u(4);
        L3P_REQUIRE(t.ndim >= 1 && t.ndim <= 4, L3P_E_FORMAT, "GGUF: tensor %s has %u dims", t.name.c_str(), t.ndim);
        for (int d = 0; d < 4; ++d) t.ne[d] = 1;
        for (uint32_t d = 0; d < t.ndim; ++d) t.ne[d] = r.u(8);
        t.type = (uint32_t)r.u(4);
        t.off = r.u(8);
        g.ti.push_back(std::move(t));
    }
    const uint64_t align = (uint64_t)g.geti("general.alignment", 32);   // c:2617-2621
    L3P_REQUIRE(align > 0, L3P_E_FORMAT, "GGUF: zero alignment");
    const uint64_t hdr = (uint64_t)(r.p - (const uint8_t*)bytes);
    const uint64_t doff = (hdr + align - 1) / align * align;
    L3P_REQUIRE(doff <= len, L3P_E_FORMAT, "GGUF: truncated before tensor data");
    g.data = (const uint8_t*)bytes + doff;
    g.data_len = len - doff;
    for (const auto& t : g.ti) {
        const int be = type_block_elems((int)t.type);
        L3P_REQUIRE(be > 0, L3P_E_UNSUPPORTED, "Unsupported quantization type: %u (tensor %s)", t.type, t.name.c_str());
        const uint64_t ne = t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
        const uint64_t bytes_t = ne / be * type_block_bytes((int)t.type);
        L3P_REQUIRE(t.off <= g.data_len && bytes_t <= g.data_len - t.off, L3P_E_FORMAT,
                    "GGUF: tensor %s data out of file", t.name.c_str());
    }
    return g;
}

uint64_t tensor_bytes(const TI& t) {
    const uint64_t ne = t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
    return ne / type_block_elems((int)t.type) * type_block_bytes((int)t.type);
}

// RoPE tables exactly as malloc_run_state builds them (c:381-422), with the
// host C library's powf / cosf / sinf.  Called through pointers so the
// compiler cannot fuse or constant-fold them.
float (*volatile p_powf)(float, float) = powf;
float (*volatile p_cosf)(float) = cosf;
float (*volatile p_sinf)(float) = sinf;

void rope_tables(int seq, int hs, float theta, std::vector<float>& c, std::vector<float>& s) {
    const int half = hs / 2;
    std::vector<float> fr(half);
    for (int i = 0; i < half; ++i) fr[i] = 1.0f / p_powf(theta, (float)(i * 2) / (float)hs);
    c.resize((size_t)seq * half);
    s.resize((size_t)seq * half);
    for (int p = 0; p < seq; ++p)
        for (int i = 0; i < half; ++i) {
            volatile float val = p * fr[i];
            c[(size_t)p * half + i] = p_cosf(val);
            s[(size_t)p * half + i] = p_sinf(val);
        }
}

// q8_func && !deq_func (c:2091-2133, c:3221): the activation goes to Q8_0
bool q8_class(int t) {
    return t == L3P_Q4_0 || t == L3P_Q4_1 || t == L3P_Q5_0 || t == L3P_Q5_1 || t == L3P_IQ4_NL;
}

}  // namespace

// ---------------------------------------------------------------------------
// load
// ---------------------------------------------------------------------------
static Model* load_model(l3p_ctx* c, const void* bytes, size_t len, const l3p_load_opts* opts) {
    Gguf g = parse(bytes, len);
    std::unique_ptr<Model> mp(new Model());
    Model& m = *mp;

    // config, as main() reads it (c:5049-5182)
    const std::string arch = g.gets("general.architecture");
    m.is_gemma = arch == "gemma3" || arch == "gemma2" || arch == "gemma";
    std::string pre = "llama";
    if (m.is_gemma) {
        pre = "gemma3";
        if (g.geti("gemma3.embedding_length", 0) == 0) {
            if (g.geti("gemma2.embedding_length", 0) != 0) pre = "gemma2";
            else if (g.geti("gemma.embedding_length", 0) != 0) pre = "gemma";
        }
    }
    auto K = [&](const char* s) { return pre + "." + s; };
    m.swa_window = (int)g.geti(K("attention.sliding_window"), 0);
    m.theta_swa = g.getf(K("rope.freq_base_swa"), 10000.0f);
    m.swa_pattern = 6;
    m.dim = (int)g.geti(K("embedding_length"), 4096);
    m.hidden = (int)g.geti(K("feed_forward_length"), 11008);
    m.n_layers = (int)g.geti(K("block_count"), 32);
    m.n_heads = (int)g.geti(K("attention.head_count"), 32);
    m.n_kv = (int)g.geti(K("attention.head_count_kv"), m.n_heads);
    m.vocab = (int)g.geti(K("vocab_size"), 32000);
    m.seq_len = (int)g.geti(K("context_length"), 2048);
    m.theta = g.getf(K("rope.freq_base"), m.is_gemma ? 1000000.0f : 500000.0f);
    L3P_REQUIRE(m.n_heads > 0, L3P_E_FORMAT, "GGUF: head_count is 0");
    m.hs = (int)g.geti(K("attention.key_length"), m.dim / m.n_heads);
    m.eps = g.getf(K("attention.layer_norm_rms_epsilon"), 1e-6f);
    m.softcap = g.getf(K("final_logit_softcapping"), 0.0f);
    if (const KV* tk = g.find("tokenizer.ggml.tokens"))   // vocab from the token list (c:5152-5157)
        if (tk->type == 9 && tk->atype == 8 && tk->alen > 0) m.vocab = (int)tk->alen;
    if (opts && opts->context_size > 0 && opts->context_size < m.seq_len) m.seq_len = opts->context_size;
    if (opts) {
        L3P_REQUIRE(opts->swa_pattern >= 0 && opts->attn_softcap >= 0.0f && std::isfinite(opts->attn_softcap),
                    L3P_E_INVALID, "load: swa_pattern %d and attn_softcap %g must be finite and not negative",
                    opts->swa_pattern, (double)opts->attn_softcap);
        if (opts->swa_pattern > 0) m.swa_pattern = opts->swa_pattern;
        m.attn_softcap = opts->attn_softcap;
    }
    L3P_REQUIRE(m.seq_len <= 262144, L3P_E_UNSUPPORTED, "context length %d exceeds 262144", m.seq_len);

    L3P_REQUIRE(m.dim > 0 && m.hidden > 0 && m.n_layers > 0 && m.vocab > 0 && m.seq_len > 0, L3P_E_FORMAT,
                "GGUF: bad dimensions");
    L3P_REQUIRE(m.n_kv > 0 && m.n_heads % m.n_kv == 0, L3P_E_UNSUPPORTED, "n_heads %d not a multiple of n_kv %d",
                m.n_heads, m.n_kv);
    L3P_REQUIRE(m.hs % 32 == 0 && m.hs >= 32 && m.hs <= 256, L3P_E_UNSUPPORTED,
                "head_dim %d unsupported (need a multiple of 32 up to 256)", m.hs);
    L3P_REQUIRE(m.n_heads / m.n_kv <= 16, L3P_E_UNSUPPORTED, "GQA group of %d heads unsupported", m.n_heads / m.n_kv);
    m.kv_dim = m.n_kv * m.hs;
    m.q_dim = m.n_heads * m.hs;
    m.max_dim = std::max(m.dim, m.q_dim);
    m.kv_mul = m.n_heads / m.n_kv;
    m.hq8 = m.hs / 32 * 34;
    m.head_seq = (size_t)m.seq_len * m.hq8;
    m.layer_kv = (size_t)m.n_kv * m.head_seq;
    m.attn_scale = 1.0f / sqrtf((float)m.hs);
    m.embed_scale = sqrtf((float)m.dim);
    m.inv_dim = 1.0f / (float)m.dim;
    m.inv_hs = 1.0f / (float)m.hs;

    hipStream_t s = c->stream;
    auto upload_raw = [&](const TI& t) -> const uint8_t* {
        const uint64_t n = tensor_bytes(t);
        void* d = m.dalloc(n);
        L3P_HIP(hipMemcpyAsync(d, g.data + t.off, n, hipMemcpyHostToDevice, s));
        return (const uint8_t*)d;
    };
    auto mat = [&](const std::string& name, int rows, int cols, bool required = true) -> Mat {
        const TI* t = g.tensor(name);
        L3P_REQUIRE(t || !required, L3P_E_FORMAT, "tensor not found: %s", name.c_str());
        Mat M;
        if (!t) return M;
        L3P_REQUIRE(t->ne[0] == (uint64_t)cols && t->ne[1] * t->ne[2] * t->ne[3] == (uint64_t)rows, L3P_E_FORMAT,
                    "tensor %s: expected %d x %d", name.c_str(), rows, cols);
        M.w = upload_raw(*t);
        M.type = (int)t->type;
        M.rows = rows;
        M.cols = cols;
        M.rb = type_row_bytes(M.type, cols);
        return M;
    };
    // norms become fp32 on the device (load_tensor_float, c:2838-2869)
    auto vec = [&](const std::string& name, int n) -> float* {
        const TI* t = g.tensor(name);
        L3P_REQUIRE(t, L3P_E_FORMAT, "tensor not found: %s", name.c_str());
        L3P_REQUIRE(t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3] == (uint64_t)n, L3P_E_FORMAT, "tensor %s: expected %d values",
                    name.c_str(), n);
        float* d = (float*)m.dalloc((size_t)n * 4);
        if (t->type == L3P_F32) {
            L3P_HIP(hipMemcpyAsync(d, g.data + t->off, (size_t)n * 4, hipMemcpyHostToDevice, s));
        } else {
            const uint8_t* raw = upload_raw(*t);
            launch_dequant((int)t->type, raw, n, d, s);
        }
        return d;
    };

    const TI* te = g.tensor("token_embd.weight");
    L3P_REQUIRE(te, L3P_E_FORMAT, "Failed to load token embeddings");
    m.emb = mat("token_embd.weight", m.vocab, m.dim);
    m.layers.resize(m.n_layers);
    for (int l = 0; l < m.n_layers; ++l) {
        Layer& L = m.layers[l];
        const std::string p = "blk." + std::to_string(l) + ".";
        L.att_norm = vec(p + "attn_norm.weight", m.dim);
        L.ffn_norm = vec(p + "ffn_norm.weight", m.dim);
        L.wq = mat(p + "attn_q.weight", m.q_dim, m.dim);
        L.wk = mat(p + "attn_k.weight", m.kv_dim, m.dim);
        L.wv = mat(p + "attn_v.weight", m.kv_dim, m.dim);
        L.wo = mat(p + "attn_output.weight", m.dim, m.q_dim);
        L.w1 = mat(p + "ffn_gate.weight", m.hidden, m.dim);
        L.w2 = mat(p + "ffn_down.weight", m.dim, m.hidden);
        L.w3 = mat(p + "ffn_up.weight", m.hidden, m.dim);
        if (m.is_gemma) {
            L.q_norm = vec(p + "attn_q_norm.weight", m.hs);
            L.k_norm = vec(p + "attn_k_norm.weight", m.hs);
            L.post_att = vec(p + "post_attention_norm.weight", m.dim);
            L.post_ffn = vec(p + "post_ffw_norm.weight", m.dim);
        }
        const Mat* all[7] = {&L.wq, &L.wk, &L.wv, &L.wo, &L.w1, &L.w2, &L.w3};
        for (const Mat* M : all)
            L3P_REQUIRE(gemv_supported(M->type, M->cols), L3P_E_UNSUPPORTED,
                        "layer %d: weight type %d with %d columns not supported", l, M->type, M->cols);
        L3P_REQUIRE(q8_class(L.wq.type) == q8_class(L.wk.type) && q8_class(L.wq.type) == q8_class(L.wv.type) &&
                        q8_class(L.w1.type) == q8_class(L.w3.type) && L.w1.type == L.w3.type,
                    L3P_E_UNSUPPORTED, "layer %d: mixed activation-quantized and float-input weight types", l);
    }
    m.weight_type = m.layers[0].wq.type;
    m.final_norm = vec("output_norm.weight", m.dim);
    if (g.tensor("output.weight")) m.wcls = mat("output.weight", m.vocab, m.dim);
    else m.wcls = m.emb;                                           // tied (c:3064-3079)
    L3P_REQUIRE(gemv_supported(m.wcls.type, m.dim), L3P_E_UNSUPPORTED, "output weight type %d unsupported", m.wcls.type);
    L3P_REQUIRE(type_block_elems(m.emb.type) > 0, L3P_E_UNSUPPORTED, "embedding type unsupported");

    // KV cache, zeroed like calloc (c:365-372)
    // +64 bytes: the attention kernels read whole dwords around 34-byte
    // blocks, up to 4 bytes past the last row
    m.kc = (uint8_t*)m.dalloc((size_t)m.n_layers * m.layer_kv + 64);
    m.vc = (uint8_t*)m.dalloc((size_t)m.n_layers * m.layer_kv + 64);
    L3P_HIP(hipMemsetAsync(m.kc, 0, (size_t)m.n_layers * m.layer_kv, s));
    L3P_HIP(hipMemsetAsync(m.vc, 0, (size_t)m.n_layers * m.layer_kv, s));

    // RoPE tables
    {
        std::vector<float> cd, sd;
        rope_tables(m.seq_len, m.hs, m.theta, cd, sd);
        const size_t nbytes = cd.size() * 4;
        m.cos_d = (float*)m.dalloc(nbytes);
        m.sin_d = (float*)m.dalloc(nbytes);
        L3P_HIP(hipMemcpy(m.cos_d, cd.data(), nbytes, hipMemcpyHostToDevice));
        L3P_HIP(hipMemcpy(m.sin_d, sd.data(), nbytes, hipMemcpyHostToDevice));
        if (m.is_gemma) {
            rope_tables(m.seq_len, m.hs, m.theta_swa > 0 ? m.theta_swa : 10000.0f, cd, sd);
            m.cos_s = (float*)m.dalloc(nbytes);
            m.sin_s = (float*)m.dalloc(nbytes);
            L3P_HIP(hipMemcpy(m.cos_s, cd.data(), nbytes, hipMemcpyHostToDevice));
            L3P_HIP(hipMemcpy(m.sin_s, sd.data(), nbytes, hipMemcpyHostToDevice));
        } else {
            m.cos_s = m.cos_d;
            m.sin_s = m.sin_d;
        }
        m.rope_cur = (float*)m.dalloc((size_t)2 * m.hs * 4);
    }

    // run state
    m.x = (float*)m.dalloc((size_t)m.dim * 4);
    m.x2 = (float*)m.dalloc((size_t)m.dim * 4);
    m.xw = (float*)m.dalloc((size_t)m.dim * 4);
    m.ssp = (float*)m.dalloc((size_t)kMaxSsParts * 4);
    L3P_HIP(hipMemsetAsync(m.ssp, 0, (size_t)kMaxSsParts * 4, s));
    m.xb = (float*)m.dalloc((size_t)m.max_dim * 4);
    m.xb2 = (float*)m.dalloc((size_t)m.dim * 4);
    m.q = (float*)m.dalloc((size_t)m.q_dim * 4);
    m.k = (float*)m.dalloc((size_t)m.kv_dim * 4);
    m.v = (float*)m.dalloc((size_t)m.kv_dim * 4);
    m.hb = (float*)m.dalloc((size_t)m.hidden * 4);
    m.hb2 = (float*)m.dalloc((size_t)m.hidden * 4);
    m.logits = (float*)m.dalloc((size_t)m.vocab * 4);
    // decode attention chunks: 64 positions, 32 for head_dim >= 192 (their
    // chunk workgroups have the longest per-position work, so more and
    // shorter chunks run in parallel)
    m.dec_tc = m.hs >= 192 ? 32 : 64;
    m.max_chunks = (m.seq_len + m.dec_tc - 1) / m.dec_tc;
    m.part_acc = (float*)m.dalloc((size_t)m.n_heads * m.max_chunks * attn_part_row(m.hs) * 4);
    m.step = (int*)m.dalloc(4 * sizeof(int));
    const int ncand = std::max(256, sample_groups(m.vocab)) + sample_max_k();
    m.cand_val = (float*)m.dalloc((size_t)ncand * 4);
    m.cand_idx = (int*)m.dalloc((size_t)std::max(256, sample_max_k()) * 4);
    m.out_token = (int*)m.dalloc(16);
    L3P_HIP(hipHostMalloc((void**)&m.out_token_host, 16, hipHostMallocDefault));
    L3P_HIP(hipHostMalloc((void**)&m.slot_val_host, (size_t)sample_max_k() * 4, hipHostMallocDefault));
    L3P_HIP(hipHostMalloc((void**)&m.slot_idx_host, (size_t)sample_max_k() * 4, hipHostMallocDefault));
    L3P_HIP(hipStreamSynchronize(s));
    return mp.release();
}

// ---------------------------------------------------------------------------
// forward (transformer, c:3190-3435)
// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// GEMV launch timing
// ---------------------------------------------------------------------------
hipEvent_t Profiler::event() {
    if (!pool.empty()) {
        hipEvent_t e = pool.back();
        pool.pop_back();
        return e;
    }
    hipEvent_t e;
    L3P_HIP(hipEventCreate(&e));
    return e;
}
int Profiler::stat(const std::string& name, double bytes) {
    for (size_t i = 0; i < stats.size(); ++i)
        if (stats[i].name == name) return (int)i;
    Stat st;
    st.name = name;
    st.bytes = bytes;
    stats.push_back(st);
    return (int)stats.size() - 1;
}
void Profiler::collect() {
    for (const Pending& q : pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, q.a, q.b) == hipSuccess) {
            stats[q.stat].ms += ms;
            stats[q.stat].launches += 1;
            stats[q.stat].each.push_back(ms);
        }
        pool.push_back(q.a);
        pool.push_back(q.b);
    }
    pending.clear();
}
void Profiler::reset() {
    for (const Pending& q : pending) {
        pool.push_back(q.a);
        pool.push_back(q.b);
    }
    pending.clear();
    stats.clear();
}
void Profiler::release() {
    reset();
    for (hipEvent_t e : pool) hipEventDestroy(e);
    pool.clear();
}
KernelEvents& kernel_events() {
    static thread_local KernelEvents e;
    return e;
}

// The start event is recorded on the stream and offered to the range's
// first GEMV/GEMM launch, which records both events at the kernel's own start
// and end.  A range of one kernel thus times the kernel alone; one of several
// kernels (or none) ends with a stream record of the stop event.  Ranges nest:
// the enclosing range's state is restored at the end.
ProfRange::ProfRange(Profiler& pr, hipStream_t stream, const std::string& name, double bytes) {
    if (!pr.on) return;
    p = &pr;
    s = stream;
    st = pr.stat(name, bytes);
    a = pr.event();
    b = pr.event();
    L3P_HIP(hipEventRecord(a, s));
    outer = kernel_events();
    kernel_events() = KernelEvents{a, b, 0};
}
ProfRange::~ProfRange() {
    if (!p) return;
    const int launches = kernel_events().launches;   // direct launches: nested ranges keep their own
    kernel_events() = outer;
    if (launches == 1 || hipEventRecord(b, s) == hipSuccess) p->pending.push_back({st, a, b});
    else {
        p->pool.push_back(a);
        p->pool.push_back(b);
    }
}

static const char* type_name(int t) {
    switch (t) {
    case L3P_Q4_0: return "q4_0";
    case L3P_Q4_1: return "q4_1";
    case L3P_Q5_0: return "q5_0";
    case L3P_Q5_1: return "q5_1";
    case L3P_Q8_0: return "q8_0";
    case L3P_Q2_K: return "q2_k";
    case L3P_Q3_K: return "q3_k";
    case L3P_Q4_K: return "q4_k";
    case L3P_Q5_K: return "q5_k";
    case L3P_Q6_K: return "q6_k";
    case L3P_IQ4_NL: return "iq4_nl";
    case L3P_F16: return "f16";
    case L3P_BF16: return "bf16";
    case L3P_F32: return "f32";
    default: return "other";
    }
}

// Timing label "<type> gemv <what> <rows>x<cols>" and the algorithmic bytes of
// one launch: the weight blocks, the fp32 input and the fp32 outputs.
static std::string gemv_label(const char* what, int type, int rows, int cols) {
    char b[96];
    snprintf(b, sizeof b, "%s gemv %s %dx%d", type_name(type), what, rows, cols);
    return b;
}
static double gemv_bytes(int type, int rows, int cols, int out_rows) {
    return (double)rows * (double)type_row_bytes(type, cols) + 4.0 * cols + 4.0 * out_rows;
}

// b's segments = W . rmsnorm(x) (norm != null) or W . x, all of one type,
// in one launch of the streaming GEMV (the norm runs in its prologue).
static int gemv_batch(l3p_ctx* c, int type, const GemvBatch& b, int cols, const float* x, const float* norm,
                      const char* what) {
    Model& m = *c->model;
    hipStream_t s = c->stream;
    const float eps = m.eps > 0 ? m.eps : 1e-5f;   // c:3198
    int rows = 0;
    for (int i = 0; i < (b.pair ? 2 : b.nseg); ++i) rows += b.seg[i].rows;
    const int out_rows = b.pair ? b.seg[0].rows : rows;
    ProfRange r(c->prof, s, gemv_label(what, type, rows, cols), gemv_bytes(type, rows, cols, out_rows));
    return launch_gemv(type, b, cols, x, norm, eps, s);
}

void gemv_plain(l3p_ctx* c, int type, const GemvBatch& b, int cols, const float* x) {
    int rows = 0;
    for (int i = 0; i < b.nseg; ++i) rows += b.seg[i].rows;
    ProfRange r(c->prof, c->stream, gemv_label("plain", type, rows, cols), gemv_bytes(type, rows, cols, rows));
    launch_gemv(type, b, cols, x, nullptr, 0.0f, c->stream);
}

static GemvBatch one(const Mat& W, float* y, int epi) {
    GemvBatch b{};
    b.seg[0] = GemvSegment{W.w, y, W.rows};
    b.nseg = 1;
    b.epilogue = epi;
    return b;
}

// The layer stack and the classifier of one step (c:3209-3434).  Reads the
// token and position from the device step record only, so a capture of it
// replays for any position.
static void layers_impl(l3p_ctx* c, bool with_logits) {
    Model& m = *c->model;
    hipStream_t s = c->stream;
    // Gemma's post norms (x += rmsnorm(y) . w, c:3364-3371 and c:3411-3417)
    // run in the prologue of the next GEMV that reads x, which writes the
    // updated residual to the other of two buffers: `cur` is the residual,
    // `pending` the post norm not yet applied to it.
    float* cur = m.x;
    float* alt = m.x2;
    const float* pend_y = nullptr;
    const float* pend_w = nullptr;
    auto fold = [&](GemvBatch& b) {
        if (!pend_y) return;
        if (m.dim > kMaxPostCols) {   // too wide for the fused update: apply it in place first
            launch_rmsnorm_add_rows(pend_y, m.dim, pend_w, m.dim, m.inv_dim, m.eps > 0 ? m.eps : 1e-5f, cur, m.dim,
                                    1, s);
            pend_y = nullptr;
            return;
        }
        b.post_y = pend_y;
        b.post_w = pend_w;
        b.post_out = alt;
    };
    auto folded = [&]() {
        if (!pend_y) return;
        std::swap(cur, alt);
        pend_y = nullptr;
    };
    // Without post norms the FFN's residual add (down) also writes the
    // residual times the next RMSNorm's weights (m.xw) and its workgroups'
    // sums of squares (m.ssp), so that the next layer's q|k|v (or the
    // classifier) reads one vector and a few sums instead of the residual and
    // the weights; n_ss is the number of those sums (0: the next GEMV forms
    // its norm itself).  (wo's residual add does not: its 1024 workgroups'
    // sums cost gate|up more than the weights did.)
    auto produce = [&](GemvBatch& b, const float* next_norm, int next_type, float* ssp) {
        if (m.is_gemma || !gemv_fp32_activation(next_type)) return;
        b.xw = m.xw;
        b.xw_w = next_norm;
        b.ssp = ssp;
    };
    auto consume = [&](GemvBatch& b, int n_ss, const float* ssp, const float*& x, const float*& norm) {
        if (n_ss <= 0) return;
        b.ss = ssp;
        b.n_ss = n_ss;
        x = m.xw;
        norm = nullptr;
    };
    int n_ss = 0;   // sums in m.ssp for the next q|k|v (or the classifier)
    for (int l = 0; l < m.n_layers; ++l) {
        const Layer& L = m.layers[l];
        // q, k, v = W . rmsnorm(x) (c:3211-3230), one launch when the three share a type
        if (L.wq.type == L.wk.type && L.wq.type == L.wv.type) {
            GemvBatch b{};
            b.seg[0] = GemvSegment{L.wq.w, m.q, L.wq.rows};
            b.seg[1] = GemvSegment{L.wk.w, m.k, L.wk.rows};
            b.seg[2] = GemvSegment{L.wv.w, m.v, L.wv.rows};
            b.nseg = 3;
            b.epilogue = EPI_STORE;
            fold(b);
            const float* x = cur;
            const float* norm = L.att_norm;
            consume(b, n_ss, m.ssp, x, norm);
            gemv_batch(c, L.wq.type, b, m.dim, x, norm, "qkv");
        } else {
            // each launch forms the same updated residual from `cur`
            GemvBatch bq = one(L.wq, m.q, EPI_STORE), bk = one(L.wk, m.k, EPI_STORE), bv = one(L.wv, m.v, EPI_STORE);
            fold(bq);
            fold(bk);
            fold(bv);
            gemv_batch(c, L.wq.type, bq, m.dim, cur, L.att_norm, "q");
            gemv_batch(c, L.wk.type, bk, m.dim, cur, L.att_norm, "k");
            gemv_batch(c, L.wv.type, bv, m.dim, cur, L.att_norm, "v");
        }
        folded();
        // QK-norm, RoPE, KV write, Q quantization and attention (c:3232-3359)
        launch_attention(m, l, m.xb, c->attn_per_head, s);
        // output projection + residual (c:3362-3371)
        if (m.is_gemma) {
            gemv_batch(c, L.wo.type, one(L.wo, m.xb2, EPI_STORE), m.q_dim, m.xb, nullptr, "wo");
            pend_y = m.xb2;
            pend_w = L.post_att;
        } else {
            gemv_batch(c, L.wo.type, one(L.wo, cur, EPI_ADD), m.q_dim, m.xb, nullptr, "wo");
        }
        // FFN (c:3373-3417): gate/up with the norm and the activation fused
        {
            GemvBatch b{};
            b.seg[0] = GemvSegment{L.w1.w, m.hb, L.w1.rows};
            b.seg[1] = GemvSegment{L.w3.w, m.hb2, L.w3.rows};
            b.nseg = 2;
            b.pair = 1;
            b.epilogue = m.is_gemma ? EPI_GEGLU : EPI_SWIGLU;
            fold(b);
            gemv_batch(c, L.w1.type, b, m.dim, cur, L.ffn_norm, "gate|up");
            folded();
        }
        if (m.is_gemma) {
            gemv_batch(c, L.w2.type, one(L.w2, m.xb, EPI_STORE), m.hidden, m.hb, nullptr, "down");
            pend_y = m.xb;
            pend_w = L.post_ffn;
        } else {
            GemvBatch b = one(L.w2, cur, EPI_ADD);
            const bool last = l + 1 == m.n_layers;
            const Layer* N = last ? nullptr : &m.layers[l + 1];
            // the next layer's q|k|v takes the sums only as one launch
            const bool next_one = !last && N->wq.type == N->wk.type && N->wq.type == N->wv.type;
            if (next_one || (last && with_logits))
                produce(b, last ? m.final_norm : N->att_norm, last ? m.wcls.type : N->wq.type, m.ssp);
            n_ss = gemv_batch(c, L.w2.type, b, m.hidden, m.hb, nullptr, "down");
        }
    }
    // final rmsnorm (c:3420) fused into the classifier (c:3423-3433).  Without
    // logits the last post norm is dropped: the next step's embedding
    // overwrites the residual.
    if (with_logits) {
        GemvBatch b = one(m.wcls, m.logits, EPI_STORE);
        fold(b);
        const float* x = cur;
        const float* norm = m.final_norm;
        consume(b, n_ss, m.ssp, x, norm);
        gemv_batch(c, m.wcls.type, b, m.dim, x, norm, "lm_head");
        folded();
        if (m.is_gemma && m.softcap > 0.0f) launch_softcap(m.logits, m.vocab, m.softcap, s);
    }
}

// ---------------------------------------------------------------------------
// batched prefill (transformer_prefill, c:3439-3680)
// ---------------------------------------------------------------------------
// Prompt tokens per pass over the weights: 1024 rows give the GEMMs 16 tile
// rows (several workgroups per CU) and cost 218 MB of row buffers at
// Llama-3-8B's sizes.
static constexpr int kPrefillRows = 1024;

static void ensure_prefill_rows(Model& m) {
    if (m.pf_rows) return;
    const int R = kPrefillRows;
    auto f = [&](int n) { return (float*)m.dalloc((size_t)R * n * 4 + 64); };
    m.pf_x = f(m.dim);
    m.pf_xb = f(m.max_dim);
    m.pf_xb2 = f(m.dim);
    m.pf_q = f(m.q_dim);
    m.pf_k = f(m.kv_dim);
    m.pf_v = f(m.kv_dim);
    m.pf_att = f(m.q_dim);
    m.pf_hb = f(m.hidden);
    m.pf_hb2 = f(m.hidden);
    m.pf_tok = (int*)m.dalloc((size_t)R * 4);
    m.pf_steps = (int*)m.dalloc((size_t)R * 8);
    // partials for up to R tokens at the longest context, within 512 MB
    const size_t per_token = (size_t)m.n_heads * m.max_chunks * attn_part_row(m.hs);
    m.pf_part_cap = std::max(per_token, std::min(per_token * R, (size_t)128 << 20));
    m.pf_part = (float*)m.dalloc(m.pf_part_cap * 4);
    m.pf_rows = R;
}

static std::string gemm_label(const char* what, int type, int rows, int n, int k) {
    char b[112];
    snprintf(b, sizeof b, "%s gemm %s %dx%d b%d", type_name(type), what, n, k, rows);
    return b;
}

// One matrix of a prompt pass: W . x rows into y rows [rows][ldy].
struct RowsOut {
    const Mat* W;
    float* y;
    int ldy;
    const char* what;
};

// y rows (=|+=) W . x rows for `rows` prompt tokens, for one to three
// matrices over the same x rows.  Matrices of one type and width run as one
// GEMM launch (label `what`): the fp32 matrix-core GEMM for the types the
// reference dequantizes, the int8 one for the Q8_0-activation types (the
// reference's exact integer block dots, matmul_quantized_batch, c:2305-2318).
static bool gemm_capable(int type) { return gemm_mfma_supported(type) || gemm_q8_activation(type); }

static void gemm_rows(l3p_ctx* c, std::initializer_list<RowsOut> outs, const float* x, int ldx, int rows, bool add,
                      const char* what) {
    hipStream_t s = c->stream;
    const RowsOut* o = outs.begin();
    const int n = (int)outs.size();
    bool together = gemm_capable(o[0].W->type);
    for (int i = 1; i < n; ++i) together = together && o[i].W->type == o[0].W->type && o[i].W->cols == o[0].W->cols;
    if (together) {
        GemmJob j{};
        j.type = o[0].W->type;
        j.nseg = n;
        j.k = o[0].W->cols;
        j.x = x;
        j.m = rows;
        j.ldx = ldx;
        j.add = add;
        int ntot = 0;
        double bytes = 0.0;
        for (int i = 0; i < n; ++i) {
            j.seg[i] = GemmSegment{o[i].W->w, o[i].W->rows, o[i].y, o[i].ldy};
            ntot += o[i].W->rows;
            bytes += gemv_bytes(j.type, o[i].W->rows, j.k, o[i].W->rows);
        }
        ProfRange r(c->prof, s, gemm_label(n > 1 ? what : o[0].what, j.type, rows, ntot, j.k),
                    bytes + 4.0 * rows * (j.k + ntot));
        if (gemm_q8_activation(j.type)) launch_gemm_q8a(j, c->gemm_ws, c->gemm_ws_floats, s);
        else launch_gemm(j, c->gemm_ws, c->gemm_ws_floats, s);
        return;
    }
    for (int i = 0; i < n; ++i) {
        const Mat& W = *o[i].W;
        if (gemm_capable(W.type)) {
            gemm_rows(c, {o[i]}, x, ldx, rows, add, o[i].what);
            continue;
        }
        ProfRange r(c->prof, s, gemm_label(o[i].what, W.type, rows, W.rows, W.cols),
                    gemv_bytes(W.type, W.rows, W.cols, W.rows) + 4.0 * rows * (W.cols + W.rows));
        for (int b = 0; b < rows; ++b)
            launch_gemv(W.type, one(W, o[i].y + (size_t)b * o[i].ldy, add ? EPI_ADD : EPI_STORE), W.cols,
                        x + (size_t)b * ldx, nullptr, 0.0f, s);
    }
}

// Positions [start, start + n) of a prompt, kPrefillRows tokens per pass:
// the embedding, norm, projection and FFN work of a pass runs on all its rows
// (GEMMs read every weight once per pass).  Attention follows the reference's
// per-token order (c:3496-3612) in effect: the K/V rows of all the pass's
// tokens are written first, then every token attends to the positions up to
// its own, so each sees exactly the rows written before it.
static void prefill_batched(l3p_ctx* c, const int32_t* tokens, int n, int start) {
    Model& m = *c->model;
    hipStream_t s = c->stream;
    ensure_prefill_rows(m);
    const float eps = m.eps > 0 ? m.eps : 1e-5f;   // c:3198
    const int D = m.dim, QD = m.q_dim, KD = m.kv_dim, H = m.hidden, XB = m.max_dim;
    for (int b0 = 0; b0 < n; b0 += m.pf_rows) {
        const int R = std::min(m.pf_rows, n - b0);
        L3P_HIP(hipMemcpyAsync(m.pf_tok, tokens + b0, (size_t)R * 4, hipMemcpyHostToDevice, s));
        launch_embed_rows(m.emb, m.pf_tok, R, start + b0, m.is_gemma ? m.embed_scale : 0.0f, m.pf_x, D, m.pf_steps,
                          s);
        for (int l = 0; l < m.n_layers; ++l) {
            const Layer& L = m.layers[l];
            launch_rmsnorm_rows(m.pf_x, D, L.att_norm, D, m.inv_dim, eps, m.pf_xb, XB, R, s);
            gemm_rows(c, {{&L.wq, m.pf_q, QD, "q"}, {&L.wk, m.pf_k, KD, "k"}, {&L.wv, m.pf_v, KD, "v"}}, m.pf_xb, XB,
                      R, false, "q|k|v");
            // attention of the rows, as many tokens per launch as the partials hold
            const size_t per_token =
                (size_t)m.n_heads * attention_chunks(m, l, start + b0 + R - 1) * attn_part_row(m.hs);
            const int T = (int)std::max<size_t>(1, std::min<size_t>(R, m.pf_part_cap / per_token));
            for (int z0 = 0; z0 < R; z0 += T) {
                const int nz = std::min(T, R - z0);
                launch_attention_rows(m, l,
                                      AttnIO{m.pf_q + (size_t)z0 * QD, m.pf_k + (size_t)z0 * KD,
                                             m.pf_v + (size_t)z0 * KD, m.pf_steps + 2 * z0, m.pf_att + (size_t)z0 * QD},
                                      QD, KD, QD, nz, start + b0 + z0 + nz - 1, m.pf_part, m.pf_part_cap, s);
            }
            if (m.is_gemma) {
                gemm_rows(c, {{&L.wo, m.pf_xb2, D, "wo"}}, m.pf_att, QD, R, false, "wo");
                launch_rmsnorm_add_rows(m.pf_xb2, D, L.post_att, D, m.inv_dim, eps, m.pf_x, D, R, s);
            } else {
                gemm_rows(c, {{&L.wo, m.pf_x, D, "wo"}}, m.pf_att, QD, R, true, "wo");
            }
            launch_rmsnorm_rows(m.pf_x, D, L.ffn_norm, D, m.inv_dim, eps, m.pf_xb, XB, R, s);
            gemm_rows(c, {{&L.w1, m.pf_hb, H, "gate"}, {&L.w3, m.pf_hb2, H, "up"}}, m.pf_xb, XB, R, false, "gate|up");
            launch_act_rows(m.pf_hb, m.pf_hb2, (int64_t)R * H, m.is_gemma, s);
            if (m.is_gemma) {
                gemm_rows(c, {{&L.w2, m.pf_xb2, D, "down"}}, m.pf_hb, H, R, false, "down");
                launch_rmsnorm_add_rows(m.pf_xb2, D, L.post_ffn, D, m.inv_dim, eps, m.pf_x, D, R, s);
            } else {
                gemm_rows(c, {{&L.w2, m.pf_x, D, "down"}}, m.pf_hb, H, R, true, "down");
            }
        }
    }
}

void l3p_ctx::drop_graphs() {
    for (int i = 0; i < 4; ++i) {
        if (graph[i]) hipGraphExecDestroy(graph[i]);
        graph[i] = nullptr;
        graph_runs[i] = 0;
    }
}

// L3P_PREFILL_BATCH=0 runs prompts token by token through the decode step.
static bool prefill_batching() {
    static int on = -1;
    if (on < 0) {
        const char* e = getenv("L3P_PREFILL_BATCH");
        on = e ? atoi(e) != 0 : 1;
    }
    return on != 0;
}

static bool graphs_enabled() {
    static int on = -1;
    if (on < 0) {
        const char* e = getenv("L3P_GRAPH");
        on = e ? atoi(e) != 0 : 1;
    }
    return on != 0;
}

// One step of transformer() (c:3190-3435): the embedding row and the step
// record are written by an eager launch; the layers run as a replayed HIP
// graph from the second step of each variant on (the first, eager, step also
// settles every launch configuration).  Per-launch timing runs eagerly.
static void forward_impl(l3p_ctx* c, int token, int pos, bool with_logits, const int* dtok = nullptr,
                         HostToken ht = HostToken{}) {
    Model& m = *c->model;
    hipStream_t s = c->stream;
    launch_embed_step(m, token, pos, s, dtok, ht);
    c->attn_per_head = attention_per_head(m, pos);
    const int v = (with_logits ? 1 : 0) | (c->attn_per_head ? 2 : 0);
    if (c->prof.on || !graphs_enabled() || c->graph_runs[v]++ == 0) {
        layers_impl(c, with_logits);
        return;
    }
    if (!c->graph[v]) {
        // captured on an idle stream of its own, so that steps queued on the
        // context stream (which may wait for the host) need not drain first;
        // the layer launches take c->stream, which points there meanwhile
        if (!c->cap_stream) L3P_HIP(hipStreamCreateWithFlags(&c->cap_stream, hipStreamNonBlocking));
        hipStream_t cs = c->cap_stream;
        hipGraph_t g = nullptr;
        L3P_HIP(hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal));
        c->stream = cs;
        try {
            layers_impl(c, with_logits);
        } catch (...) {
            c->stream = s;
            hipStreamEndCapture(cs, &g);
            if (g) hipGraphDestroy(g);
            throw;
        }
        c->stream = s;
        L3P_HIP(hipStreamEndCapture(cs, &g));
        hipError_t e = hipGraphInstantiate(&c->graph[v], g, nullptr, nullptr, 0);
        hipGraphDestroy(g);
        L3P_HIP(e);
    }
    L3P_HIP(hipGraphLaunch(c->graph[v], s));
}

// xorshift64* (c:4266-4276)
static float rng_f32(uint64_t* st) {
    *st ^= *st >> 12;
    *st ^= *st << 25;
    *st ^= *st >> 27;
    const uint32_t u = (uint32_t)((*st * 0x2545F4914F6CDD1Dull) >> 32);
    return (u >> 8) / 16777216.0f;
}

// The reference's arithmetic on the k top-k slots, in slot order
// (c:4850-4907): temperature softmax with expf, stable insertion sort by
// probability when top_p < 1, the top-p cut, and one xorshift64* draw.  It runs
// on the host with the same C library expf as the reference, so given the same
// logits the chosen token is the reference's.
static int sample_slots(float* val, const int* idx, int k, float temperature, float top_p, uint64_t* rng) {
    const float inv_temp = 1.0f / temperature;
    float max_v = val[0];
    for (int i = 1; i < k; ++i)
        if (val[i] > max_v) max_v = val[i];
    const float max_vt = max_v * inv_temp;
    float sum = 0.0f;
    for (int i = 0; i < k; ++i) {
        const float e = expf(val[i] * inv_temp - max_vt);
        val[i] = e;
        sum += e;
    }
    std::vector<int> id(idx, idx + k);
    int n = k;
    if (top_p < 1.0f) {
        for (int i = 1; i < k; ++i) {
            const float kv = val[i];
            const int ki = id[i];
            int j = i - 1;
            while (j >= 0 && val[j] < kv) {
                val[j + 1] = val[j];
                id[j + 1] = id[j];
                --j;
            }
            val[j + 1] = kv;
            id[j + 1] = ki;
        }
        float cum = 0.0f;
        const float thr = top_p * sum;
        n = k;
        for (int i = 0; i < k; ++i) {
            cum += val[i];
            if (cum >= thr) {
                n = i + 1;
                break;
            }
        }
        sum = 0.0f;
        for (int i = 0; i < n; ++i) sum += val[i];
    }
    const float r = rng_f32(rng) * sum;
    float cdf = 0.0f;
    int s = n - 1;
    for (int i = 0; i < n; ++i) {
        cdf += val[i];
        if (r < cdf) {
            s = i;
            break;
        }
    }
    return id[s];
}

static void sample_impl(l3p_ctx* c, const float* logits, int n, const l3p_sampler* sp, uint64_t* rng, int32_t* out) {
    Model& m = *c->model;
    hipStream_t s = c->stream;
    if (sp->temperature == 0.0f) {                               // argmax (c:4812-4813)
        launch_argmax(logits, n, m.out_token, s, m.cand_val, m.cand_idx);
        L3P_HIP(hipMemcpyAsync(m.out_token_host, m.out_token, 4, hipMemcpyDeviceToHost, s));
        L3P_HIP(hipStreamSynchronize(s));
        *out = m.out_token_host[0];
        return;
    }
    L3P_REQUIRE(rng, L3P_E_INVALID, "sampler: rng state is NULL");
    L3P_REQUIRE(sp->top_k >= 1, L3P_E_INVALID, "sampler: top_k=%d", sp->top_k);
    const int k = std::min(sp->top_k, n);                        // c:4815-4816
    const int ng = std::max(256, sample_groups(m.vocab));
    float* slot_v = m.cand_val + ng;
    launch_topk_slots(logits, n, k, m.cand_val, slot_v, m.cand_idx, s);
    L3P_HIP(hipMemcpyAsync(m.slot_val_host, slot_v, (size_t)k * 4, hipMemcpyDeviceToHost, s));
    L3P_HIP(hipMemcpyAsync(m.slot_idx_host, m.cand_idx, (size_t)k * 4, hipMemcpyDeviceToHost, s));
    L3P_HIP(hipStreamSynchronize(s));
    *out = sample_slots(m.slot_val_host, m.slot_idx_host, k, sp->temperature, sp->top_p, rng);
}

// ---------------------------------------------------------------------------
// batched matmul (matmul_quantized_batch, c:2291-2331): the int8 matrix-core
// GEMM for the Q8_0-activation types, the fp32 one for the others
// ---------------------------------------------------------------------------
void run_gemm(l3p_ctx* c, int type, const uint8_t* w, int rows, int cols, const float* x, int batch, int in_stride,
              float* y, int out_stride) {
    if (gemm_q8_activation(type)) {   // the reference's integer block dots on the int8 matrix cores
        GemmJob j{};
        j.type = type;
        j.seg[0] = GemmSegment{w, rows, y, out_stride};
        j.nseg = 1;
        j.k = cols;
        j.x = x;
        j.m = batch;
        j.ldx = in_stride;
        launch_gemm_q8a(j, c->gemm_ws, c->gemm_ws_floats, c->stream);
        return;
    }
    if (gemm_mfma_supported(type)) {
        GemmJob j{};
        j.type = type;
        j.seg[0] = GemmSegment{w, rows, y, out_stride};
        j.nseg = 1;
        j.k = cols;
        j.x = x;
        j.m = batch;
        j.ldx = in_stride;
        launch_gemm(j, c->gemm_ws, c->gemm_ws_floats, c->stream);
        return;
    }
    L3P_REQUIRE(false, L3P_E_UNSUPPORTED, "gemm: type %d", type);
}

void run_stream_read(l3p_ctx* c, const void* p, size_t bytes) {
    ProfRange r(c->prof, c->stream, "stream read " + std::to_string(bytes), (double)bytes);
    launch_stream_read(p, bytes, reinterpret_cast<uint32_t*>(c->gemm_ws), c->stream);
}

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
template <class F>
static int mguard(l3p_ctx* c, bool need_model, F&& f) {
    if (!c) return L3P_E_INVALID;
    try {
        if (need_model && !c->model) throw L3pError{L3P_E_STATE, "no model loaded"};
        L3P_HIP(hipSetDevice(c->device));
        f();
        return L3P_OK;
    } catch (const L3pError& e) {
        c->err = e.msg;
        return e.code;
    } catch (const std::bad_alloc&) {
        c->err = "host allocation failed";
        return L3P_E_NOMEM;
    }
}

extern "C" {

int l3p_load_gguf(l3p_ctx* c, const void* bytes, size_t len, const l3p_load_opts* opts) {
    return mguard(c, false, [&] {
        L3P_REQUIRE(bytes, L3P_E_INVALID, "gguf pointer is NULL");
        L3P_HIP(hipStreamSynchronize(c->stream));
        c->drop_graphs();
        delete c->model;
        c->model = nullptr;
        c->model = load_model(c, bytes, len, opts);
    });
}

int l3p_get_model_info(l3p_ctx* c, l3p_model_info* o) {
    return mguard(c, true, [&] {
        L3P_REQUIRE(o, L3P_E_INVALID, "out is NULL");
        const Model& m = *c->model;
        memset(o, 0, sizeof *o);
        o->dim = m.dim; o->hidden_dim = m.hidden; o->n_layers = m.n_layers; o->n_heads = m.n_heads;
        o->n_kv_heads = m.n_kv; o->vocab_size = m.vocab; o->seq_len = m.seq_len; o->head_dim = m.hs;
        o->is_gemma = m.is_gemma; o->swa_window = m.swa_window; o->swa_pattern = m.swa_pattern;
        o->weight_type = m.weight_type; o->rope_theta = m.theta; o->rope_theta_swa = m.theta_swa;
        o->rms_eps = m.eps; o->final_softcap = m.softcap; o->device_bytes = m.device_bytes;
        o->attn_softcap = m.attn_softcap;
    });
}

int l3p_forward(l3p_ctx* c, int32_t token, int32_t pos, int compute_logits, float* logits_host) {
    return mguard(c, true, [&] {
        const Model& m = *c->model;
        L3P_REQUIRE(token >= 0 && token < m.vocab, L3P_E_INVALID, "token %d out of range [0, %d)", token, m.vocab);
        L3P_REQUIRE(pos >= 0 && pos < m.seq_len, L3P_E_INVALID, "pos %d out of range [0, %d)", pos, m.seq_len);
        forward_impl(c, token, pos, compute_logits != 0);
        if (compute_logits && logits_host)
            L3P_HIP(hipMemcpyAsync(logits_host, m.logits, (size_t)m.vocab * 4, hipMemcpyDeviceToHost, c->stream));
        L3P_HIP(hipStreamSynchronize(c->stream));
        c->prof.collect();
    });
}

int l3p_prefill(l3p_ctx* c, const int32_t* tokens, int n, int32_t start) {
    return mguard(c, true, [&] {
        const Model& m = *c->model;
        L3P_REQUIRE(n >= 0 && (n == 0 || tokens), L3P_E_INVALID, "prefill: bad token buffer");
        L3P_REQUIRE(start >= 0 && start <= m.seq_len && n <= m.seq_len - start, L3P_E_INVALID,
                    "prefill: %d positions from %d exceed the context of %d", n, start, m.seq_len);
        for (int i = 0; i < n; ++i)
            L3P_REQUIRE(tokens[i] >= 0 && tokens[i] < m.vocab, L3P_E_INVALID, "prefill: token %d out of range",
                        tokens[i]);
        if (prefill_batching()) prefill_batched(c, tokens, n, start);
        else
            for (int i = 0; i < n; ++i) forward_impl(c, tokens[i], start + i, false);
        L3P_HIP(hipStreamSynchronize(c->stream));
        c->prof.collect();
    });
}

int l3p_decode(l3p_ctx* c, int32_t token, int32_t pos, const l3p_sampler* sp, uint64_t* rng, int32_t* out) {
    return mguard(c, true, [&] {
        const Model& m = *c->model;
        L3P_REQUIRE(sp && out, L3P_E_INVALID, "decode: null sampler/out");
        L3P_REQUIRE(token >= 0 && token < m.vocab, L3P_E_INVALID, "token %d out of range [0, %d)", token, m.vocab);
        L3P_REQUIRE(pos >= 0 && pos < m.seq_len, L3P_E_INVALID, "pos %d out of range [0, %d)", pos, m.seq_len);
        forward_impl(c, token, pos, true);
        sample_impl(c, m.logits, m.vocab, sp, rng, out);
        c->prof.collect();
    });
}

// Greedy generation, the reference's decode loop (c:5289-5309) at temperature
// 0: step i runs the forward at position pos + i and the argmax.  Step 0 takes
// `token`; every later step's embedding reads the previous argmax from device
// memory, so the host queues steps ahead of the token it is waiting for (two
// in flight) and a step starts as soon as the previous one ends.  Each token
// comes back through its own pinned slot and event.  After a stop token the
// step already queued behind it still runs: it writes the K/V rows of the next
// position for the token that a following decode call at that position would
// write there anyway (greedy steps are deterministic).
int l3p_generate_greedy(l3p_ctx* c, int32_t token, int32_t pos, int32_t max_steps, const int32_t* stop_ids,
                        int32_t n_stop, int32_t* out_tokens, int32_t* n_out) {
    return mguard(c, true, [&] {
        const Model& m = *c->model;
        L3P_REQUIRE(out_tokens && n_out, L3P_E_INVALID, "generate: null output");
        *n_out = 0;
        L3P_REQUIRE(max_steps >= 0 && n_stop >= 0 && (n_stop == 0 || stop_ids), L3P_E_INVALID,
                    "generate: max_steps=%d, n_stop=%d", max_steps, n_stop);
        L3P_REQUIRE(token >= 0 && token < m.vocab, L3P_E_INVALID, "token %d out of range [0, %d)", token, m.vocab);
        L3P_REQUIRE(pos >= 0 && pos < m.seq_len, L3P_E_INVALID, "pos %d out of range [0, %d)", pos, m.seq_len);
        const int steps = std::min(max_steps, m.seq_len - pos);   // the reference's pos < max_tokens bound
        if (steps == 0) return;
        hipStream_t s = c->stream;
        if (!c->gen_host) {
            L3P_HIP(hipHostMalloc((void**)&c->gen_host, l3p_ctx::kGenSlots * sizeof(int), hipHostMallocDefault));
            for (hipEvent_t& e : c->gen_ev) L3P_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        }
        constexpr int kAhead = 2;
        static_assert(kAhead < l3p_ctx::kGenSlots, "a slot is read before it is written again");
        int issued = 0, done = 0;
        auto issue = [&](int i) {
            forward_impl(c, token, pos + i, true, i == 0 ? nullptr : m.out_token);
            launch_argmax(m.logits, m.vocab, m.out_token, s, m.cand_val, m.cand_idx);
            const int slot = i % l3p_ctx::kGenSlots;
            L3P_HIP(hipMemcpyAsync(c->gen_host + slot, m.out_token, 4, hipMemcpyDeviceToHost, s));
            L3P_HIP(hipEventRecord(c->gen_ev[slot], s));
        };
        try {
            while (done < steps) {
                while (issued < steps && issued < done + kAhead) issue(issued++);
                const int slot = done % l3p_ctx::kGenSlots;
                L3P_HIP(hipEventSynchronize(c->gen_ev[slot]));
                const int t = c->gen_host[slot];
                out_tokens[done++] = t;
                *n_out = done;
                if (std::find(stop_ids, stop_ids + n_stop, t) != stop_ids + n_stop) break;
            }
        } catch (...) {
            (void)hipStreamSynchronize(s);
            throw;
        }
        L3P_HIP(hipStreamSynchronize(s));   // the steps queued past a stop
        c->prof.collect();
    });
}

// Sampled generation, the reference's decode loop (c:5289-5309) with
// generate_token at temperature > 0 (c:4766-4907).  The host finishes each
// step's sampler (sample_slots: the reference's expf, sort, cut and draw), so
// a step's token is known only on the host; the device runs ahead anyway:
// steps are queued two ahead, each step's top-k scan writes its k slots into
// coherent pinned memory followed by a sequence word, the host spins on that
// word, samples, and writes (seq << 32) | token into the pinned word that the
// next step's embedding kernel is polling.  The only host round trip left on
// the critical path is that handshake; no launch waits for the host.
// Sequence numbers grow across calls, so a word left by an earlier call never
// matches.  After a stop token the step already queued behind it runs with
// that token (K/V rows of the next position, its logits and slots unused).
int l3p_generate_sampled(l3p_ctx* c, int32_t token, int32_t pos, int32_t max_steps, const l3p_sampler* sp,
                         uint64_t* rng, const int32_t* stop_ids, int32_t n_stop, int32_t* out_tokens,
                         int32_t* n_out) {
    return mguard(c, true, [&] {
        Model& m = *c->model;
        L3P_REQUIRE(out_tokens && n_out && sp && rng, L3P_E_INVALID, "generate: null argument");
        *n_out = 0;
        L3P_REQUIRE(max_steps >= 0 && n_stop >= 0 && (n_stop == 0 || stop_ids), L3P_E_INVALID,
                    "generate: max_steps=%d, n_stop=%d", max_steps, n_stop);
        L3P_REQUIRE(sp->temperature > 0.0f, L3P_E_INVALID, "generate_sampled: temperature %g (0 is greedy)",
                    (double)sp->temperature);
        L3P_REQUIRE(sp->top_k >= 1, L3P_E_INVALID, "sampler: top_k=%d", sp->top_k);
        L3P_REQUIRE(token >= 0 && token < m.vocab, L3P_E_INVALID, "token %d out of range [0, %d)", token, m.vocab);
        L3P_REQUIRE(pos >= 0 && pos < m.seq_len, L3P_E_INVALID, "pos %d out of range [0, %d)", pos, m.seq_len);
        const int steps = std::min(max_steps, m.seq_len - pos);   // the reference's pos < max_tokens bound
        if (steps == 0) return;
        const int k = std::min(sp->top_k, m.vocab);                // c:4815-4816
        L3P_REQUIRE(k <= sample_max_k(), L3P_E_UNSUPPORTED, "sampler: top_k=%d above %d", k, sample_max_k());
        hipStream_t s = c->stream;
        constexpr int S = l3p_ctx::kGenSlots;
        if (!c->smp_v) {
            const size_t kmax = (size_t)sample_max_k();
            L3P_HIP(hipHostMalloc((void**)&c->smp_v, S * kmax * 4, hipHostMallocCoherent));
            L3P_HIP(hipHostMalloc((void**)&c->smp_i, S * kmax * 4, hipHostMallocCoherent));
            L3P_HIP(hipHostMalloc((void**)&c->smp_seq, S * 4, hipHostMallocCoherent));
            L3P_HIP(hipHostMalloc((void**)&c->smp_tok, S * 8, hipHostMallocCoherent));
            L3P_HIP(hipHostMalloc((void**)&c->smp_fail, 4, hipHostMallocCoherent));
            for (int i = 0; i < S; ++i) {
                c->smp_seq[i] = 0;
                c->smp_tok[i] = 0;
            }
        }
        L3P_HIP(hipStreamSynchronize(s));   // nothing of an earlier call still reads the words
        *(volatile uint32_t*)c->smp_fail = 0;
        const uint32_t base = c->smp_next;
        c->smp_next += (uint32_t)steps + 1;
        if (c->smp_next < base) c->smp_next = 1;   // wrapped (after ~4e9 steps): restart above 0
        const int ng = std::max(256, sample_groups(m.vocab));
        const size_t kmax = (size_t)sample_max_k();
        constexpr int kAhead = 2;
        static_assert(kAhead < S, "a slot is read before it is written again");
        int issued = 0, done = 0;
        auto seq = [&](int i) { return base + (uint32_t)i; };
        auto publish = [&](int i, int t) {   // the token of step i, for step i + 1's embedding
            __atomic_store_n(&c->smp_tok[i % S], ((uint64_t)seq(i) << 32) | (uint32_t)t, __ATOMIC_RELEASE);
        };
        auto issue = [&](int i) {
            HostToken ht{};
            if (i > 0) ht = HostToken{c->smp_tok + (i - 1) % S, seq(i - 1), c->smp_fail, m.vocab};
            forward_impl(c, token, pos + i, true, nullptr, ht);
            const int slot = i % S;
            launch_topk_slots(m.logits, m.vocab, k, m.cand_val, m.cand_val + ng, m.cand_idx, s,
                              HostSlots{c->smp_v + slot * kmax, c->smp_i + slot * kmax, c->smp_seq + slot, seq(i)});
        };
        try {
            while (done < steps) {
                while (issued < steps && issued < done + kAhead) issue(issued++);
                const int slot = done % S;
                const auto t0 = std::chrono::steady_clock::now();
                while (__atomic_load_n(&c->smp_seq[slot], __ATOMIC_ACQUIRE) != seq(done)) {
                    L3P_REQUIRE(__atomic_load_n(c->smp_fail, __ATOMIC_RELAXED) == 0, L3P_E_HIP,
                                "generate_sampled: a step's token wait failed on the device");
                    if (std::chrono::steady_clock::now() - t0 > std::chrono::seconds(10)) {
                        const hipError_t q = hipStreamQuery(s);
                        if (q != hipSuccess && q != hipErrorNotReady) L3P_HIP(q);
                        throw L3pError{L3P_E_HIP, "generate_sampled: no top-k slots from the device in 10 s"};
                    }
                    __builtin_ia32_pause();
                }
                const int t = sample_slots(c->smp_v + slot * kmax, c->smp_i + slot * kmax, k, sp->temperature,
                                           sp->top_p, rng);
                publish(done, t);
                out_tokens[done++] = t;
                *n_out = done;
                if (std::find(stop_ids, stop_ids + n_stop, t) != stop_ids + n_stop) break;
            }
        } catch (...) {
            // release every queued step still waiting for a token, then drain
            for (int i = done; i + 1 < issued; ++i) publish(i, 0);
            (void)hipStreamSynchronize(s);
            throw;
        }
        L3P_HIP(hipStreamSynchronize(s));   // the step queued past a stop
        L3P_REQUIRE(__atomic_load_n(c->smp_fail, __ATOMIC_RELAXED) == 0, L3P_E_HIP,
                    "generate_sampled: a step's token wait failed on the device");
        c->prof.collect();
    });
}

int l3p_sample(l3p_ctx* c, const float* logits, int n, const l3p_sampler* sp, uint64_t* rng, int32_t* out) {
    return mguard(c, true, [&] {
        L3P_REQUIRE(logits && sp && out && n > 0, L3P_E_INVALID, "sample: bad arguments");
        L3P_REQUIRE(n <= c->model->vocab, L3P_E_INVALID, "sample: n=%d exceeds the model vocabulary", n);
        sample_impl(c, logits, n, sp, rng, out);
    });
}

int l3p_logits_device(l3p_ctx* c, const float** out) {
    return mguard(c, true, [&] {
        L3P_REQUIRE(out, L3P_E_INVALID, "out is NULL");
        *out = c->model->logits;
    });
}

int l3p_copy_kv(l3p_ctx* c, int layer, int which_v, void* dst, size_t cap) {
    return mguard(c, true, [&] {
        const Model& m = *c->model;
        L3P_REQUIRE(layer >= 0 && layer < m.n_layers, L3P_E_INVALID, "layer %d out of range", layer);
        L3P_REQUIRE(dst && cap >= m.layer_kv, L3P_E_INVALID, "copy_kv: need %zu bytes", m.layer_kv);
        const uint8_t* src = (which_v ? m.vc : m.kc) + (size_t)layer * m.layer_kv;
        L3P_HIP(hipMemcpyAsync(dst, src, m.layer_kv, hipMemcpyDeviceToHost, c->stream));
        L3P_HIP(hipStreamSynchronize(c->stream));
    });
}

int l3p_profile(l3p_ctx* c, int on) {
    return mguard(c, false, [&] {
        L3P_HIP(hipStreamSynchronize(c->stream));
        c->prof.reset();
        c->prof.on = on != 0;
    });
}

int l3p_profile_read(l3p_ctx* c, l3p_kernel_stat* out, int cap, int* n) {
    return mguard(c, false, [&] {
        L3P_REQUIRE(n && (cap <= 0 || out), L3P_E_INVALID, "profile_read: bad arguments");
        L3P_HIP(hipStreamSynchronize(c->stream));
        c->prof.collect();
        *n = (int)c->prof.stats.size();
        for (int i = 0; i < *n && i < cap; ++i) {
            const Profiler::Stat& st = c->prof.stats[i];
            memset(&out[i], 0, sizeof out[i]);
            snprintf(out[i].name, sizeof out[i].name, "%s", st.name.c_str());
            out[i].launches = st.launches;
            out[i].total_ms = st.ms;
            out[i].bytes_per_launch = st.bytes;
            if (!st.each.empty()) {   // nearest-rank percentiles
                std::vector<float> v(st.each);
                std::sort(v.begin(), v.end());
                auto pct = [&](double q) { return (double)v[(size_t)(q * (double)(v.size() - 1) + 0.5)]; };
                out[i].p10_ms = pct(0.1);
                out[i].p50_ms = pct(0.5);
                out[i].p90_ms = pct(0.9);
            }
        }
    });
}

int l3p_rope_row(l3p_ctx* c, int swa, int pos, float* cos_host, float* sin_host) {
    return mguard(c, true, [&] {
        const Model& m = *c->model;
        L3P_REQUIRE(pos >= 0 && pos < m.seq_len && cos_host && sin_host, L3P_E_INVALID, "rope_row: bad arguments");
        const size_t half = m.hs / 2;
        L3P_HIP(hipMemcpy(cos_host, (swa ? m.cos_s : m.cos_d) + pos * half, half * 4, hipMemcpyDeviceToHost));
        L3P_HIP(hipMemcpy(sin_host, (swa ? m.sin_s : m.sin_d) + pos * half, half * 4, hipMemcpyDeviceToHost));
    });
}

}  // extern "C"
