/*
 * l3p_napi.c — Node.js N-API addon over the libl3p C-ABI (include/l3p.h).
 *
 * It gives the JS engine's operator boundary a device-resident backend:
 *   transformer(token, pos, computeLogits)       llama3pure-js-engine.js:6121-6128
 *   transformerPrefill(allTokens, startPos, bs)  llama3pure-js-engine.js:6130-6136
 *   sample(logits, temp)                         llama3pure-js-engine.js:6158-6267
 * plus the fused decode step (forward + on-device sampling, only the token id
 * comes back).  Calls are synchronous on the JS thread, as the reference's are.
 * Every libl3p error becomes a thrown Error whose message is l3p_last_error()
 * and whose `code` is the L3P_E_* value; llama3pure() catches and logs thrown
 * errors (js:7246-7248), so the reference's error behaviour is kept.
 */
#include <node_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../include/l3p.h"

typedef struct {
    l3p_ctx* ctx;
    uint64_t rng;      /* xorshift64* state (c:4266-4276) */
} Engine;

#define NAPI_CALL(env, call)                                                  \
    do {                                                                      \
        if ((call) != napi_ok) {                                              \
            const napi_extended_error_info* ei_ = NULL;                       \
            napi_get_last_error_info((env), &ei_);                            \
            napi_throw_error((env), NULL, ei_ && ei_->error_message ?         \
                             ei_->error_message : "N-API call failed");       \
            return NULL;                                                      \
        }                                                                     \
    } while (0)

static napi_value throw_l3p(napi_env env, const l3p_ctx* ctx, int rc) {
    char code[16];
    snprintf(code, sizeof code, "%d", rc);
    napi_value msg, err, c;
    const char* m = l3p_last_error(ctx);
    napi_create_string_utf8(env, m && *m ? m : "l3p error", NAPI_AUTO_LENGTH, &msg);
    napi_create_error(env, NULL, msg, &err);
    napi_create_int32(env, rc, &c);
    napi_set_named_property(env, err, "code", c);
    napi_throw(env, err);
    return NULL;
}

#define L3P_CALL(env, eng, call)                                              \
    do {                                                                      \
        int rc_ = (call);                                                     \
        if (rc_ != 0) return throw_l3p((env), (eng) ? (eng)->ctx : NULL, rc_); \
    } while (0)

static void finalize(napi_env env, void* data, void* hint) {
    (void)env;
    (void)hint;
    Engine* e = (Engine*)data;
    if (e->ctx) l3p_destroy(e->ctx);
    free(e);
}

static Engine* engine_of(napi_env env, napi_value v) {
    Engine* e = NULL;
    if (napi_get_value_external(env, v, (void**)&e) != napi_ok || !e) {
        napi_throw_type_error(env, NULL, "expected an engine handle");
        return NULL;
    }
    if (!e->ctx) {
        napi_throw_error(env, NULL, "engine is closed");
        return NULL;
    }
    return e;
}

static int get_args(napi_env env, napi_callback_info info, size_t want, napi_value* argv) {
    size_t argc = want;
    if (napi_get_cb_info(env, info, &argc, argv, NULL, NULL) != napi_ok) return 0;
    for (size_t i = argc; i < want; ++i) napi_get_undefined(env, &argv[i]);
    return 1;
}

static int32_t i32_of(napi_env env, napi_value v, int32_t dflt) {
    napi_valuetype t;
    int32_t r = dflt;
    if (napi_typeof(env, v, &t) == napi_ok && t == napi_number) napi_get_value_int32(env, v, &r);
    return r;
}
static double f64_of(napi_env env, napi_value v, double dflt) {
    napi_valuetype t;
    double r = dflt;
    if (napi_typeof(env, v, &t) == napi_ok && t == napi_number) napi_get_value_double(env, v, &r);
    return r;
}

/* open(device) -> engine */
static napi_value js_open(napi_env env, napi_callback_info info) {
    napi_value argv[1], out;
    if (!get_args(env, info, 1, argv)) return NULL;
    Engine* e = (Engine*)calloc(1, sizeof *e);
    if (!e) {
        napi_throw_error(env, NULL, "out of host memory");
        return NULL;
    }
    e->rng = 0x2545F4914F6CDD1DULL;
    int rc = l3p_create(i32_of(env, argv[0], 0), &e->ctx);
    if (rc != 0) {
        free(e);
        return throw_l3p(env, NULL, rc);
    }
    NAPI_CALL(env, napi_create_external(env, e, finalize, NULL, &out));
    return out;
}

/* close(engine) */
static napi_value js_close(napi_env env, napi_callback_info info) {
    napi_value argv[1];
    if (!get_args(env, info, 1, argv)) return NULL;
    Engine* e = NULL;
    NAPI_CALL(env, napi_get_value_external(env, argv[0], (void**)&e));
    if (e && e->ctx) {
        l3p_destroy(e->ctx);
        e->ctx = NULL;
    }
    return NULL;
}

static napi_value info_object(napi_env env, const l3p_model_info* mi) {
    napi_value o, v;
    NAPI_CALL(env, napi_create_object(env, &o));
#define SETI(name, val) napi_create_int32(env, (val), &v); napi_set_named_property(env, o, name, v);
#define SETF(name, val) napi_create_double(env, (val), &v); napi_set_named_property(env, o, name, v);
    SETI("dim", mi->dim) SETI("hiddenDim", mi->hidden_dim) SETI("nLayers", mi->n_layers)
    SETI("nHeads", mi->n_heads) SETI("nKvHeads", mi->n_kv_heads) SETI("vocabSize", mi->vocab_size)
    SETI("seqLen", mi->seq_len) SETI("headDim", mi->head_dim) SETI("swaWindow", mi->swa_window)
    SETI("weightType", mi->weight_type)
    SETF("ropeTheta", mi->rope_theta) SETF("rmsEps", mi->rms_eps) SETF("finalSoftcap", mi->final_softcap)
    SETF("deviceBytes", (double)mi->device_bytes)
    SETI("swaPattern", mi->swa_pattern) SETF("attnSoftcap", mi->attn_softcap)
    napi_get_boolean(env, mi->is_gemma != 0, &v);
    napi_set_named_property(env, o, "isGemma", v);
#undef SETI
#undef SETF
    return o;
}

/* loadGguf(engine, ArrayBuffer | TypedArray | Buffer, contextSize,
 *          {swaPattern, attnSoftcap}?) -> info
 * The options object is optional; absent or non-numeric fields are 0, the
 * reference's behaviour (l3p_load_opts). */
static napi_value js_load(napi_env env, napi_callback_info info) {
    napi_value argv[4];
    if (!get_args(env, info, 4, argv)) return NULL;
    Engine* e = engine_of(env, argv[0]);
    if (!e) return NULL;
    void* data = NULL;
    size_t len = 0;
    bool is_ab = false, is_ta = false;
    napi_is_arraybuffer(env, argv[1], &is_ab);
    napi_is_typedarray(env, argv[1], &is_ta);
    if (is_ab) {
        NAPI_CALL(env, napi_get_arraybuffer_info(env, argv[1], &data, &len));
    } else if (is_ta) {
        napi_typedarray_type tt;
        size_t n, off;
        napi_value ab;
        NAPI_CALL(env, napi_get_typedarray_info(env, argv[1], &tt, &n, &data, &ab, &off));
        size_t esz = (tt == napi_float64_array || tt == napi_bigint64_array || tt == napi_biguint64_array) ? 8
                     : (tt == napi_float32_array || tt == napi_int32_array || tt == napi_uint32_array) ? 4
                     : (tt == napi_int16_array || tt == napi_uint16_array) ? 2 : 1;
        len = n * esz;
    } else {
        napi_throw_type_error(env, NULL, "model must be an ArrayBuffer or a typed array");
        return NULL;
    }
    l3p_load_opts o;
    memset(&o, 0, sizeof o);
    o.context_size = i32_of(env, argv[2], 0);
    napi_valuetype ot;
    if (napi_typeof(env, argv[3], &ot) == napi_ok && ot == napi_object) {
        napi_value v;
        if (napi_get_named_property(env, argv[3], "swaPattern", &v) == napi_ok) o.swa_pattern = i32_of(env, v, 0);
        if (napi_get_named_property(env, argv[3], "attnSoftcap", &v) == napi_ok)
            o.attn_softcap = (float)f64_of(env, v, 0.0);
    }
    L3P_CALL(env, e, l3p_load_gguf(e->ctx, data, len, &o));
    l3p_model_info mi;
    L3P_CALL(env, e, l3p_get_model_info(e->ctx, &mi));
    return info_object(env, &mi);
}

/* transformer(engine, token, pos, computeLogits, outFloat32Array?) */
static napi_value js_transformer(napi_env env, napi_callback_info info) {
    napi_value argv[5];
    if (!get_args(env, info, 5, argv)) return NULL;
    Engine* e = engine_of(env, argv[0]);
    if (!e) return NULL;
    bool logits = false;
    napi_get_value_bool(env, argv[3], &logits);
    float* out = NULL;
    bool is_ta = false;
    napi_is_typedarray(env, argv[4], &is_ta);
    if (logits && is_ta) {
        napi_typedarray_type tt;
        size_t n, off;
        napi_value ab;
        NAPI_CALL(env, napi_get_typedarray_info(env, argv[4], &tt, &n, (void**)&out, &ab, &off));
        l3p_model_info mi;
        L3P_CALL(env, e, l3p_get_model_info(e->ctx, &mi));
        if (tt != napi_float32_array || n < (size_t)mi.vocab_size) {
            napi_throw_range_error(env, NULL, "logits must be a Float32Array of vocabSize elements");
            return NULL;
        }
    }
    L3P_CALL(env, e, l3p_forward(e->ctx, i32_of(env, argv[1], -1), i32_of(env, argv[2], -1), logits, out));
    return NULL;
}

/* transformerPrefill(engine, allTokens (Int32Array | Array), startPos, batchSize) */
static napi_value js_prefill(napi_env env, napi_callback_info info) {
    napi_value argv[4];
    if (!get_args(env, info, 4, argv)) return NULL;
    Engine* e = engine_of(env, argv[0]);
    if (!e) return NULL;
    const int32_t start = i32_of(env, argv[2], -1), bs = i32_of(env, argv[3], -1);
    if (start < 0 || bs < 0) {
        napi_throw_range_error(env, NULL, "startPos and batchSize must be non-negative");
        return NULL;
    }
    bool is_ta = false, is_arr = false;
    napi_is_typedarray(env, argv[1], &is_ta);
    napi_is_array(env, argv[1], &is_arr);
    int32_t* tok = (int32_t*)malloc(sizeof(int32_t) * (bs > 0 ? bs : 1));
    if (!tok) {
        napi_throw_error(env, NULL, "out of host memory");
        return NULL;
    }
    uint32_t n = 0;
    if (is_ta) {
        napi_typedarray_type tt;
        size_t len, off;
        napi_value ab;
        void* d;
        if (napi_get_typedarray_info(env, argv[1], &tt, &len, &d, &ab, &off) != napi_ok || tt != napi_int32_array) {
            free(tok);
            napi_throw_type_error(env, NULL, "allTokens must be an Int32Array or an Array");
            return NULL;
        }
        n = (uint32_t)len;
        if ((uint32_t)start + (uint32_t)bs > n) goto range;
        memcpy(tok, (int32_t*)d + start, sizeof(int32_t) * bs);
    } else if (is_arr) {
        napi_get_array_length(env, argv[1], &n);
        if ((uint32_t)start + (uint32_t)bs > n) goto range;
        for (int32_t i = 0; i < bs; ++i) {
            napi_value v;
            napi_get_element(env, argv[1], (uint32_t)(start + i), &v);
            tok[i] = i32_of(env, v, -1);
        }
    } else {
        free(tok);
        napi_throw_type_error(env, NULL, "allTokens must be an Int32Array or an Array");
        return NULL;
    }
    {
        int rc = l3p_prefill(e->ctx, tok, bs, start);
        free(tok);
        if (rc != 0) return throw_l3p(env, e->ctx, rc);
    }
    return NULL;
range:
    free(tok);
    napi_throw_range_error(env, NULL, "startPos + batchSize exceeds allTokens");
    return NULL;
}

static l3p_sampler sampler_of(napi_env env, napi_value t, napi_value k, napi_value p) {
    l3p_sampler s;
    memset(&s, 0, sizeof s);
    s.temperature = (float)f64_of(env, t, 0.0);
    s.top_k = i32_of(env, k, 40);
    s.top_p = (float)f64_of(env, p, 0.9);
    return s;
}

/* decode(engine, token, pos, temperature, topK, topP) -> next token */
static napi_value js_decode(napi_env env, napi_callback_info info) {
    napi_value argv[6], out;
    if (!get_args(env, info, 6, argv)) return NULL;
    Engine* e = engine_of(env, argv[0]);
    if (!e) return NULL;
    l3p_sampler s = sampler_of(env, argv[3], argv[4], argv[5]);
    int32_t next = -1;
    L3P_CALL(env, e, l3p_decode(e->ctx, i32_of(env, argv[1], -1), i32_of(env, argv[2], -1), &s, &e->rng, &next));
    NAPI_CALL(env, napi_create_int32(env, next, &out));
    return out;
}

/* sample(engine, temperature, topK, topP) -> token from the last forward's logits */
static napi_value js_sample(napi_env env, napi_callback_info info) {
    napi_value argv[4], out;
    if (!get_args(env, info, 4, argv)) return NULL;
    Engine* e = engine_of(env, argv[0]);
    if (!e) return NULL;
    l3p_sampler s = sampler_of(env, argv[1], argv[2], argv[3]);
    const float* lg = NULL;
    l3p_model_info mi;
    L3P_CALL(env, e, l3p_logits_device(e->ctx, &lg));
    L3P_CALL(env, e, l3p_get_model_info(e->ctx, &mi));
    int32_t next = -1;
    L3P_CALL(env, e, l3p_sample(e->ctx, lg, mi.vocab_size, &s, &e->rng, &next));
    NAPI_CALL(env, napi_create_int32(env, next, &out));
    return out;
}

/* setSeed(engine, hi, lo) / getSeed(engine) -> [hi, lo]: the xorshift64* state */
static napi_value js_set_seed(napi_env env, napi_callback_info info) {
    napi_value argv[3];
    if (!get_args(env, info, 3, argv)) return NULL;
    Engine* e = engine_of(env, argv[0]);
    if (!e) return NULL;
    uint32_t hi = 0, lo = 0;
    napi_get_value_uint32(env, argv[1], &hi);
    napi_get_value_uint32(env, argv[2], &lo);
    e->rng = ((uint64_t)hi << 32) | lo;
    return NULL;
}
static napi_value js_get_seed(napi_env env, napi_callback_info info) {
    napi_value argv[1], arr, v;
    if (!get_args(env, info, 1, argv)) return NULL;
    Engine* e = engine_of(env, argv[0]);
    if (!e) return NULL;
    NAPI_CALL(env, napi_create_array_with_length(env, 2, &arr));
    napi_create_uint32(env, (uint32_t)(e->rng >> 32), &v);
    napi_set_element(env, arr, 0, v);
    napi_create_uint32(env, (uint32_t)e->rng, &v);
    napi_set_element(env, arr, 1, v);
    return arr;
}

static napi_value init(napi_env env, napi_value exports) {
    napi_property_descriptor d[] = {
        {"open", 0, js_open, 0, 0, 0, napi_enumerable, 0},
        {"close", 0, js_close, 0, 0, 0, napi_enumerable, 0},
        {"loadGguf", 0, js_load, 0, 0, 0, napi_enumerable, 0},
        {"transformer", 0, js_transformer, 0, 0, 0, napi_enumerable, 0},
        {"transformerPrefill", 0, js_prefill, 0, 0, 0, napi_enumerable, 0},
        {"decode", 0, js_decode, 0, 0, 0, napi_enumerable, 0},
        {"sample", 0, js_sample, 0, 0, 0, napi_enumerable, 0},
        {"setSeed", 0, js_set_seed, 0, 0, 0, napi_enumerable, 0},
        {"getSeed", 0, js_get_seed, 0, 0, 0, napi_enumerable, 0},
    };
    if (napi_define_properties(env, exports, sizeof d / sizeof d[0], d) != napi_ok) return NULL;
    return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
