// api.cpp — the C-ABI of libl3p (include/l3p.h): context, device memory and
// the standalone quantized ops.  The model entry points live in model.cpp.
#include <new>

#include "internal.h"
#include "model.h"

static thread_local std::string g_create_error;

template <class F>
static int guard(l3p_ctx* c, F&& f) {
    try {
        f();
        return L3P_OK;
    } catch (const L3pError& e) {
        if (c) c->err = e.msg;
        else g_create_error = e.msg;
        return e.code;
    } catch (const std::bad_alloc&) {
        if (c) c->err = "host allocation failed";
        else g_create_error = "host allocation failed";
        return L3P_E_NOMEM;
    }
}

#define CHECK_CTX(c)                                 \
    do {                                             \
        if (!(c)) {                                  \
            g_create_error = "null context";         \
            return L3P_E_INVALID;                    \
        }                                            \
    } while (0)

extern "C" {

int l3p_create(int device, l3p_ctx** out) {
    if (!out) {
        g_create_error = "out is NULL";
        return L3P_E_INVALID;
    }
    *out = nullptr;
    return guard(nullptr, [&] {
        int n = 0;
        L3P_HIP(hipGetDeviceCount(&n));
        L3P_REQUIRE(device >= 0 && device < n, L3P_E_INVALID, "device %d out of range (%d devices)", device, n);
        L3P_HIP(hipSetDevice(device));
        auto* c = new l3p_ctx();
        c->device = device;
        hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
        if (e != hipSuccess) {
            delete c;
            throw L3pError{L3P_E_HIP, std::string("hipStreamCreate: ") + hipGetErrorString(e)};
        }
        const size_t ws_floats = kGemmWsFloats;   // 64 MB of GEMM split-K partials
        e = hipMalloc(&c->gemm_ws, ws_floats * 4);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            hipStreamDestroy(c->stream);
            delete c;
            throw L3pError{L3P_E_HIP, std::string("hipMalloc: ") + hipGetErrorString(e)};
        }
        c->gemm_ws_floats = ws_floats;
        *out = c;
    });
}

void l3p_destroy(l3p_ctx* c) {
    if (!c) return;
    hipSetDevice(c->device);
    hipStreamSynchronize(c->stream);
    c->drop_graphs();
    delete c->model;
    c->model = nullptr;
    c->prof.release();
    if (c->gemm_ws) hipFree(c->gemm_ws);
    if (c->gen_host) hipHostFree(c->gen_host);
    for (void* p : {(void*)c->smp_v, (void*)c->smp_i, (void*)c->smp_seq, (void*)c->smp_tok, (void*)c->smp_fail})
        if (p) hipHostFree(p);
    for (hipEvent_t e : c->gen_ev)
        if (e) hipEventDestroy(e);
    if (c->cap_stream) hipStreamDestroy(c->cap_stream);
    hipStreamDestroy(c->stream);
    delete c;
}

const char* l3p_last_error(const l3p_ctx* c) { return c ? c->err.c_str() : g_create_error.c_str(); }

void* l3p_stream(l3p_ctx* c) { return c ? (void*)c->stream : nullptr; }

int l3p_synchronize(l3p_ctx* c) {
    CHECK_CTX(c);
    return guard(c, [&] { L3P_HIP(hipStreamSynchronize(c->stream)); });
}

int l3p_malloc(l3p_ctx* c, size_t bytes, void** out) {
    CHECK_CTX(c);
    return guard(c, [&] {
        L3P_REQUIRE(out, L3P_E_INVALID, "out is NULL");
        L3P_HIP(hipSetDevice(c->device));
        hipError_t e = hipMalloc(out, bytes ? bytes : 1);
        if (e != hipSuccess) (void)hipGetLastError();   // consumed here: later launch checks must not see it
        if (e == hipErrorOutOfMemory) throw L3pError{L3P_E_NOMEM, "hipMalloc: out of device memory"};
        L3P_HIP(e);
    });
}

int l3p_free(l3p_ctx* c, void* p) {
    CHECK_CTX(c);
    return guard(c, [&] {
        L3P_HIP(hipStreamSynchronize(c->stream));
        L3P_HIP(hipFree(p));
    });
}

int l3p_upload(l3p_ctx* c, void* dst, const void* src, size_t n) {
    CHECK_CTX(c);
    return guard(c, [&] {
        L3P_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, c->stream));
        L3P_HIP(hipStreamSynchronize(c->stream));
    });
}

int l3p_download(l3p_ctx* c, void* dst, const void* src, size_t n) {
    CHECK_CTX(c);
    return guard(c, [&] {
        L3P_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, c->stream));
        L3P_HIP(hipStreamSynchronize(c->stream));
    });
}

size_t l3p_row_bytes(int type, int cols) { return type_row_bytes(type, cols); }

int l3p_dequant(l3p_ctx* c, int type, const void* src, int64_t n, float* dst) {
    CHECK_CTX(c);
    return guard(c, [&] {
        const int e = type_block_elems(type);
        L3P_REQUIRE(e > 0, L3P_E_UNSUPPORTED, "dequant: unsupported type %d", type);
        L3P_REQUIRE(n >= 0 && n % e == 0, L3P_E_INVALID, "dequant: n=%lld not a multiple of %d", (long long)n, e);
        L3P_REQUIRE(n == 0 || (src && dst), L3P_E_INVALID, "dequant: null pointer");
        launch_dequant(type, (const uint8_t*)src, n, dst, c->stream);
    });
}

int l3p_quantize_q8_0(l3p_ctx* c, const float* x, int64_t n, void* dst) {
    CHECK_CTX(c);
    return guard(c, [&] {
        L3P_REQUIRE(n >= 0 && n % 32 == 0, L3P_E_INVALID, "quantize_q8_0: n=%lld not a multiple of 32", (long long)n);
        L3P_REQUIRE(n == 0 || (x && dst), L3P_E_INVALID, "quantize_q8_0: null pointer");
        launch_quantize_q8_0_blocks(x, n, (uint8_t*)dst, c->stream);
    });
}

int l3p_gemv(l3p_ctx* c, int type, const void* w, int rows, int cols, const float* x, float* y) {
    CHECK_CTX(c);
    return guard(c, [&] {
        L3P_REQUIRE(rows >= 0 && cols > 0, L3P_E_INVALID, "gemv: bad shape %d x %d", rows, cols);
        L3P_REQUIRE(type_block_elems(type) > 0 && cols % type_block_elems(type) == 0, L3P_E_INVALID,
                    "gemv: cols=%d not a multiple of the block size of type %d", cols, type);
        L3P_REQUIRE(gemv_supported(type, cols), L3P_E_UNSUPPORTED,
                    "gemv: type %d with %d columns not supported", type, cols);
        if (rows == 0) return;
        L3P_REQUIRE(w && x && y, L3P_E_INVALID, "gemv: null pointer");
        L3P_HIP(hipSetDevice(c->device));
        GemvBatch b{};
        b.seg[0] = GemvSegment{(const uint8_t*)w, y, rows};
        b.nseg = 1;
        b.epilogue = EPI_STORE;
        b.standalone = 1;
        gemv_plain(c, type, b, cols, x);
    });
}

int l3p_stream_read(l3p_ctx* c, const void* buf, size_t bytes) {
    CHECK_CTX(c);
    return guard(c, [&] {
        L3P_REQUIRE(buf && ((uintptr_t)buf & 15) == 0 && bytes % 16 == 0, L3P_E_INVALID,
                    "stream_read: buffer must be 16-byte aligned and a multiple of 16 bytes");
        L3P_HIP(hipSetDevice(c->device));
        run_stream_read(c, buf, bytes);
    });
}

// Arguments of l3p_gemm / l3p_gemm_static; false when there is nothing to do.
static bool gemm_args_ok(int type, const void* w, int rows, int cols, const float* x, int batch, int in_stride,
                         const float* y, int out_stride) {
    L3P_REQUIRE(rows >= 0 && cols > 0 && batch >= 0, L3P_E_INVALID, "gemm: bad shape %d x %d, batch %d", rows, cols,
                batch);
    L3P_REQUIRE(type_block_elems(type) > 0 && cols % type_block_elems(type) == 0, L3P_E_INVALID,
                "gemm: cols=%d not a multiple of the block size of type %d", cols, type);
    L3P_REQUIRE(in_stride >= cols && out_stride >= rows, L3P_E_INVALID, "gemm: bad strides %d, %d", in_stride,
                out_stride);
    L3P_REQUIRE(in_stride % 4 == 0, L3P_E_INVALID, "gemm: in_stride %d is not a multiple of 4", in_stride);
    L3P_REQUIRE(gemv_supported(type, cols), L3P_E_UNSUPPORTED,
                "gemm: type %d with %d columns not supported", type, cols);
    if (rows == 0 || batch == 0) return false;
    L3P_REQUIRE(w && x && y, L3P_E_INVALID, "gemm: null pointer");
    return true;
}

int l3p_gemm(l3p_ctx* c, int type, const void* w, int rows, int cols, const float* x, int batch,
             int in_stride, float* y, int out_stride) {
    CHECK_CTX(c);
    return guard(c, [&] {
        if (!gemm_args_ok(type, w, rows, cols, x, batch, in_stride, y, out_stride)) return;
        L3P_HIP(hipSetDevice(c->device));
        run_gemm(c, type, (const uint8_t*)w, rows, cols, x, batch, in_stride, y, out_stride);
    });
}

int l3p_gemm_static(int type, const void* w, int rows, int cols, const float* x, int batch, int in_stride,
                    float* y, int out_stride, void* stream) {
    return guard(nullptr, [&] {
        if (!gemm_args_ok(type, w, rows, cols, x, batch, in_stride, y, out_stride)) return;
        const hipStream_t st = static_cast<hipStream_t>(stream);
        GemmJob j{};
        j.type = type;
        j.seg[0] = GemmSegment{(const uint8_t*)w, rows, y, out_stride};
        j.nseg = 1;
        j.k = cols;
        j.x = x;
        j.m = batch;
        j.ldx = in_stride;
        if (gemm_q8_activation(type)) {
            // the int8 path of l3p_gemm (no partials; each output's blocks in
            // order, so the rows per launch do not change a value), with the
            // quantized activation rows in the file-scope array
            launch_gemm_q8a(j, gemm_static_scratch(), kGemmStaticScratchFloats, st);
            return;
        }
        L3P_REQUIRE(gemm_mfma_supported(type), L3P_E_UNSUPPORTED, "gemm_static: type %d", type);
        // the plan l3p_gemm takes with its context workspace, so the values
        // are l3p_gemm's; its partials must fit the file-scope array
        const GemmPlan plan = gemm_plan(j, kGemmWsFloats);
        L3P_REQUIRE(plan.partial_floats <= kGemmStaticScratchFloats, L3P_E_UNSUPPORTED,
                    "gemm_static: %d x %d x batch %d needs %zu floats of split-K partials, more than the %zu of the "
                    "static scratch; use l3p_gemm",
                    rows, cols, batch, plan.partial_floats, kGemmStaticScratchFloats);
        launch_gemm_planned(j, plan, plan.nsplit > 1 || plan.streamk ? gemm_static_scratch() : nullptr, st);
    });
}

}  // extern "C"
