// fh_api.hip — the C ABI of libferrum_hip (contexts, weights, argument checks).
//
// Argument checking and error text follow the reference entry points each
// function replaces (cited per function); kernels live in the other
// translation units and are reached through the fh_launch_* launchers.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>

#include "fh_internal.hpp"

#include <cmath>

static thread_local std::string g_create_err;

int fh_fail(fh_ctx* ctx, int code, const std::string& msg) {
    if (ctx) ctx->err = msg;
    else g_create_err = msg;
    return code;
}

int fh_hip_fail(fh_ctx* ctx, hipError_t e, const char* what) {
    std::string m = std::string("HIP error ") + hipGetErrorName(e) + " (" + hipGetErrorString(e) +
                    ") in " + what;
    int code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? FH_ERR_OOM : FH_ERR_HIP;
    return fh_fail(ctx, code, m);
}

// Grow a plain device area; the old one is freed after the stream drains.
static int grow_area(fh_ctx* ctx, void** area, size_t* area_bytes, size_t bytes, void** out) {
    bytes = fh_align256(bytes ? bytes : 256);
    if (*area_bytes < bytes) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        FH_HIP(ctx, hipStreamIsCapturing(ctx->stream, &cs));
        if (cs != hipStreamCaptureStatusNone)
            return fh_fail(ctx, FH_ERR_INVALID,
                           "the context workspace must grow, which cannot happen during graph capture: "
                           "run the same call once outside capture first");
        if (*area) {
            // The previous area may still be read by queued kernels.
            FH_HIP(ctx, hipStreamSynchronize(ctx->stream));
            FH_HIP(ctx, hipFree(*area));
            *area = nullptr;
            *area_bytes = 0;
        }
        FH_HIP(ctx, hipMalloc(area, bytes));
        *area_bytes = bytes;
    }
    *out = *area;
    return FH_OK;
}

int fh_workspace(fh_ctx* ctx, size_t bytes, void** out) { return grow_area(ctx, &ctx->ws, &ctx->ws_bytes, bytes, out); }

int fh_act_area(fh_ctx* ctx, size_t bytes, void** out) { return grow_area(ctx, &ctx->act, &ctx->act_bytes, bytes, out); }

// Pinned host staging of the blocking calls (grown with hipHostMalloc; only
// touched by blocking calls, which synchronise before they return).
constexpr size_t kPinMax = size_t(8) << 20;  // larger arguments are copied from the caller's memory directly
static int pin_area(fh_ctx* ctx, size_t bytes, char** out) {
    bytes = fh_align256(bytes ? bytes : 256);
    if (ctx->pin_bytes < bytes) {
        if (ctx->pin) {
            FH_HIP(ctx, hipStreamSynchronize(ctx->stream));
            FH_HIP(ctx, hipHostFree(ctx->pin));
            ctx->pin = nullptr;
            ctx->pin_bytes = 0;
        }
        FH_HIP(ctx, hipHostMalloc(&ctx->pin, bytes, hipHostMallocDefault));
        ctx->pin_bytes = bytes;
    }
    *out = static_cast<char*>(ctx->pin);
    return FH_OK;
}

// The blocking calls' device buffers: kept on the context, so a call in steady
// state allocates nothing (no hipMalloc / hipFree per call).
static int io_area(fh_ctx* ctx, size_t bytes, char** out) {
    void* p = nullptr;
    const int rc = grow_area(ctx, &ctx->io, &ctx->io_bytes, bytes, &p);
    *out = static_cast<char*>(p);
    return rc;
}

// Grow a zero-initialised area (kernels leave it zeroed again).  Growing
// synchronises the stream and is refused under graph capture.
static int zeroed_area(fh_ctx* ctx, void** area, size_t* area_bytes, size_t bytes, const char* who, void** out) {
    bytes = fh_align256(bytes ? bytes : 256);
    if (*area_bytes < bytes) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        FH_HIP(ctx, hipStreamIsCapturing(ctx->stream, &cs));
        if (cs != hipStreamCaptureStatusNone)
            return fh_fail(ctx, FH_ERR_INVALID,
                           std::string(who) + " must grow, which cannot happen during graph capture: "
                           "run the same call once outside capture first");
        FH_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (*area) {
            FH_HIP(ctx, hipFree(*area));
            *area = nullptr;
            *area_bytes = 0;
        }
        FH_HIP(ctx, hipMalloc(area, bytes));
        // Zeroed on the context's stream and waited for: the stream is
        // non-blocking, so a memset on the legacy default stream would not be
        // ordered before the kernels that use the area (a kernel could start,
        // publish into it, and have the late memset wipe what it published).
        FH_HIP(ctx, hipMemsetAsync(*area, 0, bytes, ctx->stream));
        FH_HIP(ctx, hipStreamSynchronize(ctx->stream));
        *area_bytes = bytes;
    }
    *out = *area;
    return FH_OK;
}

int fh_sync_area(fh_ctx* ctx, size_t bytes, void** out) {
    return zeroed_area(ctx, &ctx->sync, &ctx->sync_bytes, bytes, "the sampler's per-row state", out);
}

int fh_counter_area(fh_ctx* ctx, size_t bytes, void** out) {
    return zeroed_area(ctx, &ctx->counters, &ctx->counters_bytes, bytes, "the GEMM's per-tile counters", out);
}

// Every entry point works on the context's device.
// (hipSetDevice only when needed, so calls stay legal under stream capture.)
static hipError_t on_device(int device) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess && cur == device) return hipSuccess;
    return hipSetDevice(device);
}
#define FH_ON_DEVICE(ctx) FH_HIP((ctx), on_device((ctx)->device))

int fh_take_status(fh_ctx* ctx) {
    unsigned bits = 0;
    FH_HIP(ctx, hipMemcpyAsync(&bits, ctx->status, sizeof(bits), hipMemcpyDeviceToHost, ctx->stream));
    FH_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (bits == 0) return FH_OK;
    FH_HIP(ctx, hipMemsetAsync(ctx->status, 0, sizeof(unsigned), ctx->stream));
    FH_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (bits & FH_STATUS_EXCHANGE) {
        // A failed exchange can leave a row's survivor count or slots behind
        // its generation: start every row over from a zeroed area (tag 0 is
        // never a live tag, so no stale slot is taken for a fresh one).
        if (ctx->sync) {
            FH_HIP(ctx, hipMemsetAsync(ctx->sync, 0, ctx->sync_bytes, ctx->stream));
            FH_HIP(ctx, hipStreamSynchronize(ctx->stream));
        }
        return fh_fail(ctx, FH_ERR_EXCHANGE,
                       "a kernel's cross-workgroup wait gave up (its workgroups were not all resident at once); "
                       "the results since the last fh_sync are unreliable");
    }
    return fh_fail(ctx, FH_ERR_INVALID, "fh_sample_rows: recent_offsets decrease");
}

extern "C" {

int fh_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int fh_ctx_create(int device, fh_ctx** out) {
    if (!out) return fh_fail(nullptr, FH_ERR_INVALID, "fh_ctx_create: out is NULL");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0)
        return fh_fail(nullptr, FH_ERR_HIP, "fh_ctx_create: no HIP device visible");
    if (device < 0 || device >= n)
        return fh_fail(nullptr, FH_ERR_INVALID,
                       "fh_ctx_create: device " + std::to_string(device) + " out of range (" +
                           std::to_string(n) + " visible)");
    fh_ctx* c = new (std::nothrow) fh_ctx();
    if (!c) return fh_fail(nullptr, FH_ERR_OOM, "fh_ctx_create: out of host memory");
    c->device = device;
    if ((e = hipSetDevice(device)) != hipSuccess ||
        (e = hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking)) != hipSuccess) {
        int code = fh_hip_fail(nullptr, e, "fh_ctx_create");
        delete c;
        return code;
    }
    c->stream = c->own;
    if (hipDeviceGetAttribute(&c->num_cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        c->num_cus < 1)
        c->num_cus = 1;
    void* st = nullptr;
    if ((e = hipMalloc(&st, 256)) != hipSuccess || (e = hipMemsetAsync(st, 0, 256, c->own)) != hipSuccess ||
        (e = hipStreamSynchronize(c->own)) != hipSuccess) {
        int code = fh_hip_fail(nullptr, e, "fh_ctx_create (status word)");
        if (st) (void)hipFree(st);
        (void)hipStreamDestroy(c->own);
        delete c;
        return code;
    }
    c->status = static_cast<unsigned*>(st);
    *out = c;
    return FH_OK;
}


void fh_ctx_destroy(fh_ctx* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->sync) (void)hipFree(ctx->sync);
    if (ctx->counters) (void)hipFree(ctx->counters);
    if (ctx->act) (void)hipFree(ctx->act);
    if (ctx->io) (void)hipFree(ctx->io);
    if (ctx->pin) (void)hipHostFree(ctx->pin);
    if (ctx->status) (void)hipFree(ctx->status);
    if (ctx->own) (void)hipStreamDestroy(ctx->own);
    delete ctx;
}

int fh_ctx_set_stream(fh_ctx* ctx, void* hip_stream) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    ctx->stream = static_cast<hipStream_t>(hip_stream);
    return FH_OK;
}

int fh_ctx_reset_stream(fh_ctx* ctx) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    ctx->stream = ctx->own;
    return FH_OK;
}

int fh_sync(fh_ctx* ctx) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    FH_ON_DEVICE(ctx);
    FH_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return fh_take_status(ctx);
}

const char* fh_last_error(const fh_ctx* ctx) { return ctx ? ctx->err.c_str() : g_create_err.c_str(); }

// ---- weights -------------------------------------------------------------------

static int alloc_weight(fh_ctx* ctx, size_t n_rows, size_t k, fh_q8_0** out) {
    if (!out) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_upload: out is NULL");
    *out = nullptr;
    if (k == 0 || k % 32 != 0)
        return fh_fail(ctx, FH_ERR_INVALID,
                       "fh_q8_0_upload: ne0 = " + std::to_string(k) +
                           " is not a positive multiple of the Q8_0 block size 32");
    if (n_rows == 0) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_upload: n_rows is 0");
    fh_q8_0* w = new (std::nothrow) fh_q8_0();
    if (!w) return fh_fail(ctx, FH_ERR_OOM, "fh_q8_0_upload: out of host memory");
    w->device = ctx->device;
    w->n = n_rows;
    w->k = k;
    w->kb = k / 32;
    size_t qbytes = fh_align256(n_rows * k), dbytes = fh_align256(n_rows * w->kb * 2), ebytes = fh_align256(n_rows);
    hipError_t e = hipMalloc(&w->base, qbytes + dbytes + ebytes);
    if (e != hipSuccess) {
        delete w;
        return fh_hip_fail(ctx, e, "hipMalloc(Q8_0 weight)");
    }
    w->qs = static_cast<int8_t*>(w->base);
    w->d = reinterpret_cast<uint16_t*>(static_cast<char*>(w->base) + qbytes);
    w->rexp = reinterpret_cast<int8_t*>(static_cast<char*>(w->base) + qbytes + dbytes);
    *out = w;
    return FH_OK;
}

int fh_q8_0_upload_device(fh_ctx* ctx, const uint8_t* d_gguf, size_t n_rows, size_t k,
                          fh_q8_0** out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (!d_gguf) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_upload: bytes is NULL");
    FH_ON_DEVICE(ctx);
    int rc = alloc_weight(ctx, n_rows, k, out);
    if (rc) return rc;
    rc = fh_launch_repack(ctx, d_gguf, n_rows, k, (*out)->qs, (*out)->d);
    if (rc == FH_OK) rc = fh_launch_row_exponents(ctx, (*out)->d, n_rows, k / 32, (*out)->rexp);
    if (rc) {
        fh_q8_0_free(*out);
        *out = nullptr;
    }
    return rc;
}

int fh_q8_0_upload(fh_ctx* ctx, const uint8_t* gguf, size_t n_rows, size_t k, fh_q8_0** out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (!gguf) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_upload: bytes is NULL");
    if (k == 0 || k % 32 != 0 || n_rows == 0) return alloc_weight(ctx, n_rows, k, out);
    FH_ON_DEVICE(ctx);
    size_t raw = n_rows * (k / 32) * 34;
    void* d_raw = nullptr;
    FH_HIP(ctx, hipMalloc(&d_raw, raw));
    hipError_t e = hipMemcpyAsync(d_raw, gguf, raw, hipMemcpyHostToDevice, ctx->stream);
    int rc = e == hipSuccess ? fh_q8_0_upload_device(ctx, static_cast<uint8_t*>(d_raw), n_rows, k, out)
                             : fh_hip_fail(ctx, e, "hipMemcpyAsync(weight upload)");
    hipError_t es = hipStreamSynchronize(ctx->stream);
    (void)hipFree(d_raw);
    if (rc == FH_OK && es != hipSuccess) {
        fh_q8_0_free(*out);
        *out = nullptr;
        return fh_hip_fail(ctx, es, "hipStreamSynchronize(weight upload)");
    }
    return rc;
}

int fh_weight_upload_f32(fh_ctx* ctx, const float* rows, size_t n_rows, size_t k, fh_q8_0** out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (!out) return fh_fail(ctx, FH_ERR_INVALID, "fh_weight_upload_f32: out is NULL");
    *out = nullptr;
    if (!rows) return fh_fail(ctx, FH_ERR_INVALID, "fh_weight_upload_f32: rows is NULL");
    if (n_rows == 0 || k == 0) return fh_fail(ctx, FH_ERR_INVALID, "fh_weight_upload_f32: empty matrix");
    if (n_rows > 0x7FFFFFFFu || k > 0x7FFFFFFFu)
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_weight_upload_f32: a dimension is above 2^31 - 1");
    FH_ON_DEVICE(ctx);
    fh_q8_0* w = new (std::nothrow) fh_q8_0();
    if (!w) return fh_fail(ctx, FH_ERR_OOM, "fh_weight_upload_f32: out of host memory");
    w->device = ctx->device;
    w->kind = FH_WEIGHT_F32;
    w->n = n_rows;
    w->k = k;
    w->pitch = (k + 15) / 16 * 16;
    hipError_t e = hipMalloc(&w->base, fh_align256(n_rows * w->pitch * sizeof(float)));
    if (e != hipSuccess) {
        delete w;
        return fh_hip_fail(ctx, e, "hipMalloc(F32 weight)");
    }
    w->f32 = static_cast<float*>(w->base);
    // rows padded to the pitch with zeros, in one strided copy
    e = hipMemsetAsync(w->f32, 0, n_rows * w->pitch * sizeof(float), ctx->stream);
    if (e == hipSuccess)
        e = hipMemcpy2DAsync(w->f32, w->pitch * sizeof(float), rows, k * sizeof(float), k * sizeof(float), n_rows,
                             hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(w->base);
        delete w;
        return fh_hip_fail(ctx, e, "fh_weight_upload_f32 copy");
    }
    *out = w;
    return FH_OK;
}

int fh_weight_kind(const fh_q8_0* w) { return w ? w->kind : -1; }

int fh_q8_0_download(fh_ctx* ctx, const fh_q8_0* w, uint8_t* gguf) {
    if (!ctx || !w || !gguf) return ctx ? fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_download: NULL argument") : FH_ERR_INVALID;
    ctx->err.clear();
    if (w->kind != FH_WEIGHT_Q8_0) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_download: the weight is F32, not Q8_0");
    FH_ON_DEVICE(ctx);
    size_t raw = w->n * w->kb * 34;
    void* d_raw = nullptr;
    FH_HIP(ctx, hipMalloc(&d_raw, raw));
    int rc = fh_launch_unpack(ctx, w->qs, w->d, w->n, w->k, static_cast<uint8_t*>(d_raw));
    if (rc == FH_OK) {
        hipError_t e = hipMemcpyAsync(gguf, d_raw, raw, hipMemcpyDeviceToHost, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) rc = fh_hip_fail(ctx, e, "fh_q8_0_download copy");
    } else {
        (void)hipStreamSynchronize(ctx->stream);
    }
    (void)hipFree(d_raw);
    return rc;
}

int fh_q8_0_dims(const fh_q8_0* w, size_t* n_rows, size_t* k) {
    if (!w) return FH_ERR_INVALID;
    if (n_rows) *n_rows = w->n;
    if (k) *k = w->k;
    return FH_OK;
}

void fh_q8_0_free(fh_q8_0* w) {
    if (!w) return;
    // The weight does not hold its context (which may be gone by now); hipFree
    // itself waits for the device's outstanding work before releasing memory.
    (void)on_device(w->device);
    if (w->base) (void)hipFree(w->base);
    delete w;
}

// ---- linear --------------------------------------------------------------------

// Shape checks of ops::linear_forward (ops.rs:236-246) / Linear::forward
// (layer/linear.rs:178-183), with the reference's messages.
static int check_linear(fh_ctx* ctx, const fh_q8_0* w, size_t k, const void* bias, size_t bias_len,
                        int numerics) {
    if (!w) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear: weight is NULL");
    if (numerics != FH_W8A32 && numerics != FH_W8A8 && numerics != FH_W8A32_EXACT && numerics != FH_W8A8_FAST)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear: unknown numerics " + std::to_string(numerics));
    if (w->device != ctx->device)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear: weight lives on another device");
    if (w->kind == FH_WEIGHT_F32 && (numerics == FH_W8A8 || numerics == FH_W8A8_FAST))
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear: FH_W8A8 needs a Q8_0 weight (this one is F32)");
    if (k != w->k)
        return fh_fail(ctx, FH_ERR_DIM, "linear_forward: input width " + std::to_string(k) +
                                            " \xe2\x89\xa0 weight rows " + std::to_string(w->k));
    if ((bias == nullptr) != (bias_len == 0) || (bias_len != 0 && bias_len != w->n))
        return fh_fail(ctx, FH_ERR_DIM, "linear_forward: bias length " + std::to_string(bias_len) +
                                            " \xe2\x89\xa0 out_features " + std::to_string(w->n));
    return FH_OK;
}

// The linear in one numerics mode; the W8A32 kernels apply the activation
// themselves, the other modes by a GELU pass after the linear.
// F32 weights take the exact kernel whatever the numerics (W8A32 and
// W8A32_EXACT agree there: the reference's f32 sums, bit for bit).
static int launch_linear(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const float* bias, float* y,
                         int numerics, int act = FH_ACT_NONE) {
    if (w->kind == FH_WEIGHT_F32) numerics = FH_W8A32_EXACT;
    if (numerics == FH_W8A32) return fh_launch_linear_w8a32(ctx, w, x, m, bias, y, act);
    int rc = numerics == FH_W8A8 || numerics == FH_W8A8_FAST
                 ? fh_launch_linear_w8a8(ctx, w, x, m, bias, y, numerics == FH_W8A8_FAST)
                 : fh_launch_linear_exact(ctx, w, x, m, bias, y);
    if (rc == FH_OK && act == FH_ACT_GELU) rc = fh_launch_gelu(ctx, y, m * w->n);
    return rc;
}

int fh_q8_0_linear_async(fh_ctx* ctx, const fh_q8_0* w, const float* d_x, size_t m, size_t k,
                         const float* d_bias, size_t bias_len, float* d_y, int numerics) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    int rc = check_linear(ctx, w, k, d_bias, bias_len, numerics);
    if (rc) return rc;
    if (m == 0) return FH_OK;
    if (!d_x || !d_y) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear: x or y is NULL");
    FH_ON_DEVICE(ctx);
    return launch_linear(ctx, w, d_x, m, d_bias, d_y, numerics);
}

int fh_q8_0_linear(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, size_t k,
                   const float* bias, size_t bias_len, float* y, int numerics) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    int rc = check_linear(ctx, w, k, bias, bias_len, numerics);
    if (rc) return rc;
    if (m == 0) return FH_OK;
    if (!x || !y) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear: x or y is NULL");
    FH_ON_DEVICE(ctx);
    size_t xb = fh_align256(m * k * 4), bb = fh_align256(bias_len * 4), yb = fh_align256(m * w->n * 4);
    // Device copies of the arguments live in the context's io area, apart
    // from ctx->ws, which the kernels themselves may use.
    char* dev = nullptr;
    if ((rc = io_area(ctx, xb + bb + yb, &dev))) return rc;
    float* dx = reinterpret_cast<float*>(dev);
    float* db = bias_len ? reinterpret_cast<float*>(dev + xb) : nullptr;
    float* dy = reinterpret_cast<float*>(dev + xb + bb);
    // Small calls (the decode shapes) go through pinned staging: x and bias
    // in one copy, y out in one; large ones copy the caller's memory directly.
    char* pin = nullptr;
    const bool staged = xb + bb <= kPinMax && yb <= kPinMax;
    if (staged && (rc = pin_area(ctx, std::max(xb + bb, yb), &pin))) return rc;
    hipError_t e;
    if (staged) {
        std::memcpy(pin, x, m * k * 4);
        if (bias_len) std::memcpy(pin + xb, bias, bias_len * 4);
        e = hipMemcpyAsync(dx, pin, xb + bias_len * 4, hipMemcpyHostToDevice, ctx->stream);
    } else {
        e = hipMemcpyAsync(dx, x, m * k * 4, hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess && db) e = hipMemcpyAsync(db, bias, bias_len * 4, hipMemcpyHostToDevice, ctx->stream);
    }
    if (e != hipSuccess) rc = fh_hip_fail(ctx, e, "fh_q8_0_linear copy-in");
    if (rc == FH_OK) rc = launch_linear(ctx, w, dx, m, db, dy, numerics);
    if (rc == FH_OK) {
        // (stream order: the staging's copy-in has finished before this reuses it)
        e = hipMemcpyAsync(staged ? static_cast<void*>(pin) : static_cast<void*>(y), dy, m * w->n * 4,
                           hipMemcpyDeviceToHost, ctx->stream);
        if (e != hipSuccess) rc = fh_hip_fail(ctx, e, "fh_q8_0_linear copy-out");
    }
    e = hipStreamSynchronize(ctx->stream);
    if (rc == FH_OK && e != hipSuccess) rc = fh_hip_fail(ctx, e, "fh_q8_0_linear sync");
    if (rc == FH_OK && staged) std::memcpy(y, pin, m * w->n * 4);
    return rc;
}

// ---- Q8_0 codec ----------------------------------------------------------------

int fh_q8_0_encode_async(fh_ctx* ctx, const float* d_x, size_t n, uint8_t* d_out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (n % 32 != 0)
        return fh_fail(ctx, FH_ERR_INVALID, "tensor length " + std::to_string(n) +
                                                " is not a multiple of block size 32");
    if (n == 0) return FH_OK;
    if (!d_x || !d_out) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_encode: NULL buffer");
    FH_ON_DEVICE(ctx);
    return fh_launch_encode(ctx, d_x, n, d_out);
}

int fh_q8_0_encode(fh_ctx* ctx, const float* x, size_t n, uint8_t* out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (n % 32 != 0)
        return fh_fail(ctx, FH_ERR_INVALID, "tensor length " + std::to_string(n) +
                                                " is not a multiple of block size 32");
    if (n == 0) return FH_OK;
    if (!x || !out) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_encode: NULL buffer");
    FH_ON_DEVICE(ctx);
    size_t xb = fh_align256(n * 4), ob = n / 32 * 34;
    char* dev = nullptr;
    int rc = io_area(ctx, xb + ob, &dev);
    if (rc) return rc;
    hipError_t e = hipMemcpyAsync(dev, x, n * 4, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) rc = fh_hip_fail(ctx, e, "fh_q8_0_encode copy-in");
    if (rc == FH_OK) rc = fh_launch_encode(ctx, reinterpret_cast<float*>(dev), n, reinterpret_cast<uint8_t*>(dev + xb));
    if (rc == FH_OK) {
        e = hipMemcpyAsync(out, dev + xb, ob, hipMemcpyDeviceToHost, ctx->stream);
        if (e != hipSuccess) rc = fh_hip_fail(ctx, e, "fh_q8_0_encode copy-out");
    }
    e = hipStreamSynchronize(ctx->stream);
    if (rc == FH_OK && e != hipSuccess) rc = fh_hip_fail(ctx, e, "fh_q8_0_encode sync");
    return rc;
}

int fh_q8_0_dequant_async(fh_ctx* ctx, const uint8_t* d_raw, size_t n, float* d_out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (n % 32 != 0)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_dequant: n = " + std::to_string(n) +
                                                " is not a multiple of block size 32");
    if (n == 0) return FH_OK;
    if (!d_raw || !d_out) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_dequant: NULL buffer");
    FH_ON_DEVICE(ctx);
    return fh_launch_dequant(ctx, d_raw, n, d_out);
}

int fh_q8_0_block_dots_async(fh_ctx* ctx, const fh_q8_0* w, const int8_t* d_qx, size_t m,
                             int32_t* d_dots) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (!w) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_block_dots: weight is NULL");
    if (w->kind != FH_WEIGHT_Q8_0) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_block_dots: the weight is F32, not Q8_0");
    if (m == 0) return FH_OK;
    if (!d_qx || !d_dots) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_block_dots: NULL buffer");
    FH_ON_DEVICE(ctx);
    return fh_launch_block_dots(ctx, w, d_qx, m, d_dots);
}

// ---- sampler -------------------------------------------------------------------

static int check_sample(fh_ctx* ctx, size_t rows, size_t vocab, int kind, const fh_sampling_params* p) {
    if (!p) return fh_fail(ctx, FH_ERR_INVALID, "fh_sample_rows: params is NULL");
    const int base = kind & ~FH_RECENT_RANGES;
    if (base != FH_LOGITS_RAW && base != FH_LOGITS_GPT2_SOFTMAX)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_sample_rows: unknown logits kind " + std::to_string(kind));
    if (vocab == 0) return fh_fail(ctx, FH_ERR_INVALID, "fh_sample_rows: vocab is 0");
    if (vocab > 0x7FFFFFFFu) return fh_fail(ctx, FH_ERR_LIMIT, "fh_sample_rows: vocab above 2^31 - 1");
    if (rows > 0x7FFFFFFFu) return fh_fail(ctx, FH_ERR_LIMIT, "fh_sample_rows: rows above 2^31 - 1");
    return FH_OK;
}

static int check_offsets(fh_ctx* ctx, const uint32_t* off, size_t rows, const void* recent) {
    if (!off) return FH_OK;
    for (size_t r = 0; r < rows; r++) {
        if (off[r + 1] < off[r])
            return fh_fail(ctx, FH_ERR_INVALID, "fh_sample_rows: recent_offsets decrease at row " + std::to_string(r));
    }
    if (off[rows] != off[0] && !recent) return fh_fail(ctx, FH_ERR_INVALID, "fh_sample_rows: recent is NULL");
    return FH_OK;
}

int fh_sample_rows_async(fh_ctx* ctx, const float* d_logits, size_t rows, size_t vocab, int kind,
                         const fh_sampling_params* p, const uint32_t* d_recent,
                         const uint32_t* d_off, const uint64_t* d_draws, uint32_t* d_out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    int rc = check_sample(ctx, rows, vocab, kind, p);
    if (rc) return rc;
    if (rows == 0) return FH_OK;
    if (!d_logits || !d_out) return fh_fail(ctx, FH_ERR_INVALID, "fh_sample_rows: logits or out_ids is NULL");
    if (!d_draws && !(p->temperature <= 0.0f))
        return fh_fail(ctx, FH_ERR_INVALID, "fh_sample_rows: draws is NULL with temperature > 0");
    // Device offsets cannot be inspected without a copy: the kernels record
    // decreasing offsets in the status word, which fh_sync reports.
    FH_ON_DEVICE(ctx);
    return fh_launch_sample(ctx, d_logits, rows, vocab, kind, p, d_recent, d_off, d_draws, d_out);
}

int fh_sample_rows(fh_ctx* ctx, const float* logits, size_t rows, size_t vocab, int kind,
                   const fh_sampling_params* p, const uint32_t* recent, const uint32_t* off,
                   const uint64_t* draws, uint32_t* out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    int rc = check_sample(ctx, rows, vocab, kind, p);
    if (rc) return rc;
    if (rows == 0) return FH_OK;
    if (!logits || !out) return fh_fail(ctx, FH_ERR_INVALID, "fh_sample_rows: logits or out_ids is NULL");
    bool sampled = !(p->temperature <= 0.0f);
    if (!draws && sampled) return fh_fail(ctx, FH_ERR_INVALID, "fh_sample_rows: draws is NULL with temperature > 0");
    if (kind & FH_RECENT_RANGES)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_sample_rows: FH_RECENT_RANGES is for fh_sample_rows_async "
                                            "(host lists go as running offsets)");
    if ((rc = check_offsets(ctx, off, rows, recent))) return rc;
    FH_ON_DEVICE(ctx);
    size_t n_recent = off ? off[rows] - off[0] : 0;
    size_t lb = fh_align256(rows * vocab * 4), rb = fh_align256(n_recent * 4 + 4),
           ob = fh_align256((rows + 1) * 4), db = fh_align256(rows * 8), yb = fh_align256(rows * 4);
    char* dev = nullptr;
    if ((rc = io_area(ctx, lb + rb + ob + db + yb, &dev))) return rc;
    float* d_logits = reinterpret_cast<float*>(dev);
    uint32_t* d_recent = reinterpret_cast<uint32_t*>(dev + lb);
    uint32_t* d_off = reinterpret_cast<uint32_t*>(dev + lb + rb);
    uint64_t* d_draws = reinterpret_cast<uint64_t*>(dev + lb + rb + ob);
    uint32_t* d_out = reinterpret_cast<uint32_t*>(dev + lb + rb + ob + db);
    hipError_t e = hipMemcpyAsync(d_logits, logits, rows * vocab * 4, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess && n_recent)
        e = hipMemcpyAsync(d_recent, recent + off[0], n_recent * 4, hipMemcpyHostToDevice, ctx->stream);
    // Rebase the offsets so the device list starts at 0.
    uint32_t* hoff = nullptr;
    if (e == hipSuccess && off) {
        hoff = new (std::nothrow) uint32_t[rows + 1];
        if (!hoff) rc = fh_fail(ctx, FH_ERR_OOM, "fh_sample_rows: out of host memory");
        else {
            for (size_t r = 0; r <= rows; r++) hoff[r] = off[r] - off[0];
            e = hipMemcpyAsync(d_off, hoff, (rows + 1) * 4, hipMemcpyHostToDevice, ctx->stream);
        }
    }
    if (e == hipSuccess && draws) e = hipMemcpyAsync(d_draws, draws, rows * 8, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess && rc == FH_OK) rc = fh_hip_fail(ctx, e, "fh_sample_rows copy-in");
    if (rc == FH_OK)
        rc = fh_launch_sample(ctx, d_logits, rows, vocab, kind, p, n_recent ? d_recent : nullptr,
                              off ? d_off : nullptr, draws ? d_draws : nullptr, d_out);
    if (rc == FH_OK) {
        e = hipMemcpyAsync(out, d_out, rows * 4, hipMemcpyDeviceToHost, ctx->stream);
        if (e != hipSuccess) rc = fh_hip_fail(ctx, e, "fh_sample_rows copy-out");
    }
    e = hipStreamSynchronize(ctx->stream);
    if (rc == FH_OK && e != hipSuccess) rc = fh_hip_fail(ctx, e, "fh_sample_rows sync");
    if (rc == FH_OK) rc = fh_take_status(ctx);
    delete[] hoff;
    return rc;
}

int fh_debug_sampler_faults(fh_ctx* ctx, int skip_segment, uint32_t spin_limit) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    ctx->test_skip_segment = skip_segment < 0 ? -1 : skip_segment;
    ctx->test_spin_limit = spin_limit;
    return FH_OK;
}

}  // extern "C"

// ---- the rest of a GPT-2 decode step --------------------------------------------

int fh_embed_one_async(fh_ctx* ctx, const float* d_token_w, const float* d_pos_w, size_t vocab, size_t max_seq,
                       size_t d, const uint32_t* d_token, size_t pos, float* d_out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (!d_token_w || !d_pos_w || !d_token || !d_out)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_embed_one: a pointer is NULL");
    if (vocab == 0 || d == 0 || vocab > 0x7FFFFFFFu || d > 0x7FFFFFFFu)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_embed_one: vocab and d must be in 1 .. 2^31");
    if (pos >= max_seq)
        return fh_fail(ctx, FH_ERR_DIM, "Position " + std::to_string(pos) + " exceeds max_seq_len " +
                                            std::to_string(max_seq));
    FH_ON_DEVICE(ctx);
    return fh_launch_embed_one(ctx, d_token_w, d_pos_w, vocab, d, d_token, pos, d_out);
}

int fh_embed_rows_pos_async(fh_ctx* ctx, const float* d_token_w, const float* d_pos_w, size_t vocab, size_t max_seq,
                            size_t d, const uint32_t* d_tokens, const uint32_t* d_pos, size_t rows, uint32_t* d_hist,
                            size_t hist_stride, float* d_out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (rows == 0) return FH_OK;
    if (!d_token_w || !d_pos_w || !d_tokens || !d_pos || !d_out)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_embed_rows_pos: a pointer is NULL");
    if (vocab == 0 || d == 0 || max_seq == 0 || vocab > 0x7FFFFFFFu || max_seq > 0x7FFFFFFFu || rows > 65535 ||
        rows * d > 0x7FFFFFFFu)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_embed_rows_pos: vocab, max_seq and rows * d in 1 .. 2^31, rows "
                                            "<= 65535");
    if (d_hist && (hist_stride == 0 || hist_stride > 0x7FFFFFFFu || rows * hist_stride > 0xFFFFFFFFu))
        return fh_fail(ctx, FH_ERR_INVALID, "fh_embed_rows_pos: hist_stride in 1 .. 2^31, rows * hist_stride "
                                            "below 2^32");
    FH_ON_DEVICE(ctx);
    return fh_launch_embed_rows_pos(ctx, d_token_w, d_pos_w, vocab, max_seq, d, d_tokens, d_pos, rows, d_hist,
                                    d_hist ? hist_stride : 0, d_out);
}

int fh_layernorm_async(fh_ctx* ctx, const float* d_x, size_t rows, size_t d, const float* d_gamma,
                       const float* d_beta, float* d_y) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (rows == 0) return FH_OK;
    if (!d_x || !d_gamma || !d_beta || !d_y) return fh_fail(ctx, FH_ERR_INVALID, "fh_layernorm: a pointer is NULL");
    if (d == 0 || d > 0x7FFFFFFFu || rows > 0x7FFFFFFFu)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_layernorm: rows and d must be in 1 .. 2^31");
    FH_ON_DEVICE(ctx);
    return fh_launch_layernorm(ctx, d_x, rows, d, d_gamma, d_beta, d_y);
}

int fh_gelu_async(fh_ctx* ctx, float* d_x, size_t n) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (n == 0) return FH_OK;
    if (!d_x) return fh_fail(ctx, FH_ERR_INVALID, "fh_gelu: x is NULL");
    FH_ON_DEVICE(ctx);
    return fh_launch_gelu(ctx, d_x, n);
}

int fh_add_async(fh_ctx* ctx, float* d_x, const float* d_y, size_t n) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (n == 0) return FH_OK;
    if (!d_x || !d_y) return fh_fail(ctx, FH_ERR_INVALID, "fh_add: x or y is NULL");
    FH_ON_DEVICE(ctx);
    return fh_launch_add(ctx, d_x, d_y, n);
}

int fh_attention_decode_async(fh_ctx* ctx, const float* d_qkv, float* d_k_cache, float* d_v_cache,
                              size_t capacity, size_t d, size_t heads, size_t pos, float* d_out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (!d_qkv || !d_k_cache || !d_v_cache || !d_out)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_attention_decode: a pointer is NULL");
    if (heads == 0 || d == 0 || d % heads != 0)
        return fh_fail(ctx, FH_ERR_DIM, "fh_attention_decode: heads (" + std::to_string(heads) +
                                            ") must divide the embedding dim (" + std::to_string(d) + ")");
    if (pos >= capacity)
        return fh_fail(ctx, FH_ERR_DIM, "KvCache full (" + std::to_string(capacity) +
                                            " positions): clear and re-prime to continue");
    if (d > 0x7FFFFFFFu || capacity > 0x7FFFFFFFu || capacity * d > (size_t(1) << 40))
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_attention_decode: cache too large");
    FH_ON_DEVICE(ctx);
    return fh_launch_attention_decode(ctx, d_qkv, d_k_cache, d_v_cache, d, heads, pos, d_out);
}

int fh_attention_prefill_async(fh_ctx* ctx, const float* d_qkv, float* d_k_cache, float* d_v_cache,
                               size_t capacity, size_t d, size_t heads, size_t pos0, size_t rows, float* d_out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (rows == 0) return FH_OK;
    if (!d_qkv || !d_k_cache || !d_v_cache || !d_out)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_attention_prefill: a pointer is NULL");
    if (heads == 0 || d == 0 || d % heads != 0)
        return fh_fail(ctx, FH_ERR_DIM, "fh_attention_prefill: heads (" + std::to_string(heads) +
                                            ") must divide the embedding dim (" + std::to_string(d) + ")");
    if (pos0 + rows > capacity)
        return fh_fail(ctx, FH_ERR_DIM, "KvCache full (" + std::to_string(capacity) +
                                            " positions): clear and re-prime to continue");
    if (d > 0x7FFFFFFFu || capacity > 0x7FFFFFFFu || capacity * d > (size_t(1) << 40) || rows > 65535)
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_attention_prefill: cache or block too large");
    FH_ON_DEVICE(ctx);
    return fh_launch_attention_prefill_seqs(ctx, d_qkv, d_k_cache, d_v_cache, 0, d, heads, pos0, rows, 1, d_out);
}

int fh_attention_prefill_seqs_async(fh_ctx* ctx, const float* d_qkv, float* d_k_cache, float* d_v_cache,
                                    size_t seq_stride, size_t capacity, size_t d, size_t heads, size_t pos0,
                                    size_t rows, size_t seqs, float* d_out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (rows == 0 || seqs == 0) return FH_OK;
    if (!d_qkv || !d_k_cache || !d_v_cache || !d_out)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_attention_prefill: a pointer is NULL");
    if (heads == 0 || d == 0 || d % heads != 0)
        return fh_fail(ctx, FH_ERR_DIM, "fh_attention_prefill: heads (" + std::to_string(heads) +
                                            ") must divide the embedding dim (" + std::to_string(d) + ")");
    if (pos0 + rows > capacity)
        return fh_fail(ctx, FH_ERR_DIM, "KvCache full (" + std::to_string(capacity) +
                                            " positions): clear and re-prime to continue");
    if (d > 0x7FFFFFFFu || capacity > 0x7FFFFFFFu || capacity * d > (size_t(1) << 40) || rows > 65535 ||
        seqs > 65535 || seqs * rows * 3 * d > (size_t(1) << 40))
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_attention_prefill: cache or block too large");
    if (seqs > 1 && seq_stride < capacity * d)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_attention_prefill: seq_stride " + std::to_string(seq_stride) +
                                                " below capacity x d = " + std::to_string(capacity * d));
    FH_ON_DEVICE(ctx);
    return fh_launch_attention_prefill_seqs(ctx, d_qkv, d_k_cache, d_v_cache, seqs > 1 ? seq_stride : 0, d, heads,
                                            pos0, rows, seqs, d_out);
}

int fh_q8_0_linear_act_async(fh_ctx* ctx, const fh_q8_0* w, const float* d_x, size_t m, size_t k,
                             const float* d_bias, size_t bias_len, float* d_y, int numerics, int activation) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (activation != FH_ACT_NONE && activation != FH_ACT_GELU)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear: unknown activation " + std::to_string(activation));
    int rc = check_linear(ctx, w, k, d_bias, bias_len, numerics);
    if (rc) return rc;
    if (m == 0) return FH_OK;
    if (!d_x || !d_y) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear: x or y is NULL");
    FH_ON_DEVICE(ctx);
    return launch_linear(ctx, w, d_x, m, d_bias, d_y, numerics, activation);
}

int fh_add_layernorm_async(fh_ctx* ctx, float* d_x, const float* d_y, size_t rows, size_t d, const float* d_gamma,
                           const float* d_beta, float* d_ln) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (rows == 0) return FH_OK;
    if (!d_x || !d_y || !d_gamma || !d_beta || !d_ln)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_add_layernorm: a pointer is NULL");
    if (d == 0 || rows > 0x7FFFFFFFu)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_add_layernorm: d must be positive");
    FH_ON_DEVICE(ctx);
    return fh_launch_add_layernorm(ctx, d_x, d_y, d_x, rows, d, d_gamma, d_beta, d_ln);
}

int fh_q8_0_linear_ln_async(fh_ctx* ctx, const fh_q8_0* w, const float* d_x, const float* d_r, float* d_s, size_t m,
                            size_t k, const float* d_gamma, const float* d_beta, const float* d_bias, size_t bias_len,
                            float* d_y, int numerics, int activation) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (activation != FH_ACT_NONE && activation != FH_ACT_GELU)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear_ln: unknown activation " + std::to_string(activation));
    int rc = check_linear(ctx, w, k, d_bias, bias_len, numerics);
    if (rc) return rc;
    if (m == 0) return FH_OK;
    if (!d_x || !d_y || !d_gamma || !d_beta)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear_ln: x, y, gamma or beta is NULL");
    if (d_s && (d_s == d_x || d_s == d_r))
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear_ln: s must not alias x or r");
    if (k > 2048) return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear_ln: rows wider than 2048");
    if (m > 0x7FFFFFFFu) return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear_ln: m is above 2^31 - 1");
    FH_ON_DEVICE(ctx);
    if (numerics == FH_W8A32 && w->kind == FH_WEIGHT_Q8_0) {
        const fh_ln_args ln{d_r, d_gamma, d_beta, d_s};
        return fh_launch_linear_ln_w8a32(ctx, w, d_x, m, ln, d_bias, d_y, activation);
    }
    void* h = nullptr;
    rc = fh_act_area(ctx, m * k * sizeof(float), &h);
    if (rc) return rc;
    float* hf = static_cast<float*>(h);
    rc = fh_launch_add_layernorm(ctx, d_x, d_r, d_s, m, k, d_gamma, d_beta, hf);
    if (rc) return rc;
    return launch_linear(ctx, w, hf, m, d_bias, d_y, numerics, activation);
}

int fh_q8_0_linear_residual_async(fh_ctx* ctx, const fh_q8_0* w, const float* d_x, size_t m, size_t k,
                                  const float* d_bias, size_t bias_len, const float* d_r, float* d_y,
                                  float* d_stats) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    int rc = check_linear(ctx, w, k, d_bias, bias_len, FH_W8A32);
    if (rc) return rc;
    if (m == 0) return FH_OK;
    if (!d_x || !d_r || !d_y) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear_residual: x, r or y is NULL");
    if (d_y == d_x) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear_residual: y must not alias x");
    if (d_stats && (w->n & 31))
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear_residual: row statistics need out_features % 32 == 0");
    if (m > 0x7FFFFFFFu || w->n > 0x7FFFFFFFu) return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear_residual: too large");
    FH_ON_DEVICE(ctx);
    if (d_stats && w->kind == FH_WEIGHT_Q8_0) {
        fh_edge e{};
        e.stats = d_stats;
        e.r = d_r;
        rc = fh_launch_skinny_res_out(ctx, w, d_x, m, e, d_bias, d_y);
        if (rc >= 0) return rc;
    }
    // other shapes: the linear into the activation area, then the add (and statistics)
    void* t = nullptr;
    rc = fh_act_area(ctx, m * w->n * sizeof(float), &t);
    if (rc) return rc;
    rc = launch_linear(ctx, w, d_x, m, d_bias, static_cast<float*>(t), FH_W8A32);
    if (rc) return rc;
    return fh_launch_residual_stats(ctx, static_cast<const float*>(t), d_r, d_y, m, w->n, d_stats);
}

int fh_q8_0_linear_normed_async(fh_ctx* ctx, const fh_q8_0* w, const float* d_x, size_t m, size_t k,
                                const float* d_stats, const float* d_gamma, const float* d_beta, float eps, int rms,
                                const float* d_bias, size_t bias_len, float* d_y, int activation) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (activation != FH_ACT_NONE && activation != FH_ACT_GELU && activation != FH_ACT_SWIGLU32)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear_normed: unknown activation " + std::to_string(activation));
    int rc = check_linear(ctx, w, k, d_bias, bias_len, FH_W8A32);
    if (rc) return rc;
    if (m == 0) return FH_OK;
    if (!d_x || !d_y || !d_stats || !d_gamma)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear_normed: x, y, stats or gamma is NULL");
    if (rms != 0 && rms != 1) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear_normed: rms must be 0 or 1");
    if (!rms && !d_beta) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear_normed: LayerNorm needs beta");
    if (k & 31) return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear_normed: row statistics need k % 32 == 0");
    if (m > 0x7FFFFFFFu) return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear_normed: m is above 2^31 - 1");
    FH_ON_DEVICE(ctx);
    fh_edge e{};
    e.stats = const_cast<float*>(d_stats);
    e.gamma = d_gamma;
    e.beta = rms ? nullptr : d_beta;
    e.eps = eps;
    e.rms = rms;
    if (activation == FH_ACT_SWIGLU32 && (w->kind != FH_WEIGHT_Q8_0 || w->n % 64 || m < 3 || m > 64 || k > 1024))
        return fh_fail(ctx, FH_ERR_LIMIT,
                       "fh_q8_0_linear_normed: FH_ACT_SWIGLU32 needs a Q8_0 weight with n % 64 == 0, "
                       "3 <= m <= 64 and k <= 1024");
    if (w->kind == FH_WEIGHT_Q8_0) {
        rc = fh_launch_skinny_norm_in(ctx, w, d_x, m, e, d_bias, d_y, activation);
        if (rc >= 0) return rc;
    }
    void* h = nullptr;
    rc = fh_act_area(ctx, m * k * sizeof(float), &h);
    if (rc) return rc;
    rc = fh_launch_norm_from_stats(ctx, d_x, m, k, e, static_cast<float*>(h));
    if (rc) return rc;
    return launch_linear(ctx, w, static_cast<float*>(h), m, d_bias, d_y, FH_W8A32, activation);
}

// ---- Llama / Qwen block pieces ---------------------------------------------------

int fh_rmsnorm_async(fh_ctx* ctx, const float* d_x, const float* d_r, float* d_s, size_t rows, size_t d,
                     const float* d_w, float eps, float* d_out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (rows == 0) return FH_OK;
    if (!d_x || !d_w || !d_out) return fh_fail(ctx, FH_ERR_INVALID, "fh_rmsnorm: x, w or out is NULL");
    if (d == 0 || rows > 0x7FFFFFFFu) return fh_fail(ctx, FH_ERR_INVALID, "fh_rmsnorm: d must be positive");
    if (d_s && d_r && d_s == d_r) return fh_fail(ctx, FH_ERR_INVALID, "fh_rmsnorm: s must not alias r");
    FH_ON_DEVICE(ctx);
    return fh_launch_rmsnorm(ctx, d_x, d_r, d_s, rows, d, d_w, eps, d_out);
}

int fh_rope_async(fh_ctx* ctx, float* d_x, size_t rows, size_t ld, size_t n_heads, size_t head_dim, size_t rope_dim,
                  const uint32_t* d_pos, float base, int rope_type, const float* d_freq_factors, float linear_factor) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (rope_dim > head_dim || rope_dim % 2 != 0)
        return fh_fail(ctx, FH_ERR_DIM, "rope_dim " + std::to_string(rope_dim) + " must be even and \u2264 head_dim " +
                                            std::to_string(head_dim));
    if (!(linear_factor > 0.0f) || !std::isfinite(linear_factor))
        return fh_fail(ctx, FH_ERR_DIM, "RoPE scaling factors must be finite and > 0");
    if (rope_type != FH_ROPE_NORM && rope_type != FH_ROPE_NEOX)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_rope: unknown rope_type " + std::to_string(rope_type));
    if (rows == 0 || n_heads == 0 || rope_dim == 0) return FH_OK;
    if (!d_x || !d_pos) return fh_fail(ctx, FH_ERR_INVALID, "fh_rope: x or pos is NULL");
    if (ld < n_heads * head_dim) return fh_fail(ctx, FH_ERR_DIM, "fh_rope: ld is below n_heads * head_dim");
    if (rows * ld > 0x7FFFFFFFu) return fh_fail(ctx, FH_ERR_LIMIT, "fh_rope: more than 2^31 - 1 values");
    FH_ON_DEVICE(ctx);
    return fh_launch_rope(ctx, d_x, rows, ld, n_heads, head_dim, rope_dim, d_pos, base, rope_type, d_freq_factors,
                          linear_factor);
}

int fh_gqa_attention_decode_async(fh_ctx* ctx, const float* d_qkv, size_t ld, size_t rows, size_t n_heads,
                                  size_t n_kv, size_t head_dim, float* d_k_cache, float* d_v_cache, size_t capacity,
                                  const uint32_t* d_pos, size_t max_pos, float* d_out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (n_kv == 0 || n_heads % n_kv != 0)
        return fh_fail(ctx, FH_ERR_DIM, "n_heads " + std::to_string(n_heads) + " must be a multiple of n_kv_heads " +
                                            std::to_string(n_kv));
    if (rows == 0 || n_heads == 0) return FH_OK;
    if (!d_qkv || !d_k_cache || !d_v_cache || !d_pos || !d_out)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_gqa_attention_decode: a pointer is NULL");
    if (capacity == 0) return fh_fail(ctx, FH_ERR_INVALID, "fh_gqa_attention_decode: capacity is 0");
    if (ld < (n_heads + 2 * n_kv) * head_dim)
        return fh_fail(ctx, FH_ERR_DIM, "fh_gqa_attention_decode: ld is below (n_heads + 2 n_kv) * head_dim");
    if (rows > 65535 || n_heads > 65535 || ld * rows > 0x7FFFFFFFu || capacity > 0x7FFFFFFFu ||
        rows * capacity * n_kv * head_dim > (size_t(1) << 40))
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_gqa_attention_decode: a dimension is too large");
    FH_ON_DEVICE(ctx);
    return fh_launch_gqa_attention_decode(ctx, d_qkv, ld, rows, n_heads, n_kv, head_dim, d_k_cache, d_v_cache,
                                          capacity, d_pos, max_pos, d_out);
}

int fh_gqa_attention_rope_decode_async(fh_ctx* ctx, float* d_qkv, size_t ld, size_t rows, size_t n_heads,
                                       size_t n_kv, size_t head_dim, float* d_k_cache, float* d_v_cache,
                                       size_t capacity, const uint32_t* d_pos, size_t max_pos, size_t rope_dim,
                                       float base, int rope_type, const float* d_freq_factors, float linear_factor,
                                       float* d_out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (rope_dim > head_dim || rope_dim % 2 != 0)
        return fh_fail(ctx, FH_ERR_DIM, "rope_dim " + std::to_string(rope_dim) + " must be even and \u2264 head_dim " +
                                            std::to_string(head_dim));
    if (!(linear_factor > 0.0f) || !std::isfinite(linear_factor))
        return fh_fail(ctx, FH_ERR_DIM, "RoPE scaling factors must be finite and > 0");
    if (rope_type != FH_ROPE_NORM && rope_type != FH_ROPE_NEOX)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_gqa_attention_rope_decode: unknown rope_type " +
                                                std::to_string(rope_type));
    if (n_kv == 0 || n_heads % n_kv != 0)
        return fh_fail(ctx, FH_ERR_DIM, "n_heads " + std::to_string(n_heads) + " must be a multiple of n_kv_heads " +
                                            std::to_string(n_kv));
    if (rows == 0 || n_heads == 0) return FH_OK;
    if (!d_qkv || !d_k_cache || !d_v_cache || !d_pos || !d_out)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_gqa_attention_rope_decode: a pointer is NULL");
    if (capacity == 0) return fh_fail(ctx, FH_ERR_INVALID, "fh_gqa_attention_rope_decode: capacity is 0");
    if (ld < (n_heads + 2 * n_kv) * head_dim)
        return fh_fail(ctx, FH_ERR_DIM, "fh_gqa_attention_rope_decode: ld is below (n_heads + 2 n_kv) * head_dim");
    if (rows > 65535 || n_heads > 65535 || ld * rows > 0x7FFFFFFFu || capacity > 0x7FFFFFFFu ||
        rows * capacity * n_kv * head_dim > (size_t(1) << 40))
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_gqa_attention_rope_decode: a dimension is too large");
    FH_ON_DEVICE(ctx);
    return fh_launch_gqa_attention_rope_decode(ctx, d_qkv, ld, rows, n_heads, n_kv, head_dim, d_k_cache, d_v_cache,
                                               capacity, d_pos, max_pos, rope_dim, base, rope_type, d_freq_factors,
                                               linear_factor, d_out);
}

int fh_swiglu_async(fh_ctx* ctx, const float* d_g, const float* d_u, size_t rows, size_t n, size_t ld, float* d_out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (rows == 0 || n == 0) return FH_OK;
    if (!d_g || !d_u || !d_out) return fh_fail(ctx, FH_ERR_INVALID, "fh_swiglu: a pointer is NULL");
    if (ld < n) return fh_fail(ctx, FH_ERR_DIM, "fh_swiglu: ld is below n");
    if (rows * ld > 0x7FFFFFFFu) return fh_fail(ctx, FH_ERR_LIMIT, "fh_swiglu: more than 2^31 - 1 values");
    FH_ON_DEVICE(ctx);
    return fh_launch_swiglu(ctx, d_g, d_u, rows, n, ld, d_out);
}

int fh_embed_rows_async(fh_ctx* ctx, const float* d_tok_w, size_t vocab, size_t d, const uint32_t* d_tokens,
                        size_t rows, float* d_out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (rows == 0 || d == 0) return FH_OK;
    if (!d_tok_w || !d_tokens || !d_out) return fh_fail(ctx, FH_ERR_INVALID, "fh_embed_rows: a pointer is NULL");
    if (rows * d > 0x7FFFFFFFu || vocab > 0x7FFFFFFFu)
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_embed_rows: more than 2^31 - 1 values");
    FH_ON_DEVICE(ctx);
    return fh_launch_embed_rows(ctx, d_tok_w, vocab, d, d_tokens, rows, d_out);
}
