// brik.node — Node N-API binding of libbrik.so (the C ABI of include/brik.h).
//
// Thin by design: every function converts JS arguments, calls one brik_* entry point and throws a JS
// Error on a negative return (err.code = "BRIK_EINVAL" etc., err.message = the library's message).
// Device pointers cross the boundary as BigInt addresses; the engine facade in js/index.js wraps them
// in DeviceBuffer objects with the reference engine's method names.
#include <node_api.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "brik.h"

namespace {

#define NAPI_CALL(env, call)                                                  \
    do {                                                                      \
        if ((call) != napi_ok) {                                              \
            napi_throw_error((env), "BRIK_NAPI", "N-API call failed: " #call); \
            return nullptr;                                                   \
        }                                                                     \
    } while (0)
// the same in a function returning bool
#define NAPI_CALL_B(env, call)                                                \
    do {                                                                      \
        if ((call) != napi_ok) {                                              \
            napi_throw_error((env), "BRIK_NAPI", "N-API call failed: " #call); \
            return false;                                                     \
        }                                                                     \
    } while (0)

const char* code_name(int rc)
{
    switch (rc) {
    case BRIK_EINVAL: return "BRIK_EINVAL";
    case BRIK_EALIGN: return "BRIK_EALIGN";
    case BRIK_EHIP: return "BRIK_EHIP";
    case BRIK_ENOMEM: return "BRIK_ENOMEM";
    case BRIK_ENODEV: return "BRIK_ENODEV";
    case BRIK_EMODULE: return "BRIK_EMODULE";
    default: return "BRIK_ERROR";
    }
}

// Throw for rc < 0. Returns true if an exception is pending.
bool check(napi_env env, brik_ctx* ctx, int rc)
{
    if (rc == BRIK_OK) return false;
    std::string msg = std::string(code_name(rc)) + ": " + (ctx ? brik_last_error(ctx) : brik_strerror(rc));
    napi_throw_error(env, code_name(rc), msg.c_str());
    return true;
}

struct Args {
    napi_value v[16];
    size_t n = 16;
};

bool get_args(napi_env env, napi_callback_info info, Args& a, size_t need)
{
    if (napi_get_cb_info(env, info, &a.n, a.v, nullptr, nullptr) != napi_ok) return false;
    if (a.n < need) {
        napi_throw_type_error(env, "BRIK_EINVAL", "too few arguments");
        return false;
    }
    return true;
}

bool get_i32(napi_env env, napi_value v, int32_t* out)
{
    if (napi_get_value_int32(env, v, out) != napi_ok) {
        napi_throw_type_error(env, "BRIK_EINVAL", "expected a number");
        return false;
    }
    return true;
}

bool get_f32(napi_env env, napi_value v, float* out)
{
    double d;
    if (napi_get_value_double(env, v, &d) != napi_ok) {
        napi_throw_type_error(env, "BRIK_EINVAL", "expected a number");
        return false;
    }
    *out = (float)d;
    return true;
}

// An element count: a non-negative integral Number (exact below 2^53).
bool get_size(napi_env env, napi_value v, size_t* out)
{
    double d;
    if (napi_get_value_double(env, v, &d) != napi_ok || !(d >= 0) || d != (double)(uint64_t)d || d > 9007199254740992.0) {
        napi_throw_type_error(env, "BRIK_EINVAL", "expected a non-negative integer count");
        return false;
    }
    *out = (size_t)d;
    return true;
}

// A device pointer: BigInt address, null/undefined (-> nullptr), or an object with a BigInt `ptr`.
bool get_ptr(napi_env env, napi_value v, void** out)
{
    napi_valuetype t;
    napi_typeof(env, v, &t);
    if (t == napi_null || t == napi_undefined) { *out = nullptr; return true; }
    if (t == napi_object) {
        napi_value p;
        if (napi_get_named_property(env, v, "ptr", &p) != napi_ok) return false;
        v = p;
        napi_typeof(env, v, &t);
    }
    if (t != napi_bigint) {
        napi_throw_type_error(env, "BRIK_EINVAL", "expected a device pointer (BigInt or {ptr: BigInt})");
        return false;
    }
    uint64_t u;
    bool lossless;
    if (napi_get_value_bigint_uint64(env, v, &u, &lossless) != napi_ok) return false;
    *out = reinterpret_cast<void*>(static_cast<uintptr_t>(u));
    return true;
}

// A context as JS holds it: the library context, and the count of the JS-side objects that keep it
// alive (the context handle itself, device buffers, plans). It is destroyed when the last one is
// finalized, so a buffer collected after its context never frees into a destroyed context.
struct CtxBox {
    brik_ctx* ctx;
    long refs;
    long live_buffers;   // device buffers allocated through allocBuffer and not yet freed
};

void box_release(CtxBox* b)
{
    if (--b->refs == 0) {
        brik_destroy(b->ctx);
        delete b;
    }
}

bool get_box(napi_env env, napi_value v, CtxBox** out)
{
    void* p = nullptr;
    if (napi_get_value_external(env, v, &p) != napi_ok || !p) {
        napi_throw_type_error(env, "BRIK_EINVAL", "expected a brik context");
        return false;
    }
    *out = static_cast<CtxBox*>(p);
    return true;
}

bool get_ctx(napi_env env, napi_value v, brik_ctx** out)
{
    CtxBox* b;
    if (!get_box(env, v, &b)) return false;
    *out = b->ctx;
    return true;
}

napi_value make_ptr(napi_env env, void* p)
{
    napi_value r;
    napi_create_bigint_uint64(env, static_cast<uint64_t>(reinterpret_cast<uintptr_t>(p)), &r);
    return r;
}

napi_value undefined(napi_env env)
{
    napi_value u;
    napi_get_undefined(env, &u);
    return u;
}

// Host bytes of a TypedArray / Buffer / ArrayBuffer / DataView.
bool get_bytes(napi_env env, napi_value v, void** data, size_t* len)
{
    bool is;
    napi_is_typedarray(env, v, &is);
    if (is) {
        napi_typedarray_type tt;
        size_t n, off;
        napi_value ab;
        if (napi_get_typedarray_info(env, v, &tt, &n, data, &ab, &off) != napi_ok) return false;
        size_t es = 1;
        switch (tt) {
        case napi_int16_array: case napi_uint16_array: es = 2; break;
        case napi_int32_array: case napi_uint32_array: case napi_float32_array: es = 4; break;
        case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: es = 8; break;
        default: es = 1;
        }
        *len = n * es;
        return true;
    }
    napi_is_arraybuffer(env, v, &is);
    if (is) return napi_get_arraybuffer_info(env, v, data, len) == napi_ok;
    napi_is_dataview(env, v, &is);
    if (is) {
        napi_value ab;
        size_t off;
        return napi_get_dataview_info(env, v, len, data, &ab, &off) == napi_ok;
    }
    napi_throw_type_error(env, "BRIK_EINVAL", "expected a TypedArray, ArrayBuffer or DataView");
    return false;
}

void ctx_finalize(napi_env, void* data, void*) { box_release(static_cast<CtxBox*>(data)); }

// ---- context / memory ------------------------------------------------------------------------

napi_value DeviceCount(napi_env env, napi_callback_info)
{
    int n = 0;
    brik_device_count(&n);
    napi_value r;
    NAPI_CALL(env, napi_create_int32(env, n, &r));
    return r;
}

napi_value CreateContext(napi_env env, napi_callback_info info)
{
    Args a;
    int32_t dev = 0;
    if (napi_get_cb_info(env, info, &a.n, a.v, nullptr, nullptr) != napi_ok) return nullptr;
    if (a.n >= 1 && !get_i32(env, a.v[0], &dev)) return nullptr;
    brik_ctx* ctx = nullptr;
    if (check(env, nullptr, brik_create(dev, &ctx))) return nullptr;
    CtxBox* box = new CtxBox{ctx, 1, 0};
    napi_value ext;
    if (napi_create_external(env, box, ctx_finalize, nullptr, &ext) != napi_ok) {
        box_release(box);
        napi_throw_error(env, "BRIK_NAPI", "napi_create_external failed");
        return nullptr;
    }
    return ext;
}

// ---- device buffers owned by JS objects -------------------------------------------------------
// allocBuffer(ctx, bytes) -> handle: a device allocation freed by freeBuffer(handle) or, if the handle
// is dropped first, by its finalizer when the garbage collector reclaims it (the reference's
// destroy()-or-GC buffer lifetime, kernels.ts:903-956). bufferPtr(handle) -> BigInt address.
struct BufBox {
    CtxBox* box;
    void* ptr;
};

void buf_release(BufBox* b)
{
    if (b->ptr) {
        brik_free(b->box->ctx, b->ptr);   // best effort: a finalizer has no caller to report to
        b->ptr = nullptr;
        --b->box->live_buffers;
    }
}

void buf_finalize(napi_env, void* data, void*)
{
    BufBox* b = static_cast<BufBox*>(data);
    buf_release(b);
    box_release(b->box);
    delete b;
}

bool get_buf(napi_env env, napi_value v, BufBox** out)
{
    void* p = nullptr;
    if (napi_get_value_external(env, v, &p) != napi_ok || !p) {
        napi_throw_type_error(env, "BRIK_EINVAL", "expected a device buffer handle");
        return false;
    }
    *out = static_cast<BufBox*>(p);
    return true;
}

napi_value AllocBuffer(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 2)) return nullptr;
    CtxBox* box;
    size_t bytes;
    if (!get_box(env, a.v[0], &box) || !get_size(env, a.v[1], &bytes)) return nullptr;
    void* p = nullptr;
    if (check(env, box->ctx, brik_alloc(box->ctx, bytes, &p))) return nullptr;
    BufBox* b = new BufBox{box, p};
    ++box->refs;
    ++box->live_buffers;
    napi_value ext;
    if (napi_create_external(env, b, buf_finalize, nullptr, &ext) != napi_ok) {
        buf_finalize(env, b, nullptr);
        napi_throw_error(env, "BRIK_NAPI", "napi_create_external failed");
        return nullptr;
    }
    return ext;
}

napi_value BufferPtr(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    BufBox* b;
    if (!get_buf(env, a.v[0], &b)) return nullptr;
    return make_ptr(env, b->ptr);
}

napi_value FreeBuffer(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    BufBox* b;
    if (!get_buf(env, a.v[0], &b)) return nullptr;
    buf_release(b);
    return undefined(env);
}

napi_value LiveBuffers(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    CtxBox* box;
    if (!get_box(env, a.v[0], &box)) return nullptr;
    napi_value r;
    NAPI_CALL(env, napi_create_int64(env, box->live_buffers, &r));
    return r;
}

// ---- asynchronous readback ------------------------------------------------------------------------
// readbackAsync(ctx, src, bytes) -> Promise<ArrayBuffer>: a fence is recorded on the context stream now
// (after everything enqueued so far, in call order), and a libuv worker waits for it and copies the
// bytes into a new ArrayBuffer; the promise resolves on the JS thread (rejects with the error code
// and message on failure), as the reference's mapAsync readback does.
struct ReadbackWork {
    napi_async_work work = nullptr;
    napi_deferred deferred = nullptr;
    napi_ref buffer = nullptr;
    void* data = nullptr;
    const void* src = nullptr;
    size_t bytes = 0;
    brik_fence* fence = nullptr;
    CtxBox* box = nullptr;   // held until completion: the context (and the memory read) outlives the copy
    int rc = BRIK_OK;
    std::string msg;
};

void readback_execute(napi_env, void* data)
{
    ReadbackWork* w = static_cast<ReadbackWork*>(data);
    w->rc = brik_fence_d2h(w->fence, w->data, w->src, w->bytes);
    if (w->rc != BRIK_OK) w->msg = std::string(code_name(w->rc)) + ": " + brik_fence_error(w->fence);
}

void readback_complete(napi_env env, napi_status status, void* data)
{
    ReadbackWork* w = static_cast<ReadbackWork*>(data);
    napi_value buf = nullptr;
    napi_get_reference_value(env, w->buffer, &buf);
    if (status == napi_ok && w->rc == BRIK_OK && buf) {
        napi_resolve_deferred(env, w->deferred, buf);
    } else {
        const std::string code = w->rc != BRIK_OK ? code_name(w->rc) : "BRIK_NAPI";
        const std::string msg = w->rc != BRIK_OK ? w->msg : "BRIK_NAPI: readback was cancelled";
        napi_value c, m, err;
        napi_create_string_utf8(env, code.c_str(), NAPI_AUTO_LENGTH, &c);
        napi_create_string_utf8(env, msg.c_str(), NAPI_AUTO_LENGTH, &m);
        napi_create_error(env, c, m, &err);
        napi_reject_deferred(env, w->deferred, err);
    }
    napi_delete_reference(env, w->buffer);
    napi_delete_async_work(env, w->work);
    brik_fence_destroy(w->fence);
    box_release(w->box);
    delete w;
}

napi_value ReadbackAsync(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 3)) return nullptr;
    CtxBox* box;
    void* src;
    size_t bytes;
    if (!get_box(env, a.v[0], &box) || !get_ptr(env, a.v[1], &src) || !get_size(env, a.v[2], &bytes)) return nullptr;
    brik_ctx* ctx = box->ctx;
    ReadbackWork* w = new ReadbackWork();
    w->src = src;
    w->bytes = bytes;
    if (check(env, ctx, brik_fence_record(ctx, &w->fence))) {
        delete w;
        return nullptr;
    }
    napi_value ab, promise, name;
    if (napi_create_arraybuffer(env, bytes, &w->data, &ab) != napi_ok ||
        napi_create_reference(env, ab, 1, &w->buffer) != napi_ok ||
        napi_create_promise(env, &w->deferred, &promise) != napi_ok ||
        napi_create_string_utf8(env, "brik.readback", NAPI_AUTO_LENGTH, &name) != napi_ok ||
        napi_create_async_work(env, nullptr, name, readback_execute, readback_complete, w, &w->work) != napi_ok ||
        napi_queue_async_work(env, w->work) != napi_ok) {
        // nothing was queued: undo what was made (a created promise is left pending and unreachable)
        if (w->work) napi_delete_async_work(env, w->work);
        if (w->buffer) napi_delete_reference(env, w->buffer);
        brik_fence_destroy(w->fence);
        delete w;
        napi_throw_error(env, "BRIK_NAPI", "readbackAsync: N-API setup failed");
        return nullptr;
    }
    w->box = box;
    ++box->refs;
    return promise;
}

// selfValidate(ctx) -> null when every check passes, else the name of the first failing check
napi_value SelfValidate(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    brik_ctx* ctx;
    if (!get_ctx(env, a.v[0], &ctx)) return nullptr;
    char stage[64];
    const int rc = brik_self_validate(ctx, stage, sizeof stage);
    if (rc == BRIK_EVALID) {
        napi_value r;
        NAPI_CALL(env, napi_create_string_utf8(env, stage, NAPI_AUTO_LENGTH, &r));
        return r;
    }
    if (check(env, ctx, rc)) return nullptr;
    napi_value n;
    NAPI_CALL(env, napi_get_null(env, &n));
    return n;
}

napi_value Alloc(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 2)) return nullptr;
    brik_ctx* ctx;
    if (!get_ctx(env, a.v[0], &ctx)) return nullptr;
    int64_t bytes = 0;
    NAPI_CALL(env, napi_get_value_int64(env, a.v[1], &bytes));
    if (bytes < 0) { napi_throw_range_error(env, "BRIK_EINVAL", "negative size"); return nullptr; }
    void* p = nullptr;
    if (check(env, ctx, brik_alloc(ctx, (size_t)bytes, &p))) return nullptr;
    return make_ptr(env, p);
}

napi_value Free(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 2)) return nullptr;
    brik_ctx* ctx;
    void* p;
    if (!get_ctx(env, a.v[0], &ctx) || !get_ptr(env, a.v[1], &p)) return nullptr;
    if (check(env, ctx, brik_free(ctx, p))) return nullptr;
    return undefined(env);
}

// h2d(ctx, dstPtr, src): copy the bytes of a TypedArray / ArrayBuffer / DataView to the device
napi_value H2D(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 3)) return nullptr;
    brik_ctx* ctx;
    void* dst;
    void* src;
    size_t len;
    if (!get_ctx(env, a.v[0], &ctx) || !get_ptr(env, a.v[1], &dst) || !get_bytes(env, a.v[2], &src, &len)) return nullptr;
    if (check(env, ctx, brik_h2d(ctx, dst, src, len))) return nullptr;
    return undefined(env);
}

// h2dAsync(ctx, dstPtr, src): the bytes are staged at once (src may be reused on return) and the copy is
// enqueued without waiting for earlier work (brik_h2d_async; the reference's queue.writeBuffer)
napi_value H2DAsync(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 3)) return nullptr;
    brik_ctx* ctx;
    void* dst;
    void* src;
    size_t len;
    if (!get_ctx(env, a.v[0], &ctx) || !get_ptr(env, a.v[1], &dst) || !get_bytes(env, a.v[2], &src, &len)) return nullptr;
    if (check(env, ctx, brik_h2d_async(ctx, dst, src, len))) return nullptr;
    return undefined(env);
}

// d2h(ctx, srcPtr, bytes) -> ArrayBuffer
napi_value D2H(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 3)) return nullptr;
    brik_ctx* ctx;
    void* src;
    int64_t bytes = 0;
    if (!get_ctx(env, a.v[0], &ctx) || !get_ptr(env, a.v[1], &src)) return nullptr;
    NAPI_CALL(env, napi_get_value_int64(env, a.v[2], &bytes));
    void* data = nullptr;
    napi_value ab;
    NAPI_CALL(env, napi_create_arraybuffer(env, (size_t)bytes, &data, &ab));
    if (check(env, ctx, brik_d2h(ctx, data, src, (size_t)bytes))) return nullptr;
    return ab;
}

napi_value Sync(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    brik_ctx* ctx;
    if (!get_ctx(env, a.v[0], &ctx)) return nullptr;
    if (check(env, ctx, brik_sync(ctx))) return nullptr;
    return undefined(env);
}

napi_value SetOption(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 3)) return nullptr;
    brik_ctx* ctx;
    int32_t k, v;
    if (!get_ctx(env, a.v[0], &ctx) || !get_i32(env, a.v[1], &k) || !get_i32(env, a.v[2], &v)) return nullptr;
    if (check(env, ctx, brik_set_option(ctx, k, v))) return nullptr;
    return undefined(env);
}

napi_value TimerBegin(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    brik_ctx* ctx;
    if (!get_ctx(env, a.v[0], &ctx)) return nullptr;
    if (check(env, ctx, brik_timer_begin(ctx))) return nullptr;
    return undefined(env);
}

napi_value TimerEnd(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    brik_ctx* ctx;
    if (!get_ctx(env, a.v[0], &ctx)) return nullptr;
    float ms = 0;
    if (check(env, ctx, brik_timer_end(ctx, &ms))) return nullptr;
    napi_value r;
    NAPI_CALL(env, napi_create_double(env, ms, &r));
    return r;
}

// ---- compute --------------------------------------------------------------------------------

// Parse (ctx, p0 .. p{np-1}, i0 .. i{ni-1}).
bool parse(napi_env env, napi_callback_info info, brik_ctx** ctx, void** p, int np, int32_t* iv, int ni)
{
    Args a;
    if (!get_args(env, info, a, (size_t)(1 + np + ni))) return false;
    if (!get_ctx(env, a.v[0], ctx)) return false;
    for (int i = 0; i < np; ++i)
        if (!get_ptr(env, a.v[1 + i], &p[i])) return false;
    for (int i = 0; i < ni; ++i)
        if (!get_i32(env, a.v[1 + np + i], &iv[i])) return false;
    return true;
}

napi_value MatmulQ8(napi_env env, napi_callback_info info)   // (ctx, x, codes, sc, y, M, K, N)
{
    brik_ctx* c; void* p[4]; int32_t i[3];
    if (!parse(env, info, &c, p, 4, i, 3)) return nullptr;
    if (check(env, c, brik_matmul_t_q8(c, (const float*)p[0], (const int8_t*)p[1], (const uint16_t*)p[2], (float*)p[3],
                                       i[0], i[1], i[2]))) return nullptr;
    return undefined(env);
}

napi_value MatmulQ4(napi_env env, napi_callback_info info)   // (ctx, x, nib, sc, mn, y, M, K, N)
{
    brik_ctx* c; void* p[5]; int32_t i[3];
    if (!parse(env, info, &c, p, 5, i, 3)) return nullptr;
    if (check(env, c, brik_matmul_t_q4(c, (const float*)p[0], (const uint8_t*)p[1], (const uint16_t*)p[2],
                                       (const uint16_t*)p[3], (float*)p[4], i[0], i[1], i[2]))) return nullptr;
    return undefined(env);
}

napi_value MatmulQ3(napi_env env, napi_callback_info info)   // (ctx, x, lo, hi, sc, mn, y, M, K, N)
{
    brik_ctx* c; void* p[6]; int32_t i[3];
    if (!parse(env, info, &c, p, 6, i, 3)) return nullptr;
    if (check(env, c, brik_matmul_t_q3(c, (const float*)p[0], (const uint32_t*)p[1], (const uint32_t*)p[2],
                                       (const uint16_t*)p[3], (const uint16_t*)p[4], (float*)p[5], i[0], i[1], i[2])))
        return nullptr;
    return undefined(env);
}

napi_value MoeMatmulQ4(napi_env env, napi_callback_info info)   // (ctx, x, rowOff, nib, sc, mn, y, E, R, K, N)
{
    brik_ctx* c; void* p[6]; int32_t i[4];
    if (!parse(env, info, &c, p, 6, i, 4)) return nullptr;
    if (check(env, c, brik_moe_matmul_t_q4(c, (const float*)p[0], (const int32_t*)p[1], (const uint8_t*)p[2],
                                           (const uint16_t*)p[3], (const uint16_t*)p[4], (float*)p[5], i[0], i[1],
                                           i[2], i[3]))) return nullptr;
    return undefined(env);
}

napi_value MoeMatmulQ4x2(napi_env env, napi_callback_info info)
// (ctx, x, rowOff, nibA, scA, mnA, yA, nibB, scB, mnB, yB, E, R, K, N)
{
    brik_ctx* c; void* p[10]; int32_t i[4];
    if (!parse(env, info, &c, p, 10, i, 4)) return nullptr;
    if (check(env, c, brik_moe_matmul_t_q4_x2(c, (const float*)p[0], (const int32_t*)p[1], (const uint8_t*)p[2],
                                              (const uint16_t*)p[3], (const uint16_t*)p[4], (float*)p[5],
                                              (const uint8_t*)p[6], (const uint16_t*)p[7], (const uint16_t*)p[8],
                                              (float*)p[9], i[0], i[1], i[2], i[3]))) return nullptr;
    return undefined(env);
}

napi_value DequantQ8(napi_env env, napi_callback_info info)   // (ctx, codes, sc, out, n)
{
    brik_ctx* c; void* p[3]; int32_t i[1];
    if (!parse(env, info, &c, p, 3, i, 1)) return nullptr;
    if (check(env, c, brik_dequant_q8_f32(c, (const int8_t*)p[0], (const uint16_t*)p[1], (float*)p[2], (size_t)i[0])))
        return nullptr;
    return undefined(env);
}

napi_value DequantQ4(napi_env env, napi_callback_info info)   // (ctx, nib, sc, mn, out, n)
{
    brik_ctx* c; void* p[4]; int32_t i[1];
    if (!parse(env, info, &c, p, 4, i, 1)) return nullptr;
    if (check(env, c, brik_dequant_q4_f32(c, (const uint8_t*)p[0], (const uint16_t*)p[1], (const uint16_t*)p[2],
                                          (float*)p[3], (size_t)i[0]))) return nullptr;
    return undefined(env);
}

napi_value DequantQ3(napi_env env, napi_callback_info info)   // (ctx, lo, hi, sc, mn, out, n)
{
    brik_ctx* c; void* p[5]; int32_t i[1];
    if (!parse(env, info, &c, p, 5, i, 1)) return nullptr;
    if (check(env, c, brik_dequant_q3_f32(c, (const uint32_t*)p[0], (const uint32_t*)p[1], (const uint16_t*)p[2],
                                          (const uint16_t*)p[3], (float*)p[4], (size_t)i[0]))) return nullptr;
    return undefined(env);
}

// (ctx, fmt, src, p0, p1, sc, mn, n): fmt 8 -> codes = p0; 4 -> nibbles = p0; 3 -> lo = p0, hi = p1
napi_value Quantize(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 8)) return nullptr;
    brik_ctx* c; int32_t fmt; void* p[5]; size_t n;
    if (!get_ctx(env, a.v[0], &c) || !get_i32(env, a.v[1], &fmt)) return nullptr;
    for (int k = 0; k < 5; ++k)
        if (!get_ptr(env, a.v[2 + k], &p[k])) return nullptr;
    if (!get_size(env, a.v[7], &n)) return nullptr;
    const float* src = (const float*)p[0];
    int rc;
    if (fmt == BRIK_FMT_Q8) rc = brik_quantize_q8(c, src, (int8_t*)p[1], (uint16_t*)p[3], n);
    else if (fmt == BRIK_FMT_Q4) rc = brik_quantize_q4(c, src, (uint8_t*)p[1], (uint16_t*)p[3], (uint16_t*)p[4], n);
    else if (fmt == BRIK_FMT_Q3)
        rc = brik_quantize_q3(c, src, (uint32_t*)p[1], (uint32_t*)p[2], (uint16_t*)p[3], (uint16_t*)p[4], n);
    else {
        napi_throw_error(env, "BRIK_EINVAL", "BRIK_EINVAL: quantize: unknown format");
        return nullptr;
    }
    if (check(env, c, rc)) return nullptr;
    return undefined(env);
}

// (ctx, fmt, inp, p0, sc, mn, bias, out, Cin, H, W, Cout, kh, kw, stride, pad); fmt 8: codes = p0, 4: nibbles
napi_value Conv2d(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 16)) return nullptr;
    brik_ctx* c; int32_t fmt; void* p[6]; int32_t i[8];
    if (!get_ctx(env, a.v[0], &c) || !get_i32(env, a.v[1], &fmt)) return nullptr;
    for (int k = 0; k < 6; ++k)
        if (!get_ptr(env, a.v[2 + k], &p[k])) return nullptr;
    for (int k = 0; k < 8; ++k)
        if (!get_i32(env, a.v[8 + k], &i[k])) return nullptr;
    int rc;
    if (fmt == BRIK_FMT_Q8)
        rc = brik_conv2d_q8(c, (const float*)p[0], (const int8_t*)p[1], (const uint16_t*)p[2], (const float*)p[4],
                            (float*)p[5], i[0], i[1], i[2], i[3], i[4], i[5], i[6], i[7]);
    else if (fmt == BRIK_FMT_Q4)
        rc = brik_conv2d_q4(c, (const float*)p[0], (const uint8_t*)p[1], (const uint16_t*)p[2], (const uint16_t*)p[3],
                            (const float*)p[4], (float*)p[5], i[0], i[1], i[2], i[3], i[4], i[5], i[6], i[7]);
    else {
        napi_throw_error(env, "BRIK_EINVAL", "BRIK_EINVAL: conv2d: the weight must be q8 or q4");
        return nullptr;
    }
    if (check(env, c, rc)) return nullptr;
    return undefined(env);
}

napi_value MatmulF16W(napi_env env, napi_callback_info info)   // (ctx, x, w, y, M, K, N)
{
    brik_ctx* c; void* p[3]; int32_t i[3];
    if (!parse(env, info, &c, p, 3, i, 3)) return nullptr;
    if (check(env, c, brik_matmul_t_f16w(c, (const float*)p[0], (const uint16_t*)p[1], (float*)p[2], i[0], i[1], i[2])))
        return nullptr;
    return undefined(env);
}

napi_value F16ToF32(napi_env env, napi_callback_info info)   // (ctx, src, out, n)
{
    Args a;
    if (!get_args(env, info, a, 4)) return nullptr;
    brik_ctx* c; void* src; void* out; size_t n;
    if (!get_ctx(env, a.v[0], &c) || !get_ptr(env, a.v[1], &src) || !get_ptr(env, a.v[2], &out) ||
        !get_size(env, a.v[3], &n)) return nullptr;
    if (check(env, c, brik_f16_to_f32(c, (const uint16_t*)src, (float*)out, n))) return nullptr;
    return undefined(env);
}

// ---- sampling pre-work -------------------------------------------------------------------------

// logitsTopK(ctx, logits, recent, ids, vals, n, nRecent, k, penalty, softcap)
napi_value LogitsTopK(napi_env env, napi_callback_info info)
{
    brik_ctx* c; void* p[4]; int32_t i[3];
    if (!parse(env, info, &c, p, 4, i, 3)) return nullptr;
    Args a;
    float pen, cap;
    if (!get_args(env, info, a, 10) || !get_f32(env, a.v[8], &pen) || !get_f32(env, a.v[9], &cap)) return nullptr;
    if (check(env, c, brik_logits_topk(c, (float*)p[0], i[0], (const int32_t*)p[1], i[1], pen, cap, i[2],
                                       (int32_t*)p[2], (float*)p[3]))) return nullptr;
    return undefined(env);
}

// lmHeadTopK(ctx, fmt, x, p0, p1, sc, mn, recent, ids, vals, K, vocab, nRecent, k, penalty, softcap)
napi_value LmHeadTopK(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 16)) return nullptr;
    brik_ctx* c;
    int32_t fmt, iv[4];
    void* p[8];
    float pen, cap;
    if (!get_ctx(env, a.v[0], &c) || !get_i32(env, a.v[1], &fmt)) return nullptr;
    for (int k = 0; k < 8; ++k)
        if (!get_ptr(env, a.v[2 + k], &p[k])) return nullptr;
    for (int k = 0; k < 4; ++k)
        if (!get_i32(env, a.v[10 + k], &iv[k])) return nullptr;
    if (!get_f32(env, a.v[14], &pen) || !get_f32(env, a.v[15], &cap)) return nullptr;
    const float* x = (const float*)p[0];
    const int32_t* rec = (const int32_t*)p[5];
    int32_t* ids = (int32_t*)p[6];
    float* vals = (float*)p[7];
    int rc;
    if (fmt == BRIK_FMT_Q8)
        rc = brik_lm_head_topk_q8(c, x, (const int8_t*)p[1], (const uint16_t*)p[3], iv[0], iv[1], rec, iv[2], pen, cap,
                                  iv[3], ids, vals);
    else if (fmt == BRIK_FMT_Q4)
        rc = brik_lm_head_topk_q4(c, x, (const uint8_t*)p[1], (const uint16_t*)p[3], (const uint16_t*)p[4], iv[0], iv[1],
                                  rec, iv[2], pen, cap, iv[3], ids, vals);
    else
        rc = brik_lm_head_topk_q3(c, x, (const uint32_t*)p[1], (const uint32_t*)p[2], (const uint16_t*)p[3],
                                  (const uint16_t*)p[4], iv[0], iv[1], rec, iv[2], pen, cap, iv[3], ids, vals);
    if (check(env, c, rc)) return nullptr;
    return undefined(env);
}

// ---- grouped GEMV plans ----------------------------------------------------------------------

struct PlanBox {
    CtxBox* box;
    brik_gemv_plan* plan;
};

void plan_finalize(napi_env, void* data, void*)
{
    PlanBox* b = static_cast<PlanBox*>(data);
    if (b->plan) brik_gemv_plan_destroy(b->box->ctx, b->plan);
    box_release(b->box);
    delete b;
}

// One job object {x, p0, p1, scales, mins, y, K, N[, gate, normW, res, eps, flags]} (the optional fields
// are those of brik_gemv_job_ex; a job without them has no fusion). False with a pending exception.
bool get_job(napi_env env, napi_value o, brik_gemv_job_ex* out)
{
    static const char* const names[6] = {"x", "p0", "p1", "scales", "mins", "y"};
    static const char* const fnames[3] = {"gate", "normW", "res"};
    napi_value f;
    void* ptrs[6];
    for (int k = 0; k < 6; ++k) {
        NAPI_CALL_B(env, napi_get_named_property(env, o, names[k], &f));
        if (!get_ptr(env, f, &ptrs[k])) return false;
    }
    int32_t K, N;
    NAPI_CALL_B(env, napi_get_named_property(env, o, "K", &f));
    if (!get_i32(env, f, &K)) return false;
    NAPI_CALL_B(env, napi_get_named_property(env, o, "N", &f));
    if (!get_i32(env, f, &N)) return false;
    void* fp[3] = {nullptr, nullptr, nullptr};
    for (int k = 0; k < 3; ++k) {
        bool has = false;
        NAPI_CALL_B(env, napi_has_named_property(env, o, fnames[k], &has));
        if (!has) continue;
        NAPI_CALL_B(env, napi_get_named_property(env, o, fnames[k], &f));
        if (!get_ptr(env, f, &fp[k])) return false;
    }
    float eps = 1e-6f;
    int32_t flags = 0;
    bool has = false;
    NAPI_CALL_B(env, napi_has_named_property(env, o, "eps", &has));
    if (has) {
        NAPI_CALL_B(env, napi_get_named_property(env, o, "eps", &f));
        if (!get_f32(env, f, &eps)) return false;
    }
    NAPI_CALL_B(env, napi_has_named_property(env, o, "flags", &has));
    if (has) {
        NAPI_CALL_B(env, napi_get_named_property(env, o, "flags", &f));
        if (!get_i32(env, f, &flags)) return false;
    }
    *out = brik_gemv_job_ex{brik_gemv_job{(const float*)ptrs[0], ptrs[1], ptrs[2], (const uint16_t*)ptrs[3],
                                          (const uint16_t*)ptrs[4], (float*)ptrs[5], K, N},
                            (const float*)fp[0], (const float*)fp[1], (const float*)fp[2], eps, flags};
    return true;
}

// A JS handle owning `plan` (and a reference to the context), or null with a pending exception.
napi_value wrap_plan(napi_env env, CtxBox* box, brik_gemv_plan* plan)
{
    PlanBox* pb = new PlanBox{box, plan};
    ++box->refs;
    napi_value ext;
    if (napi_create_external(env, pb, plan_finalize, nullptr, &ext) != napi_ok) {
        plan_finalize(env, pb, nullptr);
        napi_throw_error(env, "BRIK_NAPI", "napi_create_external failed");
        return nullptr;
    }
    return ext;
}

// gemvPlanCreate(ctx, fmt, [job, ...]) -> plan
napi_value GemvPlanCreate(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 3)) return nullptr;
    CtxBox* box;
    int32_t fmt;
    if (!get_box(env, a.v[0], &box) || !get_i32(env, a.v[1], &fmt)) return nullptr;
    brik_ctx* ctx = box->ctx;
    uint32_t n = 0;
    NAPI_CALL(env, napi_get_array_length(env, a.v[2], &n));
    std::vector<brik_gemv_job_ex> jobs(n);
    for (uint32_t j = 0; j < n; ++j) {
        napi_value o;
        NAPI_CALL(env, napi_get_element(env, a.v[2], j, &o));
        if (!get_job(env, o, &jobs[j])) return nullptr;
    }
    brik_gemv_plan* plan = nullptr;
    if (check(env, ctx, brik_gemv_plan_create_ex(ctx, fmt, jobs.data(), (int)n, &plan))) return nullptr;
    return wrap_plan(env, box, plan);
}

// gemvPlanCreateGlu(ctx, fmt, gate, up, down) -> [gateUpPlan, downPlan] (brik_gemv_plan_create_glu)
napi_value GemvPlanCreateGlu(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 5)) return nullptr;
    CtxBox* box;
    int32_t fmt;
    if (!get_box(env, a.v[0], &box) || !get_i32(env, a.v[1], &fmt)) return nullptr;
    brik_gemv_job_ex jobs[3];
    for (int k = 0; k < 3; ++k)
        if (!get_job(env, a.v[2 + k], &jobs[k])) return nullptr;
    brik_gemv_plan *gu = nullptr, *dn = nullptr;
    if (check(env, box->ctx, brik_gemv_plan_create_glu(box->ctx, fmt, &jobs[0], &jobs[1], &jobs[2], &gu, &dn)))
        return nullptr;
    napi_value hg = wrap_plan(env, box, gu);
    if (!hg) {
        brik_gemv_plan_destroy(box->ctx, dn);
        return nullptr;
    }
    napi_value hd = wrap_plan(env, box, dn);
    if (!hd) return nullptr;
    napi_value arr;
    NAPI_CALL(env, napi_create_array_with_length(env, 2, &arr));
    NAPI_CALL(env, napi_set_element(env, arr, 0, hg));
    NAPI_CALL(env, napi_set_element(env, arr, 1, hd));
    return arr;
}

napi_value GemvPlanRun(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    void* p = nullptr;
    if (napi_get_value_external(env, a.v[0], &p) != napi_ok || !p) {
        napi_throw_type_error(env, "BRIK_EINVAL", "expected a GEMV plan");
        return nullptr;
    }
    PlanBox* b = static_cast<PlanBox*>(p);
    if (!b->plan) { napi_throw_error(env, "BRIK_EINVAL", "plan was destroyed"); return nullptr; }
    if (check(env, b->box->ctx, brik_gemv_plan_run(b->box->ctx, b->plan))) return nullptr;
    return undefined(env);
}

napi_value GemvPlanDestroy(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    void* p = nullptr;
    if (napi_get_value_external(env, a.v[0], &p) != napi_ok || !p) return nullptr;
    PlanBox* b = static_cast<PlanBox*>(p);
    if (b->plan) brik_gemv_plan_destroy(b->box->ctx, b->plan);
    b->plan = nullptr;
    return undefined(env);
}

// ---- recorded launches ---------------------------------------------------------------------------
// graphBegin(ctx); ... library calls ...; graphEnd(ctx) -> graph; graphLaunch(graph); graphDestroy(graph).
// The graph is also destroyed by its finalizer if the handle is dropped.
constexpr uint32_t kGraphMagic = 0x62726b67;   // "brkg": the handle kind, checked before use

struct GraphBox {
    uint32_t magic;
    CtxBox* box;
    brik_graph* graph;
};

void graph_finalize(napi_env, void* data, void*)
{
    GraphBox* g = static_cast<GraphBox*>(data);
    if (g->graph) brik_graph_destroy(g->box->ctx, g->graph);
    box_release(g->box);
    delete g;
}

bool get_graph(napi_env env, napi_value v, GraphBox** out)
{
    void* p = nullptr;
    if (napi_get_value_external(env, v, &p) != napi_ok || !p || static_cast<GraphBox*>(p)->magic != kGraphMagic) {
        napi_throw_type_error(env, "BRIK_EINVAL", "expected a recorded graph");
        return false;
    }
    *out = static_cast<GraphBox*>(p);
    if (!(*out)->graph) {
        napi_throw_error(env, "BRIK_EINVAL", "graph was destroyed");
        return false;
    }
    return true;
}

napi_value GraphBegin(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    brik_ctx* ctx;
    if (!get_ctx(env, a.v[0], &ctx)) return nullptr;
    if (check(env, ctx, brik_graph_begin(ctx))) return nullptr;
    return undefined(env);
}

napi_value GraphEnd(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    CtxBox* box;
    if (!get_box(env, a.v[0], &box)) return nullptr;
    brik_graph* g = nullptr;
    if (check(env, box->ctx, brik_graph_end(box->ctx, &g))) return nullptr;
    GraphBox* gb = new GraphBox{kGraphMagic, box, g};
    ++box->refs;
    napi_value ext;
    if (napi_create_external(env, gb, graph_finalize, nullptr, &ext) != napi_ok) {
        graph_finalize(env, gb, nullptr);
        napi_throw_error(env, "BRIK_NAPI", "napi_create_external failed");
        return nullptr;
    }
    return ext;
}

napi_value GraphLaunch(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    GraphBox* g;
    if (!get_graph(env, a.v[0], &g)) return nullptr;
    if (check(env, g->box->ctx, brik_graph_launch(g->box->ctx, g->graph))) return nullptr;
    return undefined(env);
}

napi_value GraphDestroy(napi_env env, napi_callback_info info)
{
    Args a;
    if (!get_args(env, info, a, 1)) return nullptr;
    void* p = nullptr;
    if (napi_get_value_external(env, a.v[0], &p) != napi_ok || !p || static_cast<GraphBox*>(p)->magic != kGraphMagic)
        return undefined(env);
    GraphBox* g = static_cast<GraphBox*>(p);
    if (g->graph) brik_graph_destroy(g->box->ctx, g->graph);
    g->graph = nullptr;
    return undefined(env);
}

napi_value Init(napi_env env, napi_value exports)
{
    const napi_property_descriptor props[] = {
        {"deviceCount", nullptr, DeviceCount, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"createContext", nullptr, CreateContext, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"alloc", nullptr, Alloc, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"free", nullptr, Free, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"h2d", nullptr, H2D, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"h2dAsync", nullptr, H2DAsync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"graphBegin", nullptr, GraphBegin, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"graphEnd", nullptr, GraphEnd, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"graphLaunch", nullptr, GraphLaunch, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"graphDestroy", nullptr, GraphDestroy, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"d2h", nullptr, D2H, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"sync", nullptr, Sync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"setOption", nullptr, SetOption, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"timerBegin", nullptr, TimerBegin, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"timerEnd", nullptr, TimerEnd, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"matmulQ8", nullptr, MatmulQ8, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"matmulQ4", nullptr, MatmulQ4, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"matmulQ3", nullptr, MatmulQ3, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"moeMatmulQ4", nullptr, MoeMatmulQ4, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"moeMatmulQ4x2", nullptr, MoeMatmulQ4x2, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"dequantQ8", nullptr, DequantQ8, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"dequantQ4", nullptr, DequantQ4, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"dequantQ3", nullptr, DequantQ3, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"quantize", nullptr, Quantize, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"f16ToF32", nullptr, F16ToF32, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"conv2d", nullptr, Conv2d, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"matmulF16W", nullptr, MatmulF16W, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"logitsTopK", nullptr, LogitsTopK, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"lmHeadTopK", nullptr, LmHeadTopK, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"gemvPlanCreate", nullptr, GemvPlanCreate, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"gemvPlanCreateGlu", nullptr, GemvPlanCreateGlu, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"gemvPlanRun", nullptr, GemvPlanRun, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"gemvPlanDestroy", nullptr, GemvPlanDestroy, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"allocBuffer", nullptr, AllocBuffer, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"bufferPtr", nullptr, BufferPtr, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"freeBuffer", nullptr, FreeBuffer, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"liveBuffers", nullptr, LiveBuffers, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"readbackAsync", nullptr, ReadbackAsync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
        {"selfValidate", nullptr, SelfValidate, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
    };
    napi_define_properties(env, exports, sizeof(props) / sizeof(props[0]), props);
    return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
