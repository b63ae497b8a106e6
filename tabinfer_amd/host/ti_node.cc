// ti_node.cc — Node.js N-API addon over libtabinfer's C ABI (include/ti.h).
//
// The reference engine's kernels are closure launchers over WebGPU buffers
// (models/qwen3.js, models/lfm25.js over engine/webgpu-engine.js). This addon gives
// the JS host the same objects over the HIP library:
//   init(device) -> ctx                        E.init (engine/webgpu-engine.js:72-145)
//   buf_alloc(ctx, bytes) -> buffer            E.createBuffer (:156-160); freed by GC or buf_free
//   buf_write / buf_read / buf_copy / sync     queue.writeBuffer / E.readF32 / E.copyBuffer
//   graph_begin / graph_end / graph_launch     E.beginBatch / E.endBatch (:357-386)
//   every kernel entry point of ti.h           under its C name without the "ti_" prefix
// Buffers and the other handles are napi_external objects. A device-pointer argument
// takes a buffer (or a view of one) or null. Errors from the library (shape
// preconditions, HIP failures) become JS exceptions carrying ti_last_error().
//
// Only the plain N-API C API is used (Node 12, N-API 8); no node-addon-api.
#include <node_api.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <map>
#include <mutex>
#include <string>
#include <unordered_set>
#include <tuple>
#include <type_traits>
#include <utility>
#include <vector>

#include "ti.h"

namespace {

// ---- handles -------------------------------------------------------------------------
enum Tag : uint32_t { TAG_CTX = 0x74696378, TAG_BUF = 0x74696262, TAG_GRAPH = 0x74696767, TAG_MODEL = 0x7469716d,
                     TAG_CPUBIN = 0x74696362, TAG_BONSAI = 0x7469626e };

// A context lives until its JS handle is finalized (or shutdown() is called) AND every
// buffer, graph and model made on it is gone: they hold counted references, so a
// finalizer never runs against a context that was already shut down.
struct CtxH {
    uint32_t tag = TAG_CTX;
    ti_ctx* c = nullptr;
    int refs = 1;          // the JS handle + one per live dependent handle
    bool closed = false;
};

void ctx_unref(CtxH* h) {
    if (--h->refs == 0) {
        if (!h->closed && h->c) ti_shutdown(h->c);
        h->tag = 0;
        delete h;
    }
}

struct ModelH {
    uint32_t tag = TAG_MODEL;
    CtxH* ctx = nullptr;
    ti_qwen3* m = nullptr;     // null once destroyed
    ti_qwen3_config cfg;       // sizes of the views it hands out
};

// A device buffer, or a view into another buffer or into a model's storage. A view holds
// a reference to its parent's JS object (so the parent's handle outlives it) and checks
// the parent is still live on every use: buf_free of the parent or qwen3_destroy of the
// model turns its views dead instead of leaving them pointing into freed memory.
struct BufH {
    uint32_t tag = TAG_BUF;
    CtxH* ctx = nullptr;
    char* ptr = nullptr;       // null once freed
    size_t bytes = 0;
    bool owned = false;        // freed with ti_buf_free when collected
    napi_ref parent = nullptr; // the parent object (buffer or model), kept alive
    BufH* pbuf = nullptr;      // the parent's handle when it is a buffer
    ModelH* pmodel = nullptr;  // ... when it is a Qwen3 model
    struct BonsaiH* pbonsai = nullptr;   // ... when it is a Bonsai model
};

bool bonsai_live(const struct BonsaiH* h);

bool buf_live(const BufH* b) {
    for (; b; b = b->pbuf)
        if (!b->ptr || (b->pmodel && !b->pmodel->m) || (b->pbonsai && !bonsai_live(b->pbonsai))) return false;
    return true;
}

struct GraphH {
    uint32_t tag = TAG_GRAPH;
    CtxH* ctx = nullptr;
    ti_graph* g = nullptr;
};

// ---- error helpers ----------------------------------------------------------------------
napi_value undefined(napi_env env) {
    napi_value u;
    napi_get_undefined(env, &u);
    return u;
}

napi_value throw_msg(napi_env env, const std::string& msg) {
    napi_throw_error(env, nullptr, msg.c_str());
    return nullptr;
}

napi_value throw_ti(napi_env env, const char* fn, int rc) {
    const char* m = ti_last_error();
    char code[32];
    std::snprintf(code, sizeof code, "%d", rc);
    std::string s = std::string(fn) + " failed (" + code + "): " + (m && *m ? m : "unknown error");
    napi_value err, msg, cv;
    napi_create_string_utf8(env, s.c_str(), NAPI_AUTO_LENGTH, &msg);
    napi_create_error(env, nullptr, msg, &err);
    napi_create_int32(env, rc, &cv);
    napi_set_named_property(env, err, "code", cv);
    napi_throw(env, err);
    return nullptr;
}

bool arg_error(napi_env env, const char* fn, size_t i, const char* want) {
    char b[256];
    std::snprintf(b, sizeof b, "%s: argument %zu must be %s", fn, i, want);
    napi_throw_type_error(env, nullptr, b);
    return false;
}

template <typename H>
H* handle_of(napi_env env, napi_value v, uint32_t tag) {
    napi_valuetype t;
    if (napi_typeof(env, v, &t) != napi_ok || t != napi_external) return nullptr;
    void* p = nullptr;
    if (napi_get_value_external(env, v, &p) != napi_ok || !p) return nullptr;
    H* h = static_cast<H*>(p);
    return h->tag == tag ? h : nullptr;
}

bool is_nullish(napi_env env, napi_value v) {
    napi_valuetype t;
    napi_typeof(env, v, &t);
    return t == napi_null || t == napi_undefined;
}

CtxH* get_ctx(napi_env env, napi_value v, const char* fn) {
    CtxH* h = handle_of<CtxH>(env, v, TAG_CTX);
    if (!h) { arg_error(env, fn, 0, "a context from init()"); return nullptr; }
    if (h->closed) { throw_msg(env, std::string(fn) + ": the context was shut down"); return nullptr; }
    return h;
}

// A Bonsai ternary decoder (ti_bonsai_*); its views (tensors, KV, logits) keep it alive
// and die with it, as the Qwen3 decoder's do.
struct BonsaiH {
    uint32_t tag = TAG_BONSAI;
    CtxH* ctx = nullptr;
    ti_bonsai* m = nullptr;
    ti_bonsai_config cfg;
};

// A .cpu.bin container (host memory only; no context).
struct CpuBinH {
    uint32_t tag = TAG_CPUBIN;
    ti_cpubin* c = nullptr;   // null once closed
};

// ---- finalizers ---------------------------------------------------------------------------
bool bonsai_live(const BonsaiH* h) { return h->m != nullptr; }

void fin_bonsai(napi_env, void* data, void*) {
    BonsaiH* h = static_cast<BonsaiH*>(data);
    if (h->m && !h->ctx->closed) ti_bonsai_destroy(h->ctx->c, h->m);
    ctx_unref(h->ctx);
    h->tag = 0;
    delete h;
}

void fin_cpubin(napi_env, void* data, void*) {
    CpuBinH* h = static_cast<CpuBinH*>(data);
    if (h->c) ti_cpubin_close(h->c);
    h->tag = 0;
    delete h;
}

void fin_ctx(napi_env, void* data, void*) {
    ctx_unref(static_cast<CtxH*>(data));
}

void fin_buf(napi_env env, void* data, void*) {
    BufH* b = static_cast<BufH*>(data);
    if (b->owned && b->ptr && !b->ctx->closed) ti_buf_free(b->ctx->c, b->ptr);
    if (b->parent) napi_delete_reference(env, b->parent);
    ctx_unref(b->ctx);
    b->tag = 0;
    delete b;
}

void fin_graph(napi_env, void* data, void*) {
    GraphH* g = static_cast<GraphH*>(data);
    if (g->g && !g->ctx->closed) ti_graph_destroy(g->g);
    ctx_unref(g->ctx);
    g->tag = 0;
    delete g;
}

void fin_model(napi_env, void* data, void*) {
    ModelH* m = static_cast<ModelH*>(data);
    if (m->m && !m->ctx->closed) ti_qwen3_destroy(m->ctx->c, m->m);
    ctx_unref(m->ctx);
    m->tag = 0;
    delete m;
}

napi_value make_buf(napi_env env, CtxH* ctx, void* ptr, size_t bytes, bool owned, napi_value parent) {
    BufH* b = new BufH;
    b->ctx = ctx;
    ctx->refs++;
    b->ptr = static_cast<char*>(ptr);
    b->bytes = bytes;
    b->owned = owned;
    if (parent) {
        napi_create_reference(env, parent, 1, &b->parent);
        b->pbuf = handle_of<BufH>(env, parent, TAG_BUF);
        b->pmodel = handle_of<ModelH>(env, parent, TAG_MODEL);
        b->pbonsai = handle_of<BonsaiH>(env, parent, TAG_BONSAI);
    }
    napi_value out;
    napi_create_external(env, b, fin_buf, nullptr, &out);
    return out;
}

// ---- argument conversion for the generic kernel wrapper ------------------------------------
bool get_i64(napi_env env, napi_value v, int64_t* out, const char* fn, size_t i) {
    double d;
    if (napi_get_value_double(env, v, &d) != napi_ok) return arg_error(env, fn, i, "a number");
    if (d != (double)(int64_t)d) return arg_error(env, fn, i, "an integer");
    *out = (int64_t)d;
    return true;
}

bool get_dptr(napi_env env, napi_value v, void** out, const char* fn, size_t i) {
    if (is_nullish(env, v)) { *out = nullptr; return true; }
    BufH* b = handle_of<BufH>(env, v, TAG_BUF);
    if (!b) return arg_error(env, fn, i, "a device buffer or null");
    if (!buf_live(b)) return arg_error(env, fn, i, "a live device buffer (this one, or the buffer or model it views, was freed)");
    *out = b->ptr;
    return true;
}

template <typename T, typename Enable = void>
struct Conv;

template <typename T>
struct Conv<T, typename std::enable_if<std::is_integral<T>::value>::type> {
    T v{};
    bool get(napi_env env, napi_value x, const char* fn, size_t i) {
        int64_t t = 0;
        if (!get_i64(env, x, &t, fn, i)) return false;
        if (t < (int64_t)std::numeric_limits<T>::min() || (std::is_signed<T>::value ? t > (int64_t)std::numeric_limits<T>::max()
                                                                                   : (uint64_t)t > (uint64_t)std::numeric_limits<T>::max()))
            return arg_error(env, fn, i, "an integer in range");
        v = (T)t;
        return true;
    }
    T value() const { return v; }
};

template <>
struct Conv<float> {
    float v = 0.0f;
    bool get(napi_env env, napi_value x, const char* fn, size_t i) {
        double d;
        if (napi_get_value_double(env, x, &d) != napi_ok) return arg_error(env, fn, i, "a number");
        v = (float)d;
        return true;
    }
    float value() const { return v; }
};

// device pointers: arithmetic element types (const or not) and void
template <typename P>
struct Conv<P*, typename std::enable_if<std::is_arithmetic<typename std::remove_const<P>::type>::value ||
                                        std::is_void<typename std::remove_const<P>::type>::value>::type> {
    P* v = nullptr;
    bool get(napi_env env, napi_value x, const char* fn, size_t i) {
        void* p = nullptr;
        if (!get_dptr(env, x, &p, fn, i)) return false;
        v = static_cast<P*>(p);
        return true;
    }
    P* value() const { return v; }
};

template <typename... A, size_t... I>
napi_value invoke(napi_env env, napi_value* argv, const char* fn, int (*f)(ti_ctx*, A...), std::index_sequence<I...>) {
    CtxH* c = get_ctx(env, argv[0], fn);
    if (!c) return nullptr;
    std::tuple<Conv<A>...> cv;
    bool ok = true;
    (void)std::initializer_list<int>{(ok = ok && std::get<I>(cv).get(env, argv[I + 1], fn, I + 1), 0)...};
    if (!ok) return nullptr;
    const int rc = f(c->c, std::get<I>(cv).value()...);
    return rc ? throw_ti(env, fn, rc) : undefined(env);
}

template <typename... A>
napi_value call_entry(napi_env env, napi_callback_info info, const char* fn, int (*f)(ti_ctx*, A...)) {
    constexpr size_t N = sizeof...(A) + 1;
    size_t argc = N;
    napi_value argv[N];
    napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr);
    if (argc != N) {
        char b[160];
        std::snprintf(b, sizeof b, "%s expects %zu arguments (ctx first), got %zu", fn, N, argc);
        return throw_msg(env, b);
    }
    return invoke(env, argv, fn, f, std::index_sequence_for<A...>{});
}

// ---- hand-written entries (host memory, handles, arrays) -----------------------------------
struct Args {
    napi_value v[12];
    size_t n = 12;
    Args(napi_env env, napi_callback_info info) { napi_get_cb_info(env, info, &n, v, nullptr, nullptr); }
};

bool want_args(napi_env env, const Args& a, size_t n, const char* fn) {
    if (a.n != n) {
        char b[128];
        std::snprintf(b, sizeof b, "%s expects %zu arguments, got %zu", fn, n, a.n);
        throw_msg(env, b);
        return false;
    }
    return true;
}

napi_value num(napi_env env, double d) {
    napi_value r;
    napi_create_double(env, d, &r);
    return r;
}

napi_value js_version(napi_env env, napi_callback_info) { return num(env, ti_version()); }

napi_value js_last_error(napi_env env, napi_callback_info) {
    napi_value r;
    napi_create_string_utf8(env, ti_last_error(), NAPI_AUTO_LENGTH, &r);
    return r;
}

napi_value js_device_count(napi_env env, napi_callback_info) {
    int n = 0;
    const int rc = ti_device_count(&n);
    return rc ? throw_ti(env, "device_count", rc) : num(env, n);
}

napi_value js_init(napi_env env, napi_callback_info info) {
    Args a(env, info);
    int64_t dev = 0;
    if (a.n >= 1 && !is_nullish(env, a.v[0]) && !get_i64(env, a.v[0], &dev, "init", 0)) return nullptr;
    ti_ctx* c = nullptr;
    const int rc = ti_init((int)dev, &c);
    if (rc) return throw_ti(env, "init", rc);
    CtxH* h = new CtxH;
    h->c = c;
    napi_value out;
    napi_create_external(env, h, fin_ctx, nullptr, &out);
    return out;
}

napi_value js_shutdown(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 1, "shutdown")) return nullptr;
    CtxH* h = handle_of<CtxH>(env, a.v[0], TAG_CTX);
    if (!h) return arg_error(env, "shutdown", 0, "a context"), nullptr;
    if (!h->closed) {
        const int rc = ti_shutdown(h->c);
        h->closed = true;
        h->c = nullptr;
        if (rc) return throw_ti(env, "shutdown", rc);
    }
    return undefined(env);
}

napi_value js_buf_alloc(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 2, "buf_alloc")) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], "buf_alloc");
    int64_t bytes;
    if (!c || !get_i64(env, a.v[1], &bytes, "buf_alloc", 1)) return nullptr;
    if (bytes <= 0) return arg_error(env, "buf_alloc", 1, "a positive byte count"), nullptr;
    void* p = nullptr;
    const int rc = ti_buf_alloc(c->c, (size_t)bytes, &p);
    if (rc) return throw_ti(env, "buf_alloc", rc);
    return make_buf(env, c, p, (size_t)bytes, true, nullptr);
}

napi_value js_buf_free(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 1, "buf_free")) return nullptr;
    BufH* b = handle_of<BufH>(env, a.v[0], TAG_BUF);
    if (!b) return arg_error(env, "buf_free", 0, "a device buffer"), nullptr;
    if (b->owned && b->ptr && !b->ctx->closed) {
        const int rc = ti_buf_free(b->ctx->c, b->ptr);
        if (rc) return throw_ti(env, "buf_free", rc);
    }
    b->ptr = nullptr;
    return undefined(env);
}

// buf_view(buffer, byteOffset[, bytes]): a non-owning view that keeps `buffer` alive
napi_value js_buf_view(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (a.n < 2 || a.n > 3) return throw_msg(env, "buf_view expects (buffer, byteOffset[, bytes])");
    BufH* b = handle_of<BufH>(env, a.v[0], TAG_BUF);
    if (!b || !buf_live(b)) return arg_error(env, "buf_view", 0, "a live device buffer"), nullptr;
    int64_t off, len = -1;
    if (!get_i64(env, a.v[1], &off, "buf_view", 1)) return nullptr;
    if (a.n == 3 && !get_i64(env, a.v[2], &len, "buf_view", 2)) return nullptr;
    if (off < 0 || (size_t)off > b->bytes) return throw_msg(env, "buf_view: offset outside the buffer");
    size_t rest = b->bytes - (size_t)off;
    if (len >= 0) {
        if ((size_t)len > rest) return throw_msg(env, "buf_view: view extends past the buffer");
        rest = (size_t)len;
    }
    return make_buf(env, b->ctx, b->ptr + off, rest, false, a.v[0]);
}

napi_value js_buf_bytes(napi_env env, napi_callback_info info) {
    Args a(env, info);
    BufH* b = a.n == 1 ? handle_of<BufH>(env, a.v[0], TAG_BUF) : nullptr;
    if (!b) return arg_error(env, "buf_bytes", 0, "a device buffer"), nullptr;
    return num(env, (double)b->bytes);
}

// host bytes of a TypedArray / DataView / ArrayBuffer / Buffer
bool host_bytes(napi_env env, napi_value v, void** data, size_t* len, const char* fn, size_t i) {
    bool is;
    napi_is_typedarray(env, v, &is);
    if (is) {
        napi_typedarray_type t;
        size_t n, off;
        napi_value ab;
        napi_get_typedarray_info(env, v, &t, &n, data, &ab, &off);
        size_t es = 1;
        switch (t) {
            case napi_int16_array: case napi_uint16_array: es = 2; break;
            case napi_int32_array: case napi_uint32_array: case napi_float32_array: es = 4; break;
            case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: es = 8; break;
            default: es = 1;
        }
        *len = n * es;
        return true;
    }
    napi_is_dataview(env, v, &is);
    if (is) {
        napi_value ab;
        size_t off;
        napi_get_dataview_info(env, v, len, data, &ab, &off);
        return true;
    }
    napi_is_arraybuffer(env, v, &is);
    if (is) {
        napi_get_arraybuffer_info(env, v, data, len);
        return true;
    }
    return arg_error(env, fn, i, "a TypedArray, DataView or ArrayBuffer");
}

// buf_write(ctx, buffer, byteOffset, typedArray)
napi_value js_buf_write(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 4, "buf_write")) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], "buf_write");
    void* dst;
    int64_t off;
    void* src;
    size_t len;
    if (!c || !get_dptr(env, a.v[1], &dst, "buf_write", 1) || !get_i64(env, a.v[2], &off, "buf_write", 2) ||
        !host_bytes(env, a.v[3], &src, &len, "buf_write", 3))
        return nullptr;
    BufH* b = handle_of<BufH>(env, a.v[1], TAG_BUF);
    if (!dst || off < 0 || (size_t)off > b->bytes || len > b->bytes - (size_t)off) return throw_msg(env, "buf_write: outside the buffer");
    const int rc = ti_buf_write(c->c, dst, (size_t)off, src, len);
    return rc ? throw_ti(env, "buf_write", rc) : undefined(env);
}

// buf_read(ctx, buffer, byteOffset, bytes) -> ArrayBuffer (waits for the stream)
napi_value js_buf_read(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 4, "buf_read")) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], "buf_read");
    void* src;
    int64_t off, len;
    if (!c || !get_dptr(env, a.v[1], &src, "buf_read", 1) || !get_i64(env, a.v[2], &off, "buf_read", 2) ||
        !get_i64(env, a.v[3], &len, "buf_read", 3))
        return nullptr;
    BufH* b = handle_of<BufH>(env, a.v[1], TAG_BUF);
    if (!src || off < 0 || len < 0 || (size_t)off > b->bytes || (size_t)len > b->bytes - (size_t)off)
        return throw_msg(env, "buf_read: outside the buffer");
    void* data;
    napi_value ab;
    napi_create_arraybuffer(env, (size_t)len, &data, &ab);
    const int rc = ti_buf_read(c->c, src, (size_t)off, data, (size_t)len);
    return rc ? throw_ti(env, "buf_read", rc) : ab;
}

// sync_async(ctx) -> Promise: waits on a worker thread so the event loop keeps running.
// The caller issues nothing else on the context until the promise settles.
struct SyncWork {
    napi_async_work work = nullptr;
    napi_deferred deferred = nullptr;
    CtxH* ctx = nullptr;
    int slot = -1;         // >= 0: wait for that event slot only (event_wait_async)
    int rc = 0;
    std::string err;
};

void sync_execute(napi_env, void* data) {
    SyncWork* w = static_cast<SyncWork*>(data);
    w->rc = w->slot >= 0 ? ti_event_wait(w->ctx->c, w->slot) : ti_sync(w->ctx->c);
    if (w->rc) w->err = ti_last_error();
}

void sync_complete(napi_env env, napi_status, void* data) {
    SyncWork* w = static_cast<SyncWork*>(data);
    if (w->rc) {
        napi_value msg, err;
        napi_create_string_utf8(env, ("sync failed: " + w->err).c_str(), NAPI_AUTO_LENGTH, &msg);
        napi_create_error(env, nullptr, msg, &err);
        napi_reject_deferred(env, w->deferred, err);
    } else {
        napi_resolve_deferred(env, w->deferred, undefined(env));
    }
    napi_delete_async_work(env, w->work);
    ctx_unref(w->ctx);
    delete w;
}

napi_value js_sync_async(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 1, "sync_async")) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], "sync_async");
    if (!c) return nullptr;
    SyncWork* w = new SyncWork;
    w->ctx = c;
    c->refs++;
    napi_value promise, name;
    napi_create_promise(env, &w->deferred, &promise);
    napi_create_string_utf8(env, "ti_sync", NAPI_AUTO_LENGTH, &name);
    napi_create_async_work(env, nullptr, name, sync_execute, sync_complete, w, &w->work);
    napi_queue_async_work(env, w->work);
    return promise;
}

// event_wait_async(ctx, slot) -> Promise: resolves once the last record of the slot has
// completed; the context's owner keeps issuing work meanwhile (the slot is not re-recorded
// until the promise settles)
napi_value js_event_wait_async(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 2, "event_wait_async")) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], "event_wait_async");
    int64_t slot;
    if (!c || !get_i64(env, a.v[1], &slot, "event_wait_async", 1)) return nullptr;
    if (slot < 0 || slot >= 64) return throw_msg(env, "event_wait_async: slot out of [0, 64)");
    SyncWork* w = new SyncWork;
    w->ctx = c;
    w->slot = (int)slot;
    c->refs++;
    napi_value promise, name;
    napi_create_promise(env, &w->deferred, &promise);
    napi_create_string_utf8(env, "ti_event_wait", NAPI_AUTO_LENGTH, &name);
    napi_create_async_work(env, nullptr, name, sync_execute, sync_complete, w, &w->work);
    napi_queue_async_work(env, w->work);
    return promise;
}

// host_alloc(bytes) -> ArrayBuffer over page-locked memory, freed by host_free(ab) (which
// detaches it) or with the ArrayBuffer; the live set (start -> bytes) keeps the two from
// freeing twice and lets the asynchronous reads check that their destination lies inside
// one live allocation (memory the JS heap owns could move or be collected mid-copy).
// ti_host_free waits for the device first, so no queued copy writes freed memory.
std::mutex g_pin_mu;
std::map<const char*, size_t> g_pinned;

bool pin_release(void* p) {
    std::lock_guard<std::mutex> lk(g_pin_mu);
    return g_pinned.erase(static_cast<const char*>(p)) > 0;
}

// [p, p + len) inside one live host_alloc allocation
bool pinned_range(const void* p, size_t len) {
    const char* q = static_cast<const char*>(p);
    std::lock_guard<std::mutex> lk(g_pin_mu);
    auto it = g_pinned.upper_bound(q);
    if (it == g_pinned.begin()) return false;
    --it;
    const size_t off = (size_t)(q - it->first);
    return off <= it->second && len <= it->second - off;
}

void fin_host(napi_env, void* data, void*) {
    if (pin_release(data)) ti_host_free(data);
}

napi_value js_host_alloc(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 1, "host_alloc")) return nullptr;
    int64_t bytes;
    if (!get_i64(env, a.v[0], &bytes, "host_alloc", 0)) return nullptr;
    if (bytes <= 0 || bytes > (int64_t(1) << 32)) return throw_msg(env, "host_alloc: bytes out of (0, 4 GiB]");
    void* p = nullptr;
    const int rc = ti_host_alloc((size_t)bytes, &p);
    if (rc) return throw_ti(env, "host_alloc", rc);
    {
        std::lock_guard<std::mutex> lk(g_pin_mu);
        g_pinned[static_cast<const char*>(p)] = (size_t)bytes;
    }
    napi_value ab;
    if (napi_create_external_arraybuffer(env, p, (size_t)bytes, fin_host, nullptr, &ab) != napi_ok) {
        if (pin_release(p)) ti_host_free(p);
        return throw_msg(env, "host_alloc: cannot wrap the memory");
    }
    return ab;
}

// host_free(ab): frees a host_alloc ArrayBuffer now (it is detached: length 0 afterwards)
napi_value js_host_free(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 1, "host_free")) return nullptr;
    bool is_ab = false;
    napi_is_arraybuffer(env, a.v[0], &is_ab);
    if (!is_ab) return arg_error(env, "host_free", 0, "an ArrayBuffer from host_alloc"), nullptr;
    void* data = nullptr;
    size_t len = 0;
    napi_get_arraybuffer_info(env, a.v[0], &data, &len);
    if (!data || !pin_release(data)) return throw_msg(env, "host_free: not a live host_alloc buffer");
    napi_detach_arraybuffer(env, a.v[0]);
    const int rc = ti_host_free(data);
    return rc ? throw_ti(env, "host_free", rc) : undefined(env);
}

// bytes of a TypedArray / ArrayBuffer argument (host memory)
bool host_bytes(napi_env env, napi_value v, void** data, size_t* len) {
    bool is = false;
    napi_is_typedarray(env, v, &is);
    if (is) {
        napi_typedarray_type tt;
        size_t n, off;
        napi_value ab;
        napi_get_typedarray_info(env, v, &tt, &n, data, &ab, &off);
        size_t el = 1;
        switch (tt) {
            case napi_int16_array: case napi_uint16_array: el = 2; break;
            case napi_int32_array: case napi_uint32_array: case napi_float32_array: el = 4; break;
            case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: el = 8; break;
            default: el = 1;
        }
        *len = n * el;
        return true;
    }
    napi_is_arraybuffer(env, v, &is);
    if (is) {
        napi_get_arraybuffer_info(env, v, data, len);
        return true;
    }
    return false;
}

// buf_read_async(ctx, buf, off, dst, bytes): queued D2H into dst (host_alloc memory), no wait
napi_value js_buf_read_async(napi_env env, napi_callback_info info) {
    const char* fn = "buf_read_async";
    Args a(env, info);
    if (!want_args(env, a, 5, fn)) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], fn);
    void* src;
    int64_t off, len;
    if (!c || !get_dptr(env, a.v[1], &src, fn, 1) || !get_i64(env, a.v[2], &off, fn, 2) ||
        !get_i64(env, a.v[4], &len, fn, 4))
        return nullptr;
    BufH* b = handle_of<BufH>(env, a.v[1], TAG_BUF);
    if (!src || off < 0 || len < 0 || (size_t)off > b->bytes || (size_t)len > b->bytes - (size_t)off)
        return throw_msg(env, "buf_read_async: outside the buffer");
    void* dst;
    size_t cap;
    if (!host_bytes(env, a.v[3], &dst, &cap)) return arg_error(env, fn, 3, "a TypedArray or ArrayBuffer"), nullptr;
    if ((size_t)len > cap) return throw_msg(env, "buf_read_async: the destination is too small");
    if (len && !pinned_range(dst, (size_t)len))
        return throw_msg(env, "buf_read_async: the destination is not live host_alloc memory");
    const int rc = ti_buf_read_async(c->c, src, (size_t)off, dst, (size_t)len);
    return rc ? throw_ti(env, fn, rc) : undefined(env);
}

napi_value js_graph_end(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 1, "graph_end")) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], "graph_end");
    if (!c) return nullptr;
    ti_graph* g = nullptr;
    const int rc = ti_graph_end(c->c, &g);
    if (rc) return throw_ti(env, "graph_end", rc);
    GraphH* h = new GraphH;
    h->ctx = c;
    c->refs++;
    h->g = g;
    napi_value out;
    napi_create_external(env, h, fin_graph, nullptr, &out);
    return out;
}

napi_value js_graph_launch(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 2, "graph_launch")) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], "graph_launch");
    GraphH* g = handle_of<GraphH>(env, a.v[1], TAG_GRAPH);
    if (!c) return nullptr;
    if (!g || !g->g) return arg_error(env, "graph_launch", 1, "a live graph"), nullptr;
    const int rc = ti_graph_launch(c->c, g->g);
    return rc ? throw_ti(env, "graph_launch", rc) : undefined(env);
}

napi_value js_graph_destroy(napi_env env, napi_callback_info info) {
    Args a(env, info);
    GraphH* g = a.n == 1 ? handle_of<GraphH>(env, a.v[0], TAG_GRAPH) : nullptr;
    if (!g) return arg_error(env, "graph_destroy", 0, "a graph"), nullptr;
    if (g->g && !g->ctx->closed) ti_graph_destroy(g->g);
    g->g = nullptr;
    return undefined(env);
}

napi_value js_event_elapsed_ms(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 3, "event_elapsed_ms")) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], "event_elapsed_ms");
    int64_t s0, s1;
    if (!c || !get_i64(env, a.v[1], &s0, "event_elapsed_ms", 1) || !get_i64(env, a.v[2], &s1, "event_elapsed_ms", 2)) return nullptr;
    float ms = 0.0f;
    const int rc = ti_event_elapsed_ms(c->c, (int)s0, (int)s1, &ms);
    return rc ? throw_ti(env, "event_elapsed_ms", rc) : num(env, ms);
}

// rmsnorm_gemv_q4(ctx, x, norm_w, eps, K, [packs], [scales], [ys], [Ns], xq_out, xs_out)
napi_value js_rmsnorm_gemv_q4(napi_env env, napi_callback_info info) {
    const char* fn = "rmsnorm_gemv_q4";
    Args a(env, info);
    if (!want_args(env, a, 11, fn)) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], fn);
    void *x, *nw, *xq, *xs;
    double eps;
    int64_t K;
    if (!c || !get_dptr(env, a.v[1], &x, fn, 1) || !get_dptr(env, a.v[2], &nw, fn, 2)) return nullptr;
    if (napi_get_value_double(env, a.v[3], &eps) != napi_ok) return arg_error(env, fn, 3, "a number"), nullptr;
    if (!get_i64(env, a.v[4], &K, fn, 4) || !get_dptr(env, a.v[9], &xq, fn, 9) || !get_dptr(env, a.v[10], &xs, fn, 10)) return nullptr;
    uint32_t n[4] = {0, 0, 0, 0};
    void* arr[3][3] = {};
    int Ns[3] = {0, 0, 0};
    for (int k = 0; k < 4; k++) {
        bool is;
        napi_is_array(env, a.v[5 + k], &is);
        if (!is) return arg_error(env, fn, 5 + k, "an array"), nullptr;
        napi_get_array_length(env, a.v[5 + k], &n[k]);
        if (n[k] < 1 || n[k] > 3 || n[k] != n[0]) return throw_msg(env, "rmsnorm_gemv_q4: packs/scales/ys/Ns need 1..3 entries each, all alike");
        for (uint32_t i = 0; i < n[k]; i++) {
            napi_value e;
            napi_get_element(env, a.v[5 + k], i, &e);
            if (k < 3) {
                if (!get_dptr(env, e, &arr[k][i], fn, 5 + k)) return nullptr;
            } else {
                int64_t t;
                if (!get_i64(env, e, &t, fn, 8)) return nullptr;
                Ns[i] = (int)t;
            }
        }
    }
    const int rc = ti_rmsnorm_gemv_q4(c->c, (const float*)x, (const uint16_t*)nw, (float)eps, (int)K, (int)n[0],
                                      (const uint32_t* const*)arr[0], (const uint16_t* const*)arr[1], (float* const*)arr[2],
                                      Ns, (uint32_t*)xq, (float*)xs);
    return rc ? throw_ti(env, fn, rc) : undefined(env);
}

// an array argument of 1..3 device buffers (or of integers)
bool get_dptr_list(napi_env env, napi_value v, void** out, uint32_t* n, const char* fn, size_t i) {
    bool is;
    napi_is_array(env, v, &is);
    if (!is) return arg_error(env, fn, i, "an array of 1..3 device buffers");
    napi_get_array_length(env, v, n);
    if (*n < 1 || *n > 3) return arg_error(env, fn, i, "an array of 1..3 device buffers");
    for (uint32_t k = 0; k < *n; k++) {
        napi_value e;
        napi_get_element(env, v, k, &e);
        if (!get_dptr(env, e, &out[k], fn, i)) return false;
    }
    return true;
}

bool get_int_list(napi_env env, napi_value v, int* out, uint32_t n, const char* fn, size_t i) {
    bool is;
    napi_is_array(env, v, &is);
    uint32_t len = 0;
    if (is) napi_get_array_length(env, v, &len);
    if (!is || len != n) return arg_error(env, fn, i, "an array of integers, one per matrix");
    for (uint32_t k = 0; k < n; k++) {
        napi_value e;
        int64_t t;
        napi_get_element(env, v, k, &e);
        if (!get_i64(env, e, &t, fn, i)) return false;
        out[k] = (int)t;
    }
    return true;
}

// tern_gemv_multi(ctx, act, xsum, K, [codes], [scales], [outs], [Ns])
napi_value js_tern_gemv_multi(napi_env env, napi_callback_info info) {
    const char* fn = "tern_gemv_multi";
    Args a(env, info);
    if (!want_args(env, a, 8, fn)) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], fn);
    void *act, *xsum, *cd[3], *sc[3], *o[3];
    int64_t K;
    uint32_t n0, n1, n2;
    int Ns[3];
    if (!c || !get_dptr(env, a.v[1], &act, fn, 1) || !get_dptr(env, a.v[2], &xsum, fn, 2) || !get_i64(env, a.v[3], &K, fn, 3) ||
        !get_dptr_list(env, a.v[4], cd, &n0, fn, 4) || !get_dptr_list(env, a.v[5], sc, &n1, fn, 5) ||
        !get_dptr_list(env, a.v[6], o, &n2, fn, 6))
        return nullptr;
    if (n1 != n0 || n2 != n0) return throw_msg(env, "tern_gemv_multi: codes/scales/outs need the same length");
    if (!get_int_list(env, a.v[7], Ns, n0, fn, 7)) return nullptr;
    const int rc = ti_tern_gemv_multi(c->c, (const int8_t*)act, (const int32_t*)xsum, (int)K, (int)n0, (const uint8_t* const*)cd,
                                      (const float* const*)sc, (float* const*)o, Ns);
    return rc ? throw_ti(env, fn, rc) : undefined(env);
}

// ---- Qwen3 decoder object ---------------------------------------------------------------
bool cfg_int(napi_env env, napi_value o, const char* key, int* out, bool required, int dflt) {
    bool has;
    napi_has_named_property(env, o, key, &has);
    if (!has) {
        if (required) { throw_msg(env, std::string("qwen3_create: config.") + key + " is required"); return false; }
        *out = dflt;
        return true;
    }
    napi_value v;
    napi_get_named_property(env, o, key, &v);
    int64_t t;
    if (!get_i64(env, v, &t, key, 1)) return false;
    *out = (int)t;
    return true;
}

bool cfg_float(napi_env env, napi_value o, const char* key, float* out, float dflt) {
    bool has;
    napi_has_named_property(env, o, key, &has);
    if (!has) { *out = dflt; return true; }
    napi_value v;
    napi_get_named_property(env, o, key, &v);
    double d;
    if (napi_get_value_double(env, v, &d) != napi_ok) { arg_error(env, key, 1, "a number"); return false; }
    *out = (float)d;
    return true;
}

// qwen3_create(ctx, {layers, hidden, intermediate, n_heads, n_kv_heads, head_dim, vocab,
//                    rope_theta, rms_eps, max_ctx, max_tokens})
napi_value js_qwen3_create(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 2, "qwen3_create")) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], "qwen3_create");
    if (!c) return nullptr;
    ti_qwen3_config cfg;
    std::memset(&cfg, 0, sizeof cfg);
    napi_value o = a.v[1];
    if (!cfg_int(env, o, "layers", &cfg.layers, true, 0) || !cfg_int(env, o, "hidden", &cfg.hidden, true, 0) ||
        !cfg_int(env, o, "intermediate", &cfg.intermediate, true, 0) || !cfg_int(env, o, "n_heads", &cfg.n_heads, true, 0) ||
        !cfg_int(env, o, "n_kv_heads", &cfg.n_kv_heads, true, 0) || !cfg_int(env, o, "head_dim", &cfg.head_dim, true, 0) ||
        !cfg_int(env, o, "vocab", &cfg.vocab, true, 0) || !cfg_float(env, o, "rope_theta", &cfg.rope_theta, 1000000.0f) ||
        !cfg_float(env, o, "rms_eps", &cfg.rms_eps, 1e-6f) || !cfg_int(env, o, "max_ctx", &cfg.max_ctx, false, 4096) ||
        !cfg_int(env, o, "max_tokens", &cfg.max_tokens, false, 256))
        return nullptr;
    ti_qwen3* m = nullptr;
    const int rc = ti_qwen3_create(c->c, &cfg, &m);
    if (rc) return throw_ti(env, "qwen3_create", rc);
    ModelH* h = new ModelH;
    h->ctx = c;
    c->refs++;
    h->m = m;
    h->cfg = cfg;
    napi_value out;
    napi_create_external(env, h, fin_model, nullptr, &out);
    return out;
}

ModelH* get_model(napi_env env, napi_value v, const char* fn, size_t i) {
    ModelH* m = handle_of<ModelH>(env, v, TAG_MODEL);
    if (!m || !m->m) { arg_error(env, fn, i, "a live model from qwen3_create()"); return nullptr; }
    if (m->ctx->closed) { throw_msg(env, std::string(fn) + ": the model's context was shut down"); return nullptr; }
    return m;
}

napi_value js_qwen3_destroy(napi_env env, napi_callback_info info) {
    Args a(env, info);
    ModelH* m = a.n == 1 ? get_model(env, a.v[0], "qwen3_destroy", 0) : nullptr;
    if (!m) return a.n == 1 ? nullptr : throw_msg(env, "qwen3_destroy expects (model)");
    const int rc = ti_qwen3_destroy(m->ctx->c, m->m);
    m->m = nullptr;
    return rc ? throw_ti(env, "qwen3_destroy", rc) : undefined(env);
}

// qwen3_tensor(model, name) -> {data, dataBytes, scales|null, scaleBytes}
napi_value js_qwen3_tensor(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 2, "qwen3_tensor")) return nullptr;
    ModelH* m = get_model(env, a.v[0], "qwen3_tensor", 0);
    if (!m) return nullptr;
    char name[256];
    size_t nl;
    if (napi_get_value_string_utf8(env, a.v[1], name, sizeof name, &nl) != napi_ok) return arg_error(env, "qwen3_tensor", 1, "a string"), nullptr;
    void *d = nullptr, *s = nullptr;
    size_t db = 0, sb = 0;
    const int rc = ti_qwen3_tensor(m->m, name, &d, &db, &s, &sb);
    if (rc) return throw_ti(env, "qwen3_tensor", rc);
    napi_value o, nul;
    napi_create_object(env, &o);
    napi_get_null(env, &nul);
    napi_set_named_property(env, o, "data", make_buf(env, m->ctx, d, db, false, a.v[0]));
    napi_set_named_property(env, o, "dataBytes", num(env, (double)db));
    napi_set_named_property(env, o, "scales", s ? make_buf(env, m->ctx, s, sb, false, a.v[0]) : nul);
    napi_set_named_property(env, o, "scaleBytes", num(env, (double)sb));
    return o;
}

// qwen3_kv(model, layer) -> {kq, ks, vq, vs}
napi_value js_qwen3_kv(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 2, "qwen3_kv")) return nullptr;
    ModelH* m = get_model(env, a.v[0], "qwen3_kv", 0);
    int64_t layer;
    if (!m || !get_i64(env, a.v[1], &layer, "qwen3_kv", 1)) return nullptr;
    uint32_t *kq, *vq;
    float *ks, *vs;
    int rc = ti_qwen3_kv(m->m, (int)layer, &kq, &ks, &vq, &vs);
    int slots = 0;
    if (!rc) rc = ti_qwen3_kv_layout(m->m, &slots);
    if (rc) return throw_ti(env, "qwen3_kv", rc);
    napi_value o;
    napi_create_object(env, &o);
    const size_t scales = (size_t)m->cfg.max_ctx * m->cfg.n_kv_heads * (m->cfg.head_dim / 32) * 4;
    const size_t codes = (size_t)m->cfg.max_ctx * slots * m->cfg.head_dim;   // int8 per K or V (padded rows)
    napi_set_named_property(env, o, "kq", make_buf(env, m->ctx, kq, codes, false, a.v[0]));
    napi_set_named_property(env, o, "ks", make_buf(env, m->ctx, ks, scales, false, a.v[0]));
    napi_set_named_property(env, o, "vq", make_buf(env, m->ctx, vq, codes, false, a.v[0]));
    napi_set_named_property(env, o, "vs", make_buf(env, m->ctx, vs, scales, false, a.v[0]));
    napi_set_named_property(env, o, "slots", num(env, slots));
    return o;
}

// qwen3_kv_layout(model) -> code slots per cached position
napi_value js_qwen3_kv_layout(napi_env env, napi_callback_info info) {
    const char* fn = "qwen3_kv_layout";
    Args a(env, info);
    if (!want_args(env, a, 1, fn)) return nullptr;
    ModelH* m = get_model(env, a.v[0], fn, 0);
    if (!m) return nullptr;
    int slots = 0;
    const int rc = ti_qwen3_kv_layout(m->m, &slots);
    return rc ? throw_ti(env, fn, rc) : num(env, slots);
}

// qwen3_kv_write(ctx, model, layer, kr, v, T, pos): kvQuantWrite into the model's cache
napi_value js_qwen3_kv_write(napi_env env, napi_callback_info info) {
    const char* fn = "qwen3_kv_write";
    Args a(env, info);
    if (!want_args(env, a, 7, fn)) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], fn);
    ModelH* m = c ? get_model(env, a.v[1], fn, 1) : nullptr;
    int64_t layer, T, pos;
    void *kr, *v;
    if (!m || !get_i64(env, a.v[2], &layer, fn, 2) || !get_dptr(env, a.v[3], &kr, fn, 3) ||
        !get_dptr(env, a.v[4], &v, fn, 4) || !get_i64(env, a.v[5], &T, fn, 5) || !get_i64(env, a.v[6], &pos, fn, 6))
        return nullptr;
    const int rc = ti_qwen3_kv_write(c->c, m->m, (int)layer, static_cast<const float*>(kr), static_cast<const float*>(v),
                                     (int)T, (int)pos);
    return rc ? throw_ti(env, fn, rc) : undefined(env);
}

napi_value js_qwen3_logits(napi_env env, napi_callback_info info) {
    Args a(env, info);
    ModelH* m = a.n == 1 ? get_model(env, a.v[0], "qwen3_logits", 0) : nullptr;
    if (!m) return a.n == 1 ? nullptr : throw_msg(env, "qwen3_logits expects (model)");
    float* l = nullptr;
    const int rc = ti_qwen3_logits(m->m, &l);
    return rc ? throw_ti(env, "qwen3_logits", rc) : make_buf(env, m->ctx, l, (size_t)m->cfg.vocab * 4, false, a.v[0]);
}

bool host_i32(napi_env env, napi_value v, const int32_t** data, size_t* n, const char* fn, size_t i) {
    bool is;
    napi_is_typedarray(env, v, &is);
    if (!is) return arg_error(env, fn, i, "an Int32Array");
    napi_typedarray_type t;
    void* d;
    napi_value ab;
    size_t off;
    napi_get_typedarray_info(env, v, &t, n, &d, &ab, &off);
    if (t != napi_int32_array) return arg_error(env, fn, i, "an Int32Array");
    *data = static_cast<const int32_t*>(d);
    return true;
}

// qwen3_forward(ctx, model, ids: Int32Array | null, T, pos)
napi_value js_qwen3_forward(napi_env env, napi_callback_info info) {
    const char* fn = "qwen3_forward";
    Args a(env, info);
    if (!want_args(env, a, 5, fn)) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], fn);
    ModelH* m = c ? get_model(env, a.v[1], fn, 1) : nullptr;
    int64_t T, pos;
    if (!m || !get_i64(env, a.v[3], &T, fn, 3) || !get_i64(env, a.v[4], &pos, fn, 4)) return nullptr;
    const int32_t* ids = nullptr;
    if (!is_nullish(env, a.v[2])) {
        size_t n;
        if (!host_i32(env, a.v[2], &ids, &n, fn, 2)) return nullptr;
        if ((int64_t)n < T) return throw_msg(env, "qwen3_forward: ids holds fewer than T tokens");
    }
    const int rc = ti_qwen3_forward(c->c, m->m, ids, (int)T, (int)pos);
    return rc ? throw_ti(env, fn, rc) : undefined(env);
}

napi_value js_qwen3_decode(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 2, "qwen3_decode")) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], "qwen3_decode");
    ModelH* m = c ? get_model(env, a.v[1], "qwen3_decode", 1) : nullptr;
    if (!m) return nullptr;
    const int rc = ti_qwen3_decode(c->c, m->m);
    return rc ? throw_ti(env, "qwen3_decode", rc) : undefined(env);
}

napi_value js_qwen3_set_pos(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 3, "qwen3_set_pos")) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], "qwen3_set_pos");
    ModelH* m = c ? get_model(env, a.v[1], "qwen3_set_pos", 1) : nullptr;
    int64_t pos;
    if (!m || !get_i64(env, a.v[2], &pos, "qwen3_set_pos", 2)) return nullptr;
    const int rc = ti_qwen3_set_pos(c->c, m->m, (int)pos);
    return rc ? throw_ti(env, "qwen3_set_pos", rc) : undefined(env);
}

// qwen3_decode_splits(model, pos) -> the attention splits of a decode step captured at pos
napi_value js_qwen3_decode_splits(napi_env env, napi_callback_info info) {
    const char* fn = "qwen3_decode_splits";
    Args a(env, info);
    if (!want_args(env, a, 2, fn)) return nullptr;
    ModelH* m = get_model(env, a.v[0], fn, 0);
    int64_t pos;
    if (!m || !get_i64(env, a.v[1], &pos, fn, 1)) return nullptr;
    int n = 0;
    const int rc = ti_qwen3_decode_splits(m->m, (int)pos, &n);
    return rc ? throw_ti(env, fn, rc) : num(env, n);
}

// qwen3_sampling(ctx, model, temperature): the temperature of the following steps (0: greedy)
napi_value js_qwen3_sampling(napi_env env, napi_callback_info info) {
    const char* fn = "qwen3_sampling";
    Args a(env, info);
    if (!want_args(env, a, 3, fn)) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], fn);
    ModelH* m = c ? get_model(env, a.v[1], fn, 1) : nullptr;
    double t;
    if (!m) return nullptr;
    if (napi_get_value_double(env, a.v[2], &t) != napi_ok) return arg_error(env, fn, 2, "a number"), nullptr;
    const int rc = ti_qwen3_sampling(c->c, m->m, (float)t);
    return rc ? throw_ti(env, fn, rc) : undefined(env);
}

// qwen3_seed(ctx, model, state) / qwen3_get_seed(ctx, model) -> state: the seed stream
napi_value js_qwen3_seed(napi_env env, napi_callback_info info) {
    const char* fn = "qwen3_seed";
    Args a(env, info);
    if (!want_args(env, a, 3, fn)) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], fn);
    ModelH* m = c ? get_model(env, a.v[1], fn, 1) : nullptr;
    int64_t st;
    if (!m || !get_i64(env, a.v[2], &st, fn, 2)) return nullptr;
    const int rc = ti_qwen3_seed(c->c, m->m, (uint32_t)(st & 0xFFFFFFFF));
    return rc ? throw_ti(env, fn, rc) : undefined(env);
}

napi_value js_qwen3_get_seed(napi_env env, napi_callback_info info) {
    const char* fn = "qwen3_get_seed";
    Args a(env, info);
    if (!want_args(env, a, 2, fn)) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], fn);
    ModelH* m = c ? get_model(env, a.v[1], fn, 1) : nullptr;
    if (!m) return nullptr;
    uint32_t st = 0;
    const int rc = ti_qwen3_get_seed(c->c, m->m, &st);
    if (rc) return throw_ti(env, fn, rc);
    napi_value out;
    napi_create_uint32(env, st, &out);
    return out;
}

// qwen3_trace(model, buffer | null): parity trace of the decoder's intermediate values
napi_value js_qwen3_trace(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 2, "qwen3_trace")) return nullptr;
    ModelH* m = get_model(env, a.v[0], "qwen3_trace", 0);
    void* p = nullptr;
    if (!m || !get_dptr(env, a.v[1], &p, "qwen3_trace", 1)) return nullptr;
    BufH* b = p ? handle_of<BufH>(env, a.v[1], TAG_BUF) : nullptr;
    const int rc = ti_qwen3_trace(m->m, p, b ? b->bytes : 0);
    return rc ? throw_ti(env, "qwen3_trace", rc) : undefined(env);
}

// qwen3_write_tokens(ctx, model, from, ids: Int32Array)
napi_value js_qwen3_write_tokens(napi_env env, napi_callback_info info) {
    const char* fn = "qwen3_write_tokens";
    Args a(env, info);
    if (!want_args(env, a, 4, fn)) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], fn);
    ModelH* m = c ? get_model(env, a.v[1], fn, 1) : nullptr;
    int64_t from;
    const int32_t* ids;
    size_t n;
    if (!m || !get_i64(env, a.v[2], &from, fn, 2) || !host_i32(env, a.v[3], &ids, &n, fn, 3)) return nullptr;
    const int rc = ti_qwen3_write_tokens(c->c, m->m, (int)from, (int)n, ids);
    return rc ? throw_ti(env, fn, rc) : undefined(env);
}

// qwen3_read_tokens(ctx, model, from, count) -> Int32Array
// ---- the .cpu.bin container (binfmt.rs Container) ------------------------------------------
napi_value wrap_cpubin(napi_env env, ti_cpubin* c) {
    CpuBinH* h = new CpuBinH;
    h->c = c;
    napi_value out;
    napi_create_external(env, h, fin_cpubin, nullptr, &out);
    return out;
}

CpuBinH* get_cpubin(napi_env env, napi_value v, const char* fn) {
    CpuBinH* h = handle_of<CpuBinH>(env, v, TAG_CPUBIN);
    if (!h || !h->c) { arg_error(env, fn, 0, "an open container from cpubin_open()"); return nullptr; }
    return h;
}

// cpubin_open(path) -> container
napi_value js_cpubin_open(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 1, "cpubin_open")) return nullptr;
    char path[4096];
    size_t n;
    if (napi_get_value_string_utf8(env, a.v[0], path, sizeof path, &n) != napi_ok) return arg_error(env, "cpubin_open", 0, "a path"), nullptr;
    ti_cpubin* c = nullptr;
    const int rc = ti_cpubin_open(path, &c);
    return rc ? throw_ti(env, "cpubin_open", rc) : wrap_cpubin(env, c);
}

// cpubin_parse(bytes: TypedArray | ArrayBuffer) -> container (Container::from_bytes)
napi_value js_cpubin_parse(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 1, "cpubin_parse")) return nullptr;
    void* d;
    size_t len;
    if (!host_bytes(env, a.v[0], &d, &len, "cpubin_parse", 0)) return nullptr;
    ti_cpubin* c = nullptr;
    const int rc = ti_cpubin_parse(d, len, &c);
    return rc ? throw_ti(env, "cpubin_parse", rc) : wrap_cpubin(env, c);
}

napi_value js_cpubin_close(napi_env env, napi_callback_info info) {
    Args a(env, info);
    CpuBinH* h = a.n == 1 ? get_cpubin(env, a.v[0], "cpubin_close") : nullptr;
    if (!h) return a.n == 1 ? nullptr : throw_msg(env, "cpubin_close expects (container)");
    ti_cpubin_close(h->c);
    h->c = nullptr;
    return undefined(env);
}

// cpubin_summary(container) -> {groupSize, tensors, blobBytes}
napi_value js_cpubin_summary(napi_env env, napi_callback_info info) {
    Args a(env, info);
    CpuBinH* h = a.n == 1 ? get_cpubin(env, a.v[0], "cpubin_summary") : nullptr;
    if (!h) return a.n == 1 ? nullptr : throw_msg(env, "cpubin_summary expects (container)");
    int g = 0, n = 0;
    size_t b = 0;
    const int rc = ti_cpubin_summary(h->c, &g, &n, &b);
    if (rc) return throw_ti(env, "cpubin_summary", rc);
    napi_value o;
    napi_create_object(env, &o);
    napi_set_named_property(env, o, "groupSize", num(env, g));
    napi_set_named_property(env, o, "tensors", num(env, n));
    napi_set_named_property(env, o, "blobBytes", num(env, (double)b));
    return o;
}

// cpubin_name(container, i) -> the i-th tensor name (name order)
napi_value js_cpubin_name(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 2, "cpubin_name")) return nullptr;
    CpuBinH* h = get_cpubin(env, a.v[0], "cpubin_name");
    int64_t i;
    if (!h || !get_i64(env, a.v[1], &i, "cpubin_name", 1)) return nullptr;
    const char* name = nullptr;
    const int rc = ti_cpubin_name(h->c, (int)i, &name);
    if (rc) return throw_ti(env, "cpubin_name", rc);
    napi_value out;
    napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &out);
    return out;
}

napi_value copy_bytes(napi_env env, const void* p, size_t n) {
    void* d;
    napi_value ab, u8;
    napi_create_arraybuffer(env, n, &d, &ab);
    if (n) std::memcpy(d, p, n);
    napi_create_typedarray(env, napi_uint8_array, n, ab, 0, &u8);
    return u8;
}

// cpubin_tensor(container, name) -> {kind: 'tern'|'embed_f16'|'f32', N, K, shape, data: Uint8Array,
// scales: Uint8Array | null} (copies of the blob ranges)
napi_value js_cpubin_tensor(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 2, "cpubin_tensor")) return nullptr;
    CpuBinH* h = get_cpubin(env, a.v[0], "cpubin_tensor");
    if (!h) return nullptr;
    char name[512];
    size_t nl;
    if (napi_get_value_string_utf8(env, a.v[1], name, sizeof name, &nl) != napi_ok) return arg_error(env, "cpubin_tensor", 1, "a string"), nullptr;
    ti_cpubin_tensor_info t;
    const int rc = ti_cpubin_tensor(h->c, name, &t);
    if (rc) return throw_ti(env, "cpubin_tensor", rc);
    napi_value o, kind, shape, nul;
    napi_create_object(env, &o);
    napi_get_null(env, &nul);
    napi_create_string_utf8(env, t.kind == TI_CPUBIN_TERN ? "tern" : t.kind == TI_CPUBIN_EMBED_F16 ? "embed_f16" : "f32",
                            NAPI_AUTO_LENGTH, &kind);
    napi_set_named_property(env, o, "kind", kind);
    napi_set_named_property(env, o, "N", num(env, (double)t.N));
    napi_set_named_property(env, o, "K", num(env, (double)t.K));
    napi_create_array_with_length(env, (size_t)t.ndim, &shape);
    for (int i = 0; i < t.ndim; i++) napi_set_element(env, shape, (uint32_t)i, num(env, (double)t.shape[i]));
    napi_set_named_property(env, o, "shape", shape);
    napi_set_named_property(env, o, "data", copy_bytes(env, t.data, t.data_bytes));
    napi_set_named_property(env, o, "scales", t.scales ? copy_bytes(env, t.scales, t.scale_bytes) : nul);
    return o;
}

// cpubin_embed_row(container, name, row, dim) -> Float32Array
napi_value js_cpubin_embed_row(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 4, "cpubin_embed_row")) return nullptr;
    CpuBinH* h = get_cpubin(env, a.v[0], "cpubin_embed_row");
    if (!h) return nullptr;
    char name[512];
    size_t nl;
    int64_t row, dim;
    if (napi_get_value_string_utf8(env, a.v[1], name, sizeof name, &nl) != napi_ok) return arg_error(env, "cpubin_embed_row", 1, "a string"), nullptr;
    if (!get_i64(env, a.v[2], &row, "cpubin_embed_row", 2) || !get_i64(env, a.v[3], &dim, "cpubin_embed_row", 3)) return nullptr;
    if (dim < 0 || dim > (1 << 24)) return throw_msg(env, "cpubin_embed_row: bad dim");
    void* d;
    napi_value ab, f32;
    napi_create_arraybuffer(env, (size_t)dim * 4, &d, &ab);
    const int rc = ti_cpubin_embed_row(h->c, name, row, static_cast<float*>(d), (int)dim);
    if (rc) return throw_ti(env, "cpubin_embed_row", rc);
    napi_create_typedarray(env, napi_float32_array, (size_t)dim, ab, 0, &f32);
    return f32;
}

// ---- the Bonsai decoder (ti_bonsai_*) ------------------------------------------------------------
BonsaiH* get_bonsai(napi_env env, napi_value v, const char* fn, size_t i) {
    BonsaiH* h = handle_of<BonsaiH>(env, v, TAG_BONSAI);
    if (!h || !h->m) { arg_error(env, fn, i, "a live model from bonsai_create()"); return nullptr; }
    if (h->ctx->closed) { throw_msg(env, std::string(fn) + ": the model's context was shut down"); return nullptr; }
    return h;
}

// bonsai_create(ctx, {layers, hidden, intermediate, n_heads, n_kv_heads, head_dim, vocab,
// rope_theta, rms_eps, max_ctx}) -> model
napi_value js_bonsai_create(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 2, "bonsai_create")) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], "bonsai_create");
    if (!c) return nullptr;
    ti_bonsai_config cfg;
    std::memset(&cfg, 0, sizeof cfg);
    napi_value o = a.v[1];
    if (!cfg_int(env, o, "layers", &cfg.layers, true, 0) || !cfg_int(env, o, "hidden", &cfg.hidden, true, 0) ||
        !cfg_int(env, o, "intermediate", &cfg.intermediate, true, 0) || !cfg_int(env, o, "n_heads", &cfg.n_heads, true, 0) ||
        !cfg_int(env, o, "n_kv_heads", &cfg.n_kv_heads, true, 0) || !cfg_int(env, o, "head_dim", &cfg.head_dim, true, 0) ||
        !cfg_int(env, o, "vocab", &cfg.vocab, true, 0) || !cfg_float(env, o, "rope_theta", &cfg.rope_theta, 1000000.0f) ||
        !cfg_float(env, o, "rms_eps", &cfg.rms_eps, 1e-6f) || !cfg_int(env, o, "max_ctx", &cfg.max_ctx, false, 4096))
        return nullptr;
    ti_bonsai* m = nullptr;
    const int rc = ti_bonsai_create(c->c, &cfg, &m);
    if (rc) return throw_ti(env, "bonsai_create", rc);
    BonsaiH* h = new BonsaiH;
    h->ctx = c;
    c->refs++;
    h->m = m;
    h->cfg = cfg;
    napi_value out;
    napi_create_external(env, h, fin_bonsai, nullptr, &out);
    return out;
}

napi_value js_bonsai_destroy(napi_env env, napi_callback_info info) {
    Args a(env, info);
    BonsaiH* h = a.n == 1 ? get_bonsai(env, a.v[0], "bonsai_destroy", 0) : nullptr;
    if (!h) return a.n == 1 ? nullptr : throw_msg(env, "bonsai_destroy expects (model)");
    const int rc = ti_bonsai_destroy(h->ctx->c, h->m);
    h->m = nullptr;
    return rc ? throw_ti(env, "bonsai_destroy", rc) : undefined(env);
}

// bonsai_load(ctx, model, container)
napi_value js_bonsai_load(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 3, "bonsai_load")) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], "bonsai_load");
    BonsaiH* h = c ? get_bonsai(env, a.v[1], "bonsai_load", 1) : nullptr;
    CpuBinH* b = handle_of<CpuBinH>(env, a.v[2], TAG_CPUBIN);
    if (!h) return nullptr;
    if (!b || !b->c) return arg_error(env, "bonsai_load", 2, "an open container from cpubin_open()"), nullptr;
    const int rc = ti_bonsai_load(c->c, h->m, b->c);
    return rc ? throw_ti(env, "bonsai_load", rc) : undefined(env);
}

// bonsai_tensor(model, name) -> {data, dataBytes, scales|null, scaleBytes}
napi_value js_bonsai_tensor(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 2, "bonsai_tensor")) return nullptr;
    BonsaiH* h = get_bonsai(env, a.v[0], "bonsai_tensor", 0);
    if (!h) return nullptr;
    char name[256];
    size_t nl;
    if (napi_get_value_string_utf8(env, a.v[1], name, sizeof name, &nl) != napi_ok) return arg_error(env, "bonsai_tensor", 1, "a string"), nullptr;
    void *d = nullptr, *s = nullptr;
    size_t db = 0, sb = 0;
    const int rc = ti_bonsai_tensor(h->m, name, &d, &db, &s, &sb);
    if (rc) return throw_ti(env, "bonsai_tensor", rc);
    napi_value o, nul;
    napi_create_object(env, &o);
    napi_get_null(env, &nul);
    napi_set_named_property(env, o, "data", make_buf(env, h->ctx, d, db, false, a.v[0]));
    napi_set_named_property(env, o, "dataBytes", num(env, (double)db));
    napi_set_named_property(env, o, "scales", s ? make_buf(env, h->ctx, s, sb, false, a.v[0]) : nul);
    napi_set_named_property(env, o, "scaleBytes", num(env, (double)sb));
    return o;
}

// bonsai_kv(model, layer) -> {kc, vc}
napi_value js_bonsai_kv(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 2, "bonsai_kv")) return nullptr;
    BonsaiH* h = get_bonsai(env, a.v[0], "bonsai_kv", 0);
    int64_t layer;
    if (!h || !get_i64(env, a.v[1], &layer, "bonsai_kv", 1)) return nullptr;
    float *kc, *vc;
    const int rc = ti_bonsai_kv(h->m, (int)layer, &kc, &vc);
    if (rc) return throw_ti(env, "bonsai_kv", rc);
    const size_t bytes = (size_t)h->cfg.max_ctx * h->cfg.n_kv_heads * h->cfg.head_dim * 4;
    napi_value o;
    napi_create_object(env, &o);
    napi_set_named_property(env, o, "kc", make_buf(env, h->ctx, kc, bytes, false, a.v[0]));
    napi_set_named_property(env, o, "vc", make_buf(env, h->ctx, vc, bytes, false, a.v[0]));
    return o;
}

napi_value js_bonsai_logits(napi_env env, napi_callback_info info) {
    Args a(env, info);
    BonsaiH* h = a.n == 1 ? get_bonsai(env, a.v[0], "bonsai_logits", 0) : nullptr;
    if (!h) return a.n == 1 ? nullptr : throw_msg(env, "bonsai_logits expects (model)");
    float* l = nullptr;
    const int rc = ti_bonsai_logits(h->m, &l);
    return rc ? throw_ti(env, "bonsai_logits", rc) : make_buf(env, h->ctx, l, (size_t)h->cfg.vocab * 4, false, a.v[0]);
}

// bonsai_forward(ctx, model, ids: Int32Array | null, T, pos)
napi_value js_bonsai_forward(napi_env env, napi_callback_info info) {
    const char* fn = "bonsai_forward";
    Args a(env, info);
    if (!want_args(env, a, 5, fn)) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], fn);
    BonsaiH* h = c ? get_bonsai(env, a.v[1], fn, 1) : nullptr;
    int64_t T, pos;
    if (!h || !get_i64(env, a.v[3], &T, fn, 3) || !get_i64(env, a.v[4], &pos, fn, 4)) return nullptr;
    const int32_t* ids = nullptr;
    if (!is_nullish(env, a.v[2])) {
        size_t n;
        if (!host_i32(env, a.v[2], &ids, &n, fn, 2)) return nullptr;
        if ((int64_t)n < T) return throw_msg(env, "bonsai_forward: ids holds fewer than T tokens");
    }
    const int rc = ti_bonsai_forward(c->c, h->m, ids, (int)T, (int)pos);
    return rc ? throw_ti(env, fn, rc) : undefined(env);
}

napi_value js_bonsai_decode(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 2, "bonsai_decode")) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], "bonsai_decode");
    BonsaiH* h = c ? get_bonsai(env, a.v[1], "bonsai_decode", 1) : nullptr;
    if (!h) return nullptr;
    const int rc = ti_bonsai_decode(c->c, h->m);
    return rc ? throw_ti(env, "bonsai_decode", rc) : undefined(env);
}

napi_value js_bonsai_set_pos(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 3, "bonsai_set_pos")) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], "bonsai_set_pos");
    BonsaiH* h = c ? get_bonsai(env, a.v[1], "bonsai_set_pos", 1) : nullptr;
    int64_t pos;
    if (!h || !get_i64(env, a.v[2], &pos, "bonsai_set_pos", 2)) return nullptr;
    const int rc = ti_bonsai_set_pos(c->c, h->m, (int)pos);
    return rc ? throw_ti(env, "bonsai_set_pos", rc) : undefined(env);
}

napi_value js_bonsai_write_tokens(napi_env env, napi_callback_info info) {
    const char* fn = "bonsai_write_tokens";
    Args a(env, info);
    if (!want_args(env, a, 4, fn)) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], fn);
    BonsaiH* h = c ? get_bonsai(env, a.v[1], fn, 1) : nullptr;
    int64_t from;
    const int32_t* ids;
    size_t n;
    if (!h || !get_i64(env, a.v[2], &from, fn, 2) || !host_i32(env, a.v[3], &ids, &n, fn, 3)) return nullptr;
    const int rc = ti_bonsai_write_tokens(c->c, h->m, (int)from, (int)n, ids);
    return rc ? throw_ti(env, fn, rc) : undefined(env);
}

napi_value js_bonsai_read_tokens(napi_env env, napi_callback_info info) {
    const char* fn = "bonsai_read_tokens";
    Args a(env, info);
    if (!want_args(env, a, 4, fn)) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], fn);
    BonsaiH* h = c ? get_bonsai(env, a.v[1], fn, 1) : nullptr;
    int64_t from, count;
    if (!h || !get_i64(env, a.v[2], &from, fn, 2) || !get_i64(env, a.v[3], &count, fn, 3)) return nullptr;
    if (count < 0 || count > (1 << 26)) return throw_msg(env, "bonsai_read_tokens: bad count");
    void* data;
    napi_value ab, arr;
    napi_create_arraybuffer(env, (size_t)count * 4, &data, &ab);
    const int rc = ti_bonsai_read_tokens(c->c, h->m, (int)from, (int)count, static_cast<int32_t*>(data));
    if (rc) return throw_ti(env, fn, rc);
    napi_create_typedarray(env, napi_int32_array, (size_t)count, ab, 0, &arr);
    return arr;
}

// bonsai_trace(model, buffer | null)
napi_value js_bonsai_trace(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!want_args(env, a, 2, "bonsai_trace")) return nullptr;
    BonsaiH* h = get_bonsai(env, a.v[0], "bonsai_trace", 0);
    void* p = nullptr;
    if (!h || !get_dptr(env, a.v[1], &p, "bonsai_trace", 1)) return nullptr;
    BufH* b = p ? handle_of<BufH>(env, a.v[1], TAG_BUF) : nullptr;
    const int rc = ti_bonsai_trace(h->m, p, b ? b->bytes : 0);
    return rc ? throw_ti(env, "bonsai_trace", rc) : undefined(env);
}

// qwen3_read_tokens_async(ctx, model, from, count, int32array): queued D2H of the token
// history into the array (from host_alloc); complete once an event recorded after it is
napi_value js_qwen3_read_tokens_async(napi_env env, napi_callback_info info) {
    const char* fn = "qwen3_read_tokens_async";
    Args a(env, info);
    if (!want_args(env, a, 5, fn)) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], fn);
    ModelH* m = c ? get_model(env, a.v[1], fn, 1) : nullptr;
    int64_t from, count;
    if (!m || !get_i64(env, a.v[2], &from, fn, 2) || !get_i64(env, a.v[3], &count, fn, 3)) return nullptr;
    bool is_ta = false;
    napi_is_typedarray(env, a.v[4], &is_ta);
    if (!is_ta) return arg_error(env, fn, 4, "an Int32Array"), nullptr;
    napi_typedarray_type tt;
    size_t len;
    void* data;
    napi_value ab;
    size_t boff;
    napi_get_typedarray_info(env, a.v[4], &tt, &len, &data, &ab, &boff);
    if (tt != napi_int32_array) return arg_error(env, fn, 4, "an Int32Array"), nullptr;
    if (count < 0 || (size_t)count > len) return throw_msg(env, "qwen3_read_tokens_async: count exceeds the array");
    if (count && !pinned_range(data, (size_t)count * 4))
        return throw_msg(env, "qwen3_read_tokens_async: the array is not live host_alloc memory");
    const int rc = ti_qwen3_read_tokens_async(c->c, m->m, (int)from, (int)count, static_cast<int32_t*>(data));
    return rc ? throw_ti(env, fn, rc) : undefined(env);
}

napi_value js_qwen3_read_tokens(napi_env env, napi_callback_info info) {
    const char* fn = "qwen3_read_tokens";
    Args a(env, info);
    if (!want_args(env, a, 4, fn)) return nullptr;
    CtxH* c = get_ctx(env, a.v[0], fn);
    ModelH* m = c ? get_model(env, a.v[1], fn, 1) : nullptr;
    int64_t from, count;
    if (!m || !get_i64(env, a.v[2], &from, fn, 2) || !get_i64(env, a.v[3], &count, fn, 3)) return nullptr;
    if (count < 0 || count > (1 << 26)) return throw_msg(env, "qwen3_read_tokens: bad count");
    void* data;
    napi_value ab, arr;
    napi_create_arraybuffer(env, (size_t)count * 4, &data, &ab);
    const int rc = ti_qwen3_read_tokens(c->c, m->m, (int)from, (int)count, static_cast<int32_t*>(data));
    if (rc) return throw_ti(env, fn, rc);
    napi_create_typedarray(env, napi_int32_array, (size_t)count, ab, 0, &arr);
    return arr;
}

#define FN(js, f) {js, nullptr, f, nullptr, nullptr, nullptr, napi_enumerable, nullptr}
#define ENTRY(js, fn)                                                                                 \
    {js, nullptr, [](napi_env e, napi_callback_info i) -> napi_value { return call_entry(e, i, #fn, fn); }, \
     nullptr, nullptr, nullptr, napi_enumerable, nullptr}

napi_value module_init(napi_env env, napi_value exports) {
    const napi_property_descriptor props[] = {
        FN("version", js_version),
        FN("last_error", js_last_error),
        FN("device_count", js_device_count),
        FN("init", js_init),
        FN("shutdown", js_shutdown),
        FN("buf_alloc", js_buf_alloc),
        FN("buf_free", js_buf_free),
        FN("buf_view", js_buf_view),
        FN("buf_bytes", js_buf_bytes),
        FN("buf_write", js_buf_write),
        FN("buf_read", js_buf_read),
        ENTRY("buf_copy", ti_buf_copy),
        ENTRY("buf_fill_u32", ti_buf_fill_u32),
        ENTRY("sync", ti_sync),
        FN("sync_async", js_sync_async),
        FN("event_wait_async", js_event_wait_async),
        FN("host_alloc", js_host_alloc),
        FN("host_free", js_host_free),
        FN("buf_read_async", js_buf_read_async),
        ENTRY("graph_begin", ti_graph_begin),
        FN("graph_end", js_graph_end),
        FN("graph_launch", js_graph_launch),
        FN("graph_destroy", js_graph_destroy),
        ENTRY("event_record", ti_event_record),
        FN("event_elapsed_ms", js_event_elapsed_ms),
        ENTRY("event_wait", ti_event_wait),
        // int4 weights, activations, GEMV / GEMM
        ENTRY("quant_int4_bf16", ti_quant_int4_bf16),
        ENTRY("quant_tern_bf16", ti_quant_tern_bf16),
        ENTRY("gemv_tern2", ti_gemv_tern2),
        ENTRY("gateup_silu_tern2", ti_gateup_silu_tern2),
        ENTRY("quant_act_q8", ti_quant_act_q8),
        ENTRY("quant_act_q8_t", ti_quant_act_q8_t),
        ENTRY("rmsnorm_q8", ti_rmsnorm_q8),
        ENTRY("rmsnorm_q8_t", ti_rmsnorm_q8_t),
        ENTRY("rmsnorm", ti_rmsnorm),
        ENTRY("gemv_q4_q8", ti_gemv_q4_q8),
        ENTRY("gemv_q4_f32", ti_gemv_q4_f32),
        ENTRY("gateup_silu_q4", ti_gateup_silu_q4),
        ENTRY("linear_q4", ti_linear_q4),
        ENTRY("group_dots_q4_q8", ti_group_dots_q4_q8),
        FN("rmsnorm_gemv_q4", js_rmsnorm_gemv_q4),
        ENTRY("rmsnorm_gateup_silu_q4", ti_rmsnorm_gateup_silu_q4),
        ENTRY("rmsnorm_lm_head_argmax", ti_rmsnorm_lm_head_argmax),
        ENTRY("argmax", ti_argmax),
        ENTRY("gumbel_noise", ti_gumbel_noise),
        ENTRY("embed", ti_embed),
        // attention over the int8 KV cache
        ENTRY("attn_prep_q8", ti_attn_prep_q8),
        ENTRY("attn_decode_q8", ti_attn_decode_q8),
        ENTRY("attn_step_q8", ti_attn_step_q8),
        ENTRY("rope_qk", ti_rope_qk),
        ENTRY("kv_write_q8", ti_kv_write_q8),
        ENTRY("attn_causal_q8", ti_attn_causal_q8),
        // ternary
        ENTRY("tern_gemv", ti_tern_gemv),
        ENTRY("tern_gemm", ti_tern_gemm),
        FN("tern_gemv_multi", js_tern_gemv_multi),
        ENTRY("quant_act_tern", ti_quant_act_tern),
        ENTRY("tern_block_dots", ti_tern_block_dots),
        // int3 MoE
        ENTRY("requant43", ti_requant43),
        ENTRY("router", ti_router),
        ENTRY("moe_gemv_q3", ti_moe_gemv_q3),
        ENTRY("moe_gemm_q3", ti_moe_gemm_q3),
        ENTRY("swiglu", ti_swiglu),
        ENTRY("moe_decode_q3", ti_moe_decode_q3),
        ENTRY("moe_prefill_q3", ti_moe_prefill_q3),
        ENTRY("moe_combine", ti_moe_combine),
        // Qwen3 decoder
        FN("qwen3_create", js_qwen3_create),
        FN("qwen3_destroy", js_qwen3_destroy),
        FN("qwen3_tensor", js_qwen3_tensor),
        FN("qwen3_kv", js_qwen3_kv),
        FN("qwen3_kv_layout", js_qwen3_kv_layout),
        FN("qwen3_kv_write", js_qwen3_kv_write),
        FN("qwen3_logits", js_qwen3_logits),
        FN("qwen3_forward", js_qwen3_forward),
        FN("qwen3_decode", js_qwen3_decode),
        FN("qwen3_set_pos", js_qwen3_set_pos),
        FN("qwen3_decode_splits", js_qwen3_decode_splits),
        FN("qwen3_read_tokens_async", js_qwen3_read_tokens_async),
        FN("qwen3_sampling", js_qwen3_sampling),
        FN("qwen3_seed", js_qwen3_seed),
        FN("qwen3_get_seed", js_qwen3_get_seed),
        FN("qwen3_trace", js_qwen3_trace),
        FN("qwen3_write_tokens", js_qwen3_write_tokens),
        FN("qwen3_read_tokens", js_qwen3_read_tokens),
        FN("bonsai_create", js_bonsai_create),
        FN("bonsai_destroy", js_bonsai_destroy),
        FN("bonsai_load", js_bonsai_load),
        FN("bonsai_tensor", js_bonsai_tensor),
        FN("bonsai_kv", js_bonsai_kv),
        FN("bonsai_logits", js_bonsai_logits),
        FN("bonsai_forward", js_bonsai_forward),
        FN("bonsai_decode", js_bonsai_decode),
        FN("bonsai_set_pos", js_bonsai_set_pos),
        FN("bonsai_write_tokens", js_bonsai_write_tokens),
        FN("bonsai_read_tokens", js_bonsai_read_tokens),
        FN("bonsai_trace", js_bonsai_trace),
        FN("cpubin_open", js_cpubin_open),
        FN("cpubin_parse", js_cpubin_parse),
        FN("cpubin_close", js_cpubin_close),
        FN("cpubin_summary", js_cpubin_summary),
        FN("cpubin_name", js_cpubin_name),
        FN("cpubin_tensor", js_cpubin_tensor),
        FN("cpubin_embed_row", js_cpubin_embed_row),
    };
    napi_define_properties(env, exports, sizeof props / sizeof props[0], props);
    return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, module_init)
