// g4attn.node: Node N-API addon over the C ABI of libg4attn.so (include/g4attn.h).
//
// A thin shim: device pointers and streams travel as BigInt, Params structs as
// the uniform bytes the engine already builds (makeUniformMixed,
// src/engine.ts:460-478), copied by value into the C struct after a size
// check. A non-zero status from the library becomes a thrown JS Error carrying
// g4_last_error(). Every call enqueues on the given stream and returns; only
// download() and streamSynchronize() wait.
#include <node_api.h>
#include <stdint.h>
#include <string.h>

#include <string>
#include <vector>

#include "g4attn.h"

namespace {

#define NAPI_OK(env, call)                                  \
    do {                                                    \
        if ((call) != napi_ok) {                            \
            napi_throw_error((env), nullptr, "N-API call failed: " #call); \
            return nullptr;                                 \
        }                                                   \
    } while (0)

napi_value throw_status(napi_env env, int status) {
    std::string msg = std::string("g4attn status ") + std::to_string(status) + ": " + g4_last_error();
    napi_throw_error(env, nullptr, msg.c_str());
    return nullptr;
}

struct Args {
    napi_env env;
    std::vector<napi_value> v;
    bool ok = true;

    Args(napi_env e, napi_callback_info info, size_t expect) : env(e), v(expect) {
        size_t n = expect;
        if (napi_get_cb_info(e, info, &n, v.data(), nullptr, nullptr) != napi_ok || n < expect) {
            napi_throw_type_error(e, nullptr, ("expected " + std::to_string(expect) + " arguments").c_str());
            ok = false;
        }
    }

    // Device pointer or stream: BigInt (or 0 / null for the null stream).
    void* ptr(size_t i) {
        if (!ok) return nullptr;
        napi_valuetype t;
        napi_typeof(env, v[i], &t);
        if (t == napi_null || t == napi_undefined) return nullptr;
        if (t == napi_number) {
            int64_t x = 0;
            napi_get_value_int64(env, v[i], &x);
            if (x != 0) fail("argument " + std::to_string(i) + ": pointers are BigInt");
            return nullptr;
        }
        uint64_t x = 0;
        bool lossless = false;
        if (napi_get_value_bigint_uint64(env, v[i], &x, &lossless) != napi_ok || !lossless) {
            fail("argument " + std::to_string(i) + ": expected a BigInt pointer");
            return nullptr;
        }
        return reinterpret_cast<void*>(static_cast<uintptr_t>(x));
    }
    uint32_t u32(size_t i) {
        uint32_t x = 0;
        if (ok && napi_get_value_uint32(env, v[i], &x) != napi_ok) fail("argument " + std::to_string(i) + ": expected a number");
        return x;
    }
    double f64(size_t i) {
        double x = 0;
        if (ok && napi_get_value_double(env, v[i], &x) != napi_ok) fail("argument " + std::to_string(i) + ": expected a number");
        return x;
    }
    // Bytes of a TypedArray / DataView / Buffer argument.
    bool bytes(size_t i, void** data, size_t* len) {
        if (!ok) return false;
        bool is_ta = false, is_dv = false;
        napi_is_typedarray(env, v[i], &is_ta);
        napi_is_dataview(env, v[i], &is_dv);
        if (is_ta) {
            napi_typedarray_type type;
            size_t n;
            napi_value ab;
            size_t off;
            napi_get_typedarray_info(env, v[i], &type, &n, data, &ab, &off);
            size_t elem = 1;
            switch (type) {
                case napi_int16_array: case napi_uint16_array: elem = 2; break;
                case napi_int32_array: case napi_uint32_array: case napi_float32_array: elem = 4; break;
                case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: elem = 8; break;
                default: elem = 1;
            }
            *len = n * elem;
            return true;
        }
        if (is_dv) {
            napi_value ab;
            size_t off;
            napi_get_dataview_info(env, v[i], len, data, &ab, &off);
            return true;
        }
        fail("argument " + std::to_string(i) + ": expected a TypedArray or DataView");
        return false;
    }
    // A Params struct from its uniform bytes (at least sizeof(T); the engine pads uniforms to 16).
    template <typename T>
    bool params(size_t i, T* out) {
        void* d = nullptr;
        size_t n = 0;
        if (!bytes(i, &d, &n)) return false;
        if (n < sizeof(T)) {
            fail("argument " + std::to_string(i) + ": params are " + std::to_string(n) + " bytes, need " +
                 std::to_string(sizeof(T)));
            return false;
        }
        memcpy(out, d, sizeof(T));
        return true;
    }
    void fail(const std::string& m) {
        if (ok) napi_throw_type_error(env, nullptr, m.c_str());
        ok = false;
    }
};

napi_value undefined(napi_env env) {
    napi_value u;
    napi_get_undefined(env, &u);
    return u;
}

napi_value bigint(napi_env env, void* p) {
    napi_value r;
    napi_create_bigint_uint64(env, static_cast<uint64_t>(reinterpret_cast<uintptr_t>(p)), &r);
    return r;
}

napi_value number(napi_env env, double x) {
    napi_value r;
    napi_create_double(env, x, &r);
    return r;
}

#define CALL(env, expr)                       \
    do {                                      \
        int st_ = (expr);                     \
        if (st_ != G4_OK) return throw_status((env), st_); \
    } while (0)

// ---- device, streams, memory ------------------------------------------------

napi_value Version(napi_env env, napi_callback_info) {
    napi_value r;
    napi_create_string_utf8(env, g4_version(), NAPI_AUTO_LENGTH, &r);
    return r;
}

napi_value DeviceCount(napi_env env, napi_callback_info) {
    int n = 0;
    CALL(env, g4_device_count(&n));
    return number(env, n);
}

napi_value SetDevice(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    const uint32_t d = a.u32(0);
    if (!a.ok) return nullptr;
    CALL(env, g4_set_device((int)d));
    return undefined(env);
}

napi_value StreamCreate(napi_env env, napi_callback_info) {
    void* s = nullptr;
    CALL(env, g4_stream_create(&s));
    return bigint(env, s);
}

napi_value StreamDestroy(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    void* s = a.ptr(0);
    if (!a.ok) return nullptr;
    CALL(env, g4_stream_destroy(s));
    return undefined(env);
}

napi_value StreamSynchronize(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    void* s = a.ptr(0);
    if (!a.ok) return nullptr;
    CALL(env, g4_stream_synchronize(s));
    return undefined(env);
}

napi_value Malloc(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    const double bytes = a.f64(0);
    if (!a.ok) return nullptr;
    if (bytes <= 0) {
        napi_throw_range_error(env, nullptr, "malloc: size must be positive");
        return nullptr;
    }
    void* p = nullptr;
    CALL(env, g4_malloc(&p, (size_t)bytes));
    return bigint(env, p);
}

napi_value Free(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    void* p = a.ptr(0);
    if (!a.ok) return nullptr;
    CALL(env, g4_free(p));
    return undefined(env);
}

// upload(dst, offset, data, stream): enqueues a copy of `data`'s bytes
// (hipMemcpyAsync; the HIP runtime stages pageable source memory before it
// returns, so `data` may be reused afterwards).
napi_value Upload(napi_env env, napi_callback_info info) {
    Args a(env, info, 4);
    void* dst = a.ptr(0);
    const double off = a.f64(1);
    void* d = nullptr;
    size_t n = 0;
    a.bytes(2, &d, &n);
    void* s = a.ptr(3);
    if (!a.ok) return nullptr;
    CALL(env, g4_upload(dst, (size_t)off, d, n, s));
    return undefined(env);
}

// download(src, offset, out, stream): copies into `out` and waits for it.
napi_value Download(napi_env env, napi_callback_info info) {
    Args a(env, info, 4);
    void* src = a.ptr(0);
    const double off = a.f64(1);
    void* d = nullptr;
    size_t n = 0;
    a.bytes(2, &d, &n);
    void* s = a.ptr(3);
    if (!a.ok) return nullptr;
    CALL(env, g4_download(d, src, (size_t)off, n, s));
    return undefined(env);
}

// readAsync(src, offset, out, stream) -> Promise<void>: mapAsync's shape. The
// copy is enqueued now, on the stream (ordered after what is already there,
// and before anything enqueued later); the wait and the copy into `out` run on
// a worker thread, and the promise settles on the JS thread. `out` is held by
// a reference until then.
struct ReadWork {
    napi_async_work work = nullptr;
    napi_deferred deferred = nullptr;
    napi_ref out_ref = nullptr;
    g4_readback* handle = nullptr;
    void* dst = nullptr;
    int status = G4_OK;
    std::string msg;
};

void read_execute(napi_env, void* data) {
    ReadWork* w = static_cast<ReadWork*>(data);
    w->status = g4_readback_finish(w->handle, w->dst);
    if (w->status != G4_OK) w->msg = g4_last_error();
}

void read_complete(napi_env env, napi_status st, void* data) {
    ReadWork* w = static_cast<ReadWork*>(data);
    if (st == napi_ok && w->status == G4_OK) {
        napi_value u;
        napi_get_undefined(env, &u);
        napi_resolve_deferred(env, w->deferred, u);
    } else {
        if (st != napi_ok && w->status == G4_OK) {  // cancelled before it ran: the handle is still open
            g4_readback_finish(w->handle, nullptr);
            w->msg = "readAsync: cancelled";
        }
        const std::string text = "g4attn status " + std::to_string(w->status) + ": " + w->msg;
        napi_value m, err;
        napi_create_string_utf8(env, text.c_str(), NAPI_AUTO_LENGTH, &m);
        napi_create_error(env, nullptr, m, &err);
        napi_reject_deferred(env, w->deferred, err);
    }
    napi_delete_reference(env, w->out_ref);
    napi_delete_async_work(env, w->work);
    delete w;
}

napi_value ReadAsync(napi_env env, napi_callback_info info) {
    Args a(env, info, 4);
    void* src = a.ptr(0);
    const double off = a.f64(1);
    void* d = nullptr;
    size_t n = 0;
    a.bytes(2, &d, &n);
    void* s = a.ptr(3);
    if (!a.ok) return nullptr;
    g4_readback* h = nullptr;
    CALL(env, g4_readback_begin(src, (size_t)off, n, s, &h));
    ReadWork* w = new ReadWork;
    w->handle = h;
    w->dst = d;
    napi_value promise, name;
    if (napi_create_reference(env, a.v[2], 1, &w->out_ref) != napi_ok ||
        napi_create_promise(env, &w->deferred, &promise) != napi_ok ||
        napi_create_string_utf8(env, "g4attn.readAsync", NAPI_AUTO_LENGTH, &name) != napi_ok ||
        napi_create_async_work(env, nullptr, name, read_execute, read_complete, w, &w->work) != napi_ok ||
        napi_queue_async_work(env, w->work) != napi_ok) {
        g4_readback_finish(h, nullptr);  // the copy finishes; nothing waits for it
        if (w->out_ref) napi_delete_reference(env, w->out_ref);
        if (w->work) napi_delete_async_work(env, w->work);
        delete w;
        napi_throw_error(env, nullptr, "readAsync: could not queue the wait");
        return nullptr;
    }
    return promise;
}

// ---- timestamp queries (the engine's GPUQuerySet, src/engine.ts:3089-3110, 3208-3227, 3253-3288) ----

napi_value QuerySetCreate(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    const uint32_t count = a.u32(0);
    if (!a.ok) return nullptr;
    g4_query_set* q = nullptr;
    CALL(env, g4_query_set_create(count, &q));
    return bigint(env, q);
}

// A pass's begin and end (beginPass .. pass.end()): the kernels launched from this thread in between
// carry the pair (slot, slot + 1).
napi_value QueryBeginPass(napi_env env, napi_callback_info info) {
    Args a(env, info, 2);
    void* q = a.ptr(0);
    const uint32_t slot = a.u32(1);
    if (!a.ok) return nullptr;
    CALL(env, g4_query_begin_pass(static_cast<g4_query_set*>(q), slot));
    return undefined(env);
}

napi_value QueryEndPass(napi_env env, napi_callback_info) {
    CALL(env, g4_query_end_pass());
    return undefined(env);
}

napi_value QueryWrite(napi_env env, napi_callback_info info) {
    Args a(env, info, 3);
    void* q = a.ptr(0);
    const uint32_t slot = a.u32(1);
    void* s = a.ptr(2);
    if (!a.ok) return nullptr;
    CALL(env, g4_query_write(static_cast<g4_query_set*>(q), slot, s));
    return undefined(env);
}

napi_value float64_array(napi_env env, const std::vector<double>& x) {
    void* data = nullptr;
    napi_value ab, arr;
    NAPI_OK(env, napi_create_arraybuffer(env, x.size() * sizeof(double), &data, &ab));
    if (!x.empty()) memcpy(data, x.data(), x.size() * sizeof(double));
    NAPI_OK(env, napi_create_typedarray(env, napi_float64_array, x.size(), ab, 0, &arr));
    return arr;
}

// resolveQuerySet + mapAsync as one blocking call: Float64Array of each pair's ns (NaN: not written).
napi_value QueryResolve(napi_env env, napi_callback_info info) {
    Args a(env, info, 3);
    void* q = a.ptr(0);
    const uint32_t first = a.u32(1), n = a.u32(2);
    if (!a.ok) return nullptr;
    std::vector<double> ns(n ? n : 1);
    CALL(env, g4_query_resolve(static_cast<g4_query_set*>(q), first, n, ns.data()));
    ns.resize(n);
    return float64_array(env, ns);
}

struct QueryWork {
    napi_async_work work = nullptr;
    napi_deferred deferred = nullptr;
    g4_query_set* set = nullptr;
    uint32_t first = 0, n = 0;
    std::vector<double> ns;
    int status = G4_OK;
    std::string msg;
};

void query_execute(napi_env, void* data) {
    QueryWork* w = static_cast<QueryWork*>(data);
    w->status = g4_query_resolve(w->set, w->first, w->n, w->ns.data());
    if (w->status != G4_OK) w->msg = g4_last_error();
}

void query_complete(napi_env env, napi_status st, void* data) {
    QueryWork* w = static_cast<QueryWork*>(data);
    if (st == napi_ok && w->status == G4_OK) {
        napi_value arr = float64_array(env, w->ns);
        if (arr) napi_resolve_deferred(env, w->deferred, arr);
    } else {
        if (st != napi_ok && w->status == G4_OK) w->msg = "queryResolveAsync: cancelled";
        const std::string text = "g4attn status " + std::to_string(w->status) + ": " + w->msg;
        napi_value m, err;
        napi_create_string_utf8(env, text.c_str(), NAPI_AUTO_LENGTH, &m);
        napi_create_error(env, nullptr, m, &err);
        napi_reject_deferred(env, w->deferred, err);
    }
    napi_delete_async_work(env, w->work);
    delete w;
}

// The same, waited for off the JS thread (mapAsync's promise). The set must stay alive, and its slots
// unwritten, until the promise settles.
napi_value QueryResolveAsync(napi_env env, napi_callback_info info) {
    Args a(env, info, 3);
    void* q = a.ptr(0);
    const uint32_t first = a.u32(1), n = a.u32(2);
    if (!a.ok) return nullptr;
    if (!q || n == 0) {
        napi_throw_range_error(env, nullptr, "queryResolveAsync: no set, or no slots");
        return nullptr;
    }
    QueryWork* w = new QueryWork;
    w->set = static_cast<g4_query_set*>(q);
    w->first = first;
    w->n = n;
    w->ns.assign(n, 0.0);
    napi_value promise, name;
    if (napi_create_promise(env, &w->deferred, &promise) != napi_ok ||
        napi_create_string_utf8(env, "g4attn.queryResolveAsync", NAPI_AUTO_LENGTH, &name) != napi_ok ||
        napi_create_async_work(env, nullptr, name, query_execute, query_complete, w, &w->work) != napi_ok ||
        napi_queue_async_work(env, w->work) != napi_ok) {
        if (w->work) napi_delete_async_work(env, w->work);
        delete w;
        napi_throw_error(env, nullptr, "queryResolveAsync: could not queue the wait");
        return nullptr;
    }
    return promise;
}

napi_value QuerySetDestroy(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    void* q = a.ptr(0);
    if (!a.ok) return nullptr;
    CALL(env, g4_query_set_destroy(static_cast<g4_query_set*>(q)));
    return undefined(env);
}

napi_value Zero(napi_env env, napi_callback_info info) {
    Args a(env, info, 3);
    void* p = a.ptr(0);
    const double n = a.f64(1);
    void* s = a.ptr(2);
    if (!a.ok) return nullptr;
    CALL(env, g4_zero(p, (size_t)n, s));
    return undefined(env);
}

// ---- the six reference kernels (bindings in WGSL @binding order) -----------

napi_value FusedPerHeadNormRope(napi_env env, napi_callback_info info) {
    Args a(env, info, 5);  // data, weight, rope_freqs, params, stream
    void* data = a.ptr(0);
    void* w = a.ptr(1);
    void* rf = a.ptr(2);
    g4_norm_rope_params p;
    a.params(3, &p);
    void* s = a.ptr(4);
    if (!a.ok) return nullptr;
    CALL(env, g4_fused_per_head_norm_rope((float*)data, (const uint16_t*)w, (const uint16_t*)rf, p, s));
    return undefined(env);
}

napi_value PerHeadRmsNormNoWeight(napi_env env, napi_callback_info info) {
    Args a(env, info, 3);  // data, params, stream
    void* data = a.ptr(0);
    g4_norm_params p;
    a.params(1, &p);
    void* s = a.ptr(2);
    if (!a.ok) return nullptr;
    CALL(env, g4_per_head_rms_norm_no_weight((float*)data, p, s));
    return undefined(env);
}

napi_value KvCacheStore(napi_env env, napi_callback_info info) {
    Args a(env, info, 6);  // k_in, v_in, k_cache, v_cache, params, stream
    void* k = a.ptr(0);
    void* v = a.ptr(1);
    void* kc = a.ptr(2);
    void* vc = a.ptr(3);
    g4_kv_store_params p;
    a.params(4, &p);
    void* s = a.ptr(5);
    if (!a.ok) return nullptr;
    CALL(env, g4_kv_cache_store((const float*)k, (const float*)v, (uint16_t*)kc, (uint16_t*)vc, p, s));
    return undefined(env);
}

napi_value AttnScore(napi_env env, napi_callback_info info) {
    Args a(env, info, 5);  // q, k_cache, scores, params, stream
    void* q = a.ptr(0);
    void* kc = a.ptr(1);
    void* sc = a.ptr(2);
    g4_attn_score_params p;
    a.params(3, &p);
    void* s = a.ptr(4);
    if (!a.ok) return nullptr;
    CALL(env, g4_attn_score((const float*)q, (const uint16_t*)kc, (float*)sc, p, s));
    return undefined(env);
}

napi_value Softmax(napi_env env, napi_callback_info info) {
    Args a(env, info, 3);  // scores, params, stream
    void* sc = a.ptr(0);
    g4_softmax_params p;
    a.params(1, &p);
    void* s = a.ptr(2);
    if (!a.ok) return nullptr;
    CALL(env, g4_softmax((float*)sc, p, s));
    return undefined(env);
}

napi_value AttnOutput(napi_env env, napi_callback_info info) {
    Args a(env, info, 5);  // probs, v_cache, output, params, stream
    void* pr = a.ptr(0);
    void* vc = a.ptr(1);
    void* o = a.ptr(2);
    g4_attn_output_params p;
    a.params(3, &p);
    void* s = a.ptr(4);
    if (!a.ok) return nullptr;
    CALL(env, g4_attn_output((const float*)pr, (const uint16_t*)vc, (float*)o, p, s));
    return undefined(env);
}

// ---- sampling head: lmHead, logitSoftcap, argmax ---------------------------

napi_value MatmulQuant(napi_env env, napi_callback_info info) {
    Args a(env, info, 5);  // input, weight, output, params {M, N}, stream
    void* x = a.ptr(0);
    void* w = a.ptr(1);
    void* o = a.ptr(2);
    g4_matmul_params p;
    a.params(3, &p);
    void* s = a.ptr(4);
    if (!a.ok) return nullptr;
    CALL(env, g4_matmul_quant_f16((const float*)x, (const uint16_t*)w, (float*)o, p, s));
    return undefined(env);
}

napi_value MatmulQ8(napi_env env, napi_callback_info info) {
    Args a(env, info, 6);  // input, qweight, qscale, output, params {M, N}, stream
    void* x = a.ptr(0);
    void* q = a.ptr(1);
    void* sc = a.ptr(2);
    void* o = a.ptr(3);
    g4_matmul_params p;
    a.params(4, &p);
    void* s = a.ptr(5);
    if (!a.ok) return nullptr;
    CALL(env, g4_matmul_q8((const float*)x, (const int8_t*)q, (const uint16_t*)sc, (float*)o, p, s));
    return undefined(env);
}

napi_value MatmulQ4K(napi_env env, napi_callback_info info) {
    Args a(env, info, 6);  // input, qweight, qmeta, output, params {M, N}, stream
    void* x = a.ptr(0);
    void* q = a.ptr(1);
    void* m = a.ptr(2);
    void* o = a.ptr(3);
    g4_matmul_params p;
    a.params(4, &p);
    void* s = a.ptr(5);
    if (!a.ok) return nullptr;
    CALL(env, g4_matmul_q4k((const float*)x, (const uint32_t*)q, (const uint16_t*)m, (float*)o, p, s));
    return undefined(env);
}

napi_value LogitSoftcap(napi_env env, napi_callback_info info) {
    Args a(env, info, 3);  // logits, params {size, cap}, stream
    void* l = a.ptr(0);
    g4_softcap_params p;
    a.params(1, &p);
    void* s = a.ptr(2);
    if (!a.ok) return nullptr;
    CALL(env, g4_logit_softcap((float*)l, p, s));
    return undefined(env);
}

struct ArgmaxUniform {  // argmax.wgsl:3 (var<uniform> size: u32)
    uint32_t size;
};

napi_value Argmax(napi_env env, napi_callback_info info) {
    Args a(env, info, 4);  // logits, result, params {size}, stream
    void* l = a.ptr(0);
    void* r = a.ptr(1);
    ArgmaxUniform p;
    a.params(2, &p);
    void* s = a.ptr(3);
    if (!a.ok) return nullptr;
    CALL(env, g4_argmax((const float*)l, (uint32_t*)r, p.size, s));
    return undefined(env);
}

napi_value LmHeadWorkspaceSize(napi_env env, napi_callback_info info) {
    Args a(env, info, 3);  // vocab, hidden, cap
    g4_lm_head_params p = {a.u32(0), a.u32(1), (float)a.f64(2)};
    if (!a.ok) return nullptr;
    size_t bytes = 0;
    CALL(env, g4_lm_head_workspace_size(p, &bytes));
    return number(env, (double)bytes);
}

napi_value LmHeadArgmax(napi_env env, napi_callback_info info) {
    Args a(env, info, 10);  // hidden, weight, logits (or null), result, workspace, workspaceBytes, vocab, hidden, cap, stream
    void* h = a.ptr(0);
    void* w = a.ptr(1);
    void* l = a.ptr(2);
    void* r = a.ptr(3);
    void* ws = a.ptr(4);
    const double ws_bytes = a.f64(5);
    g4_lm_head_params p = {a.u32(6), a.u32(7), (float)a.f64(8)};
    void* s = a.ptr(9);
    if (!a.ok) return nullptr;
    CALL(env, g4_lm_head_argmax((const float*)h, (const uint16_t*)w, (float*)l, (uint32_t*)r, ws, (size_t)ws_bytes, p,
                                s));
    return undefined(env);
}

// ---- RoPE tables and the one-launch step -----------------------------------

napi_value RopeInvFreq(napi_env env, napi_callback_info info) {
    Args a(env, info, 6);  // theta, head_dim, apply_divisor, rope_freqs, out, stream
    const double theta = a.f64(0);
    const uint32_t hd = a.u32(1), div = a.u32(2);
    void* rf = a.ptr(3);
    void* out = a.ptr(4);
    void* s = a.ptr(5);
    if (!a.ok) return nullptr;
    CALL(env, g4_rope_inv_freq((float)theta, hd, div, (const uint16_t*)rf, (float*)out, s));
    return undefined(env);
}

napi_value RopeInvFreqHost(napi_env env, napi_callback_info info) {
    Args a(env, info, 5);  // theta, head_dim, apply_divisor, rope_freqs bits (Uint16Array or null), out (Float32Array)
    const double theta = a.f64(0);
    const uint32_t hd = a.u32(1), div = a.u32(2);
    if (!a.ok) return nullptr;
    napi_valuetype t;
    napi_typeof(env, a.v[3], &t);
    void* rf = nullptr;
    size_t rf_len = 0;
    if (t != napi_null && t != napi_undefined && !a.bytes(3, &rf, &rf_len)) return nullptr;
    void* out = nullptr;
    size_t out_len = 0;
    if (!a.bytes(4, &out, &out_len)) return nullptr;
    if (out_len < (size_t)hd / 2 * 4 || (rf && rf_len < (size_t)hd / 2 * 2)) {
        a.fail("ropeInvFreqHost: tables shorter than head_dim/2 values");
        return nullptr;
    }
    CALL(env, g4_rope_inv_freq_host((float)theta, hd, div, (const uint16_t*)rf, (float*)out));
    return undefined(env);
}

napi_value AttnStepWorkspaceSize(napi_env env, napi_callback_info info) {
    Args a(env, info, 4);  // n_entries, num_q_heads, num_kv_heads, head_dim
    const uint32_t n = a.u32(0), nqh = a.u32(1), nkh = a.u32(2), hd = a.u32(3);
    if (!a.ok) return nullptr;
    size_t bytes = 0;
    CALL(env, g4_attn_step_workspace_size(n, nqh, nkh, hd, &bytes));
    return number(env, (double)bytes);
}

napi_value AttnStepLayersWorkspaceSize(napi_env env, napi_callback_info info) {
    Args a(env, info, 5);  // n_layers, entries_per_layer, num_q_heads, num_kv_heads, head_dim
    const uint32_t n = a.u32(0), e = a.u32(1), nqh = a.u32(2), nkh = a.u32(3), hd = a.u32(4);
    if (!a.ok) return nullptr;
    size_t bytes = 0;
    CALL(env, g4_attn_step_layers_workspace_size(n, e, nqh, nkh, hd, &bytes));
    return number(env, (double)bytes);
}

bool get_prop(napi_env env, napi_value obj, const char* key, napi_value* out) {
    bool has = false;
    napi_has_named_property(env, obj, key, &has);
    if (!has) return false;
    napi_get_named_property(env, obj, key, out);
    napi_valuetype t;
    napi_typeof(env, *out, &t);
    return t != napi_undefined && t != napi_null;
}

// ---- the projections either side of the block: attn.linearQKV / linearOut --

// An array of {weight, out (BigInt pointers), rows} as g4_linear_seg.
bool linear_segs(Args& a, napi_value arr, const char* who, std::vector<g4_linear_seg>* segs) {
    napi_env env = a.env;
    bool is_array = false;
    napi_is_array(env, arr, &is_array);
    if (!is_array) {
        a.fail(std::string(who) + ": segments must be an array");
        return false;
    }
    uint32_t count = 0;
    napi_get_array_length(env, arr, &count);
    segs->assign(count, g4_linear_seg{});
    for (uint32_t i = 0; i < count; i++) {
        napi_value obj, v;
        napi_get_element(env, arr, i, &obj);
        const std::string at = std::string(who) + ": segment " + std::to_string(i) + ": ";
        const void* ptrs[2] = {};
        const char* keys[2] = {"weight", "out"};
        for (int k = 0; k < 2; k++) {
            uint64_t p = 0;
            bool lossless = false;
            if (!get_prop(env, obj, keys[k], &v) || napi_get_value_bigint_uint64(env, v, &p, &lossless) != napi_ok ||
                !lossless) {
                a.fail(at + keys[k] + " must be a BigInt pointer");
                return false;
            }
            ptrs[k] = reinterpret_cast<const void*>(static_cast<uintptr_t>(p));
        }
        uint32_t rows = 0;
        if (!get_prop(env, obj, "rows", &v) || napi_get_value_uint32(env, v, &rows) != napi_ok) {
            a.fail(at + "rows must be a number");
            return false;
        }
        (*segs)[i] = g4_linear_seg{static_cast<const uint16_t*>(ptrs[0]), (float*)const_cast<void*>(ptrs[1]), rows};
    }
    return true;
}

// linear(input, n, segments[{weight, out, rows}], stream): up to four f16
// weight matrices [rows][n] that read the same f32 input of length n.
napi_value Linear(napi_env env, napi_callback_info info) {
    Args a(env, info, 4);
    void* x = a.ptr(0);
    const uint32_t n = a.u32(1);
    void* s = a.ptr(3);
    if (!a.ok) return nullptr;
    std::vector<g4_linear_seg> segs;
    if (!linear_segs(a, a.v[2], "linear", &segs)) return nullptr;
    CALL(env, g4_linear_f16((const float*)x, n, segs.data(), (uint32_t)segs.size(), s));
    return undefined(env);
}

// linearQuant(input, n, format, segments[{weight, meta, out, rows}], stream): format 1 = q8, 2 = q4k.
napi_value LinearQuant(napi_env env, napi_callback_info info) {
    Args a(env, info, 5);
    void* x = a.ptr(0);
    const uint32_t n = a.u32(1), format = a.u32(2);
    void* s = a.ptr(4);
    if (!a.ok) return nullptr;
    bool is_array = false;
    napi_is_array(env, a.v[3], &is_array);
    if (!is_array) {
        a.fail("linearQuant: segments must be an array");
        return nullptr;
    }
    uint32_t count = 0;
    napi_get_array_length(env, a.v[3], &count);
    std::vector<g4_linear_qseg> segs(count);
    for (uint32_t i = 0; i < count; i++) {
        napi_value obj, v;
        napi_get_element(env, a.v[3], i, &obj);
        const std::string at = "linearQuant: segment " + std::to_string(i) + ": ";
        const void* ptrs[3] = {};
        const char* keys[3] = {"weight", "meta", "out"};
        for (int k = 0; k < 3; k++) {
            uint64_t p = 0;
            bool lossless = false;
            if (!get_prop(env, obj, keys[k], &v) || napi_get_value_bigint_uint64(env, v, &p, &lossless) != napi_ok ||
                !lossless) {
                a.fail(at + keys[k] + " must be a BigInt pointer");
                return nullptr;
            }
            ptrs[k] = reinterpret_cast<const void*>(static_cast<uintptr_t>(p));
        }
        uint32_t rows = 0;
        if (!get_prop(env, obj, "rows", &v) || napi_get_value_uint32(env, v, &rows) != napi_ok) {
            a.fail(at + "rows must be a number");
            return nullptr;
        }
        segs[i] = g4_linear_qseg{ptrs[0], static_cast<const uint16_t*>(ptrs[1]), (float*)const_cast<void*>(ptrs[2]),
                                 rows};
    }
    CALL(env, g4_linear_quant((const float*)x, n, format, segs.data(), count, s));
    return undefined(env);
}

// linearQkvPrepWorkspaceSize(numQHeads, numKvHeads): bytes of the per-head arrival counters.
napi_value LinearQkvPrepWorkspaceSize(napi_env env, napi_callback_info info) {
    Args a(env, info, 2);
    const uint32_t nqh = a.u32(0), nkh = a.u32(1);
    if (!a.ok) return nullptr;
    size_t bytes = 0;
    CALL(env, g4_linear_qkv_prep_workspace_size(nqh, nkh, &bytes));
    napi_value r;
    NAPI_OK(env, napi_create_double(env, (double)bytes, &r));
    return r;
}

// linearQkvPrep(x, n, format, segments [{weight, meta (q8 / q4k), out, rows}], qWeight, kWeight, ropeFreqs,
// ropeInvFreq, kCache, vCache, params (g4_qkv_prep_params bytes), workspace, stream): g4_linear_qkv_prep;
// kWeight and the caches null on KV-consumer layers (one segment).
napi_value LinearQkvPrep(napi_env env, napi_callback_info info) {
    Args a(env, info, 13);
    void* x = a.ptr(0);
    const uint32_t n = a.u32(1), format = a.u32(2);
    void* qw = a.ptr(4);
    void* kw = a.ptr(5);
    void* rf = a.ptr(6);
    void* inv = a.ptr(7);
    void* kc = a.ptr(8);
    void* vc = a.ptr(9);
    g4_qkv_prep_params p;
    a.params(10, &p);
    void* ws = a.ptr(11);
    void* s = a.ptr(12);
    if (!a.ok) return nullptr;
    bool is_array = false;
    napi_is_array(env, a.v[3], &is_array);
    if (!is_array) {
        a.fail("linearQkvPrep: segments must be an array");
        return nullptr;
    }
    uint32_t count = 0;
    napi_get_array_length(env, a.v[3], &count);
    std::vector<g4_linear_qseg> segs(count);
    for (uint32_t i = 0; i < count; i++) {
        napi_value obj, v;
        napi_get_element(env, a.v[3], i, &obj);
        const std::string at = "linearQkvPrep: segment " + std::to_string(i) + ": ";
        const void* ptrs[3] = {};
        const char* keys[3] = {"weight", "meta", "out"};
        for (int k = 0; k < 3; k++) {
            uint64_t q = 0;
            bool lossless = false;
            if (!get_prop(env, obj, keys[k], &v)) {
                if (k == 1) continue;  // f16 weights have no meta
                a.fail(at + keys[k] + " must be a BigInt pointer");
                return nullptr;
            }
            if (napi_get_value_bigint_uint64(env, v, &q, &lossless) != napi_ok || !lossless) {
                a.fail(at + keys[k] + " must be a BigInt pointer");
                return nullptr;
            }
            ptrs[k] = reinterpret_cast<const void*>(static_cast<uintptr_t>(q));
        }
        uint32_t rows = 0;
        if (!get_prop(env, obj, "rows", &v) || napi_get_value_uint32(env, v, &rows) != napi_ok) {
            a.fail(at + "rows must be a number");
            return nullptr;
        }
        segs[i] = g4_linear_qseg{ptrs[0], static_cast<const uint16_t*>(ptrs[1]), (float*)const_cast<void*>(ptrs[2]),
                                 rows};
    }
    CALL(env, g4_linear_qkv_prep((const float*)x, n, format, segs.data(), count, (const uint16_t*)qw,
                                 (const uint16_t*)kw, (const uint16_t*)rf, (const float*)inv, (uint16_t*)kc,
                                 (uint16_t*)vc, p, ws, s));
    return undefined(env);
}

// One g4_step_entry from a JS object with the same field names in camelCase.
bool step_entry(Args& a, napi_value obj, size_t idx, uint32_t head_dim, g4_step_entry* e) {
    napi_env env = a.env;
    memset(e, 0, sizeof *e);
    struct {
        const char* key;
        const void** dst;
        bool required;
    } ptrs[] = {
        {"q", (const void**)&e->q, true},
        {"k", (const void**)&e->k, false},  // k, v, kWeight absent: the current row is already cached
        {"v", (const void**)&e->v, false},
        {"qWeight", (const void**)&e->q_weight, true},
        {"kWeight", (const void**)&e->k_weight, false},
        {"ropeFreqs", (const void**)&e->rope_freqs, false},
        {"kCache", (const void**)&e->k_cache, true},
        {"vCache", (const void**)&e->v_cache, true},
        {"out", (const void**)&e->out, true},
    };
    for (auto& p : ptrs) {
        napi_value v;
        if (!get_prop(env, obj, p.key, &v)) {
            if (p.required) {
                a.fail("entry " + std::to_string(idx) + ": missing " + p.key);
                return false;
            }
            continue;
        }
        uint64_t x = 0;
        bool lossless = false;
        if (napi_get_value_bigint_uint64(env, v, &x, &lossless) != napi_ok || !lossless) {
            a.fail("entry " + std::to_string(idx) + ": " + p.key + " must be a BigInt pointer");
            return false;
        }
        *p.dst = reinterpret_cast<const void*>(static_cast<uintptr_t>(x));
    }
    {  // the host RoPE inverse-frequency table: a Float32Array of head_dim/2 values, read during prepare
        napi_value v;
        if (get_prop(env, obj, "ropeInvFreq", &v)) {
            bool is_ta = false;
            napi_is_typedarray(env, v, &is_ta);
            napi_typedarray_type type = napi_int8_array;
            size_t n = 0, off = 0;
            void* data = nullptr;
            napi_value ab;
            if (is_ta) napi_get_typedarray_info(env, v, &type, &n, &data, &ab, &off);
            if (!is_ta || type != napi_float32_array || n < head_dim / 2) {
                a.fail("entry " + std::to_string(idx) + ": ropeInvFreq must be a Float32Array of head_dim/2 values");
                return false;
            }
            e->rope_inv_freq_host = static_cast<const float*>(data);
        }
    }
    struct {
        const char* key;
        uint32_t* dst;
        uint32_t dflt;
        bool required;
    } u32s[] = {
        {"seqLen", &e->seq_len, 0, true},
        {"position", &e->position, 0, true},
        {"slidingWindow", &e->sliding_window, 0, false},
        {"storeKv", &e->store_kv, 1, false},
        {"applyDivisor", &e->apply_divisor, 0, false},
        {"qReady", &e->q_ready, 0, false},
    };
    for (auto& f : u32s) {
        napi_value v;
        *f.dst = f.dflt;
        if (!get_prop(env, obj, f.key, &v)) {
            if (f.required) {
                a.fail("entry " + std::to_string(idx) + ": missing " + f.key);
                return false;
            }
            continue;
        }
        napi_valuetype t;
        napi_typeof(env, v, &t);
        if (t == napi_boolean) {
            bool b = false;
            napi_get_value_bool(env, v, &b);
            *f.dst = b ? 1u : 0u;
        } else if (napi_get_value_uint32(env, v, f.dst) != napi_ok) {
            a.fail("entry " + std::to_string(idx) + ": " + f.key + " must be a number");
            return false;
        }
    }
    struct {
        const char* key;
        float* dst;
        float dflt;
        bool required;
    } f32s[] = {
        {"theta", &e->theta, 0.0f, true},
        {"scale", &e->scale, 1.0f, false},
        {"eps", &e->eps, 1e-6f, false},
    };
    for (auto& f : f32s) {
        napi_value v;
        *f.dst = f.dflt;
        if (!get_prop(env, obj, f.key, &v)) {
            if (f.required) {
                a.fail("entry " + std::to_string(idx) + ": missing " + f.key);
                return false;
            }
            continue;
        }
        double x = 0;
        if (napi_get_value_double(env, v, &x) != napi_ok) {
            a.fail("entry " + std::to_string(idx) + ": " + f.key + " must be a number");
            return false;
        }
        *f.dst = (float)x;
    }
    return true;
}

// attnStepPrepare(entries[], nqh, nkh, hd, workspace, workspaceBytes, stream) -> plan (Uint8Array)
napi_value AttnStepPrepare(napi_env env, napi_callback_info info) {
    Args a(env, info, 7);
    if (!a.ok) return nullptr;
    bool is_array = false;
    napi_is_array(env, a.v[0], &is_array);
    if (!is_array) {
        napi_throw_type_error(env, nullptr, "attnStepPrepare: entries must be an array");
        return nullptr;
    }
    uint32_t n = 0;
    napi_get_array_length(env, a.v[0], &n);
    const uint32_t nqh = a.u32(1), nkh = a.u32(2), hd = a.u32(3);
    if (!a.ok) return nullptr;
    std::vector<g4_step_entry> ents(n);
    for (uint32_t i = 0; i < n; i++) {
        napi_value obj;
        napi_get_element(env, a.v[0], i, &obj);
        if (!step_entry(a, obj, i, hd, &ents[i])) return nullptr;
    }
    void* ws = a.ptr(4);
    const double ws_bytes = a.f64(5);
    void* s = a.ptr(6);
    if (!a.ok) return nullptr;
    napi_value ab, plan;
    void* pdata = nullptr;
    NAPI_OK(env, napi_create_arraybuffer(env, sizeof(g4_decode_plan), &pdata, &ab));
    CALL(env, g4_attn_step_prepare(ents.data(), n, nqh, nkh, hd, ws, (size_t)ws_bytes,
                                   static_cast<g4_decode_plan*>(pdata), s));
    NAPI_OK(env, napi_create_typedarray(env, napi_uint8_array, sizeof(g4_decode_plan), ab, 0, &plan));
    return plan;
}

// attnStepPrepareLayers(entries[], entriesPerLayer, nqh, nkh, hd, workspace, workspaceBytes, stream) -> plan
// per layer (an array of Uint8Arrays over one ArrayBuffer); layer i is entries[i * entriesPerLayer ..).
napi_value AttnStepPrepareLayers(napi_env env, napi_callback_info info) {
    Args a(env, info, 8);
    if (!a.ok) return nullptr;
    bool is_array = false;
    napi_is_array(env, a.v[0], &is_array);
    if (!is_array) {
        napi_throw_type_error(env, nullptr, "attnStepPrepareLayers: entries must be an array");
        return nullptr;
    }
    uint32_t n = 0;
    napi_get_array_length(env, a.v[0], &n);
    const uint32_t per = a.u32(1), nqh = a.u32(2), nkh = a.u32(3), hd = a.u32(4);
    if (!a.ok) return nullptr;
    if (per == 0 || n % per) {
        napi_throw_range_error(env, nullptr, "attnStepPrepareLayers: entries are not whole layers");
        return nullptr;
    }
    std::vector<g4_step_entry> ents(n);
    for (uint32_t i = 0; i < n; i++) {
        napi_value obj;
        napi_get_element(env, a.v[0], i, &obj);
        if (!step_entry(a, obj, i, hd, &ents[i])) return nullptr;
    }
    void* ws = a.ptr(5);
    const double ws_bytes = a.f64(6);
    void* s = a.ptr(7);
    if (!a.ok) return nullptr;
    const uint32_t nl = n / per;
    napi_value ab, list;
    void* pdata = nullptr;
    NAPI_OK(env, napi_create_arraybuffer(env, (size_t)nl * sizeof(g4_decode_plan), &pdata, &ab));
    CALL(env, g4_attn_step_prepare_layers(ents.data(), nl, per, nqh, nkh, hd, ws, (size_t)ws_bytes,
                                          static_cast<g4_decode_plan*>(pdata), s));
    NAPI_OK(env, napi_create_array_with_length(env, nl, &list));
    for (uint32_t i = 0; i < nl; i++) {
        napi_value plan;
        NAPI_OK(env, napi_create_typedarray(env, napi_uint8_array, sizeof(g4_decode_plan), ab,
                                            (size_t)i * sizeof(g4_decode_plan), &plan));
        NAPI_OK(env, napi_set_element(env, list, i, plan));
    }
    return list;
}

napi_value AttnStepRun(napi_env env, napi_callback_info info) {
    Args a(env, info, 2);  // plan, stream
    void* d = nullptr;
    size_t n = 0;
    a.bytes(0, &d, &n);
    void* s = a.ptr(1);
    if (!a.ok) return nullptr;
    if (n != sizeof(g4_decode_plan)) {
        napi_throw_type_error(env, nullptr, "attnStepRun: not a plan from attnStepPrepare");
        return nullptr;
    }
    g4_decode_plan plan;
    memcpy(&plan, d, sizeof plan);
    CALL(env, g4_attn_step_run(&plan, s));
    return undefined(env);
}

// attnStepRunPair(plan1, plan2, stream): a token's head_dim-512 and head_dim-256 plans (either order) as one
// attention launch and one merge launch (g4_attn_step_run_pair).
napi_value AttnStepRunPair(napi_env env, napi_callback_info info) {
    Args a(env, info, 3);  // plan1, plan2, stream
    void* d1 = nullptr;
    void* d2 = nullptr;
    size_t n1 = 0, n2 = 0;
    a.bytes(0, &d1, &n1);
    a.bytes(1, &d2, &n2);
    void* s = a.ptr(2);
    if (!a.ok) return nullptr;
    if (n1 != sizeof(g4_decode_plan) || n2 != sizeof(g4_decode_plan)) {
        napi_throw_type_error(env, nullptr, "attnStepRunPair: not plans from attnStepPrepare");
        return nullptr;
    }
    g4_decode_plan p1, p2;
    memcpy(&p1, d1, sizeof p1);
    memcpy(&p2, d2, sizeof p2);
    CALL(env, g4_attn_step_run_pair(&p1, &p2, s));
    return undefined(env);
}

// attnStepAdvance(plan, tokens): the prepared plan moves `tokens` decode steps ahead, in place (the
// 64-byte array from attnStepPrepare / attnStepPrepareLayers); host only, nothing is enqueued.
napi_value AttnStepAdvance(napi_env env, napi_callback_info info) {
    Args a(env, info, 2);  // plan, tokens
    void* d = nullptr;
    size_t n = 0;
    a.bytes(0, &d, &n);
    const uint32_t tokens = a.u32(1);
    if (!a.ok) return nullptr;
    if (n != sizeof(g4_decode_plan)) {
        napi_throw_type_error(env, nullptr, "attnStepAdvance: not a plan from attnStepPrepare");
        return nullptr;
    }
    CALL(env, g4_attn_step_advance(static_cast<g4_decode_plan*>(d), tokens));
    return undefined(env);
}

// The plan argument of the step's run calls (a 64-byte array from attnStepPrepare).
bool step_plan_arg(Args& a, size_t i, const char* who, g4_decode_plan* plan) {
    void* d = nullptr;
    size_t n = 0;
    a.bytes(i, &d, &n);
    if (!a.ok) return false;
    if (n != sizeof(g4_decode_plan)) {
        a.fail(std::string(who) + ": not a plan from attnStepPrepare");
        return false;
    }
    memcpy(plan, d, sizeof *plan);
    return true;
}

napi_value AttnStepRunAttention(napi_env env, napi_callback_info info) {
    Args a(env, info, 2);  // plan, stream
    g4_decode_plan plan;
    if (!step_plan_arg(a, 0, "attnStepRunAttention", &plan)) return nullptr;
    void* s = a.ptr(1);
    if (!a.ok) return nullptr;
    CALL(env, g4_attn_step_run_attention(&plan, s));
    return undefined(env);
}

// attnStepRunOut(plan, segments[{weight, out, rows}], stream): attn.linearOut of every entry with the
// step's merge folded in.
napi_value AttnStepRunOut(napi_env env, napi_callback_info info) {
    Args a(env, info, 3);
    g4_decode_plan plan;
    if (!step_plan_arg(a, 0, "attnStepRunOut", &plan)) return nullptr;
    void* s = a.ptr(2);
    if (!a.ok) return nullptr;
    std::vector<g4_linear_seg> segs;
    if (!linear_segs(a, a.v[1], "attnStepRunOut", &segs)) return nullptr;
    CALL(env, g4_attn_step_run_out(&plan, segs.data(), (uint32_t)segs.size(), s));
    return undefined(env);
}

// ---- causal prefill ---------------------------------------------------------

// One g4_prefill_entry from {q, kCache, vCache, out (BigInt pointers), nTokens, start, slidingWindow, scale,
// and optionally vtCache (BigInt) with vtRows}.
bool prefill_entry(Args& a, napi_value obj, size_t idx, g4_prefill_entry* e) {
    napi_env env = a.env;
    memset(e, 0, sizeof *e);
    const std::string at = "prefill entry " + std::to_string(idx) + ": ";
    struct {
        const char* key;
        const void** dst;
    } ptrs[] = {{"q", (const void**)&e->q}, {"kCache", (const void**)&e->k_cache},
                {"vCache", (const void**)&e->v_cache}, {"out", (const void**)&e->out}};
    for (auto& p : ptrs) {
        napi_value v;
        uint64_t x = 0;
        bool lossless = false;
        if (!get_prop(env, obj, p.key, &v) || napi_get_value_bigint_uint64(env, v, &x, &lossless) != napi_ok ||
            !lossless) {
            a.fail(at + p.key + " must be a BigInt pointer");
            return false;
        }
        *p.dst = reinterpret_cast<const void*>(static_cast<uintptr_t>(x));
    }
    struct {
        const char* key;
        uint32_t* dst;
        bool required;
    } u32s[] = {{"nTokens", &e->n_tokens, true}, {"start", &e->start, true}, {"slidingWindow", &e->sliding_window, false},
                {"vtRows", &e->vt_rows, false}};
    for (auto& f : u32s) {
        napi_value v;
        if (!get_prop(env, obj, f.key, &v)) {
            if (f.required) {
                a.fail(at + "missing " + f.key);
                return false;
            }
            continue;
        }
        if (napi_get_value_uint32(env, v, f.dst) != napi_ok) {
            a.fail(at + f.key + " must be a number");
            return false;
        }
    }
    e->scale = 1.0f;
    napi_value v;
    if (get_prop(env, obj, "vtCache", &v)) {  // optional: the V^T blocks the prompt prep wrote
        uint64_t x = 0;
        bool lossless = false;
        if (napi_get_value_bigint_uint64(env, v, &x, &lossless) != napi_ok || !lossless) {
            a.fail(at + "vtCache must be a BigInt pointer");
            return false;
        }
        e->vt_cache = reinterpret_cast<const uint16_t*>(static_cast<uintptr_t>(x));
    }
    if (get_prop(env, obj, "scale", &v)) {
        double x = 0;
        if (napi_get_value_double(env, v, &x) != napi_ok) {
            a.fail(at + "scale must be a number");
            return false;
        }
        e->scale = (float)x;
    }
    return true;
}

bool prefill_entries(Args& a, size_t arg, std::vector<g4_prefill_entry>* ents) {
    bool is_array = false;
    napi_is_array(a.env, a.v[arg], &is_array);
    if (!is_array) {
        a.fail("prefill: entries must be an array");
        return false;
    }
    uint32_t n = 0;
    napi_get_array_length(a.env, a.v[arg], &n);
    ents->resize(n);
    for (uint32_t i = 0; i < n; i++) {
        napi_value obj;
        napi_get_element(a.env, a.v[arg], i, &obj);
        if (!prefill_entry(a, obj, i, &(*ents)[i])) return false;
    }
    return true;
}

// attnPrefillWorkspaceSize(entries[], nqh, nkh, hd) -> bytes
napi_value AttnPrefillWorkspaceSize(napi_env env, napi_callback_info info) {
    Args a(env, info, 4);
    std::vector<g4_prefill_entry> ents;
    if (!a.ok || !prefill_entries(a, 0, &ents)) return nullptr;
    const uint32_t nqh = a.u32(1), nkh = a.u32(2), hd = a.u32(3);
    if (!a.ok) return nullptr;
    size_t bytes = 0;
    CALL(env, g4_attn_prefill_workspace_size(ents.data(), (uint32_t)ents.size(), nqh, nkh, hd, &bytes));
    return number(env, (double)bytes);
}

// attnPrefillPrepare(entries[], nqh, nkh, hd, workspace, workspaceBytes, stream) -> plan (Uint8Array)
napi_value AttnPrefillPrepare(napi_env env, napi_callback_info info) {
    Args a(env, info, 7);
    std::vector<g4_prefill_entry> ents;
    if (!a.ok || !prefill_entries(a, 0, &ents)) return nullptr;
    const uint32_t nqh = a.u32(1), nkh = a.u32(2), hd = a.u32(3);
    void* ws = a.ptr(4);
    const double ws_bytes = a.f64(5);
    void* s = a.ptr(6);
    if (!a.ok) return nullptr;
    napi_value ab, plan;
    void* pdata = nullptr;
    NAPI_OK(env, napi_create_arraybuffer(env, sizeof(g4_decode_plan), &pdata, &ab));
    CALL(env, g4_attn_prefill_prepare(ents.data(), (uint32_t)ents.size(), nqh, nkh, hd, ws, (size_t)ws_bytes,
                                      static_cast<g4_decode_plan*>(pdata), s));
    NAPI_OK(env, napi_create_typedarray(env, napi_uint8_array, sizeof(g4_decode_plan), ab, 0, &plan));
    return plan;
}

napi_value AttnPrefillRun(napi_env env, napi_callback_info info) {
    Args a(env, info, 2);  // plan, stream
    void* d = nullptr;
    size_t n = 0;
    a.bytes(0, &d, &n);
    void* s = a.ptr(1);
    if (!a.ok) return nullptr;
    if (n != sizeof(g4_decode_plan)) {
        napi_throw_type_error(env, nullptr, "attnPrefillRun: not a plan from attnPrefillPrepare");
        return nullptr;
    }
    g4_decode_plan plan;
    memcpy(&plan, d, sizeof plan);
    CALL(env, g4_attn_prefill_run(&plan, s));
    return undefined(env);
}

// ---- chunked prompt prep -------------------------------------------------------

// attnPromptPrep(q, k, v, qWeight, kWeight, ropeFreqs, ropeInvFreq, qOut, kCache, vCache, params
// (g4_prompt_prep_params bytes), stream); k, v, kWeight, kCache, vCache null on KV-consumer layers,
// ropeInvFreq null or the layer's device table from ropeInvFreq.
napi_value AttnPromptPrep(napi_env env, napi_callback_info info) {
    Args a(env, info, 12);
    void* q = a.ptr(0);
    void* k = a.ptr(1);
    void* v = a.ptr(2);
    void* qw = a.ptr(3);
    void* kw = a.ptr(4);
    void* rf = a.ptr(5);
    void* inv = a.ptr(6);
    void* qo = a.ptr(7);
    void* kc = a.ptr(8);
    void* vc = a.ptr(9);
    g4_prompt_prep_params p;
    a.params(10, &p);
    void* s = a.ptr(11);
    if (!a.ok) return nullptr;
    CALL(env, g4_attn_prompt_prep((const float*)q, (const float*)k, (const float*)v, (const uint16_t*)qw,
                                  (const uint16_t*)kw, (const uint16_t*)rf, (const float*)inv, (uint16_t*)qo,
                                  (uint16_t*)kc, (uint16_t*)vc, p, s));
    return undefined(env);
}

// attnPromptPrepVt(q, k, v, qWeight, kWeight, ropeFreqs, ropeInvFreq, qOut, kCache, vCache, vtCache, params,
// stream): attnPromptPrep that also writes the V rows as V^T blocks (g4_attn_prompt_prep_vt).
napi_value AttnPromptPrepVt(napi_env env, napi_callback_info info) {
    Args a(env, info, 13);
    void* q = a.ptr(0);
    void* k = a.ptr(1);
    void* v = a.ptr(2);
    void* qw = a.ptr(3);
    void* kw = a.ptr(4);
    void* rf = a.ptr(5);
    void* inv = a.ptr(6);
    void* qo = a.ptr(7);
    void* kc = a.ptr(8);
    void* vc = a.ptr(9);
    void* vt = a.ptr(10);
    g4_prompt_prep_params p;
    a.params(11, &p);
    void* s = a.ptr(12);
    if (!a.ok) return nullptr;
    CALL(env, g4_attn_prompt_prep_vt((const float*)q, (const float*)k, (const float*)v, (const uint16_t*)qw,
                                     (const uint16_t*)kw, (const uint16_t*)rf, (const float*)inv, (uint16_t*)qo,
                                     (uint16_t*)kc, (uint16_t*)vc, (uint16_t*)vt, p, s));
    return undefined(env);
}

// attnPromptPrepMany(entries (n g4_prompt_prep_entry records as bytes), n, stream): several chunks' preps
// in one launch (g4_attn_prompt_prep_many).
napi_value AttnPromptPrepMany(napi_env env, napi_callback_info info) {
    Args a(env, info, 3);
    void* d = nullptr;
    size_t bytes = 0;
    a.bytes(0, &d, &bytes);
    const uint32_t n = a.u32(1);
    void* s = a.ptr(2);
    if (!a.ok) return nullptr;
    if (n == 0 || bytes != (size_t)n * sizeof(g4_prompt_prep_entry)) {
        napi_throw_type_error(env, nullptr, "attnPromptPrepMany: entries must hold n g4_prompt_prep_entry records");
        return nullptr;
    }
    std::vector<g4_prompt_prep_entry> ents(n);
    memcpy(ents.data(), d, bytes);
    CALL(env, g4_attn_prompt_prep_many(ents.data(), n, s));
    return undefined(env);
}

napi_value SizeofPromptPrepEntry(napi_env env, napi_callback_info) {
    return number(env, (double)sizeof(g4_prompt_prep_entry));
}

napi_value Init(napi_env env, napi_value exports) {
    struct {
        const char* name;
        napi_callback cb;
    } fns[] = {
        {"version", Version},
        {"deviceCount", DeviceCount},
        {"setDevice", SetDevice},
        {"streamCreate", StreamCreate},
        {"streamDestroy", StreamDestroy},
        {"streamSynchronize", StreamSynchronize},
        {"malloc", Malloc},
        {"free", Free},
        {"upload", Upload},
        {"download", Download},
        {"readAsync", ReadAsync},
        {"querySetCreate", QuerySetCreate},
        {"queryBeginPass", QueryBeginPass},
        {"queryEndPass", QueryEndPass},
        {"queryWrite", QueryWrite},
        {"queryResolve", QueryResolve},
        {"queryResolveAsync", QueryResolveAsync},
        {"querySetDestroy", QuerySetDestroy},
        {"zero", Zero},
        {"fusedPerHeadNormRope", FusedPerHeadNormRope},
        {"perHeadRmsNormNoWeight", PerHeadRmsNormNoWeight},
        {"kvCacheStore", KvCacheStore},
        {"attnScore", AttnScore},
        {"softmax", Softmax},
        {"attnOutput", AttnOutput},
        {"matmulQuant", MatmulQuant},
        {"logitSoftcap", LogitSoftcap},
        {"argmax", Argmax},
        {"lmHeadWorkspaceSize", LmHeadWorkspaceSize},
        {"lmHeadArgmax", LmHeadArgmax},
        {"linear", Linear},
        {"linearQuant", LinearQuant},
        {"linearQkvPrepWorkspaceSize", LinearQkvPrepWorkspaceSize},
        {"linearQkvPrep", LinearQkvPrep},
        {"matmulQ8", MatmulQ8},
        {"matmulQ4K", MatmulQ4K},
        {"ropeInvFreq", RopeInvFreq},
        {"ropeInvFreqHost", RopeInvFreqHost},
        {"attnStepWorkspaceSize", AttnStepWorkspaceSize},
        {"attnStepPrepare", AttnStepPrepare},
        {"attnStepLayersWorkspaceSize", AttnStepLayersWorkspaceSize},
        {"attnStepPrepareLayers", AttnStepPrepareLayers},
        {"attnStepRun", AttnStepRun},
        {"attnStepRunPair", AttnStepRunPair},
        {"attnStepAdvance", AttnStepAdvance},
        {"attnStepRunAttention", AttnStepRunAttention},
        {"attnStepRunOut", AttnStepRunOut},
        {"attnPrefillWorkspaceSize", AttnPrefillWorkspaceSize},
        {"attnPrefillPrepare", AttnPrefillPrepare},
        {"attnPrefillRun", AttnPrefillRun},
        {"attnPromptPrep", AttnPromptPrep},
        {"attnPromptPrepMany", AttnPromptPrepMany},
        {"sizeofPromptPrepEntry", SizeofPromptPrepEntry},
        {"attnPromptPrepVt", AttnPromptPrepVt},
    };
    for (auto& f : fns) {
        napi_value fn;
        NAPI_OK(env, napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &fn));
        NAPI_OK(env, napi_set_named_property(env, exports, f.name, fn));
    }
    // Struct sizes, for callers that check them against their own layouts.
    struct {
        const char* name;
        size_t size;
    } sizes[] = {
        {"sizeofNormRopeParams", sizeof(g4_norm_rope_params)},
        {"sizeofNormParams", sizeof(g4_norm_params)},
        {"sizeofKvStoreParams", sizeof(g4_kv_store_params)},
        {"sizeofAttnScoreParams", sizeof(g4_attn_score_params)},
        {"sizeofSoftmaxParams", sizeof(g4_softmax_params)},
        {"sizeofAttnOutputParams", sizeof(g4_attn_output_params)},
        {"sizeofMatmulParams", sizeof(g4_matmul_params)},
        {"sizeofSoftcapParams", sizeof(g4_softcap_params)},
        {"sizeofArgmaxParams", sizeof(ArgmaxUniform)},
        {"sizeofQkvPrepParams", sizeof(g4_qkv_prep_params)},
    };
    for (auto& s : sizes) NAPI_OK(env, napi_set_named_property(env, exports, s.name, number(env, (double)s.size)));
    return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
