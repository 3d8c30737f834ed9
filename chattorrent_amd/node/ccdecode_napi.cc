// N-API binding of the ccdecode C ABI (include/ccdecode.h) for the Node.js
// host: the JS Runner shim (runner.js) drives the MI355X pass through it the
// way the reference's Runner drives its WebGPU pass (web/model/stage.js).
//
// Targets N-API version 8. cc_step runs on a worker thread (napi_async_work)
// and settles a Promise, as the reference's pass settles on mapAsync
// (web/model/stage.js:1447-1449); every other call is synchronous. A context
// takes one step at a time: a second step while one is in flight is refused.
#define NAPI_VERSION 8
#include <node_api.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "ccdecode.h"

namespace {

struct Ctx {
    cc_ctx* ctx = nullptr;
    bool busy = false;       // a step runs on a worker thread
    bool orphan = false;     // finalized during a step: the step's completion frees it
    int32_t hidden = 0, vocab = 0;
};

#define NAPI_OK(call)                                         \
    do {                                                      \
        if ((call) != napi_ok) {                              \
            napi_throw_error(env, nullptr, "N-API call failed: " #call); \
            return nullptr;                                   \
        }                                                     \
    } while (0)

napi_value undef(napi_env env) {
    napi_value u;
    napi_get_undefined(env, &u);
    return u;
}

void throw_status(napi_env env, int st, const std::string& msg) {
    napi_value m, e, c;
    napi_create_string_utf8(env, msg.c_str(), msg.size(), &m);
    napi_create_error(env, nullptr, m, &e);
    napi_create_int32(env, st, &c);
    napi_set_named_property(env, e, "status", c);
    napi_throw(env, e);
}

bool get_prop(napi_env env, napi_value obj, const char* name, napi_value* out) {
    bool has = false;
    if (napi_has_named_property(env, obj, name, &has) != napi_ok || !has) return false;
    if (napi_get_named_property(env, obj, name, out) != napi_ok) return false;
    napi_valuetype t;
    napi_typeof(env, *out, &t);
    return t != napi_undefined && t != napi_null;
}

double num(napi_env env, napi_value obj, const char* name, double dflt) {
    napi_value v;
    if (!get_prop(env, obj, name, &v)) return dflt;
    double d = dflt;
    napi_get_value_double(env, v, &d);
    return d;
}

// A flag given as a boolean or a number.
bool flag(napi_env env, napi_value obj, const char* name) {
    napi_value v;
    if (!get_prop(env, obj, name, &v)) return false;
    napi_valuetype t;
    napi_typeof(env, v, &t);
    if (t == napi_boolean) {
        bool b = false;
        napi_get_value_bool(env, v, &b);
        return b;
    }
    double d = 0;
    napi_get_value_double(env, v, &d);
    return d != 0;
}

Ctx* unwrap(napi_env env, napi_value v) {
    void* p = nullptr;
    if (napi_get_value_external(env, v, &p) != napi_ok || !p) {
        napi_throw_type_error(env, nullptr, "not a ccdecode context");
        return nullptr;
    }
    Ctx* c = (Ctx*)p;
    if (!c->ctx) {
        napi_throw_error(env, nullptr, "the context was destroyed");
        return nullptr;
    }
    return c;
}

// A context that is not running a step: every call but step() and
// destroy() goes through here, so none races the worker thread's cc_step.
Ctx* idle(napi_env env, napi_value v, const char* what) {
    Ctx* c = unwrap(env, v);
    if (c && c->busy) {
        throw_status(env, CC_EARG, std::string(what) + "() while a step is running on this context");
        return nullptr;
    }
    return c;
}

void destroy_ctx(Ctx* c) {
    if (c->ctx) cc_destroy(c->ctx);
    c->ctx = nullptr;
    delete c;
}

// A running step holds a reference to its context's external, so this runs
// during a step only when the environment itself goes away; the step's
// completion then frees the context.
void finalize_ctx(napi_env, void* data, void*) {
    Ctx* c = (Ctx*)data;
    if (c->busy) c->orphan = true;
    else destroy_ctx(c);
}

// Typed-array contents (pointer, element count, type).
bool typed(napi_env env, napi_value v, void** data, size_t* len, napi_typedarray_type* type) {
    bool is = false;
    napi_is_typedarray(env, v, &is);
    if (!is) return false;
    napi_value ab;
    size_t off;
    return napi_get_typedarray_info(env, v, type, len, data, &ab, &off) == napi_ok;
}

// create(dims, opts) -> context. dims: hidden, n_layer, n_heads, n_kv_heads,
// head_dim, ffn, vocab, rms_eps, rope_theta, rope_scaling {factor,
// low_freq_factor, high_freq_factor, original_max_position_embeddings}, tied.
napi_value Create(napi_env env, napi_callback_info info) {
    size_t argc = 2;
    napi_value argv[2];
    NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
    if (argc < 2) {
        napi_throw_type_error(env, nullptr, "create(dims, opts)");
        return nullptr;
    }
    cc_dims d{};
    d.hidden = (int32_t)num(env, argv[0], "hidden", 0);
    d.n_layer = (int32_t)num(env, argv[0], "n_layer", 0);
    d.n_heads = (int32_t)num(env, argv[0], "n_heads", 0);
    d.n_kv_heads = (int32_t)num(env, argv[0], "n_kv_heads", 0);
    d.head_dim = (int32_t)num(env, argv[0], "head_dim", 0);
    d.ffn = (int32_t)num(env, argv[0], "ffn", 0);
    d.vocab = (int32_t)num(env, argv[0], "vocab", 0);
    d.q8_group = (int32_t)num(env, argv[0], "group_q8", 32);
    d.rms_eps = (float)num(env, argv[0], "rms_eps", 1e-5);
    d.rope_theta = num(env, argv[0], "rope_theta", 10000.0);
    d.tied = num(env, argv[0], "tied", 1) != 0;
    {
        napi_value tv;   // a boolean `tied` too
        napi_valuetype t = napi_undefined;
        if (get_prop(env, argv[0], "tied", &tv)) napi_typeof(env, tv, &t);
        if (t == napi_boolean) d.tied = flag(env, argv[0], "tied");
    }
    // hybrid checkpoints (loader.js dimsFromManifest): rot_dim, hybrid,
    // layer_types (strings), linear {nK, nV, Dk, Dv, K4}, mtp {draftVocab}
    d.rot_dim = (int32_t)num(env, argv[0], "rot_dim", 0);
    d.hybrid = flag(env, argv[0], "hybrid");
    std::vector<uint8_t> kinds;
    napi_value lt;
    if (get_prop(env, argv[0], "layer_types", &lt)) {
        bool arr = false;
        napi_is_array(env, lt, &arr);
        uint32_t n = 0;
        if (arr) napi_get_array_length(env, lt, &n);
        for (uint32_t i = 0; i < n; i++) {
            napi_value e;
            napi_get_element(env, lt, i, &e);
            char buf[32] = {0};
            size_t len = 0;
            napi_get_value_string_utf8(env, e, buf, sizeof buf, &len);
            kinds.push_back(std::string(buf) == "linear_attention" ? CC_LINEAR_ATTENTION : CC_FULL_ATTENTION);
        }
        if ((int)kinds.size() == d.n_layer) d.layer_kinds = kinds.data();
    }
    napi_value lin;
    if (get_prop(env, argv[0], "linear", &lin)) {
        d.lin_nk = (int32_t)num(env, lin, "nK", 0);
        d.lin_nv = (int32_t)num(env, lin, "nV", 0);
        d.lin_dk = (int32_t)num(env, lin, "Dk", 0);
        d.lin_dv = (int32_t)num(env, lin, "Dv", 0);
        d.lin_conv = (int32_t)num(env, lin, "K4", 0);
    }
    napi_value mtp;
    if (get_prop(env, argv[0], "mtp", &mtp)) d.mtp_vocab = (int32_t)num(env, mtp, "draftVocab", 0);
    napi_value rs;
    if (get_prop(env, argv[0], "rope_scaling", &rs)) {
        d.rope_scaling = 1;
        d.rs_factor = num(env, rs, "factor", 8.0);
        d.rs_low_freq = num(env, rs, "low_freq_factor", 1.0);
        d.rs_high_freq = num(env, rs, "high_freq_factor", 4.0);
        d.rs_orig_max_pos = num(env, rs, "original_max_position_embeddings", 8192.0);
    }
    cc_opts o{};
    o.lo = (int32_t)num(env, argv[1], "lo", 0);
    o.hi = (int32_t)num(env, argv[1], "hi", d.n_layer + 2);
    o.n_max = (int32_t)num(env, argv[1], "nMax", 0);
    o.t_max = (int32_t)num(env, argv[1], "tMax", 0);
    o.slots = (int32_t)num(env, argv[1], "slots", 1);
    o.sessions = (int32_t)num(env, argv[1], "sessions", o.slots);
    o.page_tokens = (int32_t)num(env, argv[1], "pageTokens", 64);
    o.max_jobs = (int32_t)num(env, argv[1], "maxJobs", o.sessions);
    o.device = (int32_t)num(env, argv[1], "device", 0);
    cc_ctx* ctx = nullptr;
    const cc_status st = cc_create(&d, &o, &ctx);
    if (st != CC_OK) {
        std::string msg = ctx ? cc_last_error(ctx) : "cc_create failed";
        if (ctx) cc_destroy(ctx);
        throw_status(env, st, msg);
        return nullptr;
    }
    Ctx* c = new Ctx;
    c->ctx = ctx;
    c->hidden = d.hidden;
    c->vocab = d.vocab;
    napi_value ext;
    NAPI_OK(napi_create_external(env, c, finalize_ctx, nullptr, &ext));
    return ext;
}

napi_value Destroy(napi_env env, napi_callback_info info) {
    size_t argc = 1;
    napi_value argv[1];
    NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
    void* p = nullptr;
    if (argc < 1 || napi_get_value_external(env, argv[0], &p) != napi_ok || !p) return undef(env);
    Ctx* c = (Ctx*)p;
    if (c->busy) {
        napi_throw_error(env, nullptr, "destroy() while a step is running");
        return nullptr;
    }
    if (c->ctx) cc_destroy(c->ctx);
    c->ctx = nullptr;
    return undef(env);
}

// Calls returning a cc_status: throw with the context's message on failure.
napi_value status_result(napi_env env, Ctx* c, cc_status st) {
    if (st != CC_OK) {
        throw_status(env, st, cc_last_error(c->ctx));
        return nullptr;
    }
    return undef(env);
}

uint64_t u64(napi_env env, napi_value v) {
    napi_valuetype t;
    napi_typeof(env, v, &t);
    if (t == napi_bigint) {
        uint64_t r = 0;
        bool lossless;
        napi_get_value_bigint_uint64(env, v, &r, &lossless);
        return r;
    }
    double d = 0;
    napi_get_value_double(env, v, &d);
    return (uint64_t)d;
}

napi_value FillRandom(napi_env env, napi_callback_info info) {
    size_t argc = 2;
    napi_value argv[2];
    NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
    Ctx* c = idle(env, argv[0], "fillRandom");
    if (!c) return nullptr;
    return status_result(env, c, cc_fill_random(c->ctx, argc > 1 ? u64(env, argv[1]) : 1));
}

// fillRandomKV(ctx, slot, tokens, seed, key)
napi_value FillRandomKV(napi_env env, napi_callback_info info) {
    size_t argc = 5;
    napi_value argv[5];
    NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
    Ctx* c = idle(env, argv[0], "fillRandomKV");
    if (!c) return nullptr;
    int32_t slot = 0, tokens = 0;
    napi_get_value_int32(env, argv[1], &slot);
    napi_get_value_int32(env, argv[2], &tokens);
    return status_result(env, c, cc_fill_random_kv(c->ctx, slot, tokens, u64(env, argv[3]), u64(env, argv[4])));
}

// upload(ctx, layer, tensor, data, scales|null, group = 32): data Int8Array
// [N*K] (or a Float32Array norm), scales Uint16Array (f16 bits) or
// Float32Array [N*ceil(K/group)], group a multiple of 32.
napi_value Upload(napi_env env, napi_callback_info info) {
    size_t argc = 6;
    napi_value argv[6];
    NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
    Ctx* c = idle(env, argv[0], "upload");
    if (!c) return nullptr;
    int32_t layer = 0, tensor = 0;
    napi_get_value_int32(env, argv[1], &layer);
    napi_get_value_int32(env, argv[2], &tensor);
    void* data = nullptr;
    size_t n = 0;
    napi_typedarray_type t;
    if (!typed(env, argv[3], &data, &n, &t)) {
        napi_throw_type_error(env, nullptr, "data must be a typed array");
        return nullptr;
    }
    void* sc = nullptr;
    size_t ns = 0;
    napi_typedarray_type st = napi_uint16_array;
    if (argc > 4) typed(env, argv[4], &sc, &ns, &st);
    int32_t group = 32;
    if (argc > 5) {
        napi_valuetype vt;
        napi_typeof(env, argv[5], &vt);
        if (vt == napi_number) napi_get_value_int32(env, argv[5], &group);
    }
    return status_result(env, c, cc_upload(c->ctx, layer, tensor, data, n, sc, ns,
                                           st == napi_float32_array ? CC_SCALES_F32 : CC_SCALES_F16, group));
}

// ---- step (async) ----
struct StepWork {
    Ctx* c = nullptr;
    napi_ref keep = nullptr;        // the context's external, alive until the step completes
    napi_deferred deferred = nullptr;
    napi_async_work work = nullptr;
    std::vector<cc_job> jobs;
    std::vector<std::vector<int32_t>> ids;
    std::vector<std::vector<uint16_t>> hidden;
    int32_t at = 0, to = 0, topk = 0, rows = 0, sampled = 0;
    std::vector<float> vals;
    std::vector<uint32_t> tids;
    std::vector<uint16_t> hout;
    std::vector<int32_t> status;
    cc_status st = CC_OK;
    std::string err;
};

void step_execute(napi_env, void* data) {
    StepWork* w = (StepWork*)data;
    w->st = cc_step(w->c->ctx, w->jobs.data(), (int32_t)w->jobs.size(), w->at, w->to, w->topk,
                    w->vals.empty() ? nullptr : w->vals.data(), w->tids.empty() ? nullptr : w->tids.data(),
                    w->hout.empty() ? nullptr : w->hout.data(), w->status.data());
    if (w->st != CC_OK) w->err = cc_last_error(w->c->ctx);
}

template <class T>
napi_value copy_out(napi_env env, const std::vector<T>& v, napi_typedarray_type type) {
    napi_value ab, ta;
    void* p = nullptr;
    napi_create_arraybuffer(env, v.size() * sizeof(T), &p, &ab);
    if (!v.empty()) std::memcpy(p, v.data(), v.size() * sizeof(T));
    napi_create_typedarray(env, type, v.size(), ab, 0, &ta);
    return ta;
}

void step_complete(napi_env env, napi_status, void* data) {
    StepWork* w = (StepWork*)data;
    w->c->busy = false;
    if (w->keep) napi_delete_reference(env, w->keep);
    if (w->c->orphan) destroy_ctx(w->c);
    napi_value res;
    napi_create_object(env, &res);
    napi_value code;
    napi_create_int32(env, w->st, &code);
    napi_set_named_property(env, res, "code", code);
    napi_set_named_property(env, res, "status", copy_out(env, w->status, napi_int32_array));
    if (w->st == CC_OK) {
        if (!w->vals.empty()) {
            napi_set_named_property(env, res, "vals", copy_out(env, w->vals, napi_float32_array));
            napi_set_named_property(env, res, "ids", copy_out(env, w->tids, napi_uint32_array));
        }
        if (!w->hout.empty()) napi_set_named_property(env, res, "hidden", copy_out(env, w->hout, napi_uint16_array));
    } else {
        napi_value m;
        napi_create_string_utf8(env, w->err.c_str(), w->err.size(), &m);
        napi_set_named_property(env, res, "error", m);
    }
    napi_resolve_deferred(env, w->deferred, res);
    napi_delete_async_work(env, w->work);
    delete w;
}

// step(ctx, jobs, at, to, topk) -> Promise<{code, status, vals?, ids?, hidden?, error?}>
// jobs: [{slot, past, n, sampled, ids?: Int32Array, hidden?: Uint16Array}]
napi_value Step(napi_env env, napi_callback_info info) {
    size_t argc = 5;
    napi_value argv[5];
    NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
    Ctx* c = unwrap(env, argv[0]);
    if (!c) return nullptr;
    if (c->busy) {
        throw_status(env, CC_EARG, "a step is already running on this context");
        return nullptr;
    }
    StepWork* w = new StepWork;
    w->c = c;
    napi_get_value_int32(env, argv[2], &w->at);
    napi_get_value_int32(env, argv[3], &w->to);
    napi_get_value_int32(env, argv[4], &w->topk);
    uint32_t nj = 0;
    napi_get_array_length(env, argv[1], &nj);
    w->jobs.resize(nj);
    w->ids.resize(nj);
    w->hidden.resize(nj);
    for (uint32_t j = 0; j < nj; j++) {
        napi_value o;
        napi_get_element(env, argv[1], j, &o);
        cc_job& jb = w->jobs[j];
        jb.slot = (int32_t)num(env, o, "slot", -1);
        jb.past = (int32_t)num(env, o, "past", 0);
        jb.n = (int32_t)num(env, o, "n", 0);
        jb.sampled = (int32_t)num(env, o, "sampled", 0);
        // speculation through linear_attention blocks, and the MTP fill
        jb.snap = flag(env, o, "snap");
        napi_value kv;
        if (get_prop(env, o, "keep", &kv)) {
            jb.rollback = 1;
            jb.keep = (int32_t)num(env, o, "keep", 0);
        }
        jb.mtp = flag(env, o, "mtp");
        napi_value v;
        void* data;
        size_t len;
        napi_typedarray_type t;
        if (get_prop(env, o, "ids", &v) && typed(env, v, &data, &len, &t) && t == napi_int32_array)
            w->ids[j].assign((int32_t*)data, (int32_t*)data + len);
        if (get_prop(env, o, "hidden", &v) && typed(env, v, &data, &len, &t) && t == napi_uint16_array)
            w->hidden[j].assign((uint16_t*)data, (uint16_t*)data + len);
        jb.ids = w->ids[j].empty() ? nullptr : w->ids[j].data();
        jb.hidden = w->hidden[j].empty() ? nullptr : w->hidden[j].data();
        w->rows += jb.n;
        w->sampled += jb.sampled;
    }
    w->status.assign(nj, 0);
    if (w->sampled > 0 && w->topk > 0) {
        w->vals.assign((size_t)w->sampled * w->topk, 0.f);
        w->tids.assign((size_t)w->sampled * w->topk, 0u);
    } else {
        w->hout.assign((size_t)w->rows * c->hidden, 0);
    }
    napi_value promise, name;
    NAPI_OK(napi_create_promise(env, &w->deferred, &promise));
    napi_create_string_utf8(env, "ccdecode.step", NAPI_AUTO_LENGTH, &name);
    NAPI_OK(napi_create_async_work(env, nullptr, name, step_execute, step_complete, w, &w->work));
    NAPI_OK(napi_create_reference(env, argv[0], 1, &w->keep));
    c->busy = true;
    NAPI_OK(napi_queue_async_work(env, w->work));
    return promise;
}

napi_value Release(napi_env env, napi_callback_info info) {
    size_t argc = 2;
    napi_value argv[2];
    NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
    Ctx* c = idle(env, argv[0], "release");
    if (!c) return nullptr;
    int32_t slot = 0;
    napi_get_value_int32(env, argv[1], &slot);
    return status_result(env, c, cc_release(c->ctx, slot));
}

napi_value SlotPages(napi_env env, napi_callback_info info) {
    size_t argc = 2;
    napi_value argv[2];
    NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
    Ctx* c = idle(env, argv[0], "slotPages");
    if (!c) return nullptr;
    int32_t slot = 0;
    napi_get_value_int32(env, argv[1], &slot);
    napi_value r;
    napi_create_int32(env, cc_slot_pages(c->ctx, slot), &r);
    return r;
}

napi_value FreePages(napi_env env, napi_callback_info info) {
    size_t argc = 1;
    napi_value argv[1];
    NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
    Ctx* c = idle(env, argv[0], "freePages");
    if (!c) return nullptr;
    napi_value r;
    napi_create_int32(env, cc_free_pages(c->ctx), &r);
    return r;
}

// readLogits(ctx, rows) -> Float32Array [rows * vocab]
napi_value ReadLogits(napi_env env, napi_callback_info info) {
    size_t argc = 2;
    napi_value argv[2];
    NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
    Ctx* c = idle(env, argv[0], "readLogits");
    if (!c) return nullptr;
    int32_t rows = 0;
    napi_get_value_int32(env, argv[1], &rows);
    if (rows < 1) {
        throw_status(env, CC_EARG, "rows must be positive");
        return nullptr;
    }
    std::vector<float> out((size_t)rows * c->vocab);
    const cc_status st = cc_read_logits(c->ctx, rows, out.data());
    if (st != CC_OK) {
        throw_status(env, st, cc_last_error(c->ctx));
        return nullptr;
    }
    return copy_out(env, out, napi_float32_array);
}

// mtpDraft(ctx, slot, row, token, pos, k) -> Uint32Array [k]: cc_mtp_draft
// (Runner.#mtpAfter, stage.js:296-320).
napi_value MtpDraft(napi_env env, napi_callback_info info) {
    size_t argc = 6;
    napi_value argv[6];
    NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
    if (argc < 6) {
        napi_throw_type_error(env, nullptr, "mtpDraft(ctx, slot, row, token, pos, k)");
        return nullptr;
    }
    Ctx* c = idle(env, argv[0], "mtpDraft");
    if (!c) return nullptr;
    int32_t a[5] = {0, 0, 0, 0, 0};
    for (int i = 0; i < 5; i++) napi_get_value_int32(env, argv[1 + i], &a[i]);
    std::vector<uint32_t> out((size_t)std::max(a[4], 1));
    const cc_status st = cc_mtp_draft(c->ctx, a[0], a[1], a[2], a[3], a[4], out.data());
    if (st != CC_OK) {
        throw_status(env, st, cc_last_error(c->ctx));
        return nullptr;
    }
    out.resize((size_t)std::max(a[4], 0));
    return copy_out(env, out, napi_uint32_array);
}

napi_value Stats(napi_env env, napi_callback_info info) {
    size_t argc = 1;
    napi_value argv[1];
    NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
    Ctx* c = idle(env, argv[0], "stats");
    if (!c) return nullptr;
    cc_stats s{};
    cc_stats_get(c->ctx, &s);
    napi_value o, v;
    napi_create_object(env, &o);
    const struct { const char* k; double v; } f[] = {
        {"vramBytes", (double)s.vram_bytes}, {"weightBytes", (double)s.weight_bytes},
        {"kvBytes", (double)s.kv_bytes},     {"scratchBytes", (double)s.scratch_bytes},
        {"passes", (double)s.passes},        {"rows", (double)s.rows},
        {"lastPassMs", s.last_pass_ms}};
    for (const auto& e : f) {
        napi_create_double(env, e.v, &v);
        napi_set_named_property(env, o, e.k, v);
    }
    return o;
}

napi_value LastError(napi_env env, napi_callback_info info) {
    size_t argc = 1;
    napi_value argv[1];
    NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
    Ctx* c = idle(env, argv[0], "lastError");
    if (!c) return nullptr;
    const char* m = cc_last_error(c->ctx);
    napi_value r;
    napi_create_string_utf8(env, m ? m : "", NAPI_AUTO_LENGTH, &r);
    return r;
}

napi_value Init(napi_env env, napi_value exports) {
    const struct { const char* name; napi_callback fn; } fns[] = {
        {"create", Create},         {"destroy", Destroy},     {"fillRandom", FillRandom},
        {"fillRandomKV", FillRandomKV}, {"upload", Upload},   {"step", Step},
        {"release", Release},       {"slotPages", SlotPages}, {"freePages", FreePages},
        {"readLogits", ReadLogits}, {"stats", Stats},         {"lastError", LastError},
        {"mtpDraft", MtpDraft}};
    for (const auto& f : fns) {
        napi_value fn;
        napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.fn, nullptr, &fn);
        napi_set_named_property(env, exports, f.name, fn);
    }
    return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
