// ssm_napi.cc -- Node-API addon over libssm_hip.so (include/ssm_hip.h).
//
// This is the thin C-ABI binding that the reference's TypeScript host loads in place of the
// MambaCode.js WebGPU backend (@seanhogg/mambacode.js, package-lock.json:1231-1241). index.js
// turns these functions into the module shape src/session/session.ts imports:
// initWebGPU (session.ts:274-277), HybridMambaModel (:359, forward streaming.ts:31-35,
// generate session.ts:421-425, loadWeights :394/:575, exportWeights :518), MambaTrainer
// (:506).
//
// Every call that touches the GPU for longer than a pointer swap runs in napi_async_work on
// the libuv pool and returns a Promise, so `await model.forward(...)` never blocks the event
// loop. A failing call rejects with an Error whose `code` is the reference's error string
// (ssm_status_name: 'GPU_UNAVAILABLE', 'CHECKPOINT_INVALID', 'SESSION_DESTROYED', 'UNKNOWN').
// Inputs are copied out of their typed arrays before the work is queued; outputs come back
// as fresh ArrayBuffers. Calls on one model are serialised by index.js (one HIP stream and
// one workspace per model).
#define NAPI_VERSION 8
#include <node_api.h>

#include <cstdint>
#include <cstring>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "../../include/ssm_hip.h"

namespace {

// Handles wrap the C objects together with the sizes the addon needs for its outputs.
struct Ctx { ssm_ctx* c = nullptr; };
struct Model { ssm_model* m = nullptr; int vocab = 0; };
struct State { ssm_state* s = nullptr; int batch = 0; };

#define NAPI_OK(call)                                                   \
    do {                                                                \
        if ((call) != napi_ok) {                                        \
            napi_throw_error(env, "UNKNOWN", "ssm_napi: N-API call failed: " #call); \
            return nullptr;                                             \
        }                                                               \
    } while (0)

napi_value make_error(napi_env env, const char* code, const std::string& msg) {
    napi_value c, m, e;
    napi_create_string_utf8(env, code, NAPI_AUTO_LENGTH, &c);
    napi_create_string_utf8(env, msg.c_str(), msg.size(), &m);
    napi_create_error(env, c, m, &e);
    return e;
}

void throw_status(napi_env env, ssm_status st) {
    napi_throw(env, make_error(env, ssm_status_name(st), ssm_last_error()));
}

bool get_args(napi_env env, napi_callback_info info, size_t want, napi_value* argv) {
    size_t argc = want;
    if (napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr) != napi_ok || argc < want) {
        napi_throw_type_error(env, "UNKNOWN", "ssm_napi: too few arguments");
        return false;
    }
    return true;
}

template <typename T>
T* unwrap(napi_env env, napi_value v) {
    void* p = nullptr;
    if (napi_get_value_external(env, v, &p) != napi_ok || !p) {
        napi_throw_type_error(env, "UNKNOWN", "ssm_napi: expected a handle");
        return nullptr;
    }
    return static_cast<T*>(p);
}

napi_value wrap(napi_env env, void* p) {
    napi_value v;
    napi_create_external(env, p, nullptr, nullptr, &v);
    return v;
}

int get_int(napi_env env, napi_value v, bool* ok) {
    int32_t x = 0;
    if (napi_get_value_int32(env, v, &x) != napi_ok) *ok = false;
    return x;
}

double get_double(napi_env env, napi_value v, bool* ok) {
    double x = 0.0;
    if (napi_get_value_double(env, v, &x) != napi_ok) *ok = false;
    return x;
}

// Copy the bytes of an ArrayBuffer, a TypedArray or a DataView.
bool copy_bytes(napi_env env, napi_value v, std::vector<uint8_t>& out) {
    bool is = false;
    void* data = nullptr;
    size_t len = 0;
    if (napi_is_arraybuffer(env, v, &is) == napi_ok && is) {
        napi_get_arraybuffer_info(env, v, &data, &len);
    } else if (napi_is_typedarray(env, v, &is) == napi_ok && is) {
        napi_typedarray_type t;
        size_t n = 0, off = 0;
        napi_value ab;
        napi_get_typedarray_info(env, v, &t, &n, &data, &ab, &off);
        size_t esz = 1;
        switch (t) {
            case napi_int16_array: case napi_uint16_array: esz = 2; break;
            case napi_int32_array: case napi_uint32_array: case napi_float32_array: esz = 4; break;
            case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: esz = 8; break;
            default: esz = 1;
        }
        len = n * esz;
    } else if (napi_is_dataview(env, v, &is) == napi_ok && is) {
        napi_value ab;
        size_t off = 0;
        napi_get_dataview_info(env, v, &len, &data, &ab, &off);
    } else {
        napi_throw_type_error(env, "UNKNOWN", "ssm_napi: expected an ArrayBuffer or TypedArray");
        return false;
    }
    out.assign(static_cast<uint8_t*>(data), static_cast<uint8_t*>(data) + len);
    return true;
}

// Uint32Array of token ids (any integer typed array with 4-byte elements is accepted).
bool copy_ids(napi_env env, napi_value v, std::vector<uint32_t>& out) {
    bool is = false;
    if (napi_is_typedarray(env, v, &is) != napi_ok || !is) {
        napi_throw_type_error(env, "UNKNOWN", "ssm_napi: ids must be a Uint32Array");
        return false;
    }
    napi_typedarray_type t;
    size_t n = 0, off = 0;
    void* data = nullptr;
    napi_value ab;
    napi_get_typedarray_info(env, v, &t, &n, &data, &ab, &off);
    if (t != napi_uint32_array && t != napi_int32_array) {
        napi_throw_type_error(env, "UNKNOWN", "ssm_napi: ids must be a Uint32Array");
        return false;
    }
    out.assign(static_cast<uint32_t*>(data), static_cast<uint32_t*>(data) + n);
    return true;
}

// ------------------------------------------------------------------ async work
// One queued call: `run` executes on the pool and fills the outputs; `done` builds the
// resolved value on the main thread.
struct Job {
    napi_async_work work = nullptr;
    napi_deferred deferred = nullptr;
    std::function<ssm_status()> run;
    std::function<napi_value(napi_env)> done;
    ssm_status status = SSM_OK;
    std::string message;
};

void job_execute(napi_env, void* data) {
    Job* j = static_cast<Job*>(data);
    j->status = j->run();
    if (j->status != SSM_OK) j->message = ssm_last_error();   // thread-local: read it here
}

void job_complete(napi_env env, napi_status, void* data) {
    Job* j = static_cast<Job*>(data);
    if (j->status == SSM_OK) {
        napi_value v = j->done ? j->done(env) : nullptr;
        if (!v) napi_get_undefined(env, &v);
        napi_resolve_deferred(env, j->deferred, v);
    } else {
        napi_reject_deferred(env, j->deferred,
                             make_error(env, ssm_status_name(j->status), j->message));
    }
    napi_delete_async_work(env, j->work);
    delete j;
}

napi_value queue(napi_env env, Job* j, const char* name) {
    napi_value promise, res;
    napi_create_promise(env, &j->deferred, &promise);
    napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &res);
    napi_create_async_work(env, nullptr, res, job_execute, job_complete, j, &j->work);
    napi_queue_async_work(env, j->work);
    return promise;
}

template <typename T, napi_typedarray_type TT>
napi_value typed_from(napi_env env, const std::vector<T>& v) {
    void* data = nullptr;
    napi_value ab, arr;
    napi_create_arraybuffer(env, v.size() * sizeof(T), &data, &ab);
    if (!v.empty()) std::memcpy(data, v.data(), v.size() * sizeof(T));
    napi_create_typedarray(env, TT, v.size(), ab, 0, &arr);
    return arr;
}

// ------------------------------------------------------------------ exported functions
napi_value Version(napi_env env, napi_callback_info) {
    napi_value v;
    napi_create_int32(env, ssm_abi_version(), &v);
    return v;
}

// ctxCreate(ordinal) -> Promise<ctx>     (initWebGPU + requestDevice, session.ts:263,274)
napi_value CtxCreate(napi_env env, napi_callback_info info) {
    napi_value argv[1];
    if (!get_args(env, info, 1, argv)) return nullptr;
    bool ok = true;
    const int ord = get_int(env, argv[0], &ok);
    auto* c = new Ctx();
    Job* j = new Job();
    j->run = [c, ord]() { return ssm_ctx_create(ord, &c->c); };
    j->done = [c](napi_env e) { return wrap(e, c); };
    return queue(env, j, "ssm_ctx_create");
}

// ctxDestroy(ctx)                        (device.destroy(), session.ts:592)
// Runs on the main thread. The library takes the context's lock, so it waits for a job of
// this device that a pool thread is running, and frees nothing under it. The handle is kept:
// jobs queued later reach the library, which answers SESSION_DESTROYED.
napi_value CtxDestroy(napi_env env, napi_callback_info info) {
    napi_value argv[1];
    if (!get_args(env, info, 1, argv)) return nullptr;
    Ctx* c = unwrap<Ctx>(env, argv[0]);
    if (!c) return nullptr;
    if (c->c) {
        const ssm_status st = ssm_ctx_destroy(c->c);
        if (st != SSM_OK) throw_status(env, st);
    }
    return nullptr;
}

// ctxInfo(ctx) -> {arch, computeUnits, totalMemory}
napi_value CtxInfo(napi_env env, napi_callback_info info) {
    napi_value argv[1];
    if (!get_args(env, info, 1, argv)) return nullptr;
    Ctx* c = unwrap<Ctx>(env, argv[0]);
    if (!c) return nullptr;
    char arch[64] = {0};
    int cus = 0;
    size_t mem = 0;
    const ssm_status st = ssm_ctx_info(c->c, arch, sizeof arch, &cus, &mem);
    if (st != SSM_OK) { throw_status(env, st); return nullptr; }
    napi_value o, a, n, m;
    napi_create_object(env, &o);
    napi_create_string_utf8(env, arch, NAPI_AUTO_LENGTH, &a);
    napi_create_int32(env, cus, &n);
    napi_create_double(env, (double)mem, &m);
    napi_set_named_property(env, o, "arch", a);
    napi_set_named_property(env, o, "computeUnits", n);
    napi_set_named_property(env, o, "totalMemory", m);
    return o;
}

// modelCreate(ctx, cfg, seed) -> Promise<model>     (new HybridMambaModel, session.ts:359)
// cfg: {vocabSize, dModel, numLayers, dState, dConv, expand, nHeads, nGroups, chunkLen,
//       mimoGroup, eosId, dtRank?, normEps?, layerTypes: Int32Array (SSM_LAYER_*)}
napi_value ModelCreate(napi_env env, napi_callback_info info) {
    napi_value argv[3];
    if (!get_args(env, info, 3, argv)) return nullptr;
    Ctx* c = unwrap<Ctx>(env, argv[0]);
    if (!c) return nullptr;
    auto field = [&](const char* k, int dflt) {
        napi_value v;
        bool has = false;
        napi_has_named_property(env, argv[1], k, &has);
        if (!has) return dflt;
        napi_get_named_property(env, argv[1], k, &v);
        int32_t x = dflt;
        napi_get_value_int32(env, v, &x);
        return (int)x;
    };
    ssm_config cfg{};
    cfg.vocab_size = field("vocabSize", 0);
    cfg.d_model = field("dModel", 0);
    cfg.n_layers = field("numLayers", 0);
    cfg.d_state = field("dState", 16);
    cfg.d_conv = field("dConv", 4);
    cfg.expand = field("expand", 2);
    cfg.n_heads = field("nHeads", 1);
    cfg.n_groups = field("nGroups", 1);
    cfg.chunk_len = field("chunkLen", 256);
    cfg.mimo_group = field("mimoGroup", 1);
    cfg.eos_id = field("eosId", -1);
    cfg.dt_rank = field("dtRank", 0);
    {
        napi_value v;
        bool has = false;
        double eps = 0.0;
        napi_has_named_property(env, argv[1], "normEps", &has);
        if (has && napi_get_named_property(env, argv[1], "normEps", &v) == napi_ok)
            napi_get_value_double(env, v, &eps);
        cfg.norm_eps = (float)eps;
    }
    auto* types = new std::vector<int32_t>();
    {
        napi_value v;
        NAPI_OK(napi_get_named_property(env, argv[1], "layerTypes", &v));
        std::vector<uint32_t> t;
        if (!copy_ids(env, v, t)) { delete types; return nullptr; }
        types->assign(t.begin(), t.end());
    }
    int64_t seed = 0;
    napi_get_value_int64(env, argv[2], &seed);
    if ((int)types->size() != cfg.n_layers) {
        delete types;
        napi_throw(env, make_error(env, "UNKNOWN", "ssm_napi: layerTypes must have numLayers entries"));
        return nullptr;
    }
    auto* m = new Model();
    m->vocab = cfg.vocab_size;
    Job* j = new Job();
    ssm_ctx* cc = c->c;
    j->run = [cc, cfg, types, m, seed]() mutable {
        cfg.layer_types = types->data();
        const ssm_status st = ssm_model_create(cc, &cfg, (uint64_t)seed, &m->m);
        delete types;
        return st;
    };
    j->done = [m](napi_env e) { return wrap(e, m); };
    return queue(env, j, "ssm_model_create");
}

napi_value ModelDestroy(napi_env env, napi_callback_info info) {
    napi_value argv[1];
    if (!get_args(env, info, 1, argv)) return nullptr;
    Model* m = unwrap<Model>(env, argv[0]);
    if (!m) return nullptr;
    if (m->m) {
        const ssm_status st = ssm_model_destroy(m->m);
        if (st != SSM_OK) throw_status(env, st);
    }
    return nullptr;
}

// loadWeights(model, buf) -> Promise<void>       (session.ts:394,575)
napi_value LoadWeights(napi_env env, napi_callback_info info) {
    napi_value argv[2];
    if (!get_args(env, info, 2, argv)) return nullptr;
    Model* m = unwrap<Model>(env, argv[0]);
    if (!m) return nullptr;
    auto* buf = new std::vector<uint8_t>();
    if (!copy_bytes(env, argv[1], *buf)) { delete buf; return nullptr; }
    Job* j = new Job();
    j->run = [m, buf]() {
        const ssm_status st = ssm_model_load_weights(m->m, buf->data(), buf->size());
        delete buf;
        return st;
    };
    return queue(env, j, "ssm_model_load_weights");
}

// exportWeights(model, f16) -> Promise<ArrayBuffer>   (session.ts:518)
napi_value ExportWeights(napi_env env, napi_callback_info info) {
    napi_value argv[2];
    if (!get_args(env, info, 2, argv)) return nullptr;
    Model* m = unwrap<Model>(env, argv[0]);
    if (!m) return nullptr;
    bool f16 = false;
    napi_get_value_bool(env, argv[1], &f16);
    auto out = std::make_shared<std::vector<uint8_t>>();
    Job* j = new Job();
    j->run = [m, f16, out]() {
        size_t bytes = 0;
        ssm_status st = ssm_model_export_weights(m->m, f16 ? 1 : 0, nullptr, 0, &bytes);
        if (st != SSM_OK) return st;
        out->resize(bytes);
        return ssm_model_export_weights(m->m, f16 ? 1 : 0, out->data(), bytes, &bytes);
    };
    j->done = [out](napi_env e) {
        void* data = nullptr;
        napi_value ab;
        napi_create_arraybuffer(e, out->size(), &data, &ab);
        if (!out->empty()) std::memcpy(data, out->data(), out->size());
        return ab;
    };
    return queue(env, j, "ssm_model_export_weights");
}

// forward(model, ids, batch, seqLen) -> Promise<Float32Array (batch*seqLen*V)>
// (model.forward, streaming.ts:31-35)
napi_value Forward(napi_env env, napi_callback_info info) {
    napi_value argv[4];
    if (!get_args(env, info, 4, argv)) return nullptr;
    Model* m = unwrap<Model>(env, argv[0]);
    if (!m) return nullptr;
    bool ok = true;
    const int B = get_int(env, argv[2], &ok), L = get_int(env, argv[3], &ok);
    auto ids = std::make_shared<std::vector<uint32_t>>();
    if (!copy_ids(env, argv[1], *ids)) return nullptr;
    if (!ok || B < 0 || L < 0 || (size_t)B * L != ids->size()) {
        napi_throw(env, make_error(env, "UNKNOWN", "forward: ids.length must equal batch * seqLen"));
        return nullptr;
    }
    auto out = std::make_shared<std::vector<float>>((size_t)B * L * m->vocab);
    Job* j = new Job();
    j->run = [m, ids, out, B, L]() { return ssm_forward(m->m, ids->data(), B, L, out->data()); };
    j->done = [out](napi_env e) { return typed_from<float, napi_float32_array>(e, *out); };
    return queue(env, j, "ssm_forward");
}

napi_value StateCreate(napi_env env, napi_callback_info info) {
    napi_value argv[2];
    if (!get_args(env, info, 2, argv)) return nullptr;
    Model* m = unwrap<Model>(env, argv[0]);
    if (!m) return nullptr;
    bool ok = true;
    const int B = get_int(env, argv[1], &ok);
    auto* s = new State();
    s->batch = B;
    const ssm_status st = ssm_state_create(m->m, B, &s->s);
    if (st != SSM_OK) { delete s; throw_status(env, st); return nullptr; }
    return wrap(env, s);
}

napi_value StateDestroy(napi_env env, napi_callback_info info) {
    napi_value argv[1];
    if (!get_args(env, info, 1, argv)) return nullptr;
    State* s = unwrap<State>(env, argv[0]);
    if (!s) return nullptr;
    if (s->s) {
        const ssm_status st = ssm_state_destroy(s->s);
        s->s = nullptr;
        if (st != SSM_OK) throw_status(env, st);
    }
    return nullptr;
}

// prefill(model, state, ids (batch*L), L) -> Promise<Float32Array (batch*V)> last logits
napi_value Prefill(napi_env env, napi_callback_info info) {
    napi_value argv[4];
    if (!get_args(env, info, 4, argv)) return nullptr;
    Model* m = unwrap<Model>(env, argv[0]);
    State* s = unwrap<State>(env, argv[1]);
    if (!m || !s) return nullptr;
    bool ok = true;
    const int L = get_int(env, argv[3], &ok);
    auto ids = std::make_shared<std::vector<uint32_t>>();
    if (!copy_ids(env, argv[2], *ids)) return nullptr;
    if (!ok || L <= 0 || (size_t)s->batch * L != ids->size()) {
        napi_throw(env, make_error(env, "UNKNOWN", "prefill: ids.length must equal batch * L"));
        return nullptr;
    }
    auto out = std::make_shared<std::vector<float>>((size_t)s->batch * m->vocab);
    Job* j = new Job();
    j->run = [m, s, ids, out, L]() { return ssm_prefill(m->m, s->s, ids->data(), L, out->data(), nullptr); };
    j->done = [out](napi_env e) { return typed_from<float, napi_float32_array>(e, *out); };
    return queue(env, j, "ssm_prefill");
}

// decodeStep(model, state, ids (batch)) -> Promise<Float32Array (batch*V)>
napi_value DecodeStep(napi_env env, napi_callback_info info) {
    napi_value argv[3];
    if (!get_args(env, info, 3, argv)) return nullptr;
    Model* m = unwrap<Model>(env, argv[0]);
    State* s = unwrap<State>(env, argv[1]);
    if (!m || !s) return nullptr;
    auto ids = std::make_shared<std::vector<uint32_t>>();
    if (!copy_ids(env, argv[2], *ids)) return nullptr;
    if ((int)ids->size() != s->batch) {
        napi_throw(env, make_error(env, "UNKNOWN", "decodeStep: one id per sequence"));
        return nullptr;
    }
    auto out = std::make_shared<std::vector<float>>((size_t)s->batch * m->vocab);
    Job* j = new Job();
    j->run = [m, s, ids, out]() { return ssm_decode_step(m->m, s->s, ids->data(), out->data(), nullptr); };
    j->done = [out](napi_env e) { return typed_from<float, napi_float32_array>(e, *out); };
    return queue(env, j, "ssm_decode_step");
}

// generateGreedy(model, state, prompt (batch*Lp), Lp, nNew) -> Promise<Uint32Array (batch*nNew)>
napi_value GenerateGreedy(napi_env env, napi_callback_info info) {
    napi_value argv[5];
    if (!get_args(env, info, 5, argv)) return nullptr;
    Model* m = unwrap<Model>(env, argv[0]);
    State* s = unwrap<State>(env, argv[1]);
    if (!m || !s) return nullptr;
    bool ok = true;
    const int Lp = get_int(env, argv[3], &ok), n = get_int(env, argv[4], &ok);
    auto ids = std::make_shared<std::vector<uint32_t>>();
    if (!copy_ids(env, argv[2], *ids)) return nullptr;
    if (!ok || Lp <= 0 || n < 0 || (size_t)s->batch * Lp != ids->size()) {
        napi_throw(env, make_error(env, "UNKNOWN", "generateGreedy: prompt.length must equal batch * Lp"));
        return nullptr;
    }
    auto out = std::make_shared<std::vector<uint32_t>>((size_t)s->batch * n);
    Job* j = new Job();
    j->run = [m, s, ids, out, Lp, n]() {
        return ssm_generate_greedy(m->m, s->s, ids->data(), Lp, n, out->data());
    };
    j->done = [out](napi_env e) { return typed_from<uint32_t, napi_uint32_array>(e, *out); };
    return queue(env, j, "ssm_generate_greedy");
}

// generateSample(model, state, prompt (batch*Lp), Lp, nNew, temperature, topK, topP,
//                u Float64Array (nNew*batch)) -> Promise<Uint32Array (batch*nNew)>
// u holds the Math.random() draws, token k of sequence b taking u[k*batch + b].
napi_value GenerateSample(napi_env env, napi_callback_info info) {
    napi_value argv[9];
    if (!get_args(env, info, 9, argv)) return nullptr;
    Model* m = unwrap<Model>(env, argv[0]);
    State* s = unwrap<State>(env, argv[1]);
    if (!m || !s) return nullptr;
    bool ok = true;
    const int Lp = get_int(env, argv[3], &ok), n = get_int(env, argv[4], &ok);
    const double temperature = get_double(env, argv[5], &ok);
    const int top_k = get_int(env, argv[6], &ok);
    const double top_p = get_double(env, argv[7], &ok);
    auto ids = std::make_shared<std::vector<uint32_t>>();
    if (!copy_ids(env, argv[2], *ids)) return nullptr;
    if (!ok || Lp <= 0 || n < 0 || (size_t)s->batch * Lp != ids->size()) {
        napi_throw(env, make_error(env, "UNKNOWN", "generateSample: prompt.length must equal batch * Lp"));
        return nullptr;
    }
    auto u = std::make_shared<std::vector<double>>();
    {
        bool is = false;
        napi_is_typedarray(env, argv[8], &is);
        napi_typedarray_type tt;
        size_t len = 0;
        void* data = nullptr;
        if (is) napi_get_typedarray_info(env, argv[8], &tt, &len, &data, nullptr, nullptr);
        if (!is || tt != napi_float64_array || len != (size_t)n * s->batch) {
            napi_throw(env, make_error(env, "UNKNOWN", "generateSample: u must be a Float64Array of nNew * batch draws"));
            return nullptr;
        }
        u->assign((const double*)data, (const double*)data + len);
    }
    auto out = std::make_shared<std::vector<uint32_t>>((size_t)s->batch * n);
    Job* j = new Job();
    j->run = [m, s, ids, u, out, Lp, n, temperature, top_k, top_p]() {
        return ssm_generate_sample(m->m, s->s, ids->data(), Lp, n, temperature, top_k, top_p,
                                   u->data(), out->data());
    };
    j->done = [out](napi_env e) { return typed_from<uint32_t, napi_uint32_array>(e, *out); };
    return queue(env, j, "ssm_generate_sample");
}

napi_value Init(napi_env env, napi_value exports) {
    const struct { const char* name; napi_callback fn; } fns[] = {
        {"version", Version},         {"ctxCreate", CtxCreate},       {"ctxDestroy", CtxDestroy},
        {"ctxInfo", CtxInfo},         {"modelCreate", ModelCreate},   {"modelDestroy", ModelDestroy},
        {"loadWeights", LoadWeights}, {"exportWeights", ExportWeights}, {"forward", Forward},
        {"stateCreate", StateCreate}, {"stateDestroy", StateDestroy}, {"prefill", Prefill},
        {"decodeStep", DecodeStep},   {"generateGreedy", GenerateGreedy},
        {"generateSample", GenerateSample},
    };
    for (const auto& f : fns) {
        napi_value v;
        napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.fn, nullptr, &v);
        napi_set_named_property(env, exports, f.name, v);
    }
    return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
