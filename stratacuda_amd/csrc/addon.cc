// Node-API addon: the C ABI of libstrata_mi355x.so (include/strata_mi355x.h)
// as JavaScript functions, for the HipBackend in src/backend.js. It holds no
// state of its own: a context is an external wrapping sm_ctx*, a buffer is its
// device handle as a Number (device addresses stay below 2^53). A non-zero
// return code becomes a thrown error carrying sm_last_error: SM_E_ARG as a
// RangeError (the reference's argument errors, src/backend.js:6-8), every
// other code as an Error whose `code` is the SM_E* name.
#ifndef NAPI_VERSION
#define NAPI_VERSION 8
#endif
#include <node_api.h>

#include <stdint.h>
#include <string.h>

#include <string>
#include <vector>

#include "strata_mi355x.h"

namespace {

const char *code_name(int rc) {
    switch (rc) {
    case SM_E_HIP: return "SM_E_HIP";
    case SM_E_ARG: return "SM_E_ARG";
    case SM_E_BOUNDS: return "SM_E_BOUNDS";
    case SM_E_HANDLE: return "SM_E_HANDLE";
    case SM_E_NOKERNEL: return "SM_E_NOKERNEL";
    case SM_E_ROUTE: return "SM_E_ROUTE";
    case SM_E_NOMEM: return "SM_E_NOMEM";
    case SM_E_FAULT: return "SM_E_FAULT";
    default: return "SM_E_UNKNOWN";
    }
}

// Throws for rc != 0; returns true when the caller should return at once.
bool fail(napi_env env, sm_ctx *ctx, int rc) {
    if (rc == SM_OK) return false;
    std::string msg = ctx ? sm_last_error(ctx) : "invalid argument";
    if (msg.empty()) msg = code_name(rc);
    if (rc == SM_E_ARG)
        napi_throw_range_error(env, code_name(rc), msg.c_str());
    else
        napi_throw_error(env, code_name(rc), msg.c_str());
    return true;
}

bool type_error(napi_env env, const char *what) {
    napi_throw_type_error(env, nullptr, what);
    return true;
}

struct Args {
    napi_env env;
    size_t argc = 24;
    napi_value argv[24];
    bool ok = true;
    Args(napi_env e, napi_callback_info info) : env(e) {
        napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr);
    }
    bool need(size_t n) {
        if (argc < n) {
            ok = false;
            type_error(env, "missing arguments");
        }
        return ok;
    }
    sm_ctx *ctx(size_t i) {
        void *p = nullptr;
        if (!ok || napi_get_value_external(env, argv[i], &p) != napi_ok || !p) {
            if (ok) type_error(env, "expected a context");
            ok = false;
        }
        return (sm_ctx *)p;
    }
    double num(size_t i) {
        double v = 0;
        if (!ok) return 0;
        if (napi_get_value_double(env, argv[i], &v) != napi_ok) {
            ok = false;
            type_error(env, "expected a number");
        }
        return v;
    }
    uint64_t u64(size_t i) {
        double v = num(i);
        if (ok && (v < 0 || v > 9007199254740991.0 || v != (double)(uint64_t)v)) {
            ok = false;
            napi_throw_range_error(env, nullptr, "expected a non-negative safe integer");
        }
        return (uint64_t)v;
    }
    int i32(size_t i) {
        double v = num(i);
        if (ok && (v < -2147483648.0 || v > 2147483647.0 || v != (double)(int64_t)v)) {
            ok = false;
            napi_throw_range_error(env, nullptr, "expected a 32-bit integer");
        }
        return (int)v;
    }
    bool flag(size_t i) {
        bool b = false;
        if (ok && napi_get_value_bool(env, argv[i], &b) != napi_ok) {
            ok = false;
            type_error(env, "expected a boolean");
        }
        return b;
    }
    std::string str(size_t i) {
        size_t n = 0;
        if (!ok || napi_get_value_string_utf8(env, argv[i], nullptr, 0, &n) != napi_ok) {
            if (ok) type_error(env, "expected a string");
            ok = false;
            return std::string();
        }
        std::string s(n, '\0');
        napi_get_value_string_utf8(env, argv[i], &s[0], n + 1, &n);
        return s;
    }
    // Bytes of a TypedArray, DataView, Buffer or ArrayBuffer.
    bool bytes(size_t i, void **data, size_t *len) {
        bool is = false;
        if (!ok) return false;
        if (napi_is_typedarray(env, argv[i], &is) == napi_ok && is) {
            napi_typedarray_type t;
            size_t n = 0, off = 0;
            napi_value ab;
            napi_get_typedarray_info(env, argv[i], &t, &n, data, &ab, &off);
            size_t el = 1;
            switch (t) {
            case napi_int16_array: case napi_uint16_array: el = 2; break;
            case napi_int32_array: case napi_uint32_array: case napi_float32_array: el = 4; break;
            case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: el = 8; break;
            default: el = 1;
            }
            *len = n * el;
            return true;
        }
        if (napi_is_dataview(env, argv[i], &is) == napi_ok && is) {
            napi_value ab;
            size_t off = 0;
            napi_get_dataview_info(env, argv[i], len, data, &ab, &off);
            return true;
        }
        if (napi_is_arraybuffer(env, argv[i], &is) == napi_ok && is) {
            napi_get_arraybuffer_info(env, argv[i], data, len);
            return true;
        }
        ok = false;
        type_error(env, "expected a TypedArray, DataView or ArrayBuffer");
        return false;
    }
};

napi_value undefined(napi_env env) {
    napi_value v;
    napi_get_undefined(env, &v);
    return v;
}
napi_value number(napi_env env, double d) {
    napi_value v;
    napi_create_double(env, d, &v);
    return v;
}
napi_value string(napi_env env, const std::string &s) {
    napi_value v;
    napi_create_string_utf8(env, s.c_str(), s.size(), &v);
    return v;
}

napi_value Init(napi_env env, napi_callback_info info) {
    Args a(env, info);
    int device = a.argc > 0 ? a.i32(0) : 0;
    if (!a.ok) return nullptr;
    sm_ctx *ctx = nullptr;
    if (fail(env, nullptr, sm_init(device, &ctx))) return nullptr;
    napi_value v;
    napi_create_external(env, ctx, nullptr, nullptr, &v);
    return v;
}
napi_value Shutdown(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(1)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    if (!a.ok) return nullptr;
    sm_shutdown(ctx);
    return undefined(env);
}
napi_value LastError(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(1)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    if (!a.ok) return nullptr;
    return string(env, sm_last_error(ctx));
}
napi_value Info(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(1)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    if (!a.ok) return nullptr;
    std::vector<char> buf(4096);
    int n = sm_info(ctx, buf.data(), buf.size());
    if (n < 0 && fail(env, ctx, n)) return nullptr;
    return string(env, std::string(buf.data(), (size_t)n < buf.size() ? (size_t)n : buf.size() - 1));
}
napi_value Alloc(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(3)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    uint64_t bytes = a.u64(1);
    bool zero = a.flag(2);
    if (!a.ok) return nullptr;
    uint64_t h = 0;
    if (fail(env, ctx, sm_alloc(ctx, bytes, zero ? 1 : 0, &h))) return nullptr;
    return number(env, (double)h);
}
napi_value Free(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(2)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    uint64_t h = a.u64(1);
    if (!a.ok || fail(env, ctx, sm_free(ctx, h))) return nullptr;
    return undefined(env);
}
napi_value Size(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(2)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    uint64_t h = a.u64(1), n = 0;
    if (!a.ok || fail(env, ctx, sm_size(ctx, h, &n))) return nullptr;
    return number(env, (double)n);
}
napi_value Write(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(4)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    uint64_t h = a.u64(1), off = a.u64(2);
    void *data = nullptr;
    size_t len = 0;
    a.bytes(3, &data, &len);
    if (!a.ok || fail(env, ctx, sm_write(ctx, h, off, data, len))) return nullptr;
    return undefined(env);
}
napi_value Read(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(4)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    uint64_t h = a.u64(1), off = a.u64(2), len = a.u64(3);
    if (!a.ok) return nullptr;
    void *data = nullptr;
    napi_value ab;
    if (napi_create_arraybuffer(env, (size_t)len, &data, &ab) != napi_ok) {
        napi_throw_error(env, "SM_E_NOMEM", "cannot allocate the host ArrayBuffer");
        return nullptr;
    }
    if (fail(env, ctx, sm_read(ctx, h, off, data, len))) return nullptr;
    return ab;
}
napi_value Copy(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(6)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    uint64_t s = a.u64(1), so = a.u64(2), d = a.u64(3), dof = a.u64(4), n = a.u64(5);
    if (!a.ok || fail(env, ctx, sm_copy(ctx, s, so, d, dof, n))) return nullptr;
    return undefined(env);
}
napi_value Zero(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(4)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    uint64_t h = a.u64(1), off = a.u64(2), n = a.u64(3);
    if (!a.ok || fail(env, ctx, sm_zero(ctx, h, off, n))) return nullptr;
    return undefined(env);
}
napi_value Sync(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(1)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    if (!a.ok || fail(env, ctx, sm_sync(ctx))) return nullptr;
    return undefined(env);
}
napi_value Kernels(napi_env env, napi_callback_info) {
    napi_value arr;
    const int n = sm_kernel_count();
    napi_create_array_with_length(env, (size_t)n, &arr);
    for (int i = 0; i < n; i++) napi_set_element(env, arr, (uint32_t)i, string(env, sm_kernel_name(i)));
    return arr;
}
napi_value Signature(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(1)) return nullptr;
    std::string name = a.str(0);
    if (!a.ok) return nullptr;
    const char *sig = sm_kernel_signature(name.c_str());
    if (!sig) {
        napi_value n;
        napi_get_null(env, &n);
        return n;
    }
    return string(env, sig);
}
// run(ctx, name, [gx, gy, gz], slots): slots is an array of Numbers, one
// 64-bit argument slot per kernel parameter (see sm_run).
napi_value Run(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(4)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    std::string name = a.str(1);
    if (!a.ok) return nullptr;
    uint32_t groups[3];
    for (uint32_t i = 0; i < 3; i++) {
        napi_value v;
        double d = 0;
        if (napi_get_element(env, a.argv[2], i, &v) != napi_ok || napi_get_value_double(env, v, &d) != napi_ok ||
            d < 0 || d > 4294967295.0 || d != (double)(uint64_t)d) {
            napi_throw_range_error(env, nullptr, "groups must be three non-negative integers");
            return nullptr;
        }
        groups[i] = (uint32_t)d;
    }
    uint32_t n = 0;
    if (napi_get_array_length(env, a.argv[3], &n) != napi_ok) {
        type_error(env, "slots must be an array");
        return nullptr;
    }
    std::vector<uint64_t> slots(n);
    for (uint32_t i = 0; i < n; i++) {
        napi_value v;
        double d = 0;
        napi_get_element(env, a.argv[3], i, &v);
        if (napi_get_value_double(env, v, &d) != napi_ok || d < 0 || d > 9007199254740991.0) {
            napi_throw_range_error(env, nullptr, "argument slots must be non-negative safe integers");
            return nullptr;
        }
        slots[i] = (uint64_t)d;
    }
    if (fail(env, ctx, sm_run(ctx, name.c_str(), groups, slots.data(), (int)n))) return nullptr;
    return undefined(env);
}
napi_value MoeWorkspace(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(5)) return nullptr;
    int t = a.i32(0), w = a.i32(1), f = a.i32(2), e = a.i32(3), k = a.i32(4);
    if (!a.ok) return nullptr;
    uint64_t n = 0;
    if (fail(env, nullptr, sm_moe_layer_workspace(t, w, f, e, k, &n))) return nullptr;
    return number(env, (double)n);
}
// moeLayer(ctx, X, tokens, Wr, bias, arena, stride, shared, Wsg, width, ff,
//          experts, topk, Y, ids, weights, workspace, workspaceBytes)
napi_value MoeLayer(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(18)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    uint64_t X = a.u64(1);
    int tokens = a.i32(2);
    uint64_t Wr = a.u64(3), bias = a.u64(4), arena = a.u64(5), stride = a.u64(6), shared = a.u64(7), Wsg = a.u64(8);
    int width = a.i32(9), ff = a.i32(10), experts = a.i32(11), topk = a.i32(12);
    uint64_t Y = a.u64(13), ids = a.u64(14), weights = a.u64(15), ws = a.u64(16), wsb = a.u64(17);
    if (!a.ok) return nullptr;
    if (fail(env, ctx, sm_moe_layer(ctx, X, tokens, Wr, bias, arena, stride, shared, Wsg, width, ff, experts, topk, Y,
                                    ids, weights, ws, wsb)))
        return nullptr;
    return undefined(env);
}
napi_value MoeBlockWorkspace(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(5)) return nullptr;
    int t = a.i32(0), w = a.i32(1), f = a.i32(2), e = a.i32(3), k = a.i32(4);
    if (!a.ok) return nullptr;
    uint64_t n = 0;
    if (fail(env, nullptr, sm_moe_block_workspace(t, w, f, e, k, &n))) return nullptr;
    return number(env, (double)n);
}
// moeBlock(ctx, H, tokens, gamma, eps, Wr, bias, arena, stride, shared, Wsg,
//          width, ff, experts, topk, Hout, ids, weights, workspace, workspaceBytes)
napi_value MoeBlock(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(20)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    uint64_t H = a.u64(1);
    int tokens = a.i32(2);
    uint64_t gamma = a.u64(3);
    const float eps = (float)a.num(4);
    uint64_t Wr = a.u64(5), bias = a.u64(6), arena = a.u64(7), stride = a.u64(8), shared = a.u64(9), Wsg = a.u64(10);
    int width = a.i32(11), ff = a.i32(12), experts = a.i32(13), topk = a.i32(14);
    uint64_t Hout = a.u64(15), ids = a.u64(16), weights = a.u64(17), ws = a.u64(18), wsb = a.u64(19);
    if (!a.ok) return nullptr;
    if (fail(env, ctx, sm_moe_block(ctx, H, tokens, gamma, eps, Wr, bias, arena, stride, shared, Wsg, width, ff, experts,
                                    topk, Hout, ids, weights, ws, wsb)))
        return nullptr;
    return undefined(env);
}
// moeRoute(ctx, X, tokens, width, Wr, bias, experts, topk, logits, ids, weights)
napi_value MoeRoute(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(11)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    uint64_t X = a.u64(1);
    int tokens = a.i32(2), width = a.i32(3);
    uint64_t Wr = a.u64(4), bias = a.u64(5);
    int experts = a.i32(6), topk = a.i32(7);
    uint64_t logits = a.u64(8), ids = a.u64(9), weights = a.u64(10);
    if (!a.ok) return nullptr;
    if (fail(env, ctx, sm_moe_route(ctx, X, tokens, width, Wr, bias, experts, topk, logits, ids, weights)))
        return nullptr;
    return undefined(env);
}
// moeDispatch(ctx, ids, tokens, topk, experts, offsets, rows, parts, where,
//             workspace, workspaceBytes)
napi_value MoeDispatch(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(11)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    uint64_t ids = a.u64(1);
    int tokens = a.i32(2), topk = a.i32(3), experts = a.i32(4);
    uint64_t offsets = a.u64(5), rows = a.u64(6), parts = a.u64(7), where = a.u64(8), ws = a.u64(9), wsb = a.u64(10);
    if (!a.ok) return nullptr;
    if (fail(env, ctx, sm_moe_dispatch(ctx, ids, tokens, topk, experts, offsets, rows, parts, where, ws, wsb)))
        return nullptr;
    return undefined(env);
}
// synthNormal(ctx, dst, offsetBytes, n, seed, stream, sigma) and
// synthUniformPm(ctx, dst, offsetBytes, n, seed, stream, amp)
napi_value SynthNormal(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(7)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    uint64_t d = a.u64(1), off = a.u64(2), n = a.u64(3), seed = a.u64(4), stream = a.u64(5);
    double s = a.num(6);
    if (!a.ok || fail(env, ctx, sm_synth_normal(ctx, d, off, n, seed, stream, s))) return nullptr;
    return undefined(env);
}
napi_value SynthUniformPm(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(7)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    uint64_t d = a.u64(1), off = a.u64(2), n = a.u64(3), seed = a.u64(4), stream = a.u64(5);
    double s = a.num(6);
    if (!a.ok || fail(env, ctx, sm_synth_uniform_pm(ctx, d, off, n, seed, stream, s))) return nullptr;
    return undefined(env);
}
// synthBlobs(ctx, dst, offsetBytes, stride, count, width, ff, seed, firstStream, sigma)
napi_value SynthBlobs(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(10)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    uint64_t d = a.u64(1), off = a.u64(2), stride = a.u64(3);
    int count = a.i32(4), width = a.i32(5), ff = a.i32(6);
    uint64_t seed = a.u64(7), first = a.u64(8);
    double s = a.num(9);
    if (!a.ok || fail(env, ctx, sm_synth_blobs(ctx, d, off, stride, count, width, ff, seed, first, s))) return nullptr;
    return undefined(env);
}
// loadExperts(ctx, path, fileOffset, blobBytes, count, arena, dstOffset, stride, scalesOffset)
napi_value LoadExperts(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(9)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    const std::string path = a.str(1);
    uint64_t foff = a.u64(2), bb = a.u64(3);
    int count = a.i32(4);
    uint64_t arena = a.u64(5), doff = a.u64(6), stride = a.u64(7), soff = a.u64(8);
    if (!a.ok || fail(env, ctx, sm_load_experts(ctx, path.c_str(), foff, bb, count, arena, doff, stride, soff)))
        return nullptr;
    return undefined(env);
}
napi_value EventRecord(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(2)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    int slot = a.i32(1);
    if (!a.ok || fail(env, ctx, sm_event_record(ctx, slot))) return nullptr;
    return undefined(env);
}
napi_value EventElapsed(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(3)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    int s0 = a.i32(1), s1 = a.i32(2);
    float ms = 0;
    if (!a.ok || fail(env, ctx, sm_event_elapsed(ctx, s0, s1, &ms))) return nullptr;
    return number(env, ms);
}
napi_value GraphBegin(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(1)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    if (!a.ok || fail(env, ctx, sm_graph_begin(ctx))) return nullptr;
    return undefined(env);
}
napi_value GraphEnd(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(1)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    int id = -1;
    if (!a.ok || fail(env, ctx, sm_graph_end(ctx, &id))) return nullptr;
    return number(env, id);
}
napi_value GraphLaunch(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(2)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    int id = a.i32(1);
    if (!a.ok || fail(env, ctx, sm_graph_launch(ctx, id))) return nullptr;
    return undefined(env);
}
napi_value GraphFree(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(2)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    int id = a.i32(1);
    if (!a.ok || fail(env, ctx, sm_graph_free(ctx, id))) return nullptr;
    return undefined(env);
}

// Clears the single-launch decode layer's fault (sm_fused_reset).
napi_value FusedReset(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(1)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    if (!a.ok || fail(env, ctx, sm_fused_reset(ctx))) return nullptr;
    return undefined(env);
}

// prefetchRouter(ctx, Wr, rows, width): the router matrix of the layer call
// after the next one (0: none), pulled into L2 by the next single-launch decode layer
napi_value PrefetchRouter(napi_env env, napi_callback_info info) {
    Args a(env, info);
    if (!a.need(4)) return nullptr;
    sm_ctx *ctx = a.ctx(0);
    uint64_t Wr = a.u64(1);
    int rows = a.i32(2), width = a.i32(3);
    if (!a.ok || fail(env, ctx, sm_prefetch_router(ctx, Wr, rows, width))) return nullptr;
    return undefined(env);
}

napi_value ModuleInit(napi_env env, napi_value exports) {
    struct Fn {
        const char *name;
        napi_callback cb;
    } fns[] = {{"init", Init},
               {"shutdown", Shutdown},
               {"lastError", LastError},
               {"info", Info},
               {"alloc", Alloc},
               {"free", Free},
               {"size", Size},
               {"write", Write},
               {"read", Read},
               {"copy", Copy},
               {"zero", Zero},
               {"sync", Sync},
               {"kernels", Kernels},
               {"signature", Signature},
               {"run", Run},
               {"moeWorkspace", MoeWorkspace},
               {"moeLayer", MoeLayer},
               {"moeBlockWorkspace", MoeBlockWorkspace},
               {"moeBlock", MoeBlock},
               {"moeRoute", MoeRoute},
               {"moeDispatch", MoeDispatch},
               {"synthNormal", SynthNormal},
               {"synthUniformPm", SynthUniformPm},
               {"synthBlobs", SynthBlobs},
               {"loadExperts", LoadExperts},
               {"eventRecord", EventRecord},
               {"eventElapsed", EventElapsed},
               {"graphBegin", GraphBegin},
               {"graphEnd", GraphEnd},
               {"graphLaunch", GraphLaunch},
               {"graphFree", GraphFree},
               {"fusedReset", FusedReset},
               {"prefetchRouter", PrefetchRouter}};
    for (const Fn &f : fns) {
        napi_value fn;
        napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &fn);
        napi_set_named_property(env, exports, f.name, fn);
    }
    return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, ModuleInit)
