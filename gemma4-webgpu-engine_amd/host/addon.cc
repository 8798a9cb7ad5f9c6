// N-API addon: the Node side of the g4w8a8 C ABI. The reference engine's host is TypeScript in a
// browser; this is the binding a Node host (index.js) uses to reach the same operator seam on
// MI355X. Device addresses travel as JS numbers (GPU virtual addresses fit in 53 bits). Every
// non-zero status becomes a thrown Error carrying g4_last_error().
#define NAPI_VERSION 8
#include <node_api.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/g4decode.h"
#include "../../include/g4w8a8.h"

namespace {

bool throw_status(napi_env env, int status) {
    if (status == G4_OK) return false;
    std::string msg = g4_last_error();
    if (msg.empty()) msg = "g4w8a8 call failed with status " + std::to_string(status);
    napi_value err, m, code;
    napi_create_string_utf8(env, msg.c_str(), msg.size(), &m);
    napi_create_error(env, nullptr, m, &err);
    napi_create_int32(env, status, &code);
    napi_set_named_property(env, err, "status", code);
    napi_throw(env, err);
    return true;
}

void throw_type(napi_env env, const char *msg) { napi_throw_type_error(env, nullptr, msg); }

struct Args {
    napi_env env;
    std::vector<napi_value> v;
    Args(napi_env e, napi_callback_info info, size_t n) : env(e), v(n) {
        size_t argc = n;
        napi_get_cb_info(e, info, &argc, v.data(), nullptr, nullptr);
        if (argc < n) v.resize(argc);
    }
    size_t size() const { return v.size(); }
    double num(size_t i, double dflt = 0) const {
        if (i >= v.size()) return dflt;
        napi_valuetype t;
        napi_typeof(env, v[i], &t);
        if (t == napi_undefined || t == napi_null) return dflt;
        double d = dflt;
        napi_get_value_double(env, v[i], &d);
        return d;
    }
    int i32(size_t i, int dflt = 0) const { return (int)num(i, dflt); }
    void *ptr(size_t i) const { return reinterpret_cast<void *>((uintptr_t)num(i, 0)); }
};

napi_value make_num(napi_env env, double d) {
    napi_value r;
    napi_create_double(env, d, &r);
    return r;
}

napi_value undefined(napi_env env) {
    napi_value r;
    napi_get_undefined(env, &r);
    return r;
}

// Reads a JS array of numbers (addresses or values).
std::vector<double> num_array(napi_env env, napi_value arr) {
    std::vector<double> out;
    bool is_arr = false;
    napi_is_array(env, arr, &is_arr);
    if (!is_arr) return out;
    uint32_t n = 0;
    napi_get_array_length(env, arr, &n);
    out.resize(n);
    for (uint32_t i = 0; i < n; ++i) {
        napi_value e;
        napi_get_element(env, arr, i, &e);
        napi_get_value_double(env, e, &out[i]);
    }
    return out;
}

double prop(napi_env env, napi_value obj, const char *name, double dflt = 0) {
    bool has = false;
    napi_has_named_property(env, obj, name, &has);
    if (!has) return dflt;
    napi_value v;
    napi_get_named_property(env, obj, name, &v);
    napi_valuetype t;
    napi_typeof(env, v, &t);
    if (t != napi_number) return dflt;
    double d = dflt;
    napi_get_value_double(env, v, &d);
    return d;
}

void set_num(napi_env env, napi_value obj, const char *name, double d) {
    napi_set_named_property(env, obj, name, make_num(env, d));
}

// Host bytes of a TypedArray, ArrayBuffer or Buffer.
bool host_bytes(napi_env env, napi_value v, void **data, size_t *len) {
    bool is;
    napi_is_typedarray(env, v, &is);
    if (is) {
        napi_typedarray_type type;
        size_t length, offset;
        napi_value ab;
        void *base;
        napi_get_typedarray_info(env, v, &type, &length, &base, &ab, &offset);
        size_t elem = 1;
        switch (type) {
            case napi_int16_array: case napi_uint16_array: elem = 2; break;
            case napi_int32_array: case napi_uint32_array: case napi_float32_array: elem = 4; break;
            case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: elem = 8; break;
            default: elem = 1;
        }
        *data = base;
        *len = length * elem;
        return true;
    }
    napi_is_arraybuffer(env, v, &is);
    if (is) {
        napi_get_arraybuffer_info(env, v, data, len);
        return true;
    }
    napi_is_buffer(env, v, &is);
    if (is) {
        napi_get_buffer_info(env, v, data, len);
        return true;
    }
    return false;
}

// ---- memory and sync ----

napi_value DeviceCount(napi_env env, napi_callback_info) {
    int n = 0;
    g4_device_count(&n);
    return make_num(env, n);
}

napi_value SetDevice(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    if (throw_status(env, g4_set_device(a.i32(0)))) return nullptr;
    return undefined(env);
}

napi_value Malloc(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    void *p = nullptr;
    if (throw_status(env, g4_malloc(&p, (size_t)a.num(0)))) return nullptr;
    return make_num(env, (double)(uintptr_t)p);
}

napi_value Free(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    if (throw_status(env, g4_free(a.ptr(0)))) return nullptr;
    return undefined(env);
}

napi_value Upload(napi_env env, napi_callback_info info) {
    Args a(env, info, 3);
    void *data;
    size_t len;
    if (a.size() < 2 || !host_bytes(env, a.v[1], &data, &len)) {
        throw_type(env, "upload(ptr, TypedArray|ArrayBuffer|Buffer[, stream])");
        return nullptr;
    }
    if (throw_status(env, g4_memcpy_h2d(a.ptr(0), data, len, a.ptr(2)))) return nullptr;
    return undefined(env);
}

napi_value Download(napi_env env, napi_callback_info info) {
    Args a(env, info, 3);
    size_t len = (size_t)a.num(1);
    void *data = nullptr;
    napi_value ab;
    napi_create_arraybuffer(env, len, &data, &ab);
    if (throw_status(env, g4_memcpy_d2h(data, a.ptr(0), len, a.ptr(2)))) return nullptr;
    return ab;
}

napi_value Fill(napi_env env, napi_callback_info info) {
    Args a(env, info, 4);
    if (throw_status(env, g4_fill_u8(a.ptr(0), (uint8_t)a.i32(1), (size_t)a.num(2), a.ptr(3))))
        return nullptr;
    return undefined(env);
}

napi_value Synchronize(napi_env env, napi_callback_info) {
    if (throw_status(env, g4_device_synchronize())) return nullptr;
    return undefined(env);
}

napi_value LastError(napi_env env, napi_callback_info) {
    napi_value s;
    const char *m = g4_last_error();
    napi_create_string_utf8(env, m, strlen(m), &s);
    return s;
}

// ---- the entry points (argument order = the C ABI's; the stream is the optional last
// argument, a handle from streamCreate, omitted or 0 = the default stream) ----

napi_value Qgemv(napi_env env, napi_callback_info info) {
    Args a(env, info, 13);
    int st = g4_qgemv(a.i32(0), a.ptr(1), (const float *)a.ptr(2), a.ptr(3), a.i32(4), a.ptr(5),
                      a.i32(6), a.i32(7), a.i32(8), a.i32(9, 1), (float)a.num(10), (float)a.num(11),
                      a.ptr(12));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

napi_value Qgemm(napi_env env, napi_callback_info info) {
    Args a(env, info, 13);
    int st = g4_qgemm(a.i32(0), a.ptr(1), (const float *)a.ptr(2), a.ptr(3), a.i32(4), a.ptr(5),
                      a.i32(6), a.i32(7), a.i32(8), a.i32(9, 1), (float)a.num(10), (float)a.num(11),
                      a.ptr(12));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

napi_value Linear(napi_env env, napi_callback_info info) {
    Args a(env, info, 13);
    int st = g4_linear(a.i32(0), a.ptr(1), (const float *)a.ptr(2), a.ptr(3), a.i32(4), a.ptr(5),
                       a.i32(6), a.i32(7), a.i32(8), a.i32(9, 1), (float)a.num(10),
                       (float)a.num(11), a.ptr(12));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

napi_value KernelForShape(napi_env env, napi_callback_info info) {
    Args a(env, info, 4);
    char buf[64];
    if (throw_status(env, g4_kernel_for_shape(a.i32(0), a.i32(1), a.i32(2), a.i32(3), buf, 64)))
        return nullptr;
    napi_value s;
    napi_create_string_utf8(env, buf, strlen(buf), &s);
    return s;
}

// projectionBatch(bits, [w], [s], x, xKind, [out], outKind, [rows], [inScales], [outScales], k)
napi_value ProjectionBatch(napi_env env, napi_callback_info info) {
    Args a(env, info, 12);
    if (a.size() < 11) {
        throw_type(env, "projectionBatch needs 11 arguments");
        return nullptr;
    }
    auto w = num_array(env, a.v[1]), s = num_array(env, a.v[2]), o = num_array(env, a.v[5]);
    auto rows = num_array(env, a.v[7]), ins = num_array(env, a.v[8]), outs = num_array(env, a.v[9]);
    const size_t n = w.size();
    if (s.size() != n || o.size() != n || rows.size() != n || ins.size() != n || outs.size() != n) {
        throw_type(env, "projectionBatch: per-projection arrays must have equal lengths");
        return nullptr;
    }
    std::vector<const void *> wp(n);
    std::vector<const float *> sp(n);
    std::vector<void *> op(n);
    std::vector<int> rp(n);
    std::vector<float> ip(n), up(n);
    for (size_t i = 0; i < n; ++i) {
        wp[i] = reinterpret_cast<const void *>((uintptr_t)w[i]);
        sp[i] = reinterpret_cast<const float *>((uintptr_t)s[i]);
        op[i] = reinterpret_cast<void *>((uintptr_t)o[i]);
        rp[i] = (int)rows[i];
        ip[i] = (float)ins[i];
        up[i] = (float)outs[i];
    }
    int st = g4_projection_batch(a.i32(0), (int)n, wp.data(), sp.data(), a.ptr(3), a.i32(4),
                                 op.data(), a.i32(6), rp.data(), ip.data(), up.data(), a.i32(10),
                                 a.ptr(11));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// qgemvGrouped([{wq, scales, x, dst, bits, xKind, outKind, k, numRows, inScale, outScale}])
napi_value QgemvGrouped(napi_env env, napi_callback_info info) {
    Args a(env, info, 2);
    bool is_arr = false;
    if (a.size() < 1 || (napi_is_array(env, a.v[0], &is_arr), !is_arr)) {
        throw_type(env, "qgemvGrouped(descs: object[])");
        return nullptr;
    }
    uint32_t n = 0;
    napi_get_array_length(env, a.v[0], &n);
    std::vector<g4_gemv_desc> d(n);
    for (uint32_t i = 0; i < n; ++i) {
        napi_value o;
        napi_get_element(env, a.v[0], i, &o);
        d[i].wq = reinterpret_cast<const void *>((uintptr_t)prop(env, o, "wq"));
        d[i].scales = reinterpret_cast<const float *>((uintptr_t)prop(env, o, "scales"));
        d[i].x = reinterpret_cast<const void *>((uintptr_t)prop(env, o, "x"));
        d[i].dst = reinterpret_cast<void *>((uintptr_t)prop(env, o, "dst"));
        d[i].bits = (int)prop(env, o, "bits", 4);
        d[i].x_kind = (int)prop(env, o, "xKind", G4_KIND_F16);
        d[i].out_kind = (int)prop(env, o, "outKind", G4_KIND_I8);
        d[i].k = (int)prop(env, o, "k");
        d[i].num_rows = (int)prop(env, o, "numRows");
        d[i].in_scale = (float)prop(env, o, "inScale");
        d[i].out_scale = (float)prop(env, o, "outScale");
    }
    if (throw_status(env, g4_qgemv_grouped(d.data(), (int)n, a.ptr(1)))) return nullptr;
    return undefined(env);
}

// Descriptors of a grouped GEMV from an array of plain objects (the qgemvGrouped shape).
bool gemv_descs(napi_env env, napi_value arr, std::vector<g4_gemv_desc> &d) {
    bool is_arr = false;
    if (napi_is_array(env, arr, &is_arr) != napi_ok || !is_arr) return false;
    uint32_t n = 0;
    napi_get_array_length(env, arr, &n);
    d.resize(n);
    for (uint32_t i = 0; i < n; ++i) {
        napi_value o;
        napi_get_element(env, arr, i, &o);
        d[i].wq = reinterpret_cast<const void *>((uintptr_t)prop(env, o, "wq"));
        d[i].scales = reinterpret_cast<const float *>((uintptr_t)prop(env, o, "scales"));
        d[i].x = reinterpret_cast<const void *>((uintptr_t)prop(env, o, "x"));
        d[i].dst = reinterpret_cast<void *>((uintptr_t)prop(env, o, "dst"));
        d[i].bits = (int)prop(env, o, "bits", 4);
        d[i].x_kind = (int)prop(env, o, "xKind", G4_KIND_F16);
        d[i].out_kind = (int)prop(env, o, "outKind", G4_KIND_I8);
        d[i].k = (int)prop(env, o, "k");
        d[i].num_rows = (int)prop(env, o, "numRows");
        d[i].in_scale = (float)prop(env, o, "inScale");
        d[i].out_scale = (float)prop(env, o, "outScale");
    }
    return true;
}

// qgemvPlanCreate(descs) -> handle; qgemvPlanLaunch(handle); qgemvPlanDestroy(handle).
napi_value QgemvPlanCreate(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    std::vector<g4_gemv_desc> d;
    if (a.size() < 1 || !gemv_descs(env, a.v[0], d)) {
        throw_type(env, "qgemvPlanCreate(descs: object[])");
        return nullptr;
    }
    g4_gemv_plan *plan = nullptr;
    if (throw_status(env, g4_qgemv_plan_create(d.data(), (int)d.size(), &plan))) return nullptr;
    return make_num(env, (double)(uintptr_t)plan);
}

napi_value QgemvPlanLaunch(napi_env env, napi_callback_info info) {
    Args a(env, info, 2);
    if (throw_status(env, g4_qgemv_plan_launch(reinterpret_cast<const g4_gemv_plan *>(a.ptr(0)),
                                               a.ptr(1))))
        return nullptr;
    return undefined(env);
}

napi_value QgemvPlanDestroy(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    if (throw_status(env, g4_qgemv_plan_destroy(reinterpret_cast<g4_gemv_plan *>(a.ptr(0)))))
        return nullptr;
    return undefined(env);
}

napi_value QgemvSplit(napi_env env, napi_callback_info info) {
    Args a(env, info, 12);
    int st = g4_qgemv_split(a.i32(0), a.ptr(1), (const float *)a.ptr(2), a.ptr(3), a.i32(4),
                            (float *)a.ptr(5), a.i32(6), a.i32(7), a.i32(8), a.i32(9),
                            (float)a.num(10), a.ptr(11));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// qgemv-4bit-gelu / qgemv-8bit-gelu: (bits, wq, scales, gate, gateKind, up, upKind, upOffset,
// dst, outKind, k, numRows, inScale, outScale[, gateScale, upScale])
napi_value QgemvGelu(napi_env env, napi_callback_info info) {
    Args a(env, info, 17);
    g4_gelu_act act{a.ptr(5), a.i32(6), (float)a.num(14), (float)a.num(15), (int64_t)a.num(7)};
    int st = g4_qgemv_gelu(a.i32(0), a.ptr(1), (const float *)a.ptr(2), a.ptr(3), a.i32(4), &act,
                           a.ptr(8), a.i32(9), a.i32(10), a.i32(11), (float)a.num(12),
                           (float)a.num(13), a.ptr(16));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// tile8u (qgemv.ts:870-1015): (wq, tileWq, k, numRows[, stream]) and (tileWq, scales, x, xKind,
// up, upKind, upOffset, dst, outKind, k, numRows, inScale, outScale[, gateScale, upScale, stream]);
// up null: no gelu prologue.
napi_value Tile8uRepack(napi_env env, napi_callback_info info) {
    Args a(env, info, 5);
    if (throw_status(env, g4_tile8u_repack(a.ptr(0), a.ptr(1), a.i32(2), a.i32(3), a.ptr(4)))) return nullptr;
    return undefined(env);
}

napi_value QgemvTile8u(napi_env env, napi_callback_info info) {
    Args a(env, info, 16);
    g4_gelu_act act{a.ptr(4), a.i32(5), (float)a.num(13), (float)a.num(14), (int64_t)a.num(6)};
    int st = g4_qgemv_tile8u(a.ptr(0), (const float *)a.ptr(1), a.ptr(2), a.i32(3), act.up ? &act : nullptr,
                             a.ptr(7), a.i32(8), a.i32(9), a.i32(10), (float)a.num(11), (float)a.num(12),
                             a.ptr(15));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// qgemv-4bit-gelu-exact-split: (bits, wq, scales, gate, gateKind, up, upKind, upOffset, partials,
// k, numRows, kSplits, exact, inScale[, gateScale, upScale])
napi_value QgemvGeluSplit(napi_env env, napi_callback_info info) {
    Args a(env, info, 17);
    g4_gelu_act act{a.ptr(5), a.i32(6), (float)a.num(14), (float)a.num(15), (int64_t)a.num(7)};
    int st = g4_qgemv_gelu_split(a.i32(0), a.ptr(1), (const float *)a.ptr(2), a.ptr(3), a.i32(4),
                                 &act, (float *)a.ptr(8), a.i32(9), a.i32(10), a.i32(11),
                                 a.i32(12), (float)a.num(13), a.ptr(16));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// qgemv-4bit-gelu-m2 / qgemv-8bit-gelu-m2: (bits, wq, scales, gate, gateKind, up, upKind,
// upOffset, dst, outKind, k, numRows, cols, inScale, outScale[, gateScale, upScale, stream])
napi_value QgemvGeluM2(napi_env env, napi_callback_info info) {
    Args a(env, info, 18);
    g4_gelu_act act{a.ptr(5), a.i32(6), (float)a.num(15), (float)a.num(16), (int64_t)a.num(7)};
    int st = g4_qgemv_gelu_m2(a.i32(0), a.ptr(1), (const float *)a.ptr(2), a.ptr(3), a.i32(4), &act,
                              a.ptr(8), a.i32(9), a.i32(10), a.i32(11), a.i32(12),
                              (float)a.num(13), (float)a.num(14), a.ptr(17));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// ple-gate-split: (wq, scales, x, xKind, partials, k, numRows, kSplits, inScale[, stream])
napi_value PleGateSplit(napi_env env, napi_callback_info info) {
    Args a(env, info, 10);
    int st = g4_ple_gate_split(a.ptr(0), (const float *)a.ptr(1), a.ptr(2), a.i32(3),
                               (float *)a.ptr(4), a.i32(5), a.i32(6), a.i32(7), (float)a.num(8),
                               a.ptr(9));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// ple-fold-projection: (wq, scales, gateParts, gateScales, kSplits, gateInScale, gateOutScale,
// up, upKind, upOffset, dst, outKind, k, numRows, inScale, outScale[, upScale, stream])
napi_value PleFoldProjection(napi_env env, napi_callback_info info) {
    Args a(env, info, 18);
    g4_gelu_act act{a.ptr(7), a.i32(8), 0.0f, (float)a.num(16), (int64_t)a.num(9)};
    int st = g4_ple_fold_projection(a.ptr(0), (const float *)a.ptr(1), (const float *)a.ptr(2),
                                    (const float *)a.ptr(3), a.i32(4), (float)a.num(5),
                                    (float)a.num(6), &act, a.ptr(10), a.i32(11), a.i32(12),
                                    a.i32(13), (float)a.num(14), (float)a.num(15), a.ptr(17));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// gelu-mul: (gate, up, dst, count, srqScale[, stream])
napi_value GeluMulF32(napi_env env, napi_callback_info info) {
    Args a(env, info, 6);
    int st = g4_gelu_mul_f32((const float *)a.ptr(0), (const float *)a.ptr(1), (float *)a.ptr(2),
                             (int64_t)a.num(3), (float)a.num(4), a.ptr(5));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

napi_value QgemvMerge(napi_env env, napi_callback_info info) {
    Args a(env, info, 7);
    int st = g4_qgemv_merge((const float *)a.ptr(0), a.ptr(1), a.i32(2), a.i32(3), a.i32(4),
                            (float)a.num(5), a.ptr(6));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

napi_value QgemvExactMerge(napi_env env, napi_callback_info info) {
    Args a(env, info, 9);
    int st = g4_qgemv_exact_merge((const float *)a.ptr(0), (const float *)a.ptr(1), a.ptr(2),
                                  a.i32(3), a.i32(4), a.i32(5), (float)a.num(6), (float)a.num(7),
                                  a.ptr(8));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

napi_value SrqQuantize(napi_env env, napi_callback_info info) {
    Args a(env, info, 6);
    int st = g4_srq_quantize(a.ptr(0), a.i32(1), (int8_t *)a.ptr(2), (int64_t)a.num(3),
                             (float)a.num(4), a.ptr(5));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// pleGather(codes, scales, scaleKind, ids, dst, outKind, slots, cols, groupSize, groupsPerRow,
//           sliced, sliceStartRow, sliceRowCount)
napi_value PleGather(napi_env env, napi_callback_info info) {
    Args a(env, info, 14);
    int st = g4_ple_gather(a.ptr(0), a.ptr(1), a.i32(2), (const int32_t *)a.ptr(3), a.ptr(4),
                           a.i32(5), a.i32(6), a.i32(7), a.i32(8), a.i32(9), a.i32(10),
                           (int64_t)a.num(11), (int64_t)a.num(12), a.ptr(13));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// pleGatherSplit([codes], [starts], [counts], scales, scaleKind, ids, dst, outKind, slots, cols,
//                groupSize, groupsPerRow)
napi_value PleGatherSplit(napi_env env, napi_callback_info info) {
    Args a(env, info, 13);
    if (a.size() < 12) {
        throw_type(env, "pleGatherSplit needs 12 arguments");
        return nullptr;
    }
    auto c = num_array(env, a.v[0]), s = num_array(env, a.v[1]), n = num_array(env, a.v[2]);
    if (s.size() != c.size() || n.size() != c.size()) {
        throw_type(env, "pleGatherSplit: codes, starts and counts must have equal lengths");
        return nullptr;
    }
    std::vector<const void *> cp(c.size());
    std::vector<int64_t> sp(c.size()), np(c.size());
    for (size_t i = 0; i < c.size(); ++i) {
        cp[i] = reinterpret_cast<const void *>((uintptr_t)c[i]);
        sp[i] = (int64_t)s[i];
        np[i] = (int64_t)n[i];
    }
    int st = g4_ple_gather_split(cp.data(), sp.data(), np.data(), (int)c.size(), a.ptr(3),
                                 a.i32(4), (const int32_t *)a.ptr(5), a.ptr(6), a.i32(7), a.i32(8),
                                 a.i32(9), a.i32(10), a.i32(11), a.ptr(12));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// A TableSplitPlan (tableSplit.ts:90-118) as a JS object with its slices.
napi_value plan_object(napi_env env, const g4_table_split_plan &plan,
                       const std::vector<g4_table_slice> &slices) {
    napi_value out, arr;
    napi_create_object(env, &out);
    set_num(env, out, "rows", (double)plan.rows);
    set_num(env, out, "rowBytes", (double)plan.row_bytes);
    set_num(env, out, "totalBytes", (double)plan.total_bytes);
    set_num(env, out, "limitBytes", (double)plan.limit_bytes);
    set_num(env, out, "rowsPerSlice", (double)plan.rows_per_slice);
    set_num(env, out, "storageBindingsPerDispatch", (double)plan.storage_bindings_per_dispatch);
    set_num(env, out, "bindingBudget", (double)plan.binding_budget);
    set_num(env, out, "dispatchesPerGather", (double)plan.dispatches_per_gather);
    napi_value b;
    napi_get_boolean(env, plan.single != 0, &b);
    napi_set_named_property(env, out, "single", b);
    napi_get_boolean(env, plan.feasible != 0, &b);
    napi_set_named_property(env, out, "feasible", b);
    const int64_t n = plan.num_slices < (int64_t)slices.size() ? plan.num_slices : (int64_t)slices.size();
    napi_create_array_with_length(env, (size_t)n, &arr);
    for (int64_t i = 0; i < n; ++i) {
        napi_value so;
        napi_create_object(env, &so);
        set_num(env, so, "index", (double)slices[i].index);
        set_num(env, so, "startRow", (double)slices[i].start_row);
        set_num(env, so, "rowCount", (double)slices[i].row_count);
        set_num(env, so, "byteOffset", (double)slices[i].byte_offset);
        set_num(env, so, "byteLength", (double)slices[i].byte_length);
        napi_set_element(env, arr, (uint32_t)i, so);
    }
    napi_set_named_property(env, out, "slices", arr);
    return out;
}

// planTableSplit({rows, rowBytes, maxStorageBufferBindingSize, maxBufferSize,
//                 maxStorageBuffersPerShaderStage, maxSliceBytes?}) -> plan with slices
napi_value PlanTableSplit(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    if (a.size() < 1) {
        throw_type(env, "planTableSplit(input)");
        return nullptr;
    }
    napi_value in = a.v[0];
    g4_table_split_input inp{};
    inp.rows = (int64_t)prop(env, in, "rows");
    inp.row_bytes = (int64_t)prop(env, in, "rowBytes");
    inp.max_storage_buffer_binding_size = (int64_t)prop(env, in, "maxStorageBufferBindingSize");
    inp.max_buffer_size = (int64_t)prop(env, in, "maxBufferSize");
    inp.max_storage_buffers_per_shader_stage =
        (int64_t)prop(env, in, "maxStorageBuffersPerShaderStage");
    inp.max_slice_bytes = (int64_t)prop(env, in, "maxSliceBytes", 0);
    g4_table_split_plan plan{};
    std::vector<g4_table_slice> slices(1 << 16);
    if (throw_status(env, g4_plan_table_split(&inp, &plan, slices.data(), (int64_t)slices.size())))
        return nullptr;
    return plan_object(env, plan, slices);
}

// planGatherSplit(rows, codeRowBytes, scalesPerRow, {maxStorageBufferBindingSize, maxBufferSize,
// maxStorageBuffersPerShaderStage}) -> {codes, scales, scalesSingle} (tableSplit.ts:257-287).
napi_value PlanGatherSplit(napi_env env, napi_callback_info info) {
    Args a(env, info, 4);
    if (a.size() < 4) {
        throw_type(env, "planGatherSplit(rows, codeRowBytes, scalesPerRow, limits)");
        return nullptr;
    }
    g4_gather_limits lim{};
    lim.max_storage_buffer_binding_size = (int64_t)prop(env, a.v[3], "maxStorageBufferBindingSize");
    lim.max_buffer_size = (int64_t)prop(env, a.v[3], "maxBufferSize");
    lim.max_storage_buffers_per_shader_stage =
        (int64_t)prop(env, a.v[3], "maxStorageBuffersPerShaderStage");
    g4_gather_split_plans plans{};
    std::vector<g4_table_slice> cs(1 << 16), ss(1 << 16);
    if (throw_status(env, g4_plan_gather_split((int64_t)a.num(0), (int64_t)a.num(1),
                                               (int64_t)a.num(2), &lim, &plans, cs.data(),
                                               (int64_t)cs.size(), ss.data(), (int64_t)ss.size())))
        return nullptr;
    napi_value out, b;
    napi_create_object(env, &out);
    napi_set_named_property(env, out, "codes", plan_object(env, plans.codes, cs));
    napi_set_named_property(env, out, "scales", plan_object(env, plans.scales, ss));
    napi_get_boolean(env, plans.scales_single != 0, &b);
    napi_set_named_property(env, out, "scalesSingle", b);
    return out;
}


// ---- streams, events and graphs (runtime.ts's queue and its cached per-token encode) ----

napi_value StreamCreate(napi_env env, napi_callback_info) {
    void *st = nullptr;
    if (throw_status(env, g4_stream_create(&st))) return nullptr;
    return make_num(env, (double)(uintptr_t)st);
}

napi_value StreamDestroy(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    if (throw_status(env, g4_stream_destroy(a.ptr(0)))) return nullptr;
    return undefined(env);
}

napi_value StreamSynchronize(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    if (throw_status(env, g4_stream_synchronize(a.ptr(0)))) return nullptr;
    return undefined(env);
}

napi_value EventCreate(napi_env env, napi_callback_info) {
    void *e = nullptr;
    if (throw_status(env, g4_event_create(&e))) return nullptr;
    return make_num(env, (double)(uintptr_t)e);
}

napi_value EventRecord(napi_env env, napi_callback_info info) {
    Args a(env, info, 2);
    if (throw_status(env, g4_event_record(a.ptr(0), a.ptr(1)))) return nullptr;
    return undefined(env);
}

napi_value EventElapsedMs(napi_env env, napi_callback_info info) {
    Args a(env, info, 2);
    float ms = 0;
    if (throw_status(env, g4_event_elapsed_ms(&ms, a.ptr(0), a.ptr(1)))) return nullptr;
    return make_num(env, ms);
}

napi_value EventDestroy(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    if (throw_status(env, g4_event_destroy(a.ptr(0)))) return nullptr;
    return undefined(env);
}

napi_value GraphBeginCapture(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    if (throw_status(env, g4_graph_begin_capture(a.ptr(0)))) return nullptr;
    return undefined(env);
}

napi_value GraphEndCapture(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    void *g = nullptr;
    if (throw_status(env, g4_graph_end_capture(a.ptr(0), &g))) return nullptr;
    return make_num(env, (double)(uintptr_t)g);
}

napi_value GraphLaunch(napi_env env, napi_callback_info info) {
    Args a(env, info, 2);
    if (throw_status(env, g4_graph_launch(a.ptr(0), a.ptr(1)))) return nullptr;
    return undefined(env);
}

napi_value GraphDestroy(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    if (throw_status(env, g4_graph_destroy(a.ptr(0)))) return nullptr;
    return undefined(env);
}

// ---- asynchronous waits (the reference's mapAsync readback, runtime.ts:866-878) ----
//
// The wait runs on a libuv worker thread and settles a Promise on the JS thread, so the event loop
// keeps running (the host can encode the next step) while the device works. g4_last_error is per
// thread: the worker copies its message for the settle.

struct AsyncWait {
    napi_async_work work = nullptr;
    napi_deferred deferred = nullptr;
    napi_ref buffer = nullptr;  // the ArrayBuffer a download fills (null: a plain synchronize)
    void *host = nullptr;       // the ArrayBuffer's bytes
    void *staging = nullptr;    // pinned host memory the copy lands in (a download)
    void *done = nullptr;       // event recorded behind the copy (a download)
    size_t bytes = 0;
    void *stream = nullptr;
    int status = G4_OK;
    std::string message;

    ~AsyncWait() {
        if (done) g4_event_destroy(done);
        if (staging) g4_host_free(staging);
    }
};

// The worker: a download waits for its copy's event, then moves the pinned bytes into the
// ArrayBuffer; a synchronize waits for the stream.
void async_execute(napi_env, void *data) {
    AsyncWait *w = static_cast<AsyncWait *>(data);
    if (w->buffer) {
        w->status = g4_event_synchronize(w->done);
        if (w->status == G4_OK && w->bytes) memcpy(w->host, w->staging, w->bytes);
    } else {
        w->status = g4_stream_synchronize(w->stream);
    }
    if (w->status != G4_OK) w->message = g4_last_error();
}

void async_complete(napi_env env, napi_status, void *data) {
    AsyncWait *w = static_cast<AsyncWait *>(data);
    if (w->status == G4_OK) {
        napi_value v;
        if (w->buffer) napi_get_reference_value(env, w->buffer, &v);
        else napi_get_undefined(env, &v);
        napi_resolve_deferred(env, w->deferred, v);
    } else {
        std::string msg = w->message.empty() ? "g4w8a8 async wait failed" : w->message;
        napi_value err, m, code;
        napi_create_string_utf8(env, msg.c_str(), msg.size(), &m);
        napi_create_error(env, nullptr, m, &err);
        napi_create_int32(env, w->status, &code);
        napi_set_named_property(env, err, "status", code);
        napi_reject_deferred(env, w->deferred, err);
    }
    if (w->buffer) napi_delete_reference(env, w->buffer);
    napi_delete_async_work(env, w->work);
    delete w;
}

napi_value queue_wait(napi_env env, AsyncWait *w) {
    napi_value promise, name;
    napi_create_promise(env, &w->deferred, &promise);
    napi_create_string_utf8(env, "g4w8a8.wait", NAPI_AUTO_LENGTH, &name);
    napi_create_async_work(env, nullptr, name, async_execute, async_complete, w, &w->work);
    napi_queue_async_work(env, w->work);
    return promise;
}

// synchronizeAsync(stream?) -> Promise<void>: resolves once the stream's work has finished.
napi_value SynchronizeAsync(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    AsyncWait *w = new AsyncWait();
    w->stream = a.ptr(0);
    return queue_wait(env, w);
}

// downloadAsync(ptr, bytes, stream?) -> Promise<ArrayBuffer>: the device-to-host copy is enqueued
// here, on the calling thread, into pinned staging memory, with an event behind it. So it is
// ordered after the work already enqueued on the stream and before anything the caller enqueues
// next (a later step rewriting the same buffer cannot overtake it); the worker only waits for the
// event and copies the staged bytes into the ArrayBuffer.
napi_value DownloadAsync(napi_env env, napi_callback_info info) {
    Args a(env, info, 3);
    AsyncWait *w = new AsyncWait();
    const void *device = a.ptr(0);
    w->bytes = (size_t)a.num(1);
    w->stream = a.ptr(2);
    int st = g4_host_alloc(&w->staging, w->bytes);
    if (st == G4_OK) st = g4_memcpy_d2h_async(w->staging, device, w->bytes, w->stream);
    if (st == G4_OK) st = g4_event_create(&w->done);
    if (st == G4_OK) st = g4_event_record(w->done, w->stream);
    if (st != G4_OK) {
        throw_status(env, st);  // reads the message before the cleanup below runs
        delete w;
        return nullptr;
    }
    napi_value ab;
    napi_create_arraybuffer(env, w->bytes, &w->host, &ab);
    napi_create_reference(env, ab, 1, &w->buffer);
    return queue_wait(env, w);
}

// ---- the decode runner (include/g4decode.h) ----

uint64_t u64_arg(napi_env env, napi_value v) {
    napi_valuetype t;
    napi_typeof(env, v, &t);
    if (t == napi_string) {
        char buf[32] = {0};
        size_t n = 0;
        napi_get_value_string_utf8(env, v, buf, sizeof buf, &n);
        return strtoull(buf, nullptr, 10);
    }
    if (t == napi_bigint) {
        uint64_t r = 0;
        bool lossless = false;
        napi_get_value_bigint_uint64(env, v, &r, &lossless);
        return r;
    }
    double d = 0;
    napi_get_value_double(env, v, &d);
    return (uint64_t)d;
}

// fillHashF32(ptr, n, seed, lo, hi, stream?) / fillHashU8(ptr, n, seed, stream?); seed: decimal
// string, BigInt or number.
napi_value FillHashF32(napi_env env, napi_callback_info info) {
    Args a(env, info, 6);
    if (a.size() < 5) {
        throw_type(env, "fillHashF32(ptr, n, seed, lo, hi[, stream])");
        return nullptr;
    }
    int st = g4_fill_hash_f32((float *)a.ptr(0), (int64_t)a.num(1), u64_arg(env, a.v[2]),
                              (float)a.num(3), (float)a.num(4), a.ptr(5));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

napi_value FillHashU8(napi_env env, napi_callback_info info) {
    Args a(env, info, 4);
    if (a.size() < 3) {
        throw_type(env, "fillHashU8(ptr, n, seed[, stream])");
        return nullptr;
    }
    if (throw_status(env, g4_fill_hash_u8(a.ptr(0), (int64_t)a.num(1), u64_arg(env, a.v[2]), a.ptr(3))))
        return nullptr;
    return undefined(env);
}

const void *addr_prop(napi_env env, napi_value o, const char *name) {
    return reinterpret_cast<const void *>((uintptr_t)prop(env, o, name));
}

// decodeCreate(shape, weights) -> handle. shape: the g4_decode_shape fields by their C names;
// weights: the model fields by their C names (device addresses), `layer`: an array of per-layer
// objects, and optionally `ple_slices`: [{codes, start_row, row_count}] (a split PLE table).
napi_value DecodeCreate(napi_env env, napi_callback_info info) {
    Args a(env, info, 2);
    if (a.size() < 2) {
        throw_type(env, "decodeCreate(shape, weights)");
        return nullptr;
    }
    napi_value so = a.v[0], wo = a.v[1];
    g4_decode_shape sh{};
    sh.layers = (int)prop(env, so, "layers");
    sh.kv_producers = (int)prop(env, so, "kv_producers");
    sh.hidden = (int)prop(env, so, "hidden");
    sh.ffn = (int)prop(env, so, "ffn");
    sh.q_heads = (int)prop(env, so, "q_heads");
    sh.head_dim = (int)prop(env, so, "head_dim");
    sh.ple_dim = (int)prop(env, so, "ple_dim");
    sh.global_period = (int)prop(env, so, "global_period");
    sh.sliding_window = (int)prop(env, so, "sliding_window");
    sh.kv_capacity = (int)prop(env, so, "kv_capacity");
    sh.batch = (int)prop(env, so, "batch");
    sh.vocab = (int64_t)prop(env, so, "vocab");
    sh.eps = (float)prop(env, so, "eps");
    sh.final_softcap = (float)prop(env, so, "final_softcap");
    sh.in_scale = (float)prop(env, so, "in_scale");
    sh.out_scale = (float)prop(env, so, "out_scale");
    g4_decode_weights w{};
    w.embed = addr_prop(env, wo, "embed");
    w.embed_s = (const float *)addr_prop(env, wo, "embed_s");
    w.ple_table = addr_prop(env, wo, "ple_table");
    w.ple_table_s = (const float *)addr_prop(env, wo, "ple_table_s");
    w.ple_model_proj = addr_prop(env, wo, "ple_model_proj");
    w.ple_model_proj_s = (const float *)addr_prop(env, wo, "ple_model_proj_s");
    w.ple_proj_norm = (const float *)addr_prop(env, wo, "ple_proj_norm");
    w.final_norm = (const float *)addr_prop(env, wo, "final_norm");
    w.rope_local_cos = (const float *)addr_prop(env, wo, "rope_local_cos");
    w.rope_local_sin = (const float *)addr_prop(env, wo, "rope_local_sin");
    w.rope_global_cos = (const float *)addr_prop(env, wo, "rope_global_cos");
    w.rope_global_sin = (const float *)addr_prop(env, wo, "rope_global_sin");
    napi_value layers;
    bool is_arr = false;
    napi_get_named_property(env, wo, "layer", &layers);
    napi_is_array(env, layers, &is_arr);
    uint32_t nl = 0;
    if (is_arr) napi_get_array_length(env, layers, &nl);
    if (!is_arr || (int)nl != sh.layers) {
        throw_type(env, "decodeCreate: weights.layer must hold one object per layer");
        return nullptr;
    }
    std::vector<g4_decode_layer> L(nl);
    for (uint32_t l = 0; l < nl; ++l) {
        napi_value o;
        napi_get_element(env, layers, l, &o);
        g4_decode_layer &x = L[l];
        const void **vp[] = {&x.q, &x.k, &x.v, &x.o, &x.gate, &x.up, &x.down, &x.ple_gate, &x.ple_proj};
        const char *vn[] = {"q", "k", "v", "o", "gate", "up", "down", "ple_gate", "ple_proj"};
        for (int i = 0; i < 9; ++i) *vp[i] = addr_prop(env, o, vn[i]);
        const float **fp[] = {&x.q_s, &x.k_s, &x.v_s, &x.o_s, &x.gate_s, &x.up_s, &x.down_s,
                              &x.ple_gate_s, &x.ple_proj_s, &x.input_norm, &x.post_attn_norm,
                              &x.pre_ffn_norm, &x.post_ffn_norm, &x.post_ple_norm, &x.q_norm,
                              &x.k_norm};
        const char *fn[] = {"q_s", "k_s", "v_s", "o_s", "gate_s", "up_s", "down_s", "ple_gate_s",
                            "ple_proj_s", "input_norm", "post_attn_norm", "pre_ffn_norm",
                            "post_ffn_norm", "post_ple_norm", "q_norm", "k_norm"};
        for (int i = 0; i < 16; ++i) *fp[i] = (const float *)addr_prop(env, o, fn[i]);
        x.layer_scalar = (float)prop(env, o, "layer_scalar", 1.0);
    }
    w.layer = L.data();
    std::vector<const void *> sc;
    std::vector<int64_t> ss, sn;
    bool has = false;
    napi_has_named_property(env, wo, "ple_slices", &has);
    if (has) {
        napi_value arr;
        napi_get_named_property(env, wo, "ple_slices", &arr);
        napi_is_array(env, arr, &is_arr);
        uint32_t n = 0;
        if (is_arr) napi_get_array_length(env, arr, &n);
        for (uint32_t i = 0; i < n; ++i) {
            napi_value o;
            napi_get_element(env, arr, i, &o);
            sc.push_back(addr_prop(env, o, "codes"));
            ss.push_back((int64_t)prop(env, o, "start_row"));
            sn.push_back((int64_t)prop(env, o, "row_count"));
        }
        w.ple_num_slices = (int)n;
        w.ple_slice_codes = sc.data();
        w.ple_slice_start = ss.data();
        w.ple_slice_rows = sn.data();
    }
    g4_decode *d = nullptr;
    if (throw_status(env, g4_decode_create(&sh, &w, &d))) return nullptr;
    return make_num(env, (double)(uintptr_t)d);
}

napi_value DecodeDestroy(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
    if (throw_status(env, g4_decode_destroy((g4_decode *)a.ptr(0)))) return nullptr;
    return undefined(env);
}

// decodeStep(handle, tokens, nextTokens, stream?): launches only.
napi_value DecodeStep(napi_env env, napi_callback_info info) {
    Args a(env, info, 4);
    int st = g4_decode_step((g4_decode *)a.ptr(0), (const int32_t *)a.ptr(1), (int32_t *)a.ptr(2),
                            a.ptr(3));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// decodeSetPosition(handle, pos, stream?): the position word written in stream order.
napi_value DecodeSetPosition(napi_env env, napi_callback_info info) {
    Args a(env, info, 3);
    if (throw_status(env, g4_decode_set_position((g4_decode *)a.ptr(0), a.i32(1), a.ptr(2))))
        return nullptr;
    return undefined(env);
}

napi_value DecodeKv(napi_env env, napi_callback_info info) {
    Args a(env, info, 2);
    float *k = nullptr, *v = nullptr;
    int64_t stride = 0;
    if (throw_status(env, g4_decode_kv((g4_decode *)a.ptr(0), a.i32(1), &k, &v, &stride)))
        return nullptr;
    napi_value o;
    napi_create_object(env, &o);
    set_num(env, o, "k", (double)(uintptr_t)k);
    set_num(env, o, "v", (double)(uintptr_t)v);
    set_num(env, o, "rowStride", (double)stride);
    return o;
}

napi_value DecodeBuffer(napi_env env, napi_callback_info info) {
    Args a(env, info, 2);
    char name[64] = {0};
    size_t n = 0;
    if (a.size() < 2 || napi_get_value_string_utf8(env, a.v[1], name, sizeof name, &n) != napi_ok) {
        throw_type(env, "decodeBuffer(handle, name)");
        return nullptr;
    }
    void *p = nullptr;
    size_t bytes = 0;
    if (throw_status(env, g4_decode_buffer((g4_decode *)a.ptr(0), name, &p, &bytes))) return nullptr;
    napi_value o;
    napi_create_object(env, &o);
    set_num(env, o, "addr", (double)(uintptr_t)p);
    set_num(env, o, "bytes", (double)bytes);
    return o;
}

napi_value DecodeSetStop(napi_env env, napi_callback_info info) {
    Args a(env, info, 2);
    if (throw_status(env, g4_decode_set_stop((g4_decode *)a.ptr(0), a.i32(1, -1)))) return nullptr;
    return undefined(env);
}

napi_value QgemmNoalloc(napi_env env, napi_callback_info info) {
    Args a(env, info, 13);
    int st = g4_qgemm_noalloc(a.i32(0), a.ptr(1), (const float *)a.ptr(2), a.ptr(3), a.i32(4),
                              a.ptr(5), a.i32(6), a.i32(7), a.i32(8), a.i32(9, 1), (float)a.num(10),
                              (float)a.num(11), a.ptr(12));
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

napi_value Init(napi_env env, napi_value exports) {
    struct Fn {
        const char *name;
        napi_callback cb;
    } fns[] = {
        {"deviceCount", DeviceCount}, {"setDevice", SetDevice}, {"malloc", Malloc},
        {"free", Free}, {"upload", Upload}, {"download", Download}, {"fill", Fill},
        {"synchronize", Synchronize}, {"lastError", LastError}, {"qgemv", Qgemv},
        {"qgemm", Qgemm}, {"linear", Linear}, {"kernelForShape", KernelForShape},
        {"projectionBatch", ProjectionBatch}, {"qgemvGrouped", QgemvGrouped},
        {"qgemvSplit", QgemvSplit}, {"qgemvMerge", QgemvMerge},
        {"qgemvGelu", QgemvGelu}, {"qgemvGeluSplit", QgemvGeluSplit},
        {"tile8uRepack", Tile8uRepack}, {"qgemvTile8u", QgemvTile8u},
        {"qgemvGeluM2", QgemvGeluM2}, {"pleGateSplit", PleGateSplit},
        {"pleFoldProjection", PleFoldProjection}, {"geluMulF32", GeluMulF32},
        {"qgemvExactMerge", QgemvExactMerge}, {"srqQuantize", SrqQuantize},
        {"pleGather", PleGather}, {"pleGatherSplit", PleGatherSplit},
        {"planTableSplit", PlanTableSplit}, {"qgemvPlanCreate", QgemvPlanCreate},
        {"qgemvPlanLaunch", QgemvPlanLaunch}, {"qgemvPlanDestroy", QgemvPlanDestroy},
        {"planGatherSplit", PlanGatherSplit}, {"qgemmNoalloc", QgemmNoalloc},
        {"streamCreate", StreamCreate}, {"streamDestroy", StreamDestroy},
        {"streamSynchronize", StreamSynchronize}, {"eventCreate", EventCreate},
        {"eventRecord", EventRecord}, {"eventElapsedMs", EventElapsedMs},
        {"eventDestroy", EventDestroy}, {"graphBeginCapture", GraphBeginCapture},
        {"graphEndCapture", GraphEndCapture}, {"graphLaunch", GraphLaunch},
        {"graphDestroy", GraphDestroy}, {"synchronizeAsync", SynchronizeAsync},
        {"downloadAsync", DownloadAsync}, {"fillHashF32", FillHashF32}, {"fillHashU8", FillHashU8},
        {"decodeCreate", DecodeCreate}, {"decodeDestroy", DecodeDestroy},
        {"decodeStep", DecodeStep}, {"decodeSetPosition", DecodeSetPosition},
        {"decodeKv", DecodeKv}, {"decodeBuffer", DecodeBuffer}, {"decodeSetStop", DecodeSetStop},
    };
    for (const Fn &f : fns) {
        napi_value v;
        napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &v);
        napi_set_named_property(env, exports, f.name, v);
    }
    set_num(env, exports, "ABI_VERSION", g4_abi_version());
    return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
