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
    Args a(env, info, 2);
    void *data;
    size_t len;
    if (a.size() < 2 || !host_bytes(env, a.v[1], &data, &len)) {
        throw_type(env, "upload(ptr, TypedArray|ArrayBuffer|Buffer)");
        return nullptr;
    }
    if (throw_status(env, g4_memcpy_h2d(a.ptr(0), data, len, nullptr))) return nullptr;
    return undefined(env);
}

napi_value Download(napi_env env, napi_callback_info info) {
    Args a(env, info, 2);
    size_t len = (size_t)a.num(1);
    void *data = nullptr;
    napi_value ab;
    napi_create_arraybuffer(env, len, &data, &ab);
    if (throw_status(env, g4_memcpy_d2h(data, a.ptr(0), len, nullptr))) return nullptr;
    return ab;
}

napi_value Fill(napi_env env, napi_callback_info info) {
    Args a(env, info, 3);
    if (throw_status(env, g4_fill_u8(a.ptr(0), (uint8_t)a.i32(1), (size_t)a.num(2), nullptr)))
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

// ---- the entry points (argument order = the C ABI's, stream omitted = default stream) ----

napi_value Qgemv(napi_env env, napi_callback_info info) {
    Args a(env, info, 12);
    int st = g4_qgemv(a.i32(0), a.ptr(1), (const float *)a.ptr(2), a.ptr(3), a.i32(4), a.ptr(5),
                      a.i32(6), a.i32(7), a.i32(8), a.i32(9, 1), (float)a.num(10), (float)a.num(11),
                      nullptr);
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

napi_value Qgemm(napi_env env, napi_callback_info info) {
    Args a(env, info, 12);
    int st = g4_qgemm(a.i32(0), a.ptr(1), (const float *)a.ptr(2), a.ptr(3), a.i32(4), a.ptr(5),
                      a.i32(6), a.i32(7), a.i32(8), a.i32(9, 1), (float)a.num(10), (float)a.num(11),
                      nullptr);
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

napi_value Linear(napi_env env, napi_callback_info info) {
    Args a(env, info, 12);
    int st = g4_linear(a.i32(0), a.ptr(1), (const float *)a.ptr(2), a.ptr(3), a.i32(4), a.ptr(5),
                       a.i32(6), a.i32(7), a.i32(8), a.i32(9, 1), (float)a.num(10),
                       (float)a.num(11), nullptr);
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
    Args a(env, info, 11);
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
                                 nullptr);
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// qgemvGrouped([{wq, scales, x, dst, bits, xKind, outKind, k, numRows, inScale, outScale}])
napi_value QgemvGrouped(napi_env env, napi_callback_info info) {
    Args a(env, info, 1);
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
    if (throw_status(env, g4_qgemv_grouped(d.data(), (int)n, nullptr))) return nullptr;
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
    Args a(env, info, 1);
    if (throw_status(env, g4_qgemv_plan_launch(reinterpret_cast<const g4_gemv_plan *>(a.ptr(0)),
                                               nullptr)))
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
    Args a(env, info, 11);
    int st = g4_qgemv_split(a.i32(0), a.ptr(1), (const float *)a.ptr(2), a.ptr(3), a.i32(4),
                            (float *)a.ptr(5), a.i32(6), a.i32(7), a.i32(8), a.i32(9),
                            (float)a.num(10), nullptr);
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// qgemv-4bit-gelu / qgemv-8bit-gelu: (bits, wq, scales, gate, gateKind, up, upKind, upOffset,
// dst, outKind, k, numRows, inScale, outScale[, gateScale, upScale])
napi_value QgemvGelu(napi_env env, napi_callback_info info) {
    Args a(env, info, 16);
    g4_gelu_act act{a.ptr(5), a.i32(6), (float)a.num(14), (float)a.num(15), (int64_t)a.num(7)};
    int st = g4_qgemv_gelu(a.i32(0), a.ptr(1), (const float *)a.ptr(2), a.ptr(3), a.i32(4), &act,
                           a.ptr(8), a.i32(9), a.i32(10), a.i32(11), (float)a.num(12),
                           (float)a.num(13), nullptr);
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// qgemv-4bit-gelu-exact-split: (bits, wq, scales, gate, gateKind, up, upKind, upOffset, partials,
// k, numRows, kSplits, exact, inScale[, gateScale, upScale])
napi_value QgemvGeluSplit(napi_env env, napi_callback_info info) {
    Args a(env, info, 16);
    g4_gelu_act act{a.ptr(5), a.i32(6), (float)a.num(14), (float)a.num(15), (int64_t)a.num(7)};
    int st = g4_qgemv_gelu_split(a.i32(0), a.ptr(1), (const float *)a.ptr(2), a.ptr(3), a.i32(4),
                                 &act, (float *)a.ptr(8), a.i32(9), a.i32(10), a.i32(11),
                                 a.i32(12), (float)a.num(13), nullptr);
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

napi_value QgemvMerge(napi_env env, napi_callback_info info) {
    Args a(env, info, 6);
    int st = g4_qgemv_merge((const float *)a.ptr(0), a.ptr(1), a.i32(2), a.i32(3), a.i32(4),
                            (float)a.num(5), nullptr);
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

napi_value QgemvExactMerge(napi_env env, napi_callback_info info) {
    Args a(env, info, 8);
    int st = g4_qgemv_exact_merge((const float *)a.ptr(0), (const float *)a.ptr(1), a.ptr(2),
                                  a.i32(3), a.i32(4), a.i32(5), (float)a.num(6), (float)a.num(7),
                                  nullptr);
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

napi_value SrqQuantize(napi_env env, napi_callback_info info) {
    Args a(env, info, 5);
    int st = g4_srq_quantize(a.ptr(0), a.i32(1), (int8_t *)a.ptr(2), (int64_t)a.num(3),
                             (float)a.num(4), nullptr);
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// pleGather(codes, scales, scaleKind, ids, dst, outKind, slots, cols, groupSize, groupsPerRow,
//           sliced, sliceStartRow, sliceRowCount)
napi_value PleGather(napi_env env, napi_callback_info info) {
    Args a(env, info, 13);
    int st = g4_ple_gather(a.ptr(0), a.ptr(1), a.i32(2), (const int32_t *)a.ptr(3), a.ptr(4),
                           a.i32(5), a.i32(6), a.i32(7), a.i32(8), a.i32(9), a.i32(10),
                           (int64_t)a.num(11), (int64_t)a.num(12), nullptr);
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
}

// pleGatherSplit([codes], [starts], [counts], scales, scaleKind, ids, dst, outKind, slots, cols,
//                groupSize, groupsPerRow)
napi_value PleGatherSplit(napi_env env, napi_callback_info info) {
    Args a(env, info, 12);
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
                                 a.i32(9), a.i32(10), a.i32(11), nullptr);
    if (throw_status(env, st)) return nullptr;
    return undefined(env);
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
        {"qgemvExactMerge", QgemvExactMerge}, {"srqQuantize", SrqQuantize},
        {"pleGather", PleGather}, {"pleGatherSplit", PleGatherSplit},
        {"planTableSplit", PlanTableSplit}, {"qgemvPlanCreate", QgemvPlanCreate},
        {"qgemvPlanLaunch", QgemvPlanLaunch}, {"qgemvPlanDestroy", QgemvPlanDestroy},
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
