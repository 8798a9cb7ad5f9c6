// The on-disk format of the checkpoint (host code): the safetensors directory, the lm_head tie and
// its guard, QUANT_RULES family resolution and the text-tensor allow list; payload reads go straight
// to device memory through a pinned bounce buffer.
//
// Reference: src/safetensors.ts (the container rules, parseHeader :163-295, coverageGaps :297-307,
// TIED_TENSORS / applyTies :616-705, checkTieGuard :706-800, textTensorNames :930-985) and
// src/quant.ts (QUANT_RULES / resolveQuantBits :430-513, modulePathForTensor :649-663). The
// validation rules and messages follow the reference's; the JSON reader and SHA-256 are written
// here from RFC 8259 and FIPS 180-4.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <regex>
#include <string>
#include <vector>

#include "../../include/g4ckpt.h"

namespace g4 {
int set_error(int status, const char *fmt, ...);
int hip_status(hipError_t err, const char *what);
}  // namespace g4

namespace {

int st_error(const char *code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int st_error(const char *code, const char *fmt, ...) {
    char msg[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof msg, fmt, ap);
    va_end(ap);
    return g4::set_error(G4_ERR_INVALID, "safetensors %s: %s", code, msg);
}

// ---- a small JSON reader (RFC 8259): objects, arrays, strings, numbers, literals ---------------

struct JVal {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0.0;
    std::string str;                                  // Str; the source text for Num
    std::vector<JVal> arr;                            // Arr
    std::vector<std::pair<std::string, JVal>> obj;   // Obj, in source order
    size_t begin = 0, end = 0;                        // span in the source
};

struct JParser {
    const char *s;
    size_t n, i = 0;
    std::string err;
    int depth = 0;

    bool fail(const char *what) {
        if (err.empty()) {
            char b[160];
            snprintf(b, sizeof b, "%s at position %zu", what, i);
            err = b;
        }
        return false;
    }
    void ws() {
        while (i < n && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r')) ++i;
    }
    static void utf8(std::string &o, uint32_t cp) {
        if (cp < 0x80) {
            o += (char)cp;
        } else if (cp < 0x800) {
            o += (char)(0xC0 | (cp >> 6));
            o += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            o += (char)(0xE0 | (cp >> 12));
            o += (char)(0x80 | ((cp >> 6) & 0x3F));
            o += (char)(0x80 | (cp & 0x3F));
        } else {
            o += (char)(0xF0 | (cp >> 18));
            o += (char)(0x80 | ((cp >> 12) & 0x3F));
            o += (char)(0x80 | ((cp >> 6) & 0x3F));
            o += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t &v) {
        if (i + 4 > n) return fail("short \\u escape");
        v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = s[i++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool string(std::string &o) {
        if (i >= n || s[i] != '"') return fail("expected a string");
        ++i;
        while (i < n) {
            const unsigned char c = (unsigned char)s[i++];
            if (c == '"') return true;
            if (c < 0x20) return fail("control character in a string");
            if (c != '\\') {
                o += (char)c;
                continue;
            }
            if (i >= n) break;
            const char e = s[i++];
            switch (e) {
                case '"': o += '"'; break;
                case '\\': o += '\\'; break;
                case '/': o += '/'; break;
                case 'b': o += '\b'; break;
                case 'f': o += '\f'; break;
                case 'n': o += '\n'; break;
                case 'r': o += '\r'; break;
                case 't': o += '\t'; break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00 && i + 1 < n && s[i] == '\\' && s[i + 1] == 'u') {
                        const size_t save = i;
                        i += 2;
                        uint32_t lo;
                        if (!hex4(lo)) return false;
                        if (lo >= 0xDC00 && lo < 0xE000) cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                        else i = save;
                    }
                    utf8(o, cp);
                    break;
                }
                default: return fail("bad escape");
            }
        }
        return fail("unterminated string");
    }
    bool number(JVal &v) {
        const size_t b = i;
        if (i < n && s[i] == '-') ++i;
        if (i >= n || !(s[i] >= '0' && s[i] <= '9')) return fail("bad number");
        if (s[i] == '0') ++i;
        else while (i < n && s[i] >= '0' && s[i] <= '9') ++i;
        if (i < n && s[i] == '.') {
            ++i;
            if (i >= n || !(s[i] >= '0' && s[i] <= '9')) return fail("bad number");
            while (i < n && s[i] >= '0' && s[i] <= '9') ++i;
        }
        if (i < n && (s[i] == 'e' || s[i] == 'E')) {
            ++i;
            if (i < n && (s[i] == '+' || s[i] == '-')) ++i;
            if (i >= n || !(s[i] >= '0' && s[i] <= '9')) return fail("bad number");
            while (i < n && s[i] >= '0' && s[i] <= '9') ++i;
        }
        v.kind = JVal::Num;
        v.str.assign(s + b, i - b);
        v.num = strtod(v.str.c_str(), nullptr);
        return true;
    }
    bool literal(const char *w, size_t len) {
        if (i + len > n || strncmp(s + i, w, len) != 0) return fail("unexpected token");
        i += len;
        return true;
    }
    bool value(JVal &v) {
        if (++depth > 64) return fail("nesting too deep");
        ws();
        v.begin = i;
        if (i >= n) return fail("unexpected end");
        bool ok;
        const char c = s[i];
        if (c == '{') {
            v.kind = JVal::Obj;
            ++i;
            ws();
            ok = true;
            if (i < n && s[i] == '}') {
                ++i;
            } else {
                for (;;) {
                    ws();
                    std::pair<std::string, JVal> kv;
                    if (!string(kv.first)) { ok = false; break; }
                    ws();
                    if (i >= n || s[i] != ':') { ok = fail("expected ':'"); break; }
                    ++i;
                    if (!value(kv.second)) { ok = false; break; }
                    v.obj.push_back(std::move(kv));
                    ws();
                    if (i < n && s[i] == ',') { ++i; continue; }
                    if (i < n && s[i] == '}') { ++i; break; }
                    ok = fail("expected ',' or '}'");
                    break;
                }
            }
        } else if (c == '[') {
            v.kind = JVal::Arr;
            ++i;
            ws();
            ok = true;
            if (i < n && s[i] == ']') {
                ++i;
            } else {
                for (;;) {
                    JVal e;
                    if (!value(e)) { ok = false; break; }
                    v.arr.push_back(std::move(e));
                    ws();
                    if (i < n && s[i] == ',') { ++i; continue; }
                    if (i < n && s[i] == ']') { ++i; break; }
                    ok = fail("expected ',' or ']'");
                    break;
                }
            }
        } else if (c == '"') {
            v.kind = JVal::Str;
            ok = string(v.str);
        } else if (c == 't') {
            v.kind = JVal::Bool, v.b = true;
            ok = literal("true", 4);
        } else if (c == 'f') {
            v.kind = JVal::Bool, v.b = false;
            ok = literal("false", 5);
        } else if (c == 'n') {
            v.kind = JVal::Null;
            ok = literal("null", 4);
        } else {
            ok = number(v);
        }
        v.end = i;
        --depth;
        return ok;
    }
};

// ---- the directory ----------------------------------------------------------------------------

struct DtypeSize {
    const char *name;
    int bytes;
};
constexpr DtypeSize kDtypes[] = {  // DTYPE_BYTES, safetensors.ts:37-53
    {"BOOL", 1}, {"U8", 1},  {"I8", 1},  {"F8_E4M3", 1}, {"F8_E5M2", 1},
    {"U16", 2},  {"I16", 2}, {"F16", 2}, {"BF16", 2},    {"U32", 4},
    {"I32", 4},  {"F32", 4}, {"U64", 8}, {"I64", 8},     {"F64", 8},
};

int dtype_bytes(const std::string &d) {
    for (const DtypeSize &t : kDtypes)
        if (d == t.name) return t.bytes;
    return 0;
}

// isSafeCount (safetensors.ts:122-124): a non-negative integer no larger than 2^53 - 1.
bool safe_count(const JVal &v, int64_t &out) {
    if (v.kind != JVal::Num || !std::isfinite(v.num) || v.num < 0 || v.num > 9007199254740991.0 ||
        std::floor(v.num) != v.num)
        return false;
    out = (int64_t)v.num;
    return true;
}

struct Entry {
    std::string name, dtype;
    std::vector<int64_t> shape;
    int64_t data_start = 0, data_end = 0, byte_length = 0, elements = 0;
};

struct Tie {
    const char *alias, *source;
    int64_t bytes;
};
// safetensors.ts:623-637: the lm_head pair is byte for byte the embed_tokens pair on the pinned
// revision.
constexpr Tie kTies[] = {
    {"lm_head.weight", "model.language_model.embed_tokens.embedding_quantized", 100663296},
    {"lm_head.weight_scale", "model.language_model.embed_tokens.embedding_scale", 1048576},
};

std::string shape_text(const std::vector<int64_t> &shape) {
    std::string t = "[";
    for (size_t k = 0; k < shape.size(); ++k) {
        if (k) t += ",";
        t += std::to_string(shape[k]);
    }
    return t + "]";
}

}  // namespace

struct g4_st {
    int64_t header_length = 0;
    int64_t payload_start = 0;
    int64_t payload_length = 0;
    std::vector<Entry> tensors;                // payload order
    std::map<std::string, size_t> by_name;     // into tensors (ties remap aliases)
    std::map<std::string, std::string> metadata;
    bool has_metadata = false;
    int fd = -1;
    ~g4_st() {
        if (fd >= 0) close(fd);
    }
};

namespace {

int fill_tensor(const g4_st *st, size_t idx, g4_st_tensor *out) {
    const Entry &e = st->tensors[idx];
    if (e.shape.size() > G4_ST_MAX_DIMS)
        return st_error("bad-shape", "tensor %s has %zu dims (this reader keeps %d)", e.name.c_str(),
                        e.shape.size(), G4_ST_MAX_DIMS);
    out->name = e.name.c_str();
    out->dtype = e.dtype.c_str();
    out->ndim = (int)e.shape.size();
    for (int k = 0; k < G4_ST_MAX_DIMS; ++k) out->shape[k] = k < out->ndim ? e.shape[k] : 0;
    out->data_start = e.data_start;
    out->data_end = e.data_end;
    out->file_start = st->payload_start + e.data_start;
    out->file_end = st->payload_start + e.data_end;
    out->byte_length = e.byte_length;
    out->element_count = e.elements;
    return G4_OK;
}

int read_header_length(const uint8_t *bytes, size_t n, int64_t *len) {
    if (n < G4_ST_HEADER_PREFIX_BYTES)
        return st_error("short-prefix", "need %d bytes to read the header length, got %zu",
                        G4_ST_HEADER_PREFIX_BYTES, n);
    uint64_t raw = 0;
    for (int k = 7; k >= 0; --k) raw = (raw << 8) | bytes[k];
    if (raw > (uint64_t)G4_ST_MAX_HEADER_BYTES)
        return st_error("bad-header-length", "header length %llu exceeds the %d byte ceiling",
                        (unsigned long long)raw, G4_ST_MAX_HEADER_BYTES);
    if (raw == 0) return st_error("bad-header-length", "header length 0 is not a positive integer");
    *len = (int64_t)raw;
    return G4_OK;
}

int parse_into(const uint8_t *bytes, size_t n, bool reject_overlaps, g4_st &st) {
    int64_t hlen = 0;
    int rc = read_header_length(bytes, n, &hlen);
    if (rc) return rc;
    const int64_t needed = G4_ST_HEADER_PREFIX_BYTES + hlen;
    if ((int64_t)n < needed)
        return st_error("truncated-header", "header claims %lld JSON bytes so %lld are needed, got %zu",
                        (long long)hlen, (long long)needed, n);
    JParser p{reinterpret_cast<const char *>(bytes) + G4_ST_HEADER_PREFIX_BYTES, (size_t)hlen};
    JVal root;
    bool ok = p.value(root);
    if (ok) {
        p.ws();
        if (p.i != p.n) ok = p.fail("trailing characters");
    }
    if (!ok) return st_error("bad-json", "header JSON did not parse: %s", p.err.c_str());
    if (root.kind != JVal::Obj) return st_error("bad-json", "header JSON is not an object");
    st.header_length = hlen;
    st.payload_start = needed;
    // JSON.parse keeps the last value of a repeated key
    std::map<std::string, const JVal *> last;
    std::vector<std::string> order;
    for (const auto &kv : root.obj) {
        if (!last.count(kv.first)) order.push_back(kv.first);
        last[kv.first] = &kv.second;
    }
    for (const std::string &name : order) {
        const JVal &v = *last[name];
        if (name == "__metadata__") {
            if (v.kind != JVal::Obj)
                return st_error("bad-entry", "__metadata__ is present but is not an object");
            st.has_metadata = true;
            for (const auto &m : v.obj)
                st.metadata[m.first] = m.second.kind == JVal::Str
                                           ? m.second.str
                                           : std::string(p.s + m.second.begin, m.second.end - m.second.begin);
            continue;
        }
        if (v.kind != JVal::Obj) return st_error("bad-entry", "tensor %s is not an object", name.c_str());
        const JVal *dtype = nullptr, *shape = nullptr, *offsets = nullptr;
        for (const auto &f : v.obj) {
            if (f.first == "dtype") dtype = &f.second;
            else if (f.first == "shape") shape = &f.second;
            else if (f.first == "data_offsets") offsets = &f.second;
        }
        if (!dtype || dtype->kind != JVal::Str || dtype_bytes(dtype->str) == 0) {
            const std::string shown = !dtype ? "undefined"
                                      : dtype->kind == JVal::Str ? dtype->str
                                      : std::string(p.s + dtype->begin, dtype->end - dtype->begin);
            return st_error("bad-dtype", "tensor %s has dtype %s", name.c_str(), shown.c_str());
        }
        Entry e;
        e.name = name;
        e.dtype = dtype->str;
        if (!shape || shape->kind != JVal::Arr)
            return st_error("bad-shape", "tensor %s has a shape that is not a list of counts", name.c_str());
        long double count = 1;
        for (const JVal &d : shape->arr) {
            int64_t dim;
            if (!safe_count(d, dim))
                return st_error("bad-shape", "tensor %s has a shape that is not a list of counts", name.c_str());
            e.shape.push_back(dim);
            count *= (long double)dim;
        }
        if (count > 9007199254740991.0L)
            return st_error("bad-shape", "tensor %s has an element count that overflows", name.c_str());
        e.elements = (int64_t)count;
        if (!offsets || offsets->kind != JVal::Arr || offsets->arr.size() != 2 ||
            !safe_count(offsets->arr[0], e.data_start) || !safe_count(offsets->arr[1], e.data_end))
            return st_error("bad-offsets", "tensor %s has data_offsets that are not a pair of counts",
                            name.c_str());
        if (e.data_end < e.data_start)
            return st_error("bad-offsets", "tensor %s ends at %lld before it starts at %lld", name.c_str(),
                            (long long)e.data_end, (long long)e.data_start);
        e.byte_length = e.data_end - e.data_start;
        const long double expected = (long double)e.elements * dtype_bytes(e.dtype);
        if ((long double)e.byte_length != expected)
            return st_error("size-mismatch", "tensor %s spans %lld bytes but %s %s needs %.0Lf",
                            name.c_str(), (long long)e.byte_length, e.dtype.c_str(),
                            shape_text(e.shape).c_str(), expected);
        st.tensors.push_back(std::move(e));
    }
    std::sort(st.tensors.begin(), st.tensors.end(), [](const Entry &a, const Entry &b) {
        if (a.data_start != b.data_start) return a.data_start < b.data_start;
        if (a.data_end != b.data_end) return a.data_end < b.data_end;
        return a.name < b.name;
    });
    if (reject_overlaps) {
        for (size_t k = 1; k < st.tensors.size(); ++k) {
            const Entry &prev = st.tensors[k - 1], &cur = st.tensors[k];
            if (cur.byte_length > 0 && prev.byte_length > 0 && cur.data_start < prev.data_end)
                return st_error("overlap", "tensor %s starts at %lld inside %s which ends at %lld",
                                cur.name.c_str(), (long long)cur.data_start, prev.name.c_str(),
                                (long long)prev.data_end);
        }
    }
    for (const Entry &e : st.tensors) st.payload_length = std::max(st.payload_length, e.data_end);
    for (size_t k = 0; k < st.tensors.size(); ++k) st.by_name[st.tensors[k].name] = k;
    return G4_OK;
}

const Entry *find_entry(const g4_st *st, const char *name) {
    auto it = st->by_name.find(name);
    return it == st->by_name.end() ? nullptr : &st->tensors[it->second];
}

bool read_exact(int fd, void *dst, size_t n, int64_t at) {
    uint8_t *d = reinterpret_cast<uint8_t *>(dst);
    while (n) {
        const ssize_t r = pread(fd, d, n, (off_t)at);
        if (r <= 0) return false;
        d += r;
        at += r;
        n -= (size_t)r;
    }
    return true;
}

// ---- SHA-256 (FIPS 180-4) ---------------------------------------------------------------------

constexpr uint32_t kK[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

inline uint32_t rotr(uint32_t x, int r) { return (x >> r) | (x << (32 - r)); }

void sha256_block(uint32_t h[8], const uint8_t *p) {
    uint32_t w[64];
    for (int t = 0; t < 16; ++t)
        w[t] = ((uint32_t)p[4 * t] << 24) | ((uint32_t)p[4 * t + 1] << 16) | ((uint32_t)p[4 * t + 2] << 8) |
               (uint32_t)p[4 * t + 3];
    for (int t = 16; t < 64; ++t) {
        const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
        const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
        w[t] = w[t - 16] + s0 + w[t - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int t = 0; t < 64; ++t) {
        const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
        const uint32_t ch = (e & f) ^ (~e & g);
        const uint32_t t1 = hh + S1 + ch + kK[t] + w[t];
        const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
        const uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
        const uint32_t t2 = S0 + mj;
        hh = g, g = f, f = e, e = d + t1, d = c, c = b, b = a, a = t1 + t2;
    }
    h[0] += a, h[1] += b, h[2] += c, h[3] += d, h[4] += e, h[5] += f, h[6] += g, h[7] += hh;
}

// ---- QUANT_RULES (quant.ts:449-461, the checkpoint's module_quant_configs in config.json order) --

struct Rule {
    const char *pattern;
    int bits;
};
constexpr Rule kRules[] = {
    {"^lm_head$", 2},
    {"audio_tower(?!.*lconv1d\\.linear_start)", 2},
    {"audio_tower\\.layers\\.\\d+\\.lconv1d\\.linear_start\\.", 4},
    {"language_model\\.embed_tokens$", 2},
    {"language_model\\.embed_tokens_per_layer$", 4},
    {"language_model\\.layers\\.(\\d|1[0-4])\\.mlp\\.", 4},
    {"language_model\\.layers\\.\\d+\\.mlp\\.", 2},
    {"language_model\\.layers\\.\\d+\\.per_layer_input_gate$", 8},
    {"language_model\\.layers\\.\\d+\\.per_layer_projection$", 8},
    {"language_model\\.layers\\.\\d+\\.self_attn\\.", 4},
    {"vision_tower", 8},
};
constexpr int kDefaultBits = 4;  // quantization_config.num_bits
constexpr const char *kNotConverted[] = {  // modules_to_not_convert
    "model.vision_tower.patch_embedder", "model.audio_tower.subsample_conv_projection",
    "model.audio_tower.output_proj",     "relative_k_proj",
    "model.embed_audio",                 "model.embed_vision",
    "per_layer_model_projection"};
constexpr const char *kNeverQuantizedLeaves[] = {"layer_scalar", "k_cache_scale", "v_cache_scale"};

const std::vector<std::regex> &compiled_rules() {
    static const std::vector<std::regex> rules = [] {
        std::vector<std::regex> r;
        for (const Rule &x : kRules) r.emplace_back(x.pattern, std::regex::ECMAScript);
        return r;
    }();
    return rules;
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    const int exp = (h >> 10) & 0x1F;
    const uint32_t man = h & 0x3FF;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {  // subnormal: value = man * 2^-24, exact in f32
            const float v = (float)man * 0x1p-24f;
            uint32_t vb;
            memcpy(&vb, &v, 4);
            bits = sign | vb;
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((uint32_t)(exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

}  // namespace

extern "C" {

int g4_st_parse(const uint8_t *bytes, size_t n, int reject_overlaps, g4_st **out) {
    if (!out || (!bytes && n)) return g4::set_error(G4_ERR_INVALID, "g4_st_parse: null argument");
    *out = nullptr;
    std::unique_ptr<g4_st> st(new g4_st());
    int rc = parse_into(bytes, n, reject_overlaps != 0, *st);
    if (rc) return rc;
    *out = st.release();
    return G4_OK;
}

int g4_st_open(const char *path, g4_st **out) {
    if (!path || !out) return g4::set_error(G4_ERR_INVALID, "g4_st_open: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return g4::set_error(G4_ERR_INVALID, "g4_st_open: cannot open %s", path);
    std::unique_ptr<g4_st> st(new g4_st());
    st->fd = fd;
    struct stat sb;
    if (fstat(fd, &sb) != 0) return g4::set_error(G4_ERR_INVALID, "g4_st_open: cannot stat %s", path);
    uint8_t prefix[G4_ST_HEADER_PREFIX_BYTES];
    const size_t got = sb.st_size < (off_t)sizeof prefix ? (size_t)sb.st_size : sizeof prefix;
    if (!read_exact(fd, prefix, got, 0)) return g4::set_error(G4_ERR_INVALID, "g4_st_open: read failed");
    int64_t hlen = 0;
    int rc = read_header_length(prefix, got, &hlen);
    if (rc) return rc;
    const int64_t avail = std::min<int64_t>((int64_t)sb.st_size, G4_ST_HEADER_PREFIX_BYTES + hlen);
    std::vector<uint8_t> head((size_t)avail);
    if (!read_exact(fd, head.data(), head.size(), 0))
        return g4::set_error(G4_ERR_INVALID, "g4_st_open: read failed");
    rc = parse_into(head.data(), head.size(), true, *st);
    if (rc) return rc;
    const int64_t file_end = st->payload_start + st->payload_length;
    if (file_end > (int64_t)sb.st_size)
        return st_error("short-range", "payload ends at %lld but %s holds %lld bytes",
                        (long long)file_end, path, (long long)sb.st_size);
    *out = st.release();
    return G4_OK;
}

int g4_st_close(g4_st *st) {
    delete st;
    return G4_OK;
}

int g4_st_info(const g4_st *st, int64_t *header_length, int64_t *payload_start,
               int64_t *payload_length, int64_t *file_length) {
    if (!st) return g4::set_error(G4_ERR_INVALID, "g4_st_info: null directory");
    if (header_length) *header_length = st->header_length;
    if (payload_start) *payload_start = st->payload_start;
    if (payload_length) *payload_length = st->payload_length;
    if (file_length) *file_length = st->payload_start + st->payload_length;
    return G4_OK;
}

int64_t g4_st_count(const g4_st *st) { return st ? (int64_t)st->tensors.size() : 0; }

int g4_st_tensor_at(const g4_st *st, int64_t i, g4_st_tensor *out) {
    if (!st || !out || i < 0 || i >= (int64_t)st->tensors.size())
        return g4::set_error(G4_ERR_INVALID, "g4_st_tensor_at: index %lld out of range", (long long)i);
    return fill_tensor(st, (size_t)i, out);
}

int g4_st_find(const g4_st *st, const char *name, g4_st_tensor *out) {
    if (!st || !name || !out) return g4::set_error(G4_ERR_INVALID, "g4_st_find: null argument");
    auto it = st->by_name.find(name);
    if (it == st->by_name.end())
        return st_error("bad-entry", "tensor %s is not in this checkpoint", name);
    int rc = fill_tensor(st, it->second, out);
    if (rc == G4_OK) out->name = it->first.c_str();  // the name asked for (an alias stays an alias)
    return rc;
}

const char *g4_st_metadata(const g4_st *st, const char *key) {
    if (!st || !key) return nullptr;
    auto it = st->metadata.find(key);
    return it == st->metadata.end() ? nullptr : it->second.c_str();
}

int64_t g4_st_coverage_gaps(const g4_st *st, int64_t *starts, int64_t *ends, int64_t cap) {
    if (!st) return 0;
    int64_t count = 0, cursor = 0;
    for (const Entry &e : st->tensors) {
        if (e.byte_length == 0) continue;
        if (e.data_start > cursor) {
            if (count < cap && starts && ends) starts[count] = cursor, ends[count] = e.data_start;
            ++count;
        }
        cursor = std::max(cursor, e.data_end);
    }
    return count;
}

int g4_st_apply_ties(g4_st *st) {
    if (!st) return g4::set_error(G4_ERR_INVALID, "g4_st_apply_ties: null directory");
    for (const Tie &t : kTies)
        if (!st->by_name.count(t.source))
            return st_error("bad-entry", "tie %s points at %s and this checkpoint does not carry it",
                            t.alias, t.source);
    for (const Tie &t : kTies) st->by_name[t.alias] = st->by_name[t.source];
    return G4_OK;
}

int g4_st_tie_count(void) { return (int)(sizeof kTies / sizeof kTies[0]); }

int g4_st_tie(int i, const char **alias, const char **source, int64_t *byte_length) {
    if (i < 0 || i >= g4_st_tie_count()) return g4::set_error(G4_ERR_INVALID, "g4_st_tie: index %d", i);
    if (alias) *alias = kTies[i].alias;
    if (source) *source = kTies[i].source;
    if (byte_length) *byte_length = kTies[i].bytes;
    return G4_OK;
}

int g4_st_read(const g4_st *st, const char *name, int64_t offset, void *host_dst, size_t bytes) {
    if (!st || !name || (!host_dst && bytes)) return g4::set_error(G4_ERR_INVALID, "g4_st_read: null argument");
    if (st->fd < 0) return g4::set_error(G4_ERR_INVALID, "g4_st_read: the directory was parsed, not opened");
    const Entry *e = find_entry(st, name);
    if (!e) return st_error("bad-entry", "tensor %s is not in this checkpoint", name);
    if (offset < 0 || offset + (int64_t)bytes > e->byte_length)
        return st_error("short-range", "tensor %s holds %lld bytes, asked for %zu at %lld", name,
                        (long long)e->byte_length, bytes, (long long)offset);
    if (!read_exact(st->fd, host_dst, bytes, st->payload_start + e->data_start + offset))
        return g4::set_error(G4_ERR_INVALID, "g4_st_read: read of %s failed", name);
    return G4_OK;
}

int g4_st_upload(const g4_st *st, const char *name, void *device_dst, size_t dst_bytes,
                 void *stream) {
    if (!st || !name || !device_dst) return g4::set_error(G4_ERR_INVALID, "g4_st_upload: null argument");
    const Entry *e = find_entry(st, name);
    if (!e) return st_error("bad-entry", "tensor %s is not in this checkpoint", name);
    if ((int64_t)dst_bytes < e->byte_length)
        return g4::set_error(G4_ERR_INVALID, "g4_st_upload: %s needs %lld bytes, the buffer has %zu", name,
                             (long long)e->byte_length, dst_bytes);
    constexpr size_t kChunk = 64u << 20;
    const size_t total = (size_t)e->byte_length;
    if (total == 0) return G4_OK;
    void *pinned = nullptr;
    const size_t cap = std::min(kChunk, total);
    hipError_t err = hipHostMalloc(&pinned, cap, hipHostMallocDefault);
    if (err != hipSuccess) return g4::hip_status(err, "g4_st_upload: hipHostMalloc");
    int rc = G4_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    for (size_t off = 0; off < total && rc == G4_OK; off += cap) {
        const size_t n = std::min(cap, total - off);
        rc = g4_st_read(st, name, (int64_t)off, pinned, n);
        if (rc) break;
        err = hipMemcpyAsync(reinterpret_cast<uint8_t *>(device_dst) + off, pinned, n,
                             hipMemcpyHostToDevice, s);
        if (err == hipSuccess) err = hipStreamSynchronize(s);  // the bounce buffer is reused
        if (err != hipSuccess) rc = g4::hip_status(err, "g4_st_upload: copy");
    }
    (void)hipHostFree(pinned);
    return rc;
}

int g4_st_upload_split(const g4_st *st, const char *name, const g4_table_slice *slices,
                       int num_slices, void *const *slice_dst, void *stream) {
    if (!st || !name) return g4::set_error(G4_ERR_INVALID, "g4_st_upload_split: null argument");
    if (num_slices < 1 || !slices || !slice_dst)
        return g4::set_error(G4_ERR_INVALID, "BufferManager.declareSplit: %s needs at least one range",
                             name);
    const Entry *e = find_entry(st, name);
    if (!e) return st_error("bad-entry", "tensor %s is not in this checkpoint", name);
    // declareSplit (buffers.ts:291-327): the ranges partition the tensor in offset order
    int64_t expect = 0;
    for (int i = 0; i < num_slices; ++i) {
        const g4_table_slice &r = slices[i];
        if (r.byte_offset != expect)
            return g4::set_error(G4_ERR_INVALID,
                                 "BufferManager.declareSplit: %s slice %lld starts at %lld, not at "
                                 "%lld; the ranges have to partition the tensor in offset order",
                                 name, (long long)r.index, (long long)r.byte_offset,
                                 (long long)expect);
        if (r.byte_offset % 4 != 0)
            return g4::set_error(G4_ERR_INVALID,
                                 "BufferManager.declareSplit: %s slice %lld starts at %lld, which is "
                                 "not four byte aligned", name, (long long)r.index,
                                 (long long)r.byte_offset);
        if (r.byte_length <= 0 || !slice_dst[i])
            return g4::set_error(G4_ERR_INVALID, "g4_st_upload_split: %s slice %lld has no bytes or no buffer",
                                 name, (long long)r.index);
        expect += r.byte_length;
    }
    if (expect != e->byte_length)
        return g4::set_error(G4_ERR_INVALID,
                             "BufferManager.uploadWeight: %s is %lld bytes and the declared slices "
                             "cover %lld, so a piece would fall outside every declared slice",
                             name, (long long)e->byte_length, (long long)expect);
    constexpr size_t kChunk = 64u << 20;
    const int64_t total = e->byte_length;
    void *pinned = nullptr;
    const size_t cap = (size_t)std::min<int64_t>((int64_t)kChunk, total);
    hipError_t err = hipHostMalloc(&pinned, cap, hipHostMallocDefault);
    if (err != hipSuccess) return g4::hip_status(err, "g4_st_upload_split: hipHostMalloc");
    int rc = G4_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    for (int64_t piece = 0; piece < total && rc == G4_OK; piece += (int64_t)cap) {
        const int64_t n = std::min<int64_t>((int64_t)cap, total - piece);
        rc = g4_st_read(st, name, piece, pinned, (size_t)n);
        if (rc) break;
        // uploadSplitWeight (buffers.ts:384-423): the piece's intersection with each slice, rebased
        for (int i = 0; i < num_slices && err == hipSuccess; ++i) {
            const int64_t from = std::max(piece, slices[i].byte_offset);
            const int64_t to = std::min(piece + n, slices[i].byte_offset + slices[i].byte_length);
            if (to <= from) continue;
            err = hipMemcpyAsync(reinterpret_cast<uint8_t *>(slice_dst[i]) + (from - slices[i].byte_offset),
                                 reinterpret_cast<uint8_t *>(pinned) + (from - piece),
                                 (size_t)(to - from), hipMemcpyHostToDevice, s);
        }
        if (err == hipSuccess) err = hipStreamSynchronize(s);  // the bounce buffer is reused
        if (err != hipSuccess) rc = g4::hip_status(err, "g4_st_upload_split: copy");
    }
    (void)hipHostFree(pinned);
    return rc;
}

int g4_st_plan_ple_split(const g4_st *st, const char *codes_name, int64_t groups_per_row,
                         const g4_gather_limits *limits, g4_gather_split_plans *plans,
                         g4_table_slice *slices, int64_t max_slices) {
    if (!st || !codes_name || !limits || !plans)
        return g4::set_error(G4_ERR_INVALID, "g4_st_plan_ple_split: null argument");
    const Entry *e = find_entry(st, codes_name);
    if (!e) return st_error("bad-entry", "tensor %s is not in this checkpoint", codes_name);
    const int64_t rows = e->shape.empty() ? 0 : e->shape[0];
    if (rows <= 0 || e->byte_length % rows != 0)
        return g4::set_error(G4_ERR_INVALID,
                             "gemma4 engine: %s has shape %s and %lld bytes, which is not a whole "
                             "number of bytes per vocabulary row, so its split cannot be planned. A "
                             "table that cannot be split cannot be loaded on an adapter that needs one.",
                             codes_name, shape_text(e->shape).c_str(), (long long)e->byte_length);
    int rc = g4_plan_gather_split(rows, e->byte_length / rows, groups_per_row, limits, plans, slices,
                                  slices ? max_slices : 0, nullptr, 0);
    if (rc) return rc;
    if (plans->codes.single) return G4_OK;
    if (!plans->codes.feasible)
        return g4::set_error(G4_ERR_UNSUPPORTED,
                             "gemma4 engine: %s codes need %lld slices of 4 storage bindings against "
                             "a budget of %lld", codes_name, (long long)plans->codes.num_slices,
                             (long long)plans->codes.binding_budget);
    if (!plans->scales_single)
        return g4::set_error(G4_ERR_UNSUPPORTED,
                             "gemma4 engine: %s scales do NOT fit in one binding on this adapter, and "
                             "the sliced gather addresses scales by the absolute vocabulary row, so "
                             "this configuration needs a second slice index before it is correct",
                             codes_name);
    return G4_OK;
}

int g4_st_upload_f32(const g4_st *st, const char *name, float *device_dst, int64_t count,
                     void *stream) {
    if (!st || !name || !device_dst) return g4::set_error(G4_ERR_INVALID, "g4_st_upload_f32: null argument");
    const Entry *e = find_entry(st, name);
    if (!e) return st_error("bad-entry", "tensor %s is not in this checkpoint", name);
    if (e->dtype != "BF16" && e->dtype != "F16" && e->dtype != "F32")
        return g4::set_error(G4_ERR_UNSUPPORTED, "g4_st_upload_f32: %s is %s, not BF16, F16 or F32", name,
                             e->dtype.c_str());
    if (count != e->elements)
        return g4::set_error(G4_ERR_INVALID, "g4_st_upload_f32: %s holds %lld values, the buffer %lld", name,
                             (long long)e->elements, (long long)count);
    std::vector<uint8_t> raw((size_t)e->byte_length);
    int rc = g4_st_read(st, name, 0, raw.data(), raw.size());
    if (rc) return rc;
    std::vector<float> vals((size_t)count);
    for (int64_t k = 0; k < count; ++k) {
        if (e->dtype == "F32") {
            memcpy(&vals[k], raw.data() + 4 * k, 4);
        } else {
            const uint16_t h = (uint16_t)(raw[2 * k] | (raw[2 * k + 1] << 8));
            if (e->dtype == "BF16") {
                const uint32_t bits = (uint32_t)h << 16;  // bf16ToF32, quant.ts:400-411
                memcpy(&vals[k], &bits, 4);
            } else {
                vals[k] = f16_to_f32(h);
            }
        }
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipError_t err = hipMemcpyAsync(device_dst, vals.data(), sizeof(float) * vals.size(),
                                    hipMemcpyHostToDevice, s);
    if (err == hipSuccess) err = hipStreamSynchronize(s);
    if (err != hipSuccess) return g4::hip_status(err, "g4_st_upload_f32");
    return G4_OK;
}

void g4_sha256_hex(const uint8_t *data, size_t n, char *out65) {
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                     0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    size_t full = n / 64;
    for (size_t b = 0; b < full; ++b) sha256_block(h, data + 64 * b);
    uint8_t tail[128] = {0};
    const size_t rem = n - 64 * full;
    if (rem) memcpy(tail, data + 64 * full, rem);
    tail[rem] = 0x80;
    const size_t blocks = rem + 9 <= 64 ? 1 : 2;
    const uint64_t bits = (uint64_t)n * 8;
    for (int k = 0; k < 8; ++k) tail[64 * blocks - 1 - k] = (uint8_t)(bits >> (8 * k));
    for (size_t b = 0; b < blocks; ++b) sha256_block(h, tail + 64 * b);
    static const char *hex = "0123456789abcdef";
    for (int k = 0; k < 8; ++k)
        for (int j = 0; j < 4; ++j) {
            const uint8_t byte = (uint8_t)(h[k] >> (24 - 8 * j));
            out65[8 * k + 2 * j] = hex[byte >> 4];
            out65[8 * k + 2 * j + 1] = hex[byte & 15];
        }
    out65[64] = 0;
}

// safetensors.ts:706-722: the revision the tie was verified on and the digest of the first
// 256 KiB of the embed tensor there.
static const char *kTieRevision = "dd693ff40353f057ca5f07e945ad867f4afbf2ec";
static const char *kTieSampleSha256 = "2bb8a288ec1d80f80f79eef5c447e37658037d281335079d99db2fd85a146fb5";
static const size_t kTieSampleBytes = 256 * 1024;
static const char *kTieSource = "model.language_model.embed_tokens.embedding_quantized";

int g4_tie_guard(const uint8_t *sample, size_t n, const char *revision, char *digest_hex,
                 char *reason, size_t reason_len) {
    char digest[65] = {0};
    char msg[512];
    int tied = 0;
    if (!revision || strcmp(revision, kTieRevision) != 0) {
        snprintf(msg, sizeof msg,
                 "tie guard: revision %s is not the pinned %s, so the lm_head tie was never verified "
                 "against this checkpoint. Fetching both tensors.",
                 revision ? revision : "(none)", kTieRevision);
    } else if (n != kTieSampleBytes || !sample) {
        snprintf(msg, sizeof msg, "tie guard: sample is %zu bytes, expected %zu. Fetching both tensors.",
                 n, kTieSampleBytes);
    } else {
        g4_sha256_hex(sample, n, digest);
        if (strcmp(digest, kTieSampleSha256) != 0) {
            snprintf(msg, sizeof msg,
                     "tie guard: %s sample hashes to %s, pinned %s. The checkpoint is not the one the "
                     "tie was verified on. Fetching both tensors.",
                     kTieSource, digest, kTieSampleSha256);
        } else {
            snprintf(msg, sizeof msg, "tie guard: sample matches the pinned digest");
            tied = 1;
        }
    }
    if (digest_hex) memcpy(digest_hex, digest, 65);
    if (reason && reason_len) {
        strncpy(reason, msg, reason_len - 1);
        reason[reason_len - 1] = 0;
    }
    return tied;
}

int g4_quant_bits(const char *module_path) {
    if (!module_path) return g4::set_error(G4_ERR_INVALID, "g4_quant_bits: null path"), -1;
    const std::string m(module_path);
    for (const char *skip : kNotConverted)
        if (m.find(skip) != std::string::npos) return 0;
    const std::string leaf = m.substr(m.rfind('.') == std::string::npos ? 0 : m.rfind('.') + 1);
    if (leaf.size() >= 4 && leaf.compare(leaf.size() - 4, 4, "norm") == 0) return 0;
    for (const char *l : kNeverQuantizedLeaves)
        if (leaf == l) return 0;
    const auto &rules = compiled_rules();
    long best = -1;
    int bits = kDefaultBits;
    for (size_t r = 0; r < rules.size(); ++r) {
        std::smatch mt;
        if (!std::regex_search(m, mt, rules[r])) continue;
        const long at = (long)mt.position(0);
        if (best < 0 || at < best) best = at, bits = kRules[r].bits;
    }
    return bits;
}

int g4_module_path_for_tensor(const char *tensor_name, char *buf, size_t len) {
    if (!tensor_name || !buf || !len) return g4::set_error(G4_ERR_INVALID, "g4_module_path_for_tensor: null argument");
    static const char *suffixes[] = {".weight_scale", ".input_activation_scale", ".output_activation_scale",
                                     ".embedding_quantized", ".embedding_scale", ".weight"};
    std::string t(tensor_name);
    for (const char *suf : suffixes) {
        const size_t sl = strlen(suf);
        if (t.size() >= sl && t.compare(t.size() - sl, sl, suf) == 0) {
            t.resize(t.size() - sl);
            break;
        }
    }
    if (t.size() + 1 > len) return g4::set_error(G4_ERR_INVALID, "g4_module_path_for_tensor: buffer too small");
    memcpy(buf, t.c_str(), t.size() + 1);
    return G4_OK;
}

int64_t g4_text_tensor_names(int layers, int kv_shared, int fetch_tied_pair, char *buf,
                             size_t len, size_t *needed) {
    layers = std::max(0, layers);
    kv_shared = std::max(0, kv_shared);
    const int producers = std::max(0, layers - kv_shared);
    std::vector<std::string> names = {
        "lm_head.input_activation_scale",
        "lm_head.output_activation_scale",
        "model.language_model.embed_tokens.embedding_quantized",
        "model.language_model.embed_tokens.embedding_scale",
        "model.language_model.embed_tokens_per_layer.embedding_quantized",
        "model.language_model.embed_tokens_per_layer.embedding_scale",
        "model.language_model.norm.weight",
        "model.language_model.per_layer_model_projection.weight",
        "model.language_model.per_layer_projection_norm.weight",
    };
    static const char *linear_suffixes[] = {"weight", "weight_scale", "input_activation_scale",
                                            "output_activation_scale"};
    for (int l = 0; l < layers; ++l) {
        const std::string base = "model.language_model.layers." + std::to_string(l);
        for (const char *n : {".input_layernorm.weight", ".post_attention_layernorm.weight",
                              ".pre_feedforward_layernorm.weight", ".post_feedforward_layernorm.weight",
                              ".post_per_layer_input_norm.weight", ".layer_scalar",
                              ".self_attn.q_norm.weight", ".self_attn.k_cache_scale",
                              ".self_attn.v_cache_scale"})
            names.push_back(base + n);
        const bool producer = l < producers;
        if (producer) names.push_back(base + ".self_attn.k_norm.weight");
        std::vector<const char *> linears = {"self_attn.q_proj", "self_attn.o_proj", "mlp.gate_proj",
                                             "mlp.up_proj", "mlp.down_proj", "per_layer_input_gate",
                                             "per_layer_projection"};
        if (producer) {
            linears.push_back("self_attn.k_proj");
            linears.push_back("self_attn.v_proj");
        }
        for (const char *lin : linears)
            for (const char *suf : linear_suffixes) names.push_back(base + "." + lin + "." + suf);
    }
    if (fetch_tied_pair)
        for (const Tie &t : kTies) names.push_back(t.alias);
    std::string joined;
    for (size_t k = 0; k < names.size(); ++k) {
        if (k) joined += '\n';
        joined += names[k];
    }
    if (needed) *needed = joined.size() + 1;
    if (buf && len) {
        const size_t n = std::min(len - 1, joined.size());
        memcpy(buf, joined.data(), n);
        buf[n] = 0;
    }
    return (int64_t)names.size();
}

}  // extern "C"
