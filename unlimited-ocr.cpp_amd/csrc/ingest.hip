// Weight ingest on the host: a safetensors reader, the pre-quantized (GPTQ)
// INT4 matrices with their `uocr_int4` group metadata, and the AWQ expert
// input-scale fold. Counterparts: uocr::SafetensorsFile
// (src/runtime/safetensors.cpp:30-137), make_quantized's pre-quantized branch
// (src/runtime/weights.cpp:129-166) and apply_expert_input_scale / scale_columns
// (weights.cpp:185-207). The file format (8-byte little-endian header length,
// a JSON header of {name: {dtype, shape, data_offsets}} plus "__metadata__",
// then the raw tensor bytes) and the tensor names (<weight>.packed U8
// [rows, ceil(cols/2)], .scales / .zeros F32 [rows, n_groups],
// tools/reference/quantize_gptq.py:20-22,380-382,412) are the reference's.
// No device work here.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "launch.hpp"
#include "uocr_hip/moe_capi.h"

namespace {

// ---- a small JSON reader: enough for a safetensors header (objects, arrays,
// strings with escapes, integers, numbers, true / false / null)
struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0.0;
    long long integer = 0;
    bool is_int = false;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;  // file order
    const Json* get(const std::string& k) const {
        for (const auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct JsonParser {
    const char* p;
    const char* end;
    std::string err;
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool fail(const char* m) {
        if (err.empty()) err = m;
        return false;
    }
    static void put_utf8(std::string& s, unsigned cp) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xC0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += (char)(0xE0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xF0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 0x3F));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(unsigned& v) {
        if (end - p < 4) return fail("truncated \\u escape");
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool string(std::string& s) {
        if (p >= end || *p != '"') return fail("expected string");
        ++p;
        while (p < end && *p != '"') {
            char c = *p++;
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p >= end) return fail("truncated escape");
            c = *p++;
            switch (c) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    unsigned cp = 0;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                        p += 2;
                        unsigned lo = 0;
                        if (!hex4(lo)) return false;
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(s, cp);
                    break;
                }
                default: return fail("bad escape");
            }
        }
        if (p >= end) return fail("unterminated string");
        ++p;
        return true;
    }
    bool value(Json& v, int depth) {
        if (depth > 64) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("unexpected end");
        const char c = *p;
        if (c == '{') {
            v.kind = Json::Obj;
            ++p;
            ws();
            if (p < end && *p == '}') {
                ++p;
                return true;
            }
            for (;;) {
                ws();
                std::string k;
                if (!string(k)) return false;
                ws();
                if (p >= end || *p != ':') return fail("expected ':'");
                ++p;
                Json child;
                if (!value(child, depth + 1)) return false;
                v.obj.emplace_back(std::move(k), std::move(child));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == '}') {
                    ++p;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            v.kind = Json::Arr;
            ++p;
            ws();
            if (p < end && *p == ']') {
                ++p;
                return true;
            }
            for (;;) {
                Json child;
                if (!value(child, depth + 1)) return false;
                v.arr.push_back(std::move(child));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == ']') {
                    ++p;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = Json::Str;
            return string(v.str);
        }
        auto word = [&](const char* w) {
            const size_t n = std::strlen(w);
            if ((size_t)(end - p) >= n && std::memcmp(p, w, n) == 0) {
                p += n;
                return true;
            }
            return false;
        };
        if (word("true")) {
            v.kind = Json::Bool;
            v.b = true;
            return true;
        }
        if (word("false")) {
            v.kind = Json::Bool;
            return true;
        }
        if (word("null")) return true;
        // number
        const char* s0 = p;
        if (p < end && (*p == '-' || *p == '+')) ++p;
        bool frac = false;
        while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '-' || *p == '+')) {
            if (*p == '.' || *p == 'e' || *p == 'E') frac = true;
            ++p;
        }
        if (p == s0) return fail("unexpected character");
        const std::string t(s0, p);
        v.kind = Json::Num;
        char* e = nullptr;
        v.num = std::strtod(t.c_str(), &e);
        if (!e || *e) return fail("bad number");
        if (!frac) {
            v.is_int = true;
            v.integer = std::strtoll(t.c_str(), nullptr, 10);
        }
        return true;
    }
};

bool parse_json(const char* s, size_t n, Json& out, std::string& err) {
    JsonParser jp{s, s + n, {}};
    if (!jp.value(out, 0)) {
        err = jp.err;
        return false;
    }
    jp.ws();
    if (jp.p != jp.end) {
        err = "trailing characters";
        return false;
    }
    return true;
}

enum class DType { F32, BF16, F16, I32, I8, U8, I4, U4 };

// dtype names (safetensors.cpp:16-26)
bool parse_dtype(const std::string& s, DType& d) {
    if (s == "F32" || s == "FLOAT") d = DType::F32;
    else if (s == "BF16" || s == "BFLOAT16") d = DType::BF16;
    else if (s == "F16" || s == "FLOAT16") d = DType::F16;
    else if (s == "I32" || s == "INT32") d = DType::I32;
    else if (s == "I8" || s == "INT8") d = DType::I8;
    else if (s == "U8" || s == "UINT8") d = DType::U8;
    else if (s == "I4") d = DType::I4;
    else if (s == "U4") d = DType::U4;
    else return false;
    return true;
}

float bf16_to_f32(uint16_t h) {
    const uint32_t b = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

// IEEE binary16 -> binary32, exact (subnormals, inf and NaN included)
float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t exp = (h >> 10) & 0x1F, man = h & 0x3FF, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {  // subnormal: normalise
            int e = -1;
            do {
                man <<= 1;
                ++e;
            } while (!(man & 0x400));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FF) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

struct TensorInfo {
    DType dtype;
    std::vector<long long> shape;
    size_t begin = 0, end = 0;
    size_t numel() const {
        size_t n = 1;
        for (long long d : shape) n *= (size_t)d;
        return n;
    }
};

}  // namespace

struct uocr_hip_st_file {
    std::vector<unsigned char> bytes;  // the whole file
    size_t data_start = 0;
    std::map<std::string, TensorInfo> tensors;
    std::map<std::string, std::string> metadata;  // string-valued entries only
    // matrices handed out by uocr_hip_gptq_qmatrix (owned until close)
    struct Held {
        std::vector<uint8_t> packed;
        std::vector<float> scales, zeros;
    };
    std::vector<std::unique_ptr<Held>> held;
};

namespace {

int find_tensor(const uocr_hip_st_file* f, const char* name, const TensorInfo** out) {
    if (!f || !name) return uocr_hip::set_error(UOCR_HIP_EINVAL, "null argument");
    auto it = f->tensors.find(name);
    if (it == f->tensors.end()) return uocr_hip::set_error(UOCR_HIP_EINVAL, std::string("tensor not found: ") + name);
    *out = &it->second;
    return UOCR_HIP_OK;
}

// SafetensorsFile::read_f32 (safetensors.cpp:88-127): F32 / BF16 / F16 / I32 /
// I8 / U8 converted to f32
int read_f32(const uocr_hip_st_file* f, const char* name, std::vector<float>& out) {
    const TensorInfo* in = nullptr;
    if (int rc = find_tensor(f, name, &in)) return rc;
    const size_t n = in->numel();
    const unsigned char* src = f->bytes.data() + f->data_start + in->begin;
    size_t esz = 0;
    switch (in->dtype) {
        case DType::F32: case DType::I32: esz = 4; break;
        case DType::BF16: case DType::F16: esz = 2; break;
        case DType::I8: case DType::U8: esz = 1; break;
        default: return uocr_hip::set_error(UOCR_HIP_EINVAL, std::string("read_f32: unsupported dtype for ") + name);
    }
    if (n * esz > in->end - in->begin)
        return uocr_hip::set_error(UOCR_HIP_EINVAL, std::string("tensor shorter than its shape: ") + name);
    out.resize(n);
    for (size_t i = 0; i < n; ++i) {
        switch (in->dtype) {
            case DType::F32: std::memcpy(&out[i], src + 4 * i, 4); break;
            case DType::I32: {
                int32_t v;
                std::memcpy(&v, src + 4 * i, 4);
                out[i] = (float)v;
                break;
            }
            case DType::BF16: {
                uint16_t v;
                std::memcpy(&v, src + 2 * i, 2);
                out[i] = bf16_to_f32(v);
                break;
            }
            case DType::F16: {
                uint16_t v;
                std::memcpy(&v, src + 2 * i, 2);
                out[i] = f16_to_f32(v);
                break;
            }
            case DType::I8: out[i] = (float)(int8_t)src[i]; break;
            default: out[i] = (float)src[i]; break;
        }
    }
    return UOCR_HIP_OK;
}

// SafetensorsFile::read_u8 (safetensors.cpp:129-137): U8 / I8 bytes
int read_u8(const uocr_hip_st_file* f, const char* name, std::vector<uint8_t>& out) {
    const TensorInfo* in = nullptr;
    if (int rc = find_tensor(f, name, &in)) return rc;
    if (in->dtype != DType::U8 && in->dtype != DType::I8)
        return uocr_hip::set_error(UOCR_HIP_EINVAL, std::string("read_u8: expected U8/I8 tensor for ") + name);
    const size_t n = in->numel();
    if (n > in->end - in->begin)
        return uocr_hip::set_error(UOCR_HIP_EINVAL, std::string("tensor shorter than its shape: ") + name);
    out.assign(f->bytes.begin() + f->data_start + in->begin, f->bytes.begin() + f->data_start + in->begin + n);
    return UOCR_HIP_OK;
}

}  // namespace

extern "C" {

int uocr_hip_st_open(const char* path, uocr_hip_st_file** out) {
    using uocr_hip::set_error;
    if (!path || !out) return set_error(UOCR_HIP_EINVAL, "null argument");
    *out = nullptr;
    std::unique_ptr<uocr_hip_st_file> f(new uocr_hip_st_file);
    FILE* fp = std::fopen(path, "rb");
    if (!fp) return set_error(UOCR_HIP_EINVAL, std::string("cannot open safetensors file: ") + path);
    std::fseek(fp, 0, SEEK_END);
    const long sz = std::ftell(fp);
    std::fseek(fp, 0, SEEK_SET);
    if (sz < 8) {
        std::fclose(fp);
        return set_error(UOCR_HIP_EINVAL, std::string("not a safetensors file: ") + path);
    }
    f->bytes.resize((size_t)sz);
    const size_t got = std::fread(f->bytes.data(), 1, (size_t)sz, fp);
    std::fclose(fp);
    if (got != (size_t)sz) return set_error(UOCR_HIP_EINVAL, std::string("short read: ") + path);
    uint64_t hlen = 0;
    for (int i = 0; i < 8; ++i) hlen |= (uint64_t)f->bytes[i] << (8 * i);
    if (hlen > (uint64_t)sz - 8) return set_error(UOCR_HIP_EINVAL, "safetensors header out of range");
    f->data_start = 8 + (size_t)hlen;
    Json root;
    std::string err;
    if (!parse_json(reinterpret_cast<const char*>(f->bytes.data()) + 8, (size_t)hlen, root, err) ||
        root.kind != Json::Obj)
        return set_error(UOCR_HIP_EINVAL, "safetensors header: " + (err.empty() ? std::string("not an object") : err));
    for (const auto& kv : root.obj) {
        if (kv.first == "__metadata__") {
            if (kv.second.kind == Json::Obj)
                for (const auto& m : kv.second.obj)
                    if (m.second.kind == Json::Str) f->metadata[m.first] = m.second.str;
            continue;
        }
        const Json* dt = kv.second.get("dtype");
        const Json* shape = kv.second.get("shape");
        const Json* offs = kv.second.get("data_offsets");
        TensorInfo ti;
        if (!dt || dt->kind != Json::Str || !parse_dtype(dt->str, ti.dtype))
            return set_error(UOCR_HIP_EINVAL, "unsupported or missing dtype: " + kv.first);
        if (!shape || shape->kind != Json::Arr || !offs || offs->kind != Json::Arr || offs->arr.size() != 2)
            return set_error(UOCR_HIP_EINVAL, "bad shape / data_offsets: " + kv.first);
        size_t elems = 1;  // checked: a crafted shape must not wrap the byte counts below
        for (const Json& d : shape->arr) {
            if (!d.is_int || d.integer < 0) return set_error(UOCR_HIP_EINVAL, "bad shape: " + kv.first);
            if (d.integer != 0 && elems > (SIZE_MAX / 8) / (size_t)d.integer)
                return set_error(UOCR_HIP_EINVAL, "shape too large: " + kv.first);
            elems *= (size_t)d.integer;
            ti.shape.push_back(d.integer);
        }
        if (!offs->arr[0].is_int || !offs->arr[1].is_int || offs->arr[0].integer < 0 ||
            offs->arr[1].integer < offs->arr[0].integer)
            return set_error(UOCR_HIP_EINVAL, "bad data_offsets: " + kv.first);
        ti.begin = (size_t)offs->arr[0].integer;
        ti.end = (size_t)offs->arr[1].integer;
        if (f->data_start + ti.end > (size_t)sz) return set_error(UOCR_HIP_EINVAL, "tensor beyond file end: " + kv.first);
        f->tensors[kv.first] = std::move(ti);
    }
    *out = f.release();
    return UOCR_HIP_OK;
}

int uocr_hip_st_close(uocr_hip_st_file* f) {
    delete f;
    return UOCR_HIP_OK;
}

int uocr_hip_st_contains(const uocr_hip_st_file* f, const char* name) {
    return f && name && f->tensors.count(name) ? 1 : 0;
}

int uocr_hip_st_numel(const uocr_hip_st_file* f, const char* name, size_t* n) {
    const TensorInfo* in = nullptr;
    if (!n) return uocr_hip::set_error(UOCR_HIP_EINVAL, "null argument");
    if (int rc = find_tensor(f, name, &in)) return rc;
    *n = in->numel();
    return UOCR_HIP_OK;
}

int uocr_hip_st_read_f32(const uocr_hip_st_file* f, const char* name, float* dst, size_t n) {
    std::vector<float> v;
    if (!dst) return uocr_hip::set_error(UOCR_HIP_EINVAL, "null argument");
    if (int rc = read_f32(f, name, v)) return rc;
    if (v.size() != n)
        return uocr_hip::set_error(UOCR_HIP_EINVAL, std::string("element count mismatch for ") + name + ": file " +
                                                        std::to_string(v.size()) + ", caller " + std::to_string(n));
    std::memcpy(dst, v.data(), n * 4);
    return UOCR_HIP_OK;
}

int uocr_hip_st_read_u8(const uocr_hip_st_file* f, const char* name, uint8_t* dst, size_t n) {
    std::vector<uint8_t> v;
    if (!dst) return uocr_hip::set_error(UOCR_HIP_EINVAL, "null argument");
    if (int rc = read_u8(f, name, v)) return rc;
    if (v.size() != n)
        return uocr_hip::set_error(UOCR_HIP_EINVAL, std::string("element count mismatch for ") + name);
    std::memcpy(dst, v.data(), n);
    return UOCR_HIP_OK;
}

int uocr_hip_st_metadata(const uocr_hip_st_file* f, const char* key, const char** value) {
    if (!f || !key || !value) return uocr_hip::set_error(UOCR_HIP_EINVAL, "null argument");
    auto it = f->metadata.find(key);
    *value = it == f->metadata.end() ? nullptr : it->second.c_str();
    return UOCR_HIP_OK;
}

// weights.cpp:140-151: the quantizer's group size from the "uocr_int4" JSON
// metadata entry, converted as nlohmann's get<int>() converts it; the
// caller's group when the entry is absent, not JSON, or has no convertible
// "group".
int uocr_hip_gptq_group(const uocr_hip_st_file* f, int fallback_group) {
    if (!f) return fallback_group;
    auto it = f->metadata.find("uocr_int4");
    if (it == f->metadata.end()) return fallback_group;
    Json j;
    std::string err;
    if (!parse_json(it->second.data(), it->second.size(), j, err) || j.kind != Json::Obj) return fallback_group;
    const Json* g = j.get("group");
    if (!g) return fallback_group;
    // nlohmann's get<int>() converts any number (a float truncated toward
    // zero, e.g. 128.0 -> 128) and a boolean; other kinds throw, and the
    // reference then keeps the caller's group
    if (g->kind == Json::Bool) return g->b ? 1 : 0;
    if (g->kind != Json::Num) return fallback_group;
    if (g->is_int) return (g->integer < INT32_MIN || g->integer > INT32_MAX) ? fallback_group : (int)g->integer;
    if (!(g->num > -2147483649.0 && g->num < 2147483648.0)) return fallback_group;  // NaN or beyond int
    return (int)g->num;
}

int uocr_hip_gptq_qmatrix(const uocr_hip_st_file* f, const char* weight_name, int rows, int cols,
                          int fallback_group, uocr_hip_qmatrix* out) {
    using uocr_hip::set_error;
    if (!f || !weight_name || !out) return set_error(UOCR_HIP_EINVAL, "null argument");
    if (rows <= 0 || cols <= 0) return set_error(UOCR_HIP_EINVAL, "rows and cols must be positive");
    const std::string base(weight_name);
    if (!f->tensors.count(base + ".packed"))
        return set_error(UOCR_HIP_ENOTFOUND, "no pre-quantized tensor " + base + ".packed");
    const int group = uocr_hip_gptq_group(f, fallback_group);
    if (group <= 0) return set_error(UOCR_HIP_EINVAL, "group size must be positive");
    std::unique_ptr<uocr_hip_st_file::Held> h(new uocr_hip_st_file::Held);
    if (int rc = read_u8(f, (base + ".packed").c_str(), h->packed)) return rc;
    if (int rc = read_f32(f, (base + ".scales").c_str(), h->scales)) return rc;
    if (int rc = read_f32(f, (base + ".zeros").c_str(), h->zeros)) return rc;
    const size_t ng = ((size_t)cols + group - 1) / group;
    // the reference's element-count checks (weights.cpp:157-163)
    if (h->packed.size() != (size_t)rows * (((size_t)cols + 1) / 2))
        return set_error(UOCR_HIP_EINVAL, "packed shape mismatch for " + base);
    if (h->scales.size() != (size_t)rows * ng || h->zeros.size() != (size_t)rows * ng)
        return set_error(UOCR_HIP_EINVAL, "scales/zeros shape mismatch for " + base);
    out->packed = h->packed.data();
    out->scales = h->scales.data();
    out->zeros = h->zeros.data();
    out->rows = rows;
    out->cols = cols;
    out->group_size = group;
    const_cast<uocr_hip_st_file*>(f)->held.push_back(std::move(h));
    return UOCR_HIP_OK;
}

// weights.cpp:185-197 (scale_columns) on f32 values
int uocr_hip_scale_columns_f32(const float* w, int rows, int cols, const float* s, float* out) {
    if (!w || !s || !out || rows < 0 || cols < 0) return uocr_hip::set_error(UOCR_HIP_EINVAL, "bad argument");
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) out[(size_t)r * cols + c] = w[(size_t)r * cols + c] * s[c];
    return UOCR_HIP_OK;
}

// weights.cpp:199-207 (apply_expert_input_scale) for the norm and the router
int uocr_hip_fold_expert_input_scale(const float* s, int hidden, float* rms_weight, const uint16_t* router_bf16,
                                     int n_experts, float* router_f32) {
    if (!s || !rms_weight || !router_bf16 || !router_f32 || hidden <= 0 || n_experts <= 0)
        return uocr_hip::set_error(UOCR_HIP_EINVAL, "bad argument");
    for (int j = 0; j < hidden; ++j) rms_weight[j] /= s[j];
    for (int e = 0; e < n_experts; ++e)
        for (int c = 0; c < hidden; ++c)
            router_f32[(size_t)e * hidden + c] = bf16_to_f32(router_bf16[(size_t)e * hidden + c]) * s[c];
    return UOCR_HIP_OK;
}

}  // extern "C"
