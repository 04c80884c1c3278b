// The model-file side: a safetensors reader, tensor inventories and their
// check against a file, the Depth Anything V2 inventory, and the conversions
// from a checkpoint's layouts to the IR's (include/beatlm_load.h).
//
// Host code, no GPU. The reader follows the safetensors format as version
// 0.8.0 of its reference implementation reads it (the version
// crates/beatlm's Cargo.lock pins): an 8-byte little-endian header length n
// (at most 100 000 000), n bytes of UTF-8 JSON — an object of tensor name ->
// {"dtype", "shape", "data_offsets": [begin, end]} plus an optional
// "__metadata__" object of strings — then the data. Tensors, taken in
// data-offset order, must tile the data exactly, each spanning its shape's
// element count times its type's width.
#include "../../include/beatlm_load.h"

#include <algorithm>
#include <cmath>
#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

// The bicubic resampling and the conversions do their f32 arithmetic in the
// written order, each operation rounded: no contraction into fused
// multiply-adds, as the reference computes.
#pragma clang fp contract(off)

namespace {

thread_local std::string g_error;

int fail(int code, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

uint64_t saturating_add(uint64_t a, uint64_t b) { return a > UINT64_MAX - b ? UINT64_MAX : a + b; }
uint64_t saturating_mul(uint64_t a, uint64_t b) { return (a != 0 && b > UINT64_MAX / a) ? UINT64_MAX : a * b; }

// element_count (reader.rs:160-167): the product, saturating; a scalar is 1.
uint64_t element_count(const std::vector<uint64_t> &shape) {
    uint64_t n = 1;
    for (uint64_t e : shape) n = saturating_mul(n, e);
    return n;
}

// ---- element types ----

struct DtypeInfo {
    const char *name;
    uint32_t bits;
    uint32_t stored;  // the StoredType the reader hands out
};
// The format's element types (safetensors 0.8.0 Dtype) with their widths.
const DtypeInfo DTYPES[] = {
    {"BOOL", 8, BLF_OTHER},        {"F4", 4, BLF_OTHER},          {"F6_E2M3", 6, BLF_OTHER},
    {"F6_E3M2", 6, BLF_OTHER},     {"U8", 8, BLF_U8},             {"I8", 8, BLF_OTHER},
    {"F8_E5M2", 8, BLF_OTHER},     {"F8_E4M3", 8, BLF_OTHER},     {"F8_E8M0", 8, BLF_OTHER},
    {"F8_E4M3FNUZ", 8, BLF_OTHER}, {"F8_E5M2FNUZ", 8, BLF_OTHER}, {"I16", 16, BLF_OTHER},
    {"U16", 16, BLF_OTHER},        {"F16", 16, BLF_F16},          {"BF16", 16, BLF_BF16},
    {"I32", 32, BLF_I32},          {"U32", 32, BLF_OTHER},        {"F32", 32, BLF_F32},
    {"C64", 64, BLF_OTHER},        {"F64", 64, BLF_F64},          {"I64", 64, BLF_I64},
    {"U64", 64, BLF_OTHER},
};

// ---- a strict JSON reader for the header ----
//
// RFC 8259 syntax; what the header's schema expects is checked as it is read:
// shape and offsets are arrays of non-negative integers that fit 64 bits (a
// fraction, an exponent or a sign is refused, as a float where an integer
// belongs), a tensor entry has each of its three fields exactly once (other
// fields are read and ignored), "__metadata__" at most once, as null or an
// object of strings. A tensor name given twice keeps its last entry.
struct Json {
    const char *p, *end;
    std::string why;

    bool error(const char *what) {
        if (why.empty()) why = what;
        return false;
    }
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool eat(char c) {
        ws();
        if (p < end && *p == c) {
            p++;
            return true;
        }
        return false;
    }
    bool hex4(uint32_t &v) {
        if (end - p < 4) return error("a \\u escape needs four hex digits");
        v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return error("a \\u escape needs four hex digits");
        }
        return true;
    }
    static void utf8(std::string &out, uint32_t cp) {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        } else {
            out += (char)(0xF0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3F));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool string(std::string &out) {
        ws();
        if (p >= end || *p != '"') return error("expected a string");
        p++;
        out.clear();
        while (true) {
            if (p >= end) return error("unterminated string");
            const unsigned char c = (unsigned char)*p;
            if (c == '"') {
                p++;
                return true;
            }
            if (c < 0x20) return error("control character in a string");
            if (c != '\\') {
                out += (char)c;
                p++;
                continue;
            }
            p++;
            if (p >= end) return error("unterminated escape");
            const char e = *p++;
            switch (e) {
            case '"': out += '"'; break;
            case '\\': out += '\\'; break;
            case '/': out += '/'; break;
            case 'b': out += '\b'; break;
            case 'f': out += '\f'; break;
            case 'n': out += '\n'; break;
            case 'r': out += '\r'; break;
            case 't': out += '\t'; break;
            case 'u': {
                uint32_t cp;
                if (!hex4(cp)) return false;
                if (cp >= 0xDC00 && cp <= 0xDFFF) return error("lone trailing surrogate");
                if (cp >= 0xD800 && cp <= 0xDBFF) {
                    uint32_t lo;
                    if (end - p < 2 || p[0] != '\\' || p[1] != 'u') return error("lone leading surrogate");
                    p += 2;
                    if (!hex4(lo)) return false;
                    if (lo < 0xDC00 || lo > 0xDFFF) return error("invalid surrogate pair");
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8(out, cp);
                break;
            }
            default: return error("invalid escape");
            }
        }
    }
    // Any JSON number; integer-only callers use uinteger().
    bool number() {
        ws();
        const char *q = p;
        if (q < end && *q == '-') q++;
        if (q >= end) return error("invalid number");
        if (*q == '0') q++;
        else if (*q >= '1' && *q <= '9') while (q < end && *q >= '0' && *q <= '9') q++;
        else return error("invalid number");
        if (q < end && *q == '.') {
            q++;
            if (q >= end || *q < '0' || *q > '9') return error("invalid number");
            while (q < end && *q >= '0' && *q <= '9') q++;
        }
        if (q < end && (*q == 'e' || *q == 'E')) {
            q++;
            if (q < end && (*q == '+' || *q == '-')) q++;
            if (q >= end || *q < '0' || *q > '9') return error("invalid number");
            while (q < end && *q >= '0' && *q <= '9') q++;
        }
        p = q;
        return true;
    }
    bool uinteger(uint64_t &v) {
        ws();
        const char *start = p;
        if (!number()) return false;
        v = 0;
        for (const char *q = start; q < p; q++) {
            if (*q < '0' || *q > '9') return error("expected a non-negative integer");
            const uint64_t d = (uint64_t)(*q - '0');
            if (v > (UINT64_MAX - d) / 10) return error("integer out of range");
            v = v * 10 + d;
        }
        return true;
    }
    bool literal(const char *word) {
        const size_t n = strlen(word);
        if ((size_t)(end - p) < n || memcmp(p, word, n) != 0) return error("expected a value");
        p += n;
        return true;
    }
    bool skip_value(int depth = 0) {
        if (depth > 128) return error("nesting too deep");
        ws();
        if (p >= end) return error("expected a value");
        const char c = *p;
        if (c == '"') {
            std::string s;
            return string(s);
        }
        if (c == '{') {
            p++;
            if (eat('}')) return true;
            do {
                std::string k;
                if (!string(k)) return false;
                if (!eat(':')) return error("expected ':'");
                if (!skip_value(depth + 1)) return false;
            } while (eat(','));
            return eat('}') || error("expected ',' or '}'");
        }
        if (c == '[') {
            p++;
            if (eat(']')) return true;
            do {
                if (!skip_value(depth + 1)) return false;
            } while (eat(','));
            return eat(']') || error("expected ',' or ']'");
        }
        if (c == 't') return literal("true");
        if (c == 'f') return literal("false");
        if (c == 'n') return literal("null");
        return number();
    }
    bool uint_array(std::vector<uint64_t> &out) {
        out.clear();
        if (!eat('[')) return error("expected an array");
        if (eat(']')) return true;
        do {
            uint64_t v;
            if (!uinteger(v)) return false;
            out.push_back(v);
        } while (eat(','));
        return eat(']') || error("expected ',' or ']'");
    }
};

struct Info {
    uint32_t dtype_index;
    std::vector<uint64_t> shape;
    uint64_t begin, end;
};

bool parse_info(Json &j, Info &info) {
    if (!j.eat('{')) return j.error("a tensor entry is not an object");
    bool has_dtype = false, has_shape = false, has_offsets = false;
    if (!j.eat('}')) {
        do {
            std::string key;
            if (!j.string(key)) return false;
            if (!j.eat(':')) return j.error("expected ':'");
            if (key == "dtype") {
                if (has_dtype) return j.error("duplicate field `dtype`");
                has_dtype = true;
                std::string name;
                if (!j.string(name)) return false;
                bool found = false;
                for (uint32_t i = 0; i < sizeof DTYPES / sizeof DTYPES[0]; i++)
                    if (name == DTYPES[i].name) {
                        info.dtype_index = i;
                        found = true;
                    }
                if (!found) return j.error("unknown element type");
            } else if (key == "shape") {
                if (has_shape) return j.error("duplicate field `shape`");
                has_shape = true;
                if (!j.uint_array(info.shape)) return false;
            } else if (key == "data_offsets") {
                if (has_offsets) return j.error("duplicate field `data_offsets`");
                has_offsets = true;
                std::vector<uint64_t> off;
                if (!j.uint_array(off)) return false;
                if (off.size() != 2) return j.error("data_offsets needs two integers");
                info.begin = off[0];
                info.end = off[1];
            } else if (!j.skip_value()) {
                return false;
            }
        } while (j.eat(','));
        if (!j.eat('}')) return j.error("expected ',' or '}'");
    }
    if (!has_dtype) return j.error("missing field `dtype`");
    if (!has_shape) return j.error("missing field `shape`");
    if (!has_offsets) return j.error("missing field `data_offsets`");
    return true;
}

// Strict UTF-8 (no overlong forms, no surrogates, nothing past U+10FFFF).
bool valid_utf8(const uint8_t *s, uint64_t n) {
    uint64_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) {
            i++;
            continue;
        }
        int len;
        uint32_t cp, min;
        if ((c & 0xE0) == 0xC0) len = 2, cp = c & 0x1F, min = 0x80;
        else if ((c & 0xF0) == 0xE0) len = 3, cp = c & 0x0F, min = 0x800;
        else if ((c & 0xF8) == 0xF0) len = 4, cp = c & 0x07, min = 0x10000;
        else return false;
        if (n - i < (uint64_t)len) return false;
        for (int k = 1; k < len; k++) {
            if ((s[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3F);
        }
        if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
        i += (uint64_t)len;
    }
    return true;
}

struct Tensor {
    std::string name;
    uint32_t dtype;
    std::vector<uint64_t> shape;
    const uint8_t *data;
    uint64_t bytes;
};

void fill(const Tensor &t, blf_tensor *out) {
    out->name = t.name.c_str();
    out->dtype = t.dtype;
    out->rank = (uint32_t)t.shape.size();
    out->shape = t.shape.data();
    out->data = t.data;
    out->bytes = t.bytes;
}

}  // namespace

struct blf_archive {
    std::vector<uint8_t> owned;    // the file's bytes when the archive read them
    std::vector<Tensor> tensors;   // in name order
    std::map<std::string, size_t> by_name;
};

namespace {

constexpr uint64_t MAX_HEADER = 100000000;

int parse_into(blf_archive *a, const uint8_t *bytes, uint64_t len) {
    if (len < 8) return fail(BLF_ERR_FORMAT, "not a valid safetensors file: header too small");
    uint64_t n = 0;
    for (int i = 7; i >= 0; i--) n = (n << 8) | bytes[i];
    if (n > MAX_HEADER) return fail(BLF_ERR_FORMAT, "not a valid safetensors file: header too large");
    if (n > len - 8) return fail(BLF_ERR_FORMAT, "not a valid safetensors file: invalid header length");
    const uint8_t *h = bytes + 8;
    if (!valid_utf8(h, n)) return fail(BLF_ERR_FORMAT, "not a valid safetensors file: invalid UTF-8 in header");
    Json j{(const char *)h, (const char *)h + n, {}};
    std::map<std::string, Info> infos;
    bool has_meta = false;
    if (!j.eat('{')) return fail(BLF_ERR_FORMAT, "not a valid safetensors file: the header is not a JSON object");
    bool ok = true;
    if (!j.eat('}')) {
        do {
            std::string name;
            if (!(ok = j.string(name))) break;
            if (!(ok = j.eat(':') || j.error("expected ':'"))) break;
            if (name == "__metadata__") {
                if (!(ok = !has_meta || j.error("duplicate field `__metadata__`"))) break;
                has_meta = true;
                j.ws();
                if (j.end - j.p >= 4 && memcmp(j.p, "null", 4) == 0) {
                    j.p += 4;
                    continue;
                }
                if (!(ok = j.eat('{') || j.error("__metadata__ is not an object"))) break;
                if (j.eat('}')) continue;
                do {
                    std::string k, v;
                    if (!(ok = j.string(k) && (j.eat(':') || j.error("expected ':'")) && j.string(v))) break;
                } while (j.eat(','));
                if (!ok) break;
                if (!(ok = j.eat('}') || j.error("expected ',' or '}'"))) break;
                continue;
            }
            Info info{};
            if (!(ok = parse_info(j, info))) break;
            infos[name] = info;  // a name given twice keeps its last entry
        } while (j.eat(','));
        if (ok) ok = j.eat('}') || j.error("expected ',' or '}'");
    }
    if (ok) {
        j.ws();
        if (j.p != j.end) ok = j.error("trailing characters after the header's object");
    }
    if (!ok) return fail(BLF_ERR_FORMAT, "not a valid safetensors file: invalid JSON in header: %s", j.why.c_str());

    // The tensors in data order must tile the data exactly.
    std::vector<std::pair<std::string, const Info *>> order;
    for (auto &kv : infos) order.push_back({kv.first, &kv.second});
    std::stable_sort(order.begin(), order.end(), [](const auto &x, const auto &y) {
        return std::make_pair(x.second->begin, x.second->end) < std::make_pair(y.second->begin, y.second->end);
    });
    uint64_t at = 0;
    for (auto &[name, info] : order) {
        if (info->begin != at || info->end < info->begin)
            return fail(BLF_ERR_FORMAT, "not a valid safetensors file: invalid offset for tensor `%s`", name.c_str());
        at = info->end;
        uint64_t elements = 1;
        for (uint64_t e : info->shape) {
            if (e != 0 && elements > UINT64_MAX / e)
                return fail(BLF_ERR_FORMAT, "not a valid safetensors file: overflow computing the size of `%s`", name.c_str());
            elements *= e;
        }
        const uint32_t bits = DTYPES[info->dtype_index].bits;
        if (elements > UINT64_MAX / bits)
            return fail(BLF_ERR_FORMAT, "not a valid safetensors file: overflow computing the size of `%s`", name.c_str());
        if (elements * bits % 8 != 0)
            return fail(BLF_ERR_FORMAT, "not a valid safetensors file: `%s` does not end on a byte", name.c_str());
        if (info->end - info->begin != elements * bits / 8)
            return fail(BLF_ERR_FORMAT, "not a valid safetensors file: invalid shape, data type, or offset for tensor `%s`",
                        name.c_str());
    }
    if (at != len - 8 - n)
        return fail(BLF_ERR_FORMAT, "not a valid safetensors file: incomplete metadata, file not fully covered");

    const uint8_t *data = h + n;
    a->tensors.clear();
    a->by_name.clear();
    for (auto &kv : infos) {  // std::map: name order
        Tensor t;
        t.name = kv.first;
        t.dtype = DTYPES[kv.second.dtype_index].stored;
        t.shape = kv.second.shape;
        t.data = data + kv.second.begin;
        t.bytes = kv.second.end - kv.second.begin;
        a->by_name[t.name] = a->tensors.size();
        a->tensors.push_back(std::move(t));
    }
    return BLF_OK;
}

// ---- layouts and conversions ----

std::string layout_text(uint32_t dtype, const std::vector<uint64_t> &shape) {
    std::string s = blf_stored_type_name(dtype);
    s += " [";
    for (size_t i = 0; i < shape.size(); i++) {
        if (i) s += ", ";
        s += std::to_string(shape[i]);
    }
    return s + "]";
}

// The cubic convolution with A = -0.75 (positions.rs:55-67): the weight at a
// distance x of at most one, and between one and two.
constexpr float CUBIC_A = -0.75f;
float near_weight(float x) { return ((CUBIC_A + 2.0f) * x - (CUBIC_A + 3.0f)) * x * x + 1.0f; }
float far_weight(float x) { return ((CUBIC_A * x - 5.0f * CUBIC_A) * x + 8.0f * CUBIC_A) * x - 4.0f * CUBIC_A; }

struct Tap {
    uint64_t at[4];
    float w[4];
};

// One axis of n samples resampled to m (positions.rs:72-91): output o reads
// source position ratio (o + 0.5) - 0.5 with ratio = n / m in f32, its floor
// clamped to n - 1, the fraction clamped to [0, 1], the four indices around
// it clamped to the axis.
std::vector<Tap> axis(uint64_t n, uint64_t m) {
    std::vector<Tap> taps(m);
    const int64_t last = (int64_t)n - 1;
    const float ratio = (float)n / (float)m;
    for (uint64_t o = 0; o < m; o++) {
        const float real = ratio * ((float)o + 0.5f) - 0.5f;
        const int64_t index = std::min((int64_t)std::floor(real), last);
        const float t = std::min(std::max(real - (float)index, 0.0f), 1.0f);
        const float rest = 1.0f - t;
        taps[o].w[0] = far_weight(t + 1.0f);
        taps[o].w[1] = near_weight(t);
        taps[o].w[2] = near_weight(rest);
        taps[o].w[3] = far_weight(rest + 1.0f);
        for (int k = 0; k < 4; k++) taps[o].at[k] = (uint64_t)std::min(std::max(index - 1 + k, (int64_t)0), last);
    }
    return taps;
}

// The grid [from_h][from_w][c] resampled to [to_h][to_w][c] (positions.rs:93-
// 120): along the width first for each of the four rows, then down the height.
void resample(const float *grid, uint64_t from_h, uint64_t from_w, uint64_t to_h, uint64_t to_w, uint64_t c, float *out) {
    const std::vector<Tap> rows = axis(from_h, to_h), cols = axis(from_w, to_w);
    auto at = [&](uint64_t y, uint64_t x, uint64_t ch) { return grid[(y * from_w + x) * c + ch]; };
    for (const Tap &ty : rows)
        for (const Tap &tx : cols)
            for (uint64_t ch = 0; ch < c; ch++) {
                auto along = [&](uint64_t y) {
                    return at(y, tx.at[0], ch) * tx.w[0] + at(y, tx.at[1], ch) * tx.w[1] + at(y, tx.at[2], ch) * tx.w[2] +
                           at(y, tx.at[3], ch) * tx.w[3];
                };
                *out++ = along(ty.at[0]) * ty.w[0] + along(ty.at[1]) * ty.w[1] + along(ty.at[2]) * ty.w[2] +
                         along(ty.at[3]) * ty.w[3];
            }
}

uint64_t isqrt(uint64_t v) {
    uint64_t r = (uint64_t)std::sqrt((double)v);
    while (r * r > v) r--;
    while ((r + 1) * (r + 1) <= v) r++;
    return r;
}

// convert() (model/mod.rs:274-335) into out (out_len elements): false when
// the conversion does not apply to the shape.
bool convert(uint32_t how, const float *v, const std::vector<uint64_t> &shape, uint32_t height, uint32_t width,
             std::vector<float> &out, uint64_t &cols) {
    const uint64_t n = element_count(shape);
    switch (how) {
    case BLF_AS_STORED:
        out.assign(v, v + n);
        cols = shape.empty() ? 1 : shape.back();
        return true;
    case BLF_LINEAR: {
        if (shape.size() != 2) return false;
        const uint64_t o_n = shape[0], i_n = shape[1];
        out.assign(n, 0.0f);
        for (uint64_t o = 0; o < o_n; o++)
            for (uint64_t i = 0; i < i_n; i++) out[i * o_n + o] = v[o * i_n + i];
        cols = o_n;
        return true;
    }
    case BLF_CONV: {
        if (shape.size() != 4) return false;
        const uint64_t o_n = shape[0], i_n = shape[1], kh = shape[2], kw = shape[3];
        out.assign(n, 0.0f);
        for (uint64_t o = 0; o < o_n; o++)
            for (uint64_t i = 0; i < i_n; i++)
                for (uint64_t y = 0; y < kh; y++)
                    for (uint64_t x = 0; x < kw; x++) out[((y * kw + x) * i_n + i) * o_n + o] = v[((o * i_n + i) * kh + y) * kw + x];
        cols = o_n;
        return true;
    }
    case BLF_CONV_TRANSPOSE: {
        if (shape.size() != 4) return false;
        const uint64_t i_n = shape[0], o_n = shape[1], kh = shape[2], kw = shape[3];
        out.assign(n, 0.0f);
        for (uint64_t i = 0; i < i_n; i++)
            for (uint64_t o = 0; o < o_n; o++)
                for (uint64_t y = 0; y < kh; y++)
                    for (uint64_t x = 0; x < kw; x++) out[((y * kw + x) * i_n + i) * o_n + o] = v[((i * o_n + o) * kh + y) * kw + x];
        cols = o_n;
        return true;
    }
    case BLF_INTERPOLATE_POSITIONS: {
        // interpolate() (positions.rs:122-146): the class row kept, the square
        // grid behind it resampled to height x width.
        if (shape.size() != 3 || shape[0] != 1 || shape[1] == 0) return false;
        const uint64_t rows = shape[1], c = shape[2], positions = rows - 1, side = isqrt(positions);
        if (side * side != positions || side == 0 || c == 0 || height == 0 || width == 0) return false;
        out.assign((1 + (uint64_t)height * width) * c, 0.0f);
        std::copy(v, v + c, out.begin());
        resample(v + c, side, side, height, width, c, out.data() + c);
        cols = c;
        return true;
    }
    default: return false;
    }
}

}  // namespace

// ---- element types ----

extern "C" const char *blf_last_error(void) { return g_error.c_str(); }

extern "C" uint32_t blf_stored_type_size(uint32_t dtype) {
    switch (dtype) {
    case BLF_F32:
    case BLF_I32: return 4;
    case BLF_F16:
    case BLF_BF16: return 2;
    case BLF_F64:
    case BLF_I64: return 8;
    case BLF_U8: return 1;
    default: return 0;
    }
}

extern "C" const char *blf_stored_type_name(uint32_t dtype) {
    static const char *names[] = {"F32", "F16", "BF16", "F64", "U8", "I32", "I64", "other"};
    return names[dtype < BLF_OTHER ? dtype : BLF_OTHER];
}

// ---- the reader ----

extern "C" int blf_archive_parse(const uint8_t *bytes, uint64_t len, blf_archive **out) {
    if (!out || (!bytes && len)) return fail(BLF_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    blf_archive *a = new blf_archive();
    const int rc = parse_into(a, bytes, len);
    if (rc != BLF_OK) {
        delete a;
        return rc;
    }
    *out = a;
    return BLF_OK;
}

extern "C" int blf_archive_open(const char *path, blf_archive **out) {
    if (!path || !out) return fail(BLF_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    FILE *f = fopen(path, "rb");
    if (!f) return fail(BLF_ERR_IO, "cannot read %s: %s", path, strerror(errno));
    blf_archive *a = new blf_archive();
    bool ok = fseek(f, 0, SEEK_END) == 0;
    const long size = ok ? ftell(f) : -1;
    ok = ok && size >= 0 && fseek(f, 0, SEEK_SET) == 0;
    if (ok) {
        a->owned.resize((size_t)size);
        ok = size == 0 || fread(a->owned.data(), 1, (size_t)size, f) == (size_t)size;
    }
    const int err = errno;
    fclose(f);
    if (!ok) {
        delete a;
        return fail(BLF_ERR_IO, "cannot read %s: %s", path, strerror(err));
    }
    const int rc = parse_into(a, a->owned.data(), a->owned.size());
    if (rc != BLF_OK) {
        delete a;
        return rc;
    }
    *out = a;
    return BLF_OK;
}

extern "C" void blf_archive_destroy(blf_archive *a) { delete a; }

extern "C" uint64_t blf_archive_len(const blf_archive *a) { return a ? a->tensors.size() : 0; }

extern "C" int blf_archive_at(const blf_archive *a, uint64_t index, blf_tensor *out) {
    if (!a || !out) return fail(BLF_ERR_INVALID_ARGUMENT, "null argument");
    if (index >= a->tensors.size()) return fail(BLF_ERR_INVALID_ARGUMENT, "there is no tensor %llu", (unsigned long long)index);
    fill(a->tensors[index], out);
    return BLF_OK;
}

extern "C" int blf_archive_get(const blf_archive *a, const char *name, blf_tensor *out) {
    if (!a || !name || !out) return fail(BLF_ERR_INVALID_ARGUMENT, "null argument");
    auto it = a->by_name.find(name);
    if (it == a->by_name.end()) return fail(BLF_ERR_MISSING_TENSOR, "tensor `%s` is not in the file", name);
    fill(a->tensors[it->second], out);
    return BLF_OK;
}

extern "C" uint64_t blf_archive_parameter_count(const blf_archive *a) {
    uint64_t n = 0;
    if (a)
        for (const Tensor &t : a->tensors) n = saturating_add(n, element_count(t.shape));
    return n;
}

// ---- inventories ----

struct blf_inventory {
    struct Spec {
        std::string name;
        uint32_t dtype;
        std::vector<uint64_t> shape;
        blf_role role;
    };
    std::vector<Spec> specs;
    std::map<std::string, size_t> by_name;
};

namespace {
void fill_spec(const blf_inventory::Spec &s, blf_spec *out) {
    out->name = s.name.c_str();
    out->dtype = s.dtype;
    out->rank = (uint32_t)s.shape.size();
    out->shape = s.shape.data();
    out->role = s.role;
}
bool same_role(const blf_role &a, const blf_role &b) {
    return a.kind == b.kind && a.index == b.index && a.part == b.part && a.param == b.param && a.unit == b.unit && a.conv == b.conv;
}
int inventory_from(std::vector<blf_inventory::Spec> specs, blf_inventory **out) {
    blf_inventory *inv = new blf_inventory();
    for (size_t i = 0; i < specs.size(); i++) {
        if (!inv->by_name.emplace(specs[i].name, i).second) {
            const std::string name = specs[i].name;
            delete inv;
            return fail(BLF_ERR_DUPLICATE_NAME, "tensor name `%s` appears twice in the inventory", name.c_str());
        }
    }
    inv->specs = std::move(specs);
    *out = inv;
    return BLF_OK;
}
}  // namespace

extern "C" int blf_inventory_new(const blf_spec *specs, uint64_t count, blf_inventory **out) {
    if (!out || (!specs && count)) return fail(BLF_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    std::vector<blf_inventory::Spec> v;
    v.reserve(count);
    for (uint64_t i = 0; i < count; i++) {
        if (!specs[i].name || (!specs[i].shape && specs[i].rank)) return fail(BLF_ERR_INVALID_ARGUMENT, "spec %llu: null name or shape", (unsigned long long)i);
        v.push_back({specs[i].name, specs[i].dtype, std::vector<uint64_t>(specs[i].shape, specs[i].shape + specs[i].rank), specs[i].role});
    }
    return inventory_from(std::move(v), out);
}

extern "C" void blf_inventory_destroy(blf_inventory *inv) { delete inv; }
extern "C" uint64_t blf_inventory_len(const blf_inventory *inv) { return inv ? inv->specs.size() : 0; }

extern "C" int blf_inventory_at(const blf_inventory *inv, uint64_t index, blf_spec *out) {
    if (!inv || !out) return fail(BLF_ERR_INVALID_ARGUMENT, "null argument");
    if (index >= inv->specs.size()) return fail(BLF_ERR_INVALID_ARGUMENT, "there is no spec %llu", (unsigned long long)index);
    fill_spec(inv->specs[index], out);
    return BLF_OK;
}

extern "C" int blf_inventory_get(const blf_inventory *inv, const char *name, blf_spec *out) {
    if (!inv || !name || !out) return fail(BLF_ERR_INVALID_ARGUMENT, "null argument");
    auto it = inv->by_name.find(name);
    if (it == inv->by_name.end()) return fail(BLF_ERR_MISSING_TENSOR, "tensor `%s` is not in the inventory", name);
    fill_spec(inv->specs[it->second], out);
    return BLF_OK;
}

extern "C" int blf_inventory_by_role(const blf_inventory *inv, const blf_role *role, blf_spec *out) {
    if (!inv || !role || !out) return fail(BLF_ERR_INVALID_ARGUMENT, "null argument");
    for (const auto &s : inv->specs)
        if (same_role(s.role, *role)) {
            fill_spec(s, out);
            return BLF_OK;
        }
    return fail(BLF_ERR_UNKNOWN_ROLE, "no tensor of role (kind %u, index %u, part %u, param %u, unit %u, conv %u)", role->kind,
                role->index, role->part, role->param, role->unit, role->conv);
}

extern "C" uint64_t blf_inventory_parameter_count(const blf_inventory *inv) {
    uint64_t n = 0;
    if (inv)
        for (const auto &s : inv->specs) n = saturating_add(n, element_count(s.shape));
    return n;
}

struct blf_report {
    struct Layout {
        uint32_t dtype;
        std::vector<uint64_t> shape;
    };
    struct Mismatch {
        std::string name;
        Layout expected, found;
    };
    std::vector<std::string> missing, unexpected;
    std::vector<Mismatch> mismatched;
    uint64_t expected_parameters = 0, file_parameters = 0;
    std::string text;
};

extern "C" int blf_inventory_check(const blf_inventory *inv, const blf_archive *a, blf_report **out) {
    if (!inv || !a || !out) return fail(BLF_ERR_INVALID_ARGUMENT, "null argument");
    blf_report *r = new blf_report();
    for (const auto &s : inv->specs) {
        auto it = a->by_name.find(s.name);
        if (it == a->by_name.end()) {
            r->missing.push_back(s.name);
            continue;
        }
        const Tensor &t = a->tensors[it->second];
        if (t.dtype != s.dtype || t.shape != s.shape) r->mismatched.push_back({s.name, {s.dtype, s.shape}, {t.dtype, t.shape}});
    }
    for (const Tensor &t : a->tensors)
        if (!inv->by_name.count(t.name)) r->unexpected.push_back(t.name);
    r->expected_parameters = blf_inventory_parameter_count(inv);
    r->file_parameters = blf_archive_parameter_count(a);
    // CheckReport's Display (inventory.rs:210-245).
    if (r->missing.empty() && r->unexpected.empty() && r->mismatched.empty()) {
        r->text = "the file matches the inventory exactly: " + std::to_string(r->file_parameters) + " parameters";
    } else {
        r->text = "the file does not match the inventory: " + std::to_string(r->missing.size()) + " missing, " +
                  std::to_string(r->unexpected.size()) + " unexpected, " + std::to_string(r->mismatched.size()) +
                  " mismatched (inventory " + std::to_string(r->expected_parameters) + " parameters, file " +
                  std::to_string(r->file_parameters) + ")";
        for (const auto &n : r->missing) r->text += "\n  missing    " + n;
        for (const auto &n : r->unexpected) r->text += "\n  unexpected " + n;
        for (const auto &m : r->mismatched)
            r->text += "\n  mismatch   " + m.name + ": expected " + layout_text(m.expected.dtype, m.expected.shape) + ", found " +
                       layout_text(m.found.dtype, m.found.shape);
    }
    *out = r;
    return BLF_OK;
}

extern "C" void blf_report_destroy(blf_report *r) { delete r; }
extern "C" int blf_report_is_exact(const blf_report *r) {
    return r && r->missing.empty() && r->unexpected.empty() && r->mismatched.empty();
}
extern "C" uint64_t blf_report_missing_len(const blf_report *r) { return r ? r->missing.size() : 0; }
extern "C" const char *blf_report_missing(const blf_report *r, uint64_t i) {
    return r && i < r->missing.size() ? r->missing[i].c_str() : nullptr;
}
extern "C" uint64_t blf_report_unexpected_len(const blf_report *r) { return r ? r->unexpected.size() : 0; }
extern "C" const char *blf_report_unexpected(const blf_report *r, uint64_t i) {
    return r && i < r->unexpected.size() ? r->unexpected[i].c_str() : nullptr;
}
extern "C" uint64_t blf_report_mismatched_len(const blf_report *r) { return r ? r->mismatched.size() : 0; }
extern "C" int blf_report_mismatch(const blf_report *r, uint64_t i, const char **name, blf_tensor *expected, blf_tensor *found) {
    if (!r || !name || !expected || !found) return fail(BLF_ERR_INVALID_ARGUMENT, "null argument");
    if (i >= r->mismatched.size()) return fail(BLF_ERR_INVALID_ARGUMENT, "there is no mismatch %llu", (unsigned long long)i);
    const auto &m = r->mismatched[i];
    *name = m.name.c_str();
    *expected = blf_tensor{m.name.c_str(), m.expected.dtype, (uint32_t)m.expected.shape.size(), m.expected.shape.data(), nullptr, 0};
    *found = blf_tensor{m.name.c_str(), m.found.dtype, (uint32_t)m.found.shape.size(), m.found.shape.data(), nullptr, 0};
    return BLF_OK;
}
extern "C" uint64_t blf_report_expected_parameters(const blf_report *r) { return r ? r->expected_parameters : 0; }
extern "C" uint64_t blf_report_file_parameters(const blf_report *r) { return r ? r->file_parameters : 0; }
extern "C" const char *blf_report_text(const blf_report *r) { return r ? r->text.c_str() : ""; }

// ---- Depth Anything V2 ----

extern "C" void blf_dav2_small(blf_dav2_config *c) {
    if (!c) return;
    *c = blf_dav2_config{};
    c->image_size = 518;
    c->patch_size = 14;
    c->num_channels = 3;
    c->hidden_size = 384;
    c->num_layers = 12;
    c->num_heads = 6;
    c->mlp_ratio = 4;
    c->mask_token = 1;
    c->stages = 4;
    const uint32_t taps[4] = {3, 6, 9, 12}, necks[4] = {48, 96, 192, 384};
    const uint32_t kinds[4] = {BLF_UP, BLF_UP, BLF_KEEP, BLF_DOWN}, factors[4] = {4, 2, 0, 2};
    for (int i = 0; i < 4; i++) {
        c->out_indices[i] = taps[i];
        c->neck_hidden_sizes[i] = necks[i];
        c->resample[i] = kinds[i];
        c->factor[i] = factors[i];
    }
    c->fusion_hidden_size = 64;
    c->head_hidden_size = 32;
}

namespace {
int config_fail(uint32_t *variant, uint32_t which, const char *fmt, ...) {
    if (variant) *variant = which;
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return BLF_ERR_CONFIG;
}
}  // namespace

// Config::validate (depth_anything_v2.rs:170-250), its rules in its order.
extern "C" int blf_dav2_validate(const blf_dav2_config *c, uint32_t *variant) {
    if (variant) *variant = 0;
    if (!c) return fail(BLF_ERR_INVALID_ARGUMENT, "null argument");
    const std::pair<const char *, uint32_t> sizes[] = {
        {"image_size", c->image_size},     {"patch_size", c->patch_size},   {"num_channels", c->num_channels},
        {"hidden_size", c->hidden_size},   {"num_layers", c->num_layers},   {"num_heads", c->num_heads},
        {"mlp_ratio", c->mlp_ratio},       {"fusion_hidden_size", c->fusion_hidden_size},
        {"head_hidden_size", c->head_hidden_size}};
    for (auto &[field, value] : sizes)
        if (value == 0) return config_fail(variant, BLF_CONFIG_ZERO, "`%s` must be positive", field);
    if (c->hidden_size % c->num_heads)
        return config_fail(variant, BLF_CONFIG_HEADS_DO_NOT_DIVIDE_HIDDEN, "hidden size %u is not divisible by %u heads",
                           c->hidden_size, c->num_heads);
    if (c->image_size % c->patch_size)
        return config_fail(variant, BLF_CONFIG_IMAGE_NOT_WHOLE_PATCHES, "image size %u is not a multiple of patch size %u",
                           c->image_size, c->patch_size);
    if (c->fusion_hidden_size % 2)
        return config_fail(variant, BLF_CONFIG_FUSION_WIDTH_ODD, "fusion width %u is odd, and the head halves it",
                           c->fusion_hidden_size);
    // One count serves the three stage lists here; a list of another length
    // cannot be given through this struct, so `stages` out of range is the
    // mismatch.
    if (c->stages == 0 || c->stages > BLF_MAX_STAGES)
        return config_fail(variant, BLF_CONFIG_STAGE_COUNT_MISMATCH, "stage lists disagree: %u stages", c->stages);
    for (uint32_t s = 0; s < c->stages; s++)
        if (c->neck_hidden_sizes[s] == 0) return config_fail(variant, BLF_CONFIG_ZERO, "`neck_hidden_sizes` must be positive");
    for (uint32_t s = 0; s < c->stages; s++)
        if (c->resample[s] != BLF_KEEP && c->factor[s] == 0) return config_fail(variant, BLF_CONFIG_ZERO, "`reassemble` must be positive");
    for (uint32_t s = 0; s < c->stages; s++)
        if (c->resample[s] != BLF_KEEP && c->factor[s] == 1)
            return config_fail(variant, BLF_CONFIG_RESAMPLE_BY_ONE, "stage %u resamples by a factor of one; use `Resample::Keep`", s);
    for (uint32_t s = 0; s < c->stages; s++)
        if (c->resample[s] > BLF_DOWN) return fail(BLF_ERR_INVALID_ARGUMENT, "stage %u: resample kind %u", s, c->resample[s]);
    for (uint32_t s = 0; s < c->stages; s++)
        if (c->out_indices[s] == 0 || c->out_indices[s] > c->num_layers)
            return config_fail(variant, BLF_CONFIG_OUT_INDEX_OUT_OF_RANGE, "out index %u is not a layer of a %u-layer transformer",
                               c->out_indices[s], c->num_layers);
    for (uint32_t s = 1; s < c->stages; s++)
        if (c->out_indices[s - 1] >= c->out_indices[s])
            return config_fail(variant, BLF_CONFIG_OUT_INDICES_NOT_INCREASING, "out indices are not strictly increasing");
    return BLF_OK;
}

// inventory() (depth_anything_v2.rs:462-620): the checkpoint's tensors in the
// reference's order, every one F32.
extern "C" int blf_dav2_inventory(const blf_dav2_config *c, blf_inventory **out, uint32_t *variant) {
    if (!out) return fail(BLF_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    const int rc = blf_dav2_validate(c, variant);
    if (rc != BLF_OK) return rc;
    std::vector<blf_inventory::Spec> specs;
    auto push = [&](std::string name, std::vector<uint64_t> shape, blf_role role) {
        specs.push_back({std::move(name), BLF_F32, std::move(shape), role});
    };
    auto role = [](uint32_t kind, uint32_t index = 0, uint32_t part = 0, uint32_t param = 0, uint32_t unit = 0, uint32_t conv = 0) {
        return blf_role{kind, index, part, param, unit, conv};
    };
    const uint64_t hidden = c->hidden_size, mlp = (uint64_t)c->hidden_size * c->mlp_ratio;
    const uint64_t grid = c->image_size / c->patch_size, tokens = grid * grid + 1;

    push("backbone.embeddings.cls_token", {1, 1, hidden}, role(BLF_ROLE_CLASS_TOKEN));
    if (c->mask_token) push("backbone.embeddings.mask_token", {1, hidden}, role(BLF_ROLE_MASK_TOKEN));
    push("backbone.embeddings.position_embeddings", {1, tokens, hidden}, role(BLF_ROLE_POSITION_EMBEDDING));
    const std::string patch = "backbone.embeddings.patch_embeddings.projection";
    push(patch + ".weight", {hidden, c->num_channels, c->patch_size, c->patch_size},
         role(BLF_ROLE_PATCH_PROJECTION, 0, 0, BLF_PARAM_WEIGHT));
    push(patch + ".bias", {hidden}, role(BLF_ROLE_PATCH_PROJECTION, 0, 0, BLF_PARAM_BIAS));

    for (uint32_t layer = 0; layer < c->num_layers; layer++) {
        const std::string p = "backbone.encoder.layer." + std::to_string(layer) + ".";
        auto block = [&](const char *suffix, std::vector<uint64_t> shape, uint32_t part, uint32_t param = 0) {
            push(p + suffix, std::move(shape), role(BLF_ROLE_BLOCK, layer, part, param));
        };
        block("norm1.weight", {hidden}, BLF_BLOCK_NORM1, BLF_PARAM_WEIGHT);
        block("norm1.bias", {hidden}, BLF_BLOCK_NORM1, BLF_PARAM_BIAS);
        block("attention.attention.query.weight", {hidden, hidden}, BLF_BLOCK_QUERY, BLF_PARAM_WEIGHT);
        block("attention.attention.query.bias", {hidden}, BLF_BLOCK_QUERY, BLF_PARAM_BIAS);
        block("attention.attention.key.weight", {hidden, hidden}, BLF_BLOCK_KEY, BLF_PARAM_WEIGHT);
        block("attention.attention.key.bias", {hidden}, BLF_BLOCK_KEY, BLF_PARAM_BIAS);
        block("attention.attention.value.weight", {hidden, hidden}, BLF_BLOCK_VALUE, BLF_PARAM_WEIGHT);
        block("attention.attention.value.bias", {hidden}, BLF_BLOCK_VALUE, BLF_PARAM_BIAS);
        block("attention.output.dense.weight", {hidden, hidden}, BLF_BLOCK_ATTENTION_OUTPUT, BLF_PARAM_WEIGHT);
        block("attention.output.dense.bias", {hidden}, BLF_BLOCK_ATTENTION_OUTPUT, BLF_PARAM_BIAS);
        block("layer_scale1.lambda1", {hidden}, BLF_BLOCK_LAYER_SCALE1);
        block("norm2.weight", {hidden}, BLF_BLOCK_NORM2, BLF_PARAM_WEIGHT);
        block("norm2.bias", {hidden}, BLF_BLOCK_NORM2, BLF_PARAM_BIAS);
        block("mlp.fc1.weight", {mlp, hidden}, BLF_BLOCK_MLP_FC1, BLF_PARAM_WEIGHT);
        block("mlp.fc1.bias", {mlp}, BLF_BLOCK_MLP_FC1, BLF_PARAM_BIAS);
        block("mlp.fc2.weight", {hidden, mlp}, BLF_BLOCK_MLP_FC2, BLF_PARAM_WEIGHT);
        block("mlp.fc2.bias", {hidden}, BLF_BLOCK_MLP_FC2, BLF_PARAM_BIAS);
        block("layer_scale2.lambda1", {hidden}, BLF_BLOCK_LAYER_SCALE2);
    }
    push("backbone.layernorm.weight", {hidden}, role(BLF_ROLE_FINAL_NORM, 0, 0, BLF_PARAM_WEIGHT));
    push("backbone.layernorm.bias", {hidden}, role(BLF_ROLE_FINAL_NORM, 0, 0, BLF_PARAM_BIAS));

    const uint64_t fusion = c->fusion_hidden_size;
    for (uint32_t stage = 0; stage < c->stages; stage++) {
        const uint64_t ch = c->neck_hidden_sizes[stage];
        const std::string p = "neck.reassemble_stage.layers." + std::to_string(stage) + ".";
        push(p + "projection.weight", {ch, hidden, 1, 1}, role(BLF_ROLE_REASSEMBLE, stage, BLF_PART_PROJECTION, BLF_PARAM_WEIGHT));
        push(p + "projection.bias", {ch}, role(BLF_ROLE_REASSEMBLE, stage, BLF_PART_PROJECTION, BLF_PARAM_BIAS));
        if (c->resample[stage] != BLF_KEEP) {
            const uint64_t kernel = c->resample[stage] == BLF_UP ? c->factor[stage] : 3;
            push(p + "resize.weight", {ch, ch, kernel, kernel}, role(BLF_ROLE_REASSEMBLE, stage, BLF_PART_RESIZE, BLF_PARAM_WEIGHT));
            push(p + "resize.bias", {ch}, role(BLF_ROLE_REASSEMBLE, stage, BLF_PART_RESIZE, BLF_PARAM_BIAS));
        }
        push("neck.convs." + std::to_string(stage) + ".weight", {fusion, ch, 3, 3}, role(BLF_ROLE_NECK_CONV, stage));
    }
    for (uint32_t layer = 0; layer < c->stages; layer++) {
        const std::string p = "neck.fusion_stage.layers." + std::to_string(layer) + ".";
        push(p + "projection.weight", {fusion, fusion, 1, 1}, role(BLF_ROLE_FUSION, layer, BLF_PART_PROJECTION, BLF_PARAM_WEIGHT));
        push(p + "projection.bias", {fusion}, role(BLF_ROLE_FUSION, layer, BLF_PART_PROJECTION, BLF_PARAM_BIAS));
        for (uint32_t unit = 0; unit < 2; unit++)
            for (uint32_t conv = 0; conv < 2; conv++) {
                const std::string stem = p + "residual_layer" + std::to_string(unit + 1) + ".convolution" + std::to_string(conv + 1);
                push(stem + ".weight", {fusion, fusion, 3, 3}, role(BLF_ROLE_FUSION, layer, BLF_PART_RESIDUAL, BLF_PARAM_WEIGHT, unit, conv));
                push(stem + ".bias", {fusion}, role(BLF_ROLE_FUSION, layer, BLF_PART_RESIDUAL, BLF_PARAM_BIAS, unit, conv));
            }
    }
    const uint64_t half = fusion / 2, head = c->head_hidden_size;
    const std::vector<uint64_t> shapes[3] = {{half, fusion, 3, 3}, {head, half, 3, 3}, {1, head, 1, 1}};
    const uint64_t biases[3] = {half, head, 1};
    for (uint32_t conv = 0; conv < 3; conv++) {
        const std::string p = "head.conv" + std::to_string(conv + 1);
        push(p + ".weight", shapes[conv], role(BLF_ROLE_HEAD, 0, 0, BLF_PARAM_WEIGHT, 0, conv));
        push(p + ".bias", {biases[conv]}, role(BLF_ROLE_HEAD, 0, 0, BLF_PARAM_BIAS, 0, conv));
    }
    return inventory_from(std::move(specs), out);
}

// ---- conversions ----

extern "C" int blf_convert(uint32_t how, const float *values, const uint64_t *shape, uint32_t rank, uint32_t height,
                           uint32_t width, float *out, uint64_t out_len, uint64_t *written, uint64_t *cols) {
    if ((!values && rank) || (!shape && rank) || !out || !written || !cols) return fail(BLF_ERR_INVALID_ARGUMENT, "null argument");
    const std::vector<uint64_t> sh(shape, shape + rank);
    std::vector<float> result;
    uint64_t c = 0;
    if (!convert(how, values, sh, height, width, result, c))
        return fail(BLF_ERR_CONVERT, "conversion %u does not apply to a tensor of shape %s", how, layout_text(BLF_F32, sh).c_str() + 4);
    if (result.size() > out_len)
        return fail(BLF_ERR_INVALID_ARGUMENT, "the result has %llu elements, the buffer %llu", (unsigned long long)result.size(),
                    (unsigned long long)out_len);
    std::copy(result.begin(), result.end(), out);
    *written = result.size();
    *cols = c;
    return BLF_OK;
}

extern "C" int blf_weight_numbers(const blf_inventory *inv, const blf_archive *a, const blf_role *parts, uint32_t n_parts,
                                  uint32_t how, uint32_t height, uint32_t width, float *out, uint64_t elements) {
    if (!inv || !a || (!parts && n_parts) || (!out && elements)) return fail(BLF_ERR_INVALID_ARGUMENT, "null argument");
    std::vector<std::pair<std::vector<float>, uint64_t>> converted;
    for (uint32_t i = 0; i < n_parts; i++) {
        blf_spec spec;
        int rc = blf_inventory_by_role(inv, &parts[i], &spec);
        if (rc != BLF_OK) return rc;
        blf_tensor t;
        rc = blf_archive_get(a, spec.name, &t);
        if (rc != BLF_OK) return rc;
        const std::vector<uint64_t> want(spec.shape, spec.shape + spec.rank), got(t.shape, t.shape + t.rank);
        if (t.dtype != BLF_F32 || got != want)
            return fail(BLF_ERR_LAYOUT, "tensor `%s` is stored as %s, expected %s", spec.name, layout_text(t.dtype, got).c_str(),
                        layout_text(BLF_F32, want).c_str());
        // Little-endian f32 bytes, read without assuming their alignment.
        std::vector<float> values(element_count(got));
        memcpy(values.data(), t.data, values.size() * sizeof(float));
        std::vector<float> result;
        uint64_t cols = 0;
        if (!convert(how, values.data(), got, height, width, result, cols))
            return fail(BLF_ERR_CONVERT, "conversion %u does not apply to `%s` of shape %s", how, spec.name,
                        layout_text(BLF_F32, got).c_str() + 4);
        converted.push_back({std::move(result), cols});
    }
    // side_by_side (model/mod.rs:337-353): row r of every part in turn.
    uint64_t given = 0;
    for (auto &p : converted) given = saturating_add(given, p.first.size());
    auto size_error = [&](uint64_t g) {
        return fail(BLF_ERR_SOURCE_SIZE, "the parts give %llu numbers, the weight has %llu", (unsigned long long)g,
                    (unsigned long long)elements);
    };
    std::vector<float> numbers;
    if (converted.size() == 1) {
        numbers = std::move(converted[0].first);
    } else if (!converted.empty()) {
        auto rows_of = [](const std::pair<std::vector<float>, uint64_t> &p, uint64_t &rows) {
            if (p.second == 0) return false;
            rows = p.first.size() / p.second;
            return true;
        };
        uint64_t rows = 0;
        if (!rows_of(converted[0], rows)) return size_error(given);
        for (auto &p : converted) {
            uint64_t r;
            if (!rows_of(p, r) || r != rows) return size_error(given);
        }
        numbers.reserve(given);
        for (uint64_t r = 0; r < rows; r++)
            for (auto &p : converted) numbers.insert(numbers.end(), p.first.begin() + r * p.second, p.first.begin() + (r + 1) * p.second);
    }
    if (numbers.size() != elements) return size_error(numbers.size());
    std::copy(numbers.begin(), numbers.end(), out);
    return BLF_OK;
}
