// qweights.cpp -- safetensors header parsing for quantized linear layers
// (host code; the device upload is in hip_backend.hip).
//
// File: u64 little-endian header length H, H bytes of UTF-8 JSON (an object
// mapping tensor names to {"dtype", "shape", "data_offsets"}, plus an
// optional "__metadata__" object of string values), then the data; offsets
// are relative to the first data byte.
#include "qweights.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

namespace lxq {

MappedFile::~MappedFile() {
    if (data) munmap(const_cast<uint8_t*>(data), size);
}

bool MappedFile::open(const char* path) {
    if (!path) return false;
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return false;
    struct stat st;
    bool ok = fstat(fd, &st) == 0 && S_ISREG(st.st_mode) && st.st_size > 0;
    if (ok) {
        void* p = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
        ok = p != MAP_FAILED;
        if (ok) {
            data = static_cast<const uint8_t*>(p);
            size = (size_t)st.st_size;
        }
    }
    ::close(fd);
    return ok;
}

namespace {

// ---- a small JSON reader: enough for safetensors headers ------------------

struct JValue {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    std::string text;                                 // String value, or Number literal
    std::vector<JValue> items;                        // Array
    std::vector<std::pair<std::string, JValue>> members;  // Object (file order)

    const JValue* get(const std::string& k) const {
        if (kind != Object) return nullptr;
        for (const auto& m : members)
            if (m.first == k) return &m.second;
        return nullptr;
    }
};

class JParser {
  public:
    JParser(const char* p, const char* end) : p_(p), end_(end) {}

    bool parse_document(JValue& v) {
        if (!value(v, 0)) return false;
        ws();
        return p_ == end_;
    }

  private:
    const char* p_;
    const char* end_;

    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
    }
    bool lit(const char* s) {
        const size_t n = std::strlen(s);
        if ((size_t)(end_ - p_) < n || std::memcmp(p_, s, n) != 0) return false;
        p_ += n;
        return true;
    }
    static void put_utf8(std::string& o, uint32_t c) {
        if (c < 0x80) {
            o += (char)c;
        } else if (c < 0x800) {
            o += (char)(0xC0 | (c >> 6));
            o += (char)(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            o += (char)(0xE0 | (c >> 12));
            o += (char)(0x80 | ((c >> 6) & 0x3F));
            o += (char)(0x80 | (c & 0x3F));
        } else {
            o += (char)(0xF0 | (c >> 18));
            o += (char)(0x80 | ((c >> 12) & 0x3F));
            o += (char)(0x80 | ((c >> 6) & 0x3F));
            o += (char)(0x80 | (c & 0x3F));
        }
    }
    bool hex4(uint32_t& c) {
        if (end_ - p_ < 4) return false;
        c = 0;
        for (int i = 0; i < 4; i++) {
            const char h = *p_++;
            c <<= 4;
            if (h >= '0' && h <= '9') c |= (uint32_t)(h - '0');
            else if (h >= 'a' && h <= 'f') c |= (uint32_t)(h - 'a' + 10);
            else if (h >= 'A' && h <= 'F') c |= (uint32_t)(h - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool string(std::string& o) {
        if (p_ >= end_ || *p_ != '"') return false;
        p_++;
        while (p_ < end_ && *p_ != '"') {
            const unsigned char ch = (unsigned char)*p_;
            if (ch < 0x20) return false;
            if (ch != '\\') {
                o += (char)ch;
                p_++;
                continue;
            }
            if (++p_ >= end_) return false;
            const char e = *p_++;
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
                uint32_t c;
                if (!hex4(c)) return false;
                if (c >= 0xD800 && c < 0xDC00) {  // surrogate pair
                    uint32_t lo;
                    if (!lit("\\u") || !hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
                    c = 0x10000 + ((c - 0xD800) << 10) + (lo - 0xDC00);
                } else if (c >= 0xDC00 && c < 0xE000) {
                    return false;
                }
                put_utf8(o, c);
                break;
            }
            default: return false;
            }
        }
        if (p_ >= end_) return false;
        p_++;  // closing quote
        return true;
    }
    bool number(std::string& o) {
        const char* s = p_;
        if (p_ < end_ && *p_ == '-') p_++;
        while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' ||
                             *p_ == '+' || *p_ == '-'))
            p_++;
        if (p_ == s) return false;
        o.assign(s, p_);
        return true;
    }
    bool value(JValue& v, int depth) {
        if (depth > 64) return false;
        ws();
        if (p_ >= end_) return false;
        const char c = *p_;
        if (c == '{') {
            p_++;
            v.kind = JValue::Object;
            ws();
            if (p_ < end_ && *p_ == '}') { p_++; return true; }
            for (;;) {
                ws();
                std::string k;
                if (!string(k)) return false;
                ws();
                if (p_ >= end_ || *p_++ != ':') return false;
                JValue m;
                if (!value(m, depth + 1)) return false;
                v.members.emplace_back(std::move(k), std::move(m));
                ws();
                if (p_ >= end_) return false;
                if (*p_ == ',') { p_++; continue; }
                if (*p_ == '}') { p_++; return true; }
                return false;
            }
        }
        if (c == '[') {
            p_++;
            v.kind = JValue::Array;
            ws();
            if (p_ < end_ && *p_ == ']') { p_++; return true; }
            for (;;) {
                JValue it;
                if (!value(it, depth + 1)) return false;
                v.items.push_back(std::move(it));
                ws();
                if (p_ >= end_) return false;
                if (*p_ == ',') { p_++; continue; }
                if (*p_ == ']') { p_++; return true; }
                return false;
            }
        }
        if (c == '"') { v.kind = JValue::String; return string(v.text); }
        if (lit("true") || lit("false")) { v.kind = JValue::Bool; return true; }
        if (lit("null")) { v.kind = JValue::Null; return true; }
        v.kind = JValue::Number;
        return number(v.text);
    }
};

// a non-negative integer literal (no sign, fraction or exponent)
bool to_u64(const JValue* v, uint64_t& out) {
    if (!v || v->kind != JValue::Number || v->text.empty()) return false;
    for (char ch : v->text)
        if (ch < '0' || ch > '9') return false;
    errno = 0;
    char* e = nullptr;
    const unsigned long long r = std::strtoull(v->text.c_str(), &e, 10);
    if (errno || *e) return false;
    out = r;
    return true;
}

// a decimal integer in a string entry ("4"), as MLX-style metadata stores it
bool str_int(const JValue* v, int& out) {
    if (!v || v->kind != JValue::String || v->text.empty() || v->text.size() > 9) return false;
    int r = 0;
    for (char ch : v->text) {
        if (ch < '0' || ch > '9') return false;
        r = r * 10 + (ch - '0');
    }
    out = r;
    return true;
}

struct Tensor {
    std::string dtype;
    std::vector<uint64_t> shape;
    uint64_t begin = 0, end = 0;  // relative to the data start
};

// a tensor entry, checked against the data section's size
LuxBackendError get_tensor(const JValue& root, const std::string& name, uint64_t data_bytes, Tensor& t,
                           bool& found) {
    found = false;
    const JValue* e = root.get(name);
    if (!e) return LUX_BACKEND_OK;
    found = true;
    if (e->kind != JValue::Object) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    const JValue* dt = e->get("dtype");
    const JValue* sh = e->get("shape");
    const JValue* off = e->get("data_offsets");
    if (!dt || dt->kind != JValue::String || !sh || sh->kind != JValue::Array || !off ||
        off->kind != JValue::Array || off->items.size() != 2)
        return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    t.dtype = dt->text;
    for (const auto& d : sh->items) {
        uint64_t x;
        if (!to_u64(&d, x)) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
        t.shape.push_back(x);
    }
    if (!to_u64(&off->items[0], t.begin) || !to_u64(&off->items[1], t.end) || t.begin > t.end ||
        t.end > data_bytes)
        return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    return LUX_BACKEND_OK;
}

// size of one element; 0 for dtypes the format does not use
uint64_t dtype_bytes(const std::string& dt) {
    if (dt == "F32" || dt == "U32") return 4;
    if (dt == "F16" || dt == "BF16") return 2;
    return 0;
}

bool float_dtype(const std::string& dt, LuxBackendDtype& out) {
    if (dt == "F32") out = LUX_DTYPE_FLOAT32;
    else if (dt == "F16") out = LUX_DTYPE_FLOAT16;
    else if (dt == "BF16") out = LUX_DTYPE_BFLOAT16;
    else return false;
    return true;
}

// bytes the shape holds, or false on overflow
bool shape_bytes(const Tensor& t, uint64_t esize, uint64_t& out) {
    unsigned __int128 n = esize;
    for (uint64_t d : t.shape) {
        n *= d;
        if (n > (unsigned __int128)UINT64_MAX) return false;
    }
    out = (uint64_t)n;
    return true;
}

}  // namespace

LuxBackendError linear_describe(const char* path, const char* prefix, int group_size, int bits,
                                lux_quant_linear_info* out) {
    if (!path || !prefix || !out || group_size < 0 || bits < 0) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    std::memset(out, 0, sizeof(*out));
    MappedFile f;
    if (!f.open(path) || f.size < 8) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    uint64_t H = 0;
    for (int i = 7; i >= 0; i--) H = (H << 8) | f.data[i];
    if (H == 0 || H > (100ull << 20) || H > f.size - 8) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    const char* js = reinterpret_cast<const char*>(f.data + 8);
    JValue root;
    if (!JParser(js, js + H).parse_document(root) || root.kind != JValue::Object)
        return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    const uint64_t data0 = 8 + H, data_bytes = f.size - data0;

    const std::string P(prefix);
    Tensor w, s, b, bias;
    bool fw, fs, fb, fbias;
    LuxBackendError e;
    if ((e = get_tensor(root, P + ".weight", data_bytes, w, fw)) != LUX_BACKEND_OK) return e;
    if ((e = get_tensor(root, P + ".scales", data_bytes, s, fs)) != LUX_BACKEND_OK) return e;
    if ((e = get_tensor(root, P + ".biases", data_bytes, b, fb)) != LUX_BACKEND_OK) return e;
    if ((e = get_tensor(root, P + ".bias", data_bytes, bias, fbias)) != LUX_BACKEND_OK) return e;
    if (!fw || !fs || !fb) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;

    // quantization parameters: the arguments, else __metadata__'s
    // "P.group_size" / "P.bits", else its "group_size" / "bits"
    const JValue* meta = root.get("__metadata__");
    if (meta && meta->kind != JValue::Object) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    if (group_size == 0 && !(meta && str_int(meta->get(P + ".group_size"), group_size)) &&
        !(meta && str_int(meta->get("group_size"), group_size)))
        return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    if (bits == 0 && !(meta && str_int(meta->get(P + ".bits"), bits)) && !(meta && str_int(meta->get("bits"), bits)))
        return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    if (bits != 2 && bits != 3 && bits != 4 && bits != 5 && bits != 6 && bits != 8)
        return LUX_BACKEND_ERROR_NOT_SUPPORTED;
    if (group_size != 32 && group_size != 64 && group_size != 128) return LUX_BACKEND_ERROR_NOT_SUPPORTED;

    // dtypes
    LuxBackendDtype sdt, bdt, biasdt = LUX_DTYPE_FLOAT32;
    if (w.dtype != "U32") return LUX_BACKEND_ERROR_NOT_SUPPORTED;
    if (!float_dtype(s.dtype, sdt) || !float_dtype(b.dtype, bdt)) return LUX_BACKEND_ERROR_NOT_SUPPORTED;
    if (sdt != bdt) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    if (fbias && !float_dtype(bias.dtype, biasdt)) return LUX_BACKEND_ERROR_NOT_SUPPORTED;

    // shapes: weight [N, K*bits/32], scales = biases [N, K/g], bias [N]
    if (w.shape.size() != 2 || s.shape.size() != 2 || b.shape != s.shape) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    const uint64_t N = w.shape[0], G = s.shape[1];
    if (s.shape[0] != N || N == 0 || G == 0 || N > INT32_MAX) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    const uint64_t K = G * (uint64_t)group_size;
    if (K > INT32_MAX || (K * (uint64_t)bits) % 32 != 0 || w.shape[1] != K * (uint64_t)bits / 32)
        return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    if (fbias && (bias.shape.size() != 1 || bias.shape[0] != N)) return LUX_BACKEND_ERROR_INVALID_ARGUMENT;

    // each entry's byte range holds exactly its shape
    const Tensor* all[4] = {&w, &s, &b, fbias ? &bias : nullptr};
    for (const Tensor* t : all) {
        if (!t) continue;
        uint64_t nb;
        if (!shape_bytes(*t, dtype_bytes(t->dtype), nb) || nb != t->end - t->begin)
            return LUX_BACKEND_ERROR_INVALID_ARGUMENT;
    }

    out->N = (int32_t)N;
    out->K = (int32_t)K;
    out->group_size = group_size;
    out->bits = bits;
    out->sb_dtype = sdt;
    out->bias_dtype = biasdt;
    out->has_bias = fbias ? 1 : 0;
    out->weight_offset = data0 + w.begin;
    out->weight_bytes = w.end - w.begin;
    out->scales_offset = data0 + s.begin;
    out->scales_bytes = s.end - s.begin;
    out->biases_offset = data0 + b.begin;
    out->biases_bytes = b.end - b.begin;
    if (fbias) {
        out->bias_offset = data0 + bias.begin;
        out->bias_bytes = bias.end - bias.begin;
    }
    return LUX_BACKEND_OK;
}

}  // namespace lxq
