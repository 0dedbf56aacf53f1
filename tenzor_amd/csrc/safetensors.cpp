// safetensors parse / load / write (io/safetensors.zig:172-409) and the
// quantize_arctic_xs tool (quantize_arctic_xs.zig:42-145) on the host.
#include "safetensors.h"

#include <cmath>
#include <cstdio>
#include <cstring>

#include "common.h"

namespace {

const char *kNames[] = {"F16", "BF16", "F32", "F64", "I8", "I16", "I32", "I64", "U8", "U16", "U32", "U64", "BOOL"};
const int kSizes[] = {2, 2, 4, 8, 1, 2, 4, 8, 1, 2, 4, 8, 1};

// Minimal JSON reader for the safetensors header: objects, arrays, strings,
// integers (and other scalars, skipped).
struct Json {
    const char *p, *e;
    void ws() {
        while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
    }
    bool lit(char c) {
        ws();
        if (p < e && *p == c) { p++; return true; }
        return false;
    }
    bool str(std::string &out) {
        ws();
        if (p >= e || *p != '"') return false;
        p++;
        out.clear();
        while (p < e && *p != '"') {
            if (*p == '\\') {
                if (++p >= e) return false;
                switch (*p) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'u': {
                    if (e - p < 5) return false;
                    unsigned v = 0;
                    for (int i = 1; i <= 4; i++) {
                        char c = p[i];
                        v <<= 4;
                        if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
                        else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
                        else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
                        else return false;
                    }
                    if (v < 0x80) out += (char)v;
                    else if (v < 0x800) { out += (char)(0xc0 | (v >> 6)); out += (char)(0x80 | (v & 0x3f)); }
                    else { out += (char)(0xe0 | (v >> 12)); out += (char)(0x80 | ((v >> 6) & 0x3f)); out += (char)(0x80 | (v & 0x3f)); }
                    p += 4;
                    break;
                }
                default: return false;
                }
                p++;
            } else {
                out += *p++;
            }
        }
        if (p >= e) return false;
        p++;
        return true;
    }
    bool integer(int64_t &v) {
        ws();
        const char *s = p;
        bool neg = false;
        if (p < e && *p == '-') { neg = true; p++; }
        if (p >= e || *p < '0' || *p > '9') { p = s; return false; }
        int64_t x = 0;
        while (p < e && *p >= '0' && *p <= '9') x = x * 10 + (*p++ - '0');
        if (p < e && (*p == '.' || *p == 'e' || *p == 'E')) { p = s; return false; }
        v = neg ? -x : x;
        return true;
    }
    bool skip() {  // skip any value
        ws();
        if (p >= e) return false;
        if (*p == '"') { std::string s; return str(s); }
        if (*p == '{') {
            p++;
            if (lit('}')) return true;
            do {
                std::string k;
                if (!str(k) || !lit(':') || !skip()) return false;
            } while (lit(','));
            return lit('}');
        }
        if (*p == '[') {
            p++;
            if (lit(']')) return true;
            do {
                if (!skip()) return false;
            } while (lit(','));
            return lit(']');
        }
        while (p < e && *p != ',' && *p != '}' && *p != ']') p++;
        return true;
    }
    bool int_array(std::vector<int64_t> &out) {
        out.clear();
        if (!lit('[')) return false;
        if (lit(']')) return true;
        do {
            int64_t v;
            if (!integer(v)) return false;
            out.push_back(v);
        } while (lit(','));
        return lit(']');
    }
};

}  // namespace

int st_dtype_size(int32_t dtype) { return (dtype >= 0 && dtype <= TZH_BOOL) ? kSizes[dtype] : 0; }
const char *st_dtype_name(int32_t dtype) { return (dtype >= 0 && dtype <= TZH_BOOL) ? kNames[dtype] : "?"; }

const StTensor *StFile::get(const std::string &name) const {
    for (const auto &t : tensors)
        if (t.name == name) return &t;
    return nullptr;
}

int st_parse(std::vector<uint8_t> &&bytes, StFile &out) {
    out = StFile();
    out.bytes = std::move(bytes);
    if (out.bytes.size() < 8) return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: file shorter than 8 bytes");
    uint64_t hs = 0;
    for (int i = 7; i >= 0; i--) hs = (hs << 8) | out.bytes[i];
    if (hs > out.bytes.size() - 8) return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: header size %llu too large",
                                                   (unsigned long long)hs);
    out.header_size = hs;
    Json j{(const char *)out.bytes.data() + 8, (const char *)out.bytes.data() + 8 + hs};
    if (!j.lit('{')) return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: header is not a JSON object");
    const uint64_t data_len = out.bytes.size() - 8 - hs;
    if (!j.lit('}')) {
        do {
            std::string name;
            if (!j.str(name) || !j.lit(':')) return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: bad header key");
            if (name == "__metadata__") {
                if (!j.skip()) return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: bad __metadata__");
                continue;
            }
            if (!j.lit('{')) return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: tensor %s is not an object", name.c_str());
            StTensor t;
            t.name = name;
            bool have_dtype = false, have_shape = false, have_off = false;
            int32_t dtype = -1;
            std::vector<int64_t> offs;
            if (!j.lit('}')) {
                do {
                    std::string key;
                    if (!j.str(key) || !j.lit(':')) return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: bad field");
                    if (key == "dtype") {
                        std::string ds;
                        if (!j.str(ds)) return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: dtype not a string");
                        for (int d = 0; d <= TZH_BOOL; d++)
                            if (ds == kNames[d]) dtype = d;
                        if (dtype < 0) return tzh_fail(TZH_ERR_UNSUPPORTED_DTYPE, "safetensors: unsupported dtype %s", ds.c_str());
                        have_dtype = true;
                    } else if (key == "shape") {
                        if (!j.int_array(t.shape)) return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: bad shape");
                        have_shape = true;
                    } else if (key == "data_offsets") {
                        if (!j.int_array(offs) || offs.size() != 2) return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: bad data_offsets");
                        have_off = true;
                    } else if (!j.skip()) {
                        return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: bad field value");
                    }
                } while (j.lit(','));
                if (!j.lit('}')) return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: unterminated tensor entry");
            }
            if (!have_dtype || !have_shape || !have_off)
                return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: tensor %s lacks dtype/shape/data_offsets", name.c_str());
            t.dtype = dtype;
            for (int64_t d : t.shape)
                if (d < 0) return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: negative dim in %s", name.c_str());
            if (offs[0] < 0 || offs[1] < offs[0] || (uint64_t)offs[1] > data_len)
                return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: offsets of %s out of range", name.c_str());
            t.start = (uint64_t)offs[0];
            t.end = (uint64_t)offs[1];
            if ((int64_t)(t.end - t.start) != t.numel() * st_dtype_size(dtype))
                return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: size of %s does not match its shape", name.c_str());
            out.tensors.push_back(std::move(t));
        } while (j.lit(','));
        if (!j.lit('}')) return tzh_fail(TZH_ERR_INVALID_FORMAT, "safetensors: unterminated header");
    }
    return TZH_OK;
}

int st_load(const char *path, StFile &out) {
    if (!path) return tzh_fail(TZH_ERR_INVALID_ARGS, "null path");
    FILE *f = std::fopen(path, "rb");
    if (!f) return tzh_fail(TZH_ERR_IO, "cannot open %s", path);
    std::fseek(f, 0, SEEK_END);
    const long sz = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    if (sz < 0) { std::fclose(f); return tzh_fail(TZH_ERR_IO, "cannot stat %s", path); }
    std::vector<uint8_t> bytes((size_t)sz);
    const size_t got = sz ? std::fread(bytes.data(), 1, (size_t)sz, f) : 0;
    std::fclose(f);
    if (got != (size_t)sz) return tzh_fail(TZH_ERR_IO, "short read of %s", path);
    return st_parse(std::move(bytes), out);
}

static void json_string(std::string &h, const std::string &s) {
    h += '"';
    for (unsigned char ch : s) {  // safetensors.zig:316-337
        switch (ch) {
        case '"': h += "\\\""; break;
        case '\\': h += "\\\\"; break;
        case '\n': h += "\\n"; break;
        case '\r': h += "\\r"; break;
        case '\t': h += "\\t"; break;
        default:
            if (ch < 0x20) {
                char b[8];
                std::snprintf(b, sizeof b, "\\u%04X", ch);
                h += b;
            } else {
                h += (char)ch;
            }
        }
    }
    h += '"';
}

int st_write(const char *path, const std::vector<StWrite> &tensors) {
    std::string h = "{";
    uint64_t off = 0;
    for (size_t i = 0; i < tensors.size(); i++) {
        const StWrite &t = tensors[i];
        int64_t n = 1;
        for (int64_t d : t.shape) n *= d;
        if ((size_t)(n * st_dtype_size(t.dtype)) != t.bytes)
            return tzh_fail(TZH_ERR_INVALID_ARGS, "safetensors write: DataSizeMismatch for %s", t.name.c_str());
        if (i) h += ',';
        json_string(h, t.name);
        h += ":{\"dtype\":";
        json_string(h, st_dtype_name(t.dtype));
        h += ",\"shape\":[";
        for (size_t k = 0; k < t.shape.size(); k++) {
            if (k) h += ',';
            h += std::to_string(t.shape[k]);
        }
        h += "],\"data_offsets\":[";
        h += std::to_string(off);
        h += ',';
        off += t.bytes;
        h += std::to_string(off);
        h += "]}";
    }
    h += '}';
    while (h.size() % 8) h += ' ';  // safetensors.zig:392-394
    FILE *f = std::fopen(path, "wb");
    if (!f) return tzh_fail(TZH_ERR_IO, "cannot create %s", path);
    uint8_t hs[8];
    uint64_t v = h.size();
    for (int i = 0; i < 8; i++) { hs[i] = (uint8_t)(v & 0xff); v >>= 8; }
    bool ok = std::fwrite(hs, 1, 8, f) == 8 && std::fwrite(h.data(), 1, h.size(), f) == h.size();
    for (const StWrite &t : tensors)
        if (ok && t.bytes) ok = std::fwrite(t.data, 1, t.bytes, f) == t.bytes;
    ok = (std::fclose(f) == 0) && ok;
    return ok ? TZH_OK : tzh_fail(TZH_ERR_IO, "write to %s failed", path);
}

// ---------------------------------------------------------------------------
// quantizer (host): quantize_arctic_xs.zig:94-115
// ---------------------------------------------------------------------------
extern "C" int tzh_quantize_rows_host(const float *w, int64_t rows, int64_t cols, int8_t *q, uint16_t *scale) {
    tzh_clear_error();
    if (rows < 0 || cols < 0) return tzh_fail(TZH_ERR_INVALID_ARGS, "negative shape");
    if ((rows * cols > 0 && (!w || !q)) || (rows > 0 && !scale)) return tzh_fail(TZH_ERR_INVALID_ARGS, "null pointer");
    for (int64_t r = 0; r < rows; r++) {
        const float *row = w + r * cols;
        float max_abs = 0.0f;
        for (int64_t c = 0; c < cols; c++) {
            const float a = std::fabs(row[c]);
            if (a > max_abs) max_abs = a;
        }
        const float s32 = max_abs == 0.0f ? 1.0f : max_abs / 127.0f;
        const uint16_t s16 = tzh_host_f32_to_f16(s32);
        scale[r] = s16;
        const float inv = 1.0f / tzh_host_f16_to_f32(s16);
        for (int64_t c = 0; c < cols; c++) {
            const float qf = std::round(row[c] * inv);  // @round: half away from zero
            // clamp before converting: a zero f16 scale gives +-inf / NaN here
            // (undefined in the reference); saturate to +-127 and map NaN to 0
            const int32_t qi = std::isnan(qf) ? 0 : qf >= 127.0f ? 127 : qf <= -127.0f ? -127 : (int32_t)qf;
            q[r * cols + c] = (int8_t)qi;
        }
    }
    return TZH_OK;
}

// quantize_arctic_xs.zig:22-34
static bool should_quantize(const StTensor &t) {
    if (t.dtype != TZH_F32) return false;
    if (t.shape.size() != 2) return false;
    const std::string &n = t.name;
    if (n.size() < 7 || n.compare(n.size() - 7, 7, ".weight") != 0) return false;
    if (n.find("LayerNorm") != std::string::npos) return false;
    if (t.shape[0] == 0 || t.shape[1] == 0) return false;
    return t.shape[0] * t.shape[1] >= 4096;
}

extern "C" int tzh_quantize_safetensors(const char *in_path, const char *out_path, int32_t *n_quantized) {
    tzh_clear_error();
    if (!in_path || !out_path) return tzh_fail(TZH_ERR_INVALID_ARGS, "null path");
    StFile st;
    TZH_TRY(st_load(in_path, st));
    std::vector<std::vector<int8_t>> qs;
    std::vector<std::vector<uint16_t>> ss;
    std::vector<std::vector<float>> tmp;
    qs.reserve(st.tensors.size());
    ss.reserve(st.tensors.size());
    tmp.reserve(st.tensors.size());
    std::vector<StWrite> out;
    int32_t count = 0;
    for (const StTensor &t : st.tensors) {
        const uint8_t *raw = st.data(t);
        if (!should_quantize(t)) {
            out.push_back({t.name, t.dtype, t.shape, raw, (size_t)(t.end - t.start)});
            continue;
        }
        const int64_t rows = t.shape[0], cols = t.shape[1];
        tmp.emplace_back((size_t)(rows * cols));
        std::memcpy(tmp.back().data(), raw, (size_t)(rows * cols) * 4);  // little-endian f32
        qs.emplace_back((size_t)(rows * cols));
        ss.emplace_back((size_t)rows);
        TZH_TRY(tzh_quantize_rows_host(tmp.back().data(), rows, cols, qs.back().data(), ss.back().data()));
        out.push_back({t.name, TZH_I8, t.shape, qs.back().data(), (size_t)(rows * cols)});
        out.push_back({t.name + ".scale", TZH_F16, {rows}, ss.back().data(), (size_t)rows * 2});
        count++;
    }
    TZH_TRY(st_write(out_path, out));
    if (n_quantized) *n_quantized = count;
    return TZH_OK;
}
