// focr_focrq.cpp — the weight container: `.focrq` (and raw safetensors)
// reader with the reference's validation, the canonical `.focrq` writer, and
// the upload-once path from a container into HBM-resident engine handles.
//
// Reader: src/native_engine/weights.rs:443-540 (from_bytes /
// from_focrq_bytes), :546-620 (safetensors), :634-670 (census), :744-923
// (tensor / mat / vec / qint8 / qint4 accessors), :949-990
// (validate_directory). Writer: src/quant/focrq.rs:279-714. Format:
// docs/focrq-format.md. Error texts are the reference's FormatMismatch
// messages, so a binding can re-raise them unchanged.
//
// A container opened from a path is memory-mapped read-only; payload bytes
// go to the device straight from the mapping. Uploads copy each stored tensor
// to HBM raw and convert it there (widening, per-channel int8 quantization,
// int4 re-tiling), so the host never holds a widened copy of a weight.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "focr_internal.hpp"

using namespace focr;

namespace {

std::string fmt(const char* f, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    return buf;
}

int32_t format_err(const std::string& msg) { return fail(FOCR_HIP_E_FORMAT, msg); }

// Rust's `{:?}` of a str: quoted, with \" \\ \n \r \t \0 and other control
// characters escaped.
std::string dbg(const std::string& s) {
    std::string o = "\"";
    for (unsigned char c : s) {
        switch (c) {
            case '"': o += "\\\""; break;
            case '\\': o += "\\\\"; break;
            case '\n': o += "\\n"; break;
            case '\r': o += "\\r"; break;
            case '\t': o += "\\t"; break;
            case '\0': o += "\\0"; break;
            default:
                if (c < 0x20 || c == 0x7f) o += fmt("\\u{%x}", c);
                else o += static_cast<char>(c);
        }
    }
    return o + "\"";
}

// Rust's `{:?}` of a Vec<usize>: "[2, 3]".
std::string dbg_shape(const std::vector<uint64_t>& v) {
    std::string o = "[";
    for (size_t i = 0; i < v.size(); ++i) o += (i ? ", " : "") + std::to_string(v[i]);
    return o + "]";
}

// ---- JSON (RFC 8259, strict: no trailing commas, comments or NaN) ---------

struct JVal {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    bool is_uint = false;  // a non-negative integer literal that fits in u64
    uint64_t u = 0;
    std::string s;  // string value, or the number's literal text
    std::vector<JVal> a;
    std::vector<std::pair<std::string, JVal>> o;

    const char* kind_name() const {
        switch (kind) {
            case Null: return "null";
            case Bool: return "boolean";
            case Num: return "number";
            case Str: return "string";
            case Arr: return "sequence";
            default: return "map";
        }
    }
};

class Json {
   public:
    Json(const uint8_t* p, size_t n) : b_(p), p_(p), e_(p + n) {}

    bool parse(JVal& out, std::string& err) {
        ws();
        if (!value(out, 0)) {
            err = err_;
            return false;
        }
        ws();
        if (p_ != e_) {
            err = where("trailing characters");
            return false;
        }
        return true;
    }

   private:
    const uint8_t *b_, *p_, *e_;
    std::string err_;

    std::string where(const char* what) const {
        size_t line = 1, col = 0;
        for (const uint8_t* q = b_; q < p_; ++q) {
            if (*q == '\n') {
                ++line;
                col = 0;
            } else {
                ++col;
            }
        }
        return fmt("%s at line %zu column %zu", what, line, col + (p_ < e_ ? 1 : 0));
    }
    bool bad(const char* what) {
        if (err_.empty()) err_ = where(what);
        return false;
    }
    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* word) {
        size_t n = strlen(word);
        if (static_cast<size_t>(e_ - p_) < n || memcmp(p_, word, n) != 0) return bad("expected value");
        p_ += n;
        return true;
    }

    bool value(JVal& v, int depth) {
        if (depth > 128) return bad("recursion limit exceeded");
        if (p_ >= e_) return bad("EOF while parsing a value");
        switch (*p_) {
            case 'n': v.kind = JVal::Null; return lit("null");
            case 't': v.kind = JVal::Bool; v.b = true; return lit("true");
            case 'f': v.kind = JVal::Bool; v.b = false; return lit("false");
            case '"': v.kind = JVal::Str; return str(v.s);
            case '[': {
                v.kind = JVal::Arr;
                ++p_;
                ws();
                if (p_ < e_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                for (;;) {
                    v.a.emplace_back();
                    ws();
                    if (!value(v.a.back(), depth + 1)) return false;
                    ws();
                    if (p_ >= e_) return bad("EOF while parsing a list");
                    if (*p_ == ',') {
                        ++p_;
                        continue;
                    }
                    if (*p_ == ']') {
                        ++p_;
                        return true;
                    }
                    return bad("expected `,` or `]`");
                }
            }
            case '{': {
                v.kind = JVal::Obj;
                ++p_;
                ws();
                if (p_ < e_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                for (;;) {
                    ws();
                    if (p_ >= e_) return bad("EOF while parsing an object");
                    if (*p_ != '"') return bad("key must be a string");
                    std::string key;
                    if (!str(key)) return false;
                    ws();
                    if (p_ >= e_ || *p_ != ':') return bad("expected `:`");
                    ++p_;
                    ws();
                    v.o.emplace_back(std::move(key), JVal());
                    if (!value(v.o.back().second, depth + 1)) return false;
                    ws();
                    if (p_ >= e_) return bad("EOF while parsing an object");
                    if (*p_ == ',') {
                        ++p_;
                        continue;
                    }
                    if (*p_ == '}') {
                        ++p_;
                        return true;
                    }
                    return bad("expected `,` or `}`");
                }
            }
            default:
                if (*p_ == '-' || (*p_ >= '0' && *p_ <= '9')) return num(v);
                return bad("expected value");
        }
    }

    bool num(JVal& v) {
        v.kind = JVal::Num;
        const uint8_t* s = p_;
        bool neg = false, integral = true;
        if (*p_ == '-') {
            neg = true;
            ++p_;
        }
        if (p_ >= e_ || *p_ < '0' || *p_ > '9') return bad("invalid number");
        if (*p_ == '0') {
            ++p_;
        } else {
            while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < e_ && *p_ == '.') {
            integral = false;
            ++p_;
            if (p_ >= e_ || *p_ < '0' || *p_ > '9') return bad("invalid number");
            while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < e_ && (*p_ == 'e' || *p_ == 'E')) {
            integral = false;
            ++p_;
            if (p_ < e_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= e_ || *p_ < '0' || *p_ > '9') return bad("invalid number");
            while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        v.s.assign(reinterpret_cast<const char*>(s), p_ - s);
        // An integer literal decodes into usize when it is >= 0; "-0" counts
        // (serde_json reads it as the i64 0).
        if (integral && (!neg || (p_ - s == 2 && s[1] == '0'))) {
            uint64_t acc = 0;
            bool fits = true;
            for (const uint8_t* q = s + (neg ? 1 : 0); q < p_; ++q) {
                const uint64_t d = *q - '0';
                if (acc > (std::numeric_limits<uint64_t>::max() - d) / 10) {
                    fits = false;
                    break;
                }
                acc = acc * 10 + d;
            }
            v.is_uint = fits;
            v.u = acc;
        }
        return true;
    }

    static void put_utf8(std::string& o, uint32_t cp) {
        if (cp < 0x80) {
            o += static_cast<char>(cp);
        } else if (cp < 0x800) {
            o += static_cast<char>(0xC0 | (cp >> 6));
            o += static_cast<char>(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            o += static_cast<char>(0xE0 | (cp >> 12));
            o += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            o += static_cast<char>(0x80 | (cp & 0x3F));
        } else {
            o += static_cast<char>(0xF0 | (cp >> 18));
            o += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
            o += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            o += static_cast<char>(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t& cp) {
        if (e_ - p_ < 4) return bad("EOF while parsing a string");
        cp = 0;
        for (int i = 0; i < 4; ++i, ++p_) {
            const uint8_t c = *p_;
            const int d = (c >= '0' && c <= '9') ? c - '0' : (c >= 'a' && c <= 'f') ? c - 'a' + 10
                          : (c >= 'A' && c <= 'F') ? c - 'A' + 10 : -1;
            if (d < 0) return bad("invalid escape");
            cp = cp * 16 + d;
        }
        return true;
    }
    // One well-formed UTF-8 sequence starting at p_ (appended verbatim).
    bool utf8(std::string& o) {
        const uint8_t c = *p_;
        int n = 0;
        uint32_t cp = 0, min = 0;
        if (c >= 0xC2 && c <= 0xDF) { n = 1; cp = c & 0x1F; min = 0x80; }
        else if (c >= 0xE0 && c <= 0xEF) { n = 2; cp = c & 0x0F; min = 0x800; }
        else if (c >= 0xF0 && c <= 0xF4) { n = 3; cp = c & 0x07; min = 0x10000; }
        else return bad("invalid unicode code point");
        if (e_ - p_ <= n) return bad("EOF while parsing a string");
        for (int i = 1; i <= n; ++i) {
            if ((p_[i] & 0xC0) != 0x80) return bad("invalid unicode code point");
            cp = (cp << 6) | (p_[i] & 0x3F);
        }
        if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return bad("invalid unicode code point");
        o.append(reinterpret_cast<const char*>(p_), n + 1);
        p_ += n + 1;
        return true;
    }
    bool str(std::string& o) {
        ++p_;  // opening quote
        for (;;) {
            if (p_ >= e_) return bad("EOF while parsing a string");
            const uint8_t c = *p_;
            if (c == '"') {
                ++p_;
                return true;
            }
            if (c < 0x20) return bad("control character (\\u0000-\\u001F) found while parsing a string");
            if (c >= 0x80) {
                if (!utf8(o)) return false;
                continue;
            }
            if (c != '\\') {
                o += static_cast<char>(c);
                ++p_;
                continue;
            }
            if (++p_ >= e_) return bad("EOF while parsing a string");
            const uint8_t x = *p_++;
            switch (x) {
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
                    if (cp >= 0xD800 && cp <= 0xDBFF) {
                        uint32_t lo;
                        if (e_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return bad("unexpected end of hex escape");
                        p_ += 2;
                        if (!hex4(lo)) return false;
                        if (lo < 0xDC00 || lo > 0xDFFF) return bad("lone leading surrogate in hex escape");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
                        return bad("lone leading surrogate in hex escape");
                    }
                    put_utf8(o, cp);
                    break;
                }
                default: return bad("invalid escape");
            }
        }
    }
};

// ---- typed field extraction (serde's rules for the reference's structs) ----

bool get_u64(const JVal& v, const char* field, uint64_t& out, std::string& err) {
    if (v.kind != JVal::Num || !v.is_uint) {
        err = fmt("invalid type: %s %s, expected usize for field `%s`", v.kind_name(),
                  v.kind == JVal::Num ? v.s.c_str() : "", field);
        return false;
    }
    out = v.u;
    return true;
}

bool get_u8(const JVal& v, const char* field, uint8_t& out, std::string& err) {
    uint64_t u;
    if (!get_u64(v, field, u, err)) return false;
    if (u > 255) {
        err = fmt("invalid value: integer `%llu`, expected u8 for field `%s`", (unsigned long long)u, field);
        return false;
    }
    out = static_cast<uint8_t>(u);
    return true;
}

bool get_str(const JVal& v, const char* field, std::string& out, std::string& err) {
    if (v.kind != JVal::Str) {
        err = fmt("invalid type: %s, expected a string for field `%s`", v.kind_name(), field);
        return false;
    }
    out = v.s;
    return true;
}

bool get_shape(const JVal& v, const char* field, std::vector<uint64_t>& out, std::string& err) {
    if (v.kind != JVal::Arr) {
        err = fmt("invalid type: %s, expected a sequence for field `%s`", v.kind_name(), field);
        return false;
    }
    out.clear();
    for (const JVal& d : v.a) {
        uint64_t u;
        if (!get_u64(d, field, u, err)) return false;
        out.push_back(u);
    }
    return true;
}

const char* kDTypeNames[] = {"F32", "F16", "BF16", "QInt8PerChan", "QInt4PerGroup"};

bool parse_dtype(const JVal& v, int32_t& dt, std::string& err) {
    if (v.kind != JVal::Str) {
        err = fmt("invalid type: %s, expected a DType variant", v.kind_name());
        return false;
    }
    for (int i = 0; i < 5; ++i)
        if (v.s == kDTypeNames[i]) {
            dt = i;
            return true;
        }
    err = fmt("unknown variant `%s`, expected one of `F32`, `F16`, `BF16`, `QInt8PerChan`, `QInt4PerGroup`",
              v.s.c_str());
    return false;
}

// ---- the model registry (src/native_engine/model_arch.rs:186-196, :313-401,
// :417-443): id and the license notice each architecture requires ----------

const char* const kDefaultNotice = "Baidu Unlimited-OCR - Copyright (c) 2026 Baidu, MIT License";
struct Arch {
    const char* id;
    const char* notice;
};
const Arch kRegistry[] = {
    {"unlimited-ocr", kDefaultNotice},
    {"got-ocr2", "GOT-OCR2.0 (StepFun) - Apache-2.0"},
    {"smolvlm2", "SmolVLM2 (HuggingFaceTB) - Apache-2.0"},
    {"onechart", "OneChart - Apache-2.0"},
    {"tromr", "Polyphonic-TrOMR (NetEase) - Apache-2.0"},
    {"trocr", "TrOCR (Microsoft) - MIT"},
    {"pix2tex", "pix2tex / LaTeX-OCR - MIT"},
};
const Arch* arch_by_id(const std::string& id) {
    for (const Arch& a : kRegistry)
        if (id == a.id) return &a;
    return nullptr;
}

std::string hex(const uint8_t* p, size_t n) {
    static const char* d = "0123456789abcdef";
    std::string s;
    for (size_t i = 0; i < n; ++i) {
        s += d[p[i] >> 4];
        s += d[p[i] & 15];
    }
    return s;
}

bool checked_mul(uint64_t a, uint64_t b, uint64_t& out) { return !__builtin_mul_overflow(a, b, &out); }

}  // namespace

// ---- the container --------------------------------------------------------

struct FocrqRecord {
    int32_t dtype = 0;
    std::vector<uint64_t> shape;
    uint64_t byte_offset = 0, byte_len = 0, scales_offset = 0, scales_len = 0, group_size = 0;
    uint8_t tier = 0;
};

struct focr_hip_focrq {
    std::vector<uint8_t> owned;  // from_bytes copy
    void* map = nullptr;         // mmap of an opened file
    size_t map_len = 0;
    const uint8_t* bytes = nullptr;
    size_t len = 0;
    size_t payload_base = 0;
    std::map<std::string, FocrqRecord> dir;
    std::vector<const std::string*> names;  // sorted, for index access
    uint8_t arch_target = 0;
    std::string sha, license, model_id = "unlimited-ocr";
    bool is_focrq = false;

    ~focr_hip_focrq() {
        if (map) munmap(map, map_len);
    }
};

namespace {

// TensorRecord::checked_numel / expected_byte_len (weights.rs:232-277).
int32_t expected_byte_len(const std::string& name, const FocrqRecord& r, uint64_t& out) {
    uint64_t numel = 1;
    for (uint64_t d : r.shape)
        if (!checked_mul(numel, d, numel))
            return format_err(fmt("tensor %s: shape %s element count overflows usize", dbg(name).c_str(),
                                  dbg_shape(r.shape).c_str()));
    if (r.dtype == FOCR_HIP_DT_QINT4_PER_GROUP) {
        if (numel % 2)
            return format_err(fmt("tensor %s: QInt4 shape %s has odd element count %llu", dbg(name).c_str(),
                                  dbg_shape(r.shape).c_str(), (unsigned long long)numel));
        out = numel / 2;
        return FOCR_HIP_OK;
    }
    const uint64_t eb = r.dtype == FOCR_HIP_DT_F32 ? 4 : (r.dtype == FOCR_HIP_DT_QINT8_PER_CHAN ? 1 : 2);
    if (!checked_mul(numel, eb, out))
        return format_err(fmt("tensor %s: byte length for %s, shape %s overflows usize", dbg(name).c_str(),
                              kDTypeNames[r.dtype], dbg_shape(r.shape).c_str()));
    return FOCR_HIP_OK;
}

// weights.rs:949-990 validate_directory, in the reference's check order.
int32_t validate_directory(const std::map<std::string, FocrqRecord>& dir, uint64_t payload_len) {
    for (const auto& kv : dir) {
        const std::string& name = kv.first;
        const FocrqRecord& r = kv.second;
        uint64_t end;
        if (__builtin_add_overflow(r.byte_offset, r.byte_len, &end))
            return format_err(fmt("tensor %s byte range overflows", dbg(name).c_str()));
        if (end > payload_len)
            return format_err(fmt("tensor %s ends at %llu but payload is %llu bytes", dbg(name).c_str(),
                                  (unsigned long long)end, (unsigned long long)payload_len));
        uint64_t expected = 0;
        if (int32_t st = expected_byte_len(name, r, expected)) return st;
        if (r.byte_len != expected)
            return format_err(fmt("tensor %s: byte_len %llu != shape\xC3\x97" "dtype %llu (%s, shape %s)",
                                  dbg(name).c_str(), (unsigned long long)r.byte_len, (unsigned long long)expected,
                                  kDTypeNames[r.dtype], dbg_shape(r.shape).c_str()));
        uint64_t send;
        if (__builtin_add_overflow(r.scales_offset, r.scales_len, &send))
            return format_err(fmt("tensor %s scales range overflows", dbg(name).c_str()));
        if (send > payload_len)
            return format_err(fmt("tensor %s scales end at %llu but payload is %llu bytes", dbg(name).c_str(),
                                  (unsigned long long)send, (unsigned long long)payload_len));
    }
    return FOCR_HIP_OK;
}

// The `tensors` map of a .focrq header (weights.rs:196-230 TensorRecord).
int32_t parse_focrq_directory(const JVal& t, std::map<std::string, FocrqRecord>& dir) {
    auto invalid = [](const std::string& e) { return format_err(".focrq header JSON invalid: " + e); };
    if (t.kind != JVal::Obj)
        return invalid(fmt("invalid type: %s, expected a map for field `tensors`", t.kind_name()));
    for (const auto& kv : t.o) {
        const JVal& v = kv.second;
        if (v.kind != JVal::Obj) return invalid(fmt("invalid type: %s, expected struct TensorRecord", v.kind_name()));
        FocrqRecord r;
        bool have_dtype = false, have_shape = false, have_off = false, have_len = false;
        std::set<std::string> seen;
        std::string err;
        for (const auto& f : v.o) {
            const std::string& k = f.first;
            if (!seen.insert(k).second &&
                (k == "dtype" || k == "shape" || k == "byte_offset" || k == "byte_len" || k == "scales_offset" ||
                 k == "scales_len" || k == "group_size" || k == "tier"))
                return invalid(fmt("duplicate field `%s`", k.c_str()));
            bool ok = true;
            if (k == "dtype") ok = have_dtype = parse_dtype(f.second, r.dtype, err);
            else if (k == "shape") ok = have_shape = get_shape(f.second, "shape", r.shape, err);
            else if (k == "byte_offset") ok = have_off = get_u64(f.second, "byte_offset", r.byte_offset, err);
            else if (k == "byte_len") ok = have_len = get_u64(f.second, "byte_len", r.byte_len, err);
            else if (k == "scales_offset") ok = get_u64(f.second, "scales_offset", r.scales_offset, err);
            else if (k == "scales_len") ok = get_u64(f.second, "scales_len", r.scales_len, err);
            else if (k == "group_size") ok = get_u64(f.second, "group_size", r.group_size, err);
            else if (k == "tier") ok = get_u8(f.second, "tier", r.tier, err);
            if (!ok) return invalid(err);
        }
        if (!have_dtype) return invalid("missing field `dtype`");
        if (!have_shape) return invalid("missing field `shape`");
        if (!have_off) return invalid("missing field `byte_offset`");
        if (!have_len) return invalid("missing field `byte_len`");
        dir[kv.first] = std::move(r);  // a repeated name keeps its last record
    }
    return FOCR_HIP_OK;
}

// weights.rs:462-540 from_focrq_bytes (magic already matched).
int32_t parse_focrq(focr_hip_focrq* f) {
    const size_t kPreamble = 6 + 4 + 1 + 32 + 8;
    const uint8_t* b = f->bytes;
    if (f->len < kPreamble)
        return format_err(fmt(".focrq truncated: %zu bytes < %zu-byte preamble", f->len, kPreamble));
    uint32_t version;
    memcpy(&version, b + 6, 4);
    if (version > 1)
        return format_err(fmt(".focrq format_version %u is newer than this binary supports (max 1)", version));
    const uint8_t preamble_arch = b[10];
    const std::string preamble_sha = hex(b + 11, 32);
    uint64_t header_len;
    memcpy(&header_len, b + 43, 8);
    uint64_t header_end;
    if (__builtin_add_overflow(static_cast<uint64_t>(kPreamble), header_len, &header_end))
        return format_err(".focrq header_len overflows");
    if (header_end > f->len)
        return format_err(fmt(".focrq header (%llu bytes) overruns file (%zu bytes)", (unsigned long long)header_len,
                              f->len));
    JVal h;
    std::string err;
    if (!Json(b + kPreamble, header_len).parse(h, err)) return format_err(".focrq header JSON invalid: " + err);
    if (h.kind != JVal::Obj)
        return format_err(fmt(".focrq header JSON invalid: invalid type: %s, expected struct FocrqHeader",
                              h.kind_name()));
    // FocrqHeader (weights.rs:283-318): tensors required, the rest default.
    bool have_tensors = false;
    uint8_t arch = 0;
    std::string sha, license, model_id;
    std::set<std::string> seen;
    for (const auto& kv : h.o) {
        const std::string& k = kv.first;
        const bool known =
            k == "tensors" || k == "arch_target" || k == "source_sha256" || k == "license_notice" || k == "model_id";
        if (known && !seen.insert(k).second)
            return format_err(fmt(".focrq header JSON invalid: duplicate field `%s`", k.c_str()));
        bool ok = true;
        if (k == "tensors") {  // fields decode in document order, as serde does
            if (int32_t st = parse_focrq_directory(kv.second, f->dir)) return st;
            have_tensors = true;
        } else if (k == "arch_target") ok = get_u8(kv.second, "arch_target", arch, err);
        else if (k == "source_sha256") ok = get_str(kv.second, "source_sha256", sha, err);
        else if (k == "license_notice") ok = get_str(kv.second, "license_notice", license, err);
        else if (k == "model_id") ok = get_str(kv.second, "model_id", model_id, err);
        if (!ok) return format_err(".focrq header JSON invalid: " + err);
    }
    if (!have_tensors) return format_err(".focrq header JSON invalid: missing field `tensors`");

    // resolve_model_id (weights.rs:71-83): absent -> the default architecture.
    if (model_id.empty()) {
        model_id = kRegistry[0].id;
    } else if (!arch_by_id(model_id)) {
        return format_err(fmt(".focrq declares unknown model_id %s (not in the model registry; this binary cannot "
                              "load it)", dbg(model_id).c_str()));
    }
    // validate_license_notice (weights.rs:97-121).
    if (model_id == kRegistry[0].id) {
        const bool ok = license == kDefaultNotice || (license.find("Copyright (c) 2026 Baidu") != std::string::npos &&
                                                      license.find("MIT License") != std::string::npos);
        if (!ok) return format_err(".focrq license_notice must include Copyright (c) 2026 Baidu and MIT License");
    } else {
        const Arch* a = arch_by_id(model_id);
        if (license != a->notice)
            return format_err(fmt(".focrq license_notice does not match the registered %s notice (expected %s)",
                                  model_id.c_str(), dbg(a->notice).c_str()));
    }
    // validate_source_sha256_hex (weights.rs:123-136).
    if (!sha.empty()) {
        bool ok = sha.size() == 64;
        for (char c : sha) ok = ok && ((c >= '0' && c <= '9') || (c >= 'a' && c <= 'f'));
        if (!ok) return format_err(".focrq source_sha256 must be 64 lowercase hex chars when present");
    }
    f->payload_base = header_end;
    if (int32_t st = validate_directory(f->dir, f->len - header_end)) return st;
    f->arch_target = arch != 0 ? arch : preamble_arch;
    f->sha = sha.empty() ? preamble_sha : sha;
    f->license = license;
    f->model_id = model_id;
    f->is_focrq = true;
    return FOCR_HIP_OK;
}

// weights.rs:546-620 from_safetensors_bytes.
int32_t parse_safetensors(focr_hip_focrq* f) {
    if (f->len < 8)
        return format_err(fmt("safetensors truncated: %zu bytes < 8-byte header length prefix", f->len));
    uint64_t header_len;
    memcpy(&header_len, f->bytes, 8);
    uint64_t header_end;
    if (__builtin_add_overflow(static_cast<uint64_t>(8), header_len, &header_end))
        return format_err("safetensors header_len overflows");
    if (header_end > f->len)
        return format_err(fmt("safetensors header (%llu bytes) overruns file (%zu bytes)",
                              (unsigned long long)header_len, f->len));
    JVal h;
    std::string err;
    if (!Json(f->bytes + 8, header_len).parse(h, err)) return format_err("safetensors header JSON invalid: " + err);
    if (h.kind != JVal::Obj)
        return format_err(fmt("safetensors header JSON invalid: invalid type: %s, expected a map", h.kind_name()));
    for (const auto& kv : h.o) {
        const std::string& name = kv.first;
        if (name == "__metadata__") continue;
        auto invalid = [&](const std::string& e) {
            return format_err(fmt("safetensors entry %s invalid: ", dbg(name).c_str()) + e);
        };
        const JVal& v = kv.second;
        if (v.kind != JVal::Obj) return invalid(fmt("invalid type: %s, expected struct StEntry", v.kind_name()));
        std::string dtype;
        std::vector<uint64_t> shape, offs;
        bool hd = false, hs = false, ho = false;
        for (const auto& fv : v.o) {
            bool ok = true;
            if (fv.first == "dtype") ok = hd = get_str(fv.second, "dtype", dtype, err);
            else if (fv.first == "shape") ok = hs = get_shape(fv.second, "shape", shape, err);
            else if (fv.first == "data_offsets") {
                ok = ho = get_shape(fv.second, "data_offsets", offs, err);
                if (ok && offs.size() != 2) {
                    err = fmt("invalid length %zu, expected an array of length 2", offs.size());
                    ok = false;
                }
            }
            if (!ok) return invalid(err);
        }
        if (!hd) return invalid("missing field `dtype`");
        if (!hs) return invalid("missing field `shape`");
        if (!ho) return invalid("missing field `data_offsets`");
        if (offs[1] < offs[0])
            return format_err(fmt("safetensors entry %s has end %llu < beg %llu", dbg(name).c_str(),
                                  (unsigned long long)offs[1], (unsigned long long)offs[0]));
        FocrqRecord r;
        if (dtype == "F32") r.dtype = FOCR_HIP_DT_F32;
        else if (dtype == "F16") r.dtype = FOCR_HIP_DT_F16;
        else if (dtype == "BF16") r.dtype = FOCR_HIP_DT_BF16;
        else
            return format_err(fmt("unsupported safetensors dtype %s (expected F32/F16/BF16; the upstream "
                                  "Unlimited-OCR shard is BF16)", dbg(dtype).c_str()));
        r.shape = shape;
        r.byte_offset = offs[0];
        r.byte_len = offs[1] - offs[0];
        f->dir[name] = std::move(r);
    }
    f->payload_base = header_end;
    if (int32_t st = validate_directory(f->dir, f->len - header_end)) return st;
    f->is_focrq = false;
    return FOCR_HIP_OK;
}

// weights.rs:443-453 from_bytes: the magic picks the format.
int32_t parse_container(focr_hip_focrq* f) {
    static const uint8_t kMagic[6] = {'F', 'O', 'C', 'R', 'Q', 0};
    const int32_t st = (f->len >= 6 && memcmp(f->bytes, kMagic, 6) == 0) ? parse_focrq(f) : parse_safetensors(f);
    if (st) return st;
    for (const auto& kv : f->dir) f->names.push_back(&kv.first);
    return FOCR_HIP_OK;
}

// weights.rs:744-764 tensor(): the record plus bounds-checked payload ranges.
struct View {
    const FocrqRecord* rec;
    const uint8_t* data;
    const uint8_t* scales;
};

int32_t payload_slice(const focr_hip_focrq* f, const std::string& name, uint64_t off, uint64_t len,
                      const uint8_t** out) {
    uint64_t start, end;
    if (__builtin_add_overflow(static_cast<uint64_t>(f->payload_base), off, &start) ||
        __builtin_add_overflow(start, len, &end))
        return format_err(fmt("tensor %s byte range overflows", dbg(name).c_str()));
    if (end > f->len) {
        uint64_t re;
        const std::string range_end =
            __builtin_add_overflow(off, len, &re) ? std::string("<overflow>") : std::to_string(re);
        return format_err(fmt("tensor %s range [%llu, %s) overruns payload", dbg(name).c_str(),
                              (unsigned long long)off, range_end.c_str()));
    }
    *out = f->bytes + start;
    return FOCR_HIP_OK;
}

int32_t tensor_view(const focr_hip_focrq* f, const std::string& name, View& v) {
    auto it = f->dir.find(name);
    if (it == f->dir.end())
        return format_err(fmt("tensor %s not found in weights directory", dbg(name).c_str()));
    v.rec = &it->second;
    if (int32_t st = payload_slice(f, name, v.rec->byte_offset, v.rec->byte_len, &v.data)) return st;
    v.scales = nullptr;
    if (v.rec->scales_len != 0)
        if (int32_t st = payload_slice(f, name, v.rec->scales_offset, v.rec->scales_len, &v.scales)) return st;
    return FOCR_HIP_OK;
}

int32_t shape_len(const std::string& name, uint64_t a, uint64_t b, const char* expr, uint64_t& out) {
    if (!checked_mul(a, b, out))
        return format_err(fmt("tensor %s: %s overflows usize (%llu * %llu)", dbg(name).c_str(), expr,
                              (unsigned long long)a, (unsigned long long)b));
    return FOCR_HIP_OK;
}

// weights.rs:776-799 mat(): rank 1 -> [1, len], rank 2 -> [rows, cols];
// quantized dtypes are refused (decode_f32, weights.rs:997-1022).
int32_t mat_view(const focr_hip_focrq* f, const std::string& name, View& v, uint64_t& rows, uint64_t& cols) {
    if (int32_t st = tensor_view(f, name, v)) return st;
    const auto& s = v.rec->shape;
    if (s.size() == 1) {
        rows = 1;
        cols = s[0];
    } else if (s.size() == 2) {
        rows = s[0];
        cols = s[1];
    } else {
        return format_err(fmt("tensor %s has rank %zu; mat() needs a 1-D or 2-D tensor", dbg(name).c_str(),
                              s.size()));
    }
    const int32_t dt = v.rec->dtype;
    if (dt == FOCR_HIP_DT_QINT8_PER_CHAN || dt == FOCR_HIP_DT_QINT4_PER_GROUP)
        return format_err(fmt("tensor %s: decode_f32: %s is quantized; use qint8()/qint4()", dbg(name).c_str(),
                              kDTypeNames[dt]));
    const uint64_t eb = dt == FOCR_HIP_DT_F32 ? 4 : 2;
    if (v.rec->byte_len % eb)
        return format_err(fmt("tensor %s: %s byte len %llu is not a multiple of %llu", dbg(name).c_str(),
                              kDTypeNames[dt], (unsigned long long)v.rec->byte_len, (unsigned long long)eb));
    uint64_t expected;
    if (int32_t st = shape_len(name, rows, cols, "rows*cols", expected)) return st;
    if (v.rec->byte_len / eb != expected)
        return format_err(fmt("tensor %s element count %llu != rows*cols %llu", dbg(name).c_str(),
                              (unsigned long long)(v.rec->byte_len / eb), (unsigned long long)expected));
    return FOCR_HIP_OK;
}

// weights.rs:821-862 qint8() checks.
int32_t qint8_view(const focr_hip_focrq* f, const std::string& name, View& v, uint64_t& n, uint64_t& k) {
    if (int32_t st = tensor_view(f, name, v)) return st;
    if (v.rec->dtype != FOCR_HIP_DT_QINT8_PER_CHAN)
        return format_err(fmt("tensor %s is %s, not QInt8PerChan", dbg(name).c_str(), kDTypeNames[v.rec->dtype]));
    if (v.rec->shape.size() != 2)
        return format_err(fmt("QInt8 tensor %s has rank %zu; expected 2 ([n, k])", dbg(name).c_str(),
                              v.rec->shape.size()));
    n = v.rec->shape[0];
    k = v.rec->shape[1];
    uint64_t expected;
    if (int32_t st = shape_len(name, n, k, "n*k", expected)) return st;
    if (v.rec->byte_len != expected)
        return format_err(fmt("QInt8 tensor %s: %llu payload bytes != n*k %llu", dbg(name).c_str(),
                              (unsigned long long)v.rec->byte_len, (unsigned long long)expected));
    if (v.rec->scales_len % 4)
        return format_err(fmt("F32 byte len %llu is not a multiple of 4", (unsigned long long)v.rec->scales_len));
    if (v.rec->scales_len / 4 != n)
        return format_err(fmt("QInt8 tensor %s: %llu scales != n %llu", dbg(name).c_str(),
                              (unsigned long long)(v.rec->scales_len / 4), (unsigned long long)n));
    return FOCR_HIP_OK;
}

// weights.rs:866-923 qint4() checks.
int32_t qint4_view(const focr_hip_focrq* f, const std::string& name, View& v, uint64_t& n, uint64_t& k) {
    if (int32_t st = tensor_view(f, name, v)) return st;
    const FocrqRecord& r = *v.rec;
    if (r.dtype != FOCR_HIP_DT_QINT4_PER_GROUP)
        return format_err(fmt("tensor %s is %s, not QInt4PerGroup", dbg(name).c_str(), kDTypeNames[r.dtype]));
    if (r.shape.size() != 2)
        return format_err(fmt("QInt4 tensor %s has rank %zu; expected 2 ([n, k])", dbg(name).c_str(),
                              r.shape.size()));
    n = r.shape[0];
    k = r.shape[1];
    if (k % 2)
        return format_err(fmt("QInt4 tensor %s: k %llu is not even (two nibbles per byte)", dbg(name).c_str(),
                              (unsigned long long)k));
    if (r.group_size != 16 && r.group_size != 32)
        return format_err(fmt("QInt4 tensor %s: group_size %llu must be 16 or 32", dbg(name).c_str(),
                              (unsigned long long)r.group_size));
    if (k % r.group_size)
        return format_err(fmt("QInt4 tensor %s: group_size %llu does not divide k %llu", dbg(name).c_str(),
                              (unsigned long long)r.group_size, (unsigned long long)k));
    uint64_t packed;
    if (int32_t st = shape_len(name, n, k / 2, "n*k/2", packed)) return st;
    if (r.byte_len != packed)
        return format_err(fmt("QInt4 tensor %s: %llu packed bytes != n*k/2 %llu", dbg(name).c_str(),
                              (unsigned long long)r.byte_len, (unsigned long long)packed));
    if (r.scales_len % 4)
        return format_err(fmt("F32 byte len %llu is not a multiple of 4", (unsigned long long)r.scales_len));
    uint64_t ns;
    if (int32_t st = shape_len(name, n, k / r.group_size, "n*(k/group_size)", ns)) return st;
    if (r.scales_len / 4 != ns)
        return format_err(fmt("QInt4 tensor %s: %llu scales != n*(k/group_size) %llu", dbg(name).c_str(),
                              (unsigned long long)(r.scales_len / 4), (unsigned long long)ns));
    return FOCR_HIP_OK;
}

// Host widening (weights.rs:997-1035 decode_f32): exact for every dtype.
float f16_to_f32(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000) << 16;
    const uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FF;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {  // subnormal: m * 2^-24, exact in f32
            const float v = std::ldexp(static_cast<float>(m), -24);
            uint32_t vb;
            memcpy(&vb, &v, 4);
            bits = sign | vb;
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13) | (m ? 0x00400000u : 0u);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

void widen_host(int32_t dt, const uint8_t* src, uint64_t count, float* out) {
    for (uint64_t i = 0; i < count; ++i) {
        if (dt == FOCR_HIP_DT_F32) {
            memcpy(out + i, src + 4 * i, 4);
        } else {
            uint16_t h;
            memcpy(&h, src + 2 * i, 2);
            if (dt == FOCR_HIP_DT_BF16) {
                const uint32_t bits = static_cast<uint32_t>(h) << 16;
                memcpy(out + i, &bits, 4);
            } else {
                out[i] = f16_to_f32(h);
            }
        }
    }
}

int32_t copy_str(const std::string& s, char* buf, size_t cap) {
    if (!buf) return FOCR_HIP_OK;
    if (cap == 0) return fail(FOCR_HIP_E_ARG, "buffer capacity is 0");
    const size_t n = std::min(s.size(), cap - 1);
    memcpy(buf, s.data(), n);
    buf[n] = 0;
    if (n < s.size()) return fail(FOCR_HIP_E_ARG, fmt("buffer of %zu bytes is too small for %zu bytes", cap, s.size() + 1));
    return FOCR_HIP_OK;
}

#define FQ_HANDLE(f)                                                              \
    do {                                                                          \
        if (!(f)) return fail(FOCR_HIP_E_BAD_HANDLE, "null weight container");    \
        clear_error();                                                            \
    } while (0)

}  // namespace

extern "C" {

// weights.rs:416-421 load(): an unreadable path is ModelNotFound.
int32_t focr_hip_focrq_open(const char* path, focr_hip_focrq** out) {
    if (!out || !path) return fail(FOCR_HIP_E_ARG, "focrq_open: null argument");
    *out = nullptr;
    clear_error();
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0)
        return fail(FOCR_HIP_E_NOT_FOUND, fmt("cannot read weights at %s: %s", path, strerror(errno)));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        const int e = errno;
        close(fd);
        return fail(FOCR_HIP_E_NOT_FOUND, fmt("cannot read weights at %s: %s", path, strerror(e)));
    }
    if (!S_ISREG(st.st_mode)) {
        close(fd);
        return fail(FOCR_HIP_E_NOT_FOUND, fmt("cannot read weights at %s: %s", path,
                                              S_ISDIR(st.st_mode) ? "Is a directory" : "not a regular file"));
    }
    std::unique_ptr<focr_hip_focrq> f(new focr_hip_focrq());
    f->len = static_cast<size_t>(st.st_size);
    if (f->len > 0) {
        void* m = mmap(nullptr, f->len, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            const int e = errno;
            close(fd);
            return fail(FOCR_HIP_E_NOT_FOUND, fmt("cannot read weights at %s: %s", path, strerror(e)));
        }
        f->map = m;
        f->map_len = f->len;
        f->bytes = static_cast<const uint8_t*>(m);
    } else {
        f->bytes = f->owned.data();
    }
    close(fd);
    if (int32_t st2 = parse_container(f.get())) return st2;
    *out = f.release();
    return FOCR_HIP_OK;
}

int32_t focr_hip_focrq_from_bytes(const uint8_t* bytes, size_t len, focr_hip_focrq** out) {
    if (!out || (!bytes && len)) return fail(FOCR_HIP_E_ARG, "focrq_from_bytes: null argument");
    *out = nullptr;
    clear_error();
    std::unique_ptr<focr_hip_focrq> f(new focr_hip_focrq());
    f->owned.assign(bytes, bytes + len);
    f->bytes = f->owned.data();
    f->len = len;
    if (int32_t st = parse_container(f.get())) return st;
    *out = f.release();
    return FOCR_HIP_OK;
}

int32_t focr_hip_focrq_close(focr_hip_focrq* f) {
    delete f;
    return FOCR_HIP_OK;
}

int32_t focr_hip_focrq_info(const focr_hip_focrq* f, int32_t* is_focrq, uint8_t* arch_target, size_t* n_tensors,
                            char* source_sha256, size_t sha_cap, char* model_id, size_t id_cap, char* license,
                            size_t license_cap) {
    FQ_HANDLE(f);
    if (is_focrq) *is_focrq = f->is_focrq ? 1 : 0;
    if (arch_target) *arch_target = f->arch_target;
    if (n_tensors) *n_tensors = f->dir.size();
    if (int32_t st = copy_str(f->sha, source_sha256, sha_cap)) return st;
    if (int32_t st = copy_str(f->model_id, model_id, id_cap)) return st;
    return copy_str(f->license, license, license_cap);
}

int32_t focr_hip_focrq_name(const focr_hip_focrq* f, size_t index, char* buf, size_t cap) {
    FQ_HANDLE(f);
    if (index >= f->names.size())
        return fail(FOCR_HIP_E_ARG, fmt("tensor index %zu out of range (%zu tensors)", index, f->names.size()));
    return copy_str(*f->names[index], buf, cap);
}

int32_t focr_hip_focrq_record(const focr_hip_focrq* f, const char* name, int32_t* dtype, uint64_t* shape,
                              size_t shape_cap, size_t* rank, uint64_t* byte_offset, uint64_t* byte_len,
                              uint64_t* scales_offset, uint64_t* scales_len, uint64_t* group_size, uint8_t* tier) {
    FQ_HANDLE(f);
    if (!name) return fail(FOCR_HIP_E_ARG, "focrq_record: null name");
    auto it = f->dir.find(name);
    if (it == f->dir.end()) return format_err(fmt("tensor %s not found in weights directory", dbg(name).c_str()));
    const FocrqRecord& r = it->second;
    if (dtype) *dtype = r.dtype;
    if (rank) *rank = r.shape.size();
    if (shape) {
        if (shape_cap < r.shape.size())
            return fail(FOCR_HIP_E_ARG, fmt("shape buffer holds %zu dims, tensor has %zu", shape_cap, r.shape.size()));
        std::copy(r.shape.begin(), r.shape.end(), shape);
    }
    if (byte_offset) *byte_offset = r.byte_offset;
    if (byte_len) *byte_len = r.byte_len;
    if (scales_offset) *scales_offset = r.scales_offset;
    if (scales_len) *scales_len = r.scales_len;
    if (group_size) *group_size = r.group_size;
    if (tier) *tier = r.tier;
    return FOCR_HIP_OK;
}

// weights.rs:634-670 census: the loaded name set must equal the expected set.
int32_t focr_hip_focrq_census(const focr_hip_focrq* f, const char* const* names, size_t count) {
    FQ_HANDLE(f);
    if (count && !names) return fail(FOCR_HIP_E_ARG, "focrq_census: null names");
    std::set<std::string> expected;
    for (size_t i = 0; i < count; ++i) {
        if (!names[i]) return fail(FOCR_HIP_E_ARG, "focrq_census: null name");
        expected.insert(names[i]);
    }
    std::vector<std::string> missing, unexpected;
    for (const auto& n : expected)
        if (!f->dir.count(n)) missing.push_back(n);
    for (const auto& kv : f->dir)
        if (!expected.count(kv.first)) unexpected.push_back(kv.first);
    if (missing.empty() && unexpected.empty()) return FOCR_HIP_OK;
    // weights.rs:1069-1076 preview(): up to 6 names, then ", …".
    auto preview = [](const std::vector<std::string>& v) {
        std::string s = "[";
        const size_t shown = std::min<size_t>(v.size(), 6);
        for (size_t i = 0; i < shown; ++i) s += (i ? ", " : "") + v[i];
        if (v.size() > shown) s += ", \xE2\x80\xA6";
        return s + "]";
    };
    return format_err(fmt("weights census failed: expected %zu tensors, found %zu (missing %zu: %s; unexpected %zu: "
                          "%s)", expected.size(), f->dir.size(), missing.size(), preview(missing).c_str(),
                          unexpected.size(), preview(unexpected).c_str()));
}

// weights.rs:776-819 mat()/vec(): F32/F16/BF16 widened to f32 on the host.
// out (nullable, for a size query) must hold *numel floats.
int32_t focr_hip_focrq_read_f32(const focr_hip_focrq* f, const char* name, float* out, size_t cap,
                                uint64_t* rows, uint64_t* cols) {
    FQ_HANDLE(f);
    if (!name) return fail(FOCR_HIP_E_ARG, "focrq_read_f32: null name");
    View v;
    uint64_t r, c;
    if (int32_t st = mat_view(f, name, v, r, c)) return st;
    if (rows) *rows = r;
    if (cols) *cols = c;
    if (!out) return FOCR_HIP_OK;
    if (cap < r * c) return fail(FOCR_HIP_E_ARG, fmt("focrq_read_f32: out holds %zu floats, tensor has %llu", cap,
                                                     (unsigned long long)(r * c)));
    widen_host(v.rec->dtype, v.data, r * c, out);
    return FOCR_HIP_OK;
}

// weights.rs:821-862 qint8(): int8 weights [n,k] + n scales (host copies).
int32_t focr_hip_focrq_read_qint8(const focr_hip_focrq* f, const char* name, int8_t* w, size_t w_cap, float* scales,
                                  size_t s_cap, uint64_t* n, uint64_t* k) {
    FQ_HANDLE(f);
    if (!name) return fail(FOCR_HIP_E_ARG, "focrq_read_qint8: null name");
    View v;
    uint64_t nn, kk;
    if (int32_t st = qint8_view(f, name, v, nn, kk)) return st;
    if (n) *n = nn;
    if (k) *k = kk;
    if (w) {
        if (w_cap < nn * kk) return fail(FOCR_HIP_E_ARG, "focrq_read_qint8: weight buffer too small");
        memcpy(w, v.data, nn * kk);
    }
    if (scales) {
        if (s_cap < nn) return fail(FOCR_HIP_E_ARG, "focrq_read_qint8: scale buffer too small");
        memcpy(scales, v.scales, nn * 4);
    }
    return FOCR_HIP_OK;
}

// weights.rs:866-923 qint4(): packed [n, k/2] + n*(k/group) scales.
int32_t focr_hip_focrq_read_qint4(const focr_hip_focrq* f, const char* name, uint8_t* packed, size_t p_cap,
                                  float* scales, size_t s_cap, uint64_t* n, uint64_t* k, uint64_t* group_size,
                                  uint8_t* tier) {
    FQ_HANDLE(f);
    if (!name) return fail(FOCR_HIP_E_ARG, "focrq_read_qint4: null name");
    View v;
    uint64_t nn, kk;
    if (int32_t st = qint4_view(f, name, v, nn, kk)) return st;
    if (n) *n = nn;
    if (k) *k = kk;
    if (group_size) *group_size = v.rec->group_size;
    if (tier) *tier = v.rec->tier;
    if (packed) {
        if (p_cap < v.rec->byte_len) return fail(FOCR_HIP_E_ARG, "focrq_read_qint4: packed buffer too small");
        memcpy(packed, v.data, v.rec->byte_len);
    }
    if (scales) {
        if (s_cap < v.rec->scales_len / 4) return fail(FOCR_HIP_E_ARG, "focrq_read_qint4: scale buffer too small");
        memcpy(scales, v.scales, v.rec->scales_len);
    }
    return FOCR_HIP_OK;
}

}  // extern "C"

// ---- uploads into HBM -------------------------------------------------------

namespace {

struct DevBuf {  // a device allocation freed on scope exit unless released
    void* p = nullptr;
    ~DevBuf() {
        if (p) hipFree(p);
    }
    template <typename T>
    T* as() const {
        return static_cast<T*>(p);
    }
    void* release() {
        void* q = p;
        p = nullptr;
        return q;
    }
};

int32_t dev_alloc(DevBuf& b, size_t bytes, const char* what) {
    FOCR_HIP_TRY(hipMalloc(&b.p, std::max<size_t>(bytes, 16)), what);
    return FOCR_HIP_OK;
}

// decoder.rs:1777-1786 quant_oc_loaded, into device arrays w [n][k] and
// scales [n]: a QInt8PerChan record is copied verbatim; an F32/F16/BF16
// record is copied raw and quantized per output channel on the device
// (src/quant/int8.rs:104-163 rule). out_channels = 0 takes the record's rows.
int32_t quant_oc_to_device(focr_hip_ctx* ctx, const focr_hip_focrq* f, const std::string& name, uint64_t out_channels,
                           int8_t* w, float* scales, uint64_t* n_out, uint64_t* k_out, bool dry) {
    auto it = f->dir.find(name);
    if (it != f->dir.end() && it->second.dtype == FOCR_HIP_DT_QINT8_PER_CHAN) {
        View v;
        uint64_t n, k;
        if (int32_t st = qint8_view(f, name, v, n, k)) return st;
        *n_out = n;
        *k_out = k;
        if (dry) return FOCR_HIP_OK;
        FOCR_HIP_TRY(hipMemcpyAsync(w, v.data, n * k, hipMemcpyHostToDevice, ctx->stream), "H2D int8 weight");
        FOCR_HIP_TRY(hipMemcpyAsync(scales, v.scales, n * 4, hipMemcpyHostToDevice, ctx->stream), "H2D int8 scales");
        return FOCR_HIP_OK;
    }
    View v;
    uint64_t rows, cols;
    if (int32_t st = mat_view(f, name, v, rows, cols)) return st;
    const uint64_t numel = rows * cols;
    const uint64_t n = out_channels ? out_channels : rows;
    if (n == 0 || numel % n)
        return fail(FOCR_HIP_E_SHAPE, fmt("quant_oc: tensor %s has %llu elements, not a multiple of out %llu",
                                          dbg(name).c_str(), (unsigned long long)numel, (unsigned long long)n));
    *n_out = n;
    *k_out = numel / n;
    if (dry) return FOCR_HIP_OK;
    if (n > static_cast<uint64_t>(std::numeric_limits<int>::max()) ||
        *k_out > static_cast<uint64_t>(std::numeric_limits<int>::max()))
        return fail(FOCR_HIP_E_SHAPE, fmt("quant_oc: tensor %s is too large for one launch", dbg(name).c_str()));
    DevBuf raw;
    if (int32_t st = dev_alloc(raw, v.rec->byte_len, "hipMalloc weight staging")) return st;
    FOCR_HIP_TRY(hipMemcpyAsync(raw.p, v.data, v.rec->byte_len, hipMemcpyHostToDevice, ctx->stream), "H2D raw weight");
    FOCR_HIP_TRY(launch_quant_weight_i8(ctx->stream, raw.p, v.rec->dtype, static_cast<int>(n),
                                        static_cast<int>(*k_out), w, scales),
                 "quant_weight_i8");
    // The staging buffer is freed when this returns: wait for the kernel.
    FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return FOCR_HIP_OK;
}

// weights.rs:776-799 mat() widened on the device into dst (rows*cols f32).
int32_t mat_to_device(focr_hip_ctx* ctx, const focr_hip_focrq* f, const std::string& name, float* dst,
                      uint64_t* rows_out, uint64_t* cols_out, bool dry) {
    View v;
    uint64_t rows, cols;
    if (int32_t st = mat_view(f, name, v, rows, cols)) return st;
    *rows_out = rows;
    *cols_out = cols;
    if (dry) return FOCR_HIP_OK;
    if (v.rec->dtype == FOCR_HIP_DT_F32) {
        FOCR_HIP_TRY(hipMemcpyAsync(dst, v.data, v.rec->byte_len, hipMemcpyHostToDevice, ctx->stream), "H2D f32");
        return FOCR_HIP_OK;
    }
    DevBuf raw;
    if (int32_t st = dev_alloc(raw, v.rec->byte_len, "hipMalloc f32 staging")) return st;
    FOCR_HIP_TRY(hipMemcpyAsync(raw.p, v.data, v.rec->byte_len, hipMemcpyHostToDevice, ctx->stream), "H2D raw");
    FOCR_HIP_TRY(launch_widen(ctx->stream, raw.p, v.rec->dtype, rows * cols, dst), "widen");
    FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return FOCR_HIP_OK;
}

int32_t expect_dims(const std::string& name, uint64_t n, uint64_t k, uint64_t en, uint64_t ek) {
    if (n != en || k != ek)
        return format_err(fmt("tensor %s has shape [%llu, %llu]; expected [%llu, %llu]", dbg(name).c_str(),
                              (unsigned long long)n, (unsigned long long)k, (unsigned long long)en,
                              (unsigned long long)ek));
    return FOCR_HIP_OK;
}

std::string layer_name(size_t layer, const char* rest) { return fmt("model.layers.%zu.mlp.%s", layer, rest); }

}  // namespace

extern "C" {

int32_t focr_hip_focrq_upload_qint8(focr_hip_ctx* ctx, const focr_hip_focrq* f, const char* name,
                                    uint64_t out_channels, focr_hip_qint8** out) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null context");
    FQ_HANDLE(f);
    if (!name || !out) return fail(FOCR_HIP_E_ARG, "focrq_upload_qint8: null argument");
    *out = nullptr;
    FOCR_HIP_TRY(ctx->bind(), "hipSetDevice");
    std::lock_guard<std::mutex> lk(ctx->mu);
    uint64_t n, k;
    if (int32_t st = quant_oc_to_device(ctx, f, name, out_channels, nullptr, nullptr, &n, &k, true)) return st;
    if (k % 16 != 0 || k == 0 || n == 0 || n > static_cast<uint64_t>(std::numeric_limits<int32_t>::max()))
        return fail(FOCR_HIP_E_SHAPE, fmt("QInt8: gfx950 tier needs k a positive multiple of 16 and 0 < n < 2^31 "
                                          "(n=%llu k=%llu)", (unsigned long long)n, (unsigned long long)k));
    DevBuf w, s;
    if (int32_t st = dev_alloc(w, n * k, "hipMalloc qint8 w")) return st;
    if (int32_t st = dev_alloc(s, n * 4, "hipMalloc qint8 scales")) return st;
    if (int32_t st = quant_oc_to_device(ctx, f, name, out_channels, w.as<int8_t>(), s.as<float>(), &n, &k, false))
        return st;
    FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    focr_hip_qint8* q = new focr_hip_qint8();
    q->ctx = ctx;
    q->n = n;
    q->k = k;
    q->owned = true;
    q->w = static_cast<int8_t*>(w.release());
    q->scales = static_cast<float*>(s.release());
    *out = q;
    return FOCR_HIP_OK;
}

int32_t focr_hip_focrq_upload_f32(focr_hip_ctx* ctx, const focr_hip_focrq* f, const char* name, float** dev,
                                  uint64_t* rows, uint64_t* cols) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null context");
    FQ_HANDLE(f);
    if (!name || !dev) return fail(FOCR_HIP_E_ARG, "focrq_upload_f32: null argument");
    *dev = nullptr;
    FOCR_HIP_TRY(ctx->bind(), "hipSetDevice");
    std::lock_guard<std::mutex> lk(ctx->mu);
    uint64_t r, c;
    if (int32_t st = mat_to_device(ctx, f, name, nullptr, &r, &c, true)) return st;
    DevBuf d;
    if (int32_t st = dev_alloc(d, r * c * 4, "hipMalloc f32 tensor")) return st;
    if (int32_t st = mat_to_device(ctx, f, name, d.as<float>(), &r, &c, false)) return st;
    FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (rows) *rows = r;
    if (cols) *cols = c;
    *dev = static_cast<float*>(d.release());
    return FOCR_HIP_OK;
}

// decoder.rs:2069-2098 (the MoE arm of DecoderWeightCacheI8::build) for one
// layer: router `model.layers.{l}.mlp.gate.weight` [E, hidden] widened to
// f32; experts `...mlp.experts.{e}.{gate,up,down}_proj.weight` and, with
// with_shared, `...mlp.shared_experts.*` through quant_oc_loaded.
int32_t focr_hip_focrq_moe_layer(focr_hip_ctx* ctx, const focr_hip_focrq* f, size_t layer, size_t n_experts,
                                 size_t top_k, int32_t with_shared, focr_hip_moe_layer** out) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null context");
    FQ_HANDLE(f);
    if (!out) return fail(FOCR_HIP_E_ARG, "focrq_moe_layer: null out");
    *out = nullptr;
    if (n_experts == 0) return fail(FOCR_HIP_E_SHAPE, "focrq_moe_layer: n_experts must be positive");
    // Shapes first (no device work), so a malformed container fails cleanly.
    const std::string router = layer_name(layer, "gate.weight");
    uint64_t re, hidden, inter, n, k;
    {
        View v;
        if (int32_t st = mat_view(f, router, v, re, hidden)) return st;
        if (re != n_experts)
            return format_err(fmt("tensor %s has %llu rows; expected n_experts %zu", dbg(router).c_str(),
                                  (unsigned long long)re, n_experts));
    }
    const char* proj[3] = {"gate_proj", "up_proj", "down_proj"};
    if (int32_t st = quant_oc_to_device(ctx, f, layer_name(layer, "experts.0.gate_proj.weight"), 0, nullptr, nullptr,
                                        &inter, &k, true))
        return st;
    for (size_t e = 0; e < n_experts; ++e)
        for (int p = 0; p < 3; ++p) {
            const std::string nm = layer_name(layer, fmt("experts.%zu.%s.weight", e, proj[p]).c_str());
            if (int32_t st = quant_oc_to_device(ctx, f, nm, p == 2 ? hidden : inter, nullptr, nullptr, &n, &k, true))
                return st;
            if (int32_t st = expect_dims(nm, n, k, p == 2 ? hidden : inter, p == 2 ? inter : hidden)) return st;
        }
    uint64_t shared_inter = 0;
    if (with_shared) {
        if (int32_t st = quant_oc_to_device(ctx, f, layer_name(layer, "shared_experts.gate_proj.weight"), 0, nullptr,
                                            nullptr, &shared_inter, &k, true))
            return st;
        for (int p = 0; p < 3; ++p) {
            const std::string nm = layer_name(layer, fmt("shared_experts.%s.weight", proj[p]).c_str());
            if (int32_t st = quant_oc_to_device(ctx, f, nm, p == 2 ? hidden : shared_inter, nullptr, nullptr, &n, &k,
                                                true))
                return st;
            if (int32_t st = expect_dims(nm, n, k, p == 2 ? hidden : shared_inter, p == 2 ? shared_inter : hidden))
                return st;
        }
    }
    // Device-resident stacked arrays, filled expert by expert.
    FOCR_HIP_TRY(ctx->bind(), "hipSetDevice");
    const size_t E = n_experts, H = hidden, I = inter;
    DevBuf rt, wg, wu, wd, sg, su, sd;
    int32_t st = FOCR_HIP_OK;
    if ((st = dev_alloc(rt, E * H * 4, "hipMalloc router")) || (st = dev_alloc(wg, E * I * H, "hipMalloc w_gate")) ||
        (st = dev_alloc(wu, E * I * H, "hipMalloc w_up")) || (st = dev_alloc(wd, E * H * I, "hipMalloc w_down")) ||
        (st = dev_alloc(sg, E * I * 4, "hipMalloc s_gate")) || (st = dev_alloc(su, E * I * 4, "hipMalloc s_up")) ||
        (st = dev_alloc(sd, E * H * 4, "hipMalloc s_down")))
        return st;
    {
        std::lock_guard<std::mutex> lk(ctx->mu);
        if ((st = mat_to_device(ctx, f, router, rt.as<float>(), &re, &hidden, false))) return st;
        for (size_t e = 0; e < E && !st; ++e) {
            st = quant_oc_to_device(ctx, f, layer_name(layer, fmt("experts.%zu.gate_proj.weight", e).c_str()), I,
                                    wg.as<int8_t>() + e * I * H, sg.as<float>() + e * I, &n, &k, false);
            if (!st)
                st = quant_oc_to_device(ctx, f, layer_name(layer, fmt("experts.%zu.up_proj.weight", e).c_str()), I,
                                        wu.as<int8_t>() + e * I * H, su.as<float>() + e * I, &n, &k, false);
            if (!st)
                st = quant_oc_to_device(ctx, f, layer_name(layer, fmt("experts.%zu.down_proj.weight", e).c_str()), H,
                                        wd.as<int8_t>() + e * H * I, sd.as<float>() + e * H, &n, &k, false);
        }
        const hipError_t se = hipStreamSynchronize(ctx->stream);
        if (st) return st;
        FOCR_HIP_TRY(se, "hipStreamSynchronize");
    }
    focr_hip_moe_layer* L = nullptr;
    if ((st = focr_hip_moe_layer_create(ctx, H, I, E, top_k, rt.as<float>(), wg.as<int8_t>(), sg.as<float>(),
                                        wu.as<int8_t>(), su.as<float>(), wd.as<int8_t>(), sd.as<float>(), 1, &L)))
        return st;
    // The layer was created over these arrays; hand their ownership to it.
    L->owned = true;
    rt.release(), wg.release(), wu.release(), wd.release(), sg.release(), su.release(), sd.release();
    if (with_shared) {
        const size_t S = shared_inter;
        DevBuf xg, xu, xd, yg, yu, yd;
        if ((st = dev_alloc(xg, S * H, "hipMalloc shared w_gate")) || (st = dev_alloc(xu, S * H, "hipMalloc shared w_up")) ||
            (st = dev_alloc(xd, H * S, "hipMalloc shared w_down")) || (st = dev_alloc(yg, S * 4, "hipMalloc shared s")) ||
            (st = dev_alloc(yu, S * 4, "hipMalloc shared s")) || (st = dev_alloc(yd, H * 4, "hipMalloc shared s"))) {
            focr_hip_moe_layer_free(L);
            return st;
        }
        {
            std::lock_guard<std::mutex> lk(ctx->mu);
            st = quant_oc_to_device(ctx, f, layer_name(layer, "shared_experts.gate_proj.weight"), S, xg.as<int8_t>(),
                                    yg.as<float>(), &n, &k, false);
            if (!st)
                st = quant_oc_to_device(ctx, f, layer_name(layer, "shared_experts.up_proj.weight"), S,
                                        xu.as<int8_t>(), yu.as<float>(), &n, &k, false);
            if (!st)
                st = quant_oc_to_device(ctx, f, layer_name(layer, "shared_experts.down_proj.weight"), H,
                                        xd.as<int8_t>(), yd.as<float>(), &n, &k, false);
            const hipError_t se = hipStreamSynchronize(ctx->stream);
            if (!st && se != hipSuccess) st = hip_fail(se, "hipStreamSynchronize");
        }
        if (!st)
            st = focr_hip_moe_layer_set_shared(L, S, xg.as<int8_t>(), yg.as<float>(), xu.as<int8_t>(), yu.as<float>(),
                                               xd.as<int8_t>(), yd.as<float>(), 1);
        if (st) {
            focr_hip_moe_layer_free(L);
            return st;
        }
        L->shared_owned = true;
        xg.release(), xu.release(), xd.release(), yg.release(), yu.release(), yd.release();
    }
    *out = L;
    return FOCR_HIP_OK;
}

// The int4 expert set of one layer (QInt4PerGroup records,
// weights.rs:866-923) for chunked prefill: the packed bytes and scales of
// every expert are staged in HBM in the reference layout and re-tiled once by
// focr_hip_moe_layer_i4_create. Every record must share one group_size.
int32_t focr_hip_focrq_moe_layer_i4(focr_hip_ctx* ctx, const focr_hip_focrq* f, size_t layer, size_t n_experts,
                                    focr_hip_moe_layer_i4** out) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null context");
    FQ_HANDLE(f);
    if (!out) return fail(FOCR_HIP_E_ARG, "focrq_moe_layer_i4: null out");
    *out = nullptr;
    if (n_experts == 0) return fail(FOCR_HIP_E_SHAPE, "focrq_moe_layer_i4: n_experts must be positive");
    const char* proj[3] = {"gate_proj", "up_proj", "down_proj"};
    uint64_t inter = 0, hidden = 0, group = 0;
    for (size_t e = 0; e < n_experts; ++e)
        for (int p = 0; p < 3; ++p) {
            const std::string nm = layer_name(layer, fmt("experts.%zu.%s.weight", e, proj[p]).c_str());
            View v;
            uint64_t n, k;
            if (int32_t st = qint4_view(f, nm, v, n, k)) return st;
            if (e == 0 && p == 0) {
                inter = n;
                hidden = k;
                group = v.rec->group_size;
            }
            if (int32_t st = expect_dims(nm, n, k, p == 2 ? hidden : inter, p == 2 ? inter : hidden)) return st;
            if (v.rec->group_size != group)
                return format_err(fmt("tensor %s: group_size %llu differs from the layer's %llu", dbg(nm).c_str(),
                                      (unsigned long long)v.rec->group_size, (unsigned long long)group));
        }
    FOCR_HIP_TRY(ctx->bind(), "hipSetDevice");
    const size_t E = n_experts, H = hidden, I = inter, G = group;
    const size_t nb_gu = I * (H / 2), ns_gu = I * (H / G), nb_d = H * (I / 2), ns_d = H * (I / G);
    DevBuf bg, bu, bd, cg, cu, cd;
    int32_t st = FOCR_HIP_OK;
    if ((st = dev_alloc(bg, E * nb_gu, "hipMalloc int4 staging")) || (st = dev_alloc(bu, E * nb_gu, "hipMalloc int4 staging")) ||
        (st = dev_alloc(bd, E * nb_d, "hipMalloc int4 staging")) ||
        (st = dev_alloc(cg, E * ns_gu * 4, "hipMalloc int4 staging")) ||
        (st = dev_alloc(cu, E * ns_gu * 4, "hipMalloc int4 staging")) ||
        (st = dev_alloc(cd, E * ns_d * 4, "hipMalloc int4 staging")))
        return st;
    {
        std::lock_guard<std::mutex> lk(ctx->mu);
        uint8_t* bdst[3] = {bg.as<uint8_t>(), bu.as<uint8_t>(), bd.as<uint8_t>()};
        float* sdst[3] = {cg.as<float>(), cu.as<float>(), cd.as<float>()};
        const size_t nb[3] = {nb_gu, nb_gu, nb_d}, ns[3] = {ns_gu, ns_gu, ns_d};
        for (size_t e = 0; e < E; ++e)
            for (int p = 0; p < 3; ++p) {
                View v;
                uint64_t n, k;
                qint4_view(f, layer_name(layer, fmt("experts.%zu.%s.weight", e, proj[p]).c_str()), v, n, k);
                FOCR_HIP_TRY(hipMemcpyAsync(bdst[p] + e * nb[p], v.data, nb[p], hipMemcpyHostToDevice, ctx->stream),
                             "H2D int4 packed");
                FOCR_HIP_TRY(hipMemcpyAsync(sdst[p] + e * ns[p], v.scales, ns[p] * 4, hipMemcpyHostToDevice,
                                            ctx->stream),
                             "H2D int4 scales");
            }
        FOCR_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    }
    // The layer re-tiles the staged arrays into buffers it owns.
    return focr_hip_moe_layer_i4_create(ctx, H, I, E, G, bg.as<uint8_t>(), cg.as<float>(), bu.as<uint8_t>(),
                                        cu.as<float>(), bd.as<uint8_t>(), cd.as<float>(), 1, out);
}

// src/quant/int8.rs:145-163 quantize_int8_f32 / int4.rs:142-205
// pack_int4_f32 over device arrays (src of dtype F32/F16/BF16), the
// converter-side quantizers behind QInt8PerChan / QInt4PerGroup records.
int32_t focr_hip_quantize_weight_i8(focr_hip_ctx* ctx, const void* src, int32_t src_dtype, size_t n, size_t k,
                                    int8_t* q, float* scales) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null context");
    clear_error();
    if (src_dtype != FOCR_HIP_DT_F32 && src_dtype != FOCR_HIP_DT_F16 && src_dtype != FOCR_HIP_DT_BF16)
        return fail(FOCR_HIP_E_ARG, fmt("quantize_weight_i8: src dtype %d is not F32/F16/BF16", src_dtype));
    if (n * k && (!src || !q || !scales)) return fail(FOCR_HIP_E_ARG, "quantize_weight_i8: null device pointer");
    if (n > static_cast<size_t>(std::numeric_limits<int>::max()) || k > static_cast<size_t>(std::numeric_limits<int>::max()))
        return fail(FOCR_HIP_E_SHAPE, fmt("quantize_weight_i8: n %zu / k %zu exceed i32", n, k));
    FOCR_HIP_TRY(ctx->bind(), "hipSetDevice");
    std::lock_guard<std::mutex> lk(ctx->mu);
    FOCR_HIP_TRY(launch_quant_weight_i8(ctx->stream, src, src_dtype, static_cast<int>(n), static_cast<int>(k), q, scales),
                 "quant_weight_i8");
    return FOCR_HIP_OK;
}

int32_t focr_hip_pack_weight_i4(focr_hip_ctx* ctx, const void* src, int32_t src_dtype, size_t n, size_t k,
                                size_t group, uint8_t* packed, float* scales) {
    if (!ctx) return fail(FOCR_HIP_E_BAD_HANDLE, "null context");
    clear_error();
    if (src_dtype != FOCR_HIP_DT_F32 && src_dtype != FOCR_HIP_DT_F16 && src_dtype != FOCR_HIP_DT_BF16)
        return fail(FOCR_HIP_E_ARG, fmt("pack_weight_i4: src dtype %d is not F32/F16/BF16", src_dtype));
    // int4.rs:157-166 asserts, same texts.
    if (group != 16 && group != 32)
        return fail(FOCR_HIP_E_SHAPE, fmt("pack_int4_f32: group_size %zu must be 16 or 32", group));
    if (k % 2) return fail(FOCR_HIP_E_SHAPE, fmt("pack_int4_f32: k %zu must be even", k));
    if (k % group)
        return fail(FOCR_HIP_E_SHAPE, fmt("pack_int4_f32: group_size %zu must divide k %zu (reader requires exact "
                                          "division)", group, k));
    if (n * k && (!src || !packed || !scales)) return fail(FOCR_HIP_E_ARG, "pack_weight_i4: null device pointer");
    if (n > static_cast<size_t>(std::numeric_limits<int>::max()) || k > static_cast<size_t>(std::numeric_limits<int>::max()))
        return fail(FOCR_HIP_E_SHAPE, fmt("pack_weight_i4: n %zu / k %zu exceed i32", n, k));
    FOCR_HIP_TRY(ctx->bind(), "hipSetDevice");
    std::lock_guard<std::mutex> lk(ctx->mu);
    FOCR_HIP_TRY(launch_pack_weight_i4(ctx->stream, src, src_dtype, static_cast<int>(n), static_cast<int>(k),
                                       static_cast<int>(group), packed, scales),
                 "pack_weight_i4");
    return FOCR_HIP_OK;
}

}  // extern "C"

// ---- the canonical writer (src/quant/focrq.rs:170-714) ---------------------

struct focr_hip_focrq_writer {
    struct Pending {
        int32_t dtype;
        std::vector<uint64_t> shape;
        std::vector<uint8_t> data, scales;
        uint64_t group_size;
        uint8_t tier;
    };
    uint8_t arch_target = 0;
    uint8_t sha[32] = {0};
    std::string license = kDefaultNotice;
    std::string model_id;
    std::string provenance, model_config, packing_manifest;  // canonical JSON text, "" = omitted
    bool align = false;
    std::map<std::string, Pending> tensors;
};

namespace {

// focrq.rs:695-712 push_json_string.
void json_str(std::string& s, const std::string& v) {
    s += '"';
    for (unsigned char c : v) {
        switch (c) {
            case '"': s += "\\\""; break;
            case '\\': s += "\\\\"; break;
            case '\n': s += "\\n"; break;
            case '\r': s += "\\r"; break;
            case '\t': s += "\\t"; break;
            default:
                if (c < 0x20) s += fmt("\\u%04x", c);
                else s += static_cast<char>(c);
        }
    }
    s += '"';
}

bool is_quantized(int32_t dt) { return dt == FOCR_HIP_DT_QINT8_PER_CHAN || dt == FOCR_HIP_DT_QINT4_PER_GROUP; }

// `{:?}` of the writer's dtype enum (focrq.rs:77-89 WriteDType).
const char* write_dtype_dbg(int32_t dt) { return dt == FOCR_HIP_DT_BF16 ? "Bf16" : kDTypeNames[dt]; }

// focrq.rs:351-463 insert_checked + validate_scales.
int32_t writer_insert(focr_hip_focrq_writer* w, const std::string& name, int32_t dt, const uint64_t* shape,
                      size_t rank, const uint8_t* data, size_t len, const uint8_t* scales, size_t scales_len,
                      uint64_t group_size, uint8_t tier) {
    if (w->tensors.count(name)) return format_err(fmt("add tensor: duplicate name %s", dbg(name).c_str()));
    std::vector<uint64_t> sh(shape, shape + rank);
    uint64_t numel = 1;
    for (uint64_t d : sh)
        if (!checked_mul(numel, d, numel))
            return format_err(fmt("tensor %s: shape %s element count overflows usize", dbg(name).c_str(),
                                  dbg_shape(sh).c_str()));
    uint64_t expected;
    if (dt == FOCR_HIP_DT_QINT4_PER_GROUP) {
        if (numel % 2)
            return format_err(fmt("tensor %s: QInt4 shape %s has odd element count %llu", dbg(name).c_str(),
                                  dbg_shape(sh).c_str(), (unsigned long long)numel));
        expected = numel / 2;
    } else if (dt == FOCR_HIP_DT_QINT8_PER_CHAN) {
        expected = numel;
    } else if (!checked_mul(numel, dt == FOCR_HIP_DT_F32 ? 4 : 2, expected)) {
        return format_err(fmt("tensor %s: shape*dtype bytes overflows usize (%llu * %d)", dbg(name).c_str(),
                              (unsigned long long)numel, dt == FOCR_HIP_DT_F32 ? 4 : 2));
    }
    if (len != expected)
        return format_err(fmt("tensor %s: data len %zu != shape\xC3\x97" "dtype %llu (%s, shape %s)", dbg(name).c_str(),
                              len, (unsigned long long)expected, write_dtype_dbg(dt), dbg_shape(sh).c_str()));
    if (!is_quantized(dt)) {
        if (scales_len || group_size || tier)
            return format_err(fmt("tensor %s: high-precision tensors must not carry quant metadata", dbg(name).c_str()));
    } else if (dt == FOCR_HIP_DT_QINT8_PER_CHAN) {
        if (sh.size() != 2)
            return format_err(fmt("tensor %s: QInt8 shape must be rank-2 [n,k], got %s", dbg(name).c_str(),
                                  dbg_shape(sh).c_str()));
        if (group_size || tier)
            return format_err(fmt("tensor %s: QInt8 group_size and tier must be zero", dbg(name).c_str()));
        if (scales_len != sh[0] * 4)
            return format_err(fmt("tensor %s: scale bytes %zu != qint8 n*f32 %llu", dbg(name).c_str(), scales_len,
                                  (unsigned long long)(sh[0] * 4)));
    } else {
        if (sh.size() != 2)
            return format_err(fmt("tensor %s: QInt4 shape must be rank-2 [n,k], got %s", dbg(name).c_str(),
                                  dbg_shape(sh).c_str()));
        if (group_size != 16 && group_size != 32)
            return format_err(fmt("tensor %s: QInt4 group_size %llu must be 16 or 32", dbg(name).c_str(),
                                  (unsigned long long)group_size));
        if (sh[1] % 2)
            return format_err(fmt("tensor %s: QInt4 k %llu must be even", dbg(name).c_str(), (unsigned long long)sh[1]));
        if (sh[1] % group_size)
            return format_err(fmt("tensor %s: QInt4 k %llu must be divisible by group_size %llu", dbg(name).c_str(),
                                  (unsigned long long)sh[1], (unsigned long long)group_size));
        uint64_t sc;
        if (!checked_mul(sh[0], sh[1] / group_size, sc) || !checked_mul(sc, 4, sc))
            return format_err(fmt("tensor %s: qint4 n*(k/group_size) overflows usize", dbg(name).c_str()));
        if (scales_len != sc)
            return format_err(fmt("tensor %s: scale bytes %zu != qint4 n*(k/group_size)*f32 %llu", dbg(name).c_str(),
                                  scales_len, (unsigned long long)sc));
    }
    focr_hip_focrq_writer::Pending p;
    p.dtype = dt;
    p.shape = std::move(sh);
    p.data.assign(data, data + len);
    if (scales_len) p.scales.assign(scales, scales + scales_len);
    p.group_size = group_size;
    p.tier = tier;
    w->tensors.emplace(name, std::move(p));
    return FOCR_HIP_OK;
}

// focrq.rs:479-533 build(): payload layout, canonical header, preamble.
std::vector<uint8_t> writer_build(const focr_hip_focrq_writer* w) {
    std::vector<uint8_t> payload;
    auto align = [&]() {
        if (w->align && payload.size() % 64) payload.resize(payload.size() + (64 - payload.size() % 64), 0);
    };
    std::string tj = "\"tensors\":{";
    bool first = true;
    for (const auto& kv : w->tensors) {
        const auto& t = kv.second;
        align();
        const size_t off = payload.size();
        payload.insert(payload.end(), t.data.begin(), t.data.end());
        size_t soff = 0, slen = 0;
        if (is_quantized(t.dtype)) {
            align();
            soff = payload.size();
            payload.insert(payload.end(), t.scales.begin(), t.scales.end());
            slen = t.scales.size();
        }
        // focrq.rs:654-692 push_record_json: keys in sorted order.
        if (!first) tj += ',';
        first = false;
        json_str(tj, kv.first);
        tj += fmt(":{\"byte_len\":%zu,\"byte_offset\":%zu,\"dtype\":", t.data.size(), off);
        json_str(tj, kDTypeNames[t.dtype]);
        if (is_quantized(t.dtype))
            tj += fmt(",\"group_size\":%llu,\"scales_len\":%zu,\"scales_offset\":%zu",
                      (unsigned long long)t.group_size, slen, soff);
        tj += ",\"shape\":[";
        for (size_t i = 0; i < t.shape.size(); ++i) tj += (i ? "," : "") + std::to_string(t.shape[i]);
        tj += "]";
        if (is_quantized(t.dtype)) tj += fmt(",\"tier\":%u", t.tier);
        tj += "}";
    }
    tj += "}";
    // focrq.rs:559-651 build_header_json: fixed key order.
    std::string h = "{";
    h += fmt("\"arch_target\":%u,\"format_version\":1,\"license_notice\":", w->arch_target);
    json_str(h, w->license);
    h += ',';
    if (!w->model_config.empty()) h += "\"model_config\":" + w->model_config + ",";
    if (!w->model_id.empty() && w->model_id != kRegistry[0].id) {
        h += "\"model_id\":";
        json_str(h, w->model_id);
        h += ',';
    }
    if (!w->packing_manifest.empty()) h += "\"packing_manifest\":" + w->packing_manifest + ",";
    if (!w->provenance.empty()) h += "\"provenance\":" + w->provenance + ",";
    h += "\"source_sha256\":";
    json_str(h, hex(w->sha, 32));
    h += "," + tj + "}";

    std::vector<uint8_t> blob;
    blob.reserve(51 + h.size() + payload.size());
    const uint8_t magic[6] = {'F', 'O', 'C', 'R', 'Q', 0};
    blob.insert(blob.end(), magic, magic + 6);
    const uint32_t version = 1;
    const uint8_t* vb = reinterpret_cast<const uint8_t*>(&version);
    blob.insert(blob.end(), vb, vb + 4);
    blob.push_back(w->arch_target);
    blob.insert(blob.end(), w->sha, w->sha + 32);
    const uint64_t hl = h.size();
    const uint8_t* hb = reinterpret_cast<const uint8_t*>(&hl);
    blob.insert(blob.end(), hb, hb + 8);
    blob.insert(blob.end(), h.begin(), h.end());
    blob.insert(blob.end(), payload.begin(), payload.end());
    return blob;
}

}  // namespace

extern "C" {

int32_t focr_hip_focrq_writer_new(focr_hip_focrq_writer** out) {
    if (!out) return fail(FOCR_HIP_E_ARG, "focrq_writer_new: null out");
    clear_error();
    *out = new focr_hip_focrq_writer();
    return FOCR_HIP_OK;
}

int32_t focr_hip_focrq_writer_free(focr_hip_focrq_writer* w) {
    delete w;
    return FOCR_HIP_OK;
}

int32_t focr_hip_focrq_writer_set_meta(focr_hip_focrq_writer* w, uint8_t arch_target, const uint8_t* source_sha256,
                                       const char* license_notice, const char* model_id, int32_t align) {
    if (!w) return fail(FOCR_HIP_E_BAD_HANDLE, "null focrq writer");
    clear_error();
    w->arch_target = arch_target;
    if (source_sha256) memcpy(w->sha, source_sha256, 32);
    if (license_notice) w->license = license_notice;
    if (model_id) w->model_id = model_id;
    w->align = align != 0;
    return FOCR_HIP_OK;
}

// focrq.rs:246-270: caller-supplied canonical JSON for `provenance`,
// `model_config` or `packing_manifest` (NULL or "" omits the field). The
// text must be one JSON value; it is emitted verbatim.
int32_t focr_hip_focrq_writer_set_json(focr_hip_focrq_writer* w, const char* field, const char* json) {
    if (!w) return fail(FOCR_HIP_E_BAD_HANDLE, "null focrq writer");
    if (!field) return fail(FOCR_HIP_E_ARG, "focrq_writer_set_json: null field");
    clear_error();
    std::string text = json ? json : "";
    if (!text.empty()) {
        JVal v;
        std::string err;
        if (!Json(reinterpret_cast<const uint8_t*>(text.data()), text.size()).parse(v, err))
            return fail(FOCR_HIP_E_ARG, fmt("focrq_writer_set_json: %s is not one JSON value: %s", field, err.c_str()));
    }
    const std::string fld = field;
    if (fld == "provenance") w->provenance = text;
    else if (fld == "model_config") w->model_config = text;
    else if (fld == "packing_manifest") w->packing_manifest = text;
    else return fail(FOCR_HIP_E_ARG, fmt("focrq_writer_set_json: unknown field %s", dbg(fld).c_str()));
    return FOCR_HIP_OK;
}

// focrq.rs:299-313 add_tensor (F32/F16/BF16 raw little-endian bytes).
int32_t focr_hip_focrq_writer_add_tensor(focr_hip_focrq_writer* w, const char* name, int32_t dtype,
                                         const uint64_t* shape, size_t rank, const void* data, size_t len) {
    if (!w) return fail(FOCR_HIP_E_BAD_HANDLE, "null focrq writer");
    if (!name || (rank && !shape) || (len && !data)) return fail(FOCR_HIP_E_ARG, "focrq_writer_add_tensor: null argument");
    clear_error();
    if (dtype < 0 || dtype > 4) return fail(FOCR_HIP_E_ARG, fmt("unknown dtype code %d", dtype));
    if (is_quantized(dtype))
        return format_err(fmt("add_tensor: %s is a quantized dtype %s; use add_quantized", dbg(name).c_str(),
                              write_dtype_dbg(dtype)));
    return writer_insert(w, name, dtype, shape, rank, static_cast<const uint8_t*>(data), len, nullptr, 0, 0, 0);
}

// focrq.rs:327-349 add_quantized (QInt8PerChan / QInt4PerGroup + f32 scales).
int32_t focr_hip_focrq_writer_add_quantized(focr_hip_focrq_writer* w, const char* name, int32_t dtype,
                                            const uint64_t* shape, size_t rank, const void* data, size_t len,
                                            const float* scales, size_t n_scales, uint64_t group_size, uint8_t tier) {
    if (!w) return fail(FOCR_HIP_E_BAD_HANDLE, "null focrq writer");
    if (!name || (rank && !shape) || (len && !data) || (n_scales && !scales))
        return fail(FOCR_HIP_E_ARG, "focrq_writer_add_quantized: null argument");
    clear_error();
    if (dtype < 0 || dtype > 4) return fail(FOCR_HIP_E_ARG, fmt("unknown dtype code %d", dtype));
    if (!is_quantized(dtype))
        return format_err(fmt("add_quantized: %s dtype %s is not quantized; use add_tensor", dbg(name).c_str(),
                              write_dtype_dbg(dtype)));
    return writer_insert(w, name, dtype, shape, rank, static_cast<const uint8_t*>(data), len,
                         reinterpret_cast<const uint8_t*>(scales), n_scales * 4, group_size, tier);
}

// The built blob: out == NULL queries *len; otherwise cap must hold it.
int32_t focr_hip_focrq_writer_build(const focr_hip_focrq_writer* w, uint8_t* out, size_t cap, size_t* len) {
    if (!w) return fail(FOCR_HIP_E_BAD_HANDLE, "null focrq writer");
    if (!len) return fail(FOCR_HIP_E_ARG, "focrq_writer_build: null len");
    clear_error();
    const std::vector<uint8_t> blob = writer_build(w);
    *len = blob.size();
    if (!out) return FOCR_HIP_OK;
    if (cap < blob.size()) return fail(FOCR_HIP_E_ARG, fmt("focrq_writer_build: buffer of %zu bytes < %zu", cap, blob.size()));
    memcpy(out, blob.data(), blob.size());
    return FOCR_HIP_OK;
}

// focrq.rs:535-541 write().
int32_t focr_hip_focrq_writer_write(const focr_hip_focrq_writer* w, const char* path) {
    if (!w) return fail(FOCR_HIP_E_BAD_HANDLE, "null focrq writer");
    if (!path) return fail(FOCR_HIP_E_ARG, "focrq_writer_write: null path");
    clear_error();
    const std::vector<uint8_t> blob = writer_build(w);
    FILE* fp = fopen(path, "wb");
    if (!fp) return fail(FOCR_HIP_E_ARG, fmt("writing .focrq to %s: %s", path, strerror(errno)));
    const size_t wr = fwrite(blob.data(), 1, blob.size(), fp);
    const int ce = fclose(fp);
    if (wr != blob.size() || ce != 0) return fail(FOCR_HIP_E_ARG, fmt("writing .focrq to %s: short write", path));
    return FOCR_HIP_OK;
}

}  // extern "C"
