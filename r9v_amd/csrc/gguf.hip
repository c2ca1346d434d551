/*
 * gguf.hip -- GGUF ingestion (include/r9vx_gguf.h): the container reader,
 * table validation, shard sets, per-entry XXH3, and the bind/upload step that
 * moves a checkpoint's Q4_K / IQ4_XS tensors into device memory.  Host code
 * only; the single device call is the host-to-device copy.
 *
 * Behaviour follows crates/r9v-format/src/container.rs for standard files:
 * the header/metadata/tensor-info decode of parse_internal (:952-1025) with
 * the checked little-endian cursor (:737-880), the collect-all table
 * validation of validate (:1046-1470), TensorType's wire sizes (:572-700),
 * tensor_bytes (:2074), entry_xxh3 (:2136) and ShardSet (:3469-3614).
 * Error texts follow crates/r9v-format/src/error.rs so a caller can match on
 * them.
 */
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <unordered_map>
#include <vector>

#include <hip/hip_runtime.h>

#include "r9vx.h"
#include "r9vx_gguf.h"
#include "r9vx_internal.h"
#include "r9vx_xxh3.h"

void r9vx_set_last_error(const std::string &text);  // r9vx_api.hip

namespace {

thread_local uint32_t g_problem_kinds = 0;

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" little-endian
constexpr uint64_t kDefaultAlignment = 32;

/* ------------------------------------------------------------ type table */

struct TypeRow {
    uint32_t code;
    const char *name;
    uint32_t block_len;
    uint32_t block_bytes;
};

/* gguf-py 0.19.0 GGMLQuantizationType codes and GGML_QUANT_SIZES, as
 * transcribed by TensorType (container.rs:411-612). */
constexpr TypeRow kTypes[] = {
    {0, "F32", 1, 4},        {1, "F16", 1, 2},         {2, "Q4_0", 32, 18},
    {3, "Q4_1", 32, 20},     {6, "Q5_0", 32, 22},      {7, "Q5_1", 32, 24},
    {8, "Q8_0", 32, 34},     {9, "Q8_1", 32, 40},      {10, "Q2_K", 256, 84},
    {11, "Q3_K", 256, 110},  {12, "Q4_K", 256, 144},   {13, "Q5_K", 256, 176},
    {14, "Q6_K", 256, 210},  {15, "Q8_K", 256, 292},   {16, "IQ2_XXS", 256, 66},
    {17, "IQ2_XS", 256, 74}, {18, "IQ3_XXS", 256, 98}, {19, "IQ1_S", 256, 50},
    {20, "IQ4_NL", 32, 18},  {21, "IQ3_S", 256, 110},  {22, "IQ2_S", 256, 82},
    {23, "IQ4_XS", 256, 136}, {24, "I8", 1, 1},        {25, "I16", 1, 2},
    {26, "I32", 1, 4},       {27, "I64", 1, 8},        {28, "F64", 1, 8},
    {29, "IQ1_M", 256, 56},  {30, "BF16", 1, 2},       {34, "TQ1_0", 256, 54},
    {35, "TQ2_0", 256, 66},  {39, "MXFP4", 32, 17},    {40, "NVFP4", 64, 36},
    {41, "Q1_0", 128, 18},
};

const TypeRow *type_row(uint32_t code) {
    for (const TypeRow &r : kTypes)
        if (r.code == code) return &r;
    return nullptr;
}

/* R9V native tensor type ids: 1000 + SchemeId code 1..22
 * (R9vTensorType::from_code, container.rs:294-300; scheme.rs:144-167). */
bool native_type(uint32_t code) { return code >= 1001 && code <= 1022; }

const char *kv_type_name(uint32_t t) {
    static const char *names[] = {"UINT8", "INT8",  "UINT16", "INT16", "UINT32", "INT32", "FLOAT32",
                                  "BOOL",  "STRING", "ARRAY", "UINT64", "INT64", "FLOAT64"};
    return t <= 12 ? names[t] : "?";
}

/* ------------------------------------------------------------- problems */

std::string fmt(const char *f, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    return buf;
}

struct Problem {
    uint32_t kind;
    int code;
    std::string text;
};

struct ParseError {
    Problem p;
};

Problem truncated(uint64_t offset, uint64_t need, const char *what) {
    return {R9VX_GGUF_P_TRUNCATED, R9VX_ERR_INVALID,
            fmt("truncated GGUF at offset %llu: needed %llu byte(s) for %s", (unsigned long long)offset,
                (unsigned long long)need, what)};
}
Problem malformed(uint64_t offset, const std::string &detail) {
    return {R9VX_GGUF_P_MALFORMED, R9VX_ERR_INVALID,
            fmt("malformed GGUF at offset %llu: ", (unsigned long long)offset) + detail};
}
Problem bad_range(const std::string &name, uint64_t start, uint64_t end, const std::string &reason) {
    return {R9VX_GGUF_P_BAD_RANGE, R9VX_ERR_INVALID,
            "tensor \"" + name + "\" data range [" + std::to_string(start) + ", " +
                std::to_string(end) + ") is invalid: " + reason};
}
Problem kv_type_mismatch(const std::string &key, uint32_t found, const char *expected) {
    return {R9VX_GGUF_P_KV_TYPE, R9VX_ERR_INVALID,
            "metadata key \"" + key + "\" has type " + kv_type_name(found) + ", expected " + expected};
}
Problem missing_key(const std::string &key) {
    return {R9VX_GGUF_P_MISSING_KEY, R9VX_ERR_INVALID, "missing metadata key \"" + key + "\""};
}
Problem overflow(const char *what, const std::string &detail) {
    return {R9VX_GGUF_P_OVERFLOW, R9VX_ERR_INVALID,
            std::string("size computation for ") + what + " overflowed: " + detail};
}

/* Reports every problem (FormatError::collect, error.rs:286): nothing when
 * empty, else one message joining them all. */
int report(const char *op, const std::vector<Problem> &problems) {
    if (problems.empty()) {
        g_problem_kinds = 0;
        return R9VX_OK;
    }
    uint32_t kinds = 0;
    int code = problems[0].code;
    std::string text = std::string(op) + ": ";
    for (size_t i = 0; i < problems.size(); ++i) {
        kinds |= problems[i].kind;
        if (i) text += "; ";
        text += problems[i].text;
    }
    g_problem_kinds = kinds;
    r9vx_set_last_error(text);
    return code;
}

int refuse(const char *op, int code, const std::string &text) {
    r9vx_set_last_error(std::string(op) + ": " + text);
    return code;
}

/* Strict UTF-8 (no overlong forms, no surrogates, at most U+10FFFF), the
 * acceptance rule of Rust's str::from_utf8 that read_str applies. */
bool valid_utf8(const uint8_t *s, uint64_t n) {
    uint64_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) {
            ++i;
            continue;
        }
        int extra;
        uint32_t cp, min;
        if ((c & 0xE0) == 0xC0) {
            extra = 1, cp = c & 0x1F, min = 0x80;
        } else if ((c & 0xF0) == 0xE0) {
            extra = 2, cp = c & 0x0F, min = 0x800;
        } else if ((c & 0xF8) == 0xF0) {
            extra = 3, cp = c & 0x07, min = 0x10000;
        } else {
            return false;
        }
        if (n - i <= (uint64_t)extra) return false;
        for (int j = 1; j <= extra; ++j) {
            if ((s[i + j] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + j] & 0x3F);
        }
        if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
        i += extra + 1;
    }
    return true;
}

/* ---------------------------------------------------------------- model */

struct Kv {
    std::string key;
    uint32_t type = 0;
    uint32_t elem = 0;
    std::vector<uint64_t> bits;     // numeric items
    std::vector<std::string> strs;  // string items
    uint64_t count() const { return type == R9VX_KV_STR || elem == R9VX_KV_STR ? strs.size() : bits.size(); }
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;
    uint64_t nbytes = 0;
};

/* Checked little-endian reader (container.rs:737-880): every read is bounds-
 * checked and a short read is a Truncated problem with its offset. */
struct Cursor {
    const uint8_t *b;
    uint64_t n;
    uint64_t pos = 0;

    const uint8_t *take(uint64_t len, const char *what) {
        if (len > n - pos) throw ParseError{truncated(pos, len, what)};
        const uint8_t *p = b + pos;
        pos += len;
        return p;
    }
    uint64_t u(int bytes, const char *what) {
        const uint8_t *p = take(bytes, what);
        uint64_t v = 0;
        for (int i = bytes - 1; i >= 0; --i) v = (v << 8) | p[i];
        return v;
    }
    std::string str(const char *what) {
        const uint64_t at = pos;
        const uint64_t len = u(8, "string length");
        const uint8_t *p = take(len, what);
        if (!valid_utf8(p, len)) throw ParseError{malformed(at, std::string("invalid UTF-8 in ") + what)};
        return std::string(reinterpret_cast<const char *>(p), len);
    }
    uint32_t kv_type(const char *what) {
        const uint64_t at = pos;
        const uint32_t t = (uint32_t)u(4, what);
        if (t > 12) throw ParseError{malformed(at, fmt("unknown GGUF metadata type code %u", t))};
        return t;
    }
    /* One scalar of type t into kv (read_scalar, container.rs:834-860). */
    void scalar(uint32_t t, Kv &kv) {
        switch (t) {
            case R9VX_KV_U8: kv.bits.push_back(u(1, "u8 value")); break;
            case R9VX_KV_I8: kv.bits.push_back((uint64_t)(int64_t)(int8_t)u(1, "i8 value")); break;
            case R9VX_KV_U16: kv.bits.push_back(u(2, "u16 value")); break;
            case R9VX_KV_I16: kv.bits.push_back((uint64_t)(int64_t)(int16_t)u(2, "i16 value")); break;
            case R9VX_KV_U32: kv.bits.push_back(u(4, "u32 value")); break;
            case R9VX_KV_I32: kv.bits.push_back((uint64_t)(int64_t)(int32_t)u(4, "i32 value")); break;
            case R9VX_KV_F32: kv.bits.push_back(u(4, "f32 value")); break;
            case R9VX_KV_BOOL: {
                const uint64_t at = pos;
                const uint64_t v = u(1, "bool value");
                if (v > 1) throw ParseError{malformed(at, fmt("BOOL value %llu is not 0 or 1", (unsigned long long)v))};
                kv.bits.push_back(v);
                break;
            }
            case R9VX_KV_STR: kv.strs.push_back(str("string value")); break;
            case R9VX_KV_U64: kv.bits.push_back(u(8, "u64 value")); break;
            case R9VX_KV_I64: kv.bits.push_back(u(8, "i64 value")); break;
            case R9VX_KV_F64: kv.bits.push_back(u(8, "f64 value")); break;
            default: throw ParseError{malformed(pos, "nested arrays are not valid GGUF metadata")};
        }
    }
};

/* Wire byte size of a tensor (TensorType::data_nbytes, container.rs:673-700)
 * or the problem that prevents sizing it (tensor_nbytes, :2017-2068). */
bool size_tensor(const Tensor &t, uint64_t *nbytes, Problem *why) {
    const TypeRow *row = type_row(t.type);
    if (!row) {
        *why = {R9VX_GGUF_P_UNKNOWN_TYPE, R9VX_ERR_INVALID,
                fmt("unknown tensor type code %u for tensor \"", t.type) + t.name + "\""};
        return false;
    }
    std::string dims = "[";
    for (size_t i = 0; i < t.dims.size(); ++i) dims += (i ? ", " : "") + std::to_string(t.dims[i]);
    dims += "]";
    if (t.dims.empty()) {
        *why = malformed(0, "tensor \"" + t.name + "\" has zero dimensions");
        return false;
    }
    for (uint64_t d : t.dims)
        if (d == 0) {
            *why = malformed(0, "tensor \"" + t.name + "\" has zero dimension in " + dims);
            return false;
        }
    if (t.dims[0] % row->block_len) {
        *why = malformed(0, "tensor \"" + t.name + "\" (" + row->name + "): innermost dimension " +
                                std::to_string(t.dims[0]) + " is not a multiple of block length " +
                                std::to_string(row->block_len));
        return false;
    }
    uint64_t elems = 1;
    bool ok = true;
    for (uint64_t d : t.dims) ok = ok && !__builtin_mul_overflow(elems, d, &elems);
    uint64_t bytes = 0;
    ok = ok && !__builtin_mul_overflow(elems / row->block_len, (uint64_t)row->block_bytes, &bytes);
    if (!ok) {
        *why = malformed(0, "tensor \"" + t.name + "\" (" + row->name + "): " +
                                std::to_string(UINT64_MAX) + " element(s) are not a whole number of blocks");
        return false;
    }
    *nbytes = bytes;
    return true;
}

}  // namespace

struct r9vx_gguf {
    uint32_t version = 0;
    uint64_t alignment = kDefaultAlignment;
    std::vector<Kv> kvs;
    std::unordered_map<std::string, size_t> kv_index;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> tensor_index;
    uint64_t data_start = 0;
    uint64_t file_size = 0;
    uint64_t ranges[6] = {};

    const Kv *kv(const char *key) const {
        auto it = kv_index.find(key);
        return it == kv_index.end() ? nullptr : &kvs[it->second];
    }
    const Tensor *tensor(const char *name) const {
        auto it = tensor_index.find(name);
        return it == tensor_index.end() ? nullptr : &tensors[it->second];
    }
    bool has_split_keys() const {
        for (const Kv &k : kvs)
            if (k.key.compare(0, 6, "split.") == 0) return true;
        return false;
    }
};

struct r9vx_gguf_shards {
    std::vector<const r9vx_gguf *> shards;
    std::vector<std::pair<uint32_t, size_t>> order;
};

namespace {

/* Table-level validation (GgufFile::validate, container.rs:1046-1470, the
 * standard-file part): every problem is collected. */
void validate(r9vx_gguf &f, bool size_explicit, std::vector<Problem> &pr) {
    for (size_t i = 0; i < f.kvs.size(); ++i)
        if (!f.kv_index.emplace(f.kvs[i].key, i).second)
            pr.push_back({R9VX_GGUF_P_DUPLICATE_KEY, R9VX_ERR_INVALID,
                          "duplicate metadata key \"" + f.kvs[i].key + "\""});
    for (size_t i = 0; i < f.tensors.size(); ++i)
        if (!f.tensor_index.emplace(f.tensors[i].name, i).second)
            pr.push_back({R9VX_GGUF_P_DUPLICATE_TENSOR, R9VX_ERR_INVALID,
                          "duplicate tensor name \"" + f.tensors[i].name + "\""});

    /* general.alignment: a nonzero power-of-two UINT32 (:1071-1090); a bad
     * one is reported and the default kept for the range checks below. */
    uint64_t alignment = kDefaultAlignment;
    if (const Kv *a = f.kv("general.alignment")) {
        if (a->type != R9VX_KV_U32) {
            pr.push_back(kv_type_mismatch("general.alignment", a->type, "UINT32"));
        } else {
            const uint64_t v = a->bits[0];
            if (v == 0 || (v & (v - 1)))
                pr.push_back({R9VX_GGUF_P_BAD_ALIGNMENT, R9VX_ERR_INVALID,
                              fmt("invalid alignment %llu: must be a nonzero power of two", (unsigned long long)v)});
            else
                alignment = v;
        }
    }
    f.alignment = alignment;

    /* split.* declarations must be coherent (:1146-1240). */
    if (f.has_split_keys()) {
        const Kv *no = f.kv("split.no"), *count = f.kv("split.count"), *tc = f.kv("split.tensors.count");
        bool have = true;
        auto typed = [&](const Kv *k, const char *key, uint32_t want, const char *want_name) {
            if (!k) {
                pr.push_back(missing_key(key));
                have = false;
            } else if (k->type != want) {
                pr.push_back(kv_type_mismatch(key, k->type, want_name));
                have = false;
            }
        };
        typed(no, "split.no", R9VX_KV_U16, "UINT16");
        typed(count, "split.count", R9VX_KV_U16, "UINT16");
        typed(tc, "split.tensors.count", R9VX_KV_I32, "INT32");
        if (have) {
            const uint64_t n = no->bits[0], c = count->bits[0];
            const int64_t t = (int64_t)tc->bits[0];
            if (c == 0)
                pr.push_back(malformed(0, "split.count must be >= 1"));
            else if (n >= c)
                pr.push_back(malformed(0, fmt("split.no %llu must be < split.count %llu", (unsigned long long)n,
                                              (unsigned long long)c)));
            if (t < 0) {
                pr.push_back(malformed(0, fmt("split.tensors.count %lld must be >= 0", (long long)t)));
            } else if (c == 1) {
                if (n != 0) pr.push_back(malformed(0, fmt("single-shard split.no is %llu, expected 0", (unsigned long long)n)));
                if ((uint64_t)t != f.tensors.size())
                    pr.push_back(malformed(0, fmt("split.tensors.count is %lld, expected %zu", (long long)t, f.tensors.size())));
            } else if (f.tensors.size() > (uint64_t)t) {
                pr.push_back(malformed(0, fmt("shard tensor count %zu exceeds total split.tensors.count %lld",
                                              f.tensors.size(), (long long)t)));
            }
        }
    }

    const uint64_t ti_end = f.ranges[5];
    if (ti_end > UINT64_MAX - (alignment - 1)) {
        pr.push_back(overflow("data_start", fmt("ti_end=%llu align=%llu", (unsigned long long)ti_end,
                                                (unsigned long long)alignment)));
    } else {
        f.data_start = (ti_end + alignment - 1) / alignment * alignment;
    }
    if (size_explicit && f.file_size < f.data_start) {
        pr.push_back(malformed(0, fmt("logical file size %llu is smaller than data section start %llu",
                                      (unsigned long long)f.file_size, (unsigned long long)f.data_start)));
        return;
    }

    /* Every tensor's range: aligned offset, sizable type, inside the file,
     * and no two ranges overlapping (:1280-1390). */
    struct Span {
        uint64_t start, end;
        size_t index;
        bool operator<(const Span &o) const {
            return start != o.start ? start < o.start : end != o.end ? end < o.end : index < o.index;
        }
    };
    std::vector<Span> spans;
    for (size_t i = 0; i < f.tensors.size(); ++i) {
        Tensor &t = f.tensors[i];
        uint64_t start;
        if (__builtin_add_overflow(f.data_start, t.offset, &start)) {
            pr.push_back(bad_range(t.name, UINT64_MAX, UINT64_MAX,
                                   fmt("data_start %llu + offset %llu overflows", (unsigned long long)f.data_start,
                                       (unsigned long long)t.offset)));
            continue;
        }
        if (t.offset % alignment)
            pr.push_back(bad_range(t.name, start, start,
                                   fmt("tensor offset %llu is not a multiple of alignment %llu",
                                       (unsigned long long)t.offset, (unsigned long long)alignment)));
        Problem why;
        if (!size_tensor(t, &t.nbytes, &why)) {
            pr.push_back(why);
            continue;
        }
        uint64_t end;
        if (__builtin_add_overflow(start, t.nbytes, &end)) {
            pr.push_back(bad_range(t.name, start, UINT64_MAX,
                                   fmt("range end %llu + %llu bytes overflows", (unsigned long long)start,
                                       (unsigned long long)t.nbytes)));
            continue;
        }
        if (end > f.file_size) {
            pr.push_back(bad_range(t.name, start, end,
                                   fmt("range end %llu is beyond file size %llu", (unsigned long long)end,
                                       (unsigned long long)f.file_size)));
            continue;
        }
        spans.push_back({start, end, i});
    }
    std::sort(spans.begin(), spans.end());
    if (!spans.empty()) {
        Span widest = spans[0];
        for (size_t i = 1; i < spans.size(); ++i) {
            const Span &s = spans[i];
            if (s.start < widest.end)
                pr.push_back(bad_range(f.tensors[s.index].name, s.start, s.end,
                                       "overlaps \"" + f.tensors[widest.index].name + "\" [" +
                                           std::to_string(widest.start) + ", " + std::to_string(widest.end) + ")"));
            if (s.end > widest.end) widest = s;
        }
    }
}

int parse(const uint8_t *bytes, uint64_t len, uint64_t file_size, bool size_explicit, r9vx_gguf **out) {
    const char *op = size_explicit ? "gguf_parse_table" : "gguf_parse";
    if (!out) return refuse(op, R9VX_ERR_NULL, "out is NULL");
    *out = nullptr;
    if (!bytes && len) return refuse(op, R9VX_ERR_NULL, "bytes is NULL");
    std::vector<Problem> pr;
    r9vx_gguf *f = new (std::nothrow) r9vx_gguf;
    if (!f) return refuse(op, R9VX_ERR_INVALID, "out of host memory");
    try {
        Cursor c{bytes, len};
        const uint32_t magic = (uint32_t)c.u(4, "magic");
        if (magic != kMagic)
            throw ParseError{{R9VX_GGUF_P_BAD_MAGIC, R9VX_ERR_INVALID,
                              fmt("bad GGUF magic %#010x, expected 0x46554747", magic)}};
        f->version = (uint32_t)c.u(4, "version");
        if (f->version != 2 && f->version != 3)
            throw ParseError{{R9VX_GGUF_P_BAD_VERSION, R9VX_ERR_INVALID,
                              fmt("unsupported GGUF version %u, accepts [2, 3]", f->version)}};
        const uint64_t n_tensors = c.u(8, "tensor count");
        const uint64_t n_kv = c.u(8, "metadata count");
        f->ranges[0] = 0, f->ranges[1] = c.pos;
        f->ranges[2] = c.pos;
        for (uint64_t i = 0; i < n_kv; ++i) {
            Kv kv;
            kv.key = c.str("metadata key");
            kv.type = c.kv_type("metadata type");
            if (kv.type == R9VX_KV_ARRAY) {
                kv.elem = c.kv_type("array element type");
                const uint64_t count = c.u(8, "array length");
                for (uint64_t j = 0; j < count; ++j) c.scalar(kv.elem, kv);
            } else {
                kv.elem = kv.type;
                c.scalar(kv.type, kv);
            }
            f->kvs.push_back(std::move(kv));
        }
        f->ranges[3] = c.pos;
        f->ranges[4] = c.pos;
        for (uint64_t i = 0; i < n_tensors; ++i) {
            Tensor t;
            t.name = c.str("tensor name");
            const uint32_t nd = (uint32_t)c.u(4, "tensor dimension count");
            for (uint32_t d = 0; d < nd; ++d) t.dims.push_back(c.u(8, "tensor dimension"));
            t.type = (uint32_t)c.u(4, "tensor type");
            t.offset = c.u(8, "tensor offset");
            f->tensors.push_back(std::move(t));
        }
        f->ranges[5] = c.pos;
        f->data_start = c.pos;
    } catch (const ParseError &e) {
        delete f;
        return report(op, {e.p});
    } catch (const std::bad_alloc &) {
        delete f;
        return refuse(op, R9VX_ERR_INVALID, "out of host memory while reading the tables");
    }
    f->file_size = size_explicit ? file_size : len;

    bool native = false;
    for (const Kv &k : f->kvs) native = native || k.key.compare(0, 4, "r9v.") == 0;
    for (const Tensor &t : f->tensors) native = native || native_type(t.type);
    if (native) {
        delete f;
        return report(op, {{R9VX_GGUF_P_NATIVE, R9VX_ERR_UNSUPPORTED,
                            "native R9V container (r9v.* metadata or tensor type ids 1001-1022): "
                            "this reader loads standard GGUF wire tensors only"}});
    }
    validate(*f, size_explicit, pr);
    const int rc = report(op, pr);
    if (rc != R9VX_OK) {
        delete f;
        return rc;
    }
    *out = f;
    return R9VX_OK;
}

void fill_tensor(const Tensor &t, r9vx_gguf_tensor *out) {
    const TypeRow *row = type_row(t.type);
    out->name = t.name.c_str();
    out->name_len = t.name.size();
    out->dims = t.dims.data();
    out->n_dims = (uint32_t)t.dims.size();
    out->type = t.type;
    out->offset = t.offset;
    out->nbytes = t.nbytes;
    out->block_len = row ? row->block_len : 0;
    out->block_bytes = row ? row->block_bytes : 0;
}

/* Checked slice of one entry (GgufFile::tensor_bytes, container.rs:2074-2116). */
int entry_range(const char *op, const r9vx_gguf *f, const char *name, const uint8_t *bytes, uint64_t len,
                const Tensor **tensor, const uint8_t **data) {
    if (!f || !name) return refuse(op, R9VX_ERR_NULL, "file and name are required");
    const Tensor *t = f->tensor(name);
    if (!t) return refuse(op, R9VX_ERR_INVALID, std::string("no tensor named \"") + name + "\" in this shard");
    const uint64_t start = f->data_start + t->offset;  // validated at parse: no overflow
    if (start + t->nbytes > len)
        return refuse(op, R9VX_ERR_INVALID,
                      bad_range(t->name, start, start + t->nbytes,
                                fmt("range end %llu is beyond buffer size %llu",
                                    (unsigned long long)(start + t->nbytes), (unsigned long long)len))
                          .text);
    if (!bytes) return refuse(op, R9VX_ERR_NULL, "bytes is NULL");
    *tensor = t;
    *data = bytes + start;
    return R9VX_OK;
}

/* The GGUF ggml type ids of the tensors this path reads (crates/r9v-format/
 * src/ggml.rs:38).  They are file data: a static always carries the scheme
 * code r9vx_scheme_from_ggml_type gives for them. */
constexpr uint32_t kGgmlQ8_0 = 8, kGgmlQ4_K = 12, kGgmlQ6_K = 14, kGgmlIQ3_S = 21, kGgmlIQ4_XS = 23;
bool path_scheme(uint32_t type) { return type == kGgmlQ4_K || type == kGgmlIQ4_XS; }
bool split_type(uint32_t type) { return type == kGgmlQ8_0 || type == kGgmlQ6_K; }
/* IQ3_S: repacked on the host into the 112-byte device blocks while uploading */
bool repack_type(uint32_t type) { return type == kGgmlIQ3_S; }

/* Element type and device layout of the weights this path reads per type. */
uint32_t type_dtype(uint32_t type) { return split_type(type) ? R9VX_DTYPE_I8 : R9VX_DTYPE_I4; }
uint32_t type_layout(uint32_t type) {
    return split_type(type) ? R9VX_LAYOUT_SPLIT : repack_type(type) ? R9VX_LAYOUT_IQ3S_112 : R9VX_LAYOUT_GGUF_WIRE;
}

/* Device bytes of a tensor of nbytes wire bytes. */
uint64_t device_bytes(uint32_t type, uint64_t nbytes) {
    return repack_type(type) ? nbytes / R9VX_IQ3S_BYTES * R9VX_IQ3S_DEV_BYTES : nbytes;
}

/* Host copy of `nblocks` IQ3_S wire blocks as 112-byte device blocks (the
 * layout r9vx_repack_launch writes); counts blocks whose d is not finite
 * (check_wire_f16, crates/r9v-format/src/ggml.rs:421) into *bad. */
bool iq3s_repack_host(const uint8_t *wire, uint64_t nblocks, std::vector<uint8_t> &out, uint64_t *bad) {
    try {
        out.assign(nblocks * R9VX_IQ3S_DEV_BYTES, 0);
    } catch (const std::bad_alloc &) {
        return false;
    }
    for (uint64_t b = 0; b < nblocks; ++b) {
        const uint8_t *w = wire + b * R9VX_IQ3S_BYTES;
        uint8_t *o = &out[b * R9VX_IQ3S_DEV_BYTES];
        for (uint32_t j = 0; j < R9VX_IQ3S_BYTES; ++j) o[j] = w[r9vx_iq3s_wire_byte(j)];
        *bad += (w[1] & 0x7Cu) == 0x7Cu; /* f16 exponent all ones: inf or NaN */
    }
    return true;
}

std::string dims_text(const Tensor &t) {
    std::string s = "{";
    for (size_t i = 0; i < t.dims.size(); ++i) s += (i ? ", " : "") + std::to_string(t.dims[i]);
    return s + "}";
}

int hip_rc(const char *op, hipError_t rc) {
    if (rc == hipSuccess) return R9VX_OK;
    return refuse(op, (int)rc, fmt("HIP error %d (%s)", (int)rc, hipGetErrorString(rc)));
}

}  // namespace

extern "C" {

/* GgmlType::scheme (crates/r9v-format/src/ggml.rs:253-276) restricted to the
 * five types this path reads. */
uint32_t r9vx_scheme_from_ggml_type(uint32_t ggml_type) {
    switch (ggml_type) {
    case kGgmlQ8_0: return R9VX_SCHEME_Q8_0;
    case kGgmlQ4_K: return R9VX_SCHEME_Q4_K;
    case kGgmlQ6_K: return R9VX_SCHEME_Q6_K;
    case kGgmlIQ3_S: return R9VX_SCHEME_IQ3_S;
    case kGgmlIQ4_XS: return R9VX_SCHEME_IQ4_XS;
    default: return 0;
    }
}

int r9vx_gguf_parse(const uint8_t *bytes, uint64_t len, r9vx_gguf **out) {
    return parse(bytes, len, len, false, out);
}

int r9vx_gguf_parse_table(const uint8_t *bytes, uint64_t len, uint64_t file_size, r9vx_gguf **out) {
    return parse(bytes, len, file_size, true, out);
}

void r9vx_gguf_free(r9vx_gguf *f) { delete f; }

uint32_t r9vx_gguf_last_problems(void) { return g_problem_kinds; }

uint32_t r9vx_gguf_version(const r9vx_gguf *f) { return f ? f->version : 0; }
uint64_t r9vx_gguf_alignment(const r9vx_gguf *f) { return f ? f->alignment : 0; }
uint64_t r9vx_gguf_data_start(const r9vx_gguf *f) { return f ? f->data_start : 0; }
uint64_t r9vx_gguf_file_size(const r9vx_gguf *f) { return f ? f->file_size : 0; }

void r9vx_gguf_ranges(const r9vx_gguf *f, uint64_t out[6]) {
    if (!f || !out) return;
    for (int i = 0; i < 6; ++i) out[i] = f->ranges[i];
}

uint64_t r9vx_gguf_n_kv(const r9vx_gguf *f) { return f ? f->kvs.size() : 0; }

int64_t r9vx_gguf_find_kv(const r9vx_gguf *f, const char *key) {
    if (!f || !key) return -1;
    auto it = f->kv_index.find(key);
    return it == f->kv_index.end() ? -1 : (int64_t)it->second;
}

int r9vx_gguf_kv_info(const r9vx_gguf *f, uint64_t i, const char **key, uint64_t *key_len, uint32_t *type,
                      uint32_t *elem, uint64_t *count) {
    if (!f) return refuse("gguf_kv_info", R9VX_ERR_NULL, "file is NULL");
    if (i >= f->kvs.size()) return refuse("gguf_kv_info", R9VX_ERR_INVALID, fmt("entry %llu out of range", (unsigned long long)i));
    const Kv &k = f->kvs[i];
    if (key) *key = k.key.c_str();
    if (key_len) *key_len = k.key.size();
    if (type) *type = k.type;
    if (elem) *elem = k.elem;
    if (count) *count = k.count();
    return R9VX_OK;
}

int r9vx_gguf_kv_value(const r9vx_gguf *f, uint64_t i, uint64_t item, r9vx_gguf_value *out) {
    if (!f || !out) return refuse("gguf_kv_value", R9VX_ERR_NULL, "file and out are required");
    if (i >= f->kvs.size()) return refuse("gguf_kv_value", R9VX_ERR_INVALID, fmt("entry %llu out of range", (unsigned long long)i));
    const Kv &k = f->kvs[i];
    if (item >= k.count())
        return refuse("gguf_kv_value", R9VX_ERR_INVALID,
                      fmt("item %llu of \"%s\" out of range (%llu items)", (unsigned long long)item, k.key.c_str(),
                          (unsigned long long)k.count()));
    memset(out, 0, sizeof *out);
    out->type = k.elem;
    if (k.elem == R9VX_KV_STR) {
        out->str = k.strs[item].data();
        out->str_len = k.strs[item].size();
    } else {
        out->bits = k.bits[item];
    }
    return R9VX_OK;
}

uint64_t r9vx_gguf_n_tensors(const r9vx_gguf *f) { return f ? f->tensors.size() : 0; }

int64_t r9vx_gguf_find_tensor(const r9vx_gguf *f, const char *name) {
    if (!f || !name) return -1;
    auto it = f->tensor_index.find(name);
    return it == f->tensor_index.end() ? -1 : (int64_t)it->second;
}

int r9vx_gguf_tensor_at(const r9vx_gguf *f, uint64_t i, r9vx_gguf_tensor *out) {
    if (!f || !out) return refuse("gguf_tensor_at", R9VX_ERR_NULL, "file and out are required");
    if (i >= f->tensors.size())
        return refuse("gguf_tensor_at", R9VX_ERR_INVALID, fmt("tensor %llu out of range", (unsigned long long)i));
    fill_tensor(f->tensors[i], out);
    return R9VX_OK;
}

int r9vx_gguf_tensor_bytes(const r9vx_gguf *f, const char *name, const uint8_t *bytes, uint64_t len,
                           const uint8_t **data, uint64_t *nbytes) {
    if (!data || !nbytes) return refuse("gguf_tensor_bytes", R9VX_ERR_NULL, "data and nbytes are required");
    const Tensor *t;
    const int rc = entry_range("gguf_tensor_bytes", f, name, bytes, len, &t, data);
    if (rc != R9VX_OK) return rc;
    *nbytes = t->nbytes;
    return R9VX_OK;
}

int r9vx_gguf_entry_xxh3(const r9vx_gguf *f, const char *name, const uint8_t *bytes, uint64_t len,
                         uint64_t *hash) {
    if (!hash) return refuse("gguf_entry_xxh3", R9VX_ERR_NULL, "hash is NULL");
    const Tensor *t;
    const uint8_t *data;
    const int rc = entry_range("gguf_entry_xxh3", f, name, bytes, len, &t, &data);
    if (rc != R9VX_OK) return rc;
    *hash = r9vx_xxh3::xxh3_64(data, t->nbytes);
    return R9VX_OK;
}

int r9vx_gguf_is_native(const r9vx_gguf *f) {
    (void)f;
    return 0;
}

int r9vx_gguf_type_size(uint32_t type, uint32_t *block_len, uint32_t *block_bytes) {
    const TypeRow *row = type_row(type);
    if (!row) return refuse("gguf_type_size", R9VX_ERR_UNSUPPORTED, fmt("tensor type code %u has no wire size", type));
    if (block_len) *block_len = row->block_len;
    if (block_bytes) *block_bytes = row->block_bytes;
    return R9VX_OK;
}

const char *r9vx_gguf_type_name(uint32_t type) {
    const TypeRow *row = type_row(type);
    return row ? row->name : "UNKNOWN";
}

uint64_t r9vx_xxh3_64(const void *data, uint64_t len) {
    if (!data && len) return 0;
    return r9vx_xxh3::xxh3_64(data, len);
}

/* ------------------------------------------------------------ shard sets */

int r9vx_gguf_shards_open(const r9vx_gguf *const *shards, uint32_t n, r9vx_gguf_shards **out) {
    const char *op = "gguf_shards_open";
    if (!out) return refuse(op, R9VX_ERR_NULL, "out is NULL");
    *out = nullptr;
    if (n == 0) return report(op, {malformed(0, "split shard set is empty")});
    if (!shards) return refuse(op, R9VX_ERR_NULL, "shards is NULL");
    for (uint32_t i = 0; i < n; ++i)
        if (!shards[i]) return refuse(op, R9VX_ERR_NULL, fmt("shard %u is NULL", i));
    std::vector<Problem> pr;
    auto *s = new r9vx_gguf_shards;
    std::unordered_map<std::string, uint32_t> seen;
    bool split_keys = false;
    for (uint32_t si = 0; si < n; ++si) {
        split_keys = split_keys || shards[si]->has_split_keys();
        s->shards.push_back(shards[si]);
        for (size_t ti = 0; ti < shards[si]->tensors.size(); ++ti) {
            const std::string &name = shards[si]->tensors[ti].name;
            auto ins = seen.emplace(name, si);
            if (!ins.second)
                pr.push_back({R9VX_GGUF_P_DUPLICATE_TENSOR, R9VX_ERR_INVALID,
                              "duplicate tensor name \"" + name + fmt(" (shards %u and %u)\"", ins.first->second, si)});
            else
                s->order.emplace_back(si, ti);
        }
    }
    /* Split cross-checks (ShardSet::open, container.rs:3498-3575): every
     * shard agrees on split.count = set size, split.no = its position, and
     * split.tensors.count = merged tensor count. */
    if (n > 1 || split_keys) {
        for (uint32_t si = 0; si < n; ++si) {
            const r9vx_gguf &f = *shards[si];
            const Kv *count = f.kv("split.count"), *no = f.kv("split.no"), *tc = f.kv("split.tensors.count");
            if (!count)
                pr.push_back(missing_key("split.count"));
            else if (count->type != R9VX_KV_U16)
                pr.push_back(kv_type_mismatch("split.count", count->type, "UINT16"));
            else if (count->bits[0] != n)
                pr.push_back(malformed(0, fmt("shard %u: split.count is %llu, set holds %u shards", si,
                                              (unsigned long long)count->bits[0], n)));
            if (!no)
                pr.push_back(missing_key("split.no"));
            else if (no->type != R9VX_KV_U16)
                pr.push_back(kv_type_mismatch("split.no", no->type, "UINT16"));
            else if (no->bits[0] != si)
                pr.push_back(malformed(0, fmt("shard %u: split.no is %llu, expected %u", si,
                                              (unsigned long long)no->bits[0], si)));
            if (!tc) {
                pr.push_back(missing_key("split.tensors.count"));
            } else if (tc->type != R9VX_KV_I32) {
                pr.push_back(kv_type_mismatch("split.tensors.count", tc->type, "INT32"));
            } else {
                const int64_t v = (int64_t)tc->bits[0];
                if (v < 0 || (uint64_t)v != seen.size())
                    pr.push_back(malformed(0, fmt("shard %u: split.tensors.count is %lld, expected total tensor count %zu",
                                                  si, (long long)v, seen.size())));
            }
        }
    }
    const int rc = report(op, pr);
    if (rc != R9VX_OK) {
        delete s;
        return rc;
    }
    *out = s;
    return R9VX_OK;
}

void r9vx_gguf_shards_free(r9vx_gguf_shards *s) { delete s; }

uint64_t r9vx_gguf_shards_len(const r9vx_gguf_shards *s) { return s ? s->order.size() : 0; }

int r9vx_gguf_shards_tensor_at(const r9vx_gguf_shards *s, uint64_t i, uint32_t *shard, r9vx_gguf_tensor *out) {
    if (!s || !out) return refuse("gguf_shards_tensor_at", R9VX_ERR_NULL, "set and out are required");
    if (i >= s->order.size())
        return refuse("gguf_shards_tensor_at", R9VX_ERR_INVALID, fmt("row %llu out of range", (unsigned long long)i));
    const auto &o = s->order[i];
    if (shard) *shard = o.first;
    fill_tensor(s->shards[o.first]->tensors[o.second], out);
    return R9VX_OK;
}

int64_t r9vx_gguf_shards_find(const r9vx_gguf_shards *s, const char *name) {
    if (!s || !name) return -1;
    for (size_t i = 0; i < s->shards.size(); ++i)
        if (s->shards[i]->tensor(name)) return (int64_t)i;
    return -1;
}

/* ------------------------------------------------------ binding / upload */

int r9vx_gguf_matmul_static(const r9vx_gguf *f, const char *name, r9vx_matmul_static *st) {
    const char *op = "gguf_matmul_static";
    if (!f || !name || !st) return refuse(op, R9VX_ERR_NULL, "file, name and static are required");
    const Tensor *t = f->tensor(name);
    if (!t) return refuse(op, R9VX_ERR_INVALID, std::string("no tensor named \"") + name + "\"");
    if (!path_scheme(t->type) && !split_type(t->type) && !repack_type(t->type))
        return refuse(op, R9VX_ERR_UNSUPPORTED,
                      "tensor \"" + t->name + "\" is " + r9vx_gguf_type_name(t->type) +
                          "; this path multiplies Q4_K, IQ4_XS, Q6_K, Q8_0 and IQ3_S (GGUF types 12, 23, 14, 8, 21) weights");
    if (t->dims.size() != 2 || t->dims[0] > UINT32_MAX || t->dims[1] > UINT32_MAX)
        return refuse(op, R9VX_ERR_INVALID,
                      "tensor \"" + t->name + "\" dims " + dims_text(*t) + " are not a {K, N} matrix of u32 sizes");
    if (t->dims[0] % 256)
        return refuse(op, R9VX_ERR_UNSUPPORTED,
                      "tensor \"" + t->name + "\" has K=" + std::to_string(t->dims[0]) +
                          "; the matmul kernels take K in multiples of 256");
    st->k = (uint32_t)t->dims[0];
    st->n = (uint32_t)t->dims[1];
    st->w_scheme = r9vx_scheme_from_ggml_type(t->type);
    st->w_dtype = type_dtype(t->type);
    st->w_layout = type_layout(t->type);
    return R9VX_OK;
}

int r9vx_gguf_moe_ffn_static(const r9vx_gguf *f, const char *gate, const char *up, const char *down,
                             r9vx_moe_ffn_static *st) {
    const char *op = "gguf_moe_ffn_static";
    if (!f || !gate || !down || !st) return refuse(op, R9VX_ERR_NULL, "file, gate, down and static are required");
    const Tensor *g = f->tensor(gate), *u = up ? f->tensor(up) : nullptr, *d = f->tensor(down);
    std::vector<Problem> pr;
    auto need = [&](const Tensor *t, const char *name, bool gate_up) {
        if (!t) {
            pr.push_back({0, R9VX_ERR_INVALID, std::string("no tensor named \"") + name + "\""});
            return false;
        }
        bool ok = true;
        (void)gate_up;
        if (!path_scheme(t->type) && !repack_type(t->type) && !split_type(t->type)) {
            pr.push_back({0, R9VX_ERR_UNSUPPORTED, "tensor \"" + t->name + "\" is " + r9vx_gguf_type_name(t->type) +
                                                       "; experts must be Q4_K (12), IQ4_XS (23), IQ3_S (21), Q8_0 (8) "
                                                       "or Q6_K (14)"});
            ok = false;
        }
        if (t->dims.size() != 3 || t->dims[0] > UINT32_MAX || t->dims[1] > UINT32_MAX || t->dims[2] > UINT32_MAX) {
            pr.push_back({0, R9VX_ERR_INVALID, "tensor \"" + t->name + "\" dims " + dims_text(*t) +
                                                   " are not a stacked-expert {K, rows, E} of u32 sizes"});
            ok = false;
        }
        return ok;
    };
    const bool gok = need(g, gate, true), dok = need(d, down, false);
    const bool uok = up ? need(u, up, true) : true;
    if (gok && dok && uok) {
        const uint64_t dm = g->dims[0], e = g->dims[2];
        uint64_t dff = g->dims[1];
        if (up) {
            if (u->dims != g->dims || u->type != g->type)
                pr.push_back({0, R9VX_ERR_INVALID, "gate \"" + g->name + "\" " + dims_text(*g) + " " +
                                                       r9vx_gguf_type_name(g->type) + " and up \"" + u->name + "\" " +
                                                       dims_text(*u) + " " + r9vx_gguf_type_name(u->type) +
                                                       " must agree in dims and type"});
        } else if (dff % 2) {
            pr.push_back({0, R9VX_ERR_INVALID, "fused gate_up \"" + g->name + "\" has an odd row count " +
                                                   std::to_string(dff)});
        } else {
            dff /= 2;
        }
        if (d->dims[0] != dff || d->dims[1] != dm || d->dims[2] != e)
            pr.push_back({0, R9VX_ERR_INVALID, "down \"" + d->name + "\" dims " + dims_text(*d) + " must be {" +
                                                   std::to_string(dff) + ", " + std::to_string(dm) + ", " +
                                                   std::to_string(e) + "} to match the gate/up experts"});
        if (pr.empty()) {
            st->e_local = (uint32_t)e;
            st->dm = (uint32_t)dm;
            st->dff = (uint32_t)dff;
            st->gate_up = r9vx_moe_ffn_proj{type_dtype(g->type), r9vx_scheme_from_ggml_type(g->type), type_layout(g->type)};
            st->down = r9vx_moe_ffn_proj{type_dtype(d->type), r9vx_scheme_from_ggml_type(d->type), type_layout(d->type)};
        }
    }
    if (pr.empty()) return R9VX_OK;
    std::string text;
    int code = pr[0].code;
    for (size_t i = 0; i < pr.size(); ++i) text += (i ? "; " : "") + pr[i].text;
    return refuse(op, code, text);
}

int r9vx_gguf_upload(const r9vx_gguf *f, const uint8_t *bytes, uint64_t len, const char *name, void *dst,
                     uint64_t dst_bytes, r9vx_stream_t stream) {
    const char *op = "gguf_upload";
    const Tensor *t;
    const uint8_t *data;
    const int rc = entry_range(op, f, name, bytes, len, &t, &data);
    if (rc != R9VX_OK) return rc;
    if (split_type(t->type))
        return refuse(op, R9VX_ERR_UNSUPPORTED,
                      "tensor \"" + t->name + "\" is " + r9vx_gguf_type_name(t->type) +
                          "; Q8_0 / Q6_K load into the split layout with r9vx_gguf_upload_split");
    if (!dst) return refuse(op, R9VX_ERR_NULL, "dst is NULL");
    const uint64_t need = device_bytes(t->type, t->nbytes);
    if (dst_bytes < need)
        return refuse(op, R9VX_ERR_INVALID,
                      fmt("dst holds %llu bytes, tensor \"%s\" needs %llu%s", (unsigned long long)dst_bytes,
                          t->name.c_str(), (unsigned long long)need,
                          repack_type(t->type) ? " (112-byte IQ3_S device blocks)" : ""));
    if (!repack_type(t->type))
        return hip_rc(op, hipMemcpyAsync(dst, data, t->nbytes, hipMemcpyHostToDevice, (hipStream_t)stream));
    std::vector<uint8_t> dev;
    uint64_t bad = 0;
    if (!iq3s_repack_host(data, t->nbytes / R9VX_IQ3S_BYTES, dev, &bad))
        return refuse(op, R9VX_ERR_INVALID, "out of host memory for the IQ3_S repack");
    if (bad)
        return refuse(op, R9VX_ERR_INVALID,
                      fmt("tensor \"%s\": %llu block(s) carry a non-finite scale", t->name.c_str(),
                          (unsigned long long)bad));
    hipStream_t s = (hipStream_t)stream;
    const int cp = hip_rc(op, hipMemcpyAsync(dst, dev.data(), dev.size(), hipMemcpyHostToDevice, s));
    const int sync = hip_rc(op, hipStreamSynchronize(s)); /* the host copy dies with this call */
    return cp != R9VX_OK ? cp : sync;
}

int r9vx_gguf_upload_split(const r9vx_gguf *f, const uint8_t *bytes, uint64_t len, const char *name, void *body,
                           uint64_t body_bytes, uint16_t *scales, uint64_t scales_bytes, r9vx_stream_t stream) {
    const char *op = "gguf_upload_split";
    const Tensor *t;
    const uint8_t *data;
    int rc = entry_range(op, f, name, bytes, len, &t, &data);
    if (rc != R9VX_OK) return rc;
    if (!split_type(t->type))
        return refuse(op, R9VX_ERR_UNSUPPORTED,
                      "tensor \"" + t->name + "\" is " + r9vx_gguf_type_name(t->type) +
                          "; the split layout is for Q8_0 (8) and Q6_K (14)");
    if (!body || !scales) return refuse(op, R9VX_ERR_NULL, "body and scales are required");
    const TypeRow *row = type_row(t->type);
    const uint64_t nblocks = t->nbytes / row->block_bytes;
    const uint32_t body_block = row->block_bytes - 2, d_off = t->type == kGgmlQ8_0 ? 0 : 208;
    if (body_bytes < nblocks * body_block || scales_bytes < nblocks * 2)
        return refuse(op, R9VX_ERR_INVALID,
                      fmt("body holds %llu and scales %llu bytes; tensor \"%s\" needs %llu and %llu",
                          (unsigned long long)body_bytes, (unsigned long long)scales_bytes, t->name.c_str(),
                          (unsigned long long)(nblocks * body_block), (unsigned long long)(nblocks * 2)));
    /* split on the host (body = the block without d, d to its own array),
     * refusing non-finite d (check_wire_f16, crates/r9v-format/src/ggml.rs:421) */
    std::vector<uint8_t> hb;
    std::vector<uint16_t> hs;
    try {
        hb.resize(nblocks * body_block);
        hs.resize(nblocks);
    } catch (const std::bad_alloc &) {
        return refuse(op, R9VX_ERR_INVALID, "out of host memory for the split copy");
    }
    uint64_t bad = 0;
    for (uint64_t b = 0; b < nblocks; ++b) {
        const uint8_t *blk = data + b * row->block_bytes;
        const uint16_t d = (uint16_t)(blk[d_off] | (blk[d_off + 1] << 8));
        bad += (d & 0x7C00u) == 0x7C00u;
        hs[b] = d;
        if (d_off == 0)
            memcpy(&hb[b * body_block], blk + 2, body_block);
        else
            memcpy(&hb[b * body_block], blk, body_block);
    }
    if (bad)
        return refuse(op, R9VX_ERR_INVALID,
                      fmt("tensor \"%s\": %llu block(s) carry a non-finite scale", t->name.c_str(),
                          (unsigned long long)bad));
    hipStream_t s = (hipStream_t)stream;
    rc = hip_rc(op, hipMemcpyAsync(body, hb.data(), hb.size(), hipMemcpyHostToDevice, s));
    if (rc == R9VX_OK) rc = hip_rc(op, hipMemcpyAsync(scales, hs.data(), hs.size() * 2, hipMemcpyHostToDevice, s));
    /* the host copies die with this call */
    const int sync = hip_rc(op, hipStreamSynchronize(s));
    return rc != R9VX_OK ? rc : sync;
}

int r9vx_gguf_upload_gate_up(const r9vx_gguf *gate_file, const uint8_t *gate_bytes, uint64_t gate_len,
                             const char *gate, const r9vx_gguf *up_file, const uint8_t *up_bytes, uint64_t up_len,
                             const char *up, void *dst, uint64_t dst_bytes, r9vx_stream_t stream) {
    const char *op = "gguf_upload_gate_up";
    const Tensor *g, *u;
    const uint8_t *gdata, *udata;
    int rc = entry_range(op, gate_file, gate, gate_bytes, gate_len, &g, &gdata);
    if (rc != R9VX_OK) return rc;
    rc = entry_range(op, up_file, up, up_bytes, up_len, &u, &udata);
    if (rc != R9VX_OK) return rc;
    if ((!path_scheme(g->type) && !repack_type(g->type)) || g->dims.size() != 3 || u->dims != g->dims ||
        u->type != g->type)
        return refuse(op, R9VX_ERR_INVALID,
                      "gate \"" + g->name + "\" " + dims_text(*g) + " " + r9vx_gguf_type_name(g->type) + " and up \"" +
                          u->name + "\" " + dims_text(*u) + " " + r9vx_gguf_type_name(u->type) +
                          " must be stacked Q4_K / IQ4_XS / IQ3_S experts {K, rows, E} of one dims and type");
    if (!dst) return refuse(op, R9VX_ERR_NULL, "dst is NULL");
    const uint64_t need = 2 * device_bytes(g->type, g->nbytes);
    if (dst_bytes < need)
        return refuse(op, R9VX_ERR_INVALID,
                      fmt("dst holds %llu bytes, the stacked gate_up needs %llu%s", (unsigned long long)dst_bytes,
                          (unsigned long long)need, repack_type(g->type) ? " (112-byte IQ3_S device blocks)" : ""));
    const TypeRow *row = type_row(g->type);
    const uint64_t blocks_per_expert = g->dims[0] / row->block_len * g->dims[1];
    const uint64_t experts = g->dims[2];
    uint8_t *d = static_cast<uint8_t *>(dst);
    hipStream_t s = (hipStream_t)stream;
    if (!repack_type(g->type)) {
        const uint64_t slab = blocks_per_expert * row->block_bytes;  // one expert's rows
        rc = hip_rc(op, hipMemcpy2DAsync(d, 2 * slab, gdata, slab, slab, experts, hipMemcpyHostToDevice, s));
        if (rc != R9VX_OK) return rc;
        return hip_rc(op, hipMemcpy2DAsync(d + slab, 2 * slab, udata, slab, slab, experts, hipMemcpyHostToDevice, s));
    }
    /* IQ3_S: both tensors repacked on the host, then stacked the same way */
    std::vector<uint8_t> gdev, udev;
    uint64_t bad = 0;
    if (!iq3s_repack_host(gdata, blocks_per_expert * experts, gdev, &bad) ||
        !iq3s_repack_host(udata, blocks_per_expert * experts, udev, &bad))
        return refuse(op, R9VX_ERR_INVALID, "out of host memory for the IQ3_S repack");
    if (bad)
        return refuse(op, R9VX_ERR_INVALID,
                      fmt("gate \"%s\" / up \"%s\": %llu block(s) carry a non-finite scale", g->name.c_str(),
                          u->name.c_str(), (unsigned long long)bad));
    const uint64_t slab = blocks_per_expert * R9VX_IQ3S_DEV_BYTES;
    rc = hip_rc(op, hipMemcpy2DAsync(d, 2 * slab, gdev.data(), slab, slab, experts, hipMemcpyHostToDevice, s));
    if (rc == R9VX_OK)
        rc = hip_rc(op, hipMemcpy2DAsync(d + slab, 2 * slab, udev.data(), slab, slab, experts, hipMemcpyHostToDevice, s));
    const int sync = hip_rc(op, hipStreamSynchronize(s)); /* the host copies die with this call */
    return rc != R9VX_OK ? rc : sync;
}

int r9vx_gguf_upload_gate_up_split(const r9vx_gguf *gate_file, const uint8_t *gate_bytes, uint64_t gate_len,
                                   const char *gate, const r9vx_gguf *up_file, const uint8_t *up_bytes,
                                   uint64_t up_len, const char *up, void *body, uint64_t body_bytes, uint16_t *scales,
                                   uint64_t scales_bytes, r9vx_stream_t stream) {
    const char *op = "gguf_upload_gate_up_split";
    const Tensor *g, *u;
    const uint8_t *gdata, *udata;
    int rc = entry_range(op, gate_file, gate, gate_bytes, gate_len, &g, &gdata);
    if (rc != R9VX_OK) return rc;
    rc = entry_range(op, up_file, up, up_bytes, up_len, &u, &udata);
    if (rc != R9VX_OK) return rc;
    if (!split_type(g->type) || g->dims.size() != 3 || u->dims != g->dims || u->type != g->type)
        return refuse(op, R9VX_ERR_INVALID,
                      "gate \"" + g->name + "\" " + dims_text(*g) + " " + r9vx_gguf_type_name(g->type) + " and up \"" +
                          u->name + "\" " + dims_text(*u) + " " + r9vx_gguf_type_name(u->type) +
                          " must be stacked Q8_0 / Q6_K experts {K, rows, E} of one dims and type");
    if (!body || !scales) return refuse(op, R9VX_ERR_NULL, "body and scales are required");
    const TypeRow *row = type_row(g->type);
    const uint64_t per_expert = g->dims[0] / row->block_len * g->dims[1]; /* blocks */
    const uint64_t experts = g->dims[2], nblocks = per_expert * experts;
    const uint32_t body_block = row->block_bytes - 2, d_off = g->type == kGgmlQ8_0 ? 0 : 208;
    if (body_bytes < 2 * nblocks * body_block || scales_bytes < 2 * nblocks * 2)
        return refuse(op, R9VX_ERR_INVALID,
                      fmt("body holds %llu and scales %llu bytes; the stacked gate_up needs %llu and %llu",
                          (unsigned long long)body_bytes, (unsigned long long)scales_bytes,
                          (unsigned long long)(2 * nblocks * body_block), (unsigned long long)(4 * nblocks)));
    /* expert x's gate blocks, then its up blocks, split on the host into the
     * body and the d array (non-finite d refused, check_wire_f16,
     * crates/r9v-format/src/ggml.rs:421) */
    std::vector<uint8_t> hb;
    std::vector<uint16_t> hs;
    try {
        hb.resize(2 * nblocks * body_block);
        hs.resize(2 * nblocks);
    } catch (const std::bad_alloc &) {
        return refuse(op, R9VX_ERR_INVALID, "out of host memory for the split copy");
    }
    uint64_t bad = 0;
    for (uint64_t x = 0; x < experts; ++x)
        for (int half = 0; half < 2; ++half) {
            const uint8_t *src = (half ? udata : gdata) + x * per_expert * row->block_bytes;
            const uint64_t at = (2 * x + half) * per_expert;
            for (uint64_t b = 0; b < per_expert; ++b) {
                const uint8_t *blk = src + b * row->block_bytes;
                const uint16_t d = (uint16_t)(blk[d_off] | (blk[d_off + 1] << 8));
                bad += (d & 0x7C00u) == 0x7C00u;
                hs[at + b] = d;
                memcpy(&hb[(at + b) * body_block], d_off == 0 ? blk + 2 : blk, body_block);
            }
        }
    if (bad)
        return refuse(op, R9VX_ERR_INVALID,
                      fmt("gate \"%s\" / up \"%s\": %llu block(s) carry a non-finite scale", g->name.c_str(),
                          u->name.c_str(), (unsigned long long)bad));
    hipStream_t s = (hipStream_t)stream;
    rc = hip_rc(op, hipMemcpyAsync(body, hb.data(), hb.size(), hipMemcpyHostToDevice, s));
    if (rc == R9VX_OK) rc = hip_rc(op, hipMemcpyAsync(scales, hs.data(), hs.size() * 2, hipMemcpyHostToDevice, s));
    const int sync = hip_rc(op, hipStreamSynchronize(s)); /* the host copies die with this call */
    return rc != R9VX_OK ? rc : sync;
}

}  // extern "C"
