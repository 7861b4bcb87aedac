// safetensors bundles into device buffers (include/minifield_loader.h).
//
// The header checks restate parse_safetensors_header and its document
// visitors (crates/executor-core/src/loader/header.rs:18-357) with the same
// statuses and messages; the upload path follows the loader's tensor decode
// (crates/executor-core/src/loader.rs:408-485, 1130-1200).  The JSON reader
// is this file's own: the header grammar needs objects, arrays of unsigned
// integers and strings only, and anything else is "invalid safetensors
// header JSON".
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "../../include/minifield_convert.h"
#include "../../include/minifield_loader.h"
#include "internal.hpp"
#include "kernels.hpp"

namespace {

thread_local const char *g_error = "no error";

mfh_status fail_s(mfh_status status, const char *message)
{
    g_error = message;
    return status;
}

struct Tensor {
    std::string name;
    mfs_dtype dtype = MFS_F32;
    uint32_t rank = 0;
    uint64_t dims[4] = {0, 0, 0, 0};
    uint64_t elements = 0;
    uint64_t offset = 0;  // from the start of the file
    uint64_t bytes = 0;
};

uint64_t dtype_width(mfs_dtype d)
{
    return d == MFS_F32 ? 4 : d == MFS_U8 ? 1 : 2;
}

// ---- the header's JSON ------------------------------------------------------

struct Json {
    const char *p, *end;
    mfh_status status = MFH_OK;
    const char *message = nullptr;

    bool bad(mfh_status s, const char *m)
    {
        if (status == MFH_OK) {
            status = s;
            message = m;
        }
        return false;
    }
    bool invalid() { return bad(MFH_INVALID_ARGUMENT, "invalid safetensors header JSON"); }
    void space()
    {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r'))
            ++p;
    }
    bool eat(char c)
    {
        space();
        if (p < end && *p == c) {
            ++p;
            return true;
        }
        return false;
    }
    static void put_utf8(std::string &out, uint32_t cp)
    {
        if (cp < 0x80) {
            out += char(cp);
        } else if (cp < 0x800) {
            out += char(0xC0 | (cp >> 6));
            out += char(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += char(0xE0 | (cp >> 12));
            out += char(0x80 | ((cp >> 6) & 0x3F));
            out += char(0x80 | (cp & 0x3F));
        } else {
            out += char(0xF0 | (cp >> 18));
            out += char(0x80 | ((cp >> 12) & 0x3F));
            out += char(0x80 | ((cp >> 6) & 0x3F));
            out += char(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t *v)
    {
        if (end - p < 4)
            return false;
        uint32_t r = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p++;
            r <<= 4;
            if (c >= '0' && c <= '9')
                r |= uint32_t(c - '0');
            else if (c >= 'a' && c <= 'f')
                r |= uint32_t(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F')
                r |= uint32_t(c - 'A' + 10);
            else
                return false;
        }
        *v = r;
        return true;
    }
    bool string(std::string *out)
    {
        space();
        if (p >= end || *p != '"')
            return invalid();
        ++p;
        out->clear();
        while (p < end && *p != '"') {
            const unsigned char c = static_cast<unsigned char>(*p);
            if (c < 0x20)
                return invalid();
            if (c != '\\') {
                *out += char(c);
                ++p;
                continue;
            }
            if (++p >= end)
                return invalid();
            const char e = *p++;
            switch (e) {
            case '"': *out += '"'; break;
            case '\\': *out += '\\'; break;
            case '/': *out += '/'; break;
            case 'b': *out += '\b'; break;
            case 'f': *out += '\f'; break;
            case 'n': *out += '\n'; break;
            case 'r': *out += '\r'; break;
            case 't': *out += '\t'; break;
            case 'u': {
                uint32_t cp = 0;
                if (!hex4(&cp))
                    return invalid();
                if (cp >= 0xD800 && cp < 0xDC00) {
                    uint32_t lo = 0;
                    if (end - p < 2 || p[0] != '\\' || p[1] != 'u')
                        return invalid();
                    p += 2;
                    if (!hex4(&lo) || lo < 0xDC00 || lo >= 0xE000)
                        return invalid();
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                } else if (cp >= 0xDC00 && cp < 0xE000) {
                    return invalid();
                }
                put_utf8(*out, cp);
                break;
            }
            default: return invalid();
            }
        }
        if (p >= end)
            return invalid();
        ++p;
        return true;
    }
    bool u64(uint64_t *v)
    {
        space();
        if (p >= end || *p < '0' || *p > '9')
            return invalid();
        if (*p == '0' && p + 1 < end && p[1] >= '0' && p[1] <= '9')
            return invalid();  // no leading zeros
        uint64_t r = 0;
        while (p < end && *p >= '0' && *p <= '9') {
            const uint64_t d = uint64_t(*p - '0');
            if (r > (UINT64_MAX - d) / 10)
                return invalid();
            r = r * 10 + d;
            ++p;
        }
        if (p < end && (*p == '.' || *p == 'e' || *p == 'E'))
            return invalid();
        *v = r;
        return true;
    }
    // Any JSON value (RFC 8259); its text is kept only when it is a string.
    bool value(std::string *text, bool *is_string, int depth = 0)
    {
        space();
        if (p >= end)
            return invalid();
        *is_string = *p == '"';
        if (*is_string)
            return string(text);
        if (depth > 64)
            return invalid();
        std::string skip;
        bool nested = false;
        if (eat('{')) {
            if (eat('}'))
                return true;
            do {
                if (!string(&skip) || !eat(':') || !value(&skip, &nested, depth + 1))
                    return invalid();
            } while (eat(','));
            return eat('}') ? true : invalid();
        }
        if (eat('[')) {
            if (eat(']'))
                return true;
            do {
                if (!value(&skip, &nested, depth + 1))
                    return false;
            } while (eat(','));
            return eat(']') ? true : invalid();
        }
        for (const char *word : {"true", "false", "null"}) {
            const size_t n = std::strlen(word);
            if (size_t(end - p) >= n && std::memcmp(p, word, n) == 0) {
                p += n;
                return true;
            }
        }
        // -?(0|[1-9][0-9]*)(.[0-9]+)?([eE][+-]?[0-9]+)?
        auto digits = [&] {
            const char *q = p;
            while (p < end && *p >= '0' && *p <= '9')
                ++p;
            return p > q;
        };
        if (p < end && *p == '-')
            ++p;
        if (p < end && *p == '0')
            ++p;
        else if (!digits())
            return invalid();
        if (p < end && *p == '.' && (++p, !digits()))
            return invalid();
        if (p < end && (*p == 'e' || *p == 'E')) {
            ++p;
            if (p < end && (*p == '+' || *p == '-'))
                ++p;
            if (!digits())
                return invalid();
        }
        return true;
    }
    bool u64_array(std::vector<uint64_t> *out)
    {
        if (!eat('['))
            return invalid();
        out->clear();
        if (eat(']'))
            return true;
        do {
            uint64_t v = 0;
            if (!u64(&v))
                return false;
            out->push_back(v);
        } while (eat(','));
        return eat(']') ? true : invalid();
    }
};

// StorageDType::parse (loader.rs:59-73).
bool parse_dtype(Json &j, const std::string &text, mfs_dtype *out)
{
    if (text == "F32")
        *out = MFS_F32;
    else if (text == "BF16")
        *out = MFS_BF16;
    else if (text == "F16")
        *out = MFS_F16;
    else if (text == "U8")
        *out = MFS_U8;
    else if (text == "F64")
        return j.bad(MFH_UNSUPPORTED, "safetensors storage dtype is unsupported by this loader");
    else
        return j.bad(MFH_INVALID_DTYPE, "unknown safetensors storage dtype");
    return true;
}

struct RawTensor {
    std::string name;
    mfs_dtype dtype = MFS_F32;
    std::vector<uint64_t> shape;
    uint64_t start = 0, stop = 0;
};

// TensorVisitor (header.rs:280-320): exactly dtype, shape and data_offsets.
bool parse_tensor(Json &j, RawTensor *t)
{
    if (!j.eat('{'))
        return j.invalid();
    std::set<std::string> fields;
    bool have_dtype = false, have_shape = false, have_offsets = false;
    if (!j.eat('}')) {
        do {
            std::string key;
            if (!j.string(&key))
                return false;
            if (!j.eat(':'))
                return j.invalid();
            if (!fields.insert(key).second)
                return j.bad(MFH_DUPLICATE_NAME, "duplicate name");
            if (key == "dtype") {
                std::string text;
                if (!j.string(&text) || !parse_dtype(j, text, &t->dtype))
                    return false;
                have_dtype = true;
            } else if (key == "shape") {
                if (!j.u64_array(&t->shape))
                    return false;
                have_shape = true;
            } else if (key == "data_offsets") {
                std::vector<uint64_t> offsets;
                if (!j.u64_array(&offsets))
                    return false;
                if (offsets.size() != 2)
                    return j.invalid();
                t->start = offsets[0];
                t->stop = offsets[1];
                have_offsets = true;
            } else {
                return j.invalid();  // unknown safetensors tensor field
            }
        } while (j.eat(','));
        if (!j.eat('}'))
            return j.invalid();
    }
    if (!have_dtype || !have_shape || !have_offsets)
        return j.invalid();
    return true;
}

// MetadataVisitor (header.rs:236-258): a string-to-string object.
bool parse_metadata(Json &j, std::map<std::string, std::string> *out)
{
    if (!j.eat('{'))
        return j.invalid();
    if (j.eat('}'))
        return true;
    do {
        std::string key, value;
        if (!j.string(&key))
            return false;
        if (!j.eat(':'))
            return j.invalid();
        if (out->count(key))
            return j.bad(MFH_DUPLICATE_NAME, "duplicate name");
        if (!j.string(&value))
            return false;
        (*out)[key] = value;
    } while (j.eat(','));
    return j.eat('}') ? true : j.invalid();
}

}  // namespace

struct mfs_file {
    int fd = -1;
    const uint8_t *map = nullptr;
    uint64_t size = 0;
    std::vector<Tensor> tensors;
    std::map<std::string, size_t> by_name;
    std::map<std::string, std::string> metadata;

    ~mfs_file()
    {
        if (map)
            munmap(const_cast<uint8_t *>(map), size);
        if (fd >= 0)
            close(fd);
    }
    const Tensor *find(const std::string &name) const
    {
        auto it = by_name.find(name);
        return it == by_name.end() ? nullptr : &tensors[it->second];
    }
};

namespace {

// parse_safetensors_header (header.rs:18-133) over the mapped file.
mfh_status parse_file(mfs_file *f, uint64_t max_header_bytes)
{
    if (f->size < 8)
        return fail_s(MFH_INVALID_ARGUMENT, "header prefix has invalid length");
    uint64_t header_bytes = 0;
    for (int i = 7; i >= 0; --i)
        header_bytes = (header_bytes << 8) | f->map[i];
    if (header_bytes == 0 || header_bytes > max_header_bytes)
        return fail_s(MFH_RESOURCE_LIMIT, "header exceeds configured byte limit");
    if (header_bytes > f->size - 8)
        return fail_s(MFH_OUT_OF_BOUNDS, "header extends beyond declared asset bytes");
    const char *text = reinterpret_cast<const char *>(f->map + 8);
    if (text[0] != '{')
        return fail_s(MFH_INVALID_ARGUMENT, "safetensors header must begin with an object brace");
    const uint64_t payload_start = 8 + header_bytes;
    const uint64_t payload_bytes = f->size - payload_start;

    Json j{text, text + header_bytes};
    std::vector<RawTensor> raw;
    std::set<std::string> names;
    bool ok = j.eat('{');
    if (ok && !j.eat('}')) {
        do {
            std::string name;
            if (!(ok = j.string(&name)))
                break;
            if (!(ok = j.eat(':'))) {
                j.invalid();
                break;
            }
            if (!names.insert(name).second) {
                ok = j.bad(MFH_DUPLICATE_NAME, "duplicate name");
                break;
            }
            if (name == "__metadata__") {
                if (!(ok = parse_metadata(j, &f->metadata)))
                    break;
            } else {
                RawTensor t;
                t.name = name;
                if (!(ok = parse_tensor(j, &t)))
                    break;
                raw.push_back(std::move(t));
            }
        } while (j.eat(','));
        if (ok && !j.eat('}'))
            ok = j.invalid();
    }
    if (!ok)
        return fail_s(j.status, j.message);
    j.space();
    if (j.p != j.end)
        return fail_s(MFH_INVALID_ARGUMENT, "safetensors header has trailing data");

    for (const RawTensor &r : raw) {
        if (r.name.empty() || r.name.size() > 1024)
            return fail_s(MFH_INVALID_ARGUMENT, "tensor name exceeds configured loader limit");
        if (r.shape.size() > 4)
            return fail_s(MFH_INVALID_SHAPE, "tensor rank exceeds configured loader limit");
        Tensor t;
        t.name = r.name;
        t.dtype = r.dtype;
        t.rank = uint32_t(r.shape.size());
        uint64_t elements = 1;
        for (uint32_t i = 0; i < t.rank; ++i) {
            t.dims[i] = r.shape[i];
            if (r.shape[i] && elements > UINT64_MAX / r.shape[i])
                return fail_s(MFH_OVERFLOW, "element count overflows u64");
            elements *= r.shape[i];
        }
        t.elements = elements;
        if (r.stop < r.start)
            return fail_s(MFH_INVALID_LAYOUT, "tensor data offsets are reversed");
        const uint64_t len = r.stop - r.start;
        const uint64_t width = dtype_width(r.dtype);
        if (elements > UINT64_MAX / width)
            return fail_s(MFH_OVERFLOW, "tensor source bytes overflow u64");
        if (len != elements * width)
            return fail_s(MFH_INVALID_LAYOUT,
                          "tensor source range differs from shape and storage dtype");
        if (r.stop > payload_bytes)
            return fail_s(MFH_OUT_OF_BOUNDS, "tensor source range exceeds payload bytes");
        t.offset = payload_start + r.start;
        t.bytes = len;
        f->by_name[t.name] = f->tensors.size();
        f->tensors.push_back(std::move(t));
    }
    // validate_payload_coverage (header.rs:135-160).
    std::vector<const Tensor *> ordered;
    for (const Tensor &t : f->tensors)
        ordered.push_back(&t);
    std::sort(ordered.begin(), ordered.end(), [](const Tensor *a, const Tensor *b) {
        return a->offset != b->offset ? a->offset < b->offset : a->bytes < b->bytes;
    });
    uint64_t expected = payload_start;
    for (const Tensor *t : ordered) {
        if (t->offset != expected)
            return fail_s(MFH_INVALID_LAYOUT,
                          "tensor ranges do not cover payload without holes or overlap");
        expected = t->offset + t->bytes;
    }
    if (expected != payload_start + payload_bytes)
        return fail_s(MFH_INVALID_LAYOUT, "tensor ranges do not cover complete payload");
    return MFH_OK;
}

// f16_to_f32 (loader.rs:408-421), for the host-side finite check.
bool f16_finite(uint16_t bits)
{
    return ((bits >> 10) & 0x1F) != 31;
}

float bf16_to_f32(uint16_t bits)
{
    const uint32_t w = uint32_t(bits) << 16;
    float v;
    std::memcpy(&v, &w, 4);
    return v;
}

}  // namespace

extern "C" {

const char *mfs_error(void)
{
    return g_error;
}

mfh_status mfs_open(const char *path, uint64_t max_header_bytes, mfs_file **out)
{
    if (!path || !out)
        return fail_s(MFH_INVALID_ARGUMENT, "path or output pointer is null");
    *out = nullptr;
    auto f = std::make_unique<mfs_file>();
    f->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (f->fd < 0)
        return fail_s(MFH_INVALID_ARGUMENT, "safetensors file cannot be opened");
    struct stat st;
    if (fstat(f->fd, &st) != 0 || st.st_size < 0)
        return fail_s(MFH_INVALID_ARGUMENT, "safetensors prefix is unreadable");
    f->size = uint64_t(st.st_size);
    if (f->size) {
        void *m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
        if (m == MAP_FAILED)
            return fail_s(MFH_RESOURCE_LIMIT, "safetensors file cannot be mapped");
        f->map = static_cast<const uint8_t *>(m);
    }
    mfh_status s = parse_file(f.get(), max_header_bytes ? max_header_bytes : (uint64_t(1) << 27));
    if (s)
        return s;
    *out = f.release();
    return MFH_OK;
}

void mfs_close(mfs_file *file)
{
    delete file;
}

size_t mfs_tensor_count(const mfs_file *file)
{
    return file ? file->tensors.size() : 0;
}

const char *mfs_tensor_name(const mfs_file *file, size_t index)
{
    if (!file || index >= file->tensors.size())
        return nullptr;
    return file->tensors[index].name.c_str();
}

mfh_status mfs_tensor_info(const mfs_file *file, const char *name, mfs_dtype *dtype,
                           uint32_t *rank, uint64_t *dims)
{
    if (!file || !name)
        return fail_s(MFH_INVALID_ARGUMENT, "file or name pointer is null");
    const Tensor *t = file->find(name);
    if (!t)
        return fail_s(MFH_MISSING_REQUIRED_TENSOR, "required tensor is missing");
    if (dtype)
        *dtype = t->dtype;
    if (rank)
        *rank = t->rank;
    if (dims)
        for (uint32_t i = 0; i < t->rank; ++i)
            dims[i] = t->dims[i];
    return MFH_OK;
}

const char *mfs_metadata(const mfs_file *file, const char *key)
{
    if (!file || !key)
        return nullptr;
    auto it = file->metadata.find(key);
    return it == file->metadata.end() ? nullptr : it->second.c_str();
}

mfh_status mfs_matmul_scheme(const mfs_file *file, const char *name, mfs_scheme *out)
{
    if (!file || !name || !out)
        return fail_s(MFH_INVALID_ARGUMENT, "null argument");
    // format_from_marker (weights.rs:74-85).
    mfs_scheme bundle = MFS_SCHEME_DENSE;
    bool mixed = false;
    auto format = file->metadata.find("format");
    if (format != file->metadata.end()) {
        const std::string &m = format->second;
        if (m == "pt")
            bundle = MFS_SCHEME_DENSE;
        else if (m == "minifield.ternary.v1")
            bundle = MFS_SCHEME_TERNARY;
        else if (m == "minifield.nf4.v1")
            bundle = MFS_SCHEME_NF4;
        else if (m == "minifield.int8.v1")
            bundle = MFS_SCHEME_INT8;
        else if (m == "minifield.mixed.v1")
            mixed = true;
        else
            return fail_s(MFH_UNSUPPORTED, "unrecognized LFM2 weight format");
    }
    // parse_lfm2_tensor_quantization (weights.rs:92-135): a JSON-encoded map
    // in the metadata, every entry of which must name a known level (a
    // string) before any is used.  A repeated name keeps its last entry, as
    // a JSON map deserialized into serde_json::Map does.
    auto map = file->metadata.find("tensor_quantization");
    if (map != file->metadata.end()) {
        const std::string &text = map->second;
        Json j{text.data(), text.data() + text.size()};
        std::map<std::string, mfs_scheme> levels;
        bool level_error = false;
        bool ok = j.eat('{');
        if (ok && !j.eat('}')) {
            do {
                std::string key, level;
                bool is_string = false;
                if (!(ok = j.string(&key) && j.eat(':') && j.value(&level, &is_string)))
                    break;
                mfs_scheme scheme = MFS_SCHEME_DENSE;
                if (is_string && level == "ternary-v1")
                    scheme = MFS_SCHEME_TERNARY;
                else if (is_string && level == "nf4-v1")
                    scheme = MFS_SCHEME_NF4;
                else if (is_string && level == "int8-v1")
                    scheme = MFS_SCHEME_INT8;
                else if (!(is_string && (level == "dense" || level == "bf16" || level == "f16" ||
                                         level == "f32")))
                    level_error = true;
                levels[key] = scheme;
            } while (j.eat(','));
            ok = ok && j.eat('}');
        }
        if (!ok || (j.space(), j.p != j.end))
            return fail_s(MFH_INVALID_ARGUMENT, "tensor_quantization metadata is not valid JSON");
        if (level_error)
            return fail_s(MFH_INVALID_ARGUMENT,
                          "tensor_quantization level must be ternary-v1, nf4-v1, int8-v1, or a "
                          "dense dtype");
        auto it = levels.find(name);
        if (it != levels.end()) {
            *out = it->second;
            return MFH_OK;
        }
    }
    *out = mixed ? MFS_SCHEME_DENSE : bundle;
    return MFH_OK;
}

mfh_status mfs_upload_packed(mfh_ctx *ctx, const mfs_file *file, const char *base,
                             mfh_alloc_class cls, mfh_buf **codes_out, mfh_buf **scales_out)
{
    if (!ctx || !file || !base || !codes_out || !scales_out)
        return fail_s(MFH_INVALID_ARGUMENT, "null argument");
    *codes_out = *scales_out = nullptr;
    const std::string b(base);
    const Tensor *codes = file->find(b + ".codes");
    const Tensor *scales = file->find(b + ".scales");
    if (!codes || !scales)
        return fail_s(MFH_MISSING_REQUIRED_TENSOR, "required tensor is missing");
    if (codes->dtype != MFS_U8 || scales->dtype != MFS_F16)
        return fail_s(MFH_INVALID_DTYPE,
                      "packed streams are U8 codes and F16 scales");
    if (codes->rank != 2 || scales->rank != 2 || codes->dims[0] != scales->dims[0])
        return fail_s(MFH_INVALID_SHAPE, "packed weight requirement must be rank two");
    const uint8_t *cbytes = file->map + codes->offset;
    const uint16_t *sbits = reinterpret_cast<const uint16_t *>(file->map + scales->offset);
    // An INT8 stream (one code per weight) must not hold the reserved -128
    // (loader.rs:1154-1162); checked before anything is uploaded.
    if (scales->dims[1] <= UINT64_MAX / 128 && codes->dims[1] == scales->dims[1] * 128 &&
        codes->bytes && std::memchr(cbytes, 0x80, codes->bytes))
        return fail_s(MFH_INVALID_ARGUMENT, "INT8 -128 code is reserved");
    if (scales->offset % 2)
        return fail_s(MFH_INVALID_LAYOUT, "F16 scale stream is not 2-byte aligned");
    for (uint64_t i = 0; i < scales->elements; ++i)
        if (!f16_finite(sbits[i]))
            return fail_s(MFH_BACKEND_FAILURE, "decoded model tensor contains non-finite values");
    mfh_buf *c = nullptr, *s = nullptr;
    mfh_status st = mfh_upload_u8(ctx, codes->dims, 2, cbytes, codes->bytes, cls, &c);
    if (!st)
        st = mfh::upload_scales_f16(ctx, scales->dims, sbits, scales->elements, cls, &s);
    if (!st)
        st = mfh_prepare_packed(ctx, c, s);
    if (st) {
        g_error = mfh_last_error(ctx);
        mfh_release(c);
        mfh_release(s);
        return st;
    }
    *codes_out = c;
    *scales_out = s;
    return MFH_OK;
}

mfh_status mfs_upload_dense(mfh_ctx *ctx, const mfs_file *file, const char *name,
                            mfh_alloc_class cls, mfh_buf **out)
{
    if (!ctx || !file || !name || !out)
        return fail_s(MFH_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    const Tensor *t = file->find(name);
    if (!t)
        return fail_s(MFH_MISSING_REQUIRED_TENSOR, "required tensor is missing");
    if (t->dtype == MFS_U8)
        return fail_s(MFH_INVALID_DTYPE,
                      "u8 packed payloads upload byte-exact and never decode to f32");
    std::vector<float> values(t->elements);
    const uint8_t *src = file->map + t->offset;
    for (uint64_t i = 0; i < t->elements; ++i) {
        float v = 0.0f;
        if (t->dtype == MFS_F32) {
            std::memcpy(&v, src + 4 * i, 4);
        } else {
            uint16_t bits;
            std::memcpy(&bits, src + 2 * i, 2);
            v = t->dtype == MFS_BF16 ? bf16_to_f32(bits) : mfc_f16_to_f32(bits);
        }
        if (!std::isfinite(v))
            return fail_s(MFH_BACKEND_FAILURE, "decoded model tensor contains non-finite values");
        values[i] = v;
    }
    mfh_status st = mfh_upload_f32(ctx, t->dims, t->rank, values.data(), values.size(), cls, out);
    if (st)
        g_error = mfh_last_error(ctx);
    return st;
}

}  // extern "C"

