// NXF weight files: reader and writer of the reference's on-disk format
// (nexus/src/format/nxf.h, nxf_reader.cpp, nxf_writer.cpp), with every chunk
// checksum computed and verified on the GPU (k_xxh32).
//
// Layout of a file (all offsets 16 KiB aligned):
//   [0, 64)            header: magic "NXF1", version 1, flags, manifest and
//                      tensor-index (offset, size), data offset 16384, file size
//   [16384, ...)       chunk data, each chunk at the next 16 KiB boundary
//   tensor index       per tensor: u32 name length, name, u32 ndim, i64 shape[ndim],
//                      u8 dtype, u32 chunk count, 24-byte chunk descriptors
//   manifest           flat JSON object
//   padding to 16 KiB
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstddef>
#include <cstring>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/nexus_nxf.h"
#include "nx_internal.h"
#include "nx_kernels.h"

namespace {

constexpr uint32_t kMagic = 0x3146584Eu;  // "NXF1" little-endian
constexpr uint16_t kVersion = 1;
constexpr uint64_t kAlign = 16384;

struct FileHeader {
    uint32_t magic;
    uint16_t version, flags;
    uint64_t manifest_offset, manifest_size, tensor_index_offset, tensor_index_size, data_offset, total_file_size;
    uint8_t reserved[8];
};
static_assert(sizeof(FileHeader) == 64, "header is 64 bytes on disk");

struct DiskChunk {
    uint64_t file_offset;
    uint32_t compressed_size, decompressed_size, checksum;
    uint8_t codec, group_size, reserved[2];
};
static_assert(sizeof(DiskChunk) == 24, "chunk descriptor is 24 bytes on disk");

struct Tensor {
    std::string name;
    std::vector<int64_t> shape;
    uint8_t dtype = 0;
    std::vector<DiskChunk> chunks;
};

thread_local std::string g_err;

nx_status ferr(nx_status code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

nx_status ctx_err(nx_ctx* ctx, nx_status code) {
    g_err = ctx ? ctx->err : std::string("no context");
    return code;
}

uint64_t align_up(uint64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

bool pread_all(int fd, void* dst, size_t n, uint64_t off) {
    auto* p = static_cast<uint8_t*>(dst);
    while (n > 0) {
        const ssize_t r = ::pread(fd, p, n, (off_t)off);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        p += r;
        n -= (size_t)r;
        off += (uint64_t)r;
    }
    return true;
}

bool pwrite_all(int fd, const void* src, size_t n, uint64_t off) {
    const auto* p = static_cast<const uint8_t*>(src);
    while (n > 0) {
        const ssize_t r = ::pwrite(fd, p, n, (off_t)off);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        p += r;
        n -= (size_t)r;
        off += (uint64_t)r;
    }
    return true;
}

// ------------------------------------------------------------ manifest --
// The manifest is a flat JSON object of string and number values
// (nxf_writer.cpp:93-129 writes it, nxf_reader.cpp:125-182 reads it).
void json_escape_into(std::string& out, const char* s) {
    for (; *s; ++s) {
        switch (*s) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '\n': out += "\\n"; break;
            case '\t': out += "\\t"; break;
            default: out += *s;
        }
    }
}

// Same keys, order and number formats as the reference writer, so a
// manifest round-trips to identical bytes.
std::string manifest_json(const nx_nxf_manifest& m) {
    std::string s = "{\n  \"architecture\": \"";
    json_escape_into(s, m.architecture);
    s += "\",\n  \"name\": \"";
    json_escape_into(s, m.name);
    s += "\",\n";
    char buf[128];
    auto field = [&](const char* key, const char* fmt, auto v, bool last = false) {
        snprintf(buf, sizeof(buf), fmt, v);
        s += "  \"";
        s += key;
        s += "\": ";
        s += buf;
        s += last ? "\n" : ",\n";
    };
    field("num_layers", "%u", m.num_layers);
    field("hidden_dim", "%u", m.hidden_dim);
    field("num_heads", "%u", m.num_heads);
    field("num_kv_heads", "%u", m.num_kv_heads);
    field("head_dim", "%u", m.head_dim);
    field("vocab_size", "%u", m.vocab_size);
    field("max_seq_len", "%u", m.max_seq_len);
    field("rope_theta", "%.1f", (double)m.rope_theta);
    field("rms_norm_eps", "%.10g", (double)m.rms_norm_eps);
    field("num_experts", "%u", m.num_experts);
    field("num_active_experts", "%u", m.num_active_experts);
    field("default_codec", "%u", (unsigned)m.default_codec);
    field("default_group_size", "%u", (unsigned)m.default_group_size, true);
    s += "}";
    return s;
}

// A manifest value: the NXF manifest holds only strings and numbers.
struct JsonValue {
    bool is_str = false;
    std::string str;
    double num = 0.0;
};

// Tokenizer of one flat JSON object, {"key": value, ...} with string or
// number values, into (key, value) pairs in file order.  Standard JSON
// (RFC 8259) for those two kinds, with the reference reader's leniencies
// (format/nxf_reader.cpp:75-180) where files of the reference writer need
// them: raw control bytes inside strings (its escaper, nxf_writer.cpp:76-89,
// writes \r and the other control bytes unescaped) and anything after the
// closing brace.  Nested objects, arrays, literals and trailing commas are
// rejected.
class FlatJson {
  public:
    FlatJson(const char* data, size_t len) : s_(data), n_(len) {}

    bool parse(std::vector<std::pair<std::string, JsonValue>>& out) {
        skip_ws();
        if (!eat('{')) return false;
        skip_ws();
        if (eat('}')) return at_end();
        for (;;) {
            std::pair<std::string, JsonValue> kv;
            skip_ws();
            if (!string(kv.first)) return false;
            skip_ws();
            if (!eat(':')) return false;
            skip_ws();
            if (i_ < n_ && s_[i_] == '"') {
                kv.second.is_str = true;
                if (!string(kv.second.str)) return false;
            } else if (!number(kv.second.num)) {
                return false;
            }
            out.push_back(std::move(kv));
            skip_ws();
            if (eat('}')) return at_end();
            if (!eat(',')) return false;
        }
    }

  private:
    const char* s_;
    size_t n_, i_ = 0;

    void skip_ws() {
        while (i_ < n_ && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) ++i_;
    }
    bool eat(char c) {
        if (i_ < n_ && s_[i_] == c) {
            ++i_;
            return true;
        }
        return false;
    }
    // the object is complete at its closing brace; what follows is ignored
    bool at_end() { return true; }
    static int hex(char c) {
        if (c >= '0' && c <= '9') return c - '0';
        if (c >= 'a' && c <= 'f') return c - 'a' + 10;
        if (c >= 'A' && c <= 'F') return c - 'A' + 10;
        return -1;
    }
    // "..." with the JSON escapes; \uXXXX below 0x80 becomes that byte,
    // other code points are written as UTF-8.
    bool string(std::string& out) {
        if (!eat('"')) return false;
        while (i_ < n_) {
            const char c = s_[i_++];
            if (c == '"') return true;
            if (c != '\\') {  // raw bytes, control bytes included, are taken as they are
                out += c;
                continue;
            }
            if (i_ >= n_) return false;
            const char e = s_[i_++];
            switch (e) {
                case '"': case '\\': case '/': out += e; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    if (i_ + 4 > n_) return false;
                    unsigned cp = 0;
                    for (int k = 0; k < 4; ++k) {
                        const int h = hex(s_[i_ + k]);
                        if (h < 0) return false;
                        cp = cp * 16 + (unsigned)h;
                    }
                    i_ += 4;
                    if (cp < 0x80) {
                        out += (char)cp;
                    } else if (cp < 0x800) {
                        out += (char)(0xC0 | (cp >> 6));
                        out += (char)(0x80 | (cp & 0x3F));
                    } else {
                        out += (char)(0xE0 | (cp >> 12));
                        out += (char)(0x80 | ((cp >> 6) & 0x3F));
                        out += (char)(0x80 | (cp & 0x3F));
                    }
                    break;
                }
                default: return false;
            }
        }
        return false;
    }
    // -?(0|[1-9][0-9]*)(.[0-9]+)?([eE][+-]?[0-9]+)?, converted by strtod
    bool number(double& v) {
        const size_t b = i_;
        auto digits = [&]() {
            const size_t d = i_;
            while (i_ < n_ && s_[i_] >= '0' && s_[i_] <= '9') ++i_;
            return i_ > d;
        };
        eat('-');
        if (eat('0')) {
        } else if (!digits()) {
            return false;
        }
        if (eat('.') && !digits()) return false;
        if (i_ < n_ && (s_[i_] == 'e' || s_[i_] == 'E')) {
            ++i_;
            if (!eat('+')) eat('-');
            if (!digits()) return false;
        }
        const std::string text(s_ + b, i_ - b);
        v = strtod(text.c_str(), nullptr);
        return true;
    }
};

// The manifest fields (nxf.h:73-96) and the range each must lie in.
enum class FieldKind { Text, U32, U8, F32 };
struct ManifestField {
    const char* key;
    FieldKind kind;
    size_t offset;
    size_t size;  // Text: capacity including the terminator
};
#define NX_MF(field, kind) {#field, FieldKind::kind, offsetof(nx_nxf_manifest, field), sizeof(nx_nxf_manifest::field)}
const ManifestField kManifestFields[] = {
    NX_MF(architecture, Text), NX_MF(name, Text), NX_MF(num_layers, U32), NX_MF(hidden_dim, U32),
    NX_MF(num_heads, U32), NX_MF(num_kv_heads, U32), NX_MF(head_dim, U32), NX_MF(vocab_size, U32),
    NX_MF(max_seq_len, U32), NX_MF(rope_theta, F32), NX_MF(rms_norm_eps, F32), NX_MF(num_experts, U32),
    NX_MF(num_active_experts, U32), NX_MF(default_codec, U8), NX_MF(default_group_size, U8),
};
#undef NX_MF

// Store one value into its field: text into a string field (truncated to
// the field), a number into a numeric field (default_codec also as quoted
// text).  Integer fields take integral values in [0, 2^32 - 1] (bytes:
// [0, 255]); floats any finite value that rounds to a finite float.
// Anything else rejects the manifest.
bool assign_field(nx_nxf_manifest& m, const ManifestField& f, const JsonValue& v) {
    char* dst = reinterpret_cast<char*>(&m) + f.offset;
    if (f.kind == FieldKind::Text) {
        if (!v.is_str) return false;
        const size_t k = std::min(f.size - 1, v.str.size());
        memcpy(dst, v.str.data(), k);
        dst[k] = 0;
        return true;
    }
    double num = v.num;
    if (v.is_str) {
        // a quoted default_codec is read as the reference reader reads it
        // (atoi of the text, format/nxf_reader.cpp:162): leading spaces, an
        // optional sign and the digits that follow; no digits read as 0
        if (strcmp(f.key, "default_codec") != 0) return false;
        const char* t = v.str.c_str();
        while (*t == ' ' || (*t >= '\t' && *t <= '\r')) ++t;
        const bool neg = *t == '-';
        if (*t == '-' || *t == '+') ++t;
        num = 0.0;
        for (int k = 0; *t >= '0' && *t <= '9' && k < 12; ++t, ++k) num = num * 10.0 + (*t - '0');
        if (neg) num = -num;
    }
    if (!std::isfinite(num)) return false;
    if (f.kind == FieldKind::F32) {
        const float x = (float)num;
        if (!std::isfinite(x)) return false;
        memcpy(dst, &x, sizeof(x));
        return true;
    }
    const double hi = f.kind == FieldKind::U8 ? 255.0 : 4294967295.0;
    if (num < 0.0 || num > hi || num != std::floor(num)) return false;
    if (f.kind == FieldKind::U8) {
        const uint8_t x = (uint8_t)num;
        memcpy(dst, &x, 1);
    } else {
        const uint32_t x = (uint32_t)num;
        memcpy(dst, &x, 4);
    }
    return true;
}

// Manifest JSON -> struct.  Keys outside the format are ignored (as the
// reference reader does); a known key with the wrong kind or an
// out-of-range value fails the open.
bool parse_manifest(const char* data, size_t len, nx_nxf_manifest& m) {
    std::vector<std::pair<std::string, JsonValue>> kvs;
    if (!FlatJson(data, len).parse(kvs)) return false;
    for (const auto& kv : kvs)
        for (const ManifestField& f : kManifestFields)
            if (kv.first == f.key && !assign_field(m, f, kv.second)) return false;
    return true;
}

// ---------------------------------------------------------------- index --
std::vector<uint8_t> index_blob(const std::vector<Tensor>& ts) {
    std::vector<uint8_t> b;
    auto put = [&](const void* p, size_t n) {
        const auto* c = static_cast<const uint8_t*>(p);
        b.insert(b.end(), c, c + n);
    };
    for (const Tensor& t : ts) {
        const uint32_t nl = (uint32_t)t.name.size(), nd = (uint32_t)t.shape.size(), nc = (uint32_t)t.chunks.size();
        put(&nl, 4);
        put(t.name.data(), nl);
        put(&nd, 4);
        put(t.shape.data(), 8 * (size_t)nd);
        put(&t.dtype, 1);
        put(&nc, 4);
        put(t.chunks.data(), sizeof(DiskChunk) * (size_t)nc);
    }
    return b;
}

bool parse_index(const uint8_t* p, const uint8_t* end, std::vector<Tensor>& out) {
    auto get = [&](void* dst, size_t n) {
        if ((size_t)(end - p) < n) return false;
        memcpy(dst, p, n);
        p += n;
        return true;
    };
    while (p < end) {
        Tensor t;
        uint32_t nl = 0, nd = 0, nc = 0;
        if (!get(&nl, 4)) return true;  // a trailing fragment shorter than a length ends the index
        if ((size_t)(end - p) < nl) return false;
        t.name.assign(reinterpret_cast<const char*>(p), nl);
        p += nl;
        if (!get(&nd, 4) || nd > 64) return false;
        t.shape.resize(nd);
        if (!get(t.shape.data(), 8 * (size_t)nd)) return false;
        if (!get(&t.dtype, 1) || !get(&nc, 4)) return false;
        if ((size_t)(end - p) / sizeof(DiskChunk) < nc) return false;
        t.chunks.resize(nc);
        if (!get(t.chunks.data(), sizeof(DiskChunk) * (size_t)nc)) return false;
        out.push_back(std::move(t));
    }
    return true;
}

// -------------------------------------------------------- device hashing --
// Hash n ranges of device memory at data (range offsets relative to data)
// into hashes_dev[slot]; ranges are sorted by length so each wavefront's
// quads loop about equally long.
struct HashScratch {
    nx::HashRange* ranges = nullptr;
    uint32_t* hashes = nullptr;
    size_t cap = 0;
    ~HashScratch() {
        if (ranges) (void)hipFree(ranges);
        if (hashes) (void)hipFree(hashes);
    }
    nx_status ensure(nx_ctx* ctx, size_t n) {
        if (n <= cap) return NX_OK;
        if (ranges) (void)hipFree(ranges);
        if (hashes) (void)hipFree(hashes);
        ranges = nullptr;
        hashes = nullptr;
        cap = 0;
        NX_HIP(ctx, hipMalloc(reinterpret_cast<void**>(&ranges), n * sizeof(nx::HashRange)));
        NX_HIP(ctx, hipMalloc(reinterpret_cast<void**>(&hashes), n * sizeof(uint32_t)));
        cap = n;
        return NX_OK;
    }
};

void sort_ranges(std::vector<nx::HashRange>& r) {
    std::stable_sort(r.begin(), r.end(), [](const nx::HashRange& a, const nx::HashRange& b) { return a.len > b.len; });
}

}  // namespace

struct nx_nxf {
    int fd = -1;
    FileHeader hdr{};
    nx_nxf_manifest man{};
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int> by_name;
    std::vector<std::pair<void*, size_t>> maps;
};

struct nx_nxf_writer {
    nx_ctx* ctx = nullptr;
    int fd = -1;
    uint64_t pos = 0;
    nx_nxf_manifest man{};
    std::vector<Tensor> tensors;
    Tensor cur;
    bool in_tensor = false;
    // chunks of the current tensor waiting for their checksum: copies in
    // pinned host memory, hashed on the device in one launch per flush
    uint8_t* stage = nullptr;
    size_t stage_cap = 0, stage_used = 0;
    std::vector<std::pair<int, size_t>> pending;  // (chunk index in cur, stage offset)
    uint8_t* dstage = nullptr;
    size_t dstage_cap = 0;
    HashScratch hs;
    ~nx_nxf_writer() {
        if (stage) (void)hipHostFree(stage);
        if (dstage) (void)hipFree(dstage);
        if (fd >= 0) ::close(fd);
    }
};

namespace {

// Hash the pending chunks of the current tensor on the device and store
// their checksums in its descriptors.
nx_status writer_flush(nx_nxf_writer* w) {
    if (w->pending.empty()) return NX_OK;
    nx_ctx* ctx = w->ctx;
    if (w->stage_used > w->dstage_cap) {
        if (w->dstage) (void)hipFree(w->dstage);
        w->dstage = nullptr;
        w->dstage_cap = 0;
        if (hipMalloc(reinterpret_cast<void**>(&w->dstage), w->stage_used) != hipSuccess)
            return ferr(NX_ERR_OOM, "nxf writer: device staging of %zu bytes", w->stage_used);
        w->dstage_cap = w->stage_used;
    }
    std::vector<nx::HashRange> r(w->pending.size());
    for (size_t i = 0; i < w->pending.size(); ++i)
        r[i] = nx::HashRange{w->pending[i].second, w->cur.chunks[(size_t)w->pending[i].first].compressed_size,
                             (uint32_t)i};
    sort_ranges(r);
    if (w->hs.ensure(ctx, r.size()) != NX_OK) return ctx_err(ctx, NX_ERR_HIP);
    hipStream_t st = ctx->stream;
    std::vector<uint32_t> h(r.size());
    if (hipMemcpyAsync(w->dstage, w->stage, w->stage_used, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(w->hs.ranges, r.data(), r.size() * sizeof(nx::HashRange), hipMemcpyHostToDevice, st) !=
            hipSuccess ||
        nx::xxh32_launch(w->dstage, w->hs.ranges, (int)r.size(), w->hs.hashes, st) != hipSuccess ||
        hipMemcpyAsync(h.data(), w->hs.hashes, h.size() * 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return ferr(NX_ERR_HIP, "nxf writer: chunk hashing on the device failed");
    for (size_t i = 0; i < w->pending.size(); ++i) w->cur.chunks[(size_t)w->pending[i].first].checksum = h[i];
    w->pending.clear();
    w->stage_used = 0;
    return NX_OK;
}

nx_status writer_pad(nx_nxf_writer* w) {
    const uint64_t target = align_up(w->pos);
    if (target == w->pos) return NX_OK;
    static const uint8_t zeros[kAlign] = {};
    if (!pwrite_all(w->fd, zeros, (size_t)(target - w->pos), w->pos))
        return ferr(NX_ERR_IO, "nxf writer: padding write failed: %s", strerror(errno));
    w->pos = target;
    return NX_OK;
}

nx_status writer_put(nx_nxf_writer* w, const void* data, size_t n) {
    if (!pwrite_all(w->fd, data, n, w->pos)) return ferr(NX_ERR_IO, "nxf writer: write failed: %s", strerror(errno));
    w->pos += n;
    return NX_OK;
}

}  // namespace

extern "C" {

const char* nx_nxf_error(void) { return g_err.c_str(); }

// ------------------------------------------------------------------ reader --
nx_status nx_nxf_open(const char* path, nx_nxf** out) {
    if (!path || !out) return ferr(NX_ERR_INVALID, "nx_nxf_open: null argument");
    *out = nullptr;
    nx_nxf* r = new nx_nxf();
    auto bad = [&](nx_status code, const char* fmt, const char* a = "", unsigned long long x = 0,
                   unsigned long long y = 0) {
        ferr(code, fmt, a, x, y);
        nx_nxf_close(r);
        return code;
    };
    r->fd = ::open(path, O_RDONLY);
    if (r->fd < 0) return bad(NX_ERR_IO, "nxf: cannot open '%s'", path);
    if (!pread_all(r->fd, &r->hdr, sizeof(FileHeader), 0)) return bad(NX_ERR_IO, "nxf: short header in '%s'", path);
    if (r->hdr.magic != kMagic)
        return bad(NX_ERR_IO, "nxf: bad magic in '%s' (0x%08llX)", path, (unsigned long long)r->hdr.magic);
    if (r->hdr.version != kVersion)
        return bad(NX_ERR_IO, "nxf: unsupported version in '%s' (%llu)", path, (unsigned long long)r->hdr.version);
    struct stat st;
    if (fstat(r->fd, &st) != 0 || (uint64_t)st.st_size != r->hdr.total_file_size)
        return bad(NX_ERR_IO, "nxf: file size of '%s' (%llu) differs from the header's (%llu)", path,
                   (unsigned long long)st.st_size, (unsigned long long)r->hdr.total_file_size);
    const uint64_t fsz = r->hdr.total_file_size;
    auto inside = [&](uint64_t off, uint64_t n) { return off <= fsz && n <= fsz - off; };
    if (r->hdr.manifest_size > 0) {
        if (!inside(r->hdr.manifest_offset, r->hdr.manifest_size))
            return bad(NX_ERR_IO, "nxf: manifest of '%s' lies outside the file", path);
        std::vector<char> buf(r->hdr.manifest_size);
        if (!pread_all(r->fd, buf.data(), buf.size(), r->hdr.manifest_offset) ||
            !parse_manifest(buf.data(), buf.size(), r->man))
            return bad(NX_ERR_IO, "nxf: malformed manifest in '%s'", path);
    }
    if (r->hdr.tensor_index_size > 0) {
        if (!inside(r->hdr.tensor_index_offset, r->hdr.tensor_index_size))
            return bad(NX_ERR_IO, "nxf: tensor index of '%s' lies outside the file", path);
        std::vector<uint8_t> buf(r->hdr.tensor_index_size);
        if (!pread_all(r->fd, buf.data(), buf.size(), r->hdr.tensor_index_offset) ||
            !parse_index(buf.data(), buf.data() + buf.size(), r->tensors))
            return bad(NX_ERR_IO, "nxf: truncated tensor index in '%s'", path);
    }
    for (size_t i = 0; i < r->tensors.size(); ++i) {
        for (const DiskChunk& c : r->tensors[i].chunks)
            if (!inside(c.file_offset, c.compressed_size))
                return bad(NX_ERR_IO, "nxf: a chunk of '%s' lies outside the file", r->tensors[i].name.c_str());
        r->by_name.emplace(r->tensors[i].name, (int)i);  // the first of equal names wins
    }
    *out = r;
    return NX_OK;
}

nx_status nx_nxf_close(nx_nxf* r) {
    if (!r) return ferr(NX_ERR_INVALID, "nx_nxf_close: null reader");
    for (auto& m : r->maps) ::munmap(m.first, m.second);
    if (r->fd >= 0) ::close(r->fd);
    delete r;
    return NX_OK;
}

nx_status nx_nxf_get_manifest(nx_nxf* r, nx_nxf_manifest* out) {
    if (!r || !out) return ferr(NX_ERR_INVALID, "nx_nxf_get_manifest: null argument");
    *out = r->man;
    return NX_OK;
}

nx_status nx_nxf_num_tensors(nx_nxf* r, int* n) {
    if (!r || !n) return ferr(NX_ERR_INVALID, "nx_nxf_num_tensors: null argument");
    *n = (int)r->tensors.size();
    return NX_OK;
}

nx_status nx_nxf_tensor_at(nx_nxf* r, int i, nx_nxf_tensor* out) {
    if (!r || !out) return ferr(NX_ERR_INVALID, "nx_nxf_tensor_at: null argument");
    if (i < 0 || i >= (int)r->tensors.size()) return ferr(NX_ERR_INVALID, "nx_nxf_tensor_at: no tensor %d", i);
    const Tensor& t = r->tensors[(size_t)i];
    if (t.shape.size() > 8) return ferr(NX_ERR_UNSUPPORTED, "tensor '%s' has more than 8 dimensions", t.name.c_str());
    memset(out, 0, sizeof(*out));
    out->name = t.name.c_str();
    out->ndim = (int)t.shape.size();
    for (size_t d = 0; d < t.shape.size(); ++d) out->shape[d] = t.shape[d];
    out->dtype = t.dtype;
    out->num_chunks = (int)t.chunks.size();
    for (const DiskChunk& c : t.chunks) {
        out->compressed_bytes += c.compressed_size;
        out->decompressed_bytes += c.decompressed_size;
    }
    return NX_OK;
}

nx_status nx_nxf_find(nx_nxf* r, const char* name, int* index) {
    if (!r || !name || !index) return ferr(NX_ERR_INVALID, "nx_nxf_find: null argument");
    auto it = r->by_name.find(name);
    *index = it == r->by_name.end() ? -1 : it->second;
    return NX_OK;
}

nx_status nx_nxf_chunk_at(nx_nxf* r, int tensor, int chunk, nx_nxf_chunk* out) {
    if (!r || !out) return ferr(NX_ERR_INVALID, "nx_nxf_chunk_at: null argument");
    if (tensor < 0 || tensor >= (int)r->tensors.size() || chunk < 0 ||
        chunk >= (int)r->tensors[(size_t)tensor].chunks.size())
        return ferr(NX_ERR_INVALID, "nx_nxf_chunk_at: no chunk (%d, %d)", tensor, chunk);
    const DiskChunk& c = r->tensors[(size_t)tensor].chunks[(size_t)chunk];
    out->file_offset = c.file_offset;
    out->compressed_size = c.compressed_size;
    out->decompressed_size = c.decompressed_size;
    out->checksum = c.checksum;
    out->codec = c.codec;
    out->group_size = c.group_size;
    return NX_OK;
}

nx_status nx_nxf_map_chunk(nx_nxf* r, int tensor, int chunk, const void** data) {
    nx_nxf_chunk c;
    if (!data) return ferr(NX_ERR_INVALID, "nx_nxf_map_chunk: null argument");
    nx_status s = nx_nxf_chunk_at(r, tensor, chunk, &c);
    if (s != NX_OK) return s;
    const uint64_t base = c.file_offset / kAlign * kAlign, within = c.file_offset - base;
    const size_t len = (size_t)(within + c.compressed_size);
    if (len == 0) return ferr(NX_ERR_INVALID, "nx_nxf_map_chunk: empty chunk");
    void* p = ::mmap(nullptr, len, PROT_READ, MAP_PRIVATE, r->fd, (off_t)base);
    if (p == MAP_FAILED) return ferr(NX_ERR_IO, "nxf: mmap of %zu bytes failed: %s", len, strerror(errno));
    r->maps.emplace_back(p, len);
    *data = static_cast<const uint8_t*>(p) + within;
    return NX_OK;
}

nx_status nx_nxf_unmap_chunk(nx_nxf* r, const void* data) {
    if (!r || !data) return ferr(NX_ERR_INVALID, "nx_nxf_unmap_chunk: null argument");
    const auto* q = static_cast<const uint8_t*>(data);
    for (auto it = r->maps.begin(); it != r->maps.end(); ++it) {
        const auto* b = static_cast<const uint8_t*>(it->first);
        if (q >= b && q < b + it->second) {
            ::munmap(it->first, it->second);
            r->maps.erase(it);
            return NX_OK;
        }
    }
    return ferr(NX_ERR_INVALID, "nx_nxf_unmap_chunk: pointer was not mapped by this reader");
}

nx_status nx_nxf_read_chunk(nx_nxf* r, int tensor, int chunk, void* dst) {
    nx_nxf_chunk c;
    if (!dst) return ferr(NX_ERR_INVALID, "nx_nxf_read_chunk: null destination");
    nx_status s = nx_nxf_chunk_at(r, tensor, chunk, &c);
    if (s != NX_OK) return s;
    if (!pread_all(r->fd, dst, c.compressed_size, c.file_offset)) return ferr(NX_ERR_IO, "nxf: short chunk read");
    return NX_OK;
}

nx_status nx_nxf_verify(nx_ctx* ctx, nx_nxf* r, int* bad_tensor, int* bad_chunk, uint64_t* bytes) {
    if (!ctx || !r || !bad_tensor || !bad_chunk) return ferr(NX_ERR_INVALID, "nx_nxf_verify: null argument");
    *bad_tensor = *bad_chunk = -1;
    if (bytes) *bytes = 0;
    // every chunk in index order; batches of up to 256 MiB (or one chunk)
    struct Item {
        int t, c;
        const DiskChunk* d;
    };
    std::vector<Item> items;
    uint64_t total = 0, largest = 0;
    for (size_t t = 0; t < r->tensors.size(); ++t)
        for (size_t c = 0; c < r->tensors[t].chunks.size(); ++c) {
            const DiskChunk* d = &r->tensors[t].chunks[c];
            items.push_back({(int)t, (int)c, d});
            total += d->compressed_size;
            largest = std::max<uint64_t>(largest, d->compressed_size);
        }
    if (items.empty()) return NX_OK;
    auto stride = [](uint64_t n) { return (n + 255) / 256 * 256; };  // chunk starts 256-byte aligned
    const uint64_t cap = std::max<uint64_t>(std::min<uint64_t>(256ull << 20, stride(total)), stride(largest));
    uint8_t* host[2] = {nullptr, nullptr};
    uint8_t* dev = nullptr;
    hipEvent_t copied[2] = {nullptr, nullptr};
    HashScratch hs;
    nx_status status = NX_OK;
    hipStream_t st = ctx->stream;
    std::vector<uint32_t> got(items.size());
    do {
        if (hipHostMalloc(reinterpret_cast<void**>(&host[0]), cap, hipHostMallocDefault) != hipSuccess ||
            hipHostMalloc(reinterpret_cast<void**>(&host[1]), cap, hipHostMallocDefault) != hipSuccess ||
            hipMalloc(reinterpret_cast<void**>(&dev), cap) != hipSuccess ||
            hipEventCreateWithFlags(&copied[0], hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&copied[1], hipEventDisableTiming) != hipSuccess) {
            status = ferr(NX_ERR_OOM, "nx_nxf_verify: staging of %llu bytes", (unsigned long long)cap);
            break;
        }
        if (hs.ensure(ctx, items.size()) != NX_OK) {
            status = ctx_err(ctx, NX_ERR_HIP);
            break;
        }
        // batch i: read on the host into host[i & 1] while the device copies
        // and hashes batch i - 1 (same stream, so the device buffer is reused
        // only after the previous hash launch)
        size_t i0 = 0;
        int bi = 0;
        std::vector<std::vector<nx::HashRange>> ranges(2);
        while (i0 < items.size() && status == NX_OK) {
            uint8_t* hb = host[bi & 1];
            if (bi >= 2 && hipEventSynchronize(copied[bi & 1]) != hipSuccess) {
                status = ferr(NX_ERR_HIP, "nx_nxf_verify: event wait failed");
                break;
            }
            std::vector<nx::HashRange>& rg = ranges[bi & 1];
            rg.clear();
            uint64_t used = 0;
            size_t i = i0;
            for (; i < items.size(); ++i) {
                const uint64_t n = items[i].d->compressed_size;
                if (used + n > cap) break;
                if (!pread_all(r->fd, hb + used, (size_t)n, items[i].d->file_offset)) {
                    status = ferr(NX_ERR_IO, "nxf: short read of a chunk of '%s'", r->tensors[(size_t)items[i].t].name.c_str());
                    break;
                }
                rg.push_back(nx::HashRange{used, (uint32_t)n, (uint32_t)i});
                used = stride(used + n);
            }
            if (status != NX_OK) break;
            sort_ranges(rg);
            // the range table is copied from pageable memory: the copy is
            // complete when hipMemcpyAsync returns
            if (hipMemcpyAsync(dev, hb, (size_t)std::min(used, cap), hipMemcpyHostToDevice, st) != hipSuccess ||
                hipEventRecord(copied[bi & 1], st) != hipSuccess ||
                hipMemcpy(hs.ranges + i0, rg.data(), rg.size() * sizeof(nx::HashRange), hipMemcpyHostToDevice) != hipSuccess ||
                nx::xxh32_launch(dev, hs.ranges + i0, (int)rg.size(), hs.hashes, st) != hipSuccess) {
                status = ferr(NX_ERR_HIP, "nx_nxf_verify: upload or hash launch failed");
                break;
            }
            i0 = i;
            ++bi;
        }
        if (status != NX_OK) break;
        if (hipMemcpyAsync(got.data(), hs.hashes, got.size() * 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess) {
            status = ferr(NX_ERR_HIP, "nx_nxf_verify: reading the hashes failed");
            break;
        }
        for (size_t i = 0; i < items.size(); ++i)
            if (got[i] != items[i].d->checksum) {
                *bad_tensor = items[i].t;
                *bad_chunk = items[i].c;
                status = ferr(NX_ERR_CHECKSUM, "nxf: checksum mismatch in chunk %d of '%s' (stored %08x, data %08x)",
                              items[i].c, r->tensors[(size_t)items[i].t].name.c_str(), items[i].d->checksum, got[i]);
                break;
            }
        if (status == NX_OK && bytes) *bytes = total;
    } while (false);
    (void)hipStreamSynchronize(st);
    for (int k = 0; k < 2; ++k) {
        if (host[k]) (void)hipHostFree(host[k]);
        if (copied[k]) (void)hipEventDestroy(copied[k]);
    }
    if (dev) (void)hipFree(dev);
    return status;
}

// ------------------------------------------------------------------ writer --
nx_status nx_nxf_writer_create(nx_ctx* ctx, const char* path, nx_nxf_writer** out) {
    if (!ctx || !path || !out) return ferr(NX_ERR_INVALID, "nx_nxf_writer_create: null argument");
    *out = nullptr;
    nx_nxf_writer* w = new nx_nxf_writer();
    w->ctx = ctx;
    w->fd = ::open(path, O_WRONLY | O_CREAT | O_TRUNC, 0644);
    if (w->fd < 0) {
        delete w;
        return ferr(NX_ERR_IO, "nxf: cannot create '%s': %s", path, strerror(errno));
    }
    // the header's 64 bytes are written by finalize; data starts at 16 KiB
    static const uint8_t zeros[kAlign] = {};
    if (!pwrite_all(w->fd, zeros, kAlign, 0)) {
        delete w;
        return ferr(NX_ERR_IO, "nxf: cannot reserve the header of '%s'", path);
    }
    w->pos = kAlign;
    *out = w;
    return NX_OK;
}

nx_status nx_nxf_writer_set_manifest(nx_nxf_writer* w, const nx_nxf_manifest* m) {
    if (!w || !m) return ferr(NX_ERR_INVALID, "nx_nxf_writer_set_manifest: null argument");
    w->man = *m;
    w->man.architecture[sizeof(w->man.architecture) - 1] = 0;
    w->man.name[sizeof(w->man.name) - 1] = 0;
    return NX_OK;
}

nx_status nx_nxf_writer_begin_tensor(nx_nxf_writer* w, const char* name, const int64_t* shape, int ndim, int dtype) {
    if (!w || !name || (ndim > 0 && !shape) || ndim < 0 || ndim > 8 || dtype < 0 || dtype > 255)
        return ferr(NX_ERR_INVALID, "nx_nxf_writer_begin_tensor: bad argument");
    if (w->in_tensor) return ferr(NX_ERR_STATE, "nxf writer: begin_tensor inside tensor '%s'", w->cur.name.c_str());
    w->cur = Tensor{};
    w->cur.name = name;
    w->cur.shape.assign(shape, shape + ndim);
    w->cur.dtype = (uint8_t)dtype;
    w->in_tensor = true;
    return NX_OK;
}

nx_status nx_nxf_writer_add_chunk(nx_nxf_writer* w, const void* data, size_t size, int codec, int group_size) {
    if (!w) return ferr(NX_ERR_INVALID, "nx_nxf_writer_add_chunk: null writer");
    if (!w->in_tensor) return ferr(NX_ERR_STATE, "nxf writer: add_chunk outside a tensor");
    if (!data || size == 0) return NX_OK;  // nothing is written, as in the reference
    if (size > 0xFFFFFFFFull) return ferr(NX_ERR_INVALID, "nxf writer: chunk of %zu bytes exceeds 4 GiB", size);
    if (codec < 0 || codec > 255 || group_size < 0 || group_size > 255)
        return ferr(NX_ERR_INVALID, "nxf writer: codec and group size are bytes");
    nx_status s = writer_pad(w);
    if (s != NX_OK) return s;
    DiskChunk d{};
    d.file_offset = w->pos;
    d.compressed_size = d.decompressed_size = (uint32_t)size;
    d.codec = (uint8_t)codec;
    d.group_size = (uint8_t)group_size;
    if ((s = writer_put(w, data, size)) != NX_OK) return s;
    // keep a copy for the device hash (16-byte aligned in the stage)
    const size_t at = (w->stage_used + 255) / 256 * 256;
    if (at + size > w->stage_cap) {
        if ((s = writer_flush(w)) != NX_OK) return s;
        if (size > w->stage_cap) {
            if (w->stage) (void)hipHostFree(w->stage);
            w->stage = nullptr;
            const size_t cap = std::max<size_t>(size, 64ull << 20);
            if (hipHostMalloc(reinterpret_cast<void**>(&w->stage), cap, hipHostMallocDefault) != hipSuccess) {
                w->stage_cap = 0;
                return ferr(NX_ERR_OOM, "nxf writer: host staging of %zu bytes", cap);
            }
            w->stage_cap = cap;
        }
    }
    const size_t off = (w->stage_used + 255) / 256 * 256;
    memcpy(w->stage + off, data, size);
    w->stage_used = off + size;
    w->pending.emplace_back((int)w->cur.chunks.size(), off);
    w->cur.chunks.push_back(d);
    return NX_OK;
}

nx_status nx_nxf_writer_end_tensor(nx_nxf_writer* w) {
    if (!w) return ferr(NX_ERR_INVALID, "nx_nxf_writer_end_tensor: null writer");
    if (!w->in_tensor) return ferr(NX_ERR_STATE, "nxf writer: end_tensor without begin_tensor");
    nx_status s = writer_flush(w);
    if (s != NX_OK) return s;
    w->tensors.push_back(std::move(w->cur));
    w->cur = Tensor{};
    w->in_tensor = false;
    return NX_OK;
}

nx_status nx_nxf_writer_finalize(nx_nxf_writer* w) {
    if (!w) return ferr(NX_ERR_INVALID, "nx_nxf_writer_finalize: null writer");
    nx_status s = NX_OK;
    do {
        if (w->in_tensor && (s = nx_nxf_writer_end_tensor(w)) != NX_OK) break;
        if ((s = writer_pad(w)) != NX_OK) break;
        const std::vector<uint8_t> idx = index_blob(w->tensors);
        FileHeader h{};
        h.magic = kMagic;
        h.version = kVersion;
        h.tensor_index_offset = w->pos;
        h.tensor_index_size = idx.size();
        if (!idx.empty() && (s = writer_put(w, idx.data(), idx.size())) != NX_OK) break;
        if ((s = writer_pad(w)) != NX_OK) break;
        const std::string js = manifest_json(w->man);
        h.manifest_offset = w->pos;
        h.manifest_size = js.size();
        if ((s = writer_put(w, js.data(), js.size())) != NX_OK) break;
        if ((s = writer_pad(w)) != NX_OK) break;
        h.data_offset = kAlign;
        h.total_file_size = w->pos;
        if (!pwrite_all(w->fd, &h, sizeof(h), 0)) {
            s = ferr(NX_ERR_IO, "nxf writer: header write failed: %s", strerror(errno));
            break;
        }
        if (::close(w->fd) != 0) s = ferr(NX_ERR_IO, "nxf writer: close failed: %s", strerror(errno));
        w->fd = -1;
    } while (false);
    delete w;
    return s;
}

nx_status nx_nxf_writer_destroy(nx_nxf_writer* w) {
    if (!w) return ferr(NX_ERR_INVALID, "nx_nxf_writer_destroy: null writer");
    delete w;
    return NX_OK;
}

// ----------------------------------------------------------------- hashing --
nx_status nx_xxh32_chunks(nx_ctx* ctx, nx_buf data, const uint64_t* offsets, const uint32_t* sizes, int n,
                          uint32_t* hashes) {
    if (!ctx) return NX_ERR_INVALID;
    if (n < 0 || (n > 0 && (!offsets || !sizes || !hashes))) return nx::fail(ctx, NX_ERR_INVALID, "nx_xxh32_chunks: bad arguments");
    if (n == 0) return NX_OK;
    const size_t bsz = nx::buf_size(ctx, data);
    if (bsz == 0) return nx::fail(ctx, NX_ERR_INVALID, "nx_xxh32_chunks: unknown buffer");
    std::vector<nx::HashRange> r((size_t)n);
    for (int i = 0; i < n; ++i) {
        if (offsets[i] % 16 || offsets[i] > bsz || sizes[i] > bsz - offsets[i])
            return nx::fail(ctx, NX_ERR_INVALID, "nx_xxh32_chunks: range %d [%llu, +%u) is unaligned or outside the buffer",
                            i, (unsigned long long)offsets[i], sizes[i]);
        r[(size_t)i] = nx::HashRange{offsets[i], sizes[i], (uint32_t)i};
    }
    sort_ranges(r);
    HashScratch hs;
    nx_status s = hs.ensure(ctx, r.size());
    if (s != NX_OK) return s;
    hipStream_t st = ctx->stream;
    NX_HIP(ctx, hipMemcpyAsync(hs.ranges, r.data(), r.size() * sizeof(nx::HashRange), hipMemcpyHostToDevice, st));
    NX_HIP(ctx, nx::xxh32_launch(reinterpret_cast<const uint8_t*>(static_cast<uintptr_t>(data)), hs.ranges, n, hs.hashes, st));
    NX_HIP(ctx, hipMemcpyAsync(hashes, hs.hashes, (size_t)n * 4, hipMemcpyDeviceToHost, st));
    NX_HIP(ctx, hipStreamSynchronize(st));
    return NX_OK;
}

nx_status nx_time_xxh32(nx_ctx* ctx, nx_buf data, size_t bytes, uint32_t chunk_bytes, int iters, double* avg_ms,
                        uint32_t* hashes) {
    if (!ctx || !avg_ms || iters < 1 || chunk_bytes == 0 || chunk_bytes % 16 || bytes == 0)
        return nx::fail(ctx, NX_ERR_INVALID, "nx_time_xxh32: bad arguments");
    NX_NEED(ctx, data, bytes, "data");
    const size_t n = (bytes + chunk_bytes - 1) / chunk_bytes;
    if (n > (size_t)0x7FFFFFFF) return nx::fail(ctx, NX_ERR_INVALID, "nx_time_xxh32: too many chunks");
    std::vector<nx::HashRange> r(n);
    for (size_t i = 0; i < n; ++i)
        r[i] = nx::HashRange{(uint64_t)i * chunk_bytes, (uint32_t)std::min<uint64_t>(chunk_bytes, bytes - (uint64_t)i * chunk_bytes),
                             (uint32_t)i};
    sort_ranges(r);
    HashScratch hs;
    nx_status s = hs.ensure(ctx, n);
    if (s != NX_OK) return s;
    hipStream_t st = ctx->stream;
    const uint8_t* d = reinterpret_cast<const uint8_t*>(static_cast<uintptr_t>(data));
    NX_HIP(ctx, hipMemcpyAsync(hs.ranges, r.data(), n * sizeof(nx::HashRange), hipMemcpyHostToDevice, st));
    NX_HIP(ctx, nx::xxh32_launch(d, hs.ranges, (int)n, hs.hashes, st));  // warm-up
    NX_HIP(ctx, hipEventRecord(ctx->ev0, st));
    for (int i = 0; i < iters; ++i) NX_HIP(ctx, nx::xxh32_launch(d, hs.ranges, (int)n, hs.hashes, st));
    NX_HIP(ctx, hipEventRecord(ctx->ev1, st));
    NX_HIP(ctx, hipEventSynchronize(ctx->ev1));
    float ms = 0.0f;
    NX_HIP(ctx, hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1));
    *avg_ms = (double)ms / iters;
    if (hashes) {
        NX_HIP(ctx, hipMemcpyAsync(hashes, hs.hashes, n * 4, hipMemcpyDeviceToHost, st));
        NX_HIP(ctx, hipStreamSynchronize(st));
    }
    return NX_OK;
}

}  // extern "C"
