// C-ABI shim over reference sources, compiled from /root/reference in place.
// CHECKER ONLY: loaded by the tests to pin the oracle against the reference's
// own functions; never part of the product.  Each entry point names the
// reference function it drives.
#include <cstring>
#include <vector>

#include <algorithm>
#include <cstdio>
#include <string>

#include "format/nxf.h"
#include "kv/paged_attention.h"
#include "kv/turbo_quant.h"
#include "model/hybrid_model.h"
#include "model/moe_router.h"
#include "quant/gptq.h"

extern "C" {

// model/hybrid_model.h:123-140 (HybridKVCache fp16 conversions of the flat KV cache)
void ref_f32_to_f16_kv(const float* in, uint16_t* out, int n) {
    for (int i = 0; i < n; ++i) out[i] = nexus::model::HybridKVCache::f32_to_f16(in[i]);
}
void ref_f16_to_f32_kv(const uint16_t* in, float* out, int n) {
    for (int i = 0; i < n; ++i) out[i] = nexus::model::HybridKVCache::f16_to_f32(in[i]);
}

// kv/turbo_quant.cpp:172-219 (TurboQuantKV::build_codebook via the constructor)
int ref_tq_codebook(int d, int bits, float* centroids, float* boundaries) {
    nexus::kv::TurboQuantKV tq(d, bits, 42);
    const auto& cb = tq.codebook_;
    std::memcpy(centroids, cb.centroids.data(), sizeof(float) * cb.centroids.size());
    std::memcpy(boundaries, cb.boundaries.data(), sizeof(float) * cb.boundaries.size());
    return static_cast<int>(cb.centroids.size());
}

// kv/turbo_quant.cpp:19-32 (LloydMaxCodebook::encode)
void ref_tq_encode_scalar(int d, int bits, const float* x, int n, uint8_t* codes) {
    nexus::kv::TurboQuantKV tq(d, bits, 42);
    for (int i = 0; i < n; ++i) codes[i] = tq.codebook_.encode(x[i]);
}

// kv/turbo_quant.cpp:249-268 / :270-285
void ref_pack_codes(uint8_t* packed, const uint8_t* codes, int n, int bits) {
    nexus::kv::TurboQuantKV::pack_codes(packed, codes, n, bits);
}
void ref_unpack_codes(uint8_t* codes, const uint8_t* packed, int n, int bits) {
    nexus::kv::TurboQuantKV::unpack_codes(codes, packed, n, bits);
}

// kv/turbo_quant.cpp:289-357 with the rotation replaced by the identity, so
// quantize() reduces to norm, normalize, encode and pack.
void ref_tq_quantize_identity(int d, int bits, const float* x, int n, uint8_t* packed,
                              float* norms) {
    nexus::kv::TurboQuantKV tq(d, bits, 42);
    for (int i = 0; i < d; ++i)
        for (int j = 0; j < d; ++j) {
            tq.rotation_[i * d + j] = (i == j) ? 1.0f : 0.0f;
            tq.rotation_t_[i * d + j] = (i == j) ? 1.0f : 0.0f;
        }
    tq.quantize(packed, norms, x, n);
}

// quant/gptq.cpp:9-27
void ref_dequant_int4(float* out, const uint8_t* data, const float* scales, const float* zeros,
                      int n, int group_size) {
    nexus::quant::dequant_int4(out, data, scales, zeros, n, group_size);
}

// kv/paged_attention.cpp:81-128 (insert_kv) and :161-230 (get_vectors): insert n
// positions of one layer, then gather them back as contiguous [n][hkv*hd].
void ref_paged_gather(int hkv, int hd, int page_size, const float* k, const float* v, int n,
                      float* kout, float* vout) {
    nexus::kv::PagedKVCache cache(1, hkv, hd, n, page_size);
    for (int p = 0; p < n; ++p)
        cache.insert_kv(0, p, k + (size_t)p * hkv * hd, v + (size_t)p * hkv * hd);
    std::memcpy(kout, cache.get_keys(0, 0, n), sizeof(float) * (size_t)n * hkv * hd);
    std::memcpy(vout, cache.get_values(0, 0, n), sizeof(float) * (size_t)n * hkv * hd);
}

// model/moe_router.cpp:55-113 (first call: expert biases are zero)
int ref_moe_route(int E, int k, int d, const float* gate_w, const float* hidden, int* ids,
                  float* weights) {
    nexus::model::MoERouter r(E, k, d);
    r.load_gate_weights(gate_w);
    auto res = r.route(hidden);
    int i = 0;
    for (auto& [e, w] : res.expert_weights) {
        ids[i] = e;
        weights[i] = w;
        ++i;
    }
    return i;
}

// ------------------------------------------------------------------ NXF --
// Manifest and tensors in plain C for the NXF entry points below.
struct ref_manifest {
    char architecture[64];
    char name[128];
    uint32_t num_layers, hidden_dim, num_heads, num_kv_heads, head_dim, vocab_size, max_seq_len;
    float rope_theta, rms_norm_eps;
    uint32_t num_experts, num_active_experts;
    uint8_t default_codec, default_group_size;
};
struct ref_tensor {
    const char* name;
    int ndim;
    const int64_t* shape;
    int dtype;
    int nchunks;
    const void* const* data;
    const uint64_t* sizes;
    const int* codecs;
    const int* groups;
};

// format/nxf_writer.cpp:197-338 (create, set_manifest, begin_tensor,
// add_chunk, end_tensor, finalize)
int ref_nxf_write(const char* path, const ref_manifest* rm, const ref_tensor* ts, int n) {
    using namespace nexus::format;
    auto w = NXFWriter::create(path);
    if (!w) return 1;
    ModelManifest m{};
    m.architecture = rm->architecture;
    m.name = rm->name;
    m.num_layers = rm->num_layers;
    m.hidden_dim = rm->hidden_dim;
    m.num_heads = rm->num_heads;
    m.num_kv_heads = rm->num_kv_heads;
    m.head_dim = rm->head_dim;
    m.vocab_size = rm->vocab_size;
    m.max_seq_len = rm->max_seq_len;
    m.rope_theta = rm->rope_theta;
    m.rms_norm_eps = rm->rms_norm_eps;
    m.num_experts = rm->num_experts;
    m.num_active_experts = rm->num_active_experts;
    m.default_codec = static_cast<nexus::Codec>(rm->default_codec);
    m.default_group_size = rm->default_group_size;
    w->set_manifest(m);
    for (int i = 0; i < n; ++i) {
        const ref_tensor& t = ts[i];
        w->begin_tensor(t.name, std::vector<int64_t>(t.shape, t.shape + t.ndim), static_cast<nexus::DType>(t.dtype));
        for (int c = 0; c < t.nchunks; ++c)
            w->add_chunk(t.data[c], t.sizes[c], static_cast<nexus::Codec>(t.codecs[c]),
                         static_cast<uint8_t>(t.groups[c]));
        w->end_tensor();
    }
    w->finalize();
    return 0;
}

// format/nxf_reader.cpp:192-235: open, manifest(), tensor_names() and
// get_tensor(), printed as text: the manifest fields, then per tensor (by
// name) its shape, dtype and chunk descriptors.  Returns the text length
// (the text is cut at cap - 1 bytes), -1 if the reader refused the file.
long ref_nxf_summary(const char* path, char* out, size_t cap) {
    using namespace nexus::format;
    auto r = NXFReader::open(path);
    if (!r) return -1;
    const ModelManifest& m = r->manifest();
    std::string s;
    char buf[512];
    snprintf(buf, sizeof(buf), "manifest %s|%s|%u %u %u %u %u %u %u|%.9g %.9g|%u %u|%u %u\n", m.architecture.c_str(),
             m.name.c_str(), m.num_layers, m.hidden_dim, m.num_heads, m.num_kv_heads, m.head_dim, m.vocab_size,
             m.max_seq_len, (double)m.rope_theta, (double)m.rms_norm_eps, m.num_experts, m.num_active_experts,
             (unsigned)m.default_codec, (unsigned)m.default_group_size);
    s += buf;
    auto names = r->tensor_names();
    std::sort(names.begin(), names.end());
    for (const auto& nm : names) {
        const TensorInfo* t = r->get_tensor(nm);
        s += "tensor " + nm + " shape";
        for (int64_t d : t->shape) s += " " + std::to_string(d);
        s += " dtype " + std::to_string((int)t->dtype) + "\n";
        for (const ChunkDesc& c : t->chunks) {
            snprintf(buf, sizeof(buf), "  chunk %llu %u %u %08x %u %u\n", (unsigned long long)c.file_offset,
                     c.compressed_size, c.decompressed_size, c.checksum, (unsigned)c.codec, (unsigned)c.group_size);
            s += buf;
        }
    }
    if (cap > 0) {
        const size_t k = std::min(cap - 1, s.size());
        std::memcpy(out, s.data(), k);
        out[k] = 0;
    }
    return (long)s.size();
}

// format/nxf_reader.cpp:237-258 (map_chunk): the stored bytes of chunk c of
// tensor `name`; returns their count, -1 if absent.
long ref_nxf_chunk_bytes(const char* path, const char* name, int c, uint8_t* out, size_t cap) {
    using namespace nexus::format;
    auto r = NXFReader::open(path);
    if (!r) return -1;
    const TensorInfo* t = r->get_tensor(name);
    if (!t || c < 0 || c >= (int)t->chunks.size()) return -1;
    const void* p = r->map_chunk(t->chunks[(size_t)c]);
    if (!p) return -1;
    const size_t n = t->chunks[(size_t)c].compressed_size;
    std::memcpy(out, p, std::min(n, cap));
    r->unmap_chunk(p);
    return (long)n;
}
}
