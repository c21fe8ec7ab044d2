// C-ABI shim over reference sources, compiled from /root/reference in place.
// CHECKER ONLY: loaded by the tests to pin the oracle against the reference's
// own functions; never part of the product.  Each entry point names the
// reference function it drives.
#include <cstring>
#include <vector>

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
}
