// Resident decode runner: the MI355X counterpart of HybridModel
// (nexus/src/model/hybrid_model.cpp:319-774) for Llama-style dense and MoE
// decoders.  All weights live in HBM (generated on the device from the
// seed), the KV cache is paged (16-token pages, shuffled block table), and
// one decode step -- embedding of the pending token, every layer, the
// lm_head and the greedy argmax -- is a single captured HIP graph whose
// kernels read the positions and the pending token from device memory, so
// consecutive steps run back to back with no host round trip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "../../include/nexus_nxf.h"
#include "nx_common.h"
#include "nx_internal.h"
#include "nx_kernels.h"

using nx::fail;

namespace {

struct Layer {
    uint8_t* wqkv = nullptr;  // [qdim + 2 kvdim][Gd*16]  rows: q | k | v
    uint16_t* sqkv = nullptr;
    uint8_t* wo = nullptr;    // [d][Gq*16]
    uint16_t* so = nullptr;
    uint8_t* w13 = nullptr;   // dense [2F][Gd*16] (gate/up interleaved) or experts [E][2F][Gd*16]
    uint16_t* s13 = nullptr;
    uint8_t* w2 = nullptr;    // dense [d][Gf*16] or experts [E][d][Gf*16]
    uint16_t* s2 = nullptr;
    uint8_t* wr = nullptr;    // router [E][Gd*16]
    uint16_t* sr = nullptr;
    uint16_t *kpool = nullptr, *vpool = nullptr;
    uint8_t *kc4 = nullptr, *kc3 = nullptr, *vc4 = nullptr, *vc3 = nullptr;
    uint16_t *kn = nullptr, *vn = nullptr;
    uint8_t *kcc = nullptr, *vcc = nullptr;    // Cool pages [blocks][hkv][16][48] (three tiers)
    uint16_t *kcn = nullptr, *vcn = nullptr;
    float *ksign = nullptr, *vsign = nullptr;
    int32_t* moe_count = nullptr;  // [E]
    float* norm_attn = nullptr;    // RMSNorm weights [d]; nullptr = 1.0
    float* norm_ffn = nullptr;
    float* qnorm = nullptr;        // per-head Q/K RMSNorm weights [hd] (qk_norm); nullptr = 1.0
    float* knorm = nullptr;
};

size_t qbytes(size_t N, int K) { return N * (size_t)((K + 31) / 32) * 18; }

}  // namespace

struct nx_model {
    nx_ctx* ctx = nullptr;
    nx_model_config c{};
    int qdim = 0, kvdim = 0, nqkv = 0, Gd = 0, Gq = 0, Gf = 0, Fp = 0;
    std::vector<void*> allocs;
    uint16_t* embed = nullptr;
    uint8_t* lm_w = nullptr;
    uint16_t* lm_s = nullptr;
    float* norm_final = nullptr;  // final RMSNorm weights [d]; nullptr = 1.0
    std::vector<Layer> layers;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    int max_blocks = 0, n_blocks = 0;
    int32_t* block_table = nullptr;
    int32_t *pos = nullptr, *base = nullptr, *out_tokens = nullptr, *prompt = nullptr;
    unsigned long long* best = nullptr;
    int out_stride = 0;
    float* h = nullptr;
    float* q = nullptr;
    uint16_t* att16 = nullptr;
    uint16_t* act16 = nullptr;
    float* kpart = nullptr;  // K-part sums of the batched down projection and wo ([kparts_max][batch][d])
    int kparts_max = 0;
    float* logits = nullptr;
    float* kv_tmp = nullptr;
    uint16_t* xn16 = nullptr;
    float* router_logits = nullptr;
    int32_t* moe_ids = nullptr;
    float* moe_w = nullptr;
    int32_t* moe_slots = nullptr;
    int32_t* moe_plan = nullptr;   // [moe_plan_rows][kMoePlanInts]
    unsigned* moe_counter = nullptr;  // arrival counter of the MoE routing launch (zero between launches)
    uint16_t* moe_act = nullptr;
    float* moe_y = nullptr;
    float* moe_kpart = nullptr;  // K-part sums of the batched routed down projection
    float* attn_part = nullptr;
    // tiered pages: the fp16 window's ring of hot_pages pages per sequence
    // (hot_bt[b][p] = b * hot_pages + p % hot_pages, the same max_blocks
    // stride as block_table)
    int hot_pages = 0;
    int32_t* hot_bt = nullptr;
    // three tiers (warm_window > 0): block_table is the TurboQuant (Warm)
    // range's ring of warm_pages pages per sequence (block_table[b][p] = b *
    // warm_pages + p % warm_pages), cool_bt the Cool pages (a seeded
    // permutation of the pool, max_blocks per sequence)
    int warm_pages = 0;
    int32_t* cool_bt = nullptr;
    // shared page pool (kv_blocks > 0): the sequence-length table (block_table,
    // or cool_bt with three tiers) takes pages on demand from a free list of
    // kv_blocks pages and gives them back when the slot retires or starts
    // over; entries without a page name the spare page pool_trash, which
    // parked and held slots may write and nothing reads
    int pool_trash = -1;
    int32_t* long_table = nullptr;
    std::vector<int32_t> h_table;            // host copy of long_table
    std::vector<std::vector<int32_t>> owned;  // pages of each slot, in position order
    std::vector<int32_t> free_pages;
    // with a Cool window (cool_window > 0), cool_bt is the Cool range's ring of
    // cool_pages pages per sequence and older pages are evicted
    int cool_pages = 0;
    unsigned* attn_counts = nullptr;  // split-completion counters of the fp16 attention
    int32_t* h_stage = nullptr;  // pinned host staging [batch]
    int32_t* h_out = nullptr;    // pinned host [batch][out_stride]
    hipGraphExec_t exec = nullptr;        // one decode step
    hipGraphExec_t exec_multi = nullptr;  // kStepsPerGraph decode steps
    std::vector<int> hpos;       // host mirror of pos (last processed position)
    int prefill_batched = 1;     // batched (GEMM) prefill where the model allows it
    int prenorm = 1;             // batch 2-8: RMSNorm as its own launch before the GEMVs that take it
    int wo_kparts = 2;           // batch 2-8: K parts of wo (0: one launch over all of K)
    // sampling (temperature <= 0: greedy argmax of the lm_head epilogue)
    float temperature = 0.0f, top_p = 1.0f, u_fixed = -1.0f;
    int top_k = 0;
    float* smp_scratch = nullptr;  // [batch][vocab] then [batch][kSmpPartFloats], allocated when sampling is first set
    // per-slot serving state: a slot holds one sequence (active) or none
    // (free: parked at position 0 by the step graph); feed / fpos tell the
    // embedding kernel what each slot consumes at a step (kFeed*)
    std::vector<char> active;
    int32_t* feed = nullptr;     // device [batch]
    int32_t* fpos = nullptr;     // device [batch]
    int32_t* h_feed = nullptr;   // pinned host [2 * batch]: feed then fpos
};

namespace {

template <class T>
nx_status dalloc(nx_model* m, T** out, size_t count) {
    void* p = nullptr;
    const size_t bytes = count * sizeof(T) > 0 ? count * sizeof(T) : 16;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return nx::hip_fail(m->ctx, e, "hipMalloc (model)");
    m->allocs.push_back(p);
    e = hipMemsetAsync(p, 0, bytes, m->ctx->stream);
    if (e != hipSuccess) return nx::hip_fail(m->ctx, e, "hipMemsetAsync (model)");
    *out = static_cast<T*>(p);
    return NX_OK;
}

#define NX_TRY(expr)                      \
    do {                                  \
        nx_status nx_s_ = (expr);         \
        if (nx_s_ != NX_OK) return nx_s_; \
    } while (0)
#define NX_LAUNCH(m, expr)                                                       \
    do {                                                                         \
        hipError_t nx_e_ = (expr);                                               \
        if (nx_e_ != hipSuccess) return nx::hip_fail((m)->ctx, nx_e_, #expr);    \
    } while (0)

void host_shuffle(std::vector<int32_t>& perm, int n, uint64_t seed, uint32_t tid) {
    perm.resize(n);
    for (int i = 0; i < n; ++i) perm[i] = i;
    const uint64_t key = nx::stream_key(seed, tid);
    for (int i = n - 1; i >= 1; --i) {
        const int j = (int)(nx::rand_at(key, (uint64_t)i) % (uint64_t)(i + 1));
        std::swap(perm[i], perm[j]);
    }
}

nx_status generate_weights(nx_model* m) {
    const nx_model_config& c = m->c;
    hipStream_t st = m->ctx->stream;
    const uint64_t seed = c.seed;
    const float k02 = nx::normal_k(0.02);
    const int d = c.d_model, F = c.ffn, E = c.n_experts;
    NX_LAUNCH(m, nx::gen_f16_launch(m->embed, (size_t)c.vocab * d, seed, nx::kTidEmbed, k02, st));
    NX_LAUNCH(m, nx::gen_quant_launch(m->lm_w, m->lm_s, c.vocab, d, seed, nx::kTidLmHead, k02, 0, 1, st));
    // RMSNorm weights 1 + N(0, norm_sigma), generated on the host (n = d, or
    // head_dim for the Q/K norms)
    auto gen_norm = [&](float* dst, uint32_t tid, int n) -> nx_status {
        if (!dst) return NX_OK;
        std::vector<float> w((size_t)n);
        const uint64_t key = nx::stream_key(seed, tid);
        const float kn = nx::normal_k((double)c.norm_sigma);
        for (int i = 0; i < n; ++i) w[(size_t)i] = 1.0f + nx::normal_from(nx::rand_at(key, (uint64_t)i), kn);
        NX_HIP(m->ctx, hipMemcpyAsync(dst, w.data(), w.size() * 4, hipMemcpyHostToDevice, st));
        NX_HIP(m->ctx, hipStreamSynchronize(st));  // w is released on return
        return NX_OK;
    };
    NX_TRY(gen_norm(m->norm_final, nx::kTidFinalNorm, d));
    for (int L = 0; L < c.n_layers; ++L) {
        Layer& ly = m->layers[L];
        NX_TRY(gen_norm(ly.norm_attn, nx::tid_layer(L, nx::N_ATTN), d));
        NX_TRY(gen_norm(ly.norm_ffn, nx::tid_layer(L, nx::N_FFN), d));
        NX_TRY(gen_norm(ly.qnorm, nx::tid_layer(L, nx::N_QNORM), c.head_dim));
        NX_TRY(gen_norm(ly.knorm, nx::tid_layer(L, nx::N_KNORM), c.head_dim));
        NX_LAUNCH(m, nx::gen_quant_launch(ly.wqkv, ly.sqkv, m->qdim, d, seed, nx::tid_layer(L, nx::W_Q), k02, 0, 1, st));
        NX_LAUNCH(m, nx::gen_quant_launch(ly.wqkv, ly.sqkv, m->kvdim, d, seed, nx::tid_layer(L, nx::W_K), k02, m->qdim, 1, st));
        NX_LAUNCH(m, nx::gen_quant_launch(ly.wqkv, ly.sqkv, m->kvdim, d, seed, nx::tid_layer(L, nx::W_V), k02,
                                          m->qdim + m->kvdim, 1, st));
        NX_LAUNCH(m, nx::gen_quant_launch(ly.wo, ly.so, d, m->qdim, seed, nx::tid_layer(L, nx::W_O), k02, 0, 1, st));
        if (E == 0) {
            NX_LAUNCH(m, nx::gen_quant_launch(ly.w13, ly.s13, F, d, seed, nx::tid_layer(L, nx::W_GATE), k02, 0, 2, st));
            NX_LAUNCH(m, nx::gen_quant_launch(ly.w13, ly.s13, F, d, seed, nx::tid_layer(L, nx::W_UP), k02, 1, 2, st));
            NX_LAUNCH(m, nx::gen_quant_launch(ly.w2, ly.s2, d, F, seed, nx::tid_layer(L, nx::W_DOWN), k02, 0, 1, st));
        } else {
            NX_LAUNCH(m, nx::gen_quant_launch(ly.wr, ly.sr, E, d, seed, nx::tid_layer(L, nx::W_ROUTER),
                                              nx::normal_k(1.0 / std::sqrt((double)d)), 0, 1, st));
            for (int e = 0; e < E; ++e) {
                NX_LAUNCH(m, nx::gen_quant_launch(ly.w13, ly.s13, F, d, seed, nx::tid_expert(L, e, 0), k02, e * 2 * F, 2, st));
                NX_LAUNCH(m, nx::gen_quant_launch(ly.w13, ly.s13, F, d, seed, nx::tid_expert(L, e, 1), k02, e * 2 * F + 1, 2, st));
                NX_LAUNCH(m, nx::gen_quant_launch(ly.w2, ly.s2, d, F, seed, nx::tid_expert(L, e, 2), k02, e * d, 1, st));
            }
        }
    }
    return NX_OK;
}

// Sampling of sequences [b0, b0 + nb) from the lm_head logits: the sampled
// token replaces the argmax as the pending token.
nx_status enqueue_sample(nx_model* m, int b0, int nb) {
    nx::SampleArgs s{};
    s.logits = m->logits + (size_t)b0 * m->c.vocab;
    s.V = m->c.vocab;
    s.ldl = m->c.vocab;
    s.temperature = m->temperature;
    s.top_k = m->top_k;
    s.top_p = m->top_p;
    s.u_fixed = m->u_fixed;
    s.key = m->c.seed ^ 0x5A4D504C45ull;  // draws of seed 0, keyed by (sequence, position)
    s.pos = m->pos + b0;
    s.best = m->best + b0;
    s.scratch = m->smp_scratch + (size_t)b0 * m->c.vocab;
    s.part = m->smp_scratch + (size_t)m->c.batch * m->c.vocab + (size_t)b0 * nx::kSmpPartFloats;
    NX_LAUNCH(m, nx::sample_launch(s, nb, m->ctx->stream));
    return NX_OK;
}

// Arguments of the batch-1 QKV GEMV (RMSNorm of h, RoPE, page write) and of
// the wo GEMV (attention output, residual add into h) of layer L.
nx::GemvArgs qkv_args(const nx_model* m, const Layer& ly) {
    const nx_model_config& c = m->c;
    nx::GemvArgs a{};
    a.W = ly.wqkv;
    a.S = ly.sqkv;
    a.N = m->nqkv;
    a.K = c.d_model;
    a.G = m->Gd;
    a.batch = c.batch;
    a.h32 = m->h;
    a.ldx = c.d_model;
    a.eps = c.eps;
    a.norm_w = ly.norm_attn;
    a.q32 = m->q;
    a.qdim = m->qdim;
    a.kvdim = m->kvdim;
    a.hd = c.head_dim;
    a.hkv = c.n_kv_heads;
    a.pos = m->pos;
    a.cos_t = m->rope_cos;
    a.sin_t = m->rope_sin;
    a.block_table = c.kv_kind == 2 ? m->hot_bt : m->block_table;
    a.max_blocks = m->max_blocks;
    if (c.kv_kind != 1 && !c.qk_norm) {
        a.kpool = ly.kpool;
        a.vpool = ly.vpool;
    } else {
        a.kv_tmp = m->kv_tmp;
    }
    if (c.qk_norm) {
        // the projection only: q to q32, k and v to kv_tmp, no RoPE; the
        // Q/K norm launch then normalizes, rotates and writes the pages
        a.cos_t = nullptr;
        a.sin_t = nullptr;
    }
    return a;
}

// Per-head Q/K RMSNorm + RoPE + the page write of K/V (qk_norm models),
// after the QKV GEMV of layer ly left q in q32 and k, v in kv_tmp.
hipError_t qk_norm_launch(nx_model* m, const Layer& ly, hipStream_t st) {
    const nx_model_config& c = m->c;
    nx::QknArgs a{};
    a.q32 = m->q;
    a.kv_tmp = m->kv_tmp;
    a.qn = ly.qnorm;
    a.kn = ly.knorm;
    a.cos_t = m->rope_cos;
    a.sin_t = m->rope_sin;
    a.pos = m->pos;
    a.block_table = c.kv_kind == 2 ? m->hot_bt : m->block_table;
    a.max_blocks = m->max_blocks;
    if (c.kv_kind != 1) {  // TurboQuant pages: the attention launch appends from kv_tmp
        a.kpool = ly.kpool;
        a.vpool = ly.vpool;
    }
    a.hq = c.n_heads;
    a.hkv = c.n_kv_heads;
    a.hd = c.head_dim;
    a.eps = c.eps;
    return nx::qk_norm_rope_launch(a, c.batch, st);
}

nx::GemvArgs wo_args(const nx_model* m, const Layer& ly) {
    nx::GemvArgs o{};
    o.W = ly.wo;
    o.S = ly.so;
    o.N = m->c.d_model;
    o.K = m->qdim;
    o.G = m->Gq;
    o.batch = m->c.batch;
    o.x16 = m->att16;
    o.ldx = m->qdim;
    o.y32 = m->h;
    o.ldy = m->c.d_model;
    return o;
}

nx::AttnArgs attn_args(const nx_model* m, const Layer& ly) {
    const nx_model_config& c = m->c;
    nx::AttnArgs at{};
    at.q = m->q;
    at.kpool = ly.kpool;
    at.vpool = ly.vpool;
    at.kc4 = ly.kc4;
    at.kc3 = ly.kc3;
    at.vc4 = ly.vc4;
    at.vc3 = ly.vc3;
    at.kn = ly.kn;
    at.vn = ly.vn;
    at.ksign = ly.ksign;
    at.vsign = ly.vsign;
    at.block_table = m->block_table;
    at.ctx_lens = nullptr;
    at.pos = m->pos;
    at.out16 = m->att16;
    at.batch = c.batch;
    at.hq = c.n_heads;
    at.hkv = c.n_kv_heads;
    at.hd = c.head_dim;
    at.max_blocks = m->max_blocks;
    at.max_ctx = c.max_seq;
    at.part = m->attn_part;
    at.counts = m->attn_counts;
    return at;
}

// Attention of layer ly for every sequence (q in m->q, output m->att16).
// TurboQuant pages: the launch also appends this step's K and V (kv_tmp),
// unless `append` is false (the pages already hold every position).
// Tiered pages: one launch whose blocks read either the compressed pages
// (TurboQuant) or the fp16 window, merged by the last block, and compress the
// page that leaves the window at this step.
hipError_t attention_launch(nx_model* m, const Layer& ly, hipStream_t st, bool append = true) {
    const nx_model_config& c = m->c;
    nx::AttnArgs at = attn_args(m, ly);
    if (c.kv_kind == 0) return nx::attn_f16_launch(at, st);
    if (c.kv_kind == 1) {
        if (append) at.kv_cur = m->kv_tmp;  // the launch also encodes this step's K and V into the pages
        return nx::attn_tq_launch(at, st);
    }
    at.hot_window = c.hot_window;
    at.hot_table = m->hot_bt;
    at.warm_window = c.warm_window;
    at.cool_window = c.cool_window;
    at.cool_table = m->cool_bt;
    at.kcc = ly.kcc;
    at.vcc = ly.vcc;
    at.kcn = ly.kcn;
    at.vcn = ly.vcn;
    return nx::attn_tiered_launch(at, st);
}

// Tier boundaries of a sequence whose next attention covers ctx positions:
// [0, evict) evicted, [evict, cool) Cool, [cool, cold) TurboQuant, [cold,
// ctx) fp16.
void tier_bounds(const nx_model_config& c, int ctx, int& cool, int& cold, int& evict) {
    evict = 0;
    if (c.kv_kind != 2) {
        cool = 0;
        cold = c.kv_kind == 1 ? ctx : 0;
        return;
    }
    auto edge = [&](int w) { return nx::kPage * std::max(0, (ctx - 1 - w) / nx::kPage); };
    cold = edge(c.hot_window);
    cool = c.warm_window > 0 ? edge(c.hot_window + c.warm_window) : 0;
    if (c.warm_window > 0 && c.cool_window > 0) evict = edge(c.hot_window + c.warm_window + c.cool_window);
}

// KV bytes one attention pass reads for sequences at hpos (TurboQuant: 58
// bytes per vector, Cool 50; tiered: Cool, then TurboQuant before the
// window, fp16 in it; evicted positions are read from no memory).
double kv_bytes(const nx_model* m) {
    const nx_model_config& c = m->c;
    const double f16 = 2.0 * c.n_kv_heads * c.head_dim * 2, tq = 2.0 * c.n_kv_heads * 58, cl = 2.0 * c.n_kv_heads * 50;
    double kv = 0.0;
    for (int b = 0; b < c.batch; ++b) {
        const int ctx = m->hpos[b] + 1;
        int cool = 0, cold = 0, evict = 0;
        tier_bounds(c, ctx, cool, cold, evict);  // the attention's boundaries
        kv += (cool - evict) * cl + (cold - cool) * tq + (ctx - cold) * f16;
    }
    return kv;
}

// Shared page pool: pages for positions up to last_pos of every slot that
// `want` names (slot -> last position, -1 = none), all or nothing; the
// table rows that changed are uploaded before anything reads them.
nx_status pool_ensure(nx_model* m, const std::vector<int>& want) {
    if (m->c.kv_blocks <= 0) return NX_OK;
    size_t need = 0;
    for (size_t b = 0; b < want.size(); ++b) {
        const size_t n = want[b] >= 0 ? (size_t)(want[b] / nx::kPage + 1) : 0;
        if (n > m->owned[b].size()) need += n - m->owned[b].size();
    }
    if (need > m->free_pages.size())
        return fail(m->ctx, NX_ERR_CAPACITY, "kv page pool: %zu pages needed, %zu free", need, m->free_pages.size());
    for (size_t b = 0; b < want.size(); ++b) {
        if (want[b] < 0) continue;
        const size_t n = (size_t)(want[b] / nx::kPage + 1), first = m->owned[b].size();
        if (n <= first) continue;
        for (size_t i = first; i < n; ++i) {
            const int32_t blk = m->free_pages.back();
            m->free_pages.pop_back();
            m->owned[b].push_back(blk);
            m->h_table[b * m->max_blocks + i] = blk;
        }
        const size_t off = b * m->max_blocks + first;
        NX_HIP(m->ctx, hipMemcpyAsync(m->long_table + off, m->h_table.data() + off, (n - first) * 4,
                                      hipMemcpyHostToDevice, m->ctx->stream));
    }
    NX_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    return NX_OK;
}

// The pages of slot b back to the free list (its rows name the spare page).
nx_status pool_release(nx_model* m, int b) {
    if (m->c.kv_blocks <= 0 || m->owned[(size_t)b].empty()) return NX_OK;
    std::vector<int32_t>& own = m->owned[(size_t)b];
    for (size_t i = own.size(); i-- > 0;) m->free_pages.push_back(own[i]);
    const size_t off = (size_t)b * m->max_blocks;
    std::fill(m->h_table.begin() + off, m->h_table.begin() + off + own.size(), m->pool_trash);
    NX_HIP(m->ctx, hipMemcpyAsync(m->long_table + off, m->h_table.data() + off, own.size() * 4, hipMemcpyHostToDevice,
                                  m->ctx->stream));
    NX_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    own.clear();
    return NX_OK;
}

// What each slot consumes at the following steps: feed[b] (a kFeed* mode or
// a token id) and fpos[b] (the position of a held slot); stream ordered.
nx_status upload_feed(nx_model* m, const int32_t* feed, const int32_t* fpos) {
    const int B = m->c.batch;
    for (int b = 0; b < B; ++b) {
        m->h_feed[b] = feed[b];
        m->h_feed[B + b] = fpos ? fpos[b] : 0;
    }
    NX_HIP(m->ctx, hipMemcpyAsync(m->feed, m->h_feed, (size_t)B * 4, hipMemcpyHostToDevice, m->ctx->stream));
    NX_HIP(m->ctx, hipMemcpyAsync(m->fpos, m->h_feed + B, (size_t)B * 4, hipMemcpyHostToDevice, m->ctx->stream));
    // the pinned staging is rewritten by the next call
    NX_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    return NX_OK;
}

// Active slots decode, free slots are parked.
nx_status feed_decode(nx_model* m) {
    std::vector<int32_t> f((size_t)m->c.batch);
    for (int b = 0; b < m->c.batch; ++b) f[(size_t)b] = m->active[(size_t)b] ? nx::kFeedDecode : nx::kFeedPark;
    return upload_feed(m, f.data(), nullptr);
}

// Batch 2-8 with pre-normalized GEMV inputs (m->prenorm): RMSNorm(h) is
// written once per token as fp16 (m->xn16) and the GEMVs that take it stage
// that, instead of every block of the matrix-core GEMV reading and reducing
// the whole fp32 h.
bool prenorm_on(const nx_model* m) { return m->prenorm && m->c.batch > 1; }

// A GEMV whose input is RMSNorm(h32) with weights norm_w: at batch 1 the
// kernel normalizes h itself while it stages it; with prenorm_on the input
// is m->xn16, written by a small launch here, or already (xn_ready) by the
// launch before, which normalized the rows it finished.
hipError_t norm_gemv_launch(nx_model* m, int epi, nx::GemvArgs a, hipStream_t st, bool xn_ready = false) {
    if (!prenorm_on(m)) return nx::gemv_launch(nx::X_RMSNORM, epi, a, st);
    if (!xn_ready) {
        const hipError_t e = nx::rmsnorm_launch(a.h32, a.norm_w, m->xn16, a.K, a.eps, a.batch, st);
        if (e != hipSuccess) return e;
    }
    a.x16 = m->xn16;
    a.ldx = a.K;
    a.h32 = nullptr;
    a.norm_w = nullptr;
    return nx::gemv_launch(nx::X_F16, epi, a, st);
}

// One decode step for every sequence, enqueued on the context stream.
nx_status enqueue_step(nx_model* m) {
    const nx_model_config& c = m->c;
    hipStream_t st = m->ctx->stream;
    const int B = c.batch, d = c.d_model, F = c.ffn, E = c.n_experts;
    NX_LAUNCH(m, nx::embed_launch(m->best, m->pos, m->base, m->out_tokens, m->out_stride, m->embed, m->h, d,
                                  c.vocab, B, st, m->feed, m->fpos));
    bool xn_ready = false;  // m->xn16 holds RMSNorm(h) for the next RMSNorm-input GEMV
    for (int L = 0; L < c.n_layers; ++L) {
        Layer& ly = m->layers[L];
        {
            // RMSNorm + QKV + RoPE + paged KV append, attention, wo + residual
            NX_LAUNCH(m, norm_gemv_launch(m, nx::E_QKV, qkv_args(m, ly), st, xn_ready));
            if (c.qk_norm) NX_LAUNCH(m, qk_norm_launch(m, ly, st));
            NX_LAUNCH(m, attention_launch(m, ly, st));
            nx::GemvArgs wo = wo_args(m, ly);
            if (prenorm_on(m) && m->kpart && m->wo_kparts > 0 &&
                nx::gemv_parts_for(m->qdim, B, m->wo_kparts) <= m->kparts_max) {
                // K split, the part-sum launch normalizes the new h for gate/up
                wo.kpart = m->kpart;
                wo.want_kparts = m->wo_kparts;
                if (E == 0) {
                    wo.post_norm_w = ly.norm_ffn;
                    wo.post_x16 = m->xn16;
                    wo.post_eps = c.eps;
                }
            }
            NX_LAUNCH(m, nx::gemv_launch(nx::X_F16, nx::E_ACC, wo, st));
            xn_ready = wo.post_x16 != nullptr;
        }
        if (E == 0) {
            // RMSNorm + gate/up + SwiGLU, then down + residual
            nx::GemvArgs f{};
            f.W = ly.w13;
            f.S = ly.s13;
            f.N = 2 * F;
            f.K = d;
            f.G = m->Gd;
            f.batch = B;
            f.h32 = m->h;
            f.ldx = d;
            f.eps = c.eps;
            f.norm_w = ly.norm_ffn;
            f.act16 = m->act16;
            f.lda = m->Fp;
            NX_LAUNCH(m, norm_gemv_launch(m, nx::E_SWIGLU, f, st, xn_ready));
            nx::GemvArgs dn{};
            dn.W = ly.w2;
            dn.S = ly.s2;
            dn.N = d;
            dn.K = F;
            dn.G = m->Gf;
            dn.batch = B;
            dn.x16 = m->act16;
            dn.ldx = m->Fp;
            dn.y32 = m->h;
            dn.ldy = d;
            dn.kpart = m->kpart;
            if (prenorm_on(m)) {
                // the new h rows normalized for the next layer's QKV (or the lm_head)
                dn.post_norm_w = L + 1 < c.n_layers ? m->layers[(size_t)L + 1].norm_attn : m->norm_final;
                dn.post_x16 = m->xn16;
                dn.post_eps = c.eps;
            }
            NX_LAUNCH(m, nx::gemv_launch(nx::X_F16, nx::E_ACC, dn, st));
            xn_ready = prenorm_on(m);
        } else {
            nx::MoeArgs ma{};
            ma.logits = m->router_logits;
            ma.E = E;
            ma.k = c.top_k;
            ma.batch = B;
            ma.ids = m->moe_ids;
            ma.weights = m->moe_w;
            ma.expert_count = ly.moe_count;
            ma.expert_slots = m->moe_slots;
            ma.plan = m->moe_plan;
            const bool fused_b1 = B == 1 && nx::moe_b1_fused_fits(d, F, E, c.top_k);
            if (fused_b1) {
                // batch 1: the routing runs in the gate/up launch below
                ma.h = m->h;
                ma.eps = c.eps;
                ma.norm_w = ly.norm_ffn;
                ma.d = d;
                ma.wr = ly.wr;
                ma.sr = ly.sr;
            } else if (nx::moe_norm_route_fits(d, E, c.top_k, B)) {
                // RMSNorm, router and routing in one launch
                ma.h = m->h;
                ma.eps = c.eps;
                ma.norm_w = ly.norm_ffn;
                ma.d = d;
                ma.wr = ly.wr;
                ma.sr = ly.sr;
                ma.xn16 = m->xn16;
                ma.counter = m->moe_counter;
                NX_LAUNCH(m, nx::moe_norm_route_launch(ma, st));
            } else {
                NX_LAUNCH(m, nx::rmsnorm_launch(m->h, ly.norm_ffn, m->xn16, d, c.eps, B, st));
                nx::GemvArgs r{};
                r.W = ly.wr;
                r.S = ly.sr;
                r.N = E;
                r.K = d;
                r.G = m->Gd;
                r.batch = B;
                r.x16 = m->xn16;
                r.ldx = d;
                r.y32 = m->router_logits;
                r.ldy = E;
                NX_LAUNCH(m, nx::gemv_launch(nx::X_F16, nx::E_F32, r, st));
                NX_LAUNCH(m, nx::moe_route_launch(ma, st));
            }
            nx::MoeFfnArgs mf{};
            mf.x16 = m->xn16;
            mf.ldx = d;
            mf.w13 = ly.w13;
            mf.s13 = ly.s13;
            mf.w2 = ly.w2;
            mf.s2 = ly.s2;
            mf.d = d;
            mf.F = F;
            mf.E = E;
            mf.k = c.top_k;
            mf.batch = B;
            mf.plan = m->moe_plan;
            mf.weights = m->moe_w;
            mf.act16 = m->moe_act;
            mf.y32 = m->moe_y;
            mf.kpart = m->moe_kpart;
            mf.out = m->h;
            mf.accumulate = 1;
            if (fused_b1) {
                NX_LAUNCH(m, nx::moe_b1_gate_up_launch(ma, mf, st));
                if (nx::moe_b1_down_combine_fits(F, c.top_k)) {
                    NX_LAUNCH(m, nx::moe_b1_down_combine_launch(mf, m->moe_ids, st));
                } else {
                    NX_LAUNCH(m, nx::moe_down_launch(mf, st));
                    NX_LAUNCH(m, nx::moe_combine_launch(mf, st));
                }
                xn_ready = false;
            } else {
                NX_LAUNCH(m, nx::moe_gate_up_launch(mf, st));
                NX_LAUNCH(m, nx::moe_down_launch(mf, st));
                if (prenorm_on(m) && nx::moe_combine_norm_fits(mf)) {
                    // the new h rows normalized for the next layer's QKV (or the lm_head)
                    const float* nw = L + 1 < c.n_layers ? m->layers[(size_t)L + 1].norm_attn : m->norm_final;
                    NX_LAUNCH(m, nx::moe_combine_norm_launch(mf, nw, m->xn16, c.eps, st));
                    xn_ready = true;
                } else {
                    NX_LAUNCH(m, nx::moe_combine_launch(mf, st));
                    xn_ready = false;
                }
            }
        }
    }
    // final RMSNorm + lm_head + greedy argmax
    nx::GemvArgs lm{};
    lm.W = m->lm_w;
    lm.S = m->lm_s;
    lm.N = c.vocab;
    lm.K = d;
    lm.G = m->Gd;
    lm.batch = B;
    lm.h32 = m->h;
    lm.ldx = d;
    lm.eps = c.eps;
    lm.norm_w = m->norm_final;
    lm.y32 = m->logits;
    lm.ldy = c.vocab;
    lm.best = m->best;
    NX_LAUNCH(m, norm_gemv_launch(m, nx::E_LOGITS, lm, st, xn_ready));
    if (m->temperature > 0.0f) NX_TRY(enqueue_sample(m, 0, B));
    return NX_OK;
}

// Decode steps per multi-step graph: a graph launch has a fixed cost of a few
// microseconds, paid once per kStepsPerGraph tokens in nx_model_decode.
constexpr int kStepsPerGraph = 8;

nx_status capture_steps(nx_model* m, int steps, hipGraphExec_t* out) {
    hipStream_t st = m->ctx->stream;
    NX_HIP(m->ctx, hipStreamSynchronize(st));
    NX_HIP(m->ctx, hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    nx_status s = NX_OK;
    for (int i = 0; i < steps && s == NX_OK; ++i) s = enqueue_step(m);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(st, &g);
    if (s != NX_OK) {
        if (g) (void)hipGraphDestroy(g);
        return s;
    }
    if (e != hipSuccess) return nx::hip_fail(m->ctx, e, "hipStreamEndCapture");
    e = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
        *out = nullptr;
        return nx::hip_fail(m->ctx, e, "hipGraphInstantiate (decode step)");
    }
    return NX_OK;
}

nx_status ensure_graph(nx_model* m) {
    if (!m->exec) NX_TRY(capture_steps(m, 1, &m->exec));
    if (!m->exec_multi) NX_TRY(capture_steps(m, kStepsPerGraph, &m->exec_multi));
    return NX_OK;
}

nx_status free_model(nx_model* m) {
    if (m->ctx) (void)hipStreamSynchronize(m->ctx->stream);
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->exec_multi) (void)hipGraphExecDestroy(m->exec_multi);
    for (void* p : m->allocs) (void)hipFree(p);
    if (m->h_stage) (void)hipHostFree(m->h_stage);
    if (m->h_out) (void)hipHostFree(m->h_out);
    if (m->h_feed) (void)hipHostFree(m->h_feed);
    delete m;
    return NX_OK;
}

// Allocate the model; synthetic: generate the weights from the seed,
// otherwise leave them for the loader (norm weights always allocated).
nx_status create_impl(nx_model* m, bool synthetic) {
    const nx_model_config& c = m->c;
    const int B = c.batch, d = c.d_model, F = c.ffn, E = c.n_experts, L = c.n_layers;
    m->qdim = c.n_heads * c.head_dim;
    m->kvdim = c.n_kv_heads * c.head_dim;
    m->nqkv = m->qdim + 2 * m->kvdim;
    m->Gd = (d + 31) / 32;
    m->Gq = (m->qdim + 31) / 32;
    m->Gf = (F + 31) / 32;
    m->Fp = m->Gf * 32;
    m->max_blocks = c.max_seq / nx::kPage;
    m->n_blocks = c.kv_blocks > 0 ? c.kv_blocks + 1 : m->max_blocks * B;
    m->hot_pages = c.kv_kind == 2 ? c.hot_window / nx::kPage + 1 : 0;
    m->warm_pages = c.kv_kind == 2 && c.warm_window > 0 ? c.warm_window / nx::kPage + 1 : 0;
    m->cool_pages = m->warm_pages > 0 && c.cool_window > 0 ? c.cool_window / nx::kPage + 1 : 0;
    m->out_stride = c.max_seq;
    m->layers.resize(L);
    m->hpos.assign(B, -1);

    NX_TRY(dalloc(m, &m->embed, (size_t)c.vocab * d));
    NX_TRY(dalloc(m, &m->lm_w, (size_t)c.vocab * m->Gd * 16));
    NX_TRY(dalloc(m, &m->lm_s, (size_t)c.vocab * m->Gd));
    const bool norms = !synthetic || c.norm_sigma != 0.0f;
    if (norms) NX_TRY(dalloc(m, &m->norm_final, (size_t)d));
    const size_t pool_elems = (size_t)m->n_blocks * c.n_kv_heads * nx::kPage * c.head_dim;
    const size_t pool_vecs = (size_t)m->n_blocks * c.n_kv_heads * nx::kPage;
    for (int l = 0; l < L; ++l) {
        Layer& ly = m->layers[l];
        NX_TRY(dalloc(m, &ly.wqkv, (size_t)m->nqkv * m->Gd * 16));
        NX_TRY(dalloc(m, &ly.sqkv, (size_t)m->nqkv * m->Gd));
        NX_TRY(dalloc(m, &ly.wo, (size_t)d * m->Gq * 16));
        NX_TRY(dalloc(m, &ly.so, (size_t)d * m->Gq));
        const size_t ne = E == 0 ? 1 : (size_t)E;
        NX_TRY(dalloc(m, &ly.w13, ne * 2 * F * m->Gd * 16));
        NX_TRY(dalloc(m, &ly.s13, ne * 2 * F * m->Gd));
        NX_TRY(dalloc(m, &ly.w2, ne * d * m->Gf * 16));
        NX_TRY(dalloc(m, &ly.s2, ne * d * m->Gf));
        if (norms) {
            NX_TRY(dalloc(m, &ly.norm_attn, (size_t)d));
            NX_TRY(dalloc(m, &ly.norm_ffn, (size_t)d));
            if (c.qk_norm) {
                NX_TRY(dalloc(m, &ly.qnorm, (size_t)c.head_dim));
                NX_TRY(dalloc(m, &ly.knorm, (size_t)c.head_dim));
            }
        }
        if (E > 0) {
            NX_TRY(dalloc(m, &ly.wr, (size_t)E * m->Gd * 16));
            NX_TRY(dalloc(m, &ly.sr, (size_t)E * m->Gd));
            NX_TRY(dalloc(m, &ly.moe_count, (size_t)E));
        }
        if (c.kv_kind == 0) {
            NX_TRY(dalloc(m, &ly.kpool, pool_elems));
            NX_TRY(dalloc(m, &ly.vpool, pool_elems));
        }
        if (c.kv_kind == 2) {
            const size_t hot_elems = (size_t)B * m->hot_pages * c.n_kv_heads * nx::kPage * c.head_dim;
            NX_TRY(dalloc(m, &ly.kpool, hot_elems));
            NX_TRY(dalloc(m, &ly.vpool, hot_elems));
        }
        if (c.kv_kind != 0) {
            // three tiers: the TurboQuant pool holds only the Warm ring
            const size_t tq_vecs =
                m->warm_pages > 0 ? (size_t)B * m->warm_pages * c.n_kv_heads * nx::kPage : pool_vecs;
            NX_TRY(dalloc(m, &ly.kc4, tq_vecs * 32));
            NX_TRY(dalloc(m, &ly.kc3, tq_vecs * 24));
            NX_TRY(dalloc(m, &ly.vc4, tq_vecs * 32));
            NX_TRY(dalloc(m, &ly.vc3, tq_vecs * 24));
            NX_TRY(dalloc(m, &ly.kn, tq_vecs));
            NX_TRY(dalloc(m, &ly.vn, tq_vecs));
        }
        if (m->warm_pages > 0) {
            // with a Cool window the Cool pool holds only the Cool ring
            const size_t cool_vecs =
                m->cool_pages > 0 ? (size_t)B * m->cool_pages * c.n_kv_heads * nx::kPage : pool_vecs;
            NX_TRY(dalloc(m, &ly.kcc, cool_vecs * 48));
            NX_TRY(dalloc(m, &ly.vcc, cool_vecs * 48));
            NX_TRY(dalloc(m, &ly.kcn, cool_vecs));
            NX_TRY(dalloc(m, &ly.vcn, cool_vecs));
        }
        NX_TRY(dalloc(m, &ly.ksign, 128));
        NX_TRY(dalloc(m, &ly.vsign, 128));
        float sg[2][128];
        for (int kv = 0; kv < 2; ++kv) {
            const uint64_t key = nx::stream_key(c.seed, nx::tid_layer(l, kv ? nx::TQ_VSIGN : nx::TQ_KSIGN));
            for (int i = 0; i < 128; ++i) sg[kv][i] = (nx::rand_at(key, (uint64_t)i) & 1u) ? -1.0f : 1.0f;
        }
        NX_HIP(m->ctx, hipMemcpyAsync(ly.ksign, sg[0], sizeof(sg[0]), hipMemcpyHostToDevice, m->ctx->stream));
        NX_HIP(m->ctx, hipMemcpyAsync(ly.vsign, sg[1], sizeof(sg[1]), hipMemcpyHostToDevice, m->ctx->stream));
        NX_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    }
    // rope tables
    {
        const int half = c.head_dim / 2;
        std::vector<float> cs((size_t)c.max_seq * half), sn((size_t)c.max_seq * half);
        for (int p = 0; p < c.max_seq; ++p)
            for (int i = 0; i < half; ++i) {
                const double inv_freq = std::pow((double)c.rope_theta, -(2.0 * i) / (double)c.head_dim);
                const double ang = (double)p * inv_freq;
                cs[(size_t)p * half + i] = (float)std::cos(ang);
                sn[(size_t)p * half + i] = (float)std::sin(ang);
            }
        NX_TRY(dalloc(m, &m->rope_cos, cs.size()));
        NX_TRY(dalloc(m, &m->rope_sin, sn.size()));
        NX_HIP(m->ctx, hipMemcpyAsync(m->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, m->ctx->stream));
        NX_HIP(m->ctx, hipMemcpyAsync(m->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice, m->ctx->stream));
        NX_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    }
    // block table: a seeded permutation of the pool, max_blocks per sequence
    // (three tiers: the Cool table; the block table is the Warm ring); with a
    // shared pool every entry starts at the spare page and the free list is the
    // seeded permutation of the others
    {
        std::vector<int32_t> perm;
        host_shuffle(perm, m->n_blocks, c.seed, nx::kTidShuffle);
        if (c.kv_blocks > 0) {
            m->pool_trash = c.kv_blocks;
            m->free_pages.clear();
            for (int32_t blk : perm)
                if (blk != m->pool_trash) m->free_pages.push_back(blk);
            std::reverse(m->free_pages.begin(), m->free_pages.end());  // taken from the back
            m->owned.assign((size_t)B, {});
            perm.assign((size_t)B * m->max_blocks, m->pool_trash);
            m->h_table = perm;
        }
        if (m->warm_pages > 0) {
            std::vector<int32_t> cool = perm;
            if (m->cool_pages > 0)
                for (int b = 0; b < B; ++b)
                    for (int p = 0; p < m->max_blocks; ++p)
                        cool[(size_t)b * m->max_blocks + p] = b * m->cool_pages + p % m->cool_pages;
            NX_TRY(dalloc(m, &m->cool_bt, cool.size()));
            NX_HIP(m->ctx, hipMemcpyAsync(m->cool_bt, cool.data(), cool.size() * 4, hipMemcpyHostToDevice, m->ctx->stream));
            NX_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
            for (int b = 0; b < B; ++b)
                for (int p = 0; p < m->max_blocks; ++p)
                    perm[(size_t)b * m->max_blocks + p] = b * m->warm_pages + p % m->warm_pages;
        }
        NX_TRY(dalloc(m, &m->block_table, perm.size()));
        NX_HIP(m->ctx, hipMemcpyAsync(m->block_table, perm.data(), perm.size() * 4, hipMemcpyHostToDevice, m->ctx->stream));
        NX_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
        if (c.kv_blocks > 0) m->long_table = m->warm_pages > 0 ? m->cool_bt : m->block_table;
    }
    NX_TRY(dalloc(m, &m->pos, B));
    NX_TRY(dalloc(m, &m->base, B));
    NX_TRY(dalloc(m, &m->best, B));
    NX_TRY(dalloc(m, &m->out_tokens, (size_t)B * m->out_stride));
    NX_TRY(dalloc(m, &m->prompt, (size_t)B * c.max_seq));
    NX_TRY(dalloc(m, &m->h, (size_t)B * d));
    NX_TRY(dalloc(m, &m->q, (size_t)B * m->qdim));
    NX_TRY(dalloc(m, &m->att16, (size_t)B * m->qdim));
    NX_TRY(dalloc(m, &m->act16, (size_t)B * m->Fp));
    // K-part sums of the batch 2-8 down projection and of wo (both N = d)
    m->kparts_max = std::max(nx::gemv_kparts(c.ffn, B), nx::gemv_parts_for(m->qdim, B, m->wo_kparts));
    if (m->kparts_max > 0) NX_TRY(dalloc(m, &m->kpart, (size_t)m->kparts_max * B * d));
    NX_TRY(dalloc(m, &m->logits, (size_t)B * c.vocab));
    NX_TRY(dalloc(m, &m->kv_tmp, (size_t)B * 2 * m->kvdim));
    NX_TRY(dalloc(m, &m->xn16, (size_t)B * d));
    if (E > 0) {
        NX_TRY(dalloc(m, &m->router_logits, (size_t)B * E));
        NX_TRY(dalloc(m, &m->moe_ids, (size_t)B * c.top_k));
        NX_TRY(dalloc(m, &m->moe_w, (size_t)B * c.top_k));
        NX_TRY(dalloc(m, &m->moe_slots, (size_t)E * B * c.top_k));
        NX_TRY(dalloc(m, &m->moe_plan, (size_t)nx::moe_plan_rows(E, B, c.top_k) * nx::kMoePlanInts));
        NX_TRY(dalloc(m, &m->moe_counter, 64));
        NX_TRY(dalloc(m, &m->moe_act, (size_t)B * c.top_k * m->Fp));
        NX_TRY(dalloc(m, &m->moe_y, (size_t)B * c.top_k * d));
        if (nx::gemv_kparts(F, B) > 0)
            NX_TRY(dalloc(m, &m->moe_kpart, (size_t)nx::gemv_kparts(F, B) * B * c.top_k * d));
    }
    NX_TRY(dalloc(m, &m->attn_counts, nx::attn_count_words(B, c.n_kv_heads)));
    if (c.kv_kind == 2) {
        std::vector<int32_t> ring((size_t)B * m->max_blocks);
        for (int b = 0; b < B; ++b)
            for (int p = 0; p < m->max_blocks; ++p) ring[(size_t)b * m->max_blocks + p] = b * m->hot_pages + p % m->hot_pages;
        NX_TRY(dalloc(m, &m->hot_bt, ring.size()));
        NX_HIP(m->ctx, hipMemcpyAsync(m->hot_bt, ring.data(), ring.size() * 4, hipMemcpyHostToDevice, m->ctx->stream));
        NX_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    }
    NX_TRY(dalloc(m, &m->attn_part,
                  std::max(nx::attn_workspace_bytes(B, c.n_heads, c.n_kv_heads, c.head_dim, c.max_seq),
                           c.kv_kind == 2 ? nx::attn_tiered_workspace_bytes(B, c.n_heads, c.n_kv_heads) : 0) /
                          4 +
                      1));
    {
        std::vector<int32_t> minus1(B, -1);
        NX_HIP(m->ctx, hipMemcpyAsync(m->pos, minus1.data(), (size_t)B * 4, hipMemcpyHostToDevice, m->ctx->stream));
        NX_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    }
    NX_TRY(dalloc(m, &m->feed, (size_t)B));
    NX_TRY(dalloc(m, &m->fpos, (size_t)B));
    NX_HIP(m->ctx, hipHostMalloc((void**)&m->h_feed, sizeof(int32_t) * 2 * B, hipHostMallocDefault));
    m->active.assign((size_t)B, 1);
    NX_TRY(feed_decode(m));
    NX_HIP(m->ctx, hipHostMalloc((void**)&m->h_stage, sizeof(int32_t) * B, hipHostMallocDefault));
    NX_HIP(m->ctx, hipHostMalloc((void**)&m->h_out, sizeof(int32_t) * (size_t)B * m->out_stride, hipHostMallocDefault));
    if (synthetic) NX_TRY(generate_weights(m));
    NX_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    return NX_OK;
}

nx_status check_config(nx_ctx* ctx, const nx_model_config& c) {
    if (c.n_layers < 1 || c.d_model < 32 || c.n_heads < 1 || c.n_kv_heads < 1 || c.n_heads % c.n_kv_heads ||
        c.ffn < 2 || c.vocab < 2 || c.max_seq < nx::kPage || c.max_seq % nx::kPage || c.batch < 1 || c.batch > 8 ||
        c.kv_kind < 0 || c.kv_kind > 2 || c.eps <= 0.0f || c.rope_theta <= 0.0f ||
        !(c.norm_sigma >= 0.0f && c.norm_sigma < 1e3f) || (c.qk_norm != 0 && c.qk_norm != 1))
        return fail(ctx, NX_ERR_INVALID, "nx_model_create: invalid configuration");
    const int G = c.n_heads / c.n_kv_heads;
    if (G != 1 && G != 2 && G != 4 && G != 8) return fail(ctx, NX_ERR_UNSUPPORTED, "hq/hkv must be 1, 2, 4 or 8");
    if (c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256)
        return fail(ctx, NX_ERR_UNSUPPORTED, "head_dim must be 64, 128 or 256");
    if (c.kv_kind != 0 && c.head_dim != 128) return fail(ctx, NX_ERR_UNSUPPORTED, "TurboQuant pages need head_dim 128");
    if (c.kv_kind == 2 && (c.hot_window < nx::kPage || c.hot_window % nx::kPage || c.hot_window >= c.max_seq))
        return fail(ctx, NX_ERR_INVALID, "hot_window must be a positive multiple of 16 below max_seq");
    if (c.warm_window < 0 || c.warm_window % nx::kPage || (c.warm_window > 0 && c.kv_kind != 2))
        return fail(ctx, NX_ERR_INVALID, "warm_window must be 0 or (tiered pages) a positive multiple of 16");
    if (c.cool_window < 0 || c.cool_window % nx::kPage || (c.cool_window > 0 && c.warm_window == 0))
        return fail(ctx, NX_ERR_INVALID, "cool_window must be 0 or (with a warm_window) a positive multiple of 16");
    if (c.kv_blocks < 0 || c.kv_blocks > (1 << 24))
        return fail(ctx, NX_ERR_INVALID, "kv_blocks must be 0 (a full-length table per sequence) or a page count");
    if (c.kv_blocks > 0 && c.cool_window > 0)
        return fail(ctx, NX_ERR_INVALID, "kv_blocks: with a cool_window every table is a per-sequence ring");
    if (c.kv_kind == 2 && c.max_seq > nx::attn_max_ctx() / 2)
        return fail(ctx, NX_ERR_UNSUPPORTED, "max_seq above the tiered attention limit");
    if (c.d_model % 32 || (c.n_heads * c.head_dim) % 32) return fail(ctx, NX_ERR_UNSUPPORTED, "d_model and hq*hd must be multiples of 32");
    if (c.max_seq > nx::attn_max_ctx()) return fail(ctx, NX_ERR_UNSUPPORTED, "max_seq above the attention limit");
    // GEMV K: RMSNorm inputs (QKV, gate/up, lm_head: d_model) up to 14336,
    // fp16 inputs (wo: hq * hd, the dense down projection: ffn) up to 28672;
    // routed experts' down projection up to 14336
    if (c.d_model > 14336 || c.n_heads * c.head_dim > 28672 || c.ffn > (c.n_experts > 0 ? 14336 : 28672))
        return fail(ctx, NX_ERR_UNSUPPORTED, "GEMV K above its limit (d_model 14336, hq*hd 28672, ffn 28672)");
    if (c.n_experts < 0 || c.n_experts > nx::kMoeMaxExperts ||
        (c.n_experts > 0 && (c.top_k < 1 || c.top_k > nx::kMoeMaxTopK || c.top_k > c.n_experts)))
        return fail(ctx, NX_ERR_INVALID, "invalid expert configuration (experts <= 256, 1 <= top_k <= min(16, experts))");
    return NX_OK;
}

}  // namespace

extern "C" {

nx_status nx_model_create(nx_ctx* ctx, const nx_model_config* cfg, nx_model** out) {
    if (!ctx || !cfg || !out) return NX_ERR_INVALID;
    *out = nullptr;
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "nx_model_create inside a token batch");
    NX_TRY(check_config(ctx, *cfg));
    nx_model* m = new nx_model();
    m->ctx = ctx;
    m->c = *cfg;
    nx_status s = create_impl(m, true);
    if (s != NX_OK) {
        free_model(m);
        return s;
    }
    *out = m;
    return NX_OK;
}

nx_status nx_model_destroy(nx_model* m) {
    if (!m) return NX_ERR_INVALID;
    return free_model(m);
}

}  // extern "C"

namespace {

constexpr int kPrefillChunk = 2048;  // prompt tokens per pass through the layers (each weight read once per pass)

// Device scratch of one prefill call, released on every exit path.
struct PrefillScratch {
    std::vector<void*> p;
    ~PrefillScratch() {
        for (void* q : p) (void)hipFree(q);
    }
    template <class T>
    hipError_t get(T** out, size_t count) {
        void* q = nullptr;
        hipError_t e = hipMalloc(&q, std::max<size_t>(count * sizeof(T), 16));
        if (e == hipSuccess) p.push_back(q);
        *out = static_cast<T*>(q);
        return e;
    }
};

// The prompt of sequence b (P tokens, at positions hpos[b] + 1 on) through
// every layer, kPrefillChunk tokens at a time: RMSNorm rows, QKV GEMM, RoPE
// and page writes, causal attention over the pages (16 queries per
// wavefront), output projection and FFN GEMMs with the residual accumulated
// in place.  Then the final RMSNorm,
// lm_head and argmax of the last token leave its greedy successor pending,
// as after P decode steps.  Dense models.  TurboQuant pages (kv_kind 1):
// the chunk's K and V rows are encoded into the pages, and the attention runs
// over the sequence's pages decoded to fp16 (positions up to the chunk's
// last), so every query sees the stored (quantized) K and V of the positions
// before it and of its own, as the decode steps would.  Tiered pages
// (kv_kind 2, two tiers): per layer and chunk, the positions not yet
// TurboQuant (the window's ring before the chunk, the chunk's rows rounded
// to fp16) go to fp16 pages of the block table, those the decode steps up
// to the chunk's last position would have compressed are encoded into the
// TurboQuant pages, the window's last pages into the ring; the attention
// reads each page-aligned query tile's pages before its cold boundary from
// the decoded TurboQuant pages and the rest as fp16, as the decode step at
// that position would.
// Models the batched prefill takes: dense or MoE, fp16, TurboQuant or
// two-tier tiered pages.
bool batched_prefill_ok(const nx_model* m) {
    const nx_model_config& c = m->c;
    // (tiered pages with a Warm range, whose TurboQuant pages are a ring of
    // their own, prefill one step per token)
    return m->prefill_batched && (c.kv_kind == 0 || c.kv_kind == 1 || (c.kv_kind == 2 && c.warm_window == 0));
}

nx_status prefill_batched(nx_model* m, int b, const int32_t* tokens, int P) {
    const nx_model_config& c = m->c;
    nx_ctx* ctx = m->ctx;
    hipStream_t st = ctx->stream;
    const int d = c.d_model, F = c.ffn, hq = c.n_heads, hkv = c.n_kv_heads, hd = c.head_dim;
    const int C = std::min(P, kPrefillChunk), p0 = m->hpos[(size_t)b] + 1, MB = m->max_blocks;
    const int pend = p0 + P;  // first position after the prompt
    PrefillScratch sc;
    int32_t* tok = nullptr;
    float *h = nullptr, *qkv = nullptr, *q = nullptr;
    uint16_t *x16 = nullptr, *att = nullptr, *act = nullptr;
    if (sc.get(&tok, C) != hipSuccess || sc.get(&h, (size_t)C * d) != hipSuccess ||
        sc.get(&qkv, (size_t)C * m->nqkv) != hipSuccess || sc.get(&q, (size_t)C * m->qdim) != hipSuccess ||
        sc.get(&x16, (size_t)C * d) != hipSuccess || sc.get(&att, (size_t)C * m->qdim) != hipSuccess ||
        sc.get(&act, (size_t)C * m->Fp) != hipSuccess)
        return fail(ctx, NX_ERR_OOM, "prefill: scratch for %d tokens", C);
    // MoE layers: router logits, routing, token slots grouped by expert
    // (gathered x rows, their activations and outputs)
    const int E = c.n_experts, kx = c.top_k, S = C * std::max(kx, 1);
    float *rlog = nullptr, *rw = nullptr, *yg = nullptr;
    int32_t *rid = nullptr, *row_tok = nullptr, *slot_row = nullptr, *counts = nullptr;
    uint16_t *xg = nullptr, *actg = nullptr;
    if (E > 0 && (sc.get(&rlog, (size_t)C * E) != hipSuccess || sc.get(&rw, (size_t)S) != hipSuccess ||
                  sc.get(&rid, (size_t)S) != hipSuccess || sc.get(&row_tok, (size_t)S) != hipSuccess ||
                  sc.get(&slot_row, (size_t)S) != hipSuccess || sc.get(&counts, (size_t)2 * E) != hipSuccess ||
                  sc.get(&xg, (size_t)S * d) != hipSuccess || sc.get(&actg, (size_t)S * m->Fp) != hipSuccess ||
                  sc.get(&yg, (size_t)S * d) != hipSuccess))
        return fail(ctx, NX_ERR_OOM, "prefill: expert scratch for %d tokens", C);
    std::vector<int32_t> hcounts((size_t)2 * std::max(E, 1));
    const bool tq = c.kv_kind == 1, tier = c.kv_kind == 2;
    float* kvrows = nullptr;
    uint16_t *k16 = nullptr, *k16lo = nullptr, *v16 = nullptr;  // decoded pages (every block of the pool)
    uint16_t *wk = nullptr, *wv = nullptr, *zlo = nullptr;      // tiered: fp16 pages, a page of zeros
    if (tq || tier) {
        const size_t pool = (size_t)m->n_blocks * hkv * nx::kPage * hd;
        if (sc.get(&kvrows, (size_t)C * 2 * m->kvdim) != hipSuccess || sc.get(&k16, pool) != hipSuccess ||
            sc.get(&k16lo, pool) != hipSuccess || sc.get(&v16, pool) != hipSuccess)
            return fail(ctx, NX_ERR_OOM, "prefill: decoded pages");
        if (tier) {
            if (sc.get(&wk, pool) != hipSuccess || sc.get(&wv, pool) != hipSuccess ||
                sc.get(&zlo, (size_t)nx::kPage * hd) != hipSuccess)
                return fail(ctx, NX_ERR_OOM, "prefill: fp16 pages");
            NX_HIP(ctx, hipMemsetAsync(zlo, 0, (size_t)nx::kPage * hd * sizeof(uint16_t), st));
        }
    }
    // tiered pages: positions that are TurboQuant once the positions before p
    // are written (the pages the decode steps have compressed by then)
    auto tq_upto = [&](int p) { return p >= c.hot_window ? nx::kPage * ((p - c.hot_window) / nx::kPage) : 0; };
    int last = 0;
    for (int done = 0; done < P; done += C) {
        const int n = std::min(C, P - done), pb = p0 + done;
        NX_HIP(ctx, hipMemcpyAsync(tok, tokens + done, (size_t)n * 4, hipMemcpyHostToDevice, st));
        NX_LAUNCH(m, nx::pf_embed_launch(tok, n, m->embed, h, d, c.vocab, st));
        for (int L = 0; L < c.n_layers; ++L) {
            Layer& ly = m->layers[(size_t)L];
            NX_LAUNCH(m, nx::rmsnorm_launch(h, ly.norm_attn, x16, d, c.eps, n, st));
            nx::PfGemmArgs g{};
            g.x = x16;
            g.ldx = d;
            g.W = ly.wqkv;
            g.S = ly.sqkv;
            g.M = n;
            g.N = m->nqkv;
            g.K = d;
            g.G = m->Gd;
            g.y32 = qkv;
            g.ldy = m->nqkv;
            NX_LAUNCH(m, nx::pf_gemm_launch(nx::PF_F32, g, st));
            if (c.qk_norm)  // per-head Q/K RMSNorm of the chunk's rows, before RoPE
                NX_LAUNCH(m, nx::head_rmsnorm_launch(qkv, m->nqkv, qkv + m->qdim, m->nqkv, n, hq, hkv, hd, ly.qnorm,
                                                     ly.knorm, c.eps, st));
            const int32_t* bt = m->block_table + (size_t)b * MB;
            NX_LAUNCH(m, nx::pf_rope_kv_launch(qkv, m->nqkv, n, pb, m->qdim, m->kvdim, hd, hkv, m->rope_cos, m->rope_sin,
                                               bt, ly.kpool, ly.vpool, q, st, kvrows));
            if (tier) {
                const int pe = pb + n, lo = tq_upto(pb), tq_hi = tq_upto(pe);
                // the ring's pages at the chunk's end: the last hot_pages
                const int ring_lo = std::max(pb, nx::kPage * ((pe - 1) / nx::kPage - m->hot_pages + 1));
                NX_LAUNCH(m, nx::pf_tier_rows_launch(kvrows, pb, lo, pe, tq_hi, ring_lo, hkv, b, m->block_table, m->hot_bt,
                                                     MB, ly.kpool, ly.vpool, wk, wv, ly.ksign, ly.vsign, ly.kc4, ly.kc3,
                                                     ly.kn, ly.vc4, ly.vc3, ly.vn, st));
                NX_LAUNCH(m, nx::tq_decode_pages_launch(ly.kc4, ly.kc3, ly.kn, ly.vc4, ly.vc3, ly.vn, ly.ksign,
                                                        ly.vsign, bt, tq_hi, hkv, k16, v16, k16lo, st));
            }
            if (tq) {
                NX_LAUNCH(m, nx::tq_encode_rows_launch(kvrows, n, pb, hkv, ly.ksign, ly.vsign, ly.kc4, ly.kc3, ly.kn,
                                                       ly.vc4, ly.vc3, ly.vn, bt, st));
                NX_LAUNCH(m, nx::tq_decode_pages_launch(ly.kc4, ly.kc3, ly.kn, ly.vc4, ly.vc3, ly.vn, ly.ksign,
                                                        ly.vsign, bt, pb + n, hkv, k16, v16, k16lo, st));
            }
            nx::AttnArgs at{};
            at.q = q;
            at.kpool = tq || tier ? k16 : ly.kpool;
            at.vpool = tq || tier ? v16 : ly.vpool;
            at.kpool_lo = tq || tier ? k16lo : nullptr;
            if (tier) {
                at.kpool_win = wk;
                at.vpool_win = wv;
                at.lo_zero = zlo;
                at.hot_window = c.hot_window;
            }
            at.block_table = m->block_table + (size_t)b * MB;
            at.out16 = att;
            at.batch = 1;
            at.hq = hq;
            at.hkv = hkv;
            at.hd = hd;
            at.max_blocks = MB;
            at.max_ctx = pend;
            NX_LAUNCH(m, nx::attn_prefill_launch(at, pb, n, st));
            nx::PfGemmArgs o{};
            o.x = att;
            o.ldx = m->qdim;
            o.W = ly.wo;
            o.S = ly.so;
            o.M = n;
            o.N = d;
            o.K = m->qdim;
            o.G = m->Gq;
            o.y32 = h;
            o.ldy = d;
            NX_LAUNCH(m, nx::pf_gemm_launch(nx::PF_ACC, o, st));
            NX_LAUNCH(m, nx::rmsnorm_launch(h, ly.norm_ffn, x16, d, c.eps, n, st));
            if (E > 0) {
                // router GEMM, routing as the decode step routes, then each
                // active expert's gate/up and down GEMMs over its gathered
                // token rows, and the weighted combine into h
                nx::PfGemmArgs r{};
                r.x = x16;
                r.ldx = d;
                r.W = ly.wr;
                r.S = ly.sr;
                r.M = n;
                r.N = E;
                r.K = d;
                r.G = m->Gd;
                r.y32 = rlog;
                r.ldy = E;
                NX_LAUNCH(m, nx::pf_gemm_launch(nx::PF_F32, r, st));
                NX_LAUNCH(m, nx::pf_route_launch(rlog, n, E, kx, rid, rw, row_tok, slot_row, counts, st));
                NX_LAUNCH(m, nx::pf_gather_launch(x16, row_tok, n * kx, d, xg, st));
                NX_HIP(ctx, hipMemcpyAsync(hcounts.data(), counts, (size_t)2 * E * 4, hipMemcpyDeviceToHost, st));
                NX_HIP(ctx, hipStreamSynchronize(st));
                for (int e = 0; e < E; ++e) {
                    const int ne = hcounts[(size_t)e], oe = hcounts[(size_t)E + e];
                    if (ne == 0) continue;
                    nx::PfGemmArgs f{};
                    f.x = xg + (size_t)oe * d;
                    f.ldx = d;
                    f.W = ly.w13 + (size_t)e * 2 * F * m->Gd * 16;
                    f.S = ly.s13 + (size_t)e * 2 * F * m->Gd;
                    f.M = ne;
                    f.N = 2 * F;
                    f.K = d;
                    f.G = m->Gd;
                    f.act16 = actg + (size_t)oe * m->Fp;
                    f.lda = m->Fp;
                    NX_LAUNCH(m, nx::pf_gemm_launch(nx::PF_SWIGLU, f, st));
                    nx::PfGemmArgs dn{};
                    dn.x = actg + (size_t)oe * m->Fp;
                    dn.ldx = m->Fp;
                    dn.W = ly.w2 + (size_t)e * d * m->Gf * 16;
                    dn.S = ly.s2 + (size_t)e * d * m->Gf;
                    dn.M = ne;
                    dn.N = d;
                    dn.K = F;
                    dn.G = m->Gf;
                    dn.y32 = yg + (size_t)oe * d;
                    dn.ldy = d;
                    NX_LAUNCH(m, nx::pf_gemm_launch(nx::PF_F32, dn, st));
                }
                NX_LAUNCH(m, nx::pf_moe_combine_launch(yg, slot_row, rw, n, kx, d, h, st));
                continue;
            }
            nx::PfGemmArgs f{};
            f.x = x16;
            f.ldx = d;
            f.W = ly.w13;
            f.S = ly.s13;
            f.M = n;
            f.N = 2 * F;
            f.K = d;
            f.G = m->Gd;
            f.act16 = act;
            f.lda = m->Fp;
            NX_LAUNCH(m, nx::pf_gemm_launch(nx::PF_SWIGLU, f, st));
            nx::PfGemmArgs dn{};
            dn.x = act;
            dn.ldx = m->Fp;
            dn.W = ly.w2;
            dn.S = ly.s2;
            dn.M = n;
            dn.N = d;
            dn.K = F;
            dn.G = m->Gf;
            dn.y32 = h;
            dn.ldy = d;
            NX_LAUNCH(m, nx::pf_gemm_launch(nx::PF_ACC, dn, st));
        }
        last = n - 1;
        NX_HIP(ctx, hipStreamSynchronize(st));  // the token staging is refilled next
    }
    // the last prompt token: final RMSNorm, lm_head and argmax into best[b]
    NX_HIP(ctx, hipMemsetAsync(m->best + b, 0, sizeof(unsigned long long), st));
    nx::GemvArgs lm{};
    lm.W = m->lm_w;
    lm.S = m->lm_s;
    lm.N = c.vocab;
    lm.K = d;
    lm.G = m->Gd;
    lm.batch = 1;
    lm.h32 = h + (size_t)last * d;
    lm.ldx = d;
    lm.eps = c.eps;
    lm.norm_w = m->norm_final;
    lm.y32 = m->logits + (size_t)b * c.vocab;
    lm.ldy = c.vocab;
    lm.best = m->best + b;
    NX_LAUNCH(m, nx::gemv_launch(nx::X_RMSNORM, nx::E_LOGITS, lm, st));
    const int32_t plast = pend - 1;
    if (m->temperature > 0.0f) {
        NX_HIP(ctx, hipMemcpyAsync(m->pos + b, &plast, 4, hipMemcpyHostToDevice, st));  // the draw's key
        NX_TRY(enqueue_sample(m, b, 1));
    }
    NX_HIP(ctx, hipMemcpyAsync(m->pos + b, &plast, 4, hipMemcpyHostToDevice, st));
    NX_HIP(ctx, hipStreamSynchronize(st));
    m->hpos[(size_t)b] = plast;
    return NX_OK;
}

}  // namespace

extern "C" {

nx_status nx_model_set_sampling(nx_model* m, float temperature, int top_k, float top_p, uint64_t seed) {
    if (!m) return NX_ERR_INVALID;
    const int V = m->c.vocab;
    if (temperature > 0.0f) {
        if (top_k < 0 || !(top_p > 0.0f) || top_p > 1.0f) return fail(m->ctx, NX_ERR_INVALID, "sampling: bad parameters");
    }
    if (temperature > 0.0f && !m->smp_scratch)
        NX_TRY(dalloc(m, &m->smp_scratch, (size_t)m->c.batch * ((size_t)V + nx::kSmpPartFloats)));
    m->temperature = temperature > 0.0f ? temperature : 0.0f;
    m->top_k = top_k;
    m->top_p = top_p;
    m->u_fixed = seed ? nx::sample_draw(seed) : -1.0f;
    // the step graphs hold the sampling launch (or not): capture them again
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->exec_multi) (void)hipGraphExecDestroy(m->exec_multi);
    m->exec = nullptr;
    m->exec_multi = nullptr;
    return NX_OK;
}

nx_status nx_model_set_prefill(nx_model* m, int batched) {
    if (!m || (batched != 0 && batched != 1)) return NX_ERR_INVALID;
    m->prefill_batched = batched;
    return NX_OK;
}

nx_status nx_model_prefill(nx_model* m, const int32_t* prompt, int P, int32_t* next_tokens) {
    if (!m || !prompt || P < 1) return NX_ERR_INVALID;
    const nx_model_config& c = m->c;
    const int B = c.batch;
    for (int b = 0; b < B; ++b) {
        if (m->hpos[b] + P >= c.max_seq) return fail(m->ctx, NX_ERR_CAPACITY, "prefill exceeds max_seq");
        for (int i = 0; i < P; ++i)
            if (prompt[(size_t)b * P + i] < 0 || prompt[(size_t)b * P + i] >= c.vocab)
                return fail(m->ctx, NX_ERR_INVALID, "prompt token out of vocabulary");
    }
    {
        std::vector<int> want((size_t)B);
        for (int b = 0; b < B; ++b) want[(size_t)b] = m->hpos[(size_t)b] + P;
        NX_TRY(pool_ensure(m, want));
    }
    for (int b = 0; b < B; ++b) m->active[(size_t)b] = 1;
    if (batched_prefill_ok(m)) {
        for (int b = 0; b < B; ++b) NX_TRY(prefill_batched(m, b, prompt + (size_t)b * P, P));
        if (next_tokens) NX_TRY(nx_model_pending(m, next_tokens));
        return NX_OK;
    }
    NX_TRY(ensure_graph(m));
    NX_TRY(feed_decode(m));
    hipStream_t st = m->ctx->stream;
    // token-major copy of the prompt: prompt_dev[i][b]
    std::vector<int32_t> tm((size_t)P * B);
    for (int b = 0; b < B; ++b)
        for (int i = 0; i < P; ++i) tm[(size_t)i * B + b] = prompt[(size_t)b * P + i];
    NX_HIP(m->ctx, hipMemcpyAsync(m->prompt, tm.data(), tm.size() * 4, hipMemcpyHostToDevice, st));
    // nothing is recorded while prefilling
    for (int b = 0; b < B; ++b) m->h_stage[b] = 1 << 30;
    NX_HIP(m->ctx, hipMemcpyAsync(m->base, m->h_stage, (size_t)B * 4, hipMemcpyHostToDevice, st));
    NX_HIP(m->ctx, hipStreamSynchronize(st));
    for (int i = 0; i < P; ++i) {
        NX_LAUNCH(m, nx::set_tokens_launch(m->best, m->prompt + (size_t)i * B, B, st));
        NX_HIP(m->ctx, hipGraphLaunch(m->exec, st));
    }
    std::vector<unsigned long long> best(B);
    NX_HIP(m->ctx, hipMemcpyAsync(best.data(), m->best, (size_t)B * 8, hipMemcpyDeviceToHost, st));
    NX_HIP(m->ctx, hipStreamSynchronize(st));
    for (int b = 0; b < B; ++b) {
        m->hpos[b] += P;
        if (next_tokens) next_tokens[b] = (int32_t)(0xFFFFFFFFu - (uint32_t)(best[b] & 0xFFFFFFFFull));
    }
    return NX_OK;
}

nx_status nx_model_fill_context(nx_model* m, int ctx_len, int n_outlier) {
    if (!m) return NX_ERR_INVALID;
    const nx_model_config& c = m->c;
    if (ctx_len < 1 || ctx_len >= c.max_seq) return fail(m->ctx, NX_ERR_CAPACITY, "context must leave room in max_seq");
    if (n_outlier < 0 || n_outlier > 16 || n_outlier > c.head_dim) return fail(m->ctx, NX_ERR_INVALID, "n_outlier out of range");
    hipStream_t st = m->ctx->stream;
    const int hkv = c.n_kv_heads, hd = c.head_dim, B = c.batch;
    // every sequence starts over with ctx_len positions (a shared pool: its
    // pages for them)
    for (int b = 0; b < B; ++b) NX_TRY(pool_release(m, b));
    NX_TRY(pool_ensure(m, std::vector<int>((size_t)B, ctx_len - 1)));
    const float k1 = nx::normal_k(1.0);
    int32_t* och = nullptr;
    NX_TRY(dalloc(m, &och, (size_t)2 * hkv * (n_outlier > 0 ? n_outlier : 1)));
    float* raw = nullptr;
    if (c.kv_kind != 0) NX_TRY(dalloc(m, &raw, (size_t)ctx_len * hkv * hd));
    int cool = 0, cold = 0, evict = 0;
    tier_bounds(c, ctx_len + 1, cool, cold, evict);  // the boundaries of the first decode step
    cold = std::min(cold, ctx_len);  // TurboQuant pages: every filled position (raw holds ctx_len rows)
    std::vector<int32_t> ho((size_t)2 * hkv * (n_outlier > 0 ? n_outlier : 1));
    for (int L = 0; L < c.n_layers; ++L) {
        Layer& ly = m->layers[L];
        for (int kv = 0; kv < 2; ++kv)
            for (int h = 0; h < hkv; ++h) {
                std::vector<int32_t> perm;
                host_shuffle(perm, hd, c.seed, nx::tid_outlier(L, kv, h));
                for (int j = 0; j < n_outlier; ++j) ho[((size_t)kv * hkv + h) * n_outlier + j] = perm[j];
            }
        NX_HIP(m->ctx, hipMemcpyAsync(och, ho.data(), ho.size() * 4, hipMemcpyHostToDevice, st));
        if (c.kv_kind == 0) {
            NX_LAUNCH(m, nx::gen_ctx_f16_launch(ly.kpool, ly.vpool, m->block_table, m->max_blocks, B, ctx_len, hkv, hd, L,
                                                c.seed, k1, och, n_outlier, st));
        } else {
            // tiered: the values rounded to fp16 (what the window holds), the
            // pages in [evict, cool) encoded Cool, those in [cool, cold)
            // encoded, the rest into the window's ring
            for (int b = 0; b < B; ++b)
                for (int kv = 0; kv < 2; ++kv) {
                    NX_LAUNCH(m, nx::gen_ctx_raw_launch(raw, ctx_len, hkv, hd, L, b, kv, c.seed, k1,
                                                        och + (size_t)kv * hkv * n_outlier, n_outlier, st));
                    if (c.kv_kind == 2) NX_LAUNCH(m, nx::round_f16_launch(raw, (size_t)ctx_len * hkv * hd, st));
                    if (cool > evict)
                        NX_LAUNCH(m, nx::cool_encode_ctx_launch(raw, evict, cool, hkv, kv ? ly.vsign : ly.ksign,
                                                                kv ? ly.vcc : ly.kcc, kv ? ly.vcn : ly.kcn, m->cool_bt,
                                                                m->max_blocks, b, st));
                    if (cold > cool)
                        NX_LAUNCH(m, nx::tq_encode_ctx_launch(raw, cold, hkv, kv ? ly.vsign : ly.ksign, nullptr, nullptr,
                                                              kv ? ly.vc4 : ly.kc4, kv ? ly.vc3 : ly.kc3,
                                                              kv ? ly.vn : ly.kn, m->block_table, m->max_blocks, b, st,
                                                              cool));
                    if (c.kv_kind == 2)
                        NX_LAUNCH(m, nx::put_hot_launch(raw, ctx_len, cold, hkv, hd, b, m->hot_bt, m->max_blocks,
                                                        ly.kpool, ly.vpool, kv, st));
                }
        }
        NX_HIP(m->ctx, hipStreamSynchronize(st));
    }
    // positions and the seeded start tokens
    std::vector<int32_t> p(B, ctx_len - 1), start(B);
    const uint64_t key = nx::stream_key(c.seed, nx::kTidStart);
    for (int b = 0; b < B; ++b) start[b] = (int32_t)(nx::rand_at(key, (uint64_t)b) % (uint64_t)c.vocab);
    NX_HIP(m->ctx, hipMemcpyAsync(m->pos, p.data(), (size_t)B * 4, hipMemcpyHostToDevice, st));
    NX_HIP(m->ctx, hipMemcpyAsync(m->prompt, start.data(), (size_t)B * 4, hipMemcpyHostToDevice, st));
    NX_LAUNCH(m, nx::set_tokens_launch(m->best, m->prompt, B, st));
    NX_HIP(m->ctx, hipStreamSynchronize(st));
    for (int b = 0; b < B; ++b) {
        m->hpos[b] = ctx_len - 1;
        m->active[(size_t)b] = 1;
    }
    // the scratch buffers are released with the model; drop them now
    for (void* ptr : {static_cast<void*>(och), static_cast<void*>(raw)}) {
        if (!ptr) continue;
        for (auto it = m->allocs.begin(); it != m->allocs.end(); ++it)
            if (*it == ptr) {
                (void)hipFree(ptr);
                m->allocs.erase(it);
                break;
            }
    }
    return NX_OK;
}

nx_status nx_model_kv_read(nx_model* m, int layer, int b, int pos, int kv, int* form, void* out, size_t cap) {
    if (!m || !form || !out) return NX_ERR_INVALID;
    const nx_model_config& c = m->c;
    if (layer < 0 || layer >= c.n_layers || b < 0 || b >= c.batch || kv < 0 || kv > 1 || pos < 0 ||
        pos > m->hpos[(size_t)b])
        return fail(m->ctx, NX_ERR_INVALID, "nx_model_kv_read: no such position");
    const int hkv = c.n_kv_heads, hd = c.head_dim, page = pos / nx::kPage, slot = pos % nx::kPage;
    int cool = 0, cold = 0, evict = 0;
    tier_bounds(c, m->hpos[(size_t)b] + 2, cool, cold, evict);  // the boundaries of the next decode step
    *form = pos < evict ? 3 : pos < cool ? 2 : pos < cold ? 1 : 0;
    if (*form == 3) return NX_OK;  // evicted: nothing stored
    const size_t need = *form == 2 ? (size_t)50 * hkv : *form ? (size_t)58 * hkv : (size_t)2 * hkv * hd;
    if (cap < need) return fail(m->ctx, NX_ERR_INVALID, "nx_model_kv_read: %zu bytes needed", need);
    const Layer& ly = m->layers[layer];
    hipStream_t st = m->ctx->stream;
    uint8_t* dst = static_cast<uint8_t*>(out);
    int32_t blk = 0;
    const int32_t* bt = *form == 2 ? m->cool_bt : *form || c.kv_kind == 0 ? m->block_table : m->hot_bt;
    NX_HIP(m->ctx, hipMemcpyAsync(&blk, bt + (size_t)b * m->max_blocks + page, 4, hipMemcpyDeviceToHost, st));
    NX_HIP(m->ctx, hipStreamSynchronize(st));
    for (int h = 0; h < hkv; ++h) {
        if (*form == 2) {
            const size_t vi = ((size_t)blk * hkv + h) * nx::kPage + slot;
            uint8_t* o = dst + (size_t)50 * h;
            NX_HIP(m->ctx, hipMemcpyAsync(o, (kv ? ly.vcc : ly.kcc) + vi * 48, 48, hipMemcpyDeviceToHost, st));
            NX_HIP(m->ctx, hipMemcpyAsync(o + 48, (kv ? ly.vcn : ly.kcn) + vi, 2, hipMemcpyDeviceToHost, st));
        } else if (*form) {
            const size_t vi = ((size_t)blk * hkv + h) * nx::kPage + slot;
            uint8_t* o = dst + (size_t)58 * h;
            NX_HIP(m->ctx, hipMemcpyAsync(o, (kv ? ly.vc4 : ly.kc4) + vi * 32, 32, hipMemcpyDeviceToHost, st));
            NX_HIP(m->ctx, hipMemcpyAsync(o + 32, (kv ? ly.vc3 : ly.kc3) + vi * 24, 24, hipMemcpyDeviceToHost, st));
            NX_HIP(m->ctx, hipMemcpyAsync(o + 56, (kv ? ly.vn : ly.kn) + vi, 2, hipMemcpyDeviceToHost, st));
        } else {
            // K pages are token-major [16][hd], V pages dimension-major [hd][16]
            const uint16_t* pg = (kv ? ly.vpool : ly.kpool) + ((size_t)blk * hkv + h) * nx::kPage * hd;
            uint16_t* o = reinterpret_cast<uint16_t*>(dst) + (size_t)h * hd;
            if (kv)
                NX_HIP(m->ctx, hipMemcpy2DAsync(o, 2, pg + slot, 2 * nx::kPage, 2, hd, hipMemcpyDeviceToHost, st));
            else
                NX_HIP(m->ctx, hipMemcpyAsync(o, pg + (size_t)slot * hd, 2 * (size_t)hd, hipMemcpyDeviceToHost, st));
        }
    }
    NX_HIP(m->ctx, hipStreamSynchronize(st));
    return NX_OK;
}

nx_status nx_model_pending(nx_model* m, int32_t* tokens) {
    if (!m || !tokens) return NX_ERR_INVALID;
    std::vector<unsigned long long> best(m->c.batch);
    NX_HIP(m->ctx, hipMemcpyAsync(best.data(), m->best, best.size() * 8, hipMemcpyDeviceToHost, m->ctx->stream));
    NX_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    for (int b = 0; b < m->c.batch; ++b) tokens[b] = (int32_t)(0xFFFFFFFFu - (uint32_t)(best[b] & 0xFFFFFFFFull));
    return NX_OK;
}

nx_status nx_model_decode(nx_model* m, int steps, int32_t* out_tokens) {
    if (!m || steps < 1) return NX_ERR_INVALID;
    const nx_model_config& c = m->c;
    const int B = c.batch;
    int nact = 0;
    for (int b = 0; b < B; ++b) {
        if (!m->active[b]) continue;
        ++nact;
        if (m->hpos[b] < 0) return fail(m->ctx, NX_ERR_STATE, "decode before prefill or fill_context");
        if (m->hpos[b] + steps >= c.max_seq) return fail(m->ctx, NX_ERR_CAPACITY, "decode exceeds max_seq");
    }
    if (nact == 0) return fail(m->ctx, NX_ERR_STATE, "decode with no active sequence");
    if (steps > m->out_stride) return fail(m->ctx, NX_ERR_CAPACITY, "too many steps for one call");
    {
        std::vector<int> want((size_t)B, -1);
        for (int b = 0; b < B; ++b)
            if (m->active[(size_t)b]) want[(size_t)b] = m->hpos[(size_t)b] + steps;
        NX_TRY(pool_ensure(m, want));
    }
    NX_TRY(ensure_graph(m));
    NX_TRY(feed_decode(m));
    hipStream_t st = m->ctx->stream;
    for (int b = 0; b < B; ++b) m->h_stage[b] = m->active[b] ? m->hpos[b] + 1 : 1 << 30;
    NX_HIP(m->ctx, hipMemcpyAsync(m->base, m->h_stage, (size_t)B * 4, hipMemcpyHostToDevice, st));
    int s = 0;
    for (; s + kStepsPerGraph <= steps; s += kStepsPerGraph) NX_HIP(m->ctx, hipGraphLaunch(m->exec_multi, st));
    for (; s < steps; ++s) NX_HIP(m->ctx, hipGraphLaunch(m->exec, st));
    NX_LAUNCH(m, nx::finish_tokens_launch(m->best, m->pos, m->base, m->out_tokens, m->out_stride, B, st));
    if (out_tokens)
        NX_HIP(m->ctx, hipMemcpyAsync(m->h_out, m->out_tokens, (size_t)B * m->out_stride * 4, hipMemcpyDeviceToHost, st));
    NX_HIP(m->ctx, hipStreamSynchronize(st));
    for (int b = 0; b < B; ++b) {
        if (m->active[b]) m->hpos[b] += steps;
        if (!out_tokens) continue;
        if (m->active[b])
            std::memcpy(out_tokens + (size_t)b * steps, m->h_out + (size_t)b * m->out_stride, (size_t)steps * 4);
        else
            std::fill(out_tokens + (size_t)b * steps, out_tokens + (size_t)(b + 1) * steps, -1);
    }
    return NX_OK;
}

nx_status nx_model_get_config(nx_model* m, nx_model_config* out) {
    if (!m || !out) return NX_ERR_INVALID;
    *out = m->c;
    return NX_OK;
}

nx_ctx* nx_model_context(nx_model* m) { return m ? m->ctx : nullptr; }

nx_status nx_model_retire(nx_model* m, int slot) {
    if (!m || slot < 0 || slot >= m->c.batch) return NX_ERR_INVALID;
    m->active[(size_t)slot] = 0;
    return pool_release(m, slot);
}

nx_status nx_model_kv_pages(nx_model* m, int* total, int* free_pages) {
    if (!m) return NX_ERR_INVALID;
    const bool shared = m->c.kv_blocks > 0;
    if (total) *total = shared ? m->c.kv_blocks : m->max_blocks * m->c.batch;
    if (free_pages) {
        int used = 0;
        if (!shared)
            for (int b = 0; b < m->c.batch; ++b) used += m->hpos[(size_t)b] >= 0 ? m->hpos[(size_t)b] / nx::kPage + 1 : 0;
        *free_pages = shared ? (int)m->free_pages.size() : m->max_blocks * m->c.batch - used;
    }
    return NX_OK;
}

nx_status nx_model_slot_active(nx_model* m, int slot, int* active) {
    if (!m || !active || slot < 0 || slot >= m->c.batch) return NX_ERR_INVALID;
    *active = m->active[(size_t)slot] ? 1 : 0;
    return NX_OK;
}

nx_status nx_model_admit(nx_model* m, int slot, const int32_t* prompt, int P, int32_t* next_token) {
    if (!m || !prompt || P < 1 || slot < 0 || slot >= m->c.batch) return NX_ERR_INVALID;
    const nx_model_config& c = m->c;
    const int B = c.batch;
    if (P >= c.max_seq) return fail(m->ctx, NX_ERR_CAPACITY, "admit: prompt of %d exceeds max_seq", P);
    for (int i = 0; i < P; ++i)
        if (prompt[i] < 0 || prompt[i] >= c.vocab) return fail(m->ctx, NX_ERR_INVALID, "prompt token out of vocabulary");
    hipStream_t st = m->ctx->stream;
    // the slot starts over: position -1, its pages are overwritten from
    // position 0 (a shared pool: its pages go back, the prompt's are taken)
    m->active[(size_t)slot] = 0;
    m->hpos[(size_t)slot] = -1;
    NX_TRY(pool_release(m, slot));
    {
        std::vector<int> want((size_t)B, -1);
        want[(size_t)slot] = P - 1;
        NX_TRY(pool_ensure(m, want));
    }
    const int32_t minus1 = -1;
    NX_HIP(m->ctx, hipMemcpyAsync(m->pos + slot, &minus1, 4, hipMemcpyHostToDevice, st));
    NX_HIP(m->ctx, hipStreamSynchronize(st));
    if (batched_prefill_ok(m)) {
        // the slot's prompt alone through the batched prefill
        NX_TRY(prefill_batched(m, slot, prompt, P));
    } else {
        // one step per prompt token for this slot; the other active sequences
        // are held (each step writes a position they have not reached, and
        // their pending tokens are put back), free slots are parked
        std::vector<int32_t> feed((size_t)B), fpos((size_t)B, 0);
        for (int b = 0; b < B; ++b) {
            const bool hold = b != slot && m->active[(size_t)b] && m->hpos[(size_t)b] >= 0;
            if (hold && m->hpos[(size_t)b] + 1 >= c.max_seq)
                return fail(m->ctx, NX_ERR_CAPACITY, "admit: sequence in slot %d is at max_seq", b);
            feed[(size_t)b] = hold ? nx::kFeedHold : nx::kFeedPark;
            fpos[(size_t)b] = hold ? m->hpos[(size_t)b] + 1 : 0;
        }
        NX_TRY(ensure_graph(m));
        std::vector<unsigned long long> saved((size_t)B);
        NX_HIP(m->ctx, hipMemcpyAsync(saved.data(), m->best, (size_t)B * 8, hipMemcpyDeviceToHost, st));
        for (int b = 0; b < B; ++b) m->h_stage[b] = 1 << 30;  // nothing is recorded
        NX_HIP(m->ctx, hipMemcpyAsync(m->base, m->h_stage, (size_t)B * 4, hipMemcpyHostToDevice, st));
        for (int i = 0; i < P; ++i) {
            feed[(size_t)slot] = prompt[i];
            NX_TRY(upload_feed(m, feed.data(), fpos.data()));
            NX_HIP(m->ctx, hipGraphLaunch(m->exec, st));
        }
        // held and parked slots go back to where they were
        std::vector<unsigned long long> best((size_t)B);
        NX_HIP(m->ctx, hipMemcpyAsync(best.data(), m->best, (size_t)B * 8, hipMemcpyDeviceToHost, st));
        NX_HIP(m->ctx, hipStreamSynchronize(st));
            std::vector<int32_t> pos((size_t)B);
        for (int b = 0; b < B; ++b) {
            pos[(size_t)b] = b == slot ? P - 1 : m->hpos[(size_t)b];
            if (b != slot) best[(size_t)b] = saved[(size_t)b];
        }
        NX_HIP(m->ctx, hipMemcpyAsync(m->pos, pos.data(), (size_t)B * 4, hipMemcpyHostToDevice, st));
        NX_HIP(m->ctx, hipMemcpyAsync(m->best, best.data(), (size_t)B * 8, hipMemcpyHostToDevice, st));
        NX_HIP(m->ctx, hipStreamSynchronize(st));
        m->hpos[(size_t)slot] = P - 1;
    }
    m->active[(size_t)slot] = 1;
    NX_TRY(feed_decode(m));
    if (next_token) {
        unsigned long long k = 0;
        NX_HIP(m->ctx, hipMemcpyAsync(&k, m->best + slot, 8, hipMemcpyDeviceToHost, st));
        NX_HIP(m->ctx, hipStreamSynchronize(st));
        *next_token = (int32_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull));
    }
    return NX_OK;
}

nx_status nx_model_decode_forced(nx_model* m, const int32_t* tokens, int steps, float* logits) {
    if (!m || !tokens || steps < 1) return NX_ERR_INVALID;
    const nx_model_config& c = m->c;
    const int B = c.batch;
    int nact = 0;
    for (int b = 0; b < B; ++b) {
        if (!m->active[(size_t)b]) continue;
        ++nact;
        if (m->hpos[(size_t)b] < 0) return fail(m->ctx, NX_ERR_STATE, "decode before prefill or fill_context");
        if (m->hpos[(size_t)b] + steps >= c.max_seq) return fail(m->ctx, NX_ERR_CAPACITY, "decode exceeds max_seq");
        for (int s = 0; s < steps; ++s) {
            const int32_t t = tokens[(size_t)b * steps + s];
            if (t < 0 || t >= c.vocab) return fail(m->ctx, NX_ERR_INVALID, "forced token out of vocabulary");
        }
    }
    if (nact == 0) return fail(m->ctx, NX_ERR_STATE, "decode with no active sequence");
    {
        std::vector<int> want((size_t)B, -1);
        for (int b = 0; b < B; ++b)
            if (m->active[(size_t)b]) want[(size_t)b] = m->hpos[(size_t)b] + steps;
        NX_TRY(pool_ensure(m, want));
    }
    NX_TRY(ensure_graph(m));
    hipStream_t st = m->ctx->stream;
    for (int b = 0; b < B; ++b) m->h_stage[b] = 1 << 30;  // nothing is recorded
    NX_HIP(m->ctx, hipMemcpyAsync(m->base, m->h_stage, (size_t)B * 4, hipMemcpyHostToDevice, st));
    std::vector<int32_t> feed((size_t)B);
    const size_t V = (size_t)c.vocab;
    for (int s = 0; s < steps; ++s) {
        for (int b = 0; b < B; ++b) feed[(size_t)b] = m->active[(size_t)b] ? tokens[(size_t)b * steps + s] : nx::kFeedPark;
        NX_TRY(upload_feed(m, feed.data(), nullptr));
        NX_HIP(m->ctx, hipGraphLaunch(m->exec, st));
        if (logits)
            for (int b = 0; b < B; ++b)
                NX_HIP(m->ctx, hipMemcpyAsync(logits + ((size_t)b * steps + s) * V, m->logits + (size_t)b * V, V * 4,
                                              hipMemcpyDeviceToHost, st));
    }
    NX_HIP(m->ctx, hipStreamSynchronize(st));
    for (int b = 0; b < B; ++b)
        if (m->active[(size_t)b]) m->hpos[(size_t)b] += steps;
    return feed_decode(m);
}

nx_status nx_model_logits(nx_model* m, float* out) {
    if (!m || !out) return NX_ERR_INVALID;
    NX_HIP(m->ctx, hipMemcpyAsync(out, m->logits, (size_t)m->c.batch * m->c.vocab * 4, hipMemcpyDeviceToHost, m->ctx->stream));
    NX_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    return NX_OK;
}

nx_status nx_model_position(nx_model* m, int b, int* p) {
    if (!m || !p || b < 0 || b >= m->c.batch) return NX_ERR_INVALID;
    *p = m->hpos[b];
    return NX_OK;
}

nx_status nx_model_step_bytes(nx_model* m, double* bytes) {
    if (!m || !bytes) return NX_ERR_INVALID;
    const nx_model_config& c = m->c;
    const int d = c.d_model, F = c.ffn, E = c.n_experts;
    double w = (double)qbytes(c.vocab, d);  // lm_head
    for (int L = 0; L < c.n_layers; ++L) {
        w += (double)qbytes(m->nqkv, d) + (double)qbytes(d, m->qdim);
        if (E == 0) {
            w += (double)qbytes(2 * (size_t)F, d) + (double)qbytes(d, F);
        } else {
            std::vector<int32_t> cnt(E, 0);
            NX_HIP(m->ctx, hipMemcpy(cnt.data(), m->layers[L].moe_count, (size_t)E * 4, hipMemcpyDeviceToHost));
            int active = 0;
            for (int e = 0; e < E; ++e) active += cnt[e] > 0;
            if (active == 0) active = c.top_k;  // before the first step
            w += (double)qbytes(E, d) + active * ((double)qbytes(2 * (size_t)F, d) + (double)qbytes(d, F));
        }
    }
    *bytes = w + kv_bytes(m) * c.n_layers;
    return NX_OK;
}

nx_status nx_model_time_ffn_gemv(nx_model* m, int iters, double* avg_ms, double* bytes) {
    if (!m || !avg_ms || iters < 1) return NX_ERR_INVALID;
    const nx_model_config& c = m->c;
    const int E = c.n_experts;
    hipStream_t st = m->ctx->stream;
    // launch i uses layer i % n_layers, so consecutive launches stream
    // different weights (every layer's gate/up, 2 GB at the 8B shape, is far
    // larger than the last-level cache) as they do inside a decode step
    std::function<hipError_t(int)> launch;
    double nbytes = 0.0;
    if (E == 0) {
        launch = [&](int i) {
            const Layer& ly = m->layers[i % c.n_layers];
            nx::GemvArgs f{};
            f.W = ly.w13;
            f.S = ly.s13;
            f.N = 2 * c.ffn;
            f.K = c.d_model;
            f.G = m->Gd;
            f.batch = c.batch;
            f.h32 = m->h;
            f.ldx = c.d_model;
            f.eps = c.eps;
            f.norm_w = ly.norm_ffn;
            f.act16 = m->act16;
            f.lda = m->Fp;
            return nx::gemv_launch(nx::X_RMSNORM, nx::E_SWIGLU, f, st);
        };
        nbytes = (double)qbytes(2 * (size_t)c.ffn, c.d_model) + (double)c.batch * (4.0 * c.d_model + 2.0 * c.ffn);
    } else {
        // the routed gate/up expert GEMV with the routing of the last step's
        // last layer (the routing plan is shared by the layers and holds that
        // layer's routing), over the weights of layer i % n_layers
        const Layer& last = m->layers[c.n_layers - 1];
        std::vector<int32_t> cnt(E, 0);
        NX_HIP(m->ctx, hipMemcpy(cnt.data(), last.moe_count, (size_t)E * 4, hipMemcpyDeviceToHost));
        int active = 0, slots = 0;
        for (int e = 0; e < E; ++e) {
            active += cnt[e] > 0;
            slots += cnt[e];
        }
        if (active == 0) return fail(m->ctx, NX_ERR_STATE, "no routed step to time (decode once first)");
        const bool fused_b1 = c.batch == 1 && nx::moe_b1_fused_fits(c.d_model, c.ffn, E, c.top_k);
        launch = [&](int i) {
            const Layer& ly = m->layers[i % c.n_layers];
            nx::MoeFfnArgs mf{};
            mf.x16 = m->xn16;
            mf.ldx = c.d_model;
            mf.w13 = ly.w13;
            mf.s13 = ly.s13;
            mf.w2 = ly.w2;
            mf.s2 = ly.s2;
            mf.d = c.d_model;
            mf.F = c.ffn;
            mf.E = E;
            mf.k = c.top_k;
            mf.batch = c.batch;
            mf.plan = m->moe_plan;
            mf.weights = m->moe_w;
            mf.act16 = m->moe_act;
            mf.y32 = m->moe_y;
            mf.out = m->h;
            mf.accumulate = 1;
            if (fused_b1) {
                // the launch of the decode step: routing of h with layer i's
                // router, then the chosen experts' gate/up
                nx::MoeArgs ma{};
                ma.logits = m->router_logits;
                ma.E = E;
                ma.k = c.top_k;
                ma.batch = 1;
                ma.ids = m->moe_ids;
                ma.weights = m->moe_w;
                ma.expert_count = ly.moe_count;
                ma.expert_slots = m->moe_slots;
                ma.plan = m->moe_plan;
                ma.h = m->h;
                ma.norm_w = ly.norm_ffn;
                ma.eps = c.eps;
                ma.d = c.d_model;
                ma.wr = ly.wr;
                ma.sr = ly.sr;
                return nx::moe_b1_gate_up_launch(ma, mf, st);
            }
            return nx::moe_gate_up_launch(mf, st);
        };
        nbytes = active * (double)qbytes(2 * (size_t)c.ffn, c.d_model) + (double)slots * (2.0 * c.d_model + 2.0 * c.ffn);
        if (fused_b1)  // every block reads h (fp32) and the router once from HBM
            nbytes = c.top_k * (double)qbytes(2 * (size_t)c.ffn, c.d_model) + (double)qbytes((size_t)E, c.d_model) +
                     4.0 * c.d_model + 2.0 * c.top_k * c.ffn;
    }
    for (int i = 0; i < c.n_layers; ++i) NX_LAUNCH(m, launch(i));
    NX_HIP(m->ctx, hipEventRecord(m->ctx->ev0, st));
    for (int i = 0; i < iters; ++i) NX_LAUNCH(m, launch(i));
    NX_HIP(m->ctx, hipEventRecord(m->ctx->ev1, st));
    NX_HIP(m->ctx, hipEventSynchronize(m->ctx->ev1));
    float ms = 0.0f;
    NX_HIP(m->ctx, hipEventElapsedTime(&ms, m->ctx->ev0, m->ctx->ev1));
    *avg_ms = (double)ms / iters;
    if (bytes) *bytes = nbytes;
    return NX_OK;
}

nx_status nx_model_time_attention(nx_model* m, int iters, double* avg_ms, double* bytes) {
    if (!m || !avg_ms || iters < 1) return NX_ERR_INVALID;
    const nx_model_config& c = m->c;
    for (int b = 0; b < c.batch; ++b)
        if (m->hpos[b] < 0) return fail(m->ctx, NX_ERR_STATE, "no context to attend over");
    hipStream_t st = m->ctx->stream;
    // launch i attends over layer i % n_layers (a separate cache per layer),
    // whose pages already hold every position (TurboQuant pages: no append)
    auto launch = [&](int i) { return attention_launch(m, m->layers[i % c.n_layers], st, false); };
    for (int i = 0; i < c.n_layers; ++i) NX_LAUNCH(m, launch(i));
    NX_HIP(m->ctx, hipEventRecord(m->ctx->ev0, st));
    for (int i = 0; i < iters; ++i) NX_LAUNCH(m, launch(i));
    NX_HIP(m->ctx, hipEventRecord(m->ctx->ev1, st));
    NX_HIP(m->ctx, hipEventSynchronize(m->ctx->ev1));
    float ms = 0.0f;
    NX_HIP(m->ctx, hipEventElapsedTime(&ms, m->ctx->ev0, m->ctx->ev1));
    *avg_ms = (double)ms / iters;
    if (bytes) *bytes = kv_bytes(m);
    return NX_OK;
}

}  // extern "C"

// ------------------------------------------------------------- NXF files --
// Tensors of a model in an NXF file.  Matrix shapes follow the reference's
// {in, out} convention (hybrid_model.cpp:366-391: wq.shape[1] is the q
// width, output.weight.shape[1] the vocabulary, experts.w1 is {E, d, F});
// the payload of the build's codecs holds `out` rows of `in` elements.  A
// file row r lands on device row (r / R) * GS + (r % R) * S + O of the
// runner's buffer, which interleaves gate and up rows and stacks q, k, v.
namespace {

struct RowMap {
    size_t R, GS, S, O;
    size_t dev(size_t r) const { return (r / R) * GS + (r % R) * S + O; }
};

struct NxfTensorSpec {
    std::string name;
    std::vector<int64_t> shape;
    int dtype;          // NX_DTYPE_*
    size_t rows;        // file rows
    size_t row_bytes;   // codes (I4), fp16 (F16) or fp32 (F32) bytes per row
    size_t srow_bytes;  // I4: scale bytes per row
    uint8_t* w;         // device rows
    uint16_t* s;        // I4: device scale rows
    RowMap map;
};

std::vector<NxfTensorSpec> nxf_specs(nx_model* m) {
    const nx_model_config& c = m->c;
    const size_t d = (size_t)c.d_model, F = (size_t)c.ffn, E = (size_t)c.n_experts, V = (size_t)c.vocab;
    const size_t qd = (size_t)m->qdim, kvd = (size_t)m->kvdim;
    const size_t Gd = (size_t)m->Gd, Gq = (size_t)m->Gq, Gf = (size_t)m->Gf;
    auto plain = [](size_t rows, size_t off = 0) { return RowMap{rows ? rows : 1, 0, 1, off}; };
    std::vector<NxfTensorSpec> t;
    auto i4 = [&](const std::string& name, std::vector<int64_t> shape, size_t rows, size_t G, uint8_t* w, uint16_t* sc,
                  RowMap mp) {
        t.push_back({name, std::move(shape), NX_DTYPE_I4, rows, G * 16, G * 2, w, sc, mp});
    };
    auto f32 = [&](const std::string& name, float* w, size_t n) {
        t.push_back({name, {(int64_t)n}, NX_DTYPE_F32, 1, n * 4, 0, reinterpret_cast<uint8_t*>(w), nullptr, plain(1)});
    };
    t.push_back({"tok_embeddings.weight", {(int64_t)d, (int64_t)V}, NX_DTYPE_F16, V, d * 2, 0,
                 reinterpret_cast<uint8_t*>(m->embed), nullptr, plain(V)});
    f32("norm.weight", m->norm_final, d);
    i4("output.weight", {(int64_t)d, (int64_t)V}, V, Gd, m->lm_w, m->lm_s, plain(V));
    for (int L = 0; L < c.n_layers; ++L) {
        Layer& ly = m->layers[(size_t)L];
        const std::string p = "layers." + std::to_string(L) + ".";
        f32(p + "attention_norm.weight", ly.norm_attn, d);
        f32(p + "ffn_norm.weight", ly.norm_ffn, d);
        if (c.qk_norm) {  // the Q/K norms of hybrid_model.cpp:1952-1953, head_dim long
            f32(p + "attn_q_norm.weight", ly.qnorm, (size_t)c.head_dim);
            f32(p + "attn_k_norm.weight", ly.knorm, (size_t)c.head_dim);
        }
        i4(p + "attention.wq.weight", {(int64_t)d, (int64_t)qd}, qd, Gd, ly.wqkv, ly.sqkv, plain(qd, 0));
        i4(p + "attention.wk.weight", {(int64_t)d, (int64_t)kvd}, kvd, Gd, ly.wqkv, ly.sqkv, plain(kvd, qd));
        i4(p + "attention.wv.weight", {(int64_t)d, (int64_t)kvd}, kvd, Gd, ly.wqkv, ly.sqkv, plain(kvd, qd + kvd));
        i4(p + "attention.wo.weight", {(int64_t)qd, (int64_t)d}, d, Gq, ly.wo, ly.so, plain(d));
        if (E == 0) {
            i4(p + "feed_forward.w1.weight", {(int64_t)d, (int64_t)F}, F, Gd, ly.w13, ly.s13, RowMap{F, 0, 2, 0});
            i4(p + "feed_forward.w3.weight", {(int64_t)d, (int64_t)F}, F, Gd, ly.w13, ly.s13, RowMap{F, 0, 2, 1});
            i4(p + "feed_forward.w2.weight", {(int64_t)F, (int64_t)d}, d, Gf, ly.w2, ly.s2, plain(d));
        } else {
            i4(p + "feed_forward.gate.weight", {(int64_t)d, (int64_t)E}, E, Gd, ly.wr, ly.sr, plain(E));
            i4(p + "feed_forward.experts.w1.weight", {(int64_t)E, (int64_t)d, (int64_t)F}, E * F, Gd, ly.w13, ly.s13,
               RowMap{F, 2 * F, 2, 0});
            i4(p + "feed_forward.experts.w3.weight", {(int64_t)E, (int64_t)d, (int64_t)F}, E * F, Gd, ly.w13, ly.s13,
               RowMap{F, 2 * F, 2, 1});
            i4(p + "feed_forward.experts.w2.weight", {(int64_t)E, (int64_t)F, (int64_t)d}, E * d, Gf, ly.w2, ly.s2,
               RowMap{d, d, 1, 0});
        }
    }
    return t;
}

// Copy file rows [r0, r0 + n) between a host/staging buffer (packed rows)
// and the device rows of map, one strided copy per run of rows in the
// same group.
nx_status copy_rows(nx_ctx* ctx, uint8_t* dev_base, uint8_t* packed, size_t rb, const RowMap& mp, size_t r0, size_t n,
                    hipMemcpyKind kind) {
    size_t r = r0;
    while (r < r0 + n) {
        const size_t run = std::min(r0 + n - r, mp.R - r % mp.R);
        uint8_t* dv = dev_base + mp.dev(r) * rb;
        uint8_t* pk = packed + (r - r0) * rb;
        if (kind == hipMemcpyDeviceToHost)
            NX_HIP(ctx, hipMemcpy2DAsync(pk, rb, dv, mp.S * rb, rb, run, kind, ctx->stream));
        else
            NX_HIP(ctx, hipMemcpy2DAsync(dv, mp.S * rb, pk, rb, rb, run, kind, ctx->stream));
        r += run;
    }
    return NX_OK;
}

nx_status nxf_fail(nx_ctx* ctx, nx_status s) { return fail(ctx, s, "%s", nx_nxf_error()); }

// Whole rows per chunk, at most 64 KiB (one row if a row is larger).
nx_status write_rows(nx_ctx* ctx, nx_nxf_writer* w, const uint8_t* host, size_t rows, size_t rb, int codec, int gs) {
    const size_t per = std::max<size_t>(1, (64u << 10) / rb);
    for (size_t r = 0; r < rows; r += per) {
        const size_t n = std::min(per, rows - r);
        nx_status s = nx_nxf_writer_add_chunk(w, host + r * rb, n * rb, codec, gs);
        if (s != NX_OK) return nxf_fail(ctx, s);
    }
    return NX_OK;
}

}  // namespace

extern "C" {

nx_status nx_model_save_nxf(nx_model* m, const char* path) {
    if (!m || !path) return NX_ERR_INVALID;
    nx_ctx* ctx = m->ctx;
    const nx_model_config& c = m->c;
    NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    nx_nxf_writer* w = nullptr;
    nx_status s = nx_nxf_writer_create(ctx, path, &w);
    if (s != NX_OK) return nxf_fail(ctx, s);
    nx_nxf_manifest man{};
    snprintf(man.architecture, sizeof(man.architecture), "%s", c.n_experts ? "mixtral" : "llama");
    snprintf(man.name, sizeof(man.name), "nexus-int4-g32");
    man.num_layers = (uint32_t)c.n_layers;
    man.hidden_dim = (uint32_t)c.d_model;
    man.num_heads = (uint32_t)c.n_heads;
    man.num_kv_heads = (uint32_t)c.n_kv_heads;
    man.head_dim = (uint32_t)c.head_dim;
    man.vocab_size = (uint32_t)c.vocab;
    man.max_seq_len = (uint32_t)c.max_seq;
    man.rope_theta = c.rope_theta;
    man.rms_norm_eps = c.eps;
    man.num_experts = (uint32_t)c.n_experts;
    man.num_active_experts = (uint32_t)c.top_k;
    man.default_codec = NX_CODEC_INT4;
    man.default_group_size = 32;
    nx_nxf_writer_set_manifest(w, &man);
    std::vector<uint8_t> host;
    for (const NxfTensorSpec& t : nxf_specs(m)) {
        s = nx_nxf_writer_begin_tensor(w, t.name.c_str(), t.shape.data(), (int)t.shape.size(), t.dtype);
        if (s != NX_OK) break;
        host.resize(t.rows * t.row_bytes);
        if (t.w) {
            if ((s = copy_rows(ctx, t.w, host.data(), t.row_bytes, t.map, 0, t.rows, hipMemcpyDeviceToHost)) != NX_OK) break;
            if (hipStreamSynchronize(ctx->stream) != hipSuccess) {
                s = fail(ctx, NX_ERR_HIP, "nx_model_save_nxf: device copy failed");
                break;
            }
        } else {  // RMSNorm weights of 1.0
            for (size_t i = 0; i < t.row_bytes / 4; ++i) reinterpret_cast<float*>(host.data())[i] = 1.0f;
        }
        const int codec = t.dtype == NX_DTYPE_I4 ? NX_CODEC_INT4 : t.dtype == NX_DTYPE_F16 ? NX_CODEC_FP16 : NX_CODEC_FP32;
        if ((s = write_rows(ctx, w, host.data(), t.rows, t.row_bytes, codec, t.dtype == NX_DTYPE_I4 ? 32 : 0)) != NX_OK) break;
        if (t.dtype == NX_DTYPE_I4) {  // the fp16 scales: sidecar chunks of the same tensor
            host.resize(t.rows * t.srow_bytes);
            if ((s = copy_rows(ctx, reinterpret_cast<uint8_t*>(t.s), host.data(), t.srow_bytes, t.map, 0, t.rows,
                               hipMemcpyDeviceToHost)) != NX_OK)
                break;
            if (hipStreamSynchronize(ctx->stream) != hipSuccess) {
                s = fail(ctx, NX_ERR_HIP, "nx_model_save_nxf: device copy failed");
                break;
            }
            if ((s = write_rows(ctx, w, host.data(), t.rows, t.srow_bytes, NX_CODEC_FP16, 32)) != NX_OK) break;
        }
        if ((s = nx_nxf_writer_end_tensor(w)) != NX_OK) {
            s = nxf_fail(ctx, s);
            break;
        }
    }
    if (s != NX_OK) {
        nx_nxf_writer_destroy(w);
        return s;
    }
    s = nx_nxf_writer_finalize(w);
    return s == NX_OK ? NX_OK : nxf_fail(ctx, s);
}

nx_status nx_model_load_nxf(nx_ctx* ctx, const char* path, const nx_model_config* run, nx_model** out) {
    if (!ctx || !path || !run || !out) return NX_ERR_INVALID;
    *out = nullptr;
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "nx_model_load_nxf inside a token batch");
    nx_nxf* r = nullptr;
    nx_status s = nx_nxf_open(path, &r);
    if (s != NX_OK) return nxf_fail(ctx, s);
    nx_model* m = nullptr;
    uint8_t* host = nullptr;
    uint8_t* dev = nullptr;
    nx::HashRange* dranges = nullptr;
    uint32_t* dhash = nullptr;
    do {
        nx_nxf_manifest man{};
        nx_nxf_get_manifest(r, &man);
        nx_model_config c = *run;
        c.n_layers = (int)man.num_layers;
        c.d_model = (int)man.hidden_dim;
        c.n_heads = (int)man.num_heads;
        c.n_kv_heads = (int)man.num_kv_heads;
        c.head_dim = (int)man.head_dim;
        c.vocab = (int)man.vocab_size;
        c.n_experts = (int)man.num_experts;
        // no count in the manifest: ten experts per token, as the reference
        // runs it (hybrid_model.cpp:1648, capped at the expert count, :1675)
        c.top_k = c.n_experts > 0 && man.num_active_experts == 0 ? std::min(10, c.n_experts)
                                                                   : (int)man.num_active_experts;
        c.rope_theta = man.rope_theta;
        c.eps = man.rms_norm_eps;
        c.norm_sigma = 0.0f;
        // the FFN width from the first layer's gate projection
        int ti = -1;
        nx_nxf_tensor info{};
        nx_nxf_find(r, c.n_experts ? "layers.0.feed_forward.experts.w1.weight" : "layers.0.feed_forward.w1.weight", &ti);
        if (ti < 0 || nx_nxf_tensor_at(r, ti, &info) != NX_OK || info.ndim < 2) {
            s = fail(ctx, NX_ERR_INVALID, "nxf '%s': no FFN gate tensor in layer 0", path);
            break;
        }
        c.ffn = (int)info.shape[info.ndim - 1];
        // per-head Q/K norms where the file has them (hybrid_model.cpp:1952-1953
        // loads each when present); both or neither
        int tq = -1, tk = -1;
        nx_nxf_find(r, "layers.0.attn_q_norm.weight", &tq);
        nx_nxf_find(r, "layers.0.attn_k_norm.weight", &tk);
        if ((tq < 0) != (tk < 0)) {
            s = fail(ctx, NX_ERR_UNSUPPORTED, "nxf '%s': a Q norm without a K norm (or the reverse)", path);
            break;
        }
        c.qk_norm = tq >= 0 ? 1 : 0;
        if ((s = check_config(ctx, c)) != NX_OK) break;
        m = new nx_model();
        m->ctx = ctx;
        m->c = c;
        if ((s = create_impl(m, false)) != NX_OK) break;
        const std::vector<NxfTensorSpec> specs = nxf_specs(m);
        // staging large enough for the biggest tensor, chunks 256-byte aligned
        size_t cap = 0, maxchunks = 0;
        for (const NxfTensorSpec& t : specs) {
            if (nx_nxf_find(r, t.name.c_str(), &ti) != NX_OK || ti < 0) {
                s = fail(ctx, NX_ERR_INVALID, "nxf '%s': tensor '%s' is missing", path, t.name.c_str());
                break;
            }
            nx_nxf_tensor_at(r, ti, &info);
            bool same = info.ndim == (int)t.shape.size() && info.dtype == t.dtype;
            for (int k = 0; same && k < info.ndim; ++k) same = info.shape[k] == t.shape[(size_t)k];
            if (!same) {
                s = fail(ctx, NX_ERR_INVALID, "nxf '%s': tensor '%s' has another shape or dtype than the manifest implies",
                         path, t.name.c_str());
                break;
            }
            size_t need = 0;
            for (int k = 0; k < info.num_chunks; ++k) {
                nx_nxf_chunk ch{};
                nx_nxf_chunk_at(r, ti, k, &ch);
                need += (ch.compressed_size + 255) / 256 * 256;
            }
            cap = std::max(cap, need);
            maxchunks = std::max(maxchunks, (size_t)info.num_chunks);
        }
        if (s != NX_OK) break;
        cap = std::max<size_t>(cap, 256);
        if (hipHostMalloc(reinterpret_cast<void**>(&host), cap, hipHostMallocDefault) != hipSuccess ||
            hipMalloc(reinterpret_cast<void**>(&dev), cap) != hipSuccess ||
            hipMalloc(reinterpret_cast<void**>(&dranges), std::max<size_t>(maxchunks, 1) * sizeof(nx::HashRange)) != hipSuccess ||
            hipMalloc(reinterpret_cast<void**>(&dhash), std::max<size_t>(maxchunks, 1) * 4) != hipSuccess) {
            s = fail(ctx, NX_ERR_OOM, "nx_model_load_nxf: staging of %zu bytes", cap);
            break;
        }
        hipStream_t st = ctx->stream;
        for (const NxfTensorSpec& t : specs) {
            nx_nxf_find(r, t.name.c_str(), &ti);
            nx_nxf_tensor_at(r, ti, &info);
            std::vector<nx_nxf_chunk> ch((size_t)info.num_chunks);
            std::vector<size_t> at(ch.size());
            std::vector<nx::HashRange> rg;
            size_t used = 0;
            for (size_t k = 0; k < ch.size() && s == NX_OK; ++k) {
                nx_nxf_chunk_at(r, ti, (int)k, &ch[k]);
                at[k] = used;
                if (nx_nxf_read_chunk(r, ti, (int)k, host + used) != NX_OK) s = nxf_fail(ctx, NX_ERR_IO);
                rg.push_back(nx::HashRange{used, ch[k].compressed_size, (uint32_t)k});
                used += (ch[k].compressed_size + 255) / 256 * 256;
            }
            if (s != NX_OK) break;
            // verify every chunk on the device before any is used
            std::stable_sort(rg.begin(), rg.end(), [](const nx::HashRange& a, const nx::HashRange& b) { return a.len > b.len; });
            std::vector<uint32_t> got(ch.size());
            if (!ch.empty() &&
                (hipMemcpyAsync(dev, host, used, hipMemcpyHostToDevice, st) != hipSuccess ||
                 hipMemcpyAsync(dranges, rg.data(), rg.size() * sizeof(nx::HashRange), hipMemcpyHostToDevice, st) !=
                     hipSuccess ||
                 nx::xxh32_launch(dev, dranges, (int)rg.size(), dhash, st) != hipSuccess ||
                 hipMemcpyAsync(got.data(), dhash, got.size() * 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
                 hipStreamSynchronize(st) != hipSuccess)) {
                s = fail(ctx, NX_ERR_HIP, "nx_model_load_nxf: upload or hashing of '%s' failed", t.name.c_str());
                break;
            }
            for (size_t k = 0; k < ch.size() && s == NX_OK; ++k)
                if (got[k] != ch[k].checksum)
                    s = fail(ctx, NX_ERR_CHECKSUM, "nxf '%s': checksum mismatch in chunk %zu of '%s' (stored %08x, data %08x)",
                             path, k, t.name.c_str(), ch[k].checksum, got[k]);
            if (s != NX_OK) break;
            // place the rows: codes (or values) chunks first, then for I4 the
            // fp16 scale chunks, each holding whole rows
            const int vcodec = t.dtype == NX_DTYPE_I4 ? NX_CODEC_INT4 : t.dtype == NX_DTYPE_F16 ? NX_CODEC_FP16 : NX_CODEC_FP32;
            size_t vrow = 0, srow = 0;
            for (size_t k = 0; k < ch.size() && s == NX_OK; ++k) {
                const bool is_scale = t.dtype == NX_DTYPE_I4 && ch[k].codec == NX_CODEC_FP16;
                if (!is_scale && ch[k].codec != vcodec) {
                    s = fail(ctx, NX_ERR_UNSUPPORTED, "nxf '%s': chunk %zu of '%s' has codec %u", path, k, t.name.c_str(),
                             (unsigned)ch[k].codec);
                    break;
                }
                if (t.dtype == NX_DTYPE_I4 && ch[k].group_size != 32) {
                    s = fail(ctx, NX_ERR_UNSUPPORTED, "nxf '%s': chunk %zu of '%s' has group size %u (32 expected)", path,
                             k, t.name.c_str(), (unsigned)ch[k].group_size);
                    break;
                }
                const size_t rb = is_scale ? t.srow_bytes : t.row_bytes;
                size_t& row = is_scale ? srow : vrow;
                if (ch[k].compressed_size % rb || row + ch[k].compressed_size / rb > t.rows) {
                    s = fail(ctx, NX_ERR_INVALID, "nxf '%s': chunk %zu of '%s' does not hold whole rows within the tensor",
                             path, k, t.name.c_str());
                    break;
                }
                const size_t n = ch[k].compressed_size / rb;
                s = copy_rows(ctx, is_scale ? reinterpret_cast<uint8_t*>(t.s) : t.w, dev + at[k], rb, t.map, row, n,
                              hipMemcpyDeviceToDevice);
                row += n;
            }
            if (s != NX_OK) break;
            if (vrow != t.rows || (t.dtype == NX_DTYPE_I4 && srow != t.rows)) {
                s = fail(ctx, NX_ERR_INVALID, "nxf '%s': tensor '%s' holds %zu value and %zu scale rows of %zu", path,
                         t.name.c_str(), vrow, srow, t.rows);
                break;
            }
            if (hipStreamSynchronize(st) != hipSuccess) {  // the staging is reused by the next tensor
                s = fail(ctx, NX_ERR_HIP, "nx_model_load_nxf: placing '%s' failed", t.name.c_str());
                break;
            }
        }
    } while (false);
    (void)hipStreamSynchronize(ctx->stream);
    if (host) (void)hipHostFree(host);
    if (dev) (void)hipFree(dev);
    if (dranges) (void)hipFree(dranges);
    if (dhash) (void)hipFree(dhash);
    nx_nxf_close(r);
    if (s != NX_OK) {
        if (m) free_model(m);
        return s;
    }
    *out = m;
    return NX_OK;
}

}  // extern "C"
