// The attention half of one decoder layer at batch 1 over fp16 pages in a
// single launch: h -> RMSNorm -> QKV GEMV -> RoPE + page write -> paged
// attention -> wo GEMV -> h += (hybrid_model.cpp:1257-1443, the first
// residual block, with the attention of :1447-1565).
//
// As separate kernels these are three launches whose run time is mostly
// latency: every launch begins with an idle memory pipe, and the attention
// split kernel is a chain of dependent round trips (table, pages, record,
// counter, merge).  Here one block per CU does all three, and every byte
// that does not depend on this step -- its QKV weight rows, its KV pages,
// its wo weight rows -- is requested at the start, in the order it is used.
// The data that does depend on the step moves between blocks through
// agent-scope (cross-XCD coherent) stores, counted in per-layer counters:
//   1. each block computes its QKV row pairs (RMSNorm staged once per block)
//      and stores q (fp32) and the new K/V (fp16, into the page slot of the
//      position); it then counts itself in the counter of every kv head
//      whose rows it wrote;
//   2. the blocks of kv head g (nsplit of them; pages dealt round-robin as
//      in the split kernel) wait for g's counter, read q and patch the
//      position's K/V slot into the page they hold (it was requested before
//      it was written), run the page-pair product on the matrix cores and
//      store a split record; the last of them merges the records, stores g's
//      slice of the attention output and counts the head done;
//   3. every block waits for all heads, stages the attention output and
//      reduces its wo rows (requested at the start) into h.
// A wait gives up after kSpinTicks of the 100 MHz constant clock: it sets
// the error word, later waits return at once, and the launch finishes with
// wrong values that the host reports instead of using.  The grid is one
// block per CU and needs every block resident at once (checked by the
// planner with the occupancy API).
#include <algorithm>

#include "nx_attn_dev.h"
#include "nx_gemv_dev.h"

namespace nx {

#ifdef NX_LAYER_TRACE
// Phase timestamps (100 MHz constant clock) of every block of the last
// launch; a build made only to study the launch's timeline.
__device__ unsigned long long g_layer_trace[1024 * 16];
#define NX_TRACE(i) \
    if (threadIdx.x == 0) g_layer_trace[blockIdx.x * 16 + (i)] = __builtin_amdgcn_s_memrealtime()
#define NX_TRACE_BY(i, t) \
    if (threadIdx.x == (t)) g_layer_trace[blockIdx.x * 16 + (i)] = __builtin_amdgcn_s_memrealtime()
#else
#define NX_TRACE(i)
#define NX_TRACE_BY(i, t)
#endif

namespace {

using namespace at;
using namespace gv;

constexpr int kLWaves = kAttnWaves;
constexpr int kLThreads = kLWaves * kWave;
constexpr int kQkvRows = 4;                          // QKV rows per wavefront (two pairs)
constexpr unsigned long long kSpinTicks = 20000000ull;  // 200 ms of the 100 MHz clock
constexpr int kBufFlags = 0x00020000;
constexpr int kSc1 = 16;  // cache-policy bit of an agent-scope buffer load

typedef float f4v __attribute__((ext_vector_type(4)));
typedef float f2v __attribute__((ext_vector_type(2)));

__device__ inline __amdgpu_buffer_rsrc_t rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, kBufFlags);
}
__device__ inline uint4 ld_coh16(__amdgpu_buffer_rsrc_t rs, int off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kSc1));
}
__device__ inline uint2 ld_coh8(__amdgpu_buffer_rsrc_t rs, int off) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, kSc1));
}

// Wait (the whole block) until *ctr has reached target (modulo 2^32), or
// the error word is set, or kSpinTicks have passed (then set it).
__device__ inline void wait_count(const unsigned* ctr, unsigned target, unsigned* err, int trace_slot = -1) {
    if (threadIdx.x < kWave) {
        const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
        [[maybe_unused]] bool firstp = true;
        for (;;) {
            const unsigned v = __hip_atomic_load(const_cast<unsigned*>(ctr), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const unsigned e = __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#ifdef NX_LAYER_TRACE
            if (firstp && trace_slot >= 0 && threadIdx.x == 0 && v + e != 0x7FFFFFFFu)
                g_layer_trace[blockIdx.x * 16 + trace_slot] = __builtin_amdgcn_s_memrealtime();
#endif
            firstp = false;
            if ((int)(v - target) >= 0 || e != 0u) break;
            if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinTicks) {
                __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
}

// kv heads whose rows lie in [r0, r1): q rows [0, qdim) in groups of G*hd,
// then k and v rows in groups of hd.
__host__ __device__ inline unsigned qkv_heads(int r0, int r1, int qdim, int kvdim, int G, int hd, int hkv) {
    unsigned mask = 0;
    const int off[3] = {0, qdim, qdim + kvdim}, span[3] = {G * hd, hd, hd};
    for (int k = 0; k < 3; ++k) {
        const int lo = r0 > off[k] ? r0 : off[k];
        const int hi = r1 < off[k] + hkv * span[k] ? r1 : off[k] + hkv * span[k];
        for (int g = 0; g < hkv; ++g)
            if (lo < hi && lo < off[k] + (g + 1) * span[k] && hi > off[k] + g * span[k]) mask |= 1u << g;
    }
    return mask;
}

// Page a of a pair alone (page b holds no token): page b's operands are
// zero and fully masked, as load_pair leaves a page with no valid token.
template <int HD>
__device__ inline void load_page_a(PairRaw<HD>& r, const AttnArgs& a, int blka, int na, int kvh, int lane) {
    const int g = lane >> 4, t = lane & 15;
    const size_t base = ((size_t)blka * a.hkv + kvh) * kPage * HD;
#pragma unroll
    for (int s = 0; s < HD / 32; ++s) {
        r.k[0][s] = *reinterpret_cast<const uint4*>(a.kpool + base + (size_t)t * HD + 32 * s + 8 * g);
        r.k[1][s] = make_uint4(0u, 0u, 0u, 0u);
    }
    (void)na;
#pragma unroll
    for (int nt = 0; nt < HD / 16; ++nt) {
        r.v[nt][0] = *reinterpret_cast<const uint2*>(a.vpool + base + (size_t)(16 * nt + t) * kPage + 4 * g);
        r.v[nt][1] = make_uint2(0u, 0u);
    }
}

// The attention output (fp16, K values) into the LDS pair layout of the wo
// GEMV, read with agent-scope loads (merging blocks stored it in this
// launch).  K % 8 == 0; thread t takes chunks t, t + 512, ...
template <int CPT>
__device__ inline void stage_att(const GemvArgs& a, uint32_t* sp, float* s8) {
    const int nch = a.G * 4, nvalid = a.K / 8;
    const __amdgpu_buffer_rsrc_t rs = rsrc(a.x16, a.K * 2);
    uint32_t X[CPT][4];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = threadIdx.x + j * kLThreads;
        const bool ok = c < nvalid;
        const uint4 v = ld_coh16(rs, 16 * (ok ? c : 0));
        X[j][0] = ok ? v.x : 0u;
        X[j][1] = ok ? v.y : 0u;
        X[j][2] = ok ? v.z : 0u;
        X[j][3] = ok ? v.w : 0u;
    }
#pragma unroll
    for (int j = 0; j < CPT; ++j)
        if (threadIdx.x + j * kLThreads < nch) put_chunk(threadIdx.x + j * kLThreads, X[j], sp, s8);
    __syncthreads();
}

template <int G, int HD, int GPL, int GPLO>
__global__ __launch_bounds__(kLThreads, 1) void k_attn_block_b1(LayerArgs L) {
    constexpr int CPT = (4 * GPL + kLWaves - 1) / kLWaves;    // h chunks per thread (RMSNorm staging)
    constexpr int CPTO = (4 * GPLO + kLWaves - 1) / kLWaves;  // attention-output chunks per thread
    constexpr int GPLM = GPL > GPLO ? GPL : GPLO;
    constexpr int REC = rec_floats(G, HD), MO = G * HD, LO = G * HD + G;
    __shared__ __align__(16) uint32_t sp[kWave * GPLM * 16];
    __shared__ float s8[kWave * GPLM];
    __shared__ float red[kLWaves];
    __shared__ __align__(16) float lds[kLWaves * REC];
    __shared__ int last;

    NX_TRACE(12);
    const GemvArgs& qa = L.qkv;
    const GemvArgs& oa = L.wo;
    const AttnArgs& at = L.at;
    const int lane = threadIdx.x & 63, blk = blockIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g4 = lane >> 4, t = lane & 15;
    const unsigned ep = *L.epoch;
    NX_TRACE(0);

    // ---- requests, in the order they are used --------------------------
    // the block-table entries of this wavefront's pages first (the page
    // requests wait for them): wavefront w of split s takes pages
    // s + nsplit (w + 8 i), at most two (the planner bounds the context);
    // lane i holds page i's entry
    const int hkv = at.hkv, nsplit = L.nsplit;
    const bool has_attn = blk < nsplit * hkv;
    const int kvh = has_attn ? blk / nsplit : 0, split = blk % nsplit;
    const int stride = nsplit * kLWaves, first = split + nsplit * wave;
    const int bt_lane = at.block_table[min(first + stride * lane, at.max_blocks - 1)];
    const int qp = qa.pos[0];
    // h and the norm weights for the RMSNorm
    StageRegs<CPT, X_RMSNORM> sr;
    stage_issue<CPT, X_RMSNORM, kLThreads, true>(qa, 0, sr);
    NX_TRACE(13);
    __syncthreads();  // every wavefront's share of h ahead of any weight tile
    NX_TRACE(14);
    // QKV rows: block b owns pairs [b P, b P + P), wavefront w a share of them
    const int npairs = qa.N / 2;
    const int pb0 = min(blk * L.qkv_pairs, npairs), pb1 = min(pb0 + L.qkv_pairs, npairs);
    int r0, r1;
    wave_rows(RowSplit{(pb1 - pb0) / kLWaves, (pb1 - pb0) % kLWaves, 1, kLWaves}, wave, 2 * (pb1 - pb0), r0, r1);
    r0 += 2 * pb0;
    r1 += 2 * pb0;
    Tile<GPL, kQkvRows> tq;
    load_tile_u<GPL, kQkvRows>(tq, qa.W, qa.S, qa.G, r0, r1, r0, lane);
    // the storing wavefront's RoPE factors (lane l: the block's pair l) and
    // the block of the position's page
    float qc, qs;
    {
        const int row = min(2 * (pb0 + lane), qa.qdim + qa.kvdim - 2);
        const int i = (row % qa.hd) >> 1;
        qc = qa.cos_t[(size_t)qp * (qa.hd >> 1) + i];
        qs = qa.sin_t[(size_t)qp * (qa.hd >> 1) + i];
    }
    const int qblk = qa.block_table[qp / kPage];
    NX_TRACE(15);

    // ---- 1. QKV ----------------------------------------------------------
    // Each wavefront reduces its rows into LDS; then it requests its page
    // pair and its wo rows, which stream while q / k / v are handed over.
    // One wavefront stores the block's q / k / v and counts the block in:
    // it has no other load in flight then, so waiting for its stores does
    // not wait for page or weight data.
    __shared__ float qres[kLWaves * kQkvRows];
    stage_finish<CPT, X_RMSNORM, kLThreads>(qa, sr, sp, s8, red);
    NX_TRACE(2);
    {
        XPairs<GPL> xp;
        load_pairs_lds<GPL>(xp, sp, s8, qa.G, lane);
        float res[kQkvRows];
        tile_dot<GPL, kQkvRows>(tq, xp, res);
        if (lane == 0)
#pragma unroll
            for (int r = 0; r < kQkvRows; ++r)
                if (r0 + r < r1) qres[r0 - 2 * pb0 + r] = res[r];
    }
    const int ctx = qp + 1, npages = (ctx + kPage - 1) / kPage;
    const int npw = first < npages ? min((npages - first + stride - 1) / stride, 2) : 0;
    auto valid_of = [&](int i) { return i < npw ? min(ctx - (first + stride * i) * kPage, kPage) : 0; };
    const int blka = __builtin_amdgcn_readlane(bt_lane, 0), blkb = __builtin_amdgcn_readlane(bt_lane, 1);
    int o0, o1;
    wave_rows(RowSplit{L.wo_rows.base, L.wo_rows.extra, (int)gridDim.x, kLWaves}, blk * kLWaves + wave, oa.N, o0, o1);
    PairRaw<HD> pr;
    Tile<GPLO, 2> to;
    constexpr int kStorer = kLWaves - 1;
    __syncthreads();
    if (wave == kStorer) {
        // lane l: the block's pair l -- RoPE on q / k rows, q -> q32, k / v
        // -> the fp16 page slot of the position (agent-scope stores)
        const int pi = lane, row = 2 * (pb0 + pi);
        if (pi < pb1 - pb0) {
            float v0 = qres[2 * pi], v1 = qres[2 * pi + 1];
            if (row < qa.qdim + qa.kvdim) {
                const float r0v = v0 * qc - v1 * qs;
                const float r1v = v0 * qs + v1 * qc;
                v0 = r0v;
                v1 = r1v;
            }
            if (row < qa.qdim) {
                st_coh(qa.q32 + row, v0);
                st_coh(qa.q32 + row + 1, v1);
            } else {
                const int kv = row < qa.qdim + qa.kvdim ? 0 : 1;
                const int idx = row - qa.qdim - kv * qa.kvdim;
                const int kh = idx / HD, dd = idx % HD, slot = qp % kPage;
                const size_t page = ((size_t)qblk * hkv + kh) * kPage * HD;
                if (kv) {  // V pages are dimension-major: [hd][16]
                    st_coh_u16(qa.vpool + page + (size_t)dd * kPage + slot, f2h_bits(v0));
                    st_coh_u16(qa.vpool + page + (size_t)(dd + 1) * kPage + slot, f2h_bits(v1));
                } else {   // K pages are token-major: [16][hd]; dd is even
                    st_coh_u32(reinterpret_cast<uint32_t*>(qa.kpool + page + (size_t)slot * HD + dd),
                               (uint32_t)f2h_bits(v0) | ((uint32_t)f2h_bits(v1) << 16));
                }
            }
        }
    }
    // the stores are requested ahead of any page or wo load of the CU (a CU
    // returns its requests in order), so their completion is one round trip
    __syncthreads();
    if (wave == kStorer) {
        // every store of the wavefront is complete before it counts the block in
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        NX_TRACE_BY(4, kStorer * kWave);
        if (lane == 0) {
            const unsigned mask = qkv_heads(2 * pb0, 2 * pb1, qa.qdim, qa.kvdim, G, HD, hkv);
            for (int g = 0; g < hkv; ++g)
                if (mask & (1u << g))
                    __hip_atomic_fetch_add(L.sync + g * kAttnCountStride, 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // this wavefront's pages (page b only when it holds tokens) and wo rows
    if (valid_of(1) > 0) {
        load_pair<HD>(pr, at, blka, valid_of(0), blkb, valid_of(1), kvh, lane);
    } else {
        load_page_a<HD>(pr, at, blka, valid_of(0), kvh, lane);
    }
    load_tile_u<GPLO, 2>(to, oa.W, oa.S, oa.G, o0, o1, o0, lane);
    NX_TRACE(3);

    // ---- 2. attention ----------------------------------------------------
    if (has_attn) {
        wait_count(L.sync + kvh * kAttnCountStride, (unsigned)L.qkv_expect[kvh] * ep, L.err, 1);
        NX_TRACE(5);
        // q of the G heads (B operand: column t = head, k = 8 g4 + j of each
        // 32-dim step; columns past G repeat head G - 1)
        h8_t qh[HD / 32], ql[HD / 32];
        {
            const __amdgpu_buffer_rsrc_t rq = rsrc(at.q, at.hq * HD * 4);
            const int qo = ((kvh * G + min(t, G - 1)) * HD + 8 * g4) * 4;
            uint4 x[HD / 32][2];
#pragma unroll
            for (int s = 0; s < HD / 32; ++s) {
                x[s][0] = ld_coh16(rq, qo + 128 * s);
                x[s][1] = ld_coh16(rq, qo + 128 * s + 16);
            }
            // the position's K / V slot, if this wavefront holds its page
            const int pc = qp / kPage, js = qp % kPage;
            const int ic = (pc >= first && (pc - first) % stride == 0) ? (pc - first) / stride : -1;
            if (ic == 0 || ic == 1) {
                const int cb = ic ? blkb : blka;
                const size_t page = ((size_t)cb * hkv + kvh) * kPage * HD;
                const __amdgpu_buffer_rsrc_t rk = rsrc(at.kpool + page, kPage * HD * 2);
                const __amdgpu_buffer_rsrc_t rv = rsrc(at.vpool + page, kPage * HD * 2);
                uint4 kn[HD / 32];
                uint2 vn[HD / 16];
#pragma unroll
                for (int s = 0; s < HD / 32; ++s) kn[s] = ld_coh16(rk, (js * HD + 32 * s + 8 * g4) * 2);
#pragma unroll
                for (int nt = 0; nt < HD / 16; ++nt) vn[nt] = ld_coh8(rv, ((16 * nt + t) * kPage + 4 * g4) * 2);
                const bool krow = t == js, vcol = g4 == js / 4;
#pragma unroll
                for (int s = 0; s < HD / 32; ++s) {
                    if (ic == 0 && krow) pr.k[0][s] = kn[s];
                    if (ic == 1 && krow) pr.k[1][s] = kn[s];
                }
#pragma unroll
                for (int nt = 0; nt < HD / 16; ++nt) {
                    if (ic == 0 && vcol) pr.v[nt][0] = vn[nt];
                    if (ic == 1 && vcol) pr.v[nt][1] = vn[nt];
                }
            }
#pragma unroll
            for (int s = 0; s < HD / 32; ++s) {
                const uint32_t w[8] = {x[s][0].x, x[s][0].y, x[s][0].z, x[s][0].w,
                                       x[s][1].x, x[s][1].y, x[s][1].z, x[s][1].w};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float v = __builtin_bit_cast(float, w[j]);
                    qh[s][j] = (_Float16)v;
                    ql[s][j] = (_Float16)(v - (float)qh[s][j]);
                }
            }
        }
        const float scale = 1.0f / sqrtf((float)HD);
        float m = -__builtin_inff(), lsum = 0.0f;
        f4_t o[HD / 16];
#pragma unroll
        for (int nt = 0; nt < HD / 16; ++nt) o[nt] = f4_t{0.f, 0.f, 0.f, 0.f};
        if (npw > 0) pair_update<HD>(pr, qh, ql, scale, valid_of(0), valid_of(1), m, lsum, o, lane);
        lsum += __shfl_xor(lsum, 16, 64);
        lsum += __shfl_xor(lsum, 32, 64);
        NX_TRACE(6);
        float* my = lds + wave * REC;
#pragma unroll
        for (int nt = 0; nt < HD / 16; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (4 * g4 + i < G) my[(4 * g4 + i) * HD + 16 * nt + t] = o[nt][i];
        if (g4 == 0 && t < G) {
            my[MO + t] = m;
            my[LO + t] = lsum;
        }
        float* parts = at.part + (size_t)kvh * nsplit * REC;
        merge_waves_store<G, HD, true>(parts + (size_t)split * REC, lds);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned* cnt = at.counts + (size_t)kvh * kAttnCountStride;
            const unsigned prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = prev == (unsigned)nsplit - 1u;
            if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        NX_TRACE(7);
        if (last) {
            merge_last<G, HD, false, true>(at, nsplit, 0, kvh, 0);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (threadIdx.x == 0)
                __hip_atomic_fetch_add(L.sync + hkv * kAttnCountStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            NX_TRACE(8);
        }
    }

    // ---- 3. wo + residual ----------------------------------------------
    wait_count(L.sync + hkv * kAttnCountStride, (unsigned)hkv * ep, L.err);
    NX_TRACE(9);
    stage_att<CPTO>(oa, sp, s8);
    NX_TRACE(10);
    {
        XPairs<GPLO> xo;
        load_pairs_lds<GPLO>(xo, sp, s8, oa.G, lane);
        float res[2];
        tile_dot<GPLO, 2>(to, xo, res);
        float bv = 0.0f;
        int bi = 0;
        if (lane == 0) epilogue<E_ACC, 2>(oa, 0, o0, o1, res, bv, bi);
    }
    NX_TRACE(11);
}

// The kernel instantiation for (G, head_dim, groups per lane of d and of
// hq * head_dim), or nullptr.
const void* layer_kernel(int G, int HD, int gpl, int gplo) {
#define NX_LAYER_CASE(GG, HH, P1, P2) \
    if (G == GG && HD == HH && gpl == P1 && gplo == P2) return (const void*)k_attn_block_b1<GG, HH, P1, P2>;
#define NX_LAYER_G(GG, HH)         \
    NX_LAYER_CASE(GG, HH, 1, 1)    \
    NX_LAYER_CASE(GG, HH, 1, 2)    \
    NX_LAYER_CASE(GG, HH, 2, 1)    \
    NX_LAYER_CASE(GG, HH, 2, 2)
    NX_LAYER_G(1, 64)
    NX_LAYER_G(2, 64)
    NX_LAYER_G(4, 64)
    NX_LAYER_G(8, 64)
    NX_LAYER_G(1, 128)
    NX_LAYER_G(2, 128)
    NX_LAYER_G(4, 128)
    NX_LAYER_G(8, 128)
#undef NX_LAYER_G
#undef NX_LAYER_CASE
    return nullptr;
}

}  // namespace

bool attn_block_b1_plan(int d, int hq, int hkv, int hd, int max_ctx, LayerArgs& p) {
    const int G = hkv > 0 ? hq / hkv : 0;
    if (hkv <= 0 || hkv > 32 || hq % hkv || (G != 1 && G != 2 && G != 4 && G != 8) || (hd != 64 && hd != 128))
        return false;
    const int qdim = hq * hd, kvdim = hkv * hd;
    if (d % 8 || d > 4096 || qdim > 4096 || max_ctx < 1) return false;
    const int gpl = ((d + 31) / 32 + kWave - 1) / kWave, gplo = ((qdim + 31) / 32 + kWave - 1) / kWave;
    const void* fn = layer_kernel(G, hd, gpl, gplo);
    if (!fn) return false;
    const int NB = device_cus();
    const int nw = NB * kLWaves;
    // every block resident at once: one per CU
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, kLThreads, 0) != hipSuccess || occ < 1) return false;
    // QKV pairs: at most kQkvRows / 2 per wavefront
    const int npairs = (qdim + 2 * kvdim) / 2;
    const int pb = (npairs + NB - 1) / NB;
    if (pb > kLWaves * kQkvRows / 2) return false;
    // wo: at most one pair per wavefront
    if ((d + 1) / 2 > nw) return false;
    // attention: nsplit per kv head, at most two pages per wavefront
    const int pages = (max_ctx + kPage - 1) / kPage;
    const int nsplit = std::min(std::min(NB / hkv, pages), kMaxSplits);
    if (nsplit < 1 || (pages + nsplit * kLWaves - 1) / (nsplit * kLWaves) > 2) return false;
    p.nsplit = nsplit;
    p.qkv_pairs = pb;
    p.wo_rows = gv_rowsplit_t{((d + 1) / 2) / nw, ((d + 1) / 2) % nw};
    for (int g = 0; g < 32; ++g) p.qkv_expect[g] = 0;
    for (int b = 0; b < NB; ++b) {
        const int a0 = std::min(b * pb, npairs), a1 = std::min(a0 + pb, npairs);
        const unsigned mask = qkv_heads(2 * a0, 2 * a1, qdim, kvdim, G, hd, hkv);
        for (int g = 0; g < hkv; ++g)
            if (mask & (1u << g)) ++p.qkv_expect[g];
    }
    return true;
}

#ifdef NX_LAYER_TRACE
extern "C" int nx_debug_layer_trace(unsigned long long* out) {
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(g_layer_trace), sizeof(unsigned long long) * 1024 * 16);
}
#endif

hipError_t attn_block_b1_launch(const LayerArgs& a, hipStream_t st) {
    const int G = a.at.hq / a.at.hkv;
    const int gpl = (a.qkv.G + kWave - 1) / kWave, gplo = (a.wo.G + kWave - 1) / kWave;
    const void* fn = layer_kernel(G, a.at.hd, gpl, gplo);
    if (!fn) return hipErrorInvalidValue;
    void* args[] = {const_cast<LayerArgs*>(&a)};
    return hipLaunchKernel(fn, dim3(device_cus()), dim3(kLThreads), args, 0, st);
}

}  // namespace nx
