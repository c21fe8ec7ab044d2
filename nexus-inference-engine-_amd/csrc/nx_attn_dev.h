// Device building blocks of the paged decode attention kernels (nx_attn.hip):
// split records and their merge, the fp16 page-pair product on the matrix
// cores, and the agent-scope (cross-XCD coherent) accesses used for the
// hand-off of split records to the merging block of the same launch.
#pragma once

#include "nx_common.h"
#include "nx_kernels.h"

namespace nx {
namespace at {

constexpr int kAttnWaves = 8;
constexpr int kAttnThreads = kAttnWaves * kWave;
constexpr int kMaxSplits = 64;  // splits per (sequence, kv head)

// Split partial record, float offsets: O[G][HD] at 0, M[G], L[G], padded to 16 bytes.
__host__ __device__ constexpr int rec_floats(int G, int HD) { return (G * HD + 2 * G + 3) / 4 * 4; }


// Agent-scope (coherent across XCDs) store and load of a split record word,
// for records handed to the block that merges them within the same launch.
__device__ inline void st_coh(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float ld_coh(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The arguments a split block reads first, requested together from the
// argument segment (the compiler would otherwise fetch them in several
// dependent rounds as each is first needed).
__device__ inline void attn_args_early(const AttnArgs& a) {
    asm volatile("" ::"s"(a.q), "s"(a.block_table), "s"(a.ctx_lens), "s"(a.pos), "s"(a.hq), "s"(a.hkv),
                 "s"(a.max_blocks), "s"(a.hot_window), "s"(a.check_blocks));
}

// The part of sequence b's context a block covers: all of it (range 0), or
// with tiered pages the TurboQuant pages [cool, cold) (range 1, from page
// cool / 16 on), the fp16 window [cold, ctx) (range 2, read from page cold /
// 16 of the hot table on) or the Cool pages [evict, cool) (range 3).  cold = 16
// floor((ctx - 1 - hot_window) / 16), at least 0: the pages compressed
// before this step (the page that leaves the window at this step is
// compressed by the same launch and read here as fp16); cool likewise with
// hot_window + warm_window, 0 without a Cool tier (warm_window 0), evict
// with hot_window + warm_window + cool_window, 0 without eviction.
__device__ inline void attn_range(const AttnArgs& a, int b, int range, int& ctx, int& pg0) {
    ctx = a.ctx_lens ? a.ctx_lens[b] : a.pos[b] + 1;
    pg0 = 0;
    if (range != 0) {
        const int cold = kPage * max(0, (ctx - 1 - a.hot_window) / kPage);
        const int cool = a.warm_window > 0 ? kPage * max(0, (ctx - 1 - a.hot_window - a.warm_window) / kPage) : 0;
        if (range == 1) {  // Warm: [cool, cold)
            pg0 = cool / kPage;
            ctx = cold - cool;
        } else if (range == 3) {  // Cool: [evict, cool)
            const int evict =
                a.cool_window > 0 ? kPage * max(0, (ctx - 1 - a.hot_window - a.warm_window - a.cool_window) / kPage)
                                  : 0;
            pg0 = evict / kPage;
            ctx = max(cool - evict, 0);
        } else {  // fp16: [cold, ctx)
            pg0 = cold / kPage;
            ctx -= cold;
        }
    }
}

// Cross-wavefront merge of the block: lds holds one record per wavefront
// (O[G][HD], M[G], L[G]); every wavefront has written its own before the
// barrier.  The rescale factors exp(m_w - M) are computed once per (wavefront,
// head) by the first G * kAttnWaves lanes of wavefront 0 (max and sum over
// groups of kAttnWaves lanes), then every thread sums its O elements over the
// wavefronts.  The merged split record goes to `part` (COH: agent-scope
// stores).
template <int G, int HD, bool COH = false>
__device__ inline void merge_waves_store(float* __restrict__ part, const float* lds) {
    constexpr int REC = rec_floats(G, HD), MO = G * HD, LO = G * HD + G;
    static_assert(G * kAttnWaves <= kWave, "one lane of wavefront 0 per (wavefront, head)");
    __shared__ float fw[kAttnWaves * G];
    __syncthreads();
    const int t = threadIdx.x;
    if (t < kWave) {
        const bool act = t < G * kAttnWaves;
        const int h = act ? t / kAttnWaves : 0, w = t % kAttnWaves;
        const float m = act ? lds[w * REC + MO + h] : -__builtin_inff();
        float M = m;
#pragma unroll
        for (int o = 1; o < kAttnWaves; o <<= 1) M = fmaxf(M, __shfl_xor(M, o, kWave));
        const float f = (M == -__builtin_inff()) ? 0.0f : __expf(m - M);
        float L = act ? f * lds[w * REC + LO + h] : 0.0f;
#pragma unroll
        for (int o = 1; o < kAttnWaves; o <<= 1) L += __shfl_xor(L, o, kWave);
        if (act) {
            fw[w * G + h] = f;
            if (w == 0) {
                if (COH) {
                    st_coh(part + MO + h, M);
                    st_coh(part + LO + h, L);
                } else {
                    part[MO + h] = M;
                    part[LO + h] = L;
                }
            }
        }
    }
    __syncthreads();
    for (int idx = t; idx < G * HD; idx += kAttnThreads) {
        const int h = idx / HD;
        float acc = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) acc = fmaf(lds[w * REC + idx], fw[w * G + h], acc);
        if (COH)
            st_coh(part + idx, acc);
        else
            part[idx] = acc;
    }
}

// ------------------------------------------------------------ fp16 pages --
// q.K^T and P.V run on the matrix cores (v_mfma_f32_16x16x32_f16, wave64):
//   A operand (16 x 32): lane l holds row l%16, k = 8(l/16) .. +7
//   B operand (32 x 16): lane l holds column l%16, k = 8(l/16) .. +7
//   C (16 x 16 fp32):    lane l holds column l%16, rows 4(l/16) .. +3
// Scores S = K q^T per page: M = the page's 16 tokens, N = query heads (G of
// 16 columns used), K = head dims.  A K page row is read straight into the A
// operand (16 bytes per lane per k-step).  q enters as fp16 hi + lo parts
// (q = hi + lo to 2^-22), so the two products give the fp32 score; K is exact
// fp16 and the products accumulate in fp32.
// Values O = P V per page pair: M = heads, N = 16 dims per tile, K = the 32
// tokens of two pages.  The token order of that K dimension is chosen so the
// probabilities a lane needs are exactly the 8 scores it holds in the S
// layout (k = 8g + j: page a token 4g + j for j < 4, page b token 4g + j - 4),
// and V pages are stored dimension-major ([hd][16] per page), so the B
// operand is two 8-byte reads per lane.  P enters as fp16 hi + lo as well.
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

__device__ inline h8_t as_h8(uint4 v) { return __builtin_bit_cast(h8_t, v); }

template <int HD>
struct PairRaw {
    uint4 k[2][HD / 32];  // K of pages a, b: A operand per k-step
    uint2 v[HD / 16][2];  // V of pages a, b: tokens 4g..4g+3 of dim 16 nt + l%16
};

// The low fp16 parts (K - fp16(K)) of a pair's K, same layout as PairRaw::k.
template <int HD>
struct PairKlo {
    uint4 k[2][HD / 32];
};

// Bits of a lane's V words (tokens 4g .. 4g+3, fp16 each) that hold the first
// n tokens of the page.
__device__ inline uint2 vmask_of(int n, int g) {
    const int valid = min(max(n - 4 * g, 0), 4);
    return make_uint2((uint32_t)(0xFFFFFFFFull >> (16 * (2 - min(valid, 2)))),
                      (uint32_t)(0xFFFFFFFFull >> (16 * (2 - max(valid - 2, 0)))));
}

// Load pages a and b of a pair; na / nb = valid tokens of each (0 = none).
// A page's loads are issued unconditionally, because a branch or a select
// around a load makes the compiler wait for that load at once and the page
// would arrive one round trip per tile: K rows of tokens past the valid count
// are left as loaded (their scores are masked in pair_update), and the V
// words of those tokens are cleared with masks (vmask_of, in pair_update).
// Page b with no valid token (nb <= 0, the same for the whole wavefront) is
// not requested at all: its registers are zero, its scores masked and its V
// words cleared.  (Re-reading page a instead cost the one-page wavefronts of
// a batch-1 split 1 us per launch: 8B decode attention 10.5 against 9.5 us.)
template <int HD>
__device__ inline void load_pair(PairRaw<HD>& r, const AttnArgs& a, int blka, int na, int blkb,
                                 int nb, int kvh, int lane) {
    const int g = lane >> 4, t = lane & 15;
#pragma unroll
    for (int pg = 0; pg < 2; ++pg) {
        if (pg == 1 && nb <= 0) {
#pragma unroll
            for (int s = 0; s < HD / 32; ++s) r.k[1][s] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
            for (int nt = 0; nt < HD / 16; ++nt) r.v[nt][1] = make_uint2(0u, 0u);
            break;
        }
        const int blk = pg ? blkb : blka;
        const size_t base = ((size_t)blk * a.hkv + kvh) * kPage * HD;
#pragma unroll
        for (int s = 0; s < HD / 32; ++s)
            r.k[pg][s] = *reinterpret_cast<const uint4*>(a.kpool + base + (size_t)t * HD + 32 * s + 8 * g);
#pragma unroll
        for (int nt = 0; nt < HD / 16; ++nt)
            r.v[nt][pg] = *reinterpret_cast<const uint2*>(a.vpool + base + (size_t)(16 * nt + t) * kPage + 4 * g);
    }
    // keep the V loads ahead of the first product (the scheduler would sink
    // them below the wait for K, costing a second round trip)
    __builtin_amdgcn_sched_barrier(0);
}

// load_pair with each page's pools given (ka / va for page a, kb / vb for
// page b; wavefront-uniform choices): the tiered prefill reads a query
// tile's pages before its cold boundary from the decoded TurboQuant pages
// and the others from fp16 pages.  Page b with no valid token re-reads page a.
template <int HD>
__device__ inline void load_pair_from(PairRaw<HD>& r, const uint16_t* ka, const uint16_t* va, int blka,
                                      const uint16_t* kb, const uint16_t* vb, int blkb, int nb, int hkv, int kvh,
                                      int lane) {
    const int g = lane >> 4, t = lane & 15;
    const bool dup = nb <= 0;
#pragma unroll
    for (int pg = 0; pg < 2; ++pg) {
        const int blk = pg && !dup ? blkb : blka;
        const uint16_t* kp = pg && !dup ? kb : ka;
        const uint16_t* vp = pg && !dup ? vb : va;
        const size_t base = ((size_t)blk * hkv + kvh) * kPage * HD;
#pragma unroll
        for (int s = 0; s < HD / 32; ++s)
            r.k[pg][s] = *reinterpret_cast<const uint4*>(kp + base + (size_t)t * HD + 32 * s + 8 * g);
#pragma unroll
        for (int nt = 0; nt < HD / 16; ++nt)
            r.v[nt][pg] = *reinterpret_cast<const uint2*>(vp + base + (size_t)(16 * nt + t) * kPage + 4 * g);
    }
    __builtin_amdgcn_sched_barrier(0);
}

// Fold one page pair into the wavefront's state: m (running max of head l%16),
// lsum (this lane's share of the softmax denominator), O (C layout, rows =
// heads 4(l/16) + i, columns = dims 16 nt + l%16).
// CAUSAL (prefill): the columns are query tokens instead of heads; token
// 4(l/16) + i of page a (b) is at position pos_a (pos_b) + 4(l/16) + i and
// is masked for the query at position qpos (this lane's column) when later.
// KLO: K is fp16 hi + lo (kl), a third product K_lo q_hi per step.
// QL (256-long heads): q's hi and lo operands are read from LDS per k-step
// (qls[2s], qls[2s + 1]) instead of qh / ql, so they take no registers across
// the page pair (a pair's K and V take 128 VGPRs there).
template <int HD, bool CAUSAL = false, bool KLO = false, bool QL = false>
__device__ inline void pair_update(const PairRaw<HD>& r, const h8_t (&qh)[HD / 32],
                                   const h8_t (&ql)[HD / 32], float scale, int na, int nb, float& m,
                                   float& lsum, f4_t (&o)[HD / 16], int lane, int pos_a = 0, int pos_b = 0,
                                   int qpos = 0, const PairKlo<HD>* kl = nullptr, const uint4* qls = nullptr) {
    const int g = lane >> 4;
    f4_t sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < HD / 32; ++s) {
        h8_t qhs, qls_;
        if constexpr (QL) {
            qhs = as_h8(qls[2 * s]);
            qls_ = as_h8(qls[2 * s + 1]);
        } else {
            qhs = qh[s];
            qls_ = ql[s];
        }
        sa = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(r.k[0][s]), qhs, sa, 0, 0, 0);
        sa = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(r.k[0][s]), qls_, sa, 0, 0, 0);
        sb = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(r.k[1][s]), qhs, sb, 0, 0, 0);
        sb = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(r.k[1][s]), qls_, sb, 0, 0, 0);
        if constexpr (KLO) {
            sa = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(kl->k[0][s]), qhs, sa, 0, 0, 0);
            sb = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(kl->k[1][s]), qhs, sb, 0, 0, 0);
        }
    }
    float p[8];
    float mloc = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const bool va = 4 * g + i < na && (!CAUSAL || pos_a + 4 * g + i <= qpos);
        const bool vb = 4 * g + i < nb && (!CAUSAL || pos_b + 4 * g + i <= qpos);
        p[i] = va ? sa[i] * scale : -__builtin_inff();
        p[4 + i] = vb ? sb[i] * scale : -__builtin_inff();
        mloc = fmaxf(mloc, fmaxf(p[i], p[4 + i]));
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    const float mn = fmaxf(m, mloc);
    const bool none = mn == -__builtin_inff();
    const float corr = none ? 1.0f : __expf(m - mn);
    float ps = 0.0f;
    h8_t ph, pl;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float e = none ? 0.0f : __expf(p[j] - mn);
        ps += e;
        ph[j] = (_Float16)e;
        pl[j] = (_Float16)(e - (float)ph[j]);
    }
    lsum = lsum * corr + ps;
    m = mn;
    // V words of tokens past the valid counts are cleared (they may hold
    // anything, and their zero weights must not meet a NaN)
    const uint2 ma = vmask_of(na, g), mb = vmask_of(nb, g);
    // rows of O in this lane are heads 4g + i; their rescale factors live in
    // the lanes whose column is that head
    float c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = __shfl(corr, 4 * g + i, 64);
#pragma unroll
    for (int nt = 0; nt < HD / 16; ++nt) {
        f4_t acc = o[nt];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] *= c[i];
        const h8_t vb = as_h8(make_uint4(r.v[nt][0].x & ma.x, r.v[nt][0].y & ma.y, r.v[nt][1].x & mb.x,
                                         r.v[nt][1].y & mb.y));
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, vb, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, vb, acc, 0, 0, 0);
        o[nt] = acc;
    }
}


// FWHT of one vector of 128 held by a wavefront, lane l holding elements l
// (u0) and l + 64 (u1): the canonical butterfly network, stages h = 1, 2,
// .., 64 each taking (x_j, x_{j+h}) -> (x_j + x_{j+h}, x_j - x_{j+h}) for the
// j with bit h clear (h <= 32 across lanes, h = 64 inside the lane).  On
// return element l is u0 and element l + 64 is u1.
__device__ inline void wave_fwht128(float& u0, float& u1) {
    const int lane = threadIdx.x & 63;
    for (int h = 1; h < 64; h <<= 1) {
        const float p0 = __shfl_xor(u0, h, 64), p1 = __shfl_xor(u1, h, 64);
        if (lane & h) {
            u0 = p0 - u0;
            u1 = p1 - u1;
        } else {
            u0 = u0 + p0;
            u1 = u1 + p1;
        }
    }
    const float a = u0 + u1, b = u0 - u1;
    u0 = a;
    u1 = b;
}

constexpr float kTqScale = 0.08838834764831845f;  // float(1/sqrt(128))

// Run by the last split block of a (sequence, kv head) to finish: merges the
// nsplit records of its G query heads and writes the fp16 output.  The
// records were stored by other blocks with agent-scope stores, each complete
// before its block counted itself, so they are read with agent-scope (sc1)
// loads.  Wavefront w computes the weights exp(m_s - M) / L of heads
// w, w + 4, ... with lane s holding split s (nsplit <= 64).  Thread t then
// owns float4 column t % NC of O (NC = G * HD / 4) for the splits
// s = t / NC (mod NG), NG = 256 / NC; it requests all of them at once
// (16-byte buffer loads with the sc1 bit, skipped past nsplit, where the
// weight is zero), and the NG partial sums meet in LDS.
// TQ: the value sums of records [0, ntq) are in the rotated domain (all of
// them for TurboQuant pages, the compressed part for tiered pages); their
// merged sum is rotated back (o = D_v H o~ / sqrt(128), an FWHT in LDS) and
// added to the merged sum of the fp16 records [ntq, nsplit).
template <int G, int HD, bool TQ = false>
__device__ inline void merge_last(const AttnArgs& a, int nsplit, int ntq, int kvh, int b) {
    constexpr int REC = rec_floats(G, HD), MO = G * HD, LO = G * HD + G;
    constexpr int NC = G * HD / 4, NG = kAttnThreads / NC;
    constexpr int KMAX = (kMaxSplits + NG - 1) / NG, U = KMAX < 16 ? KMAX : 16;
    constexpr int kSc1 = 16;  // cache-policy bit of the agent-scope load
    static_assert(kMaxSplits <= kWave, "one split per lane");
    static_assert(NC * NG == kAttnThreads, "float4 columns tile the block");
    __shared__ float wgt[G * kMaxSplits];
    __shared__ float4 acc4[kAttnThreads];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const float* parts = a.part + ((size_t)b * a.hkv + kvh) * nsplit * REC;
    const int c = tid % NC, sg = tid / NC, h = 4 * c / HD;
    // evicted positions (three tiers with a Cool window): zero keys and
    // values, each a score of 0 in the softmax and nothing in the sum
    float nev = 0.0f;
    if constexpr (TQ) {
        if (a.cool_window > 0 && a.warm_window > 0) {
            const int ctx = a.ctx_lens ? a.ctx_lens[b] : a.pos[b] + 1;
            nev = (float)(kPage * max(0, (ctx - 1 - a.hot_window - a.warm_window - a.cool_window) / kPage));
        }
    }
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(parts), 0, nsplit * REC * 4, 0x00020000);
    typedef float f4v __attribute__((ext_vector_type(4)));
    // the first batch of O columns is requested together with the split
    // maxima and denominators: one round trip for both
    // (s is uniform within a wavefront, as NC is a multiple of 64 or NG
    // divides the wavefront evenly; every load is consumed only after all
    // of them are issued)
    f4v v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int sx = sg + u * NG;
        v[u] = sx < nsplit ? __builtin_amdgcn_raw_buffer_load_b128(rs, (sx * REC + 4 * c) * 4, 0, kSc1)
                           : f4v{0.f, 0.f, 0.f, 0.f};
    }
    for (int hh = wave; hh < G; hh += kAttnWaves) {
        const bool ok = lane < nsplit;
        const int sl = ok ? lane : nsplit - 1;
        const float m = ld_coh(parts + (size_t)sl * REC + MO + hh);
        const float l = ld_coh(parts + (size_t)sl * REC + LO + hh);
        const float M = nev > 0.0f ? fmaxf(wave_max(m), 0.0f) : wave_max(m);
        const float e = (ok && M != -__builtin_inff()) ? __expf(m - M) : 0.0f;
        const float L = wave_sum(e * l) + (nev > 0.0f ? nev * __expf(-M) : 0.0f);
        // a NaN denominator (NaN scores, or a sequence the kernel's table
        // check rejected) stays NaN in the output rather than becoming zero
        wgt[hh * kMaxSplits + lane] = L > 0.0f ? e / L : (L == L ? 0.0f : L);
    }
    f4v acc = {0.f, 0.f, 0.f, 0.f}, accp = {0.f, 0.f, 0.f, 0.f};  // rotated, plain records
    __syncthreads();
    for (int s0 = sg;;) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int sx = s0 + u * NG;
            const float w = wgt[h * kMaxSplits + min(sx, kMaxSplits - 1)] * (sx < nsplit ? 1.0f : 0.0f);
            if constexpr (TQ) {
                const float wr = sx < ntq ? w : 0.0f;
                acc += wr * v[u];
                accp += (w - wr) * v[u];
            } else {
                acc += w * v[u];
            }
        }
        s0 += NG * U;
        if (s0 >= nsplit) break;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int sx = s0 + u * NG;
            v[u] = sx < nsplit ? __builtin_amdgcn_raw_buffer_load_b128(rs, (sx * REC + 4 * c) * 4, 0, kSc1)
                               : f4v{0.f, 0.f, 0.f, 0.f};
        }
    }
    auto group_sum = [&]() {
        float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
        if (tid < NC) {
            r = acc4[tid];
            for (int gi = 1; gi < NG; ++gi) {
                const float4 q = acc4[gi * NC + tid];
                r.x += q.x;
                r.y += q.y;
                r.z += q.z;
                r.w += q.w;
            }
        }
        return r;
    };
    acc4[tid] = make_float4(acc.x, acc.y, acc.z, acc.w);
    __syncthreads();
    const float4 r = group_sum();
    uint16_t* out = a.out16 + ((size_t)b * a.hq + (size_t)kvh * G) * HD;
    if constexpr (TQ) {
        static_assert(HD == 128, "TurboQuant vectors are 128 long");
        __shared__ float ov[G * HD], ovp[G * HD];
        if (tid < NC) *reinterpret_cast<float4*>(&ov[4 * tid]) = r;
        __syncthreads();
        acc4[tid] = make_float4(accp.x, accp.y, accp.z, accp.w);
        __syncthreads();
        const float4 rp = group_sum();
        if (tid < NC) *reinterpret_cast<float4*>(&ovp[4 * tid]) = rp;
        __syncthreads();
        // head w rotated back in wavefront w
        for (int hh = wave; hh < G; hh += kAttnWaves) {
            float u0 = ov[hh * HD + lane], u1 = ov[hh * HD + lane + 64];
            wave_fwht128(u0, u1);
            out[hh * HD + lane] = f2h_bits(u0 * kTqScale * a.vsign[lane] + ovp[hh * HD + lane]);
            out[hh * HD + lane + 64] = f2h_bits(u1 * kTqScale * a.vsign[lane + 64] + ovp[hh * HD + lane + 64]);
        }
    } else if (tid < NC) {
        const uint32_t w0 = (uint32_t)f2h_bits(r.x) | ((uint32_t)f2h_bits(r.y) << 16);
        const uint32_t w1 = (uint32_t)f2h_bits(r.z) | ((uint32_t)f2h_bits(r.w) << 16);
        *reinterpret_cast<uint2*>(out + 4 * tid) = make_uint2(w0, w1);
    }
}

}  // namespace at
}  // namespace nx
