// Paged decode attention on gfx950 over fp16 pages and TurboQuant pages.
//
// Grid (split, kv head, sequence); 4 wavefronts per block.  A block owns a
// contiguous range of 16-token pages of one kv head and serves the G = hq/hkv
// query heads that share it, so every K/V byte is read once per step.
// Within a wavefront lane l owns dims [l%16 * DPL, +DPL) of the tokens
// l/16, l/16+4, l/16+8, l/16+12 of each page; a score is reduced over the 16
// lanes of a DPP row.  A block owns 8 pages (more for very long contexts);
// each wavefront requests its block-table entries with q and then keeps two
// pairs of pages in flight.  Each DPP row keeps its own online-softmax state
// (m, l, o); rows and wavefronts are merged with the usual rescaling and the
// block stores one split record.  fp16 pages: the last block of a (sequence,
// kv head) to count itself done merges its split records and writes the fp16
// output; records and counters use agent-scope (cross-XCD coherent) relaxed
// accesses, with each block's stores complete before it counts, and no
// device-scope fence.  TurboQuant pages: a second small launch merges.
//
// TurboQuant pages are scored in the rotated domain: the block rotates q once
// (q~ = H D q / sqrt(128)), scores are n_t * <q~, c[code_t]>, V is summed in the
// rotated domain and rotated back (D H o~ / sqrt(128)) once after the merge.
#include "nx_common.h"
#include "nx_kernels.h"

namespace nx {

namespace {

constexpr int kAttnWaves = 8;
constexpr int kAttnThreads = kAttnWaves * kWave;
constexpr int kMaxSplits = 64;  // splits per (sequence, kv head)

struct SplitPlan {
    int nsplit, pps;  // splits per (sequence, kv head), pages per split
};

// A split is 8 pages (two per wavefront, all in flight at once) until
// kMaxSplits splits per (sequence, kv head) are reached; longer contexts get
// more pages per split.  A wavefront keeps its block-table entries one per
// lane, which bounds a split at 4 * 64 pages: contexts up to
// kMaxSplits * 256 pages (attn_max_ctx() tokens).
constexpr int kPagesPerSplitMin = 2 * kAttnWaves;
constexpr int kPagesPerSplitMax = kAttnWaves * kWave;

SplitPlan plan_splits(int max_ctx) {
    const int pages = (max_ctx + kPage - 1) / kPage;
    int pps = kPagesPerSplitMin;
    if ((pages + pps - 1) / pps > kMaxSplits) pps = (pages + kMaxSplits - 1) / kMaxSplits;
    int nsplit = (pages + pps - 1) / pps;
    if (nsplit < 1) nsplit = 1;
    return {nsplit, pps};
}

// Split partial record, float offsets: O[G][HD] at 0, M[G], L[G], padded to 16 bytes.
__host__ __device__ constexpr int rec_floats(int G, int HD) { return (G * HD + 2 * G + 3) / 4 * 4; }


// Online-softmax state of one lane: G heads x DPL dims.
template <int G, int DPL>
struct State {
    float m[G], l[G], o[G][DPL];
};

template <int G, int DPL>
__device__ inline void state_init(State<G, DPL>& s) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
        s.m[h] = -__builtin_inff();
        s.l[h] = 0.0f;
#pragma unroll
        for (int d = 0; d < DPL; ++d) s.o[h][d] = 0.0f;
    }
}

// Fold four token scores (per head) and their value rows into the state.
template <int G, int DPL>
__device__ inline void state_update(State<G, DPL>& s, const float (&sc)[4][G],
                                    const float (&v)[4][DPL]) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float mn = s.m[h];
#pragma unroll
        for (int j = 0; j < 4; ++j) mn = fmaxf(mn, sc[j][h]);
        if (mn == -__builtin_inff()) continue;  // nothing valid yet
        const float corr = __expf(s.m[h] - mn);
        float p[4], psum = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            p[j] = __expf(sc[j][h] - mn);
            psum += p[j];
        }
        s.l[h] = s.l[h] * corr + psum;
#pragma unroll
        for (int d = 0; d < DPL; ++d) {
            float acc = s.o[h][d] * corr;
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = fmaf(p[j], v[j][d], acc);
            s.o[h][d] = acc;
        }
        s.m[h] = mn;
    }
}

// Lane-wise sum over the four DPP rows (lanes i, i^16, i^32, i^48): every
// lane ends with the total of its column, in a fixed order.
__device__ inline float cols4_sum(float v) {
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// Merge the four DPP rows of a wavefront; every row ends with the merged state.
template <int G, int DPL>
__device__ inline void state_merge_rows(State<G, DPL>& s) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float M = s.m[h];
        M = fmaxf(M, readlane_f(s.m[h], 0));
        M = fmaxf(M, readlane_f(s.m[h], 16));
        M = fmaxf(M, readlane_f(s.m[h], 32));
        M = fmaxf(M, readlane_f(s.m[h], 48));
        const float f = (M == -__builtin_inff()) ? 0.0f : __expf(s.m[h] - M);
        s.l[h] = cols4_sum(s.l[h] * f);
#pragma unroll
        for (int d = 0; d < DPL; ++d) s.o[h][d] = cols4_sum(s.o[h][d] * f);
        s.m[h] = M;
    }
}

// Agent-scope (coherent across XCDs) store and load of a split record word,
// for records handed to the block that merges them within the same launch.
__device__ inline void st_coh(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float ld_coh(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// Block-level merge of the wavefronts' online-softmax states (row layout of
// the TurboQuant kernel) through LDS, then store this split's record.
template <int G, int HD>
__device__ inline void block_merge_store(const State<G, HD / 16>& s, float* __restrict__ part,
                                         float* lds) {
    constexpr int DPL = HD / 16, REC = rec_floats(G, HD), MO = G * HD, LO = G * HD + G;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float* my = lds + wave * REC;
    if (lane < 16) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            if (lane == 0) {
                my[MO + h] = s.m[h];
                my[LO + h] = s.l[h];
            }
#pragma unroll
            for (int d = 0; d < DPL; ++d) my[h * HD + lane * DPL + d] = s.o[h][d];
        }
    }
    merge_waves_store<G, HD>(part, lds);
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
    uint2 vmask[2];       // per page: bits of the V words that hold valid tokens
};

// Load pages a and b of a pair; na / nb = valid tokens of each (0 = none).
// Every load is issued unconditionally, because a branch or a select around a
// load makes the compiler wait for that load at once and the page would
// arrive one round trip per tile: page b with no valid token re-reads page a
// (blka must be a valid block), K rows of tokens past the valid count are
// left as loaded (their scores are masked in pair_update), and the V words
// of those tokens are cleared with masks.
template <int HD>
__device__ inline void load_pair(PairRaw<HD>& r, const AttnArgs& a, int blka, int na, int blkb,
                                 int nb, int kvh, int lane) {
    const int g = lane >> 4, t = lane & 15;
    const int pb = nb > 0 ? blkb : blka;
#pragma unroll
    for (int pg = 0; pg < 2; ++pg) {
        const int blk = pg ? pb : blka, n = pg ? nb : na;
        const size_t base = ((size_t)blk * a.hkv + kvh) * kPage * HD;
#pragma unroll
        for (int s = 0; s < HD / 32; ++s)
            r.k[pg][s] = *reinterpret_cast<const uint4*>(a.kpool + base + (size_t)t * HD + 32 * s + 8 * g);
        // tokens 4g .. 4g+3 of the V words: the first `valid` are kept
        // (applied in pair_update, so that nothing here waits for the data)
        const int valid = min(max(n - 4 * g, 0), 4);
        r.vmask[pg] = make_uint2((uint32_t)(0xFFFFFFFFull >> (16 * (2 - min(valid, 2)))),
                                 (uint32_t)(0xFFFFFFFFull >> (16 * (2 - max(valid - 2, 0)))));
#pragma unroll
        for (int nt = 0; nt < HD / 16; ++nt)
            r.v[nt][pg] = *reinterpret_cast<const uint2*>(a.vpool + base + (size_t)(16 * nt + t) * kPage + 4 * g);
    }
    // keep the V loads ahead of the first product (the scheduler would sink
    // them below the wait for K, costing a second round trip)
    __builtin_amdgcn_sched_barrier(0);
}

// Fold one page pair into the wavefront's state: m (running max of head l%16),
// lsum (this lane's share of the softmax denominator), O (C layout, rows =
// heads 4(l/16) + i, columns = dims 16 nt + l%16).
template <int HD>
__device__ inline void pair_update(const PairRaw<HD>& r, const h8_t (&qh)[HD / 32],
                                   const h8_t (&ql)[HD / 32], float scale, int na, int nb, float& m,
                                   float& lsum, f4_t (&o)[HD / 16], int lane) {
    const int g = lane >> 4;
    f4_t sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < HD / 32; ++s) {
        sa = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(r.k[0][s]), qh[s], sa, 0, 0, 0);
        sa = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(r.k[0][s]), ql[s], sa, 0, 0, 0);
        sb = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(r.k[1][s]), qh[s], sb, 0, 0, 0);
        sb = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(r.k[1][s]), ql[s], sb, 0, 0, 0);
    }
    float p[8];
    float mloc = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        p[i] = 4 * g + i < na ? sa[i] * scale : -__builtin_inff();
        p[4 + i] = 4 * g + i < nb ? sb[i] * scale : -__builtin_inff();
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
        const h8_t vb = as_h8(make_uint4(r.v[nt][0].x & r.vmask[0].x, r.v[nt][0].y & r.vmask[0].y,
                                         r.v[nt][1].x & r.vmask[1].x, r.v[nt][1].y & r.vmask[1].y));
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, vb, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, vb, acc, 0, 0, 0);
        o[nt] = acc;
    }
}


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
template <int G, int HD>
__device__ inline void merge_last(const AttnArgs& a, int nsplit, int kvh, int b) {
    constexpr int REC = rec_floats(G, HD), MO = G * HD, LO = G * HD + G;
    constexpr int NC = G * HD / 4, NG = kAttnThreads / NC;
    constexpr int KMAX = (kMaxSplits + NG - 1) / NG, U = KMAX < 16 ? KMAX : 16;
    constexpr int kSc1 = 16;  // cache-policy bit of the agent-scope load
    static_assert(kMaxSplits <= kWave, "one split per lane");
    static_assert(NC * NG == kAttnThreads, "float4 columns tile the block");
    __shared__ float wgt[G * kMaxSplits];
    __shared__ float4 acc4[kAttnThreads];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* parts = a.part + ((size_t)b * a.hkv + kvh) * nsplit * REC;
    const int c = tid % NC, sg = tid / NC, h = 4 * c / HD;
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
        const float M = wave_max(m);
        const float e = (ok && M != -__builtin_inff()) ? __expf(m - M) : 0.0f;
        const float L = wave_sum(e * l);
        wgt[hh * kMaxSplits + lane] = L > 0.0f ? e / L : 0.0f;
    }
    f4v acc = {0.f, 0.f, 0.f, 0.f};
    __syncthreads();
    for (int s0 = sg;;) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int sx = s0 + u * NG;
            const float w = wgt[h * kMaxSplits + min(sx, kMaxSplits - 1)] * (sx < nsplit ? 1.0f : 0.0f);
            acc += w * v[u];
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
    acc4[tid] = make_float4(acc.x, acc.y, acc.z, acc.w);
    __syncthreads();
    if (tid < NC) {
        float4 r = acc4[tid];
        for (int gi = 1; gi < NG; ++gi) {
            const float4 q = acc4[gi * NC + tid];
            r.x += q.x;
            r.y += q.y;
            r.z += q.z;
            r.w += q.w;
        }
        uint16_t* out = a.out16 + ((size_t)b * a.hq + (size_t)kvh * G) * HD + 4 * tid;
        *reinterpret_cast<uint2*>(out) = make_uint2((uint32_t)f2h_bits(r.x) | ((uint32_t)f2h_bits(r.y) << 16),
                                                    (uint32_t)f2h_bits(r.z) | ((uint32_t)f2h_bits(r.w) << 16));
    }
}

// One split of one (kv head, sequence): 8 pages (more for very long
// contexts) shared by the block's four wavefronts, two pages per wavefront
// step.  PIPE: more than one page pair per wavefront, two pairs in flight.
// The block stores its record, counts itself in a.counts for its (sequence,
// kv head), and the last of the nsplit blocks merges the records
// (merge_last) and resets the counter to zero for the next launch.
template <int G, int HD, bool PIPE>
__device__ inline void attn_f16_run(const AttnArgs& a, int nsplit, int pps, int split, int kvh, int b) {
    constexpr int REC = rec_floats(G, HD), MO = G * HD, LO = G * HD + G;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, t = lane & 15;
    __shared__ __align__(16) float lds[kAttnWaves * REC];

    // The context length and this wavefront's block-table entries (page
    // p0 + wave + 4i in lane i) are requested together: one round trip.
    const int ctx = a.ctx_lens ? a.ctx_lens[b] : a.pos[b] + 1;
    const int p0 = split * pps;
    const int npw_max = (pps - wave + kAttnWaves - 1) / kAttnWaves;
    const int my_page = p0 + wave + kAttnWaves * lane;
    const int bt_lane = (lane < npw_max && my_page < a.max_blocks)
                            ? a.block_table[(size_t)b * a.max_blocks + my_page]
                            : 0;
    // q as the B operand (column = head t, k = 8g + j of each 32-dim step).
    // Columns t >= G repeat head G - 1 (loads without a branch, so all of q
    // is requested at once); their scores and output rows are never used.
    h8_t qh[HD / 32], ql[HD / 32];
    {
        const float* qsrc = a.q + ((size_t)b * a.hq + kvh * G + min(t, G - 1)) * HD + 8 * g;
        float4 x[HD / 32][2];
#pragma unroll
        for (int s = 0; s < HD / 32; ++s) {
            x[s][0] = *reinterpret_cast<const float4*>(qsrc + 32 * s);
            x[s][1] = *reinterpret_cast<const float4*>(qsrc + 32 * s + 4);
        }
#pragma unroll
        for (int s = 0; s < HD / 32; ++s) {
            const float v[8] = {x[s][0].x, x[s][0].y, x[s][0].z, x[s][0].w,
                                x[s][1].x, x[s][1].y, x[s][1].z, x[s][1].w};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                qh[s][j] = (_Float16)v[j];
                ql[s][j] = (_Float16)(v[j] - (float)qh[s][j]);
            }
        }
    }
    const float scale = 1.0f / sqrtf((float)HD);

    const int npages = (ctx + kPage - 1) / kPage;
    const int p1 = min(p0 + pps, npages);
    // pages of this wavefront: p0 + wave + 4i for i < npw, taken in pairs
    const int npw = p1 > p0 + wave ? (p1 - p0 - wave + kAttnWaves - 1) / kAttnWaves : 0;
    auto valid_of = [&](int i) { return i < npw ? min(ctx - (p0 + wave + kAttnWaves * i) * kPage, kPage) : 0; };
    auto blk_of = [&](int i) { return __builtin_amdgcn_readlane(bt_lane, min(i, kWave - 1)); };
    float m = -__builtin_inff(), lsum = 0.0f;
    f4_t o[HD / 16];
#pragma unroll
    for (int nt = 0; nt < HD / 16; ++nt) o[nt] = f4_t{0.f, 0.f, 0.f, 0.f};
    if constexpr (PIPE) {
        PairRaw<HD> ra, rb;
        if (npw > 0) load_pair<HD>(ra, a, blk_of(0), valid_of(0), blk_of(1), valid_of(1), kvh, lane);
        for (int i = 0; i < npw; i += 4) {
            if (i + 2 < npw)
                load_pair<HD>(rb, a, blk_of(i + 2), valid_of(i + 2), blk_of(i + 3), valid_of(i + 3), kvh, lane);
            pair_update<HD>(ra, qh, ql, scale, valid_of(i), valid_of(i + 1), m, lsum, o, lane);
            if (i + 2 >= npw) break;
            if (i + 4 < npw)
                load_pair<HD>(ra, a, blk_of(i + 4), valid_of(i + 4), blk_of(i + 5), valid_of(i + 5), kvh, lane);
            pair_update<HD>(rb, qh, ql, scale, valid_of(i + 2), valid_of(i + 3), m, lsum, o, lane);
        }
    } else {
        PairRaw<HD> ra;
        if (npw > 0) {
            load_pair<HD>(ra, a, blk_of(0), valid_of(0), blk_of(1), valid_of(1), kvh, lane);
            pair_update<HD>(ra, qh, ql, scale, valid_of(0), valid_of(1), m, lsum, o, lane);
        }
    }
    // the head's denominator: sum of the four lanes that share its column
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    // wavefront record into LDS: rows h = 4g + i < G of O, m / l of head t
    float* my = lds + wave * REC;
#pragma unroll
    for (int nt = 0; nt < HD / 16; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (4 * g + i < G) my[(4 * g + i) * HD + 16 * nt + t] = o[nt][i];
    if (g == 0 && t < G) {
        my[MO + t] = m;
        my[LO + t] = lsum;
    }
    float* parts = a.part + ((size_t)b * a.hkv + kvh) * nsplit * REC;
    merge_waves_store<G, HD, true>(parts + (size_t)split * REC, lds);
    // every thread's record stores are complete before the block counts itself
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __shared__ int last;
    if (threadIdx.x == 0) {
        unsigned* cnt = a.counts + ((size_t)b * a.hkv + kvh) * kAttnCountStride;
        const unsigned prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = prev == (unsigned)nsplit - 1u;
        if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (last) merge_last<G, HD>(a, nsplit, kvh, b);
}

// PIPE: more than one page pair per wavefront (pps > 8), two pairs in
// flight; otherwise the single pair is loaded up front and the kernel fits
// two blocks per CU.
template <int G, int HD, bool PIPE>
__global__ __launch_bounds__(kAttnThreads, 1) void k_attn_f16(AttnArgs a, int nsplit, int pps) {
    attn_f16_run<G, HD, PIPE>(a, nsplit, pps, blockIdx.x, blockIdx.y, blockIdx.z);
}

// ------------------------------------------------------ TurboQuant pages --
__constant__ float c_tq_c4[16];
__constant__ float c_tq_b4[15];
__constant__ float c_tq_c3[8];
__constant__ float c_tq_b3[7];
__constant__ float c_tq_cb[24];  // c_tq_c4 then c_tq_c3

// In-LDS FWHT of G vectors of 128 (canonical butterfly network).
template <int G>
__device__ inline void lds_fwht(float* v) {
    for (int h = 1; h < 128; h <<= 1) {
        __syncthreads();
        for (int t = threadIdx.x; t < G * 64; t += kAttnThreads) {
            const int g = t >> 6, k = t & 63;
            const int j = ((k / h) * 2 * h) + (k % h);
            const float x = v[g * 128 + j], y = v[g * 128 + j + h];
            v[g * 128 + j] = x + y;
            v[g * 128 + j + h] = x - y;
        }
    }
    __syncthreads();
}

constexpr float kTqScale = 0.08838834764831845f;  // float(1/sqrt(128))

// One page for one lane (c = l%16, tg = l/16): the codes of dims [8c, 8c+8)
// of tokens 4tg .. 4tg+3, for K and V, and those tokens' norms.  Lanes c < 8
// hold 8 4-bit codes in one dword of the 32-byte record; lanes c >= 8 hold 8
// 3-bit codes, the 3 bytes at 3(c-8) of the 24-byte record, which span at
// most two dwords (w0, w1; joined with alignbyte once they have arrived).
struct TqRaw {
    uint32_t k0[4], k1[4], v0[4], v1[4];
    uint2 kn, vn;  // fp16 norms of the 4 tokens
};

// Lane constants of the code layout: where the lane's first dword of a
// token's K and V codes lies (record base plus byte offset), distance to the
// second dword, record stride, and the decode parameters (byte shift, code
// width, codebook offset).  Computed once, so that a page's addresses are one
// multiply-add per lane.
struct TqLane {
    const uint8_t *kb, *vb;
    int d1, stride, shift, bits, cbo;
    __device__ TqLane(const AttnArgs& a, int c) {
        const bool b4 = c < 8;
        const int j = c - 8;
        const int off = b4 ? 4 * c : 4 * ((3 * j) >> 2);
        kb = (b4 ? a.kc4 : a.kc3) + off;
        vb = (b4 ? a.vc4 : a.vc3) + off;
        d1 = b4 ? 0 : 4 * (((3 * j + 2) >> 2) - ((3 * j) >> 2));
        stride = b4 ? 32 : 24;
        shift = b4 ? 0 : (3 * j) & 3;
        bits = b4 ? 4 : 3;
        cbo = b4 ? 0 : 16;
    }
};

// Every load is issued unconditionally (see load_pair): blk must be a valid
// block; tokens past the context are masked when the page is processed.
__device__ inline void load_page_tq(TqRaw& r, const AttnArgs& a, const TqLane& ln, int blk, int kvh,
                                    int tg) {
    const size_t rec = ((size_t)blk * a.hkv + kvh) * kPage + 4 * tg;
    const size_t cofs = rec * (size_t)ln.stride;
    const uint8_t* kb = ln.kb + cofs;
    const uint8_t* vb = ln.vb + cofs;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        r.k0[j] = *reinterpret_cast<const uint32_t*>(kb + j * ln.stride);
        r.k1[j] = *reinterpret_cast<const uint32_t*>(kb + j * ln.stride + ln.d1);
        r.v0[j] = *reinterpret_cast<const uint32_t*>(vb + j * ln.stride);
        r.v1[j] = *reinterpret_cast<const uint32_t*>(vb + j * ln.stride + ln.d1);
    }
    r.kn = *reinterpret_cast<const uint2*>(a.kn + rec);
    r.vn = *reinterpret_cast<const uint2*>(a.vn + rec);
}

// Codebook values of the lane's 8 codes (cb: 16 4-bit levels, then 8 3-bit).
__device__ inline void tq_lookup8(uint32_t w0, uint32_t w1, const TqLane& ln, const float* cb,
                                  float (&out)[8]) {
    const uint32_t w = __builtin_amdgcn_alignbyte(w1, w0, ln.shift);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = cb[ln.cbo + __builtin_amdgcn_ubfe(w, ln.bits * i, ln.bits)];
}

// n = valid tokens of the page (0..16).
template <int G>
__device__ inline void process_page_tq(State<G, 8>& st, const TqRaw& r, const float (&q)[G][8],
                                       float scale, int n, int tg, const TqLane& ln, const float* cb) {
    float vf[4][8];
    float sc[4][G];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const bool valid = 4 * tg + j < n;
        const uint32_t nw = j < 2 ? r.kn.x : r.kn.y, vw = j < 2 ? r.vn.x : r.vn.y;
        const uint32_t sh = 16 * (j & 1);
        // the V norm of a token past the context is cleared (its bits may be
        // anything), so its zero probability meets a finite value
        const float vn = h2f_bits((uint16_t)((vw >> sh) & (valid ? 0xFFFFu : 0u)));
        const float kn = h2f_bits((uint16_t)(nw >> sh));
        float kf[8];
        tq_lookup8(r.k0[j], r.k1[j], ln, cb, kf);
        tq_lookup8(r.v0[j], r.v1[j], ln, cb, vf[j]);
#pragma unroll
        for (int d = 0; d < 8; ++d) vf[j][d] *= vn;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float dot = 0.0f;
#pragma unroll
            for (int d = 0; d < 8; ++d) dot = fmaf(q[h][d], kf[d], dot);
            dot = row16_sum(dot) * kn * scale;
            sc[j][h] = valid ? dot : -__builtin_inff();
        }
    }
    state_update(st, sc, vf);
}

template <int G>
__global__ __launch_bounds__(kAttnThreads) void k_attn_tq(AttnArgs a, int nsplit, int pps) {
    constexpr int HD = 128, DPL = 8, REC = rec_floats(G, HD);
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, tg = lane >> 4;
    __shared__ __align__(16) float lds[kAttnWaves * REC];
    __shared__ float qrot[G * HD];
    __shared__ float cb[24];

    // context length and block-table entries first (see attn_f16_run)
    const int ctx = a.ctx_lens ? a.ctx_lens[b] : a.pos[b] + 1;
    const int p0 = split * pps;
    const int npw_max = (pps - wave + kAttnWaves - 1) / kAttnWaves;
    const int my_page = p0 + wave + kAttnWaves * lane;
    const int bt_lane = (lane < npw_max && my_page < a.max_blocks)
                            ? a.block_table[(size_t)b * a.max_blocks + my_page]
                            : 0;
    const int npages = (ctx + kPage - 1) / kPage;
    const int p1 = min(p0 + pps, npages);
    const int npw = p1 > p0 + wave ? (p1 - p0 - wave + kAttnWaves - 1) / kAttnWaves : 0;
    // page i of this wavefront; pages past npw re-read the last one (or the
    // entry of lane 0, a valid block, when there is none) with no valid token
    auto blk_of = [&](int i) { return __builtin_amdgcn_readlane(bt_lane, min(i, max(npw - 1, 0))); };
    auto valid_of = [&](int i) { return i < npw ? min(ctx - (p0 + wave + kAttnWaves * i) * kPage, kPage) : 0; };
    const TqLane ln(a, c);
    // q, the K signs and the codebook, one clamped load per value and thread,
    // then the first two pages: every load is in flight before q is rotated
    constexpr int QPT = (G * HD + kAttnThreads - 1) / kAttnThreads;
    float qv[QPT], sv[QPT];
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
        const int idx = min((int)threadIdx.x + u * kAttnThreads, G * HD - 1);
        qv[u] = a.q[((size_t)b * a.hq + kvh * G) * HD + idx];
        sv[u] = a.ksign[idx % HD];
    }
    const float cbv = c_tq_cb[min((int)threadIdx.x, 23)];
    TqRaw a0, a1, b0, b1;
    load_page_tq(a0, a, ln, blk_of(0), kvh, tg);
    load_page_tq(a1, a, ln, blk_of(1), kvh, tg);

    if (threadIdx.x < 24) cb[threadIdx.x] = cbv;
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
        const int idx = threadIdx.x + u * kAttnThreads;
        if (idx < G * HD) qrot[idx] = sv[u] * qv[u];
    }
    lds_fwht<G>(qrot);

    const float scale = kTqScale / sqrtf((float)HD);  // rotation normalisation and 1/sqrt(hd)
    float q[G][DPL];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int d = 0; d < DPL; ++d) q[h][d] = qrot[h * HD + c * DPL + d];

    State<G, DPL> st;
    state_init(st);
    // two pairs of pages in flight; both pairs are requested on every pass
    // (past the last page they re-read it), and only the processing of a
    // pair with no page is skipped, a branch with no load in it
    for (int i = 0; i < npw; i += 4) {
        load_page_tq(b0, a, ln, blk_of(i + 2), kvh, tg);
        load_page_tq(b1, a, ln, blk_of(i + 3), kvh, tg);
        process_page_tq<G>(st, a0, q, scale, valid_of(i), tg, ln, cb);
        if (i + 1 < npw) process_page_tq<G>(st, a1, q, scale, valid_of(i + 1), tg, ln, cb);
        load_page_tq(a0, a, ln, blk_of(i + 4), kvh, tg);
        load_page_tq(a1, a, ln, blk_of(i + 5), kvh, tg);
        if (i + 2 < npw) process_page_tq<G>(st, b0, q, scale, valid_of(i + 2), tg, ln, cb);
        if (i + 3 < npw) process_page_tq<G>(st, b1, q, scale, valid_of(i + 3), tg, ln, cb);
    }
    state_merge_rows(st);

    float* parts = a.part + ((size_t)b * a.hkv + kvh) * nsplit * REC;
    block_merge_store<G, HD>(st, parts + (size_t)split * REC, lds);
}

// Merge the split records of one query head: block (h, kv head, sequence),
// one thread per dimension.  Every thread requests its nsplit partial sums at
// once, and lane s of every wavefront the maximum and denominator of split s
// (nsplit <= 64), so the split weights exp(m_s - M) and the denominator come
// from wavefront reductions with no LDS round trip; the weighted sum reads
// each weight from its lane.  TQ: the merged value sum is still in the
// rotated domain and is rotated back once, o = D_v H o~ / sqrt(128).
template <int G, int HD, bool TQ>
__global__ __launch_bounds__(HD) void k_attn_merge(AttnArgs a, int nsplit) {
    constexpr int REC = rec_floats(G, HD), MO = G * HD, LO = G * HD + G;
    static_assert(kMaxSplits <= kWave, "one split per lane");
    const int h = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z, t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const float* parts = a.part + ((size_t)b * a.hkv + kvh) * nsplit * REC;
    float o[kMaxSplits];
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s) o[s] = s < nsplit ? parts[(size_t)s * REC + h * HD + t] : 0.0f;
    const float ms = lane < nsplit ? parts[(size_t)lane * REC + MO + h] : -__builtin_inff();
    const float ls = lane < nsplit ? parts[(size_t)lane * REC + LO + h] : 0.0f;
    const float M = wave_max(ms);
    const float f = (lane >= nsplit || M == -__builtin_inff()) ? 0.0f : __expf(ms - M);
    const float L = wave_sum(f * ls);
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s)
        if (s < nsplit) acc = fmaf(o[s], readlane_f(f, s), acc);
    if (TQ) {
        __shared__ float ov[HD];
        ov[t] = acc;
        for (int hh = 1; hh < HD; hh <<= 1) {
            __syncthreads();
            if (t < HD / 2) {
                const int j = ((t / hh) * 2 * hh) + (t % hh);
                const float x = ov[j], y = ov[j + hh];
                ov[j] = x + y;
                ov[j + hh] = x - y;
            }
        }
        __syncthreads();
        acc = ov[t] * kTqScale * a.vsign[t];
    }
    const float out = L > 0.0f ? acc / L : 0.0f;
    a.out16[((size_t)b * a.hq + kvh * G + h) * HD + t] = f2h_bits(out);
}

// ----------------------------------------------------- TurboQuant encode --
// One wavefront per vector; lane l holds coordinates l and l + 64.
__device__ inline void tq_encode_wave(const float* __restrict__ x, const float* __restrict__ sign,
                                      uint8_t* __restrict__ c4, uint8_t* __restrict__ c3,
                                      uint16_t* __restrict__ norm, uint8_t* lds_codes) {
    const int lane = threadIdx.x & 63;
    const float x0 = x[lane], x1 = x[lane + 64];
    const float a0 = x0 * x0;
    const float a1 = x1 * x1;
    float w = a0 + a1;
    for (int s = 32; s >= 1; s >>= 1) {
        const float o = __shfl_down(w, s, 64);
        w = w + o;
    }
    const float ss = readlane_f(w, 0);
    const float n = __fsqrt_rn(ss);
    float u0 = 0.0f, u1 = 0.0f;
    if (n > 1e-12f) {
        const float inv = __fdiv_rn(1.0f, n);
        u0 = (sign[lane] * x0) * inv;
        u1 = (sign[lane + 64] * x1) * inv;
    }
    // FWHT: stages h = 1 .. 32 across lanes, h = 64 inside the lane.
    for (int h = 1; h < 64; h <<= 1) {
        const float p0 = __shfl_xor(u0, h, 64);
        const float p1 = __shfl_xor(u1, h, 64);
        if (lane & h) {
            u0 = p0 - u0;
            u1 = p1 - u1;
        } else {
            u0 = u0 + p0;
            u1 = u1 + p1;
        }
    }
    {
        const float t0 = u0 + u1, t1 = u0 - u1;
        u0 = t0;
        u1 = t1;
    }
    const float y0 = u0 * kTqScale, y1 = u1 * kTqScale;
    int q0 = 0, q1 = 0;
#pragma unroll
    for (int j = 0; j < 15; ++j) q0 += (y0 < c_tq_b4[j]) ? 0 : 1;
#pragma unroll
    for (int j = 0; j < 7; ++j) q1 += (y1 < c_tq_b3[j]) ? 0 : 1;
    lds_codes[lane] = (uint8_t)q0;
    lds_codes[lane + 64] = (uint8_t)q1;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < 32) c4[lane] = (uint8_t)(lds_codes[2 * lane] | (lds_codes[2 * lane + 1] << 4));
    if (lane < 24) {
        const int g = lane / 3, r = lane % 3;
        uint32_t bits = 0;
#pragma unroll
        for (int m = 0; m < 8; ++m) bits |= (uint32_t)lds_codes[64 + 8 * g + m] << (3 * m);
        c3[lane] = (uint8_t)(bits >> (8 * r));
    }
    if (lane == 0) *norm = f2h_bits(n);
}

__global__ __launch_bounds__(256) void k_tq_encode(const float* x, int nvec, const float* signs,
                                                   uint8_t* c4, uint8_t* c3, uint16_t* norms,
                                                   const int32_t* idx) {
    __shared__ uint8_t codes[4][128];
    const int wave = threadIdx.x >> 6;
    const int v = blockIdx.x * 4 + wave;
    if (v >= nvec) return;
    const int dst = idx ? idx[v] : v;
    tq_encode_wave(x + (size_t)v * 128, signs, c4 + (size_t)dst * 32, c3 + (size_t)dst * 24,
                   norms + dst, codes[wave]);
}

// Context rows [ctx][hkv][128] of sequence b -> pages.
__global__ __launch_bounds__(256) void k_tq_encode_ctx(const float* x, int ctx, int hkv,
                                                       const float* signs, uint8_t* c4,
                                                       uint8_t* c3, uint16_t* norms,
                                                       const int32_t* block_table, int max_blocks,
                                                       int b) {
    __shared__ uint8_t codes[4][128];
    const int wave = threadIdx.x >> 6;
    const int v = blockIdx.x * 4 + wave;
    if (v >= ctx * hkv) return;
    const int t = v / hkv, h = v % hkv;
    const int blk = block_table[(size_t)b * max_blocks + t / kPage];
    const size_t dst = ((size_t)blk * hkv + h) * kPage + t % kPage;
    tq_encode_wave(x + (size_t)v * 128, signs, c4 + dst * 32, c3 + dst * 24, norms + dst,
                   codes[wave]);
}

// One token per sequence from kv_tmp [batch][2][hkv*128].
__global__ __launch_bounds__(256) void k_tq_append(const float* kv_tmp, int batch, int hkv,
                                                   const float* ksign, const float* vsign,
                                                   uint8_t* kc4, uint8_t* kc3, uint16_t* kn,
                                                   uint8_t* vc4, uint8_t* vc3, uint16_t* vn,
                                                   const int32_t* block_table, const int32_t* pos,
                                                   int max_blocks) {
    __shared__ uint8_t codes[4][128];
    const int wave = threadIdx.x >> 6;
    const int v = blockIdx.x * 4 + wave;  // (b, kv, h)
    if (v >= batch * 2 * hkv) return;
    const int b = v / (2 * hkv), kv = (v / hkv) % 2, h = v % hkv;
    const int p = pos[b];
    const int blk = block_table[(size_t)b * max_blocks + p / kPage];
    const size_t dst = ((size_t)blk * hkv + h) * kPage + p % kPage;
    const float* src = kv_tmp + ((size_t)b * 2 + kv) * hkv * 128 + (size_t)h * 128;
    if (kv == 0)
        tq_encode_wave(src, ksign, kc4 + dst * 32, kc3 + dst * 24, kn + dst, codes[wave]);
    else
        tq_encode_wave(src, vsign, vc4 + dst * 32, vc3 + dst * 24, vn + dst, codes[wave]);
}

}  // namespace

size_t attn_workspace_bytes(int batch, int hq, int hkv, int hd, int max_ctx) {
    const SplitPlan sp = plan_splits(max_ctx);
    const int G = hq / hkv;
    return sizeof(float) * (size_t)batch * hkv * sp.nsplit * rec_floats(G, hd);
}

int attn_max_ctx() { return kMaxSplits * kPagesPerSplitMax * kPage; }

hipError_t attn_f16_launch(const AttnArgs& a, hipStream_t st) {
    if (!a.counts || !a.part) return hipErrorInvalidValue;
    const SplitPlan sp = plan_splits(a.max_ctx);
    const dim3 grid(sp.nsplit, a.hkv, a.batch);
    const int G = a.hq / a.hkv;
    const bool pipe = sp.pps > kPagesPerSplitMin;
#define NX_ATTN_CASE(GG, HH)                                                                      \
    if (G == GG && a.hd == HH) {                                                                  \
        if (pipe)                                                                                 \
            hipLaunchKernelGGL((k_attn_f16<GG, HH, true>), grid, dim3(kAttnThreads), 0, st, a,     \
                               sp.nsplit, sp.pps);                                                \
        else                                                                                      \
            hipLaunchKernelGGL((k_attn_f16<GG, HH, false>), grid, dim3(kAttnThreads), 0, st, a,    \
                               sp.nsplit, sp.pps);                                                \
        return hipGetLastError();                                                                 \
    }
    NX_ATTN_CASE(1, 64)
    NX_ATTN_CASE(2, 64)
    NX_ATTN_CASE(4, 64)
    NX_ATTN_CASE(8, 64)
    NX_ATTN_CASE(1, 128)
    NX_ATTN_CASE(2, 128)
    NX_ATTN_CASE(4, 128)
    NX_ATTN_CASE(8, 128)
#undef NX_ATTN_CASE
    return hipErrorInvalidValue;
}

hipError_t attn_tq_launch(const AttnArgs& a, hipStream_t st) {
    const SplitPlan sp = plan_splits(a.max_ctx);
    const dim3 grid(sp.nsplit, a.hkv, a.batch), mgrid(a.hq / a.hkv, a.hkv, a.batch);
    const int G = a.hq / a.hkv;
    if (a.hd != 128) return hipErrorInvalidValue;
#define NX_ATTN_CASE(GG)                                                                          \
    if (G == GG) {                                                                                \
        hipLaunchKernelGGL((k_attn_tq<GG>), grid, dim3(kAttnThreads), 0, st, a, sp.nsplit,        \
                           sp.pps);                                                               \
        hipLaunchKernelGGL((k_attn_merge<GG, 128, true>), mgrid, dim3(128), 0, st, a,             \
                           sp.nsplit);                                                            \
        return hipGetLastError();                                                                 \
    }
    NX_ATTN_CASE(1)
    NX_ATTN_CASE(2)
    NX_ATTN_CASE(4)
    NX_ATTN_CASE(8)
#undef NX_ATTN_CASE
    return hipErrorInvalidValue;
}

void tq_set_codebooks(const float* c4, const float* b4, const float* c3, const float* b3) {
    (void)hipMemcpyToSymbol(HIP_SYMBOL(c_tq_c4), c4, sizeof(float) * 16);
    (void)hipMemcpyToSymbol(HIP_SYMBOL(c_tq_b4), b4, sizeof(float) * 15);
    (void)hipMemcpyToSymbol(HIP_SYMBOL(c_tq_c3), c3, sizeof(float) * 8);
    (void)hipMemcpyToSymbol(HIP_SYMBOL(c_tq_b3), b3, sizeof(float) * 7);
    (void)hipMemcpyToSymbol(HIP_SYMBOL(c_tq_cb), c4, sizeof(float) * 16);
    (void)hipMemcpyToSymbol(HIP_SYMBOL(c_tq_cb), c3, sizeof(float) * 8, sizeof(float) * 16);
}

hipError_t tq_encode_launch(const float* x, int nvec, const float* signs, const float* b4,
                            const float* b3, uint8_t* c4, uint8_t* c3, uint16_t* norms,
                            const int32_t* idx, hipStream_t st) {
    (void)b4;
    (void)b3;
    if (nvec <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_tq_encode, dim3((nvec + 3) / 4), dim3(256), 0, st, x, nvec, signs, c4, c3,
                       norms, idx);
    return hipGetLastError();
}

hipError_t tq_encode_ctx_launch(const float* x, int ctx, int hkv, const float* signs,
                                const float* b4, const float* b3, uint8_t* c4, uint8_t* c3,
                                uint16_t* norms, const int32_t* block_table, int max_blocks, int b,
                                hipStream_t st) {
    (void)b4;
    (void)b3;
    const int nvec = ctx * hkv;
    if (nvec <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_tq_encode_ctx, dim3((nvec + 3) / 4), dim3(256), 0, st, x, ctx, hkv, signs,
                       c4, c3, norms, block_table, max_blocks, b);
    return hipGetLastError();
}

hipError_t tq_append_launch(const float* kv_tmp, int batch, int hkv, const float* ksign,
                            const float* vsign, const float* b4, const float* b3, uint8_t* kc4,
                            uint8_t* kc3, uint16_t* kn, uint8_t* vc4, uint8_t* vc3, uint16_t* vn,
                            const int32_t* block_table, const int32_t* pos, int max_blocks,
                            hipStream_t st) {
    (void)b4;
    (void)b3;
    const int nvec = batch * 2 * hkv;
    hipLaunchKernelGGL(k_tq_append, dim3((nvec + 3) / 4), dim3(256), 0, st, kv_tmp, batch, hkv,
                       ksign, vsign, kc4, kc3, kn, vc4, vc3, vn, block_table, pos, max_blocks);
    return hipGetLastError();
}

}  // namespace nx
