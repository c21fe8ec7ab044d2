// Paged decode attention on gfx950 over fp16 pages and TurboQuant pages.
//
// Grid (split, kv head, sequence); 8 wavefronts per block.  A block owns a
// contiguous range of 16-token pages of one kv head and serves the G = hq/hkv
// query heads that share it, so every K/V byte is read once per step.  Each
// wavefront requests its block-table entries with q and then processes its
// pages in pairs on the matrix cores (two pairs in flight when it has more
// than one), keeping an online-softmax state per query head.  Wavefronts are
// merged through LDS and the block stores one split record; the last block of
// a (sequence, kv head) to count itself done merges the split records and
// writes the fp16 output.  Records and counters use agent-scope (cross-XCD
// coherent) relaxed accesses, with each block's stores complete before it
// counts, and no device-scope fence.
//
// TurboQuant pages are scored in the rotated domain: the block rotates q once
// (q~ = H D q), scores are n_t * <q~, c[code_t]> / sqrt(128 * 128), V is summed
// in the rotated domain and rotated back (D H o~ / sqrt(128)) by the merging
// block.
#include "nx_attn_dev.h"

namespace nx {

namespace {

using namespace at;



struct SplitPlan {
    int nsplit, pps;  // splits per (sequence, kv head), pages per split
};

// A split is kPagesPerSplitMin = 16 pages (two per wavefront of the
// 8-wavefront block, all in flight at once) until kMaxSplits splits per
// (sequence, kv head) are reached; longer contexts get more pages per split.
// A wavefront keeps its block-table entries one per lane, which bounds a
// split at kAttnWaves * 64 pages: contexts up to kMaxSplits * 512 pages
// (attn_max_ctx() tokens).
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

// ------------------------------------------------- TurboQuant constants --
__constant__ float c_tq_c4[16];
__constant__ float c_tq_b4[15];
__constant__ float c_tq_c3[8];
__constant__ float c_tq_b3[7];
__constant__ float c_tq_cb[24];  // c_tq_c4 then c_tq_c3
constexpr int kTqTbl4 = 256, kTqTbl = kTqTbl4 + 64;  // LDS pair tables of the attention

// One split of one (kv head, sequence): the pages s, s + nsplit, ... of
// split s, shared by the block's kAttnWaves wavefronts, two pages per
// wavefront step.  PIPE: more than one page pair per wavefront (the launcher
// decides from the longest context), two pairs in flight.
// The block stores its record, counts itself in a.counts for its (sequence,
// kv head), and the last of the nsplit blocks merges the records
// (merge_last) and resets the counter to zero for the next launch.
// range, slot, nrec, ntq: the part of the context (attn_range), this
// block's record among the nrec records of its (sequence, kv head), and the
// rotated records among them (tiered pages: the TurboQuant blocks' [0, ntq),
// merged by merge_last<G, 128, true> when TIER).
template <int G, int HD, bool PIPE, bool TIER = false>
__device__ inline void attn_f16_run(const AttnArgs& a, int nsplit, int split, int kvh, int b,
                                    int range = 0, int slot = -1, int nrec = 0, int ntq = 0) {
    constexpr int REC = rec_floats(G, HD), MO = G * HD, LO = G * HD + G;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, t = lane & 15;
    __shared__ __align__(16) float lds[kAttnWaves * REC];
    attn_args_early(a);
    asm volatile("" ::"s"(a.kpool), "s"(a.vpool), "s"(nsplit));

    // The context length and this wavefront's block-table entries (page
    // p0 + wave + kAttnWaves * i in lane i) are requested together: one round trip.
    if (slot < 0) {
        slot = split;
        nrec = nsplit;
    }
    int ctx, pg0;
    attn_range(a, b, range, ctx, pg0);
    bool bad = false;
    if (a.check_blocks > 0 && (ctx < 0 || ctx > a.max_blocks * kPage)) {
        bad = true;
        ctx = min(max(ctx, 0), a.max_blocks * kPage);
    }
    // Pages are dealt to the splits round-robin and to a split's wavefronts
    // in turn: wavefront w of split s takes pages s + nsplit (w + 8 i), so
    // the pages a block reads do not depend on the context length (every
    // block-table entry is requested before the length arrives) and a
    // context of any length spreads over all the splits.  Lane i holds the
    // entry of page i.
    const int stride = nsplit * kAttnWaves;
    const int first = split + nsplit * wave;
    const int my_page = first + stride * lane;
    int bt_lane = (pg0 + my_page < a.max_blocks)
                      ? (range == 2 ? a.hot_table : a.block_table)[(size_t)b * a.max_blocks + pg0 + my_page]
                      : 0;
    if (a.check_blocks > 0) {
        // entries of pages inside the context must name a block of the pool
        const bool used = my_page * kPage < ctx;
        const bool inval = used && (bt_lane < 0 || bt_lane >= a.check_blocks);
        bad = bad || __any(inval);
        bt_lane = inval ? 0 : bt_lane;
    }
    // q as the B operand (column = head t, k = 8g + j of each 32-dim step).
    // Columns t >= G repeat head G - 1 (loads without a branch, so all of q
    // is requested at once); their scores and output rows are never used.
    const float* qsrc = a.q + ((size_t)b * a.hq + kvh * G + min(t, G - 1)) * HD + 8 * g;
    float4 qx[HD / 32][2];
#pragma unroll
    for (int s = 0; s < HD / 32; ++s) {
        qx[s][0] = *reinterpret_cast<const float4*>(qsrc + 32 * s);
        qx[s][1] = *reinterpret_cast<const float4*>(qsrc + 32 * s + 4);
    }
    const int npages = (ctx + kPage - 1) / kPage;
    // pages of this wavefront: first + stride * i for i < npw, taken in pairs
    const int npw = first < npages ? (npages - first + stride - 1) / stride : 0;
    auto valid_of = [&](int i) { return i < npw ? min(ctx - (first + stride * i) * kPage, kPage) : 0; };
    auto blk_of = [&](int i) { return __builtin_amdgcn_readlane(bt_lane, min(i, kWave - 1)); };
    // a pair past the wavefront's pages re-reads its first page and is not processed
    auto blk_or0 = [&](int i) { return i < npw ? blk_of(i) : blk_of(0); };
    // the first page pair is requested before q is converted (its addresses
    // need only the block table), so the pages do not wait for q's round trip
    constexpr bool kEarly = !(PIPE && HD > 128);
    PairRaw<HD> ra;
    if constexpr (kEarly) load_pair<HD>(ra, a, blk_or0(0), valid_of(0), blk_or0(1), valid_of(1), kvh, lane);
    h8_t qh[HD / 32], ql[HD / 32];
#pragma unroll
    for (int s = 0; s < HD / 32; ++s) {
        const float v[8] = {qx[s][0].x, qx[s][0].y, qx[s][0].z, qx[s][0].w,
                            qx[s][1].x, qx[s][1].y, qx[s][1].z, qx[s][1].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            qh[s][j] = (_Float16)v[j];
            ql[s][j] = (_Float16)(v[j] - (float)qh[s][j]);
        }
    }
    const float scale = 1.0f / sqrtf((float)HD);
    // 256-long heads: q's operands go to LDS (every wavefront writes the same
    // values, then reads its own), read per k-step by pair_update
    constexpr bool QL = HD > 128;
    __shared__ __align__(16) uint4 qlds[QL ? G * 4 * (HD / 32) * 2 : 1];
    const uint4* qls = nullptr;
    if constexpr (QL) {
        if (t < G)
#pragma unroll
            for (int s = 0; s < HD / 32; ++s) {
                qlds[((t * 4 + g) * (HD / 32) + s) * 2] = __builtin_bit_cast(uint4, qh[s]);
                qlds[((t * 4 + g) * (HD / 32) + s) * 2 + 1] = __builtin_bit_cast(uint4, ql[s]);
            }
        qls = qlds + (min(t, G - 1) * 4 + g) * (HD / 32) * 2;
    }
    float m = -__builtin_inff(), lsum = 0.0f;
    f4_t o[HD / 16];
#pragma unroll
    for (int nt = 0; nt < HD / 16; ++nt) o[nt] = f4_t{0.f, 0.f, 0.f, 0.f};
    if constexpr (PIPE && HD > 128) {
        // 256-long heads: one pair in flight (a second pair's K and V would
        // not fit the registers of two wavefronts per SIMD)
        for (int i = 0; i < npw; i += 2) {
            load_pair<HD>(ra, a, blk_of(i), valid_of(i), blk_of(i + 1), valid_of(i + 1), kvh, lane);
            pair_update<HD, false, false, QL>(ra, qh, ql, scale, valid_of(i), valid_of(i + 1), m, lsum, o, lane, 0,
                                              0, 0, nullptr, qls);
        }
    } else if constexpr (PIPE) {
        // the next pair is requested before the current one is used, so the
        // wait for the current pair leaves the next one in flight; nothing is
        // requested past the wavefront's last pair (a re-read of its first
        // page there was a round trip before the record: batch-8 attention
        // 31.5 -> 30.5 us)
        PairRaw<HD> rb;
        for (int i = 0; i < npw; i += 4) {
            if (i + 2 < npw)
                load_pair<HD>(rb, a, blk_or0(i + 2), valid_of(i + 2), blk_or0(i + 3), valid_of(i + 3), kvh, lane);
            pair_update<HD>(ra, qh, ql, scale, valid_of(i), valid_of(i + 1), m, lsum, o, lane);
            if (i + 2 >= npw) break;
            if (i + 4 < npw)
                load_pair<HD>(ra, a, blk_or0(i + 4), valid_of(i + 4), blk_or0(i + 5), valid_of(i + 5), kvh, lane);
            pair_update<HD>(rb, qh, ql, scale, valid_of(i + 2), valid_of(i + 3), m, lsum, o, lane);
        }
    } else {
        if (npw > 0)
            pair_update<HD, false, false, QL>(ra, qh, ql, scale, valid_of(0), valid_of(1), m, lsum, o, lane, 0, 0, 0,
                                              nullptr, qls);
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
        my[LO + t] = bad ? __builtin_nanf("") : lsum;
    }
    float* parts = a.part + ((size_t)b * a.hkv + kvh) * nrec * REC;
    merge_waves_store<G, HD, true>(parts + (size_t)slot * REC, lds);
    // every thread's record stores are complete before the block counts itself
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __shared__ int last;
    if (threadIdx.x == 0) {
        unsigned* cnt = a.counts + ((size_t)b * a.hkv + kvh) * kAttnCountStride;
        const unsigned prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = prev == (unsigned)nrec - 1u;
        if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (last) merge_last<G, HD, TIER>(a, nrec, ntq, kvh, b);
}

// PIPE: more than one page pair per wavefront, two pairs in flight;
// otherwise the single pair is loaded up front.
template <int G, int HD, bool PIPE>
__global__ __launch_bounds__(kAttnThreads, 1) void k_attn_f16(AttnArgs a, int nsplit) {
    attn_f16_run<G, HD, PIPE>(a, nsplit, blockIdx.x, blockIdx.y, blockIdx.z);
}

// ------------------------------------------------------ TurboQuant pages --

// TurboQuant pages on the matrix cores, in the layouts of the fp16 kernel
// above.  Records are token-major (a 32-byte 4-bit part: dimensions 0..63 as
// eight chunks of 8 codes, a 24-byte 3-bit part: dimensions 64..127 as eight
// chunks of 3 bytes).  The assignment of dimensions to the k slots of the
// score product and to the output columns of P.V is free, and is chosen so
// that every operand a lane needs is one or two dwords of a record:
//   scores S = K q~^T (A = K: row = token t = l%16, k slice g = l/16):
//     k-step s < 2 takes 4-bit chunk 2g + s (dimensions 16g + 8s .. +7),
//     s >= 2 the 3-bit chunk 2g + s - 2 (dimensions 64 + 16g + 8(s-2) .. +7);
//     q~ (B, column = head) is staged in the same order;
//   P.V (B = V: column n = l%16, k = the pair's tokens 8g + j, j < 4 from page
//     a, j >= 4 from page b): tile nt holds code nt of chunk n of each token,
//     so output column n of tile nt is dimension 8n + nt.
// Codebook values enter the scores as fp16 hi + lo, q~ as hi + lo: three
// products per step give fp32-accurate scores (their errors would pass through
// exp).  P enters as hi + lo and the codebook values of V as fp16 (rounded to
// nearest: at most 2^-12 relative per value, an error that stays linear in the
// output): two products per tile.  Codes are looked up in LDS pair tables:
// entry f of the 4-bit table (256 entries) holds the fp16 hi pair and lo pair
// of (c4[f & 15], c4[f >> 4]), of the 3-bit table (64 entries, from entry
// 256) those of (c3[f & 7], c3[f >> 3]), so one 8-byte lookup gives two
// score operand values (fewer instructions than a lookup per code, which
// needs two perms per pair, for more bank conflicts); for the value operand
// the low 32 bits of the entry of two adjacent codes of a token, the hi
// values of both, feed two tiles.  The V norm is folded into P, the K norm
// and the scale into the scores.
// Cool pages (COOL) hold 48-byte records, 3-bit codes on every dimension:
// chunk n (dimensions 8n .. 8n+7) at byte 3n, so dimensions 0..63 form a
// 24-byte half laid out as the 3-bit part above, 64..127 a second one.  The
// same operand layouts apply, every chunk decoded through the 3-bit table.
struct TqPair {
    uint2 k4[2], k3[2];           // pages a, b: 4-bit chunks (2g, 2g+1) of token l%16 (Cool: the 8 bytes holding its chunks 2g, 2g+1); the 8 bytes holding its 3-bit chunks (2g, 2g+1) (Cool: chunks 8+2g, 9+2g)
    uint32_t v0[2][4], v1[2][4];  // pages a, b, tokens 4g + j: the dwords holding chunk l%16
    uint2 kn[2], vn[2];           // pages a, b: fp16 norms of tokens 4g .. 4g+3
};

// Lane constants of the V operand (chunk n = l%16): where the chunk's first
// dword lies in a token's record, the distance to the second, the record
// stride, and the decode parameters (byte shift, code width, codebook
// offset).  Chunks n < 8 are one dword of the 4-bit part; chunks n >= 8 are 3
// bytes of the 3-bit part, at most two dwords.
struct TqLane {
    const uint8_t* vb;
    int d1, stride, shift, bits, cbo;
    __device__ TqLane(const AttnArgs& a, int n, bool cool = false) {
        if (cool) {  // chunk n: 3 bytes at byte 3n of a 48-byte record
            vb = a.vcc + 4 * ((3 * n) >> 2);
            d1 = 4 * (((3 * n + 2) >> 2) - ((3 * n) >> 2));
            stride = 48;
            shift = (3 * n) & 3;
            bits = 3;
            cbo = kTqTbl4;
            return;
        }
        const bool b4 = n < 8;
        const int j = n - 8;
        vb = (b4 ? a.vc4 : a.vc3) + (b4 ? 4 * n : 4 * ((3 * j) >> 2));
        d1 = b4 ? 0 : 4 * (((3 * j + 2) >> 2) - ((3 * j) >> 2));
        stride = b4 ? 32 : 24;
        shift = b4 ? 0 : (3 * j) & 3;
        bits = b4 ? 4 : 3;
        cbo = b4 ? 0 : kTqTbl4;
    }
};

// A page's loads have no per-lane condition (see load_pair): page b with no
// valid token re-reads page a (blka is a valid block); tokens past the valid
// counts are masked when the pair is processed.
template <bool COOL = false>
__device__ inline void tq_load_pair(TqPair& r, const AttnArgs& a, const TqLane& ln, int blka, int blkb,
                                    int nb, int kvh, int lane) {
    const int t = lane & 15, g = lane >> 4;
    const int o3 = 4 * ((3 * g) >> 1);  // dword holding byte 6g of a 3-bit part
#pragma unroll
    for (int pg = 0; pg < 2; ++pg) {
        const int blk = pg && nb > 0 ? blkb : blka;
        const size_t rec = ((size_t)blk * a.hkv + kvh) * kPage;
        if constexpr (COOL) {
            r.k4[pg] = *reinterpret_cast<const uint2*>(a.kcc + (rec + t) * 48 + o3);
            r.k3[pg] = *reinterpret_cast<const uint2*>(a.kcc + (rec + t) * 48 + 24 + o3);
        } else {
            r.k4[pg] = *reinterpret_cast<const uint2*>(a.kc4 + (rec + t) * 32 + 8 * g);
            r.k3[pg] = *reinterpret_cast<const uint2*>(a.kc3 + (rec + t) * 24 + o3);
        }
        const uint8_t* vb = ln.vb + (rec + 4 * g) * (size_t)ln.stride;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            r.v0[pg][j] = *reinterpret_cast<const uint32_t*>(vb + j * ln.stride);
            r.v1[pg][j] = *reinterpret_cast<const uint32_t*>(vb + j * ln.stride + ln.d1);
        }
        r.kn[pg] = *reinterpret_cast<const uint2*>((COOL ? a.kcn : a.kn) + rec + 4 * g);
        r.vn[pg] = *reinterpret_cast<const uint2*>((COOL ? a.vcn : a.vn) + rec + 4 * g);
    }
    __builtin_amdgcn_sched_barrier(0);
}

// fp16 hi and lo operands of 8 codes (width `bits`, from bit 0 of w): four
// pair-table lookups, codes 2i and 2i + 1 in dword i.
__device__ inline void tq_dequant8(uint32_t w, int bits, const uint2* tbl, h8_t& hi, h8_t& lo) {
    const int pb = 2 * bits;
    const uint2* t = tbl + (bits == 4 ? 0 : kTqTbl4);
    const uint2 e0 = t[__builtin_amdgcn_ubfe(w, 0, pb)], e1 = t[__builtin_amdgcn_ubfe(w, pb, pb)];
    const uint2 e2 = t[__builtin_amdgcn_ubfe(w, 2 * pb, pb)], e3 = t[__builtin_amdgcn_ubfe(w, 3 * pb, pb)];
    hi = as_h8(make_uint4(e0.x, e1.x, e2.x, e3.x));
    lo = as_h8(make_uint4(e0.y, e1.y, e2.y, e3.y));
}

// Fold one page pair into the wavefront's state (as pair_update: m and lsum
// of head l%16, O in the C layout with rows = heads 4(l/16) + i, tile nt
// column n = dimension 8n + nt).  na / nb: valid tokens of the two pages.
template <bool COOL = false>
__device__ inline void tq_pair_update(const TqPair& r, const TqLane& ln, const h8_t (&qh)[4], const h8_t (&ql)[4],
                                      const uint2* cbk, float scale, int na, int nb, float& m, float& lsum,
                                      f4_t (&o)[8], int lane) {
    const int g = lane >> 4;
    const int sh3 = 8 * ((6 * g) & 3);
    f4_t sc[2];
#pragma unroll
    for (int pg = 0; pg < 2; ++pg) {
        const uint64_t w3 = ((uint64_t)r.k3[pg].y << 32 | r.k3[pg].x) >> sh3;
        uint32_t chunk[4] = {r.k4[pg].x, r.k4[pg].y, (uint32_t)w3 & 0xFFFFFFu, (uint32_t)(w3 >> 24) & 0xFFFFFFu};
        if constexpr (COOL) {
            const uint64_t wa = ((uint64_t)r.k4[pg].y << 32 | r.k4[pg].x) >> sh3;
            chunk[0] = (uint32_t)wa & 0xFFFFFFu;
            chunk[1] = (uint32_t)(wa >> 24) & 0xFFFFFFu;
        }
        f4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            h8_t kh, kl;
            tq_dequant8(chunk[s], COOL || s >= 2 ? 3 : 4, cbk, kh, kl);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[s], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[s], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[s], acc, 0, 0, 0);
        }
        sc[pg] = acc;
    }
    // scores of tokens 4g + i: K norm and scale; tokens past the valid counts
    // get -inf, and their V norms are cleared (a zero probability then meets
    // a finite value)
    float p[8];
    uint32_t vnb[8];
    float mloc = -__builtin_inff();
#pragma unroll
    for (int pg = 0; pg < 2; ++pg) {
        const int n = pg ? nb : na;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t kw = i < 2 ? r.kn[pg].x : r.kn[pg].y, vw = i < 2 ? r.vn[pg].x : r.vn[pg].y;
            const bool valid = 4 * g + i < n;
            const float kn = h2f_bits((uint16_t)(kw >> (16 * (i & 1))));
            const float v = sc[pg][i] * kn * scale;
            p[4 * pg + i] = valid ? v : -__builtin_inff();
            vnb[4 * pg + i] = (vw >> (16 * (i & 1))) & (valid ? 0xFFFFu : 0u);
            mloc = fmaxf(mloc, p[4 * pg + i]);
        }
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
        const float ev = e * h2f_bits((uint16_t)vnb[j]);
        ph[j] = (_Float16)ev;
        pl[j] = (_Float16)(ev - (float)ph[j]);
    }
    lsum = lsum * corr + ps;
    m = mn;
    float c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = __shfl(corr, 4 * g + i, 64);
    // V chunk words of the 8 tokens (k = 8g + j)
    uint32_t vw[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
        vw[j] = __builtin_amdgcn_alignbyte(r.v1[j >> 2][j & 3], r.v0[j >> 2][j & 3], ln.shift);
    // tiles nt and nt + 1 from one pair-table lookup per token: codes nt and
    // nt + 1 of a chunk are adjacent, and the low 32 bits of their pair's entry
    // are (hi(c[code nt]), hi(c[code nt + 1]))
#pragma unroll
    for (int nt = 0; nt < 8; nt += 2) {
        uint32_t e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) e[j] = cbk[ln.cbo + __builtin_amdgcn_ubfe(vw[j], ln.bits * nt, 2 * ln.bits)].x;
        const uint4 h0 = make_uint4(__builtin_amdgcn_perm(e[1], e[0], 0x05040100u),
                                    __builtin_amdgcn_perm(e[3], e[2], 0x05040100u),
                                    __builtin_amdgcn_perm(e[5], e[4], 0x05040100u),
                                    __builtin_amdgcn_perm(e[7], e[6], 0x05040100u));
        const uint4 h1 = make_uint4(__builtin_amdgcn_perm(e[1], e[0], 0x07060302u),
                                    __builtin_amdgcn_perm(e[3], e[2], 0x07060302u),
                                    __builtin_amdgcn_perm(e[5], e[4], 0x07060302u),
                                    __builtin_amdgcn_perm(e[7], e[6], 0x07060302u));
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint4 h = u ? h1 : h0;
            f4_t acc = o[nt + u];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] *= c[i];
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, as_h8(h), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, as_h8(h), acc, 0, 0, 0);
            o[nt + u] = acc;
        }
    }
}

template <bool COOL>
__device__ inline float tq_codes_lane(float x0, float x1, const float* __restrict__ sign, int& q0, int& q1);
template <bool COOL>
__device__ inline void tq_store_codes(int q0, int q1, float n, uint8_t* __restrict__ ca, uint8_t* __restrict__ cb,
                                      uint16_t* __restrict__ norm, uint8_t* lds_codes);

// The token being written at this step (a.kv_cur: its fp32 K and V), in
// wavefront 0 of one extra block of the launch that reads no page: encode K
// and V into the TurboQuant pages at position pos[b] (what a separate
// append launch would store) and form the token's softmax record from its
// codes -- score n_k * scale * sum_i c[code_i] q~_i for each head, value
// n_v * c[code_i] in the rotated domain -- in the layouts of the page loop
// (m and l of head l%16, l on the lanes of group 0; O rows 4(l/16) + i,
// column t of tile nt = dimension 8t + nt).  The page splits stop before
// this position.
template <int G>
__device__ inline void tq_current_record(const AttnArgs& a, int b, int kvh, const float* qrot, float scale, float& m,
                                         float& lsum, f4_t (&o)[8]) {
    constexpr int HD = 128;
    __shared__ float scratch[64 + 128];  // packing rows of the K and V codes, then the value
    const int lane = threadIdx.x & 63, g = lane >> 4, t = lane & 15;
    const int p = a.pos[b];
    const float* kx = a.kv_cur + (size_t)b * 2 * a.hkv * HD + (size_t)kvh * HD;
    const float* vx = kx + (size_t)a.hkv * HD;
    const size_t dst = ((size_t)a.block_table[(size_t)b * a.max_blocks + p / kPage] * a.hkv + kvh) * kPage + p % kPage;
    // the TurboQuant pools, written here for the later steps
    uint8_t* codes = reinterpret_cast<uint8_t*>(scratch);
    int kq0, kq1, vq0, vq1;
    const float nk = tq_codes_lane<false>(kx[lane], kx[lane + 64], a.ksign, kq0, kq1);
    tq_store_codes<false>(kq0, kq1, nk, const_cast<uint8_t*>(a.kc4) + dst * 32, const_cast<uint8_t*>(a.kc3) + dst * 24,
                          const_cast<uint16_t*>(a.kn) + dst, codes);
    const float nv = tq_codes_lane<false>(vx[lane], vx[lane + 64], a.vsign, vq0, vq1);
    tq_store_codes<false>(vq0, vq1, nv, const_cast<uint8_t*>(a.vc4) + dst * 32, const_cast<uint8_t*>(a.vc3) + dst * 24,
                          const_cast<uint16_t*>(a.vn) + dst, codes + 128);
    // scores of the G heads (the norms as stored, fp16)
    const float k0 = c_tq_cb[kq0], k1 = c_tq_cb[16 + kq1];
    const float kscale = h2f_bits(f2h_bits(nk)) * scale;
    float s[G];
#pragma unroll
    for (int h = 0; h < G; ++h) s[h] = wave_sum(k0 * qrot[h * HD + lane] + k1 * qrot[h * HD + lane + 64]) * kscale;
    // the value in the rotated domain, redistributed to the C layout (column
    // t of tile nt is dimension 8t + nt)
    float* v = scratch + 64;
    v[lane] = c_tq_cb[vq0];
    v[lane + 64] = c_tq_cb[16 + vq1];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float vscale = h2f_bits(f2h_bits(nv));
    float st = s[0];
#pragma unroll
    for (int h = 1; h < G; ++h) st = t == h ? s[h] : st;
    m = st;
    lsum = g == 0 ? 1.0f : 0.0f;  // exp(st - m); the record's sum over the lane groups
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[nt][i] = vscale * v[8 * t + nt];
}

// One split of one (kv head, sequence) over TurboQuant pages: the page
// schedule of attn_f16_run (pairs, two in flight when a wavefront has more
// than one), q rotated once per block (q~ = H D q in LDS); the last block
// of the (sequence, kv head) merges the records and rotates the value sums
// back (merge_last<G, 128, true>).
// CUR: the extra block of a launch with kv_cur (the position being written,
// no pages; tq_current_record).
template <int G, bool PIPE, bool COOL = false, bool CUR = false>
__device__ inline void attn_tq_run(const AttnArgs& a, int nsplit, int pps, int split, int kvh, int b,
                                   int range = 0, int slot = -1, int nrec = 0, int ntq = 0) {
    constexpr int HD = 128, REC = rec_floats(G, HD), MO = G * HD, LO = G * HD + G;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, t = lane & 15;
    __shared__ __align__(16) float lds[kAttnWaves * REC];
    __shared__ float qrot[G * HD];
    __shared__ uint2 cbk[kTqTbl];

    attn_args_early(a);
    asm volatile("" ::"s"(a.kc4), "s"(a.kc3), "s"(a.vc4), "s"(a.vc3), "s"(a.kn), "s"(a.vn), "s"(a.ksign),
                 "s"(a.vsign), "s"(nsplit), "s"(pps));
    if (slot < 0) {
        slot = split;
        nrec = nsplit;
        ntq = nsplit;  // every record rotated
    }
    int ctx, pg0;
    attn_range(a, b, range, ctx, pg0);
    const bool cur = range == 0 && a.kv_cur != nullptr;  // the current position comes from kv_cur
    if (cur) ctx -= 1;
    const int p0 = split * pps;
    const int npw_max = (pps - wave + kAttnWaves - 1) / kAttnWaves;
    const int my_page = p0 + wave + kAttnWaves * lane;
    const int bt_lane = (lane < npw_max && pg0 + my_page < a.max_blocks)
                            ? (COOL ? a.cool_table : a.block_table)[(size_t)b * a.max_blocks + pg0 + my_page]
                            : 0;
    const int npages = (ctx + kPage - 1) / kPage;
    const int p1 = min(p0 + pps, npages);
    const int npw = p1 > p0 + wave ? (p1 - p0 - wave + kAttnWaves - 1) / kAttnWaves : 0;
    auto valid_of = [&](int i) { return i < npw ? min(ctx - (p0 + wave + kAttnWaves * i) * kPage, kPage) : 0; };
    auto blk_of = [&](int i) { return __builtin_amdgcn_readlane(bt_lane, min(i, kWave - 1)); };
    const TqLane ln(a, t, COOL);

    // q and the K signs (wavefront w: head min(w, G - 1), lane l: dimensions
    // l and l + 64), the codebook, then the first pair of pages: all in
    // flight before q is rotated
    const float* qsrc = a.q + ((size_t)b * a.hq + kvh * G + min(wave, G - 1)) * HD;
    const float q0 = qsrc[lane], q1 = qsrc[lane + 64];
    const float s0 = a.ksign[lane], s1 = a.ksign[lane + 64];
    // pair-table entry of this thread (threads < kTqTbl)
    const int te = min((int)threadIdx.x, kTqTbl - 1);
    const float cb0 = te < kTqTbl4 ? c_tq_cb[te & 15] : c_tq_cb[16 + ((te - kTqTbl4) & 7)];
    const float cb1 = te < kTqTbl4 ? c_tq_cb[te >> 4] : c_tq_cb[16 + ((te - kTqTbl4) >> 3)];
    // page pair p (pages 2p, 2p + 1 of the wavefront); pairs past the
    // wavefront's pages are not requested (the first pair always is: a
    // wavefront with no pages re-reads its first page and processes nothing;
    // re-reading it for every pair past the last cost 32K attention 0.5 us)
    auto blk_or0 = [&](int i) { return i < npw ? blk_of(i) : blk_of(0); };
    auto load_p = [&](TqPair& r, int p) {
        if (p == 0 || 2 * p < npw)
            tq_load_pair<COOL>(r, a, ln, blk_or0(2 * p), blk_or0(2 * p + 1), valid_of(2 * p + 1), kvh, lane);
    };
    TqPair r0, r1, r2;
    load_p(r0, 0);
    if constexpr (PIPE) load_p(r1, 1);

    if (threadIdx.x < kTqTbl) {
        const _Float16 h0 = (_Float16)cb0, h1 = (_Float16)cb1;
        const _Float16 l0 = (_Float16)(cb0 - (float)h0), l1 = (_Float16)(cb1 - (float)h1);
        cbk[threadIdx.x] = make_uint2(
            (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16),
            (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16));
    }
    // q~ = H D q of head w in wavefront w
    if (wave < G) {
        float u0 = s0 * q0, u1 = s1 * q1;
        wave_fwht128(u0, u1);
        qrot[wave * HD + lane] = u0;
        qrot[wave * HD + lane + 64] = u1;
    }
    __syncthreads();

    // q~ as the B operand: column = head t (columns past G repeat head G-1),
    // k-step s in the dimension order of the K operand
    h8_t qh[4], ql[4];
    {
        const float* qr = qrot + min(t, G - 1) * HD;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int d0 = (s < 2 ? 0 : 64) + 16 * g + 8 * (s & 1);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float v = qr[d0 + j];
                qh[s][j] = (_Float16)v;
                ql[s][j] = (_Float16)(v - (float)qh[s][j]);
            }
        }
    }
    const float scale = kTqScale / sqrtf((float)HD);  // rotation normalisation and 1/sqrt(hd)

    float m = -__builtin_inff(), lsum = 0.0f;
    f4_t o[8];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) o[nt] = f4_t{0.f, 0.f, 0.f, 0.f};
    auto upd = [&](const TqPair& r, int p) {
        tq_pair_update<COOL>(r, ln, qh, ql, cbk, scale, valid_of(2 * p), valid_of(2 * p + 1), m, lsum, o, lane);
    };
    if constexpr (CUR) {
        if (wave == 0) tq_current_record<G>(a, b, kvh, qrot, scale, m, lsum, o);
    } else if constexpr (PIPE) {
        // three register sets in rotation: pair p + 2 is requested before
        // pair p is used, so two pairs stay in flight
        const int np = (npw + 1) / 2;
        for (int p = 0; p < np; p += 3) {
            load_p(r2, p + 2);
            upd(r0, p);
            if (p + 1 >= np) break;
            load_p(r0, p + 3);
            upd(r1, p + 1);
            if (p + 2 >= np) break;
            load_p(r1, p + 4);
            upd(r2, p + 2);
        }
    } else {
        if (npw > 0) upd(r0, 0);
    }
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    // wavefront record: rows h = 4g + i < G of O (column t of tile nt is
    // dimension 8t + nt), m / l of head t
    float* my = lds + wave * REC;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (4 * g + i < G) my[(4 * g + i) * HD + 8 * t + nt] = o[nt][i];
    if (g == 0 && t < G) {
        my[MO + t] = m;
        my[LO + t] = lsum;
    }
    float* parts = a.part + ((size_t)b * a.hkv + kvh) * nrec * REC;
    merge_waves_store<G, HD, true>(parts + (size_t)slot * REC, lds);
    // as attn_f16_run: the record is stored before the block counts itself;
    // the last of the nrec blocks merges, rotates back and resets the counter
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __shared__ int last;
    if (threadIdx.x == 0) {
        unsigned* cnt = a.counts + ((size_t)b * a.hkv + kvh) * kAttnCountStride;
        const unsigned prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = prev == (unsigned)nrec - 1u;
        if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (last) merge_last<G, HD, true>(a, nrec, ntq, kvh, b);
}

// With kv_cur the last block of each (sequence, kv head) takes the position
// being written (its own instantiation, so the page loop's registers are
// not shared with it).
template <int G, bool PIPE>
__global__ __launch_bounds__(kAttnThreads, 1) void k_attn_tq(AttnArgs a, int nsplit, int pps) {
    if (a.kv_cur && (int)blockIdx.x == nsplit - 1)
        attn_tq_run<G, false, false, true>(a, nsplit, pps, blockIdx.x, blockIdx.y, blockIdx.z);
    else
        attn_tq_run<G, PIPE>(a, nsplit, pps, blockIdx.x, blockIdx.y, blockIdx.z);
}

// ----------------------------------------------------- TurboQuant encode --
// One wavefront per vector; lane l holds coordinates l and l + 64.
// Norm, rotation and codes (the oracle's arithmetic in its order): returns
// n = |x|; q0, q1 = the codes of coordinates l and l + 64, the first from the
// 16-level boundaries (Cool: the 8-level ones), the second from the 8-level.
template <bool COOL>
__device__ inline float tq_codes_lane(float x0, float x1, const float* __restrict__ sign, int& q0, int& q1) {
    const int lane = threadIdx.x & 63;
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
    wave_fwht128(u0, u1);
    const float y0 = u0 * kTqScale, y1 = u1 * kTqScale;
    q0 = 0;
    q1 = 0;
    if constexpr (COOL) {
#pragma unroll
        for (int j = 0; j < 7; ++j) q0 += (y0 < c_tq_b3[j]) ? 0 : 1;
    } else {
#pragma unroll
        for (int j = 0; j < 15; ++j) q0 += (y0 < c_tq_b4[j]) ? 0 : 1;
    }
#pragma unroll
    for (int j = 0; j < 7; ++j) q1 += (y1 < c_tq_b3[j]) ? 0 : 1;
    return n;
}

// Pack and store one vector's codes (a wavefront, through its own LDS row):
// TurboQuant: 64 x 4 bits LSB-first at ca (32 B), 64 x 3 bits at cb (24 B);
// Cool: 128 x 3 bits at ca (48 B).  Then the fp16 norm.
template <bool COOL>
__device__ inline void tq_store_codes(int q0, int q1, float n, uint8_t* __restrict__ ca, uint8_t* __restrict__ cb,
                                      uint16_t* __restrict__ norm, uint8_t* lds_codes) {
    const int lane = threadIdx.x & 63;
    lds_codes[lane] = (uint8_t)q0;
    lds_codes[lane + 64] = (uint8_t)q1;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if constexpr (COOL) {
        if (lane < 48) {
            const int g = lane / 3, r = lane % 3;
            uint32_t bits = 0;
#pragma unroll
            for (int m = 0; m < 8; ++m) bits |= (uint32_t)lds_codes[8 * g + m] << (3 * m);
            ca[lane] = (uint8_t)(bits >> (8 * r));
        }
    } else {
        if (lane < 32) ca[lane] = (uint8_t)(lds_codes[2 * lane] | (lds_codes[2 * lane + 1] << 4));
        if (lane < 24) {
            const int g = lane / 3, r = lane % 3;
            uint32_t bits = 0;
#pragma unroll
            for (int m = 0; m < 8; ++m) bits |= (uint32_t)lds_codes[64 + 8 * g + m] << (3 * m);
            cb[lane] = (uint8_t)(bits >> (8 * r));
        }
    }
    if (lane == 0) *norm = f2h_bits(n);
}

__device__ inline void tq_encode_vals(float x0, float x1, const float* __restrict__ sign,
                                      uint8_t* __restrict__ c4, uint8_t* __restrict__ c3,
                                      uint16_t* __restrict__ norm, uint8_t* lds_codes) {
    int q0, q1;
    const float n = tq_codes_lane<false>(x0, x1, sign, q0, q1);
    tq_store_codes<false>(q0, q1, n, c4, c3, norm, lds_codes);
}

// Codes of coordinates l and l + 64 of a stored TurboQuant vector.
__device__ inline void tq_load_codes_lane(const uint8_t* c4, const uint8_t* c3, int& q0, int& q1) {
    const int lane = threadIdx.x & 63;
    q0 = (c4[lane >> 1] >> (4 * (lane & 1))) & 15;
    const int bit = 3 * lane, byte = bit >> 3;
    q1 = ((c3[byte] | (c3[min(byte + 1, 23)] << 8)) >> (bit & 7)) & 7;
}

// Decoded coordinates l and l + 64 of a TurboQuant vector from its codes:
// u = codebook values, the FWHT, then ((u / sqrt(128)) * sign) * norm.
__device__ inline void tq_values_lane(int q0, int q1, uint16_t norm, const float* __restrict__ sign, float& x0,
                                      float& x1) {
    const int lane = threadIdx.x & 63;
    float u0 = c_tq_cb[q0], u1 = c_tq_cb[16 + q1];
    wave_fwht128(u0, u1);
    const float nrm = h2f_bits(norm);
    x0 = ((u0 * kTqScale) * sign[lane]) * nrm;
    x1 = ((u1 * kTqScale) * sign[lane + 64]) * nrm;
}

// One vector of 128 from memory: lane l takes entries l and l + 64.
__device__ inline void tq_encode_wave(const float* __restrict__ x, const float* __restrict__ sign,
                                      uint8_t* __restrict__ c4, uint8_t* __restrict__ c3,
                                      uint16_t* __restrict__ norm, uint8_t* lds_codes) {
    const int lane = threadIdx.x & 63;
    tq_encode_vals(x[lane], x[lane + 64], sign, c4, c3, norm, lds_codes);
}

__global__ __launch_bounds__(256) void k_tq_encode(const float* x, int nvec, const float* signs,
                                                   uint8_t* c4, uint8_t* c3, uint16_t* norms,
                                                   const int32_t* idx) {
    __shared__ uint8_t codes[4][128];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int v = blockIdx.x * 4 + wave;
    if (v >= nvec) return;
    const int dst = idx ? idx[v] : v;
    tq_encode_wave(x + (size_t)v * 128, signs, c4 + (size_t)dst * 32, c3 + (size_t)dst * 24,
                   norms + dst, codes[wave]);
}

// Context rows [p0, ctx) of x [ctx][hkv][128] of sequence b -> pages.
__global__ __launch_bounds__(256) void k_tq_encode_ctx(const float* x, int ctx, int hkv,
                                                       const float* signs, uint8_t* c4,
                                                       uint8_t* c3, uint16_t* norms,
                                                       const int32_t* block_table, int max_blocks,
                                                       int b, int p0) {
    __shared__ uint8_t codes[4][128];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int v = p0 * hkv + blockIdx.x * 4 + wave;
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
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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

// A prompt chunk's K and V rows [n][2][hkv*128] (positions p0 + t) into the
// sequence's pages, one wavefront per vector (the encoder of k_tq_append).
__global__ __launch_bounds__(256) void k_tq_encode_rows(const float* kvrows, int n, int p0, int hkv,
                                                        const float* ksign, const float* vsign, uint8_t* kc4,
                                                        uint8_t* kc3, uint16_t* kn, uint8_t* vc4, uint8_t* vc3,
                                                        uint16_t* vn, const int32_t* bt) {
    __shared__ uint8_t codes[4][128];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int v = blockIdx.x * 4 + wave;  // (t, kv, h)
    if (v >= n * 2 * hkv) return;
    const int t = v / (2 * hkv), kv = (v / hkv) % 2, h = v % hkv, p = p0 + t;
    const size_t dst = ((size_t)bt[p / kPage] * hkv + h) * kPage + p % kPage;
    const float* src = kvrows + ((size_t)t * 2 + kv) * hkv * 128 + (size_t)h * 128;
    if (kv == 0)
        tq_encode_wave(src, ksign, kc4 + dst * 32, kc3 + dst * 24, kn + dst, codes[wave]);
    else
        tq_encode_wave(src, vsign, vc4 + dst * 32, vc3 + dst * 24, vn + dst, codes[wave]);
}

// TurboQuant vectors of positions < npos of one sequence back to fp16 pages
// of the same blocks, one wavefront per vector: u_i = codebook value of code
// i (4-bit for i < 64, 3-bit after), the FWHT, then ((u_i / sqrt(128)) *
// sign_i) * norm -- the decoder's arithmetic in its order -- rounded to fp16.
// K also as its fp16 remainder (klo = K - fp16(K)), for scores to fp32
// accuracy.
__global__ __launch_bounds__(256) void k_tq_decode_pages(const uint8_t* kc4, const uint8_t* kc3, const uint16_t* kn,
                                                         const uint8_t* vc4, const uint8_t* vc3, const uint16_t* vn,
                                                         const float* ksign, const float* vsign, const int32_t* bt,
                                                         int npos, int hkv, uint16_t* kpool, uint16_t* vpool,
                                                         uint16_t* klo) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int v = blockIdx.x * 4 + wave;  // (p, kv, h)
    if (v >= npos * 2 * hkv) return;
    const int p = v / (2 * hkv), kv = (v / hkv) % 2, h = v % hkv;
    const size_t blk = (size_t)bt[p / kPage], vec = (blk * hkv + h) * kPage + p % kPage;
    int q0, q1;
    tq_load_codes_lane((kv ? vc4 : kc4) + vec * 32, (kv ? vc3 : kc3) + vec * 24, q0, q1);
    float x0, x1;
    tq_values_lane(q0, q1, (kv ? vn : kn)[vec], kv ? vsign : ksign, x0, x1);
    const uint16_t o0 = f2h_bits(x0), o1 = f2h_bits(x1);
    const size_t page = (blk * hkv + h) * kPage * 128;
    const int slot = p % kPage;
    if (kv) {  // V pages are dimension-major [128][16]
        vpool[page + (size_t)lane * kPage + slot] = o0;
        vpool[page + (size_t)(lane + 64) * kPage + slot] = o1;
    } else {   // K pages are token-major [16][128]
        kpool[page + (size_t)slot * 128 + lane] = o0;
        kpool[page + (size_t)slot * 128 + lane + 64] = o1;
        klo[page + (size_t)slot * 128 + lane] = f2h_bits(x0 - h2f_bits(o0));
        klo[page + (size_t)slot * 128 + lane + 64] = f2h_bits(x1 - h2f_bits(o1));
    }
}

// Causal prefill attention over fp16 pages: query rows t < P of one sequence
// (positions p0 + t) attend to the positions <= their own.  A wavefront takes
// 16 consecutive queries of one head as the columns of the decode layout
// (S = K q^T per page, O = P V per page pair), a block the G heads of one kv
// head for the same queries, whose page loads are the same addresses and
// meet in the L1.  Each wavefront walks the page pairs up to its last
// query's position; the scores get the causal mask per (token, query).
// Blocks are numbered from the last query tile down, so the longest walks
// start first.
// KLO: K pages are fp16 hi (kpool) + lo (kpool_lo), a third product per step
// (prefill over TurboQuant pages decoded for it).
// hsub blocks share a kv head (grid row y = kvh * hsub + sub), each taking G
// of its G * hsub query heads, sub * G + w.
// TIER (tiered pages, with KLO): query tiles are page-aligned positions (the
// first tile starts p0 % 16 queries before the prompt), so a tile's queries
// share one cold boundary; pages before it come from the decoded TurboQuant
// pools, the rest from the fp16 pages kpool_win / vpool_win (K lo zero).
template <int G, int HD, bool KLO = false, bool TIER = false>
__global__ __launch_bounds__(64 * G) void k_attn_prefill(AttnArgs a, int p0, int P, int hsub) {
    static_assert(!TIER || KLO, "tiered prefill reads decoded TurboQuant pages as hi + lo");
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), g = lane >> 4, t = lane & 15;
    const int kvh = (int)blockIdx.y / hsub, h = kvh * G * hsub + ((int)blockIdx.y - kvh * hsub) * G + w;
    const int qoff = TIER ? p0 % kPage : 0;
    const int q0 = ((int)gridDim.x - 1 - (int)blockIdx.x) * 16 - qoff;
    const int qi = min(max(q0 + t, 0), P - 1);  // this lane's query (clamped into the prompt)
    const int lastpos = p0 + min(q0 + 15, P - 1);
    const int npages = lastpos / kPage + 1;
    // the tile's cold boundary in pages (positions p0 + q0 .. + 15 share it)
    const int bnd = TIER ? max(0, (p0 + q0 - a.hot_window) / kPage) : 0;
    // q as the B operand: column t = query q0 + t (clamped: columns past the
    // prompt repeat its last query and are not written), k = 8g + j
    h8_t qh[HD / 32], ql[HD / 32];
    {
        const float* qsrc = a.q + ((size_t)qi * a.hq + h) * HD + 8 * g;
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
    const int qpos = p0 + qi;
    float m = -__builtin_inff(), lsum = 0.0f;
    f4_t o[HD / 16];
#pragma unroll
    for (int nt = 0; nt < HD / 16; ++nt) o[nt] = f4_t{0.f, 0.f, 0.f, 0.f};
    if constexpr (HD > 128) {
        // 256-long heads: each lane's q operands go to its own LDS slots and
        // are read per k-step (registers hold one page pair, its products
        // and O), one pair in flight
        static_assert(!KLO, "256-long heads have fp16 pages only");
        __shared__ __align__(16) uint4 qlds[G * kWave * (HD / 32) * 2];
        uint4* qls = qlds + ((size_t)w * kWave + lane) * (HD / 32) * 2;
#pragma unroll
        for (int s = 0; s < HD / 32; ++s) {
            qls[2 * s] = __builtin_bit_cast(uint4, qh[s]);
            qls[2 * s + 1] = __builtin_bit_cast(uint4, ql[s]);
        }
        auto blk1 = [&](int p) { return a.block_table[min(p, npages - 1)]; };
        auto valid1 = [&](int p) { return p < npages ? min(max(lastpos + 1 - kPage * p, 0), kPage) : 0; };
        PairRaw<HD> r1;
        for (int pa = 0; pa < npages; pa += 2) {
            load_pair<HD>(r1, a, blk1(pa), valid1(pa), blk1(pa + 1), valid1(pa + 1), kvh, lane);
            pair_update<HD, true, false, true>(r1, qh, ql, scale, valid1(pa), valid1(pa + 1), m, lsum, o, lane,
                                               kPage * pa, kPage * (pa + 1), qpos, nullptr, qls);
        }
    } else {
        // page pairs with the next pair in flight: it is requested unconditionally
        // (pages past the walk re-read its last page with no valid tokens), so
        // the wait for the current pair leaves the next one outstanding
        auto blk_of = [&](int p) { return a.block_table[min(p, npages - 1)]; };
        auto valid_of = [&](int p) { return p < npages ? min(max(lastpos + 1 - kPage * p, 0), kPage) : 0; };
        PairRaw<HD> ra, rb;
        PairKlo<HD> la, lb;
        // K lo of a pair (KLO), the same addresses in kpool_lo (TIER: pages from
        // the boundary on read the zero page)
        auto load_lo = [&](PairKlo<HD>& r, int pa_, int pb_) {
            if constexpr (KLO) {
#pragma unroll
                for (int pg = 0; pg < 2; ++pg) {
                    const int pp = pg && valid_of(pb_) > 0 ? pb_ : pa_;
                    const size_t base = ((size_t)blk_of(pp) * a.hkv + kvh) * kPage * HD;
                    const uint16_t* lo = TIER && pp >= bnd ? a.lo_zero : a.kpool_lo + base;
#pragma unroll
                    for (int s = 0; s < HD / 32; ++s)
                        r.k[pg][s] = *reinterpret_cast<const uint4*>(lo + (size_t)t * HD + 32 * s + 8 * g);
                }
            }
        };
        auto load_p = [&](PairRaw<HD>& r, int pa_, int pb_) {
            if constexpr (TIER) {
                const bool wa = pa_ >= bnd, wb = pb_ >= bnd;
                load_pair_from<HD>(r, wa ? a.kpool_win : a.kpool, wa ? a.vpool_win : a.vpool, blk_of(pa_),
                                   wb ? a.kpool_win : a.kpool, wb ? a.vpool_win : a.vpool, blk_of(pb_), valid_of(pb_),
                                   a.hkv, kvh, lane);
            } else {
                load_pair<HD>(r, a, blk_of(pa_), valid_of(pa_), blk_of(pb_), valid_of(pb_), kvh, lane);
            }
        };
        load_lo(la, 0, 1);
        load_p(ra, 0, 1);
        for (int pa = 0; pa < npages; pa += 4) {
            load_lo(lb, pa + 2, pa + 3);
            load_p(rb, pa + 2, pa + 3);
            pair_update<HD, true, KLO>(ra, qh, ql, scale, valid_of(pa), valid_of(pa + 1), m, lsum, o, lane, kPage * pa,
                                       kPage * (pa + 1), qpos, &la);
            if (pa + 2 >= npages) break;
            load_lo(la, pa + 4, pa + 5);
            load_p(ra, pa + 4, pa + 5);
            pair_update<HD, true, KLO>(rb, qh, ql, scale, valid_of(pa + 2), valid_of(pa + 3), m, lsum, o, lane,
                                       kPage * (pa + 2), kPage * (pa + 3), qpos, &lb);
        }
    }
    // the query's denominator: sum of the four lanes that share its column
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    // rows of O in this lane are queries 4g + i, their denominators in lanes 4g + i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float L = __shfl(lsum, 4 * g + i, 64);
        const int q = q0 + 4 * g + i;
        if (q >= 0 && q < P) {
            uint16_t* out = a.out16 + ((size_t)q * a.hq + h) * HD + t;
#pragma unroll
            for (int nt = 0; nt < HD / 16; ++nt) out[16 * nt] = f2h_bits(o[nt][i] / L);
        }
    }
}

// Tiered pages, the page that leaves the fp16 window at this step: when
// the position p being written completes page q = (p - H + 1) / 16 - 1
// outside the window (p - H + 1 a positive multiple of 16), its fp16 K or V
// (ring page hot_table[q]) is encoded into the TurboQuant page
// block_table[q]: block `part` of the four of each kind encodes slots
// 4 part .. 4 part + 3 on its first wavefront.  On the other steps the block
// leaves at once.  The attention blocks of the same launch
// read page q as fp16 and the TurboQuant pages before it only.
constexpr int kCompressParts = 4;
constexpr int kCompressWaves = kPage / kCompressParts;  // one slot per wavefront
static_assert(kCompressWaves <= kAttnWaves, "a compressing block holds one wavefront per slot of its part");
// Block `part` of the K (kv 0) or V (kv 1) compression: wavefront w encodes
// slot part * kCompressWaves + w of the page that left the window.  Each
// wavefront packs its codes through its own row of LDS scratch; a single row
// shared by the block would let one wavefront overwrite the codes another
// is still packing.
__device__ inline void tq_compress_block(const AttnArgs& a, int kv, int part, int h, int b) {
    __shared__ uint8_t codes[kCompressWaves][128];
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int done = a.pos[b] - a.hot_window + 1;
    if (w >= kCompressWaves || done < kPage || done % kPage) return;
    const int q = done / kPage - 1;
    const int slot = part * kCompressWaves + w;
    const size_t hot = (size_t)a.hot_table[(size_t)b * a.max_blocks + q] * a.hkv + h;
    const size_t dst = ((size_t)a.block_table[(size_t)b * a.max_blocks + q] * a.hkv + h) * kPage + slot;
    // the TurboQuant pools, written only here
    uint8_t* c4 = const_cast<uint8_t*>(kv ? a.vc4 : a.kc4);
    uint8_t* c3 = const_cast<uint8_t*>(kv ? a.vc3 : a.kc3);
    uint16_t* nr = const_cast<uint16_t*>(kv ? a.vn : a.kn);
    const float* sign = kv ? a.vsign : a.ksign;
    float x0, x1;
    if (kv == 0) {  // K pages are token-major [16][128]
        const uint16_t* src = a.kpool + (hot * kPage + slot) * kTqD;
        x0 = h2f_bits(src[lane]);
        x1 = h2f_bits(src[lane + 64]);
    } else {        // V pages are dimension-major [128][16]
        const uint16_t* src = a.vpool + hot * kPage * kTqD;
        x0 = h2f_bits(src[(size_t)lane * kPage + slot]);
        x1 = h2f_bits(src[(size_t)(lane + 64) * kPage + slot]);
    }
    tq_encode_vals(x0, x1, sign, c4 + dst * 32, c3 + dst * 24, nr + dst, codes[w]);
}

// Three tiers, the page that leaves the Warm range at this step: when the
// position p being written completes page q = (p - H - W + 1) / 16 - 1
// outside the last H + W positions, its TurboQuant vectors (block_table[q])
// are decoded to fp32 and encoded Cool into cool_table[q] -- the Warm ->
// Cool step of compress_tier (kv/paged_attention.cpp:262-285), per page.
// Block `part` of the four of each kind takes slots 4 part .. 4 part + 3,
// one per wavefront.  The TurboQuant page is only read here, and the Warm
// splits of the same launch still read page q in that form; the Hot -> Warm
// compressor of the launch writes page q + W / 16, a different block of the
// Warm ring.
__device__ inline void cool_compress_block(const AttnArgs& a, int kv, int part, int h, int b) {
    __shared__ uint8_t codes[kCompressWaves][128];
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int done = a.pos[b] - a.hot_window - a.warm_window + 1;
    if (w >= kCompressWaves || done < kPage || done % kPage) return;
    const int q = done / kPage - 1;
    const int slot = part * kCompressWaves + w;
    const size_t src = ((size_t)a.block_table[(size_t)b * a.max_blocks + q] * a.hkv + h) * kPage + slot;
    const size_t dst = ((size_t)a.cool_table[(size_t)b * a.max_blocks + q] * a.hkv + h) * kPage + slot;
    const float* sign = kv ? a.vsign : a.ksign;
    int q0, q1;
    tq_load_codes_lane((kv ? a.vc4 : a.kc4) + src * 32, (kv ? a.vc3 : a.kc3) + src * 24, q0, q1);
    float x0, x1;
    tq_values_lane(q0, q1, (kv ? a.vn : a.kn)[src], sign, x0, x1);
    // the Cool pools, written only here and by the context fill
    uint8_t* cc = const_cast<uint8_t*>(kv ? a.vcc : a.kcc);
    uint16_t* cn = const_cast<uint16_t*>(kv ? a.vcn : a.kcn);
    const float n = tq_codes_lane<true>(x0, x1, sign, q0, q1);
    tq_store_codes<true>(q0, q1, n, cc + dst * 48, nullptr, cn + dst, codes[w]);
}

// Tiered pages in one launch: blocks x < ntq are TurboQuant splits of the
// compressed pages, the next nf fp16 splits of the window (the last of these
// ntq + nf blocks of a (sequence, kv head) merges both kinds of record), and
// the last 2 kCompressParts compress the page leaving the window (K, V).
template <int G, bool PT, bool PF>
__global__ __launch_bounds__(kAttnThreads, 1) void k_attn_tiered(AttnArgs a, int ntq, int ppt, int nf, int ppf) {
    const int x = blockIdx.x;
    if (x < ntq)
        attn_tq_run<G, PT>(a, ntq, ppt, x, blockIdx.y, blockIdx.z, 1, x, ntq + nf, ntq);
    else if (x < ntq + nf)
        attn_f16_run<G, 128, PF, true>(a, nf, x - ntq, blockIdx.y, blockIdx.z, 2, x, ntq + nf, ntq);
    else
        tq_compress_block(a, (x - ntq - nf) / kCompressParts, (x - ntq - nf) % kCompressParts, blockIdx.y,
                          blockIdx.z);
}

// Split plan of three tiers: nc Cool splits of ppc pages, nw TurboQuant
// splits of ppw pages, nf fp16 splits of ppf pages.
struct TierPlan3 {
    int nc, ppc, nw, ppw, nf, ppf;
};

// Three tiers in one launch: blocks x < nc are Cool splits, the next nw
// TurboQuant splits, the next nf fp16 splits (the last of these nc + nw + nf
// blocks of a (sequence, kv head) merges the three kinds of record, the
// first nc + nw in the rotated domain); then 2 kCompressParts blocks
// compress the page leaving the fp16 window (K, V) and 2 kCompressParts the
// page leaving the Warm range.
template <int G, bool PC, bool PW, bool PF>
__global__ __launch_bounds__(kAttnThreads, 1) void k_attn_tiered3(AttnArgs a, TierPlan3 p) {
    const int x = blockIdx.x, nrot = p.nc + p.nw, nrec = nrot + p.nf;
    if (x < p.nc) {
        attn_tq_run<G, PC, true>(a, p.nc, p.ppc, x, blockIdx.y, blockIdx.z, 3, x, nrec, nrot);
    } else if (x < nrot) {
        attn_tq_run<G, PW>(a, p.nw, p.ppw, x - p.nc, blockIdx.y, blockIdx.z, 1, x, nrec, nrot);
    } else if (x < nrec) {
        attn_f16_run<G, 128, PF, true>(a, p.nf, x - nrot, blockIdx.y, blockIdx.z, 2, x, nrec, nrot);
    } else {
        const int c = x - nrec;
        if (c < 2 * kCompressParts)
            tq_compress_block(a, c / kCompressParts, c % kCompressParts, blockIdx.y, blockIdx.z);
        else
            cool_compress_block(a, (c - 2 * kCompressParts) / kCompressParts, c % kCompressParts, blockIdx.y,
                                blockIdx.z);
    }
}

// Context fill of Cool pages: positions [p0, n) of x [ctx][hkv][128] (fp32,
// the fp16 values) of sequence b, one wavefront per vector, encoded
// TurboQuant, decoded, and encoded Cool (what the per-page compressors give
// a position that passed through both steps) into cool_table's pages.
__global__ __launch_bounds__(256) void k_cool_encode_ctx(const float* x, int p0, int n, int hkv, const float* signs,
                                                         uint8_t* cc, uint16_t* cn, const int32_t* cool_table,
                                                         int max_blocks, int b) {
    __shared__ uint8_t codes[4][128];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int v = p0 * hkv + blockIdx.x * 4 + wave;
    if (v >= n * hkv) return;
    const int t = v / hkv, h = v % hkv;
    const size_t dst = ((size_t)cool_table[(size_t)b * max_blocks + t / kPage] * hkv + h) * kPage + t % kPage;
    const float* src = x + (size_t)v * 128;
    int q0, q1;
    const float nw = tq_codes_lane<false>(src[lane], src[lane + 64], signs, q0, q1);
    float x0, x1;
    tq_values_lane(q0, q1, f2h_bits(nw), signs, x0, x1);
    const float nc = tq_codes_lane<true>(x0, x1, signs, q0, q1);
    tq_store_codes<true>(q0, q1, nc, cc + dst * 48, nullptr, cn + dst, codes[wave]);
}

// Context fill of tiered pages: positions [cold, ctx) of raw [ctx][hkv][hd]
// (fp32) as fp16 into the window's pages of sequence b.
__global__ __launch_bounds__(256) void k_put_hot(const float* raw, int ctx, int cold, int hkv, int hd, int b,
                                                 const int32_t* hot_bt, int max_blocks, uint16_t* kpool,
                                                 uint16_t* vpool, int kv) {
    const long n = (long)(ctx - cold) * hkv * hd;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
        const int p = cold + (int)(i / (hkv * hd)), h = (int)(i / hd % hkv), d = (int)(i % hd);
        const size_t page = ((size_t)hot_bt[(size_t)b * max_blocks + p / kPage] * hkv + h) * kPage * hd;
        const uint16_t v = f2h_bits(raw[((size_t)p * hkv + h) * hd + d]);
        if (kv == 0)
            kpool[page + (size_t)(p % kPage) * hd + d] = v;
        else
            vpool[page + (size_t)d * kPage + p % kPage] = v;
    }
}

// x = fp32(fp16(x)), RNE (the values the fp16 window holds).
__global__ __launch_bounds__(256) void k_round_f16(float* x, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        x[i] = h2f_bits(f2h_bits(x[i]));
}

// Batched prefill over tiered pages (pf_tier_rows_launch): one wavefront per
// (position t in [lo, pe), K or V, kv head), lane l holding coordinates l
// and l + 64 of the fp16 value -- from the window's ring page before pb,
// from the chunk's row (rounded) after.  ring = 0: the value goes to the
// fp16 page of the block table (vk / vv) and, below tq_hi, is encoded into
// the TurboQuant page; ring = 1 (lo >= pb): it goes to the ring page.  (The
// ring is written in a launch of its own: a long chunk's last pages share
// ring slots with the pages before pb that the first launch reads.)
__global__ __launch_bounds__(256) void k_pf_tier_rows(const float* kvrows, int pb, int lo, int pe, int tq_hi,
                                                      int ring, int hkv, int b, const int32_t* bt,
                                                      const int32_t* hot_bt, int max_blocks, uint16_t* ring_k,
                                                      uint16_t* ring_v, uint16_t* vk, uint16_t* vv,
                                                      const float* ksign, const float* vsign, uint8_t* kc4,
                                                      uint8_t* kc3, uint16_t* kn, uint8_t* vc4, uint8_t* vc3,
                                                      uint16_t* vn) {
    constexpr int HD = kTqD;
    __shared__ uint8_t codes[4][128];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int v = blockIdx.x * 4 + wave;  // ((t - lo), kv, h)
    const int t = lo + v / (2 * hkv), kv = (v / hkv) % 2, h = v % hkv;
    if (t >= pe) return;
    const int slot = t % kPage;
    // K pages are token-major [16][128], V pages dimension-major [128][16]
    auto at = [&](int d) { return kv ? (size_t)d * kPage + slot : (size_t)slot * HD + d; };
    uint16_t* const rp = kv ? ring_v : ring_k;
    const size_t rpage = ((size_t)hot_bt[(size_t)b * max_blocks + t / kPage] * hkv + h) * kPage * HD;
    uint16_t x0, x1;
    if (ring) {
        const float* r = kvrows + ((size_t)(t - pb) * 2 + kv) * hkv * HD + (size_t)h * HD;
        rp[rpage + at(lane)] = f2h_bits(r[lane]);
        rp[rpage + at(lane + 64)] = f2h_bits(r[lane + 64]);
        return;
    }
    if (t < pb) {
        x0 = rp[rpage + at(lane)];
        x1 = rp[rpage + at(lane + 64)];
    } else {
        const float* r = kvrows + ((size_t)(t - pb) * 2 + kv) * hkv * HD + (size_t)h * HD;
        x0 = f2h_bits(r[lane]);
        x1 = f2h_bits(r[lane + 64]);
    }
    const int blk = bt[(size_t)b * max_blocks + t / kPage];
    uint16_t* const vp = kv ? vv : vk;
    const size_t vpage = ((size_t)blk * hkv + h) * kPage * HD;
    vp[vpage + at(lane)] = x0;
    vp[vpage + at(lane + 64)] = x1;
    if (t < tq_hi) {
        const size_t dst = ((size_t)blk * hkv + h) * kPage + slot;
        tq_encode_vals(h2f_bits(x0), h2f_bits(x1), kv ? vsign : ksign, (kv ? vc4 : kc4) + dst * 32,
                       (kv ? vc3 : kc3) + dst * 24, (kv ? vn : kn) + dst, codes[wave]);
    }
}

}  // namespace

hipError_t put_hot_launch(const float* raw, int ctx, int cold, int hkv, int hd, int b, const int32_t* hot_bt,
                          int max_blocks, uint16_t* kpool, uint16_t* vpool, int kv, hipStream_t st) {
    if (ctx <= cold) return hipSuccess;
    hipLaunchKernelGGL(k_put_hot, dim3(256), dim3(256), 0, st, raw, ctx, cold, hkv, hd, b, hot_bt, max_blocks, kpool,
                       vpool, kv);
    return hipGetLastError();
}

hipError_t pf_tier_rows_launch(const float* kvrows, int pb, int lo, int pe, int tq_hi, int ring_lo, int hkv, int b,
                               const int32_t* bt, const int32_t* hot_bt, int max_blocks, uint16_t* ring_k,
                               uint16_t* ring_v, uint16_t* vk, uint16_t* vv, const float* ksign, const float* vsign,
                               uint8_t* kc4, uint8_t* kc3, uint16_t* kn, uint8_t* vc4, uint8_t* vc3, uint16_t* vn,
                               hipStream_t st) {
    // the ring holds the positions before pb that are not yet TurboQuant
    if (lo < 0 || lo > pb || pb > pe || tq_hi < lo || tq_hi > pe || ring_lo < pb || hkv < 1) return hipErrorInvalidValue;
    for (int ring = 0; ring < 2; ++ring) {
        const int from = ring ? ring_lo : lo;
        const long nvec = (long)(pe - from) * 2 * hkv;
        if (nvec <= 0) continue;
        hipLaunchKernelGGL(k_pf_tier_rows, dim3((unsigned)((nvec + 3) / 4)), dim3(256), 0, st, kvrows, pb, from, pe,
                           tq_hi, ring, hkv, b, bt, hot_bt, max_blocks, ring_k, ring_v, vk, vv, ksign, vsign, kc4, kc3,
                           kn, vc4, vc3, vn);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t round_f16_launch(float* x, size_t n, hipStream_t st) {
    hipLaunchKernelGGL(k_round_f16, dim3(1024), dim3(256), 0, st, x, n);
    return hipGetLastError();
}

// K hi + lo pages (kpool_lo) for head_dim 128: at most 4 query heads per
// block (with 8, the kernel's two wavefronts per SIMD cannot hold the lo
// operands), so 8 heads per kv head take two blocks of 4 that read the same
// pages (the second block's reads meet the first's in the L2).
template <int G, int HD>
hipError_t attn_prefill_case(const AttnArgs& a, int p0, int P, dim3 grid, hipStream_t st) {
    if constexpr (HD == 128) {
        if (a.kpool_lo) {
            constexpr int GB = G <= 4 ? G : 4, HS = G / GB;
            static_assert(GB * HS == G, "query heads per kv head split into blocks of at most 4");
            if (a.kpool_win) {
                // tiered pages: page-aligned query tiles, one more when the
                // prompt starts inside a page
                if (!a.vpool_win || !a.lo_zero || a.hot_window < kPage || a.hot_window % kPage)
                    return hipErrorInvalidValue;
                hipLaunchKernelGGL((k_attn_prefill<GB, HD, true, true>), dim3((P + p0 % kPage + 15) / 16, grid.y * HS),
                                   dim3(64 * GB), 0, st, a, p0, P, HS);
                return hipGetLastError();
            }
            hipLaunchKernelGGL((k_attn_prefill<GB, HD, true>), dim3(grid.x, grid.y * HS), dim3(64 * GB), 0, st, a,
                               p0, P, HS);
            return hipGetLastError();
        }
    }
    if (a.kpool_lo || a.kpool_win) return hipErrorInvalidValue;
    hipLaunchKernelGGL((k_attn_prefill<G, HD>), grid, dim3(64 * G), 0, st, a, p0, P, 1);
    return hipGetLastError();
}

hipError_t attn_prefill_launch(const AttnArgs& a, int p0, int P, hipStream_t st) {
    if (P < 1 || p0 < 0 || !a.block_table) return hipErrorInvalidValue;
    const dim3 grid((P + 15) / 16, a.hkv);
    const int G = a.hq / a.hkv;
#define NX_PF_ATTN_CASE(GG, HH) \
    if (G == GG && a.hd == HH) return attn_prefill_case<GG, HH>(a, p0, P, grid, st);
    NX_PF_ATTN_CASE(1, 64)
    NX_PF_ATTN_CASE(2, 64)
    NX_PF_ATTN_CASE(4, 64)
    NX_PF_ATTN_CASE(8, 64)
    NX_PF_ATTN_CASE(1, 128)
    NX_PF_ATTN_CASE(2, 128)
    NX_PF_ATTN_CASE(4, 128)
    NX_PF_ATTN_CASE(8, 128)
    NX_PF_ATTN_CASE(1, 256)
    NX_PF_ATTN_CASE(2, 256)
    NX_PF_ATTN_CASE(4, 256)
    NX_PF_ATTN_CASE(8, 256)
#undef NX_PF_ATTN_CASE
    return hipErrorInvalidValue;
}

SplitPlan plan_splits_f16(int max_ctx, int hkv, int batch);
size_t attn_workspace_bytes(int batch, int hq, int hkv, int hd, int max_ctx) {
    // TurboQuant pages in the decode step: one more record (the position being written)
    const int nsplit = max(min(plan_splits(max_ctx).nsplit + 1, kMaxSplits), plan_splits_f16(max_ctx, hkv, batch).nsplit);
    const int G = hq / hkv;
    return sizeof(float) * (size_t)batch * hkv * nsplit * rec_floats(G, hd);
}

int attn_max_ctx() { return kMaxSplits * kPagesPerSplitMax * kPage; }

SplitPlan plan_splits_f16(int max_ctx, int hkv, int batch);
size_t attn_f16_workspace_bytes(int batch, int hq, int hkv, int hd, int max_ctx) {
    const SplitPlan sp = plan_splits_f16(max_ctx, hkv, batch);
    return sizeof(float) * (size_t)batch * hkv * sp.nsplit * rec_floats(hq / hkv, hd);
}

// TurboQuant splits: about one block per CU over all (kv head, sequence)
// pairs (the pipelined kernel holds one 8-wavefront block per CU), never
// more splits than plan_splits (which sizes the workspace); `extra` blocks
// per pair that read no pages (the position being written) count against
// the CUs too.
SplitPlan plan_splits_tq(int max_ctx, int hkv, int batch, int extra = 0) {
    const SplitPlan base = plan_splits(max_ctx);
    const int pages = (max_ctx + kPage - 1) / kPage;
    const int want = (device_cus() + hkv * batch - 1) / (hkv * batch) - extra;
    int nsplit = min(base.nsplit, max(want, 1));
    const int pps = min(max((pages + nsplit - 1) / nsplit, 1), kPagesPerSplitMax);
    nsplit = max((pages + pps - 1) / pps, 1);
    return {nsplit, pps};
}

// fp16 splits: as many as fill the CUs with one block each over all (kv
// head, sequence) pairs, at most kMaxSplits and at most one per page of the
// longest context.  Pages are dealt round-robin (attn_f16_run), so pps is
// the most pages any split takes; more than two per wavefront (pps >
// kPagesPerSplitMin) selects the pipelined kernel.
SplitPlan plan_splits_f16(int max_ctx, int hkv, int batch) {
    const int pages = max((max_ctx + kPage - 1) / kPage, 1);
    const int want = max(device_cus() / max(hkv * batch, 1), 1);
    // a wavefront holds the block-table entries of its pages one per lane
    const int least = (pages + kPagesPerSplitMax - 1) / kPagesPerSplitMax;
    const int nsplit = min(max(min(want, pages), least), kMaxSplits);
    return {nsplit, (pages + nsplit - 1) / nsplit};
}

// Scratch of nx_attn_decode_paged_f16_noalloc (records, then counters).
// In host code the name is only a stand-in: the device address comes from
// attn_noalloc_scratch.
static __device__ __align__(256) unsigned char g_attn_scratch[kNoAllocRecordBytes + 4 * kNoAllocCountWords];

hipError_t attn_noalloc_scratch(void** out) {
    return hipGetSymbolAddress(out, HIP_SYMBOL(g_attn_scratch));
}

__global__ __launch_bounds__(256) void k_zero_u32(unsigned* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = 0u;
}

hipError_t zero_u32_launch(unsigned* p, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 1024);
    hipLaunchKernelGGL(k_zero_u32, dim3(blocks), dim3(256), 0, st, p, n);
    return hipGetLastError();
}


hipError_t attn_f16_launch(const AttnArgs& a, hipStream_t st) {
    if (!a.counts || !a.part) return hipErrorInvalidValue;
    const SplitPlan sp = plan_splits_f16(a.max_ctx, a.hkv, a.batch);
    const dim3 grid(sp.nsplit, a.hkv, a.batch);
    const int G = a.hq / a.hkv;
    const bool pipe = sp.pps > kPagesPerSplitMin;
#define NX_ATTN_CASE(GG, HH)                                                                      \
    if (G == GG && a.hd == HH) {                                                                  \
        if (pipe)                                                                                 \
            hipLaunchKernelGGL((k_attn_f16<GG, HH, true>), grid, dim3(kAttnThreads), 0, st, a,     \
                               sp.nsplit);                                                        \
        else                                                                                      \
            hipLaunchKernelGGL((k_attn_f16<GG, HH, false>), grid, dim3(kAttnThreads), 0, st, a,    \
                               sp.nsplit);                                                        \
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
    NX_ATTN_CASE(1, 256)
    NX_ATTN_CASE(2, 256)
    NX_ATTN_CASE(4, 256)
    NX_ATTN_CASE(8, 256)
#undef NX_ATTN_CASE
    return hipErrorInvalidValue;
}

hipError_t attn_tq_launch(const AttnArgs& a, hipStream_t st) {
    if (!a.counts || !a.part) return hipErrorInvalidValue;
    SplitPlan sp = plan_splits_tq(a.max_ctx, a.hkv, a.batch, a.kv_cur ? 1 : 0);
    if (a.kv_cur && sp.nsplit >= kMaxSplits) {
        // room for the current position's block among the records
        const int pages = (a.max_ctx + kPage - 1) / kPage;
        sp.pps = (pages + kMaxSplits - 2) / (kMaxSplits - 1);
        sp.nsplit = (pages + sp.pps - 1) / sp.pps;
        if (sp.pps > kPagesPerSplitMax) return hipErrorInvalidValue;
    }
    // with kv_cur, one more block: the position being written (no pages)
    if (a.kv_cur) sp.nsplit += 1;
    const dim3 grid(sp.nsplit, a.hkv, a.batch);
    const int G = a.hq / a.hkv;
    if (a.hd != 128) return hipErrorInvalidValue;
#define NX_ATTN_CASE(GG)                                                                          \
    if (G == GG) {                                                                                \
        if (sp.pps > kPagesPerSplitMin)                                                           \
            hipLaunchKernelGGL((k_attn_tq<GG, true>), grid, dim3(kAttnThreads), 0, st, a,          \
                               sp.nsplit, sp.pps);                                                \
        else                                                                                      \
            hipLaunchKernelGGL((k_attn_tq<GG, false>), grid, dim3(kAttnThreads), 0, st, a,         \
                               sp.nsplit, sp.pps);                                                \
        return hipGetLastError();                                                                 \
    }
    NX_ATTN_CASE(1)
    NX_ATTN_CASE(2)
    NX_ATTN_CASE(4)
    NX_ATTN_CASE(8)
#undef NX_ATTN_CASE
    return hipErrorInvalidValue;
}

// Tiered split plan: about one block per CU over all (kv head, sequence)
// pairs, shared between the compressed pages (TurboQuant, at most
// (max_ctx - hot_window) / 16 + 1 pages) and the window (hot_window / 16 + 1
// pages) in proportion to their cost, a TurboQuant page taking about 0.8 of
// an fp16 page's time.
struct TierPlan {
    int ntq, ppt, nf, ppf;
};
TierPlan plan_tiered(int max_ctx, int hot_window, int hkv, int batch) {
    const int pt = max(1, (max_ctx - hot_window) / kPage + 1), pf = hot_window / kPage + 2;
    const int S = min(max(2, (device_cus() + hkv * batch - 1) / (hkv * batch)), kMaxSplits);
    const double ct = 0.8 * pt, cf = pf;
    const int nt0 = min(max(1, (int)(S * ct / (ct + cf) + 0.5)), S - 1);
    TierPlan p;
    p.ppt = min(max((pt + nt0 - 1) / nt0, 1), kPagesPerSplitMax);
    p.ntq = (pt + p.ppt - 1) / p.ppt;
    const int nf0 = max(1, S - p.ntq);
    p.ppf = min(max((pf + nf0 - 1) / nf0, 1), kPagesPerSplitMax);
    p.nf = (pf + p.ppf - 1) / p.ppf;
    return p;
}

size_t attn_tiered_workspace_bytes(int batch, int hq, int hkv) {
    return sizeof(float) * (size_t)batch * hkv * kMaxSplits * rec_floats(hq / hkv, 128);
}

// Three tiers: the Cool pages (at most (max_ctx - H - W) / 16 + 1, or C / 16
// + 1 with a Cool window C), the Warm range (W / 16 + 1 pages) and the
// window (H / 16 + 2 pages) share about one block per CU over all (kv head,
// sequence) pairs in proportion to their cost (a TurboQuant or Cool page
// taking about 0.8 of an fp16 page's time).
TierPlan3 plan_tiered3(int max_ctx, int hot_window, int warm_window, int cool_window, int hkv, int batch) {
    int pc = max(1, (max_ctx - hot_window - warm_window) / kPage + 1);
    if (cool_window > 0) pc = min(pc, cool_window / kPage + 1);
    const int pw = warm_window / kPage + 1, pf = hot_window / kPage + 2;
    const int S = min(max(3, (device_cus() + hkv * batch - 1) / (hkv * batch)), kMaxSplits);
    const double cc = 0.8 * pc, cw = 0.8 * pw, cf = pf, tot = cc + cw + cf;
    auto part = [&](int pages, double cost, int avail, int& n, int& pp) {
        const int n0 = min(max(1, (int)(S * cost / tot + 0.5)), max(avail, 1));
        pp = min(max((pages + n0 - 1) / n0, 1), kPagesPerSplitMax);
        n = (pages + pp - 1) / pp;
    };
    TierPlan3 p;
    part(pc, cc, S - 2, p.nc, p.ppc);
    part(pw, cw, S - p.nc - 1, p.nw, p.ppw);
    part(pf, cf, S - p.nc - p.nw, p.nf, p.ppf);
    return p;
}

hipError_t attn_tiered3_launch(const AttnArgs& a, hipStream_t st) {
    if (!a.cool_table || !a.kcc || !a.vcc || !a.kcn || !a.vcn || a.warm_window % kPage || a.cool_window < 0 ||
        a.cool_window % kPage)
        return hipErrorInvalidValue;
    const TierPlan3 p = plan_tiered3(a.max_ctx, a.hot_window, a.warm_window, a.cool_window, a.hkv, a.batch);
    if (p.nc + p.nw + p.nf > kMaxSplits) return hipErrorInvalidValue;
    const dim3 grid(p.nc + p.nw + p.nf + 4 * kCompressParts, a.hkv, a.batch);
    const int G = a.hq / a.hkv;
    const bool pc = p.ppc > kPagesPerSplitMin, pw = p.ppw > kPagesPerSplitMin, pf = p.ppf > kPagesPerSplitMin;
#define NX_TIER3_CASE(GG, PC, PW, PF)                                                                     \
    if (G == GG && pc == PC && pw == PW && pf == PF) {                                                    \
        hipLaunchKernelGGL((k_attn_tiered3<GG, PC, PW, PF>), grid, dim3(kAttnThreads), 0, st, a, p);      \
        return hipGetLastError();                                                                         \
    }
#define NX_TIER3_PW(GG, PC, PW) NX_TIER3_CASE(GG, PC, PW, true) NX_TIER3_CASE(GG, PC, PW, false)
#define NX_TIER3_PC(GG, PC) NX_TIER3_PW(GG, PC, true) NX_TIER3_PW(GG, PC, false)
#define NX_TIER3_G(GG) NX_TIER3_PC(GG, true) NX_TIER3_PC(GG, false)
    NX_TIER3_G(1)
    NX_TIER3_G(2)
    NX_TIER3_G(4)
    NX_TIER3_G(8)
#undef NX_TIER3_G
#undef NX_TIER3_PC
#undef NX_TIER3_PW
#undef NX_TIER3_CASE
    return hipErrorInvalidValue;
}

hipError_t attn_tiered_launch(const AttnArgs& a, hipStream_t st) {
    if (!a.counts || !a.part || a.hd != 128 || a.hot_window < kPage) return hipErrorInvalidValue;
    if (a.warm_window > 0) return attn_tiered3_launch(a, st);
    const TierPlan p = plan_tiered(a.max_ctx, a.hot_window, a.hkv, a.batch);
    if (p.ntq + p.nf > kMaxSplits) return hipErrorInvalidValue;
    const dim3 grid(p.ntq + p.nf + 2 * kCompressParts, a.hkv, a.batch);
    const int G = a.hq / a.hkv;
    const bool pt = p.ppt > kPagesPerSplitMin, pf = p.ppf > kPagesPerSplitMin;
#define NX_TIER_CASE(GG, PT, PF)                                                                  \
    if (G == GG && pt == PT && pf == PF) {                                                        \
        hipLaunchKernelGGL((k_attn_tiered<GG, PT, PF>), grid, dim3(kAttnThreads), 0, st, a, p.ntq, \
                           p.ppt, p.nf, p.ppf);                                                   \
        return hipGetLastError();                                                                 \
    }
#define NX_TIER_G(GG)               \
    NX_TIER_CASE(GG, true, true)    \
    NX_TIER_CASE(GG, true, false)   \
    NX_TIER_CASE(GG, false, true)   \
    NX_TIER_CASE(GG, false, false)
    NX_TIER_G(1)
    NX_TIER_G(2)
    NX_TIER_G(4)
    NX_TIER_G(8)
#undef NX_TIER_G
#undef NX_TIER_CASE
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
                                hipStream_t st, int p0) {
    (void)b4;
    (void)b3;
    const int nvec = (ctx - p0) * hkv;
    if (nvec <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_tq_encode_ctx, dim3((nvec + 3) / 4), dim3(256), 0, st, x, ctx, hkv, signs,
                       c4, c3, norms, block_table, max_blocks, b, p0);
    return hipGetLastError();
}

hipError_t cool_encode_ctx_launch(const float* x, int p0, int n, int hkv, const float* signs, uint8_t* cc,
                                  uint16_t* cn, const int32_t* cool_table, int max_blocks, int b, hipStream_t st) {
    const int nvec = (n - p0) * hkv;
    if (nvec <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_cool_encode_ctx, dim3((nvec + 3) / 4), dim3(256), 0, st, x, p0, n, hkv, signs, cc, cn,
                       cool_table, max_blocks, b);
    return hipGetLastError();
}

hipError_t tq_encode_rows_launch(const float* kvrows, int n, int p0, int hkv, const float* ksign, const float* vsign,
                                 uint8_t* kc4, uint8_t* kc3, uint16_t* kn, uint8_t* vc4, uint8_t* vc3, uint16_t* vn,
                                 const int32_t* bt, hipStream_t st) {
    const int nvec = n * 2 * hkv;
    if (nvec <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_tq_encode_rows, dim3((nvec + 3) / 4), dim3(256), 0, st, kvrows, n, p0, hkv, ksign, vsign, kc4,
                       kc3, kn, vc4, vc3, vn, bt);
    return hipGetLastError();
}

hipError_t tq_decode_pages_launch(const uint8_t* kc4, const uint8_t* kc3, const uint16_t* kn, const uint8_t* vc4,
                                  const uint8_t* vc3, const uint16_t* vn, const float* ksign, const float* vsign,
                                  const int32_t* bt, int npos, int hkv, uint16_t* kpool, uint16_t* vpool,
                                  uint16_t* klo, hipStream_t st) {
    const int nvec = npos * 2 * hkv;
    if (nvec <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_tq_decode_pages, dim3((nvec + 3) / 4), dim3(256), 0, st, kc4, kc3, kn, vc4, vc3, vn, ksign,
                       vsign, bt, npos, hkv, kpool, vpool, klo);
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
