// Host-side launchers of the gfx950 decode kernels.  All pointers are
// device pointers; every launcher enqueues on `st` and returns the launch
// status.  Shapes are validated by the callers (the C-ABI layer and the
// runner) before any launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nx {

// ----------------------------------------------------------------- GEMV --
// Where the GEMV input x comes from.
enum XSrc : int {
    X_F16 = 0,      // x fp16 [batch][K] (row stride ldx elements)
    X_RMSNORM = 1,  // x = fp16((h * 1/sqrt(mean(h^2)+eps)) * w), h fp32 [batch][K]
};
// What the GEMV does with each output row.
enum Epi : int {
    E_F16 = 0,      // y16[b][n] = y
    E_F32 = 1,      // y32[b][n] = y
    E_ACC = 2,      // y32[b][n] += y   (residual add)
    E_QKV = 3,      // RoPE on q/k rows (none without cos_t); q -> q32; k,v -> fp16 pages (or fp32 kv_tmp)
    E_SWIGLU = 4,   // rows (2j, 2j+1) = (gate j, up j) -> act16[b][j] = fp16(silu(g)*u)
    E_LOGITS = 5,   // y32[b][n] = y and running argmax into best[b]
    E_PART = 6,     // kpart[part][b][n] = partial sum over the block's K part
};

struct GemvArgs {
    const uint8_t* W;       // [N][G*16]
    const uint16_t* S;      // [N][G]
    int N, K, G;
    int batch;
    // input
    const uint16_t* x16;    // X_F16
    int ldx;                // elements between batch rows of x16 / h32
    const float* h32;       // X_RMSNORM
    const float* norm_w;    // X_RMSNORM (nullptr = ones)
    float eps;
    // outputs
    uint16_t* y16;
    float* y32;
    int ldy;                // elements between batch rows of y
    // E_QKV
    float* q32;             // [batch][qdim]
    int qdim, kvdim, hd, hkv;
    const int32_t* pos;     // [batch] position of the token being processed
    const float* cos_t;     // [max_pos][hd/2]; nullptr: no RoPE (the projection alone)
    const float* sin_t;
    uint16_t* kpool;        // fp16 pages (kv_kind 0)
    uint16_t* vpool;
    float* kv_tmp;          // [batch][2][kvdim] fp32 (kv_kind 1)
    const int32_t* block_table;
    int max_blocks;
    // E_SWIGLU
    uint16_t* act16;        // [batch][lda]
    int lda;
    // E_LOGITS
    unsigned long long* best;  // [batch] packed (ordered value, ~index)
    // Routed experts (launched through moe_gate_up_launch / moe_down_launch):
    // grid row y takes the active expert of moe_plan + y * kMoePlanInts; its
    // weights are at W + e * moe_wstride and S + e * moe_sstride, and batch
    // row i reads x row (moe_xslot ? slot i : token i) and writes output row
    // slot i.
    const int32_t* moe_plan;
    size_t moe_wstride, moe_sstride;
    int moe_xslot;
    // Batch 2..8 with fp16 x and K beyond 4096 (the down projection): K is
    // split over gemv_kparts(K) groups of blocks, which write partial sums
    // [part][batch][N] here; a second launch adds them in part order and
    // runs the epilogue.  nullptr: one launch streams all of K per block.
    float* kpart;
    int kparts;      // set by the launcher
    int kpart_rows;  // rows of one part: batch, or batch * k slots for routed experts
    // Optional (E_ACC / E_F32, ldy == N): also write post_x16 [batch][N] =
    // fp16(RMSNorm(y32 row) * post_norm_w) of the rows just written, the
    // input of the next RMSNorm-input GEMV.  The K-split path does it in its
    // part-sum launch; the others in a launch of their own.
    const float* post_norm_w;  // nullptr = ones
    uint16_t* post_x16;
    float post_eps;
    // > 0: K parts of the batch 2..8 split (instead of gemv_kparts(K)),
    // when kpart holds want_kparts * batch * N floats
    int want_kparts;
};

// Parts of a K-split batch-2..8 GEMV (0: none); the workspace is
// gemv_kparts(K) * batch * N floats.
inline int gemv_kparts(int K, int batch) { return batch >= 2 && K > 4096 && K % 32 == 0 ? (K + 4095) / 4096 : 0; }
// The parts a batch 2..8 GEMV with want_kparts = want splits K into (a part
// stages at most 4096 k in LDS); its workspace is that many * batch * N floats.
inline int gemv_parts_for(int K, int batch, int want) {
    const int base = gemv_kparts(K, batch);
    return want > 0 && batch >= 2 && K % 32 == 0 ? (want > base ? want : base) : base;
}

// Routing plan of one active expert (int32 words): [0] expert id (-1: no
// expert for this grid row), [1] its number of token slots n (<= 8),
// [8 + i] slot i (= b * k + j), [16 + i] token b of slot i, for i < n.
constexpr int kMoePlanInts = 32;
constexpr int kMoePlanMaxSlots = 8;
// Routing limits: experts per layer, experts per token (the reference's
// default is 10 when the manifest names none, hybrid_model.cpp:1648), and
// sequences per step.
constexpr int kMoeMaxExperts = 256;
constexpr int kMoeMaxTopK = 16;
constexpr int kMoeMaxBatch = 8;
// Plan rows a step needs: the most experts that can be active at once.
__host__ __device__ inline int moe_plan_rows(int E, int batch, int k) { return E < batch * k ? E : batch * k; }

hipError_t gemv_launch(int xsrc, int epi, const GemvArgs& a, hipStream_t st);

// ------------------------------------------------------------ attention --
struct AttnArgs {
    const float* q;            // [batch][hq][hd]
    const uint16_t* kpool;     // fp16 pages
    const uint16_t* vpool;
    const uint16_t* kpool_lo;  // prefill over decoded TurboQuant pages: K - fp16(K), or nullptr
    // prefill over tiered pages: fp16 pages (through block_table) of the
    // positions from the first query tile's cold boundary on; a tile of 16
    // queries (page-aligned positions) reads the pages before its cold
    // boundary (16 floor((position - hot_window) / 16), clamped at 0) from
    // kpool / vpool / kpool_lo (the decoded TurboQuant pages) and the rest
    // from these, with K lo read from lo_zero (one page of zeros)
    const uint16_t *kpool_win, *vpool_win, *lo_zero;
    // TurboQuant pages (head_dim 128)
    const uint8_t *kc4, *kc3, *vc4, *vc3;
    const uint16_t *kn, *vn;
    const float *ksign, *vsign;  // [128] of +-1
    const int32_t* block_table;  // [batch][max_blocks]
    const int32_t* ctx_lens;     // [batch] (nullptr: use pos[b] + 1)
    const int32_t* pos;
    uint16_t* out16;             // [batch][hq][hd]
    int batch, hq, hkv, hd, max_blocks;
    int max_ctx;                 // upper bound of ctx_lens (sizes the split grid)
    // workspace
    float* part;                 // partial (m, l, o) per split
    // fp16 pages: split-completion counter of each (sequence, kv head) at
    // counts[(b * hkv + kvh) * kAttnCountStride]; zero before a launch, and
    // the launch leaves them at zero
    unsigned* counts;
    // tiered pages (attn_tiered_launch): positions [0, cold) are read from
    // the TurboQuant pages through block_table, [cold, ctx) from the fp16
    // pages through hot_table (entries from cold / 16 on), cold = 16
    // floor((ctx - 1 - hot_window) / 16) clamped at 0; the same launch
    // compresses the page that leaves the window at this step
    int hot_window;
    const int32_t* hot_table;
    // three tiers (warm_window > 0): positions [0, cool) are read from the
    // Cool pages through cool_table (3-bit codes on all 128 coordinates,
    // [blocks][hkv][16][48], fp16 norms [blocks][hkv][16]), [cool, cold) from
    // the TurboQuant (Warm) pages through block_table; cool = 16 floor((ctx -
    // 1 - hot_window - warm_window) / 16) clamped at 0.  The same launch
    // re-encodes the page that leaves the Warm range into the Cool pages.
    int warm_window;
    // Cold (cool_window > 0 with three tiers): positions [0, evict) are
    // evicted, evict = 16 floor((ctx - 1 - hot_window - warm_window -
    // cool_window) / 16) clamped at 0; they enter the softmax as zero keys
    // and values (score 0), and the Cool range is [evict, cool)
    int cool_window;
    const int32_t* cool_table;
    const uint8_t *kcc, *vcc;
    const uint16_t *kcn, *vcn;
    // TurboQuant pages in the decode step (attn_tq_launch): the fp32 K and V
    // of the token being written ([batch][2][hkv * 128]); the launch encodes
    // them into the pages at pos[b] and attends over them with the pages
    // before (nullptr: the pages already hold every position)
    const float* kv_cur;
    // > 0 (fp16 pages, standalone): the kernel itself checks each sequence's
    // context length against max_blocks * 16 and the block-table entries of
    // its pages against [0, check_blocks); an entry outside reads block 0
    // instead and the sequence's output rows become NaN (no host check)
    int check_blocks;
};
constexpr int kAttnCountStride = 64;  // counters 256 bytes apart
// Split records and counters of nx_attn_decode_paged_f16_noalloc: a
// file-scope device array of kNoAllocRecordBytes of records followed by
// kNoAllocCountWords counters, one copy per device.
constexpr size_t kNoAllocRecordBytes = (size_t)4 << 20;
constexpr size_t kNoAllocCountWords = 16384;
// Device address of that array on the current device (hipGetSymbolAddress).
hipError_t attn_noalloc_scratch(void** out);
// Zero n words at p (a kernel, so it may be captured into a graph).
hipError_t zero_u32_launch(unsigned* p, size_t n, hipStream_t st);
size_t attn_workspace_bytes(int batch, int hq, int hkv, int hd, int max_ctx);
// Workspace of attn_f16_launch for exactly this (batch, max_ctx): the split
// plan it launches, which has fewer splits than attn_workspace_bytes assumes
// when batch x kv heads exceeds the CU count.
size_t attn_f16_workspace_bytes(int batch, int hq, int hkv, int hd, int max_ctx);
inline size_t attn_count_words(int batch, int hkv) { return (size_t)batch * hkv * kAttnCountStride; }
// Longest context the attention kernels accept.
int attn_max_ctx();
// One launch each: the split blocks, the last of each (sequence, kv head)
// merging the records.
hipError_t attn_f16_launch(const AttnArgs& a, hipStream_t st);
hipError_t attn_tq_launch(const AttnArgs& a, hipStream_t st);
// Causal prefill attention over fp16 pages: q rows t < P ([P][hq][hd]) of
// one sequence at positions p0 + t, block_table = that sequence's row,
// out16 [P][hq][hd]; row t attends to positions <= p0 + t.  No workspace.
hipError_t attn_prefill_launch(const AttnArgs& a, int p0, int P, hipStream_t st);
// Attention over tiered pages in one launch, which also compresses the page
// leaving the window (max_ctx bounds ctx_lens) and, with three tiers
// (warm_window > 0), re-encodes Cool the page leaving the Warm range.
hipError_t attn_tiered_launch(const AttnArgs& a, hipStream_t st);
size_t attn_tiered_workspace_bytes(int batch, int hq, int hkv);
// Tiered pages: fill the window's pages from raw fp32 [ctx][hkv][hd]; round
// fp32 values through fp16.
hipError_t put_hot_launch(const float* raw, int ctx, int cold, int hkv, int hd, int b, const int32_t* hot_bt,
                          int max_blocks, uint16_t* kpool, uint16_t* vpool, int kv, hipStream_t st);
hipError_t round_f16_launch(float* x, size_t n, hipStream_t st);

// ---------------------------------------------------------------- misc --
hipError_t rmsnorm_launch(const float* x, const float* w, uint16_t* out, int dim, float eps,
                          int batch, hipStream_t st);
hipError_t rope_launch(float* x, const int32_t* pos, const float* cos_t, const float* sin_t,
                       int heads, int hd, int batch, hipStream_t st);
hipError_t swiglu_launch(const float* g, const float* u, uint16_t* out, int n, int batch,
                         hipStream_t st);
hipError_t residual_add_launch(const float* a, const float* b, float* out, int n, hipStream_t st);
// Per-head Q/K RMSNorm (hybrid_model.cpp:1325-1349) + RoPE + the paged
// write of K/V for one decode step: q [batch][hq * hd] in q32 and k, v
// [batch][2][hkv * hd] in kv_tmp hold the raw projection; every head_dim
// slice of q and k is normalized with the head_dim weights (nullptr: 1.0),
// then rotated at pos[b]; q goes back to q32, k and v to the fp16 pages at
// block_table[b][pos / 16] (kpool == nullptr: k back to kv_tmp, for the
// TurboQuant attention's append).  head_dim <= 256.
struct QknArgs {
    float* q32;
    float* kv_tmp;
    const float *qn, *kn;
    const float *cos_t, *sin_t;
    const int32_t* pos;
    const int32_t* block_table;
    int max_blocks;
    uint16_t *kpool, *vpool;
    int hq, hkv, hd;
    float eps;
};
hipError_t qk_norm_rope_launch(const QknArgs& a, int batch, hipStream_t st);
// The same normalization alone, in place, over `rows` rows: q heads at
// q + r * ldq, k heads at k + r * ldk (the batched prefill's QKV rows).
hipError_t head_rmsnorm_launch(float* q, int ldq, float* k, int ldk, int rows, int hq, int hkv, int hd,
                               const float* qn, const float* kn, float eps, hipStream_t st);
hipError_t kv_append_f16_launch(const float* k, const float* v, uint16_t* kpool, uint16_t* vpool,
                                const int32_t* block_table, const int32_t* pos, int batch,
                                int hkv, int hd, int max_blocks, hipStream_t st);
hipError_t argmax_launch(const float* logits, int32_t* out, int V, int batch, hipStream_t st);
hipError_t unpack_int4_launch(const uint8_t* packed, uint8_t* codes, size_t n, hipStream_t st);
hipError_t quantize_int4_launch(const float* w, uint8_t* codes, uint16_t* scales, int N, int K,
                                hipStream_t st);
// Synthetic weights: W[N][K] ~ normal(k) from stream (seed, tid), quantized
// int4-g32 in one pass (bit-identical to quantizing the generated floats).
// row_offset/rows_total place the matrix at row `row_offset` of a larger
// allocation with `row_stride` rows between consecutive generated rows
// (row_stride 2 interleaves gate/up).
hipError_t gen_quant_launch(uint8_t* codes, uint16_t* scales, int N, int K, uint64_t seed,
                            uint32_t tid, float k, int row_offset, int row_stride,
                            hipStream_t st);
hipError_t gen_f16_launch(uint16_t* out, size_t n, uint64_t seed, uint32_t tid, float k,
                          hipStream_t st);
// Synthetic fp16 context for layer L, positions [0, ctx) of every sequence.
hipError_t gen_ctx_f16_launch(uint16_t* kpool, uint16_t* vpool, const int32_t* block_table,
                              int max_blocks, int batch, int ctx, int hkv, int hd, int L,
                              uint64_t seed, float k, const int32_t* outlier_ch, int n_outlier,
                              hipStream_t st);
// Synthetic raw K/V fp32 [ctx][hkv][hd] of (L, b, kv) into dst (for TurboQuant encode).
hipError_t gen_ctx_raw_launch(float* dst, int ctx, int hkv, int hd, int L, int b, int kv,
                              uint64_t seed, float k, const int32_t* outlier_ch, int n_outlier,
                              hipStream_t st);

// TurboQuant: encode nvec vectors (rows of x, stride 128) into the given
// destinations; dst index of vector i is idx ? idx[i] : i.
hipError_t tq_encode_launch(const float* x, int nvec, const float* signs, const float* b4,
                            const float* b3, uint8_t* c4, uint8_t* c3, uint16_t* norms,
                            const int32_t* idx, hipStream_t st);
// Encode context rows [ctx][hkv][128] of sequence b into pages.
hipError_t tq_encode_ctx_launch(const float* x, int ctx, int hkv, const float* signs,
                                const float* b4, const float* b3, uint8_t* c4, uint8_t* c3,
                                uint16_t* norms, const int32_t* block_table, int max_blocks,
                                int b, hipStream_t st, int p0 = 0);
// Context fill of Cool pages: positions [p0, n) of x [.][hkv][128] of
// sequence b encoded TurboQuant, decoded and encoded Cool (48-byte codes,
// fp16 norms) into the pages of cool_table.
hipError_t cool_encode_ctx_launch(const float* x, int p0, int n, int hkv, const float* signs, uint8_t* cc,
                                  uint16_t* cn, const int32_t* cool_table, int max_blocks, int b, hipStream_t st);
// Append one token per sequence from kv_tmp [batch][2][hkv*128].
// Encode the K and V rows [n][2][hkv*128] of positions p0 .. p0 + n - 1 of
// one sequence (block table bt of that sequence) into its pages.
hipError_t tq_encode_rows_launch(const float* kvrows, int n, int p0, int hkv, const float* ksign, const float* vsign,
                                 uint8_t* kc4, uint8_t* kc3, uint16_t* kn, uint8_t* vc4, uint8_t* vc3, uint16_t* vn,
                                 const int32_t* bt, hipStream_t st);
// Batched prefill over tiered pages, one layer and chunk of sequence b: the
// fp16 K and V of positions [lo, pe) -- the window's ring pages (hot_bt)
// before pb, the chunk's rows kvrows [pe - pb][2][hkv*128] rounded to fp16
// from pb on -- into the fp16 pages vk / vv (block table bt), into the
// TurboQuant pages for positions below tq_hi (encoded from those fp16 values,
// as the decode step's compression encodes a page leaving the window), and
// into the ring for positions from ring_lo (>= pb) on.
hipError_t pf_tier_rows_launch(const float* kvrows, int pb, int lo, int pe, int tq_hi, int ring_lo, int hkv, int b,
                               const int32_t* bt, const int32_t* hot_bt, int max_blocks, uint16_t* ring_k,
                               uint16_t* ring_v, uint16_t* vk, uint16_t* vv, const float* ksign, const float* vsign,
                               uint8_t* kc4, uint8_t* kc3, uint16_t* kn, uint8_t* vc4, uint8_t* vc3, uint16_t* vn,
                               hipStream_t st);
// Decode positions 0 .. npos - 1 of one sequence's TurboQuant pages into fp16
// pages of the same blocks (K token-major, V dimension-major), K also as its
// fp16 remainder klo (same layout).
hipError_t tq_decode_pages_launch(const uint8_t* kc4, const uint8_t* kc3, const uint16_t* kn, const uint8_t* vc4,
                                  const uint8_t* vc3, const uint16_t* vn, const float* ksign, const float* vsign,
                                  const int32_t* bt, int npos, int hkv, uint16_t* kpool, uint16_t* vpool,
                                  uint16_t* klo, hipStream_t st);
hipError_t tq_append_launch(const float* kv_tmp, int batch, int hkv, const float* ksign,
                            const float* vsign, const float* b4, const float* b3, uint8_t* kc4,
                            uint8_t* kc3, uint16_t* kn, uint8_t* vc4, uint8_t* vc3, uint16_t* vn,
                            const int32_t* block_table, const int32_t* pos, int max_blocks,
                            hipStream_t st);
void tq_set_codebooks(const float* c4, const float* b4, const float* c3, const float* b3);

// Step start: tok[b] = token decoded from best[b]; best[b] = 0; pos[b] += 1;
// h[b] = fp32(embed[tok]).
// The token consumed at new position p is recorded at out_tokens[b][p - base[b] - 1]
// when that index is in [0, out_stride).
// feed (optional, [batch]): what each sequence slot consumes at this step --
// kFeedDecode its pending token (recorded as output), a token id >= 0 (a
// prompt token, not recorded), kFeedPark (a free slot: token 0 at position
// 0) or kFeedHold (a paused sequence: token 0 at position fpos[b], one it
// has not reached, so nothing it holds is overwritten).  Both parked and
// held slots leave pos[b] at that position, for the host to restore.
constexpr int kFeedDecode = -1, kFeedPark = -2, kFeedHold = -3;
hipError_t embed_launch(unsigned long long* best, int32_t* pos, const int32_t* base,
                        int32_t* out_tokens, int out_stride, const uint16_t* embed, float* h,
                        int d, int vocab, int batch, hipStream_t st, const int32_t* feed = nullptr,
                        const int32_t* fpos = nullptr);
// Record the pending tokens (decoded from best) at out_tokens[b][pos[b] - base[b]].
hipError_t finish_tokens_launch(const unsigned long long* best, const int32_t* pos,
                                const int32_t* base, int32_t* out_tokens, int out_stride,
                                int batch, hipStream_t st);

// Make tokens[b] the pending token of sequence b (as if sampled).
hipError_t set_tokens_launch(unsigned long long* best, const int32_t* tokens, int batch,
                             hipStream_t st);

// MoE
struct MoeArgs {
    float* logits;              // [batch][E] (read by moe_route_launch, written by moe_norm_route_launch)
    int E, k, batch;
    int32_t* ids;               // [batch][k]
    float* weights;             // [batch][k]
    int32_t* expert_count;      // [E]
    int32_t* expert_slots;      // [E][batch*k] : entries b*k + j
    int32_t* plan;              // [moe_plan_rows][kMoePlanInts] or nullptr (batch <= 8)
    // moe_norm_route_launch: the block input h fp32 [batch][d] (RMSNorm with
    // norm_w, nullptr = ones, and eps) to fp16 x16 [batch][d], and the router
    // int4-g32 rows wr [E][G*16], sr [E][G] whose products with x16 are the
    // logits it writes to `logits`
    const float* h;
    const float* norm_w;
    float eps;
    int d;
    const uint8_t* wr;
    const uint16_t* sr;
    uint16_t* xn16;
    unsigned* counter;  // one word, zero before a launch (batch > 1); the launch leaves it at zero
};
// Routing from logits [batch][E].
hipError_t moe_route_launch(const MoeArgs& a, hipStream_t st);
// RMSNorm + router GEMV + routing in one launch (shapes moe_norm_route_fits).
bool moe_norm_route_fits(int d, int E, int k, int batch);
hipError_t moe_norm_route_launch(const MoeArgs& a, hipStream_t st);
struct MoeFfnArgs {
    const uint16_t* x16;        // [batch][ldx] normed hidden (fp16)
    int ldx;
    const uint8_t* w13;         // [E][2F][d/2]
    const uint16_t* s13;        // [E][2F][d/32]
    const uint8_t* w2;          // [E][d][Fp/2]
    const uint16_t* s2;
    int d, F, E, k, batch;
    const int32_t* plan;        // [moe_plan_rows][kMoePlanInts]
    const float* weights;       // [batch][k]
    uint16_t* act16;            // [batch*k][Fp]
    float* y32;                 // [batch*k][d]
    float* out;                 // [batch][d]
    int accumulate;
    // batch >= 2: the down projection's K-part sums [gemv_kparts(F, batch)]
    // [batch*k][d], added by the combine (nullptr: y32 holds the sums)
    float* kpart;
};
// Batched prefill of MoE layers: routing of n tokens from their logits
// [n][E] (as decode routes them), token slots grouped by expert (counts:
// cnt[E] then offsets[E]; row_tok[row] = token, slot_row[t * k + j] = row);
// gathering fp16 rows; the weighted combine h[t] += sum_j w yg[row].
hipError_t pf_route_launch(const float* logits, int n, int E, int k, int32_t* ids, float* w, int32_t* row_tok,
                           int32_t* slot_row, int32_t* counts, hipStream_t st);
hipError_t pf_gather_launch(const uint16_t* x16, const int32_t* row_tok, int rows, int d, uint16_t* xg,
                            hipStream_t st);
hipError_t pf_moe_combine_launch(const float* yg, const int32_t* slot_row, const float* w, int n, int k, int d,
                                 float* h, hipStream_t st);
// Whether the routed down projection writes K-part sums (a.kpart) for the
// combine to add; decided once here for both launches.
bool moe_down_split(const MoeFfnArgs& a);
// The combine (a.out += sum_j w_j y_j, accumulate set), then the RMSNorm of
// each new row with weights w (nullptr = ones) into x16 [batch][d]: the next
// RMSNorm-input GEMV's input, with no launch of its own.
bool moe_combine_norm_fits(const MoeFfnArgs& a);
hipError_t moe_combine_norm_launch(const MoeFfnArgs& a, const float* w, uint16_t* x16, float eps, hipStream_t st);
// Batch 1 (nx_moe.hip): the routing folded into the gate/up launch (every
// block normalizes h = m.h with m.norm_w, computes the router logits and the
// routing; block (0, 0) writes ids, weights, counts, slot lists and the
// plan), and the down projection with the weighted combine into f.out (h +=
// sum_j w_j y_j, top-k 1 or 2; f.weights and ids from the gate/up launch).
bool moe_b1_fused_fits(int d, int F, int E, int k);
bool moe_b1_down_combine_fits(int F, int k);
hipError_t moe_b1_gate_up_launch(const MoeArgs& m, const MoeFfnArgs& f, hipStream_t st);
hipError_t moe_b1_down_combine_launch(const MoeFfnArgs& f, const int32_t* ids, hipStream_t st);
hipError_t moe_gate_up_launch(const MoeFfnArgs& a, hipStream_t st);
hipError_t moe_down_launch(const MoeFfnArgs& a, hipStream_t st);
hipError_t moe_combine_launch(const MoeFfnArgs& a, hipStream_t st);

// Batched prefill (nx_prefill.hip): int4-g32 GEMM Y = X W^T on the matrix
// cores, X fp16 [M][ldx] (K and ldx multiples of 8, 16-byte aligned rows).
enum { PF_F32 = 0, PF_ACC = 1, PF_SWIGLU = 2 };
struct PfGemmArgs {
    const uint16_t* x;
    int ldx;
    const uint8_t* W;    // codes [N][G*16]
    const uint16_t* S;   // fp16 scales [N][G]
    int M, N, K, G;
    float* y32;          // PF_F32: y32[m][n] = y; PF_ACC: y32[m][n] += y
    int ldy;
    uint16_t* act16;     // PF_SWIGLU: rows 2f, 2f+1 = gate f, up f -> act16[m][f]
    int lda;
};
hipError_t pf_gemm_launch(int epi, const PfGemmArgs& a, hipStream_t st);
hipError_t pf_embed_launch(const int32_t* tokens, int P, const uint16_t* embed, float* h, int d, int vocab,
                           hipStream_t st);
hipError_t pf_rope_kv_launch(const float* qkv, int ld, int P, int p0, int qdim, int kvdim, int hd, int hkv,
                             const float* cos_t, const float* sin_t, const int32_t* bt, uint16_t* kpool,
                             uint16_t* vpool, float* q32, hipStream_t st, float* kvrows = nullptr);

// Sampling (nx_sample.hip): sample_token of hybrid_model.cpp:2023-2099 per
// sequence; the draw is u_fixed when >= 0, else u[b], else a counter-based
// draw keyed by (key, sequence, pos[b]).  Writes out[b] and/or
// best[b] (the pending-token encoding read by the embedding kernel).
struct SampleArgs {
    const float* logits;  // [batch][ldl]
    int V, ldl;
    float temperature;    // > 0 (greedy is the argmax kernel)
    int top_k;            // 0 or >= V: off; otherwise at most 1024
    float top_p;          // (0, 1]; < 1 needs top-k
    float u_fixed;
    const float* u;       // [batch], or nullptr: draws keyed by (key, b, pos[b])
    uint64_t key;
    const int32_t* pos;
    int32_t* out;
    unsigned long long* best;
    float* scratch;       // [batch][V] floats
    float* part;          // [batch][kSmpPartFloats] floats
};
// Per-block partials of the sampler's first passes (max, sum, candidate
// counts of each of kSmpBlocks blocks per sequence), then the top-k
// candidates (kSmpCandMax probabilities, then as many indices).
constexpr int kSmpBlocks = 64, kSmpCandMax = 4096;
constexpr int kSmpCandOff = kSmpBlocks * 10;
constexpr int kSmpPartFloats = kSmpCandOff + 2 * kSmpCandMax;
hipError_t sample_launch(const SampleArgs& a, int batch, hipStream_t st);
// The reference's draw for a seed: std::uniform_real_distribution<float>(0, 1)
// of the first output of std::mt19937(seed) (seed 0: std::random_device).
float sample_draw(uint64_t seed);

// fp32 GEMM C[M][N] = A[M][K] B[K][N], row-major, on the matrix cores (nx_gemm.hip).
hipError_t gemm_f32_launch(const float* A, const float* B, float* C, int M, int N, int K, hipStream_t st);

// XXH32 (seed 0) of byte ranges of one device buffer: range i is
// [off, off + len) (off a multiple of 16); its hash goes to out[slot].
struct HashRange {
    uint64_t off;
    uint32_t len;
    uint32_t slot;
};
hipError_t xxh32_launch(const uint8_t* data, const HashRange* ranges, int n, uint32_t* out, hipStream_t st);

}  // namespace nx
