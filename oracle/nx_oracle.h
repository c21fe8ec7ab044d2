/*
 * CPU oracle for the NEXUS per-token decode loop.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP
 * implementation is compared against, and the timed CPU baseline.  Only the
 * test suite, the smoke check and the CPU-baseline leg of the benchmark may
 * load it.  The product (libnexus_hip.so) never links or calls it.
 *
 * Every function restates the reference algorithm it cites (paths are
 * relative to the reference repository root, nexus/src/...).  Where the
 * reference has no consistent semantics (see the notes per function) the
 * build's own definition is stated here and mirrored bit for bit by the HIP
 * kernels where bit-exactness is required (int4 codes, TurboQuant codes).
 *
 * Floating point: compiled with -ffp-contract=off and without -ffast-math,
 * so every expression rounds exactly as written.  Where an FMA is part of a
 * definition it is written as fmaf().
 */
#ifndef NX_ORACLE_H
#define NX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ RNG -- */
/* Counter-based generator keyed by (seed, tensor id, element index).
 * stream = fmix(fmix(seed + G1) + tensor * G2); r = fmix(stream + (index+1)*G1)
 * with the splitmix64 finalizer fmix.  Identical on host and device. */
uint64_t nxo_rand_u64(uint64_t seed, uint32_t tensor, uint64_t index);
/* Approximately normal sample: s = sum of the four 16-bit fields of r,
 * value = float(2*s - 262140) * k, where k = nxo_normal_k(sigma) is the float
 * nearest sigma / (2*sqrt((65536^2-1)/3)).  Mean 0, standard deviation sigma
 * (Irwin-Hall with 4 terms); a single correctly rounded multiply, so host and
 * device agree bit for bit. */
float nxo_normal_k(double sigma);
float nxo_normal_from_u64(uint64_t r, float k);
void nxo_gen_normal(float* out, size_t n, uint64_t seed, uint32_t tensor, float k);
void nxo_gen_tokens(int32_t* out, int n, uint64_t seed, uint32_t tensor, int vocab);
/* Fisher-Yates permutation of 0..n-1: for i=n-1..1, j = rand(i) % (i+1). */
void nxo_shuffle_perm(int32_t* perm, int n, uint64_t seed, uint32_t tensor);

/* ---------------------------------------------------------------- fp16 -- */
uint16_t nxo_f32_to_f16(float f);        /* IEEE round-to-nearest-even */
float nxo_f16_to_f32(uint16_t h);        /* exact, subnormals kept */
/* Truncating conversion of the reference's flat fp16 KV cache
 * (model/hybrid_model.h:123-131): mantissa truncated, exponent underflow -> +-0. */
uint16_t nxo_f32_to_f16_trunc(float f);
float nxo_f16_to_f32_ref(uint16_t h);    /* model/hybrid_model.h:132-140 (subnormals -> 0) */
void nxo_f32_to_f16_array(const float* in, uint16_t* out, size_t n);
void nxo_f16_to_f32_array(const uint16_t* in, float* out, size_t n);

/* ---------------------------------------------------------- int4 g32 ---- */
/* Storage: codes [N][Kp/2] bytes, Kp = ceil(K/32)*32, low nibble = even k
 * (quant/gptq.cpp:18-24); scales fp16 [N][G], G = Kp/32.  Symmetric:
 * value = (q - 8) * scale, i.e. the reference (q - zero) * scale with zero=8
 * (quant/gptq.cpp:19).  Quantizer (the build's own; the reference quant_int4
 * at quant/gptq.cpp:37-70 is asymmetric min/max): s = fp16(amax/7);
 * q = clamp(roundf(w / float(s)), -8, 7) + 8; s == 0 -> all q = 8.
 * Columns k >= K of a ragged last group hold q = 8. */
void nxo_quantize_int4_g32(const float* w, int N, int K, uint8_t* codes, uint16_t* scales);
/* Rows [n0, n0+count) of the synthetic matrix W[N][K] ~ normal(sigma) of
 * stream (seed, tensor), element (n, k) at index n*K + k, quantized as above
 * into codes [count][G*16] / scales [count][G]. */
void nxo_gen_quant_rows(int n0, int count, int K, uint64_t seed, uint32_t tensor, double sigma,
                        uint8_t* codes, uint16_t* scales);
/* Unpack n codes (n even) from packed bytes, low nibble first (quant/gptq.cpp:12-25). */
void nxo_unpack_int4(const uint8_t* packed, size_t n, uint8_t* codes);
/* Dequantize [N][K] (gptq.cpp:9-27 with zero = 8, per-row groups along K as in
 * compute/cpu/dequant_neon.cpp:172-272). */
void nxo_dequant_int4_g32(const uint8_t* codes, const uint16_t* scales, int N, int K, float* w);
/* y[b][n] = sum_g s[n][g] * sum_{k in g} (q[n][k]-8) * x[b][k]   (fp32, OpenMP over rows)
 * Follows the grouped form of compute/cpu/dequant_neon.cpp:249-259. */
void nxo_gemv_int4_g32(const uint8_t* codes, const uint16_t* scales, const float* x,
                       int N, int K, int B, float* y);

/* ------------------------------------------------------- elementwise ---- */
/* compute/accelerate/gemm.cpp:96-114: inv = 1/sqrt(sum(x^2)/d + eps); out = x*inv*w */
void nxo_rmsnorm(const float* x, const float* w, int d, float eps, float* out);
/* RoPE, absent in the reference (model/transformer.cpp:255 "TODO").  Build's
 * definition: interleaved pairs (x[2i], x[2i+1]) of each head, angle =
 * pos * theta^(-2i/hd) evaluated in double, cos/sin rounded to float;
 * (a,b) -> (a*c - b*s, a*s + b*c). */
void nxo_rope_table(int max_pos, int hd, double theta, float* cos_tab, float* sin_tab);
void nxo_rope(float* x, int n_heads, int hd, int pos, const float* cos_tab, const float* sin_tab);
/* The Q/K norm of model/hybrid_model.cpp:1325-1349: every hd-long slice of
 * x[n_heads * hd] through nxo_rmsnorm with the same hd weights (NULL = 1.0),
 * in place. */
void nxo_head_rmsnorm(float* x, int n_heads, int hd, const float* w, float eps);
/* model/hybrid_model.cpp:1627-1630: out = g / (1 + expf(-g)) * u */
void nxo_swiglu(const float* g, const float* u, int n, float* out);
/* model/hybrid_model.cpp:2027-2038: first maximum wins (strict >). */
int nxo_argmax(const float* v, int n);

/* ----------------------------------------------------- paged attention -- */
/* Page pools fp16: K [num_blocks][hkv][16][hd] (token-major), V
 * [num_blocks][hkv][hd][16] (dimension-major, the layout the matrix-core
 * attention reads); block_table [B][max_blocks]; position p of sequence b
 * lives in block block_table[b][p/16], slot p%16 (the gather of
 * kv/paged_attention.cpp:161-230 with 16-token pages).
 * Attention follows model/hybrid_model.cpp:1493-1550: scores q.k * 1/sqrt(hd),
 * max-subtracted expf softmax divided by the sum, then the V weighted sum;
 * GQA maps query head h to kv head h / (hq/hkv) (:1471, :1502). */
#define NXO_PAGE 16
void nxo_kv_append_f16(const float* k, const float* v, uint16_t* kpool, uint16_t* vpool,
                       const int32_t* block_table, int max_blocks, int b, int pos,
                       int hkv, int hd);
void nxo_attn_decode_paged_f16(const float* q, const uint16_t* kpool, const uint16_t* vpool,
                               const int32_t* block_table, int max_blocks,
                               const int32_t* ctx_lens, int B, int hq, int hkv, int hd,
                               float* out);
/* Contiguous attention over [ctx][hkv][hd] fp32 K/V (the gather target). */
void nxo_attn_decode_contig(const float* q, const float* K, const float* V, int ctx,
                            int hq, int hkv, int hd, float* out);

/* ----------------------------------------------------------- TurboQuant -- */
/* Lloyd-Max codebook for N(0, 1/d): kv/turbo_quant.cpp:172-219 restated in
 * the same float arithmetic (init uniform in +-3 sigma, 100 iterations, tails
 * +-10 sigma, tol 1e-7 sigma). */
void nxo_tq_codebook(int d, int bits, float* centroids, float* boundaries);
/* code = first j with x < boundaries[j], else n-1 (kv/turbo_quant.cpp:19-32). */
uint8_t nxo_tq_encode_scalar(float x, const float* boundaries, int n_centroids);
/* LSB-first bit packing (kv/turbo_quant.cpp:249-268) and its inverse (:270-285). */
void nxo_pack_codes(uint8_t* packed, const uint8_t* codes, int n_codes, int bits);
void nxo_unpack_codes(uint8_t* codes, const uint8_t* packed, int n_codes, int bits);
/* Build's TurboQuant vector format (d = 128):
 *   n = sqrt(ss) with ss the canonical tree sum of x_i*x_i (products rounded,
 *   then w_i = v_i + v_{i+64}, then for s = 32..1: w_i = w_i + w_{i+s});
 *   u_i = (sign_i * x_i) * (1/n)  (u = 0 when n <= 1e-12);
 *   in-place FWHT, butterflies (a+b, a-b) for h = 1,2,..,64;
 *   y_i = u_i * float(1/sqrt(128));
 *   codes: coordinates 0..63 use the 16-level codebook, 64..127 the 8-level one;
 *   codes4 = 64 x 4 bits LSB-first (32 B), codes3 = 64 x 3 bits LSB-first (24 B),
 *   norm = fp16(n).  58 bytes per vector.
 * signs: 128 floats of +-1. */
#define NXO_TQ_D 128
void nxo_tq_signs(float* signs, uint64_t seed, uint32_t tensor);
float nxo_tq_sumsq(const float* x);
void nxo_fwht128(float* u);
void nxo_tq_encode(const float* x, int n, const float* signs, const float* b4, const float* b3,
                   uint8_t* codes4, uint8_t* codes3, uint16_t* norms, uint8_t* codes_unpacked);
/* x_hat = n * D * H(c[code]) / sqrt(128)  (inverse of the rotation above). */
void nxo_tq_decode(const uint8_t* codes4, const uint8_t* codes3, const uint16_t* norms, int n,
                   const float* signs, const float* c4, const float* c3, float* out);
/* Cool vector format, the reference's Cool quantizer (TurboQuantKV(head_dim,
 * 3, 42), kv/paged_attention.cpp:31-32: 3-bit codes on every coordinate) in
 * the build's rotation and norm: y as above, every coordinate coded with the
 * 8-level codebook; codes = 128 x 3 bits LSB-first (48 B; coordinates 0..63
 * fill bytes 0..23), norm = fp16(n).  50 bytes per vector. */
#define NXO_COOL_CODES 48
void nxo_cool_encode(const float* x, int n, const float* signs, const float* b3, uint8_t* codes,
                     uint16_t* norms);
void nxo_cool_decode(const uint8_t* codes, const uint16_t* norms, int n, const float* signs, const float* c3,
                     float* out);
/* Warm -> Cool, the step of compress_tier (kv/paged_attention.cpp:262-285):
 * the TurboQuant vector decoded to fp32 (nxo_tq_decode), then encoded Cool. */
void nxo_tq_to_cool(const uint8_t* codes4, const uint8_t* codes3, const uint16_t* norms, int n, const float* signs,
                    const float* c4, const float* c3, const float* b3, uint8_t* cool, uint16_t* cool_norms);
/* TQ page pool: codes4 [blocks][hkv][16][32], codes3 [blocks][hkv][16][24],
 * norms [blocks][hkv][16] fp16. */
void nxo_tq_append(const float* k, const float* v, int hkv,
                   const float* ksigns, const float* vsigns,
                   const float* b4, const float* b3,
                   uint8_t* kc4, uint8_t* kc3, uint16_t* kn,
                   uint8_t* vc4, uint8_t* vc3, uint16_t* vn,
                   const int32_t* block_table, int max_blocks, int b, int pos);
/* Dequantize every context vector, then the attention above. */
void nxo_attn_decode_paged_tq(const float* q,
                              const uint8_t* kc4, const uint8_t* kc3, const uint16_t* kn,
                              const uint8_t* vc4, const uint8_t* vc3, const uint16_t* vn,
                              const float* ksigns, const float* vsigns,
                              const float* c4, const float* c3,
                              const int32_t* block_table, int max_blocks,
                              const int32_t* ctx_lens, int B, int hq, int hkv, float* out);
/* Tiered pages (kv_kind 2), after the reference's PagedKVCache
 * (kv/paged_attention.cpp): positions are written as fp16 (Hot,
 * insert_kv :81-128) and a page is compressed to TurboQuant once it lies
 * wholly outside the window of the last hot_window positions (the Hot ->
 * Warm step of compress_tier :244-291, run per page as it leaves the
 * window).  The restatement keeps both forms of every position: append
 * writes the fp16 page and the TurboQuant codes of the fp16 values (the
 * codes a later compression of that page produces), and attention reads
 * position t < cold from the codes, t >= cold from fp16, in one softmax
 * (the mixed-tier gather of get_vectors :161-230).  cold = 16 floor((ctx -
 * 1 - hot_window) / 16) clamped at 0: the pages compressed before the step
 * that attends over ctx positions (a page is compressed by the step whose
 * position completes it outside the window, after that step's attention). */
void nxo_tiered_append(const float* k, const float* v, int hkv, const float* ksigns, const float* vsigns,
                       const float* b4, const float* b3, uint16_t* kpool, uint16_t* vpool, uint8_t* kc4,
                       uint8_t* kc3, uint16_t* kn, uint8_t* vc4, uint8_t* vc3, uint16_t* vn,
                       const int32_t* block_table, int max_blocks, int b, int pos);
int nxo_tiered_cold(int ctx, int hot_window);
/* Three tiers (warm_window > 0): pages also leave the Warm range [cool,
 * cold) once they lie wholly outside the last hot_window + warm_window
 * positions, and are then read in the Cool form, the Warm codes decoded and
 * encoded Cool (the Warm -> Cool step of compress_tier, per page).  cool =
 * nxo_tiered_cold(ctx, hot_window + warm_window), 0 when warm_window is 0.
 * append_cool writes the Cool form of position pos from its Warm codes
 * (pools [blocks][hkv][16][48] and [blocks][hkv][16] fp16 norms); the
 * attention reads t < cool Cool, cool <= t < cold Warm, the rest fp16. */
int nxo_tiered_cool(int ctx, int hot_window, int warm_window);
/* Cold (evicted) pages, after evict_cold_pages (kv/paged_attention.cpp:
 * 295-310): with warm_window and cool_window > 0, pages wholly outside the
 * last hot_window + warm_window + cool_window positions are dropped, and
 * get_vectors gathers zero vectors for them (:172, :219), so attention
 * scores them 0 with value 0 in its softmax.  evict = nxo_tiered_cold(ctx,
 * hot_window + warm_window + cool_window), 0 when either window is 0. */
int nxo_tiered_evict(int ctx, int hot_window, int warm_window, int cool_window);
void nxo_tiered_append_cool(int hkv, const float* ksigns, const float* vsigns, const float* c4, const float* c3,
                            const float* b3, const uint8_t* kc4, const uint8_t* kc3, const uint16_t* kn,
                            const uint8_t* vc4, const uint8_t* vc3, const uint16_t* vn, uint8_t* kcc,
                            uint16_t* kcn, uint8_t* vcc, uint16_t* vcn, const int32_t* block_table, int max_blocks,
                            int b, int pos);
void nxo_attn_decode_tiered_cool(const float* q, const uint16_t* kpool, const uint16_t* vpool, const uint8_t* kc4,
                                 const uint8_t* kc3, const uint16_t* kn, const uint8_t* vc4, const uint8_t* vc3,
                                 const uint16_t* vn, const uint8_t* kcc, const uint16_t* kcn, const uint8_t* vcc,
                                 const uint16_t* vcn, const float* ksigns, const float* vsigns, const float* c4,
                                 const float* c3, const int32_t* block_table, int max_blocks, const int32_t* ctx_lens,
                                 int hot_window, int warm_window, int B, int hq, int hkv, float* out);
/* As above with positions t < evict (nxo_tiered_evict) read as zero K and V. */
void nxo_attn_decode_tiered_evict(const float* q, const uint16_t* kpool, const uint16_t* vpool, const uint8_t* kc4,
                                  const uint8_t* kc3, const uint16_t* kn, const uint8_t* vc4, const uint8_t* vc3,
                                  const uint16_t* vn, const uint8_t* kcc, const uint16_t* kcn, const uint8_t* vcc,
                                  const uint16_t* vcn, const float* ksigns, const float* vsigns, const float* c4,
                                  const float* c3, const int32_t* block_table, int max_blocks,
                                  const int32_t* ctx_lens, int hot_window, int warm_window, int cool_window, int B,
                                  int hq, int hkv, float* out);
void nxo_attn_decode_tiered(const float* q, const uint16_t* kpool, const uint16_t* vpool, const uint8_t* kc4,
                            const uint8_t* kc3, const uint16_t* kn, const uint8_t* vc4, const uint8_t* vc3,
                            const uint16_t* vn, const float* ksigns, const float* vsigns, const float* c4,
                            const float* c3, const int32_t* block_table, int max_blocks, const int32_t* ctx_lens,
                            int hot_window, int B, int hq, int hkv, float* out);

/* ------------------------------------------------------------------ MoE -- */
/* model/hybrid_model.cpp:1662-1694: softmax over E (max-subtract, expf,
 * divide by sum), top-k by probability (ties: lower expert id first),
 * renormalize over the selected experts. */
void nxo_moe_route(const float* logits, int E, int k, int32_t* ids, float* weights);

/* ---------------------------------------------------------------- model -- */
/* Llama-style decoder with the build's synthetic weights (all projections
 * int4-g32, norm weights 1.0, embedding fp16), standard-mode semantics:
 * the sampled token is embedded for the next step (unlike the reference's
 * decode_step, model/hybrid_model.cpp:695-750, which re-runs the last
 * hidden state), RoPE applied, fp16 paged KV with round-to-nearest-even.
 * Layer order follows model/hybrid_model.cpp:1257-1425.
 * GEMV inputs are rounded to fp16; residual stream, q/k/v fp32. */
typedef struct {
    int n_layers, d_model, n_heads, n_kv_heads, head_dim, ffn, vocab;
    int n_experts, top_k;          /* n_experts == 0: dense SwiGLU FFN */
    int max_seq;                   /* per sequence, multiple of 16 */
    int batch;                     /* sequences */
    int kv_kind;                   /* 0 = fp16 pages, 1 = TurboQuant pages, 2 = tiered:
                                      the last hot_window positions (and the partly
                                      filled page) fp16, older pages TurboQuant */
    float rope_theta;
    float eps;
    uint64_t seed;
    float norm_sigma;              /* RMSNorm weights: 0 = 1.0, else 1 + N(0, norm_sigma) */
    int hot_window;                /* kv_kind 2: tokens kept fp16, a multiple of 16 */
    int warm_window;               /* kv_kind 2: 0 = two tiers; else the positions before the
                                      fp16 window kept Warm (a multiple of 16), older pages Cool */
    int cool_window;               /* kv_kind 2 with warm_window: 0 = keep every Cool page; else
                                      the positions kept Cool (a multiple of 16), older pages evicted */
    int kv_blocks;                 /* the GPU runner's shared page pool; which physical page holds a
                                      position changes no result, so the restatement ignores it */
    int qk_norm;                   /* 1: per-head RMSNorm of q and k after the projection, before
                                      RoPE, with head_dim-long weights per layer (attn_q_norm /
                                      attn_k_norm, model/hybrid_model.cpp:1325-1349) */
} nxo_cfg;

typedef struct nxo_model nxo_model;
nxo_model* nxo_model_create(const nxo_cfg* cfg);
void nxo_model_free(nxo_model* m);
/* Run one token per sequence through every layer at the sequence's current
 * position; logits [B][V] out; positions advance by one. */
void nxo_model_forward(nxo_model* m, const int32_t* tokens, float* logits);
/* Greedy generation of one sequence batch: prompt [B][P] is run token by
 * token, then n_new tokens are produced ([B][n_new]); margins [B][n_new]
 * (top1 - top2 logit) optional. */
void nxo_model_generate(nxo_model* m, const int32_t* prompt, int P, int n_new,
                        int32_t* out_tokens, float* margins);
/* Fill positions [0, ctx) of every layer's KV for every sequence with
 * synthetic N(0,1) values (outlier channels x10 when n_outlier > 0), in the
 * cache's format; positions become ctx. */
void nxo_model_fill_context(nxo_model* m, int ctx, int n_outlier);
int nxo_model_position(const nxo_model* m, int b);
/* Accessors used by the tests (host copies of the model's tensors). */
const int32_t* nxo_model_block_table(const nxo_model* m);
/* The stored form of position pos (all kv heads) of layer `layer`, K (kv 0)
 * or V (kv 1): form 0 = fp16 [hkv][hd], form 1 = TurboQuant [hkv] x (32 B
 * 4-bit codes, 24 B 3-bit codes, fp16 norm), form 2 = Cool [hkv] x (48 B
 * 3-bit codes, fp16 norm); the model must hold that form
 * (tiered models hold both).  Returns the bytes written, 0 if absent. */
int nxo_model_kv_read(const nxo_model* m, int layer, int b, int pos, int kv, int form, uint8_t* out);
int nxo_model_max_blocks(const nxo_model* m);
/* Time one forward step split into layers and the lm_head (seconds). */
void nxo_model_forward_timed(nxo_model* m, const int32_t* tokens, float* logits,
                             double* t_layers, double* t_head);
int nxo_num_threads(void);
void nxo_set_num_threads(int n);

/* ------------------------------------------------------------ sampling -- */
/* MT19937 (Matsumoto & Nishimura, the generator of std::mt19937): the first
 * n 32-bit outputs after seeding with `seed` (the standard's seeding rule). */
void nxo_mt19937(uint32_t seed, int n, uint32_t* out);
/* std::uniform_real_distribution<float>(0, 1) applied to one 32-bit
 * generator output x, as libstdc++ computes it (generate_canonical<float,24>
 * with k = 1): float(x) / 2^32, values reaching 1 replaced by the largest
 * float below 1. */
float nxo_canonical_f32(uint32_t x);
/* HybridModel::Impl::sample_token (model/hybrid_model.cpp:2023-2099) with the
 * draw given as u in [0, 1) (the reference draws u from a fresh
 * std::mt19937(seed) at every call): temperature <= 0 -> first maximum;
 * else fp32 softmax of logits / T (sequential sums), top-k (top_k in
 * (0, V)), top-p (top_p < 1: kept in descending order until the running
 * sum exceeds top_p, that element included), renormalize, r = u * sum, and
 * the first index whose running sum (index order) reaches r (V - 1 if
 * none).  Ties in the sorts keep the lower index first (the reference's
 * partial_sort / sort order for ties is unspecified). */
int nxo_sample(const float* logits, int V, float temperature, int top_k, float top_p, float u);

/* ------------------------------------------------------------ NXF -- */
/* XXH32 of a byte range (the published xxHash 32-bit algorithm): the chunk
 * checksum of NXF files, format/nxf_writer.cpp:33-72 (stored by
 * NXFWriter::add_chunk, :255) and format/nxf_reader.cpp:32-71. */
uint32_t nxo_xxh32(const void* data, size_t len, uint32_t seed);

/* Tensor ids of the synthetic model (shared with the device generator). */
#define NXO_TID_EMBED        1u
#define NXO_TID_LMHEAD       2u
#define NXO_TID_PROMPT       4u
#define NXO_TID_PAGE_SHUFFLE 7u
#define NXO_TID_FINAL_NORM   3u
#define NXO_TID_LAYER(L, kind) (0x100u * ((uint32_t)(L) + 1u) + (uint32_t)(kind))
enum { NXO_W_Q = 0, NXO_W_K = 1, NXO_W_V = 2, NXO_W_O = 3, NXO_W_GATE = 4, NXO_W_UP = 5,
       NXO_W_DOWN = 6, NXO_W_ROUTER = 7, NXO_TQ_KSIGN = 8, NXO_TQ_VSIGN = 9, NXO_N_ATTN = 10,
       NXO_N_FFN = 11, NXO_N_QNORM = 12, NXO_N_KNORM = 13 };
/* expert e of layer L: NXO_TID_EXPERT(L, e, 0=gate,1=up,2=down) */
#define NXO_TID_EXPERT(L, e, w) (0x01000000u + 0x1000u * (uint32_t)(L) + 4u * (uint32_t)(e) + (uint32_t)(w))
/* synthetic context of sequence b, layer L, kv = 0 (K) / 1 (V) */
#define NXO_TID_CTX(L, b, kv) (0x10000000u + 0x10000u * (uint32_t)(L) + 2u * (uint32_t)(b) + (uint32_t)(kv))

#ifdef __cplusplus
}
#endif
#endif
