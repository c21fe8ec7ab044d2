/*
 * nexus_hip.h -- C-ABI of the MI355X (gfx950) decode-loop library
 * libnexus_hip.so.
 *
 * This is the drop-in boundary for the NEXUS per-token decode loop.  The
 * reference's runner calls nexus::compute::ComputeDispatch
 * (nexus/src/compute/compute_dispatch.h:22-323), which wraps MetalBackend
 * (nexus/src/compute/metal/metal_backend.h:38-228).  Each entry point below
 * names the reference member it replaces.
 *
 * Conventions (all entry points):
 *   - return nx_status: NX_OK (0) or an error code; on error nothing is
 *     zero-filled (the reference writes zeros on failure at
 *     compute_dispatch.cpp:174-175, :220-223, :273-274; this library never
 *     does) and nx_last_error() describes the failure;
 *   - buffers are opaque nx_buf handles (the reference's uint64_t buffer_id,
 *     metal_backend.h:41) owned by the context; every op checks that each
 *     buffer exists and is large enough for the shapes given;
 *   - every op is enqueued asynchronously on the context's one HIP stream, in
 *     call order; nx_synchronize() / nx_download() wait for it;
 *   - a context is single-threaded by contract, like the reference's global
 *     ComputeDispatch (compute_dispatch.cpp:18-27).
 *
 * Formats:
 *   int4-g32 weights: codes [N][Kp/2] bytes (Kp = ceil(K/32)*32), low nibble
 *     = even k; scales fp16 [N][Kp/32]; value = (q - 8) * scale.  Columns
 *     k >= K of a ragged last group hold q = 8.
 *   fp16 paged KV: K pool [num_blocks][hkv][16][head_dim] fp16 (token-major),
 *     V pool [num_blocks][hkv][head_dim][16] fp16 (dimension-major, so the
 *     attention's value product reads it as a matrix-core operand);
 *     block_table int32 [batch][max_blocks]; position p of sequence b lives
 *     in block block_table[b][p/16], slot p%16.
 *   TurboQuant paged KV (head_dim 128): codes4 [num_blocks][hkv][16][32] u8,
 *     codes3 [num_blocks][hkv][16][24] u8, norms [num_blocks][hkv][16] fp16;
 *     58 bytes per vector (see nx_tq_encode).
 */
#ifndef NEXUS_HIP_H
#define NEXUS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int nx_status;
#define NX_OK 0
#define NX_ERR_INVALID 1      /* bad argument, unknown buffer, size mismatch */
#define NX_ERR_HIP 2          /* HIP runtime error */
#define NX_ERR_OOM 3          /* device allocation failed */
#define NX_ERR_UNSUPPORTED 4  /* shape or mode this build does not implement */
#define NX_ERR_STATE 5        /* call out of order (e.g. token_end without begin) */
#define NX_ERR_NO_DEVICE 6    /* no usable gfx950 device */
#define NX_ERR_CAPACITY 7     /* sequence or cache capacity exhausted */
#define NX_ERR_TIMEOUT 8      /* reserved: a wait inside a launch timed out (no entry point waits inside a launch) */

typedef struct nx_ctx nx_ctx;
typedef uint64_t nx_buf; /* 0 = none */

/* ------------------------------------------------------------ lifecycle -- */
/* ComputeDispatch::init_gpu (compute_dispatch.h:29, compute_dispatch.cpp:47-71) */
nx_status nx_init(nx_ctx** out, int device);
/* ComputeDispatch::~ComputeDispatch; frees every buffer of the context. */
nx_status nx_destroy(nx_ctx* ctx);
/* ComputeDispatch::has_gpu (compute_dispatch.h:32): 1 if a gfx950 device is visible. */
int nx_has_gpu(void);
/* ComputeDispatch::gpu_name (compute_dispatch.h:35) */
nx_status nx_device_name(nx_ctx* ctx, char* buf, size_t n);
/* Message of the last failed call on this context ("" if none). */
const char* nx_last_error(nx_ctx* ctx);
/* Message of the last nx_init failure (no context exists then). */
const char* nx_init_error(void);
/* SHA-1 of the sources the library was built from (csrc/ and include/, as
 * the Makefile concatenates them).  No counterpart in the reference: lets a
 * binding refuse a library that is older than the sources beside it. */
const char* nx_source_hash(void);

/* --------------------------------------------------------------- memory -- */
/* MetalBackend::alloc_shared_buffer / free_buffer (metal_backend.mm:760-768, :859-864).
 * Device memory, zero-filled. */
nx_status nx_alloc(nx_ctx* ctx, size_t bytes, nx_buf* out);
nx_status nx_free(nx_ctx* ctx, nx_buf buf);
/* ComputeDispatch::upload_to_gpu (compute_dispatch.h:203); replaces the UMA
 * memcpy into a shared MTLBuffer (metal_backend.mm:836-850).  Synchronous. */
nx_status nx_upload(nx_ctx* ctx, nx_buf dst, size_t dst_offset, const void* src, size_t bytes);
/* ComputeDispatch::download_from_gpu (compute_dispatch.h:207); waits for the stream. */
nx_status nx_download(nx_ctx* ctx, void* dst, nx_buf src, size_t src_offset, size_t bytes);
/* The wrapped-pointer weight cache keyed by host pointer
 * (compute_dispatch.h:311, compute_dispatch.cpp:148-154) and
 * upload_small_buffer (compute_dispatch.h:129): the first call uploads
 * `bytes` from `src` into a new device buffer remembered under `host_key`;
 * later calls with the same key return that buffer without copying. */
nx_status nx_weight_cache(nx_ctx* ctx, const void* host_key, const void* src, size_t bytes,
                          nx_buf* out);
/* ComputeDispatch::get_cached_buffer (compute_dispatch.h:273); NX_ERR_INVALID if absent. */
nx_status nx_get_cached_buffer(nx_ctx* ctx, const void* host_key, nx_buf* out);
/* ComputeDispatch::clear_buffer_cache (compute_dispatch.h:270): frees cached weights. */
nx_status nx_clear_buffer_cache(nx_ctx* ctx);
/* Size in bytes of a buffer of this context. */
nx_status nx_buffer_size(nx_ctx* ctx, nx_buf buf, size_t* bytes);
/* Wait for all work enqueued on the context's stream. */
nx_status nx_synchronize(nx_ctx* ctx);

/* ------------------------------------------------------------- batching -- */
/* ComputeDispatch::begin_token / end_token (compute_dispatch.h:106-110,
 * compute_dispatch.cpp:798-833).  Ops between the two are captured into one
 * HIP graph; end_token launches it and waits.  When the captured sequence
 * has the same shape as the previous token's, the instantiated graph is
 * updated in place instead of re-instantiated. */
nx_status nx_token_begin(nx_ctx* ctx);
nx_status nx_token_end(nx_ctx* ctx);
/* ComputeDispatch::flush_token / resume_token (compute_dispatch.h:120-123,
 * compute_dispatch.cpp:816-833; called around the CPU parts of a decode step,
 * hybrid_model.cpp:820-1241): flush launches the ops captured so far in the
 * token batch and waits, so their results can be read; resume captures the
 * following ops into a new segment, launched by the next flush or by
 * nx_token_end.  Each segment keeps its own graph, updated in place from
 * token to token.  A flush after a flush, or a resume without a flush, is a
 * no-op (as in the reference); either outside nx_token_begin/end is
 * NX_ERR_STATE. */
nx_status nx_token_flush(nx_ctx* ctx);
nx_status nx_token_resume(nx_ctx* ctx);

/* ------------------------------------------------------------------ ops -- */
/* int4-g32 GEMV: y[b][n] = sum_k x[b][k] * (q[n][k] - 8) * s[n][k/32], fp32
 * accumulation, y stored fp16.  x fp16 [batch][K].  batch 1..8, K up to
 * 28672 (NX_ERR_UNSUPPORTED above).  Any K and alignment work; batch 2..8
 * runs its fastest form when K % 256 == 0 (whole groups, a multiple of 8 per
 * row) and the scales start 16-byte aligned.
 * Replaces ComputeDispatch::gemm_int4 (compute_dispatch.h:59,
 * compute_dispatch.cpp:142-176) -> MetalBackend::gemv_int4_nr8
 * (metal_backend.mm:607-642), and gemv_int4 (compute_dispatch.h:47) whose
 * grouped semantics it follows. */
nx_status nx_gemv_int4_g32(nx_ctx* ctx, nx_buf x_f16, nx_buf wq, nx_buf scales_f16,
                           nx_buf y_f16, int N, int K, int batch);
/* Same product with fp32 output; accumulate != 0 adds into y (the residual
 * add of hybrid_model.cpp:1397-1400 fused).  Replaces gemm_int4_gpu
 * (compute_dispatch.h:197) + gpu_residual_add (compute_dispatch.h:221). */
nx_status nx_gemv_int4_g32_f32(nx_ctx* ctx, nx_buf x_f16, nx_buf wq, nx_buf scales_f16,
                               nx_buf y_f32, int N, int K, int batch, int accumulate);
/* Unpack n int4 codes (low nibble first) to one byte each -- the bit-exact
 * check hook for the GPU unpack (quant::dequant_int4, gptq.cpp:12-25). */
nx_status nx_unpack_int4(nx_ctx* ctx, nx_buf packed, nx_buf codes_u8, size_t n);
/* GEMM of M rows: y[M][N] (fp32) = x[M][K] (fp16) . W^T, W int4-g32 as for
 * the GEMV; accumulate != 0 adds into y.  The matrix-core kernel of the
 * batched prefill: exact (q - 8) x products per group, scaled in fp32, as
 * in the GEMV.  K must be a multiple of 8.  Replaces gemm_int4
 * (compute_dispatch.h:59) with M activation rows. */
nx_status nx_gemm_int4_g32(nx_ctx* ctx, nx_buf x_f16, nx_buf wq, nx_buf scales_f16, nx_buf y_f32, int M, int N,
                           int K, int accumulate);
/* Device symmetric int4-g32 quantizer of w fp32 [N][K]: s = fp16(amax/7),
 * q = clamp(roundf(w/s), -8, 7) + 8.  (Replaces the offline quant_int4,
 * gptq.cpp:37-70, whose asymmetric output the GPU kernels never consumed.) */
nx_status nx_quantize_int4_g32(nx_ctx* ctx, nx_buf w_f32, nx_buf wq, nx_buf scales_f16, int N,
                               int K);
/* RMSNorm: out = fp16((x * 1/sqrt(mean(x^2) + eps)) * w), x fp32 [batch][dim];
 * w fp32 [dim] or 0 for ones.  ComputeDispatch::rmsnorm / gpu_rmsnorm
 * (compute_dispatch.h:66, :215; compute::rms_norm gemm.cpp:96-114). */
nx_status nx_rmsnorm(nx_ctx* ctx, nx_buf x_f32, nx_buf w_f32, nx_buf out_f16, int dim, float eps,
                     int batch);
/* RoPE in place on x fp32 [batch][heads][head_dim]: interleaved pairs,
 * angle pos*theta^(-2i/hd) from the cos/sin tables fp32 [max_pos][hd/2].
 * The reference has none (transformer.cpp:255). */
nx_status nx_rope(nx_ctx* ctx, nx_buf x_f32, nx_buf positions_i32, nx_buf cos_tab, nx_buf sin_tab,
                  int heads, int head_dim, int batch, int max_pos);
/* SwiGLU: out = fp16(g / (1 + exp(-g)) * u), fp32 inputs [batch][n].
 * ComputeDispatch::swiglu / gpu_swiglu (compute_dispatch.h:72, :211). */
nx_status nx_swiglu(nx_ctx* ctx, nx_buf gate_f32, nx_buf up_f32, nx_buf out_f16, int n, int batch);
/* out = a + b, fp32 [n].  ComputeDispatch::gpu_residual_add (compute_dispatch.h:221). */
nx_status nx_residual_add(nx_ctx* ctx, nx_buf a, nx_buf b, nx_buf out, int n);
/* Append one token's K/V (fp32 [batch][hkv][head_dim], converted to fp16
 * round-to-nearest-even) at positions[b] through the block table.  The
 * cache write of MetalBackend::attention_gpu (attention_gpu.metal:40-64) and
 * of gqa_attention (hybrid_model.cpp:1460-1468, which truncates instead). */
nx_status nx_kv_append_f16(nx_ctx* ctx, nx_buf k_f32, nx_buf v_f32, nx_buf kpool, nx_buf vpool,
                           nx_buf block_table, nx_buf positions_i32, int batch, int hkv,
                           int head_dim, int max_blocks, int num_blocks);
/* Paged fp16 decode attention: out[b][h] = softmax(q.K^T / sqrt(hd)) V over
 * positions [0, ctx_lens[b]), GQA kv head = h / (hq/hkv); q fp32
 * [batch][hq][hd]; out fp16 [batch][hq][hd].  Replaces
 * ComputeDispatch::attention_gpu / fused_attention (compute_dispatch.h:176,
 * :187) and the CPU gqa_attention (hybrid_model.cpp:1447-1565). */
nx_status nx_attn_decode_paged_f16(nx_ctx* ctx, nx_buf q_f32, nx_buf kpool, nx_buf vpool,
                                   nx_buf block_table, nx_buf ctx_lens_i32, nx_buf out_f16,
                                   int batch, int hq, int hkv, int head_dim, int max_blocks,
                                   int num_blocks);
/* nx_attn_decode_paged_f16 for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments and result;
 * the split records and counters live in a static device array of the
 * library (4 MiB of records + 16384 counters per device, held until the
 * process ends), so the call allocates nothing and does not synchronize:
 * it may be captured.  The context length and block-table checks run in the
 * kernel instead of on the host: a sequence whose length exceeds
 * max_blocks * 16 or whose table names a block outside [0, num_blocks) gets
 * NaN output rows (its pages are not read).  NX_ERR_UNSUPPORTED when the
 * split plan of (batch, hq, hkv, head_dim, max_blocks) needs more records or
 * counters than the array holds.  Every call on one device shares the array:
 * calls that overlap on one device (two streams, two contexts) race. */
nx_status nx_attn_decode_paged_f16_noalloc(nx_ctx* ctx, nx_buf q_f32, nx_buf kpool, nx_buf vpool,
                                           nx_buf block_table, nx_buf ctx_lens_i32, nx_buf out_f16,
                                           int batch, int hq, int hkv, int head_dim, int max_blocks,
                                           int num_blocks);
/* TurboQuant codebooks (Lloyd-Max for N(0,1/128), kv/turbo_quant.cpp:172-219)
 * as computed by this library on the host: c4[16], b4[15], c3[8], b3[7]. */
nx_status nx_tq_codebooks(float* c4, float* b4, float* c3, float* b3);
/* TurboQuant encode of nvec vectors x fp32 [nvec][128]:
 *   n = sqrt(canonical sum of squares); u = (sign .* x) * (1/n);
 *   y = FWHT128(u) * float(1/sqrt(128)); code_i = first j with y_i < b[j]
 *   (4-bit codebook for i < 64, 3-bit for i >= 64); codes packed LSB-first
 *   (kv/turbo_quant.cpp:249-268); norm stored fp16.
 * signs fp32 [128] of +-1.  Replaces TurboQuantKV::quantize
 * (kv/turbo_quant.cpp:289-327) with a randomized Hadamard rotation. */
nx_status nx_tq_encode(nx_ctx* ctx, nx_buf x_f32, nx_buf signs_f32, nx_buf codes4, nx_buf codes3,
                       nx_buf norms_f16, int nvec);
/* Append one token's K/V (fp32 [batch][hkv][128]) to TurboQuant pages. */
nx_status nx_tq_append(nx_ctx* ctx, nx_buf k_f32, nx_buf v_f32, nx_buf ksigns, nx_buf vsigns,
                       nx_buf kc4, nx_buf kc3, nx_buf kn, nx_buf vc4, nx_buf vc3, nx_buf vn,
                       nx_buf block_table, nx_buf positions_i32, int batch, int hkv,
                       int max_blocks, int num_blocks);
/* Decode attention over TurboQuant pages (head_dim 128), scored in the
 * rotated domain: score = n_t * <Pi q, c[code_t]> / sqrt(128), V summed in
 * the rotated domain and rotated back once.  out fp16 [batch][hq][128]. */
nx_status nx_attn_decode_paged_tq(nx_ctx* ctx, nx_buf q_f32, nx_buf kc4, nx_buf kc3, nx_buf kn,
                                  nx_buf vc4, nx_buf vc3, nx_buf vn, nx_buf ksigns, nx_buf vsigns,
                                  nx_buf block_table, nx_buf ctx_lens_i32, nx_buf out_f16,
                                  int batch, int hq, int hkv, int max_blocks, int num_blocks);
/* MoE routing: softmax over E logits fp32 [batch][E], top-k by probability
 * (ties: lower id), renormalized weights.  hybrid_model.cpp:1656-1694.
 * E <= 256, k <= min(16, E), batch <= 64. */
nx_status nx_moe_route_topk(nx_ctx* ctx, nx_buf logits_f32, nx_buf ids_i32, nx_buf weights_f32,
                            int E, int k, int batch);
/* Expert SwiGLU FFN for routed tokens: out[b] (+)= sum_j w[b][j] *
 * W2_e(fp16(silu(W1_e x) * W3_e x)), e = ids[b][j].  Expert weights are
 * int4-g32: w13 [E][2F][d] with gate/up rows interleaved (row 2f = gate f,
 * 2f+1 = up f), s13 its scales; w2 [E][d][F], s2.  x fp16 [batch][d].
 * batch <= 8; at most 8 slots may name one expert (NX_ERR_INVALID).
 * ComputeDispatch::batched_moe_ffn (compute_dispatch.h:84,
 * compute_dispatch.cpp:211-275; batched_expert_gemv.metal:47-160). */
nx_status nx_moe_expert_ffn(nx_ctx* ctx, nx_buf x_f16, nx_buf w13, nx_buf s13, nx_buf w2,
                            nx_buf s2, nx_buf ids_i32, nx_buf weights_f32, nx_buf out_f32, int d,
                            int F, int E, int k, int batch, int accumulate);
/* GEMM C[M][N] = A[M][K] B[K][N], all fp32 row-major, on the matrix cores
 * (fp32 products and sums).  ComputeDispatch::gemm (compute_dispatch.h:42,
 * the dense-weight path of hybrid_model.cpp:121; compute::gemm_f32). */
nx_status nx_gemm_f32(nx_ctx* ctx, nx_buf A, nx_buf B, nx_buf C, int M, int N, int K);
/* SwiGLU FFN of int4-g32 weights: y[b] (+)= W2 (fp16(silu(W1 x_b) * W3 x_b))
 * for batch rows of x fp16 [batch][d]; w13 [2F][d] holds W1 / W3 rows
 * interleaved (row 2f = W1 row f, 2f+1 = W3 row f), s13 their scales, w2
 * [d][F] and s2; y fp32 [batch][d]; d up to 14336, F up to 28672.  The four dispatches of
 * ComputeDispatch::gpu_ffn_fused (compute_dispatch.h:254,
 * compute_dispatch.cpp:682-727) as two launches (the SwiGLU is the gate/up
 * GEMV's epilogue); the intermediate activations stay on the device in a
 * workspace of the context (grown outside capture, or reserved with
 * nx_reserve_workspace). */
nx_status nx_ffn_int4_g32(nx_ctx* ctx, nx_buf x_f16, nx_buf w13, nx_buf s13, nx_buf w2, nx_buf s2, nx_buf y_f32,
                          int d, int F, int batch, int accumulate);
/* Greedy sampling: first maximum of logits fp32 [batch][V]
 * (hybrid_model.cpp:2027-2038). */
nx_status nx_argmax(nx_ctx* ctx, nx_buf logits_f32, nx_buf out_i32, int V, int batch);
/* HybridModel::Impl::sample_token (hybrid_model.cpp:2023-2099) on the device
 * for each of `batch` rows of logits: temperature <= 0 is the greedy argmax;
 * otherwise softmax of logits / T, top-k (0 or >= V = off), top-p over what
 * top-k keeps (1 = off; the entry whose running sum in descending order
 * first exceeds top_p is kept), renormalize, and the first index whose
 * running sum reaches u * sum.  u comes from a fresh MT19937 seeded with `seed` at
 * every call, as in the reference (std::uniform_real_distribution<float>
 * as libstdc++ computes it); seed 0 draws from std::random_device.  Ties in
 * the top-k and top-p orders keep the lower index. */
nx_status nx_sample(nx_ctx* ctx, nx_buf logits_f32, nx_buf out_i32, int V, int batch, float temperature, int top_k,
                    float top_p, uint64_t seed);

/* -------------------------------------------------- set-up and residency -- */
/* The persistent activation buffers of a decode step
 * (ComputeDispatch::GPUBufferPool, compute_dispatch.h:137-155): device
 * buffers of the context, zero-filled, `batch` rows each, freed with
 * nx_free or nx_destroy.  GEMV inputs are fp16 here (norm, attn_out,
 * ffn_act); the reference keeps them fp32. */
typedef struct {
    nx_buf hidden;    /* fp32 [batch][hidden] */
    nx_buf residual;  /* fp32 [batch][hidden] */
    nx_buf norm;      /* fp16 [batch][hidden] (the reference's norm_buf) */
    nx_buf q;         /* fp32 [batch][max_q] */
    nx_buf k, v;      /* fp32 [batch][max_kv] */
    nx_buf attn_out;  /* fp16 [batch][max_q] */
    nx_buf ffn_gate;  /* fp32 [batch][max_ffn] */
    nx_buf ffn_up;    /* fp32 [batch][max_ffn] */
    nx_buf ffn_act;   /* fp16 [batch][max_ffn rounded up to 8] SwiGLU output */
    nx_buf ffn_out;   /* fp32 [batch][hidden] */
    nx_buf logits;    /* fp32 [batch][vocab] */
    nx_buf token;     /* int32 [batch] */
} nx_gpu_pool;
/* ComputeDispatch::init_gpu_pool (compute_dispatch.h:163,
 * hybrid_model.cpp:540). */
nx_status nx_init_gpu_pool(nx_ctx* ctx, int hidden, int max_q, int max_kv, int max_ffn, int vocab, int batch,
                           nx_gpu_pool* out);
/* ComputeDispatch::init_kv_cache (compute_dispatch.h:170,
 * compute_dispatch.cpp:357-385; hybrid_model.cpp:550): the GPU-resident KV
 * cache as fp16 pages of 16 tokens for the paged entry points --
 * kpools[l] / vpools[l] (num_layers buffers each, zero-filled) of
 * num_blocks = batch * max_blocks pages of n_kv_heads x 16 x head_dim, and a
 * block table int32 [batch][max_blocks] mapping sequence b's page p to block
 * b * max_blocks + p (max_blocks = ceil(max_seq / 16)).  The reference
 * keeps fp32 K/V contiguous per layer. */
nx_status nx_init_kv_cache(nx_ctx* ctx, int num_layers, int max_seq, int n_kv_heads, int head_dim, int batch,
                           nx_buf* kpools, nx_buf* vpools, nx_buf* block_table, int* max_blocks, int* num_blocks);
/* ComputeDispatch::pre_allocate_activation_buffer (compute_dispatch.h:281,
 * compute_dispatch.cpp:862-870; hybrid_model.cpp:519): grows every
 * workspace the entry points keep per context -- FFN activations, sampler
 * rows, attention split records and counters -- to what calls up to these
 * sizes need, so those calls allocate nothing (and may be captured).  A size
 * of 0 skips its workspace.  The reference reserves staging bytes; this
 * library takes the shapes the bytes come from. */
nx_status nx_reserve_workspace(nx_ctx* ctx, int batch, int max_ffn, int vocab, int n_heads, int n_kv_heads,
                               int head_dim, int max_ctx);
/* ComputeDispatch::preload_all_buffers (compute_dispatch.h:285,
 * compute_dispatch.cpp:872-887; hybrid_model.cpp:581, :639): the reference
 * touches every cached weight buffer to fault its pages into RAM.  Device
 * memory is resident once allocated, so this waits for every upload on the
 * context's stream to finish and reports the number of cached weight
 * buffers (n_buffers may be NULL). */
nx_status nx_preload_all_buffers(nx_ctx* ctx, size_t* n_buffers);

/* ----------------------------------------------------------- the runner -- */
/* A resident decoder driven by this library: the counterpart of
 * HybridModel (hybrid_model.h, hybrid_model.cpp:319-774) for Llama-style
 * dense and MoE models, with synthetic int4-g32 weights generated on the
 * device from a seed (counter-based RNG shared with the test oracle). */
typedef struct {
    int n_layers, d_model, n_heads, n_kv_heads, head_dim, ffn, vocab;
    int n_experts, top_k;   /* n_experts == 0: dense SwiGLU */
    int max_seq;            /* per sequence, multiple of 16 */
    int batch;              /* sequences decoded together (1..8) */
    int kv_kind;            /* 0 = fp16 pages, 1 = TurboQuant pages (head_dim 128),
                               2 = tiered: the last hot_window positions fp16 (a ring of
                               hot_window / 16 + 1 pages per sequence), older pages
                               compressed to TurboQuant on the device as they leave
                               the window (head_dim 128) */
    float rope_theta;
    float eps;
    uint64_t seed;
    float norm_sigma;       /* RMSNorm weights: 0 = all 1.0, else 1 + N(0, norm_sigma)
                               seeded per tensor (synthetic models) */
    int hot_window;         /* kv_kind 2: positions kept fp16, a positive multiple of 16 */
    int warm_window;        /* kv_kind 2: 0 = two tiers (fp16, TurboQuant); else a positive
                               multiple of 16: the positions before the window kept TurboQuant
                               (Warm, a ring of warm_window / 16 + 1 pages per sequence), older
                               pages re-encoded on the device to the Cool form (3-bit codes on
                               every coordinate, 50 bytes per vector) as they leave that range:
                               the Hot -> Warm -> Cool tiers of PagedKVCache
                               (kv/paged_attention.h:18-24, compress_tier
                               kv/paged_attention.cpp:244-291) as a per-page policy */
    int cool_window;        /* kv_kind 2 with a warm_window: 0 = keep every Cool page; else a
                               positive multiple of 16: the positions kept Cool (a ring of
                               cool_window / 16 + 1 pages per sequence), older pages evicted --
                               the Cold tier of evict_cold_pages (kv/paged_attention.cpp:295-310):
                               attention reads an evicted position as the zero key and value
                               get_vectors gathers for a page it does not hold (:172, :219) */
    int kv_blocks;          /* 0 = every sequence holds a full-length page table (batch *
                               max_seq / 16 pages); else the pages of one shared pool, taken
                               as sequences grow and given back when a slot retires or starts
                               over (the page table of PagedKVCache, kv/paged_attention.cpp:
                               59-77, whose pages are created on first insert); a step that
                               needs more than are free fails with NX_ERR_CAPACITY before it
                               runs.  Not with a cool_window (every table is then a ring). */
    int qk_norm;            /* 1: per-head RMSNorm of q and k after the QKV projection (every
                               head_dim slice normalized with the layer's head_dim-long
                               attn_q_norm / attn_k_norm weights, hybrid_model.cpp:1325-1349),
                               applied before RoPE; 0: none */
} nx_model_config;

typedef struct nx_model nx_model;

/* HybridModel::create (hybrid_model.cpp:319-600): allocate and generate weights. */
nx_status nx_model_create(nx_ctx* ctx, const nx_model_config* cfg, nx_model** out);
nx_status nx_model_destroy(nx_model* m);
/* HybridModel::prefill (hybrid_model.cpp:604-644): run prompt [batch][P]
 * (batched or token by token, nx_model_set_prefill); afterwards the greedy
 * token of the last prompt position is pending as the next input and written
 * to next_tokens [batch] (optional). */
nx_status nx_model_prefill(nx_model* m, const int32_t* prompt, int P, int32_t* next_tokens);
/* Prefill mode: 1 (default) = batched -- for dense and MoE models with fp16,
 * TurboQuant or tiered pages, each sequence's prompt goes
 * through every layer in chunks of up to 2048 tokens as int4-g32 GEMMs on
 * the matrix cores (routed experts over their gathered tokens), with causal
 * attention over the pages; 0 = one decode step per prompt token (the
 * reference's HybridModel::prefill loop, hybrid_model.cpp:604-644).  Tiered
 * pages with a Warm range always prefill one token per step. */
nx_status nx_model_set_prefill(nx_model* m, int batched);
/* The configuration the model was created with. */
nx_status nx_model_get_config(nx_model* m, nx_model_config* out);
/* The context the model runs on. */
nx_ctx* nx_model_context(nx_model* m);

/* Sequence slots.  Each of the `batch` slots holds one sequence (active) or
 * none (free).  nx_model_prefill and nx_model_fill_context make every slot
 * active; nx_model_decode advances the active slots only (a free slot's
 * output tokens are -1, and the step computes nothing it keeps).  The
 * reference serves one request per Engine::generate
 * (nexus/src/core/engine.cpp:124-184); these let sequences of different
 * prompt lengths join and leave a batch between decode calls.
 * nx_model_admit: sequence `slot` starts over with prompt[P] (any P below
 * max_seq): the prompt is prefilled into that slot alone -- batched GEMMs
 * where the model allows it, otherwise one step per prompt token during
 * which the other active sequences are held (they compute a position they
 * have not reached and keep their state) -- and its first generated token
 * is written to next_token (optional).  nx_model_retire frees a slot. */
nx_status nx_model_admit(nx_model* m, int slot, const int32_t* prompt, int P, int32_t* next_token);
nx_status nx_model_retire(nx_model* m, int slot);
nx_status nx_model_slot_active(nx_model* m, int slot, int* active);

/* Request scheduler over a model's slots (the serving loop of
 * Engine::generate, engine.cpp:124-184, for many requests): requests wait
 * in arrival order and are admitted into free slots; active slots decode in
 * chunks of up to 8 steps; a request completes after max_new tokens (its
 * first is the token after the prompt) or once it emits `stop` (-1: none),
 * and its slot goes to the next waiting request.  Creating a scheduler
 * frees every slot of the model. */
typedef struct nx_sched nx_sched;
nx_status nx_sched_create(nx_model* m, nx_sched** out);
nx_status nx_sched_destroy(nx_sched* s);
nx_status nx_sched_submit(nx_sched* s, const int32_t* prompt, int P, int max_new, int stop, int* id);
/* One round: admit what fits, decode one chunk, retire what completed. */
nx_status nx_sched_step(nx_sched* s, int* n_active, int* n_waiting);
/* Rounds until no request is waiting or active. */
nx_status nx_sched_run(nx_sched* s);
/* The tokens of request id so far (up to cap into out), their number and
 * whether the request is complete.  A request whose admission failed (the
 * nx_sched_step that tried it returned the error) is complete with no tokens,
 * and this call returns that admission's status. */
nx_status nx_sched_result(nx_sched* s, int id, int32_t* out, int cap, int* n, int* done);
/* Sampling of the decode loop (SamplingParams, core/config.h:60-66):
 * temperature <= 0 = greedy (the default); otherwise every step samples
 * with nx_sample's rules inside the step graph.  seed != 0: the draw of
 * std::mt19937(seed), the same at every step as in the reference; seed 0:
 * a counter-based draw keyed by (sequence, position) (the reference uses
 * std::random_device). */
nx_status nx_model_set_sampling(nx_model* m, float temperature, int top_k, float top_p, uint64_t seed);
/* Fill positions [0, ctx) of every layer's cache with synthetic N(0,1) K/V
 * (n_outlier channels per head scaled x10); the pending token of every
 * sequence becomes a seeded start token. */
nx_status nx_model_fill_context(nx_model* m, int ctx, int n_outlier);
/* The stored form of position pos of sequence b in layer `layer`, all kv
 * heads, K (kv 0) or V (kv 1): form 0 = fp16 [hkv][head_dim] (2 * hkv *
 * head_dim bytes), form 1 = TurboQuant [hkv] x (32 bytes of 4-bit codes, 24
 * of 3-bit codes, fp16 norm) (58 * hkv bytes), form 2 = Cool [hkv] x (48
 * bytes of 3-bit codes, fp16 norm) (50 * hkv bytes); *form tells which
 * (tiered pages: 1 before the window, 0 in it, 2 before the Warm range with
 * three tiers, 3 = evicted, no bytes).  The per-position read-back of
 * PagedKVCache::get_vectors (kv/paged_attention.cpp:161-230), as stored
 * rather than decompressed; cap = bytes available at out. */
nx_status nx_model_kv_read(nx_model* m, int layer, int b, int pos, int kv, int* form, void* out, size_t cap);
/* Pages of the model's KV pool (per layer) and how many are free: with a
 * shared pool (kv_blocks) its free list, else batch * max_seq / 16 less the
 * pages the sequences' positions cover.  Either pointer may be NULL. */
nx_status nx_model_kv_pages(nx_model* m, int* total, int* free_pages);
/* The pending (next input) token of every sequence, [batch]. */
nx_status nx_model_pending(nx_model* m, int32_t* tokens);
/* Engine::generate's loop (engine.cpp:155-173) of `steps` decode_step calls
 * (hybrid_model.cpp:648-774) with the sampled token fed back: out_tokens
 * [batch][steps] receives the greedy token produced by each step.  The
 * whole step is one HIP graph launch; nothing is copied to the host between
 * steps. */
nx_status nx_model_decode(nx_model* m, int steps, int32_t* out_tokens);
/* The same steps with the input token of every step given instead of fed
 * back (teacher forcing): active sequence b consumes tokens[b][s] at step s
 * (tokens [batch][steps]), and logits [batch][steps][V] (optional) receive
 * the fp32 logits each step produced.  Positions advance by steps; the
 * pending token afterwards is the last step's greedy token.  One graph
 * launch per step, with the step's tokens uploaded before it. */
nx_status nx_model_decode_forced(nx_model* m, const int32_t* tokens, int steps, float* logits);
/* Logits fp32 [batch][V] of the last step. */
nx_status nx_model_logits(nx_model* m, float* out);
/* Current position of sequence b. */
nx_status nx_model_position(nx_model* m, int b, int* pos);
/* Algorithmic HBM bytes of one decode step at the current positions. */
nx_status nx_model_step_bytes(nx_model* m, double* bytes);

/* ---------------------------------------------------------- measurement -- */
/* Average device duration (ms) of the dominant decode kernel -- the fused
 * RMSNorm + gate/up int4 GEMV + SwiGLU -- over `iters` back-to-back launches
 * on the model's buffers, launch i on layer i % n_layers (cold weights, as
 * in a decode step), timed with HIP events on the library stream; bytes =
 * its algorithmic bytes per launch.  MoE models: the routed gate/up expert
 * GEMV + SwiGLU with the last decode step's routing of the last layer (at
 * least one step must have run; NX_ERR_STATE otherwise), bytes = the active
 * experts' gate/up weights plus the gathered inputs and outputs. */
nx_status nx_model_time_ffn_gemv(nx_model* m, int iters, double* avg_ms, double* bytes);
/* Average device time (ms) per launch of nx_gemv_int4_g32 of shape N x K,
 * batch: `iters` launches captured as one graph, one warm replay, then one
 * replay between HIP events (so the figure includes the kernel boundary a
 * decode step's graph pays per launch).  Launch i uses weight copy
 * i % ncopies (wq[], scales_f16[]), so with enough copies every launch
 * streams its weights from HBM rather than from the last-level cache. */
nx_status nx_time_gemv(nx_ctx* ctx, nx_buf x_f16, const nx_buf* wq, const nx_buf* scales_f16,
                       int ncopies, nx_buf y_f16, int N, int K, int batch, int iters,
                       double* avg_ms);
/* Same for the paged attention of the model's cache kind (split and merge
 * launches together), launch i over layer i % n_layers. */
nx_status nx_model_time_attention(nx_model* m, int iters, double* avg_ms, double* bytes);
/* Average device time (ms) of nx_gemm_int4_g32 (no accumulate) over iters
 * launches, HIP events on the library stream. */
nx_status nx_time_gemm(nx_ctx* ctx, nx_buf x_f16, nx_buf wq, nx_buf scales_f16, nx_buf y_f32, int M, int N, int K,
                       int iters, double* avg_ms);

#ifdef __cplusplus
}
#endif
#endif
