// Small decode-loop kernels on gfx950: standalone RMSNorm / RoPE / SwiGLU /
// residual add / KV append / argmax, int4 unpack and quantize, the device
// side of the synthetic generator, the step-start embedding kernel and MoE
// routing.  None of these is on the HBM-heavy path; they favour simplicity.
#include "nx_common.h"
#include "nx_kernels.h"
#include "nx_route_dev.h"

namespace nx {

namespace {

__device__ inline float block_sum256(float v, float* red) {
    v = wave_sum(v);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    const float t = red[0] + red[1] + red[2] + red[3];
    __syncthreads();
    return t;
}

__global__ __launch_bounds__(256) void k_rmsnorm(const float* x, const float* w, uint16_t* out,
                                                 int dim, float eps) {
    __shared__ float red[4];
    const float* xb = x + (size_t)blockIdx.x * dim;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < dim; i += 256) ss += xb[i] * xb[i];
    ss = block_sum256(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = threadIdx.x; i < dim; i += 256) {
        const float v = xb[i] * inv;
        out[(size_t)blockIdx.x * dim + i] = f2h_bits(w ? v * w[i] : v);
    }
}

// One row per block of 1024 threads, 16-byte loads: every x and weight
// chunk of the row is requested at once (thread t holds chunks t, t + 1024,
// ..., at most kNormChunks), one reduction, the normalized row from
// registers.  Rows of up to 16384 with dim % 4 == 0 and 16-byte aligned
// pointers.
constexpr int kNormThreads = 1024, kNormChunks = 4;
__global__ __launch_bounds__(kNormThreads) void k_rmsnorm_vec(const float* x, const float* w, uint16_t* out,
                                                              int dim, float eps) {
    __shared__ float red[kNormThreads / 64];
    const int nc = dim / 4, t = threadIdx.x;
    const float4* xb = reinterpret_cast<const float4*>(x + (size_t)blockIdx.x * dim);
    const float4* wb = reinterpret_cast<const float4*>(w);
    float4 v[kNormChunks], wv[kNormChunks];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < kNormChunks; ++j) {
        const int c = t + j * kNormThreads;
        v[j] = c < nc ? xb[c] : make_float4(0.f, 0.f, 0.f, 0.f);
        wv[j] = w && c < nc ? wb[c] : make_float4(1.f, 1.f, 1.f, 1.f);
    }
#pragma unroll
    for (int j = 0; j < kNormChunks; ++j) ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
    ss = wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormThreads / 64; ++i) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / (float)dim + eps);
    uint2* ob = reinterpret_cast<uint2*>(out + (size_t)blockIdx.x * dim);
#pragma unroll
    for (int j = 0; j < kNormChunks; ++j) {
        const int c = t + j * kNormThreads;
        if (c >= nc) break;
        const uint32_t lo = (uint32_t)f2h_bits(v[j].x * inv * wv[j].x) | ((uint32_t)f2h_bits(v[j].y * inv * wv[j].y) << 16);
        const uint32_t hi = (uint32_t)f2h_bits(v[j].z * inv * wv[j].z) | ((uint32_t)f2h_bits(v[j].w * inv * wv[j].w) << 16);
        ob[c] = make_uint2(lo, hi);
    }
}

__global__ void k_rope(float* x, const int32_t* pos, const float* cos_t, const float* sin_t,
                       int heads, int hd, int batch) {
    const int half = hd / 2;
    const int total = batch * heads * half;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int b = t / (heads * half), r = t % (heads * half);
    const int h = r / half, i = r % half;
    const int p = pos[b];
    float* v = x + ((size_t)b * heads + h) * hd;
    const float c = cos_t[(size_t)p * half + i], s = sin_t[(size_t)p * half + i];
    const float a = v[2 * i], bb = v[2 * i + 1];
    v[2 * i] = a * c - bb * s;
    v[2 * i + 1] = a * s + bb * c;
}

// Per-head Q/K RMSNorm (HybridModel, hybrid_model.cpp:1325-1349: every
// head_dim slice of q and of k through rmsnorm with the head_dim-long
// weights), then RoPE and the page write of one decode step.  Block (head,
// sequence), one wavefront: heads [0, hq) of q, [hq, hq + hkv) of k, then
// hkv heads of v (written to the pages unchanged).  Lane l holds the RoPE
// pairs j = l and l + 64 (elements 2j, 2j + 1), hd <= 256.  The arithmetic
// is the oracle's: ((x * inv) * w), then the rotation.
__global__ __launch_bounds__(64) void k_qk_norm_rope(QknArgs a) {
    const int h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
    const int hd = a.hd, half = hd >> 1, qdim = a.hq * hd, kvdim = a.hkv * hd;
    const int kind = h < a.hq ? 0 : h < a.hq + a.hkv ? 1 : 2;  // q, k, v
    const int hh = kind == 0 ? h : kind == 1 ? h - a.hq : h - a.hq - a.hkv;
    float* x = kind == 0 ? a.q32 + (size_t)b * qdim + (size_t)hh * hd
                         : a.kv_tmp + ((size_t)b * 2 + (kind == 2 ? 1 : 0)) * kvdim + (size_t)hh * hd;
    const int p = a.pos[b];
    float v0[2], v1[2];
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int j = lane + 64 * u;
        v0[u] = j < half ? x[2 * j] : 0.0f;
        v1[u] = j < half ? x[2 * j + 1] : 0.0f;
        ss += v0[u] * v0[u] + v1[u] * v1[u];
    }
    if (kind != 2) {
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)hd + a.eps);
        const float* w = kind == 0 ? a.qn : a.kn;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int j = lane + 64 * u;
            if (j >= half) continue;
            float x0 = v0[u] * inv, x1 = v1[u] * inv;
            if (w) {
                x0 = x0 * w[2 * j];
                x1 = x1 * w[2 * j + 1];
            }
            const float c = a.cos_t[(size_t)p * half + j], s = a.sin_t[(size_t)p * half + j];
            v0[u] = x0 * c - x1 * s;
            v1[u] = x0 * s + x1 * c;
        }
    }
    const size_t page = a.kpool ? ((size_t)a.block_table[(size_t)b * a.max_blocks + p / kPage] * a.hkv + hh) *
                                      kPage * hd
                                : 0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int j = lane + 64 * u;
        if (j >= half) continue;
        if (kind == 0 || (kind == 1 && !a.kpool)) {
            x[2 * j] = v0[u];
            x[2 * j + 1] = v1[u];
        } else if (kind == 1) {  // K pages are token-major [16][hd]
            a.kpool[page + (size_t)(p % kPage) * hd + 2 * j] = f2h_bits(v0[u]);
            a.kpool[page + (size_t)(p % kPage) * hd + 2 * j + 1] = f2h_bits(v1[u]);
        } else if (a.kpool) {    // V pages are dimension-major [hd][16]
            a.vpool[page + (size_t)(2 * j) * kPage + p % kPage] = f2h_bits(v0[u]);
            a.vpool[page + (size_t)(2 * j + 1) * kPage + p % kPage] = f2h_bits(v1[u]);
        }
    }
}

// The normalization alone, in place: block (head, row), heads [0, hq) of
// q + row * ldq, [hq, hq + hkv) of k + row * ldk; lane l holds elements l,
// l + 64, ... (hd <= 256).
__global__ __launch_bounds__(64) void k_head_rmsnorm(float* q, int ldq, float* k, int ldk, int hq, int hd,
                                                     const float* qn, const float* kn, float eps) {
    const int h = blockIdx.x, row = blockIdx.y, lane = threadIdx.x;
    const bool isq = h < hq;
    float* x = isq ? q + (size_t)row * ldq + (size_t)h * hd : k + (size_t)row * ldk + (size_t)(h - hq) * hd;
    const float* w = isq ? qn : kn;
    float v[4];
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = lane + 64 * u;
        v[u] = i < hd ? x[i] : 0.0f;
        ss += v[u] * v[u];
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)hd + eps);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = lane + 64 * u;
        if (i < hd) x[i] = w ? (v[u] * inv) * w[i] : v[u] * inv;
    }
}

__global__ void k_swiglu(const float* g, const float* u, uint16_t* out, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float gv = g[i];
    out[i] = f2h_bits(gv / (1.0f + expf(-gv)) * u[i]);
}

__global__ void k_residual_add(const float* a, const float* b, float* out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

__global__ void k_kv_append_f16(const float* k, const float* v, uint16_t* kpool, uint16_t* vpool,
                                const int32_t* block_table, const int32_t* pos, int batch, int hkv,
                                int hd, int max_blocks) {
    const int total = batch * hkv * hd;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int b = t / (hkv * hd), r = t % (hkv * hd);
    const int h = r / hd, d = r % hd;
    const int p = pos[b];
    const int blk = block_table[(size_t)b * max_blocks + p / kPage];
    const size_t page = ((size_t)blk * hkv + h) * kPage * hd;
    kpool[page + (size_t)(p % kPage) * hd + d] = f2h_bits(k[(size_t)b * hkv * hd + r]);
    vpool[page + (size_t)d * kPage + p % kPage] = f2h_bits(v[(size_t)b * hkv * hd + r]);
}

__device__ inline unsigned long long pack_best(float v, int idx) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)ord << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)idx);
}

__global__ __launch_bounds__(256) void k_argmax(const float* logits, int32_t* out, int V) {
    __shared__ unsigned long long red[256];
    const float* l = logits + (size_t)blockIdx.x * V;
    unsigned long long best = 0;
    for (int i = threadIdx.x; i < V; i += 256) {
        const unsigned long long k = pack_best(l[i], i);
        if (k > best) best = k;
    }
    red[threadIdx.x] = best;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (threadIdx.x < s && red[threadIdx.x + s] > red[threadIdx.x])
            red[threadIdx.x] = red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[blockIdx.x] = (int32_t)(0xFFFFFFFFu - (uint32_t)(red[0] & 0xFFFFFFFFull));
}

__global__ void k_unpack_int4(const uint8_t* packed, uint8_t* codes, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint8_t b = packed[i >> 1];
    codes[i] = (i & 1) ? (uint8_t)(b >> 4) : (uint8_t)(b & 0x0F);
}

// One thread per (row, group): s = fp16(amax/7); q = clamp(roundf(w/s), -8, 7) + 8.
__device__ inline void quantize_group(const float (&w)[32], int valid, uint8_t* dst,
                                      uint16_t* sdst) {
    float amax = 0.0f;
    for (int j = 0; j < valid; ++j) amax = fmaxf(amax, fabsf(w[j]));
    const uint16_t s16 = f2h_bits(__fdiv_rn(amax, 7.0f));
    const float s = h2f_bits(s16);
    uint32_t words[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        int q = 8;
        if (j < valid && s != 0.0f) {
            int r = (int)roundf(__fdiv_rn(w[j], s));
            r = r < -8 ? -8 : (r > 7 ? 7 : r);
            q = r + 8;
        }
        words[j >> 3] |= (uint32_t)q << (4 * (j & 7));
    }
    *reinterpret_cast<uint4*>(dst) = make_uint4(words[0], words[1], words[2], words[3]);
    *sdst = s16;
}

__global__ void k_quantize_int4(const float* w, uint8_t* codes, uint16_t* scales, int N, int K) {
    const int G = (K + 31) / 32;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (size_t)N * G) return;
    const int n = (int)(t / G), g = (int)(t % G);
    const int k0 = g * 32, valid = min(32, K - k0);
    float v[32];
    for (int j = 0; j < 32; ++j) v[j] = j < valid ? w[(size_t)n * K + k0 + j] : 0.0f;
    quantize_group(v, valid, codes + ((size_t)n * G + g) * 16, scales + (size_t)n * G + g);
}

__global__ void k_gen_quant(uint8_t* codes, uint16_t* scales, int N, int K, uint64_t key, float kf,
                            int row_offset, int row_stride) {
    const int G = (K + 31) / 32;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (size_t)N * G) return;
    const int n = (int)(t / G), g = (int)(t % G);
    const int k0 = g * 32, valid = min(32, K - k0);
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j)
        v[j] = j < valid ? normal_from(rand_at(key, (uint64_t)n * K + k0 + j), kf) : 0.0f;
    const size_t row = (size_t)row_offset + (size_t)n * row_stride;
    quantize_group(v, valid, codes + (row * G + g) * 16, scales + row * G + g);
}

__global__ void k_gen_f16(uint16_t* out, size_t n, uint64_t key, float kf) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = f2h_bits(normal_from(rand_at(key, i), kf));
}

__device__ inline float ctx_value(uint64_t key, size_t idx, float kf, const int32_t* och,
                                  int n_outlier, int d) {
    float v = normal_from(rand_at(key, idx), kf);
    for (int j = 0; j < n_outlier; ++j)
        if (och[j] == d) v *= 10.0f;
    return v;
}

// Thread per (b, p, kv, h, d).
__global__ void k_gen_ctx_f16(uint16_t* kpool, uint16_t* vpool, const int32_t* block_table,
                              int max_blocks, int batch, int ctx, int hkv, int hd, int L,
                              uint64_t seed, float kf, const int32_t* outlier_ch, int n_outlier) {
    const size_t per_pos = (size_t)2 * hkv * hd;
    const size_t total = (size_t)batch * ctx * per_pos;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int b = (int)(t / ((size_t)ctx * per_pos));
    const size_t r = t % ((size_t)ctx * per_pos);
    const int p = (int)(r / per_pos);
    const int r2 = (int)(r % per_pos);
    const int kv = r2 / (hkv * hd), i = r2 % (hkv * hd);
    const int h = i / hd, d = i % hd;
    const uint64_t key = stream_key(seed, tid_ctx(L, b, kv));
    const float v = ctx_value(key, (size_t)p * hkv * hd + i, kf,
                              outlier_ch + ((size_t)kv * hkv + h) * n_outlier, n_outlier, d);
    const int blk = block_table[(size_t)b * max_blocks + p / kPage];
    const size_t page = ((size_t)blk * hkv + h) * kPage * hd;
    if (kv)
        vpool[page + (size_t)d * kPage + p % kPage] = f2h_bits(v);
    else
        kpool[page + (size_t)(p % kPage) * hd + d] = f2h_bits(v);
}

__global__ void k_gen_ctx_raw(float* dst, int ctx, int hkv, int hd, uint64_t key, float kf,
                              const int32_t* outlier_ch, int n_outlier) {
    const size_t total = (size_t)ctx * hkv * hd;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int i = (int)(t % ((size_t)hkv * hd));
    const int h = i / hd, d = i % hd;
    dst[t] = ctx_value(key, t, kf, outlier_ch + (size_t)h * n_outlier, n_outlier, d);
}

// Block per sequence.
__global__ __launch_bounds__(256) void k_embed(unsigned long long* best, int32_t* pos,
                                               const int32_t* base, int32_t* out_tokens,
                                               int out_stride, const uint16_t* embed, float* h,
                                               int d, int vocab, const int32_t* feed, const int32_t* fpos) {
    __shared__ int tok_s;
    const int b = blockIdx.x;
    if (threadIdx.x == 0) {
        const int f = feed ? feed[b] : kFeedDecode;
        int tok, p;
        if (f == kFeedPark) {  // a free slot: token 0 at position 0 of its own pages
            tok = 0;
            p = 0;
        } else if (f == kFeedHold) {  // a paused sequence: a position it has not reached yet
            tok = 0;
            p = fpos[b];
        } else {
            const unsigned long long k = best[b];
            tok = f >= 0 ? f : (int)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull));
            p = pos[b] + 1;
            const int idx = p - base[b] - 1;
            if (f == kFeedDecode && out_tokens && idx >= 0 && idx < out_stride)
                out_tokens[(size_t)b * out_stride + idx] = tok;
        }
        if (tok < 0 || tok >= vocab) tok = 0;  // never index outside the table
        tok_s = tok;
        best[b] = 0ull;
        pos[b] = p;
    }
    __syncthreads();
    const int tok = tok_s;
    const uint16_t* src = embed + (size_t)tok * d;
    float* dst = h + (size_t)b * d;
    if ((d & 7) == 0) {
        // 16-byte chunks, both of a thread's loads in flight together
        // (one round trip for a 4096-wide row)
        const int nch = d / 8;
        for (int c0 = threadIdx.x; c0 < nch; c0 += 512) {
            const int c1 = c0 + 256 < nch ? c0 + 256 : c0;
            const uint4 v0 = reinterpret_cast<const uint4*>(src)[c0];
            const uint4 v1 = reinterpret_cast<const uint4*>(src)[c1];
            const uint32_t w[2][4] = {{v0.x, v0.y, v0.z, v0.w}, {v1.x, v1.y, v1.z, v1.w}};
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int c = j ? c0 + 256 : c0;
                if (c >= nch) break;
                float4 lo, hi;
                lo.x = h2f_bits((uint16_t)(w[j][0] & 0xFFFFu)); lo.y = h2f_bits((uint16_t)(w[j][0] >> 16));
                lo.z = h2f_bits((uint16_t)(w[j][1] & 0xFFFFu)); lo.w = h2f_bits((uint16_t)(w[j][1] >> 16));
                hi.x = h2f_bits((uint16_t)(w[j][2] & 0xFFFFu)); hi.y = h2f_bits((uint16_t)(w[j][2] >> 16));
                hi.z = h2f_bits((uint16_t)(w[j][3] & 0xFFFFu)); hi.w = h2f_bits((uint16_t)(w[j][3] >> 16));
                reinterpret_cast<float4*>(dst)[2 * c] = lo;
                reinterpret_cast<float4*>(dst)[2 * c + 1] = hi;
            }
        }
    } else {
        for (int i = threadIdx.x; i < d; i += 256) dst[i] = h2f_bits(src[i]);
    }
}

__global__ void k_finish_tokens(const unsigned long long* best, const int32_t* pos,
                                const int32_t* base, int32_t* out_tokens, int out_stride,
                                int batch) {
    const int b = threadIdx.x;
    if (b >= batch) return;
    const int idx = pos[b] - base[b];
    const int tok = (int)(0xFFFFFFFFu - (uint32_t)(best[b] & 0xFFFFFFFFull));
    if (idx >= 0 && idx < out_stride) out_tokens[(size_t)b * out_stride + idx] = tok;
}

__global__ void k_set_tokens(unsigned long long* best, const int32_t* tokens, int batch) {
    const int b = threadIdx.x;
    if (b < batch) best[b] = 0xFFFFFFFFull - (unsigned long long)(uint32_t)tokens[b];
}

// Routing of one sequence (hybrid_model.cpp:1656-1694): softmax over the E
// logits, the k largest probabilities (ties: lower id), weights renormalized
// over the chosen k.  A probability is recomputed where it is compared
// (expf(l - max) / sum, the same value every time) instead of being kept, so
// any E up to kMoeMaxExperts needs only the taken bitmask as scratch.
// ids, w: the k outputs; taken: kMoeMaxExperts / 32 words of scratch.
__device__ inline void route_row(const float* lg, int E, int k, int* ids, float* w, uint32_t* taken) {
    float mx = lg[0];
    for (int e = 1; e < E; ++e) mx = fmaxf(mx, lg[e]);
    float sum = 0.0f;
    for (int e = 0; e < E; ++e) sum += expf(lg[e] - mx);
    auto prob = [&](int e) {
        const float x = expf(lg[e] - mx);
        return sum > 0.0f ? x / sum : x;
    };
    for (int i = 0; i < (E + 31) / 32; ++i) taken[i] = 0u;
    float active = 0.0f;
    for (int j = 0; j < k; ++j) {
        int best = -1;
        float bp = 0.0f;
        for (int e = 0; e < E; ++e) {
            if ((taken[e >> 5] >> (e & 31)) & 1u) continue;
            const float pe = prob(e);
            if (best < 0 || pe > bp) {
                best = e;
                bp = pe;
            }
        }
        taken[best >> 5] |= 1u << (best & 31);
        ids[j] = best;
        w[j] = bp;
        active += bp;
    }
    for (int j = 0; j < k; ++j) w[j] = active > 0.0f ? w[j] / active : 1.0f / (float)k;
}

// Per-expert slot lists in (b, j) order and the routing plan (the active
// experts in ascending order; a token's k experts are distinct, so an expert
// holds at most `batch` slots), from the chosen ids [batch][k] (LDS).  Run by
// every thread of the block: thread e lists expert e's slots, wavefront 0
// ranks the active experts (ballots over 64 experts at a time), then the
// plan rows are written in parallel.  cnt, rank: E ints of LDS scratch.
__device__ inline void build_lists(const MoeArgs& a, const int32_t* ids, int* cnt, int* rank) {
    const int t = threadIdx.x, nt = blockDim.x, E = a.E, n = a.batch * a.k;
    for (int e = t; e < E; e += nt) {
        int c = 0;
        for (int sl = 0; sl < n; ++sl)
            if (ids[sl] == e) a.expert_slots[(size_t)e * n + c++] = sl;
        cnt[e] = c;
        a.expert_count[e] = c;
    }
    __syncthreads();
    if (!a.plan) return;
    __shared__ int nact;
    if (t < kWave) {
        int base = 0;
        for (int c0 = 0; c0 < E; c0 += kWave) {
            const int e = c0 + t;
            const bool act = e < E && cnt[e] > 0;
            const unsigned long long bal = __ballot(act);
            if (act) rank[e] = base + __popcll(bal & ((1ull << t) - 1ull));
            base += __popcll(bal);
        }
        if (t == 0) nact = base;
    }
    __syncthreads();
    const int rows = moe_plan_rows(E, a.batch, a.k);
    for (int e = t; e < E; e += nt) {
        if (cnt[e] == 0 || rank[e] >= rows) continue;
        int32_t* pl = a.plan + (size_t)rank[e] * kMoePlanInts;
        pl[0] = e;
        pl[1] = cnt[e];
        int c = 0;
        for (int sl = 0; sl < n; ++sl)
            if (ids[sl] == e) {
                pl[8 + c] = sl;
                pl[16 + c] = sl / a.k;
                ++c;
            }
    }
    for (int r = nact + t; r < rows; r += nt) a.plan[(size_t)r * kMoePlanInts] = -1;
}

// Single wavefront: sequences routed in turn (route_wave), then the
// per-expert token lists and the routing plan.
__global__ __launch_bounds__(64) void k_moe_route(MoeArgs a) {
    __shared__ int32_t sid[64 * kMoeMaxTopK];
    __shared__ int scnt[kMoeMaxExperts], srank[kMoeMaxExperts];
    __shared__ float sw[64 * kMoeMaxTopK];
    for (int b = 0; b < a.batch; ++b) route_wave(a.logits + (size_t)b * a.E, a.E, a.k, sid + b * a.k, sw + b * a.k);
    __syncthreads();
    for (int s = threadIdx.x; s < a.batch * a.k; s += 64) {
        a.ids[s] = sid[s];
        a.weights[s] = sw[s];
    }
    build_lists(a, sid, scnt, srank);
}

// The MoE block's input and routing in one launch (batch <= 8, E <= 16,
// d <= 4096, d % 32 == 0).  Block b takes sequence b: the RMSNorm of h[b] to
// fp16 x (xn16[b], also kept in LDS; hybrid_model.cpp:1647-1655) and the
// router logits of x (int4-g32 rows of wr: wavefront w takes rows w, w + 16,
// ..., its lanes the groups, so every sum has a fixed order).  h and the
// router rows are requested together up front.  Each block publishes its
// logits with agent-scope stores, waits for them, and counts itself in
// *counter; the last block resets the counter and routes every sequence
// (k_moe_route's routing) from the published logits.  With one sequence the
// block routes from its own logits in LDS at once.
constexpr int kNrThreads = 1024;
constexpr int kNrWaves = kNrThreads / kWave;
constexpr int kNrMaxD = 4096;
constexpr int kNrMaxE = 16;
constexpr int kNrMaxG = kNrMaxD / 32;
__global__ __launch_bounds__(kNrThreads) void k_moe_norm_route(MoeArgs a) {
    constexpr int PER = kNrMaxD / kNrThreads, RW = kNrMaxE / kNrWaves, JG = kNrMaxG / kWave;
    __shared__ __align__(16) uint16_t xs[kNrMaxD];  // pair-major: [pair m of the group][group g]
    __shared__ float red[kNrWaves];
    __shared__ float inv_s;
    __shared__ float lg[kMoeMaxBatch * kNrMaxE];
    __shared__ int32_t sid[kMoeMaxBatch * kMoeMaxTopK];
    __shared__ float sw[kMoeMaxBatch * kMoeMaxTopK];
    __shared__ int scnt[kNrMaxE], srank[kNrMaxE];
    __shared__ int last;
    // the arguments the prologue uses, requested in one round
    asm volatile("" ::"s"(a.h), "s"(a.wr), "s"(a.sr), "s"(a.d), "s"(a.batch), "s"(a.E), "s"(a.norm_w),
                 "s"(a.xn16), "s"(a.eps));
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(tid >> 6), b = blockIdx.x;
    const int d = a.d, B = a.batch, E = a.E, G = d / 32;
    const float* hb = a.h + (size_t)b * d;
    float hv[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) hv[j] = hb[min(tid + kNrThreads * j, d - 1)];
    uint4 wc[RW][JG];
    uint16_t wsc[RW][JG];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int j = 0; j < JG; ++j) {
            const int e = min(wave + kNrWaves * r, E - 1), g = min(lane + kWave * j, G - 1);
            wc[r][j] = *reinterpret_cast<const uint4*>(a.wr + ((size_t)e * G + g) * 16);
            wsc[r][j] = a.sr[(size_t)e * G + g];
        }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; ++j) ss += tid + kNrThreads * j < d ? hv[j] * hv[j] : 0.0f;
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    if (tid == 0) {
        float t = 0.0f;
        for (int w = 0; w < kNrWaves; ++w) t += red[w];
        inv_s = 1.0f / sqrtf(t / (float)d + a.eps);
    }
    __syncthreads();
    const float inv = inv_s;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int i = tid + kNrThreads * j;
        if (i < d) {
            const float x = hv[j] * inv;
            const uint16_t u = f2h_bits(a.norm_w ? x * a.norm_w[i] : x);
            // the router's lanes (consecutive groups) read consecutive words
            xs[(((i >> 1) & 15) * G + (i >> 5)) * 2 + (i & 1)] = u;
            a.xn16[(size_t)b * d + i] = u;
        }
    }
    __syncthreads();
    // router logits: y[e] = sum_g s_g * sum_k (q_k - 8) x[32g + k]
    const uint32_t* xw = reinterpret_cast<const uint32_t*>(xs);
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const int e = wave + kNrWaves * r;
        if (e >= E) continue;
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < JG; ++j) {
            const int g = lane + kWave * j;
            if (g < G) {
                const uint32_t cw[4] = {wc[r][j].x, wc[r][j].y, wc[r][j].z, wc[r][j].w};
                float dot = 0.0f;
#pragma unroll
                for (int m = 0; m < 16; ++m) {
                    // x pair (2m, 2m+1) meets the low and high nibble of byte m
                    const uint32_t byte = (cw[m >> 2] >> (8 * (m & 3))) & 0xFFu, xp = xw[m * G + g];
                    dot = fmaf((float)(int)(byte & 15u) - 8.0f, h2f_bits((uint16_t)(xp & 0xFFFFu)), dot);
                    dot = fmaf((float)(int)(byte >> 4) - 8.0f, h2f_bits((uint16_t)(xp >> 16)), dot);
                }
                acc = fmaf(dot, h2f_bits(wsc[r][j]), acc);
            }
        }
        acc = wave_sum(acc);
        if (lane == 0) {
            __hip_atomic_store(a.logits + (size_t)b * E + e, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            lg[b * E + e] = acc;  // batch 1: the routing reads them here
        }
    }
    if (B > 1) {
        // this block's logits are stored before it counts itself
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0) {
            const unsigned prev = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = prev == (unsigned)B - 1u;
            if (last) __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!last) return;
        for (int idx = tid; idx < B * E; idx += kNrThreads)
            lg[idx] = __hip_atomic_load(a.logits + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (wave < B) route_wave(lg + wave * E, E, a.k, sid + wave * a.k, sw + wave * a.k);
    __syncthreads();
    if (tid < B * a.k) {
        a.ids[tid] = sid[tid];
        a.weights[tid] = sw[tid];
    }
    build_lists(a, sid, scnt, srank);
}

// kparts > 0: slot s's down projection is the sum, in part order, of the K
// parts kpart[q][s] instead of y32[s].
__global__ void k_moe_combine(const float* y32, const float* kpart, int kparts, const float* weights, float* out,
                              int d, int k, int batch, int accumulate) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= batch * d) return;
    const int b = t / d, i = t % d;
    float acc = 0.0f;
    for (int j = 0; j < k; ++j) {
        const size_t s = (size_t)b * k + j;
        float y;
        if (kparts > 0) {
            y = 0.0f;
            for (int q = 0; q < kparts; ++q) y += kpart[((size_t)q * batch * k + s) * d + i];
        } else {
            y = y32[s * d + i];
        }
        acc += weights[s] * y;
    }
    out[t] = accumulate ? out[t] + acc : acc;
}

// The combine of k_moe_combine (accumulate into h, the same sums in the same
// order), then the RMSNorm of each finished row with weights w (nullptr =
// ones) into x16, the input of the next RMSNorm-input GEMV: one block per
// sequence, 16-byte chunks (d % 4 == 0, d <= 4 * kCnThreads * kCnChunks).
constexpr int kCnThreads = 1024, kCnChunks = 4;
__global__ __launch_bounds__(kCnThreads) void k_moe_combine_norm(const float* y32, const float* kpart, int kparts,
                                                                 const float* weights, float* h, int d, int k,
                                                                 int batch, const float* w, uint16_t* x16,
                                                                 float eps) {
    __shared__ float red[kCnThreads / 64];
    const int b = blockIdx.x, t = threadIdx.x, nc = d / 4;
    float4 v[kCnChunks];
    float ss = 0.0f;
#pragma unroll
    for (int jc = 0; jc < kCnChunks; ++jc) {
        const int c = t + jc * kCnThreads;
        v[jc] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (c >= nc) continue;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int j = 0; j < k; ++j) {
            const size_t sl = (size_t)b * k + j;
            float4 y;
            if (kparts > 0) {
                y = make_float4(0.f, 0.f, 0.f, 0.f);
                for (int q = 0; q < kparts; ++q) {
                    const float4 p = reinterpret_cast<const float4*>(kpart + ((size_t)q * batch * k + sl) * d)[c];
                    y.x += p.x;
                    y.y += p.y;
                    y.z += p.z;
                    y.w += p.w;
                }
            } else {
                y = reinterpret_cast<const float4*>(y32 + sl * d)[c];
            }
            const float ws = weights[sl];
            acc.x += ws * y.x;
            acc.y += ws * y.y;
            acc.z += ws * y.z;
            acc.w += ws * y.w;
        }
        float4* hp = reinterpret_cast<float4*>(h + (size_t)b * d) + c;
        const float4 o = *hp;
        const float4 r = make_float4(o.x + acc.x, o.y + acc.y, o.z + acc.z, o.w + acc.w);
        *hp = r;
        v[jc] = r;
        ss += r.x * r.x + r.y * r.y + r.z * r.z + r.w * r.w;
    }
    ss = wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kCnThreads / 64; ++i) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / (float)d + eps);
    uint2* ob = reinterpret_cast<uint2*>(x16 + (size_t)b * d);
#pragma unroll
    for (int jc = 0; jc < kCnChunks; ++jc) {
        const int c = t + jc * kCnThreads;
        if (c >= nc) break;
        const float4 wv = w ? reinterpret_cast<const float4*>(w)[c] : make_float4(1.f, 1.f, 1.f, 1.f);
        const uint32_t lo = (uint32_t)f2h_bits(v[jc].x * inv * wv.x) | ((uint32_t)f2h_bits(v[jc].y * inv * wv.y) << 16);
        const uint32_t hi = (uint32_t)f2h_bits(v[jc].z * inv * wv.z) | ((uint32_t)f2h_bits(v[jc].w * inv * wv.w) << 16);
        ob[c] = make_uint2(lo, hi);
    }
}

inline dim3 grid1(size_t n, int threads) { return dim3((unsigned)((n + threads - 1) / threads)); }

// Prefill routing of n tokens (logits [n][E]): each token routed as a decode
// step routes it (route_row), then the token slots (t, j) grouped by expert
// in (t, j) order: expert e's rows are off[e] .. off[e] + cnt[e] - 1 of the
// gathered buffers, row r holding token row_tok[r]; slot_row[t * k + j] is
// the row of slot (t, j).  counts: cnt[E] then off[E].  One block.
constexpr int kPfRouteThreads = 256;
__global__ __launch_bounds__(kPfRouteThreads) void k_pf_route(const float* logits, int n, int E, int k, int32_t* ids,
                                                              float* w, int32_t* row_tok, int32_t* slot_row,
                                                              int32_t* counts) {
    __shared__ uint32_t tk[kPfRouteThreads][kMoeMaxExperts / 32];
    __shared__ int sid[kPfRouteThreads][kMoeMaxTopK];
    __shared__ float sw[kPfRouteThreads][kMoeMaxTopK];
    __shared__ int cnt[kMoeMaxExperts], off[kMoeMaxExperts];
    const int tid = threadIdx.x;
    for (int t = tid; t < n; t += kPfRouteThreads) {
        route_row(logits + (size_t)t * E, E, k, sid[tid], sw[tid], tk[tid]);
        for (int j = 0; j < k; ++j) {
            ids[(size_t)t * k + j] = sid[tid][j];
            w[(size_t)t * k + j] = sw[tid][j];
        }
    }
    __syncthreads();
    if (tid != 0) return;
    for (int e = 0; e < E; ++e) cnt[e] = 0;
    for (int s = 0; s < n * k; ++s) cnt[ids[s]] += 1;
    int acc = 0;
    for (int e = 0; e < E; ++e) {
        off[e] = acc;
        acc += cnt[e];
        counts[e] = cnt[e];
        counts[E + e] = off[e];
        cnt[e] = 0;
    }
    for (int s = 0; s < n * k; ++s) {
        const int e = ids[s], r = off[e] + cnt[e];
        cnt[e] += 1;
        row_tok[r] = s / k;
        slot_row[s] = r;
    }
}

// xg[r] = x16[row_tok[r]] (fp16 rows of d, d % 8 == 0), 8 elements a thread.
__global__ __launch_bounds__(256) void k_pf_gather(const uint16_t* x16, const int32_t* row_tok, int rows, int d,
                                                   uint16_t* xg) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x, per = d / 8;
    if (i >= (long)rows * per) return;
    const int r = (int)(i / per), c = (int)(i % per);
    reinterpret_cast<uint4*>(xg + (size_t)r * d)[c] = reinterpret_cast<const uint4*>(x16 + (size_t)row_tok[r] * d)[c];
}

// h[t] += sum_j w[t][j] * yg[slot_row[t * k + j]] (the decode combine's order).
__global__ void k_pf_moe_combine(const float* yg, const int32_t* slot_row, const float* w, int n, int k, int d,
                                 float* h) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)n * d) return;
    const int t = (int)(i / d), c = (int)(i % d);
    float acc = 0.0f;
    for (int j = 0; j < k; ++j) acc += w[(size_t)t * k + j] * yg[(size_t)slot_row[(size_t)t * k + j] * d + c];
    h[i] = h[i] + acc;
}

}  // namespace

hipError_t rmsnorm_launch(const float* x, const float* w, uint16_t* out, int dim, float eps,
                          int batch, hipStream_t st) {
    const bool vec = dim % 4 == 0 && dim <= 4 * kNormThreads * kNormChunks &&
                     ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                       reinterpret_cast<uintptr_t>(out)) & 15u) == 0;
    if (vec)
        hipLaunchKernelGGL(k_rmsnorm_vec, dim3(batch), dim3(kNormThreads), 0, st, x, w, out, dim, eps);
    else
        hipLaunchKernelGGL(k_rmsnorm, dim3(batch), dim3(256), 0, st, x, w, out, dim, eps);
    return hipGetLastError();
}

hipError_t rope_launch(float* x, const int32_t* pos, const float* cos_t, const float* sin_t,
                       int heads, int hd, int batch, hipStream_t st) {
    const size_t n = (size_t)batch * heads * (hd / 2);
    hipLaunchKernelGGL(k_rope, grid1(n, 256), dim3(256), 0, st, x, pos, cos_t, sin_t, heads, hd,
                       batch);
    return hipGetLastError();
}

hipError_t qk_norm_rope_launch(const QknArgs& a, int batch, hipStream_t st) {
    if (a.hd < 2 || a.hd > 256 || a.hd % 2 || a.hq < 1 || a.hkv < 1 || batch < 1 || !a.q32 || !a.kv_tmp ||
        !a.cos_t || !a.sin_t || !a.pos || (a.kpool && (!a.vpool || !a.block_table)))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_qk_norm_rope, dim3(a.hq + 2 * a.hkv, batch), dim3(64), 0, st, a);
    return hipGetLastError();
}

hipError_t head_rmsnorm_launch(float* q, int ldq, float* k, int ldk, int rows, int hq, int hkv, int hd,
                               const float* qn, const float* kn, float eps, hipStream_t st) {
    if (hd < 1 || hd > 256 || hq < 1 || hkv < 1 || rows < 0) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(k_head_rmsnorm, dim3(hq + hkv, rows), dim3(64), 0, st, q, ldq, k, ldk, hq, hd, qn, kn, eps);
    return hipGetLastError();
}

hipError_t swiglu_launch(const float* g, const float* u, uint16_t* out, int n, int batch,
                         hipStream_t st) {
    const size_t total = (size_t)n * batch;
    hipLaunchKernelGGL(k_swiglu, grid1(total, 256), dim3(256), 0, st, g, u, out, total);
    return hipGetLastError();
}

hipError_t residual_add_launch(const float* a, const float* b, float* out, int n, hipStream_t st) {
    hipLaunchKernelGGL(k_residual_add, grid1(n, 256), dim3(256), 0, st, a, b, out, n);
    return hipGetLastError();
}

hipError_t kv_append_f16_launch(const float* k, const float* v, uint16_t* kpool, uint16_t* vpool,
                                const int32_t* block_table, const int32_t* pos, int batch,
                                int hkv, int hd, int max_blocks, hipStream_t st) {
    const size_t n = (size_t)batch * hkv * hd;
    hipLaunchKernelGGL(k_kv_append_f16, grid1(n, 256), dim3(256), 0, st, k, v, kpool, vpool,
                       block_table, pos, batch, hkv, hd, max_blocks);
    return hipGetLastError();
}

hipError_t argmax_launch(const float* logits, int32_t* out, int V, int batch, hipStream_t st) {
    hipLaunchKernelGGL(k_argmax, dim3(batch), dim3(256), 0, st, logits, out, V);
    return hipGetLastError();
}

hipError_t unpack_int4_launch(const uint8_t* packed, uint8_t* codes, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_unpack_int4, grid1(n, 256), dim3(256), 0, st, packed, codes, n);
    return hipGetLastError();
}

hipError_t quantize_int4_launch(const float* w, uint8_t* codes, uint16_t* scales, int N, int K,
                                hipStream_t st) {
    const size_t n = (size_t)N * ((K + 31) / 32);
    hipLaunchKernelGGL(k_quantize_int4, grid1(n, 256), dim3(256), 0, st, w, codes, scales, N, K);
    return hipGetLastError();
}

hipError_t gen_quant_launch(uint8_t* codes, uint16_t* scales, int N, int K, uint64_t seed,
                            uint32_t tid, float k, int row_offset, int row_stride,
                            hipStream_t st) {
    const size_t n = (size_t)N * ((K + 31) / 32);
    hipLaunchKernelGGL(k_gen_quant, grid1(n, 256), dim3(256), 0, st, codes, scales, N, K,
                       stream_key(seed, tid), k, row_offset, row_stride);
    return hipGetLastError();
}

hipError_t gen_f16_launch(uint16_t* out, size_t n, uint64_t seed, uint32_t tid, float k,
                          hipStream_t st) {
    hipLaunchKernelGGL(k_gen_f16, grid1(n, 256), dim3(256), 0, st, out, n, stream_key(seed, tid), k);
    return hipGetLastError();
}

hipError_t gen_ctx_f16_launch(uint16_t* kpool, uint16_t* vpool, const int32_t* block_table,
                              int max_blocks, int batch, int ctx, int hkv, int hd, int L,
                              uint64_t seed, float k, const int32_t* outlier_ch, int n_outlier,
                              hipStream_t st) {
    const size_t n = (size_t)batch * ctx * 2 * hkv * hd;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_gen_ctx_f16, grid1(n, 256), dim3(256), 0, st, kpool, vpool, block_table,
                       max_blocks, batch, ctx, hkv, hd, L, seed, k, outlier_ch, n_outlier);
    return hipGetLastError();
}

hipError_t gen_ctx_raw_launch(float* dst, int ctx, int hkv, int hd, int L, int b, int kv,
                              uint64_t seed, float k, const int32_t* outlier_ch, int n_outlier,
                              hipStream_t st) {
    const size_t n = (size_t)ctx * hkv * hd;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_gen_ctx_raw, grid1(n, 256), dim3(256), 0, st, dst, ctx, hkv, hd,
                       stream_key(seed, tid_ctx(L, b, kv)), k, outlier_ch, n_outlier);
    return hipGetLastError();
}

hipError_t embed_launch(unsigned long long* best, int32_t* pos, const int32_t* base,
                        int32_t* out_tokens, int out_stride, const uint16_t* embed, float* h,
                        int d, int vocab, int batch, hipStream_t st, const int32_t* feed,
                        const int32_t* fpos) {
    hipLaunchKernelGGL(k_embed, dim3(batch), dim3(256), 0, st, best, pos, base, out_tokens,
                       out_stride, embed, h, d, vocab, feed, fpos);
    return hipGetLastError();
}

hipError_t finish_tokens_launch(const unsigned long long* best, const int32_t* pos,
                                const int32_t* base, int32_t* out_tokens, int out_stride,
                                int batch, hipStream_t st) {
    hipLaunchKernelGGL(k_finish_tokens, dim3(1), dim3(64), 0, st, best, pos, base, out_tokens,
                       out_stride, batch);
    return hipGetLastError();
}

hipError_t set_tokens_launch(unsigned long long* best, const int32_t* tokens, int batch,
                             hipStream_t st) {
    hipLaunchKernelGGL(k_set_tokens, dim3(1), dim3(64), 0, st, best, tokens, batch);
    return hipGetLastError();
}

bool moe_norm_route_fits(int d, int E, int k, int batch) {
    // whole 32-element groups, so the router's last group reads no x past its row
    return batch >= 1 && batch <= kMoeMaxBatch && E >= 1 && E <= kNrMaxE && k >= 1 && k <= kMoeMaxTopK && k <= E &&
           d >= 32 &&
           d % 32 == 0 && d <= kNrMaxD;
}

hipError_t moe_norm_route_launch(const MoeArgs& a, hipStream_t st) {
    if (!moe_norm_route_fits(a.d, a.E, a.k, a.batch) || !a.h || !a.wr || !a.sr || !a.xn16 || !a.logits ||
        (a.batch > 1 && !a.counter))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_moe_norm_route, dim3(a.batch), dim3(kNrThreads), 0, st, a);
    return hipGetLastError();
}

hipError_t moe_route_launch(const MoeArgs& a, hipStream_t st) {
    if (a.batch < 1 || a.batch > 64 || a.E < 1 || a.E > kMoeMaxExperts || a.k < 1 || a.k > kMoeMaxTopK || a.k > a.E)
        return hipErrorInvalidValue;
    if (a.plan && a.batch > kMoePlanMaxSlots) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_moe_route, dim3(1), dim3(64), 0, st, a);
    return hipGetLastError();
}

hipError_t pf_route_launch(const float* logits, int n, int E, int k, int32_t* ids, float* w, int32_t* row_tok,
                           int32_t* slot_row, int32_t* counts, hipStream_t st) {
    if (n < 1 || E < 1 || E > kMoeMaxExperts || k < 1 || k > kMoeMaxTopK || k > E) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pf_route, dim3(1), dim3(kPfRouteThreads), 0, st, logits, n, E, k, ids, w, row_tok, slot_row,
                       counts);
    return hipGetLastError();
}

hipError_t pf_gather_launch(const uint16_t* x16, const int32_t* row_tok, int rows, int d, uint16_t* xg,
                            hipStream_t st) {
    if (d % 8 || rows < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pf_gather, grid1((size_t)rows * (d / 8), 256), dim3(256), 0, st, x16, row_tok, rows, d, xg);
    return hipGetLastError();
}

hipError_t pf_moe_combine_launch(const float* yg, const int32_t* slot_row, const float* w, int n, int k, int d,
                                 float* h, hipStream_t st) {
    hipLaunchKernelGGL(k_pf_moe_combine, grid1((size_t)n * d, 256), dim3(256), 0, st, yg, slot_row, w, n, k, d, h);
    return hipGetLastError();
}

bool moe_combine_norm_fits(const MoeFfnArgs& a) {
    return a.accumulate && a.d % 4 == 0 && a.d <= 4 * kCnThreads * kCnChunks &&
           (reinterpret_cast<uintptr_t>(a.out) & 15u) == 0 && (reinterpret_cast<uintptr_t>(a.y32) & 15u) == 0 &&
           (!a.kpart || (reinterpret_cast<uintptr_t>(a.kpart) & 15u) == 0);
}

hipError_t moe_combine_norm_launch(const MoeFfnArgs& a, const float* w, uint16_t* x16, float eps, hipStream_t st) {
    if (!moe_combine_norm_fits(a) || !x16) return hipErrorInvalidValue;
    const int kparts = moe_down_split(a) ? gemv_kparts(a.F, a.batch) : 0;
    hipLaunchKernelGGL(k_moe_combine_norm, dim3(a.batch), dim3(kCnThreads), 0, st, a.y32, a.kpart, kparts, a.weights,
                       a.out, a.d, a.k, a.batch, w, x16, eps);
    return hipGetLastError();
}

hipError_t moe_combine_launch(const MoeFfnArgs& a, hipStream_t st) {
    const size_t n = (size_t)a.batch * a.d;
    const int kparts = moe_down_split(a) ? gemv_kparts(a.F, a.batch) : 0;
    hipLaunchKernelGGL(k_moe_combine, grid1(n, 256), dim3(256), 0, st, a.y32, a.kpart, kparts, a.weights, a.out,
                       a.d, a.k, a.batch, a.accumulate);
    return hipGetLastError();
}

}  // namespace nx
