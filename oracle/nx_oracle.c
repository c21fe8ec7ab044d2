/*
 * CPU oracle for the NEXUS per-token decode loop -- TEST INFRASTRUCTURE ONLY.
 * Loaded by the tests, the smoke check and the CPU-baseline leg of the
 * benchmark; never by the product library.  See nx_oracle.h for the
 * definitions and the reference lines each function restates.
 */
#include "nx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ RNG -- */
#define G1 0x9E3779B97F4A7C15ull
#define G2 0xD1B54A32D192ED03ull

static inline uint64_t fmix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint64_t stream_key(uint64_t seed, uint32_t tensor) {
    return fmix64(fmix64(seed + G1) + (uint64_t)tensor * G2);
}

uint64_t nxo_rand_u64(uint64_t seed, uint32_t tensor, uint64_t index) {
    return fmix64(stream_key(seed, tensor) + (index + 1) * G1);
}

float nxo_normal_k(double sigma) {
    return (float)(sigma / (2.0 * sqrt((65536.0 * 65536.0 - 1.0) / 3.0)));
}

float nxo_normal_from_u64(uint64_t r, float k) {
    int32_t s = (int32_t)(r & 0xFFFFu) + (int32_t)((r >> 16) & 0xFFFFu) +
                (int32_t)((r >> 32) & 0xFFFFu) + (int32_t)(r >> 48);
    return (float)(2 * s - 262140) * k;
}

void nxo_gen_normal(float* out, size_t n, uint64_t seed, uint32_t tensor, float k) {
    const uint64_t key = stream_key(seed, tensor);
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i)
        out[i] = nxo_normal_from_u64(fmix64(key + ((uint64_t)i + 1) * G1), k);
}

void nxo_gen_tokens(int32_t* out, int n, uint64_t seed, uint32_t tensor, int vocab) {
    for (int i = 0; i < n; ++i)
        out[i] = (int32_t)(nxo_rand_u64(seed, tensor, (uint64_t)i) % (uint64_t)vocab);
}

void nxo_shuffle_perm(int32_t* perm, int n, uint64_t seed, uint32_t tensor) {
    for (int i = 0; i < n; ++i) perm[i] = i;
    for (int i = n - 1; i >= 1; --i) {
        int j = (int)(nxo_rand_u64(seed, tensor, (uint64_t)i) % (uint64_t)(i + 1));
        int32_t t = perm[i];
        perm[i] = perm[j];
        perm[j] = t;
    }
}

/* ---------------------------------------------------------------- fp16 -- */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t nxo_f32_to_f16(float f) {
    const uint32_t x = f2u(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);      /* >= 65520 -> inf */
    if (ax < 0x38800000u) {                                         /* |f| < 2^-14 */
        if (ax < 0x33000000u) return (uint16_t)sign;                /* < 2^-25 -> 0 */
        const uint32_t e = ax >> 23;
        const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e;                            /* 14..24 */
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return (uint16_t)(sign | r);
    }
    uint32_t r = (ax >> 13) - (112u << 10);
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}

float nxo_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    const uint32_t m = (uint32_t)h & 0x3FFu;
    if (e == 0) {
        const float v = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7F800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t nxo_f32_to_f16_trunc(float f) {
    const uint32_t x = f2u(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int exp = (int)((x >> 23) & 0xFFu) - 127 + 15;
    const uint32_t mant = (x >> 13) & 0x3FFu;
    if (exp <= 0) return (uint16_t)sign;
    if (exp >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)exp << 10) | mant);
}

float nxo_f16_to_f32_ref(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t exp = ((uint32_t)h >> 10) & 0x1Fu;
    const uint32_t mant = (uint32_t)h & 0x3FFu;
    if (exp == 0) return u2f(sign);
    if (exp == 31) return u2f(sign | 0x7F800000u | (mant << 13));
    return u2f(sign | ((exp + 112u) << 23) | (mant << 13));
}

void nxo_f32_to_f16_array(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = nxo_f32_to_f16(in[i]);
}

void nxo_f16_to_f32_array(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = nxo_f16_to_f32(in[i]);
}

static inline float round_f16(float f) { return nxo_f16_to_f32(nxo_f32_to_f16(f)); }

/* ---------------------------------------------------------- int4 g32 ---- */
void nxo_quantize_int4_g32(const float* w, int N, int K, uint8_t* codes, uint16_t* scales) {
    const int G = (K + 31) / 32;
    const int rowbytes = G * 16;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n) {
        const float* row = w + (size_t)n * K;
        uint8_t* crow = codes + (size_t)n * rowbytes;
        for (int g = 0; g < G; ++g) {
            const int k0 = g * 32;
            const int k1 = k0 + 32 < K ? k0 + 32 : K;
            float amax = 0.0f;
            for (int k = k0; k < k1; ++k) {
                const float a = fabsf(row[k]);
                if (a > amax) amax = a;
            }
            const uint16_t s16 = nxo_f32_to_f16(amax / 7.0f);
            const float s = nxo_f16_to_f32(s16);
            scales[(size_t)n * G + g] = s16;
            uint8_t q[32];
            for (int j = 0; j < 32; ++j) {
                const int k = k0 + j;
                int v = 8;
                if (k < k1 && s != 0.0f) {
                    int r = (int)roundf(row[k] / s);
                    if (r < -8) r = -8;
                    if (r > 7) r = 7;
                    v = r + 8;
                }
                q[j] = (uint8_t)v;
            }
            for (int j = 0; j < 16; ++j)
                crow[g * 16 + j] = (uint8_t)(q[2 * j] | (q[2 * j + 1] << 4));
        }
    }
}

void nxo_gen_quant_rows(int n0, int count, int K, uint64_t seed, uint32_t tensor, double sigma,
                        uint8_t* codes, uint16_t* scales) {
    const uint64_t key = stream_key(seed, tensor);
    const float k = nxo_normal_k(sigma);
    float* w = (float*)malloc(sizeof(float) * (size_t)count * K);
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)count * K; ++i) {
        const uint64_t idx = (uint64_t)n0 * (uint64_t)K + (uint64_t)i;
        w[i] = nxo_normal_from_u64(fmix64(key + (idx + 1) * G1), k);
    }
    nxo_quantize_int4_g32(w, count, K, codes, scales);
    free(w);
}

void nxo_unpack_int4(const uint8_t* packed, size_t n, uint8_t* codes) {
    for (size_t i = 0; i < n; i += 2) {
        const uint8_t b = packed[i / 2];
        codes[i] = b & 0x0F;
        if (i + 1 < n) codes[i + 1] = (b >> 4) & 0x0F;
    }
}

void nxo_dequant_int4_g32(const uint8_t* codes, const uint16_t* scales, int N, int K, float* w) {
    const int G = (K + 31) / 32;
    for (int n = 0; n < N; ++n) {
        const uint8_t* crow = codes + (size_t)n * G * 16;
        for (int k = 0; k < K; ++k) {
            const uint8_t b = crow[k / 2];
            const int q = (k & 1) ? (b >> 4) : (b & 0x0F);
            w[(size_t)n * K + k] = (float)(q - 8) * nxo_f16_to_f32(scales[(size_t)n * G + k / 32]);
        }
    }
}

void nxo_gemv_int4_g32(const uint8_t* codes, const uint16_t* scales, const float* x,
                       int N, int K, int B, float* y) {
    const int G = (K + 31) / 32;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n) {
        const uint8_t* crow = codes + (size_t)n * G * 16;
        const uint16_t* srow = scales + (size_t)n * G;
        for (int b = 0; b < B; ++b) {
            const float* xb = x + (size_t)b * K;
            float acc = 0.0f;
            for (int g = 0; g < G; ++g) {
                const float s = nxo_f16_to_f32(srow[g]);
                const int k0 = g * 32;
                const int k1 = k0 + 32 < K ? k0 + 32 : K;
                float part = 0.0f;
                for (int k = k0; k < k1; ++k) {
                    const uint8_t bb = crow[k / 2];
                    const int q = (k & 1) ? (bb >> 4) : (bb & 0x0F);
                    part += (float)(q - 8) * xb[k];
                }
                acc += part * s;
            }
            y[(size_t)b * N + n] = acc;
        }
    }
}

/* ------------------------------------------------------- elementwise ---- */
void nxo_rmsnorm(const float* x, const float* w, int d, float eps, float* out) {
    float ss = 0.0f;
    for (int i = 0; i < d; ++i) ss += x[i] * x[i];
    const float inv = 1.0f / sqrtf(ss / (float)d + eps);
    for (int i = 0; i < d; ++i) out[i] = (x[i] * inv) * (w ? w[i] : 1.0f);
}

void nxo_rope_table(int max_pos, int hd, double theta, float* cos_tab, float* sin_tab) {
    const int half = hd / 2;
    for (int p = 0; p < max_pos; ++p) {
        for (int i = 0; i < half; ++i) {
            const double inv_freq = pow(theta, -(2.0 * i) / (double)hd);
            const double a = (double)p * inv_freq;
            cos_tab[(size_t)p * half + i] = (float)cos(a);
            sin_tab[(size_t)p * half + i] = (float)sin(a);
        }
    }
}

void nxo_rope(float* x, int n_heads, int hd, int pos, const float* cos_tab, const float* sin_tab) {
    const int half = hd / 2;
    const float* c = cos_tab + (size_t)pos * half;
    const float* s = sin_tab + (size_t)pos * half;
    for (int h = 0; h < n_heads; ++h) {
        float* v = x + (size_t)h * hd;
        for (int i = 0; i < half; ++i) {
            const float a = v[2 * i], b = v[2 * i + 1];
            v[2 * i] = a * c[i] - b * s[i];
            v[2 * i + 1] = a * s[i] + b * c[i];
        }
    }
}

void nxo_head_rmsnorm(float* x, int n_heads, int hd, const float* w, float eps) {
    for (int h = 0; h < n_heads; ++h) nxo_rmsnorm(x + (size_t)h * hd, w, hd, eps, x + (size_t)h * hd);
}

void nxo_swiglu(const float* g, const float* u, int n, float* out) {
    for (int i = 0; i < n; ++i) out[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}

int nxo_argmax(const float* v, int n) {
    int best = 0;
    float bv = v[0];
    for (int i = 1; i < n; ++i)
        if (v[i] > bv) { bv = v[i]; best = i; }
    return best;
}

/* ----------------------------------------------------- paged attention -- */
void nxo_kv_append_f16(const float* k, const float* v, uint16_t* kpool, uint16_t* vpool,
                       const int32_t* block_table, int max_blocks, int b, int pos,
                       int hkv, int hd) {
    const int blk = block_table[(size_t)b * max_blocks + pos / NXO_PAGE];
    const int slot = pos % NXO_PAGE;
    for (int h = 0; h < hkv; ++h) {
        const size_t page = ((size_t)blk * hkv + h) * NXO_PAGE * hd;
        for (int d = 0; d < hd; ++d) {
            kpool[page + (size_t)slot * hd + d] = nxo_f32_to_f16(k[(size_t)h * hd + d]);
            vpool[page + (size_t)d * NXO_PAGE + slot] = nxo_f32_to_f16(v[(size_t)h * hd + d]);
        }
    }
}

/* One query head against gathered K/V rows (row t at K + t*stride). */
static void attend_head(const float* qh, const float* K, const float* V, size_t stride,
                        int ctx, int hd, float* out, float* scores) {
    const float scale = 1.0f / sqrtf((float)hd);
    float mx = -1e30f;
    for (int t = 0; t < ctx; ++t) {
        const float* kt = K + (size_t)t * stride;
        float dot = 0.0f;
        for (int d = 0; d < hd; ++d) dot += qh[d] * kt[d];
        scores[t] = dot * scale;
        if (scores[t] > mx) mx = scores[t];
    }
    float sum = 0.0f;
    for (int t = 0; t < ctx; ++t) {
        scores[t] = expf(scores[t] - mx);
        sum += scores[t];
    }
    if (sum > 0.0f)
        for (int t = 0; t < ctx; ++t) scores[t] /= sum;
    for (int d = 0; d < hd; ++d) out[d] = 0.0f;
    for (int t = 0; t < ctx; ++t) {
        const float* vt = V + (size_t)t * stride;
        for (int d = 0; d < hd; ++d) out[d] += scores[t] * vt[d];
    }
}

void nxo_attn_decode_contig(const float* q, const float* K, const float* V, int ctx,
                            int hq, int hkv, int hd, float* out) {
    const int grp = hq / hkv;
    float* scores = (float*)malloc(sizeof(float) * (size_t)(ctx > 0 ? ctx : 1));
    for (int h = 0; h < hq; ++h) {
        const int kvh = h / grp;
        attend_head(q + (size_t)h * hd, K + (size_t)kvh * hd, V + (size_t)kvh * hd,
                    (size_t)hkv * hd, ctx, hd, out + (size_t)h * hd, scores);
    }
    free(scores);
}

/* Gather one kv head of a paged pool into contiguous fp32 rows [ctx][hd]. */
/* Gather positions [0, ctx) of kv head h into dst [ctx][hd]; token-major
 * pages ([16][hd], K) or dimension-major pages ([hd][16], V). */
static void gather_f16(const uint16_t* pool, const int32_t* bt, int ctx, int hkv, int h, int hd,
                       int dim_major, float* dst) {
    for (int t = 0; t < ctx; ++t) {
        const int blk = bt[t / NXO_PAGE], slot = t % NXO_PAGE;
        const uint16_t* page = pool + ((size_t)blk * hkv + h) * NXO_PAGE * hd;
        for (int d = 0; d < hd; ++d)
            dst[(size_t)t * hd + d] =
                nxo_f16_to_f32(dim_major ? page[(size_t)d * NXO_PAGE + slot] : page[(size_t)slot * hd + d]);
    }
}

void nxo_attn_decode_paged_f16(const float* q, const uint16_t* kpool, const uint16_t* vpool,
                               const int32_t* block_table, int max_blocks,
                               const int32_t* ctx_lens, int B, int hq, int hkv, int hd,
                               float* out) {
    const int grp = hq / hkv;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int b = 0; b < B; ++b) {
        for (int kvh = 0; kvh < hkv; ++kvh) {
            const int ctx = ctx_lens[b];
            const int32_t* bt = block_table + (size_t)b * max_blocks;
            float* K = (float*)malloc(sizeof(float) * (size_t)(ctx > 0 ? ctx : 1) * hd);
            float* V = (float*)malloc(sizeof(float) * (size_t)(ctx > 0 ? ctx : 1) * hd);
            float* scores = (float*)malloc(sizeof(float) * (size_t)(ctx > 0 ? ctx : 1));
            gather_f16(kpool, bt, ctx, hkv, kvh, hd, 0, K);
            gather_f16(vpool, bt, ctx, hkv, kvh, hd, 1, V);
            for (int j = 0; j < grp; ++j) {
                const int h = kvh * grp + j;
                attend_head(q + ((size_t)b * hq + h) * hd, K, V, (size_t)hd, ctx, hd,
                            out + ((size_t)b * hq + h) * hd, scores);
            }
            free(K);
            free(V);
            free(scores);
        }
    }
}

/* ----------------------------------------------------------- TurboQuant -- */
static float normal_pdf(float x, float sigma) {
    const float z = x / sigma;
    return expf(-0.5f * z * z) / (sigma * sqrtf(2.0f * (float)M_PI));
}

static float normal_cdf(float x, float sigma) {
    const float z = x / sigma;
    return 0.5f * erfcf(-z * (float)M_SQRT1_2);
}

static float conditional_mean(float a, float b, float sigma) {
    const float pa = normal_pdf(a, sigma);
    const float pb = normal_pdf(b, sigma);
    const float ca = normal_cdf(a, sigma);
    const float cb = normal_cdf(b, sigma);
    const float denom = cb - ca;
    if (denom < 1e-12f) return 0.5f * (a + b);
    return sigma * sigma * (pa - pb) / denom;
}

void nxo_tq_codebook(int d, int bits, float* c, float* bnd) {
    const int n = 1 << bits;
    const float sigma = 1.0f / sqrtf((float)d);
    const float lo = -3.0f * sigma;
    const float hi = 3.0f * sigma;
    for (int i = 0; i < n; ++i) c[i] = lo + (hi - lo) * ((float)i + 0.5f) / (float)n;
    for (int iter = 0; iter < 100; ++iter) {
        for (int i = 0; i < n - 1; ++i) bnd[i] = 0.5f * (c[i] + c[i + 1]);
        float max_delta = 0.0f;
        for (int i = 0; i < n; ++i) {
            const float a = (i == 0) ? -10.0f * sigma : bnd[i - 1];
            const float b = (i == n - 1) ? 10.0f * sigma : bnd[i];
            const float nc = conditional_mean(a, b, sigma);
            const float delta = fabsf(nc - c[i]);
            if (delta > max_delta) max_delta = delta;
            c[i] = nc;
        }
        if (max_delta < 1e-7f * sigma) break;
    }
    for (int i = 0; i < n - 1; ++i) bnd[i] = 0.5f * (c[i] + c[i + 1]);
}

uint8_t nxo_tq_encode_scalar(float x, const float* boundaries, int n_centroids) {
    for (int i = 0; i < n_centroids - 1; ++i)
        if (x < boundaries[i]) return (uint8_t)i;
    return (uint8_t)(n_centroids - 1);
}

void nxo_pack_codes(uint8_t* packed, const uint8_t* codes, int n_codes, int bits) {
    const size_t total_bytes = ((size_t)n_codes * bits + 7) / 8;
    memset(packed, 0, total_bytes);
    uint32_t bit_pos = 0;
    for (int i = 0; i < n_codes; ++i) {
        const uint8_t val = codes[i];
        const uint32_t byte_idx = bit_pos / 8, bit_off = bit_pos % 8;
        packed[byte_idx] |= (uint8_t)(val << bit_off);
        if (bit_off + (uint32_t)bits > 8) packed[byte_idx + 1] |= (uint8_t)(val >> (8 - bit_off));
        bit_pos += (uint32_t)bits;
    }
}

void nxo_unpack_codes(uint8_t* codes, const uint8_t* packed, int n_codes, int bits) {
    const uint8_t mask = (uint8_t)((1u << bits) - 1u);
    uint32_t bit_pos = 0;
    for (int i = 0; i < n_codes; ++i) {
        const uint32_t byte_idx = bit_pos / 8, bit_off = bit_pos % 8;
        uint16_t word = packed[byte_idx];
        if (bit_off + (uint32_t)bits > 8) word |= (uint16_t)(packed[byte_idx + 1] << 8);
        codes[i] = (uint8_t)((word >> bit_off) & mask);
        bit_pos += (uint32_t)bits;
    }
}

void nxo_tq_signs(float* signs, uint64_t seed, uint32_t tensor) {
    for (int i = 0; i < NXO_TQ_D; ++i)
        signs[i] = (nxo_rand_u64(seed, tensor, (uint64_t)i) & 1u) ? -1.0f : 1.0f;
}

float nxo_tq_sumsq(const float* x) {
    float w[64];
    for (int i = 0; i < 64; ++i) {
        const float a = x[i] * x[i];
        const float b = x[i + 64] * x[i + 64];
        w[i] = a + b;
    }
    for (int s = 32; s >= 1; s >>= 1)
        for (int i = 0; i < s; ++i) w[i] = w[i] + w[i + s];
    return w[0];
}

void nxo_fwht128(float* u) {
    for (int h = 1; h < NXO_TQ_D; h <<= 1)
        for (int i = 0; i < NXO_TQ_D; i += 2 * h)
            for (int j = i; j < i + h; ++j) {
                const float a = u[j], b = u[j + h];
                u[j] = a + b;
                u[j + h] = a - b;
            }
}

static const float kTqScale = 0.08838834764831845f; /* float(1/sqrt(128)) */

/* y = H D (x / n) / sqrt(128) of one vector; returns n (y = 0 when n <= 1e-12). */
static float tq_rotate(const float* xv, const float* signs, float* y) {
    const float nrm = sqrtf(nxo_tq_sumsq(xv));
    if (nrm > 1e-12f) {
        const float inv = 1.0f / nrm;
        for (int i = 0; i < NXO_TQ_D; ++i) y[i] = (signs[i] * xv[i]) * inv;
    } else {
        for (int i = 0; i < NXO_TQ_D; ++i) y[i] = 0.0f;
    }
    nxo_fwht128(y);
    for (int i = 0; i < NXO_TQ_D; ++i) y[i] = y[i] * kTqScale;
    return nrm;
}

/* o = ((H u / sqrt(128)) * D) * n: the inverse rotation of codebook values u (overwritten). */
static void tq_unrotate(float* u, uint16_t norm, const float* signs, float* o) {
    nxo_fwht128(u);
    const float nrm = nxo_f16_to_f32(norm);
    for (int i = 0; i < NXO_TQ_D; ++i) o[i] = ((u[i] * kTqScale) * signs[i]) * nrm;
}

void nxo_tq_encode(const float* x, int n, const float* signs, const float* b4, const float* b3,
                   uint8_t* codes4, uint8_t* codes3, uint16_t* norms, uint8_t* codes_unpacked) {
    for (int v = 0; v < n; ++v) {
        float y[NXO_TQ_D];
        norms[v] = nxo_f32_to_f16(tq_rotate(x + (size_t)v * NXO_TQ_D, signs, y));
        uint8_t c[NXO_TQ_D];
        for (int i = 0; i < NXO_TQ_D; ++i)
            c[i] = (i < 64) ? nxo_tq_encode_scalar(y[i], b4, 16) : nxo_tq_encode_scalar(y[i], b3, 8);
        nxo_pack_codes(codes4 + (size_t)v * 32, c, 64, 4);
        nxo_pack_codes(codes3 + (size_t)v * 24, c + 64, 64, 3);
        if (codes_unpacked) memcpy(codes_unpacked + (size_t)v * NXO_TQ_D, c, NXO_TQ_D);
    }
}

void nxo_tq_decode(const uint8_t* codes4, const uint8_t* codes3, const uint16_t* norms, int n,
                   const float* signs, const float* c4, const float* c3, float* out) {
    for (int v = 0; v < n; ++v) {
        uint8_t c[NXO_TQ_D];
        nxo_unpack_codes(c, codes4 + (size_t)v * 32, 64, 4);
        nxo_unpack_codes(c + 64, codes3 + (size_t)v * 24, 64, 3);
        float u[NXO_TQ_D];
        for (int i = 0; i < NXO_TQ_D; ++i) u[i] = (i < 64) ? c4[c[i]] : c3[c[i]];
        tq_unrotate(u, norms[v], signs, out + (size_t)v * NXO_TQ_D);
    }
}

void nxo_cool_encode(const float* x, int n, const float* signs, const float* b3, uint8_t* codes,
                     uint16_t* norms) {
    for (int v = 0; v < n; ++v) {
        float y[NXO_TQ_D];
        norms[v] = nxo_f32_to_f16(tq_rotate(x + (size_t)v * NXO_TQ_D, signs, y));
        uint8_t c[NXO_TQ_D];
        for (int i = 0; i < NXO_TQ_D; ++i) c[i] = nxo_tq_encode_scalar(y[i], b3, 8);
        nxo_pack_codes(codes + (size_t)v * NXO_COOL_CODES, c, NXO_TQ_D, 3);
    }
}

void nxo_cool_decode(const uint8_t* codes, const uint16_t* norms, int n, const float* signs, const float* c3,
                     float* out) {
    for (int v = 0; v < n; ++v) {
        uint8_t c[NXO_TQ_D];
        nxo_unpack_codes(c, codes + (size_t)v * NXO_COOL_CODES, NXO_TQ_D, 3);
        float u[NXO_TQ_D];
        for (int i = 0; i < NXO_TQ_D; ++i) u[i] = c3[c[i]];
        tq_unrotate(u, norms[v], signs, out + (size_t)v * NXO_TQ_D);
    }
}

void nxo_tq_to_cool(const uint8_t* codes4, const uint8_t* codes3, const uint16_t* norms, int n, const float* signs,
                    const float* c4, const float* c3, const float* b3, uint8_t* cool, uint16_t* cool_norms) {
    for (int v = 0; v < n; ++v) {
        float x[NXO_TQ_D];
        nxo_tq_decode(codes4 + (size_t)v * 32, codes3 + (size_t)v * 24, norms + v, 1, signs, c4, c3, x);
        nxo_cool_encode(x, 1, signs, b3, cool + (size_t)v * NXO_COOL_CODES, cool_norms + v);
    }
}

void nxo_tq_append(const float* k, const float* v, int hkv,
                   const float* ksigns, const float* vsigns,
                   const float* b4, const float* b3,
                   uint8_t* kc4, uint8_t* kc3, uint16_t* kn,
                   uint8_t* vc4, uint8_t* vc3, uint16_t* vn,
                   const int32_t* block_table, int max_blocks, int b, int pos) {
    const int blk = block_table[(size_t)b * max_blocks + pos / NXO_PAGE];
    const int slot = pos % NXO_PAGE;
    for (int h = 0; h < hkv; ++h) {
        const size_t vi = ((size_t)blk * hkv + h) * NXO_PAGE + slot;
        nxo_tq_encode(k + (size_t)h * NXO_TQ_D, 1, ksigns, b4, b3, kc4 + vi * 32, kc3 + vi * 24,
                      kn + vi, NULL);
        nxo_tq_encode(v + (size_t)h * NXO_TQ_D, 1, vsigns, b4, b3, vc4 + vi * 32, vc3 + vi * 24,
                      vn + vi, NULL);
    }
}

void nxo_attn_decode_paged_tq(const float* q,
                              const uint8_t* kc4, const uint8_t* kc3, const uint16_t* kn,
                              const uint8_t* vc4, const uint8_t* vc3, const uint16_t* vn,
                              const float* ksigns, const float* vsigns,
                              const float* c4, const float* c3,
                              const int32_t* block_table, int max_blocks,
                              const int32_t* ctx_lens, int B, int hq, int hkv, float* out) {
    const int hd = NXO_TQ_D;
    const int grp = hq / hkv;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int b = 0; b < B; ++b) {
        for (int kvh = 0; kvh < hkv; ++kvh) {
            const int ctx = ctx_lens[b];
            const int32_t* bt = block_table + (size_t)b * max_blocks;
            const size_t rows = (size_t)(ctx > 0 ? ctx : 1);
            float* K = (float*)malloc(sizeof(float) * rows * hd);
            float* V = (float*)malloc(sizeof(float) * rows * hd);
            float* scores = (float*)malloc(sizeof(float) * rows);
            for (int t = 0; t < ctx; ++t) {
                const size_t vi = ((size_t)bt[t / NXO_PAGE] * hkv + kvh) * NXO_PAGE + t % NXO_PAGE;
                nxo_tq_decode(kc4 + vi * 32, kc3 + vi * 24, kn + vi, 1, ksigns, c4, c3,
                              K + (size_t)t * hd);
                nxo_tq_decode(vc4 + vi * 32, vc3 + vi * 24, vn + vi, 1, vsigns, c4, c3,
                              V + (size_t)t * hd);
            }
            for (int j = 0; j < grp; ++j) {
                const int h = kvh * grp + j;
                attend_head(q + ((size_t)b * hq + h) * hd, K, V, (size_t)hd, ctx, hd,
                            out + ((size_t)b * hq + h) * hd, scores);
            }
            free(K);
            free(V);
            free(scores);
        }
    }
}

/* Tiered pages: see nx_oracle.h. */
void nxo_tiered_append(const float* k, const float* v, int hkv, const float* ksigns, const float* vsigns,
                       const float* b4, const float* b3, uint16_t* kpool, uint16_t* vpool, uint8_t* kc4,
                       uint8_t* kc3, uint16_t* kn, uint8_t* vc4, uint8_t* vc3, uint16_t* vn,
                       const int32_t* block_table, int max_blocks, int b, int pos) {
    const size_t n = (size_t)hkv * NXO_TQ_D;
    float* r = (float*)malloc(sizeof(float) * 2 * n);
    for (size_t i = 0; i < n; ++i) {
        r[i] = round_f16(k[i]);
        r[n + i] = round_f16(v[i]);
    }
    nxo_kv_append_f16(r, r + n, kpool, vpool, block_table, max_blocks, b, pos, hkv, NXO_TQ_D);
    nxo_tq_append(r, r + n, hkv, ksigns, vsigns, b4, b3, kc4, kc3, kn, vc4, vc3, vn, block_table, max_blocks,
                  b, pos);
    free(r);
}

int nxo_tiered_cold(int ctx, int hot_window) {
    const int c = ctx - 1 - hot_window;
    return c > 0 ? NXO_PAGE * (c / NXO_PAGE) : 0;
}

int nxo_tiered_cool(int ctx, int hot_window, int warm_window) {
    if (warm_window <= 0) return 0;
    return nxo_tiered_cold(ctx, hot_window + warm_window);
}

int nxo_tiered_evict(int ctx, int hot_window, int warm_window, int cool_window) {
    if (warm_window <= 0 || cool_window <= 0) return 0;
    return nxo_tiered_cold(ctx, hot_window + warm_window + cool_window);
}

void nxo_tiered_append_cool(int hkv, const float* ksigns, const float* vsigns, const float* c4, const float* c3,
                            const float* b3, const uint8_t* kc4, const uint8_t* kc3, const uint16_t* kn,
                            const uint8_t* vc4, const uint8_t* vc3, const uint16_t* vn, uint8_t* kcc,
                            uint16_t* kcn, uint8_t* vcc, uint16_t* vcn, const int32_t* block_table, int max_blocks,
                            int b, int pos) {
    const int blk = block_table[(size_t)b * max_blocks + pos / NXO_PAGE];
    for (int h = 0; h < hkv; ++h) {
        const size_t vi = ((size_t)blk * hkv + h) * NXO_PAGE + pos % NXO_PAGE;
        nxo_tq_to_cool(kc4 + vi * 32, kc3 + vi * 24, kn + vi, 1, ksigns, c4, c3, b3, kcc + vi * NXO_COOL_CODES,
                       kcn + vi);
        nxo_tq_to_cool(vc4 + vi * 32, vc3 + vi * 24, vn + vi, 1, vsigns, c4, c3, b3, vcc + vi * NXO_COOL_CODES,
                       vcn + vi);
    }
}

void nxo_attn_decode_tiered_cool(const float* q, const uint16_t* kpool, const uint16_t* vpool, const uint8_t* kc4,
                                 const uint8_t* kc3, const uint16_t* kn, const uint8_t* vc4, const uint8_t* vc3,
                                 const uint16_t* vn, const uint8_t* kcc, const uint16_t* kcn, const uint8_t* vcc,
                                 const uint16_t* vcn, const float* ksigns, const float* vsigns, const float* c4,
                                 const float* c3, const int32_t* block_table, int max_blocks, const int32_t* ctx_lens,
                                 int hot_window, int warm_window, int B, int hq, int hkv, float* out) {
    nxo_attn_decode_tiered_evict(q, kpool, vpool, kc4, kc3, kn, vc4, vc3, vn, kcc, kcn, vcc, vcn, ksigns, vsigns, c4,
                                 c3, block_table, max_blocks, ctx_lens, hot_window, warm_window, 0, B, hq, hkv, out);
}

void nxo_attn_decode_tiered_evict(const float* q, const uint16_t* kpool, const uint16_t* vpool, const uint8_t* kc4,
                                  const uint8_t* kc3, const uint16_t* kn, const uint8_t* vc4, const uint8_t* vc3,
                                  const uint16_t* vn, const uint8_t* kcc, const uint16_t* kcn, const uint8_t* vcc,
                                  const uint16_t* vcn, const float* ksigns, const float* vsigns, const float* c4,
                                  const float* c3, const int32_t* block_table, int max_blocks,
                                  const int32_t* ctx_lens, int hot_window, int warm_window, int cool_window, int B,
                                  int hq, int hkv, float* out) {
    const int hd = NXO_TQ_D;
    const int grp = hq / hkv;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int b = 0; b < B; ++b) {
        for (int kvh = 0; kvh < hkv; ++kvh) {
            const int ctx = ctx_lens[b], cold = nxo_tiered_cold(ctx, hot_window);
            const int cool = nxo_tiered_cool(ctx, hot_window, warm_window);
            const int evict = nxo_tiered_evict(ctx, hot_window, warm_window, cool_window);
            const int32_t* bt = block_table + (size_t)b * max_blocks;
            const size_t rows = (size_t)(ctx > 0 ? ctx : 1);
            float* K = (float*)malloc(sizeof(float) * rows * hd);
            float* V = (float*)malloc(sizeof(float) * rows * hd);
            float* scores = (float*)malloc(sizeof(float) * rows);
            gather_f16(kpool, bt, ctx, hkv, kvh, hd, 0, K);
            gather_f16(vpool, bt, ctx, hkv, kvh, hd, 1, V);
            for (int t = 0; t < cold; ++t) {
                const size_t vi = ((size_t)bt[t / NXO_PAGE] * hkv + kvh) * NXO_PAGE + t % NXO_PAGE;
                if (t < evict) {  /* evicted: the zero vectors get_vectors gathers */
                    memset(K + (size_t)t * hd, 0, sizeof(float) * hd);
                    memset(V + (size_t)t * hd, 0, sizeof(float) * hd);
                } else if (t < cool) {
                    nxo_cool_decode(kcc + vi * NXO_COOL_CODES, kcn + vi, 1, ksigns, c3, K + (size_t)t * hd);
                    nxo_cool_decode(vcc + vi * NXO_COOL_CODES, vcn + vi, 1, vsigns, c3, V + (size_t)t * hd);
                } else {
                    nxo_tq_decode(kc4 + vi * 32, kc3 + vi * 24, kn + vi, 1, ksigns, c4, c3, K + (size_t)t * hd);
                    nxo_tq_decode(vc4 + vi * 32, vc3 + vi * 24, vn + vi, 1, vsigns, c4, c3, V + (size_t)t * hd);
                }
            }
            for (int j = 0; j < grp; ++j) {
                const int h = kvh * grp + j;
                attend_head(q + ((size_t)b * hq + h) * hd, K, V, (size_t)hd, ctx, hd,
                            out + ((size_t)b * hq + h) * hd, scores);
            }
            free(K);
            free(V);
            free(scores);
        }
    }
}

void nxo_attn_decode_tiered(const float* q, const uint16_t* kpool, const uint16_t* vpool, const uint8_t* kc4,
                            const uint8_t* kc3, const uint16_t* kn, const uint8_t* vc4, const uint8_t* vc3,
                            const uint16_t* vn, const float* ksigns, const float* vsigns, const float* c4,
                            const float* c3, const int32_t* block_table, int max_blocks, const int32_t* ctx_lens,
                            int hot_window, int B, int hq, int hkv, float* out) {
    nxo_attn_decode_tiered_cool(q, kpool, vpool, kc4, kc3, kn, vc4, vc3, vn, NULL, NULL, NULL, NULL, ksigns, vsigns,
                                c4, c3, block_table, max_blocks, ctx_lens, hot_window, 0, B, hq, hkv, out);
}

/* ------------------------------------------------------------------ MoE -- */
void nxo_moe_route(const float* logits, int E, int k, int32_t* ids, float* weights) {
    float p[256];
    int idx[256];
    float mx = logits[0];
    for (int e = 1; e < E; ++e)
        if (logits[e] > mx) mx = logits[e];
    float sum = 0.0f;
    for (int e = 0; e < E; ++e) {
        p[e] = expf(logits[e] - mx);
        sum += p[e];
    }
    if (sum > 0.0f)
        for (int e = 0; e < E; ++e) p[e] /= sum;
    /* selection of the k largest, scanning ids upward with a strict '>' so
     * that equal probabilities keep the lower expert id first */
    unsigned char taken[256] = {0};
    for (int i = 0; i < k; ++i) {
        int best = -1;
        for (int e = 0; e < E; ++e)
            if (!taken[e] && (best < 0 || p[e] > p[best])) best = e;
        taken[best] = 1;
        idx[i] = best;
    }
    float active = 0.0f;
    for (int i = 0; i < k; ++i) active += p[idx[i]];
    for (int i = 0; i < k; ++i) {
        ids[i] = idx[i];
        weights[i] = active > 0.0f ? p[idx[i]] / active : 1.0f / (float)k;
    }
}

/* ---------------------------------------------------------------- model -- */
typedef struct {
    uint8_t* codes;
    uint16_t* scales;
    int N, K;
} qmat;

typedef struct {
    qmat wq, wk, wv, wo, w1, w3, w2, router;
    qmat* ew1;
    qmat* ew3;
    qmat* ew2;
    uint16_t *kpool, *vpool;                 /* fp16 pages */
    uint8_t *kc4, *kc3, *vc4, *vc3;          /* TurboQuant pages */
    uint16_t *kn, *vn;
    uint8_t *kcc, *vcc;                      /* Cool codes (tiered with warm_window > 0) */
    uint16_t *kcn, *vcn;
    float ksign[NXO_TQ_D], vsign[NXO_TQ_D];
    float *norm_attn, *norm_ffn;             /* RMSNorm weights, NULL = 1.0 */
    float *qnorm, *knorm;                    /* per-head Q/K RMSNorm weights [hd] (qk_norm), NULL = 1.0 */
} layer_t;

struct nxo_model {
    nxo_cfg c;
    int qdim, kvdim;
    uint16_t* embed;
    qmat lm;
    layer_t* layers;
    float* norm_final;                       /* NULL = 1.0 */
    float *rope_cos, *rope_sin;
    int max_blocks, n_blocks;
    int32_t* block_table;
    int32_t* pos;
    float c4[16], b4[15], c3[8], b3[7];
    /* scratch */
    float *h, *xn, *q, *k, *v, *att, *tmp, *g, *u, *a, *dn, *acc, *logits_r;
};

static void make_qmat(qmat* m, int N, int K, uint64_t seed, uint32_t tid, double sigma) {
    const int G = (K + 31) / 32;
    m->N = N;
    m->K = K;
    m->codes = (uint8_t*)malloc((size_t)N * G * 16);
    m->scales = (uint16_t*)malloc((size_t)N * G * 2);
    float* w = (float*)malloc(sizeof(float) * (size_t)N * K);
    nxo_gen_normal(w, (size_t)N * K, seed, tid, nxo_normal_k(sigma));
    nxo_quantize_int4_g32(w, N, K, m->codes, m->scales);
    free(w);
}

/* RMSNorm weights 1 + N(0, sigma) of one tensor id; NULL for sigma 0. */
static float* make_norm(int d, uint64_t seed, uint32_t tid, double sigma) {
    if (sigma == 0.0) return NULL;
    float* w = (float*)malloc(sizeof(float) * (size_t)d);
    nxo_gen_normal(w, (size_t)d, seed, tid, nxo_normal_k(sigma));
    for (int i = 0; i < d; ++i) w[i] = 1.0f + w[i];
    return w;
}

static void free_qmat(qmat* m) {
    free(m->codes);
    free(m->scales);
    m->codes = NULL;
    m->scales = NULL;
}

static void gemv(const qmat* m, const float* x, int B, float* y) {
    nxo_gemv_int4_g32(m->codes, m->scales, x, m->N, m->K, B, y);
}

nxo_model* nxo_model_create(const nxo_cfg* cfg) {
    nxo_model* m = (nxo_model*)calloc(1, sizeof(nxo_model));
    m->c = *cfg;
    const nxo_cfg* c = &m->c;
    const int d = c->d_model, hd = c->head_dim, B = c->batch;
    m->qdim = c->n_heads * hd;
    m->kvdim = c->n_kv_heads * hd;
    const uint64_t seed = c->seed;
    /* embedding [V][d] fp16 */
    {
        float* e = (float*)malloc(sizeof(float) * (size_t)c->vocab * d);
        nxo_gen_normal(e, (size_t)c->vocab * d, seed, NXO_TID_EMBED, nxo_normal_k(0.02));
        m->embed = (uint16_t*)malloc(2 * (size_t)c->vocab * d);
        nxo_f32_to_f16_array(e, m->embed, (size_t)c->vocab * d);
        free(e);
    }
    make_qmat(&m->lm, c->vocab, d, seed, NXO_TID_LMHEAD, 0.02);
    m->norm_final = make_norm(d, seed, NXO_TID_FINAL_NORM, c->norm_sigma);
    m->max_blocks = c->max_seq / NXO_PAGE;
    m->n_blocks = m->max_blocks * B;
    m->block_table = (int32_t*)malloc(sizeof(int32_t) * (size_t)m->n_blocks);
    nxo_shuffle_perm(m->block_table, m->n_blocks, seed, NXO_TID_PAGE_SHUFFLE);
    m->pos = (int32_t*)calloc((size_t)B, sizeof(int32_t));
    m->rope_cos = (float*)malloc(sizeof(float) * (size_t)c->max_seq * (hd / 2));
    m->rope_sin = (float*)malloc(sizeof(float) * (size_t)c->max_seq * (hd / 2));
    nxo_rope_table(c->max_seq, hd, (double)c->rope_theta, m->rope_cos, m->rope_sin);
    nxo_tq_codebook(NXO_TQ_D, 4, m->c4, m->b4);
    nxo_tq_codebook(NXO_TQ_D, 3, m->c3, m->b3);
    m->layers = (layer_t*)calloc((size_t)c->n_layers, sizeof(layer_t));
    const size_t pool_elems = (size_t)m->n_blocks * c->n_kv_heads * NXO_PAGE * hd;
    const size_t pool_vecs = (size_t)m->n_blocks * c->n_kv_heads * NXO_PAGE;
    for (int L = 0; L < c->n_layers; ++L) {
        layer_t* ly = &m->layers[L];
        make_qmat(&ly->wq, m->qdim, d, seed, NXO_TID_LAYER(L, NXO_W_Q), 0.02);
        make_qmat(&ly->wk, m->kvdim, d, seed, NXO_TID_LAYER(L, NXO_W_K), 0.02);
        make_qmat(&ly->wv, m->kvdim, d, seed, NXO_TID_LAYER(L, NXO_W_V), 0.02);
        make_qmat(&ly->wo, d, m->qdim, seed, NXO_TID_LAYER(L, NXO_W_O), 0.02);
        ly->norm_attn = make_norm(d, seed, NXO_TID_LAYER(L, NXO_N_ATTN), c->norm_sigma);
        ly->norm_ffn = make_norm(d, seed, NXO_TID_LAYER(L, NXO_N_FFN), c->norm_sigma);
        if (c->qk_norm) {
            ly->qnorm = make_norm(hd, seed, NXO_TID_LAYER(L, NXO_N_QNORM), c->norm_sigma);
            ly->knorm = make_norm(hd, seed, NXO_TID_LAYER(L, NXO_N_KNORM), c->norm_sigma);
        }
        if (c->n_experts == 0) {
            make_qmat(&ly->w1, c->ffn, d, seed, NXO_TID_LAYER(L, NXO_W_GATE), 0.02);
            make_qmat(&ly->w3, c->ffn, d, seed, NXO_TID_LAYER(L, NXO_W_UP), 0.02);
            make_qmat(&ly->w2, d, c->ffn, seed, NXO_TID_LAYER(L, NXO_W_DOWN), 0.02);
        } else {
            make_qmat(&ly->router, c->n_experts, d, seed, NXO_TID_LAYER(L, NXO_W_ROUTER),
                      1.0 / sqrt((double)d));
            ly->ew1 = (qmat*)calloc((size_t)c->n_experts, sizeof(qmat));
            ly->ew3 = (qmat*)calloc((size_t)c->n_experts, sizeof(qmat));
            ly->ew2 = (qmat*)calloc((size_t)c->n_experts, sizeof(qmat));
            for (int e = 0; e < c->n_experts; ++e) {
                make_qmat(&ly->ew1[e], c->ffn, d, seed, NXO_TID_EXPERT(L, e, 0), 0.02);
                make_qmat(&ly->ew3[e], c->ffn, d, seed, NXO_TID_EXPERT(L, e, 1), 0.02);
                make_qmat(&ly->ew2[e], d, c->ffn, seed, NXO_TID_EXPERT(L, e, 2), 0.02);
            }
        }
        if (c->kv_kind != 1) {
            ly->kpool = (uint16_t*)calloc(pool_elems, 2);
            ly->vpool = (uint16_t*)calloc(pool_elems, 2);
        }
        if (c->kv_kind != 0) {
            ly->kc4 = (uint8_t*)calloc(pool_vecs, 32);
            ly->kc3 = (uint8_t*)calloc(pool_vecs, 24);
            ly->vc4 = (uint8_t*)calloc(pool_vecs, 32);
            ly->vc3 = (uint8_t*)calloc(pool_vecs, 24);
            ly->kn = (uint16_t*)calloc(pool_vecs, 2);
            ly->vn = (uint16_t*)calloc(pool_vecs, 2);
        }
        if (c->kv_kind == 2 && c->warm_window > 0) {
            ly->kcc = (uint8_t*)calloc(pool_vecs, NXO_COOL_CODES);
            ly->vcc = (uint8_t*)calloc(pool_vecs, NXO_COOL_CODES);
            ly->kcn = (uint16_t*)calloc(pool_vecs, 2);
            ly->vcn = (uint16_t*)calloc(pool_vecs, 2);
        }
        nxo_tq_signs(ly->ksign, seed, NXO_TID_LAYER(L, NXO_TQ_KSIGN));
        nxo_tq_signs(ly->vsign, seed, NXO_TID_LAYER(L, NXO_TQ_VSIGN));
    }
    const int big = c->ffn > c->vocab ? c->ffn : c->vocab;
    const int wide = (m->qdim > d ? m->qdim : d) + 32;
    m->h = (float*)calloc((size_t)B * d, sizeof(float));
    m->xn = (float*)calloc((size_t)B * wide, sizeof(float));
    m->q = (float*)calloc((size_t)B * m->qdim, sizeof(float));
    m->k = (float*)calloc((size_t)B * m->kvdim, sizeof(float));
    m->v = (float*)calloc((size_t)B * m->kvdim, sizeof(float));
    m->att = (float*)calloc((size_t)B * m->qdim, sizeof(float));
    m->tmp = (float*)calloc((size_t)B * d, sizeof(float));
    m->g = (float*)calloc((size_t)B * c->ffn, sizeof(float));
    m->u = (float*)calloc((size_t)B * c->ffn, sizeof(float));
    m->a = (float*)calloc((size_t)B * (c->ffn + 32), sizeof(float));
    m->dn = (float*)calloc((size_t)B * d, sizeof(float));
    m->acc = (float*)calloc((size_t)B * d, sizeof(float));
    m->logits_r = (float*)calloc((size_t)B * big, sizeof(float));
    return m;
}

void nxo_model_free(nxo_model* m) {
    if (!m) return;
    for (int L = 0; L < m->c.n_layers; ++L) {
        layer_t* ly = &m->layers[L];
        free_qmat(&ly->wq); free_qmat(&ly->wk); free_qmat(&ly->wv); free_qmat(&ly->wo);
        if (m->c.n_experts == 0) {
            free_qmat(&ly->w1); free_qmat(&ly->w3); free_qmat(&ly->w2);
        } else {
            free_qmat(&ly->router);
            for (int e = 0; e < m->c.n_experts; ++e) {
                free_qmat(&ly->ew1[e]); free_qmat(&ly->ew3[e]); free_qmat(&ly->ew2[e]);
            }
            free(ly->ew1); free(ly->ew3); free(ly->ew2);
        }
        free(ly->kpool); free(ly->vpool);
        free(ly->kc4); free(ly->kc3); free(ly->vc4); free(ly->vc3); free(ly->kn); free(ly->vn);
        free(ly->kcc); free(ly->vcc); free(ly->kcn); free(ly->vcn);
        free(ly->norm_attn); free(ly->norm_ffn);
        free(ly->qnorm); free(ly->knorm);
    }
    free(m->norm_final);
    free(m->layers);
    free_qmat(&m->lm);
    free(m->embed); free(m->block_table); free(m->pos); free(m->rope_cos); free(m->rope_sin);
    free(m->h); free(m->xn); free(m->q); free(m->k); free(m->v); free(m->att); free(m->tmp);
    free(m->g); free(m->u); free(m->a); free(m->dn); free(m->acc); free(m->logits_r);
    free(m);
}

int nxo_model_position(const nxo_model* m, int b) { return m->pos[b]; }
const int32_t* nxo_model_block_table(const nxo_model* m) { return m->block_table; }
int nxo_model_kv_read(const nxo_model* m, int layer, int b, int pos, int kv, int form, uint8_t* out) {
    const nxo_cfg* c = &m->c;
    const int hkv = c->n_kv_heads, hd = c->head_dim;
    const layer_t* ly = &m->layers[layer];
    const int blk = m->block_table[(size_t)b * m->max_blocks + pos / NXO_PAGE], slot = pos % NXO_PAGE;
    if (form == 0 && !ly->kpool) return 0;
    if (form == 1 && !ly->kc4) return 0;
    if (form == 2 && !ly->kcc) return 0;
    for (int h = 0; h < hkv; ++h) {
        if (form == 2) {
            const size_t vi = ((size_t)blk * hkv + h) * NXO_PAGE + slot;
            memcpy(out + (size_t)(NXO_COOL_CODES + 2) * h, (kv ? ly->vcc : ly->kcc) + vi * NXO_COOL_CODES,
                   NXO_COOL_CODES);
            memcpy(out + (size_t)(NXO_COOL_CODES + 2) * h + NXO_COOL_CODES, (kv ? ly->vcn : ly->kcn) + vi, 2);
        } else if (form == 1) {
            const size_t vi = ((size_t)blk * hkv + h) * NXO_PAGE + slot;
            memcpy(out + (size_t)58 * h, (kv ? ly->vc4 : ly->kc4) + vi * 32, 32);
            memcpy(out + (size_t)58 * h + 32, (kv ? ly->vc3 : ly->kc3) + vi * 24, 24);
            memcpy(out + (size_t)58 * h + 56, (kv ? ly->vn : ly->kn) + vi, 2);
        } else {
            const uint16_t* pg = (kv ? ly->vpool : ly->kpool) + ((size_t)blk * hkv + h) * NXO_PAGE * hd;
            for (int d = 0; d < hd; ++d) {
                const uint16_t v = kv ? pg[(size_t)d * NXO_PAGE + slot] : pg[(size_t)slot * hd + d];
                memcpy(out + ((size_t)h * hd + d) * 2, &v, 2);
            }
        }
    }
    return form == 2 ? (NXO_COOL_CODES + 2) * hkv : form == 1 ? 58 * hkv : 2 * hkv * hd;
}
int nxo_model_max_blocks(const nxo_model* m) { return m->max_blocks; }

/* Tiered append of one position: fp16 and Warm forms, and the Cool form
 * (from the Warm codes) when the model has a Cool tier. */
static void tiered_append(nxo_model* m, layer_t* ly, const float* k, const float* v, int b, int pos) {
    const int hkv = m->c.n_kv_heads;
    nxo_tiered_append(k, v, hkv, ly->ksign, ly->vsign, m->b4, m->b3, ly->kpool, ly->vpool, ly->kc4, ly->kc3, ly->kn,
                      ly->vc4, ly->vc3, ly->vn, m->block_table, m->max_blocks, b, pos);
    if (ly->kcc)
        nxo_tiered_append_cool(hkv, ly->ksign, ly->vsign, m->c4, m->c3, m->b3, ly->kc4, ly->kc3, ly->kn, ly->vc4,
                               ly->vc3, ly->vn, ly->kcc, ly->kcn, ly->vcc, ly->vcn, m->block_table, m->max_blocks, b,
                               pos);
}

/* x (fp32) -> fp16-rounded RMSNorm output with weights w (NULL = 1.0). */
static void norm_to_f16(const float* x, const float* w, int d, float eps, float* out) {
    nxo_rmsnorm(x, w, d, eps, out);
    for (int i = 0; i < d; ++i) out[i] = round_f16(out[i]);
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static void ffn_dense(nxo_model* m, layer_t* ly, const float* xn, int B, float* out) {
    const int F = m->c.ffn;
    gemv(&ly->w1, xn, B, m->g);
    gemv(&ly->w3, xn, B, m->u);
    for (int b = 0; b < B; ++b) {
        nxo_swiglu(m->g + (size_t)b * F, m->u + (size_t)b * F, F, m->a + (size_t)b * F);
        for (int i = 0; i < F; ++i) m->a[(size_t)b * F + i] = round_f16(m->a[(size_t)b * F + i]);
    }
    gemv(&ly->w2, m->a, B, out);
}

static void ffn_moe(nxo_model* m, layer_t* ly, const float* xn, int B, float* out) {
    const int d = m->c.d_model, F = m->c.ffn, E = m->c.n_experts, k = m->c.top_k;
    float logits[256];
    int32_t ids[256];
    float w[256];
    for (int b = 0; b < B; ++b) {
        const float* xb = xn + (size_t)b * d;
        gemv(&ly->router, xb, 1, logits);
        nxo_moe_route(logits, E, k, ids, w);
        float* ob = out + (size_t)b * d;
        for (int i = 0; i < d; ++i) ob[i] = 0.0f;
        for (int j = 0; j < k; ++j) {
            const int e = ids[j];
            gemv(&ly->ew1[e], xb, 1, m->g);
            gemv(&ly->ew3[e], xb, 1, m->u);
            nxo_swiglu(m->g, m->u, F, m->a);
            for (int i = 0; i < F; ++i) m->a[i] = round_f16(m->a[i]);
            gemv(&ly->ew2[e], m->a, 1, m->acc);  /* expert output (out aliases m->dn) */
            for (int i = 0; i < d; ++i) ob[i] += w[j] * m->acc[i];
        }
    }
}

static void forward_impl(nxo_model* m, const int32_t* tokens, float* logits, double* t_layers,
                         double* t_head) {
    const nxo_cfg* c = &m->c;
    const int B = c->batch, d = c->d_model, hd = c->head_dim, hq = c->n_heads, hkv = c->n_kv_heads;
    const double t0 = now_s();
    for (int b = 0; b < B; ++b)
        for (int i = 0; i < d; ++i)
            m->h[(size_t)b * d + i] = nxo_f16_to_f32(m->embed[(size_t)tokens[b] * d + i]);
    int32_t* ctx = (int32_t*)malloc(sizeof(int32_t) * (size_t)B);
    for (int b = 0; b < B; ++b) ctx[b] = m->pos[b] + 1;
    for (int L = 0; L < c->n_layers; ++L) {
        layer_t* ly = &m->layers[L];
        for (int b = 0; b < B; ++b) norm_to_f16(m->h + (size_t)b * d, ly->norm_attn, d, c->eps, m->xn + (size_t)b * d);
        gemv(&ly->wq, m->xn, B, m->q);
        gemv(&ly->wk, m->xn, B, m->k);
        gemv(&ly->wv, m->xn, B, m->v);
        for (int b = 0; b < B; ++b) {
            float* qb = m->q + (size_t)b * m->qdim;
            float* kb = m->k + (size_t)b * m->kvdim;
            float* vb = m->v + (size_t)b * m->kvdim;
            if (c->qk_norm) {  /* model/hybrid_model.cpp:1325-1349, before RoPE */
                nxo_head_rmsnorm(qb, hq, hd, ly->qnorm, c->eps);
                nxo_head_rmsnorm(kb, hkv, hd, ly->knorm, c->eps);
            }
            nxo_rope(qb, hq, hd, m->pos[b], m->rope_cos, m->rope_sin);
            nxo_rope(kb, hkv, hd, m->pos[b], m->rope_cos, m->rope_sin);
            if (c->kv_kind == 0)
                nxo_kv_append_f16(kb, vb, ly->kpool, ly->vpool, m->block_table, m->max_blocks, b,
                                  m->pos[b], hkv, hd);
            else if (c->kv_kind == 2)
                tiered_append(m, ly, kb, vb, b, m->pos[b]);
            else
                nxo_tq_append(kb, vb, hkv, ly->ksign, ly->vsign, m->b4, m->b3, ly->kc4, ly->kc3,
                              ly->kn, ly->vc4, ly->vc3, ly->vn, m->block_table, m->max_blocks, b,
                              m->pos[b]);
        }
        if (c->kv_kind == 0)
            nxo_attn_decode_paged_f16(m->q, ly->kpool, ly->vpool, m->block_table, m->max_blocks,
                                      ctx, B, hq, hkv, hd, m->att);
        else if (c->kv_kind == 2)
            nxo_attn_decode_tiered_evict(m->q, ly->kpool, ly->vpool, ly->kc4, ly->kc3, ly->kn, ly->vc4, ly->vc3,
                                         ly->vn, ly->kcc, ly->kcn, ly->vcc, ly->vcn, ly->ksign, ly->vsign, m->c4,
                                         m->c3, m->block_table, m->max_blocks, ctx, c->hot_window, c->warm_window,
                                         c->cool_window, B, hq, hkv, m->att);
        else
            nxo_attn_decode_paged_tq(m->q, ly->kc4, ly->kc3, ly->kn, ly->vc4, ly->vc3, ly->vn,
                                     ly->ksign, ly->vsign, m->c4, m->c3, m->block_table,
                                     m->max_blocks, ctx, B, hq, hkv, m->att);
        for (size_t i = 0; i < (size_t)B * m->qdim; ++i) m->att[i] = round_f16(m->att[i]);
        gemv(&ly->wo, m->att, B, m->tmp);
        for (size_t i = 0; i < (size_t)B * d; ++i) m->h[i] = m->h[i] + m->tmp[i];
        for (int b = 0; b < B; ++b) norm_to_f16(m->h + (size_t)b * d, ly->norm_ffn, d, c->eps, m->xn + (size_t)b * d);
        if (c->n_experts == 0)
            ffn_dense(m, ly, m->xn, B, m->dn);
        else
            ffn_moe(m, ly, m->xn, B, m->dn);
        for (size_t i = 0; i < (size_t)B * d; ++i) m->h[i] = m->h[i] + m->dn[i];
    }
    const double t1 = now_s();
    for (int b = 0; b < B; ++b) norm_to_f16(m->h + (size_t)b * d, m->norm_final, d, c->eps, m->xn + (size_t)b * d);
    gemv(&m->lm, m->xn, B, logits ? logits : m->logits_r);
    const double t2 = now_s();
    for (int b = 0; b < B; ++b) m->pos[b] += 1;
    free(ctx);
    if (t_layers) *t_layers = t1 - t0;
    if (t_head) *t_head = t2 - t1;
}

void nxo_model_forward(nxo_model* m, const int32_t* tokens, float* logits) {
    forward_impl(m, tokens, logits, NULL, NULL);
}

void nxo_model_forward_timed(nxo_model* m, const int32_t* tokens, float* logits,
                             double* t_layers, double* t_head) {
    forward_impl(m, tokens, logits, t_layers, t_head);
}

static float margin_of(const float* v, int n, int best) {
    float second = -INFINITY;
    for (int i = 0; i < n; ++i)
        if (i != best && v[i] > second) second = v[i];
    return v[best] - second;
}

void nxo_model_generate(nxo_model* m, const int32_t* prompt, int P, int n_new,
                        int32_t* out_tokens, float* margins) {
    const int B = m->c.batch, V = m->c.vocab;
    float* logits = (float*)malloc(sizeof(float) * (size_t)B * V);
    int32_t* tok = (int32_t*)malloc(sizeof(int32_t) * (size_t)B);
    for (int i = 0; i < P; ++i) {
        for (int b = 0; b < B; ++b) tok[b] = prompt[(size_t)b * P + i];
        forward_impl(m, tok, logits, NULL, NULL);
    }
    for (int j = 0; j < n_new; ++j) {
        for (int b = 0; b < B; ++b) {
            const float* lb = logits + (size_t)b * V;
            tok[b] = nxo_argmax(lb, V);
            out_tokens[(size_t)b * n_new + j] = tok[b];
            if (margins) margins[(size_t)b * n_new + j] = margin_of(lb, V, tok[b]);
        }
        if (j + 1 < n_new) forward_impl(m, tok, logits, NULL, NULL);
    }
    free(logits);
    free(tok);
}

/* Outlier channels of (layer, kv, head): the first n of a seeded shuffle of 0..hd-1. */
static void outlier_channels(uint64_t seed, int L, int kv, int h, int hd, int n, int32_t* out) {
    int32_t perm[512];
    nxo_shuffle_perm(perm, hd, seed, 0x20000000u + 0x10000u * (uint32_t)L + 0x100u * (uint32_t)kv + (uint32_t)h);
    for (int i = 0; i < n; ++i) out[i] = perm[i];
}

void nxo_model_fill_context(nxo_model* m, int ctx, int n_outlier) {
    const nxo_cfg* c = &m->c;
    const int hkv = c->n_kv_heads, hd = c->head_dim;
    const float k1 = nxo_normal_k(1.0);
    float* kv = (float*)malloc(sizeof(float) * (size_t)hkv * hd * 2);
    for (int L = 0; L < c->n_layers; ++L) {
        layer_t* ly = &m->layers[L];
        int32_t och[2][64][16];
        for (int kvk = 0; kvk < 2; ++kvk)
            for (int h = 0; h < hkv; ++h) outlier_channels(c->seed, L, kvk, h, hd, n_outlier, och[kvk][h]);
        for (int b = 0; b < c->batch; ++b) {
            for (int p = 0; p < ctx; ++p) {
                for (int kvk = 0; kvk < 2; ++kvk) {
                    const uint32_t tid = NXO_TID_CTX(L, b, kvk);
                    float* dst = kv + (size_t)kvk * hkv * hd;
                    for (int i = 0; i < hkv * hd; ++i)
                        dst[i] = nxo_normal_from_u64(nxo_rand_u64(c->seed, tid, (uint64_t)p * hkv * hd + i), k1);
                    for (int h = 0; h < hkv; ++h)
                        for (int j = 0; j < n_outlier; ++j) dst[h * hd + och[kvk][h][j]] *= 10.0f;
                }
                if (c->kv_kind == 0)
                    nxo_kv_append_f16(kv, kv + (size_t)hkv * hd, ly->kpool, ly->vpool, m->block_table,
                                      m->max_blocks, b, p, hkv, hd);
                else if (c->kv_kind == 2)
                    tiered_append(m, ly, kv, kv + (size_t)hkv * hd, b, p);
                else
                    nxo_tq_append(kv, kv + (size_t)hkv * hd, hkv, ly->ksign, ly->vsign, m->b4, m->b3,
                                  ly->kc4, ly->kc3, ly->kn, ly->vc4, ly->vc3, ly->vn, m->block_table,
                                  m->max_blocks, b, p);
            }
        }
    }
    for (int b = 0; b < c->batch; ++b) m->pos[b] = ctx;
    free(kv);
}

int nxo_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void nxo_set_num_threads(int n) {
#ifdef _OPENMP
    omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* --------------------------------------------------------------- NXF ---- */
/* XXH32 (format/nxf_writer.cpp:33-72): four lanes v1..v4 over 16-byte
 * stripes, v = rotl(v + w * P2, 13) * P1; merge rotl(v1,1) + rotl(v2,7) +
 * rotl(v3,12) + rotl(v4,18) (seed + P5 below 16 bytes); add the length;
 * remaining 4-byte words h = rotl(h + w * P3, 17) * P4, bytes
 * h = rotl(h + b * P5, 11) * P1; avalanche >>15 *P2 >>13 *P3 >>16. */
static uint32_t xxh_rotl(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }
static uint32_t xxh_le32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

uint32_t nxo_xxh32(const void* data, size_t len, uint32_t seed) {
    const uint32_t P1 = 0x9E3779B1u, P2 = 0x85EBCA77u, P3 = 0xC2B2AE3Du, P4 = 0x27D4EB2Fu,
                   P5 = 0x165667B1u;
    const uint8_t* p = (const uint8_t*)data;
    const size_t nstripe = len / 16;
    uint32_t h;
    if (nstripe > 0) {
        uint32_t v[4] = {seed + P1 + P2, seed + P2, seed, seed - P1};
        for (size_t s = 0; s < nstripe; ++s)
            for (int l = 0; l < 4; ++l) v[l] = xxh_rotl(v[l] + xxh_le32(p + 16 * s + 4 * l) * P2, 13) * P1;
        h = xxh_rotl(v[0], 1) + xxh_rotl(v[1], 7) + xxh_rotl(v[2], 12) + xxh_rotl(v[3], 18);
    } else {
        h = seed + P5;
    }
    h += (uint32_t)len;
    size_t i = 16 * nstripe;
    for (; i + 4 <= len; i += 4) h = xxh_rotl(h + xxh_le32(p + i) * P3, 17) * P4;
    for (; i < len; ++i) h = xxh_rotl(h + (uint32_t)p[i] * P5, 11) * P1;
    h ^= h >> 15;
    h *= P2;
    h ^= h >> 13;
    h *= P3;
    h ^= h >> 16;
    return h;
}

/* ------------------------------------------------------------ sampling ---- */
void nxo_mt19937(uint32_t seed, int n, uint32_t* out) {
    uint32_t mt[624];
    mt[0] = seed;
    for (int i = 1; i < 624; ++i) mt[i] = 1812433253u * (mt[i - 1] ^ (mt[i - 1] >> 30)) + (uint32_t)i;
    int idx = 624;
    for (int o = 0; o < n; ++o) {
        if (idx >= 624) {
            for (int i = 0; i < 624; ++i) {
                const uint32_t y = (mt[i] & 0x80000000u) | (mt[(i + 1) % 624] & 0x7FFFFFFFu);
                mt[i] = mt[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908B0DFu : 0u);
            }
            idx = 0;
        }
        uint32_t y = mt[idx++];
        y ^= y >> 11;
        y ^= (y << 7) & 0x9D2C5680u;
        y ^= (y << 15) & 0xEFC60000u;
        y ^= y >> 18;
        out[o] = y;
    }
}

float nxo_canonical_f32(uint32_t x) {
    const float r = (float)x / 4294967296.0f;
    return r >= 1.0f ? nextafterf(1.0f, 0.0f) : r;
}

/* descending by value, ties by ascending index */
static const float* g_sort_vals;
static int cmp_desc_idx(const void* a, const void* b) {
    const int i = *(const int*)a, j = *(const int*)b;
    const float x = g_sort_vals[i], y = g_sort_vals[j];
    if (x > y) return -1;
    if (x < y) return 1;
    return i < j ? -1 : (i > j);
}

int nxo_sample(const float* logits, int V, float temperature, int top_k, float top_p, float u) {
    if (temperature <= 0.0f) {
        int best = 0;
        for (int i = 1; i < V; ++i)
            if (logits[i] > logits[best]) best = i;
        return best;
    }
    float* probs = (float*)malloc(sizeof(float) * (size_t)V);
    int* idx = (int*)malloc(sizeof(int) * (size_t)V);
    float mx = logits[0];
    for (int i = 1; i < V; ++i) mx = logits[i] > mx ? logits[i] : mx;
    float sum = 0.0f;
    for (int i = 0; i < V; ++i) {
        probs[i] = expf((logits[i] - mx) / temperature);
        sum += probs[i];
    }
    for (int i = 0; i < V; ++i) probs[i] /= sum;
    g_sort_vals = probs;
    if (top_k > 0 && top_k < V) {
        for (int i = 0; i < V; ++i) idx[i] = i;
        qsort(idx, (size_t)V, sizeof(int), cmp_desc_idx);
        for (int i = top_k; i < V; ++i) probs[idx[i]] = 0.0f;
    }
    if (top_p < 1.0f) {
        for (int i = 0; i < V; ++i) idx[i] = i;
        qsort(idx, (size_t)V, sizeof(int), cmp_desc_idx);
        float cum = 0.0f;
        for (int i = 0; i < V; ++i) {
            cum += probs[idx[i]];
            if (cum > top_p) {
                for (int j = i + 1; j < V; ++j) probs[idx[j]] = 0.0f;
                break;
            }
        }
    }
    sum = 0.0f;
    for (int i = 0; i < V; ++i) sum += probs[i];
    int tok = V - 1;
    if (sum <= 0.0f) {
        tok = 0;
    } else {
        const float r = u * sum;
        float cum = 0.0f;
        for (int i = 0; i < V; ++i) {
            cum += probs[i];
            if (cum >= r) {
                tok = i;
                break;
            }
        }
    }
    free(probs);
    free(idx);
    return tok;
}
