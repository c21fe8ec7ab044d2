// Device-side building blocks of the int4 group-32 GEMV (see nx_gemv.hip for
// the design): input staging, weight tiles, the nibble dot product, the
// fused epilogues and the batch-1 streaming body.
#pragma once

#include "nx_common.h"
#include "nx_kernels.h"

namespace nx {
namespace gv {


constexpr int kWavesPerBlock = 4;
constexpr int kBlockThreads = kWavesPerBlock * kWave;

template <int GPL>
struct XPairs {
    uint32_t p[GPL][16];  // fp16 pairs (x[8d+j], x[8d+j+4]) per group
    float s8[GPL];        // 8 * sum of the group's x (fp32)
};

__device__ inline void build_pairs(const uint32_t (&X)[16], uint32_t (&P)[16]) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        P[4 * d + 0] = __builtin_amdgcn_perm(X[4 * d + 2], X[4 * d + 0], 0x05040100u);
        P[4 * d + 1] = __builtin_amdgcn_perm(X[4 * d + 2], X[4 * d + 0], 0x07060302u);
        P[4 * d + 2] = __builtin_amdgcn_perm(X[4 * d + 3], X[4 * d + 1], 0x05040100u);
        P[4 * d + 3] = __builtin_amdgcn_perm(X[4 * d + 3], X[4 * d + 1], 0x07060302u);
    }
}

__device__ inline float group_sum16(const uint32_t (&X)[16]) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        s += h2f_bits((uint16_t)(X[j] & 0xFFFFu));
        s += h2f_bits((uint16_t)(X[j] >> 16));
    }
    return s;
}

// x fp16 row -> pair registers.  Elements k >= K read as 0.
template <int GPL>
__device__ inline void load_x16(XPairs<GPL>& xp, const uint16_t* __restrict__ x, int K, int G,
                                int lane) {
#pragma unroll
    for (int i = 0; i < GPL; ++i) {
        const int g = lane + kWave * i;
        uint32_t X[16];
        const uint16_t* src = x + 32 * g;
        if (g < G && 32 * g + 32 <= K && ((reinterpret_cast<uintptr_t>(src) & 15u) == 0)) {
            const uint4* s4 = reinterpret_cast<const uint4*>(src);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 v = s4[q];
                X[4 * q + 0] = v.x;
                X[4 * q + 1] = v.y;
                X[4 * q + 2] = v.z;
                X[4 * q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int k = 32 * g + 2 * j;
                const uint32_t lo = (g < G && k < K) ? src[2 * j] : 0u;
                const uint32_t hi = (g < G && k + 1 < K) ? src[2 * j + 1] : 0u;
                X[j] = lo | (hi << 16);
            }
        }
        build_pairs(X, xp.p[i]);
        xp.s8[i] = 8.0f * group_sum16(X);
    }
}

// 1/sqrt(mean(h^2) + eps) of one fp32 row, wave-uniform.
template <int GPL>
__device__ inline float rms_inv(const float* __restrict__ h, int K, int G, float eps, int lane) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < GPL; ++i) {
        const int g = lane + kWave * i;
        if (g < G) {
            const float* src = h + 32 * g;
            if (32 * g + 32 <= K && ((reinterpret_cast<uintptr_t>(src) & 15u) == 0)) {
                const float4* s4 = reinterpret_cast<const float4*>(src);
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const float4 v = s4[q];
                    ss += v.x * v.x;
                    ss += v.y * v.y;
                    ss += v.z * v.z;
                    ss += v.w * v.w;
                }
            } else {
                for (int j = 0; j < 32; ++j)
                    if (32 * g + j < K) ss += src[j] * src[j];
            }
        }
    }
    ss = wave_sum(ss);
    return 1.0f / sqrtf(ss / (float)K + eps);
}

// x = fp16((h * inv) * w) -> pair registers.
template <int GPL>
__device__ inline void load_x_norm(XPairs<GPL>& xp, const float* __restrict__ h,
                                   const float* __restrict__ w, float inv, int K, int G,
                                   int lane) {
#pragma unroll
    for (int i = 0; i < GPL; ++i) {
        const int g = lane + kWave * i;
        uint32_t X[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int k = 32 * g + 2 * j;
            uint32_t lo = 0, hi = 0;
            if (g < G && k < K) {
                const float v = h[k] * inv;
                lo = f2h_bits(w ? v * w[k] : v);
            }
            if (g < G && k + 1 < K) {
                const float v = h[k + 1] * inv;
                hi = f2h_bits(w ? v * w[k + 1] : v);
            }
            X[j] = lo | (hi << 16);
        }
        build_pairs(X, xp.p[i]);
        xp.s8[i] = 8.0f * group_sum16(X);
    }
}

__device__ inline half2_t as_h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }

// sum_{k in group} (q_k - 8) x_k for one 16-byte group of codes.
__device__ inline float group_dot(uint4 w, const uint32_t (&P)[16], float s8) {
    float accA = 0.0f, accB = 0.0f;
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t a = wd[d] & 0x000F000Fu;
        const uint32_t b = wd[d] & 0x00F000F0u;
        const uint32_t w8 = wd[d] >> 8;
        const uint32_t c = w8 & 0x000F000Fu;
        const uint32_t e = w8 & 0x00F000F0u;
        accA = __builtin_amdgcn_fdot2(as_h2(a), as_h2(P[4 * d + 0]), accA, false);
        accA = __builtin_amdgcn_fdot2(as_h2(c), as_h2(P[4 * d + 2]), accA, false);
        accB = __builtin_amdgcn_fdot2(as_h2(b), as_h2(P[4 * d + 1]), accB, false);
        accB = __builtin_amdgcn_fdot2(as_h2(e), as_h2(P[4 * d + 3]), accB, false);
    }
    return fmaf(accB, 0x1p20f, accA * 0x1p24f) - s8;
}

template <int GPL, int R>
struct Tile {
    uint4 w[R][GPL];
    uint16_t s[R][GPL];  // raw fp16 scales, converted at use so no wait is forced at load
};

// Load rows [n0, n0 + R) of the weight matrix; rows at or beyond `nlim`
// (the end of this wavefront's row range) are not read and count as zero.
template <int GPL, int R>
__device__ inline void load_tile(Tile<GPL, R>& t, const uint8_t* __restrict__ W,
                                 const uint16_t* __restrict__ S, int G, int nlim, int n0,
                                 int lane) {
    const size_t rowbytes = (size_t)G * 16;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = n0 + r;
#pragma unroll
        for (int i = 0; i < GPL; ++i) {
            const int g = lane + kWave * i;
            if (row < nlim && g < G) {
                t.w[r][i] = *reinterpret_cast<const uint4*>(W + (size_t)row * rowbytes + 16 * (size_t)g);
                t.s[r][i] = S[(size_t)row * G + g];
            } else {
                t.w[r][i] = make_uint4(0u, 0u, 0u, 0u);
                t.s[r][i] = 0;
            }
        }
    }
}

// Rows [n0, n0 + R) of a wavefront whose rows are [rlo, rhi), loaded
// without a branch or a select (a select lets the compiler move the load
// under a branch): rows at or beyond rhi re-read row rhi - 1, which the
// epilogue ignores, and lanes whose group is at or beyond G re-read group
// G - 1, whose product is zero because the staged x of those groups is zero
// (codes and scales are finite).
template <int GPL, int R>
__device__ inline void load_tile_u(Tile<GPL, R>& t, const uint8_t* __restrict__ W,
                                   const uint16_t* __restrict__ S, int G, int rlo, int rhi, int n0,
                                   int lane) {
    const size_t rowbytes = (size_t)G * 16;
    const int rlast = rhi > rlo ? rhi - 1 : (rlo > 0 ? rlo - 1 : 0);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = n0 + r < rlast ? n0 + r : rlast;
#pragma unroll
        for (int i = 0; i < GPL; ++i) {
            const int g = lane + kWave * i < G ? lane + kWave * i : G - 1;
            t.w[r][i] = *reinterpret_cast<const uint4*>(W + (size_t)row * rowbytes + 16 * (size_t)g);
            t.s[r][i] = S[(size_t)row * G + g];
        }
    }
}

template <int GPL, int R>
__device__ inline void tile_dot(const Tile<GPL, R>& t, const XPairs<GPL>& xp, float (&res)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < GPL; ++i)
            acc = fmaf(group_dot(t.w[r][i], xp.p[i], xp.s8[i]), h2f_bits(t.s[r][i]), acc);
        res[r] = wave_sum(acc);
    }
}

__device__ inline unsigned long long pack_best(float v, int idx) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)ord << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)idx);
}

// Values the QKV epilogue needs, fetched before the tile is reduced so the
// epilogue does not wait on memory: the position, RoPE cos/sin of each row
// pair of the tile and the block of the page the new K/V go to.
struct RopePre {
    bool valid;
    int p, blk;
    float c[4], s[4];
};

// Rows at or beyond `nlim` are not stored.  The residual add (E_ACC) is a
// no-return atomic add: each element has exactly one writer, so the sum is
// the plain y + res, and the wavefront does not wait for a read of y.
template <int EPI, int R>
__device__ inline void epilogue(const GemvArgs& a, int b, int n0, int nlim, const float (&res)[R],
                                float& best_v, int& best_i, const RopePre* pre = nullptr) {
    if (EPI == E_F16) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (n0 + r < nlim) a.y16[(size_t)b * a.ldy + n0 + r] = f2h_bits(res[r]);
    } else if (EPI == E_F32) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (n0 + r < nlim) a.y32[(size_t)b * a.ldy + n0 + r] = res[r];
    } else if (EPI == E_ACC) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (n0 + r < nlim)
                __hip_atomic_fetch_add(a.y32 + (size_t)b * a.ldy + n0 + r, res[r], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
    } else if (EPI == E_QKV) {
        const bool have = pre && pre->valid;
        const int p = have ? pre->p : a.pos[b];
        const int half = a.hd >> 1;
#pragma unroll
        for (int r = 0; r < R; r += 2) {
            const int row = n0 + r;
            if (row >= nlim) break;
            float v0 = res[r], v1 = res[r + 1];
            if (row < a.qdim + a.kvdim && a.cos_t) {  // no tables: the projection alone
                const int i = (row % a.hd) >> 1;
                const float c = have ? pre->c[r / 2] : a.cos_t[(size_t)p * half + i];
                const float s = have ? pre->s[r / 2] : a.sin_t[(size_t)p * half + i];
                const float r0 = v0 * c - v1 * s;
                const float r1 = v0 * s + v1 * c;
                v0 = r0;
                v1 = r1;
            }
            if (row < a.qdim) {
                a.q32[(size_t)b * a.qdim + row] = v0;
                a.q32[(size_t)b * a.qdim + row + 1] = v1;
            } else {
                const int kv = row < a.qdim + a.kvdim ? 0 : 1;
                const int idx = row - a.qdim - kv * a.kvdim;
                if (a.kpool) {
                    const int kvh = idx / a.hd, dd = idx % a.hd;
                    const int blk = have ? pre->blk : a.block_table[(size_t)b * a.max_blocks + p / kPage];
                    const size_t page = ((size_t)blk * a.hkv + kvh) * kPage * a.hd;
                    uint16_t* v0p;
                    uint16_t* v1p;
                    if (kv) {  // V pages are dimension-major: [hd][16]
                        v0p = a.vpool + page + (size_t)dd * kPage + p % kPage;
                        v1p = a.vpool + page + (size_t)(dd + 1) * kPage + p % kPage;
                    } else {   // K pages are token-major: [16][hd]
                        v0p = a.kpool + page + (size_t)(p % kPage) * a.hd + dd;
                        v1p = v0p + 1;
                    }
                    *v0p = f2h_bits(v0);
                    *v1p = f2h_bits(v1);
                } else {
                    float* dst = a.kv_tmp + ((size_t)b * 2 + kv) * a.kvdim + idx;
                    dst[0] = v0;
                    dst[1] = v1;
                }
            }
        }
    } else if (EPI == E_SWIGLU) {
#pragma unroll
        for (int r = 0; r < R; r += 2) {
            const int row = n0 + r;
            if (row >= nlim) break;
            const float g = res[r], u = res[r + 1];
            a.act16[(size_t)b * a.lda + (row >> 1)] = f2h_bits(g / (1.0f + expf(-g)) * u);
        }
    } else if (EPI == E_LOGITS) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (n0 + r < nlim) {
                a.y32[(size_t)b * a.ldy + n0 + r] = res[r];
                if (res[r] > best_v) {
                    best_v = res[r];
                    best_i = n0 + r;
                }
            }
    }
}

// Eight consecutive inputs starting at k0 (zero beyond K).
__device__ inline void load_h8(const float* __restrict__ h, int k0, int K, bool vec, float (&v)[8]) {
    if (vec && k0 + 8 <= K) {
        const float4 a = *reinterpret_cast<const float4*>(h + k0);
        const float4 c = *reinterpret_cast<const float4*>(h + k0 + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = c.x; v[5] = c.y; v[6] = c.z; v[7] = c.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = k0 + j < K ? h[k0 + j] : 0.0f;
    }
}
__device__ inline void load_x8(const uint16_t* __restrict__ x, int k0, int K, bool vec, uint32_t (&X)[4]) {
    if (vec && k0 + 8 <= K) {
        const uint4 v = *reinterpret_cast<const uint4*>(x + k0);
        X[0] = v.x; X[1] = v.y; X[2] = v.z; X[3] = v.w;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t lo = k0 + 2 * j < K ? x[k0 + 2 * j] : 0u;
            const uint32_t hi = k0 + 2 * j + 1 < K ? x[k0 + 2 * j + 1] : 0u;
            X[j] = lo | (hi << 16);
        }
    }
}

// Chunk c (8 elements) of a row whose first nvalid chunks lie inside K,
// loaded without a branch: a chunk at or beyond nvalid reads chunk 0 and is
// zeroed.  Requires K % 8 == 0 and a 16-byte aligned row.  The batch-1
// kernel issues its input and its first tiles as straight-line code so that
// the compiler's wait before the input is used counts the tile loads issued
// after it (a branch around a load makes it wait for every load).
__device__ inline void load_x8_u(const uint16_t* __restrict__ x, int c, int nvalid, uint32_t (&X)[4]) {
    const bool ok = c < nvalid;
    const uint4 v = *reinterpret_cast<const uint4*>(x + 8 * (ok ? c : 0));
    X[0] = ok ? v.x : 0u;
    X[1] = ok ? v.y : 0u;
    X[2] = ok ? v.z : 0u;
    X[3] = ok ? v.w : 0u;
}
__device__ inline void load_h8_u(const float* __restrict__ h, int c, int nvalid, float (&v)[8]) {
    const bool ok = c < nvalid;
    const float4* src = reinterpret_cast<const float4*>(h + 8 * (ok ? c : 0));
    const float4 a = src[0], b = src[1];
    v[0] = ok ? a.x : 0.0f; v[1] = ok ? a.y : 0.0f; v[2] = ok ? a.z : 0.0f; v[3] = ok ? a.w : 0.0f;
    v[4] = ok ? b.x : 0.0f; v[5] = ok ? b.y : 0.0f; v[6] = ok ? b.z : 0.0f; v[7] = ok ? b.w : 0.0f;
}

// Store one 8-element chunk c (fp16 values X) in the pair layout and its
// contribution to the group sum.
__device__ inline void put_chunk(int c, const uint32_t (&X)[4], uint32_t* sp, float* s8) {
    uint32_t* dst = sp + (c >> 2) * 16 + (c & 3) * 4;
    dst[0] = __builtin_amdgcn_perm(X[2], X[0], 0x05040100u);
    dst[1] = __builtin_amdgcn_perm(X[2], X[0], 0x07060302u);
    dst[2] = __builtin_amdgcn_perm(X[3], X[1], 0x05040100u);
    dst[3] = __builtin_amdgcn_perm(X[3], X[1], 0x07060302u);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        s += h2f_bits((uint16_t)(X[j] & 0xFFFFu));
        s += h2f_bits((uint16_t)(X[j] >> 16));
    }
    // the 4 chunks of a group sit in one DPP quad (nthr and nch are multiples of 4)
    s += dpp<kQuadXor1>(s);
    s += dpp<kQuadXor2>(s);
    if ((c & 3) == 0) s8[c >> 2] = 8.0f * s;
}

// fp16((v * inv) * w) of one 8-element chunk at k0; the weights w were
// loaded with the chunk (has_w false: weights of one).
__device__ inline void norm_chunk(const float (&v)[8], const float (&w)[8], bool has_w, int k0, int K,
                                  float inv, uint32_t (&X)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t lo = 0, hi = 0;
        const int k = k0 + 2 * j;
        if (k < K) {
            const float t = v[2 * j] * inv;
            lo = f2h_bits(has_w ? t * w[2 * j] : t);
        }
        if (k + 1 < K) {
            const float t = v[2 * j + 1] * inv;
            hi = f2h_bits(has_w ? t * w[2 * j + 1] : t);
        }
        X[j] = lo | (hi << 16);
    }
}

// Block-cooperative staging of one x row into LDS in the pair layout:
// sp[g*16 + 4d + j] = (x[32g+8d+j], x[32g+8d+j+4]) and s8[g] = 8 * sum of
// group g.  Thread t of the NT handles the 8-element chunks t, t + NT, ...
// (at most CPT of them, CPT = ceil(G * 4 / NT)).  The staging is split in two
// so the caller can request its weight tiles in between: the row is
// requested first (stage_issue) and converted afterwards (stage_finish).
// Loads complete in issue order, so waiting for the row then does not wait
// for the weights, and a wavefront's first tile can be reduced as soon as it
// arrives.  For X_RMSNORM the block reduces sum(h^2) once and converts from
// the registers; the norm weights of a chunk are requested with it (loads
// issued later, inside the conversion, would wait for every tile in
// flight).  stage_finish ends with a barrier.
template <int CPT, int XS>
struct StageRegs {
    float v[XS == X_RMSNORM ? CPT : 1][8];
    float w[XS == X_RMSNORM ? CPT : 1][8];
    uint32_t X[XS == X_F16 ? CPT : 1][4];
};

template <int CPT, int XS, int NT = kBlockThreads, bool XVEC = false>
__device__ inline void stage_issue(const GemvArgs& a, int b, StageRegs<CPT, XS>& r) {
    const int K = a.K, nch = a.G * 4, tid = threadIdx.x;
    if (XVEC) {
        // K % 8 == 0 and an aligned row (checked by the launcher)
        const int nvalid = K / 8;
        // without norm weights the loads read h again (values unused)
        const float* wsrc = a.norm_w ? a.norm_w : a.h32 + (size_t)b * a.ldx;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            if (XS == X_F16) {
                load_x8_u(a.x16 + (size_t)b * a.ldx, tid + j * NT, nvalid, r.X[j]);
            } else {
                load_h8_u(a.h32 + (size_t)b * a.ldx, tid + j * NT, nvalid, r.v[j]);
                load_h8_u(wsrc, tid + j * NT, nvalid, r.w[j]);
            }
        }
        return;
    }
    if (XS == X_F16) {
        const uint16_t* x = a.x16 + (size_t)b * a.ldx;
        const bool vec = (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (a.ldx & 7) == 0;
#pragma unroll
        for (int j = 0; j < CPT; ++j)
            if (tid + j * NT < nch) load_x8(x, 8 * (tid + j * NT), K, vec, r.X[j]);
    } else {
        const float* h = a.h32 + (size_t)b * a.ldx;
        const bool vec = (reinterpret_cast<uintptr_t>(h) & 15u) == 0 && (a.ldx & 3) == 0;
        const float* w = a.norm_w ? a.norm_w : h;
        const bool wvec = vec && (reinterpret_cast<uintptr_t>(w) & 15u) == 0;
#pragma unroll
        for (int j = 0; j < CPT; ++j)
            if (tid + j * NT < nch) {
                load_h8(h, 8 * (tid + j * NT), K, vec, r.v[j]);
                load_h8(w, 8 * (tid + j * NT), K, wvec, r.w[j]);
            }
    }
}

template <int CPT, int XS, int NT = kBlockThreads>
__device__ inline void stage_finish(const GemvArgs& a, StageRegs<CPT, XS>& r, uint32_t* sp,
                                    float* s8, float* red) {
    const int K = a.K, nch = a.G * 4, tid = threadIdx.x;
    if (XS == X_F16) {
#pragma unroll
        for (int j = 0; j < CPT; ++j)
            if (tid + j * NT < nch) put_chunk(tid + j * NT, r.X[j], sp, s8);
    } else {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < CPT; ++j)
            if (tid + j * NT < nch)
#pragma unroll
                for (int e = 0; e < 8; ++e) ss += r.v[j][e] * r.v[j][e];
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float tot = 0.0f;
        for (int w = 0; w < NT / kWave; ++w) tot += red[w];
        const float inv = 1.0f / sqrtf(tot / (float)K + a.eps);
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = tid + j * NT;
            if (c < nch) {
                uint32_t X[4];
                norm_chunk(r.v[j], r.w[j], a.norm_w != nullptr, 8 * c, K, inv, X);
                put_chunk(c, X, sp, s8);
            }
        }
    }
    __syncthreads();
}

template <int GPL>
__device__ inline void load_pairs_lds(XPairs<GPL>& xp, const uint32_t* sp, const float* s8, int G,
                                      int lane) {
#pragma unroll
    for (int i = 0; i < GPL; ++i) {
        const int g = lane + kWave * i;
        if (g < G) {
            const uint4* src = reinterpret_cast<const uint4*>(sp + g * 16);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 v = src[q];
                xp.p[i][4 * q + 0] = v.x;
                xp.p[i][4 * q + 1] = v.y;
                xp.p[i][4 * q + 2] = v.z;
                xp.p[i][4 * q + 3] = v.w;
            }
            xp.s8[i] = s8[g];
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) xp.p[i][j] = 0u;
            xp.s8[i] = 0.0f;
        }
    }
}

// Grid of a batch-1 GEMV: nb blocks of wpb wavefronts, to whose nb * wpb
// wavefronts the R-row tiles are dealt in turn (paired epilogues use even R,
// so a RoPE or SwiGLU pair is never split).
struct RowSplit {
    int nb = 1, wpb = 1;
};

// Tile product with x read from the LDS pair layout (used where holding x in
// registers would cost GPL * 17 VGPRs and limit occupancy).  The layout's
// groups from G to kWave * GPL hold zeros (zero_pairs_lds), so every lane
// reads its groups without a branch (a branch around the reads made the
// compiler keep every group's pairs live at once and spill).
template <int GPL, int R>
__device__ inline void tile_dot_lds(const Tile<GPL, R>& t, const uint32_t* sp, const float* s8,
                                    int G, int lane, float (&res)[R]) {
    (void)G;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < GPL; ++i) {
        const int g = lane + kWave * i;
        uint32_t P[16];
        {
            const uint4* src = reinterpret_cast<const uint4*>(sp + g * 16);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 v = src[q];
                P[4 * q + 0] = v.x;
                P[4 * q + 1] = v.y;
                P[4 * q + 2] = v.z;
                P[4 * q + 3] = v.w;
            }
        }
        const float sx = s8[g];
#pragma unroll
        for (int r = 0; r < R; ++r)
            acc[r] = fmaf(group_dot(t.w[r][i], P, sx), h2f_bits(t.s[r][i]), acc[r]);
        // keep the scheduler from hoisting the next groups' LDS reads (their
        // registers would push the kernel below two wavefronts per SIMD)
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) res[r] = wave_sum(acc[r]);
}

// Zeros in the pair layout's groups [G, GPL * kWave) and their sums (the
// groups no staged chunk writes), for tile_dot_lds; the caller's barrier
// orders them before the reads.
template <int GPL, int NT>
__device__ inline void zero_pairs_lds(uint32_t* sp, float* s8, int G) {
    for (int i = G * 16 + (int)threadIdx.x; i < GPL * kWave * 16; i += NT) sp[i] = 0u;
    for (int g = G + (int)threadIdx.x; g < GPL * kWave; g += NT) s8[g] = 0.0f;
}

// Batch 1, persistent: every wavefront streams its own contiguous row range
// as R-row tiles through a ring of DEPTH register tiles.  A buffer is
// refilled as soon as its tile has been reduced, so DEPTH - 1 tiles are in
// flight while one is reduced, and the first DEPTH tiles are requested
// before the input is staged, so the HBM stream starts with the kernel.
// XLDS: x is read from LDS per group instead of being held in registers.
// `block` is the block's index within the grid.
template <int GPL, int R, int DEPTH, bool XLDS, int XS, int EPI, int WPB = kWavesPerBlock,
          bool XVEC = false, bool XFIRST = false>
__device__ inline void gemv_b1_run(const GemvArgs& a, const RowSplit& rs, int block) {
    constexpr int NT = WPB * kWave, CPT = (4 * GPL + WPB - 1) / WPB;
    __shared__ __align__(16) uint32_t sp[kWave * GPL * 16];
    __shared__ float s8[kWave * GPL];
    __shared__ float red[WPB];
    const int lane = threadIdx.x & (kWave - 1);
    // Tiles of R rows are dealt to the grid's NW wavefronts in turn: the k-th
    // tile of wavefront w holds rows (w + k NW) R .., so at any moment the
    // grid streams one contiguous window of the matrix (contiguous row
    // ranges per wavefront, 2048 separate streams, were 7% slower on the
    // 28672 x 4096 gate/up).  Wavefront j of block b deals as w = j nb + b,
    // so a last partial round spreads over every block (CU) rather than
    // filling the first ones.  Requests of a deeper ring past the
    // wavefront's last tile re-read that tile.
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * rs.nb + block;
    const int NW = rs.nb * rs.wpb, T = (a.N + R - 1) / R;
    const int nt = wid < T ? (T - wid + NW - 1) / NW : 0;
    auto trow = [&](int k) { return (wid + min(k, max(nt - 1, 0)) * NW) * R; };
    // QKV: the position (a scalar load) first, the RoPE tables and the page
    // block after the tiles; lane l holds pair l % PPT of the wavefront's
    // tile l / PPT
    constexpr int PPT = R / 2;
    const bool rope_pre = EPI == E_QKV && R % 2 == 0 && nt * PPT <= kWave;
    const int qp = EPI == E_QKV ? a.pos[0] : 0;
    StageRegs<CPT, XS> sr;
    stage_issue<CPT, XS, NT, XVEC>(a, 0, sr);
    // A CU returns load data in request order across its wavefronts: with the
    // whole CU in one block, this barrier puts every wavefront's share of x
    // ahead of every weight tile, so x arrives after one round trip instead
    // of behind the first tiles of all the other wavefronts.
    if (WPB > kWavesPerBlock) __syncthreads();
    Tile<GPL, R> t[DEPTH];
    if (!XFIRST) {
#pragma unroll
        for (int j = 0; j < DEPTH; ++j) load_tile_u<GPL, R>(t[j], a.W, a.S, a.G, 0, a.N, trow(j), lane);
    }
    float qc = 0.0f, qs = 0.0f;
    int qblk = 0;
    if (EPI == E_QKV && rope_pre) {
        const int kk = lane / max(PPT, 1), row = (wid + kk * NW) * R + 2 * (lane % max(PPT, 1));
        if (kk < nt && row < a.N && row < a.qdim + a.kvdim && a.cos_t) {
            const int i = (row % a.hd) >> 1;
            qc = a.cos_t[(size_t)qp * (a.hd >> 1) + i];
            qs = a.sin_t[(size_t)qp * (a.hd >> 1) + i];
        }
        if (a.kpool) qblk = a.block_table[qp / kPage];
    }
    if constexpr (XLDS) zero_pairs_lds<GPL, NT>(sp, s8, a.G);
    stage_finish<CPT, XS, NT>(a, sr, sp, s8, red);  // block barrier: every wavefront takes part
    // XFIRST: the first tiles are requested only once x is staged (x then
    // arrives without weight traffic queued beside it)
    if (XFIRST) {
#pragma unroll
        for (int j = 0; j < DEPTH; ++j) load_tile_u<GPL, R>(t[j], a.W, a.S, a.G, 0, a.N, trow(j), lane);
    }
    float best_v = -__builtin_inff();
    int best_i = -1;
    if (nt > 0) {
        XPairs<XLDS ? 1 : GPL> xp;
        if (!XLDS) load_pairs_lds<XLDS ? 1 : GPL>(xp, sp, s8, a.G, lane);
        float res[R];
        for (int i = 0; i < nt; i += DEPTH) {
#pragma unroll
            for (int j = 0; j < DEPTH; ++j) {
                if (i + j >= nt) break;
                if constexpr (XLDS)
                    tile_dot_lds<GPL, R>(t[j], sp, s8, a.G, lane, res);
                else
                    tile_dot<GPL, R>(t[j], xp, res);
                // the slot's next tile.  With a ring of one (QKV, wo and the
                // down projection: one or two tiles per wavefront) nothing is
                // requested past the wavefront's last tile: re-reading it was
                // a second round trip before the wavefront could end (8B
                // decode 690 -> 700 tok/s).  Deeper rings keep the request
                // unconditional (the condition made gate/up slower).
                if (DEPTH > 1 || i + j + DEPTH < nt)
                    load_tile_u<GPL, R>(t[j], a.W, a.S, a.G, 0, a.N, trow(i + j + DEPTH), lane);
                RopePre pre{};
                if (EPI == E_QKV && rope_pre) {
                    const int u0 = (i + j) * PPT;  // the lane of the tile's first pair
                    pre.valid = true;
                    pre.p = qp;
                    pre.blk = qblk;
#pragma unroll
                    for (int q = 0; q < (R + 1) / 2 && q < 4; ++q) {
                        pre.c[q] = readlane_f(qc, min(u0 + q, kWave - 1));
                        pre.s[q] = readlane_f(qs, min(u0 + q, kWave - 1));
                    }
                }
                if (lane == 0) epilogue<EPI, R>(a, 0, trow(i + j), a.N, res, best_v, best_i, &pre);
            }
        }
    }
    if (EPI == E_LOGITS) {
        // one atomic per block: the wavefronts' maxima meet in LDS first
        __shared__ unsigned long long bk[WPB];
        if (lane == 0) bk[threadIdx.x >> 6] = best_i >= 0 ? pack_best(best_v, best_i) : 0ull;
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long m = 0ull;
            for (int w = 0; w < WPB; ++w) m = bk[w] > m ? bk[w] : m;
            if (m) atomicMax(&a.best[0], m);
        }
    }
}



// Default wavefronts per CU of the batch-1 GEMV: two per SIMD.
constexpr int kB1WavesPerCU = 8;

// Grid of the batch-1 GEMV over N rows with R-row tiles: waves_per_cu
// wavefronts per CU, each with at least one full tile, in blocks of wpb
// wavefronts (rs).  share > 1: that many such grids (routed experts) divide
// the CUs.  Returns the number of blocks.
inline int b1_plan(int N, int R, int waves_per_cu, RowSplit& rs, int wpb = kWavesPerBlock, int share = 1) {
    const int units = (N + 1) / 2;
    const int min_units = (R + 1) / 2;  // at least one full tile per wavefront
    int waves = device_cus() * waves_per_cu / (share > 0 ? share : 1);
    const int maxw = (units + min_units - 1) / min_units;
    if (waves > maxw) waves = maxw;
    waves = (waves + wpb - 1) / wpb * wpb;
    rs = RowSplit{waves / wpb, wpb};
    return waves / wpb;
}

}  // namespace gv
}  // namespace nx
