// int4 group-32 GEMV for decode on gfx950 (CDNA4), HBM-bandwidth bound.
//
// y[b][n] = sum_g s[n][g] * sum_{k in g} (q[n][k] - 8) * x[b][k]
//
// Work split: a 64-lane wavefront owns one output row at a time and all 64
// lanes cover that row's K range, lane l holding groups g = l + 64*i
// (i < GPL).  Each lane keeps the x values of its groups in registers for
// the whole launch, pre-paired for the nibble layout, so weights are the only
// HBM stream: one 16-byte load (one group = 32 codes) plus one 2-byte scale
// per lane per row, coalesced into 1 KiB per wave instruction.  R rows are
// issued together to keep R*GPL loads in flight per lane.
//
// Dequantisation without per-code conversion: the four masks
//   A = w & 0x000F000F   (k0, k4)      B = w & 0x00F000F0   (k1, k5) * 16
//   C = (w>>8) & 0x000F000F (k2, k6)   D = (w>>8) & 0x00F000F0 (k3, k7) * 16
// of each code dword are read directly as fp16 pairs whose values are the
// codes times 2^-24 (fp16 subnormals), and v_dot2_f32_f16 multiplies them by
// the matching x pairs with fp32 accumulation.  The products are exact in
// fp32, so sum_k q_k x_k = (accA + accB/16) * 2^24 and the symmetric offset
// is removed with the group sum: sum (q-8) x = sum q x - 8 sum x.
//
// The row result is reduced across the wavefront with DPP (fixed order) and
// handed to an epilogue: plain fp16/fp32 store, residual add, QKV with RoPE
// and the paged KV append, SwiGLU of interleaved gate/up rows, or logits
// with a running argmax.  The input is either fp16 x or the fused RMSNorm of
// an fp32 hidden state, computed redundantly per wavefront.
#include "nx_common.h"
#include "nx_kernels.h"

namespace nx {

namespace {

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
    float s[R][GPL];
};

template <int GPL, int R>
__device__ inline void load_tile(Tile<GPL, R>& t, const uint8_t* __restrict__ W,
                                 const uint16_t* __restrict__ S, int G, int N, int n0,
                                 int lane) {
    const size_t rowbytes = (size_t)G * 16;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = n0 + r;
#pragma unroll
        for (int i = 0; i < GPL; ++i) {
            const int g = lane + kWave * i;
            if (row < N && g < G) {
                t.w[r][i] = *reinterpret_cast<const uint4*>(W + (size_t)row * rowbytes + 16 * (size_t)g);
                t.s[r][i] = h2f_bits(S[(size_t)row * G + g]);
            } else {
                t.w[r][i] = make_uint4(0u, 0u, 0u, 0u);
                t.s[r][i] = 0.0f;
            }
        }
    }
}

template <int GPL, int R>
__device__ inline void tile_dot(const Tile<GPL, R>& t, const XPairs<GPL>& xp, float (&res)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < GPL; ++i) acc = fmaf(group_dot(t.w[r][i], xp.p[i], xp.s8[i]), t.s[r][i], acc);
        res[r] = wave_sum(acc);
    }
}

__device__ inline unsigned long long pack_best(float v, int idx) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)ord << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)idx);
}

template <int EPI, int R>
__device__ inline void epilogue(const GemvArgs& a, int b, int n0, const float (&res)[R],
                                float& best_v, int& best_i) {
    if (EPI == E_F16) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (n0 + r < a.N) a.y16[(size_t)b * a.ldy + n0 + r] = f2h_bits(res[r]);
    } else if (EPI == E_F32) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (n0 + r < a.N) a.y32[(size_t)b * a.ldy + n0 + r] = res[r];
    } else if (EPI == E_ACC) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (n0 + r < a.N) {
                float* y = a.y32 + (size_t)b * a.ldy + n0 + r;
                *y = *y + res[r];
            }
    } else if (EPI == E_QKV) {
        const int p = a.pos[b];
        const int half = a.hd >> 1;
#pragma unroll
        for (int r = 0; r < R; r += 2) {
            const int row = n0 + r;
            if (row >= a.N) break;
            float v0 = res[r], v1 = res[r + 1];
            if (row < a.qdim + a.kvdim) {
                const int i = (row % a.hd) >> 1;
                const float c = a.cos_t[(size_t)p * half + i];
                const float s = a.sin_t[(size_t)p * half + i];
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
                    const int blk = a.block_table[(size_t)b * a.max_blocks + p / kPage];
                    uint16_t* pool = kv ? a.vpool : a.kpool;
                    const size_t off = (((size_t)blk * a.hkv + kvh) * kPage + (p % kPage)) * a.hd + dd;
                    pool[off] = f2h_bits(v0);
                    pool[off + 1] = f2h_bits(v1);
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
            if (row >= a.N) break;
            const float g = res[r], u = res[r + 1];
            a.act16[(size_t)b * a.lda + (row >> 1)] = f2h_bits(g / (1.0f + expf(-g)) * u);
        }
    } else if (EPI == E_LOGITS) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (n0 + r < a.N) {
                a.y32[(size_t)b * a.ldy + n0 + r] = res[r];
                if (res[r] > best_v) {
                    best_v = res[r];
                    best_i = n0 + r;
                }
            }
    }
}

constexpr int kB1MaxThreads = 512;

// Block-cooperative staging of one x row into LDS in the pair layout:
// sp[g*16 + 4d + j] = (x[32g+8d+j], x[32g+8d+j+4]) and s8[g] = 8 * sum of
// group g.  Each thread converts 8-element chunks; for X_RMSNORM the block
// first reduces sum(h^2) once, so the hidden state is read twice per block
// rather than per wavefront.  Ends with a barrier.
template <int XS>
__device__ inline void stage_x(const GemvArgs& a, int b, uint32_t* sp, float* s8, float* red) {
    const int K = a.K, nch = a.G * 4;
    const int tid = threadIdx.x, nthr = blockDim.x;
    float inv = 1.0f;
    const float* h = a.h32 + (size_t)b * a.ldx;
    const uint16_t* x = a.x16 + (size_t)b * a.ldx;
    if (XS == X_RMSNORM) {
        float ss = 0.0f;
        for (int c = tid; c < nch; c += nthr) {
            const int k0 = 8 * c;
            if (k0 + 8 <= K && ((reinterpret_cast<uintptr_t>(h + k0) & 15u) == 0)) {
                const float4 v0 = *reinterpret_cast<const float4*>(h + k0);
                const float4 v1 = *reinterpret_cast<const float4*>(h + k0 + 4);
                ss += v0.x * v0.x;
                ss += v0.y * v0.y;
                ss += v0.z * v0.z;
                ss += v0.w * v0.w;
                ss += v1.x * v1.x;
                ss += v1.y * v1.y;
                ss += v1.z * v1.z;
                ss += v1.w * v1.w;
            } else {
                for (int j = 0; j < 8; ++j)
                    if (k0 + j < K) ss += h[k0 + j] * h[k0 + j];
            }
        }
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float tot = 0.0f;
        for (int w = 0; w < (nthr >> 6); ++w) tot += red[w];
        inv = 1.0f / sqrtf(tot / (float)K + a.eps);
    }
    for (int c = tid; c < nch; c += nthr) {
        const int k0 = 8 * c;
        uint32_t X[4];
        if (XS == X_F16) {
            if (k0 + 8 <= K && ((reinterpret_cast<uintptr_t>(x + k0) & 15u) == 0)) {
                const uint4 v = *reinterpret_cast<const uint4*>(x + k0);
                X[0] = v.x;
                X[1] = v.y;
                X[2] = v.z;
                X[3] = v.w;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t lo = k0 + 2 * j < K ? x[k0 + 2 * j] : 0u;
                    const uint32_t hi = k0 + 2 * j + 1 < K ? x[k0 + 2 * j + 1] : 0u;
                    X[j] = lo | (hi << 16);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t lo = 0, hi = 0;
                const int k = k0 + 2 * j;
                if (k < K) {
                    const float v = h[k] * inv;
                    lo = f2h_bits(a.norm_w ? v * a.norm_w[k] : v);
                }
                if (k + 1 < K) {
                    const float v = h[k + 1] * inv;
                    hi = f2h_bits(a.norm_w ? v * a.norm_w[k + 1] : v);
                }
                X[j] = lo | (hi << 16);
            }
        }
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

// Batch 1.
template <int GPL, int R, int XS, int EPI>
__global__ __launch_bounds__(kB1MaxThreads) void k_gemv_b1(GemvArgs a) {
    __shared__ uint32_t sp[kWave * GPL * 16];
    __shared__ float s8[kWave * GPL];
    __shared__ float red[kB1MaxThreads / kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wpb = blockDim.x >> 6;
    const int wid = blockIdx.x * wpb + (threadIdx.x >> 6);
    const int nw = gridDim.x * wpb;
    stage_x<XS>(a, 0, sp, s8, red);
    XPairs<GPL> xp;
    load_pairs_lds<GPL>(xp, sp, s8, a.G, lane);
    float best_v = -__builtin_inff();
    int best_i = -1;
    for (int n0 = wid * R; n0 < a.N; n0 += nw * R) {
        Tile<GPL, R> t;
        load_tile<GPL, R>(t, a.W, a.S, a.G, a.N, n0, lane);
        float res[R];
        tile_dot<GPL, R>(t, xp, res);
        if (lane == 0) epilogue<EPI, R>(a, 0, n0, res, best_v, best_i);
    }
    if (EPI == E_LOGITS && lane == 0 && best_i >= 0) atomicMax(&a.best[0], pack_best(best_v, best_i));
}

// Batch 2..8: the weight tile is loaded once and applied to every row of x.
template <int GPL, int R, int XS, int EPI>
__global__ __launch_bounds__(kBlockThreads) void k_gemv_bn(GemvArgs a) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const int nw = gridDim.x * kWavesPerBlock;
    float inv[8];
    if (XS == X_RMSNORM) {
        for (int b = 0; b < a.batch; ++b)
            inv[b] = rms_inv<GPL>(a.h32 + (size_t)b * a.ldx, a.K, a.G, a.eps, lane);
    }
    float best_v[8];
    int best_i[8];
    for (int b = 0; b < 8; ++b) {
        best_v[b] = -__builtin_inff();
        best_i[b] = -1;
    }
    for (int n0 = wid * R; n0 < a.N; n0 += nw * R) {
        Tile<GPL, R> t;
        load_tile<GPL, R>(t, a.W, a.S, a.G, a.N, n0, lane);
        for (int b = 0; b < a.batch; ++b) {
            XPairs<GPL> xp;
            if (XS == X_F16)
                load_x16<GPL>(xp, a.x16 + (size_t)b * a.ldx, a.K, a.G, lane);
            else
                load_x_norm<GPL>(xp, a.h32 + (size_t)b * a.ldx, a.norm_w, inv[b], a.K, a.G, lane);
            float res[R];
            tile_dot<GPL, R>(t, xp, res);
            if (lane == 0) epilogue<EPI, R>(a, b, n0, res, best_v[b], best_i[b]);
        }
    }
    if (EPI == E_LOGITS && lane == 0)
        for (int b = 0; b < a.batch; ++b)
            if (best_i[b] >= 0) atomicMax(&a.best[b], pack_best(best_v[b], best_i[b]));
}

// MoE expert GEMV with gathered tokens: blockIdx.y is the expert; its rows
// are applied to every token slot routed to it (expert_slots), so each
// active expert's weights are read once per step whatever the batch.
//   GATEUP: rows (2f, 2f+1) = (gate f, up f) of w13[e]; x = x16 of the slot's
//           sequence; act16[slot][f] = fp16(silu(g) * u).
//   down:   rows of w2[e]; x = act16[slot]; y32[slot][n] = y.
template <int GPL, int R, bool GATEUP>
__global__ __launch_bounds__(kBlockThreads) void k_moe_gemv(MoeFfnArgs m) {
    const int e = blockIdx.y;
    const int ntok = m.expert_count[e];
    if (ntok == 0) return;
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const int nw = gridDim.x * kWavesPerBlock;
    const int Fp = (m.F + 31) / 32 * 32;
    const int N = GATEUP ? 2 * m.F : m.d;
    const int K = GATEUP ? m.d : m.F;
    const int G = (K + 31) / 32;
    const uint8_t* W = (GATEUP ? m.w13 : m.w2) + (size_t)e * N * G * 16;
    const uint16_t* S = (GATEUP ? m.s13 : m.s2) + (size_t)e * N * G;
    const int32_t* slots = m.expert_slots + (size_t)e * m.batch * m.k;
    for (int n0 = wid * R; n0 < N; n0 += nw * R) {
        Tile<GPL, R> t;
        load_tile<GPL, R>(t, W, S, G, N, n0, lane);
        for (int i = 0; i < ntok; ++i) {
            const int slot = slots[i];
            XPairs<GPL> xp;
            if (GATEUP)
                load_x16<GPL>(xp, m.x16 + (size_t)(slot / m.k) * m.ldx, K, G, lane);
            else
                load_x16<GPL>(xp, m.act16 + (size_t)slot * Fp, K, G, lane);
            float res[R];
            tile_dot<GPL, R>(t, xp, res);
            if (lane == 0) {
                if (GATEUP) {
#pragma unroll
                    for (int r = 0; r < R; r += 2) {
                        const int row = n0 + r;
                        if (row >= N) break;
                        const float g = res[r], u = res[r + 1];
                        m.act16[(size_t)slot * Fp + (row >> 1)] = f2h_bits(g / (1.0f + expf(-g)) * u);
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        if (n0 + r < N) m.y32[(size_t)slot * m.d + n0 + r] = res[r];
                }
            }
        }
    }
}

template <bool GATEUP>
hipError_t moe_launch(const MoeFfnArgs& m, hipStream_t st) {
    const int N = GATEUP ? 2 * m.F : m.d;
    const int K = GATEUP ? m.d : m.F;
    const int G = (K + 31) / 32;
    const int gpl = (G + kWave - 1) / kWave;
    auto blocks_for = [&](int R) {
        int b = ((N + R - 1) / R + kWavesPerBlock - 1) / kWavesPerBlock;
        return b > 512 ? 512 : b;
    };
    if (gpl <= 1) {
        hipLaunchKernelGGL((k_moe_gemv<1, 4, GATEUP>), dim3(blocks_for(4), m.E), dim3(kBlockThreads), 0, st, m);
    } else if (gpl <= 2) {
        hipLaunchKernelGGL((k_moe_gemv<2, 4, GATEUP>), dim3(blocks_for(4), m.E), dim3(kBlockThreads), 0, st, m);
    } else if (gpl <= 4) {
        hipLaunchKernelGGL((k_moe_gemv<4, 2, GATEUP>), dim3(blocks_for(2), m.E), dim3(kBlockThreads), 0, st, m);
    } else if (gpl <= 7) {
        hipLaunchKernelGGL((k_moe_gemv<7, 2, GATEUP>), dim3(blocks_for(2), m.E), dim3(kBlockThreads), 0, st, m);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int GPL, int R, int XS, int EPI>
hipError_t launch_t(const GemvArgs& a, hipStream_t st) {
    const int tiles = (a.N + R - 1) / R;
    if (a.batch == 1) {
        // one wavefront per R-row tile; wavefronts per block chosen so the
        // grid covers the 256 CUs, up to 8 per block (2 blocks of 8 per CU
        // fit when the kernel stays under 128 VGPRs, 1 block otherwise)
        int wpb = 1;
        while (wpb < 8 && tiles >= 256 * wpb * 2) wpb *= 2;
        int blocks = (tiles + wpb - 1) / wpb;
        const int cap = GPL >= 7 ? 256 : 512;
        if (wpb == 8 && blocks > cap) blocks = cap;
        hipLaunchKernelGGL((k_gemv_b1<GPL, R, XS, EPI>), dim3(blocks), dim3(wpb * kWave), 0, st, a);
        return hipGetLastError();
    }
    int blocks = (tiles + kWavesPerBlock - 1) / kWavesPerBlock;
    if (blocks > 1024) blocks = 1024;
    hipLaunchKernelGGL((k_gemv_bn<GPL, R, XS, EPI>), dim3(blocks), dim3(kBlockThreads), 0, st, a);
    return hipGetLastError();
}

template <int XS, int EPI>
hipError_t launch_gpl(const GemvArgs& a, hipStream_t st) {
    const int gpl = (a.G + kWave - 1) / kWave;
    if (gpl <= 1) return launch_t<1, 4, XS, EPI>(a, st);
    if (gpl <= 2) return launch_t<2, 4, XS, EPI>(a, st);
    if (gpl <= 4) return launch_t<4, 2, XS, EPI>(a, st);
    if (gpl <= 7) return launch_t<7, 2, XS, EPI>(a, st);
    return hipErrorInvalidValue;
}

}  // namespace

hipError_t gemv_launch(int xsrc, int epi, const GemvArgs& a, hipStream_t st) {
    if (a.batch < 1 || a.batch > 8) return hipErrorInvalidValue;
    if (xsrc == X_F16) {
        switch (epi) {
            case E_F16: return launch_gpl<X_F16, E_F16>(a, st);
            case E_F32: return launch_gpl<X_F16, E_F32>(a, st);
            case E_ACC: return launch_gpl<X_F16, E_ACC>(a, st);
            default: return hipErrorInvalidValue;
        }
    }
    switch (epi) {
        case E_F32: return launch_gpl<X_RMSNORM, E_F32>(a, st);
        case E_QKV: return launch_gpl<X_RMSNORM, E_QKV>(a, st);
        case E_SWIGLU: return launch_gpl<X_RMSNORM, E_SWIGLU>(a, st);
        case E_LOGITS: return launch_gpl<X_RMSNORM, E_LOGITS>(a, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t moe_gate_up_launch(const MoeFfnArgs& a, hipStream_t st) { return moe_launch<true>(a, st); }
hipError_t moe_down_launch(const MoeFfnArgs& a, hipStream_t st) { return moe_launch<false>(a, st); }

}  // namespace nx
