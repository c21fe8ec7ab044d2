// Shared host/device definitions of the decode-loop library: the synthetic
// data generator, fp16 bit conversion, int4-g32 format constants and the
// gfx950 wavefront (64-lane) reductions built on DPP.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define NX_HD __host__ __device__ inline

namespace nx {

constexpr int kPage = 16;      // tokens per KV page
constexpr int kGroup = 32;     // int4 group size along K
constexpr int kWave = 64;      // CDNA wavefront
constexpr int kTqD = 128;      // TurboQuant head dim

// ------------------------------------------------------------ generator --
// Counter-based RNG keyed by (seed, tensor id, element index): splitmix64
// finalizer over stream = fmix(fmix(seed + G1) + tensor * G2) and
// r = fmix(stream + (index + 1) * G1).
constexpr uint64_t kG1 = 0x9E3779B97F4A7C15ull;
constexpr uint64_t kG2 = 0xD1B54A32D192ED03ull;

NX_HD uint64_t fmix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
NX_HD uint64_t stream_key(uint64_t seed, uint32_t tensor) {
    return fmix64(fmix64(seed + kG1) + (uint64_t)tensor * kG2);
}
NX_HD uint64_t rand_at(uint64_t key, uint64_t index) { return fmix64(key + (index + 1) * kG1); }
// Approximately normal: sum of the four 16-bit fields (Irwin-Hall, n = 4),
// centred and scaled by k (float nearest sigma / (2 sqrt((2^32-1)/3))).
NX_HD float normal_from(uint64_t r, float k) {
    int32_t s = (int32_t)(r & 0xFFFFu) + (int32_t)((r >> 16) & 0xFFFFu) +
                (int32_t)((r >> 32) & 0xFFFFu) + (int32_t)(r >> 48);
    return (float)(2 * s - 262140) * k;
}
inline float normal_k(double sigma) {
    return (float)(sigma / (2.0 * __builtin_sqrt((65536.0 * 65536.0 - 1.0) / 3.0)));
}

// Synthetic tensor ids (one stream per tensor).
constexpr uint32_t kTidEmbed = 1u, kTidLmHead = 2u, kTidFinalNorm = 3u, kTidStart = 5u, kTidShuffle = 7u;
NX_HD uint32_t tid_layer(int L, int kind) { return 0x100u * ((uint32_t)L + 1u) + (uint32_t)kind; }
enum { W_Q = 0, W_K = 1, W_V = 2, W_O = 3, W_GATE = 4, W_UP = 5, W_DOWN = 6, W_ROUTER = 7,
       TQ_KSIGN = 8, TQ_VSIGN = 9, N_ATTN = 10, N_FFN = 11, N_QNORM = 12, N_KNORM = 13 };
NX_HD uint32_t tid_expert(int L, int e, int w) {
    return 0x01000000u + 0x1000u * (uint32_t)L + 4u * (uint32_t)e + (uint32_t)w;
}
NX_HD uint32_t tid_ctx(int L, int b, int kv) {
    return 0x10000000u + 0x10000u * (uint32_t)L + 2u * (uint32_t)b + (uint32_t)kv;
}
NX_HD uint32_t tid_outlier(int L, int kv, int h) {
    return 0x20000000u + 0x10000u * (uint32_t)L + 0x100u * (uint32_t)kv + (uint32_t)h;
}

// ---------------------------------------------------------------- fp16 --
// IEEE binary16 round-to-nearest-even from float bits (host side; the
// device uses the hardware conversion, which rounds the same way).
inline uint16_t f32_to_f16_bits(float f) {
    uint32_t x = __builtin_bit_cast(uint32_t, f);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return (uint16_t)sign;
        uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u, sh = 126u - e;
        uint32_t r = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return (uint16_t)(sign | r);
    }
    uint32_t r = (ax >> 13) - (112u << 10), rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}
inline float f16_bits_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16, e = ((uint32_t)h >> 10) & 0x1Fu,
             m = (uint32_t)h & 0x3FFu;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (e == 31) return __builtin_bit_cast(float, sign | 0x7F800000u | (m << 13));
    return __builtin_bit_cast(float, sign | ((e + 112u) << 23) | (m << 13));
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ inline uint16_t f2h_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);  // v_cvt_f16_f32, RNE
}
__device__ inline float h2f_bits(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// ------------------------------------------------------------------ DPP --
template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF>
__device__ inline float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                           BANK_MASK, false));
}
constexpr int kQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;
constexpr int kRowBcast15 = 0x142;
constexpr int kRowBcast31 = 0x143;

// Sum over the 16 lanes of each DPP row; every lane of the row gets it.
__device__ inline float row16_sum(float v) {
    v += dpp<kQuadXor1>(v);
    v += dpp<kQuadXor2>(v);
    v += dpp<kRowHalfMirror>(v);
    v += dpp<kRowMirror>(v);
    return v;
}
__device__ inline float row16_max(float v) {
    v = fmaxf(v, dpp<kQuadXor1>(v));
    v = fmaxf(v, dpp<kQuadXor2>(v));
    v = fmaxf(v, dpp<kRowHalfMirror>(v));
    v = fmaxf(v, dpp<kRowMirror>(v));
    return v;
}
__device__ inline float readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
// Full 64-lane sum in a fixed order; the result is wave-uniform.
__device__ inline float wave_sum(float v) {
    v = row16_sum(v);
    v += dpp<kRowBcast15, 0xA>(v);
    v += dpp<kRowBcast31, 0xC>(v);
    return readlane_f(v, 63);
}
__device__ inline float wave_max(float v) {
    v = row16_max(v);
    float a = readlane_f(v, 0), b = readlane_f(v, 16), c = readlane_f(v, 32), d = readlane_f(v, 48);
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}
// Sum across the four DPP rows when every lane of a row already holds its
// row's value; the total lands in the lanes of row 3 (lanes 48..63).
__device__ inline float rows4_sum_to_row3(float v) {
    v += dpp<kRowBcast15, 0xA>(v);
    v += dpp<kRowBcast31, 0xC>(v);
    return v;
}

// Compute units of the current device (cached per device).
inline int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

}  // namespace nx
