// int4 group-32 GEMV for decode on gfx950 (CDNA4), HBM-bandwidth bound.
//
// y[b][n] = sum_g s[n][g] * sum_{k in g} (q[n][k] - 8) * x[b][k]
//
// Work split: a 64-lane wavefront owns one output row at a time and all 64
// lanes cover that row's K range, lane l holding groups g = l + 64*i
// (i < GPL).  Each lane keeps the x values of its groups in registers for
// the whole launch, pre-paired for the nibble layout, so weights are the only
// HBM stream: one 16-byte load (one group = 32 codes) plus one 2-byte scale
// per lane per row, coalesced into 1 KiB per wave instruction.  R rows form a
// tile whose R*GPL loads are in flight together.  At batch 1 the grid is
// persistent (one block of 8 wavefronts per CU), the tiles are dealt to the
// wavefronts in turn (the grid streams one window of the matrix at a time),
// each wavefront requests its next tile before the current one is reduced,
// and the first tiles are requested right after the input.  The
// loads up to the first wait are straight-line code, so the wait for the
// input counts the tile loads behind it instead of waiting for all of them.
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
// an fp32 hidden state, computed once per block into LDS.
#include <algorithm>
#include <type_traits>

#include "nx_gemv_dev.h"

namespace nx {

namespace {

using namespace gv;

// Batch 1 kernel: the whole grid runs one GEMV, one block of WPB
// wavefronts per CU.
template <int GPL, int R, int DEPTH, bool XLDS, int XS, int EPI, int WPB, bool XVEC, bool XFIRST, bool MOE = false>
__global__ __launch_bounds__(WPB * kWave, 1) void k_gemv_b1(GemvArgs a, RowSplit rs) {
    if constexpr (MOE) {
        // routed expert of grid row y, one token slot (batch 1)
        const int32_t* pl = a.moe_plan + blockIdx.y * kMoePlanInts;
        const int e = pl[0];
        if (e < 0) return;
        const int slot = pl[8], xr = a.moe_xslot ? slot : pl[16];
        GemvArgs m = a;
        m.W += (size_t)e * a.moe_wstride;
        m.S += (size_t)e * a.moe_sstride;
        m.x16 += (size_t)xr * a.ldx;
        m.act16 += (size_t)slot * a.lda;
        m.y32 += (size_t)slot * a.ldy;
        gemv_b1_run<GPL, R, DEPTH, XLDS, XS, EPI, WPB, XVEC, XFIRST>(m, rs, blockIdx.x);
    } else {
        gemv_b1_run<GPL, R, DEPTH, XLDS, XS, EPI, WPB, XVEC, XFIRST>(a, rs, blockIdx.x);
    }
}

// ---------------------------------------------------------- batch 2..8 --
// The weights of 16 rows meet the batch's x on the matrix cores
// (v_mfma_f32_16x16x32_f16, one 32-element group per product):
//   A (16 x 32): lane l holds row l%16, k = 8(l/16) .. +7 of the group: its
//      code dword gives the fp16 values (q - 8) in the k order
//      (0 4 1 5 2 6 3 7): a low nibble ORed into 0x6400 is 1024 + q and a high
//      nibble 1024 + 16 q, both exact in fp16 (codes_to_h8);
//   B (32 x 16): lane l holds batch column l%16 with the same k order (x is
//      staged in LDS in that order; columns past the batch are never stored);
//   C (16 x 16 fp32): lane l holds column l%16, rows 4(l/16) .. +3.
// Each product is a group sum (exact int4 x fp16 products, fp32 sums), which
// is scaled by its row's group scale and accumulated in fp32, as in the
// batch-1 kernel.  A block of 8 wavefronts takes whole 16-row tiles; K up to
// 4096 is staged in LDS once, and the wavefronts stream (tile, 16-group pass)
// items.  Longer K with fp16 x (the down projection) streams the same way
// with each wavefront owning an eighth of K and loading its x straight from
// memory with the weights (x is small and stays in the L2).  The
// wavefronts' partial tiles meet in LDS.  Every load before a wait is
// unconditional (clamped rows, groups and stage entries), so the compiler's
// waits count exactly.
typedef _Float16 mh8_t __attribute__((ext_vector_type(8)));
typedef float mf4_t __attribute__((ext_vector_type(4)));


constexpr int kMfmaWaves = 8;
constexpr int kMfmaThreads = kMfmaWaves * kWave;
constexpr int kMfmaCols = 8;                       // batch rows held in LDS
constexpr int kMfmaKC = 4096;                      // K per stage
constexpr int kMfmaGC = kMfmaKC / 32;              // groups per stage
constexpr int kMfmaGW = kMfmaGC / kMfmaWaves;      // groups per wavefront per stage
constexpr int kMfmaEPT = kMfmaGC * 4 * kMfmaCols / kMfmaThreads;  // stage entries per thread

typedef _Float16 mh2_t __attribute__((ext_vector_type(2)));

// The 8 codes of a dword as fp16 (q - 8) in the k order (0 4 1 5 2 6 3 7):
// byte i holds k = 2i (low nibble) and 2i + 1 (high nibble).  (w & 0x000F000F)
// | 0x64006400 is the pair (1024 + q0, 1024 + q4); with mask 0x00F000F0 it is
// (1024 + 16 q1, 1024 + 16 q5); w >> 8 gives k 2, 6 and 3, 7 the same way.
// Then q - 8 = t - 1032 or t / 16 - 72, exact (one rounding of an exact
// value) -- four v_and_or_b32, one shift, two packed adds, two packed fmas.
// (w & mask) | bits in one instruction (the compiler splits it in two when
// both constants are literals); mask in a VGPR, bits in an SGPR.
__device__ inline uint32_t and_or(uint32_t w, uint32_t mask, uint32_t bits) {
    uint32_t d;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(w), "v"(mask), "s"(bits));
    return d;
}

__device__ inline mh8_t codes_to_h8(uint32_t w) {
    const uint32_t m = 0x64006400u, w8 = w >> 8;
    const mh2_t a = __builtin_bit_cast(mh2_t, and_or(w, 0x000F000Fu, m));
    const mh2_t b = __builtin_bit_cast(mh2_t, and_or(w, 0x00F000F0u, m));
    const mh2_t c = __builtin_bit_cast(mh2_t, and_or(w8, 0x000F000Fu, m));
    const mh2_t d = __builtin_bit_cast(mh2_t, and_or(w8, 0x00F000F0u, m));
    const mh2_t off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const mh2_t sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f}, off16 = {(_Float16)-72.0f, (_Float16)-72.0f};
    const mh2_t r0 = a + off, r1 = __builtin_elementwise_fma(b, sixteenth, off16);
    const mh2_t r2 = c + off, r3 = __builtin_elementwise_fma(d, sixteenth, off16);
    return mh8_t{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
}

// Eight consecutive fp16 inputs (as 4 dwords) in the k order (0 4 1 5 2 6 3 7).
__device__ inline uint4 perm_x8(const uint32_t (&X)[4]) {
    return make_uint4(__builtin_amdgcn_perm(X[2], X[0], 0x05040100u), __builtin_amdgcn_perm(X[2], X[0], 0x07060302u),
                      __builtin_amdgcn_perm(X[3], X[1], 0x05040100u), __builtin_amdgcn_perm(X[3], X[1], 0x07060302u));
}

// The x values of a thread's stage entries, held between the requests and
// their use (XVEC staging).
template <int XS>
struct StageRegs {
    uint32_t X[kMfmaEPT][4];
    float V[XS == X_RMSNORM ? kMfmaEPT : 1][8];
    float NW[XS == X_RMSNORM ? kMfmaEPT : 1][8];
};

// XVEC staging, first half: request the thread's entries (all before any
// use).  The norm weights are requested only when there are any.
template <int XS>
__device__ inline void stage_issue(const GemvArgs& a, int k0, int gc, StageRegs<XS>& r, int xrow) {
    const int tid = threadIdx.x, K = a.K, ne = gc * 4 * kMfmaCols, nb = a.batch;
    const bool has_w = a.norm_w != nullptr;
#pragma unroll
    for (int j = 0; j < kMfmaEPT; ++j) {
        const int e = min(tid + j * kMfmaThreads, ne - 1);
        const int b = min(e % kMfmaCols, nb - 1), q = (e / kMfmaCols) & 3, g = e / (4 * kMfmaCols);
        const int kb = min(k0 + 32 * g + 8 * q, K - 8);
        const size_t xo = (size_t)(xrow >= 0 ? xrow : b) * a.ldx + kb;
        if (XS == X_F16) {
            const uint4 v = *reinterpret_cast<const uint4*>(a.x16 + xo);
            r.X[j][0] = v.x; r.X[j][1] = v.y; r.X[j][2] = v.z; r.X[j][3] = v.w;
        } else {
            const float4* src = reinterpret_cast<const float4*>(a.h32 + xo);
            const float4 u = src[0], w = src[1];
            r.V[j][0] = u.x; r.V[j][1] = u.y; r.V[j][2] = u.z; r.V[j][3] = u.w;
            r.V[j][4] = w.x; r.V[j][5] = w.y; r.V[j][6] = w.z; r.V[j][7] = w.w;
        }
    }
    if (XS == X_RMSNORM && has_w) {
#pragma unroll
        for (int j = 0; j < kMfmaEPT; ++j) {
            const int e = min(tid + j * kMfmaThreads, ne - 1);
            const int q = (e / kMfmaCols) & 3, g = e / (4 * kMfmaCols);
            const int kb = min(k0 + 32 * g + 8 * q, K - 8);
            const float4* ws = reinterpret_cast<const float4*>(a.norm_w + kb);
            const float4 wu = ws[0], ww = ws[1];
            r.NW[j][0] = wu.x; r.NW[j][1] = wu.y; r.NW[j][2] = wu.z; r.NW[j][3] = wu.w;
            r.NW[j][4] = ww.x; r.NW[j][5] = ww.y; r.NW[j][6] = ww.z; r.NW[j][7] = ww.w;
        }
    }
}

// XVEC staging, second half: (NORM: 1/rms per batch row from the staged
// values, reduced through LDS in red) convert and store the entries.
template <int XS, bool NORM>
__device__ inline void stage_finish(const GemvArgs& a, int k0, int gc, StageRegs<XS>& r, uint4* xs, float* inv,
                                    float (*red)[kMfmaCols]) {
    const int tid = threadIdx.x, K = a.K, ne = gc * 4 * kMfmaCols, nb = a.batch;
    const bool has_w = a.norm_w != nullptr;
    if (XS == X_RMSNORM && NORM) {
        // a thread's entries all belong to batch row tid % kMfmaCols
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < kMfmaEPT; ++j) {
            const int e = tid + j * kMfmaThreads;
            const int kb = k0 + 32 * (e / (4 * kMfmaCols)) + 8 * ((e / kMfmaCols) & 3);
            if (e < ne && kb < K)
#pragma unroll
                for (int h = 0; h < 8; ++h) ss = fmaf(r.V[j][h], r.V[j][h], ss);
        }
        // lanes with the same tid % kMfmaCols: a stride-8 sum within the wavefront
        ss += __shfl_xor(ss, 8, kWave);
        ss += __shfl_xor(ss, 16, kWave);
        ss += __shfl_xor(ss, 32, kWave);
        const int lane = tid & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        if (lane < kMfmaCols) red[wave][lane] = ss;
        __syncthreads();
        if (tid < kMfmaCols) {
            float t = 0.0f;
            for (int w = 0; w < kMfmaWaves; ++w) t += red[w][tid];
            inv[tid] = 1.0f / sqrtf(t / (float)K + a.eps);
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < kMfmaEPT; ++j) {
        const int e = tid + j * kMfmaThreads;
        if (e >= ne) break;
        const int b = e % kMfmaCols, q = (e / kMfmaCols) & 3, g = e / (4 * kMfmaCols);
        const int kb = k0 + 32 * g + 8 * q;
        if (b >= nb) continue;
        if (XS == X_RMSNORM) {
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const int k = kb + 2 * h;
                const float t0 = r.V[j][2 * h] * inv[b], t1 = r.V[j][2 * h + 1] * inv[b];
                const uint32_t lo = k < K ? f2h_bits(has_w ? t0 * r.NW[j][2 * h] : t0) : 0u;
                const uint32_t hi = k + 1 < K ? f2h_bits(has_w ? t1 * r.NW[j][2 * h + 1] : t1) : 0u;
                r.X[j][h] = lo | (hi << 16);
            }
        } else if (kb >= K) {
            r.X[j][0] = r.X[j][1] = r.X[j][2] = r.X[j][3] = 0u;
        }
        xs[e] = perm_x8(r.X[j]);
    }
}

// Stage x[b][k0 .. k0 + 32 gc) of every batch row into LDS: entry
// (g * 4 + q) * kMfmaCols + b holds x[b][k0 + 32g + 8q + (0 4 1 5 2 6 3 7)].
// XVEC: K % 8 == 0 and 16-byte aligned rows, one 16-byte load per entry (X_F16)
// or two (X_RMSNORM); all loads of a thread are issued before any is used.
// X_RMSNORM needs inv[b] = 1 / sqrt(mean(h_b^2) + eps).
// NORM (X_RMSNORM, K in one stage): inv is computed here from the staged
// values (sums of squares per batch row over the thread's entries, reduced
// through LDS in red), so the input costs one round trip.
template <int XS, bool XVEC, bool NORM = false>
__device__ inline void mfma_stage_x(const GemvArgs& a, int k0, int gc, uint4* xs, float* inv,
                                    float (*red)[kMfmaCols] = nullptr, int xrow = -1) {
    const int tid = threadIdx.x, K = a.K, ne = gc * 4 * kMfmaCols, nb = a.batch;
    if (XVEC) {
        StageRegs<XS> r;
        stage_issue<XS>(a, k0, gc, r, xrow);
        stage_finish<XS, NORM>(a, k0, gc, r, xs, inv, red);
        return;
    }
    for (int e = tid; e < ne; e += kMfmaThreads) {
        const int b = e % kMfmaCols, q = (e / kMfmaCols) & 3, g = e / (4 * kMfmaCols);
        if (b >= nb) continue;
        const int kb = k0 + 32 * g + 8 * q;
        const size_t xo = (size_t)(xrow >= 0 ? xrow : b) * a.ldx;
        uint32_t X[4];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const int k = kb + 2 * h;
            uint32_t lo = 0, hi = 0;
            if (XS == X_F16) {
                if (k < K) lo = a.x16[xo + k];
                if (k + 1 < K) hi = a.x16[xo + k + 1];
            } else {
                if (k < K) lo = f2h_bits(a.h32[xo + k] * inv[b] * (a.norm_w ? a.norm_w[k] : 1.0f));
                if (k + 1 < K)
                    hi = f2h_bits(a.h32[xo + k + 1] * inv[b] * (a.norm_w ? a.norm_w[k + 1] : 1.0f));
            }
            X[h] = lo | (hi << 16);
        }
        xs[e] = perm_x8(X);
    }
}

// The product of one group is one MFMA with the batch's x as A (row = batch
// row, k-quad l/16 of lane l) and the weight codes as B (column = weight row
// l%16, same k-quad), so lane l's accumulators hold weight row l%16 for batch
// rows 4(l/16)..+3 and every lane needs one scale per group.
//
// One wavefront's share (groups [gs, ge) of the stage starting at group
// gbase) of a 16-row tile, requested without branches: lane (c, kq) loads the
// whole 16-byte groups gs + 4u + kq (u < 4) of row c, so each request moves
// 16 bytes per lane (64 contiguous bytes of each of the 16 rows); the MFMA
// needs quarter kq of every group in lane row kq, which a 4 x 4 exchange
// across the four 16-lane rows provides (quad_transpose).  SALIGN: G % 8 == 0
// and 16-byte aligned scales, so a lane's 16 scales (row c, groups gs ..
// gs + 15, gs a multiple of 16) are two 16-byte loads, half the requests and
// cache-line lookups of four 8-byte loads (128256 x 4096 at batch 8: 72.6 us
// with four, 67.5 with two, 59.2 with no scale loads at all).  XG items start
// at any group, so they keep 8-byte loads (G % 4 == 0).
// XG: the wavefront's x of the item's groups too (x loaded from memory with
// the weights instead of staged in LDS), lane (c, kq) holding quarter kq of
// each group for batch row c % 8.
template <bool XG = false>
struct MfmaRegs {
    uint4 code[kMfmaGW / 4];
    uint32_t sc[kMfmaGW / 2];  // fp16 scale pairs (groups 2u, 2u+1) of the lane's weight row
    uint4 x[XG ? kMfmaGW : 1];
};

// keep = 0: a request with no use (past the block's last tile); every lane
// then reads the first 16 bytes of row min(row0, N-1) of the stage, one cache
// line.  FULL: groups gs .. gs + 15 all exist (no clamping).  XG: x of the
// same groups from row offset xoff.
template <bool SALIGN, bool FULL, bool XG>
__device__ inline void mfma_load(const GemvArgs& a, int row0, int gbase, int gs, int ge, MfmaRegs<XG>& r,
                                 int keep = 1, size_t xoff = 0) {
    const int lane = threadIdx.x & (kWave - 1), c = lane & 15, kq = lane >> 4;
    const int G = a.G;
    const int gl = ge - 1;  // last group of the stage (ge == stage groups when the wavefront has none)
    const size_t row = (size_t)min(row0 + c * keep, a.N - 1);
    const uint16_t* srow = a.S + row * G + gbase;
    if (SALIGN && !XG) {
        // a stage's group count is a multiple of 8, so the clamped load stays
        // inside the stage's groups of the row
#pragma unroll
        for (int h = 0; h < kMfmaGW / 8; ++h) {
            const int g = FULL ? gs + 8 * h : min(gs + 8 * h, gl & ~7);
            const uint4 v = *reinterpret_cast<const uint4*>(srow + g * keep);
            r.sc[4 * h] = v.x;
            r.sc[4 * h + 1] = v.y;
            r.sc[4 * h + 2] = v.z;
            r.sc[4 * h + 3] = v.w;
        }
    } else if (SALIGN) {
#pragma unroll
        for (int u4 = 0; u4 < kMfmaGW / 4; ++u4) {
            const int g = FULL ? gs + 4 * u4 : min(gs + 4 * u4, gl & ~3);
            const uint2 v = *reinterpret_cast<const uint2*>(srow + g * keep);
            r.sc[2 * u4] = v.x;
            r.sc[2 * u4 + 1] = v.y;
        }
    } else {
#pragma unroll
        for (int u2 = 0; u2 < kMfmaGW / 2; ++u2)
            r.sc[u2] = (uint32_t)srow[min(gs + 2 * u2, gl) * keep] |
                       ((uint32_t)srow[min(gs + 2 * u2 + 1, gl) * keep] << 16);
    }
    const uint8_t* wrow = a.W + row * G * 16 + (size_t)gbase * 16;
#pragma unroll
    for (int u4 = 0; u4 < kMfmaGW / 4; ++u4) {
        const int g = FULL ? gs + 4 * u4 + kq : min(gs + 4 * u4 + kq, gl);
        r.code[u4] = *reinterpret_cast<const uint4*>(wrow + (size_t)(g * keep) * 16);
    }
    if constexpr (XG) {
#pragma unroll
        for (int u = 0; u < kMfmaGW; ++u)
            r.x[u] = *reinterpret_cast<const uint4*>(a.x16 + xoff + 32 * min(gs + u, gl) + 8 * kq);
    }
}

// 4 x 4 exchange across the 16-lane rows: on entry lane row r holds the four
// quarters (q.x .. q.w) of group 4u + r; on exit register j holds, in lane
// row r, quarter r of group 4u + j.  v_permlane32_swap exchanges the upper
// half of its first operand with the lower half of its second, and
// v_permlane16_swap the odd rows of the first with the even rows of the
// second.
__device__ inline void quad_transpose(const uint4& q, uint32_t (&o)[4]) {
    const auto p02 = __builtin_amdgcn_permlane32_swap(q.x, q.z, false, false);
    const auto p13 = __builtin_amdgcn_permlane32_swap(q.y, q.w, false, false);
    const auto s01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
    const auto s23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
    o[0] = s01[0];
    o[1] = s01[1];
    o[2] = s23[0];
    o[3] = s23[1];
}

// The A operands (x of the batch) of the wavefront's groups, from LDS.
template <bool FULL>
__device__ inline void mfma_load_x(const uint4* xs, int gs, int ge, uint4 (&xv)[kMfmaGW]) {
    const int lane = threadIdx.x & (kWave - 1), c = lane & 15, kq = lane >> 4;
    const int gl = ge - 1;
#pragma unroll
    for (int u = 0; u < kMfmaGW; ++u)
        xv[u] = xs[((FULL ? gs + u : min(gs + u, gl)) * 4 + kq) * kMfmaCols + (c & (kMfmaCols - 1))];
}

// The A operands from an XG item's registers, in the MFMA's k order.
__device__ inline void mfma_perm_x(const uint4 (&x)[kMfmaGW], uint4 (&xv)[kMfmaGW]) {
#pragma unroll
    for (int u = 0; u < kMfmaGW; ++u) {
        const uint32_t X[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
        xv[u] = perm_x8(X);
    }
}

// Group sums of the wavefront's share, scaled and accumulated into acc
// (fully unrolled, so the register arrays stay in registers; unless FULL,
// groups past ge repeat a valid group with weight zero).
template <bool FULL, bool XG>
__device__ inline void mfma_compute(const MfmaRegs<XG>& r, const uint4 (&xv)[kMfmaGW], int gs, int ge, mf4_t& acc) {
    uint32_t code[kMfmaGW];
#pragma unroll
    for (int u4 = 0; u4 < kMfmaGW / 4; ++u4) {
        uint32_t o[4];
        quad_transpose(r.code[u4], o);
#pragma unroll
        for (int j = 0; j < 4; ++j) code[4 * u4 + j] = o[j];
    }
    // group u's product is requested before group u - 1's is scaled and
    // accumulated, so the conversion of u's codes, not wait states, covers
    // the matrix core's latency
    const mf4_t z = {0.f, 0.f, 0.f, 0.f};
    auto product = [&](int u) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mh8_t, xv[u]), codes_to_h8(code[u]), z, 0,
                                                      0, 0);
    };
    auto fold = [&](int u, const mf4_t& cg) {
        const uint32_t pr = r.sc[u >> 1];
        float sv = h2f_bits((uint16_t)((u & 1) ? (pr >> 16) : (pr & 0xFFFFu)));
        if (!FULL) sv *= gs + u < ge ? 1.0f : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = fmaf(cg[i], sv, acc[i]);
    };
    mf4_t prev = product(0);
#pragma unroll
    for (int u = 1; u < kMfmaGW; ++u) {
        const mf4_t cg = product(u);
        fold(u - 1, prev);
        prev = cg;
    }
    fold(kMfmaGW - 1, prev);
}

// FULL: K <= 4096 and every wavefront's K slice is whole passes of 16 groups.
template <int XS, int EPI, bool XVEC, bool SALIGN, bool MOE, bool FULL>
__global__ __launch_bounds__(kMfmaThreads, 1) void k_gemv_mfma(GemvArgs args, int nb, int ks) {
    __shared__ __align__(16) uint4 xs[kMfmaGC * 4 * kMfmaCols];
    __shared__ __align__(16) float part[2][kMfmaWaves * 16 * kMfmaCols];  // [wave][weight row][batch row]
    __shared__ float inv[kMfmaCols];
    __shared__ float red[kMfmaWaves][kMfmaCols];
    __shared__ unsigned long long bk[kMfmaThreads];
    // The arguments the prologue uses, requested together: the compiler
    // would otherwise fetch them from the argument segment in several
    // dependent rounds as each is first needed.
    asm volatile("" ::"s"(args.W), "s"(args.S), "s"(args.x16), "s"(args.h32), "s"(args.N), "s"(args.K),
                 "s"(args.G), "s"(args.batch), "s"(args.ldx), "s"(args.kparts), "s"(args.moe_plan), "s"(nb),
                 "s"(ks));
    if constexpr (EPI == E_SWIGLU) asm volatile("" ::"s"(args.act16), "s"(args.lda));
    if constexpr (EPI == E_ACC || EPI == E_F32) asm volatile("" ::"s"(args.y32), "s"(args.ldy));
    if constexpr (EPI == E_PART) asm volatile("" ::"s"(args.kpart), "s"(args.kpart_rows));
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 15, kq = lane >> 4;
    const int N = args.N, K = args.K;
    // E_PART: block x is row group x / kparts over K part x % kparts, groups
    // [gbase0, gbase0 + Gx); otherwise all of K
    int bx = blockIdx.x, gq = 0, gbase0 = 0, Gx = args.G;
    if constexpr (EPI == E_PART) {
        gq = blockIdx.x % args.kparts;
        bx = blockIdx.x / args.kparts;
        const int gpp = ((args.G + args.kparts - 1) / args.kparts + kMfmaGW - 1) / kMfmaGW * kMfmaGW;
        gbase0 = gq * gpp;
        Gx = min(args.G, gbase0 + gpp) - gbase0;
    }
    // the nb blocks of a grid row share the tiles evenly: block x takes
    // [x ntile / nb, (x + 1) ntile / nb), at most tpb tiles
    const int ntile = (N + 15) / 16, tpb = (ntile + nb - 1) / nb;
    // 32-bit tile arithmetic: either a block per tile (nb == ntile, the
    // several-stage path) or nb at most the launcher's block count of one
    // round (<= 2^10) with ntile <= 2^20 (N <= 2^24), so (bx + 1) * ntile < 2^30
    const bool one = nb == ntile;
    const int t0 = one ? bx : (int)((unsigned)(bx * ntile) / (unsigned)nb);
    const int nt = one ? 1 : (int)((unsigned)((bx + 1) * ntile) / (unsigned)nb) - t0;
    if (nt <= 0 || Gx <= 0) return;
    static_assert(!MOE || XS == X_F16, "routed experts take fp16 x");
    GemvArgs a = args;
    // routed experts: grid row y's expert and its token slots; x row of this
    // thread's batch row, output row of lane column c
    int xrow = -1, yrow = c;
    if constexpr (MOE) {
        const int32_t* pl = args.moe_plan + blockIdx.y * kMoePlanInts;
        const int e = pl[0];
        if (e < 0) return;
        a.batch = pl[1];
        a.W += (size_t)e * args.moe_wstride;
        a.S += (size_t)e * args.moe_sstride;
        xrow = pl[(args.moe_xslot ? 8 : 16) + min(tid % kMfmaCols, a.batch - 1)];
        yrow = pl[8 + min(c, kMoePlanMaxSlots - 1)];
    }
    const int nstage = EPI == E_PART ? 1 : (K + kMfmaKC - 1) / kMfmaKC;
    // the input: staged in LDS for one stage (and RMSNorm's 1/rms per batch
    // row); run by the streaming loop after its first weight requests
    auto stage_input = [&]() {
        if (XS == X_RMSNORM && XVEC && nstage == 1) {
            mfma_stage_x<XS, XVEC, true>(a, 0, (K + 31) / 32, xs, inv, red, xrow);
        } else if (XS == X_RMSNORM) {
            // sum of h^2 per batch row over all of K
            float ss[kMfmaCols];
#pragma unroll
            for (int b = 0; b < kMfmaCols; ++b) ss[b] = 0.0f;
            for (int k = tid; k < K; k += kMfmaThreads)
#pragma unroll
                for (int b = 0; b < kMfmaCols; ++b)
                    if (b < a.batch) {
                        const float v = a.h32[(size_t)b * a.ldx + k];
                        ss[b] = fmaf(v, v, ss[b]);
                    }
#pragma unroll
            for (int b = 0; b < kMfmaCols; ++b) {
                const float t = wave_sum(ss[b]);
                if (lane == 0) red[wave][b] = t;
            }
            __syncthreads();
            if (tid < kMfmaCols) {
                float t = 0.0f;
                for (int w = 0; w < kMfmaWaves; ++w) t += red[w][tid];
                inv[tid] = 1.0f / sqrtf(t / (float)K + a.eps);
            }
            __syncthreads();
        }
        if (nstage == 1 && !(XS == X_RMSNORM && XVEC))
            mfma_stage_x<XS, XVEC>(a, 0, (K + 31) / 32, xs, inv, nullptr, xrow);
        if (nstage == 1) __syncthreads();  // x staged
    };
    float best_v = -__builtin_inff();
    int best_i = -1;
    const int gs = wave * kMfmaGW;
    // tile t: every wavefront stores its partial sums in part[t & 1]; after
    // the barrier wavefront t % 8 adds them, lane (c, kq) taking batch row c
    // and weight rows 4kq..+3, and runs the epilogue
    auto finish = [&](int t, int row0, const mf4_t& acc) {
        if (kq < 2)  // lanes kq >= 2 hold batch rows 8..15, which repeat 0..7
            *reinterpret_cast<float4*>(&part[t & 1][(wave * 16 + c) * kMfmaCols + 4 * kq]) =
                make_float4(acc[0], acc[1], acc[2], acc[3]);
        __syncthreads();
        if (wave == (t & (kMfmaWaves - 1)) && c < a.batch) {
            float res[4] = {0.f, 0.f, 0.f, 0.f};
            for (int w = 0; w < kMfmaWaves; ++w)
#pragma unroll
                for (int i = 0; i < 4; ++i) res[i] += part[t & 1][(w * 16 + 4 * kq + i) * kMfmaCols + c];
            epilogue<EPI, 4>(a, yrow, row0 + 4 * kq, N, res, best_v, best_i);
        }
    };
    // fp16 x with K beyond one LDS stage: x straight from memory (XG)
    constexpr bool kXG = XS == X_F16 && XVEC && SALIGN && !FULL;
    // A tile is split over ks wavefronts along K (ks = 1 for large N).
    // Wavefront (tsub, kslice) = (wave / ks, wave % ks) takes tiles
    // t0 + tsub + (8 / ks) i and, of each, the groups of its K slice in
    // passes of 16; it streams these (tile, pass) items with the next item
    // requested before the current one is computed.  Only at a tile's end do
    // the wavefronts meet: partial sums go to LDS and, after the barrier,
    // wavefront kslice 0 of each tile adds them and runs the epilogue.  (A
    // barrier per pass made every wavefront wait for the others' prefetched
    // data, which a CU returns in request order.)  The item loop takes whole
    // pairs with no exit inside, so each request it carries across the back
    // edge is consumed in the next pass and the compiler's waits stay exact.
    // XG (several stages, ks = 8): K slices of ceil(G / 8) groups, x of the
    // item's groups loaded with its weights.
    auto stream = [&](auto xg_tag) {
        constexpr bool XG = decltype(xg_tag)::value;
        const int G = Gx, wpt = kMfmaWaves / ks, kslice = wave % ks, tsub = wave / ks;
        const int gps = XG ? (G + ks - 1) / ks : ((G + ks - 1) / ks + kMfmaGW - 1) / kMfmaGW * kMfmaGW;
        const int npass = (gps + kMfmaGW - 1) / kMfmaGW, send = min(G, (kslice + 1) * gps);
        const int iters = (tpb + wpt - 1) / wpt, nitem = iters * npass;
        const size_t xoff = XG ? (size_t)(xrow >= 0 ? xrow : min(c & (kMfmaCols - 1), a.batch - 1)) * a.ldx : 0;
        auto item_tile = [&](int j) { return t0 + tsub + wpt * (j / npass); };
        auto item_gs = [&](int j) { return kslice * gps + kMfmaGW * (j % npass); };
        auto load_item = [&](int j, MfmaRegs<XG>& r) {
            const int gs = item_gs(j), keep = j < nitem && item_tile(j) < t0 + nt ? 1 : 0;
            mfma_load<SALIGN, FULL, XG>(a, item_tile(j) * 16, gbase0, gs, min(send, gs + kMfmaGW), r, keep, xoff);
        };
        auto tile_end = [&](int j, const mf4_t& acc) {
            const int slot = (j / npass) & 1, t = item_tile(j);
            if (kq < 2)
                *reinterpret_cast<float4*>(&part[slot][(wave * 16 + c) * kMfmaCols + 4 * kq]) =
                    make_float4(acc[0], acc[1], acc[2], acc[3]);
            // ks = 1: the wavefront holds whole tiles and reads back only its
            // own slot (LDS operations of one wavefront complete in order)
            if (ks == 1) {
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            } else {
                __syncthreads();
            }
            if (kslice == 0 && c < a.batch && t < t0 + nt) {
                float res[4] = {0.f, 0.f, 0.f, 0.f};
                for (int s2 = 0; s2 < ks; ++s2)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        res[i] += part[slot][((tsub * ks + s2) * 16 + 4 * kq + i) * kMfmaCols + c];
                if constexpr (EPI == E_PART) {
                    // routed experts: the partial row of the lane's token slot
                    float* dst = a.kpart + ((size_t)gq * a.kpart_rows + (MOE ? yrow : c)) * N + t * 16 + 4 * kq;
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (t * 16 + 4 * kq + i < N) dst[i] = res[i];
                } else {
                    epilogue<EPI, 4>(a, yrow, t * 16 + 4 * kq, N, res, best_v, best_i);
                }
            }
        };
        mf4_t acc = {0.f, 0.f, 0.f, 0.f};
        MfmaRegs<XG> ra, rb;
        if constexpr (!XG && XVEC) {
            // the input's requests go first, the first two items' right
            // behind them (a CU returns data in request order, so x is not
            // held up), and only then is the input used
            StageRegs<XS> sr;
            stage_issue<XS>(a, 32 * gbase0, Gx, sr, xrow);
            load_item(0, ra);
            load_item(1, rb);
            __builtin_amdgcn_sched_barrier(0);
            stage_finish<XS, XS == X_RMSNORM>(a, 32 * gbase0, Gx, sr, xs, inv, red);
            __syncthreads();  // x staged
        } else {
            stage_input();
            load_item(0, ra);
            if constexpr (!XG) load_item(1, rb);
        }
        // one pass per tile (ks = 8 at K = 4096): the wavefront's x is the
        // same for every item, read from LDS once
        uint4 xh[kMfmaGW];
        const bool xhold = !XG && FULL && npass == 1;
        if (xhold) mfma_load_x<FULL>(xs, min(kslice * gps, G - 1), min(send, kslice * gps + kMfmaGW), xh);
        auto step = [&](int j, const MfmaRegs<XG>& r) {
            const int gs = item_gs(j), ge = min(send, gs + kMfmaGW);
            uint4 xv[kMfmaGW];
            if constexpr (XG) {
                mfma_perm_x(r.x, xv);
            } else if (xhold) {
#pragma unroll
                for (int u = 0; u < kMfmaGW; ++u) xv[u] = xh[u];
            } else {
                mfma_load_x<FULL>(xs, min(gs, G - 1), ge, xv);
            }
            mfma_compute<FULL, XG>(r, xv, gs, ge, acc);
            if (j % npass == npass - 1) {
                tile_end(j, acc);
                acc = mf4_t{0.f, 0.f, 0.f, 0.f};
            }
        };
        if constexpr (XG) {
            // two items in flight (an XG item holds its x too)
            int j = 0;
            for (; j + 1 < nitem; j += 2) {
                load_item(j + 1, rb);
                __builtin_amdgcn_sched_barrier(0);
                step(j, ra);
                load_item(j + 2, ra);
                __builtin_amdgcn_sched_barrier(0);
                step(j + 1, rb);
            }
            if (j < nitem) step(j, ra);
            return;
        }
        // three items in flight: item j + 2 is requested before item j is
        // used (loads past the last item read a valid line and are unused)
        MfmaRegs<XG> rc;
        int j = 0;
        for (; j + 2 < nitem; j += 3) {
            load_item(j + 2, rc);
            // the next items' requests stay ahead of this item's first use (the
            // scheduler would otherwise hoist the use, which then waits for all)
            __builtin_amdgcn_sched_barrier(0);
            step(j, ra);
            load_item(j + 3, ra);
            __builtin_amdgcn_sched_barrier(0);
            step(j + 1, rb);
            load_item(j + 4, rb);
            __builtin_amdgcn_sched_barrier(0);
            step(j + 2, rc);
        }
        if (j < nitem) step(j, ra);
        if (j + 1 < nitem) step(j + 1, rb);
    };
    if (nstage == 1) {
        stream(std::integral_constant<bool, false>{});
    } else if constexpr (kXG) {
        stream(std::integral_constant<bool, true>{});
    } else {
        stage_input();
        // K in several stages: x restaged per stage
        for (int t = 0; t < nt; ++t) {
            const int row0 = (t0 + t) * 16;
            mf4_t acc = {0.f, 0.f, 0.f, 0.f};
            for (int st = 0; st < nstage; ++st) {
                const int k0 = st * kMfmaKC, gc = (min(kMfmaKC, K - k0) + 31) / 32;
                const int ge = min(gc, gs + kMfmaGW);
                MfmaRegs<false> rg;
                mfma_load<SALIGN, false, false>(a, row0, k0 / 32, gs, ge, rg);
                __syncthreads();  // the previous stage's readers are done
                mfma_stage_x<XS, XVEC>(a, k0, gc, xs, inv, nullptr, xrow);
                __syncthreads();
                uint4 xv[kMfmaGW];
                mfma_load_x<false>(xs, gs, ge, xv);
                mfma_compute<false, false>(rg, xv, gs, ge, acc);
            }
            finish(t, row0, acc);
        }
    }
    if (EPI == E_LOGITS) {
        bk[tid] = (c < a.batch && best_i >= 0) ? pack_best(best_v, best_i) : 0ull;
        __syncthreads();
        if (tid < a.batch) {
            unsigned long long m = 0ull;
            for (int w = 0; w < kMfmaWaves; ++w)
                for (int q = 0; q < 4; ++q) {
                    const unsigned long long v = bk[w * kWave + q * 16 + tid];
                    m = v > m ? v : m;
                }
            if (m) atomicMax(&a.best[tid], m);
        }
    }
}

// Batch 1: a persistent grid of WPB wavefronts per CU in one block each
// (see b1_plan).
// MOE: ny grid rows of routed experts share the CUs.
template <int GPL, int R, int DEPTH, bool XLDS, int XS, int EPI, int WPB = kB1WavesPerCU, bool XFIRST = false,
          bool MOE = false>
hipError_t launch_b1(const GemvArgs& a, hipStream_t st, int ny = 1) {
    RowSplit rs;
    const int blocks = b1_plan(a.N, R, WPB, rs, WPB, ny);
    // the branch-free input loads need whole 8-element chunks on 16 bytes
    // (for routed experts, every row of x as well)
    const void* x = XS == X_F16 ? static_cast<const void*>(a.x16) : static_cast<const void*>(a.h32);
    const bool xvec = a.K % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (!MOE || a.ldx % 8 == 0);
    if (xvec)
        hipLaunchKernelGGL((k_gemv_b1<GPL, R, DEPTH, XLDS, XS, EPI, WPB, true, XFIRST, MOE>), dim3(blocks, ny),
                           dim3(WPB * kWave), 0, st, a, rs);
    else
        hipLaunchKernelGGL((k_gemv_b1<GPL, R, DEPTH, XLDS, XS, EPI, WPB, false, XFIRST, MOE>), dim3(blocks, ny),
                           dim3(WPB * kWave), 0, st, a, rs);
    return hipGetLastError();
}

// Sum of the K parts of a split GEMV in part order, then the epilogue
// (E_ACC: y32 += sum, E_F32: y32 = sum, E_F16: y16 = fp16(sum)).
template <int EPI>
__global__ __launch_bounds__(256) void k_gemv_ksum(const float* __restrict__ part, int kparts, int B, int N,
                                                   float* y32, uint16_t* y16, int ldy) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= B * N) return;
    const int b = i / N, n = i - b * N;
    float s = 0.0f;
    for (int q = 0; q < kparts; ++q) s += part[((size_t)q * B + b) * N + n];
    if (EPI == E_ACC) y32[(size_t)b * ldy + n] += s;
    else if (EPI == E_F32) y32[(size_t)b * ldy + n] = s;
    else y16[(size_t)b * ldy + n] = f2h_bits(s);
}

// The same sum, then (post_x16) the RMSNorm of each finished row: one block
// of kNormRowThreads per batch row, 16-byte chunks (N % 4 == 0, N <=
// 4 * kNormRowThreads * kNormRowChunks), every element summed exactly as
// k_gemv_ksum sums it.  KP parts, CH chunks per thread: every load of a
// thread (its parts, the residual, the norm weights) is requested before
// any is used, so the launch waits for one round trip (loads of chunks
// past the row re-read its last chunk and are not used).
constexpr int kNormRowThreads = 1024, kNormRowChunks = 4, kNormMaxParts = 8;
template <int EPI, int KP, int CH>
__global__ __launch_bounds__(kNormRowThreads) void k_gemv_ksum_norm(const float* __restrict__ part, int B, int N,
                                                                     float* y32, const float* w, uint16_t* x16,
                                                                     float eps) {
    __shared__ float red[kNormRowThreads / 64];
    const int b = blockIdx.x, t = threadIdx.x, nc = N / 4;
    // chunks whose loads are in flight together (all of them unless that
    // would not fit the registers of 1024 threads)
    constexpr int CL = CH * (KP + 2) <= 24 ? CH : 1;
    float4 v[CH], wv[CH];
    float ss = 0.0f;
#pragma unroll
    for (int j0 = 0; j0 < CH; j0 += CL) {
        float4 pv[CL][KP], yv[CL];
#pragma unroll
        for (int i = 0; i < CL; ++i) {
            const int c = min(t + (j0 + i) * kNormRowThreads, nc - 1);
#pragma unroll
            for (int q = 0; q < KP; ++q)
                pv[i][q] = reinterpret_cast<const float4*>(part + ((size_t)q * B + b) * N)[c];
            yv[i] = EPI == E_ACC ? reinterpret_cast<const float4*>(y32 + (size_t)b * N)[c]
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
            wv[j0 + i] = w ? reinterpret_cast<const float4*>(w)[c] : make_float4(1.f, 1.f, 1.f, 1.f);
        }
#pragma unroll
        for (int i = 0; i < CL; ++i) {
            const int c = t + (j0 + i) * kNormRowThreads;
            float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int q = 0; q < KP; ++q) {
                s.x += pv[i][q].x;
                s.y += pv[i][q].y;
                s.z += pv[i][q].z;
                s.w += pv[i][q].w;
            }
            if (EPI == E_ACC) {
                s.x = yv[i].x + s.x;
                s.y = yv[i].y + s.y;
                s.z = yv[i].z + s.z;
                s.w = yv[i].w + s.w;
            }
            v[j0 + i] = s;
            if (c < nc) {
                reinterpret_cast<float4*>(y32 + (size_t)b * N)[c] = s;
                ss += s.x * s.x + s.y * s.y + s.z * s.z + s.w * s.w;
            }
        }
    }
    ss = wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormRowThreads / 64; ++i) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / (float)N + eps);
    uint2* ob = reinterpret_cast<uint2*>(x16 + (size_t)b * N);
#pragma unroll
    for (int j = 0; j < CH; ++j) {
        const int c = t + j * kNormRowThreads;
        if (c >= nc) break;
        const uint32_t lo = (uint32_t)f2h_bits(v[j].x * inv * wv[j].x) | ((uint32_t)f2h_bits(v[j].y * inv * wv[j].y) << 16);
        const uint32_t hi = (uint32_t)f2h_bits(v[j].z * inv * wv[j].z) | ((uint32_t)f2h_bits(v[j].w * inv * wv[j].w) << 16);
        ob[c] = make_uint2(lo, hi);
    }
}

template <int EPI, int KP>
hipError_t ksum_norm_launch_kp(const GemvArgs& a, hipStream_t st) {
    if (a.N <= 4 * kNormRowThreads)
        hipLaunchKernelGGL((k_gemv_ksum_norm<EPI, KP, 1>), dim3(a.batch), dim3(kNormRowThreads), 0, st, a.kpart,
                           a.batch, a.N, a.y32, a.post_norm_w, a.post_x16, a.post_eps);
    else
        hipLaunchKernelGGL((k_gemv_ksum_norm<EPI, KP, kNormRowChunks>), dim3(a.batch), dim3(kNormRowThreads), 0, st,
                           a.kpart, a.batch, a.N, a.y32, a.post_norm_w, a.post_x16, a.post_eps);
    return hipGetLastError();
}

// The part sums + RMSNorm launch for kp parts (1 <= kp <= kNormMaxParts).
template <int EPI>
hipError_t ksum_norm_launch(const GemvArgs& a, int kp, hipStream_t st) {
    switch (kp) {
        case 1: return ksum_norm_launch_kp<EPI, 1>(a, st);
        case 2: return ksum_norm_launch_kp<EPI, 2>(a, st);
        case 3: return ksum_norm_launch_kp<EPI, 3>(a, st);
        case 4: return ksum_norm_launch_kp<EPI, 4>(a, st);
        case 5: return ksum_norm_launch_kp<EPI, 5>(a, st);
        case 6: return ksum_norm_launch_kp<EPI, 6>(a, st);
        case 7: return ksum_norm_launch_kp<EPI, 7>(a, st);
        case 8: return ksum_norm_launch_kp<EPI, 8>(a, st);
        default: return hipErrorInvalidValue;
    }
}

// RMSNorm of the rows a GEMV just wrote (post_x16), where its launch did not.
hipError_t post_norm_launch(const GemvArgs& a, hipStream_t st) {
    if (!a.post_x16) return hipSuccess;
    if (a.ldy != a.N || !a.y32) return hipErrorInvalidValue;
    return rmsnorm_launch(a.y32, a.post_norm_w, a.post_x16, a.N, a.post_eps, a.batch, st);
}

// Batch 2..8 on the matrix cores.  One stage (K <= 4096): ks wavefronts per
// tile, the fewest that still give every wavefront of one block per CU a
// tile, and enough tiles per block for one round of blocks.  Longer K with
// fp16 x (whole groups, aligned): the same streaming with ks = 8, x from
// memory.  Otherwise several LDS stages, one tile per block.
// MOE: ny grid rows of routed experts share the CUs.
template <int XS, int EPI, bool MOE = false>
hipError_t launch_mfma(const GemvArgs& a, hipStream_t st, int ny = 1) {
    // the kernel's 32-bit tile arithmetic: N <= 2^24, and a grid of one
    // round has at most 2^10 blocks per row (or one block per tile)
    const int ntile = (a.N + 15) / 16, cus = device_cus();
    if (a.N > (1 << 24) || cus > (1 << 10)) return hipErrorInvalidValue;
    const void* x = XS == X_F16 ? static_cast<const void*>(a.x16) : static_cast<const void*>(a.h32);
    const bool xvec = a.K % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0 &&
                      a.ldx % (XS == X_F16 ? 8 : 4) == 0;
    const bool salign = a.G % 8 == 0 && (reinterpret_cast<uintptr_t>(a.S) & 15u) == 0 &&
                        (!MOE || a.moe_sstride % 8 == 0);
    if constexpr (XS == X_F16 && (MOE ? EPI == E_F32 : (EPI == E_F16 || EPI == E_F32 || EPI == E_ACC))) {
        // K split over gemv_kparts(K) groups of blocks: each stages its part
        // of x once for its tiles (a block holding all of K would read all of
        // x for 16 rows); the part sums meet in a second launch (routed
        // experts: in the combine)
        const int kp = gemv_parts_for(a.K, a.batch, a.want_kparts);
        if (kp > 0 && a.kpart && xvec && salign) {
            GemvArgs p = a;
            p.kparts = kp;
            if (!MOE) p.kpart_rows = a.batch;
            const int rg = std::max(1, std::min(ntile, cus / (kp * ny)));
            const int per_block = (ntile + rg - 1) / rg;
            const int ksp = per_block <= 1 ? 8 : per_block <= 2 ? 4 : per_block <= 4 ? 2 : 1;
            hipLaunchKernelGGL((k_gemv_mfma<X_F16, E_PART, true, true, MOE, false>), dim3(rg * kp, ny),
                               dim3(kMfmaThreads), 0, st, p, rg, ksp);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess || MOE) return e;
            if constexpr (EPI == E_ACC || EPI == E_F32) {
                const bool vec = a.N % 4 == 0 && a.N <= 4 * kNormRowThreads * kNormRowChunks && a.ldy == a.N &&
                                 ((reinterpret_cast<uintptr_t>(a.y32) | reinterpret_cast<uintptr_t>(a.post_norm_w) |
                                   reinterpret_cast<uintptr_t>(a.post_x16)) & 15u) == 0;
                if (a.post_x16 && vec && kp <= kNormMaxParts) return ksum_norm_launch<EPI>(a, kp, st);
            }
            const int n = a.batch * a.N;
            hipLaunchKernelGGL((k_gemv_ksum<EPI>), dim3((n + 255) / 256), dim3(256), 0, st, a.kpart, kp, a.batch,
                               a.N, a.y32, a.y16, a.ldy);
            const hipError_t e2 = hipGetLastError();
            return e2 != hipSuccess ? e2 : post_norm_launch(a, st);
        }
    }
    const bool xg = XS == X_F16 && a.K > kMfmaKC && a.K % 32 == 0 && xvec && salign;
    int blocks = ntile, ks = 1;
    if (a.K <= kMfmaKC || xg) {
        // one round: the grid rows (experts) share the CUs, a block's tiles
        // are an even share of its row's
        blocks = std::max(1, std::min(ntile, (cus + ny - 1) / ny));
        const int per_block = (ntile + blocks - 1) / blocks;
        ks = xg || per_block <= 1 ? 8 : per_block <= 2 ? 4 : per_block <= 4 ? 2 : 1;
    }
    const bool full = a.K <= kMfmaKC && xvec && salign && a.G % (kMfmaGW * ks) == 0;
#define NX_MFMA(XV, SA, FL)                                                                                   \
    hipLaunchKernelGGL((k_gemv_mfma<XS, EPI, XV, SA, MOE, FL>), dim3(blocks, ny), dim3(kMfmaThreads), 0, st, a, \
                       blocks, ks)
    if (full) NX_MFMA(true, true, true);
    else if (xvec && salign) NX_MFMA(true, true, false);
    else if (xvec) NX_MFMA(true, false, false);
    else if (salign) NX_MFMA(false, true, false);
    else NX_MFMA(false, false, false);
#undef NX_MFMA
    const hipError_t e = hipGetLastError();
    return e != hipSuccess || MOE ? e : post_norm_launch(a, st);
}

// Tile shapes per groups-per-lane (K <= 64 * 32 * GPL), chosen by measuring
// the 8B decode shapes on cold weights; batch 1 runs one block of 8
// wavefronts per CU.  K = 4096: QKV and gate/up in 2-row tiles (a pair, as
// the RoPE and SwiGLU epilogues need), in a ring of 1 (QKV: 1.5 tiles per
// wavefront) and of 2; lm_head in a ring of 3; 2-row tiles in a ring of 1
// otherwise (wo: one tile per wavefront).
// K = 14336 without paired rows: one row per tile with x in registers.
// Paired epilogues at GPL >= 4 keep x in LDS (at GPL 7 one pair in flight
// per wavefront: two spilled).  (Measured at batch 1 against these: QKV in
// 4-row tiles, a ring of 2 or of 3; wo as single rows in a ring of 3 or 1;
// gate/up in a ring of 1 or 3, in 4-row tiles, or with 12 or 16 wavefronts
// per CU; down in a ring of 2 (x in registers or in LDS) or as 2-row tiles:
// all slower; lm_head in a ring of 1 or 2, or in 4-row tiles: the same.)
template <int XS, int EPI>
hipError_t launch_b1_gpl(const GemvArgs& a, hipStream_t st) {
    const int gpl = (a.G + kWave - 1) / kWave;
    constexpr bool kPairs = EPI == E_QKV || EPI == E_SWIGLU;
    if (gpl <= 1) return launch_b1<1, 4, 2, false, XS, EPI>(a, st);
    if (gpl <= 2) {
        if constexpr (EPI == E_QKV) return launch_b1<2, 2, 1, false, XS, EPI>(a, st);
        if constexpr (EPI == E_SWIGLU) return launch_b1<2, 2, 2, false, XS, EPI>(a, st);
        if constexpr (EPI == E_LOGITS) return launch_b1<2, 2, 3, false, XS, EPI>(a, st);
        return launch_b1<2, 2, 1, false, XS, EPI>(a, st);
    }
    if (gpl <= 4) return launch_b1<4, 2, 2, true, XS, EPI>(a, st);
    if (gpl > 7) {
        // K up to 28672 (a 70B-class down projection): single rows in a ring
        // of 2 with x in LDS (57 KB); fp16 inputs with a plain, fp32 or
        // residual epilogue only
        if constexpr (XS == X_F16 && (EPI == E_F16 || EPI == E_F32 || EPI == E_ACC))
            if (gpl <= 14) return launch_b1<14, 1, 2, true, XS, EPI>(a, st);
        return hipErrorInvalidValue;
    }
    if constexpr (kPairs) return launch_b1<7, 2, 1, true, XS, EPI>(a, st);
    return launch_b1<7, 1, 1, false, XS, EPI>(a, st);
}

// Batch 1 on the row kernels, batch 2..8 on the matrix cores; then the
// post-GEMV RMSNorm where the launch asks for one.
template <int XS, int EPI>
hipError_t launch_gpl(const GemvArgs& a, hipStream_t st) {
    const int gpl = (a.G + kWave - 1) / kWave;
    if (a.batch == 1) {
        const hipError_t e = launch_b1_gpl<XS, EPI>(a, st);
        return e != hipSuccess ? e : post_norm_launch(a, st);
    }
    if (gpl > 14) return hipErrorInvalidValue;
    return launch_mfma<XS, EPI>(a, st);
}

}  // namespace


hipError_t gemv_launch(int xsrc, int epi, const GemvArgs& a, hipStream_t st) {
    if (a.batch < 1 || a.batch > 8) return hipErrorInvalidValue;
    if (xsrc == X_F16) {
        switch (epi) {
            case E_F16: return launch_gpl<X_F16, E_F16>(a, st);
            case E_F32: return launch_gpl<X_F16, E_F32>(a, st);
            case E_ACC: return launch_gpl<X_F16, E_ACC>(a, st);
            case E_SWIGLU: return launch_gpl<X_F16, E_SWIGLU>(a, st);
            case E_QKV: return launch_gpl<X_F16, E_QKV>(a, st);
            case E_LOGITS: return launch_gpl<X_F16, E_LOGITS>(a, st);
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

namespace {

// Routed expert GEMVs on the dense kernels: grid row y takes the y-th
// active expert of the routing plan (rows without one exit at once), the
// expert's weights and its gathered token rows.  Batch 1 (one slot per
// expert) runs the batch-1 kernel, with the CUs shared by the possible
// active experts; larger batches run the matrix-core kernel over each
// expert's slots.
//   gate/up: rows (2f, 2f+1) = (gate f, up f) of w13[e]; x = the token's
//            x16 row; act16[slot][f] = fp16(silu(g) * u).
//   down:    rows of w2[e]; x = act16[slot]; y32[slot][n] = y.
template <bool GATEUP>
hipError_t moe_launch(const MoeFfnArgs& m, hipStream_t st) {
    if (!m.plan || m.batch < 1 || m.batch > kMoePlanMaxSlots) return hipErrorInvalidValue;
    const int N = GATEUP ? 2 * m.F : m.d, K = GATEUP ? m.d : m.F;
    const int G = (K + 31) / 32, Fp = (m.F + 31) / 32 * 32;
    GemvArgs a{};
    a.W = GATEUP ? m.w13 : m.w2;
    a.S = GATEUP ? m.s13 : m.s2;
    a.N = N;
    a.K = K;
    a.G = G;
    a.batch = m.batch;
    a.x16 = GATEUP ? m.x16 : m.act16;
    a.ldx = GATEUP ? m.ldx : Fp;
    a.act16 = m.act16;
    a.lda = Fp;
    a.y32 = m.y32;
    a.ldy = m.d;
    a.moe_plan = m.plan;
    a.moe_wstride = (size_t)N * G * 16;
    a.moe_sstride = (size_t)N * G;
    a.moe_xslot = GATEUP ? 0 : 1;
    if (!GATEUP && moe_down_split(m)) {
        a.kpart = m.kpart;
        a.kpart_rows = m.batch * m.k;
    }
    const int ny = moe_plan_rows(m.E, m.batch, m.k);
    constexpr int EPI = GATEUP ? E_SWIGLU : E_F32;
    const int gpl = (G + kWave - 1) / kWave;
    if (gpl > 7) return hipErrorInvalidValue;
    if (m.batch > 1) return launch_mfma<X_F16, EPI, true>(a, st, ny);
    constexpr int W = kB1WavesPerCU;
    if (gpl <= 1) return launch_b1<1, 4, 2, false, X_F16, EPI, W, false, true>(a, st, ny);
    if (gpl <= 2) {
        if constexpr (GATEUP) return launch_b1<2, 2, 2, false, X_F16, EPI, W, false, true>(a, st, ny);
        return launch_b1<2, 1, 3, false, X_F16, EPI, W, false, true>(a, st, ny);
    }
    if (gpl <= 4) return launch_b1<4, 2, 2, true, X_F16, EPI, W, false, true>(a, st, ny);
    if constexpr (GATEUP) return launch_b1<7, 2, 2, true, X_F16, EPI, W, false, true>(a, st, ny);
    return launch_b1<7, 1, 1, false, X_F16, EPI, W, false, true>(a, st, ny);
}

}  // namespace

// The conditions of launch_mfma's K split for the routed down projection
// (x = act16 rows of Fp elements, G = F / 32 groups).
bool moe_down_split(const MoeFfnArgs& m) {
    const int Fp = (m.F + 31) / 32 * 32, G = (m.F + 31) / 32;
    return m.kpart && gemv_kparts(m.F, m.batch) > 0 && m.F % 8 == 0 && Fp % 8 == 0 && G % 4 == 0 &&
           (reinterpret_cast<uintptr_t>(m.act16) & 15u) == 0;
}

hipError_t moe_gate_up_launch(const MoeFfnArgs& a, hipStream_t st) { return moe_launch<true>(a, st); }
hipError_t moe_down_launch(const MoeFfnArgs& a, hipStream_t st) { return moe_launch<false>(a, st); }

}  // namespace nx
