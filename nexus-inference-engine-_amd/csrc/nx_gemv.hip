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
// persistent (one block of 8 wavefronts per CU), each wavefront streams a
// contiguous row range with the next tile requested before the current one
// is reduced, and the first tiles are requested right after the input.  The
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
#include "nx_gemv_dev.h"

namespace nx {

namespace {

using namespace gv;

// Batch 1 kernel: the whole grid runs one GEMV, one block of WPB
// wavefronts per CU.
template <int GPL, int R, int DEPTH, bool XLDS, int XS, int EPI, int WPB, bool XVEC>
__global__ __launch_bounds__(WPB * kWave, 1) void k_gemv_b1(GemvArgs a, RowSplit rs) {
    gemv_b1_run<GPL, R, DEPTH, XLDS, XS, EPI, WPB, XVEC>(a, rs, blockIdx.x);
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
            if (lane == 0) epilogue<EPI, R>(a, b, n0, a.N, res, best_v[b], best_i[b]);
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

// Batch 1: a persistent grid of WPB wavefronts per CU in one block each
// (see b1_plan).
template <int GPL, int R, int DEPTH, bool XLDS, int XS, int EPI, int WPB = kB1WavesPerCU>
hipError_t launch_b1(const GemvArgs& a, hipStream_t st) {
    RowSplit rs;
    const int blocks = b1_plan(a.N, R, WPB, rs, WPB);
    // the branch-free input loads need whole 8-element chunks on 16 bytes
    const void* x = XS == X_F16 ? static_cast<const void*>(a.x16) : static_cast<const void*>(a.h32);
    const bool xvec = a.K % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    if (xvec)
        hipLaunchKernelGGL((k_gemv_b1<GPL, R, DEPTH, XLDS, XS, EPI, WPB, true>), dim3(blocks), dim3(WPB * kWave),
                           0, st, a, rs);
    else
        hipLaunchKernelGGL((k_gemv_b1<GPL, R, DEPTH, XLDS, XS, EPI, WPB, false>), dim3(blocks),
                           dim3(WPB * kWave), 0, st, a, rs);
    return hipGetLastError();
}

// Batch 2..8.
template <int GPL, int R, int XS, int EPI>
hipError_t launch_bn(const GemvArgs& a, hipStream_t st) {
    const int tiles = (a.N + R - 1) / R;
    int blocks = (tiles + kWavesPerBlock - 1) / kWavesPerBlock;
    if (blocks > 1024) blocks = 1024;
    hipLaunchKernelGGL((k_gemv_bn<GPL, R, XS, EPI>), dim3(blocks), dim3(kBlockThreads), 0, st, a);
    return hipGetLastError();
}

// Tile shapes per groups-per-lane (K <= 64 * 32 * GPL), chosen by measuring
// the 8B decode shapes on cold weights; batch 1 runs one block of 8
// wavefronts per CU.  K = 4096: QKV in 4-row tiles, gate/up and lm_head in
// 2-row tiles (a pair, as the SwiGLU epilogue needs) in a ring of 2, single
// rows in a ring of 3 otherwise.  K = 14336 without paired rows: one row per
// tile with x in registers.  Paired epilogues at GPL >= 4 keep x in LDS.
template <int XS, int EPI>
hipError_t launch_gpl(const GemvArgs& a, hipStream_t st) {
    const int gpl = (a.G + kWave - 1) / kWave;
    constexpr bool kPairs = EPI == E_QKV || EPI == E_SWIGLU;
    if (a.batch == 1) {
        if (gpl <= 1) return launch_b1<1, 4, 2, false, XS, EPI>(a, st);
        if (gpl <= 2) {
            if constexpr (EPI == E_QKV) return launch_b1<2, 4, 1, false, XS, EPI>(a, st);
            if constexpr (EPI == E_SWIGLU || EPI == E_LOGITS) return launch_b1<2, 2, 2, false, XS, EPI>(a, st);
            return launch_b1<2, 1, 3, false, XS, EPI>(a, st);
        }
        if (gpl <= 4) return launch_b1<4, 2, 2, true, XS, EPI>(a, st);
        if (gpl > 7) return hipErrorInvalidValue;
        if constexpr (kPairs) return launch_b1<7, 2, 2, true, XS, EPI>(a, st);
        return launch_b1<7, 1, 1, false, XS, EPI>(a, st);
    }
    if (gpl <= 1) return launch_bn<1, 4, XS, EPI>(a, st);
    if (gpl <= 2) return launch_bn<2, 4, XS, EPI>(a, st);
    if (gpl <= 4) return launch_bn<4, 2, XS, EPI>(a, st);
    if (gpl <= 7) return launch_bn<7, 2, XS, EPI>(a, st);
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
