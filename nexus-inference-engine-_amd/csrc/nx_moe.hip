// Routed experts of one sequence (batch 1) in two launches instead of four.
//
// The MoE block of a decode step is RMSNorm -> router -> top-k -> each chosen
// expert's gate/up + SwiGLU -> down -> h += sum_j w_j y_j
// (hybrid_model.cpp:1647-1711).  The separate launches for the routing
// (a few KB of router weights on one CU) and for the weighted combine (a
// few KB of sums) cost a launch boundary and a dependent chain each while
// the CUs idle.  Here:
//
//   k_moe_b1_gate_up     every block normalizes h into LDS and computes the
//                        router logits and the routing itself (the router
//                        rows, 16 KB at 8 experts, are requested with h), then
//                        streams the gate/up rows of its grid row's expert.
//                        Every block computes the same routing with the same
//                        instructions on the same inputs, so all agree; block
//                        (0, 0) publishes it (ids, weights, counts, slot lists
//                        and the plan) for the down projection.
//   k_moe_b1_down_combine a block owns output rows n of every chosen expert
//                        (one group of its wavefronts per slot, each with its
//                        slot's activation in registers); the sums meet in
//                        LDS and the block adds sum_j w_j y_j[n] to h[n] in
//                        slot order -- the combine's arithmetic, with no
//                        second pass.  Top-k up to 2; larger k keeps the
//                        separate down projection and combine.
#include "nx_gemv_dev.h"
#include "nx_route_dev.h"

namespace nx {

namespace {

using namespace gv;

constexpr int kMoeWpb = kB1WavesPerCU;  // one block of 8 wavefronts per CU
constexpr int kMoeThreads = kMoeWpb * kWave;

// The routing outputs of the separate routing launch (k_moe_norm_route /
// build_lists at batch 1): ids, weights, per-expert counts and slot lists,
// and the plan (chosen experts in ascending order, one slot each).
__device__ inline void publish_route(const MoeArgs& m, const int* ids, const float* w) {
    const int t = threadIdx.x, E = m.E, k = m.k;
    for (int e = t; e < E; e += kMoeThreads) {
        int slot = -1;
        for (int j = 0; j < k; ++j) slot = ids[j] == e ? j : slot;
        m.expert_count[e] = slot >= 0 ? 1 : 0;
        if (slot >= 0) m.expert_slots[(size_t)e * k] = slot;
    }
    if (t < k) {
        m.ids[t] = ids[t];
        m.weights[t] = w[t];
        int rank = 0;
        for (int j = 0; j < k; ++j) rank += ids[j] < ids[t] ? 1 : 0;
        int32_t* pl = m.plan + (size_t)rank * kMoePlanInts;
        pl[0] = ids[t];
        pl[1] = 1;
        pl[8] = t;
        pl[16] = 0;
    }
}

// Gate/up of the routed experts with the routing in the prologue.  a: W/S =
// w13/s13 of expert 0 (experts moe_wstride / moe_sstride apart), N = 2F,
// K = d, h32 = h, norm_w, eps, act16 / lda; m: router rows, E, k and the
// routing outputs.  Grid row y takes the y-th smallest chosen expert.
// XLDS: x is read from LDS per group (long rows) instead of registers.
template <int GPL, int R, int DEPTH, bool XLDS, bool XVEC>
__global__ __launch_bounds__(kMoeThreads, 1) void k_moe_b1_gate_up(GemvArgs a, RowSplit rs, MoeArgs m) {
    constexpr int WPB = kMoeWpb, NT = kMoeThreads, CPT = (4 * GPL + WPB - 1) / WPB;
    __shared__ __align__(16) uint32_t sp[kWave * GPL * 16];
    __shared__ float s8[kWave * GPL];
    __shared__ float red[WPB];
    __shared__ float lg[kMoeMaxExperts];
    __shared__ int sel[kMoeMaxTopK];
    __shared__ float sw[kMoeMaxTopK];
    asm volatile("" ::"s"(a.h32), "s"(a.norm_w), "s"(m.wr), "s"(m.sr), "s"(m.E), "s"(a.G), "s"(a.K));
    const int lane = threadIdx.x & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int E = m.E, G = a.G;
    // the grid row's tiles dealt to its wavefronts in turn (as the dense
    // batch-1 GEMV deals them)
    const int NW = rs.nb * rs.wpb, T = (a.N + R - 1) / R, wid = wave * rs.nb + blockIdx.x;
    const int nt = wid < T ? (T - wid + NW - 1) / NW : 0;
    auto trow = [&](int k) { return (wid + min(k, max(nt - 1, 0)) * NW) * R; };
    // h with its norm weights, and this wavefront's first router row
    StageRegs<CPT, X_RMSNORM> sr;
    stage_issue<CPT, X_RMSNORM, NT, XVEC>(a, 0, sr);
    Tile<GPL, 1> rt;
    {
        const int e0 = min(wave, E - 1);
        load_tile_u<GPL, 1>(rt, m.wr, m.sr, G, e0, e0 + 1, e0, lane);
    }
    if constexpr (XLDS) zero_pairs_lds<GPL, NT>(sp, s8, G);
    stage_finish<CPT, X_RMSNORM, NT>(a, sr, sp, s8, red);  // block barrier
    XPairs<XLDS ? 1 : GPL> xp;
    if constexpr (!XLDS) load_pairs_lds<GPL>(xp, sp, s8, G, lane);
    // router logits: wavefront w takes rows w, w + WPB, ... (fixed order
    // within each, so every block computes the same values)
    for (int e = wave; e < E; e += WPB) {
        if (e != wave) load_tile_u<GPL, 1>(rt, m.wr, m.sr, G, e, e + 1, e, lane);
        float res[1];
        if constexpr (XLDS)
            tile_dot_lds<GPL, 1>(rt, sp, s8, G, lane, res);
        else
            tile_dot<GPL, 1>(rt, xp, res);
        if (lane == 0) lg[e] = res[0];
    }
    __syncthreads();
    if (wave == 0) route_wave(lg, E, m.k, sel, sw);
    __syncthreads();
    if (blockIdx.x == 0 && blockIdx.y == 0) publish_route(m, sel, sw);
    // this grid row's expert: the blockIdx.y-th smallest chosen id, and its slot
    int slot = 0;
    for (int j = 0; j < m.k; ++j) {
        int rank = 0;
        for (int i = 0; i < m.k; ++i) rank += sel[i] < sel[j] ? 1 : 0;
        slot = rank == (int)blockIdx.y ? j : slot;
    }
    const int e = sel[slot];
    GemvArgs g = a;
    g.W += (size_t)e * a.moe_wstride;
    g.S += (size_t)e * a.moe_sstride;
    g.act16 += (size_t)slot * a.lda;
    Tile<GPL, R> t[DEPTH];
#pragma unroll
    for (int j = 0; j < DEPTH; ++j) load_tile_u<GPL, R>(t[j], g.W, g.S, G, 0, a.N, trow(j), lane);
    float best_v = 0.0f;
    int best_i = 0;
    float res[R];
    for (int i = 0; i < nt; i += DEPTH) {
#pragma unroll
        for (int j = 0; j < DEPTH; ++j) {
            if (i + j >= nt) break;
            if constexpr (XLDS)
                tile_dot_lds<GPL, R>(t[j], sp, s8, G, lane, res);
            else
                tile_dot<GPL, R>(t[j], xp, res);
            load_tile_u<GPL, R>(t[j], g.W, g.S, G, 0, a.N, trow(i + j + DEPTH), lane);
            if (lane == 0) epilogue<E_SWIGLU, R>(g, 0, trow(i + j), a.N, res, best_v, best_i);
        }
    }
}

// Down projection of the KS chosen experts and the weighted combine.  A
// block owns output rows [n0, n1) (at most kDcRows): its wavefronts are KS
// groups, group j streaming those rows of slot j's expert with slot j's
// activation held in registers (as the separate routed down projection
// does), the sums meet in LDS, and the block adds h[n] += sum_j w_j y_j[n]
// (j in slot order, the sum started at zero, as the separate combine adds).
// a: W/S = w2/s2 of expert 0, N = d, K = F, x16 = act16 (slot rows lda
// apart), y32 = h; ids / wts: the routing of the gate/up launch.
constexpr int kDcRows = 64;
template <int GPL, int KS, int DEPTH, bool XLDS, bool XVEC>
__global__ __launch_bounds__(kMoeThreads, 1) void k_moe_b1_down_combine(GemvArgs a, int rows_per_block,
                                                                         const int32_t* ids, const float* wts) {
    constexpr int WPB = kMoeWpb, NT = kMoeThreads, CPT = (4 * GPL + WPB - 1) / WPB, WG = WPB / KS;
    static_assert(WPB % KS == 0, "whole wavefront groups per slot");
    __shared__ __align__(16) uint32_t sp[KS * kWave * GPL * 16];
    __shared__ float s8[KS * kWave * GPL];
    __shared__ float ys[KS * kDcRows];
    asm volatile("" ::"s"(a.x16), "s"(a.W), "s"(a.S), "s"(ids), "s"(wts), "s"(a.G), "s"(a.K), "s"(a.N));
    const int lane = threadIdx.x & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slot = wave / WG, wj = wave % WG;
    const int n0 = blockIdx.x * rows_per_block, n1 = min(n0 + rows_per_block, a.N);
    // this wavefront's rows: a contiguous share of the block's
    const int per = (n1 - n0 + WG - 1) / WG;
    const int r0 = min(n0 + wj * per, n1), r1 = min(r0 + per, n1);
    // the slot's expert, then the slots' activations and the first rows
    const int e = __builtin_amdgcn_readfirstlane(ids[slot]);
    StageRegs<CPT, X_F16> sr[KS];
#pragma unroll
    for (int j = 0; j < KS; ++j) {
        GemvArgs aj = a;
        aj.x16 = a.x16 + (size_t)j * a.lda;
        stage_issue<CPT, X_F16, NT, XVEC>(aj, 0, sr[j]);
    }
    const uint8_t* W = a.W + (size_t)e * a.moe_wstride;
    const uint16_t* S = a.S + (size_t)e * a.moe_sstride;
    Tile<GPL, 1> t[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) load_tile_u<GPL, 1>(t[d], W, S, a.G, r0, r1, r0 + d, lane);
    uint32_t* spj = sp + slot * kWave * GPL * 16;
    float* s8j = s8 + slot * kWave * GPL;
    if constexpr (XLDS)
#pragma unroll
        for (int j = 0; j < KS; ++j) zero_pairs_lds<GPL, NT>(sp + j * kWave * GPL * 16, s8 + j * kWave * GPL, a.G);
#pragma unroll
    for (int j = 0; j < KS; ++j) {
        GemvArgs aj = a;
        aj.x16 = a.x16 + (size_t)j * a.lda;
        stage_finish<CPT, X_F16, NT>(aj, sr[j], sp + j * kWave * GPL * 16, s8 + j * kWave * GPL, nullptr);
    }
    XPairs<XLDS ? 1 : GPL> xp;
    if constexpr (!XLDS) load_pairs_lds<GPL>(xp, spj, s8j, a.G, lane);
    const int nt = r1 - r0;
    float res[1];
    for (int i = 0; i < nt; i += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            if (i + d >= nt) break;
            if constexpr (XLDS)
                tile_dot_lds<GPL, 1>(t[d], spj, s8j, a.G, lane, res);
            else
                tile_dot<GPL, 1>(t[d], xp, res);
            load_tile_u<GPL, 1>(t[d], W, S, a.G, r0, r1, r0 + i + d + DEPTH, lane);
            if (lane == 0) ys[slot * kDcRows + (r0 - n0) + i + d] = res[0];
        }
    }
    __syncthreads();
    const int t0 = threadIdx.x;
    if (t0 < n1 - n0) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < KS; ++j) acc += wts[j] * ys[j * kDcRows + t0];
        __hip_atomic_fetch_add(a.y32 + n0 + t0, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

inline int gpl_of(int G) { return (G + kWave - 1) / kWave; }

template <int GPL, int R, int DEPTH, bool XLDS>
hipError_t launch_gate_up(const GemvArgs& a, const MoeArgs& m, hipStream_t st) {
    RowSplit rs;
    const int blocks = b1_plan(a.N, R, kMoeWpb, rs, kMoeWpb, m.k);
    const bool xvec = a.K % 8 == 0 && (reinterpret_cast<uintptr_t>(a.h32) & 15u) == 0 &&
                      (!a.norm_w || (reinterpret_cast<uintptr_t>(a.norm_w) & 15u) == 0);
    if (xvec)
        hipLaunchKernelGGL((k_moe_b1_gate_up<GPL, R, DEPTH, XLDS, true>), dim3(blocks, m.k), dim3(kMoeThreads), 0, st, a,
                           rs, m);
    else
        hipLaunchKernelGGL((k_moe_b1_gate_up<GPL, R, DEPTH, XLDS, false>), dim3(blocks, m.k), dim3(kMoeThreads), 0, st, a,
                           rs, m);
    return hipGetLastError();
}

template <int GPL, int KS, int DEPTH, bool XLDS>
hipError_t launch_down(const GemvArgs& a, const MoeFfnArgs& f, const int32_t* ids, hipStream_t st) {
    // one block per CU, at most kDcRows rows each
    int blocks = device_cus();
    if (blocks * kDcRows < a.N) blocks = (a.N + kDcRows - 1) / kDcRows;
    const int rpb = (a.N + blocks - 1) / blocks;
    blocks = (a.N + rpb - 1) / rpb;
    const bool xvec = a.K % 8 == 0 && a.lda % 8 == 0 && (reinterpret_cast<uintptr_t>(a.x16) & 15u) == 0;
    if (xvec)
        hipLaunchKernelGGL((k_moe_b1_down_combine<GPL, KS, DEPTH, XLDS, true>), dim3(blocks), dim3(kMoeThreads), 0,
                           st, a, rpb, ids, f.weights);
    else
        hipLaunchKernelGGL((k_moe_b1_down_combine<GPL, KS, DEPTH, XLDS, false>), dim3(blocks), dim3(kMoeThreads), 0,
                           st, a, rpb, ids, f.weights);
    return hipGetLastError();
}

}  // namespace

bool moe_b1_fused_fits(int d, int F, int E, int k) {
    const int gd = gpl_of((d + 31) / 32), gf = gpl_of((F + 31) / 32);
    return d % 2 == 0 && (gd == 1 || gd == 2 || gd == 4 || gd == 7) &&
           (gf == 1 || gf == 2 || gf == 4 || gf == 7) && E >= 1 && E <= kMoeMaxExperts && k >= 1 &&
           k <= kMoeMaxTopK && k <= E;
}

bool moe_b1_down_combine_fits(int F, int k) {
    const int gf = gpl_of((F + 31) / 32);
    return (k == 1 || k == 2) && (gf == 1 || gf == 2 || gf == 4 || gf == 7);
}

hipError_t moe_b1_gate_up_launch(const MoeArgs& m, const MoeFfnArgs& f, hipStream_t st) {
    if (f.batch != 1 || m.batch != 1 || !m.plan || !moe_b1_fused_fits(f.d, f.F, f.E, f.k) || m.k != f.k ||
        m.E != f.E || m.d != f.d)
        return hipErrorInvalidValue;
    GemvArgs a{};
    a.W = f.w13;
    a.S = f.s13;
    a.N = 2 * f.F;
    a.K = f.d;
    a.G = (f.d + 31) / 32;
    a.batch = 1;
    a.h32 = m.h;
    a.ldx = f.d;
    a.norm_w = m.norm_w;
    a.eps = m.eps;
    a.act16 = f.act16;
    a.lda = (f.F + 31) / 32 * 32;
    a.moe_wstride = (size_t)a.N * a.G * 16;
    a.moe_sstride = (size_t)a.N * a.G;
    switch (gpl_of(a.G)) {
        case 1: return launch_gate_up<1, 2, 2, false>(a, m, st);
        case 2: return launch_gate_up<2, 2, 2, false>(a, m, st);
        case 4: return launch_gate_up<4, 2, 2, true>(a, m, st);
        case 7: return launch_gate_up<7, 2, 1, true>(a, m, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t moe_b1_down_combine_launch(const MoeFfnArgs& f, const int32_t* ids, hipStream_t st) {
    if (f.batch != 1 || !ids || !f.weights || !moe_b1_down_combine_fits(f.F, f.k)) return hipErrorInvalidValue;
    GemvArgs a{};
    a.W = f.w2;
    a.S = f.s2;
    a.N = f.d;
    a.K = f.F;
    a.G = (f.F + 31) / 32;
    a.batch = 1;
    a.x16 = f.act16;
    a.lda = (f.F + 31) / 32 * 32;
    a.ldx = a.lda;
    a.y32 = f.out;
    a.moe_wstride = (size_t)a.N * a.G * 16;
    a.moe_sstride = (size_t)a.N * a.G;
    const int gf = gpl_of(a.G);
    if (f.k == 1) {
        switch (gf) {
            case 1: return launch_down<1, 1, 2, false>(a, f, ids, st);
            case 2: return launch_down<2, 1, 2, false>(a, f, ids, st);
            case 4: return launch_down<4, 1, 2, false>(a, f, ids, st);
            case 7: return launch_down<7, 1, 1, false>(a, f, ids, st);
            default: return hipErrorInvalidValue;
        }
    }
    switch (gf) {
        case 1: return launch_down<1, 2, 2, false>(a, f, ids, st);
        case 2: return launch_down<2, 2, 2, false>(a, f, ids, st);
        case 4: return launch_down<4, 2, 2, false>(a, f, ids, st);
        case 7: return launch_down<7, 2, 1, false>(a, f, ids, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace nx
