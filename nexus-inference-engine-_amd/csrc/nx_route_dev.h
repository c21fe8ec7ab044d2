// Routing of one sequence by one wavefront (decode): the softmax, top-k and
// renormalization of the router logits, spread over the lanes.
#pragma once

#include "nx_common.h"
#include "nx_kernels.h"

namespace nx {

constexpr int kRoutePerLane = kMoeMaxExperts / kWave;

// Routing of one sequence from its logits lg[E], run by one whole wavefront
// with the arithmetic of the sequential routing (route_row in nx_misc.hip,
// hybrid_model.cpp:1656-1694), so both give the same ids and weights: the
// max, the sum of expf(l - max) in expert order, p_e = expf(l_e - max) / sum,
// the k largest p with ties to the lower id, the weights renormalized over the
// chosen k in slot order.  Lane l holds experts l, l + 64, ...; ids / w (slot
// order, LDS) are written by lane 0.
__device__ inline void route_wave(const float* lg, int E, int k, int* ids, float* w) {
    const int lane = threadIdx.x & (kWave - 1);
    float l[kRoutePerLane];
    float mx = -__builtin_inff();
#pragma unroll
    for (int p = 0; p < kRoutePerLane; ++p) {
        const int e = lane + kWave * p;
        l[p] = e < E ? lg[e] : -__builtin_inff();
        mx = fmaxf(mx, l[p]);
    }
    mx = wave_max(mx);
    float x[kRoutePerLane];
#pragma unroll
    for (int p = 0; p < kRoutePerLane; ++p) x[p] = lane + kWave * p < E ? expf(l[p] - mx) : 0.0f;
    // the sum in expert order, as the sequential routing adds it
    float sum = 0.0f;
#pragma unroll
    for (int p = 0; p < kRoutePerLane; ++p)
        for (int q = 0; q < kWave && kWave * p + q < E; ++q) sum += readlane_f(x[p], q);
    // keys: (probability bits, ~expert); probabilities are >= 0, so their
    // bits order as their values, and the larger key is the larger p with the
    // lower id
    unsigned long long key[kRoutePerLane];
#pragma unroll
    for (int p = 0; p < kRoutePerLane; ++p) {
        const int e = lane + kWave * p;
        const float pe = sum > 0.0f ? x[p] / sum : x[p];
        key[p] = e < E ? ((unsigned long long)__builtin_bit_cast(uint32_t, pe) << 32) |
                             (unsigned long long)(0xFFFFFFFFu - (uint32_t)e)
                       : 0ull;
    }
    float active = 0.0f;
    for (int j = 0; j < k; ++j) {
        unsigned long long b = key[0];
#pragma unroll
        for (int p = 1; p < kRoutePerLane; ++p) b = key[p] > b ? key[p] : b;
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
            const uint32_t hi = __shfl_xor((uint32_t)(b >> 32), o, kWave);
            const uint32_t lo = __shfl_xor((uint32_t)b, o, kWave);
            const unsigned long long c = ((unsigned long long)hi << 32) | lo;
            b = c > b ? c : b;
        }
        const int e = (int)(0xFFFFFFFFu - (uint32_t)b);
        const float bp = __builtin_bit_cast(float, (uint32_t)(b >> 32));
#pragma unroll
        for (int p = 0; p < kRoutePerLane; ++p)
            if (key[p] == b) key[p] = 0ull;  // taken
        if (lane == 0) {
            ids[j] = e;
            w[j] = bp;
        }
        active += bp;
    }
    if (lane == 0)
        for (int j = 0; j < k; ++j) w[j] = active > 0.0f ? w[j] / active : 1.0f / (float)k;
}

}  // namespace nx
