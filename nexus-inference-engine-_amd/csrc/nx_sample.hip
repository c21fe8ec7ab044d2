// Token sampling on the device: HybridModel::Impl::sample_token
// (nexus/src/model/hybrid_model.cpp:2023-2099) -- temperature softmax,
// top-k, top-p, renormalize, one uniform draw, the first vocabulary index
// whose running sum reaches it -- so the logits never leave HBM.
//
// One block of 1024 threads per sequence; thread t owns the contiguous
// vocabulary slice [t S, (t + 1) S), so block-wide prefix sums follow the
// vocabulary order.  e_i = expf((l_i - max) / T) is recomputed from the
// logits in every pass (no scratch).
//  - top-k (0 < k <= 1024, k < V): four 8-bit radix passes over the bits of
//    e_i (positive floats order as their bits) find the k-th largest value;
//    ties at that value keep the lowest indices (the reference's
//    partial_sort leaves their order unspecified).  The k survivors go to
//    LDS in index order; top-p sorts them (bitonic, ties by index) and one
//    lane takes the running sum in that order; the renormalization and the
//    draw's scan run over the survivors in index order in one lane, the
//    reference's own summation order.
//  - no top-k (k == 0 or k >= V) with top_p = 1: the draw's scan is a
//    block-wide prefix sum over the vocabulary (fp32 partial sums in a fixed
//    order).  No top-k with top_p < 1 is refused by the launcher.
// The softmax denominator is a fixed-order block sum; the reference's is a
// sequential fp32 sum, so probabilities agree to rounding.
#include "nx_common.h"
#include "nx_kernels.h"

namespace nx {
namespace {

constexpr int kSmpThreads = 1024;
constexpr int kSmpMaxK = 1024;

__device__ inline float smp_block_max(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    if (l == 0) red[w] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = red[0];
        for (int i = 1; i < kSmpThreads / 64; ++i) m = fmaxf(m, red[i]);
        red[16] = m;
    }
    __syncthreads();
    const float r = red[16];
    __syncthreads();
    return r;
}

// Prefix sums of one value per thread, in thread order, with a fixed order
// of additions (a Hillis-Steele scan in each wavefront, then the wavefront
// totals in order).  Returns the exclusive prefix; *incl receives the
// inclusive one and *total the sum.  A thread's inclusive prefix is the same
// float as the next thread's exclusive prefix, so the intervals
// [excl, incl] of consecutive threads meet exactly.
template <class T>
__device__ inline T smp_block_scan(T v, T* wsum, T* incl, T* total) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    T x = v;
    for (int o = 1; o < 64; o <<= 1) {
        const T y = __shfl_up(x, o, 64);
        if (l >= o) x = x + y;
    }
    const T xp = __shfl_up(x, 1, 64);  // the previous lane's inclusive sum
    if (l == 63) wsum[w] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        T acc = T(0);
        for (int i = 0; i < kSmpThreads / 64; ++i) {
            const T s = wsum[i];
            wsum[i] = acc;
            acc = acc + s;
        }
        wsum[16] = acc;
    }
    __syncthreads();
    const T ex = l == 0 ? wsum[w] : wsum[w] + xp;
    *incl = wsum[w] + x;
    *total = wsum[16];
    __syncthreads();
    return ex;
}

__global__ __launch_bounds__(kSmpThreads) void k_sample(SampleArgs a) {
    __shared__ float redf[17];
    __shared__ float scanf_[17];
    __shared__ int scani[17];
    __shared__ int hist[256];
    __shared__ float cand_p[kSmpMaxK];
    __shared__ int cand_i[kSmpMaxK];
    __shared__ int sel_tok;
    const int b = blockIdx.x, tid = threadIdx.x, V = a.V;
    const float* lg = a.logits + (size_t)b * a.ldl;
    const int S = (V + kSmpThreads - 1) / kSmpThreads, i0 = min(tid * S, V), i1 = min(i0 + S, V);
    const float T = a.temperature;

    float mx = -__builtin_inff();
    for (int i = i0; i < i1; ++i) mx = fmaxf(mx, lg[i]);
    mx = smp_block_max(mx, redf);
    auto e_of = [&](int i) { return expf((lg[i] - mx) / T); };
    // softmax denominator: per-thread sums in index order, then thread order
    float part = 0.0f;
    for (int i = i0; i < i1; ++i) part += e_of(i);
    float sum_e = 0.0f, fin = 0.0f;
    (void)smp_block_scan<float>(part, scanf_, &fin, &sum_e);
    // the draw: fixed, per sequence, or keyed by the sequence's position
    float u = a.u_fixed;
    if (u < 0.0f) {
        if (a.u) {
            u = a.u[b];
        } else {
            const uint32_t x = (uint32_t)rand_at(stream_key(a.key, (uint32_t)b), (uint64_t)a.pos[b]);
            u = (float)x / 4294967296.0f;
            if (u >= 1.0f) u = 0.99999994f;  // the largest float below 1
        }
    }

    const bool topk = a.top_k > 0 && a.top_k < V;
    if (topk) {
        // the k-th largest e: radix select over its bits, 8 at a time
        uint32_t prefix = 0, pmask = 0;
        int need = a.top_k;  // still to take at or below the prefix
        for (int sh = 24; sh >= 0; sh -= 8) {
            for (int j = tid; j < 256; j += kSmpThreads) hist[j] = 0;
            __syncthreads();
            for (int i = i0; i < i1; ++i) {
                const uint32_t bits = __builtin_bit_cast(uint32_t, e_of(i) / sum_e);
                if ((bits & pmask) == prefix) atomicAdd(&hist[(bits >> sh) & 0xFF], 1);
            }
            __syncthreads();
            if (tid == 0) {
                int bin = 255, above = 0;
                for (; bin > 0; --bin) {
                    if (above + hist[bin] >= need) break;
                    above += hist[bin];
                }
                hist[0] = bin;      // reuse: chosen bin
                scani[16] = above;  // elements in higher bins
            }
            __syncthreads();
            const int bin = hist[0];
            need -= scani[16];
            prefix |= (uint32_t)bin << sh;
            pmask |= 0xFFu << sh;
            __syncthreads();
        }
        // survivors: values above the k-th, and the first `need` ties by index
        int nab = 0, ntie = 0;
        for (int i = i0; i < i1; ++i) {
            const uint32_t bits = __builtin_bit_cast(uint32_t, e_of(i) / sum_e);
            nab += bits > prefix;
            ntie += bits == prefix;
        }
        int tot = 0, iin = 0;
        const int tie_ex = smp_block_scan<int>(ntie, scani, &iin, &tot);
        int ntake = nab + max(0, min(ntie, need - tie_ex));
        const int at = smp_block_scan<int>(ntake, scani, &iin, &tot);
        int o = at, tr = tie_ex;
        for (int i = i0; i < i1; ++i) {
            const float p = e_of(i) / sum_e;
            const uint32_t bits = __builtin_bit_cast(uint32_t, p);
            bool keep = bits > prefix;
            if (bits == prefix) keep = tr++ < need;
            if (keep && o < kSmpMaxK) {
                cand_p[o] = p;
                cand_i[o] = i;
                ++o;
            }
        }
        __syncthreads();
        const int n = min(tot, kSmpMaxK);
        // top-p: descending order (ties by index) by a bitonic sort of
        // positions 0..n-1 over the next power of two, padding sorting last
        __shared__ int ord[kSmpMaxK];
        int np2 = 1;
        while (np2 < n) np2 <<= 1;
        if (a.top_p < 1.0f) {
            for (int j = tid; j < np2; j += kSmpThreads) ord[j] = j;
            __syncthreads();
            auto before = [&](int x, int y) {  // x sorts before y
                if (x >= n) return false;
                if (y >= n) return true;
                return cand_p[x] > cand_p[y] || (cand_p[x] == cand_p[y] && cand_i[x] < cand_i[y]);
            };
            for (int k2 = 2; k2 <= np2; k2 <<= 1)
                for (int j = k2 >> 1; j > 0; j >>= 1) {
                    for (int x = tid; x < np2; x += kSmpThreads) {
                        const int y = x ^ j;
                        if (y > x) {
                            const int ox = ord[x], oy = ord[y];
                            const bool up = (x & k2) == 0;
                            if (up ? before(oy, ox) : before(ox, oy)) {
                                ord[x] = oy;
                                ord[y] = ox;
                            }
                        }
                    }
                    __syncthreads();
                }
            if (tid == 0) {
                float cum = 0.0f;
                int cut = n;
                for (int j = 0; j < n; ++j) {
                    cum += cand_p[ord[j]];
                    if (cum > a.top_p) {
                        cut = j + 1;
                        break;
                    }
                }
                for (int j = cut; j < n; ++j) cand_p[ord[j]] = 0.0f;
            }
            __syncthreads();
        }
        if (tid == 0) {
            // renormalize and draw over the survivors in index order
            float s = 0.0f;
            for (int j = 0; j < n; ++j) s += cand_p[j];
            int tok = V - 1;
            if (s <= 0.0f) {
                tok = 0;
            } else {
                const float r = u * s;
                float cum = 0.0f;
                if (r <= 0.0f) {
                    tok = 0;  // the running sum reaches 0 at index 0
                } else {
                    for (int j = 0; j < n; ++j) {
                        cum += cand_p[j];
                        if (cum >= r) {
                            tok = cand_i[j];
                            break;
                        }
                    }
                }
            }
            sel_tok = tok;
        }
        __syncthreads();
    } else {
        // all V kept: r = u * (sum of p), scan in vocabulary order
        float ps = 0.0f;
        for (int i = i0; i < i1; ++i) ps += e_of(i) / sum_e;
        float total = 0.0f, inc = 0.0f;
        const float ex = smp_block_scan<float>(ps, scanf_, &inc, &total);
        const float r = u * total;
        if (tid == 0) sel_tok = r <= 0.0f ? 0 : V - 1;
        __syncthreads();
        if (r > 0.0f && ex < r && inc >= r) {  // this slice holds the crossing (exactly one does)
            float cum = ex;
            int tok = -1, last = -1;
            for (int i = i0; i < i1; ++i) {
                const float p = e_of(i) / sum_e;
                if (p > 0.0f) last = i;
                cum += p;
                if (cum >= r) {
                    tok = i;
                    break;
                }
            }
            sel_tok = tok >= 0 ? tok : (last >= 0 ? last : i0);
        }
        __syncthreads();
    }
    if (tid == 0) {
        if (a.out) a.out[b] = sel_tok;
        if (a.best) a.best[b] = 0xFFFFFFFFull - (unsigned long long)(uint32_t)sel_tok;
    }
}

}  // namespace

hipError_t sample_launch(const SampleArgs& a, int batch, hipStream_t st) {
    if (a.V < 1 || batch < 1 || a.temperature <= 0.0f || a.top_k < 0 || (a.top_k > kSmpMaxK && a.top_k < a.V) ||
        !(a.top_p > 0.0f) || ((a.top_k == 0 || a.top_k >= a.V) && a.top_p < 1.0f) ||
        (a.u_fixed < 0.0f && !a.u && !a.pos))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_sample, dim3(batch), dim3(kSmpThreads), 0, st, a);
    return hipGetLastError();
}

}  // namespace nx
