// Token sampling on the device: HybridModel::Impl::sample_token
// (nexus/src/model/hybrid_model.cpp:2023-2099) -- temperature softmax,
// top-k, top-p, renormalize, one uniform draw, the first vocabulary index
// whose running sum reaches it -- so the logits never leave HBM.
//
// Three launches: the maximum logit, then e_i = expf((l_i - max) / T) into a
// scratch row with partial sums and candidate counts, each over 64 blocks
// per sequence (k_sample_max, k_sample_exp); then one block of 1024 threads
// per sequence (k_sample) for the selection and the draw.  In k_sample,
// wavefront w owns the contiguous vocabulary chunk [w C, (w + 1) C) and
// walks it 64 consecutive entries at a time (coalesced), so wavefront order
// then iteration order then lane order is vocabulary order; ballots keep
// that order where it matters.  Later passes read p_i = e_i / sum.
//  - top-k (0 < k <= 1024, k < V): four 8-bit radix passes over the bits of
//    p_i (positive floats order as their bits) find the k-th largest value;
//    ties at that value keep the lowest indices (the reference's
//    partial_sort leaves their order unspecified).  The k survivors go to
//    LDS in index order; top-p sorts them (bitonic, ties by index) and one
//    lane takes the running sum in that order; the renormalization and the
//    draw's scan run over the survivors in index order in one lane, the
//    reference's own summation order.
//  - otherwise (no top-k, or k above 1024; with or without top-p): every
//    entry is a candidate.  A radix selection by counts finds the k-th
//    largest p, a radix selection by probability mass (exact 40-bit
//    fixed-point sums) finds where the running sum in descending order
//    first exceeds top_p; ties at either value keep the lowest indices.
//    The draw's scan runs over the kept entries in wavefront, iteration and
//    lane order with fp32 partial sums in a fixed order.
// The softmax denominator is a fixed-order sum (per block, then the blocks
// in order); the reference's is a sequential fp32 sum, so probabilities
// agree to rounding.
#include "nx_common.h"
#include "nx_kernels.h"

namespace nx {
namespace {

constexpr int kSmpThreads = 1024;
constexpr int kSmpMaxK = 1024;
constexpr int kSmpCand = kSmpCandMax;  // top-k candidates held in LDS
constexpr int kSmpThr = 8;      // candidate thresholds e >= exp(-D)
__constant__ float c_smp_D[kSmpThr] = {24.0f, 16.0f, 12.0f, 8.0f, 5.0f, 3.0f, 2.0f, 1.0f};

constexpr int kSmpWaves = kSmpThreads / 64;

__device__ inline float smp_wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
template <class T>
__device__ inline T smp_wave_sum(T v) {
    for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o, 64);
    return v;
}
// inclusive prefix over the 64 lanes (Hillis-Steele, fixed order)
__device__ inline float smp_wave_scan(float x) {
    const int l = threadIdx.x & 63;
    for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_up(x, o, 64);
        if (l >= o) x = x + y;
    }
    return x;
}
__device__ inline int popc_below(unsigned long long m, int l) {
    return __popcll(m & ((1ull << l) - 1ull));
}

// Prefix sums of one value per thread in thread order, fixed order of
// additions (a Hillis-Steele scan per wavefront, then the wavefront totals
// in order); wsum holds kSmpWaves + 1 entries.  Returns the exclusive
// prefix; *incl the inclusive one, *total the sum.
template <class T>
__device__ inline T smp_block_scan(T v, T* wsum, T* incl, T* total) {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63;
    T x = v;
    for (int o = 1; o < 64; o <<= 1) {
        const T y = __shfl_up(x, o, 64);
        if (l >= o) x = x + y;
    }
    const T xp = __shfl_up(x, 1, 64);
    if (l == 63) wsum[w] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        T acc = T(0);
        for (int i = 0; i < kSmpWaves; ++i) {
            const T t = wsum[i];
            wsum[i] = acc;
            acc = acc + t;
        }
        wsum[kSmpWaves] = acc;
    }
    __syncthreads();
    const T ex = l == 0 ? wsum[w] : wsum[w] + xp;
    *incl = wsum[w] + x;
    *total = wsum[kSmpWaves];
    __syncthreads();
    return ex;
}

// One pass of a wavefront over its chunk [c0, c1): kSmpU loads per lane are
// requested before any is used (a block has only 16 wavefronts to hide the
// memory latency with), then use(i0, valid, value) runs for the 64-entry
// steps i0 in order (entry i0 + lane).  Indices past c1 load c1 - 1 and
// are passed as not valid.
constexpr int kSmpU = 16;
template <class Load, class Use>
__device__ inline void smp_pass(int c0, int c1, Load load, Use use) {
    const int l = threadIdx.x & 63;
    for (int base = c0; base < c1; base += 64 * kSmpU) {
        float v[kSmpU];
#pragma unroll
        for (int u = 0; u < kSmpU; ++u) v[u] = load(min(base + 64 * u + l, c1 - 1));
#pragma unroll
        for (int u = 0; u < kSmpU; ++u) use(base + 64 * u, base + 64 * u + l < c1, v[u]);
    }
}

// The first two passes over the vocabulary, spread over kSmpBlocks blocks
// per sequence (on the one block of k_sample they took 50 of its 85 us):
// block p = 4 w + q covers quarter q of k_sample wavefront w's chunk.
// k_sample_max writes each block's maximum logit; k_sample_exp takes the
// maximum of those (exact in any order), writes e_i = expf((l_i - max) / T)
// into the scratch row and each block's sum of e (per thread in index
// order, wavefront tree, wavefronts in order) and its counts at each
// candidate threshold.  k_sample adds the sums in block order.
constexpr int kSmpPThreads = 256, kSmpPWaves = kSmpPThreads / 64;
static_assert(kSmpBlocks == 4 * kSmpWaves && kSmpBlocks == 64, "four blocks per k_sample wavefront chunk, one per lane");
static_assert(kSmpCandOff == kSmpBlocks * (2 + kSmpThr), "partials: max, sum, counts");
__device__ inline void smp_block_range(int V, int p, int& c0, int& c1) {
    const int C = ((V + kSmpWaves - 1) / kSmpWaves + 63) / 64 * 64, Q = C / 4;
    c0 = min((p / 4) * C + (p % 4) * Q, V);
    c1 = min(c0 + Q, V);
}

__global__ __launch_bounds__(kSmpPThreads) void k_sample_max(SampleArgs a) {
    __shared__ float wm[kSmpPWaves];
    const int p = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const float* lg = a.logits + (size_t)b * a.ldl;
    int c0, c1;
    smp_block_range(a.V, p, c0, c1);
    float mx = -__builtin_inff();
    for (int i = c0 + tid; i < c1; i += kSmpPThreads) mx = fmaxf(mx, lg[i]);
    mx = smp_wave_max(mx);
    if ((tid & 63) == 0) wm[tid >> 6] = mx;
    __syncthreads();
    if (tid == 0) {
        float m = wm[0];
        for (int j = 1; j < kSmpPWaves; ++j) m = fmaxf(m, wm[j]);
        a.part[(size_t)b * kSmpPartFloats + p] = m;
    }
}

__global__ __launch_bounds__(kSmpPThreads) void k_sample_exp(SampleArgs a) {
    __shared__ float wm[kSmpPWaves];
    __shared__ int wc[kSmpThr][kSmpPWaves];
    const int p = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63;
    const float* lg = a.logits + (size_t)b * a.ldl;
    float* e = a.scratch + (size_t)b * a.V;
    float* pt = a.part + (size_t)b * kSmpPartFloats;
    int c0, c1;
    smp_block_range(a.V, p, c0, c1);
    // the sequence's maximum: every wavefront takes it from the blocks' maxima
    const float mx = smp_wave_max(pt[l]);
    const float T = a.temperature;
    float sum = 0.0f, thr[kSmpThr];
    int cnt[kSmpThr];
#pragma unroll
    for (int j = 0; j < kSmpThr; ++j) {
        thr[j] = expf(-c_smp_D[j]);
        cnt[j] = 0;
    }
    for (int i = c0 + tid; i < c1; i += kSmpPThreads) {
        const float v = expf((lg[i] - mx) / T);
        e[i] = v;
        sum += v;
#pragma unroll
        for (int j = 0; j < kSmpThr; ++j) cnt[j] += v >= thr[j];
    }
    sum = smp_wave_sum(sum);
#pragma unroll
    for (int j = 0; j < kSmpThr; ++j) {
        const int c = smp_wave_sum(cnt[j]);
        if (l == 0) wc[j][w] = c;
    }
    if (l == 0) wm[w] = sum;
    __syncthreads();
    if (tid == 0) {
        float s = 0.0f;
        for (int j = 0; j < kSmpPWaves; ++j) s += wm[j];
        pt[kSmpBlocks + p] = s;
    }
    if (tid < kSmpThr) {
        int c = 0;
        for (int j = 0; j < kSmpPWaves; ++j) c += wc[tid][j];
        pt[2 * kSmpBlocks + kSmpThr * p + tid] = (float)c;  // exact: c <= V < 2^24
    }
}

// Top-k (k <= kSmpMaxK) with a candidate threshold that fits kSmpCand: the
// threshold pick of k_sample (the smallest D whose count of e >= exp(-D) is
// at least k), then block p writes the entries of its range at or above it,
// in index order, at the sum of the earlier blocks' counts -- the candidate
// list k_sample would gather with one pass over the row on one CU.
__global__ __launch_bounds__(kSmpPThreads) void k_sample_gather(SampleArgs a) {
    __shared__ int wsum[kSmpPWaves];
    __shared__ int pk[2];
    __shared__ float sm;
    const int p = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63;
    if (!(a.top_k > 0 && a.top_k < a.V && a.top_k <= kSmpMaxK)) return;
    const float* e = a.scratch + (size_t)b * a.V;
    float* pt = a.part + (size_t)b * kSmpPartFloats;
    if (w == 0) {
        // lane q: block q's counts; totals in a fixed order (exact integers)
        int pick = -1, base = 0;
        for (int j = 0; j < kSmpThr; ++j) {
            const int c = (int)pt[2 * kSmpBlocks + kSmpThr * l + j];
            const int tot = smp_wave_sum(c);
            if (tot >= a.top_k) {
                pick = tot <= kSmpCand ? j : -2;
                base = smp_wave_sum(l < p ? c : 0);
            }
        }
        if (l == 0) {
            pk[0] = pick;
            pk[1] = base;
        }
    }
    if (tid == 0) {
        float acc = 0.0f;
        for (int j = 0; j < kSmpBlocks; ++j) acc += pt[kSmpBlocks + j];
        sm = acc;
    }
    __syncthreads();
    const int pick = pk[0];
    if (pick < 0) return;
    int base = pk[1];
    const float sum_e = sm, th = expf(-c_smp_D[pick]);
    float* cp = pt + kSmpCandOff;
    int* ci = reinterpret_cast<int*>(cp + kSmpCandMax);
    int c0, c1;
    smp_block_range(a.V, p, c0, c1);
    for (int i0 = c0; i0 < c1; i0 += kSmpPThreads) {
        const int i = i0 + tid;
        const float ev = i < c1 ? e[i] : 0.0f;
        const bool keep = i < c1 && ev >= th;
        const unsigned long long km = __ballot(keep);
        if (l == 0) wsum[w] = __popcll(km);
        __syncthreads();
        int before = 0, all = 0;
        for (int j = 0; j < kSmpPWaves; ++j) {
            before += j < w ? wsum[j] : 0;
            all += wsum[j];
        }
        if (keep) {
            const int at = base + before + popc_below(km, l);
            cp[at] = ev / sum_e;
            ci[at] = i;
        }
        base += all;
        __syncthreads();
    }
}

__global__ __launch_bounds__(kSmpThreads) void k_sample(SampleArgs a) {
    __shared__ float wf[kSmpWaves + 1];
    __shared__ int wi[4][kSmpWaves + 1];
    __shared__ int hist[256];
    __shared__ int sel;
    __shared__ float cand_p[kSmpCand];
    __shared__ int cand_i[kSmpCand];
    __shared__ int ord[kSmpCand];
    __shared__ int tcnt[kSmpThr][kSmpWaves + 1];
    const int b = blockIdx.x, tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, V = a.V;
    const float* e = a.scratch + (size_t)b * V;
    const int C = ((V + kSmpWaves - 1) / kSmpWaves + 63) / 64 * 64;
    const int c0 = min(w * C, V), c1 = min(c0 + C, V);

    // the e row, its sum (the blocks' sums in block order) and per wavefront
    // chunk the entries at or above each candidate threshold exp(-D), from
    // k_sample_max / k_sample_exp
    const float* pt = a.part + (size_t)b * kSmpPartFloats;
    if (tid < kSmpThr * kSmpWaves) {
        const int j = tid / kSmpWaves, ww = tid % kSmpWaves;
        float c = 0.0f;
        for (int q = 0; q < 4; ++q) c += pt[2 * kSmpBlocks + kSmpThr * (4 * ww + q) + j];
        tcnt[j][ww] = (int)c;
    }
    if (tid == 0) {
        float acc = 0.0f;
        for (int j = 0; j < kSmpBlocks; ++j) acc += pt[kSmpBlocks + j];
        wf[kSmpWaves] = acc;
    }
    __syncthreads();
    const float sum_e = wf[kSmpWaves];
    __syncthreads();
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

    if (a.top_k > 0 && a.top_k < V && a.top_k <= kSmpMaxK) {
        // candidates: the entries with e >= exp(-D) for the smallest D whose
        // count is at least k (they hold the top k: p orders as e), if that
        // count fits in LDS; otherwise a radix selection over all of p finds
        // exactly k
        if (w == 0) {
            // lane j < kSmpThr: threshold j's exclusive prefix over the
            // wavefronts and its total; D decreases with j, so the pick is
            // the last threshold whose count reaches k (-2 if that count
            // does not fit the candidate list, -1 if none reaches k)
            int tot = 0;
            if (l < kSmpThr) {
                for (int q = 0; q < kSmpWaves; ++q) {
                    const int c = tcnt[l][q];
                    tcnt[l][q] = tot;
                    tot += c;
                }
                tcnt[l][kSmpWaves] = tot;
            }
            const unsigned long long ok = __ballot(l < kSmpThr && tot >= a.top_k);
            const int jm = ok ? 63 - __clzll(ok) : 0;
            const int tj = __shfl(tot, jm, kWave);
            if (l == 0) wi[0][3] = ok ? (tj <= kSmpCand ? jm : -2) : -1;
        }
        __syncthreads();
        int n = 0;
        const int pick = wi[0][3];
        if (pick >= 0) {
            // the candidates gathered by k_sample_gather, in index order
            n = tcnt[pick][kSmpWaves];
            const float* cp = a.part + (size_t)b * kSmpPartFloats + kSmpCandOff;
            const int* ci = reinterpret_cast<const int*>(cp + kSmpCandMax);
            for (int j = tid; j < n; j += kSmpThreads) {
                cand_p[j] = cp[j];
                cand_i[j] = ci[j];
            }
        } else {
        // the k-th largest p: radix select over its bits, 8 at a time
        uint32_t prefix = 0, pmask = 0;
        int need = a.top_k;  // still to take at or below the prefix
        for (int sh = 24; sh >= 0; sh -= 8) {
            for (int j = tid; j < 256; j += kSmpThreads) hist[j] = 0;
            __syncthreads();
            smp_pass(c0, c1, [&](int i) { return e[i]; }, [&](int, bool ok, float ev) {
                const uint32_t bits = __builtin_bit_cast(uint32_t, ev / sum_e);
                if (ok && (bits & pmask) == prefix) atomicAdd(&hist[(bits >> sh) & 0xFF], 1);
            });
            __syncthreads();
            if (tid == 0) {
                int bin = 255, above = 0;
                for (; bin > 0; --bin) {
                    if (above + hist[bin] >= need) break;
                    above += hist[bin];
                }
                wi[0][0] = bin;
                wi[0][1] = above;
            }
            __syncthreads();
            prefix |= (uint32_t)wi[0][0] << sh;
            pmask |= 0xFFu << sh;
            need -= wi[0][1];
            __syncthreads();
        }
        // per wavefront: values above the k-th and ties with it
        int nab = 0, ntie = 0;
        smp_pass(c0, c1, [&](int i) { return e[i]; }, [&](int, bool ok, float ev) {
            const uint32_t bits = __builtin_bit_cast(uint32_t, ev / sum_e);
            nab += ok && bits > prefix;
            ntie += ok && bits == prefix;
        });
        nab = smp_wave_sum(nab);
        ntie = smp_wave_sum(ntie);
        if (l == 0) {
            wi[1][w] = nab;
            wi[2][w] = ntie;
        }
        __syncthreads();
        if (tid == 0) {  // ties before each wavefront, and its first output slot
            int tb = 0, ob = 0;
            for (int j = 0; j < kSmpWaves; ++j) {
                const int nt = wi[2][j];
                wi[2][j] = tb;
                wi[3][j] = ob;
                ob += wi[1][j] + max(0, min(nt, need - tb));
                tb += nt;
            }
            wi[0][2] = ob;  // survivors
        }
        __syncthreads();
        // gather the survivors in index order
        int trun = wi[2][w], orun = wi[3][w];
        smp_pass(c0, c1, [&](int i) { return e[i]; }, [&](int i0, bool in, float ev) {
            const float p = ev / sum_e;
            const uint32_t bits = __builtin_bit_cast(uint32_t, p);
            const bool tie = in && bits == prefix;
            const unsigned long long tm = __ballot(tie);
            const bool keep = in && (bits > prefix || (tie && trun + popc_below(tm, l) < need));
            const unsigned long long km = __ballot(keep);
            const int at = orun + popc_below(km, l);
            if (keep && at < kSmpMaxK) {
                cand_p[at] = p;
                cand_i[at] = i0 + l;
            }
            trun += __popcll(tm);
            orun += __popcll(km);
        });
        n = min(wi[0][2], kSmpMaxK);
        }
        __syncthreads();
        // descending order of p (ties by index): a bitonic sort of positions
        // 0..n-1 over the next power of two, padding sorting last; the first
        // k are the top k, then top-p cuts along the same order
        const int kk = min(a.top_k, n);
        int np2 = 1;
        while (np2 < n) np2 <<= 1;
        if (n > kk || a.top_p < 1.0f) {
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
            // top-p: the running sum in sorted order by one wavefront (lane
            // j holds entry j, read in order), then the entries past the cut
            // are cleared by the block
            if (w == 0) {
                int cut = kk;
                if (a.top_p < 1.0f) {
                    if (kk <= kWave) {
                        const float pv = l < kk ? cand_p[ord[l]] : 0.0f;
                        float cum = 0.0f;
                        for (int j = 0; j < kk; ++j) {
                            cum += readlane_f(pv, j);
                            if (cum > a.top_p) {
                                cut = j + 1;
                                break;
                            }
                        }
                    } else {
                        float cum = 0.0f;
                        for (int j = 0; j < kk; ++j) {
                            cum += cand_p[ord[j]];
                            if (cum > a.top_p) {
                                cut = j + 1;
                                break;
                            }
                        }
                    }
                }
                if (l == 0) wi[0][0] = cut;
            }
            __syncthreads();
            const int cut = wi[0][0];
            for (int j = cut + tid; j < n; j += kSmpThreads) cand_p[ord[j]] = 0.0f;
            __syncthreads();
        }
        // the kept entries (at most k) in index order, compacted in parallel
        // (thread t holds candidates 4t .. 4t+3), then renormalized and drawn
        // from by one lane in that order
        int nk = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) nk += 4 * tid + q < n && cand_p[4 * tid + q] > 0.0f;
        int ktot = 0, kin = 0;
        const int kat = smp_block_scan<int>(nk, wi[1], &kin, &ktot);
        {
            int o = kat;
            float kp[4];
            int ki[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int j = 4 * tid + q;
                kp[q] = j < n ? cand_p[j] : 0.0f;
                ki[q] = j < n ? cand_i[j] : 0;
            }
            __syncthreads();  // the candidate arrays are rewritten in place
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (kp[q] > 0.0f) {
                    cand_p[o] = kp[q];
                    cand_i[o] = ki[q];
                    ++o;
                }
        }
        __syncthreads();
        // renormalization and draw by one wavefront, in index order (lane j
        // holds kept entry j when there are at most 64, read in order)
        if (w == 0) {
            const bool lanes = ktot <= kWave;
            const float pv = lanes && l < ktot ? cand_p[l] : 0.0f;
            const int iv = lanes && l < ktot ? cand_i[l] : 0;
            auto p_at = [&](int j) { return lanes ? readlane_f(pv, j) : cand_p[j]; };
            float sm = 0.0f;
            for (int j = 0; j < ktot; ++j) sm += p_at(j);
            int tok = V - 1;
            const float r = u * sm;
            if (sm <= 0.0f || r <= 0.0f) {
                tok = 0;  // nothing kept, or the running sum reaches r = 0 at index 0
            } else {
                float cum = 0.0f;
                for (int j = 0; j < ktot; ++j) {
                    cum += p_at(j);
                    if (cum >= r) {
                        tok = lanes ? __builtin_amdgcn_readlane(iv, j) : cand_i[j];
                        break;
                    }
                }
            }
            if (l == 0) sel = tok;
        }
        __syncthreads();
    } else {
        // Every entry is a candidate: no top-k, or top-k above the candidate
        // list (kSmpMaxK), each with or without top-p.  A top-k cut keeps the
        // entries above the k-th largest p and, of the entries equal to it,
        // the lowest indices (radix selection of the k-th value by counts).
        // A top-p cut keeps, in descending order of p (ties by index), the
        // entries up to the first whose running sum exceeds top_p (radix
        // selection of that value by probability mass; the masses are summed
        // as 40-bit fixed-point integers, exact and independent of order,
        // where the reference adds fp32 in its sorted order).  The kept
        // entries are renormalized and drawn from in vocabulary order.
        const bool use_k = a.top_k > 0 && a.top_k < V;
        const bool use_p = a.top_p < 1.0f;
        // --- top-k: the k-th largest p (bits kb) and how many of its ties to keep
        uint32_t kb = 0;
        int kneed = 0;
        if (use_k) {
            uint32_t prefix = 0, pmask = 0;
            int need = a.top_k;
            for (int sh = 24; sh >= 0; sh -= 8) {
                for (int j2 = tid; j2 < 256; j2 += kSmpThreads) hist[j2] = 0;
                __syncthreads();
                smp_pass(c0, c1, [&](int i) { return e[i]; }, [&](int, bool ok, float ev) {
                    const uint32_t bits = __builtin_bit_cast(uint32_t, ev / sum_e);
                    if (ok && (bits & pmask) == prefix) atomicAdd(&hist[(bits >> sh) & 0xFF], 1);
                });
                __syncthreads();
                if (tid == 0) {
                    int bin = 255, above = 0;
                    for (; bin > 0; --bin) {
                        if (above + hist[bin] >= need) break;
                        above += hist[bin];
                    }
                    wi[0][0] = bin;
                    wi[0][1] = above;
                }
                __syncthreads();
                prefix |= (uint32_t)wi[0][0] << sh;
                pmask |= 0xFFu << sh;
                need -= wi[0][1];
                __syncthreads();
            }
            kb = prefix;
            kneed = need;
        }
        // tie ranks in vocabulary order: each wavefront's count of ties, then
        // the exclusive prefix over the wavefronts (ranks[w])
        auto wave_base = [&](int cnt, int* base) {
            cnt = smp_wave_sum(cnt);
            if (l == 0) base[w] = cnt;
            __syncthreads();
            if (tid == 0) {
                int acc = 0;
                for (int q = 0; q < kSmpWaves; ++q) {
                    const int c = base[q];
                    base[q] = acc;
                    acc += c;
                }
                base[kSmpWaves] = acc;
            }
            __syncthreads();
            return base[w];
        };
        int ktb = 0;
        if (use_k) {
            int cnt = 0;
            smp_pass(c0, c1, [&](int i) { return e[i]; }, [&](int, bool ok, float ev) {
                cnt += ok && __builtin_bit_cast(uint32_t, ev / sum_e) == kb;
            });
            ktb = wave_base(cnt, wi[1]);
        }
        // keep-by-k of the 64 entries of one step (krun: ties of kb before them)
        auto kept_k = [&](bool ok, uint32_t bits, int& krun) {
            const bool tie = ok && use_k && bits == kb;
            const unsigned long long tm = __ballot(tie);
            const bool keep = ok && (!use_k || bits > kb || (tie && krun + popc_below(tm, l) < kneed));
            krun += __popcll(tm);
            return keep;
        };
        // --- top-p over the entries top-k keeps: the value pb at which the
        // running mass first exceeds top_p, the mass above it, and how many
        // of its ties to keep
        __shared__ unsigned long long hmass[256];
        __shared__ int pinfo[1];
        bool pcut = false;
        uint32_t pb = 0;
        int pneed = 0;
        if (use_p) {
            const unsigned long long tp = (unsigned long long)((double)a.top_p * 1099511627776.0);
            uint32_t prefix = 0, pmask = 0;
            unsigned long long above = 0;
            bool cut = true;
            for (int sh = 24; sh >= 0 && cut; sh -= 8) {
                for (int j2 = tid; j2 < 256; j2 += kSmpThreads) hmass[j2] = 0ull;
                __syncthreads();
                int krun = ktb;
                smp_pass(c0, c1, [&](int i) { return e[i]; }, [&](int, bool ok, float ev) {
                    const float pv = ev / sum_e;
                    const uint32_t bits = __builtin_bit_cast(uint32_t, pv);
                    const bool keep = kept_k(ok, bits, krun);
                    if (keep && (bits & pmask) == prefix)
                        atomicAdd(&hmass[(bits >> sh) & 0xFF], (unsigned long long)(pv * 1099511627776.0f));
                });
                __syncthreads();
                if (tid == 0) {
                    int bin = 255;
                    unsigned long long ab = above;
                    for (; bin >= 0; --bin) {
                        if (ab + hmass[bin] > tp) break;
                        ab += hmass[bin];
                    }
                    pinfo[0] = bin;  // -1: the kept mass never exceeds top_p
                    // mass above the crossing bin, carried in LDS as two words
                    wi[0][1] = (int)(uint32_t)(ab & 0xFFFFFFFFull);
                    wi[0][2] = (int)(uint32_t)(ab >> 32);
                }
                __syncthreads();
                const int bin = pinfo[0];
                if (bin < 0) {
                    cut = false;
                } else {
                    prefix |= (uint32_t)bin << sh;
                    pmask |= 0xFFu << sh;
                    above = (unsigned long long)(uint32_t)wi[0][1] | ((unsigned long long)(uint32_t)wi[0][2] << 32);
                }
                __syncthreads();
            }
            if (cut) {
                pcut = true;
                pb = prefix;
                const unsigned long long unit =
                    (unsigned long long)(__builtin_bit_cast(float, pb) * 1099511627776.0f);
                // smallest m >= 1 with above + m * unit > tp
                pneed = unit > 0 ? (int)min((tp - above) / unit + 1ull, (unsigned long long)V) : V;
            }
        }
        int ptb = 0;
        if (pcut) {
            int cnt = 0, krun = ktb;
            smp_pass(c0, c1, [&](int i) { return e[i]; }, [&](int, bool ok, float ev) {
                const uint32_t bits = __builtin_bit_cast(uint32_t, ev / sum_e);
                const bool keep = kept_k(ok, bits, krun);
                cnt += keep && bits == pb;
            });
            ptb = wave_base(cnt, wi[2]);
        }
        // the kept p of one step's entry (krun, prun: ties before the step)
        auto kept_p = [&](bool ok, float ev, int& krun, int& prun) {
            const float pv = ev / sum_e;
            const uint32_t bits = __builtin_bit_cast(uint32_t, pv);
            const bool keep = kept_k(ok, bits, krun);
            const bool tie = keep && pcut && bits == pb;
            const unsigned long long tm = __ballot(tie);
            const bool kp = keep && (!pcut || bits > pb || (tie && prun + popc_below(tm, l) < pneed));
            prun += __popcll(tm);
            return kp ? pv : 0.0f;
        };
        // --- the draw: running sums per wavefront (64-lane scans, iterations
        // in order), wavefronts in order
        float run = 0.0f;
        {
            int krun = ktb, prun = ptb;
            smp_pass(c0, c1, [&](int i) { return e[i]; }, [&](int, bool ok, float ev) {
                const float x = smp_wave_scan(kept_p(ok, ev, krun, prun));
                run = run + __shfl(x, 63, 64);
            });
        }
        if (l == 0) wf[w] = run;
        __syncthreads();
        if (tid == 0) {
            float acc = 0.0f;
            for (int j2 = 0; j2 < kSmpWaves; ++j2) {
                const float t = wf[j2];
                wf[j2] = acc;
                acc = acc + t;
            }
            wf[kSmpWaves] = acc;
            sel = -1;
        }
        __syncthreads();
        const float base = wf[w], next = w + 1 < kSmpWaves ? wf[w + 1] : wf[kSmpWaves];
        const float r = u * wf[kSmpWaves];
        if (r > 0.0f && base < r && next >= r) {  // this wavefront holds the crossing (exactly one does)
            float rr = 0.0f;
            int tok = -1, lastnz = -1, krun = ktb, prun = ptb;
            smp_pass(c0, c1, [&](int i) { return e[i]; }, [&](int i0, bool ok, float ev) {
                const float p = kept_p(ok, ev, krun, prun);  // every step: the tie counts advance
                if (tok >= 0) return;  // uniform: found in an earlier step
                const float x = smp_wave_scan(p);
                const float it = __shfl(x, 63, 64);
                const unsigned long long nz = __ballot(p > 0.0f);
                if (base + (rr + it) >= r) {
                    const unsigned long long hit = __ballot(base + (rr + x) >= r && p > 0.0f);
                    tok = hit ? i0 + __ffsll((long long)hit) - 1 : (nz ? i0 + 63 - __clzll((long long)nz) : lastnz);
                }
                if (nz) lastnz = i0 + 63 - __clzll((long long)nz);
                rr = rr + it;
            });
            if (l == 0) sel = tok >= 0 ? tok : (lastnz >= 0 ? lastnz : c0);
        }
        __syncthreads();
        if (tid == 0 && sel < 0) sel = r <= 0.0f ? 0 : V - 1;
        __syncthreads();
    }
    if (tid == 0) {
        if (a.out) a.out[b] = sel;
        if (a.best) a.best[b] = 0xFFFFFFFFull - (unsigned long long)(uint32_t)sel;
    }
}

}  // namespace

hipError_t sample_launch(const SampleArgs& a, int batch, hipStream_t st) {
    if (a.V < 1 || a.V >= (1 << 24) || batch < 1 || a.temperature <= 0.0f || a.top_k < 0 || !(a.top_p > 0.0f) ||
        a.top_p > 1.0f || (a.u_fixed < 0.0f && !a.u && !a.pos) || !a.scratch || !a.part)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_sample_max, dim3(kSmpBlocks, batch), dim3(kSmpPThreads), 0, st, a);
    hipLaunchKernelGGL(k_sample_exp, dim3(kSmpBlocks, batch), dim3(kSmpPThreads), 0, st, a);
    if (a.top_k > 0 && a.top_k < a.V && a.top_k <= kSmpMaxK)
        hipLaunchKernelGGL(k_sample_gather, dim3(kSmpBlocks, batch), dim3(kSmpPThreads), 0, st, a);
    hipLaunchKernelGGL(k_sample, dim3(batch), dim3(kSmpThreads), 0, st, a);
    return hipGetLastError();
}

}  // namespace nx
