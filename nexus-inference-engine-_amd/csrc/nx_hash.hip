// Chunk checksums on the device: XXH32 (seed 0) of many byte ranges of one
// device buffer.  It is the checksum NXFWriter::add_chunk stores for every
// NXF chunk (nexus/src/format/nxf_writer.cpp:33-72, :255), computed here
// where the chunk bytes already are after an upload, so a whole model is
// verified at HBM speed instead of on one host core.
//
// XXH32 is sequential inside a chunk: four accumulators v1..v4 each take one
// 4-byte word of every 16-byte stripe.  The parallelism is therefore across
// chunks: a quad of lanes owns a chunk, lane q keeps accumulator q, and a
// wavefront hashes 16 chunks.  Each lane loads whole 16-byte stripes (lane q
// stripes 4u + q of each group of four, so a quad reads 64 contiguous bytes
// per load) and a 4 x 4 transpose inside the quad (two DPP exchanges) hands
// lane q word q of the four stripes.  The host sorts the ranges by length so
// the quads of a wavefront run loops of similar length.
#include "nx_common.h"
#include "nx_kernels.h"

namespace nx {
namespace {

constexpr uint32_t kP1 = 0x9E3779B1u, kP2 = 0x85EBCA77u, kP3 = 0xC2B2AE3Du, kP4 = 0x27D4EB2Fu,
                   kP5 = 0x165667B1u;
constexpr int kHashThreads = 256;
constexpr int kHashUnroll = 4;  // steps of 8 stripes requested together

__device__ inline uint32_t rotl32(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

// DPP quad permutations: lane q reads lane q ^ 1 / q ^ 2 of its quad.
__device__ inline uint32_t quad_xor1(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
}
__device__ inline uint32_t quad_xor2(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
}

// Lane q of a quad holds stripe q (w = its words 0..3); afterwards it holds
// word q of stripes 0..3.  First the off-diagonal 2 x 2 blocks are exchanged
// between lanes q and q ^ 2, then the off-diagonal words of each block
// between lanes q and q ^ 1.
__device__ inline void quad_transpose(uint4& w, int q) {
    const bool lo2 = (q & 2) == 0;
    uint32_t r0 = quad_xor2(lo2 ? w.z : w.x), r1 = quad_xor2(lo2 ? w.w : w.y);
    if (lo2) {
        w.z = r0;
        w.w = r1;
    } else {
        w.x = r0;
        w.y = r1;
    }
    const bool lo1 = (q & 1) == 0;
    r0 = quad_xor1(lo1 ? w.y : w.x);
    r1 = quad_xor1(lo1 ? w.w : w.z);
    if (lo1) {
        w.y = r0;
        w.w = r1;
    } else {
        w.x = r0;
        w.z = r1;
    }
}

__global__ __launch_bounds__(kHashThreads) void k_xxh32(const uint8_t* __restrict__ data,
                                                        const HashRange* __restrict__ ranges, int n,
                                                        uint32_t* __restrict__ out) {
    const int r = (int)((blockIdx.x * kHashThreads + threadIdx.x) >> 2), q = threadIdx.x & 3;
    if (r >= n) return;  // the four lanes of a quad leave together
    const HashRange rg = ranges[r];
    const uint8_t* base = data + rg.off;
    const uint32_t nstripe = rg.len >> 4;
    uint32_t v = q == 0 ? kP1 + kP2 : q == 1 ? kP2 : q == 2 ? 0u : 0u - kP1;
    if (nstripe > 0) {
        // a step is 8 stripes: lane q loads stripes 8t + q and 8t + 4 + q;
        // requests past the last stripe re-read it (their words are unused)
        const uint32_t last = nstripe - 1, nstep = (nstripe + 7) >> 3;
        for (uint32_t t0 = 0; t0 < nstep; t0 += kHashUnroll) {
            uint4 w[kHashUnroll][2];
#pragma unroll
            for (int u = 0; u < kHashUnroll; ++u)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t s = min(8u * (t0 + u) + 4u * h + (uint32_t)q, last);
                    w[u][h] = *reinterpret_cast<const uint4*>(base + 16ull * s);
                }
#pragma unroll
            for (int u = 0; u < kHashUnroll; ++u) {
                const int rem = (int)nstripe - 8 * (int)(t0 + u);  // stripes left from this step on
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    quad_transpose(w[u][h], q);
                    const uint32_t wd[4] = {w[u][h].x, w[u][h].y, w[u][h].z, w[u][h].w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t nv = rotl32(v + wd[j] * kP2, 13) * kP1;
                        v = 4 * h + j < rem ? nv : v;
                    }
                }
            }
        }
    }
    // merge the four accumulators: rotl(v1,1) + rotl(v2,7) + rotl(v3,12) + rotl(v4,18)
    uint32_t m = rotl32(v, q == 0 ? 1 : q == 1 ? 7 : q == 2 ? 12 : 18);
    m += quad_xor1(m);
    m += quad_xor2(m);
    if (q != 0) return;
    uint32_t h = (nstripe > 0 ? m : kP5) + rg.len;
    const uint8_t* p = base + 16ull * nstripe;
    uint32_t rest = rg.len & 15u;
    for (; rest >= 4; rest -= 4, p += 4) h = rotl32(h + *reinterpret_cast<const uint32_t*>(p) * kP3, 17) * kP4;
    for (; rest > 0; --rest, ++p) h = rotl32(h + (uint32_t)*p * kP5, 11) * kP1;
    h ^= h >> 15;
    h *= kP2;
    h ^= h >> 13;
    h *= kP3;
    h ^= h >> 16;
    out[rg.slot] = h;
}

}  // namespace

hipError_t xxh32_launch(const uint8_t* data, const HashRange* ranges, int n, uint32_t* out, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const int blocks = (int)(((long)n * 4 + kHashThreads - 1) / kHashThreads);
    hipLaunchKernelGGL(k_xxh32, dim3(blocks), dim3(kHashThreads), 0, st, data, ranges, n, out);
    return hipGetLastError();
}

}  // namespace nx
