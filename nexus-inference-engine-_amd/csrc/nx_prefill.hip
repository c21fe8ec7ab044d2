// Batched prefill of a prompt: the reference runs a prompt one token at a
// time through the decode layers (HybridModel::prefill,
// nexus/src/model/hybrid_model.cpp:604-644); here a chunk of P prompt tokens
// goes through each layer at once, so every projection is a GEMM
// [P x K] x [K x N] on the matrix cores instead of P weight-streaming GEMVs.
//
// k_pf_gemm: Y = X W^T with X fp16 [M][ldx] (tokens) and W int4-g32 (codes
// [N][G*16], fp16 scales [N][G]).  A block computes 128 tokens x 64 weight
// rows; its four wavefronts take 64 x 32 each as 4 x 2 tiles of
// v_mfma_f32_16x16x32_f16 (A = X: row = token; B = W: column = weight row;
// one 32-k group per product).  Per stage of four groups the block stages X
// in LDS in the k order (0 2 4 6 1 3 5 7) of each 8-k chunk -- the order in
// which a code dword turns into fp16 with two byte permutes -- and the codes
// and scales of its 64 rows; the next stage's loads are in flight while the
// current one is multiplied.
// Exact scaling without per-group fp32 work: the group's fp16 scale s is
// split into s_hi (its 7 leading significant bits) and s_lo = s - s_hi (the
// 4 trailing bits), so (q - 8) s_hi and (q - 8) s_lo 2^10 are both exact in
// fp16 (4-bit x 7-bit and 4-bit x 4-bit products).  They go to two
// accumulators, combined once at the end as hi + lo 2^-10: the products are
// exactly (q - 8) s x, summed in fp32 -- the numerics of the decode GEMV at
// two matrix-core products per group and no vector work per output.
// Epilogues: fp32 store, fp32 accumulate (residual), SwiGLU of interleaved
// gate/up rows to fp16.
#include "nx_common.h"
#include "nx_kernels.h"

namespace nx {
namespace {

typedef _Float16 ph8_t __attribute__((ext_vector_type(8)));
typedef float pf4_t __attribute__((ext_vector_type(4)));

constexpr int kPfBM = 128, kPfThreads = 256;
constexpr int kPfXcds = 8;  // blocks are dealt to the XCDs round-robin by block index
// Tile shapes: BN weight rows x BM tokens per block, BK k per stage; the
// four wavefronts form WM x (4 / WM) sub-tiles.  When 128 x 128 tiles give
// at least kPfWideTiles blocks (two per CU), each wavefront takes 32 rows and
// all 128 tokens, so it dequantizes each weight fragment once for 8 token
// fragments; smaller products keep 64-row tiles (2 x 2 wavefronts) for
// enough blocks.
constexpr long kPfWideTiles = 512;

// Code dword (8 nibbles, low nibble = even k) -> fp16 (q - 8) in the k order
// (0 2 4 6 1 3 5 7): each nibble byte joined with 0x64 is the fp16 1024 + q.
__device__ inline ph8_t pf_codes_to_h8(uint32_t w) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu, k64 = 0x64646464u;
    const uint4 r = make_uint4(__builtin_amdgcn_perm(k64, lo, 0x04010400u), __builtin_amdgcn_perm(k64, lo, 0x04030402u),
                               __builtin_amdgcn_perm(k64, hi, 0x04010400u), __builtin_amdgcn_perm(k64, hi, 0x04030402u));
    return __builtin_bit_cast(ph8_t, r) - (_Float16)1032.0f;
}

// Eight fp16 of consecutive k (4 dwords) into the k order (0 2 4 6 1 3 5 7).
__device__ inline uint4 pf_perm_x8(uint4 x) {
    return make_uint4(__builtin_amdgcn_perm(x.y, x.x, 0x05040100u), __builtin_amdgcn_perm(x.w, x.z, 0x05040100u),
                      __builtin_amdgcn_perm(x.y, x.x, 0x07060302u), __builtin_amdgcn_perm(x.w, x.z, 0x07060302u));
}

__device__ inline float lane_xor1(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
}

template <int EPI, int kPfBN, int kPfBK, int WM>
__global__ __launch_bounds__(kPfThreads, 2) void k_pf_gemm(PfGemmArgs a) {
    constexpr int kPfGPS = kPfBK / 32;     // groups per stage
    constexpr int kPfAStride = kPfBK + 8;  // fp16 per LDS row of X: rows 4 banks apart, 16 rows read conflict-free
    constexpr int kPfAChunks = kPfBM * kPfBK / 8 / kPfThreads;  // 16-byte chunks of X per thread per stage
    constexpr int WN = 4 / WM, RM = kPfBM / WM, RN = kPfBN / WN, NI = RM / 16, NJ = RN / 16;
    static_assert(kPfBN * kPfGPS <= kPfThreads, "one code group and one scale per thread");
    static_assert(WM * WN == 4 && NI * 16 == RM && NJ * 16 == RN, "wavefront sub-tiles");
    __shared__ __align__(16) uint16_t As[2][kPfBM * kPfAStride];
    __shared__ __align__(16) uint32_t Bs[2][kPfBN * kPfGPS * 4];  // [row][group][4 dwords]
    __shared__ uint16_t Ss[2][kPfBN * kPfGPS];                    // [row][group]
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 15, kq = lane >> 4;
    // XCD-aware tile order: the blocks of XCD x (block index % 8 == x) take
    // the column tiles [x nt / 8, (x + 1) nt / 8), all of one row tile before
    // the next, so an X row tile is fetched into that XCD's L2 once and
    // shared by the XCD's concurrent blocks
    const int ntn = (a.N + kPfBN - 1) / kPfBN, ntm = (a.M + kPfBM - 1) / kPfBM;
    const int xcd = (int)(blockIdx.x % kPfXcds), local = (int)(blockIdx.x / kPfXcds);
    const int nb0 = xcd * ntn / kPfXcds, nn = (xcd + 1) * ntn / kPfXcds - nb0;
    if (nn <= 0 || local >= nn * ntm) return;  // the block count is rounded up to 8 x the largest share
    const int n0 = (nb0 + local % nn) * kPfBN, m0 = (local / nn) * kPfBM;
    const int wm = wave % WM, wn = wave / WM;
    const int M = a.M, N = a.N, K = a.K, G = a.G;
    const int nstage = (G + kPfGPS - 1) / kPfGPS;

    // global -> registers for stage s; every address is clamped into its
    // tensor and out-of-range values are zeroed after the load
    constexpr int CPR = kPfBK / 8;  // 16-byte chunks per row of the X tile
    uint4 ra[kPfAChunks], rb = make_uint4(0, 0, 0, 0);
    uint16_t rs = 0;
    auto load = [&](int s) {
        const int kb = s * kPfBK;
#pragma unroll
        for (int j = 0; j < kPfAChunks; ++j) {
            const int ch = tid + kPfThreads * j, row = ch / CPR, k = kb + 8 * (ch % CPR);
            const int m = min(m0 + row, M - 1);
            const uint4 v = *reinterpret_cast<const uint4*>(a.x + (size_t)m * a.ldx + min(k, K - 8));
            const bool ok = k < K && m0 + row < M;
            ra[j] = ok ? v : make_uint4(0, 0, 0, 0);
        }
        if (tid < kPfBN * kPfGPS) {
            const int n = min(n0 + tid / kPfGPS, N - 1), g = min(kPfGPS * s + tid % kPfGPS, G - 1);
            rb = *reinterpret_cast<const uint4*>(a.W + ((size_t)n * G + g) * 16);
            rs = a.S[(size_t)n * G + g];
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int j = 0; j < kPfAChunks; ++j) {
            const int ch = tid + kPfThreads * j, row = ch / CPR;
            *reinterpret_cast<uint4*>(&As[buf][row * kPfAStride + 8 * (ch % CPR)]) = pf_perm_x8(ra[j]);
        }
        if (tid < kPfBN * kPfGPS) {
            *reinterpret_cast<uint4*>(&Bs[buf][tid * 4]) = rb;  // row tid / GPS, group tid % GPS
            Ss[buf][tid] = rs;
        }
    };

    pf4_t acc[NI][NJ], acl[NI][NJ];  // (q - 8) s_hi x and (q - 8) s_lo 2^10 x
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = acl[i][j] = pf4_t{0.f, 0.f, 0.f, 0.f};

    load(0);
    store(0);
    __syncthreads();
    for (int s = 0; s < nstage; ++s) {
        const int buf = s & 1;
        if (s + 1 < nstage) load(s + 1);
#pragma unroll
        for (int g = 0; g < kPfGPS; ++g) {
            ph8_t af[NI];
#pragma unroll
            for (int i = 0; i < NI; ++i)
                af[i] = __builtin_bit_cast(
                    ph8_t, *reinterpret_cast<const uint4*>(&As[buf][(RM * wm + 16 * i + c) * kPfAStride + 32 * g + 8 * kq]));
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int row = RN * wn + 16 * j + c;
                const ph8_t w = pf_codes_to_h8(Bs[buf][(row * kPfGPS + g) * 4 + kq]);
                const uint16_t sb = Ss[buf][row * kPfGPS + g];
                const _Float16 shi = __builtin_bit_cast(_Float16, (uint16_t)(sb & 0xFFF0u));
                const _Float16 slo = (__builtin_bit_cast(_Float16, sb) - shi) * (_Float16)1024.0f;
                const ph8_t wh = w * shi, wl = w * slo;
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], wh, acc[i][j], 0, 0, 0);
                    acl[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], wl, acl[i][j], 0, 0, 0);
                }
            }
        }
        if (s + 1 < nstage) store(buf ^ 1);
        __syncthreads();
    }

    // tile (i, j): lane (c, kq) holds weight row n0 + RN wn + 16 j + c for
    // tokens m0 + RM wm + 16 i + 4 kq + r, r < 4
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int n = n0 + RN * wn + 16 * j + c;
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + RM * wm + 16 * i + 4 * kq + r;
                const float v = fmaf(acl[i][j][r], 0.0009765625f, acc[i][j][r]);
                if (EPI == PF_SWIGLU) {
                    const float u = lane_xor1(v);  // the up row n + 1 sits in lane c + 1
                    if ((c & 1) == 0 && m < M && n + 1 < N)
                        // hardware exp and reciprocal (a few ulp in fp32, below the fp16
                        // rounding of the stored activation)
                        a.act16[(size_t)m * a.lda + (n >> 1)] =
                            f2h_bits(v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)) * u);
                } else if (m < M && n < N) {
                    float* y = a.y32 + (size_t)m * a.ldy + n;
                    *y = EPI == PF_ACC ? *y + v : v;
                }
            }
    }
}

__global__ __launch_bounds__(256) void k_pf_embed(const int32_t* tokens, const uint16_t* embed, float* h, int d,
                                                  int vocab) {
    int tok = tokens[blockIdx.x];
    if (tok < 0 || tok >= vocab) tok = 0;  // the host checked the prompt; never index outside the table
    const uint16_t* src = embed + (size_t)tok * d;
    float* dst = h + (size_t)blockIdx.x * d;
    for (int i = threadIdx.x; i < d; i += 256) dst[i] = h2f_bits(src[i]);
}

// RoPE of the q and k rows of token t at position p0 + t (the rotation of
// the decode QKV epilogue), q to q32 [P][qdim], k and v (fp16, RNE) into
// the pages of the sequence (block table row bt).
// kvrows != nullptr (TurboQuant pages): K and V rows go there as fp32
// [P][2][kvdim] for the encoder instead of into fp16 pages.
__global__ __launch_bounds__(256) void k_pf_rope_kv(const float* qkv, int ld, int P, int p0, int qdim, int kvdim,
                                                    int hd, int hkv, const float* cos_t, const float* sin_t,
                                                    const int32_t* bt, uint16_t* kpool, uint16_t* vpool, float* q32,
                                                    float* kvrows) {
    const int npair = (qdim + 2 * kvdim) / 2;
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long)P * npair) return;
    const int t = (int)(idx / npair), row = 2 * (int)(idx % npair), p = p0 + t, half = hd >> 1;
    float v0 = qkv[(size_t)t * ld + row], v1 = qkv[(size_t)t * ld + row + 1];
    if (row < qdim + kvdim) {
        const int i = (row % hd) >> 1;
        const float c = cos_t[(size_t)p * half + i], s = sin_t[(size_t)p * half + i];
        const float r0 = v0 * c - v1 * s;
        const float r1 = v0 * s + v1 * c;
        v0 = r0;
        v1 = r1;
    }
    if (row < qdim) {
        q32[(size_t)t * qdim + row] = v0;
        q32[(size_t)t * qdim + row + 1] = v1;
        return;
    }
    const int kv = row < qdim + kvdim ? 0 : 1, j = row - qdim - kv * kvdim, kvh = j / hd, dd = j % hd;
    if (kvrows) {
        kvrows[((size_t)t * 2 + kv) * kvdim + j] = v0;
        kvrows[((size_t)t * 2 + kv) * kvdim + j + 1] = v1;
        return;
    }
    const size_t page = ((size_t)bt[p / kPage] * hkv + kvh) * kPage * hd;
    if (kv) {  // V pages are dimension-major [hd][16]
        vpool[page + (size_t)dd * kPage + p % kPage] = f2h_bits(v0);
        vpool[page + (size_t)(dd + 1) * kPage + p % kPage] = f2h_bits(v1);
    } else {   // K pages are token-major [16][hd]
        kpool[page + (size_t)(p % kPage) * hd + dd] = f2h_bits(v0);
        kpool[page + (size_t)(p % kPage) * hd + dd + 1] = f2h_bits(v1);
    }
}

}  // namespace

hipError_t pf_gemm_launch(int epi, const PfGemmArgs& a, hipStream_t st) {
    // 16-byte rows of x (K and ldx multiples of 8, aligned base), at least one
    // full 8-k chunk
    if (a.M < 1 || a.N < 1 || a.K < 8 || a.K % 8 || a.ldx % 8 || (reinterpret_cast<uintptr_t>(a.x) & 15) ||
        a.G != (a.K + 31) / 32 || (epi == PF_SWIGLU && a.N % 2))
        return hipErrorInvalidValue;
    const bool wide = (long)((a.N + 127) / 128) * ((a.M + kPfBM - 1) / kPfBM) >= kPfWideTiles;
    const long BN = wide ? 128 : 64;
    const long ntn = (a.N + BN - 1) / BN, ntm = (a.M + kPfBM - 1) / kPfBM;
    const long share = (ntn + kPfXcds - 1) / kPfXcds;  // largest column-tile share of an XCD
    const long blocks = (long)kPfXcds * share * ntm;
    if (blocks > 0x7FFFFFFFL) return hipErrorInvalidValue;
    const dim3 grid((unsigned)blocks);
#define NX_PF_CASE(E)                                                                                   \
    case E:                                                                                             \
        if (wide)                                                                                       \
            hipLaunchKernelGGL((k_pf_gemm<E, 128, 64, 1>), grid, dim3(kPfThreads), 0, st, a);          \
        else                                                                                            \
            hipLaunchKernelGGL((k_pf_gemm<E, 64, 128, 2>), grid, dim3(kPfThreads), 0, st, a);          \
        break;
    switch (epi) {
        NX_PF_CASE(PF_F32)
        NX_PF_CASE(PF_ACC)
        NX_PF_CASE(PF_SWIGLU)
        default: return hipErrorInvalidValue;
    }
#undef NX_PF_CASE
    return hipGetLastError();
}

hipError_t pf_embed_launch(const int32_t* tokens, int P, const uint16_t* embed, float* h, int d, int vocab,
                           hipStream_t st) {
    hipLaunchKernelGGL(k_pf_embed, dim3(P), dim3(256), 0, st, tokens, embed, h, d, vocab);
    return hipGetLastError();
}

hipError_t pf_rope_kv_launch(const float* qkv, int ld, int P, int p0, int qdim, int kvdim, int hd, int hkv,
                             const float* cos_t, const float* sin_t, const int32_t* bt, uint16_t* kpool,
                             uint16_t* vpool, float* q32, hipStream_t st, float* kvrows) {
    const long n = (long)P * ((qdim + 2 * kvdim) / 2);
    hipLaunchKernelGGL(k_pf_rope_kv, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, qkv, ld, P, p0, qdim, kvdim,
                       hd, hkv, cos_t, sin_t, bt, kpool, vpool, q32, kvrows);
    return hipGetLastError();
}

}  // namespace nx
