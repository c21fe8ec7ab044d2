// fp32 GEMM C[M][N] = A[M][K] B[K][N] (row-major) on the matrix cores:
// the dense-weight path of the runner (compute::gemm_f32 / ComputeDispatch::
// gemm, compute_dispatch.h:42; called for non-int4 weights at
// hybrid_model.cpp:121).
//
// A block of 4 wavefronts computes a 64 x 64 tile of C; wavefront w owns the
// 32 x 32 quarter (w / 2, w % 2) as 2 x 2 tiles of v_mfma_f32_16x16x4f32:
//   A (16 x 4): lane l holds row l%16, k = l/16
//   B (4 x 16): lane l holds column l%16, k = l/16
//   C (16 x 16): lane l holds column l%16, rows 4(l/16) .. +3
// K advances in steps of 16 through LDS tiles of A (64 x 16) and B (16 x 64),
// each thread loading 4 + 4 elements (zero past the matrix edges).  Products
// and sums are fp32.
#include "nx_common.h"
#include "nx_kernels.h"

namespace nx {

namespace {

constexpr int kGT = 64;   // C tile edge per block
constexpr int kGK = 16;   // K per LDS stage
typedef float gf4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_gemm_f32(const float* __restrict__ A, const float* __restrict__ B,
                                                  float* __restrict__ C, int M, int N, int K) {
    __shared__ float As[kGT][kGK + 1];
    __shared__ float Bs[kGK][kGT + 4];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m0 = blockIdx.y * kGT, n0 = blockIdx.x * kGT;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    gf4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = gf4{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < K; k0 += kGK) {
        // A tile: 64 rows x 16 k; thread t loads row t / 4, k (t % 4) * 4 .. +3
        {
            const int r = tid >> 2, c = (tid & 3) * 4;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int gm = m0 + r, gk = k0 + c + e;
                As[r][c + e] = (gm < M && gk < K) ? A[(size_t)gm * K + gk] : 0.0f;
            }
        }
        // B tile: 16 k x 64 columns; thread t loads k t / 16, columns (t % 16) * 4 .. +3
        {
            const int r = tid >> 4, c = (tid & 15) * 4;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int gk = k0 + r, gn = n0 + c + e;
                Bs[r][c + e] = (gk < K && gn < N) ? B[(size_t)gk * N + gn] : 0.0f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kGK; kk += 4) {
            const int ka = kk + (lane >> 4);
            float a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) a[i] = As[wm + 16 * i + (lane & 15)][ka];
#pragma unroll
            for (int j = 0; j < 2; ++j) b[j] = Bs[ka][wn + 16 * j + (lane & 15)];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn + 16 * j + (lane & 15);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = m0 + wm + 16 * i + 4 * (lane >> 4) + e;
                if (row < M && col < N) C[(size_t)row * N + col] = acc[i][j][e];
            }
        }
}

}  // namespace

hipError_t gemm_f32_launch(const float* A, const float* B, float* C, int M, int N, int K, hipStream_t st) {
    if (M <= 0 || N <= 0 || K <= 0) return hipErrorInvalidValue;
    const dim3 grid((N + kGT - 1) / kGT, (M + kGT - 1) / kGT);
    hipLaunchKernelGGL(k_gemm_f32, grid, dim3(256), 0, st, A, B, C, M, N, K);
    return hipGetLastError();
}

}  // namespace nx
