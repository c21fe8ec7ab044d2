// C-ABI of the decode-loop library: context, buffer registry, weight cache,
// token-level HIP graphs and the validated op entry points.  Every entry
// point checks its buffers and shapes on the host before enqueueing a
// kernel, and reports errors as status codes (never zero-filled outputs).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <random>

#include "nx_common.h"
#include "nx_internal.h"
#include "nx_kernels.h"

using nx::fail;

namespace {
thread_local std::string g_init_error;

bool device_is_gfx950(int dev) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) return false;
    return std::strncmp(p.gcnArchName, "gfx950", 6) == 0;
}

nx_status ensure_attn_ws(nx_ctx* ctx, size_t bytes) {
    if (bytes <= ctx->attn_ws_bytes) return NX_OK;
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "attention workspace must grow outside capture");
    NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->attn_ws) (void)hipFree(ctx->attn_ws);
    ctx->attn_ws = nullptr;
    ctx->attn_ws_bytes = 0;
    NX_HIP(ctx, hipMalloc(&ctx->attn_ws, bytes));
    ctx->attn_ws_bytes = bytes;
    return NX_OK;
}

// Split-completion counters of the fp16 attention: zeroed when allocated,
// and every launch leaves them at zero.
nx_status ensure_attn_counts(nx_ctx* ctx, size_t words) {
    if (words <= ctx->attn_count_words) return NX_OK;
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "attention counters must grow outside capture");
    NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->attn_counts) (void)hipFree(ctx->attn_counts);
    ctx->attn_counts = nullptr;
    ctx->attn_count_words = 0;
    NX_HIP(ctx, hipMalloc(reinterpret_cast<void**>(&ctx->attn_counts), words * sizeof(unsigned)));
    NX_HIP(ctx, hipMemsetAsync(ctx->attn_counts, 0, words * sizeof(unsigned), ctx->stream));
    ctx->attn_count_words = words;
    return NX_OK;
}

template <class T>
T* dptr(nx_buf b) {
    return reinterpret_cast<T*>(static_cast<uintptr_t>(b));
}

nx_status launched(nx_ctx* ctx, hipError_t e, const char* what) {
    if (e != hipSuccess) return nx::hip_fail(ctx, e, what);
    return NX_OK;
}
nx_status ensure_smp_ws(nx_ctx* ctx, size_t floats);
}  // namespace

// ------------------------------------------------------------------ draw --
namespace nx {
// First output of MT19937 seeded with `seed` (the generator and seeding of
// std::mt19937), as libstdc++'s uniform_real_distribution<float>(0, 1)
// turns it into a float: x / 2^32 in float, 1 replaced by the largest float
// below 1.  The reference draws from a fresh std::mt19937(seed) at every
// sample_token call (hybrid_model.cpp:2089-2091); seed 0 means
// std::random_device there and here.
float sample_draw(uint64_t seed) {
    uint32_t s32 = (uint32_t)seed;
    if (seed == 0) s32 = std::random_device{}();
    uint32_t mt[624];
    mt[0] = s32;
    for (uint32_t i = 1; i < 624; ++i) mt[i] = 1812433253u * (mt[i - 1] ^ (mt[i - 1] >> 30)) + i;
    // the first output only needs the first twist step
    const uint32_t y0 = (mt[0] & 0x80000000u) | (mt[1] & 0x7FFFFFFFu);
    uint32_t y = mt[397] ^ (y0 >> 1) ^ ((y0 & 1u) ? 0x9908B0DFu : 0u);
    y ^= y >> 11;
    y ^= (y << 7) & 0x9D2C5680u;
    y ^= (y << 15) & 0xEFC60000u;
    y ^= y >> 18;
    const float r = (float)y / 4294967296.0f;
    return r >= 1.0f ? std::nextafter(1.0f, 0.0f) : r;
}
}  // namespace nx

// ---------------------------------------------------------------- codebook --
namespace nx {
static float cb_normal_pdf(float x, float sigma) {
    const float z = x / sigma;
    return std::exp(-0.5f * z * z) / (sigma * std::sqrt(2.0f * static_cast<float>(M_PI)));
}
static float cb_normal_cdf(float x, float sigma) {
    const float z = x / sigma;
    return 0.5f * std::erfc(-z * static_cast<float>(M_SQRT1_2));
}
static float cb_conditional_mean(float a, float b, float sigma) {
    const float pa = cb_normal_pdf(a, sigma), pb = cb_normal_pdf(b, sigma);
    const float ca = cb_normal_cdf(a, sigma), cb = cb_normal_cdf(b, sigma);
    const float denom = cb - ca;
    if (denom < 1e-12f) return 0.5f * (a + b);
    return sigma * sigma * (pa - pb) / denom;
}
void tq_codebook(int d, int bits, float* c, float* bnd) {
    const int n = 1 << bits;
    const float sigma = 1.0f / std::sqrt(static_cast<float>(d));
    const float lo = -3.0f * sigma, hi = 3.0f * sigma;
    for (int i = 0; i < n; ++i) c[i] = lo + (hi - lo) * (i + 0.5f) / n;
    for (int iter = 0; iter < 100; ++iter) {
        for (int i = 0; i < n - 1; ++i) bnd[i] = 0.5f * (c[i] + c[i + 1]);
        float max_delta = 0.0f;
        for (int i = 0; i < n; ++i) {
            const float a = (i == 0) ? -10.0f * sigma : bnd[i - 1];
            const float b = (i == n - 1) ? 10.0f * sigma : bnd[i];
            const float nc = cb_conditional_mean(a, b, sigma);
            const float delta = std::fabs(nc - c[i]);
            if (delta > max_delta) max_delta = delta;
            c[i] = nc;
        }
        if (max_delta < 1e-7f * sigma) break;
    }
    for (int i = 0; i < n - 1; ++i) bnd[i] = 0.5f * (c[i] + c[i + 1]);
}
}  // namespace nx

extern "C" {

// ---------------------------------------------------------------- lifecycle --
int nx_has_gpu(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    for (int i = 0; i < n; ++i)
        if (device_is_gfx950(i)) return 1;
    return 0;
}

const char* nx_init_error(void) { return g_init_error.c_str(); }

nx_status nx_init(nx_ctx** out, int device) {
    if (!out) return NX_ERR_INVALID;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) {
        g_init_error = "no HIP device " + std::to_string(device);
        return NX_ERR_NO_DEVICE;
    }
    if (!device_is_gfx950(device)) {
        g_init_error = "device is not gfx950";
        return NX_ERR_NO_DEVICE;
    }
    if (hipSetDevice(device) != hipSuccess) {
        g_init_error = "hipSetDevice failed";
        return NX_ERR_HIP;
    }
    nx_ctx* ctx = new nx_ctx();
    ctx->device = device;
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&ctx->ev0) != hipSuccess || hipEventCreate(&ctx->ev1) != hipSuccess) {
        g_init_error = "stream/event creation failed";
        delete ctx;
        return NX_ERR_HIP;
    }
    // the no-allocation attention's scratch: its address on this device
    // (hipSetDevice above made it current)
    if (nx::attn_noalloc_scratch(&ctx->na_scratch) != hipSuccess || !ctx->na_scratch) {
        g_init_error = "hipGetSymbolAddress of the attention scratch failed";
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return NX_ERR_HIP;
    }
    nx::tq_codebook(128, 4, ctx->c4, ctx->b4);
    nx::tq_codebook(128, 3, ctx->c3, ctx->b3);
    nx::tq_set_codebooks(ctx->c4, ctx->b4, ctx->c3, ctx->b3);
    if (hipDeviceSynchronize() != hipSuccess) {
        g_init_error = "device synchronize failed";
        delete ctx;
        return NX_ERR_HIP;
    }
    *out = ctx;
    return NX_OK;
}

nx_status nx_destroy(nx_ctx* ctx) {
    if (!ctx) return NX_ERR_INVALID;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->token_exec) (void)hipGraphExecDestroy(ctx->token_exec);
    for (hipGraphExec_t e : ctx->seg_exec)
        if (e) (void)hipGraphExecDestroy(e);
    if (ctx->ffn_ws) (void)hipFree(ctx->ffn_ws);
    for (auto& kv : ctx->bufs) (void)hipFree(reinterpret_cast<void*>(kv.first));
    if (ctx->attn_ws) (void)hipFree(ctx->attn_ws);
    if (ctx->attn_counts) (void)hipFree(ctx->attn_counts);
    if (ctx->smp_ws) (void)hipFree(ctx->smp_ws);
    if (ctx->gemv_ws) (void)hipFree(ctx->gemv_ws);
    (void)hipEventDestroy(ctx->ev0);
    (void)hipEventDestroy(ctx->ev1);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return NX_OK;
}

nx_status nx_device_name(nx_ctx* ctx, char* buf, size_t n) {
    if (!ctx || !buf || n == 0) return NX_ERR_INVALID;
    hipDeviceProp_t p;
    NX_HIP(ctx, hipGetDeviceProperties(&p, ctx->device));
    std::snprintf(buf, n, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    return NX_OK;
}

const char* nx_last_error(nx_ctx* ctx) { return ctx ? ctx->err.c_str() : "null context"; }

// ------------------------------------------------------------------- memory --
nx_status nx_alloc(nx_ctx* ctx, size_t bytes, nx_buf* out) {
    if (!ctx || !out) return NX_ERR_INVALID;
    if (bytes == 0) return fail(ctx, NX_ERR_INVALID, "nx_alloc: zero bytes");
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "nx_alloc inside a token batch");
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return nx::hip_fail(ctx, e, "hipMalloc");
    e = hipMemsetAsync(p, 0, bytes, ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(p);
        return nx::hip_fail(ctx, e, "hipMemsetAsync");
    }
    ctx->bufs[reinterpret_cast<uint64_t>(p)] = bytes;
    *out = reinterpret_cast<uint64_t>(p);
    return NX_OK;
}

nx_status nx_free(nx_ctx* ctx, nx_buf b) {
    if (!ctx) return NX_ERR_INVALID;
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "nx_free inside a token batch");
    auto it = ctx->bufs.find(b);
    if (it == ctx->bufs.end()) return fail(ctx, NX_ERR_INVALID, "nx_free: unknown buffer");
    NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    NX_HIP(ctx, hipFree(reinterpret_cast<void*>(b)));
    ctx->bufs.erase(it);
    for (auto w = ctx->wcache.begin(); w != ctx->wcache.end();)
        w = (w->second == b) ? ctx->wcache.erase(w) : std::next(w);
    return NX_OK;
}

nx_status nx_buffer_size(nx_ctx* ctx, nx_buf b, size_t* bytes) {
    if (!ctx || !bytes) return NX_ERR_INVALID;
    *bytes = nx::buf_size(ctx, b);
    return *bytes ? NX_OK : fail(ctx, NX_ERR_INVALID, "unknown buffer");
}

nx_status nx_upload(nx_ctx* ctx, nx_buf dst, size_t off, const void* src, size_t bytes) {
    if (!ctx || (!src && bytes)) return NX_ERR_INVALID;
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "nx_upload inside a token batch");
    NX_NEED(ctx, dst, off + bytes, "nx_upload dst");
    if (bytes == 0) return NX_OK;
    NX_HIP(ctx, hipMemcpyAsync(dptr<char>(dst) + off, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return NX_OK;
}

nx_status nx_download(nx_ctx* ctx, void* dst, nx_buf src, size_t off, size_t bytes) {
    if (!ctx || (!dst && bytes)) return NX_ERR_INVALID;
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "nx_download inside a token batch");
    NX_NEED(ctx, src, off + bytes, "nx_download src");
    if (bytes == 0) return NX_OK;
    NX_HIP(ctx, hipMemcpyAsync(dst, dptr<char>(src) + off, bytes, hipMemcpyDeviceToHost, ctx->stream));
    NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return NX_OK;
}

nx_status nx_weight_cache(nx_ctx* ctx, const void* key, const void* src, size_t bytes, nx_buf* out) {
    if (!ctx || !key || !out) return NX_ERR_INVALID;
    auto it = ctx->wcache.find(key);
    if (it != ctx->wcache.end()) {
        if (nx::buf_size(ctx, it->second) < bytes)
            return fail(ctx, NX_ERR_INVALID, "nx_weight_cache: cached buffer smaller than request");
        *out = it->second;
        return NX_OK;
    }
    nx_buf b = 0;
    nx_status s = nx_alloc(ctx, bytes, &b);
    if (s != NX_OK) return s;
    s = nx_upload(ctx, b, 0, src, bytes);
    if (s != NX_OK) {
        (void)nx_free(ctx, b);
        return s;
    }
    ctx->wcache[key] = b;
    *out = b;
    return NX_OK;
}

nx_status nx_get_cached_buffer(nx_ctx* ctx, const void* key, nx_buf* out) {
    if (!ctx || !out) return NX_ERR_INVALID;
    auto it = ctx->wcache.find(key);
    if (it == ctx->wcache.end()) return fail(ctx, NX_ERR_INVALID, "no cached buffer for key");
    *out = it->second;
    return NX_OK;
}

nx_status nx_clear_buffer_cache(nx_ctx* ctx) {
    if (!ctx) return NX_ERR_INVALID;
    std::vector<nx_buf> bs;
    for (auto& kv : ctx->wcache) bs.push_back(kv.second);
    ctx->wcache.clear();
    for (nx_buf b : bs) {
        nx_status s = nx_free(ctx, b);
        if (s != NX_OK) return s;
    }
    return NX_OK;
}

nx_status nx_synchronize(nx_ctx* ctx) {
    if (!ctx) return NX_ERR_INVALID;
    NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return NX_OK;
}

// ----------------------------------------------------------------- batching --
nx_status nx_token_begin(nx_ctx* ctx) {
    if (!ctx) return NX_ERR_INVALID;
    if (ctx->capturing || ctx->token_flushed) return fail(ctx, NX_ERR_STATE, "token batch already open");
    NX_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
    ctx->token_seg = 0;
    return NX_OK;
}

// End the capture of the current segment of the token batch, launch its
// graph and wait.  Segment s keeps its own instantiated graph, updated in
// place while the captured sequence keeps its shape.
static nx_status run_segment(nx_ctx* ctx) {
    ctx->capturing = false;
    hipGraph_t g = nullptr;
    NX_HIP(ctx, hipStreamEndCapture(ctx->stream, &g));
    const int seg = ctx->token_seg;
    if (seg > 0 && (int)ctx->seg_exec.size() < seg) ctx->seg_exec.resize(seg, nullptr);
    hipGraphExec_t& ex = seg == 0 ? ctx->token_exec : ctx->seg_exec[seg - 1];
    bool ok = false;
    if (ex) {
        hipGraphNode_t err_node = nullptr;
        hipGraphExecUpdateResult res;
        if (hipGraphExecUpdate(ex, g, &err_node, &res) == hipSuccess && res == hipGraphExecUpdateSuccess)
            ok = true;
        else {
            (void)hipGetLastError();
            (void)hipGraphExecDestroy(ex);
            ex = nullptr;
        }
    }
    if (!ok) {
        hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            (void)hipGraphDestroy(g);
            ex = nullptr;
            return nx::hip_fail(ctx, e, "hipGraphInstantiate");
        }
    }
    (void)hipGraphDestroy(g);
    NX_HIP(ctx, hipGraphLaunch(ex, ctx->stream));
    NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return NX_OK;
}

nx_status nx_token_end(nx_ctx* ctx) {
    if (!ctx) return NX_ERR_INVALID;
    if (ctx->token_flushed) {  // flushed and not resumed: nothing is pending
        ctx->token_flushed = false;
        return NX_OK;
    }
    if (!ctx->capturing) return fail(ctx, NX_ERR_STATE, "nx_token_end without nx_token_begin");
    return run_segment(ctx);
}

nx_status nx_token_flush(nx_ctx* ctx) {
    if (!ctx) return NX_ERR_INVALID;
    if (ctx->token_flushed) return NX_OK;  // already flushed (as the reference: a no-op)
    if (!ctx->capturing) return fail(ctx, NX_ERR_STATE, "nx_token_flush outside a token batch");
    nx_status s = run_segment(ctx);
    if (s != NX_OK) return s;
    ctx->token_flushed = true;
    return NX_OK;
}

nx_status nx_token_resume(nx_ctx* ctx) {
    if (!ctx) return NX_ERR_INVALID;
    if (ctx->capturing) return NX_OK;  // not flushed: batching continues (a no-op)
    if (!ctx->token_flushed) return fail(ctx, NX_ERR_STATE, "nx_token_resume outside a token batch");
    NX_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->token_flushed = false;
    ctx->capturing = true;
    ++ctx->token_seg;
    return NX_OK;
}

// ---------------------------------------------------------------------- ops --
// The K-part workspace of a batched GEMV (nx::gemv_kparts), grown outside
// capture; under capture without room it stays null and the GEMV runs in
// one launch.
static nx_status gemv_kpart_ws(nx_ctx* ctx, int N, int K, int batch, float** out) {
    *out = nullptr;
    const int kp = nx::gemv_kparts(K, batch);
    if (kp == 0) return NX_OK;
    const size_t need = (size_t)kp * batch * N;
    if (need > ctx->gemv_ws_floats) {
        if (ctx->capturing) return NX_OK;
        NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (ctx->gemv_ws) (void)hipFree(ctx->gemv_ws);
        ctx->gemv_ws = nullptr;
        ctx->gemv_ws_floats = 0;
        NX_HIP(ctx, hipMalloc(reinterpret_cast<void**>(&ctx->gemv_ws), need * sizeof(float)));
        ctx->gemv_ws_floats = need;
    }
    *out = ctx->gemv_ws;
    return NX_OK;
}

static nx_status gemv_common(nx_ctx* ctx, nx_buf x, nx_buf wq, nx_buf sc, nx_buf y, int N, int K,
                             int batch, int out_bytes, const char* name, nx::GemvArgs& a) {
    if (!ctx) return NX_ERR_INVALID;
    if (N <= 0 || K <= 0 || batch < 1 || batch > 8)
        return fail(ctx, NX_ERR_INVALID, "%s: bad shape N=%d K=%d batch=%d", name, N, K, batch);
    const int G = (K + 31) / 32;
    if (G > 14 * 64) return fail(ctx, NX_ERR_UNSUPPORTED, "%s: K=%d above 28672", name, K);
    NX_NEED(ctx, x, (size_t)batch * K * 2, "x");
    NX_NEED(ctx, wq, (size_t)N * G * 16, "weights");
    NX_NEED(ctx, sc, (size_t)N * G * 2, "scales");
    NX_NEED(ctx, y, (size_t)batch * N * out_bytes, "y");
    a = nx::GemvArgs{};
    a.W = dptr<const uint8_t>(wq);
    a.S = dptr<const uint16_t>(sc);
    a.N = N;
    a.K = K;
    a.G = G;
    a.batch = batch;
    a.x16 = dptr<const uint16_t>(x);
    a.ldx = K;
    a.ldy = N;
    return gemv_kpart_ws(ctx, N, K, batch, &a.kpart);
}

nx_status nx_gemv_int4_g32(nx_ctx* ctx, nx_buf x, nx_buf wq, nx_buf sc, nx_buf y, int N, int K,
                           int batch) {
    nx::GemvArgs a;
    nx_status s = gemv_common(ctx, x, wq, sc, y, N, K, batch, 2, "nx_gemv_int4_g32", a);
    if (s != NX_OK) return s;
    a.y16 = dptr<uint16_t>(y);
    return launched(ctx, nx::gemv_launch(nx::X_F16, nx::E_F16, a, ctx->stream), "gemv");
}

nx_status nx_gemv_int4_g32_f32(nx_ctx* ctx, nx_buf x, nx_buf wq, nx_buf sc, nx_buf y, int N, int K,
                               int batch, int accumulate) {
    nx::GemvArgs a;
    nx_status s = gemv_common(ctx, x, wq, sc, y, N, K, batch, 4, "nx_gemv_int4_g32_f32", a);
    if (s != NX_OK) return s;
    a.y32 = dptr<float>(y);
    return launched(ctx, nx::gemv_launch(nx::X_F16, accumulate ? nx::E_ACC : nx::E_F32, a, ctx->stream),
                    "gemv");
}

nx_status nx_gemm_int4_g32(nx_ctx* ctx, nx_buf x, nx_buf wq, nx_buf sc, nx_buf y, int M, int N, int K,
                           int accumulate) {
    if (!ctx) return NX_ERR_INVALID;
    if (M < 1 || N < 1 || K < 8) return fail(ctx, NX_ERR_INVALID, "nx_gemm_int4_g32: bad shape");
    if (K % 8) return fail(ctx, NX_ERR_UNSUPPORTED, "nx_gemm_int4_g32: K must be a multiple of 8");
    const int G = (K + 31) / 32;
    NX_NEED(ctx, x, (size_t)M * K * 2, "x");
    NX_NEED(ctx, wq, (size_t)N * G * 16, "codes");
    NX_NEED(ctx, sc, (size_t)N * G * 2, "scales");
    NX_NEED(ctx, y, (size_t)M * N * 4, "y");
    nx::PfGemmArgs a{};
    a.x = dptr<const uint16_t>(x);
    a.ldx = K;
    a.W = dptr<const uint8_t>(wq);
    a.S = dptr<const uint16_t>(sc);
    a.M = M;
    a.N = N;
    a.K = K;
    a.G = G;
    a.y32 = dptr<float>(y);
    a.ldy = N;
    return launched(ctx, nx::pf_gemm_launch(accumulate ? nx::PF_ACC : nx::PF_F32, a, ctx->stream), "gemm");
}

nx_status nx_time_gemm(nx_ctx* ctx, nx_buf x, nx_buf wq, nx_buf sc, nx_buf y, int M, int N, int K, int iters,
                       double* avg_ms) {
    if (!ctx || !avg_ms || iters < 1) return NX_ERR_INVALID;
    nx_status s = nx_gemm_int4_g32(ctx, x, wq, sc, y, M, N, K, 0);  // validation and warm-up
    if (s != NX_OK) return s;
    NX_HIP(ctx, hipEventRecord(ctx->ev0, ctx->stream));
    for (int i = 0; i < iters; ++i)
        if ((s = nx_gemm_int4_g32(ctx, x, wq, sc, y, M, N, K, 0)) != NX_OK) return s;
    NX_HIP(ctx, hipEventRecord(ctx->ev1, ctx->stream));
    NX_HIP(ctx, hipEventSynchronize(ctx->ev1));
    float ms = 0.0f;
    NX_HIP(ctx, hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1));
    *avg_ms = (double)ms / iters;
    return NX_OK;
}

nx_status nx_unpack_int4(nx_ctx* ctx, nx_buf packed, nx_buf codes, size_t n) {
    if (!ctx) return NX_ERR_INVALID;
    if (n % 2) return fail(ctx, NX_ERR_INVALID, "nx_unpack_int4: n must be even");
    NX_NEED(ctx, packed, n / 2, "packed");
    NX_NEED(ctx, codes, n, "codes");
    return launched(ctx, nx::unpack_int4_launch(dptr<const uint8_t>(packed), dptr<uint8_t>(codes), n, ctx->stream),
                    "unpack");
}

nx_status nx_quantize_int4_g32(nx_ctx* ctx, nx_buf w, nx_buf wq, nx_buf sc, int N, int K) {
    if (!ctx) return NX_ERR_INVALID;
    if (N <= 0 || K <= 0) return fail(ctx, NX_ERR_INVALID, "nx_quantize_int4_g32: bad shape");
    const int G = (K + 31) / 32;
    NX_NEED(ctx, w, (size_t)N * K * 4, "w");
    NX_NEED(ctx, wq, (size_t)N * G * 16, "codes");
    NX_NEED(ctx, sc, (size_t)N * G * 2, "scales");
    return launched(ctx, nx::quantize_int4_launch(dptr<const float>(w), dptr<uint8_t>(wq), dptr<uint16_t>(sc), N, K, ctx->stream),
                    "quantize");
}

nx_status nx_rmsnorm(nx_ctx* ctx, nx_buf x, nx_buf w, nx_buf out, int dim, float eps, int batch) {
    if (!ctx) return NX_ERR_INVALID;
    if (dim <= 0 || batch < 1) return fail(ctx, NX_ERR_INVALID, "nx_rmsnorm: bad shape");
    NX_NEED(ctx, x, (size_t)batch * dim * 4, "x");
    if (w) NX_NEED(ctx, w, (size_t)dim * 4, "w");
    NX_NEED(ctx, out, (size_t)batch * dim * 2, "out");
    return launched(ctx, nx::rmsnorm_launch(dptr<const float>(x), w ? dptr<const float>(w) : nullptr,
                                            dptr<uint16_t>(out), dim, eps, batch, ctx->stream),
                    "rmsnorm");
}

nx_status nx_rope(nx_ctx* ctx, nx_buf x, nx_buf pos, nx_buf cs, nx_buf sn, int heads, int hd,
                  int batch, int max_pos) {
    if (!ctx) return NX_ERR_INVALID;
    if (heads <= 0 || hd <= 0 || hd % 2 || batch < 1 || max_pos <= 0)
        return fail(ctx, NX_ERR_INVALID, "nx_rope: bad shape");
    NX_NEED(ctx, x, (size_t)batch * heads * hd * 4, "x");
    NX_NEED(ctx, pos, (size_t)batch * 4, "positions");
    NX_NEED(ctx, cs, (size_t)max_pos * (hd / 2) * 4, "cos");
    NX_NEED(ctx, sn, (size_t)max_pos * (hd / 2) * 4, "sin");
    std::vector<int32_t> hp(batch);
    // positions are validated against the tables on the host
    NX_HIP(ctx, hipMemcpyAsync(hp.data(), dptr<void>(pos), (size_t)batch * 4, hipMemcpyDeviceToHost, ctx->stream));
    NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    for (int b = 0; b < batch; ++b)
        if (hp[b] < 0 || hp[b] >= max_pos) return fail(ctx, NX_ERR_INVALID, "nx_rope: position %d out of table", hp[b]);
    return launched(ctx, nx::rope_launch(dptr<float>(x), dptr<const int32_t>(pos), dptr<const float>(cs),
                                         dptr<const float>(sn), heads, hd, batch, ctx->stream),
                    "rope");
}

nx_status nx_swiglu(nx_ctx* ctx, nx_buf g, nx_buf u, nx_buf out, int n, int batch) {
    if (!ctx) return NX_ERR_INVALID;
    if (n <= 0 || batch < 1) return fail(ctx, NX_ERR_INVALID, "nx_swiglu: bad shape");
    NX_NEED(ctx, g, (size_t)batch * n * 4, "gate");
    NX_NEED(ctx, u, (size_t)batch * n * 4, "up");
    NX_NEED(ctx, out, (size_t)batch * n * 2, "out");
    return launched(ctx, nx::swiglu_launch(dptr<const float>(g), dptr<const float>(u), dptr<uint16_t>(out), n, batch, ctx->stream),
                    "swiglu");
}

nx_status nx_residual_add(nx_ctx* ctx, nx_buf a, nx_buf b, nx_buf out, int n) {
    if (!ctx) return NX_ERR_INVALID;
    if (n <= 0) return fail(ctx, NX_ERR_INVALID, "nx_residual_add: bad shape");
    NX_NEED(ctx, a, (size_t)n * 4, "a");
    NX_NEED(ctx, b, (size_t)n * 4, "b");
    NX_NEED(ctx, out, (size_t)n * 4, "out");
    return launched(ctx, nx::residual_add_launch(dptr<const float>(a), dptr<const float>(b), dptr<float>(out), n, ctx->stream),
                    "residual_add");
}

// Host-side validation of a block table and per-sequence positions.
static nx_status check_table(nx_ctx* ctx, nx_buf bt, nx_buf lens, int batch, int max_blocks,
                             int num_blocks, bool lens_are_positions, const char* name) {
    NX_NEED(ctx, bt, (size_t)batch * max_blocks * 4, "block_table");
    NX_NEED(ctx, lens, (size_t)batch * 4, lens_are_positions ? "positions" : "ctx_lens");
    std::vector<int32_t> t((size_t)batch * max_blocks), l(batch);
    NX_HIP(ctx, hipMemcpyAsync(t.data(), dptr<void>(bt), t.size() * 4, hipMemcpyDeviceToHost, ctx->stream));
    NX_HIP(ctx, hipMemcpyAsync(l.data(), dptr<void>(lens), l.size() * 4, hipMemcpyDeviceToHost, ctx->stream));
    NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    for (int b = 0; b < batch; ++b) {
        const int len = lens_are_positions ? l[b] + 1 : l[b];
        if (len < 0 || len > max_blocks * nx::kPage)
            return fail(ctx, NX_ERR_CAPACITY, "%s: sequence %d length %d exceeds %d", name, b, len, max_blocks * nx::kPage);
        for (int p = 0; p < (len + nx::kPage - 1) / nx::kPage; ++p) {
            const int blk = t[(size_t)b * max_blocks + p];
            if (blk < 0 || blk >= num_blocks)
                return fail(ctx, NX_ERR_INVALID, "%s: block %d of sequence %d out of pool", name, blk, b);
        }
    }
    return NX_OK;
}

nx_status nx_kv_append_f16(nx_ctx* ctx, nx_buf k, nx_buf v, nx_buf kpool, nx_buf vpool, nx_buf bt,
                           nx_buf pos, int batch, int hkv, int hd, int max_blocks, int num_blocks) {
    if (!ctx) return NX_ERR_INVALID;
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "nx_kv_append_f16 validates positions on the host; not capturable");
    if (batch < 1 || hkv <= 0 || hd <= 0 || max_blocks <= 0 || num_blocks <= 0)
        return fail(ctx, NX_ERR_INVALID, "nx_kv_append_f16: bad shape");
    NX_NEED(ctx, k, (size_t)batch * hkv * hd * 4, "k");
    NX_NEED(ctx, v, (size_t)batch * hkv * hd * 4, "v");
    const size_t pool = (size_t)num_blocks * hkv * nx::kPage * hd * 2;
    NX_NEED(ctx, kpool, pool, "kpool");
    NX_NEED(ctx, vpool, pool, "vpool");
    nx_status s = check_table(ctx, bt, pos, batch, max_blocks, num_blocks, true, "nx_kv_append_f16");
    if (s != NX_OK) return s;
    return launched(ctx, nx::kv_append_f16_launch(dptr<const float>(k), dptr<const float>(v), dptr<uint16_t>(kpool),
                                                  dptr<uint16_t>(vpool), dptr<const int32_t>(bt), dptr<const int32_t>(pos),
                                                  batch, hkv, hd, max_blocks, ctx->stream),
                    "kv_append");
}

nx_status nx_attn_decode_paged_f16(nx_ctx* ctx, nx_buf q, nx_buf kpool, nx_buf vpool, nx_buf bt,
                                   nx_buf lens, nx_buf out, int batch, int hq, int hkv, int hd,
                                   int max_blocks, int num_blocks) {
    if (!ctx) return NX_ERR_INVALID;
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "nx_attn_decode_paged_f16 validates the block table on the host; not capturable");
    if (batch < 1 || hkv <= 0 || hq <= 0 || hq % hkv || (hd != 64 && hd != 128 && hd != 256) || max_blocks <= 0 ||
        num_blocks <= 0)
        return fail(ctx, NX_ERR_INVALID, "nx_attn_decode_paged_f16: bad shape");
    const int G = hq / hkv;
    if (G != 1 && G != 2 && G != 4 && G != 8)
        return fail(ctx, NX_ERR_UNSUPPORTED, "nx_attn_decode_paged_f16: hq/hkv = %d", G);
    NX_NEED(ctx, q, (size_t)batch * hq * hd * 4, "q");
    const size_t pool = (size_t)num_blocks * hkv * nx::kPage * hd * 2;
    NX_NEED(ctx, kpool, pool, "kpool");
    NX_NEED(ctx, vpool, pool, "vpool");
    NX_NEED(ctx, out, (size_t)batch * hq * hd * 2, "out");
    nx_status s = check_table(ctx, bt, lens, batch, max_blocks, num_blocks, false, "nx_attn_decode_paged_f16");
    if (s != NX_OK) return s;
    const int max_ctx = max_blocks * nx::kPage;
    if (max_ctx > nx::attn_max_ctx()) return fail(ctx, NX_ERR_UNSUPPORTED, "max_blocks above the attention limit");
    s = ensure_attn_ws(ctx, nx::attn_workspace_bytes(batch, hq, hkv, hd, max_ctx));
    if (s != NX_OK) return s;
    s = ensure_attn_counts(ctx, nx::attn_count_words(batch, hkv));
    if (s != NX_OK) return s;
    nx::AttnArgs a{};
    a.counts = ctx->attn_counts;
    a.q = dptr<const float>(q);
    a.kpool = dptr<const uint16_t>(kpool);
    a.vpool = dptr<const uint16_t>(vpool);
    a.block_table = dptr<const int32_t>(bt);
    a.ctx_lens = dptr<const int32_t>(lens);
    a.out16 = dptr<uint16_t>(out);
    a.batch = batch;
    a.hq = hq;
    a.hkv = hkv;
    a.hd = hd;
    a.max_blocks = max_blocks;
    a.max_ctx = max_ctx;
    a.part = static_cast<float*>(ctx->attn_ws);
    return launched(ctx, nx::attn_f16_launch(a, ctx->stream), "attn_f16");
}

// The fp16 paged attention with its split records and counters in the
// library's static scratch (g_attn_scratch in nx_attn.hip, whose device
// address nx_init took): no allocation, no host synchronization, so it may be
// captured into a graph.  Its kernels check the context lengths and table
// entries themselves (check_blocks); a sequence that fails gets NaN rows.
nx_status nx_attn_decode_paged_f16_noalloc(nx_ctx* ctx, nx_buf q, nx_buf kpool, nx_buf vpool, nx_buf bt,
                                           nx_buf lens, nx_buf out, int batch, int hq, int hkv, int hd,
                                           int max_blocks, int num_blocks) {
    if (!ctx) return NX_ERR_INVALID;
    if (batch < 1 || hkv <= 0 || hq <= 0 || hq % hkv || (hd != 64 && hd != 128 && hd != 256) || max_blocks <= 0 ||
        num_blocks <= 0)
        return fail(ctx, NX_ERR_INVALID, "nx_attn_decode_paged_f16_noalloc: bad shape");
    const int G = hq / hkv;
    if (G != 1 && G != 2 && G != 4 && G != 8)
        return fail(ctx, NX_ERR_UNSUPPORTED, "nx_attn_decode_paged_f16_noalloc: hq/hkv = %d", G);
    NX_NEED(ctx, q, (size_t)batch * hq * hd * 4, "q");
    const size_t pool = (size_t)num_blocks * hkv * nx::kPage * hd * 2;
    NX_NEED(ctx, kpool, pool, "kpool");
    NX_NEED(ctx, vpool, pool, "vpool");
    NX_NEED(ctx, out, (size_t)batch * hq * hd * 2, "out");
    NX_NEED(ctx, bt, (size_t)batch * max_blocks * 4, "block_table");
    NX_NEED(ctx, lens, (size_t)batch * 4, "ctx_lens");
    const int max_ctx = max_blocks * nx::kPage;
    if (max_ctx > nx::attn_max_ctx()) return fail(ctx, NX_ERR_UNSUPPORTED, "max_blocks above the attention limit");
    const size_t rec = nx::attn_f16_workspace_bytes(batch, hq, hkv, hd, max_ctx);
    const size_t words = nx::attn_count_words(batch, hkv);
    if (rec > nx::kNoAllocRecordBytes || words > nx::kNoAllocCountWords)
        return fail(ctx, NX_ERR_UNSUPPORTED,
                    "nx_attn_decode_paged_f16_noalloc: needs %zu bytes of split records and %zu counters; "
                    "the static scratch holds %zu and %zu",
                    rec, words, nx::kNoAllocRecordBytes, nx::kNoAllocCountWords);
    char* base = static_cast<char*>(ctx->na_scratch);
    unsigned* counts = reinterpret_cast<unsigned*>(base + nx::kNoAllocRecordBytes);
    // counters start at zero (a launch that completes leaves them at zero;
    // cleared here by a kernel, not a memset, so the call can be captured)
    hipError_t e = nx::zero_u32_launch(counts, words, ctx->stream);
    if (e != hipSuccess) return launched(ctx, e, "attn_noalloc zero counters");
    nx::AttnArgs a{};
    a.counts = counts;
    a.part = reinterpret_cast<float*>(base);
    a.q = dptr<const float>(q);
    a.kpool = dptr<const uint16_t>(kpool);
    a.vpool = dptr<const uint16_t>(vpool);
    a.block_table = dptr<const int32_t>(bt);
    a.ctx_lens = dptr<const int32_t>(lens);
    a.out16 = dptr<uint16_t>(out);
    a.batch = batch;
    a.hq = hq;
    a.hkv = hkv;
    a.hd = hd;
    a.max_blocks = max_blocks;
    a.max_ctx = max_ctx;
    a.check_blocks = num_blocks;
    return launched(ctx, nx::attn_f16_launch(a, ctx->stream), "attn_f16_noalloc");
}

nx_status nx_tq_codebooks(float* c4, float* b4, float* c3, float* b3) {
    if (!c4 || !b4 || !c3 || !b3) return NX_ERR_INVALID;
    nx::tq_codebook(128, 4, c4, b4);
    nx::tq_codebook(128, 3, c3, b3);
    return NX_OK;
}

nx_status nx_tq_encode(nx_ctx* ctx, nx_buf x, nx_buf signs, nx_buf c4, nx_buf c3, nx_buf norms,
                       int nvec) {
    if (!ctx) return NX_ERR_INVALID;
    if (nvec <= 0) return fail(ctx, NX_ERR_INVALID, "nx_tq_encode: nvec must be positive");
    NX_NEED(ctx, x, (size_t)nvec * 128 * 4, "x");
    NX_NEED(ctx, signs, 128 * 4, "signs");
    NX_NEED(ctx, c4, (size_t)nvec * 32, "codes4");
    NX_NEED(ctx, c3, (size_t)nvec * 24, "codes3");
    NX_NEED(ctx, norms, (size_t)nvec * 2, "norms");
    return launched(ctx, nx::tq_encode_launch(dptr<const float>(x), nvec, dptr<const float>(signs), nullptr, nullptr,
                                              dptr<uint8_t>(c4), dptr<uint8_t>(c3), dptr<uint16_t>(norms), nullptr,
                                              ctx->stream),
                    "tq_encode");
}

nx_status nx_tq_append(nx_ctx* ctx, nx_buf k, nx_buf v, nx_buf ksg, nx_buf vsg, nx_buf kc4,
                       nx_buf kc3, nx_buf kn, nx_buf vc4, nx_buf vc3, nx_buf vn, nx_buf bt,
                       nx_buf pos, int batch, int hkv, int max_blocks, int num_blocks) {
    if (!ctx) return NX_ERR_INVALID;
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "nx_tq_append validates positions on the host; not capturable");
    if (batch < 1 || hkv <= 0 || max_blocks <= 0 || num_blocks <= 0)
        return fail(ctx, NX_ERR_INVALID, "nx_tq_append: bad shape");
    const size_t nv = (size_t)num_blocks * hkv * nx::kPage;
    NX_NEED(ctx, k, (size_t)batch * hkv * 128 * 4, "k");
    NX_NEED(ctx, v, (size_t)batch * hkv * 128 * 4, "v");
    NX_NEED(ctx, ksg, 512, "ksigns");
    NX_NEED(ctx, vsg, 512, "vsigns");
    NX_NEED(ctx, kc4, nv * 32, "kc4");
    NX_NEED(ctx, kc3, nv * 24, "kc3");
    NX_NEED(ctx, kn, nv * 2, "kn");
    NX_NEED(ctx, vc4, nv * 32, "vc4");
    NX_NEED(ctx, vc3, nv * 24, "vc3");
    NX_NEED(ctx, vn, nv * 2, "vn");
    nx_status s = check_table(ctx, bt, pos, batch, max_blocks, num_blocks, true, "nx_tq_append");
    if (s != NX_OK) return s;
    // the append kernel reads K and V from one [batch][2][hkv*128] staging layout
    const size_t stage = (size_t)batch * 2 * hkv * 128 * 4;
    s = ensure_attn_ws(ctx, stage > ctx->attn_ws_bytes ? stage : ctx->attn_ws_bytes);
    if (s != NX_OK) return s;
    float* tmp = static_cast<float*>(ctx->attn_ws);
    for (int b = 0; b < batch; ++b) {
        NX_HIP(ctx, hipMemcpyAsync(tmp + ((size_t)b * 2 + 0) * hkv * 128, dptr<float>(k) + (size_t)b * hkv * 128,
                                   (size_t)hkv * 128 * 4, hipMemcpyDeviceToDevice, ctx->stream));
        NX_HIP(ctx, hipMemcpyAsync(tmp + ((size_t)b * 2 + 1) * hkv * 128, dptr<float>(v) + (size_t)b * hkv * 128,
                                   (size_t)hkv * 128 * 4, hipMemcpyDeviceToDevice, ctx->stream));
    }
    return launched(ctx, nx::tq_append_launch(tmp, batch, hkv, dptr<const float>(ksg), dptr<const float>(vsg), nullptr,
                                              nullptr, dptr<uint8_t>(kc4), dptr<uint8_t>(kc3), dptr<uint16_t>(kn),
                                              dptr<uint8_t>(vc4), dptr<uint8_t>(vc3), dptr<uint16_t>(vn),
                                              dptr<const int32_t>(bt), dptr<const int32_t>(pos), max_blocks, ctx->stream),
                    "tq_append");
}

nx_status nx_attn_decode_paged_tq(nx_ctx* ctx, nx_buf q, nx_buf kc4, nx_buf kc3, nx_buf kn,
                                  nx_buf vc4, nx_buf vc3, nx_buf vn, nx_buf ksg, nx_buf vsg,
                                  nx_buf bt, nx_buf lens, nx_buf out, int batch, int hq, int hkv,
                                  int max_blocks, int num_blocks) {
    if (!ctx) return NX_ERR_INVALID;
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "nx_attn_decode_paged_tq validates the block table on the host; not capturable");
    if (batch < 1 || hkv <= 0 || hq <= 0 || hq % hkv || max_blocks <= 0 || num_blocks <= 0)
        return fail(ctx, NX_ERR_INVALID, "nx_attn_decode_paged_tq: bad shape");
    const int G = hq / hkv;
    if (G != 1 && G != 2 && G != 4 && G != 8)
        return fail(ctx, NX_ERR_UNSUPPORTED, "nx_attn_decode_paged_tq: hq/hkv = %d", G);
    const size_t nv = (size_t)num_blocks * hkv * nx::kPage;
    NX_NEED(ctx, q, (size_t)batch * hq * 128 * 4, "q");
    NX_NEED(ctx, kc4, nv * 32, "kc4");
    NX_NEED(ctx, kc3, nv * 24, "kc3");
    NX_NEED(ctx, kn, nv * 2, "kn");
    NX_NEED(ctx, vc4, nv * 32, "vc4");
    NX_NEED(ctx, vc3, nv * 24, "vc3");
    NX_NEED(ctx, vn, nv * 2, "vn");
    NX_NEED(ctx, ksg, 512, "ksigns");
    NX_NEED(ctx, vsg, 512, "vsigns");
    NX_NEED(ctx, out, (size_t)batch * hq * 128 * 2, "out");
    nx_status s = check_table(ctx, bt, lens, batch, max_blocks, num_blocks, false, "nx_attn_decode_paged_tq");
    if (s != NX_OK) return s;
    const int max_ctx = max_blocks * nx::kPage;
    if (max_ctx > nx::attn_max_ctx()) return fail(ctx, NX_ERR_UNSUPPORTED, "max_blocks above the attention limit");
    s = ensure_attn_ws(ctx, nx::attn_workspace_bytes(batch, hq, hkv, 128, max_ctx));
    if (s != NX_OK) return s;
    nx::AttnArgs a{};
    a.q = dptr<const float>(q);
    a.kc4 = dptr<const uint8_t>(kc4);
    a.kc3 = dptr<const uint8_t>(kc3);
    a.kn = dptr<const uint16_t>(kn);
    a.vc4 = dptr<const uint8_t>(vc4);
    a.vc3 = dptr<const uint8_t>(vc3);
    a.vn = dptr<const uint16_t>(vn);
    a.ksign = dptr<const float>(ksg);
    a.vsign = dptr<const float>(vsg);
    a.block_table = dptr<const int32_t>(bt);
    a.ctx_lens = dptr<const int32_t>(lens);
    a.out16 = dptr<uint16_t>(out);
    a.batch = batch;
    a.hq = hq;
    a.hkv = hkv;
    a.hd = 128;
    a.max_blocks = max_blocks;
    a.max_ctx = max_ctx;
    a.part = static_cast<float*>(ctx->attn_ws);
    s = ensure_attn_counts(ctx, nx::attn_count_words(batch, hkv));
    if (s != NX_OK) return s;
    a.counts = ctx->attn_counts;
    return launched(ctx, nx::attn_tq_launch(a, ctx->stream), "attn_tq");
}

nx_status nx_moe_route_topk(nx_ctx* ctx, nx_buf logits, nx_buf ids, nx_buf w, int E, int k, int batch) {
    if (!ctx) return NX_ERR_INVALID;
    if (E < 1 || E > nx::kMoeMaxExperts || k < 1 || k > nx::kMoeMaxTopK || k > E || batch < 1 || batch > 64)
        return fail(ctx, NX_ERR_INVALID, "nx_moe_route_topk: bad shape E=%d k=%d batch=%d", E, k, batch);
    NX_NEED(ctx, logits, (size_t)batch * E * 4, "logits");
    NX_NEED(ctx, ids, (size_t)batch * k * 4, "ids");
    NX_NEED(ctx, w, (size_t)batch * k * 4, "weights");
    // per-expert token lists live in the attention workspace
    const size_t extra = ((size_t)E + (size_t)E * batch * k) * 4;
    nx_status s = ensure_attn_ws(ctx, extra > ctx->attn_ws_bytes ? extra : ctx->attn_ws_bytes);
    if (s != NX_OK) return s;
    nx::MoeArgs a{};
    a.logits = dptr<float>(logits);
    a.E = E;
    a.k = k;
    a.batch = batch;
    a.ids = dptr<int32_t>(ids);
    a.weights = dptr<float>(w);
    a.expert_count = static_cast<int32_t*>(ctx->attn_ws);
    a.expert_slots = a.expert_count + E;
    return launched(ctx, nx::moe_route_launch(a, ctx->stream), "moe_route");
}

nx_status nx_moe_expert_ffn(nx_ctx* ctx, nx_buf x, nx_buf w13, nx_buf s13, nx_buf w2, nx_buf s2,
                            nx_buf ids, nx_buf w, nx_buf out, int d, int F, int E, int k, int batch,
                            int accumulate) {
    if (!ctx) return NX_ERR_INVALID;
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "nx_moe_expert_ffn validates expert ids on the host; not capturable");
    if (d <= 0 || F <= 0 || E < 1 || E > nx::kMoeMaxExperts || k < 1 || k > nx::kMoeMaxTopK || k > E || batch < 1 ||
        batch > nx::kMoeMaxBatch)
        return fail(ctx, NX_ERR_INVALID, "nx_moe_expert_ffn: bad shape");
    const int Gd = (d + 31) / 32, Gf = (F + 31) / 32;
    if (Gd > 448 || Gf > 448) return fail(ctx, NX_ERR_UNSUPPORTED, "nx_moe_expert_ffn: K above 14336");
    const int Fp = Gf * 32;
    NX_NEED(ctx, x, (size_t)batch * d * 2, "x");
    NX_NEED(ctx, w13, (size_t)E * 2 * F * Gd * 16, "w13");
    NX_NEED(ctx, s13, (size_t)E * 2 * F * Gd * 2, "s13");
    NX_NEED(ctx, w2, (size_t)E * d * Gf * 16, "w2");
    NX_NEED(ctx, s2, (size_t)E * d * Gf * 2, "s2");
    NX_NEED(ctx, ids, (size_t)batch * k * 4, "ids");
    NX_NEED(ctx, w, (size_t)batch * k * 4, "weights");
    NX_NEED(ctx, out, (size_t)batch * d * 4, "out");
    std::vector<int32_t> hid((size_t)batch * k);
    NX_HIP(ctx, hipMemcpyAsync(hid.data(), dptr<void>(ids), hid.size() * 4, hipMemcpyDeviceToHost, ctx->stream));
    NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    // routing plan (the layout moe_route writes): the experts that hold slots
    // in ascending order, each with its slots b * k + j and their tokens b
    std::vector<int32_t> count(E, 0);
    for (int b = 0; b < batch; ++b)
        for (int j = 0; j < k; ++j) {
            const int e = hid[(size_t)b * k + j];
            if (e < 0 || e >= E) return fail(ctx, NX_ERR_INVALID, "nx_moe_expert_ffn: expert id %d out of range", e);
            if (++count[e] > nx::kMoePlanMaxSlots)
                return fail(ctx, NX_ERR_INVALID, "nx_moe_expert_ffn: more than %d slots on expert %d",
                            nx::kMoePlanMaxSlots, e);
        }
    const int rows = nx::moe_plan_rows(E, batch, k);
    std::vector<int32_t> plan((size_t)rows * nx::kMoePlanInts, 0);
    int r = 0;
    for (int e = 0; e < E; ++e) {
        if (count[e] == 0) continue;
        if (r == rows) return fail(ctx, NX_ERR_INVALID, "nx_moe_expert_ffn: more active experts than slots");
        int32_t* pl = plan.data() + (size_t)r * nx::kMoePlanInts;
        pl[0] = e;
        int n = 0;
        for (int b = 0; b < batch; ++b)
            for (int j = 0; j < k; ++j)
                if (hid[(size_t)b * k + j] == e) {
                    pl[8 + n] = b * k + j;
                    pl[16 + n] = b;
                    ++n;
                }
        pl[1] = n;
        ++r;
    }
    for (; r < rows; ++r) plan[(size_t)r * nx::kMoePlanInts] = -1;
    // workspace: plan | act16[batch*k][Fp] | y32[batch*k][d] | K-part sums
    // of the down projection [kparts][batch*k][d]
    const size_t off_act = (plan.size() * 4 + 255) / 256 * 256;
    const size_t off_y = (off_act + (size_t)batch * k * Fp * 2 + 255) / 256 * 256;
    const size_t off_kp = (off_y + (size_t)batch * k * d * 4 + 255) / 256 * 256;
    const size_t total = off_kp + (size_t)nx::gemv_kparts(F, batch) * batch * k * d * 4;
    nx_status s = ensure_attn_ws(ctx, total);
    if (s != NX_OK) return s;
    char* ws = static_cast<char*>(ctx->attn_ws);
    NX_HIP(ctx, hipMemcpyAsync(ws, plan.data(), plan.size() * 4, hipMemcpyHostToDevice, ctx->stream));
    NX_HIP(ctx, hipMemsetAsync(ws + off_act, 0, (size_t)batch * k * Fp * 2, ctx->stream));
    nx::MoeFfnArgs a{};
    a.x16 = dptr<const uint16_t>(x);
    a.ldx = d;
    a.w13 = dptr<const uint8_t>(w13);
    a.s13 = dptr<const uint16_t>(s13);
    a.w2 = dptr<const uint8_t>(w2);
    a.s2 = dptr<const uint16_t>(s2);
    a.d = d;
    a.F = F;
    a.E = E;
    a.k = k;
    a.batch = batch;
    a.plan = reinterpret_cast<const int32_t*>(ws);
    a.weights = dptr<const float>(w);
    a.act16 = reinterpret_cast<uint16_t*>(ws + off_act);
    a.y32 = reinterpret_cast<float*>(ws + off_y);
    a.kpart = nx::gemv_kparts(F, batch) > 0 ? reinterpret_cast<float*>(ws + off_kp) : nullptr;
    a.out = dptr<float>(out);
    a.accumulate = accumulate;
    hipError_t e = nx::moe_gate_up_launch(a, ctx->stream);
    if (e == hipSuccess) e = nx::moe_down_launch(a, ctx->stream);
    if (e == hipSuccess) e = nx::moe_combine_launch(a, ctx->stream);
    return launched(ctx, e, "moe_expert_ffn");
}

nx_status nx_sample(nx_ctx* ctx, nx_buf logits, nx_buf out, int V, int batch, float temperature, int top_k,
                    float top_p, uint64_t seed) {
    if (!ctx) return NX_ERR_INVALID;
    if (temperature <= 0.0f) return nx_argmax(ctx, logits, out, V, batch);
    if (V <= 0 || batch < 1) return fail(ctx, NX_ERR_INVALID, "nx_sample: bad shape");
    if (top_k < 0 || !(top_p > 0.0f) || top_p > 1.0f) return fail(ctx, NX_ERR_INVALID, "nx_sample: bad parameters");
    NX_NEED(ctx, logits, (size_t)batch * V * 4, "logits");
    NX_NEED(ctx, out, (size_t)batch * 4, "out");
    nx_status ws = ensure_smp_ws(ctx, (size_t)batch * ((size_t)V + nx::kSmpPartFloats));
    if (ws != NX_OK) return ws;
    nx::SampleArgs a{};
    a.scratch = ctx->smp_ws;
    a.part = ctx->smp_ws + (size_t)batch * V;
    a.logits = dptr<const float>(logits);
    a.V = V;
    a.ldl = V;
    a.temperature = temperature;
    a.top_k = top_k;
    a.top_p = top_p;
    a.u_fixed = nx::sample_draw(seed);
    a.out = dptr<int32_t>(out);
    return launched(ctx, nx::sample_launch(a, batch, ctx->stream), "sample");
}

nx_status nx_argmax(nx_ctx* ctx, nx_buf logits, nx_buf out, int V, int batch) {
    if (!ctx) return NX_ERR_INVALID;
    if (V <= 0 || batch < 1) return fail(ctx, NX_ERR_INVALID, "nx_argmax: bad shape");
    NX_NEED(ctx, logits, (size_t)batch * V * 4, "logits");
    NX_NEED(ctx, out, (size_t)batch * 4, "out");
    return launched(ctx, nx::argmax_launch(dptr<const float>(logits), dptr<int32_t>(out), V, batch, ctx->stream), "argmax");
}

nx_status nx_time_gemv(nx_ctx* ctx, nx_buf x, const nx_buf* wq, const nx_buf* sc, int ncopies,
                       nx_buf y, int N, int K, int batch, int iters, double* avg_ms) {
    if (!ctx || !avg_ms || !wq || !sc || ncopies < 1 || iters < 1) return NX_ERR_INVALID;
    for (int c = 0; c < ncopies; ++c) {  // warm-up and validation of every copy
        nx_status s = nx_gemv_int4_g32(ctx, x, wq[c], sc[c], y, N, K, batch);
        if (s != NX_OK) return s;
    }
    // the launches as one graph, as a decode step runs them: the average
    // includes the kernel boundary a step pays per launch, not the host's
    // per-launch submission cost
    NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    NX_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    nx_status s = NX_OK;
    for (int i = 0; i < iters && s == NX_OK; ++i)
        s = nx_gemv_int4_g32(ctx, x, wq[i % ncopies], sc[i % ncopies], y, N, K, batch);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    if (s != NX_OK || e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return s != NX_OK ? s : nx::hip_fail(ctx, e, "hipStreamEndCapture");
    }
    hipGraphExec_t ge = nullptr;
    const hipError_t ei = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ei != hipSuccess) return nx::hip_fail(ctx, ei, "hipGraphInstantiate");
    float ms = 0.0f;
    hipError_t er = hipGraphLaunch(ge, ctx->stream);  // warm
    if (er == hipSuccess) er = hipEventRecord(ctx->ev0, ctx->stream);
    if (er == hipSuccess) er = hipGraphLaunch(ge, ctx->stream);
    if (er == hipSuccess) er = hipEventRecord(ctx->ev1, ctx->stream);
    if (er == hipSuccess) er = hipEventSynchronize(ctx->ev1);
    if (er == hipSuccess) er = hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1);
    (void)hipGraphExecDestroy(ge);
    if (er != hipSuccess) return nx::hip_fail(ctx, er, "timing graph");
    *avg_ms = (double)ms / iters;
    return NX_OK;
}

}  // extern "C"

// ------------------------------------------------- dispatch-layer entries --
// The remaining ComputeDispatch members the runner calls
// (hybrid_model.cpp:121, :512-581, :639, :820-1241).

nx_status nx_gemm_f32(nx_ctx* ctx, nx_buf A, nx_buf B, nx_buf C, int M, int N, int K) {
    if (!ctx) return NX_ERR_INVALID;
    if (M <= 0 || N <= 0 || K <= 0 || M > 4194240)
        return fail(ctx, NX_ERR_INVALID, "nx_gemm_f32: bad shape M=%d N=%d K=%d", M, N, K);
    NX_NEED(ctx, A, (size_t)M * K * 4, "A");
    NX_NEED(ctx, B, (size_t)K * N * 4, "B");
    NX_NEED(ctx, C, (size_t)M * N * 4, "C");
    return launched(ctx, nx::gemm_f32_launch(dptr<const float>(A), dptr<const float>(B), dptr<float>(C), M, N, K,
                                             ctx->stream),
                    "gemm_f32");
}

namespace {
// Grow-only fp16 activation workspace of nx_ffn_int4_g32.
nx_status ensure_ffn_ws(nx_ctx* ctx, size_t bytes) {
    if (bytes <= ctx->ffn_ws_bytes) return NX_OK;
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "FFN workspace must grow outside capture");
    NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->ffn_ws) (void)hipFree(ctx->ffn_ws);
    ctx->ffn_ws = nullptr;
    ctx->ffn_ws_bytes = 0;
    NX_HIP(ctx, hipMalloc(&ctx->ffn_ws, bytes));
    ctx->ffn_ws_bytes = bytes;
    return NX_OK;
}

nx_status ensure_smp_ws(nx_ctx* ctx, size_t floats) {
    if (floats <= ctx->smp_ws_floats) return NX_OK;
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "sampler scratch must grow outside capture");
    NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->smp_ws) (void)hipFree(ctx->smp_ws);
    ctx->smp_ws = nullptr;
    ctx->smp_ws_floats = 0;
    NX_HIP(ctx, hipMalloc(reinterpret_cast<void**>(&ctx->smp_ws), floats * sizeof(float)));
    ctx->smp_ws_floats = floats;
    return NX_OK;
}

size_t ffn_lda(int F) { return (size_t)(F + 7) / 8 * 8; }
}  // namespace

nx_status nx_ffn_int4_g32(nx_ctx* ctx, nx_buf x, nx_buf w13, nx_buf s13, nx_buf w2, nx_buf s2, nx_buf y, int d,
                          int F, int batch, int accumulate) {
    if (!ctx) return NX_ERR_INVALID;
    if (d <= 0 || F <= 0 || batch < 1 || batch > 8)
        return fail(ctx, NX_ERR_INVALID, "nx_ffn_int4_g32: bad shape d=%d F=%d batch=%d", d, F, batch);
    const int Gd = (d + 31) / 32, Gf = (F + 31) / 32;
    if (Gd > 7 * 64 || Gf > 14 * 64) return fail(ctx, NX_ERR_UNSUPPORTED, "nx_ffn_int4_g32: d above 14336 or F above 28672");
    NX_NEED(ctx, x, (size_t)batch * d * 2, "x");
    NX_NEED(ctx, w13, (size_t)2 * F * Gd * 16, "w13");
    NX_NEED(ctx, s13, (size_t)2 * F * Gd * 2, "s13");
    NX_NEED(ctx, w2, (size_t)d * Gf * 16, "w2");
    NX_NEED(ctx, s2, (size_t)d * Gf * 2, "s2");
    NX_NEED(ctx, y, (size_t)batch * d * 4, "y");
    const size_t lda = ffn_lda(F);
    nx_status s = ensure_ffn_ws(ctx, (size_t)batch * lda * 2);
    if (s != NX_OK) return s;
    uint16_t* act = static_cast<uint16_t*>(ctx->ffn_ws);
    nx::GemvArgs f{};
    f.W = dptr<const uint8_t>(w13);
    f.S = dptr<const uint16_t>(s13);
    f.N = 2 * F;
    f.K = d;
    f.G = Gd;
    f.batch = batch;
    f.x16 = dptr<const uint16_t>(x);
    f.ldx = d;
    f.act16 = act;
    f.lda = (int)lda;
    s = launched(ctx, nx::gemv_launch(nx::X_F16, nx::E_SWIGLU, f, ctx->stream), "ffn gate/up");
    if (s != NX_OK) return s;
    nx::GemvArgs dn{};
    dn.W = dptr<const uint8_t>(w2);
    dn.S = dptr<const uint16_t>(s2);
    dn.N = d;
    dn.K = F;
    dn.G = Gf;
    dn.batch = batch;
    dn.x16 = act;
    dn.ldx = (int)lda;
    dn.y32 = dptr<float>(y);
    dn.ldy = d;
    s = gemv_kpart_ws(ctx, d, F, batch, &dn.kpart);
    if (s != NX_OK) return s;
    return launched(ctx, nx::gemv_launch(nx::X_F16, accumulate ? nx::E_ACC : nx::E_F32, dn, ctx->stream), "ffn down");
}

nx_status nx_init_gpu_pool(nx_ctx* ctx, int hidden, int max_q, int max_kv, int max_ffn, int vocab, int batch,
                           nx_gpu_pool* out) {
    if (!ctx || !out) return NX_ERR_INVALID;
    if (hidden <= 0 || max_q <= 0 || max_kv <= 0 || max_ffn <= 0 || vocab <= 0 || batch < 1 || batch > 8)
        return fail(ctx, NX_ERR_INVALID, "nx_init_gpu_pool: bad sizes");
    const size_t B = (size_t)batch;
    struct Want {
        nx_buf* dst;
        size_t bytes;
    } want[] = {
        {&out->hidden, B * hidden * 4},  {&out->residual, B * hidden * 4}, {&out->norm, B * hidden * 2},
        {&out->q, B * max_q * 4},        {&out->k, B * max_kv * 4},        {&out->v, B * max_kv * 4},
        {&out->attn_out, B * max_q * 2}, {&out->ffn_gate, B * max_ffn * 4}, {&out->ffn_up, B * max_ffn * 4},
        {&out->ffn_act, B * ffn_lda(max_ffn) * 2}, {&out->ffn_out, B * hidden * 4},
        {&out->logits, B * vocab * 4},   {&out->token, B * 4},
    };
    const int n = (int)(sizeof(want) / sizeof(want[0]));
    for (int i = 0; i < n; ++i) {
        nx_status s = nx_alloc(ctx, want[i].bytes, want[i].dst);
        if (s != NX_OK) {
            for (int j = 0; j < i; ++j) (void)nx_free(ctx, *want[j].dst);
            return s;
        }
    }
    return NX_OK;
}

nx_status nx_init_kv_cache(nx_ctx* ctx, int num_layers, int max_seq, int n_kv_heads, int head_dim, int batch,
                           nx_buf* kpools, nx_buf* vpools, nx_buf* block_table, int* max_blocks, int* num_blocks) {
    if (!ctx || !kpools || !vpools || !block_table) return NX_ERR_INVALID;
    if (num_layers < 1 || max_seq < 1 || n_kv_heads < 1 || (head_dim != 64 && head_dim != 128) || batch < 1 ||
        batch > 8)
        return fail(ctx, NX_ERR_INVALID, "nx_init_kv_cache: bad shape");
    const int mb = (max_seq + nx::kPage - 1) / nx::kPage, nb = batch * mb;
    const size_t pool = (size_t)nb * n_kv_heads * nx::kPage * head_dim * 2;
    std::vector<int32_t> bt((size_t)batch * mb);
    for (int b = 0; b < batch; ++b)
        for (int p = 0; p < mb; ++p) bt[(size_t)b * mb + p] = b * mb + p;
    nx_status s = nx_alloc(ctx, bt.size() * 4, block_table);
    if (s != NX_OK) return s;
    s = nx_upload(ctx, *block_table, 0, bt.data(), bt.size() * 4);
    int done = 0;
    for (; s == NX_OK && done < num_layers; ++done) {
        s = nx_alloc(ctx, pool, &kpools[done]);
        if (s != NX_OK) break;
        s = nx_alloc(ctx, pool, &vpools[done]);
        if (s != NX_OK) {
            (void)nx_free(ctx, kpools[done]);
            break;
        }
    }
    if (s != NX_OK) {
        for (int j = 0; j < done; ++j) {
            (void)nx_free(ctx, kpools[j]);
            (void)nx_free(ctx, vpools[j]);
        }
        (void)nx_free(ctx, *block_table);
        return s;
    }
    if (max_blocks) *max_blocks = mb;
    if (num_blocks) *num_blocks = nb;
    return NX_OK;
}

nx_status nx_reserve_workspace(nx_ctx* ctx, int batch, int max_ffn, int vocab, int n_heads, int n_kv_heads,
                               int head_dim, int max_ctx) {
    if (!ctx) return NX_ERR_INVALID;
    if (batch < 1 || batch > 8 || max_ffn < 0 || vocab < 0 || n_heads < 0 || n_kv_heads < 0 || head_dim < 0 ||
        max_ctx < 0)
        return fail(ctx, NX_ERR_INVALID, "nx_reserve_workspace: bad sizes");
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "nx_reserve_workspace inside a token batch");
    nx_status s = NX_OK;
    if (max_ffn > 0) s = ensure_ffn_ws(ctx, (size_t)batch * ffn_lda(max_ffn) * 2);
    if (s == NX_OK && max_ffn > 0 && n_heads > 0 && head_dim > 0) {
        float* unused = nullptr;  // the down projection's K parts (d = n_heads * head_dim)
        s = gemv_kpart_ws(ctx, n_heads * head_dim, max_ffn, batch, &unused);
    }
    if (s == NX_OK && vocab > 0) s = ensure_smp_ws(ctx, (size_t)batch * ((size_t)vocab + nx::kSmpPartFloats));
    if (s == NX_OK && n_heads > 0 && n_kv_heads > 0 && head_dim > 0 && max_ctx > 0) {
        if (n_heads % n_kv_heads) return fail(ctx, NX_ERR_INVALID, "nx_reserve_workspace: n_heads % n_kv_heads");
        if (max_ctx > nx::attn_max_ctx()) return fail(ctx, NX_ERR_UNSUPPORTED, "max_ctx above the attention limit");
        s = ensure_attn_ws(ctx, nx::attn_workspace_bytes(batch, n_heads, n_kv_heads, head_dim, max_ctx));
        if (s == NX_OK) s = ensure_attn_counts(ctx, nx::attn_count_words(batch, n_kv_heads));
    }
    if (s == NX_OK) NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return s;
}

nx_status nx_preload_all_buffers(nx_ctx* ctx, size_t* n_buffers) {
    if (!ctx) return NX_ERR_INVALID;
    if (ctx->capturing) return fail(ctx, NX_ERR_STATE, "nx_preload_all_buffers inside a token batch");
    NX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (n_buffers) *n_buffers = ctx->wcache.size();
    return NX_OK;
}
