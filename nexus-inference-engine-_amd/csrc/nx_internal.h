// Internal host-side state shared by the C-ABI layer and the runner.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/nexus_hip.h"

struct nx_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::map<uint64_t, size_t> bufs;                   // device address -> bytes
    std::unordered_map<const void*, uint64_t> wcache;  // host key -> buffer
    std::string err;
    bool capturing = false;
    hipGraphExec_t token_exec = nullptr;
    // token batch split by flush / resume: the graph of each segment after
    // the first is kept per segment (segment 0 uses token_exec)
    bool token_flushed = false;
    int token_seg = 0;
    std::vector<hipGraphExec_t> seg_exec;
    // intermediate SwiGLU activations of nx_ffn_int4_g32 (grow-only, fp16)
    void* ffn_ws = nullptr;
    size_t ffn_ws_bytes = 0;
    // workspace of the standalone attention entry points
    void* attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    unsigned* attn_counts = nullptr;  // split-completion counters (zero between launches)
    size_t attn_count_words = 0;
    // device address of the static scratch array of
    // nx_attn_decode_paged_f16_noalloc on this context's device
    void* na_scratch = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    // scratch rows of nx_sample (grow-only)
    float* smp_ws = nullptr;
    size_t smp_ws_floats = 0;
    // K-part sums of batched GEMVs with K beyond 4096 (grow-only; without
    // room, under capture, one launch streams all of K)
    float* gemv_ws = nullptr;
    size_t gemv_ws_floats = 0;
    float c4[16], b4[15], c3[8], b3[7];
};

namespace nx {

inline nx_status fail(nx_ctx* ctx, nx_status code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (ctx) ctx->err = buf;
    return code;
}

inline nx_status hip_fail(nx_ctx* ctx, hipError_t e, const char* what) {
    return fail(ctx, e == hipErrorOutOfMemory ? NX_ERR_OOM : NX_ERR_HIP, "%s: %s", what,
                hipGetErrorString(e));
}

// Size of a buffer of the context, 0 if it is not one.
inline size_t buf_size(const nx_ctx* ctx, nx_buf b) {
    auto it = ctx->bufs.find(b);
    return it == ctx->bufs.end() ? 0 : it->second;
}

// Restatement of the Lloyd-Max codebook construction for N(0, 1/d)
// (kv/turbo_quant.cpp:172-219), float arithmetic as in the reference.
void tq_codebook(int d, int bits, float* centroids, float* boundaries);

}  // namespace nx

#define NX_HIP(ctx, expr)                                  \
    do {                                                   \
        hipError_t nx_e_ = (expr);                         \
        if (nx_e_ != hipSuccess) return nx::hip_fail((ctx), nx_e_, #expr); \
    } while (0)

// Check that handle `b` names a buffer of at least `bytes` bytes.
#define NX_NEED(ctx, b, bytes, name)                                                          \
    do {                                                                                      \
        size_t nx_sz_ = nx::buf_size((ctx), (b));                                             \
        if (nx_sz_ == 0) return nx::fail((ctx), NX_ERR_INVALID, "%s: unknown buffer", name); \
        if (nx_sz_ < (size_t)(bytes))                                                         \
            return nx::fail((ctx), NX_ERR_INVALID, "%s: buffer has %zu bytes, needs %zu", name, \
                            nx_sz_, (size_t)(bytes));                                         \
    } while (0)
