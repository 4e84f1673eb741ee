// runtime.hip — the C ABI of libnn-hip.so (include/nnhip.h): contexts, memory, argument
// validation and dispatch to the gfx950 kernels. Every entry point validates its arguments
// on the host (null pointers, shapes, alignment, the kernels' size limits) before any launch,
// and reports failures through the status code and the thread-local last-error string.
#include "nnhip.h"

#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <queue>
#include <string>
#include <vector>

using namespace nnhip;

// Scratch of nnhip_matmul_q_i8_noalloc (repacked weights, token-major activations, row sums):
// one copy per GPU, loaded with the code object and held until the process ends. In host code
// the name is only a stand-in for the symbol: its device address comes from
// hipGetSymbolAddress (g_scratch_dev below), never from taking the array's address here.
static __device__ __align__(256) uint8_t scratch[NNHIP_NOALLOC_SCRATCH_BYTES];

struct nnhip_ctx
{
    int device = 0;
    void* scratch = nullptr;  // this device's copy of `scratch` (device address)
    int num_cus = 256;
    hipStream_t own = nullptr;
    hipStream_t stream = nullptr;
    void* ws = nullptr;  // workspace of the reference-layout matmul_q_i8 path
    size_t ws_bytes = 0;
    // per-token absmax between the gated GEMM epilogue and the next quantization of the fused
    // FFN block: zero between calls (zero-filled when allocated, reset by its consumer)
    int gemm_tile = NNHIP_GEMM_TILE_AUTO;
    void* attn_ws = nullptr;  // per-chunk partial results of the decode attention
    size_t attn_ws_bytes = 0;
    float* ones = nullptr;  // 1.0f, the unit scales of the digit products
    size_t ones_words = 0;
    size_t ones_bytes_ = 0;
    // ranges that the next per-token quantizer call reads in extra blocks (nnhip_ctx_prefetch_next)
    Prefetch pf{};
};

namespace
{
// The pending prefetch ranges, cleared: every quantizer entry point takes them, whether or not
// its launch can carry them (only the one-token kernels, M <= 64, do).
Prefetch take_prefetch(nnhip_ctx* ctx)
{
    const Prefetch p = ctx->pf;
    ctx->pf = Prefetch{};
    return p;
}
}  // namespace

struct nnhip_group
{
    // one kernel launch over a subset of the group's problems
    struct Launch
    {
        GemvProblem* d_probs = nullptr;
        uint32_t* d_wave_start = nullptr;  // n_waves + 1 offsets into d_wave_items
        uint32_t* d_wave_items = nullptr;  // problem << 20 | row tile, grouped by wave
        XStage* d_xstage = nullptr;        // activation blocks staged in LDS (LDS variant)
        int n_xstage = 0;
        uint32_t lds_bytes = 0;
        size_t n_waves = 0;
    };
    std::vector<Launch> launches;
};

namespace
{

thread_local std::string g_err;

nnhip_status fail(nnhip_status st, const char* fn, const std::string& msg)
{
    g_err = std::string(fn) + ": " + msg;
    return st;
}

nnhip_status hip_fail(const char* fn, const char* what, hipError_t e)
{
    return fail(NNHIP_ERR_HIP, fn, std::string(what) + " failed: " + hipGetErrorString(e));
}

// Device address of `scratch` on each device, resolved once per device by the first context
// created on it (with that device current).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

nnhip_status resolve_scratch(int device, void** out, const char* fn)
{
    if (device < 0 || device >= kMaxDevices) return fail(NNHIP_ERR_UNSUPPORTED, fn, "device index beyond 63");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_dev[device])
    {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr)
        {
            (void)hipGetLastError();
            return hip_fail(fn, "hipGetSymbolAddress(scratch)", e);
        }
        g_scratch_dev[device] = ptr;
    }
    *out = g_scratch_dev[device];
    return NNHIP_OK;
}

#define NNHIP_CHECK_CTX(fn)                                                  \
    do                                                                       \
    {                                                                        \
        if (!ctx) return fail(NNHIP_ERR_INVALID_ARG, fn, "null context");   \
        const hipError_t se_ = hipSetDevice(ctx->device);                    \
        if (se_ != hipSuccess) return hip_fail(fn, "hipSetDevice", se_);     \
    } while (0)

#define NNHIP_REQUIRE(cond, fn, msg)                                         \
    do                                                                       \
    {                                                                        \
        if (!(cond)) return fail(NNHIP_ERR_INVALID_ARG, fn, msg);            \
    } while (0)

#define NNHIP_LAUNCH(fn, expr)                                               \
    do                                                                       \
    {                                                                        \
        const hipError_t le_ = (expr);                                       \
        if (le_ != hipSuccess) return hip_fail(fn, "kernel launch", le_);    \
    } while (0)

constexpr size_t kMaxDim = 0x7FFFFFFFull;  // kernels index rows/tokens with int32
// The decode GEMV accumulates 16*sum(code*x) in int32: 16 * 381 * K < 2^31.
constexpr size_t kMaxK = 262144;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool mul_ok(size_t a, size_t b) { return a == 0 || b <= SIZE_MAX / a; }

// Grow a context-owned device buffer to at least `bytes` (waits for queued work first, because
// a kernel in flight may still use the old buffer).
nnhip_status ensure_buf(nnhip_ctx* ctx, void*& buf, size_t& have, size_t bytes, const char* fn, const char* what)
{
    if (have >= bytes) return NNHIP_OK;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(fn, "hipStreamSynchronize", e);
    if (buf)
    {
        e = hipFree(buf);
        buf = nullptr;
        have = 0;
        if (e != hipSuccess) return hip_fail(fn, "hipFree", e);
    }
    e = hipMalloc(&buf, bytes);
    if (e != hipSuccess)
    {
        buf = nullptr;
        (void)hipGetLastError();
        return fail(NNHIP_ERR_OOM, fn, std::string(what) + " allocation of " + std::to_string(bytes) + " bytes failed");
    }
    have = bytes;
    return NNHIP_OK;
}

nnhip_status ensure_ws(nnhip_ctx* ctx, size_t bytes, const char* fn)
{
    return ensure_buf(ctx, ctx->ws, ctx->ws_bytes, bytes, fn, "workspace");
}

nnhip_status check_matmul_shape(const char* fn, size_t N, size_t K, size_t M)
{
    NNHIP_REQUIRE(N <= kMaxDim && M <= kMaxDim, fn, "N and M must be below 2^31");
    NNHIP_REQUIRE(K >= 1 && K <= kMaxK, fn, "K must be in [1, 262144]");
    NNHIP_REQUIRE(ceil_div(N, 16) < (1u << 20), fn, "N must be below 2^24");
    NNHIP_REQUIRE(mul_ok(round_up(K, kTileK), M) && mul_ok(N, M), fn, "size overflow");
    // the kernels address rp, xi and Y through 32-bit buffer ranges
    NNHIP_REQUIRE(round_up(N, kTileRows) * round_up(K, kTileK) / 4 < 0x7FFFFFFFull, fn,
                  "repacked weights must be below 2 GiB");
    NNHIP_REQUIRE(round_up(K, kTileK) * M < 0x7FFFFFFFull, fn, "activations must be below 2 GiB");
    NNHIP_REQUIRE(N * M * 4 < 0x7FFFFFFFull, fn, "output must be below 2 GiB");
    return NNHIP_OK;
}

nnhip_status run_matmul(nnhip_ctx* ctx, const char* fn, const void* rp, const float* tau,
                        const int8_t* xi, const float* s, const int32_t* rowsum, const float* bias,
                        size_t N, size_t K, size_t M, float* Y, int glu = 0, size_t glu_F = 0,
                        const float* res = nullptr)
{
    GemvProblem p{};
    p.rp = static_cast<const u32x4*>(rp);
    p.tau = tau;
    p.xi = xi;
    p.s = s;
    p.rowsum = rowsum;
    p.bias = bias;
    p.y = Y;
    p.N = (int32_t)N;
    p.K = (int32_t)K;
    p.M = (int32_t)M;
    p.KT = (int32_t)ceil_div(K, kTileK);
    p.xlds = -1;
    p.glu = glu;
    p.glu_F = (int32_t)glu_F;
    if (res && glu == 0 && M <= (size_t)kGemvMaxM && gemv_deep_ok(p, ctx->num_cus))
    {
        // the residual in the deep GEMV's epilogue
        p.res = res;
        NNHIP_LAUNCH(fn, launch_gemv_deep(ctx->stream, p));
        return NNHIP_OK;
    }
    if (M <= (size_t)kGemvMaxM)
        NNHIP_LAUNCH(fn, launch_gemv(ctx->stream, p, ctx->num_cus));
    else
    {
        // the prefill GEMM adds the residual in its plain epilogue (not in the gated one)
        if (res && glu == 0) p.res = res;
        NNHIP_LAUNCH(fn, launch_gemm(ctx->stream, p, ctx->num_cus, ctx->gemm_tile));
        if (p.res) return NNHIP_OK;
    }
    if (res) NNHIP_LAUNCH(fn, launch_add(ctx->stream, res, Y, N * M, Y));
    return NNHIP_OK;
}

}  // namespace

extern "C" {

const char* nnhip_last_error(void) { return g_err.c_str(); }

const char* nnhip_version(void) { return "nnhip 0.1.0 gfx950"; }

uint64_t nnhip_fnv1a64(const void* data, size_t bytes)
{
    const uint8_t* p = static_cast<const uint8_t*>(data);
    uint64_t h = 1469598103934665603ull;
    for (size_t i = 0; i < bytes && p; ++i)
    {
        h ^= p[i];
        h *= 1099511628211ull;
    }
    return h;
}

nnhip_status nnhip_device_count(int* count)
{
    if (!count) return fail(NNHIP_ERR_INVALID_ARG, "nnhip_device_count", "null output");
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess)
    {
        (void)hipGetLastError();
        *count = 0;
        return fail(NNHIP_ERR_NO_DEVICE, "nnhip_device_count", hipGetErrorString(e));
    }
    *count = n;
    return NNHIP_OK;
}

nnhip_status nnhip_ctx_create(int device, nnhip_ctx** out)
{
    const char* fn = "nnhip_ctx_create";
    NNHIP_REQUIRE(out != nullptr, fn, "null output");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0)
    {
        (void)hipGetLastError();
        return fail(NNHIP_ERR_NO_DEVICE, fn, "no HIP device visible");
    }
    NNHIP_REQUIRE(device >= 0 && device < n, fn, "device index out of range");
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return hip_fail(fn, "hipGetDeviceProperties", e);
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(NNHIP_ERR_NO_DEVICE, fn,
                    std::string("device is ") + prop.gcnArchName + ", this library is built for gfx950 only");
    e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail(fn, "hipSetDevice", e);
    void* scr = nullptr;
    const nnhip_status sst = resolve_scratch(device, &scr, fn);
    if (sst != NNHIP_OK) return sst;
    auto* ctx = new nnhip_ctx;
    ctx->device = device;
    ctx->scratch = scr;
    ctx->num_cus = prop.multiProcessorCount;
    e = hipStreamCreateWithFlags(&ctx->own, hipStreamNonBlocking);
    if (e != hipSuccess)
    {
        delete ctx;
        return hip_fail(fn, "hipStreamCreate", e);
    }
    ctx->stream = ctx->own;
    *out = ctx;
    return NNHIP_OK;
}

nnhip_status nnhip_ctx_destroy(nnhip_ctx* ctx)
{
    const char* fn = "nnhip_ctx_destroy";
    if (!ctx) return NNHIP_OK;
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->attn_ws) (void)hipFree(ctx->attn_ws);
    if (ctx->ones) (void)hipFree(ctx->ones);
    if (ctx->own) (void)hipStreamDestroy(ctx->own);
    delete ctx;
    if (e != hipSuccess) return hip_fail(fn, "hipStreamSynchronize", e);
    return NNHIP_OK;
}

nnhip_status nnhip_ctx_set_stream(nnhip_ctx* ctx, void* stream)
{
    NNHIP_CHECK_CTX("nnhip_ctx_set_stream");
    ctx->stream = static_cast<hipStream_t>(stream);
    return NNHIP_OK;
}

nnhip_status nnhip_ctx_reset_stream(nnhip_ctx* ctx)
{
    NNHIP_CHECK_CTX("nnhip_ctx_reset_stream");
    ctx->stream = ctx->own;
    return NNHIP_OK;
}

nnhip_status nnhip_ctx_get_stream(nnhip_ctx* ctx, void** stream)
{
    NNHIP_CHECK_CTX("nnhip_ctx_get_stream");
    NNHIP_REQUIRE(stream != nullptr, "nnhip_ctx_get_stream", "null output");
    *stream = ctx->stream;
    return NNHIP_OK;
}

nnhip_status nnhip_ctx_set_gemm_tile(nnhip_ctx* ctx, int tile)
{
    NNHIP_CHECK_CTX("nnhip_ctx_set_gemm_tile");
    NNHIP_REQUIRE(tile >= NNHIP_GEMM_TILE_AUTO && tile <= NNHIP_GEMM_TILE_64x64, "nnhip_ctx_set_gemm_tile",
                  "tile must be one of NNHIP_GEMM_TILE_*");
    ctx->gemm_tile = tile;
    return NNHIP_OK;
}

nnhip_status nnhip_ctx_prefetch_next(nnhip_ctx* ctx, size_t count, const void* const* ptrs, const size_t* bytes)
{
    const char* fn = "nnhip_ctx_prefetch_next";
    NNHIP_CHECK_CTX(fn);
    NNHIP_REQUIRE(count <= (size_t)kPfRanges, fn, "count must be at most 4");
    NNHIP_REQUIRE(count == 0 || (ptrs && bytes), fn, "null pointer");
    Prefetch p{};
    uint64_t total = 0;
    int k = 0;
    for (size_t i = 0; i < count; ++i)
    {
        if (!ptrs[i] || bytes[i] < 16) continue;
        NNHIP_REQUIRE(aligned16(ptrs[i]), fn, "ranges must be 16-byte aligned");
        // whole 16-byte units inside the range, at most kPfMaxUnits over all ranges
        const uint64_t n = std::min<uint64_t>(bytes[i] / 16, kPfMaxUnits - total);
        if (n == 0) continue;
        p.p[k] = ptrs[i];
        p.n16[k] = (uint32_t)n;
        total += n;
        ++k;
    }
    p.blocks = (int)ceil_div((size_t)total, (size_t)kOneThreadsHost * kPfUnitsPerThread);
    ctx->pf = p;
    return NNHIP_OK;
}

nnhip_status nnhip_sync(nnhip_ctx* ctx)
{
    NNHIP_CHECK_CTX("nnhip_sync");
    const hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail("nnhip_sync", "hipStreamSynchronize", e);
    return NNHIP_OK;
}

nnhip_status nnhip_malloc(nnhip_ctx* ctx, size_t bytes, void** out)
{
    const char* fn = "nnhip_malloc";
    NNHIP_CHECK_CTX(fn);
    NNHIP_REQUIRE(out != nullptr, fn, "null output");
    *out = nullptr;
    if (bytes == 0) return NNHIP_OK;
    const hipError_t e = hipMalloc(out, bytes);
    if (e != hipSuccess)
    {
        *out = nullptr;
        (void)hipGetLastError();
        return fail(NNHIP_ERR_OOM, fn, "allocation of " + std::to_string(bytes) + " bytes failed");
    }
    return NNHIP_OK;
}

nnhip_status nnhip_free(nnhip_ctx* ctx, void* ptr)
{
    NNHIP_CHECK_CTX("nnhip_free");
    if (!ptr) return NNHIP_OK;
    const hipError_t e = hipFree(ptr);
    if (e != hipSuccess) return hip_fail("nnhip_free", "hipFree", e);
    return NNHIP_OK;
}

static nnhip_status copy_sync(nnhip_ctx* ctx, const char* fn, void* dst, const void* src, size_t bytes,
                              hipMemcpyKind kind)
{
    NNHIP_CHECK_CTX(fn);
    if (bytes == 0) return NNHIP_OK;
    NNHIP_REQUIRE(dst && src, fn, "null pointer");
    hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, ctx->stream);
    if (e != hipSuccess) return hip_fail(fn, "hipMemcpyAsync", e);
    if (kind != hipMemcpyDeviceToDevice)
    {
        e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) return hip_fail(fn, "hipStreamSynchronize", e);
    }
    return NNHIP_OK;
}

nnhip_status nnhip_memcpy_h2d(nnhip_ctx* ctx, void* dst, const void* src, size_t bytes)
{
    return copy_sync(ctx, "nnhip_memcpy_h2d", dst, src, bytes, hipMemcpyHostToDevice);
}

nnhip_status nnhip_memcpy_d2h(nnhip_ctx* ctx, void* dst, const void* src, size_t bytes)
{
    return copy_sync(ctx, "nnhip_memcpy_d2h", dst, src, bytes, hipMemcpyDeviceToHost);
}

nnhip_status nnhip_memcpy_d2d(nnhip_ctx* ctx, void* dst, const void* src, size_t bytes)
{
    return copy_sync(ctx, "nnhip_memcpy_d2d", dst, src, bytes, hipMemcpyDeviceToDevice);
}

nnhip_status nnhip_stream_xor(nnhip_ctx* ctx, const void* src, size_t bytes, uint32_t* out)
{
    const char* fn = "nnhip_stream_xor";
    NNHIP_CHECK_CTX(fn);
    if (bytes == 0) return NNHIP_OK;
    NNHIP_REQUIRE(src && out, fn, "null pointer");
    NNHIP_REQUIRE(aligned16(src), fn, "src must be 16-byte aligned");
    NNHIP_REQUIRE((reinterpret_cast<uintptr_t>(out) & 3u) == 0, fn, "out must be 4-byte aligned");
    NNHIP_REQUIRE(bytes % 4 == 0, fn, "bytes must be a multiple of 4");
    nnhip_status st = ensure_ws(ctx, stream_xor_blocks(bytes, ctx->num_cus) * 4, fn);
    if (st != NNHIP_OK) return st;
    NNHIP_LAUNCH(fn, launch_stream_xor(ctx->stream, src, bytes, static_cast<uint32_t*>(ctx->ws), out, ctx->num_cus));
    return NNHIP_OK;
}

nnhip_status nnhip_device_info(int device, int* cus, int* clock_khz, int* mem_clock_khz, int* bus_bits)
{
    const char* fn = "nnhip_device_info";
    NNHIP_REQUIRE(cus && clock_khz && mem_clock_khz && bus_bits, fn, "null output");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0)
    {
        (void)hipGetLastError();
        return fail(NNHIP_ERR_NO_DEVICE, fn, "no HIP device visible");
    }
    NNHIP_REQUIRE(device >= 0 && device < n, fn, "device index out of range");
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return hip_fail(fn, "hipGetDeviceProperties", e);
    *cus = prop.multiProcessorCount;
    *clock_khz = prop.clockRate;
    *mem_clock_khz = prop.memoryClockRate;
    *bus_bits = prop.memoryBusWidth;
    return NNHIP_OK;
}

nnhip_status nnhip_device_name(int device, char* buf, size_t len)
{
    const char* fn = "nnhip_device_name";
    NNHIP_REQUIRE(buf && len > 0, fn, "null or empty output buffer");
    buf[0] = '\0';
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0)
    {
        (void)hipGetLastError();
        return fail(NNHIP_ERR_NO_DEVICE, fn, "no HIP device visible");
    }
    NNHIP_REQUIRE(device >= 0 && device < n, fn, "device index out of range");
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return hip_fail(fn, "hipGetDeviceProperties", e);
    std::snprintf(buf, len, "%s (%s)", prop.name, prop.gcnArchName);
    return NNHIP_OK;
}

nnhip_status nnhip_convert_f32_f16(nnhip_ctx* ctx, const float* src, size_t n, uint16_t* dst)
{
    const char* fn = "nnhip_convert_f32_f16";
    NNHIP_CHECK_CTX(fn);
    if (n == 0) return NNHIP_OK;
    NNHIP_REQUIRE(src && dst, fn, "null pointer");
    NNHIP_LAUNCH(fn, launch_f32_to_f16(ctx->stream, src, n, dst));
    return NNHIP_OK;
}

nnhip_status nnhip_convert_f16_f32(nnhip_ctx* ctx, const uint16_t* src, size_t n, float* dst)
{
    const char* fn = "nnhip_convert_f16_f32";
    NNHIP_CHECK_CTX(fn);
    if (n == 0) return NNHIP_OK;
    NNHIP_REQUIRE(src && dst, fn, "null pointer");
    NNHIP_LAUNCH(fn, launch_f16_to_f32(ctx->stream, src, n, dst));
    return NNHIP_OK;
}

nnhip_status nnhip_fill_u32(nnhip_ctx* ctx, void* dst, uint32_t value, size_t words)
{
    const char* fn = "nnhip_fill_u32";
    NNHIP_CHECK_CTX(fn);
    if (words == 0) return NNHIP_OK;
    NNHIP_REQUIRE(dst != nullptr, fn, "null pointer");
    NNHIP_REQUIRE((reinterpret_cast<uintptr_t>(dst) & 3u) == 0, fn, "dst must be 4-byte aligned");
    NNHIP_LAUNCH(fn, launch_fill_u32(ctx->stream, static_cast<uint32_t*>(dst), value, words));
    return NNHIP_OK;
}

// ------------------------------------------------------------- reference-layout primitives

nnhip_status nnhip_row_absmean(nnhip_ctx* ctx, const float* W, size_t N, size_t K, float* tau)
{
    const char* fn = "nnhip_row_absmean";
    NNHIP_CHECK_CTX(fn);
    if (N == 0) return NNHIP_OK;
    NNHIP_REQUIRE(K >= 1, fn, "K must be >= 1");
    NNHIP_REQUIRE(W && tau, fn, "null pointer");
    NNHIP_REQUIRE(mul_ok(N, K), fn, "size overflow");
    NNHIP_LAUNCH(fn, launch_row_absmean(ctx->stream, W, N, K, tau));
    return NNHIP_OK;
}

nnhip_status nnhip_trit_pack(nnhip_ctx* ctx, const float* W, const float* tau, size_t N, size_t K,
                             uint32_t* wq)
{
    const char* fn = "nnhip_trit_pack";
    NNHIP_CHECK_CTX(fn);
    if (N == 0 || K == 0) return NNHIP_OK;
    NNHIP_REQUIRE(W && tau && wq, fn, "null pointer");
    NNHIP_REQUIRE(mul_ok(N, K), fn, "size overflow");
    NNHIP_LAUNCH(fn, launch_trit_pack(ctx->stream, W, tau, N, K, wq));
    return NNHIP_OK;
}

nnhip_status nnhip_col_reduce_max(nnhip_ctx* ctx, const float* x, size_t rows, size_t cols, float* out)
{
    const char* fn = "nnhip_col_reduce_max";
    NNHIP_CHECK_CTX(fn);
    if (cols == 0) return NNHIP_OK;
    NNHIP_REQUIRE(out && (x || rows == 0), fn, "null pointer");
    NNHIP_REQUIRE(mul_ok(rows, cols), fn, "size overflow");
    NNHIP_LAUNCH(fn, launch_col_reduce_max(ctx->stream, x, rows, cols, out, false, 1.0f));
    return NNHIP_OK;
}

nnhip_status nnhip_abs(nnhip_ctx* ctx, const float* x, size_t n, float* out)
{
    const char* fn = "nnhip_abs";
    NNHIP_CHECK_CTX(fn);
    if (n == 0) return NNHIP_OK;
    NNHIP_REQUIRE(x && out, fn, "null pointer");
    NNHIP_LAUNCH(fn, launch_abs(ctx->stream, x, n, out));
    return NNHIP_OK;
}

nnhip_status nnhip_scale_inplace(nnhip_ctx* ctx, float* x, size_t n, float alpha)
{
    const char* fn = "nnhip_scale_inplace";
    NNHIP_CHECK_CTX(fn);
    if (n == 0) return NNHIP_OK;
    NNHIP_REQUIRE(x != nullptr, fn, "null pointer");
    NNHIP_LAUNCH(fn, launch_scale(ctx->stream, x, n, alpha));
    return NNHIP_OK;
}

nnhip_status nnhip_act_scale(nnhip_ctx* ctx, const float* X, size_t K, size_t M, float* s)
{
    const char* fn = "nnhip_act_scale";
    NNHIP_CHECK_CTX(fn);
    if (M == 0) return NNHIP_OK;
    NNHIP_REQUIRE(s && (X || K == 0), fn, "null pointer");
    NNHIP_REQUIRE(mul_ok(K, M), fn, "size overflow");
    NNHIP_LAUNCH(fn, launch_col_reduce_max(ctx->stream, X, K, M, s, true, 1.0f / 127.0f));
    return NNHIP_OK;
}

nnhip_status nnhip_quantize_i8(nnhip_ctx* ctx, const float* x, const float* scale, size_t rows,
                               size_t cols, int col_scale, uint32_t* out)
{
    const char* fn = "nnhip_quantize_i8";
    NNHIP_CHECK_CTX(fn);
    if (rows == 0 || cols == 0) return NNHIP_OK;
    NNHIP_REQUIRE(x && scale && out, fn, "null pointer");
    NNHIP_REQUIRE(mul_ok(rows, cols), fn, "size overflow");
    NNHIP_LAUNCH(fn, launch_quantize_i8(ctx->stream, x, scale, rows, cols, col_scale != 0, out));
    return NNHIP_OK;
}

nnhip_status nnhip_unpack_i8(nnhip_ctx* ctx, const uint32_t* packed, size_t rows, size_t cols, float* out)
{
    const char* fn = "nnhip_unpack_i8";
    NNHIP_CHECK_CTX(fn);
    if (rows == 0 || cols == 0) return NNHIP_OK;
    NNHIP_REQUIRE(packed && out, fn, "null pointer");
    NNHIP_REQUIRE(mul_ok(rows, cols), fn, "size overflow");
    NNHIP_LAUNCH(fn, launch_unpack_i8(ctx->stream, packed, rows, cols, out));
    return NNHIP_OK;
}

nnhip_status nnhip_matmul_q_i8(nnhip_ctx* ctx, const uint32_t* wq, const float* tau, const uint32_t* xq,
                               const float* s, size_t N, size_t K, size_t M, float* Y)
{
    const char* fn = "nnhip_matmul_q_i8";
    NNHIP_CHECK_CTX(fn);
    if (N == 0 || M == 0) return NNHIP_OK;
    nnhip_status st = check_matmul_shape(fn, N, K, M);
    if (st != NNHIP_OK) return st;
    NNHIP_REQUIRE(wq && tau && xq && s && Y, fn, "null pointer");
    const size_t rp_bytes = round_up(nnhip_repacked_bytes(N, K), 256);
    const size_t xi_bytes = round_up(nnhip_act_i8_bytes(K, M), 256);
    const size_t rs_bytes = round_up(M * sizeof(int32_t), 256);
    st = ensure_ws(ctx, rp_bytes + xi_bytes + rs_bytes, fn);
    if (st != NNHIP_OK) return st;
    uint8_t* base = static_cast<uint8_t*>(ctx->ws);
    uint32_t* rp = reinterpret_cast<uint32_t*>(base);
    int8_t* xi = reinterpret_cast<int8_t*>(base + rp_bytes);
    int32_t* rowsum = reinterpret_cast<int32_t*>(base + rp_bytes + xi_bytes);
    NNHIP_LAUNCH(fn, launch_repack(ctx->stream, wq, N, K, rp));
    NNHIP_LAUNCH(fn, launch_act_from_container(ctx->stream, xq, K, M, xi, rowsum));
    return run_matmul(ctx, fn, rp, tau, xi, s, rowsum, nullptr, N, K, M, Y);
}

nnhip_status nnhip_matmul_q_i8_noalloc(nnhip_ctx* ctx, const uint32_t* wq, const float* tau, const uint32_t* xq,
                                       const float* s, size_t N, size_t K, size_t M, float* Y)
{
    const char* fn = "nnhip_matmul_q_i8_noalloc";
    NNHIP_CHECK_CTX(fn);
    if (N == 0 || M == 0) return NNHIP_OK;
    nnhip_status st = check_matmul_shape(fn, N, K, M);
    if (st != NNHIP_OK) return st;
    NNHIP_REQUIRE(wq && tau && xq && s && Y, fn, "null pointer");
    NNHIP_REQUIRE(ctx->scratch != nullptr, fn, "scratch address not resolved");
    // the same split of the scratch as nnhip_matmul_q_i8's workspace
    const size_t rp_bytes = round_up(nnhip_repacked_bytes(N, K), 256);
    const size_t xi_bytes = round_up(nnhip_act_i8_bytes(K, M), 256);
    const size_t rs_bytes = round_up(M * sizeof(int32_t), 256);
    const size_t need = rp_bytes + xi_bytes + rs_bytes;
    if (need > (size_t)NNHIP_NOALLOC_SCRATCH_BYTES)
        return fail(NNHIP_ERR_UNSUPPORTED, fn,
                    "needs " + std::to_string(need) + " bytes of scratch (repacked weights " + std::to_string(rp_bytes) +
                        " + activations " + std::to_string(xi_bytes + rs_bytes) + "), more than the " +
                        std::to_string((size_t)NNHIP_NOALLOC_SCRATCH_BYTES) + " bytes this entry point has");
    // every byte used below is written by the repack / transpose before the product reads it
    // (pad codes and zero pad included), so the previous call's contents need no clearing
    uint8_t* base = static_cast<uint8_t*>(ctx->scratch);
    uint32_t* rp = reinterpret_cast<uint32_t*>(base);
    int8_t* xi = reinterpret_cast<int8_t*>(base + rp_bytes);
    int32_t* rowsum = reinterpret_cast<int32_t*>(base + rp_bytes + xi_bytes);
    NNHIP_LAUNCH(fn, launch_repack(ctx->stream, wq, N, K, rp));
    NNHIP_LAUNCH(fn, launch_act_from_container(ctx->stream, xq, K, M, xi, rowsum));
    return run_matmul(ctx, fn, rp, tau, xi, s, rowsum, nullptr, N, K, M, Y);
}

nnhip_status nnhip_matmul_q(nnhip_ctx* ctx, const uint32_t* wq, const float* tau, const void* B, int b_f16,
                            size_t N, size_t K, size_t M, void* Y, int y_f16)
{
    const char* fn = "nnhip_matmul_q";
    NNHIP_CHECK_CTX(fn);
    if (N == 0 || M == 0) return NNHIP_OK;
    NNHIP_REQUIRE(wq && tau && B && Y, fn, "null pointer");
    NNHIP_REQUIRE(K >= 1 && N <= kMaxDim && M <= kMaxDim && K <= kMaxDim, fn, "bad shape");
    NNHIP_REQUIRE(mul_ok(N, ceil_div(K, 16)) && mul_ok(K, M) && mul_ok(N, M), fn, "size overflow");
    const MatqPlan plan = plan_matmul_q(N, K, M);
    if (plan.part_bytes)
    {
        const nnhip_status st = ensure_ws(ctx, plan.part_bytes, fn);
        if (st != NNHIP_OK) return st;
    }
    NNHIP_LAUNCH(fn, launch_matmul_q(ctx->stream, wq, tau, B, b_f16 != 0, N, K, M, Y, y_f16 != 0, plan,
                                     static_cast<float*>(ctx->ws)));
    return NNHIP_OK;
}

nnhip_status nnhip_matmul_q_t(nnhip_ctx* ctx, const uint32_t* A, const float* tau, const void* B, int b_f16,
                              size_t K, size_t M, size_t N, void* Y, int y_f16)
{
    const char* fn = "nnhip_matmul_q_t";
    NNHIP_CHECK_CTX(fn);
    if (N == 0 || M == 0) return NNHIP_OK;
    NNHIP_REQUIRE(A && tau && B && Y, fn, "null pointer");
    NNHIP_REQUIRE(K >= 1 && N <= kMaxDim && M <= kMaxDim && K <= kMaxDim, fn, "bad shape");
    NNHIP_REQUIRE(mul_ok(K, ceil_div(M, 16)) && mul_ok(K, N) && mul_ok(M, N), fn, "size overflow");
    const MatqPlan plan = plan_matmul_q_t(K, M, N);
    if (plan.part_bytes)
    {
        const nnhip_status st = ensure_ws(ctx, plan.part_bytes, fn);
        if (st != NNHIP_OK) return st;
    }
    NNHIP_LAUNCH(fn, launch_matmul_q_t(ctx->stream, A, tau, B, b_f16 != 0, K, M, N, Y, y_f16 != 0, plan,
                                       static_cast<float*>(ctx->ws)));
    return NNHIP_OK;
}

nnhip_status nnhip_add_row_broadcast(nnhip_ctx* ctx, float* Y, const float* b, size_t N, size_t M)
{
    const char* fn = "nnhip_add_row_broadcast";
    NNHIP_CHECK_CTX(fn);
    if (N == 0 || M == 0) return NNHIP_OK;
    NNHIP_REQUIRE(Y && b, fn, "null pointer");
    NNHIP_REQUIRE(mul_ok(N, M), fn, "size overflow");
    NNHIP_LAUNCH(fn, launch_add_row_broadcast(ctx->stream, Y, b, N, M));
    return NNHIP_OK;
}

nnhip_status nnhip_rmsnorm(nnhip_ctx* ctx, const float* X, const float* gamma, float eps, size_t F,
                           size_t M, float* out)
{
    const char* fn = "nnhip_rmsnorm";
    NNHIP_CHECK_CTX(fn);
    if (M == 0 || F == 0) return NNHIP_OK;
    NNHIP_REQUIRE(X && gamma && out, fn, "null pointer");
    NNHIP_REQUIRE(F <= kMaxDim && M <= kMaxDim && mul_ok(F, M), fn, "size overflow");
    NNHIP_LAUNCH(fn, launch_rmsnorm(ctx->stream, X, gamma, eps, F, M, out));
    return NNHIP_OK;
}

nnhip_status nnhip_layernorm(nnhip_ctx* ctx, const float* X, const float* gamma, const float* beta, float eps,
                             size_t F, size_t M, float* out)
{
    const char* fn = "nnhip_layernorm";
    NNHIP_CHECK_CTX(fn);
    if (M == 0 || F == 0) return NNHIP_OK;
    NNHIP_REQUIRE(X && gamma && beta && out, fn, "null pointer");
    NNHIP_REQUIRE(F <= kMaxDim && M <= kMaxDim && mul_ok(F, M), fn, "size overflow");
    NNHIP_LAUNCH(fn, launch_layernorm(ctx->stream, X, gamma, beta, eps, F, M, out));
    return NNHIP_OK;
}

// ------------------------------------------------------------- MI355X-native fast path

size_t nnhip_repacked_bytes(size_t N, size_t K)
{
    return round_up(N, kTileRows) * round_up(K, kTileK) / 4;
}

nnhip_status nnhip_repack_ternary(nnhip_ctx* ctx, const uint32_t* wq, size_t N, size_t K, void* rp)
{
    const char* fn = "nnhip_repack_ternary";
    NNHIP_CHECK_CTX(fn);
    if (N == 0 || K == 0) return NNHIP_OK;
    NNHIP_REQUIRE(wq && rp, fn, "null pointer");
    NNHIP_REQUIRE(aligned16(rp), fn, "rp must be 16-byte aligned");
    NNHIP_REQUIRE(mul_ok(round_up(N, 16), round_up(K, kTileK)), fn, "size overflow");
    NNHIP_LAUNCH(fn, launch_repack(ctx->stream, wq, N, K, static_cast<uint32_t*>(rp)));
    return NNHIP_OK;
}

nnhip_status nnhip_unrepack_ternary(nnhip_ctx* ctx, const void* rp, size_t N, size_t K, uint32_t* wq)
{
    const char* fn = "nnhip_unrepack_ternary";
    NNHIP_CHECK_CTX(fn);
    if (N == 0 || K == 0) return NNHIP_OK;
    NNHIP_REQUIRE(wq && rp, fn, "null pointer");
    NNHIP_REQUIRE(aligned16(rp), fn, "rp must be 16-byte aligned");
    NNHIP_LAUNCH(fn, launch_unrepack(ctx->stream, static_cast<const uint32_t*>(rp), N, K, wq));
    return NNHIP_OK;
}

size_t nnhip_act_i8_bytes(size_t K, size_t M) { return round_up(K, kTileK) * M; }

static nnhip_status act_quant_common(nnhip_ctx* ctx, const char* fn, const float* X, const float* gamma,
                                     bool norm, float eps, size_t K, size_t M, int8_t* xi, float* s,
                                     int32_t* rowsum, uint32_t* xq_ref)
{
    NNHIP_CHECK_CTX(fn);
    const Prefetch pf = take_prefetch(ctx);
    if (M == 0) return NNHIP_OK;
    NNHIP_REQUIRE(K >= 1 && K <= kMaxK && M <= kMaxDim, fn, "K must be in [1, 262144], M below 2^31");
    NNHIP_REQUIRE(X && xi && s && rowsum && (gamma || !norm), fn, "null pointer");
    NNHIP_REQUIRE(aligned16(xi), fn, "xi must be 16-byte aligned");
    NNHIP_REQUIRE(mul_ok(round_up(K, kTileK), M), fn, "size overflow");
    NNHIP_LAUNCH(fn, launch_act_quant(ctx->stream, X, gamma, norm, eps, K, M, xi, s, rowsum, xq_ref, &pf));
    return NNHIP_OK;
}

nnhip_status nnhip_act_quant_i8(nnhip_ctx* ctx, const float* X, size_t K, size_t M, int8_t* xi, float* s,
                                int32_t* rowsum, uint32_t* xq_ref)
{
    return act_quant_common(ctx, "nnhip_act_quant_i8", X, nullptr, false, 0.0f, K, M, xi, s, rowsum,
                            xq_ref);
}

nnhip_status nnhip_rmsnorm_quant_i8(nnhip_ctx* ctx, const float* X, const float* gamma, float eps,
                                    size_t F, size_t M, int8_t* xi, float* s, int32_t* rowsum,
                                    uint32_t* xq_ref)
{
    return act_quant_common(ctx, "nnhip_rmsnorm_quant_i8", X, gamma, true, eps, F, M, xi, s, rowsum,
                            xq_ref);
}

nnhip_status nnhip_act_i8_from_container(nnhip_ctx* ctx, const uint32_t* xq, size_t K, size_t M,
                                         int8_t* xi, int32_t* rowsum)
{
    const char* fn = "nnhip_act_i8_from_container";
    NNHIP_CHECK_CTX(fn);
    if (M == 0) return NNHIP_OK;
    NNHIP_REQUIRE(K >= 1 && K <= kMaxK && M <= kMaxDim, fn, "K must be in [1, 262144], M below 2^31");
    NNHIP_REQUIRE(xq && xi && rowsum, fn, "null pointer");
    NNHIP_REQUIRE(aligned16(xi), fn, "xi must be 16-byte aligned");
    NNHIP_LAUNCH(fn, launch_act_from_container(ctx->stream, xq, K, M, xi, rowsum));
    return NNHIP_OK;
}

nnhip_status nnhip_act_i8_to_container(nnhip_ctx* ctx, const int8_t* xi, size_t K, size_t M, uint32_t* xq)
{
    const char* fn = "nnhip_act_i8_to_container";
    NNHIP_CHECK_CTX(fn);
    if (M == 0 || K == 0) return NNHIP_OK;
    NNHIP_REQUIRE(K <= kMaxK && M <= kMaxDim, fn, "K must be <= 262144, M below 2^31");
    NNHIP_REQUIRE(xq && xi, fn, "null pointer");
    NNHIP_LAUNCH(fn, launch_act_to_container(ctx->stream, xi, K, M, xq));
    return NNHIP_OK;
}

nnhip_status nnhip_ternary_matmul(nnhip_ctx* ctx, const void* rp, const float* tau, const int8_t* xi,
                                  const float* s, const int32_t* rowsum, const float* bias, size_t N,
                                  size_t K, size_t M, float* Y)
{
    const char* fn = "nnhip_ternary_matmul";
    NNHIP_CHECK_CTX(fn);
    if (N == 0 || M == 0) return NNHIP_OK;
    const nnhip_status st = check_matmul_shape(fn, N, K, M);
    if (st != NNHIP_OK) return st;
    NNHIP_REQUIRE(rp && tau && xi && s && rowsum && Y, fn, "null pointer");
    NNHIP_REQUIRE(aligned16(rp) && aligned16(xi), fn, "rp and xi must be 16-byte aligned");
    return run_matmul(ctx, fn, rp, tau, xi, s, rowsum, bias, N, K, M, Y);
}

// Slices of the split-k digit path, or 0 for the unit-scale GEMV / GEMM. It takes a few long
// tokens (M <= 4, so the 4M digit tokens are one GEMV column block) with a long reduction
// (K >= 6144) over few output rows (at most 2048 row tiles): there the whole-K GEMV runs one wave
// per 16-row tile through K / 256 sequential k tiles, too few waves to hide memory latency. The
// slices keep every slice within 14 k tiles and give at least two blocks of four row tiles per CU.
static int digit_split_slices(size_t N, size_t K, size_t M, int num_cus)
{
    const size_t KT = ceil_div(K, kTileK), RT = ceil_div(N, 16);
    if (M < 1 || M > 4 || KT < 24 || RT > 2048) return 0;
    const size_t row_groups = ceil_div(RT, 4);
    const size_t cus = num_cus > 0 ? (size_t)num_cus : 256;
    size_t S = ceil_div(KT, 14);
    if (row_groups * S < 2 * cus) S = ceil_div(2 * cus, row_groups);
    if (S > 32) S = 32;
    if (S > KT) S = KT;
    GemvProblem p{};
    p.N = (int32_t)N;
    p.M = (int32_t)(4 * M);
    p.KT = (int32_t)KT;
    for (; S >= 1; --S)
        if (gemv_part_ok(p, (int)S)) return (int)S;
    return 0;
}

static nnhip_status matmul_digits(nnhip_ctx* ctx, const char* fn, const void* rp, const float* tau,
                                  const float* kscale, const void* B, int b_f16, size_t N, size_t K, size_t M, void* Y,
                                  int y_f16)
{
    NNHIP_CHECK_CTX(fn);
    if (N == 0 || M == 0) return NNHIP_OK;
    nnhip_status st = check_matmul_shape(fn, N, K, M);
    if (st != NNHIP_OK) return st;
    NNHIP_REQUIRE(rp && B && Y, fn, "null pointer");
    NNHIP_REQUIRE(aligned16(rp), fn, "rp must be 16-byte aligned");
    NNHIP_REQUIRE(M <= kMaxDim / 4 && mul_ok(N, 4 * M), fn, "size overflow");
    // the digit products are exact integers in f32 while 128 K < 2^24
    if (K >= 131072) return fail(NNHIP_ERR_UNSUPPORTED, fn, "K must be below 131072 (use nnhip_matmul_q)");
    if (digit_gemv_ok(N, K, M, b_f16 != 0, B))
    {
        NNHIP_LAUNCH(fn, launch_digit_gemv(ctx->stream, rp, tau, kscale, static_cast<const float*>(B), N, K, M, Y,
                                           y_f16 != 0));
        return NNHIP_OK;
    }
    const size_t Kp = round_up(K, kTileK), M4 = 4 * M;
    const int S = digit_split_slices(N, K, M, ctx->num_cus);
    if (S > 0)
    {
        // a few long tokens: the digits in column chunks, the GEMV as split-k int32 slice sums, and
        // a combine that adds both (exact integers: the same bits as the path below)
        const size_t P = digit_chunks(K);
        const size_t b_xi = round_up(M4 * Kp, 256), b_rsp = round_up(M * P * 16, 256), b_ex = round_up(M * 4, 256);
        const size_t b_part = (size_t)S * M4 * N * 4;
        st = ensure_ws(ctx, b_xi + b_rsp + b_ex + b_part, fn);
        if (st != NNHIP_OK) return st;
        uint8_t* w = static_cast<uint8_t*>(ctx->ws);
        int8_t* xi = reinterpret_cast<int8_t*>(w);
        int32_t* rsp = reinterpret_cast<int32_t*>(w + b_xi);
        int32_t* ex = reinterpret_cast<int32_t*>(w + b_xi + b_rsp);
        int32_t* part = reinterpret_cast<int32_t*>(w + b_xi + b_rsp + b_ex);
        NNHIP_LAUNCH(fn, launch_digits_chunks(ctx->stream, B, b_f16 != 0, kscale, K, M, xi, rsp, ex));
        GemvProblem p{};
        p.rp = static_cast<const u32x4*>(rp);
        p.xi = xi;
        p.N = (int32_t)N;
        p.K = (int32_t)K;
        p.M = (int32_t)M4;
        p.KT = (int32_t)ceil_div(K, kTileK);
        p.xlds = -1;
        NNHIP_LAUNCH(fn, launch_gemv_part(ctx->stream, p, S, part));
        NNHIP_LAUNCH(fn, launch_digit_combine_parts(ctx->stream, part, S, rsp, P, tau, ex, static_cast<const uint32_t*>(rp),
                                                    B, b_f16 != 0, kscale, N, K, M, Y, y_f16 != 0));
        return NNHIP_OK;
    }
    const size_t b_xi = round_up(M4 * Kp, 256), b_rs = round_up(M4 * 4, 256), b_ex = round_up(M * 4, 256);
    const size_t b_yp = N * M4 * 4;
    st = ensure_ws(ctx, b_xi + b_rs + b_ex + b_yp, fn);
    if (st != NNHIP_OK) return st;
    const size_t ones = N > M4 ? N : M4;
    if (ctx->ones_words < ones)
    {
        st = ensure_buf(ctx, reinterpret_cast<void*&>(ctx->ones), ctx->ones_bytes_, ones * 4, fn, "unit scales");
        if (st != NNHIP_OK) return st;
        NNHIP_LAUNCH(fn, launch_fill_u32(ctx->stream, reinterpret_cast<uint32_t*>(ctx->ones), 0x3F800000u, ones));
        ctx->ones_words = ones;
    }
    uint8_t* w = static_cast<uint8_t*>(ctx->ws);
    int8_t* xi = reinterpret_cast<int8_t*>(w);
    int32_t* rs = reinterpret_cast<int32_t*>(w + b_xi);
    int32_t* ex = reinterpret_cast<int32_t*>(w + b_xi + b_rs);
    float* yp = reinterpret_cast<float*>(w + b_xi + b_rs + b_ex);
    NNHIP_LAUNCH(fn, launch_digits(ctx->stream, B, b_f16 != 0, kscale, K, M, xi, rs, ex));
    st = run_matmul(ctx, fn, rp, ctx->ones, xi, ctx->ones, rs, nullptr, N, K, M4, yp);
    if (st != NNHIP_OK) return st;
    NNHIP_LAUNCH(fn, launch_digit_combine(ctx->stream, yp, tau, ex, static_cast<const uint32_t*>(rp), B, b_f16 != 0,
                                          kscale, N, K, M, Y, y_f16 != 0));
    return NNHIP_OK;
}

nnhip_status nnhip_ternary_matmul_f(nnhip_ctx* ctx, const void* rp, const float* tau, const void* B, int b_f16,
                                    size_t N, size_t K, size_t M, void* Y, int y_f16)
{
    const char* fn = "nnhip_ternary_matmul_f";
    NNHIP_REQUIRE(tau != nullptr || N == 0 || M == 0, fn, "null tau");
    return matmul_digits(ctx, fn, rp, tau, nullptr, B, b_f16, N, K, M, Y, y_f16);
}

nnhip_status nnhip_ternary_matmul_t_f(nnhip_ctx* ctx, const void* rpT, const float* tau, const void* B, int b_f16,
                                      size_t K, size_t M, size_t N, void* Y, int y_f16)
{
    const char* fn = "nnhip_ternary_matmul_t_f";
    NNHIP_REQUIRE(tau != nullptr || M == 0 || N == 0, fn, "null tau");
    return matmul_digits(ctx, fn, rpT, nullptr, tau, B, b_f16, M, K, N, Y, y_f16);
}

nnhip_status nnhip_trit_transpose(nnhip_ctx* ctx, const uint32_t* A, size_t K, size_t M, uint32_t* At)
{
    const char* fn = "nnhip_trit_transpose";
    NNHIP_CHECK_CTX(fn);
    if (K == 0 || M == 0) return NNHIP_OK;
    NNHIP_REQUIRE(A && At, fn, "null pointer");
    NNHIP_REQUIRE(K <= kMaxDim && M <= kMaxDim, fn, "size out of range");
    NNHIP_LAUNCH(fn, launch_trit_transpose(ctx->stream, A, K, M, At));
    return NNHIP_OK;
}

nnhip_status nnhip_ternary_matmul_add_tokens(nnhip_ctx* ctx, const void* rp, const float* tau, const int8_t* xi,
                                             const float* s, const int32_t* rowsum, const float* bias, const float* res,
                                             size_t N, size_t K, size_t M, float* Y)
{
    const char* fn = "nnhip_ternary_matmul_add_tokens";
    NNHIP_CHECK_CTX(fn);
    if (N == 0 || M == 0) return NNHIP_OK;
    const nnhip_status st = check_matmul_shape(fn, N, K, M);
    if (st != NNHIP_OK) return st;
    NNHIP_REQUIRE(rp && tau && xi && s && rowsum && res && Y, fn, "null pointer");
    NNHIP_REQUIRE(res != Y, fn, "res must not alias Y");
    NNHIP_REQUIRE(aligned16(rp) && aligned16(xi), fn, "rp and xi must be 16-byte aligned");
    GemvProblem p{};
    p.rp = static_cast<const u32x4*>(rp);
    p.tau = tau;
    p.xi = xi;
    p.s = s;
    p.rowsum = rowsum;
    p.bias = bias;
    p.y = Y;
    p.N = (int32_t)N;
    p.K = (int32_t)K;
    p.M = (int32_t)M;
    p.KT = (int32_t)ceil_div(K, kTileK);
    p.xlds = -1;
    p.res = res;
    p.ytm = 1;
    if (M > (size_t)kGemvMaxM || !gemv_deep_ok(p, ctx->num_cus))
        return fail(NNHIP_ERR_UNSUPPORTED, fn,
                    "decode sizes only (M <= 16, K of 1024 / 2560 / 4096 / 6912 rounded to 256, at most 4 row tiles per CU)");
    NNHIP_LAUNCH(fn, launch_gemv_deep(ctx->stream, p));
    return NNHIP_OK;
}

nnhip_status nnhip_ternary_matmul_add(nnhip_ctx* ctx, const void* rp, const float* tau, const int8_t* xi,
                                      const float* s, const int32_t* rowsum, const float* bias, const float* res,
                                      size_t N, size_t K, size_t M, float* Y)
{
    const char* fn = "nnhip_ternary_matmul_add";
    NNHIP_CHECK_CTX(fn);
    if (N == 0 || M == 0) return NNHIP_OK;
    const nnhip_status st = check_matmul_shape(fn, N, K, M);
    if (st != NNHIP_OK) return st;
    NNHIP_REQUIRE(rp && tau && xi && s && rowsum && res && Y, fn, "null pointer");
    NNHIP_REQUIRE(res != Y, fn, "res must not alias Y");
    NNHIP_REQUIRE(aligned16(rp) && aligned16(xi), fn, "rp and xi must be 16-byte aligned");
    return run_matmul(ctx, fn, rp, tau, xi, s, rowsum, bias, N, K, M, Y, 0, 0, res);
}

nnhip_status nnhip_ternary_matmul_partial(nnhip_ctx* ctx, const void* rp, const int8_t* xi, size_t N, size_t K,
                                          size_t M, size_t slices, int32_t* part)
{
    const char* fn = "nnhip_ternary_matmul_partial";
    NNHIP_CHECK_CTX(fn);
    if (N == 0 || M == 0) return NNHIP_OK;
    const nnhip_status st = check_matmul_shape(fn, N, K, M);
    if (st != NNHIP_OK) return st;
    NNHIP_REQUIRE(rp && xi && part, fn, "null pointer");
    NNHIP_REQUIRE(aligned16(rp) && aligned16(xi), fn, "rp and xi must be 16-byte aligned");
    NNHIP_REQUIRE(M <= (size_t)kGemvMaxM, fn, "M must be at most 16");
    NNHIP_REQUIRE(slices >= 1 && slices <= 8, fn, "slices must be in [1, 8]");
    NNHIP_REQUIRE(mul_ok(slices * M, N) && slices * M * N * 4 < 0x7FFFFFFFull, fn, "part must stay below 2^31 bytes");
    GemvProblem p{};
    p.rp = static_cast<const u32x4*>(rp);
    p.xi = xi;
    p.N = (int32_t)N;
    p.K = (int32_t)K;
    p.M = (int32_t)M;
    p.KT = (int32_t)ceil_div(K, kTileK);
    p.xlds = -1;
    NNHIP_REQUIRE(gemv_part_ok(p, (int)slices), fn, "every slice must hold at least one k tile of at most 14");
    NNHIP_LAUNCH(fn, launch_gemv_part(ctx->stream, p, (int)slices, part));
    return NNHIP_OK;
}

static nnhip_status partial_residual_common(nnhip_ctx* ctx, const char* fn, const int32_t* part, size_t slices,
                                            const float* tau, const float* s_in, const int32_t* rowsum_in,
                                            const float* bias, const float* res, size_t N, size_t M, float* x_out,
                                            const float* gamma, float eps, int8_t* xi, float* s, int32_t* rowsum,
                                            bool tm)
{
    NNHIP_CHECK_CTX(fn);
    const Prefetch pf = take_prefetch(ctx);
    if (N == 0 || M == 0) return NNHIP_OK;
    NNHIP_REQUIRE(part && tau && s_in && rowsum_in && x_out && xi && s && rowsum, fn, "null pointer");
    NNHIP_REQUIRE(slices >= 1 && slices <= 8, fn, "slices must be in [1, 8]");
    NNHIP_REQUIRE(epilogue_quant_ok(N, M), fn, "needs M <= 64 and N <= 11264");
    NNHIP_REQUIRE(aligned16(xi), fn, "xi must be 16-byte aligned");
    NNHIP_REQUIRE(!gamma || eps >= 0.0f, fn, "eps must be >= 0");
    const EpiArgs e{part, (int)slices, tau, s_in, rowsum_in, bias, res, x_out, tm ? 1 : 0};
    NNHIP_LAUNCH(fn, launch_epilogue_quant(ctx->stream, e, gamma, gamma != nullptr, eps, N, M, xi, s, rowsum, &pf));
    return NNHIP_OK;
}

nnhip_status nnhip_partial_residual_quant_i8(nnhip_ctx* ctx, const int32_t* part, size_t slices, const float* tau,
                                             const float* s_in, const int32_t* rowsum_in, const float* bias,
                                             const float* res, size_t N, size_t M, float* x_out,
                                             const float* gamma, float eps, int8_t* xi, float* s, int32_t* rowsum)
{
    return partial_residual_common(ctx, "nnhip_partial_residual_quant_i8", part, slices, tau, s_in, rowsum_in, bias,
                                   res, N, M, x_out, gamma, eps, xi, s, rowsum, false);
}

nnhip_status nnhip_partial_residual_quant_i8_tokens(nnhip_ctx* ctx, const int32_t* part, size_t slices,
                                                    const float* tau, const float* s_in, const int32_t* rowsum_in,
                                                    const float* bias, const float* res, size_t N, size_t M,
                                                    float* x_out, const float* gamma, float eps, int8_t* xi, float* s,
                                                    int32_t* rowsum)
{
    return partial_residual_common(ctx, "nnhip_partial_residual_quant_i8_tokens", part, slices, tau, s_in, rowsum_in,
                                   bias, res, N, M, x_out, gamma, eps, xi, s, rowsum, true);
}

static nnhip_status matmul_n_common(nnhip_ctx* ctx, const char* fn, size_t count, const void* const* rp,
                                    const float* const* tau, const float* const* bias, const size_t* N,
                                    float* const* Y, const int8_t* xi, const float* s, const int32_t* rowsum, size_t K,
                                    size_t M, bool tm)
{
    NNHIP_CHECK_CTX(fn);
    if (count == 0 || M == 0) return NNHIP_OK;
    NNHIP_REQUIRE(count <= (size_t)kGemvDeepMulti, fn, "count must be in [1, 4]");
    NNHIP_REQUIRE(rp && tau && N && Y && xi && s && rowsum, fn, "null pointer");
    NNHIP_REQUIRE(aligned16(xi), fn, "xi must be 16-byte aligned");
    GemvProblem ps[kGemvDeepMulti]{};
    for (size_t i = 0; i < count; ++i)
    {
        const nnhip_status st = check_matmul_shape(fn, N[i], K, M);
        if (st != NNHIP_OK) return st;
        NNHIP_REQUIRE(N[i] >= 1 && rp[i] && tau[i] && Y[i], fn, "null pointer or empty problem");
        NNHIP_REQUIRE(aligned16(rp[i]), fn, "rp must be 16-byte aligned");
        GemvProblem& p = ps[i];
        p.rp = static_cast<const u32x4*>(rp[i]);
        p.tau = tau[i];
        p.xi = xi;
        p.s = s;
        p.rowsum = rowsum;
        p.bias = bias ? bias[i] : nullptr;
        p.y = Y[i];
        p.N = (int32_t)N[i];
        p.K = (int32_t)K;
        p.M = (int32_t)M;
        p.KT = (int32_t)ceil_div(K, kTileK);
        p.xlds = -1;
        p.ytm = tm ? 1 : 0;
    }
    if (M <= (size_t)kGemvMaxM && gemv_deep_multi_ok(ps, (int)count, ctx->num_cus))
    {
        NNHIP_LAUNCH(fn, launch_gemv_deep_multi(ctx->stream, ps, (int)count));
        return NNHIP_OK;
    }
    if (tm)
        return fail(NNHIP_ERR_UNSUPPORTED, fn,
                    "decode sizes only (M <= 16, K of 1024 / 2560 / 4096 / 6912 rounded to 256, at most 4 row tiles per CU)");
    for (size_t i = 0; i < count; ++i)
    {
        const nnhip_status st = run_matmul(ctx, fn, rp[i], tau[i], xi, s, rowsum, bias ? bias[i] : nullptr, N[i], K, M,
                                           Y[i]);
        if (st != NNHIP_OK) return st;
    }
    return NNHIP_OK;
}

nnhip_status nnhip_ternary_matmul_n(nnhip_ctx* ctx, size_t count, const void* const* rp, const float* const* tau,
                                    const float* const* bias, const size_t* N, float* const* Y, const int8_t* xi,
                                    const float* s, const int32_t* rowsum, size_t K, size_t M)
{
    return matmul_n_common(ctx, "nnhip_ternary_matmul_n", count, rp, tau, bias, N, Y, xi, s, rowsum, K, M, false);
}

nnhip_status nnhip_ternary_matmul_n_tokens(nnhip_ctx* ctx, size_t count, const void* const* rp,
                                           const float* const* tau, const float* const* bias, const size_t* N,
                                           float* const* Y, const int8_t* xi, const float* s, const int32_t* rowsum,
                                           size_t K, size_t M)
{
    return matmul_n_common(ctx, "nnhip_ternary_matmul_n_tokens", count, rp, tau, bias, N, Y, xi, s, rowsum, K, M, true);
}

nnhip_status nnhip_group_create(nnhip_ctx* ctx, const nnhip_gemv_desc* descs, size_t count,
                                nnhip_group** out)
{
    const char* fn = "nnhip_group_create";
    NNHIP_CHECK_CTX(fn);
    NNHIP_REQUIRE(out != nullptr, fn, "null output");
    *out = nullptr;
    NNHIP_REQUIRE(descs != nullptr || count == 0, fn, "null descriptors");
    NNHIP_REQUIRE(count < (1u << 12), fn, "at most 4095 problems per group");
    std::vector<GemvProblem> probs(count);
    for (size_t i = 0; i < count; ++i)
    {
        const nnhip_gemv_desc& d = descs[i];
        const nnhip_status st = check_matmul_shape(fn, d.N, d.K, d.M);
        if (st != NNHIP_OK) return st;
        NNHIP_REQUIRE(d.M >= 1 && d.M <= (uint64_t)kGemvMaxM, fn, "grouped GEMV needs 1 <= M <= 16");
        NNHIP_REQUIRE(d.rp && d.tau && d.xi && d.s && d.rowsum && d.y, fn, "null pointer in descriptor");
        NNHIP_REQUIRE(aligned16(d.rp) && aligned16(d.xi), fn, "rp and xi must be 16-byte aligned");
        GemvProblem& p = probs[i];
        p.rp = static_cast<const u32x4*>(d.rp);
        p.tau = d.tau;
        p.xi = d.xi;
        p.s = d.s;
        p.rowsum = d.rowsum;
        p.bias = d.bias;
        p.y = d.y;
        p.N = (int32_t)d.N;
        p.K = (int32_t)d.K;
        p.M = (int32_t)d.M;
        p.KT = (int32_t)ceil_div(d.K, kTileK);
        p.xlds = -1;
    }

    // Distinct activation blocks. If they fit the LDS budget together, one launch stages them all
    // and reads its B operands from LDS (LDS variant); if they fit kGemvLdsBigBudget together, one
    // launch of 16-wave blocks (one per CU) does. Otherwise the blocks that fit are packed, first
    // fit in order, into LDS launches of their own problems; a block over the budget but within
    // kGemvLdsBigBudget gets an LDS launch of its own with 16-wave blocks; the problems of still
    // larger blocks go to one launch of the register variant (activations loaded with the
    // weights). The launches run one after another on the stream.
    struct Part
    {
        std::vector<size_t> probs;  // indices into probs
        std::vector<XStage> xstage;
        uint32_t lds = 0;
    };
    std::vector<Part> parts;
    {
        std::vector<XStage> distinct;
        std::vector<int> act_of(count);
        for (size_t i = 0; i < count; ++i)
        {
            const GemvProblem& p = probs[i];
            const uint32_t bytes = (uint32_t)p.M * (uint32_t)p.KT * kTileK;
            int found = -1;
            for (size_t e = 0; e < distinct.size(); ++e)
                if (distinct[e].src == p.xi && distinct[e].bytes == bytes) found = (int)e;
            if (found < 0)
            {
                distinct.push_back(XStage{p.xi, bytes, 0, (uint32_t)p.KT * kTileK});
                found = (int)distinct.size() - 1;
            }
            act_of[i] = found;
        }
        std::vector<int> part_of(distinct.size(), -1);  // LDS part of each activation block
        int reg_part = -1;
        uint32_t total = 0;
        for (const XStage& x : distinct) total += x.bytes;
        // all blocks together within the 16-wave budget: one launch of 16-wave blocks stages them
        const bool one_big = total > kGemvLdsBudget && total <= kGemvLdsBigBudget;
        for (size_t e = 0; e < distinct.size(); ++e)
        {
            XStage x = distinct[e];
            if (one_big)
            {
                if (parts.empty()) parts.push_back(Part{});
                x.lds_off = parts[0].lds;
                parts[0].xstage.push_back(x);
                parts[0].lds += x.bytes;
                part_of[e] = 0;
                continue;
            }
            if (x.bytes > kGemvLdsBigBudget) continue;  // register variant
            if (x.bytes > kGemvLdsBudget)
            {
                // a launch of its own with 16-wave blocks, one per CU
                parts.push_back(Part{});
                x.lds_off = 0;
                parts.back().xstage.push_back(x);
                parts.back().lds = x.bytes;
                part_of[e] = (int)parts.size() - 1;
                continue;
            }
            int target = -1;
            if (total <= kGemvLdsBudget)
                target = parts.empty() ? -1 : 0;
            else
                for (size_t q = 0; q < parts.size(); ++q)
                    if (!parts[q].xstage.empty() && parts[q].lds <= kGemvLdsBudget &&
                        parts[q].lds + x.bytes <= kGemvLdsBudget)
                        target = (int)q;
            if (target < 0)
            {
                parts.push_back(Part{});
                target = (int)parts.size() - 1;
            }
            x.lds_off = parts[target].lds;
            parts[target].xstage.push_back(x);
            parts[target].lds += x.bytes;
            part_of[e] = target;
        }
        for (size_t i = 0; i < count; ++i)
        {
            const int e = act_of[i];
            if (part_of[e] >= 0)
            {
                Part& pt = parts[part_of[e]];
                for (const XStage& x : pt.xstage)
                    if (x.src == distinct[e].src && x.bytes == distinct[e].bytes) probs[i].xlds = (int32_t)x.lds_off;
                pt.probs.push_back(i);
            }
            else
            {
                if (reg_part < 0)
                {
                    parts.push_back(Part{});
                    reg_part = (int)parts.size() - 1;
                }
                parts[reg_part].probs.push_back(i);
            }
        }
    }

    auto* grp = new nnhip_group;
    auto release = [&]() {
        for (nnhip_group::Launch& l : grp->launches)
        {
            (void)hipFree(l.d_probs);
            (void)hipFree(l.d_wave_start);
            (void)hipFree(l.d_wave_items);
            (void)hipFree(l.d_xstage);
        }
        delete grp;
    };
    for (const Part& pt : parts)
    {
        const bool use_lds = !pt.xstage.empty();
        const GemvVariant var = gemv_variant(use_lds);
        std::vector<GemvProblem> lp;
        for (const size_t i : pt.probs) lp.push_back(probs[i]);
        std::vector<uint32_t> items;
        for (size_t i = 0; i < lp.size(); ++i)
        {
            const size_t rts = ceil_div((size_t)lp[i].N, 16);
            for (size_t rt = 0; rt < rts; rt += (size_t)var.row_tiles) items.push_back((uint32_t)((i << 20) | rt));
        }
        if (items.size() >= 0x7FFFFFFFull)
        {
            release();
            return fail(NNHIP_ERR_INVALID_ARG, fn, "too many row tiles");
        }

        // Longest-processing-time schedule: items (var.row_tiles row tiles of one problem) by
        // decreasing cost (weight tiles + 1 for the epilogue), each to the currently
        // least-loaded wave. Waves = the variant's resident wave slots.
        const size_t n_waves = items.empty() ? 0 : gemv_grid_waves(items.size(), ctx->num_cus, use_lds);
        std::vector<uint32_t> wave_start(n_waves + 1, 0), wave_items(items.size());
        if (n_waves > 0)
        {
            auto cost = [&](uint32_t it) {
                const GemvProblem& p = lp[it >> 20];
                const uint64_t rts = std::min<uint64_t>((uint64_t)var.row_tiles, ceil_div(p.N, 16) - (it & 0xFFFFFu));
                return (uint64_t)p.KT * rts + 1;
            };
            std::stable_sort(items.begin(), items.end(), [&](uint32_t a, uint32_t b) { return cost(a) > cost(b); });
            using Slot = std::pair<uint64_t, uint32_t>;  // (load, wave)
            std::priority_queue<Slot, std::vector<Slot>, std::greater<Slot>> heap;
            for (uint32_t w = 0; w < n_waves; ++w) heap.push({0, w});
            std::vector<std::vector<uint32_t>> lists(n_waves);
            for (const uint32_t it : items)
            {
                Slot sl = heap.top();
                heap.pop();
                lists[sl.second].push_back(it);
                sl.first += cost(it);
                heap.push(sl);
            }
            size_t pos = 0;
            for (size_t w = 0; w < n_waves; ++w)
            {
                wave_start[w] = (uint32_t)pos;
                for (const uint32_t it : lists[w]) wave_items[pos++] = it;
            }
            wave_start[n_waves] = (uint32_t)pos;
        }
        if (n_waves == 0) continue;

        nnhip_group::Launch l;
        l.n_waves = n_waves;
        l.n_xstage = (int)pt.xstage.size();
        l.lds_bytes = pt.lds;
        grp->launches.push_back(l);
        nnhip_group::Launch& L = grp->launches.back();
        hipError_t e = hipMalloc(&L.d_probs, sizeof(GemvProblem) * lp.size());
        if (e == hipSuccess && use_lds) e = hipMalloc(&L.d_xstage, sizeof(XStage) * pt.xstage.size());
        if (e == hipSuccess && use_lds)
            e = hipMemcpyAsync(L.d_xstage, pt.xstage.data(), sizeof(XStage) * pt.xstage.size(), hipMemcpyHostToDevice,
                               ctx->stream);
        if (e == hipSuccess) e = hipMalloc(&L.d_wave_start, sizeof(uint32_t) * wave_start.size());
        if (e == hipSuccess) e = hipMalloc(&L.d_wave_items, sizeof(uint32_t) * wave_items.size());
        if (e == hipSuccess)
            e = hipMemcpyAsync(L.d_probs, lp.data(), sizeof(GemvProblem) * lp.size(), hipMemcpyHostToDevice,
                               ctx->stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(L.d_wave_start, wave_start.data(), sizeof(uint32_t) * wave_start.size(),
                               hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(L.d_wave_items, wave_items.data(), sizeof(uint32_t) * wave_items.size(),
                               hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess)
        {
            release();
            return hip_fail(fn, "descriptor upload", e);
        }
    }
    *out = grp;
    return NNHIP_OK;
}

nnhip_status nnhip_group_run(nnhip_ctx* ctx, nnhip_group* group)
{
    const char* fn = "nnhip_group_run";
    NNHIP_CHECK_CTX(fn);
    NNHIP_REQUIRE(group != nullptr, fn, "null group");
    for (const nnhip_group::Launch& l : group->launches)
        NNHIP_LAUNCH(fn, launch_gemv_grouped(ctx->stream, l.d_probs, l.d_wave_start, l.d_wave_items, l.n_waves,
                                             l.d_xstage, l.n_xstage, l.lds_bytes));
    return NNHIP_OK;
}

nnhip_status nnhip_group_destroy(nnhip_ctx* ctx, nnhip_group* group)
{
    const char* fn = "nnhip_group_destroy";
    NNHIP_CHECK_CTX(fn);
    if (!group) return NNHIP_OK;
    const hipError_t e = hipStreamSynchronize(ctx->stream);
    for (const nnhip_group::Launch& l : group->launches)
    {
        (void)hipFree(l.d_probs);
        (void)hipFree(l.d_wave_start);
        (void)hipFree(l.d_wave_items);
        (void)hipFree(l.d_xstage);
    }
    delete group;
    if (e != hipSuccess) return hip_fail(fn, "hipStreamSynchronize", e);
    return NNHIP_OK;
}

nnhip_status nnhip_group_info(const nnhip_group* group, int* lds_variant, size_t* waves, size_t* lds_bytes)
{
    const char* fn = "nnhip_group_info";
    NNHIP_REQUIRE(group != nullptr, fn, "null group");
    size_t n_lds = 0, n_waves = 0, lds_max = 0;
    for (const nnhip_group::Launch& l : group->launches)
    {
        n_lds += l.n_xstage > 0 ? 1 : 0;
        n_waves += l.n_waves;
        lds_max = std::max<size_t>(lds_max, l.lds_bytes);
    }
    if (lds_variant) *lds_variant = n_lds == 0 ? 0 : (n_lds == group->launches.size() ? 1 : 2);
    if (waves) *waves = n_waves;
    if (lds_bytes) *lds_bytes = lds_max;
    return NNHIP_OK;
}

size_t nnhip_gemv_grid_waves(nnhip_ctx* ctx, size_t items)
{
    return gemv_grid_waves(items, ctx ? ctx->num_cus : 256, true);
}

}  // extern "C"

// ------------------------------------------------------------- gated feed-forward block

namespace
{

// fc1 + gated activation into h (F, M); y1 is scratch of glu_rows(F) x M floats, used only by
// the decode (GEMV) path, whose epilogue writes the plain interleaved rows first.
nnhip_status run_matmul_glu(nnhip_ctx* ctx, const char* fn, const void* rp, const float* tau, const int8_t* xi,
                            const float* s, const int32_t* rowsum, const float* bias, size_t F, size_t K, size_t M,
                            int act, float* y1, float* h)
{
    const size_t N = nnhip_glu_rows(F);
    if (M <= (size_t)kGemvMaxM)
    {
        GemvProblem p{};
        p.rp = static_cast<const u32x4*>(rp);
        p.tau = tau;
        p.xi = xi;
        p.s = s;
        p.rowsum = rowsum;
        p.bias = bias;
        p.y = h;
        p.N = (int32_t)N;
        p.K = (int32_t)K;
        p.M = (int32_t)M;
        p.KT = (int32_t)ceil_div(K, kTileK);
        p.xlds = -1;
        p.glu = act + 1;
        p.glu_F = (int32_t)F;
        if (gemv_deep_ok(p, ctx->num_cus))
        {
            // the gated activation in the deep GEMV's epilogue: no y1 round trip
            NNHIP_LAUNCH(fn, launch_gemv_deep(ctx->stream, p));
            return NNHIP_OK;
        }
        const nnhip_status st = run_matmul(ctx, fn, rp, tau, xi, s, rowsum, bias, N, K, M, y1);
        if (st != NNHIP_OK) return st;
        NNHIP_LAUNCH(fn, launch_glu(ctx->stream, y1, F, M, act, true, h));
        return NNHIP_OK;
    }
    return run_matmul(ctx, fn, rp, tau, xi, s, rowsum, bias, N, K, M, h, act + 1, F);
}

nnhip_status check_glu_args(const char* fn, size_t F, size_t K, size_t M, int act)
{
    NNHIP_REQUIRE(act == NNHIP_ACT_SWIGLU || act == NNHIP_ACT_RELU2GLU, fn, "act must be NNHIP_ACT_SWIGLU or NNHIP_ACT_RELU2GLU");
    NNHIP_REQUIRE(F >= 1 && F <= kMaxDim / 4, fn, "F must be in [1, 2^29)");
    NNHIP_REQUIRE(mul_ok(F, M) && F * M * 4 < 0x7FFFFFFFull, fn, "gated output must be below 2 GiB");
    return check_matmul_shape(fn, nnhip_glu_rows(F), K, M);
}

}  // namespace

extern "C" {

size_t nnhip_glu_rows(size_t F) { return 2 * round_up(F, 8); }

nnhip_status nnhip_glu(nnhip_ctx* ctx, const float* Y1, size_t F, size_t M, int act, float* h)
{
    const char* fn = "nnhip_glu";
    NNHIP_CHECK_CTX(fn);
    if (F == 0 || M == 0) return NNHIP_OK;
    NNHIP_REQUIRE(Y1 && h, fn, "null pointer");
    NNHIP_REQUIRE(act == NNHIP_ACT_SWIGLU || act == NNHIP_ACT_RELU2GLU, fn, "act must be NNHIP_ACT_SWIGLU or NNHIP_ACT_RELU2GLU");
    NNHIP_REQUIRE(mul_ok(2 * F, M), fn, "size overflow");
    NNHIP_LAUNCH(fn, launch_glu(ctx->stream, Y1, F, M, act, false, h));
    return NNHIP_OK;
}

nnhip_status nnhip_glu_interleave(nnhip_ctx* ctx, const uint32_t* wq, const float* tau, const float* bias, size_t F,
                                  size_t K, uint32_t* wq_out, float* tau_out, float* bias_out)
{
    const char* fn = "nnhip_glu_interleave";
    NNHIP_CHECK_CTX(fn);
    if (F == 0 || K == 0) return NNHIP_OK;
    NNHIP_REQUIRE(wq && tau && wq_out && tau_out, fn, "null pointer");
    NNHIP_REQUIRE(!bias || bias_out, fn, "bias_out is required when bias is given");
    NNHIP_REQUIRE(F <= kMaxDim / 4 && mul_ok(nnhip_glu_rows(F), ceil_div(K, 16)), fn, "size overflow");
    NNHIP_LAUNCH(fn, launch_glu_interleave(ctx->stream, wq, tau, bias, F, K, wq_out, tau_out, bias_out));
    return NNHIP_OK;
}

nnhip_status nnhip_ternary_matmul_glu(nnhip_ctx* ctx, const void* rp, const float* tau, const int8_t* xi,
                                      const float* s, const int32_t* rowsum, const float* bias, size_t F, size_t K,
                                      size_t M, int act, float* h)
{
    const char* fn = "nnhip_ternary_matmul_glu";
    NNHIP_CHECK_CTX(fn);
    if (F == 0 || M == 0) return NNHIP_OK;
    nnhip_status st = check_glu_args(fn, F, K, M, act);
    if (st != NNHIP_OK) return st;
    NNHIP_REQUIRE(rp && tau && xi && s && rowsum && h, fn, "null pointer");
    NNHIP_REQUIRE(aligned16(rp) && aligned16(xi), fn, "rp and xi must be 16-byte aligned");
    float* y1 = nullptr;
    if (M <= (size_t)kGemvMaxM)
    {
        st = ensure_ws(ctx, nnhip_glu_rows(F) * M * sizeof(float), fn);
        if (st != NNHIP_OK) return st;
        y1 = static_cast<float*>(ctx->ws);
    }
    return run_matmul_glu(ctx, fn, rp, tau, xi, s, rowsum, bias, F, K, M, act, y1, h);
}

nnhip_status nnhip_ternary_matmul_glu_tokens(nnhip_ctx* ctx, const void* rp, const float* tau, const int8_t* xi,
                                             const float* s, const int32_t* rowsum, const float* bias, size_t F,
                                             size_t K, size_t M, int act, float* h)
{
    const char* fn = "nnhip_ternary_matmul_glu_tokens";
    NNHIP_CHECK_CTX(fn);
    if (F == 0 || M == 0) return NNHIP_OK;
    const nnhip_status st = check_glu_args(fn, F, K, M, act);
    if (st != NNHIP_OK) return st;
    NNHIP_REQUIRE(rp && tau && xi && s && rowsum && h, fn, "null pointer");
    NNHIP_REQUIRE(aligned16(rp) && aligned16(xi), fn, "rp and xi must be 16-byte aligned");
    GemvProblem p{};
    p.rp = static_cast<const u32x4*>(rp);
    p.tau = tau;
    p.xi = xi;
    p.s = s;
    p.rowsum = rowsum;
    p.bias = bias;
    p.y = h;
    p.N = (int32_t)nnhip_glu_rows(F);
    p.K = (int32_t)K;
    p.M = (int32_t)M;
    p.KT = (int32_t)ceil_div(K, kTileK);
    p.xlds = -1;
    p.glu = act + 1;
    p.glu_F = (int32_t)F;
    p.ytm = 1;
    if (M > (size_t)kGemvMaxM || !gemv_deep_ok(p, ctx->num_cus))
        return fail(NNHIP_ERR_UNSUPPORTED, fn,
                    "decode sizes only (M <= 16, K of 1024 / 2560 / 4096 / 6912 rounded to 256, at most 4 row tiles per CU)");
    NNHIP_LAUNCH(fn, launch_gemv_deep(ctx->stream, p));
    return NNHIP_OK;
}

nnhip_status nnhip_rmsnorm_quant_i8_tokens(nnhip_ctx* ctx, const float* X, const float* gamma, float eps, size_t K,
                                           size_t M, int8_t* xi, float* s, int32_t* rowsum)
{
    const char* fn = "nnhip_rmsnorm_quant_i8_tokens";
    NNHIP_CHECK_CTX(fn);
    const Prefetch pf = take_prefetch(ctx);
    if (M == 0) return NNHIP_OK;
    NNHIP_REQUIRE(X && xi && s && rowsum, fn, "null pointer");
    NNHIP_REQUIRE(aligned16(xi), fn, "xi must be 16-byte aligned");
    if (!token_quant_tm_ok(K, M))
        return fail(NNHIP_ERR_UNSUPPORTED, fn, "decode sizes only (1 <= M <= 64, 1 <= K <= 11264)");
    NNHIP_LAUNCH(fn, launch_token_quant_tm(ctx->stream, X, gamma, eps, K, M, xi, s, rowsum, &pf));
    return NNHIP_OK;
}

nnhip_status nnhip_embedding_rmsnorm_quant_i8_tokens(nnhip_ctx* ctx, const float* table, const int32_t* ids,
                                                     size_t V, size_t d, size_t B, const float* gamma, float eps,
                                                     float* x, int8_t* xi, float* s, int32_t* rowsum)
{
    const char* fn = "nnhip_embedding_rmsnorm_quant_i8_tokens";
    NNHIP_CHECK_CTX(fn);
    const Prefetch pf = take_prefetch(ctx);
    if (B == 0) return NNHIP_OK;
    NNHIP_REQUIRE(table && ids && x && xi && s && rowsum, fn, "null pointer");
    NNHIP_REQUIRE(aligned16(xi), fn, "xi must be 16-byte aligned");
    NNHIP_REQUIRE(V >= 1 && V <= kMaxDim && mul_ok(V, d) && V * d < 0x7FFFFFFFull, fn, "table must be below 2^31 elements");
    if (!token_quant_tm_ok(d, B))
        return fail(NNHIP_ERR_UNSUPPORTED, fn, "decode sizes only (1 <= B <= 64, 1 <= d <= 11264)");
    NNHIP_LAUNCH(fn, launch_embed_token_quant(ctx->stream, table, ids, V, gamma, eps, d, B, x, xi, s, rowsum, &pf));
    return NNHIP_OK;
}

size_t nnhip_ffn_glu_workspace_bytes(size_t d, size_t F, size_t M)
{
    size_t b = round_up(nnhip_act_i8_bytes(d, M), 256) + round_up(nnhip_act_i8_bytes(F, M), 256);
    b += 4 * round_up(M * 4, 256);                 // s1, rowsum1, s2, rowsum2
    b += round_up(F * M * 4, 256);                 // h
    if (M <= (size_t)kGemvMaxM) b += round_up(nnhip_glu_rows(F) * M * 4, 256);  // y1 (decode)
    return b;
}

static nnhip_status ffn_glu_i8(nnhip_ctx* ctx, const char* fn, const float* X, const float* gamma, float eps,
                               size_t d, size_t F, size_t M, int act, const void* rp1, const float* tau1,
                               const float* b1, const float* gamma_sub, float eps_sub, const void* rp2,
                               const float* tau2, const float* b2, const float* res, float* Y)
{
    NNHIP_CHECK_CTX(fn);
    if (M == 0 || d == 0) return NNHIP_OK;
    nnhip_status st = check_glu_args(fn, F, d, M, act);
    if (st != NNHIP_OK) return st;
    st = check_matmul_shape(fn, d, F, M);
    if (st != NNHIP_OK) return st;
    NNHIP_REQUIRE(X && rp1 && tau1 && rp2 && tau2 && Y, fn, "null pointer");
    NNHIP_REQUIRE(aligned16(rp1) && aligned16(rp2), fn, "rp1 and rp2 must be 16-byte aligned");
    st = ensure_ws(ctx, nnhip_ffn_glu_workspace_bytes(d, F, M), fn);
    if (st != NNHIP_OK) return st;
    uint8_t* p = static_cast<uint8_t*>(ctx->ws);
    auto take = [&p](size_t bytes) {
        uint8_t* q = p;
        p += round_up(bytes, 256);
        return q;
    };
    int8_t* xi1 = reinterpret_cast<int8_t*>(take(nnhip_act_i8_bytes(d, M)));
    int8_t* xi2 = reinterpret_cast<int8_t*>(take(nnhip_act_i8_bytes(F, M)));
    float* s1 = reinterpret_cast<float*>(take(M * 4));
    int32_t* rs1 = reinterpret_cast<int32_t*>(take(M * 4));
    float* s2 = reinterpret_cast<float*>(take(M * 4));
    int32_t* rs2 = reinterpret_cast<int32_t*>(take(M * 4));
    float* h = reinterpret_cast<float*>(take(F * M * 4));
    float* y1 = M <= (size_t)kGemvMaxM ? reinterpret_cast<float*>(take(nnhip_glu_rows(F) * M * 4)) : nullptr;
    // h is quantized by the fused [RMSNorm ->] absmax -> int8 kernel. (A per-token max |h| folded
    // into fc1's epilogue, with h then quantized in one streaming pass, was slower once the
    // absmax kernel read its rows in contiguous bands: C4 185.4 against 183.3 us, M=64 53.0
    // against 46.6 us, M=16384 1192 against 1182 us, the same outputs.)
    NNHIP_LAUNCH(fn, launch_act_quant(ctx->stream, X, gamma, gamma != nullptr, eps, d, M, xi1, s1, rs1, nullptr));
    st = run_matmul_glu(ctx, fn, rp1, tau1, xi1, s1, rs1, b1, F, d, M, act, y1, h);
    if (st != NNHIP_OK) return st;
    NNHIP_LAUNCH(fn, launch_act_quant(ctx->stream, h, gamma_sub, gamma_sub != nullptr, eps_sub, F, M, xi2, s2, rs2,
                                      nullptr));
    return run_matmul(ctx, fn, rp2, tau2, xi2, s2, rs2, b2, d, F, M, Y, 0, 0, res);
}

nnhip_status nnhip_ffn_glu_i8(nnhip_ctx* ctx, const float* X, const float* gamma, float eps, size_t d, size_t F,
                              size_t M, int act, const void* rp1, const float* tau1, const float* b1,
                              const float* gamma_sub, float eps_sub, const void* rp2, const float* tau2,
                              const float* b2, float* Y)
{
    return ffn_glu_i8(ctx, "nnhip_ffn_glu_i8", X, gamma, eps, d, F, M, act, rp1, tau1, b1, gamma_sub, eps_sub, rp2,
                      tau2, b2, nullptr, Y);
}

nnhip_status nnhip_ffn_glu_i8_add(nnhip_ctx* ctx, const float* X, const float* gamma, float eps, size_t d, size_t F,
                                  size_t M, int act, const void* rp1, const float* tau1, const float* b1,
                                  const float* gamma_sub, float eps_sub, const void* rp2, const float* tau2,
                                  const float* b2, const float* res, float* Y)
{
    const char* fn = "nnhip_ffn_glu_i8_add";
    NNHIP_REQUIRE(res != nullptr, fn, "null residual");
    NNHIP_REQUIRE(res != Y, fn, "res must not alias Y");
    return ffn_glu_i8(ctx, fn, X, gamma, eps, d, F, M, act, rp1, tau1, b1, gamma_sub, eps_sub, rp2, tau2, b2, res, Y);
}

/* ------------------------------------------------ batched decode step */

nnhip_status nnhip_rope_table(size_t dk, size_t max_len, float* cos_out, float* sin_out)
{
    const char* fn = "nnhip_rope_table";
    NNHIP_REQUIRE(dk >= 2 && dk % 2 == 0, fn, "dk must be positive and even");
    NNHIP_REQUIRE(max_len == 0 || (cos_out && sin_out), fn, "null pointer");
    NNHIP_REQUIRE(max_len <= kMaxDim && mul_ok(max_len, dk / 2), fn, "size overflow");
    // RotaryEmbedding::fill_pos_column_ (include/neuralnet.cpp/compute_position_encoding.hpp:64-80),
    // in float like the reference's Scalar: theta = pos / 10000^(2j/dk), cos/sin of it
    const size_t half = dk / 2;
    for (size_t pos = 0; pos < max_len; ++pos)
    {
        const float pd = static_cast<float>(pos);
        for (size_t j = 0; j < half; ++j)
        {
            const float theta = pd / std::pow(10000.0f, static_cast<float>(2 * j) / static_cast<float>(dk));
            cos_out[pos * half + j] = std::cos(theta);
            sin_out[pos * half + j] = std::sin(theta);
        }
    }
    return NNHIP_OK;
}

size_t nnhip_attention_workspace_bytes(size_t B, size_t H, size_t Hkv, size_t dk, size_t len_bound)
{
    if (Hkv == 0 || H % Hkv != 0) return 0;
    return attn_workspace_bytes(B, H, Hkv, dk, len_bound);
}

// Shared argument checks of the decode attention entry points; grows the chunk workspace.
static nnhip_status attention_prep(nnhip_ctx* ctx, const char* fn, const float* q, const float* k, const float* v,
                                   size_t B, size_t H, size_t Hkv, size_t dk, const int32_t* pos, size_t len_bound,
                                   const float* rope_cos, const float* rope_sin, const void* k_cache,
                                   const void* v_cache, size_t max_len, float* out, size_t& wsb)
{
    NNHIP_REQUIRE(q && k && v && pos && k_cache && v_cache && out, fn, "null pointer");
    NNHIP_REQUIRE((rope_cos == nullptr) == (rope_sin == nullptr), fn, "rope_cos and rope_sin go together");
    NNHIP_REQUIRE(dk == 64 || dk == 128 || dk == 256, fn, "dk must be 64, 128 or 256");
    NNHIP_REQUIRE(Hkv >= 1 && H >= Hkv && H % Hkv == 0 && H / Hkv <= 8, fn,
                  "H must be a multiple of Hkv with at most 8 query heads per KV head");
    NNHIP_REQUIRE(B <= 65535 && Hkv <= 65535 && H * dk <= kMaxDim, fn, "B, Hkv or H*dk too large");
    NNHIP_REQUIRE(max_len >= 1 && max_len <= (1u << 24), fn, "max_len must be in [1, 2^24]");
    NNHIP_REQUIRE(len_bound >= 1 && len_bound <= max_len, fn, "len_bound must be in [1, max_len]");
    NNHIP_REQUIRE(mul_ok(B, max_len) && mul_ok(B * max_len, Hkv * dk), fn, "cache size overflow");
    // one sequence's cache is addressed through a 32-bit buffer range
    NNHIP_REQUIRE(max_len * Hkv * dk * 4 < 0x7FFFFFFFull, fn, "max_len * Hkv * dk * 4 must stay below 2^31");
    NNHIP_REQUIRE(aligned16(k_cache) && aligned16(v_cache), fn, "caches must be 16-byte aligned");
    wsb = attn_workspace_bytes(B, H, Hkv, dk, len_bound);
    if (wsb > ctx->attn_ws_bytes)
    {
        const nnhip_status st = ensure_buf(ctx, ctx->attn_ws, ctx->attn_ws_bytes, wsb, fn, "attention workspace");
        if (st != NNHIP_OK) return st;
    }
    return NNHIP_OK;
}

static nnhip_status attention_decode_common(nnhip_ctx* ctx, const char* fn, const float* q, const float* k,
                                            const float* v, size_t B, size_t H, size_t Hkv, size_t dk,
                                            const int32_t* pos, size_t len_bound, const float* rope_cos,
                                            const float* rope_sin, void* k_cache, void* v_cache, bool cache_f16,
                                            size_t max_len, float scale, float* out, bool out_tm)
{
    NNHIP_CHECK_CTX(fn);
    if (B == 0) return NNHIP_OK;
    size_t wsb = 0;
    const nnhip_status st = attention_prep(ctx, fn, q, k, v, B, H, Hkv, dk, pos, len_bound, rope_cos, rope_sin, k_cache,
                                           v_cache, max_len, out, wsb);
    if (st != NNHIP_OK) return st;
    NNHIP_LAUNCH(fn, launch_attn_decode(ctx->stream, q, k, v, B, H, Hkv, dk, pos, len_bound, rope_cos, rope_sin,
                                        k_cache, v_cache, cache_f16, max_len, scale,
                                        wsb ? static_cast<float*>(ctx->attn_ws) : nullptr, out, ctx->num_cus,
                                        out_tm));
    return NNHIP_OK;
}

nnhip_status nnhip_attention_decode(nnhip_ctx* ctx, const float* q, const float* k, const float* v, size_t B,
                                    size_t H, size_t Hkv, size_t dk, const int32_t* pos, size_t len_bound,
                                    const float* rope_cos, const float* rope_sin, float* k_cache, float* v_cache,
                                    size_t max_len, float scale, float* out)
{
    return attention_decode_common(ctx, "nnhip_attention_decode", q, k, v, B, H, Hkv, dk, pos, len_bound, rope_cos,
                                   rope_sin, k_cache, v_cache, false, max_len, scale, out, false);
}

nnhip_status nnhip_attention_decode_h(nnhip_ctx* ctx, const float* q, const float* k, const float* v, size_t B,
                                      size_t H, size_t Hkv, size_t dk, const int32_t* pos, size_t len_bound,
                                      const float* rope_cos, const float* rope_sin, uint16_t* k_cache,
                                      uint16_t* v_cache, size_t max_len, float scale, float* out)
{
    return attention_decode_common(ctx, "nnhip_attention_decode_h", q, k, v, B, H, Hkv, dk, pos, len_bound, rope_cos,
                                   rope_sin, k_cache, v_cache, true, max_len, scale, out, false);
}

nnhip_status nnhip_attention_decode_tokens(nnhip_ctx* ctx, const float* q, const float* k, const float* v, size_t B,
                                           size_t H, size_t Hkv, size_t dk, const int32_t* pos, size_t len_bound,
                                           const float* rope_cos, const float* rope_sin, float* k_cache,
                                           float* v_cache, size_t max_len, float scale, float* out)
{
    return attention_decode_common(ctx, "nnhip_attention_decode_tokens", q, k, v, B, H, Hkv, dk, pos, len_bound,
                                   rope_cos, rope_sin, k_cache, v_cache, false, max_len, scale, out, true);
}

nnhip_status nnhip_attention_decode_tokens_h(nnhip_ctx* ctx, const float* q, const float* k, const float* v, size_t B,
                                             size_t H, size_t Hkv, size_t dk, const int32_t* pos, size_t len_bound,
                                             const float* rope_cos, const float* rope_sin, uint16_t* k_cache,
                                             uint16_t* v_cache, size_t max_len, float scale, float* out)
{
    return attention_decode_common(ctx, "nnhip_attention_decode_tokens_h", q, k, v, B, H, Hkv, dk, pos, len_bound,
                                   rope_cos, rope_sin, k_cache, v_cache, true, max_len, scale, out, true);
}

static nnhip_status kv_cache_fill_common(nnhip_ctx* ctx, const char* fn, const float* k, const float* v, size_t B,
                                         size_t T, size_t Hkv, size_t dk, size_t pos0, const float* rope_cos,
                                         const float* rope_sin, void* k_cache, void* v_cache, bool cache_f16,
                                         size_t max_len)
{
    NNHIP_CHECK_CTX(fn);
    if (B == 0 || T == 0) return NNHIP_OK;
    NNHIP_REQUIRE(k && v && k_cache && v_cache, fn, "null pointer");
    NNHIP_REQUIRE((rope_cos == nullptr) == (rope_sin == nullptr), fn, "rope_cos and rope_sin must both be given or both NULL");
    if (!prefill_dk_supported(dk)) return fail(NNHIP_ERR_UNSUPPORTED, fn, "dk must be 64 or 128");
    NNHIP_REQUIRE(Hkv >= 1 && pos0 + T <= max_len && mul_ok(B, T), fn, "need Hkv >= 1 and pos0 + T <= max_len");
    NNHIP_REQUIRE(B * T <= kMaxDim && mul_ok(Hkv * dk, B * T) && Hkv * dk * B * T < 0x7FFFFFFFull, fn,
                  "k / v must be below 2^31 elements");
    NNHIP_LAUNCH(fn, launch_kv_fill(ctx->stream, k, v, B, T, Hkv, dk, pos0, rope_cos, rope_sin, k_cache, v_cache,
                                    cache_f16, max_len));
    return NNHIP_OK;
}

nnhip_status nnhip_kv_cache_fill(nnhip_ctx* ctx, const float* k, const float* v, size_t B, size_t T, size_t Hkv,
                                 size_t dk, size_t pos0, const float* rope_cos, const float* rope_sin, float* k_cache,
                                 float* v_cache, size_t max_len)
{
    return kv_cache_fill_common(ctx, "nnhip_kv_cache_fill", k, v, B, T, Hkv, dk, pos0, rope_cos, rope_sin, k_cache,
                                v_cache, false, max_len);
}

nnhip_status nnhip_kv_cache_fill_h(nnhip_ctx* ctx, const float* k, const float* v, size_t B, size_t T, size_t Hkv,
                                   size_t dk, size_t pos0, const float* rope_cos, const float* rope_sin,
                                   uint16_t* k_cache, uint16_t* v_cache, size_t max_len)
{
    return kv_cache_fill_common(ctx, "nnhip_kv_cache_fill_h", k, v, B, T, Hkv, dk, pos0, rope_cos, rope_sin, k_cache,
                                v_cache, true, max_len);
}

static nnhip_status attention_prefill_common(nnhip_ctx* ctx, const char* fn, const float* q, const void* k_cache,
                                             const void* v_cache, bool cache_f16, size_t B, size_t T, size_t H,
                                             size_t Hkv, size_t dk, size_t pos0, const float* rope_cos,
                                             const float* rope_sin, size_t max_len, float scale, float* out)
{
    NNHIP_CHECK_CTX(fn);
    if (B == 0 || T == 0) return NNHIP_OK;
    NNHIP_REQUIRE(q && k_cache && v_cache && out, fn, "null pointer");
    NNHIP_REQUIRE((rope_cos == nullptr) == (rope_sin == nullptr), fn, "rope_cos and rope_sin must both be given or both NULL");
    if (!prefill_dk_supported(dk)) return fail(NNHIP_ERR_UNSUPPORTED, fn, "dk must be 64 or 128");
    NNHIP_REQUIRE(Hkv >= 1 && H % Hkv == 0, fn, "H must be a multiple of Hkv");
    const size_t R = H / Hkv;
    if (R != 1 && R != 2 && R != 4 && R != 8)
        return fail(NNHIP_ERR_UNSUPPORTED, fn, "H / Hkv must be 1, 2, 4 or 8");
    NNHIP_REQUIRE(pos0 + T <= max_len && mul_ok(B, T), fn, "need pos0 + T <= max_len");
    NNHIP_REQUIRE(aligned16(k_cache) && aligned16(v_cache), fn, "caches must be 16-byte aligned");
    NNHIP_REQUIRE(B * T <= kMaxDim && mul_ok(H * dk, B * T) && H * dk * B * T < 0x3FFFFFFFull, fn,
                  "q / out must be below 2^30 elements");
    NNHIP_REQUIRE(max_len * Hkv * dk < 0x3FFFFFFFull, fn, "one sequence's cache must be below 2^30 elements");
    NNHIP_LAUNCH(fn, launch_attn_prefill(ctx->stream, q, k_cache, v_cache, cache_f16, B, T, H, Hkv, dk, pos0, rope_cos,
                                         rope_sin, max_len, scale, out));
    return NNHIP_OK;
}

nnhip_status nnhip_attention_prefill(nnhip_ctx* ctx, const float* q, const float* k_cache, const float* v_cache,
                                     size_t B, size_t T, size_t H, size_t Hkv, size_t dk, size_t pos0,
                                     const float* rope_cos, const float* rope_sin, size_t max_len, float scale,
                                     float* out)
{
    return attention_prefill_common(ctx, "nnhip_attention_prefill", q, k_cache, v_cache, false, B, T, H, Hkv, dk, pos0,
                                    rope_cos, rope_sin, max_len, scale, out);
}

nnhip_status nnhip_attention_prefill_h(nnhip_ctx* ctx, const float* q, const uint16_t* k_cache,
                                       const uint16_t* v_cache, size_t B, size_t T, size_t H, size_t Hkv, size_t dk,
                                       size_t pos0, const float* rope_cos, const float* rope_sin, size_t max_len,
                                       float scale, float* out)
{
    return attention_prefill_common(ctx, "nnhip_attention_prefill_h", q, k_cache, v_cache, true, B, T, H, Hkv, dk,
                                    pos0, rope_cos, rope_sin, max_len, scale, out);
}

nnhip_status nnhip_copy_columns(nnhip_ctx* ctx, const float* src, size_t rows, size_t src_cols, size_t col0,
                                size_t stride, size_t n, float* dst)
{
    const char* fn = "nnhip_copy_columns";
    NNHIP_CHECK_CTX(fn);
    if (rows == 0 || n == 0) return NNHIP_OK;
    NNHIP_REQUIRE(src && dst, fn, "null pointer");
    NNHIP_REQUIRE(mul_ok(rows, n) && mul_ok(n - 1, stride) && col0 + (n - 1) * stride < src_cols, fn,
                  "columns col0 + j * stride must lie below src_cols");
    NNHIP_LAUNCH(fn, launch_copy_cols(ctx->stream, src, rows, src_cols, col0, stride, n, dst));
    return NNHIP_OK;
}

nnhip_status nnhip_add(nnhip_ctx* ctx, const float* x, const float* y, size_t n, float* out)
{
    const char* fn = "nnhip_add";
    NNHIP_CHECK_CTX(fn);
    if (n == 0) return NNHIP_OK;
    NNHIP_REQUIRE(x && y && out, fn, "null pointer");
    NNHIP_LAUNCH(fn, launch_add(ctx->stream, x, y, n, out));
    return NNHIP_OK;
}

static nnhip_status embedding_gather_common(nnhip_ctx* ctx, const char* fn, const float* table, const int32_t* ids,
                                            size_t V, size_t d, size_t B, float* out, bool tm)
{
    NNHIP_CHECK_CTX(fn);
    if (B == 0 || d == 0) return NNHIP_OK;
    NNHIP_REQUIRE(table && ids && out, fn, "null pointer");
    NNHIP_REQUIRE(V >= 1 && V <= kMaxDim && d <= kMaxDim && B <= 65535 && mul_ok(V, d), fn, "size out of range");
    NNHIP_LAUNCH(fn, launch_embed(ctx->stream, table, ids, V, d, B, tm, out));
    return NNHIP_OK;
}

nnhip_status nnhip_embedding_gather(nnhip_ctx* ctx, const float* table, const int32_t* ids, size_t V, size_t d,
                                    size_t B, float* out)
{
    return embedding_gather_common(ctx, "nnhip_embedding_gather", table, ids, V, d, B, out, false);
}

nnhip_status nnhip_embedding_gather_tokens(nnhip_ctx* ctx, const float* table, const int32_t* ids, size_t V, size_t d,
                                           size_t B, float* out)
{
    return embedding_gather_common(ctx, "nnhip_embedding_gather_tokens", table, ids, V, d, B, out, true);
}

nnhip_status nnhip_argmax_cols(nnhip_ctx* ctx, const float* logits, size_t V, size_t B, int32_t* ids)
{
    const char* fn = "nnhip_argmax_cols";
    NNHIP_CHECK_CTX(fn);
    if (B == 0) return NNHIP_OK;
    NNHIP_REQUIRE(logits && ids, fn, "null pointer");
    NNHIP_REQUIRE(V >= 1 && V <= kMaxDim && B <= kMaxDim && mul_ok(V, B), fn, "size out of range");
    NNHIP_LAUNCH(fn, launch_argmax(ctx->stream, logits, V, B, ids));
    return NNHIP_OK;
}

nnhip_status nnhip_argmax_rows(nnhip_ctx* ctx, const float* logits, size_t V, size_t B, int32_t* ids, int32_t* pos)
{
    const char* fn = "nnhip_argmax_rows";
    NNHIP_CHECK_CTX(fn);
    if (B == 0) return NNHIP_OK;
    NNHIP_REQUIRE(logits && ids, fn, "null pointer");
    NNHIP_REQUIRE(V >= 1 && V <= kMaxDim && B <= kMaxDim && mul_ok(V, B), fn, "size out of range");
    NNHIP_LAUNCH(fn, launch_argmax(ctx->stream, logits, V, B, ids, true, pos));
    return NNHIP_OK;
}

}  // extern "C"
