// hip_engine.cpp — nn::HipEngine: the nn::ComputeEngine of libnn-hip.so. Plain C++ over the
// C ABI (include/nnhip.h); no HIP header is included here.
//
// Engine-private layouts stay behind the interface: matmul_q_i8 repacks the reference
// ternary container into the T16K256 tile layout once per (storage, write epoch) and caches
// it on the weight tensor's storage; activations are converted to the token-major int8
// layout in engine scratch. bitlinear_i8_forward runs the fused path: one quantization
// kernel (abs-max, scale, int8, row sums) and one GEMV/GEMM launch with the bias add in
// its epilogue, producing the same bits as the reference call sequence.
#include <map>
#include <mutex>
#include <optional>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>

#include "neuralnet.cpp/hip_engine.hpp"
#include "neuralnet.cpp/int8_pack.hpp"
#include "neuralnet.cpp/ternary_pack.hpp"
#include "nnhip.h"

namespace nn
{

namespace
{

thread_local std::string g_factory_error;

Error hip_error(const char* what)
{
    return Error{std::string("HipEngine: ") + what + ": " + nnhip_last_error()};
}

#define NNHIP_TRY(call, what)                         \
    do                                                \
    {                                                 \
        if ((call) != NNHIP_OK) return hip_error(what); \
    } while (0)

const float* fp(const Tensor& t) { return static_cast<const float*>(TensorAccess::ptr(t)); }
float* fpw(const Tensor& t) { return static_cast<float*>(TensorAccess::ptr(t)); }
const uint32_t* up(const Tensor& t) { return static_cast<const uint32_t*>(TensorAccess::ptr(t)); }
uint32_t* upw(const Tensor& t) { return static_cast<uint32_t*>(TensorAccess::ptr(t)); }

// Context shared with every allocation's deleter, so buffers can be freed after the engine.
// It also keeps a caching pool of device blocks: a tensor's storage goes back to the pool when
// its last copy dies and a later allocation of the same size class takes it, so a decode loop
// (a few dozen short-lived tensors per layer and step) makes no hipMalloc / hipFree calls once
// warm. Reuse is safe without events because every call of the engine is ordered on the one
// stream of the context: the kernels that used a block are queued before any that reuse it,
// and host copies into a block wait for the stream.
struct Ctx
{
    nnhip_ctx* h = nullptr;
    std::mutex mu;
    std::multimap<std::size_t, void*> pool;  // size class -> free blocks
    std::size_t pooled = 0;
    static constexpr std::size_t kPoolCap = std::size_t(8) << 30;  // bytes kept before freeing instead

    static std::size_t size_class(std::size_t bytes)
    {
        if (bytes <= 4096) return (bytes + 255) & ~std::size_t(255);
        if (bytes <= (std::size_t(1) << 20)) return (bytes + 4095) & ~std::size_t(4095);
        return (bytes + (std::size_t(1) << 20) - 1) & ~((std::size_t(1) << 20) - 1);
    }
    void* take(std::size_t cls)
    {
        std::lock_guard<std::mutex> lk(mu);
        auto it = pool.find(cls);
        if (it == pool.end()) return nullptr;
        void* p = it->second;
        pool.erase(it);
        pooled -= cls;
        return p;
    }
    void give(void* p, std::size_t cls)
    {
        {
            std::lock_guard<std::mutex> lk(mu);
            if (pooled + cls <= kPoolCap)
            {
                pool.emplace(cls, p);
                pooled += cls;
                return;
            }
        }
        (void)nnhip_free(h, p);
    }
    void release_all()
    {
        std::lock_guard<std::mutex> lk(mu);
        for (auto& kv : pool) (void)nnhip_free(h, kv.second);
        pool.clear();
        pooled = 0;
    }
    ~Ctx()
    {
        if (!h) return;
        (void)nnhip_sync(h);
        release_all();
        (void)nnhip_ctx_destroy(h);
    }
};

class HipEngine final : public ComputeEngine
{
public:
    explicit HipEngine(std::shared_ptr<Ctx> ctx, int device) : ctx_(std::move(ctx)), device_(device) {}
    ~HipEngine() override { (void)nnhip_sync(ctx_->h); }

protected:
    Result<std::shared_ptr<void>> device_alloc(std::size_t bytes)
    {
        const std::size_t cls = Ctx::size_class(bytes < 16 ? 16 : bytes);
        void* p = ctx_->take(cls);
        if (!p && nnhip_malloc(ctx_->h, cls, &p) != NNHIP_OK)
        {
            // out of memory: give the pooled blocks back to the device and try once more
            (void)nnhip_sync(ctx_->h);
            ctx_->release_all();
            p = nullptr;
            NNHIP_TRY(nnhip_malloc(ctx_->h, cls, &p), "allocation");
        }
        std::shared_ptr<Ctx> keep = ctx_;
        return std::shared_ptr<void>(p, [keep, cls](void* q) { keep->give(q, cls); });
    }

    Result<Tensor> alloc_impl(std::size_t rows, std::size_t cols, Precision p) override
    {
        auto st = std::make_shared<detail::Storage>();
        st->bytes = rows * cols * element_bytes(p);
        EX_TRY(mem, device_alloc(st->bytes));
        st->mem = *mem;
        st->owner = this;
        return TensorAccess::make(std::move(st), rows, cols, p);
    }

    Result<void> upload_impl(const Tensor& dst, const void* src, std::size_t bytes) override
    {
        NNHIP_TRY(nnhip_memcpy_h2d(ctx_->h, TensorAccess::ptr(dst), src, bytes), "upload");
        return {};
    }

    Result<void> download_impl(const Tensor& src, void* dst, std::size_t bytes) override
    {
        NNHIP_TRY(nnhip_memcpy_d2h(ctx_->h, dst, TensorAccess::ptr(src), bytes), "download");
        return {};
    }

    Result<void> copy_impl(const Tensor& dst, const Tensor& src, std::size_t bytes) override
    {
        NNHIP_TRY(nnhip_memcpy_d2d(ctx_->h, TensorAccess::ptr(dst), TensorAccess::ptr(src), bytes), "copy");
        return {};
    }

    Result<void> convert_impl(const Tensor& src, const Tensor& dst) override
    {
        if (src.precision() == Precision::F32 && dst.precision() == Precision::F16)
        {
            NNHIP_TRY(nnhip_convert_f32_f16(ctx_->h, fp(src), src.size(), static_cast<uint16_t*>(TensorAccess::ptr(dst))),
                      "f32 -> f16");
            return {};
        }
        if (src.precision() == Precision::F16 && dst.precision() == Precision::F32)
        {
            NNHIP_TRY(nnhip_convert_f16_f32(ctx_->h, static_cast<const uint16_t*>(TensorAccess::ptr(src)), src.size(),
                                            fpw(dst)),
                      "f16 -> f32");
            return {};
        }
        return Error{"convert: only f32 <-> f16"};
    }

    Result<void> trit_pack_impl(const Tensor& W, const Tensor& tau, const Tensor& out) override
    {
        NNHIP_TRY(nnhip_trit_pack(ctx_->h, fp(W), fp(tau), W.rows(), W.cols(), upw(out)), "trit_pack");
        return {};
    }

    Result<void> row_absmean_impl(const Tensor& W, const Tensor& tau) override
    {
        NNHIP_TRY(nnhip_row_absmean(ctx_->h, fp(W), W.rows(), W.cols(), fpw(tau)), "row_absmean");
        return {};
    }

    Result<void> abs_impl(const Tensor& x, const Tensor& out) override
    {
        NNHIP_TRY(nnhip_abs(ctx_->h, fp(x), x.size(), fpw(out)), "abs");
        return {};
    }

    Result<void> col_reduce_max_impl(const Tensor& x, const Tensor& out) override
    {
        NNHIP_TRY(nnhip_col_reduce_max(ctx_->h, fp(x), x.rows(), x.cols(), fpw(out)), "col_reduce_max");
        return {};
    }

    Result<void> scale_impl(const Tensor& x, Scalar s) override
    {
        NNHIP_TRY(nnhip_scale_inplace(ctx_->h, fpw(x), x.size(), s), "scale_inplace");
        return {};
    }

    Result<void> quantize_i8_impl(const Tensor& x, const Tensor& scale, bool col_scale, const Tensor& out) override
    {
        NNHIP_TRY(nnhip_quantize_i8(ctx_->h, fp(x), fp(scale), x.rows(), x.cols(), col_scale ? 1 : 0, upw(out)),
                  "quantize_i8");
        return {};
    }

    Result<void> unpack_i8_impl(const Tensor& packed, std::size_t cols, const Tensor& out) override
    {
        NNHIP_TRY(nnhip_unpack_i8(ctx_->h, up(packed), packed.rows(), cols, fpw(out)), "unpack_i8");
        return {};
    }

    // Engine-private copies derived from a weight container, kept on its storage: the T16K256
    // repack (valid for the storage's write epoch) and, for a fused gate/up container, the
    // interleaved repack with tau / bias in the same row order (valid for the epochs of the
    // container, tau and bias it was made from).
    struct WeightCache
    {
        std::shared_ptr<void> rp;
        std::uint64_t rp_epoch = ~std::uint64_t{0};
        std::shared_ptr<void> rpt;  // repack of the transposed container (M rows, K columns)
        std::uint64_t rpt_epoch = ~std::uint64_t{0};
        std::size_t rpt_m = 0;
        std::shared_ptr<void> glu_rp, glu_tau, glu_bias;
        std::uint64_t glu_epoch = ~std::uint64_t{0}, glu_tau_epoch = 0, glu_bias_epoch = 0;
        const detail::Storage* glu_tau_st = nullptr;
        const detail::Storage* glu_bias_st = nullptr;
    };

    static WeightCache& cache_of(const Tensor& wq)
    {
        detail::Storage* st = TensorAccess::storage(wq);
        if (!st->derived) st->derived = std::make_shared<WeightCache>();
        return *static_cast<WeightCache*>(st->derived.get());
    }

    // T16K256 copy of a weight container, cached on its storage for the current write epoch.
    Result<const void*> repacked(const Tensor& wq, std::size_t K)
    {
        WeightCache& c = cache_of(wq);
        if (c.rp && c.rp_epoch == wq.write_epoch()) return static_cast<const void*>(c.rp.get());
        EX_TRY(mem, device_alloc(nnhip_repacked_bytes(wq.rows(), K)));
        NNHIP_TRY(nnhip_repack_ternary(ctx_->h, up(wq), wq.rows(), K, mem->get()), "repack");
        c.rp = *mem;
        c.rp_epoch = wq.write_epoch();
        return static_cast<const void*>(c.rp.get());
    }

    // T16K256 copy of the transposed container At (M, ceil(K/16)) of A (K, ceil(M/16)), cached
    // like repacked(): the operand of the transposed product on the MFMA path.
    Result<const void*> repacked_t(const Tensor& A, std::size_t M)
    {
        WeightCache& c = cache_of(A);
        const std::size_t K = A.rows();
        if (c.rpt && c.rpt_epoch == A.write_epoch() && c.rpt_m == M) return static_cast<const void*>(c.rpt.get());
        EX_TRY(at, device_alloc(M * trit_pack::words_per_row(K) * sizeof(uint32_t)));
        EX_TRY(mem, device_alloc(nnhip_repacked_bytes(M, K)));
        NNHIP_TRY(nnhip_trit_transpose(ctx_->h, up(A), K, M, static_cast<uint32_t*>(at->get())), "transpose");
        NNHIP_TRY(nnhip_repack_ternary(ctx_->h, static_cast<const uint32_t*>(at->get()), M, K, mem->get()),
                  "repack (transposed)");
        c.rpt = *mem;
        c.rpt_epoch = A.write_epoch();
        c.rpt_m = M;
        return static_cast<const void*>(c.rpt.get());
    }

    struct GluWeights
    {
        const void* rp;
        const float* tau;
        const float* bias;
    };

    // Interleaved gate/up repack of fc1 (2F rows) plus tau / bias in that order.
    Result<GluWeights> glu_weights(const Tensor& wq1, const Tensor& tau1, const Tensor& b1, std::size_t F,
                                   std::size_t K)
    {
        WeightCache& c = cache_of(wq1);
        const detail::Storage* ts = TensorAccess::storage(tau1);
        const detail::Storage* bs = TensorAccess::storage(b1);
        if (!(c.glu_rp && c.glu_epoch == wq1.write_epoch() && c.glu_tau_st == ts &&
              c.glu_tau_epoch == tau1.write_epoch() && c.glu_bias_st == bs && c.glu_bias_epoch == b1.write_epoch()))
        {
            const std::size_t rows = nnhip_glu_rows(F);
            EX_TRY(words, device_alloc(rows * trit_pack::words_per_row(K) * sizeof(uint32_t)));
            EX_TRY(rp, device_alloc(nnhip_repacked_bytes(rows, K)));
            EX_TRY(t, device_alloc(rows * sizeof(float)));
            EX_TRY(b, device_alloc(rows * sizeof(float)));
            NNHIP_TRY(nnhip_glu_interleave(ctx_->h, up(wq1), fp(tau1), fp(b1), F, K, static_cast<uint32_t*>(words->get()),
                                           static_cast<float*>(t->get()), static_cast<float*>(b->get())),
                      "ffn (gate/up interleave)");
            NNHIP_TRY(nnhip_repack_ternary(ctx_->h, static_cast<const uint32_t*>(words->get()), rows, K, rp->get()),
                      "ffn (repack)");
            c.glu_rp = *rp;
            c.glu_tau = *t;
            c.glu_bias = *b;
            c.glu_epoch = wq1.write_epoch();
            c.glu_tau_st = ts;
            c.glu_tau_epoch = tau1.write_epoch();
            c.glu_bias_st = bs;
            c.glu_bias_epoch = b1.write_epoch();
        }
        return GluWeights{c.glu_rp.get(), static_cast<const float*>(c.glu_tau.get()),
                          static_cast<const float*>(c.glu_bias.get())};
    }

    // Token-major int8 activations + row sums, reused across calls (all work of one engine
    // is ordered on its stream); grown on demand after a sync.
    struct ActScratch
    {
        int8_t* xi;
        int32_t* rowsum;
    };

    Result<ActScratch> act_scratch(std::size_t K, std::size_t M)
    {
        const std::size_t xi_bytes = nnhip_act_i8_bytes(K, M), rs_bytes = M * sizeof(int32_t);
        if (xi_bytes > xi_cap_ || rs_bytes > rs_cap_)
        {
            NNHIP_TRY(nnhip_sync(ctx_->h), "scratch sync");
            xi_buf_.reset();
            rs_buf_.reset();
            EX_TRY(xi, device_alloc(xi_bytes > xi_cap_ ? xi_bytes : xi_cap_));
            EX_TRY(rs, device_alloc(rs_bytes > rs_cap_ ? rs_bytes : rs_cap_));
            xi_cap_ = xi_bytes > xi_cap_ ? xi_bytes : xi_cap_;
            rs_cap_ = rs_bytes > rs_cap_ ? rs_bytes : rs_cap_;
            xi_buf_ = *xi;
            rs_buf_ = *rs;
            last_quant_.reset();
        }
        return ActScratch{static_cast<int8_t*>(xi_buf_.get()), static_cast<int32_t*>(rs_buf_.get())};
    }

    Result<void> matmul_q_i8_impl(const Tensor& wq, const Tensor& tau, const Tensor& xq, const Tensor& s,
                                  const Tensor& y) override
    {
        const std::size_t N = wq.rows(), K = xq.rows(), M = s.cols();
        if (N == 0 || M == 0) return {};
        EX_TRY(rp, repacked(wq, K));
        EX_TRY(a, act_scratch(K, M));
        last_quant_.reset();  // the scratch now holds another activation
        int8_t* xi = a->xi;
        int32_t* rs = a->rowsum;
        NNHIP_TRY(nnhip_act_i8_from_container(ctx_->h, up(xq), K, M, xi, rs), "matmul_q_i8 (activations)");
        NNHIP_TRY(nnhip_ternary_matmul(ctx_->h, *rp, fp(tau), xi, fp(s), rs, nullptr, N, K, M, fpw(y)),
                  "matmul_q_i8");
        return {};
    }

    // f32 activations: the MFMA path on the cached repack (int8 digits of a per-token fixed point,
    // nnhip_ternary_matmul_f) up to its K bound, else the reference-layout VALU kernel.
    Result<void> matmul_q_impl(const Tensor& wq, const Tensor& tau, const Tensor& B, const Tensor& y) override
    {
        const std::size_t N = wq.rows(), K = B.rows(), M = B.cols();
        if (N == 0 || M == 0) return {};
        if (K < 131072)
        {
            EX_TRY(rp, repacked(wq, K));
            NNHIP_TRY(nnhip_ternary_matmul_f(ctx_->h, *rp, fp(tau), fp(B), 0, N, K, M, fpw(y), 0), "matmul_q");
            return {};
        }
        NNHIP_TRY(nnhip_matmul_q(ctx_->h, up(wq), fp(tau), fp(B), 0, N, K, M, fpw(y), 0), "matmul_q");
        return {};
    }

    // Transposed product (BitLinear's dX): the MFMA path on the cached transposed repack with tau
    // folded into the activations, up to its K bound; else the reference-layout VALU kernel.
    Result<void> matmul_q_t_impl(const Tensor& A, const Tensor& tau, const Tensor& B, std::size_t M,
                                 const Tensor& y) override
    {
        const std::size_t K = A.rows(), N = B.cols();
        if (M == 0 || N == 0) return {};
        if (K < 131072)
        {
            EX_TRY(rpt, repacked_t(A, M));
            NNHIP_TRY(nnhip_ternary_matmul_t_f(ctx_->h, *rpt, fp(tau), fp(B), 0, K, M, N, fpw(y), 0), "matmul_q_t");
            return {};
        }
        NNHIP_TRY(nnhip_matmul_q_t(ctx_->h, up(A), fp(tau), fp(B), 0, A.rows(), M, B.cols(), fpw(y), 0),
                  "matmul_q_t");
        return {};
    }

    Result<void> add_row_broadcast_impl(const Tensor& y, const Tensor& b, const Tensor& out) override
    {
        NNHIP_TRY(nnhip_memcpy_d2d(ctx_->h, TensorAccess::ptr(out), TensorAccess::ptr(y), y.size() * sizeof(float)),
                  "add_row_broadcast (copy)");
        NNHIP_TRY(nnhip_add_row_broadcast(ctx_->h, fpw(out), fp(b), y.rows(), y.cols()), "add_row_broadcast");
        return {};
    }

    Result<void> rmsnorm_impl(const Tensor& x, const Tensor& gamma, Scalar eps, const Tensor& out) override
    {
        NNHIP_TRY(nnhip_rmsnorm(ctx_->h, fp(x), fp(gamma), eps, x.rows(), x.cols(), fpw(out)), "rmsnorm");
        return {};
    }

    Result<void> layernorm_impl(const Tensor& x, const Tensor& gamma, const Tensor& beta, Scalar eps,
                                const Tensor& out) override
    {
        NNHIP_TRY(nnhip_layernorm(ctx_->h, fp(x), fp(gamma), fp(beta), eps, x.rows(), x.cols(), fpw(out)),
                  "layernorm");
        return {};
    }

    // The last input quantized into the activation scratch. Another BitLinear on the same input
    // (same storage, same write epoch, same shape; e.g. the q / k / v projections of one
    // attention input) reuses it instead of quantizing again. The storage is held weakly, so a
    // freed input never matches a new one at the same address.
    struct LastQuant
    {
        std::weak_ptr<detail::Storage> src;
        std::uint64_t epoch = 0;
        std::size_t K = 0, M = 0;
        Tensor s;
        Tensor xq;  // the reference int8 container, when that quantization wrote one
    };

    bool reuses_last_quant(const Tensor& x) const
    {
        if (!last_quant_ || last_quant_->K != x.rows() || last_quant_->M != x.cols()) return false;
        const auto src = last_quant_->src.lock();
        return src && src.get() == TensorAccess::storage(x) && last_quant_->epoch == x.write_epoch();
    }

    Result<Tensor> bitlinear_i8_impl(const Tensor& x, const Tensor& wq, const Tensor& tau, const Tensor* b,
                                     Tensor* xq_out, Tensor* s_out) override
    {
        const std::size_t K = x.rows(), M = x.cols(), N = wq.rows();
        EX_TRY(y, alloc_impl(N, M, Precision::F32));
        if (M == 0 || N == 0)
        {
            EX_TRY(s0, alloc_impl(1, M, Precision::F32));
            if (xq_out)
            {
                EX_TRY(t, alloc_impl(K, i8_pack::words_per_row(M), Precision::F32));
                *xq_out = *t;
            }
            if (s_out) *s_out = *s0;
            return *y;
        }
        EX_TRY(rp, repacked(wq, K));
        EX_TRY(a, act_scratch(K, M));
        int8_t* xi = a->xi;
        int32_t* rs = a->rowsum;
        Tensor s;
        if (reuses_last_quant(x) && (!xq_out || last_quant_->xq.valid()))
        {
            s = last_quant_->s;
            if (xq_out) *xq_out = last_quant_->xq;
        }
        else
        {
            EX_TRY(s1, alloc_impl(1, M, Precision::F32));
            s = *s1;
            Tensor xq;
            if (xq_out)
            {
                EX_TRY(t, alloc_impl(K, i8_pack::words_per_row(M), Precision::F32));
                xq = *t;
            }
            last_quant_.reset();
            NNHIP_TRY(nnhip_act_quant_i8(ctx_->h, fp(x), K, M, xi, fpw(s), rs, xq_out ? upw(xq) : nullptr),
                      "bitlinear_i8_forward (activation quantization)");
            ++act_quant_calls_;
            last_quant_ = LastQuant{TensorAccess::storage_ref(x), x.write_epoch(), K, M, s, xq};
            if (xq_out) *xq_out = xq;
        }
        NNHIP_TRY(nnhip_ternary_matmul(ctx_->h, *rp, fp(tau), xi, fp(s), rs, b ? fp(*b) : nullptr, N, K, M, fpw(*y)),
                  "bitlinear_i8_forward (ternary product)");
        if (s_out) *s_out = s;
        return *y;
    }

    std::uint64_t activation_quantizations() const noexcept override { return act_quant_calls_; }

    Result<void> glu_impl(const Tensor& y1, int act, const Tensor& out) override
    {
        NNHIP_TRY(nnhip_glu(ctx_->h, fp(y1), y1.rows() / 2, y1.cols(), act, fpw(out)), "glu");
        return {};
    }

    // The whole block in one library call: [RMSNorm ->] int8 -> fc1 with the gated activation in
    // its epilogue -> [SubLN ->] int8 -> fc2 (nnhip_ffn_glu_i8), on cached interleaved / repacked
    // weights.
    Result<Tensor> ffn_glu_i8_impl(const Tensor& x, const Tensor* gamma, Scalar eps, const Tensor& wq1,
                                   const Tensor& tau1, const Tensor& b1, const Tensor& wq2, const Tensor& tau2,
                                   const Tensor& b2, int act, const Tensor* gamma_sub, Scalar eps_sub) override
    {
        const std::size_t d = x.rows(), M = x.cols(), F = wq1.rows() / 2;
        EX_TRY(y, alloc_impl(d, M, Precision::F32));
        if (M == 0) return *y;
        EX_TRY(g1, glu_weights(wq1, tau1, b1, F, d));
        EX_TRY(rp2, repacked(wq2, F));
        NNHIP_TRY(nnhip_ffn_glu_i8(ctx_->h, fp(x), gamma ? fp(*gamma) : nullptr, eps, d, F, M, act, g1->rp, g1->tau,
                                   g1->bias, gamma_sub ? fp(*gamma_sub) : nullptr, eps_sub, *rp2, fp(tau2), fp(b2),
                                   fpw(*y)),
                  "ffn_glu_i8_forward");
        return *y;
    }

    Result<void> attention_decode_impl(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& k_cache,
                                       const Tensor& v_cache, std::size_t max_len, const Tensor& positions,
                                       std::size_t len_bound, const Tensor* rope_cos, const Tensor* rope_sin,
                                       std::size_t heads, std::size_t kv_heads, Scalar scale,
                                       const Tensor& out) override
    {
        const std::size_t dk = q.rows() / heads;
        const auto* pos = static_cast<const int32_t*>(TensorAccess::ptr(positions));
        const float* cs = rope_cos ? fp(*rope_cos) : nullptr;
        const float* sn = rope_sin ? fp(*rope_sin) : nullptr;
        if (k_cache.precision() == Precision::F16)  // compute = F16: f16 storage, f32 arithmetic
        {
            NNHIP_TRY(nnhip_attention_decode_h(ctx_->h, fp(q), fp(k), fp(v), q.cols(), heads, kv_heads, dk, pos,
                                               len_bound, cs, sn, static_cast<uint16_t*>(TensorAccess::ptr(k_cache)),
                                               static_cast<uint16_t*>(TensorAccess::ptr(v_cache)), max_len, scale,
                                               fpw(out)),
                      "attention_decode");
            return {};
        }
        NNHIP_TRY(nnhip_attention_decode(ctx_->h, fp(q), fp(k), fp(v), q.cols(), heads, kv_heads, dk, pos, len_bound,
                                         cs, sn, fpw(k_cache), fpw(v_cache), max_len, scale, fpw(out)),
                  "attention_decode");
        return {};
    }

    Result<void> add_impl(const Tensor& x, const Tensor& y, const Tensor& out) override
    {
        NNHIP_TRY(nnhip_add(ctx_->h, fp(x), fp(y), x.size(), fpw(out)), "add");
        return {};
    }

    Result<void> embedding_gather_impl(const Tensor& table, const Tensor& ids, const Tensor& out) override
    {
        NNHIP_TRY(nnhip_embedding_gather(ctx_->h, fp(table), static_cast<const int32_t*>(TensorAccess::ptr(ids)),
                                         table.rows(), table.cols(), ids.rows(), fpw(out)),
                  "embedding_gather");
        return {};
    }

    Result<void> argmax_cols_impl(const Tensor& logits, const Tensor& out) override
    {
        NNHIP_TRY(nnhip_argmax_cols(ctx_->h, fp(logits), logits.rows(), logits.cols(),
                                    static_cast<int32_t*>(TensorAccess::ptr(out))),
                  "argmax_cols");
        return {};
    }

    EngineInfo describe_impl() const override
    {
        EngineInfo i;
        i.engine = "hip";
        char name[256] = {};
        if (nnhip_device_name(device_, name, sizeof(name)) == NNHIP_OK)
            i.device = std::string(name) + " #" + std::to_string(device_);
        else
            i.device = "HIP device #" + std::to_string(device_);
        i.ternary_gemm = true;
        i.int8_dot = true;
        i.int8_dot_accelerated = true;
        return i;
    }

    void sync_impl() override { (void)nnhip_sync(ctx_->h); }

private:
    std::shared_ptr<Ctx> ctx_;
    int device_;
    std::shared_ptr<void> xi_buf_, rs_buf_;
    std::size_t xi_cap_ = 0, rs_cap_ = 0;
    std::optional<LastQuant> last_quant_;
    std::uint64_t act_quant_calls_ = 0;
};

int parse_device(const char* device)
{
    if (!device || !*device) return 0;
    const char* p = device;
    if (std::strncmp(p, "hip:", 4) == 0) p += 4;
    char* end = nullptr;
    const long v = std::strtol(p, &end, 10);
    if (end == p || *end != '\0' || v < 0) return -1;
    return static_cast<int>(v);
}

}  // namespace

std::unique_ptr<ComputeEngine> create_hip_engine(const char* device)
{
    const int dev = parse_device(device);
    if (dev < 0)
    {
        g_factory_error = std::string("create_hip_engine: bad device string '") + device + "'";
        return nullptr;
    }
    auto ctx = std::make_shared<Ctx>();
    if (nnhip_ctx_create(dev, &ctx->h) != NNHIP_OK)
    {
        g_factory_error = std::string("create_hip_engine: ") + nnhip_last_error();
        ctx->h = nullptr;
        return nullptr;
    }
    return std::make_unique<HipEngine>(std::move(ctx), dev);
}

const char* last_error() noexcept { return g_factory_error.c_str(); }

}  // namespace nn
