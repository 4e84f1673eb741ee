// compute_engine.cpp — the NVI layer of nn::ComputeEngine: domain, shape and precision
// checks, output allocation and write-epoch bookkeeping around the engine's *_impl calls.
// Shape contracts follow the reference call sites (see compute_engine.hpp).
#include "neuralnet.cpp/compute_engine.hpp"

#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "neuralnet.cpp/int8_pack.hpp"
#include "neuralnet.cpp/ternary_pack.hpp"

namespace nn
{

namespace
{
std::string shape(const Tensor& t) { return std::to_string(t.rows()) + "x" + std::to_string(t.cols()); }

Result<void> require_f32(const Tensor& t, const char* fn, const char* what)
{
    if (!t.valid()) return Error{std::string(fn) + ": " + what + " is an empty tensor"};
    if (t.precision() != Precision::F32)
        return Error{std::string(fn) + ": " + what + " has precision " + precision_name(t.precision()) +
                     "; this engine runs the W1.58A8 path in f32 containers only"};
    return {};
}

// Write-epoch guard: the destination's epoch advances when the entry returns, success or not.
struct EpochGuard
{
    const Tensor& t;
    ~EpochGuard() { TensorAccess::mark_written(t); }
};
}  // namespace

Result<void> ComputeEngine::check_owned(const Tensor& t, const char* what) const
{
    const detail::Storage* st = TensorAccess::storage(t);
    if (!st) return Error{std::string(what) + ": empty tensor"};
    if (st->owner != this) return Error{std::string(what) + ": tensor belongs to another engine"};
    return {};
}

namespace
{
bool is_float(Precision p) { return p == Precision::F32 || p == Precision::F16; }
}  // namespace

Result<Tensor> ComputeEngine::widen_f32(const Tensor& t)
{
    if (t.precision() != Precision::F16) return t;
    EX_TRY(w, alloc_impl(t.rows(), t.cols(), Precision::F32));
    if (t.size() > 0) EX_TRY_CHECK(convert_impl(t, *w));
    return *w;
}

Result<Tensor> ComputeEngine::narrow_to(const Tensor& y32, Precision p)
{
    if (p != Precision::F16) return y32;
    EX_TRY(n, alloc_impl(y32.rows(), y32.cols(), Precision::F16));
    if (y32.size() > 0) EX_TRY_CHECK(convert_impl(y32, *n));
    return *n;
}

Tensor ComputeEngine::create_tensor(std::size_t rows, std::size_t cols, Precision p, InitSpec init)
{
    if (!is_float(p)) return Tensor{};
    if (p == Precision::F16)
    {
        // the f32 values, rounded once
        const Tensor f = create_tensor(rows, cols, Precision::F32, init);
        if (!f.valid()) return Tensor{};
        auto h = narrow_to(f, Precision::F16);
        return h ? *h : Tensor{};
    }
    auto t = alloc_impl(rows, cols, p);
    if (!t) return Tensor{};
    std::vector<float> host(rows * cols, 0.0f);
    if (init.kind == InitSpec::Kind::Constant)
        for (float& v : host) v = init.a;
    else if (init.kind == InitSpec::Kind::Uniform)
    {
        std::mt19937 rng(static_cast<std::uint32_t>(init.seed));
        std::uniform_real_distribution<float> d(init.a, init.b);
        for (float& v : host) v = d(rng);
    }
    if (!host.empty() && !upload_impl(*t, host.data(), host.size() * sizeof(float))) return Tensor{};
    return *t;
}

Result<Tensor> ComputeEngine::from_matrix(const Matrix& m, Precision p)
{
    if (!is_float(p))
        return Error{std::string("from_matrix: precision ") + precision_name(p) + " is not supported by this engine"};
    EX_TRY(t, alloc_impl(m.rows(), m.cols(), Precision::F32));
    if (m.size() > 0) EX_TRY_CHECK(upload_impl(*t, m.data(), m.size() * sizeof(float)));
    return narrow_to(*t, p);   // F16: each value rounded to nearest even
}

// P is the precision of the values handed back: F32 widens f16 storage exactly; F16 rounds f32
// storage to binary16 first (the matrix itself holds floats).
Result<Matrix> ComputeEngine::to_matrix(const Tensor& t, Precision p)
{
    EX_TRY_CHECK(check_owned(t, "to_matrix"));
    if (!is_float(p)) return Error{std::string("to_matrix: precision ") + precision_name(p) + " is not supported"};
    Tensor src = t;
    if (p == Precision::F16 && t.precision() == Precision::F32)
    {
        EX_TRY(h, narrow_to(t, Precision::F16));
        src = *h;
    }
    EX_TRY(w, widen_f32(src));
    Matrix m(t.rows(), t.cols());
    if (m.size() > 0) EX_TRY_CHECK(download_impl(*w, m.data(), m.size() * sizeof(float)));
    return m;
}

Result<void> ComputeEngine::copy_from(Tensor& dst, const Matrix& src)
{
    EX_TRY_CHECK(check_owned(dst, "copy_from"));
    EpochGuard g{dst};
    if (dst.rows() != src.rows() || dst.cols() != src.cols())
        return Error{"copy_from: shape mismatch (tensor " + shape(dst) + ", matrix " + std::to_string(src.rows()) +
                     "x" + std::to_string(src.cols()) + ")"};
    if (src.size() == 0) return {};
    if (dst.precision() == Precision::F16)
    {
        EX_TRY(f, alloc_impl(src.rows(), src.cols(), Precision::F32));
        EX_TRY_CHECK(upload_impl(*f, src.data(), src.size() * sizeof(float)));
        return convert_impl(*f, dst);
    }
    return upload_impl(dst, src.data(), src.size() * sizeof(float));
}

Result<void> ComputeEngine::copy_into(Tensor& dst, const Tensor& src)
{
    EX_TRY_CHECK(check_owned(dst, "copy_into: dst"));
    EX_TRY_CHECK(check_owned(src, "copy_into: src"));
    EpochGuard g{dst};
    if (dst.rows() != src.rows() || dst.cols() != src.cols() || dst.precision() != src.precision())
        return Error{"copy_into: shape or precision mismatch (" + shape(dst) + " vs " + shape(src) + ")"};
    if (dst.same_storage(src) || dst.size() == 0) return {};
    return copy_impl(dst, src, dst.size() * element_bytes(dst.precision()));
}

Result<Tensor> ComputeEngine::trit_pack(const Tensor& W, const Tensor& tau)
{
    EX_TRY_CHECK(check_owned(W, "trit_pack"));
    EX_TRY(out, alloc_impl(W.rows(), trit_pack::words_per_row(W.cols()), Precision::F32));
    EX_TRY_CHECK(trit_pack_into(W, tau, *out));
    return *out;
}

Result<void> ComputeEngine::trit_pack_into(const Tensor& W, const Tensor& tau, Tensor& out)
{
    EX_TRY_CHECK(check_owned(W, "trit_pack_into: W"));
    EX_TRY_CHECK(check_owned(tau, "trit_pack_into: tau"));
    EX_TRY_CHECK(check_owned(out, "trit_pack_into: out"));
    EpochGuard g{out};
    EX_TRY_CHECK(require_f32(W, "trit_pack_into", "W"));
    EX_TRY_CHECK(require_f32(tau, "trit_pack_into", "tau"));
    if (tau.rows() != W.rows() || tau.cols() != 1)
        return Error{"trit_pack_into: tau must be (" + std::to_string(W.rows()) + ",1), got " + shape(tau)};
    if (out.rows() != W.rows() || out.cols() != trit_pack::words_per_row(W.cols()))
        return Error{"trit_pack_into: out must be (rows, ceil(K/16)), got " + shape(out)};
    return trit_pack_impl(W, tau, out);
}

Result<void> ComputeEngine::row_absmean_into(const Tensor& W, Tensor& tau)
{
    EX_TRY_CHECK(check_owned(W, "row_absmean_into: W"));
    EX_TRY_CHECK(check_owned(tau, "row_absmean_into: tau"));
    EpochGuard g{tau};
    EX_TRY_CHECK(require_f32(W, "row_absmean_into", "W"));
    if (tau.rows() != W.rows() || tau.cols() != 1)
        return Error{"row_absmean_into: tau must be (" + std::to_string(W.rows()) + ",1), got " + shape(tau)};
    if (W.cols() == 0) return Error{"row_absmean_into: W has no columns"};
    return row_absmean_impl(W, tau);
}

Result<Tensor> ComputeEngine::abs(const Tensor& x)
{
    EX_TRY_CHECK(check_owned(x, "abs"));
    EX_TRY_CHECK(require_f32(x, "abs", "x"));
    EX_TRY(out, alloc_impl(x.rows(), x.cols(), Precision::F32));
    EX_TRY_CHECK(abs_impl(x, *out));
    return *out;
}

Result<Tensor> ComputeEngine::col_reduce_max(const Tensor& x, Precision p)
{
    EX_TRY_CHECK(check_owned(x, "col_reduce_max"));
    EX_TRY_CHECK(require_f32(x, "col_reduce_max", "x"));
    if (p != Precision::F32) return Error{"col_reduce_max: only f32 output is supported"};
    EX_TRY(out, alloc_impl(1, x.cols(), Precision::F32));
    EX_TRY_CHECK(col_reduce_max_impl(x, *out));
    return *out;
}

Result<void> ComputeEngine::scale_inplace(Tensor& x, Scalar s)
{
    EX_TRY_CHECK(check_owned(x, "scale_inplace"));
    EpochGuard g{x};
    EX_TRY_CHECK(require_f32(x, "scale_inplace", "x"));
    return scale_impl(x, s);
}

Result<Tensor> ComputeEngine::quantize_i8(const Tensor& x, const Tensor& scale, bool col_scale)
{
    EX_TRY_CHECK(check_owned(x, "quantize_i8: x"));
    EX_TRY_CHECK(check_owned(scale, "quantize_i8: scale"));
    EX_TRY_CHECK(require_f32(x, "quantize_i8", "x"));
    EX_TRY_CHECK(require_f32(scale, "quantize_i8", "scale"));
    if (col_scale ? (scale.rows() != 1 || scale.cols() != x.cols()) : (scale.rows() != x.rows() || scale.cols() != 1))
        return Error{"quantize_i8: scale must be " +
                     std::string(col_scale ? "(1, cols)" : "(rows, 1)") + ", got " + shape(scale)};
    EX_TRY(out, alloc_impl(x.rows(), i8_pack::words_per_row(x.cols()), Precision::F32));
    EX_TRY_CHECK(quantize_i8_impl(x, scale, col_scale, *out));
    return *out;
}

Result<Tensor> ComputeEngine::unpack_i8(const Tensor& packed, std::size_t cols)
{
    EX_TRY_CHECK(check_owned(packed, "unpack_i8"));
    if (packed.cols() != i8_pack::words_per_row(cols))
        return Error{"unpack_i8: container " + shape(packed) + " does not hold " + std::to_string(cols) + " columns"};
    EX_TRY(out, alloc_impl(packed.rows(), cols, Precision::F32));
    EX_TRY_CHECK(unpack_i8_impl(packed, cols, *out));
    return *out;
}

Result<Tensor> ComputeEngine::matmul_q_i8(const Tensor& wq, const Tensor& tau, const Tensor& xq, const Tensor& s,
                                          Precision p)
{
    EX_TRY_CHECK(check_owned(wq, "matmul_q_i8: wq"));
    EX_TRY_CHECK(check_owned(tau, "matmul_q_i8: tau"));
    EX_TRY_CHECK(check_owned(xq, "matmul_q_i8: xq"));
    EX_TRY_CHECK(check_owned(s, "matmul_q_i8: s"));
    if (!is_float(p)) return Error{"matmul_q_i8: output precision must be f32 or f16"};
    EX_TRY_CHECK(require_f32(s, "matmul_q_i8", "s"));
    const std::size_t N = wq.rows(), K = xq.rows(), M = s.cols();
    if (s.rows() != 1) return Error{"matmul_q_i8: s must be (1, M), got " + shape(s)};
    if (wq.cols() != trit_pack::words_per_row(K))
        return Error{"matmul_q_i8: wq " + shape(wq) + " does not match K=" + std::to_string(K)};
    if (xq.cols() != i8_pack::words_per_row(M))
        return Error{"matmul_q_i8: xq " + shape(xq) + " does not match M=" + std::to_string(M)};
    if (tau.rows() != N || tau.cols() != 1) return Error{"matmul_q_i8: tau must be (N,1), got " + shape(tau)};
    EX_TRY(y, alloc_impl(N, M, Precision::F32));
    EX_TRY_CHECK(matmul_q_i8_impl(wq, tau, xq, s, *y));
    return narrow_to(*y, p);
}

Result<Tensor> ComputeEngine::matmul_q(const Tensor& wq, const Tensor& tau, const Tensor& B, Precision p)
{
    EX_TRY_CHECK(check_owned(wq, "matmul_q: wq"));
    EX_TRY_CHECK(check_owned(tau, "matmul_q: tau"));
    EX_TRY_CHECK(check_owned(B, "matmul_q: B"));
    if (!is_float(B.precision())) return Error{"matmul_q: B must be f32 or f16"};
    if (!is_float(p)) return Error{"matmul_q: output precision must be f32 or f16"};
    const std::size_t N = wq.rows(), K = B.rows(), M = B.cols();
    if (wq.cols() != trit_pack::words_per_row(K))
        return Error{"matmul_q: wq " + shape(wq) + " does not match K=" + std::to_string(K)};
    if (tau.rows() != N || tau.cols() != 1) return Error{"matmul_q: tau must be (N,1), got " + shape(tau)};
    EX_TRY(b32, widen_f32(B));
    EX_TRY(y, alloc_impl(N, M, Precision::F32));
    EX_TRY_CHECK(matmul_q_impl(wq, tau, *b32, *y));
    return narrow_to(*y, p);
}

Result<Tensor> ComputeEngine::matmul_q_t(const Tensor& A, const Tensor& tau, const Tensor& B, std::size_t M,
                                         Precision p)
{
    EX_TRY_CHECK(check_owned(A, "matmul_q_t: A"));
    EX_TRY_CHECK(check_owned(tau, "matmul_q_t: tau"));
    EX_TRY_CHECK(check_owned(B, "matmul_q_t: B"));
    if (!is_float(B.precision())) return Error{"matmul_q_t: B must be f32 or f16"};
    if (!is_float(p)) return Error{"matmul_q_t: output precision must be f32 or f16"};
    const std::size_t K = A.rows(), N = B.cols();
    if (A.cols() != trit_pack::words_per_row(M))
        return Error{"matmul_q_t: A " + shape(A) + " does not hold M=" + std::to_string(M) + " columns"};
    if (B.rows() != K) return Error{"matmul_q_t: B " + shape(B) + " does not match K=" + std::to_string(K)};
    if (tau.rows() != K || tau.cols() != 1) return Error{"matmul_q_t: tau must be (K,1), got " + shape(tau)};
    EX_TRY(b32, widen_f32(B));
    EX_TRY(y, alloc_impl(M, N, Precision::F32));
    EX_TRY_CHECK(matmul_q_t_impl(A, tau, *b32, M, *y));
    return narrow_to(*y, p);
}

Result<Tensor> ComputeEngine::add_row_broadcast(const Tensor& y, const Tensor& b)
{
    EX_TRY_CHECK(check_owned(y, "add_row_broadcast: y"));
    EX_TRY_CHECK(check_owned(b, "add_row_broadcast: b"));
    if (b.rows() != y.rows() || b.cols() != 1)
        return Error{"add_row_broadcast: b must be (" + std::to_string(y.rows()) + ",1), got " + shape(b)};
    if (!is_float(y.precision())) return Error{"add_row_broadcast: y must be f32 or f16"};
    EX_TRY_CHECK(require_f32(b, "add_row_broadcast", "b"));
    EX_TRY(y32, widen_f32(y));
    EX_TRY(out, alloc_impl(y.rows(), y.cols(), Precision::F32));
    EX_TRY_CHECK(add_row_broadcast_impl(*y32, b, *out));
    return narrow_to(*out, y.precision());
}

Result<Tensor> ComputeEngine::rmsnorm(const Tensor& x, const Tensor& gamma, Scalar eps)
{
    EX_TRY_CHECK(check_owned(x, "rmsnorm: x"));
    EX_TRY_CHECK(check_owned(gamma, "rmsnorm: gamma"));
    EX_TRY_CHECK(require_f32(x, "rmsnorm", "x"));
    if (gamma.rows() != x.rows() || gamma.cols() != 1)
        return Error{"rmsnorm: gamma must be (" + std::to_string(x.rows()) + ",1), got " + shape(gamma)};
    EX_TRY(out, alloc_impl(x.rows(), x.cols(), Precision::F32));
    EX_TRY_CHECK(rmsnorm_impl(x, gamma, eps, *out));
    return *out;
}

Result<Tensor> ComputeEngine::layernorm(const Tensor& x, const Tensor& gamma, const Tensor& beta, Scalar eps)
{
    EX_TRY_CHECK(check_owned(x, "layernorm: x"));
    EX_TRY_CHECK(check_owned(gamma, "layernorm: gamma"));
    EX_TRY_CHECK(check_owned(beta, "layernorm: beta"));
    if (x.precision() != Precision::F32) return Error{"layernorm: x must be f32"};
    for (const Tensor* t : {&gamma, &beta})
        if (t->rows() != x.rows() || t->cols() != 1 || t->precision() != Precision::F32)
            return Error{"layernorm: gamma and beta must be f32 (" + std::to_string(x.rows()) + ",1), got " +
                         shape(*t)};
    EX_TRY(out, alloc_impl(x.rows(), x.cols(), Precision::F32));
    EX_TRY_CHECK(layernorm_impl(x, gamma, beta, eps, *out));
    return *out;
}

Result<Tensor> ComputeEngine::bitlinear_i8_forward(const Tensor& x, const Tensor& wq, const Tensor& tau,
                                                   const Tensor& b, Precision p, Tensor* xq_out, Tensor* s_out)
{
    EX_TRY_CHECK(check_owned(x, "bitlinear_i8_forward: x"));
    EX_TRY_CHECK(check_owned(wq, "bitlinear_i8_forward: wq"));
    EX_TRY_CHECK(check_owned(tau, "bitlinear_i8_forward: tau"));
    EX_TRY_CHECK(check_owned(b, "bitlinear_i8_forward: b"));
    if (!is_float(p)) return Error{"bitlinear_i8_forward: output precision must be f32 or f16"};
    if (!is_float(x.precision())) return Error{"bitlinear_i8_forward: x must be f32 or f16"};
    if (wq.cols() != trit_pack::words_per_row(x.rows()))
        return Error{"bitlinear_i8_forward: wq " + shape(wq) + " does not match input rows " + std::to_string(x.rows())};
    if (tau.rows() != wq.rows() || b.rows() != wq.rows())
        return Error{"bitlinear_i8_forward: tau / bias rows do not match wq"};
    EX_TRY(x32, widen_f32(x));
    if (p == Precision::F32) return bitlinear_i8_impl(*x32, wq, tau, &b, xq_out, s_out);
    // f16: y = matmul_q_i8(..., F16), then y + b in F16 (compute_layer_bitlinear.hpp:454-456)
    EX_TRY(y, bitlinear_i8_impl(*x32, wq, tau, nullptr, xq_out, s_out));
    EX_TRY(y16, narrow_to(*y, Precision::F16));
    return add_row_broadcast(*y16, b);
}

// Default composition, exactly the reference layer's call sequence
// (include/neuralnet.cpp/compute_layer_bitlinear.hpp:443-456).
Result<Tensor> ComputeEngine::bitlinear_i8_impl(const Tensor& x, const Tensor& wq, const Tensor& tau, const Tensor* b,
                                                Tensor* xq_out, Tensor* s_out)
{
    EX_TRY(xabs, abs(x));
    EX_TRY(sraw, col_reduce_max(*xabs));
    EX_TRY_CHECK(scale_inplace(*sraw, 1.0f / 127.0f));
    EX_TRY(xq, quantize_i8(x, *sraw, true));
    EX_TRY(y, matmul_q_i8(wq, tau, *xq, *sraw));
    if (xq_out) *xq_out = *xq;
    if (s_out) *s_out = *sraw;
    if (!b) return *y;
    return add_row_broadcast(*y, *b);
}

Result<Tensor> ComputeEngine::glu(const Tensor& y1, int act)
{
    EX_TRY_CHECK(check_owned(y1, "glu"));
    EX_TRY_CHECK(require_f32(y1, "glu", "y1"));
    if (act != 0 && act != 1) return Error{"glu: act must be 0 (SwiGLU) or 1 (ReLU2GLU)"};
    if (y1.rows() % 2 != 0) return Error{"glu: input rows must be 2*d_ff, got " + shape(y1)};
    EX_TRY(out, alloc_impl(y1.rows() / 2, y1.cols(), Precision::F32));
    EX_TRY_CHECK(glu_impl(y1, act, *out));
    return *out;
}

Result<Tensor> ComputeEngine::ffn_glu_i8_forward(const Tensor& x, const Tensor* gamma, Scalar eps, const Tensor& wq1,
                                                 const Tensor& tau1, const Tensor& b1, const Tensor& wq2,
                                                 const Tensor& tau2, const Tensor& b2, int act, const Tensor* gamma_sub,
                                                 Scalar eps_sub)
{
    const char* fn = "ffn_glu_i8_forward";
    for (const Tensor* t : {&x, &wq1, &tau1, &b1, &wq2, &tau2, &b2}) EX_TRY_CHECK(check_owned(*t, fn));
    if (gamma) EX_TRY_CHECK(check_owned(*gamma, fn));
    if (gamma_sub) EX_TRY_CHECK(check_owned(*gamma_sub, fn));
    if (act != 0 && act != 1) return Error{"ffn_glu_i8_forward: act must be 0 (SwiGLU) or 1 (ReLU2GLU)"};
    const std::size_t d = x.rows(), F2 = wq1.rows();
    if (F2 % 2 != 0 || F2 == 0) return Error{"ffn_glu_i8_forward: fc1 must have 2*d_ff rows, got " + shape(wq1)};
    const std::size_t F = F2 / 2;
    if (wq1.cols() != trit_pack::words_per_row(d))
        return Error{"ffn_glu_i8_forward: fc1 " + shape(wq1) + " does not match d_model " + std::to_string(d)};
    if (wq2.rows() != d || wq2.cols() != trit_pack::words_per_row(F))
        return Error{"ffn_glu_i8_forward: fc2 " + shape(wq2) + " does not match (d_model, ceil(d_ff/16))"};
    if (tau1.rows() != F2 || b1.rows() != F2 || tau2.rows() != d || b2.rows() != d)
        return Error{"ffn_glu_i8_forward: tau / bias rows do not match the weights"};
    if (gamma && gamma->rows() != d) return Error{"ffn_glu_i8_forward: gamma must be (d_model, 1)"};
    if (gamma_sub && gamma_sub->rows() != F) return Error{"ffn_glu_i8_forward: gamma_sub must be (d_ff, 1)"};
    return ffn_glu_i8_impl(x, gamma, eps, wq1, tau1, b1, wq2, tau2, b2, act, gamma_sub, eps_sub);
}

Result<Tensor> ComputeEngine::attention_decode(const Tensor& q, const Tensor& k, const Tensor& v, Tensor& k_cache,
                                               Tensor& v_cache, std::size_t max_len, const Tensor& positions,
                                               std::size_t len_bound, const Tensor* rope_cos, const Tensor* rope_sin,
                                               std::size_t heads, std::size_t kv_heads, Scalar scale)
{
    const char* fn = "attention_decode";
    for (const Tensor* t : {&q, &k, &v, static_cast<const Tensor*>(&k_cache), static_cast<const Tensor*>(&v_cache), &positions})
        EX_TRY_CHECK(check_owned(*t, fn));
    if (kv_heads == 0 || heads % kv_heads != 0) return Error{"attention_decode: heads must be a multiple of kv_heads"};
    if (q.rows() % heads != 0) return Error{"attention_decode: q rows must be heads * d_k, got " + shape(q)};
    const std::size_t dk = q.rows() / heads, B = q.cols();
    if (k.rows() != kv_heads * dk || v.rows() != kv_heads * dk || k.cols() != B || v.cols() != B)
        return Error{"attention_decode: k / v must be (kv_heads * d_k, B), got " + shape(k) + " / " + shape(v)};
    if (max_len == 0 || k_cache.rows() != B * max_len || k_cache.cols() != kv_heads * dk ||
        v_cache.rows() != k_cache.rows() || v_cache.cols() != k_cache.cols())
        return Error{"attention_decode: caches must be (B * max_len, kv_heads * d_k), got " + shape(k_cache) + " / " +
                     shape(v_cache)};
    if (k_cache.precision() != v_cache.precision() ||
        (k_cache.precision() != Precision::F32 && k_cache.precision() != Precision::F16))
        return Error{"attention_decode: caches must both be f32 or both f16"};
    for (const Tensor* t : {&q, &k, &v})
        if (t->precision() != Precision::F32) return Error{"attention_decode: q, k and v must be f32"};
    if (positions.rows() != B || positions.cols() != 1)
        return Error{"attention_decode: positions must be (B, 1), got " + shape(positions)};
    if ((rope_cos == nullptr) != (rope_sin == nullptr)) return Error{"attention_decode: rope tables go together"};
    if (rope_cos)
    {
        EX_TRY_CHECK(check_owned(*rope_cos, fn));
        EX_TRY_CHECK(check_owned(*rope_sin, fn));
        if (rope_cos->rows() < max_len || rope_cos->cols() != dk / 2 || rope_sin->rows() != rope_cos->rows() ||
            rope_sin->cols() != dk / 2)
            return Error{"attention_decode: rope tables must be (>= max_len, d_k / 2)"};
    }
    EX_TRY(out, alloc_impl(q.rows(), B, Precision::F32));
    EpochGuard gk{k_cache}, gv{v_cache};
    EX_TRY_CHECK(attention_decode_impl(q, k, v, k_cache, v_cache, max_len, positions, len_bound, rope_cos, rope_sin,
                                       heads, kv_heads, scale, *out));
    return *out;
}

Result<Tensor> ComputeEngine::cast(const Tensor& t, Precision p)
{
    EX_TRY_CHECK(check_owned(t, "cast"));
    if (t.precision() == p) return t;
    if (p == Precision::F32 && t.precision() == Precision::F16) return widen_f32(t);
    if (p == Precision::F16 && t.precision() == Precision::F32) return narrow_to(t, Precision::F16);
    return Error{std::string("cast: only f32 <-> f16 (") + precision_name(t.precision()) + " -> " + precision_name(p) +
                 ")"};
}

Result<Tensor> ComputeEngine::add(const Tensor& x, const Tensor& y)
{
    EX_TRY_CHECK(check_owned(x, "add: x"));
    EX_TRY_CHECK(check_owned(y, "add: y"));
    EX_TRY_CHECK(require_f32(x, "add", "x"));
    EX_TRY_CHECK(require_f32(y, "add", "y"));
    if (x.rows() != y.rows() || x.cols() != y.cols()) return Error{"add: shape mismatch " + shape(x) + " vs " + shape(y)};
    EX_TRY(out, alloc_impl(x.rows(), x.cols(), Precision::F32));
    EX_TRY_CHECK(add_impl(x, y, *out));
    return *out;
}

Result<Tensor> ComputeEngine::embedding_gather(const Tensor& table, const Tensor& ids)
{
    EX_TRY_CHECK(check_owned(table, "embedding_gather: table"));
    EX_TRY_CHECK(check_owned(ids, "embedding_gather: ids"));
    if (ids.cols() != 1) return Error{"embedding_gather: ids must be (B, 1), got " + shape(ids)};
    EX_TRY(out, alloc_impl(table.cols(), ids.rows(), Precision::F32));
    EX_TRY_CHECK(embedding_gather_impl(table, ids, *out));
    return *out;
}

Result<Tensor> ComputeEngine::argmax_cols(const Tensor& logits)
{
    EX_TRY_CHECK(check_owned(logits, "argmax_cols"));
    EX_TRY_CHECK(require_f32(logits, "argmax_cols", "logits"));
    if (logits.rows() == 0) return Error{"argmax_cols: empty logits"};
    EX_TRY(out, alloc_impl(logits.cols(), 1, Precision::F32));
    EX_TRY_CHECK(argmax_cols_impl(logits, *out));
    return *out;
}

// Default composition in the reference layer order (compute_layer_feedforward.hpp:182-206).
Result<Tensor> ComputeEngine::ffn_glu_i8_impl(const Tensor& x, const Tensor* gamma, Scalar eps, const Tensor& wq1,
                                              const Tensor& tau1, const Tensor& b1, const Tensor& wq2,
                                              const Tensor& tau2, const Tensor& b2, int act, const Tensor* gamma_sub,
                                              Scalar eps_sub)
{
    Tensor in = x;
    if (gamma)
    {
        EX_TRY(n, rmsnorm(x, *gamma, eps));
        in = *n;
    }
    EX_TRY(y1, bitlinear_i8_forward(in, wq1, tau1, b1, Precision::F32, nullptr, nullptr));
    EX_TRY(h, glu(*y1, act));
    Tensor h2 = *h;
    if (gamma_sub)
    {
        EX_TRY(n, rmsnorm(*h, *gamma_sub, eps_sub));
        h2 = *n;
    }
    return bitlinear_i8_forward(h2, wq2, tau2, b2, Precision::F32, nullptr, nullptr);
}

}  // namespace nn
