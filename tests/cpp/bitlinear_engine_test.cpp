// bitlinear_engine_test — the reference's W1.58A8 acceptance checks, run through the nn::
// C++ API of libnn-hip.so on the HIP engine. Each section names the reference test it
// ports; host references are computed inline (int32 / double), never by the engine.
//   [1] ternary layout and codec           src/ternary_gemm_test.cpp [1] (:70-137)
//   [2] engine trit_pack == host pack_row  src/ternary_gemm_test.cpp [2] (:224-251)
//   [3] quantize_i8 values/NaN/s==0/layout src/int8_act_test.cpp [1] (:86-137)
//   [4] unpack_i8 round trip               src/int8_act_test.cpp [2] (:140-168)
//   [5] matmul_q_i8 bit-exact vs int32     src/int8_act_test.cpp [3] (:171-238)
//   [6] BitLinear tau / trits / forward    src/t1_58_test.cpp [5] (:207-345), int8 branch
//   [7] BitLinear int8 forward bound       src/int8_act_test.cpp [4] (:241-290), vs double
//   [8] write-epoch quant cache            AGENTS.md:160-164 / compute_layer_bitlinear.hpp:100-111
//   [9] deploy state + Model::add          compute_layer_bitlinear.hpp:359-380, model_container.hpp:91-125
//  [10] engine factory never falls back    cli/cli_engine_factory.hpp:11-13, :60-66
//  [11] matmul_q / matmul_q_t vs double   src/ternary_gemm_test.cpp [3][4] (:252-333), plus the
//       BitLinear f32-activation branch     compute_layer_bitlinear.hpp:459-466
//  [12] FeedForward (SwiGLU / ReLU2, int8)  compute_layer_feedforward.hpp:182-204: the fused
//       engine block equals the layer-by-layer composition bit for bit; RMSNorm + FeedForward
//       through Model::add equals the fused block with the norm folded in
//  [13] model files (v7 / v8)               model_serialization.hpp:38-82, :579-700, :1175-1311:
//       SHA-256 vectors (FIPS 180-2), header / entry parsing of the tests/golden fixtures
//       (host only), then load -> deploy state: packed words equal the file's bytes, repack ->
//       unpack on the GPU gives them back, forward matches the host W1.58A8 reference, and
//       save -> load reproduces the model
//  [14] decoder step (config C5)            compute_position_encoding.hpp:45-166,
//       compute_layer_attention.hpp:1003-1091, compute_layer_gpt.hpp:201-219, :693-851: RoPE
//       table == libnn-hip.so's host table; attention forward_step vs a host double evaluation
//       (rotation, GQA map, softmax) and the appended cache rows; batched forward_step ==
//       the reference single-sequence signature per sequence; GPTBlock::forward_step == its
//       composition of engine calls bit for bit; GPTModel greedy generation == forward_step +
//       the reference greedy loop on the host
//  [15] compute = F16                      src/t1_58_test.cpp [7a] (:407-460), [9] (:668-690),
//       compute_layer_bitlinear.hpp:454-456, :464-466: f16 tensors at the host boundary, BitLinear
//       under profile_t1_58 in both branches = its f32 output rounded as the reference's f16
//       product and f16 bias add, f16 inputs; cli::create_engine in the reference's shape
// Exit: 0 pass, 1 fail, 77 skip (no gfx950 device).
#include <algorithm>
#include <array>
#include <bit>
#include <cstring>
#include <memory>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <limits>
#include <random>
#include <string>
#include <vector>

#include "neuralnet.cpp/nn.hpp"
#include "nnhip.h"

namespace
{

int g_failures = 0;

#define CHECK(cond, msg)                                              \
    do                                                                \
    {                                                                 \
        if (cond) std::printf("  [ OK ] %s\n", msg);                  \
        else                                                          \
        {                                                             \
            std::printf("  [FAIL] %s  (%s:%d)\n", msg, __FILE__, __LINE__); \
            ++g_failures;                                             \
        }                                                             \
    } while (0)

nn::Matrix random_matrix(std::size_t rows, std::size_t cols, unsigned seed)
{
    nn::Matrix m(rows, cols);
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> d(-1.0f, 1.0f);
    for (auto& v : m.span()) v = d(rng);
    return m;
}

nn::Tensor upload(nn::ComputeEngine& e, const nn::Matrix& m)
{
    auto r = e.from_matrix(m);
    EX_UNWRAP(r.has_value(), "upload failed: " + r.error().message);
    return *r;
}

nn::Matrix download(nn::ComputeEngine& e, const nn::Tensor& t)
{
    auto r = e.to_matrix(t);
    EX_UNWRAP(r.has_value(), "download failed: " + r.error().message);
    return *r;
}

bool bitwise_equal(const nn::Matrix& a, const nn::Matrix& b)
{
    if (a.rows() != b.rows() || a.cols() != b.cols()) return false;
    for (std::size_t i = 0; i < a.size(); ++i)
        if (std::bit_cast<std::uint32_t>(a.span()[i]) != std::bit_cast<std::uint32_t>(b.span()[i])) return false;
    return true;
}

std::uint32_t word_of(const nn::Matrix& m, std::size_t r, std::size_t c)
{
    return std::bit_cast<std::uint32_t>(m.at(r, c));
}

// ---------------------------------------------------------------- [1]
void test_layout()
{
    std::puts("[1] ternary layout: 2 bit / weight, code = trit + 2, LSB first, tail code 2");
    using namespace nn::trit_pack;
    CHECK(kBits == 2 && kPerByte == 4 && kPerWord == 16, "size constants");
    CHECK(words_per_row(16) == 1 && words_per_row(17) == 2 && words_per_row(1) == 1, "words_per_row rounds up");
    CHECK(bytes_per_row(512) == 128, "K=512 -> 128 B per row");
    const float w[16] = {1.0f, -1.0f, 0.0f, 0.4f, -0.4f, 1.0f, -1.0f, 0.0f,
                         0.9f, -0.9f, 0.1f, -0.1f, 0.6f, -0.6f, 0.0f, 0.0f};
    const std::uint32_t expect[16] = {3, 1, 2, 2, 2, 3, 1, 2, 3, 1, 2, 2, 3, 1, 2, 2};
    std::uint32_t word[1] = {0};
    pack_row(w, 16, 1.0f, word);
    bool ok = true;
    for (std::uint32_t j = 0; j < 16; ++j)
        if (((word[0] >> (2 * j)) & 3u) != expect[j]) ok = false;
    CHECK(ok, "codes and bit order");
    std::uint32_t w2[1] = {0};
    pack_row(w, 5, 1.0f, w2);
    bool tail = true;
    for (std::size_t i = 0; i < 5; ++i)
        if (at(w2, i) != value_of(expect[i])) tail = false;
    for (std::size_t i = 5; i < 16; ++i)
        if (at(w2, i) != 0.0f) tail = false;
    CHECK(tail, "decode round trip, tail positions are trit 0 (code 2)");
}

// ---------------------------------------------------------------- [2]
void test_trit_pack(nn::ComputeEngine& e)
{
    std::puts("[2] engine trit_pack == host pack_row (K not a multiple of 16)");
    constexpr std::size_t ROWS = 7, K = 40;
    nn::Matrix W(ROWS, K);
    for (std::size_t r = 0; r < ROWS; ++r)
        for (std::size_t c = 0; c < K; ++c) W.set_value(r, c, 0.13f * static_cast<float>((r * 7 + c * 3) % 11) - 0.6f);
    nn::Matrix tau(ROWS, 1);
    for (std::size_t r = 0; r < ROWS; ++r)
    {
        double s = 0.0;
        for (std::size_t c = 0; c < K; ++c) s += std::fabs(static_cast<double>(W.at(r, c)));
        tau.set_value(r, 0, static_cast<float>(s / K));
    }
    auto packed = e.trit_pack(upload(e, W), upload(e, tau));
    CHECK(packed.has_value(), "trit_pack succeeds");
    if (!packed) return;
    CHECK(packed->rows() == ROWS && packed->cols() == nn::trit_pack::words_per_row(K), "container shape (rows, ceil(K/16))");
    const nn::Matrix pm = download(e, *packed);
    bool same = true;
    std::vector<std::uint32_t> ref(nn::trit_pack::words_per_row(K));
    for (std::size_t r = 0; r < ROWS; ++r)
    {
        nn::trit_pack::pack_row(W.span().data() + r * K, K, tau.at(r, 0), ref.data());
        for (std::size_t i = 0; i < ref.size(); ++i)
            if (word_of(pm, r, i) != ref[i]) same = false;
    }
    CHECK(same, "words bit-identical to pack_row");
    // tau on the engine = per-row absmean to 1e-6 of the double reference
    auto tau_e = e.create_tensor(ROWS, 1);
    auto ok = e.row_absmean_into(upload(e, W), tau_e);
    CHECK(ok.has_value(), "row_absmean_into succeeds");
    const nn::Matrix tm = download(e, tau_e);
    double worst = 0.0;
    for (std::size_t r = 0; r < ROWS; ++r)
        worst = std::max(worst, std::fabs(static_cast<double>(tm.at(r, 0)) - tau.at(r, 0)) / tau.at(r, 0));
    CHECK(worst < 1e-6, "engine tau = absmean (1e-6 relative)");
}

// ---------------------------------------------------------------- [3]
void test_quantize(nn::ComputeEngine& e)
{
    std::puts("[3] quantize_i8: round-half-away, clamp, s==0 -> 0, NaN -> 0, little-endian layout");
    constexpr std::size_t M = 5, N = 7;
    nn::Matrix xm = random_matrix(M, N, 11);
    nn::Matrix sm(1, N);
    for (std::size_t c = 0; c < N; ++c)
    {
        float mx = 0.0f;
        for (std::size_t r = 0; r < M; ++r) mx = std::max(mx, std::fabs(xm.span()[r * N + c]));
        sm.span()[c] = mx;
    }
    for (std::size_t r = 0; r < M; ++r) xm.span()[r * N + 0] = 0.0f;
    xm.span()[1 * N + 1] = std::numeric_limits<float>::quiet_NaN();
    auto q = e.quantize_i8(upload(e, xm), upload(e, sm), true);
    CHECK(q.has_value(), "quantize_i8 succeeds");
    if (!q) return;
    const nn::Matrix qm = download(e, *q);
    const std::size_t wpr = nn::i8_pack::words_per_row(N);
    CHECK(qm.rows() == M && qm.cols() == wpr, "container shape (M, ceil(N/4))");
    bool value_ok = true, layout_ok = true;
    for (std::size_t r = 0; r < M; ++r)
    {
        std::vector<std::uint32_t> words(wpr);
        for (std::size_t wi = 0; wi < wpr; ++wi) words[wi] = word_of(qm, r, wi);
        for (std::size_t c = 0; c < N; ++c)
        {
            const std::int8_t want = nn::i8_pack::quantize(xm.span()[r * N + c], sm.span()[c]);
            const std::int8_t got = nn::i8_pack::at(words.data(), c);
            if (got != want) value_ok = false;
            if ((words[c / 4] >> (8 * (c % 4)) & 0xFFu) != static_cast<std::uint8_t>(got)) layout_ok = false;
        }
        if ((words[wpr - 1] >> 24) != 0u) layout_ok = false;  // tail byte
    }
    CHECK(value_ok, "values equal the host quantize (incl. s==0 column and NaN)");
    CHECK(layout_ok, "little-endian bytes, tail byte 0");
}

// ---------------------------------------------------------------- [4]
void test_unpack(nn::ComputeEngine& e)
{
    std::puts("[4] unpack_i8: container -> f32 integers");
    constexpr std::size_t M = 3, N = 6;
    const nn::Matrix xm = random_matrix(M, N, 23);
    nn::Matrix sm(1, N);
    for (std::size_t c = 0; c < N; ++c) sm.span()[c] = std::max(0.3f, std::fabs(xm.span()[c]) + 0.1f);
    auto q = e.quantize_i8(upload(e, xm), upload(e, sm), true);
    CHECK(q.has_value(), "quantize_i8 succeeds");
    if (!q) return;
    auto u = e.unpack_i8(*q, N);
    CHECK(u.has_value(), "unpack_i8 succeeds");
    if (!u) return;
    const nn::Matrix um = download(e, *u);
    bool ok = um.rows() == M && um.cols() == N;
    for (std::size_t r = 0; r < M && ok; ++r)
        for (std::size_t c = 0; c < N; ++c)
            if (um.at(r, c) != static_cast<float>(nn::i8_pack::quantize(xm.at(r, c), sm.at(0, c)))) ok = false;
    CHECK(ok, "values are the quantized integers, exactly");
}

// ---------------------------------------------------------------- [5]
bool test_matmul_q_i8_shape(nn::ComputeEngine& e, std::size_t OUT, std::size_t K, std::size_t N, unsigned seed,
                            const char* label)
{
    std::printf("[5] matmul_q_i8 (%s): bit-identical to the host int32 loop\n", label);
    const nn::Matrix wm = random_matrix(OUT, K, seed);
    nn::Matrix tm(OUT, 1);
    for (std::size_t r = 0; r < OUT; ++r)
    {
        double acc = 0.0;
        for (std::size_t k = 0; k < K; ++k) acc += std::fabs(static_cast<double>(wm.span()[r * K + k]));
        tm.span()[r] = static_cast<float>(acc / static_cast<double>(K));
    }
    const nn::Matrix xm = random_matrix(K, N, seed + 1);
    nn::Matrix sm(1, N);
    for (std::size_t c = 0; c < N; ++c)
    {
        float mx = 0.0f;
        for (std::size_t k = 0; k < K; ++k) mx = std::max(mx, std::fabs(xm.span()[k * N + c]));
        sm.span()[c] = mx;
    }
    const nn::Tensor wt = upload(e, wm), tt = upload(e, tm), xt = upload(e, xm), st = upload(e, sm);
    auto pw = e.trit_pack(wt, tt);
    auto px = e.quantize_i8(xt, st, true);
    CHECK(pw.has_value() && px.has_value(), "trit_pack / quantize_i8 succeed");
    if (!pw || !px) return false;
    auto y = e.matmul_q_i8(*pw, tt, *px, st);
    CHECK(y.has_value(), "matmul_q_i8 succeeds");
    if (!y) return false;
    const nn::Matrix ym = download(e, *y), qm = download(e, *px);
    const std::size_t wpr_w = nn::trit_pack::words_per_row(K), wpr_q = nn::i8_pack::words_per_row(N);
    std::vector<std::uint32_t> tw(wpr_w), qw(wpr_q);
    nn::Matrix ref(OUT, N);
    for (std::size_t m = 0; m < OUT; ++m)
    {
        nn::trit_pack::pack_row(wm.span().data() + m * K, K, tm.span()[m], tw.data());
        for (std::size_t n = 0; n < N; ++n)
        {
            std::int32_t acc = 0;
            for (std::size_t k = 0; k < K; ++k)
            {
                const std::uint32_t code = (tw[k / 16] >> (2 * (k % 16))) & 3u;
                for (std::size_t wi = 0; wi < wpr_q; ++wi) qw[wi] = word_of(qm, k, wi);
                acc += static_cast<std::int32_t>(nn::trit_pack::value_of(code)) *
                       static_cast<std::int32_t>(nn::i8_pack::at(qw.data(), n));
            }
            ref.span()[m * N + n] = tm.span()[m] * sm.span()[n] * static_cast<float>(acc);
        }
    }
    CHECK(bitwise_equal(ym, ref), "bitwise equal ((tau*s)*float(acc) epilogue order)");
    return true;
}

// ---------------------------------------------------------------- [6]
void test_bitlinear_rules(nn::ComputeEngine& e)
{
    std::puts("[6] BitLinear: tau = per-row absmean, trits = RoundClip(W/tau,-1,1), forward");
    constexpr std::size_t IN = 4, OUT = 3, B = 2;
    const float kRawW[OUT][IN] = {{1.0f, 0.3f, -0.3f, 0.3f}, {0.4f, -0.4f, 0.1f, -0.1f}, {0.7f, 0.6f, 0.5f, 0.1f}};
    const float kX[IN][B] = {{1.f, -2.f}, {0.5f, 1.f}, {-1.f, 0.25f}, {2.f, -0.5f}};
    nn::BitLinear bl(IN, OUT);
    nn::PrecisionProfile prof;
    prof.param = nn::Precision::T1_58;
    bl.set_precision_profile(prof);
    auto ir = bl.init(e);
    CHECK(ir.has_value(), "BitLinear + param=T1_58 init");
    if (!ir) return;
    nn::Matrix W(OUT, IN), X(IN, B);
    for (std::size_t o = 0; o < OUT; ++o)
        for (std::size_t k = 0; k < IN; ++k) W.set_value(o, k, kRawW[o][k]);
    for (std::size_t k = 0; k < IN; ++k)
        for (std::size_t b = 0; b < B; ++b) X.set_value(k, b, kX[k][b]);
    CHECK(e.copy_from(bl.parameters()[0].get(), W).has_value(), "write known latent weights");
    bl.set_activation_quant(true);
    auto y = bl.forward(upload(e, X));
    CHECK(y.has_value(), "forward (int8 branch)");
    if (!y) return;
    double tau_ref[OUT], wq_ref[OUT][IN];
    for (std::size_t o = 0; o < OUT; ++o)
    {
        double s = 0.0;
        for (std::size_t k = 0; k < IN; ++k) s += std::fabs(static_cast<double>(kRawW[o][k]));
        tau_ref[o] = s / IN;
        for (std::size_t k = 0; k < IN; ++k)
        {
            const double w = kRawW[o][k];
            wq_ref[o][k] = (w > 0.5 * tau_ref[o]) ? 1.0 : (w < -0.5 * tau_ref[o]) ? -1.0 : 0.0;
        }
    }
    const nn::Matrix tau = download(e, bl.row_scales());
    bool tau_ok = tau.rows() == OUT && tau.cols() == 1;
    for (std::size_t o = 0; o < OUT && tau_ok; ++o)
        if (std::fabs(static_cast<double>(tau.at(o, 0)) - tau_ref[o]) >= 1e-6) tau_ok = false;
    CHECK(tau_ok, "tau = {0.475, 0.25, 0.475} (1e-6)");
    const nn::Matrix packed = download(e, bl.quantized_weights_packed());
    bool exact = true;
    for (std::size_t o = 0; o < OUT; ++o)
    {
        const std::uint32_t wd = word_of(packed, o, 0);
        for (std::size_t k = 0; k < IN; ++k)
            if (static_cast<double>(nn::trit_pack::at(&wd, k)) != wq_ref[o][k]) exact = false;
    }
    CHECK(exact, "packed trits equal RoundClip(W/tau,-1,1); 0.3 survives absmean scaling");
    // forward = (tau * s) * sum(trit * q) with s = absmax/127 (q = int8 activations)
    const nn::Matrix Y = download(e, *y);
    bool fwd = true;
    for (std::size_t b = 0; b < B; ++b)
    {
        float mx = 0.0f;
        for (std::size_t k = 0; k < IN; ++k) mx = std::max(mx, std::fabs(kX[k][b]));
        const float s = mx * (1.0f / 127.0f);
        for (std::size_t o = 0; o < OUT; ++o)
        {
            std::int32_t acc = 0;
            for (std::size_t k = 0; k < IN; ++k)
                acc += static_cast<std::int32_t>(wq_ref[o][k]) * nn::i8_pack::quantize(kX[k][b], s);
            const float ref = (tau.at(o, 0) * s) * static_cast<float>(acc) + 0.0f;
            if (std::bit_cast<std::uint32_t>(Y.at(o, b)) != std::bit_cast<std::uint32_t>(ref)) fwd = false;
        }
    }
    CHECK(fwd, "forward bit-identical to the host W1.58A8 reference (bias 0)");
}

// ---------------------------------------------------------------- [7]
void test_bitlinear_bound(nn::ComputeEngine& e)
{
    std::puts("[7] BitLinear int8 forward vs float64 dequantized product: |dY| <= tau*s*K/2");
    constexpr std::size_t IN = 64, OUT = 32, B = 8;
    nn::BitLinear layer(IN, OUT);
    nn::PrecisionProfile t1;
    t1.param = nn::Precision::T1_58;
    layer.set_precision_profile(t1);
    EX_UNWRAP(layer.init(e).has_value(), "init");
    layer.set_activation_quant(true);
    const nn::Matrix xm = random_matrix(IN, B, 5);
    auto y = layer.forward(upload(e, xm));
    CHECK(y.has_value(), "forward");
    if (!y) return;
    const nn::Matrix ym = download(e, *y), lm = download(e, layer.latent_weights());
    const nn::Matrix tm = download(e, layer.row_scales());
    double worst = 0.0;
    for (std::size_t n = 0; n < B; ++n)
    {
        float mx = 0.0f;
        for (std::size_t r = 0; r < IN; ++r) mx = std::max(mx, std::fabs(xm.at(r, n)));
        const double s = mx / 127.0;
        for (std::size_t m = 0; m < OUT; ++m)
        {
            const double tau = tm.at(m, 0);
            double ref = 0.0;
            for (std::size_t k = 0; k < IN; ++k)
            {
                const double w = lm.at(m, k);
                const double t = (w > 0.5 * tau) ? 1.0 : (w < -0.5 * tau) ? -1.0 : 0.0;
                ref += tau * t * static_cast<double>(xm.at(k, n));
            }
            const double bound = tau * s * IN * 0.5;
            if (bound > 0.0) worst = std::max(worst, std::fabs(ym.at(m, n) - ref) / bound);
        }
    }
    std::printf("    diff / bound worst = %.4f\n", worst);
    CHECK(worst <= 1.0, "within the 8-bit quantization bound");
}

// ---------------------------------------------------------------- [8]
void test_quant_cache(nn::ComputeEngine& e)
{
    std::puts("[8] quantized weights are recomputed only when the latent weights change");
    nn::BitLinear layer(48, 20);
    nn::PrecisionProfile t1;
    t1.param = nn::Precision::T1_58;
    layer.set_precision_profile(t1);
    EX_UNWRAP(layer.init(e).has_value(), "init");
    layer.set_activation_quant(true);
    const nn::Tensor x = upload(e, random_matrix(48, 3, 9));
    auto y1 = layer.forward(x);
    auto y2 = layer.forward(x);
    CHECK(y1.has_value() && y2.has_value() && layer.quantize_calls() == 1, "two forwards, one quantization");
    CHECK(bitwise_equal(download(e, *y1), download(e, *y2)), "repeat forward is bit-identical");
    CHECK(e.copy_from(layer.parameters()[0].get(), random_matrix(20, 48, 10)).has_value(), "write new latent");
    auto y3 = layer.forward(x);
    CHECK(y3.has_value() && layer.quantize_calls() == 2, "write epoch advanced -> requantized");
    CHECK(!bitwise_equal(download(e, *y1), download(e, *y3)), "new weights change the output");
}

// ---------------------------------------------------------------- [9]
void test_deploy_and_model(nn::ComputeEngine& e)
{
    std::puts("[9] packed-only deploy state and Model::add<BitLinear>");
    constexpr std::size_t IN = 80, HID = 40, OUT = 24, B = 5;
    nn::PrecisionProfile t1;
    t1.param = nn::Precision::T1_58;
    nn::BitLinear trained(IN, HID);
    trained.set_precision_profile(t1);
    EX_UNWRAP(trained.init(e).has_value(), "init");
    trained.set_activation_quant(true);
    const nn::Tensor x = upload(e, random_matrix(IN, B, 77));
    auto y_ref = trained.forward(x);
    CHECK(y_ref.has_value(), "trained-layer forward");
    // deploy: a layer built without latent weights, fed the packed words + tau
    nn::BitLinear deployed(IN, HID, /*inference_only=*/true);
    deployed.set_precision_profile(t1);
    EX_UNWRAP(deployed.init(e).has_value(), "init deploy");
    deployed.set_activation_quant(true);
    auto words = e.from_matrix(download(e, trained.quantized_weights_packed()));
    auto tau = e.from_matrix(download(e, trained.row_scales()));
    CHECK(deployed.load_packed_weights(*words, *tau).has_value() && deployed.packed_only(), "load_packed_weights");
    auto y_dep = deployed.forward(x);
    CHECK(y_dep.has_value() && bitwise_equal(download(e, *y_ref), download(e, *y_dep)),
          "deployed forward bit-identical to the trained layer");
    CHECK(!deployed.backward(x).has_value(), "deploy state refuses backward (fail fast)");

    nn::Model model(e);
    model.set_default_precision_profile(t1);
    CHECK(model.add<nn::BitLinear>(IN, HID).has_value(), "Model::add<BitLinear>");
    nn::PrecisionProfile f32;
    nn::Model norm_model(e);
    norm_model.set_default_precision_profile(f32);
    CHECK(!norm_model.add<nn::BitLinear>(IN, HID).has_value(), "param=f32 rejected by BitLinear (precision_support)");
    CHECK(model.add<nn::BitLinear>(HID, OUT).has_value(), "second BitLinear");
    for (std::size_t i = 0; i < model.num_layers(); ++i)
        static_cast<nn::BitLinear&>(model.layer_at(i)).set_activation_quant(true);
    auto my = model.forward(x);
    CHECK(my.has_value() && my->rows() == OUT && my->cols() == B, "Model::forward through two BitLinears");
    // RMSNorm -> BitLinear: the norm's output quantized by the layer
    nn::RMSNorm norm(IN, 1e-6f);
    EX_UNWRAP(norm.init(e).has_value(), "rmsnorm init");
    auto nx = norm.forward(x);
    CHECK(nx.has_value(), "RMSNorm forward");
    if (nx)
    {
        const nn::Matrix xm = download(e, x), nm = download(e, *nx);
        double worst = 0.0;
        for (std::size_t b = 0; b < B; ++b)
        {
            double ss = 0.0;
            for (std::size_t f = 0; f < IN; ++f) ss += static_cast<double>(xm.at(f, b)) * xm.at(f, b);
            const double ri = 1.0 / std::sqrt(ss / IN + 1e-6);
            for (std::size_t f = 0; f < IN; ++f)
                worst = std::max(worst, std::fabs(nm.at(f, b) - xm.at(f, b) * ri) / std::max(1e-3, std::fabs(xm.at(f, b) * ri)));
        }
        CHECK(worst < 2e-6, "RMSNorm matches the float64 formula");
    }
}

// ---------------------------------------------------------------- [10]
void test_factory()
{
    std::puts("[10] engine factory: explicit backends, no silent fallback");
    nn::cli::EngineConfig none;
    CHECK(!nn::cli::create_engine(none).has_value(), "no backend requested -> error, not a CPU fallback");
    CHECK(nn::create_hip_engine("hip:x") == nullptr && std::string(nn::last_error()).find("bad device") != std::string::npos,
          "malformed device string -> error");
}


// ---------------------------------------------------------------- [11]
// Host (tau o trit) product in double; trans = false: W (rows, k) . B; trans = true: the
// stored (rows = K, k = M) container transposed, tau per stored row.
nn::Matrix host_float_product(const std::vector<double>& trit, const std::vector<float>& tau, std::size_t rows,
                              std::size_t k, const nn::Matrix& B, bool trans)
{
    const std::size_t n_out = trans ? k : rows, red = trans ? rows : k;
    nn::Matrix out(n_out, B.cols());
    for (std::size_t o = 0; o < n_out; ++o)
        for (std::size_t c = 0; c < B.cols(); ++c)
        {
            double acc = 0.0;
            for (std::size_t r = 0; r < red; ++r)
            {
                const std::size_t row = trans ? r : o, col = trans ? o : r;
                acc += static_cast<double>(tau[row] * static_cast<float>(trit[row * k + col])) *
                       static_cast<double>(B.at(r, c));
            }
            out.set_value(o, c, static_cast<float>(acc));
        }
    return out;
}

double max_abs_diff(const nn::Matrix& a, const nn::Matrix& b)
{
    if (a.rows() != b.rows() || a.cols() != b.cols()) return std::numeric_limits<double>::infinity();
    double mx = 0.0;
    for (std::size_t i = 0; i < a.size(); ++i)
        mx = std::max(mx, std::fabs(static_cast<double>(a.span()[i]) - static_cast<double>(b.span()[i])));
    return mx;
}

// Packs `W` (rows, k) with per-row tau on the engine and returns the trits it encodes.
bool pack_on_engine(nn::ComputeEngine& e, const nn::Matrix& W, const std::vector<float>& tau, nn::Tensor& packed,
                    nn::Tensor& tau_t, std::vector<double>& trit)
{
    nn::Matrix tm(W.rows(), 1);
    for (std::size_t r = 0; r < W.rows(); ++r) tm.set_value(r, 0, tau[r]);
    tau_t = upload(e, tm);
    auto pk = e.trit_pack(upload(e, W), tau_t);
    if (!pk) return false;
    packed = *pk;
    trit.assign(W.size(), 0.0);
    for (std::size_t r = 0; r < W.rows(); ++r)
        for (std::size_t c = 0; c < W.cols(); ++c)
            trit[r * W.cols() + c] = nn::trit_pack::value_of(nn::trit_pack::code_of(W.at(r, c), tau[r]));
    return true;
}

void test_float_products(nn::ComputeEngine& e)
{
    std::puts("[11] matmul_q / matmul_q_t (float activations) vs the double host product");
    {
        // the reference's deterministic patterns, K = 40 not a multiple of 16
        constexpr std::size_t ROWS = 7, K = 40, N = 3;
        nn::Matrix W(ROWS, K), X(K, N);
        for (std::size_t r = 0; r < ROWS; ++r)
            for (std::size_t c = 0; c < K; ++c) W.set_value(r, c, 0.13f * static_cast<float>((r * 7 + c * 3) % 11) - 0.6f);
        for (std::size_t k = 0; k < K; ++k)
            for (std::size_t n = 0; n < N; ++n) X.set_value(k, n, 0.21f * static_cast<float>((k + 2 * n) % 9) - 0.8f);
        std::vector<float> tau(ROWS);
        for (std::size_t r = 0; r < ROWS; ++r)
        {
            double s = 0.0;
            for (std::size_t c = 0; c < K; ++c) s += std::fabs(static_cast<double>(W.at(r, c)));
            tau[r] = static_cast<float>(s / static_cast<double>(K));
        }
        nn::Tensor pk, tt;
        std::vector<double> trit;
        CHECK(pack_on_engine(e, W, tau, pk, tt, trit), "trit_pack (W)");
        const nn::Tensor Xt = upload(e, X);
        auto y = e.matmul_q(pk, tt, Xt);
        CHECK(y.has_value() && max_abs_diff(download(e, *y), host_float_product(trit, tau, ROWS, K, X, false)) < 1e-5,
              "matmul_q = (tau o trit) . X (1e-5)");
        // A stored (K, M = ROWS), tau 0.5 per stored row
        nn::Matrix A(K, ROWS);
        for (std::size_t k = 0; k < K; ++k)
            for (std::size_t m = 0; m < ROWS; ++m) A.set_value(k, m, 0.19f * static_cast<float>((k * 5 + m * 3) % 7) - 0.5f);
        const std::vector<float> tau_k(K, 0.5f);
        nn::Tensor pa, ta;
        std::vector<double> trit_a;
        CHECK(pack_on_engine(e, A, tau_k, pa, ta, trit_a), "trit_pack (A, transposed form)");
        auto yt = e.matmul_q_t(pa, ta, Xt, ROWS);
        CHECK(yt.has_value() && yt->rows() == ROWS && yt->cols() == N, "matmul_q_t output shape (M, N)");
        CHECK(yt.has_value() &&
                  max_abs_diff(download(e, *yt), host_float_product(trit_a, tau_k, K, ROWS, X, true)) < 1e-5,
              "matmul_q_t = (tau o trit)^T . X (1e-5)");
        CHECK(!e.matmul_q_t(pa, ta, Xt, ROWS + 16).has_value(), "matmul_q_t rejects an M the container cannot hold");
        CHECK(!e.matmul_q(pk, ta, Xt).has_value(), "matmul_q rejects a tau of the wrong length");
    }
    {
        // decode-sized random case, relative tolerance of the reference's cross-shape check
        constexpr std::size_t ROWS = 300, K = 2560, N = 2;
        const nn::Matrix W = random_matrix(ROWS, K, 71), X = random_matrix(K, N, 72);
        std::vector<float> tau(ROWS);
        for (std::size_t r = 0; r < ROWS; ++r)
        {
            double s = 0.0;
            for (std::size_t c = 0; c < K; ++c) s += std::fabs(static_cast<double>(W.at(r, c)));
            tau[r] = static_cast<float>(s / static_cast<double>(K));
        }
        nn::Tensor pk, tt;
        std::vector<double> trit;
        CHECK(pack_on_engine(e, W, tau, pk, tt, trit), "trit_pack (300 x 2560)");
        auto y = e.matmul_q(pk, tt, upload(e, X));
        bool ok = y.has_value();
        if (ok)
        {
            const nn::Matrix g = download(e, *y), ref = host_float_product(trit, tau, ROWS, K, X, false);
            for (std::size_t i = 0; i < ref.size() && ok; ++i)
                ok = std::fabs(static_cast<double>(g.span()[i]) - static_cast<double>(ref.span()[i])) <=
                     1e-4 * std::max(1.0, std::fabs(static_cast<double>(ref.span()[i])));
        }
        CHECK(ok, "matmul_q 300 x 2560, N=2 within 1e-4 x max(1, |ref|)");
    }
    {
        std::puts("[11] BitLinear f32-activation branch (activation quantization off)");
        constexpr std::size_t IN = 24, OUT = 9, B = 4;  // IN not a multiple of 16
        nn::BitLinear bl(IN, OUT);
        nn::PrecisionProfile prof;
        prof.param = nn::Precision::T1_58;
        bl.set_precision_profile(prof);
        CHECK(bl.init(e).has_value(), "BitLinear init");
        const nn::Matrix W = random_matrix(OUT, IN, 81), X = random_matrix(IN, B, 82);
        nn::Matrix bias(OUT, 1);
        for (std::size_t o = 0; o < OUT; ++o) bias.set_value(o, 0, 0.125f * static_cast<float>(o) - 0.5f);
        CHECK(e.copy_from(bl.parameters()[0].get(), W).has_value(), "write latent weights");
        CHECK(e.copy_from(bl.parameters()[1].get(), bias).has_value(), "write bias");
        bl.set_activation_quant(false);
        auto y = bl.forward(upload(e, X));
        CHECK(y.has_value(), "forward (f32 branch)");
        if (!y) return;
        const nn::Matrix tau_m = download(e, bl.row_scales());
        std::vector<float> tau(OUT);
        for (std::size_t o = 0; o < OUT; ++o) tau[o] = tau_m.at(o, 0);
        std::vector<double> trit(OUT * IN);
        for (std::size_t o = 0; o < OUT; ++o)
            for (std::size_t k = 0; k < IN; ++k)
                trit[o * IN + k] = nn::trit_pack::value_of(nn::trit_pack::code_of(W.at(o, k), tau[o]));
        nn::Matrix ref = host_float_product(trit, tau, OUT, IN, X, false);
        for (std::size_t o = 0; o < OUT; ++o)
            for (std::size_t b = 0; b < B; ++b) ref.set_value(o, b, ref.at(o, b) + bias.at(o, 0));
        CHECK(max_abs_diff(download(e, *y), ref) < 1e-5, "forward = (tau o trit) . X + b (1e-5)");
        CHECK(!bl.activation_scales().valid() && bl.input_cache().rows() == IN, "f32 branch caches the input");
    }
}

// ---------------------------------------------------------------- [12]
void test_feedforward(nn::ComputeEngine& e)
{
    std::puts("[12] FeedForward: fused gated block == layer-by-layer composition");
    constexpr std::size_t D = 48, F = 40, B = 5;  // F not a multiple of 8 or 16
    for (const auto act : {nn::ActivationType::SwiGLU, nn::ActivationType::ReLU2})
    {
        const int a = act == nn::ActivationType::ReLU2 ? 1 : 0;
        nn::FeedForward ff(D, F, act, false, nn::NormType::LayerNorm, nn::WeightQuant::T1_58);
        nn::PrecisionProfile prof;
        prof.param = nn::Precision::T1_58;
        ff.set_precision_profile(prof);
        CHECK(ff.init(e).has_value(), a ? "FeedForward(ReLU2) init" : "FeedForward(SwiGLU) init");
        if (!ff.fc1().latent_weights().valid()) return;
        auto params = ff.parameters();  // fc1 latent, fc1 bias, fc2 latent, fc2 bias
        CHECK(params.size() == 4, "parameters: two latents and two biases");
        if (params.size() != 4) return;
        CHECK(e.copy_from(params[0].get(), random_matrix(2 * F, D, 91)).has_value() &&
                  e.copy_from(params[1].get(), random_matrix(2 * F, 1, 92)).has_value() &&
                  e.copy_from(params[2].get(), random_matrix(D, F, 93)).has_value() &&
                  e.copy_from(params[3].get(), random_matrix(D, 1, 94)).has_value(),
              "write latent weights and biases");
        ff.set_activation_quant(true);
        const nn::Tensor x = upload(e, random_matrix(D, B, 95));
        auto y = ff.forward(x);
        CHECK(y.has_value() && y->rows() == D && y->cols() == B, "fused forward");
        if (!y) return;
        auto h1 = ff.fc1().forward(x);
        auto h2 = h1 ? e.glu(*h1, a) : nn::Result<nn::Tensor>(nn::Error{"fc1 failed"});
        auto y2 = h2 ? ff.fc2().forward(*h2) : nn::Result<nn::Tensor>(nn::Error{"glu failed"});
        CHECK(y2.has_value() && bitwise_equal(download(e, *y), download(e, *y2)),
              "fused block bit-identical to fc1 -> glu -> fc2");
        // with RMSNorm in front (config C4's block): Model of two layers vs the fused call
        nn::Model model(e);  // default f32 profile: the FeedForward gives its projections T1_58
        CHECK(model.add<nn::RMSNorm>(D, 1e-6f).has_value(), "Model::add<RMSNorm>");
        CHECK(model.add<nn::FeedForward>(D, F, act, false, nn::NormType::LayerNorm, nn::WeightQuant::T1_58).has_value(),
              "Model::add<FeedForward>");
        if (model.num_layers() != 2) return;
        auto& mff = static_cast<nn::FeedForward&>(model.layer_at(1));
        auto mp = mff.parameters();
        (void)e.copy_from(mp[0].get(), random_matrix(2 * F, D, 91));
        (void)e.copy_from(mp[1].get(), random_matrix(2 * F, 1, 92));
        (void)e.copy_from(mp[2].get(), random_matrix(D, F, 93));
        (void)e.copy_from(mp[3].get(), random_matrix(D, 1, 94));
        mff.set_activation_quant(true);
        auto ym = model.forward(x);
        CHECK(ym.has_value(), "Model forward (RMSNorm, FeedForward)");
        auto& norm = static_cast<nn::RMSNorm&>(model.layer_at(0));
        auto yf = e.ffn_glu_i8_forward(x, &norm.gamma(), 1e-6f, mff.fc1().quantized_weights_packed(),
                                       mff.fc1().row_scales(), mff.fc1().bias(), mff.fc2().quantized_weights_packed(),
                                       mff.fc2().row_scales(), mff.fc2().bias(), a);
        CHECK(ym.has_value() && yf.has_value() && bitwise_equal(download(e, *ym), download(e, *yf)),
              "RMSNorm + FeedForward == one fused block with the norm folded in");
        ff.set_activation_quant(false);
        auto yf32 = ff.forward(x);
        bool finite = yf32.has_value();
        if (finite)
            for (float v : download(e, *yf32).span()) finite = finite && std::isfinite(v);
        CHECK(finite, "f32-activation branch (matmul_q) runs");
    }
    // SubLN: RMSNorm(d_ff, eps 1e-5) of the gated output before fc2; its gamma is the fifth entry
    {
        nn::FeedForward sf(D, F, nn::ActivationType::SwiGLU, true, nn::NormType::RMSNorm, nn::WeightQuant::T1_58);
        CHECK(sf.init(e).has_value(), "FeedForward(SwiGLU, SubLN) init");
        auto sp = sf.parameters();  // fc1 latent, fc1 bias, fc2 latent, fc2 bias, SubLN gamma
        CHECK(sp.size() == 5 && sf.param_count() == 5 && sf.sub_norm() != nullptr, "SubLN adds one parameter");
        if (sp.size() == 5 && sf.sub_norm())
        {
            CHECK(e.copy_from(sp[0].get(), random_matrix(2 * F, D, 191)).has_value() &&
                      e.copy_from(sp[1].get(), random_matrix(2 * F, 1, 192)).has_value() &&
                      e.copy_from(sp[2].get(), random_matrix(D, F, 193)).has_value() &&
                      e.copy_from(sp[3].get(), random_matrix(D, 1, 194)).has_value() &&
                      e.copy_from(sp[4].get(), random_matrix(F, 1, 195)).has_value(),
                  "write SubLN block parameters");
            sf.set_activation_quant(true);
            const nn::Tensor x = upload(e, random_matrix(D, B, 196));
            auto y = sf.forward(x);
            auto h1 = sf.fc1().forward(x);
            auto h2 = h1 ? e.glu(*h1, 0) : nn::Result<nn::Tensor>(nn::Error{"fc1 failed"});
            auto h3 = h2 ? sf.sub_norm()->forward(*h2) : nn::Result<nn::Tensor>(nn::Error{"glu failed"});
            auto y2 = h3 ? sf.fc2().forward(*h3) : nn::Result<nn::Tensor>(nn::Error{"sub_norm failed"});
            CHECK(y.has_value() && y2.has_value() && bitwise_equal(download(e, *y), download(e, *y2)),
                  "fused SubLN block bit-identical to fc1 -> glu -> RMSNorm -> fc2");
            auto g = sf.export_param(4, nn::ModelRole::Model);
            CHECK(g.has_value() && g->kind == nn::ParamKind::Dense && g->rows == F, "SubLN gamma exports Dense");
        }
    }
    // SubLN of the reference's default norm type, LayerNorm(d_ff, eps 1e-5): gamma and beta are the
    // fifth and sixth entries; the block runs fc1 -> glu -> LayerNorm -> fc2 (no fused form)
    {
        nn::FeedForward lf(D, F, nn::ActivationType::SwiGLU, true, nn::NormType::LayerNorm, nn::WeightQuant::T1_58);
        CHECK(lf.init(e).has_value() && lf.sub_layernorm() != nullptr && lf.sub_rmsnorm() == nullptr,
              "FeedForward(SwiGLU, LayerNorm SubLN) init");
        auto lp = lf.parameters();  // fc1 latent, fc1 bias, fc2 latent, fc2 bias, SubLN gamma, SubLN beta
        CHECK(lp.size() == 6 && lf.param_count() == 6, "LayerNorm SubLN adds two parameters");
        if (lp.size() == 6 && lf.sub_layernorm())
        {
            const nn::Matrix gm = download(e, lp[4].get()), bm = download(e, lp[5].get());
            bool init_ok = gm.rows() == F && bm.rows() == F;
            for (std::size_t i = 0; init_ok && i < F; ++i) init_ok = gm.at(i, 0) == 1.0f && bm.at(i, 0) == 0.0f;
            CHECK(init_ok, "LayerNorm gamma starts at 1, beta at 0");
            CHECK(e.copy_from(lp[0].get(), random_matrix(2 * F, D, 291)).has_value() &&
                      e.copy_from(lp[1].get(), random_matrix(2 * F, 1, 292)).has_value() &&
                      e.copy_from(lp[2].get(), random_matrix(D, F, 293)).has_value() &&
                      e.copy_from(lp[3].get(), random_matrix(D, 1, 294)).has_value() &&
                      e.copy_from(lp[4].get(), random_matrix(F, 1, 295)).has_value() &&
                      e.copy_from(lp[5].get(), random_matrix(F, 1, 296)).has_value(),
                  "write LayerNorm SubLN block parameters");
            lf.set_activation_quant(true);
            const nn::Tensor x = upload(e, random_matrix(D, B, 297));
            auto y = lf.forward(x);
            auto h1 = lf.fc1().forward(x);
            auto h2 = h1 ? e.glu(*h1, 0) : nn::Result<nn::Tensor>(nn::Error{"fc1 failed"});
            auto h3 = h2 ? lf.sub_layernorm()->forward(*h2) : nn::Result<nn::Tensor>(nn::Error{"glu failed"});
            auto y2 = h3 ? lf.fc2().forward(*h3) : nn::Result<nn::Tensor>(nn::Error{"sub_norm failed"});
            CHECK(y.has_value() && y2.has_value() && bitwise_equal(download(e, *y), download(e, *y2)),
                  "LayerNorm SubLN block bit-identical to fc1 -> glu -> LayerNorm -> fc2");
            // the LayerNorm itself against a host double evaluation of the reference formula
            bool ln_ok = h2.has_value() && h3.has_value();
            double err = 0;
            if (ln_ok)
            {
                const nn::Matrix H = download(e, *h2), O = download(e, *h3);
                const nn::Matrix G = download(e, lp[4].get()), Bt = download(e, lp[5].get());
                for (std::size_t b = 0; b < B; ++b)
                {
                    double mean = 0, var = 0;
                    for (std::size_t f = 0; f < F; ++f) mean += H.at(f, b);
                    mean /= F;
                    for (std::size_t f = 0; f < F; ++f) var += (H.at(f, b) - mean) * (H.at(f, b) - mean);
                    var /= F;
                    for (std::size_t f = 0; f < F; ++f)
                    {
                        const double r = (H.at(f, b) - mean) / std::sqrt(var + 1e-5) * G.at(f, 0) + Bt.at(f, 0);
                        err = std::max(err, std::abs(O.at(f, b) - r) / std::max(1.0, std::abs(r)));
                    }
                }
            }
            CHECK(ln_ok && err < 1e-5, "LayerNorm forward within 1e-5 of a host double evaluation");
            auto bt = lf.export_param(5, nn::ModelRole::Model);
            CHECK(bt.has_value() && bt->kind == nn::ParamKind::Dense && bt->rows == F, "SubLN beta exports Dense");
        }
    }
    nn::FeedForward gelu(8, 8, nn::ActivationType::GeLU, false, nn::NormType::LayerNorm, nn::WeightQuant::T1_58);
    nn::PrecisionProfile prof;
    prof.param = nn::Precision::T1_58;
    gelu.set_precision_profile(prof);
    CHECK(!gelu.init(e).has_value(), "GeLU FeedForward is refused (only gated activations)");
    nn::FeedForward lin(8, 8, nn::ActivationType::SwiGLU);  // the reference's defaults: WeightQuant::None
    CHECK(!lin.init(e).has_value(), "WeightQuant::None (float Linear projections) is refused");
    nn::FeedForward bn(8, 8, nn::ActivationType::SwiGLU, true, nn::NormType::BatchNorm, nn::WeightQuant::T1_58);
    CHECK(!bn.init(e).has_value(), "a BatchNorm SubLN is refused");
}

// ---------------------------------------------------------------- [14]
// The q / k / v projections of an attention input (three BitLinears on one tensor; GQA shapes:
// kv narrower than d, compute_layer_attention.hpp) share one activation quantization in an engine
// that reuses it; outputs equal what each projection gives on its own input copy.
void test_shared_input_quantization(nn::ComputeEngine& e)
{
    std::puts("[14] q/k/v BitLinears on one input: one activation quantization, same bits");
    constexpr std::size_t D = 64, KV = 16, B = 20;
    nn::BitLinear q(D, D), k(D, KV), v(D, KV);
    nn::PrecisionProfile prof;
    prof.param = nn::Precision::T1_58;
    bool ok = true;
    unsigned seed = 301;
    for (nn::BitLinear* l : {&q, &k, &v})
    {
        l->set_precision_profile(prof);
        ok = ok && l->init(e).has_value();
        auto ps = l->parameters();
        ok = ok && ps.size() == 2 && e.copy_from(ps[0].get(), random_matrix(l == &q ? D : KV, D, seed++)).has_value() &&
             e.copy_from(ps[1].get(), random_matrix(l == &q ? D : KV, 1, seed++)).has_value();
        l->set_activation_quant(true);
    }
    CHECK(ok, "q/k/v init");
    if (!ok) return;
    nn::Tensor x = upload(e, random_matrix(D, B, 310));
    const std::uint64_t n0 = e.activation_quantizations();
    auto yq = q.forward(x), yk = k.forward(x), yv = v.forward(x);
    CHECK(yq.has_value() && yk.has_value() && yv.has_value(), "q/k/v forward");
    if (!(yq && yk && yv)) return;
    const std::uint64_t n1 = e.activation_quantizations();
    CHECK(n1 - n0 == 1, "one activation quantization for the three projections");
    bool same = true;
    for (auto [l, y] : {std::pair{&q, &*yq}, std::pair{&k, &*yk}, std::pair{&v, &*yv}})
    {
        const nn::Tensor xc = upload(e, random_matrix(D, B, 310));  // same values, own storage
        auto yc = l->forward(xc);
        same = same && yc.has_value() && bitwise_equal(download(e, *y), download(e, *yc));
    }
    CHECK(same, "each projection == the same projection on its own copy of the input");
    CHECK(e.activation_quantizations() - n1 == 3, "copies in their own storage are quantized anew");
    // a write to the input invalidates the shared quantization
    CHECK(e.copy_from(x, random_matrix(D, B, 311)).has_value(), "overwrite the input");
    auto yq2 = q.forward(x);
    const nn::Tensor x2 = upload(e, random_matrix(D, B, 311));
    auto yq3 = q.forward(x2);
    CHECK(yq2.has_value() && yq3.has_value() && bitwise_equal(download(e, *yq2), download(e, *yq3)) &&
              !bitwise_equal(download(e, *yq2), download(e, *yq)),
          "after a write the input is quantized again");
}

// ---------------------------------------------------------------- [13]
std::string g_golden = "tests/golden";

std::string hex(const std::array<std::uint8_t, 32>& d)
{
    static const char* x = "0123456789abcdef";
    std::string s;
    for (std::uint8_t b : d)
    {
        s += x[b >> 4];
        s += x[b & 15];
    }
    return s;
}

std::string sha_of(const std::string& msg)
{
    nn::Sha256 h;
    h.update(msg.data(), msg.size());
    return hex(h.digest());
}

bool same_bytes(const void* a, const void* b, std::size_t n) { return n == 0 || std::memcmp(a, b, n) == 0; }

void test_model_files_host()
{
    std::puts("[13] model files: SHA-256 vectors and host-side parsing");
    CHECK(sha_of("abc") == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad", "sha256(\"abc\")");
    CHECK(sha_of("") == "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855", "sha256(\"\")");
    CHECK(sha_of("abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq") ==
              "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1",
          "sha256 two-block message");
    {
        nn::Sha256 h;  // the same message fed in odd-sized pieces
        const std::string m = "abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq";
        for (std::size_t i = 0; i < m.size(); i += 7) h.update(m.data() + i, std::min<std::size_t>(7, m.size() - i));
        CHECK(hex(h.digest()) == "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1", "sha256 incremental");
    }
    const nn::ParamKind kinds[5] = {nn::ParamKind::Dense, nn::ParamKind::TernaryPacked2, nn::ParamKind::Dense,
                                    nn::ParamKind::TernaryPacked2, nn::ParamKind::Dense};
    const std::size_t shapes[5][2] = {{48, 1}, {20, 48}, {20, 1}, {12, 20}, {12, 1}};
    for (const char* name : {"nnmodel_v8.nnmodel", "nnmodel_v7.nnmodel"})
    {
        auto f = nn::read_model_file(g_golden + "/" + name, 5);
        CHECK(f.has_value(), name);
        if (!f)
        {
            std::printf("    %s\n", f.error().message.c_str());
            continue;
        }
        bool ok = f->params.size() == 5 && f->role == nn::ModelRole::Model &&
                  f->version == (std::string(name).find("v8") != std::string::npos ? 8u : 7u) &&
                  f->spec == "spec-bytes: opaque to the loader" && f->tokenizer == "NNVC-tokenizer-bytes";
        for (std::size_t i = 0; ok && i < 5; ++i)
            ok = f->params[i].kind == kinds[i] && f->params[i].rows == shapes[i][0] && f->params[i].cols == shapes[i][1];
        ok = ok && f->params[1].payload.size() == 20 * 3 * 4 && f->params[1].aux.size() == 20 * 4 &&
             f->params[3].payload.size() == 12 * 2 * 4;
        CHECK(ok, "header, spec, entry kinds / shapes / sizes, tokenizer");
    }
    auto c = nn::read_model_file(g_golden + "/nnmodel_corrupt.nnmodel", 5);
    CHECK(!c.has_value() && c.error().message.find("checksum") != std::string::npos, "a flipped byte fails the sha256 check");
    auto w = nn::read_model_file(g_golden + "/nnmodel_v8.nnmodel", 4);
    CHECK(!w.has_value(), "an entry count that does not match the file is an error");
    auto t = nn::read_model_file(g_golden + "/nnmodel_trim_f16.nnmodel", 5);
    CHECK(t.has_value() && t->params[0].precision_tag == nn::kTagF16 && t->params[3].payload.size() == 12 * 5,
          "f16 Dense entry and byte-trimmed TernaryPacked2 rows parse");
    auto k = nn::read_model_file(g_golden + "/nnmodel_ckpt.nnmodel", 5);
    CHECK(k.has_value() && k->role == nn::ModelRole::Checkpoint && k->params[1].kind == nn::ParamKind::TernaryLatent,
          "checkpoint role with TernaryLatent entries parses");
    CHECK(!nn::read_model_file(g_golden + "/does_not_exist.nnmodel", 5).has_value(), "a missing file is an error");
}

// RMSNorm(48) -> BitLinear(48, 20) -> BitLinear(20, 12), the fixtures' layout
bool build_file_model(nn::ComputeEngine& e, nn::Model& m)
{
    nn::PrecisionProfile t158;
    t158.param = nn::Precision::T1_58;
    return m.add<nn::RMSNorm>(48, 1e-6f).has_value() &&
           m.add_layer(std::make_unique<nn::BitLinear>(48, 20), t158).has_value() &&
           m.add_layer(std::make_unique<nn::BitLinear>(20, 12), t158).has_value() && (void(e), true);
}

// host W1.58A8 forward of one BitLinear from decoded words / tau / bias (x: K x B)
nn::Matrix host_bitlinear(const nn::Matrix& x, const nn::Matrix& words, const nn::Matrix& tau, const nn::Matrix& b)
{
    const std::size_t K = x.rows(), B = x.cols(), N = words.rows(), wpr = words.cols();
    nn::Matrix y(N, B);
    for (std::size_t c = 0; c < B; ++c)
    {
        float mx = 0.0f;
        for (std::size_t k = 0; k < K; ++k) mx = std::max(mx, std::fabs(x.at(k, c)));
        const float s = mx * (1.0f / 127.0f);
        for (std::size_t n = 0; n < N; ++n)
        {
            std::vector<std::uint32_t> w(wpr);
            for (std::size_t i = 0; i < wpr; ++i) w[i] = word_of(words, n, i);
            std::int32_t acc = 0;
            for (std::size_t k = 0; k < K; ++k)
                acc += static_cast<std::int32_t>(nn::trit_pack::at(w.data(), k)) * nn::i8_pack::quantize(x.at(k, c), s);
            y.set_value(n, c, (tau.at(n, 0) * s) * static_cast<float>(acc) + b.at(n, 0));
        }
    }
    return y;
}

void test_model_files_device(nn::ComputeEngine& e)
{
    std::puts("[13] model files: load -> deploy state -> repack round trip -> forward; save -> load");
    auto file = nn::read_model_file(g_golden + "/nnmodel_v8.nnmodel", 5);
    if (!file) return;
    for (const char* name : {"nnmodel_v8.nnmodel", "nnmodel_v7.nnmodel", "nnmodel_trim_f16.nnmodel"})
    {
        nn::Model m(e);
        CHECK(build_file_model(e, m), "RMSNorm + 2 x BitLinear built");
        std::uint32_t ver = 0;
        auto tok = nn::load_model(g_golden + "/" + name, m, &ver);
        CHECK(tok.has_value() && *tok == "NNVC-tokenizer-bytes", name);
        if (!tok)
        {
            std::printf("    %s\n", tok.error().message.c_str());
            continue;
        }
        auto& l1 = static_cast<nn::BitLinear&>(m.layer_at(1));
        auto& l2 = static_cast<nn::BitLinear&>(m.layer_at(2));
        CHECK(l1.packed_only() && l2.packed_only(), "BitLinear layers are in the packed deploy state");
        const nn::Matrix w1 = download(e, l1.quantized_weights_packed()), t1 = download(e, l1.row_scales());
        const nn::Matrix w2 = download(e, l2.quantized_weights_packed());
        const bool trimmed = std::string(name).find("trim") != std::string::npos;
        bool words_ok = same_bytes(w1.data(), file->params[1].payload.data(), 20 * 3 * 4) &&
                        same_bytes(t1.data(), file->params[1].aux.data(), 20 * 4);
        for (std::size_t r = 0; r < 12 && words_ok; ++r)
        {
            // rows of 20 trits: 2 words; the file's bytes 0..4 (trimmed) or 0..7, the rest code 2
            const auto* fw = file->params[3].payload.data() + r * 8;
            std::uint8_t want[8];
            std::memcpy(want, fw, 8);
            if (trimmed) std::memset(want + 5, 0xAA, 3);
            words_ok = same_bytes(w2.data() + r * 2, want, 8);
        }
        CHECK(words_ok, "packed words and tau equal the file bytes (tail bytes of trimmed rows = code 2)");
        // repack -> unrepack on the GPU gives the container back bit for bit
        const nn::Tensor& wq = l1.quantized_weights_packed();
        auto rp = e.create_tensor(nnhip_repacked_bytes(20, 48) / 4, 1);
        auto back = e.create_tensor(20, 3);
        nnhip_ctx* ctx = nullptr;
        bool rt = nnhip_ctx_create(0, &ctx) == NNHIP_OK && rp.valid() && back.valid();
        if (rt)
        {
            rt = nnhip_repack_ternary(ctx, static_cast<const uint32_t*>(nn::TensorAccess::ptr(wq)), 20, 48,
                                      nn::TensorAccess::ptr(rp)) == NNHIP_OK &&
                 nnhip_unrepack_ternary(ctx, nn::TensorAccess::ptr(rp), 20, 48,
                                        static_cast<uint32_t*>(nn::TensorAccess::ptr(back))) == NNHIP_OK &&
                 nnhip_sync(ctx) == NNHIP_OK;
            (void)nnhip_ctx_destroy(ctx);
        }
        CHECK(rt && bitwise_equal(download(e, back), w1), "file words -> repack -> unrepack on the GPU == file words");
        // forward: RMSNorm (engine) then the two BitLinears against the host reference on the file's values
        l1.set_activation_quant(true);
        l2.set_activation_quant(true);
        const nn::Matrix x = random_matrix(48, 3, 131);
        auto y = m.forward(upload(e, x));
        auto n0 = e.rmsnorm(upload(e, x), static_cast<nn::RMSNorm&>(m.layer_at(0)).gamma(), 1e-6f);
        bool fwd = y.has_value() && n0.has_value();
        if (fwd)
        {
            const nn::Matrix h1 = host_bitlinear(download(e, *n0), w1, t1, download(e, l1.bias()));
            const nn::Matrix y2 = host_bitlinear(h1, w2, download(e, l2.row_scales()), download(e, l2.bias()));
            fwd = bitwise_equal(download(e, *y), y2);
        }
        CHECK(fwd, "forward of the loaded model == host W1.58A8 reference on the file's values");
        // save -> load round trip
        const std::string tmp = "/tmp/nnhip_roundtrip_" + std::to_string(ver) + (trimmed ? "t" : "") + ".nnmodel";
        auto sv = nn::save_model(tmp, m, nn::ModelRole::Model, "spec", "tok");
        nn::Model m2(e);
        bool rt2 = sv.has_value() && build_file_model(e, m2) && nn::load_model(tmp, m2).has_value();
        if (rt2)
        {
            auto& k1 = static_cast<nn::BitLinear&>(m2.layer_at(1));
            auto& k2 = static_cast<nn::BitLinear&>(m2.layer_at(2));
            k1.set_activation_quant(true);
            k2.set_activation_quant(true);
            auto y2 = m2.forward(upload(e, x));
            rt2 = bitwise_equal(download(e, k1.quantized_weights_packed()), w1) &&
                  bitwise_equal(download(e, k2.quantized_weights_packed()), w2) && y2.has_value() && y.has_value() &&
                  bitwise_equal(download(e, *y2), download(e, *y));
        }
        CHECK(rt2, "save_model -> load_model reproduces words, tau and outputs");
        std::remove(tmp.c_str());
    }
    {
        nn::Model m(e);
        (void)build_file_model(e, m);
        auto r = nn::load_model(g_golden + "/nnmodel_packed3.nnmodel", m);
        CHECK(!r.has_value() && r.error().message.find("TernaryPacked3") != std::string::npos,
              "base-3 entries are refused with a clear error");
    }
    {
        nn::Model m(e);
        (void)build_file_model(e, m);
        nn::ModelRole role = nn::ModelRole::Model;
        auto r = nn::load_model(g_golden + "/nnmodel_ckpt.nnmodel", m, nullptr, &role);
        auto ck = nn::read_model_file(g_golden + "/nnmodel_ckpt.nnmodel", 5);
        auto& l1 = static_cast<nn::BitLinear&>(m.layer_at(1));
        bool ok = r.has_value() && ck.has_value() && role == nn::ModelRole::Checkpoint && l1.latent_weights().valid() &&
                  !l1.packed_only();
        if (ok)
        {
            const nn::Matrix lat = download(e, l1.latent_weights());
            ok = lat.rows() == 20 && lat.cols() == 48 && same_bytes(lat.data(), ck->params[1].payload.data(), 20 * 48 * 4);
        }
        CHECK(ok, "checkpoint file: TernaryLatent entries land in the latent weights");
        // the layer quantizes them on first use; its packed words equal the oracle's fixture words
        l1.set_activation_quant(true);
        auto q = l1.ensure_quantized();
        CHECK(q.has_value() && same_bytes(download(e, l1.quantized_weights_packed()).data(), file->params[1].payload.data(),
                                          20 * 3 * 4),
              "latent -> absmean tau -> trit_pack reproduces the inference file's words");
    }
}

// Host double evaluation of one sequence's decode attention: q (H*dk) of the new token,
// caches (len rows of Hkv*dk, already holding the rotated new key), RoPE at position len-1.
std::vector<double> host_attention(const std::vector<float>& q, const std::vector<float>& kc, const std::vector<float>& vc,
                                   std::size_t len, std::size_t H, std::size_t Hkv, std::size_t dk, float scale,
                                   const nn::Matrix& cosT, const nn::Matrix& sinT)
{
    const std::size_t R = H / Hkv, half = dk / 2, p = len - 1;
    std::vector<double> out(H * dk, 0.0);
    for (std::size_t h = 0; h < H; ++h)
    {
        const std::size_t g = h / R;
        std::vector<double> qr(dk);
        for (std::size_t j = 0; j < half; ++j)
        {
            const double c = cosT.at(p, j), s = sinT.at(p, j), a = q[h * dk + j], b = q[h * dk + j + half];
            qr[j] = a * c - b * s;
            qr[j + half] = b * c + a * s;
        }
        std::vector<double> w(len);
        double m = -1e300;
        for (std::size_t t = 0; t < len; ++t)
        {
            double d = 0;
            for (std::size_t i = 0; i < dk; ++i) d += qr[i] * kc[t * Hkv * dk + g * dk + i];
            w[t] = d * scale;
            m = std::max(m, w[t]);
        }
        double l = 0;
        for (auto& x : w) l += (x = std::exp(x - m));
        for (std::size_t i = 0; i < dk; ++i)
        {
            double o = 0;
            for (std::size_t t = 0; t < len; ++t) o += w[t] / l * vc[t * Hkv * dk + g * dk + i];
            out[h * dk + i] = o;
        }
    }
    return out;
}

void test_decoder(nn::ComputeEngine& e)
{
    std::puts("[14] decoder step: RoPE, attention forward_step, GPTBlock, GPTModel greedy");
    const std::size_t d = 256, H = 4, Hkv = 2, dk = 64, F = 320, max_len = 100;
    // RoPE table
    {
        nn::RotaryTable rt;
        CHECK(rt.build(e, dk, max_len).has_value(), "RotaryTable built");
        std::vector<float> c(max_len * dk / 2), s(max_len * dk / 2);
        const bool ok = nnhip_rope_table(dk, max_len, c.data(), s.data()) == NNHIP_OK;
        CHECK(ok && same_bytes(download(e, rt.cos()).data(), c.data(), c.size() * 4) &&
                  same_bytes(download(e, rt.sin()).data(), s.data(), s.size() * 4),
              "RotaryTable == nnhip_rope_table bit for bit");
    }
    nn::CausalSelfAttention attn(d, H, max_len, Hkv, true, true);
    CHECK(attn.init(e).has_value(), "CausalSelfAttention(256, 4 heads, 2 KV heads, SubLN) initialized");
    attn.set_activation_quant(true);
    CHECK(!attn.forward(upload(e, random_matrix(d, 1, 1))).has_value(), "full-sequence forward is refused");
    // three sequences at positions 0, 5, 63 (all below 128: one work-group chunk each)
    const std::size_t B = 3;
    const std::int32_t posv[B] = {0, 5, 63};
    auto cache = attn.make_cache(B);
    CHECK(cache.has_value(), "KV cache for 3 sequences");
    if (!cache) return;
    // fill the earlier rows with arbitrary keys / values
    {
        nn::Matrix kc = random_matrix(B * max_len, Hkv * dk, 301), vc = random_matrix(B * max_len, Hkv * dk, 302);
        (void)e.copy_from(cache->k, kc);
        (void)e.copy_from(cache->v, vc);
    }
    const nn::Matrix kc0 = download(e, cache->k), vc0 = download(e, cache->v);
    const nn::Matrix x = random_matrix(d, B, 303);
    auto pos = nn::upload_indices(e, posv, B);
    auto xt = upload(e, x);
    auto y = attn.forward_step(e, xt, *cache, *pos, 64);
    CHECK(y.has_value() && y->rows() == d && y->cols() == B, "batched forward_step -> (d_model, B)");
    if (!y) return;
    // the attention output itself: rerun the pieces and compare with the host double evaluation
    {
        auto q = attn.w_q().forward(xt);
        auto k = attn.w_k().forward(xt);
        auto v = attn.w_v().forward(xt);
        nn::KVCache c2{e.create_tensor(B * max_len, Hkv * dk), e.create_tensor(B * max_len, Hkv * dk), B, max_len};
        (void)e.copy_from(c2.k, kc0);
        (void)e.copy_from(c2.v, vc0);
        auto a = e.attention_decode(*q, *k, *v, c2.k, c2.v, max_len, *pos, 64, &attn.rotary()->cos(),
                                    &attn.rotary()->sin(), H, Hkv, attn.scale());
        bool ok = a.has_value();
        double err = 0;
        bool rows_ok = ok;
        if (ok)
        {
            const nn::Matrix A = download(e, *a), Q = download(e, *q), K = download(e, *k), V = download(e, *v);
            const nn::Matrix KC = download(e, c2.k), VC = download(e, c2.v);
            const nn::Matrix cosT = download(e, attn.rotary()->cos()), sinT = download(e, attn.rotary()->sin());
            for (std::size_t b = 0; b < B; ++b)
            {
                const std::size_t p = posv[b];
                std::vector<float> qb(H * dk), kcb((p + 1) * Hkv * dk), vcb((p + 1) * Hkv * dk);
                for (std::size_t i = 0; i < H * dk; ++i) qb[i] = Q.at(i, b);
                for (std::size_t t = 0; t <= p; ++t)
                    for (std::size_t i = 0; i < Hkv * dk; ++i)
                    {
                        kcb[t * Hkv * dk + i] = KC.at(b * max_len + t, i);
                        vcb[t * Hkv * dk + i] = VC.at(b * max_len + t, i);
                    }
                // appended row: value exact, key = rotation of the new key (double, to 1e-6)
                for (std::size_t g = 0; g < Hkv; ++g)
                    for (std::size_t j = 0; j < dk / 2; ++j)
                    {
                        const double c = cosT.at(p, j), s = sinT.at(p, j);
                        const double k0 = K.at(g * dk + j, b), k1 = K.at(g * dk + j + dk / 2, b);
                        rows_ok = rows_ok && std::abs(KC.at(b * max_len + p, g * dk + j) - (k0 * c - k1 * s)) < 1e-6 &&
                                  std::abs(KC.at(b * max_len + p, g * dk + j + dk / 2) - (k1 * c + k0 * s)) < 1e-6;
                    }
                for (std::size_t i = 0; i < Hkv * dk; ++i)
                    rows_ok = rows_ok && VC.at(b * max_len + p, i) == V.at(i, b);
                const auto ref = host_attention(qb, kcb, vcb, p + 1, H, Hkv, dk, attn.scale(), cosT, sinT);
                for (std::size_t i = 0; i < H * dk; ++i) err = std::max(err, std::abs(A.at(i, b) - ref[i]));
            }
        }
        CHECK(rows_ok, "appended cache rows: rotated key (vs double) and the exact value");
        CHECK(ok && err < 1e-5, "attention_decode within 1e-5 of a host double evaluation");
    }
    // f16 caches (the reference's caches under compute = F16, compute_layer_gpt.hpp:764-765): the same
    // call on f16 caches holding kc0 / vc0 rounded to f16 appends the f16 rounding of the f32 call's
    // rows (the same f32 arithmetic, one rounding), leaves every other row alone, and returns the
    // host double evaluation over the f16 cache contents it ends with
    {
        auto q = attn.w_q().forward(xt);
        auto k = attn.w_k().forward(xt);
        auto v = attn.w_v().forward(xt);
        const auto F16 = nn::Precision::F16;
        nn::KVCache ch{e.create_tensor(B * max_len, Hkv * dk, F16), e.create_tensor(B * max_len, Hkv * dk, F16), B,
                       max_len};
        nn::KVCache cf{e.create_tensor(B * max_len, Hkv * dk), e.create_tensor(B * max_len, Hkv * dk), B, max_len};
        (void)e.copy_from(ch.k, kc0);
        (void)e.copy_from(ch.v, vc0);
        (void)e.copy_from(cf.k, kc0);
        (void)e.copy_from(cf.v, vc0);
        auto a16 = e.attention_decode(*q, *k, *v, ch.k, ch.v, max_len, *pos, 64, &attn.rotary()->cos(),
                                      &attn.rotary()->sin(), H, Hkv, attn.scale());
        auto a32 = e.attention_decode(*q, *k, *v, cf.k, cf.v, max_len, *pos, 64, &attn.rotary()->cos(),
                                      &attn.rotary()->sin(), H, Hkv, attn.scale());
        bool ok = a16.has_value() && a32.has_value();
        bool rows_ok = ok;
        double err = 0;
        if (ok)
        {
            const nn::Matrix A = download(e, *a16), Q = download(e, *q);
            const nn::Matrix KH = download(e, ch.k), VH = download(e, ch.v);  // f16 widened exactly
            auto kr = e.to_matrix(cf.k, F16), vr = e.to_matrix(cf.v, F16);  // the f32 caches rounded
            rows_ok = kr.has_value() && vr.has_value() && bitwise_equal(KH, *kr) && bitwise_equal(VH, *vr);
            const nn::Matrix cosT = download(e, attn.rotary()->cos()), sinT = download(e, attn.rotary()->sin());
            for (std::size_t b = 0; b < B; ++b)
            {
                const std::size_t p = posv[b];
                std::vector<float> qb(H * dk), kcb((p + 1) * Hkv * dk), vcb((p + 1) * Hkv * dk);
                for (std::size_t i = 0; i < H * dk; ++i) qb[i] = Q.at(i, b);
                for (std::size_t t = 0; t <= p; ++t)
                    for (std::size_t i = 0; i < Hkv * dk; ++i)
                    {
                        kcb[t * Hkv * dk + i] = KH.at(b * max_len + t, i);
                        vcb[t * Hkv * dk + i] = VH.at(b * max_len + t, i);
                    }
                const auto ref = host_attention(qb, kcb, vcb, p + 1, H, Hkv, dk, attn.scale(), cosT, sinT);
                for (std::size_t i = 0; i < H * dk; ++i) err = std::max(err, std::abs(A.at(i, b) - ref[i]));
            }
        }
        CHECK(rows_ok, "f16 caches: every row == the f32 call's cache rounded to f16 (appended rows included)");
        CHECK(ok && err < 1e-5, "f16 caches: attention_decode within 1e-5 of a host double evaluation of their contents");
        auto mixed = e.attention_decode(*q, *k, *v, ch.k, cf.v, max_len, *pos, 64, &attn.rotary()->cos(),
                                        &attn.rotary()->sin(), H, Hkv, attn.scale());
        auto q16 = e.to_matrix(*q, F16);
        nn::Tensor qh = e.create_tensor(q->rows(), q->cols(), F16);
        const bool qh_ok = q16.has_value() && e.copy_from(qh, *q16).has_value();
        auto half_q = e.attention_decode(qh, *k, *v, ch.k, ch.v, max_len, *pos, 64, &attn.rotary()->cos(),
                                         &attn.rotary()->sin(), H, Hkv, attn.scale());
        CHECK(!mixed.has_value() && qh_ok && !half_q.has_value(),
              "attention_decode refuses an f16 / f32 cache pair and f16 queries");
    }
    // batched == the reference single-sequence signature, per sequence (same kernels, same chunking)
    {
        bool same = true;
        const nn::Matrix Y = download(e, *y);
        for (std::size_t b = 0; b < B && same; ++b)
        {
            nn::Matrix kb(max_len, Hkv * dk), vb(max_len, Hkv * dk), xb(d, 1);
            std::memcpy(kb.data(), kc0.data() + b * max_len * Hkv * dk, kb.size() * 4);
            std::memcpy(vb.data(), vc0.data() + b * max_len * Hkv * dk, vb.size() * 4);
            for (std::size_t i = 0; i < d; ++i) xb.set_value(i, 0, x.at(i, b));
            nn::Tensor kt = upload(e, kb), vt = upload(e, vb);
            auto yb = attn.forward_step(e, upload(e, xb), kt, vt, posv[b]);
            same = yb.has_value();
            if (!same) break;
            const nn::Matrix Yb = download(e, *yb);
            for (std::size_t i = 0; i < d; ++i) same = same && Yb.at(i, 0) == Y.at(i, b);
        }
        CHECK(same, "forward_step(x (d, B), cache, positions) == forward_step(x_b, k_cache, v_cache, cur_len) per sequence");
    }
    // GPTBlock::forward_step == its composition of engine calls
    {
        nn::GPTBlock blk(d, H, F, max_len, Hkv, nn::ActivationType::SwiGLU, true, 1e-5f);
        CHECK(blk.init(e).has_value(), "GPTBlock initialized");
        blk.set_activation_quant(true);
        auto c1 = blk.attention().make_cache(B);
        auto c2 = blk.attention().make_cache(B);
        bool ok = c1.has_value() && c2.has_value();
        if (ok)
        {
            (void)e.copy_from(c1->k, kc0);
            (void)e.copy_from(c1->v, vc0);
            (void)e.copy_from(c2->k, kc0);
            (void)e.copy_from(c2->v, vc0);
            auto yb = blk.forward_step(e, xt, *c1, *pos, 64);
            auto n1 = blk.norm1().forward(xt);
            auto a = n1 ? blk.attention().forward_step(e, *n1, *c2, *pos, 64) : nn::Result<nn::Tensor>(nn::Error{"n1"});
            auto r2 = a ? e.add(xt, *a) : nn::Result<nn::Tensor>(nn::Error{"a"});
            auto n2 = r2 ? blk.norm2().forward(*r2) : nn::Result<nn::Tensor>(nn::Error{"r2"});
            auto f = n2 ? blk.feed_forward().forward(*n2) : nn::Result<nn::Tensor>(nn::Error{"n2"});
            auto out = f ? e.add(*r2, *f) : nn::Result<nn::Tensor>(nn::Error{"f"});
            ok = yb.has_value() && out.has_value() && bitwise_equal(download(e, *yb), download(e, *out)) &&
                 bitwise_equal(download(e, c1->k), download(e, c2->k));
        }
        CHECK(ok, "GPTBlock::forward_step == norm1 -> attention -> add -> norm2 -> FeedForward -> add, bit for bit");
    }
    // GPTModel: greedy generation == forward_step + the reference greedy loop on the host, under
    // the default f32 profile and under compute = F16 (the t1_58 preset)
    const std::size_t V = 97;
    const std::vector<std::vector<std::int32_t>> prompts = {{5, 9, 2}, {1}, {40, 41, 42, 43, 44}};
    auto greedy_checks = [&](nn::GPTModel& gm, const char* tag) {
        auto gen = gm.generate_greedy(e, prompts, 6);
        auto gen2 = gm.generate_greedy(e, prompts, 6);
        CHECK(gen.has_value() && gen2.has_value() && *gen == *gen2 && (*gen)[0].size() == 6 && (*gen)[1].size() == 6,
              (std::string(tag) + "generate_greedy: 6 tokens per sequence, deterministic").c_str());
        // manual lockstep loop with host-side greedy choice
        bool same = gen.has_value();
        auto caches = gm.make_caches(prompts.size());
        std::vector<std::vector<std::int32_t>> manual(prompts.size());
        std::vector<std::int32_t> cur(prompts.size()), pv(prompts.size());
        for (std::size_t s = 0; same && s < 5 + 6 - 1; ++s)
        {
            for (std::size_t b = 0; b < prompts.size(); ++b)
            {
                if (s < prompts[b].size()) cur[b] = prompts[b][s];
                pv[b] = static_cast<std::int32_t>(s);
            }
            auto ids = nn::upload_indices(e, cur.data(), cur.size());
            auto pt = nn::upload_indices(e, pv.data(), pv.size());
            auto lg = gm.forward_step(e, *ids, *pt, s + 1, *caches);
            same = lg.has_value();
            if (!same) break;
            const nn::Matrix L = download(e, *lg);
            for (std::size_t b = 0; b < prompts.size(); ++b)
            {
                std::size_t next = 0;
                float best = L.at(0, b);
                for (std::size_t v = 1; v < V; ++v)
                    if (L.at(v, b) > best)
                    {
                        best = L.at(v, b);
                        next = v;
                    }
                if (s + 1 < prompts[b].size()) continue;
                if (manual[b].size() < 6) manual[b].push_back(static_cast<std::int32_t>(next));
                cur[b] = static_cast<std::int32_t>(next);
            }
        }
        CHECK(same && manual == *gen,
              (std::string(tag) + "generate_greedy == forward_step + the reference greedy loop on downloaded logits").c_str());
    };
    nn::GPTModel gm(V, d, 32, H, F, 2, Hkv, nn::ActivationType::SwiGLU, true, 1e-5f);
    CHECK(gm.init(e).has_value(), "GPTModel (2 blocks, vocab 97) initialized");
    gm.set_activation_quant(true);
    greedy_checks(gm, "");
    auto too_long = gm.generate_greedy(e, prompts, 40);
    CHECK(!too_long.has_value(), "prompt + new tokens beyond max_len is refused");

    // compute = F16: the same weights (every layer initializes from fixed seeds), f16 activations
    // between the layers, f16 caches, f32 logits (the head computes in the stable precision)
    nn::GPTModel g16(V, d, 32, H, F, 2, Hkv, nn::ActivationType::SwiGLU, true, 1e-5f);
    g16.set_precision_profile(nn::profile_t1_58());
    CHECK(g16.init(e).has_value(), "GPTModel under compute = F16 (profile_t1_58) initialized");
    g16.set_activation_quant(true);
    {
        auto c16 = g16.make_caches(prompts.size());
        CHECK(c16.has_value() && (*c16)[0].k.precision() == nn::Precision::F16 &&
                  (*c16)[1].v.precision() == nn::Precision::F16,
              "compute = F16: the KV caches are f16 (compute_layer_gpt.hpp:764-765)");
    }
    greedy_checks(g16, "compute = F16: ");
    // one step of both models on the same tokens: f32 logits, within a few percent of the f32 model's
    {
        auto ca = gm.make_caches(3), cb = g16.make_caches(3);
        const std::int32_t idv[3] = {5, 1, 40}, pz[3] = {0, 0, 0};
        auto ids = nn::upload_indices(e, idv, 3);
        auto pt = nn::upload_indices(e, pz, 3);
        auto la = gm.forward_step(e, *ids, *pt, 1, *ca);
        auto lb = g16.forward_step(e, *ids, *pt, 1, *cb);
        bool ok = la.has_value() && lb.has_value() && lb->precision() == nn::Precision::F32;
        double mx = 0, dm = 0;
        if (ok)
        {
            const nn::Matrix A = download(e, *la), Bm = download(e, *lb);
            for (std::size_t i = 0; i < A.size(); ++i)
            {
                mx = std::max(mx, (double)std::abs(A.span()[i]));
                dm = std::max(dm, (double)std::abs(A.span()[i] - Bm.span()[i]));
            }
        }
        CHECK(ok && mx > 0 && dm <= 0.05 * mx && dm > 0,
              "compute = F16 logits within 5 % (of the largest) of the f32 model's, and not identical");
    }
    // GPTBlock::forward_step under compute = F16 == its composition with the f16 roundings
    {
        nn::GPTBlock blk(d, H, F, max_len, Hkv, nn::ActivationType::SwiGLU, true, 1e-5f);
        blk.set_precision_profile(nn::profile_t1_58());
        CHECK(blk.init(e).has_value(), "GPTBlock under compute = F16 initialized");
        blk.set_activation_quant(true);
        auto c1 = blk.attention().make_cache(B);
        auto c2 = blk.attention().make_cache(B);
        bool ok = c1.has_value() && c2.has_value();
        if (ok)
        {
            (void)e.copy_from(c1->k, kc0);
            (void)e.copy_from(c1->v, vc0);
            (void)e.copy_from(c2->k, kc0);
            (void)e.copy_from(c2->v, vc0);
            auto x16 = e.cast(xt, nn::Precision::F16);  // the residual stream between blocks is f16
            auto yb = x16 ? blk.forward_step(e, *x16, *c1, *pos, 64) : nn::Result<nn::Tensor>(nn::Error{"x16"});
            const auto F32 = nn::Precision::F32, F16 = nn::Precision::F16;
            auto xw = e.cast(*x16, F32);
            auto n1 = blk.norm1().forward(*xw);
            auto a = n1 ? blk.attention().forward_step(e, *n1, *c2, *pos, 64) : nn::Result<nn::Tensor>(nn::Error{"n1"});
            auto aw = a ? e.cast(*a, F32) : nn::Result<nn::Tensor>(nn::Error{"a"});
            auto s1 = aw ? e.add(*xw, *aw) : nn::Result<nn::Tensor>(nn::Error{"aw"});
            auto r2 = s1 ? e.cast(*s1, F16) : nn::Result<nn::Tensor>(nn::Error{"s1"});
            auto r2w = r2 ? e.cast(*r2, F32) : nn::Result<nn::Tensor>(nn::Error{"r2"});
            auto n2 = r2w ? blk.norm2().forward(*r2w) : nn::Result<nn::Tensor>(nn::Error{"r2w"});
            auto f = n2 ? blk.feed_forward().forward(*n2) : nn::Result<nn::Tensor>(nn::Error{"n2"});
            auto fw = f ? e.cast(*f, F32) : nn::Result<nn::Tensor>(nn::Error{"f"});
            auto s2 = fw ? e.add(*r2w, *fw) : nn::Result<nn::Tensor>(nn::Error{"fw"});
            auto out = s2 ? e.cast(*s2, F16) : nn::Result<nn::Tensor>(nn::Error{"s2"});
            ok = yb.has_value() && out.has_value() && yb->precision() == F16 && a.has_value() && a->precision() == F16 &&
                 f.has_value() && f->precision() == F16 && bitwise_equal(download(e, *yb), download(e, *out)) &&
                 bitwise_equal(download(e, c1->k), download(e, c2->k)) && c1->k.precision() == F16;
        }
        CHECK(ok, "compute = F16: GPTBlock::forward_step == norm1 -> attention (f16 out) -> f32 add rounded to f16 -> "
                  "norm2 -> FeedForward (f16 out) -> f32 add rounded to f16, bit for bit");
    }
}
// ---------------------------------------------------------------- [15]
// binary16 rounding on the host (round to nearest even), widened back: fl16(v)
float fl16(float v) { return static_cast<float>(static_cast<_Float16>(v)); }

// one BitLinear of the given profile with latent weights W, bias b and the branch chosen
std::unique_ptr<nn::BitLinear> make_bitlinear(nn::ComputeEngine& e, const nn::PrecisionProfile& prof,
                                              const nn::Matrix& W, const nn::Matrix& b, bool act_quant)
{
    auto bl = std::make_unique<nn::BitLinear>(W.cols(), W.rows());
    bl->set_precision_profile(prof);
    auto r = bl->init(e);
    EX_UNWRAP(r.has_value(), "BitLinear init failed");
    EX_UNWRAP(e.copy_from(bl->parameters()[0].get(), W).has_value(), "latent upload failed");
    EX_UNWRAP(e.copy_from(bl->parameters()[1].get(), b).has_value(), "bias upload failed");
    bl->set_activation_quant(act_quant);
    return bl;
}

void test_f16_compute(nn::ComputeEngine& e)
{
    std::puts("[15] compute = F16 (profile_t1_58, src/t1_58_test.cpp:668-690): f16 tensors at the host boundary; "
              "BitLinear's f16 output = the f32 path rounded as the reference's two f16 steps");
    // host boundary: one rounding to binary16 (nearest even, overflow to inf), exact widening back
    nn::Matrix m(3, 5);
    const float vals[15] = {1.0f, 0.1f, -0.3333333f, 65504.0f, 65520.0f, -7e5f, 1e-8f, 6.1e-5f,
                            3.0f + 0x1p-11f, 3.0f + 0x1p-10f, -0.0f, 2049.0f, 2051.0f, 1234.567f, -1e-3f};
    for (std::size_t i = 0; i < 15; ++i) m.span()[i] = vals[i];
    auto t16 = e.from_matrix(m, nn::Precision::F16);
    CHECK(t16.has_value() && t16->precision() == nn::Precision::F16, "from_matrix(F16) gives an f16 tensor");
    if (!t16) return;
    nn::Matrix back = download(e, *t16), want(3, 5);
    for (std::size_t i = 0; i < 15; ++i) want.span()[i] = fl16(vals[i]);
    CHECK(bitwise_equal(back, want), "to_matrix of an f16 tensor = the values rounded once to binary16, widened exactly");
    auto r16 = e.to_matrix(upload(e, m), nn::Precision::F16);
    CHECK(r16.has_value() && bitwise_equal(*r16, want), "to_matrix(f32 tensor, F16) rounds the values to binary16");

    const nn::PrecisionProfile t1 = nn::profile_t1_58();
    nn::PrecisionProfile f32p;
    f32p.param = nn::Precision::T1_58;
    constexpr std::size_t IN = 300, OUT = 70, B = 9;
    const nn::Matrix W = random_matrix(OUT, IN, 1501);
    const nn::Matrix X = random_matrix(IN, B, 1502);
    nn::Matrix zero(OUT, 1), bias = random_matrix(OUT, 1, 1503);
    for (std::size_t o = 0; o < OUT; ++o) zero.set_value(o, 0, 0.0f);
    for (const bool act : {true, false})
    {
        const char* br = act ? "int8 branch" : "float branch";
        // bias 0: the f16 output is the f32 output rounded once
        auto a32 = make_bitlinear(e, f32p, W, zero, act);
        auto a16 = make_bitlinear(e, t1, W, zero, act);
        auto y32 = a32->forward(upload(e, X));
        auto y16 = a16->forward(upload(e, X));
        CHECK(y32.has_value() && y16.has_value(), "f32 and f16 forwards succeed");
        if (!y32 || !y16) return;
        CHECK(y16->precision() == nn::Precision::F16 && y32->precision() == nn::Precision::F32,
              "the compute slot sets the output precision");
        const nn::Matrix Y32 = download(e, *y32), Y16 = download(e, *y16);
        nn::Matrix r(OUT, B);
        for (std::size_t i = 0; i < r.size(); ++i) r.span()[i] = fl16(Y32.span()[i]);
        std::printf("    %s, bias 0:\n", br);
        CHECK(bitwise_equal(Y16, r), "f16 output = fl16(f32 output) bit for bit");
        // nonzero bias: y = product rounded to f16, then fl16(y + b) (compute_layer_bitlinear.hpp:454-456, :464-466)
        auto b16 = make_bitlinear(e, t1, W, bias, act);
        auto yb = b16->forward(upload(e, X));
        CHECK(yb.has_value(), "f16 forward with a bias succeeds");
        if (!yb) return;
        const nn::Matrix YB = download(e, *yb);
        const nn::Matrix bh = download(e, b16->bias());
        nn::Matrix rb(OUT, B);
        for (std::size_t o = 0; o < OUT; ++o)
            for (std::size_t c = 0; c < B; ++c) rb.set_value(o, c, fl16(fl16(Y32.at(o, c)) + bh.at(o, 0)));
        std::printf("    %s, bias:\n", br);
        CHECK(bitwise_equal(YB, rb), "f16 output = fl16(fl16(product) + b) bit for bit");
        // f16 input (the reference uploads activations in the compute precision): widened exactly first
        auto x16 = e.from_matrix(X, nn::Precision::F16);
        nn::Matrix Xr(IN, B);
        for (std::size_t i = 0; i < Xr.size(); ++i) Xr.span()[i] = fl16(X.span()[i]);
        auto y_in16 = a16->forward(*x16);
        auto y_inr = a16->forward(upload(e, Xr));
        CHECK(y_in16.has_value() && y_inr.has_value() &&
                  bitwise_equal(download(e, *y_in16), download(e, *y_inr)),
              "an f16 input equals its widened f32 values");
    }
    CHECK(e.describe().device.find("gfx950") != std::string::npos, "EngineInfo.device is HIP's device name (gfx950)");
}
}  // namespace

int main(int argc, char** argv)
{
    std::setvbuf(stdout, nullptr, _IOLBF, 0);  // a crash still shows the last section reached
    if (argc > 1) g_golden = argv[1];
    test_layout();
    test_factory();
    test_model_files_host();
    // the reference call site (cli/cli_engine_factory.hpp:32-77): aggregate config, shared_ptr result
    const nn::cli::EngineConfig ec{true, "0"};
    nn::Result<std::shared_ptr<nn::ComputeEngine>> eng = nn::cli::create_engine(ec, std::cout);
    if (!eng.has_value())
    {
        std::printf("HIP engine unavailable, skipping device sections: %s\n", eng.error().message.c_str());
        return g_failures == 0 ? 77 : 1;
    }
    nn::ComputeEngine& e = **eng;
    std::printf("engine: %s\n", e.describe().text().c_str());
    test_trit_pack(e);
    test_quantize(e);
    test_unpack(e);
    test_matmul_q_i8_shape(e, 130, 17, 6, 31, "K/N not multiples, crosses row blocks");
    test_matmul_q_i8_shape(e, 512, 256, 8, 41, "2B4T order");
    test_matmul_q_i8_shape(e, 300, 2560, 1, 43, "decode M=1");
    test_matmul_q_i8_shape(e, 257, 700, 40, 44, "GEMM path, tails");
    test_bitlinear_rules(e);
    test_bitlinear_bound(e);
    test_quant_cache(e);
    test_deploy_and_model(e);
    test_float_products(e);
    test_feedforward(e);
    test_model_files_device(e);
    test_shared_input_quantization(e);
    test_decoder(e);
    test_f16_compute(e);
    if (g_failures == 0) std::puts("bitlinear_engine_test: all passed");
    else std::printf("bitlinear_engine_test: %d failure(s)\n", g_failures);
    return g_failures == 0 ? 0 : 1;
}
