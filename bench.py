"""bench.py — MI355X throughput of the BitLinear W1.58A8 hot path (libnn-hip.so).

Headline (BASELINE.json metric, config 1): the M=1 ternary x int8 decode GEMV over a
BitNet-2B-class layer stack — 30 layers x {q 2560->2560, k 2560->640, v 2560->640,
o 2560->2560, gate 2560->6912, up 2560->6912, down 6912->2560}, 521,011,200 bytes of packed
ternary weights (more than twice the 256 MB MALL) — run as ONE grouped launch per step.
value = algorithmic bytes of the whole sweep / average launch time, in GB/s.

Reported beside it: the same sweep at M=16, per-shape grouped sweeps, single-GEMV launches,
the prefill GEMM (config 2: M in {256, 1024, 2048, 4096}, K=4096, N in {4096, 11008}) in TOPS
against the dense int8 MFMA peak, and the fused activation quantizers at prefill sizes
(absmax -> int8 at K=4096, RMSNorm -> absmax -> int8 at the fused block's 2560 x 2048) in GB/s.
The CPU baseline is the oracle's CpuEngine restatement (row-block decode + dense f32
microkernel) on a bounded sample of the same workload, timed on this host.

roofline.traffic (HBM bytes per headline launch) is read from the committed PMC summary
profiles/k_gemv_grouped_m1_layerstack_pmc.md, which records the two rocprofv3 --pmc runs
(FETCH_SIZE, WRITE_SIZE) and the copy-kernel calibration (`bench.py --copy-probe`).

Inputs are synthetic (seeded): W ~ N(0, 0.02) ternarized by per-tensor absmean, activations
~ N(0, 1) quantized per token by absmax. All inputs are resident in HBM before timing.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA (5.0 POP/s)
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 MFMA
LAYERS = 30
D, FFN, KV = 2560, 6912, 640
SHAPES = [("q", D, D), ("k", D, KV), ("v", D, KV), ("o", D, D),
          ("gate", D, FFN), ("up", D, FFN), ("down", FFN, D)]   # (name, K, N)


def load_pkg():
    import importlib.util
    name = "nnhip_py"
    if name in sys.modules:
        return sys.modules[name]
    pkg = os.path.join(ROOT, "neuralnet.cpp_amd")
    spec = importlib.util.spec_from_file_location(name, os.path.join(pkg, "__init__.py"),
                                                  submodule_search_locations=[pkg])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gemv_bytes(N, K, M):
    """Algorithmic bytes of one GEMV: packed weights N*K/4, int8 activations K*M, s 4M,
    tau 4N, fp32 output 4NM."""
    return N * K // 4 + K * M + 4 * M + 4 * N + 4 * N * M


class Weights:
    """The layer stack's packed ternary weights, generated, packed and repacked on the GPU."""

    def __init__(self, ctx, torch, layers):
        self.mats = []   # (layer, name, K, N, rp, tau)
        gen = torch.Generator(device="cuda")
        for layer in range(layers):
            for idx, (name, K, N) in enumerate(SHAPES):
                gen.manual_seed(0xB17A0000 + layer * 16 + idx)
                W = torch.randn((N, K), generator=gen, device="cuda", dtype=torch.float32) * 0.02
                tau = W.abs().double().mean().float().expand(N).contiguous()   # per-tensor absmean
                wq = ctx.trit_pack(W, tau)
                rp = ctx.repack(wq, K)
                del W, wq
                self.mats.append((layer, name, K, N, rp, tau))
        torch.cuda.synchronize()


def make_acts(ctx, torch, K, M, seed, outliers=False):
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    X = torch.randn((K, M), generator=gen, device="cuda", dtype=torch.float32)
    if outliers:   # config 2: 0.1% of the elements at 20x scale
        idx = torch.randperm(K * M, generator=gen, device="cuda")[: max(1, K * M // 1000)]
        X.view(-1)[idx] *= 20.0
    xi, s, rs = ctx.act_quant_i8(X)
    return X, xi, s, rs


def build_group(ctx, torch, weights, acts, M, select=None):
    probs, nbytes = [], 0
    for (layer, name, K, N, rp, tau) in weights.mats:
        if select is not None and name not in select:
            continue
        _, xi, s, rs = acts[K]
        y = torch.empty((N, M), dtype=torch.float32, device="cuda")
        probs.append(dict(rp=rp, tau=tau, xi=xi, s=s, rowsum=rs, bias=None, y=y, N=N, K=K, M=M))
        nbytes += gemv_bytes(N, K, M)
    return ctx.group_create(probs), probs, nbytes


def time_launches(torch, stream, fn, steps, warmup):
    """Average duration of `fn` over `steps` back-to-back launches, from events recorded on
    the launch stream, plus the wall clock of the timed region (synchronized both sides)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(end) / steps / 1e3, wall


def achievable_read(nn, ctx, torch, stream, steps):
    """The achievable HBM read rate: nnhip_stream_xor (non-temporal 16-byte loads, one pass,
    then a one-block fold of the per-block partials) over 2 GiB, eight times the MALL, so the
    fold's launch is under 1 % of the time; timed like the headline. Plus the dense int8 MFMA
    peak re-derived from HIP's CU count and peak clock (8192 ops per CU per clock on gfx950)."""
    nbytes = 2 << 30
    buf = torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,), dtype=torch.int32, device="cuda")
    acc = torch.zeros(1, dtype=torch.int32, device="cuda")
    t, _ = time_launches(torch, stream, lambda: ctx.stream_xor(buf, acc), steps, 5)
    del buf
    info = nn.device_info(0)
    int8_tops = info["cus"] * info["clock_khz"] * 1e3 * 8192 / 1e12
    return {"stream_read_GB/s": round(nbytes / t / 1e9, 1), "stream_read_bytes": nbytes,
            "stream_read_us": round(t * 1e6, 2), "device": info, "int8_peak_TOPS_derived": round(int8_tops, 1)}


def extra_gemv_lines(ctx, torch, stream, weights, acts1, out):
    acts16 = {K: make_acts(ctx, torch, K, 16, 0xB17A0003 + K) for K in (D, FFN)}
    grp16, _, nbytes16 = build_group(ctx, torch, weights, acts16, 16)
    t16, _ = time_launches(torch, stream, lambda: ctx.group_run(grp16), 20, 3)
    out["gemv_m16_sweep"] = {"GB/s": round(nbytes16 / t16 / 1e9, 1),
                             "frac_hbm": round(nbytes16 / t16 / 1e9 / HBM_PEAK_GBS, 4),
                             "us_per_launch": round(t16 * 1e6, 2), "bytes": nbytes16}
    log(f"M=16 sweep: {nbytes16 / t16 / 1e9:.1f} GB/s")
    ctx.group_destroy(grp16)

    per_shape = {}
    for name, K, N in SHAPES:
        g, _, nb = build_group(ctx, torch, weights, acts1, 1, select={name})
        t, _ = time_launches(torch, stream, lambda: ctx.group_run(g), 20, 3)
        per_shape[f"{name} {K}->{N} x{len(weights.mats) // len(SHAPES)}"] = {
            "GB/s": round(nb / t / 1e9, 1), "us": round(t * 1e6, 2)}
        ctx.group_destroy(g)
    out["gemv_m1_per_shape_stacks"] = per_shape

    single = {}
    for (layer, name, K, N, rp, tau) in weights.mats[:len(SHAPES)]:
        _, xi, s, rs = acts1[K]
        y = torch.empty((N, 1), dtype=torch.float32, device="cuda")
        t, _ = time_launches(torch, stream,
                             lambda: ctx.ternary_matmul(rp, tau, xi, s, rs, N, K, 1, out=y), 50, 5)
        single[f"{name} {K}->{N}"] = {"us": round(t * 1e6, 2),
                                      "GB/s": round(gemv_bytes(N, K, 1) / t / 1e9, 1)}
    out["gemv_m1_single_launch"] = single


def gemm_lines(ctx, torch, stream, steps, out):
    """Config 2: the prefill GEMM at M in {256, 1024, 2048, 4096}, K=4096, N in {4096, 11008}
    (activations with 0.1% outliers at 20x before the per-token absmax)."""
    K = 4096
    acts = {M: make_acts(ctx, torch, K, M, 0xB17A0004 + M, outliers=True) for M in (256, 1024, 2048, 4096)}
    gemm = {}
    for N in (4096, 11008):
        gen = torch.Generator(device="cuda")
        gen.manual_seed(0xB17A0005 + N)
        W = torch.randn((N, K), generator=gen, device="cuda") * 0.02
        tau = W.abs().double().mean().float().expand(N).contiguous()
        rp = ctx.repack(ctx.trit_pack(W, tau), K)
        del W
        for M, (_, xi, s, rs) in acts.items():
            y = torch.empty((N, M), dtype=torch.float32, device="cuda")
            t, _ = time_launches(torch, stream,
                                 lambda: ctx.ternary_matmul(rp, tau, xi, s, rs, N, K, M, out=y),
                                 max(10, steps // 2), 5)
            tops = 2.0 * M * N * K / t / 1e12
            gemm[f"M={M} K={K} N={N}"] = {"TOPS": round(tops, 1), "us": round(t * 1e6, 1),
                                          "frac_int8_mfma": round(tops / INT8_PEAK_TOPS, 4)}
            if M == 2048:
                gemm[f"M={M} K={K} N={N}"]["hash"] = load_pkg().fnv1a64(y)
            log(f"GEMM M={M} K={K} N={N}: {t * 1e6:.1f} us, {tops:.1f} TOPS "
                f"({tops / INT8_PEAK_TOPS:.3f} of int8 MFMA peak)")
            del y
    # context: the vendor library's dense int8 GEMM on the same shapes (torch._int_mm, int32
    # out, no ternary unpacking, no epilogue); not part of this library
    lib_lines = {}
    for N in (4096, 11008):
        Bm = torch.randint(-127, 128, (K, N), dtype=torch.int8, device="cuda")
        for M in (2048, 4096):
            Am = torch.randint(-127, 128, (M, K), dtype=torch.int8, device="cuda")
            try:
                t, _ = time_launches(torch, stream, lambda: torch._int_mm(Am, Bm), max(10, steps // 2), 5)
            except RuntimeError as e:  # not every build ships an int8 GEMM
                lib_lines[f"M={M} K={K} N={N}"] = {"error": str(e)[:80]}
                continue
            tops = 2.0 * M * N * K / t / 1e12
            lib_lines[f"M={M} K={K} N={N}"] = {"TOPS": round(tops, 1), "us": round(t * 1e6, 1),
                                              "frac_int8_mfma": round(tops / INT8_PEAK_TOPS, 4)}
        del Bm
    gemm["torch._int_mm (dense int8, library)"] = lib_lines
    log(f"torch._int_mm: {lib_lines}")
    out["prefill_gemm"] = gemm


def act_quant_lines(ctx, torch, stream, steps, out):
    """The fused activation quantizers at prefill sizes, in GB/s of algorithmic bytes
    (4KM fp32 read + M*Kp int8 + 8M written)."""
    res = {}
    for K, M, norm in ((4096, 2048, False), (2560, 2048, True), (6912, 2048, False)):
        gen = torch.Generator(device="cuda")
        gen.manual_seed(0xB17A0006 + K)
        X = torch.randn((K, M), generator=gen, device="cuda")
        g = torch.ones(K, device="cuda")
        outs = ctx._act_out(K, M)
        if norm:
            fn = lambda: ctx.rmsnorm_quant_i8(X, g, 1e-6, outs=outs)
            name = f"rmsnorm_quant K={K} M={M}"
        else:
            fn = lambda: ctx.act_quant_i8(X, outs=outs)
            name = f"act_quant K={K} M={M}"
        t, _ = time_launches(torch, stream, fn, max(10, steps // 2), 5)
        nb = 4 * K * M + M * ((K + 255) // 256 * 256) + 8 * M
        res[name] = {"GB/s": round(nb / t / 1e9, 1), "frac_hbm": round(nb / t / 1e9 / HBM_PEAK_GBS, 4),
                     "us": round(t * 1e6, 2)}
        log(f"{name}: {t * 1e6:.2f} us, {nb / t / 1e9:.1f} GB/s")
    out["act_quant"] = res


def ffn_block_line(ctx, torch, stream, steps, out):
    """Config C4: RMSNorm(eps=1e-6, gamma=1) -> absmax int8 -> fc1 (d -> 2F, gate/up) ->
    SwiGLU -> absmax int8 -> fc2 (F -> d) on 2048 tokens, d=2560, F=6912, one
    nnhip_ffn_glu_i8 call per step; also each step timed alone. Ops = 2*M*(2F*d + d*F)."""
    d, F, M = D, FFN, 2048
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0xB17A0007)
    W1 = torch.randn((2 * F, d), generator=gen, device="cuda") * 0.02
    W2 = torch.randn((d, F), generator=gen, device="cuda") * 0.02
    t1, t2 = ctx.row_absmean(W1), ctx.row_absmean(W2)
    wq1, wq2 = ctx.trit_pack(W1, t1), ctx.trit_pack(W2, t2)
    del W1, W2
    wo, to, _ = ctx.glu_interleave(wq1, t1, None, F, d)
    rp1, rp2 = ctx.repack(wo, d), ctx.repack(wq2, F)
    X = torch.randn((d, M), generator=gen, device="cuda")
    g = torch.ones(d, device="cuda")
    Y = torch.empty((d, M), device="cuda")
    ops = 2.0 * M * (2 * F * d + d * F)
    n = max(10, steps // 2)
    t, _ = time_launches(torch, stream, lambda: ctx.ffn_glu_i8(X, g, 1e-6, F, rp1, to, None, rp2, t2, None, out=Y), n, 5)
    # the steps alone (same kernels the block runs)
    a1 = ctx._act_out(d, M)
    a2 = ctx._act_out(F, M)
    h = torch.empty((F, M), device="cuda")
    ctx.rmsnorm_quant_i8(X, g, 1e-6, outs=a1)
    ctx.ternary_matmul_glu(rp1, to, *a1, F, d, M, out=h)
    ctx.act_quant_i8(h, outs=a2)
    parts = {
        "rmsnorm_quant 2560x2048": (lambda: ctx.rmsnorm_quant_i8(X, g, 1e-6, outs=a1), None),
        "fc1+SwiGLU 13824x2560x2048": (lambda: ctx.ternary_matmul_glu(rp1, to, *a1, F, d, M, out=h),
                                       2.0 * M * 2 * F * d),
        "act_quant 6912x2048": (lambda: ctx.act_quant_i8(h, outs=a2), None),
        "fc2 2560x6912x2048": (lambda: ctx.ternary_matmul(rp2, t2, *a2, d, F, M, out=Y), 2.0 * M * d * F),
    }
    res_parts = {}
    for name, (fn, pops) in parts.items():
        tp, _ = time_launches(torch, stream, fn, n, 5)
        res_parts[name] = {"us": round(tp * 1e6, 2)}
        if pops:
            res_parts[name]["TOPS"] = round(pops / tp / 1e12, 1)
    out["ffn_block_c4"] = {"us": round(t * 1e6, 2), "TOPS": round(ops / t / 1e12, 1),
                           "frac_int8_mfma": round(ops / t / 1e12 / INT8_PEAK_TOPS, 4), "ops": ops,
                           "parts": res_parts}
    log(f"C4 block: {t * 1e6:.1f} us, {ops / t / 1e12:.1f} TOPS; parts {res_parts}")


def matmul_q_lines(ctx, torch, stream, steps, out):
    """Float-activation ternary products on the reference container (the reference's default
    BitLinear branch and its dX product), per BitNet-2B shape at M (tokens) in {1, 16} and on a
    64 MiB container (32768 x 8192) at M=1, f32 in and out. GB/s of algorithmic bytes: packed
    weights N*ceil(K/16)*4 + 4*K*M (B) + 4*N (tau) + 4*N*M (Y); matmul_q_t reads the same
    container for the transposed product. Times are per Python-issued call (events), so the
    decode shapes include the launch path; kernel-only times are in the rocprof summary.
    matmul_q_mfma: the same product on the repacked weights (nnhip_ternary_matmul_f, the HIP
    engine's f32 BitLinear branch): activations split into int8 digits, int8 MFMA, int64 combine;
    same algorithmic bytes. matmul_q_t_mfma: dX on the repack of the bit-transposed container
    (nnhip_ternary_matmul_t_f), same bytes as matmul_q_t."""
    res = {}
    n = max(10, steps // 2)
    for name, K, N in (("q 2560->2560", D, D), ("gate 2560->6912", D, FFN), ("down 6912->2560", FFN, D),
                       ("big 8192->32768", 8192, 32768)):
        gen = torch.Generator(device="cuda")
        gen.manual_seed(0xB17A0008 + K + N)
        W = torch.randn((N, K), generator=gen, device="cuda") * 0.02
        tau = ctx.row_absmean(W)
        wq = ctx.trit_pack(W, tau)
        del W
        wbytes = N * ((K + 15) // 16) * 4
        for M in ((1,) if K == 8192 else (1, 16)):
            B = torch.randn((K, M), generator=gen, device="cuda")
            Y = torch.empty((N, M), device="cuda")
            t, _ = time_launches(torch, stream, lambda: ctx.matmul_q(wq, tau, B, K, out=Y), n, 5)
            nb = wbytes + 4 * K * M + 4 * N + 4 * N * M
            res[f"matmul_q {name} M={M}"] = {"us": round(t * 1e6, 2), "GB/s": round(nb / t / 1e9, 1),
                                              "frac_hbm": round(nb / t / 1e9 / HBM_PEAK_GBS, 4)}
            # the same product on the repacked weights through the int8 MFMA path (digit split)
            rp = ctx.repack(wq, K)
            t, _ = time_launches(torch, stream, lambda: ctx.ternary_matmul_f(rp, tau, B, N, K, out=Y), n, 5)
            res[f"matmul_q_mfma {name} M={M}"] = {"us": round(t * 1e6, 2), "GB/s": round(nb / t / 1e9, 1),
                                                   "frac_hbm": round(nb / t / 1e9 / HBM_PEAK_GBS, 4)}
            del rp
            # dX: (tau o A)^T . dY with A = the same (N, ceil(K/16)) container read transposed
            dY = torch.randn((N, M), generator=gen, device="cuda")
            dX = torch.empty((K, M), device="cuda")
            t, _ = time_launches(torch, stream, lambda: ctx.matmul_q_t(wq, tau, dY, K, out=dX), n, 5)
            nb = wbytes + 4 * N * M + 4 * N + 4 * K * M
            res[f"matmul_q_t {name} M={M}"] = {"us": round(t * 1e6, 2), "GB/s": round(nb / t / 1e9, 1),
                                                "frac_hbm": round(nb / t / 1e9 / HBM_PEAK_GBS, 4)}
            # the same dX on the MFMA path: the transposed repack (made once per weight), tau folded
            # into the digit split
            rpT = ctx.repack(ctx.trit_transpose(wq, K), N)
            t, _ = time_launches(torch, stream, lambda: ctx.ternary_matmul_t_f(rpT, tau, dY, K, out=dX), n, 5)
            res[f"matmul_q_t_mfma {name} M={M}"] = {"us": round(t * 1e6, 2), "GB/s": round(nb / t / 1e9, 1),
                                                     "frac_hbm": round(nb / t / 1e9 / HBM_PEAK_GBS, 4)}
            del rpT
    out["matmul_q"] = res
    log(f"matmul_q: {res}")


def decode_c5_line(ctx, torch, stream, steps, out):
    """Config C5: a 30-layer BitNet-b1.58 GPT (d=2560, 20 heads / 5 KV heads of 128, SwiGLU FFN 6912
    with SubLN, vocab 10000, BitLinear LM head), random init, 16 sequences: prefill 2048 random prompt
    tokens per sequence, then 128 greedy decode steps. The prefill is one Decoder.prefill pass (the
    32768 prompt tokens through every block on the prefill GEMM, nnhip_kv_cache_fill and the causal
    nnhip_attention_prefill; the reference runs one forward_step per prompt token,
    compute_layer_gpt.hpp:774-794); it fills the KV caches and picks each sequence's first new token.
    The decode steps continue from those caches and tokens: the step is captured once in a graph and
    replayed 128 times. Reported separately: prefill time and tokens/s, decode ms per step and
    tokens/s, the end-to-end time, one layer's prefill attention against the fp32 MFMA peak, and one
    layer's decode attention call against HBM bandwidth. The same weights and prompt run twice:
    "decode_c5" with f32 KV caches and "decode_c5_f16_cache" with f16 ones (compute = F16: the
    reference creates its caches in the profile's compute precision, compute_layer_gpt.hpp:764-765,
    F16 under the t1_58 preset), the arithmetic f32 in both."""
    nn = load_pkg()
    from nnhip_py import decoder as dm
    L, d, H, Hkv, F, V, B, ctx_len, new = 30, D, 20, 5, FFN, 10000, 16, 2048, 128
    max_len = ctx_len + new
    dk = d // H
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0xB17AC500)

    def lin(N, K):
        W = torch.randn((N, K), generator=gen, device="cuda") * 0.02
        tau = ctx.row_absmean(W)
        wq = ctx.trit_pack(W, tau)
        del W
        return wq, tau

    ones_d, ones_f = torch.ones(d, device="cuda"), torch.ones(F, device="cuda")
    blocks, wbytes = [], 0
    for _ in range(L):
        mats = {}
        for name, N, K in (("q", d, d), ("k", Hkv * dk, d), ("v", Hkv * dk, d), ("o", d, d), ("fc2", d, F)):
            wq, tau = lin(N, K)
            mats[name] = dm.Linear(ctx.repack(wq, K), tau, None, N, K)
            wbytes += N * K // 4
        wq1, t1 = lin(2 * F, d)
        wo, to, _ = ctx.glu_interleave(wq1, t1, None, F, d)
        del wq1
        wbytes += 2 * F * d // 4
        fc1 = dm.Linear(ctx.repack(wo, d), to, None, nn.glu_rows(F), d)
        blocks.append(dm.Block(g1=ones_d, q=mats["q"], k=mats["k"], v=mats["v"], o=mats["o"], g2=ones_d, fc1=fc1,
                               fc2=mats["fc2"], g_attn_sub=ones_d, g_ffn_sub=ones_f))
    hq, ht = lin(V, d)
    head = dm.Linear(ctx.repack(hq, d), ht, None, V, d)
    wbytes += V * d // 4
    emb = torch.randn((V, d), generator=gen, device="cuda")
    prompt = torch.randint(0, V, (B * ctx_len,), generator=gen, device="cuda", dtype=torch.int32)
    for key, f16 in (("decode_c5", False), ("decode_c5_f16_cache", True)):
        cfg = dm.Config(d=d, H=H, Hkv=Hkv, F=F, vocab=V, max_len=max_len, act=0, eps=1e-5, cache_f16=f16)
        dec = dm.Decoder(ctx, cfg, blocks, emb, ones_d, head, B)
        res = _c5_measure(ctx, torch, stream, steps, nn, dm, dec, cfg, prompt, wbytes)
        out[key] = res
        log(f"C5 ({'f16' if f16 else 'f32'} KV caches): {res}")
        del dec
        torch.cuda.empty_cache()


def _c5_measure(ctx, torch, stream, steps, nn, dm, dec, cfg, prompt, wbytes):
    """Prefill, graph-replayed decode steps and lone attention calls of one C5 Decoder."""
    L, B, ctx_len, new = len(dec.blocks), dec.B, 2048, 128
    max_len, H, Hkv, dk = cfg.max_len, cfg.H, cfg.Hkv, cfg.dk
    # ---- prefill: 2048 prompt tokens per sequence in one pass (repeatable: it rewrites rows 0..2047)
    dec.prefill(prompt, ctx_len)                    # warm-up: the prefill scratch is allocated here
    torch.cuda.synchronize()
    n_pf = 3
    t_prefill, _ = time_launches(torch, stream, lambda: dec.prefill(prompt, ctx_len), n_pf, 0)
    first_ids = dec.ids.clone()
    prefill_hash = nn.fnv1a64(dec.logits)
    ids = first_ids.clone()
    pos = torch.full((B,), ctx_len, device="cuda", dtype=torch.int32)

    def one_step():
        # the greedy ids land in ids and every position advances, in the step's last launch
        dec.step(ids, pos, max_len, advance=True)

    one_step()                           # warm-up: context scratch grows outside the capture
    torch.cuda.synchronize()
    t_eager, _ = time_launches(torch, stream, one_step, 5, 1)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        one_step()
    # decode from the prefilled state: the first new token and position 2048
    ids.copy_(first_ids)
    pos.fill_(ctx_len)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(new):
        g.replay()
    end.record(stream)
    torch.cuda.synchronize()
    t_step = start.elapsed_time(end) / new / 1e3
    assert int(pos[0].item()) == ctx_len + new
    tokens_hash = nn.fnv1a64(ids)

    # one layer's prefill attention at the C5 geometry (causal, 16 x 2048 tokens, 20 heads)
    pf = dec._pf
    kc, vc = dec.caches[0]
    fn_pf = lambda: ctx.attention_prefill(pf["q"], kc, vc, B, ctx_len, H, Hkv, dk, 0, cfg.scale, dec.cos, dec.sin,
                                          out=pf["a"])
    t_pfa, _ = time_launches(torch, stream, fn_pf, 10, 2)
    pfa_flops = 4.0 * B * H * dk * (ctx_len * (ctx_len + 1) / 2)   # QK^T and PV over the causal triangle
    # one layer's decode attention alone at the mean context of the run
    mid = ctx_len + new // 2
    pos.fill_(mid)
    fn = lambda: ctx.attention_decode(dec.q, dec.k, dec.v, H, Hkv, dk, pos, max_len, kc, vc, cfg.scale, dec.cos,
                                      dec.sin, out=dec.a)
    t_att, _ = time_launches(torch, stream, fn, max(10, steps // 2), 3)
    att_bytes = dm.attention_bytes(B, [mid + 1] * B, Hkv, dk, H, 2 if cfg.cache_f16 else 4)
    kv_bytes = L * att_bytes
    res = {
        "prefill_ms": round(t_prefill * 1e3, 3), "prefill_tokens_per_s": round(B * ctx_len / t_prefill, 1),
        "prefill_attention_one_layer": {"us": round(t_pfa * 1e6, 1), "TFLOP/s": round(pfa_flops / t_pfa / 1e12, 1),
                                        "frac_fp32_mfma": round(pfa_flops / t_pfa / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4),
                                        "flops": pfa_flops},
        "tokens_per_s": round(B / t_step, 1), "ms_per_step": round(t_step * 1e3, 4),
        "eager_ms_per_step": round(t_eager * 1e3, 4),
        "end_to_end_s": round(t_prefill + new * t_step, 4),
        "batch": B, "context": ctx_len, "new_tokens": new,
        "layers": L, "packed_weight_bytes": wbytes, "kv_bytes_per_step_at_mean_context": kv_bytes,
        "step_GB/s_weights_plus_kv": round((wbytes + kv_bytes) / t_step / 1e9, 1),
        "attention_one_layer": {"us": round(t_att * 1e6, 2), "bytes": att_bytes,
                                "GB/s": round(att_bytes / t_att / 1e9, 1),
                                "frac_hbm": round(att_bytes / t_att / 1e9 / HBM_PEAK_GBS, 4)},
        "kv_cache": "f16" if cfg.cache_f16 else "f32",
        "hash": {"prefill_last_logits": prefill_hash, "last_ids": tokens_hash},
    }
    return res


def profiled_traffic():
    """Calibrated HBM bytes per headline launch from the committed PMC summary, or None when the
    summary is missing or was taken on other kernel sources: it records the sha256 of the grouped
    GEMV's source files, recomputed here (the .git history does not travel to the GPU box)."""
    import hashlib
    import re
    path = os.path.join(ROOT, "profiles", "k_gemv_grouped_m1_layerstack_pmc.md")
    try:
        with open(path) as f:
            text = f.read()
        h = hashlib.sha256()
        for src in ("k_gemv.hip", "gemv_tile.hpp"):
            with open(os.path.join(ROOT, "neuralnet.cpp_amd", "csrc", src), "rb") as f:
                h.update(f.read())
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", text)
    k = re.search(r"kernel_source_sha256:\s*([0-9a-f]+)", text)
    if not m or not k:
        return None
    if k.group(1) != h.hexdigest()[:len(k.group(1))]:
        print("bench.py: the PMC summary was taken on other k_gemv sources; roofline.traffic omitted "
              "(re-take profiles/k_gemv_grouped_m1_layerstack_pmc.md)", file=sys.stderr)
        return None
    return int(m.group(1))


def copy_probe(mib):
    """A plain device copy of known size (mib MiB read + mib MiB written), ten times: the PMC
    FETCH_SIZE / WRITE_SIZE calibration kernel."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.randn(n, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": n * 4}), flush=True)


def _host_l3_bytes():
    """Total L3 of the CPUs this process may run on (distinct L3 instances summed), or None."""
    seen, total = set(), 0
    try:
        for cpu in sorted(os.sched_getaffinity(0)):
            base = f"/sys/devices/system/cpu/cpu{cpu}/cache/index3"
            with open(base + "/shared_cpu_list") as f:
                key = f.read().strip()
            if key in seen:
                continue
            seen.add(key)
            with open(base + "/size") as f:
                v = f.read().strip()
            total += int(v[:-1]) * 1024 if v.endswith("K") else int(v)
    except (OSError, ValueError):
        return None
    return total or None


def cpu_baseline(ctx, torch, weights, acts1):
    """The oracle's CpuEngine restatement (row-block RB=64 decode + dense f32 microkernel,
    oracle/nn_oracle.c orc_matmul_q_i8_rowblock) built with the reference's Release flags
    (oracle/Makefile), timed on this host:
      * the headline workload, M=1 GEMVs over a DRAM-resident sample of the layer stack: enough
        layers for at least 4x the host's L3 (all 30 if that is not enough), every pass streaming
        the reference containers from memory, with all the cores this process may use and with one;
      * the M=2048 prefill GEMM (N=K=4096) on a 1024-row block of the weights;
      * config C4's gated FFN block on 64 of its 2048 tokens (every step is per token).
    Best-of-passes wall clock, as src/layer_bench.cpp:693-715 times the reference."""
    from oracle import nn_oracle as orc   # the CPU restatement, timed as the baseline
    L, level = orc.release_lib()
    affinity = len(os.sched_getaffinity(0))
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = min(affinity, omp) if omp > 0 else affinity
    l3 = _host_l3_bytes()
    layer_bytes = sum(gemv_bytes(N, K, 1) for _, K, N in SHAPES)
    n_layers = len(weights.mats) // len(SHAPES)
    want = n_layers if l3 is None else min(n_layers, max(1, -(-4 * l3 // layer_bytes)))
    # reference containers of the sample, from the GPU's repacked words
    sample = []
    for (layer, name, K, N, rp, tau) in weights.mats:
        if layer >= want:
            break
        wq = ctx.unrepack(rp, N, K).cpu().numpy().view(np.uint32)
        sample.append((wq, tau.cpu().numpy(), K, N))
    acts_host = {}
    for K in (D, FFN):
        X, _, s, _ = acts1[K]
        s_h = s.cpu().numpy()
        acts_host[K] = (orc.quantize_i8(X.cpu().numpy(), s_h, True), s_h)
    sample_bytes = sum(gemv_bytes(N, K, 1) for (_, _, K, N) in sample)

    def sweep(nthreads, budget_s):
        best, t_all, passes = None, 0.0, 0
        while passes < 1 or (t_all < budget_s and passes < 50):
            t0 = time.perf_counter()
            for wq, tau, K, N in sample:
                xq, s = acts_host[K]
                orc.matmul_q_i8_rowblock(wq, tau, xq, s, K, 1, nthreads, L=L)
            dt = time.perf_counter() - t0
            t_all += dt
            passes += 1
            best = dt if best is None else min(best, dt)
        return sample_bytes / best / 1e9, passes, t_all

    v_all, p_all, t_all = sweep(threads, 8.0)
    v_one, p_one, t_one = sweep(1, 6.0)
    # prefill GEMM, N=K=4096, M=2048, one 256-row block
    rng = np.random.default_rng(0xB17A)
    Kg, Mg, rows = 4096, 2048, 1024
    wq = rng.integers(0, 2 ** 32, (rows, Kg // 16), dtype=np.uint32)   # the timing does not depend on the codes
    xq = rng.integers(0, 2 ** 32, (Kg, Mg // 4), dtype=np.uint32)
    tg = np.ones(rows, np.float32)
    sg = np.ones(Mg, np.float32)
    best = None
    t_g = 0.0
    while best is None or t_g < 3.0:
        t0 = time.perf_counter()
        orc.matmul_q_i8_rowblock(wq, tg, xq, sg, Kg, Mg, threads, L=L)
        dt = time.perf_counter() - t0
        t_g += dt
        best = dt if best is None else min(best, dt)
    gemm_tops = 2.0 * rows * Kg * Mg / best / 1e12
    # C4 block on 64 tokens
    d, F, Mt = D, FFN, 64
    X = rng.standard_normal((d, Mt), dtype=np.float32)
    g = np.ones(d, np.float32)
    W1 = (rng.standard_normal((2 * F, d), dtype=np.float32) * np.float32(0.02))
    W2 = (rng.standard_normal((d, F), dtype=np.float32) * np.float32(0.02))
    t1, t2 = orc.row_absmean(W1), orc.row_absmean(W2)
    wq1, wq2 = orc.trit_pack(W1, t1), orc.trit_pack(W2, t2)
    del W1, W2
    best = None
    t_c = 0.0
    while best is None or t_c < 3.0:
        t0 = time.perf_counter()
        orc.ffn_glu_i8(X, g, 1e-6, F, wq1, t1, None, wq2, t2, None, 0, threads, L=L)
        dt = time.perf_counter() - t0
        t_c += dt
        best = dt if best is None else min(best, dt)
    c4_ops = 2.0 * Mt * (2 * F * d + d * F)
    return {"value": round(v_all, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{len(sample)} GEMVs = layers 0-{want - 1} of the stack ({sample_bytes} B of reference "
                      f"containers per pass; host L3 {l3} B) at M=1, best of {p_all} passes ({t_all:.1f} s); "
                      f"oracle/nn_oracle.c orc_matmul_q_i8_rowblock built with the reference Release flags "
                      f"(x86-64-{level}), {threads} OpenMP threads of {affinity} CPUs in the affinity mask",
            "one_core": {"value": round(v_one, 3), "unit": "GB/s", "cores": 1,
                         "sample": f"the same sample, best of {p_one} passes ({t_one:.1f} s)"},
            "gemm_m2048": {"TOPS": round(gemm_tops, 4), "cores": threads,
                           "sample": f"N=K=4096, M=2048 on a {rows}-row block: {2 * rows * Kg * Mg} ops per call"},
            "ffn_block_c4": {"TOPS": round(c4_ops / best / 1e12, 4), "us_per_token": round(best / Mt * 1e6, 1),
                             "cores": threads,
                             "sample": f"RMSNorm -> int8 -> fc1 + SwiGLU -> int8 -> fc2 (d=2560, F=6912) on "
                                       f"{Mt} tokens ({c4_ops:.3g} ops per call)"}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prefill GEMM lines")
    ap.add_argument("--no-decode", action="store_true", help="skip the config C5 decode line")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the M=16 / per-shape / single-launch GEMV and the quantizer lines")
    ap.add_argument("--lines", default="all",
                    help="comma-separated lines besides the headline: gemv_extra, act_quant, matmul_q, gemm, "
                         "ffn, c5 (default all; the --no-* flags remove lines from it)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB ten times (PMC calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.copy_probe:
        copy_probe(args.copy_probe)
        return

    import torch
    nn = load_pkg()
    ctx = nn.Context(0)
    stream = torch.cuda.Stream()      # default priority
    torch.cuda.set_stream(stream)

    log(f"generating {args.layers} layers of packed ternary weights on the GPU")
    weights = Weights(ctx, torch, args.layers)
    acts1 = {K: make_acts(ctx, torch, K, 1, 0xB17A0002 + K) for K in (D, FFN)}

    # ---- headline: M=1 layer-stack sweep, one grouped launch per step
    grp, probs, nbytes = build_group(ctx, torch, weights, acts1, 1)
    wbytes = sum(N * K // 4 for (_, _, K, N, _, _) in weights.mats)
    log(f"M=1 sweep: {len(probs)} GEMVs, {wbytes} B packed weights, {nbytes} B algorithmic")
    t_launch, wall = time_launches(torch, stream, lambda: ctx.group_run(grp), args.steps, args.warmup)
    gbs = nbytes / t_launch / 1e9
    ms_per_step = wall / args.steps * 1e3
    log(f"M=1 sweep: {t_launch * 1e6:.1f} us/launch (events), {ms_per_step * 1e3:.1f} us/step wall, "
        f"{gbs:.1f} GB/s = {gbs / HBM_PEAK_GBS:.3f} of HBM peak")

    # bit hash of the sweep's outputs (the 210 Y, concatenated in problem order), as layer_bench --hash
    out_hash = nn.fnv1a64(torch.cat([p["y"].reshape(-1) for p in probs]))
    # the sweep's last output must equal the single-problem launch bit for bit
    p0 = probs[-1]
    y_single = ctx.ternary_matmul(p0["rp"], p0["tau"], p0["xi"], p0["s"], p0["rowsum"],
                                  p0["N"], p0["K"], 1)
    torch.cuda.synchronize()
    assert torch.equal(y_single, p0["y"]), "grouped GEMV differs from the single launch"

    lines = {"gemv_extra", "act_quant", "matmul_q", "gemm", "ffn", "c5"} if args.lines == "all" else \
        set(args.lines.split(","))
    if args.no_extra:
        lines -= {"gemv_extra", "act_quant", "matmul_q"}
    if args.no_gemm:
        lines -= {"gemm", "ffn"}
    if args.no_decode:
        lines -= {"c5"}
    extra = {}
    if "gemv_extra" in lines:
        extra_gemv_lines(ctx, torch, stream, weights, acts1, extra)
    if "act_quant" in lines:
        act_quant_lines(ctx, torch, stream, args.steps, extra)
    if "matmul_q" in lines:
        matmul_q_lines(ctx, torch, stream, args.steps, extra)
    if "gemm" in lines:
        gemm_lines(ctx, torch, stream, args.steps, extra)
    if "ffn" in lines:
        ffn_block_line(ctx, torch, stream, args.steps, extra)
    if "c5" in lines:
        decode_c5_line(ctx, torch, stream, args.steps, extra)
    ach = achievable_read(nn, ctx, torch, stream, args.steps)
    log(f"achievable read: {ach}")
    cpu = None
    if not args.no_cpu:
        log("timing the CPU baseline (about 25 s)")
        cpu = cpu_baseline(ctx, torch, weights, acts1)
        log(f"CPU baseline: {cpu}")

    n_items = sum((p["N"] + 15) // 16 for p in probs)
    line = {
        "metric": "M=1 ternary GEMV GB/s (% HBM peak); M=2048 GEMM int8 TOPS (% MFMA peak)",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) weights, absmean ternary; N(0,1) activations, absmax int8)",
        "config": {"workload": "M=1 ternary x int8 GEMV layer-stack sweep, one grouped launch: "
                               f"{args.layers} layers x q/k/v/o/gate/up/down of d=2560, ffn=6912, kv=640",
                   "M": 1, "layers": args.layers, "gemvs": len(probs), "row_tiles": n_items,
                   "packed_weight_bytes": wbytes, "algorithmic_bytes": nbytes,
                   "grid_waves": ctx.gemv_grid_waves(n_items), "variant": ctx.group_info(grp),
                   "output_hash": out_hash},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(),
                     "kernel": "k_gemv_grouped", "avg_launch_us": round(t_launch * 1e6, 2),
                     "achievable": ach, "frac_of_achievable": round(gbs / ach["stream_read_GB/s"], 4)},
        "cpu_baseline": cpu,
    }
    line.update(extra)
    ctx.group_destroy(grp)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
