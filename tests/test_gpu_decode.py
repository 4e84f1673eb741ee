"""GPU parity of the batched decode step (config C5): decode attention over per-sequence KV
caches (grouped-query heads, RoPE, cache append), residual add, embedding gather and greedy
argmax, against the CPU oracle.

The cache rows the kernel appends (rotated keys, values), the adds, the gathers and the greedy
ids are compared bit for bit. The attention output is compared within 5e-6 x max(1, max|out|)
of the oracle and of a float64 evaluation: its dot products and softmax sums are f32 in an
order the reference leaves open (AttentionBase::forward_step runs them as engine matmuls,
include/neuralnet.cpp/compute_layer_attention.hpp:1059-1083).
"""
import math

import numpy as np
import pytest

from conftest import normal, uniform
from test_oracle_decode import _attn64

pytestmark = pytest.mark.gpu

ATOL = 5e-6   # x max(1, max|out|)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


def say(msg):
    print(msg, flush=True)


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return a.shape == b.shape and np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def run_case(ctx, orc, nnhip, B, H, Hkv, dk, max_len, pos, len_bound, rope, seed, check64=True):
    say(f"attention B={B} H={H} Hkv={Hkv} dk={dk} max_len={max_len} pos={list(pos)[:8]} len_bound={len_bound} "
        f"rope={rope}")
    q = normal((H * dk, B), seed)
    k = normal((Hkv * dk, B), seed + 1)
    v = normal((Hkv * dk, B), seed + 2)
    kc = normal((B, max_len, Hkv * dk), seed + 3)
    vc = normal((B, max_len, Hkv * dk), seed + 4)
    cos, sin = nnhip.rope_table(dk, max_len) if rope else (None, None)
    scale = float(np.float32(1.0) / np.float32(math.sqrt(dk)))
    kc_d, vc_d = dev(kc), dev(vc)
    out_d = ctx.attention_decode(dev(q), dev(k), dev(v), H, Hkv, dk, dev(np.array(pos, np.int32)), len_bound,
                                 kc_d, vc_d, scale, None if cos is None else dev(cos), None if sin is None else dev(sin))
    out = host(out_d)
    kc_o, vc_o = kc.copy(), vc.copy()
    ref = orc.attention_decode(q, k, v, H, Hkv, dk, pos, kc_o, vc_o, scale, cos, sin)
    assert same_bits(host(kc_d), kc_o), "key cache differs"
    assert same_bits(host(vc_d), vc_o), "value cache differs"
    tol = ATOL * max(1.0, float(np.max(np.abs(ref))))
    assert np.max(np.abs(out - ref)) <= tol
    if check64:
        ref64 = _attn64(q, kc_o, vc_o, H, Hkv, dk, pos, cos, sin, scale)
        assert np.max(np.abs(out - ref64)) <= tol
    return out


@pytest.mark.parametrize("B,H,Hkv,dk,pos,rope", [
    (1, 4, 4, 64, [0], True),            # single position: out = v
    (2, 8, 2, 128, [5, 130], True),      # second chunk
    (3, 20, 5, 128, [127, 128, 300], True),  # chunk boundaries 128 / 129 positions
    (2, 4, 1, 256, [40, 3], False),      # dk 256, no rotation
    (2, 16, 2, 128, [200, 17], True),    # 8 query heads per KV head
    (4, 4, 2, 64, [63, 64, 255, 256], True),
])
def test_attention_decode_parity(ctx, orc, nnhip, B, H, Hkv, dk, pos, rope):
    max_len = 320
    run_case(ctx, orc, nnhip, B, H, Hkv, dk, max_len, pos, max(pos) + 1, rope, 0xD0 + B * 7 + dk)
    # the same with the launch sized for the whole cache
    run_case(ctx, orc, nnhip, B, H, Hkv, dk, max_len, pos, max_len, rope, 0xD1 + B * 7 + dk)


def test_attention_decode_ragged_batch16(ctx, orc, nnhip):
    """Config C5's heads (20 query / 5 KV, dk = 128) at batch 16 with ragged positions."""
    pos = [0, 1, 2, 127, 128, 129, 255, 256, 511, 700, 1000, 1023, 1024, 1500, 2047, 2100]
    run_case(ctx, orc, nnhip, 16, 20, 5, 128, 2176, pos, 2176, True, 0xC5, check64=False)


def test_attention_decode_incremental(ctx, orc, nnhip):
    """Several steps in a row from empty caches (zeros), each sequence starting at its own
    position: every step's output and both caches stay with the oracle."""
    import torch
    B, H, Hkv, dk, max_len = 3, 8, 2, 64, 300
    cos, sin = nnhip.rope_table(dk, max_len)
    cos_d, sin_d = dev(cos), dev(sin)
    kc = np.zeros((B, max_len, Hkv * dk), np.float32)
    vc = np.zeros_like(kc)
    kc_d, vc_d = dev(kc), dev(vc)
    start = np.array([0, 120, 250], np.int32)
    for step in range(10):
        say(f"incremental step {step}")
        pos = start + step
        q = normal((H * dk, B), 100 + step)
        k = normal((Hkv * dk, B), 200 + step)
        v = normal((Hkv * dk, B), 300 + step)
        out = host(ctx.attention_decode(dev(q), dev(k), dev(v), H, Hkv, dk, dev(pos), int(pos.max()) + 1,
                                        kc_d, vc_d, 0.125, cos_d, sin_d))
        ref = orc.attention_decode(q, k, v, H, Hkv, dk, pos, kc, vc, 0.125, cos, sin)
        assert np.max(np.abs(out - ref)) <= ATOL * max(1.0, float(np.max(np.abs(ref))))
    torch.cuda.synchronize()
    assert same_bits(host(kc_d), kc) and same_bits(host(vc_d), vc)


def test_attention_decode_bad_position(ctx, nnhip):
    """A position outside [0, len_bound) gives NaN outputs for that sequence and leaves its
    cache alone; the other sequences are unaffected."""
    B, H, Hkv, dk, max_len = 3, 4, 2, 64, 200
    q = normal((H * dk, B), 1)
    k = normal((Hkv * dk, B), 2)
    v = normal((Hkv * dk, B), 3)
    kc = normal((B, max_len, Hkv * dk), 4)
    vc = normal((B, max_len, Hkv * dk), 5)
    for len_bound in (150, 10):     # two chunks / one chunk
        pos = np.array([-1, 5, len_bound], np.int32)
        kc_d, vc_d = dev(kc), dev(vc)
        say(f"bad position len_bound={len_bound}")
        out = host(ctx.attention_decode(dev(q), dev(k), dev(v), H, Hkv, dk, dev(pos), len_bound, kc_d, vc_d, 0.125))
        assert np.all(np.isnan(out[:, 0])) and np.all(np.isnan(out[:, 2]))
        assert np.all(np.isfinite(out[:, 1]))
        kg, vg = host(kc_d), host(vc_d)
        assert same_bits(kg[0], kc[0]) and same_bits(kg[2], kc[2]) and same_bits(vg[2], vc[2])
        assert not same_bits(kg[1], kc[1])
    with pytest.raises(nnhip.NNHipError):    # len_bound above max_len is refused on the host
        ctx.attention_decode(dev(q), dev(k), dev(v), H, Hkv, dk, dev(np.zeros(B, np.int32)), max_len + 1,
                             dev(kc), dev(vc), 0.125)


@pytest.mark.parametrize("B,H,Hkv,dk,pos,len_bound,rope", [
    (3, 20, 5, 128, [127, 300, 2], 301, True),    # chunks and the merge
    (2, 8, 2, 64, [5, 90], 100, True),            # one chunk: the chunk kernel writes the output
    (4, 4, 1, 256, [40, -1, 3, 41], 42, False),   # dk 256, a bad position (NaN outputs)
    (16, 20, 5, 128, [2000 + 7 * b for b in range(16)], 2106, True),
])
def test_attention_decode_tokens(ctx, nnhip, B, H, Hkv, dk, pos, len_bound, rope):
    """nnhip_attention_decode_tokens on q, k, v as token-major rows: out (B, H*dk) is
    nnhip_attention_decode's out (H*dk, B) on the columns, transposed, bit for bit (NaN where the
    position is out of range), and both append the same rows to the caches."""
    say(f"attention tokens B={B} H={H} Hkv={Hkv} dk={dk} pos={pos[:4]} len_bound={len_bound}")
    max_len = len_bound + 8
    q = normal((H * dk, B), 91 + B)
    k = normal((Hkv * dk, B), 92 + B)
    v = normal((Hkv * dk, B), 93 + B)
    kc = normal((B, max_len, Hkv * dk), 94 + B)
    vc = normal((B, max_len, Hkv * dk), 95 + B)
    cos, sin = nnhip.rope_table(dk, max_len) if rope else (None, None)
    tabs = (dev(cos), dev(sin)) if rope else (None, None)
    p = dev(np.array(pos, np.int32))
    kc1, vc1, kc2, vc2 = dev(kc), dev(vc), dev(kc), dev(vc)
    ref = host(ctx.attention_decode(dev(q), dev(k), dev(v), H, Hkv, dk, p, len_bound, kc1, vc1, 0.1, *tabs))
    tr = lambda a: dev(np.ascontiguousarray(a.T))
    got = host(ctx.attention_decode(tr(q), tr(k), tr(v), H, Hkv, dk, p, len_bound, kc2, vc2, 0.1, *tabs,
                                    tokens=True))
    assert got.shape == (B, H * dk)
    assert same_bits(np.ascontiguousarray(got.T), ref)
    assert same_bits(host(kc2), host(kc1)) and same_bits(host(vc2), host(vc1))


def test_attention_decode_c5_full_context(ctx, orc, nnhip):
    """Config C5's decode step at full context: 16 sequences at position 2048 of a 2176-row
    cache, sampled sequences checked against the oracle."""
    B, H, Hkv, dk, max_len = 16, 20, 5, 128, 2176
    say("attention C5 full context")
    q = normal((H * dk, B), 11)
    k = normal((Hkv * dk, B), 12)
    v = normal((Hkv * dk, B), 13)
    kc = normal((B, max_len, Hkv * dk), 14)
    vc = normal((B, max_len, Hkv * dk), 15)
    cos, sin = nnhip.rope_table(dk, max_len)
    pos = np.full(B, 2048, np.int32)
    kc_d, vc_d = dev(kc), dev(vc)
    out = host(ctx.attention_decode(dev(q), dev(k), dev(v), H, Hkv, dk, dev(pos), 2049, kc_d, vc_d,
                                    float(np.float32(1) / np.float32(math.sqrt(dk))), dev(cos), dev(sin)))
    for b in (0, 7, 15):
        kcb, vcb = kc[b:b + 1].copy(), vc[b:b + 1].copy()
        ref = orc.attention_decode(q[:, b:b + 1], k[:, b:b + 1], v[:, b:b + 1], H, Hkv, dk, pos[b:b + 1], kcb, vcb,
                                   float(np.float32(1) / np.float32(math.sqrt(dk))), cos, sin)
        assert np.max(np.abs(out[:, b:b + 1] - ref)) <= ATOL * max(1.0, float(np.max(np.abs(ref))))
        assert same_bits(host(kc_d[b]), kcb[0])


def test_add_gather_argmax_bitexact(ctx, orc):
    say("add / gather / argmax")
    x = normal((2560, 16), 21)
    y = normal((2560, 16), 22)
    assert same_bits(host(ctx.add(dev(x), dev(y))), x + y)
    table = normal((1000, 2560), 23)
    ids = np.array([0, 999, 5, 5, 17, -3, 1000, 42], np.int32)
    assert same_bits(host(ctx.embedding_gather(dev(table), dev(ids))), orc.embedding_gather(table, ids))
    L = uniform((10000, 16), 24)
    L[:, 3] = 0.5          # all ties
    L[0, 4] = np.nan       # NaN at index 0
    L[7, 5] = np.nan
    L[11, 6] = np.inf
    L[12, 6] = np.inf
    L[:, 7] = np.nan
    L[9999, 8] = 2.0
    assert host(ctx.argmax_cols(dev(L))).tolist() == orc.argmax_cols(L).tolist()
    # a vocabulary past one load batch per thread (16 x 1024): ties across batches, all -inf
    L = uniform((40000, 4), 25)
    L[5, 0] = L[20000, 0] = 3.0        # equal maxima in different batches: the first wins
    L[39999, 1] = 3.0
    L[:, 2] = -np.inf
    L[16384, 3] = np.nan
    L[16385, 3] = 2.0
    assert host(ctx.argmax_cols(dev(L))).tolist() == orc.argmax_cols(L).tolist() == [5, 39999, 0, 16385]


@pytest.mark.parametrize("V,B", [(10000, 16), (40000, 4), (97, 3), (1, 2)])
def test_argmax_rows_and_position_advance(ctx, orc, V, B):
    """nnhip_argmax_rows on token-major logits (B, V): the oracle's greedy ids of the transpose
    (ties, NaN at index 0 and elsewhere, all-NaN, +-inf, maxima in different load batches); with
    pos the positions advance by one in the same launch, without it they are left alone."""
    import torch
    say(f"argmax_rows V={V} B={B}")
    L = uniform((V, B), 26 + V)
    L[:, 0] = 0.5                                  # all ties
    if B > 1:
        L[0, 1] = np.nan                           # NaN at index 0 keeps index 0
    if B > 2 and V > 12:
        L[7, 2] = np.nan
        L[11, 2] = L[12, 2] = np.inf
    if B > 3:
        L[:, 3] = np.nan
    if V > 20000 and B > 3:
        L[5, 3] = L[20000, 3] = 3.0               # equal maxima in different load batches
    want = orc.argmax_cols(L).tolist()
    Lt = dev(np.ascontiguousarray(L.T))
    assert host(ctx.argmax_rows(Lt)).tolist() == want == host(ctx.argmax_cols(dev(L))).tolist()
    p0 = np.arange(B, dtype=np.int32) * 7 + 3
    pos = dev(p0)
    ids = dev(np.full(B, -1, np.int32))
    ctx.argmax_rows(Lt, out=ids, pos=pos)
    torch.cuda.synchronize()
    assert host(ids).tolist() == want and host(pos).tolist() == (p0 + 1).tolist()


# ---------------------------------------------------------------- the whole decode step

def _linear(ctx, orc, N, K, seed, bias=True):
    W = normal((N, K), seed, 0.0, 0.02)
    tau = orc.row_absmean(W)
    wq = orc.trit_pack(W, tau)
    b = normal((N,), seed + 1, 0.0, 0.1) if bias else None
    return wq, tau, b


def _build_model(ctx, orc, nnhip, cfg, L, B, seed, subln):
    """Random weights as oracle containers (host) and as device Linear objects."""
    from nnhip_py import decoder as dmod
    torch = __import__("torch")
    host_blocks, dev_blocks = [], []
    d, F, dk = cfg.d, cfg.F, cfg.dk
    for l in range(L):
        s0 = seed + 100 * l
        hb = {
            "g1": normal((d,), s0, 1.0, 0.1), "g2": normal((d,), s0 + 1, 1.0, 0.1),
            "q": _linear(ctx, orc, cfg.H * dk, d, s0 + 2), "k": _linear(ctx, orc, cfg.Hkv * dk, d, s0 + 4),
            "v": _linear(ctx, orc, cfg.Hkv * dk, d, s0 + 6), "o": _linear(ctx, orc, d, cfg.H * dk, s0 + 8),
            "fc1": _linear(ctx, orc, 2 * F, d, s0 + 10), "fc2": _linear(ctx, orc, d, F, s0 + 12),
            "ga": normal((d,), s0 + 14, 1.0, 0.1) if subln else None,
            "gf": normal((F,), s0 + 15, 1.0, 0.1) if subln else None,
        }
        host_blocks.append(hb)

        def lin(t, N, K):
            wq, tau, b = t
            return dmod.Linear(ctx.repack(dev(wq.view(np.int32)), K), dev(tau), None if b is None else dev(b), N, K)

        wo, to, bo = ctx.glu_interleave(dev(hb["fc1"][0].view(np.int32)), dev(hb["fc1"][1]), dev(hb["fc1"][2]), F, d)
        fc1 = dmod.Linear(ctx.repack(wo, d), to, bo, nnhip.glu_rows(F), d)
        dev_blocks.append(dmod.Block(
            g1=dev(hb["g1"]), q=lin(hb["q"], cfg.H * dk, d), k=lin(hb["k"], cfg.Hkv * dk, d), v=lin(hb["v"], cfg.Hkv * dk, d),
            o=lin(hb["o"], d, cfg.H * dk), g2=dev(hb["g2"]), fc1=fc1, fc2=lin(hb["fc2"], d, F),
            g_attn_sub=None if hb["ga"] is None else dev(hb["ga"]),
            g_ffn_sub=None if hb["gf"] is None else dev(hb["gf"])))
    emb = normal((cfg.vocab, d), seed + 7, 0.0, 1.0)
    gfin = normal((d,), seed + 8, 1.0, 0.1)
    head = _linear(ctx, orc, cfg.vocab, d, seed + 9, bias=False)
    head_d = dmod.Linear(ctx.repack(dev(head[0].view(np.int32)), d), dev(head[1]), None, cfg.vocab, d)
    dec = dmod.Decoder(ctx, cfg, dev_blocks, dev(emb), dev(gfin), head_d, B)
    return dec, host_blocks, emb, gfin, head


def _orc_bitlinear(orc, x, lin, gamma, eps):
    """int8 BitLinear of the oracle: [RMSNorm ->] absmax int8 -> matmul_q_i8 [+ b]."""
    wq, tau, b = lin
    if gamma is None:
        s = orc.act_scale(x)
        xq = orc.quantize_i8(x, s, True)
    else:
        xq, s = orc.rmsnorm_quant_i8(x, gamma, eps)
    y = orc.matmul_q_i8(wq, tau, xq, s, x.shape[0], x.shape[1])
    return y if b is None else orc.add_row_broadcast(y, b)


@pytest.mark.parametrize("subln", [True, False])
def test_decode_step_chain(ctx, orc, nnhip, subln):
    """Three decode steps of a 2-block model for 3 sequences at ragged positions (one crossing a
    128-position chunk): every piece of the GPU chain against the oracle chain (GPTBlock::
    forward_step order), with the GPU's attention output fed to the oracle's next step so the
    int8 stages stay bit-exact: q/k/v, o, FFN, residuals, final norm + head, greedy ids bit for
    bit; attention within tolerance; the KV caches bit for bit."""
    from nnhip_py import decoder as dmod
    cfg = dmod.Config(d=256, H=4, Hkv=2, F=320, vocab=97, max_len=200, act=0, eps=1e-5)
    _decode_chain(ctx, orc, nnhip, cfg, B=3, start=np.array([0, 7, 126], np.int32),
                  ids=np.array([3, 50, 96], np.int32), subln=subln, seed=0x5EC + subln, expect_fused=True)


@pytest.mark.parametrize("B", [3, 17])
def test_decode_step_chain_f16_cache(ctx, orc, nnhip, B):
    """The decode chain with the KV caches in f16 (compute = F16, Config.cache_f16): the fused step
    (B = 3) and the unfused one (B = 17), against the oracle chain on the same f16 caches: every
    int8 stage, the logits and the greedy ids bit for bit, attention within tolerance, the caches'
    f16 elements bit for bit."""
    from nnhip_py import decoder as dmod
    cfg = dmod.Config(d=256, H=4, Hkv=2, F=320, vocab=97, max_len=200, act=0, eps=1e-5, cache_f16=True)
    start = (np.arange(B, dtype=np.int32) * 11 + 120) % 190
    ids = (np.arange(B, dtype=np.int32) * 13 + 5) % cfg.vocab
    _decode_chain(ctx, orc, nnhip, cfg, B=B, start=start, ids=ids, subln=True, seed=0x5F1 + B,
                  expect_fused=B <= 16)


def test_decode_step_chain_unfused_b17(ctx, orc, nnhip):
    """17 sequences take the unfused step (block_step, then the column argmax): the same oracle
    chain bit for bit, the last step with advance=True (ids written into the input, every
    position advanced by one)."""
    from nnhip_py import decoder as dmod
    cfg = dmod.Config(d=256, H=4, Hkv=2, F=320, vocab=97, max_len=200, act=0, eps=1e-5)
    B = 17
    start = (np.arange(B, dtype=np.int32) * 11) % 150
    ids = (np.arange(B, dtype=np.int32) * 13 + 5) % cfg.vocab
    _decode_chain(ctx, orc, nnhip, cfg, B=B, start=start, ids=ids, subln=True, seed=0x5F0, expect_fused=False,
                  advance_last=True)


def test_decode_fused_ok_limits_fall_back(ctx, orc, nnhip):
    """A model past the fused step's limits (residual stream wider than the per-token kernel
    takes, or no split-k slicing of fc2) is stepped by block_step instead of failing; the two
    paths give the same bits."""
    import torch
    from nnhip_py import decoder as dmod
    cfg = dmod.Config(d=256, H=4, Hkv=2, F=320, vocab=97, max_len=200, act=0, eps=1e-5)
    B = 4
    dec, hb, emb, gfin, head = _build_model(ctx, orc, nnhip, cfg, 2, B, 0x5F1, True)
    ref, _, _, _, _ = _build_model(ctx, orc, nnhip, cfg, 2, B, 0x5F1, True)
    assert ref.fused_ok()
    dec.fused_max_d = 128          # below d: the per-token kernel would refuse the residual stream
    assert not dec.fused_ok()
    dec2, _, _, _, _ = _build_model(ctx, orc, nnhip, cfg, 2, B, 0x5F1, True)
    dec2.slices_fc2 = 0            # no split-k slicing of fc2
    assert not dec2.fused_ok()
    ids = np.array([1, 2, 3, 4], np.int32)
    pos = np.array([0, 5, 9, 130], np.int32)
    outs = []
    for d_ in (ref, dec, dec2):
        say(f"fused_ok fallback: fused={d_.fused_ok()}")
        lg, nx = d_.step(dev(ids), dev(pos), int(pos.max()) + 1)
        outs.append((host(lg), host(nx)))
        torch.cuda.synchronize()
    for lg, nx in outs[1:]:
        assert same_bits(lg, outs[0][0]) and nx.tolist() == outs[0][1].tolist()


def _decode_chain(ctx, orc, nnhip, cfg, B, start, ids, subln, seed, expect_fused, advance_last=False):
    import torch
    L = 2
    dec, hb, emb, gfin, head = _build_model(ctx, orc, nnhip, cfg, L, B, seed, subln)
    assert dec.caches[0][0].dtype == (torch.float16 if cfg.cache_f16 else torch.float32)
    assert dec.fused_ok() == expect_fused
    cos, sin = orc.rope_table(cfg.dk, cfg.max_len)
    kc_o = [np.zeros((B, cfg.max_len, cfg.Hkv * cfg.dk), np.float32) for _ in range(L)]
    vc_o = [np.zeros_like(kc_o[0]) for _ in range(L)]
    for step in range(3):
        pos = start + step
        advance = advance_last and step == 2
        say(f"decode chain B={B} subln={subln} step {step} advance={advance}")
        attn_gpu = {}
        dec_ids, dec_pos = dev(ids), dev(pos)
        logits_d, next_d = dec.step(dec_ids, dec_pos, int(pos.max()) + 1,
                                    attn_hook=lambda i, a: attn_gpu.__setitem__(i, a.cpu().numpy()), advance=advance)
        logits, nxt = host(logits_d), host(next_d)
        if advance:
            assert host(dec_ids).tolist() == nxt.tolist() and host(dec_pos).tolist() == (pos + 1).tolist()
        # oracle chain
        x = orc.embedding_gather(emb, ids)
        for l in range(L):
            b = hb[l]
            q = _orc_bitlinear(orc, x, b["q"], b["g1"], cfg.eps)
            k = _orc_bitlinear(orc, x, b["k"], b["g1"], cfg.eps)
            v = _orc_bitlinear(orc, x, b["v"], b["g1"], cfg.eps)
            a = orc.attention_decode(q, k, v, cfg.H, cfg.Hkv, cfg.dk, pos, kc_o[l], vc_o[l], cfg.scale, cos, sin,
                                     cache_f16=cfg.cache_f16)
            ag = attn_gpu[l]
            assert np.max(np.abs(ag - a)) <= ATOL * max(1.0, float(np.max(np.abs(a))))
            o = _orc_bitlinear(orc, ag, b["o"], b["ga"], cfg.eps)
            r = x + o
            f, _ = orc.ffn_glu_i8(r, b["g2"], cfg.eps, cfg.F, *b["fc1"], *b["fc2"], 0, gamma_sub=b["gf"],
                                  eps_sub=cfg.eps)
            x = r + f
        lg = _orc_bitlinear(orc, x, head, gfin, cfg.eps)
        assert same_bits(logits, lg), "logits differ"
        assert nxt.tolist() == orc.argmax_cols(lg).tolist()
        torch.cuda.synchronize()
        for l in range(L):
            assert same_bits(host(dec.caches[l][0].float()), kc_o[l])
            assert same_bits(host(dec.caches[l][1].float()), vc_o[l])
        ids = nxt.astype(np.int32)


def test_decode_step_graph_replay(ctx, orc, nnhip):
    """The step captured in a graph (no allocation inside) and replayed: every replay equals an
    eager step from the same state, with eager work and synchronizations between replays."""
    import torch
    from nnhip_py import decoder as dmod
    cfg = dmod.Config(d=256, H=4, Hkv=2, F=320, vocab=97, max_len=300, act=1, eps=1e-5)
    L, B = 2, 4
    dec, *_ = _build_model(ctx, orc, nnhip, cfg, L, B, 0x6A, True)
    ids = dev(np.array([1, 2, 3, 4], np.int32))
    pos = dev(np.array([10, 140, 0, 255], np.int32))
    # fill the caches with arbitrary history
    for kc, vc in dec.caches:
        kc.copy_(torch.from_numpy(normal(tuple(kc.shape), 7)).cuda())
        vc.copy_(torch.from_numpy(normal(tuple(vc.shape), 8)).cuda())
    snap = [(kc.clone(), vc.clone()) for kc, vc in dec.caches]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        dec.step(ids, pos, 300)          # warm-up: grows the context scratch outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = host(dec.logits).copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        dec.step(ids, pos, 300)
    for rep in range(3):
        for (kc, vc), (k0, v0) in zip(dec.caches, snap):
            kc.copy_(k0)
            vc.copy_(v0)
        torch.cuda.synchronize()
        say(f"graph replay {rep}")
        g.replay()
        torch.cuda.synchronize()
        assert same_bits(host(dec.logits), eager)
        _ = ctx.add(dev(np.ones(64, np.float32)), dev(np.ones(64, np.float32)))   # eager work between replays
        torch.cuda.synchronize()


# ---------------------------------------------------------------- fused decode entry points

def _fast_linear(ctx, orc, N, K, seed, bias):
    W = normal((N, K), seed, 0.0, 0.02)
    tau = orc.row_absmean(W)
    wq = orc.trit_pack(W, tau)
    rp = ctx.repack(dev(wq.view(np.int32)), K)
    b = dev(normal((N,), seed + 1, 0.0, 0.1)) if bias else None
    return rp, dev(tau), b


@pytest.mark.parametrize("N,K,M", [(2560, 2560, 16), (2560, 6912, 3), (100, 520, 3), (300, 520, 40)])
def test_ternary_matmul_add_equals_unfused(ctx, orc, N, K, M):
    """Residual in the epilogue (deep GEMV) or a trailing add (other paths): the same bits as
    ternary_matmul followed by add."""
    say(f"ternary_matmul_add N={N} K={K} M={M}")
    rp, tau, b = _fast_linear(ctx, orc, N, K, 10 + N + K, True)
    xi, s, rs = ctx.act_quant_i8(dev(normal((K, M), 11)))
    res = dev(normal((N, M), 12))
    y = host(ctx.ternary_matmul_add(rp, tau, xi, s, rs, N, K, M, res, bias=b))
    ref = host(ctx.add(res, ctx.ternary_matmul(rp, tau, xi, s, rs, N, K, M, bias=b)))
    assert same_bits(y, ref)
    with pytest.raises(Exception):
        out = ctx.ternary_matmul(rp, tau, xi, s, rs, N, K, M)
        ctx.ternary_matmul_add(rp, tau, xi, s, rs, N, K, M, out, out=out)   # aliasing is refused


@pytest.mark.parametrize("N,K,M", [(2560, 2560, 256), (2560, 2560, 2048), (300, 520, 200), (1000, 6912, 130)])
def test_gemm_residual_epilogue_every_tile(ctx, orc, nnhip, N, K, M):
    """The prefill GEMM's residual epilogue (M > 16: y + res added where y is stored), for every
    block tile, interior and edge blocks: the same bits as ternary_matmul (checked against the
    oracle in the parity tests) followed by add."""
    say(f"gemm residual N={N} K={K} M={M}")
    rp, tau, b = _fast_linear(ctx, orc, N, K, 30 + N + K, True)
    X = normal((K, M), 31)
    xi, s, rs = ctx.act_quant_i8(dev(X))
    resh = normal((N, M), 32)
    res = dev(resh)
    ref = host(ctx.add(res, ctx.ternary_matmul(rp, tau, xi, s, rs, N, K, M, bias=b)))
    try:
        for tile in (nnhip.GEMM_TILE_256x128, nnhip.GEMM_TILE_128x128, nnhip.GEMM_TILE_64x64, nnhip.GEMM_TILE_AUTO):
            ctx.set_gemm_tile(tile)
            y = host(ctx.ternary_matmul_add(rp, tau, xi, s, rs, N, K, M, res, bias=b))
            assert same_bits(y, ref), tile
    finally:
        ctx.set_gemm_tile(nnhip.GEMM_TILE_AUTO)


@pytest.mark.parametrize("K,M,Ns", [(2560, 16, (2560, 640, 640)), (2560, 1, (2560, 2560, 2560, 17)),
                                    (520, 5, (100, 30)), (1024, 40, (64, 64, 64))])
def test_ternary_matmul_n_equals_separate(ctx, orc, K, M, Ns):
    """Several BitLinears on one input in one launch (deep path) or in turn: the same bits as
    separate ternary_matmul calls."""
    say(f"ternary_matmul_n K={K} M={M} Ns={Ns}")
    xi, s, rs = ctx.act_quant_i8(dev(normal((K, M), 21)))
    probs = []
    for j, N in enumerate(Ns):
        rp, tau, b = _fast_linear(ctx, orc, N, K, 30 + 7 * j, j % 2 == 1)
        probs.append((rp, tau, b, N, None))
    outs = ctx.ternary_matmul_n(probs, xi, s, rs, K, M)
    for (rp, tau, b, N, _), y in zip(probs, outs):
        ref = ctx.ternary_matmul(rp, tau, xi, s, rs, N, K, M, bias=b)
        assert same_bits(host(y), host(ref))


@pytest.mark.parametrize("d,F,M", [(2560, 6912, 16), (256, 136, 16), (320, 100, 40)])
def test_ffn_glu_i8_add_equals_unfused(ctx, orc, nnhip, d, F, M):
    """The FFN block with the residual in fc2's epilogue: the same bits as ffn_glu_i8 + add."""
    say(f"ffn_glu_i8_add d={d} F={F} M={M}")
    W1 = normal((2 * F, d), 41, 0.0, 0.02)
    t1 = orc.row_absmean(W1)
    wq1 = orc.trit_pack(W1, t1)
    wo, to, _ = ctx.glu_interleave(dev(wq1.view(np.int32)), dev(t1), None, F, d)
    rp1 = ctx.repack(wo, d)
    rp2, t2, b2 = _fast_linear(ctx, orc, d, F, 43, True)
    X = dev(normal((d, M), 44))
    g = dev(normal((d,), 45, 1.0, 0.1))
    gs = dev(normal((F,), 46, 1.0, 0.1))
    res = dev(normal((d, M), 47))
    y = host(ctx.ffn_glu_i8_add(X, g, 1e-5, F, rp1, to, None, rp2, t2, b2, res, gamma_sub=gs))
    ref = host(ctx.add(res, ctx.ffn_glu_i8(X, g, 1e-5, F, rp1, to, None, rp2, t2, b2, gamma_sub=gs)))
    assert same_bits(y, ref)

