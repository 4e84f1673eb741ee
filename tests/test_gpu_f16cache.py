"""GPU parity of the KV caches in f16 (compute = F16: the reference creates each layer's caches in
the profile's compute precision, include/neuralnet.cpp/compute_layer_gpt.hpp:764-765, F16 under the
t1_58 preset, src/t1_58_test.cpp:668-690): nnhip_attention_decode(_tokens)_h, nnhip_kv_cache_fill_h
and nnhip_attention_prefill_h against the oracle with the same caches held as float32 values of
f16 elements (oracle attention_decode with cache_f16: appended rows rounded to f16 before use).

The cache rows are compared bit for bit (the f16 elements, widened); the attention output within
5e-6 x max(1, max|out|) of that oracle, as on f32 caches. Against the f32-cache result the f16
caches stay within the reference's f16 tolerance, 4e-3 x max(1, |ref|)
(src/ternary_gemm_test.cpp:511-516).
"""
import math

import numpy as np
import pytest

from conftest import normal

pytestmark = pytest.mark.gpu

ATOL = 5e-6     # x max(1, max|out|), against the oracle on the same f16 caches
F16_TOL = 4e-3  # x max(1, max|ref|), f16 caches against f32 caches


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


def close(got, ref, tol=ATOL):
    return float(np.max(np.abs(got - ref))) <= tol * max(1.0, float(np.max(np.abs(ref))))


def f16_caches(shape, seed):
    """A cache of f16 elements: the device tensor (float16) and the same values as float32."""
    import torch
    h = normal(shape, seed).astype(np.float16)
    return torch.from_numpy(h).cuda(), h.astype(np.float32)


@pytest.mark.parametrize("B,H,Hkv,dk,pos,rope", [
    (1, 4, 4, 64, [0], True),
    (2, 8, 2, 128, [5, 130], True),
    (3, 20, 5, 128, [127, 128, 300], True),
    (2, 4, 1, 256, [40, 3], False),
    (2, 16, 2, 128, [200, 17], True),
    (16, 20, 5, 128, [0, 1, 2, 127, 128, 129, 255, 256, 300, 301, 200, 311, 100, 150, 64, 65], True),
])
def test_attention_decode_f16_cache(ctx, orc, nnhip, B, H, Hkv, dk, pos, rope):
    """One decode step over f16 caches: appended rows and output against the oracle on the same
    caches; column and token-major layouts alike; within the f16 tolerance of f32 caches."""
    import torch
    say(f"attention f16 cache B={B} H={H} Hkv={Hkv} dk={dk} pos={pos[:6]}")
    max_len = 320
    seed = 0x16 + B * 7 + dk
    q = normal((H * dk, B), seed)
    k = normal((Hkv * dk, B), seed + 1)
    v = normal((Hkv * dk, B), seed + 2)
    kc_d, kc = f16_caches((B, max_len, Hkv * dk), seed + 3)
    vc_d, vc = f16_caches((B, max_len, Hkv * dk), seed + 4)
    kc2_d, vc2_d = kc_d.clone(), vc_d.clone()
    cos, sin = nnhip.rope_table(dk, max_len) if rope else (None, None)
    tabs = (dev(cos), dev(sin)) if rope else (None, None)
    scale = float(np.float32(1.0) / np.float32(math.sqrt(dk)))
    p = dev(np.array(pos, np.int32))
    out = host(ctx.attention_decode(dev(q), dev(k), dev(v), H, Hkv, dk, p, max(pos) + 1, kc_d, vc_d, scale, *tabs))
    kc_o, vc_o = kc.copy(), vc.copy()
    ref = orc.attention_decode(q, k, v, H, Hkv, dk, pos, kc_o, vc_o, scale, cos, sin, cache_f16=True)
    assert close(out, ref)
    assert kc_d.dtype == torch.float16
    assert same_bits(host(kc_d).astype(np.float32), kc_o), "key cache differs"
    assert same_bits(host(vc_d).astype(np.float32), vc_o), "value cache differs"
    # token-major rows: the same bits and the same appended rows
    tr = lambda a: dev(np.ascontiguousarray(a.T))
    got = host(ctx.attention_decode(tr(q), tr(k), tr(v), H, Hkv, dk, p, max(pos) + 1, kc2_d, vc2_d, scale, *tabs,
                                    tokens=True))
    assert same_bits(np.ascontiguousarray(got.T), out)
    assert torch.equal(kc2_d, kc_d) and torch.equal(vc2_d, vc_d)
    # against f32 caches holding the same history: the f16 rounding of the appended rows only
    kc32, vc32 = kc.copy(), vc.copy()
    ref32 = orc.attention_decode(q, k, v, H, Hkv, dk, pos, kc32, vc32, scale, cos, sin)
    assert close(out, ref32, F16_TOL)


def test_attention_decode_f16_cache_incremental(ctx, orc, nnhip):
    """Ten steps from empty f16 caches: every output and both caches stay with the oracle."""
    import torch
    B, H, Hkv, dk, max_len = 3, 8, 2, 64, 300
    cos, sin = nnhip.rope_table(dk, max_len)
    cos_d, sin_d = dev(cos), dev(sin)
    kc = np.zeros((B, max_len, Hkv * dk), np.float32)
    vc = np.zeros_like(kc)
    kc_d = torch.zeros((B, max_len, Hkv * dk), dtype=torch.float16, device="cuda")
    vc_d = torch.zeros_like(kc_d)
    start = np.array([0, 120, 250], np.int32)
    for step in range(10):
        say(f"f16 cache incremental step {step}")
        pos = start + step
        q = normal((H * dk, B), 100 + step)
        k = normal((Hkv * dk, B), 200 + step) * np.float32(30.0)
        v = normal((Hkv * dk, B), 300 + step)
        out = host(ctx.attention_decode(dev(q), dev(k), dev(v), H, Hkv, dk, dev(pos), int(pos.max()) + 1,
                                        kc_d, vc_d, 0.125, cos_d, sin_d))
        ref = orc.attention_decode(q, k, v, H, Hkv, dk, pos, kc, vc, 0.125, cos, sin, cache_f16=True)
        assert close(out, ref)
    torch.cuda.synchronize()
    assert same_bits(host(kc_d).astype(np.float32), kc) and same_bits(host(vc_d).astype(np.float32), vc)


@pytest.mark.parametrize("B,T,H,Hkv,dk,pos0,rope", [
    (3, 100, 8, 2, 128, 0, True),
    (2, 37, 4, 4, 64, 5, False),
    (4, 33, 20, 5, 128, 2000, True),
])
def test_prefill_f16_cache(ctx, orc, nnhip, B, T, H, Hkv, dk, pos0, rope):
    """kv fill and causal prefill attention over f16 caches against T oracle decode steps on the
    same caches: the filled rows bit for bit, every token's attention within tolerance."""
    say(f"prefill f16 cache B={B} T={T} H={H} Hkv={Hkv} dk={dk} pos0={pos0}")
    max_len = 2176 if pos0 >= 2000 else pos0 + T + 7
    seed = 3000 + B + T + H + pos0
    M = B * T
    q = normal((H * dk, M), seed)
    k = normal((Hkv * dk, M), seed + 1)
    v = normal((Hkv * dk, M), seed + 2)
    kc_d, kc = f16_caches((B, max_len, Hkv * dk), seed + 3)
    vc_d, vc = f16_caches((B, max_len, Hkv * dk), seed + 4)
    cos, sin = nnhip.rope_table(dk, max_len) if rope else (None, None)
    cd, sd = (None, None) if cos is None else (dev(cos), dev(sin))
    scale = float(np.float32(1.0) / np.float32(math.sqrt(dk)))
    ctx.kv_cache_fill(dev(k), dev(v), B, T, Hkv, dk, pos0, kc_d, vc_d, cd, sd)
    out = host(ctx.attention_prefill(dev(q), kc_d, vc_d, B, T, H, Hkv, dk, pos0, scale, cd, sd))
    kc_o, vc_o = kc.copy(), vc.copy()
    cols = np.arange(B) * T
    for t in range(T):
        ref = orc.attention_decode(q[:, cols + t], k[:, cols + t], v[:, cols + t], H, Hkv, dk,
                                   np.full(B, pos0 + t, np.int32), kc_o, vc_o, scale, cos, sin, cache_f16=True)
        assert close(out[:, cols + t], ref), f"token {t}"
    assert same_bits(host(kc_d).astype(np.float32), kc_o), "key cache differs"
    assert same_bits(host(vc_d).astype(np.float32), vc_o), "value cache differs"


def test_f16_cache_rejects_mixed_dtypes(ctx, nnhip):
    import torch
    q = torch.zeros((8 * 64, 2), device="cuda")
    k = torch.zeros((2 * 64, 2), device="cuda")
    kc = torch.zeros((2, 16, 2 * 64), dtype=torch.float16, device="cuda")
    vc = torch.zeros((2, 16, 2 * 64), dtype=torch.float32, device="cuda")
    pos = torch.zeros(2, dtype=torch.int32, device="cuda")
    with pytest.raises(nnhip.NNHipError):
        ctx.attention_decode(q, k, k, 8, 2, 64, pos, 1, kc, vc, 0.125)
    with pytest.raises(nnhip.NNHipError):
        ctx.kv_cache_fill(k, k, 2, 1, 2, 64, 0, kc, vc)
