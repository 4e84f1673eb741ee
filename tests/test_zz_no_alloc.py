"""The allocation-free entry point nnhip_matmul_q_i8_noalloc, called through the C ABI: its
output equals nnhip_matmul_q_i8's (itself bit-exact against the oracle) bit for bit, on calls in a
row whose sizes shrink (so stale scratch contents from the larger call would show), and the
oracle's CpuEngine restatement agrees; sizes beyond its scratch are refused before any work."""
import numpy as np
import pytest

from conftest import normal

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).cuda()


def case(orc, N, K, M, seed):
    W = normal((N, K), seed, 0.0, 0.02)
    tau = orc.row_absmean(W)
    X = normal((K, M), seed + 1)
    s = orc.act_scale(X)
    return orc.trit_pack(W, tau), tau, orc.quantize_i8(X, s, True), s


def test_noalloc_matches_allocating_entry(ctx, orc):
    import torch
    # GEMM path (M > 16), then the GEMV path, then a ragged tail shape: each smaller than the last
    for N, K, M, seed in ((2560, 6912, 96, 11), (1024, 1024, 8, 0xB17A0001), (130, 17, 6, 31)):
        print(f"noalloc matmul_q_i8 N={N} K={K} M={M}", flush=True)
        wq, tau, xq, s = case(orc, N, K, M, seed)
        args = (dev(wq), dev(tau), dev(xq), dev(s))
        out = torch.full((N, M), float("nan"), dtype=torch.float32, device="cuda")
        Y_na = ctx.matmul_q_i8_noalloc(*args, K, M, out=out).cpu().numpy()
        Y_ref = ctx.matmul_q_i8(*args, K, M).cpu().numpy()
        assert np.array_equal(Y_na, Y_ref)
        assert np.array_equal(Y_na, orc.matmul_q_i8_rowblock(wq, tau, xq, s, K, M))


def test_noalloc_rejects_oversize(ctx, nnhip):
    import torch
    # 16384 x 8192 ternary weights repack to 32 MiB on their own: beyond the scratch
    N, K, M = 16384, 8192, 1
    wq = torch.zeros((N, K // 16), dtype=torch.int32, device="cuda")
    tau = torch.ones(N, dtype=torch.float32, device="cuda")
    xq = torch.zeros((K, 1), dtype=torch.int32, device="cuda")
    s = torch.ones(1, dtype=torch.float32, device="cuda")
    out = torch.zeros((N, M), dtype=torch.float32, device="cuda")
    with pytest.raises(nnhip.NNHipError) as e:
        ctx.matmul_q_i8_noalloc(wq, tau, xq, s, K, M, out=out)
    assert e.value.status == 5 and "scratch" in str(e.value)
    assert torch.count_nonzero(out).item() == 0   # nothing was queued
