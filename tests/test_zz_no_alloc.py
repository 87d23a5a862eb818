"""GPU check of ming_qgemm_noalloc, the batched 4-bit GEMM that stages its
activations in the device's fixed scratch array instead of allocating:
through the C ABI, its outputs equal ming_qgemm's bit for bit (same
kernels) on two calls in a row, the second with a smaller input; on a new
context it leaves the context's on-demand workspaces at 0 bytes (where
ming_qgemm then grows them); and a request larger than the fixed scratch is
rejected before any launch."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def dev_u16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)


def quantized(ming, ctx, K, N, seed):
    w = ming.synth_normal_bf16(seed, f"noalloc.w{K}x{N}", N * K, 0.0, 0.02).reshape(N, K)
    wq = torch.empty((N, K // 8), dtype=torch.int32, device="cuda")
    s = torch.empty((N, K // 64), dtype=torch.bfloat16, device="cuda")
    b = torch.empty((N, K // 64), dtype=torch.bfloat16, device="cuda")
    ctx.quantize(dev_u16(w), wq, s, b)
    return wq, s, b


def test_qgemm_noalloc_matches_qgemm(ming, ctx):
    # a large call, then a smaller one: the second must not see the first's staging
    for K, N, M, seed in ((4864, 896, 64, 1), (896, 1152, 5, 2)):
        print(f"[noalloc] K={K} N={N} M={M} seed={seed}", flush=True)
        wq, s, b = quantized(ming, ctx, K, N, seed)
        x = dev_u16(ming.synth_normal_bf16(seed + 50, f"noalloc.x{K}.{M}", M * K)).reshape(M, K)
        for dt in (torch.float32, torch.bfloat16):
            ref = torch.empty((M, N), dtype=dt, device="cuda")
            got = torch.full((M, N), 3.0, dtype=dt, device="cuda")
            ctx.qgemm(x, wq, s, b, ref, global_scale=0.5)
            ctx.qgemm_noalloc(x, wq, s, b, got, global_scale=0.5)
            ctx.sync()
            assert torch.equal(got.view(torch.int16) if dt == torch.bfloat16 else got.view(torch.int32),
                               ref.view(torch.int16) if dt == torch.bfloat16 else ref.view(torch.int32)), \
                f"noalloc differs from qgemm at K={K} N={N} M={M} {dt}"


def test_qgemm_noalloc_allocates_nothing(ming):
    K, N, M = 4864, 896, 64
    own = ming.Context(0)  # a new context: nothing has grown its workspaces yet
    try:
        wq, s, b = quantized(ming, own, K, N, 4)
        x = dev_u16(ming.synth_normal_bf16(54, "noalloc.fresh.x", M * K)).reshape(M, K)
        got = torch.full((M, N), 3.0, dtype=torch.float32, device="cuda")
        ref = torch.empty((M, N), dtype=torch.float32, device="cuda")
        own.sync()
        assert own.workspace_bytes() == 0
        own.qgemm_noalloc(x, wq, s, b, got)
        own.sync()
        assert own.workspace_bytes() == 0, "ming_qgemm_noalloc allocated a workspace"
        own.qgemm(x, wq, s, b, ref)  # the allocating entry point grows the staging (the query sees it)
        own.sync()
        assert own.workspace_bytes() > 0
        assert torch.equal(got.view(torch.int32), ref.view(torch.int32))
    finally:
        own.close()


def test_qgemm_noalloc_rejects_beyond_scratch(ming, ctx):
    K, N, M = 16384, 64, 64
    wq, s, b = quantized(ming, ctx, K, N, 3)
    x = torch.zeros((M, K), dtype=torch.bfloat16, device="cuda")
    y = torch.full((M, N), 9.0, dtype=torch.float32, device="cuda")
    ctx.sync()
    with pytest.raises(ming.MingError) as e:
        ctx.qgemm_noalloc(x, wq, s, b, y)
    assert e.value.status == ming.MING_E_UNSUPPORTED
    assert "fixed scratch" in str(e.value)
    ctx.sync()
    assert bool((y == 9.0).all()), "a rejected call wrote its output"
