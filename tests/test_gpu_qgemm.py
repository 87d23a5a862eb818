"""GPU parity of the batched MFMA 4-bit GEMM (ming_qgemm: M = 1..64 rows of
activations against one MLX-affine matrix, the batched shape of
mlx_quantized_matmul) against the oracle's M-row linear, at the five GEMV
shapes of the 4-bit sweep.

Bars: f32 accumulators within 1e-4 + 1e-5 |ref| of the oracle's f64-free
f32 group sums (the MFMA sums 32 products in f32 then the groups in f32, in
another order than the oracle); bf16 outputs within 2e-2 + 1e-2 |ref|, and
each one the rounding of its own f32 accumulator; each row of a batch agrees
with the single-row ming_qgemv of that row within the same f32 bar."""
import numpy as np
import pytest
import torch

from lmkit import assert_close_bf16

pytestmark = pytest.mark.gpu

SHAPES = [(896, 896), (896, 128), (896, 4864), (4864, 896), (896, 151936)]  # [in, out]


def dev_u16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)


def host_u16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def make(ming, ctx, K, N, M, seed=0, std=0.02):
    print(f"[qgemm] shape in={K} out={N} rows={M} seed={seed}", flush=True)
    w = ming.synth_normal_bf16(seed, f"w{K}x{N}", N * K, 0.0, std).reshape(N, K)
    x = ming.synth_normal_bf16(seed + 100, f"xm{K}.{M}", M * K, 0.0, 1.0).reshape(M, K)
    wq = torch.empty((N, K // 8), dtype=torch.int32, device="cuda")
    s = torch.empty((N, K // 64), dtype=torch.bfloat16, device="cuda")
    b = torch.empty((N, K // 64), dtype=torch.bfloat16, device="cuda")
    ctx.quantize(dev_u16(w), wq, s, b)
    ctx.sync()
    return x, wq, s, b


def close_f32(got, ref, what):
    d = np.abs(got.astype(np.float64) - ref)
    ok = d <= 1e-4 + 1e-5 * np.abs(ref)
    assert ok.all(), f"{what}: {int((~ok).sum())} of {ok.size} outside, max|d| {d.max():.3e}"
    return d.max()


@pytest.mark.parametrize("K,N", SHAPES)
@pytest.mark.parametrize("M", [16, 64])
def test_qgemm_matches_oracle(ming, oracle, ctx, K, N, M):
    x, wq, s, b = make(ming, ctx, K, N, M)
    L = oracle.Linear(wq.cpu().numpy().view(np.uint32), host_u16(s), host_u16(b))
    ref_acc = oracle.linear_acc(L, x)
    ref = oracle.linear(L, x)
    xd = dev_u16(x)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    yf = torch.empty((M, N), dtype=torch.float32, device="cuda")
    ctx.qgemm(xd, wq, s, b, y)
    ctx.qgemm(xd, wq, s, b, yf)
    ctx.sync()
    got = yf.cpu().numpy()
    df = close_f32(got, ref_acc, f"qgemm f32 [{K}x{N}] M={M}")
    md = assert_close_bf16(host_u16(y), ref, f"qgemm [{K}x{N}] M={M}")
    assert np.array_equal(host_u16(y), oracle.to_bf16(got))
    print(f"[qgemm] [{K}x{N}] M={M} max|d| bf16 {md:.3e} f32 {df:.3e}", flush=True)


@pytest.mark.parametrize("M", [1, 5, 17, 40])
def test_qgemm_ragged_rows_match_qgemv(ming, oracle, ctx, M):
    """Row counts that are not multiples of the 16-row tile: every row equals
    the single-row GEMV of that row (f32 bar), and nothing past row M is written."""
    K, N = 896, 4864
    x, wq, s, b = make(ming, ctx, K, N, M, seed=3)
    xd = dev_u16(x)
    yf = torch.full((M + 1, N), 7.0, dtype=torch.float32, device="cuda")
    ctx.qgemm(xd, wq, s, b, yf[:M])
    ctx.sync()
    for m in range(M):
        r = torch.empty(N, dtype=torch.float32, device="cuda")
        ctx.qgemv(xd[m], wq, s, b, r, f32=True)
        ctx.sync()
        close_f32(yf[m].cpu().numpy(), r.cpu().numpy().astype(np.float64), f"row {m} of {M}")
    assert bool((yf[M] == 7.0).all()), "row past M written"


def test_qgemm_global_scale(ming, oracle, ctx):
    K, N, M = 4864, 896, 16
    x, wq, s, b = make(ming, ctx, K, N, M, seed=4)
    xd = dev_u16(x)
    y1 = torch.empty((M, N), dtype=torch.float32, device="cuda")
    y2 = torch.empty((M, N), dtype=torch.float32, device="cuda")
    ctx.qgemm(xd, wq, s, b, y1)
    ctx.qgemm(xd, wq, s, b, y2, global_scale=0.5)
    ctx.sync()
    assert torch.equal(y2, y1 * 0.5)


def test_qgemm_shape_errors(ming, ctx):
    K, N = 896, 128
    x, wq, s, b = make(ming, ctx, K, N, 65)
    y = torch.empty((65, N), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ming.MingError) as e:
        ctx.qgemm(dev_u16(x), wq, s, b, y)
    assert e.value.status == ming.MING_E_UNSUPPORTED
    y = torch.empty((64, N + 1), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ming.MingError) as e:
        ctx.qgemm(dev_u16(x[:64]), wq, s, b, y)
    assert e.value.status == ming.MING_E_SHAPE
