"""FP8 prefill GEMM (krq_gemm_fp8, kernels.fp8.gemm_fp8) against the exact oracle product of the
same e4m3 operands: max|y - ref| <= 1e-2 * max|ref| (the path's tolerance), for ragged M, per
tensor / per row scales, e4m3 activations and bf16 activations quantized in the kernel; the fused
cast is bit-identical to the reference's cast followed by the GEMM."""

import numpy as np
import pytest
import torch

from kernels import fp8 as F
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-2


def rel_err(y, ref):
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def codes(t):
    return t.cpu().view(torch.uint8).numpy()


def bf(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("M,N,K,per_row", [(33, 128, 128, True), (128, 256, 256, False), (300, 384, 640, True),
                                           (257, 6144, 2560, True), (256, 2560, 9728, False),
                                           (600, 512, 384, True), (1024, 2560, 9728, False), (777, 6144, 2560, True),
                                           # 256 x 256 ring tiles (>= 128 of them): ragged M, a tile count
                                           # that is not a multiple of the 8 XCDs, several tiles per CU
                                           (2000, 4096, 2560, True), (2100, 4352, 256, True),
                                           (4096, 8192, 384, False),
                                           # 192 x 256 tiles: ragged M (20 full row tiles + 160 rows)
                                           (4000, 2560, 512, True), (4096, 2560, 4096, False),
                                           # 64 x 64 tiles: small grids that do not split K
                                           (256, 2560, 4096, True), (100, 1024, 512, False),
                                           # a whole round of 256 x 256 tiles over the first 4096
                                           # columns, then 128 x 128 tiles over the last 2048 (two
                                           # launches into one output), also with ragged M
                                           (4096, 6144, 512, False), (3900, 6144, 384, True)])
def test_gemm_fp8_matches_oracle(dev, M, N, K, per_row):
    w = bf((N, K), 1, 0.02).to(dev)
    q = F.quantize(w) if per_row else F.quantize_weight(w)
    x = bf((M, K), 2).to(dev)
    x8, xs = F.quant_rows(x)                      # e4m3 activations, per-token scales
    y = F.gemm_fp8(x8, q, xs=xs)
    _, ref = O.fp8_matmul(codes(x8), xs.cpu().numpy().reshape(-1), codes(q[0]), q[1].cpu().numpy())
    e = rel_err(y.float().cpu().numpy(), ref)
    print(f"gemm M={M} N={N} K={K}: max-rel {e:.2e}")
    assert e <= TOL


@pytest.mark.parametrize("M,N,K,pad", [(4000, 19456, 2560, 4096),   # 256 x 256, ~5 tiles per block
                                       (3900, 19456, 2560, 4096),
                                       (2000, 19456, 2560, 2048),   # 256 x 256 rounds + 128 x 128 tail
                                       (3000, 6144, 2560, 3072)])   # 192 x 256, a second tile after a ragged one
def test_gemm_ragged_multi_tile(dev, M, N, K, pad):
    """More ring tiles than blocks with M not a multiple of the tile height (gate_up and QKV
    shapes), so blocks run tiles after one with rows past M: within the bar of the oracle on a
    sample of rows (the last 256, which hold the ragged row tile, and every 61st row), and bit for
    bit the rows of a run on M padded to a whole number of tiles (the same tile plan, no ragged
    tile; each output is the same sum of the same products in the same order)."""
    w = bf((N, K), 51, 0.02).to(dev)
    q = F.quantize(w)
    x = bf((pad, K), 52).to(dev)
    x8p, xsp = F.quant_rows(x)
    x8, xs = x8p[:M].contiguous(), xsp[:M].contiguous()
    y = F.gemm_fp8(x8, q, xs=xs)
    y_pad = F.gemm_fp8(x8p, q, xs=xsp)
    assert torch.equal(y, y_pad[:M])
    rows = np.unique(np.concatenate([np.arange(0, M, 61), np.arange(M - 256, M)]))
    _, ref = O.fp8_matmul(codes(x8)[rows], xs.cpu().numpy().reshape(-1)[rows], codes(q[0]), q[1].cpu().numpy())
    e = rel_err(y.float().cpu().numpy()[rows], ref)
    print(f"gemm ragged M={M} N={N} K={K}: max-rel {e:.2e} on {rows.size} rows")
    assert e <= TOL


@pytest.mark.parametrize("M,N,K,splits", [(256, 2560, 9728, 4), (200, 2560, 9728, 4), (300, 2560, 8192, 4),
                                          (130, 4096, 8192, 4), (1024, 2560, 9728, 2),
                                          # 64 x 64 tiles split (too few 128 x 128 ones to split)
                                          (64, 2560, 9728, 4), (100, 2560, 9728, 4)])
def test_gemm_split_k(dev, M, N, K, splits):
    """Split K (krq_gemm_fp8_ws with its workspace) and the unsplit kernel (krq_gemm_fp8, or the
    workspace form given too little workspace, which must then equal it bit for bit): both within
    the bar of the oracle."""
    from kernels import _lib as L
    lib = L.lib()
    assert lib.krq_gemm_fp8_ws_bytes(L.X_FP8, M, N, K) == splits * M * N * 4
    q = F.quantize(bf((N, K), 11, 0.02).to(dev))
    x8, xs = F.quant_rows(bf((M, K), 12).to(dev))
    _, ref = O.fp8_matmul(codes(x8), xs.cpu().numpy().reshape(-1), codes(q[0]), q[1].cpu().numpy())
    y_split = F.gemm_fp8(x8, q, xs=xs)
    args = (L.ptr(x8), L.X_FP8, L.ptr(xs), None, 1, L.ptr(q[0]), L.ptr(q[1]), 1, M, N, K)
    y_plain = torch.empty_like(y_split)
    L.call("krq_gemm_fp8", *args, L.ptr(y_plain), L.stream(x8))
    small = torch.empty(splits * M * N * 4 - 16, device=dev, dtype=torch.uint8)
    y_small = torch.empty_like(y_split)
    L.call("krq_gemm_fp8_ws", *args, L.ptr(small), small.numel(), L.ptr(y_small), L.stream(x8))
    assert torch.equal(y_small, y_plain)
    for y in (y_split, y_plain):
        e = rel_err(y.float().cpu().numpy(), ref)
        print(f"gemm M={M} N={N} K={K} splits={splits}: max-rel {e:.2e}")
        assert e <= TOL


@pytest.mark.parametrize("M,N,K", [(200, 256, 128), (200, 256, 384), (512, 2560, 4096)])
def test_gemm_fused_cast_is_cast_then_gemm(dev, M, N, K):
    """bf16 x with an ActScale: gemm_fp8 (the cast fused into the 128 x 128 kernel at K = 128,
    the HIP cast then the e4m3 kernels otherwise) equals fp8._cast + the e4m3 GEMM bit for bit; the
    C ABI's fused-cast kernel (krq_gemm_fp8 on bf16 rows) and linear_fp8 (prefill) are within the
    bar of the oracle."""
    from kernels import _lib as L
    w = bf((N, K), 3, 0.02).to(dev)
    q = F.quantize_weight(w)
    x = bf((M, K), 4).to(dev)
    a = F.ActScale(x)
    y = F.gemm_fp8(x, q, a)
    y2 = F.gemm_fp8(F._cast(x, a), q, xs=a.scale.reshape(1))
    assert torch.equal(y, y2)
    y3 = torch.empty_like(y)
    L.call("krq_gemm_fp8", L.ptr(x), L.X_BF16_STATIC, L.ptr(a.scale), L.ptr(a.inv), 0, L.ptr(q[0]), L.ptr(q[1]), 0,
           M, N, K, L.ptr(y3), L.stream(x))
    _, ref = O.fp8_matmul(codes(F._cast(x, a)), a.scale.cpu().numpy(), codes(q[0]), q[1].cpu().numpy())
    assert rel_err(F.linear_fp8(x, q).float().cpu().numpy(), ref) <= TOL
    assert rel_err(y.float().cpu().numpy(), ref) <= TOL
    assert rel_err(y3.float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("M,N,K", [(128, 2560, 4096), (300, 6144, 2560), (64, 2560, 4096), (200, 256, 128)])
def test_linear_fp8_prefill_route(dev, M, N, K):
    """linear_fp8 above the decode sizes (engine/kernels/fp8.py:105-106): from PREFILL_MIN_ROWS rows,
    on weights the ring kernels take, it is gemm_fp8 on the cast rows bit for bit; below that (or
    for K = 128) the library's torch._scaled_mm bit for bit. Both within the bar of the oracle."""
    q = F.quantize_weight(bf((N, K), 31, 0.02).to(dev))
    x = bf((M, K), 32).to(dev)
    a = F.ActScale(x)
    y = F.linear_fp8(x, q, a)
    # without a given scale linear_fp8 takes its own (ActScale and the cast in two launches),
    # the same bits, and records amax in amax_out
    amax_out = torch.zeros(1, device=dev)
    assert torch.equal(F.linear_fp8(x, q, amax_out=amax_out), y)
    assert torch.equal(amax_out, a.amax.reshape(1))
    x8 = F._cast(x, a)
    if M >= F.PREFILL_MIN_ROWS and K >= 256:
        assert torch.equal(y, F.gemm_fp8(x8, q, xs=a.scale.reshape(1)))
    else:
        assert torch.equal(y, torch._scaled_mm(x8, q[0].t(), scale_a=a.scale, scale_b=q[1], out_dtype=torch.bfloat16))
    _, ref = O.fp8_matmul(codes(x8), a.scale.cpu().numpy(), codes(q[0]), q[1].cpu().numpy())
    assert rel_err(y.float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("M,N,K", [(4096, 6144, 512), (256, 2560, 9728), (300, 6144, 2560)])
def test_gemm_graph_replays(dev, M, N, K):
    """gemm_fp8 captured in a graph (the two-launch tail plan, split K with its reduce and the
    workspace, a plain ring launch): every replay, with eager work between them, equals the eager
    result bit for bit."""
    q = F.quantize(bf((N, K), 41, 0.02).to(dev))
    x8, xs = F.quant_rows(bf((M, K), 42).to(dev))
    want = F.gemm_fp8(x8, q, xs=xs)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        F.gemm_fp8(x8, q, xs=xs)  # warm-up on a side stream, as before any capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = F.gemm_fp8(x8, q, xs=xs)
    for r in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want), f"replay {r}"
        F.gemm_fp8(x8, q, xs=xs).sum().item()  # eager work between the replays
        y.zero_()
        torch.cuda.synchronize()


def test_gemm_matches_library_gemm(dev):
    """Against torch._scaled_mm (hipBLASLt) on the same operands: both within the bar of the oracle,
    and within a few bf16 ulps of each other."""
    M, N, K = 384, 2560, 2560
    q = F.quantize_weight(bf((N, K), 5, 0.02).to(dev))
    x = bf((M, K), 6).to(dev)
    a = F.ActScale(x)
    x8 = F._cast(x, a)
    ours = F.gemm_fp8(x8, q, xs=a.scale.reshape(1)).float()
    lib = torch._scaled_mm(x8, q[0].t(), scale_a=a.scale, scale_b=q[1], out_dtype=torch.bfloat16).float()
    assert rel_err(ours.cpu().numpy(), lib.cpu().numpy()) <= 2 * 2.0 ** -8


def test_gemm_rejects_bad_shapes(dev):
    q = F.quantize_weight(bf((200, 256), 7).to(dev))  # N not a multiple of 128
    x8, xs = F.quant_rows(bf((64, 256), 8).to(dev))
    with pytest.raises(ValueError):
        F.gemm_fp8(x8, q, xs=xs)
