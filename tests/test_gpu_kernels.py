"""GPU parity of the quantized GEMM and the activation quantiser against the CPU oracle.

Bar: int32 per-block dots bit-exact; fp32 outputs within 1e-3
relative (they are in fact bit-identical, which is asserted too).
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import q8_activations, random_q4_0, random_q4_k, random_q5_k, random_q8_0

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ctx():
    import nanocamelid_amd as nc
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    return nc.Context(0)


def _run_gemm(ctx, qtype, blocks, M, K, xq, xs):
    import nanocamelid_amd as nc
    w = nc.QMat(ctx, qtype, M, K, blocks)
    xt = torch.from_numpy(xq).cuda()
    st = torch.from_numpy(xs).cuda()
    out = nc.matmul_quantized_batch(ctx, w, xt, st)
    dots = nc.matmul_blockdots(ctx, w, xt)
    torch.cuda.synchronize()
    return out.cpu().numpy(), dots.cpu().numpy()


@pytest.mark.parametrize("N", [1, 2, 5, 9, 16])
def test_q4_0_small_bit_exact(ctx, N):
    import nanocamelid_amd as nc
    M, K = 320, 768  # 5 tiles, 24 blocks (3 groups)
    w = random_q4_0(M, K, seed=N)
    _, xq, xs = q8_activations(N, K, seed=100 + N)
    out, dots = _run_gemm(ctx, nc.NC_TYPE_Q4_0, w, M, K, xq, xs)
    ref = O.matmul_q4_0(xq, xs, w, N, M, K)
    ref_dots = O.matmul_q4_0_blockdots(xq, w, N, M, K)
    assert np.array_equal(dots, ref_dots)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_q4_0_partial_group_and_tile(ctx):
    # K/32 = 13 blocks (last group partial), M = 100 rows (last tile partial)
    import nanocamelid_amd as nc
    M, K, N = 100, 416, 3
    w = random_q4_0(M, K, seed=7)
    _, xq, xs = q8_activations(N, K, seed=8)
    out, dots = _run_gemm(ctx, nc.NC_TYPE_Q4_0, w, M, K, xq, xs)
    assert np.array_equal(dots, O.matmul_q4_0_blockdots(xq, w, N, M, K))
    assert np.array_equal(out, O.matmul_q4_0(xq, xs, w, N, M, K))


@pytest.mark.parametrize("N", [1, 2, 3, 4, 5, 6, 7, 8, 9, 16])
@pytest.mark.parametrize("shape", [(100, 416), (32800, 416)], ids=["r16-partial", "r64-partial"])
def test_q4_0_layouts_partial(ctx, shape, N):
    """Both device layouts (16-row tiles below 512 64-row tiles, 64-row tiles above) with a
    partial last tile, a partial last quad of blocks (13 blocks) and every batch width."""
    import nanocamelid_amd as nc
    M, K = shape
    w = random_q4_0(M, K, seed=M + N)
    _, xq, xs = q8_activations(N, K, seed=9 * N + M)
    out, dots = _run_gemm(ctx, nc.NC_TYPE_Q4_0, w, M, K, xq, xs)
    assert np.array_equal(dots, O.matmul_q4_0_blockdots(xq, w, N, M, K, nthreads=16))
    assert np.array_equal(out.view(np.uint32), O.matmul_q4_0(xq, xs, w, N, M, K, nthreads=16).view(np.uint32))


CONFIG1 = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (128256, 4096)]


@pytest.mark.parametrize("shape", CONFIG1, ids=lambda s: f"{s[0]}x{s[1]}")
def test_q4_0_config1_shapes(ctx, shape):
    """Config 1: Llama-3-8B projection shapes, N = 1, 2, 5, 9, 16, weights N(0,0.02)->Q4_0,
    activations N(0,1)->Q8_0.  Every output and every block dot is compared."""
    import nanocamelid_amd as nc
    M, K = shape
    w = random_q4_0(M, K, seed=M + K)
    q = nc.QMat(ctx, nc.NC_TYPE_Q4_0, M, K, w)
    for N in (1, 2, 5, 9, 16):
        x, xq, xs = q8_activations(N, K, seed=N * 31 + M)
        xt, st = torch.from_numpy(xq).cuda(), torch.from_numpy(xs).cuda()
        out = nc.matmul_quantized_batch(ctx, q, xt, st).cpu().numpy()
        ref = O.matmul_q4_0(xq, xs, w, N, M, K, nthreads=16)
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), N
        # fp32 within 1e-3 relative of a float64 evaluation of the same quantized product
        if M * K <= 4096 * 14336:
            wf = _dequant(w).astype(np.float64)
            xf = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 32, axis=1)
            r64 = xf @ wf.T
            err = np.abs(out - r64) / (np.abs(r64) + 1e-3 * np.abs(r64).max())
            assert err.max() < 1e-3
        if N in (1, 5, 16):
            rows = np.random.default_rng(N).choice(M, size=min(M, 512), replace=False)
            dots = nc.matmul_blockdots(ctx, q, xt).cpu().numpy()[:, rows]
            ref_dots = O.matmul_q4_0_blockdots(xq, w.reshape(M, -1)[rows], N, len(rows), K, nthreads=16)
            assert np.array_equal(dots, ref_dots)


PROMPT_SHAPES = [(4096, 4096, (17, 64, 100, 256)), (1040, 96, (33, 300)), (32816, 64, (17, 129)),
                 (14336, 4096, (48,)), (4096, 14336, (40,))]


@pytest.mark.parametrize("M,K,Ns", PROMPT_SHAPES, ids=[f"{m}x{k}" for m, k, _ in PROMPT_SHAPES])
def test_q4_0_prompt_matmul(ctx, M, K, Ns):
    """More than 16 tokens take the MFMA prompt matmul (inference.rs:1385-1418 for any batch):
    every output bit-identical to the oracle.  Covers 16-row tiles (R16) with 4096 and 3 blocks
    per row (a partial quad) and rows not a multiple of 64, 64-row tiles (R64, >= 512 tiles) with
    a partial last tile, token counts that leave partial 16- and 64-token tiles, and 300 tokens
    (two slices through the context's 256-token repack buffers); wave tiles of 16 rows (small
    matrices) and 32 rows (32816 x 64)."""
    import nanocamelid_amd as nc
    w = random_q4_0(M, K, seed=M + 7 * K)
    q = nc.QMat(ctx, nc.NC_TYPE_Q4_0, M, K, w)
    for N in Ns:
        x, xq, xs = q8_activations(N, K, seed=N * 17 + M)
        xt, st = torch.from_numpy(xq).cuda(), torch.from_numpy(xs).cuda()
        out = nc.matmul_quantized_batch(ctx, q, xt, st).cpu().numpy()
        ref = O.matmul_q4_0(xq, xs, w, N, M, K, nthreads=16)
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), N


@pytest.mark.parametrize("M,K", [(4096, 4096), (1000, 8192), (777, 3072)])
def test_q6_k_matmul(ctx, M, K):
    """Q6_K output projections (matmul_q6_k_batch, inference.rs:1882-2000, per-element f32 chain
    in Q6KBlock::dot_q8_scaled order): every output bit-identical to the oracle at 1..16 tokens,
    including a shape whose 12 super-blocks per row leave idle lanes."""
    import nanocamelid_amd as nc
    from tests.gguf_writer import random_blocks
    w = random_blocks(nc.NC_TYPE_Q6_K, M * K // 256, seed=M + K)
    q = nc.QMat(ctx, nc.NC_TYPE_Q6_K, M, K, w.reshape(M, K // 256, 210))
    for N in (1, 3, 5, 9, 16, 21):
        x, xq, xs = q8_activations(N, K, seed=N + K)
        out = nc.matmul_quantized_batch(ctx, q, torch.from_numpy(xq).cuda(), torch.from_numpy(xs).cuda()).cpu().numpy()
        ref = O.matmul_q6_k(xq, xs, w, N, M, K, nthreads=16)
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), N


Q4K_PROMPT_SHAPES = [(512, 1024, (17, 37, 64, 100, 300)), (1000, 768, (33, 129)), (16400, 256, (17, 70, 300))]


@pytest.mark.parametrize("M,K,Ns", Q4K_PROMPT_SHAPES, ids=[f"{m}x{k}" for m, k, _ in Q4K_PROMPT_SHAPES])
def test_q4_k_prompt_matmul(ctx, M, K, Ns):
    """More than 16 tokens on Q4_K matrices take the MFMA prompt matmul (matmul_q4_k_batch,
    inference.rs:2006-2132, any batch): every output bit-identical to the oracle.  16-row tiles
    (R16K) with 4 and 3 super-blocks per row and a partial last tile, 64-row tiles (R64, >= 256
    tiles) with a partial last tile; token counts that leave partial 16- and 64-token tiles, and
    300 tokens (two repack slices); wave tiles of 16 rows and, for 16400 rows at 300 tokens, 32."""
    import nanocamelid_amd as nc
    w = random_q4_k(M, K, seed=M + K)
    q = nc.QMat(ctx, nc.NC_TYPE_Q4_K, M, K, w)
    for N in Ns:
        x, xq, xs = q8_activations(N, K, seed=N + 3 * M)
        out = nc.matmul_quantized_batch(ctx, q, torch.from_numpy(xq).cuda(), torch.from_numpy(xs).cuda()).cpu().numpy()
        ref = O.matmul_q4_k(xq, xs, w, N, M, K, nthreads=16)
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), N


def _dequant(w):
    M, nb, _ = w.shape
    sc = (w[:, :, 0].astype(np.uint16) | (w[:, :, 1].astype(np.uint16) << 8)).view(np.float16).astype(np.float32)
    lo = (w[:, :, 2:] & 15).astype(np.float32) - 8
    hi = (w[:, :, 2:] >> 4).astype(np.float32) - 8
    return (np.concatenate([lo, hi], 2) * sc[:, :, None]).reshape(M, nb * 32)


@pytest.mark.parametrize("N", [1, 5, 9, 16])
def test_q4_k_bit_exact(ctx, N):
    import nanocamelid_amd as nc
    M, K = 192, 1024
    w = random_q4_k(M, K, seed=N)
    _, xq, xs = q8_activations(N, K, seed=200 + N)
    out, dots = _run_gemm(ctx, nc.NC_TYPE_Q4_K, w, M, K, xq, xs)
    ref = O.matmul_q4_k(xq, xs, w, N, M, K)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    # per 32-sub-block W_j = sum nib * x (q8.rs:1339-1376)
    for r in (0, 7, 100, 191):
        for n in range(N):
            for sb in range(K // 256):
                W, _ = O.q4_k_subblock_ints(w[r, sb], xq[n, sb * 256:(sb + 1) * 256])
                assert np.array_equal(dots[n, r, sb * 8:(sb + 1) * 8], W)


@pytest.mark.parametrize("shape", [(130, 2048), (192, 3072), (64, 8192), (4200, 3072)],
                         ids=["S8", "S12", "S8x4", "S12-ps2"])
@pytest.mark.parametrize("N", [1, 5, 9, 16])
def test_q4_k_wave_splits(ctx, shape, N):
    """Q4_K on 16-row tiles, one wave per super-block quad: 2 and 3 quads (4 waves, one round,
    a partial last tile), 8 quads (8 waves), and more tiles than CUs (4200 rows)."""
    import nanocamelid_amd as nc
    M, K = shape
    w = random_q4_k(M, K, seed=M + K + N)
    _, xq, xs = q8_activations(N, K, seed=300 + N)
    out, _ = _run_gemm(ctx, nc.NC_TYPE_Q4_K, w, M, K, xq, xs)
    ref = O.matmul_q4_k(xq, xs, w, N, M, K, nthreads=16)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("lanes", [1, 2, 3, 4])
def test_q4_k_pair_split_override_bit_exact(ctx, lanes, monkeypatch):
    """NC_Q4K_PS=<1..4>, the tuning override that runs plain 16-row-tile Q4_K matrices on the
    pair-split kernel with that many quad lanes (read at each launch): outputs bit-exact at the
    widths that kernel serves (1..9) on one quad of super-blocks, a partial last quad, a partial
    last tile and more tiles than CUs."""
    import nanocamelid_amd as nc
    monkeypatch.setenv("NC_Q4K_PS", str(lanes))
    for M, K in ((192, 1024), (130, 1280), (130, 2048), (4200, 3072)):
        w = random_q4_k(M, K, seed=M + K + lanes)
        for N in (1, 5, 9):
            _, xq, xs = q8_activations(N, K, seed=600 + N + lanes)
            out, _ = _run_gemm(ctx, nc.NC_TYPE_Q4_K, w, M, K, xq, xs)
            ref = O.matmul_q4_k(xq, xs, w, N, M, K, nthreads=16)
            assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), (M, K, N)


@pytest.mark.parametrize("shape", [(130, 1280), (16400, 1024)], ids=["r16k-partial-quad", "r64-large"])
@pytest.mark.parametrize("N", [1, 5, 16])
def test_q4_k_layouts(ctx, shape, N):
    """Q4_K matrices below 256 64-row tiles use 16-row tiles (4 super-blocks per wave
    instruction; 1280 columns leave the last quad one super-block); larger ones keep 64-row
    tiles.  Outputs and per-sub-block ints bit-exact either way."""
    import nanocamelid_amd as nc
    M, K = shape
    w = random_q4_k(M, K, seed=M + K + N)
    _, xq, xs = q8_activations(N, K, seed=400 + N)
    out, dots = _run_gemm(ctx, nc.NC_TYPE_Q4_K, w, M, K, xq, xs)
    ref = O.matmul_q4_k(xq, xs, w, N, M, K, nthreads=16)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    for r in (0, 15, 16, M - 1):
        for n in (0, N - 1):
            for sb in range(K // 256):
                W, _ = O.q4_k_subblock_ints(w[r, sb], xq[n, sb * 256:(sb + 1) * 256])
                assert np.array_equal(dots[n, r, sb * 8:(sb + 1) * 8], W)


@pytest.mark.parametrize("shape", [(130, 1024), (192, 4096), (4200, 96), (64, 32)],
                         ids=["partial-tile", "S8", "partial-group", "one-block"])
@pytest.mark.parametrize("N", [1, 5, 9, 16, 21])
def test_q8_0_bit_exact(ctx, shape, N):
    """Q8_0 matrices (matmul_q8_0_batch, inference.rs:1343-1383) on 64-row tiles with 1-8
    K-split waves, a partial last tile and a partial last group of 4 blocks; 21 tokens run as
    16-token slices.  Every output bit-identical to the oracle."""
    import nanocamelid_amd as nc
    M, K = shape
    w = random_q8_0(M, K, seed=M + K + N)
    _, xq, xs = q8_activations(N, K, seed=500 + N)
    q = nc.QMat(ctx, nc.NC_TYPE_Q8_0, M, K, w)
    out = nc.matmul_quantized_batch(ctx, q, torch.from_numpy(xq).cuda(), torch.from_numpy(xs).cuda())
    torch.cuda.synchronize()
    ref = O.matmul_q8_0(xq, xs, w, N, M, K, nthreads=16)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("shape", [(130, 1024), (64, 3072), (4200, 256), (192, 8192)],
                         ids=["partial-tile", "S12", "one-superblock", "S8x4"])
@pytest.mark.parametrize("N", [1, 5, 9, 16, 21])
def test_q5_k_bit_exact(ctx, shape, N):
    """Q5_K matrices (matmul_q5_k_batch's x86 path, inference.rs:2513-2640) on the 64-row
    K-quant kernel: one to many super-blocks per row, a partial last tile, 21 tokens as
    16-token slices.  Every output bit-identical to the oracle."""
    import nanocamelid_amd as nc
    M, K = shape
    w = random_q5_k(M, K, seed=M + K + N)
    _, xq, xs = q8_activations(N, K, seed=600 + N)
    q = nc.QMat(ctx, nc.NC_TYPE_Q5_K, M, K, w)
    out = nc.matmul_quantized_batch(ctx, q, torch.from_numpy(xq).cuda(), torch.from_numpy(xs).cuda())
    torch.cuda.synchronize()
    ref = O.matmul_q5_k(xq, xs, w, N, M, K, nthreads=16)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_quantize_q8_0_matches_oracle(ctx):
    import nanocamelid_amd as nc
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, (4, 4096)).astype(np.float32)
    x[0, :32] = 0.0                    # zero block
    x[1, :32] = np.arange(32) * 0.5   # exact .5 ties -> away from zero
    x[1, 31] = 127 * 0.5
    x[2, 64:96] = 1e-30                # tiny scale
    q, s = nc.quantize_f32_to_q8_0_batch(ctx, torch.from_numpy(x).cuda())
    q, s = q.cpu().numpy(), s.cpu().numpy()
    for n in range(4):
        rq, rs = O.quantize_q8_0(x[n])
        assert np.array_equal(q[n], rq)
        assert np.array_equal(s[n].view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("N", [1, 3, 5, 8, 9, 12, 16])
@pytest.mark.parametrize("shape", [(100, 416), (6144, 4096), (4096, 14336)], ids=["partial", "qkv", "down"])
def test_q4_0_mfma_path_bit_exact(shape, N):
    """The int8 MFMA dot path (nc_ctx_set_gemm_kernel(MFMA), the counterpart of the reference's
    Q8DotKernelSelector) gives the same bits as the oracle: partial tile and partial quad,
    K-split tiles, every MFMA token column count."""
    import nanocamelid_amd as nc
    mctx = nc.Context(0)
    mctx.set_gemm_kernel(nc._ffi.NC_GEMM_KERNEL_MFMA)
    M, K = shape
    w = random_q4_0(M, K, seed=3 * M + N)
    _, xq, xs = q8_activations(N, K, seed=5 * N + K)
    out, _ = _run_gemm(mctx, nc.NC_TYPE_Q4_0, w, M, K, xq, xs)
    assert np.array_equal(out.view(np.uint32), O.matmul_q4_0(xq, xs, w, N, M, K, nthreads=16).view(np.uint32))
