"""The allocation-free matmul entry point (nc_matmul_quantized_batch_noalloc) against the
allocating one, through the C ABI: two calls in a row, the second smaller, bit-identical."""
import ctypes as C

import numpy as np
import pytest

from tests.gpu_util import q8_activations, random_q4_0

torch = pytest.importorskip("torch")


@pytest.mark.gpu
def test_noalloc_matmul_matches_allocating_entry():
    import nanocamelid_amd as nc
    from nanocamelid_amd._ffi import NC_ERANGE, NcError, check, lib
    ctx = nc.Context(0)
    for M, K, N in ((4096, 14336, 9), (1024, 4096, 3)):  # the second call is smaller
        print(f"noalloc matmul {M}x{K} N={N}", flush=True)
        w = nc.QMat(ctx, nc.NC_TYPE_Q4_0, M, K, random_q4_0(M, K, seed=M + N))
        _, q, s = q8_activations(N, K, seed=N)
        xq = torch.from_numpy(q).cuda()
        xs = torch.from_numpy(s).cuda()
        ref = nc.matmul_quantized_batch(ctx, w, xq, xs)
        out = torch.full((N, M), float("nan"), dtype=torch.float32, device="cuda")
        stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        check(lib().nc_matmul_quantized_batch_noalloc(ctx.h, w.h, xq.data_ptr(), xs.data_ptr(), out.data_ptr(), N, M,
                                                       K, stream))
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.cpu().numpy().view(np.uint32)), (M, K, N)
    # beyond the static scratch: refused before any launch
    big = nc.QMat(ctx, nc.NC_TYPE_Q4_0, 16, 131072, random_q4_0(16, 131072, seed=1))
    xq = torch.zeros((16, 131072), dtype=torch.int8, device="cuda")
    xs = torch.zeros((16, 4096), dtype=torch.float32, device="cuda")
    out = torch.empty((16, 16), dtype=torch.float32, device="cuda")
    rc = lib().nc_matmul_quantized_batch_noalloc(ctx.h, big.h, xq.data_ptr(), xs.data_ptr(), out.data_ptr(), 16, 16,
                                                 131072, None)
    assert rc == NC_ERANGE
