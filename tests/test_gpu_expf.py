"""The device's expf (a restatement of glibc's, used by the softmax, SwiGLU and temperature
kernels) against the host's glibc expf, which Rust's f32::exp calls (inference.rs:3522-3540,
:3367-3390): every one of the 2^32 float inputs, bit for bit (NaN inputs: a NaN)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O


def test_expf_checker_counts_planted_mismatches():
    # CPU: the checker itself, on glibc's own values with two planted one-ulp changes
    first = 0x3F000000  # 0.5 and up
    vals = np.array([O.expf(np.uint32(first + i).view(np.float32)) for i in range(4096)], np.float32)
    assert O.expf_mismatches(first, vals) == (0, 0)
    bad = vals.copy()
    bad[[17, 4000]] = np.nextafter(bad[[17, 4000]], np.float32(np.inf))
    assert O.expf_mismatches(first, bad) == (2, first + 17)


@pytest.fixture(scope="module")
def ctx():
    import nanocamelid_amd as nc
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    return nc.Context(0)


@pytest.mark.gpu
def test_device_expf_all_inputs(ctx):
    import nanocamelid_amd as nc
    chunk = 1 << 27
    out = torch.empty(chunk, dtype=torch.float32, device="cuda")
    host = torch.empty(chunk, dtype=torch.float32, pin_memory=True)
    total = 0
    for c in range((1 << 32) // chunk):
        first = c * chunk
        nc.check(nc.lib().nc_debug_expf(ctx.h, first, chunk, out.data_ptr(), torch.cuda.current_stream().cuda_stream))
        host.copy_(out)
        n, fb = O.expf_mismatches(first, host.numpy(), nthreads=16)
        assert n == 0, f"{n} mismatches in [{first:#x}, {first + chunk:#x}), first at input bits {fb:#010x}"
        total += chunk
    assert total == 1 << 32
