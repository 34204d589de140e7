"""GPU parity of the fused RMSNorm + Q8_0 kernel against the CPU oracle.

The kernel evaluates the reference's sequential f32 sum of squares (inference.rs:697-706)
with a parallel method that is verified step by step against the recurrence, so its output
must be bit-identical to the sequential loop for every input.  Rows here are chosen to hit
each branch of that method: smooth data, binade-dense starts, exact ties (including more
ties than the method's list holds, which forces the sequential fallback), subnormal squares,
zero rows and leading zeros, a huge dynamic range (inexact double prefix), and heavy tails.
"""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

EPS = 1e-5


@pytest.fixture(scope="module")
def ctx():
    import nanocamelid_amd as nc
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    return nc.Context(0)


def _rows(d, rng):
    rows = {
        "normal": rng.normal(0, 1, d),
        "small": rng.normal(0, 0.02, d),
        "t3": rng.standard_t(3, d),
        "cauchy": rng.standard_cauchy(d),
        "spiky": rng.normal(0, 0.02, d) * rng.choice([1.0, 40.0], d, p=[0.99, 0.01]),
        "zeros": np.zeros(d),
        "leading_zeros": np.concatenate([np.zeros(d // 3), rng.normal(0, 1, d - d // 3)]),
        "subnormal_squares": rng.normal(0, 1e-21, d) * rng.choice([1.0, 1e20], d, p=[0.9, 0.1]),
        "tiny_first": np.concatenate([[1e-17], rng.normal(0, 3, d - 1)]),
        "growing": rng.normal(0, 1, d) * np.linspace(1e-3, 10, d),
    }
    # 2^24 then ones: every later step is an exact tie (2^24 + 1 rounds to even)
    ties = np.ones(d)
    ties[0] = 4096.0
    rows["ties_all"] = ties
    # a few dozen ties inside otherwise smooth data
    few = rng.normal(0, 1, d)
    few[0] = 4096.0
    few[1:40] = 1.0
    rows["ties_few"] = few
    return {k: v.astype(np.float32) for k, v in rows.items()}


@pytest.mark.parametrize("d", [256, 512, 768, 1024, 1536, 2048, 3072, 4096, 5120, 6144, 8192])
def test_rms_norm_q8_bit_exact(ctx, d):
    import nanocamelid_amd as nc
    rng = np.random.default_rng(d)
    rows = _rows(d, rng)
    names = list(rows)
    w = rng.normal(1.0, 0.1, d).astype(np.float32)
    for i0 in range(0, len(names), 16):
        chunk = names[i0:i0 + 16]
        x = np.stack([rows[k] for k in chunk])
        print(f"rmsnorm d={d} rows {chunk}", flush=True)
        q, s = nc.rms_norm_q8_0_batch(ctx, torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), EPS)
        torch.cuda.synchronize()
        q, s = q.cpu().numpy(), s.cpu().numpy()
        for r, name in enumerate(chunk):
            y = O.rms_norm(x[r], w, EPS)
            qo, so = O.quantize_q8_0(y)
            assert np.array_equal(s[r].view(np.uint32), so.view(np.uint32)), f"{name} d={d}: scales differ"
            assert np.array_equal(q[r], qo), f"{name} d={d}: int8 values differ"


def test_rms_norm_rejects_unsupported_width(ctx):
    import nanocamelid_amd as nc
    x = torch.zeros((1, 320), dtype=torch.float32, device="cuda")
    w = torch.ones(320, dtype=torch.float32, device="cuda")
    with pytest.raises(nc.NcError):
        nc.rms_norm_q8_0_batch(ctx, x, w, EPS)
