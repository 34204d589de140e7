"""Shared helpers for the GPU parity tests (data generation on the host)."""
import numpy as np


def quantize_q4_0_rows(W: np.ndarray) -> np.ndarray:
    """llama.cpp-style Q4_0 of a float32 [M, K] matrix -> GGUF blocks [M, K/32, 18]."""
    M, K = W.shape
    B = W.reshape(M, K // 32, 32).astype(np.float32)
    idx = np.argmax(np.abs(B), axis=2)
    mx = np.take_along_axis(B, idx[..., None], 2)[..., 0]
    d = (mx / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    q = np.minimum(np.trunc(B * inv[..., None] + np.float32(8.5)), 15).astype(np.uint8)
    out = np.zeros((M, K // 32, 18), np.uint8)
    dh = d.astype(np.float16).view(np.uint16)
    out[:, :, 0] = dh & 0xFF
    out[:, :, 1] = dh >> 8
    out[:, :, 2:] = q[:, :, :16] | (q[:, :, 16:] << 4)
    return out


def random_q4_0(M, K, seed, std=0.02):
    rng = np.random.default_rng(seed)
    return quantize_q4_0_rows(rng.normal(0, std, (M, K)).astype(np.float32))


def random_q4_k(M, K, seed):
    """Random valid Q4_K super-blocks [M, K/256, 144] (scales 6-bit, d/dmin small f16)."""
    rng = np.random.default_rng(seed)
    out = rng.integers(0, 256, (M, K // 256, 144), dtype=np.uint8)
    d = rng.uniform(1e-4, 4e-4, (M, K // 256)).astype(np.float16).view(np.uint16)
    dm = rng.uniform(1e-4, 4e-4, (M, K // 256)).astype(np.float16).view(np.uint16)
    out[:, :, 0] = d & 0xFF
    out[:, :, 1] = d >> 8
    out[:, :, 2] = dm & 0xFF
    out[:, :, 3] = dm >> 8
    return out


def random_q5_k(M, K, seed):
    """Random valid Q5_K super-blocks [M, K/256, 176] (any qh / nibble bytes, small d/dmin)."""
    rng = np.random.default_rng(seed)
    out = rng.integers(0, 256, (M, K // 256, 176), dtype=np.uint8)
    for o in (0, 2):
        v = rng.uniform(1e-4, 4e-4, (M, K // 256)).astype(np.float16).view(np.uint16)
        out[:, :, o] = v & 0xFF
        out[:, :, o + 1] = v >> 8
    return out


def random_q8_0(M, K, seed):
    """Random Q8_0 blocks [M, K/32, 34]: int8 values over the full range, small f16 scales."""
    rng = np.random.default_rng(seed)
    out = rng.integers(-128, 128, (M, K // 32, 34), dtype=np.int16).astype(np.int8).view(np.uint8)
    d = rng.uniform(5e-4, 4e-3, (M, K // 32)).astype(np.float16).view(np.uint16)
    out[:, :, 0] = d & 0xFF
    out[:, :, 1] = d >> 8
    return out


def q8_activations(N, K, seed):
    from oracle import oracle as O
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1, (N, K)).astype(np.float32)
    q, s = O.quantize_q8_0(x.ravel())
    return x, q.reshape(N, K), s.reshape(N, K // 32)
