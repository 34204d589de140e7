"""Pins the CPU oracle's block formats and per-block arithmetic.

Each check is independent of the oracle's own code: the reference's known-answer
tests (values copied as data), IEEE half decoding by numpy over all 65536 codes,
brute-force dequantised references, closed forms, and inverse-formula round trips.
"""
import numpy as np
import pytest

from oracle import oracle as O


# ---------------------------------------------------------------- f16 (q8.rs:3599-3673)
def test_f16_known_answers():
    # q8.rs:5156-5164 f16_scale_decoder_covers_q8_scale_edges
    assert O.f16_to_f32(0x0000) == 0.0
    assert np.signbit(np.float32(O.f16_to_f32(0x8000)))
    assert O.f16_to_f32(0x3C00) == 1.0
    assert O.f16_to_f32(0xBC00) == -1.0
    assert O.f16_to_f32(0x0400) == np.float32(0.000061035156)
    assert O.f16_to_f32(0x7C00) == float("inf")
    # q8.rs:4486-4500 Q8_0 block scale 0x3800 decodes to 0.5
    assert O.f16_to_f32(0x3800) == 0.5


def test_f16_decode_exhaustive_against_ieee():
    codes = np.arange(65536, dtype=np.uint16)
    ref = codes.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(c)) for c in codes], np.float32)
    finite = ~np.isnan(ref)
    assert np.array_equal(ref[finite].view(np.uint32), got[finite].view(np.uint32))
    assert np.all(np.isnan(got[~finite]))


def test_f32_to_f16_trunc_known_answers():
    # q8.rs:5178-5195 fast_f32_to_f16_covers_representative_values
    cases = [(0.0, 0x0000), (-0.0, 0x8000), (1.0, 0x3C00), (-1.0, 0xBC00), (0.5, 0x3800),
             (2.0, 0x4000), (65504.0, 0x7BFF), (float("inf"), 0x7C00), (float("-inf"), 0xFC00)]
    for v, bits in cases:
        assert O.f32_to_f16_trunc(v) == bits, v
    nan_bits = O.f32_to_f16_trunc(float("nan"))
    assert nan_bits & 0x7C00 == 0x7C00 and nan_bits & 0x03FF != 0


def test_f32_to_f16_trunc_is_round_toward_zero():
    # Closed form: for normal-range values the truncating conversion equals IEEE
    # round-toward-zero, i.e. the largest-magnitude half not exceeding |x|.
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.normal(0, 0.02, 2000), rng.normal(0, 100, 2000)]).astype(np.float32)
    for x in xs:
        h = O.f32_to_f16_trunc(float(x))
        v = np.float32(np.uint16(h).view(np.float16))
        assert abs(v) <= abs(x)
        nxt = np.float32(np.uint16((h & 0x7FFF) + 1).view(np.float16))
        assert abs(x) < nxt
        assert (v == 0) or (np.signbit(v) == np.signbit(x))


# ---------------------------------------------------------------- int dots (q8.rs)
def test_dot_i8_known_answer():
    # q8.rs:4343-4348 scalar_dot_handles_signed_q8_values
    assert O.dot_i8([-3, -2, -1, 0, 1, 2, 3], [4, -5, 6, -7, 8, -9, 10]) == 12


def _unit(j):
    x = np.zeros(32, np.int8)
    x[j] = 1
    return x


def test_q4_0_nibble_order_known_answer():
    # q8.rs:4514-4530 q4_0_block_decodes_low_then_high_nibbles: byte idx = idx | (15-idx)<<4
    blk = np.zeros(18, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    for idx in range(16):
        blk[2 + idx] = idx | ((15 - idx) << 4)
    vals = [O.dot_q4_0_q8_0(blk, _unit(j)) for j in range(32)]
    assert vals[0] == -8 and vals[15] == 7 and vals[16] == 7 and vals[31] == -8
    # full element map from the same fixture: low nibbles then high nibbles
    assert vals == [i - 8 for i in range(16)] + [7 - i for i in range(16)]


def test_q4_0_dot_known_block_brute_force():
    # q8.rs:4533-4565 fixture block and activation idx-16
    blk = np.array([0x00, 0x3C, 0x80, 0x91, 0xA2, 0xB3, 0xC4, 0xD5, 0xE6, 0xF7, 0x08, 0x19, 0x2A,
                    0x3B, 0x4C, 0x5D, 0x6E, 0x7F], np.uint8)
    x = np.arange(32, dtype=np.int64) - 16
    lo = (blk[2:] & 0x0F).astype(np.int64) - 8
    hi = (blk[2:] >> 4).astype(np.int64) - 8
    expected = int(np.dot(np.concatenate([lo, hi]), x))
    assert O.dot_q4_0_q8_0(blk, x.astype(np.int8)) == expected


def test_q4_0_dot_extremes():
    # |dot| <= 32*8*127 = 32512: all nibbles 0 (value -8) against +127 and -127
    blk = np.zeros(18, np.uint8)
    assert O.dot_q4_0_q8_0(blk, np.full(32, 127, np.int8)) == -32512
    assert O.dot_q4_0_q8_0(blk, np.full(32, -127, np.int8)) == 32512
    blk[2:] = 0xFF  # value 7
    assert O.dot_q4_0_q8_0(blk, np.full(32, -128, np.int8)) == -7 * 128 * 32


# ---------------------------------------------------------------- activation quantiser
def test_quantize_q8_0_closed_forms():
    # scale = amax/127 (f32), q = round-half-away(x * (1/scale)), zero block -> zeros.
    x = np.zeros(64, np.float32)
    x[0] = 127.0
    x[1] = 2.5   # exact tie -> 3 (away from zero)
    x[2] = -2.5  # -> -3
    x[3] = 0.5   # -> 1
    x[4] = -0.49999997
    q, s = O.quantize_q8_0(x)
    assert s[0] == 1.0 and s[1] == 0.0
    assert list(q[:5]) == [127, 3, -3, 1, 0]
    assert np.all(q[32:] == 0)
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, 4096).astype(np.float32)
    q, s = O.quantize_q8_0(x)
    for b in range(128):
        chunk = x[b * 32:(b + 1) * 32]
        sc = np.float32(np.max(np.abs(chunk)) / np.float32(127.0))
        assert s[b] == sc
        inv = np.float32(1.0) / sc
        v = chunk * inv
        ref = np.clip(np.sign(v) * np.floor(np.abs(v) + 0.5), -127, 127)
        # floor(|v|+0.5) equals round-half-away except where |v|+0.5 rounds up in f32;
        # compare in float64 to stay exact.
        vd = v.astype(np.float64)
        ref = np.clip(np.sign(vd) * np.floor(np.abs(vd) + 0.5), -127, 127)
        assert np.array_equal(q[b * 32:(b + 1) * 32], ref.astype(np.int8))


# ---------------------------------------------------------------- matmul (inference.rs)
def q4_block(scale_bits, seed):
    # inference.rs:5477-5485 test fixture generator
    vals = []
    for idx in range(16):
        low = (seed + idx * 3) % 16
        high = (seed + (idx + 16) * 3) % 16
        vals.append(low | (high << 4))
    return np.array([scale_bits & 0xFF, scale_bits >> 8] + vals, np.uint8)


def _dequant_q4_0(blocks, M, K):
    blk = blocks.reshape(M, K // 32, 18)
    sc = blk[:, :, 0].astype(np.uint16) | (blk[:, :, 1].astype(np.uint16) << 8)
    scf = sc.view(np.float16).astype(np.float64)
    lo = (blk[:, :, 2:] & 0x0F).astype(np.float64) - 8
    hi = (blk[:, :, 2:] >> 4).astype(np.float64) - 8
    vals = np.concatenate([lo, hi], axis=2) * scf[:, :, None]
    return vals.reshape(M, K)


def test_matmul_q4_matches_dequantized_reference():
    # inference.rs:6027-6075 (rows 3, cols 64, tolerance 1e-5)
    rows, cols = 3, 64
    x = np.array([((i * 5) % 61) - 30 for i in range(cols)], np.int8)
    xs = np.array([0.25, 0.5], np.float32)
    w = np.concatenate([q4_block(b, s) for b, s in
                        [(0x3800, 1), (0x3C00, 2), (0x4000, 3), (0x4200, 4), (0x4400, 5), (0x4600, 6)]])
    got = O.matmul_q4_0(x, xs, w, 1, rows, cols)[0]
    deq = _dequant_q4_0(w, rows, cols)
    xf = x.astype(np.float64) * np.repeat(xs.astype(np.float64), 32)
    ref = deq @ xf
    assert np.all(np.abs(got - ref) < 1e-5)


def test_matmul_q4_0_random_vs_float64_and_blockdots():
    rng = np.random.default_rng(2)
    N, M, K = 3, 16, 256
    w = rng.integers(0, 256, M * (K // 32) * 18, dtype=np.uint8).reshape(M, K // 32, 18)
    scales = (rng.normal(0, 0.002, (M, K // 32)).astype(np.float16)).view(np.uint16)
    w[:, :, 0] = scales & 0xFF
    w[:, :, 1] = scales >> 8
    w = w.ravel()
    x = rng.integers(-127, 128, N * K, dtype=np.int8)
    xs = rng.uniform(0.001, 0.02, N * (K // 32)).astype(np.float32)
    got = O.matmul_q4_0(x, xs, w, N, M, K)
    dots = O.matmul_q4_0_blockdots(x, w, N, M, K)
    # int32 block dots against a numpy brute force
    blk = w.reshape(M, K // 32, 18)
    vals = np.concatenate([(blk[:, :, 2:] & 0x0F).astype(np.int64) - 8,
                           (blk[:, :, 2:] >> 4).astype(np.int64) - 8], axis=2)
    xb = x.reshape(N, K // 32, 32).astype(np.int64)
    ref_dots = np.einsum("mbj,nbj->nmb", vals, xb)
    assert np.array_equal(dots, ref_dots)
    # f32 sequential chain equals a float64 evaluation within f32 rounding noise
    ws = scales.view(np.float16).astype(np.float64)
    ref = np.einsum("mb,nb,nmb->nm", ws, xs.reshape(N, -1).astype(np.float64), ref_dots.astype(np.float64))
    assert np.allclose(got, ref, rtol=1e-4, atol=1e-6)
    # the oracle's order: sequential f32 over blocks of ((ws*xs)*dot)
    n, m = 1, 5
    acc = np.float32(0)
    for b in range(K // 32):
        acc = np.float32(acc + np.float32(np.float32(np.float32(ws[m, b]) * xs[n * (K // 32) + b]) * np.float32(ref_dots[n, m, b])))
    assert got[n, m] == acc


def k_scales(seed):
    # inference.rs:5519-5525
    return [((seed + idx * 5) % 64) for idx in range(12)]


def q4_k_block(scale_bits, min_bits, seed):
    # inference.rs:5565-5573
    vals = []
    for idx in range(128):
        low = (seed + idx * 3) % 16
        high = (seed + idx * 7) % 16
        vals.append(low | (high << 4))
    return np.array([scale_bits & 0xFF, scale_bits >> 8, min_bits & 0xFF, min_bits >> 8] + k_scales(seed) + vals,
                    np.uint8)


def test_matmul_q4_k_matches_dequantized_reference():
    # inference.rs:6516-6558 (rows 2, cols 512, tolerance 1e-4)
    rows, cols = 2, 512
    x = np.array([((i * 5) % 61) - 30 for i in range(cols)], np.int8)
    xs = np.array([0.125 + i * 0.03125 for i in range(cols // 32)], np.float32)
    w = np.concatenate([q4_k_block(0x3800, 0x3000, 1), q4_k_block(0x3C00, 0x3400, 2),
                        q4_k_block(0x4000, 0x3800, 3), q4_k_block(0x4200, 0x3A00, 4)])
    got = O.matmul_q4_k(x, xs, w, 1, rows, cols)[0]
    for r in range(rows):
        s = np.float32(0)
        for b in range(2):
            vals = O.q4_k_dequantize(w[(r * 2 + b) * 144:(r * 2 + b + 1) * 144])
            for i in range(256):
                xi = b * 256 + i
                s = np.float32(s + np.float32(np.float32(vals[i] * np.float32(x[xi])) * xs[xi // 32]))
        assert abs(got[r] - s) < 1e-4


def pack_q4_k_scales(sc, mn):
    """llama.cpp Q4_K 6-bit scale/min packing (the encoder side of get_scale_min_k4)."""
    q = [0] * 12
    for j in range(8):
        ls, lm = sc[j], mn[j]
        if j < 4:
            q[j] = ls
            q[j + 4] = lm
        else:
            q[j + 4] = (ls & 0x0F) | ((lm & 0x0F) << 4)
            q[j - 4] |= (ls >> 4) << 6
            q[j] |= (lm >> 4) << 6
    return q


def test_q4_k_scale_min_round_trip():
    # Encoder (above) and the oracle's decoder are inverse formulas: any index/shift slip fails.
    rng = np.random.default_rng(3)
    for _ in range(200):
        sc = [int(v) for v in rng.integers(0, 64, 8)]
        mn = [int(v) for v in rng.integers(0, 64, 8)]
        blk = np.zeros(144, np.uint8)
        blk[0:2] = [0x00, 0x3C]  # d = 1
        blk[2:4] = [0x00, 0x3C]  # dmin = 1
        blk[4:16] = pack_q4_k_scales(sc, mn)
        # qs: all nibbles 0 -> value = -mn_j ; nibble 1 -> sc_j - mn_j
        vals0 = O.q4_k_dequantize(blk)
        blk[16:] = 0x11
        vals1 = O.q4_k_dequantize(blk)
        for j in range(8):
            pair, half = divmod(j, 2)
            e = pair * 64 + half * 32
            assert vals0[e] == -mn[j]
            assert vals1[e] == sc[j] - mn[j]


def test_q4_k_element_order():
    # element map: pair p low nibble -> 64p + l, high nibble -> 64p + 32 + l
    blk = np.zeros(144, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[4:16] = pack_q4_k_scales([1] * 8, [0] * 8)
    for pos in [0, 5, 31, 32, 63, 64, 100, 255]:
        p, r = divmod(pos, 64)
        half, l = divmod(r, 32)
        b = blk.copy()
        b[16 + p * 32 + l] = (3 << 4) if half else 3
        v = O.q4_k_dequantize(b)
        assert v[pos] == 3 and np.count_nonzero(v) == 1


def test_q4_k_preloaded_fixture_matches_dequantized():
    # q8.rs:4708-4726 fixture; dot equals the f64 dequantised dot within f32 noise
    scales = [(idx * 7 + 11) % 64 for idx in range(12)]
    vals = [((idx * 3 + 5) % 16) | (((idx * 11 + 13) % 16) << 4) for idx in range(128)]
    blk = np.array([0x00, 0x3C, 0x00, 0x38] + scales + vals, np.uint8)
    x = np.array([((i * 13 + 17) % 127) - 63 for i in range(256)], np.int8)
    xs = np.array([0.015625 * (1 + (i % 5)) for i in range(8)], np.float32)
    got = O.matmul_q4_k(x, xs, blk, 1, 1, 256)[0, 0]
    deq = O.q4_k_dequantize(blk).astype(np.float64)
    ref = np.sum(deq * x.astype(np.float64) * np.repeat(xs.astype(np.float64), 32))
    assert abs(got - ref) <= 1e-4 * max(1.0, abs(ref))


# ---------------------------------------------------------------- tied head requantiser
def test_quantize_q4_0_tied_reconstructs_within_scale():
    # q8.rs:4187-4245 fixture and bound err <= |d| + 1e-4; zero block -> zeros
    rows, cols = 8, 64
    vals = np.zeros(rows * cols, np.float32)
    for row in range(rows):
        for col in range(cols):
            idx = row * cols + col
            block = col // 32
            if row == 0:
                vals[idx] = 0.0
            elif row == 1 and block == 0:
                vals[idx] = -12.5 if col == 0 else (0.25 * col if col % 2 == 0 else -0.125 * col)
            else:
                sign = 1.0 if (row + col) % 2 == 0 else -1.0
                vals[idx] = sign * (0.03 * idx + 0.5)
    blocks = O.quantize_q4_0_tied(vals, rows, cols).reshape(rows, 2, 18)
    for r in range(rows):
        for b in range(2):
            blk = blocks[r, b]
            d = O.f16_to_f32(int(blk[0]) | (int(blk[1]) << 8))
            rec = [O.dot_q4_0_q8_0(blk, _unit(j)) for j in range(32)]
            for kk in range(32):
                err = abs(rec[kk] * d - vals[r * cols + b * 32 + kk])
                assert err <= abs(d) + 1e-4
    assert O.f16_to_f32(int(blocks[0, 0, 0]) | (int(blocks[0, 0, 1]) << 8)) == 0.0
    assert all(O.dot_q4_0_q8_0(blocks[0, 0], _unit(j)) == 0 for j in range(32))


def test_quantize_q4_0_tied_closed_form():
    # d = max/-8 (signed max of the first |max| element), nibble = clamp(trunc(x/d + 8.5), 0, 15)
    vals = np.linspace(-1.0, 0.5, 32).astype(np.float32)
    blk = O.quantize_q4_0_tied(vals, 1, 32)
    d = O.f16_to_f32(int(blk[0]) | (int(blk[1]) << 8))
    assert d == O.f16_to_f32(O.f32_to_f16_trunc(np.float32(-1.0) / np.float32(-8.0)))
    nib = [O.dot_q4_0_q8_0(blk, _unit(j)) + 8 for j in range(32)]
    assert nib[0] == 0  # x = -1 -> -1 * (1/0.125) + 8.5 = 0.5 -> 0
    assert max(nib) <= 15 and min(nib) >= 0


def q6_k_block(scale_bits, seed):
    """inference.rs:5589-5603 q6_k_block fixture."""
    ql = [(seed + i * 5) % 256 for i in range(128)]
    qh = [(seed + i * 7) % 256 for i in range(64)]
    sc = [((seed + i * 3) % 15) - 7 for i in range(16)]
    return np.array(ql + qh + [s & 0xFF for s in sc] + [scale_bits & 0xFF, scale_bits >> 8], np.uint8)


def test_matmul_q6_k_matches_dequantized_reference():
    # inference.rs:6605-6640 (rows 2, cols 512, tolerance 1e-4); the dequantised values come from
    # the oracle's load_f32_or_f16 restatement, itself pinned by the reference's Q6_K known answers
    rows, cols = 2, 512
    x = np.array([((i * 5) % 61) - 30 for i in range(cols)], np.int8)
    xs = np.array([0.125 + i * 0.03125 for i in range(cols // 32)], np.float32)
    w = np.concatenate([q6_k_block(0x3800, 1), q6_k_block(0x3C00, 2), q6_k_block(0x4000, 3), q6_k_block(0x4200, 4)])
    got = O.matmul_q6_k(x, xs, w, 1, rows, cols)[0]
    for r in range(rows):
        s = np.float32(0)
        for b in range(2):
            vals = O.dequantize_f32(14, w[(r * 2 + b) * 210:(r * 2 + b + 1) * 210], 256)
            for i in range(256):
                xi = b * 256 + i
                s = np.float32(s + np.float32(np.float32(vals[i] * np.float32(x[xi])) * xs[xi // 32]))
        assert abs(got[r] - s) < 1e-4


def test_q6_k_dot_float64_and_term_order():
    # the dot against a float64 evaluation of sum(d * sc * q * x * xs) over the block, and the
    # reference's term order: one term moved to the front of the chain changes nothing only if
    # the chain is the same multiset -- so check that the f32 result equals a float32 left-to-right
    # sum in the order (half, l, k), and differs in general from the order (half, k, l)
    rng = np.random.default_rng(14)
    blk = q6_k_block(0x2E66, 9)
    x = rng.integers(-127, 128, 256).astype(np.int8)
    xs = rng.uniform(0.01, 0.05, 8).astype(np.float32)
    got = O.q6_k_dot(blk, x, xs)
    vals = O.dequantize_f32(14, blk, 256).astype(np.float64)
    exact = float(np.sum(vals * x.astype(np.float64) * np.repeat(xs.astype(np.float64), 32)))
    assert abs(got - exact) <= 1e-5 * max(1.0, abs(exact))
    d = np.float32(O.f16_to_f32(0x2E66))
    sc = blk[192:208].view(np.int8)
    ql, qh = blk[:128].astype(int), blk[128:192].astype(int)

    def chain(order):
        s = np.float32(0)
        for half, l, k in order:
            lo, hi, hb = ql[64 * half + l], ql[64 * half + l + 32], qh[32 * half + l]
            q = [(lo & 15) | ((hb & 3) << 4), (hi & 15) | (((hb >> 2) & 3) << 4),
                 (lo >> 4) | (((hb >> 4) & 3) << 4), (hi >> 4) | (((hb >> 6) & 3) << 4)][k] - 32
            g = 8 * half + 2 * k + (l >= 16)
            c = np.float32(np.float32(d * np.float32(sc[g])) * xs[4 * half + k])
            s = np.float32(s + np.float32(np.float32(c * np.float32(q)) * np.float32(x[128 * half + 32 * k + l])))
        return s

    ref_order = [(h, l, k) for h in range(2) for l in range(32) for k in range(4)]
    assert np.float32(got) == chain(ref_order)
    # the check is order-sensitive: the (half, k, l) order rounds differently for some inputs
    other = [(h, l, k) for h in range(2) for k in range(4) for l in range(32)]
    differs = False
    for seed in range(20):
        x = np.random.default_rng(seed).integers(-127, 128, 256).astype(np.int8)
        assert np.float32(O.q6_k_dot(blk, x, xs)) == chain(ref_order)
        differs |= bool(chain(other) != chain(ref_order))
    assert differs


# ---------------------------------------------------------------- Q8_0 matrices (inference.rs:1343-1383)
def q8_block(scale_bits, vals):
    return np.concatenate([np.array([scale_bits & 0xFF, scale_bits >> 8], np.uint8),
                           np.asarray(vals, np.int8).view(np.uint8)])


def test_matmul_q8_0_block_dot_known_answer():
    # q8.rs:5050-5058: a [2]*32 block scaled 2.0 against [-3]*32 scaled 0.5: dot -192, -192.0
    w = q8_block(0x4000, [2] * 32)
    x = np.full(32, -3, np.int8)
    out = O.matmul_q8_0(x, np.array([0.5], np.float32), w, 1, 1, 32)
    assert out[0, 0] == np.float32(-192.0)


def test_matmul_q8_0_reference_fixture_vs_float64():
    # the fixture of inference.rs:6815-6860 (q8_block helper :5399-5405): 3 tokens x 3 rows x 64
    N, M, K = 3, 3, 64
    x = np.array([((i * 5) % 61) - 30 for i in range(N * K)], np.int8)
    xs = np.array([0.125 + i * 0.03125 for i in range(N * (K // 32))], np.float32)
    blocks = []
    for idx in range(M * (K // 32)):
        seed = idx + 1
        blocks.append(q8_block(0x3800 + idx, [((seed + j * 7) % 63) - 31 for j in range(32)]))
    w = np.concatenate(blocks)
    got = O.matmul_q8_0(x, xs, w, N, M, K)
    blk = w.reshape(M, K // 32, 34)
    ws = blk[:, :, :2].copy().view(np.float16)[:, :, 0].astype(np.float64)
    q = blk[:, :, 2:].copy().view(np.int8).astype(np.float64)
    deq = (q * ws[:, :, None]).reshape(M, K)
    xf = x.reshape(N, K).astype(np.float64) * np.repeat(xs.reshape(N, -1).astype(np.float64), 32, axis=1)
    ref = xf @ deq.T
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-6)
    # batch rows equal single-token calls (the fixture's own assertion)
    for n in range(N):
        one = O.matmul_q8_0(x[n * K:(n + 1) * K], xs[n * 2:(n + 1) * 2], w, 1, M, K)[0]
        assert np.array_equal(one, got[n])


def test_matmul_q8_0_left_to_right_order():
    # terms 2^24, 1, -2^24 in block order: left to right gives 0 (2^24 + 1 rounds back to
    # 2^24), any other grouping or the float64 sum gives 1
    w = np.concatenate([q8_block(0x6400, [1] * 32), q8_block(0x3C00, [1] * 32), q8_block(0x6400, [-1] * 32)])
    x = np.concatenate([np.full(32, 32, np.int8), np.full(32, 1, np.int8), np.full(32, 32, np.int8)])
    xs = np.array([16.0, 0.03125, 16.0], np.float32)
    out = O.matmul_q8_0(x, xs, w, 1, 1, 96)
    assert out[0, 0] == np.float32(0.0)


def test_matmul_q8_0_random_vs_float64():
    rng = np.random.default_rng(8)
    N, M, K = 4, 24, 512
    blk = rng.integers(-128, 128, (M, K // 32, 34), dtype=np.int16).astype(np.int8).view(np.uint8)
    scales = rng.uniform(0.0005, 0.004, (M, K // 32)).astype(np.float16).view(np.uint16)
    blk[:, :, 0] = scales & 0xFF
    blk[:, :, 1] = scales >> 8
    x = rng.integers(-127, 128, N * K, dtype=np.int8)
    xs = rng.uniform(0.001, 0.02, N * (K // 32)).astype(np.float32)
    got = O.matmul_q8_0(x, xs, blk.ravel(), N, M, K)
    q = blk[:, :, 2:].copy().view(np.int8).astype(np.int64)
    dots = np.einsum("mbj,nbj->nmb", q, x.reshape(N, K // 32, 32).astype(np.int64))
    ref = np.einsum("mb,nb,nmb->nm", scales.view(np.float16).astype(np.float64),
                    xs.reshape(N, -1).astype(np.float64), dots.astype(np.float64))
    assert np.allclose(got, ref, rtol=1e-4, atol=1e-6)


# ---------------------------------------------------------------- Q5_K matrices (inference.rs:2513-2640)
def q5_k_block(scale_bits, min_bits, seed):
    # inference.rs:5575-5587 (k_scales :5519-5525)
    high = [((seed + i * 11) % 256) for i in range(32)]
    vals = [((seed + i * 3) % 16) | (((seed + i * 5) % 16) << 4) for i in range(128)]
    return np.array([scale_bits & 0xFF, scale_bits >> 8, min_bits & 0xFF, min_bits >> 8] + k_scales(seed) + high + vals,
                    np.uint8)


def _dequant_q5_k_f64(blk):
    # GGML Q5_K: value = d * sc_j * q5 - dmin * mn_j, q5 = nibble + 16 * (qh bit), sub-block j
    d = float(np.frombuffer(blk[0:2].tobytes(), np.float16)[0])
    dmin = float(np.frombuffer(blk[2:4].tobytes(), np.float16)[0])
    sc = blk[4:16]
    qh = blk[16:48]
    qs = blk[48:176]
    out = np.zeros(256)
    for j in range(8):
        if j < 4:
            s, m = sc[j] & 63, sc[j + 4] & 63
        else:
            s = (sc[j + 4] & 0x0F) | ((sc[j - 4] >> 6) << 4)
            m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4)
        pair, half = j // 2, j % 2
        for l in range(32):
            q = ((qs[pair * 32 + l] >> (4 * half)) & 0x0F) + (16 if (qh[l] >> j) & 1 else 0)
            out[pair * 64 + 32 * half + l] = d * s * q - dmin * m
    return out


def test_matmul_q5_k_matches_dequantized_reference():
    # inference.rs:6561-6603: rows 2, cols 512, four fixture blocks, tolerance 1e-4
    rows, cols = 2, 512
    x = np.array([((i * 5) % 61) - 30 for i in range(cols)], np.int8)
    xs = np.array([0.125 + i * 0.03125 for i in range(cols // 32)], np.float32)
    w = np.concatenate([q5_k_block(0x3800, 0x3000, 1), q5_k_block(0x3C00, 0x3400, 2),
                        q5_k_block(0x4000, 0x3800, 3), q5_k_block(0x4200, 0x3A00, 4)])
    got = O.matmul_q5_k(x, xs, w, 1, rows, cols)[0]
    deq = np.stack([np.concatenate([_dequant_q5_k_f64(w[(r * 2 + b) * 176:(r * 2 + b + 1) * 176]) for b in range(2)])
                    for r in range(rows)])
    ref = deq @ (x.astype(np.float64) * np.repeat(xs.astype(np.float64), 32))
    assert np.all(np.abs(got - ref) < 1e-4)
    # the high bit matters: the same blocks with qh cleared give a different product
    w0 = w.copy().reshape(4, 176)
    w0[:, 16:48] = 0
    assert not np.allclose(O.matmul_q5_k(x, xs, w0.ravel(), 1, rows, cols)[0], got)


def test_matmul_q5_k_batch_and_float64():
    # inference.rs:7329-7375 fixture (3 tokens x 2 rows x 512): batch rows equal single calls;
    # random blocks against a float64 decode
    N, rows, cols = 3, 2, 512
    x = np.array([((i * 5) % 61) - 30 for i in range(N * cols)], np.int8)
    xs = np.array([0.125 + i * 0.03125 for i in range(N * (cols // 32))], np.float32)
    w = np.concatenate([q5_k_block(0x3800 + i, 0x3000 + i, i + 1) for i in range(rows * 2)])
    got = O.matmul_q5_k(x, xs, w, N, rows, cols)
    for n in range(N):
        one = O.matmul_q5_k(x[n * cols:(n + 1) * cols], xs[n * 16:(n + 1) * 16], w, 1, rows, cols)[0]
        assert np.array_equal(one, got[n])
    rng = np.random.default_rng(13)
    M, K = 6, 768
    blk = rng.integers(0, 256, (M, K // 256, 176), dtype=np.uint8)
    for o in (0, 2):
        v = rng.uniform(1e-4, 4e-4, (M, K // 256)).astype(np.float16).view(np.uint16)
        blk[:, :, o], blk[:, :, o + 1] = v & 0xFF, v >> 8
    xr = rng.integers(-127, 128, 2 * K, dtype=np.int8)
    xsr = rng.uniform(0.001, 0.02, 2 * (K // 32)).astype(np.float32)
    got = O.matmul_q5_k(xr, xsr, blk.ravel(), 2, M, K)
    deq = np.stack([np.concatenate([_dequant_q5_k_f64(blk[r, b]) for b in range(K // 256)]) for r in range(M)])
    xf = xr.reshape(2, K).astype(np.float64) * np.repeat(xsr.reshape(2, -1).astype(np.float64), 32, axis=1)
    assert np.allclose(got, xf @ deq.T, rtol=1e-4, atol=1e-6)
