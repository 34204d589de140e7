"""Pins the CPU oracle's row ops, Philox and the attention head.

Checks: reference closed-form RoPE tests (inference.rs:7423-7468), published Philox
known-answer vectors, float64 brute force for attention/softmax/norm, and the
first-max-wins argmax rule.
"""
import math

import numpy as np

from oracle import oracle as O


def test_rms_norm_closed_form():
    x = np.array([3.0, 4.0], np.float32)
    w = np.array([1.0, 2.0], np.float32)
    out = O.rms_norm(x, w, 0.0)
    # mean square = 12.5 -> scale = 1/sqrt(12.5)
    s = np.float32(1.0) / np.sqrt(np.float32(12.5))
    assert out[0] == np.float32(np.float32(3.0) * s) * np.float32(1.0)
    assert out[1] == np.float32(np.float32(4.0) * s) * np.float32(2.0)
    rng = np.random.default_rng(0)
    x = rng.normal(0, 1, 2048).astype(np.float32)
    w = rng.normal(1, 0.1, 2048).astype(np.float32)
    out = O.rms_norm(x, w, 1e-5)
    ref = x.astype(np.float64) / math.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5) * w
    assert np.allclose(out, ref, rtol=1e-5, atol=1e-6)


def test_rope_partial_dimension_known_answer():
    # inference.rs:7423-7440: pos 1, head_dim 4, rope_dim 2, base 1e4: (1,0) -> (cos 1, sin 1)
    d = O.rope(np.array([1.0, 0.0, 10.0, 20.0], np.float32), 1, 1, 4, 2, 10000.0, 0)
    assert abs(d[0] - math.cos(1.0)) < 1e-6 and abs(d[1] - math.sin(1.0)) < 1e-6
    assert d[2] == 10.0 and d[3] == 20.0


def test_rope_neox_pairs_known_answer():
    # inference.rs:7443-7468
    d = O.rope(np.array([1.0, 2.0, 3.0, 4.0], np.float32), 1, 1, 4, 4, 10000.0, 1)
    t0, t1 = 1.0, 10000.0 ** (-2.0 / 4.0)
    s0, c0, s1, c1 = math.sin(t0), math.cos(t0), math.sin(t1), math.cos(t1)
    assert abs(d[0] - (1 * c0 - 3 * s0)) < 1e-5 and abs(d[2] - (1 * s0 + 3 * c0)) < 1e-5
    assert abs(d[1] - (2 * c1 - 4 * s1)) < 1e-5 and abs(d[3] - (2 * s1 + 4 * c1)) < 1e-5
    norm = O.rope(np.array([1.0, 2.0, 3.0, 4.0], np.float32), 3, 1, 4, 4, 10000.0, 0)
    neox = O.rope(np.array([1.0, 2.0, 3.0, 4.0], np.float32), 3, 1, 4, 4, 10000.0, 1)
    assert not np.array_equal(norm, neox)


def test_rope_norm_matches_float64_rotation():
    hd, pos, base = 64, 37, 500000.0
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, 2 * hd).astype(np.float32)
    got = O.rope(x, pos, 2, hd, hd, base, 0)
    for h in range(2):
        for i in range(hd // 2):
            th = base ** (-(2.0 * i) / hd)
            a = pos * th
            x0, x1 = float(x[h * hd + 2 * i]), float(x[h * hd + 2 * i + 1])
            assert abs(got[h * hd + 2 * i] - (x0 * math.cos(a) - x1 * math.sin(a))) < 2e-4
            assert abs(got[h * hd + 2 * i + 1] - (x0 * math.sin(a) + x1 * math.cos(a))) < 2e-4


def test_softmax_and_expf():
    x = np.array([1.0, 2.0, 3.0, -1.0], np.float32)
    p = O.softmax(x)
    e = np.exp(x.astype(np.float64) - 3.0)
    assert np.allclose(p, e / e.sum(), rtol=1e-6)
    assert O.expf(0.0) == 1.0 and O.expf(-float("inf")) == 0.0
    assert abs(O.expf(1.0) - math.e) < 3e-7


def test_silu_mul_closed_form():
    g = np.array([0.0, 1.0, -2.0, 30.0, -120.0], np.float32)
    u = np.array([5.0, 2.0, 1.0, 1.0, 1.0], np.float32)
    out = O.silu_mul(g, u)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert out[0] == 0.0
    assert np.allclose(out, ref, rtol=1e-6, atol=1e-30)


def test_argmax_first_max_wins():
    # inference.rs:4836-4846 strict '>' keeps the earliest maximum
    assert O.argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert O.argmax([5.0, 5.0]) == 0
    assert O.argmax([-1.0, -0.5, -0.5]) == 1


def test_attention_head_brute_force():
    rng = np.random.default_rng(2)
    hd, kvw, pos = 8, 16, 6
    k = rng.normal(0, 1, (pos + 1, kvw)).astype(np.float32)
    v = rng.normal(0, 1, (pos + 1, kvw)).astype(np.float32)
    q = rng.normal(0, 1, hd).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    for kvh in range(2):
        got = O.attention_head(q, k, v, pos, kvw, kvh, hd, float(scale))
        kk = k[:, kvh * hd:(kvh + 1) * hd].astype(np.float64)
        vv = v[:, kvh * hd:(kvh + 1) * hd].astype(np.float64)
        s = kk @ q.astype(np.float64) * float(scale)
        p = np.exp(s - s.max())
        p /= p.sum()
        assert np.allclose(got, p @ vv, rtol=1e-5, atol=1e-6)


def test_philox4x32_10_known_answers():
    # Random123 / SC'11 known-answer vectors for philox4x32 with 10 rounds.
    kat = [
        ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
        ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
        ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
         [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
    ]
    for ctr, key, out in kat:
        assert list(O.philox4x32_10(ctr, key)) == out


def test_uniform_prompt_and_oracle_drafter():
    ids = O.uniform_prompt(1234, 4096, 128256)
    assert ids.max() < 128256 and len(set(ids.tolist())) > 4000
    assert np.array_equal(ids, O.uniform_prompt(1234, 4096, 128256))
    greedy = np.arange(100, 200, dtype=np.uint32)
    hits = [O.oracle_draft(7, 32 + i, 0.8, greedy, 32, 128256) == greedy[i] for i in range(100)]
    assert 60 <= sum(hits) <= 95  # ~alpha of the drafts copy the greedy stream
    assert all(O.oracle_draft(7, 32 + i, 1.0, greedy, 32, 128256) == greedy[i] for i in range(100))


def test_inverse_cdf_and_temperature_probs():
    p = np.array([0.0, 0.25, 0.0, 0.75], np.float32)
    assert O.sample_inverse_cdf(p, 0.0) == 1
    assert O.sample_inverse_cdf(p, 0.2) == 1
    assert O.sample_inverse_cdf(p, 0.3) == 3
    assert O.sample_inverse_cdf(p, 0.999) == 3
    lg = np.array([1.0, 2.0, 0.5], np.float32)
    pr = O.temperature_probs(lg, 1.0)
    e = np.exp(lg.astype(np.float64) - 2.0)
    assert np.allclose(pr, e / e.sum(), rtol=1e-6)


def test_fixed_point_sampler_boundaries():
    # weights 1:2:3:4 (exact in 2^-40 fixed point): u in [0, .1) -> 0, [.1, .3) -> 1,
    # [.3, .6) -> 2, [.6, 1) -> 3; u = k/2^24 on either side of each boundary
    w = np.array([1, 2, 3, 4], np.float32) / np.float32(16)
    for lo, hi, idx in ((0.0, 0.1, 0), (0.1, 0.3, 1), (0.3, 0.6, 2), (0.6, 1.0, 3)):
        first = int(np.ceil(lo * 2**24))
        last = int(np.ceil(hi * 2**24)) - 1
        assert O.sample_inverse_cdf(w, np.float32(first / 2**24)) == idx, (lo, idx)
        assert O.sample_inverse_cdf(w, np.float32(last / 2**24)) == idx, (hi, idx)
    # weights below 2^-40 carry no mass; zero-mass ids are never returned
    w2 = np.array([1e-13, 0.5, 0.0, 1e-13, 0.5], np.float32)
    got = {O.sample_inverse_cdf(w2, np.float32(k / 64)) for k in range(64)}
    assert got == {1, 4}
    # mass is additive: a distribution split across duplicated ids samples the same ranges
    rng = np.random.default_rng(3)
    v = rng.random(50).astype(np.float32)
    v /= v.sum()
    us = rng.integers(0, 2**24, 300) / 2**24
    for u in us:
        i = O.sample_inverse_cdf(v, np.float32(u))
        assert v[i] > 0
        cum = np.cumsum(np.floor(v.astype(np.float64) * 2**40))
        # the chosen id's fixed-point interval contains u * total (integer arithmetic)
        target = (int(u * 2**24) * int(cum[-1])) >> 24
        assert (cum[i - 1] if i else 0) <= target < cum[i]


def test_speculative_sampling_preserves_target_distribution():
    # The defining property of speculative sampling: whatever the draft distribution q,
    # the first emitted token (the draft if accepted, else the residual resample) is
    # distributed as p.  Chi-square over 20000 seeds on a 6-token vocabulary.
    from scipy.stats import chisquare
    V, N = 6, 20000
    p_logits = np.array([[0.3, -1.0, 1.2, 0.0, -0.4, 0.8], [0.0] * 6], np.float32)
    q = O.temperature_probs(np.array([1.5, 0.2, -0.5, 0.9, 0.0, -1.2], np.float32), 1.0)[None, :]
    p0 = O.temperature_probs(p_logits[0], 1.0).astype(np.float64)
    rng = np.random.default_rng(11)
    counts = np.zeros(V)
    acc = 0
    for s in range(N):
        d = O.sample_inverse_cdf(q[0], np.float32(rng.integers(0, 2**24) / 2**24))
        na, nt = O.stochastic_accept(p_logits, q, np.array([d], np.uint32), 1.0, s, 10)
        counts[d if na == 1 else nt] += 1
        acc += na
    assert chisquare(counts, p0 / p0.sum() * N).pvalue > 1e-4
    # acceptance rate = sum_x min(p, q)
    assert abs(acc / N - np.minimum(p0, q[0]).sum()) < 0.02


def test_stochastic_accept_invariants():
    rng = np.random.default_rng(4)
    V, k = 50, 4
    p_logits = rng.normal(0, 1, (k + 1, V)).astype(np.float32)
    # q == p: every draft is accepted (u*q < p holds whenever u < 1 and p > 0)
    q = np.stack([O.temperature_probs(p_logits[i], 1.0) for i in range(k)])
    drafts = np.array([int(np.argmax(q[i])) for i in range(k)], np.uint32)
    na, nt = O.stochastic_accept(p_logits, q, drafts, 1.0, 99, 10)
    assert na == k and nt < V
    # q puts all mass on a token p gives zero probability -> rejected at once, resample
    # from max(0, p - q) which excludes that token
    p0 = p_logits.copy()
    p0[0, 7] = -1e30
    q0 = np.zeros((k, V), np.float32)
    q0[:, 7] = 1.0
    d0 = np.full(k, 7, np.uint32)
    na, nt = O.stochastic_accept(p0, q0, d0, 1.0, 99, 10)
    assert na == 0 and nt != 7
