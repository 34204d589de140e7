"""Could the reference's weighted-V sum (apply_attention_head, src/inference.rs:3603-3623: for
each output dim, o = fl(o + fl(p_i * v_i)) over the positions in order) be evaluated in parallel
and still bit-exactly, the way the device evaluates the non-negative RMSNorm and softmax sums
(nanocamelid_amd/csrc/nc_chain.h)?  A CPU prototype of that scheme for signed terms, and the
measurement that decides it.

Scheme: cut the P terms of a dim into segments of E; guess each segment's start as the f32
rounding of the double prefix; run the segment from the guess; the segment is "sensitive" when
a step rounds an exact tie (Fast2Sum error = half an ulp), when any state of the run leaves the
guess's binade (sign and exponent), or when it comes within 256 ulps of a binade edge; for an
insensitive segment the true end is the true start plus the run's increment (both on one ulp
grid).  A walk advances the true state over the segments in order, sequentially only through
the sensitive ones; every segment is then recomputed from its corrected start and each end
checked against the next start, so the result is exact whatever the guesses were.

Measured on N(0, 1) keys and values with real softmax weights at 700 and 8192 positions (the
config-2 and config-4 row lengths), 30-85% of the segments are sensitive: the softmax puts most
of the mass on a few positions, so terms are often as large as the running sum (ties), and the
sum changes sign and binade as it cancels.  The walk would then be sequential through most of the
chain, on top of two extra passes over every term; the device keeps the sequential chain.
"""
import numpy as np
import pytest

F = np.float32


def _terms(P, seed, hd=128, dims=32):
    rng = np.random.default_rng(seed)
    q = rng.normal(0, 1, hd).astype(F)
    K = rng.normal(0, 1, (P, hd)).astype(F)
    V = rng.normal(0, 1, (P, dims)).astype(F)
    sc = (K @ q / np.float32(np.sqrt(hd))).astype(F)
    e = np.exp((sc - sc.max()).astype(np.float64)).astype(F)
    p = (e * (F(1) / e.sum(dtype=F))).astype(F)
    return (p[:, None] * V).astype(F)


def _sequential(t):
    s = np.zeros(t.shape[1], F)
    for row in t:
        s = (s + row).astype(F)
    return s


def _parallel_exact(t, E, margin=256):
    """Returns (chain end per dim, fraction of sensitive segments, dims that needed the fallback)."""
    P, D = t.shape
    nseg = -(-P // E)
    tt = np.concatenate([t, np.zeros((nseg * E - P, D), F)]).reshape(nseg, E, D)
    pre = np.cumsum(tt.astype(np.float64).sum(axis=1), axis=0)
    g = np.concatenate([np.zeros((1, D)), pre[:-1]]).astype(F)  # guesses; segment 0 exact (0)
    x, eg = g.copy(), g.view(np.uint32) >> 23
    sens = np.zeros((nseg, D), bool)
    for j in range(E):
        r = (x + tt[:, j, :]).astype(F)
        err = tt[:, j, :].astype(np.float64) - (r.astype(np.float64) - x.astype(np.float64))
        sens |= np.abs(err) == np.spacing(np.abs(r)).astype(np.float64) / 2
        br = r.view(np.uint32)
        sens |= (br >> 23) != eg
        m = br & 0x7fffff
        sens |= (m < margin) | (m + margin >= (1 << 23))
        x = r
    sens |= ((g.view(np.uint32) >> 23) & 0xff) < 25
    sens[0] = False
    inc = x.astype(np.float64) - g.astype(np.float64)  # run increments (exact in double)
    # walk: true starts, sequential only through the sensitive segments
    starts = np.zeros((nseg, D), F)
    S = np.zeros(D, F)
    for k in range(nseg):
        starts[k] = S
        run = S.copy()
        for j in range(E):
            run = (run + tt[k, j, :]).astype(F)
        S = np.where(sens[k], run, (S.astype(np.float64) + inc[k]).astype(F))
    # verify: every segment recomputed from its start must end at the next start
    ends = starts.copy()
    for j in range(E):
        ends = (ends + tt[:, j, :]).astype(F)
    ok = np.all(ends[:-1] == starts[1:], axis=0)
    out = np.where(ok, ends[-1], _sequential(t))  # fallback: the sequential chain
    return out, float(sens[1:].mean()), int((~ok).sum())


@pytest.mark.parametrize("P,dims", [(700, 32), (8192, 8)])
def test_parallel_scheme_is_exact_but_mostly_sensitive(P, dims):
    t = _terms(P, P, dims=dims)
    want = _sequential(t)
    for E in (8, 32):
        got, frac, fallbacks = _parallel_exact(t, E)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        print(f"P {P} E {E}: sensitive segments {frac:.3f}, fallbacks {fallbacks}/{dims}")
        assert frac > 0.15  # the walk stays on the critical path: the sequential chain is kept


def test_nonnegative_sums_are_rarely_sensitive():
    # the same test on a sum of squares (the RMSNorm case the device evaluates in parallel):
    # few segments are sensitive, because a non-negative sum only grows and crosses each binade once
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (4096, 8)).astype(F)
    t = (x * x).astype(F)
    got, frac, _ = _parallel_exact(t, 8)
    assert np.array_equal(got.view(np.uint32), _sequential(t).view(np.uint32))
    assert frac < 0.05
