"""The N(0, 1) KV fill behind config 4's "8192-token KV cache filled with N(0, 1) keys and values"
and the config-position parity tests: the library's generator (nc_synth_kv_values, host only, the
values nc_session_fill_kv uploads) against the oracle's restatement (or_synth_kv_values), both
against float64 Box-Muller on the oracle's Philox words, their distribution against N(0, 1), and
the oracle's placement of the values in its cache against the float64 forward of
tests/refmodel_np.py given the same rows.  CPU only."""
import numpy as np
import pytest
from scipy import stats

import nanocamelid_amd as nc
from oracle import oracle as O
from tests import refmodel_np as R

CASES = [(7, 0, 0, 0, 1000), (7, 79, 1, 8191 * 1024, 2048), (2**40 + 3, 3, 1, 123456, 4096), (1, 1, 0, 2**33, 64)]


@pytest.mark.parametrize("seed,layer,kind,start,count", CASES)
def test_library_and_oracle_streams_are_identical(seed, layer, kind, start, count):
    a = nc.synth_kv_values(seed, layer, kind, start, count)
    b = O.synth_kv_values(seed, layer, kind, start, count)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_stream_is_box_muller_on_philox():
    # float64 restatement from the oracle's Philox words (pinned by the Random123 known answers):
    # u1 = (53-bit word + 1) / 2^53, u2 = 53-bit word / 2^53, z = sqrt(-2 ln u1) (cos, sin)(2 pi u2)
    seed, layer, kind, start, count = 99, 5, 1, 4096, 2000
    got = O.synth_kv_values(seed, layer, kind, start, count).astype(np.float64)
    ref = np.zeros(count)
    for e in range(0, count, 2):
        j = (start + e) // 2
        w = O.philox4x32_10([j & 0xFFFFFFFF, j >> 32, 2 * layer + kind, 10], [seed & 0xFFFFFFFF, seed >> 32])
        w = [int(x) for x in w]
        u1 = (float(((w[0] >> 5) << 26) | (w[1] >> 6)) + 1.0) / 2.0**53
        u2 = float(((w[2] >> 5) << 26) | (w[3] >> 6)) / 2.0**53
        r = np.sqrt(-2.0 * np.log(u1))
        ref[e], ref[e + 1] = r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - ref) <= ulp), np.max(np.abs(got - ref) / ulp)
    # a planted mistake (cos and sin swapped) is far outside that bound
    assert np.max(np.abs(got[0::2] - ref[1::2])) > 0.5


def test_stream_distribution_is_standard_normal():
    x = np.concatenate([nc.synth_kv_values(2024, l, k, 0, 200000) for l in (0, 40) for k in (0, 1)]).astype(np.float64)
    assert abs(x.mean()) < 0.005 and abs(x.std() - 1.0) < 0.005
    assert stats.kstest(x, "norm").pvalue > 1e-3
    # streams of other layers, kinds and seeds are different draws
    a, b = nc.synth_kv_values(5, 0, 0, 0, 4096), nc.synth_kv_values(5, 0, 1, 0, 4096)
    c, d = nc.synth_kv_values(5, 1, 0, 0, 4096), nc.synth_kv_values(6, 0, 0, 0, 4096)
    for y in (b, c, d):
        assert abs(np.corrcoef(a, y)[0, 1]) < 0.06


@pytest.mark.parametrize("spec", [
    dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512, vocab_size=600,
         tied=1, norm_mode=1),
    dict(layers=2, embedding_length=512, head_count=4, head_count_kv=1, feed_forward_length=512, vocab_size=500,
         tied=0, norm_mode=1),
])
def test_oracle_fill_places_rows_as_the_float64_forward_reads_them(spec):
    # verify rows at start = n after the fill, against the float64 forward given the streams'
    # rows as its past keys (already rotated, as the cache stores them) and values
    img = nc.synth_gguf(**spec, context_length=128, seed=31)
    n, toks = 52, nc.uniform_prompt(8, 5, spec["vocab_size"])
    s = O.Session(O.Model(data=img.tobytes()), 96, 16)
    s.fill_kv(n, 17)
    _, _, got = s.verify_greedy(toks, n, want_logits=True)
    m = R.Model(img)
    kw = m.Hkv * m.hd
    past = [(O.synth_kv_values(17, l, 0, 0, n * kw), O.synth_kv_values(17, l, 1, 0, n * kw)) for l in range(m.L)]
    ref = m.logits(toks, start=n, past=past)
    scale = float(np.max(np.abs(ref)))
    rel = float(np.max(np.abs(ref - got))) / scale
    assert rel < 1e-3, rel
    # the same comparison with keys and values exchanged, or the layers' rows exchanged, fails
    for wrong in ([(v, k) for k, v in past], past[::-1]):
        bad = float(np.max(np.abs(m.logits(toks, start=n, past=wrong) - got))) / scale
        assert bad > 10 * 1e-3, bad
