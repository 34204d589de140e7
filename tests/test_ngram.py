"""n-gram prompt-lookup speculation (NGramDrafter::draft, speculative.rs:81-103, and
ngram_speculative_step, speculative.rs:122-286) on the CPU.

The oracle's drafter is pinned by the reference's own known answers (speculative.rs:562-595)
and by the defining properties of its proposal on random tiny histories; the product's
host-side drafter (nc_ngram_draft, no device involved) must agree with it exactly.  The
decode loop must emit the plain greedy stream, cut before the first stop token.
"""
import numpy as np
import pytest

import nanocamelid_amd as nc
from oracle import oracle as O

TINY = dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512, vocab_size=1000,
            context_length=512, tied=1, norm_mode=1)


def test_oracle_drafter_known_answers():
    # speculative.rs:562-567: suffix [1, 2, 3, 4] matches at the start
    assert list(O.ngram_draft([1, 2, 3, 4, 5, 6, 9, 9, 1, 2, 3, 4], 3)) == [5, 6, 9]
    # :570-576: the most recent earlier occurrence wins
    assert list(O.ngram_draft([3, 4, 7, 0, 3, 4, 8, 0, 3, 4], 2)) == [8, 0]
    # :579-584: no repeat, too short, empty
    assert len(O.ngram_draft([1, 2, 3, 4, 5], 4)) == 0
    assert len(O.ngram_draft([1, 2], 4)) == 0
    assert len(O.ngram_draft(np.zeros(0, np.uint32), 4)) == 0
    # :587-595: capped at the requested count and at the end of the history
    assert list(O.ngram_draft([1, 2, 9, 8, 7, 6, 1, 2], 2, 2, 3)) == [9, 8]
    assert list(O.ngram_draft([1, 2, 9, 8, 7, 6, 1, 2], 10, 2, 3)) == [9, 8, 7, 6, 1, 2]
    # max_tokens 0 and min_ngram 0 propose nothing (speculative.rs:82)
    assert len(O.ngram_draft([1, 2, 3, 1, 2, 3], 0)) == 0
    assert len(O.ngram_draft([1, 2, 3, 1, 2, 3], 4, 0, 4)) == 0


def _occurs_before(h, n):
    """Start indices of earlier occurrences of the length-n suffix of h."""
    L = len(h)
    return [s for s in range(L - n) if list(h[s:s + n]) == list(h[L - n:])]


@pytest.mark.parametrize("seed", range(4))
def test_oracle_drafter_properties(seed):
    rng = np.random.default_rng(seed)
    for _ in range(400):
        L = int(rng.integers(0, 24))
        h = rng.integers(0, int(rng.integers(2, 5)), L).astype(np.uint32)
        mn = int(rng.integers(1, 4))
        mx = mn + int(rng.integers(0, 3))
        mt = int(rng.integers(1, 7))
        got = list(O.ngram_draft(h, mt, mn, mx))
        top = min(mx, L - 1)
        lens = [n for n in range(mn, top + 1) if L > mn and _occurs_before(h, n)]
        if not lens:
            assert got == []
            continue
        n = max(lens)                      # the longest suffix with an earlier occurrence
        s = max(_occurs_before(h, n))      # its most recent earlier occurrence
        assert got == list(h[s + n:min(s + n + mt, L)])
        assert 1 <= len(got) <= mt


def test_product_drafter_matches_oracle():
    rng = np.random.default_rng(11)
    for _ in range(2000):
        L = int(rng.integers(0, 80))
        h = rng.integers(0, int(rng.integers(2, 7)), L).astype(np.uint32)
        mn = int(rng.integers(1, 5))
        mx = mn + int(rng.integers(0, 4))
        mt = int(rng.integers(0, 10))
        assert np.array_equal(nc.ngram_draft(h, mt, mn, mx), O.ngram_draft(h, mt, mn, mx)), (list(h), mt, mn, mx)
    assert list(nc.ngram_draft([1, 2, 3, 4, 5, 6, 9, 9, 1, 2, 3, 4], 3)) == [5, 6, 9]


@pytest.fixture(scope="module")
def tiny():
    return O.Model(data=nc.synth_gguf(**TINY, seed=21).tobytes())


def _repetitive_prompt():
    base = nc.uniform_prompt(9, 6, 1000)
    return np.concatenate([base, base, base, nc.uniform_prompt(10, 4, 1000), base[:4]]).astype(np.uint32)


def test_oracle_ngram_stream_equals_greedy(tiny):
    prompt = _repetitive_prompt()
    greedy = O.Session(tiny, 256, 16).generate_greedy(prompt, 48)
    for k in (1, 4, 8):
        out, drafted, accepted, steps = O.Session(tiny, 256, 16).generate_speculative_ngram(prompt, 48, k)
        assert np.array_equal(out, greedy), k
        assert drafted > 0 and 0 < accepted <= drafted
        assert steps < 48
    # a stop token: the stream ends just before its first occurrence in the greedy stream
    j = 17
    out, _, _, _ = O.Session(tiny, 256, 16).generate_speculative_ngram(prompt, 48, 4, stop=[int(greedy[j])])
    first = int(np.where(greedy == greedy[j])[0][0])
    assert np.array_equal(out, greedy[:first])
    # stop on the very first token: nothing emitted
    out, _, _, _ = O.Session(tiny, 256, 16).generate_speculative_ngram(prompt, 48, 4, stop=[int(greedy[0])])
    assert len(out) == 0
