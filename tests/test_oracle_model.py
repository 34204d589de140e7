"""Model-level invariants of the CPU oracle on small synthetic models.

These are the reference's own end-to-end invariants: batched rows equal single-token
forwards bit for bit (inference.rs:6866-6912), speculative greedy decoding emits the
plain greedy stream (docs/bench/phase2_spec_decode.md:45-48), and a draft identical to
the target is always accepted.
"""
import numpy as np
import pytest

import nanocamelid_amd as nc
from oracle import oracle as O

# Untied: with a tied N(0, 0.02) head the hidden state stays close to the input embedding and the
# greedy stream repeats the last prompt token, which would make stream checks vacuous.
TINY = dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512, vocab_size=1000,
            context_length=512, tied=0, norm_mode=1)
MIN_DISTINCT = 8  # floor on distinct ids in a checked stream


@pytest.fixture(scope="module")
def tiny():
    img = nc.synth_gguf(**TINY, seed=21)
    return img, O.Model(data=img.tobytes())


def test_batch_rows_equal_single_token_forwards(tiny):
    _, m = tiny
    toks = nc.uniform_prompt(3, 12, 1000)
    s1 = O.Session(m, 64, 16)
    preds, margins, logits = s1.verify_greedy(toks, 0, want_logits=True)
    s2 = O.Session(m, 64, 1)
    for i, t in enumerate(toks):
        lg = s2.forward_pass(t, i)
        assert np.array_equal(lg.view(np.uint32), logits[i].view(np.uint32)), i
        assert preds[i] == int(np.argmax(lg))  # argmax picks the first max as well


def test_chunked_prefill_equals_one_batch(tiny):
    _, m = tiny
    toks = nc.uniform_prompt(4, 10, 1000)
    a = O.Session(m, 64, 16)
    pa, _, la = a.verify_greedy(toks, 0, want_logits=True)
    b = O.Session(m, 64, 16)
    b.prefill_pass_batch(toks[:6], 0)
    pb, _, lb = b.verify_greedy(toks[6:], 6, want_logits=True)
    assert np.array_equal(la[6:], lb)


def test_speculative_streams_equal_greedy(tiny):
    _, m = tiny
    prompt = nc.uniform_prompt(6, 16, 1000)
    greedy = O.Session(m, 256, 16).generate_greedy(prompt, 40)
    assert len(set(greedy.tolist())) >= MIN_DISTINCT
    # oracle drafter, k+1 form
    for alpha in (0.5, 0.8, 1.0):
        out, drafted, accepted, steps = O.Session(m, 256, 16).generate_speculative_oracle(
            prompt, 40, 4, alpha, 99, greedy)
        assert np.array_equal(out, greedy), alpha
        if alpha == 1.0:
            assert accepted == drafted
    # draft model identical to the target: acceptance exactly 1.0
    out, drafted, accepted, steps = O.generate_speculative_draft(O.Session(m, 256, 16), O.Session(m, 256, 4),
                                                                 prompt, 40, 4)
    assert np.array_equal(out, greedy)
    assert accepted == drafted and drafted > 0


def test_q4_k_model_batch_equals_single(tmp_path):
    img = nc.synth_gguf(layers=1, embedding_length=256, head_count=2, head_count_kv=1, feed_forward_length=512,
                        vocab_size=777, weight_type=nc.NC_TYPE_Q4_K, tied=1, context_length=128, seed=8)
    m = O.Model(data=img.tobytes())
    toks = nc.uniform_prompt(1, 5, 777)
    _, _, logits = O.Session(m, 32, 8).verify_greedy(toks, 0, want_logits=True)
    s = O.Session(m, 32, 1)
    for i, t in enumerate(toks):
        assert np.array_equal(s.forward_pass(t, i), logits[i])


def test_stochastic_speculation(tiny):
    img, m = tiny
    prompt = nc.uniform_prompt(5, 16, 1000)
    # draft identical to the target: q == p bit for bit, so every draft is accepted
    out, drafted, accepted, steps = O.generate_speculative_stochastic(O.Session(m, 256, 16), O.Session(m, 256, 4),
                                                                      prompt, 40, 4, 1.0, 77)
    assert len(out) == 40 and accepted == drafted and drafted > 0
    # a different draft model over the same vocabulary: deterministic, partial acceptance,
    # and independent of how the prompt is chunked
    dimg = nc.synth_gguf(layers=1, embedding_length=256, head_count=2, head_count_kv=1, feed_forward_length=256,
                         vocab_size=1000, context_length=512, tied=1, seed=5)
    dm = O.Model(data=dimg.tobytes())
    a = O.generate_speculative_stochastic(O.Session(m, 256, 16), O.Session(dm, 256, 8), prompt, 40, 4, 1.0, 77)
    b = O.generate_speculative_stochastic(O.Session(m, 256, 16), O.Session(dm, 256, 8), prompt, 40, 4, 1.0, 77,
                                          prefill_batch=5)
    assert np.array_equal(a[0], b[0]) and a[1:] == b[1:]
    assert 0 < a[2] < a[1]
    assert np.all(a[0] < 1000)


def test_draft_model_rejection_path(tiny):
    """speculative_decoding_step (speculative.rs:384-447) with a draft that disagrees part of
    the time: the draft has the target's weights but unit norm weights.  The rejections run
    the corrective token and the corrective forwards on both models; the emitted stream must
    still be the target's greedy stream, with 0 < accepted < drafted."""
    img, m = tiny
    dimg = nc.synth_gguf(**dict(TINY, norm_mode=0), seed=21)
    dm = O.Model(data=dimg.tobytes())
    prompt = nc.uniform_prompt(78, 20, 1000)
    greedy = O.Session(m, 300, 16).generate_greedy(prompt, 60)
    assert len(set(greedy.tolist())) >= MIN_DISTINCT
    for k in (1, 4, 8):
        out, drafted, accepted, steps = O.generate_speculative_draft(O.Session(m, 300, 16), O.Session(dm, 300, 8),
                                                                     prompt, 60, k)
        assert np.array_equal(out, greedy), k
        assert 0 < accepted < drafted, (k, accepted, drafted)
