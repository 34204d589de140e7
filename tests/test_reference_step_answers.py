"""The reference's own step tests (src/speculative.rs:598-842), ported to the oracle's decode loops.

The reference builds a model with all-zero weights, so every logit is equal and greedy
sampling returns token 0, then checks the step's bookkeeping:
  ngram_step_keeps_pos_and_context_consistent (:598-645): a history of zeros makes the n-gram
    drafter propose zeros, which all verify; exit invariant pos == context_tokens.len();
  ngram_step_returns_stop_without_emitting (:647-689): the first sampled token is a stop token,
    so the step emits nothing, drafts nothing and leaves pos and the context as they were;
  test_speculative_greedy_decoding (:691-773): draft == target, draft_k = 2: both drafts drafted
    and accepted, the emitted tokens the greedy ones;
  speculative_step_clamps_draft_k_to_batch_workspace (:775-842): draft_k = 16 against a batch
    workspace of 2 rows drafts at most 2 per step and does not fail.
Here the zero-weight model is the synthetic writer's with weight_std = 0 (its logits are all 0,
so the first-max rule gives token 0, as the reference's pre-set logits give their token).  The
exit invariant is checked where it can fail: with random weights, after each loop the session's
KV rows must be those of a fresh prefill of the consumed history (prompt + every emitted token
but the pending last one), so the last token's forward at position len(prompt) + len(out) - 1
gives the same logits bit for bit.  CPU (oracle); tests/test_gpu_reference_steps.py runs the
same cases on the device loops.
"""
import numpy as np
import pytest

import nanocamelid_amd as nc
from oracle import oracle as O

ZERO = dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512, vocab_size=64,
            context_length=64, tied=0, norm_mode=0, weight_std=0.0)
TINY = dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512, vocab_size=1000,
            context_length=256, tied=0, norm_mode=1)


@pytest.fixture(scope="module")
def zero_model():
    m = O.Model(data=nc.synth_gguf(**ZERO, seed=1).tobytes())
    s = O.Session(m, 64, 16)
    s.prefill_pass_batch(np.zeros(3, np.uint32), 0)
    lg = s.batch_row_logits(2)
    assert np.all(lg == 0.0)  # every logit equal: greedy picks token 0
    return m


def test_ngram_step_zero_history_all_verify(zero_model):
    s = O.Session(zero_model, 64, 16)
    out, drafted, accepted, steps = s.generate_speculative_ngram(np.zeros(6, np.uint32), 10, 4, stop=(3,))
    assert out.tolist() == [0] * 10
    assert drafted > 0 and accepted == drafted
    out, drafted, accepted, steps, _ = s.generate_speculative_ngram_temp(np.zeros(6, np.uint32), 10, 4, 0.0,
                                                                         stop=(3,))
    assert out.tolist() == [0] * 10
    assert drafted > 0 and accepted == drafted


def test_steps_return_stop_without_emitting(zero_model):
    prompt = np.array([0, 1, 2], np.uint32)
    t, d = O.Session(zero_model, 64, 16), O.Session(zero_model, 64, 16)
    out, drafted, accepted, steps = t.generate_speculative_ngram(prompt, 8, 4, stop=(0,))
    assert len(out) == 0 and drafted == 0
    out, drafted, accepted, steps, _ = t.generate_speculative_ngram_temp(prompt, 8, 4, 0.0, stop=(0,))
    assert len(out) == 0 and drafted == 0
    # the draft-model step drafts first: the stop token is drafted (and not run on the draft),
    # the target agrees and accepts it, and the generate loop ends the turn before emitting it
    # (speculative.rs:327-350, :403-412; main.rs:9852-9866)
    out, drafted, accepted, steps, _ = O.generate_speculative_draft_temp(t, d, prompt, 8, 4, 0.0, stop=(0,))
    assert len(out) == 0 and (drafted, accepted) == (1, 1)
    out, _ = O.generate_plain(t, prompt, 8, 0.0, stop=(0,))
    assert len(out) == 0


def test_speculative_greedy_draft_k_2(zero_model):
    t, d = O.Session(zero_model, 64, 16), O.Session(zero_model, 64, 16)
    out, drafted, accepted, steps, _ = O.generate_speculative_draft_temp(t, d, np.zeros(1, np.uint32), 3, 2, 0.0,
                                                                         stop=(3,))
    assert out.tolist() == [0, 0, 0]
    assert (drafted, accepted, steps) == (2, 2, 1)


def test_draft_k_clamped_to_batch_workspace(zero_model):
    t, d = O.Session(zero_model, 64, 2), O.Session(zero_model, 64, 2)
    out, drafted, accepted, steps, _ = O.generate_speculative_draft_temp(t, d, np.zeros(1, np.uint32), 12, 16, 0.0,
                                                                         prefill_batch=2, stop=(3,))
    assert out.tolist() == [0] * 12
    assert 0 < drafted <= 2 * steps and accepted == drafted


def _fresh_last_logits(model, prompt, out, max_ctx, chunk=16, alter=False):
    hist = np.concatenate([prompt, out[:-1]]).astype(np.uint32)
    if alter:  # a history whose last consumed token differs: the check must see it
        hist[-1] = (hist[-1] + 1) % TINY["vocab_size"]
    s = O.Session(model, max_ctx, chunk)
    for i in range(0, len(hist), chunk):
        s.prefill_pass_batch(hist[i:i + chunk], i)
    return s.forward_pass(int(out[-1]), len(hist))


@pytest.mark.parametrize("loop", ["ngram", "ngram_temp", "draft_temp", "draft_greedy", "plain"])
def test_exit_invariant_kv_rows_match_consumed_history(loop):
    img = nc.synth_gguf(**TINY, seed=77)
    m, dm = O.Model(data=img.tobytes()), O.Model(data=nc.synth_gguf(**TINY, seed=78).tobytes())
    prompt = nc.uniform_prompt(12, 20, TINY["vocab_size"])
    s, d = O.Session(m, 256, 16), O.Session(dm, 256, 16)
    if loop == "ngram":
        out = s.generate_speculative_ngram(prompt, 40, 4, min_ngram=1, max_ngram=2)[0]
    elif loop == "ngram_temp":
        out = s.generate_speculative_ngram_temp(prompt, 40, 4, 0.9, min_ngram=1, max_ngram=2)[0]
    elif loop == "draft_temp":
        out = O.generate_speculative_draft_temp(s, d, prompt, 40, 4, 0.9)[0]
    elif loop == "draft_greedy":
        out = O.generate_speculative_draft_temp(s, d, prompt, 40, 4, 0.0)[0]
    else:
        out = O.generate_plain(s, prompt, 40, 0.9)[0]
    assert len(out) == 40
    got = s.forward_pass(int(out[-1]), len(prompt) + len(out) - 1)
    want = _fresh_last_logits(m, prompt, out, 256)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert not np.array_equal(got, _fresh_last_logits(m, prompt, out, 256, alter=True))
