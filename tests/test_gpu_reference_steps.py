"""The reference's step tests (src/speculative.rs:598-842) on the device loops: the cases of
tests/test_reference_step_answers.py (all-zero weights: zeros proposed and verified, a stop token
as the first sample, draft_k = 2, draft_k = 16 against a 2-row batch) and the exit invariant with
random weights (after each loop the session's KV rows are those of a fresh prefill of the
consumed history: the last token's forward gives the same logits bit for bit)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

ZERO = dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512, vocab_size=64,
            context_length=64, tied=0, norm_mode=0, weight_std=0.0)
TINY = dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512, vocab_size=1000,
            context_length=256, tied=0, norm_mode=1)


@pytest.fixture(scope="module")
def ctx():
    import nanocamelid_amd as nc
    assert torch.cuda.is_available()
    return nc.Context(0)


@pytest.fixture(scope="module")
def zero_model(ctx):
    import nanocamelid_amd as nc
    return nc.Model(ctx, data=nc.synth_gguf(**ZERO, seed=1))


def test_zero_weights_all_verify(zero_model):
    import nanocamelid_amd as nc
    print("zero weights: n-gram loops", flush=True)
    s = nc.Session(zero_model, 64, 16)
    out, st = s.generate_speculative_ngram(np.zeros(6, np.uint32), 10, 4, stop=(3,))
    assert out.tolist() == [0] * 10 and st.drafted > 0 and st.accepted == st.drafted
    out, st, _ = s.generate_speculative_ngram_temp(np.zeros(6, np.uint32), 10, 4, 0.0, stop=(3,))
    assert out.tolist() == [0] * 10 and st.drafted > 0 and st.accepted == st.drafted


def test_stop_without_emitting(zero_model):
    import nanocamelid_amd as nc
    print("zero weights: stop token first", flush=True)
    prompt = np.array([0, 1, 2], np.uint32)
    t, d = nc.Session(zero_model, 64, 16), nc.Session(zero_model, 64, 16)
    out, st = t.generate_speculative_ngram(prompt, 8, 4, stop=(0,))
    assert len(out) == 0 and st.drafted == 0
    out, st, _ = t.generate_speculative_ngram_temp(prompt, 8, 4, 0.0, stop=(0,))
    assert len(out) == 0 and st.drafted == 0
    out, st, _ = nc.generate_speculative_draft_temp(t, d, prompt, 8, 4, 0.0, stop=(0,))
    assert len(out) == 0 and (st.drafted, st.accepted) == (1, 1)
    out, st, _ = t.generate_plain(prompt, 8, 0.0, stop=(0,))
    assert len(out) == 0


def test_draft_k_2_and_clamp(zero_model):
    import nanocamelid_amd as nc
    print("zero weights: draft_k 2; draft_k 16 on a 2-row batch", flush=True)
    t, d = nc.Session(zero_model, 64, 16), nc.Session(zero_model, 64, 16)
    out, st, _ = nc.generate_speculative_draft_temp(t, d, np.zeros(1, np.uint32), 3, 2, 0.0, stop=(3,))
    assert out.tolist() == [0, 0, 0] and (st.drafted, st.accepted, st.steps) == (2, 2, 1)
    t, d = nc.Session(zero_model, 64, 2), nc.Session(zero_model, 64, 2)
    out, st, _ = nc.generate_speculative_draft_temp(t, d, np.zeros(1, np.uint32), 12, 16, 0.0, stop=(3,))
    assert out.tolist() == [0] * 12 and 0 < st.drafted <= 2 * st.steps and st.accepted == st.drafted


@pytest.mark.parametrize("loop", ["ngram", "ngram_temp", "draft_temp", "draft_greedy", "plain"])
def test_exit_invariant(ctx, loop):
    import nanocamelid_amd as nc
    print(f"exit invariant: {loop}", flush=True)
    m = nc.Model(ctx, data=nc.synth_gguf(**TINY, seed=77))
    dm = nc.Model(ctx, data=nc.synth_gguf(**TINY, seed=78))
    prompt = nc.uniform_prompt(12, 20, TINY["vocab_size"])
    s, d = nc.Session(m, 256, 16), nc.Session(dm, 256, 16)
    if loop == "ngram":
        out = s.generate_speculative_ngram(prompt, 40, 4, min_ngram=1, max_ngram=2)[0]
    elif loop == "ngram_temp":
        out = s.generate_speculative_ngram_temp(prompt, 40, 4, 0.9, min_ngram=1, max_ngram=2)[0]
    elif loop == "draft_temp":
        out = nc.generate_speculative_draft_temp(s, d, prompt, 40, 4, 0.9)[0]
    elif loop == "draft_greedy":
        out = nc.generate_speculative_draft_temp(s, d, prompt, 40, 4, 0.0)[0]
    else:
        out = s.generate_plain(prompt, 40, 0.9)[0]
    assert len(out) == 40
    _, got = s.forward_pass(int(out[-1]), len(prompt) + len(out) - 1)
    hist = np.concatenate([prompt, out[:-1]]).astype(np.uint32)
    f = nc.Session(m, 256, 16)
    f.prefill_pass_batch(hist, 0, want_logits=False)
    _, want = f.forward_pass(int(out[-1]), len(hist))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
