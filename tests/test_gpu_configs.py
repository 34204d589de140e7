"""GPU tests at the benchmark configurations' full shapes (3 and 4).

Where the CPU oracle can run the model in seconds, the GPU logits and streams are checked bit
for bit against it; at the full workload sizes, size-independent properties stand in:
  config 2 (Llama-3-8B shape, Q4_0): one 5-row verify bit-exact vs the oracle after a short
    prompt; at a 512-token prompt the speculative stream equals the GPU greedy record for
    k in {2, 4, 8} x alpha in {0.5, 0.8}, with consistent statistics.
  config 3 (Llama-3.2-3B shape Q4_K target, 1B-shape Q4_0 draft, T = 1): the stochastic stream
    and statistics equal the oracle's at a short prompt; at a 4096-position context a draft
    identical to the target is always accepted and the stream does not depend on how the
    draft's prompt was chunked.
  config 4 (Llama-3-70B shape, Q4_0): after an 8192-token prefill, the 9-row verify of the
    greedy continuation accepts all 8 drafts and its 9 rows' logits equal nine single-token
    forwards bit for bit.
"""
import os

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

THREADS = min(16, len(os.sched_getaffinity(0)))


@pytest.fixture(scope="module")
def ctx():
    import nanocamelid_amd as nc
    assert torch.cuda.is_available()
    return nc.Context(0)


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_config2_llama3_8b(ctx):
    import nanocamelid_amd as nc
    spec = dict(nc.SYNTH_CONFIGS["llama-3-8b"], context_length=8192)
    print("config 2: synthesising the 8B-shape model", flush=True)
    img = nc.synth_gguf(**spec, seed=2024, nthreads=THREADS)
    gm = nc.Model(ctx, data=img, nthreads=THREADS)
    V = gm.config["vocab_size"]
    # (a) one 5-row verify after an 8-token prompt, every row's logits bit-exact
    print("config 2: oracle 8-token prefill + 5-row verify", flush=True)
    om = O.Model(data=img.tobytes(), nthreads=THREADS)
    toks = nc.uniform_prompt(2024, 13, V)
    gs, os_ = nc.Session(gm, 64, 16), O.Session(om, 64, 16)
    gs.prefill_pass_batch(toks[:8], 0)
    os_.prefill_pass_batch(toks[:8], 0)
    a, nxt, newpos, preds = gs.verify_greedy(toks[8:], 8)
    opreds, _, ologits = os_.verify_greedy(toks[8:], 8, want_logits=True)
    assert np.array_equal(preds, opreds)
    for i in range(5):
        assert _same(gs.logits(i), ologits[i]), i
    os_.close()
    om.close()
    del om
    # (b) 512-token prompt: speculative streams equal the greedy record at every (k, alpha)
    print("config 2: 512-token prompt, greedy record and speculative decodes", flush=True)
    prompt = nc.uniform_prompt(2024, 512, V)
    n_new = 160
    sess = nc.Session(gm, 512 + n_new + 48, 16)
    greedy, _ = sess.generate_greedy(prompt, n_new + 16)
    assert len(set(greedy.tolist())) >= 16
    for k in (2, 4, 8):
        for alpha in (0.5, 0.8):
            out, st = sess.generate_speculative_oracle(prompt, n_new, k, alpha, 99, greedy)
            assert np.array_equal(out, greedy[:n_new]), (k, alpha)
            assert st.emitted == n_new and 0 < st.accepted <= st.drafted <= k * st.steps, (k, alpha)
            assert st.emitted <= st.steps + st.accepted + 1, (k, alpha)


def test_config3_q4k_target_stochastic(ctx):
    import nanocamelid_amd as nc
    print("config 3: synthesising the 3B Q4_K target and the 1B draft", flush=True)
    timg = nc.synth_gguf(**nc.SYNTH_CONFIGS["llama-3.2-3b-q4k"], context_length=8192, seed=7, nthreads=THREADS)
    dimg = nc.synth_gguf(**nc.SYNTH_CONFIGS["llama-3.2-1b"], context_length=8192, seed=8, nthreads=THREADS)
    tm, dm = nc.Model(ctx, data=timg, nthreads=THREADS), nc.Model(ctx, data=dimg, nthreads=THREADS)
    V = tm.config["vocab_size"]
    # (a) short prompt: the device loop equals the oracle's stream and statistics
    print("config 3: oracle stochastic decode at a 16-token prompt", flush=True)
    tmo, dmo = O.Model(data=timg.tobytes(), nthreads=THREADS), O.Model(data=dimg.tobytes(), nthreads=THREADS)
    prompt = nc.uniform_prompt(3, 16, V)
    out, st = nc.generate_speculative_stochastic(nc.Session(tm, 64, 16), nc.Session(dm, 64, 16), prompt, 12, 4, 1.0,
                                                 123)
    o_out, drafted, accepted, steps = O.generate_speculative_stochastic(O.Session(tmo, 64, 16),
                                                                        O.Session(dmo, 64, 16), prompt, 12, 4, 1.0,
                                                                        123)
    assert np.array_equal(out, o_out)
    assert (st.drafted, st.accepted, st.steps) == (drafted, accepted, steps)
    tmo.close()
    dmo.close()
    # (b) 4096-position context: draft == target => every draft accepted; the stream does not
    # depend on the draft session's prefill chunking
    print("config 3: 4000-token prompt, draft == target", flush=True)
    prompt = nc.uniform_prompt(4, 4000, V)
    runs = []
    for draft_batch in (16, 5):
        o, s = nc.generate_speculative_stochastic(nc.Session(tm, 4096, 16), nc.Session(tm, 4096, draft_batch), prompt,
                                                  64, 4, 1.0, 5)
        assert s.accepted == s.drafted and s.drafted > 0
        runs.append((o, s.steps))
    assert np.array_equal(runs[0][0], runs[1][0]) and runs[0][1] == runs[1][1]
    assert len(set(runs[0][0].tolist())) >= 8


def test_config4_llama3_70b_verify(ctx):
    import nanocamelid_amd as nc
    print("config 4: synthesising the 70B-shape model (~40 GB)", flush=True)
    img = nc.synth_gguf(**nc.SYNTH_CONFIGS["llama-3-70b"], context_length=8192 + 64, seed=70, nthreads=THREADS)
    gm = nc.Model(ctx, data=img, nthreads=THREADS)
    del img
    V = gm.config["vocab_size"]
    n_prompt, n = 8192, 9
    prompt = nc.uniform_prompt(70, n_prompt, V)
    sess = nc.Session(gm, n_prompt + 64, 16)
    print("config 4: 8192-token prefill", flush=True)
    sess.prefill_pass_batch(prompt, 0, want_logits=False)
    # greedy continuation by single-token passes, keeping every row's logits
    pending, lg = sess.forward_pass(int(prompt[-1]), n_prompt - 1)
    greedy, single = [pending], []
    for i in range(n - 1):
        nxt, lg = sess.forward_pass(greedy[-1], n_prompt + i)
        single.append(lg)
        greedy.append(nxt)
    _, lg = sess.forward_pass(greedy[-1], n_prompt + n - 1)
    single.append(lg)
    print("config 4: 9-row verify of the greedy continuation", flush=True)
    a, nxt, newpos, preds = sess.verify_greedy(np.array(greedy, np.uint32), n_prompt)
    assert a == n - 1 and np.array_equal(preds[:n - 1], greedy[1:]) and newpos == n_prompt + n
    for i in range(n):
        assert _same(sess.logits(i), single[i]), i
