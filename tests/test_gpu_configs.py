"""GPU tests at the benchmark configurations' full shapes (3 and 4).

The GPU logits are checked bit for bit against the CPU oracle at each configuration's own
positions, with the KV cache filled by the seeded N(0, 1) streams both sides draw identically
(nc_session_fill_kv / or_session_fill_kv); where the oracle cannot run the whole workload,
size-independent properties stand in:
  config 2 (Llama-3-8B shape, Q4_0): one 5-row verify bit-exact vs the oracle after a short
    prompt and one at position 1024 over 1024 N(0, 1) positions; at a 512-token prompt the
    speculative stream equals the GPU greedy record for k in {2, 4, 8} x alpha in {0.5, 0.8},
    with consistent statistics.
  config 3 (Llama-3.2-3B shape Q4_K target, 1B-shape Q4_0 draft, T = 1): the stochastic stream
    and statistics equal the oracle's at a short prompt; a 5-row verify of the target at position
    4000 over 4000 N(0, 1) positions is bit-exact vs the oracle; at a 4096-position context a
    draft identical to the target is always accepted and the stream does not depend on how the
    draft's prompt was chunked.
  config 4 (Llama-3-70B shape, Q4_0, 9-row verify over an 8192-token KV cache of N(0, 1) keys and
    values): a two-layer model at the 70B width (d 8192, 64 heads, 8 KV heads, hd 128, FFN 28672,
    vocab 128256: the same matmul shapes and attention tiers) is bit-exact vs the oracle at
    position 8192; the full 80-layer model's 9-row verify of its greedy continuation accepts all
    8 drafts and its rows' logits equal nine single-token forwards bit for bit.
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
    # (a') the config's own positions: 1024 N(0, 1) positions, then a 5-row verify at 1024
    print("config 2: N(0, 1) fill of 1024 positions, 5-row verify at 1024 vs the oracle", flush=True)
    n = 1024
    gs, os_ = nc.Session(gm, n + 16, 16), O.Session(om, n + 16, 16)
    gs.fill_kv(n, 2)
    os_.fill_kv(n, 2)
    toks = nc.uniform_prompt(1024, 5, V)
    a, nxt, newpos, preds = gs.verify_greedy(toks, n)
    opreds, _, ologits = os_.verify_greedy(toks, n, want_logits=True)
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
    # (a') the target at the config's context: a 5-row verify at position 4000 over 4000 N(0, 1)
    # positions, every row bit-exact
    print("config 3: N(0, 1) fill of 4000 positions, target 5-row verify at 4000 vs the oracle", flush=True)
    n = 4000
    gs, os_ = nc.Session(tm, n + 16, 16), O.Session(tmo, n + 16, 16)
    gs.fill_kv(n, 3)
    os_.fill_kv(n, 3)
    toks = nc.uniform_prompt(4000, 5, V)
    _, _, _, preds = gs.verify_greedy(toks, n)
    opreds, _, ologits = os_.verify_greedy(toks, n, want_logits=True)
    assert np.array_equal(preds, opreds)
    for i in range(5):
        assert _same(gs.logits(i), ologits[i]), i
    os_.close()
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


def test_config4_70b_width_two_layers_vs_oracle(ctx):
    import nanocamelid_amd as nc
    spec = dict(nc.SYNTH_CONFIGS["llama-3-70b"], layers=2, context_length=8192 + 64)
    print("config 4: two-layer model at the 70B width", flush=True)
    img = nc.synth_gguf(**spec, seed=71, nthreads=THREADS)
    gm = nc.Model(ctx, data=img, nthreads=THREADS)
    om = O.Model(data=img.tobytes(), nthreads=THREADS)
    del img
    V = gm.config["vocab_size"]
    n, rows = 8192, 9
    gs, os_ = nc.Session(gm, n + 16, 16), O.Session(om, n + 16, 16)
    print("config 4: N(0, 1) fill of 8192 positions on both sides", flush=True)
    gs.fill_kv(n, 70)
    os_.fill_kv(n, 70)
    toks = nc.uniform_prompt(8192, rows, V)
    print("config 4: 9-row verify at 8192 (rows of 8193..8201 positions)", flush=True)
    _, _, _, preds = gs.verify_greedy(toks, n)
    opreds, _, ologits = os_.verify_greedy(toks, n, want_logits=True)
    assert np.array_equal(preds, opreds)
    for i in range(rows):
        assert _same(gs.logits(i), ologits[i]), i
    os_.close()
    om.close()


def test_config4_llama3_70b_verify(ctx):
    import nanocamelid_amd as nc
    print("config 4: synthesising the 70B-shape model (~40 GB)", flush=True)
    img = nc.synth_gguf(**nc.SYNTH_CONFIGS["llama-3-70b"], context_length=8192 + 64, seed=70, nthreads=THREADS)
    gm = nc.Model(ctx, data=img, nthreads=THREADS)
    del img
    V = gm.config["vocab_size"]
    n_ctx, n = 8192, 9
    sess = nc.Session(gm, n_ctx + 64, 16)
    print("config 4: N(0, 1) fill of the 8192-position KV cache", flush=True)
    sess.fill_kv(n_ctx, 70)
    # greedy continuation by single-token passes from position 8192, keeping every row's logits
    greedy, single = [int(nc.uniform_prompt(70, 1, V)[0])], []
    for i in range(n):
        nxt, lg = sess.forward_pass(greedy[-1], n_ctx + i)
        single.append(lg)
        greedy.append(nxt)
    print("config 4: 9-row verify of the greedy continuation", flush=True)
    a, nxt, newpos, preds = sess.verify_greedy(np.array(greedy[:n], np.uint32), n_ctx)
    assert a == n - 1 and np.array_equal(preds, greedy[1:]) and newpos == n_ctx + n
    for i in range(n):
        assert _same(sess.logits(i), single[i]), i
