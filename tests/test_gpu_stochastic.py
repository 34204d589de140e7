"""GPU parity of the stochastic (temperature) speculative path against the CPU oracle.

The specification has no reference counterpart (the reference's temperature path matches
tokens, speculative.rs:403); the oracle restates the library's own: temperature softmax
with the reference's formula and a left-to-right f32 sum (inference.rs:3522-3540,
4857-4862), Philox4x32-10 uniforms, min(1, p/q) acceptance and fixed-point inverse-CDF
sampling.  Every probability must be bit-identical and every sampled token identical.
"""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TINY = dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512, vocab_size=1000,
            context_length=512, tied=1, norm_mode=1)


@pytest.fixture(scope="module")
def ctx():
    import nanocamelid_amd as nc
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    return nc.Context(0)


def _rows(V, rng):
    rows = {
        "normal": rng.normal(0, 2, V),
        "flat": np.zeros(V),                               # every term exactly 1
        "peaked": np.concatenate([[40.0], rng.normal(0, 1, V - 1)]),
        "wide": rng.normal(0, 30, V),                      # most terms underflow to 0
        "ties": np.round(rng.normal(0, 1, V) * 4) / 4,     # many equal logits
        "ramp": np.linspace(-20, 5, V),
    }
    if V >= 16384:
        # ~e^-80 terms first: the partial sums stay below 2^-102 for thousands of terms, where
        # every run is sensitive; a parallel segment lists at most 256 of them, so the row takes
        # the segment-after-segment evaluation
        rows["tiny_prefix"] = np.concatenate([rng.normal(-80, 0.5, 12000), rng.normal(0, 1, V - 12000)])
    return {k: v.astype(np.float32) for k, v in rows.items()}


@pytest.mark.parametrize("V", [7, 1000, 16384, 128256, 300000])
@pytest.mark.parametrize("temp", [1.0, 0.7, 2.5])
def test_temperature_probs_bit_exact(ctx, V, temp):
    import nanocamelid_amd as nc
    rows = _rows(V, np.random.default_rng(V))
    names = list(rows)
    x = np.stack([rows[k] for k in names])
    print(f"temperature probs V={V} T={temp}", flush=True)
    got = nc.temperature_probs_batch(ctx, torch.from_numpy(x).cuda(), temp)
    paths = dict(zip(names, nc.temperature_paths(ctx, len(names), torch.cuda.current_stream().cuda_stream)))
    got = got.cpu().numpy()
    for r, name in enumerate(names):
        ref = O.temperature_probs(x[r], temp)
        assert np.array_equal(got[r].view(np.uint32), ref.view(np.uint32)), f"{name} V={V} T={temp}"
    # which evaluation gave each sum: segments in parallel up to 262144 terms; the tiny prefix
    # (at T = 1, where its terms stay near e^-80) forces the sequential one
    for name in ("normal", "flat", "peaked", "ramp"):
        assert paths[name] == (1 if V <= 262144 else 0), (name, V, temp)
    if "tiny_prefix" in paths and temp == 1.0:
        assert paths["tiny_prefix"] == 0


def _accept_case(ctx, p_logits, q, drafts, temp, seed, start):
    import nanocamelid_amd as nc
    k = len(drafts)
    pt = nc.temperature_probs_batch(ctx, torch.from_numpy(p_logits).cuda(), temp)
    qt = torch.from_numpy(np.ascontiguousarray(q, np.float32)).cuda()
    dt = torch.from_numpy(np.asarray(drafts, np.int32)).cuda()
    a, nxt, newpos = nc.stochastic_accept(ctx, pt, qt, dt, seed, start)
    oa, onxt = O.stochastic_accept(p_logits, q, np.asarray(drafts, np.uint32), temp, seed, start)
    assert (a, nxt, newpos) == (oa, onxt, start + oa + 1), (seed, start)
    return a


@pytest.mark.parametrize("V", [1000, 128256])
def test_stochastic_accept_matches_oracle(ctx, V):
    rng = np.random.default_rng(V + 1)
    seen = set()
    for trial in range(12):
        k = (0, 1, 4, 8)[trial % 4]
        temp = (1.0, 0.8)[trial % 2]
        p_logits = rng.normal(0, 2, (k + 1, V)).astype(np.float32)
        # draft distribution: a perturbed copy of the target rows, drafts sampled from it
        q_logits = p_logits[:k] + rng.normal(0, 1.0, (k, V)).astype(np.float32)
        q = np.stack([O.temperature_probs(q_logits[i], temp) for i in range(k)]) if k else np.zeros((0, V), np.float32)
        drafts = [O.sample_inverse_cdf(q[i], np.float32(rng.integers(0, 2**24) / 2**24)) for i in range(k)]
        print(f"accept V={V} trial={trial} k={k}", flush=True)
        seen.add(_accept_case(ctx, p_logits, q, drafts, temp, 1000 + trial, 50 + 7 * trial) == k)
    assert seen == {True, False}  # both the bonus and the resample branch ran


def test_stochastic_accept_edge_cases(ctx):
    rng = np.random.default_rng(8)
    V, k = 1000, 4
    p_logits = rng.normal(0, 1, (k + 1, V)).astype(np.float32)
    p = np.stack([O.temperature_probs(p_logits[i], 1.0) for i in range(k + 1)])
    # q == p: every draft accepted, bonus sample from row k
    drafts = [int(np.argmax(p[i])) for i in range(k)]
    assert _accept_case(ctx, p_logits, p[:k], drafts, 1.0, 5, 10) == k
    # q concentrated on a token p gives zero mass: rejected at row 0, resampled elsewhere
    p0 = p_logits.copy()
    p0[0, 7] = -1e30
    q0 = np.zeros((k, V), np.float32)
    q0[:, 7] = 1.0
    assert _accept_case(ctx, p0, q0, [7] * k, 1.0, 5, 10) == 0
    # q = p except q(x) = 2 p(x): the residual max(0, p - q) is empty, so a rejection
    # resamples from p; find seeds (by the oracle) where row 0 rejects
    q2 = p[:k].copy()
    x = int(np.argmax(p[0]))
    q2[0, x] = 2 * p[0, x]
    hit = 0
    for seed in range(40):
        oa, _ = O.stochastic_accept(p_logits, q2, np.array([x] + [0] * (k - 1), np.uint32), 1.0, seed, 3)
        if oa == 0:
            assert _accept_case(ctx, p_logits, q2, [x] + [0] * (k - 1), 1.0, seed, 3) == 0
            hit += 1
    assert hit >= 3
    # an id outside the vocabulary is rejected without reading past the rows
    import nanocamelid_amd as nc
    pt = nc.temperature_probs_batch(ctx, torch.from_numpy(p_logits).cuda(), 1.0)
    a, nxt, _ = nc.stochastic_accept(ctx, pt, torch.from_numpy(p[:k]).cuda(),
                                     torch.tensor([V + 5, 0, 0, 0], dtype=torch.int32, device="cuda"), 9, 0)
    assert a == 0 and nxt < V


def _models(ctx, spec, seed):
    import nanocamelid_amd as nc
    img = nc.synth_gguf(**spec, seed=seed)
    return nc.Model(ctx, data=img), O.Model(data=img.tobytes(), nthreads=16)


def test_verify_stochastic_session(ctx):
    import nanocamelid_amd as nc
    gm, om = _models(ctx, TINY, seed=12)
    gs = nc.Session(gm, 256, 16)
    os_ = O.Session(om, 256, 16)
    rng = np.random.default_rng(2)
    pos = 0
    prompt = nc.uniform_prompt(3, 20, 1000)
    gs.prefill_pass_batch(prompt, 0)
    for i in range(0, 20, 16):  # the oracle's batch pass takes at most max_batch rows
        os_.prefill_pass_batch(prompt[i:i + 16], i)
    pos = 20
    for step, k in enumerate((4, 2, 8, 0, 4)):
        toks = nc.uniform_prompt(100 + step, k + 1, 1000)
        q_logits = rng.normal(0, 2, (k, 1000)).astype(np.float32)
        q = np.stack([O.temperature_probs(q_logits[i], 0.9) for i in range(k)]) if k else np.zeros((1, 1000), np.float32)
        print(f"verify_stochastic step={step} k={k} pos={pos}", flush=True)
        a, nxt, newpos = gs.verify_stochastic(toks, pos, torch.from_numpy(q).cuda(), 0.9, 42)
        _, _, lg = os_.verify_greedy(toks, pos, want_logits=True)
        oa, onxt = O.stochastic_accept(lg, q[:k], toks[1:], 0.9, 42, pos)
        assert (a, nxt, newpos) == (oa, onxt, pos + oa + 1)
        pos += k + 1


def test_generate_speculative_stochastic(ctx):
    import nanocamelid_amd as nc
    gm, om = _models(ctx, TINY, seed=31)
    dspec = dict(TINY, layers=1, feed_forward_length=256, head_count=2, head_count_kv=1)
    dgm, dom = _models(ctx, dspec, seed=5)
    prompt = nc.uniform_prompt(77, 24, 1000)
    for k, temp, seed in ((4, 1.0, 7), (2, 0.6, 8), (8, 1.3, 9)):
        print(f"stochastic stream k={k} T={temp}", flush=True)
        g_out, st = nc.generate_speculative_stochastic(nc.Session(gm, 400, 16), nc.Session(dgm, 400, 16), prompt, 80,
                                                       k, temp, seed)
        o_out, drafted, accepted, steps = O.generate_speculative_stochastic(
            O.Session(om, 400, 16), O.Session(dom, 400, 16), prompt, 80, k, temp, seed)
        assert np.array_equal(g_out, o_out), (k, temp)
        assert (st.drafted, st.accepted, st.steps) == (drafted, accepted, steps)
        assert 0 < accepted < drafted
    # draft identical to the target: every draft is accepted
    g_out, st = nc.generate_speculative_stochastic(nc.Session(gm, 400, 16), nc.Session(gm, 400, 16), prompt, 60, 4,
                                                   1.0, 3)
    o_out, drafted, accepted, steps = O.generate_speculative_stochastic(O.Session(om, 400, 16), O.Session(om, 400, 16),
                                                                        prompt, 60, 4, 1.0, 3)
    assert np.array_equal(g_out, o_out)
    assert st.accepted == st.drafted > 0


# ---------------------------------------------------------------- the reference's sampler
# sample_logits (inference.rs:4834-4873) with the reference's LCG (rand_simple, :4876-4883):
# every id and the LCG state after the draws identical to the oracle's, on rows whose
# subtraction walk crosses many binades (flat: e = 1 everywhere), stays on one term (peaked),
# skips long runs of zero terms (wide) or ends past several 16384-term segments.
@pytest.mark.parametrize("V", [7, 1000, 16385, 128256])
@pytest.mark.parametrize("temp", [0.0, 0.5, 1.0, 1.7])
def test_sample_logits_batch_matches_oracle(ctx, V, temp):
    import nanocamelid_amd as nc
    rng = np.random.default_rng(V + 3)
    base = list(_rows(V, rng).values())
    x = np.stack(base + [rng.normal(0, 1 + r, V).astype(np.float32) for r in range(16 - len(base))])
    xt = torch.from_numpy(x).cuda()
    st = O.REFERENCE_RNG_STATE
    for call in range(3):
        print(f"sample_logits V={V} T={temp} call={call}", flush=True)
        ids, st_gpu = nc.sample_logits_batch(ctx, xt, temp, st)
        want = []
        for r in range(x.shape[0]):
            i, st = O.sample_logits(x[r], temp, st)
            want.append(i)
        assert ids.tolist() == want, (V, temp, call)
        assert st_gpu == st


TINY_UNTIED = dict(TINY, tied=0)


@pytest.mark.parametrize("draft_seed,k,temp", [(72, 2, 0.3), (71, 4, 0.05)])
def test_speculative_draft_temp_matches_oracle(ctx, draft_seed, k, temp):
    """speculative_decoding_step at temp > 0 (speculative.rs:299-494): the GPU loop's tokens,
    drafted/accepted counts and final LCG state equal the oracle's, with a draft that is another
    model (every draft rejected) and one with the target's weights at a low temperature (drafts
    accepted and rejected)."""
    import nanocamelid_amd as nc
    imgs = {s: nc.synth_gguf(**TINY_UNTIED, seed=s) for s in {71, draft_seed}}
    gt, gd = nc.Model(ctx, data=imgs[71]), nc.Model(ctx, data=imgs[draft_seed])
    ot, od = O.Model(data=imgs[71].tobytes(), nthreads=16), O.Model(data=imgs[draft_seed].tobytes(), nthreads=16)
    prompt = nc.uniform_prompt(73, 20, 1000)
    print(f"draft temp loop draft={draft_seed} k={k} T={temp}", flush=True)
    toks, stats, st = nc.generate_speculative_draft_temp(nc.Session(gt, 512, 16), nc.Session(gd, 512, 16), prompt,
                                                         40, k, temp)
    otoks, odrafted, oacc, osteps, ost = O.generate_speculative_draft_temp(O.Session(ot, 512, 16),
                                                                           O.Session(od, 512, 16), prompt, 40, k, temp)
    assert np.array_equal(toks, otoks)
    assert (stats.drafted, stats.accepted, stats.steps, st) == (odrafted, oacc, osteps, ost)
    if temp < 0.1:
        assert 0 < stats.accepted < stats.drafted


@pytest.mark.parametrize("draft_seed,temp", [(71, 0.05), (71, 0.0), (72, 0.3)])
def test_speculative_draft_stop_tokens_match_oracle(ctx, draft_seed, temp):
    """Stop tokens in the draft-model loop (is_stop_token, speculative.rs:305-447, and the
    generate loop's turn end, main.rs:9852-9866), at temperature and greedy: for stop ids taken
    from the unstopped stream (so that drafted, accepted, corrective and trailing stops occur),
    the GPU loop's tokens, counts, steps and LCG state equal the oracle's, and no stop token is
    emitted."""
    import nanocamelid_amd as nc
    imgs = {s: nc.synth_gguf(**TINY_UNTIED, seed=s) for s in {71, draft_seed}}
    gt, gd = nc.Model(ctx, data=imgs[71]), nc.Model(ctx, data=imgs[draft_seed])
    ot, od = O.Model(data=imgs[71].tobytes(), nthreads=16), O.Model(data=imgs[draft_seed].tobytes(), nthreads=16)
    prompt = nc.uniform_prompt(73, 20, 1000)
    free = O.generate_speculative_draft_temp(O.Session(ot, 512, 16), O.Session(od, 512, 16), prompt, 40, 4, temp)[0]
    for cut in (3, 12, 21, 33):
        stop = (int(free[cut]), 999)
        print(f"draft stop loop draft={draft_seed} T={temp} stop={stop}", flush=True)
        toks, stats, st = nc.generate_speculative_draft_temp(nc.Session(gt, 512, 16), nc.Session(gd, 512, 16),
                                                             prompt, 40, 4, temp, stop=stop)
        otoks, odrafted, oacc, osteps, ost = O.generate_speculative_draft_temp(
            O.Session(ot, 512, 16), O.Session(od, 512, 16), prompt, 40, 4, temp, stop=stop)
        assert np.array_equal(toks, otoks), cut
        assert (stats.drafted, stats.accepted, stats.steps, st) == (odrafted, oacc, osteps, ost), cut
        assert stop[0] not in toks.tolist()


@pytest.mark.parametrize("temp", [0.0, 0.7, 1.3])
def test_plain_loop_matches_oracle(ctx, temp):
    """The plain decode loop (main.rs:9894-9928) with sample_logits, the reference's LCG and stop
    tokens: the GPU loop's tokens and LCG state equal the oracle's, with and without stops, and
    a run stops before the first stop token of the unstopped stream."""
    import nanocamelid_amd as nc
    img = nc.synth_gguf(**TINY_UNTIED, seed=71)
    gm, om = nc.Model(ctx, data=img), O.Model(data=img.tobytes(), nthreads=16)
    prompt = nc.uniform_prompt(75, 20, 1000)
    print(f"plain loop T={temp}", flush=True)
    free, stats, st = nc.Session(gm, 512, 16).generate_plain(prompt, 30, temp)
    ofree, ost = O.generate_plain(O.Session(om, 512, 16), prompt, 30, temp)
    assert np.array_equal(free, ofree) and st == ost and stats.emitted == 30
    for cut in (0, 7, 22):
        stop = (int(free[cut]), 5)
        toks, stats, st = nc.Session(gm, 512, 16).generate_plain(prompt, 30, temp, stop=stop)
        otoks, ost = O.generate_plain(O.Session(om, 512, 16), prompt, 30, temp, stop=stop)
        assert np.array_equal(toks, otoks) and st == ost, cut
        assert np.array_equal(toks, free[:free.tolist().index(stop[0])]) or 5 in free[:len(toks) + 1].tolist()


@pytest.mark.parametrize("temp,prompt_seed", [(0.0, 77), (0.08, 78), (0.12, 79)])
def test_ngram_loop_temp_matches_oracle(ctx, temp, prompt_seed):
    """ngram_speculative_step at temperature (speculative.rs:122-286, main.rs:9729-9776): the GPU
    loop's tokens, drafted/accepted counts, steps and LCG state equal the oracle's on repetitive
    prompts (drafts accepted and rejected), with and without stop tokens; greedy (temp 0) runs
    the k+1 fast path, whose counts must agree with the oracle's step form too."""
    import nanocamelid_amd as nc
    img = nc.synth_gguf(**TINY_UNTIED, seed=71)
    gm, om = nc.Model(ctx, data=img), O.Model(data=img.tobytes(), nthreads=16)
    prompt = np.tile(nc.uniform_prompt(prompt_seed, 6, 1000), 8 if temp == 0.12 else 5)
    base, stops_done = None, []
    for stop in [()] + [None] * 3:
        if stop is None:
            stop = (int(base[3 + 9 * len(stops_done)]),)
        print(f"ngram loop T={temp} stop={stop}", flush=True)
        toks, stats, st = nc.Session(gm, 512, 16).generate_speculative_ngram_temp(prompt, 40, 4, temp, stop=stop)
        otoks, odr, oacc, osteps, ost = O.Session(om, 512, 16).generate_speculative_ngram_temp(prompt, 40, 4, temp,
                                                                                            stop=stop)
        assert np.array_equal(toks, otoks), stop
        assert (stats.drafted, stats.accepted, stats.steps, st) == (odr, oacc, osteps, ost), stop
        if base is None:
            base = toks
            assert stats.drafted > 0
        else:
            stops_done.append(stop)
            assert stop[0] not in toks.tolist()


def test_ngram_loop_temp_k_beyond_batch(ctx):
    """k larger than a verify batch holds (20 > max_batch - 1): drafts are capped by the batch as
    ngram_speculative_step truncates them (speculative.rs:154-159), same as the oracle."""
    import nanocamelid_amd as nc
    img = nc.synth_gguf(**TINY_UNTIED, seed=71)
    gm, om = nc.Model(ctx, data=img), O.Model(data=img.tobytes(), nthreads=16)
    prompt = np.tile(nc.uniform_prompt(78, 6, 1000), 5)
    toks, stats, st = nc.Session(gm, 512, 16).generate_speculative_ngram_temp(prompt, 40, 20, 0.08)
    otoks, odr, oacc, osteps, ost = O.Session(om, 512, 16).generate_speculative_ngram_temp(prompt, 40, 20, 0.08)
    assert np.array_equal(toks, otoks)
    assert (stats.drafted, stats.accepted, stats.steps, st) == (odr, oacc, osteps, ost)
