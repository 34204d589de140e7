"""The reference's own temperature sampling (CPU): rand_simple, sample_logits and the
temperature draft-model step, each pinned by an independent restatement.

  rand_simple (inference.rs:4876-4883): Python integers for the 64-bit LCG, numpy float32 for
    the u32 -> f32 conversion and the division by u32::MAX as f32 (IEEE, correctly rounded);
  sample_logits (inference.rs:4834-4873): the reference loop emulated in numpy float32 (each
    subtraction, division, sum and multiply rounded as IEEE f32), with glibc expf (the oracle's
    or_expf, which Rust's f32::exp calls) for the exponentials;
  speculative_decoding_step at temp > 0 (speculative.rs:299-494): the step rewritten in Python
    over the oracle session's forward_pass / prefill_pass_batch / batch_row_logits and the
    sampler above, against the oracle's C loop: same tokens, counts and final LCG state.
"""
import numpy as np
import pytest

import nanocamelid_amd as nc
from oracle import oracle as O

F = np.float32


def _lcg_py(state, n):
    out = []
    for _ in range(n):
        state = (state * 6364136223846793005 + 1) % (1 << 64)
        out.append(F(np.uint32(state >> 32)) / F(4294967295))  # u32::MAX as f32 == 2^32
    return out, state


def test_rand_simple_matches_integer_lcg():
    want, st_end = _lcg_py(O.REFERENCE_RNG_STATE, 2000)
    st = O.REFERENCE_RNG_STATE
    for i, w in enumerate(want):
        u, st = O.rand_simple(st)
        assert F(u).view(np.uint32) == F(w).view(np.uint32), i
    assert st == st_end
    assert all(0.0 <= w <= 1.0 for w in want)


def _sample_emulated(logits, temp, state):
    """inference.rs:4846-4873 step by step in float32."""
    l = np.asarray(logits, F)
    mx = l[0]
    for v in l:
        if v > mx:
            mx = v
    e = np.array([O.expf(F(F(v - mx) / F(temp))) for v in l], F)
    s = F(0.0)
    for v in e:
        s = F(s + v)
    (u,), state = _lcg_py(state, 1)
    r = F(u * s)
    for i, v in enumerate(e):
        r = F(r - v)
        if r <= 0:
            return i, state
    return len(l) - 1, state


@pytest.mark.parametrize("V", [7, 100, 1000])
@pytest.mark.parametrize("temp", [0.5, 1.0, 1.7])
def test_sample_logits_matches_float32_emulation(V, temp):
    rng = np.random.default_rng(V + int(temp * 10))
    st_o = st_e = O.REFERENCE_RNG_STATE
    rows = [rng.normal(0, 2, V), np.zeros(V), np.round(rng.normal(0, 1, V) * 4) / 4, np.linspace(-20, 5, V)]
    for trial in range(40):
        l = np.asarray(rows[trial % len(rows)], F)
        io, st_o = O.sample_logits(l, temp, st_o)
        ie, st_e = _sample_emulated(l, temp, st_e)
        assert (io, st_o) == (ie, st_e), trial


def test_sample_logits_edges():
    st = O.REFERENCE_RNG_STATE
    l = np.array([0.5, 3.0, -1.0, 3.0], F)
    assert O.sample_logits(l, 0.0, st) == (1, st)  # greedy: first maximum, no draw
    hot = np.full(50, -200.0, F)
    hot[17] = 0.0
    for _ in range(20):  # one term carries all the mass (the others underflow to 0)
        i, st = O.sample_logits(hot, 1.0, st)
        assert i == 17


def _models(spec, seed):
    img = nc.synth_gguf(**spec, seed=seed)
    return O.Model(data=img.tobytes(), nthreads=8)


TINY = dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512, vocab_size=1000,
            context_length=512, tied=0, norm_mode=1)


def _step_loop_python(tg, dr, prompt, n_new, k, temp, state, max_batch=16, stop=(), kinds=None):
    """speculative.rs:299-494 with its is_stop_token, driven as main.rs:9643-9706 / 9799-9870,
    in Python.  Also returns how the run ended: "n_new", "accepted-stop" (a drafted stop
    token the target accepted), "corrective-stop" or "trailing-stop"; kinds (a list) receives
    "draft", "corrective" or "trailing" for each emitted token."""
    n = len(prompt)
    for s in (tg, dr):
        for i in range(0, n - 1, 16):
            s.prefill_pass_batch(prompt[i:min(i + 16, n - 1)], i)
    tl = tg.forward_pass(prompt[-1], n - 1)
    dl = dr.forward_pass(prompt[-1], n - 1)
    pos, out, drafted, accepted, steps, end = n, [], 0, 0, 0, "n_new"
    while end == "n_new" and len(out) < n_new:
        kk = min(k, n_new - len(out), max_batch, 512 - (pos + 1))
        drafts = []
        for i in range(kk):  # drafting: a stop token is kept but not run on the draft
            t, state = O.sample_logits(dl, temp, state)
            drafts.append(t)
            if t in stop:
                break
            dl = dr.forward_pass(t, pos + i)
        tg.prefill_pass_batch(np.array(drafts, np.uint32), pos)
        drafted += len(drafts)
        emitted, rejected, how, kind = [], False, "trailing-stop", []
        for i in range(len(drafts)):
            lg = tl if i == 0 else tg.batch_row_logits(i - 1)
            tt, state = O.sample_logits(lg, temp, state)
            emitted.append(tt)
            kind.append("draft" if tt == drafts[i] else "corrective")
            if tt == drafts[i]:
                accepted += 1
                if tt in stop:  # verification ends, no trailing token
                    pos, rejected, how = pos + i + 1, True, "accepted-stop"
                    break
                continue
            tl, dl = tg.forward_pass(tt, pos + i), dr.forward_pass(tt, pos + i)
            pos, rejected, how = pos + i + 1, True, "corrective-stop"
            break
        if not rejected:
            tt, state = O.sample_logits(tg.batch_row_logits(len(drafts) - 1), temp, state)
            emitted.append(tt)
            kind.append("trailing")
            tl, dl = tg.forward_pass(tt, pos + len(drafts)), dr.forward_pass(tt, pos + len(drafts))
            pos += len(drafts) + 1
        for t, kd in zip(emitted, kind):  # main.rs:9852-9866: the stop token ends the turn, unemitted
            if t in stop:
                end = how
                break
            if len(out) < n_new:
                out.append(t)
                if kinds is not None:
                    kinds.append(kd)
        steps += 1
    return np.array(out, np.uint32), drafted, accepted, steps, state, end


@pytest.mark.parametrize("draft_seed,k,temp", [(72, 2, 0.3), (71, 4, 1.0), (71, 4, 0.05)])
def test_speculative_draft_temp_loop_matches_python_restatement(draft_seed, k, temp):
    """Another model as draft (every draft rejected), and the target's own weights as draft, where
    a low temperature makes the two draws agree often: acceptances and rejections both occur."""
    tm, dm = _models(TINY, 71), _models(TINY, draft_seed)
    prompt = nc.uniform_prompt(73, 20, 1000)
    res_py = _step_loop_python(O.Session(tm, 512, 16), O.Session(dm, 512, 16), prompt, 40, k, temp,
                               O.REFERENCE_RNG_STATE)
    res_c = O.generate_speculative_draft_temp(O.Session(tm, 512, 16), O.Session(dm, 512, 16), prompt, 40, k, temp)
    assert np.array_equal(res_py[0], res_c[0])
    assert res_py[1:5] == res_c[1:] and res_py[5] == "n_new"
    assert len(set(res_c[0].tolist())) >= 8
    if temp < 0.1:
        assert 0 < res_c[2] < res_c[1]  # drafted, accepted


def test_speculative_draft_stop_tokens_match_python_restatement():
    """Stop tokens (is_stop_token, speculative.rs:305-447; the generate loop's turn end,
    main.rs:9852-9866) at temperature and greedy, with the target's own weights as draft (many
    acceptances) and another model: the oracle's C loop equals the Python restatement in
    tokens, counts and LCG state; no stop token is emitted; greedy runs end just before the
    first stop token of the unstopped stream; every way a stop can end a run occurs (an
    accepted stop draft, a corrective and a trailing stop)."""
    tm = _models(TINY, 71)
    prompt = nc.uniform_prompt(73, 20, 1000)
    ends = set()
    for draft_seed, temp in ((71, 0.05), (71, 0.0), (72, 0.3), (71, 1.0)):
        dm = _models(TINY, draft_seed)
        kinds = []
        free = _step_loop_python(O.Session(tm, 512, 16), O.Session(dm, 512, 16), prompt, 40, 4, temp,
                                 O.REFERENCE_RNG_STATE, kinds=kinds)[0]
        # first occurrences of a value as a corrective or trailing token end the run there
        firsts = [i for i in range(40) if free[i] not in free[:i].tolist()]
        extra = [next((i for i in firsts if kinds[i] == kd), 3) for kd in ("corrective", "trailing")]
        for cut in (3, 9, 17, 26, 34, *extra):
            stop = (int(free[cut]), 999)
            res_py = _step_loop_python(O.Session(tm, 512, 16), O.Session(dm, 512, 16), prompt, 40, 4, temp,
                                       O.REFERENCE_RNG_STATE, stop=stop)
            res_c = O.generate_speculative_draft_temp(O.Session(tm, 512, 16), O.Session(dm, 512, 16), prompt, 40,
                                                      4, temp, stop=stop)
            assert np.array_equal(res_py[0], res_c[0]), (draft_seed, temp, cut)
            assert res_py[1:5] == res_c[1:], (draft_seed, temp, cut)
            assert stop[0] not in res_c[0].tolist()
            if temp == 0.0:  # greedy: the stream is the unstopped one cut before the stop token
                first = free.tolist().index(stop[0])
                assert np.array_equal(res_c[0], free[:first]) and res_py[5] != "n_new"
            # (at temperature a stop token changes the draws that follow, so the run may not meet it)
            ends.add(res_py[5])
    assert ends >= {"accepted-stop", "corrective-stop", "trailing-stop"}, ends


def _plain_loop_python(s, prompt, n_new, temp, state, stop=(), max_ctx=512):
    """main.rs:9676-9706 prefill and the plain loop of main.rs:9894-9928, in Python."""
    n = len(prompt)
    for i in range(0, n - 1, 16):
        s.prefill_pass_batch(prompt[i:min(i + 16, n - 1)], i)
    lg, pos, out = s.forward_pass(prompt[-1], n - 1), n, []
    while True:
        t, state = O.sample_logits(lg, temp, state)
        if t in stop or pos >= max_ctx or len(out) >= n_new:
            break
        out.append(t)
        if len(out) >= n_new:
            break
        lg = s.forward_pass(t, pos)
        pos += 1
    return np.array(out, np.uint32), state


@pytest.mark.parametrize("temp", [0.0, 0.7, 1.3])
def test_plain_loop_matches_python_restatement(temp):
    """The oracle's plain decode loop with sampling and stop tokens against the restatement:
    same tokens and LCG state; greedy runs are the unstopped stream cut before the stop token;
    a context end stops the run too."""
    tm = _models(TINY, 71)
    prompt = nc.uniform_prompt(75, 20, 1000)
    free, st_free = O.generate_plain(O.Session(tm, 512, 16), prompt, 30, temp)
    assert len(free) == 30
    py, st_py = _plain_loop_python(O.Session(tm, 512, 16), prompt, 30, temp, O.REFERENCE_RNG_STATE)
    assert np.array_equal(free, py) and st_free == st_py
    if temp == 0.0:
        assert st_free == O.REFERENCE_RNG_STATE  # the argmax draws nothing
    for cut in (0, 7, 22):
        stop = (int(free[cut]),)
        got, st = O.generate_plain(O.Session(tm, 512, 16), prompt, 30, temp, stop=stop)
        py, st_py = _plain_loop_python(O.Session(tm, 512, 16), prompt, 30, temp, O.REFERENCE_RNG_STATE, stop)
        assert np.array_equal(got, py) and st == st_py
        first = free.tolist().index(stop[0])
        assert np.array_equal(got, free[:first])  # the draws before the stop are unchanged
    short, _ = O.generate_plain(O.Session(tm, 26, 16), prompt, 30, temp)
    assert np.array_equal(short, free[:6])  # positions 20..25: six tokens fit the context


def _ngram_loop_python(s, prompt, n_new, k, temp, state, stop=(), max_ctx=512, max_batch=16):
    """ngram_speculative_step (speculative.rs:122-286) driven by main.rs:9729-9776, in Python."""
    n = len(prompt)
    for i in range(0, n - 1, 16):
        s.prefill_pass_batch(prompt[i:min(i + 16, n - 1)], i)
    live = s.forward_pass(prompt[-1], n - 1)
    hist, pos, out, drafted, accepted, steps = list(prompt), n, [], 0, 0, 0
    while pos < max_ctx and len(out) < n_new:
        ck = min(k, n_new - len(out) - 1)  # a step emits at most the token budget
        t0, state = O.sample_logits(live, temp, state)
        if t0 in stop:
            break
        hist.append(t0)
        drafts = [int(t) for t in O.ngram_draft(hist, ck)] if ck > 0 else []
        drafts = drafts[:min(max_batch - 1, max_ctx - (pos + 1))]
        steps += 1
        if not drafts:
            live = s.forward_pass(t0, pos)
            out.append(t0)
            pos += 1
            continue
        drafted += len(drafts)
        s.prefill_pass_batch(np.array([t0] + drafts, np.uint32), pos)
        emitted, hit, done = [t0], False, False
        for i, d in enumerate(drafts):
            tt, state = O.sample_logits(s.batch_row_logits(i), temp, state)
            accepted += d == tt
            if tt in stop:  # neither emitted nor consumed
                hit, done, pos = True, True, pos + i + 1
                break
            emitted.append(tt)
            if d != tt:  # corrective forward
                live, pos, done = s.forward_pass(tt, pos + i + 1), pos + i + 2, True
                break
        if not done:
            live, pos = s.batch_row_logits(len(drafts)), pos + len(drafts) + 1
        hist += emitted[1:]
        out += emitted
        if hit:
            break
    return np.array(out, np.uint32), drafted, accepted, steps, state


def _ngram_kplus1_python(s, prompt, n_new, k, stop=(), max_ctx=512, max_batch=16):
    """The greedy n-gram loop in the k+1 verify form (cluster_tcp_smoke.rs:905-979: [pending] +
    drafts in one pass, next pending = pred[accepted]) with main.rs:9729-9776's budget clamp and
    ngram_speculative_step's stop handling (counting ends at a stop prediction), in Python."""
    n = len(prompt)
    for i in range(0, n - 1, 16):
        s.prefill_pass_batch(prompt[i:min(i + 16, n - 1)], i)
    pending = int(np.argmax(s.forward_pass(prompt[-1], n - 1)))
    hist, pos, out, drafted, accepted, steps = list(prompt), n, [], 0, 0, 0
    while len(out) < n_new and pending not in stop:
        out.append(pending)
        hist.append(pending)
        if len(out) >= n_new or pos + 1 >= max_ctx:
            break
        kk = min(k, n_new - len(out), max_batch - 1, max_ctx - pos - 1)
        drafts = [int(t) for t in O.ngram_draft(hist, kk)] if kk > 0 else []
        batch = [pending] + drafts
        s.prefill_pass_batch(np.array(batch, np.uint32), pos)
        pred = [int(np.argmax(s.batch_row_logits(i))) for i in range(len(batch))]
        a = 0
        while a < len(drafts) and drafts[a] == pred[a]:
            a += 1
        drafted, steps, counted, stopped = drafted + len(drafts), steps + 1, a, False
        for i in range(1, a + 1):
            if batch[i] in stop:
                counted, stopped = i, True
                break
            if len(out) < n_new:
                out.append(batch[i])
                hist.append(batch[i])
        accepted += counted
        pending, pos = pred[a], pos + a + 1
        if stopped:
            break
    return np.array(out, np.uint32), drafted, accepted, steps


@pytest.mark.parametrize("temp,prompt_seed", [(0.0, 77), (0.08, 78), (0.12, 79)])
def test_ngram_loop_matches_python_restatement(temp, prompt_seed):
    """The oracle's n-gram loops against Python restatements, with the budget clamp and stop
    tokens, on repetitive prompts where drafts are both accepted and rejected.  At temperature
    (the step form: t0 draw, one draw per verified row, corrective forward): same tokens,
    counts, steps and LCG state.  Greedy (the k+1 verify form): same tokens, counts and steps;
    the stream is the step form's and the plain greedy loop's, cut before a stop token."""
    tm = _models(TINY, 71)
    prompt = np.tile(nc.uniform_prompt(prompt_seed, 6, 1000), 8 if temp == 0.12 else 5)
    cases, base = [()], None
    while cases:
        stop = cases.pop(0)
        got = O.Session(tm, 512, 16).generate_speculative_ngram_temp(prompt, 40, 4, temp, stop=stop)
        step = _ngram_loop_python(O.Session(tm, 512, 16), prompt, 40, 4, temp, O.REFERENCE_RNG_STATE, stop)
        if temp > 0:
            assert np.array_equal(got[0], step[0]) and got[1:] == step[1:], stop
        else:
            k1 = _ngram_kplus1_python(O.Session(tm, 512, 16), prompt, 40, 4, stop)
            assert np.array_equal(got[0], k1[0]) and got[1:4] == k1[1:], stop
            assert np.array_equal(got[0], step[0]) and got[4] == O.REFERENCE_RNG_STATE, stop
        if base is None:
            base = got
            cases = [(int(base[0][c]),) for c in (2, 11, 30)]
        else:
            assert stop[0] not in got[0].tolist()
    toks, drafted, acc = base[:3]
    assert 0 < acc < drafted
    if temp == 0.0:
        plain, _ = O.generate_plain(O.Session(tm, 512, 16), prompt, 40, 0.0)
        assert np.array_equal(toks, plain)
        for c in (2, 11, 30):
            st = int(toks[c])
            cut = O.Session(tm, 512, 16).generate_speculative_ngram(prompt, 40, 4, stop=(st,))[0]
            assert np.array_equal(cut, toks[:toks.tolist().index(st)])


# ---------------------------------------------------------------- pins fixed by the mathematics
_LCG_A = 6364136223846793005
_LCG_A_INV = pow(_LCG_A, -1, 1 << 64)


def _state_drawing(x: int) -> int:
    """The LCG state whose next draw has upper word x (rand_simple then returns f32(x) / 2^32)."""
    return ((((x << 32) - 1) * _LCG_A_INV) % (1 << 64))


def test_lcg_state_construction():
    for x in (0, 1, 2**31, 2**32 - 1):
        u, _ = O.rand_simple(_state_drawing(x))
        assert F(u) == F(np.uint32(x)) / F(4294967295)


# Hand-worked walks: logits whose exponentials are exact (equal logits give e = 1, a logit 1000
# below the maximum gives expf(-1000) = 0), so S and every r are exact and the boundary u·S = a
# prefix sum can be hit on the nose.  The walk r -= e_i, stop at the first r <= 0.
@pytest.mark.parametrize("logits,temp,x,want", [
    # V = 2, e = [1, 1], S = 2: r = 2u; u = 1/2 gives r - 1 = 0 <= 0 -> id 0 (on the boundary)
    ([0.0, 0.0], 1.0, 2**31, 0),
    ([0.0, 0.0], 1.0, 2**31 - 128, 0),      # u just below 1/2: r - 1 < 0 -> id 0
    ([0.0, 0.0], 1.0, 2**31 + 256, 1),      # u just above 1/2 (next f32): r - 1 > 0 -> id 1
    ([0.0, 0.0], 0.25, 2**31 + 256, 1),     # temperature does not move equal logits
    ([0.0, 0.0], 1.0, 0, 0),                # u = 0: r = 0 <= 0 at the first step
    ([0.0, 0.0], 1.0, 2**32 - 1, 1),        # u = 1 (x rounds to 2^32): r = 2 - 1 - 1 = 0 -> last id
    # V = 3, e = [1, 0, 1], S = 2: the zero-mass id 1 is never returned; above the first
    # boundary the walk passes it (r stays > 0) and stops at id 2
    ([0.0, -1000.0, 0.0], 1.0, 2**31, 0),
    ([0.0, -1000.0, 0.0], 1.0, 2**31 + 256, 2),
    # V = 3, e = [1, 1, 1], S = 3: r = fl(3u); u = f32(1/3) = 11184811 * 2^-25 gives
    # 3u = 1 + 2^-25 -> r = 1.0 -> id 0; the next f32 above gives r = 1 + 2^-23 -> id 1;
    # u = f32(2/3) = 11184811 * 2^-24: 3u = 2 + 2^-24 -> r = 2.0 -> id 1; next above -> id 2
    ([0.0, 0.0, 0.0], 1.0, 1431655808, 0),
    ([0.0, 0.0, 0.0], 1.0, 1431655808 + 128, 1),
    ([0.0, 0.0, 0.0], 1.0, 2863311616, 1),
    ([0.0, 0.0, 0.0], 1.0, 2863311616 + 256, 2),
])
def test_sample_logits_hand_worked_boundaries(logits, temp, x, want):
    st0 = _state_drawing(x)
    i, st = O.sample_logits(np.array(logits, F), temp, st0)
    assert i == want
    assert st == (st0 * _LCG_A + 1) % (1 << 64)  # exactly one draw


def _chi2_pvalue(counts, p):
    from scipy import stats
    exp = p * counts.sum()
    return stats.chi2.sf(float(((counts - exp) ** 2 / exp).sum()), len(p) - 1)


@pytest.mark.parametrize("temp", [0.7, 1.3])
def test_sample_logits_frequencies_follow_softmax(temp):
    # the distribution sample_logits draws from is softmax(l / T): chi-square over 60000 draws
    # of the reference's LCG, against float64 softmax; a planted mistake (the temperature
    # dropped) is rejected by the same statistic
    l = np.array([1.0, 0.5, 0.0, -0.5, 2.0, -1.0], F)
    st, counts = O.REFERENCE_RNG_STATE, np.zeros(len(l))
    for _ in range(60000):
        i, st = O.sample_logits(l, temp, st)
        counts[i] += 1
    z = l.astype(np.float64) / temp
    p = np.exp(z - z.max())
    p /= p.sum()
    assert _chi2_pvalue(counts, p) > 1e-4
    q = np.exp(l.astype(np.float64) - l.max())
    q /= q.sum()
    assert _chi2_pvalue(counts, q) < 1e-12
