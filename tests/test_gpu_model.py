"""End-to-end parity of the GPU verify path against the CPU oracle.

Logits of every verify row must be bit-identical to the oracle's (hence fp32 within
1e-3 and identical argmax); greedy and speculative token streams must be identical
to the oracle's streams; a draft identical to the target must be accepted every time.
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
    assert torch.cuda.is_available()
    return nc.Context(0)


def _models(ctx, spec, seed):
    import nanocamelid_amd as nc
    img = nc.synth_gguf(**spec, seed=seed)
    return img, nc.Model(ctx, data=img), O.Model(data=img.tobytes(), nthreads=16)


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("hd", [64, 128])
def test_verify_logits_bit_exact(ctx, hd):
    import nanocamelid_amd as nc
    spec = dict(TINY, head_count=256 // hd * 2, head_count_kv=256 // hd, embedding_length=512)
    _, gm, om = _models(ctx, spec, seed=hd)
    gs = nc.Session(gm, 256, 16)
    os_ = O.Session(om, 256, 16)
    toks = nc.uniform_prompt(5, 150, 1000)
    pos = 0
    for n in (16, 16, 5, 1, 9, 16, 3, 16, 16, 16, 13):  # crosses several 64-position tiles
        batch = toks[pos:pos + n] if pos + n <= len(toks) else nc.uniform_prompt(pos, n, 1000)
        a, nxt, newpos, preds = gs.verify_greedy(batch, pos)
        opreds, _, ologits = os_.verify_greedy(batch, pos, want_logits=True)
        for i in range(n):
            assert _same(gs.logits(i), ologits[i]), (pos, i)
        assert np.array_equal(preds, opreds)
        acc = 0
        while acc < n - 1 and batch[acc + 1] == opreds[acc]:
            acc += 1
        assert a == acc and nxt == opreds[acc] and newpos == pos + acc + 1
        pos += n


def test_verify_every_width(ctx):
    """Every verify width 1..16 once (each width has its own GEMM, SwiGLU-epilogue and
    attention instantiations): all rows' logits bit-identical to the oracle's."""
    import nanocamelid_amd as nc
    _, gm, om = _models(ctx, TINY, seed=31)
    gs = nc.Session(gm, 256, 16)
    os_ = O.Session(om, 256, 16)
    pos = 0
    for n in range(1, 17):
        batch = nc.uniform_prompt(100 + n, n, 1000)
        a, nxt, newpos, preds = gs.verify_greedy(batch, pos)
        opreds, _, ologits = os_.verify_greedy(batch, pos, want_logits=True)
        for i in range(n):
            assert _same(gs.logits(i), ologits[i]), (n, i)
        assert np.array_equal(preds, opreds), n
        pos += n


def test_hidden_and_forward_pass_match(ctx):
    import nanocamelid_amd as nc
    _, gm, om = _models(ctx, TINY, seed=4)
    gs = nc.Session(gm, 64, 1)
    os_ = O.Session(om, 64, 1)
    for i, t in enumerate(nc.uniform_prompt(9, 20, 1000)):
        pred, lg = gs.forward_pass(t, i)
        olg = os_.forward_pass(t, i)
        assert _same(lg, olg) and pred == int(np.argmax(olg))


def test_greedy_and_speculative_streams(ctx):
    import nanocamelid_amd as nc
    _, gm, om = _models(ctx, TINY, seed=31)
    prompt = nc.uniform_prompt(77, 24, 1000)
    ref = O.Session(om, 400, 16).generate_greedy(prompt, 96)
    out, st = nc.Session(gm, 400, 16).generate_greedy(prompt, 96)
    assert np.array_equal(out, ref)
    for k, alpha in ((2, 0.5), (4, 0.8), (8, 0.8), (4, 1.0)):
        g_out, st = nc.Session(gm, 400, 16).generate_speculative_oracle(prompt, 96, k, alpha, 1234, ref)
        o_out, drafted, accepted, steps = O.Session(om, 400, 16).generate_speculative_oracle(prompt, 96, k, alpha,
                                                                                             1234, ref)
        assert np.array_equal(g_out, ref) and np.array_equal(o_out, ref)
        assert (st.drafted, st.accepted, st.steps) == (drafted, accepted, steps)


def test_ngram_speculation_streams(ctx):
    # ngram_speculative_step (speculative.rs:122-286), k+1 form: same stream, drafts, acceptances
    # and steps as the oracle; the stream is the greedy stream cut before the first stop token
    import nanocamelid_amd as nc
    _, gm, om = _models(ctx, TINY, seed=21)
    base = nc.uniform_prompt(9, 6, 1000)
    prompt = np.concatenate([base, base, base, nc.uniform_prompt(10, 4, 1000), base[:4]]).astype(np.uint32)
    ref = O.Session(om, 256, 16).generate_greedy(prompt, 64)
    for k, mn, mx in ((1, 3, 4), (4, 3, 4), (8, 2, 5), (15, 3, 4)):
        print(f"ngram k={k} n={mn}..{mx}", flush=True)
        g_out, st = nc.Session(gm, 256, 16).generate_speculative_ngram(prompt, 64, k, mn, mx)
        o_out, drafted, accepted, steps = O.Session(om, 256, 16).generate_speculative_ngram(prompt, 64, k, mn, mx)
        assert np.array_equal(g_out, ref) and np.array_equal(o_out, ref), k
        assert (st.drafted, st.accepted, st.steps) == (drafted, accepted, steps), k
        assert drafted > 0 and accepted > 0
    stop = [int(ref[20]), 999999]
    g_out, _ = nc.Session(gm, 256, 16).generate_speculative_ngram(prompt, 64, 4, stop=stop)
    o_out, _, _, _ = O.Session(om, 256, 16).generate_speculative_ngram(prompt, 64, 4, stop=stop)
    assert np.array_equal(g_out, o_out)
    assert np.array_equal(g_out, ref[:int(np.where(ref == ref[20])[0][0])])


def test_draft_model_speculation(ctx):
    import nanocamelid_amd as nc
    _, gm, om = _models(ctx, TINY, seed=32)
    prompt = nc.uniform_prompt(78, 20, 1000)
    ref = O.Session(om, 300, 16).generate_greedy(prompt, 60)
    out, st = nc.generate_speculative_draft(nc.Session(gm, 300, 16), nc.Session(gm, 300, 4), prompt, 60, 4)
    assert np.array_equal(out, ref)
    assert st.accepted == st.drafted and st.drafted > 0


def test_q4_k_model_logits(ctx):
    import nanocamelid_amd as nc
    spec = dict(layers=2, embedding_length=512, head_count=4, head_count_kv=2, feed_forward_length=1024,
                vocab_size=777, weight_type=nc.NC_TYPE_Q4_K, tied=1, context_length=256, norm_mode=1)
    _, gm, om = _models(ctx, spec, seed=12)
    gs, os_ = nc.Session(gm, 128, 16), O.Session(om, 128, 16)
    toks = nc.uniform_prompt(2, 40, 777)
    for pos, n in ((0, 16), (16, 16), (32, 8)):
        _, _, _, preds = gs.verify_greedy(toks[pos:pos + n], pos)
        opreds, _, ologits = os_.verify_greedy(toks[pos:pos + n], pos, want_logits=True)
        assert np.array_equal(preds, opreds)
        for i in range(n):
            assert _same(gs.logits(i), ologits[i])


@pytest.mark.parametrize("hd,checks", [(128, (2045, 4093)), (64, (8190,)), (128, (510, 765, 1021, 1277, 1533)),
                                       (64, (766, 1534))],
                         ids=["hd128-4k", "hd64-8k", "hd128-fused-tiers", "hd64-fused-tiers"])
def test_long_context_logits(ctx, hd, checks):
    """Verify logits bit-exact at long contexts: 5-row passes that straddle the softmax
    instantiation boundaries at 2048, 4096 and 8192 positions (the 8192 one switches the
    softmax to 512 threads), and the single-kernel attention's row tiers (512, 768, 1024,
    1280 and 1536 positions; past 1536 two kernels)."""
    import nanocamelid_amd as nc
    upto = checks[-1] + 5
    spec = dict(layers=1, embedding_length=2 * hd * 2, head_count=4, head_count_kv=2, feed_forward_length=512,
                vocab_size=1000, context_length=upto + 64, tied=1, norm_mode=1)
    _, gm, om = _models(ctx, spec, seed=hd)
    prompt = nc.uniform_prompt(hd, upto, 1000)
    gs, os_ = nc.Session(gm, upto + 16, 16), O.Session(om, upto + 16, 16)
    pos = 0
    for c in checks:
        print(f"long context hd={hd}: prefill to {c}, verify 5 rows", flush=True)
        gs.prefill_pass_batch(prompt[pos:c], pos)
        for i in range(pos, c, 16):
            os_.prefill_pass_batch(prompt[i:min(i + 16, c)], i)
        batch = nc.uniform_prompt(c, 5, 1000)
        _, _, _, preds = gs.verify_greedy(batch, c)
        opreds, _, ologits = os_.verify_greedy(batch, c, want_logits=True)
        assert np.array_equal(preds, opreds)
        for i in range(5):
            assert _same(gs.logits(i), ologits[i]), (c, i)
        pos = c


@pytest.mark.slow
def test_config0_plumbing_run(ctx):
    """Config 0: Llama-3.2-1B shape, tied Q4_0 head, 32-token seeded prompt, greedy, k=4,
    64 new tokens, draft = the same model: GPU stream == oracle stream, acceptance 1.0."""
    import nanocamelid_amd as nc
    spec = dict(nc.SYNTH_CONFIGS["llama-3.2-1b"], context_length=8192)
    img = nc.synth_gguf(**spec, seed=2024)
    gm = nc.Model(ctx, data=img)
    prompt = nc.uniform_prompt(2024, 32, 128256)
    out, st = nc.generate_speculative_draft(nc.Session(gm, 256, 16), nc.Session(gm, 256, 4), prompt, 64, 4)
    assert st.accepted == st.drafted
    om = O.Model(data=img.tobytes(), nthreads=16)
    ref, drafted, accepted, steps = O.generate_speculative_draft(O.Session(om, 256, 16), O.Session(om, 256, 4),
                                                                 prompt, 64, 4)
    assert accepted == drafted
    assert np.array_equal(out, ref)
