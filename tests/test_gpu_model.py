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

# Untied: a tied N(0, 0.02) head keeps predicting the last input token, so its streams would
# repeat one id and stream checks would be near-vacuous.  Every checked stream has a floor of
# distinct ids.
TINY = dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512, vocab_size=1000,
            context_length=512, tied=0, norm_mode=1)
MIN_DISTINCT = 8


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


@pytest.mark.parametrize("hd,tied", [(64, 1), (128, 0)])
def test_verify_logits_bit_exact(ctx, hd, tied):
    import nanocamelid_amd as nc
    spec = dict(TINY, head_count=256 // hd * 2, head_count_kv=256 // hd, embedding_length=512, tied=tied)
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


def test_verify_every_width_mfma_path(ctx):
    """The int8 MFMA dot path through every epilogue of a model pass (fused q,k,v with RoPE into
    the KV cache, residual, the four-tile SwiGLU + Q8_0, the head): logits bit-identical to the
    oracle's at every verify width."""
    import nanocamelid_amd as nc
    mctx = nc.Context(0)
    mctx.set_gemm_kernel(nc._ffi.NC_GEMM_KERNEL_MFMA)
    _, gm, om = _models(mctx, TINY, seed=33)
    gs = nc.Session(gm, 256, 16)
    os_ = O.Session(om, 256, 16)
    pos = 0
    for n in (1, 4, 5, 8, 9, 13, 16):
        batch = nc.uniform_prompt(200 + n, n, 1000)
        _, _, _, preds = gs.verify_greedy(batch, pos)
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
    assert len(set(ref.tolist())) >= MIN_DISTINCT
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
    assert len(set(ref.tolist())) >= MIN_DISTINCT
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
    _, gm, om = _models(ctx, TINY, seed=21)
    prompt = nc.uniform_prompt(78, 20, 1000)
    ref = O.Session(om, 300, 16).generate_greedy(prompt, 60)
    assert len(set(ref.tolist())) >= MIN_DISTINCT
    out, st = nc.generate_speculative_draft(nc.Session(gm, 300, 16), nc.Session(gm, 300, 4), prompt, 60, 4)
    assert np.array_equal(out, ref)
    assert st.accepted == st.drafted and st.drafted > 0


def test_draft_model_rejection_path(ctx):
    """speculative_decoding_step (speculative.rs:384-447) with a draft that disagrees part of the
    time (the target's weights with unit norm weights): corrective tokens, the corrective
    forwards on both models and pos = at + 1 all run.  GPU stream == oracle stream == target
    greedy stream, identical statistics, 0 < accepted < drafted."""
    import nanocamelid_amd as nc
    img, gm, om = _models(ctx, TINY, seed=21)
    dimg = nc.synth_gguf(**dict(TINY, norm_mode=0), seed=21)
    dm, odm = nc.Model(ctx, data=dimg), O.Model(data=dimg.tobytes())
    prompt = nc.uniform_prompt(78, 20, 1000)
    ref = O.Session(om, 300, 16).generate_greedy(prompt, 60)
    for k in (1, 4, 8):
        out, st = nc.generate_speculative_draft(nc.Session(gm, 300, 16), nc.Session(dm, 300, 8), prompt, 60, k)
        o_out, drafted, accepted, steps = O.generate_speculative_draft(O.Session(om, 300, 16), O.Session(odm, 300, 8),
                                                                       prompt, 60, k)
        assert np.array_equal(out, ref) and np.array_equal(o_out, ref), k
        assert (st.drafted, st.accepted, st.steps) == (drafted, accepted, steps), k
        assert 0 < st.accepted < st.drafted, k


def test_error_contract_keeps_session_usable(ctx):
    """Bounds the reference enforces by panicking come back as NC_ERANGE / NC_EINVAL before any
    launch, and the session still verifies bit-exactly afterwards."""
    import nanocamelid_amd as nc
    from nanocamelid_amd import NcError
    _, gm, om = _models(ctx, TINY, seed=4)
    gs, os_ = nc.Session(gm, 128, 16), O.Session(om, 128, 16)
    toks = nc.uniform_prompt(3, 21, 1000)
    gs.prefill_pass_batch(toks[:16], 0)
    os_.prefill_pass_batch(toks[:16], 0)
    bad = toks[16:].copy()
    bad[2] = 1000  # == vocab_size (inference.rs:3728-3733 panics on the embedding index)
    for call in (lambda: gs.verify_greedy(bad, 16), lambda: gs.forward_pass(5000, 16),
                 lambda: gs.prefill_pass_batch(bad, 16),
                 lambda: gs.generate_speculative_oracle(toks[:8], 8, 4, 0.8, 1, np.array([1, 2, 1000], np.uint32))):
        with pytest.raises(NcError) as e:
            call()
        assert e.value.code == nc._ffi.NC_ERANGE
    with pytest.raises(NcError) as e:  # a session longer than the attention kernels' rows
        nc.Session(nc.Model(ctx, data=nc.synth_gguf(**dict(TINY, context_length=20000), seed=4)), 16385, 4)
    assert e.value.code == nc._ffi.NC_ERANGE
    other = nc.Model(ctx, data=nc.synth_gguf(**dict(TINY, vocab_size=999), seed=4))
    with pytest.raises(NcError) as e:  # draft ids index the target's embedding
        nc.generate_speculative_draft(gs, nc.Session(other, 128, 4), toks[:8], 8, 4)
    assert e.value.code == nc._ffi.NC_EINVAL
    _, _, _, preds = gs.verify_greedy(toks[16:], 16)
    opreds, _, ologits = os_.verify_greedy(toks[16:], 16, want_logits=True)
    assert np.array_equal(preds, opreds)
    for i in range(5):
        assert _same(gs.logits(i), ologits[i]), i


def test_prefill_without_logits_then_verify(ctx):
    """nc_prefill with want_logits = 0 runs no head pass: the KV written is the same and the
    following verify is still bit-identical; with want_logits = 1 the last chunk's logits are
    readable and equal the oracle's."""
    import nanocamelid_amd as nc
    _, gm, om = _models(ctx, TINY, seed=9)
    toks = nc.uniform_prompt(12, 45, 1000)
    gs, os_ = nc.Session(gm, 128, 16), O.Session(om, 128, 16)
    gs.prefill_pass_batch(toks[:40], 0, want_logits=False)
    for i in range(0, 40, 16):
        os_.prefill_pass_batch(toks[i:min(i + 16, 40)], i)
    _, _, _, preds = gs.verify_greedy(toks[40:], 40)
    opreds, _, ologits = os_.verify_greedy(toks[40:], 40, want_logits=True)
    assert np.array_equal(preds, opreds)
    for i in range(5):
        assert _same(gs.logits(i), ologits[i]), i
    gs2, os2 = nc.Session(gm, 128, 16), O.Session(om, 128, 16)
    gs2.prefill_pass_batch(toks[:20], 0)  # want_logits = 1: rows of the last chunk (16..19)
    os2.prefill_pass_batch(toks[:16], 0)
    os2.prefill_pass_batch(toks[16:20], 16)
    for i in range(4):
        assert _same(gs2.logits(i), os2.batch_row_logits(i)), i


def test_rope_scaling_model_logits(ctx):
    """A Llama-3.1/3.2-style file with llama.rope.scaling.* keys: the host RoPE table applies the
    frequency scaling of cached_rope_angles (inference.rs:875-893) and the logits stay
    bit-identical to the oracle's across several positions."""
    import nanocamelid_amd as nc
    spec = dict(TINY, rope_freq_base=10000.0, rope_scaling=(8.0, 64, 1.0, 4.0))
    _, gm, om = _models(ctx, spec, seed=17)
    assert gm.config["rope_scaling"] == 1 and gm.config["rope_scaling_factor"] == 8.0
    gs, os_ = nc.Session(gm, 256, 16), O.Session(om, 256, 16)
    toks = nc.uniform_prompt(8, 100, 1000)
    for pos in range(0, 96, 16):
        _, _, _, preds = gs.verify_greedy(toks[pos:pos + 16], pos)
        opreds, _, ologits = os_.verify_greedy(toks[pos:pos + 16], pos, want_logits=True)
        assert np.array_equal(preds, opreds)
        for i in range(16):
            assert _same(gs.logits(i), ologits[i]), (pos, i)


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


@pytest.mark.parametrize("hd,wt", [(64, 2), (128, 2), (128, 12), (128, 8), (64, 13)],
                         ids=["hd64-q4_0", "hd128-q4_0", "hd128-q4_k", "hd128-q8_0", "hd64-q5_k"])
def test_prompt_passes_match_oracle(ctx, hd, wt):
    """Prompts of 32 or more tokens on Q4_0 and Q4_K models run as MFMA prompt passes of up to
    256 tokens, Q8_0 and Q5_K models as the same passes with their matmuls in 16-token slices of the
    verify kernel (epilogues as separate kernels, attention in 64-row groups): a 300-token prompt
    without logits (passes of 256 + 44) and 400 more with logits (passes of 256 + 128, then the
    last 16 rows as a verify-sized pass), then a 9-row verify: every logit bit-identical to the
    oracle's after 16-token chunks, i.e. the same KV cache bits."""
    import nanocamelid_amd as nc
    spec = dict(TINY, head_count=512 // hd, head_count_kv=256 // hd, embedding_length=512, context_length=1024,
                weight_type=wt)
    _, gm, om = _models(ctx, spec, seed=40 + hd)
    prompt = nc.uniform_prompt(41, 700, 1000)
    gs, os_ = nc.Session(gm, 1024, 16), O.Session(om, 1024, 16)
    gs.prefill_pass_batch(prompt[:300], 0, want_logits=False)
    gs.prefill_pass_batch(prompt[300:700], 300)
    for i in range(0, 700, 16):
        os_.prefill_pass_batch(prompt[i:min(i + 16, 700)], i)
    batch = nc.uniform_prompt(700, 9, 1000)
    _, _, _, preds = gs.verify_greedy(batch, 700)
    opreds, _, ologits = os_.verify_greedy(batch, 700, want_logits=True)
    assert np.array_equal(preds, opreds)
    for i in range(9):
        assert _same(gs.logits(i), ologits[i]), i


@pytest.mark.parametrize("ty", [1, 30, 8, 3, 6, 13, 14])
def test_embedding_types_model_logits(ctx, ty):
    """Token embeddings stored as F16, BF16, Q8_0, Q4_1, Q5_0, Q5_K or Q6_K (load_f32_or_f16,
    model.rs:1081-1229) load through the memory-mapped file path and give logits bit-identical
    to the oracle's, which decodes them independently."""
    import os
    import tempfile
    import nanocamelid_amd as nc
    from tests import gguf_writer as GW
    meta, ts = GW.read(nc.synth_gguf(**TINY, seed=50 + ty).tobytes())
    d, V = TINY["embedding_length"], TINY["vocab_size"]
    raw = GW.random_blocks(ty, d * V // GW.LAYOUT[ty][0], seed=ty).tobytes()
    ts = [("token_embd.weight", [d, V], ty, raw) if t[0] == "token_embd.weight" else t for t in ts]
    img = GW.write(meta, ts)
    with tempfile.NamedTemporaryFile(suffix=".gguf", delete=False) as f:
        f.write(img)
    try:
        gm = nc.Model(ctx, path=f.name)
    finally:
        os.unlink(f.name)
    om = O.Model(data=img)
    gs, os_ = nc.Session(gm, 64, 16), O.Session(om, 64, 16)
    toks = nc.uniform_prompt(ty, 12, V)
    _, _, _, preds = gs.verify_greedy(toks, 0)
    opreds, _, ologits = os_.verify_greedy(toks, 0, want_logits=True)
    assert np.array_equal(preds, opreds)
    for i in range(12):
        assert _same(gs.logits(i), ologits[i]), i


def test_q6_k_head_model_logits(ctx):
    """An untied Q6_K output.weight (llama.cpp keeps the head in Q6_K in its Q4_0 and Q4_K_M
    files): verify logits and greedy predictions bit-identical to the oracle at several widths."""
    import nanocamelid_amd as nc
    from tests import gguf_writer as GW
    meta, ts = GW.read(nc.synth_gguf(**TINY, seed=61).tobytes())
    d, V = TINY["embedding_length"], TINY["vocab_size"]
    raw = GW.random_blocks(nc.NC_TYPE_Q6_K, d * V // 256, seed=61).tobytes()
    ts = [("output.weight", [d, V], nc.NC_TYPE_Q6_K, raw) if t[0] == "output.weight" else t for t in ts]
    img = GW.write(meta, ts)
    gm, om = nc.Model(ctx, data=np.frombuffer(img, np.uint8)), O.Model(data=img)
    gs, os_ = nc.Session(gm, 128, 16), O.Session(om, 128, 16)
    pos = 0
    for n in (1, 5, 16, 9):
        batch = nc.uniform_prompt(300 + n, n, V)
        _, _, _, preds = gs.verify_greedy(batch, pos)
        opreds, _, ologits = os_.verify_greedy(batch, pos, want_logits=True)
        assert np.array_equal(preds, opreds), n
        for i in range(n):
            assert _same(gs.logits(i), ologits[i]), (n, i)
        pos += n


def test_q8_0_model_logits(ctx):
    """A Q8_0 model (llama.cpp's Q8_0 files: every layer matrix and the untied head in Q8_0,
    matmul_q8_0_batch inference.rs:1343-1383): fused q,k,v with RoPE, the interleaved gate,up
    with SwiGLU + Q8_0 and the residual epilogues on the 64-row Q8_0 kernel; verify logits and
    predictions bit-identical to the oracle at widths 1, 5, 16, 9."""
    import nanocamelid_amd as nc
    from tests import gguf_writer as GW
    spec = dict(TINY, tied=0, weight_type=nc.NC_TYPE_Q8_0)
    meta, ts = GW.read(nc.synth_gguf(**spec, seed=71).tobytes())
    d, V = TINY["embedding_length"], TINY["vocab_size"]
    raw = GW.random_blocks(nc.NC_TYPE_Q8_0, d * V // 32, seed=71).tobytes()
    ts = [("output.weight", [d, V], nc.NC_TYPE_Q8_0, raw) if t[0] == "output.weight" else t for t in ts]
    img = GW.write(meta, ts)
    gm, om = nc.Model(ctx, data=np.frombuffer(img, np.uint8)), O.Model(data=img)
    assert gm.config["weight_type"] == nc.NC_TYPE_Q8_0
    gs, os_ = nc.Session(gm, 128, 16), O.Session(om, 128, 16)
    pos = 0
    for n in (1, 5, 16, 9):
        batch = nc.uniform_prompt(400 + n, n, V)
        _, _, _, preds = gs.verify_greedy(batch, pos)
        opreds, _, ologits = os_.verify_greedy(batch, pos, want_logits=True)
        assert np.array_equal(preds, opreds), n
        for i in range(n):
            assert _same(gs.logits(i), ologits[i]), (n, i)
        pos += n


def test_q5_k_model_logits(ctx):
    """A Q5_K model (the layer matrices of llama.cpp's Q5_K_M files; matmul_q5_k_batch
    inference.rs:2513-2640) and a Q4_0 output.weight: fused q,k,v, the
    interleaved gate,up and the residual epilogues on the 64-row K-quant kernel; verify logits
    and predictions bit-identical to the oracle at widths 1, 5, 16, 9."""
    import nanocamelid_amd as nc
    spec = dict(TINY, weight_type=nc.NC_TYPE_Q5_K)
    _, gm, om = _models(ctx, spec, seed=81)
    assert gm.config["weight_type"] == nc.NC_TYPE_Q5_K
    gs, os_ = nc.Session(gm, 128, 16), O.Session(om, 128, 16)
    V = TINY["vocab_size"]
    pos = 0
    for n in (1, 5, 16, 9):
        batch = nc.uniform_prompt(500 + n, n, V)
        _, _, _, preds = gs.verify_greedy(batch, pos)
        opreds, _, ologits = os_.verify_greedy(batch, pos, want_logits=True)
        assert np.array_equal(preds, opreds), n
        for i in range(n):
            assert _same(gs.logits(i), ologits[i]), (n, i)
        pos += n


@pytest.mark.parametrize("base", ["q4_k", "q4_0"])
def test_mixed_type_layers_model_logits(ctx, base):
    """Layers whose matrices differ in type, as in llama.cpp's Q4_K_M files (attn_v and ffn_down
    in Q6_K on some layers): q,k,v and gate,up that no longer share one type run as separate
    matmuls storing plain rows, followed by the RoPE / cache and SwiGLU kernels, and Q6_K
    attn_output / ffn_down add their rows to the residual in a separate kernel.  A 40-token
    prefill (one prompt pass: split matmuls on the MFMA prompt kernels, Q6_K ones in 16-row
    slices), then verify logits and greedy predictions bit-identical to the oracle at widths
    1, 5, 16 and 9."""
    import nanocamelid_amd as nc
    from tests import gguf_writer as GW
    from tests.test_reference_forward import mixed_model_image, MIXED_SPEC
    if base == "q4_k":
        img, V = mixed_model_image(), MIXED_SPEC["vocab_size"]
    else:
        types = {"blk.0.attn_v.weight": 14, "blk.0.ffn_up.weight": 14, "blk.1.ffn_down.weight": 14,
                 "blk.1.attn_output.weight": 14}
        img = np.frombuffer(GW.with_types(nc.synth_gguf(**TINY, seed=29), types, seed=29), np.uint8)
        V = TINY["vocab_size"]
    gm, om = nc.Model(ctx, data=img), O.Model(data=img.tobytes())
    gs, os_ = nc.Session(gm, 128, 16), O.Session(om, 128, 16)
    prompt = nc.uniform_prompt(31, 40, V)
    gs.prefill_pass_batch(prompt, 0, want_logits=False)
    for i in range(0, 40, 16):
        os_.prefill_pass_batch(prompt[i:i + 16], i)
    pos = 40
    for n in (1, 5, 16, 9):
        batch = nc.uniform_prompt(400 + n, n, V)
        _, _, _, preds = gs.verify_greedy(batch, pos)
        opreds, _, ologits = os_.verify_greedy(batch, pos, want_logits=True)
        assert np.array_equal(preds, opreds), n
        for i in range(n):
            assert _same(gs.logits(i), ologits[i]), (n, i)
        pos += n
    assert len(set(preds.tolist())) >= 3


def test_loader_refuses_output_major_matrix(ctx):
    import nanocamelid_amd as nc
    from tests import gguf_writer as GW
    meta, ts = GW.read(nc.synth_gguf(**TINY, seed=5).tobytes())
    # attn_k is [d, kv_width] = [256, 128]: stored output-major it reads [128, 256]
    ts = [(n, [dims[1], dims[0]], ty, raw) if n == "blk.0.attn_k.weight" else (n, dims, ty, raw)
          for n, dims, ty, raw in ts]
    with pytest.raises(nc.NcError, match="transposed"):
        nc.Model(ctx, data=np.frombuffer(GW.write(meta, ts), np.uint8))


def test_long_context_many_units(ctx):
    """Long rows with more (row, head) units than CUs (9 rows x 32 heads = 288) take the
    256-thread softmax tiers and the software-pipelined weighted-V loop: 9-row verify logits
    bit-exact vs the oracle past 1536 and past 2048 positions (the 8192-position tier is
    checked against single-row passes in the 70B-shape configuration test)."""
    import nanocamelid_amd as nc
    spec = dict(layers=1, embedding_length=32 * 64, head_count=32, head_count_kv=8, feed_forward_length=512,
                vocab_size=1000, context_length=2048 + 128, tied=1, norm_mode=1)
    _, gm, om = _models(ctx, spec, seed=288)
    prompt = nc.uniform_prompt(288, 2100, 1000)
    gs, os_ = nc.Session(gm, 2160, 16), O.Session(om, 2160, 16)
    pos = 0
    for c in (1600, 2100):
        print(f"many units: prefill to {c}, verify 9 rows", flush=True)
        gs.prefill_pass_batch(prompt[pos:c], pos)
        for i in range(pos, c, 16):
            os_.prefill_pass_batch(prompt[i:min(i + 16, c)], i)
        batch = nc.uniform_prompt(c, 9, 1000)
        _, _, _, preds = gs.verify_greedy(batch, c)
        opreds, _, ologits = os_.verify_greedy(batch, c, want_logits=True)
        assert np.array_equal(preds, opreds)
        for i in range(9):
            assert _same(gs.logits(i), ologits[i]), (c, i)
        pos = c


@pytest.mark.parametrize("hd", [64, 128])
def test_long_prompt_many_unit_tiers_vs_oracle(ctx, hd):
    """A 4300-token prompt on a two-layer model with 8 query heads: its prompt passes run the
    attention of 64-row groups (512 (row, head) units) through the one-kernel tiers, then the
    256-thread softmax tiers at up to 2048, 4096 and 8192 positions with the software-pipelined
    weighted-V loop.  Layer 0's attention outputs feed layer 1's keys and values, so a 9-row
    verify at 4300 whose every logit is bit-identical to the oracle's (16-token chunks) pins
    those tiers."""
    import nanocamelid_amd as nc
    spec = dict(layers=2, embedding_length=8 * hd, head_count=8, head_count_kv=2, feed_forward_length=512,
                vocab_size=1000, context_length=4400, tied=1, norm_mode=1)
    _, gm, om = _models(ctx, spec, seed=4300 + hd)
    n = 4300
    prompt = nc.uniform_prompt(4300 + hd, n, 1000)
    gs, os_ = nc.Session(gm, n + 16, 16), O.Session(om, n + 16, 16)
    print(f"long prompt hd={hd}: {n} tokens in prompt passes", flush=True)
    gs.prefill_pass_batch(prompt, 0, want_logits=False)
    for i in range(0, n, 16):
        os_.prefill_pass_batch(prompt[i:min(i + 16, n)], i)
    batch = nc.uniform_prompt(n, 9, 1000)
    _, _, _, preds = gs.verify_greedy(batch, n)
    opreds, _, ologits = os_.verify_greedy(batch, n, want_logits=True)
    assert np.array_equal(preds, opreds)
    for i in range(9):
        assert _same(gs.logits(i), ologits[i]), i


def test_long_context_many_units_past_8192(ctx):
    """9 rows x 32 heads (288 units) at 8193..8201 positions take the 256-thread tier with one
    extra position per thread (its e joins the exact chain after the first 8192): every verify
    row's logits equal single-row passes at the same positions, which take the 512-thread tier
    that the oracle pins at 8190 positions (test_long_context_logits)."""
    import nanocamelid_amd as nc
    spec = dict(layers=1, embedding_length=32 * 64, head_count=32, head_count_kv=8, feed_forward_length=512,
                vocab_size=1000, context_length=8192 + 64, tied=1, norm_mode=1)
    img = nc.synth_gguf(**spec, seed=8201)
    gm = nc.Model(ctx, data=img)
    prompt = nc.uniform_prompt(8201, 8192, 1000)
    sess = nc.Session(gm, 8192 + 32, 16)
    sess.prefill_pass_batch(prompt, 0, want_logits=False)
    batch = nc.uniform_prompt(9, 9, 1000)
    single = []
    for i in range(9):
        _, lg = sess.forward_pass(int(batch[i]), 8192 + i)
        single.append(lg)
    sess.verify_greedy(batch, 8192)
    for i in range(9):
        assert _same(sess.logits(i), single[i]), i


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
