"""Split-order attention (nc_ctx_set_attention(NC_ATTN_SPLIT)) against the CPU oracle.

The split order takes each row's positions in 64-position chunks and combines the chunks'
max, sum of exp and exp-weighted V sums.  The oracle restates that order operation for
operation (or_attention_head_split, its session in attention order 1), so the device's logits
must be bit-identical to the oracle's and its token streams equal; the split order itself is
pinned against the reference's sequential attention and a float64 softmax on the CPU
(tests/test_oracle_attention_split.py).  Batch independence is exact: a row's logits are
bit-identical whether it is verified in a batch of 16 or decoded alone.
"""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TINY = dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512, vocab_size=1000,
            context_length=512, tied=0, norm_mode=1)


@pytest.fixture(scope="module")
def sctx():
    import nanocamelid_amd as nc
    assert torch.cuda.is_available()
    c = nc.Context(0)
    c.set_attention(nc._ffi.NC_ATTN_SPLIT)
    return c


def _models(ctx, spec, seed):
    import nanocamelid_amd as nc
    img = nc.synth_gguf(**spec, seed=seed)
    return img, nc.Model(ctx, data=img), O.Model(data=img.tobytes(), nthreads=16)


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def _osession(om, max_ctx, max_batch):
    s = O.Session(om, max_ctx, max_batch)
    s.set_attention(1)
    return s


def _check_rows(gs, preds, opreds, ologits, n, where):
    for i in range(n):
        assert _same(gs.logits(i), ologits[i]), (where, i)
    assert np.array_equal(preds, opreds), where


def test_mode_switch_rejects_unknown_order():
    import nanocamelid_amd as nc
    c = nc.Context(0)
    with pytest.raises(nc.NcError):
        c.set_attention(7)
    c.set_attention(nc._ffi.NC_ATTN_SPLIT)
    c.set_attention(nc._ffi.NC_ATTN_SEQUENTIAL)


@pytest.mark.parametrize("hd,tied", [(64, 1), (128, 0)])
def test_split_logits_bit_exact(sctx, hd, tied):
    """Widths 1..16 at positions that cross the 64-position chunk boundaries."""
    import nanocamelid_amd as nc
    spec = dict(TINY, head_count=256 // hd * 2, head_count_kv=256 // hd, embedding_length=512, tied=tied)
    _, gm, om = _models(sctx, spec, seed=hd + 1)
    gs = nc.Session(gm, 256, 16)
    os_ = _osession(om, 256, 16)
    pos = 0
    for n in (16, 16, 5, 1, 9, 16, 3, 16, 16, 16, 13, 2, 7, 4, 6, 8, 10, 11, 12, 14, 15):
        batch = nc.uniform_prompt(pos + 3, n, 1000)
        _, _, _, preds = gs.verify_greedy(batch, pos)
        opreds, _, ologits = os_.verify_greedy(batch, pos, want_logits=True)
        _check_rows(gs, preds, opreds, ologits, n, pos)
        pos += n


def test_split_batch_independent(sctx):
    """A 16-row verify pass and 16 single-token passes at the same positions: bit-identical
    logits row by row (the split order is fixed by absolute positions, not by the batch)."""
    import nanocamelid_amd as nc
    _, gm, _ = _models(sctx, TINY, seed=41)
    toks = nc.uniform_prompt(41, 200, 1000)
    a, b = nc.Session(gm, 256, 16), nc.Session(gm, 256, 16)
    for pos in range(0, 192, 16):  # 16-row passes straddle chunk boundaries at 64 and 128
        a.verify_greedy(toks[pos:pos + 16], pos)
        rows = [np.array(a.logits(i), np.float32) for i in range(16)]
        for i in range(16):
            _, lg = b.forward_pass(int(toks[pos + i]), pos + i)
            assert _same(lg, rows[i]), (pos, i)


@pytest.mark.parametrize("hd,checks", [(128, (700, 2045)), (64, (4093,))], ids=["hd128", "hd64"])
def test_split_long_context(sctx, hd, checks):
    """Rows of hundreds to thousands of positions (up to 64 chunks per row), KV filled by
    prompt passes; one layer, so the cache contents do not depend on the attention order."""
    import nanocamelid_amd as nc
    upto = checks[-1] + 9
    spec = dict(layers=1, embedding_length=2 * hd * 2, head_count=4, head_count_kv=2, feed_forward_length=512,
                vocab_size=1000, context_length=upto + 64, tied=1, norm_mode=1)
    _, gm, om = _models(sctx, spec, seed=hd + 7)
    prompt = nc.uniform_prompt(hd + 7, upto, 1000)
    gs, os_ = nc.Session(gm, upto + 16, 16), _osession(om, upto + 16, 16)
    pos = 0
    for c in checks:
        print(f"split long context hd={hd}: prefill to {c}, verify 9 rows", flush=True)
        gs.prefill_pass_batch(prompt[pos:c], pos)
        for i in range(pos, c, 16):
            os_.prefill_pass_batch(prompt[i:min(i + 16, c)], i)
        batch = nc.uniform_prompt(c, 9, 1000)
        _, _, _, preds = gs.verify_greedy(batch, c)
        opreds, _, ologits = os_.verify_greedy(batch, c, want_logits=True)
        _check_rows(gs, preds, opreds, ologits, 9, c)
        pos = c


def test_split_streams_equal_oracle(sctx):
    """Greedy, oracle-drafter speculative (k = 2, 4, 8) and draft-model speculative streams in
    the split order equal the oracle's split-order greedy stream, with the oracle's acceptance
    statistics."""
    import nanocamelid_amd as nc
    _, gm, om = _models(sctx, TINY, seed=31)
    prompt = nc.uniform_prompt(77, 24, 1000)
    ref = _osession(om, 400, 16).generate_greedy(prompt, 96)
    assert len(set(ref.tolist())) >= 8
    out, _ = nc.Session(gm, 400, 16).generate_greedy(prompt, 96)
    assert np.array_equal(out, ref)
    for k, alpha in ((2, 0.5), (4, 0.8), (8, 0.8)):
        g_out, st = nc.Session(gm, 400, 16).generate_speculative_oracle(prompt, 96, k, alpha, 1234, ref)
        _, drafted, accepted, steps = _osession(om, 400, 16).generate_speculative_oracle(prompt, 96, k, alpha, 1234,
                                                                                         ref)
        assert np.array_equal(g_out, ref)
        assert (st.drafted, st.accepted, st.steps) == (drafted, accepted, steps)
    # a draft that disagrees part of the time (the target's weights with unit norm weights):
    # rejections, corrective tokens and the corrective forwards, same stream
    dm = nc.Model(sctx, data=nc.synth_gguf(**dict(TINY, norm_mode=0), seed=31))
    d_out, st = nc.generate_speculative_draft(nc.Session(gm, 400, 16), nc.Session(dm, 400, 8), prompt, 96, 4)
    assert np.array_equal(d_out, ref)
    assert 0 < st.accepted < st.drafted


@pytest.mark.parametrize("ctx_len", [2000, 8192])
def test_split_many_queries_long_rows_batch_independent(sctx, ctx_len):
    """Many query vectors per KV head (4 heads x 9 rows) over long rows: the launch takes 16
    queries per wave (and one chunk per wave at 8192 positions), the shapes of the 70B
    verify; every 9-row verify row equals a single-token pass at its position, bit for bit
    (those take 4 queries per wave)."""
    import nanocamelid_amd as nc
    spec = dict(layers=1, embedding_length=32 * 64, head_count=32, head_count_kv=8, feed_forward_length=512,
                vocab_size=1000, context_length=ctx_len + 64, tied=1, norm_mode=1)
    gm = nc.Model(sctx, data=nc.synth_gguf(**spec, seed=ctx_len))
    prompt = nc.uniform_prompt(ctx_len, ctx_len, 1000)
    batch = nc.uniform_prompt(ctx_len + 1, 9, 1000)
    a, b = nc.Session(gm, ctx_len + 16, 16), nc.Session(gm, ctx_len + 16, 16)
    print(f"split many queries: prefill {ctx_len}, verify 9 rows", flush=True)
    a.prefill_pass_batch(prompt, 0)
    b.prefill_pass_batch(prompt, 0)
    a.verify_greedy(batch, ctx_len)
    rows = [np.array(a.logits(i), np.float32) for i in range(9)]
    for i in range(9):
        _, lg = b.forward_pass(int(batch[i]), ctx_len + i)
        assert _same(lg, rows[i]), (ctx_len, i)
