"""The split attention order (the device's NC_ATTN_SPLIT) pinned on the CPU.

or_attention_head_split restates the device's order: 64-position chunks with a chunk max, a
butterfly sum of exp and an fma chain of exp-weighted values, combined in chunk order.  It has
no counterpart in the reference; what fixes it is the mathematics: it must equal a float64
softmax attention, and the reference's sequential attention (or_attention_head), up to f32
rounding, at lengths that end inside, on and just past chunk boundaries.  A dropped chunk, a
wrong rescale exponent or an off-by-one mask moves the result far outside these bounds.
"""
import numpy as np
import pytest

from oracle import oracle as O

HD, KVW = 128, 256  # two KV heads of 128 dims per cache row


def _case(seed, ctx):
    rng = np.random.default_rng(seed)
    q = rng.normal(0, 1, HD).astype(np.float32)
    k = rng.normal(0, 1, (ctx, KVW)).astype(np.float32)
    v = rng.normal(0, 1, (ctx, KVW)).astype(np.float32)
    return q, k, v


def _f64_attention(q, k, v, pos, kvh, scale):
    kk = k[:pos + 1, kvh * HD:(kvh + 1) * HD].astype(np.float64)
    vv = v[:pos + 1, kvh * HD:(kvh + 1) * HD].astype(np.float64)
    s = kk @ q.astype(np.float64) * scale
    e = np.exp(s - s.max())
    return (e / e.sum()) @ vv


@pytest.mark.parametrize("pos", [0, 1, 62, 63, 64, 65, 127, 128, 200, 1000, 4095, 4100])
def test_split_matches_float64_and_sequential(pos):
    q, k, v = _case(pos, pos + 70)
    scale = 1.0 / np.sqrt(HD)
    for kvh in (0, 1):
        want = _f64_attention(q, k, v, pos, kvh, scale)
        split = O.attention_head_split(q, k, v, pos, pos, KVW, kvh, HD, np.float32(scale)).astype(np.float64)
        seq = O.attention_head(q, k, v, pos, KVW, kvh, HD, np.float32(scale)).astype(np.float64)
        mag = np.max(np.abs(want))
        assert np.max(np.abs(split - want)) <= 2e-6 * mag, (pos, kvh)
        assert np.max(np.abs(split - seq)) <= 4e-6 * mag, (pos, kvh)


def test_split_values_past_the_pass_are_not_read():
    """Cache rows past plast (the pass's last position) may hold any bits on the device: a row
    at pos < plast ignores them, and NaNs there do not reach the output."""
    pos, plast = 70, 75
    q, k, v = _case(7, 200)
    scale = np.float32(1.0 / np.sqrt(HD))
    a = O.attention_head_split(q, k, v, pos, plast, KVW, 0, HD, scale)
    v2 = v.copy()
    v2[plast + 1:] = np.nan
    k2 = k.copy()
    k2[pos + 1:] = np.nan
    b = O.attention_head_split(q, k2, v2, pos, plast, KVW, 0, HD, scale)
    assert np.all(np.isfinite(b)) and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_split_ignores_positions_past_the_row():
    """Positions pos+1..plast (later rows of the same pass) carry weight 0: changing their keys
    and values leaves the output's bits unchanged."""
    pos, plast = 100, 110
    q, k, v = _case(9, 200)
    scale = np.float32(1.0 / np.sqrt(HD))
    a = O.attention_head_split(q, k, v, pos, plast, KVW, 1, HD, scale)
    k2, v2 = k.copy(), v.copy()
    k2[pos + 1:plast + 1] *= 3.0
    v2[pos + 1:plast + 1] = 1e6
    b = O.attention_head_split(q, k2, v2, pos, plast, KVW, 1, HD, scale)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_split_session_batch_independent():
    """Oracle sessions in the split order: a 16-row verify pass and single-token passes at the
    same positions give bit-identical logits (the order depends on absolute positions only)."""
    import nanocamelid_amd as nc
    spec = dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512,
                vocab_size=1000, context_length=256, tied=0, norm_mode=1)
    om = O.Model(data=nc.synth_gguf(**spec, seed=5).tobytes(), nthreads=4)
    toks = nc.uniform_prompt(5, 96, 1000)
    a, b = O.Session(om, 128, 16), O.Session(om, 128, 16)
    a.set_attention(1)
    b.set_attention(1)
    for pos in range(0, 96, 16):
        _, _, rows = a.verify_greedy(toks[pos:pos + 16], pos, want_logits=True)
        for i in range(16):
            lg = b.forward_pass(int(toks[pos + i]), pos + i)
            assert np.array_equal(np.asarray(lg, np.float32).view(np.uint32),
                                  np.asarray(rows[i], np.float32).view(np.uint32)), (pos, i)
