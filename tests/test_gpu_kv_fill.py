"""The device's N(0, 1) KV fill (nc_session_fill_kv) against the oracle's (or_session_fill_kv):
a verify pass over the filled rows gives bit-identical logits, at fill lengths that do and do
not end on a value position quad, for head_dim 64 and 128."""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ctx():
    import nanocamelid_amd as nc
    assert torch.cuda.is_available()
    return nc.Context(0)


@pytest.mark.parametrize("hd,n", [(64, 300), (64, 301), (128, 258), (128, 1537)])
def test_fill_then_verify_matches_oracle(ctx, hd, n):
    import nanocamelid_amd as nc
    spec = dict(layers=2, embedding_length=4 * hd, head_count=4, head_count_kv=2, feed_forward_length=512,
                vocab_size=900, tied=1, norm_mode=1, context_length=2048)
    print(f"fill: hd {hd}, n {n}", flush=True)
    img = nc.synth_gguf(**spec, seed=hd + n)
    gs = nc.Session(nc.Model(ctx, data=img), n + 32, 16)
    os_ = O.Session(O.Model(data=img.tobytes()), n + 32, 16)
    gs.fill_kv(n, 4242)
    os_.fill_kv(n, 4242)
    toks = nc.uniform_prompt(n, 7, spec["vocab_size"])
    a, nxt, newpos, preds = gs.verify_greedy(toks, n)
    opreds, _, ologits = os_.verify_greedy(toks, n, want_logits=True)
    assert np.array_equal(preds, opreds)
    for i in range(len(toks)):
        assert np.array_equal(gs.logits(i).view(np.uint32), ologits[i].view(np.uint32)), i
    # the fill writes only rows [0, n): a second fill with another seed changes the logits
    gs.fill_kv(n, 4243)
    gs.verify_greedy(toks, n)
    assert not np.array_equal(gs.logits(0), ologits[0])
