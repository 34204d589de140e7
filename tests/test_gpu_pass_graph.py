"""Verify and decode passes replayed from captured HIP graphs (nc_ctx_set_pass_launch(NC_PASS_GRAPH))
against the same passes launched kernel by kernel (NC_PASS_DIRECT, the path the oracle tests pin).

Both contexts load the same model image and follow the same schedule, so every logit row,
prediction and acceptance result must be bit-identical.  The schedule replays each captured graph
several times with other graphs, eager kernels on the context stream and host synchronisations in
between; it crosses every attention variant the key separates (the one-kernel tiers at 512, 768,
1024, 1280 positions and the two-kernel path past 1536, whose score grid changes every 512
positions) and replays one two-kernel graph at a position 450 rows further on inside its grid.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

SPEC = dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512, vocab_size=1000,
            context_length=4096, tied=0, norm_mode=1)


def _same(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.fixture(scope="module")
def pair():
    import nanocamelid_amd as nc
    assert torch.cuda.is_available()
    dctx, gctx = nc.Context(0), nc.Context(0)
    gctx.set_pass_launch(nc._ffi.NC_PASS_GRAPH)
    img = nc.synth_gguf(**SPEC, seed=7)
    return dctx, gctx, nc.Model(dctx, data=img), nc.Model(gctx, data=img)


def _check_verify(ds, gs, batch, pos):
    rd = ds.verify_greedy(batch, pos)
    rg = gs.verify_greedy(batch, pos)
    assert rd[:3] == rg[:3], (len(batch), pos)
    assert np.array_equal(rd[3], rg[3]), (len(batch), pos)
    for i in range(len(batch)):
        assert _same(ds.logits(i), gs.logits(i)), (len(batch), pos, i)


def test_graph_replays_match_direct_passes(pair):
    import nanocamelid_amd as nc
    dctx, gctx, dm, gm = pair
    ds, gs = nc.Session(dm, 2700, 16), nc.Session(gm, 2700, 16)
    for s in (ds, gs):
        s.fill_kv(2600, seed=3)  # every position a pass reads holds the same N(0, 1) rows
    schedule = [(5, 300), (5, 305), (5, 310), (1, 315), (9, 316), (16, 400), (5, 320), (5, 600), (5, 605),
                (5, 900), (16, 1100), (5, 1400), (5, 1700), (5, 1710), (3, 2040), (5, 2050), (5, 2500), (5, 300)]
    x = torch.from_numpy(np.random.default_rng(1).standard_normal((3, 256)).astype(np.float32)).cuda()
    for j, (n, pos) in enumerate(schedule):
        batch = nc.uniform_prompt(1000 + j, n, SPEC["vocab_size"])
        _check_verify(ds, gs, batch, pos)
        if j % 4 == 1:  # eager kernels of the library between replays, then a device-wide wait
            nc.quantize_f32_to_q8_0_batch(gctx, x)
            torch.cuda.synchronize()
    # single-row decode passes (nc_forward1) at both ends of the schedule's positions
    for pos in (330, 331, 2520, 2521):
        tok = int(nc.uniform_prompt(pos, 1, SPEC["vocab_size"])[0])
        (pd, ld), (pg, lg) = ds.forward_pass(tok, pos), gs.forward_pass(tok, pos)
        assert pd == pg and _same(ld, lg), pos
    captures, replays = gs.pass_graphs()
    assert ds.pass_graphs() == (0, 0)
    assert replays == len(schedule) + 4
    # keys (width, attention variant): (5, <=512) (1, <=512) (9, <=512) (16, <=512) (5, <=768)
    # (5, <=1024) (16, <=1280) (5, <=1536) (5, <=2048 grid 32) (3, <=2048 grid 32)
    # (5, <=4096 grid 40) (1, <=4096 grid 40); the decode passes at 330 and 331 replay (1, <=512)
    assert captures == 12, (captures, replays)


def test_graph_decode_loops_match_direct(pair):
    """Whole decode loops on both launch modes: the oracle-drafter verify loop (nc_verify_greedy
    per step) and the stochastic draft-model loop, whose draft passes, temperature sampling and
    target verify are queued without a host wait inside the step."""
    import nanocamelid_amd as nc
    dctx, gctx, dm, gm = pair
    V = SPEC["vocab_size"]
    prompt = nc.uniform_prompt(11, 700, V)
    greedy, _ = nc.Session(dm, 1200, 16).generate_greedy(prompt, 160)
    gg, _ = nc.Session(gm, 1200, 16).generate_greedy(prompt, 160)
    assert np.array_equal(greedy, gg)
    outs = []
    for m in (dm, gm):
        s = nc.Session(m, 1200, 16)
        out, st = s.generate_speculative_oracle(prompt, 160, 4, 0.8, 5, greedy)
        outs.append((out, st.steps, st.accepted))
        if m is gm:
            assert s.pass_graphs()[1] == st.steps + 1  # + the prompt's last-chunk pass
        else:
            assert s.pass_graphs() == (0, 0)
    assert np.array_equal(outs[0][0], outs[1][0]) and outs[0][1:] == outs[1][1:]
    assert np.array_equal(outs[0][0], greedy[:len(outs[0][0])])
    img2 = nc.synth_gguf(**SPEC, seed=8)
    streams = []
    for ctx, tmod in ((dctx, dm), (gctx, gm)):
        drm = nc.Model(ctx, data=img2)
        ts, ds = nc.Session(tmod, 1200, 16), nc.Session(drm, 1200, 16)
        out, st = nc.generate_speculative_stochastic(ts, ds, prompt, 120, 4, 1.0, 21)
        streams.append((np.asarray(out), st.steps, st.drafted, st.accepted))
        if ctx is gctx:
            assert ts.pass_graphs()[1] > 0 and ds.pass_graphs()[1] > 0
    assert np.array_equal(streams[0][0], streams[1][0])
    assert streams[0][1:] == streams[1][1:]


def test_graph_cache_starts_over(pair):
    """More distinct passes than the session keeps graphs for (48): the cache is cleared and the
    passes captured again; every pass still matches the direct launch."""
    import nanocamelid_amd as nc
    dctx, gctx, dm, gm = pair
    ds, gs = nc.Session(dm, 1300, 16), nc.Session(gm, 1300, 16)
    for s in (ds, gs):
        s.fill_kv(1250, seed=4)
    j = 0
    for pos in (100, 600, 900):
        for n in range(1, 17):
            _check_verify(ds, gs, nc.uniform_prompt(3000 + j, n, SPEC["vocab_size"]), pos)
            j += 1
    assert gs.pass_graphs() == (48, 48)
    for n, pos in ((5, 1100), (5, 110), (5, 1100)):  # a 49th key clears the cache
        _check_verify(ds, gs, nc.uniform_prompt(3000 + j, n, SPEC["vocab_size"]), pos)
        j += 1
    assert gs.pass_graphs() == (50, 51)
