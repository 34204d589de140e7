"""Golden fixtures (tests/golden/, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every fixture bit for bit, and the synthetic model image it
is built from has not drifted.  GPU: the device path reproduces the same fixtures through the
C ABI (the GPU box has no reference tree and no oracle is needed for these checks).
"""
import hashlib
import json
import os

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(HERE, name), allow_pickle=False)


def _toy_meta(z):
    return json.loads(str(z["meta"]))


def test_oracle_reproduces_blockdots():
    from oracle import oracle as O
    z = _load("blockdots.npz")
    w, xq, xs = z["w"], z["xq"], z["xs"]
    N, K = xq.shape
    M = w.shape[0]
    assert np.array_equal(O.matmul_q4_0_blockdots(xq, w, N, M, K), z["dots"])
    assert np.array_equal(O.matmul_q4_0(xq, xs, w, N, M, K).view(np.uint32), z["out"].view(np.uint32))
    # row 1 block 0 is the reference's dot fixture against activation idx-16 (q8.rs:4533-4565)
    blk = w[1, 0]
    lo = (blk[2:] & 0x0F).astype(np.int64) - 8
    hi = (blk[2:] >> 4).astype(np.int64) - 8
    assert z["dots"][0, 1, 0] == int(np.dot(np.concatenate([lo, hi]), np.arange(32) - 16))


def test_oracle_reproduces_toy_model():
    import nanocamelid_amd as nc
    from oracle import oracle as O
    z = _load("toy_model.npz")
    meta = _toy_meta(z)
    img = nc.synth_gguf(**meta["toy"], seed=meta["toy_seed"])
    assert hashlib.sha256(img.tobytes()).hexdigest() == meta["toy_sha256"]
    om = O.Model(data=img.tobytes())
    prompt = z["prompt"]
    s = O.Session(om, 256, 16)
    for i in range(0, len(prompt), 16):
        s.prefill_pass_batch(prompt[i:i + 16], i)
    for j, (start, _, _) in enumerate(meta["batches"]):
        _, _, lg = s.verify_greedy(z[f"batch{j}"], start, want_logits=True)
        assert np.array_equal(lg.view(np.uint32), z[f"logits{j}"])
    greedy = O.Session(om, 256, 16).generate_greedy(prompt, meta["n_stream"])
    assert np.array_equal(greedy, z["greedy"])


@pytest.mark.gpu
def test_gpu_blockdots_golden():
    import torch

    import nanocamelid_amd as nc
    z = _load("blockdots.npz")
    w, xq, xs = z["w"], z["xq"], z["xs"]
    ctx = nc.Context(0)
    q = nc.QMat(ctx, nc.NC_TYPE_Q4_0, w.shape[0], xq.shape[1], w)
    xt, st = torch.from_numpy(xq).cuda(), torch.from_numpy(xs).cuda()
    assert np.array_equal(nc.matmul_blockdots(ctx, q, xt).cpu().numpy(), z["dots"])
    out = nc.matmul_quantized_batch(ctx, q, xt, st).cpu().numpy()
    assert np.array_equal(out.view(np.uint32), z["out"].view(np.uint32))


@pytest.mark.gpu
def test_gpu_toy_model_golden():
    import torch

    import nanocamelid_amd as nc
    z = _load("toy_model.npz")
    meta = _toy_meta(z)
    assert torch.cuda.is_available()
    ctx = nc.Context(0)
    img = nc.synth_gguf(**meta["toy"], seed=meta["toy_seed"])
    dimg = nc.synth_gguf(**meta["draft"], seed=meta["draft_seed"])
    assert hashlib.sha256(img.tobytes()).hexdigest() == meta["toy_sha256"]
    assert hashlib.sha256(dimg.tobytes()).hexdigest() == meta["draft_sha256"]
    gm, dm = nc.Model(ctx, data=img), nc.Model(ctx, data=dimg)
    prompt = z["prompt"]
    s = nc.Session(gm, 256, 16)
    s.prefill_pass_batch(prompt, 0)
    for j, (start, _, n) in enumerate(meta["batches"]):
        s.verify_greedy(z[f"batch{j}"], start)
        got = np.stack([s.logits(i) for i in range(n)])
        assert np.array_equal(got.view(np.uint32), z[f"logits{j}"]), j
    n = meta["n_stream"]
    greedy, _ = nc.Session(gm, 256, 16).generate_greedy(prompt, n)
    assert np.array_equal(greedy, z["greedy"])
    sp = meta["speculative"]
    spec, _ = nc.Session(gm, 256, 16).generate_speculative_oracle(prompt, n, sp["k"], sp["alpha"], sp["seed"],
                                                                  z["greedy"])
    assert np.array_equal(spec, z["speculative"])
    so = meta["stochastic"]
    stoch, st = nc.generate_speculative_stochastic(nc.Session(gm, 256, 16), nc.Session(dm, 256, 16), prompt, n,
                                                   so["k"], so["temp"], so["seed"])
    assert np.array_equal(stoch, z["stochastic"])
    assert (st.drafted, st.accepted, st.steps) == (so["drafted"], so["accepted"], so["steps"])
