"""Writes the golden fixtures in tests/golden/ from the CPU oracle.

The reference is Rust and cannot be built in this image, so its outputs cannot be recorded
directly; the fixtures are produced by the oracle (the C++ restatement of the reference's
portable x86 path, itself pinned by the reference's known answers and closed forms in
tests/test_oracle_*.py) and freeze its results so that every later change of the oracle or
of the GPU path is compared against the same numbers.

  blockdots.npz   Q4_0 blocks (the reference's known-answer blocks from q8.rs:4514-4530 and
                  q8.rs:4533-4565, then seeded random blocks), int8 activations with f32
                  scales, the int32 per-block dots and the f32 block-ordered matmul outputs.
  toy_model.npz   a seeded 2-layer Llama model (rebuilt from its synthetic spec, not stored;
                  the image's sha256 is kept to detect drift): prompt, two k+1 verify batches
                  with the bits of every row's logits, and the greedy, oracle-drafter
                  speculative and stochastic (draft-model, Philox) token streams.

Run from the repository root:  python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
HERE = os.path.dirname(os.path.abspath(__file__))

TOY = dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512, vocab_size=1000,
           context_length=512, tied=1, norm_mode=1)
TOY_SEED = 21
DRAFT = dict(TOY, layers=1, feed_forward_length=256, head_count=2, head_count_kv=1)
DRAFT_SEED = 5
PROMPT = (5, 24)                 # uniform_prompt(seed, n)
BATCHES = ((24, 100, 5), (29, 101, 9))  # (start_pos, uniform_prompt seed, rows)
N_STREAM = 48


def reference_blocks():
    """The reference's Q4_0 test blocks: nibble order (q8.rs:4514-4530) and the dot fixture
    (q8.rs:4533-4565)."""
    a = np.zeros(18, np.uint8)
    a[0:2] = [0x00, 0x3C]  # f16 1.0
    for idx in range(16):
        a[2 + idx] = idx | ((15 - idx) << 4)
    b = np.array([0x00, 0x3C, 0x80, 0x91, 0xA2, 0xB3, 0xC4, 0xD5, 0xE6, 0xF7, 0x08, 0x19, 0x2A, 0x3B, 0x4C, 0x5D,
                  0x6E, 0x7F], np.uint8)
    return a, b


def make_blockdots(O):
    from tests.gpu_util import random_q4_0
    M, K, N = 8, 128, 3
    w = random_q4_0(M, K, seed=77)                   # [M][K/32][18]
    a, b = reference_blocks()
    w[0, :] = a
    w[1, :] = b
    w[2, 0], w[2, 1] = a, b
    rng = np.random.default_rng(78)
    xq = rng.integers(-127, 128, (N, K)).astype(np.int8)
    xq[0, :32] = np.arange(32) - 16                  # the fixture's activation idx - 16
    xq[1, :32] = 127
    xs = rng.uniform(0.001, 0.05, (N, K // 32)).astype(np.float32)
    dots = O.matmul_q4_0_blockdots(xq, w, N, M, K)
    out = O.matmul_q4_0(xq, xs, w, N, M, K)
    np.savez_compressed(os.path.join(HERE, "blockdots.npz"), w=w, xq=xq, xs=xs, dots=dots, out=out)


def make_toy(O, nc):
    img = nc.synth_gguf(**TOY, seed=TOY_SEED)
    dimg = nc.synth_gguf(**DRAFT, seed=DRAFT_SEED)
    om, dm = O.Model(data=img.tobytes()), O.Model(data=dimg.tobytes())
    prompt = nc.uniform_prompt(*PROMPT, TOY["vocab_size"])
    s = O.Session(om, 256, 16)
    for i in range(0, len(prompt), 16):
        s.prefill_pass_batch(prompt[i:i + 16], i)
    logits, batches = [], []
    for start, seed, n in BATCHES:
        toks = nc.uniform_prompt(seed, n, TOY["vocab_size"])
        _, _, lg = s.verify_greedy(toks, start, want_logits=True)
        batches.append(toks)
        logits.append(lg.view(np.uint32))
    greedy = O.Session(om, 256, 16).generate_greedy(prompt, N_STREAM)
    spec, _, _, _ = O.Session(om, 256, 16).generate_speculative_oracle(prompt, N_STREAM, 4, 0.8, 99, greedy)
    stoch, drafted, accepted, steps = O.generate_speculative_stochastic(O.Session(om, 256, 16), O.Session(dm, 256, 16),
                                                                        prompt, N_STREAM, 4, 1.0, 7)
    meta = dict(toy=TOY, toy_seed=TOY_SEED, draft=DRAFT, draft_seed=DRAFT_SEED, prompt=PROMPT, batches=BATCHES,
                n_stream=N_STREAM, speculative=dict(k=4, alpha=0.8, seed=99),
                stochastic=dict(k=4, temp=1.0, seed=7, drafted=drafted, accepted=accepted, steps=steps),
                toy_sha256=hashlib.sha256(img.tobytes()).hexdigest(),
                draft_sha256=hashlib.sha256(dimg.tobytes()).hexdigest())
    np.savez_compressed(os.path.join(HERE, "toy_model.npz"), meta=np.array(json.dumps(meta)), prompt=prompt,
                        batch0=batches[0], batch1=batches[1], logits0=logits[0], logits1=logits[1], greedy=greedy,
                        speculative=spec, stochastic=stoch)


def main():
    import nanocamelid_amd as nc
    from oracle import oracle as O
    make_blockdots(O)
    make_toy(O, nc)
    for f in ("blockdots.npz", "toy_model.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
