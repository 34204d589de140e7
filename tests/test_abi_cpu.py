"""CPU checks of the product library: it loads, exports the whole C ABI, and its host-only
pieces (synthetic GGUF writer, Philox prompt/drafter) agree with the oracle.
No GPU call is made here."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nanocamelid_gpu.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(nc_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    import nanocamelid_amd._ffi as F
    lib = C.CDLL(F.LIB_PATH)
    names = _declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the ctypes table covers the same set
    assert set(F.SIGNATURES) == set(names)


def test_version_and_error_channel():
    import nanocamelid_amd as nc
    from nanocamelid_amd._ffi import lib
    assert b"gfx950" in lib().nc_version()
    with pytest.raises(nc.NcError):
        nc.uniform_prompt(1, 4, 0)  # vocab 0 -> NC_EINVAL, no GPU touched
    assert b"bad arguments" in lib().nc_last_error()


TINY = dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512, vocab_size=1000,
            context_length=512, tied=1)


def test_synth_gguf_parses_in_oracle_and_is_deterministic():
    import nanocamelid_amd as nc
    a = nc.synth_gguf(**TINY, seed=5, nthreads=1)
    b = nc.synth_gguf(**TINY, seed=5, nthreads=8)
    assert np.array_equal(a, b)
    c = nc.synth_gguf(**TINY, seed=6)
    assert not np.array_equal(a, c)
    m = O.Model(data=a.tobytes())
    assert m.info["d"] == 256 and m.info["layers"] == 2 and m.info["vocab"] == 1000
    assert m.info["heads"] == 4 and m.info["kv_heads"] == 2 and m.info["head_dim"] == 64
    assert m.info["has_output"] == 0 and m.info["weight_type"] == 2
    assert abs(m.rope_base - 500000.0) < 1 and abs(m.eps - 1e-5) < 1e-9


def test_synth_weight_statistics():
    # token_embd is the first tensor: dequantised values should look like N(0, 0.02)
    import nanocamelid_amd as nc
    img = nc.synth_gguf(layers=1, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512,
                        vocab_size=4096, tied=0, seed=11)
    m = O.Model(data=img.tobytes())
    head = m.head_q4_0().reshape(4096, 8, 18)
    sc = (head[:, :, 0].astype(np.uint16) | (head[:, :, 1].astype(np.uint16) << 8)).view(np.float16).astype(np.float64)
    vals = np.concatenate([(head[:, :, 2:] & 15).astype(np.float64) - 8, (head[:, :, 2:] >> 4).astype(np.float64) - 8],
                          axis=2) * sc[:, :, None]
    assert abs(vals.mean()) < 1e-3
    assert 0.017 < vals.std() < 0.023


def test_synth_q4_k_model_parses():
    import nanocamelid_amd as nc
    img = nc.synth_gguf(layers=1, embedding_length=256, head_count=2, head_count_kv=2, feed_forward_length=512,
                        vocab_size=512, weight_type=nc.NC_TYPE_Q4_K, tied=1, seed=3)
    m = O.Model(data=img.tobytes())
    assert m.info["weight_type"] == 12


def test_prompt_and_oracle_drafter_match_oracle():
    import nanocamelid_amd as nc
    assert np.array_equal(nc.uniform_prompt(42, 512, 128256), O.uniform_prompt(42, 512, 128256))
    greedy = np.arange(5000, 6000, dtype=np.uint32)
    for p in range(32, 400, 7):
        for alpha in (0.5, 0.8):
            assert nc.oracle_draft(9, p, alpha, greedy, 32, 128256) == O.oracle_draft(9, p, alpha, greedy, 32, 128256)
