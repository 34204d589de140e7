"""End-of-generation ids from a GGUF's tokenizer metadata (nc_gguf_stop_tokens): the set that
is_generation_stop_token tests (src/main.rs:8518-8520), SpecialTokens::eog as Tokenizer::from_gguf
builds it (src/tokenizer.rs:203-360): eos, eot, eom and Phi-3's "<|end|>", from metadata or the
reference's defaults, every special id range-checked (validate_token_id, :1180-1189).  Host only.
The expected sets below are worked out by hand from those rules."""
import numpy as np
import pytest

import nanocamelid_amd as nc
from tests import gguf_writer as GW

BASE = dict(layers=1, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512,
            vocab_size=1000, context_length=64)


def _image(model, texts, extra=()):
    meta, ts = GW.read(nc.synth_gguf(**BASE, seed=3).tobytes())
    meta = list(meta)
    if model is not None:
        meta.append(("tokenizer.ggml.model", GW.T_STR, model))
    if texts is not None:
        meta.append(("tokenizer.ggml.tokens", GW.T_ARR, (GW.T_STR, texts)))
    meta += list(extra)
    return GW.write(meta, ts)


def _vocab(n, specials):
    t = [f"tok{i}" for i in range(n)]
    for i, s in specials.items():
        t[i] = s
    return t


def test_gpt2_vocabulary_defaults_by_text():
    texts = _vocab(40, {5: "<|begin_of_text|>", 6: "<|end_of_text|>", 9: "<|eot_id|>", 12: "<|eom_id|>"})
    # eos = "<|end_of_text|>", eot = "<|eot_id|>"; eom has no default
    assert nc.gguf_stop_tokens(_image("gpt2", texts)).tolist() == [6, 9]


def test_metadata_ids_take_precedence():
    texts = _vocab(40, {6: "<|end_of_text|>", 9: "<|eot_id|>"})
    extra = [("tokenizer.ggml.eos_token_id", GW.T_U32, 7), ("tokenizer.ggml.eom_token_id", GW.T_U32, 30)]
    assert nc.gguf_stop_tokens(_image("gpt2", texts, extra)).tolist() == [7, 9, 30]
    extra.append(("tokenizer.ggml.eot_token_id", GW.T_U32, 7))  # the set is distinct
    assert nc.gguf_stop_tokens(_image("gpt2", texts, extra)).tolist() == [7, 30]


def test_llama3_metadata():
    """Llama-3 GGUFs: eos 128001 "<|end_of_text|>", eom 128008, eot 128009."""
    texts = _vocab(128256, {128000: "<|begin_of_text|>", 128001: "<|end_of_text|>", 128008: "<|eom_id|>",
                            128009: "<|eot_id|>"})
    extra = [("tokenizer.ggml.bos_token_id", GW.T_U32, 128000), ("tokenizer.ggml.eos_token_id", GW.T_U32, 128001),
             ("tokenizer.ggml.eot_token_id", GW.T_U32, 128009), ("tokenizer.ggml.eom_token_id", GW.T_U32, 128008)]
    assert nc.gguf_stop_tokens(_image("gpt2", texts, extra)).tolist() == [128001, 128008, 128009]


def test_sentencepiece_defaults_and_phi_end():
    assert nc.gguf_stop_tokens(_image("llama", _vocab(50, {}))).tolist() == [2]
    # Phi-3 ends assistant turns with "<|end|>" besides its eos
    phi = _vocab(50, {32: "<|endoftext|>", 47: "<|end|>"})
    extra = [("tokenizer.ggml.eos_token_id", GW.T_U32, 32)]
    assert nc.gguf_stop_tokens(_image("llama", phi, extra)).tolist() == [32, 47]


def test_text_lookup_takes_the_last_duplicate():
    texts = _vocab(40, {9: "<|eot_id|>", 21: "<|eot_id|>", 6: "<|end_of_text|>"})
    assert nc.gguf_stop_tokens(_image("gpt2", texts)).tolist() == [6, 21]


@pytest.mark.parametrize("key", ["eos", "unk", "eom", "padding", "mask", "seperator"])
def test_special_ids_outside_the_vocabulary_are_refused(key):
    name = {"unk": "unknown"}.get(key, key)
    extra = [(f"tokenizer.ggml.{name}_token_id", GW.T_U32, 50)]
    with pytest.raises(nc.NcError, match="out of range for vocab size 50"):
        nc.gguf_stop_tokens(_image("llama", _vocab(50, {}), extra))


def test_files_without_a_usable_tokenizer_are_refused():
    with pytest.raises(nc.NcError, match="tokenizer.ggml.model missing"):
        nc.gguf_stop_tokens(_image(None, None))
    with pytest.raises(nc.NcError, match="unsupported tokenizer model: bert"):
        nc.gguf_stop_tokens(_image("bert", _vocab(10, {})))
    with pytest.raises(nc.NcError, match="tokens missing or invalid"):
        nc.gguf_stop_tokens(_image("llama", None))
    with pytest.raises(nc.NcError, match="must not be empty"):
        nc.gguf_stop_tokens(_image("llama", []))
    meta, ts = GW.read(nc.synth_gguf(**BASE, seed=3).tobytes())
    img = GW.write(list(meta) + [("tokenizer.ggml.model", GW.T_STR, "llama"),
                                 ("tokenizer.ggml.tokens", GW.T_ARR, (GW.T_U32, [1, 2, 3]))], ts)
    with pytest.raises(nc.NcError, match="tokens missing or invalid"):
        nc.gguf_stop_tokens(img)


def test_stop_ids_from_a_file_path(tmp_path):
    p = tmp_path / "m.gguf"
    p.write_bytes(_image("gpt2", _vocab(40, {6: "<|end_of_text|>"})))
    assert nc.gguf_stop_tokens(str(p)).tolist() == [6]
