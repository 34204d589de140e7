"""GGUF reader, tensor validation and f32 decoding of the loader (CPU, no GPU).

Pins, per function:
  tensor_nbytes / the type layout table: the reference's own known answers (gguf.rs:440-451,
    Q5_0/Q5_1 at [896, 151936]) and its layout table (gguf.rs:154-185), plus its error cases
    (unknown type, first dimension not a whole number of blocks, duplicate names, bad alignment);
  load_f32_or_f16 (model.rs:1081-1229): the reference's block-decoding known answers
    (q8.rs:4566-4589 Q4_1, q8.rs:4647-4665 Q6_K), product == oracle bit for bit on random blocks
    of every type, and both within float32 rounding of a float64 decoder written from the GGML
    block formats (which would catch a wrong index, nibble order or sign);
  validate_model_tensors (model.rs:851-1036): each refusal, on images edited from a valid one.
"""
import struct

import numpy as np
import pytest

import nanocamelid_amd as nc
from oracle import oracle as O
from tests import gguf_writer as GW
from tests.gguf_writer import random_blocks

# GgufTensorType::layout (gguf.rs:154-185): id -> (values per block, bytes per block)
REF_LAYOUT = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 36),
              10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292),
              16: (256, 66), 17: (256, 74), 18: (256, 98), 19: (256, 50), 20: (32, 18), 21: (256, 110),
              22: (256, 82), 23: (256, 136), 24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8),
              29: (256, 56), 30: (1, 2)}


def _header_only(tensors):
    return GW.write([("general.alignment", GW.T_U32, 32)], [(n, d, t, b"") for n, d, t in tensors], data=False)


def test_tensor_nbytes_reference_known_answers():
    # gguf.rs:440-451 q5_0_and_q5_1_have_distinct_block_sizes
    img = _header_only([("q5_0", [896, 151936], 6), ("q5_1", [896, 151936], 7)])
    ts = {name: (ty, nb) for name, dims, ty, off, nb in nc.gguf_tensors(img)}
    assert ts["q5_0"] == (6, 93_592_576)
    assert ts["q5_1"] == (7, 102_100_992)


def test_type_layout_table():
    for ty, (bs, tsz) in REF_LAYOUT.items():
        img = _header_only([("t", [bs * 4, 3], ty)])
        (_, dims, t, off, nb), = nc.gguf_tensors(img)
        assert (t, nb) == (ty, 4 * 3 * tsz), ty


@pytest.mark.parametrize("tensors,msg", [
    ([("x", [32, 2], 4)], "unknown or removed GGML type"),        # id 4 (Q4_2) was removed
    ([("x", [32, 2], 99)], "unknown or removed GGML type"),
    ([("x", [48, 2], 2)], "not divisible by block size"),
    ([("x", [32], 0), ("x", [32], 0)], "duplicate tensor name"),
])
def test_reader_refusals(tensors, msg):
    with pytest.raises(nc.NcError, match=msg):
        nc.gguf_tensors(_header_only(tensors))


def test_reader_alignment_and_data_start():
    bad = GW.write([("general.alignment", GW.T_U32, 24)], [("x", [32], 0, b"")], alignment=32, data=False)
    with pytest.raises(nc.NcError, match="alignment"):
        nc.gguf_tensors(bad)
    img = _header_only([("x", [32], 0)])
    with pytest.raises(nc.NcError, match="overflows file|truncated"):
        nc.gguf_tensors(img[:len(img) - 8])


# ---------------------------------------------------------------- f32 decoding
def _k_scale_min(sc, j):
    # 6-bit scale and min of sub-block j from the 12 packed bytes (GGML get_scale_min_k4)
    if j < 4:
        return sc[..., j] & 63, sc[..., j + 4] & 63
    return ((sc[..., j + 4] & 15) | ((sc[..., j - 4] >> 6) << 4),
            (sc[..., j + 4] >> 4) | ((sc[..., j] >> 6) << 4))


def decode_f64(ty, raw, n):
    """float64 decode written from the GGML block formats."""
    h = lambda a: a.copy().view(np.float16).astype(np.float64)  # noqa: E731
    if ty == 0:
        return raw.view(np.float32).astype(np.float64)
    if ty == 1:
        return raw.view(np.float16).astype(np.float64)
    if ty == 30:
        return (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    bs, tsz = REF_LAYOUT[ty]
    b = raw.reshape(-1, tsz)
    out = np.zeros((b.shape[0], bs))
    if ty == 8:
        return (h(b[:, :2]).ravel()[:, None] * b[:, 2:].view(np.int8)).ravel()
    if ty in (2, 3, 6, 7):
        d = h(b[:, :2]).ravel()[:, None]
        m = h(b[:, 2:4]).ravel()[:, None] if ty in (3, 7) else 0.0
        qh_off = {2: None, 3: None, 6: 2, 7: 4}[ty]
        qs = b[:, {2: 2, 3: 4, 6: 6, 7: 8}[ty]:].astype(np.int64)
        q = np.concatenate([qs & 15, qs >> 4], axis=1)
        if qh_off is not None:
            hb = b[:, qh_off:qh_off + 4].copy().view(np.uint32).astype(np.int64)
            q = q | (((hb >> np.arange(32)) & 1) << 4)
        if ty == 2:
            q = q - 8
        if ty == 6:
            q = q - 16
        return (d * q + m).ravel()
    if ty in (12, 13):
        d, dmin = h(b[:, 0:2]).ravel(), h(b[:, 2:4]).ravel()
        sc = b[:, 4:16].astype(np.int64)
        qs = b[:, 16:].astype(np.int64) if ty == 12 else b[:, 48:].astype(np.int64)
        qh = b[:, 16:48].astype(np.int64) if ty == 13 else None
        for j in range(8):
            s, mn = _k_scale_min(sc, j)
            p, hi = j // 2, j % 2
            q = (qs[:, 32 * p:32 * p + 32] >> (4 * hi)) & 15
            if qh is not None:
                q = q + 16 * ((qh >> j) & 1)
            out[:, 32 * j:32 * j + 32] = (d * s)[:, None] * q - (dmin * mn)[:, None]
        return out.ravel()
    if ty == 14:
        ql, qh = b[:, :128].astype(np.int64), b[:, 128:192].astype(np.int64)
        sc, d = b[:, 192:208].view(np.int8).astype(np.int64), h(b[:, 208:210]).ravel()
        for half in range(2):
            for l in range(32):
                lo, hi, hb = ql[:, 64 * half + l], ql[:, 64 * half + l + 32], qh[:, 32 * half + l]
                qv = [(lo & 15) | ((hb & 3) << 4), (hi & 15) | (((hb >> 2) & 3) << 4),
                      (lo >> 4) | (((hb >> 4) & 3) << 4), (hi >> 4) | (((hb >> 6) & 3) << 4)]
                for k in range(4):
                    out[:, 128 * half + 32 * k + l] = d * sc[:, 8 * half + l // 16 + 2 * k] * (qv[k] - 32)
        return out.ravel()
    raise ValueError(ty)


def test_dequant_reference_known_answers():
    # q8.rs:4647-4665 q6_k_block_dequantizes_quantized_values_and_scales
    ql, qh = np.zeros(128, np.uint8), np.zeros(64, np.uint8)
    ql[0], ql[32], qh[0] = 0x10, 0x02, 0b11_10_01_00
    blk = np.concatenate([ql, qh, np.ones(16, np.int8).view(np.uint8), np.frombuffer(struct.pack("<H", 0x3c00), np.uint8)])
    for v in (nc.dequantize_f32(14, blk, 256), O.dequantize_f32(14, blk, 256)):
        assert (v[0], v[32], v[64], v[96]) == (-32.0, -14.0, 1.0, 16.0)
    # q8.rs:4566-4589 q4_1_block_decodes_low_then_high_nibbles_with_scale_and_min: scale 1.0,
    # min 0.5, bytes idx | (15 - idx) << 4 -> values v0 = 0, v15 = 15, v16 = 15, v31 = 0
    q41 = np.concatenate([np.frombuffer(struct.pack("<HH", 0x3c00, 0x3800), np.uint8),
                          np.array([i | ((15 - i) << 4) for i in range(16)], np.uint8)])
    for v in (nc.dequantize_f32(3, q41, 32), O.dequantize_f32(3, q41, 32)):
        assert (v[0], v[15], v[16], v[31]) == (0.5, 15.5, 15.5, 0.5)


@pytest.mark.parametrize("ty", [0, 1, 30, 8, 2, 3, 6, 7, 12, 13, 14])
def test_dequant_product_equals_oracle_and_format(ty):
    bs, _ = REF_LAYOUT[ty]
    nblk = 64 if bs > 1 else 4096
    raw = random_blocks(ty, nblk, seed=ty)
    n = nblk * bs
    got, ref = nc.dequantize_f32(ty, raw, n), O.dequantize_f32(ty, raw, n)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    exact = decode_f64(ty, raw, n)
    assert np.all(np.abs(got - exact) <= 4e-7 * np.abs(exact) + 1e-30), ty


def test_dequant_refuses_unsupported_types():
    with pytest.raises(nc.NcError, match="unsupported type"):
        nc.dequantize_f32(10, np.zeros(84, np.uint8), 256)  # Q2_K: no embedding decode in this build


# ---------------------------------------------------------------- validate_model_tensors
SPEC = dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512, vocab_size=300,
            context_length=128)


@pytest.fixture(scope="module")
def base():
    return GW.read(nc.synth_gguf(**SPEC, seed=3).tobytes())


def _edit(base, drop=(), add=(), replace=None):
    meta, ts = base
    out = [t for t in ts if t[0] not in drop]
    if replace:
        out = [replace.get(t[0], t) for t in out]
    return GW.write(meta, out + list(add))


def test_valid_image_and_config(base):
    cfg = nc.gguf_read_config(_edit(base))
    assert (cfg["embedding_length"], cfg["vocab_size"], cfg["block_count"]) == (256, 300, 2)


def _norm(name, n=256):
    return (name, [n], 0, np.ones(n, np.float32).tobytes())


@pytest.mark.parametrize("case,msg", [
    (dict(drop=["blk.1.ffn_norm.weight"]), "blk.1.ffn_norm.weight not found"),
    (dict(replace={"output_norm.weight": _norm("output_norm.weight", 512)}), "output norm tensor .* expected descriptor shape"),
    (dict(add=[("blk.0.attn_qkv.weight", [256, 512], 2, bytes(512 * 8 * 18))]), "fused q|k|v"),
    (dict(add=[_norm("blk.0.attn_q.bias")]), "attention biases"),
    (dict(add=[("blk.1.ffn_gate_inp.weight", [256, 4], 0, bytes(256 * 4 * 4))]), "mixture-of-experts"),
    (dict(drop=["blk.0.ffn_gate.weight"]), "fused ffn gate"),
    (dict(replace={"blk.0.attn_k.weight": ("blk.0.attn_k.weight", [256, 256], 2, bytes(256 * 8 * 18))}),
     "layer 0 attention k tensor .* expected descriptor shape \\[256, 128\\] or \\[128, 256\\]"),
])
def test_validation_refusals(base, case, msg):
    with pytest.raises(nc.NcError, match=msg):
        nc.gguf_read_config(_edit(base, **case))


def test_transposed_matrix_passes_validation(base):
    # the reference accepts either descriptor orientation at validation (model.rs:1459-1475);
    # the upload then refuses output-major storage, which this build does not run
    meta, ts = base
    q = [t for t in ts if t[0] == "blk.0.attn_k.weight"][0]
    assert q[1] == [256, 128]
    nc.gguf_read_config(_edit(base, replace={q[0]: (q[0], [128, 256], q[2], q[3])}))


@pytest.mark.parametrize("ty", [1, 30, 8, 3, 14])
def test_embedding_types_pass_validation(base, ty):
    raw = random_blocks(ty, 256 * 300 // REF_LAYOUT[ty][0], seed=ty).tobytes()
    img = _edit(base, replace={"token_embd.weight": ("token_embd.weight", [256, 300], ty, raw)})
    assert nc.gguf_read_config(img)["vocab_size"] == 300


def test_weight_type_names_the_first_attention_query_matrix():
    # weight_type reports blk.0.attn_q.weight's type; a file that mixes types per matrix (the
    # Q4_K_M recipe's Q6_K attn_v / ffn_down) keeps it, whatever the other matrices are
    img = nc.synth_gguf(**SPEC, seed=3)
    assert nc.gguf_read_config(bytes(img))["weight_type"] == nc.NC_TYPE_Q4_0
    mixed = GW.with_types(img, {"blk.0.attn_v.weight": nc.NC_TYPE_Q6_K, "blk.1.ffn_down.weight": nc.NC_TYPE_Q6_K,
                             "blk.1.attn_q.weight": nc.NC_TYPE_Q6_K})
    assert nc.gguf_read_config(mixed)["weight_type"] == nc.NC_TYPE_Q4_0
    first_q6 = GW.with_types(img, {"blk.0.attn_q.weight": nc.NC_TYPE_Q6_K})
    assert nc.gguf_read_config(first_q6)["weight_type"] == nc.NC_TYPE_Q6_K
