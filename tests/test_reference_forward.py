"""Model-level pin of the CPU oracle: its logits against an independent float64 forward.

tests/refmodel_np.py restates the reference's dense Llama layer (inference.rs:3747-4111) and
head (inference.rs:4783-4832) in float64 numpy with its own GGUF reader.  The oracle's
verify logits must agree with it within 1e-3 relative (max |diff| / max |logit|) with the
same argmax wherever the float64 top-2 margin is not a near tie.  The toys cover tied and
untied heads, Q4_0 and Q4_K, grouped-query attention (2 and 4 query heads per KV head),
head_dim 64 and 128, and Llama-3 RoPE frequency scaling.

Sensitivity: each planted mistake in the float64 restatement (the residual, the GQA mapping,
RoPE pairing or key position, SwiGLU operand, the final norm, the attention scale) must move the
comparison far outside the tolerance, so the tolerance pins the composition rather than
passing anything.
"""
import numpy as np
import pytest

import nanocamelid_amd as nc
from oracle import oracle as O
from tests import refmodel_np as R

SPECS = {
    "tied-gqa2-hd64": dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512,
                           vocab_size=1000, tied=1, norm_mode=1),
    "untied-gqa4-hd64": dict(layers=2, embedding_length=256, head_count=4, head_count_kv=1, feed_forward_length=768,
                             vocab_size=777, tied=0, norm_mode=1),
    "untied-hd128": dict(layers=1, embedding_length=512, head_count=4, head_count_kv=2, feed_forward_length=512,
                         vocab_size=640, tied=0, norm_mode=1),
    "q4k-tied": dict(layers=2, embedding_length=512, head_count=4, head_count_kv=2, feed_forward_length=1024,
                     vocab_size=500, tied=1, norm_mode=1, weight_type=nc.NC_TYPE_Q4_K),
    "q8_0-untied": dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512,
                        vocab_size=700, tied=0, norm_mode=1, weight_type=nc.NC_TYPE_Q8_0),
    "q5_k": dict(layers=2, embedding_length=512, head_count=4, head_count_kv=2, feed_forward_length=512,
                 vocab_size=600, tied=1, norm_mode=1, weight_type=nc.NC_TYPE_Q5_K),
    "rope-scaled": dict(layers=2, embedding_length=256, head_count=4, head_count_kv=2, feed_forward_length=512,
                        vocab_size=1000, tied=0, norm_mode=1, rope_freq_base=10000.0,
                        rope_scaling=(8.0, 64, 1.0, 4.0)),
}

TOL = 1e-3


def _compare(ref, got):
    scale = float(np.max(np.abs(ref)))
    rel = float(np.max(np.abs(ref - got))) / scale
    top2 = np.sort(ref, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 4 * TOL * scale  # not a near tie in float64
    same = np.argmax(ref, axis=1) == np.argmax(got, axis=1)
    return rel, bool(np.all(same[clear])), int(clear.sum())


def _oracle_logits(img, toks):
    om = O.Model(data=img.tobytes())
    s = O.Session(om, 64, 16)
    _, _, lg = s.verify_greedy(toks, 0, want_logits=True)
    return lg.astype(np.float64)


@pytest.fixture(scope="module", params=sorted(SPECS))
def case(request):
    spec = dict(SPECS[request.param], context_length=256)
    img = nc.synth_gguf(**spec, seed=11 + len(request.param))
    toks = nc.uniform_prompt(5, 14, spec["vocab_size"])
    return request.param, img, toks, _oracle_logits(img, toks)


def test_oracle_logits_match_float64_forward(case):
    name, img, toks, got = case
    ref = R.Model(img).logits(toks)
    rel, argmax_ok, n_clear = _compare(ref, got)
    print(f"{name}: max rel diff {rel:.2e}, argmax checked on {n_clear}/{len(toks)} rows")
    assert rel < TOL, (name, rel)
    assert argmax_ok and n_clear >= len(toks) // 2, name


MUTATIONS = ["no_attn_residual", "gqa_modulo", "rope_neox_pairs", "rope_off_k", "rope_k_pos_plus1",
             "swiglu_swapped", "no_final_norm", "attn_scale_hd"]


def _mutated_logits(m: R.Model, toks, mutation):
    """The float64 forward with one planted mistake."""
    T = len(toks)
    pos = np.arange(T, dtype=np.float64)
    h = m.emb[np.asarray(toks, np.int64)].copy()
    G = m.H // m.Hkv
    causal = np.tril(np.ones((T, T), bool))

    def rope(x, heads, shift=0.0):
        if mutation != "rope_neox_pairs":
            return m._rope(x, pos + shift, heads)
        th = m.theta()
        out = x.copy().reshape(T, heads, m.hd)
        half = m.rope_dim // 2
        ang = pos[:, None] * th[None, :]
        c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        x0, x1 = out[:, :, :half].copy(), out[:, :, half:m.rope_dim].copy()
        out[:, :, :half], out[:, :, half:m.rope_dim] = x0 * c - x1 * s, x0 * s + x1 * c
        return out.reshape(x.shape)

    for ly in m.layers:
        x = R.q8_0(m._norm(h, ly["an"]))
        q = rope(x @ ly["q"].T, m.H).reshape(T, m.H, m.hd)
        kk = x @ ly["k"].T
        shift = 1.0 if mutation == "rope_k_pos_plus1" else 0.0  # keys rotated for the next position
        k = (kk if mutation == "rope_off_k" else rope(kk, m.Hkv, shift)).reshape(T, m.Hkv, m.hd)
        v = (x @ ly["v"].T).reshape(T, m.Hkv, m.hd)
        att = np.zeros((T, m.H, m.hd))
        for hh in range(m.H):
            kv = hh % m.Hkv if mutation == "gqa_modulo" else hh // G
            div = m.hd if mutation == "attn_scale_hd" else np.sqrt(m.hd)
            sc = np.where(causal, (q[:, hh, :] @ k[:, kv, :].T) / div, -np.inf)
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            att[:, hh, :] = (p / p.sum(axis=1, keepdims=True)) @ v[:, kv, :]
        o = R.q8_0(att.reshape(T, -1)) @ ly["o"].T
        h = o if mutation == "no_attn_residual" else h + o
        x = R.q8_0(m._norm(h, ly["fn"]))
        gt, up = x @ ly["g"].T, x @ ly["u"].T
        if mutation == "swiglu_swapped":
            gt, up = up, gt
        h = h + R.q8_0(gt / (1.0 + np.exp(-gt)) * up) @ ly["dn"].T
    hn = h * m.out_norm if mutation == "no_final_norm" else m._norm(h, m.out_norm)
    return R.q8_0(hn) @ m.head.T


@pytest.mark.parametrize("mutation", MUTATIONS)
def test_planted_mistakes_exceed_tolerance(mutation):
    spec = dict(SPECS["tied-gqa2-hd64"], context_length=256)
    img = nc.synth_gguf(**spec, seed=3)
    toks = nc.uniform_prompt(6, 14, spec["vocab_size"])
    got = _oracle_logits(img, toks)
    m = R.Model(img)
    rel_ok, _, _ = _compare(m.logits(toks), got)
    rel_bad, _, _ = _compare(_mutated_logits(m, toks, mutation), got)
    assert rel_ok < TOL
    assert rel_bad > 10 * TOL, (mutation, rel_bad)


def test_rope_scaling_regimes():
    """or_rope_theta with Llama-3 scaling (inference.rs:874-893): pairs whose wavelength is
    below orig/high keep the unscaled theta bit for bit; above orig/low theta is exactly
    theta/factor; between, theta lies in [theta/factor, theta] and falls with the wavelength;
    a factor of 1 changes nothing by more than an ulp; the float64 rule agrees to 1e-6."""
    base, rope_dim = 500000.0, 128
    sc = (32.0, 8192.0, 1.0, 4.0)  # the Llama-3.2 values (main.rs:7132-7155)
    th0 = np.array([O.rope_theta(i, rope_dim, base) for i in range(rope_dim // 2)], np.float32)
    th1 = np.array([O.rope_theta(i, rope_dim, base, sc) for i in range(rope_dim // 2)], np.float32)
    wl = 2 * np.float32(np.pi) / th0
    short, long_ = wl < sc[1] / sc[3], wl > sc[1] / sc[2]
    mid = ~short & ~long_
    assert short.any() and long_.any() and mid.any()
    assert np.array_equal(th1[short].view(np.uint32), th0[short].view(np.uint32))
    assert np.array_equal(th1[long_], (th0[long_] / np.float32(sc[0])).astype(np.float32))
    assert np.all(th1[mid] <= th0[mid]) and np.all(th1[mid] >= th0[mid] / np.float32(sc[0]))
    assert np.all(np.diff(th1[mid] / th0[mid]) <= 0)  # more scaling for longer wavelengths
    th_one = np.array([O.rope_theta(i, rope_dim, base, (1.0, 8192.0, 1.0, 4.0)) for i in range(64)], np.float32)
    assert np.all(np.abs(th_one.view(np.int32) - th0.view(np.int32)) <= 1)
    m = R.Model.__new__(R.Model)
    m.base, m.rope_dim, m.rope_scaling = base, rope_dim, sc
    assert np.allclose(th1, m.theta(), rtol=1e-6, atol=0)


def test_q6_k_float64_decode_matches_oracle():
    """The float64 Q6_K decode against the oracle's (itself pinned by the reference's Q6_K known
    answers), on realistic and full-range random blocks."""
    from tests import gguf_writer as GW
    for raw in (GW.q6_k_weights(40, seed=1), GW.random_blocks(14, 40, seed=2)):
        got = O.dequantize_f32(14, raw, 40 * 256).astype(np.float64)
        ref = R._dequant_q6_k(np.asarray(raw, np.uint8))
        assert np.allclose(got, ref, rtol=1e-6, atol=0)
        assert np.abs(ref).max() > 0


# A Q4_K model with some matrices in other types, as llama.cpp's Q4_K_M recipe stores attn_v
# and ffn_down in Q6_K on some layers: q,k,v and gate,up then no longer share one type.
MIXED_SPEC = dict(layers=2, embedding_length=512, head_count=4, head_count_kv=2, feed_forward_length=1024,
                  vocab_size=500, tied=0, norm_mode=1, weight_type=nc.NC_TYPE_Q4_K, context_length=256)
MIXED_TYPES = {"blk.0.attn_v.weight": 14, "blk.0.attn_output.weight": 14, "blk.1.ffn_down.weight": 14,
               "blk.1.ffn_gate.weight": 14, "blk.1.attn_k.weight": 2}


def mixed_model_image(seed=23):
    from tests import gguf_writer as GW
    return np.frombuffer(GW.with_types(nc.synth_gguf(**MIXED_SPEC, seed=seed), MIXED_TYPES, seed=seed), np.uint8)


def test_mixed_type_layers_match_float64_forward():
    img = mixed_model_image()
    toks = nc.uniform_prompt(6, 14, MIXED_SPEC["vocab_size"])
    ref = R.Model(img).logits(toks)
    rel, argmax_ok, n_clear = _compare(ref, _oracle_logits(img, toks))
    assert rel < TOL, rel
    assert argmax_ok and n_clear >= len(toks) // 2
