"""Independent float64 restatement of the Llama forward pass, for pinning the oracle's layer
composition (test infrastructure; imports neither the product nor the oracle).

It reads a GGUF v3 image with its own parser (gguf.rs:454-551 describes the format), dequantises
Q4_0 / Q4_K weights to float64, and runs the reference's dense layer in float64 with the Q8_0
activation rule applied before every quantized matmul, as run_layer_range_batch does
(inference.rs:3747-4111):

    x = h; h_n = rms_norm(h) * w_attn; q, k, v = W_q/k/v . q8(h_n); RoPE (NORM pairs) on q, k;
    attention of query head h over KV head h // (H / Hkv), causal, softmax(q.k / sqrt(hd));
    h = x + W_o . q8(attn); h_n = rms_norm(h) * w_ffn; a = silu(W_gate . q8(h_n)) * (W_up . q8(h_n));
    h = h + W_down . q8(a); logits = W_head . q8(rms_norm(h) * w_out)          (inference.rs:4783-4832)

A tied model's head is the Q4_0 requantisation of the embedding table (model.rs:471-532 with
q8.rs:2442-2488: d = max/-8 with the signed value of largest magnitude, scale stored as f16
rounded toward zero, q = min(15, trunc(x/d + 8.5))).  Everything is evaluated in float64, so
the results differ from the reference's f32 arithmetic only by rounding, never by structure:
a wrong residual, head mapping, RoPE pairing or norm placement moves the logits far beyond
the 1e-3 relative tolerance the tests use.
"""
from __future__ import annotations

import struct

import numpy as np

# GGUF value types (gguf.rs:25-40): fixed sizes, 8 = string, 9 = array.
_FIXED = {0: ("<B", 1), 1: ("<b", 1), 2: ("<H", 2), 3: ("<h", 2), 4: ("<I", 4), 5: ("<i", 4), 6: ("<f", 4),
          7: ("<?", 1), 10: ("<Q", 8), 11: ("<q", 8), 12: ("<d", 8)}
# tensor types used here: (block elements, block bytes)
_LAYOUT = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


class Gguf:
    def __init__(self, buf: bytes):
        self.buf = memoryview(buf)
        self.pos = 0
        if bytes(self.buf[:4]) != b"GGUF":
            raise ValueError("not a GGUF image")
        self.pos = 4
        self.version = self._u32()
        n_tensors, n_kv = self._u64(), self._u64()
        self.meta = {}
        for _ in range(n_kv):
            key = self._str()
            self.meta[key] = self._value(self._u32())
        infos = []
        for _ in range(n_tensors):
            name = self._str()
            dims = [self._u64() for _ in range(self._u32())]
            infos.append((name, dims, self._u32(), self._u64()))
        align = int(self.meta.get("general.alignment", 32))
        start = (self.pos + align - 1) // align * align
        self.tensors = {n: (d, t, start + off) for n, d, t, off in infos}

    def _take(self, fmt, size):
        v = struct.unpack_from(fmt, self.buf, self.pos)[0]
        self.pos += size
        return v

    def _u32(self):
        return self._take("<I", 4)

    def _u64(self):
        return self._take("<Q", 8)

    def _str(self):
        n = self._u64()
        s = bytes(self.buf[self.pos:self.pos + n]).decode()
        self.pos += n
        return s

    def _value(self, t):
        if t in _FIXED:
            return self._take(*_FIXED[t])
        if t == 8:
            return self._str()
        if t == 9:
            et, n = self._u32(), self._u64()
            return [self._value(et) for _ in range(n)]
        raise ValueError(f"unknown GGUF value type {t}")

    def raw(self, name):
        dims, t, off = self.tensors[name]
        el = int(np.prod(dims))
        be, bb = _LAYOUT[t]
        return t, dims, np.frombuffer(self.buf, np.uint8, el // be * bb, off)

    def f64(self, name) -> np.ndarray:
        """Tensor dequantised to float64, shaped [rows][cols] (GGUF dims are [cols, rows])."""
        t, dims, b = self.raw(name)
        if t == 0:
            v = b.view(np.float32).astype(np.float64)
        elif t == 1:
            v = b.view(np.float16).astype(np.float64)
        elif t == 2:
            v = _dequant_q4_0(b)
        elif t == 8:
            v = _dequant_q8_0(b)
        elif t == 12:
            v = _dequant_q4_k(b)
        elif t == 13:
            v = _dequant_q5_k(b)
        elif t == 14:
            v = _dequant_q6_k(b)
        else:
            raise ValueError(f"type {t}")
        return v.reshape(list(reversed(dims))) if len(dims) > 1 else v


def _dequant_q4_0(b):
    blk = b.reshape(-1, 18)
    d = blk[:, :2].copy().view(np.float16).astype(np.float64)  # [nb, 1]
    q = blk[:, 2:]
    nib = np.concatenate([q & 0x0F, q >> 4], axis=1).astype(np.float64) - 8.0  # element j<16 low, j>=16 high
    return (nib * d).reshape(-1)


def _dequant_q8_0(b):
    # GGML Q8_0 block: f16 scale d, then 32 int8 values q; value = d * q
    blk = b.reshape(-1, 34)
    d = blk[:, :2].copy().view(np.float16).astype(np.float64)
    return (blk[:, 2:].copy().view(np.int8).astype(np.float64) * d).reshape(-1)


def _dequant_q5_k(b):
    # GGML Q5_K: d, dmin (f16), the Q4_K 6-bit scales, qh[32], qs[128]; the value of element
    # 64*pr + 32*half + l is the nibble plus 16 when bit 2*pr + half of qh[l] is set
    blk = b.reshape(-1, 176)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    dmin = blk[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
    sc = blk[:, 4:16].astype(np.int64)
    qh = blk[:, 16:48].astype(np.int64)
    qs = blk[:, 48:].astype(np.int64)
    out = np.zeros((blk.shape[0], 256))
    for j in range(8):
        if j < 4:
            s, m = sc[:, j] & 63, sc[:, j + 4] & 63
        else:
            s = (sc[:, j + 4] & 0x0F) | ((sc[:, j - 4] >> 6) << 4)
            m = (sc[:, j + 4] >> 4) | ((sc[:, j] >> 6) << 4)
        pr, hi = divmod(j, 2)
        byte = qs[:, pr * 32:(pr + 1) * 32]
        q = ((byte >> 4) if hi else (byte & 0x0F)) + 16 * ((qh >> j) & 1)
        out[:, j * 32:(j + 1) * 32] = (d * s)[:, None] * q - (dmin * m)[:, None]
    return out.reshape(-1)


def _dequant_q4_k(b):
    blk = b.reshape(-1, 144)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    dmin = blk[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
    sc = blk[:, 4:16].astype(np.int64)
    qs = blk[:, 16:]
    out = np.zeros((blk.shape[0], 256))
    for j in range(8):  # 6-bit scale / min of sub-block j (the Q4_K packing, q8.rs:2008-2018)
        if j < 4:
            s, m = sc[:, j] & 63, sc[:, j + 4] & 63
        else:
            s = (sc[:, j + 4] & 0x0F) | ((sc[:, j - 4] >> 6) << 4)
            m = (sc[:, j + 4] >> 4) | ((sc[:, j] >> 6) << 4)
        pr, hi = divmod(j, 2)
        byte = qs[:, pr * 32:(pr + 1) * 32]
        nib = (byte >> 4) if hi else (byte & 0x0F)
        out[:, j * 32:(j + 1) * 32] = (d * s)[:, None] * nib - (dmin * m)[:, None]
    return out.reshape(-1)


def _dequant_q6_k(b):
    """Q6_K super-blocks of 256 (ql 128 | qh 64 | int8 scales 16 | f16 d), in llama.cpp's
    published layout: per 128-element half h and l < 32, element 128h + l + 32k takes the low
    (k = 0, 1) or high (k = 2, 3) nibble of ql[64h + l + 32(k % 2)], two bits 2k.. of
    qh[32h + l] on top, minus 32, times d * scale[8h + l // 16 + 2k]."""
    blk = b.reshape(-1, 210)
    ql = blk[:, :128].astype(np.int64)
    qh = blk[:, 128:192].astype(np.int64)
    sc = blk[:, 192:208].view(np.int8).astype(np.float64)
    d = blk[:, 208:210].copy().view(np.float16).astype(np.float64)[:, 0]
    y = np.empty((blk.shape[0], 256))
    for h in range(2):
        for l in range(32):
            lo, hi, bits = ql[:, 64 * h + l], ql[:, 64 * h + l + 32], qh[:, 32 * h + l]
            qs = ((lo & 15) | ((bits & 3) << 4), (hi & 15) | (((bits >> 2) & 3) << 4),
                  (lo >> 4) | (((bits >> 4) & 3) << 4), (hi >> 4) | (((bits >> 6) & 3) << 4))
            for k in range(4):
                y[:, 128 * h + l + 32 * k] = d * sc[:, 8 * h + l // 16 + 2 * k] * (qs[k] - 32)
    return y.ravel()


def q8_0(x: np.ndarray) -> np.ndarray:
    """Q8_0 activation quantisation of the last axis then dequantisation (float64):
    scale = amax/127 per 32-block, q = round half away from zero, clamped to +-127
    (inference.rs:1012-1029)."""
    shp = x.shape
    b = x.reshape(-1, 32)
    amax = np.abs(b).max(axis=1, keepdims=True)
    scale = amax / 127.0
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(scale > 0, b / scale, 0.0)
    q = np.clip(np.sign(r) * np.floor(np.abs(r) + 0.5), -127, 127)
    return (q * scale).reshape(shp)


def _f16_toward_zero(v32: np.ndarray) -> np.ndarray:
    h = v32.astype(np.float16)
    over = np.abs(h.astype(np.float32)) > np.abs(v32)
    h[over] = np.nextafter(h[over], np.float16(0))
    return h


def tied_head_q4_0(emb: np.ndarray) -> np.ndarray:
    """Q4_0 requantisation of the f32 embedding table as the reference builds a tied head,
    returned dequantised (float64)."""
    e = emb.astype(np.float32).reshape(-1, 32)
    idx = np.argmax(np.abs(e), axis=1)  # first index of the largest magnitude
    mx = e[np.arange(e.shape[0]), idx]
    d = (mx / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    q = np.clip(np.trunc((e * inv[:, None] + np.float32(8.5)).astype(np.float32)), 0, 15)
    dh = _f16_toward_zero(d).astype(np.float64)
    return ((q.astype(np.float64) - 8.0) * dh[:, None]).reshape(emb.shape)


class Model:
    def __init__(self, image):
        g = Gguf(bytes(image))
        m = g.meta
        self.d = int(m["llama.embedding_length"])
        self.L = int(m["llama.block_count"])
        self.H = int(m["llama.attention.head_count"])
        self.Hkv = int(m.get("llama.attention.head_count_kv", self.H))
        self.hd = int(m.get("llama.attention.key_length", self.d // self.H))
        self.rope_dim = int(m.get("llama.rope.dimension_count", self.hd))
        self.base = float(m.get("llama.rope.freq_base", 10000.0))
        self.eps = float(m.get("llama.attention.layer_norm_rms_epsilon", 1e-5))
        keys = ("factor", "original_context_length", "low_freq_factor", "high_freq_factor")
        sc = [m.get("llama.rope.scaling." + k) for k in keys]
        self.rope_scaling = tuple(float(v) for v in sc) if all(v is not None for v in sc) else None
        self.emb = g.f64("token_embd.weight")
        self.out_norm = g.f64("output_norm.weight")
        if "output.weight" in g.tensors:
            self.head = g.f64("output.weight")
        else:
            self.head = tied_head_q4_0(self.emb)
        self.layers = []
        for i in range(self.L):
            b = f"blk.{i}."
            self.layers.append({k: g.f64(b + n + ".weight") for k, n in (
                ("an", "attn_norm"), ("fn", "ffn_norm"), ("q", "attn_q"), ("k", "attn_k"), ("v", "attn_v"),
                ("o", "attn_output"), ("g", "ffn_gate"), ("u", "ffn_up"), ("dn", "ffn_down"))})

    def theta(self) -> np.ndarray:
        """RoPE angles per pair; the Llama-3 frequency scaling (Meta's published rule) when the
        file carries it: long wavelengths / factor, short ones unchanged, a linear blend of the
        two in between (inference.rs:874-893)."""
        i = np.arange(self.rope_dim // 2, dtype=np.float64)
        th = self.base ** (-2.0 * i / self.rope_dim)
        if self.rope_scaling:
            factor, orig, low, high = self.rope_scaling
            wl = 2.0 * np.pi / th
            smooth = (orig / wl - low) / (high - low)
            blended = (1.0 - smooth) * th / factor + smooth * th
            th = np.where(wl < orig / high, th, np.where(wl > orig / low, th / factor, blended))
        return th

    def _norm(self, x, w):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.eps) * w

    def _rope(self, x, pos, heads):
        th = self.theta()
        out = x.copy().reshape(x.shape[0], heads, self.hd)
        ang = pos[:, None] * th[None, :]  # [T, pairs]
        c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        x0 = out[:, :, 0:self.rope_dim:2].copy()
        x1 = out[:, :, 1:self.rope_dim:2].copy()
        out[:, :, 0:self.rope_dim:2] = x0 * c - x1 * s  # NORM pairs (2i, 2i+1)
        out[:, :, 1:self.rope_dim:2] = x0 * s + x1 * c
        return out.reshape(x.shape)

    def logits(self, tokens, start=0, past=None) -> np.ndarray:
        """Logits [T][V] of every position of `tokens` at positions start..start+T-1, causal.
        past[layer] = (keys, values), each [start][Hkv*hd]: the cache rows before `start` as
        stored (keys after RoPE)."""
        T = len(tokens)
        pos = np.arange(start, start + T, dtype=np.float64)
        h = self.emb[np.asarray(tokens, np.int64)].copy()
        G = self.H // self.Hkv
        causal = np.arange(start + T)[None, :] <= (start + np.arange(T))[:, None]
        for li, ly in enumerate(self.layers):
            x = q8_0(self._norm(h, ly["an"]))
            q = self._rope(x @ ly["q"].T, pos, self.H).reshape(T, self.H, self.hd)
            k = self._rope(x @ ly["k"].T, pos, self.Hkv).reshape(T, self.Hkv, self.hd)
            v = (x @ ly["v"].T).reshape(T, self.Hkv, self.hd)
            if start:
                k = np.concatenate([np.asarray(past[li][0], np.float64).reshape(start, self.Hkv, self.hd), k])
                v = np.concatenate([np.asarray(past[li][1], np.float64).reshape(start, self.Hkv, self.hd), v])
            att = np.zeros((T, self.H, self.hd))
            for hh in range(self.H):
                kv = hh // G
                sc = (q[:, hh, :] @ k[:, kv, :].T) / np.sqrt(self.hd)
                sc = np.where(causal, sc, -np.inf)
                p = np.exp(sc - sc.max(axis=1, keepdims=True))
                p /= p.sum(axis=1, keepdims=True)
                att[:, hh, :] = p @ v[:, kv, :]
            h = h + q8_0(att.reshape(T, -1)) @ ly["o"].T
            x = q8_0(self._norm(h, ly["fn"]))
            gt, up = x @ ly["g"].T, x @ ly["u"].T
            a = gt / (1.0 + np.exp(-gt)) * up
            h = h + q8_0(a) @ ly["dn"].T
        return q8_0(self._norm(h, self.out_norm)) @ self.head.T
