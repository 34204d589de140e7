"""ctypes wrapper over the CPU oracle (oracle/_build/libncoracle.so).

TEST INFRASTRUCTURE ONLY: the oracle is a restatement of the reference's
portable x86 path (see oracle/nc_oracle.h).  Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg import this module; the product package never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libncoracle.so")

_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i64 = C.c_int64

_lib = None


def build() -> None:
    """Compile the oracle with its own Makefile (g++ -O2 -ffp-contract=off)."""
    subprocess.run(["make", "-B", "-C", _HERE], check=True, capture_output=True)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = C.CDLL(LIB_PATH)
    sig = {
        "or_f16_to_f32": (C.c_float, [C.c_uint16]),
        "or_f32_to_f16_trunc": (C.c_uint16, [C.c_float]),
        "or_dot_q4_0_q8_0": (C.c_int32, [_u8p, _i8p]),
        "or_dot_i8": (C.c_int32, [_i8p, _i8p, _i64]),
        "or_q4_k_subblock_ints": (None, [_u8p, _i8p, _i32p, _i32p]),
        "or_q4_k_dot": (C.c_float, [_u8p, _i8p, _f32p]),
        "or_q4_k_dequantize": (None, [_u8p, _f32p]),
        "or_dequantize_f32": (C.c_int, [C.c_int, _u8p, _i64, _f32p]),
        "or_quantize_q8_0": (None, [_f32p, _i64, _i8p, _f32p]),
        "or_quantize_q4_0_tied": (None, [_f32p, _i64, _i64, _u8p]),
        "or_matmul_q4_0": (None, [_f32p, _i8p, _f32p, _u8p, _i64, _i64, _i64, C.c_int]),
        "or_matmul_q4_0_blockdots": (None, [_i32p, _i8p, _u8p, _i64, _i64, _i64, C.c_int]),
        "or_matmul_q8_0": (None, [_f32p, _i8p, _f32p, _u8p, _i64, _i64, _i64, C.c_int]),
        "or_matmul_q5_k": (None, [_f32p, _i8p, _f32p, _u8p, _i64, _i64, _i64, C.c_int]),
        "or_matmul_q4_k": (None, [_f32p, _i8p, _f32p, _u8p, _i64, _i64, _i64, C.c_int]),
        "or_matmul_q6_k": (None, [_f32p, _i8p, _f32p, _u8p, _i64, _i64, _i64, C.c_int]),
        "or_q6_k_dot": (C.c_float, [_u8p, _i8p, _f32p]),
        "or_rms_norm": (None, [_f32p, _f32p, _f32p, _i64, C.c_float]),
        "or_rope": (None, [_f32p, _i64, _i64, _i64, _i64, C.c_float, C.c_int]),
        "or_rope_sincos": (None, [_i64, _i64, _i64, C.c_float, C.POINTER(C.c_float), C.POINTER(C.c_float)]),
        "or_rope_theta": (C.c_float, [_i64, _i64, C.c_float, C.c_void_p]),
        "or_softmax": (None, [_f32p, _i64]),
        "or_expf": (C.c_float, [C.c_float]),
        "or_expf_mismatches": (C.c_int64, [C.c_uint32, C.c_int64, C.c_void_p, C.c_int, C.c_void_p]),
        "or_silu_mul": (None, [_f32p, _f32p, _f32p, _i64]),
        "or_argmax": (_i64, [_f32p, _i64]),
        "or_rand_simple": (C.c_float, [C.POINTER(C.c_uint64)]),
        "or_sample_logits": (_i64, [_f32p, _i64, C.c_float, C.POINTER(C.c_uint64)]),
        "or_generate_speculative_draft_temp": (_i64, [C.c_void_p, C.c_void_p, _u32p, _i64, _i64, _i64, C.c_float,
                                                      C.POINTER(C.c_uint64), _u32p, _i64, _i64, _u32p, _i64p,
                                                      _i64p]),
        "or_attention_head": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, C.c_float]),
        "or_attention_head_split": (None, [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64, C.c_float]),
        "or_philox4x32_10": (None, [_u32p, _u32p, _u32p]),
        "or_model_load": (C.c_void_p, [C.c_char_p, C.c_int, C.c_char_p, C.c_int]),
        "or_model_load_memory": (C.c_void_p, [C.c_void_p, C.c_size_t, C.c_int, C.c_char_p, C.c_int]),
        "or_model_free": (None, [C.c_void_p]),
        "or_model_info": (None, [C.c_void_p, _i64p]),
        "or_model_info_f": (None, [C.c_void_p, _f32p]),
        "or_model_head_q4_0": (_i64, [C.c_void_p, _u8p, _i64]),
        "or_session_create": (C.c_void_p, [C.c_void_p, _i64, _i64]),
        "or_model_set_threads": (None, [C.c_void_p, C.c_int]),
        "or_session_fill_kv": (None, [C.c_void_p, _i64, C.c_uint64]),
        "or_synth_kv_values": (None, [C.c_uint64, C.c_int32, C.c_int32, _i64, _i64, _f32p]),
        "or_session_free": (None, [C.c_void_p]),
        "or_session_set_attention": (None, [C.c_void_p, C.c_int]),
        "or_prefill_pass_batch": (None, [C.c_void_p, _u32p, _i64, _i64]),
        "or_forward_pass": (None, [C.c_void_p, C.c_uint32, _i64]),
        "or_batch_row_logits": (None, [C.c_void_p, _i64, _f32p]),
        "or_session_logits": (C.POINTER(C.c_float), [C.c_void_p]),
        "or_session_batch_hidden": (C.POINTER(C.c_float), [C.c_void_p]),
        "or_verify_greedy": (None, [C.c_void_p, _u32p, _i64, _i64, _u32p, C.c_void_p, C.c_void_p]),
        "or_generate_greedy": (C.c_int, [C.c_void_p, _u32p, _i64, _i64, _i64, _u32p]),
        "or_generate_plain": (_i64, [C.c_void_p, _u32p, _i64, _i64, C.c_float, C.POINTER(C.c_uint64), _u32p,
                                     _i64, _i64, _u32p]),
        "or_generate_speculative_draft": (_i64, [C.c_void_p, C.c_void_p, _u32p, _i64, _i64, _i64, _i64, _u32p, _i64p, _i64p]),
        "or_generate_speculative_stochastic": (_i64, [C.c_void_p, C.c_void_p, _u32p, _i64, _i64, _i64, C.c_float, C.c_uint64, _i64, _u32p, _i64p, _i64p]),
        "or_generate_speculative_oracle": (_i64, [C.c_void_p, _u32p, _i64, _i64, _i64, C.c_float, C.c_uint64, _u32p, _i64, _u32p, _i64p, _i64p]),
        "or_oracle_draft": (C.c_uint32, [C.c_uint64, _i64, C.c_float, _u32p, _i64, _i64, C.c_uint32]),
        "or_ngram_draft": (_i64, [_u32p, _i64, _i64, _i64, _i64, _u32p]),
        "or_generate_speculative_ngram": (_i64, [C.c_void_p, _u32p, _i64, _i64, _i64, _i64, _i64, _u32p, _i64, _i64,
                                                 _u32p, _i64p, _i64p]),
        "or_generate_speculative_ngram_temp": (_i64, [C.c_void_p, _u32p, _i64, _i64, _i64, _i64, _i64, C.c_float,
                                                      C.POINTER(C.c_uint64), _u32p, _i64, _i64, _u32p, _i64p,
                                                      _i64p]),
        "or_uniform_prompt": (None, [C.c_uint64, _i64, C.c_uint32, _u32p]),
        "or_stochastic_accept": (None, [_f32p, _f32p, _u32p, _i64, _i64, C.c_float, C.c_uint64, _i64, C.POINTER(_i64), C.POINTER(C.c_uint32)]),
        "or_temperature_probs": (None, [_f32p, _i64, C.c_float, _f32p]),
        "or_sample_inverse_cdf": (C.c_uint32, [_f32p, _i64, C.c_float]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- formats / ops
def f16_to_f32(bits: int) -> float:
    return lib().or_f16_to_f32(bits)


def f32_to_f16_trunc(v: float) -> int:
    return lib().or_f32_to_f16_trunc(v)


def dot_q4_0_q8_0(block18, x32) -> int:
    return lib().or_dot_q4_0_q8_0(_c(block18, np.uint8), _c(x32, np.int8))


def dot_i8(a, b) -> int:
    a = _c(a, np.int8)
    return lib().or_dot_i8(a, _c(b, np.int8), a.size)


def quantize_q8_0(x):
    x = _c(x, np.float32)
    q = np.zeros(x.size, np.int8)
    s = np.zeros(x.size // 32, np.float32)
    lib().or_quantize_q8_0(x.ravel(), x.size, q, s)
    return q, s


def quantize_q4_0_tied(values, rows, cols):
    out = np.zeros(rows * (cols // 32) * 18, np.uint8)
    lib().or_quantize_q4_0_tied(_c(values, np.float32).ravel(), rows, cols, out)
    return out


def matmul_q4_0(x_i8, x_scales, w_blocks, N, M, K, nthreads=8):
    out = np.zeros(N * M, np.float32)
    lib().or_matmul_q4_0(out, _c(x_i8, np.int8).ravel(), _c(x_scales, np.float32).ravel(),
                         _c(w_blocks, np.uint8).ravel(), N, M, K, nthreads)
    return out.reshape(N, M)


def matmul_q4_0_blockdots(x_i8, w_blocks, N, M, K, nthreads=8):
    out = np.zeros(N * M * (K // 32), np.int32)
    lib().or_matmul_q4_0_blockdots(out, _c(x_i8, np.int8).ravel(), _c(w_blocks, np.uint8).ravel(), N, M, K, nthreads)
    return out.reshape(N, M, K // 32)


def matmul_q8_0(x_i8, x_scales, w_blocks, N, M, K, nthreads=8):
    out = np.zeros(N * M, np.float32)
    lib().or_matmul_q8_0(out, _c(x_i8, np.int8).ravel(), _c(x_scales, np.float32).ravel(),
                         _c(w_blocks, np.uint8).ravel(), N, M, K, nthreads)
    return out.reshape(N, M)


def matmul_q5_k(x_i8, x_scales, w_blocks, N, M, K, nthreads=8):
    out = np.zeros(N * M, np.float32)
    lib().or_matmul_q5_k(out, _c(x_i8, np.int8).ravel(), _c(x_scales, np.float32).ravel(),
                         _c(w_blocks, np.uint8).ravel(), N, M, K, nthreads)
    return out.reshape(N, M)


def matmul_q4_k(x_i8, x_scales, w_blocks, N, M, K, nthreads=8):
    out = np.zeros(N * M, np.float32)
    lib().or_matmul_q4_k(out, _c(x_i8, np.int8).ravel(), _c(x_scales, np.float32).ravel(),
                         _c(w_blocks, np.uint8).ravel(), N, M, K, nthreads)
    return out.reshape(N, M)


def matmul_q6_k(x_i8, x_scales, w_blocks, N, M, K, nthreads=8):
    out = np.zeros(N * M, np.float32)
    lib().or_matmul_q6_k(out, _c(x_i8, np.int8).ravel(), _c(x_scales, np.float32).ravel(),
                         _c(w_blocks, np.uint8).ravel(), N, M, K, nthreads)
    return out.reshape(N, M)


def q6_k_dot(block210, x256, xs8) -> float:
    return float(lib().or_q6_k_dot(_c(block210, np.uint8).ravel(), _c(x256, np.int8).ravel(),
                                   _c(xs8, np.float32).ravel()))


def q4_k_subblock_ints(block144, x256):
    W = np.zeros(8, np.int32)
    A = np.zeros(8, np.int32)
    lib().or_q4_k_subblock_ints(_c(block144, np.uint8), _c(x256, np.int8), W, A)
    return W, A


def q4_k_dequantize(block144):
    out = np.zeros(256, np.float32)
    lib().or_q4_k_dequantize(_c(block144, np.uint8), out)
    return out


def dequantize_f32(ggml_type, data, n):
    """load_f32_or_f16 (model.rs:1081-1229): n values of one tensor's bytes as f32."""
    out = np.zeros(n, np.float32)
    if lib().or_dequantize_f32(int(ggml_type), _c(data, np.uint8).ravel(), n, out) != 0:
        raise ValueError(f"unsupported GGML type {ggml_type}")
    return out


def rms_norm(x, w, eps):
    x = _c(x, np.float32)
    out = np.zeros_like(x)
    lib().or_rms_norm(out, x, _c(w, np.float32), x.size, eps)
    return out


def rope(data, pos, heads, head_dim, rope_dim, base, style=0):
    d = _c(data, np.float32).copy()
    lib().or_rope(d, pos, heads, head_dim, rope_dim, base, style)
    return d


def rope_sincos(pos, i, rope_dim, base):
    s, c = C.c_float(), C.c_float()
    lib().or_rope_sincos(pos, i, rope_dim, base, C.byref(s), C.byref(c))
    return s.value, c.value


def rope_theta(i, rope_dim, base, scaling=None):
    """theta of RoPE pair i (inference.rs:874-893), Llama-3 scaled when scaling =
    (factor, original_context_length, low_freq_factor, high_freq_factor)."""
    sc = np.asarray(scaling, np.float32) if scaling is not None else None
    return lib().or_rope_theta(i, rope_dim, base, sc.ctypes.data if sc is not None else None)


def softmax(x):
    x = _c(x, np.float32).copy()
    lib().or_softmax(x, x.size)
    return x


def expf(x: float) -> float:
    return lib().or_expf(x)


def expf_mismatches(first: int, vals: np.ndarray, nthreads: int = 16):
    """(mismatch count, first mismatching input bits) of vals[i] against glibc expf of the float
    with bits first + i."""
    vals = np.ascontiguousarray(vals, np.float32)
    fb = C.c_uint32(0)
    n = lib().or_expf_mismatches(first, vals.size, vals.ctypes.data, nthreads, C.byref(fb))
    return int(n), int(fb.value)


def silu_mul(g, u):
    g = _c(g, np.float32)
    out = np.zeros_like(g)
    lib().or_silu_mul(out, g, _c(u, np.float32), g.size)
    return out


def argmax(logits) -> int:
    logits = _c(logits, np.float32)
    return lib().or_argmax(logits, logits.size)


REFERENCE_RNG_STATE = 0x123456789ABCDEF0  # inference.rs:4875


def rand_simple(state: int):
    """inference.rs:4876-4883: (u, new state)."""
    st = C.c_uint64(state)
    u = lib().or_rand_simple(C.byref(st))
    return u, int(st.value)


def sample_logits(logits, temp: float, state: int = REFERENCE_RNG_STATE):
    """inference.rs:4834-4873: (index, new state)."""
    st = C.c_uint64(state)
    i = lib().or_sample_logits(_c(logits, np.float32), np.asarray(logits).size, float(temp), C.byref(st))
    return int(i), int(st.value)


def attention_head(q_head, k_cache, v_cache, pos, kv_width, kv_h, head_dim, scale):
    out = np.zeros(head_dim, np.float32)
    scores = np.zeros(pos + 1, np.float32)
    lib().or_attention_head(out, scores, _c(q_head, np.float32), _c(k_cache, np.float32).ravel(),
                            _c(v_cache, np.float32).ravel(), pos, kv_width, kv_h, head_dim, scale)
    return out


def attention_head_split(q_head, k_cache, v_cache, pos, plast, kv_width, kv_h, head_dim, scale):
    """The device's split-order attention head (64-position chunks combined in order)."""
    out = np.zeros(head_dim, np.float32)
    lib().or_attention_head_split(out, _c(q_head, np.float32), _c(k_cache, np.float32).ravel(),
                                  _c(v_cache, np.float32).ravel(), pos, plast, kv_width, kv_h, head_dim, scale)
    return out


def philox4x32_10(ctr, key):
    out = np.zeros(4, np.uint32)
    lib().or_philox4x32_10(_c(ctr, np.uint32), _c(key, np.uint32), out)
    return out


def synth_kv_values(seed, layer, kind, start, count):
    out = np.zeros(count, np.float32)
    lib().or_synth_kv_values(seed, layer, kind, start, count, out)
    return out


def uniform_prompt(seed, n, vocab):
    ids = np.zeros(n, np.uint32)
    lib().or_uniform_prompt(seed, n, vocab, ids)
    return ids


def oracle_draft(seed, p, alpha, greedy, n_prompt, vocab):
    g = _c(greedy, np.uint32)
    return lib().or_oracle_draft(seed, p, alpha, g, n_prompt, g.size, vocab)


def ngram_draft(history, max_tokens, min_ngram=3, max_ngram=4):
    """NGramDrafter::draft (speculative.rs:81-103); defaults as NGramDrafter::default."""
    h = _c(history, np.uint32)
    out = np.zeros(max(int(max_tokens), 1), np.uint32)
    n = lib().or_ngram_draft(h, h.size, min_ngram, max_ngram, max_tokens, out)
    return out[:n]


def temperature_probs(logits, temp):
    logits = _c(logits, np.float32)
    out = np.zeros_like(logits)
    lib().or_temperature_probs(logits, logits.size, temp, out)
    return out


def sample_inverse_cdf(probs, u):
    probs = _c(probs, np.float32)
    return lib().or_sample_inverse_cdf(probs, probs.size, u)


def stochastic_accept(p_logits, q_probs, drafts, temp, seed, start_pos):
    p_logits = _c(p_logits, np.float32)
    k = len(drafts)
    V = p_logits.shape[-1]
    na = _i64()
    nt = C.c_uint32()
    lib().or_stochastic_accept(p_logits.ravel(), _c(q_probs, np.float32).ravel(), _c(drafts, np.uint32),
                               k, V, temp, seed, start_pos, C.byref(na), C.byref(nt))
    return na.value, nt.value


# ---------------------------------------------------------------- model / session
MODEL_FIELDS = ("context_length", "d", "layers", "ffn", "heads", "kv_heads", "head_dim", "rope_dim",
                "vocab", "attn_width", "kv_width", "has_output", "weight_type")


class Model:
    def __init__(self, path=None, data=None, nthreads=8):
        err = C.create_string_buffer(512)
        L = lib()
        if data is not None:
            self._buf = data  # keep alive: the oracle parses the image in place
            arr = np.frombuffer(data, np.uint8)
            h = L.or_model_load_memory(arr.ctypes.data, arr.size, nthreads, err, 512)
        else:
            h = L.or_model_load(path.encode(), nthreads, err, 512)
        if not h:
            raise RuntimeError("oracle model load failed: " + err.value.decode())
        self.h = h
        info = np.zeros(16, np.int64)
        L.or_model_info(h, info)
        self.info = {k: int(v) for k, v in zip(MODEL_FIELDS, info)}
        fl = np.zeros(2, np.float32)
        L.or_model_info_f(h, fl)
        self.rope_base, self.eps = float(fl[0]), float(fl[1])

    def set_threads(self, n: int):
        lib().or_model_set_threads(self.h, int(n))

    def head_q4_0(self):
        n = self.info["vocab"] * (self.info["d"] // 32) * 18
        out = np.zeros(n, np.uint8)
        assert lib().or_model_head_q4_0(self.h, out, n) == n
        return out

    def close(self):
        if self.h:
            lib().or_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Session:
    def __init__(self, model: Model, max_ctx: int, max_batch: int):
        self.model = model
        self.h = lib().or_session_create(model.h, max_ctx, max_batch)
        self.V = model.info["vocab"]
        self.d = model.info["d"]

    def prefill_pass_batch(self, toks, start_pos):
        t = _c(toks, np.uint32)
        lib().or_prefill_pass_batch(self.h, t, t.size, start_pos)

    def forward_pass(self, tok, pos):
        lib().or_forward_pass(self.h, int(tok), pos)
        return np.ctypeslib.as_array(lib().or_session_logits(self.h), (self.V,)).copy()

    def set_attention(self, order):
        """0: the reference's attention order (default); 1: the device's split order."""
        lib().or_session_set_attention(self.h, int(order))

    def fill_kv(self, n, seed=1):
        """N(0, 1) keys and values in KV rows [0, n) of every layer (or_synth_kv_values streams)."""
        lib().or_session_fill_kv(self.h, n, seed)

    def batch_row_logits(self, row):
        out = np.zeros(self.V, np.float32)
        lib().or_batch_row_logits(self.h, row, out)
        return out

    def batch_hidden(self, n):
        return np.ctypeslib.as_array(lib().or_session_batch_hidden(self.h), (n * self.d,)).copy().reshape(n, self.d)

    def verify_greedy(self, toks, start_pos, want_logits=False):
        t = _c(toks, np.uint32)
        n = t.size
        preds = np.zeros(n, np.uint32)
        margins = np.zeros(n, np.float32)
        logits = np.zeros((n, self.V), np.float32) if want_logits else None
        lib().or_verify_greedy(self.h, t, n, start_pos, preds, margins.ctypes.data,
                               logits.ctypes.data if want_logits else None)
        return preds, margins, logits

    def generate_greedy(self, prompt, n_new, prefill_batch=16):
        p = _c(prompt, np.uint32)
        out = np.zeros(n_new, np.uint32)
        lib().or_generate_greedy(self.h, p, p.size, n_new, prefill_batch, out)
        return out

    def generate_speculative_oracle(self, prompt, n_new, k, alpha, seed, greedy, prefill_batch=16):
        p = _c(prompt, np.uint32)
        out = np.zeros(n_new, np.uint32)
        stats = np.zeros(2, np.int64)
        steps = np.zeros(1, np.int64)
        n = lib().or_generate_speculative_oracle(self.h, p, p.size, n_new, k, alpha, seed,
                                                 _c(greedy, np.uint32), prefill_batch, out, stats, steps)
        return out[:n], int(stats[0]), int(stats[1]), int(steps[0])

    def generate_speculative_ngram(self, prompt, n_new, k, min_ngram=3, max_ngram=4, stop=(), prefill_batch=16):
        p = _c(prompt, np.uint32)
        st = _c(np.asarray(stop, np.uint32).reshape(-1) if len(stop) else np.zeros(1, np.uint32), np.uint32)
        out = np.zeros(n_new, np.uint32)
        stats = np.zeros(2, np.int64)
        steps = np.zeros(1, np.int64)
        n = lib().or_generate_speculative_ngram(self.h, p, p.size, n_new, k, min_ngram, max_ngram, st, len(stop),
                                                prefill_batch, out, stats, steps)
        return out[:n], int(stats[0]), int(stats[1]), int(steps[0])

    def generate_speculative_ngram_temp(self, prompt, n_new, k, temp, rng_state=REFERENCE_RNG_STATE, min_ngram=3,
                                        max_ngram=4, stop=(), prefill_batch=16):
        """ngram_speculative_step at temperature (speculative.rs:122-286, main.rs:9729-9776);
        returns (tokens, drafted, accepted, steps, rng_state)."""
        p = _c(prompt, np.uint32)
        st = _c(np.asarray(stop, np.uint32).reshape(-1) if len(stop) else np.zeros(1, np.uint32), np.uint32)
        out = np.zeros(n_new, np.uint32)
        stats = np.zeros(2, np.int64)
        steps = np.zeros(1, np.int64)
        rs = C.c_uint64(rng_state)
        n = lib().or_generate_speculative_ngram_temp(self.h, p, p.size, n_new, k, min_ngram, max_ngram, float(temp),
                                                     C.byref(rs), st, len(stop), prefill_batch, out, stats, steps)
        return out[:n], int(stats[0]), int(stats[1]), int(steps[0]), int(rs.value)

    def close(self):
        if self.h:
            lib().or_session_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def generate_plain(s: Session, prompt, n_new, temp, rng_state=REFERENCE_RNG_STATE, stop=(), prefill_batch=16):
    """The plain decode loop (main.rs:9894-9928) at temperature temp with stop tokens; returns
    (tokens, rng_state)."""
    p = _c(prompt, np.uint32)
    sp = _c(np.array(list(stop) or [0], np.uint32), np.uint32)
    out = np.zeros(n_new, np.uint32)
    st = C.c_uint64(rng_state)
    n = lib().or_generate_plain(s.h, p, p.size, n_new, float(temp), C.byref(st), sp, len(stop), prefill_batch, out)
    return out[:n], int(st.value)


def generate_speculative_draft(target: Session, draft: Session, prompt, n_new, draft_k, prefill_batch=16):
    p = _c(prompt, np.uint32)
    out = np.zeros(n_new, np.uint32)
    stats = np.zeros(2, np.int64)
    steps = np.zeros(1, np.int64)
    n = lib().or_generate_speculative_draft(target.h, draft.h, p, p.size, n_new, draft_k, prefill_batch,
                                            out, stats, steps)
    return out[:n], int(stats[0]), int(stats[1]), int(steps[0])


def generate_speculative_draft_temp(target: Session, draft: Session, prompt, n_new, draft_k, temp,
                                    rng_state=REFERENCE_RNG_STATE, prefill_batch=16, stop=()):
    """speculative.rs:299-494 at temperature temp (greedy at temp <= 0) with the reference's
    sampler and LCG and its stop tokens; returns (tokens, drafted, accepted, steps, rng_state)."""
    p = _c(prompt, np.uint32)
    sp = _c(np.array(list(stop) or [0], np.uint32), np.uint32)
    out = np.zeros(n_new, np.uint32)
    stats = np.zeros(2, np.int64)
    steps = np.zeros(1, np.int64)
    st = C.c_uint64(rng_state)
    n = lib().or_generate_speculative_draft_temp(target.h, draft.h, p, p.size, n_new, draft_k, float(temp),
                                                 C.byref(st), sp, len(stop), prefill_batch, out, stats, steps)
    return out[:n], int(stats[0]), int(stats[1]), int(steps[0]), int(st.value)


def generate_speculative_stochastic(target: Session, draft: Session, prompt, n_new, k, temp, seed, prefill_batch=16):
    """Draft-model speculative sampling (k+1 form, Philox acceptance); returns
    (tokens, drafted, accepted, steps)."""
    p = _c(prompt, np.uint32)
    out = np.zeros(n_new, np.uint32)
    stats = np.zeros(2, np.int64)
    steps = np.zeros(1, np.int64)
    n = lib().or_generate_speculative_stochastic(target.h, draft.h, p, p.size, n_new, k, temp, seed, prefill_batch,
                                                 out, stats, steps)
    return out[:n], int(stats[0]), int(stats[1]), int(steps[0])
