"""nanocamelid_amd: MI355X-native speculative-decoding verify path.

Python mirror of the reference's operator and step interface over the C ABI of
libnanocamelid_hip.so.  Names follow the reference:

* ``matmul_quantized_batch``   -- src/inference.rs:1246 (device tensors in, device tensor out)
* ``quantize_f32_to_q8_0_batch`` -- src/inference.rs:967
* ``Model`` / ``Session``       -- LlamaWeights::load (src/model.rs:461) + LlamaKvCache /
  workspaces (src/inference.rs:505-695)
* ``Session.prefill_pass_batch`` -- src/inference.rs:3695
* ``Session.forward_pass``       -- src/inference.rs:3649
* ``Session.verify_greedy``      -- the k+1 verify of src/speculative.rs:122-286
* ``generate_speculative_draft`` -- speculative_decoding_step, src/speculative.rs:299-494

Everything runs in the native library on the GPU; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._ffi import (NC_TYPE_Q4_0, NC_TYPE_Q4_K, NC_TYPE_Q5_K, NC_TYPE_Q6_K, NC_TYPE_Q8_0, DecodeStats, LoadOpts, ModelConfig, NcError, SynthSpec,
                   VerifyResult, check, lib)

__all__ = ["Context", "QMat", "Model", "Session", "matmul_quantized_batch", "matmul_blockdots",
           "quantize_f32_to_q8_0_batch", "synth_gguf", "uniform_prompt", "oracle_draft",
           "generate_speculative_draft", "NcError", "NC_TYPE_Q4_0", "NC_TYPE_Q4_K", "NC_TYPE_Q5_K", "NC_TYPE_Q8_0",
           "SYNTH_CONFIGS"]


def _u32(a):
    a = np.ascontiguousarray(a, dtype=np.uint32)
    return a, a.ctypes.data_as(C.POINTER(C.c_uint32))


def _stream_of(t):
    import torch
    return C.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


class Context:
    """Device context (nc_ctx)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        check(lib().nc_ctx_create(device, C.byref(h)))
        self.h = h
        self.device = device

    def synchronize(self):
        check(lib().nc_ctx_synchronize(self.h))

    def set_gemm_kernel(self, kernel: int):
        """Dot-product path of the quantized matmuls (NC_GEMM_KERNEL_AUTO / _DOT4 / _MFMA), the
        counterpart of the reference's Q8DotKernelSelector (src/q8.rs:42-46)."""
        check(lib().nc_ctx_set_gemm_kernel(self.h, int(kernel)))

    def set_attention(self, order: int):
        """Summation order of the verify and decode passes' attention: NC_ATTN_SEQUENTIAL (the
        reference's left-to-right sums, bit-identical) or NC_ATTN_SPLIT (64-position chunks
        combined in a fixed order; equal up to f32 rounding, batch-independent)."""
        check(lib().nc_ctx_set_attention(self.h, int(order)))

    def set_pass_launch(self, mode: int):
        """How sessions launch verify and decode passes: NC_PASS_DIRECT (kernel by kernel, the
        default) or NC_PASS_GRAPH (captured HIP graphs, replayed); results are identical."""
        check(lib().nc_ctx_set_pass_launch(self.h, int(mode)))

    def close(self):
        if getattr(self, "h", None):
            lib().nc_ctx_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class QMat:
    """Device-resident repacked Q4_0 / Q4_K / Q5_K / Q8_0 / Q6_K matrix (QuantizedMatrix, src/model.rs:294-310)."""

    def __init__(self, ctx: Context, qtype: int, rows: int, cols: int, gguf_blocks: np.ndarray):
        blocks = np.ascontiguousarray(gguf_blocks, dtype=np.uint8)
        h = C.c_void_p()
        check(lib().nc_qmat_upload(ctx.h, qtype, rows, cols, blocks.ctypes.data, C.byref(h)))
        self.h, self.ctx, self.rows, self.cols, self.qtype = h, ctx, rows, cols, qtype

    @property
    def device_bytes(self) -> int:
        return int(lib().nc_qmat_device_bytes(self.h))

    def close(self):
        if getattr(self, "h", None):
            lib().nc_qmat_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def matmul_quantized_batch(ctx: Context, w: QMat, x_i8, x_scales, out=None):
    """out[t][r] = sum_b (w_scale*x_scale)*dot in block order (src/inference.rs:1246).

    x_i8: torch int8 [batch, cols] on the GPU; x_scales: torch float32 [batch, cols/32]."""
    import torch
    n = x_i8.shape[0]
    if out is None:
        out = torch.empty((n, w.rows), dtype=torch.float32, device=x_i8.device)
    check(lib().nc_matmul_quantized_batch(ctx.h, w.h, x_i8.data_ptr(), x_scales.data_ptr(), out.data_ptr(), n,
                                          w.rows, w.cols, _stream_of(x_i8)))
    return out


def dequantize_f32(ggml_type: int, data: np.ndarray, n: int) -> np.ndarray:
    """Host decode of one GGUF tensor's bytes to f32 as the loader does for token embeddings and
    norms (load_f32_or_f16, src/model.rs:1081-1229).  Needs no GPU."""
    src = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.zeros(n, np.float32)
    check(lib().nc_dequantize_f32(int(ggml_type), src.ctypes.data, n, out.ctypes.data))
    return out


def gguf_read_config(data) -> dict:
    """Header-only GGUF checks (read_file + LlamaModelConfig::from_gguf + validate_model_tensors,
    src/gguf.rs:454-551, src/model.rs:48-186, :851-1036) on an in-memory image; no GPU.  Raises
    NcError with the reference-style message when the file is refused."""
    buf = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray)) else data,
                               dtype=np.uint8)
    cfg = ModelConfig()
    check(lib().nc_gguf_read_config(buf.ctypes.data, buf.size, C.byref(cfg)))
    return {f: getattr(cfg, f) for f, _ in ModelConfig._fields_}


def gguf_stop_tokens(data) -> np.ndarray:
    """The ids that end a turn (SpecialTokens::eog of the file's tokenizer, src/tokenizer.rs:287-323,
    tested by is_generation_stop_token, src/main.rs:8518-8520), from an image or a path (mapped,
    not read); no GPU."""
    if isinstance(data, str):
        data = np.memmap(data, dtype=np.uint8, mode="r")
    buf = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray)) else data,
                               dtype=np.uint8)
    out = np.zeros(16, np.uint32)
    n = C.c_int32()
    check(lib().nc_gguf_stop_tokens(buf.ctypes.data, buf.size, out.ctypes.data_as(C.POINTER(C.c_uint32)), 16,
                                    C.byref(n)))
    return out[:n.value]


def gguf_tensors(data) -> list:
    """gguf::read_file tensor descriptors: (name, dims, type, absolute offset, n_bytes)."""
    buf = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray)) else data,
                               dtype=np.uint8)
    n = lib().nc_gguf_tensor_count(buf.ctypes.data, buf.size)
    check(int(n) if n < 0 else 0)
    out = []
    for i in range(n):
        name = C.create_string_buffer(512)
        nd, ty = C.c_int32(), C.c_int32()
        dims = (C.c_uint64 * 4)()
        off, nb = C.c_uint64(), C.c_uint64()
        check(lib().nc_gguf_tensor_info(buf.ctypes.data, buf.size, i, name, 512, C.byref(nd), dims, C.byref(ty),
                                        C.byref(off), C.byref(nb)))
        out.append((name.value.decode(), [int(dims[k]) for k in range(nd.value)], ty.value, off.value, nb.value))
    return out


def matmul_blockdots(ctx: Context, w: QMat, x_i8):
    """int32 per-block dot products [batch, rows, cols/32] (q8.rs:2699 per block)."""
    import torch
    n = x_i8.shape[0]
    dots = torch.empty((n, w.rows, w.cols // 32), dtype=torch.int32, device=x_i8.device)
    check(lib().nc_matmul_blockdots(ctx.h, w.h, x_i8.data_ptr(), dots.data_ptr(), n, w.rows, w.cols,
                                    _stream_of(x_i8)))
    return dots


def quantize_f32_to_q8_0_batch(ctx: Context, x):
    """Q8_0 activation quantisation on the GPU (src/inference.rs:967-1029)."""
    import torch
    n, dim = x.shape
    q = torch.empty((n, dim), dtype=torch.int8, device=x.device)
    s = torch.empty((n, dim // 32), dtype=torch.float32, device=x.device)
    check(lib().nc_quantize_q8_0_batch(ctx.h, x.data_ptr(), q.data_ptr(), s.data_ptr(), n, dim, _stream_of(x)))
    return q, s


def rms_norm_q8_0_batch(ctx: Context, x, w, eps: float):
    """RMSNorm (sequential f32 sum of squares, bit-identical) then Q8_0 quantisation on the
    GPU (src/inference.rs:949-967 and :967-1029, as run at :3802-3808)."""
    import torch
    n, dim = x.shape
    q = torch.empty((n, dim), dtype=torch.int8, device=x.device)
    s = torch.empty((n, dim // 32), dtype=torch.float32, device=x.device)
    check(lib().nc_rms_norm_q8_0_batch(ctx.h, x.data_ptr(), w.data_ptr(), float(eps), q.data_ptr(), s.data_ptr(), n,
                                       dim, _stream_of(x)))
    return q, s


def temperature_probs_batch(ctx: Context, logits, temp: float, out=None):
    """Temperature softmax of each row on the GPU: p = expf((l - max)/temp) * (1/sum), the sum
    left to right in f32 (the reference's softmax formula, src/inference.rs:3522-3540,
    4857-4862).  logits: [rows][vocab] f32 device tensor."""
    import torch
    rows, vocab = logits.shape
    out = torch.empty_like(logits) if out is None else out
    check(lib().nc_temperature_probs_batch(ctx.h, logits.data_ptr(), out.data_ptr(), rows, vocab, float(temp),
                                           _stream_of(logits)))
    return out


def temperature_paths(ctx: Context, rows: int, stream=None):
    """Debug: for each of the last temperature pass's rows on this context, 1 if its exact sum
    came from the parallel-segment evaluation, 0 if from the segment-after-segment one."""
    import numpy as np
    out = np.zeros(rows, np.int32)
    check(lib().nc_debug_temperature_paths(ctx.h, rows, out.ctypes.data, stream))
    return out


# The reference's initial rand_simple state (src/inference.rs:4875).
REFERENCE_RNG_STATE = 0x123456789ABCDEF0


def sample_logits_batch(ctx: Context, logits, temp: float, rng_state: int = REFERENCE_RNG_STATE):
    """sample_logits (src/inference.rs:4834-4873) of each row on the GPU: temp <= 0 the first
    maximum; temp > 0 the reference's draw (r = rand_simple() * sum e, r -= e_j until r <= 0),
    one LCG draw per row in row order.  logits: [rows][vocab] f32 device tensor (rows <= 16).
    Returns (ids, rng_state after the draws)."""
    import torch
    rows, vocab = logits.shape
    work = torch.empty_like(logits) if temp > 0 else None
    st = C.c_uint64(rng_state)
    ids = np.zeros(rows, np.uint32)
    check(lib().nc_sample_logits_batch(ctx.h, logits.data_ptr(), rows, vocab, float(temp), C.byref(st),
                                       work.data_ptr() if work is not None else None,
                                       ids.ctypes.data_as(C.POINTER(C.c_uint32)), _stream_of(logits)))
    return ids, int(st.value)


def stochastic_accept(ctx: Context, p_probs, q_probs, drafts, seed: int, start_pos: int):
    """k+1 stochastic acceptance on the GPU (no reference counterpart; the library's Philox /
    min(1, p/q) / fixed-point resampling specification).  p_probs [k+1][V], q_probs [k][V]
    f32 and drafts [k] int32/uint32 device tensors.  Returns (n_accepted, next_token, new_pos)."""
    import torch
    k = p_probs.shape[0] - 1
    res = torch.zeros(4, dtype=torch.int32, device=p_probs.device)
    check(lib().nc_stochastic_accept(ctx.h, p_probs.data_ptr(), q_probs.data_ptr() if k else None,
                                     drafts.data_ptr() if k else None, k, p_probs.shape[1], seed, start_pos,
                                     res.data_ptr(), _stream_of(p_probs)))
    r = res.cpu().tolist()
    return r[0], r[1], r[2]


class Model:
    """Llama weights on the device (LlamaWeights::load, src/model.rs:461-545)."""

    def __init__(self, ctx: Context, path: str | None = None, data: np.ndarray | None = None, nthreads: int = 0):
        opts = LoadOpts()
        opts.nthreads = nthreads
        h = C.c_void_p()
        if data is not None:
            buf = np.ascontiguousarray(data, dtype=np.uint8)
            check(lib().nc_model_load_gguf_memory(ctx.h, buf.ctypes.data, buf.size, C.byref(opts), C.byref(h)))
        else:
            check(lib().nc_model_load_gguf(ctx.h, path.encode(), C.byref(opts), C.byref(h)))
        self.h, self.ctx = h, ctx
        cfg = ModelConfig()
        check(lib().nc_model_get_config(h, C.byref(cfg)))
        self.config = {f: getattr(cfg, f) for f, _ in ModelConfig._fields_}

    def close(self):
        if getattr(self, "h", None):
            lib().nc_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Session:
    """One sequence: KV cache, workspaces, stream (LlamaKvCache + workspaces)."""

    def __init__(self, model: Model, max_ctx: int, max_batch: int = 16):
        h = C.c_void_p()
        check(lib().nc_session_create(model.h, max_ctx, max_batch, C.byref(h)))
        self.h, self.model = h, model
        self.vocab = model.config["vocab_size"]
        self.d = model.config["embedding_length"]

    def prefill_pass_batch(self, toks, start_pos: int, want_logits: bool = True):
        """prefill_pass_batch (src/inference.rs:3695-3744) in max_batch chunks; want_logits: also
        run the head on the last chunk's rows (readable with logits(row))."""
        a, p = _u32(toks)
        check(lib().nc_prefill(self.h, p, a.size, start_pos, 1 if want_logits else 0))

    def forward_pass(self, tok: int, pos: int, want_logits: bool = True):
        pred = C.c_uint32()
        logits = np.empty(self.vocab, np.float32) if want_logits else None
        lp = logits.ctypes.data_as(C.POINTER(C.c_float)) if want_logits else None
        check(lib().nc_forward1(self.h, int(tok), pos, lp, C.byref(pred)))
        return pred.value, logits

    def verify_greedy(self, toks, start_pos: int):
        a, p = _u32(toks)
        preds = np.zeros(a.size, np.uint32)
        r = VerifyResult()
        check(lib().nc_verify_greedy(self.h, p, a.size, start_pos, C.byref(r),
                                     preds.ctypes.data_as(C.POINTER(C.c_uint32))))
        return r.n_accepted, r.next_token, r.new_pos, preds

    def verify_stochastic(self, toks, start_pos: int, q_probs, temp: float, seed: int):
        """toks = [pending] + drafts; q_probs: [len(drafts)][vocab] f32 device tensor."""
        a, p = _u32(toks)
        r = VerifyResult()
        check(lib().nc_verify_stochastic(self.h, p, a.size, start_pos, q_probs.data_ptr() if a.size > 1 else None,
                                         float(temp), seed, C.byref(r)))
        return r.n_accepted, r.next_token, r.new_pos

    def fill_kv(self, n: int, seed: int):
        """Benchmark/test helper: N(0, 1) keys and values in KV rows [0, n) of every layer
        (synth_kv_values streams), so a pass at start_pos = n attends over n such positions."""
        check(lib().nc_session_fill_kv(self.h, n, seed))

    def pass_graphs(self):
        """Debug: (passes captured into HIP graphs, passes replayed from them) of this session."""
        cap, rep = C.c_int64(0), C.c_int64(0)
        check(lib().nc_debug_pass_graphs(self.h, C.byref(cap), C.byref(rep)))
        return cap.value, rep.value

    def logits(self, row: int) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        check(lib().nc_session_logits(self.h, row, out.ctypes.data_as(C.POINTER(C.c_float))))
        return out

    def hidden(self, n: int) -> np.ndarray:
        out = np.empty((n, self.d), np.float32)
        check(lib().nc_session_hidden(self.h, n, out.ctypes.data_as(C.POINTER(C.c_float))))
        return out

    def generate_greedy(self, prompt, n_new: int):
        a, p = _u32(prompt)
        out = np.zeros(n_new, np.uint32)
        st = DecodeStats()
        check(lib().nc_generate_greedy(self.h, p, a.size, n_new, out.ctypes.data_as(C.POINTER(C.c_uint32)),
                                       C.byref(st)))
        return out, st

    def generate_plain(self, prompt, n_new: int, temp: float, rng_state: int = REFERENCE_RNG_STATE, stop=()):
        """The plain decode loop (src/main.rs:9894-9928) with sample_logits, the reference's LCG and
        stop tokens; returns (tokens, stats, rng_state after the run)."""
        a, p = _u32(prompt)
        sa, sp = _u32(np.array(list(stop) or [0], np.uint32))
        out = np.zeros(n_new, np.uint32)
        st = DecodeStats()
        rs = C.c_uint64(rng_state)
        check(lib().nc_generate_plain(self.h, p, a.size, n_new, float(temp), C.byref(rs), sp, len(stop),
                                      out.ctypes.data_as(C.POINTER(C.c_uint32)), C.byref(st)))
        return out[:st.emitted], st, int(rs.value)

    def generate_speculative_oracle(self, prompt, n_new: int, k: int, alpha: float, seed: int, greedy,
                                    max_steps: int = 0):
        a, p = _u32(prompt)
        g, gp = _u32(greedy)
        out = np.zeros(n_new, np.uint32)
        st = DecodeStats()
        check(lib().nc_generate_speculative_oracle(self.h, p, a.size, n_new, max_steps, k, alpha, seed, gp, g.size,
                                                   out.ctypes.data_as(C.POINTER(C.c_uint32)), C.byref(st)))
        return out[:st.emitted], st

    def generate_speculative_ngram(self, prompt, n_new: int, k: int, min_ngram: int = 3, max_ngram: int = 4,
                                   stop=()):
        """ngram_speculative_step (speculative.rs:122-286), greedy, k+1 verify form; returns
        (tokens, stats).  The stream ends before the first stop token."""
        a, p = _u32(prompt)
        so, sp = _u32(np.asarray(stop, np.uint32).reshape(-1) if len(stop) else np.zeros(1, np.uint32))
        out = np.zeros(n_new, np.uint32)
        st = DecodeStats()
        check(lib().nc_generate_speculative_ngram(self.h, p, a.size, n_new, k, min_ngram, max_ngram, sp, len(stop),
                                                  out.ctypes.data_as(C.POINTER(C.c_uint32)), C.byref(st)))
        return out[:st.emitted], st

    def generate_speculative_ngram_temp(self, prompt, n_new: int, k: int, temp: float,
                                        rng_state: int = REFERENCE_RNG_STATE, min_ngram: int = 3, max_ngram: int = 4,
                                        stop=()):
        """ngram_speculative_step at temperature (speculative.rs:122-286, main.rs:9729-9776) with
        sample_logits and the reference's LCG; returns (tokens, stats, rng_state)."""
        a, p = _u32(prompt)
        so, sp = _u32(np.asarray(stop, np.uint32).reshape(-1) if len(stop) else np.zeros(1, np.uint32))
        out = np.zeros(n_new, np.uint32)
        st = DecodeStats()
        rs = C.c_uint64(rng_state)
        check(lib().nc_generate_speculative_ngram_temp(self.h, p, a.size, n_new, k, min_ngram, max_ngram, float(temp),
                                                       C.byref(rs), sp, len(stop),
                                                       out.ctypes.data_as(C.POINTER(C.c_uint32)), C.byref(st)))
        return out[:st.emitted], st, int(rs.value)

    def timing(self, enable: bool):
        check(lib().nc_session_timing_enable(self.h, 1 if enable else 0))

    def stage_timing(self, enable: bool):
        """Per-stage timing of verify and decode passes (the reference's trace stages)."""
        check(lib().nc_session_timing_enable(self.h, 2 if enable else 0))

    def stages(self) -> dict:
        """{stage name: (total ms, passes)} since stage_timing(True)."""
        n = lib().nc_session_stage_timing(self.h, -1, None, 0, None, None)
        if n < 0:
            check(n)
        out = {}
        for i in range(n):
            name = C.create_string_buffer(96)
            ms, calls = C.c_double(), C.c_int64()
            check(min(0, lib().nc_session_stage_timing(self.h, i, name, 96, C.byref(ms), C.byref(calls))))
            out[name.value.decode()] = (ms.value, int(calls.value))
        return out

    def gemm_timing(self):
        ms = C.c_double()
        by = C.c_int64()
        n = lib().nc_session_kernel_timing(self.h, b"gemm_q4_0", C.byref(ms), C.byref(by))
        return int(n), ms.value, int(by.value)

    def close(self):
        if getattr(self, "h", None):
            lib().nc_session_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def generate_speculative_draft(target: Session, draft: Session, prompt, n_new: int, draft_k: int):
    a, p = _u32(prompt)
    out = np.zeros(n_new, np.uint32)
    st = DecodeStats()
    check(lib().nc_generate_speculative_draft(target.h, draft.h, p, a.size, n_new, draft_k,
                                              out.ctypes.data_as(C.POINTER(C.c_uint32)), C.byref(st)))
    return out[:st.emitted], st


def generate_speculative_draft_temp(target: Session, draft: Session, prompt, n_new: int, draft_k: int, temp: float,
                                    rng_state: int = REFERENCE_RNG_STATE, stop=()):
    """speculative_decoding_step at temperature temp (src/speculative.rs:299-494; greedy at
    temp <= 0): drafts and target tokens drawn with sample_logits and the reference's LCG,
    acceptance by id match, stop tokens as the step and the generate loop treat them.
    Returns (tokens, stats, rng_state after the run)."""
    a, p = _u32(prompt)
    sa, sp = _u32(np.array(list(stop) or [0], np.uint32))
    out = np.zeros(n_new, np.uint32)
    st = DecodeStats()
    rs = C.c_uint64(rng_state)
    check(lib().nc_generate_speculative_draft_temp(target.h, draft.h, p, a.size, n_new, draft_k, float(temp),
                                                   C.byref(rs), sp, len(stop),
                                                   out.ctypes.data_as(C.POINTER(C.c_uint32)), C.byref(st)))
    return out[:st.emitted], st, int(rs.value)


def generate_speculative_stochastic(target: Session, draft: Session, prompt, n_new: int, k: int, temp: float,
                                    seed: int):
    """Draft-model speculative sampling at temperature temp (Philox acceptance), k+1 form."""
    a, p = _u32(prompt)
    out = np.zeros(n_new, np.uint32)
    st = DecodeStats()
    check(lib().nc_generate_speculative_stochastic(target.h, draft.h, p, a.size, n_new, k, float(temp), seed,
                                                   out.ctypes.data_as(C.POINTER(C.c_uint32)), C.byref(st)))
    return out[:st.emitted], st


# Model shapes of the benchmark configurations.
SYNTH_CONFIGS = {
    "llama-3.2-1b": dict(layers=16, embedding_length=2048, head_count=32, head_count_kv=8, feed_forward_length=8192,
                         vocab_size=128256, tied=1, weight_type=NC_TYPE_Q4_0),
    "llama-3-8b": dict(layers=32, embedding_length=4096, head_count=32, head_count_kv=8, feed_forward_length=14336,
                       vocab_size=128256, tied=0, weight_type=NC_TYPE_Q4_0),
    "llama-3.2-3b-q4k": dict(layers=28, embedding_length=3072, head_count=24, head_count_kv=8,
                             feed_forward_length=8192, vocab_size=128256, tied=1, weight_type=NC_TYPE_Q4_K),
    "llama-3-70b": dict(layers=80, embedding_length=8192, head_count=64, head_count_kv=8, feed_forward_length=28672,
                        vocab_size=128256, tied=0, weight_type=NC_TYPE_Q4_0),
}


def synth_gguf(layers, embedding_length, head_count, head_count_kv, feed_forward_length, vocab_size,
               context_length=8192, weight_type=NC_TYPE_Q4_0, tied=1, norm_mode=0, rope_freq_base=500000.0,
               rms_norm_epsilon=1e-5, weight_std=0.02, seed=0, nthreads=0, rope_scaling=None) -> np.ndarray:
    """Seeded random-init Llama GGUF v3 image (weights N(0, std) -> Q4_0 / Q4_K).

    rope_scaling: optional (factor, original_context_length, low_freq_factor, high_freq_factor),
    written as the llama.rope.scaling.* keys (Llama-3.1/3.2 files carry (32, 8192, 1, 4))."""
    fac, orig, lo, hi = rope_scaling if rope_scaling else (0.0, 0, 0.0, 0.0)
    s = SynthSpec(layers, embedding_length, head_count, head_count_kv, feed_forward_length, vocab_size,
                  context_length, weight_type, tied, norm_mode, rope_freq_base, rms_norm_epsilon, weight_std, seed,
                  fac, lo, hi, int(orig))
    size = C.c_uint64()
    check(lib().nc_synth_size(C.byref(s), C.byref(size)))
    buf = np.empty(size.value, np.uint8)
    check(lib().nc_synth_write(C.byref(s), buf.ctypes.data, size.value, nthreads))
    return buf


def synth_kv_values(seed: int, layer: int, kind: int, start: int, count: int) -> np.ndarray:
    """Host-only: elements [start, start + count) of the N(0, 1) stream of layer `layer`'s keys
    (kind 0) or values (kind 1) that Session.fill_kv writes (element p * kv_width + i = row p, i)."""
    out = np.empty(count, np.float32)
    check(lib().nc_synth_kv_values(seed, layer, kind, start, count, out.ctypes.data_as(C.POINTER(C.c_float))))
    return out


def uniform_prompt(seed: int, n: int, vocab: int) -> np.ndarray:
    out = np.zeros(n, np.uint32)
    check(lib().nc_uniform_prompt(seed, n, vocab, out.ctypes.data_as(C.POINTER(C.c_uint32))))
    return out


def ngram_draft(history, max_tokens: int, min_ngram: int = 3, max_ngram: int = 4):
    """NGramDrafter::draft (speculative.rs:81-103); defaults as NGramDrafter::default."""
    h, hp = _u32(history if len(history) else np.zeros(1, np.uint32))
    out = np.zeros(max(int(max_tokens), 1), np.uint32)
    n = lib().nc_ngram_draft(hp, len(history), min_ngram, max_ngram, max_tokens,
                             out.ctypes.data_as(C.POINTER(C.c_uint32)))
    return out[:n]


def oracle_draft(seed: int, p: int, alpha: float, greedy, n_prompt: int, vocab: int) -> int:
    g, gp = _u32(greedy)
    return int(lib().nc_oracle_draft(seed, p, alpha, gp, n_prompt, g.size, vocab))
