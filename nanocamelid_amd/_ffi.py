"""ctypes binding of libnanocamelid_hip.so (include/nanocamelid_gpu.h).

The shared library is the product: HIP kernels for gfx950 plus a C++ host runtime.
This module only declares the C signatures.  It raises ImportError-style
RuntimeError when the library has not been built: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os

try:  # keep one HIP runtime per process: torch's libamdhip64 must be the one loaded first
    import torch  # noqa: F401
except Exception:  # pragma: no cover - torch is always present in this image
    torch = None

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libnanocamelid_hip.so")

NC_OK, NC_EINVAL, NC_ENOMEM, NC_EHIP, NC_EFORMAT, NC_ERANGE = 0, -1, -2, -3, -4, -5
NC_TYPE_F32, NC_TYPE_Q4_0, NC_TYPE_Q8_0, NC_TYPE_Q4_K, NC_TYPE_Q5_K, NC_TYPE_Q6_K = 0, 2, 8, 12, 13, 14
NC_GEMM_KERNEL_AUTO, NC_GEMM_KERNEL_DOT4, NC_GEMM_KERNEL_MFMA = 0, 1, 2
NC_ATTN_SEQUENTIAL, NC_ATTN_SPLIT = 0, 1
NC_PASS_DIRECT, NC_PASS_GRAPH = 0, 1


class ModelConfig(C.Structure):
    _fields_ = [(n, C.c_int64) for n in (
        "context_length", "embedding_length", "block_count", "feed_forward_length", "head_count",
        "head_count_kv", "head_dim", "rope_dimension_count", "vocab_size", "attention_output_width",
        "kv_width")] + [("weight_type", C.c_int32), ("tied_head", C.c_int32),
                        ("rope_freq_base", C.c_float), ("rms_norm_epsilon", C.c_float),
                        ("device_weight_bytes", C.c_int64), ("verify_weight_bytes", C.c_int64),
                        ("rope_scaling", C.c_int32), ("rope_scaling_factor", C.c_float),
                        ("rope_scaling_original_context_length", C.c_float),
                        ("rope_scaling_low_freq_factor", C.c_float), ("rope_scaling_high_freq_factor", C.c_float)]


class LoadOpts(C.Structure):
    _fields_ = [("nthreads", C.c_int32), ("reserved", C.c_int32 * 7)]


class VerifyResult(C.Structure):
    _fields_ = [("n_accepted", C.c_int32), ("next_token", C.c_uint32), ("new_pos", C.c_int64)]


class DecodeStats(C.Structure):
    _fields_ = [("steps", C.c_int64), ("drafted", C.c_int64), ("accepted", C.c_int64), ("emitted", C.c_int64),
                ("decode_seconds", C.c_double), ("prefill_seconds", C.c_double)]


class SynthSpec(C.Structure):
    _fields_ = [("layers", C.c_int32), ("embedding_length", C.c_int32), ("head_count", C.c_int32),
                ("head_count_kv", C.c_int32), ("feed_forward_length", C.c_int32), ("vocab_size", C.c_int32),
                ("context_length", C.c_int32), ("weight_type", C.c_int32), ("tied", C.c_int32),
                ("norm_mode", C.c_int32), ("rope_freq_base", C.c_float), ("rms_norm_epsilon", C.c_float),
                ("weight_std", C.c_float), ("seed", C.c_uint64), ("rope_scaling_factor", C.c_float),
                ("rope_scaling_low_freq_factor", C.c_float), ("rope_scaling_high_freq_factor", C.c_float),
                ("rope_scaling_original_context_length", C.c_uint32)]


_vp, _i32, _i64, _u32p, _f32p = C.c_void_p, C.c_int32, C.c_int64, C.POINTER(C.c_uint32), C.POINTER(C.c_float)

# name: (restype, argtypes)
SIGNATURES = {
    "nc_last_error": (C.c_char_p, []),
    "nc_version": (C.c_char_p, []),
    "nc_ctx_create": (C.c_int, [C.c_int, C.POINTER(_vp)]),
    "nc_ctx_free": (None, [_vp]),
    "nc_ctx_synchronize": (C.c_int, [_vp]),
    "nc_ctx_set_gemm_kernel": (C.c_int, [_vp, C.c_int]),
    "nc_ctx_set_attention": (C.c_int, [_vp, C.c_int]),
    "nc_ctx_set_pass_launch": (C.c_int, [_vp, C.c_int]),
    "nc_qmat_upload": (C.c_int, [_vp, C.c_int, _i64, _i64, _vp, C.POINTER(_vp)]),
    "nc_qmat_free": (None, [_vp]),
    "nc_qmat_device_bytes": (_i64, [_vp]),
    "nc_matmul_quantized_batch": (C.c_int, [_vp, _vp, _vp, _vp, _vp, C.c_int, _i64, _i64, _vp]),
    "nc_matmul_quantized_batch_noalloc": (C.c_int, [_vp, _vp, _vp, _vp, _vp, C.c_int, _i64, _i64, _vp]),
    "nc_matmul_blockdots": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int, _i64, _i64, _vp]),
    "nc_debug_expf": (C.c_int, [_vp, C.c_uint32, _i64, _vp, _vp]),
    "nc_debug_temperature_paths": (C.c_int, [_vp, C.c_int32, _vp, _vp]),
    "nc_debug_pass_graphs": (C.c_int, [_vp, _vp, _vp]),
    "nc_quantize_q8_0_batch": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int, _i64, _vp]),
    "nc_rms_norm_q8_0_batch": (C.c_int, [_vp, _vp, _vp, C.c_float, _vp, _vp, C.c_int, _i64, _vp]),
    "nc_bench_matmul": (C.c_int, [_vp, _vp, _i32, _vp, _vp, _vp, _i32, _i32, _vp]),
    "nc_temperature_probs_batch": (C.c_int, [_vp, _vp, _vp, _i32, _i64, C.c_float, _vp]),
    "nc_sample_logits_batch": (C.c_int, [_vp, _vp, _i32, _i64, C.c_float, C.POINTER(C.c_uint64), _vp, _u32p, _vp]),
    "nc_stochastic_accept": (C.c_int, [_vp, _vp, _vp, _vp, _i32, _i64, C.c_uint64, _i64, _vp, _vp]),
    "nc_model_load_gguf": (C.c_int, [_vp, C.c_char_p, C.POINTER(LoadOpts), C.POINTER(_vp)]),
    "nc_model_load_gguf_memory": (C.c_int, [_vp, _vp, C.c_size_t, C.POINTER(LoadOpts), C.POINTER(_vp)]),
    "nc_model_get_config": (C.c_int, [_vp, C.POINTER(ModelConfig)]),
    "nc_dequantize_f32": (C.c_int, [C.c_int32, _vp, _i64, _vp]),
    "nc_gguf_read_config": (C.c_int, [_vp, C.c_size_t, C.POINTER(ModelConfig)]),
    "nc_gguf_stop_tokens": (C.c_int, [_vp, C.c_size_t, _u32p, _i32, C.POINTER(C.c_int32)]),
    "nc_gguf_tensor_count": (_i64, [_vp, C.c_size_t]),
    "nc_gguf_tensor_info": (C.c_int, [_vp, C.c_size_t, _i64, C.c_char_p, _i64, C.POINTER(C.c_int32),
                                      C.POINTER(C.c_uint64), C.POINTER(C.c_int32), C.POINTER(C.c_uint64),
                                      C.POINTER(C.c_uint64)]),
    "nc_model_free": (None, [_vp]),
    "nc_session_create": (C.c_int, [_vp, _i64, _i32, C.POINTER(_vp)]),
    "nc_session_free": (None, [_vp]),
    "nc_prefill": (C.c_int, [_vp, _u32p, _i32, _i64, _i32]),
    "nc_forward1": (C.c_int, [_vp, C.c_uint32, _i64, _f32p, _u32p]),
    "nc_verify_greedy": (C.c_int, [_vp, _u32p, _i32, _i64, C.POINTER(VerifyResult), _u32p]),
    "nc_verify_stochastic": (C.c_int, [_vp, _u32p, _i32, _i64, _vp, C.c_float, C.c_uint64, C.POINTER(VerifyResult)]),
    "nc_session_logits": (C.c_int, [_vp, _i32, _f32p]),
    "nc_session_hidden": (C.c_int, [_vp, _i32, _f32p]),
    "nc_generate_greedy": (C.c_int, [_vp, _u32p, _i32, _i32, _u32p, C.POINTER(DecodeStats)]),
    "nc_generate_plain": (C.c_int, [_vp, _u32p, _i32, _i32, C.c_float, C.POINTER(C.c_uint64), _u32p, _i32, _u32p,
                                    C.POINTER(DecodeStats)]),
    "nc_generate_speculative_oracle": (C.c_int, [_vp, _u32p, _i32, _i32, _i32, _i32, C.c_float, C.c_uint64, _u32p,
                                                 _i32, _u32p, C.POINTER(DecodeStats)]),
    "nc_generate_speculative_draft": (C.c_int, [_vp, _vp, _u32p, _i32, _i32, _i32, _u32p, C.POINTER(DecodeStats)]),
    "nc_generate_speculative_draft_temp": (C.c_int, [_vp, _vp, _u32p, _i32, _i32, _i32, C.c_float,
                                                     C.POINTER(C.c_uint64), _u32p, _i32, _u32p,
                                                     C.POINTER(DecodeStats)]),
    "nc_generate_speculative_stochastic": (C.c_int, [_vp, _vp, _u32p, _i32, _i32, _i32, C.c_float, C.c_uint64, _u32p,
                                                     C.POINTER(DecodeStats)]),
    "nc_synth_size": (C.c_int, [C.POINTER(SynthSpec), C.POINTER(C.c_uint64)]),
    "nc_synth_write": (C.c_int, [C.POINTER(SynthSpec), _vp, C.c_uint64, _i32]),
    "nc_uniform_prompt": (C.c_int, [C.c_uint64, _i64, C.c_uint32, _u32p]),
    "nc_oracle_draft": (C.c_uint32, [C.c_uint64, _i64, C.c_float, _u32p, _i64, _i64, C.c_uint32]),
    "nc_ngram_draft": (C.c_int32, [_u32p, _i64, _i32, _i32, _i32, _u32p]),
    "nc_generate_speculative_ngram": (C.c_int, [_vp, _u32p, _i32, _i32, _i32, _i32, _i32, _u32p, _i32, _u32p, _vp]),
    "nc_generate_speculative_ngram_temp": (C.c_int, [_vp, _u32p, _i32, _i32, _i32, _i32, _i32, C.c_float,
                                                     C.POINTER(C.c_uint64), _u32p, _i32, _u32p, _vp]),
    "nc_synth_kv_values": (C.c_int, [C.c_uint64, _i32, _i32, _i64, _i64, _f32p]),
    "nc_session_fill_kv": (C.c_int, [_vp, _i64, C.c_uint64]),
    "nc_session_kernel_timing": (_i64, [_vp, C.c_char_p, C.POINTER(C.c_double), C.POINTER(C.c_int64)]),
    "nc_session_timing_enable": (C.c_int, [_vp, _i32]),
    "nc_session_stage_timing": (C.c_int32, [_vp, _i32, C.c_char_p, _i32, C.POINTER(C.c_double),
                                            C.POINTER(C.c_int64)]),
}

_lib = None


def lib():
    """Loads the native library (built by __graft_entry__.build()); raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"libnanocamelid_hip.so not found at {LIB_PATH}: build it first (python -c "
            "'import __graft_entry__ as g; g.build()'). There is no CPU fallback.")
    L = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


class NcError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"nanocamelid error {code}: {msg}")
        self.code = code


def check(rc):
    if rc != NC_OK:
        raise NcError(rc, lib().nc_last_error().decode(errors="replace"))
    return rc
