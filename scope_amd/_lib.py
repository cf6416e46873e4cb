"""ctypes binding of ``libscope_amd.so`` (the C ABI declared in
``include/scope_amd.h``).

The library is loaded lazily on first use.  There is no fallback: if the
shared library is missing or does not load, every operation raises.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("SCOPE_AMD_LIB", os.path.join(HERE, "libscope_amd.so"))
ABI_VERSION = 3

c_int, c_int64, c_float, c_void_p, c_char_p, c_uint64 = C.c_int, C.c_int64, C.c_float, C.c_void_p, C.c_char_p, C.c_uint64


class PtrRefParams(C.Structure):
    _fields_ = [("H", c_int), ("M", c_int), ("bs", c_int), ("T", c_int64), ("stride_h", c_int64),
                ("stride_t", c_int64), ("rep_mean", c_int), ("local_blocks", c_int), ("ptr_half_blocks", c_int),
                ("global_blocks_cfg", c_int), ("global_active", c_int), ("radius_mode_pi", c_int),
                ("budget_rem", c_int), ("budget_temp", c_float), ("mask_active", c_int), ("half_active", c_int),
                ("gumbel_k", c_int), ("gumbel_tau", c_float), ("eps", c_float)]


class PtrScoreParams(C.Structure):
    _fields_ = [("H", c_int), ("NB", c_int), ("D", c_int), ("bs", c_int), ("window", c_int), ("n_global", c_int),
                ("budget", c_int), ("temp", c_float), ("logit_scale", c_float), ("noise_mode", c_int),
                ("seed", c_uint64), ("eps", c_float), ("prior_head_stride", c_int64), ("flags", c_int)]

PTR_LOGITS_SCRATCH = 1  # SCOPE_PTR_LOGITS_SCRATCH


class StatsParams(C.Structure):
    _fields_ = [("H", c_int), ("QB", c_int), ("bs", c_int), ("M", c_int), ("T", c_int64), ("stride_h", c_int64),
                ("stride_t", c_int64), ("rep_mean", c_int), ("has_docs", c_int), ("docstart_enabled", c_int),
                ("local_blocks_cfg", c_int), ("eps", c_float), ("maxkv_bins", c_int), ("radius_bins", c_int),
                ("extra_bins", c_int), ("budget", c_int), ("bs_local_blocks", c_int)]


class AttnParams(C.Structure):
    _fields_ = [("H", c_int), ("D", c_int), ("bs", c_int), ("maxkv", c_int), ("T", c_int64), ("scale", c_float),
                ("beta", c_float), ("bias_mode", c_int), ("K", c_int), ("use_slope", c_int),
                ("subtract_b0", c_int), ("gate_kind", c_int), ("ramp_lambda", c_float), ("tau", c_float),
                ("q_sh", c_int64), ("q_st", c_int64), ("k_sh", c_int64), ("k_st", c_int64), ("v_sh", c_int64),
                ("v_st", c_int64), ("o_sh", c_int64), ("o_st", c_int64), ("pair_bias", c_void_p),
                ("dpair_bias", c_void_p)]


class PtrBwdParams(C.Structure):
    _fields_ = [("H", c_int), ("NB", c_int), ("D", c_int), ("bs", c_int), ("maxkv", c_int),
                ("logit_scale", c_float), ("soft_temp", c_float), ("q_sh", c_int64), ("q_st", c_int64),
                ("k_sh", c_int64), ("k_st", c_int64)]


class CoeffParams(C.Structure):
    _fields_ = [("M", c_int), ("K", c_int), ("rows", c_int64), ("L", c_int64), ("y_cols", c_int),
                ("y_stride", c_int), ("y_bf16", c_int), ("use_slope", c_int), ("subtract_b0", c_int),
                ("training", c_int), ("delta_cap", c_float), ("logw_min", c_float), ("logw_max", c_float),
                ("c_scale", c_float), ("width_min", c_float), ("width_max", c_float), ("eps", c_float),
                ("lambda_omega", c_float), ("lambda_entropy", c_float), ("lambda_zero_mean", c_float),
                ("lambda_delta_edge", c_float), ("entropy_floor", c_float), ("delta_edge_eps", c_float)]


class WgradParams(C.Structure):
    _fields_ = [("rows", c_int64), ("seg", c_int64), ("M", c_int), ("N", c_int), ("a_ss", c_int64),
                ("a_rs", c_int64), ("b_ss", c_int64), ("b_rs", c_int64), ("round_bf16", c_int)]


class MlpParams(C.Structure):
    _fields_ = [("rows", c_int64), ("seg", c_int64), ("q_ss", c_int64), ("q_rs", c_int64), ("D", c_int), ("H", c_int),
                ("O", c_int)]


class DecodeParams(C.Structure):
    _fields_ = [("H", c_int), ("D", c_int), ("bs", c_int), ("maxkv", c_int), ("T_cap", c_int64), ("t", c_int64),
                ("scale", c_float), ("q_sh", c_int64), ("k_sh", c_int64), ("k_st", c_int64), ("v_sh", c_int64),
                ("v_st", c_int64), ("o_sh", c_int64)]


P = c_void_p
_PROTOS = {
    "scope_abi_version": (c_int, []),
    "scope_last_error": (c_char_p, []),
    "scope_doc_starts": (c_int, [P, c_int64, c_int, c_int, c_int, P, P, P, P]),
    "scope_ptr_ref_maxkv": (c_int, [C.POINTER(PtrRefParams)]),
    "scope_pointer_mask_ref": (c_int, [C.POINTER(PtrRefParams), P, P, P, P, P, P, P, P, P, P]),
    "scope_block_means": (c_int, [P, P, c_int, c_int64, c_int, c_int, c_int64, c_int64, c_int64, c_int64, P, P, P]),
    "scope_block_means_docs": (c_int, [P, P, P, c_int, c_int64, c_int, c_int, c_int64, c_int64, c_int64, c_int64,
                                       c_int, c_int, P, P, P, P, P, P]),
    "scope_pointer_select": (c_int, [C.POINTER(PtrScoreParams), P, P, P, P, P, P, P, P, P, P, P, P]),
    "scope_pointer_pair_bias": (c_int, [C.POINTER(PtrScoreParams), c_float, P, P, P, P, P, P, P, P, P]),
    "scope_pointer_bwd_workspace_bytes": (c_int64, [C.POINTER(PtrBwdParams)]),
    "scope_pointer_bwd": (c_int, [C.POINTER(PtrBwdParams)] + [P] * 12),
    "scope_transpose_workspace_bytes": (c_int64, [c_int, c_int]),
    "scope_transpose_blocks": (c_int, [P, P, c_int, c_int, c_int, c_int, P, P, P, P]),
    "scope_transpose_blocks_noalloc": (c_int, [P, P, c_int, c_int, c_int, c_int, P, P, P]),
    "scope_check_lists": (c_int, [P, P, c_int, c_int, c_int, c_int, c_int, P, P]),
    "scope_coeff_head_workspace_bytes": (c_int64, [C.POINTER(CoeffParams)]),
    "scope_coeff_head_fwd": (c_int, [C.POINTER(CoeffParams)] + [P] * 17),
    "scope_coeff_head_bwd": (c_int, [C.POINTER(CoeffParams)] + [P] * 18),
    "scope_linear_wgrad_workspace_bytes": (c_int64, [C.POINTER(WgradParams)]),
    "scope_linear_wgrad": (c_int, [C.POINTER(WgradParams)] + [P] * 6),
    "scope_coeff_mlp_fwd": (c_int, [C.POINTER(MlpParams)] + [P] * 7),
    "scope_coeff_mlp_bwd": (c_int, [C.POINTER(MlpParams)] + [P] * 11),
    "scope_coeff_mlp_wgrad_workspace_bytes": (c_int64, [C.POINTER(MlpParams)]),
    "scope_coeff_mlp_wgrad": (c_int, [C.POINTER(MlpParams)] + [P] * 11),
    "scope_swa_width": (c_int, [c_int64, c_int, c_int]),
    "scope_swa_blockmask": (c_int, [P, c_int64, c_int, c_int, P, P, P, P, P, P, P, P]),
    "scope_stats_counts_len": (c_int64, [C.POINTER(StatsParams)]),
    "scope_stats_workspace_bytes": (c_int64, [C.POINTER(StatsParams)]),
    "scope_mask_stats": (c_int, [C.POINTER(StatsParams), P, P, P, P, P, P, P, P, P, P, P, P, P]),
    "scope_spectral_table_bytes": (c_int64, [c_int, c_int64, c_int]),
    "scope_spectral_table": (c_int, [c_int, P, c_int, c_int64, c_int, P, P]),
    "scope_attn_fwd": (c_int, [C.POINTER(AttnParams)] + [P] * 17),
    "scope_attn_block_mass": (c_int, [C.POINTER(AttnParams)] + [P] * 16),
    "scope_attn_bwd_workspace_bytes": (c_int64, [C.POINTER(AttnParams)]),
    "scope_decode_workspace_bytes": (c_int64, [C.POINTER(DecodeParams)]),
    "scope_decode_attn": (c_int, [C.POINTER(DecodeParams)] + [P] * 10),
    "scope_decode_attn_at": (c_int, [C.POINTER(DecodeParams)] + [P] * 11),
    "scope_decoder_qkv_glue": (c_int, [c_int, c_int, c_int, c_int64, c_float, c_float, c_float, P, P, P, P, P,
                                       c_int64, c_int64, P, P, P, c_int64, c_int64, c_int64, c_int64, c_int, P]),
    "scope_decoder_gemv": (c_int, [c_int, c_int, c_int64, c_int, c_float, c_int, P, P, P, P, P, P, P]),
    "scope_argmax_f32": (c_int, [P, c_int64, P, P]),
    "scope_decode_attn_glue_at": (c_int, [C.POINTER(DecodeParams), P, P, P, c_float, c_float, c_float, P, P, c_int64,
                                          c_int64, P, P, P, P, P, P, P, P, P, P]),
    "scope_decoder_step_prologue": (c_int, [P, P, c_int64, c_int64, c_int, c_float, c_int64, P, P, P, P, P, P, P, P,
                                            P]),
    "scope_attn_bwd": (c_int, [C.POINTER(AttnParams)] + [P] * 30),
    "scope_attn_bwd_phase": (c_int, [C.POINTER(AttnParams), c_int] + [P] * 30),
    "scope_probe_mfma_flops": (c_int64, [c_int, c_int]),
    "scope_probe_mfma": (c_int, [P, c_int, c_int, P]),
    "scope_probe_mfma_data": (c_int, [P, P, c_int, c_int, P]),
    "scope_probe_copy": (c_int, [P, P, c_int64, P]),
}

_lib = None
_lock = threading.Lock()


class ScopeLibraryError(RuntimeError):
    """The native library is missing, failed to load, or an entry point failed."""


def load(path: str | None = None) -> C.CDLL:
    """Load (once) and return the native library; raises if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise ScopeLibraryError(
                f"libscope_amd.so not found at {p}; build it with `python -m scope_amd.build` "
                "(there is no CPU fallback)")
        lib = C.CDLL(p, mode=C.RTLD_GLOBAL)
        for name, (res, args) in _PROTOS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        v = lib.scope_abi_version()
        if v != ABI_VERSION:
            raise ScopeLibraryError(f"libscope_amd.so ABI {v} != expected {ABI_VERSION}")
        if path is None:
            _lib = lib
        return lib


def call(name: str, *args) -> None:
    """Call an int-returning entry point and raise on a non-zero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.scope_last_error().decode(errors="replace")
        raise ScopeLibraryError(f"{name} failed ({rc}): {msg}")


def query(name: str, *args):
    return getattr(load(), name)(*args)
