"""ctypes binding of libds4hip.so (the C-ABI declared in include/ds4hip.h).

The library is loaded from the package directory only; there is no fallback:
if it is missing, every call raises.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libds4hip.so"

_vp, _i, _ll, _sz = C.c_void_p, C.c_int, C.c_longlong, C.c_size_t

# name -> argtypes (all return int)
SIGNATURES: dict[str, list] = {
    "ds4hip_get_last_error": [],
    "ds4hip_set_last_error": [_i],
    "ds4hip_clear_last_error": [],
    "ds4hip_version": [],
    "ds4hip_fp8_kv_quantize_round_trip_f32": [_vp, _vp, _i, _i, _i, _vp],
    "ds4hip_fp8_kv_quantize_append": [_vp, _i, _i, _i, _vp, _vp, _vp, _ll, _vp, _vp],
    "ds4hip_flash_attn_decode_raw_f32": [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp],
    "ds4hip_flash_attn_decode_mixed_f32": [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp],
    "ds4hip_flash_attn_decode_f32_workspace_size": [_ll, C.POINTER(_sz)],
    "ds4hip_flash_attn_decode_raw_f32_prealloc": [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp, _sz,
                                                  _vp],
    "ds4hip_flash_attn_decode_mixed_f32_noalloc": [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i,
                                                   _vp],
    "ds4hip_flash_attn_decode_mixed_f32_prealloc": [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i,
                                                    _vp, _sz, _vp],
    "ds4hip_flash_attn_decode_fp8_workspace_size": [_vp, _i, C.POINTER(_sz)],
    "ds4hip_flash_attn_decode_fp8": [
        _vp, _i, _ll, _vp, _ll, _vp, _ll, _vp, _vp, _vp, _vp, _i, _vp, _ll, _vp, _ll, _vp, _i,
        _i, _i, _i, _i, _ll, _vp, _vp, _sz, _i, _vp],
    "ds4hip_flash_attn_prefill_fp8_workspace_size": [_i],
    "ds4hip_flash_attn_prefill_fp8": [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _sz, _i,
                                      _vp],
    "ds4hip_tail_rope_yarn_f32": [_vp, _vp, _i, _i, _i, _i, _i, _vp],
    "ds4hip_tail_rope_yarn_inverse_f32": [_vp, _vp, _i, _i, _i, _i, _i, _vp],
    "ds4hip_mul_mv_f16_f32": [_vp, _vp, _vp, _i, _i, _vp],
    "ds4hip_mul_mv_f16_scaled_f32": [_vp, _vp, _vp, _i, _i, C.c_float, _vp],
    "ds4hip_mul_mv_f16_rope_f32": [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp],
    "ds4hip_attn_out_decode_workspace_bytes": [_i, _i, _i, _i],
    "ds4hip_token_prologue_f32": [_vp, _vp],
    "ds4hip_batch_rows_push_f32": [_vp, _vp, _vp, _vp, _i, _i, _vp],
    "ds4hip_compressor_pair_batch_scratch_bytes": [_i, _i, _i, _i, _i],
    "ds4hip_compressor_pair_step_batch_w32": [_i, _vp, _i, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _sz, _vp],
    "ds4hip_session_claim_raw_row": [_vp, _i, C.POINTER(_ll)],
    "ds4hip_flash_attn_q_prep_f32": [_vp, _ll, _i, _vp, _ll, _vp],
    "ds4hip_flash_attn_q_prep_words": [],
    "ds4hip_compressor_emit_f32": [_i, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp],
    "ds4hip_attn_out_decode_f32": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _sz, _vp],
    "ds4hip_attn_out_decode_q8_f32": [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _sz, _vp],
    "ds4hip_mul_mv_q8_0_q8_0_grouped_f32": [_vp, _vp, _vp, _i, _i, _i, _vp],
    "ds4hip_mul_mv_q8_0_q8_0_grouped_f32_prealloc": [_vp, _vp, _vp, _i, _i, _i, _vp, _vp, _vp],
    "ds4hip_mul_mv_q8_0_q8_0_f32_prealloc": [_vp, _vp, _vp, _i, _i, _vp, _vp, _vp],
    "ds4hip_mul_mm_workspace_bytes": [_i, _i, _i],
    "ds4hip_mul_mm_bf16_f32": [_vp, _vp, _vp, _i, _i, _i, _vp, _sz, _vp],
    "ds4hip_indexer_allowed_short_circuit_i32": [_vp, _i, _i, _vp],
    "ds4hip_scale_inplace_f32": [_vp, _i, C.c_float, _vp],
    "ds4hip_indexer_score_topk_i32": [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp],
    "ds4hip_indexer_score_topk_f32_i32": [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp],
    "ds4hip_indexer_select_scratch_bytes": [_i],
    "ds4hip_indexer_topk_positions": [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp,
                                      _vp],
    "ds4hip_compressor_decode_step_f32_prealloc": [_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i,
                                                   _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    "ds4hip_compressor_decode_step_f32": [_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp,
                                          _vp, _vp, _vp, _vp],
    "ds4hip_compressor_decode_step_w32": [_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp,
                                          _vp, _vp, _vp, _vp],
    "ds4hip_mul_mm_f32_f32": [_vp, _vp, _vp, _i, _i, _i, _vp, _sz, _vp],
    "ds4hip_compressor_batch_scratch_bytes": [_i, _i, _i, _i],
    "ds4hip_tail_rope_yarn_batch_f32": [_vp, _vp, _i, _i, _i, _i, _vp, _i, _i, _vp],
    "ds4hip_indexer_topk_positions_batch": [_vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _i, _i, _vp,
                                            _vp, _i, _vp],
    "ds4hip_compressor_decode_step_batch_w32": [_i, _i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp,
                                                _vp, _i, _vp, _vp, _ll, _vp, _vp, _vp, _sz,
                                                _vp],
    "ds4hip_swa_push_f32": [_vp, C.POINTER(_i), _i, _vp, _i, _vp],
    "ds4hip_comp_push_f32": [_vp, C.POINTER(_i), _i, _vp, _i, _vp],
    "ds4hip_session_state_arena_bytes": [_i],
    "ds4hip_session_state_alloc": [_vp, _i],
    "ds4hip_session_state_free": [_vp],
    "ds4hip_session_state_reset": [_vp, _vp],
    "ds4hip_session_push_raw": [_vp, _i, _vp, _vp],
    "ds4hip_session_push_comp": [_vp, _i, _vp, _vp],
    "ds4hip_session_push_index_comp": [_vp, _i, _vp, _vp],
    "ds4hip_rows_scatter_f32": [_vp, _i, _i, _vp, _vp, _vp],
    "ds4hip_session_layer_rows": [_vp, _i, _i, C.POINTER(_vp), C.POINTER(_ll), C.POINTER(_vp)],
    "ds4hip_session_set_selection": [_vp, _i, _vp, _i, _vp],
    "ds4hip_rms_norm_f32": [_vp, _vp, _vp, _i, C.c_float, _vp],
    "ds4hip_rms_norm_batch_f32": [_vp, _vp, _i, _vp, _i, _i, C.c_float, _vp],
    "ds4hip_attn_qkv_decode_workspace_bytes": [],
    "ds4hip_attn_qkv_decode_f32": [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _sz,
                                   _vp],
    "ds4hip_session_chunk_rows": [_vp, _i, _i, _i, _vp, _vp, _vp, _i, _vp, _i, _vp, _vp],
    "ds4hip_session_chunk_rows_host": [_vp, _i, _i, _i, _vp, _vp, _vp, _i, _vp, _i, _vp],
    "ds4hip_session_state_describe": [_vp, _i],
    "ds4hip_session_save_to_disk": [_vp, _vp, _i, C.c_char_p],
    "ds4hip_session_load_from_disk": [_vp, C.c_char_p, C.POINTER(_i), C.POINTER(_i)],
    "ds4hip_ds4cudak_probe": [C.c_char_p, _vp],
    "ds4hip_session_import_ds4cudak": [_vp, C.c_char_p, C.POINTER(_i), C.POINTER(_i)],
    "ds4hip_session_export_ds4cudak": [_vp, _vp, _i, C.c_char_p],
}

# entry points that return a value rather than a status
RESTYPES = {"ds4hip_indexer_select_scratch_bytes": C.c_size_t,
            "ds4hip_flash_attn_prefill_fp8_workspace_size": C.c_size_t,
            "ds4hip_session_state_arena_bytes": C.c_size_t,
            "ds4hip_mul_mm_workspace_bytes": C.c_size_t,
            "ds4hip_compressor_batch_scratch_bytes": C.c_size_t,
            "ds4hip_attn_qkv_decode_workspace_bytes": C.c_size_t,
            "ds4hip_attn_out_decode_workspace_bytes": C.c_size_t,
            "ds4hip_flash_attn_q_prep_words": C.c_longlong,
            "ds4hip_compressor_pair_batch_scratch_bytes": C.c_size_t}

_lib = None


class Ds4HipError(RuntimeError):
    def __init__(self, name: str, code: int):
        kind = "invalid argument" if code == -22 else (
            f"hip error {-1000 - code}" if code <= -1000 else "error")
        super().__init__(f"{name} failed: {code} ({kind})")
        self.code = code


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m ds4cuda_amd.build` "
                "(there is no CPU fallback)")
        l = C.CDLL(str(LIB_PATH))
        for name, args in SIGNATURES.items():
            fn = getattr(l, name)
            fn.argtypes = args
            fn.restype = RESTYPES.get(name, C.c_int)
        _lib = l
    return _lib


def call(name: str, *args) -> int:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise Ds4HipError(name, rc)
    return rc
