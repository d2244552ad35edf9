"""ctypes binding of libqvex.so (the C ABI declared in include/qvex.h).

The library is loaded from this directory; there is no fallback: every op of
the package raises if the HIP library is missing or fails.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libqvex.so"

P = ctypes.c_void_p
I = ctypes.c_int
U64 = ctypes.c_uint64
F = ctypes.c_float
LNG = ctypes.c_long

# name -> argtypes (all return int status)
SIGNATURES: dict[str, list] = {
    "qvex_qmv_w4g64": [P, P, P, P, P, I, I, I, P],
    "qvex_qmv_w4g64_tiled": [P, P, P, P, P, I, I, I, I, I, P],
    "qvex_read_roof": [P, U64, P, I, P],
    "qvex_read_probe": [P, U64, P, I, I, I, P],
    "qvex_qmv_w4g64_mfma": [P, P, P, P, P, I, I, I, I, I, P],
    "qvex_qmv_affine": [P, P, P, P, P, I, I, I, I, I, P],
    "qvex_embed_affine": [P, I, P, P, P, I, I, I, I, P, P],
    "qvex_affine_widen_w4g64": [P, P, P, I, I, I, I, P, P, P, P],
    "qvex_w4g64_pack": [P, P, P, I, I, P, U64, P],
    "qvex_w4g64_dequant": [P, P, P, I, I, P, P],
    "qvex_w4g64_packed_gemm": [P, P, P, I, I, I, P],
    "qvex_w4g64_packed_gemm_swiglu": [P, P, P, I, I, I, P],
    "qvex_qmv_w4g64_packed": [P, P, P, I, I, I, P],
    "qvex_qmv_w4g64_packed_tiled": [P, P, P, I, I, I, I, I, I, P],
    "qvex_qmv_w4g64_packed_resid": [P, P, I, I, I, P, P, P, P, P, P],
    "qvex_qmv_w4g64_packed_rstd": [P, P, P, I, I, I, P, I, I, F, I, P],
    "qvex_qmv_w4g64_packed_rstd_tilemax": [P, P, P, I, I, I, P, I, I, F, P, P],
    "qvex_qmv_w4g64_packed_gnorm_resid": [P, P, I, I, I, P, I, F, P, P, P, P, P, P],
    "qvex_rms_parts": [P, P, P, P, I, I, P],
    "qvex_qmv_w4g64_packed_argmax": [P, P, I, I, I, P, I, I, F, P, P, U64, P],
    "qvex_w4g64_pack_swiglu": [P, P, P, I, I, P, U64, P],
    "qvex_qmv_w4g64_packed_swiglu": [P, P, P, I, I, I, P],
    "qvex_gdn_recurrent": [P, P, P, P, P, P, P, P, P, I, P, I, I, I, I, I, I, P],
    "qvex_gdn_recurrent_ring": [P, P, P, P, P, P, P, P, I, P, I, P, I, I, I, I, I, I, P],
    "qvex_gdn_decode_fused": [P, LNG, P, I, P, P, I, I, I, F, F, F, P, P, I, I, P, I, I, P, F, P, I, I, I, I, I, P],
    "qvex_gdn_decode_split": [P, LNG, P, I, P, P, I, I, I, F, F, F, P, P, I, I, P, I, I, P, P, P, I, I, I, I, I, I, P],
    "qvex_gdn_chunked": [P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, I, P, U64, P],
    "qvex_spec_accept": [P, P, P, P, P, F, P, P, I, I, I, P, U64, P],
    "qvex_spec_accept_filtered": [P, P, P, P, P, F, P, F, I, F, P, P, I, I, I, P, U64, P],
    "qvex_spec_accept_filtered_bf16": [P, P, P, P, P, F, P, F, I, F, P, P, I, I, I, P, U64, P],
    "qvex_spec_accept_tiles_bf16": [P, P, P, P, P, F, P, F, I, F, P, P, I, I, I, P, U64, P],
    "qvex_spec_accept_tiles_rows_bf16": [P, P, P, P, P, F, P, F, I, F, P, I, I, I, P, U64, P],
    "qvex_tile_max_bf16": [P, I, I, P, P],
    "qvex_spec_accept_filtered_bf16_noalloc": [P, P, P, P, P, F, P, F, I, F, P, P, I, I, I, P],
    "qvex_sampler_scores": [P, I, I, I, P, F, F, I, F, P, P, U64, P],
    "qvex_mark_seen": [P, I, P, I, P, I, P],
    "qvex_embed_w4g64": [P, I, P, P, P, I, I, P, P],
    "qvex_mtp_input": [P, I, P, I, P, P, P, P, P, I, I, P, P, LNG, P, P, P, LNG, F, P, I, P, I, P],
    "qvex_embed_rms_parts": [P, I, P, I, P, I, P, P, P, I, I, P, P, P, P, P],
    "qvex_rmsnorm": [P, LNG, P, P, LNG, I, I, F, F, P],
    "qvex_add_rmsnorm": [P, P, P, P, P, I, I, F, P],
    "qvex_rmsnorm_pair": [P, LNG, P, P, P, LNG, P, P, LNG, I, I, F, P],
    "qvex_gdn_conv_qk": [P, LNG, P, I, P, P, I, P, P, P, P, P, I, I, I, I, I, F, F, F, P],
    "qvex_commit_step": [P, I, P, I, P],
    "qvex_gather_row": [P, LNG, P, I, P, I, P],
    "qvex_assemble_ids": [P, P, I, P, P],
    "qvex_cycle_finish_ex": [P, I, P, P, P, P, P, P, P, P, I, I, P, I, I, U64, P, I, P, P, P, P],
    "qvex_cycle_finish": [P, I, P, P, P, P, P, P, P],
    "qvex_philox_uniforms": [U64, P, I, P, P],
    "qvex_gated_rmsnorm": [P, P, LNG, I, P, P, I, I, F, P],
    "qvex_swiglu": [P, P, I, I, P],
    "qvex_bf16_to_f32": [P, P, LNG, P],
    "qvex_attn_qk_rope": [P, LNG, P, P, P, I, I, I, I, I, F, F, P, P, P, I, P, I, P],
    "qvex_attention": [P, P, P, P, I, I, I, I, I, I, I, I, P, LNG, P, P, U64, P],
    "qvex_attention_decode": [P, LNG, P, P, P, I, I, I, I, I, F, P, I, P, P, I, I, I, P, P, U64, P],
    "qvex_rope_table": [I, F, I, P, P],
}

# qvex_abi_version() of the library these bindings match (8: the RoPE table of
# qvex_attn_qk_rope; 7: the rows argument of qvex_cycle_finish_ex; 6: the done flag of qvex_cycle_finish_ex; 4: qvex_mtp_input, qvex_embed_rms_parts, the deferred
# reduction of qvex_qmv_w4g64_packed_argmax)
ABI_VERSION = 8

_lib: ctypes.CDLL | None = None


class QvexError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise QvexError(f"{LIB_PATH} is not built: run `python -m qvex.build` "
                            "(or __graft_entry__.build()) first")
        L = ctypes.CDLL(str(LIB_PATH))
        L.qvex_last_error.restype = ctypes.c_char_p
        L.qvex_last_error.argtypes = []
        L.qvex_abi_version.restype = I
        L.qvex_abi_version.argtypes = []
        if L.qvex_abi_version() != ABI_VERSION:
            raise QvexError(f"{LIB_PATH} has ABI version {L.qvex_abi_version()}, these bindings need "
                            f"{ABI_VERSION}: rebuild it")
        L.qvex_spec_accept_workspace_bytes.restype = U64
        L.qvex_spec_accept_workspace_bytes.argtypes = [I, I, I, I]
        L.qvex_attn_workspace_bytes.restype = U64
        L.qvex_attn_workspace_bytes.argtypes = [I, I, I, I, I, I]
        L.qvex_w4g64_packed_bytes.restype = U64
        L.qvex_w4g64_packed_bytes.argtypes = [I, I]
        L.qvex_spec_accept_filtered_workspace_bytes.restype = U64
        L.qvex_spec_accept_filtered_workspace_bytes.argtypes = [I, I, I, I, I]
        L.qvex_gdn_chunked_workspace_bytes.restype = U64
        L.qvex_gdn_chunked_workspace_bytes.argtypes = [I, I, I, I, I, I]
        L.qvex_sampler_scores_workspace_bytes.restype = U64
        L.qvex_sampler_scores_workspace_bytes.argtypes = [I, I, I]
        L.qvex_qmv_w4g64_argmax_workspace_bytes.restype = U64
        L.qvex_qmv_w4g64_argmax_workspace_bytes.argtypes = [I, I]
        L.qvex_spec_accept_tiles_applies.restype = I          # 1 / 0, not a status
        L.qvex_spec_accept_tiles_applies.argtypes = [I, I, I, F, I, F]
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = I
        _lib = L
    return _lib


def call(name: str, *args) -> None:
    """Call an entry point and raise QvexError with the library's message on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().qvex_last_error().decode(errors="replace")
        raise QvexError(f"{name} failed (status {rc}): {msg}")


def exported_symbols() -> list[str]:
    return ["qvex_last_error", "qvex_abi_version", "qvex_spec_accept_workspace_bytes",
            "qvex_attn_workspace_bytes", "qvex_w4g64_packed_bytes",
            "qvex_gdn_chunked_workspace_bytes", "qvex_spec_accept_filtered_workspace_bytes",
            "qvex_qmv_w4g64_argmax_workspace_bytes", "qvex_sampler_scores_workspace_bytes",
            "qvex_spec_accept_tiles_applies", *SIGNATURES]
