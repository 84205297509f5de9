"""ctypes binding of ``librecir_hstu.so`` (the C ABI declared in ``include/recir_hstu.h``)."""
from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
# RECIR_HSTU_LIB names another build of the same library (deployments that keep the binary
# elsewhere, A/B measurements of two builds); there is still no fallback if it is missing
LIB_PATH = os.environ.get("RECIR_HSTU_LIB") or os.path.join(_PKG, "librecir_hstu.so")

ABI_VERSION = 6

DTYPE_BF16 = 0
DTYPE_FP32 = 1
DTYPE_FP8_E4M3 = 2
DTYPE_FP16 = 3

FLAG_OFFSETS_I32 = 0x1
FLAG_CTX_REFERENCE = 0x2
FLAG_SCALE_PER_TOKEN = 0x4
FLAG_REUSE_PLAN = 0x8
FLAG_GROUPED_LISTS = 0x10000
FLAG_MASK_NONCAUSAL = 0x20000
FLAG_TILED_ONLY = 0x40000
FLAG_KERNEL_SHIFT = 8
NOALLOC_SCRATCH_BYTES = 4 << 20

# every symbol include/recir_hstu.h declares
EXPORTS = (
    "recir_hstu_attn_fwd",
    "recir_hstu_attn_fwd_noalloc",
    "recir_hstu_attn_fwd_workspace_bytes",
    "recir_hstu_attn_bwd",
    "recir_hstu_attn_bwd_workspace_bytes",
    "recir_hstu_attn_bwd_rab_grad_workspace_bytes",
    "recir_hstu_quantize_e4m3_per_head",
    "recir_hstu_quantize_e4m3_per_head_rows",
    "recir_hstu_calibration_copy",
    "recir_hstu_calibration_mfma_loop",
    "recir_hstu_last_error",
    "recir_hstu_abi_version",
    "recir_hstu_last_kernel",
)
# every symbol include/recir_jagged.h declares
JAGGED_EXPORTS = (
    "recir_jagged_to_padded_dense",
    "recir_dense_to_jagged",
    "recir_concat_2d_jagged",
    "recir_split_2d_jagged",
    "recir_add_timestamp_position_embeddings",
    "recir_add_timestamp_position_embeddings_workspace_bytes",
)

_lib = None


class HipExtensionMissing(RuntimeError):
    """The compiled HIP library is absent; there is no other implementation to fall back on."""


def load() -> ctypes.CDLL:
    """Load the library built by ``recir_amd.build`` (never builds, never falls back)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise HipExtensionMissing(
            f"{LIB_PATH} not found: build it with `python -m recir_amd.build` "
            "(hipcc --offload-arch=gfx950); this package has no CPU or eager fallback")
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, u32, f32, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_uint32, ctypes.c_float, ctypes.c_size_t
    L.recir_hstu_attn_fwd.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                      i32, i32, i32, i32, i32, i32, i32, i32, i32, f32, i32, u32, vp, sz, vp]
    L.recir_hstu_attn_fwd.restype = ctypes.c_int
    L.recir_hstu_attn_fwd_noalloc.argtypes = L.recir_hstu_attn_fwd.argtypes[:22] + [vp]
    L.recir_hstu_attn_fwd_noalloc.restype = ctypes.c_int
    L.recir_hstu_attn_fwd_workspace_bytes.argtypes = [i32, i32, i32, i32, i32, i32]
    L.recir_hstu_attn_fwd_workspace_bytes.restype = sz
    L.recir_hstu_attn_bwd.argtypes = [vp] * 12 + [i32] * 9 + [f32, i32, u32, vp, sz, vp]
    L.recir_hstu_attn_bwd.restype = ctypes.c_int
    L.recir_hstu_attn_bwd_workspace_bytes.argtypes = [i32, i32, i32, i32, i32, i32]
    L.recir_hstu_attn_bwd_workspace_bytes.restype = sz
    L.recir_hstu_attn_bwd_rab_grad_workspace_bytes.argtypes = [i32, i32]
    L.recir_hstu_attn_bwd_rab_grad_workspace_bytes.restype = sz
    L.recir_hstu_quantize_e4m3_per_head.argtypes = [vp, vp, vp, i32, i32, i32, vp]
    L.recir_hstu_quantize_e4m3_per_head.restype = ctypes.c_int
    L.recir_hstu_quantize_e4m3_per_head_rows.argtypes = [vp, vp, vp, i32, i32, i32, vp, i32, u32, vp]
    L.recir_hstu_quantize_e4m3_per_head_rows.restype = ctypes.c_int
    L.recir_hstu_calibration_copy.argtypes = [vp, vp, sz, vp]
    L.recir_hstu_calibration_copy.restype = ctypes.c_int
    L.recir_hstu_calibration_mfma_loop.argtypes = [i32, i32, vp, vp, vp, sz, i32, i32, i32, f32, vp, vp, vp]
    L.recir_hstu_calibration_mfma_loop.restype = ctypes.c_int
    i64 = ctypes.c_int64
    L.recir_jagged_to_padded_dense.argtypes = [vp, vp, vp, i64, i32, i32, i64, i32, ctypes.c_uint64, u32, vp]
    L.recir_dense_to_jagged.argtypes = [vp, vp, vp, i64, i32, i32, i64, u32, vp]
    L.recir_concat_2d_jagged.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i64, i64, i64, i32, i32, u32, vp]
    L.recir_split_2d_jagged.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i64, i64, i64, i32, u32, vp]
    L.recir_add_timestamp_position_embeddings.argtypes = [vp] * 12 + [i64] + [i32] * 11 + [u32, vp, sz, vp]
    L.recir_add_timestamp_position_embeddings_workspace_bytes.argtypes = [i64, i32, i32]
    for name in JAGGED_EXPORTS:
        getattr(L, name).restype = ctypes.c_int
    L.recir_add_timestamp_position_embeddings_workspace_bytes.restype = sz
    L.recir_hstu_last_error.argtypes = []
    L.recir_hstu_last_error.restype = ctypes.c_char_p
    L.recir_hstu_last_kernel.argtypes = []
    L.recir_hstu_last_kernel.restype = ctypes.c_char_p
    L.recir_hstu_abi_version.argtypes = []
    L.recir_hstu_abi_version.restype = ctypes.c_int
    if L.recir_hstu_abi_version() != ABI_VERSION:
        raise RuntimeError(f"ABI mismatch: library {L.recir_hstu_abi_version()} vs binding {ABI_VERSION}")
    _lib = L
    return L


def last_error() -> str:
    return load().recir_hstu_last_error().decode()


def last_kernel() -> str:
    return load().recir_hstu_last_kernel().decode()
