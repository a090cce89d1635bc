"""ctypes binding of libaffmae.so (the C ABI in include/affmae.h).

The library is loaded after torch so that it binds to the HIP runtime torch
already loaded (both use the soname libamdhip64.so.7); stream handles from
``torch.cuda.current_stream().cuda_stream`` are therefore valid here.  There
is no CPU fallback: every op raises if the library or a GPU is missing.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libaffmae.so"

AFF_OK = 0
AFF_ERR_INVALID_ARG = 1
AFF_ERR_UNSUPPORTED = 2
AFF_ERR_WORKSPACE = 3
AFF_ERR_LAUNCH = 4

AFF_F32, AFF_F16, AFF_BF16 = 0, 1, 2
KNN_NOALLOC_SCRATCH_BYTES = 16 << 20   # AFF_KNN_NOALLOC_SCRATCH_BYTES
DTYPE_CODE = {torch.float32: AFF_F32, torch.float16: AFF_F16, torch.bfloat16: AFF_BF16}

ABI_VERSION = 8

P = ctypes.c_void_p
I32 = ctypes.c_int
I64 = ctypes.c_int64
F32 = ctypes.c_float
SZ = ctypes.c_size_t


class NbhdAttnArgs(ctypes.Structure):
    """Mirror of ``aff_nbhd_attn_args`` (include/affmae.h)."""
    _fields_ = [
        ("dtype", I32), ("B", I32), ("H", I32), ("N", I32), ("M", I32), ("D", I32),
        ("scale", F32),
        ("q", P), ("q_sb", I64), ("q_sh", I64), ("q_sn", I64),
        ("k", P), ("k_sb", I64), ("k_sh", I64), ("k_sn", I64),
        ("v", P), ("v_sb", I64), ("v_sh", I64), ("v_sn", I64),
        ("member_idx", P), ("idx_is_i64", I32), ("mi_sb", I64), ("mi_sn", I64),
        ("bias_mode", I32),
        ("bias", P), ("bias_dtype", I32), ("bias_sb", I64), ("bias_sh", I64), ("bias_sn", I64),
        ("pe_idx", P), ("pe_is_i64", I32), ("pe_sb", I64), ("pe_sn", I64),
        ("table", P), ("table_dtype", I32), ("table_rows", I64),
        ("pos", P), ("pos_sb", I64), ("pos_sn", I64),
        ("rel_width", I32),
        ("pos_w", P), ("pos_b", P),
        ("mask", P), ("mask_sb", I64), ("mask_sh", I64), ("mask_sn", I64),
        ("blank_k", P), ("blank_v", P),
        ("out", P), ("o_sb", I64), ("o_sh", I64), ("o_sn", I64),
        ("lse", P),
        ("ws", P), ("ws_bytes", SZ),
    ]


class NbhdAttnBwdArgs(ctypes.Structure):
    """Mirror of ``aff_nbhd_attn_bwd_args`` (include/affmae.h)."""
    _fields_ = [
        ("fwd", NbhdAttnArgs),
        ("dout", P), ("do_sb", I64), ("do_sh", I64), ("do_sn", I64),
        ("dq", P), ("dq_sb", I64), ("dq_sh", I64), ("dq_sn", I64),
        ("dk", P), ("dk_sb", I64), ("dk_sh", I64), ("dk_sn", I64),
        ("dv", P), ("dv_sb", I64), ("dv_sh", I64), ("dv_sn", I64),
        ("dbias", P), ("dtable", P), ("dblank_k", P), ("dblank_v", P),
        ("ws", P), ("ws_bytes", SZ),
    ]


DEFORM_MAX_LEVELS = 8
DEFORM_SHEPARD, DEFORM_IDW = 0, 1


class DeformArgs(ctypes.Structure):
    """Mirror of ``aff_deform_args`` (include/affmae.h)."""
    _fields_ = [
        ("mode", I32), ("B", I32), ("Nq", I32), ("H", I32), ("L", I32), ("P", I32), ("K", I32), ("C", I32),
        ("query_pos", P), ("qp_sb", I64), ("qp_sn", I64),
        ("kv_pos", P), ("kp_sb", I64), ("kp_sn", I64),
        ("level_start", I32 * (DEFORM_MAX_LEVELS + 1)),
        ("offsets", P), ("off_dtype", I32), ("off_sb", I64), ("off_sn", I64), ("off_sh", I64),
        ("attn", P), ("attn_dtype", I32), ("at_sb", I64), ("at_sn", I64), ("at_sh", I64),
        ("dtype", I32), ("values", P), ("v_sb", I64), ("v_sn", I64), ("v_sh", I64),
        ("power", P),
        ("out", P), ("o_sb", I64), ("o_sn", I64), ("o_sh", I64),
        ("knn_idx", P), ("knn_d2", P),
    ]


DEFORM_BWD_SHEPARD, DEFORM_BWD_IDW, DEFORM_BWD_SAMPLE, DEFORM_BWD_SAMPLE_SQ, DEFORM_BWD_GIVEN = 0, 1, 2, 3, 4


class DeformBwdArgs(ctypes.Structure):
    """Mirror of ``aff_deform_bwd_args`` (include/affmae.h)."""
    _fields_ = [
        ("mode", I32), ("B", I32), ("Q", I32), ("H", I32), ("S", I32), ("K", I32), ("C", I32), ("D", I32),
        ("P", I32), ("Nkv", I32),
        ("level_start", I32 * (DEFORM_MAX_LEVELS + 1)),
        ("loc", P), ("loc_sb", I64), ("loc_sn", I64),
        ("offsets", P), ("off_dtype", I32), ("off_sb", I64), ("off_sn", I64), ("off_sh", I64),
        ("kv_pos", P), ("kp_sb", I64), ("kp_sn", I64),
        ("idx", P), ("idx_is_i64", I32), ("i_sb", I64), ("i_sn", I64), ("i_sh", I64),
        ("attn", P), ("attn_dtype", I32), ("at_sb", I64), ("at_sn", I64), ("at_sh", I64),
        ("weights", P), ("w_dtype", I32), ("w_sb", I64), ("w_sn", I64), ("w_sh", I64),
        ("dtype", I32),
        ("values", P), ("v_sb", I64), ("v_sn", I64), ("v_sh", I64),
        ("dout", P), ("do_sb", I64), ("do_sn", I64), ("do_sh", I64),
        ("d_w_in", P), ("dwi_sb", I64), ("dwi_sn", I64), ("dwi_sh", I64),
        ("power", P),
        ("d_loc", P), ("d_attn", P), ("d_weights", P), ("d_kv_pos", P), ("d_values", P), ("d_power", P),
    ]


SFC_MAX_LEVELS = 16
SFC_SCANLINE, SFC_PEANO, SFC_HILBERT = 0, 1, 2


class SfcCurveArgs(ctypes.Structure):
    """Mirror of ``aff_sfc_curve_args`` (include/affmae.h)."""
    _fields_ = [
        ("pos", P), ("p_sb", I64), ("p_sn", I64),
        ("B", I32), ("N", I32), ("curve", I32), ("w", I32), ("levels", I32), ("first_w", I32),
        ("cur_h", F32 * SFC_MAX_LEVELS), ("inv_h", F32 * SFC_MAX_LEVELS), ("level_scale", F32 * SFC_MAX_LEVELS),
        ("keys", P),
    ]


class SfcAnchorArgs(ctypes.Structure):
    """Mirror of ``aff_sfc_anchor_args`` (include/affmae.h)."""
    _fields_ = [
        ("pos", P), ("p_sb", I64), ("p_sn", I64),
        ("B", I32), ("N", I32), ("plw", F32), ("plh", F32), ("npw", I32), ("ncell", I32),
        ("cell_rank", P), ("prev_c", P), ("next_c", P), ("keys", P),
    ]


# Every symbol include/affmae.h declares, with (restype, argtypes).
SIGNATURES = {
    "aff_last_error": (ctypes.c_char_p, []),
    "aff_abi_version": (I32, []),
    "aff_knn_workspace_bytes": (SZ, [I32, I32, I32, I32, I32]),
    "aff_knn": (I32, [P, I64, I64, P, I64, I64, I32, I32, I32, I32, I32, P, I32, P, P, SZ, P]),
    "aff_knn_noalloc": (I32, [P, I64, I64, P, I64, I64, I32, I32, I32, I32, I32, P, I32, P, P]),
    "aff_nbhd_attn_workspace_bytes": (SZ, [ctypes.POINTER(NbhdAttnArgs)]),
    "aff_nbhd_attn_fwd": (I32, [ctypes.POINTER(NbhdAttnArgs), P]),
    "aff_nbhd_attn_path": (I32, [ctypes.POINTER(NbhdAttnArgs)]),
    "aff_nbhd_attn_proj_fwd": (I32, [ctypes.POINTER(NbhdAttnArgs), P, P, P]),
    "aff_nbhd_attn_bwd_workspace_bytes": (SZ, [ctypes.POINTER(NbhdAttnBwdArgs)]),
    "aff_nbhd_attn_bwd": (I32, [ctypes.POINTER(NbhdAttnBwdArgs), P]),
    "aff_weighted_features_fwd": (I32, [P, I32, I64, I64, I64, I64, P, I32, I64, I64, P, I32, I64, I64,
                                        I32, I32, I32, I32, I32, I32, P, I64, I64, I64, P]),
    "aff_weighted_features_bwd_workspace_bytes": (SZ, [I32, I32, I32, I32]),
    "aff_weighted_features_bwd": (I32, [P, I64, I64, I64, P, I32, I64, I64, I64, I64, P, I32, I64, I64, P, I32,
                                        I64, I64, I32, I32, I32, I32, I32, I32, P, I32, P, P, SZ, P]),
    "aff_weighted_gather_fwd": (I32, [P, I32, I64, I64, P, I32, I64, I64, P, I32, I64, I64,
                                      I32, I32, I32, I32, I32, P, I64, I64, P]),
    "aff_softmax_merge_fwd": (I32, [P, I64, I64, P, I64, I64, P, I32, I64, I64, P, I32, I64, I64,
                                    I32, I32, I32, I32, I32, F32, P, I64, I64, P, I64, I64, P, P]),
    "aff_deform_workspace_bytes": (SZ, [ctypes.POINTER(DeformArgs)]),
    "aff_deform_fwd": (I32, [ctypes.POINTER(DeformArgs), P, SZ, P]),
    "aff_deform_sample_fwd": (I32, [I32, P, I64, I64, P, I64, I64, P, I32, I64, I64, P, I32, I32, I32, I32, I32,
                                    P, I32, I64, I64, P, I32, I64, I64, I32, P, I64, I64, P, I32, I64, I64, P]),
    "aff_msdetrpc_fwd": (I32, [P, I32, I64, I64, I64, P, I32, I64, I64, I64, P, I32, I64, I64, P, I32, I64, I64,
                               I32, I32, I32, I32, I32, I32, P, I64, I64, P]),
    "aff_cluster_members": (I32, [P, I32, I64, I64, P, I32, I64, I64, P, I64, I64, P, I64, I64,
                                  I32, I32, I32, I32, I32, I32, P, I32, P, P, I32, P]),
    "aff_deform_bwd_workspace_bytes": (SZ, [ctypes.POINTER(DeformBwdArgs)]),
    "aff_deform_bwd": (I32, [ctypes.POINTER(DeformBwdArgs), P, SZ, P]),
    "aff_sfc_curve_keys": (I32, [ctypes.POINTER(SfcCurveArgs), P]),
    "aff_sfc_anchor_workspace_bytes": (SZ, [I32, I32]),
    "aff_sfc_anchor_keys": (I32, [ctypes.POINTER(SfcAnchorArgs), P, SZ, P]),
    "aff_sfc_argsort_workspace_bytes": (SZ, [I32, I32]),
    "aff_sfc_argsort": (I32, [P, I32, I32, P, P, SZ, P]),
    "aff_layer_norm_fwd": (I32, [P, I32, I64, P, I32, I64, P, P, I64, I32, F32, P]),
    "aff_layer_norm_map_fwd": (I32, [P, I32, P, I32, P, P, P, I32, I32, I32, I32, I32, I32, I32, F32, P]),
}

_lib = None


class AffLaunchError(RuntimeError):
    """The HIP runtime rejected a kernel launch."""


def load() -> ctypes.CDLL:
    """Load libaffmae.so and declare its signatures (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m affmae_amd.build_lib` "
                "(there is no CPU fallback for the HIP kernels)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.aff_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"libaffmae ABI version {ver} != expected {ABI_VERSION}; rebuild")
        _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status == AFF_OK:
        return
    msg = load().aff_last_error().decode(errors="replace")
    if status == AFF_ERR_INVALID_ARG:
        raise ValueError(f"{what}: {msg}")
    if status == AFF_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    if status == AFF_ERR_WORKSPACE:
        raise RuntimeError(f"{what}: {msg}")
    raise AffLaunchError(f"{what}: {msg}")


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_cuda(*tensors: torch.Tensor) -> torch.device:
    """Assert that every tensor lives on one GPU (the reference asserts the same)."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        assert t.is_cuda, "Inputs must be on CUDA"
        if dev is None:
            dev = t.device
        assert t.device == dev, f"all inputs must be on one device ({dev} vs {t.device})"
    return dev
