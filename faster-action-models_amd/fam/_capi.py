"""ctypes binding of libfam_hip.so, the C ABI declared in include/fam_hip.h.

This module is the only place that touches the shared library.  Loading fails loudly
when the library has not been built: there is no other implementation to fall back to.
"""
from __future__ import annotations

import ctypes as C
import os

LIB_NAME = "libfam_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

FAM_OK = 0
FAM_ERR_INVALID_ARG = 1
FAM_ERR_UNSUPPORTED = 2
FAM_ERR_LAUNCH = 3
FAM_ABI_VERSION = 3

FAM_MASK_NONE, FAM_MASK_BOOL, FAM_MASK_ADD_F32, FAM_MASK_ADD_BF16 = 0, 1, 2, 3
FAM_PRO_NONE, FAM_PRO_LAYERNORM, FAM_PRO_ADALN, FAM_PRO_LN_FOLDED = 0, 1, 2, 3
FAM_ACT_NONE, FAM_ACT_GELU_TANH, FAM_ACT_SILU, FAM_ACT_RELU, FAM_ACT_GELU_ERF = 0, 1, 2, 3, 4
FAM_ROWSRC_PARTIALS, FAM_ROWSRC_SMALLK = 0, 1
FAM_ROWNORM_NONE, FAM_ROWNORM_LAYERNORM, FAM_ROWNORM_ADALN, FAM_ROWNORM_RMS = 0, 1, 2, 3
FAM_Q8_ROW, FAM_Q8_GELU, FAM_Q8_LN_MOD, FAM_Q8_ADD_LN_MOD = 0, 1, 2, 3

_i64 = C.c_int64
_vp = C.c_void_p


class FamError(RuntimeError):
    """Raised when an entry point of libfam_hip.so returns an error code."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed (code {code}): {msg}")
        self.code = code


class AttnDesc(C.Structure):
    """fam_attn_desc (include/fam_hip.h)."""
    _fields_ = [
        ("q", _vp), ("q_bs", _i64), ("q_rs", _i64), ("q_hs", _i64),
        ("k0", _vp), ("k0_bs", _i64), ("k0_rs", _i64), ("k0_hs", _i64),
        ("v0", _vp), ("v0_bs", _i64), ("v0_rs", _i64), ("v0_hs", _i64),
        ("k1", _vp), ("k1_bs", _i64), ("k1_rs", _i64), ("k1_hs", _i64),
        ("v1", _vp), ("v1_bs", _i64), ("v1_rs", _i64), ("v1_hs", _i64),
        ("o", _vp), ("o_bs", _i64), ("o_rs", _i64), ("o_hs", _i64),
        ("batch", _i64), ("heads", _i64), ("sq", _i64), ("sk0", _i64), ("sk1", _i64), ("head_dim", _i64),
        ("scale", C.c_float),
        ("mask", _vp), ("mask_kind", C.c_int), ("mask_bs", _i64), ("mask_hs", _i64), ("mask_qs", _i64),
        ("num_splits", C.c_int), ("part_o", _vp), ("part_ml", _vp),
        ("qk_norm", C.c_int), ("q_sumsq", _vp), ("k_sumsq", _vp),
        ("ss_row_stride", _i64), ("ss_batch_rows", _i64), ("q_group0", _i64), ("k_group0", _i64), ("norm_width", _i64),
        ("q_norm_w", _vp), ("k_norm_w", _vp), ("norm_eps", C.c_float),
        ("rope_cos", _vp), ("rope_sin", _vp), ("rope_row_stride", _i64),
    ]


class GemmDesc(C.Structure):
    """fam_gemm_desc (include/fam_hip.h)."""
    _fields_ = [
        ("a", _vp), ("lda", _i64),
        ("w", _vp), ("ldw", _i64),
        ("bias", _vp),
        ("out", _vp), ("ldo", _i64),
        ("M", _i64), ("N", _i64), ("K", _i64),
        ("prologue", C.c_int),
        ("pro_w", _vp), ("pro_b", _vp),
        ("pro_shift", _vp), ("pro_scale", _vp),
        ("pro_mod_bs", _i64), ("pro_mod_rs", _i64),
        ("pro_eps", C.c_float),
        ("act", C.c_int),
        ("res", _vp), ("ldr", _i64),
        ("gate", _vp), ("gate_bs", _i64), ("gate_rs", _i64), ("gate_ns", _i64),
        ("rows_per_batch", _i64),
        ("out_f32", C.c_int),
    ]


class RowopDesc(C.Structure):
    """fam_rowop_desc (include/fam_hip.h)."""
    _fields_ = [
        ("src", C.c_int),
        ("partials", _vp), ("splits", _i64), ("split_stride", _i64),
        ("x_in", _vp), ("ldx", _i64), ("k_in", _i64), ("w_in", _vp),
        ("M", _i64), ("N", _i64),
        ("bias", _vp), ("act", C.c_int),
        ("res", _vp), ("ldr", _i64),
        ("gate", _vp), ("gate_bs", _i64), ("gate_rs", _i64), ("gate_ns", _i64), ("rows_per_batch", _i64),
        ("out", _vp), ("ldo", _i64), ("out_f32", C.c_int),
        ("norm", C.c_int), ("eps", C.c_float),
        ("ln_weight", _vp), ("ln_bias", _vp),
        ("shift", _vp), ("scale", _vp), ("mod_bs", _i64), ("mod_rs", _i64),
        ("nseg", C.c_int), ("seg_col0", _i64 * 2), ("seg_width", _i64), ("seg_weight", _vp * 2),
        ("rope_cos", _vp), ("rope_sin", _vp), ("rope_row_stride", _i64), ("rope_elem_stride", _i64),
        ("head_dim", _i64), ("seq_len", _i64),
        ("nout", _vp), ("ldn", _i64), ("ldp", _i64),
    ]


# name -> (restype, argtypes); every symbol declared in include/fam_hip.h
class CaeDesc(C.Structure):
    """fam_cae_desc (include/fam_hip.h)."""
    _fields_ = [
        ("z", _vp), ("batch", _i64), ("tokens", _i64), ("latent_dim", _i64),
        ("suite", _vp),
        ("hidden", _i64), ("horizon", _i64), ("action_dim", _i64), ("nstages", _i64), ("strides", _i64 * 3),
        ("in_w", _vp), ("in_b", _vp),
        ("up_w", _vp * 3), ("up_b", _vp * 3), ("gn_w", _vp * 3), ("gn_b", _vp * 3),
        ("r1_w", _vp * 3), ("r1_b", _vp * 3), ("rg1_w", _vp * 3), ("rg1_b", _vp * 3),
        ("r2_w", _vp * 3), ("r2_b", _vp * 3), ("rg2_w", _vp * 3), ("rg2_b", _vp * 3),
        ("out_w", _vp), ("out_b", _vp),
        ("work", _vp), ("out", _vp),
        ("gn_eps", C.c_float),
    ]


class TinyDesc(C.Structure):
    """fam_tiny_desc (include/fam_hip.h)."""
    _fields_ = [
        ("batch", C.c_int32), ("seq", C.c_int32), ("hidden", C.c_int32), ("heads", C.c_int32),
        ("head_dim", C.c_int32), ("ffn", C.c_int32), ("action_dim", C.c_int32), ("layers", C.c_int32),
        ("steps", C.c_int32), ("video_len", C.c_int32), ("ctx_len", C.c_int32), ("slice", C.c_int32),
        ("eps", C.c_float), ("scale", C.c_float),
        ("noise", _vp), ("mods", _vp), ("deltas", _vp),
        ("rope_cos", _vp), ("rope_sin", _vp),
        ("ctxkv", _vp), ("ctx_ld", _i64),
        ("video_k", _vp), ("video_v", _vp), ("video_bs", _i64), ("video_rs", _i64),
        ("video_mask", _vp), ("mask_rs", _i64),
        ("enc_w", _vp), ("enc_b", _vp), ("head_w", _vp), ("head_b", _vp),
        ("qkv_w", _vp), ("qkv_b", _vp), ("nq_w", _vp), ("nk_w", _vp), ("o_w", _vp), ("o_b", _vp),
        ("n3_w", _vp), ("n3_b", _vp), ("cq_w", _vp), ("cq_b", _vp), ("cnq_w", _vp),
        ("co_w", _vp), ("co_b", _vp), ("ff0_w", _vp), ("ff0_b", _vp), ("ff2_w", _vp), ("ff2_b", _vp),
        ("gram", _vp), ("gram_c", _vp), ("gram_b", _vp),
        ("lat", _vp), ("xa", _vp), ("xb", _vp), ("part_s", _vp), ("part_c", _vp), ("out", _vp),
        ("ctx_emb", _vp), ("ctx_emb_ld", _i64),
        ("ck_wt", _vp), ("ck_b", _vp), ("cnk_w", _vp), ("cv_w", _vp), ("cv_b", _vp),
        ("ctx_rs", _vp),
        ("key_splits", C.c_int32), ("part_x", _vp),
    ]


class RowQ8Desc(C.Structure):
    """fam_rowq8_desc (include/fam_hip.h)."""
    _fields_ = [
        ("mode", C.c_int), ("x", _vp), ("ldx", _i64), ("x2", _vp), ("ldx2", _i64),
        ("shift", _vp), ("scale", _vp), ("eps", C.c_float),
        ("y", _vp), ("ldy", _i64), ("s", _vp), ("xo", _vp), ("ldxo", _i64),
        ("M", _i64), ("D", _i64),
    ]


SIGNATURES = {
    "fam_version": (C.c_int, []),
    "fam_last_error": (C.c_char_p, []),
    "fam_set_launch_events": (C.c_int, [_vp, _vp]),
    "fam_adaln": (C.c_int, [_vp, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, C.c_float, _vp]),
    "fam_rmsnorm_rope": (C.c_int, [_vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, C.c_float, _vp, _vp, _i64, _i64,
                                   _i64, _vp]),
    "fam_rmsnorm_grouped": (C.c_int, [_vp, _i64, _vp, _i64, _i64, _i64, _vp, _i64, C.c_float, _vp]),
    "fam_headnorm_rope": (C.c_int, [_vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64, C.c_float,
                                    _vp, _vp, _i64, _vp]),
    "fam_act_rows": (C.c_int, [_vp, _i64, _vp, _i64, _i64, _i64, C.c_int, _vp]),
    "fam_attention": (C.c_int, [C.POINTER(AttnDesc), _vp]),
    "fam_attention_combine": (C.c_int, [C.POINTER(AttnDesc), _vp]),
    "fam_attention_key_splits": (C.c_int, [_i64, _i64, _i64, _i64, _i64]),
    "fam_attention_noalloc": (C.c_int, [C.POINTER(AttnDesc), _vp]),
    "fam_attention_noalloc_max_bytes": (_i64, []),
    "fam_gemm_partial": (C.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _vp]),
    "fam_cae_decode": (C.c_int, [C.POINTER(CaeDesc), _vp]),
    "fam_tiny_expert": (C.c_int, [C.POINTER(TinyDesc), _i64, _i64, _vp]),
    "fam_tiny_context": (C.c_int, [C.POINTER(TinyDesc), _vp]),
    "fam_tiny_key_splits": (C.c_int, [C.POINTER(TinyDesc)]),
    "fam_row_q8": (C.c_int, [C.POINTER(RowQ8Desc), _vp]),
    "fam_mask_bias": (C.c_int, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp]),
    "fam_gemm_final": (C.c_int, [_vp, _i64, _vp, _i64, _vp, C.c_int, _vp, _i64, _vp, _i64, _i64, _i64, _vp]),
    "fam_gemm_partial_splits": (C.c_int, [_i64, _i64, _i64]),
    "fam_rowop": (C.c_int, [C.POINTER(RowopDesc), _vp]),
    "fam_gemm": (C.c_int, [C.POINTER(GemmDesc), _vp]),
    "fam_linear_smallk": (C.c_int, [_vp, _i64, C.c_int, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "fam_euler_step": (C.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "fam_sinusoid": (C.c_int, [_vp, _vp, _i64, _i64, _vp]),
    "fam_add_modulation": (C.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "fam_patchify": (C.c_int, [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp]),
    "fam_unpatchify": (C.c_int, [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp]),
    "fam_gather_rows": (C.c_int, [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _vp]),
    "fam_gemm_ws": (C.c_int, [_vp, _vp, _i64, _vp]),
    "fam_gemm_ws_floats": (_i64, [_i64, _i64, _i64]),
    "fam_vae_patch_im2col": (C.c_int, [_vp, _i64, _i64, _vp, _i64, _vp]),
    "fam_im2col3x3": (C.c_int, [_vp, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _i64, _vp]),
    "fam_chan_rmsnorm": (C.c_int, [_vp, _i64, _i64, _i64, _vp, C.c_int, _vp, _i64, _vp]),
    "fam_vae_avgdown": (C.c_int, [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp]),
    "fam_softmax_rows": (C.c_int, [_vp, _i64, _i64, _i64, C.c_float, _vp, _i64, _vp]),
    "fam_chan_affine_nchw": (C.c_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
}

_lib = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Load the library once; raise with build instructions if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(
            f"{path} not found: build the HIP library first "
            "(python faster-action-models_amd/build_hip.py, or __graft_entry__.build())")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    v = lib.fam_version()
    if v != FAM_ABI_VERSION:
        raise ImportError(f"{path}: ABI version {v}, expected {FAM_ABI_VERSION}; rebuild it")
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    """Call an int-returning entry point and raise FamError on a non-zero code."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != FAM_OK:
        msg = lib.fam_last_error().decode(errors="replace")
        raise FamError(name, rc, msg)


def lib() -> C.CDLL:
    return load()
