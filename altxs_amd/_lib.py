"""ctypes binding of libaltxs_hip.so (declarations mirror include/altxs.h).

The library is built in-tree by ``altxs_amd.build`` (hipcc, gfx950).  There is
no fallback: if the library is missing or fails to load, every entry point
raises :class:`AltxsLibraryError`.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libaltxs_hip.so")
ABI_VERSION = 8

MAX_LAYERS = 32
MAX_SLOTS = 64

F32, BF16, F16 = 0, 1, 2

F_SMEAR = 1 << 0
F_SPARSE_GATE = 1 << 1
F_SKIP_GATES = 1 << 2
F_ASYM_SOFTCAP = 1 << 3
F_COMMIT = 1 << 4
F_RENORM = 1 << 5
F_FINAL_ATTN = 1 << 6
F_FINAL_MLP = 1 << 7
F_FUSE_O = 1 << 8  # decode: the out-projection inside the attention launch (same bits)
CDF_RENORM = 1
ATTN_OPS_BF16 = 1
ATTN_ROWS = 2
ATTN_XCD_ROWS = 4
KV_TILE = 64
KV_F32, KV_BF16, KV_BF16_NATURAL = 0, 1, 2  # AltxsStepDesc.kv_bf16 / AltxsAttnArgs.kv_bf16
STEP_SCRATCH_BYTES = 24 << 20  # ALTXS_STEP_SCRATCH_BYTES

SLOT_SEQ, SLOT_PAR = 0, 1

EXPORTS = (
    "altxs_abi_version",
    "altxs_last_error",
    "altxs_scale_cum",
    "altxs_scale_cum_f64",
    "altxs_softmax_cdf",
    "altxs_dequant",
    "altxs_expand_codes",
    "altxs_qgemm",
    "altxs_qgemm_stream",
    "altxs_qgemv",
    "altxs_qgemv_stream",
    "altxs_rms_qgemm",
    "altxs_ffn_stage_rows",
    "altxs_attn_gate",
    "altxs_decode_attn",
    "altxs_step_workspace_bytes",
    "altxs_step_fuses_out_proj",
    "altxs_step_plan_bytes",
    "altxs_step_plan_build",
    "altxs_step",
    "altxs_step_noalloc",
    "altxs_range_init",
    "altxs_range_encode",
    "altxs_range_finish",
    "altxs_range_seed",
    "altxs_range_decode",
    "altxs_codec_decode",
    "altxs_pack_dense",
    "altxs_pack_dense32",
)


class AltxsLibraryError(RuntimeError):
    pass


class QTensor(ctypes.Structure):
    _fields_ = [("codes", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("N", ctypes.c_int64), ("K", ctypes.c_int64),
                ("bits", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("expanded", ctypes.c_void_p)]


class AttnArgs(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int32), ("W", ctypes.c_int32), ("H", ctypes.c_int32),
                ("Hkv", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("max_len", ctypes.c_int32), ("kv_bf16", ctypes.c_int32),
                ("y_bf16", ctypes.c_int32),
                ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
                ("kv_seg_stride", ctypes.c_int64), ("pos", ctypes.c_void_p),
                ("gate", ctypes.c_void_p), ("use_xsa", ctypes.c_int32),
                ("flags", ctypes.c_int32), ("kv_tail_end", ctypes.c_int32),
                ("reserved", ctypes.c_int32), ("y", ctypes.c_void_p), ("err", ctypes.c_void_p)]


class FfnStageArgs(ctypes.Structure):
    _fields_ = [("win", ctypes.c_int32), ("d", ctypes.c_int32), ("mlp", ctypes.c_int32),
                ("act_dtype", ctypes.c_int32), ("parallel", ctypes.c_int32),
                ("skip_dst", ctypes.c_int32), ("eps", ctypes.c_float), ("reserved", ctypes.c_int32),
                ("out_w", QTensor), ("up_w", QTensor), ("down_w", QTensor)] + [
                    (n, ctypes.c_void_p) for n in ("y", "hid", "a_sc", "xin", "attn_s", "src", "ln", "scr",
                                                   "m_sc", "x", "lane0", "lane1", "pr", "pp", "skips")]


class Layer(ctypes.Structure):
    _fields_ = [("qkv", QTensor), ("o", QTensor), ("up", QTensor), ("down", QTensor),
                ("resid_mix", ctypes.c_void_p), ("attn_scale", ctypes.c_void_p),
                ("mlp_scale", ctypes.c_void_p), ("q_gain", ctypes.c_void_p),
                ("attn_gate_w", ctypes.c_void_p), ("par_resid", ctypes.c_void_p),
                ("par_post", ctypes.c_void_p),
                ("ln_scale", ctypes.c_float),
                ("use_xsa", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class Slot(ctypes.Structure):
    _fields_ = [("layer", ctypes.c_int32), ("kind", ctypes.c_int32),
                ("skip_idx", ctypes.c_int32), ("skip_src", ctypes.c_int32),
                ("first_parallel", ctypes.c_int32), ("lora_scale", ctypes.c_float),
                ("lora_q_a", ctypes.c_void_p), ("lora_q_b", ctypes.c_void_p),
                ("lora_v_a", ctypes.c_void_p), ("lora_v_b", ctypes.c_void_p)]


class StepDesc(ctypes.Structure):
    _fields_ = [("abi_version", ctypes.c_int32),
                ("B", ctypes.c_int32), ("W", ctypes.c_int32), ("D", ctypes.c_int32),
                ("H", ctypes.c_int32), ("Hkv", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("F", ctypes.c_int32), ("V", ctypes.c_int32),
                ("n_layers", ctypes.c_int32), ("n_slots", ctypes.c_int32),
                ("max_len", ctypes.c_int32), ("gate_window", ctypes.c_int32),
                ("rope_dims", ctypes.c_int32), ("lora_rank", ctypes.c_int32),
                ("act_bf16", ctypes.c_int32), ("kv_bf16", ctypes.c_int32),
                ("kv_tail_end", ctypes.c_int32), ("flags", ctypes.c_int32),
                ("norm_eps", ctypes.c_float), ("gate_scale", ctypes.c_float),
                ("logit_softcap", ctypes.c_float),
                ("layers", Layer * MAX_LAYERS), ("slots", Slot * MAX_SLOTS),
                ("emb", QTensor),
                ("skip_weights", ctypes.c_void_p), ("skip_gates", ctypes.c_void_p),
                ("smear_w", ctypes.c_void_p), ("smear_lambda", ctypes.c_void_p),
                ("softcap_pn", ctypes.c_void_p), ("rope_cos", ctypes.c_void_p),
                ("rope_sin", ctypes.c_void_p),
                ("tokens", ctypes.c_void_p), ("pos", ctypes.c_void_p),
                ("prev_raw", ctypes.c_void_p), ("cand_raw", ctypes.c_void_p),
                ("kv", ctypes.c_void_p), ("ws", ctypes.c_void_p), ("ws_bytes", ctypes.c_int64),
                ("logits", ctypes.c_void_p), ("probs", ctypes.c_void_p),
                ("cum", ctypes.c_void_p), ("err", ctypes.c_void_p),
                ("attn_events", ctypes.c_void_p),
                ("aux_stream", ctypes.c_void_p), ("sync_events", ctypes.c_void_p),
                ("plan_dev", ctypes.c_void_p), ("plan_host", ctypes.c_void_p),
                ("plan_bytes", ctypes.c_int64)]


_lib = None


def load():
    """Load (once) and type the in-tree library (``LIB_PATH``, the only one this
    package loads); raise AltxsLibraryError if it is missing or unusable."""
    global _lib
    if _lib is not None:
        return _lib
    path = LIB_PATH
    if not os.path.exists(path):
        raise AltxsLibraryError(
            f"{path} not found: build it with `python -m altxs_amd.build` "
            "(hipcc --offload-arch=gfx950); there is no CPU fallback")
    try:
        L = ctypes.CDLL(path)
    except OSError as e:
        raise AltxsLibraryError(f"cannot load {path}: {e}") from e
    i32, i64, p = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p
    L.altxs_abi_version.restype = i32
    L.altxs_abi_version.argtypes = []
    L.altxs_last_error.restype = ctypes.c_char_p
    L.altxs_last_error.argtypes = []
    L.altxs_scale_cum.restype = i32
    L.altxs_scale_cum.argtypes = [p, i64, i64, p, p]
    L.altxs_scale_cum_f64.restype = i32
    L.altxs_scale_cum_f64.argtypes = [p, i64, i64, p, p]
    L.altxs_softmax_cdf.restype = i32
    L.altxs_softmax_cdf.argtypes = [p, i64, i64, i32, p, p, p]
    L.altxs_dequant.restype = i32
    L.altxs_dequant.argtypes = [ctypes.POINTER(QTensor), p, p]
    L.altxs_expand_codes.restype = i32
    L.altxs_expand_codes.argtypes = [ctypes.POINTER(QTensor), p, p]
    L.altxs_qgemm.restype = i32
    L.altxs_qgemm.argtypes = [ctypes.POINTER(QTensor), p, i32, i64, p, p]
    L.altxs_qgemm_stream.restype = i32
    L.altxs_qgemm_stream.argtypes = [ctypes.POINTER(QTensor), i64, i64, i64, p, i32, i64, p, p]
    L.altxs_qgemv.restype = i32
    L.altxs_qgemv.argtypes = [ctypes.POINTER(QTensor), p, i32, i64, p, p]
    L.altxs_qgemv_stream.restype = i32
    L.altxs_qgemv_stream.argtypes = [ctypes.POINTER(QTensor), i64, i64, i64, p, i32, i64, p, p]
    L.altxs_rms_qgemm.restype = i32
    L.altxs_rms_qgemm.argtypes = [ctypes.POINTER(QTensor), p, i64, ctypes.c_float, ctypes.c_float, i32, p, p]
    L.altxs_ffn_stage_rows.restype = i32
    L.altxs_ffn_stage_rows.argtypes = [ctypes.POINTER(FfnStageArgs), p]
    L.altxs_attn_gate.restype = i32
    L.altxs_attn_gate.argtypes = [p, i32, i64, p, i32, i32, i32, p, p]
    L.altxs_decode_attn.restype = i32
    L.altxs_decode_attn.argtypes = [ctypes.POINTER(AttnArgs), p]
    L.altxs_step_workspace_bytes.restype = i64
    L.altxs_step_workspace_bytes.argtypes = [ctypes.POINTER(StepDesc)]
    L.altxs_step_fuses_out_proj.restype = i32
    L.altxs_step_fuses_out_proj.argtypes = [ctypes.POINTER(StepDesc), i32]
    L.altxs_step_plan_bytes.restype = i64
    L.altxs_step_plan_bytes.argtypes = [ctypes.POINTER(StepDesc)]
    L.altxs_step_plan_build.restype = i32
    L.altxs_step_plan_build.argtypes = [ctypes.POINTER(StepDesc), p, p, i64, p]
    L.altxs_step.restype = i32
    L.altxs_step.argtypes = [ctypes.POINTER(StepDesc), p]
    L.altxs_step_noalloc.restype = i32
    L.altxs_step_noalloc.argtypes = [ctypes.POINTER(StepDesc), p]
    L.altxs_range_init.restype = i32
    L.altxs_range_init.argtypes = [p, i32, p]
    L.altxs_range_encode.restype = i32
    L.altxs_range_encode.argtypes = [p, i32, i32, p, p, i32, p, i64, p]
    L.altxs_range_finish.restype = i32
    L.altxs_range_finish.argtypes = [p, i32, p, i64, p]
    L.altxs_range_seed.restype = i32
    L.altxs_range_seed.argtypes = [p, i32, p, i64, p, p]
    L.altxs_range_decode.restype = i32
    L.altxs_range_decode.argtypes = [p, i32, p, i32, p, i64, p, i64, p]
    L.altxs_codec_decode.restype = i32
    L.altxs_codec_decode.argtypes = [ctypes.POINTER(CodecGroups), p, p, i64, i64, p, i64, i64, p, p]
    L.altxs_pack_dense.restype = i32
    L.altxs_pack_dense.argtypes = [p, p, i64, i64, i64, p, p]
    L.altxs_pack_dense32.restype = i32
    L.altxs_pack_dense32.argtypes = [p, p, i64, i64, i64, p, i64, p]
    v = L.altxs_abi_version()
    if v != ABI_VERSION:
        raise AltxsLibraryError(f"{path}: ABI version {v} != {ABI_VERSION}")
    _lib = L
    return L


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().altxs_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


class CoderState(ctypes.Structure):
    """AltxsCoderState (include/altxs.h): one range-coder stream."""
    _fields_ = [("low", ctypes.c_uint64), ("high", ctypes.c_uint64), ("pending", ctypes.c_uint64),
                ("value", ctypes.c_uint64), ("nbits", ctypes.c_int64), ("nbytes", ctypes.c_int64),
                ("partial", ctypes.c_uint32), ("err", ctypes.c_int32)]


CODEBOOK_MODES = {"lloyd": 0, "symmetric": 1, "shared": 2, "fp4": 3, "hybrid_fp4_symmetric": 4}


class CodecGroups(ctypes.Structure):
    """AltxsCodecGroups (include/altxs.h): the three width groups of one bank."""
    _fields_ = [("packed", ctypes.c_void_p * 3), ("codebook", ctypes.c_void_p * 3),
                ("shared", ctypes.c_void_p * 3), ("n_codes", ctypes.c_int64 * 3),
                ("n_book", ctypes.c_int64 * 3), ("mode", ctypes.c_int32), ("reserved", ctypes.c_int32)]
