"""ctypes binding of the C-ABI in include/flaxchat_amd.h.

The structures below mirror the header field for field. `lib()` loads the
in-tree `libflaxchat_amd.so` and raises if it is missing: there is no
fallback path.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, Structure, c_float, c_int32, c_int64, c_uint64, c_void_p, c_char_p

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libflaxchat_amd.so")

FC_F32, FC_BF16 = 0, 1
EPI_STORE, EPI_ADD, EPI_RELU2, EPI_SOFTCAP = 0, 1, 2, 4
RES_STRIDE = 40
PMAX = 16  # FC_PMAX: pending tokens per row and model


class FcLayer(Structure):
    _fields_ = [("wqkv", c_void_p), ("wo", c_void_p), ("wfc", c_void_p), ("wproj", c_void_p),
                ("ve", c_void_p), ("ve_gate", c_void_p), ("window", c_int32),
                ("resid_lambda", c_float), ("x0_lambda", c_float)]


class FcModel(Structure):
    _fields_ = [("n_layer", c_int32), ("n_embd", c_int32), ("n_head", c_int32), ("n_kv_head", c_int32),
                ("head_dim", c_int32), ("vocab", c_int32), ("vocab_pad", c_int32), ("dtype", c_int32),
                ("wte", c_void_p), ("lm_head", c_void_p), ("smear_gate", c_void_p),
                ("smear_lambda", c_float), ("backout_lambda", c_float),
                ("rope_cos", c_void_p), ("rope_sin", c_void_p), ("rope_len", c_int32),
                ("layers", POINTER(FcLayer))]


class FcCache(Structure):
    _fields_ = [("k", c_void_p), ("v", c_void_p), ("hist", c_void_p), ("batch", c_int32), ("cap", c_int32)]


FC_CHUNK_FULL_SMEAR = 1  # fc_chunk.flags: the full-sequence forward's smear


class FcChunk(Structure):
    _fields_ = [("max_tokens", c_int32), ("max_per_row", c_int32), ("typ_tokens", c_int32),
                ("tokens", c_void_p), ("row_off", c_void_p), ("start", c_void_p),
                ("n_out", c_int32), ("logits", c_void_p), ("logits_stride", c_int64), ("flags", c_int32)]


class FcRowstat(Structure):
    _fields_ = [("mx", c_float), ("sum", c_float), ("tau", c_float), ("tie_idx", c_int32),
                ("argmax", c_int32), ("pad", c_int32 * 3)]


_SPEC_PTRS = ["t_len", "d_len", "t_pend", "d_pend", "t_pend_n", "d_pend_n", "t_dirty", "d_dirty",
              "gen", "gen_n", "prompt_len", "round", "stall", "result",
              "tok_d0", "off_d0", "start_d", "tok_ds", "off_ds", "tok_v", "off_v", "start_v", "drafts",
              "q_logits", "p_logits", "q_stats", "p_stats"]


class FcSpecState(Structure):
    _fields_ = ([("batch", c_int32), ("k", c_int32), ("max_tokens", c_int32), ("gen_cap", c_int32),
                 ("vocab", c_int32), ("temperature", c_float), ("top_k", c_int32), ("seed", c_uint64)]
                + [(n, c_void_p) for n in _SPEC_PTRS] + [("part", c_void_p), ("part_bytes", c_int64)])


EXPORTS = ["fc_last_error", "fc_version", "fc_forward_workspace_bytes", "fc_forward", "fc_gemm", "fc_pack_operand",
           "fc_attention_workspace_bytes", "fc_attention", "fc_attention_noalloc", "fc_attention_noalloc_max_bytes",
           "fc_attn_prologue", "fc_attn_qkv_workspace_bytes", "fc_attn_qkv", "fc_row_stats", "fc_spec_workspace_bytes",
           "fc_spec_round", "fc_spec_accept", "fc_spec_part_bytes", "fc_fast_sample", "fc_engine_sample",
           "fc_cross_entropy", "fc_read_probe", "fc_l2_read_probe", "fc_walk_probe", "fc_gemm_walk_probe",
           "fc_gemm_walk_probe_words", "fc_graph_begin", "fc_graph_end", "fc_graph_launch", "fc_graph_destroy"]

_lib = None


def _declare(L):
    vp, i32, i64, f32 = c_void_p, c_int32, c_int64, c_float
    L.fc_last_error.restype = c_char_p
    L.fc_version.restype = i32
    L.fc_forward_workspace_bytes.argtypes = [POINTER(FcModel), i32, i32, i32, i32]
    L.fc_forward_workspace_bytes.restype = i64
    L.fc_forward.argtypes = [POINTER(FcModel), POINTER(FcCache), POINTER(FcChunk), vp, i64, vp]
    L.fc_forward.restype = i32
    L.fc_gemm.argtypes = [vp, vp, vp, i32, i32, i32, i32, i32, vp]
    L.fc_gemm.restype = i32
    L.fc_pack_operand.argtypes = [vp, vp, i32, i32, vp]
    L.fc_pack_operand.restype = i32
    L.fc_attention_workspace_bytes.argtypes = [i32, i32, i32, i32, i32, i32]
    L.fc_attention_workspace_bytes.restype = i64
    L.fc_attn_prologue.argtypes = [POINTER(FcModel), i32, POINTER(FcCache), vp, vp, vp, vp, vp, i32, vp, vp]
    L.fc_attention.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp, vp, i32, i32, i32, vp, i64,
                               vp]
    L.fc_attn_qkv_workspace_bytes.argtypes = [POINTER(FcModel), i32, i32]
    L.fc_attn_qkv_workspace_bytes.restype = i64
    L.fc_attn_qkv.argtypes = [POINTER(FcModel), i32, POINTER(FcCache), vp, vp, vp, vp, i32, i32, vp, vp, i64, vp]
    L.fc_attn_qkv.restype = i32
    L.fc_attention_noalloc.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp, vp, i32, i32, i32, vp]
    L.fc_attention_noalloc.restype = i32
    L.fc_attention_noalloc_max_bytes.argtypes = []
    L.fc_attention_noalloc_max_bytes.restype = i64
    L.fc_spec_workspace_bytes.argtypes = [POINTER(FcModel), POINTER(FcModel), i32, i32]
    L.fc_spec_workspace_bytes.restype = i64
    L.fc_attention.restype = i32
    L.fc_row_stats.argtypes = [vp, i32, i32, f32, i32, vp, vp]
    L.fc_row_stats.restype = i32
    L.fc_spec_round.argtypes = [POINTER(FcModel), POINTER(FcCache), POINTER(FcModel), POINTER(FcCache),
                                POINTER(FcSpecState), vp, i64, vp]
    L.fc_spec_round.restype = i32
    L.fc_spec_accept.argtypes = [POINTER(FcSpecState), vp]
    L.fc_spec_accept.restype = i32
    L.fc_spec_part_bytes.argtypes = [i32, i32, i32]
    L.fc_spec_part_bytes.restype = i64
    L.fc_fast_sample.argtypes = [vp, i32, i32, f32, i32, c_uint64, i32, vp, i32, vp, vp, vp, vp, vp, vp, vp]
    L.fc_fast_sample.restype = i32
    L.fc_engine_sample.argtypes = [vp, i32, i32, f32, i32, c_uint64, vp, vp, i32, vp, vp, vp, vp, vp]
    L.fc_engine_sample.restype = i32
    L.fc_cross_entropy.argtypes = [vp, i64, vp, i32, i32, vp, vp]
    L.fc_cross_entropy.restype = i32
    L.fc_read_probe.argtypes = [vp, i64, vp, i32, vp]
    L.fc_read_probe.restype = i32
    L.fc_l2_read_probe.argtypes = [vp, i64, i64, vp, i32, vp]
    L.fc_l2_read_probe.restype = i32
    L.fc_walk_probe.argtypes = [vp, i32, i32, vp, vp]
    L.fc_walk_probe.restype = i32
    L.fc_gemm_walk_probe.argtypes = [vp, vp, i32, i32, i32, i32, i32, i32, i32, vp, vp]
    L.fc_gemm_walk_probe.restype = i32
    L.fc_gemm_walk_probe_words.argtypes = [i32, i32, i32, i32, i32]
    L.fc_gemm_walk_probe_words.restype = i32
    L.fc_graph_begin.argtypes = [vp]
    L.fc_graph_begin.restype = i32
    L.fc_graph_end.argtypes = [vp, POINTER(c_void_p)]
    L.fc_graph_end.restype = i32
    L.fc_graph_launch.argtypes = [vp, vp]
    L.fc_graph_launch.restype = i32
    L.fc_graph_destroy.argtypes = [vp]
    L.fc_graph_destroy.restype = i32


def lib():
    """The loaded HIP library. Raises RuntimeError when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"flaxchat_amd HIP library missing at {LIB_PATH}; "
                               "build it with `python -m flaxchat_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        _declare(L)
        _lib = L
    return _lib


def check(rc: int, what: str = "fc call"):
    if rc != 0:
        msg = lib().fc_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")
