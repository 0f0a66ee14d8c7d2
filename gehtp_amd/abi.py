"""ctypes view of the C ABI in include/oplist_parse.h, oplist_exec.h, gehtp_kernels.h.

Struct layouts here must match the C headers byte for byte; tests check the sizes
and offsets against what the library itself reports through wt_parse.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

WT_MAX_SLOTS = 4096
WT_MAX_OPS = 65536
WT_MAX_ARGS = 16
WT_EXEC_MAX_TEMPS = 4096
WT_MAX_STATES = 64
WT_BLOB_VER = 1
WT_BLOB_VER_2 = 2
WT_ENDIAN_CHK = 0x1234
WT_WEIGHT_ALIGN = 128
WT_SLOT_EXT_IN = 0xFFFFFFFF
WT_SLOT_EXT_OUT = 0xFFFFFFFE
WT_SLOT_TEMPOFF = 0xFFFFFFFD
WT_SLOT_EXT_WGT = 0xFFFFFFFC
WT_SLOT_STATE = 0xFFFFFFFB
WT_KV_POS_AUTO = 0xFFFFFFFA
WT_REF_SLOT = 0x8000
WT_REF_VTCM_FLAG = 0x4000
WT_REF_STATE_FLAG = 0x6000
WT_REF_ENG_FLAG = 0xC000

WT_ERR = {
    0: "OK", -1: "SHORT", -2: "MAGIC", -3: "VER", -4: "ENDIAN", -5: "NSLOTS", -6: "NOPS",
    -7: "SLOTS_OVERRUN", -8: "WEIGHT_OVERRUN", -9: "OP_TRUNC", -10: "OPCODE", -11: "ARITY",
    -12: "BAD_REF", -13: "ALIGN",
}


class opcodes:
    NOP = 0
    MATMUL_W4A16 = 1
    RMSNORM_F16 = 2
    PIN = 3
    SILU_F16 = 4
    IM2COL = 5
    CONV2D_F16 = 6
    ADD_F16 = 7
    SPILL = 8
    FILL = 9
    TRANSPOSE_F16 = 10
    UNARY_F16 = 11
    BINARY_F16 = 12
    SOFTMAX_F16 = 13
    CONCAT_F16 = 14
    STRIDED_SLICE_F16 = 15
    SPLIT_F16 = 16
    REDUCE_F16 = 17
    CUMSUM_F32 = 18
    CONV1D_SSM_F16 = 19
    GATHER_F16 = 20
    ARGMAX_F16 = 21
    KV_APPEND_F16 = 22
    KV_GATHER_F16 = 23
    MATMUL_F16 = 24
    RMSNORM2_F16 = 25
    BROADCAST_F16 = 26
    TRANSPOSE_GEN_F16 = 27
    SCATTER_ND_F16 = 28
    CONV1D_SSM_STEP_F16 = 29
    DELTA_CHUNK_F16 = 30
    DMA = 33
    PAD_F16 = 34
    MATMUL_F16_SPLIT = 35
    MATMUL_W4G_F16 = 40
    ATTN_F16 = 41
    ATTN_DECODE_F16 = 42
    ROPE_F16 = 43
    KV_APPEND_N_F16 = 44
    W4G_FUSED_F16 = 45
    QK_ROPE_KV_F16 = 46
    ATTN_DECODE_QKV_F16 = 47


WT_REF_NONE = 0xFFFFFFFF


# Arity table (include/oplist_parse.h); opcodes absent here are unknown to wt_parse.
ARITY = {
    0: 0, 1: 6, 2: 4, 3: 1, 4: 3, 5: 15, 6: 13, 7: 4, 8: 4, 9: 4, 10: 6, 11: 4, 12: 5, 13: 4,
    14: 16, 15: 16, 16: 16, 17: 9, 18: 7, 19: 6, 20: 15, 21: 3, 22: 4, 23: 7, 24: 7, 25: 5,
    26: 12, 27: 8, 28: 14, 29: 6, 30: 12, 33: 8, 34: 7, 35: 9,
    40: 9, 41: 10, 42: 8, 43: 8, 44: 6, 45: 11, 46: 12, 47: 10,
}


class WtSlot(C.Structure):
    _fields_ = [("len", C.c_uint32), ("count", C.c_uint32), ("offset", C.c_uint64),
                ("addr", C.c_uint32)]


class WtOp(C.Structure):
    _fields_ = [("opcode", C.c_uint16), ("n_args", C.c_uint16),
                ("args", C.c_uint32 * WT_MAX_ARGS)]


class WtBlob(C.Structure):
    _fields_ = [("ver", C.c_uint16), ("n_slots", C.c_uint32), ("n_ops", C.c_uint32),
                ("weight_off", C.c_uint32), ("slots", WtSlot * WT_MAX_SLOTS),
                ("ops", WtOp * WT_MAX_OPS), ("weight_base", C.POINTER(C.c_uint8)),
                ("weight_bytes", C.c_size_t)]


class WtExecStats(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in (
        "ops", "nop", "matmul", "rmsnorm", "silu", "pin", "pin_skipped",
        "im2col", "conv2d", "add", "spill", "fill", "transpose")]


class WtOpTs(C.Structure):
    _fields_ = [("start_us", C.c_uint32), ("dur_us", C.c_uint32), ("dma_us", C.c_uint32),
                ("dma_bytes", C.c_uint32), ("engine", C.c_uint32)]


_u8p = C.POINTER(C.c_uint8)
_vp = C.c_void_p
_u32 = C.c_uint32
_i = C.c_int

# Every function the C headers declare: name -> (restype, argtypes).
EXPORTS = {
    # oplist_parse.h
    "wt_parse": (_i, [_u8p, C.c_size_t, C.POINTER(WtBlob)]),
    "wt_err_str": (C.c_char_p, [_i]),
    # oplist_exec.h
    "wt_exec_run": (_i, [C.POINTER(WtBlob), C.POINTER(_u32), C.POINTER(C.c_int64), C.c_char_p, C.c_size_t]),
    "wt_exec_run_range": (_i, [C.POINTER(WtBlob), _u32, _u32, C.POINTER(_u32), C.POINTER(C.c_int64),
                               C.c_char_p, C.c_size_t]),
    "wt_exec_run_io": (_i, [C.POINTER(WtBlob), _vp, _vp, _u32, C.POINTER(_u32), C.POINTER(C.c_int64),
                            C.c_char_p, C.c_size_t]),
    "wt_exec_run_steps": (_i, [C.POINTER(WtBlob), _u32, _vp, _vp, _u32, C.POINTER(_u32), C.c_char_p, C.c_size_t]),
    "wt_exec_temp": (_u8p, [_u32]),
    "wt_exec_temp_bytes": (_u32, [_u32]),
    "wt_exec_temp_last_bytes": (_u32, [_u32]),
    "wt_exec_shutdown": (None, []),
    "wt_exec_state_reset": (None, []),
    "wt_exec_pool_init": (None, [_u8p, _u32, _u32, C.POINTER(_u32)]),
    "wt_exec_get_stats": (None, [C.POINTER(WtExecStats)]),
    "wt_exec_set_ext_weights": (None, [_vp]),
    "wt_exec_set_ts": (None, [C.POINTER(WtOpTs), _u32]),
    "wt_exec_set_trace": (None, [_i]),
    "wt_exec_set_hook": (None, [C.c_char_p]),
    "wt_exec_set_graphs": (_i, [_i]),
    "wt_exec_graph_stats": (None, [C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]),
    "wt_exec_set_fusion": (_i, [_i]),
    "wt_exec_set_input_device": (None, [_vp, C.c_size_t]),
    "wt_exec_fusion_stats": (None, [C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "wt_exec_fusion_detail": (None, [C.POINTER(WtBlob), C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                                     C.POINTER(C.c_uint32), C.POINTER(C.c_uint64)]),
    "wt_exec_qkv_rope_fused": (C.c_uint64, []),
    "wt_exec_qkv_attn_fused": (C.c_uint64, []),
    "wt_exec_merge_oproj_fused": (C.c_uint64, []),
    "wt_w3_report": (None, [C.c_char_p, _u8p, C.c_size_t, C.POINTER(WtBlob),
                            C.CFUNCTYPE(None, C.c_char_p, _vp), _vp]),
    # gehtp_kernels.h
    "gehtp_w4g_matmul": (_i, [_vp, _u32, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp]),
    "gehtp_w4g_gemv": (_i, [_vp, _u32, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp]),
    "gehtp_w4g_gemm": (_i, [_vp, _u32, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp]),
    "gehtp_w4g_dequant": (_i, [_vp, _vp, _vp, _u32, _u32, _vp]),
    "gehtp_w4g_fused": (_i, [_vp, _u32, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp, _vp, _u32, _u32, _vp]),
    "gehtp_w4g_split_bytes": (C.c_size_t, [_u32, _u32, _u32]),
    "gehtp_w4g_fused_ws": (_i, [_vp, _u32, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp, _vp, _u32, _u32, _vp,
                                C.c_size_t, _vp]),
    "gehtp_qk_rope_kv": (_i, [_vp, _u32, _u32, _u32, _vp, _vp, C.c_float, _vp, _vp, _vp, _vp, _u32, _vp, _vp]),
    "gehtp_matmul_f16": (_i, [_vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _vp]),
    "gehtp_rmsnorm2": (_i, [_vp, _vp, _vp, _vp, _u32, _u32, _vp]),
    "gehtp_softmax": (_i, [_vp, _vp, _u32, _u32, _vp]),
    "gehtp_attn_prefill": (_i, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, C.c_float, _i, _vp]),
    "gehtp_attn_decode": (_i, [_vp, _vp, _u32, _vp, _u32, _u32, _u32, _u32, C.c_float, _vp, _u32, _vp]),
    "gehtp_attn_decode_work_floats": (_u32, [_u32, _u32, _u32]),
    "gehtp_attn_decode_noalloc": (_i, [_vp, _vp, _u32, _vp, _u32, _u32, _u32, _u32, C.c_float, _vp]),
    "gehtp_attn_decode_qkv": (_i, [_vp, _u32, _u32, _vp, _vp, C.c_float, C.c_float, _vp, _u32, _vp, _vp, _vp,
                                   _u32, _vp]),
    "gehtp_attn_qkv_fused_work_floats": (_u32, [_u32, _u32, _u32]),
    "gehtp_qkv_attn_oproj_decode": (_i, [_vp, _vp, _vp, _vp, _u32, _vp, _u32, _u32, _vp, _vp, C.c_float, C.c_float,
                                         _vp, _u32, _vp, _vp, _vp, _vp, _vp, _u32, _vp, _vp, _u32, _vp]),
    "gehtp_qkv_attn_decode": (_i, [_vp, _vp, _vp, _vp, _u32, _vp, _u32, _u32, _vp, _vp, C.c_float, C.c_float, _vp,
                                   _u32, _vp, _vp, _vp, _u32, _vp]),
    "gehtp_kv_append": (_i, [_vp, _u32, _vp, _vp, _u32, _u32, _u32, _vp]),
    "gehtp_rope": (_i, [_vp, _vp, _u32, _u32, _u32, _u32, C.c_float, _u32, _vp]),
    "gehtp_argmax": (_i, [_vp, _u32, _vp, _vp]),
    "gehtp_crouton_encode": (_i, [_vp, _vp, _u32, _u32, _vp]),
    "gehtp_crouton_decode": (_i, [_vp, _vp, _u32, _u32, _vp]),
    "gehtp_matmul_w4a16": (_i, [_vp, _vp, _vp, _u32, _u32, _u32, _vp]),
    "gehtp_rmsnorm_crouton": (_i, [_vp, _vp, _vp, _u32, _u32, _vp]),
    "gehtp_version": (C.c_char_p, []),
}

_cache: dict = {}


def load_library(path: str | Path):
    """dlopen libgehtp.so and attach prototypes. Raises if it is missing."""
    path = Path(path)
    key = str(path)
    if key in _cache:
        return _cache[key]
    if not path.exists():
        raise FileNotFoundError(
            f"{path} is not built: run `python -m gehtp_amd.build` (there is no CPU fallback)")
    # One HIP runtime per process: PyTorch-ROCm bundles its own libamdhip64.so.7. When
    # torch is present, load it first so libgehtp's libamdhip64.so.7 dependency binds to
    # that already-loaded copy (same SONAME) and device pointers from torch tensors are
    # valid in the runtime our kernels launch through. Without torch the system ROCm
    # runtime is used.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(str(path))
    for name, (res, args) in EXPORTS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _cache[key] = lib
    return lib
