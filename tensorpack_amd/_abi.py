"""ctypes mirror of include/mtc_hip.h (struct layout, constants, prototypes)."""

import ctypes

ABI_VERSION = 11

MTC_OK = 0
MTC_DTYPE_F32 = 0
MTC_DTYPE_BF16 = 1
MTC_FLAG_FP32_SCALES = 0x1
MTC_FLAG_MX_LAYOUT = 0x2                 # payload in the matrix-core decode layout (packer.LAYOUT_MX)
MTC_FLAG_COLS_GATHERED = 0x4             # tile stream with columns in the original order (8-word cells)

ERROR_NAMES = {
    -1: "MTC_E_NULL", -2: "MTC_E_DESC", -3: "MTC_E_SHAPE", -4: "MTC_E_DTYPE",
    -5: "MTC_E_WORKSPACE", -6: "MTC_E_LAUNCH", -7: "MTC_E_VERSION",
}

EXPORTED = ("mtc_abi_version", "mtc_last_error", "mtc_check_desc", "mtc_dequant", "mtc_gemv_lds_bytes",
            "mtc_gemv_workspace_bytes", "mtc_gemv_f32", "mtc_gemv_f32_group", "mtc_check_tile_desc", "mtc_gemm_workspace_bytes",
            "mtc_gemm_bf16", "mtc_gemm_group_workspace_bytes", "mtc_gemm_bf16_group", "mtc_gemv_batch_plan",
            "mtc_gemv_f32_batch", "mtc_gemv_noalloc_scratch_bytes", "mtc_gemv_f32_noalloc", "mtc_gemm_batch_plan",
            "mtc_gemm_bf16_batch", "mtc_gemm_f32_workspace_bytes", "mtc_gemm_f32",
            "mtc_set_prefill_decode_once")


class MtcStreamDesc(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("K", ctypes.c_int32),
        ("N", ctypes.c_int32),
        ("chunk_rows", ctypes.c_int32),
        ("n_panels", ctypes.c_int32),
        ("n_chunks", ctypes.c_int32),
        ("n_buckets", ctypes.c_int32),
        ("max_unit_words", ctypes.c_int32),
        ("max_unit_words4", ctypes.c_int32),
        ("fixed_steps", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("n_leaves", ctypes.c_int64),
        ("payload_dwords", ctypes.c_int64),
        ("payload", ctypes.c_void_p),
        ("buckets", ctypes.c_void_p),
        ("unit_hdr", ctypes.c_void_p),
        ("leaf_word", ctypes.c_void_p),
        ("leaf_scale", ctypes.c_void_p),
        ("row_perm", ctypes.c_void_p),
        ("col_perm", ctypes.c_void_p),
        ("steps", ctypes.c_void_p),
        ("n_steps", ctypes.c_int64),
    ]


DescP = ctypes.POINTER(MtcStreamDesc)


class MtcTileDesc(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("K", ctypes.c_int32),
        ("N", ctypes.c_int32),
        ("n_ksteps", ctypes.c_int32),
        ("n_col_tiles", ctypes.c_int32),
        ("payload_dwords", ctypes.c_int64),
        ("cells", ctypes.c_void_p),
        ("step_off", ctypes.c_void_p),
        ("payload", ctypes.c_void_p),
        ("row_perm", ctypes.c_void_p),
        ("col_perm", ctypes.c_void_p),
    ]


TileDescP = ctypes.POINTER(MtcTileDesc)


class MtcGemvBatchItem(ctypes.Structure):
    _fields_ = [
        ("desc", DescP),
        ("X", ctypes.c_void_p),
        ("ldx", ctypes.c_int64),
        ("Y", ctypes.c_void_p),
        ("ldy", ctypes.c_int64),
    ]


class MtcGemmBatchItem(ctypes.Structure):
    _fields_ = [
        ("desc", TileDescP),
        ("X", ctypes.c_void_p),
        ("ldx", ctypes.c_int64),
        ("Y", ctypes.c_void_p),
        ("ldy", ctypes.c_int64),
    ]


MAX_GROUP = 4                        # MTC_MAX_GROUP: matrices per mtc_gemv_f32_group launch


def declare(lib: ctypes.CDLL) -> None:
    vp, i32, i64, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
    lib.mtc_abi_version.restype = i32
    lib.mtc_abi_version.argtypes = []
    lib.mtc_last_error.restype = ctypes.c_char_p
    lib.mtc_last_error.argtypes = []
    lib.mtc_check_desc.restype = i32
    lib.mtc_check_desc.argtypes = [DescP]
    lib.mtc_dequant.restype = i32
    lib.mtc_dequant.argtypes = [DescP, vp, vp]
    lib.mtc_gemv_lds_bytes.restype = sz
    lib.mtc_gemv_lds_bytes.argtypes = [i32, i32, i32, i32]
    lib.mtc_gemv_workspace_bytes.restype = sz
    lib.mtc_gemv_workspace_bytes.argtypes = [DescP, i32]
    lib.mtc_gemv_f32.restype = i32
    lib.mtc_gemv_f32.argtypes = [DescP, vp, i64, vp, i64, i32, vp, sz, vp]
    lib.mtc_gemv_f32_group.restype = i32
    lib.mtc_gemv_f32_group.argtypes = [ctypes.POINTER(DescP), i32, vp, i64, ctypes.POINTER(vp),
                                       ctypes.POINTER(i64), i32, vp]
    lib.mtc_gemv_noalloc_scratch_bytes.restype = sz
    lib.mtc_gemv_noalloc_scratch_bytes.argtypes = []
    lib.mtc_gemv_f32_noalloc.restype = i32
    lib.mtc_gemv_f32_noalloc.argtypes = [DescP, vp, i64, vp, i64, i32, vp]
    lib.mtc_gemv_batch_plan.restype = i32
    lib.mtc_gemv_batch_plan.argtypes = [ctypes.POINTER(MtcGemvBatchItem), i32, i32, vp, sz, vp, sz,
                                        ctypes.POINTER(sz), ctypes.POINTER(sz)]
    lib.mtc_gemv_f32_batch.restype = i32
    lib.mtc_gemv_f32_batch.argtypes = [vp, vp, vp]
    lib.mtc_gemm_batch_plan.restype = i32
    lib.mtc_gemm_batch_plan.argtypes = [ctypes.POINTER(MtcGemmBatchItem), i32, i32, i32, i32, vp, sz, vp, sz,
                                        ctypes.POINTER(sz), ctypes.POINTER(sz)]
    lib.mtc_gemm_bf16_batch.restype = i32
    lib.mtc_gemm_bf16_batch.argtypes = [vp, vp, vp]
    lib.mtc_check_tile_desc.restype = i32
    lib.mtc_check_tile_desc.argtypes = [TileDescP]
    lib.mtc_gemm_workspace_bytes.restype = sz
    lib.mtc_gemm_workspace_bytes.argtypes = [TileDescP, i32, i32]
    lib.mtc_gemm_bf16.restype = i32
    lib.mtc_gemm_bf16.argtypes = [TileDescP, vp, i32, i64, vp, i32, i64, i32, vp, sz, vp]
    lib.mtc_gemm_f32_workspace_bytes.restype = sz
    lib.mtc_gemm_f32_workspace_bytes.argtypes = [TileDescP, i32]
    lib.mtc_set_prefill_decode_once.restype = i32
    lib.mtc_set_prefill_decode_once.argtypes = [i32]
    lib.mtc_gemm_f32.restype = i32
    lib.mtc_gemm_f32.argtypes = [TileDescP, vp, i64, vp, i64, i32, vp, sz, vp]
    lib.mtc_gemm_group_workspace_bytes.restype = sz
    lib.mtc_gemm_group_workspace_bytes.argtypes = [ctypes.POINTER(TileDescP), i32, i32, i32]
    lib.mtc_gemm_bf16_group.restype = i32
    lib.mtc_gemm_bf16_group.argtypes = [ctypes.POINTER(TileDescP), i32, vp, i32, i64, ctypes.POINTER(vp), i32,
                                        ctypes.POINTER(i64), i32, vp, sz, vp]


class MtcError(RuntimeError):
    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with {ERROR_NAMES.get(code, code)}: {msg}")
        self.code = code


def check(lib: ctypes.CDLL, fn: str, code: int) -> None:
    if code != MTC_OK:
        raise MtcError(fn, code, (lib.mtc_last_error() or b"").decode(errors="replace"))
