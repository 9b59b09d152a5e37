"""ctypes binding of libhxmi.so (the C ABI in include/hx.h).

Loading fails loudly when the library has not been built: there is no CPU or
eager fallback behind these entry points.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libhxmi.so"

# dtype / layout / status / family codes -- mirror include/hx.h
F16, BF16, F32, I8, I32 = 1, 2, 3, 4, 5
LAYOUT_KN, LAYOUT_NK = 0, 1
OK = 0
ERRORS = {
    -1: "HX_ERR_ARG", -2: "HX_ERR_SHAPE", -3: "HX_ERR_DTYPE", -4: "HX_ERR_LAYOUT",
    -5: "HX_ERR_HIP", -6: "HX_ERR_NOMEM", -7: "HX_ERR_UNSUPPORTED", -8: "HX_ERR_HANDLE",
    -9: "HX_ERR_NODEVICE",
}
OP_GEMM_I8, OP_MATMUL_F16, OP_MATMUL_BF16, OP_MATMUL_W8, OP_SWIGLU_W8, OP_GEMV_W8 = 1, 2, 3, 4, 5, 6
OP_GEMV_F16, OP_GEMV_BF16 = 7, 8
OP_SOFTMAX, OP_RMSNORM, OP_LAYERNORM = 9, 10, 11  # row families: (m, n, k) = (rows, cols, dtype)
OP_NAMES = {OP_GEMM_I8: "gemm_i8", OP_MATMUL_F16: "matmul_f16", OP_MATMUL_BF16: "matmul_bf16",
            OP_MATMUL_W8: "matmul_w8", OP_SWIGLU_W8: "swiglu_w8", OP_GEMV_W8: "gemv_w8",
            OP_GEMV_F16: "gemv_f16", OP_GEMV_BF16: "gemv_bf16", OP_SOFTMAX: "softmax",
            OP_RMSNORM: "rmsnorm", OP_LAYERNORM: "layernorm"}


class MemRef2D(ctypes.Structure):
    _fields_ = [("allocated", ctypes.c_void_p), ("aligned", ctypes.c_void_p),
                ("offset", ctypes.c_int64), ("sizes", ctypes.c_int64 * 2),
                ("strides", ctypes.c_int64 * 2)]


class MemRef4D(ctypes.Structure):
    _fields_ = [("allocated", ctypes.c_void_p), ("aligned", ctypes.c_void_p),
                ("offset", ctypes.c_int64), ("sizes", ctypes.c_int64 * 4),
                ("strides", ctypes.c_int64 * 4)]


class MemRef1D(ctypes.Structure):
    _fields_ = [("allocated", ctypes.c_void_p), ("aligned", ctypes.c_void_p),
                ("offset", ctypes.c_int64), ("sizes", ctypes.c_int64 * 1),
                ("strides", ctypes.c_int64 * 1)]


class KernelConfig(ctypes.Structure):
    _fields_ = [("op", ctypes.c_int32), ("index", ctypes.c_int32), ("bm", ctypes.c_int32),
                ("bn", ctypes.c_int32), ("bk", ctypes.c_int32), ("waves_m", ctypes.c_int32),
                ("waves_n", ctypes.c_int32), ("lds_stages", ctypes.c_int32),
                ("split_k", ctypes.c_int32), ("col_tiles", ctypes.c_int32),
                ("lds_bytes", ctypes.c_int32), ("name", ctypes.c_char * 40)]


class TuneOptions(ctypes.Structure):
    _fields_ = [("reps", ctypes.c_int32), ("min_iters", ctypes.c_int32), ("max_iters", ctypes.c_int32),
                ("budget_us", ctypes.c_double), ("canary_reference_us", ctypes.c_double),
                ("pin", ctypes.c_int32), ("seed", ctypes.c_uint64)]


class TuneEntry(ctypes.Structure):
    _fields_ = [("index", ctypes.c_int32), ("status", ctypes.c_int32), ("q50_us", ctypes.c_double),
                ("q20_us", ctypes.c_double), ("q80_us", ctypes.c_double), ("reason", ctypes.c_char * 24)]


TUNE_MAX_ENTRIES = 64


class TuneReport(ctypes.Structure):
    _fields_ = [("op", ctypes.c_int32), ("m", ctypes.c_int64), ("n", ctypes.c_int64), ("k", ctypes.c_int64),
                ("iters", ctypes.c_int32), ("control_index", ctypes.c_int32), ("best_index", ctypes.c_int32),
                ("champion_index", ctypes.c_int32), ("control_q50_us", ctypes.c_double),
                ("best_q50_us", ctypes.c_double), ("margin", ctypes.c_double), ("gate", ctypes.c_double),
                ("canary_index", ctypes.c_int32), ("canary_m", ctypes.c_int64), ("canary_n", ctypes.c_int64),
                ("canary_k", ctypes.c_int64), ("canary_status", ctypes.c_int32),
                ("canary_q50_us", ctypes.c_double), ("canary_reference_us", ctypes.c_double),
                ("canary_shift", ctypes.c_double), ("canary_gate", ctypes.c_double),
                ("round_valid", ctypes.c_int32), ("pinned", ctypes.c_int32), ("n_entries", ctypes.c_int32),
                ("entries", TuneEntry * TUNE_MAX_ENTRIES)]


TUNE_TIMED, TUNE_REFUSED, TUNE_LAUNCH_FAILED, TUNE_WRONG = 0, 1, 2, 3
TUNE_STATUS = {0: "timed", 1: "refused", 2: "launch-failed", 3: "wrong"}
CANARY_BASELINE, CANARY_STEADY, CANARY_DRIFT, CANARY_FAILED = 0, 1, 2, 3
CANARY_STATUS = {0: "baseline", 1: "steady", 2: "drift", 3: "failed"}


class HXError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{ERRORS.get(code, code)}: {message}")
        self.code = code


_P2 = ctypes.POINTER(MemRef2D)
_P1 = ctypes.POINTER(MemRef1D)
_vp, _i, _i64, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float

SIGNATURES = {
    "hx_init": ([], _i),
    "hx_last_error": ([], ctypes.c_char_p),
    "hx_build_id": ([], ctypes.c_char_p),
    "hx_matmul": ([_P2, _i, _P2, _i, _i, _P1, _i, _P2, _i, _P2, _i, _vp], _i),
    "hx_gemm_i8": ([_P2, _P2, _i, _P1, _P1, _P2, _i, _vp], _i),
    "hx_gemv_w8a16": ([_P2, _P2, _i, _P1, _i, _P2, _vp], _i),
    "hx_softmax": ([_P2, _P2, _i, _vp], _i),
    "hx_rmsnorm": ([_P2, _P1, _f, _P2, _i, _vp], _i),
    "hx_layernorm": ([_P2, _P1, _P1, _f, _P2, _P1, _P1, _i, _vp], _i),
    "hx_silu_mul": ([_P2, _P2, _P2, _i, _vp], _i),
    "hx_weight_register": ([_P2, _i, _i, _P1, _i, _vp, ctypes.POINTER(_vp)], _i),
    "hx_weight_release": ([_vp], _i),
    "hx_weight_info": ([_vp, ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i),
                        ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(_i)], _i),
    "hx_matmul_resident": ([_P2, _i, _vp, _P2, _i, _P2, _i, _vp], _i),
    "hx_swiglu_ffn": ([_P2, _P1, _f, _vp, _vp, _vp, _P2, _vp], _i),
    "hx_swiglu_ffn_noalloc": ([_P2, _P1, _f, _vp, _vp, _vp, _P2, _vp], _i),
    "hx_config_count": ([_i], _i),
    "hx_config_get": ([_i, _i, ctypes.POINTER(KernelConfig)], _i),
    "hx_config_select": ([_i, _i64, _i64, _i64, _i], _i),
    "hx_config_lookup": ([_i, _i64, _i64, _i64, ctypes.POINTER(_i)], _i),
    "hx_config_pins_save": ([ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)], _i),
    "hx_config_pins_load": ([ctypes.c_char_p], _i),
    "hx_attention": ([ctypes.POINTER(MemRef4D)] * 4 + [_f, _i, _i, _vp], _i),
    "hx_tune": ([_i, _i64, _i64, _i64, ctypes.POINTER(TuneOptions), ctypes.POINTER(TuneReport), _vp], _i),
    "hx_tune_decide": ([ctypes.POINTER(TuneEntry), _i, _i, ctypes.POINTER(TuneEntry), ctypes.c_double,
                        ctypes.POINTER(TuneReport)], _i),
    "hx_manifest_enable": ([_i], _i),
    "hx_manifest_clear": ([], _i),
    "hx_manifest_json": ([ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)], _i),
    "hx_clock_probe": ([_i], _i),
    "hx_clock_read": ([ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                       ctypes.POINTER(ctypes.c_longlong)], _i),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libhxmi.so, raising ImportError if it was never built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                              "(hexagon-mlir_amd/build.py); there is no fallback path")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def last_error() -> str:
    msg = load().hx_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc != OK:
        raise HXError(rc, f"{what}: {last_error()}")
