"""Torch-facing operator surface over libhxmi.

The functions take device tensors (torch is only the allocator and stream
provider here) and enqueue the hand-written gfx950 kernels on torch's current
stream through the C ABI.  Names and argument meaning follow the operator
surface the hexagon-mlir tests exercise:

  matmul(a, b)                     tl.dot / linalg.matmul, C = A . B
                                   (test/python/triton/test_matmul.py:47-79)
  gemm_i8(a, b, ...)               linalg.matmul i8 x i8 -> i32 (+ dequant)
  gemv_w8a16(x, w, scale)          skinny W8A16 matmul
  softmax(x)                       torch.nn.functional.softmax(x, dim=-1)
                                   (test/python/triton/test_softmax.py:88)
  rms_norm(x, weight, eps)         torch.nn.functional.rms_norm
                                   (test/python/triton/test_rms_norm.py:82)
  layer_norm(x, weight, bias, eps) torch.nn.functional.layer_norm, optionally
                                   returning mean / rstd
                                   (test/python/triton/test_layer_norm.py:70-72)
  ResidentWeight                   registered, pre-packed weights
                                   (QHB/backend/hmx_weight_prepack.py)
  swiglu_ffn(...)                  RMSNorm -> gate/up -> SiLU*mul -> down
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _abi
from ._abi import (BF16, F16, F32, I8, I32, LAYOUT_KN, LAYOUT_NK, MemRef1D, MemRef2D, MemRef4D,
                   check, load)

_DT = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32, torch.int8: I8,
       torch.int32: I32}
_LAYOUT = {"kn": LAYOUT_KN, "nk": LAYOUT_NK}


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def _dev(t: torch.Tensor, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a tensor")
    if not t.is_cuda:
        raise ValueError(f"{name}: expected a device tensor (HIP), got {t.device}")
    return t


def memref2d(t: torch.Tensor, name: str = "tensor") -> MemRef2D:
    _dev(t, name)
    if t.dim() != 2:
        raise ValueError(f"{name}: expected 2-D, got {tuple(t.shape)}")
    m = MemRef2D()
    m.allocated = m.aligned = t.data_ptr()
    m.offset = 0
    m.sizes[0], m.sizes[1] = t.shape
    m.strides[0], m.strides[1] = t.stride()
    return m


def memref1d(t: torch.Tensor, name: str = "tensor") -> MemRef1D:
    _dev(t, name)
    if t.dim() != 1:
        raise ValueError(f"{name}: expected 1-D, got {tuple(t.shape)}")
    m = MemRef1D()
    m.allocated = m.aligned = t.data_ptr()
    m.offset = 0
    m.sizes[0] = t.shape[0]
    m.strides[0] = t.stride()[0]
    return m


def memref4d(t: torch.Tensor, name: str = "tensor") -> MemRef4D:
    _dev(t, name)
    if t.dim() != 4:
        raise ValueError(f"{name}: expected 4-D [Z, H, N, D], got {tuple(t.shape)}")
    m = MemRef4D()
    m.allocated = m.aligned = t.data_ptr()
    m.offset = 0
    for i in range(4):
        m.sizes[i] = t.shape[i]
        m.strides[i] = t.stride()[i]
    return m


def _ref(m):
    return None if m is None else ctypes.byref(m)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


# --------------------------------------------------------------------------- #
# Matmul family
# --------------------------------------------------------------------------- #

def matmul(a: torch.Tensor, b: torch.Tensor, *, b_layout: str = "kn",
           col_scale: Optional[torch.Tensor] = None, residual: Optional[torch.Tensor] = None,
           out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """C = A . B (* col_scale) (+ residual), binary32 accumulation.

    a: [M, K] f16/bf16.  b: [K, N] ("kn") or [N, K] ("nk"), same dtype as a,
    or int8 with an f16 a (W8A16).  f32 operands (with f16 / f32 partners,
    or an f32 a with an int8 b) are quantised to f16 first ((x + 0) rounded
    to nearest even), as the reference's f32 pack does.  out dtype defaults
    to a's dtype."""
    lay = _LAYOUT[b_layout]
    M = a.shape[0]
    N = b.shape[1] if lay == LAYOUT_KN else b.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype or a.dtype, device=a.device)
    ma, mb, mc = memref2d(a, "a"), memref2d(b, "b"), memref2d(out, "out")
    ms = memref1d(col_scale, "col_scale") if col_scale is not None else None
    mr = memref2d(residual, "residual") if residual is not None else None
    check(load().hx_matmul(ctypes.byref(ma), dtype_code(a), ctypes.byref(mb), dtype_code(b), lay,
                           _ref(ms), dtype_code(col_scale) if col_scale is not None else 0,
                           _ref(mr), dtype_code(residual) if residual is not None else 0,
                           ctypes.byref(mc), dtype_code(out), _stream()), "hx_matmul")
    return out


def gemm_i8(a: torch.Tensor, b: torch.Tensor, *, b_layout: str = "kn",
            row_scale: Optional[torch.Tensor] = None, col_scale: Optional[torch.Tensor] = None,
            out_dtype: torch.dtype = torch.int32, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Exact int32 C = A . B for int8 operands; with a floating out_dtype,
    RNE(((float)C * row_scale[i]) * col_scale[j])."""
    lay = _LAYOUT[b_layout]
    M = a.shape[0]
    N = b.shape[1] if lay == LAYOUT_KN else b.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    ma, mb, mc = memref2d(a, "a"), memref2d(b, "b"), memref2d(out, "out")
    mrs = memref1d(row_scale, "row_scale") if row_scale is not None else None
    mcs = memref1d(col_scale, "col_scale") if col_scale is not None else None
    check(load().hx_gemm_i8(ctypes.byref(ma), ctypes.byref(mb), lay, _ref(mrs), _ref(mcs),
                            ctypes.byref(mc), dtype_code(out), _stream()), "hx_gemm_i8")
    return out


def gemv_w8a16(x: torch.Tensor, w: torch.Tensor, scale: torch.Tensor, *, w_layout: str = "kn",
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Y = RNE_f16((X . W) * scale) with int8 W; X f16 [M, K]."""
    lay = _LAYOUT[w_layout]
    N = w.shape[1] if lay == LAYOUT_KN else w.shape[0]
    if out is None:
        out = torch.empty((x.shape[0], N), dtype=torch.float16, device=x.device)
    mx, mw, my, ms = memref2d(x, "x"), memref2d(w, "w"), memref2d(out, "out"), memref1d(scale, "scale")
    check(load().hx_gemv_w8a16(ctypes.byref(mx), ctypes.byref(mw), lay, ctypes.byref(ms),
                               dtype_code(scale), ctypes.byref(my), _stream()), "hx_gemv_w8a16")
    return out


# --------------------------------------------------------------------------- #
# Row reductions
# --------------------------------------------------------------------------- #

def softmax(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    if out is None:
        out = torch.empty_like(x)
    mx, my = memref2d(x, "x"), memref2d(out, "out")
    check(load().hx_softmax(ctypes.byref(mx), ctypes.byref(my), dtype_code(x), _stream()), "hx_softmax")
    return out


def rms_norm(x: torch.Tensor, weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    if out is None:
        out = torch.empty_like(x)
    mx, my = memref2d(x, "x"), memref2d(out, "out")
    mg = memref1d(weight, "weight") if weight is not None else None
    check(load().hx_rmsnorm(ctypes.byref(mx), _ref(mg), float(eps), ctypes.byref(my), dtype_code(x),
                            _stream()), "hx_rmsnorm")
    return out


def layer_norm(x: torch.Tensor, weight: Optional[torch.Tensor] = None,
               bias: Optional[torch.Tensor] = None, eps: float = 1e-5,
               out: Optional[torch.Tensor] = None, return_stats: bool = False):
    if out is None:
        out = torch.empty_like(x)
    mean = rstd = None
    if return_stats:
        mean = torch.empty(x.shape[0], dtype=torch.float32, device=x.device)
        rstd = torch.empty(x.shape[0], dtype=torch.float32, device=x.device)
    mx, my = memref2d(x, "x"), memref2d(out, "out")
    mw = memref1d(weight, "weight") if weight is not None else None
    mb = memref1d(bias, "bias") if bias is not None else None
    mm = memref1d(mean, "mean") if mean is not None else None
    mr = memref1d(rstd, "rstd") if rstd is not None else None
    check(load().hx_layernorm(ctypes.byref(mx), _ref(mw), _ref(mb), float(eps), ctypes.byref(my),
                              _ref(mm), _ref(mr), dtype_code(x), _stream()), "hx_layernorm")
    return (out, mean, rstd) if return_stats else out


def silu_mul(g: torch.Tensor, u: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    if out is None:
        out = torch.empty_like(g)
    mg, mu, mo = memref2d(g, "g"), memref2d(u, "u"), memref2d(out, "out")
    check(load().hx_silu_mul(ctypes.byref(mg), ctypes.byref(mu), ctypes.byref(mo), dtype_code(g),
                             _stream()), "hx_silu_mul")
    return out


# --------------------------------------------------------------------------- #
# Resident weights
# --------------------------------------------------------------------------- #

class ResidentWeight:
    """A weight registered once with the library (K-contiguous device image +
    f32 per-channel scales), keyed by content.  Mirrors the reference's
    prepacked, VTCM-resident weight (QHB/backend/hmx_weight_prepack.py:124-168,
    QHB/bin/runtime/include/HexagonCAPI.h:39-57)."""

    def __init__(self, w: torch.Tensor, scale: Optional[torch.Tensor] = None, layout: str = "kn"):
        handle = ctypes.c_void_p()
        mw = memref2d(w, "w")
        ms = memref1d(scale, "scale") if scale is not None else None
        check(load().hx_weight_register(ctypes.byref(mw), dtype_code(w), _LAYOUT[layout], _ref(ms),
                                        dtype_code(scale) if scale is not None else 0, _stream(),
                                        ctypes.byref(handle)), "hx_weight_register")
        self.handle = handle.value
        # an f32 weight is held as its f16 quantisation
        self.dtype = torch.float16 if w.dtype == torch.float32 else w.dtype

    def info(self) -> dict:
        k, n, dt, rc = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int(), ctypes.c_int()
        h = ctypes.c_uint64()
        check(load().hx_weight_info(self.handle, ctypes.byref(k), ctypes.byref(n), ctypes.byref(dt),
                                    ctypes.byref(h), ctypes.byref(rc)), "hx_weight_info")
        return {"K": k.value, "N": n.value, "dtype": dt.value, "hash": h.value, "refcount": rc.value}

    def release(self) -> None:
        if self.handle is not None:
            check(load().hx_weight_release(self.handle), "hx_weight_release")
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.release()


def matmul_resident(x: torch.Tensor, w: ResidentWeight, residual: Optional[torch.Tensor] = None,
                    out: Optional[torch.Tensor] = None,
                    out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    info_n = w.info()["N"]
    if out is None:
        out = torch.empty((x.shape[0], info_n), dtype=out_dtype or x.dtype, device=x.device)
    mx, my = memref2d(x, "x"), memref2d(out, "out")
    mr = memref2d(residual, "residual") if residual is not None else None
    check(load().hx_matmul_resident(ctypes.byref(mx), dtype_code(x), w.handle, _ref(mr),
                                    dtype_code(residual) if residual is not None else 0,
                                    ctypes.byref(my), dtype_code(out), _stream()),
          "hx_matmul_resident")
    return out


def swiglu_ffn(x: torch.Tensor, gamma: Optional[torch.Tensor], eps: float, w_gate: ResidentWeight,
               w_up: ResidentWeight, w_down: ResidentWeight,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    if out is None:
        out = torch.empty_like(x)
    mx, my = memref2d(x, "x"), memref2d(out, "out")
    mg = memref1d(gamma, "gamma") if gamma is not None else None
    check(load().hx_swiglu_ffn(ctypes.byref(mx), _ref(mg), float(eps), w_gate.handle, w_up.handle,
                               w_down.handle, ctypes.byref(my), _stream()), "hx_swiglu_ffn")
    return out


# --------------------------------------------------------------------------- #
# Kernel configurations
# --------------------------------------------------------------------------- #

def config_count(op: int) -> int:
    n = load().hx_config_count(op)
    if n < 0:
        check(n, "hx_config_count")
    return n


def config_get(op: int, index: int) -> dict:
    c = _abi.KernelConfig()
    check(load().hx_config_get(op, index, ctypes.byref(c)), "hx_config_get")
    return {"op": c.op, "index": c.index, "bm": c.bm, "bn": c.bn, "bk": c.bk,
            "waves_m": c.waves_m, "waves_n": c.waves_n, "lds_stages": c.lds_stages,
            "split_k": c.split_k, "col_tiles": c.col_tiles, "lds_bytes": c.lds_bytes,
            "name": c.name.decode()}


def config_select(op: int, m: int, n: int, k: int, index: int) -> None:
    check(load().hx_config_select(op, m, n, k, index), "hx_config_select")


def config_lookup(op: int, m: int, n: int, k: int) -> int:
    idx = ctypes.c_int()
    check(load().hx_config_lookup(op, m, n, k, ctypes.byref(idx)), "hx_config_lookup")
    return idx.value


def build_id() -> str:
    return load().hx_build_id().decode()


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: Optional[float] = None,
              causal: bool = False, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused O = softmax(Q K^T * scale) V for [Z, H, N, D] fp16/bf16 tensors
    (D = 64 or 128); the arithmetic of the reference's FlashAttention test
    (test/python/triton/test_flash_attention.py).  scale defaults to
    1/sqrt(D) like torch.nn.functional.scaled_dot_product_attention."""
    if scale is None:
        scale = q.shape[-1] ** -0.5
    if out is None:
        out = torch.empty_like(q)
    mq, mk, mv, mo = memref4d(q, "q"), memref4d(k, "k"), memref4d(v, "v"), memref4d(out, "out")
    check(load().hx_attention(ctypes.byref(mq), ctypes.byref(mk), ctypes.byref(mv), ctypes.byref(mo),
                              float(scale), 1 if causal else 0, dtype_code(q), _stream()),
          "hx_attention")
    return out


def config_pins_save() -> str:
    """The current device's pinned configs as text (see hx_config_pins_save)."""
    L = load()
    need = ctypes.c_size_t(0)
    L.hx_config_pins_save(None, 0, ctypes.byref(need))
    buf = ctypes.create_string_buffer(need.value + 1024)
    check(L.hx_config_pins_save(buf, len(buf), ctypes.byref(need)), "hx_config_pins_save")
    return buf.value.decode()


def config_pins_load(text: str) -> None:
    check(load().hx_config_pins_load(text.encode()), "hx_config_pins_load")


def manifest_enable(on: bool = True) -> bool:
    """Start (or stop) recording the plan of every matmul-family call;
    returns the previous state."""
    return bool(load().hx_manifest_enable(1 if on else 0))


def manifest_clear() -> None:
    load().hx_manifest_clear()


def manifest() -> dict:
    """The recorded plans: {"schema", "build", "records": [{entry, m, n, k,
    a, b, c, plan, config, config_source, reason, weight, calls}, ...]}."""
    import json
    L = load()
    need = ctypes.c_size_t(0)
    L.hx_manifest_json(None, 0, ctypes.byref(need))
    buf = ctypes.create_string_buffer(need.value + 4096)
    check(L.hx_manifest_json(buf, len(buf), ctypes.byref(need)), "hx_manifest_json")
    return json.loads(buf.value.decode())


def clock_probe(enable: bool) -> None:
    """Start (zeroing the counters) or stop the tiled GEMM kernels' clock
    stamps on the current device (hx_clock_probe)."""
    check(load().hx_clock_probe(1 if enable else 0), "hx_clock_probe")


def clock_read() -> dict:
    """Mean shader clock of the stamped GEMM workgroups (hx_clock_read)."""
    mhz, us, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_longlong()
    check(load().hx_clock_read(ctypes.byref(mhz), ctypes.byref(us), ctypes.byref(n)), "hx_clock_read")
    return {"mhz": mhz.value, "workgroup_us": us.value, "workgroups": n.value}


# --------------------------------------------------------------------------- #
# Pre-bound calls: descriptors built once, so a repeated call costs one C-ABI
# entry (for timing loops and serving loops; tensors must stay alive).
# --------------------------------------------------------------------------- #

class Bound:
    """A zero-argument callable around one C-ABI call with fixed arguments."""

    def __init__(self, fn, args, keep):
        self._fn, self._args, self._keep = fn, args, keep

    def __call__(self):
        rc = self._fn(*self._args)
        if rc != 0:
            check(rc, self._fn.__name__)


def bind_gemm_i8(a, b, out, *, b_layout="kn", row_scale=None, col_scale=None) -> Bound:
    ma, mb, mc = memref2d(a, "a"), memref2d(b, "b"), memref2d(out, "out")
    mrs = memref1d(row_scale, "row_scale") if row_scale is not None else None
    mcs = memref1d(col_scale, "col_scale") if col_scale is not None else None
    args = (ctypes.byref(ma), ctypes.byref(mb), _LAYOUT[b_layout], _ref(mrs), _ref(mcs),
            ctypes.byref(mc), dtype_code(out), _stream())
    return Bound(load().hx_gemm_i8, args, (ma, mb, mc, mrs, mcs, a, b, out, row_scale, col_scale))


def bind_matmul(a, b, out, *, b_layout="kn") -> Bound:
    ma, mb, mc = memref2d(a, "a"), memref2d(b, "b"), memref2d(out, "out")
    args = (ctypes.byref(ma), dtype_code(a), ctypes.byref(mb), dtype_code(b), _LAYOUT[b_layout], None, 0, None, 0,
            ctypes.byref(mc), dtype_code(out), _stream())
    return Bound(load().hx_matmul, args, (ma, mb, mc, a, b, out))


def bind_matmul_resident(x, w: ResidentWeight, out) -> Bound:
    mx, my = memref2d(x, "x"), memref2d(out, "out")
    args = (ctypes.byref(mx), dtype_code(x), w.handle, None, 0, ctypes.byref(my), dtype_code(out),
            _stream())
    return Bound(load().hx_matmul_resident, args, (mx, my, x, out, w))


def bind_row_op(op: str, x, out, weight=None, bias=None, eps: float = 1e-6) -> Bound:
    mx, my = memref2d(x, "x"), memref2d(out, "out")
    mw = memref1d(weight, "weight") if weight is not None else None
    mb = memref1d(bias, "bias") if bias is not None else None
    L = load()
    if op == "softmax":
        args, fn = (ctypes.byref(mx), ctypes.byref(my), dtype_code(x), _stream()), L.hx_softmax
    elif op == "rmsnorm":
        args, fn = (ctypes.byref(mx), _ref(mw), float(eps), ctypes.byref(my), dtype_code(x),
                    _stream()), L.hx_rmsnorm
    else:
        args, fn = (ctypes.byref(mx), _ref(mw), _ref(mb), float(eps), ctypes.byref(my), None, None,
                    dtype_code(x), _stream()), L.hx_layernorm
    return Bound(fn, args, (mx, my, mw, mb, x, out, weight, bias))
