"""CPU oracle for the hx hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in plain C (``hx_oracle.c``), the linalg semantics the
Hexagon-MLIR backend lowers for matmul / softmax / RMSNorm / LayerNorm, and
wraps it for numpy.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or
as the timed CPU port.  The product library never links or calls it.

Pinning (every function is checked by ``tests/test_oracle.py``):

=====================  ======================================================
function               pinned by
=====================  ======================================================
f32<->f16 / bf16       numpy ``astype(float16)`` and torch-CPU ``bfloat16``
                       (both IEEE RNE) on edge classes + 2^20 random values
gemm_i8_i32            numpy int64 matmul (exact), brute force on 5x7x3,
                       identity, all-(+-127) closed form, K=1 outer product
dequant_i32_f16        numpy binary32 products + ``astype(float16)``, bitwise
matmul (f16/bf16/i8)   numpy float64 matmul within the binary32 accumulation
                       bound; identity B reproduces A exactly; residual and
                       scale each checked by a dropped-term negative control;
                       scale and residual together against float64
                       (A.B).s + R, the swapped order (A.B + R).s failing;
                       the column-split form bit-equal to the row form
softmax                numpy float64; rows sum to 1; shift invariance;
                       torch-CPU softmax at the reference test's shape/atol
rmsnorm                numpy float64; scale invariance; torch-CPU rms_norm at
                       the reference test's shape/atol
layernorm              numpy float64 incl. mean/rstd; torch-CPU layer_norm at
                       the reference test's shape/atol
silu_mul               numpy float64
attention              numpy float64 softmax(QK^T s)V; V = 1 gives 1;
                       one key returns its value row; causal row 0 is v[0];
                       torch-CPU scaled_dot_product_attention at the reference
                       test's shape and relative-error bound
swiglu_ffn             an independent float64 composition (numpy matmuls, no
                       fp16 stages) within the bound of five fp16 roundings;
                       negative controls: gate/up swapped, per-channel scales
                       on the wrong channels, gamma dropped, silu on the up
                       branch; row independence (a row subset is bit-equal)
=====================  ======================================================
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "hx_oracle.c"
LIB = HERE / "liboracle.so"

F16, BF16, F32, I8, I32 = 1, 2, 3, 4, 5

_lib = None


def build(force: bool = True) -> Path:
    """Compile the C restatement into ``oracle/liboracle.so`` with gcc.

    x86-64-v3 (AVX2/FMA) is the floor of every EPYC host an MI355X sits in;
    -ffp-contract=off keeps each multiply and add separately rounded."""
    if LIB.exists() and not force:
        return LIB
    tmp = LIB.with_suffix(".so.tmp")
    cmd = ["gcc", "-O3", "-march=x86-64-v3", "-fopenmp", "-ffp-contract=off",
           "-fno-math-errno", "-fPIC", "-shared", str(SRC), "-o", str(tmp), "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


def use_native_build() -> str:
    """Compile the C restatement for the host it runs on (-march=native,
    the CPU baseline's build) into a temporary directory and make it the
    library every function below calls.  The in-tree build targets
    x86-64-v3 so that it loads on any x86 host; this one uses every vector
    extension the host has.  Returns the -march flags gcc resolved."""
    global _lib
    import tempfile
    d = Path(tempfile.mkdtemp(prefix="hx_oracle_native_"))
    out = d / "liboracle_native.so"
    r = subprocess.run(["gcc", "-march=native", "-Q", "--help=target"], capture_output=True, text=True)
    enabled = {ln.split()[0] for ln in r.stdout.splitlines() if ln.strip().endswith("[enabled]")}
    march = next((ln.split()[-1] for ln in r.stdout.splitlines() if ln.strip().startswith("-march=")), "native")
    # an older gcc that does not know the host's core model resolves
    # -march=native to an older one without its AVX-512: add what the CPU
    # reports (the extensions gcc 11 can target)
    try:
        cpu = set(open("/proc/cpuinfo").read().split())
    except OSError:
        cpu = set()
    extra = [f"-m{f}" for f in ("avx512f", "avx512bw", "avx512dq", "avx512vl", "avx512cd", "avx512vnni")
             if f in cpu and f"-m{f}" not in enabled]
    subprocess.run(["gcc", "-O3", "-march=native", *extra, "-fopenmp", "-ffp-contract=off", "-fno-math-errno",
                    "-fPIC", "-shared", str(SRC), "-o", str(out), "-lm"], check=True)
    _lib = None
    _bind(ctypes.CDLL(str(out)))
    return march + ("" if not extra else " " + " ".join(extra))


def lib():
    if _lib is None:
        if not LIB.exists():
            build()
        _bind(ctypes.CDLL(str(LIB)))
    return _lib


def _bind(L):
    """Declare the C signatures on a loaded copy and make it the active one."""
    global _lib
    if True:  # noqa: SIM108 -- one block of declarations
        vp, i64, i32, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        L.hxo_f32_to_f16_array.argtypes = [vp, vp, i64]
        L.hxo_f16_to_f32_array.argtypes = [vp, vp, i64]
        L.hxo_f32_to_bf16_array.argtypes = [vp, vp, i64]
        L.hxo_gemm_i8_i32.argtypes = [vp, i64, vp, i64, i32, vp, i64, i64, i64, i64]
        L.hxo_dequant_i32_f16.argtypes = [vp, i64, vp, vp, vp, i64, i64, i64]
        L.hxo_matmul.argtypes = [vp, i32, i64, vp, i32, i64, i32, vp, vp, i32, i64,
                                 vp, i32, i64, i64, i64, i64]
        L.hxo_matmul_ncols.argtypes = L.hxo_matmul.argtypes
        L.hxo_softmax.argtypes = [vp, vp, i32, i64, i64, i64, i64]
        L.hxo_rmsnorm.argtypes = [vp, vp, f32, vp, i32, i64, i64, i64, i64]
        L.hxo_layernorm.argtypes = [vp, vp, vp, f32, vp, vp, vp, i32, i64, i64, i64, i64]
        L.hxo_silu_mul.argtypes = [vp, vp, vp, i32, i64, i64, i64, i64, i64]
        L.hxo_attention.argtypes = [vp, vp, vp, vp, i32, i64, i64, i64, i64, f32, i32]
        _lib = L


# --------------------------------------------------------------------------- #
# dtype plumbing: fp16 lives in numpy float16; bf16 travels as uint16 bits.
# --------------------------------------------------------------------------- #

def _code(a: np.ndarray, bf16: bool = False) -> int:
    if bf16:
        assert a.dtype == np.uint16
        return BF16
    return {np.dtype(np.float16): F16, np.dtype(np.float32): F32,
            np.dtype(np.int8): I8, np.dtype(np.int32): I32}[a.dtype]


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _rowmajor(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    return a


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().hxo_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().hxo_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().hxo_f32_to_bf16_array(_p(x), _p(out), x.size)
    return out


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# --------------------------------------------------------------------------- #
# Operators
# --------------------------------------------------------------------------- #

def gemm_i8_i32(a: np.ndarray, b: np.ndarray, b_trans: bool = False) -> np.ndarray:
    """Exact int32 C = A.B for int8 A [M,K] and B [K,N] (or [N,K] if b_trans)."""
    a, b = _rowmajor(a), _rowmajor(b)
    assert a.dtype == np.int8 and b.dtype == np.int8
    M, K = a.shape
    N = b.shape[0] if b_trans else b.shape[1]
    assert (b.shape[1] if b_trans else b.shape[0]) == K
    c = np.empty((M, N), np.int32)
    lib().hxo_gemm_i8_i32(_p(a), K, _p(b), b.shape[1], int(b_trans), _p(c), N, M, N, K)
    return c


def dequant_i32_f16(c: np.ndarray, sa=None, sb=None) -> np.ndarray:
    c = _rowmajor(c).astype(np.int32, copy=False)
    M, N = c.shape
    sa = None if sa is None else np.ascontiguousarray(sa, np.float32)
    sb = None if sb is None else np.ascontiguousarray(sb, np.float32)
    out = np.empty((M, N), np.uint16)
    lib().hxo_dequant_i32_f16(_p(c), N, _p(sa), _p(sb), _p(out), N, M, N)
    return out.view(np.float16)


def matmul(a, b, *, b_trans=False, scale_n=None, residual=None, out_dtype=np.float16,
           a_bf16=False, b_bf16=False, r_bf16=False, out_bf16=False, split_cols=False) -> np.ndarray:
    """out = round(acc * scale_n + residual), acc in binary32 (i,k,j) order.

    fp16 arrays are numpy float16; bf16 arrays are passed as uint16 bit
    patterns with the matching ``*_bf16`` flag.  ``split_cols`` spreads the
    host threads over output columns instead of rows (few-row products);
    the result is bit-identical."""
    a, b = _rowmajor(a), _rowmajor(b)
    M, K = a.shape
    N = b.shape[0] if b_trans else b.shape[1]
    sc = None if scale_n is None else np.ascontiguousarray(scale_n, np.float32)
    r = None if residual is None else _rowmajor(residual)
    if out_bf16:
        out, ocode = np.empty((M, N), np.uint16), BF16
    else:
        out = np.empty((M, N), np.dtype(out_dtype))
        ocode = _code(out)
    fn = lib().hxo_matmul_ncols if split_cols else lib().hxo_matmul
    fn(_p(a), _code(a, a_bf16), K, _p(b), _code(b, b_bf16), b.shape[1],
       int(b_trans), _p(sc), _p(r), 0 if r is None else _code(r, r_bf16),
       0 if r is None else r.shape[1], _p(out), ocode, N, M, N, K)
    return out


def softmax(x: np.ndarray, bf16: bool = False) -> np.ndarray:
    x = _rowmajor(x)
    R, C = x.shape
    y = np.empty_like(x)
    lib().hxo_softmax(_p(x), _p(y), _code(x, bf16), R, C, C, C)
    return y


def rmsnorm(x: np.ndarray, gamma=None, eps: float = 1e-6, bf16: bool = False) -> np.ndarray:
    x = _rowmajor(x)
    R, C = x.shape
    g = None if gamma is None else _rowmajor(gamma)
    y = np.empty_like(x)
    lib().hxo_rmsnorm(_p(x), _p(g), eps, _p(y), _code(x, bf16), R, C, C, C)
    return y


def layernorm(x, w=None, b=None, eps: float = 1e-5, bf16: bool = False):
    x = _rowmajor(x)
    R, C = x.shape
    w = None if w is None else _rowmajor(w)
    b = None if b is None else _rowmajor(b)
    y = np.empty_like(x)
    mean = np.empty(R, np.float32)
    rstd = np.empty(R, np.float32)
    lib().hxo_layernorm(_p(x), _p(w), _p(b), eps, _p(y), _p(mean), _p(rstd),
                        _code(x, bf16), R, C, C, C)
    return y, mean, rstd


def silu_mul(g: np.ndarray, u: np.ndarray, bf16: bool = False) -> np.ndarray:
    g, u = _rowmajor(g), _rowmajor(u)
    R, C = g.shape
    out = np.empty_like(g)
    lib().hxo_silu_mul(_p(g), _p(u), _p(out), _code(g, bf16), R, C, C, C, C)
    return out


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, causal: bool = False,
              bf16: bool = False) -> np.ndarray:
    """O = softmax(Q K^T * scale) V over [..., N, D] arrays (fp16, or bf16
    bits as uint16 with ``bf16``); binary32 throughout, one rounding of O."""
    q, k, v = _rowmajor(q), _rowmajor(k), _rowmajor(v)
    lead = q.shape[:-2]
    Nq, D = q.shape[-2:]
    Nk = k.shape[-2]
    if Nk > 16384:
        raise ValueError("oracle attention: Nk <= 16384")
    B = int(np.prod(lead)) if lead else 1
    out = np.empty_like(q)
    lib().hxo_attention(_p(q), _p(k), _p(v), _p(out), _code(q, bf16), B, Nq, Nk, D,
                        ctypes.c_float(scale), 1 if causal else 0)
    return out


def swiglu_ffn(x, gamma, eps, wg, sg, wu, su, wd, sd):
    """RMSNorm -> gate/up W8A16 GEMMs (per-channel scales) -> SiLU*mul -> down.

    The composition of BASELINE config C5; each stage rounds to fp16 as a
    separate linalg op would.  Weights are int8 in the linalg [K, N]
    orientation, scales per output channel."""
    h = rmsnorm(x, gamma, eps)
    g = matmul(h, wg, scale_n=sg.astype(np.float32))
    u = matmul(h, wu, scale_n=su.astype(np.float32))
    a = silu_mul(g, u)
    return matmul(a, wd, scale_n=sd.astype(np.float32))
