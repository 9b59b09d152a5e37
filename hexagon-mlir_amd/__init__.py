"""hexagon-mlir_amd -- MI355X (gfx950) implementation of the hexagon-mlir hot
path: weight-resident MFMA matmul (int8 and f16/bf16), W8A16 decode GEMV,
softmax / RMSNorm / LayerNorm row reductions, the SwiGLU FFN composition, and
the tile-autotune protocol.

The kernels live in ``csrc/`` (HIP for gfx950) behind the C ABI of
``include/hx.h``, built into ``libhxmi.so`` by ``build.py``.  This package is
the host side: ``ops`` binds the ABI for torch device tensors, ``search``
restates the autotune protocol of QHB/backend/hmx_search.py.

The directory name is not a Python identifier; load it with
``__graft_entry__.load_package()`` (registered as ``hexagon_mlir_amd``).
"""
from . import _abi, ops, search  # noqa: F401
from ._abi import HXError, load  # noqa: F401
from .ops import (Bound, ResidentWeight, attention, bind_gemm_i8, bind_matmul, bind_matmul_resident, bind_row_op,  # noqa: F401
                  build_id, clock_probe, clock_read, config_count, config_pins_load, config_pins_save, manifest, manifest_clear, manifest_enable, config_get, config_lookup,  # noqa: F401
                  config_select, gemm_i8, gemv_w8a16, layer_norm, matmul, matmul_resident,
                  rms_norm, silu_mul, softmax, swiglu_ffn)
