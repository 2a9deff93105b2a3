"""locomp_amd: locomp's int4/int8 quantized-inference path, native on MI355X.

Drop-in surface for locomp's quantized examples (38, 52, 58): device tensors
(``tensor / empty / zeros / ones``), dtype markers, the four kernel objects
with ``kernel[(N,), (128,)](...)`` launches, the ``gpu_*`` wrappers and the
GPU weight producers ``quantize_int4 / quantize_int4_ref / quantize_int8``.
Kernels are hand-written HIP for gfx950 in ``_liblocomp_amd.so`` (built by
``python -m locomp_amd.build``), called through its C ABI.
"""

import numpy as _np

from .tensor import Tensor, bfloat16, empty, ones, tensor, zeros
from .kernels import (dequant_int4, dequant_int8, dequant_matmul_int4, dequant_matmul_int8,
                      dequant_matvec_int4, dequant_matvec_int8, quant_matvec_int8)
from .ops import (gpu_dequant_int4, gpu_dequant_int8, gpu_matvec_int4, gpu_matvec_int4_silu_mul,
                  gpu_matvec_int8, interleave_gate_up)
from .quantize import quantize_int4, quantize_int4_ref, quantize_int8
from .checkpoint import QuantizedLinear, load_packed, quantize_checkpoint, read_packed, save_packed
from ._lib import LocompAMDError, get_policy, release_workspaces, set_policy

__version__ = "0.1.0"

# Parameter dtype markers (locomp/frontend.py:18-55): the element type each
# kernel parameter accepts.
float32 = _np.float32
float16 = _np.float16
uint8 = _np.uint8
int8 = _np.int8
int32 = _np.int32
Float16 = _np.float16
UInt8 = _np.uint8
Int8 = _np.int8
Int32 = _np.int32
BFloat16 = bfloat16


class constexpr:  # noqa: N801 - locomp's marker name
    """Marker for integer kernel parameters (locomp/frontend.py:18-21)."""



__all__ = [
    "Tensor", "tensor", "empty", "zeros", "ones", "bfloat16",
    "dequant_int4", "dequant_int8", "dequant_matvec_int4", "dequant_matvec_int8",
    "dequant_matmul_int4", "dequant_matmul_int8", "quant_matvec_int8",
    "gpu_matvec_int4", "gpu_matvec_int8", "gpu_dequant_int4", "gpu_dequant_int8",
    "gpu_matvec_int4_silu_mul", "interleave_gate_up",
    "quantize_int4", "quantize_int4_ref", "quantize_int8",
    "QuantizedLinear", "quantize_checkpoint", "save_packed", "read_packed", "load_packed",
    "LocompAMDError", "set_policy", "get_policy", "release_workspaces",
    "Float16", "UInt8", "Int8", "Int32", "BFloat16", "constexpr",
]
