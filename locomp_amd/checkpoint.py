"""Quantized on-disk format: safetensors checkpoints -> packed int4 weights.

The reference reads a safetensors checkpoint into float32 NumPy arrays
(``load_weights``, examples/54_smollm2_inference.py:331-339) and has no
quantized format.  This module adds one, in the layout the dequant-matmul
kernels consume (locomp examples/38_quantized_matmul.py:30-87):

* ``<name>.qweight``: uint8 [N, K/2], byte j = q[2j] | q[2j+1] << 4
* ``<name>.scales``:  float16 (or float32) [N, K/G]
* file metadata ``{"format": "locomp_amd.int4", "group_size": "<G>",
  "quantizer": "examples/38 quantize_int4"}``

``quantize_checkpoint`` reads every 2-D floating tensor whose name passes
``select`` (default: names ending in ``.weight`` with K a multiple of the
group size), uploads it in its stored dtype (bf16 stays bf16), quantizes it on
the GPU (``quantize_int4``, bit-identical to the reference producer) and
returns ``{name: QuantizedLinear}`` with the packed weights and scales on the
device.  ``save_packed`` / ``load_packed`` write and read the format; files
are read with safetensors only (no pickle, nothing executed from the file).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .tensor import Tensor, bfloat16, tensor

FORMAT = "locomp_amd.int4"


@dataclass
class QuantizedLinear:
    """One int4 linear layer on the device: y = x @ dequant(qweight)^T."""

    qweight: Tensor        # uint8 [N, K/2]
    scales: Tensor         # float16 / float32 [N, K/G]
    N: int
    K: int
    group_size: int

    def __call__(self, x, out_dtype=None):
        """x: [K] or [M, K] host array or device Tensor -> host ndarray."""
        from .ops import gpu_matvec_int4
        return gpu_matvec_int4(x, self.qweight, self.scales, self.group_size, out_dtype=out_dtype)


def _torch():
    import torch
    return torch


def _default_select(group_size):
    def sel(name, shape):
        return name.endswith(".weight") and len(shape) == 2 and shape[1] % group_size == 0 \
            and shape[1] % 2 == 0
    return sel


def _to_device(t):
    """torch CPU tensor (any float dtype) -> device Tensor in the same dtype
    (bf16 goes through float32, which round-trips it exactly)."""
    import torch
    if t.dtype == torch.bfloat16:
        return tensor(t.to(torch.float32).contiguous().numpy(), dtype=bfloat16)
    if t.dtype == torch.float16:
        return tensor(t.contiguous().numpy())
    return tensor(t.to(torch.float32).contiguous().numpy())


def quantize_checkpoint(path, group_size=32, scale_dtype=np.float32, select=None):
    """Quantize the selected 2-D weights of a safetensors file on the GPU.

    Scales stay float32 by default, as the reference's producers return them
    (examples/52_dequantize.py:126); ``scale_dtype=np.float16`` halves their
    size and raises ``ValueError`` if a scale overflows to inf or a nonzero
    one underflows to zero in fp16."""
    from safetensors import safe_open

    from .quantize import quantize_int4
    select = select or _default_select(group_size)
    out = {}
    with safe_open(str(path), framework="pt") as f:
        for name in f.keys():
            sl = f.get_slice(name)
            shape = tuple(sl.get_shape())
            if not select(name, shape):
                continue
            t = f.get_tensor(name)
            if not t.is_floating_point():
                continue
            dev = _to_device(t)
            P, S = quantize_int4(dev, group_size, as_tensors=True)
            dev.free()
            if np.dtype(scale_dtype) == np.float16:      # cast on the device
                s32 = S.torch
                s16 = s32.to(_torch().float16)
                bad = _torch().isinf(s16) | ((s16 == 0) & (s32 != 0))
                if bool(bad.any()):
                    raise ValueError(f"{name}: {int(bad.sum())} scales do not fit float16 "
                                     "(overflow or underflow); use scale_dtype=np.float32")
                S = Tensor(s16, np.dtype(np.float16), S.shape)
            elif np.dtype(scale_dtype) != np.float32:
                raise ValueError("scale_dtype must be float16 or float32")
            out[name] = QuantizedLinear(P, S, shape[0], shape[1], group_size)
    return out


def save_packed(path, layers, group_size=None):
    """Write {name: QuantizedLinear or (qweight, scales) host arrays} in the format."""
    from safetensors.numpy import save_file
    tensors = {}
    gs = group_size
    for name, layer in layers.items():
        if isinstance(layer, QuantizedLinear):
            q, s, g = layer.qweight.numpy(), layer.scales.numpy(), layer.group_size
        else:
            q, s = layer
            q, s = np.asarray(q), np.asarray(s)
            g = q.shape[1] * 2 // s.shape[1]
        if q.dtype != np.uint8 or q.ndim != 2 or s.ndim != 2 or s.shape[0] != q.shape[0]:
            raise ValueError(f"{name}: expected uint8 [N, K/2] and [N, K/G] scales")
        if gs is None:
            gs = g
        elif gs != g:
            raise ValueError(f"{name}: group size {g} differs from {gs}")
        tensors[f"{name}.qweight"] = np.ascontiguousarray(q)
        tensors[f"{name}.scales"] = np.ascontiguousarray(s)
    meta = {"format": FORMAT, "group_size": str(gs), "quantizer": "examples/38 quantize_int4"}
    save_file(tensors, str(path), metadata=meta)


def read_packed(path):
    """Host-side read: ({name: (qweight uint8 [N, K/2], scales [N, K/G])}, group_size)."""
    from safetensors import safe_open
    with safe_open(str(path), framework="np") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT:
            raise ValueError(f"{path}: not a {FORMAT} file (metadata {meta})")
        gs = int(meta["group_size"])
        names = sorted({k.rsplit(".", 1)[0] for k in f.keys()})
        out = {}
        for n in names:
            q = f.get_tensor(f"{n}.qweight")
            s = f.get_tensor(f"{n}.scales")
            if q.dtype != np.uint8 or s.shape[0] != q.shape[0] or q.shape[1] * 2 != s.shape[1] * gs:
                raise ValueError(f"{path}: {n} has inconsistent shapes {q.shape} / {s.shape}")
            out[n] = (q, s)
    return out, gs


def load_packed(path):
    """Read the format onto the device: {name: QuantizedLinear}."""
    host, gs = read_packed(path)
    return {n: QuantizedLinear(tensor(q), tensor(s), q.shape[0], q.shape[1] * 2, gs)
            for n, (q, s) in host.items()}
