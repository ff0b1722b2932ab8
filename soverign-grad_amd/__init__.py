"""Python binding of libsgq.so, the MI355X (gfx950) quantized-linear library.

The product is the C ABI declared in ``include/sgq.h`` and the C++17 host layer
in ``host/``; this module binds the same C ABI with ctypes so that tests and
``bench.py`` can drive it with PyTorch device tensors (PyTorch only supplies
device memory and streams).  Function names and argument meanings follow the
reference's ``quantization::`` namespace
(include/sovereigngrad/quantization.hpp:28-37):

    quantize_int8(x, scheme=PER_CHANNEL)      src/quantization.cpp:11-78
    dequantize_int8(qx)                       src/quantization.cpp:80-111
    quantize_int4(x, group_size=32)           src/quantization.cpp:113-159
    dequantize_int4(qx)                       src/quantization.cpp:161-187
    quantized_matmul_int8(x, qw, bias=None)   src/quantization.cpp:189-197
    quantized_matmul_int4(x, qw, bias=None)   src/quantization.cpp:199-206

There is no CPU fallback: every call runs the HIP kernels, and loading fails
loudly when libsgq.so is missing.
"""
from __future__ import annotations

import ctypes
import os
import threading
from dataclasses import dataclass, field
from pathlib import Path
from typing import List, Optional

import torch

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libsgq.so"

SGQ_OK = 0
PER_TENSOR = 0  # QuantizationScheme::PerTensorSymmetric
PER_CHANNEL = 1  # QuantizationScheme::PerChannelSymmetric
GROUPED = 2  # QuantizationScheme::GroupedAsymmetric
LAYOUT_INT4_TILED = 0
LAYOUT_INT4_FLAT = 1

# Every entry point of include/sgq.h with its ctypes signature.
_i64, _int, _vp = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
SIGNATURES = {
    "sgq_last_error": (ctypes.c_char_p, []),
    "sgq_abi_version": (_int, []),
    "sgq_int8_packed_bytes": (_i64, [_i64, _i64]),
    "sgq_int4_layout": (_int, [_i64, _i64, _i64]),
    "sgq_int4_packed_bytes": (_i64, [_i64, _i64, _i64]),
    "sgq_int4_devscale_count": (_i64, [_i64, _i64, _i64]),
    "sgq_int8_scale_count": (_i64, [_i64, _i64, _int]),
    "sgq_int4_scale_count": (_i64, [_i64, _i64, _i64]),
    "sgq_quantize_workspace_bytes": (_i64, [_int, _i64, _i64, _i64]),
    "sgq_linear_workspace_bytes": (_i64, [_int, _i64, _i64, _i64]),
    "sgq_linear_plan": (_int, [_int, _i64, _i64, _i64, _i64, _int, ctypes.POINTER(_int), ctypes.POINTER(_int)]),
    "sgq_gemm_xcd_plan": (_int, [_int, _i64, _i64, _i64, _i64, _int, _int, ctypes.POINTER(_int),
                                 ctypes.POINTER(_int)]),
    "sgq_workspace_init": (_int, [_vp, _i64, _vp]),
    "sgq_quantize_int8": (_int, [_vp, _i64, _i64, _int, _vp, _vp, _vp, _vp, _i64, _vp]),
    "sgq_quantize_int4": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _vp]),
    "sgq_pack_int8": (_int, [_vp, _i64, _i64, _vp, _vp, _i64, _vp]),
    "sgq_pack_int4": (_int, [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp]),
    "sgq_unpack_int8": (_int, [_vp, _i64, _i64, _vp, _vp]),
    "sgq_unpack_int4": (_int, [_vp, _i64, _i64, _i64, _vp, _vp]),
    "sgq_dequantize_int8": (_int, [_vp, _vp, _int, _i64, _i64, _vp, _vp]),
    "sgq_dequantize_int4": (_int, [_vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "sgq_dequantize_codes": (_int, [_vp, _vp, _int, _int, _i64, _i64, _i64, _vp, _vp]),
    "sgq_linear_int8": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _int, _vp, _vp, _vp, _i64, _vp]),
    "sgq_linear_int4": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp]),
    "sgq_linear_int4_noalloc": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp]),
    "sgq_swiglu_workspace_bytes": (_i64, [_int, _i64, _i64, _i64, _i64]),
    "sgq_swiglu_int8": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _int, _vp, _vp, _i64, _vp]),
    "sgq_swiglu_int4": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _i64,
                               _vp]),
    "sgq_llama_decode_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "sgq_llama_block_decode_int4": (_int, [_vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _i64, _vp]),
    "sgq_rms_norm": (_int, [_vp, _i64, _i64, _vp, ctypes.c_float, _vp, _vp]),
    "sgq_embedding": (_int, [_vp, _i64, _vp, _i64, _i64, _vp, _vp]),
}

_lib = None
_lib_lock = threading.Lock()


def load_library(path: Optional[os.PathLike] = None) -> ctypes.CDLL:
    """Loads libsgq.so and declares every signature.  Raises if it is missing."""
    global _lib
    with _lib_lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path else LIB_PATH
        if not p.exists():
            raise ImportError(
                f"libsgq.so not found at {p}; build it first (python -c 'import __graft_entry__ as g; g.build()')"
            )
        lib = ctypes.CDLL(str(p))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


class SGQError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"sgq status {status}: {message}")
        self.status = status


def _check(status: int) -> None:
    if status != SGQ_OK:
        msg = load_library().sgq_last_error().decode(errors="replace")
        raise SGQError(status, msg)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("sgq: expected a device tensor")
    return t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _dev_f32(t: torch.Tensor) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError("sgq: expected a device tensor")
    return t.contiguous().to(torch.float32)


class _Workspaces:
    """One zero-initialised workspace per (device, stream, thread), grown to the
    largest size sgq_linear_workspace_bytes / sgq_swiglu_workspace_bytes has
    asked for on it (split-K partials, the gated MLP's up projection)."""

    def __init__(self):
        self._local = threading.local()

    def get(self, nbytes: int, device: torch.device):
        if nbytes < 0:
            raise SGQError(1, "bad shape for the workspace query")
        if nbytes == 0:
            return None, 0
        cache = getattr(self._local, "cache", None)
        if cache is None:
            cache = self._local.cache = {}
        key = (device.index, _stream(device))
        ws = cache.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
            _check(load_library().sgq_workspace_init(ws.data_ptr(), ws.numel(), _stream(device)))
            cache[key] = ws
        return ws.data_ptr(), ws.numel()


_linear_ws = _Workspaces()


@dataclass
class QuantizedTensor:
    """Mirror of quantization::QuantizedTensor (quantization.hpp:17-25) plus the
    packed device buffers.  ``qdata``/``scales`` are the reference-layout
    tensors (fp32 codes in the weight's shape, fp32 scales)."""

    qdata: Optional[torch.Tensor]
    scales: torch.Tensor
    scheme: int
    original_shape: List[int]
    group_size: int
    bits: int
    packed: Optional[torch.Tensor] = None
    devscales: Optional[torch.Tensor] = None
    zero_points: Optional[torch.Tensor] = field(default=None)

    @property
    def rows(self) -> int:
        return _view2d(self.original_shape)[0]

    @property
    def cols(self) -> int:
        return _view2d(self.original_shape)[1]


def _view2d(shape) -> tuple:
    """[rows, cols] view of a weight: rows = shape[0] (src/quantization.cpp:44-45),
    rank-1 tensors are one row."""
    if len(shape) >= 2:
        cols = 1
        for d in shape[1:]:
            cols *= int(d)
        return int(shape[0]), cols
    return 1, (int(shape[0]) if len(shape) == 1 else 1)


def quantize_int8(x: torch.Tensor, scheme: int = PER_CHANNEL, keep_qdata: bool = True) -> QuantizedTensor:
    """quantization::quantize_int8 on the device (src/quantization.cpp:11-78)."""
    lib = load_library()
    x = _dev_f32(x)
    dev = x.device
    rows, cols = _view2d(x.shape)
    eff = PER_TENSOR if (scheme == PER_TENSOR or x.dim() < 2) else PER_CHANNEL
    nscales = lib.sgq_int8_scale_count(rows, cols, eff)
    scales = torch.empty(nscales, dtype=torch.float32, device=dev)
    qdata = torch.empty(x.shape, dtype=torch.float32, device=dev) if keep_qdata else None
    packed = torch.empty(max(lib.sgq_int8_packed_bytes(rows, cols), 16), dtype=torch.uint8, device=dev)
    ws = torch.empty(lib.sgq_quantize_workspace_bytes(8, rows, cols, 0), dtype=torch.uint8, device=dev)
    _check(
        lib.sgq_quantize_int8(
            _ptr(x), rows, cols, eff, _ptr(qdata), _ptr(scales), _ptr(packed), _ptr(ws), ws.numel(), _stream(dev)
        )
    )
    return QuantizedTensor(qdata, scales, scheme, list(x.shape), rows * cols, 8, packed, None)


def quantize_int4(x: torch.Tensor, group_size: int = 32, keep_qdata: bool = True) -> QuantizedTensor:
    """quantization::quantize_int4 on the device (src/quantization.cpp:113-159)."""
    lib = load_library()
    x = _dev_f32(x)
    dev = x.device
    if group_size <= 0:
        group_size = 32
    rows, cols = _view2d(x.shape)
    nscales = lib.sgq_int4_scale_count(rows, cols, group_size)
    scales = torch.empty(max(nscales, 0), dtype=torch.float32, device=dev)
    qdata = torch.empty(x.shape, dtype=torch.float32, device=dev) if keep_qdata else None
    packed = torch.empty(max(lib.sgq_int4_packed_bytes(rows, cols, group_size), 16), dtype=torch.uint8, device=dev)
    ndev = lib.sgq_int4_devscale_count(rows, cols, group_size)
    devscales = torch.empty(max(ndev, 4), dtype=torch.float32, device=dev)
    ws = torch.empty(lib.sgq_quantize_workspace_bytes(4, rows, cols, group_size), dtype=torch.uint8, device=dev)
    _check(
        lib.sgq_quantize_int4(
            _ptr(x), rows, cols, group_size, _ptr(qdata), _ptr(scales), _ptr(packed), _ptr(devscales),
            _ptr(ws), ws.numel(), _stream(dev),
        )
    )
    return QuantizedTensor(qdata, scales, GROUPED, list(x.shape), group_size, 4, packed, devscales)


def pack_int8(qdata: torch.Tensor, scales: torch.Tensor, scheme: int = PER_CHANNEL) -> QuantizedTensor:
    """Builds the device layout from reference-layout fp32 codes (load_state_dict path)."""
    lib = load_library()
    qdata = _dev_f32(qdata)
    dev = qdata.device
    rows, cols = _view2d(qdata.shape)
    packed = torch.empty(max(lib.sgq_int8_packed_bytes(rows, cols), 16), dtype=torch.uint8, device=dev)
    ws = torch.empty(lib.sgq_quantize_workspace_bytes(8, rows, cols, 0), dtype=torch.uint8, device=dev)
    _check(lib.sgq_pack_int8(_ptr(qdata), rows, cols, _ptr(packed), _ptr(ws), ws.numel(), _stream(dev)))
    return QuantizedTensor(qdata, _dev_f32(scales), scheme, list(qdata.shape), rows * cols, 8, packed, None)


def pack_int4(qdata: torch.Tensor, scales: torch.Tensor, group_size: int = 32) -> QuantizedTensor:
    lib = load_library()
    qdata = _dev_f32(qdata)
    scales = _dev_f32(scales)
    dev = qdata.device
    if group_size <= 0:
        group_size = 32
    rows, cols = _view2d(qdata.shape)
    packed = torch.empty(max(lib.sgq_int4_packed_bytes(rows, cols, group_size), 16), dtype=torch.uint8, device=dev)
    devscales = torch.empty(max(lib.sgq_int4_devscale_count(rows, cols, group_size), 4), dtype=torch.float32,
                            device=dev)
    ws = torch.empty(lib.sgq_quantize_workspace_bytes(4, rows, cols, group_size), dtype=torch.uint8, device=dev)
    _check(
        lib.sgq_pack_int4(_ptr(qdata), _ptr(scales), rows, cols, group_size, _ptr(packed), _ptr(devscales),
                          _ptr(ws), ws.numel(), _stream(dev))
    )
    return QuantizedTensor(qdata, scales, GROUPED, list(qdata.shape), group_size, 4, packed, devscales)


def unpack_codes(qx: QuantizedTensor) -> torch.Tensor:
    """fp32 codes in reference layout, read back from the packed buffer."""
    lib = load_library()
    dev = qx.packed.device
    out = torch.empty(qx.original_shape, dtype=torch.float32, device=dev)
    if qx.bits == 8:
        _check(lib.sgq_unpack_int8(_ptr(qx.packed), qx.rows, qx.cols, _ptr(out), _stream(dev)))
    else:
        _check(lib.sgq_unpack_int4(_ptr(qx.packed), qx.rows, qx.cols, qx.group_size, _ptr(out), _stream(dev)))
    return out


def _int8_branch(qx: QuantizedTensor) -> int:
    # dequantize_int8 takes the per-tensor branch when the scheme says so or a
    # single scale exists (src/quantization.cpp:90).
    return PER_TENSOR if (qx.scheme == PER_TENSOR or qx.scales.numel() == 1) else PER_CHANNEL


def dequantize_int8(qx: QuantizedTensor) -> torch.Tensor:
    lib = load_library()
    dev = qx.packed.device
    out = torch.empty(qx.original_shape, dtype=torch.float32, device=dev)
    _check(lib.sgq_dequantize_int8(_ptr(qx.packed), _ptr(qx.scales), _int8_branch(qx), qx.rows, qx.cols, _ptr(out),
                                   _stream(dev)))
    return out


def dequantize_int4(qx: QuantizedTensor) -> torch.Tensor:
    lib = load_library()
    dev = qx.packed.device
    out = torch.empty(qx.original_shape, dtype=torch.float32, device=dev)
    _check(lib.sgq_dequantize_int4(_ptr(qx.packed), _ptr(qx.scales), qx.rows, qx.cols, qx.group_size, _ptr(out),
                                   _stream(dev)))
    return out


def dequantize_codes(qx: QuantizedTensor) -> torch.Tensor:
    """dequantize_int8/int4 from the reference-layout fp32 codes (bit-exact,
    -0.0 codes included)."""
    lib = load_library()
    q = _dev_f32(qx.qdata)
    dev = q.device
    out = torch.empty(qx.original_shape, dtype=torch.float32, device=dev)
    branch = _int8_branch(qx) if qx.bits == 8 else 0
    _check(lib.sgq_dequantize_codes(_ptr(q), _ptr(_dev_f32(qx.scales)), qx.bits, branch, qx.rows, qx.cols,
                                    qx.group_size, _ptr(out), _stream(dev)))
    return out


def _linear_args(x: torch.Tensor, qw: QuantizedTensor, bias: Optional[torch.Tensor]):
    if x.dim() != 2:
        raise ValueError("matmul currently requires 2D tensors!")  # src/ops.cpp:380-382
    K, N = qw.rows, qw.cols
    if x.shape[1] != K:
        raise ValueError("Matrix inner dimensions must match for matmul!")  # src/ops.cpp:387-389
    x = _dev_f32(x)
    b = None
    if bias is not None:
        b = _dev_f32(bias).reshape(-1)
        if b.numel() != N:
            raise ValueError("bias must have out_features elements")
    return x, K, N, b


def quantized_matmul_int8(x: torch.Tensor, qw: QuantizedTensor, bias: Optional[torch.Tensor] = None,
                          out: Optional[torch.Tensor] = None) -> torch.Tensor:
    lib = load_library()
    x, K, N, b = _linear_args(x, qw, bias)
    M = x.shape[0]
    dev = x.device
    y = out if out is not None else torch.empty((M, N), dtype=torch.float32, device=dev)
    ws, nws = _linear_ws.get(lib.sgq_linear_workspace_bytes(8, M, K, N), dev)
    _check(lib.sgq_linear_int8(_ptr(x), M, K, N, _ptr(qw.packed), _ptr(qw.scales), _int8_branch(qw), _ptr(b),
                               _ptr(y), ws, nws, _stream(dev)))
    return y


def quantized_matmul_int4(x: torch.Tensor, qw: QuantizedTensor, bias: Optional[torch.Tensor] = None,
                          out: Optional[torch.Tensor] = None) -> torch.Tensor:
    lib = load_library()
    x, K, N, b = _linear_args(x, qw, bias)
    M = x.shape[0]
    dev = x.device
    y = out if out is not None else torch.empty((M, N), dtype=torch.float32, device=dev)
    ws, nws = _linear_ws.get(lib.sgq_linear_workspace_bytes(4, M, K, N), dev)
    _check(lib.sgq_linear_int4(_ptr(x), M, K, N, _ptr(qw.packed), _ptr(qw.scales), _ptr(qw.devscales),
                               qw.group_size, _ptr(b), _ptr(y), ws, nws, _stream(dev)))
    return y


def quantized_swiglu(x: torch.Tensor, w_gate: QuantizedTensor, w_up: QuantizedTensor,
                     bias_gate: Optional[torch.Tensor] = None, bias_up: Optional[torch.Tensor] = None,
                     out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """silu(x . w_gate + bias_gate) * (x . w_up + bias_up): the gated half of
    SwiGLU::forward (include/sovereigngrad/nn.hpp:151-154) with quantized
    projections, in one library call."""
    lib = load_library()
    if w_gate.bits != w_up.bits or (w_gate.rows, w_gate.cols) != (w_up.rows, w_up.cols):
        raise ValueError("gate and up weights must have the same shape and bit width")
    if w_gate.bits == 8 and _int8_branch(w_gate) != _int8_branch(w_up):
        raise ValueError("gate and up weights must use the same INT8 scheme")
    if w_gate.bits == 4 and w_gate.group_size != w_up.group_size:
        raise ValueError("gate and up weights must use the same group size")
    x, K, N, bg = _linear_args(x, w_gate, bias_gate)
    _, _, _, bu = _linear_args(x, w_up, bias_up)
    M = x.shape[0]
    dev = x.device
    h = out if out is not None else torch.empty((M, N), dtype=torch.float32, device=dev)
    ws, nws = _linear_ws.get(lib.sgq_swiglu_workspace_bytes(w_gate.bits, M, K, N, w_gate.group_size), dev)
    if w_gate.bits == 8:
        _check(lib.sgq_swiglu_int8(_ptr(x), M, K, N, _ptr(w_gate.packed), _ptr(w_gate.scales), _ptr(bg),
                                   _ptr(w_up.packed), _ptr(w_up.scales), _ptr(bu), _int8_branch(w_gate), _ptr(h),
                                   ws, nws, _stream(dev)))
    else:
        _check(lib.sgq_swiglu_int4(_ptr(x), M, K, N, _ptr(w_gate.packed), _ptr(w_gate.scales),
                                   _ptr(w_gate.devscales), _ptr(bg), _ptr(w_up.packed), _ptr(w_up.scales),
                                   _ptr(w_up.devscales), _ptr(bu), w_gate.group_size, _ptr(h), ws, nws,
                                   _stream(dev)))
    return h


def quantized_matmul(x: torch.Tensor, qw: QuantizedTensor, bias: Optional[torch.Tensor] = None,
                     out: Optional[torch.Tensor] = None) -> torch.Tensor:
    if qw.bits == 8:
        return quantized_matmul_int8(x, qw, bias, out)
    return quantized_matmul_int4(x, qw, bias, out)
