"""Python entry points of the MI355X INT4 weight-only linear path.

Drop-in for the int4 part of the reference's ``kernelforge/ops.py``
(:171-214, :277-302): same function names, signatures, defaults, validation
order, exception types and messages, and the same
``torch.library.custom_op("kernelforge::int4_matmul")`` with a fake impl.
Underneath, every op calls the C ABI of ``libkf_int4.so`` (gfx950 HIP
kernels) on torch's current HIP stream; outputs and split-K workspaces come
from torch's caching allocator, so the ops are hipGraph-capturable.

Inference only: no backward formulas are registered.
"""

from __future__ import annotations

import contextlib
import ctypes
from typing import Optional

import torch
from torch._subclasses.fake_tensor import FakeTensor

from kernelforge import _lib

# Measured GEMV/GEMM crossover on one MI355X (dispatch_sweep.py beside bench.py): the
# largest M at which the sum of GEMV times over the layer shapes beats the GEMM's
# (reference rule, bench/sweep_int4_dispatch.py:51-57).  Above it int4_gemm runs the
# skinny MFMA kernel for small M, then the tiled MFMA kernels.
GEMV_MAX_M = 4
# The reference's int4_matmul sends M <= 7 to its GEMV, which accepts every N, and M >= 8
# to its GEMM, which rejects N % 64 != 0 (kernelforge/ops.py:193,204-214).  Our MFMA kernels
# need N % 64 == 0 as well, so between GEMV_MAX_M and 7 a shape the GEMM cannot take stays
# on the GEMV: int4_matmul accepts exactly what the reference's accepts and raises the same
# ValueError for the rest.
_GEMV_LIMIT_M = 7


def _use_gemv(m: int, n: int) -> bool:
    return m <= GEMV_MAX_M or (m <= _GEMV_LIMIT_M and n % 64 != 0)


def _stream_ptr(device: torch.device) -> int:
    """The raw handle of torch's current HIP stream on `device`."""
    return torch._C._cuda_getCurrentRawStream(device.index if device.index is not None else torch.cuda.current_device())


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


_PLAIN = (torch.Tensor, torch.nn.Parameter)


def _traced(tensors) -> bool:
    """True when a tracer must see the registered op instead of a kernel launch: torch is
    compiling, a TorchDispatchMode is active (FakeTensorMode, make_fx's proxy mode, ...), or an
    input is a tensor subclass (a FakeTensor made outside its mode, a functional tensor, ...).
    Eager calls on plain tensors return False and skip the op dispatcher."""
    if torch.compiler.is_compiling() or torch._C._len_torch_dispatch_stack() > 0:
        return True
    return any(t is not None and type(t) not in _PLAIN for t in tensors)


def _on(device: torch.device):
    """Makes `device` current for the launch; a no-op context when it already is (the common
    case, which then costs no device switch)."""
    if device.index is None or device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


def _check_int4(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int) -> None:
    """Reference kernelforge/ops.py:171-182 (same order, types and messages)."""
    if not isinstance(x, torch.Tensor) or not x.is_cuda or x.dtype != torch.float16 or x.dim() != 2:
        raise TypeError("x must be a 2-D fp16 CUDA tensor [M, K]")
    if not x.is_contiguous():
        raise ValueError("x must be contiguous")
    if packed.dtype != torch.int32 or scales.dtype != torch.float16:
        raise TypeError("packed must be int32 and scales fp16 (see kernelforge.quantize)")
    k = x.shape[1]
    if k % group_size != 0:
        raise ValueError(f"K={k} is not a multiple of group_size={group_size}")
    if packed.shape[1] * 8 != k:
        raise ValueError(f"packed has K/8={packed.shape[1]} columns but x has K={k}")


def _check_native(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int) -> None:
    """Tensor checks the reference makes in C++ (csrc/gemm/dequant_gemv.cu:5-19); RuntimeError like TORCH_CHECK.

    Valid inputs pass one combined test (a few microseconds less host time per problem); anything
    else goes through the checks one by one, which raise in the reference's order."""
    dev = x.get_device()
    if (type(x) in _PLAIN and type(packed) in _PLAIN and type(scales) in _PLAIN
            and x.is_cuda and packed.is_cuda and scales.is_cuda and x.is_contiguous() and packed.is_contiguous()
            and scales.is_contiguous() and packed.get_device() == dev and scales.get_device() == dev
            and packed.dim() == 2 and scales.dim() == 2 and (group_size == 64 or group_size == 128)
            and scales.shape[0] == packed.shape[0] and scales.shape[1] == x.shape[1] // group_size
            and not (x.data_ptr() | packed.data_ptr()) & 15):
        return
    _check_native_each(x, packed, scales, group_size)


def _check_native_each(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int) -> None:
    """_check_native's conditions one at a time, raising the first that fails."""
    for name, t in (("x", x), ("packed", packed), ("scales", scales)):
        if isinstance(t, FakeTensor) or t.is_meta:
            raise RuntimeError(f"{name} has no device memory (a fake or meta tensor): trace through int4_linear / "
                               "kernelforge::int4_matmul, whose fake impl gives the output shape")
        if not t.is_cuda:
            raise RuntimeError(f"{name} must be a CUDA tensor")
        if not t.is_contiguous():
            raise RuntimeError(f"{name} must be contiguous")
        if t.device != x.device:
            raise RuntimeError(f"{name} is on {t.device} but x is on {x.device}")
    if packed.dim() != 2:
        raise RuntimeError("packed must be int32 [N, K / 8]")
    if scales.dim() != 2:
        raise RuntimeError("scales must be fp16 [N, K / group]")
    if group_size not in (64, 128):
        raise RuntimeError(f"group size must be 64 or 128, got {group_size}")
    k, n = x.shape[1], packed.shape[0]
    if scales.shape[0] != n or scales.shape[1] != k // group_size:
        raise RuntimeError("scales must be [N, K / group]")
    if x.data_ptr() % 16 or packed.data_ptr() % 16:
        raise RuntimeError("INT4 kernels need 16-byte aligned inputs")


def int4_gemv(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """Fused INT4 dequant GEMV for M in [1, 8]: x [M, K] fp16 @ W_hat^T -> [M, N] fp16.

    Reference kernelforge/ops.py:185-190; kernel csrc/kf_gemv.hip.
    """
    _check_int4(x, packed, scales, group_size)
    if not 1 <= x.shape[0] <= 8:
        raise ValueError(f"int4_gemv handles M in [1, 8], got M={x.shape[0]}")
    _check_native(x, packed, scales, group_size)
    return _launch_gemv(x, packed, scales, int(group_size))


def _launch_gemv(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """kf_int4_gemv on validated inputs."""
    lib = _lib.load()
    m, k = x.shape
    n = packed.shape[0]
    dev = x.device
    y = torch.empty(m, n, dtype=torch.float16, device=dev)
    with _on(dev):
        status = lib.kf_int4_gemv(x.data_ptr(), packed.data_ptr(), scales.data_ptr(), y.data_ptr(), m, n, k,
                                  group_size, _stream_ptr(dev))
    _lib.check(status, "int4_gemv")
    return y


# The MFMA-16 block copy of a weight (kf_int4_reorder_mfma16) makes the skinny MFMA kernel's
# weight loads contiguous (7-15% faster at M <= 32) and is bit-identical in results, at the cost
# of a second copy of the weight in device memory (0.74x the INT4 weights of a TinyLlama whose
# layers all run the skinny kernel once) and one host wait when it is built.  Opt-in, two ways:
# prepare_mfma16(packed, scales) attaches a copy to one weight, which int4_gemm then reads
# whenever it runs the skinny kernel on it; MFMA16_CACHE = True makes int4_gemm build and attach
# one by itself the first time any weight runs the skinny kernel at M <= MFMA16_MAX_M (outside
# HIP-graph capture).  Off, the skinny kernel reads the public layout.
MFMA16_CACHE = False
MFMA16_MAX_M = 32
_MFMA16_ATTR = "_kf_mfma16"


def int4_reorder_mfma16(packed: torch.Tensor, scales: torch.Tensor,
                        group_size: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """The MFMA-16 block copy (packed_r int32, scales_r fp16) of a packed weight; K % 128 == 0.

    An internal layout (the public packed format is unchanged); kernel csrc/kf_skinny.hip.
    """
    if packed.dtype != torch.int32 or scales.dtype != torch.float16 or not packed.is_cuda:
        raise TypeError("int4_reorder_mfma16 expects int32 packed and fp16 scales on a CUDA device")
    if not packed.is_contiguous() or not scales.is_contiguous():
        raise ValueError("packed and scales must be contiguous")
    n, k = packed.shape[0], packed.shape[1] * 8
    lib = _lib.load()
    pb, sb = ctypes.c_size_t(), ctypes.c_size_t()
    _lib.check(lib.kf_int4_mfma16_sizes(n, k, int(group_size), ctypes.byref(pb), ctypes.byref(sb)), "mfma16 sizes")
    packed_r = torch.empty(pb.value // 4, dtype=torch.int32, device=packed.device)
    scales_r = torch.empty(sb.value // 2, dtype=torch.float16, device=packed.device)
    with _on(packed.device):
        _lib.check(lib.kf_int4_reorder_mfma16(_ptr(packed), _ptr(scales), _ptr(packed_r), _ptr(scales_r), n, k,
                                              int(group_size), _stream_ptr(packed.device)), "int4_reorder_mfma16")
    return packed_r, scales_r


def _mfma16_key(packed: torch.Tensor, scales: torch.Tensor, group_size: int) -> tuple:
    """What the cached copy must match.  Tensors made under torch.inference_mode() keep no
    version counter, so an in-place update of them cannot be seen: their key has no versions."""
    versions = None if packed.is_inference() or scales.is_inference() else (packed._version, scales._version)
    return (int(group_size), packed.data_ptr(), scales.data_ptr(), versions)


def prepare_mfma16(packed: torch.Tensor, scales: torch.Tensor, group_size: int = 128) -> None:
    """Builds the MFMA-16 copy of a weight now and keeps it on `packed` for int4_gemm.

    The per-weight opt-in: int4_gemm reads the copy whenever it runs the skinny kernel on this
    weight (with MFMA16_CACHE on it would build one by itself on first use, except for tensors
    created under torch.inference_mode(), which have no version counter to notice in-place
    updates: for those this is the only way, and the caller promises not to modify packed /
    scales in place afterwards).  An in-place update of a weight with version counters makes
    int4_gemm ignore the stale copy.  Not during HIP-graph capture.  The host waits for the copy
    to be written before it is attached, so a later int4_gemm on any stream reads a complete copy.
    """
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("prepare_mfma16 launches a kernel and allocates; call it outside HIP-graph capture")
    packed_r, scales_r = int4_reorder_mfma16(packed, scales, group_size)
    done = torch.cuda.Event()
    done.record(torch.cuda.current_stream(packed.device))
    done.synchronize()
    setattr(packed, _MFMA16_ATTR, (_mfma16_key(packed, scales, group_size), packed_r, scales_r))


def _mfma16_copy(packed: torch.Tensor, scales: torch.Tensor, group_size: int, m: int):
    """The MFMA-16 copy of (packed, scales) attached by prepare_mfma16 (or, with MFMA16_CACHE, built
    here on first use); None when there is none or it does not apply."""
    if m > MFMA16_MAX_M or packed.shape[1] % 16 != 0:
        return None
    cached = getattr(packed, _MFMA16_ATTR, None)
    if cached is None and not MFMA16_CACHE:
        return None
    key = _mfma16_key(packed, scales, group_size)
    if cached is not None and cached[0] == key:
        return cached[1], cached[2]
    if not MFMA16_CACHE or key[3] is None or torch.cuda.is_current_stream_capturing():
        return None  # inference tensors: only a copy made by prepare_mfma16
    if gemm_plan(m, packed.shape[0], packed.shape[1] * 8, group_size, packed.device)["kernel"] != "skinny":
        return None  # only the skinny kernel reads the copy
    prepare_mfma16(packed, scales, group_size)
    cached = getattr(packed, _MFMA16_ATTR)
    return cached[1], cached[2]


def int4_gemm(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """Fused INT4 dequant GEMM on the MFMA matrix cores, any M, N a multiple of 64.

    Reference kernelforge/ops.py:196-201; kernels csrc/kf_gemm.hip, csrc/kf_skinny.hip.
    """
    _check_int4(x, packed, scales, group_size)
    if packed.shape[0] % 64 != 0:
        raise ValueError(f"int4_gemm needs N to be a multiple of 64, got N={packed.shape[0]}")
    _check_native(x, packed, scales, group_size)
    if x.shape[0] < 1:  # csrc/gemm/dequant_gemm_tc.cu:14 (its TORCH_CHECK text)
        raise RuntimeError(f"bad M {x.shape[0]}")
    return _launch_gemm(x, packed, scales, int(group_size))


def _launch_gemm(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """kf_int4_gemm (or its MFMA-16-copy variant) on validated inputs."""
    lib = _lib.load()
    m, k = x.shape
    n = packed.shape[0]
    dev = x.device
    y = torch.empty(m, n, dtype=torch.float16, device=dev)
    with _on(dev):
        ws_bytes = lib.kf_int4_gemm_workspace_bytes(m, n, k, group_size)
        ws = torch.empty((ws_bytes + 3) // 4, dtype=torch.float32, device=dev) if ws_bytes else None
        copy = _mfma16_copy(packed, scales, group_size, m)
        if copy is not None:
            status = lib.kf_int4_gemm_mfma16(_ptr(x), _ptr(packed), _ptr(scales), _ptr(copy[0]), _ptr(copy[1]),
                                             _ptr(y), _ptr(ws) if ws is not None else None, ws_bytes, m, n, k,
                                             group_size, _stream_ptr(dev))
        else:
            status = lib.kf_int4_gemm(_ptr(x), _ptr(packed), _ptr(scales), _ptr(y),
                                      _ptr(ws) if ws is not None else None, ws_bytes, m, n, k, group_size,
                                      _stream_ptr(dev))
    _lib.check(status, "int4_gemm")
    return y


def gemm_plan(m: int, n: int, k: int, group_size: int = 128, device: torch.device | None = None) -> dict:
    """The kernel int4_gemm runs for an [m, k] x [n, k]^T problem on `device` (default: current).

    Returns {"kernel": "skinny" or the tile-table index, "num_kernels": table size,
    "splits": split-K factor, "tile": (BM, BN)}.  Diagnostics; no reference counterpart.
    """
    lib = _lib.load()
    out = [ctypes.c_int() for _ in range(5)]
    with torch.cuda.device(device if device is not None else torch.cuda.current_device()):
        status = lib.kf_int4_gemm_plan(int(m), int(n), int(k), int(group_size), *[ctypes.byref(v) for v in out])
    _lib.check(status, "gemm_plan")
    kernel, num, splits, bm, bn = (v.value for v in out)
    return {"kernel": "skinny" if kernel < 0 else kernel, "num_kernels": num, "splits": splits, "tile": (bm, bn)}


def int4_matmul(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """y = x @ W_hat^T for INT4 weights from kernelforge.quantize, choosing the kernel by M.

    M <= GEMV_MAX_M: the bandwidth-bound GEMV; larger M: the MFMA GEMM (M <= 7 with N not
    a multiple of 64 stays on the GEMV, as in the reference).  Reference kernelforge/ops.py:204-214.
    """
    if _use_gemv(x.shape[0], packed.shape[0]):
        return int4_gemv(x, packed, scales, group_size)
    return int4_gemm(x, packed, scales, group_size)


def _matmul_checked(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """int4_matmul after _check_int4 has passed (int4_linear's eager path): the remaining checks of
    int4_gemv / int4_gemm in their order, then the launch, without validating twice."""
    m, n = x.shape[0], packed.shape[0]
    if _use_gemv(m, n):
        if not 1 <= m <= 8:
            raise ValueError(f"int4_gemv handles M in [1, 8], got M={m}")
        _check_native(x, packed, scales, group_size)
        return _launch_gemv(x, packed, scales, group_size)
    if n % 64 != 0:
        raise ValueError(f"int4_gemm needs N to be a multiple of 64, got N={n}")
    _check_native(x, packed, scales, group_size)
    return _launch_gemm(x, packed, scales, group_size)


_QUANT_DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}  # KF_DTYPE_* of the C ABI


def int4_quantize(weight: torch.Tensor, group_size: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """(packed int32 [N, K/8], scales fp16 [N, K/G]) of a weight [N, K] on the GPU.

    The gfx950 quantize + pack kernel; bit-identical to ``kernelforge.quantize.quantize_weight``
    of the same weight on the CPU (the reference's quantize_int4 + pack_int4,
    kernelforge/quantize.py:61-105).  fp32, fp16 or bf16 weights with finite values.
    """
    if weight.dim() != 2:
        raise ValueError(f"weight must be 2-D [N, K], got shape {tuple(weight.shape)}")
    if group_size not in (64, 128):
        raise ValueError(f"group_size must be one of (64, 128), got {group_size}")
    n, k = weight.shape
    if k % group_size:
        raise ValueError(f"K={k} is not a multiple of group_size={group_size}. Pad K or pick another group size.")
    if not weight.is_cuda:
        raise TypeError("int4_quantize needs a CUDA tensor")
    code = _QUANT_DTYPES.get(weight.dtype)
    if code is None:
        raise TypeError(f"int4_quantize supports float32, float16 and bfloat16 weights, got {weight.dtype}")
    w = weight.contiguous()
    if w.data_ptr() % 16:
        w = w.clone()
    lib = _lib.load()
    packed = torch.empty(n, k // 8, dtype=torch.int32, device=w.device)
    scales = torch.empty(n, k // group_size, dtype=torch.float16, device=w.device)
    with _on(w.device):
        status = lib.kf_int4_quantize(_ptr(w), code, _ptr(packed), _ptr(scales), n, k, int(group_size),
                                      _stream_ptr(w.device))
    _lib.check(status, "int4_quantize")
    return packed, scales


def int4_dequant_fp16(packed: torch.Tensor, scales: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """W_hat = fp16(q * s) [N, K] on the GPU, the exact operand the GEMM feeds to the matrix cores.

    Counterpart of the reference's ``quantize.dequantize(qw, torch.float16)``
    (kernelforge/quantize.py:108-113), exported for bit-exactness checks.
    """
    if packed.dtype != torch.int32 or scales.dtype != torch.float16:
        raise TypeError("packed must be int32 and scales fp16 (see kernelforge.quantize)")
    if not packed.is_cuda or not scales.is_cuda:
        raise TypeError("packed and scales must be CUDA tensors")
    if not packed.is_contiguous() or not scales.is_contiguous():
        raise ValueError("packed and scales must be contiguous")
    n, k = packed.shape[0], packed.shape[1] * 8
    if scales.shape != (n, k // group_size):
        raise ValueError("scales must be [N, K / group]")
    lib = _lib.load()
    w_hat = torch.empty(n, k, dtype=torch.float16, device=packed.device)
    with _on(packed.device):
        status = lib.kf_int4_dequant_fp16(_ptr(packed), _ptr(scales), _ptr(w_hat), n, k, int(group_size),
                                          _stream_ptr(packed.device))
    _lib.check(status, "int4_dequant_fp16")
    return w_hat


def int4_gemv_grouped(xs: list[torch.Tensor], packed: list[torch.Tensor], scales: list[torch.Tensor],
                      group_size: int = 128, *, _checked: bool = False) -> list[torch.Tensor]:
    """Several independent INT4 GEMVs (common M in [1, 8]) in one kernel launch per 8 problems.

    Each output equals ``int4_gemv(xs[i], packed[i], scales[i], group_size)`` bit for bit.
    This is the multi-problem launch of the GEMV (no reference counterpart as
    an entry point): on MI355X a launch's fixed cost exceeds the time to stream
    a small decode linear, so independent linears (q|k|v, gate|up, or separate
    layers) should share a launch.  Kernel: csrc/kf_gemv.hip.
    """
    if not (len(xs) == len(packed) == len(scales)) or not xs:
        raise ValueError("xs, packed and scales must be non-empty lists of equal length")
    m = xs[0].shape[0] if isinstance(xs[0], torch.Tensor) and xs[0].dim() == 2 else -1
    for x, p, s in zip(xs, packed, scales):
        if not _checked:
            _check_int4(x, p, s, group_size)
        if x.shape[0] != m:
            raise ValueError(f"all problems must share M, got {x.shape[0]} and {m}")
        if x.device != xs[0].device:
            raise RuntimeError("all problems must be on one device")
        _check_native(x, p, s, group_size)
    if not 1 <= m <= 8:
        raise ValueError(f"int4_gemv handles M in [1, 8], got M={m}")
    lib = _lib.load()
    dev = xs[0].device
    # One tensor per output: the registered grouped op may not return outputs that alias each other.
    ns = [p.shape[0] for p in packed]
    ys = [torch.empty(m, n, dtype=torch.float16, device=dev) for n in ns]
    problem = _lib.GemvProblem
    with _on(dev):
        stream = _stream_ptr(dev)
        for b0 in range(0, len(xs), _lib.GEMV_MAX_GROUP):
            b1 = min(b0 + _lib.GEMV_MAX_GROUP, len(xs))
            probs = (problem * (b1 - b0))(*[problem(xs[i].data_ptr(), packed[i].data_ptr(), scales[i].data_ptr(),
                                                    ys[i].data_ptr(), ns[i], xs[i].shape[1]) for i in range(b0, b1)])
            status = lib.kf_int4_gemv_grouped(probs, b1 - b0, m, int(group_size), stream)
            _lib.check(status, "int4_gemv_grouped")
    return ys


@torch.library.custom_op("kernelforge::int4_matmul", mutates_args=())
def _int4_matmul_op(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    return int4_matmul(x, packed, scales, group_size)


@_int4_matmul_op.register_fake
def _(x, packed, scales, group_size):
    return x.new_empty(x.shape[0], packed.shape[0])


def _matmul_grouped(xs: list[torch.Tensor], packed: list[torch.Tensor], scales: list[torch.Tensor],
                    group_size: int, checked: bool = False) -> list[torch.Tensor]:
    """checked: _check_int4 has passed on every problem (int4_linear_grouped's eager path)."""
    if all(_use_gemv(x.shape[0], p.shape[0]) for x, p in zip(xs, packed)):
        return int4_gemv_grouped(xs, packed, scales, group_size, _checked=checked)
    if xs[0].shape[0] <= _GEMV_LIMIT_M:
        return [int4_matmul(x, p, s, group_size) for x, p, s in zip(xs, packed, scales)]
    return [int4_gemm(x, p, s, group_size) for x, p, s in zip(xs, packed, scales)]


@torch.library.custom_op("kernelforge::int4_matmul_grouped", mutates_args=())
def _int4_matmul_grouped_op(xs: list[torch.Tensor], packed: list[torch.Tensor], scales: list[torch.Tensor],
                            group_size: int) -> list[torch.Tensor]:
    return _matmul_grouped(xs, packed, scales, group_size)


@_int4_matmul_grouped_op.register_fake
def _(xs, packed, scales, group_size):
    return [x.new_empty(x.shape[0], p.shape[0]) for x, p in zip(xs, packed)]


def int4_linear_grouped(xs: list[torch.Tensor], packed: list[torch.Tensor], scales: list[torch.Tensor],
                        group_size: int = 128, biases: list[torch.Tensor | None] | None = None
                        ) -> list[torch.Tensor]:
    """``[int4_linear(xs[i], packed[i], scales[i], group_size, biases[i]) ...]`` with one GEMV launch
    for all problems at decode sizes (common flattened M <= GEMV_MAX_M); results are bit-identical."""
    flat = []
    for x in xs:
        x2 = x if x.dim() == 2 else x.reshape(-1, x.shape[-1])
        flat.append(x2 if x2.is_contiguous() else x2.contiguous())
    for x2, p, s in zip(flat, packed, scales):
        _check_int4(x2, p, s, group_size)
    if _traced([*flat, *packed, *scales]):
        ys = _int4_matmul_grouped_op(flat, list(packed), list(scales), int(group_size))
    else:  # eager: the op's implementation without the dispatcher (as in int4_linear), checked once
        ys = _matmul_grouped(flat, list(packed), list(scales), int(group_size), checked=True)
    out = []
    for i, y in enumerate(ys):
        b = biases[i] if biases is not None else None
        if b is not None:
            y = y + b
        out.append(y if xs[i].dim() == 2 else y.reshape(*xs[i].shape[:-1], packed[i].shape[0]))
    return out


def int4_linear(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int = 128,
                bias: torch.Tensor | None = None) -> torch.Tensor:
    """y = x @ W_hat^T (+ bias) for INT4 weights from kernelforge.quantize. x: [..., K] fp16.

    Leading dimensions are flattened into M like nn.Linear; the bias add is a
    separate fp16 add, as in the reference (kernelforge/ops.py:287-302).
    """
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    _check_int4(x2, packed, scales, group_size)
    # The registered op kernelforge::int4_matmul whenever torch compiles or any tracer or dispatch
    # mode is looking (torch.compile, FakeTensorMode, make_fx, ...), as the reference always calls
    # it; eager calls on plain tensors go straight to its implementation (same result), skipping
    # ~14 us of op dispatch.
    if _traced((x2, packed, scales)):
        y = _int4_matmul_op(x2, packed, scales, int(group_size))
    else:
        y = _matmul_checked(x2, packed, scales, int(group_size))
    if bias is not None:
        y = y + bias
    return y.reshape(*lead, packed.shape[0])


def int4_linear_fused(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int = 128, *,
                      norm_weight: torch.Tensor | None = None, eps: float = 1e-5, up: torch.Tensor | None = None,
                      residual: torch.Tensor | None = None) -> torch.Tensor:
    """A decoder linear with the work around it: ``residual + int4_linear(prologue(x))``.

    prologue: with ``norm_weight``, RMSNorm ``x * rsqrt(mean(x^2) + eps) * norm_weight`` (fp32
    inside); with ``up``, SwiGLU ``silu(x) * up`` where x is the gate (the fp16 roundings of torch's
    ``silu(x) * up``); neither: x itself.  ``residual`` ([..., N] fp16), when given, is added to the
    fp16 result exactly as ``residual + y`` would be.

    At decode size (one row of x, K <= 10240) all of it is one GEMV launch
    (``kf_int4_gemv_fused``): the prologue runs on the workgroup's LDS copy of x and the residual
    joins the store, with the product bit-identical to ``int4_linear``'s.  Other sizes run the
    same steps as separate torch ops around ``int4_linear``.  No reference counterpart.
    """
    if norm_weight is not None and up is not None:
        raise ValueError("int4_linear_fused takes norm_weight or up, not both")
    lead = x.shape[:-1]
    k = x.shape[-1]
    n = packed.shape[0]
    x2 = x.reshape(-1, k)
    m = x2.shape[0]
    res2 = residual.reshape(-1, n) if residual is not None else None
    if res2 is not None and (res2.shape[0] != m or res2.dtype != torch.float16 or res2.device != x.device):
        raise ValueError(f"residual must be fp16 [..., {n}] on {x.device} with the leading dims of x")
    aux = norm_weight if norm_weight is not None else up
    if aux is not None and (aux.dtype != torch.float16 or aux.device != x.device):
        raise ValueError("norm_weight / up must be fp16 on the device of x")
    if up is not None and up.shape != x.shape:
        raise ValueError(f"up must have the shape of x, {tuple(x.shape)}, got {tuple(up.shape)}")
    if norm_weight is not None and norm_weight.shape != (k,):
        raise ValueError(f"norm_weight must be [{k}], got {tuple(norm_weight.shape)}")
    prologue = (_lib.KF_PROLOGUE_RMSNORM if norm_weight is not None
                else _lib.KF_PROLOGUE_SWIGLU if up is not None else _lib.KF_PROLOGUE_NONE)
    fused = (m == 1 and k <= _lib.KF_GEMV_FUSED_MAX_K and x.is_cuda and x2.is_contiguous()
             and (aux is None or aux.is_contiguous()) and (res2 is None or res2.is_contiguous()))
    if not fused:
        return _fused_composition(x2, packed, scales, group_size, prologue, aux, eps, res2).reshape(*lead, n)
    _check_int4(x2, packed, scales, group_size)
    if _traced((x2, packed, scales, aux, res2)):
        y = _int4_linear_fused_op(x2, packed, scales, int(group_size), prologue, aux, float(eps), res2)
    else:
        y = _launch_fused(x2, packed, scales, int(group_size), prologue, aux, float(eps), res2)
    return y.reshape(*lead, n)


def _fused_composition(x2: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int, prologue: int,
                       aux: torch.Tensor | None, eps: float, res2: torch.Tensor | None) -> torch.Tensor:
    """int4_linear_fused's steps as separate torch ops around int4_linear (shapes the fused launch
    does not take); x2 [M, K] -> y [M, N]."""
    k = x2.shape[1]
    if prologue == _lib.KF_PROLOGUE_RMSNORM:
        x2 = torch.nn.functional.rms_norm(x2, (k,), aux, eps)
    elif prologue == _lib.KF_PROLOGUE_SWIGLU:
        x2 = torch.nn.functional.silu(x2) * aux.reshape(-1, k)
    y = int4_linear(x2, packed, scales, group_size)
    return y if res2 is None else res2 + y


def _launch_fused(x2: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int, prologue: int,
                  aux: torch.Tensor | None, eps: float, res2: torch.Tensor | None) -> torch.Tensor:
    """kf_int4_gemv_fused on int4_linear_fused's validated one-row inputs; y [1, N].  x or the
    prologue operand off a 16-byte boundary (the launch's LDS copies need it) takes the
    composition instead, with the same result."""
    if x2.data_ptr() % 16 or (aux is not None and aux.data_ptr() % 16):
        return _fused_composition(x2, packed, scales, group_size, prologue, aux, eps, res2)
    _check_native(x2, packed, scales, group_size)
    lib = _lib.load()
    n, k = packed.shape[0], x2.shape[1]
    y = torch.empty(1, n, dtype=torch.float16, device=x2.device)
    with _on(x2.device):
        status = lib.kf_int4_gemv_fused(_ptr(x2), _ptr(packed), _ptr(scales), _ptr(y), 1, n, k, group_size,
                                        prologue, _ptr(aux) if aux is not None else None, eps,
                                        _ptr(res2) if res2 is not None else None, _stream_ptr(x2.device))
    _lib.check(status, "int4_gemv_fused")
    return y


@torch.library.custom_op("kernelforge::int4_linear_fused", mutates_args=())
def _int4_linear_fused_op(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int,
                          prologue: int, aux: Optional[torch.Tensor], eps: float,
                          residual: Optional[torch.Tensor]) -> torch.Tensor:
    return _launch_fused(x, packed, scales, group_size, prologue, aux, eps, residual)


@_int4_linear_fused_op.register_fake
def _(x, packed, scales, group_size, prologue, aux, eps, residual):
    return x.new_empty(1, packed.shape[0])


def int4_qkv_rope_cache(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int, *,
                        cos: torch.Tensor, sin: torch.Tensor, pos: torch.Tensor, cache_k: torch.Tensor,
                        cache_v: torch.Tensor, heads: int, kv_heads: int, head_dim: int,
                        norm_weight: torch.Tensor | None = None, eps: float = 1e-5) -> torch.Tensor:
    """The q|k|v projection of one decode token with RoPE and the KV-cache update in one launch.

    x: one row [..., K] fp16 (RMSNorm-ed first when ``norm_weight`` is given); packed / scales: the
    q|k|v weights concatenated along N = (heads + 2 kv_heads) head_dim; cos / sin: fp16
    [max_seq, head_dim] tables (sin with the rotate-half sign folded in: -sin on the first half);
    pos: int64 [1] on the device; cache_k: fp16 [kv_heads, head_dim, max_seq] (K transposed),
    cache_v: fp16 [kv_heads, max_seq, head_dim].  Returns y [..., N]: q and k rotated, v as is.
    k and v are also written at position pos of the caches; a pos outside [0, max_seq) writes no
    cache entry (and rotates with the tables' row 0).  Kernel: kf_int4_gemv_qkv_rope.
    No reference counterpart.
    """
    k = x.shape[-1]
    n = packed.shape[0]
    x2 = x.reshape(-1, k)
    if x2.shape[0] != 1:
        raise ValueError(f"int4_qkv_rope_cache takes one token, got {x2.shape[0]} rows")
    if (heads + 2 * kv_heads) * head_dim != n:
        raise ValueError(f"packed has N={n} rows, not (heads + 2 kv_heads) * head_dim")
    max_seq = cos.shape[0]
    for name, t, numel in (("cos", cos, max_seq * head_dim), ("sin", sin, max_seq * head_dim),
                           ("cache_k", cache_k, kv_heads * head_dim * max_seq),
                           ("cache_v", cache_v, kv_heads * max_seq * head_dim)):
        if t.dtype != torch.float16 or not t.is_contiguous() or t.numel() != numel or t.device != x.device:
            raise ValueError(f"{name} must be a contiguous fp16 tensor of {numel} elements on {x.device}")
    if pos.dtype != torch.int64 or pos.numel() != 1 or pos.device != x.device:
        raise ValueError("pos must be one int64 on the device of x")
    if norm_weight is not None and (norm_weight.dtype != torch.float16 or norm_weight.shape != (k,)
                                    or not norm_weight.is_contiguous()):
        raise ValueError(f"norm_weight must be a contiguous, 16-byte aligned fp16 [{k}]")
    x2 = x2.contiguous()
    _check_int4(x2, packed, scales, group_size)
    args = (x2, packed, scales, int(group_size), cos, sin, pos, cache_k, cache_v, int(heads), int(kv_heads),
            int(head_dim), norm_weight, float(eps))
    y = _int4_qkv_rope_cache_op(*args) if _traced((x2, packed, scales, cos, sin, pos, cache_k, cache_v,
                                                   norm_weight)) else _launch_qkv_rope(*args)
    return y.reshape(*x.shape[:-1], n)


def _launch_qkv_rope(x2, packed, scales, group_size, cos, sin, pos, cache_k, cache_v, heads, kv_heads, head_dim,
                     norm_weight, eps) -> torch.Tensor:
    """kf_int4_gemv_qkv_rope on int4_qkv_rope_cache's validated inputs; y [1, N]."""
    _check_native(x2, packed, scales, group_size)
    for name, t in (("cos", cos), ("sin", sin), ("pos", pos), ("cache_k", cache_k), ("cache_v", cache_v),
                    ("norm_weight", norm_weight)):
        if t is not None and (isinstance(t, FakeTensor) or t.is_meta):
            raise RuntimeError(f"{name} has no device memory (a fake or meta tensor)")
    if norm_weight is not None and norm_weight.data_ptr() % 16:
        raise ValueError(f"norm_weight must be a contiguous, 16-byte aligned fp16 [{x2.shape[1]}]")
    lib = _lib.load()
    n, k = packed.shape[0], x2.shape[1]
    y = torch.empty(1, n, dtype=torch.float16, device=x2.device)
    rc = _lib.RopeCache(_ptr(cos), _ptr(sin), _ptr(pos), _ptr(cache_k), _ptr(cache_v), heads, kv_heads, head_dim,
                        cos.shape[0])
    with _on(x2.device):
        status = lib.kf_int4_gemv_qkv_rope(_ptr(x2), _ptr(packed), _ptr(scales), _ptr(y), n, k, group_size,
                                           _ptr(norm_weight) if norm_weight is not None else None, eps,
                                           ctypes.byref(rc), _stream_ptr(x2.device))
    _lib.check(status, "int4_gemv_qkv_rope")
    return y


@torch.library.custom_op("kernelforge::int4_qkv_rope_cache", mutates_args=("cache_k", "cache_v"))
def _int4_qkv_rope_cache_op(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int,
                            cos: torch.Tensor, sin: torch.Tensor, pos: torch.Tensor, cache_k: torch.Tensor,
                            cache_v: torch.Tensor, heads: int, kv_heads: int, head_dim: int,
                            norm_weight: Optional[torch.Tensor], eps: float) -> torch.Tensor:
    return _launch_qkv_rope(x, packed, scales, group_size, cos, sin, pos, cache_k, cache_v, heads, kv_heads,
                            head_dim, norm_weight, eps)


@_int4_qkv_rope_cache_op.register_fake
def _(x, packed, scales, group_size, cos, sin, pos, cache_k, cache_v, heads, kv_heads, head_dim, norm_weight, eps):
    return x.new_empty(1, packed.shape[0])



def decode_argmax_step(logits: torch.Tensor, token: torch.Tensor, pos: torch.Tensor, history: torch.Tensor,
                       mask: torch.Tensor | None = None) -> None:
    """The greedy step of a graph-captured decode loop in one launch (kf_decode_argmax_step).

    logits: fp16 [n] on the GPU; token, pos: int64 [1]; history: int64 [max_seq]; mask: None or
    fp16 with max_seq elements.  Computes idx = torch.argmax(logits) (same tie and NaN rules) and
    then, on the device: pos += 1; token = idx; history[pos] = idx and mask[pos] = 0 when pos <
    max_seq.  Asynchronous on the current stream; capturable.  No reference counterpart (the
    reference's decode loop does these steps as separate torch ops).
    """
    if logits.dtype != torch.float16 or logits.dim() != 1 or not logits.is_cuda or not logits.is_contiguous():
        raise TypeError("logits must be a contiguous 1-D fp16 CUDA tensor")
    for name, t in (("token", token), ("pos", pos)):
        if t.dtype != torch.int64 or t.numel() != 1 or t.device != logits.device:
            raise ValueError(f"{name} must be one int64 on {logits.device}")
    if history.dtype != torch.int64 or history.dim() != 1 or not history.is_contiguous() or \
            history.device != logits.device:
        raise ValueError(f"history must be a contiguous 1-D int64 tensor on {logits.device}")
    max_seq = history.numel()
    if mask is not None and (mask.dtype != torch.float16 or mask.numel() != max_seq or not mask.is_contiguous()
                             or mask.device != logits.device):
        raise ValueError(f"mask must be a contiguous fp16 tensor of {max_seq} elements on {logits.device}")
    if _traced((logits, token, pos, history, mask)):
        raise RuntimeError("decode_argmax_step updates device buffers in place and has no traceable form")
    lib = _lib.load()
    with _on(logits.device):
        status = lib.kf_decode_argmax_step(_ptr(logits), logits.numel(), _ptr(token), _ptr(pos), _ptr(history),
                                           max_seq, _ptr(mask) if mask is not None else None,
                                           _stream_ptr(logits.device))
    _lib.check(status, "decode_argmax_step")
