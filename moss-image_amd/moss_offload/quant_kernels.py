"""Weight-only int8 linear on MFMA: drop-in for the Triton path of MOSS-Image's
``training/quant_kernels.py`` (:100-228, ``triton_int8_linear_forward/backward``).

The GEMMs are hand-written gfx950 kernels in ``csrc/mo_gemm.hip`` (bf16 MFMA; the int8
weight decoded to bf16 in registers on its way into the MFMA), reached through
``mo_int8_linear_forward`` and ``mo_int8_linear_backward``. From ``LIBRARY_ROWS`` rows or
``LIBRARY_WEIGHT`` weight elements up, a call whose reduction is not long against its output
width instead decodes the weight in one HIP pass (``mo_int8_decode``) and runs the same library
GEMM as the eager path, bit for bit equal to it and faster by the decode. Backend selection mirrors the reference's ``auto | eager | triton``
with ``hip`` in place of ``triton``: ``auto`` takes the HIP kernels whenever the call is
supported (bf16 activations and weight dtype on a HIP device, int8 weights, fp32 scales,
feature sizes multiples of 16, contiguous operands) and the eager path otherwise; an explicit
``hip`` request that is not supported raises. The eager path is the reference's own eager
backend (decode the weight, then ``F.linear``), not a substitute for a missing library.

The reference's module interface for this path is kept under its own names, so that
``training/quantization.py`` runs unchanged on top of this module: ``validate_quantized_backend``,
``resolve_quantized_backend`` (``"triton"`` names the fused-kernel backend, here the HIP
kernels), ``autocast_compute_dtype``, ``triton_is_available``, ``triton_int8_linear_forward``
and ``triton_int8_linear_backward`` (reference ``quant_kernels.py:30-99, 294-374``). The HIP
kernels take bf16 activations and a bf16 weight dtype; the reference's Triton kernels also take
fp16 and fp32, which ``auto`` sends to the eager path here.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _native

BACKENDS = {"auto", "eager", "hip", "triton"}  # "triton": the reference's name for "hip"


def unsupported_reason(tokens: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor,
                       weight_dtype: torch.dtype) -> str | None:
    """Why the HIP kernels cannot run this call (None when they can)."""

    if tokens.device.type != "cuda":
        return "the input is not on a HIP device"
    if weight.device != tokens.device or scale.device != tokens.device:
        return "the quantized weight and scale are not on the input device"
    if tokens.dtype != torch.bfloat16 or weight_dtype != torch.bfloat16:
        return f"only bf16 activations and weights are supported (got {tokens.dtype}, {weight_dtype})"
    if weight.dtype != torch.int8 or scale.dtype != torch.float32:
        return "weights must be int8 and scales float32"
    if weight.ndim != 2 or tokens.shape[-1] != weight.shape[1]:
        return "input and weight dimensions do not match"
    out_features, in_features = weight.shape
    if in_features % 16 or out_features % 16:
        return "feature sizes must be multiples of 16"
    if not weight.is_contiguous() or not scale.is_contiguous():
        return "weight and scale must be contiguous"
    if tokens.numel() == 0:
        return "empty input"
    return None


def resolve_backend(backend: str, tokens: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor,
                    weight_dtype: torch.dtype) -> str:
    """``auto`` -> ``hip`` or ``eager``; an explicit ``hip`` must be supported."""

    if backend not in BACKENDS:
        raise ValueError("quantized backend must be auto, eager or hip.")
    if backend == "triton":
        backend = "hip"
    if backend == "eager":
        return backend
    reason = unsupported_reason(tokens, weight, scale, weight_dtype)
    if backend == "auto":
        return "eager" if reason is not None else "hip"
    if reason is not None:
        raise RuntimeError(f"HIP int8 backend is unavailable: {reason}.")
    return backend


def decode(weight: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """The decoded weight, bf16(q * bf16(scale)) for bf16 (reference quant_kernels.py:126-131)."""

    return weight.to(dtype) * scale.to(dtype)[:, None]


# A call with at least LIBRARY_ROWS rows, or a weight of at least LIBRARY_WEIGHT elements,
# decodes the weight once (mo_int8_decode) and runs the library GEMM on it, unless its
# reduction is at least LONG_REDUCTION times its output width and the fused kernels' launch
# plan splits that reduction (rows that do not fill a round of large tiles): there the fused
# kernels run. Any other call runs the fused kernels. Measured on MI355X, library time / fused
# time (forward, input gradient):
#   rows:                 256        512        1024       2048       4096       8192       17792
#   qkvo 3072x3072       1.19 0.84  0.97 1.07  0.98 1.10  0.90 0.93  0.89 0.75  0.91 0.89  0.86 0.90
#   up_gate 24576x3072   1.46 2.04  1.20 2.01  1.08 1.56  0.98 1.28  0.88 0.70  0.85 0.86  0.83 1.04
#   down 3072x12288      1.54 0.97  1.50 0.90  1.20 0.87  1.09 0.91  0.74 0.88  0.90 0.89  1.04 0.91
# The rule takes the fused kernels for up_gate's input gradient (24576-long reduction) and
# down's forward (12288) at 256-2048 and 17792 rows, where the library's GEMM runs its weakest
# and the split reduction fills the GPU; the library otherwise. On square and wide shapes the
# library's MFMA loop runs 10-15 % faster than the fused kernels' (which also decode each
# weight tile again for every row tile).
LIBRARY_ROWS = 2048
LIBRARY_WEIGHT = 16 << 20
LONG_REDUCTION = 4
PATHS = ("auto", "fused", "library")


def decode_hip(weight: torch.Tensor, scale: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """``decode(weight, scale, bfloat16)`` in one HIP pass (``mo_int8_decode``), bit for bit."""

    lib = _native.load()
    out_features, in_features = weight.shape
    out = _output(out, (out_features, in_features), weight.device, "decoded-weight")
    _native.check("mo_int8_decode", lib.mo_int8_decode(weight.data_ptr(), scale.data_ptr(), out.data_ptr(),
                                                       out_features, in_features, _stream(weight)))
    return out


def _library(rows: int, weight: torch.Tensor, path: str, reduction: int, width: int, split) -> bool:
    """Whether a call takes the library path; ``split()`` tells whether the fused plan splits a
    reduction (asked only when the rule needs it)."""

    if path not in PATHS:
        raise ValueError(f"path must be one of {PATHS}")
    if path != "auto":
        return path == "library"
    if rows < LIBRARY_ROWS and weight.numel() < LIBRARY_WEIGHT:
        return False
    return not (reduction >= LONG_REDUCTION * width and split())


def _stream(tensor: torch.Tensor) -> int:
    return torch.cuda.current_stream(tensor.device).cuda_stream


def _output(out: torch.Tensor | None, shape: tuple[int, int], device: torch.device, what: str) -> torch.Tensor:
    if out is None:
        return torch.empty(shape, dtype=torch.bfloat16, device=device)
    if out.dtype != torch.bfloat16 or not out.is_contiguous() or out.numel() != shape[0] * shape[1] \
            or out.device != device:
        raise ValueError(f"HIP {what} buffer has the wrong dtype, size or device, or is not contiguous.")
    return out.view(shape)


def int8_linear_forward(tokens: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor,
                        bias: torch.Tensor | None = None, *, out: torch.Tensor | None = None,
                        path: str = "auto") -> torch.Tensor:
    """``tokens @ decode(weight).T (+ bias)``; the call must be supported. ``path``: ``fused`` (the
    MFMA kernels), ``library`` (``decode_hip``, then the same ``addmm``/``mm`` as the reference's
    eager path, bit for bit), ``auto`` (library from ``LIBRARY_ROWS`` rows or ``LIBRARY_WEIGHT``
    weight elements up)."""

    lib = _native.load()
    matrix = tokens.reshape(-1, tokens.shape[-1]).contiguous()
    rows, in_features = matrix.shape
    out_features = weight.shape[0]
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
    nbytes = lib.mo_int8_forward_workspace_bytes(rows, in_features, out_features)
    if _library(rows, weight, path, in_features, out_features, lambda: nbytes > 0):
        decoded = decode_hip(weight, scale)
        if out is None:
            # the eager path's own call (F.linear): with an output buffer, PyTorch-ROCm picks
            # a different GEMM solution on some shapes, up to 15 % slower at qkvo's
            result = F.linear(matrix, decoded, bias)
        else:
            out = _output(out, (rows, out_features), tokens.device, "output")
            result = torch.mm(matrix, decoded.t(), out=out) if bias is None else \
                torch.addmm(bias, matrix, decoded.t(), out=out)
        return result.reshape(*tokens.shape[:-1], out_features)
    out = _output(out, (rows, out_features), tokens.device, "output")
    # fp32 partial sums of split reductions (freed to the caching allocator after the call;
    # stream order keeps them alive for the kernels)
    workspace = torch.empty(nbytes, dtype=torch.uint8, device=tokens.device) if nbytes else None
    _native.check(
        "mo_int8_linear_forward",
        lib.mo_int8_linear_forward(matrix.data_ptr(), weight.data_ptr(), scale.data_ptr(),
                                   0 if bias is None else bias.data_ptr(), out.data_ptr(), rows, in_features,
                                   out_features, 0 if workspace is None else workspace.data_ptr(), nbytes,
                                   _stream(tokens)),
    )
    return out.reshape(*tokens.shape[:-1], out_features)


def int8_linear_backward(gradient: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor,
                         input_shape: torch.Size, *, out: torch.Tensor | None = None,
                         path: str = "auto") -> torch.Tensor:
    """``gradient @ decode(weight)``: the input gradient of the frozen int8 linear (``path`` as in
    ``int8_linear_forward``)."""

    lib = _native.load()
    matrix = gradient.reshape(-1, gradient.shape[-1]).to(torch.bfloat16).contiguous()
    rows, out_features = matrix.shape
    in_features = weight.shape[1]
    nbytes = lib.mo_int8_backward_workspace_bytes(rows, in_features, out_features)
    transposed = (in_features * out_features + 255) // 256 * 256
    if _library(rows, weight, path, out_features, in_features, lambda: nbytes > transposed):
        if out is None:  # the eager path's call (see int8_linear_forward)
            return matrix.matmul(decode_hip(weight, scale)).reshape(input_shape)
        out = _output(out, (rows, in_features), gradient.device, "input-gradient")
        torch.mm(matrix, decode_hip(weight, scale), out=out)
        return out.reshape(input_shape)
    out = _output(out, (rows, in_features), gradient.device, "input-gradient")
    # the transposed int8 weight for the large tiles and the partial sums of split reductions
    # (freed to the caching allocator after the call; stream order keeps it alive for the kernels)
    workspace = torch.empty(nbytes, dtype=torch.uint8, device=gradient.device)
    _native.check(
        "mo_int8_linear_backward",
        lib.mo_int8_linear_backward(matrix.data_ptr(), weight.data_ptr(), scale.data_ptr(), out.data_ptr(), rows,
                                    in_features, out_features, workspace.data_ptr(), nbytes, _stream(gradient)),
    )
    return out.reshape(input_shape)


def launch_plan(rows: int, cols: int, reduction: int, cus: int, kernel: str = "registers") -> list[dict]:
    """The fused kernels' launches for a call with a workspace (``mo_int8_launch_plan``): ``cols``
    output columns (out_features for the forward, in_features for the input gradient) from a
    ``reduction`` (in_features, or out_features) on a device of ``cus`` CUs. Each part is
    ``{"tile": "large" | "small" | "split", "row0", "rows", "splits", "split_steps"}``."""

    import ctypes

    lib = _native.load()
    code = {"registers": _native.MO_INT8_KERNEL_REGISTERS, "lds": _native.MO_INT8_KERNEL_LDS}[kernel]
    n = ctypes.c_uint32(0)
    raw = (ctypes.c_uint32 * 10)()
    _native.check("mo_int8_launch_plan", lib.mo_int8_launch_plan(rows, cols, reduction, cus, code, ctypes.byref(n), raw))
    names = ("large", "small", "split")
    return [{"tile": names[raw[5 * i]], "row0": raw[5 * i + 1], "rows": raw[5 * i + 2], "splits": raw[5 * i + 3],
             "split_steps": raw[5 * i + 4]} for i in range(n.value)]


def set_kernel(kernel: str) -> None:
    """Which kernel takes the large tiles of the fused path, process-wide: ``registers`` (default:
    weights decoded in registers, activations through LDS) or ``lds`` (the weight tile decoded
    into LDS). Same results bit for bit; for measuring one against the other."""

    code = {"registers": _native.MO_INT8_KERNEL_REGISTERS, "lds": _native.MO_INT8_KERNEL_LDS}[kernel]
    _native.check("mo_int8_set_kernel", _native.load().mo_int8_set_kernel(code))


# ---- the reference module's interface (training/quant_kernels.py), same names and meaning ----

def validate_quantized_backend(backend: str) -> str:
    """``auto``, ``eager`` or ``triton`` (reference ``quant_kernels.py:30-33``)."""

    if backend not in {"auto", "eager", "triton"}:
        raise ValueError("quantized backend must be auto, eager or triton.")
    return backend


def triton_is_available() -> bool:
    """Whether the fused-kernel backend can run: the HIP library loads and a HIP device is
    present (reference ``quant_kernels.py:36-38``, with the HIP kernels in place of Triton)."""

    if not torch.cuda.is_available():
        return False
    try:
        _native.load()
    except (OSError, RuntimeError):
        return False
    return True


def resolve_quantized_backend(backend: str, tokens: torch.Tensor, weight: torch.Tensor,
                              scale: torch.Tensor) -> str:
    """``auto`` -> ``triton`` when the fused kernels support the call, else ``eager``; an explicit
    ``triton`` must be supported (reference ``quant_kernels.py:64-79``). The weight dtype is
    the input's, as the reference's callers convert the input to it before the kernel."""

    selected = validate_quantized_backend(backend)
    if selected == "eager":
        return selected
    reason = unsupported_reason(tokens, weight, scale, tokens.dtype)
    if reason is None and not triton_is_available():
        reason = "the HIP library or device is unavailable"
    if selected == "auto":
        return "eager" if reason is not None else "triton"
    if reason is not None:
        raise RuntimeError(f"Triton quantized backend is unavailable: {reason}.")
    return selected


def autocast_compute_dtype(tokens: torch.Tensor, module_dtype: torch.dtype) -> torch.dtype:
    """The dtype autocast gives a linear on ``tokens`` (reference ``quant_kernels.py:82-96``)."""

    if tokens.device.type != "cuda" or not torch.is_autocast_enabled("cuda"):
        return module_dtype
    return torch.get_autocast_dtype("cuda")


def triton_int8_linear_forward(tokens: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor,
                               bias: torch.Tensor | None, output_dtype: torch.dtype, weight_dtype: torch.dtype,
                               *, out: torch.Tensor | None = None) -> torch.Tensor:
    """Reference ``quant_kernels.py:294-334`` on the HIP kernel: bf16 output and weight dtype."""

    if output_dtype != torch.bfloat16 or weight_dtype != torch.bfloat16:
        raise TypeError(f"HIP int8 kernels compute in bf16 (got output {output_dtype}, weight {weight_dtype}).")
    if bias is not None and (bias.device != tokens.device or not bias.is_contiguous()):
        raise RuntimeError("Triton quantized bias must be contiguous and on the input device.")
    return int8_linear_forward(tokens, weight, scale, bias, out=out)


def triton_int8_linear_backward(gradient: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor,
                                input_shape: torch.Size, input_dtype: torch.dtype, weight_dtype: torch.dtype,
                                *, out: torch.Tensor | None = None) -> torch.Tensor:
    """Reference ``quant_kernels.py:337-373`` on the HIP kernel: the input gradient only."""

    if input_dtype != torch.bfloat16 or weight_dtype != torch.bfloat16:
        raise TypeError(f"HIP int8 kernels compute in bf16 (got input {input_dtype}, weight {weight_dtype}).")
    return int8_linear_backward(gradient.contiguous(), weight, scale, input_shape, out=out)

