"""Weight-only int8 linear on MFMA: drop-in for the Triton path of MOSS-Image's
``training/quant_kernels.py`` (:100-228, ``triton_int8_linear_forward/backward``).

The GEMMs are hand-written gfx950 kernels in ``csrc/mo_gemm.hip`` (bf16 MFMA, int8 tiles
decoded to bf16 on their way into LDS), reached through ``mo_int8_linear_forward`` and
``mo_int8_linear_backward``. Backend selection mirrors the reference's ``auto | eager | triton``
with ``hip`` in place of ``triton``: ``auto`` takes the HIP kernels whenever the call is
supported (bf16 activations and weight dtype on a HIP device, int8 weights, fp32 scales,
feature sizes multiples of 16, contiguous operands) and the eager path otherwise; an explicit
``hip`` request that is not supported raises. The eager path is the reference's own eager
backend (decode the weight, then ``F.linear``), not a substitute for a missing library.
"""

from __future__ import annotations

import torch

from . import _native

BACKENDS = {"auto", "eager", "hip"}


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


def _stream(tensor: torch.Tensor) -> int:
    return torch.cuda.current_stream(tensor.device).cuda_stream


def int8_linear_forward(tokens: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor,
                        bias: torch.Tensor | None = None) -> torch.Tensor:
    """``tokens @ decode(weight).T (+ bias)`` on the HIP kernel; the call must be supported."""

    lib = _native.load()
    matrix = tokens.reshape(-1, tokens.shape[-1]).contiguous()
    rows, in_features = matrix.shape
    out_features = weight.shape[0]
    out = torch.empty((rows, out_features), dtype=torch.bfloat16, device=tokens.device)
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
    _native.check(
        "mo_int8_linear_forward",
        lib.mo_int8_linear_forward(matrix.data_ptr(), weight.data_ptr(), scale.data_ptr(),
                                   0 if bias is None else bias.data_ptr(), out.data_ptr(), rows, in_features,
                                   out_features, _stream(tokens)),
    )
    return out.reshape(*tokens.shape[:-1], out_features)


def int8_linear_backward(gradient: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor,
                         input_shape: torch.Size) -> torch.Tensor:
    """``gradient @ decode(weight)``: the input gradient of the frozen int8 linear."""

    lib = _native.load()
    matrix = gradient.reshape(-1, gradient.shape[-1]).to(torch.bfloat16).contiguous()
    rows, out_features = matrix.shape
    in_features = weight.shape[1]
    out = torch.empty((rows, in_features), dtype=torch.bfloat16, device=gradient.device)
    _native.check(
        "mo_int8_linear_backward",
        lib.mo_int8_linear_backward(matrix.data_ptr(), weight.data_ptr(), scale.data_ptr(), out.data_ptr(), rows,
                                    in_features, out_features, _stream(gradient)),
    )
    return out.reshape(input_shape)
