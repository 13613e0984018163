"""CPU checks of moss_offload.quant_kernels' backend selection (no kernel runs here).

The module keeps the reference's interface for the int8 path under its own names
(training/quant_kernels.py:30-99, 294-374), which training/quantization.py imports; ``triton``
is the reference's name for the fused-kernel backend, here the HIP kernels. The HIP kernels
need a HIP device, so every call on CPU tensors resolves ``auto`` to the eager path and an
explicit fused-kernel request raises, as the reference does without CUDA.
"""

from __future__ import annotations

import pytest
import torch

from moss_offload import quant_kernels as qk


def _operands(dtype=torch.bfloat16, in_f=32, out_f=16):
    return torch.randn(4, in_f).to(dtype), torch.zeros(out_f, in_f, dtype=torch.int8), torch.ones(out_f)


def test_reference_interface_names_exist() -> None:
    for name in ("validate_quantized_backend", "resolve_quantized_backend", "autocast_compute_dtype",
                 "triton_is_available", "triton_int8_linear_forward", "triton_int8_linear_backward"):
        assert callable(getattr(qk, name)), name


def test_validate_quantized_backend_matches_the_reference_contract() -> None:
    for name in ("auto", "eager", "triton"):
        assert qk.validate_quantized_backend(name) == name
    with pytest.raises(ValueError, match="auto, eager or triton"):
        qk.validate_quantized_backend("hip")  # the reference's names only
    with pytest.raises(ValueError, match="auto, eager or hip"):
        qk.resolve_backend("cuda-graph", *_operands(), torch.bfloat16)


def test_cpu_calls_resolve_to_eager_and_fused_requests_raise() -> None:
    x, w, s = _operands()
    assert qk.resolve_quantized_backend("auto", x, w, s) == "eager"
    assert qk.resolve_quantized_backend("eager", x, w, s) == "eager"
    with pytest.raises(RuntimeError, match="Triton quantized backend is unavailable: the input is not on a HIP device"):
        qk.resolve_quantized_backend("triton", x, w, s)
    assert qk.resolve_backend("auto", x, w, s, torch.bfloat16) == "eager"
    with pytest.raises(RuntimeError, match="HIP int8 backend is unavailable"):
        qk.resolve_backend("hip", x, w, s, torch.bfloat16)


def test_device_is_checked_first() -> None:
    x, w, s = _operands()
    assert qk.unsupported_reason(x, w, s, torch.bfloat16) == "the input is not on a HIP device"
    assert qk.unsupported_reason(x.float(), w, s, torch.float32) == "the input is not on a HIP device"


def test_autocast_compute_dtype_off_cuda_is_the_module_dtype() -> None:
    x, _, _ = _operands(torch.float32)
    assert qk.autocast_compute_dtype(x, torch.bfloat16) == torch.bfloat16
    assert qk.decode(torch.tensor([[3, -2]], dtype=torch.int8), torch.tensor([0.5]), torch.bfloat16).tolist() == [[1.5, -1.0]]
