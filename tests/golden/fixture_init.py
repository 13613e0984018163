"""Deterministic parameters and inputs shared by the reference-fixture writer and its test.

``make_reference_fixtures.py`` applies these to the reference model (imported in the build
container only) and records what autograd saves and what a step computes; the CPU test
applies the same rule to the harness model in ``moss_offload/dit.py`` and compares. Both
models use the released state-dict names, so one rule keyed by parameter name gives both the
same values, whatever order or default initialiser either constructor uses.

The rule is chosen so that a dropped term shows: norm scales are 1 + N(0, 0.1) instead of
exactly 1, biases are N(0, 0.02) instead of 0, and LoRA B is N(0, 0.03) instead of the
reference's zeros (which would zero every LoRA A gradient).

This module imports neither the reference nor the product.
"""

from __future__ import annotations

import zlib

import torch

# one joint block, hidden 512, 8 heads x 64, MLP 2048, fp32, batch 1,
# 16 x 16 image tokens and 64 text tokens. text_dim / freq_dim / latent channels are the
# harness's small choices (they only size the embedders around the block).
CONFIG1 = dict(dim=512, ffn_dim=2048, num_heads=8, num_layers=1, text_dim=64, freq_dim=32, latent_channels=16)
LORA_RANK = 8
LORA_ALPHA = 16.0  # scale alpha / rank = 2, so a dropped LoRA scale shows
TIMESTEP = 500.0
IMAGE = (16, 16)
TEXT_TOKENS = 64


def init_parameters(model: torch.nn.Module) -> None:
    """Set every parameter from a generator seeded by the CRC-32 of its name."""

    with torch.no_grad():
        for name, parameter in sorted(model.named_parameters()):
            generator = torch.Generator().manual_seed(zlib.crc32(name.encode()))
            noise = torch.randn(parameter.shape, generator=generator, dtype=torch.float32)
            if name.endswith("lora_B"):
                value = noise * 0.03
            elif name.endswith("lora_A") or parameter.dim() >= 2:
                value = noise * 0.02
            elif "norm" in name:
                value = 1.0 + 0.1 * noise
            else:
                value = noise * 0.02
            parameter.copy_(value.to(parameter.dtype))


def inputs(latent_channels: int = CONFIG1["latent_channels"], text_dim: int = CONFIG1["text_dim"]):
    """Latents ``[1, C, 16, 16]`` and text states ``[1, 64, text_dim]``, N(0, 1), seed 0."""

    generator = torch.Generator().manual_seed(0)
    latent = torch.randn(1, latent_channels, *IMAGE, generator=generator)
    context = torch.randn(1, TEXT_TOKENS, text_dim, generator=generator)
    return latent, context


def parameter_checksums(model: torch.nn.Module) -> dict[str, list[float]]:
    """Per parameter: float64 sum and sum of squares (to detect a different initialisation)."""

    out = {}
    for name, parameter in sorted(model.named_parameters()):
        value = parameter.detach().double()
        out[name] = [float(value.sum()), float(value.square().sum())]
    return out


class SaveRecorder:
    """Saved-tensor hooks that record what autograd saves, then return the tensor unchanged.

    Per save: shape, stride, storage offset, dtype, device type, whether its storage belongs to
    a parameter or buffer of the model (the reference's resident rule), and the index of the
    first save with the same storage ("storage group") and with the same storage, offset, shape
    and stride ("view group").
    """

    def __init__(self, model: torch.nn.Module) -> None:
        self.records: list[dict] = []
        self._storages: dict[int, int] = {}
        self._views: dict[tuple, int] = {}
        self._resident = {
            t.untyped_storage().data_ptr() for t in (*model.parameters(), *model.buffers()) if t.untyped_storage().nbytes()
        }

    def hooks(self):
        return torch.autograd.graph.saved_tensors_hooks(self._pack, lambda saved: saved)

    def _pack(self, tensor: torch.Tensor) -> torch.Tensor:
        index = len(self.records)
        ptr = tensor.untyped_storage().data_ptr()
        view_key = (ptr, tensor.storage_offset(), tuple(tensor.shape), tuple(tensor.stride()), tensor.dtype)
        self.records.append(
            dict(
                shape=list(tensor.shape),
                stride=list(tensor.stride()),
                offset=int(tensor.storage_offset()),
                dtype=str(tensor.dtype).replace("torch.", ""),
                device=tensor.device.type,
                resident=ptr in self._resident,
                storage_group=self._storages.setdefault(ptr, index),
                view_group=self._views.setdefault(view_key, index),
            )
        )
        return tensor
