"""CPU tests of block placement (moss_offload.memory, drop-in for training/memory.py).

Validation runs before anything is moved, as in the reference (training/memory.py:366-413;
its tests training/tests/test_async_memory.py:429-447). Synchronous swapping runs entirely on
the CPU: a model whose last blocks are swapped with ``offloaded_block`` computes exactly what
the resident model computes.
"""

from __future__ import annotations

import copy

import pytest
import torch

from moss_offload import dit
from moss_offload.memory import offloaded_block, place_model


def _tiny(layers=4):
    return dit.MOSSImageTransformer(
        dim=32, ffn_dim=64, num_heads=4, num_layers=layers, text_dim=16, freq_dim=8, latent_channels=4,
        gradient_checkpointing=True,
    )


def _lora(model):
    dit.init_weights(model)
    dit.inject_lora(model, rank=2, alpha=4.0, b_std=0.03)
    return model


def test_async_rejects_full_training_before_mutating_the_model() -> None:
    model = _tiny()
    ids = {name: id(p) for name, p in model.named_parameters()}
    with pytest.raises(ValueError, match="H2D-only.*frozen base weights"):
        place_model(model, torch.device("cuda"), 2, block_swap_mode="async")
    assert {name: id(p) for name, p in model.named_parameters()} == ids
    assert all(p.device.type == "cpu" for p in model.parameters())
    assert not hasattr(model, "block_swap_manager")


def test_async_rejects_cpu_and_unknown_mode_before_mutating_the_model() -> None:
    model = _lora(_tiny())
    ids = {name: id(p) for name, p in model.named_parameters() if p.requires_grad}
    with pytest.raises(ValueError, match="requires a CUDA device"):
        place_model(model, torch.device("cpu"), 2, block_swap_mode="async")
    with pytest.raises(ValueError, match="block_swap_mode must be 'sync' or 'async'"):
        place_model(model, torch.device("cpu"), 2, block_swap_mode="overlap")
    with pytest.raises(ValueError, match="blocks_to_swap must be between"):
        place_model(model, torch.device("cpu"), 5, block_swap_mode="sync")
    with pytest.raises(ValueError, match="async_full requires at least one trainable"):
        frozen = _tiny()
        for p in frozen.parameters():
            p.requires_grad_(False)
        place_model(frozen, torch.device("cuda"), 2, block_swap_mode="async_full")
    assert {name: id(p) for name, p in model.named_parameters() if p.requires_grad} == ids
    assert all(p.device.type == "cpu" for p in model.parameters())
    assert not hasattr(model, "block_swap_manager")


def _step(model, latent, context, t):
    model.zero_grad(set_to_none=True)
    out = model(latent, t, context)
    out.float().square().mean().backward()
    grads = {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None}
    return out.detach(), grads


def test_sync_swapping_matches_resident_model_bitwise() -> None:
    torch.manual_seed(91)
    resident = _lora(_tiny()).train()
    swapped = copy.deepcopy(resident).train()
    place_model(resident, torch.device("cpu"), 0)
    place_model(swapped, torch.device("cpu"), 2, block_swap_mode="sync")
    assert swapped.blocks_to_swap == 2 and swapped.block_swap_manager is None
    g = torch.Generator().manual_seed(3)
    latent, context, t = torch.randn(1, 4, 3, 5, generator=g), torch.randn(1, 4, 16, generator=g), torch.tensor([400.0])
    expected = _step(resident, latent, context, t)
    actual = _step(swapped, latent, context, t)
    assert torch.equal(actual[0], expected[0])
    assert actual[1].keys() == expected[1].keys() and len(actual[1]) > 0
    for name in expected[1]:
        assert torch.equal(actual[1][name], expected[1][name]), name
    # skipping layers skips swapped and resident blocks alike
    with torch.no_grad():
        a = swapped(latent, t, context, skip_layers=(1, 3))
        b = resident(latent, t, context, skip_layers=(1, 3))
    assert torch.equal(a, b)


def test_offloaded_block_copies_parameters_to_the_input_device_each_call() -> None:
    torch.manual_seed(92)
    layer = torch.nn.Linear(8, 8)
    x = torch.randn(2, 8, requires_grad=True)
    y = offloaded_block(layer, x)
    y.sum().backward()
    torch.testing.assert_close(y, layer(x))
    assert layer.weight.grad is not None and x.grad is not None
    with torch.no_grad():
        assert torch.equal(offloaded_block(layer, x), layer(x))


def test_trainable_streamer_rejects_non_cuda_without_initializing_cuda() -> None:
    from moss_offload.trainable_offload import TrainableBlockStreamer

    model = _tiny()
    with pytest.raises(ValueError, match="requires a CUDA device"):
        TrainableBlockStreamer(model.layers, "cpu")
    with pytest.raises(ValueError, match="requires a CUDA device"):
        place_model(model, torch.device("cpu"), 2, block_swap_mode="async_full")
    assert all(p.device.type == "cpu" for p in model.parameters())


def test_async_full_rejects_shared_and_integer_parameters_before_mutating() -> None:
    model = _tiny()
    model.layers[3].proj["q"].weight = model.layers[2].proj["q"].weight
    with pytest.raises(ValueError, match="shared across streamed blocks"):
        place_model(model, torch.device("cuda"), 2, block_swap_mode="async_full")
    model = _tiny()
    model.layers[3].register_parameter("steps", torch.nn.Parameter(torch.zeros(2, dtype=torch.int64), requires_grad=False))
    with pytest.raises(TypeError, match="non-floating parameter"):
        place_model(model, torch.device("cuda"), 2, block_swap_mode="async_full")
    assert not hasattr(model, "block_swap_manager")
