"""Async frozen-block streaming on the GPU: a streamed LoRA model trains like a resident one.

Restates the scenarios of the reference's training/tests/test_async_memory.py (seeds 83-113,
same tiny model sizes and tolerances) against moss_offload.memory: dense, bf16 and int8 bases;
two optimizer steps; grad-enabled eval; two live graphs with one backward; autograd.grad;
retained graphs; a failing recomputation followed by a fresh placement; teardown by CPU
placement. The streamer's slot fills run on an SDMA engine; masters live in one pinned arena.
"""

from __future__ import annotations

import copy
import gc

import pytest
import torch

import moss_offload
from moss_offload import dit
from moss_offload.memory import AsyncBlockStreamer, place_model

from gpu_util import assert_bitwise, requires_gpu

pytestmark = requires_gpu


def _tiny(dtype=torch.float32):
    return dit.MOSSImageTransformer(
        dim=32, ffn_dim=64, num_heads=4, num_layers=4, text_dim=16, freq_dim=8, latent_channels=4,
        gradient_checkpointing=True,
    ).to(dtype=dtype)


def _prepare(quantization: str, dtype) -> dit.MOSSImageTransformer:
    model = _tiny(dtype)
    dit.init_weights(model)
    if quantization == "int8":
        dit.quantize_joint_linears(model, torch.Generator().manual_seed(5))
    dit.inject_lora(model, rank=2, alpha=4.0, b_std=0.03)
    return model


def _frozen(model):
    tensors = {f"p.{n}": p for n, p in model.layers.named_parameters() if not p.requires_grad}
    tensors.update({f"b.{n}": b for n, b in model.layers.named_buffers()})
    return tensors


def _trainables(model):
    return {n: p for n, p in model.named_parameters() if p.requires_grad}


def _inputs(device, dtype):
    return [
        {"hidden_states": torch.randn(1, 4, 4, 4, device=device, dtype=dtype), "timestep": torch.tensor([250.0], device=device),
         "encoder_hidden_states": torch.randn(1, 3, 16, device=device, dtype=dtype)},
        {"hidden_states": torch.randn(1, 4, 3, 5, device=device, dtype=dtype), "timestep": torch.tensor([750.0], device=device),
         "encoder_hidden_states": torch.randn(1, 4, 16, device=device, dtype=dtype)},
    ]


def _optimization_step(model, optimizer, batches, autocast):
    optimizer.zero_grad(set_to_none=True)
    outputs = []
    for batch in batches:
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            output = model(**batch)
            loss = output.float().square().mean() / 2
        outputs.append(output.detach().cpu())
        loss.backward()
    params = _trainables(model)
    assert params and all(p.grad is not None and torch.isfinite(p.grad).all() for p in params.values())
    assert all(torch.count_nonzero(p.grad).item() > 0 for n, p in params.items() if n.endswith("lora_A"))
    grads = {n: p.grad.detach().cpu().clone() for n, p in params.items()}
    optimizer.step()
    return outputs, grads, {n: p.detach().cpu().clone() for n, p in params.items()}


def _close(actual, expected, atol, rtol):
    assert actual.keys() == expected.keys()
    for name in actual:
        torch.testing.assert_close(actual[name], expected[name], atol=atol, rtol=rtol, msg=lambda m: f"{name}: {m}")


@pytest.mark.parametrize("precision,quantization", [("fp32", "dense"), ("bf16", "dense"), ("fp32", "int8"), ("bf16", "int8")])
def test_async_frozen_lora_matches_resident_training_and_eval(precision, quantization) -> None:
    torch.manual_seed(83)
    dtype = torch.bfloat16 if precision == "bf16" else torch.float32
    resident = _prepare(quantization, dtype).train()
    streamed = copy.deepcopy(resident).train()
    frozen_before = {n: t.detach().clone() for n, t in _frozen(streamed).items()}
    adapter_ids = {n: id(p) for n, p in _trainables(streamed).items()}
    device = torch.device("cuda", 0)
    place_model(resident, device, 0)
    place_model(streamed, device, len(streamed.layers), block_swap_mode="async")
    manager = streamed.block_swap_manager
    assert isinstance(manager, AsyncBlockStreamer)
    assert {n: id(p) for n, p in _trainables(streamed).items()} == adapter_ids
    assert all(p.device.type == "cuda" for p in _trainables(streamed).values())
    placed = _frozen(streamed)
    assert placed.keys() == frozen_before.keys()
    assert all(t.device.type == "cpu" and (t.numel() == 0 or t.is_pinned()) for t in placed.values())
    int8 = [n for n in placed if n.endswith("weight_int8")]
    assert bool(int8) == (quantization == "int8") and all(placed[n].dtype == torch.int8 for n in int8)

    opt_r = torch.optim.AdamW(_trainables(resident).values(), lr=2e-3)
    opt_s = torch.optim.AdamW(_trainables(streamed).values(), lr=2e-3)
    atol, rtol = (4e-3, 3e-2) if precision == "bf16" else (2e-5, 2e-3)
    for step in range(2):
        torch.manual_seed(200 + step)
        batches = _inputs(device, dtype)
        r = _optimization_step(resident, opt_r, batches, precision == "bf16")
        s = _optimization_step(streamed, opt_s, batches, precision == "bf16")
        for a, b in zip(s[0], r[0]):
            torch.testing.assert_close(a, b, atol=atol, rtol=rtol)
        _close(s[1], r[1], atol, rtol)
        _close(s[2], r[2], atol, rtol)
        if step == 0:
            resident.eval()
            streamed.eval()
            negative = dict(batches[1], encoder_hidden_states=-batches[1]["encoder_hidden_states"])
            with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=precision == "bf16"):
                rc, ru = resident(**batches[1]), resident(**negative, skip_layers=(1, 3))
                sc, su = streamed(**batches[1]), streamed(**negative, skip_layers=(1, 3))
            torch.testing.assert_close(sc, rc, atol=atol, rtol=rtol)
            torch.testing.assert_close(su, ru, atol=atol, rtol=rtol)
            resident.train()
            streamed.train()
    assert 1 <= manager.peak_resident_blocks <= 2
    assert manager.h2d_copy_count > 0
    stats = manager.stats()
    assert stats["fills"] == manager.h2d_copy_count and stats["copy_failures"] == 0
    frozen_after = _frozen(streamed)
    for name, original in frozen_before.items():
        assert frozen_after[name].device.type == "cpu"
        assert torch.equal(frozen_after[name], original), name


def test_streamed_forward_is_bitwise_the_resident_forward() -> None:
    torch.manual_seed(84)
    resident = _prepare("dense", torch.float32).train()
    streamed = copy.deepcopy(resident).train()
    device = torch.device("cuda", 0)
    place_model(resident, device, 0)
    place_model(streamed, device, 4, block_swap_mode="async")
    batch = _inputs(device, torch.float32)[1]
    with torch.no_grad():
        assert_bitwise(streamed(**batch), resident(**batch))


def test_partial_async_swap_supports_two_live_graphs_and_one_backward() -> None:
    torch.manual_seed(97)
    resident = _prepare("dense", torch.float32).train()
    streamed = copy.deepcopy(resident).train()
    device = torch.device("cuda", 0)
    place_model(resident, device, 0)
    place_model(streamed, device, 2, block_swap_mode="async")
    for layer in streamed.layers[:2]:
        assert all(p.device.type == "cuda" for p in layer.parameters())
    for layer in streamed.layers[2:]:
        assert all(p.device.type == ("cuda" if p.requires_grad else "cpu") for p in layer.parameters())
    batches = _inputs(device, torch.float32)
    results = []
    for model in (resident, streamed):
        opt = torch.optim.AdamW(_trainables(model).values(), lr=2e-3)
        opt.zero_grad(set_to_none=True)
        outputs = [model(**b) for b in batches]
        sum(o.float().square().mean() / len(outputs) for o in outputs).backward()
        grads = {n: p.grad.detach().cpu().clone() for n, p in _trainables(model).items()}
        opt.step()
        results.append(([o.detach().cpu() for o in outputs], grads))
    for a, b in zip(results[1][0], results[0][0]):
        torch.testing.assert_close(a, b, atol=2e-5, rtol=2e-3)
    _close(results[1][1], results[0][1], 2e-5, 2e-3)
    assert 1 <= streamed.block_swap_manager.peak_resident_blocks <= 2


def test_grad_enabled_eval_forward_backpropagates_through_four_streamed_blocks() -> None:
    torch.manual_seed(101)
    resident = _prepare("dense", torch.float32).eval()
    streamed = copy.deepcopy(resident).eval()
    device = torch.device("cuda", 0)
    place_model(resident, device, 0)
    place_model(streamed, device, 4, block_swap_mode="async")
    batch = _inputs(device, torch.float32)[0]
    r, s = resident(**batch), streamed(**batch)
    assert r.grad_fn is not None and s.grad_fn is not None
    r.float().square().mean().backward()
    s.float().square().mean().backward()
    torch.testing.assert_close(s, r, atol=2e-5, rtol=2e-3)
    _close({n: p.grad.cpu() for n, p in _trainables(streamed).items()},
           {n: p.grad.cpu() for n, p in _trainables(resident).items()}, 2e-5, 2e-3)


def test_autograd_grad_releases_blocks_for_next_iteration_and_teardown() -> None:
    torch.manual_seed(103)
    model = _prepare("dense", torch.float32).train()
    device = torch.device("cuda", 0)
    place_model(model, device, 4, block_swap_mode="async")
    manager = model.block_swap_manager
    params = _trainables(model)
    opt = torch.optim.AdamW(params.values(), lr=2e-3)
    batches = _inputs(device, torch.float32)
    grads = torch.autograd.grad(model(**batches[0]).float().square().mean(), tuple(params.values()))
    assert len(grads) == len(params) and all(torch.isfinite(g).all() for g in grads)
    assert all(p.grad is None for p in params.values())
    opt.zero_grad(set_to_none=True)
    model(**batches[1]).float().square().mean().backward()
    assert all(p.grad is not None and torch.isfinite(p.grad).all() for p in params.values())
    opt.step()
    place_model(model, torch.device("cpu"), 0)
    assert manager.closed and manager.resident_block_indices == ()
    assert model.block_swap_manager is None
    assert all(p.device.type == "cpu" for p in model.parameters())


def test_retained_graph_supports_two_backward_traversals() -> None:
    torch.manual_seed(107)
    model = _prepare("dense", torch.float32).train()
    device = torch.device("cuda", 0)
    place_model(model, device, 4, block_swap_mode="async")
    params = _trainables(model)
    loss = model(**_inputs(device, torch.float32)[0]).float().square().mean()
    loss.backward(retain_graph=True)
    first = {n: p.grad.detach().clone() for n, p in params.items()}
    loss.backward()
    for n, p in params.items():
        torch.testing.assert_close(p.grad, first[n] * 2, atol=2e-5, rtol=2e-3)


def test_recompute_exception_allows_cleanup_and_fresh_placement() -> None:
    torch.manual_seed(109)
    model = _prepare("dense", torch.float32).train()
    device = torch.device("cuda", 0)
    place_model(model, device, 4, block_swap_mode="async")
    failed = model.block_swap_manager
    layer = model.layers[-1]
    original = layer.forward
    calls = 0

    def fail_during_recompute(*args, **kwargs):
        nonlocal calls
        calls += 1
        if calls == 2:
            raise RuntimeError("recompute failure")
        return original(*args, **kwargs)

    layer.forward = fail_during_recompute
    loss = model(**_inputs(device, torch.float32)[0]).float().square().mean()
    try:
        with pytest.raises(RuntimeError, match="recompute failure"):
            loss.backward()
    finally:
        layer.forward = original
    assert calls == 2
    del loss
    gc.collect()
    place_model(model, torch.device("cpu"), 0)
    assert failed.closed and failed.resident_block_indices == () and model.block_swap_manager is None
    place_model(model, device, 4, block_swap_mode="async")
    recovered = model.block_swap_manager
    assert recovered is not failed
    model.zero_grad(set_to_none=True)
    model(**_inputs(device, torch.float32)[1]).float().square().mean().backward()
    assert all(p.grad is not None and torch.isfinite(p.grad).all() for p in _trainables(model).values())
    place_model(model, torch.device("cpu"), 0)
    assert recovered.closed


def test_cpu_placement_closes_manager_after_eval_prefetch() -> None:
    torch.manual_seed(113)
    model = _prepare("dense", torch.float32).eval()
    device = torch.device("cuda", 0)
    place_model(model, device, 4, block_swap_mode="async")
    manager = model.block_swap_manager
    assert manager.h2d_copy_count == 0
    with torch.no_grad():
        output = model(**_inputs(device, torch.float32)[0])
    assert output.is_cuda and manager.resident_block_indices
    assert manager.h2d_copy_count == len(model.layers)
    place_model(model, torch.device("cpu"), 0)
    assert manager.closed and manager.resident_block_indices == () and model.block_swap_manager is None
    assert all(p.device.type == "cpu" for p in model.parameters())
    assert all(b.device.type == "cpu" for b in model.buffers())


def test_activation_offload_with_async_streaming_keeps_slots_resident() -> None:
    """The low-VRAM combination: streamed frozen int8 blocks plus offloaded activations. The
    staging slots count as weight-backed (never offloaded), and training matches the resident
    model without offload."""

    torch.manual_seed(115)
    resident = _prepare("int8", torch.bfloat16).train()
    streamed = copy.deepcopy(resident).train()
    device = torch.device("cuda", 0)
    place_model(resident, device, 0)
    place_model(streamed, device, 4, block_swap_mode="async")
    streamed.activation_offload = True
    batches = _inputs(device, torch.bfloat16)
    r = _optimization_step(resident, torch.optim.AdamW(_trainables(resident).values(), lr=2e-3), batches, True)
    s = _optimization_step(streamed, torch.optim.AdamW(_trainables(streamed).values(), lr=2e-3), batches, True)
    for a, b in zip(s[0], r[0]):
        torch.testing.assert_close(a, b, atol=4e-3, rtol=3e-2)
    _close(s[1], r[1], 4e-3, 3e-2)
    slots = streamed.block_swap_manager.owned_cuda_buffers()
    assert slots
    ctx = moss_offload.activation_cpu_offload(streamed, True, device)
    assert all(ctx.is_weight_backed(slot[64:128]) for slot in slots)
    assert moss_offload.get_engine(device).stats()["bytes_packed"] > 0
