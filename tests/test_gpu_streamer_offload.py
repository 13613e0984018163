"""Activation offload combined with block swapping, on the GPU.

Restates the two combination scenarios of the reference (training/tests/test_packed_cuda.py:
173-231, seeds 903 and 904, three layers, two swapped, one packed traversal of two samples):

- frozen-block swapping (sync and async) with activation offload matches the same placement
  without offload, within the reference's fp32 tolerance (rtol 5e-5, atol 5e-6); the async
  streamer's slots are weight storage the hook never offloads;
- the trainable ring (``async_full``) with activation offload: the streamed forward matches a
  resident model, backward runs the in-backward optimizer through both streamed blocks, and
  both are written back to their masters.
"""

from __future__ import annotations

import copy
import gc

import pytest
import torch

import moss_offload
from moss_offload import dit
from moss_offload.memory import place_model

from gpu_util import requires_gpu

pytestmark = requires_gpu


def _tiny(layers=3):
    model = dit.MOSSImageTransformer(
        dim=32, ffn_dim=64, num_heads=4, num_layers=layers, text_dim=16, freq_dim=8, latent_channels=4,
        gradient_checkpointing=True,
    )
    dit.init_weights(model, std=0.05)
    return model


def _inputs(device, seed=902):
    g = torch.Generator().manual_seed(seed)
    targets = [torch.randn(4, 3, 5, generator=g).to(device).requires_grad_(),
               torch.randn(4, 2, 4, generator=g).to(device).requires_grad_()]
    contexts = [torch.randn(5, 16, generator=g).to(device), torch.randn(3, 16, generator=g).to(device)]
    return targets, torch.tensor([250.0, 750.0], device=device), contexts


def _clone(inputs):
    targets, t, contexts = inputs
    return [x.detach().clone().requires_grad_() for x in targets], t.clone(), [c.clone() for c in contexts]


def _packed_backward(model, inputs):
    targets, t, contexts = inputs
    outputs = model.forward_packed(targets, t, contexts)
    sum(o.float().square().mean() for o in outputs).backward()
    grads = {n: p.grad.detach().cpu().clone() for n, p in model.named_parameters() if p.grad is not None}
    return [o.detach().cpu() for o in outputs], grads, [x.grad.detach().cpu() for x in targets]


def _assert_close(actual, expected, rtol=5e-5, atol=5e-6):
    outs, grads, input_grads = actual
    e_outs, e_grads, e_input_grads = expected
    for a, b in zip(outs + input_grads, e_outs + e_input_grads):
        torch.testing.assert_close(a, b, rtol=rtol, atol=atol)
    assert grads.keys() == e_grads.keys() and grads
    for name in grads:
        torch.testing.assert_close(grads[name], e_grads[name], rtol=rtol, atol=atol, msg=name)


@pytest.mark.parametrize("swap_mode", ["sync", "async"])
def test_activation_offload_matches_with_frozen_block_swapping(swap_mode) -> None:
    torch.manual_seed(903)
    baseline = _tiny().train()
    if swap_mode == "async":
        dit.inject_lora(baseline, rank=2, alpha=4.0, b_std=0.03)
    offloaded = copy.deepcopy(baseline).train()
    offloaded.activation_offload = True
    device = torch.device("cuda", 0)
    place_model(baseline, device, 2, block_swap_mode=swap_mode)
    place_model(offloaded, device, 2, block_swap_mode=swap_mode)
    engine = moss_offload.get_engine(device)
    packed_before = engine.stats()["bytes_packed"]
    try:
        inputs = _inputs(device)
        expected = _packed_backward(baseline, inputs)
        actual = _packed_backward(offloaded, _clone(inputs))
        _assert_close(actual, expected)
        assert engine.stats()["bytes_packed"] > packed_before
        if swap_mode == "async":
            slots = offloaded.block_swap_manager.owned_cuda_buffers()
            assert slots
            hook = moss_offload.activation_cpu_offload(offloaded, True, device)
            assert all(hook.is_weight_backed(slot[256:512]) for slot in slots)
    finally:
        for model in (baseline, offloaded):
            if model.block_swap_manager is not None:
                model.block_swap_manager.close()
        gc.collect()


class _InBackwardSGD:
    """Plain SGD applied by post-accumulate-grad hooks, reporting each update to the ring."""

    def __init__(self, model, lr, streamer):
        self.lr, self.streamer, self.updates = lr, streamer, 0
        for p in model.parameters():
            if p.requires_grad:
                p.register_post_accumulate_grad_hook(self._hook)

    def _hook(self, p):
        grad, p.grad = p.grad, None
        with torch.no_grad():
            p.add_(grad, alpha=-self.lr)
        self.updates += 1
        self.streamer.mark_updated(p)


def test_async_full_with_activation_offload_runs_one_streamed_graph() -> None:
    torch.manual_seed(904)
    cpu_model = _tiny().train()
    device = torch.device("cuda", 0)
    resident = copy.deepcopy(cpu_model).to(device).eval()
    streamed = cpu_model
    streamed.activation_offload = True
    place_model(streamed, device, 2, block_swap_mode="async_full")
    manager = streamed.block_swap_manager
    optimizer = _InBackwardSGD(streamed, 2e-3, manager)
    inputs = _inputs(device)
    reference_inputs = _clone(inputs)
    engine = moss_offload.get_engine(device)
    packed_before = engine.stats()["bytes_packed"]
    try:
        with torch.no_grad():
            expected = resident.forward_packed(*reference_inputs)
        manager.set_step_enabled(True)
        outputs = streamed.forward_packed(*inputs)
        for actual, reference in zip(outputs, expected):
            torch.testing.assert_close(actual, reference, rtol=5e-5, atol=5e-6)
        sum(o.float().square().mean() for o in outputs).backward()
        manager.finish_backward()
        assert optimizer.updates == len([p for p in streamed.parameters() if p.requires_grad])
        assert manager.d2h_copy_count == 2  # both streamed blocks written back
        assert inputs[0][0].grad is not None
        assert engine.stats()["bytes_packed"] > packed_before
        assert manager.resident_block_indices == ()
        for layer in streamed.layers[1:]:
            assert all(p.device.type == "cpu" and p.is_pinned() for p in layer.parameters())
    finally:
        manager.close()
        gc.collect()
