"""Closed-form cases for the oracle's gate and resident rule (CPU only).

The oracle restates the reference's gate (training/activation_offload.py:92-93) and its
resident rule (``is_weight_backed``, :95-114) in ``oracle/reference_hooks.py``. Each case
below has an answer fixed by construction: disabled, a CPU device, ``no_grad`` and
``inference_mode`` give ``nullcontext()``; a parameter, a view of a parameter, a buffer and a
block-swap staging slot stay resident; a plain activation, an activation that merely equals a
parameter's values, and a slot of another device type do not. Three planted mutants of the
rule (owned buffers ignored, buffers ignored, identity compared by tensor instead of storage)
must each get one case wrong, and the product's own hook makes the same decisions as the
oracle on the CPU cases.
"""

from __future__ import annotations

from contextlib import nullcontext

import pytest
import torch
from torch import nn

from oracle import reference_hooks as ref


class _Manager:
    def __init__(self, buffers):
        self._buffers = buffers

    def owned_cuda_buffers(self):
        return self._buffers


class _Model(nn.Module):
    def __init__(self):
        super().__init__()
        self.linear = nn.Linear(8, 8)
        self.register_buffer("table", torch.arange(16.0))
        self.register_buffer("empty", torch.empty(0))


def _cases():
    model = _Model()
    slot = torch.zeros(64, dtype=torch.uint8)
    model.block_swap_manager = _Manager([slot])
    activation = torch.randn(4, 8)
    return model, {
        "parameter": (model.linear.weight, True),
        "parameter transposed view": (model.linear.weight.t(), True),
        "parameter row": (model.linear.weight[3], True),
        "bias": (model.linear.bias, True),
        "buffer": (model.table, True),
        "buffer slice": (model.table[4:9], True),
        "staging slot view": (slot[16:48].view(torch.int32), True),
        "activation": (activation, False),
        "activation equal to a parameter": (model.linear.weight.detach().clone(), False),
        "activation view": (activation[1:], False),
    }


def test_gate_returns_nullcontext_exactly_when_the_reference_does() -> None:
    model = _Model()
    cuda, cpu = torch.device("cuda", 0), torch.device("cpu")
    assert isinstance(ref.activation_cpu_offload(model, False, cuda), nullcontext)
    assert isinstance(ref.activation_cpu_offload(model, True, cpu), nullcontext)
    with torch.no_grad():
        assert isinstance(ref.activation_cpu_offload(model, True, cuda), nullcontext)
    with torch.inference_mode():
        assert isinstance(ref.activation_cpu_offload(model, True, cuda), nullcontext)
    # enabled, a CUDA device and grad mode: the hook pair (nothing touches the device until a
    # CUDA tensor is saved)
    hooks = ref.activation_cpu_offload(model, True, cuda)
    assert isinstance(hooks, torch.autograd.graph.saved_tensors_hooks)


def test_resident_rule_closed_form_cases() -> None:
    model, cases = _cases()
    resident = ref._resident_storages(model, "cpu")
    for name, (tensor, expected) in cases.items():
        assert ref._weight_backed(model, resident, tensor, "cpu") is expected, name
    # empty storages are left out of the resident set (reference :95-99 checks nbytes())
    assert all(key[2] != model.empty.untyped_storage().data_ptr() or model.empty.untyped_storage().nbytes()
               for key in resident)
    # a slot of another device type never matches
    assert ref._weight_backed(model, resident, model.block_swap_manager._buffers[0], "cuda") is False


def test_resident_rule_without_a_manager_and_with_a_non_callable_one() -> None:
    model, cases = _cases()
    del model.block_swap_manager
    resident = ref._resident_storages(model, "cpu")
    slot = cases["staging slot view"][0]
    assert ref._weight_backed(model, resident, slot, "cpu") is False
    model.block_swap_manager = object()  # no owned_cuda_buffers
    assert ref._weight_backed(model, resident, slot, "cpu") is False


def test_emulated_hooks_keep_resident_saves_and_offload_the_rest() -> None:
    model = _Model()
    recorder = ref.Recorder()
    x = torch.randn(3, 8, requires_grad=True)
    with ref.emulated_offload(model, recorder):
        y = model.linear(x).square().sum()
    # Linear saves its input x and its weight (resident); square saves its input
    assert recorder.resident >= 1
    assert all(not any(p is t for p in model.parameters()) for t, _ in recorder.packed)
    y.backward()
    assert x.grad is not None


@pytest.mark.parametrize("mutant", ["ignore_owned", "ignore_buffers", "tensor_identity"])
def test_planted_mutants_of_the_resident_rule_disagree(mutant) -> None:
    def ignore_owned(model, resident, tensor, device_type):
        return ref.storage_key(tensor) in resident

    def ignore_buffers(model, resident, tensor, device_type):
        params = {ref.storage_key(p) for p in model.parameters()}
        if ref.storage_key(tensor) in params:
            return True
        manager = getattr(model, "block_swap_manager", None)
        owned = getattr(manager, "owned_cuda_buffers", None)
        return callable(owned) and any(ref.storage_key(b) == ref.storage_key(tensor) for b in owned())

    def tensor_identity(model, resident, tensor, device_type):
        return any(tensor is t for t in (*model.parameters(), *model.buffers()))

    planted = {"ignore_owned": ignore_owned, "ignore_buffers": ignore_buffers, "tensor_identity": tensor_identity}
    model, cases = _cases()
    resident = ref._resident_storages(model, "cpu")
    wrong = [name for name, (t, expected) in cases.items() if planted[mutant](model, resident, t, "cpu") is not expected]
    assert wrong, f"mutant {mutant} agrees with every case"


def test_product_hook_makes_the_oracles_resident_decisions() -> None:
    # The product's rule (activation_offload.py, is_weight_backed) is written for HIP devices:
    # its resident set holds the model's storages and it matches staging slots on "cuda"
    # tensors only. On these CPU tensors it must agree with the oracle run for device type
    # "cuda" on the slot, and for "cpu" on everything else.
    from moss_offload.activation_offload import _ActivationOffload

    model, cases = _cases()
    hook = _ActivationOffload.__new__(_ActivationOffload)
    hook.model = model
    hook.resident_storages = ref._resident_storages(model, "cpu")
    for name, (tensor, expected) in cases.items():
        oracle = ref._weight_backed(model, hook.resident_storages, tensor, "cuda" if "slot" in name else "cpu")
        assert hook.is_weight_backed(tensor) is oracle, name
