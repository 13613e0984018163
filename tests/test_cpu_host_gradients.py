"""CPU checks of moss_offload.host_gradients.HostGradientAccumulator (drop-in for
FusedAdafactor's ``_host_gradients`` mapping, training/fused_adafactor.py:327-369) and of the
harness optimizer's host mode.

The scenarios restate the reference's own training/tests/test_host_gradients.py:27-95 on CPU
tensors. Host accumulation over early micro-batches, followed by the boundary micro-batch, equals
plain accumulation over all micro-batches bit for bit: for fp32 parameters the host sum
(g1 + g2) added to g3 equals (g1 + g2) + g3, because one IEEE add is commutative. A parameter
seen only in early micro-batches is still updated, and an unused one is left alone. No CUDA
state is created on this path.
"""

from __future__ import annotations

import copy

import pytest
import torch

from moss_offload.harness_optim import HostModeSGD
from moss_offload.host_gradients import HostGradientAccumulator


def _loss(model, batch):
    return model(batch).square().sum().mul(1 / 37)


@pytest.mark.parametrize("stash", ["engine", "reference"])
def test_host_accumulation_releases_early_grads_and_matches_device_accumulation(stash) -> None:
    cuda_before = torch.cuda.is_initialized()
    torch.manual_seed(104)
    host_model = torch.nn.Sequential(torch.nn.Linear(5, 7), torch.nn.SiLU(), torch.nn.Linear(7, 3))
    reference_model = copy.deepcopy(host_model)
    host = HostModeSGD(host_model.parameters(), lr=0.02, stash=stash)
    initial = {name: p.detach().clone() for name, p in host_model.named_parameters()}
    batches = [torch.randn(4, 5), torch.randn(2, 5), torch.randn(6, 5)]

    host.set_step_enabled(False)
    for batch in batches[:-1]:
        _loss(host_model, batch).backward()
    assert all(p.grad is None for p in host_model.parameters())
    assert all(torch.equal(p, initial[name]) for name, p in host_model.named_parameters())
    assert len(host.host_gradients) == len(list(host_model.parameters()))
    assert all(v.device.type == "cpu" and v.dtype == torch.float32 for v in host.host_gradients.values())

    host.set_step_enabled(True)
    _loss(host_model, batches[-1]).backward()
    host.finish_backward()

    for batch in batches:
        _loss(reference_model, batch).backward()
    with torch.no_grad():
        for p in reference_model.parameters():
            p.add_(p.grad, alpha=-0.02)
    assert host.host_gradients == {}
    assert all(p.grad is None for p in host_model.parameters())
    for actual, expected in zip(host_model.parameters(), reference_model.parameters()):
        assert torch.equal(actual, expected)
    host.close()
    assert torch.cuda.is_initialized() == cuda_before


def test_host_only_gradient_is_updated_and_never_used_parameter_is_ignored() -> None:
    early = torch.nn.Parameter(torch.tensor([0.4, -0.7]))
    final = torch.nn.Parameter(torch.tensor([-0.2, 0.9]))
    unused = torch.nn.Parameter(torch.tensor([1.5, -1.1]))
    opt = HostModeSGD([early, final, unused], lr=0.03)
    initial = [t.detach().clone() for t in (early, final, unused)]
    opt.set_step_enabled(False)
    (early.square().sum() * 0.4).backward()
    assert early.grad is None and id(early) in opt.host_gradients
    opt.set_step_enabled(True)
    (final.square().sum() * 0.6).backward()
    opt.finish_backward()
    assert opt.updated == {id(early), id(final)}
    assert torch.equal(early, initial[0] - 0.03 * (0.8 * initial[0]))
    assert not torch.equal(final, initial[1]) and torch.equal(unused, initial[2])
    opt.close()


def test_mapping_interface() -> None:
    acc = HostGradientAccumulator()
    a, b = torch.tensor([1.0, 2.0]), torch.tensor([0.5, -0.25], dtype=torch.bfloat16)
    acc.accumulate("w", a)
    acc.accumulate("w", b)
    acc["v"] = torch.zeros(3)
    assert "w" in acc and "v" in acc and "u" not in acc and len(acc) == 2 and sorted(acc) == ["v", "w"]
    assert torch.equal(acc["w"], torch.tensor([1.5, 1.75]))
    assert torch.equal(acc.pop("w"), torch.tensor([1.5, 1.75])) and acc.pop("w", None) is None
    del acc["v"]
    assert acc == {} and not acc
    acc.accumulate("w", a)  # a new step starts the entry afresh
    assert torch.equal(acc["w"], a) and acc["w"].data_ptr() != a.data_ptr()
    acc.clear()
    assert len(acc) == 0
    with pytest.raises(TypeError):
        acc["x"] = [1.0]
    with pytest.raises(ValueError, match="CUDA"):
        HostGradientAccumulator("cpu")
    acc.close()
    with pytest.raises(RuntimeError, match="closed"):
        acc.accumulate("w", a)
