"""Frozen-block streaming (``moss_offload.memory``) on the GPU, against a resident model.

Every case builds one seeded model twice: one copy stays resident, the other streams its frozen
blocks through the native block ring (SDMA fills into two device slots, masters in one pinned
arena). The cases are rows of two tables, each run by one driver:

- ``TRAINING``: two AdamW steps, then a grad-free eval with and without skipped blocks, for
  each precision and base (dense / int8). Streamed and resident runs are compared with
  ``assert_bitwise`` where the streamed block computes on the same bits with the same kernels
  (fp32), and within the reference's tolerances where it does not have to (bf16 autocast).
- ``LIFECYCLE``: graphs and teardown the streamer must survive: two live graphs before one
  backward, a grad-enabled eval, ``torch.autograd.grad``, a retained graph, a recomputation that
  raises, CPU placement after an eval prefetch, and activation offload on top of streaming.

The scenarios and their data (seeds, tiny-model sizes, sample shapes and timesteps, learning
rate, tolerances) are the behavioural contract of the reference's
``training/tests/test_async_memory.py`` (:22-33 sizes, :101-115 samples, :137-236 training and
eval, :239-425 lifecycle); the harness around them is this repository's.
"""

from __future__ import annotations

import copy
import gc
from dataclasses import dataclass
from typing import Callable

import pytest
import torch

import moss_offload
from moss_offload import dit
from moss_offload.memory import AsyncBlockStreamer, place_model

from gpu_util import assert_bitwise, requires_gpu

pytestmark = requires_gpu

DEVICE = torch.device("cuda", 0)
# tiny joint-block model of the reference's streaming tests (test_async_memory.py:22-33)
TINY = dict(dim=32, ffn_dim=64, num_heads=4, num_layers=4, text_dim=16, freq_dim=8, latent_channels=4)
# (latent grid, timestep, text tokens) of the two samples (test_async_memory.py:101-115)
SAMPLES = (((4, 4), 250.0, 3), ((3, 5), 750.0, 4))
LR = 2e-3


@dataclass(frozen=True)
class Tol:
    atol: float
    rtol: float


FP32 = Tol(2e-5, 2e-3)  # test_async_memory.py:186, :281
BF16 = Tol(4e-3, 3e-2)  # test_async_memory.py:186


def _agree(actual: torch.Tensor, expected: torch.Tensor, tol: Tol | None, what: str) -> None:
    """Bitwise when ``tol`` is None, else within it."""

    if tol is None:
        assert_bitwise(actual.detach(), expected.detach())
    else:
        torch.testing.assert_close(actual, expected, atol=tol.atol, rtol=tol.rtol, msg=lambda m: f"{what}: {m}")


def _agree_all(actual: dict, expected: dict, tol: Tol | None, what: str) -> None:
    assert actual.keys() == expected.keys() and actual
    for name in actual:
        _agree(actual[name], expected[name], tol, f"{what} {name}")


def _samples(dtype: torch.dtype) -> list[dict]:
    out = []
    for (h, w), t, text in SAMPLES:
        out.append(dict(hidden_states=torch.randn(1, TINY["latent_channels"], h, w, device=DEVICE, dtype=dtype),
                        timestep=torch.tensor([t], device=DEVICE),
                        encoder_hidden_states=torch.randn(1, text, TINY["text_dim"], device=DEVICE, dtype=dtype)))
    return out


def _adapters(model) -> dict:
    return {n: p for n, p in model.named_parameters() if p.requires_grad}


def _frozen_tensors(model) -> dict:
    found = {f"param {n}": p for n, p in model.layers.named_parameters() if not p.requires_grad}
    found.update({f"buffer {n}": b for n, b in model.layers.named_buffers()})
    return found


class Twin:
    """One seeded LoRA model, placed twice: ``resident`` on the device, ``streamed`` with its
    last ``streamed_blocks`` blocks on the frozen-block ring."""

    def __init__(self, seed: int, dtype=torch.float32, int8=False, streamed_blocks=4, train=True) -> None:
        torch.manual_seed(seed)
        model = dit.MOSSImageTransformer(**TINY, gradient_checkpointing=True).to(dtype=dtype)
        dit.init_weights(model)
        if int8:
            dit.quantize_joint_linears(model, torch.Generator().manual_seed(5))
        dit.inject_lora(model, rank=2, alpha=4.0, b_std=0.03)
        model.train(train)
        self.streamed = copy.deepcopy(model)
        self.resident = model
        self.masters_before = {n: t.detach().clone() for n, t in _frozen_tensors(self.streamed).items()}
        self.adapter_ids = {n: id(p) for n, p in _adapters(self.streamed).items()}
        place_model(self.resident, DEVICE, 0)
        place_model(self.streamed, DEVICE, streamed_blocks, block_swap_mode="async")
        self.dtype = dtype

    @property
    def manager(self) -> AsyncBlockStreamer:
        return self.streamed.block_swap_manager

    def models(self):
        return self.resident, self.streamed


def _losses_of(model, samples, autocast: bool):
    """Each sample's output and half mean-square, forward only (the reference trainer's
    per-sample backward follows the caller)."""

    for sample in samples:
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            output = model(**sample)
            yield output, output.float().square().mean() / 2


class Trainer:
    """AdamW on a model's adapters, one backward per sample (test_async_memory.py:118-134)."""

    def __init__(self, model, dtype: torch.dtype, autocast: bool) -> None:
        self.model, self.dtype, self.autocast = model, dtype, autocast
        self.optimizer = torch.optim.AdamW(_adapters(model).values(), lr=LR)

    def step(self, index: int) -> tuple[list, dict, dict]:
        """Outputs, gradients and the adapters after the update (on the host)."""

        torch.manual_seed(200 + index)  # per-step samples, test_async_memory.py:189
        self.optimizer.zero_grad(set_to_none=True)
        outputs = []
        for output, loss in _losses_of(self.model, _samples(self.dtype), self.autocast):
            outputs.append(output.detach().cpu())
            loss.backward()
        adapters = _adapters(self.model)
        grads = {n: p.grad for n, p in adapters.items()}
        assert all(g is not None and torch.isfinite(g).all() for g in grads.values())
        # B starts non-zero (b_std), so A receives gradient in the first step already
        assert all(torch.count_nonzero(g) > 0 for n, g in grads.items() if n.endswith("lora_A"))
        grads = {n: g.detach().cpu().clone() for n, g in grads.items()}
        self.optimizer.step()
        return outputs, grads, {n: p.detach().cpu().clone() for n, p in adapters.items()}


# ---- table 1: training and eval, per precision and base -----------------------------------

@dataclass(frozen=True)
class Training:
    name: str
    dtype: torch.dtype
    int8: bool
    tol: Tol | None  # None: bitwise


TRAINING = (
    Training("fp32-dense", torch.float32, False, None),
    Training("bf16-dense", torch.bfloat16, False, BF16),
    Training("fp32-int8", torch.float32, True, None),
    Training("bf16-int8", torch.bfloat16, True, BF16),
)


@pytest.mark.parametrize("case", TRAINING, ids=[c.name for c in TRAINING])
def test_streamed_lora_trains_and_evaluates_like_the_resident_model(case: Training) -> None:
    twin = Twin(83, case.dtype, case.int8)  # seed: test_async_memory.py:140
    manager = twin.manager
    # placement: adapters stay the same Parameter objects on the device, frozen tensors become
    # pinned host masters (int8 bases keep their dtype)
    assert {n: id(p) for n, p in _adapters(twin.streamed).items()} == twin.adapter_ids
    assert all(p.is_cuda for p in _adapters(twin.streamed).values())
    masters = _frozen_tensors(twin.streamed)
    assert masters.keys() == twin.masters_before.keys()
    assert all(t.device.type == "cpu" and (t.numel() == 0 or t.is_pinned()) for t in masters.values())
    int8 = [t for n, t in masters.items() if n.endswith("weight_int8")]
    assert bool(int8) == case.int8 and all(t.dtype == torch.int8 for t in int8)

    autocast = case.dtype == torch.bfloat16
    trainers = [Trainer(model, case.dtype, autocast) for model in twin.models()]
    runs = [[t.step(0)] for t in trainers]
    # eval between the steps: conditional, and unconditional with blocks 1 and 3 skipped
    evals = []
    for model in twin.models():
        model.eval()
        torch.manual_seed(300)
        sample = _samples(case.dtype)[1]
        negative = dict(sample, encoder_hidden_states=-sample["encoder_hidden_states"])
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            evals.append((model(**sample), model(**negative, skip_layers=(1, 3))))
        model.train()
    for run, trainer in zip(runs, trainers):
        run.append(trainer.step(1))
    resident, streamed = runs
    for step, ((r_out, r_grad, r_after), (s_out, s_grad, s_after)) in enumerate(zip(resident, streamed)):
        for k, (a, b) in enumerate(zip(s_out, r_out)):
            _agree(a, b, case.tol, f"step {step} output {k}")
        _agree_all(s_grad, r_grad, case.tol, f"step {step} gradient")
        _agree_all(s_after, r_after, case.tol, f"step {step} adapter")
    for what, a, b in zip(("conditional", "skip_layers"), evals[1], evals[0]):
        _agree(a, b, case.tol, f"eval {what}")

    assert 1 <= manager.peak_resident_blocks <= 2
    stats = manager.stats()
    assert stats["fills"] == manager.h2d_copy_count > 0 and stats["copy_failures"] == 0
    # the masters never change: the streamer only reads them
    for name, before in twin.masters_before.items():
        after = _frozen_tensors(twin.streamed)[name]
        assert after.device.type == "cpu"
        assert_bitwise(after, before)


def test_streamed_forward_is_bitwise_the_resident_forward() -> None:
    twin = Twin(84)
    sample = _samples(torch.float32)[1]
    with torch.no_grad():
        assert_bitwise(twin.streamed(**sample), twin.resident(**sample))


# ---- table 2: graphs and teardown -----------------------------------------------------------

def _two_live_graphs_one_backward(twin: Twin) -> None:
    """Both samples' forwards before a single backward; two of four blocks streamed."""

    for layer in twin.streamed.layers[:2]:
        assert all(p.is_cuda for p in layer.parameters())
    for layer in twin.streamed.layers[2:]:
        assert all(p.is_cuda == p.requires_grad for p in layer.parameters())
    results = []
    for model in twin.models():
        torch.manual_seed(400)
        optimizer = torch.optim.AdamW(_adapters(model).values(), lr=LR)
        outputs = [model(**s) for s in _samples(torch.float32)]
        sum(o.float().square().mean() / len(outputs) for o in outputs).backward()
        grads = {n: p.grad.detach().clone() for n, p in _adapters(model).items()}
        optimizer.step()
        results.append((outputs, grads, {n: p.detach().clone() for n, p in _adapters(model).items()}))
    (r_out, r_grad, r_after), (s_out, s_grad, s_after) = results
    for a, b in zip(s_out, r_out):
        _agree(a, b, None, "output")
    _agree_all(s_grad, r_grad, None, "gradient")
    _agree_all(s_after, r_after, None, "adapter")
    assert 1 <= twin.manager.peak_resident_blocks <= 2


def _grad_enabled_eval(twin: Twin) -> None:
    """An eval-mode forward with grad enabled builds a graph through all four streamed blocks."""

    grads = []
    torch.manual_seed(401)
    sample = _samples(torch.float32)[0]
    for model in twin.models():
        output = model(**sample)
        assert output.grad_fn is not None
        output.float().square().mean().backward()
        grads.append((output, {n: p.grad for n, p in _adapters(model).items()}))
    _agree(grads[1][0], grads[0][0], None, "output")
    _agree_all(grads[1][1], grads[0][1], None, "gradient")


def _autograd_grad_then_backward_then_cpu(twin: Twin) -> None:
    """``torch.autograd.grad`` leaves ``.grad`` unset and the ring ready for the next step; CPU
    placement then closes the streamer and brings every tensor home."""

    model, manager = twin.streamed, twin.manager
    adapters = _adapters(model)
    samples = _samples(torch.float32)
    grads = torch.autograd.grad(model(**samples[0]).float().square().mean(), tuple(adapters.values()))
    assert len(grads) == len(adapters) and all(torch.isfinite(g).all() for g in grads)
    assert all(p.grad is None for p in adapters.values())
    model(**samples[1]).float().square().mean().backward()
    assert all(p.grad is not None and torch.isfinite(p.grad).all() for p in adapters.values())
    torch.optim.AdamW(adapters.values(), lr=LR).step()
    place_model(model, torch.device("cpu"), 0)
    assert manager.closed and manager.resident_block_indices == () and model.block_swap_manager is None
    assert all(p.device.type == "cpu" for p in model.parameters())


def _retained_graph(twin: Twin) -> None:
    """Two backwards over one retained graph accumulate twice the gradient, and the second
    traversal recomputes every streamed block again."""

    model = twin.streamed
    adapters = _adapters(model)
    loss = model(**_samples(torch.float32)[0]).float().square().mean()
    loss.backward(retain_graph=True)
    once = {n: p.grad.detach().clone() for n, p in adapters.items()}
    fills = twin.manager.h2d_copy_count
    loss.backward()
    assert twin.manager.h2d_copy_count > fills
    _agree_all({n: p.grad for n, p in adapters.items()}, {n: 2 * g for n, g in once.items()}, FP32, "twice")


def _recomputation_raises(twin: Twin) -> None:
    """A streamed block that raises while backward recomputes it: the error reaches the caller,
    the streamer can still be torn down, and a fresh placement trains."""

    model, failed = twin.streamed, twin.manager
    last = model.layers[-1]

    def refuse_recompute(module, args):
        if failed._phase.active:
            raise RuntimeError("recomputation refused")

    hook = last.register_forward_pre_hook(refuse_recompute)
    loss = model(**_samples(torch.float32)[0]).float().square().mean()  # the forward runs
    try:
        with pytest.raises(RuntimeError, match="recomputation refused"):
            loss.backward()
    finally:
        hook.remove()
    del loss
    gc.collect()
    place_model(model, torch.device("cpu"), 0)
    assert failed.closed and failed.resident_block_indices == () and model.block_swap_manager is None
    place_model(model, DEVICE, 4, block_swap_mode="async")
    assert model.block_swap_manager is not failed
    model.zero_grad(set_to_none=True)
    model(**_samples(torch.float32)[1]).float().square().mean().backward()
    assert all(p.grad is not None and torch.isfinite(p.grad).all() for p in _adapters(model).values())
    recovered = model.block_swap_manager
    place_model(model, torch.device("cpu"), 0)
    assert recovered.closed


def _cpu_placement_after_eval_prefetch(twin: Twin) -> None:
    """An eval forward fills every block once (the last ones stay resident); CPU placement
    closes the streamer and returns parameters and buffers to the host."""

    model, manager = twin.streamed, twin.manager
    assert manager.h2d_copy_count == 0
    with torch.no_grad():
        output = model(**_samples(torch.float32)[0])
    assert output.is_cuda and manager.resident_block_indices
    assert manager.h2d_copy_count == len(model.layers)
    place_model(model, torch.device("cpu"), 0)
    assert manager.closed and manager.resident_block_indices == () and model.block_swap_manager is None
    assert all(t.device.type == "cpu" for t in (*model.parameters(), *model.buffers()))


def _with_activation_offload(twin: Twin) -> None:
    """The low-VRAM combination (int8 bases streamed, activations offloaded): the ring's slots
    count as weight-backed, never offloaded, and a step matches the resident model without
    offload."""

    twin.streamed.activation_offload = True
    results = [Trainer(model, torch.bfloat16, autocast=True).step(0) for model in twin.models()]
    (r_out, r_grad, _), (s_out, s_grad, _) = results
    for a, b in zip(s_out, r_out):
        _agree(a, b, BF16, "output")
    _agree_all(s_grad, r_grad, BF16, "gradient")
    slots = twin.manager.owned_cuda_buffers()
    assert slots
    ctx = moss_offload.activation_cpu_offload(twin.streamed, True, DEVICE)
    assert all(ctx.is_weight_backed(slot[64:128]) for slot in slots)
    assert moss_offload.get_engine(DEVICE).stats()["bytes_packed"] > 0


@dataclass(frozen=True)
class Lifecycle:
    name: str
    seed: int  # test_async_memory.py:240, :288, :313, :342, :360, :408
    run: Callable[[Twin], None]
    streamed_blocks: int = 4
    train: bool = True
    dtype: torch.dtype = torch.float32
    int8: bool = False


LIFECYCLE = (
    Lifecycle("two-live-graphs-one-backward", 97, _two_live_graphs_one_backward, streamed_blocks=2),
    Lifecycle("grad-enabled-eval", 101, _grad_enabled_eval, train=False),
    Lifecycle("autograd-grad-then-cpu", 103, _autograd_grad_then_backward_then_cpu),
    Lifecycle("retained-graph", 107, _retained_graph),
    Lifecycle("recomputation-raises", 109, _recomputation_raises),
    Lifecycle("cpu-after-eval-prefetch", 113, _cpu_placement_after_eval_prefetch, train=False),
    Lifecycle("with-activation-offload", 115, _with_activation_offload, dtype=torch.bfloat16, int8=True),
)


@pytest.mark.parametrize("case", LIFECYCLE, ids=[c.name for c in LIFECYCLE])
def test_streamer_lifecycle(case: Lifecycle) -> None:
    twin = Twin(case.seed, case.dtype, case.int8, case.streamed_blocks, case.train)
    case.run(twin)
