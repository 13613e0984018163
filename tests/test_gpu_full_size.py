"""Parity at BASELINE's real sizes (configs 2-5) on the GPU.

The reference's parity method (training/tests/test_packed_cuda.py:173-201) runs the same
seeded model with and without offload and compares the loss and gradients. Here that runs on
the shapes ``bench.py`` measures, through the drop-in ``activation_cpu_offload``:

- config 2: one regime-B block's saved set at 1024^2 (the bench's block microbench) through
  pack -> D2H -> H2D -> unpack with each transport, every tensor bitwise;
- config 3 (40 blocks, 1024^2, LoRA r32, autocast bf16): regime B, where every transformation
  of the hook acts (narrowed casts, recomputed products, aliased equal casts, deduplicated
  views); regime A; and checkpoint_fraction 0.5, where checkpointed and plain blocks alternate
  in one traversal;
- config 3 at 16 blocks against the oracle's restatement of the reference hooks (16 blocks
  keep the reference's per-save pinned copies within the host's pinned-memory cap);
- config 4 (2048^2 + 4096 text tokens) in regime A;
- config 5 (int8 bases + LoRA r16, four aspect buckets) grouped and packed.

In every step test each restored tensor is compared bitwise with a copy of the save taken at
pack time; the loss must be bitwise equal to the hooks-off run (the forward never sees a
restore) and every LoRA gradient within 1e-3 relative of it, the north-star tolerance (the
runs so far are bitwise; the test reports it).
"""

from __future__ import annotations

import gc

import pytest
import torch
from torch import nn

import bench
import moss_offload
from moss_offload.activation_offload import _ActivationOffload, _CheckedAlias, _DerivedTensor, _OffloadedTensor
from oracle import reference_hooks

from gpu_util import assert_bitwise, requires_gpu

pytestmark = requires_gpu

GRAD_RTOL = 1e-3


class _Checked(_ActivationOffload):
    """The engine's context, plus a device copy of every save it takes over, compared bitwise
    with what unpack returns."""

    saves: dict = {}
    checked = 0
    kinds = (_OffloadedTensor, _DerivedTensor, _CheckedAlias)

    def pack(self, tensor):
        handle = super().pack(tensor)
        if isinstance(handle, _Checked.kinds):
            _Checked.saves[id(handle)] = tensor.detach().clone()
        return handle

    def unpack(self, saved):
        restored = super().unpack(saved)
        expected = _Checked.saves.get(id(saved)) if isinstance(saved, _Checked.kinds) else None
        if expected is not None:
            stride = saved.stride if hasattr(saved, "stride") else expected.stride()
            assert restored.shape == expected.shape and restored.stride() == stride
            assert_bitwise(restored, expected)
            _Checked.checked += 1
        return restored


def _checked_context(model, enabled, device):
    if not enabled or device.type != "cuda" or not torch.is_grad_enabled():
        return moss_offload.activation_cpu_offload(model, enabled, device)
    return _Checked(model, device)


def _step(model, inputs, forward, context, enabled):
    model.activation_offload = enabled
    model.offload_context = context
    model.zero_grad(set_to_none=True)
    loss = bench.loss_and_backward(model, inputs, forward)
    torch.cuda.synchronize()
    grads = {n: p.grad.detach().float().clone() for n, p in model.named_parameters() if p.grad is not None}
    model.zero_grad(set_to_none=True)
    return loss.float(), grads


def _compare(actual, expected, label, loss_rtol=0.0, grad_rtol=GRAD_RTOL):
    loss, grads = actual
    e_loss, e_grads = expected
    if loss_rtol:
        rel = abs(loss.item() - e_loss.item()) / abs(e_loss.item())
        assert rel <= loss_rtol, f"{label}: loss {loss.item()} vs {e_loss.item()} (relative {rel:.2e})"
    else:
        assert torch.equal(loss, e_loss), f"{label}: loss {loss.item()} vs {e_loss.item()}"
    assert grads.keys() == e_grads.keys() and grads
    worst, bitwise = 0.0, True
    for name, grad in grads.items():
        ref = e_grads[name]
        rel = float((grad - ref).norm() / ref.norm().clamp_min(1e-30))
        worst = max(worst, rel)
        bitwise = bitwise and torch.equal(grad, ref)
        assert rel <= grad_rtol, f"{label}: {name} relative error {rel:.3e}"
    print(f"{label}: loss {'bitwise' if torch.equal(loss, e_loss) else 'within tolerance'}, worst LoRA gradient "
          f"relative error {worst:.3e}, bitwise {bitwise}", flush=True)


def _release_pinned() -> None:
    """Give pinned host memory back between steps: the engine's idle pool chunks and torch's
    cached pinned blocks (the reference hooks pin one tensor per save). A process may pin about
    65 GiB on the GPU box, and the tests run one after another in one process."""

    from moss_offload import engine as engine_mod

    gc.collect()
    torch.cuda.synchronize()
    for engine in list(engine_mod._ENGINES.values()):
        engine.synchronize()
        engine.trim()
    torch._C._host_emptyCache()


def _engine_step(model, inputs, forward=bench.config3_forward):
    """One step through the checked engine context; returns (loss, grads) and what the hook did."""

    _Checked.saves.clear()
    _Checked.checked = 0
    moss_offload.reset_hook_counters()
    result = _step(model, inputs, forward, _checked_context, True)
    counters = moss_offload.hook_counters()
    checked = _Checked.checked
    _Checked.saves.clear()
    _release_pinned()
    return result, counters, checked


def _regime(model, regime, fraction=1.0):
    model.gradient_checkpointing = regime == "A"
    model.checkpoint_fraction = fraction


@pytest.fixture(scope="module")
def config3_model():
    device = torch.device("cuda", 0)
    model = bench.build_model(device, bench.CONFIG3["num_layers"])
    yield model
    del model
    gc.collect()
    torch.cuda.empty_cache()
    moss_offload.reset_engines()


@pytest.mark.parametrize("link", ["sdma", "hipdma"])
def test_config2_block_saves_round_trip_bitwise(config3_model, link) -> None:
    device = torch.device("cuda", 0)
    inputs = bench.make_inputs(device)
    tensors, narrow = bench.capture_block_saves(config3_model, inputs)
    payload = sum(t.numel() * t.element_size() for t in tensors)
    assert len(tensors) >= 50 and payload > 1.4e9  # one 1024^2 block: 55 unique saves, 1.43 GB
    result = bench.micro(device, tensors, iters=2, warmup=1, slot_mib=128, stage_slots=4, restore_slots=4,
                         narrow=narrow, link=link)
    assert result["bitwise_first"] and result["bitwise_last"]
    assert result["copy_failures"] == 0
    del tensors
    gc.collect()


@pytest.mark.parametrize("wire_coding", ["auto", "off"])
def test_config3_regime_b_40_blocks_matches_no_offload(config3_model, wire_coding) -> None:
    """Regime B at 40 blocks with the default engine (wire coding "auto": the forward's backlog
    makes it code most segments) and with wire coding off."""

    from moss_offload import engine as engine_mod

    device = torch.device("cuda", 0)
    inputs = bench.make_inputs(device)
    _regime(config3_model, "B")
    expected = _step(config3_model, inputs, bench.config3_forward, moss_offload.activation_cpu_offload, False)
    previous = engine_mod._DEFAULT_CONFIG
    moss_offload.reset_engines()
    moss_offload.configure(wire_coding=wire_coding)
    try:
        actual, counters, checked = _engine_step(config3_model, inputs)
        st = engine_mod.get_engine(device).stats()
    finally:
        moss_offload.reset_engines()
        engine_mod._DEFAULT_CONFIG = previous
    _compare(actual, expected, f"config 3 regime B, wire coding {wire_coding}")
    print(f"hook counters: {counters}, restores checked {checked}, wire segments {st['wire_segments']}, "
          f"coded/raw {st['wire_bytes'] / max(st['wire_raw_bytes'], 1):.3f}", flush=True)
    if wire_coding == "auto":
        assert st["wire_segments"] > 100 and st["wire_bytes"] < 0.85 * st["wire_raw_bytes"]
    else:
        assert st["wire_segments"] == 0
    # every transformation of the hook acted at this shape, and every restore was checked
    for kind in ("offloaded", "narrowed", "derived", "aliased", "deduplicated"):
        assert counters.get(kind, 0) >= 40, (kind, counters)
    assert checked > counters["offloaded"] // 2


@pytest.mark.parametrize("fraction", [1.0, 0.5])
def test_config3_regime_a_and_mixed_fraction_match_no_offload(config3_model, fraction) -> None:
    device = torch.device("cuda", 0)
    inputs = bench.make_inputs(device)
    _regime(config3_model, "A", fraction)
    expected = _step(config3_model, inputs, bench.config3_forward, moss_offload.activation_cpu_offload, False)
    actual, counters, checked = _engine_step(config3_model, inputs)
    _compare(actual, expected, f"config 3 checkpoint_fraction {fraction}")
    assert checked > 0 and counters.get("offloaded", 0) > 0
    if fraction < 1.0:
        # plain blocks between checkpointed ones: their activations went through the transformations
        assert counters.get("narrowed", 0) > 0 and counters.get("derived", 0) > 0
    _regime(config3_model, "B")


def test_config3_16_blocks_engine_matches_the_reference_hooks(config3_model) -> None:
    device = torch.device("cuda", 0)
    inputs = bench.make_inputs(device)
    layers = config3_model.layers
    config3_model.layers = nn.ModuleList(list(layers)[:16])
    try:
        _regime(config3_model, "B")
        none = _step(config3_model, inputs, bench.config3_forward, moss_offload.activation_cpu_offload, False)
        reference = _step(config3_model, inputs, bench.config3_forward, reference_hooks.activation_cpu_offload, True)
        _release_pinned()
        engine, _, checked = _engine_step(config3_model, inputs)
    finally:
        config3_model.layers = layers
    _compare(reference, none, "16 blocks: reference hooks vs none")
    _compare(engine, reference, "16 blocks: engine vs reference hooks")
    assert checked > 0


def test_config4_regime_a_2048_matches_no_offload(config3_model) -> None:
    device = torch.device("cuda", 0)
    inputs = bench.make_inputs(device, bench.C4_GRID, bench.C4_TEXT, seed=4)
    _regime(config3_model, "A")
    expected = _step(config3_model, inputs, bench.config3_forward, moss_offload.activation_cpu_offload, False)
    actual, counters, checked = _engine_step(config3_model, inputs)
    _compare(actual, expected, "config 4 regime A")
    assert checked > 0
    _regime(config3_model, "B")


def test_config4_regime_b_2048_matches_no_offload(config3_model) -> None:
    """Config 4 not checkpointed (2048^2 + 4096 text tokens, the reference's plain-block branch,
    training/model.py:708-709), where the host link sets the pace: about 6.3 GB of saves per
    block. On 12 blocks (their coded saves fit the host's pinned-memory cap with room to
    spare): every restore bitwise, the loss bitwise and the LoRA gradients within 1e-3."""

    from moss_offload import engine as engine_mod

    device = torch.device("cuda", 0)
    inputs = bench.make_inputs(device, bench.C4_GRID, bench.C4_TEXT, seed=4)
    layers = config3_model.layers
    config3_model.layers = nn.ModuleList(list(layers)[:12])
    try:
        _regime(config3_model, "B")
        expected = _step(config3_model, inputs, bench.config3_forward, moss_offload.activation_cpu_offload, False)
        engine_mod.get_engine(device).reset_stats()
        actual, counters, checked = _engine_step(config3_model, inputs)
        st = engine_mod.get_engine(device).stats()
    finally:
        config3_model.layers = layers
    _compare(actual, expected, "config 4 regime B, 12 blocks")
    print(f"config 4 regime B: {counters}, restores checked {checked}, D2H {st['bytes_d2h'] / 1e9:.1f} GB, "
          f"H2D {st['bytes_h2d'] / 1e9:.1f} GB, wire segments {st['wire_segments']}", flush=True)
    assert checked > counters["offloaded"] // 2 and counters.get("narrowed", 0) >= 12
    assert st["wire_segments"] > 0  # the link fell behind and the engine coded


def _bit_sum(tensor):
    width = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[tensor.element_size()]
    return tensor.detach().contiguous().view(width).sum(dtype=torch.int64)


def _fingerprint(model, inputs):
    """Bit sums of every parameter, buffer and input tensor (device scalars, no host wait)."""

    named = dict(model.named_parameters())
    named.update(model.named_buffers())
    leaves = torch.utils._pytree.tree_flatten(inputs)[0]
    named.update({f"input {i}": t for i, t in enumerate(leaves) if isinstance(t, torch.Tensor)})
    return {name: _bit_sum(t) for name, t in named.items() if t.numel()}


class _BlockTrace:
    """Bit sums of the text adapter's and every joint block's outputs, in call order (the forward
    and, for checkpointed blocks, the recomputation in backward)."""

    def __init__(self, model):
        self.sums = []
        modules = [("text_embedder", model.text_embedder)] + [(f"layers.{i}", m) for i, m in enumerate(model.layers)]
        self.handles = [m.register_forward_hook(self._hook(name)) for name, m in modules]

    def _hook(self, name):
        def record(module, args, output):
            self.sums.append((name, _bit_sum(output)))
        return record

    def close(self):
        for h in self.handles:
            h.remove()
        return [(name, int(s)) for name, s in self.sums]


def _first_difference(a, b):
    for i, (x, y) in enumerate(zip(a, b)):
        if x != y:
            return f"call {i}: {x[0]} (of {len(a)} and {len(b)} calls)"
    return None if len(a) == len(b) else f"call counts {len(a)} vs {len(b)}"


def _config5_steps(packed):
    """Hooks off, then the checked engine context, on config 5 (int8 bases, LoRA r16, four
    buckets). Parameters, buffers and inputs must keep their bits through both steps (the engine
    writes only memory it owns); on a loss mismatch the first block whose output differed is
    named."""

    device = torch.device("cuda", 0)
    gc.collect()
    torch.cuda.empty_cache()
    model = bench.build_c5_model(device, bench.CONFIG3["num_layers"])
    batch = bench.make_c5_batch(device)
    forward = bench.packed_forward if packed else bench.grouped_forward
    _regime(model, "A")
    try:
        before = _fingerprint(model, batch)
        trace = _BlockTrace(model)
        expected = _step(model, batch, forward, moss_offload.activation_cpu_offload, False)
        expected_trace = trace.close()
        between = _fingerprint(model, batch)
        trace = _BlockTrace(model)
        actual, counters, checked = _engine_step(model, batch, forward)
        actual_trace = trace.close()
        after = _fingerprint(model, batch)
        for label, state in (("hooks-off step", between), ("engine step", after)):
            changed = [name for name in before if not torch.equal(before[name], state[name])]
            assert not changed, f"the {label} changed {len(changed)} parameters/buffers/inputs: {changed[:5]}"
        first = _first_difference(expected_trace, actual_trace)
        print(f"config 5 {'packed' if packed else 'grouped'}: losses {expected[0].item():.7f} (hooks off), "
              f"{actual[0].item():.7f} (engine); first differing block output: {first}", flush=True)
    finally:
        del model
        gc.collect()
        torch.cuda.empty_cache()
    assert checked > 0 and counters.get("offloaded", 0) > 0
    return actual, expected


@pytest.mark.parametrize("packed", [False, True], ids=["grouped", "packed"])
def test_config5_int8_lora_buckets_match_no_offload(packed) -> None:
    """Config 5 grouped (four graphs before one backward) and packed (one varlen traversal):
    every restore bitwise, the loss bitwise and the LoRA gradients within the north-star 1e-3
    (so far bitwise)."""

    actual, expected = _config5_steps(packed=packed)
    _compare(actual, expected, f"config 5 {'packed' if packed else 'grouped'}")


def _lora_state(model):
    return {n: p.detach().clone() for n, p in model.named_parameters() if p.requires_grad}


@pytest.mark.parametrize("regime,fraction", [("B", 1.0), ("A", 0.5)], ids=["regime-B", "fraction-0.5"])
def test_config3_three_adamw_steps_match_no_offload(config3_model, regime, fraction) -> None:
    """Three optimizer steps from one state with the engine and with hooks off (the reference's
    trainer-level test, training/tests/test_training_controls_cuda.py:18-66, runs two steps with
    activation_offload, checkpoint_fraction 0.5 and bf16): after every step the loss and every
    LoRA parameter are compared, so the engine's steady state is covered (wire coding after the
    staging ring has wrapped, restores staged from the previous step's ring, pool reuse, trim)."""

    device = torch.device("cuda", 0)
    inputs = bench.make_inputs(device, seed=7)
    _regime(config3_model, regime, fraction)
    start = _lora_state(config3_model)

    def run(enabled):
        with torch.no_grad():
            for n, p in config3_model.named_parameters():
                if p.requires_grad:
                    p.copy_(start[n])
        params = [p for p in config3_model.parameters() if p.requires_grad]
        opt = torch.optim.AdamW(params, lr=1e-3, weight_decay=0.01)
        config3_model.activation_offload = enabled
        config3_model.offload_context = moss_offload.activation_cpu_offload
        trace, coded = [], []
        for _ in range(3):
            opt.zero_grad(set_to_none=True)
            loss = bench.loss_and_backward(config3_model, inputs)
            opt.step()
            torch.cuda.synchronize()
            trace.append((loss.float(), _lora_state(config3_model)))
            if enabled:
                engine = moss_offload.get_engine(device)
                engine.synchronize()
                coded.append(engine.stats()["wire_segments"])
        return trace, coded

    try:
        expected, _ = run(False)
        moss_offload.get_engine(device).reset_stats()
        actual, coded = run(True)
    finally:
        with torch.no_grad():
            for n, p in config3_model.named_parameters():
                if p.requires_grad:
                    p.copy_(start[n])
                    p.grad = None
        _regime(config3_model, "B")
        _release_pinned()
    for step, ((loss, state), (e_loss, e_state)) in enumerate(zip(actual, expected), 1):
        assert torch.equal(loss, e_loss), f"step {step}: loss {loss.item()} vs {e_loss.item()}"
        worst = max(float((state[n] - e_state[n]).float().norm() / e_state[n].float().norm().clamp_min(1e-30))
                    for n in state)
        assert worst <= GRAD_RTOL, f"step {step}: LoRA parameters differ by {worst:.3e}"
        print(f"{regime} fraction {fraction} step {step}: loss {loss.item():.6f} bitwise, LoRA parameters "
              f"{'bitwise' if all(torch.equal(state[n], e_state[n]) for n in state) else f'within {worst:.2e}'}",
              flush=True)
    assert actual[2][0] != actual[0][0]  # the optimizer moved the model
    if regime == "B":
        # the non-checkpointed forward codes segments in every step once the ring is behind
        assert coded[0] > 0 and coded[1] > coded[0] and coded[2] > coded[1], coded
