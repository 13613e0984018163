"""The harness block against fixtures written from the reference model itself (CPU, fp32).

``tests/golden/make_reference_fixtures.py`` imported the reference ``training/model.py`` and
``training/lora.py`` in the build container, gave them the parameters and inputs of
``tests/golden/fixture_init.py`` (keyed by parameter name), and recorded what autograd saved
and what the step computed. Here ``moss_offload/dit.py`` gets the same parameters and inputs
and must reproduce:

- the saved-tensor manifests (order, shape, stride, storage offset, dtype, resident rule and
  aliasing structure) of BASELINE config 1 in regime B (no checkpointing), regime A (every
  block checkpointed), a two-block model at checkpoint_fraction 0.5 (one block of each), and a
  packed two-sample traversal: this is the input contract of the pack hook;
- the loss of each, the regime-B output and every LoRA gradient, to fp32 round-off;
- the reference's choice of checkpointed blocks (``_checkpointed_layer_indices``).

``test_planted_harness_mistakes_are_caught`` plants four mistakes in the harness (a norm
without its scale, a LoRA scale of 1, SiTU without its hidden cap, RoPE not applied) and
checks that the regime-B comparison rejects each.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import pytest
import torch
from safetensors.torch import load_file

from moss_offload import dit

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import fixture_init as fx  # noqa: E402

DOC = json.loads((GOLDEN / "reference_manifest.json").read_text())
TENSORS = load_file(str(GOLDEN / "reference_config1.safetensors"))

# fp32 on the CPU: the harness runs the reference's ops in the reference's order, so only
# the summation order inside library kernels may differ (it does not, on one machine, but
# the tolerance does not rely on that).
RTOL, ATOL = 1e-5, 1e-7


def _model(**overrides) -> dit.MOSSImageTransformer:
    config = dict(fx.CONFIG1)
    config.update(overrides)
    model = dit.MOSSImageTransformer(**config)
    dit.inject_lora(model, rank=fx.LORA_RANK, alpha=fx.LORA_ALPHA)
    fx.init_parameters(model)
    model.activation_offload = False
    return model.train()


def _step(model):
    latent, context = fx.inputs()
    recorder = fx.SaveRecorder(model)
    model.zero_grad(set_to_none=True)
    with recorder.hooks():
        out = model(latent, torch.tensor([fx.TIMESTEP]), context)
        loss = out.square().mean()
    loss.backward()
    grads = {n: p.grad.detach().clone() for n, p in sorted(model.named_parameters()) if p.grad is not None}
    return recorder.records, out.detach(), loss.detach(), grads


def _packed_step(model):
    latent, context = fx.inputs()
    recorder = fx.SaveRecorder(model)
    targets = [latent[0], latent[0, :, :8, :12].contiguous()]
    contexts = [context[0], context[0, :40].contiguous()]
    with recorder.hooks():
        outs = model.forward_packed(targets, torch.tensor([fx.TIMESTEP, fx.TIMESTEP]), contexts)
        loss = sum(o.square().mean() for o in outs)
    loss.backward()
    return recorder.records, float(loss.detach())


def _assert_manifest(actual, expected):
    assert len(actual) == len(expected), f"{len(actual)} saves, reference {len(expected)}"
    for index, (a, e) in enumerate(zip(actual, expected)):
        assert a == e, f"save {index}: harness {a}, reference {e}"


def test_parameters_match_the_reference_names_and_values() -> None:
    model = _model()
    assert fx.parameter_checksums(model) == DOC["parameter_checksums"]


def test_regime_b_manifest_loss_output_and_lora_gradients() -> None:
    records, out, loss, grads = _step(_model())
    _assert_manifest(records, DOC["manifests"]["regime_b"])
    torch.testing.assert_close(out, TENSORS["output"], rtol=RTOL, atol=ATOL)
    assert loss.item() == pytest.approx(DOC["loss"]["regime_b"], rel=RTOL)
    expected = {k[len("grad."):]: v for k, v in TENSORS.items() if k.startswith("grad.")}
    assert sorted(grads) == sorted(expected)
    assert len(expected) == 12  # A and B of q, k, v, o, ffn_up_gate, ffn_down
    for name, grad in grads.items():
        torch.testing.assert_close(grad, expected[name], rtol=RTOL, atol=ATOL, msg=name)


def test_regime_a_manifest_and_loss() -> None:
    records, _, loss, _ = _step(_model(gradient_checkpointing=True))
    _assert_manifest(records, DOC["manifests"]["regime_a"])
    assert loss.item() == pytest.approx(DOC["loss"]["regime_a"], rel=RTOL)


def test_mixed_checkpoint_fraction_manifest_and_loss() -> None:
    records, _, loss, _ = _step(_model(num_layers=2, gradient_checkpointing=True, checkpoint_fraction=0.5))
    _assert_manifest(records, DOC["manifests"]["mixed_two_blocks"])
    assert loss.item() == pytest.approx(DOC["loss"]["mixed_two_blocks"], rel=RTOL)


def test_packed_traversal_manifest_and_loss() -> None:
    records, loss = _packed_step(_model())
    _assert_manifest(records, DOC["manifests"]["packed_two_samples"])
    assert loss == pytest.approx(DOC["loss"]["packed_two_samples"], rel=RTOL)


def test_checkpointed_layer_indices_match_the_reference() -> None:
    for key, expected in DOC["checkpointed_layer_indices"].items():
        depth, fraction = key.split(":")
        assert sorted(dit.checkpointed_layer_indices(int(depth), float(fraction))) == expected, key


def _matches_regime_b(records, out, loss, grads) -> bool:
    """The comparison of the regime-B test, as a predicate."""

    expected = {k[len("grad."):]: v for k, v in TENSORS.items() if k.startswith("grad.")}
    return (
        records == DOC["manifests"]["regime_b"]
        and torch.allclose(out, TENSORS["output"], rtol=RTOL, atol=ATOL)
        and loss.item() == pytest.approx(DOC["loss"]["regime_b"], rel=RTOL)
        and sorted(grads) == sorted(expected)
        and all(torch.allclose(grads[n], expected[n], rtol=RTOL, atol=ATOL) for n in grads)
    )


def test_planted_harness_mistakes_are_caught(monkeypatch) -> None:
    # Each mistake is planted in the harness for one step; the regime-B comparison must reject
    # every one of them, and accept the harness as it is.
    assert _matches_regime_b(*_step(_model()))

    def norm_without_scale(m):
        def forward(self, tokens):
            normalized = tokens.float() * torch.rsqrt(tokens.float().square().mean(-1, keepdim=True) + 1e-6)
            return normalized.to(tokens.dtype)

        m.setattr(dit.RMSNorm, "forward", forward)

    def lora_scale_one(m):
        original = dit.LoRALinear.forward

        def forward(self, tokens):
            saved, self.scale = self.scale, 1.0
            try:
                return original(self, tokens)
            finally:
                self.scale = saved

        m.setattr(dit.LoRALinear, "forward", forward)

    def situ_without_hidden_cap(m):
        m.setattr(dit, "situ", lambda hidden, gate: (4.0 * torch.tanh(gate / 4.0) * torch.sigmoid(gate)) * hidden)

    def rope_not_applied(m):
        m.setattr(dit, "rotate_rope", lambda tokens, rope: tokens * 1.0)

    for patch in (norm_without_scale, lora_scale_one, situ_without_hidden_cap, rope_not_applied):
        with monkeypatch.context() as m:
            patch(m)
            result = _step(_model())
        assert not _matches_regime_b(*result), patch.__name__
