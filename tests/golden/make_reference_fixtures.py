"""Write the reference-model fixtures for the harness block (run in the build container only).

What nothing else pins is whether the harness model in ``moss_offload/dit.py`` IS the
reference model as far as the hooks can tell: which tensors autograd saves, in which order,
with which layouts and aliasing, and what a step computes. This script imports the reference
(``training/model.py``, ``training/lora.py`` under ``$MOSS_REFERENCE``, default
``/root/reference``), runs it on the CPU in fp32 at BASELINE config 1, and writes data only:

  reference_manifest.json      saved-tensor manifests (regime B, regime A, a mixed
                               checkpoint_fraction = 0.5 two-block model, and a packed
                               two-sample traversal), parameter checksums, the loss, and
                               known answers of ``_checkpointed_layer_indices``
  reference_config1.safetensors  the regime-B model output and every LoRA gradient

The parameters and inputs come from ``fixture_init.py`` (keyed by parameter name), which the
test applies to the harness model in the same way. The reference itself never leaves this
container and nothing under tests/ imports it except this script.

Usage: python tests/golden/make_reference_fixtures.py
"""

from __future__ import annotations

import json
import os
import sys
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
import fixture_init as fx  # noqa: E402

REFERENCE = Path(os.environ.get("MOSS_REFERENCE", "/root/reference"))


def _reference():
    sys.path.insert(0, str(REFERENCE))
    from training import lora as ref_lora  # noqa: WPS433
    from training import model as ref_model

    return ref_model, ref_lora


def _build(ref_model, ref_lora, **overrides):
    config = dict(fx.CONFIG1)
    config.update(overrides)
    model = ref_model.MOSSImageTransformer(**config)
    ref_lora.inject_lora(model, rank=fx.LORA_RANK, alpha=fx.LORA_ALPHA, targets="joint")
    fx.init_parameters(model)
    return model.train()


def _step(model, latent, context):
    recorder = fx.SaveRecorder(model)
    model.zero_grad(set_to_none=True)
    with recorder.hooks():
        out = model(latent, torch.tensor([fx.TIMESTEP]), context)
        loss = out.square().mean()
    loss.backward()
    grads = {n: p.grad.detach().clone() for n, p in sorted(model.named_parameters()) if p.grad is not None}
    return recorder.records, out.detach(), loss.detach(), grads


def _packed_step(model, latent, context):
    # Two samples of different sizes in one traversal: the first at 16 x 16 with 64 text
    # tokens, the second a 8 x 12 crop of it with 40 text tokens.
    recorder = fx.SaveRecorder(model)
    targets = [latent[0], latent[0, :, :8, :12].contiguous()]
    contexts = [context[0], context[0, :40].contiguous()]
    with recorder.hooks():
        outs = model.forward_packed(targets, torch.tensor([fx.TIMESTEP, fx.TIMESTEP]), contexts)
        loss = sum(o.square().mean() for o in outs)
    loss.backward()
    return recorder.records, float(loss.detach())


def main() -> None:
    from safetensors.torch import save_file

    ref_model, ref_lora = _reference()
    torch.manual_seed(0)
    latent, context = fx.inputs()

    model_b = _build(ref_model, ref_lora)
    manifest_b, out_b, loss_b, grads_b = _step(model_b, latent, context)

    model_a = _build(ref_model, ref_lora, gradient_checkpointing=True)
    manifest_a, out_a, loss_a, _ = _step(model_a, latent, context)

    model_mixed = _build(ref_model, ref_lora, num_layers=2, gradient_checkpointing=True, checkpoint_fraction=0.5)
    manifest_mixed, _, loss_mixed, _ = _step(model_mixed, latent, context)

    model_packed = _build(ref_model, ref_lora)
    manifest_packed, loss_packed = _packed_step(model_packed, latent, context)

    fractions = {}
    for depth in (1, 2, 3, 40, 42):
        for fraction in (0.0, 0.1, 0.25, 0.5, 0.75, 0.9, 1.0):
            key = f"{depth}:{fraction}"
            fractions[key] = sorted(ref_model._checkpointed_layer_indices(depth, fraction))

    doc = {
        "source": "reference training/model.py + training/lora.py, CPU fp32, BASELINE config 1",
        "config": fx.CONFIG1,
        "lora": {"rank": fx.LORA_RANK, "alpha": fx.LORA_ALPHA, "targets": "joint"},
        "timestep": fx.TIMESTEP,
        "torch": torch.__version__,
        "parameter_checksums": fx.parameter_checksums(model_b),
        "loss": {
            "regime_b": float(loss_b),
            "regime_a": float(loss_a),
            "mixed_two_blocks": float(loss_mixed),
            "packed_two_samples": loss_packed,
        },
        "manifests": {
            "regime_b": manifest_b,
            "regime_a": manifest_a,
            "mixed_two_blocks": manifest_mixed,
            "packed_two_samples": manifest_packed,
        },
        "checkpointed_layer_indices": fractions,
    }
    (HERE / "reference_manifest.json").write_text(json.dumps(doc, indent=1, sort_keys=True) + "\n")
    tensors = {"output": out_b.contiguous()}
    tensors.update({f"grad.{name}": grad.contiguous() for name, grad in grads_b.items()})
    save_file(tensors, str(HERE / "reference_config1.safetensors"))
    print(
        f"regime B: {len(manifest_b)} saves, regime A: {len(manifest_a)}, mixed: {len(manifest_mixed)}, "
        f"packed: {len(manifest_packed)}; loss {float(loss_b):.9g}; {len(grads_b)} gradients"
    )


if __name__ == "__main__":
    main()
