"""The drop-in ``activation_cpu_offload`` on the MOSS DiT harness, on the GPU.

Parity gates, following the reference's own (training/tests/test_packed_cuda.py:173-231):
the same seeded model is run with hooks off, with the engine, and with the oracle's
restatement of the reference hooks; outputs and gradients must agree. On top of the
reference's tolerance checks, every tensor the engine restores is compared bitwise with the
tensor that was saved, and the forward output with the engine is bitwise equal to the one
without hooks (the hooks only move data).
"""

from __future__ import annotations

import copy
import gc

import pytest
import torch

import moss_offload
from moss_offload import dit
from moss_offload.activation_offload import (
    _ActivationOffload,
    _CheckedAlias,
    _DerivedTensor,
    _OffloadedTensor,
)
from oracle import reference_hooks

from gpu_util import assert_bitwise, requires_gpu

pytestmark = requires_gpu


class _Recording(_ActivationOffload):
    """Engine context that also checks every restored tensor against a copy of the save."""

    log: dict = {}
    checked = 0

    kinds = (_OffloadedTensor, _DerivedTensor, _CheckedAlias)

    def pack(self, tensor):
        handle = super().pack(tensor)
        if isinstance(handle, _Recording.kinds):
            _Recording.log[id(handle)] = tensor.detach().clone()
        return handle

    def unpack(self, saved):
        restored = super().unpack(saved)
        # a derived save restores its inputs through handles of its own, which pack never
        # returned: those are checked through the derived result
        if isinstance(saved, _Recording.kinds) and id(saved) in _Recording.log:
            expected = _Recording.log[id(saved)]
            # an alias stands for a dense cast: its save's strides are the clone's
            stride = saved.stride if hasattr(saved, "stride") else expected.stride()
            assert restored.shape == expected.shape and restored.stride() == stride
            assert_bitwise(restored, expected)
            _Recording.checked += 1
        return restored


def _recording_context(model, enabled, device):
    if not enabled or device.type != "cuda" or not torch.is_grad_enabled():
        return moss_offload.activation_cpu_offload(model, enabled, device)
    return _Recording(model, device)


def _tiny(layers=3, checkpointing=False, lora=False, dim=32, ffn=64, heads=4):
    model = dit.MOSSImageTransformer(
        dim=dim, ffn_dim=ffn, num_heads=heads, num_layers=layers, text_dim=16, freq_dim=8, latent_channels=4,
        gradient_checkpointing=checkpointing,
    )
    dit.init_weights(model)
    if lora:
        dit.inject_lora(model, rank=2, alpha=4.0)
    return model


def _inputs(device, seed=902, shapes=((4, 3, 5),), text=(6,)):
    g = torch.Generator(device="cpu").manual_seed(seed)
    latents = [torch.randn(1, c, h, w, generator=g).to(device) for c, h, w in shapes]
    contexts = [torch.randn(1, n, 16, generator=g).to(device) for n in text]
    return latents, contexts


def _run(model, context_factory, enabled, latents, contexts, autocast=False, retain=1):
    model.activation_offload = enabled
    model.offload_context = context_factory
    model.zero_grad(set_to_none=True)
    t = torch.tensor([500.0], device=latents[0].device)
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        outputs = [model(x, t, c) for x, c in zip(latents, contexts)]
        loss = sum(o.float().square().mean() for o in outputs)
    for k in range(retain):
        loss.backward(retain_graph=k + 1 < retain)
    grads = {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None}
    return [o.detach() for o in outputs], loss.detach(), grads


def _compare(actual, expected, rtol, atol, bitwise_outputs=True):
    outs, loss, grads = actual
    e_outs, e_loss, e_grads = expected
    for a, b in zip(outs, e_outs):
        if bitwise_outputs:
            assert_bitwise(a, b)
        else:
            torch.testing.assert_close(a, b, rtol=rtol, atol=atol)
    torch.testing.assert_close(loss, e_loss, rtol=rtol, atol=atol)
    assert grads.keys() == e_grads.keys()
    for name in grads:
        torch.testing.assert_close(grads[name], e_grads[name], rtol=rtol, atol=atol, msg=name)


@pytest.mark.parametrize("checkpointing", [False, True])
@pytest.mark.parametrize("lora", [False, True])
def test_fp32_step_matches_no_offload_and_reference_hooks(checkpointing, lora) -> None:
    device = torch.device("cuda", 0)
    torch.manual_seed(903)
    base = _tiny(checkpointing=checkpointing, lora=lora).to(device).train()
    latents, contexts = _inputs(device)
    expected = _run(copy.deepcopy(base), moss_offload.activation_cpu_offload, False, latents, contexts)
    reference = _run(copy.deepcopy(base), reference_hooks.activation_cpu_offload, True, latents, contexts)
    _Recording.log, _Recording.checked = {}, 0
    actual = _run(copy.deepcopy(base), _recording_context, True, latents, contexts)
    assert _Recording.checked > 0
    _compare(actual, expected, rtol=5e-5, atol=5e-6)
    _compare(actual, reference, rtol=5e-5, atol=5e-6)


@pytest.mark.parametrize("mlp", dit.MLP_VARIANTS)
def test_config1_block_fp32_restores_bit_exact(mlp) -> None:
    """BASELINE config 1 on the GPU: hidden 512, 8x64 heads, MLP 2048 (the reference's SiTU-GLU,
    and the GELU MLP BASELINE names), 256 image + 64 text."""

    device = torch.device("cuda", 0)
    torch.manual_seed(0)
    model = dit.MOSSImageTransformer(
        dim=512, ffn_dim=2048, num_heads=8, num_layers=1, text_dim=64, freq_dim=32, latent_channels=16, mlp=mlp,
    )
    dit.init_weights(model)
    model = model.to(device).train()
    g = torch.Generator(device="cpu").manual_seed(0)
    latents = [torch.randn(1, 16, 16, 16, generator=g).to(device)]
    contexts = [torch.randn(1, 64, 64, generator=g).to(device)]
    expected = _run(copy.deepcopy(model), moss_offload.activation_cpu_offload, False, latents, contexts)
    _Recording.log, _Recording.checked = {}, 0
    actual = _run(copy.deepcopy(model), _recording_context, True, latents, contexts)
    assert _Recording.checked > 30
    _compare(actual, expected, rtol=5e-5, atol=5e-6)


@pytest.mark.parametrize("checkpointing", [False, True])
def test_bf16_lora_step_within_north_star_tolerance(checkpointing) -> None:
    device = torch.device("cuda", 0)
    torch.manual_seed(904)
    base = _tiny(layers=4, checkpointing=checkpointing, lora=True, dim=64, ffn=256, heads=4).to(device)
    base = base.to(torch.bfloat16).train()
    for module in base.modules():
        if isinstance(module, dit.LoRALinear):
            module.lora_A.data = module.lora_A.data.float()
            module.lora_B.data = module.lora_B.data.float()
    latents, contexts = _inputs(device, shapes=((4, 8, 8),), text=(12,))
    expected = _run(copy.deepcopy(base), moss_offload.activation_cpu_offload, False, latents, contexts, autocast=True)
    _Recording.log, _Recording.checked = {}, 0
    actual = _run(copy.deepcopy(base), _recording_context, True, latents, contexts, autocast=True)
    assert _Recording.checked > 0
    _compare(actual, expected, rtol=1e-3, atol=1e-5)


@pytest.fixture
def hipdma_engine():
    """Engines created inside the test use the HIP-stream DMA transport."""

    from moss_offload import engine as engine_mod

    engine_mod.reset_engines()
    previous = engine_mod.configure()
    engine_mod.configure(link="hipdma")
    yield
    gc.collect()
    torch.cuda.synchronize()
    engine_mod.reset_engines()
    engine_mod.configure(link=previous.link)


@pytest.mark.parametrize("checkpointing", [False, True])
def test_hipdma_link_bf16_lora_step_restores_bit_exact(hipdma_engine, checkpointing) -> None:
    from moss_offload import engine as engine_mod

    device = torch.device("cuda", 0)
    torch.manual_seed(904)
    model = _tiny(layers=4, checkpointing=checkpointing, lora=True, dim=64, ffn=128).to(device).train()
    latents, contexts = _inputs(device, shapes=((4, 8, 8),), text=(12,))
    expected = _run(model, moss_offload.activation_cpu_offload, False, latents, contexts, autocast=True)
    _Recording.checked = 0
    actual = _run(model, _recording_context, True, latents, contexts, autocast=True)
    assert _Recording.checked > 0
    _compare(actual, expected, rtol=1e-3, atol=1e-5)
    engine = engine_mod.get_engine(device)
    assert engine.link_name() == "hipdma"
    assert engine.stats()["host_blocks"] == 0


def test_retain_graph_subset_grad_and_dropped_graph() -> None:
    device = torch.device("cuda", 0)
    torch.manual_seed(905)
    base = _tiny(lora=True).to(device).train()
    latents, contexts = _inputs(device)
    expected = _run(copy.deepcopy(base), moss_offload.activation_cpu_offload, False, latents, contexts, retain=2)
    actual = _run(copy.deepcopy(base), moss_offload.activation_cpu_offload, True, latents, contexts, retain=2)
    _compare(actual, expected, rtol=5e-5, atol=5e-6)

    engine = moss_offload.get_engine(device)
    # torch.autograd.grad over a subset of the graph
    model = copy.deepcopy(base)
    model.activation_offload = True
    t = torch.tensor([500.0], device=device)
    out = model(latents[0], t, contexts[0])
    target = [p for n, p in model.named_parameters() if p.requires_grad and n.startswith("layers.2.")]
    (sub,) = torch.autograd.grad(out.square().mean(), target[:1])
    ref_model = copy.deepcopy(base)
    ref_out = ref_model(latents[0], t, contexts[0])
    ref_target = [p for n, p in ref_model.named_parameters() if p.requires_grad and n.startswith("layers.2.")]
    (ref_sub,) = torch.autograd.grad(ref_out.square().mean(), ref_target[:1])
    torch.testing.assert_close(sub, ref_sub, rtol=5e-5, atol=5e-6)
    del out, sub
    # a graph that is never backpropagated
    out = model(latents[0], t, contexts[0])
    assert engine.live_groups() > 0
    del out
    gc.collect()
    torch.cuda.synchronize(device)
    assert engine.live_groups() == 0
    engine.synchronize()
    assert engine.stats()["host_bytes_in_use"] == 0


def test_several_forwards_one_backward() -> None:
    """Config-5 unpacked mode: one forward per shape group, one backward over all graphs."""

    device = torch.device("cuda", 0)
    torch.manual_seed(906)
    base = _tiny(lora=True, checkpointing=True).to(device).train()
    latents, contexts = _inputs(device, shapes=((4, 4, 4), (4, 3, 5), (4, 5, 3), (4, 4, 2)), text=(6, 4, 5, 3))
    expected = _run(copy.deepcopy(base), moss_offload.activation_cpu_offload, False, latents, contexts)
    _Recording.log, _Recording.checked = {}, 0
    actual = _run(copy.deepcopy(base), _recording_context, True, latents, contexts)
    _compare(actual, expected, rtol=5e-5, atol=5e-6)


def _config5_tiny(device):
    torch.manual_seed(907)
    model = _tiny(layers=3, checkpointing=True, dim=64, ffn=128, heads=4)
    model = model.to(device).to(torch.bfloat16)
    dit.quantize_joint_linears(model, torch.Generator(device=device).manual_seed(5))
    dit.inject_lora(model, rank=4, alpha=4.0)
    return model.train()


def _packed_run(model, context_factory, enabled, latents, contexts):
    model.activation_offload = enabled
    model.offload_context = context_factory
    model.zero_grad(set_to_none=True)
    t = torch.linspace(200.0, 800.0, len(latents), device=latents[0].device)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        outputs = model.forward_packed([x[0] for x in latents], t, [c[0] for c in contexts])
        loss = sum(o.float().square().mean() for o in outputs)
    loss.backward()
    grads = {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None}
    return [o.detach() for o in outputs], loss.detach(), grads


def test_config5_int8_lora_grouped_and_packed_match_no_offload() -> None:
    """Config-5 shape: int8 weight-only bases (their int8 weights and fp32 scales are buffers and
    stay resident), LoRA, checkpointed blocks, four aspect buckets, both batching modes."""

    device = torch.device("cuda", 0)
    base = _config5_tiny(device)
    latents, contexts = _inputs(device, shapes=((4, 4, 4), (4, 3, 5), (4, 5, 3), (4, 4, 6)), text=(6, 4, 5, 3))
    for runner in (_run, _packed_run):
        kwargs = {"autocast": True} if runner is _run else {}
        expected = runner(copy.deepcopy(base), moss_offload.activation_cpu_offload, False, latents, contexts, **kwargs)
        _Recording.log, _Recording.checked = {}, 0
        actual = runner(copy.deepcopy(base), _recording_context, True, latents, contexts, **kwargs)
        assert _Recording.checked > 0
        assert len(expected[2]) > 0
        # every restored tensor was checked bitwise above; outputs and gradients within the
        # north_star bf16 tolerance (backward reductions may order differently run to run)
        _compare(actual, expected, rtol=1e-3, atol=1e-5)


def test_weight_backed_and_staging_buffers_stay_resident() -> None:
    device = torch.device("cuda", 0)
    model = _tiny().to(device).train()
    staging = torch.randn(64, device=device, requires_grad=False)

    class Manager:
        def owned_cuda_buffers(self):
            return (staging,)

    model.block_swap_manager = Manager()
    ctx = moss_offload.activation_cpu_offload(model, True, device)
    with ctx:
        weight_view = model.layers[0].proj["q"].weight.t()
        assert ctx.pack(weight_view) is weight_view
        assert ctx.pack(staging[8:]) is not None and isinstance(ctx.pack(staging[8:]), torch.Tensor)
        cpu = torch.randn(3)
        assert ctx.pack(cpu) is cpu
        overlapping = torch.randn(16, device=device).as_strided((3, 3), (1, 1))
        assert ctx.pack(overlapping) is overlapping
        handle = ctx.pack(torch.randn(4, 0, device=device))
        assert isinstance(handle, _OffloadedTensor) and ctx.unpack(handle).shape == (4, 0)


def test_keep_last_blocks_keeps_the_tail_resident_and_matches_no_offload() -> None:
    device = torch.device("cuda", 0)
    torch.manual_seed(911)
    base = _tiny(layers=3, checkpointing=False).to(device).train()
    latents, contexts = _inputs(device, seed=912)
    expected = _run(copy.deepcopy(base), moss_offload.activation_cpu_offload, False, latents, contexts)
    engine = moss_offload.get_engine(device)
    packed = {}
    try:
        for keep in (0, 1, 3):
            engine.config.keep_last_blocks = keep
            engine.synchronize()
            engine.reset_stats()
            actual = _run(copy.deepcopy(base), moss_offload.activation_cpu_offload, True, latents, contexts)
            engine.synchronize()
            packed[keep] = engine.stats()["bytes_packed"]
            _compare(actual, expected, rtol=5e-5, atol=5e-6)
    finally:
        engine.config.keep_last_blocks = 0
    # one of three blocks kept: about a third less; every block kept: only the saves outside blocks
    assert 0 < packed[1] < packed[0] and packed[3] < packed[1]
    assert packed[1] <= packed[0] * 0.8


class _SavesAliasingViews(torch.autograd.Function):
    """Saves three views of one storage (the same bytes in the same order) and one slice of
    another region; backward reads every save through its own view."""

    @staticmethod
    def forward(ctx, x):
        heads = x.view(x.shape[0], x.shape[1], 4, -1).permute(0, 2, 1, 3)  # [B,H,T,hd] over [B,T,D]
        flat = x.view(-1, x.shape[-1])
        tail = x[:, 1:]
        ctx.save_for_backward(x, heads, flat, tail)
        return x * 2.0

    @staticmethod
    def backward(ctx, grad):
        x, heads, flat, tail = ctx.saved_tensors
        assert heads.shape[1] == 4 and heads.stride() == (x.stride(0), x.shape[-1] // 4, x.stride(1), 1)
        merged = heads.permute(0, 2, 1, 3).reshape(x.shape) + flat.view(x.shape) - x
        out = grad * 2.0 + merged * 0.0
        out[:, 1:] += tail * 0.0
        return out + (merged - x).abs().sum() + (tail - x[:, 1:]).abs().sum()


def test_views_of_the_same_bytes_cross_the_link_once() -> None:
    """Dedupe by payload bytes: a transposed or reshaped view of an already offloaded tensor
    reuses its host copy; a slice covering other bytes is copied on its own."""

    device = torch.device("cuda", 0)
    model = _tiny().to(device)
    torch.manual_seed(913)
    x = torch.randn(2, 24, 32, device=device, requires_grad=True)
    base = x * 1.0
    engine = moss_offload.get_engine(device)
    engine.synchronize()
    engine.reset_stats()
    _Recording.log, _Recording.checked = {}, 0
    with _Recording(model, device):
        y = _SavesAliasingViews.apply(base)
    engine.synchronize()
    packed = engine.stats()["bytes_packed"]
    element = base.element_size()
    assert packed == base.numel() * element + base[:, 1:].numel() * element
    y.sum().backward()
    assert _Recording.checked == 4
    torch.testing.assert_close(x.grad, torch.full_like(x, 2.0), rtol=0, atol=0)


def test_bf16_casts_cross_narrowed_and_restore_bit_exact() -> None:
    """Under bf16 autocast the harness's RMSNorm saves float32 casts of bfloat16 tokens. Those
    cross the link as their high halves (MO_TENSOR_BF16_HIGH): fewer bytes packed, every
    restored tensor still bitwise the save, and the step matches the run without offloading."""

    device = torch.device("cuda", 0)
    torch.manual_seed(914)
    base = _tiny(layers=2, checkpointing=False, lora=True, dim=64, ffn=128).to(device).train()
    latents, contexts = _inputs(device, seed=915, shapes=((4, 8, 8),), text=(12,))
    expected = _run(copy.deepcopy(base), moss_offload.activation_cpu_offload, False, latents, contexts, autocast=True)
    engine = moss_offload.get_engine(device)
    packed = {}
    try:
        for narrow in (False, True):
            engine.config.narrow_bf16_casts = narrow
            engine.synchronize()
            engine.reset_stats()
            _Recording.log, _Recording.checked = {}, 0
            actual = _run(copy.deepcopy(base), _recording_context, True, latents, contexts, autocast=True)
            engine.synchronize()
            packed[narrow] = engine.stats()["bytes_packed"]
            assert _Recording.checked > 0  # every restore compared bitwise with its save
            _compare(actual, expected, rtol=1e-3, atol=1e-5)
    finally:
        engine.config.narrow_bf16_casts = True
    # two float32 casts per RMSNorm (square and scale), each crossing at half size
    assert packed[True] < packed[False]


def test_products_are_recomputed_not_offloaded_and_restore_bit_exact() -> None:
    """The SiTU-GLU activation (reference training/model.py:38) saves 4 tanh(g/4), 25 tanh(h/25),
    their product chain and a view of the result: products of saves already held. Those are
    recomputed on unpack by the same torch.mul (no bytes over the link), every restore is bitwise
    the save, and the step matches the run without offloading, in fp32 and under bf16 autocast."""

    device = torch.device("cuda", 0)
    torch.manual_seed(916)
    base = _tiny(layers=2, checkpointing=False, lora=True, dim=64, ffn=128).to(device).train()
    latents, contexts = _inputs(device, seed=917, shapes=((4, 8, 8),), text=(12,))
    engine = moss_offload.get_engine(device)
    for autocast in (False, True):
        expected = _run(copy.deepcopy(base), moss_offload.activation_cpu_offload, False, latents, contexts,
                        autocast=autocast)
        packed, derived = {}, {}
        try:
            for recompute in (False, True):
                engine.config.recompute_products = recompute
                engine.synchronize()
                engine.reset_stats()
                _Recording.log, _Recording.checked = {}, 0
                _derived_ids.clear()
                actual = _run(copy.deepcopy(base), _recording_context, True, latents, contexts, autocast=autocast)
                engine.synchronize()
                packed[recompute] = engine.stats()["bytes_packed"]
                assert _Recording.checked > 0
                derived[recompute] = sum(1 for k in _Recording.log if k in _derived_ids)
                if autocast:
                    _compare(actual, expected, rtol=1e-3, atol=1e-5)
                else:
                    _compare(actual, expected, rtol=5e-5, atol=5e-6)
        finally:
            engine.config.recompute_products = True
        assert packed[True] < packed[False]
        assert derived[True] > 0 and derived[False] == 0


_derived_ids: set = set()
_base_pack = _Recording.pack


_made_handles: list = []  # aliases returned by pack, in order


def _pack_noting_derived(self, tensor):
    handle = _base_pack(self, tensor)
    if isinstance(handle, _DerivedTensor):
        _derived_ids.add(id(handle))
    if isinstance(handle, _CheckedAlias):
        _made_handles.append(handle)
    return handle


_Recording.pack = _pack_noting_derived


def test_equal_casts_restore_bit_exact() -> None:
    """Under bf16 autocast each RMSNorm of the harness block saves two float32 casts of the same
    bfloat16 tokens (reference training/model.py:171). The second restores from the first one's
    entry once the device has found the bytes equal: fewer bytes packed, every restore bitwise
    the save, and the step matches the run without offloading."""

    device = torch.device("cuda", 0)
    torch.manual_seed(918)
    # dim 512 and 640 joint tokens: a float32 cast of [T, D] is 1.3 MB, above the aliasing floor
    # of 1 MiB (the text adapter's 64-token casts stay below it)
    base = _tiny(layers=2, checkpointing=False, lora=True, dim=512, ffn=1024, heads=8).to(device).train()
    latents, contexts = _inputs(device, seed=919, shapes=((4, 24, 24),), text=(64,))
    expected = _run(copy.deepcopy(base), moss_offload.activation_cpu_offload, False, latents, contexts, autocast=True)
    engine = moss_offload.get_engine(device)
    packed, made = {}, {}
    try:
        for on in (False, True):
            engine.config.alias_equal_casts = on
            engine.synchronize()
            engine.reset_stats()
            _Recording.log, _Recording.checked = {}, 0
            _made_handles.clear()
            actual = _run(copy.deepcopy(base), _recording_context, True, latents, contexts, autocast=True)
            engine.synchronize()
            packed[on] = engine.stats()["bytes_packed"]
            made[on] = len(_made_handles)
            # every alias settles as equal: the casts it stands for were never written
            assert all(h.settle(True) and h.tensor is None and h.target is not None for h in _made_handles)
            assert _Recording.checked > 0
            _compare(actual, expected, rtol=1e-3, atol=1e-5)
    finally:
        _made_handles.clear()
        engine.config.alias_equal_casts = True
    # at least the q- and k-norms of both blocks (bfloat16 inputs); one cast of each pair moves
    assert made[False] == 0 and made[True] >= 4, made
    assert packed[True] < packed[False]


def test_cast_written_between_casts_stays_resident_and_matches() -> None:
    """Two casts of one tensor with a ``no_grad`` write in between share an autograd origin but
    not their bytes: the device comparison finds the difference, the second cast stays on the
    device as saved, and the gradients are bitwise those of the run without hooks."""

    device = torch.device("cuda", 0)
    model = _tiny().to(device)
    g = torch.Generator(device=device).manual_seed(920)
    x0 = torch.randn(512, 1024, device=device, generator=g).to(torch.bfloat16)

    def step(context):
        x = x0.clone().requires_grad_(True)
        t = x * 1.0
        with context:
            b = t.float()
            y1 = b.square()  # saves b, offloaded
            with torch.no_grad():
                t.add_(1.0)  # not seen by either cast's node
            a = t.float()
            y2 = a.square()  # saves a: same origin as b, other bytes
        (y1.sum() + y2.sum()).backward()
        return x.grad

    expected = step(torch.enable_grad())
    _Recording.log, _Recording.checked = {}, 0
    _made_handles.clear()
    got = step(_Recording(model, device))
    aliases = [h for h in _made_handles if isinstance(h, _CheckedAlias)]
    _made_handles.clear()
    assert len(aliases) == 1
    alias = aliases[0]
    assert alias.ticket == 0 and alias.target is None and alias.tensor is not None
    assert _Recording.checked == 2
    assert_bitwise(got, expected)
