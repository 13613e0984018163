"""CPU tests of the drop-in's host logic: the gate, the config-1 plumbing and the manifest probe.

- The gate of ``activation_cpu_offload`` (reference training/activation_offload.py:92-93): on
  the CPU, when disabled and under ``no_grad``, the drop-in is an exact no-op and never touches
  the native library. ``test_activation_offload_is_cpu_noop`` restates the reference's own test
  (training/tests/test_packed_features.py:188-198, seed 33, same tiny model sizes).
- BASELINE config 1 on the CPU: one reference-topology block (hidden 512, 8x64 heads, MLP 2048,
  fp32, 16x16 image + 64 text tokens), with the reference's SiTU-GLU MLP and with the GELU MLP
  that BASELINE names, through the oracle's emulation of the reference hooks
  with CPU payloads. Every restored tensor is bitwise equal to its save, and the loss and
  every gradient are bitwise equal to the run without hooks. The manifest probe records the
  same offloaded set the hooks packed.
- The dedupe key of the engine's hook (``_payload_key``): equal for every view of the same
  bytes (transposed, reshaped, expanded), different for a shifted, strided, partial or
  same-size view of other bytes; the manifest counts aliasing views once.
- The narrowing test of the hook (``_bf16_exact``): only the untouched float32 output of a
  bfloat16 -> float32 cast qualifies.
- The manifest probe lets the graph go when the forward is dropped (regression: a pack hook
  that returns its argument ties outputs saved by their own node into an uncollectable cycle).
"""

from __future__ import annotations

import copy
import weakref
import gc
from contextlib import nullcontext

import pytest
import torch

import moss_offload
from moss_offload import dit, engine
from moss_offload.activation_offload import _bf16_exact, _offload_view, _payload_key
from moss_offload.manifest import ManifestRecorder
from oracle import reference_hooks


def _tiny(layers=2, checkpointing=False):
    # sizes of the reference's _tiny (training/tests/test_packed_features.py:31-41)
    return dit.MOSSImageTransformer(
        dim=32, ffn_dim=64, num_heads=4, num_layers=layers, text_dim=16, freq_dim=8, latent_channels=4,
        gradient_checkpointing=checkpointing,
    )


def test_activation_offload_is_cpu_noop() -> None:
    torch.manual_seed(33)
    base = _tiny().train()
    offloaded = copy.deepcopy(base).train()
    offloaded.activation_offload = True
    target = torch.randn(1, 4, 2, 2)
    context = torch.randn(1, 2, 16)
    expected = base(target, torch.tensor([250.0]), context)
    actual = offloaded(target, torch.tensor([250.0]), context)
    torch.testing.assert_close(actual, expected)
    actual.sum().backward()
    assert not engine._ENGINES  # the CPU path never created a device engine


def test_gate_returns_nullcontext_without_touching_the_engine() -> None:
    model = _tiny()
    cuda = torch.device("cuda", 0)
    assert isinstance(moss_offload.activation_cpu_offload(model, True, torch.device("cpu")), nullcontext)
    assert isinstance(moss_offload.activation_cpu_offload(model, False, cuda), nullcontext)
    with torch.no_grad():
        assert isinstance(moss_offload.activation_cpu_offload(model, True, cuda), nullcontext)
    with torch.inference_mode():
        assert isinstance(moss_offload.activation_cpu_offload(model, True, cuda), nullcontext)
    assert not engine._ENGINES


def _config1(mlp="situ"):
    torch.manual_seed(0)
    model = dit.MOSSImageTransformer(
        dim=512, ffn_dim=2048, num_heads=8, num_layers=1, text_dim=64, freq_dim=32, latent_channels=16, mlp=mlp,
    )
    dit.init_weights(model)
    dit.inject_lora(model, rank=8, alpha=8.0, b_std=0.03)
    g = torch.Generator(device="cpu").manual_seed(0)
    latent = torch.randn(1, 16, 16, 16, generator=g)
    context = torch.randn(1, 64, 64, generator=g)
    return model.train(), latent, context


def _step(model, latent, context, hooks):
    model.zero_grad(set_to_none=True)
    with hooks:
        out = model(latent, torch.tensor([500.0]), context)
        loss = out.square().mean()
    loss.backward()
    grads = {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None}
    return out.detach(), loss.detach(), grads


@pytest.mark.parametrize("mlp", dit.MLP_VARIANTS)
def test_config1_block_through_emulated_reference_hooks_is_bitwise_identity(mlp) -> None:
    """Config 1 with the reference's SiTU-GLU block and with the GELU MLP BASELINE names."""

    model, latent, context = _config1(mlp)
    expected = _step(copy.deepcopy(model), latent, context, nullcontext())
    recorder = reference_hooks.Recorder()
    hooked = copy.deepcopy(model)
    actual = _step(hooked, latent, context, reference_hooks.emulated_offload(hooked, recorder))
    assert reference_hooks.bitwise_equal(actual[0], expected[0])
    assert reference_hooks.bitwise_equal(actual[1], expected[1])
    assert actual[2].keys() == expected[2].keys() and len(actual[2]) > 0
    for name in expected[2]:
        assert reference_hooks.bitwise_equal(actual[2][name], expected[2][name]), name
    # every offloaded save came back with its layout and bits
    assert len(recorder.packed) > 30 and len(recorder.restored) == len(recorder.packed)
    originals = {id(p): t for t, p in recorder.packed}
    assert len(originals) == len(recorder.packed)
    for original, payload in recorder.packed:
        assert payload.is_contiguous()
    by_bits = {}
    for original, _ in recorder.packed:
        by_bits.setdefault((tuple(original.shape), tuple(original.stride()), original.dtype), []).append(original)
    for restored in recorder.restored:
        candidates = by_bits[(tuple(restored.shape), tuple(restored.stride()), restored.dtype)]
        assert any(reference_hooks.bitwise_equal(restored, c) for c in candidates)


def test_manifest_matches_the_hooks_offloaded_set() -> None:
    model, latent, context = _config1()
    recorder = reference_hooks.Recorder()
    hooked = copy.deepcopy(model)
    with reference_hooks.emulated_offload(hooked, recorder):
        hooked(latent, torch.tensor([500.0]), context).square().mean()
    probe = ManifestRecorder(model, device_type="cpu")
    with probe:
        model(latent, torch.tensor([500.0]), context).square().mean()
    offloaded = probe.offloaded()
    assert len(offloaded) == len(recorder.packed)
    assert sum(r.resident != "" for r in probe.records) == recorder.resident
    assert probe.payload_bytes(unique=False) == recorder.payload_bytes
    assert [tuple(r.shape) for r in offloaded] == [tuple(t.shape) for t, _ in recorder.packed]
    # dup structure: fp32 RMSNorm saves its rsqrt statistic twice (square and mul)
    assert any(r.dup_of is not None for r in offloaded)
    assert probe.payload_bytes(unique=True) < probe.payload_bytes(unique=False)


def _key(tensor):
    return _payload_key(_offload_view(tensor)[0])


def test_payload_key_names_bytes_not_views() -> None:
    a = torch.randn(1, 7, 4, 5)
    same = (a.view(1, 7, 20), a.permute(0, 2, 1, 3), a.view(7, 20).t(), a.unsqueeze(0), a.view(140))
    assert all(_key(v) == _key(a) for v in same)
    assert _key(a) == (0, ((140, 4),), 4)
    other = (a[:, 1:], a[..., :4], a[:, ::2], a.view(35, 4)[:, :2], a.view(140)[1:], a.view(140)[:-1])
    keys = {_key(v) for v in other}
    assert _key(a) not in keys and len(keys) == len(other)
    # expanded dimensions are narrowed before keying: a broadcast view names its source's bytes
    c = torch.randn(2, 3)
    assert _key(c[:, None, :].expand(2, 4, 3)) == _key(c)
    # equal element counts at different positions
    x = torch.randn(6, 8)
    assert _key(x[:, :4]) != _key(x[:3])
    # half of a [B,T,H,hd] tensor by head vs by token: same count, different bytes
    y = torch.randn(2, 6, 4, 8)
    assert _key(y[:, :, :2]) != _key(y[:, :3])


def test_manifest_counts_aliasing_views_once() -> None:
    class SavesViews(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x):
            ctx.save_for_backward(x, x.view(x.shape[0], -1, 4, 8).transpose(1, 2), x.view(-1), x[:, 1:])
            return x.clone()

        @staticmethod
        def backward(ctx, grad):
            return grad

    x = torch.randn(2, 6, 32) * 1.0
    probe = ManifestRecorder(device_type="cpu")
    with probe:
        SavesViews.apply(x.requires_grad_())
    offloaded = probe.offloaded()
    assert len(offloaded) == 4
    assert [r.dup_of for r in offloaded] == [None, offloaded[0].index, offloaded[0].index, None]
    assert probe.payload_bytes(unique=True) == (x.numel() + x[:, 1:].numel()) * 4


def test_bf16_exact_reads_the_cast_from_the_graph() -> None:
    def ok(t):
        return _bf16_exact(t, _offload_view(t)[0])

    x = torch.randn(64, 32, dtype=torch.bfloat16, requires_grad=True)
    assert ok((x * 2).float())  # cast of an op's bf16 output
    assert ok(x.to(torch.float32))  # cast of a bf16 leaf
    assert torch.equal(x.float().to(torch.bfloat16).float(), x.float())
    h = torch.randn(64, 32, dtype=torch.float16, requires_grad=True)
    assert not ok((h * 2).float())  # float16 source
    f = torch.randn(64, 32, requires_grad=True)
    assert not ok((f * 2).float())  # float32 -> float32 is no cast
    y = (x * 2).float()
    assert not ok(y.view(32, 64))  # a view: its own node
    assert not ok((x * 2).float()[:, :16])
    with torch.no_grad():
        z = (x * 2).float()
    assert not ok(z)  # no graph, no proof
    w = (x * 2).float()
    with torch.no_grad():
        w.mul_(1.5)  # the node still reads ToCopyBackward0, the version does not
    assert not ok(w)
    assert not ok((x * 2).float() * 1.0)


def _live_tensor_ids():
    gc.collect()
    return {id(o) for o in gc.get_objects() if type(o) is torch.Tensor}


def test_manifest_probe_releases_the_graph() -> None:
    torch.manual_seed(1)
    model = _tiny(layers=2).train()
    latent, context = torch.randn(1, 4, 4, 4), torch.randn(1, 3, 16)
    model(latent, torch.tensor([300.0]), context).sum().backward()  # warm caches
    before = _live_tensor_ids()
    probe = ManifestRecorder(model, device_type="cpu")
    with probe:
        out = model(latent, torch.tensor([300.0]), context).sum()
    assert len(probe.records) > 10
    del out
    assert _live_tensor_ids() - before == set()


def test_manifest_probe_leaves_gradients_unchanged() -> None:
    torch.manual_seed(2)
    model = _tiny(layers=2).train()
    dit.inject_lora(model, rank=2, alpha=4.0, b_std=0.03)
    latent, context = torch.randn(1, 4, 4, 4), torch.randn(1, 3, 16)
    expected = _step(copy.deepcopy(model), latent, context, nullcontext())
    probed = copy.deepcopy(model)
    actual = _step(probed, latent, context, ManifestRecorder(probed, device_type="cpu"))
    for name in expected[2]:
        assert reference_hooks.bitwise_equal(actual[2][name], expected[2][name]), name


class _StubEngine:
    """Bookkeeping of the device engine, with the byte comparison done at once on the CPU."""

    class config:
        dedupe = True
        narrow_bf16_casts = True
        recompute_products = True
        alias_equal_casts = True
        keep_last_blocks = 0

    def __init__(self):
        self.results = {}
        self.discarded = []
        self.acquired = []  # (group, entry, reader) of every extra reference taken

    def acquire(self, gid, idx, reader=True):
        self.acquired.append((gid, idx, reader))
        return True

    def drop(self, gid, idx, reader=True):
        pass

    def equal(self, a, b, stream):
        ticket = len(self.results) + len(self.discarded) + 1
        same = a.numel() == b.numel() and torch.equal(a.reshape(-1).view(torch.uint8), b.reshape(-1).view(torch.uint8))
        self.results[ticket] = 1 if same else 2
        return ticket

    def equal_result(self, ticket, wait):
        return self.results.pop(ticket)

    def equal_discard(self, ticket):
        self.discarded.append(self.results.pop(ticket))


def _derive_context():
    from moss_offload.activation_offload import _ActivationOffload

    ctx = _ActivationOffload.__new__(_ActivationOffload)
    ctx.engine = _StubEngine()
    ctx.recompute = True
    ctx.alias = True
    ctx._made = {}
    ctx._casts = {}
    ctx._pending = []
    return ctx


def test_recomputed_products_are_found_from_the_graph() -> None:
    """The rule of ``_ActivationOffload._derive``: a save is recomputed only when it is the
    untouched output of ``torch.mul`` over saves already held (tensor x tensor of one shape, or
    tensor x Python number), or a dense view of one. The activation is the reference's SiTU-GLU
    (training/model.py:38)."""

    from moss_offload.activation_offload import _DerivedTensor, _OffloadedTensor

    ctx = _derive_context()

    def held(t, gid):
        h = _OffloadedTensor(None, gid, 0, t.device, t.dtype, tuple(t.shape), tuple(t.stride()), tuple(t.shape))
        ctx._remember(t, h)
        return h

    gate = torch.randn(6, 16, dtype=torch.bfloat16, requires_grad=True) * 1.0
    hidden = torch.randn(6, 16, dtype=torch.bfloat16, requires_grad=True) * 1.0
    t1 = torch.tanh(gate / 4.0)
    s = torch.sigmoid(gate)
    t2 = torch.tanh(hidden / 25.0)
    held(t1, 1), held(s, 2), held(t2, 3)
    a4 = 4.0 * t1
    d4 = ctx._derive(a4)
    assert isinstance(d4, _DerivedTensor) and d4.scalar == 4.0 and len(d4.inputs) == 1
    # the replay only reads its input: its reference is not a reader's
    assert ctx.engine.acquired[-1] == (1, 0, False) and not d4.inputs[0].reader
    ctx._remember(a4, d4)
    p = a4 * s
    dp = ctx._derive(p)
    assert isinstance(dp, _DerivedTensor) and dp.scalar is None and len(dp.inputs) == 2
    ctx._remember(p, dp)
    b25 = 25.0 * t2
    d25 = ctx._derive(b25)
    assert d25 is not None and d25.scalar == 25.0
    ctx._remember(b25, d25)
    y = p * b25  # not saved itself: only a view of it is
    view = y.view(96)
    dv = ctx._derive(view)
    assert isinstance(dv, _DerivedTensor) and dv.shape == (96,)
    # replaying the recorded muls gives the same bits
    assert torch.equal((4.0 * t1.detach()).view(torch.int16), a4.detach().view(torch.int16))
    # rejected: an input never saved; a product of a tensor not saved through the context
    assert ctx._derive(torch.tanh(gate) * 3.0) is None
    u = torch.randn(6, 16, dtype=torch.bfloat16, requires_grad=True) * 1.0
    assert ctx._derive(t1 * u) is None
    # rejected: a constant tensor operand (saved through the hooks in a real context)
    c = torch.randn(6, 16, dtype=torch.bfloat16)
    assert ctx._derive(t1 * c) is None
    # rejected: broadcasting, a changed input, a written output, a partial view, non-mul ops
    assert ctx._derive(t1 * s[:1]) is None
    assert ctx._derive(t1 + s) is None
    w = 2.0 * t2
    with torch.no_grad():
        w.add_(1.0)
    assert ctx._derive(w) is None
    assert ctx._derive(y[:3]) is None
    with torch.no_grad():
        t2.mul_(1.0)  # t2 changed after its save: products of it are no longer recomputable
    assert ctx._derive(25.0 * t2) is None
    # a freed input (a temporary, as in the reference's activation) still counts: only a handle
    # of it is held
    import weakref

    t3 = torch.tanh(hidden)
    held(t3, 4)
    b3 = 3.0 * t3
    key = (t3.grad_fn, t3.output_nr)
    handle, _, version, meta = ctx._made[key]
    ctx._made[key] = (handle, weakref.ref(torch.zeros(1)), version, meta)  # the referent is gone
    assert ctx._made[key][1]() is None
    assert ctx._derive(b3) is not None


def test_equal_casts_are_aliased_only_after_the_bytes_compare_equal() -> None:
    """The rule of ``_ActivationOffload._alias``: a second cast of the same autograd output as
    an offloaded cast (RMSNorm's two ``tokens.float()``, training/model.py:171) is compared with
    it on the device; equal bytes restore from the first cast's entry, different bytes keep the
    save itself. The graph alone cannot tell: a write under ``no_grad`` between the casts
    leaves both casts' nodes pointing at the same output."""

    from moss_offload.activation_offload import _CheckedAlias, _OffloadedTensor, _cast_origin

    def offloaded(ctx, t, gid):
        h = _OffloadedTensor(None, gid, 0, t.device, t.dtype, tuple(t.shape), tuple(t.stride()), tuple(t.shape))
        ctx._casts[_cast_origin(t)] = (h, weakref.ref(t), t._version, 0)
        return h

    tokens = torch.randn(512, 1024, dtype=torch.bfloat16, requires_grad=True) * 1.0
    ctx = _derive_context()
    second = tokens.float()  # saved first (by square's node in RMSNorm)
    h = offloaded(ctx, second, 7)
    first = tokens.float()
    assert _cast_origin(first) == _cast_origin(second)
    alias = ctx._alias(first, _cast_origin(first), 0)
    assert isinstance(alias, _CheckedAlias) and alias.tensor is first and ctx._pending == [alias]
    assert alias.settle(False) and alias.tensor is None and alias.target.group == h.group
    # the alias hands its target's restore to autograd: a reader's reference
    assert ctx.engine.acquired[-1] == (7, 0, True) and alias.target.reader
    # a write between the casts that autograd does not see: the bytes differ, the save stays
    ctx = _derive_context()
    second = tokens.float()
    offloaded(ctx, second, 8)
    with torch.no_grad():
        tokens.add_(1.0)
    first = tokens.float()
    alias = ctx._alias(first, _cast_origin(first), 0)
    assert alias is not None and alias.settle(True) and alias.target is None and alias.tensor is first
    # rejected: the earlier cast freed or written, another stream, another shape, a small cast
    ctx = _derive_context()
    offloaded(ctx, tokens.float(), 9)  # freed at once
    assert ctx._alias(tokens.float(), _cast_origin(tokens.float()), 0) is None
    second = tokens.float()
    offloaded(ctx, second, 10)
    assert ctx._alias(tokens.float(), _cast_origin(second), 1) is None
    with torch.no_grad():
        second.mul_(1.0)
    assert ctx._alias(tokens.float(), _cast_origin(second), 0) is None
    part = tokens[:256].float()
    offloaded(ctx, tokens[:256].float(), 11)
    assert ctx._alias(tokens.float(), _cast_origin(part), 0) is None
    small = torch.randn(64, 64, dtype=torch.bfloat16, requires_grad=True) * 1.0
    kept = small.float()
    offloaded(ctx, kept, 12)
    assert ctx._alias(small.float(), _cast_origin(kept), 0) is None
    # an alias dropped before its result gives its ticket back
    ctx = _derive_context()
    second = tokens.float()
    offloaded(ctx, second, 13)
    alias = ctx._alias(tokens.float(), _cast_origin(second), 0)
    ctx._pending.clear()
    del alias
    assert ctx.engine.discarded == [1]


def test_each_reader_of_a_deduplicated_entry_gets_its_own_tensor() -> None:
    """``OffloadEngine._take_cached``: an entry restored once is handed out once per reference.
    An autograd consumer while another reader is still to take it gets a copy of its own (the
    reference's restore copies for every unpack, training/activation_offload.py:75-77); the last
    reader gets the restored tensor itself; a replay's read shares it; a take after an in-place
    write to the cached tensor finds it stale."""

    from moss_offload.engine import EngineConfig, OffloadEngine, _EntryState

    def engine(private):
        e = OffloadEngine.__new__(OffloadEngine)
        e.config, e.device = EngineConfig(private_restores=private), torch.device("cpu")
        return e

    padded = torch.arange(64, dtype=torch.float32).as_strided((3, 5), (8, 1))  # gaps between rows

    def entry(readers, internal):
        ent = _EntryState(torch.float32, (3, 5), (8, 1), 60)
        ent.readers, ent.refs = readers, readers + internal
        ent.restored = torch.empty_strided((3, 5), (8, 1))
        ent.restored.copy_(padded)
        ent.restored_version = ent.restored._version
        return ent

    e = engine(True)
    ent = entry(readers=2, internal=1)
    cached = ent.restored
    first = e._take_cached(ent, reader=True)  # another reader is still to come: a copy
    assert first is not cached and first.untyped_storage().data_ptr() != cached.untyped_storage().data_ptr()
    assert first.stride() == (8, 1) and torch.equal(first, padded)
    replay = e._take_cached(ent, reader=False)  # a replay's read shares the cached tensor
    assert replay is cached
    ent.readers, ent.refs = 1, 2  # the first reader's node ran and let go of its save
    last = e._take_cached(ent, reader=True)
    assert last is cached and ent.restored is cached  # still cached for the replay's reference
    ent.refs = 1
    assert e._take_cached(ent, reader=False) is cached and ent.restored is None
    # an in-place write to a cached tensor is seen at the next take: restore again
    ent = entry(readers=2, internal=0)
    with torch.no_grad():
        ent.restored.add_(1.0)
    assert e._take_cached(ent, reader=True) is None and ent.restored is None
    # private_restores=False: every reader shares the one restored tensor
    e = engine(False)
    ent = entry(readers=2, internal=0)
    assert e._take_cached(ent, reader=True) is ent.restored


def test_hook_features_probe_reports_each_graph_reading_feature() -> None:
    # On this torch every feature works; when a probe's private state is gone it reports it off
    # (and the hook then offloads those saves whole).
    from moss_offload import activation_offload as ao

    assert moss_offload.hook_features() == {
        "narrow_bf16_casts": True,
        "alias_equal_casts": True,
        "recompute_products": True,
    }
    original = ao._bf16_exact
    try:
        ao._bf16_exact = lambda tensor, source: False
        assert moss_offload.hook_features()["narrow_bf16_casts"] is False
    finally:
        ao._bf16_exact = original
    original = ao._cast_origin
    try:
        ao._cast_origin = lambda tensor: None
        assert moss_offload.hook_features()["alias_equal_casts"] is False
    finally:
        ao._cast_origin = original


def test_missing_feature_is_reported_once_as_a_warning(monkeypatch) -> None:
    import warnings

    from moss_offload import activation_offload as ao

    monkeypatch.setattr(ao, "_REPORTED", False)
    monkeypatch.setattr(ao, "hook_features", lambda: {"narrow_bf16_casts": False, "alias_equal_casts": True,
                                                      "recompute_products": True})
    config = engine.EngineConfig()
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        ao._report_features(config)
        ao._report_features(config)
    messages = [str(w.message) for w in caught]
    assert len(messages) == 1 and "narrow_bf16_casts" in messages[0]


@pytest.mark.parametrize(
    "kw, rings",
    [
        ({}, (4, 16, 8, 32, 24)),  # growth to 8 + 32 and 24 small slots by default
        ({"stage_slots_max": 0, "restore_slots_max": 0}, (4, 16, 4, 16, 24)),  # fixed rings
        ({"stage_slots": 3, "restore_slots": 2}, (3, 2, 8, 32, 24)),
        ({"restore_slots": 48}, (4, 48, 8, 48, 8)),  # a cap never below the ring
        ({"restore_slots": 60}, (4, 60, 4, 60, 0)),  # the caps give way within 64 slots
        ({"stage_slots": 12, "restore_slots": 52}, (12, 52, 12, 52, 0)),
        ({"stage_slots_max": 2}, (4, 16, 4, 32, 24)),
        ({"restore_small_slots": 0}, (4, 16, 8, 32, 0)),
        ({"restore_small_slots": 40}, (4, 16, 8, 32, 24)),  # small slots take what the caps leave
    ],
)
def test_engine_config_ring_caps(kw, rings) -> None:
    """The growth caps EngineConfig hands the library: at least the configured rings, at most
    64 slots in all with the small restore slots (the library rejects anything else), 0 for a
    fixed ring."""

    cfg = engine.EngineConfig(**kw).native()
    got = (cfg.stage_slots, cfg.restore_slots, cfg.stage_slots_max, cfg.restore_slots_max, cfg.restore_small_slots)
    assert got == rings
    assert cfg.stage_slots_max + cfg.restore_slots_max + cfg.restore_small_slots <= 64


@pytest.mark.parametrize("name", ["stage_slots_max", "restore_slots_max", "restore_small_slots"])
def test_engine_config_rejects_negative_ring_caps(name) -> None:
    with pytest.raises(ValueError, match=name):
        engine.EngineConfig(**{name: -1})
