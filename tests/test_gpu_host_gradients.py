"""Host fp32 gradient accumulation on the GPU (moss_offload.host_gradients, csrc/mo_gradacc.cpp).

Oracle: the reference's own stash (training/fused_adafactor.py:336-352): an fp32 host copy of
each gradient, then host fp32 ``add_`` in call order. torch's CPU fp32 adds are plain IEEE
single-precision adds, as are the native worker's, so the two are compared bit for bit,
including chunking over staging slots, every fp16 and bf16 bit pattern (NaN payloads, infinities,
subnormals), gradients freed immediately after the call, and backpressure when every slot is in
flight. At model level, host accumulation over two early micro-batches followed by the boundary
micro-batch equals plain device accumulation bit for bit for fp32 parameters, and the engine
stash equals the reference stash for bf16 parameters.
"""

from __future__ import annotations

import copy
import time

import pytest
import torch

from moss_offload.harness_optim import HostModeSGD
from moss_offload.host_gradients import HostGradientAccumulator

from gpu_util import requires_gpu

pytestmark = requires_gpu

DEV = torch.device("cuda", 0)


def _oracle(grads):
    acc = grads[0].detach().to("cpu", torch.float32).clone()
    for g in grads[1:]:
        acc.add_(g.detach().to("cpu", torch.float32))
    return acc


def _bits(t):
    return t.contiguous().view(torch.int32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("numel", [1, 4097, 3_000_001])
def test_accumulation_is_bitwise_the_reference(dtype, numel) -> None:
    g = torch.Generator(device=DEV).manual_seed(numel)
    grads = [torch.randn(numel, device=DEV, generator=g).mul_(10 ** k).to(dtype) for k in range(-1, 3)]
    acc = HostGradientAccumulator(DEV, slots=3, slot_bytes=1 << 20, host_threads=4)
    for x in grads:
        acc.accumulate("p", x)
    got = acc["p"]
    assert got.dtype == torch.float32 and got.device.type == "cpu" and got.shape == grads[0].shape
    assert torch.equal(_bits(got), _bits(_oracle(grads)))
    st = acc.stats()
    assert st["calls"] == 4 and st["elements"] == 4 * numel and st["pending_chunks"] == 0
    assert st["bytes"] == 4 * numel * grads[0].element_size()
    acc.close()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_every_bit_pattern_converts_exactly(dtype) -> None:
    patterns = torch.arange(-(1 << 15), 1 << 15, dtype=torch.int32).to(torch.int16).to(DEV).view(dtype)
    acc = HostGradientAccumulator(DEV, slot_bytes=1 << 16)
    acc.accumulate(0, patterns)
    assert torch.equal(_bits(acc[0]), _bits(patterns.float().cpu()))
    # and one add on top: inf + -inf = NaN, finite + inf = inf, as the reference's host add_
    finite = patterns.clone()
    finite[~torch.isfinite(finite.float())] = 0
    acc.accumulate(0, finite)
    oracle = _oracle([patterns, finite])
    got = acc[0]
    same_nan = torch.isnan(got) & torch.isnan(oracle)
    assert torch.equal(torch.isnan(got), torch.isnan(oracle))
    assert torch.equal(_bits(got)[~same_nan], _bits(oracle)[~same_nan])
    acc.close()


def test_gradient_may_be_freed_and_overwritten_right_after_the_call() -> None:
    acc = HostGradientAccumulator(DEV, slots=2, slot_bytes=1 << 20)
    expect = []
    for i in range(6):
        x = torch.randn(1 << 19, device=DEV).to(torch.bfloat16)
        expect.append(x.clone())
        acc.accumulate("p", x)
        del x
        # reuse the freed block at once on the same stream
        junk = [torch.full((1 << 19,), float(i), device=DEV, dtype=torch.bfloat16) for _ in range(4)]
        del junk
    assert torch.equal(_bits(acc["p"]), _bits(_oracle(expect)))
    acc.close()


def test_backpressure_blocks_the_host_and_stays_exact() -> None:
    acc = HostGradientAccumulator(DEV, slots=2, slot_bytes=1 << 20, host_threads=2)
    grads = [torch.randn(4 << 20, device=DEV) for _ in range(3)]  # 16 MiB each: 16 chunks, 2 slots
    for x in grads:
        acc.accumulate("p", x)
    assert torch.equal(_bits(acc["p"]), _bits(_oracle(grads)))
    st = acc.stats()
    assert st["host_blocks"] > 0 and st["chunks"] == 48 and st["copy_failures"] == 0
    acc.close()


def test_accumulate_returns_before_the_copy_finishes() -> None:
    acc = HostGradientAccumulator(DEV)  # 4 x 64 MiB slots
    x = torch.randn(96 << 20, device=DEV).to(torch.bfloat16)  # 192 MiB: 3 chunks, no blocking
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    acc.accumulate("p", x)
    call_s = time.perf_counter() - t0
    pending = acc.stats()["pending_chunks"]
    got = acc["p"]
    st = acc.stats()
    assert pending >= 1, "the call waited for its copies"
    assert st["host_blocks"] >= 1  # the read above had to wait
    assert st["d2h_ms"] > 0 and call_s * 1e3 < st["d2h_ms"] + st["accumulate_ms"]
    assert torch.equal(_bits(got), _bits(_oracle([x])))
    acc.close()


def _model(dtype):
    torch.manual_seed(7)
    return torch.nn.Sequential(torch.nn.Linear(96, 256), torch.nn.GELU(), torch.nn.Linear(256, 64)).to(DEV, dtype)


def _train(model, opt, batches):
    opt.set_step_enabled(False)
    for b in batches[:-1]:
        model(b).float().square().mean().backward()
    assert all(p.grad is None for p in model.parameters())
    opt.set_step_enabled(True)
    model(batches[-1]).float().square().mean().backward()
    opt.finish_backward()


def test_fp32_training_matches_device_accumulation_bitwise() -> None:
    batches = [torch.randn(n, 96, device=DEV) for n in (16, 8, 24)]
    host_model = _model(torch.float32)
    device_model = copy.deepcopy(host_model)
    opt = HostModeSGD(host_model.parameters(), lr=0.05, stash="engine")
    _train(host_model, opt, batches)
    for b in batches:
        device_model(b).float().square().mean().backward()
    with torch.no_grad():
        for p in device_model.parameters():
            p.add_(p.grad, alpha=-0.05)
    for a, b in zip(host_model.parameters(), device_model.parameters()):
        assert torch.equal(a, b)
    assert opt.host_gradients == {}
    opt.close()


def test_bf16_training_engine_stash_equals_reference_stash() -> None:
    batches = [torch.randn(n, 96, device=DEV).to(torch.bfloat16) for n in (16, 8, 24)]
    engine_model = _model(torch.bfloat16)
    ref_model = copy.deepcopy(engine_model)
    engine = HostModeSGD(engine_model.parameters(), lr=0.05, stash="engine")
    reference = HostModeSGD(ref_model.parameters(), lr=0.05, stash="reference")
    _train(engine_model, engine, batches)
    _train(ref_model, reference, batches)
    for a, b in zip(engine_model.parameters(), ref_model.parameters()):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    engine.close()
    reference.close()


def test_host_entry_continued_by_a_device_gradient_and_dtype_errors() -> None:
    acc = HostGradientAccumulator(DEV)
    a = torch.randn(1000)
    b = torch.randn(1000, device=DEV)
    acc.accumulate("p", a)  # the CPU path
    acc.accumulate("p", b)  # continued in the native buffer
    assert torch.equal(_bits(acc["p"]), _bits(_oracle([a, b])))
    with pytest.raises(TypeError, match="fp16, bf16 or fp32"):
        acc.accumulate("q", torch.zeros(4, device=DEV, dtype=torch.float64))
    with pytest.raises(ValueError, match="changed size"):
        acc.accumulate("p", torch.zeros(5, device=DEV))
    acc.close()


def test_pop_to_device_prefetches_in_first_contribution_order_and_is_exact() -> None:
    acc = HostGradientAccumulator(DEV, slots=4, slot_bytes=1 << 20, prefetch=3)
    shapes = [(17,), (300, 7), (1 << 18,), (64, 64), (5,), (2048, 33), (3,)]
    for step in range(2):
        grads = {k: [torch.randn(sh, device=DEV).to(torch.bfloat16) for _ in range(2)] for k, sh in enumerate(shapes)}
        for rnd in range(2):
            for k in grads:
                acc.accumulate(k, grads[k][rnd])
        order = list(grads) if step == 0 else [3, 0, 6, 1, 5, 2, 4]  # in order, then out of order
        for i, k in enumerate(order):
            got = acc.pop_to_device(k, DEV)
            assert got.device == DEV and got.dtype == torch.float32 and got.shape == shapes[k]
            assert torch.equal(_bits(got.cpu()), _bits(_oracle(grads[k])))
            if step == 0 and i == 0:
                assert len(acc._prefetched) == 3  # the next three entries are on their way
        assert acc == {} and acc.pop_to_device(0) is None
    # a prefetched entry that gets another contribution is re-read, not stale
    a, b = torch.randn(1000, device=DEV), torch.randn(1000, device=DEV)
    acc.accumulate("x", a)
    acc.accumulate("y", a)
    acc.pop_to_device("x")  # prefetches "y"
    acc.accumulate("y", b)
    assert torch.equal(_bits(acc.pop_to_device("y").cpu()), _bits(_oracle([a, b])))
    acc.close()

