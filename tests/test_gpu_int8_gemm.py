"""Weight-only int8 GEMMs on MFMA (mo_int8_linear_forward / backward) on the GPU.

- Decode parity: with one-hot inputs each output element is a single product, so the kernels
  must reproduce the decoded weight bit for bit: bf16(q * bf16(scale)), the decode of the
  reference's Triton kernels (training/quant_kernels.py:126-131) and of its eager path
  (quantization.py:23-24).
- Products: random shapes including ragged rows, columns and reduction lengths (partial
  tiles and reduction steps), against an fp64 reference of the same decoded weight, within
  the bound of fp32 accumulation plus the final bf16 rounding.
- Module level: the harness's int8 LoRA model trains the same with the HIP backend and with
  the eager backend (the reference's own parity criterion between its backends).
"""

from __future__ import annotations

import copy

import pytest
import torch
import torch.nn.functional as F

from moss_offload import dit, quant_kernels

from gpu_util import requires_gpu

pytestmark = requires_gpu

DEV = torch.device("cuda", 0)


def _operands(rows, in_f, out_f, seed, bias=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, in_f, generator=g).to(torch.bfloat16).to(DEV)
    w = torch.randint(-127, 128, (out_f, in_f), dtype=torch.int8, generator=g).to(DEV)
    scale = torch.empty(out_f).uniform_(0.001, 0.02, generator=g).to(DEV)
    b = torch.randn(out_f, generator=g).to(torch.bfloat16).to(DEV) if bias else None
    return x, w, scale, b


def _within_accumulation_bound(actual, exact, magnitude, terms):
    err = (actual.double() - exact).abs()
    bound = 2.0**-8 * exact.abs() + terms * 2.0**-23 * magnitude + 1e-30
    bad = err > bound
    assert not bad.any(), f"{int(bad.sum())} elements outside the bound; worst excess {(err - bound).max().item()}"


@pytest.mark.parametrize("in_f,out_f", [(16, 16), (64, 128), (80, 48), (256, 384)])
def test_forward_reproduces_the_decoded_weight_bitwise(in_f, out_f) -> None:
    _, w, scale, _ = _operands(1, in_f, out_f, seed=in_f + out_f)
    eye = torch.eye(in_f, dtype=torch.bfloat16, device=DEV)
    y = quant_kernels.int8_linear_forward(eye, w, scale)
    decoded = quant_kernels.decode(w, scale, torch.bfloat16)
    assert torch.equal(y.view(torch.int16), decoded.t().contiguous().view(torch.int16))


@pytest.mark.parametrize("in_f,out_f", [(16, 16), (64, 128), (80, 48), (256, 384)])
def test_backward_reproduces_the_decoded_weight_bitwise(in_f, out_f) -> None:
    _, w, scale, _ = _operands(1, in_f, out_f, seed=in_f * 3 + out_f)
    eye = torch.eye(out_f, dtype=torch.bfloat16, device=DEV)
    dx = quant_kernels.int8_linear_backward(eye, w, scale, torch.Size((out_f, in_f)))
    decoded = quant_kernels.decode(w, scale, torch.bfloat16)
    assert torch.equal(dx.view(torch.int16), decoded.view(torch.int16))


SHAPES = [(1, 16, 16), (100, 80, 48), (128, 64, 128), (257, 256, 384), (300, 1040, 208), (1024, 3072, 3072)]


@pytest.mark.parametrize("rows,in_f,out_f", SHAPES)
@pytest.mark.parametrize("bias", [False, True])
def test_forward_matches_fp64_reference(rows, in_f, out_f, bias) -> None:
    x, w, scale, b = _operands(rows, in_f, out_f, seed=rows + 7 * in_f + out_f, bias=bias)
    y = quant_kernels.int8_linear_forward(x, w, scale, b)
    assert y.shape == (rows, out_f) and y.dtype == torch.bfloat16
    decoded = quant_kernels.decode(w, scale, torch.bfloat16).double()
    exact = x.double() @ decoded.t()
    if b is not None:
        exact = exact + b.double()
    magnitude = x.double().abs() @ decoded.abs().t()
    _within_accumulation_bound(y, exact, magnitude, in_f)


@pytest.mark.parametrize("rows,in_f,out_f", SHAPES)
def test_backward_matches_fp64_reference(rows, in_f, out_f) -> None:
    _, w, scale, _ = _operands(rows, in_f, out_f, seed=rows + 11 * in_f + out_f)
    g = torch.Generator().manual_seed(rows)
    dy = torch.randn(rows, out_f, generator=g).to(torch.bfloat16).to(DEV)
    dx = quant_kernels.int8_linear_backward(dy, w, scale, torch.Size((rows, in_f)))
    decoded = quant_kernels.decode(w, scale, torch.bfloat16).double()
    exact = dy.double() @ decoded
    magnitude = dy.double().abs() @ decoded.abs()
    _within_accumulation_bound(dx, exact, magnitude, out_f)


# Launch plans on a 256-CU MI355X (csrc/mo_gemm.cpp): the large tile alone (a grid of exactly
# 256 large tiles), the large tile plus a small-tile launch for the rows of a partial last round
# (17792 x 3072: 840 tiles), the small tile alone (small shapes above); each with a reduction
# length that is and is not a multiple of 64.
PLAN_SHAPES = [(4096, 4096, 4096), (4096, 1040, 4096), (17792, 3072, 3072), (17792, 1040, 3072),
               (4000, 4096, 4000)]  # the last: large tiles only, with ragged rows and columns


@pytest.mark.parametrize("rows,in_f,out_f", PLAN_SHAPES)
def test_forward_launch_plans_match_fp64_reference(rows, in_f, out_f) -> None:
    x, w, scale, b = _operands(rows, in_f, out_f, seed=rows + in_f + 3 * out_f, bias=True)
    y = quant_kernels.int8_linear_forward(x, w, scale, b, path="fused")
    decoded = quant_kernels.decode(w, scale, torch.bfloat16).double()
    exact = x.double() @ decoded.t() + b.double()
    magnitude = x.double().abs() @ decoded.abs().t()
    _within_accumulation_bound(y, exact, magnitude, in_f)


@pytest.mark.parametrize("rows,in_f,out_f", [(4096, 4096, 4096), (4096, 4096, 1040), (17792, 3072, 3072),
                                             (17792, 3072, 1040), (4000, 4000, 4096)])
def test_backward_launch_plans_match_fp64_reference(rows, in_f, out_f) -> None:
    _, w, scale, _ = _operands(1, in_f, out_f, seed=rows + 5 * in_f + out_f)
    g = torch.Generator().manual_seed(rows + 1)
    dy = torch.randn(rows, out_f, generator=g).to(torch.bfloat16).to(DEV)
    dx = quant_kernels.int8_linear_backward(dy, w, scale, torch.Size((rows, in_f)), path="fused")
    decoded = quant_kernels.decode(w, scale, torch.bfloat16).double()
    exact = dy.double() @ decoded
    magnitude = dy.double().abs() @ decoded.abs()
    _within_accumulation_bound(dx, exact, magnitude, out_f)


def test_tile_choice_does_not_change_results() -> None:
    # 17792 rows: large tiles for rows < 16384, then one launch with the reduction split three
    # ways for the last 1408; 4096 rows alone run on small tiles, which add the large tile's
    # products in its order, and 1408 rows alone run the same split launch as that tail.
    rows, in_f, out_f = 17792, 3072, 3072
    x, w, scale, b = _operands(rows, in_f, out_f, seed=77, bias=True)
    fused = {"path": "fused"}
    full = quant_kernels.int8_linear_forward(x, w, scale, b, **fused)
    assert torch.equal(quant_kernels.int8_linear_forward(x[:4096], w, scale, b, **fused).view(torch.int16),
                       full[:4096].view(torch.int16))
    assert torch.equal(quant_kernels.int8_linear_forward(x[16384:], w, scale, b, **fused).view(torch.int16),
                       full[16384:].view(torch.int16))
    dy = x[:, :out_f].contiguous()
    dfull = quant_kernels.int8_linear_backward(dy, w, scale, torch.Size((rows, in_f)), **fused)
    part = quant_kernels.int8_linear_backward(dy[:4096], w, scale, torch.Size((4096, in_f)), **fused)
    assert torch.equal(part.view(torch.int16), dfull[:4096].view(torch.int16))


def test_unsupported_calls_are_reported_and_auto_falls_back_to_eager() -> None:
    x, w, scale, _ = _operands(4, 24, 16, seed=5)  # in_features not a multiple of 16
    assert quant_kernels.unsupported_reason(x, w, scale, torch.bfloat16) is not None
    assert quant_kernels.resolve_backend("auto", x, w, scale, torch.bfloat16) == "eager"
    with pytest.raises(RuntimeError, match="HIP int8 backend is unavailable"):
        quant_kernels.resolve_backend("hip", x, w, scale, torch.bfloat16)
    x, w, scale, _ = _operands(4, 32, 16, seed=6)
    assert quant_kernels.resolve_backend("auto", x, w, scale, torch.bfloat16) == "hip"
    assert quant_kernels.resolve_backend("auto", x.float(), w, scale, torch.float32) == "eager"


@pytest.mark.parametrize("case,reason", [
    ("dtype", "only bf16"), ("wdtype", "int8 and scales float32"), ("shape", "dimensions do not match"),
    ("ragged", "multiples of 16"), ("strided", "contiguous"), ("empty", "empty input"),
])
def test_unsupported_reasons_name_the_cause(case, reason) -> None:
    x, w, scale, _ = _operands(4, 32, 16, seed=9)
    dtype = torch.bfloat16
    if case == "dtype":
        x, dtype = x.float(), torch.float32
    elif case == "wdtype":
        scale = scale.double()
    elif case == "shape":
        w = torch.zeros(16, 48, dtype=torch.int8, device=DEV)
    elif case == "ragged":
        x, w, scale, _ = _operands(4, 24, 16, seed=9)
    elif case == "strided":
        w = torch.zeros(32, 16, dtype=torch.int8, device=DEV).t()
    elif case == "empty":
        x = x[:0]
    got = quant_kernels.unsupported_reason(x, w, scale, dtype)
    assert got is not None and reason in got
    assert quant_kernels.resolve_quantized_backend("auto", x, w, scale) == "eager"


def test_reference_interface_runs_the_hip_kernels() -> None:
    # the sequence of the reference's _FrozenInt8Linear (quantization.py:28-61) on this module
    x, w, scale, b = _operands(300, 1040, 208, seed=31, bias=True)
    assert quant_kernels.triton_is_available()
    assert quant_kernels.resolve_quantized_backend("auto", x, w, scale) == "triton"
    assert quant_kernels.resolve_quantized_backend("triton", x, w, scale) == "triton"
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out_dtype = quant_kernels.autocast_compute_dtype(x, torch.bfloat16)
    assert out_dtype == torch.bfloat16
    y = quant_kernels.triton_int8_linear_forward(x, w, scale, b, out_dtype, torch.bfloat16)
    assert torch.equal(y.view(torch.int16), quant_kernels.int8_linear_forward(x, w, scale, b).view(torch.int16))
    buf = torch.empty(300 * 208, dtype=torch.bfloat16, device=DEV)
    y2 = quant_kernels.triton_int8_linear_forward(x, w, scale, b, out_dtype, torch.bfloat16, out=buf)
    assert y2.data_ptr() == buf.data_ptr() and torch.equal(y2.view(torch.int16), y.view(torch.int16))
    g = torch.randn(300, 208, device=DEV).to(torch.bfloat16)
    dx = quant_kernels.triton_int8_linear_backward(g, w, scale, x.shape, torch.bfloat16, torch.bfloat16)
    assert dx.shape == x.shape
    assert torch.equal(dx.view(torch.int16),
                       quant_kernels.int8_linear_backward(g, w, scale, x.shape).view(torch.int16))
    with pytest.raises(TypeError, match="bf16"):
        quant_kernels.triton_int8_linear_forward(x.float(), w, scale, None, torch.float32, torch.float32)
    with pytest.raises(ValueError, match="buffer"):
        quant_kernels.triton_int8_linear_forward(x, w, scale, None, out_dtype, torch.bfloat16,
                                                 out=torch.empty(5, dtype=torch.bfloat16, device=DEV))


def test_int8_lora_model_hip_backend_matches_eager() -> None:
    torch.manual_seed(121)
    model = dit.MOSSImageTransformer(dim=64, ffn_dim=128, num_heads=4, num_layers=2, text_dim=16, freq_dim=8,
                                     latent_channels=4, gradient_checkpointing=True)
    model = model.to(DEV).to(torch.bfloat16)
    dit.init_weights(model)
    dit.quantize_joint_linears(model, torch.Generator(device=DEV).manual_seed(5))
    dit.inject_lora(model, rank=4, alpha=4.0)
    results = {}
    g = torch.Generator().manual_seed(3)
    latent = torch.randn(1, 4, 6, 8, generator=g).to(DEV)
    context = torch.randn(1, 5, 16, generator=g).to(DEV)
    for backend in ("eager", "hip"):
        m = copy.deepcopy(model).train()
        assert dit.configure_quantized_backend(m, backend)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out = m(latent, torch.tensor([400.0], device=DEV), context)
            loss = out.float().square().mean()
        loss.backward()
        results[backend] = (out.detach().float(), {n: p.grad.float() for n, p in m.named_parameters() if p.grad is not None})
    (eo, eg), (ho, hg) = results["eager"], results["hip"]
    torch.testing.assert_close(ho, eo, rtol=2e-2, atol=2e-2)
    assert eg.keys() == hg.keys() and eg
    for name in eg:
        torch.testing.assert_close(hg[name], eg[name], rtol=5e-2, atol=1e-3, msg=name)


@pytest.mark.parametrize("out_f,in_f", [(16, 16), (48, 80), (3072, 1040), (4097, 16), (24576, 3072)])
def test_decode_kernel_matches_the_reference_decode_bitwise(out_f, in_f) -> None:
    """mo_int8_decode writes bf16(q * bf16(scale)) exactly as the reference's eager decode
    (quant_kernels.py:126-131); scales span normal fp32 magnitudes and bf16 rounding ties."""

    g = torch.Generator().manual_seed(out_f + in_f)
    w = torch.randint(-128, 128, (out_f, in_f), dtype=torch.int8, generator=g).to(DEV)
    scale = torch.empty(out_f).uniform_(1e-3, 2e-2, generator=g)
    scale[::7] = torch.empty(scale[::7].shape).uniform_(-3.0, 3.0, generator=g)
    scale[::11] = 1.0 + 2.0**-8  # halfway between two bf16 values
    scale = scale.to(DEV)
    got = quant_kernels.decode_hip(w, scale)
    want = quant_kernels.decode(w, scale, torch.bfloat16)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("rows,in_f,out_f", [(4096, 1040, 3072), (4100, 3072, 1040)])
def test_library_path_is_the_eager_path_bit_for_bit(rows, in_f, out_f) -> None:
    """From LIBRARY_ROWS rows up, ``auto`` decodes once and runs the library GEMM: the result is the
    reference eager path's (decode, then F.linear / matmul) bit for bit, with and without bias,
    and within the fp64 accumulation bound like the fused kernels."""

    assert rows >= quant_kernels.LIBRARY_ROWS
    x, w, scale, b = _operands(rows, in_f, out_f, seed=rows + in_f, bias=True)
    decoded = quant_kernels.decode(w, scale, torch.bfloat16)
    for bias in (None, b):
        y = quant_kernels.int8_linear_forward(x, w, scale, bias)
        assert torch.equal(y.view(torch.int16), F.linear(x, decoded, bias).view(torch.int16))
    g = torch.Generator().manual_seed(rows)
    dy = torch.randn(rows, out_f, generator=g).to(torch.bfloat16).to(DEV)
    dx = quant_kernels.int8_linear_backward(dy, w, scale, torch.Size((rows, in_f)))
    assert torch.equal(dx.view(torch.int16), dy.matmul(decoded).view(torch.int16))
    exact = x.double() @ decoded.double().t() + b.double()
    _within_accumulation_bound(y, exact, x.double().abs() @ decoded.double().abs().t(), in_f)
    # below the threshold auto is the fused kernel
    small = x[: quant_kernels.LIBRARY_ROWS - 1]
    assert torch.equal(quant_kernels.int8_linear_forward(small, w, scale, b).view(torch.int16),
                       quant_kernels.int8_linear_forward(small, w, scale, b, path="fused").view(torch.int16))
    with pytest.raises(ValueError):
        quant_kernels.int8_linear_forward(x, w, scale, b, path="triton")


def _large_tile_rows(rows: int, cols: int, reduction: int) -> int:
    """Rows the register kernel's launch plan gives the large tile on this device."""

    cus = torch.cuda.get_device_properties(DEV).multi_processor_count
    parts = quant_kernels.launch_plan(rows, cols, reduction, cus)
    return parts[0]["rows"] if parts[0]["tile"] == "large" else 0


# Besides the config-5 shapes: 8000 x 1024 x 5008 (forward) and 8000 x 5008 x 1024 (input
# gradient) run the register kernel alone on 640 large tiles with ragged rows and columns, over
# a reduction of 16 steps that its six-step loop pads to 18.
@pytest.mark.parametrize("rows,in_f,out_f", [(17792, 3072, 3072), (17792, 3072, 24576), (17792, 12288, 3072),
                                             (4000, 4096, 4000), (8000, 1024, 5008), (8000, 5008, 1024)])
def test_register_and_lds_kernels_agree_bitwise(rows, in_f, out_f) -> None:
    """The large tile's two kernels (weights decoded in registers, or into LDS) add the same
    products in the same order: forward and input gradient are equal bit for bit on the rows the
    large tile computes. The rest (a split reduction with the register kernel, the small tile
    with the LDS kernel) round differently and are held to the fp64 bound."""

    x, w, scale, b = _operands(rows, in_f, out_f, seed=rows + in_f + out_f, bias=True)
    g = torch.Generator().manual_seed(5)
    dy = torch.randn(rows, out_f, generator=g).to(torch.bfloat16).to(DEV)
    results = {}
    try:
        for kernel in ("lds", "registers"):
            quant_kernels.set_kernel(kernel)
            y = quant_kernels.int8_linear_forward(x, w, scale, b, path="fused")
            dx = quant_kernels.int8_linear_backward(dy, w, scale, torch.Size((rows, in_f)), path="fused")
            results[kernel] = (y, dx)
    finally:
        quant_kernels.set_kernel("registers")
    decoded = quant_kernels.decode(w, scale, torch.bfloat16).double()
    for k, (a, e) in enumerate(zip(results["registers"], results["lds"])):
        main = _large_tile_rows(rows, *((out_f, in_f) if k == 0 else (in_f, out_f)))
        assert torch.equal(a[:main].view(torch.int16), e[:main].view(torch.int16))
        if main == rows:
            continue
        if k == 0:
            xs = x[main:].double()
            exact, magnitude, terms = xs @ decoded.t() + b.double(), xs.abs() @ decoded.abs().t(), in_f
        else:
            ds = dy[main:].double()
            exact, magnitude, terms = ds @ decoded, ds.abs() @ decoded.abs(), out_f
        _within_accumulation_bound(a[main:], exact, magnitude, terms)
        _within_accumulation_bound(e[main:], exact, magnitude, terms)


# One-hot operands through split reductions: 3136 x 1040 outputs from a 3136-long reduction
# (49 steps of 64, split 18 + 18 + 13 over 65 large tiles; the transposed weight's last row and
# column tiles are partial). Each output element is one product plus zeros, so every split plan
# must reproduce the decoded weight bit for bit.
def test_split_reductions_reproduce_the_decoded_weight_bitwise() -> None:
    _, w, scale, _ = _operands(1, 3136, 1040, seed=31)  # forward: in 3136, out 1040
    eye = torch.eye(3136, dtype=torch.bfloat16, device=DEV)
    decoded = quant_kernels.decode(w, scale, torch.bfloat16)
    y = quant_kernels.int8_linear_forward(eye, w, scale, path="fused")
    assert torch.equal(y.view(torch.int16), decoded.t().contiguous().view(torch.int16))
    _, w, scale, _ = _operands(1, 1040, 3136, seed=32)  # input gradient: reduction over out 3136
    decoded = quant_kernels.decode(w, scale, torch.bfloat16)
    dx = quant_kernels.int8_linear_backward(eye, w, scale, torch.Size((3136, 1040)), path="fused")
    assert torch.equal(dx.view(torch.int16), decoded.view(torch.int16))


@pytest.mark.parametrize("direction", ["forward", "backward"])
def test_split_reductions_are_deterministic_and_within_bound(direction) -> None:
    # config 5's down_proj forward (12288-long reduction) and up_gate input gradient (24576):
    # the last 1408 rows run split three ways
    rows = 17792
    in_f, out_f = (12288, 3072) if direction == "forward" else (3072, 24576)
    x, w, scale, b = _operands(rows, in_f, out_f, seed=41, bias=direction == "forward")
    decoded = quant_kernels.decode(w, scale, torch.bfloat16).double()
    if direction == "forward":
        first = quant_kernels.int8_linear_forward(x, w, scale, b, path="fused")
        again = quant_kernels.int8_linear_forward(x, w, scale, b, path="fused")
        tail = x[16384:].double()
        exact, magnitude, terms = tail @ decoded.t() + b.double(), tail.abs() @ decoded.abs().t(), in_f
    else:
        g = torch.Generator().manual_seed(42)
        dy = torch.randn(rows, out_f, generator=g).to(torch.bfloat16).to(DEV)
        first = quant_kernels.int8_linear_backward(dy, w, scale, torch.Size((rows, in_f)), path="fused")
        again = quant_kernels.int8_linear_backward(dy, w, scale, torch.Size((rows, in_f)), path="fused")
        tail = dy[16384:].double()
        exact, magnitude, terms = tail @ decoded, tail.abs() @ decoded.abs(), out_f
    assert torch.equal(first.view(torch.int16), again.view(torch.int16))
    _within_accumulation_bound(first[16384:], exact, magnitude, terms)
    # a reduction at least four times the output width with a split launch: auto takes the
    # fused kernels
    if direction == "forward":
        auto = quant_kernels.int8_linear_forward(x, w, scale, b)
    else:
        auto = quant_kernels.int8_linear_backward(dy, w, scale, torch.Size((rows, in_f)))
    assert torch.equal(auto.view(torch.int16), first.view(torch.int16))


def test_long_reduction_without_a_split_takes_the_library() -> None:
    # 8192 rows of down_proj's forward fill one and a half rounds of large tiles: no split
    # launch, so auto runs the library GEMM (the eager path's result bit for bit)
    x, w, scale, _ = _operands(8192, 12288, 3072, seed=43)
    decoded = quant_kernels.decode(w, scale, torch.bfloat16)
    assert torch.equal(quant_kernels.int8_linear_forward(x, w, scale).view(torch.int16),
                       F.linear(x, decoded).view(torch.int16))


def test_workspace_smaller_than_the_plan_needs_is_rejected() -> None:
    from moss_offload import _native

    lib = _native.load()
    rows, in_f, out_f = 1408, 3072, 3072  # a split launch alone
    x, w, scale, _ = _operands(rows, in_f, out_f, seed=9)
    y = torch.empty(rows, out_f, dtype=torch.bfloat16, device=DEV)
    need = lib.mo_int8_forward_workspace_bytes(rows, in_f, out_f)
    assert need >= 3 * rows * out_f * 4
    small = torch.empty(need - 256, dtype=torch.uint8, device=DEV)
    stream = torch.cuda.current_stream(DEV).cuda_stream
    rc = lib.mo_int8_linear_forward(x.data_ptr(), w.data_ptr(), scale.data_ptr(), 0, y.data_ptr(), rows, in_f,
                                    out_f, small.data_ptr(), need - 256, stream)
    assert rc == _native.MO_E_INVALID and b"workspace" in lib.mo_last_error()
    dneed = lib.mo_int8_backward_workspace_bytes(rows, in_f, out_f)
    assert dneed >= in_f * out_f + 3 * rows * in_f * 4
    rc = lib.mo_int8_linear_backward(x.data_ptr(), w.data_ptr(), scale.data_ptr(), y.data_ptr(), rows, in_f,
                                     out_f, small.data_ptr(), in_f * out_f, stream)
    assert rc == _native.MO_E_INVALID and b"workspace" in lib.mo_last_error()
