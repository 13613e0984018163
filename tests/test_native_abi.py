"""The C-ABI library on the CPU: it loads, exports every declared symbol, and its structs,
host-side layout logic and fast division agree with independent computations. No GPU calls.
"""

from __future__ import annotations

import ctypes
import random
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from moss_offload import _native
from oracle import layout

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "moss_offload.h"
CSRC = ROOT / "moss-image_amd" / "csrc"


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"^(?:int|uint64_t|const char\*)\s+(mo_\w+)\(", text, flags=re.M)


def test_library_exports_every_declared_symbol() -> None:
    lib = _native.load()
    names = _declared_functions()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name
        assert name in _native.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_native.SIGNATURES) == set(names)
    assert lib.mo_abi_version() == _native.MO_ABI_VERSION


def _c_layouts(tmp_path: Path) -> dict[str, int]:
    """sizeof / offsetof of the ABI structs as the C compiler sees them."""

    fields = {
        "mo_tensor": ["ptr", "elem_bytes", "ndim", "size", "stride", "flags", "reserved"],
        "mo_config": [f for f, _ in _native.MoConfig._fields_],
        "mo_ref": [f for f, _ in _native.MoRef._fields_],
        "mo_stats": [f for f, _ in _native.MoStats._fields_],
        "mo_streamer_stats": [f for f, _ in _native.MoStreamerStats._fields_],
        "mo_gradacc_stats": [f for f, _ in _native.MoGradaccStats._fields_],
    }
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void) {"]
    for struct, names in fields.items():
        lines.append(f'printf("{struct} %zu\\n", sizeof({struct}));')
        for name in names:
            lines.append(f'printf("{struct}.{name} %zu\\n", offsetof({struct}, {name}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "abi.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "abi"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    return {k: int(v) for k, v in (line.split() for line in out.splitlines())}


def test_struct_layouts_match_ctypes(tmp_path) -> None:
    c = _c_layouts(tmp_path)
    for struct, cls in (("mo_tensor", _native.MoTensor), ("mo_config", _native.MoConfig), ("mo_ref", _native.MoRef),
                        ("mo_stats", _native.MoStats), ("mo_streamer_stats", _native.MoStreamerStats),
                        ("mo_gradacc_stats", _native.MoGradaccStats)):
        assert c[struct] == ctypes.sizeof(cls), struct
        for name, _ in cls._fields_:
            assert c[f"{struct}.{name}"] == getattr(cls, name).offset, f"{struct}.{name}"


def _descs(views):
    arr = (_native.MoTensor * max(len(views), 1))()
    for i, v in enumerate(views):
        _native.describe(v, arr[i])
    return arr


def test_payload_layout_offsets_and_errors() -> None:
    lib = _native.load()
    views = [torch.zeros(3, 5), torch.zeros(7, dtype=torch.bfloat16), torch.zeros(0), torch.zeros(4, 4).t()]
    arr = _descs(views)
    offsets = (ctypes.c_uint64 * 4)()
    total = ctypes.c_uint64()
    _native.check("mo_payload_layout", lib.mo_payload_layout(arr, 4, offsets, ctypes.byref(total)))
    pos, expected = 0, []
    for v in views:
        pos = (pos + 255) // 256 * 256
        expected.append(pos)
        pos += v.numel() * v.element_size()
    assert list(offsets) == expected and total.value == pos
    base = torch.zeros(64)
    bad = _descs([base.as_strided((3, 3), (1, 1))])
    assert lib.mo_payload_layout(bad, 1, offsets, ctypes.byref(total)) == _native.MO_E_LAYOUT
    assert b"overlapping" in lib.mo_last_error()
    interleaved = _descs([base.as_strided((3, 3), (12, 16))])  # overlap-free but not nested
    assert layout.interleaved_overlap_free((3, 3), (12, 16))
    assert lib.mo_payload_layout(interleaved, 1, offsets, ctypes.byref(total)) == _native.MO_E_LAYOUT
    odd = _descs([base])
    odd[0].elem_bytes = 3
    assert lib.mo_payload_layout(odd, 1, offsets, ctypes.byref(total)) == _native.MO_E_INVALID
    expanded = _descs([torch.zeros(5).expand(3, 5)])
    assert lib.mo_payload_layout(expanded, 1, offsets, ctypes.byref(total)) == _native.MO_E_LAYOUT


def test_bf16_high_payload_is_half_size_and_only_for_contiguous_float32() -> None:
    """MO_TENSOR_BF16_HIGH: the payload of a contiguous float32 tensor whose values are exact
    bfloat16 keeps the high half of each element, numel x 2 bytes."""

    lib = _native.load()
    views = [torch.zeros(3, 5), torch.zeros(1000), torch.zeros(2, 8, 4)]
    arr = _descs(views)
    arr[1].flags = _native.MO_TENSOR_BF16_HIGH
    arr[2].flags = _native.MO_TENSOR_BF16_HIGH
    offsets = (ctypes.c_uint64 * 3)()
    total = ctypes.c_uint64()
    _native.check("mo_payload_layout", lib.mo_payload_layout(arr, 3, offsets, ctypes.byref(total)))
    assert list(offsets) == [0, 256, 256 + 2048] and total.value == 256 + 2048 + 2 * 64
    rejected = [
        (torch.zeros(8, dtype=torch.bfloat16), _native.MO_E_INVALID),  # not float32
        (torch.zeros(4, 8)[:, :6], _native.MO_E_LAYOUT),  # gaps between rows
        (torch.zeros(16)[::2], _native.MO_E_LAYOUT),
    ]
    # a transposed view of a dense tensor is dense in storage order: accepted
    dense_t = _descs([torch.zeros(4, 6).t()])
    dense_t[0].flags = _native.MO_TENSOR_BF16_HIGH
    _native.check("mo_payload_layout", lib.mo_payload_layout(dense_t, 1, offsets, ctypes.byref(total)))
    assert total.value == 48
    for view, code in rejected:
        bad = _descs([view])
        bad[0].flags = _native.MO_TENSOR_BF16_HIGH
        assert lib.mo_payload_layout(bad, 1, offsets, ctypes.byref(total)) == code
    unknown = _descs([torch.zeros(4)])
    unknown[0].flags = 0x80
    assert lib.mo_payload_layout(unknown, 1, offsets, ctypes.byref(total)) == _native.MO_E_INVALID
    assert b"unknown tensor flags" in lib.mo_last_error()


DRIVER = r"""
#include <stdio.h>
#include <stdlib.h>
#include "mo_layout.h"
// stdin: lines "ndim s0..sN t0..tN" -> stdout: "rc nd size.. stride.." canonical form
// argv[1] == "div": check fast division on random and edge operands, print failures
int main(int argc, char** argv) {
  if (argc > 1) {
    unsigned long long seed = 88172645463325252ull; long bad = 0;
    const uint32_t edges[] = {1u, 2u, 3u, 5u, 7u, 0x7fffffffu, 0x80000000u, 0x80000001u, 0xfffffffeu, 0xffffffffu};
    for (int i = 0; i < 2000000; ++i) {
      seed ^= seed << 13; seed ^= seed >> 7; seed ^= seed << 17;
      uint32_t d = (uint32_t)(seed >> 32); if (i % 3 == 0) d >>= (seed & 31); if (!d) d = 1;
      if (i < 100) d = edges[i % 10];
      uint32_t n = (uint32_t)seed; if (i % 5 == 0) n = 0xffffffffu - (uint32_t)(i % 7);
      mo::FastDiv f = mo::make_fastdiv(d);
      if (mo::fastdiv_host(n, f) != n / d) { if (bad < 5) printf("%u/%u\n", n, d); ++bad; }
    }
    printf("bad %ld\n", bad); return 0;
  }
  int nd;
  while (scanf("%d", &nd) == 1) {
    mo_tensor t = {}; t.ptr = 4096; t.elem_bytes = 4; t.ndim = nd;
    for (int i = 0; i < nd; ++i) scanf("%lld", (long long*)&t.size[i]);
    for (int i = 0; i < nd; ++i) scanf("%lld", (long long*)&t.stride[i]);
    mo::Canon c; std::string err; int rc = mo::canonicalize(t, c, err);
    printf("%d %d", rc, c.nd);
    for (int i = 0; i < c.nd; ++i) printf(" %lld", (long long)c.size[i]);
    for (int i = 0; i < c.nd; ++i) printf(" %lld", (long long)(c.stride[i] / 4));
    printf("\n");
  }
  return 0;
}
"""


@pytest.fixture(scope="module")
def driver(tmp_path_factory) -> Path:
    d = tmp_path_factory.mktemp("driver")
    src = d / "driver.cpp"
    src.write_text(DRIVER)
    exe = d / "driver"
    subprocess.run(
        ["g++", "-std=c++17", "-O1", f"-I{CSRC}", f"-I{ROOT / 'include'}", "-o", str(exe), str(src)], check=True
    )
    return exe


def test_fast_division_is_exact(driver) -> None:
    out = subprocess.run([str(driver), "div"], check=True, capture_output=True, text=True).stdout
    assert out.strip().endswith("bad 0"), out


def test_canonical_form_enumerates_storage_order(driver) -> None:
    """The engine's canonical dims, walked as an odometer, visit exactly the sorted offsets."""

    rng = random.Random(3)
    cases = []
    for _ in range(1500):
        ndim = rng.randint(0, 6)
        shape = [rng.choice([1, 1, 2, 3, 4, 5]) for _ in range(ndim)]
        stride = [rng.choice([1, 2, 3, 4, 6, 8, 12, 16, 20, 24, 48, 64, 96]) for _ in range(ndim)]
        cases.append((shape, stride))
    text = "".join(f"{len(s)} {' '.join(map(str, s))} {' '.join(map(str, t))}\n" for s, t in cases)
    out = subprocess.run([str(driver)], input=text, check=True, capture_output=True, text=True).stdout.splitlines()
    accepted = 0
    for (shape, stride), line in zip(cases, out):
        vals = list(map(int, line.split()))
        rc, nd = vals[0], vals[1]
        if not layout.offloadable(shape, stride):
            assert rc == _native.MO_E_LAYOUT, (shape, stride)
            continue
        assert rc == 0, (shape, stride, line)
        accepted += 1
        csize, cstride = vals[2 : 2 + nd], vals[2 + nd : 2 + 2 * nd]
        walk = layout.element_offsets(csize, cstride) if nd else np.zeros(1 if np.prod(shape) else 0, dtype=np.int64)
        assert np.array_equal(walk, np.sort(layout.element_offsets(shape, stride))), (shape, stride, line)
        # merged: no two neighbours could have been merged
        for i in range(nd - 1):
            assert cstride[i] != csize[i + 1] * cstride[i + 1]
    assert accepted > 300
