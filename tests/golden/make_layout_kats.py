"""Write tests/golden/layout_kats.json: the reference's layout known-answer tests as data.

The cases are the ones of RyukoMatoiFan/MOSS-Image ``training/tests/test_packed_features.py``
:201-235 (``test_activation_layout_round_trip_preserves_padding_and_expansion``), restated as
inputs and expected outputs:

- padded:      ``arange(64).as_strided((1, 1, 5, 5), (64, 64, 8, 1))`` is offloadable, its
               payload shape is the full shape, and the restored view keeps strides
               ``(64, 64, 8, 1)`` and values;
- expanded:    ``arange(5).view(1, 5).expand(3, 5)`` narrows to payload shape ``(1, 5)`` and
               restores with strides ``(0, 1)``;
- overlapping: ``arange(64).as_strided((3, 3), (1, 1))`` is not offloadable.

Expected values are computed here from the definitions above (numpy, no reference import).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "layout_kats.json"


def main() -> None:
    backing = np.arange(64, dtype=np.float32)
    padded_shape, padded_stride = (1, 1, 5, 5), (64, 64, 8, 1)
    padded_values = np.lib.stride_tricks.as_strided(
        backing, shape=padded_shape, strides=tuple(s * 4 for s in padded_stride)
    ).copy()
    expanded_values = np.broadcast_to(np.arange(5, dtype=np.float32).reshape(1, 5), (3, 5)).copy()
    cases = [
        {
            "name": "padded",
            "backing": "arange64",
            "shape": list(padded_shape),
            "stride": list(padded_stride),
            "offloadable": True,
            "payload_shape": list(padded_shape),
            "restored_stride": list(padded_stride),
            "values": padded_values.reshape(-1).tolist(),
        },
        {
            "name": "expanded",
            "backing": "arange5",
            "shape": [3, 5],
            "stride": [0, 1],
            "offloadable": True,
            "payload_shape": [1, 5],
            "restored_stride": [0, 1],
            "values": expanded_values.reshape(-1).tolist(),
        },
        {
            "name": "overlapping",
            "backing": "arange64",
            "shape": [3, 3],
            "stride": [1, 1],
            "offloadable": False,
        },
    ]
    OUT.write_text(json.dumps({"source": "training/tests/test_packed_features.py:201-235", "cases": cases}, indent=1))
    print(OUT)


if __name__ == "__main__":
    main()
