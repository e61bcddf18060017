"""Writes the quantized .tl golden fixtures with the reference's own exporter.

    python tests/golden/make_tl_fixtures.py [/root/reference]

Run once, in the build container only (the reference checkout is not present
on the GPU box).  It imports the reference's format module,
tools/tl_format.py (pure struct + numpy, tools/tl_format.py:11-14), and calls
its `export_tensors` (tools/tl_format.py:250-360) on a small set of seeded
tensors in every format the module writes: f32, q8_0, q4_0, q8_k and f16.
The files it writes under tests/golden/tl/ are data -- the exporter's bytes,
including its own quantizers' output (np.round, half to even;
tools/tl_format.py:33-188) -- and the float inputs go to
exporter_inputs.npz.  Tests read both; nothing imports the reference at test
time.

Tensors (chosen to exercise the framing and the quantizers' edge cases):
  w      [64, 32]   N(0, 0.02), seed 2002 -- a weight in the [in, out] layout
  odd    [37]       N(0, 1), seed 1001    -- odd length: a lone trailing Q4
                                             nibble, a partial Q8_K block
  cube   [3, 5, 7]  N(0, 1), seed 3003    -- rank 3, 105 elements
  zeros  [40]       all zero              -- the max == 0 rule (scale 1)
  ties8  [8]        max 127: x / scale = x, so the .5 values are rounding
                    ties for q8_0 and q8_k (half to even in the exporter)
  ties4  [8]        max 7: the same for q4_0
"""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "tl")
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from tomoul_amd import synth  # noqa: E402

FORMATS = {"f32": 0, "q8_0": 1, "q4_0": 2, "q8_k": 3, "f16": 4}


def inputs() -> dict:
    return {
        "w": synth.normal_matrix(2002, 64, 32, 0.02),
        "odd": synth.normal(1001, 37),
        "cube": synth.normal(3003, 105).reshape(3, 5, 7),
        "zeros": np.zeros(40, dtype=np.float32),
        "ties8": np.array([127.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5, 126.5], dtype=np.float32),
        "ties4": np.array([7.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5, -6.5], dtype=np.float32),
    }


def main(ref_root: str) -> None:
    path = os.path.join(ref_root, "tools", "tl_format.py")
    spec = importlib.util.spec_from_file_location("reference_tl_format", path)
    tlf = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(tlf)
    tens = inputs()
    os.makedirs(OUT, exist_ok=True)
    np.savez(os.path.join(OUT, "exporter_inputs.npz"), **tens)
    for name, code in FORMATS.items():
        tlf.export_tensors(dict(tens), os.path.join(OUT, f"exporter_{name}.tl"), quant_format=code, verify=True)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
