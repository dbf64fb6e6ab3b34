"""Write tests/golden/packed_q6_soa_reference.npz from the reference's own packer.

Run in the build container only (the reference tree is not present where the
GPU tests run):

    python tests/golden/make_soa_golden.py

It loads the reference's NumPy-only modules kaggle/packed_q6/layout.py
(``pack_q6``, layout q6_k_soa_n64_k256_v1) and kaggle/packed_q6/reference.py
(``fixture``) straight from their files, packs a few GGUF Q6_K inputs and
stores inputs and outputs as data: the raw blocks, ``input_features`` and the
``data``/``scales`` planes the reference packer produced. No reference code is
copied into this repository; the fixture holds bytes only.
"""

import importlib.util
from pathlib import Path

import numpy as np

REFERENCE = Path("/root/reference/kaggle/packed_q6")
OUT = Path(__file__).resolve().parent / "packed_q6_soa_reference.npz"


def _load(name):
    spec = importlib.util.spec_from_file_location(f"reference_packed_q6_{name}", REFERENCE / f"{name}.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def main():
    layout, reference = _load("layout"), _load("reference")
    cases = {}
    # two output tiles x two K blocks with a partial last block of each
    cases["r65_k300"] = (reference.fixture(65, 300, seed=11), 300)
    # three ragged output tiles x three K blocks
    cases["r130_k520"] = (reference.fixture(130, 520, seed=12), 520)
    # every sub-scale byte value and FP16 extremes (the reference test's case)
    raw = reference.fixture(64, 256, seed=13)
    raw[:, :, 192:208] = np.arange(1024, dtype=np.uint16).astype(np.uint8).reshape(64, 1, 16)
    raw[:4, 0, 208:210] = np.array([65504, -65504, 2**-24, -(2**-14)], "<f2").view(np.uint8).reshape(4, 2)
    cases["r64_k256_all_scales"] = (raw, 256)
    arrays = {}
    for name, (raw, inputs) in cases.items():
        packed = layout.pack_q6(raw, inputs)
        arrays[f"{name}_raw"] = raw
        arrays[f"{name}_inputs"] = np.array(inputs, np.int64)
        arrays[f"{name}_data"] = np.asarray(packed.data)
        arrays[f"{name}_scales"] = np.asarray(packed.scales)
        arrays[f"{name}_outputs"] = np.array(packed.output_features, np.int64)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes): {', '.join(cases)}")


if __name__ == "__main__":
    main()
