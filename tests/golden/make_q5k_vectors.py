"""Writes tests/golden/q5k_ref_vectors.npz from the reference's own Q5_K decoder.

Q5_K has no native implementation in the reference, and its rounding (a
float64 middle step, src/flatrun/dequant/gguf.py:257-262) is not pinned by
any reference test beyond the all-zero block. This script imports
``flatrun.dequant.gguf.dequant_q5_k`` from the reference checkout (in the
build container only; the reference never travels to the GPU machine) and
records input blocks and decoded outputs as a small fixture.

    python tests/golden/make_q5k_vectors.py [/root/reference]

Blocks: seeded random blocks with the benchmark distributions, blocks with
large fp16 scales and mins (where the f64 -> f32 double rounding is most
likely to differ from a single f32 rounding), fp16 subnormal scales, and a
ragged (non-multiple-of-256) size.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]


def blocks() -> dict[str, np.ndarray]:
    sys.path.insert(0, str(ROOT))
    from flatrun_amd import synth

    rng = np.random.default_rng(20261201)
    out = {}
    out["random"] = synth.make_blocks("Q5_K", 8, 1024, seed=11)           # 32 blocks
    # wide-range scales: d, dmin spanning fp16 normal range, full 6-bit scales
    nb = 24
    raw = rng.integers(0, 256, size=(nb, 176), dtype=np.uint8)
    d = (rng.uniform(-1, 1, nb) * 2.0 ** rng.integers(-14, 15, nb)).astype(np.float16).view(np.uint16)
    dm = (rng.uniform(-1, 1, nb) * 2.0 ** rng.integers(-14, 15, nb)).astype(np.float16).view(np.uint16)
    raw[:, 0], raw[:, 1] = d & 0xFF, d >> 8
    raw[:, 2], raw[:, 3] = dm & 0xFF, dm >> 8
    out["wide"] = raw.reshape(-1)
    # subnormal fp16 scales
    nb = 8
    raw = rng.integers(0, 256, size=(nb, 176), dtype=np.uint8)
    sub = rng.integers(1, 0x400, size=(nb, 2)).astype(np.uint16)
    raw[:, 0], raw[:, 1] = sub[:, 0] & 0xFF, sub[:, 0] >> 8
    raw[:, 2], raw[:, 3] = sub[:, 1] & 0xFF, sub[:, 1] >> 8
    out["subnormal"] = raw.reshape(-1)
    return out


def main(ref_root: str = "/root/reference") -> None:
    sys.path.insert(0, str(Path(ref_root) / "src"))
    from flatrun.dequant.gguf import dequant_q5_k  # the reference decoder

    arrays = {}
    for name, raw in blocks().items():
        n = raw.size // 176 * 256
        arrays[f"{name}_raw"] = raw
        arrays[f"{name}_out"] = dequant_q5_k(raw.copy(), (n,), np.float32)
    ragged = blocks()["random"][: 3 * 176]
    arrays["ragged_raw"] = ragged
    arrays["ragged_out"] = dequant_q5_k(ragged.copy(), (700,), np.float32)   # 3 blocks, tail trimmed
    np.savez_compressed(HERE / "q5k_ref_vectors.npz", **arrays)
    print("wrote", HERE / "q5k_ref_vectors.npz", {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main(*sys.argv[1:])
