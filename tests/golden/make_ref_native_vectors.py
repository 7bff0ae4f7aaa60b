"""Writes tests/golden/ref_native_vectors.npz from the reference's native build.

The reference's pybind11 module ``flatrun_native._C`` is compiled from its
sources (``make -C oracle ref``, in the build container only) and run on
seeded blocks; inputs and outputs are stored so the oracle can be checked
against them on any machine, including the GPU host where the reference does
not exist.

    python tests/golden/make_ref_native_vectors.py

Per format (Q4_K, Q6_K, Q8_0): benchmark-distribution blocks with every
packed field random (K-quant scale high bits included), plus a handful of
edge blocks (zero scales, negative / large fp16 scales), dequant output and
the matmul output for one x, and the batched output for a 3-row x.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))


def main() -> None:
    from flatrun_amd import synth
    from oracle.loader import build, ref_C

    build()
    R = ref_C()
    if R is None:
        raise SystemExit("reference _C module not built (is /root/reference present?)")
    rng = np.random.default_rng(7)
    arrays = {}
    shapes = {"Q4_K": (24, 512), "Q6_K": (24, 512), "Q8_0": (24, 256)}
    for q, (n, k) in shapes.items():
        raw = synth.make_blocks(q, n, k, seed=100 + len(arrays))
        bb = synth.BLOCK[q][0]
        blocks = raw.reshape(-1, bb)
        # edge blocks: zero scale, negative scale, large scale
        f16_off = {"Q4_K": [0, 2], "Q6_K": [208], "Q8_0": [0]}[q]
        for row, val in ((0, 0.0), (1, -0.75), (2, 3000.0)):
            h = np.float16(val).view(np.uint16)
            for off in f16_off:
                blocks[row, off] = h & 0xFF
                blocks[row, off + 1] = h >> 8
        x = rng.standard_normal(k).astype(np.float32)
        x3 = rng.standard_normal((3, k)).astype(np.float32)
        tag = q.lower()
        arrays[f"{tag}_raw"] = raw
        arrays[f"{tag}_shape"] = np.array([n, k])
        arrays[f"{tag}_x"] = x
        arrays[f"{tag}_x3"] = x3
        arrays[f"{tag}_dequant"] = getattr(R, f"dequant_{tag}")(raw, (n, k))
        arrays[f"{tag}_matmul"] = getattr(R, f"matmul_{tag}")(x, raw, n, k)
        arrays[f"{tag}_matmul3"] = getattr(R, f"matmul_{tag}_batched")(x3, raw, n, k)
    arrays["version"] = np.frombuffer(R.version().encode(), dtype=np.uint8)
    np.savez_compressed(HERE / "ref_native_vectors.npz", **arrays)
    print("wrote", HERE / "ref_native_vectors.npz", sum(v.nbytes for v in arrays.values()), "bytes")


if __name__ == "__main__":
    main()
