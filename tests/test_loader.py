"""Host logic of flatrun_amd.loader.dequant_handle (the reference's
src/flatrun/dequant/loader.py:51-88): paths that decide before any GPU work."""

from __future__ import annotations

from types import SimpleNamespace as NS

import numpy as np
import pytest

from flatrun_amd import loader


def handle(q, shape, arr):
    return NS(metadata=NS(quantization=q, shape=shape), as_numpy=lambda: arr)


def test_untagged_tensor_is_cast_to_dtype():
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    out = loader.dequant_handle(handle(None, (3, 4), a))         # default dtype float16
    assert out.dtype == np.float16 and np.array_equal(out, a.astype(np.float16))
    same = loader.dequant_handle(handle(None, (3, 4), a), dtype="float32")
    assert same is a                                                  # no copy when the dtype matches
    h = a.astype(np.float16)
    assert loader.dequant_handle(handle(None, (3, 4), h)) is h


@pytest.mark.parametrize("q,msg", [("MLX_4BIT", "dequant_mlx_weight"), ("IQ3_XXS", "no decoder"),
                                   ("Q2_K", "no decoder")])
def test_unsupported_tags_raise_value_error(q, msg):
    with pytest.raises(ValueError, match=msg):
        loader.dequant_handle(handle(q, (4, 256), np.zeros(144 * 4, np.uint8)))


def test_decoder_table_matches_the_reference_formats():
    assert sorted(loader.GGUF_DECODERS) == sorted(["Q1_0", "Q4_0", "Q5_0", "Q5_1", "Q8_0", "Q4_K", "Q5_K", "Q6_K"])


@pytest.mark.parametrize("q,shape,nbytes", [("Q4_K", (2, 256), 144), ("Q8_0", (3, 32), 34 * 3 + 1),
                                            ("Q1_0", (300,), 18 * 2)])
def test_wrong_byte_count_raises_value_error(q, shape, nbytes):
    with pytest.raises(ValueError, match="bytes of blocks"):
        loader.dequant_handle(handle(q, shape, np.zeros(nbytes, np.uint8)))


@pytest.mark.parametrize("dtype", ["float16", "float32", "float64"])
def test_empty_tensor(dtype):
    out = loader.dequant_handle(handle("Q4_K", (0, 256), np.zeros(0, np.uint8)), dtype=dtype)
    assert out.shape == (0, 256) and out.dtype == np.dtype(dtype)
