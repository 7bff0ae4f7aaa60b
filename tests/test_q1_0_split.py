"""The matrix-core Q1_0 GEMV's arithmetic (tests/q1_0_split.py), on the CPU:
balanced digits reconstruct every |m| < 2^30, the digit sums give the
group's sum of +-m exactly, the 30-bit truncation stays within 2^-24 of each
group's sum |x| (so, as |w| = |d| across a block, of its sum |w x|) on
adversarial groups, and the whole model meets the 1e-5 contract against the
fp64 oracle with outliers, tiny and subnormal values."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import MATVEC_RTOL, matvec_errors
from flatrun_amd import synth
from oracle import gguf_np as G
from q1_0_split import GROUP, balanced_digits, default_blocks_per_wave, emulate, group_split


def test_balanced_digits_reconstruct():
    rng = np.random.default_rng(1)
    m = np.concatenate([np.array([0, 1, -1, 127, 128, -128, -129, 255, 256, 2**30 - 1, -(2**30 - 1), 0x808080,
                                  -0x808080, 0x7F7F7F, -0x7F7F7F]),
                        rng.integers(-(2**30 - 1), 2**30, 20000)]).astype(np.int64)
    d = balanced_digits(m).astype(np.int64)
    assert np.array_equal((d * (256 ** np.arange(4))).sum(axis=1), m)
    assert d.min() >= -128 and d.max() <= 127


def test_digit_sums_give_signed_sum():
    """S = sum_i 256^i (2 C_i - J_i) with C_i over the set bits and J_i over
    all 32 elements equals sum(+-m), and its int32 halves stay below 2^22."""
    rng = np.random.default_rng(2)
    for _ in range(200):
        m = rng.integers(-(2**30 - 1), 2**30, GROUP)
        bits = rng.integers(0, 2, GROUP)
        d = balanced_digits(m).astype(np.int64)
        C = (d * bits[:, None]).sum(axis=0)
        J = d.sum(axis=0)
        p01 = 2 * (C[0] + 256 * C[1]) - (J[0] + 256 * J[1])
        p23 = 2 * (C[2] + 256 * C[3]) - (J[2] + 256 * J[3])
        assert p01 + 65536 * p23 == np.sum(np.where(bits == 1, m, -m))
        assert abs(p01) < 2**22 and abs(p23) < 2**22


def _adversarial_groups(rng, count):
    out = []
    for _ in range(count):
        g = (rng.standard_normal(GROUP) * 10.0 ** rng.uniform(-30, 30)).astype(np.float32)
        kind = rng.integers(0, 4)
        if kind == 0:                                           # one outlier, the rest tiny
            g[rng.integers(GROUP)] = np.float32(2.0 ** rng.integers(0, 60))
        elif kind == 1:                                         # subnormals
            g = (rng.standard_normal(GROUP) * 1e-40).astype(np.float32)
        elif kind == 2:                                         # largest finite values
            g[: 4] = np.float32(3.4e38) * rng.choice([-1, 1], 4)
        out.append(g)
    return np.stack(out)


def test_truncation_bound():
    """|sum(+-x) - 2^(e-30) sum(+-m)| < 32 * 2^(e-30) <= 2^-24 * max|x| per
    group, for every sign pattern (checked on random ones)."""
    rng = np.random.default_rng(3)
    groups = _adversarial_groups(rng, 2000)
    # one group per 128-element block (group 0), the block's other groups zero
    m, eo = group_split(np.stack([np.concatenate([g, np.zeros(3 * GROUP, np.float32)]) for g in groups]).reshape(-1))
    m, eo = m[:, 0, :], eo[:, 0]
    for i, g in enumerate(groups):
        s = rng.choice([-1.0, 1.0], GROUP)
        exact = float(np.sum(s * g.astype(np.float64)))
        approx = float(np.ldexp(np.sum(s * m[i].astype(np.float64)), int(eo[i])))
        bound = 2.0**-24 * float(np.max(np.abs(g.astype(np.float64))))
        assert abs(exact - approx) <= bound, (i, exact, approx, bound)


@pytest.mark.parametrize("n,k", [(40, 4096), (17, 1024), (5, 16384)])
def test_model_meets_contract(n, k):
    raw = synth.make_blocks("Q1_0", n, k, seed=n + k)
    rng = np.random.default_rng(k)
    x = synth.make_x(k, seed=k)
    x[0], x[1:32] = 2.0**30, x[1:32] * np.float32(1e-6)
    x[64:96] = (rng.standard_normal(32) * 1e-40).astype(np.float32)
    for gi in range(3, k // 32):
        x[32 * gi:32 * gi + 32] *= np.float32(2.0 ** int(rng.integers(-100, 100)))
    y = emulate(raw, x, n, k, default_blocks_per_wave(k // 128))
    nw, cw = matvec_errors(y, G.matmul_f64("Q1_0", x, raw, n, k), G.abs_matmul_f64("Q1_0", x, raw, n, k))
    assert nw < MATVEC_RTOL / 10 and cw < MATVEC_RTOL / 10, (nw, cw)
