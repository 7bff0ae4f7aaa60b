"""Pins the oracle (oracle/gguf_np.py, oracle/native_ref.c) beyond the reference KATs.

* Hand-built blocks written byte by byte from the layout rules stated in the
  reference (gguf.py docstrings :84-95, :176-180, :234-237, :381-384, :274-282)
  -- not through the oracle's own code -- so a permuted nibble order, a lost
  scale high bit or a swapped Q6_K qh pair fails here.
* Exactness facts that make the bit-exact contract well defined.
* Committed fixtures written from the reference's own code
  (tests/golden/make_*.py) and, where oracle/_ref is built, the live
  reference module.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import GOLDEN, bits_equal
from oracle import gguf_np as G
from oracle.loader import c_oracle

F32 = np.float32


def _f16(v) -> bytes:
    return np.float16(v).tobytes()


# ---------------------------------------------------------------- Q4_K / Q5_K

def _q4k_order_block(d=1.0, dmin=0.0):
    """qs byte 32g+i = lo | hi << 4 with lo = i % 16, hi = 15 - i % 16;
    scales sc_j = j + 1, mins m_j = 2j + 1 (all < 16: no high bits)."""
    sc = list(range(1, 9))
    mn = [2 * j + 1 for j in range(8)]
    s12 = bytearray(12)
    for j in range(4):
        s12[j] = sc[j]
        s12[j + 4] = mn[j]
        s12[j + 8] = sc[j + 4] | (mn[j + 4] << 4)
    qs = bytes((i % 16) | ((15 - i % 16) << 4) for g in range(4) for i in range(32))
    raw = _f16(d) + _f16(dmin) + bytes(s12) + qs
    exp = np.empty(256, np.float64)
    for g in range(4):
        for i in range(32):
            exp[64 * g + i] = d * sc[2 * g] * (i % 16) - dmin * mn[2 * g]
            exp[64 * g + 32 + i] = d * sc[2 * g + 1] * (15 - i % 16) - dmin * mn[2 * g + 1]
    return raw, exp


def test_q4_k_element_order_and_scales():
    raw, exp = _q4k_order_block(d=1.0, dmin=0.0)
    assert np.array_equal(G.dequant_q4_k(raw, (256,)), exp.astype(F32))
    raw, exp = _q4k_order_block(d=0.0, dmin=1.0)             # mins only
    assert np.array_equal(G.dequant_q4_k(raw, (256,)), exp.astype(F32))
    raw, exp = _q4k_order_block(d=0.5, dmin=0.25)
    assert np.array_equal(G.dequant_q4_k(raw, (256,)), exp.astype(F32))
    c = c_oracle().dequant("Q4_K", np.frombuffer(raw, np.uint8), 256)
    assert bits_equal(c, exp.astype(F32))


def test_k_scale_high_bits():
    """Sub-blocks 4..7 take their top two bits from bytes 0..7 (gguf.py:139-147).
    Bytes: b[j] = 0b11000000 | j (j<4), b[j+4] = 0b10000000 | (j+8), b[j+8] = 0x5A."""
    s12 = bytes([0xC0 | j for j in range(4)] + [0x80 | (j + 8) for j in range(4)] + [0x5A] * 4)
    sc, m = G.scale_min_k4(np.frombuffer(s12, np.uint8)[None, :])
    exp_sc = [0, 1, 2, 3] + [(0x5A & 15) | (3 << 4)] * 4          # 10 | 48 = 58
    exp_m = [8, 9, 10, 11] + [(0x5A >> 4) | (2 << 4)] * 4         # 5 | 32 = 37
    assert sc[0].tolist() == exp_sc and m[0].tolist() == exp_m
    # through the full decoder: d=1, dmin=0, all nibbles 1 -> output = sc of the sub-block
    raw = _f16(1.0) + _f16(0.0) + s12 + bytes([0x11]) * 128
    out = G.dequant_q4_k(raw, (256,))
    assert np.array_equal(out, np.repeat(np.array(exp_sc, F32), 32))
    assert np.array_equal(c_oracle().dequant("Q4_K", np.frombuffer(raw, np.uint8), 256), out)
    # Q5_K shares the scale field
    raw5 = _f16(1.0) + _f16(0.0) + s12 + bytes(32) + bytes([0x11]) * 128
    assert np.array_equal(G.dequant_q5_k(raw5, (256,)), out)


def test_q5_k_high_bit_per_group():
    """Group g tests qh bit 2g (low nibbles) and 2g+1 (high nibbles), +16 each
    (gguf.py:234-237). qh[i] = 1 << (i % 8) sets exactly one sub-block per byte."""
    s12 = bytes([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1])              # all sc = 1, m = 0
    qh = bytes(1 << (i % 8) for i in range(32))
    raw = _f16(1.0) + _f16(0.0) + s12 + qh + bytes(128)
    out = G.dequant_q5_k(raw, (256,))
    exp = np.zeros(256, F32)
    for i in range(32):
        j = i % 8                                                  # sub-block 2g + hi
        g, hi = j // 2, j % 2
        exp[64 * g + 32 * hi + i] = 16.0
    assert np.array_equal(out, exp)


def test_k_quant_products_are_exact():
    """Every product in the K-quant / Q6_K / Q8_0 decoders is exact in fp32:
    an fp16 value has <= 11 significant bits, a 6-bit scale <= 6, a stored
    value <= 6 (Q6_K: int8 scale 8 bits, q-32 6 bits), so products need <= 24.
    Hence the only rounding in dequant is the final Q4_K / Q5_K subtraction,
    and Q5_K's float64 middle step (gguf.py:257-262) cannot change a result.
    Checked exhaustively over all finite fp16 d and all scale values."""
    h = np.arange(0x10000, dtype=np.uint16).view(np.float16)
    d = h[np.isfinite(h)].astype(np.float64)
    for sc in range(64):
        p = d * sc
        assert np.array_equal(p.astype(F32).astype(np.float64), p)          # fl32(d*sc) exact
        for v in (31, 29, 27, 23, 19, 17, 15):                              # max-width odd v <= 31
            pv = p * v
            assert np.array_equal(pv.astype(F32).astype(np.float64), pv)    # (d*sc)*v exact
    for sc in range(-128, 128, 7):                                          # Q6_K: d*sc*(q-32)
        p = d * sc
        assert np.array_equal(p.astype(F32).astype(np.float64), p)
        for v in (-32, -31, 31, 29):
            pv = p * v
            ok = np.isfinite(pv)
            assert np.array_equal(pv[ok].astype(F32).astype(np.float64), pv[ok])


# ---------------------------------------------------------------- Q6_K

def test_q6_k_layout_all_groups():
    """Element 128h + 32k + l from ql / qh / scales as in gguf.py:381-384:
    q1..q4 = ql[l] lo, ql[l+32] lo, ql[l] hi, ql[l+32] hi, each | qh pair k."""
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for h in range(2):
        for l in range(32):
            ql[64 * h + l] = (l % 16) | ((15 - l % 16) << 4)
            ql[64 * h + 32 + l] = ((l + 3) % 16) | (((l + 7) % 16) << 4)
            qh[32 * h + l] = 0xE4 if h == 0 else 0x1B                       # pairs (0,1,2,3) / (3,2,1,0)
    scales = np.array([(-1) ** i * (i + 1) for i in range(16)], np.int8)
    raw = ql.tobytes() + qh.tobytes() + scales.tobytes() + _f16(0.5)
    exp = np.empty(256, np.float64)
    for h in range(2):
        pairs = (0, 1, 2, 3) if h == 0 else (3, 2, 1, 0)
        for l in range(32):
            nib = [l % 16, (l + 3) % 16, 15 - l % 16, (l + 7) % 16]
            for k in range(4):
                q = nib[k] | (pairs[k] << 4)
                exp[128 * h + 32 * k + l] = 0.5 * scales[8 * h + l // 16 + 2 * k] * (q - 32)
    out = G.dequant_q6_k(raw, (256,))
    assert np.array_equal(out, exp.astype(F32))
    assert np.array_equal(c_oracle().dequant("Q6_K", np.frombuffer(raw, np.uint8), 256), out)


# ---------------------------------------------------------------- Q1_0 / Q8_0

def test_q1_0_lsb_first_random():
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 2, size=(5, 128)).astype(np.uint8)
    raw = b"".join(_f16(0.125 * (b + 1)) + bytes(
        sum(int(bits[b, 8 * i + j]) << j for j in range(8)) for i in range(16)) for b in range(5))
    exp = np.where(bits == 1, 1.0, -1.0) * (0.125 * (np.arange(5)[:, None] + 1))
    assert np.array_equal(G.dequant_q1_0(raw, (640,)), exp.reshape(-1).astype(F32))


def test_q8_0_signed_values():
    q = np.arange(-128, 128, 8, dtype=np.int8)
    raw = _f16(-0.375) + q.tobytes()
    assert np.array_equal(G.dequant_q8_0(raw, (32,)), (q.astype(np.float64) * -0.375).astype(F32))


# ---------------------------------------------------------------- fp16 edge cases

def test_fp16_subnormal_reference_native_discrepancy():
    """NumPy (the dequant contract) converts fp16 subnormals exactly; the
    reference's native fp16_to_fp32 (q4_k.h:64-70) uses exponent 112 - shift
    and returns half the value. The C restatement keeps that behaviour."""
    for hbits in (0x0001, 0x0200, 0x03FF, 0x8001):
        ieee = float(np.array([hbits], np.uint16).view(np.float16)[0])
        assert c_oracle().fp16_to_fp32(hbits) == ieee / 2
    for hbits in (0x0400, 0x3C00, 0x7BFF, 0xFBFF, 0x0000, 0x8000, 0x7C00, 0xFC00):
        ieee = float(np.array([hbits], np.uint16).view(np.float16)[0])
        assert c_oracle().fp16_to_fp32(hbits) == ieee


def test_fp16_subnormal_in_reference_build(ref_C):
    raw = np.frombuffer(np.uint16(0x0200).tobytes() + np.full(32, 3, np.int8).tobytes(), np.uint8)
    ref = ref_C.dequant_q8_0(raw, (1, 32))
    ours = G.dequant_q8_0(raw, (1, 32))
    assert np.array_equal(ref * 2, ours)       # reference native halves fp16 subnormal scales


# ---------------------------------------------------------------- golden fixtures

NATIVE = np.load(GOLDEN / "ref_native_vectors.npz")


@pytest.mark.parametrize("q", ["Q4_K", "Q6_K", "Q8_0"])
def test_oracle_vs_reference_native_vectors(q):
    t = q.lower()
    raw, (n, k) = NATIVE[f"{t}_raw"], NATIVE[f"{t}_shape"]
    assert bits_equal(G.DEQUANT[q](raw, (n, k)), NATIVE[f"{t}_dequant"])
    assert bits_equal(c_oracle().dequant(q, raw, n * k).reshape(n, k), NATIVE[f"{t}_dequant"])
    assert bits_equal(c_oracle().matmul(q, NATIVE[f"{t}_x"], raw, n, k), NATIVE[f"{t}_matmul"])
    assert bits_equal(c_oracle().matmul(q, NATIVE[f"{t}_x3"], raw, n, k), NATIVE[f"{t}_matmul3"])
    # the NumPy matvec (BLAS order) agrees with the native order to ~1e-6
    y = G.matmul_numpy(q, NATIVE[f"{t}_x"], raw, n, k)
    r = NATIVE[f"{t}_matmul"]
    assert np.max(np.abs(y - r)) <= 1e-5 * np.max(np.abs(r))


Q5K = np.load(GOLDEN / "q5k_ref_vectors.npz")


@pytest.mark.parametrize("name", ["random", "wide", "subnormal"])
def test_oracle_vs_reference_q5_k_vectors(name):
    raw, out = Q5K[f"{name}_raw"], Q5K[f"{name}_out"]
    assert bits_equal(G.dequant_q5_k(raw, (out.size,)), out)


def test_oracle_q5_k_ragged_vector():
    assert bits_equal(G.dequant_q5_k(Q5K["ragged_raw"], (700,)), Q5K["ragged_out"])


# ---------------------------------------------------------------- live reference build

@pytest.mark.parametrize("q,n,k,seed", [("Q4_K", 33, 768, 1), ("Q6_K", 17, 1024, 2), ("Q8_0", 40, 96, 3)])
def test_oracle_vs_live_reference(ref_C, q, n, k, seed):
    from flatrun_amd import synth

    raw = synth.make_blocks(q, n, k, seed=seed)
    t = q.lower()
    assert bits_equal(G.DEQUANT[q](raw, (n, k)), getattr(ref_C, f"dequant_{t}")(raw, (n, k)))
    x = synth.make_x(k, seed=seed + 10)
    assert bits_equal(c_oracle().matmul(q, x, raw, n, k), getattr(ref_C, f"matmul_{t}")(x, raw, n, k))


def test_c_oracle_threads_match_single(ref_C):
    from flatrun_amd import synth

    raw = synth.make_blocks("Q4_K", 64, 1024, seed=9)
    x = synth.make_x(1024, seed=4)
    assert bits_equal(c_oracle().matmul("Q4_K", x, raw, 64, 1024, threads=4),
                      c_oracle().matmul("Q4_K", x, raw, 64, 1024, threads=1))


# ---------------------------------------------------------------- Q4_0 / Q5_0 / Q5_1
# One nibble or one qh bit is changed at a time; exactly the element it belongs
# to (low nibble of byte j -> element j, high nibble -> j + 16, qh bit b ->
# element b) must move, by the closed-form amount.

def _blk32(q, d=0.5, m=0.25, qh=0, qs=None):
    qs = np.zeros(16, np.uint8) if qs is None else qs
    head = np.float16(d).tobytes()
    if q == "Q5_1":
        head += np.float16(m).tobytes()
    if q in ("Q5_0", "Q5_1"):
        head += np.uint32(qh).tobytes()
    return np.frombuffer(head + qs.tobytes(), np.uint8)


def test_q4_0_each_nibble_lands_on_its_element():
    base = np.full(16, 0x88, np.uint8)                      # every element (8 - 8) * d = 0
    assert np.array_equal(G.dequant_q4_0(_blk32("Q4_0", qs=base), (32,)), np.zeros(32, np.float32))
    for j in range(16):
        for hi in (False, True):
            qs = base.copy()
            qs[j] = 0x8F if not hi else 0xF8                # nibble 15: (15 - 8) * 0.5 = 3.5
            out = G.dequant_q4_0(_blk32("Q4_0", qs=qs), (32,))
            exp = np.zeros(32, np.float32)
            exp[j + 16 * hi] = 3.5
            assert np.array_equal(out, exp), (j, hi)


@pytest.mark.parametrize("q", ["Q5_0", "Q5_1"])
def test_q5_each_qh_bit_lands_on_its_element(q):
    d, m = 0.5, 0.25
    low = -16 * d if q == "Q5_0" else m                     # qs = 0, no high bit
    for b in range(32):
        out = G.DEQUANT[q](_blk32(q, d=d, m=m, qh=1 << b), (32,))
        exp = np.full(32, low, np.float32)
        exp[b] = low + 16 * d
        assert np.array_equal(out, exp), (q, b)


@pytest.mark.parametrize("q", ["Q5_0", "Q5_1"])
def test_q5_nibbles_and_high_bit_combine(q):
    """q = nibble | 16 * bit, for every (nibble, bit) on every position."""
    rng = np.random.default_rng(3)
    for _ in range(20):
        qs = rng.integers(0, 256, 16, dtype=np.uint8)
        qh = int(rng.integers(0, 2 ** 32, dtype=np.uint64))
        d = float(np.float16(rng.uniform(1e-3, 1e-2)))
        m = float(np.float16(rng.uniform(-0.1, 0.1)))
        out = G.DEQUANT[q](_blk32(q, d=d, m=m, qh=qh, qs=qs), (32,)).astype(np.float64)
        for e in range(32):
            nib = (int(qs[e % 16]) >> (4 * (e // 16))) & 15
            v = nib + 16 * ((qh >> e) & 1)
            ref = (v - 16) * d if q == "Q5_0" else np.float32(np.float32(d) * np.float32(v) + np.float32(m))
            assert out[e] == ref, (q, e)
