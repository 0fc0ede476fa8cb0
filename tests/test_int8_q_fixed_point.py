"""The int8 decode's fixed-point q, checked exhaustively on the CPU.

For an int8 cache the HIP kernel multiplies the stored K bytes with q held per
head as an integer: with e chosen from the head's max|q| (max|q| * 2^e in
[2^13, 2^14)), t = floor(q * 2^e + 128.5) = round(q * 2^e) + 128, and the two
int8 MFMA operands are hi = byte 1 of t and lo = byte 0 of t with its top bit
flipped. These tests restate that arithmetic in numpy and check, for every
finite fp16 q and every exponent e a head can get, that:
  * the fp32 sum the kernel forms before the floor never moves it: t is
    exactly round-half-up(q * 2^e) + 128;
  * 256 * hi + lo reconstructs round(q * 2^e) exactly;
  * hi stays within [-64, 64] and lo within [-128, 127], so the int32 score
    256 * (K.hi) + K.lo cannot overflow for |K| <= 128 and head_dim <= 256;
  * |q - 2^-e round(q * 2^e)| <= 2^-14 max|q|.
GPU parity of the kernel itself is in tests/test_gpu_*.py.
"""

from __future__ import annotations

import numpy as np


def _all_fp16() -> np.ndarray:
    q = np.arange(1 << 16, dtype=np.uint16).view(np.float16).astype(np.float64)
    return q[np.isfinite(q)]


def _exponent(amax: float) -> int:
    # frexp: amax = m * 2^x, m in [0.5, 1); e = 14 - x puts amax * 2^e in [2^13, 2^14)
    _, x = np.frexp(amax)
    return 14 - int(x)


def _split(q: np.ndarray, e: int):
    # the kernel's v_fma_f32(q, 2^e, 128.5): q * 2^e is exact in fp32 (an fp16
    # value times a power of two), so the fma is one fp32 rounding of the sum
    s32 = (q.astype(np.float32) * np.float32(2.0 ** e)) + np.float32(128.5)
    t = np.floor(s32.astype(np.float64)).astype(np.int64)
    hi = ((t >> 8) & 0xFF).astype(np.uint8).view(np.int8).astype(np.int64)
    lo = ((t & 0xFF) ^ 0x80).astype(np.uint8).view(np.int8).astype(np.int64)
    return t, hi, lo


def test_split_reconstructs_every_fp16_value_at_every_exponent():
    q_all = _all_fp16()
    # every head max|q| exponent a finite fp16 head can have
    amaxes = np.unique(np.abs(q_all[q_all != 0]))
    exps = sorted({_exponent(a) for a in amaxes})
    for e in exps:
        # a head with this exponent holds values of magnitude <= its max < 2^(14 - e)
        lim = 2.0 ** (14 - e)
        q = q_all[np.abs(q_all) < lim]
        t, hi, lo = _split(q, e)
        rounded = t - 128
        # the fp32 sum never moves the floor: t is exactly round-half-up(q 2^e) + 128
        assert np.array_equal(rounded, np.floor(q * 2.0 ** e + 0.5).astype(np.int64)), e
        assert np.array_equal(256 * hi + lo, rounded), e
        assert hi.min() >= -64 and hi.max() <= 64, e
        assert lo.min() >= -128 and lo.max() <= 127, e
        # round half up of the exactly scaled value: within half a step
        assert np.all(np.abs(q * 2.0 ** e - rounded) <= 0.5), e


def test_quantisation_error_is_within_2_pow_minus_14_of_the_head_max():
    rng = np.random.default_rng(3)
    for scale in (1e-6, 1e-3, 0.5, 1.0, 3.0, 1e3, 1e4):
        q = (rng.standard_normal((64, 128)) * scale).astype(np.float16).astype(np.float64)
        assert np.isfinite(q).all()
        for row in q:
            amax = np.abs(row).max()
            if amax == 0:
                continue
            e = _exponent(amax)
            t, hi, lo = _split(row, e)
            back = (256 * hi + lo) * 2.0 ** -e
            assert np.abs(back - row).max() <= 2.0 ** -14 * amax, (scale, amax)


def test_int32_score_cannot_overflow():
    # |K| <= 128 (any int8), |hi| <= 64, |lo| <= 128, head_dim <= 256
    worst = 256 * (128 * 64 * 256) + 128 * 128 * 256
    assert worst < 2 ** 31
