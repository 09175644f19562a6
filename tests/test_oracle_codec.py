"""Pins the oracle's INT4 codec and dequantization (both restatements).

Known-answer vectors are the reference's own test expectations
(tests/test_quantization.py, tests/test_phase_e_correctness.py,
tests/test_triton_unpack.py); the exhaustive tables check the closed form of
quantization.py:49 / :70-78 / :258 on every byte and every code x zero pair.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle.oracle import PackingFormat

CANON = PackingFormat.CANONICAL
LEGACY = PackingFormat.LEGACY_SIGNED_ADD


def _sext4(n):
    n = np.asarray(n, dtype=np.int16)
    return np.where(n >= 8, n - 16, n)


@pytest.mark.parametrize("packing", list(PackingFormat))
def test_pack_unpack_round_trip(packing, c_oracle):
    # tests/test_quantization.py:15-19
    codes = np.array([-7, -6, -1, 0, 1, 6, 7, -3], dtype=np.int8)
    for impl in (O, c_oracle):
        np.testing.assert_array_equal(impl.unpack_int4(impl.pack_int4(codes, packing), packing), codes)


def test_canonical_raw_byte_layout(c_oracle):
    # tests/test_quantization.py:22-25: K-even -1 -> low 0xF; K-odd 2 -> high 0x2.
    for impl in (O, c_oracle):
        assert impl.pack_int4(np.array([-1, 2], dtype=np.int8), CANON).tolist() == [0x2F]


def test_legacy_borrow_is_not_canonical_unpacking(c_oracle):
    # tests/test_quantization.py:28-32
    for impl in (O, c_oracle):
        packed = impl.pack_int4(np.array([3, -2], dtype=np.int8), LEGACY)
        assert impl.unpack_int4(packed, CANON).tolist() == [-2, 2]
        assert impl.unpack_int4(packed, LEGACY).tolist() == [3, -2]


def test_packed_signed_zero_points_use_canonical_nibble_order(c_oracle):
    # tests/test_phase_e_correctness.py:102-108
    signed = np.array([-8, -1, 0, 7], dtype=np.int8)
    for impl in (O, c_oracle):
        packed = impl.pack_int4(signed, CANON)
        assert packed.tolist() == [0xF8, 0x70]
        np.testing.assert_array_equal(impl.unpack_int4(packed, CANON), signed)


@pytest.mark.parametrize("codes", [[-8, -7, -1, 0, 1, 6, 7, -8], [7, -8, 0, -1, 3, -4, -5, 6]])
def test_unpack_boundary_patterns(codes, c_oracle):
    # tests/test_triton_unpack.py:28-38
    codes = np.array(codes, dtype=np.int8)
    for impl in (O, c_oracle):
        np.testing.assert_array_equal(impl.unpack_int4(impl.pack_int4(codes, CANON), CANON), codes)


def test_unpack_random_bytes_odd_element_count(c_oracle):
    # tests/test_triton_unpack.py:41-46 (same seed and generator)
    torch.manual_seed(20260831)
    packed = torch.randint(0, 256, (513,), dtype=torch.uint8).numpy()
    expected = np.empty(1026, dtype=np.int16)
    expected[0::2] = _sext4(packed & 0x0F)
    expected[1::2] = _sext4(packed >> 4)
    for impl in (O, c_oracle):
        np.testing.assert_array_equal(impl.unpack_int4(packed, CANON, elements=1025), expected[:1025])
    with pytest.raises(ValueError):
        O.unpack_int4(packed, CANON, elements=1027)
    with pytest.raises(ValueError):
        c_oracle.unpack_int4(packed, CANON, elements=1027)


def test_exhaustive_byte_table(c_oracle):
    every = np.arange(256, dtype=np.uint8)
    lo, hi = _sext4(every & 0x0F), _sext4(every >> 4)
    canonical = np.stack([lo, hi], axis=1).reshape(-1)
    # legacy: the low nibble borrowed from the high one when negative (:65-69),
    # and the first logical value sits in the high nibble (:73-75).
    legacy_hi = _sext4((np.asarray(every >> 4, dtype=np.int16) + ((every & 0x0F) >= 8)) & 0x0F)
    legacy = np.stack([legacy_hi, lo], axis=1).reshape(-1)
    for impl in (O, c_oracle):
        np.testing.assert_array_equal(impl.unpack_int4(every, CANON), canonical)
        np.testing.assert_array_equal(impl.unpack_int4(every, LEGACY), legacy)


def test_exhaustive_pair_table(c_oracle):
    pairs = np.array([(a, b) for a in range(-8, 8) for b in range(-8, 8)], dtype=np.int8).reshape(-1)
    expected = np.array([((a & 0xF) | ((b & 0xF) << 4)) for a in range(-8, 8) for b in range(-8, 8)],
                        dtype=np.uint8)
    for impl in (O, c_oracle):
        packed = impl.pack_int4(pairs, CANON)
        np.testing.assert_array_equal(packed, expected)
        np.testing.assert_array_equal(impl.unpack_int4(packed, CANON), pairs)
        legacy = impl.pack_int4(pairs, LEGACY)
        np.testing.assert_array_equal(impl.unpack_int4(legacy, LEGACY), pairs)


def test_pack_rejects_odd_count_and_range():
    with pytest.raises(ValueError, match="even"):
        O.pack_int4(np.array([1, 2, 3], dtype=np.int8))
    with pytest.raises(ValueError, match=r"\[-8, 7\]"):
        O.pack_int4(np.array([8, 0], dtype=np.int16))


def test_groupwise_dequantization_indexes_scales_along_k(c_oracle):
    # tests/test_quantization.py:35-49
    codes = np.array([[1, 2, 3, 4], [-1, -2, -3, -4]], dtype=np.int8)
    scales = np.array([[0.5, 2.0], [1.0, 0.25]], dtype=np.float16)
    packed = O.pack_int4(codes, CANON)
    zeros = np.zeros(2, dtype=np.uint8)
    expected = np.array([[0.5, 1.0, 6.0, 8.0], [-1.0, -2.0, -0.75, -1.0]], dtype=np.float32)
    got = O.dequantize_groupwise(packed, scales, out_features=2, in_features=4, group_size=2,
                                 packing=CANON, zeros=zeros)
    np.testing.assert_array_equal(got, expected)
    np.testing.assert_array_equal(c_oracle.dequantize_groupwise(packed, scales, zeros, 2, 4, 2), expected)


def test_asymmetric_w4g64_dequantization_uses_each_group_zero_and_scale(c_oracle):
    # tests/test_phase_e_correctness.py:111-121
    codes = np.array([[-8] * 64 + [7] * 64], dtype=np.int8)
    scales = np.array([[0.25, 2.0]], dtype=np.float16)
    zeros = O.pack_int4(np.array([-7, 5], dtype=np.int8), CANON)
    for got in (
        O.dequantize_groupwise(O.pack_int4(codes, CANON), scales, out_features=1, in_features=128,
                               group_size=64, packing=CANON, zeros=zeros),
        c_oracle.dequantize_groupwise(O.pack_int4(codes, CANON), scales, zeros, 1, 128, 64),
    ):
        np.testing.assert_array_equal(got[:, :64], np.full((1, 64), -0.25, dtype=np.float32))
        np.testing.assert_array_equal(got[:, 64:], np.full((1, 64), 4.0, dtype=np.float32))


def test_dequant_exhaustive_code_zero_table(c_oracle):
    """Every (code, zero) pair against (c - z) * s evaluated exactly in float64."""
    codes = np.repeat(np.arange(-8, 8), 16).astype(np.int8)          # 256 = one row of K=256
    zero_codes = np.arange(-8, 8).astype(np.int8)                     # 16 rows, one zero per row-group
    n, k = 16, 256
    qcodes = np.tile(codes, n).reshape(n, k)
    rng = np.random.default_rng(7)
    scales = rng.uniform(1e-4, 60.0, size=(n, k // 64)).astype(np.float16)
    zeros_list = np.repeat(zero_codes, k // 64)                       # row r uses zero r in every group
    zeros = O.pack_int4(zeros_list, CANON)
    exact = ((qcodes.astype(np.float64) - np.repeat(zeros_list.reshape(n, -1), 64, axis=1))
             * np.repeat(scales.astype(np.float64), 64, axis=1)).astype(np.float32)
    got_np = O.dequantize_groupwise(O.pack_int4(qcodes, CANON), scales, out_features=n, in_features=k,
                                    group_size=64, packing=CANON, zeros=zeros)
    got_c = c_oracle.dequantize_groupwise(O.pack_int4(qcodes, CANON), scales, zeros, n, k, 64)
    np.testing.assert_array_equal(got_np, exact)
    np.testing.assert_array_equal(got_c, exact)


@pytest.mark.parametrize("shape", [(3, 64), (5, 128), (256, 1536)])
def test_dequant_numpy_and_c_agree_bitwise(shape, c_oracle):
    # shapes of tests/test_triton_unpack.py:59-72 (odd zero counts included)
    rng = np.random.default_rng(shape[0] * 10000 + shape[1])
    weight = rng.standard_normal(shape, dtype=np.float32) * np.float32(0.1)
    qweight, scales, zeros = O.quantize_asymmetric_rtn(weight, group_size=64)
    a = O.dequantize_groupwise(qweight, scales, out_features=shape[0], in_features=shape[1], group_size=64,
                               packing=CANON, zeros=zeros)
    b = c_oracle.dequantize_groupwise(qweight, scales, zeros, shape[0], shape[1], 64)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_dequant_size_checks():
    with pytest.raises(ValueError, match="qweight must contain"):
        O.dequantize_groupwise(np.zeros(63, np.uint8), np.ones((1, 2), np.float16), out_features=1,
                               in_features=128, group_size=64, packing=CANON, zeros=np.zeros(1, np.uint8))
    with pytest.raises(ValueError, match="zeros must contain"):
        O.dequantize_groupwise(np.zeros(64, np.uint8), np.ones((1, 2), np.float16), out_features=1,
                               in_features=128, group_size=64, packing=CANON, zeros=np.zeros(2, np.uint8))
    with pytest.raises(ValueError, match="divisible"):
        O.dequantize_groupwise(np.zeros(48, np.uint8), np.ones((1, 2), np.float16), out_features=1,
                               in_features=96, group_size=64, packing=CANON)


def test_half_and_bfloat16_conversions(c_oracle):
    rng = np.random.default_rng(3)
    values = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(1000.0),
        rng.standard_normal(50000).astype(np.float32) * np.float32(1e-5),      # fp16 subnormal range
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e30, -1e30, np.inf, -np.inf,
                  2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -26, 1.0 + 2.0 ** -11,
                  1.0 + 3 * 2.0 ** -11, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8], dtype=np.float32),
    ])
    # exact ties for fp16 (mantissa bit 12 set, lower bits clear)
    ties = (rng.integers(0x38800000, 0x47000000, size=20000).astype(np.uint32) & ~np.uint32(0xFFF)) | 0x1000
    values = np.concatenate([values, ties.view(np.float32)])
    np.testing.assert_array_equal(c_oracle.f32_to_f16_bits(values), values.astype(np.float16).view(np.uint16))
    bf16_torch = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(c_oracle.f32_to_bf16_bits(values), bf16_torch)
    np.testing.assert_array_equal(O.f32_to_bf16_bits(values), bf16_torch)
    every_half = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = (every_half & 0x7C00) != 0x7C00
    np.testing.assert_array_equal(c_oracle.f16_bits_to_f32(every_half)[finite],
                                  every_half.view(np.float16).astype(np.float32)[finite])
