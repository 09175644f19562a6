"""Pins the oracle's quantizers and linear.

Quantizers (quantization.py:87-162): hand-derived vectors whose expected codes
depend on round-half-even, on using the fp32 (not the fp16) scale for the
codes, on the asymmetric zero/clamp rules and on the zero-list padding; plus
the reference's own properties and a bitwise numpy-vs-C cross-check.

Linear (backends.py:73-150): the reference's exact zero-point boundary case
(tests/test_backends.py:91-104) worked out by hand, one-hot and linearity
properties, double-precision brute force, and the LPU emulation tolerance.
"""

import numpy as np
import pytest

from oracle import oracle as O
from oracle.oracle import PackingFormat

CANON = PackingFormat.CANONICAL


def _both(c_oracle):
    return (O, c_oracle)


def test_symmetric_rtn_ties_round_half_even(c_oracle):
    # amax 7 -> s = 1 exactly; 3.5 -> 4, -3.5 -> -4, 2.5 -> 2, 0.5 -> 0, -2.5 -> -2
    w = np.array([[7.0, 3.5, -3.5, 0.5, 1.5, 2.5, -0.5, -2.5]], dtype=np.float32)
    codes = np.array([7, 4, -4, 0, 2, 2, 0, -2], dtype=np.int8)
    for impl in _both(c_oracle):
        q, s = impl.quantize_symmetric_rtn(w, group_size=8)
        np.testing.assert_array_equal(q.reshape(-1), O.pack_int4(codes))
        assert s.view(np.uint16).tolist() == [[0x3C00]]


def test_symmetric_rtn_codes_use_fp32_scale(c_oracle):
    # amax 1: s32 = 1/7 -> 0.5/s32 = 3.4999998 -> 3 ; with the fp16 scale it would be 3.5009 -> 4.
    w = np.array([[1.0, 0.5, -0.5, 0.0]], dtype=np.float32)
    for impl in _both(c_oracle):
        q, s = impl.quantize_symmetric_rtn(w, group_size=4)
        np.testing.assert_array_equal(impl.unpack_int4(q), np.array([7, 3, -3, 0], dtype=np.int8))
        assert s.view(np.uint16).tolist() == [[0x3092]]   # fp16(1/7) = 0.142822265625


def test_symmetric_rtn_zero_group_gets_unit_scale(c_oracle):
    w = np.zeros((1, 4), dtype=np.float32)
    for impl in _both(c_oracle):
        q, s = impl.quantize_symmetric_rtn(w, group_size=4)
        assert q.reshape(-1).tolist() == [0, 0] and s.astype(np.float32).tolist() == [[1.0]]


def test_symmetric_rtn_self_consistency_and_bounds(c_oracle):
    # tests/test_quantization.py:86-102 plus |w - deq| <= s/2 (+ fp16 scale error)
    w = np.array([[-1.0, -0.75, -0.5, 0.0, 0.25, 0.5, 0.75, 1.0]], dtype=np.float32)
    q, s = O.quantize_symmetric_rtn(w, group_size=4)
    restored = O.dequantize_groupwise(q, s, out_features=1, in_features=8, group_size=4, packing=CANON,
                                      zeros=np.zeros(1, dtype=np.uint8))
    assert q.dtype == np.uint8 and s.shape == (1, 2)
    cos = float(np.dot(w[0], restored[0]) / np.linalg.norm(w) / np.linalg.norm(restored))
    assert cos > 0.99
    rng = np.random.default_rng(11)
    big = rng.standard_normal((64, 256), dtype=np.float32)
    q, s = O.quantize_symmetric_rtn(big, group_size=64)
    codes = O.unpack_int4(q).reshape(64, 256)
    assert codes.min() >= -7 and codes.max() <= 7
    deq = O.dequantize_groupwise(q, s, out_features=64, in_features=256, group_size=64, packing=CANON,
                                 zeros=np.zeros(64 * 4 // 2, np.uint8))
    bound = np.repeat(s.astype(np.float32), 64, axis=1) * 0.5 + np.abs(big) * 2e-3
    assert np.all(np.abs(deq - big) <= bound)


def test_asymmetric_rtn_hand_vector(c_oracle):
    # mn=-3, mx=4: s=7/15, z=round(6.43)=6; codes round(w/s)+6 = [0, 4, 7, 15] -> signed [-8,-4,-1,7]
    w = np.array([[-3.0, -1.0, 0.5, 4.0]], dtype=np.float32)
    for impl in _both(c_oracle):
        q, s, z = impl.quantize_asymmetric_rtn(w, group_size=4)
        assert q.reshape(-1).tolist() == [0xC8, 0x7F]
        assert z.reshape(-1).tolist() == [0x0E]            # z-8 = -2 -> 0xE, padded with a 0 nibble
        assert s.shape == (1, 1)


def test_asymmetric_rtn_ties_and_one_sided_group(c_oracle):
    # range 15 -> s = 1: z = 5; 2.5 -> 2, 3.5 -> 4 (half even): u = [0, 15, 7, 9]
    w = np.array([[-5.0, 10.0, 2.5, 3.5], [1.0, 1.0, 1.0, 1.0]], dtype=np.float32)
    for impl in _both(c_oracle):
        q, s, z = impl.quantize_asymmetric_rtn(w, group_size=4)
        assert q.reshape(-1).tolist() == [0x78, 0x1F, 0x77, 0x77]
        # zeros: row0 z=5 -> -3 (0xD), row1 z=0 -> -8 (0x8): one byte 0x8D
        assert z.reshape(-1).tolist() == [0x8D]
        assert s.view(np.uint16).reshape(-1).tolist() == [0x3C00, 0x2C44]   # 1.0, fp16(1/15)


def test_asymmetric_rtn_clip_max(c_oracle):
    # clip to +-2: mn=-2, mx=2, s=4/15, z=round(7.4999995)=7; u = [0, 14, 14, 14]
    w = np.array([[-5.0, 10.0, 2.5, 3.5]], dtype=np.float32)
    clip = np.array([[2.0]], dtype=np.float32)
    for impl in _both(c_oracle):
        q, s, z = impl.quantize_asymmetric_rtn(w, group_size=4, clip_max=clip)
        assert q.reshape(-1).tolist() == [0x68, 0x66]
        assert z.reshape(-1).tolist() == [0x0F]
    with pytest.raises(ValueError, match="finite and positive"):
        O.quantize_asymmetric_rtn(w, group_size=4, clip_max=np.array([[0.0]], dtype=np.float32))


def test_asymmetric_rtn_round_trip_properties():
    # tests/test_quantization.py:52-83
    weight = np.array([[-3.0, -1.0, 0.5, 4.0, -0.2, 0.0, 0.4, 1.8]], dtype=np.float32)
    q, s, z = O.quantize_asymmetric_rtn(weight, group_size=4)
    restored = O.dequantize_groupwise(q, s, out_features=1, in_features=8, group_size=4, packing=CANON,
                                      zeros=z)
    assert z.shape == (1, 1) and np.count_nonzero(z) > 0
    cos = float(np.dot(weight[0], restored[0]) / np.linalg.norm(weight) / np.linalg.norm(restored))
    assert cos > 0.99
    one_sided = np.array([[1.0, 1.0, 1.0, 1.0]], dtype=np.float32)
    q, s, z = O.quantize_asymmetric_rtn(one_sided, group_size=4)
    restored = O.dequantize_groupwise(q, s, out_features=1, in_features=4, group_size=4, packing=CANON,
                                      zeros=z)
    np.testing.assert_allclose(restored, one_sided, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("packing", list(PackingFormat))
@pytest.mark.parametrize("shape", [(3, 64), (7, 192), (64, 1536)])
def test_quantizers_numpy_and_c_agree_bitwise(shape, packing, c_oracle):
    rng = np.random.default_rng(shape[0] + shape[1])
    w = rng.standard_normal(shape, dtype=np.float32) * np.float32(0.05)
    qa, sa = O.quantize_symmetric_rtn(w, group_size=64, packing=packing)
    qb, sb = c_oracle.quantize_symmetric_rtn(w, group_size=64, packing=packing)
    np.testing.assert_array_equal(qa, qb)
    np.testing.assert_array_equal(sa.view(np.uint16), sb.view(np.uint16))
    clip = np.abs(rng.standard_normal((shape[0], shape[1] // 64)).astype(np.float32)) * np.float32(0.05) + 0.01
    for clip_max in (None, clip):
        qa, sa, za = O.quantize_asymmetric_rtn(w, group_size=64, clip_max=clip_max, packing=packing)
        qb, sb, zb = c_oracle.quantize_asymmetric_rtn(w, group_size=64, clip_max=clip_max, packing=packing)
        np.testing.assert_array_equal(qa, qb)
        np.testing.assert_array_equal(sa.view(np.uint16), sb.view(np.uint16))
        np.testing.assert_array_equal(za, zb)


def test_linear_boundary_zero_points_exact(c_oracle):
    # tests/test_backends.py:91-104, worked out by hand:
    # row0: g0 (z=-8, s=0.25): w=[0, 3.75] -> -3.75/pair; g1 (z=7, s=0.5): w=[-7.5, 0] -> -7.5/pair
    #       32 pairs each: -120 - 240 = -360
    # row1: g0 (z=7, s=1): w=[-15, 0] -> -15/pair; g1 (z=-8, s=2): w=[0, 30] -> -30/pair: -1440
    out_features, in_features = 2, 128
    codes = np.tile(np.array([-8, 7], dtype=np.int8), out_features * in_features // 2)
    qweight = O.pack_int4(codes)
    zeros = O.pack_int4(np.array([-8, 7, 7, -8], dtype=np.int8))
    scales = np.array([[0.25, 0.5], [1.0, 2.0]], dtype=np.float16)
    x = np.tile(np.array([1.0, -1.0], dtype=np.float16), in_features // 2).reshape(1, in_features)
    expected = np.array([[-360.0, -1440.0]], dtype=np.float16)
    got = O.reference_linear(x, qweight, scales, zeros, None, out_features=2, in_features=128, x_dtype="fp16")
    np.testing.assert_array_equal(got, expected)
    lpu = O.lpu_functional_linear(x, qweight, scales, zeros, None, out_features=2, in_features=128,
                                  x_dtype="fp16")
    np.testing.assert_array_equal(lpu, expected)
    w = c_oracle.dequantize_groupwise(qweight, scales, zeros, 2, 128)
    np.testing.assert_array_equal(c_oracle.linear_f32(x.astype(np.float32), w), expected.astype(np.float32))


def test_linear_one_hot_selects_weight_columns_and_bias():
    rng = np.random.default_rng(5)
    qweight, scales, zeros = O.asymmetric_weights(48, 192, seed=5)
    w = O.dequantize_groupwise(qweight, scales, out_features=48, in_features=192, group_size=64,
                               packing=CANON, zeros=zeros)
    bias = O.f32_to_bf16_bits(rng.standard_normal(48).astype(np.float32))
    eye = np.eye(192, dtype=np.float32)[[0, 63, 64, 191]]
    got = O.reference_linear(eye, qweight, scales, zeros, bias, out_features=48, in_features=192,
                             x_dtype="fp32", bias_dtype="bf16")
    expected = w[:, [0, 63, 64, 191]].T + O.bf16_bits_to_f32(bias)[None, :]
    np.testing.assert_array_equal(got, expected.astype(np.float32))
    zero = O.reference_linear(np.zeros((2, 192), np.float16), qweight, scales, zeros, bias, out_features=48,
                              in_features=192, x_dtype="fp16", bias_dtype="bf16")
    np.testing.assert_array_equal(zero, np.tile(O.bf16_bits_to_f32(bias).astype(np.float16), (2, 1)))


def test_linear_matches_double_brute_force_and_linearity(c_oracle):
    rng = np.random.default_rng(9)
    qweight, scales, zeros = O.symmetric_weights(40, 256, seed=9)
    w = c_oracle.dequantize_groupwise(qweight, scales, zeros, 40, 256)
    x1 = rng.standard_normal((3, 256)).astype(np.float32)
    x2 = rng.standard_normal((3, 256)).astype(np.float32)
    exact = x1.astype(np.float64) @ w.T.astype(np.float64)
    got = O.reference_linear(x1, qweight, scales, zeros, None, out_features=40, in_features=256,
                             x_dtype="fp32")
    np.testing.assert_allclose(got, exact, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(c_oracle.linear_f32(x1, w), exact, rtol=1e-6, atol=1e-7)
    lin = O.reference_linear(2 * x1 + x2, qweight, scales, zeros, None, out_features=40, in_features=256,
                             x_dtype="fp32")
    parts = 2 * got + O.reference_linear(x2, qweight, scales, zeros, None, out_features=40,
                                         in_features=256, x_dtype="fp32")
    np.testing.assert_allclose(lin, parts, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("rows", [1, 3, 8])
def test_lpu_emulation_matches_reference_linear(dtype, rows):
    # tests/test_backends.py:47-58 (deterministic weights of :17-22)
    values = np.arange(6 * 128, dtype=np.float32)
    weight = ((np.remainder(values, 31) - 15) / 8).reshape(6, 128).astype(np.float32)
    qweight, scales, zeros = O.quantize_asymmetric_rtn(weight, group_size=64)
    x = O._from_f32(np.linspace(-3, 3, rows * 128, dtype=np.float32).reshape(rows, 128), dtype)
    bias = O.f32_to_bf16_bits(np.linspace(-0.25, 0.25, 6, dtype=np.float32))
    ref = O.reference_linear(x, qweight, scales, zeros, bias, out_features=6, in_features=128, x_dtype=dtype)
    lpu = O.lpu_functional_linear(x, qweight, scales, zeros, bias, out_features=6, in_features=128,
                                  x_dtype=dtype)
    np.testing.assert_allclose(O._to_f32(lpu, dtype), O._to_f32(ref, dtype), rtol=2e-3, atol=2e-3)


def test_tensor_metrics_known_values():
    ref = np.array([1.0, -2.0, 0.0, 4.0], dtype=np.float32)
    got = np.array([1.0, -2.5, 0.0, 4.0], dtype=np.float32)
    m = O.tensor_metrics(ref, got)
    assert m["max_abs"] == 0.5 and m["mean_abs"] == 0.125
    assert abs(m["rmse"] - 0.25) < 1e-7
    assert abs(m["mean_relative"] - 0.0625) < 1e-7
    assert O.tensor_metrics(np.zeros(3), np.zeros(3))["cosine"] == 1.0


def test_synthetic_generators_are_deterministic():
    a = O.symmetric_weights(64, 128, seed=1)
    b = O.symmetric_weights(64, 128, seed=1)
    for u, v in zip(a, b):
        np.testing.assert_array_equal(u, v)
    q, s, z = O.asymmetric_weights(64, 128, seed=2)
    zero_codes = O.unpack_int4(z, elements=64 * 2)
    assert zero_codes.min() >= -4 and zero_codes.max() <= 3            # z in [4, 11] stored as z-8
    assert np.all(s.astype(np.float32) > 0)


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
def test_torch_restatement_matches_numpy_oracle(dtype):
    import torch

    q, s, z = O.asymmetric_weights(72, 320, seed=21)
    x = O.activations(5, 320, seed=22, dtype=dtype)
    bias = O.f32_to_bf16_bits(np.linspace(-1, 1, 72, dtype=np.float32))
    ref = O._to_f32(O.reference_linear(x, q, s, z, bias, out_features=72, in_features=320, x_dtype=dtype), dtype)
    if dtype == "bf16":
        xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    else:
        xt = torch.from_numpy(x)
    bt = torch.from_numpy(bias.view(np.int16)).view(torch.bfloat16)
    got = O.reference_linear_torch(xt, torch.from_numpy(q), torch.from_numpy(s), torch.from_numpy(z), bt,
                                   out_features=72, in_features=320)
    assert got.dtype == xt.dtype
    np.testing.assert_allclose(got.float().numpy(), ref, rtol=1e-2, atol=1e-2)
