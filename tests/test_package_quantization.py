"""The package's torch quantization API (mirror of src/qwen_int4/quantization.py)
against the oracle, bit for bit, plus the reference's own known answers
(tests/test_quantization.py:15-49, tests/test_phase_e_correctness.py:100-123).
The CPU cases run everywhere; the device cases check that running on the GPU
gives the same bits."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from qwen_int4_hip import quantization as Q

PACKINGS = [Q.PackingFormat.CANONICAL, Q.PackingFormat.LEGACY_SIGNED_ADD]


def test_known_answers_match_reference_tests():
    assert Q.pack_int4(torch.tensor([-1, 2])).tolist() == [0x2F]
    assert Q.pack_int4(torch.tensor([-8, -1, 0, 7])).tolist() == [0xF8, 0x70]
    codes = torch.tensor([-7, -6, -1, 0, 1, 6, 7, -3], dtype=torch.int8)
    for packing in PACKINGS:
        assert torch.equal(Q.unpack_int4(Q.pack_int4(codes, packing=packing), packing=packing), codes)
    # group-scale indexing (tests/test_quantization.py:35-49)
    packed = Q.pack_int4(torch.tensor([1, 2, 3, 4, -1, -2, -3, -4]), packing="canonical")
    got = Q.dequantize_groupwise(packed, torch.tensor([[0.5, 2.0], [1.0, 0.25]], dtype=torch.float16),
                                 out_features=2, in_features=4, group_size=2, packing="canonical")
    assert got.tolist() == [[0.5, 1.0, 6.0, 8.0], [-1.0, -2.0, -0.75, -1.0]]
    # each group's zero and scale (tests/test_phase_e_correctness.py:109-119)
    codes = torch.tensor([[-8] * 64 + [7] * 64], dtype=torch.int8)
    zeros = Q.pack_int4(torch.tensor([-7, 5], dtype=torch.int8))
    got = Q.dequantize_groupwise(Q.pack_int4(codes), torch.tensor([[0.25, 2.0]], dtype=torch.float16),
                                 out_features=1, in_features=128, group_size=64, packing="canonical", zeros=zeros)
    assert got[0, :64].eq(-0.25).all() and got[0, 64:].eq(4.0).all()
    # the legacy borrow (tests/test_quantization.py:28-31, tests/test_phase_e_correctness.py:121-123)
    packed = Q.pack_int4(torch.tensor([3, -2], dtype=torch.int8), packing=Q.PackingFormat.LEGACY_SIGNED_ADD)
    assert Q.unpack_int4(packed, packing="canonical").tolist() == [-2, 2]
    assert Q.unpack_int4(packed, packing=Q.PackingFormat.LEGACY_SIGNED_ADD).tolist() == [3, -2]


def test_validation_messages_match_reference():
    with pytest.raises(ValueError, match="even number"):
        Q.pack_int4(torch.tensor([1, 2, 3]))
    with pytest.raises(ValueError, match=r"\[-8, 7\]"):
        Q.pack_int4(torch.tensor([8, 0]))
    with pytest.raises(ValueError, match="invalid element count"):
        Q.unpack_int4(torch.tensor([1], dtype=torch.uint8), elements=3)
    with pytest.raises(ValueError, match="divisible"):
        Q.quantize_symmetric_rtn(torch.zeros(2, 65), group_size=64)
    with pytest.raises(ValueError, match="2D"):
        Q.quantize_asymmetric_rtn(torch.zeros(64), group_size=64)
    with pytest.raises(ValueError, match="clip_max"):
        Q.quantize_asymmetric_rtn(torch.zeros(2, 64), group_size=64, clip_max=torch.ones(3, 1))
    with pytest.raises(ValueError, match="qweight must contain"):
        Q.dequantize_groupwise(torch.zeros(3, dtype=torch.uint8), torch.ones(2, 1, dtype=torch.float16),
                               out_features=2, in_features=4, group_size=4)


@pytest.mark.parametrize("packing", PACKINGS)
def test_codec_matches_oracle_exhaustively(packing):
    all_bytes = np.arange(256, dtype=np.uint8)
    got = Q.unpack_int4(torch.from_numpy(all_bytes), packing=packing).numpy()
    np.testing.assert_array_equal(got, O.unpack_int4(all_bytes, packing))
    rng = np.random.default_rng(O.BASE_SEED)
    codes = rng.integers(-8, 8, size=4097 * 2, dtype=np.int8)
    np.testing.assert_array_equal(Q.pack_int4(torch.from_numpy(codes), packing=packing).numpy(),
                                  O.pack_int4(codes, packing))


def _weights(n, k, seed, scale=0.02):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(scale)).astype(np.float32)
    w[0, :64] = 0.0  # an all-zero group (scale 1)
    w[1, 64:128] = np.linspace(-3.5, 3.5, 64, dtype=np.float32)  # exact half-way codes
    return w


@pytest.mark.parametrize(("n", "k", "g"), [(6, 128, 64), (96, 1536, 64), (7, 192, 64), (5, 256, 128)])
def test_quantizers_match_oracle_bitwise(n, k, g):
    w = _weights(n, k, n * k)
    q, s = Q.quantize_symmetric_rtn(torch.from_numpy(w), group_size=g)
    oq, os_ = O.quantize_symmetric_rtn(w, g)
    np.testing.assert_array_equal(q.numpy(), oq)
    np.testing.assert_array_equal(s.numpy().view(np.uint16), os_.view(np.uint16))
    clip = np.abs(w.reshape(n, k // g, g)).max(axis=-1).astype(np.float32) * np.float32(0.8) + np.float32(1e-3)
    for limit in (None, clip):
        q, s, z = Q.quantize_asymmetric_rtn(torch.from_numpy(w), group_size=g,
                                            clip_max=None if limit is None else torch.from_numpy(limit))
        oq, os_, oz = O.quantize_asymmetric_rtn(w, g, limit)
        np.testing.assert_array_equal(q.numpy(), oq)
        np.testing.assert_array_equal(s.numpy().view(np.uint16), os_.view(np.uint16))
        np.testing.assert_array_equal(z.numpy(), oz)
        deq = Q.dequantize_groupwise(q, s, out_features=n, in_features=k, group_size=g, packing="canonical", zeros=z)
        ref = O.dequantize_groupwise(oq, os_, out_features=n, in_features=k, group_size=g, packing="canonical",
                                     zeros=oz)
        np.testing.assert_array_equal(deq.numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")
def test_quantizers_on_device_match_cpu_bitwise():
    w = torch.from_numpy(_weights(1536, 1536, 11))
    for fn in (Q.quantize_symmetric_rtn, Q.quantize_asymmetric_rtn):
        cpu = fn(w, group_size=64)
        gpu = fn(w.cuda(), group_size=64)
        for a, b in zip(cpu, gpu):
            assert torch.equal(a, b.cpu())
    q, s, z = Q.quantize_asymmetric_rtn(w, group_size=64)
    cpu = Q.dequantize_groupwise(q, s, out_features=1536, in_features=1536, group_size=64, packing="canonical",
                                 zeros=z)
    gpu = Q.dequantize_groupwise(q.cuda(), s.cuda(), out_features=1536, in_features=1536, group_size=64,
                                 packing="canonical", zeros=z.cuda())
    assert torch.equal(cpu, gpu.cpu())
