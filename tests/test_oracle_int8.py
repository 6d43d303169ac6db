"""Pins of the oracle's INT8 K/V storage restatement (quantize, dequantize and
bfloat16 rounding) and the product's CPU quantizer against it.  CPU only."""

from __future__ import annotations

import numpy as np
import torch

from oracle.seqattn_oracle import dequantize_int8_groups, quantize_int8_groups, round_f32_to_bf16_bits
from seqattn.quantization import dequantize_int8_per_token_group, quantize_int8_per_token_group


def test_bf16_rounding_matches_torch_including_ties():
    rng = np.random.default_rng(0)
    values = np.concatenate([
        rng.standard_normal(4096).astype(np.float32) * 10.0 ** rng.integers(-6, 6, 4096),
        # Exact ties between two bf16 neighbours: low 16 bits 0x8000.
        (np.arange(1, 200, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
        np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 3.0e38, 1e-40], dtype=np.float32),
    ])
    expected = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(round_f32_to_bf16_bits(values), expected)
    assert round_f32_to_bf16_bits(np.array([np.nan], np.float32))[0] & 0x7F80 == 0x7F80


def test_quantize_known_answers():
    # amax 127 -> step 1: integer values come back unchanged; ties round to even.
    x = np.zeros((4, 1, 8), dtype=np.float32)
    x[0, 0] = [127, -127, 3, -5, 0, 1, 2, 100]
    x[1, 0] = [0.5, 1.5, 2.5, -0.5, -1.5, 126.5, -2.5, 3.5]
    q, scales = quantize_int8_groups(x, group_tokens=64)
    assert scales.shape == (1, 1) and scales[0, 0] == np.float16(1.0)
    assert q[0, 0].tolist() == [127, -127, 3, -5, 0, 1, 2, 100]
    assert q[1, 0].tolist() == [0, 2, 2, 0, -2, 126, -2, 4]
    # All-zero group: step 1, zeros.
    q0, s0 = quantize_int8_groups(np.zeros((3, 2, 16), np.float32))
    assert (q0 == 0).all() and (s0 == np.float16(1.0)).all()
    # amax 1: step = float32(1/127), stored as float16; +-1 map to +-127.
    ones = np.ones((2, 1, 16), np.float32)
    ones[1] = -1
    q1, s1 = quantize_int8_groups(ones)
    assert s1[0, 0] == np.float16(np.float32(1.0) / np.float32(127.0))
    assert q1[0].min() == 127 and q1[1].max() == -127
    # Groups are per 64 tokens and per head: 130 tokens -> 3 groups, the last partial.
    rng = np.random.default_rng(1)
    y = rng.standard_normal((130, 3, 16)).astype(np.float32)
    y[129, 2, 0] = 50.0
    qy, sy = quantize_int8_groups(y)
    assert sy.shape == (3, 3)
    assert sy[2, 2] == np.float16(np.float32(50.0) / np.float32(127.0))
    assert qy[129, 2, 0] == 127


def test_quantize_reconstruction_bound():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((300, 4, 32)) * rng.uniform(0.01, 30, (1, 4, 1))).astype(np.float32)
    q, scales = quantize_int8_groups(x)
    for g in range(scales.shape[0]):
        rows = slice(64 * g, min(64 * g + 64, x.shape[0]))
        block = x[rows].astype(np.float64)
        step32 = (np.abs(x[rows]).max(axis=(0, 2)) / np.float32(127)).astype(np.float64)
        stored = scales[g].astype(np.float64)
        recon = q[rows].astype(np.float64) * stored[None, :, None]
        bound = step32 / 2 * 1.0001 + 127 * np.abs(stored - step32)
        assert (np.abs(block - recon) <= bound[None, :, None]).all()


def test_dequantize_offset_rule_and_rounding():
    rng = np.random.default_rng(3)
    q = rng.integers(-127, 128, (200, 2, 16), dtype=np.int8)
    scales = rng.uniform(0.001, 0.2, (4, 2)).astype(np.float16)
    full = dequantize_int8_groups(q, scales)
    assert np.array_equal(dequantize_int8_groups(q[10:], scales, token_offset=10), full[10:])
    # Brute force: one float32 product, then bfloat16 round-to-nearest-even.
    for j, h, d in [(0, 0, 0), (63, 1, 5), (64, 0, 15), (199, 1, 7)]:
        product = np.float32(q[j, h, d]) * np.float32(scales[j // 64, h])
        assert full[j, h, d] == round_f32_to_bf16_bits(np.array([product]))[0]
    # The product's torch dequantizer forms the same bits.
    torch_bits = dequantize_int8_per_token_group(
        torch.from_numpy(q), torch.from_numpy(scales), dtype=torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(torch_bits, full)


def test_product_quantizer_matches_the_oracle_bit_for_bit():
    gen = torch.Generator().manual_seed(4)
    for dtype in (torch.bfloat16, torch.float16, torch.float32):
        x = torch.randn((333, 3, 64), generator=gen) * torch.rand((1, 3, 1), generator=gen) * 5
        x[17, 1, :] *= 40  # an outlier row sets one group's scale
        x[128:192, 2] = 0  # an all-zero group
        x = x.to(dtype)
        groups = -(-x.shape[0] // 64)
        q = torch.empty(x.shape, dtype=torch.int8)
        s = torch.empty((groups, 3), dtype=torch.float16)
        quantize_int8_per_token_group(x, q, s, group_tokens=64)
        xin = x.view(torch.int16).numpy().view(np.uint16) if dtype == torch.bfloat16 else x.float().numpy()
        q_ref, s_ref = quantize_int8_groups(xin)
        assert np.array_equal(q.numpy(), q_ref), dtype
        assert np.array_equal(s.numpy(), s_ref), dtype
