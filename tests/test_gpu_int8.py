"""GPU parity of the INT8 K/V update kernel (update_attention_state_int8).

The kernel dequantizes K/V as the reference does (kernels/streaming.py:113-120:
dtype(fp32(k) * fp32(scale))), so on the same inputs it must equal the 16-bit
kernel run on K/V dequantized on the host bit for bit, state and output.
Against the FP32 oracle fed with the same dequantized K/V (oracle
dequantize_int8_groups), the usual tolerances apply.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.seqattn_oracle import chunked_attention, dequantize_int8_groups
from seqattn.kernels import finalize_attention, update_attention_state, update_attention_state_int8
from seqattn.quantization import dequantize_int8_per_token_group, quantize_int8_per_token_group

pytestmark = pytest.mark.gpu


def announce(name: str) -> None:
    print(f"[gpu case] {name}", flush=True)


def quantized_kv(n_k, kv_heads, d, gen, group=64, outliers=True):
    """(K int8, K scales), (V int8, V scales); per-head magnitudes differ and,
    with ``outliers``, 1% of key rows are scaled x8 (a softmax stress; V keeps
    N(0,1)-sized rows so outputs stay O(1))."""
    out = []
    for tensor in range(2):
        x = torch.randn((n_k, kv_heads, d), generator=gen) * (0.5 + torch.rand((1, kv_heads, 1), generator=gen))
        if outliers and tensor == 0:
            idx = torch.randperm(n_k, generator=gen)[: max(1, n_k // 100)]
            x[idx] *= 8
        q = torch.empty((n_k, kv_heads, d), dtype=torch.int8)
        s = torch.empty((math.ceil(n_k / group), kv_heads), dtype=torch.float16)
        quantize_int8_per_token_group(x, q, s, group_tokens=group)
        out.append((q, s))
    return out


def run_chunks(q, k, v, chunks, *, causal, causal_shift, int8_scales=None, group=64):
    """Apply K/V in ``chunks`` [(start, stop)] to a fresh state; returns (out, lse, m, l, acc)."""
    n_q, heads, d = q.shape
    m = torch.empty((n_q, heads), device="cuda")
    l = torch.empty_like(m)
    acc = torch.empty((n_q, heads, d), device="cuda")
    for i, (s, e) in enumerate(chunks):
        common = dict(q_tokens=n_q, kv_tokens=e - s, q_local_offset=0, kv_local_offset=s,
                      causal_shift=causal_shift, softmax_scale=d**-0.5, causal=causal, initialize=i == 0)
        if int8_scales is None:
            update_attention_state(q, k[s:e], v[s:e], m, l, acc, **common)
        else:
            ks, vs = int8_scales
            update_attention_state_int8(q, k[s:e], v[s:e], ks, vs, m, l, acc, storage_token_offset=s,
                                        quant_group_tokens=group, **common)
    out = torch.empty((n_q, heads, d), dtype=q.dtype, device="cuda")
    lse = torch.empty((heads, n_q), device="cuda")
    finalize_attention(acc, l, out, q_tokens=n_q, running_max=m, lse=lse)
    torch.cuda.synchronize()
    return out, lse, m, l, acc


CASES = [
    # head_dim, q_heads, kv_heads, dtype, causal
    (16, 4, 4, torch.bfloat16, False),
    (32, 4, 2, torch.float16, True),
    (48, 2, 1, torch.bfloat16, False),
    (64, 8, 2, torch.bfloat16, True),
    (80, 4, 2, torch.bfloat16, True),
    (96, 2, 2, torch.float16, False),
    (112, 6, 3, torch.float16, False),
    (128, 8, 4, torch.bfloat16, False),
    (128, 4, 4, torch.bfloat16, True),
]


@pytest.mark.parametrize("d,hq,hkv,dtype,causal", CASES)
def test_int8_kernel_equals_16bit_kernel_on_dequantized_kv(d, hq, hkv, dtype, causal):
    announce(f"int8 vs 16-bit d={d} hq={hq} hkv={hkv} {dtype} causal={causal}")
    gen = torch.Generator().manual_seed(1000 + d + hq)
    n_q, n_k = 700, 1000
    q = torch.randn((n_q, hq, d), generator=gen).to(dtype).cuda()
    (kq, ks), (vq, vs) = quantized_kv(n_k, hkv, d, gen)
    k_deq = dequantize_int8_per_token_group(kq, ks, dtype=dtype).cuda()
    v_deq = dequantize_int8_per_token_group(vq, vs, dtype=dtype).cuda()
    # Chunk starts that are not multiples of the 64-token scale group.
    chunks = [(0, 333), (333, 700), (700, 1000)]
    ref = run_chunks(q, k_deq, v_deq, chunks, causal=causal, causal_shift=n_k - n_q)
    got = run_chunks(q, kq.cuda(), vq.cuda(), chunks, causal=causal, causal_shift=n_k - n_q,
                     int8_scales=(ks.cuda(), vs.cuda()))
    for name, a, b in zip(("out", "lse", "m", "l", "acc"), got, ref):
        assert torch.equal(a, b), name


def test_int8_per_token_scales_and_oracle_parity():
    """Scale group of one token (the paged runtime's per-row scales) and the
    FP32 oracle on the oracle's own dequantization of the same bytes."""
    announce("int8 per-token scales + oracle")
    gen = torch.Generator().manual_seed(77)
    n_q, n_k, hq, hkv, d = 1000, 1500, 8, 2, 128
    q = torch.randn((n_q, hq, d), generator=gen).to(torch.bfloat16)
    (kq, ks), (vq, vs) = quantized_kv(n_k, hkv, d, gen, group=64)
    # Expand the 64-token groups to one scale per token.
    ks_tok = ks.repeat_interleave(64, dim=0)[:n_k].contiguous()
    vs_tok = vs.repeat_interleave(64, dim=0)[:n_k].contiguous()
    chunks = [(0, 512), (512, 1100), (1100, 1500)]
    qd = q.cuda()
    grouped = run_chunks(qd, kq.cuda(), vq.cuda(), chunks, causal=True, causal_shift=n_k - n_q,
                         int8_scales=(ks.cuda(), vs.cuda()))
    per_token = run_chunks(qd, kq.cuda(), vq.cuda(), chunks, causal=True, causal_shift=n_k - n_q,
                           int8_scales=(ks_tok.cuda(), vs_tok.cuda()), group=1)
    for a, b in zip(grouped, per_token):
        assert torch.equal(a, b)
    k_bits = dequantize_int8_groups(kq.numpy(), ks.numpy())
    v_bits = dequantize_int8_groups(vq.numpy(), vs.numpy())
    q_bits = q.view(torch.int16).numpy().view(np.uint16)
    ref_o, ref_l = chunked_attention(q_bits, k_bits, v_bits, [0, n_q], [0, n_k], q_chunk_tokens=n_q,
                                     kv_chunk_tokens=512, causal=True)
    out, lse = grouped[0].float().cpu().numpy(), grouped[1].cpu().numpy()
    diff = np.abs(out - ref_o)
    rel_l2 = float(np.linalg.norm(diff) / np.linalg.norm(ref_o))
    rms = float(np.sqrt(np.mean(np.square(ref_o, dtype=np.float64))))
    scaled = float((diff / (np.abs(ref_o) + rms)).max())
    print(f"  max|dO| {diff.max():.3e} relL2 {rel_l2:.3e} scaled {scaled:.3e} "
          f"max|dLSE| {np.abs(lse - ref_l).max():.3e}", flush=True)
    # 2e-2 absolute for O(1) outputs; a bf16 output of magnitude above 1
    # carries a relative rounding, so the bound grows with |ref| there (the
    # K outliers make some rows attend to a single V row of magnitude ~4).
    assert (diff <= 2e-2 * np.maximum(1.0, np.abs(ref_o))).all()
    assert rel_l2 <= 5e-3 and scaled <= 2.0**-5
    assert np.abs(lse - ref_l).max() <= 1e-3

