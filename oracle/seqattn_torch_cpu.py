"""The reference's CPU chunked attention restated with torch on the CPU.
TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and the ``cpu_baseline`` leg of ``bench.py`` may use this
module, never as the thing that is measured on the GPU or shipped; the
product package (``stream-attn_amd/seqattn``) never imports it.

``chunked_attention_torch`` follows streaming_attention_reference (reference
src/seqattn_core/reference.py:11-117) step for step with torch.matmul on
float32 CPU tensors, which is how the reference's own CPU path computes: it
is the CPU baseline's timed loop, run on torch's intra-op threads.  Parity
pin: tests/test_oracle.py checks it against the numpy oracle
(``oracle.seqattn_oracle.chunked_attention``) on GQA, causal, multi-segment
and empty-segment cases.
"""

from __future__ import annotations

import torch


@torch.inference_mode()
def chunked_attention_torch(q, k, v, cu_q, cu_k, *, q_chunk_tokens: int, kv_chunk_tokens: int,
                            softmax_scale: float | None = None, causal: bool = False,
                            head_batch: int | None = None):
    """FP32 online-softmax attention on the CPU; returns (O [T, H, D] fp32,
    LSE [H, T] fp32), the numpy oracle's contract.

    Per segment (reference.py:44), per Q tile of q_chunk_tokens (L50), state
    m = -inf, l = 0, o = 0 (L53-61); per K/V tile of kv_chunk_tokens (L68):
    GQA by repeating K/V heads (L73-75), s = q k^T * scale (L78), the
    bottom-right causal mask k_pos <= q_pos + (Lk - Lq) (L79-88), m' =
    max(m, rowmax s), alpha = exp(m - m') where m' is finite else 1, p =
    exp(s - m') where s is finite else 0, l = l alpha + sum p, o = o alpha +
    p v (L90-107); out = o / l where l > 0 else 0 (L109-113).  LSE is m +
    ln(l), -inf where l == 0.  ``head_batch`` query heads go through one
    batched matmul at a time (all of them by default).
    """
    q = torch.as_tensor(q)
    k = torch.as_tensor(k)
    v = torch.as_tensor(v)
    tokens, heads, head_dim = q.shape
    group = heads // k.shape[1]
    scale = head_dim**-0.5 if softmax_scale is None else float(softmax_scale)
    batch = heads if head_batch is None else max(1, int(head_batch))
    cu_q = [int(x) for x in cu_q]
    cu_k = [int(x) for x in cu_k]
    out = torch.zeros((tokens, heads, head_dim), dtype=torch.float32)
    lse = torch.full((heads, tokens), float("-inf"), dtype=torch.float32)
    for q_start, q_stop, k_start, k_stop in zip(cu_q[:-1], cu_q[1:], cu_k[:-1], cu_k[1:]):
        shift = (k_stop - k_start) - (q_stop - q_start)
        for t0 in range(q_start, q_stop, q_chunk_tokens):
            t1 = min(t0 + q_chunk_tokens, q_stop)
            q_pos = torch.arange(t0 - q_start, t1 - q_start)
            qt = q[t0:t1].float().transpose(0, 1)  # [H, n, D]
            m = torch.full((heads, t1 - t0), float("-inf"))
            l = torch.zeros((heads, t1 - t0))
            o = torch.zeros((heads, t1 - t0, head_dim))
            for c0 in range(k_start, k_stop, kv_chunk_tokens):
                c1 = min(c0 + kv_chunk_tokens, k_stop)
                kc = k[c0:c1].float()
                vc = v[c0:c1].float()
                if group != 1:
                    kc = kc.repeat_interleave(group, dim=1)
                    vc = vc.repeat_interleave(group, dim=1)
                kc = kc.transpose(0, 1)  # [H, n_k, D]
                vc = vc.transpose(0, 1)
                mask = None
                if causal:
                    k_pos = torch.arange(c0 - k_start, c1 - k_start)
                    mask = k_pos[None, :] > (q_pos[:, None] + shift)
                for h0 in range(0, heads, batch):
                    h1 = min(h0 + batch, heads)
                    s = torch.matmul(qt[h0:h1], kc[h0:h1].transpose(1, 2)) * scale
                    if mask is not None:
                        s = s.masked_fill(mask, float("-inf"))
                    m_h = m[h0:h1]
                    merged = torch.maximum(m_h, s.amax(dim=-1))
                    finite = torch.isfinite(merged)
                    alpha = torch.where(finite, torch.exp(m_h - merged), torch.ones_like(m_h))
                    p = torch.exp(s - merged[..., None])
                    if mask is not None:
                        p = torch.where(torch.isfinite(s), p, torch.zeros_like(p))
                    l[h0:h1] = l[h0:h1] * alpha + p.sum(dim=-1)
                    o[h0:h1] = o[h0:h1] * alpha[..., None] + torch.matmul(p, vc[h0:h1])
                    m[h0:h1] = torch.where(finite, merged, m_h)
            positive = l > 0
            safe = torch.where(positive, l, torch.ones_like(l))
            out[t0:t1] = torch.where(positive[..., None], o / safe[..., None], torch.zeros_like(o)).transpose(0, 1)
            lse[:, t0:t1] = torch.where(positive, m + torch.log(safe), torch.full_like(m, float("-inf")))
    return out, lse
