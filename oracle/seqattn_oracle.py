"""CPU oracle of the streamed exact-attention path.  TEST INFRASTRUCTURE ONLY.

This module is the reference the GPU path is checked against: only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and never as the thing that is measured or shipped.  The product
package (``stream-attn_amd/seqattn``) never imports it.

Every function is a numpy restatement of the reference algorithm; each cites
the reference file:line it follows.  Parity pins (see tests/test_oracle.py):

* ``chunked_attention`` (O and LSE) against a dense float64 closed form
  ``softmax(QK^T s)V`` / ``logsumexp(QK^T s)``, against the reference test's
  known answers (segment isolation 0 / 10, "queries but no keys"), against a
  brute-force per-row float64 loop on tiny inputs, and across chunk sizes
  (chunking must not change the result beyond fp32 rounding).
* ``chunked_attention_rows`` equals ``chunked_attention`` on the same rows.
* ``quantize_int8_groups`` / ``dequantize_int8_groups`` /
  ``round_f32_to_bf16_bits`` against hand-worked known answers (exact
  integer groups, all-zero groups, ties rounding to even, clamping, the
  float16 scale), the reconstruction bound |x - deq| <= step / 2 (+ scale
  rounding), torch's own bfloat16 conversion, and the group offset rule.
* ``seeded_normal_chunks`` reproduces torch's generator stream exactly (it
  calls torch's CPU generator, the same calls the reference's benchmark
  makes) and is checked element-for-element against a direct torch call.
"""

from __future__ import annotations

import math

import numpy as np


def segment_bounds(cu: np.ndarray | list[int], total: int, name: str) -> list[int]:
    """Validated cumulative bounds (reference src/seqattn_core/validation.py:18-26)."""
    bounds = [int(x) for x in np.asarray(cu).reshape(-1).tolist()]
    if len(bounds) < 2:
        raise ValueError(f"{name} must be a one-dimensional CPU tensor")
    if bounds[0] != 0 or bounds[-1] != total:
        raise ValueError(f"{name} must span [0, {total}], got {bounds}")
    if any(b < a for a, b in zip(bounds[:-1], bounds[1:])):
        raise ValueError(f"{name} must be non-decreasing")
    return bounds


def as_f32(x: np.ndarray) -> np.ndarray:
    """float32 view of an input: uint16 arrays hold bfloat16 bit patterns
    (numpy has no bfloat16), which widen exactly by a 16-bit shift."""
    if x.dtype == np.uint16:
        return (x.astype(np.uint32) << 16).view(np.float32)
    return x.astype(np.float32, copy=False)


def _validate(q, k, v, cu_q, cu_k):
    """Shape/segment checks of reference validation.py:6-47."""
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError("q, k, and v must use packed [tokens, heads, head_dim] layout")
    if k.shape != v.shape:
        raise ValueError("k and v must have identical shapes")
    if q.shape[2] != k.shape[2]:
        raise ValueError("q and k/v must use the same head_dim")
    if q.shape[1] % k.shape[1]:
        raise ValueError("the number of query heads must be divisible by the number of KV heads")
    qb = segment_bounds(cu_q, q.shape[0], "cu_seqlens_q")
    kb = segment_bounds(cu_k, k.shape[0], "cu_seqlens_k")
    if len(qb) != len(kb):
        raise ValueError("cu_seqlens_q and cu_seqlens_k must describe the same batch size")
    for i in range(len(qb) - 1):
        if qb[i + 1] > qb[i] and kb[i + 1] == kb[i]:
            raise ValueError(f"sequence {i} has queries but no keys")
    return qb, kb


def _attend_heads(q_tile, k, v, kv_range, group, k_start, k_stop, kv_chunk, scale, causal,
                  q_pos, causal_shift):
    """Online-softmax recurrence of one Q tile over one segment's K/V for the
    K/V heads in kv_range and their query heads (reference reference.py:53-107)."""
    a, b = kv_range
    qt = np.ascontiguousarray(as_f32(q_tile[:, a * group : b * group]).transpose(1, 0, 2))  # [h, n, D]
    heads, n, head_dim = qt.shape
    m = np.full((heads, n), -np.inf, dtype=np.float32)
    l = np.zeros((heads, n), dtype=np.float32)
    o = np.zeros((heads, n, head_dim), dtype=np.float32)
    for kv_start in range(k_start, k_stop, kv_chunk):
        kv_stop = min(kv_start + kv_chunk, k_stop)
        kt = as_f32(k[kv_start:kv_stop, a:b])
        vt = as_f32(v[kv_start:kv_stop, a:b])
        if group != 1:
            kt = np.repeat(kt, group, axis=1)
            vt = np.repeat(vt, group, axis=1)
        kt = np.ascontiguousarray(kt.transpose(1, 0, 2))  # [h, n_k, D]
        vt = np.ascontiguousarray(vt.transpose(1, 0, 2))
        s = np.matmul(qt, kt.transpose(0, 2, 1))
        s *= np.float32(scale)
        if causal:
            k_pos = np.arange(kv_start - k_start, kv_stop - k_start)
            visible = k_pos[None, :] <= (q_pos[:, None] + causal_shift)
            s = np.where(visible[None], s, -np.inf).astype(np.float32)
        tile_max = s.max(axis=-1)
        merged = np.maximum(m, tile_max)
        finite = np.isfinite(merged)
        with np.errstate(invalid="ignore"):
            alpha = np.where(finite, np.exp(m - merged), np.float32(1.0)).astype(np.float32)
            if causal:
                p = np.where(np.isfinite(s), np.exp(s - merged[..., None]), np.float32(0.0))
                p = p.astype(np.float32)
            else:
                # Without a mask every logit is finite: p = exp(s - m') in place.
                p = s
                p -= merged[..., None]
                np.exp(p, out=p)
        l = l * alpha + p.sum(axis=-1, dtype=np.float32)
        o = o * alpha[..., None] + np.matmul(p, vt)
        m = np.where(finite, merged, m)
    return m, l, o


def chunked_attention(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    cu_q,
    cu_k,
    *,
    q_chunk_tokens: int,
    kv_chunk_tokens: int,
    softmax_scale: float | None = None,
    causal: bool = False,
    rows: np.ndarray | None = None,
    workers: int = 1,
) -> tuple[np.ndarray, np.ndarray]:
    """FP32 online-softmax attention; returns (O [T, H, D] fp32, LSE [H, T] fp32).

    Follows streaming_attention_reference (reference src/seqattn_core/reference.py:11-117):
    per segment (L44), per Q tile of q_chunk_tokens (L50), state m=-inf, l=0,
    o=0 (L53-61); per K/V tile of kv_chunk_tokens (L68): GQA by repeating K/V
    heads (L73-75), s = q k^T * scale (L78), bottom-right causal mask
    k_pos <= q_pos + (Lk - Lq) (L79-88), m' = max(m, rowmax s), alpha =
    exp(m - m') where m' is finite else 1, p = exp(s - m') where s is finite
    else 0, l = l*alpha + sum p, o = o*alpha + p v (L90-107); out = o / l
    where l > 0 else 0 (L109-113).  LSE (absent from the reference) is
    m + ln(l), -inf where l == 0.

    ``rows`` (optional, sorted global query indices) restricts the work to
    those query rows: each Q tile is intersected with them, which leaves the
    per-row recurrence unchanged.  Returned arrays are full-size; rows not
    computed are NaN.  ``workers > 1`` splits the K/V heads over threads
    (numpy releases the GIL in its kernels); each head's arithmetic is the
    same as with one worker.
    """
    q = np.asarray(q)
    k = np.asarray(k)
    v = np.asarray(v)
    qb, kb = _validate(q, k, v, cu_q, cu_k)
    if q_chunk_tokens <= 0 or kv_chunk_tokens <= 0:
        raise ValueError("q_chunk_tokens and kv_chunk_tokens must be positive")
    tokens, heads, head_dim = q.shape
    group = heads // k.shape[1]
    scale = head_dim**-0.5 if softmax_scale is None else float(softmax_scale)
    out = np.full((tokens, heads, head_dim), np.nan, dtype=np.float32)
    lse = np.full((heads, tokens), np.nan, dtype=np.float32)
    row_mask = None
    if rows is not None:
        row_mask = np.zeros(tokens, dtype=bool)
        row_mask[np.asarray(rows, dtype=np.int64)] = True

    for q_start, q_stop, k_start, k_stop in zip(qb[:-1], qb[1:], kb[:-1], kb[1:]):
        causal_shift = (k_stop - k_start) - (q_stop - q_start)
        for tile_start in range(q_start, q_stop, q_chunk_tokens):
            tile_stop = min(tile_start + q_chunk_tokens, q_stop)
            idx = np.arange(tile_start, tile_stop)
            if row_mask is not None:
                idx = idx[row_mask[tile_start:tile_stop]]
                if idx.size == 0:
                    continue
            q_pos = idx - q_start
            q_tile = q[idx]
            kv_heads = k.shape[1]
            if workers > 1 and kv_heads > 1:
                from concurrent.futures import ThreadPoolExecutor

                groups = np.array_split(np.arange(kv_heads), min(workers, kv_heads))
                jobs = [(int(g[0]), int(g[-1]) + 1) for g in groups if g.size]
                with ThreadPoolExecutor(max_workers=len(jobs)) as pool:
                    parts = list(pool.map(
                        lambda job: _attend_heads(
                            q_tile, k, v, job, group, k_start, k_stop, kv_chunk_tokens, scale, causal,
                            q_pos, causal_shift),
                        jobs))
                m = np.concatenate([p[0] for p in parts])
                l = np.concatenate([p[1] for p in parts])
                o = np.concatenate([p[2] for p in parts])
            else:
                m, l, o = _attend_heads(q_tile, k, v, (0, kv_heads), group, k_start, k_stop,
                                        kv_chunk_tokens, scale, causal, q_pos, causal_shift)
            positive = l > 0
            with np.errstate(divide="ignore", invalid="ignore"):
                normalized = np.where(positive[..., None], o / l[..., None], np.float32(0.0))
                lse_tile = np.where(positive, m + np.log(l), -np.inf)
            out[idx] = normalized.transpose(1, 0, 2)
            lse[:, idx] = lse_tile
    return out, lse


def dense_attention_f64(q, k, v, cu_q, cu_k, *, softmax_scale=None, causal=False, rows=None):
    """Closed form softmax(QK^T s)V and logsumexp(QK^T s) in float64.

    The oracle's pin: an independent, unchunked computation of the same
    quantity (reference tests/test_reference.py:13-38 uses the same closed
    form to pin its chunked reference).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    qb, kb = _validate(q, k, v, cu_q, cu_k)
    tokens, heads, head_dim = q.shape
    group = heads // k.shape[1]
    scale = head_dim**-0.5 if softmax_scale is None else float(softmax_scale)
    out = np.full((tokens, heads, head_dim), np.nan)
    lse = np.full((heads, tokens), np.nan)
    selected = None if rows is None else set(int(r) for r in rows)
    for qs, qe, ks, ke in zip(qb[:-1], qb[1:], kb[:-1], kb[1:]):
        idx = np.arange(qs, qe)
        if selected is not None:
            idx = np.array([i for i in idx if i in selected], dtype=np.int64)
        if idx.size == 0:
            continue
        kk = np.repeat(k[ks:ke], group, axis=1).transpose(1, 0, 2)
        vv = np.repeat(v[ks:ke], group, axis=1).transpose(1, 0, 2)
        s = np.matmul(q[idx].transpose(1, 0, 2), kk.transpose(0, 2, 1)) * scale
        if causal:
            shift = (ke - ks) - (qe - qs)
            visible = np.arange(ke - ks)[None, :] <= (idx - qs)[:, None] + shift
            s = np.where(visible[None], s, -np.inf)
        mx = s.max(axis=-1, keepdims=True)
        safe = np.where(np.isfinite(mx), mx, 0.0)
        e = np.exp(s - safe)
        total = e.sum(axis=-1, keepdims=True)
        with np.errstate(divide="ignore", invalid="ignore"):
            o = np.where(total > 0, np.matmul(e, vv) / total, 0.0)
            ls = np.where(total[..., 0] > 0, safe[..., 0] + np.log(total[..., 0]), -np.inf)
        out[idx] = o.transpose(1, 0, 2)
        lse[:, idx] = ls
    return out, lse


def brute_force_row(q_row, k_seg, v_seg, *, scale, visible_keys=None):
    """One query row of one head by explicit loops in float64 (tiny inputs only)."""
    n_keys = k_seg.shape[0] if visible_keys is None else visible_keys
    if n_keys <= 0:
        return np.zeros(k_seg.shape[1]), -math.inf
    logits = [float(np.dot(q_row, k_seg[j])) * scale for j in range(n_keys)]
    top = max(logits)
    weights = [math.exp(x - top) for x in logits]
    total = sum(weights)
    o = sum(w * v_seg[j] for j, w in enumerate(weights)) / total
    return o, top + math.log(total)


def seeded_normal_chunks(tokens: int, heads: int, head_dim: int, *, seed: int, tensor_index: int,
                         chunk_tokens: int = 4096, dtype=None):
    """Input tensor as the reference benchmark fills it
    (src/seqattn_core/benchmarking/common.py:45-71).

    Chunk c of tensor t is ``normal_`` from a CPU generator seeded with
    ``seed + t * 1_000_003 + c``.  Returns a torch tensor (the generator
    stream is torch's, so the values are bit-identical to the reference's).
    """
    import torch

    dtype = torch.bfloat16 if dtype is None else dtype
    out = torch.empty((tokens, heads, head_dim), dtype=dtype)
    for c, start in enumerate(range(0, tokens, chunk_tokens)):
        g = torch.Generator(device="cpu").manual_seed(seed + tensor_index * 1_000_003 + c)
        out[start : min(start + chunk_tokens, tokens)].normal_(generator=g)
    return out


def round_f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns (uint16) of float32 values, round to nearest even
    (the conversion torch and the reference kernels use); NaN stays NaN."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = bits + np.uint32(0x7FFF) + ((bits >> 16) & np.uint32(1))
    out = (rounded >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.uint16(0x7FC0)
    return out


def quantize_int8_groups(x: np.ndarray, group_tokens: int = 64) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric INT8 storage of ``x [tokens, heads, head_dim]`` (float32 view).

    Follows quantize_int8_per_token_group (reference
    src/seqattn_core/quantization.py:8-35): per group of ``group_tokens`` rows
    and per head, step = amax / 127 in float32 (1 where amax is 0),
    q = clamp(round_half_even(x / step), -127, 127), and the stored scale is
    float16(step).  Returns (q int8, scales float16 [groups, heads]).
    """
    x = as_f32(np.asarray(x))
    tokens, heads, _ = x.shape
    groups = -(-tokens // group_tokens)
    q = np.empty(x.shape, dtype=np.int8)
    scales = np.empty((groups, heads), dtype=np.float16)
    for g in range(groups):
        block = x[g * group_tokens : min((g + 1) * group_tokens, tokens)]
        step = (np.abs(block).max(axis=(0, 2)) / np.float32(127.0)).astype(np.float32)
        step = np.where(step > 0, step, np.float32(1.0)).astype(np.float32)
        scales[g] = step.astype(np.float16)
        q[g * group_tokens : g * group_tokens + block.shape[0]] = np.clip(
            np.round(block / step[None, :, None]), -127, 127).astype(np.int8)
    return q, scales


def dequantize_int8_groups(q: np.ndarray, scales: np.ndarray, *, group_tokens: int = 64,
                           token_offset: int = 0, to_bf16: bool = True) -> np.ndarray:
    """Dequantized K or V as the reference's INT8 update kernel forms it
    (reference src/seqattn_core/kernels/streaming.py:113-120): row j uses
    scale[(token_offset + j) // group_tokens]; the product float32(q) *
    float32(scale) is rounded once in float32 and then to the query dtype.
    Returns bf16 bit patterns (uint16) by default, else the float32 product."""
    q = np.asarray(q)
    rows = (token_offset + np.arange(q.shape[0])) // group_tokens
    product = q.astype(np.float32) * np.asarray(scales, dtype=np.float16).astype(np.float32)[rows][:, :, None]
    return round_f32_to_bf16_bits(product) if to_bf16 else product


__all__ = [
    "brute_force_row",
    "dequantize_int8_groups",
    "quantize_int8_groups",
    "round_f32_to_bf16_bits",
    "chunked_attention",
    "dense_attention_f64",
    "seeded_normal_chunks",
    "segment_bounds",
]
