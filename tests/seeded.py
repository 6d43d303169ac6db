"""Seeded inputs and sampled-row parity checks for the GPU configuration tests.

Inputs follow the reference benchmark's scheme
(src/seqattn_core/benchmarking/common.py:45-71):
chunk c (4,096 tokens) of tensor t is ``normal_`` from a CPU generator seeded
with ``seed + t * 1_000_003 + c``; here the chunks are filled by a thread
pool straight into page-locked tensors.
"""

from __future__ import annotations

import gc
import math
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

class RunModeNotice(UserWarning):
    """Names the mode a GPU configuration test ran in (for example whether a
    store was read with O_DIRECT), so that the mode shows in pytest's
    warnings summary even under -q."""


O_TOL = 2e-2
LSE_TOL = 1e-3
REL_L2_TOL = 5e-3
SCALED_TOL = 2.0**-5


def cpu_threads() -> int:
    """Threads for host-side work: the CPUs this process may use, capped by
    OMP_NUM_THREADS when it is set (a GPU host's CPU share per job)."""
    try:
        share = len(os.sched_getaffinity(0))
    except AttributeError:
        share = os.cpu_count() or 1
    try:
        share = min(share, int(os.environ["OMP_NUM_THREADS"]))
    except (KeyError, ValueError):
        pass
    return max(1, share)


def seeded_qkv(tokens, heads, head_dim, *, seed=0, kv_heads=None, pinned=True, chunk_tokens=4096,
               k_head_scale=None):
    """(q, k, v) bf16 ``[tokens, heads, head_dim]``; ``k_head_scale`` (float32,
    one per K/V head) multiplies K as bf16(float32(k) * scale)."""
    kv_heads = heads if kv_heads is None else kv_heads
    shapes = ((tokens, heads, head_dim), (tokens, kv_heads, head_dim), (tokens, kv_heads, head_dim))
    tensors = tuple(torch.empty(shape, dtype=torch.bfloat16, pin_memory=pinned) for shape in shapes)
    scale = None if k_head_scale is None else torch.as_tensor(k_head_scale, dtype=torch.float32)[None, :, None]

    def fill(task):
        t, c, start = task
        stop = min(start + chunk_tokens, tokens)
        gen = torch.Generator(device="cpu").manual_seed(seed + t * 1_000_003 + c)
        block = tensors[t][start:stop]
        block.normal_(generator=gen)
        if t == 1 and scale is not None:
            block.copy_((block.float() * scale).to(torch.bfloat16))

    tasks = [(t, c, start) for t in range(3) for c, start in enumerate(range(0, tokens, chunk_tokens))]
    with ThreadPoolExecutor(max_workers=cpu_threads()) as pool:
        list(pool.map(fill, tasks))
    return tensors


def signature_and_random_rows(n, count, seed=0):
    """The reference large-tier signature rows {0, N/4, N/2, 3N/4, N-1}
    (benchmarks/large_tier_comparison.py:62-66) plus ``count`` seeded rows."""
    rng = np.random.default_rng(seed)
    signature = np.array([0, n // 4, n // 2, 3 * n // 4, n - 1])
    return np.unique(np.concatenate([signature, rng.choice(n, min(count, n), replace=False)]))


def u16(t: torch.Tensor) -> np.ndarray:
    """bf16/fp16 bit patterns of a CPU tensor as uint16 (no copy)."""
    return t.view(torch.int16).numpy().view(np.uint16)


def oracle_rows(q, k, v, rows, *, kv_chunk, scale=None):
    """Oracle O and LSE of query ``rows`` of one segment covering all of k/v."""
    from threadpoolctl import threadpool_limits

    from oracle.seqattn_oracle import chunked_attention

    with threadpool_limits(1):
        return chunked_attention(u16(q[torch.from_numpy(rows)]), u16(k), u16(v), [0, rows.size], [0, k.shape[0]],
                                 q_chunk_tokens=rows.size, kv_chunk_tokens=kv_chunk, softmax_scale=scale,
                                 workers=cpu_threads())


def check_parity(o, lse, ref_o, ref_l, label=""):
    """Tolerances against the FP32 oracle: O max-abs <= 2e-2, LSE max-abs <=
    1e-3, O relative L2 <= 5e-3, and every element within 2^-5 (|ref| + rms)."""
    o = np.asarray(o, dtype=np.float32)
    l = np.asarray(lse, dtype=np.float32)
    assert np.isfinite(o).all(), label
    diff = np.abs(o - ref_o)
    ref_norm = float(np.sqrt(np.square(ref_o, dtype=np.float64).sum()))
    rel_l2 = float(np.sqrt(np.square(diff, dtype=np.float64).sum())) / ref_norm if ref_norm > 0 else 0.0
    rms = ref_norm / math.sqrt(ref_o.size) if ref_o.size else 0.0
    scaled = float((diff / (np.abs(ref_o) + rms)).max()) if rms > 0 else 0.0
    finite = np.isfinite(ref_l)
    assert np.array_equal(np.isfinite(l), finite), f"{label}: LSE -inf pattern differs"
    err_l = float(np.abs(l[finite] - ref_l[finite]).max()) if finite.any() else 0.0
    err_o = float(diff.max()) if diff.size else 0.0
    print(f"    {label} max|dO|={err_o:.3e} relL2={rel_l2:.3e} scaled={scaled:.3e} max|dLSE|={err_l:.3e}",
          flush=True)
    assert err_o <= O_TOL, err_o
    assert rel_l2 <= REL_L2_TOL, rel_l2
    assert scaled <= SCALED_TOL, scaled
    assert err_l <= LSE_TOL, err_l
    return {"max_abs_o": err_o, "rel_l2": rel_l2, "scaled": scaled, "max_abs_lse": err_l}


def release_host_memory() -> None:
    """Return freed page-locked blocks to the OS (torch caches them)."""
    gc.collect()
    if torch.cuda.is_available():
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    torch._C._host_emptyCache()
