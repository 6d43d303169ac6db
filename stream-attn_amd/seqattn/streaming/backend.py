"""Backend selection (reference src/seqattn_core/streaming/backend.py:8-29).

The only execution backend of this package is ``"hip"``: the gfx950 kernels
and transfer pipeline in libseqattn_hip.so.  ``"triton"`` is accepted as an
alias so existing configurations run unchanged.  The reference's FP32 torch
path (``"reference"``) is not shipped as a backend: a CPU restatement of it
exists only as the test oracle, so every run of this package executes on the
GPU and fails loudly when the native library or the GPU is missing.
"""

from __future__ import annotations

import torch

from .. import _native


def _hip_unavailable_reason() -> str | None:
    if not _native.library_is_built():
        return f"{_native.LIB_PATH} is not built"
    if torch.version.hip is None:
        return "this torch build has no ROCm/HIP support"
    if not torch.cuda.is_available():
        return "no ROCm GPU is visible"
    return None


def resolve_backend(
    name: str, dtype: torch.dtype, device: torch.device, *, head_dim: int | None = None
) -> str:
    device = torch.device(device)
    if name == "reference":
        raise ValueError(
            "backend='reference' (the FP32 CPU path) is not part of this package; "
            "use backend='hip' (or 'auto') on a ROCm device"
        )
    if name not in {"auto", "hip", "triton"}:
        raise ValueError(f"unsupported backend: {name}")
    if device.type != "cuda":
        raise ValueError("the HIP backend requires a ROCm ('cuda') device")
    if dtype not in {torch.float16, torch.bfloat16}:
        raise ValueError("the HIP backend requires float16 or bfloat16 inputs")
    if head_dim is not None and head_dim < 16:
        raise ValueError("the HIP backend requires head_dim >= 16 (one 16-wide MFMA slice)")
    reason = _hip_unavailable_reason()
    if reason is not None:
        raise RuntimeError(f"the HIP backend is not available: {reason}")
    return "hip"


__all__ = ["resolve_backend"]
