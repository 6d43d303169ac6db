"""ctypes binding of libseqattn_hip.so (declared in include/seqattn_hip.h).

The library links against ``libamdhip64.so.7``.  PyTorch-ROCm ships its own
copy of that runtime; importing torch first makes the dynamic loader reuse the
already-loaded runtime, so device pointers and streams created by torch are
valid inside the library.  There is no fallback: when the library is missing
every GPU entry point raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libseqattn_hip.so"
ABI_VERSION = 3

SA_DTYPE_BF16 = 0
SA_DTYPE_FP16 = 1
SA_FLAG_CAUSAL = 1
SA_FLAG_INITIALIZE = 2

c_int32 = ctypes.c_int32
c_int64 = ctypes.c_int64
c_double = ctypes.c_double
c_void_p = ctypes.c_void_p
c_float_p = ctypes.POINTER(ctypes.c_float)


class PipelineStats(ctypes.Structure):
    _fields_ = [
        ("h2d_bytes", c_int64),
        ("d2h_bytes", c_int64),
        ("q_chunks", c_int64),
        ("kv_tiles", c_int64),
        ("max_resident_q_tokens", c_int64),
    ]


# name -> (restype, argtypes); the single source of the Python-side ABI.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "sa_abi_version": (c_int32, []),
    "sa_last_error": (ctypes.c_char_p, []),
    "sa_update_attention_state": (
        c_int32,
        [c_void_p] * 6
        + [c_int64] * 10
        + [c_int32] * 8
        + [c_double, c_int32, c_int32, c_void_p],
    ),
    "sa_update_attention_state_int8": (
        c_int32,
        [c_void_p] * 8
        + [c_int64] * 14
        + [c_int32] * 9
        + [c_double, c_int32, c_int32, c_int32, c_void_p],
    ),
    "sa_finalize_attention": (
        c_int32,
        [c_void_p] * 5 + [c_int64] * 8 + [c_int32] * 4 + [c_void_p],
    ),
    "sa_pipeline_create": (
        c_int32,
        [ctypes.POINTER(c_void_p), c_int32, c_void_p, ctypes.POINTER(c_void_p),
         ctypes.POINTER(c_void_p), c_int32, c_void_p, c_void_p, c_void_p,
         ctypes.POINTER(c_void_p), c_int32] + [c_int32] * 6 + [c_void_p, c_void_p],
    ),
    "sa_pipeline_create_head_groups": (
        c_int32,
        [ctypes.POINTER(c_void_p), c_int32] + [ctypes.POINTER(c_void_p)] * 4 + [c_int64, c_int32, c_int64, c_int64]
        + [c_int32] * 6 + [c_void_p, c_void_p],
    ),
    "sa_pipeline_destroy": (c_int32, [c_void_p]),
    "sa_pipeline_run": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
         ctypes.POINTER(c_int64), ctypes.POINTER(c_int64), c_int32, c_double, c_int32,
         c_void_p, ctypes.POINTER(PipelineStats)],
    ),
    "sa_pipeline_run_device_output": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64,
         ctypes.POINTER(c_int64), ctypes.POINTER(c_int64), c_int32, c_double, c_int32,
         c_void_p, ctypes.POINTER(PipelineStats)],
    ),
    "sa_pipeline_load_q": (
        c_int32, [c_void_p, c_void_p, c_int32, c_void_p, ctypes.POINTER(PipelineStats)]
    ),
    "sa_pipeline_stream_kv": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_double, c_int32,
         c_void_p, ctypes.POINTER(PipelineStats)],
    ),
    "sa_pipeline_stream_kv_span": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, ctypes.POINTER(c_int32), c_int32, c_int32,
         c_int32, c_double, c_int32, c_void_p, ctypes.POINTER(PipelineStats)],
    ),
    "sa_pipeline_stream_kv_gather": (
        c_int32,
        [c_void_p, ctypes.POINTER(c_void_p), ctypes.POINTER(c_void_p), ctypes.POINTER(c_int32), c_int32,
         c_int32, ctypes.POINTER(c_int32), c_int32, c_int32, c_int32, c_double, c_int32, c_void_p,
         ctypes.POINTER(PipelineStats)],
    ),
    "sa_pipeline_attach_int8_scales": (
        c_int32,
        [c_void_p, ctypes.POINTER(c_void_p), ctypes.POINTER(c_void_p), c_int32],
    ),
    "sa_pipeline_stream_kv_gather_int8": (
        c_int32,
        [c_void_p, ctypes.POINTER(c_void_p), ctypes.POINTER(c_void_p), ctypes.POINTER(c_void_p),
         ctypes.POINTER(c_void_p), ctypes.POINTER(c_int32), c_int32, c_int32, ctypes.POINTER(c_int32),
         c_int32, c_int32, c_int32, c_double, c_int32, c_void_p, ctypes.POINTER(PipelineStats)],
    ),
    "sa_pipeline_run_resident": (
        c_int32,
        [c_void_p] * 6 + [c_int64] * 9
        + [ctypes.POINTER(c_int64), ctypes.POINTER(c_int64), c_int32, c_double, c_int32, c_void_p,
           ctypes.POINTER(PipelineStats)],
    ),
    "sa_run_resident_noalloc": (
        c_int32,
        [c_void_p] * 4 + [c_void_p] + [c_int64] * 9
        + [ctypes.POINTER(c_int64), ctypes.POINTER(c_int64)] + [c_int32] * 6 + [c_double, c_int32, c_void_p],
    ),
    "sa_pipeline_finalize": (
        c_int32, [c_void_p, c_int32, c_int32, c_void_p, c_int64, c_int64, c_void_p]
    ),
    "sa_pipeline_finalize_into": (
        c_int32, [c_void_p, c_void_p, c_int64, c_int64, c_int32, c_void_p, c_int64, c_int64, c_void_p]
    ),
    "sa_pipeline_release_q": (c_int32, [c_void_p, c_void_p]),
    "sa_pipeline_d2h": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int32, c_void_p,
         ctypes.POINTER(PipelineStats)],
    ),
    "sa_pipeline_synchronize": (c_int32, [c_void_p]),
    "sa_pipeline_attach_resident_scratch": (c_int32, [c_void_p, c_void_p, c_int64]),
    "sa_pipeline_attach_host_staging": (c_int32, [c_void_p, c_void_p, c_int64]),
    "sa_pipeline_set_kernel_timing": (c_int32, [c_void_p, c_int32]),
    "sa_pipeline_set_trace_ranges": (c_int32, [c_void_p, c_int32]),
    "sa_pipeline_kernel_timing": (
        c_int32, [c_void_p, ctypes.POINTER(c_double), ctypes.POINTER(c_int64)]
    ),
    "sa_pipeline_kernel_busy": (
        c_int32, [c_void_p, ctypes.POINTER(c_double), ctypes.POINTER(c_double), ctypes.POINTER(c_int64)]
    ),
    "sa_pipeline_stream": (c_void_p, [c_void_p, c_int32]),
    "sa_pipeline_output_slot": (c_void_p, [c_void_p, c_int32]),
    "sa_pipeline_q_buffer": (c_void_p, [c_void_p]),
}

_lib: ctypes.CDLL | None = None
_load_error: str | None = None


def _load() -> ctypes.CDLL:
    global _lib, _load_error
    if _lib is not None:
        return _lib
    path = Path(os.environ.get("SEQATTN_HIP_LIBRARY", LIB_PATH))
    if not path.exists():
        _load_error = (
            f"{path} is missing; build it with `python stream-attn_amd/build_native.py` "
            "(or __graft_entry__.build())"
        )
        raise RuntimeError(_load_error)
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.sa_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"libseqattn_hip ABI {version} does not match the binding ({ABI_VERSION})")
    _lib = lib
    return lib


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError when it is not built."""
    return _load()


def library_is_built() -> bool:
    return Path(os.environ.get("SEQATTN_HIP_LIBRARY", LIB_PATH)).exists()


def hip_is_available() -> bool:
    """True when the native library is built and a ROCm GPU is visible."""
    return library_is_built() and torch.version.hip is not None and torch.cuda.is_available()


def check(status: int, what: str) -> None:
    """Raise RuntimeError for a non-zero status of a library call."""
    if status != 0:
        message = lib().sa_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {status}): {message}")


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return SA_DTYPE_BF16
    if dtype == torch.float16:
        return SA_DTYPE_FP16
    raise ValueError(f"the HIP backend requires float16 or bfloat16 tensors, got {dtype}")


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()


def stream_handle(stream: torch.cuda.Stream) -> int:
    return stream.cuda_stream


__all__ = [
    "ABI_VERSION",
    "LIB_PATH",
    "PipelineStats",
    "SIGNATURES",
    "check",
    "dtype_code",
    "hip_is_available",
    "lib",
    "library_is_built",
]
