"""seqattn for AMD MI355X: streamed exact attention over host-resident Q/K/V.

Drop-in for the reference package's tensor-mode and device-consumer API
(reference src/seqattn_core/__init__.py:1-77).  Q/K/V stay in caller-owned
(pinned) host DRAM; a resident Q super-block and a K/V ring live in a bounded
HBM workspace; the chunk-update / finalize kernels and the copy pipeline are
native gfx950 code in ``_lib/libseqattn_hip.so``.  Paged mode
(``PagedAttentionRunner`` over memory or aligned on-disk page stores) runs on
the same kernels and pipeline, and ``ProjectedAttentionRunner`` fuses a
caller's QKV and output projections around the streamed attention.
"""

from .api import StreamingAttentionRunner, clear_runner_cache, streaming_attn_func, streaming_attn_varlen_func
from .config import PagedAttentionConfig, ProjectionPipelineConfig, StreamingAttentionConfig
from .paged import (
    CallbackOutputSink,
    HostMemoryPlan,
    HostMemorySnapshot,
    KVLayout,
    MemoryPageSink,
    MemoryPageSource,
    PagedAttentionRunner,
    PageDescriptor,
    PageSink,
    PageSource,
    TensorLayout,
)
from .planner import AttentionPlan, build_plan
from .projection import (
    OutputProjector,
    ProjectedAttentionRunner,
    QKVProjector,
    streaming_projected_self_attention,
)
from .stats import PagedAttentionStats, ProjectedAttentionStats, StreamingAttentionStats
from .storage import NvmeOutputSink, NvmeQKVStore, NvmeQKVWriter, ephemeral_nvme_directory, load_nvme_output

__all__ = [
    "AttentionPlan",
    "CallbackOutputSink",
    "HostMemoryPlan",
    "HostMemorySnapshot",
    "KVLayout",
    "MemoryPageSink",
    "MemoryPageSource",
    "NvmeOutputSink",
    "NvmeQKVStore",
    "NvmeQKVWriter",
    "OutputProjector",
    "PageDescriptor",
    "PageSink",
    "PageSource",
    "PagedAttentionConfig",
    "PagedAttentionRunner",
    "PagedAttentionStats",
    "ProjectedAttentionRunner",
    "ProjectedAttentionStats",
    "ProjectionPipelineConfig",
    "QKVProjector",
    "StreamingAttentionConfig",
    "StreamingAttentionRunner",
    "StreamingAttentionStats",
    "TensorLayout",
    "build_plan",
    "ephemeral_nvme_directory",
    "load_nvme_output",
    "clear_runner_cache",
    "streaming_attn_func",
    "streaming_attn_varlen_func",
    "streaming_projected_self_attention",
]

__version__ = "0.3.0+mi355x"
