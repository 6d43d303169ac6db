"""Device staging of the QKV projection producer (reference
src/seqattn_core/projection/workspace.py:8-38).

``num_projection_buffers`` hidden slots ``[projection_chunk_tokens,
hidden_features]`` in HBM, an H2D and a D2H stream (default priority) beside
the compute stream, and per slot three events: hidden rows landed
(``input_ready``), projection enqueued (``projected_ready``) and the slot's
Q/K/V copies out of it done (``copy_done``).  A slot is reused only after its
``copy_done`` has completed on the host, which bounds the projected tiles in
flight to the slot count.
"""

from __future__ import annotations

import torch

from ..config import ProjectionPipelineConfig
from ..streaming.workspace import copy_streams


class ProjectionWorkspace:
    def __init__(
        self,
        *,
        hidden_features: int,
        dtype: torch.dtype,
        device: torch.device,
        config: ProjectionPipelineConfig,
    ) -> None:
        self.hidden_features = hidden_features
        self.hidden = [
            torch.empty((config.projection_chunk_tokens, hidden_features), dtype=dtype, device=device)
            for _ in range(config.num_projection_buffers)
        ]
        self.compute_stream = torch.cuda.current_stream(device)
        # The per-device copy stream pair shared with the attention pipeline
        # (the projection copies and the attention copies do not overlap).
        self.h2d_stream, self.d2h_stream = copy_streams(device)
        self.input_ready = [torch.cuda.Event() for _ in self.hidden]
        self.projected_ready = [torch.cuda.Event() for _ in self.hidden]
        self.copy_done = [torch.cuda.Event() for _ in self.hidden]
        self.busy = [False for _ in self.hidden]
        self.keepalive: list[tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None] = [None for _ in self.hidden]

    def reclaim(self, slot: int) -> None:
        """Wait until ``slot``'s previous tile has left its buffers."""
        if self.busy[slot]:
            self.copy_done[slot].synchronize()
            self.keepalive[slot] = None
            self.busy[slot] = False

    def drain(self) -> None:
        self.d2h_stream.synchronize()
        self.compute_stream.synchronize()
        for slot in range(len(self.hidden)):
            self.keepalive[slot] = None
            self.busy[slot] = False


__all__ = ["ProjectionWorkspace"]
