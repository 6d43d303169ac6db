"""Host-side schedule of the paged runtime: Q blocks built from pages and the
queue of K/V row fragments that feeds gathered ring chunks.

The reference runs one resident Q block per query page and one kernel launch
per K/V page (paged/runtime/triton.py:62-238).  Here query pages are packed
into Q blocks of up to the planner's resident size, and K/V pages are packed
into launches of the planner's K/V chunk, aligned to multiples of the chunk
within the segment (the same chunk boundaries tensor mode uses).
"""

from __future__ import annotations

from collections import deque
from collections.abc import Sequence
from dataclasses import dataclass, field

from .layout import PageDescriptor


@dataclass(frozen=True)
class QPiece:
    """Rows [page_offset, page_offset + rows) of a query page, placed at row
    ``block_offset`` of its Q block."""

    page: PageDescriptor
    page_offset: int
    rows: int
    block_offset: int

    @property
    def whole_page(self) -> bool:
        return self.page_offset == 0 and self.rows == self.page.valid_tokens


@dataclass(frozen=True)
class QBlock:
    """One resident Q block: segment rows [segment_start, segment_start + rows);
    its output lands at row ``group_offset`` of its group's output slot."""

    segment_start: int
    rows: int
    pieces: tuple[QPiece, ...]
    group_offset: int


@dataclass(frozen=True)
class QGroup:
    """Consecutive Q blocks whose output pages complete together: either
    whole pages packed into one block, or one page larger than a block split
    over several blocks."""

    blocks: tuple[QBlock, ...]
    pages: tuple[PageDescriptor, ...]
    rows: int


def plan_q_groups(pages: Sequence[PageDescriptor], block_rows: int) -> list[QGroup]:
    """Pack one segment's query pages (in order) into Q groups."""
    if block_rows <= 0:
        raise ValueError("block_rows must be positive")
    groups: list[QGroup] = []
    current: list[PageDescriptor] = []
    current_rows = 0

    def flush() -> None:
        nonlocal current, current_rows
        if not current:
            return
        pieces, offset = [], 0
        for page in current:
            pieces.append(QPiece(page, 0, page.valid_tokens, offset))
            offset += page.valid_tokens
        start = current[0].segment_token_start
        groups.append(QGroup((QBlock(start, offset, tuple(pieces), 0),), tuple(current), offset))
        current, current_rows = [], 0

    for page in pages:
        if page.valid_tokens > block_rows:
            flush()
            blocks = []
            for off in range(0, page.valid_tokens, block_rows):
                n = min(block_rows, page.valid_tokens - off)
                blocks.append(QBlock(page.segment_token_start + off, n, (QPiece(page, off, n, 0),), off))
            groups.append(QGroup(tuple(blocks), (page,), page.valid_tokens))
            continue
        if current_rows + page.valid_tokens > block_rows:
            flush()
        current.append(page)
        current_rows += page.valid_tokens
    flush()
    return groups


@dataclass
class Fragment:
    """Contiguous host rows of K and V (addresses) plus the owner released
    once the rows have been copied; INT8 pages also carry per-row K and V
    scale addresses."""

    k_address: int
    v_address: int
    rows: int
    owner: object = None
    ks_address: int = 0
    vs_address: int = 0


@dataclass
class FragmentQueue:
    """K/V rows waiting for their H2D copy, in segment order."""

    row_bytes: int
    scale_row_bytes: int = 0
    fragments: deque = field(default_factory=deque)
    rows: int = 0

    def push(self, fragment: Fragment) -> None:
        if fragment.rows > 0:
            self.fragments.append(fragment)
            self.rows += fragment.rows

    def take(self, rows: int) -> tuple[list[tuple[int, int, int, int, int]], list[object]]:
        """Remove the first ``rows`` rows: returns (k, v, rows, k_scales,
        v_scales) pieces and the owners whose rows have now all been taken."""
        if rows > self.rows:
            raise ValueError("not enough queued rows")
        pieces: list[tuple[int, int, int, int, int]] = []
        finished: list[object] = []
        left = rows
        while left:
            head = self.fragments[0]
            n = min(left, head.rows)
            pieces.append((head.k_address, head.v_address, n, head.ks_address, head.vs_address))
            if n == head.rows:
                self.fragments.popleft()
                finished.append(head.owner)
            else:
                step = n * self.row_bytes
                head.k_address += step
                head.v_address += step
                if self.scale_row_bytes:
                    head.ks_address += n * self.scale_row_bytes
                    head.vs_address += n * self.scale_row_bytes
                head.rows -= n
            left -= n
        self.rows -= rows
        return pieces, finished


__all__ = ["Fragment", "FragmentQueue", "QBlock", "QGroup", "QPiece", "plan_q_groups"]
