"""Segment routing: which rows of one call use which adapter.

The reference runs one module call per role (student/generator, fake critic,
teacher), each over its own batch (training/dmd.py:301-353), and the LiveWan
critic toggles its adapter off for the teacher pass on a shared base
(reference/livewan_wan21/wanstreamer/lora.py:65-74). Here the roles' rows are
concatenated and described by integer segments: rows
[seg_offsets[s], seg_offsets[s+1]) use adapter adapter_ids[s], -1 meaning the
frozen base alone. All routing is host-side integer arithmetic and is exact.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Iterator, Sequence

BASE_ONLY = -1


@dataclass(frozen=True)
class SegmentRouting:
    seg_offsets: tuple[int, ...]
    adapter_ids: tuple[int, ...]

    def __post_init__(self):
        off, ids = tuple(int(v) for v in self.seg_offsets), tuple(int(v) for v in self.adapter_ids)
        object.__setattr__(self, "seg_offsets", off)
        object.__setattr__(self, "adapter_ids", ids)
        if len(off) != len(ids) + 1 or not ids:
            raise ValueError("segment routing: need len(seg_offsets) == len(adapter_ids) + 1 >= 2")
        if off[0] != 0:
            raise ValueError("segment routing: seg_offsets[0] must be 0")
        if any(b < a for a, b in zip(off, off[1:])):
            raise ValueError("segment routing: seg_offsets must be nondecreasing")
        if any(a < BASE_ONLY for a in ids):
            raise ValueError("segment routing: adapter ids are -1 (base only) or >= 0")

    @classmethod
    def from_lengths(cls, lengths: Sequence[int], adapter_ids: Sequence[int]) -> "SegmentRouting":
        if len(lengths) != len(adapter_ids):
            raise ValueError("segment routing: one adapter id per segment length")
        if any(int(n) < 0 for n in lengths):
            raise ValueError("segment routing: segment lengths must be >= 0")
        off = [0]
        for n in lengths:
            off.append(off[-1] + int(n))
        return cls(tuple(off), tuple(adapter_ids))

    @classmethod
    def single(cls, rows: int, adapter_id: int = 0) -> "SegmentRouting":
        return cls((0, int(rows)), (int(adapter_id),))

    @property
    def num_rows(self) -> int:
        return self.seg_offsets[-1]

    @property
    def num_segments(self) -> int:
        return len(self.adapter_ids)

    def lengths(self) -> tuple[int, ...]:
        return tuple(b - a for a, b in zip(self.seg_offsets, self.seg_offsets[1:]))

    def validate_for(self, rows: int, n_adapters: int) -> None:
        if self.num_rows != rows:
            raise ValueError(f"segment routing covers {self.num_rows} rows, input has {rows}")
        if any(a >= n_adapters for a in self.adapter_ids):
            raise ValueError(f"segment routing names adapter >= {n_adapters}")

    def row_adapter(self) -> list[int]:
        """Adapter id of every row (for tests and small inputs)."""
        out: list[int] = []
        for (a, b), ad in zip(zip(self.seg_offsets, self.seg_offsets[1:]), self.adapter_ids):
            out.extend([ad] * (b - a))
        return out

    def groups(self, max_segments: int) -> Iterator[tuple[int, int, tuple[int, ...], tuple[int, ...]]]:
        """Split into row ranges of at most ``max_segments`` segments each.

        Yields (row_start, row_end, local_offsets, local_ids); local offsets
        start at 0. One group when the routing already fits one call.
        """
        n = self.num_segments
        for s0 in range(0, n, max_segments):
            s1 = min(n, s0 + max_segments)
            base = self.seg_offsets[s0]
            yield (base, self.seg_offsets[s1],
                   tuple(o - base for o in self.seg_offsets[s0:s1 + 1]),
                   self.adapter_ids[s0:s1])
