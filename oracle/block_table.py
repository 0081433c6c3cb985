"""Pure-Python restatement of the reference block allocator (test oracle).

Follows crates/ai-engine-candle/src/paged/block_table.rs line by line in
meaning; used by tests to check the product's C++ allocator
(``pkv_allocator_*`` in libpagedkv) on random operation sequences.  Pinned by
the reference's five KATs (block_table.rs:65-116), replayed in
tests/test_oracle.py against this class and in tests/test_allocator.py
against the product.
"""
from __future__ import annotations


class CapacityError(Exception):
    """ensure_capacity could not be satisfied (the reference's Err(()))."""


class BlockTable:
    """block_table.rs:10-14: the ordered physical blocks of one sequence."""

    def __init__(self) -> None:
        self.blocks: list[int] = []


class BlockAllocator:
    """block_table.rs:5-8,16-58."""

    def __init__(self, num_blocks: int, block_size: int) -> None:
        # :17-21 -- free list reversed so pops hand out 0, 1, 2, ...
        self.block_size = block_size
        self.free = list(range(num_blocks - 1, -1, -1))

    def free_count(self) -> int:  # :23-25
        return len(self.free)

    def blocks_for(self, n_tokens: int) -> int:  # :27-30 (div_ceil)
        return -(-n_tokens // self.block_size)

    def ensure_capacity(self, table: BlockTable, n_tokens: int) -> None:  # :32-47
        need = self.blocks_for(n_tokens)
        if need <= len(table.blocks):
            return
        extra = need - len(table.blocks)
        if extra > len(self.free):
            raise CapacityError()
        for _ in range(extra):
            table.blocks.append(self.free.pop())

    def release(self, table: BlockTable) -> None:  # :49-52
        self.free.extend(table.blocks)
        table.blocks.clear()

    def locate(self, table: BlockTable, pos: int) -> tuple[int, int]:  # :54-58
        return table.blocks[pos // self.block_size], pos % self.block_size
