"""Paged-KV-cache fixtures shared by the oracle and GPU tests.

Built the way the reference's tests build theirs
(tests/cuda/test_paged_attention.cu:105-157): more physical blocks than the
sequences use, handed out in reverse, so a kernel that ignored the block table
(reading token t at slot t) would disagree with the oracle.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class PagedCase:
    query: np.ndarray      # [S, H, D] float32
    k_cache: np.ndarray    # [blocks, block_size, KVH, D] float32
    v_cache: np.ndarray
    tables: np.ndarray     # [S, max_blocks] uint32
    context: np.ndarray    # [S] int32
    scale: float

    @property
    def dims(self) -> tuple[int, int, int, int, int, int]:
        s, h, d = self.query.shape
        return s, h, self.k_cache.shape[2], d, self.k_cache.shape[1], self.tables.shape[1]


def make_case(sequences: int, heads: int, kv_heads: int, head_dim: int, block_size: int,
              context: list[int], seed: int, spare: int = 3) -> PagedCase:
    gen = np.random.Generator(np.random.PCG64(seed))
    blocks_of = [(n + block_size - 1) // block_size for n in context]
    max_blocks = max(max(blocks_of), 1)
    total = sum(blocks_of) + spare
    shape = (total, block_size, kv_heads, head_dim)
    k_cache = gen.standard_normal(shape, dtype=np.float32)
    v_cache = gen.standard_normal(shape, dtype=np.float32)
    query = gen.standard_normal((sequences, heads, head_dim), dtype=np.float32)
    tables = np.zeros((sequences, max_blocks), dtype=np.uint32)
    nxt = total - 1
    for s, count in enumerate(blocks_of):
        for logical in range(count):
            tables[s, logical] = nxt
            nxt = total - 1 if nxt == 0 else nxt - 1
    return PagedCase(query, k_cache, v_cache, tables, np.asarray(context, dtype=np.int32),
                     1.0 / float(np.sqrt(head_dim)))


# The reference's parity cases (tests/cuda/test_paged_attention.cu:196-199):
# (sequences, heads, kv_heads, head_dim, block_size, context lengths).
REFERENCE_CASES = [
    (1, 1, 1, 32, 4, [1]),
    (1, 2, 2, 64, 8, [8]),
    (3, 2, 2, 32, 4, [5, 12, 1]),
    (2, 4, 2, 64, 16, [33, 7]),
    (2, 8, 2, 128, 8, [17, 64]),
]
