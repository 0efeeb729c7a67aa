"""The paged KV-cache store (``src/llmopt/cache/paged_cache.py``).

Only :class:`PagedKVCache`, the tensor store that decode attention reads, is provided here.
The reference's block pool, block table and prefix cache (``block_pool.py``,
``paged_cache.py:10-134``, ``prefix_cache.py``) are host-side bookkeeping of its engine and
are not part of this package.
"""

from __future__ import annotations

from llmopt.cache.paged_cache import PagedKVCache

__all__ = ["PagedKVCache"]
