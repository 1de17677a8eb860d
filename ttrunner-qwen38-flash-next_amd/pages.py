"""Physical K/V pages shared by the sequences (slots) of a cache.

The reference's device engine gives every slot a fixed run of blocks and a
static page table (tt/model.py:625-648); its page table exists so that the
attention ops read positions from device memory, and slots are recycled by
``reset_slot`` (tt/model.py:2373-2431). For continuous batching with
sequences of very different lengths, this pool lets slots draw pages as they
grow instead: a slot maps a page when its first token there is written, gives
its pages back when it is reset, and a slot that continues another's prefix
maps the same pages (reference counts) instead of copying them.

Host bookkeeping only: the kernels see the result as the int32 page table.
"""

from __future__ import annotations


class PoolExhausted(MemoryError):
    """No free page is left in the pool."""


class PagePool:
    """``n_pages`` physical pages with reference counts.

    ``alloc`` hands out a free page with count 1 (lowest id first, so a fresh
    pool fills the way the static identity table would), ``share`` adds a
    mapping of a page already in use, ``release`` drops one and frees the page
    when none is left.
    """

    def __init__(self, n_pages: int):
        if n_pages <= 0:
            raise ValueError("a page pool needs at least one page")
        self.n_pages = n_pages
        self._ref = [0] * n_pages
        self._free = list(range(n_pages - 1, -1, -1))

    @property
    def n_free(self) -> int:
        return len(self._free)

    def refcount(self, page: int) -> int:
        return self._ref[page]

    def alloc(self) -> int:
        if not self._free:
            raise PoolExhausted(f"all {self.n_pages} pages are in use")
        page = self._free.pop()
        self._ref[page] = 1
        return page

    def share(self, page: int) -> int:
        if self._ref[page] <= 0:
            raise ValueError(f"page {page} is free and cannot be shared")
        self._ref[page] += 1
        return page

    def release(self, page: int) -> None:
        if self._ref[page] <= 0:
            raise ValueError(f"page {page} released more often than mapped")
        self._ref[page] -= 1
        if self._ref[page] == 0:
            self._free.append(page)
