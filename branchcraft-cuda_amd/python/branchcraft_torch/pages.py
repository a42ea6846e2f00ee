"""Host-side page owner for the copy-on-write KV transaction.

Pure Python bookkeeping, no tensors: page refcounts, a LIFO free list,
per-request page tables and lengths, snapshots, and the commit plan
(copy-on-write clone of a shared partial page, fresh pages, destination
page/slot of every accepted token).  ``PagedTreeCache`` in
``transaction.py`` executes the plans with the HIP ops.

Semantics follow python/branchcraft_torch/transaction.py:23-150 of the
reference, which the page tables must match bit for bit:

* the free list is a LIFO stack initialised so that pages come out in
  ascending order (0, 1, 2, ...); released pages are pushed back on top;
* a snapshot holds one reference on each page it remembers;
* a commit that appends to a partial last page whose refcount is above one
  clones that page into a freshly allocated one first;
* token position ``pos`` lands in page ``pages[pos // 16]`` at slot
  ``pos % 16``.
"""

from __future__ import annotations

from dataclasses import dataclass, field

PAGE_SIZE = 16


@dataclass
class Snapshot:
    request: int
    pages: list[int]
    length: int
    active: bool = True


@dataclass
class CommitPlan:
    """What a commit does on the device, in order."""

    request: int
    cow: tuple[int, int] | None  # (old page, fresh page) to clone first
    dest_pages: list[int] = field(default_factory=list)
    dest_slots: list[int] = field(default_factory=list)
    new_length: int = 0


class PageOwner:
    def __init__(self, physical_pages: int):
        if physical_pages < 1:
            raise ValueError("physical_pages must be positive")
        self.physical_pages = physical_pages
        self.refcount = [0] * physical_pages
        self.free = list(range(physical_pages - 1, -1, -1))  # pop() -> 0, 1, ...
        self.pages: dict[int, list[int]] = {}
        self.lengths: dict[int, int] = {}
        self._next_request = 0

    # -- allocation ------------------------------------------------------
    def alloc(self) -> int:
        if not self.free:
            raise RuntimeError("KV page pool exhausted")
        page = self.free.pop()
        if self.refcount[page] != 0:
            raise RuntimeError(f"free list holds referenced page {page}")
        self.refcount[page] = 1
        return page

    def release(self, page: int) -> None:
        if self.refcount[page] <= 0:
            raise RuntimeError(f"page {page} released more often than referenced")
        self.refcount[page] -= 1
        if self.refcount[page] == 0:
            self.free.append(page)

    # -- requests ----------------------------------------------------------
    def new(self, tokens: int) -> int:
        """Register a request of ``tokens`` prefix tokens on fresh pages."""
        if tokens < 0:
            raise ValueError("negative prefix length")
        count = (tokens + PAGE_SIZE - 1) // PAGE_SIZE
        if len(self.free) < count:
            raise RuntimeError("KV page pool exhausted")
        request = self._next_request
        self._next_request += 1
        self.pages[request] = [self.alloc() for _ in range(count)]
        self.lengths[request] = tokens
        return request

    def fork(self, source: int) -> int:
        request = self._next_request
        self._next_request += 1
        self.pages[request] = list(self.pages[source])
        self.lengths[request] = self.lengths[source]
        for page in self.pages[request]:
            self.refcount[page] += 1
        return request

    def checkpoint(self, request: int) -> Snapshot:
        pages = list(self.pages[request])
        for page in pages:
            self.refcount[page] += 1
        return Snapshot(request, pages, self.lengths[request])

    def rollback(self, snapshot: Snapshot) -> None:
        """Restore the snapshot's mapping; its references pass to the request."""
        if not snapshot.active:
            raise RuntimeError("snapshot already consumed")
        for page in self.pages[snapshot.request]:
            self.release(page)
        self.pages[snapshot.request] = snapshot.pages
        self.lengths[snapshot.request] = snapshot.length
        snapshot.active = False

    def accept(self, snapshot: Snapshot) -> None:
        """Keep the current mapping and drop the snapshot's references."""
        if not snapshot.active:
            raise RuntimeError("snapshot already consumed")
        for page in snapshot.pages:
            self.release(page)
        snapshot.active = False

    def plan_commit(self, request: int, count: int) -> CommitPlan:
        """Reserve pages for ``count`` appended tokens and return the plan.

        Raises before changing any state when the pool cannot hold them."""
        if count < 1:
            raise ValueError("path is empty")
        old_length = self.lengths[request]
        pages = self.pages[request]
        new_page_count = (old_length + count + PAGE_SIZE - 1) // PAGE_SIZE
        copy_partial = old_length % PAGE_SIZE != 0 and self.refcount[pages[-1]] > 1
        needed = new_page_count - len(pages) + int(copy_partial)
        if len(self.free) < needed:
            raise RuntimeError("KV page pool exhausted")
        cow = None
        if copy_partial:
            old = pages[-1]
            fresh = self.alloc()
            pages[-1] = fresh
            self.release(old)
            cow = (old, fresh)
        while len(pages) < new_page_count:
            pages.append(self.alloc())
        positions = range(old_length, old_length + count)
        plan = CommitPlan(request, cow,
                          [pages[pos // PAGE_SIZE] for pos in positions],
                          [pos % PAGE_SIZE for pos in positions],
                          old_length + count)
        self.lengths[request] = plan.new_length
        return plan

    def check_invariants(self) -> None:
        """Refcounts equal live references; the free list holds exactly the
        unreferenced pages, once each."""
        counts = [0] * self.physical_pages
        for pages in self.pages.values():
            for p in pages:
                counts[p] += 1
        free = sorted(self.free)
        if len(set(free)) != len(free):
            raise AssertionError("free list holds a page twice")
        for p in range(self.physical_pages):
            if (self.refcount[p] == 0) != (p in set(free)):
                raise AssertionError(f"page {p}: refcount {self.refcount[p]} vs free list")
            if self.refcount[p] < counts[p]:
                raise AssertionError(f"page {p}: refcount below live mappings")
