"""Copy-on-write paged KV transaction driving the HIP ops.

Mirrors ``PagedTreeCache`` of the reference
(python/branchcraft_torch/transaction.py:23-150): an FP16 pool
[physical_pages, 16, kv_heads, head_dim] for K and for V, requests that can
be forked and checkpointed, tree verification against a request's pages and
a commit of an accepted root-to-leaf path.  The bookkeeping lives in
:class:`~branchcraft_torch.pages.PageOwner`; the device work -- the clone of
a shared partial page and the accepted-path copy -- runs as the
``copy_pages_`` and ``commit_path_`` HIP ops on the current stream.
``commit_many`` commits several requests with two launches in all (every
clone, then every accepted node) and leaves the same pages and page tables
as committing them one by one in the same order.
"""

from __future__ import annotations

import torch

from . import commit_path_, commit_paths_, copy_pages_, tree_verify
from .pages import CommitPlan, PageOwner, Snapshot

__all__ = ["PagedTreeCache", "Snapshot", "CommitPlan"]


class PagedTreeCache:
    def __init__(self, physical_pages: int, kv_heads: int, head_dim: int,
                 device: str = "cuda"):
        if head_dim not in (64, 128) or physical_pages < 1:
            raise ValueError("head_dim must be 64/128; physical_pages must be positive")
        self.owner = PageOwner(physical_pages)
        self.k = torch.zeros((physical_pages, 16, kv_heads, head_dim),
                             device=device, dtype=torch.float16)
        self.v = torch.zeros_like(self.k)

    # The reference exposes these as attributes.
    @property
    def pages(self) -> dict[int, list[int]]:
        return self.owner.pages

    @property
    def lengths(self) -> dict[int, int]:
        return self.owner.lengths

    @property
    def refcount(self) -> list[int]:
        return self.owner.refcount

    @property
    def free(self) -> list[int]:
        return self.owner.free

    def new(self, prefix_k: torch.Tensor, prefix_v: torch.Tensor) -> int:
        """Create one request from [tokens, KV heads, head dim] FP16 tensors."""
        if prefix_k.shape != prefix_v.shape or prefix_k.ndim != 3:
            raise ValueError("prefix K/V shapes must match [tokens, heads, dim]")
        if prefix_k.dtype != torch.float16 or prefix_k.device != self.k.device:
            raise ValueError("prefix must be FP16 on the cache device")
        if tuple(prefix_k.shape[1:]) != tuple(self.k.shape[2:]):
            raise ValueError("prefix head shape differs from cache")
        tokens = prefix_k.shape[0]
        request = self.owner.new(tokens)
        for i, page in enumerate(self.owner.pages[request]):
            n = min(16, tokens - 16 * i)
            self.k[page, :n].copy_(prefix_k[16 * i:16 * i + n])
            self.v[page, :n].copy_(prefix_v[16 * i:16 * i + n])
        return request

    def fork(self, source: int) -> int:
        return self.owner.fork(source)

    def checkpoint(self, request: int) -> Snapshot:
        return self.owner.checkpoint(request)

    def rollback(self, snapshot: Snapshot) -> None:
        self.owner.rollback(snapshot)

    def accept(self, snapshot: Snapshot) -> None:
        self.owner.accept(snapshot)

    def verify(self, request: int, q: torch.Tensor, draft_k: torch.Tensor,
               draft_v: torch.Tensor, parent: torch.Tensor) -> torch.Tensor:
        """Verify one request; draft inputs have leading batch dimension 1."""
        pages = self.owner.pages[request] or [0]  # unused when the prefix is empty
        dev = self.k.device
        page_table = torch.tensor([pages], device=dev, dtype=torch.int32)
        length = torch.tensor([self.owner.lengths[request]], device=dev, dtype=torch.int32)
        return tree_verify(q, self.k, self.v, page_table, length, draft_k, draft_v, parent)

    def commit(self, request: int, path: list[int], draft_k: torch.Tensor,
               draft_v: torch.Tensor) -> CommitPlan:
        """Append an accepted root-to-leaf path, preserving shared pages."""
        if not path or len(path) > draft_k.shape[1]:
            raise ValueError("path is empty or longer than draft")
        if draft_k.shape != draft_v.shape or draft_k.shape[0] != 1:
            raise ValueError("draft K/V must match and have batch size 1")
        if any(node < 0 or node >= draft_k.shape[1] for node in path):
            raise ValueError("path node out of range")
        plan = self.owner.plan_commit(request, len(path))
        dev = self.k.device
        if plan.cow is not None:
            old, fresh = plan.cow
            copy_pages_(self.k, self.v,
                        torch.tensor([old], device=dev, dtype=torch.int32),
                        torch.tensor([fresh], device=dev, dtype=torch.int32))
        commit_path_(self.k, self.v, draft_k, draft_v,
                     torch.tensor(path, device=dev, dtype=torch.int32),
                     torch.tensor(plan.dest_pages, device=dev, dtype=torch.int32),
                     torch.tensor(plan.dest_slots, device=dev, dtype=torch.int32), 0)
        return plan

    def commit_many(self, requests: list[int], paths: list[list[int]],
                    draft_k: torch.Tensor, draft_v: torch.Tensor) -> list[CommitPlan]:
        """Commit ``paths[i]`` of request ``requests[i]`` from ``draft_k[i]``.

        Plans are made in list order, as consecutive ``commit`` calls would
        make them.  All clones run first, then all accepted nodes: a page a
        clone reads is shared, so no commit in the batch writes it, and every
        commit target is either a fresh page or one its request owns alone.
        If the pool runs out part way, the plans made so far are still
        executed before the error is raised."""
        if len(requests) != len(paths) or len(set(requests)) != len(requests):
            raise ValueError("requests must be distinct and match paths")
        if draft_k.shape != draft_v.shape or draft_k.shape[0] != len(requests):
            raise ValueError("draft K/V must match and have one row per request")
        nodes = draft_k.shape[1]
        for path in paths:
            if not path or len(path) > nodes:
                raise ValueError("path is empty or longer than draft")
            if any(node < 0 or node >= nodes for node in path):
                raise ValueError("path node out of range")
        plans: list[CommitPlan] = []
        error = None
        for request, path in zip(requests, paths):
            try:
                plans.append(self.owner.plan_commit(request, len(path)))
            except RuntimeError as exc:  # pool exhausted: run what was planned
                error = exc
                break
        self._run_plans(plans, paths, draft_k, draft_v)
        if error is not None:
            raise error
        return plans

    def _run_plans(self, plans, paths, draft_k, draft_v) -> None:
        if not plans:
            return
        cows = [p.cow for p in plans if p.cow is not None]
        # copy_pages_ runs every pair at once: a destination must be fresh,
        # so distinct and never another pair's source (the page owner only
        # hands out free pages as clone targets).
        dsts = [fresh for _, fresh in cows]
        if len(set(dsts)) != len(dsts) or set(dsts) & {old for old, _ in cows}:
            raise RuntimeError("copy-on-write clones overlap")
        rows = [(i, node, page, slot) for i, (p, path) in enumerate(zip(plans, paths))
                for node, page, slot in zip(path, p.dest_pages, p.dest_slots)]
        flat = [x for c in cows for x in c] + [x for r in rows for x in r]
        idx = torch.tensor(flat, dtype=torch.int32).to(self.k.device)
        if cows:
            pairs = idx[:2 * len(cows)].view(-1, 2)
            copy_pages_(self.k, self.v, pairs[:, 0].contiguous(), pairs[:, 1].contiguous())
        table = idx[2 * len(cows):].view(-1, 4)
        commit_paths_(self.k, self.v, draft_k, draft_v, *(table[:, j].contiguous()
                                                          for j in range(4)))
