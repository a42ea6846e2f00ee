"""Host-side page owner (branchcraft_torch.pages.PageOwner) on the CPU.

Pins the reference transaction's bookkeeping
(python/branchcraft_torch/transaction.py:23-150 and
tests/test_transaction.py:8-29): ascending LIFO allocation, copy-on-write of
a shared partial page, destination page/slot math, rollback and accept.
A seeded random-operation stress test then checks, after every step, that
each live request reads back exactly the tokens it was given, that forks and
snapshots are isolated, and that refcounts and the free list agree.
"""

import random

import pytest

from branchcraft_torch.pages import PAGE_SIZE, PageOwner


def test_reference_transaction_plan():
    own = PageOwner(8)
    original = own.new(19)
    assert own.pages[original] == [0, 1]  # pages come out ascending
    sibling = own.fork(original)
    snap = own.checkpoint(original)
    plan = own.plan_commit(original, 3)
    assert plan.cow == (1, 2)  # shared partial page cloned into fresh page 2
    assert plan.dest_pages == [2, 2, 2] and plan.dest_slots == [3, 4, 5]
    assert own.lengths[original] == 22
    assert own.pages[original] == [0, 2] and own.pages[sibling] == [0, 1]
    own.rollback(snap)
    assert own.pages[original] == [0, 1] and own.lengths[original] == 19
    own.check_invariants()
    assert own.free[-1] == 2  # the clone went back on top of the LIFO stack
    assert own.alloc() == 2


def test_commit_without_sharing_writes_in_place_and_grows():
    own = PageOwner(4)
    r = own.new(30)  # pages [0, 1], 14 slots used in page 1
    plan = own.plan_commit(r, 5)  # fills page 1 (2 slots), spills 3 into page 2
    assert plan.cow is None
    assert plan.dest_pages == [1, 1, 2, 2, 2] and plan.dest_slots == [14, 15, 0, 1, 2]
    assert own.pages[r] == [0, 1, 2]
    own.check_invariants()


def test_full_last_page_is_never_cloned():
    own = PageOwner(6)
    r = own.new(32)
    own.fork(r)
    plan = own.plan_commit(r, 1)
    assert plan.cow is None and plan.dest_pages == [2] and plan.dest_slots == [0]


def test_exhaustion_leaves_state_unchanged():
    own = PageOwner(3)
    r = own.new(40)  # 3 pages
    with pytest.raises(RuntimeError):
        own.new(1)
    before = (list(own.pages[r]), own.lengths[r], list(own.refcount), list(own.free))
    with pytest.raises(RuntimeError):
        own.plan_commit(r, 16)
    assert (own.pages[r], own.lengths[r], own.refcount, own.free) == \
        (before[0], before[1], before[2], before[3])


def test_snapshot_consumed_once():
    own = PageOwner(4)
    r = own.new(5)
    snap = own.checkpoint(r)
    own.accept(snap)
    with pytest.raises(RuntimeError):
        own.accept(snap)
    with pytest.raises(RuntimeError):
        own.rollback(snap)
    own.check_invariants()


def test_bad_arguments():
    with pytest.raises(ValueError):
        PageOwner(0)
    own = PageOwner(2)
    with pytest.raises(ValueError):
        own.new(-1)
    r = own.new(3)
    with pytest.raises(ValueError):
        own.plan_commit(r, 0)


class Model:
    """Token-level simulation: cache[page][slot] holds a token id; every
    request must read back exactly its own token list."""

    def __init__(self, own: PageOwner):
        self.own = own
        self.cache = [[None] * PAGE_SIZE for _ in range(own.physical_pages)]
        self.tokens: dict[int, list] = {}
        self.snaps = []  # (snapshot, tokens at checkpoint)

    def apply(self, request, plan, new_tokens):
        if plan.cow is not None:
            old, fresh = plan.cow
            self.cache[fresh] = list(self.cache[old])
        for tok, p, s in zip(new_tokens, plan.dest_pages, plan.dest_slots):
            self.cache[p][s] = tok

    def read(self, request):
        n = self.own.lengths[request]
        pages = self.own.pages[request]
        return [self.cache[pages[t // PAGE_SIZE]][t % PAGE_SIZE] for t in range(n)]


@pytest.mark.parametrize("seed", range(6))
def test_random_transaction_stress(seed):
    rnd = random.Random(seed)
    own = PageOwner(48)
    model = Model(own)
    counter = 0
    for _ in range(600):
        op = rnd.choice(["new", "fork", "checkpoint", "commit", "commit", "rollback", "accept"])
        live = list(model.tokens)
        try:
            if op == "new" or not live:
                n = rnd.randrange(0, 40)
                r = own.new(n)
                plan_tokens = [f"t{counter + i}" for i in range(n)]
                counter += n
                # new() fills pages in order
                for i, tok in enumerate(plan_tokens):
                    model.cache[own.pages[r][i // PAGE_SIZE]][i % PAGE_SIZE] = tok
                model.tokens[r] = plan_tokens
            elif op == "fork":
                src = rnd.choice(live)
                r = own.fork(src)
                model.tokens[r] = list(model.tokens[src])
            elif op == "checkpoint":
                r = rnd.choice(live)
                model.snaps.append((own.checkpoint(r), list(model.tokens[r])))
            elif op == "commit":
                r = rnd.choice(live)
                k = rnd.randrange(1, 8)
                new = [f"t{counter + i}" for i in range(k)]
                counter += k
                plan = own.plan_commit(r, k)
                model.apply(r, plan, new)
                model.tokens[r] = model.tokens[r] + new
            elif op in ("rollback", "accept") and model.snaps:
                snap, toks = model.snaps.pop(rnd.randrange(len(model.snaps)))
                if op == "rollback":
                    own.rollback(snap)
                    model.tokens[snap.request] = toks
                else:
                    own.accept(snap)
        except RuntimeError as e:
            assert "exhausted" in str(e)
        own.check_invariants()
        for r, toks in model.tokens.items():
            assert model.read(r) == toks, f"request {r} corrupted after {op}"
