"""PyTorch dispatcher ops for Branchcraft's MI355X (gfx950) kernels.

Importing this module loads ``_C.so`` (built in-tree by
``branchcraft-cuda_amd/build.py``) which registers ``torch.ops.branchcraft``
with the reference's schemas (bindings/torch_ops.cpp:144-148 of
Haaziq386/branchcraft-cuda) plus ``paged_decode`` (the reference's C++
``branchcraft::decode``), ``copy_pages_`` and ``commit_paths_``.  There is
no CPU or Python fallback: a missing extension raises ImportError, and the
ops have only a GPU implementation.

FakeTensor implementations follow python/branchcraft_torch/__init__.py:18-31
of the reference so that ``torch.compile`` can trace the ops.
"""

from pathlib import Path

import torch

_library = Path(__file__).with_name("_C.so")
if not _library.exists():
    raise ImportError(
        "Branchcraft HIP extension is missing; run `python branchcraft-cuda_amd/build.py`")
torch.ops.load_library(str(_library))
LIBRARY_PATH = str(_library)


@torch.library.register_fake("branchcraft::tree_verify")
def _fake_tree_verify(q, prefix_k, prefix_v, pages, lengths, draft_k, draft_v, parent):
    return q.new_empty(q.shape, dtype=torch.float32)


@torch.library.register_fake("branchcraft::packed_decode_out")
def _fake_packed_decode_out(q, packed_kv, pages, lengths, output, scale):
    return output


@torch.library.register_fake("branchcraft::paged_decode")
def _fake_paged_decode(q, k, v, pages, lengths, splits=0):
    return q.new_empty(q.shape, dtype=torch.float32)


@torch.library.register_fake("branchcraft::commit_path_")
def _fake_commit_path(cache_k, cache_v, draft_k, draft_v, path_nodes, dest_pages,
                      dest_slots, request):
    return None


@torch.library.register_fake("branchcraft::copy_pages_")
def _fake_copy_pages(cache_k, cache_v, src_pages, dst_pages):
    return None


@torch.library.register_fake("branchcraft::commit_paths_")
def _fake_commit_paths(cache_k, cache_v, draft_k, draft_v, requests, path_nodes,
                       dest_pages, dest_slots):
    return None


def tree_verify(q, prefix_k, prefix_v, pages, lengths, draft_k, draft_v, parent):
    """FP32 [batch, node, query head, dim] outputs; every node attends to its
    request's paged prefix and its own ancestor chain (itself included)."""
    return torch.ops.branchcraft.tree_verify(
        q, prefix_k, prefix_v, pages, lengths, draft_k, draft_v, parent)


def packed_decode_out(q, packed_kv, pages, lengths, output, scale):
    """Decode into a preallocated FP16 output (safe for HIP graph capture).

    ``packed_kv`` is the logical [pages, kv_heads, 16, 2*dim] view of a vLLM
    cache (any outer strides) or a [pages, 2, 16, kv_heads, dim] tensor."""
    return torch.ops.branchcraft.packed_decode_out(
        q, packed_kv, pages, lengths, output, scale)


def paged_decode(q, k, v, pages, lengths, splits=0):
    """Paged GQA decode (the reference's C++ ``branchcraft::decode``): FP32
    [batch, query head, dim] output over K/V pages [P, 16, kv_heads, dim].
    ``splits=0`` picks the split count from the shape (no host sync)."""
    return torch.ops.branchcraft.paged_decode(q, k, v, pages, lengths, splits)


def commit_path_(cache_k, cache_v, draft_k, draft_v, path_nodes, dest_pages,
                 dest_slots, request):
    """Write accepted draft K/V to preallocated physical destinations."""
    return torch.ops.branchcraft.commit_path_(
        cache_k, cache_v, draft_k, draft_v, path_nodes, dest_pages, dest_slots, request)


def copy_pages_(cache_k, cache_v, src_pages, dst_pages):
    """Clone whole pages (K and V): cache[dst[i]] <- cache[src[i]].  All
    pairs copy at once: destinations must be distinct and none may also be
    a source."""
    return torch.ops.branchcraft.copy_pages_(cache_k, cache_v, src_pages, dst_pages)


def commit_paths_(cache_k, cache_v, draft_k, draft_v, requests, path_nodes, dest_pages,
                  dest_slots):
    """Commit the accepted nodes of several requests in one launch: entry i
    writes draft[requests[i], path_nodes[i]] to (dest_pages[i], dest_slots[i])."""
    return torch.ops.branchcraft.commit_paths_(
        cache_k, cache_v, draft_k, draft_v, requests, path_nodes, dest_pages, dest_slots)


__all__ = ["tree_verify", "packed_decode_out", "paged_decode",
           "commit_path_", "copy_pages_", "commit_paths_", "LIBRARY_PATH"]
