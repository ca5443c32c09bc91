"""Token -> expert routing permutation (oracle, test infrastructure only).

Restates ``experts4bit_qlora/engines/fast.py:125-133`` (and the identical block at
``:209-216``)::

    flat       = top_k_index.reshape(-1)
    order      = argsort(flat, stable=True)     # expert-grouped, ties in flat order
    token_rows = order // k
    top_pos    = order - token_rows * k
    counts     = bincount(flat, minlength=E)
    active     = nonzero(counts)                # ascending expert ids
    sizes      = counts[active]

plus the inverse permutation ``inv[order[r]] = r`` that the combine uses to find the sorted
row of a ``(token, slot)`` pair, and the exclusive prefix ``offsets`` of ``counts``.

The routers that produce ``top_k_index`` / ``top_k_weights`` (inputs of the path, not on it)
are restated by ``router_topk`` from ``experts4bit_qlora/engines/cpu_router.py:100-120``.
"""
from __future__ import annotations

import numpy as np


def route(top_k_index, num_experts: int) -> dict:
    idx = np.asarray(top_k_index, dtype=np.int64)
    if idx.ndim != 2:
        raise ValueError("top_k_index must be [tokens, k]")
    T, k = idx.shape
    flat = idx.reshape(-1)
    if flat.size and (flat.min() < 0 or flat.max() >= num_experts):
        raise ValueError("expert index out of range")
    order = np.argsort(flat, kind="stable").astype(np.int64)
    token_rows = order // k
    top_pos = order - token_rows * k
    counts = np.bincount(flat, minlength=num_experts).astype(np.int64)
    active = np.nonzero(counts)[0].astype(np.int64)
    offsets = np.zeros(num_experts + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(counts)
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size, dtype=np.int64)
    return {
        "order": order,
        "token_rows": token_rows,
        "top_pos": top_pos,
        "counts": counts,
        "active": active,
        "sizes": counts[active],
        "offsets": offsets,
        "inv": inv,
    }


def route_bruteforce(top_k_index, num_experts: int) -> np.ndarray:
    """Pure-Python stable counting sort; an independent check of ``route``'s ``order``."""
    flat = [int(v) for v in np.asarray(top_k_index).reshape(-1)]
    buckets: list[list[int]] = [[] for _ in range(num_experts)]
    for i, e in enumerate(flat):
        buckets[e].append(i)
    return np.array([i for b in buckets for i in b], dtype=np.int64)


def m_tiles(counts, tile_m: int):
    """The (expert, first sorted row) pairs of every ``tile_m``-row tile, experts ascending."""
    counts = np.asarray(counts, dtype=np.int64)
    off = np.concatenate([[0], np.cumsum(counts)])
    out = []
    for e, c in enumerate(counts):
        for t in range(-(-int(c) // tile_m)):
            out.append((e, int(off[e]) + t * tile_m))
    return out


SOFTMAX_THEN_TOPK = "softmax_then_topk"  # OLMoE / Qwen3-MoE (cpu_router.py:63-67)
TOPK_THEN_SOFTMAX = "topk_then_softmax"  # gpt-oss


def router_topk(logits, k: int, kind: str = SOFTMAX_THEN_TOPK, renorm: bool = False):
    """The routing epilogue in fp32 (``cpu_router.py:100-120``): top-k by a stable descending
    sort (ties to the lower expert index, ``deterministic_topk`` at ``:100-105``); for
    ``softmax_then_topk`` the weights are the softmax over ALL logits gathered at the top-k
    (renormalised over the k when ``renorm``), for ``topk_then_softmax`` the softmax over the k
    selected logits. Returns ``(weights [T, k] fp32, indices [T, k] int64)``."""
    z = np.asarray(logits, dtype=np.float32)
    order = np.argsort(-z, axis=-1, kind="stable")[:, :k].astype(np.int64)
    top = np.take_along_axis(z, order, axis=-1)

    def softmax(v):
        e = np.exp((v - v.max(axis=-1, keepdims=True)).astype(np.float32)).astype(np.float32)
        return (e / e.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)

    if kind == SOFTMAX_THEN_TOPK:
        w = np.take_along_axis(softmax(z), order, axis=-1)
        if renorm:
            w = (w / w.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    elif kind == TOPK_THEN_SOFTMAX:
        w = softmax(top)
    else:
        raise ValueError(f"unknown router kind {kind!r}")
    return w.astype(np.float32), order
