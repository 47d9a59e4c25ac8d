"""Floating-point restatement of TriangleMix paged GQA masked attention.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference sources restated here:

* paged gather + per-row masked softmax (torch, fp32) ....
  operator/tests/triangle_v2_reference.py:490-587 (``torch_reference_attention``)
* the same in pure arithmetic ..............................
  operator/tests/triangle_v2_reference.py:374-434 (``reference_attention_python``)
* joint and online softmax ..................................
  operator/tests/triangle_v2_reference.py:304-371,
  operator/tests/test_boundary_mask_alignment_design.py:274-300

Semantics: query ``[Tq, 32, 128]``, K/V caches ``[pages, 128, 8, 128]``
(BSND pages), block table ``[1, >= ceil(seq_len/128)]``; query head ``h``
reads KV head ``h // 4``; row ``query_start + r`` attends the keys of
``geometry.selected_intervals``; one softmax over all of them.

How it is pinned (tests/test_oracle_attention.py):

* the reference's two sentinels (joint-softmax value (8*10+513)/521 at q=521
  with a poisoned token 8; GQA head -> KV-head map [1,1,1,1,2,...,8]);
* closed form for Q = 0: every row equals the mean of V over its selected
  keys (computed from the set-builder mask, so a dropped or extra key fails);
* a library routine: ``torch.nn.functional.scaled_dot_product_attention``
  with an explicit boolean mask on an identity page table;
* page-permutation invariance; float64 numpy vs float32 torch agreement;
* online softmax over split blocks == joint softmax; a fully masked
  non-first block leaves the online state unchanged.
"""

from __future__ import annotations

import math
from typing import Iterable, Sequence

import numpy as np

from . import geometry as G


# --------------------------------------------------------------------------
# softmax restatements (triangle_v2_reference.py:304-371)
# --------------------------------------------------------------------------

def joint_softmax_weighted_sum(scores: Sequence[float], values: Sequence[Sequence[float]]) -> list[float]:
    if not scores or len(scores) != len(values):
        raise ValueError("scores and values must be non-empty and equal length")
    m = max(float(s) for s in scores)
    w = [math.exp(float(s) - m) for s in scores]
    den = math.fsum(w)
    dim = len(values[0])
    return [math.fsum(wi * float(v[i]) for wi, v in zip(w, values)) / den for i in range(dim)]


def online_softmax_weighted_sum(blocks: Iterable[tuple[Sequence[float], Sequence[Sequence[float]]]]) -> list[float]:
    """One (max, sum, accumulator) state carried across all blocks.

    Masked entries may be given as ``-inf`` or as the finite -3.4028e38 the
    reference kernel writes (block_epilogue_online_softmax.hpp:147 under
    operator/op_kernel/vendor/cann_9_0_1/block_sparse_attention/attn_infra/
    epilogue/block/); either contributes 0.
    """
    m = -math.inf
    l = 0.0
    acc: list[float] | None = None
    for scores, values in blocks:
        if not scores:
            continue
        dim = len(values[0])
        if acc is None:
            acc = [0.0] * dim
        bm = max(float(s) for s in scores)
        nm = max(m, bm)
        corr = 0.0 if m == -math.inf else math.exp(m - nm)
        w = [math.exp(float(s) - nm) for s in scores]
        acc = [acc[i] * corr + math.fsum(wi * float(v[i]) for wi, v in zip(w, values)) for i in range(dim)]
        l = l * corr + math.fsum(w)
        m = nm
    if acc is None or l == 0.0:
        raise ValueError("online softmax needs at least one finite score")
    return [a / l for a in acc]


# --------------------------------------------------------------------------
# paged gather
# --------------------------------------------------------------------------

def _logical_cache_np(cache: np.ndarray, block_table: np.ndarray, seq_len: int) -> np.ndarray:
    pages = -(-seq_len // G.PAGE_SIZE)
    table = np.asarray(block_table).reshape(-1)[:pages].astype(np.int64)
    if table.size < pages:
        raise ValueError("block_table does not cover seq_len")
    if (table < 0).any():
        raise ValueError("negative physical page")
    return cache[table].reshape(-1, G.KV_HEADS, G.HEAD_DIM)[:seq_len]


def attention_np(query: np.ndarray, key_cache: np.ndarray, value_cache: np.ndarray,
                 block_table: np.ndarray, query_start: int, seq_len: int,
                 prompt_len: int, scale: float, *, dense: bool = False) -> np.ndarray:
    """float64 paged masked GQA attention; ``dense=True`` gives plain causal.

    Inputs are float arrays holding the bf16 values (use ``.float().numpy()``
    on the bf16 tensors).  Returns float64 ``[Tq, 32, 128]``.
    """
    tq = query.shape[0]
    if query_start + tq > seq_len:
        raise ValueError("query rows extend beyond seq_len")
    lk = _logical_cache_np(key_cache, block_table, seq_len).astype(np.float64)
    lv = _logical_cache_np(value_cache, block_table, seq_len).astype(np.float64)
    q64 = query.astype(np.float64).reshape(tq, G.KV_HEADS, G.GROUP, G.HEAD_DIM)
    out = np.empty((tq, G.QUERY_HEADS, G.HEAD_DIM), dtype=np.float64)
    for r in range(tq):
        q = query_start + r
        if dense:
            ivs = ((0, min(q + 1, seq_len)),)
        else:
            ivs = G.selected_intervals(q, seq_len, prompt_len)
        idx = np.concatenate([np.arange(b, e) for b, e in ivs])
        k = lk[idx]  # [n, 8, 128]
        v = lv[idx]
        s = np.einsum("gjd,ngd->gjn", q64[r], k) * scale
        s -= s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        out[r] = np.einsum("gjn,ngd->gjd", p, v).reshape(G.QUERY_HEADS, G.HEAD_DIM)
    return out


def attention_torch(query, key_cache, value_cache, block_table, query_start: int,
                    seq_len: int, prompt_len: int, scale: float, *, dense: bool = False):
    """float32 PyTorch CPU restatement of ``torch_reference_attention``.

    One row at a time: gather the row's selected logical keys through the
    block table, one softmax over all of them in fp32, weighted sum of V
    (triangle_v2_reference.py:539-587).  Returns fp32 ``[Tq, 32, 128]``.
    This is also the timed CPU baseline of ``bench.py``.
    """
    import torch

    tq = query.shape[0]
    if query_start + tq > seq_len:
        raise ValueError("query rows extend beyond seq_len")
    pages = -(-seq_len // G.PAGE_SIZE)
    table = block_table.reshape(-1).to(device="cpu", dtype=torch.int64)
    if table.numel() < pages:
        raise ValueError("block_table does not cover seq_len")
    table = table[:pages]
    lk = key_cache.index_select(0, table).float().reshape(-1, G.KV_HEADS, G.HEAD_DIM)[:seq_len]
    lv = value_cache.index_select(0, table).float().reshape(-1, G.KV_HEADS, G.HEAD_DIM)[:seq_len]
    qf = query.float()
    out = torch.empty_like(qf)
    for r in range(tq):
        q = query_start + r
        ivs = ((0, min(q + 1, seq_len)),) if dense else G.selected_intervals(q, seq_len, prompt_len)
        parts = [torch.arange(b, e, dtype=torch.int64) for b, e in ivs]
        idx = parts[0] if len(parts) == 1 else torch.cat(parts)
        k = lk.index_select(0, idx)
        v = lv.index_select(0, idx)
        gq = qf[r].reshape(G.KV_HEADS, G.GROUP, G.HEAD_DIM)
        s = torch.einsum("gjd,ngd->gjn", gq, k)
        p = torch.softmax(s * float(scale), dim=-1)
        out[r] = torch.einsum("gjn,ngd->gjd", p, v).reshape(G.QUERY_HEADS, G.HEAD_DIM)
    return out


def attended_mask(rows, keys, seq_len: int, prompt_len: int, *, dense: bool = False):
    """Boolean ``[len(rows), len(keys)]``: key ``k`` attended by row ``q``.

    The rule of ``geometry.selected_intervals`` written as a predicate
    (triangle_v2_reference.py:193-232): ``k < min(q + 1, seq_len)`` and, for a
    sparse row (``521 <= q < max(0, prompt_len - 128)``), ``k < 8`` or
    ``k >= q - 512``.  ``rows`` and ``keys`` are int64 torch tensors.
    """
    q = rows.reshape(-1, 1)
    k = keys.reshape(1, -1)
    keep = k < (q + 1).clamp(max=seq_len)
    if dense:
        return keep
    sparse_end = max(0, prompt_len - G.DENSE_TAIL)
    sparse = (q >= G.SPARSE_BEGIN) & (q < sparse_end)
    return keep & (~sparse | (k < G.SINK) | (k >= q - G.WINDOW))


def attention_torch_blocked(query, key_cache, value_cache, block_table, query_start: int, seq_len: int,
                            prompt_len: int, scale: float, *, dense: bool = False, device=None,
                            max_scores: int = 1 << 26):
    """float32 restatement of ``torch_reference_attention`` over blocks of rows, on any torch device.

    The same softmax as ``attention_torch`` (one softmax in fp32 over each
    row's selected keys, then the weighted sum of V), computed for a block of
    rows at once: the block gathers the keys any of its rows may attend --
    ``[0, 8)`` plus ``[first_row - 512, last_row]`` when every row is sparse,
    ``[0, last_row]`` otherwise -- and masks each row with ``attended_mask``.
    Blocks hold at most ``max_scores`` scores.  Inputs may live on the CPU;
    the work runs on ``device`` (default: the query's).  Returns fp32
    ``[Tq, 32, 128]`` on that device.  Pinned against ``attention_torch`` and
    ``attention_np`` (tests/test_oracle_attention.py).
    """
    import torch

    dev = torch.device(device) if device is not None else query.device
    tq = query.shape[0]
    if query_start + tq > seq_len:
        raise ValueError("query rows extend beyond seq_len")
    pages = -(-seq_len // G.PAGE_SIZE)
    table = block_table.reshape(-1).to(device=dev, dtype=torch.int64)
    if table.numel() < pages:
        raise ValueError("block_table does not cover seq_len")
    table = table[:pages]
    # logical K as [8, 128, seq] and V as [8, seq, 128], fp32: a block's keys are slices of them
    kt = key_cache.to(dev).index_select(0, table).reshape(-1, G.KV_HEADS, G.HEAD_DIM)[:seq_len]
    kt = kt.float().permute(1, 2, 0).contiguous()
    vt = value_cache.to(dev).index_select(0, table).reshape(-1, G.KV_HEADS, G.HEAD_DIM)[:seq_len]
    vt = vt.float().permute(1, 0, 2).contiguous()
    qf = query.to(dev).float().reshape(tq, G.KV_HEADS, G.GROUP, G.HEAD_DIM)
    out = torch.empty(tq, G.QUERY_HEADS, G.HEAD_DIM, dtype=torch.float32, device=dev)
    sparse_end = max(0, prompt_len - G.DENSE_TAIL)
    r = 0
    while r < tq:
        q0 = query_start + r
        rows = tq - r
        while rows > 1 and rows * G.QUERY_HEADS * min(q0 + rows, seq_len) > max_scores:
            rows = (rows + 1) // 2
        q1 = query_start + r + rows  # rows [q0, q1)
        if not dense and q0 >= G.SPARSE_BEGIN and q1 <= sparse_end:  # every row sparse
            lo = max(G.SINK, q0 - G.WINDOW)
            keys = torch.cat([torch.arange(0, G.SINK, device=dev), torch.arange(lo, q1, device=dev)])
            k = torch.cat([kt[:, :, :G.SINK], kt[:, :, lo:q1]], dim=2)
            v = torch.cat([vt[:, :G.SINK], vt[:, lo:q1]], dim=1)
        else:
            hi = min(q1, seq_len)
            keys = torch.arange(0, hi, device=dev)
            k, v = kt[:, :, :hi], vt[:, :hi]
        qb = qf[r:r + rows].permute(1, 0, 2, 3).reshape(G.KV_HEADS, rows * G.GROUP, G.HEAD_DIM)
        s = torch.bmm(qb, k).reshape(G.KV_HEADS, rows, G.GROUP, -1)  # [8, rows, 4, n]
        mask = attended_mask(torch.arange(q0, q1, device=dev), keys, seq_len, prompt_len, dense=dense)
        s = s.masked_fill(~mask.reshape(1, rows, 1, -1), float("-inf"))
        p = torch.softmax(s * float(scale), dim=-1).reshape(G.KV_HEADS, rows * G.GROUP, -1)
        o = torch.bmm(p, v).reshape(G.KV_HEADS, rows, G.GROUP, G.HEAD_DIM)
        out[r:r + rows] = o.permute(1, 0, 2, 3).reshape(rows, G.QUERY_HEADS, G.HEAD_DIM)
        r += rows
    return out


def error_metrics(actual, expected) -> dict:
    """max/mean abs and relative L2 (npu_v2_correctness.py:298-314)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    d = np.abs(a - e)
    return {
        "finite": bool(np.isfinite(a).all() and np.isfinite(e).all()),
        "max_abs": float(d.max()) if d.size else 0.0,
        "mean_abs": float(d.mean()) if d.size else 0.0,
        "relative_l2": float(np.linalg.norm(d) / max(np.linalg.norm(e), 1e-12)),
    }
