"""Device-side ownership of the ``.out`` ops' output buffer.

Restates the reference's device check (operator/tests/npu_adapter_out_correctness.py:26-141;
contract in operator/tests/test_adapter_out_contract.py:197-220) on MI355X, for
the sparse ``.out`` op, its in-tree alias ``npu_triangle_paged_sparse_attention``
and the dense companion's ``.out``:

* ``out`` is a contiguous view with a nonzero storage offset inside a buffer
  whose first and last rows are guards (17.0) and whose body is pre-filled
  (-31.0);
* the op returns the very tensor it was given (same data pointer, same
  storage offset), writes exactly the functional op's result into it, and
  leaves both guard rows untouched;
* ``out`` aliasing ``query`` is refused with a RuntimeError before any launch.

The case is the reference's: rows 766..800 of a 2048-token prompt (ragged,
crossing pages), seed 3101.
"""

from __future__ import annotations

import pytest
import torch

from trianglemix.workload import SCALE, make_inputs

pytestmark = pytest.mark.gpu

QS, TQ, SEQ, PROMPT, SEED = 766, 35, 801, 2048, 3101


def _inputs(gpu):
    q, k, v, bt = make_inputs(QS, TQ, SEQ, SEED)
    return q.to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu)


def _guarded(q):
    guarded = torch.full((TQ + 2, 32, 128), 17.0, dtype=torch.bfloat16, device=q.device)
    out = guarded[1:-1]
    out.fill_(-31.0)
    assert out.is_contiguous() and out.storage_offset() > 0
    return guarded, out


def _check(guarded, out, returned, expected, ptr, offset):
    torch.cuda.synchronize()
    assert returned.data_ptr() == ptr and out.data_ptr() == ptr
    assert returned.storage_offset() == offset
    assert torch.equal(out, expected)
    assert torch.all(guarded[0] == 17.0) and torch.all(guarded[-1] == 17.0)


def test_sparse_out_and_alias_respect_caller_buffer(gpu):
    q, k, v, bt = _inputs(gpu)
    expected = torch.ops.trianglemix_reference.triangle_paged_sparse_attention(q, k, v, bt, QS, SEQ, PROMPT, SCALE)
    for name in ("out", "alias"):
        guarded, out = _guarded(q)
        ptr, offset = out.data_ptr(), out.storage_offset()
        if name == "out":
            returned = torch.ops.trianglemix.triangle_paged_sparse_attention.out(
                q, k, v, bt, QS, SEQ, PROMPT, SCALE, out=out)
        else:
            returned = torch.ops.trianglemix.npu_triangle_paged_sparse_attention(
                q, k, v, bt, QS, SEQ, PROMPT, SCALE, out)
        _check(guarded, out, returned, expected, ptr, offset)


def test_dense_out_respects_caller_buffer(gpu):
    q, k, v, bt = _inputs(gpu)
    expected = torch.ops.trianglemix_reference.dense_paged_causal_attention(q, k, v, bt, QS, SEQ, SCALE)
    guarded, out = _guarded(q)
    ptr, offset = out.data_ptr(), out.storage_offset()
    returned = torch.ops.trianglemix.dense_paged_causal_attention.out(q, k, v, bt, QS, SEQ, SCALE, out=out)
    _check(guarded, out, returned, expected, ptr, offset)


def test_out_aliasing_query_is_refused(gpu):
    q, k, v, bt = _inputs(gpu)
    before = q.clone()
    with pytest.raises(RuntimeError):
        torch.ops.trianglemix.triangle_paged_sparse_attention.out(q, k, v, bt, QS, SEQ, PROMPT, SCALE, out=q)
    with pytest.raises(RuntimeError):
        torch.ops.trianglemix.npu_triangle_paged_sparse_attention(q, k, v, bt, QS, SEQ, PROMPT, SCALE, q)
    with pytest.raises(RuntimeError):
        torch.ops.trianglemix.dense_paged_causal_attention.out(q, k, v, bt, QS, SEQ, SCALE, out=q)
    # a view of out that overlaps query through a shared buffer is refused as well
    buf = torch.empty((2 * TQ, 32, 128), dtype=torch.bfloat16, device=gpu)
    buf[:TQ].copy_(q)
    with pytest.raises(RuntimeError):
        torch.ops.trianglemix.triangle_paged_sparse_attention.out(buf[:TQ], k, v, bt, QS, SEQ, PROMPT, SCALE,
                                                                   out=buf[TQ // 2:TQ // 2 + TQ])
    torch.cuda.synchronize()
    assert torch.equal(q, before)  # nothing was launched
