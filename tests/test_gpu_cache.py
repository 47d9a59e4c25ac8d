"""GPU parity of the paged KV write (``tm_reshape_and_cache``) against the CPU oracle.

Bit-exact (it only moves bf16 rows): the caches after the kernel must equal,
bit for bit, the caches after ``oracle.cache.reshape_and_cache`` on the same
inputs.  Cases: a permuted slot mapping with padding (-1) and out-of-range
slots, row-strided K / V taken from a fused QKV buffer, an empty chunk, the
torch op against the C ABI, and a chunked prefill whose pages are filled by
the kernel chunk by chunk, which must attend exactly like pre-filled pages.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import cache as OC
from trianglemix import cabi
from trianglemix.workload import SCALE, make_cache, make_query, prompt_chunks

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


def _oracle(key, value, kc, vc, slots):
    """The oracle's scatter on the bf16 bit patterns (it moves rows verbatim)."""
    kc_o, vc_o = kc.clone(), vc.clone()
    kk, vv = kc_o.view(torch.int16).numpy(), vc_o.view(torch.int16).numpy()
    OC.reshape_and_cache(key.contiguous().view(torch.int16).numpy(), value.contiguous().view(torch.int16).numpy(),
                         kk, vv, slots)
    return kc_o, vc_o


@pytest.mark.parametrize("tokens,pages,seed", [(512, 12, 1), (77, 3, 2), (1, 1, 3)])
def test_scatter_matches_oracle_bit_exact(gpu, tokens, pages, seed):
    print(f"kv write tokens={tokens} pages={pages} seed={seed}", flush=True)
    g = torch.Generator().manual_seed(seed)
    key = torch.randn(tokens, 8, 128, generator=g).to(torch.bfloat16)
    value = torch.randn(tokens, 8, 128, generator=g).to(torch.bfloat16)
    kc = torch.randn(pages, 128, 8, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(pages, 128, 8, 128, generator=g).to(torch.bfloat16)
    slots = torch.randperm(pages * 128, generator=g)[:tokens].to(torch.int64)
    if tokens > 8:
        slots[3] = -1                  # padding
        slots[5] = pages * 128 + 17    # past the cache: skipped
    want_k, want_v = _oracle(key, value, kc, vc, slots.numpy())
    kd, vd = kc.to(gpu), vc.to(gpu)
    cabi.reshape_and_cache(key.to(gpu), value.to(gpu), kd, vd, slots.to(gpu))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(kd), _bits(want_k))
    assert np.array_equal(_bits(vd), _bits(want_v))


def test_strided_rows_from_fused_qkv(gpu):
    g = torch.Generator().manual_seed(7)
    tokens, pages = 300, 4
    qkv = torch.randn(tokens, 48, 128, generator=g).to(torch.bfloat16)  # 32 query + 8 key + 8 value heads
    key, value = qkv[:, 32:40], qkv[:, 40:48]
    kc = torch.zeros(pages, 128, 8, 128, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    slots = torch.arange(tokens, dtype=torch.int64) * 3 % (pages * 128)
    slots = torch.unique(slots)[:tokens]
    key, value = key[: slots.numel()], value[: slots.numel()]
    want_k, want_v = _oracle(key, value, kc, vc, slots.numpy())
    qkv_d = qkv.to(gpu)
    kd, vd = kc.to(gpu), vc.to(gpu)
    n = slots.numel()
    cabi.reshape_and_cache(qkv_d[:n, 32:40], qkv_d[:n, 40:48], kd, vd, slots.to(gpu))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(kd), _bits(want_k))
    assert np.array_equal(_bits(vd), _bits(want_v))


def test_empty_chunk_and_torch_op(gpu):
    g = torch.Generator().manual_seed(9)
    kc = torch.randn(2, 128, 8, 128, generator=g).to(torch.bfloat16).to(gpu)
    vc = torch.randn(2, 128, 8, 128, generator=g).to(torch.bfloat16).to(gpu)
    before_k, before_v = _bits(kc), _bits(vc)
    empty = torch.empty(0, 8, 128, dtype=torch.bfloat16, device=gpu)
    torch.ops.trianglemix.reshape_and_cache(empty, empty, kc, vc, torch.empty(0, dtype=torch.int64, device=gpu))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(kc), before_k) and np.array_equal(_bits(vc), before_v)
    key = torch.randn(40, 8, 128, generator=g).to(torch.bfloat16)
    value = torch.randn(40, 8, 128, generator=g).to(torch.bfloat16)
    slots = torch.randperm(256, generator=g)[:40].to(torch.int64)
    k2, v2 = kc.clone(), vc.clone()
    torch.ops.trianglemix.reshape_and_cache(key.to(gpu), value.to(gpu), kc, vc, slots.to(gpu))
    cabi.reshape_and_cache(key.to(gpu), value.to(gpu), k2, v2, slots.to(gpu))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(kc), _bits(k2)) and np.array_equal(_bits(vc), _bits(v2))
    with pytest.raises(RuntimeError, match="INT64"):
        torch.ops.trianglemix.reshape_and_cache(key.to(gpu), value.to(gpu), kc, vc, slots.to(torch.int32).to(gpu))


def test_chunked_prefill_with_written_pages_attends_like_prefilled(gpu):
    """Config-2 order at L=2048: before each chunk, write its K/V into its pages, then attend."""
    L, chunk = 2048, 512
    k_full, v_full, bt = make_cache(L, 11)
    q_full = make_query(L, 12)
    btd = bt.to(gpu)
    kd_ref, vd_ref = k_full.to(gpu), v_full.to(gpu)
    kd = torch.zeros_like(kd_ref)
    vd = torch.zeros_like(vd_ref)
    # the fresh K/V of each token, in logical order (as a model would produce them)
    table = bt[0].tolist()
    logical = torch.tensor([table[t // 128] * 128 + t % 128 for t in range(L)], dtype=torch.int64)
    k_tokens = k_full.view(-1, 8, 128)[logical]
    v_tokens = v_full.view(-1, 8, 128)[logical]
    for c in prompt_chunks(L, chunk):
        n = c.query_tokens
        slots = torch.from_numpy(OC.chunk_slots(bt, c.query_start, n))
        cabi.reshape_and_cache(k_tokens[c.query_start:c.seq_len].to(gpu), v_tokens[c.query_start:c.seq_len].to(gpu),
                               kd, vd, slots.to(gpu))
        q = q_full[c.query_start:c.seq_len].to(gpu)
        out_written = torch.empty_like(q)
        out_ref = torch.empty_like(q)
        cabi.triangle_paged_sparse_attention(q, kd, vd, btd, out_written, query_start=c.query_start,
                                             seq_len=c.seq_len, prompt_len=L, scale=SCALE)
        cabi.triangle_paged_sparse_attention(q, kd_ref, vd_ref, btd, out_ref, query_start=c.query_start,
                                             seq_len=c.seq_len, prompt_len=L, scale=SCALE)
        torch.cuda.synchronize()
        print(f"chunk {c.query_start}..{c.seq_len}", flush=True)
        assert np.array_equal(_bits(out_written), _bits(out_ref))
