"""The one-launch plan + pooling of small batches (k_plan_pool, used by the
whole-operator entry points for 16-bit inputs and at most 16 sequences)
against the separate k_plan and k_pool launches of the staged entry points
(fp_plan, fp_pool_k), through the C ABI on the same inputs:

* sequence tables, status word, chunk-unit records and the unit count equal;
* work items equal as a set and in heaviest-first level order (the order of
  equal levels is free: k_plan places them by LDS atomics);
* pooled K bit-equal (both are fp64 sums rounded through fp32), and equal to
  the oracle's pooling;
* the selection and output of the whole call equal to the staged call's.

Cases: one sequence (4K with split rows, partial last block), ragged batches
with zero-length sequences, the uniform (batched) layout, block 64, d = 64,
fp16, 16 sequences (the largest batch planned inside the pooling launch),
bad cu_seqlens (status flags) and 17 sequences (separate launches)."""

import pytest
import torch

from flashprefill_amd.runtime import FlashPrefillCall
from oracle import flashprefill_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _inputs(T, hq, hkv, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(T, hq, d, generator=g) * 1.5).to(dtype)
    k = (torch.randn(T, hkv, d, generator=g) * 1.5).to(dtype)
    v = torch.randn(T, hkv, d, generator=g).to(dtype)
    return q.to(DEV), k.to(DEV), v.to(DEV)


def _tables(call):
    tile, tri, start, lens = call.seq_tables()
    L = call.layout
    items = call._view(L.items_off, torch.int32, 8 * max(tile[-1], 1)).view(-1, 8)[:tile[-1]]
    units = call._view(L.units_off, torch.int32, 16 + 12 * L.unit_cap).cpu()
    return tile, tri, start, lens, items.cpu(), units


def _check(lens, *, hq=8, hkv=2, d=128, dtype=torch.bfloat16, block=128, cu=None, uniform=0,
           T=None, seed=0, max_len=None, expect_status=0, last_n=2):
    if cu is None and not uniform:
        cu = [0]
        for n in lens:
            cu.append(cu[-1] + n)
    T = T if T is not None else (cu[-1] if cu is not None else uniform * len(lens))
    q, k, v = _inputs(T, hq, hkv, d, dtype, seed)
    max_len = max_len or max(max(lens), 1)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=DEV) if cu is not None else None
    kw = dict(alpha=0.12, attention_sink=1, window_size=2, last_n_block=last_n, block_size=block)
    if cu is None:
        kw.update(batch=len(lens), uniform_seq_len=uniform)
    staged_o = torch.full_like(q, float("nan"))
    staged = FlashPrefillCall(q, k, v, staged_o, cu_t, max_len, **kw)
    staged.plan()
    staged.pool()
    staged.search()
    staged.attn()
    whole_o = torch.full_like(q, float("nan"))
    whole = FlashPrefillCall(q, k, v, whole_o, cu_t, max_len, **kw)
    whole.run()  # plan + pool in one launch when the batch is small
    torch.cuda.synchronize()
    assert staged.status() == whole.status() == expect_status
    a, b = _tables(staged), _tables(whole)
    assert a[:4] == b[:4], "sequence tables differ"
    ia, ib = a[4], b[4]
    assert sorted(map(tuple, ia.tolist())) == sorted(map(tuple, ib.tolist())), "items differ"
    assert torch.equal(ia[:, 1], ib[:, 1]), "items not in the same level order"
    ua, ub = a[5], b[5]  # count at word 0, 48-byte records from byte 64
    n = int(ua[0])
    assert int(ub[0]) == n and torch.equal(ua[16:16 + 12 * n], ub[16:16 + 12 * n]), \
        "chunk units differ"
    mk_a, mk_b = staged.pooled_k().cpu(), whole.pooled_k().cpu()
    assert torch.equal(mk_a.view(torch.int16), mk_b.view(torch.int16)), "pooled K differs"
    tile, _, start, ln = a[:4]
    kc = k.cpu()
    for s in range(len(ln)):
        if ln[s]:
            mk_o = O.pool_k(kc[start[s]:start[s] + ln[s]], block)
            assert torch.equal(mk_b[tile[s]:tile[s + 1]].view(torch.int16),
                               mk_o.view(torch.int16)), f"pooled K of sequence {s} != oracle"
    assert [torch.equal(x, y) for x, y in zip(staged.selection_masks(), whole.selection_masks())] \
        == [True] * len(ln)
    assert torch.equal(staged_o.nan_to_num(7.0), whole_o.nan_to_num(7.0)), "outputs differ"
    return whole


def test_single_sequence_with_split_rows():
    whole = _check([4096 + 77], hq=32, hkv=8)
    assert whole.layout.split_blocks > 0


def test_ragged_batches_with_empty_sequences():
    _check([300, 0, 1, 2048, 129, 0, 700], hq=8, hkv=2, seed=1)
    _check([5000, 17, 128, 64], hq=4, hkv=4, d=64, dtype=torch.float16, seed=2, last_n=3)


def test_uniform_batch_block_64():
    _check([1000] * 3, uniform=1000, hq=8, hkv=2, block=64, seed=3)


def test_sixteen_and_seventeen_sequences():
    lens = [97 * (b + 1) for b in range(16)]
    _check(lens, seed=4)
    _check(lens + [333], seed=5)  # 17: separate plan and pooling launches


def test_bad_cu_seqlens_flags_match():
    # a sequence that starts before an earlier one, and one past the end
    _check([512, 512, 512], cu=[0, 512, 256, 768], seed=6, expect_status=2)
    _check([512, 512], cu=[0, 512, 2000], T=1024, max_len=2048, seed=7, expect_status=2)
    _check([4096], cu=[0, 4096], max_len=1024, seed=8, expect_status=1)
