"""GPU tests of the vLLM backend hook: the KV-cache write kernel
(fp_kv_cache_write) against an index-copy reference, and a prefill step then
a decode step through the hooked forward (stand-in impl and metadata; the
prefill output equals a direct flash_prefill_varlen_func call bit for bit,
the decode output matches explicit fp32 attention over the cached keys), and
one mixed v0-engine step (prefill rows, then decode rows) through the v0
forward."""

import math
from types import SimpleNamespace

import pytest
import torch

from flashprefill_amd import flash_prefill_varlen_func
from flashprefill_amd import vllm_backend as vb

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _ref_cache_write(key, value, kc, vc, slots):
    bs = kc.shape[1]
    for t, s in enumerate(slots.tolist()):
        if 0 <= s < kc.shape[0] * bs:
            kc[s // bs, s % bs] = key[t]
            vc[s // bs, s % bs] = value[t]


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float16, 64)])
def test_kv_cache_write_matches_index_copy(dtype, d):
    g = torch.Generator().manual_seed(1)
    T, Hq, Hkv, nblk, bs = 300, 8, 2, 40, 16
    # key / value as strided views of one fused qkv projection, as in vLLM
    qkv = torch.randn(T + 5, Hq + 2 * Hkv, d, generator=g).to(dtype).to(DEV)
    key, value = qkv[:, Hq:Hq + Hkv], qkv[:, Hq + Hkv:]
    slots = torch.randperm(nblk * bs, generator=g)[:T].to(DEV)
    slots[::17] = -1  # padding tokens
    slots[5] = nblk * bs + 3  # past the cache: skipped
    kv = torch.full((2, nblk, bs, Hkv, d), 3.0, dtype=dtype, device=DEV)
    want = kv.cpu()
    vb.reshape_and_cache(key, value, kv[0], kv[1], slots)
    torch.cuda.synchronize()
    _ref_cache_write(key.cpu(), value.cpu(), want[0], want[1], slots.cpu())
    assert torch.equal(kv.cpu(), want)


def test_prefill_then_decode_through_the_hooked_forward():
    g = torch.Generator().manual_seed(2)
    Hq, Hkv, d, bs, nblk = 8, 2, 128, 16, 200
    lens = [700, 300, 129]
    T = sum(lens)
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    # paged cache with a shuffled block table
    per_seq = [(n + 1 + bs - 1) // bs for n in lens]  # room for one decode token
    perm = torch.randperm(nblk, generator=g).tolist()
    table = torch.zeros(len(lens), max(per_seq), dtype=torch.int32)
    pos = 0
    for b, m in enumerate(per_seq):
        table[b, :m] = torch.tensor(perm[pos:pos + m])
        pos += m
    table = table.to(DEV)

    def slots_for(b, positions):
        return [int(table[b, p // bs]) * bs + p % bs for p in positions]

    pad = 7  # vLLM pads the token dimension; the slot mapping does not cover the padding
    q = (torch.randn(T + pad, Hq, d, generator=g) * 1.5).to(torch.bfloat16).to(DEV)
    k = (torch.randn(T + pad, Hkv, d, generator=g) * 1.5).to(torch.bfloat16).to(DEV)
    v = torch.randn(T + pad, Hkv, d, generator=g).to(torch.bfloat16).to(DEV)
    kv = torch.zeros(2, nblk, bs, Hkv, d, dtype=torch.bfloat16, device=DEV)
    impl = SimpleNamespace(attn_type="decoder", kv_sharing_target_layer_name=None,
                           kv_cache_dtype="auto", dcp_world_size=1, scale=1 / math.sqrt(d))
    fwd = vb.make_forward(vb.ATTENTION_CONFIGS["flashprefill_llama"])

    # prefill step
    slot_mapping = torch.tensor(sum((slots_for(b, range(n)) for b, n in enumerate(lens)), []),
                                device=DEV)
    meta = SimpleNamespace(num_actual_tokens=T,
                           query_start_loc=torch.tensor(cu, dtype=torch.int32, device=DEV),
                           max_query_len=max(lens), seq_lens=torch.tensor(lens, device=DEV),
                           block_table=table, slot_mapping=slot_mapping, use_cascade=False)
    out = torch.full((T + pad, Hq, d), 5.0, dtype=torch.bfloat16, device=DEV)
    assert fwd(impl, None, q, k, v, kv, meta, output=out) is out
    want = torch.empty(T, Hq, d, dtype=torch.bfloat16, device=DEV)
    flash_prefill_varlen_func(q[:T], k[:T], v[:T], want, meta.query_start_loc, max(lens), 0.18,
                              128, 2, 4, 2)
    torch.cuda.synchronize()
    assert torch.equal(out[:T], want)
    assert (out[T:] == 5.0).all()
    for b, n in enumerate(lens):  # the cache holds every prefill token at its slot
        for p in (0, n // 2, n - 1):
            s = slots_for(b, [p])[0]
            assert torch.equal(kv[0, s // bs, s % bs], k[cu[b] + p])
            assert torch.equal(kv[1, s // bs, s % bs], v[cu[b] + p])

    # decode step: one new token per sequence
    qd = (torch.randn(3, Hq, d, generator=g) * 1.5).to(torch.bfloat16).to(DEV)
    kd = (torch.randn(3, Hkv, d, generator=g) * 1.5).to(torch.bfloat16).to(DEV)
    vd = torch.randn(3, Hkv, d, generator=g).to(torch.bfloat16).to(DEV)
    meta_d = SimpleNamespace(num_actual_tokens=3,
                             query_start_loc=torch.tensor([0, 1, 2, 3], dtype=torch.int32,
                                                          device=DEV),
                             max_query_len=1, seq_lens=torch.tensor([n + 1 for n in lens],
                                                                    device=DEV),
                             block_table=table, use_cascade=False,
                             slot_mapping=torch.tensor([slots_for(b, [n])[0]
                                                        for b, n in enumerate(lens)], device=DEV))
    out_d = torch.empty(3, Hq, d, dtype=torch.bfloat16, device=DEV)
    fwd(impl, None, qd, kd, vd, kv, meta_d, output=out_d)
    torch.cuda.synchronize()
    for b, n in enumerate(lens):
        ks = torch.cat([k[cu[b]:cu[b + 1]], kd[b:b + 1]]).float()
        vs = torch.cat([v[cu[b]:cu[b + 1]], vd[b:b + 1]]).float()
        for h in range(Hq):
            s = ks[:, h // (Hq // Hkv)] @ qd[b, h].float() / math.sqrt(d)
            o = torch.softmax(s, 0) @ vs[:, h // (Hq // Hkv)]
            assert (out_d[b, h].float() - o).abs().max().item() <= 2e-2


def test_v0_mixed_step_prefill_rows_then_decode_rows():
    # the v0 engine's batch: prefill tokens of two new sequences first, then
    # one decode token of each of two sequences already in the cache
    g = torch.Generator().manual_seed(3)
    Hq, Hkv, d, bs, nblk = 8, 2, 128, 16, 120
    pre = [600, 257]
    old = [300, 90]  # cached lengths of the decoding sequences (without the new token)
    P, Dn = sum(pre), len(old)
    perm = torch.randperm(nblk, generator=g).tolist()
    need = [(n + bs - 1) // bs for n in pre] + [(n + 1 + bs - 1) // bs for n in old]
    table = torch.zeros(len(need), max(need), dtype=torch.int32)
    pos = 0
    for r, m in enumerate(need):
        table[r, :m] = torch.tensor(perm[pos:pos + m])
        pos += m
    table = table.to(DEV)

    def slot(r, p):
        return int(table[r, p // bs]) * bs + p % bs

    kv = torch.zeros(2, nblk, bs, Hkv, d, dtype=torch.bfloat16, device=DEV)
    # earlier tokens of the decoding sequences, already cached
    hist_k = [(torch.randn(n, Hkv, d, generator=g) * 1.5).to(torch.bfloat16).to(DEV) for n in old]
    hist_v = [torch.randn(n, Hkv, d, generator=g).to(torch.bfloat16).to(DEV) for n in old]
    for j, n in enumerate(old):
        for p in range(n):
            s = slot(2 + j, p)
            kv[0, s // bs, s % bs] = hist_k[j][p]
            kv[1, s // bs, s % bs] = hist_v[j][p]
    T = P + Dn
    q = (torch.randn(T, Hq, d, generator=g) * 1.5).to(torch.bfloat16).to(DEV)
    k = (torch.randn(T, Hkv, d, generator=g) * 1.5).to(torch.bfloat16).to(DEV)
    v = torch.randn(T, Hkv, d, generator=g).to(torch.bfloat16).to(DEV)
    slots = [slot(0, p) for p in range(pre[0])] + [slot(1, p) for p in range(pre[1])] + \
        [slot(2 + j, n) for j, n in enumerate(old)]
    cu = torch.tensor([0, pre[0], P], dtype=torch.int32, device=DEV)
    pm = SimpleNamespace(seq_start_loc=cu, max_prefill_seq_len=max(pre), query_start_loc=cu,
                         seq_lens_tensor=torch.tensor(pre, device=DEV), block_tables=None)
    dm = SimpleNamespace(seq_lens_tensor=torch.tensor([n + 1 for n in old], device=DEV),
                         max_decode_query_len=1, query_start_loc=None,
                         block_tables=table[2:])
    meta = SimpleNamespace(num_prefill_tokens=P, num_decode_tokens=Dn,
                           slot_mapping=torch.tensor(slots, device=DEV),
                           prefill_metadata=pm, decode_metadata=dm)
    impl = SimpleNamespace(attn_type="decoder", kv_cache_dtype="auto", scale=1 / math.sqrt(d))
    fwd = vb.make_forward_v0(vb.ATTENTION_CONFIGS["flashprefill_qwen2"])
    out = torch.full((T, Hq, d), 5.0, dtype=torch.bfloat16, device=DEV)
    assert fwd(impl, None, q, k, v, kv, meta, output=out) is out
    want = torch.empty(P, Hq, d, dtype=torch.bfloat16, device=DEV)
    flash_prefill_varlen_func(q[:P], k[:P], v[:P], want, cu, max(pre), 0.08, 128, 2, 4, 2)
    torch.cuda.synchronize()
    assert torch.equal(out[:P], want)
    for t in (0, pre[0] - 1, pre[0], P - 1):  # prefill rows reached the cache
        s = slots[t]
        assert torch.equal(kv[0, s // bs, s % bs], k[t]) and torch.equal(kv[1, s // bs, s % bs], v[t])
    G = Hq // Hkv
    for j, n in enumerate(old):
        ks = torch.cat([hist_k[j], k[P + j:P + j + 1]]).float()
        vs = torch.cat([hist_v[j], v[P + j:P + j + 1]]).float()
        for h in range(Hq):
            sc = ks[:, h // G] @ q[P + j, h].float() / math.sqrt(d)
            o = torch.softmax(sc, 0) @ vs[:, h // G]
            assert (out[P + j, h].float() - o).abs().max().item() <= 2e-2
