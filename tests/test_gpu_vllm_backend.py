"""GPU tests of the vLLM backend hook: the KV-cache write kernel
(fp_kv_cache_write) against an index-copy reference, and a prefill step then
a decode step through the hooked forward (stand-in impl and metadata; the
prefill output equals a direct flash_prefill_varlen_func call bit for bit,
the decode output matches explicit fp32 attention over the cached keys)."""

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
