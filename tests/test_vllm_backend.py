"""CPU tests of the vLLM backend hook (flashprefill_amd/vllm_backend.py): the
dispatch of the hooked FlashAttentionImpl.forward against the reference
patch's (patches/patch_loader_vllm_0_12_0.py:57-253), with stand-ins for
vLLM's impl object and metadata and recording fakes for the operations, and
the paged decode fallback against explicit attention."""

import math
from types import SimpleNamespace

import pytest
import torch

from flashprefill_amd import vllm_backend as vb


class FakeImpl:
    def __init__(self, **kw):
        self.attn_type = "decoder"
        self.kv_sharing_target_layer_name = None
        self.kv_cache_dtype = "auto"
        self.dcp_world_size = 1
        self.scale = 0.125
        self.__dict__.update(kw)

    def forward(self, *a, **k):  # replaced by apply_patch
        return "original"


def _meta(n, cu, max_q, seq_lens=None, **kw):
    m = SimpleNamespace(num_actual_tokens=n, query_start_loc=torch.tensor(cu, dtype=torch.int32),
                        max_query_len=max_q, seq_lens=torch.tensor(seq_lens or [0]),
                        block_table=torch.zeros(len(cu) - 1, 4, dtype=torch.int32),
                        slot_mapping=torch.arange(n), use_cascade=False)
    m.__dict__.update(kw)
    return m


def _recording_ops():
    calls = []
    ops = vb.HookOps(cache_write=lambda *a: calls.append(("cache", a)),
                     prefill=lambda *a: calls.append(("prefill", a)),
                     decode=lambda *a: calls.append(("decode", a)),
                     encoder=lambda *a: calls.append(("encoder", a)) or "enc",
                     cascade=lambda *a: calls.append(("cascade", a)) or "casc")
    return calls, ops


def _tensors(T=10, pad=3, hq=4, hkv=2, d=8):
    q = torch.randn(T + pad, hq, d)
    k = torch.randn(T + pad, hkv, d)
    v = torch.randn(T + pad, hkv, d)
    kv = torch.zeros(2, 6, 4, hkv, d)
    out = torch.full((T + pad, hq, d), 9.0)
    return q, k, v, kv, out


def test_apply_patch_replaces_forward_and_returns_the_original():
    class Impl(FakeImpl):
        pass
    calls, ops = _recording_ops()
    orig = vb.apply_patch(Impl, "flashprefill_llama", ops)
    assert orig is FakeImpl.forward
    assert Impl.forward is not FakeImpl.forward


def test_prefill_dispatch_matches_the_reference_call():
    calls, ops = _recording_ops()
    fwd = vb.make_forward(vb.ATTENTION_CONFIGS["flashprefill_qwen3moe"], ops)
    q, k, v, kv, out = _tensors()
    meta = _meta(10, [0, 7, 10], 7)
    res = fwd(FakeImpl(), None, q, k, v, kv, meta, output=out)
    assert res is out
    assert [c[0] for c in calls] == ["cache", "prefill"]
    # cache write on the full (padded) key / value with the slot mapping
    ck, cv, kc, vc, slots = calls[0][1]
    assert ck is k and cv is v and slots is meta.slot_mapping
    assert torch.equal(kc, kv[0]) and torch.equal(vc, kv[1])
    # prefill on the step's own rows, cu_seqlens / max_query_len and the cfg
    a = calls[1][1]
    assert [t.shape[0] for t in a[:4]] == [10, 10, 10, 10]
    assert a[0].data_ptr() == q.data_ptr() and a[3].data_ptr() == out.data_ptr()
    assert a[4] is meta.query_start_loc and a[5] == 7
    assert a[6:] == (0.12, 128, 2, 4, 2)


def test_decode_dispatch_when_every_query_has_one_token():
    calls, ops = _recording_ops()
    fwd = vb.make_forward(vb.ATTENTION_CONFIGS["flashprefill_llama"], ops)
    q, k, v, kv, out = _tensors(T=3)
    meta = _meta(3, [0, 1, 2, 3], 1, seq_lens=[5, 9, 2])
    fwd(FakeImpl(scale=0.3), None, q, k, v, kv, meta, output=out)
    assert [c[0] for c in calls] == ["cache", "decode"]
    a = calls[1][1]
    assert a[0].shape[0] == 3 and a[5] is meta.seq_lens and a[6] is meta.block_table
    assert a[7] == 0.3


def test_profiling_run_zero_fills_and_guards():
    calls, ops = _recording_ops()
    fwd = vb.make_forward(vb.ATTENTION_CONFIGS["flashprefill_qwen2"], ops)
    q, k, v, kv, out = _tensors()
    assert fwd(FakeImpl(), None, q, k, v, kv, None, output=out) is out
    assert (out == 0).all() and calls == []
    with pytest.raises(ValueError):
        fwd(FakeImpl(), None, q, k, v, kv, _meta(10, [0, 10], 10), output=None)
    with pytest.raises(NotImplementedError):
        fwd(FakeImpl(), None, q, k, v, kv, _meta(10, [0, 10], 10), output=out,
            output_scale=torch.ones(1))
    with pytest.raises(NotImplementedError):
        fwd(FakeImpl(kv_cache_dtype="fp8_e4m3"), None, q, k, v, kv, _meta(10, [0, 10], 10),
            output=out)
    with pytest.raises(NotImplementedError):
        fwd(FakeImpl(dcp_world_size=2), None, q, k, v, kv, _meta(10, [0, 10], 10), output=out)


def test_shared_kv_skips_the_cache_write_and_encoder_cascade_delegate():
    calls, ops = _recording_ops()
    fwd = vb.make_forward(vb.ATTENTION_CONFIGS["flashprefill_qwen2"], ops)
    q, k, v, kv, out = _tensors()
    fwd(FakeImpl(kv_sharing_target_layer_name="layers.0"), None, q, k, v, kv,
        _meta(10, [0, 10], 10), output=out)
    assert [c[0] for c in calls] == ["prefill"]
    calls.clear()
    assert fwd(FakeImpl(attn_type="encoder_only"), None, q, k, v, kv, _meta(10, [0, 10], 10),
               output=out) == "enc"
    assert [c[0] for c in calls] == ["encoder"]
    calls.clear()
    assert fwd(FakeImpl(), None, q, k, v, kv, _meta(10, [0, 10], 10, use_cascade=True),
               output=out) == "casc"
    assert [c[0] for c in calls] == ["cache", "cascade"]


def test_paged_decode_attention_matches_explicit_attention():
    # CPU run of the decode fallback: 3 sequences with 1, 1 and 2 query rows
    # over a shuffled block table, against fp64 causal attention
    g = torch.Generator().manual_seed(0)
    nblk, bs, hkv, hq, d = 10, 4, 2, 4, 16
    kc = torch.randn(nblk, bs, hkv, d, generator=g)
    vc = torch.randn(nblk, bs, hkv, d, generator=g)
    table = torch.tensor([[3, 7, 1, 0], [9, 2, 0, 0], [5, 4, 8, 6]], dtype=torch.int32)
    used = torch.tensor([10, 5, 15])
    cu = torch.tensor([0, 1, 2, 4], dtype=torch.int32)
    q = torch.randn(4, hq, d, generator=g)
    out = torch.zeros(4, hq, d)
    scale = 1 / math.sqrt(d)
    vb.paged_decode_attention(q, kc, vc, out, cu, used, table, scale)
    for b in range(3):
        n = int(used[b])
        ks = torch.cat([kc[int(j)] for j in table[b]])[:n].double()
        vs = torch.cat([vc[int(j)] for j in table[b]])[:n].double()
        for r in range(int(cu[b]), int(cu[b + 1])):
            pos = n - (int(cu[b + 1]) - r)
            for h in range(hq):
                s = ks[:pos + 1, h // 2] @ q[r, h].double() * scale
                want = torch.softmax(s, 0) @ vs[:pos + 1, h // 2]
                assert torch.allclose(out[r, h].double(), want, atol=1e-5)


# --------------------------------------------------------------------------
# v0 engine forward (patches/patch_loader_vllm_0_10_0.py:78-376)
# --------------------------------------------------------------------------

def _meta_v0(n_pre, n_dec, *, prefill=None, decode=None, **kw):
    m = SimpleNamespace(num_prefill_tokens=n_pre, num_decode_tokens=n_dec,
                        slot_mapping=torch.arange(n_pre + n_dec).view(-1, 1),
                        prefill_metadata=prefill, decode_metadata=decode)
    m.__dict__.update(kw)
    return m


def _prefill_meta(cu, tables=None):
    cu_t = torch.tensor(cu, dtype=torch.int32)
    lens = [cu[b + 1] - cu[b] for b in range(len(cu) - 1)]
    return SimpleNamespace(seq_start_loc=cu_t, max_prefill_seq_len=max(lens),
                           query_start_loc=cu_t, seq_lens_tensor=torch.tensor(lens),
                           block_tables=tables)


def _decode_meta(seq_lens, max_q=1, cu=None):
    return SimpleNamespace(seq_lens_tensor=torch.tensor(seq_lens), max_decode_query_len=max_q,
                           query_start_loc=None if cu is None else torch.tensor(cu),
                           block_tables=torch.zeros(len(seq_lens), 4, dtype=torch.int32))


def test_v0_mixed_batch_prefill_then_decode_rows():
    # 7 + 3 prefill tokens (no block tables: the step's own rows), then 2
    # decode tokens with one query each; the write uses the flattened mapping
    calls, ops = _recording_ops()
    fwd = vb.make_forward_v0(vb.ATTENTION_CONFIGS["flashprefill_llama"], ops)
    q, k, v, kv, out = _tensors(T=12)
    pm, dm = _prefill_meta([0, 7, 10]), _decode_meta([30, 12])
    meta = _meta_v0(10, 2, prefill=pm, decode=dm)
    assert fwd(FakeImpl(scale=0.2), None, q, k, v, kv, meta, output=out) is out
    assert [c[0] for c in calls] == ["cache", "prefill", "decode"]
    ck, cv, kc, vc, slots = calls[0][1]
    assert ck is k and cv is v and slots.shape == (12,)
    assert torch.equal(kc, kv[0]) and torch.equal(vc, kv[1])
    a = calls[1][1]
    assert [t.shape[0] for t in a[:4]] == [10, 10, 10, 10]
    assert a[0].data_ptr() == q.data_ptr() and a[3].data_ptr() == out.data_ptr()
    assert a[4] is pm.seq_start_loc and a[5] == 7 and a[6:] == (0.18, 128, 2, 4, 2)
    d = calls[2][1]
    assert d[0].shape[0] == 2 and d[0].data_ptr() == q[10].data_ptr()
    assert d[3].data_ptr() == out[10].data_ptr()
    assert d[4].tolist() == [0, 1, 2] and d[5] is dm.seq_lens_tensor
    assert d[6] is dm.block_tables and d[7] == 0.2


def test_v0_prefix_cached_prefill_and_varlen_decode_use_the_paged_cache():
    calls, ops = _recording_ops()
    fwd = vb.make_forward_v0(vb.ATTENTION_CONFIGS["flashprefill_qwen2"], ops)
    q, k, v, kv, out = _tensors(T=9)
    tables = torch.ones(2, 4, dtype=torch.int32)
    pm = _prefill_meta([0, 4, 6], tables=tables)
    dm = _decode_meta([20, 8], max_q=2, cu=[0, 2, 3])
    fwd(FakeImpl(), None, q, k, v, kv, _meta_v0(6, 3, prefill=pm, decode=dm), output=out)
    assert [c[0] for c in calls] == ["cache", "decode", "decode"]
    p = calls[1][1]
    assert p[0].shape[0] == 6 and torch.equal(p[1], kv[0]) and p[4] is pm.query_start_loc
    assert p[5] is pm.seq_lens_tensor and p[6] is tables
    d = calls[2][1]
    assert d[0].shape[0] == 3 and d[4] is dm.query_start_loc


def test_v0_profiling_run_guards_and_delegation():
    calls, ops = _recording_ops()
    fwd = vb.make_forward_v0(vb.ATTENTION_CONFIGS["flashprefill_qwen2"], ops)
    q, k, v, kv, out = _tensors()
    # an unallocated cache (profiling run): no write, prefill on the step's rows
    fwd(FakeImpl(), None, q, k, v, torch.empty(0), _meta_v0(10, 0, prefill=_prefill_meta([0, 10])),
        output=out)
    assert [c[0] for c in calls] == ["prefill"]
    calls.clear()
    # encoder-decoder layers are delegated whole, their cache write included
    enc_dec = FakeImpl(attn_type="encoder_decoder")
    assert fwd(enc_dec, None, q, k, v, kv, _meta_v0(10, 0), output=out) == "enc"
    assert [c[0] for c in calls] == ["encoder"]
    with pytest.raises(ValueError):
        fwd(FakeImpl(), None, q, k, v, kv, _meta_v0(10, 0), output=None)
    with pytest.raises(NotImplementedError):
        fwd(FakeImpl(), None, q, k, v, kv, _meta_v0(10, 0), output=out,
            output_scale=torch.ones(1))
    with pytest.raises(NotImplementedError):
        fwd(FakeImpl(kv_cache_dtype="fp8"), None, q, k, v, kv, _meta_v0(10, 0), output=out)
    plain = vb.make_forward_v0(vb.ATTENTION_CONFIGS["flashprefill_qwen2"])
    with pytest.raises(NotImplementedError):
        plain(FakeImpl(attn_type="encoder"), None, q, k, v, kv, _meta_v0(10, 0), output=out)


def test_apply_patch_v0_replaces_forward():
    class Impl(FakeImpl):
        pass
    _, ops = _recording_ops()
    orig = vb.apply_patch_v0(Impl, "flashprefill_qwen3moe", ops)
    assert orig is FakeImpl.forward and Impl.forward is not FakeImpl.forward
