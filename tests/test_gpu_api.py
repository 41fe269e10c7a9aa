"""GPU tests of the public operator surface (the reference's two entry points)
and of the C ABI's error / status behaviour."""

import pytest
import torch

from flashprefill_amd import FlashPrefillCall, flash_prefill, flash_prefill_varlen_func
from flashprefill_amd import _lib
from oracle import flashprefill_oracle as O
from tests._parity import OUT_MAX_ABS, OUT_MEAN_ABS

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _rand(shape, seed, dtype=torch.bfloat16, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _close(out, ref, flips_ok=True):
    d = (out.float().cpu() - ref.float()).abs()
    assert not torch.isnan(d).any()
    assert d.mean().item() <= OUT_MEAN_ABS, d.mean().item()
    assert d.max().item() <= OUT_MAX_ABS, d.max().item()


def test_varlen_api_matches_oracle_and_is_deterministic():
    lens = [513, 1024, 77]
    T = sum(lens)
    q, k, v = _rand((T, 8, 128), 1, scale=1.5), _rand((T, 2, 128), 2, scale=1.5), _rand((T, 2, 128), 3)
    cu = torch.tensor([0, 513, 1537, T], dtype=torch.int32)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o1 = torch.empty_like(qd)
    o2 = torch.empty_like(qd)
    flash_prefill_varlen_func(qd, kd, vd, o1, cu.to(DEV), 1024, 0.18)
    flash_prefill_varlen_func(qd, kd, vd, o2, cu.to(DEV), 1024, 0.18, 128, 2, 4, 2)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    ref = O.flash_prefill_varlen_func(q, k, v, cu, 1024, 0.18).out
    _close(o1, ref)


def test_native_batched_api_matches_oracle():
    B, S, Hq, Hkv, d = 2, 1000, 8, 8, 128
    q, k, v = _rand((B, S, Hq, d), 4, scale=1.5), _rand((B, S, Hkv, d), 5, scale=1.5), _rand((B, S, Hkv, d), 6)
    out = torch.empty(B, S, Hq, d, dtype=torch.bfloat16, device=DEV)
    flash_prefill(q.to(DEV), k.to(DEV), v.to(DEV), out, 128, 2, 4, 0.7, 2, 0)
    torch.cuda.synchronize()
    ref = O.flash_prefill(q, k, v, 128, 2, 4, 0.7, 2, 0).out
    _close(out, ref)


def test_class_level_entry_points_match_the_functions():
    # FlashPrefill_varlen.apply / FlashPrefill.apply (the reference's
    # autograd.Function entry points) give the function entry points' output
    # bit for bit
    from ops.flashprefill_native_forward import FlashPrefill
    from ops.flashprefill_varlen_func import FlashPrefill_varlen
    lens = [700, 300]
    T = sum(lens)
    q, k, v = _rand((T, 8, 128), 21, scale=1.5), _rand((T, 2, 128), 22, scale=1.5), _rand((T, 2, 128), 23)
    cu = torch.tensor([0, 700, T], dtype=torch.int32, device=DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o1, o2 = torch.empty_like(qd), torch.empty_like(qd)
    flash_prefill_varlen_func(qd, kd, vd, o1, cu, 700, 0.12, 128, 2, 4, 2)
    assert FlashPrefill_varlen.apply(qd, kd, vd, o2, cu, 700, 128, 128, 2, 4, 0.12, 2) is None
    B, S = 2, 500
    qb, kb, vb = (x.to(DEV) for x in (_rand((B, S, 8, 128), 24, scale=1.5),
                                      _rand((B, S, 2, 128), 25, scale=1.5), _rand((B, S, 2, 128), 26)))
    o3, o4 = torch.empty_like(qb), torch.empty_like(qb)
    flash_prefill(qb, kb, vb, o3, 128, 2, 4, 0.7, 2, 3)
    assert FlashPrefill.apply(qb, kb, vb, o4, 128, 128, 2, 4, 0.7, 2, 0, 3, 0) is None
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert torch.equal(o3, o4)


def test_strided_inputs_match_contiguous():
    # q/k/v carved out of one fused qkv projection output, as vLLM does
    T, Hq, Hkv, d = 900, 8, 2, 128
    qkv = _rand((T, Hq + 2 * Hkv, d), 7, scale=1.5).to(DEV)
    q, k, v = qkv[:, :Hq], qkv[:, Hq:Hq + Hkv], qkv[:, Hq + Hkv:]
    assert not q.is_contiguous()
    cu = torch.tensor([0, 400, T], dtype=torch.int32, device=DEV)
    o_strided = torch.empty(T, 2 * Hq, d, dtype=torch.bfloat16, device=DEV)[:, :Hq]
    o_ref = torch.empty(T, Hq, d, dtype=torch.bfloat16, device=DEV)
    flash_prefill_varlen_func(q, k, v, o_strided, cu, 500, 0.18)
    flash_prefill_varlen_func(q.contiguous(), k.contiguous(), v.contiguous(), o_ref, cu, 500, 0.18)
    torch.cuda.synchronize()
    assert torch.equal(o_strided, o_ref)


def test_all_blocks_selected_is_dense_causal():
    T, Hq, Hkv, d = 640, 4, 2, 64
    q, k, v = _rand((T, Hq, d), 8, scale=1.5), _rand((T, Hkv, d), 9, scale=1.5), _rand((T, Hkv, d), 10)
    o = torch.empty(T, Hq, d, dtype=torch.bfloat16, device=DEV)
    cu = torch.tensor([0, T], dtype=torch.int32, device=DEV)
    flash_prefill_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), o, cu, T, 0.0)  # alpha 0: S >= 0
    torch.cuda.synchronize()
    qq = q.double().permute(1, 0, 2)
    kk = k.double().permute(1, 0, 2).repeat_interleave(2, 0)
    vv = v.double().permute(1, 0, 2).repeat_interleave(2, 0)
    ref = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, is_causal=True)
    _close(o, ref.permute(1, 0, 2))


def test_all_blocks_selected_long_rows():
    # 8300 tokens: 65 blocks per row, a partial last block of 108 rows, dense
    # causal attention against fp32 SDPA
    T, Hq, Hkv, d = 8300, 4, 1, 128
    q, k, v = _rand((T, Hq, d), 21, scale=1.5), _rand((T, Hkv, d), 22, scale=1.5), _rand((T, Hkv, d), 23)
    o = torch.empty(T, Hq, d, dtype=torch.bfloat16, device=DEV)
    cu = torch.tensor([0, T], dtype=torch.int32, device=DEV)
    flash_prefill_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), o, cu, T, 0.0)
    torch.cuda.synchronize()
    qq = q.float().permute(1, 0, 2).contiguous().to(DEV)
    kk = k.float().permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0).contiguous().to(DEV)
    vv = v.float().permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0).contiguous().to(DEV)
    ref = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, is_causal=True)
    _close(o, ref.permute(1, 0, 2).cpu())


@pytest.mark.parametrize("step", [70.0, 23.5, 8.0])
def test_growing_logits_rescale(step):
    # every key block's logits exceed the previous block's by step / sqrt(d)
    # * log2(e) log2 units: ~9 (the block maximum alone moves the running max
    # by more than 2^8 on every block), ~3 (a lane's partial row sum of
    # P = 2^3-ish values passes 2^8 while no single P does) and ~1 (P grows
    # past 1 over several blocks before the row sum forces a move), so the
    # attention kernel's rescale path is taken on every block, on the row-sum
    # trigger alone, and after runs of blocks kept against a stale maximum.
    # The last query rows attend almost only to their own (diagonal) block.
    # All blocks selected (alpha 0): dense causal attention vs fp32 SDPA.
    T, Hq, Hkv, d = 2048, 2, 1, 128
    g = torch.Generator().manual_seed(31)
    e = torch.zeros(d)
    e[0] = 1.0
    q = (e + 0.05 * torch.randn(T, Hq, d, generator=g)).to(torch.bfloat16)
    blk = (torch.arange(T) // 128).float()
    k = (step * blk[:, None, None] * e + torch.randn(T, Hkv, d, generator=g)).to(torch.bfloat16)
    v = torch.randn(T, Hkv, d, generator=g).to(torch.bfloat16)
    o = torch.empty(T, Hq, d, dtype=torch.bfloat16, device=DEV)
    cu = torch.tensor([0, T], dtype=torch.int32, device=DEV)
    flash_prefill_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), o, cu, T, 0.0)
    torch.cuda.synchronize()
    qq = q.float().permute(1, 0, 2).contiguous().to(DEV)
    kk = k.float().permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0).contiguous().to(DEV)
    vv = v.float().permute(1, 0, 2).repeat_interleave(Hq // Hkv, 0).contiguous().to(DEV)
    ref = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, is_causal=True)
    _close(o, ref.permute(1, 0, 2).cpu())


@pytest.mark.parametrize("block,dtype,d", [(128, torch.bfloat16, 128), (64, torch.bfloat16, 128),
                                           (128, torch.float16, 64)])
def test_persistent_attention_queues_rearm(block, dtype, d):
    # 16K (block 128) / 32K (block 64) tokens x 32 heads give at least 8
    # attention slots per resident workgroup, so the attention stage runs as
    # the persistent grid over per-XCD claim queues. The plan kernel empties
    # the queues once; every attention launch after that must empty them
    # again itself: attention-only launches repeated on the planned
    # workspace, and a second full call, give the first call's output bit for
    # bit.
    T, Hq, Hkv = 16384 if block == 128 else 32768, 32, 8
    q, k, v = (_rand((T, Hq, d), 41, dtype, scale=1.5).to(DEV),
               _rand((T, Hkv, d), 42, dtype, scale=1.5).to(DEV), _rand((T, Hkv, d), 43, dtype).to(DEV))
    cu = torch.tensor([0, T], dtype=torch.int32, device=DEV)
    o = torch.empty_like(q)
    call = FlashPrefillCall(q, k, v, o, cu, T, alpha=0.18, block_size=block)
    call.run()
    torch.cuda.synchronize()
    ref = o.clone()
    for _ in range(3):
        o.fill_(float("nan"))
        call.attn()
        torch.cuda.synchronize()
        assert torch.equal(o, ref)
    o.fill_(float("nan"))
    call.run()
    torch.cuda.synchronize()
    assert torch.equal(o, ref)
    # sampled rows against the oracle's row pipeline (rows whose selection
    # differs by a threshold flip are skipped; at most one is allowed)
    tile, tri, _, _ = call.seq_tables()
    nb = tile[-1]
    cnt, idx = call.counts().cpu(), call.index_lists().cpu()
    rows = [(h, i) for h in (0, 13, 31) for i in (0, nb // 3, nb - 1)]
    res = O.flashprefill_rows(q.cpu(), k.cpu(), v.cpu(), rows, alpha=0.18, attention_sink=2,
                              window=4, last_n=2, native=False, block=block)
    flips = 0
    for (h, i), (sel_o, out_o) in res.items():
        base = tri[0] + i * (i + 1) // 2
        gsel = torch.zeros(nb, dtype=torch.bool)
        gsel[idx[h, base:base + int(cnt[h, i])].long()] = True
        if not torch.equal(gsel, sel_o):
            flips += int((gsel != sel_o).sum())
            continue
        got = o[i * block:(i + 1) * block, h].float().cpu()
        d_ = (got - out_o.float()).abs()
        assert d_.max().item() <= OUT_MAX_ABS and d_.mean().item() <= OUT_MEAN_ABS
    assert flips <= 1


def test_status_flags_and_untouched_output():
    T, Hq, Hkv, d = 1000, 4, 1, 128
    q, k, v = _rand((T, Hq, d), 11).to(DEV), _rand((T, Hkv, d), 12).to(DEV), _rand((T, Hkv, d), 13).to(DEV)
    o = torch.full((T, Hq, d), 7.0, dtype=torch.bfloat16, device=DEV)
    cu = torch.tensor([0, 300, 1000], dtype=torch.int32, device=DEV)  # second seq has 700 > 512
    call = FlashPrefillCall(q, k, v, o, cu, 512, alpha=0.18)
    call.run()
    assert call.status() == _lib.FP_STATUS_SEQ_TOO_LONG
    assert (o[300:] == 7.0).all()
    assert not (o[:300] == 7.0).all()
    cu_bad = torch.tensor([0, 300, 2000], dtype=torch.int32, device=DEV)
    call = FlashPrefillCall(q, k, v, o, cu_bad, 2000, alpha=0.18)
    call.run()
    assert call.status() & _lib.FP_STATUS_BAD_CU_SEQLENS
    # overlapping sequences [0, T, 0, T]: the second has negative length and
    # the third starts before an earlier entry, so both are skipped and the
    # block count stays within the workspace capacity; the first sequence's
    # output equals a call on [0, T] alone
    o_ov = torch.full((T, Hq, d), 7.0, dtype=torch.bfloat16, device=DEV)
    cu_ov = torch.tensor([0, T, 0, T], dtype=torch.int32, device=DEV)
    call = FlashPrefillCall(q, k, v, o_ov, cu_ov, T, alpha=0.18)
    call.run()
    assert call.status() == _lib.FP_STATUS_BAD_CU_SEQLENS
    tile, tri, start, lens = call.seq_tables()
    assert lens == [T, 0, 0]
    assert tile[-1] == (T + 127) // 128 <= call.layout.nb_sum_cap
    o_one = torch.full((T, Hq, d), 7.0, dtype=torch.bfloat16, device=DEV)
    FlashPrefillCall(q, k, v, o_one, torch.tensor([0, T], dtype=torch.int32, device=DEV), T,
                     alpha=0.18).run()
    torch.cuda.synchronize()
    assert torch.equal(o_ov, o_one)
    # a sequence skipped by the plan keeps the caller's output rows also when
    # o is not writable in place (the operator writes a copy and copies back)
    flat = torch.full((T * Hq * d + 4,), 7.0, dtype=torch.bfloat16, device=DEV)
    o_view = flat[4:].view(T, Hq, d)  # 8-byte aligned: not writable in place
    assert o_view.data_ptr() % 16 != 0
    flash_prefill_varlen_func(q, k, v, o_view, torch.tensor([0, 300, 1000], dtype=torch.int32,
                              device=DEV), 512, 0.18)
    torch.cuda.synchronize()
    assert (o_view[300:] == 7.0).all()
    assert not (o_view[:300] == 7.0).all()


def test_error_paths():
    T = 256
    q = torch.zeros(T, 4, 128, dtype=torch.float32, device=DEV)
    cu = torch.tensor([0, T], dtype=torch.int32, device=DEV)
    with pytest.raises(NotImplementedError):  # float64 is not built
        flash_prefill_varlen_func(q.double(), q[:, :1].double(), q[:, :1].double(),
                                  q.double(), cu, T, 0.1)
    with pytest.raises(ValueError):  # mixed dtypes
        flash_prefill_varlen_func(q, q[:, :1].to(torch.bfloat16), q[:, :1], q.clone(), cu, T, 0.1)
    qb = q.to(torch.bfloat16)
    with pytest.raises(ValueError):
        flash_prefill_varlen_func(qb, qb[:, :3].contiguous(), qb[:, :3].contiguous(), qb.clone(),
                                  cu, T, 0.1)
    q96 = torch.zeros(T, 4, 96, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(NotImplementedError):
        flash_prefill_varlen_func(q96, q96[:, :1].contiguous(), q96[:, :1].contiguous(),
                                  q96.clone(), cu, T, 0.1)
    with pytest.raises(NotImplementedError):
        flash_prefill_varlen_func(qb, qb[:, :1].contiguous(), qb[:, :1].contiguous(), qb.clone(),
                                  cu, T, 0.1, block_size=512)
    q256 = torch.zeros(T, 4, 256, dtype=torch.float32, device=DEV)
    with pytest.raises(NotImplementedError):  # head_dim 256 is built for 16-bit inputs
        flash_prefill_varlen_func(q256, q256[:, :1].contiguous(), q256[:, :1].contiguous(),
                                  q256.clone(), cu, T, 0.1)


def _entry_case(seed):
    """Random shapes for the whole-operator entry points: ragged varlen batches
    with zero-length and 1-token sequences, or a batched native call with
    min_budget; blocks 64 / 128 / 256, head_dims 64 / 128 / 256, fp32."""
    import random
    rnd = random.Random(7000 + seed)
    block = rnd.choice([64, 128, 128, 256])
    d = rnd.choice([64, 128, 128, 256])
    dtype = rnd.choice([torch.bfloat16, torch.float16, torch.bfloat16])
    if d == 256 and block == 256:
        d = 128
    if rnd.random() < 0.15 and d != 256 and block != 256:
        dtype = torch.float32
    hkv = rnd.choice([1, 2, 4, 8])
    hq = hkv * rnd.choice([1, 2, 4, 7])
    lens = [rnd.choice([0, 1, rnd.randint(2, 600), rnd.randint(600, 5000)])
            for _ in range(rnd.randint(1, 5))]
    if sum(lens) == 0:
        lens[0] = 1
    params = dict(alpha=rnd.choice([0.0, 0.05, 0.12, 0.18, 0.5]), sink=rnd.randint(0, 3),
                  window=rnd.randint(0, 6), last_n=rnd.randint(0, 3))
    native = rnd.random() < 0.3
    min_budget = rnd.randint(1, 10) if native and rnd.random() < 0.5 else 0
    return block, d, dtype, hq, hkv, lens, params, native, min_budget


@pytest.mark.parametrize("seed", range(32))
def test_whole_operator_entry_points_equal_the_staged_path(seed):
    """The public entry points (plan and pooling in one launch for small
    batches, cached workspace) write the same bits as the staged C-ABI calls
    (plan, pool, search, attention) that the parity tests pin to the oracle."""
    block, d, dtype, hq, hkv, lens, p, native, mb = _entry_case(seed)
    print(f"\n  seed={seed} lens={lens} hq={hq} hkv={hkv} d={d} {dtype} block={block} {p} "
          f"native={native} min_budget={mb}", flush=True)
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    if not native:
        T = sum(lens)
        q, k, v = (_rand((T, hq, d), seed, dtype, 2.0), _rand((T, hkv, d), seed + 1, dtype, 2.0),
                   _rand((T, hkv, d), seed + 2, dtype))
        qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
        cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32,
                          device=DEV)
        S = max(lens)
        o_pub = torch.full_like(qd, 7.0)
        flash_prefill_varlen_func(qd, kd, vd, o_pub, cu, S, p["alpha"], block, p["sink"],
                                  p["window"], p["last_n"])
        o_st = torch.full_like(qd, 7.0)
        call = FlashPrefillCall(qd, kd, vd, o_st, cu, S, alpha=p["alpha"], attention_sink=p["sink"],
                                window_size=p["window"], last_n_block=p["last_n"],
                                block_size=block)
    else:
        B, L = min(len(lens), 3), max(max(lens), 1)
        q = _rand((B, L, hq, d), seed, dtype, 2.0)
        k, v = _rand((B, L, hkv, d), seed + 1, dtype, 2.0), _rand((B, L, hkv, d), seed + 2, dtype)
        qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
        o4 = torch.full_like(qd, 7.0)
        flash_prefill(qd, kd, vd, o4, block, p["sink"], p["window"], p["alpha"], p["last_n"], mb)
        o_pub = o4.view(B * L, hq, d)
        o_st = torch.full_like(o_pub, 7.0)
        call = FlashPrefillCall(qd.view(B * L, hq, d), kd.view(B * L, hkv, d),
                                vd.view(B * L, hkv, d), o_st, None, L, alpha=p["alpha"],
                                attention_sink=p["sink"], window_size=p["window"],
                                last_n_block=p["last_n"], native_normalize=True, min_budget=mb,
                                block_size=block, batch=B, uniform_seq_len=L)
    call.plan()
    call.pool()
    call.search()
    call.attn()
    torch.cuda.synchronize()
    assert call.status() == 0
    assert not torch.isnan(o_pub.float()).any()
    assert torch.equal(o_pub.view(bits), o_st.view(bits))


def test_concurrent_calls_on_two_streams():
    """Two public calls in flight at once on two streams (default priority),
    each at a size where the attention runs as the persistent grid: each
    stream takes its own cached workspace (so its own claim queues), and both
    outputs equal those of the same calls made one after the other."""
    from flashprefill_amd.runtime import release_workspaces
    T, Hq, Hkv, d = 16384, 32, 8, 128
    cu = torch.tensor([0, T], dtype=torch.int32, device=DEV)
    ins = []
    for s in (61, 71):
        ins.append((_rand((T, Hq, d), s, scale=1.5).to(DEV), _rand((T, Hkv, d), s + 1, scale=1.5).to(DEV),
                    _rand((T, Hkv, d), s + 2).to(DEV)))
    refs = []
    for q, k, v in ins:  # one after the other on the current stream
        o = torch.empty_like(q)
        flash_prefill_varlen_func(q, k, v, o, cu, T, 0.18)
        refs.append(o)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [torch.full_like(q, float("nan")) for q, _, _ in ins]
    torch.cuda.synchronize()
    for rep in range(3):
        for (q, k, v), o, st in zip(ins, outs, streams):
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        for (q, k, v), o, st in zip(ins, outs, streams):
            with torch.cuda.stream(st):
                flash_prefill_varlen_func(q, k, v, o, cu, T, 0.18)
        torch.cuda.synchronize()
        for o, r in zip(outs, refs):
            assert torch.equal(o, r), rep
    release_workspaces()
