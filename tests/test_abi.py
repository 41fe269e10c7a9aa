"""CPU checks of the C ABI: the library loads, exports every entry point that
include/flashprefill.h declares, and validates arguments on the host (no GPU
call is made: the descriptors below are rejected before any launch, and the
layout query is pure host arithmetic)."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from flashprefill_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "flashprefill.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fp_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    assert set(_declared()) == set(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.fp_abi_version() == _lib.ABI_VERSION


def _problem(**kw):
    P = _lib.FpProblem()
    P.q = P.k = P.v = P.o = 0x10000
    P.q_stride_tok, P.q_stride_head = 8 * 128, 128
    P.k_stride_tok, P.k_stride_head = 2 * 128, 128
    P.v_stride_tok, P.v_stride_head = 2 * 128, 128
    P.o_stride_tok, P.o_stride_head = 8 * 128, 128
    P.cu_seqlens = 0x20000
    P.batch, P.max_seq_len, P.total_tokens = 3, 4096, 6000
    P.num_q_heads, P.num_kv_heads, P.head_dim = 8, 2, 128
    P.dtype, P.block_size, P.alpha = _lib.FP_DTYPE_BF16, 128, 0.18
    P.attention_sink, P.window_size, P.last_n_block = 2, 4, 2
    for k, v in kw.items():
        setattr(P, k, v)
    return P


def _layout(P):
    L = _lib.FpWsLayout()
    rc = _lib.load().fp_workspace_layout(ctypes.byref(P), ctypes.byref(L))
    return rc, L


def test_layout_bounds():
    rc, L = _layout(_problem())
    assert rc == _lib.FP_OK
    assert L.nb_max == 32
    assert L.nb_sum_cap == (6000 + 127 * 3) // 128
    # worst packing: full sequences of 32 blocks + remainder
    cap = L.nb_sum_cap
    assert L.tri_cap == (cap // 32) * 32 * 33 // 2 + (cap % 32) * (cap % 32 + 1) // 2
    offs = [L.status_off, L.seq_tile_off, L.seq_tri_off, L.seq_start_off, L.seq_len_off,
            L.items_off, L.mk_off, L.cnt_off, L.rowrec_off, L.idx_off, L.units_off,
            L.part_off]
    assert offs == sorted(offs) and all(o % 256 == 0 for o in offs)
    assert L.units_off >= L.idx_off + 4 * 8 * L.tri_cap
    assert L.total_bytes >= L.part_off + 4 * 8 * L.unit_cap * (128 * 128 + 2 * 128)
    assert _lib.load().fp_workspace_bytes(ctypes.byref(_problem())) == L.total_bytes


def test_split_row_policy():
    # last_n rows select every causal block; on 16-bit inputs rows longer than C
    # blocks run as chunks of at most C, where C is about one resident slot's
    # share of a lower bound of the attention's blocks (forced blocks of every
    # row plus the last_n rows' full lists over 512 slots at block 128), at
    # least 8 and at most 8 chunks per row, evened out over the longest row
    rc, L = _layout(_problem())  # 3 sequences, NB <= 32, 8 heads: C = 8, 3 x 2 rows x 4 chunks
    assert rc == _lib.FP_OK and L.split_blocks == 8 and L.unit_cap == 24

    def one(S, hq, hkv):
        return dict(batch=1, max_seq_len=S, total_tokens=S, num_q_heads=hq, num_kv_heads=hkv,
                    q_stride_tok=hq * 128, k_stride_tok=hkv * 128, v_stride_tok=hkv * 128,
                    o_stride_tok=hq * 128)
    # 32 heads: 4K rows of 32 blocks in two chunks (32 x 32 x (6 + 2) / 512 = 16 blocks a
    # slot), 128K in two chunks of 512
    rc, L = _layout(_problem(**one(4096, 32, 8)))
    assert rc == _lib.FP_OK and L.split_blocks == 16 and L.unit_cap == 2 * 2
    rc, L = _layout(_problem(**one(131072, 32, 8)))
    assert rc == _lib.FP_OK and L.split_blocks == 512 and L.unit_cap == 2 * 2
    # one TP = 8 shard of 128K (4 q / 1 kv head): a slot's share is 64 blocks, so the
    # dense rows run as 8 chunks (the most) instead of being the kernel's critical path
    rc, L = _layout(_problem(**one(131072, 4, 1)))
    assert rc == _lib.FP_OK and L.split_blocks == 128 and L.unit_cap == 2 * 8
    for off in (dict(dtype=_lib.FP_DTYPE_F32), dict(last_n_block=0),
                dict(max_seq_len=1024, total_tokens=3 * 1024)):  # fp32, no dense rows, NB <= 8
        rc, L = _layout(_problem(**off))
        assert rc == _lib.FP_OK and L.split_blocks == 0 and L.unit_cap == 0
    # many long sequences: every row's share is small anyway, so no split
    rc, L = _layout(_problem(batch=512, max_seq_len=8192, total_tokens=512 * 8192,
                             num_q_heads=32))
    assert rc == _lib.FP_OK and L.split_blocks == 0


@pytest.mark.parametrize("B,S,hq,d,block", [(256, 4096, 32, 128, 128), (512, 2048, 32, 128, 128),
                                            (64, 4096, 28, 128, 64), (4, 4096, 32, 128, 128),
                                            (1, 4096, 32, 128, 128), (2, 32768, 64, 128, 128),
                                            (4096, 1024, 32, 64, 64)])
def test_split_partials_stay_within_their_byte_budget(B, S, hq, d, block):
    # the chunk partials (fp32 O^T, m, l per unit and query head) are held to
    # 64 MiB, so batches of many short sequences keep a workspace of tens of MB
    rc, L = _layout(_problem(batch=B, max_seq_len=S, total_tokens=B * S, num_q_heads=hq,
                             num_kv_heads=hq // 4, head_dim=d, block_size=block,
                             q_stride_tok=hq * d, q_stride_head=d, k_stride_tok=hq // 4 * d,
                             k_stride_head=d, v_stride_tok=hq // 4 * d, v_stride_head=d,
                             o_stride_tok=hq * d, o_stride_head=d))
    assert rc == _lib.FP_OK
    assert L.total_bytes - L.part_off <= 64 << 20
    assert L.unit_cap * hq * 4 * (block * d + 2 * block) <= 64 << 20
    if B == 1:
        assert L.split_blocks > 0  # a single 4K sequence still splits its dense rows


def test_layout_block_256_plans_in_128_token_blocks():
    # block_size 256 selects 256-token blocks over a 128-token plan: the
    # items, counts, lists and pooled-key slots are those of block 128
    rc256, L256 = _layout(_problem(block_size=256))
    rc128, L128 = _layout(_problem(block_size=128))
    assert rc256 == rc128 == _lib.FP_OK
    for f in ("nb_max", "nb_sum_cap", "tri_cap", "mk_off", "cnt_off", "rowrec_off", "idx_off",
              "total_bytes"):
        assert getattr(L256, f) == getattr(L128, f), f
    # up to 8192 plan blocks per sequence: 1,048,576 tokens
    rc, _ = _layout(_problem(block_size=256, max_seq_len=8192 * 128, total_tokens=8192 * 128,
                             batch=1))
    assert rc == _lib.FP_OK
    rc, _ = _layout(_problem(block_size=256, max_seq_len=8192 * 128 + 1, batch=1))
    assert rc == _lib.FP_E_INVALID_ARG


@pytest.mark.parametrize("field,value,code", [
    ("dtype", _lib.FP_DTYPE_F32, _lib.FP_E_UNSUPPORTED),
    ("head_dim", 96, _lib.FP_E_UNSUPPORTED),
    ("q_stride_tok", 100, _lib.FP_E_INVALID_ARG),
    ("num_positions", 0, _lib.FP_E_INVALID_ARG),
    ("positions", None, _lib.FP_E_INVALID_ARG),
])
def test_rope_arguments_rejected_on_host(field, value, code):
    a = _lib.FpRopeArgs()
    a.q = a.k = a.positions = a.cos_table = a.sin_table = 0x10000
    a.q_stride_tok, a.q_stride_head = 12 * 128, 128
    a.k_stride_tok, a.k_stride_head = 12 * 128, 128
    a.num_tokens, a.num_positions = 5, 8
    a.num_q_heads, a.num_kv_heads, a.head_dim, a.dtype = 8, 2, 128, _lib.FP_DTYPE_BF16
    setattr(a, field, value)
    lib = _lib.load()
    assert lib.fp_rope_qk(ctypes.byref(a), None) == code
    assert lib.fp_last_error()


def test_split_units_never_exceed_the_capacity():
    # restatement of the plan kernel's chunk emission (fp_plan_pool.hip, pass 2) on
    # random ragged batches: the units it writes stay within the host's unit_cap
    import random
    rnd = random.Random(5)
    for trial in range(300):
        B = rnd.choice([1, 2, 3, 5, 17])
        hq = rnd.choice([2, 8, 32])
        block = rnd.choice([64, 128])
        max_len = rnd.choice([700, 2048, 5000, 20000])
        lens = [rnd.randint(0, max_len) for _ in range(B)]
        lens[0] = max_len
        last_n = rnd.choice([1, 2, 3, 7])
        T = sum(lens) + rnd.randint(0, 300)
        rc, L = _layout(_problem(batch=B, max_seq_len=max_len, total_tokens=T,
                                 block_size=block, last_n_block=last_n, num_q_heads=hq,
                                 num_kv_heads=2 if hq > 2 else 1, q_stride_tok=hq * 128,
                                 o_stride_tok=hq * 128))
        assert rc == _lib.FP_OK
        C = L.split_blocks
        n = 0
        for Ls in lens:
            nb = -(-Ls // block)
            for i in range(max(nb - last_n, 0), nb):
                if C > 0 and i + 1 > C:
                    assert -(-(i + 1) // C) <= 8  # the merges combine at most 8
                    n += -(-(i + 1) // C)
        assert n <= L.unit_cap, (lens, block, last_n, C, n, L.unit_cap)


def test_layout_bounds_block_64():
    rc, L = _layout(_problem(block_size=64))
    assert rc == _lib.FP_OK
    assert L.nb_max == 64
    assert L.nb_sum_cap == (6000 + 63 * 3) // 64
    cap = L.nb_sum_cap
    assert L.tri_cap == (cap // 64) * 64 * 65 // 2 + (cap % 64) * (cap % 64 + 1) // 2
    # 8192 blocks per sequence: 524288 tokens at block 64
    rc, _ = _layout(_problem(block_size=64, max_seq_len=8192 * 64, total_tokens=8192 * 64,
                             batch=1))
    assert rc == _lib.FP_OK
    rc, _ = _layout(_problem(block_size=64, max_seq_len=8192 * 64 + 1, batch=1))
    assert rc == _lib.FP_E_INVALID_ARG


@pytest.mark.parametrize("field,value,code", [
    ("dtype", 7, _lib.FP_E_UNSUPPORTED),
    ("head_dim", 96, _lib.FP_E_UNSUPPORTED),
    ("head_dim", 512, _lib.FP_E_UNSUPPORTED),
    ("block_size", 512, _lib.FP_E_UNSUPPORTED),
    ("block_size", 96, _lib.FP_E_UNSUPPORTED),
    ("num_kv_heads", 3, _lib.FP_E_INVALID_ARG),
    ("batch", 0, _lib.FP_E_INVALID_ARG),
    ("max_seq_len", 0, _lib.FP_E_INVALID_ARG),
    ("q", 0x10002, _lib.FP_E_INVALID_ARG),
    ("k_stride_tok", 100, _lib.FP_E_INVALID_ARG),
    ("min_budget", -1, _lib.FP_E_INVALID_ARG),
    ("native_normalize", 2, _lib.FP_E_INVALID_ARG),
])
def test_invalid_arguments_rejected_on_host(field, value, code):
    rc, _ = _layout(_problem(**{field: value}))
    assert rc == code
    assert _lib.load().fp_last_error()


def test_pooled_keys_of_many_kv_heads():
    # pooled keys are addressed chunk-major from a 64-bit base per chunk row,
    # so the kv-head count does not bound the pooled keys of one sequence
    def wide(hkv):
        return _problem(batch=1, max_seq_len=32768, total_tokens=32768, num_q_heads=hkv,
                        num_kv_heads=hkv, q_stride_tok=hkv * 128, o_stride_tok=hkv * 128,
                        k_stride_tok=hkv * 128, v_stride_tok=hkv * 128)
    rc, _ = _layout(wide(32768))  # 2^31 bytes of pooled keys
    assert rc == _lib.FP_OK


def test_uniform_batch_bounds():
    rc, _ = _layout(_problem(cu_seqlens=None, uniform_seq_len=2000, batch=3))
    assert rc == _lib.FP_OK
    rc, _ = _layout(_problem(cu_seqlens=None, uniform_seq_len=5000, batch=1))
    assert rc == _lib.FP_E_INVALID_ARG  # longer than max_seq_len


def test_check_maps_codes_to_python_exceptions():
    rc, _ = _layout(_problem(head_dim=96))
    with pytest.raises(NotImplementedError):
        _lib.check(rc)
    rc, _ = _layout(_problem(num_kv_heads=3))
    with pytest.raises(ValueError):
        _lib.check(rc)


def test_ops_shim_exposes_the_reference_module_layout():
    # the reference's callers import `from ops import ...` and
    # `from ops.flashprefill_native_forward import flash_prefill`
    import inspect
    import ops
    from ops.flashprefill_native_forward import flash_prefill
    from ops.flashprefill_varlen_func import flash_prefill_varlen_func
    import flashprefill_amd
    assert ops.flash_prefill is flash_prefill is flashprefill_amd.flash_prefill
    assert ops.flash_prefill_varlen_func is flash_prefill_varlen_func is \
        flashprefill_amd.flash_prefill_varlen_func
    assert list(inspect.signature(flash_prefill_varlen_func).parameters)[:11] == [
        "q", "k", "v", "o", "cu_seqlens", "max_seq_len", "alpha", "block_size",
        "attention_sink", "window_size", "last_n_block"]


def test_class_level_forwards_map_arguments_like_the_reference(monkeypatch):
    # FlashPrefill.apply / FlashPrefill_varlen.apply (the reference's
    # autograd.Function entry points) hand their arguments to the function
    # entry points exactly as the reference's wrappers do, and check k_stride
    import torch
    import flashprefill_amd.flashprefill_native_forward as nf
    import flashprefill_amd.flashprefill_varlen_func as vf
    from ops.flashprefill_native_forward import FlashPrefill
    from ops.flashprefill_varlen_func import FlashPrefill_varlen
    seen = {}
    monkeypatch.setattr(nf, "flash_prefill", lambda *a: seen.setdefault("native", a))
    monkeypatch.setattr(vf, "flash_prefill_varlen_func", lambda *a: seen.setdefault("varlen", a))
    q, k, v, o = (torch.zeros(1) for _ in range(4))
    assert FlashPrefill.apply(q, k, v, o, 128, 128, 3, 5, 0.25, 1, 7, 11, 13) is None
    assert seen["native"][4:] == (128, 3, 5, 0.25, 1, 11)
    cu = torch.zeros(2, dtype=torch.int32)
    assert FlashPrefill_varlen.apply(q, k, v, o, cu, 4096, 128, 128, 3, 5, 0.25, 1) is None
    assert seen["varlen"][5:] == (4096, 0.25, 128, 3, 5, 1)
    with pytest.raises(ValueError):
        FlashPrefill.apply(q, k, v, o, 128, 64)
    with pytest.raises(ValueError):
        FlashPrefill_varlen.apply(q, k, v, o, cu, 4096, 128, 64)


def _plan_block_count(cu, total, max_len, reject_overlap=True):
    """The plan kernel's per-sequence rule restated on the host: sequences
    outside [0, total], of negative length or (with ``reject_overlap``)
    starting before an earlier cu_seqlens entry are skipped, as are those
    longer than max_len; returns (sum NB, sum NB (NB + 1) / 2) of the kept."""
    nb_sum = tri_sum = 0
    run_max = None
    for b in range(len(cu) - 1):
        start, end = cu[b], cu[b + 1]
        run_max = start if run_max is None else max(run_max, start)
        n = end - start
        if start < 0 or n < 0 or end > total or (reject_overlap and run_max > start):
            continue
        if n > max_len:
            continue
        nb = (n + 127) // 128
        nb_sum += nb
        tri_sum += nb * (nb + 1) // 2
    return nb_sum, tri_sum


def test_plan_rule_keeps_block_count_within_workspace_capacity():
    # [0, T, 0, T]: checking each sequence on its own keeps sequences 0 and 2
    # (2048 blocks at T = 131072, twice the capacity); rejecting a sequence
    # that starts before an earlier entry keeps only sequence 0
    T = 131072
    rc, L = _layout(_problem(batch=3, max_seq_len=T, total_tokens=T))
    assert rc == _lib.FP_OK
    cu = [0, T, 0, T]
    assert _plan_block_count(cu, T, T, reject_overlap=False)[0] == 2048 > L.nb_sum_cap
    nb_sum, tri_sum = _plan_block_count(cu, T, T)
    assert nb_sum == 1024 <= L.nb_sum_cap and tri_sum <= L.tri_cap


def test_plan_rule_bound_holds_for_arbitrary_cu_seqlens():
    # any int32 cu_seqlens (decreasing, negative, overlapping, past the end):
    # the kept sequences never need more than the layout's capacities
    import random
    rnd = random.Random(5)
    for _ in range(2000):
        B = rnd.randint(1, 12)
        T = rnd.randint(0, 5000)
        max_len = rnd.randint(1, 4000)
        cu = [rnd.choice([rnd.randint(-50, T + 50), rnd.randint(0, T)]) for _ in range(B + 1)]
        if rnd.random() < 0.5:
            cu = sorted(cu)
        rc, L = _layout(_problem(batch=B, max_seq_len=max_len, total_tokens=T))
        assert rc == _lib.FP_OK
        nb_sum, tri_sum = _plan_block_count(cu, T, max_len)
        assert nb_sum <= L.nb_sum_cap and tri_sum <= L.tri_cap, (cu, T, max_len)


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    # the GPU path has no CPU fallback: without the built library loading it
    # raises, and CPU tensors are refused rather than computed some other way
    monkeypatch.setattr(_lib, "_LIB", None)
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load(tmp_path / "libflashprefill.so")
    from flashprefill_amd import flash_prefill_varlen_func
    q = torch.zeros(4, 2, 64, dtype=torch.bfloat16)
    kv = torch.zeros(4, 1, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensor"):
        flash_prefill_varlen_func(q, kv, kv, torch.empty_like(q),
                                  torch.tensor([0, 4], dtype=torch.int32), 4, 0.18)
