"""CPU checks of the GPU parity tests' own pooled-K criterion (tests/_parity.py
pool_errors / assert_pool): a block mean computed the way the pooling kernel
computes it (fp64 row-group sums, fp64 division, cast through fp32) is bit
equal to the oracle's, cancelling columns included; the same mean summed in
fp32 fails the bar where the block mean cancels; a planted error fails. The
output criterion (output_errors): the max-abs bar on elements whose output
spacing is within it, one ulp on the others. The closed-form checker of every
output row agrees with the oracle and catches planted mistakes."""

import torch

from oracle import flashprefill_oracle as O
from tests._parity import (StageReport, assert_pool, every_row_vs_closed_form, output_errors,
                           output_spacing, pool_errors, ulp_diff_16)


def _kernel_pool(k: torch.Tensor, block: int, acc_dtype=torch.float64) -> torch.Tensor:
    # the pooling kernel's order: 256 threads = R row groups x d/8 chunks;
    # row group rg sums rows rg, rg + R, ...; the R partials are added in
    # row-group order; the mean is divided in the accumulation type and cast
    # to the dtype through fp32
    S, H, d = k.shape
    R = 256 // (d // 8)
    nb = (S + block - 1) // block
    kp = torch.zeros(nb * block, H, d, dtype=acc_dtype)
    kp[:S] = k.to(acc_dtype)
    kb = kp.view(nb, block, H, d)
    total = torch.zeros(nb, H, d, dtype=acc_dtype)
    for rg in range(R):
        part = torch.zeros(nb, H, d, dtype=acc_dtype)
        for r in range(rg, block, R):
            part = part + kb[:, r]
        total = total + part
    cnt = torch.clamp(S - torch.arange(nb) * block, max=block).to(acc_dtype)
    return (total / cnt.view(nb, 1, 1)).float().to(k.dtype)


def _cancelling(dtype):
    # a column of +-3 whose block mean is 2^-6 / 128 (cancellation), beside
    # columns of large random values
    g = torch.Generator().manual_seed(11)
    k = (torch.randn(128, 2, 64, generator=g) * 40).to(dtype)
    k[:, 0, 0] = 3.0
    k[1::2, 0, 0] = -3.0
    k[0, 0, 0] = 3.015625
    return k


def test_kernel_order_fp64_means_are_bit_equal():
    g = torch.Generator().manual_seed(21)
    for S, block, dtype, d in [(2048, 128, torch.bfloat16, 128), (1000, 128, torch.bfloat16, 64),
                               (129, 64, torch.float16, 64), (1, 128, torch.bfloat16, 128),
                               (4096, 128, torch.float16, 128)]:
        k = (torch.randn(S, 4, d, generator=g) * 2).to(dtype)
        ulp, diff, _ = pool_errors(_kernel_pool(k, block), O.pool_k(k, block))
        assert ulp == 0 and diff == 0
    k = _cancelling(torch.bfloat16)
    assert pool_errors(_kernel_pool(k, 128), O.pool_k(k, 128))[:2] == (0, 0)


def test_fp32_summed_mean_fails_where_the_mean_cancels():
    # rows of +-1024 that cancel pairwise plus two rows of ~2^-20: an fp32
    # partial sum of ~1024 drops the small rows (its ulp is 2^-13), so the
    # fp32-summed mean is 0 where the exact mean is ~2^-27; the plain ulp bar
    # sees it (the former fp32-summation allowance let such elements pass)
    g = torch.Generator().manual_seed(3)
    k = torch.randn(128, 1, 128, generator=g).to(torch.bfloat16)
    k[0:126:2, 0, 0] = 1024.0
    k[1:126:2, 0, 0] = -1024.0
    k[126, 0, 0] = 2.0 ** -20
    k[127, 0, 0] = 3 * 2.0 ** -22
    mk_o = O.pool_k(k, 128)
    assert mk_o[0, 0, 0].item() > 0
    ulp, diff, worst = pool_errors(_kernel_pool(k, 128, torch.float32), mk_o)
    assert ulp > 1 and diff >= 1, worst
    assert pool_errors(_kernel_pool(k, 128), mk_o)[:2] == (0, 0)


def test_planted_error_fails():
    g = torch.Generator().manual_seed(5)
    k = (torch.randn(640, 2, 128, generator=g) * 1.5).to(torch.bfloat16)
    mk_o = O.pool_k(k, 128)
    gpu = _kernel_pool(k, 128)
    i = int(mk_o.float().abs().flatten().argmax())
    one = gpu.clone()
    one.view(torch.int16).view(-1)[i] += 1  # one ulp: inside the <= 1 bar, but not bit-equal
    ulp, diff, _ = pool_errors(one, mk_o)
    assert ulp == 1 and diff == 1
    rep = StageReport(pool_ulp=ulp, pool_mismatch=diff, pool_exact=True)
    try:
        assert_pool(rep)
    except AssertionError:
        pass
    else:
        raise AssertionError("a 16-bit mismatch must fail the bit-equality bar")
    assert_pool(StageReport(pool_ulp=ulp, pool_mismatch=diff, pool_exact=False))
    gpu.view(-1)[i] = (gpu.view(-1)[i].float() * 1.02).to(torch.bfloat16)
    ulp, diff, worst = pool_errors(gpu, mk_o)
    assert ulp >= 2 and diff >= 1 and "oracle" in worst
    assert ulp_diff_16(gpu, mk_o) == ulp


def test_signed_zeros_are_equal():
    a = torch.tensor([0.0, -0.0, 1.0], dtype=torch.bfloat16)
    b = torch.tensor([-0.0, 0.0, 1.0], dtype=torch.bfloat16)
    assert pool_errors(a, b)[:2] == (0, 0)


def test_output_spacing_matches_the_dtypes():
    for dt, mant in ((torch.bfloat16, 7), (torch.float16, 10), (torch.float32, 23)):
        x = torch.tensor([1.0, 3.5, 4.0, 6.25, -5.0, 0.75], dtype=dt)
        want = torch.tensor([2.0 ** (e - mant) for e in (0, 1, 2, 2, 2, -1)])
        assert torch.equal(output_spacing(x), want), dt
        # one step of the dtype up from x is x + spacing
        step = (x.float() + want).to(dt)
        assert torch.equal(_next_up(x), step), dt


def _next_up(x):
    # the next representable value of x's dtype above x (x > 0 or x < 0, finite)
    i = x.view(torch.int16 if x.element_size() == 2 else torch.int32)
    up = torch.where(x >= 0, i + 1, i - 1)  # sign-magnitude bit patterns
    return up.view(x.dtype)


def test_output_errors_hold_coarse_elements_to_one_ulp():
    bar = 2e-2
    ref = torch.tensor([0.5, 1.5, 3.9, 4.5, -6.0, 9.0], dtype=torch.bfloat16)
    # every element one ulp up: only the coarse ones (|ref| >= 4, spacing
    # 2^-5 and 2^-4 > bar) are exempt from the bar, and they are at 1 ulp
    out = _next_up(ref)
    main, every, n, ulp = output_errors(out, ref, bar)
    assert n == 3 and ulp == 1
    assert main.numel() == 3 and float(main.max()) == 2.0 ** -6  # 3.9: spacing 2^-6 < bar
    assert every.numel() == 6 and float(every.max()) == 2.0 ** -4
    # two ulps on a coarse element are reported as such
    out2 = out.clone()
    out2[3] = _next_up(out[3:4])[0]
    assert output_errors(out2, ref, bar)[3] == 2
    # below 4 the bar applies: 3.9 + 2 ulps (0.031) is above it
    out3 = ref.clone()
    out3[2] = _next_up(_next_up(ref[2:3]))[0]
    main3 = output_errors(out3, ref, bar)[0]
    assert float(main3.max()) > bar
    # fp16 and fp32 outputs of this size have spacings far below the bar
    for dt in (torch.float16, torch.float32):
        r = ref.to(dt)
        assert output_errors(_next_up(r), r, bar)[2] == 0


class _ListsCall:
    """The parts of FlashPrefillCall that every_row_vs_closed_form reads, on
    CPU tensors: sequence tables and per-row index lists in the workspace
    layout (counts at tile[b] + i, list of row i at tri[b] + i(i+1)/2)."""

    def __init__(self, q, k, v, cu, sels):
        self.tensors = (q, k, v, None)
        self.Hq, self.Hkv, self.d = q.shape[1], k.shape[1], q.shape[2]
        nbs = [s.shape[1] for s in sels]
        self.tile = [0]
        self.tri = [0]
        for nb in nbs:
            self.tile.append(self.tile[-1] + nb)
            self.tri.append(self.tri[-1] + nb * (nb + 1) // 2)
        self.start = cu[:-1]
        self.lens = [cu[b + 1] - cu[b] for b in range(len(nbs))]
        self.cnt = torch.zeros(self.Hq, max(self.tile[-1], 1), dtype=torch.int32)
        self.idx = torch.full((self.Hq, max(self.tri[-1], 1)), -7, dtype=torch.int32)
        for b, s in enumerate(sels):
            for h in range(self.Hq):
                for i in range(s.shape[1]):
                    js = torch.nonzero(s[h, i]).flatten()
                    self.cnt[h, self.tile[b] + i] = js.numel()
                    base = self.tri[b] + i * (i + 1) // 2
                    self.idx[h, base:base + js.numel()] = js.to(torch.int32)

    def seq_tables(self):
        return self.tile, self.tri, self.start, self.lens

    def counts(self):
        return self.cnt

    def index_lists(self):
        return self.idx


def _lists_case(block):
    g = torch.Generator().manual_seed(9)
    lens = [300, block, 1, 5 * block + 17]
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    T, Hq, Hkv, d = cu[-1], 4, 2, 64
    q = torch.randn(T, Hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(T, Hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(T, Hkv, d, generator=g).to(torch.bfloat16)
    sels, out = [], torch.zeros(T, Hq, d, dtype=torch.bfloat16)
    for b, n in enumerate(lens):
        nb = (n + block - 1) // block
        sel = torch.tril(torch.rand(Hq, nb, nb, generator=g) < 0.5)
        sel[:, torch.arange(nb), torch.arange(nb)] |= torch.rand(Hq, nb, generator=g) < 0.8
        sels.append(sel)
        s0, s1 = cu[b], cu[b + 1]
        out[s0:s1] = O.sparse_attention(q[s0:s1], k[s0:s1], v[s0:s1], sel, block, min(block, 64))
    return _ListsCall(q, k, v, cu, sels), out


def test_closed_form_checker_agrees_with_the_oracle_attention():
    # the oracle's tiled online softmax (P rounded to bf16, output rounded)
    # against the checker's closed form over the same lists: rounding-level
    # differences only, empty rows (zero output) and partial blocks included
    for block in (128, 64):
        call, out = _lists_case(block)
        assert int((call.cnt == 0).sum()) > 0  # some rows select nothing
        mx, mean, rows = every_row_vs_closed_form(call, out, block=block, max_blocks=7)
        assert rows == sum(call.tile[-1] for _ in range(call.Hq))
        assert mx <= 2e-2 and mean <= 2e-3, (block, mx, mean)


def test_closed_form_checker_catches_planted_mistakes():
    call, out = _lists_case(128)
    mx0, _, _ = every_row_vs_closed_form(call, out, block=128)
    # a wrong output value deep inside a long sequence
    bad = out.clone()
    bad[call.start[3] + 4 * 128 + 9, 2, 5] += 0.25
    assert every_row_vs_closed_form(call, bad, block=128)[0] >= 0.2
    # the outputs of two query heads of one GQA group exchanged
    swapped = out.clone()
    swapped[:, [0, 1]] = out[:, [1, 0]]
    assert every_row_vs_closed_form(call, swapped, block=128)[0] > 10 * max(mx0, 1e-3)
    # one list entry moved to the neighbouring key block
    h, b, i = 1, 3, 4
    c = int(call.cnt[h, call.tile[b] + i])
    base = call.tri[b] + i * (i + 1) // 2
    lst = call.idx[h, base:base + c].tolist()
    free = [j for j in range(i) if j not in lst]
    assert lst and free
    call.idx[h, base] = free[0]
    call.idx[h, base:base + c] = torch.sort(call.idx[h, base:base + c]).values
    assert every_row_vs_closed_form(call, out, block=128)[0] > 10 * max(mx0, 1e-3)
