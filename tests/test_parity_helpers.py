"""CPU checks of the GPU parity tests' own pooled-K criterion (tests/_parity.py
pool_errors): a block mean summed in fp32 and rounded once passes, including
near cancellation, and a planted error in a well-conditioned element fails."""

import torch

from oracle import flashprefill_oracle as O
from tests._parity import pool_errors, ulp_diff_16


def _fp32_pool(k: torch.Tensor, block: int) -> torch.Tensor:
    # what the pooling kernel computes: rows summed in fp32 in row order,
    # times the reciprocal of the valid row count, rounded once
    S, H, d = k.shape
    nb = (S + block - 1) // block
    kp = torch.zeros(nb * block, H, d)
    kp[:S] = k.float()
    acc = torch.zeros(nb, H, d)
    for r in range(block):
        acc = acc + kp.view(nb, block, H, d)[:, r]
    cnt = torch.clamp(S - torch.arange(nb) * block, max=block).float()
    return (acc * (1.0 / cnt).view(nb, 1, 1)).to(k.dtype)


def test_fp32_summed_means_pass_including_cancellation():
    g = torch.Generator().manual_seed(21)
    for S, block, dtype in [(2048, 128, torch.bfloat16), (1000, 128, torch.bfloat16),
                            (129, 64, torch.float16), (1, 128, torch.bfloat16)]:
        k = (torch.randn(S, 4, 64, generator=g) * 2).to(dtype)
        mk_o = O.pool_k(k, block)
        ulp, bad, _ = pool_errors(_fp32_pool(k, block), mk_o, k, block)
        assert ulp <= 1 and bad == 0


def test_cancelling_mean_is_checked_by_the_bound_not_the_ulp():
    # a column whose mean is ~0: fp32 and fp64 sums differ by many bf16 ulps
    # around zero but stay inside the summation bound
    k = torch.ones(128, 1, 1, dtype=torch.bfloat16) * 3.0
    k[1::2] = -3.0
    k[0, 0, 0] = 3.015625
    mk_o = O.pool_k(k, 128)
    gpu = mk_o.clone()
    gpu[0, 0, 0] = mk_o[0, 0, 0].float() + 2.0 ** -16  # < 128 * 2^-24 * 3
    assert ulp_diff_16(gpu, mk_o) > 8
    ulp, bad, _ = pool_errors(gpu, mk_o, k, 128)
    assert bad == 0 and ulp == 0  # the element is not well conditioned, so not in the ulp figure


def test_planted_error_fails():
    g = torch.Generator().manual_seed(5)
    k = (torch.randn(640, 2, 128, generator=g) * 1.5).to(torch.bfloat16)
    mk_o = O.pool_k(k, 128)
    gpu = _fp32_pool(k, 128)
    i = int(mk_o.float().abs().flatten().argmax())
    gpu.view(-1)[i] = (gpu.view(-1)[i].float() * 1.02).to(torch.bfloat16)
    ulp, bad, worst = pool_errors(gpu, mk_o, k, 128)
    assert ulp >= 2 and bad >= 1 and "oracle" in worst
