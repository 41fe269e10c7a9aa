"""Seeded synthetic prefill inputs with the structure FlashPrefill searches for.

The inputs are Q/K/V of one or more sequences (packed along tokens, varlen
style) with heads laid out ``(T, H, d)``. Every random draw comes from one
``torch.Generator`` seeded by the caller, so a given spec reproduces the same
tensors on the CPU and (up to the device RNG stream) on the GPU; the CPU
stream is the canonical one used by the parity tests.

Structure, each term described in the units of the attention logit
``s = q.k / sqrt(d)`` (natural log):

* background: Q, K, V ~ N(0, 1) * base, ``base = 1/sqrt(d)`` when ``scaled``
  (the Llama-shaped configs) and 1 otherwise (the 4K fp32 plumbing config);
* sink: K rows 0..sink_rows-1 are multiplied by ``sink_scale`` and aligned
  with a per-KV-head direction that every query shares (token logit
  ``sink_logit``);
* vertical stripes: ``n_stripes`` key positions (runs of ``stripe_width``
  tokens) aligned with a per-KV-head direction shared by all queries (token
  logit ``stripe_logit``);
* slash / local band: a shared multi-frequency rotary phase on a dedicated
  subspace, so ``q_t . k_u`` grows with ``cos(theta (t - u))`` (peak logit
  ``band_logit`` at ``t == u``);
* topic segments: piecewise-constant random offsets over segments of
  64..512 tokens on both Q and K (block-coherent background with logit spread
  ``topic_logit``), which gives the long tail of block scores;
* hot blocks: ``hot_blocks`` random causal (q-block, k-block) pairs per query
  head whose Q and K rows share a per-head direction (logit ``hot_logit``).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field, replace
from typing import List, Optional, Sequence, Tuple

import torch


@dataclass(frozen=True)
class SynthSpec:
    seq_lens: Tuple[int, ...]
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    dtype: torch.dtype = torch.bfloat16
    seed: int = 0
    scaled: bool = True
    sink_rows: int = 4
    sink_scale: float = 4.0
    sink_logit: float = 6.0
    n_stripes: int = 64
    stripe_width: int = 8
    stripe_logit: float = 5.0
    band_logit: float = 3.0
    band_freqs: int = 8
    topic_logit: float = 1.0
    hot_blocks: int = 8
    hot_logit: float = 4.0
    block: int = 128

    @property
    def total_tokens(self) -> int:
        return int(sum(self.seq_lens))

    def cu_seqlens(self) -> List[int]:
        cu = [0]
        for s in self.seq_lens:
            cu.append(cu[-1] + int(s))
        return cu


def config1_spec(seed: int = 0) -> SynthSpec:
    """Config 1: 4096 tokens, 8q/2kv, d=64, fp32, unscaled N(0,1),
    K rows 0-3 x4 (sink) and 16 stripe columns."""
    return SynthSpec(seq_lens=(4096,), num_q_heads=8, num_kv_heads=2, head_dim=64,
                     dtype=torch.float32, seed=seed, scaled=False, sink_logit=0.0,
                     n_stripes=16, stripe_width=1, stripe_logit=3.0, band_logit=0.0,
                     topic_logit=0.0, hot_blocks=0)


def llama_spec(seq_len: int, seed: int, dtype=torch.bfloat16) -> SynthSpec:
    """Configs 2/3: Llama-3-8B head shapes (32q/8kv, d=128)."""
    return SynthSpec(seq_lens=(seq_len,), num_q_heads=32, num_kv_heads=8, head_dim=128,
                     dtype=dtype, seed=seed)


def qwen_varlen_spec(seq_lens: Sequence[int] = (262144, 65536, 17408, 3072, 1024),
                     seed: int = 7, dtype=torch.bfloat16) -> SynthSpec:
    """Config 4: Qwen2.5-7B head shapes (28q/4kv, d=128), ragged batch."""
    return SynthSpec(seq_lens=tuple(int(s) for s in seq_lens), num_q_heads=28,
                     num_kv_heads=4, head_dim=128, dtype=dtype, seed=seed)


def _unit(g: torch.Generator, n: int, d: int, device) -> torch.Tensor:
    x = torch.randn(n, d, generator=g, device=device)
    return x / x.norm(dim=-1, keepdim=True)


def _seq_structure(g: torch.Generator, spec: SynthSpec, S: int,
                   q: torch.Tensor, k: torch.Tensor, device, meta: Optional[dict] = None) -> None:
    """Add the structured terms to one sequence's q (S,Hq,d), k (S,Hkv,d) in place.

    A shared direction with amplitude ``a`` on both a query and a key adds
    ``a*a/sqrt(d)`` to their logit, so ``a = sqrt(logit * sqrt(d))``. When
    ``meta`` is given, the planted positions are recorded in it: "stripes"
    (first token of each stripe run) and "hot" ((head, q-block, k-block)
    triples); the random draws are the same either way.
    """
    Hq, Hkv, d = spec.num_q_heads, spec.num_kv_heads, spec.head_dim
    G = Hq // Hkv
    rd = math.sqrt(d)
    nb = (S + spec.block - 1) // spec.block

    def amp(logit: float) -> float:
        return math.sqrt(max(logit, 0.0) * rd)

    def kv_to_q(x: torch.Tensor) -> torch.Tensor:  # (Hkv, d) -> (Hq, d)
        return x.repeat_interleave(G, dim=0)

    # sink: scaled rows, optionally aligned with a direction all queries share
    if spec.sink_rows > 0:
        r = min(spec.sink_rows, S)
        k[:r] *= spec.sink_scale
        if spec.sink_logit > 0:
            c = _unit(g, Hkv, d, device)
            a = amp(spec.sink_logit)
            k[:r] += a * c.unsqueeze(0)
            q += a * kv_to_q(c).unsqueeze(0)
    # vertical stripes: runs of keys aligned with a direction all queries share
    if spec.n_stripes > 0 and S > spec.block:
        u = _unit(g, Hkv, d, device)
        a = amp(spec.stripe_logit)
        starts = torch.randint(spec.block, S, (spec.n_stripes,), generator=g, device=device)
        if meta is not None:
            meta["stripes"] = starts.tolist()
        for s0 in starts.tolist():
            s1 = min(S, s0 + spec.stripe_width)
            k[s0:s1] = a * u.unsqueeze(0) + 0.25 * k[s0:s1]
        q += a * kv_to_q(u).unsqueeze(0)
    # local band: a shared multi-frequency rotary phase on a random subspace
    if spec.band_logit > 0 and spec.band_freqs > 0:
        F = min(spec.band_freqs, d // 2)
        periods = torch.logspace(math.log10(256.0), math.log10(8192.0), F, device=device)
        theta = 2 * math.pi / periods
        t = torch.arange(S, device=device, dtype=torch.float32)
        ang = t.view(S, 1) * theta.view(1, F)
        rot = torch.stack([torch.cos(ang), torch.sin(ang)], dim=-1).reshape(S, 2 * F)
        basis = torch.linalg.qr(torch.randn(d, 2 * F, generator=g, device=device))[0].T
        band = amp(spec.band_logit / F) * (rot @ basis)  # (S, d); q_t.k_u peaks at t == u
        q += band.unsqueeze(1)
        k += band.unsqueeze(1)
    # topic segments: piecewise-constant offsets over 64..512-token segments
    if spec.topic_logit > 0:
        a = math.sqrt(spec.topic_logit)
        pos = 0
        while pos < S:
            L = int(torch.randint(64, 513, (1,), generator=g, device=device).item())
            e = min(S, pos + L)
            q[pos:e] += a * torch.randn(Hq, d, generator=g, device=device).unsqueeze(0)
            k[pos:e] += a * torch.randn(Hkv, d, generator=g, device=device).unsqueeze(0)
            pos = e
    # hot blocks: causal (q-block, k-block) pairs sharing a per-query-head direction
    if spec.hot_blocks > 0 and nb > 6:
        w = _unit(g, Hq, d, device)
        a = amp(spec.hot_logit)
        for h in range(Hq):
            for _ in range(spec.hot_blocks):
                qb = int(torch.randint(5, nb, (1,), generator=g, device=device).item())
                kb = int(torch.randint(0, qb - 4, (1,), generator=g, device=device).item())
                if meta is not None:
                    meta.setdefault("hot", []).append((h, qb, kb))
                q0, q1 = qb * spec.block, min(S, (qb + 1) * spec.block)
                k0, k1 = kb * spec.block, min(S, (kb + 1) * spec.block)
                q[q0:q1, h] += a * w[h]
                k[k0:k1, h // G] += a * w[h]


def make_inputs(spec: SynthSpec, device="cpu", metas: Optional[List[dict]] = None
                ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Return packed q (T,Hq,d), k (T,Hkv,d), v (T,Hkv,d) in spec.dtype and
    cu_seqlens (B+1,) int32 on ``device``. With ``metas`` (a list), one dict
    per sequence of the planted positions is appended to it."""
    device = torch.device(device)
    Hq, Hkv, d = spec.num_q_heads, spec.num_kv_heads, spec.head_dim
    assert Hq % Hkv == 0
    base = 1.0 / math.sqrt(d) if spec.scaled else 1.0
    T = spec.total_tokens
    qs, ks, vs = [], [], []
    for b, S in enumerate(spec.seq_lens):
        g = torch.Generator(device=device)
        g.manual_seed(spec.seed * 1000003 + b)
        q = torch.randn(S, Hq, d, generator=g, device=device) * base
        k = torch.randn(S, Hkv, d, generator=g, device=device) * base
        v = torch.randn(S, Hkv, d, generator=g, device=device) * base
        meta = {"stripes": [], "hot": []} if metas is not None else None
        _seq_structure(g, spec, S, q, k, device, meta)
        if metas is not None:
            metas.append(meta)
        qs.append(q.to(spec.dtype))
        ks.append(k.to(spec.dtype))
        vs.append(v.to(spec.dtype))
    q = torch.cat(qs) if qs else torch.zeros(0, Hq, d, dtype=spec.dtype, device=device)
    k = torch.cat(ks) if ks else torch.zeros(0, Hkv, d, dtype=spec.dtype, device=device)
    v = torch.cat(vs) if vs else torch.zeros(0, Hkv, d, dtype=spec.dtype, device=device)
    cu = torch.tensor(spec.cu_seqlens(), dtype=torch.int32, device=device)
    assert q.shape[0] == T
    return q, k, v, cu
