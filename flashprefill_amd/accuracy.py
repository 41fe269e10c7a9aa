"""Weight-free accuracy harness: needle retrieval on synthetic prefill inputs.

The reference validates FlashPrefill only end to end, by RULER accuracy of
real models (``ruler/eval.py:183-231``, scoring ``ruler/data.py:506-512``),
which needs model weights that are not available here. This harness measures
what that accuracy rests on, directly on the attention operator:

* needles: a span of ``needle_len`` keys starting at a random position
  ``p`` (the "fact") and a span of ``question_len`` query rows starting at
  ``r`` further on (the "question") share a random direction (logit
  ``needle_logit`` nats per key); a (needle, query head) pair is recalled
  when the fact's block is in the selection of the question's q-block for
  that head. Facts and questions sit outside the forced blocks (after the
  sink blocks, more than the window apart, before the last dense
  q-blocks), so only the score threshold can keep them. A single-token
  needle is invisible to block scoring on principle: the pooled key of a
  block carries 1/128 of any one key;
* the structure ``synth`` plants: recall of the hot (q-block, k-block) pairs
  per head, and of the vertical-stripe blocks over every later row;
* dense-mass recall: the share of dense causal attention's probability mass
  (fp32, the same q / k) that falls in the selected blocks, on the needle
  rows and on a random sample of rows;
* output error against dense causal attention (fp32) on the needle rows.

Run ``python -m flashprefill_amd.accuracy [--lengths 4096,...]`` on a GPU:
one JSON line per length.
"""

from __future__ import annotations

import argparse
import json
import math
from typing import Dict, List, Sequence, Tuple

import torch

from . import synth
from .runtime import FlashPrefillCall

BLOCK = 128


def plant_needles(q: torch.Tensor, k: torch.Tensor, S: int, num_kv_heads: int, n: int,
                  logit: float, g: torch.Generator, needle_len: int = 64,
                  question_len: int = 32, sink: int = 2, window: int = 4,
                  last_n: int = 2) -> List[Tuple[int, int, int]]:
    """Add ``n`` needles to one sequence's q (S, Hq, d) / k (S, Hkv, d) in
    place; returns (kv head, first fact key, first question row) triples.
    Each span lies inside one block; fact blocks avoid the sink blocks,
    question blocks the window after the fact and the last dense q-blocks."""
    Hq, d = q.shape[1], q.shape[2]
    G = Hq // num_kv_heads
    nb = (S + BLOCK - 1) // BLOCK
    a = math.sqrt(logit * math.sqrt(d))
    out = []
    hi_blk = nb - last_n - 1  # last q-block that is not forced dense
    if hi_blk - window <= sink:
        raise ValueError(f"sequence of {S} tokens is too short for needles")
    for _ in range(n):
        kvh = int(torch.randint(0, num_kv_heads, (1,), generator=g))
        kb = int(torch.randint(sink, hi_blk - window + 1, (1,), generator=g))
        qb = int(torch.randint(kb + window, hi_blk + 1, (1,), generator=g))
        p = kb * BLOCK + int(torch.randint(0, BLOCK - needle_len + 1, (1,), generator=g))
        r = qb * BLOCK + int(torch.randint(0, BLOCK - question_len + 1, (1,), generator=g))
        u = torch.randn(d, generator=g)
        u = (u / u.norm()).to(q.device)
        k[p:p + needle_len, kvh] += (a * u).to(k.dtype)
        q[r:r + question_len, kvh * G:(kvh + 1) * G] += (a * u).to(q.dtype)
        out.append((kvh, p, r))
    return out


def _dense_row(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, r: int, h: int, G: int
               ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Dense causal attention of query row r, head h in fp32: (probabilities
    over keys 0..r, output)."""
    kk = k[:r + 1, h // G].float()
    s = kk @ q[r, h].float() / math.sqrt(q.shape[-1])
    p = torch.softmax(s, dim=0)
    return p, p @ v[:r + 1, h // G].float()


def evaluate_length(S: int, *, seed: int = 0, alpha: float = 0.18, n_needles: int = 32,
                    needle_logit: float = 8.0, needle_len: int = 64, question_len: int = 32,
                    sample_rows: int = 64, device: str = "cuda:0") -> Dict:
    """One single-sequence case with Llama-3-8B heads (32 q / 8 kv, d 128,
    bf16) and the bench's structured background."""
    dev = torch.device(device)
    spec = synth.llama_spec(S, seed=seed)
    metas: List[dict] = []
    q, k, v, cu = synth.make_inputs(spec, device=dev, metas=metas)
    g = torch.Generator().manual_seed(10_000 + seed)
    needles = plant_needles(q, k, S, spec.num_kv_heads, n_needles, needle_logit, g,
                            needle_len, question_len)
    Hq, G = spec.num_q_heads, spec.num_q_heads // spec.num_kv_heads
    o = torch.empty_like(q)
    call = FlashPrefillCall(q, k, v, o, cu, S, alpha=alpha)
    call.run()
    torch.cuda.synchronize()
    if call.status():
        raise RuntimeError(f"status flags {call.status():#x}")
    sel = call.selection_masks()[0]  # (Hq, nb, nb) bool
    nb = sel.shape[-1]

    # needles: recall per (needle, head); dense mass, fact mass and output
    # error on the question rows (every 8th row of each question span)
    hit = pairs = 0
    err_max, err_sum, n_err, mass_needle, fact_mass = 0.0, 0.0, 0, [], []
    for kvh, p, r0 in needles:
        for h in range(kvh * G, (kvh + 1) * G):
            hit += bool(sel[h, r0 // BLOCK, p // BLOCK])
            pairs += 1
            for r in range(r0, r0 + question_len, 8):
                probs, o_dense = _dense_row(q, k, v, r, h, G)
                keep = sel[h, r // BLOCK].to(dev).repeat_interleave(BLOCK)[:r + 1]
                mass_needle.append(float(probs[keep].sum()))
                fact_mass.append(float(probs[p:p + needle_len].sum()))
                d_ = (o[r, h].float() - o_dense).abs()
                err_max = max(err_max, float(d_.max()))
                err_sum += float(d_.sum())
                n_err += d_.numel()
    # planted structure
    hot = metas[0]["hot"]
    hot_hits = sum(bool(sel[h, qb, kb]) for h, qb, kb in hot)
    stripe_blocks = sorted({s0 // BLOCK for s0 in metas[0]["stripes"]})
    stripe_hits = stripe_total = 0
    for kb in stripe_blocks:
        col = sel[:, kb + 1:, kb]  # every later row of every head
        stripe_hits += int(col.sum())
        stripe_total += col.numel()
    # dense-mass recall on random rows
    gr = torch.Generator().manual_seed(20_000 + seed)
    mass_rand = []
    for _ in range(sample_rows):
        h = int(torch.randint(0, Hq, (1,), generator=gr))
        r = int(torch.randint(0, S, (1,), generator=gr))
        probs, _ = _dense_row(q, k, v, r, h, G)
        keep = sel[h, r // BLOCK].to(dev).repeat_interleave(BLOCK)[:r + 1]
        mass_rand.append(float(probs[keep].sum()))
    causal = Hq * nb * (nb + 1) // 2
    return {
        "seq_len": S, "alpha": alpha, "density": int(sel.sum()) / causal,
        "needles": len(needles), "needle_logit": needle_logit, "needle_len": needle_len,
        "question_len": question_len, "needle_recall": hit / pairs,
        "fact_dense_mass_mean": sum(fact_mass) / len(fact_mass),
        "needle_dense_mass_recall_mean": sum(mass_needle) / len(mass_needle),
        "needle_dense_mass_recall_min": min(mass_needle),
        "needle_out_err_vs_dense_max": err_max, "needle_out_err_vs_dense_mean": err_sum / n_err,
        "hot_block_recall": hot_hits / max(len(hot), 1),
        "stripe_block_recall": stripe_hits / max(stripe_total, 1),
        "random_rows_dense_mass_recall_mean": sum(mass_rand) / len(mass_rand),
        "random_rows_dense_mass_recall_min": min(mass_rand),
    }


def main(argv: Sequence[str] = ()) -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--lengths", default="4096,16384,32768,65536,131072,262144")
    ap.add_argument("--alpha", type=float, default=0.18)
    ap.add_argument("--needles", type=int, default=32)
    ap.add_argument("--needle-logit", type=float, default=8.0)
    ap.add_argument("--needle-len", type=int, default=64)
    ap.add_argument("--question-len", type=int, default=32)
    args = ap.parse_args(list(argv) or None)
    for S in (int(x) for x in args.lengths.split(",")):
        res = evaluate_length(S, alpha=args.alpha, n_needles=args.needles,
                              needle_logit=args.needle_logit, needle_len=args.needle_len,
                              question_len=args.question_len)
        print(json.dumps({k: (round(v, 5) if isinstance(v, float) else v)
                          for k, v in res.items()}), flush=True)
        torch.cuda.empty_cache()


if __name__ == "__main__":
    main()
