"""GPU runs of the weight-free accuracy harness (flashprefill_amd/accuracy.py).

* alpha 0 selects every causal block: the harness must then report full
  recall of needles, hot blocks and stripes, a dense-mass recall of 1 and an
  output equal to its own fp32 dense attention within the bf16 tolerance
  (this checks the harness's bookkeeping and dense reference);
* block-sized needles (a 128-key fact and a 128-row question sharing a
  direction of 8 nats per key) at 32K and alpha 0.18: the selection keeps
  the fact's block for at least 90 % of (needle, query head) pairs."""

import pytest

from flashprefill_amd.accuracy import evaluate_length

pytestmark = pytest.mark.gpu


def test_every_block_selected_gives_full_recall():
    r = evaluate_length(4096, alpha=0.0, n_needles=16, sample_rows=16)
    print(f"\n  {r}", flush=True)
    assert r["density"] == 1.0
    for key in ("needle_recall", "hot_block_recall", "stripe_block_recall"):
        assert r[key] == 1.0, key
    assert abs(r["needle_dense_mass_recall_min"] - 1.0) < 1e-4
    assert abs(r["random_rows_dense_mass_recall_min"] - 1.0) < 1e-4
    assert r["needle_out_err_vs_dense_max"] <= 2e-2


def test_block_sized_needles_are_retrieved():
    r = evaluate_length(32768, alpha=0.18, n_needles=32, needle_len=128, question_len=128,
                        sample_rows=16)
    print(f"\n  {r}", flush=True)
    assert r["needle_recall"] >= 0.9
    assert r["needle_out_err_vs_dense_mean"] <= 2e-2
