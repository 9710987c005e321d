"""bench.py pieces that need no GPU: the single-GPU guard and the contest score model."""

from __future__ import annotations

import pytest

import bench

# Per-case (kernel us, score) of the reference's final C500 submission, as recorded in
# SOTA:submission_clean_cu_67.36.txt:3-6 (total 67.36).
REFERENCE_RESULTS = {1: (7, 84), 2: (7, 84), 3: (9, 83), 4: (19, 75), 5: (15, 75), 6: (24, 67),
                     7: (204, 57), 8: (71, 60), 9: (207, 60), 10: (37, 63), 11: (182, 57),
                     12: (352, 61), 13: (169, 58), 14: (115, 59)}


def test_score_model_reproduces_the_reference_contest_scores():
    """round(100 R / (R + t)) with the fixed per-case R gives every recorded case score and the
    recorded total 67.36 from the recorded kernel times."""
    scores = []
    for case, (t_us, expected) in REFERENCE_RESULTS.items():
        R = bench.C500_SCORE_R_US[case]
        score = round(100 * R / (R + t_us))
        assert score == expected, case
        assert bench.C500_CLEAN_US[case] == t_us
        scores.append(score)
    assert round(sum(scores) / len(scores), 2) == 67.36


def test_case_table_matches_the_reference_harness():
    # bench_all.py:10-16 (batch, seqlen_cap, num_heads_k) and its official iteration counts
    assert bench.W.C500_CASES[1] == (1, 1, 4) and bench.W.C500_CASES[14] == (1, 61519, 4)
    assert set(bench.W.C500_CASES) == set(bench.C500_SCORE_R_US) == set(range(1, 15))


@pytest.mark.parametrize("argv", [["--gpus", "2"], ["--gpus", "8"]])
def test_more_than_one_gpu_is_refused(argv, capsys):
    assert bench.main(argv) == 2
    assert "one GPU" in capsys.readouterr().err


def test_settle_runs_calls_for_the_requested_time(monkeypatch):
    """settle_device issues calls in synchronised batches of 64 until settle_ms has passed, and
    none for settle_ms <= 0 (the host side only: the synchronisation is stubbed)."""
    syncs = []
    monkeypatch.setattr(bench.torch.cuda, "synchronize", lambda: syncs.append(1))
    calls = []
    assert bench.settle_device(calls.append, 0) == 0 and calls == [] and syncs == []
    n = bench.settle_device(calls.append, 5.0)
    assert n == len(calls) and n >= 64 and n % 64 == 0
    assert calls == list(range(n)) and len(syncs) == n // 64
