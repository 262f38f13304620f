"""The drafter call surface on the host (hsd/mtp.py:67-88): ScriptedDrafter's forced
drafts, trim and reset, and the seeded scripted acceptance counts."""
import numpy as np
import torch

from hsd import mtp


def test_scripted_drafter_forces_the_accept_count():
    d = mtp.ScriptedDrafter(vocab=100, n_draft=2)
    h = torch.zeros((1, 8))
    d.script([5, 7], 2)
    assert d(h, None)[0].tolist() == [5, 7]
    d.script([5, 7], 1)
    assert d(h, None)[0].tolist() == [5, 8]            # the first rejected position is wrong
    d.script([5, 99], 0)
    assert d(h, None)[0].tolist() == [6, 99]
    d.script([99, 3], 0)
    assert d(h, None)[0].tolist() == [0, 3]            # wrong modulo the vocabulary
    pred, hn = d(h, None)
    assert hn is h                                     # the hidden state passes through


def test_scripted_drafter_rows_trim_reset():
    d = mtp.ScriptedDrafter(vocab=10)
    d.script([1, 2], 2)
    d(torch.zeros((3, 4)), None)
    d(torch.zeros((1, 4)), None)
    assert d.rows == 4
    d.trim(2)
    assert d.rows == 2
    d.trim(5)
    assert d.rows == 0
    d(torch.zeros((2, 4)), None)
    d.reset()
    assert d.rows == 0


def test_scripted_accepts_are_seeded_and_follow_the_probabilities():
    a = mtp.scripted_accepts(20000, (0.2, 0.34, 0.46), seed=5)
    b = mtp.scripted_accepts(20000, (0.2, 0.34, 0.46), seed=5)
    assert np.array_equal(a, b) and set(np.unique(a)) <= {0, 1, 2}
    freq = np.bincount(a, minlength=3) / a.size
    assert np.all(np.abs(freq - np.array([0.2, 0.34, 0.46])) < 0.015)
    assert np.all(mtp.scripted_accepts(50, (0.0, 0.0, 1.0), seed=1) == 2)
