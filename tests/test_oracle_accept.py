"""Pins the oracle's greedy acceptance (hsd/model.py:419-427) by brute force over every
draft/target combination of a tiny vocabulary, and argmax's first-index tie rule."""
import itertools

import numpy as np

from oracle import hsd_oracle as O


def test_accept_brute_force():
    V, k = 3, 2
    for draft in itertools.product(range(V), repeat=k):
        for tgt in itertools.product(range(V), repeat=k + 1):
            a, emitted, n_keep = O.greedy_accept(draft, tgt)
            # a is the length of the longest prefix on which draft and target agree
            want = 0
            while want < k and draft[want] == tgt[want]:
                want += 1
            assert a == want and n_keep == a + 1
            assert emitted == list(draft[:a]) + [tgt[a]]


def test_argmax_first_index():
    x = np.array([[1.0, 3.0, 3.0, 2.0], [5.0, 5.0, 5.0, 5.0], [-1.0, -2.0, -1.0, -3.0]], np.float32)
    assert O.argmax_first(x).tolist() == [1, 0, 0]
