"""The oracle's sample() at temperature 0 (src/inference.rs:104-127): the
repetition penalty over the last 64 ids of the prompt-plus-generated history,
then the argmax over ids 1..V-1 in total order with ties to the lower id.
Each case is fixed by the rule's own arithmetic (exact in f32)."""
import numpy as np

from oracle import oracle as O


def test_no_penalty_is_the_plain_argmax():
    lg = np.float32([9.0, 2.0, 1.9, -0.5, 1.0])
    assert O.sample_greedy(lg, [1, 1, 2], 1.0) == 1 == O.greedy(lg)  # id 0 never wins


def test_positive_logits_are_divided_negative_ones_multiplied():
    lg = np.float32([9.0, 2.0, 1.9, -0.5, 1.0])
    assert O.sample_greedy(lg, [1], 1.25) == 2  # 2.0 / 1.25 = 1.6 < 1.9
    lg = np.float32([0.0, -1.0, -1.1])
    assert O.sample_greedy(lg, [1], 1.25) == 2  # -1.0 * 1.25 = -1.25 < -1.1
    lg = np.float32([0.0, 0.0, -1e-30])
    assert O.sample_greedy(lg, [1, 1, 1], 2.0) == 1  # 0 * 2 stays 0


def test_each_occurrence_applies_again_within_the_last_64():
    lg = np.float32([0.0, 4.0, 1.5])
    assert O.sample_greedy(lg, [1], 2.0) == 1          # 2.0 > 1.5
    assert O.sample_greedy(lg, [1, 1], 2.0) == 2       # 1.0 < 1.5
    assert O.sample_greedy(lg, [1, 1] + [0] * 63, 2.0) == 1   # one occurrence left in the window
    assert O.sample_greedy(lg, [1, 1] + [0] * 64, 2.0) == 1   # none left


def test_ties_after_the_penalty_go_to_the_lower_id():
    lg = np.float32([0.0, 2.5, 2.0])
    assert O.sample_greedy(lg, [1], 1.25) == 1  # 2.5 / 1.25 == 2.0 exactly


def test_non_finite_logits_are_an_error():
    for bad in (np.nan, np.inf, -np.inf):
        lg = np.float32([bad, 1.0, 2.0])
        assert O.sample_greedy(lg, [], 1.0) == -1
