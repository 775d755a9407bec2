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


# ---- sample() at temperature > 0 (src/inference.rs:128-178) ----------------
# Equal logits make every probability exactly 1/n and the cumulative sums
# exact multiples of it, so the chosen id follows from the drawn u32 alone:
# the expected ids below are fixed by that arithmetic, the generator's own
# next_u32 (pinned by the reference initialisation fixture) and numpy's IEEE
# f32 operations, not by the oracle's code.


def _norm(u: int) -> np.float32:
    return np.float32(u) / np.float32(4294967295.0)


def test_temperature_zero_is_greedy_and_draws_nothing():
    lg = np.float32([9.0, 2.0, 1.9, -0.5, 1.0])
    r = O.Rng(1337)
    s0 = r.state.value
    assert O.sample(lg, [1, 2], r, 0.0, 0.85, 24, 1.25) == O.sample_greedy(lg, [1, 2], 1.25)
    assert r.state.value == s0


def test_top_k_one_is_the_argmax_after_one_draw():
    lg = np.float32([50.0, 0.3, 2.0, 1.0])  # id 0 never competes
    r, probe = O.Rng(7), O.Rng(7)
    for _ in range(5):
        assert O.sample(lg, [], r, 0.7, 1.0, 1) == 2
        probe.next_u32()
        assert r.state.value == probe.state.value
    # The penalty applies first: 2.0 / 2 = 1.0 ties id 3 at 1.0; ties go to the lower id.
    assert O.sample(np.float32([0.0, 0.3, 2.0, 1.0]), [2], r, 1.0, 1.0, 1, 2.0) == 2


def test_equal_logits_pick_the_bucket_of_the_draw():
    lg = np.float32([100.0, 1.0, 1.0, 1.0, 1.0])  # four candidates, p = 0.25 each
    r, probe = O.Rng(1337), O.Rng(1337)
    seen = set()
    for _ in range(64):
        draw = _norm(probe.next_u32()) * np.float32(1.0)  # mass = 4 * 0.25 = 1
        want = 1 + next(i for i in range(4) if draw <= np.float32(0.25) * np.float32(i + 1))
        assert O.sample(lg, [], r, 0.9, 1.0, 24) == want
        seen.add(want)
    assert seen == {1, 2, 3, 4}


def test_top_p_and_top_k_cut_the_candidates():
    lg = np.float32([0.0, 1.0, 1.0, 1.0, 1.0])
    # top_p 0.5: the running sum reaches 0.5 at the second candidate (>=).
    r, probe = O.Rng(99), O.Rng(99)
    for _ in range(64):
        draw = _norm(probe.next_u32()) * np.float32(0.5)
        assert O.sample(lg, [], r, 0.5, 0.5, 24) == (1 if draw <= np.float32(0.25) else 2)
    # top_k 3, top_p 1: ids 1..3, mass 0.75.
    r, probe = O.Rng(5), O.Rng(5)
    for _ in range(64):
        draw = _norm(probe.next_u32()) * np.float32(0.75)
        want = 1 + next(i for i in range(3) if draw <= np.float32(0.25) * np.float32(i + 1))
        assert O.sample(lg, [], r, 2.0, 1.0, 3) == want


def test_frequencies_follow_the_softmax():
    # T = 1: p(2) / p(1) = e^(ln 3) = 3, so id 1 is drawn a quarter of the time.
    lg = np.float32([0.0, 0.0, np.log(3.0)])
    r = O.Rng(2024)
    n = 20000
    ones = sum(O.sample(lg, [], r, 1.0, 1.0, 24) == 1 for _ in range(n))
    assert abs(ones / n - 0.25) < 0.012
    # Temperature 0.5 squares the ratio: 1 in 10.
    ones = sum(O.sample(lg, [], r, 0.5, 1.0, 24) == 1 for _ in range(n))
    assert abs(ones / n - 0.1) < 0.008


def test_sampling_refuses_non_finite_logits():
    r = O.Rng(1)
    for bad in (np.nan, np.inf, -np.inf):
        assert O.sample(np.float32([0.0, bad, 1.0]), [], r, 0.7, 0.85, 24) == -1
