"""The memory value cap in the oracle (set_value_cap / clamp_value,
src/memory.rs:114-170), pinned by the reference's own bank tests
(src/memory.rs:695-800) and a closed form."""
import numpy as np

from oracle import oracle as O


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32).copy()


def assert_capped(values, cap):
    v = np.asarray(values, np.float64)
    assert np.all(np.isfinite(v))
    assert np.sum(v * v) <= float(np.float32(cap)) ** 2


def metadata(bank):
    return (bits(bank.keys).tolist(), bits(bank.norm_sq).tolist(), bank.count, bank._blk.mem_write_head,
            bits(bank.confidence).tolist(), bank.last_seen.tolist())


def test_clamp_closed_form():
    np.testing.assert_array_equal(O.clamp_value([3.0, 4.0], 2.5), np.float32([1.5, 2.0]))
    np.testing.assert_array_equal(O.clamp_value([0.3, 0.4], 2.5), np.float32([0.3, 0.4]))
    for cap in (1e-3, 0.7, 3.0):
        v = O.clamp_value(np.random.default_rng(1).standard_normal(77) * 5, cap)
        assert_capped(v, cap)


def test_value_cap_clamps_insert_and_ring_overwrite_without_changing_metadata():
    """src/memory.rs:695-713."""
    uncapped, capped = O.Bank(2, 2, 2), O.Bank(2, 2, 2)
    capped.set_value_cap(2.0)
    for key, value in [([0.25, -0.125], [6.0, 8.0]), ([-0.5, 0.25], [0.0, -1.0]), ([0.125, 0.0], [30.0, -40.0])]:
        idx = uncapped.insert(key, value)
        assert capped.insert(key, value) == idx
        assert metadata(capped) == metadata(uncapped)
        for stored in capped.values:
            assert_capped(stored, 2.0)
    assert capped._blk.mem_write_head == 1
    np.testing.assert_array_equal(capped.values[1], [0.0, -1.0])


def test_value_cap_clamps_protected_writes_but_not_defended_values():
    """src/memory.rs:715-737."""
    bank = O.Bank(1, 1, 2)
    bank.set_value_cap(1.0)
    assert bank.insert_protected([0.1], [3.0, 4.0], 0.0, 1) == 0
    assert_capped(bank.values, 1.0)
    before = (bits(bank.values), bits(bank.keys), bits(bank.norm_sq))
    assert bank.insert_protected([0.2], [30.0, 40.0], 0.0, 2) == -1
    after = (bits(bank.values), bits(bank.keys), bits(bank.norm_sq))
    for a, b in zip(before, after):
        np.testing.assert_array_equal(a, b)
    assert bank.insert_protected([0.2], [-30.0, 40.0], 1e6, 1000) == 0
    assert_capped(bank.values, 1.0)
    assert bank.values[0, 0] < 0.0
    np.testing.assert_array_equal(bank.keys[:, 0], np.float32([0.2]))
    assert bank.norm_sq[0] == O.squared_norm(np.float32([0.2]))
    assert bank.confidence[0] == 1.0 and bank.last_seen[0] == 1000


def test_enabling_value_cap_clamps_existing_and_unused_slots_only():
    """src/memory.rs:739-756."""
    bank = O.Bank(3, 2, 2)
    bank.insert([0.25, -0.5], [3.0, 4.0])
    bank.insert([-0.125, 0.25], [0.125, -0.25])
    bank.values[2] = [10.0, -20.0]  # checkpoints store every capacity slot
    bank.confidence[0] = 3.5
    bank.last_seen[0] = 42
    before = metadata(bank)
    kept = bits(bank.values[1])
    bank.set_value_cap(1.0)
    assert bank.value_cap == 1.0
    assert metadata(bank) == before
    for v in bank.values:
        assert_capped(v, 1.0)
    np.testing.assert_array_equal(bits(bank.values[1]), kept)


def test_value_cap_can_be_tightened_and_disabled_without_restoring_values():
    """src/memory.rs:758-777."""
    bank = O.Bank(1, 1, 2)
    bank.insert([0.0], [3.0, 4.0])
    bank.set_value_cap(4.0)
    assert_capped(bank.values, 4.0)
    capped = bits(bank.values)
    bank.set_value_cap(10.0)
    np.testing.assert_array_equal(bits(bank.values), capped)
    bank.set_value_cap(0.5)
    assert_capped(bank.values, 0.5)
    capped = bits(bank.values)
    bank.set_value_cap(None)
    assert bank.value_cap is None
    np.testing.assert_array_equal(bits(bank.values), capped)
    bank.insert([0.0], [30.0, 40.0])
    np.testing.assert_array_equal(bits(bank.values), bits([[30.0, 40.0]]))


def test_disabled_value_cap_preserves_exact_copy_bits():
    """src/memory.rs:779-800."""
    bank = O.Bank(1, 1, 8)
    value = np.array([0.0, -0.0, np.finfo(np.float32).max, -np.finfo(np.float32).max, 0.0, np.inf, -np.inf, 0.0],
                     np.float32)
    value.view(np.uint32)[4] = 0x7FC01234
    value.view(np.uint32)[7] = 1
    bank.insert([0.0], value)
    np.testing.assert_array_equal(bits(bank.values[0]), bits(value))


def test_product_host_cap_equals_the_oracle_clamp_bit_for_bit():
    """ModelWeights.set_value_cap (the library's host code) against the
    oracle's clamp_value on every slot, including unused ones."""
    from pssa_amd import ModelWeights, PSSAConfig
    cfg = PSSAConfig(depth=2, d_vocab=20, d_latent=24, d_state=4, d_mem_key=4, mem_capacity=12)
    w = ModelWeights.init(cfg, 3, "baseline")
    w.populate_banks(4, 9)
    rng = np.random.default_rng(5)
    for b in w.blocks:
        b.mem_values[:] = (rng.standard_normal(b.mem_values.shape) * rng.uniform(0.01, 3, (12, 1))).astype(np.float32)
    want = [np.stack([O.clamp_value(v, 0.75) for v in b.mem_values]) for b in w.blocks]
    w.set_value_cap(0.75)
    for b, wv in zip(w.blocks, want):
        np.testing.assert_array_equal(bits(b.mem_values), bits(wv))
        assert b.mem_value_cap == np.float32(0.75)
    w.set_value_cap(None)
    assert all(b.mem_value_cap == 0.0 for b in w.blocks)


def test_non_finite_capped_values_are_refused_and_nothing_changes():
    """clamp_value asserts a finite squared norm (src/memory.rs:151-152):
    the oracle, the library's host cap and a capped insert refuse a value
    with an infinite or NaN component and leave every bank as it was."""
    from pssa_amd import ModelWeights, PSSAConfig
    from pssa_amd._abi import HipError
    import pytest

    for bad in (np.inf, np.nan):
        with pytest.raises(ValueError, match="must be finite"):
            O.clamp_value([1.0, bad, 0.5], 0.5)
        bank = O.Bank(3, 1, 2)
        bank.insert([0.1], [3.0, 4.0])
        bank.insert([0.2], [bad, 1.0])
        before = bits(bank.values).tolist()
        with pytest.raises(ValueError, match="must be finite"):
            bank.set_value_cap(1.0)
        assert bits(bank.values).tolist() == before and bank.value_cap is None
        capped = O.Bank(2, 1, 2)
        capped.set_value_cap(1.0)
        with pytest.raises(ValueError, match="must be finite"):
            capped.insert([0.1], [bad, 0.0])
        assert capped.count == 0

    cfg = PSSAConfig(depth=2, d_vocab=20, d_latent=8, d_state=4, d_mem_key=4, mem_capacity=6)
    w = ModelWeights.init(cfg, 3, "baseline")
    w.populate_banks(4, 6)
    w.blocks[1].mem_values[4, 2] = np.inf
    before = [bits(b.mem_values).copy() for b in w.blocks]
    with pytest.raises(HipError, match="must be finite"):
        w.set_value_cap(0.01)
    for b, v in zip(w.blocks, before):
        np.testing.assert_array_equal(bits(b.mem_values), v)
        assert b.mem_value_cap == 0.0
