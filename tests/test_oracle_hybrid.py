"""Hybrid read and gated writes in the oracle (src/memory.rs:488-665), pinned by
the reference's own tests (src/memory.rs:893-1010, src/pssa.rs:4185-4230) and
by a float64 closed form of the weight rule."""
import numpy as np
import pytest

from oracle import oracle as O
from pssa_amd import ModelWeights, PSSAConfig


def _lcg_unit(seed):
    """The reference test's generator: seed*6364136223846793005 + 1442695040888963407,
    x = (seed >> 11) / 2^53 * 2 - 1 (src/memory.rs:896-901)."""
    seed = (seed * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
    return seed, np.float32(((seed >> 11) / float(1 << 53)) * 2.0 - 1.0)


def _ball(seed, n):
    v = []
    for _ in range(n):
        seed, x = _lcg_unit(seed)
        v.append(x)
    v = np.float32(v)
    norm = np.float32(np.sqrt(np.float32(sum(np.float32(x * x) for x in v))))
    return seed, np.float32(0.5) * v / norm


def test_hybrid_read_at_neutral_settings_matches_soft_read_bitwise():
    """src/memory.rs:893-929."""
    bank = O.Bank(8, 4, 3)
    seed = 7
    for i in range(5):
        seed, k = _ball(seed, 4)
        bank.insert(k, [i, 2 * i, 3 * i])
        bank.bump_hybrid_ages()
    _, q = _ball(seed, 4)
    sv, sw, smin = bank.retrieve_soft(q, 0.7)
    hv, hw, hmin = bank.retrieve_hybrid(q, 0.7, 1.0)
    np.testing.assert_array_equal(sv.view(np.uint32), hv.view(np.uint32))
    np.testing.assert_array_equal(sw[:bank.count].view(np.uint32), hw[:bank.count].view(np.uint32))
    assert smin.view(np.uint32) == hmin.view(np.uint32)
    assert np.all(bank.age[:5] == np.arange(5, 0, -1))


def test_hybrid_read_resolves_rebinding_by_recency():
    """src/memory.rs:930-955."""
    bank = O.Bank(4, 2, 2)
    k = [0.5, 0.0]
    bank.insert(k, [1.0, 0.0])
    bank.bump_hybrid_ages(5000)
    bank.insert(k, [0.0, 1.0])
    bank.bump_hybrid_ages(5000)
    val, _, _ = bank.retrieve_hybrid(k, 0.5, 0.999)
    assert val[1] > 0.99 and val[0] < 0.01, val
    val, _, _ = bank.retrieve_hybrid(k, 0.5, 1.0)
    assert 0.45 < val[0] < 0.55, val


def test_hybrid_gate_zero_slots_drop_out_of_the_read():
    """src/memory.rs:957-968."""
    bank = O.Bank(4, 2, 2)
    bank.insert_gated([0.5, 0.0], [1.0, 0.0], 0.0)
    bank.insert_gated([0.0, 0.5], [0.0, 1.0], 1.0)
    val, w, _ = bank.retrieve_hybrid([0.5, 0.0], 0.5, 0.999)
    assert val[1] > 0.999, val
    assert w[0] == 0.0


def test_fully_gated_read_falls_back_to_unweighted_softmax():
    """src/memory.rs:970-985: every live weight gated to zero -> the soft read."""
    bank = O.Bank(4, 2, 2)
    bank.insert_gated([0.5, 0.0], [1.0, 0.0], 0.0)
    bank.insert_gated([0.0, 0.5], [0.0, 1.0], 0.0)
    val, _, _ = bank.retrieve_hybrid([0.5, 0.0], 0.5, 1.0)
    soft, _, _ = bank.retrieve_soft([0.5, 0.0], 0.5)
    assert val[0] > 0.9 and abs(val[0] - soft[0]) < 1e-6


def test_hybrid_metadata_resets_on_ring_overwrite_and_bad_gates_are_rejected():
    """src/memory.rs:1000-1027 (the reference panics on a negative gate; the
    oracle refuses the write)."""
    bank = O.Bank(2, 2, 2)
    bank.insert_gated([0.5, 0.0], [1.0, 0.0], 0.25)
    bank.insert([0.0, 0.5], [0.0, 1.0])
    bank.bump_hybrid_ages(3)
    bank.insert_gated([0.5, 0.0], [1.0, 1.0], 0.75)
    assert bank.gate[0] == np.float32(0.75) and bank.age[0] == 0
    assert bank.gate[1] == 1.0 and bank.age[1] == 3
    assert bank.insert_gated([0.5, 0.0], [1.0, 0.0], -0.1) == -1
    assert bank.insert_gated([0.5, 0.0], [1.0, 0.0], float("nan")) == -1


def test_gated_protected_write_follows_the_refractory_gate():
    """insert_gated_protected (src/memory.rs:520-556): with free slots it is a
    gated insert stamped with the step; on a full bank a defended write changes
    neither the slot nor its hybrid metadata."""
    bank = O.Bank(2, 2, 2)
    assert bank.insert_gated_protected([0.5, 0.0], [1.0, 0.0], 0.3, 9.0, 10) == 0
    assert bank.last_seen[0] == 10 and bank.gate[0] == np.float32(0.3)
    assert bank.insert_gated_protected([0.0, 0.5], [0.0, 1.0], 0.6, 9.0, 11) == 1
    bank.bump_hybrid_ages(2)
    # Full: the write head (slot 0) was seen one step ago -> gain 0.005, damage tiny.
    assert bank.insert_gated_protected([0.2, 0.2], [5.0, 5.0], 0.9, 4.0, 11) == -1
    assert bank.gate[0] == np.float32(0.3) and bank.age[0] == 2
    np.testing.assert_array_equal(bank.values[0], [1.0, 0.0])


@pytest.mark.parametrize("top_k", [0, 3])
def test_hybrid_weights_match_float64_closed_form(top_k):
    """w_i = exp((min - d_i)/tau) * g_i * lam^age_i over the live slots, renormalised."""
    rng = np.random.default_rng(3)
    C, dk, dv, n = 12, 5, 4, 6
    keys = rng.standard_normal((C, dk)).astype(np.float32)
    keys *= (rng.uniform(0, 0.8, (C, 1)) / np.linalg.norm(keys, axis=1, keepdims=True)).astype(np.float32)
    nsq = np.array([O.squared_norm(k) for k in keys], np.float32)
    vals = rng.standard_normal((C, dv)).astype(np.float32)
    q = rng.standard_normal((n, dk)).astype(np.float32)
    q *= (0.5 / np.linalg.norm(q, axis=1, keepdims=True)).astype(np.float32)
    gate = rng.uniform(0.0, 1.0, C).astype(np.float32)
    age = rng.integers(0, 40, C).astype(np.uint64)
    lam, tau = 0.93, 0.3
    out, mn, idx, w = O.retrieve_hybrid_batch(keys, nsq, vals, C, q, tau, gate, age, lam, top_k)
    for i in range(n):
        d = np.array([O.poincare_distance(q[i], k) for k in keys], np.float64)
        live = np.ones(C, bool)
        if top_k:
            order = sorted(range(C), key=lambda s: (np.float32(d[s]).view(np.uint32), s))[:top_k]
            live[:] = False
            live[order] = True
            assert sorted(order) == list(idx[i])
        e = np.where(live, np.exp((d.min() - d) / tau) * gate * lam ** age.astype(np.float64), 0.0)
        ref = e / e.sum()
        np.testing.assert_allclose(w[i], ref, rtol=2e-5, atol=1e-7)
        np.testing.assert_allclose(out[i], ref @ vals, rtol=1e-4, atol=1e-6)
        assert mn[i] == np.float32(d.min())


def _hybrid_model(lam):
    cfg = PSSAConfig(depth=2, d_vocab=40, d_latent=16, d_state=4, d_mem_key=4, mem_capacity=10)
    w = ModelWeights.init(cfg, 8, "baseline")
    w.populate_banks(5, 8)
    rng = np.random.default_rng(1)
    for b in w.blocks:
        b.mem_hybrid_gate[:8] = rng.uniform(0.1, 1.0, 8).astype(np.float32)
        b.mem_hybrid_age[:8] = rng.integers(0, 20, 8).astype(np.uint64)
    w.set_hybrid_read(True, lam)
    return w


def test_hybrid_forward_at_neutral_settings_matches_standard():
    """src/pssa.rs:4185-4196: gates 1 and lam 1 give the standard forward bit for bit."""
    cfg = PSSAConfig(depth=2, d_vocab=40, d_latent=16, d_state=4, d_mem_key=4, mem_capacity=10)
    a, b = (ModelWeights.init(cfg, 8, "baseline") for _ in range(2))
    for m in (a, b):
        m.populate_banks(5, 8)
    a.set_hybrid_read(True, 1.0)
    oa, ob = O.OracleModel(a), O.OracleModel(b)
    sa, sb = oa.zero_state(), ob.zero_state()
    la, lb = oa.prefill(sa, [3, 9, 1, 30]), ob.prefill(sb, [3, 9, 1, 30])
    np.testing.assert_array_equal(la, lb)
    np.testing.assert_array_equal(sa, sb)
    assert np.all(a.blocks[0].mem_hybrid_age[:8] == 4) and np.all(b.blocks[0].mem_hybrid_age == 0)


def test_hybrid_prefill_equals_token_loop_and_lanes_advance_together():
    """forward_inference bumps then reads (src/pssa.rs:1153-1162); a prefill of T
    tokens equals T single steps and leaves the ages T higher; lanes advance
    together (each lane of a T-token prefill reads with the same ages)."""
    w1, w2, w3 = (_hybrid_model(0.9) for _ in range(3))
    o1, o2, o3 = (O.OracleModel(w) for w in (w1, w2, w3))
    ids = [4, 17, 2, 2, 33]
    s1, s2 = o1.zero_state(), o2.zero_state()
    l1 = o1.prefill(s1, ids)
    for t in ids[:-1]:
        o2.forward_inference(s2, t, logits=False)
    l2 = o2.forward_inference(s2, ids[-1])
    np.testing.assert_array_equal(l1, l2)
    np.testing.assert_array_equal(s1, s2)
    for b1, b2 in zip(w1.blocks, w2.blocks):
        np.testing.assert_array_equal(b1.mem_hybrid_age, b2.mem_hybrid_age)
    states = o3.zero_state(2)
    lanes = o3.prefill_lanes(states, np.array([ids, ids], np.uint32), threads=2)
    np.testing.assert_array_equal(lanes[0], l1)
    np.testing.assert_array_equal(lanes[1], l1)
    for b1, b3 in zip(w1.blocks, w3.blocks):
        np.testing.assert_array_equal(b1.mem_hybrid_age, b3.mem_hybrid_age)
    # Recency decay changes the read: the same prompt without the hybrid read differs.
    w4 = _hybrid_model(0.9)
    w4.set_hybrid_read(False, 1.0)
    o4 = O.OracleModel(w4)
    assert not np.array_equal(o4.prefill(o4.zero_state(), ids), l1)


def test_set_hybrid_read_validates_lam():
    """src/pssa.rs:4168-4179."""
    w = _hybrid_model(0.5)
    for bad in (0.0, 1.2, float("nan")):
        with pytest.raises(ValueError):
            w.set_hybrid_read(True, bad)
    w.set_hybrid_read(False, 1.0)
    assert not w.blocks[0].mem_hybrid_enabled


def test_memory_top_k_at_or_above_count_is_the_full_read():
    """retrieve_soft_into reads every slot when top_k >= count
    (self.top_k.filter(|&k| k < self.count), src/memory.rs:380); a smaller
    top_k changes the forward."""
    cfg = PSSAConfig(depth=2, d_vocab=40, d_latent=16, d_state=4, d_mem_key=4, mem_capacity=10)
    full, topk, small = (ModelWeights.init(cfg, 8, "baseline") for _ in range(3))
    for m in (full, topk, small):
        m.populate_banks(5, 8)
    topk.set_memory_top_k(8)
    small.set_memory_top_k(2)
    ids = [3, 9, 1, 30, 7]
    outs = []
    for m in (full, topk, small):
        om = O.OracleModel(m)
        outs.append(om.prefill(om.zero_state(), ids))
    np.testing.assert_array_equal(outs[0], outs[1])
    assert not np.array_equal(outs[0], outs[2])
    with pytest.raises(ValueError):
        small.set_memory_top_k(0)
