"""The hybrid read (retrieve_hybrid_into, src/memory.rs:568-660) and gated
bank writes on the GPU, through the C ABI, against the CPU oracle.

Gates: retrieved slot indices and minimum distances bit-exact; weights and
readouts within 1e-5 normwise; model logits within 1e-4 (fp32 weights);
hybrid ages and write gates equal to the oracle's exactly; graph replay
equal to eager stepping bit for bit.
"""
import numpy as np
import pytest

from conftest import assert_parity, rel_err
from oracle import oracle as O
from pssa_amd import ModelWeights, PSSAConfig, PSSALayer
from pssa_amd._abi import HipError
from test_oracle_closed_forms import bank

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def ball(rng, n, d, rmax=0.8):
    v = rng.standard_normal((n, d))
    return (v / np.linalg.norm(v, axis=1, keepdims=True) * rng.uniform(0, rmax, (n, 1))).astype(np.float32)


@pytest.mark.parametrize("n_q,C,count,dk,dv,k", [(1, 4, 3, 2, 3, 0), (37, 64, 64, 8, 16, 0),
                                                 (300, 512, 512, 32, 48, 8), (130, 512, 300, 768, 64, 8),
                                                 (65, 100, 77, 7, 5, 3)])
def test_retrieve_hybrid_matches_oracle(hip, n_q, C, count, dk, dv, k):
    """Gates in [0, 1] with some exactly zero, ages up to 2^64-1 (lam^age
    underflows to 0 in f32 as in the reference), lam 0.97."""
    say("retrieve hybrid", n_q, C, count, dk, dv, k)
    rng = np.random.default_rng(C * 7 + dk)
    keys, vals, q = ball(rng, count, dk), ball(rng, count, dv), ball(rng, n_q, dk)
    q[0] = keys[count - 1]
    K, N, V, cnt = bank(C, keys, vals)
    gate = rng.uniform(0.0, 1.0, count).astype(np.float32)
    gate[::5] = 0.0
    age = rng.integers(0, 400, count).astype(np.uint64)
    age[1::7] = np.uint64(2**64 - 1)
    out, mn, idx, w = hip.retrieve_hybrid(q, K, N, V, cnt, 0.2, gate, age, 0.97, top_k=k, want_weights=True)
    r_out, r_min, r_idx, r_w = O.retrieve_hybrid_batch(K, N, V, cnt, q, 0.2, gate, age, 0.97, k, threads=8)
    if k:
        np.testing.assert_array_equal(idx, r_idx)
    np.testing.assert_array_equal(mn.view(np.uint32), r_min.view(np.uint32))
    assert rel_err(w, r_w) < 1e-5
    assert rel_err(out, r_out) < 1e-5
    assert not w[:, count:].any()


def test_retrieve_hybrid_neutral_and_fully_gated(hip):
    """Gates 1 and lam 1 read exactly like the soft read (src/memory.rs:893-929);
    a bank whose every live weight is gated to 0 falls back to the soft read
    (src/memory.rs:970-985).  The plain top-k read takes the ranked kernels,
    which sum the readout in another order: there indices and minima are
    bit-exact and the rest within 1e-6."""
    say("retrieve hybrid neutral / fully gated")
    rng = np.random.default_rng(21)
    C, dk, dv, n_q = 48, 16, 24, 40
    keys, vals, q = ball(rng, C, dk), ball(rng, C, dv), ball(rng, n_q, dk)
    K, N, V, cnt = bank(C, keys, vals)
    for k in (0, 8):
        soft = hip.retrieve(q, K, N, V, cnt, 0.3, top_k=k, want_weights=True)
        neutral = hip.retrieve_hybrid(q, K, N, V, cnt, 0.3, np.ones(C, np.float32), np.arange(C, dtype=np.uint64),
                                      1.0, top_k=k, want_weights=True)
        gated = hip.retrieve_hybrid(q, K, N, V, cnt, 0.3, np.zeros(C, np.float32), np.zeros(C, np.uint64), 0.5,
                                    top_k=k, want_weights=True)
        for h in (neutral, gated):
            for i, (a, b) in enumerate(zip(h, soft)):
                if a is None:
                    continue
                if k == 0 or i in (1, 2):
                    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
                else:
                    assert rel_err(a, b) < 1e-6


def test_retrieve_hybrid_rejects_bad_arguments(hip):
    say("retrieve hybrid validation")
    K, N, V, cnt = bank(4, [[0.1], [0.2]], [[1.0], [2.0]])
    q = np.float32([[0.0]])
    with pytest.raises(HipError, match="nonnegative"):
        hip.retrieve_hybrid(q, K, N, V, cnt, 0.5, [1.0, -0.5], [0, 0], 0.9)
    with pytest.raises(HipError, match="lam"):
        hip.retrieve_hybrid(q, K, N, V, cnt, 0.5, [1.0, 1.0], [0, 0], 1.5)


def hybrid_model(seed, lam, depth=2, full_banks=True, confidence=None):
    cfg = PSSAConfig(depth=depth, d_vocab=97, d_latent=48, d_state=32, d_mem_key=8, mem_capacity=24)
    w = ModelWeights.init(cfg, seed, "baseline")
    count = cfg.mem_capacity if full_banks else 10
    w.populate_banks(seed + 1, count=count)
    rng = np.random.default_rng(seed + 2)
    for b in w.blocks:
        b.mem_hybrid_gate[:count] = rng.uniform(0.05, 1.0, count).astype(np.float32)
        b.mem_hybrid_gate[::6] = 0.0
        b.mem_hybrid_age[:count] = rng.integers(0, 60, count).astype(np.uint64)
        if confidence is not None:  # confidence 0: a full bank gives way to every write
            b.mem_confidence[:count] = confidence
    w.set_hybrid_read(True, lam)
    return w


def test_hybrid_prefill_matches_oracle_lanes(hip):
    """A hybrid prefill of 3 lanes x 11 tokens: logits and carries against the
    oracle's lockstep lanes, the ages 11 higher on both; the device's token
    loop equals its prefill bit for bit, and the hybrid read changes the
    logits against the plain one."""
    say("hybrid prefill vs oracle")
    lanes, T = 3, 11
    ids = np.random.default_rng(6).integers(0, 97, (lanes, T), dtype=np.uint32)
    w, ref = hybrid_model(31, 0.9), hybrid_model(31, 0.9)
    om = O.OracleModel(ref)
    st = om.zero_state(lanes)
    r_lg = om.prefill_lanes(st, ids, threads=lanes)
    layer = PSSALayer(hip, w, lanes=lanes, max_tokens=64)
    lg = layer.prefill_inference(ids)
    assert_parity(lg, r_lg, 1e-4, 'lg')
    assert_parity(layer.get_carry(), st, 1e-4, 'layer.get_carry()')
    for l in range(w.cfg.depth):
        gate, age = layer.get_hybrid(l)
        np.testing.assert_array_equal(gate, ref.blocks[l].mem_hybrid_gate)
        np.testing.assert_array_equal(age, ref.blocks[l].mem_hybrid_age)
        np.testing.assert_array_equal(age, w.blocks[l].mem_hybrid_age + T)
    layer.close()
    loop = PSSALayer(hip, w, lanes=lanes, max_tokens=64)
    for t in range(T):
        step = loop.forward_inference(ids[:, t])
    np.testing.assert_array_equal(step, lg)
    for l in range(w.cfg.depth):
        np.testing.assert_array_equal(loop.get_hybrid(l)[1], ref.blocks[l].mem_hybrid_age)
    loop.set_hybrid_read(False, 1.0)
    loop.reset_recurrent_state()
    plain = loop.prefill_inference(ids)
    assert not np.array_equal(plain, lg)
    loop.close()


@pytest.mark.parametrize("graph", [False, True])
def test_hybrid_plastic_decode_matches_oracle(hip, graph):
    """Plastic decode on hybrid blocks: every write is a gated protected insert
    whose gate is the lane's mean memory-injection gate, and it resets the
    slot's age; ids, bank counters, gates and ages equal the oracle's."""
    say("hybrid plastic decode vs oracle, graph", graph)
    lanes, steps = 3, 4
    w, ref = hybrid_model(41, 0.95, confidence=0.0), hybrid_model(41, 0.95, confidence=0.0)
    ids = np.random.default_rng(4).integers(0, 97, (lanes, 6), dtype=np.uint32)
    om = O.OracleModel(ref)
    st = om.zero_state(lanes)
    lg = om.prefill_lanes(st, ids, threads=lanes)
    layer = PSSALayer(hip, w, lanes=lanes, max_tokens=64)
    layer.prefill_inference(ids)
    first = [O.greedy(lg[i]) for i in range(lanes)]
    got, glog = layer.decode(steps, first_ids=first, plastic=True, graph=graph, want_logits=True)
    ref_ids, ref_lg, ref_sp = om.decode(st, first, steps=steps, plastic=True)
    np.testing.assert_array_equal(got, ref_ids)
    assert_parity(glog, ref_lg, 1e-4, 'glog')
    for l in range(w.cfg.depth):
        dev = layer.get_plastic(l)
        rb = ref.blocks[l]
        assert dev["mem_count"] == rb.mem_count and dev["mem_write_head"] == rb.mem_write_head
        np.testing.assert_array_equal(dev["mem_last_seen"], rb.mem_last_seen)
        np.testing.assert_allclose(dev["mem_confidence"], rb.mem_confidence, rtol=1e-5, atol=1e-6)
        assert_parity(dev["mem_values"], rb.mem_values, 1e-4, 'dev["mem_values"]')
        assert_parity(dev["mem_keys"], rb.mem_keys, 1e-4, 'dev["mem_keys"]')
        gate, age = layer.get_hybrid(l)
        np.testing.assert_array_equal(age, rb.mem_hybrid_age)
        np.testing.assert_allclose(gate, rb.mem_hybrid_gate, rtol=1e-5, atol=1e-7)
        # A defended slot is only re-stamped; a written one restarts its age.
        written = np.any(dev["mem_values"] != w.blocks[l].mem_values, axis=1)
        assert written.any()
        assert np.all(age[written] < steps) and np.all((gate[written] >= 0) & (gate[written] <= 1))
    layer.close()


def test_hybrid_decode_free_slots_take_gated_inserts(hip):
    """Free slots take gated inserts at `count` (insert_gated_protected,
    src/memory.rs:520-556): gate = the lane's mean injection gate in [0, 1]."""
    say("hybrid decode free slots")
    w, ref = hybrid_model(13, 0.9, depth=1, full_banks=False), hybrid_model(13, 0.9, depth=1, full_banks=False)
    ids = np.array([[1, 2, 3], [4, 5, 6]], np.uint32)
    layer = PSSALayer(hip, w, lanes=2, max_tokens=16)
    layer.prefill_inference(ids)
    layer.decode(4, plastic=True)  # the choice from the prefill logits, then three steps
    om = O.OracleModel(ref)
    st = om.zero_state(2)
    lg = om.prefill_lanes(st, ids, threads=2)
    om.decode(st, [O.greedy(lg[i]) for i in range(2)], steps=3, plastic=True)
    gate, age = layer.get_hybrid(0)
    assert layer.get_plastic(0)["mem_count"] == 16
    assert np.all((gate[10:16] >= 0.0) & (gate[10:16] <= 1.0))
    np.testing.assert_allclose(gate, ref.blocks[0].mem_hybrid_gate, rtol=1e-5, atol=1e-7)
    np.testing.assert_array_equal(age, ref.blocks[0].mem_hybrid_age)
    layer.close()


def test_hybrid_toggle_recaptures_decode_graph(hip):
    """set_hybrid_read between graph decodes must not replay a graph captured
    for the other read: graph and eager runs agree across the toggle."""
    say("hybrid toggle graph")
    res = []
    ids = np.random.default_rng(8).integers(0, 97, (2, 5), dtype=np.uint32)
    for graph in (False, True):
        w = hybrid_model(51, 0.9)
        layer = PSSALayer(hip, w, lanes=2, max_tokens=32)
        layer.prefill_inference(ids)
        a, la = layer.decode(3, graph=graph, want_logits=True)
        layer.set_hybrid_read(False, 1.0)
        b, lb = layer.decode(3, first_ids=a[-1], graph=graph, want_logits=True)
        layer.set_hybrid_read(True, 0.8)
        c, lc = layer.decode(3, first_ids=b[-1], graph=graph, want_logits=True)
        res.append((a, la, b, lb, c, lc, layer.get_hybrid(0)[1]))
        layer.close()
    for x, y in zip(*res):
        np.testing.assert_array_equal(x, y)
