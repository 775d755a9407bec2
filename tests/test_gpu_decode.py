"""Greedy decode on the GPU through the C ABI against the CPU oracle.

Plain decode is the reference's forward_inference + sample() at temperature 0
(src/pssa.rs:2387-2391, src/inference.rs:123-127): generated ids must equal
the oracle's, logits and carries within 1e-4 (fp32 weights).  Plastic decode
adds the lane-ordered protected bank writes and Hebbian adapter updates
(oracle_decode); the bank counters, ages and written slots must match, the
fast weights within 1e-4.  Graph replay must equal eager stepping bit for bit.
"""
import numpy as np
import pytest

from conftest import assert_parity, elem_rel_err, rel_err
from oracle import oracle as O
from pssa_amd import ModelWeights, PSSAConfig, PSSALayer
from pssa_amd._abi import HipError

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def small_model(seed=5, full_banks=True, depth=2):
    cfg = PSSAConfig(depth=depth, d_vocab=97, d_latent=48, d_state=32, d_mem_key=8, mem_capacity=24)
    w = ModelWeights.init(cfg, seed, "baseline")
    w.populate_banks(seed + 1, count=cfg.mem_capacity if full_banks else 10)
    return w


def prefill_both(w, lanes, T, seed=0):
    ids = np.random.default_rng(seed).integers(0, w.cfg.d_vocab, (lanes, T), dtype=np.uint32)
    om = O.OracleModel(w)
    st = om.zero_state(lanes)
    lg = om.prefill_lanes(st, ids, threads=lanes)
    return ids, st, lg


def test_decode_matches_oracle_forward_loop(hip):
    say("decode plain vs oracle")
    w = small_model()
    ids, st, lg = prefill_both(w, 3, 9)
    layer = PSSALayer(hip, w, lanes=3, max_tokens=64)
    layer.prefill_inference(ids)
    first = [O.greedy(lg[i]) for i in range(3)]
    # Continuing the prefill: row 0 is the choice from its logits, then one
    # forward step per further row (src/inference.rs:367-379).
    got, glog = layer.decode(7, want_logits=True)
    ref_w = ModelWeights.init(w.cfg, 5, "baseline")
    ref_w.populate_banks(6, count=w.cfg.mem_capacity)
    ref_ids, ref_lg, _ = O.OracleModel(ref_w).decode(st, first, steps=6)
    np.testing.assert_array_equal(got[0], first)
    np.testing.assert_array_equal(got[1:], ref_ids)
    assert_parity(glog, ref_lg, 1e-4, 'glog')
    assert_parity(layer.get_carry(), st, 1e-4, 'layer.get_carry()')
    layer.close()


def test_decode_graph_replay_equals_eager(hip):
    """Two lane sets from the same state: eager steps vs a captured step
    replayed, with eager work on the same stream between the replays."""
    say("decode graph == eager")
    w = small_model(seed=8)
    ids = np.random.default_rng(3).integers(0, w.cfg.d_vocab, (4, 7), dtype=np.uint32)
    res = []
    for graph in (False, True):
        layer = PSSALayer(hip, w, lanes=4, max_tokens=64)
        layer.prefill_inference(ids)
        a = layer.decode(3, graph=graph)
        layer.get_carry()  # eager traffic between replays
        b, lg = layer.decode(5, first_ids=a[-1], graph=graph, want_logits=True)
        res.append((a, b, lg, layer.get_carry()))
        layer.close()
    for x, y in zip(*res):
        np.testing.assert_array_equal(x, y)


@pytest.mark.parametrize("graph", [False, True])
def test_plastic_decode_matches_oracle(hip, graph):
    say("plastic decode vs oracle, graph", graph)
    lanes, steps = 3, 4
    w = small_model(seed=11)
    for b in w.blocks:
        b.adapter_up[:] = (np.random.default_rng(2).standard_normal(b.adapter_up.shape) * 0.05).astype(np.float32)
    ids, st, lg = prefill_both(w, lanes, 6, seed=4)
    layer = PSSALayer(hip, w, lanes=lanes, max_tokens=64)
    layer.prefill_inference(ids)
    first = [O.greedy(lg[i]) for i in range(lanes)]
    got, glog = layer.decode(steps, first_ids=first, plastic=True, graph=graph, want_logits=True)
    ref = ModelWeights.init(w.cfg, 11, "baseline")
    ref.populate_banks(12, count=w.cfg.mem_capacity)
    for b, b0 in zip(ref.blocks, w.blocks):
        b.adapter_up[:] = b0.adapter_up
    ref_ids, ref_lg, ref_sp = O.OracleModel(ref).decode(st, first, steps=steps, plastic=True)
    np.testing.assert_array_equal(got, ref_ids)
    assert_parity(glog, ref_lg, 1e-4, 'glog')
    assert np.all(ref_sp > 3.5)  # every lane writes (small random model: flat logits)
    for l in range(w.cfg.depth):
        dev = layer.get_plastic(l)
        rb = ref.blocks[l]
        assert dev["mem_count"] == rb.mem_count and dev["mem_write_head"] == rb.mem_write_head
        np.testing.assert_array_equal(dev["mem_last_seen"], rb.mem_last_seen)
        assert dev["step"] == steps
        np.testing.assert_allclose(dev["mem_confidence"], rb.mem_confidence, rtol=1e-5, atol=1e-6)
        assert_parity(dev["mem_keys"], rb.mem_keys, 1e-4, 'dev["mem_keys"]')
        assert_parity(dev["mem_values"], rb.mem_values, 1e-4, 'dev["mem_values"]')
        assert_parity(dev["mem_norm_sq"], rb.mem_norm_sq, 1e-4, 'dev["mem_norm_sq"]')
        assert_parity(dev["adapter_up"], rb.adapter_up, 1e-4, 'dev["adapter_up"]')
        assert not np.array_equal(dev["adapter_up"], w.blocks[l].adapter_up)
    layer.close()


def test_plastic_decode_fills_free_slots_first(hip):
    """A bank with free slots takes plain inserts at `count` before any
    protected overwrite (insert_protected, src/memory.rs:318-322)."""
    say("plastic decode free slots")
    w = small_model(seed=13, full_banks=False, depth=1)
    layer = PSSALayer(hip, w, lanes=2, max_tokens=16)
    layer.prefill_inference([[1, 2, 3], [4, 5, 6]])
    layer.decode(4, plastic=True)  # the choice from the prefill logits, then three steps
    dev = layer.get_plastic(0)
    assert dev["mem_count"] == 10 + 6 and dev["mem_write_head"] == 0
    assert set(dev["mem_last_seen"][10:16].tolist()) == {1, 2, 3}
    assert np.all(dev["mem_confidence"][10:16] == 1.0)
    assert np.all(dev["mem_norm_sq"][10:16] < 1.0)
    layer.close()


def test_decode_rejects_bad_arguments(hip):
    say("decode validation")
    w = small_model(seed=1, depth=1)
    layer = PSSALayer(hip, w, lanes=2, max_tokens=16)
    with pytest.raises(HipError, match="outside model vocabulary"):
        layer.decode(2, first_ids=[1, 97])
    with pytest.raises(HipError, match="n_lanes"):
        layer.decode(2, first_ids=[1, 2, 3])
    with pytest.raises(HipError, match="last prefill"):
        layer.decode(2, n_lanes=1)
    # Only a prefill's logits can be continued without first ids: not those of
    # a decode (its last token is unconsumed), nor any after a reset or a
    # carry change.
    layer.prefill_inference([[1, 2], [3, 4]])
    out = layer.decode(2)
    with pytest.raises(HipError, match="last prefill"):
        layer.decode(2, n_lanes=2)
    layer.decode(2, first_ids=out[-1])
    layer.prefill_inference([[1, 2], [3, 4]])
    layer.reset_recurrent_state()
    with pytest.raises(HipError, match="last prefill"):
        layer.decode(2, n_lanes=2)
    layer.prefill_inference([[1, 2], [3, 4]])
    layer.set_carry(layer.get_carry())
    with pytest.raises(HipError, match="last prefill"):
        layer.decode(2, n_lanes=2)
    layer.close()


def test_decode_at_105m_width_graph_equals_eager(hip):
    """The config-5 model width (d=768, s=256, k=32, C=512, V=16384, bf16) on
    8 lanes x 2 layers: plastic graph replay equals plastic eager steps."""
    say("decode 105M width")
    cfg = PSSAConfig(depth=2, d_vocab=16384, d_latent=768, d_state=256, d_mem_key=32, mem_capacity=512)
    w = ModelWeights.init(cfg, 0, "baseline")
    w.populate_banks(1)
    ids = np.random.default_rng(9).integers(0, cfg.d_vocab, (8, 16), dtype=np.uint32)
    outs = []
    for graph in (False, True):
        layer = PSSALayer(hip, w, lanes=8, max_tokens=128, weight_dtype="bf16")
        layer.prefill_inference(ids)
        g, lg = layer.decode(4, plastic=True, graph=graph, want_logits=True)
        outs.append((g, lg, layer.get_carry(), layer.get_plastic(1)["adapter_up"]))
        layer.close()
    for x, y in zip(*outs):
        np.testing.assert_array_equal(x, y)
    assert np.all(np.isfinite(outs[0][1]))


@pytest.mark.parametrize("hybrid", [False, True])
def test_lane_group_steps_eager_equal_graph_replay(hip, hybrid):
    """Steps of 96 lanes run as lane groups on their own streams, eagerly or
    as parallel branches of the captured step: at the config-5 width (bf16)
    and with the plastic writes, both give the same ids, logits, carries,
    taps-driven bank rows and Hebbian weights bit for bit (a lane's rows are
    computed the same way in any group; the plastic writes follow the
    join)."""
    say("eager lane groups == graph", hybrid)
    cfg = PSSAConfig(depth=2, d_vocab=4096, d_latent=768, d_state=256, d_mem_key=32, mem_capacity=512)
    w = ModelWeights.init(cfg, 5, "baseline")
    w.populate_banks(6, count=400)
    if hybrid:
        rng = np.random.default_rng(8)
        for b in w.blocks:
            b.mem_hybrid_gate[:400] = rng.uniform(0.05, 1.0, 400).astype(np.float32)
            b.mem_hybrid_age[:400] = rng.integers(0, 60, 400).astype(np.uint64)
        w.set_hybrid_read(True, 0.9)
    lanes = 96
    ids = np.random.default_rng(7).integers(0, cfg.d_vocab, (lanes, 8), dtype=np.uint32)
    outs = []
    for graph in (False, True):
        layer = PSSALayer(hip, w, lanes=lanes, max_tokens=lanes * 8, weight_dtype="bf16")
        layer.prefill_inference(ids)
        g, lg = layer.decode(5, plastic=True, graph=graph, want_logits=True)
        pl = [layer.get_plastic(l) for l in range(cfg.depth)]
        outs.append((g, lg, layer.get_carry(), *[p["adapter_up"] for p in pl], *[p["mem_values"] for p in pl],
                     *[p["mem_last_seen"] for p in pl]))
        layer.close()
    for x, y in zip(*outs):
        np.testing.assert_array_equal(x, y)
    assert np.all(np.isfinite(outs[0][1]))


def test_plastic_decode_many_lanes_and_layers_matches_oracle(hip):
    """64 lanes x 12 blocks: the per-(block, lane) Hebbian rates and the
    per-block bank writes of one launch cover every block."""
    say("plastic decode 64 lanes x 12 layers")
    cfg = PSSAConfig(depth=12, d_vocab=61, d_latent=16, d_state=8, d_mem_key=4, mem_capacity=24)
    w = ModelWeights.init(cfg, 21, "baseline")
    w.populate_banks(22, count=24)
    ref = ModelWeights.init(cfg, 21, "baseline")
    ref.populate_banks(22, count=24)
    lanes = 64
    ids = np.random.default_rng(6).integers(0, cfg.d_vocab, (lanes, 3), dtype=np.uint32)
    om = O.OracleModel(ref)
    st = om.zero_state(lanes)
    lg = om.prefill_lanes(st, ids, threads=8)
    first = [O.greedy(lg[i]) for i in range(lanes)]
    layer = PSSALayer(hip, w, lanes=lanes, max_tokens=lanes * 3)
    layer.prefill_inference(ids)
    got = layer.decode(3, plastic=True, graph=True)
    ref_ids, _, _ = om.decode(st, first, steps=2, plastic=True, threads=8)
    np.testing.assert_array_equal(got[0], first)
    np.testing.assert_array_equal(got[1:], ref_ids)
    for l in (0, 5, 11):
        dev = layer.get_plastic(l)
        rb = ref.blocks[l]
        np.testing.assert_array_equal(dev["mem_last_seen"], rb.mem_last_seen)
        assert dev["mem_write_head"] == rb.mem_write_head
        assert_parity(dev["adapter_up"], rb.adapter_up, 1e-4, 'dev["adapter_up"]')
    layer.close()


def oracle_penalised_decode(w, ids, steps, penalty):
    """The reference's generate loop at temperature 0 with max_new_tokens =
    steps (src/inference.rs:345-391): the first token from the prefill
    logits, then forward + sample per further token, the window being the
    prompt and every token chosen so far.  Returns every generated token."""
    om = O.OracleModel(w)
    out = np.zeros((steps, ids.shape[0]), np.uint32)
    for i, prompt in enumerate(ids):
        st = om.zero_state()
        hist = [int(t) for t in prompt]
        cur = O.sample_greedy(om.prefill(st, prompt), hist, penalty)
        out[0, i] = cur
        for s in range(1, steps):
            hist.append(cur)
            cur = O.sample_greedy(om.forward_inference(st, cur), hist, penalty)
            out[s, i] = cur
    return out


@pytest.mark.parametrize("graph", [False, True])
def test_decode_repetition_penalty_matches_oracle_sample(hip, graph):
    """Greedy decode with the reference's default repetition penalty 1.25
    against the oracle's sample() over the same windows; the penalty changes
    the ids here, so the test is not the plain argmax again."""
    say("decode repetition penalty, graph", graph)
    w = small_model(seed=23)
    ids = np.random.default_rng(7).integers(1, w.cfg.d_vocab, (3, 9), dtype=np.uint32)
    steps = 12
    layer = PSSALayer(hip, w, lanes=3, max_tokens=64)
    layer.set_repetition_penalty(1.25)
    layer.prefill_inference(ids)
    got = layer.decode(steps, graph=graph)
    ref = oracle_penalised_decode(w, ids, steps, 1.25)
    np.testing.assert_array_equal(got, ref)
    assert not np.array_equal(ref, oracle_penalised_decode(w, ids, steps, 1.0))
    # A reset empties the window: the same prompt gives the same ids again.
    layer.reset_recurrent_state()
    layer.prefill_inference(ids)
    np.testing.assert_array_equal(layer.decode(steps, graph=graph), ref)
    layer.set_repetition_penalty(1.0)
    layer.reset_recurrent_state()
    layer.prefill_inference(ids)
    np.testing.assert_array_equal(layer.decode(steps, graph=graph), oracle_penalised_decode(w, ids, steps, 1.0))
    layer.close()


def test_repetition_penalty_validation_and_non_finite_logits(hip):
    say("decode penalty validation / non-finite logits")
    w = small_model(seed=2, depth=1)
    layer = PSSALayer(hip, w, lanes=2, max_tokens=16)
    for bad in (0.5, float("nan"), float("inf")):
        with pytest.raises(HipError, match="finite and >= 1"):
            layer.set_repetition_penalty(bad)
    layer.close()
    w.unembed[5] = np.nan
    layer = PSSALayer(hip, w, lanes=2, max_tokens=16)
    layer.prefill_inference([[1, 2], [3, 4]])
    with pytest.raises(HipError, match="non-finite logits"):
        layer.decode(2)
    layer.close()


def test_value_cap_on_device_matches_host_clamp_and_oracle_decode(hip):
    """set_value_cap (src/memory.rs:121-170) on a loaded model equals the host
    clamp bit for bit, a recorded cap clamps on load, the next prefill reads
    the capped bank, and plastic bank writes store capped values as the
    oracle's capped inserts do."""
    say("value cap")
    cap = 0.35
    w = small_model(seed=29)
    host = small_model(seed=29)
    host.set_value_cap(cap)
    layer = PSSALayer(hip, w, lanes=3, max_tokens=64)
    layer.set_value_cap(cap)
    for l in range(w.cfg.depth):
        np.testing.assert_array_equal(layer.get_plastic(l)["mem_values"], host.blocks[l].mem_values)
    recorded = small_model(seed=29)
    for b in recorded.blocks:
        b.mem_value_cap = cap
    loaded = PSSALayer(hip, recorded, lanes=3, max_tokens=64)
    for l in range(w.cfg.depth):
        np.testing.assert_array_equal(loaded.get_plastic(l)["mem_values"], host.blocks[l].mem_values)
    loaded.close()
    ids = np.random.default_rng(5).integers(0, w.cfg.d_vocab, (3, 8), dtype=np.uint32)
    lg = layer.prefill_inference(ids)
    om = O.OracleModel(host)
    st = om.zero_state(3)
    ref_lg = om.prefill_lanes(st, ids, threads=3)
    assert_parity(lg, ref_lg, 1e-4, 'lg')
    layer.close()
    # Plastic writes on banks that give way (confidence 0) store capped values.
    dev_w, ref_w = small_model(seed=29), small_model(seed=29)
    for m in (dev_w, ref_w):
        for b in m.blocks:
            b.mem_confidence[:] = 0.0
        m.set_value_cap(cap)
    layer = PSSALayer(hip, dev_w, lanes=3, max_tokens=64)
    layer.prefill_inference(ids)
    om = O.OracleModel(ref_w)
    st = om.zero_state(3)
    lg = om.prefill_lanes(st, ids, threads=3)
    first = [O.greedy(lg[i]) for i in range(3)]
    got = layer.decode(3, first_ids=first, plastic=True)
    ref_ids, _, _ = om.decode(st, first, steps=3, plastic=True)
    np.testing.assert_array_equal(got, ref_ids)
    for l in range(dev_w.cfg.depth):
        vals = layer.get_plastic(l)["mem_values"]
        assert_parity(vals, ref_w.blocks[l].mem_values, 1e-4, 'vals')
        assert np.all((vals.astype(np.float64) ** 2).sum(axis=1) <= float(np.float32(cap)) ** 2)
        assert not np.array_equal(vals, host.blocks[l].mem_values)  # the decode wrote slots
    layer.close()


def sync_oracle_to_device(ref, layer, cfg):
    """Copies the device's plastic block state (fast weights, banks) into
    the oracle's weights."""
    for l in range(cfg.depth):
        dev = layer.get_plastic(l)
        b = ref.blocks[l]
        b.adapter_up[:] = dev["adapter_up"]
        b.mem_keys[:] = dev["mem_keys"]
        b.mem_values[:] = dev["mem_values"]
        b.mem_norm_sq[:] = dev["mem_norm_sq"]
        b.mem_confidence[:] = dev["mem_confidence"]
        b.mem_last_seen[:] = dev["mem_last_seen"]
        b.mem_count = dev["mem_count"]
        b.mem_write_head = dev["mem_write_head"]


def lane_block_err(got, want, floor):
    """Element-wise relative error |got - want| / max(|want|, floor) per
    (lane, block) of carries [lanes, depth, d*s]."""
    w64 = want.astype(np.float64)
    return (np.abs(got.astype(np.float64) - w64) / np.maximum(np.abs(w64), floor)).max(axis=2)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_config5_width_and_depth_plastic_decode_matches_oracle(hip, dtype):
    """Config 5 as the benchmark runs it: 256 streams x 12 blocks at d=768,
    s=256, k=32, C=512, V=16384, a 512-token prefill per stream, the first
    token from the prefill's logits and 127 free-running plastic graph steps
    (128 generated ids), then three more plastic graph steps, each against
    the oracle taking the same step from the same state: before each step
    the oracle is given the device's carries, banks and fast weights, and
    both consume the same tokens.  fp32 weights meet the reference's
    arithmetic (its AVX2 dot tree) at 1e-4; bf16 weights meet the oracle's
    restatement of the bf16 mode (same rounded weights, every product's
    activation operand rounded) at 2e-2.
    Why per step: the random 105M model amplifies rounding differences
    through the recurrence over time, and with bf16 operands any fp32-level
    difference flips some roundings by one bf16 ulp, so a free-running
    comparison would measure the model's conditioning rather than the step.
    fp32: carries, written bank rows (keys and values), confidences and
    fast weights are gated element-wise at 1e-4 (assert_parity).  Each step
    also runs the reference's other dot tree (portable instead of AVX2) from
    the same state and reports how far the reference moves from itself: the
    device's per-(lane, block) error is set beside that spread.  (After an
    8-token prompt a few lanes amplify any rounding difference from block to
    block; there the reference's two trees differ by up to 2e-4 of an
    element's size, lane 6 block 9, and the device by 4.5e-4.  At this
    512-token state the spread is about 2e-5 and the device within 3.5e-5.)
    bf16: carries and written bank rows are gated normwise (a flipped bf16
    rounding moves an element by a few percent of its size) and their
    element-wise errors are reported.
    A chosen id may differ from the oracle's only where its two logits lie
    within the gate.  The 256-way lane-ordered protected writes into each
    block's shared bank (insert_protected, src/memory.rs:305-342) must make
    the oracle's decisions: count, write head and last-seen steps equal;
    confidences, keys, values and fast weights within the gate."""
    say("config 5 width/depth plastic decode", dtype)
    cfg = PSSAConfig(depth=12, d_vocab=16384, d_latent=768, d_state=256, d_mem_key=32, mem_capacity=512)
    w = ModelWeights.init(cfg, 0, "baseline")
    w.populate_banks(1)
    bf16 = dtype == "bf16"
    ref = w.to_bf16_values() if bf16 else ModelWeights.init(cfg, 0, "baseline")
    if not bf16:
        ref.populate_banks(1)
    ref_p = None if bf16 else ModelWeights.init(cfg, 0, "baseline")  # the portable-tree twin
    tol = 2e-2 if bf16 else 1e-4
    S, P, free, steps = 256, 512, 128, 3
    ids = np.random.default_rng(31).integers(0, cfg.d_vocab, (S, P), dtype=np.uint32)
    layer = PSSALayer(hip, w, lanes=S, max_tokens=S * P, weight_dtype=dtype)
    layer.stage_ids(ids)
    layer.prefill_staged()
    gen = layer.decode(free, n_lanes=S, plastic=True, graph=True)
    assert gen.shape == (free, S) and int(gen.max()) < cfg.d_vocab
    say(f"{S} x {P}-token prefill and {free} free-running steps done")
    cur = gen[-1].copy()
    ties = 0
    for t in range(steps):
        st = layer.get_carry()
        step0 = layer.get_plastic(0)["step"]
        sync_oracle_to_device(ref, layer, cfg)
        if not bf16:
            sync_oracle_to_device(ref_p, layer, cfg)
        om = O.OracleModel(ref, bf16_operands=bf16)
        got, glog = layer.decode(1, first_ids=cur, plastic=True, graph=True, want_logits=True)
        st_p = None if bf16 else st.copy()
        with O.Dot(True):
            want, r_lg, _ = om.decode(st, cur, steps=1, plastic=True, step_base=step0, threads=16)
        for i in np.nonzero(got[0] != want[0])[0]:
            gap = abs(float(r_lg[i, got[0, i]]) - float(r_lg[i, want[0, i]]))
            assert gap <= tol * float(np.max(np.abs(r_lg[i]))), (t, i, got[0, i], want[0, i], gap)
            ties += 1
        assert_parity(glog, r_lg, tol, f"step {t} logits")
        car = layer.get_carry()
        rms = float(np.sqrt(np.mean(st.astype(np.float64) ** 2)))
        nw = rel_err(car, st)
        ew = lane_block_err(car, st, rms)
        say(f"step {t} carries: normwise {nw:.3e}, element-wise {ew.max():.3e} (lane {np.unravel_index(ew.argmax(), ew.shape)})")
        assert nw < tol
        if not bf16:
            # The same step under the reference's portable dot tree, from the
            # same state (the device's carries, banks and fast weights).
            om_p = O.OracleModel(ref_p)
            with O.Dot(False):
                om_p.decode(st_p, cur, steps=1, plastic=True, step_base=step0, threads=16)
            spread = lane_block_err(st_p, st, rms)
            worst = np.unravel_index(np.argmax(ew), ew.shape)
            say(f"step {t} fp32 carries: reference tree spread max {spread.max():.3e}; device worst (lane, block) "
                f"{worst}: {ew[worst]:.3e}, the reference's spread there {spread[worst]:.3e}")
            assert_parity(car, st, tol, f"step {t} carries")
        else:
            say(f"step {t} bf16 carries: element-wise {elem_rel_err(car, st):.3e} (normwise gate)")
        for l in range(cfg.depth):
            dev = layer.get_plastic(l)
            rb = ref.blocks[l]
            assert dev["step"] == step0 + 1
            assert dev["mem_count"] == rb.mem_count and dev["mem_write_head"] == rb.mem_write_head, (t, l)
            np.testing.assert_array_equal(dev["mem_last_seen"], rb.mem_last_seen)
            assert_parity(dev["mem_confidence"], rb.mem_confidence, tol, f"confidence {t} {l}")
            # Written rows are a lane's projected query and z_final: state
            # vectors like the carries (element-wise at fp32, normwise at bf16).
            if bf16:
                assert rel_err(dev["mem_keys"], rb.mem_keys) < tol, (t, l)
                assert rel_err(dev["mem_values"], rb.mem_values) < tol, (t, l)
                say(f"step {t} block {l} bf16 written rows: element-wise keys "
                    f"{elem_rel_err(dev['mem_keys'], rb.mem_keys):.3e}, values "
                    f"{elem_rel_err(dev['mem_values'], rb.mem_values):.3e}")
            else:
                assert_parity(dev["mem_keys"], rb.mem_keys, tol, f"keys {t} {l}")
                assert_parity(dev["mem_values"], rb.mem_values, tol, f"values {t} {l}")
            assert_parity(dev["adapter_up"], rb.adapter_up, tol, f"adapter_up {t} {l}")
        cur = want[0].copy()
    say("near-tie choices", ties, "of", S * steps)
    assert ties <= S * steps // 20
    layer.close()


def oracle_sampled_decode(w, ids, steps, penalty, temperature, top_p, top_k, seed=1337):
    """The reference's generate loop (src/inference.rs:345-391) with sample()
    at a temperature: one SimpleRng per lane (the engine's, seeded with
    `seed`), the first token from the prefill logits, then forward + sample."""
    om = O.OracleModel(w)
    out = np.zeros((steps, ids.shape[0]), np.uint32)
    for i, prompt in enumerate(ids):
        st = om.zero_state()
        rng = O.Rng(seed)
        hist = [int(t) for t in prompt]
        cur = O.sample(om.prefill(st, prompt), hist, rng, temperature, top_p, top_k, penalty)
        out[0, i] = cur
        for s in range(1, steps):
            hist.append(cur)
            cur = O.sample(om.forward_inference(st, cur), hist, rng, temperature, top_p, top_k, penalty)
            out[s, i] = cur
    return out


@pytest.mark.parametrize("graph", [False, True])
def test_decode_sampling_matches_oracle_sample(hip, graph):
    """Decode at the reference's default InferenceConfig (temperature 0.7,
    top-p 0.85, top-k 24, repetition penalty 1.25) against the oracle's
    sample() with the same generators: the same ids, a different sequence from
    the greedy one, and the generators carry on across decode calls."""
    say("decode sampling, graph", graph)
    w = small_model(seed=31)
    ids = np.random.default_rng(11).integers(1, w.cfg.d_vocab, (3, 9), dtype=np.uint32)
    steps = 12
    ref = oracle_sampled_decode(w, ids, steps, 1.25, 0.7, 0.85, 24)
    assert not np.array_equal(ref, oracle_penalised_decode(w, ids, steps, 1.25))
    layer = PSSALayer(hip, w, lanes=3, max_tokens=64)
    layer.set_repetition_penalty(1.25)
    layer.set_sampling(0.7, 0.85, 24, seed=1337)
    layer.prefill_inference(ids)
    np.testing.assert_array_equal(layer.decode(steps, graph=graph), ref)
    # Continuing: the generators were not reset, so a second prompt pass
    # after a reset draws the oracle's next values.
    layer.set_sampling(0.7, 0.85, 24, seed=1337)
    layer.reset_recurrent_state()
    layer.prefill_inference(ids)
    first = layer.decode(5, graph=graph)
    rest = layer.decode(steps - 5, first_ids=first[-1], graph=graph)
    np.testing.assert_array_equal(np.concatenate([first, rest]), ref)
    # Temperature 0 is the greedy choice again and draws nothing.
    layer.set_sampling(0.0)
    layer.reset_recurrent_state()
    layer.prefill_inference(ids)
    np.testing.assert_array_equal(layer.decode(steps, graph=graph), oracle_penalised_decode(w, ids, steps, 1.25))
    layer.close()


@pytest.mark.parametrize("vocab,penalty", [(3000, 1.0), (40000, 1.25)])
def test_decode_sampling_wide_vocabulary_and_top_k(hip, vocab, penalty):
    """Wide vocabularies (several passes of the workgroup per row; 40000 ids
    also take the global scratch row instead of LDS), top-k 64 and top-p 1
    (every kept candidate drawn from), seed 0 (the generator's fixed non-zero
    start), with and without the penalty window."""
    say("decode sampling, wide vocabulary", vocab, penalty)
    cfg = PSSAConfig(depth=1, d_vocab=vocab, d_latent=64, d_state=32, d_mem_key=8, mem_capacity=16)
    w = ModelWeights.init(cfg, 3, "baseline")
    w.populate_banks(4, count=cfg.mem_capacity)
    ids = np.random.default_rng(2).integers(1, cfg.d_vocab, (2, 5), dtype=np.uint32)
    ref = oracle_sampled_decode(w, ids, 10, penalty, 1.3, 1.0, 64, seed=0)
    layer = PSSALayer(hip, w, lanes=2, max_tokens=16)
    layer.set_repetition_penalty(penalty)
    layer.set_sampling(1.3, 1.0, 64, seed=0)
    layer.prefill_inference(ids)
    np.testing.assert_array_equal(layer.decode(10), ref)
    layer.close()


def test_sampling_validation(hip):
    say("decode sampling validation")
    w = small_model(seed=2, depth=1)
    layer = PSSALayer(hip, w, lanes=2, max_tokens=16)
    for t in (-0.1, float("nan"), float("inf")):
        with pytest.raises(HipError, match="temperature must be finite"):
            layer.set_sampling(t)
    for p in (0.0, 1.5, float("nan")):
        with pytest.raises(HipError, match="top-p must be finite"):
            layer.set_sampling(0.7, p)
    with pytest.raises(HipError, match="top-k must be positive"):
        layer.set_sampling(0.7, 0.85, 0)
    with pytest.raises(HipError, match="top-k up to 64"):
        layer.set_sampling(0.7, 0.85, 65)
    layer.set_sampling(0.0, 0.85, 1000)  # greedy: any top-k
    layer.close()
