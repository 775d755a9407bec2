"""Recurrent depth loops (set_loops, src/pssa.rs:2171-2184; the looped
forward_inference_features, src/pssa.rs:2338-2373) on the GPU against the
oracle's looped model (pinned by composition from its single-loop path,
tests/test_oracle_loops.py).  Gates: 1e-4 fp32, 2e-2 bf16 weights."""
import numpy as np
import pytest

from conftest import assert_parity
from oracle import oracle as O
from pssa_amd import ModelWeights, PSSAConfig, PSSALayer
from pssa_amd._abi import HipError

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def model(depth=2, seed=3, d_vocab=97):
    cfg = PSSAConfig(depth=depth, d_vocab=d_vocab, d_latent=48, d_state=32, d_mem_key=8, mem_capacity=24)
    w = ModelWeights.init(cfg, seed, "baseline")
    w.populate_banks(seed + 1, count=20)
    return w


@pytest.mark.parametrize("lanes,T,loops,dtype", [(3, 12, 3, "f32"), (4, 70, 2, "f32"), (4, 70, 2, "bf16")])
def test_looped_prefill_matches_oracle(hip, lanes, T, loops, dtype):
    """Logits of the last token and every (block, loop) carry; 4 x 70 runs as
    two lane groups on two streams."""
    say("looped prefill", lanes, T, loops, dtype)
    w = model()
    ids = np.random.default_rng(5).integers(1, w.cfg.d_vocab, (lanes, T), dtype=np.uint32)
    wr = w.to_bf16_values() if dtype == "bf16" else w
    om = O.OracleModel(wr, bf16_operands=dtype == "bf16")
    om.set_loops(loops)
    st = om.zero_state(lanes)
    ref = om.prefill_lanes(st, ids, threads=lanes)
    layer = PSSALayer(hip, w, lanes=lanes, max_tokens=lanes * T, weight_dtype=dtype)
    layer.set_loops(loops)
    got = layer.prefill_inference(ids)
    tol = 1e-4 if dtype == "f32" else 2e-2
    assert_parity(got, ref, tol, "logits")
    assert layer.get_carry().shape == st.shape
    assert_parity(layer.get_carry(), st, tol, "carries")
    layer.close()


def test_looped_token_loop_equals_prefill_and_decode_matches_oracle(hip):
    say("looped token loop / decode")
    w = model(depth=3, seed=8)
    ids = np.random.default_rng(9).integers(1, w.cfg.d_vocab, (2, 11), dtype=np.uint32)
    a = PSSALayer(hip, w, lanes=2, max_tokens=64)
    b = PSSALayer(hip, w, lanes=2, max_tokens=64)
    a.set_loops(2)
    b.set_loops(2)
    la = a.prefill_inference(ids)
    for t in range(ids.shape[1]):
        lb = b.forward_inference(ids[:, t])
    np.testing.assert_array_equal(la, lb)
    np.testing.assert_array_equal(a.get_carry(), b.get_carry())
    # Greedy decode (graph) against the oracle's token loop.
    steps = 6
    got = a.decode(steps, graph=True)
    om = O.OracleModel(w)
    om.set_loops(2)
    for i, prompt in enumerate(ids):
        st = om.zero_state()
        cur = O.greedy(om.prefill(st, prompt))
        want = [cur]
        for _ in range(steps - 1):
            cur = O.greedy(om.forward_inference(st, cur))
            want.append(cur)
        np.testing.assert_array_equal(got[:, i], want)
    a.close()
    b.close()


def test_set_loops_keeps_loop_zero_and_validates(hip):
    say("set_loops carries / validation")
    w = model(seed=4)
    ids = np.random.default_rng(2).integers(1, w.cfg.d_vocab, (2, 9), dtype=np.uint32)
    layer = PSSALayer(hip, w, lanes=2, max_tokens=64)
    layer.prefill_inference(ids[:, :5], want_logits=False)
    c1 = layer.get_carry()
    layer.set_loops(3)
    c3 = layer.get_carry()
    np.testing.assert_array_equal(c3[:, :, 0], c1)
    assert not c3[:, :, 1:].any()
    # Continuing from there equals the oracle continuing from the same state.
    om = O.OracleModel(w)
    om.set_loops(3)
    st = c3.copy()
    ref = om.prefill_lanes(st, ids[:, 5:], threads=2)
    assert_parity(layer.prefill_inference(ids[:, 5:]), ref, 1e-4, "continued logits")
    layer.reset_recurrent_state()
    assert not layer.get_carry().any()
    for bad in (0, 33):
        with pytest.raises(HipError, match="between 1 and 32"):
            layer.set_loops(bad)
    with pytest.raises(HipError, match="one loop here"):
        layer.decode(2, first_ids=[1, 2], plastic=True)
    layer.set_loops(1)
    assert layer.get_carry().shape == (2, w.cfg.depth, w.cfg.d_latent * w.cfg.d_state)
    layer.close()


def test_loops_with_hybrid_read_refused_before_any_kernel(hip):
    """Loops and the hybrid read are not combined here: set_loops refuses while
    the hybrid read is on, and a decode over looped lanes whose model turned
    it on afterwards is refused before the choice kernel runs, so no lane's
    generator advances and the prefill's logits are still there to continue
    from (the sampled ids equal a fresh layer's)."""
    say("loops x hybrid read refusal")
    w = model(seed=6)
    ids = np.random.default_rng(4).integers(1, w.cfg.d_vocab, (2, 7), dtype=np.uint32)

    def fresh():
        layer = PSSALayer(hip, w, lanes=2, max_tokens=64)
        layer.set_sampling(0.8, 0.9, 8, 77)
        return layer

    a = fresh()
    a.set_hybrid_read(True, 0.9)
    with pytest.raises(HipError, match="one loop here"):
        a.set_loops(2)
    a.set_hybrid_read(False, 1.0)
    a.set_loops(2)
    a.prefill_inference(ids, want_logits=False)
    a.set_hybrid_read(True, 0.9)
    with pytest.raises(HipError, match="one loop here"):
        a.decode(4, graph=True)
    a.set_hybrid_read(False, 1.0)
    got = a.decode(4, graph=True)
    b = fresh()
    b.set_loops(2)
    b.prefill_inference(ids, want_logits=False)
    want = b.decode(4, graph=True)
    np.testing.assert_array_equal(got, want)
    a.close()
    b.close()
