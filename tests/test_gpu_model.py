"""Model-level parity on the GPU: prefill_inference / forward_inference through
the C ABI against the CPU oracle on the same seeded weights and ids.

Gates: fp32 weights 1e-4 and bf16 weights 2e-2 max normwise relative error on
the last-token logits and on every lane's carry."""
import os

import numpy as np
import pytest

from conftest import GOLDEN, assert_parity, rel_err
from oracle import oracle as O
from pssa_amd import ModelWeights, PSSAConfig, PSSALayer, checkpoint
from pssa_amd._abi import HipError

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def oracle_prefill(w, ids, carry=None, threads=8, bf16=False):
    """The oracle's prefill; bf16 restates the device's bf16 mode (weights
    rounded by the caller, every product's activation operand rounded)."""
    om = O.OracleModel(w, bf16_operands=bf16)
    lanes = ids.shape[0]
    states = om.zero_state(lanes) if carry is None else carry.copy()
    logits = om.prefill_lanes(states, ids, threads=threads)
    return logits, states


def test_golden_fixture_model(hip):
    """The reference's depth-one fixture model (tests/golden/*_initial.pssa) with
    its populated bank, nonzero carry and adapter, run through the HIP path."""
    say("golden fixture model")
    ck = checkpoint.load(os.path.join(GOLDEN, "depth_one_main85d9d33_initial.pssa"))
    w = ck.weights
    layer = PSSALayer(hip, w, lanes=1, max_tokens=8)
    layer.set_carry(ck.carry[None])
    got = layer.prefill_inference([[1, 2, 1]])
    ref, st = oracle_prefill(w, np.array([[1, 2, 1]], np.uint32), ck.carry[None])
    assert_parity(got, ref, 1e-5, 'got')
    assert_parity(layer.get_carry(), st, 1e-5, 'layer.get_carry()')
    for tok in (4, 3, 2):
        g = layer.forward_inference([tok])
        r = O.OracleModel(w).forward_inference(st[0], tok)
        assert_parity(g[0], r, 1e-5, 'g[0]')
    layer.close()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_prefill_matches_oracle_small(hip, dtype):
    say("prefill small", dtype)
    cfg = PSSAConfig(depth=3, d_vocab=301, d_latent=64, d_state=24, d_mem_key=8, mem_capacity=40)
    w = ModelWeights.init(cfg, 7, "baseline")
    w.populate_banks(8, count=33)
    rng = np.random.default_rng(0)
    ids = rng.integers(0, cfg.d_vocab, (3, 37), dtype=np.uint32)
    layer = PSSALayer(hip, w, lanes=3, max_tokens=3 * 37, weight_dtype=dtype)
    got = layer.prefill_inference(ids)
    ref_w = w if dtype == "f32" else w.to_bf16_values()
    ref, st = oracle_prefill(ref_w, ids, bf16=dtype == "bf16")
    tol = 1e-4 if dtype == "f32" else 2e-2
    assert_parity(got, ref, tol, 'got')
    assert_parity(layer.get_carry(), st, tol, 'layer.get_carry()')
    layer.close()


@pytest.mark.parametrize("init", ["baseline", "reference"])
def test_config1_shape_fp32_and_bf16(hip, init):
    """Config 1 (d=128, s=64, depth 2, V=8192, 512-slot bank of dim 128),
    B=1, T=512, seed 0: the config's own initialisation (baseline: N(0, 0.02)
    matrices, stable rates) and the reference's, each with a populated bank."""
    cfg = PSSAConfig(depth=2, d_vocab=8192, d_latent=128, d_state=64, d_mem_key=128, mem_capacity=512)
    w = ModelWeights.init(cfg, 0, init)
    w.populate_banks(1)
    ids = np.random.default_rng(0).integers(0, cfg.d_vocab, (1, 512), dtype=np.uint32)
    ref, st = oracle_prefill(w, ids)
    ref_bf, st_bf = oracle_prefill(w.to_bf16_values(), ids, bf16=True)
    for dtype, r, s, tol in (("f32", ref, st, 1e-4), ("bf16", ref_bf, st_bf, 2e-2)):
        say("config1", init, dtype)
        layer = PSSALayer(hip, w, lanes=1, max_tokens=512, weight_dtype=dtype)
        got = layer.prefill_inference(ids)
        assert_parity(got, r, tol, 'got')
        assert_parity(layer.get_carry(), s, tol, 'layer.get_carry()')
        assert int(np.argmax(got[0, 1:])) == int(np.argmax(r[0, 1:]))
        layer.close()


def test_token_loop_equals_prefill_bitwise(hip):
    """forward_inference token by token reproduces prefill bit for bit
    (the reference's prefill/decode identity, src/inference.rs:1069-1113)."""
    say("token loop == prefill")
    cfg = PSSAConfig(depth=2, d_vocab=97, d_latent=48, d_state=32, d_mem_key=8, mem_capacity=24)
    w = ModelWeights.init(cfg, 3, "baseline")
    w.populate_banks(2, count=20)
    ids = np.random.default_rng(1).integers(0, cfg.d_vocab, (2, 19), dtype=np.uint32)
    a = PSSALayer(hip, w, lanes=2, max_tokens=64)
    b = PSSALayer(hip, w, lanes=2, max_tokens=64)
    la = a.prefill_inference(ids)
    for t in range(ids.shape[1]):
        lb = b.forward_inference(ids[:, t])
    np.testing.assert_array_equal(la, lb)
    np.testing.assert_array_equal(a.get_carry(), b.get_carry())
    # Split prefill continues the carry exactly.
    c = PSSALayer(hip, w, lanes=2, max_tokens=64)
    c.prefill_inference(ids[:, :7], want_logits=False)
    lc = c.prefill_inference(ids[:, 7:])
    np.testing.assert_array_equal(la, lc)
    for layer in (a, b, c):
        layer.close()


def test_scan_variants_keep_token_loop_identity(hip):
    """d_state=256 at d_latent=768: a 32-lane 5-token prefill runs the
    four-wave J=32 scan on one stream (12 x 32 x 2 = 768 workgroups), a
    16-lane 9-token prefill the eight-wave J=16 scan (384 workgroups, fewer
    than three waves per SIMD), a 32-lane 67-token prefill two concurrent lane
    groups with the four-wave scan, and single tokens the step kernel.  All
    of them sum the readout in one order, so the prefill/decode identity holds
    across them (src/inference.rs:1069-1113 checks lengths 1 .. 1024 without
    resets in between)."""
    say("scan variants token loop == prefill")
    cfg = PSSAConfig(depth=1, d_vocab=64, d_latent=768, d_state=256, d_mem_key=8, mem_capacity=16)
    w = ModelWeights.init(cfg, 7, "baseline")
    w.populate_banks(8, count=12)
    lanes = 32
    rng = np.random.default_rng(4)
    a = PSSALayer(hip, w, lanes=lanes, max_tokens=lanes * 67)
    b = PSSALayer(hip, w, lanes=lanes, max_tokens=lanes * 67)
    for n, T in ((32, 5), (16, 9), (32, 67), (32, 1)):
        ids = rng.integers(0, cfg.d_vocab, (n, T), dtype=np.uint32)
        la = a.prefill_inference(ids)
        for t in range(T):
            lb = b.forward_inference(ids[:, t])
        np.testing.assert_array_equal(la, lb)
        np.testing.assert_array_equal(a.get_carry(), b.get_carry())
    a.close()
    b.close()


@pytest.mark.parametrize("hybrid,capacity", [(False, 64), (True, 64), (False, 200), (True, 512)])
def test_bf16_token_loop_equals_prefill_with_fused_query(hip, hybrid, capacity):
    """bf16 weights at d_latent 256 and d_mem_key 32: a single-token step
    forms the memory query inside the soft read (no separate query product),
    a prefill runs the product as a GEMM; both give the same logits and
    carries bit for bit (src/inference.rs:1069-1113).  Five lanes leave the
    second four-query workgroup with three rows past the batch, which load
    a clamped row and are discarded; bank capacities 64, 200 and 512 take
    the soft read's 1, 4 and 8 slots per lane."""
    say("bf16 token loop == prefill, fused query", hybrid, capacity)
    cfg = PSSAConfig(depth=2, d_vocab=61, d_latent=256, d_state=32, d_mem_key=32, mem_capacity=capacity)
    w = ModelWeights.init(cfg, 11, "baseline")
    count = capacity * 3 // 4
    w.populate_banks(12, count=count)
    if hybrid:
        rng = np.random.default_rng(13)
        for b in w.blocks:
            b.mem_hybrid_gate[:count] = rng.uniform(0.05, 1.0, count).astype(np.float32)
            b.mem_hybrid_age[:count] = rng.integers(0, 60, count).astype(np.uint64)
        w.set_hybrid_read(True, 0.9)
    ids = np.random.default_rng(14).integers(0, cfg.d_vocab, (5, 9), dtype=np.uint32)
    a = PSSALayer(hip, w, lanes=5, max_tokens=5 * 9, weight_dtype="bf16")
    b = PSSALayer(hip, w, lanes=5, max_tokens=5 * 9, weight_dtype="bf16")
    la = a.prefill_inference(ids)
    for t in range(ids.shape[1]):
        lb = b.forward_inference(ids[:, t])
    np.testing.assert_array_equal(la, lb)
    np.testing.assert_array_equal(a.get_carry(), b.get_carry())
    a.close()
    b.close()


def test_shape_errors_fail_before_anything_runs(hip):
    say("prefill shape errors")
    cfg = PSSAConfig(depth=1, d_vocab=10, d_latent=16, d_state=4, d_mem_key=4, mem_capacity=4)
    w = ModelWeights.init(cfg, 1, "baseline")
    layer = PSSALayer(hip, w, lanes=1, max_tokens=8)
    layer.prefill_inference([[1, 2]])
    before = layer.get_carry()
    with pytest.raises(HipError, match="at least one token"):
        layer.prefill_inference(np.zeros((1, 0), np.uint32))
    with pytest.raises(HipError, match="max_tokens"):
        layer.prefill_inference(np.ones((1, 9), np.uint32))
    np.testing.assert_array_equal(layer.get_carry(), before)
    layer.reset_recurrent_state()
    assert not layer.get_carry().any()
    layer.close()


def prefix_fixture():
    cfg = PSSAConfig(depth=2, d_vocab=37, d_latent=16, d_state=8, d_mem_key=4, mem_capacity=8)
    w = ModelWeights.init(cfg, 23, "baseline")
    w.populate_banks(5, 6)
    return w


def test_prefill_cancellation_and_invalid_ids_keep_the_processed_prefix(hip):
    """src/inference.rs:1114-1160 on the device: a prefill cancelled at the
    check before token `stop` (asked before every token) or stopped by an
    invalid id at `stop` leaves the carry where a token loop over ids[:stop]
    leaves it, and produces no logits."""
    say("prefill cancellation / invalid-id prefix")
    w = prefix_fixture()
    ids = np.array([[t % 37 for t in range(67)]], np.uint32)
    for stop in (0, 1, 31, 32, 33, 66):
        ref = PSSALayer(hip, w, lanes=1, max_tokens=128)
        for t in ids[0, :stop]:
            ref.forward_inference([t])
        layer = PSSALayer(hip, w, lanes=1, max_tokens=128)
        checks = [0]

        def cancelled():
            checks[0] += 1
            return checks[0] - 1 == stop

        done, processed, lg = layer.prefill_cancellable(ids, cancelled, chunk=1)
        assert (done, processed, lg, checks[0]) == (False, stop, None, stop + 1)
        np.testing.assert_array_equal(layer.get_carry(), ref.get_carry())
        bad = ids.copy()
        bad[0, stop] = 37
        inv = PSSALayer(hip, w, lanes=1, max_tokens=128)
        with pytest.raises(HipError, match="prompt ID 37 outside model vocabulary"):
            inv.prefill_inference(bad)
        np.testing.assert_array_equal(inv.get_carry(), ref.get_carry())
        for x in (ref, layer, inv):
            x.close()


def test_invalid_ids_advance_each_lane_through_its_own_prefix(hip):
    """Lanes stop at their own first invalid id; the error names the first
    lane's; every lane equals its one-lane prefill of the valid prefix, bit
    for bit, and the oracle's lanes."""
    say("invalid-id prefixes over lanes")
    w = prefix_fixture()
    ids = np.array([[1, 2, 3, 4], [5, 37, 6, 7], [8, 9, 10, 40]], np.uint32)
    layer = PSSALayer(hip, w, lanes=3, max_tokens=16)
    with pytest.raises(HipError, match="prompt ID 37 outside model vocabulary"):
        layer.prefill_inference(ids)
    car = layer.get_carry()
    for lane, n in enumerate((4, 1, 3)):
        one = PSSALayer(hip, w, lanes=1, max_tokens=16)
        one.prefill_inference(ids[lane:lane + 1, :n])
        np.testing.assert_array_equal(car[lane], one.get_carry()[0])
        one.close()
    states = O.OracleModel(w).zero_state(3)
    with pytest.raises(ValueError):
        O.OracleModel(w).prefill_lanes(states, ids)
    assert_parity(car, states, 1e-4, 'car')
    layer.close()


def test_chunked_cancellable_prefill_equals_prefill(hip):
    say("chunked prefill == prefill")
    w = prefix_fixture()
    ids = np.random.default_rng(4).integers(0, 37, (2, 67), dtype=np.uint32)
    a = PSSALayer(hip, w, lanes=2, max_tokens=256)
    b = PSSALayer(hip, w, lanes=2, max_tokens=256)
    done, processed, lg = a.prefill_cancellable(ids, lambda: False, chunk=8)
    assert done and processed == 67
    np.testing.assert_array_equal(lg, b.prefill_inference(ids))
    np.testing.assert_array_equal(a.get_carry(), b.get_carry())
    a.close()
    b.close()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_config3_full_model_prefix_against_oracle(hip, dtype):
    """The 105M-scale model (d=768, s=256, 12 layers, V=16384, k=32, 512-slot
    banks) at its real per-layer shape: 32 lanes x 64 tokens on the GPU, which
    run as two concurrent lane groups of 16 (lanes 0-15 on the library's
    stream, 16-31 on the second); the first and last lane of each group are
    replayed by the oracle."""
    say("config3 prefix", dtype)
    cfg = PSSAConfig(depth=12, d_vocab=16384, d_latent=768, d_state=256, d_mem_key=32, mem_capacity=512)
    w = ModelWeights.init(cfg, 0, "baseline")
    w.populate_banks(1)
    ids = np.random.default_rng(2).integers(0, cfg.d_vocab, (32, 64), dtype=np.uint32)
    layer = PSSALayer(hip, w, lanes=32, max_tokens=32 * 64, weight_dtype=dtype)
    got = layer.prefill_inference(ids)
    carry = layer.get_carry()
    ref_w = w if dtype == "f32" else w.to_bf16_values()
    pick = [0, 15, 16, 31]
    ref, st = oracle_prefill(ref_w, ids[pick], threads=4, bf16=dtype == "bf16")
    tol = 1e-4 if dtype == "f32" else 2e-2
    for j, lane in enumerate(pick):
        assert_parity(got[lane], ref[j], tol, f"logits lane {lane}")
        assert_parity(carry[lane], st[j], tol, f"carry lane {lane}")
    layer.close()


def test_config3_full_length_properties(hip):
    """Full benchmark shape (32 x 1024, bf16): finite, deterministic, and a
    512 + 512 split prefill equals the single 1024-token prefill bit for bit."""
    say("config3 full length")
    cfg = PSSAConfig(depth=12, d_vocab=16384, d_latent=768, d_state=256, d_mem_key=32, mem_capacity=512)
    w = ModelWeights.init(cfg, 0, "baseline")
    w.populate_banks(1)
    ids = np.random.default_rng(3).integers(0, cfg.d_vocab, (32, 1024), dtype=np.uint32)
    layer = PSSALayer(hip, w, lanes=32, max_tokens=32 * 1024, weight_dtype="bf16")
    a = layer.prefill_inference(ids)
    ca = layer.get_carry()
    assert np.all(np.isfinite(a)) and np.all(np.isfinite(ca))
    layer.reset_recurrent_state()
    b = layer.prefill_inference(ids)
    np.testing.assert_array_equal(a, b)
    layer.reset_recurrent_state()
    layer.prefill_inference(ids[:, :512], want_logits=False)
    c = layer.prefill_inference(ids[:, 512:])
    np.testing.assert_array_equal(a, c)
    np.testing.assert_array_equal(layer.get_carry(), ca)
    layer.close()


def test_ragged_prefill_matches_oracle_and_single_lanes(hip):
    """Prompts of their own length per lane (the inference row's lens[B]):
    every lane's last logits and carry against the oracle's prefill of that
    lane alone, and bit for bit against the device's one-lane prefill; equal
    lengths reproduce the rectangular prefill bit for bit."""
    say("ragged prefill")
    cfg = PSSAConfig(depth=2, d_vocab=151, d_latent=48, d_state=24, d_mem_key=8, mem_capacity=30)
    w = ModelWeights.init(cfg, 17, "baseline")
    w.populate_banks(18, count=25)
    rng = np.random.default_rng(3)
    lens = [7, 1, 70, 7, 3]
    seqs = [rng.integers(0, cfg.d_vocab, n, dtype=np.uint32) for n in lens]
    carry0 = (rng.standard_normal((5, cfg.depth, 48 * 24)) * 0.1).astype(np.float32)
    layer = PSSALayer(hip, w, lanes=5, max_tokens=128)
    layer.set_carry(carry0)
    got = layer.prefill_ragged(seqs)
    car = layer.get_carry()
    om = O.OracleModel(w)
    for i, q in enumerate(seqs):
        st = carry0[i].copy()
        ref = om.prefill(st, q)
        assert_parity(got[i], ref, 1e-4, i)
        assert_parity(car[i], st, 1e-4, i)
        one = PSSALayer(hip, w, lanes=1, max_tokens=128)
        one.set_carry(carry0[i:i + 1])
        np.testing.assert_array_equal(one.prefill_inference(q[None])[0], got[i])
        np.testing.assert_array_equal(one.get_carry()[0], car[i])
        one.close()
    ids = rng.integers(0, cfg.d_vocab, (5, 9), dtype=np.uint32)
    layer.set_carry(carry0)
    a = layer.prefill_ragged(list(ids))
    layer.set_carry(carry0)
    np.testing.assert_array_equal(layer.prefill_inference(ids), a)
    for bad, msg in [([seqs[0], np.zeros(0, np.uint32)], "at least one token"),
                     ([np.zeros(129, np.uint32)], "max_tokens"),
                     ([np.array([1, 151], np.uint32)], "outside model vocabulary")]:
        with pytest.raises(HipError, match=msg):
            layer.prefill_ragged(bad)
    layer.close()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_memory_top_k_model_matches_oracle(hip, dtype):
    """set_memory_top_k on the model (src/pssa.rs:2215-2226): prefill and
    greedy decode read the top-k slots, against the oracle's model with the
    same top_k; with the hybrid read on too; toggling re-captures the decode
    graph."""
    say("model memory top-k", dtype)
    cfg = PSSAConfig(depth=2, d_vocab=97, d_latent=48, d_state=32, d_mem_key=8, mem_capacity=24)
    w = ModelWeights.init(cfg, 31, "baseline")
    w.populate_banks(32, count=20)
    ids = np.random.default_rng(2).integers(0, 97, (3, 11), dtype=np.uint32)
    tol = 1e-4 if dtype == "f32" else 2e-2
    for k, hybrid in ((3, False), (1, False), (4, True)):
        dev_w = ModelWeights.init(cfg, 31, "baseline")
        dev_w.populate_banks(32, count=20)
        dev_w.set_memory_top_k(k)
        ref_w = ModelWeights.init(cfg, 31, "baseline")
        ref_w.populate_banks(32, count=20)
        ref_w.set_memory_top_k(k)
        if hybrid:
            for m in (dev_w, ref_w):
                for b in m.blocks:
                    b.mem_hybrid_gate[:20] = np.linspace(0.1, 1.0, 20, dtype=np.float32)
                m.set_hybrid_read(True, 0.9)
        layer = PSSALayer(hip, dev_w, lanes=3, max_tokens=64, weight_dtype=dtype)
        got = layer.prefill_inference(ids)
        om = O.OracleModel(ref_w if dtype == "f32" else ref_w.to_bf16_values(), bf16_operands=dtype == "bf16")
        st = om.zero_state(3)
        ref = om.prefill_lanes(st, ids, threads=3)
        assert_parity(got, ref, tol, (k, hybrid))
        assert_parity(layer.get_carry(), st, tol, (k, hybrid))
        layer.close()
    # Graph decode across a top-k toggle equals eager decode.
    res = []
    for graph in (False, True):
        layer = PSSALayer(hip, w, lanes=3, max_tokens=64, weight_dtype=dtype)
        layer.prefill_inference(ids)
        a = layer.decode(3, graph=graph)
        layer.set_memory_top_k(2)
        b = layer.decode(3, first_ids=a[-1], graph=graph)
        layer.set_memory_top_k(None)
        c = layer.decode(3, first_ids=b[-1], graph=graph)
        res.append((a, b, c, layer.get_carry()))
        layer.close()
    for x, y in zip(*res):
        np.testing.assert_array_equal(x, y)


def test_reference_v6_fixture_model(hip):
    """The reference's V6 checkpoint (tests/fixtures/v6-word-pre-bpe.pssa,
    read through the V6 branch of the payload order, src/checkpoint.rs:
    1344-1418) with its stored carry: prefill then token steps on the
    device against the oracle."""
    say("v6 fixture model")
    ck = checkpoint.load(os.path.join(GOLDEN, "v6-word-pre-bpe.pssa"))
    assert ck.version == 6
    w = ck.weights
    V = w.cfg.d_vocab
    ids = np.array([[1, min(2, V - 1), 1, min(3, V - 1), 0]], np.uint32)
    layer = PSSALayer(hip, w, lanes=1, max_tokens=16)
    layer.set_carry(ck.carry[None])
    got = layer.prefill_inference(ids)
    ref, st = oracle_prefill(w, ids, ck.carry[None])
    assert_parity(got, ref, 1e-5, "v6 prefill logits")
    assert_parity(layer.get_carry(), st, 1e-5, "v6 carry")
    for tok in (min(4, V - 1), 1):
        g = layer.forward_inference([tok])
        r = O.OracleModel(w).forward_inference(st[0], tok)
        assert_parity(g[0], r, 1e-5, "v6 step logits")
    layer.close()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_reference_legacy_v5_fixture_model(hip, dtype):
    """The reference's legacy V5 checkpoint (tests/fixtures/legacy-v5-model.pssa,
    load_v5, src/checkpoint.rs:1444-1545: inference-only, 11 bank slots, raw
    rates from the stored physical A): a 3-lane prefill on the device against
    the oracle on the loaded weights (bf16: against the oracle's bf16-operand
    restatement on the rounded weights), then greedy decode ids."""
    say("legacy v5 fixture model", dtype)
    ck = checkpoint.load(os.path.join(GOLDEN, "legacy-v5-model.pssa"))
    assert ck.format == "LegacyV5InferenceOnly"
    w = ck.weights
    ids = np.random.default_rng(3).integers(0, w.cfg.d_vocab, (3, 40), dtype=np.uint32)
    layer = PSSALayer(hip, w, lanes=3, max_tokens=3 * 40, weight_dtype=dtype)
    got = layer.prefill_inference(ids)
    wr = w.to_bf16_values() if dtype == "bf16" else w
    om = O.OracleModel(wr, bf16_operands=dtype == "bf16")
    st = om.zero_state(3)
    ref = om.prefill_lanes(st, ids, threads=3)
    tol = 1e-4 if dtype == "f32" else 2e-2
    assert_parity(got, ref, tol, f"v5 {dtype} prefill logits")
    assert_parity(layer.get_carry(), st, tol, f"v5 {dtype} carries")
    if dtype == "f32":
        gen = layer.decode(4, graph=True)
        for i in range(3):
            s_i = st[i].copy()
            cur = O.greedy(ref[i])
            want = [cur]
            for _ in range(3):
                cur = O.greedy(om.forward_inference(s_i, cur))
                want.append(cur)
            np.testing.assert_array_equal(gen[:, i], want)
    layer.close()
