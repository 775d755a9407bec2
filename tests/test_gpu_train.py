"""Batch training forward (SequenceBatch::forward, src/sequence_batch.rs:233-384)
on the GPU through the C ABI, against the reference's golden words and the
CPU oracle's forward_train_chunk (src/pssa.rs:2597-2752).

Gates: fp32 weights 1e-4 and bf16 weights 2e-2 max normwise relative error on
logits, per-token losses and carries; the loss of the reference's depth-one
fixture chunk within 1e-5 of the reference's own recorded words.
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN, assert_parity, rel_err
from oracle import oracle as O
from pssa_amd import ModelWeights, PSSAConfig, PSSALayer, Sequence, checkpoint
from pssa_amd._abi import HipError

pytestmark = pytest.mark.gpu

AVX2_OBSERVED = os.path.join(GOLDEN, "depth_one_main014f617_avx2_observed.bin")


def say(*a):
    print("[case]", *a, flush=True)


def oracle_batch(w, carries, seqs, bf16=False):
    """Per-sequence forward_train_chunk on each lane's carry (forward_stacked,
    src/sequence_batch.rs:560-609): token losses and logits in packed order,
    the token-mean loss, and the carries after the batch (bf16: the device's
    bf16 operand rounding restated, weights rounded by the caller)."""
    om = O.OracleModel(w, bf16_operands=bf16)
    carries = carries.copy()
    losses, logits = [], []
    for s in seqs:
        if s.reset:
            carries[s.lane] = 0.0
        _, lg = om.train_chunk_forward(carries[s.lane], s.inputs, s.targets)
        lg64 = lg.astype(np.float64)
        mx = lg64.max(axis=1)
        lse = mx + np.log(np.exp(lg64 - mx[:, None]).sum(axis=1))
        losses.append(lse - lg64[np.arange(len(s.targets)), np.asarray(s.targets)])
        logits.append(lg)
    tl = np.concatenate(losses)
    return tl.mean(), tl, np.concatenate(logits), carries


def test_fixture_chunks_match_reference_golden_words(hip):
    """Words 0..22 of the reference's depth-one run (tests/support/
    depth_one_reference.rs:47-55): chunk [1,2,1] -> [2,1,3] (loss, 3x7
    scaled logits), then chunk [4] -> [5] from the continued carry."""
    say("train forward golden words")
    ck = checkpoint.load(os.path.join(GOLDEN, "depth_one_main85d9d33_initial.pssa"))
    words = np.fromfile(AVX2_OBSERVED, dtype="<u4")[:23].view(np.float32)
    layer = PSSALayer(hip, ck.weights, lanes=1, max_tokens=8)
    layer.set_carry(ck.carry[None])
    loss, lg = layer.batch_forward([Sequence(0, [1, 2, 1], [2, 1, 3])], want_logits=True)
    assert abs(loss - words[0]) <= 1e-5 * abs(words[0])
    assert_parity(lg.ravel(), words[1:22], 1e-5, 'lg.ravel()')
    loss2 = layer.batch_forward([(0, [4], [5])])
    assert abs(loss2 - words[22]) <= 1e-5 * abs(words[22])
    layer.close()


def small(depth=2, seed=3, V=211):
    cfg = PSSAConfig(depth=depth, d_vocab=V, d_latent=48, d_state=24, d_mem_key=8, mem_capacity=30)
    w = ModelWeights.init(cfg, seed, "baseline")
    w.populate_banks(seed + 1, count=27)
    return w


def random_seqs(rng, V, spec):
    return [Sequence(lane, rng.integers(0, V, n, dtype=np.uint32), rng.integers(0, V, n, dtype=np.uint32), reset)
            for lane, n, reset in spec]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_ragged_batch_matches_oracle(hip, dtype):
    """Ragged sequences on permuted lanes with one reset and one lane left
    out; then a second batch continues the carries."""
    say("train forward ragged", dtype)
    w = small()
    V = w.cfg.d_vocab
    rng = np.random.default_rng(11)
    lanes = 5
    carry0 = (rng.standard_normal((lanes, w.cfg.depth, 48 * 24)) * 0.1).astype(np.float32)
    layer = PSSALayer(hip, w, lanes=lanes, max_tokens=64, weight_dtype=dtype)
    layer.set_carry(carry0)
    ref_w = w if dtype == "f32" else w.to_bf16_values()
    tol = 1e-4 if dtype == "f32" else 2e-2
    carries = carry0
    for spec in ([(3, 7, False), (0, 12, True), (4, 1, False), (1, 7, False)],
                 [(0, 5, False), (2, 9, False)]):
        seqs = random_seqs(rng, V, spec)
        loss, tl, lg = layer.batch_forward(seqs, want_token_losses=True, want_logits=True)
        r_loss, r_tl, r_lg, carries = oracle_batch(ref_w, carries, seqs, bf16=dtype == "bf16")
        assert_parity(lg, r_lg, tol, 'lg')
        assert_parity(tl, r_tl, tol, 'tl')
        assert abs(loss - r_loss) <= tol * abs(r_loss)
        np.testing.assert_allclose(loss, np.float32(sum(np.float32(x) for x in tl) / np.float32(tl.size)), rtol=1e-6)
        got = layer.get_carry()
        assert_parity(got, carries, tol, 'got')
    layer.close()


def test_lane_groups_and_permuted_lanes_match_oracle(hip):
    """Sequences long enough for the concurrent lane-group schedule (T >= 64),
    on lanes given out of order, against the oracle; the carries equal those
    of prefill_inference over the same ids bit for bit."""
    say("train forward lane groups")
    w = small(depth=2, seed=9)
    V = w.cfg.d_vocab
    rng = np.random.default_rng(5)
    T = 70
    seqs = random_seqs(rng, V, [(2, T, False), (0, T, False), (3, T, False), (1, T, False)])
    layer = PSSALayer(hip, w, lanes=4, max_tokens=4 * T)
    loss, tl, lg = layer.batch_forward(seqs, want_token_losses=True, want_logits=True)
    r_loss, r_tl, r_lg, r_car = oracle_batch(w, np.zeros((4, 2, 48 * 24), np.float32), seqs)
    assert_parity(lg, r_lg, 1e-4, 'logits')
    assert_parity(tl, r_tl, 1e-4, 'token losses')
    assert_parity(layer.get_carry(), r_car, 1e-4, 'layer.get_carry()')
    trained = layer.get_carry()
    pre = PSSALayer(hip, w, lanes=4, max_tokens=4 * T)
    ids = np.zeros((4, T), np.uint32)
    for s in seqs:
        ids[s.lane] = s.inputs
    pre.prefill_inference(ids)
    np.testing.assert_array_equal(pre.get_carry(), trained)
    layer.close()
    pre.close()


def test_config3_width_batch_properties(hip):
    """The config-3 model (d=768, s=256, k=32, C=512, V=16384, 12 layers,
    bf16) on 8 lanes x 40 tokens: per-token losses equal the cross entropy of
    the returned logits (f64), the carries equal prefill's bit for bit, and
    the run is deterministic."""
    say("train forward config3 width")
    cfg = PSSAConfig(depth=12, d_vocab=16384, d_latent=768, d_state=256, d_mem_key=32, mem_capacity=512)
    w = ModelWeights.init(cfg, 0, "baseline")
    w.populate_banks(1)
    rng = np.random.default_rng(2)
    seqs = random_seqs(rng, cfg.d_vocab, [(i, 40, False) for i in range(8)])
    outs = []
    for _ in range(2):
        layer = PSSALayer(hip, w, lanes=8, max_tokens=320, weight_dtype="bf16")
        loss, tl, lg = layer.batch_forward(seqs, want_token_losses=True, want_logits=True)
        outs.append((loss, tl, lg, layer.get_carry()))
        layer.close()
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)
    loss, tl, lg, car = outs[0]
    lg64 = lg.astype(np.float64)
    mx = lg64.max(axis=1)
    ce = mx + np.log(np.exp(lg64 - mx[:, None]).sum(axis=1)) - lg64[np.arange(320), np.concatenate([s.targets for s in seqs])]
    np.testing.assert_allclose(tl, ce, rtol=1e-5, atol=1e-5)
    assert np.isfinite(loss) and abs(loss - np.log(cfg.d_vocab)) < 1.0
    pre = PSSALayer(hip, w, lanes=8, max_tokens=320, weight_dtype="bf16")
    pre.prefill_inference(np.stack([s.inputs for s in seqs]))
    np.testing.assert_array_equal(pre.get_carry(), car)
    pre.close()


def test_batch_forward_rejects_bad_batches_before_running(hip):
    say("train forward validation")
    w = small(depth=1)
    layer = PSSALayer(hip, w, lanes=3, max_tokens=16)
    carry = (np.random.default_rng(1).standard_normal(layer.carry_shape()) * 0.1).astype(np.float32)
    layer.set_carry(carry)
    cases = [
        ([], "sequence count"),
        ([(0, [1], [2])] * 4, "sequence count"),
        ([(0, [1], [2]), (0, [3], [4])], "distinct lane"),
        ([(3, [1], [2])], "distinct lane"),
        ([(0, [], [])], "nonempty"),
        ([(0, [1] * 17, [2] * 17)], "no longer than"),
        ([(0, [1] * 9, [2] * 9), (1, [1] * 8, [2] * 8)], "max_tokens"),
        ([(0, [1, 211], [2, 3])], "outside the model vocabulary"),
        ([(0, [1, 2], [2, 211])], "outside the model vocabulary"),
    ]
    for seqs, msg in cases:
        with pytest.raises(HipError, match=msg):
            layer.batch_forward(seqs)
    np.testing.assert_array_equal(layer.get_carry(), carry)
    layer.close()
    w.set_hybrid_read(True, 0.9)
    hyb = PSSALayer(hip, w, lanes=1, max_tokens=4)
    with pytest.raises(HipError, match="hybrid read"):
        hyb.batch_forward([(0, [1], [2])])
    hyb.close()
