"""Pins the CPU oracle (and the product's host-side initialisation) to the
reference's own golden fixtures, copied unchanged into tests/golden/:

  depth_one_main85d9d33_initial.pssa      PSSALayerV2::new after the recipe of
                                           tests/support/depth_one_reference.rs:4-45
  depth_one_main014f617_avx2_observed.bin  67 f32 words of reference::advance();
                                           words 0..22 are pure forward
  depth_one_main85d9d33_observed.bin       the same from the pre-SIMD commit
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import oracle as O
from pssa_amd import ModelWeights, checkpoint

INITIAL = os.path.join(GOLDEN, "depth_one_main85d9d33_initial.pssa")
AVX2_OBSERVED = os.path.join(GOLDEN, "depth_one_main014f617_avx2_observed.bin")
SCALAR_OBSERVED = os.path.join(GOLDEN, "depth_one_main85d9d33_observed.bin")
TRAINED = [os.path.join(GOLDEN, f) for f in ("depth_one_main85d9d33_trained.pssa",
                                              "depth_one_main014f617_avx2_trained.pssa")]

MATS = ["a_raw", "w_delta", "w_b", "w_c", "w_qx", "w_qh", "w_gate", "w_proj", "adapter_down",
        "mlp_w1", "norm_gamma", "norm_beta"]


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def initial():
    return checkpoint.load(INITIAL)


def test_checkpoint_reader_parses_fixture(initial):
    w = initial.weights
    assert initial.version == 7
    assert (w.cfg.d_vocab, w.cfg.d_latent, w.cfg.d_state, w.cfg.d_mem_key, w.cfg.mem_capacity) == (7, 4, 2, 2, 3)
    assert np.float32(w.cfg.tau_mem) == np.float32(0.8)
    assert initial.vocabulary == ["<unk>", "one", "two", "three", "four", "five", "six"]
    assert initial.rng_state == 0x78CAF14A3C5BACC5
    b = w.blocks[0]
    # Recipe: two inserted memories and a patterned carry (depth_one_reference.rs:35-40).
    assert b.mem_count == 2 and b.mem_write_head == 0
    np.testing.assert_array_equal(b.mem_keys[:2], np.float32([[0.1, -0.2], [-0.2, 0.15]]))
    np.testing.assert_array_equal(initial.carry[0], np.float32([np.float32(i) * np.float32(0.005) - np.float32(0.01) for i in range(8)]))
    # squared_norm keeps f64 accumulation, then rounds (src/memory.rs:181-192).
    assert b.mem_norm_sq[0] == O.squared_norm(b.mem_keys[0])
    assert b.mem_norm_sq[1] == O.squared_norm(b.mem_keys[1])


@pytest.mark.parametrize("path", TRAINED)
def test_checkpoint_reader_verifies_trained_fixtures(path):
    ck = checkpoint.load(path)
    assert ck.version == 7 and ck.weights.cfg.depth == 1
    with open(path, "rb") as f:
        raw = bytearray(f.read())
    raw[-1] ^= 1
    with pytest.raises(checkpoint.CheckpointError, match="checksum"):
        checkpoint.load_bytes(bytes(raw))


@pytest.mark.parametrize("source", ["oracle", "product"])
def test_reference_init_is_bit_identical_to_fixture(initial, source):
    cfg = initial.weights.cfg
    if source == "oracle":
        m = ModelWeights(cfg)
        state = O.OracleModel(m).init_reference(192)
    else:
        m = ModelWeights.init(cfg, 192, "reference")
        state = m.rng_state
    assert state == initial.rng_state
    ref = initial.weights
    np.testing.assert_array_equal(bits(m.embed), bits(ref.embed))
    np.testing.assert_array_equal(bits(m.unembed), bits(ref.unembed))
    for name in MATS:
        np.testing.assert_array_equal(bits(getattr(m.blocks[0], name)), bits(getattr(ref.blocks[0], name)), err_msg=name)
    # Zero-initialised fast paths (src/pssa.rs:683, src/adapter.rs:19) that the
    # recipe then overwrites; the fixture holds the recipe's patterns.
    assert not m.blocks[0].mlp_w2.any() and not m.blocks[0].adapter_up.any()
    recipe_w2 = np.float32([np.sin(np.float32(i) * np.float32(0.23)) * np.float32(0.07) for i in range(32)])
    np.testing.assert_allclose(ref.blocks[0].mlp_w2.ravel(), recipe_w2, rtol=0, atol=1e-7)


def _forward_words(ck, avx2: bool):
    om = O.OracleModel(ck.weights)
    state = ck.carry.copy()
    with O.Dot(avx2):
        loss, logits = om.train_chunk_forward(state, [1, 2, 1], [2, 1, 3])
        loss2, _ = om.train_chunk_forward(state, [4], [5])
    return bits(np.concatenate([[loss], logits.ravel(), [loss2]]))


def test_forward_words_match_avx2_golden_bitwise(initial):
    """Words 0..22 of reference::advance (tests/support/depth_one_reference.rs:47-55):
    chunk [1,2,1]->[2,1,3] loss and 3x7 scaled logits, then chunk [4]->[5] loss
    from the continued carry.  This is the golden the reference's own parity test
    selects on x86-64 with AVX2/FMA (tests/depth_one_parity.rs:23-30)."""
    expected = np.fromfile(AVX2_OBSERVED, dtype="<u4")[:23]
    np.testing.assert_array_equal(_forward_words(initial, avx2=True), expected)


def test_pre_simd_golden_differs_only_in_second_token(initial):
    """The pre-SIMD commit's golden predates rounding changes the reference made
    on purpose (tests/depth_one_parity.rs:1-3).  The oracle, which restates the
    current reference, reproduces all of it except the second token's logits."""
    expected = np.fromfile(SCALAR_OBSERVED, dtype="<u4")[:23]
    got = _forward_words(initial, avx2=False)
    diff = {i for i in range(23) if got[i] != expected[i]}
    assert diff <= set(range(8, 15)), diff
    assert len(diff) <= 7
    g, e = got.view(np.float32), expected.view(np.float32)
    assert np.max(np.abs(g - e)) < 1e-6


def test_portable_and_avx2_trees_agree_on_eight_wide_dots():
    # For n == 8 both trees add the same rounded products in the same order.
    rng = np.random.default_rng(3)
    for _ in range(100):
        a, b = rng.standard_normal(8, dtype=np.float32), rng.standard_normal(8, dtype=np.float32)
        with O.Dot(True):
            x = O.dot(a, b)
        with O.Dot(False):
            y = O.dot(a, b)
        assert bits(x) == bits(y)


def test_dot_trees_match_their_definitions():
    rng = np.random.default_rng(7)
    for n in (1, 3, 4, 7, 9, 16, 31, 33, 100, 768):
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        # portable: four scalar chains, ((c0+c1)+(c2+c3)), scalar tail (src/linalg.rs:282-298)
        acc = [np.float32(0)] * 4
        i = 0
        while i + 4 <= n:
            for q in range(4):
                acc[q] = np.float32(acc[q] + np.float32(a[i + q] * b[i + q]))
            i += 4
        s = np.float32(np.float32(acc[0] + acc[1]) + np.float32(acc[2] + acc[3]))
        while i < n:
            s = np.float32(s + np.float32(a[i] * b[i]))
            i += 1
        with O.Dot(False):
            assert bits(O.dot(a, b)) == bits(s), n
        with O.Dot(True):
            assert abs(float(O.dot(a, b)) - float(np.dot(a.astype(np.float64), b))) < 1e-4 * (1 + np.abs(a * b).sum())
