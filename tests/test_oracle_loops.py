"""The oracle's recurrent depth loops (set_loops, src/pssa.rs:2171-2184;
forward_inference_features, src/pssa.rs:2338-2373), pinned by composing them
from its single-loop path, which the reference's fixtures pin: a depth-one,
single-loop model whose only block is block l of the looped model and whose
embedding row 0 is a chosen vector returns that block's output for the vector
(its features), advancing the carry it is given.  The looped model must equal
the reference's composition of such block applications, one carry per
(block, loop), bit for bit."""
import dataclasses

import numpy as np
import pytest

from oracle import oracle as O
from pssa_amd import ModelWeights, PSSAConfig


def _model(depth, seed=3):
    cfg = PSSAConfig(depth=depth, d_vocab=41, d_latent=24, d_state=16, d_mem_key=8, mem_capacity=12)
    w = ModelWeights.init(cfg, seed, "baseline")
    w.populate_banks(seed + 1, count=cfg.mem_capacity)
    return w


def _block_models(w):
    """One depth-one model per block of w, sharing the block's arrays."""
    out = []
    for b in w.blocks:
        w1 = ModelWeights(dataclasses.replace(w.cfg, depth=1))
        w1.blocks = [b]
        w1.unembed = w.unembed
        out.append((w1, O.OracleModel(w1)))
    return out


def _apply(bm, vec, carry):
    w1, om1 = bm
    w1.embed[0] = vec
    return om1.features(carry, 0)


@pytest.mark.parametrize("depth,loops", [(1, 2), (2, 3), (3, 2)])
def test_loops_compose_block_passes(depth, loops):
    w = _model(depth)
    om = O.OracleModel(w)
    om.set_loops(loops)
    state = om.zero_state()
    assert state.shape == (depth, loops, w.cfg.d_latent * w.cfg.d_state)
    blocks = _block_models(w)
    carries = [[np.zeros((1, w.cfg.d_latent * w.cfg.d_state), np.float32) for _ in range(loops)]
               for _ in range(depth)]
    ls = np.float32(1.0) / np.float32(loops)
    scale = np.float32(1.0) / np.sqrt(np.float32(depth))
    for tok in (5, 17, 5, 40):
        got = om.features(state, tok)
        f = w.embed[tok].copy()
        for l in range(depth):
            inputs = f.copy()
            for k in range(loops):
                f = (f + ls * _apply(blocks[l], f, carries[l][k])).astype(np.float32)
            if l > 0:
                f = (inputs + scale * f).astype(np.float32)
        np.testing.assert_array_equal(got, f)
        for l in range(depth):
            for k in range(loops):
                np.testing.assert_array_equal(state[l, k], carries[l][k][0])


def test_one_loop_is_the_original_model_and_prefill_is_the_token_loop():
    w = _model(2)
    om = O.OracleModel(w)
    ids = np.array([3, 9, 27, 1, 8], np.uint32)
    s1 = om.zero_state()
    lg1 = om.prefill(s1, ids)
    om.set_loops(1)
    s2 = om.zero_state()
    np.testing.assert_array_equal(om.prefill(s2, ids), lg1)
    om.set_loops(3)
    s3, s4 = om.zero_state(), om.zero_state()
    lg3 = om.prefill(s3, ids)
    for t in ids[:-1]:
        om.forward_inference(s4, int(t), logits=False)
    np.testing.assert_array_equal(om.forward_inference(s4, int(ids[-1])), lg3)
    np.testing.assert_array_equal(s3, s4)
    assert not np.array_equal(lg3, lg1)
    with pytest.raises(ValueError):
        om.set_loops(33)
