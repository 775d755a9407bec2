"""The `.pssa` reader (pssa_amd/checkpoint.py) on the reference's V6 fixture
and on V8 files written here from the format (src/checkpoint.rs:912-1066),
including the reference's load-time refusals."""
import struct

import numpy as np
import pytest

from pssa_amd import ModelWeights, PSSAConfig
from pssa_amd import checkpoint as ck

GOLDEN = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden")


class Writer:
    """The reference's Writer primitives (src/checkpoint.rs:488-519): little
    endian u64 / f32, float arrays as a u64 length then the values."""

    def __init__(self):
        self.b = bytearray()

    def u64(self, n):
        self.b += struct.pack("<Q", n)

    def f32(self, x):
        self.b += struct.pack("<f", x)

    def floats(self, a):
        a = np.asarray(a, np.float32).ravel()
        self.u64(a.size)
        self.b += a.astype("<f4").tobytes()

    def usizes(self, a):
        a = np.asarray(a, np.uint64).ravel()
        self.u64(a.size)
        self.b += a.astype("<u8").tobytes()

    def param(self, a):
        """write_matrix / write_vector: data, grad, m, v (src/checkpoint.rs:613-645)."""
        for x in (a, np.zeros_like(a), np.zeros_like(a), np.zeros_like(a)):
            self.floats(x)


def v8_bytes(w: ModelWeights, carry, *, depth=None, scales=None, step=7, vocab=None):
    """payload_for_v8 + write_block (src/checkpoint.rs:958-1010) with an empty
    tokenizer/schedule tail (the reader stops before it)."""
    c = w.cfg
    depth = c.depth if depth is None else depth
    if scales is None:
        scales = [np.float32(1.0) / np.sqrt(np.float32(depth))] * (depth - 1)
    p = Writer()
    for n in (c.d_vocab, c.d_latent, c.d_state, c.d_mem_key, c.mem_capacity, 8):
        p.u64(n)
    for x in (1e-3, 0.9, 0.999, 0.0, 1e-8, c.tau_mem, 0.5):
        p.f32(x)
    p.u64(depth)
    p.floats(scales)
    p.u64(step)
    p.u64(0x1234)
    vocab = vocab if vocab is not None else []
    p.u64(len(vocab))
    for t in vocab:
        p.u64(len(t.encode()))
        p.b += t.encode()
    p.param(w.embed)
    p.param(w.unembed)
    for l, b in enumerate(w.blocks):
        for a in (b.a_raw, b.w_delta, b.w_b, b.w_c, b.w_qx, b.w_qh, b.w_gate, b.w_proj, b.mlp_w1, b.mlp_w2):
            p.param(a)
        p.param(b.norm_gamma)
        p.param(b.norm_beta)
        p.floats(carry[l])
        p.u64(b.mem_count)
        p.u64(b.mem_write_head)
        p.floats(b.mem_keys)
        p.floats(b.mem_values)
        p.floats(b.mem_norm_sq)
        p.floats(b.mem_confidence)
        p.usizes(b.mem_last_seen)
        p.param(b.adapter_down)
        p.param(b.adapter_up)
        p.floats(b.adapter_slow)
    p.usizes(np.zeros(c.d_vocab, np.uint64))
    payload = bytes(p.b)
    return b"PSSA" + struct.pack("<HQQ", 8, len(payload), ck.fnv1a64(payload)) + payload


def depth2():
    cfg = PSSAConfig(depth=2, d_vocab=11, d_latent=8, d_state=4, d_mem_key=4, mem_capacity=5)
    w = ModelWeights.init(cfg, 9, "baseline")
    w.populate_banks(10, count=5)
    rng = np.random.default_rng(2)
    for b in w.blocks:
        b.adapter_up[:] = rng.standard_normal(b.adapter_up.shape).astype(np.float32)
        b.adapter_slow[:] = rng.standard_normal(b.adapter_slow.shape).astype(np.float32)
        b.mem_write_head = 3
        b.mem_last_seen[:] = np.arange(5, dtype=np.uint64) + 40
    carry = rng.standard_normal((2, cfg.d_latent * cfg.d_state)).astype(np.float32)
    return w, carry


def test_v8_round_trip_of_a_depth_two_model():
    w, carry = depth2()
    vocab = ["<unk>"] + [f"t{i}" for i in range(1, 11)]
    got = ck.load_bytes(v8_bytes(w, carry, vocab=vocab))
    assert got.version == 8 and got.step_counter == 7 and got.vocabulary == vocab
    import dataclasses
    assert dataclasses.replace(got.weights.cfg, tau_mem=w.cfg.tau_mem) == w.cfg
    assert np.float32(got.weights.cfg.tau_mem) == np.float32(w.cfg.tau_mem)
    np.testing.assert_array_equal(got.carry, carry)
    np.testing.assert_array_equal(got.weights.embed, w.embed)
    np.testing.assert_array_equal(got.weights.unembed, w.unembed)
    for b, a in zip(got.weights.blocks, w.blocks):
        for name in ("a_raw", "w_delta", "w_b", "w_c", "w_qx", "w_qh", "w_gate", "w_proj", "mlp_w1", "mlp_w2",
                     "norm_gamma", "norm_beta", "mem_keys", "mem_values", "mem_norm_sq", "mem_confidence",
                     "mem_last_seen", "adapter_down", "adapter_up", "adapter_slow"):
            np.testing.assert_array_equal(getattr(b, name), getattr(a, name), err_msg=name)
        assert (b.mem_count, b.mem_write_head) == (a.mem_count, a.mem_write_head)


@pytest.mark.parametrize("kw,msg", [
    (dict(depth=1, scales=[]), "V8 requires stacked depth"),
    (dict(depth=33, scales=[0.5] * 32), "depth must be in 1..=32"),
    (dict(scales=[0.7071, 0.7071]), "residual scales length"),
    (dict(scales=[0.7071]), "residual scales must equal 1/sqrt"),
    (dict(scales=[np.nextafter(np.float32(1) / np.sqrt(np.float32(2)), np.float32(1))]),
     "residual scales must equal 1/sqrt"),
    (dict(step=(1 << 64) - 1), "step_counter is exhausted"),
    (dict(vocab=["a"] + ["t"] * 10), "index 0 must be <unk>"),
    (dict(vocab=["<unk>"] + ["t"] * 10), "must be unique"),
    (dict(vocab=["<unk>", "x"]), "zero or d_vocab"),
])
def test_v8_load_refusals(kw, msg):
    """load_v8 / read_vocab refusals (src/checkpoint.rs:732-830, 1050-1066)."""
    w, carry = depth2()
    with pytest.raises(ck.CheckpointError, match=msg):
        ck.load_bytes(v8_bytes(w, carry, **kw))


def test_container_refusals():
    w, carry = depth2()
    good = v8_bytes(w, carry)
    bad_sum = bytearray(good)
    bad_sum[-1] ^= 1
    with pytest.raises(ck.CheckpointError, match="checksum"):
        ck.load_bytes(bytes(bad_sum))
    with pytest.raises(ck.CheckpointError, match="payload length"):
        ck.load_bytes(good[:-1])
    with pytest.raises(ck.CheckpointError, match="not a PSSA"):
        ck.load_bytes(b"PSSX" + good[4:])
    v9 = bytearray(good)
    v9[4:6] = struct.pack("<H", 9)
    with pytest.raises(ck.CheckpointError, match="unsupported checkpoint version"):
        ck.load_bytes(bytes(v9))


def test_reference_v6_fixture_loads():
    """tests/fixtures/v6-word-pre-bpe.pssa, which the reference loads as V6
    without a tokenizer (tests/bpe_repair.rs:94-96): the V6 branch of the
    payload order (src/checkpoint.rs:1344-1418)."""
    got = ck.load(f"{GOLDEN}/v6-word-pre-bpe.pssa")
    c = got.weights.cfg
    assert got.version == 6 and c.depth == 1
    assert got.vocabulary and got.vocabulary[0] == "<unk>" and len(got.vocabulary) == c.d_vocab
    b = got.weights.blocks[0]
    assert b.mem_count <= c.mem_capacity
    assert np.all(np.isfinite(got.weights.embed)) and np.all(np.isfinite(got.carry))
    # Every byte before the embed row marks is consumed by the fields the
    # reader keeps: the file's payload ends right after those marks.
    assert np.all(b.mem_norm_sq[: b.mem_count] < 1.0)
