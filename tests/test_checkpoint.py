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


# ---- legacy V5 (src/checkpoint.rs:1444-1545) ---------------------------------
def v5_bytes(w, mem_count):
    """A V5 file of a depth-one model, as the reference's test writes one
    (tests/checkpoint_repair.rs:380-440): u32 header words, u32-length f32
    slices, physical A = -ln(1 + e^a_raw) in f32, the first mem_count slots."""
    import ctypes

    libm = ctypes.CDLL("libm.so.6")
    for name in ("expf", "log1pf"):
        getattr(libm, name).restype = ctypes.c_float
        getattr(libm, name).argtypes = [ctypes.c_float]
    c, b = w.cfg, w.blocks[0]
    out = bytearray(b"PSSA" + struct.pack("<H", 5))
    for n in (c.d_vocab, c.d_latent, c.d_state, c.d_mem_key, c.mem_capacity, 64, mem_count, 1):
        out += struct.pack("<I", n)

    def f(a):
        nonlocal out
        a = np.asarray(a, np.float32).ravel()
        out += struct.pack("<I", a.size) + a.astype("<f4").tobytes()

    f(w.embed)
    f(b.norm_gamma)
    f(b.norm_beta)
    f([-libm.log1pf(libm.expf(float(x))) for x in b.a_raw.ravel()])
    for name in ("w_delta", "w_b", "w_c", "w_qx", "w_qh", "w_gate", "w_proj", "mlp_w1", "mlp_w2"):
        f(getattr(b, name))
    f(w.unembed)
    f(b.mem_keys[:mem_count])
    f(b.mem_values[:mem_count])
    out += struct.pack("<I", 16)
    f(b.adapter_down)
    f(b.adapter_up)
    return bytes(out)


def test_reference_legacy_v5_fixture_loads():
    """tests/fixtures/legacy-v5-model.pssa (the reference's data/model.pssa):
    inference-only, no vocabulary, step 0, write head 0, the 11 stored slots
    with their norms recomputed, physical A converted to finite raw rates
    (load_checkpoint returns LegacyV5InferenceOnly, tests/checkpoint_repair.rs:
    460-467)."""
    c = ck.load(__import__("os").path.join(GOLDEN, "legacy-v5-model.pssa"))
    assert c.version == 5 and c.format == "LegacyV5InferenceOnly"
    cfg = c.weights.cfg
    assert (cfg.depth, cfg.d_vocab, cfg.d_latent, cfg.d_state, cfg.d_mem_key, cfg.mem_capacity) == \
        (1, 88, 256, 16, 32, 512)
    assert c.vocabulary == [] and c.step_counter == 0 and not c.carry.any()
    b = c.weights.blocks[0]
    assert b.mem_count == 11 and b.mem_write_head == 0
    assert np.all(np.isfinite(b.a_raw))
    # -softplus(a_raw) gives back the file's physical A (within a few ulp).
    raw = open(__import__("os").path.join(GOLDEN, "legacy-v5-model.pssa"), "rb").read()
    off = 38
    for n in (88 * 256, 256, 256):
        off += 4 + 4 * n
    phys = np.frombuffer(raw[off + 4: off + 4 + 4 * 256 * 16], "<f4")
    back = -np.logaddexp(0.0, b.a_raw.astype(np.float64)).ravel()
    np.testing.assert_allclose(back, phys, rtol=4e-6)
    norms = (b.mem_keys[:11].astype(np.float64) ** 2).sum(axis=1)
    np.testing.assert_allclose(b.mem_norm_sq[:11], norms, rtol=1e-6)
    assert np.all(b.mem_norm_sq[:11] < 1.0) and not b.mem_keys[11:].any() and not b.mem_norm_sq[11:].any()
    assert not b.adapter_slow.any()


def test_legacy_v5_round_trip_keeps_the_forward():
    """tests/checkpoint_repair.rs:443-468: a model written as V5 (one bank
    slot, zero consolidated fast weights) and loaded back gives the same
    logits within 2e-6 (the raw rates pass through -softplus and its
    inverse in f32)."""
    from oracle import oracle as O

    cfg = PSSAConfig(depth=1, d_vocab=5, d_latent=4, d_state=3, d_mem_key=2, mem_capacity=3)
    w = ModelWeights.init(cfg, 7, "reference")
    b = w.blocks[0]
    b.adapter_slow[:] = 0.0
    b.mem_keys[0] = [0.3, -0.2]
    b.mem_values[0] = [0.5, -1.0, 0.25, 2.0]
    b.mem_norm_sq[0] = 0.13
    b.mem_count, b.mem_write_head = 1, 0
    b.mem_keys[1:] = 0.0
    b.mem_values[1:] = 0.0
    loaded = ck.load_bytes(v5_bytes(w, 1))
    assert loaded.format == "LegacyV5InferenceOnly"
    lw = loaded.weights
    assert lw.blocks[0].mem_count == 1
    om, ol = O.OracleModel(w), O.OracleModel(lw)
    la = om.forward_inference(om.zero_state(), 1)
    lb = ol.forward_inference(ol.zero_state(), 1)
    assert np.max(np.abs(la - lb)) < 2e-6


def test_legacy_v5_malformed_count_and_rank_are_rejected():
    """tests/checkpoint_repair.rs:470-488: a count above the stored slots and an
    adapter rank other than 16 are refused; so are a truncated header and a
    count above the capacity."""
    cfg = PSSAConfig(depth=1, d_vocab=5, d_latent=4, d_state=3, d_mem_key=2, mem_capacity=3)
    w = ModelWeights.init(cfg, 7, "reference")
    w.blocks[0].mem_keys[0] = [0.3, -0.2]
    good = bytearray(v5_bytes(w, 1))
    ck.load_bytes(bytes(good))
    x = bytearray(good)
    x[30:34] = struct.pack("<I", 2)
    with pytest.raises(ck.CheckpointError):
        ck.load_bytes(bytes(x))
    x[30:34] = struct.pack("<I", 4)
    with pytest.raises(ck.CheckpointError, match="exceeds capacity"):
        ck.load_bytes(bytes(x))
    x = bytearray(good)
    rank = len(x) - (4 + 64 * 4) * 2 - 4
    assert struct.unpack("<I", x[rank:rank + 4])[0] == 16
    x[rank:rank + 4] = struct.pack("<I", 15)
    with pytest.raises(ck.CheckpointError, match="adapter rank"):
        ck.load_bytes(bytes(x))
    with pytest.raises(ck.CheckpointError, match="truncated"):
        ck.load_bytes(bytes(good[:30]))
