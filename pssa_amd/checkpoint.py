"""Reader of the reference's `.pssa` checkpoints (V6, V7 and V8, and the
legacy inference-only V5).

Container (src/checkpoint.rs:3-27, 1116-1126, 1288-1307):
  b"PSSA" | version:u16 | payload_len:u64 | fnv1a64(payload):u64 | payload
V6/V7 payload order: src/checkpoint.rs:912-956 (V7 appends the tokenizer /
schedule tail, src/checkpoint.rs:1309-1342); V8: src/checkpoint.rs:961-1048.
Only what the inference path needs is kept: parameters, banks and the
per-block recurrent carry (h_persistent).  Gradients and Adam moments are
read and dropped.
V5 (load_v5, src/checkpoint.rs:1444-1545) has no container: b"PSSA" |
version:u16 | eight u32 (d_vocab, d_latent, d_state, d_mem_key, mem_capacity,
chunk_len, mem_count, adapter_count) | u32-length-prefixed f32 slices.
"""
from __future__ import annotations

import dataclasses
import struct

import numpy as np

from .weights import ADAPTER_RANK, ModelWeights, PSSAConfig

HEADER_LEN = 22
MAX_MODEL_DEPTH = 32  # src/checkpoint.rs:41
U64_MAX = (1 << 64) - 1


def fnv1a64(data: bytes) -> int:
    h = 0xCBF29CE484222325
    for b in data:
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


class CheckpointError(ValueError):
    pass


class _Reader:
    def __init__(self, b: bytes):
        self.b = b
        self.o = 0

    def take(self, n: int, what: str) -> bytes:
        if self.o + n > len(self.b):
            raise CheckpointError(f"truncated while reading {what}")
        out = self.b[self.o:self.o + n]
        self.o += n
        return out

    def u64(self, what: str) -> int:
        return struct.unpack("<Q", self.take(8, what))[0]

    def f32(self, what: str) -> float:
        x = struct.unpack("<f", self.take(4, what))[0]
        if not np.isfinite(x):
            raise CheckpointError(f"non-finite {what}")
        return x

    def floats(self, n_expected: int, what: str, nonneg: bool = False) -> np.ndarray:
        n = self.u64(f"{what} length")
        if n != n_expected:
            raise CheckpointError(f"{what} length {n}, expected {n_expected}")
        a = np.frombuffer(self.take(4 * n, what), dtype="<f4").astype(np.float32)
        if not np.all(np.isfinite(a)):
            raise CheckpointError(f"non-finite {what}")
        if nonneg and np.any(a < 0):
            raise CheckpointError(f"negative {what}")
        return a

    def usizes(self, n_expected: int, what: str) -> np.ndarray:
        n = self.u64(f"{what} length")
        if n != n_expected:
            raise CheckpointError(f"{what} length {n}, expected {n_expected}")
        return np.frombuffer(self.take(8 * n, what), dtype="<u8").astype(np.uint64)

    def matrix(self, n: int, what: str) -> np.ndarray:
        data = self.floats(n, what)
        self.floats(n, f"{what}.grad")
        self.floats(n, f"{what}.m")
        self.floats(n, f"{what}.v", nonneg=True)
        return data


@dataclasses.dataclass
class LoadedCheckpoint:
    version: int
    weights: ModelWeights
    carry: np.ndarray  # [depth, d*s] h_persistent per block
    step_counter: int
    rng_state: int
    vocabulary: list[str]
    hyper: dict
    # CheckpointFormat (src/checkpoint.rs:72-78): "V6", "V7", "V8", or
    # "LegacyV5InferenceOnly" (no recoverable training state).
    format: str = ""


def _config(r: _Reader):
    """config_from_payload + validate_config (src/checkpoint.rs:110-147, 683-700)."""
    dims = [r.u64(n) for n in ("d_vocab", "d_latent", "d_state", "d_mem_key", "mem_capacity", "chunk_len")]
    hyper = {n: r.f32(n) for n in ("lr", "beta1", "beta2", "weight_decay", "eps", "tau_mem", "ema_alpha")}
    if any(x == 0 for x in dims):
        raise CheckpointError("all dimensions, memory capacity, and chunk length must be positive")
    if not (hyper["lr"] > 0 and hyper["eps"] > 0 and hyper["tau_mem"] > 0):
        raise CheckpointError("lr, eps, and tau_mem must be finite and positive")
    if not (0.0 <= hyper["beta1"] < 1.0 and 0.0 <= hyper["beta2"] < 1.0):
        raise CheckpointError("Adam betas must be in [0, 1)")
    if not (hyper["weight_decay"] >= 0.0 and 0.0 <= hyper["ema_alpha"] <= 1.0):
        raise CheckpointError("weight decay/ema alpha invalid")
    return dims, hyper


def _residual_scales(r: _Reader, depth: int) -> None:
    """The V8 scale words (src/checkpoint.rs:1053-1061, 817-830): depth - 1
    of them, each bit-equal to 1/sqrt(depth) in f32 (the device applies that
    constant)."""
    scales = r.floats(depth - 1, "residual scales")
    expected = np.float32(1.0) / np.sqrt(np.float32(depth))
    if np.any(scales.view(np.uint32) != np.float32(expected).view(np.uint32)):
        raise CheckpointError("residual scales must equal 1/sqrt(depth)")


def _vocab(r: _Reader, d_vocab: int) -> list[str]:
    """read_vocab + validate_vocab (src/checkpoint.rs:701-757)."""
    n = r.u64("vocabulary count")
    if n not in (0, d_vocab):
        raise CheckpointError("vocabulary count must be zero or d_vocab")
    if n > (len(r.b) - r.o) // 8:
        raise CheckpointError("vocabulary count exceeds remaining checkpoint bytes")
    try:
        v = [r.take(r.u64("vocabulary token length"), "vocabulary token").decode("utf-8") for _ in range(n)]
    except UnicodeDecodeError:
        raise CheckpointError("vocabulary token is not UTF-8") from None
    if v and v[0] != "<unk>":
        raise CheckpointError("vocabulary index 0 must be <unk>")
    if len(set(v)) != len(v):
        raise CheckpointError("vocabulary tokens must be unique")
    return v


def _block(r: _Reader, w: ModelWeights, l: int, carry: np.ndarray, embed_first: bool) -> None:
    c = w.cfg
    d, s, k, C = c.d_latent, c.d_state, c.d_mem_key, c.mem_capacity
    b = w.blocks[l]
    if embed_first:
        w.embed[:] = r.matrix(c.d_vocab * d, "embed_w").reshape(c.d_vocab, d)
    order = [("a_raw", d * s), ("w_delta", d * d), ("w_b", s * d), ("w_c", s * d), ("w_qx", k * d),
             ("w_qh", k * d), ("w_gate", d * d), ("w_proj", d * d), ("mlp_w1", 2 * d * d),
             ("mlp_w2", 2 * d * d)]
    for name, n in order:
        getattr(b, name)[...] = r.matrix(n, name).reshape(getattr(b, name).shape)
    if embed_first:
        w.unembed[:] = r.matrix(c.d_vocab * d, "unembed_w").reshape(c.d_vocab, d)
    b.norm_gamma[:] = r.matrix(d, "norm_gamma")
    b.norm_beta[:] = r.matrix(d, "norm_beta")
    carry[l] = r.floats(d * s, "h_persistent")
    b.mem_count = r.u64("memory count")
    b.mem_write_head = r.u64("memory write_head")
    if b.mem_count > C or b.mem_write_head >= C or (b.mem_count < C and b.mem_write_head != 0):
        raise CheckpointError("memory count/write head invalid")
    b.mem_keys[...] = r.floats(C * k, "memory keys").reshape(C, k)
    b.mem_values[...] = r.floats(C * d, "memory values").reshape(C, d)
    b.mem_norm_sq[:] = r.floats(C, "memory norm_sq", nonneg=True)
    b.mem_confidence[:] = r.floats(C, "memory confidence", nonneg=True)
    b.mem_last_seen[:] = r.usizes(C, "memory last_seen_step")
    b.adapter_down[...] = r.matrix(ADAPTER_RANK * d, "adapter.down").reshape(ADAPTER_RANK, d)
    b.adapter_up[...] = r.matrix(d * ADAPTER_RANK, "adapter.up").reshape(d, ADAPTER_RANK)
    b.adapter_slow[...] = r.floats(d * ADAPTER_RANK, "adapter.consolidated_up").reshape(d, ADAPTER_RANK)


# ---- legacy V5 (src/checkpoint.rs:1421-1545) ---------------------------------
HEADER_V5_LEN = 38  # src/checkpoint.rs:44


def _libm():
    import ctypes
    import ctypes.util

    m = ctypes.CDLL(ctypes.util.find_library("m") or "libm.so.6")
    for name in ("expm1f", "logf", "expf", "log1pf"):
        getattr(m, name).restype = ctypes.c_float
        getattr(m, name).argtypes = [ctypes.c_float]
    return m


def _inverse_softplus(y: np.ndarray) -> np.ndarray:
    """inverse_softplus (src/checkpoint.rs:1437-1443) in f32 with the C
    library's expm1f / logf / expf / log1pf, the functions Rust's f32
    exp_m1 / ln / exp / ln_1p call on Linux."""
    m = _libm()
    out = np.empty_like(y, dtype=np.float32)
    for i, v in enumerate(y.astype(np.float32).ravel().tolist()):
        if v > 20.0:
            out.flat[i] = np.float32(v) + np.float32(m.log1pf(-m.expf(-v)))
        else:
            out.flat[i] = m.logf(m.expm1f(v))
    return out


def _squared_norm(x: np.ndarray) -> np.float32:
    """HyperbolicEpisodicBankV2::squared_norm (src/memory.rs:181-192): the
    left-to-right f64 sum of squares, rounded to f32 with the open-ball
    guard."""
    acc = 0.0
    for v in x.astype(np.float64).tolist():
        acc += v * v
    f = np.float32(acc)
    if acc < 1.0 and f == np.float32(1.0):
        f = np.nextafter(np.float32(1.0), np.float32(0.0))
    return f


def _load_v5(data: bytes) -> LoadedCheckpoint:
    """load_v5 (src/checkpoint.rs:1444-1545): parameters of PSSALayerV2::new(cfg,
    42) overwritten by the file's tensors; physical A converted to raw rates
    by inverse_softplus(-A); the bank holds mem_count slots with write head 0
    and norms recomputed; no vocabulary, carries, step or optimizer state."""
    if len(data) < HEADER_V5_LEN:
        raise CheckpointError("truncated legacy V5 header")
    r = _Reader(data)
    r.take(4, "magic")
    r.take(2, "version")

    def u32(what: str) -> int:
        return struct.unpack("<I", r.take(4, what))[0]

    V, d, s, k, C, chunk = (u32(n) for n in ("d_vocab", "d_latent", "d_state", "d_mem_key", "mem_capacity",
                                             "chunk_len"))
    if min(V, d, s, k, C, chunk) == 0:
        raise CheckpointError("all dimensions, memory capacity, and chunk length must be positive")
    mem_count, adapter_count = u32("mem_count"), u32("adapter_count")
    if mem_count > C:
        raise CheckpointError("legacy mem_count exceeds capacity")
    if adapter_count != 1:
        raise CheckpointError("legacy requires exactly one adapter")
    # ensure_backed_by_file with the legacy count (src/checkpoint.rs:163-203).
    params = (V * d + d * s + d * d + 2 * s * d + 2 * k * d + 2 * d * d + 2 * (2 * d * d) + V * d
              + 2 * ADAPTER_RANK * d + 2 * d)
    required = 4 * params + 19 * 4 + 4 * mem_count * (k + d)
    if len(data) - r.o < required:
        raise CheckpointError("checkpoint is too short for its tensors")

    def sl(n_expected: int, what: str) -> np.ndarray:
        n = u32(f"{what} length")
        if n != n_expected:
            raise CheckpointError(f"legacy {what} length {n}, expected {n_expected}")
        a = np.frombuffer(r.take(4 * n, what), dtype="<f4").astype(np.float32)
        if not np.all(np.isfinite(a)):
            raise CheckpointError(f"non-finite {what}")
        return a

    cfg = PSSAConfig(depth=1, d_vocab=V, d_latent=d, d_state=s, d_mem_key=k, mem_capacity=C)
    w = ModelWeights.init(cfg, 42, "reference")
    b = w.blocks[0]
    w.embed[:] = sl(V * d, "embed_w").reshape(V, d)
    b.norm_gamma[:] = sl(d, "norm_gamma")
    b.norm_beta[:] = sl(d, "norm_beta")
    a_phys = sl(d * s, "a_mat physical")
    bad = int(np.count_nonzero(~(a_phys < 0.0)))
    if bad:
        raise CheckpointError(
            f"legacy physical A contains {bad} nonfinite or nonnegative entries; refusing unsafe conversion")
    a_raw = _inverse_softplus(-a_phys)
    if not np.all(np.isfinite(a_raw)):
        raise CheckpointError("legacy physical A cannot be represented as finite raw rates")
    b.a_raw[...] = a_raw.reshape(d, s)
    for name, n in (("w_delta", d * d), ("w_b", s * d), ("w_c", s * d), ("w_qx", k * d), ("w_qh", k * d),
                    ("w_gate", d * d), ("w_proj", d * d), ("mlp_w1", 2 * d * d), ("mlp_w2", 2 * d * d)):
        getattr(b, name)[...] = sl(n, name).reshape(getattr(b, name).shape)
    w.unembed[:] = sl(V * d, "unembed_w").reshape(V, d)
    b.mem_keys[:mem_count] = sl(mem_count * k, "memory keys").reshape(mem_count, k)
    b.mem_values[:mem_count] = sl(mem_count * d, "memory values").reshape(mem_count, d)
    b.mem_count = mem_count
    b.mem_write_head = 0
    for i in range(mem_count):
        sq = _squared_norm(b.mem_keys[i])
        if not (np.isfinite(sq) and sq < 1.0):
            raise CheckpointError(f"legacy memory key {i} is outside the open Poincare ball")
        b.mem_norm_sq[i] = sq
    rank = u32("adapter rank")
    if rank != ADAPTER_RANK:
        raise CheckpointError(f"legacy adapter rank {rank}; expected {ADAPTER_RANK}")
    b.adapter_down[...] = sl(ADAPTER_RANK * d, "adapter down").reshape(ADAPTER_RANK, d)
    b.adapter_up[...] = sl(d * ADAPTER_RANK, "adapter up").reshape(d, ADAPTER_RANK)
    if r.o != len(data):
        raise CheckpointError("trailing bytes after the legacy checkpoint")
    carry = np.zeros((1, d * s), dtype=np.float32)
    hyper = {"lr": 1e-3, "beta1": 0.9, "beta2": 0.999, "weight_decay": 0.01, "eps": 1e-8, "tau_mem": 0.1,
             "ema_alpha": 0.01, "chunk_len": chunk}
    return LoadedCheckpoint(5, w, carry, 0, w.rng_state, [], hyper, "LegacyV5InferenceOnly")


def load_bytes(data: bytes, verify_checksum: bool = True) -> LoadedCheckpoint:
    if len(data) < 6 or data[:4] != b"PSSA":
        raise CheckpointError("not a PSSA checkpoint")
    version = struct.unpack("<H", data[4:6])[0]
    if version == 5:
        return _load_v5(data)
    if len(data) < HEADER_LEN:
        raise CheckpointError("truncated checkpoint header")
    plen, checksum = struct.unpack("<QQ", data[6:22])
    if len(data) != HEADER_LEN + plen:
        raise CheckpointError("payload length does not match file")
    payload = data[HEADER_LEN:]
    if verify_checksum and fnv1a64(payload) != checksum:
        raise CheckpointError("payload checksum mismatch")
    if version not in (6, 7, 8):
        raise CheckpointError(f"unsupported checkpoint version {version}")
    r = _Reader(payload)
    (V, d, s, k, C, _chunk), hyper = _config(r)
    depth = 1
    if version == 8:
        depth = r.u64("depth")
        if not 1 <= depth <= MAX_MODEL_DEPTH:
            raise CheckpointError(f"depth must be in 1..={MAX_MODEL_DEPTH}")
        if depth == 1:
            raise CheckpointError("V8 requires stacked depth; use V7 for depth one")
        _residual_scales(r, depth)
    cfg = PSSAConfig(depth=depth, d_vocab=V, d_latent=d, d_state=s, d_mem_key=k, mem_capacity=C,
                     tau_mem=hyper["tau_mem"])
    w = ModelWeights(cfg)
    carry = np.zeros((depth, d * s), dtype=np.float32)
    step = r.u64("step_counter")
    if step == U64_MAX:
        raise CheckpointError("step_counter is exhausted")
    rng = r.u64("rng state")
    vocab = _vocab(r, V)
    if version == 8:
        w.embed[:] = r.matrix(V * d, "embed_w").reshape(V, d)
        w.unembed[:] = r.matrix(V * d, "unembed_w").reshape(V, d)
        for l in range(depth):
            _block(r, w, l, carry, embed_first=False)
    else:
        _block(r, w, 0, carry, embed_first=True)
    r.usizes(V, "embed_row_marks")
    # The tokenizer / schedule tail (V7/V8) is not needed by the forward path.
    w.rng_state = rng
    return LoadedCheckpoint(version, w, carry, step, rng, vocab, hyper, f"V{version}")


def load(path: str, verify_checksum: bool = True) -> LoadedCheckpoint:
    with open(path, "rb") as f:
        return load_bytes(f.read(), verify_checksum)
