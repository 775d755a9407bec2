"""Host-side model parameters of the PSSA inference path.

`PSSAConfig` mirrors the forward-path fields of the reference's PSSAConfigV2
(src/pssa.rs:254-331); `ModelWeights` holds the parameters of PSSALayerV2
(embedding, unembedding, and one `BlockWeights` per PSSAContinuousBlockV2,
src/pssa.rs:506-620) as numpy arrays and exposes them through the C ABI's
`pssa_hip_weights` view.  Initialisation runs in libpssa_hip's host code.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import math

import numpy as np

from . import _abi

ADAPTER_RANK = 16  # src/pssa.rs:644


@dataclasses.dataclass(frozen=True)
class PSSAConfig:
    depth: int = 1
    d_vocab: int = 10_000
    d_latent: int = 256
    d_state: int = 16
    d_mem_key: int = 32
    mem_capacity: int = 512
    tau_mem: float = 0.1
    adapter_rank: int = ADAPTER_RANK

    def validate(self) -> None:
        # PSSAConfigV2::validate (src/pssa.rs:272-310), forward-path subset.
        if not 1 <= self.depth <= 32:
            raise ValueError("depth must be in 1..=32")
        if min(self.d_vocab, self.d_latent, self.d_state, self.d_mem_key, self.mem_capacity,
               self.adapter_rank) <= 0:
            raise ValueError("all model dimensions and memory capacity must be positive")
        if not (math.isfinite(self.tau_mem) and self.tau_mem > 0):
            raise ValueError("tau_mem must be finite and positive")

    def to_c(self) -> _abi.Config:
        return _abi.Config(self.depth, self.d_vocab, self.d_latent, self.d_state, self.d_mem_key,
                           self.mem_capacity, self.adapter_rank, self.tau_mem, 0)

    def parameter_count(self) -> int:
        """Trainable scalars as in PSSALayerV2::parameter_count (src/pssa.rs:3744-3754)."""
        d, s, k, r, V = self.d_latent, self.d_state, self.d_mem_key, self.adapter_rank, self.d_vocab
        block = d * s + d * d + 2 * s * d + 2 * k * d + 2 * d * d + 2 * d * d + 2 * d * d + 2 * d + 2 * r * d
        return 2 * V * d + self.depth * block


class BlockWeights:
    """Parameters, carry-free bank state and adapter of one continuous block."""

    SHAPES = {
        "norm_gamma": lambda c: (c.d_latent,),
        "norm_beta": lambda c: (c.d_latent,),
        "a_raw": lambda c: (c.d_latent, c.d_state),
        "w_delta": lambda c: (c.d_latent, c.d_latent),
        "w_b": lambda c: (c.d_state, c.d_latent),
        "w_c": lambda c: (c.d_state, c.d_latent),
        "w_qx": lambda c: (c.d_mem_key, c.d_latent),
        "w_qh": lambda c: (c.d_mem_key, c.d_latent),
        "w_gate": lambda c: (c.d_latent, c.d_latent),
        "w_proj": lambda c: (c.d_latent, c.d_latent),
        "adapter_down": lambda c: (c.adapter_rank, c.d_latent),
        "adapter_up": lambda c: (c.d_latent, c.adapter_rank),
        "adapter_slow": lambda c: (c.d_latent, c.adapter_rank),
        "mlp_w1": lambda c: (2 * c.d_latent, c.d_latent),
        "mlp_w2": lambda c: (c.d_latent, 2 * c.d_latent),
        "mem_keys": lambda c: (c.mem_capacity, c.d_mem_key),
        "mem_values": lambda c: (c.mem_capacity, c.d_latent),
        "mem_norm_sq": lambda c: (c.mem_capacity,),
        "mem_confidence": lambda c: (c.mem_capacity,),
    }

    def __init__(self, cfg: PSSAConfig):
        for name, shape in self.SHAPES.items():
            setattr(self, name, np.zeros(shape(cfg), dtype=np.float32))
        self.norm_gamma[:] = 1.0
        self.mem_confidence[:] = 1.0
        self.mem_last_seen = np.zeros(cfg.mem_capacity, dtype=np.uint64)
        self.mem_count = 0
        self.mem_write_head = 0
        # Hybrid read state (src/memory.rs:19-33): runtime-only, never checkpointed.
        self.mem_hybrid_gate = np.ones(cfg.mem_capacity, dtype=np.float32)
        self.mem_hybrid_age = np.zeros(cfg.mem_capacity, dtype=np.uint64)
        self.mem_hybrid_enabled = False
        self.mem_hybrid_lam = 1.0
        # memory.top_k (src/memory.rs:102-108): runtime-only, 0 = full read.
        self.mem_top_k = 0
        # memory.value_cap (src/memory.rs:13-14): runtime-only, 0 = none.
        self.mem_value_cap = 0.0


class ModelWeights:
    def __init__(self, cfg: PSSAConfig):
        cfg.validate()
        self.cfg = cfg
        self.embed = np.zeros((cfg.d_vocab, cfg.d_latent), dtype=np.float32)
        self.unembed = np.zeros((cfg.d_vocab, cfg.d_latent), dtype=np.float32)
        self.blocks = [BlockWeights(cfg) for _ in range(cfg.depth)]
        self.rng_state: int | None = None

    # -- C view ------------------------------------------------------------
    def c_view(self):
        """Returns (pssa_hip_weights, keepalive).  Pointers alias the numpy arrays;
        bank counters are copied in, and `sync_from_c` copies them back."""
        blocks = (_abi.Block * self.cfg.depth)()
        for b, cb in zip(self.blocks, blocks):
            for name in _abi.BLOCK_FLOAT_FIELDS:
                arr = getattr(b, name)
                assert arr.dtype == np.float32 and arr.flags.c_contiguous, name
                setattr(cb, name, _abi.ptr(arr))
            cb.mem_last_seen = _abi.ptr(b.mem_last_seen, C.c_uint64)
            cb.mem_count = int(b.mem_count)
            cb.mem_write_head = int(b.mem_write_head)
            assert b.mem_hybrid_gate.dtype == np.float32 and b.mem_hybrid_age.dtype == np.uint64
            cb.mem_hybrid_gate = _abi.ptr(b.mem_hybrid_gate)
            cb.mem_hybrid_age = _abi.ptr(b.mem_hybrid_age, C.c_uint64)
            cb.mem_hybrid_enabled = 1 if b.mem_hybrid_enabled else 0
            cb.mem_hybrid_lam = float(b.mem_hybrid_lam)
            cb.mem_top_k = int(b.mem_top_k)
            cb.mem_value_cap = float(b.mem_value_cap)
        assert self.embed.flags.c_contiguous and self.unembed.flags.c_contiguous
        w = _abi.Weights(self.cfg.to_c(), _abi.ptr(self.embed), _abi.ptr(self.unembed), blocks)
        return w, blocks

    def sync_from_c(self, blocks) -> None:
        for b, cb in zip(self.blocks, blocks):
            b.mem_count = int(cb.mem_count)
            b.mem_write_head = int(cb.mem_write_head)

    def set_hybrid_read(self, enabled: bool, lam: float) -> None:
        """set_hybrid_read on every block (src/pssa.rs:2232-2243)."""
        if not (np.isfinite(lam) and 0.0 < lam <= 1.0):
            raise ValueError("hybrid decay lam must be in (0.0, 1.0]")
        for b in self.blocks:
            b.mem_hybrid_enabled = bool(enabled)
            b.mem_hybrid_lam = float(lam)

    def set_memory_top_k(self, top_k: int | None) -> None:
        """set_memory_top_k on every block (src/pssa.rs:2215-2226); None = full read."""
        if top_k is not None and top_k <= 0:
            raise ValueError("memory top-k must be positive")
        for b in self.blocks:
            b.mem_top_k = 0 if top_k is None else int(top_k)

    def set_value_cap(self, cap: float | None) -> None:
        """set_value_cap on every block (src/memory.rs:121-134): clamps every slot's
        value to norm <= cap and caps later writes; None removes the cap."""
        w, blocks = self.c_view()
        _abi.call(_abi.lib().pssa_hip_weights_set_value_cap, C.byref(w), 0.0 if cap is None else cap)
        for b, cb in zip(self.blocks, blocks):
            b.mem_value_cap = float(cb.mem_value_cap)

    # -- initialisation (libpssa_hip host code) -----------------------------
    @classmethod
    def init(cls, cfg: PSSAConfig, seed: int, mode: str = "reference") -> "ModelWeights":
        """mode 'reference': PSSALayerV2::new(cfg, seed) (src/pssa.rs:2019-2072);
        mode 'baseline': every matrix N(0, 0.02) from the same generator."""
        m = cls(cfg)
        w, blocks = m.c_view()
        state = C.c_uint64(0)
        code = _abi.INIT_REFERENCE if mode == "reference" else _abi.INIT_BASELINE
        if mode not in ("reference", "baseline"):
            raise ValueError(f"unknown init mode {mode!r}")
        _abi.call(_abi.lib().pssa_hip_weights_init, C.byref(w), seed, code, C.byref(state))
        m.sync_from_c(blocks)
        m.rng_state = int(state.value)
        return m

    def populate_banks(self, seed: int, count: int | None = None, max_radius: float = 0.9) -> None:
        """Fills every block's bank through insert() with keys/values uniform in
        direction and radius U[0, max_radius)."""
        count = self.cfg.mem_capacity if count is None else count
        w, blocks = self.c_view()
        _abi.call(_abi.lib().pssa_hip_weights_populate_banks, C.byref(w), seed, count, max_radius)
        self.sync_from_c(blocks)

    def state_width(self) -> int:
        return self.cfg.d_latent * self.cfg.d_state

    def to_bf16_values(self) -> "ModelWeights":
        """Copy whose weight matrices are rounded to bf16 (round to nearest even)
        and widened back to fp32: the parameters the bf16 path multiplies with."""
        out = ModelWeights(self.cfg)
        out.embed[:] = self.embed
        out.unembed[:] = bf16_round(self.unembed)
        # Everything the device stores in the weight dtype: projection matrices
        # and the bank values (operand of the soft-read readout product).
        mats = {"w_delta", "w_b", "w_c", "w_qx", "w_qh", "w_gate", "w_proj", "adapter_down",
                "mlp_w1", "mlp_w2", "mem_values"}
        for src, dst in zip(self.blocks, out.blocks):
            for name in BlockWeights.SHAPES:
                v = getattr(src, name)
                getattr(dst, name)[...] = bf16_round(v) if name in mats else v
            dst.mem_last_seen[:] = src.mem_last_seen
            dst.mem_count, dst.mem_write_head = src.mem_count, src.mem_write_head
            dst.mem_hybrid_gate[:] = src.mem_hybrid_gate
            dst.mem_hybrid_age[:] = src.mem_hybrid_age
            dst.mem_hybrid_enabled, dst.mem_hybrid_lam = src.mem_hybrid_enabled, src.mem_hybrid_lam
            dst.mem_top_k = src.mem_top_k
            dst.mem_value_cap = src.mem_value_cap
        return out


def bf16_round(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 (round to nearest even) -> fp32, as the device conversion."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32).reshape(a.shape)
