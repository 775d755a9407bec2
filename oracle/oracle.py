"""ctypes wrapper of oracle/liboracle.so -- TEST INFRASTRUCTURE ONLY.

The CPU restatement of the reference's scalar path (oracle/pssa_oracle.cpp).
Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
checker; never by the product path.  Model views are the product's own
`pssa_hip_weights` structs (identical layout to `oracle_model`).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "liboracle.so")

fp = C.POINTER(C.c_float)
u32p = C.POINTER(C.c_uint32)
vp = C.c_void_p

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-f", os.path.join("oracle", "Makefile"), "-B"], cwd=ROOT, check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = C.CDLL(LIB_PATH)
    sig = {
        "oracle_set_dot_avx2": ([C.c_int], None),
        "oracle_set_bf16_operands": ([C.c_int], None),
        "oracle_get_bf16_operands": ([], C.c_int),
        "oracle_bf16_round": ([C.c_float], C.c_float),
        "oracle_get_dot_avx2": ([], C.c_int),
        "oracle_rng_new": ([C.c_uint64], C.c_uint64),
        "oracle_set_loops": ([C.c_size_t], None),
        "oracle_get_loops": ([], C.c_size_t),
        "oracle_rng_next_u32": ([C.POINTER(C.c_uint64)], C.c_uint32),
        "oracle_dot": ([fp, fp, C.c_size_t], C.c_float),
        "oracle_softplus": ([C.c_float], C.c_float),
        "oracle_sigmoid": ([C.c_float], C.c_float),
        "oracle_init_reference": ([vp, C.c_uint64], C.c_uint64),
        "oracle_init_baseline": ([vp, C.c_uint64], C.c_uint64),
        "oracle_populate_banks": ([vp, C.c_uint64, C.c_uint64, C.c_float], None),
        "oracle_squared_norm": ([fp, C.c_size_t], C.c_float),
        "oracle_project": ([fp, fp, C.c_size_t], C.c_float),
        "oracle_poincare_distance": ([fp, C.c_float, fp, C.c_float, C.c_size_t], C.c_float),
        "oracle_rust_asinh": ([C.c_double], C.c_double),
        "oracle_retrieve": ([fp, fp, fp, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t, fp, C.c_float,
                             C.c_size_t, fp, fp], C.c_float),
        "oracle_retrieve_batch": ([fp, fp, fp, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t, fp, C.c_size_t,
                                   C.c_float, C.c_size_t, fp, fp, u32p, C.c_int], None),
        "oracle_bank_insert": ([vp, C.c_size_t, C.c_size_t, C.c_size_t, fp, fp], C.c_int64),
        "oracle_bank_insert_protected": ([vp, C.c_size_t, C.c_size_t, C.c_size_t, fp, fp, C.c_float,
                                          C.c_uint64], C.c_int64),
        "oracle_refractory_gain": ([C.c_uint64, C.c_float], C.c_float),
        "oracle_bank_insert_gated": ([vp, C.c_size_t, C.c_size_t, C.c_size_t, fp, fp, C.c_float], C.c_int64),
        "oracle_bank_insert_gated_protected": ([vp, C.c_size_t, C.c_size_t, C.c_size_t, fp, fp, C.c_float,
                                                C.c_float, C.c_uint64], C.c_int64),
        "oracle_bank_bump_hybrid_ages": ([vp, C.c_uint64], None),
        "oracle_bank_set_value_cap": ([vp, C.c_size_t, C.c_size_t, C.c_float], C.c_int),
        "oracle_clamp_value": ([fp, C.c_size_t, C.c_float], C.c_int),
        "oracle_retrieve_hybrid_batch": ([fp, fp, fp, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t, fp,
                                          C.c_size_t, C.c_float, C.c_size_t, fp, C.POINTER(C.c_uint64),
                                          C.c_float, fp, fp, u32p, fp, C.c_int], None),
        "oracle_gemm_xwt": ([fp, fp, C.c_size_t, C.c_size_t, C.c_size_t, fp], None),
        "oracle_ssm_forward": ([fp, fp, fp, fp, fp, fp, C.c_size_t, C.c_size_t, C.c_size_t, fp, fp, fp, fp], None),
        "oracle_forward_inference": ([vp, fp, C.c_uint32, fp], None),
        "oracle_prefill": ([vp, fp, u32p, C.c_size_t, fp], C.c_int),
        "oracle_prefill_lanes": ([vp, fp, u32p, C.c_size_t, C.c_size_t, fp, C.c_int], C.c_int),
        "oracle_train_chunk_forward": ([vp, fp, u32p, u32p, C.c_size_t, fp], C.c_float),
        "oracle_forward_features": ([vp, fp, C.c_uint32, fp], None),
        "oracle_greedy": ([fp, C.c_size_t], C.c_uint32),
        "oracle_sample_greedy": ([fp, C.c_size_t, u32p, C.c_size_t, C.c_float], C.c_int64),
        "oracle_sample": ([fp, C.c_size_t, u32p, C.c_size_t, C.c_float, C.c_float, C.c_float, C.c_size_t,
                           C.POINTER(C.c_uint64)], C.c_int64),

        "oracle_dense_scan": ([fp, fp, fp, C.c_size_t, C.c_size_t, C.c_size_t, fp, C.c_int], None),
        "oracle_hebbian_update": ([fp, fp, fp, fp, C.c_size_t, C.c_size_t], None),
        "oracle_forward_taps": ([vp, fp, C.c_uint32, fp, fp, fp, fp, fp], None),
        "oracle_decode": ([vp, fp, u32p, C.c_size_t, C.c_size_t, C.c_int, C.c_uint64, u32p, fp, fp, C.c_int],
                          C.c_int),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _lib = L
    return L


def ptr(a, ctype=C.c_float):
    if a is None:
        return None
    return a.ctypes.data_as(C.POINTER(ctype))


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class Dot:
    """Context manager selecting the reference's dot reduction tree."""

    def __init__(self, avx2: bool):
        self.avx2 = avx2

    def __enter__(self):
        self.prev = lib().oracle_get_dot_avx2()
        lib().oracle_set_dot_avx2(1 if self.avx2 else 0)

    def __exit__(self, *exc):
        lib().oracle_set_dot_avx2(self.prev)


def _operands(method):
    """Runs an OracleModel method in its operand mode (the process-wide
    oracle_set_bf16_operands switch), restoring the previous mode after."""
    import functools

    @functools.wraps(method)
    def run(self, *args, **kwargs):
        prev = lib().oracle_get_bf16_operands()
        prev_loops = lib().oracle_get_loops()
        lib().oracle_set_bf16_operands(1 if self.bf16_operands else 0)
        lib().oracle_set_loops(self.loops)
        try:
            return method(self, *args, **kwargs)
        finally:
            lib().oracle_set_bf16_operands(prev)
            lib().oracle_set_loops(prev_loops)

    return run


class OracleModel:
    """Runs the oracle on a product ModelWeights (aliasing its numpy arrays).
    bf16_operands restates the device's bf16 mode (every product's activation
    operand rounded to bf16, fp32 accumulation and state); pass weights
    already rounded (ModelWeights.to_bf16_values).  Off: the reference's
    arithmetic."""

    def __init__(self, weights, bf16_operands: bool = False):
        self.w = weights
        self.cfg = weights.cfg
        self.bf16_operands = bf16_operands
        self.view, self.keep = weights.c_view()
        self.ref = C.cast(C.pointer(self.view), vp)
        self.loops = 1

    def set_loops(self, loops: int) -> None:
        """set_loops (src/pssa.rs:2171-2184): every block runs `loops` passes
        per token, each with its own carry (states made by zero_state)."""
        if not 1 <= loops <= 32:
            raise ValueError("--loops must be between 1 and 32")
        self.loops = loops

    def sync(self):
        self.w.sync_from_c(self.keep)

    def zero_state(self, lanes: int | None = None) -> np.ndarray:
        """Carries [depth, d*s] ([depth, loops, d*s] with loops > 1), per lane."""
        ds = self.cfg.d_latent * self.cfg.d_state
        shape = (self.cfg.depth, ds) if self.loops == 1 else (self.cfg.depth, self.loops, ds)
        return np.zeros(shape if lanes is None else (lanes,) + shape, np.float32)

    def init_reference(self, seed: int) -> int:
        s = lib().oracle_init_reference(self.ref, seed)
        self.sync()
        return s

    def init_baseline(self, seed: int) -> int:
        s = lib().oracle_init_baseline(self.ref, seed)
        self.sync()
        return s

    def populate_banks(self, seed: int, count: int, max_radius: float = 0.9) -> None:
        lib().oracle_populate_banks(self.ref, seed, count, max_radius)
        self.sync()

    @_operands
    def forward_inference(self, state: np.ndarray, token: int, logits: bool = True):
        out = np.empty(self.cfg.d_vocab, np.float32) if logits else None
        lib().oracle_forward_inference(self.ref, ptr(state), token, ptr(out))
        return out

    @_operands
    def prefill(self, state: np.ndarray, ids, logits: bool = True):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.empty(self.cfg.d_vocab, np.float32) if logits else None
        rc = lib().oracle_prefill(self.ref, ptr(state), ptr(ids, C.c_uint32), ids.size, ptr(out))
        if rc:
            raise ValueError(f"oracle prefill rejected the ids ({rc})")
        return out

    @_operands
    def prefill_lanes(self, states: np.ndarray, ids: np.ndarray, threads: int = 1, logits: bool = True):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        lanes, n = ids.shape
        out = np.empty((lanes, self.cfg.d_vocab), np.float32) if logits else None
        rc = lib().oracle_prefill_lanes(self.ref, ptr(states), ptr(ids, C.c_uint32), lanes, n, ptr(out), threads)
        if rc:
            raise ValueError(f"oracle prefill rejected the ids ({rc})")
        return out

    @_operands
    def train_chunk_forward(self, state: np.ndarray, ids, targets):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        tg = np.ascontiguousarray(targets, dtype=np.uint32)
        logits = np.empty((ids.size, self.cfg.d_vocab), np.float32)
        loss = lib().oracle_train_chunk_forward(self.ref, ptr(state), ptr(ids, C.c_uint32),
                                                ptr(tg, C.c_uint32), ids.size, ptr(logits))
        return np.float32(loss), logits

    @_operands
    def forward_taps(self, state: np.ndarray, token: int):
        """forward_inference with per-block (q_pnc, z_final, adapter out, adapter act) and logits."""
        c = self.cfg
        q = np.empty((c.depth, c.d_mem_key), np.float32)
        z = np.empty((c.depth, c.d_latent), np.float32)
        a = np.empty((c.depth, c.d_latent), np.float32)
        act = np.empty((c.depth, c.adapter_rank), np.float32)
        lg = np.empty(c.d_vocab, np.float32)
        lib().oracle_forward_taps(self.ref, ptr(state), token, ptr(q), ptr(z), ptr(a), ptr(act), ptr(lg))
        return q, z, a, act, lg

    @_operands
    def decode(self, states: np.ndarray, first_ids, steps: int, plastic: bool = False, step_base: int = 0,
               threads: int = 1):
        """Greedy decode of every lane for `steps` steps (oracle_decode).  Returns
        (ids [steps, lanes], last logits [lanes, V], last surprise [lanes]).
        With plastic set the banks and adapter_up of the weights change in place."""
        ids = np.ascontiguousarray(first_ids, dtype=np.uint32).copy()
        lanes = ids.size
        out = np.empty((steps, lanes), np.uint32)
        lg = np.empty((lanes, self.cfg.d_vocab), np.float32)
        sp = np.empty(lanes, np.float32)
        rc = lib().oracle_decode(self.ref, ptr(states), ptr(ids, C.c_uint32), lanes, steps, 1 if plastic else 0,
                                 step_base, ptr(out, C.c_uint32), ptr(lg), ptr(sp), threads)
        if rc:
            raise ValueError(f"oracle decode rejected the ids ({rc})")
        self.sync()
        return out, lg, sp

    @_operands
    def features(self, state: np.ndarray, token: int) -> np.ndarray:
        out = np.empty(self.cfg.d_latent, np.float32)
        lib().oracle_forward_features(self.ref, ptr(state), token, ptr(out))
        return out


# ---- stage twins -------------------------------------------------------------

def gemm_xwt(x, w):
    x, w = f32(x), f32(w)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), np.float32)
    lib().oracle_gemm_xwt(ptr(x), ptr(w), m, n, k, ptr(y))
    return y


def ssm_forward(delta, b_proj, x_norm, rates, c_proj, initial, L, dm, ds):
    args = [f32(a).ravel() for a in (delta, b_proj, x_norm, rates, c_proj, initial)]
    w = dm * ds
    bar_a = np.empty(L * w, np.float32)
    bar_b = np.empty(L * w, np.float32)
    states = np.empty((L + 1) * w, np.float32)
    y = np.empty(L * dm, np.float32)
    lib().oracle_ssm_forward(*[ptr(a) for a in args], L, dm, ds, ptr(bar_a), ptr(bar_b), ptr(states), ptr(y))
    return bar_a, bar_b, states, y


def retrieve(keys, norm_sq, values, count, q_pnc, tau, top_k=0):
    keys, norm_sq, values, q_pnc = (f32(a) for a in (keys, norm_sq, values, q_pnc))
    capacity, dk = keys.shape
    dv = values.shape[1]
    out = np.empty(dv, np.float32)
    # The full read writes weights[..count] only (src/memory.rs:409-425).
    w = np.zeros(capacity, np.float32)
    mn = lib().oracle_retrieve(ptr(keys), ptr(norm_sq), ptr(values), count, capacity, dk, dv, ptr(q_pnc),
                               tau, top_k, ptr(out), ptr(w))
    return out, w, np.float32(mn)


def retrieve_batch(keys, norm_sq, values, count, q_pnc, tau, top_k=0, threads=1):
    keys, norm_sq, values, q_pnc = (f32(a) for a in (keys, norm_sq, values, q_pnc))
    capacity, dk = keys.shape
    dv = values.shape[1]
    n = q_pnc.shape[0]
    out = np.empty((n, dv), np.float32)
    mn = np.empty(n, np.float32)
    idx = np.empty((n, top_k), np.uint32) if top_k else None
    lib().oracle_retrieve_batch(ptr(keys), ptr(norm_sq), ptr(values), count, capacity, dk, dv, ptr(q_pnc), n,
                                tau, top_k, ptr(out), ptr(mn), ptr(idx, C.c_uint32), threads)
    return out, mn, idx


def retrieve_hybrid_batch(keys, norm_sq, values, count, q_pnc, tau, gate, age, lam, top_k=0, threads=1):
    """retrieve_hybrid_into per query against one bank state; returns
    (out_val [n, dv], min_dist [n], live idx [n, top_k] or None, weights [n, C])."""
    keys, norm_sq, values, q_pnc, gate = (f32(a) for a in (keys, norm_sq, values, q_pnc, gate))
    age = np.ascontiguousarray(age, dtype=np.uint64)
    capacity, dk = keys.shape
    dv = values.shape[1]
    n = q_pnc.shape[0]
    out = np.empty((n, dv), np.float32)
    mn = np.empty(n, np.float32)
    idx = np.empty((n, top_k), np.uint32) if top_k else None
    w = np.empty((n, capacity), np.float32)
    lib().oracle_retrieve_hybrid_batch(ptr(keys), ptr(norm_sq), ptr(values), count, capacity, dk, dv, ptr(q_pnc), n,
                                       tau, top_k, ptr(gate), ptr(age, C.c_uint64), lam, ptr(out), ptr(mn),
                                       ptr(idx, C.c_uint32), ptr(w), threads)
    return out, mn, idx, w


class Bank:
    """A single HyperbolicEpisodicBankV2 (src/memory.rs) held as numpy arrays,
    driven through the oracle's bank primitives (for the hybrid-read tests)."""

    def __init__(self, capacity: int, dk: int, dv: int):
        self.capacity, self.dk, self.dv = capacity, dk, dv
        self.keys = np.zeros((capacity, dk), np.float32)
        self.values = np.zeros((capacity, dv), np.float32)
        self.norm_sq = np.zeros(capacity, np.float32)
        self.confidence = np.ones(capacity, np.float32)
        self.last_seen = np.zeros(capacity, np.uint64)
        self.gate = np.ones(capacity, np.float32)
        self.age = np.zeros(capacity, np.uint64)
        self._blk = _OracleBlock()
        b = self._blk
        b.mem_keys, b.mem_values, b.mem_norm_sq = ptr(self.keys), ptr(self.values), ptr(self.norm_sq)
        b.mem_confidence, b.mem_last_seen = ptr(self.confidence), ptr(self.last_seen, C.c_uint64)
        b.mem_hybrid_gate, b.mem_hybrid_age = ptr(self.gate), ptr(self.age, C.c_uint64)
        b.mem_count = b.mem_write_head = 0

    @property
    def count(self) -> int:
        return int(self._blk.mem_count)

    def _ref(self):
        return C.cast(C.pointer(self._blk), vp)

    @staticmethod
    def _slot(idx) -> int:
        # -2: a capped bank refused a non-finite value (src/memory.rs:151-152).
        if idx == -2:
            raise ValueError("capped memory value must be finite")
        return int(idx)

    def insert(self, key, val) -> int:
        k, v = f32(key), f32(val)
        return self._slot(lib().oracle_bank_insert(self._ref(), self.capacity, self.dk, self.dv, ptr(k), ptr(v)))

    def insert_protected(self, key, val, surprise, step) -> int:
        k, v = f32(key), f32(val)
        return self._slot(lib().oracle_bank_insert_protected(self._ref(), self.capacity, self.dk, self.dv, ptr(k),
                                                             ptr(v), surprise, step))

    def set_value_cap(self, cap) -> None:
        """set_value_cap (src/memory.rs:121-134); None disables it."""
        if lib().oracle_bank_set_value_cap(self._ref(), self.capacity, self.dv, 0.0 if cap is None else cap) != 0:
            raise ValueError("capped memory value must be finite")

    @property
    def value_cap(self):
        cap = self._blk.mem_value_cap
        return None if cap == 0.0 else float(cap)

    def insert_gated(self, key, val, gate) -> int:
        k, v = f32(key), f32(val)
        return self._slot(lib().oracle_bank_insert_gated(self._ref(), self.capacity, self.dk, self.dv, ptr(k),
                                                         ptr(v), gate))

    def insert_gated_protected(self, key, val, gate, surprise, step) -> int:
        k, v = f32(key), f32(val)
        return self._slot(lib().oracle_bank_insert_gated_protected(self._ref(), self.capacity, self.dk, self.dv,
                                                                   ptr(k), ptr(v), gate, surprise, step))

    def bump_hybrid_ages(self, times: int = 1) -> None:
        lib().oracle_bank_bump_hybrid_ages(self._ref(), times)

    def retrieve_soft(self, q, tau):
        out, w, mn = retrieve(self.keys, self.norm_sq, self.values, self.count, q, tau)
        return out, w, mn

    def retrieve_hybrid(self, q, tau, lam, top_k=0):
        out, mn, idx, w = retrieve_hybrid_batch(self.keys, self.norm_sq, self.values, self.count,
                                                f32(q).reshape(1, -1), tau, self.gate, self.age, lam, top_k)
        return out[0], w[0], mn[0]


class _OracleBlock(C.Structure):
    """oracle_block: only the bank fields are used by the bank primitives."""
    _fields_ = [(n, fp) for n in (
        "norm_gamma", "norm_beta", "a_raw", "w_delta", "w_b", "w_c", "w_qx", "w_qh", "w_gate", "w_proj",
        "adapter_down", "adapter_up", "adapter_slow", "mlp_w1", "mlp_w2", "mem_keys", "mem_values",
        "mem_norm_sq", "mem_confidence")] + [
        ("mem_last_seen", C.POINTER(C.c_uint64)),
        ("mem_count", C.c_uint64),
        ("mem_write_head", C.c_uint64),
        ("mem_hybrid_gate", fp),
        ("mem_hybrid_age", C.POINTER(C.c_uint64)),
        ("mem_hybrid_enabled", C.c_uint32),
        ("mem_hybrid_lam", C.c_float),
        ("mem_top_k", C.c_uint64),
        ("mem_value_cap", C.c_float),
        ("_pad", C.c_uint32),
    ]


def project(q):
    q = f32(q)
    out = np.empty_like(q)
    r = lib().oracle_project(ptr(q), ptr(out), q.size)
    return out, np.float32(r)


def squared_norm(p):
    p = f32(p)
    return np.float32(lib().oracle_squared_norm(ptr(p), p.size))


def poincare_distance(u, v):
    u, v = f32(u), f32(v)
    return np.float32(lib().oracle_poincare_distance(ptr(u), squared_norm(u), ptr(v), squared_norm(v), u.size))


def dense_scan(a, b, h0=None, threads=1):
    a, b = f32(a), f32(b)
    batch, L, s = b.shape
    h0 = np.zeros((batch, s), np.float32) if h0 is None else f32(h0)
    h = np.empty((batch, L, s), np.float32)
    lib().oracle_dense_scan(ptr(a), ptr(b), ptr(h0), batch, L, s, ptr(h), threads)
    return h


def softplus(x) -> float:
    """softplus (src/linalg.rs:548-551) of one f32."""
    return float(lib().oracle_softplus(float(x)))


def greedy(logits) -> int:
    logits = f32(logits)
    return int(lib().oracle_greedy(ptr(logits), logits.size))


def clamp_value(value, cap) -> np.ndarray:
    """clamp_value (src/memory.rs:150-170) on a copy."""
    v = np.array(value, dtype=np.float32, copy=True)
    if lib().oracle_clamp_value(ptr(v), v.size, cap) != 0:
        raise ValueError("capped memory value must be finite")
    return v


def sample_greedy(logits, history, penalty: float = 1.0) -> int:
    """sample() at temperature 0 with the repetition penalty over the last 64
    history ids (the caller's copy of the logits is left alone); -1 for
    non-finite logits."""
    lg = np.array(logits, dtype=np.float32, copy=True)
    hist = np.ascontiguousarray(history, dtype=np.uint32)
    return int(lib().oracle_sample_greedy(ptr(lg), lg.size, ptr(hist, C.c_uint32), hist.size, penalty))


class Rng:
    """SimpleRng (src/linalg.rs:5-28) state, advanced by oracle calls."""

    def __init__(self, seed: int = 1337):
        self.state = C.c_uint64(lib().oracle_rng_new(seed))

    def next_u32(self) -> int:
        return int(lib().oracle_rng_next_u32(C.byref(self.state)))


def sample(logits, history, rng: Rng, temperature: float, top_p: float = 1.0, top_k: int = 1 << 30,
           penalty: float = 1.0) -> int:
    """sample() (src/inference.rs:102-178) with the repetition penalty over the
    last 64 history ids; at temperature > 0 one draw from `rng`.  -1 for
    non-finite logits, -2 for an invalid probability mass."""
    lg = np.array(logits, dtype=np.float32, copy=True)
    hist = np.ascontiguousarray(history, dtype=np.uint32)
    return int(lib().oracle_sample(ptr(lg), lg.size, ptr(hist, C.c_uint32), hist.size, penalty, temperature, top_p,
                                   top_k, C.byref(rng.state)))


def dot(a, b) -> np.float32:
    a, b = f32(a), f32(b)
    return np.float32(lib().oracle_dot(ptr(a), ptr(b), a.size))
