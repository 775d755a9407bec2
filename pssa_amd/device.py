"""Host-side mirror of the reference's device surface, backed by libpssa_hip.

`HipDevice` plays the role of `GpuDispatch::Hip` next to the reference's
`GpuDispatch::{Wgpu, Cuda}` (src/backend.rs:1025-1446): same method names,
argument meaning and error behaviour (shape errors raise before anything runs;
device failures are fatal and never fall back to the CPU).

`PSSALayer` carries the model-level inference entry points of PSSALayerV2
(`forward_inference`, `prefill_inference`, `reset_recurrent_state`,
src/pssa.rs:2245-2442) for a batch of independent lanes
(SequenceBatch, src/sequence_batch.rs:21-78).
"""
from __future__ import annotations

import ctypes as C
import weakref
from dataclasses import dataclass

import numpy as np

from . import _abi
from .weights import ModelWeights


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class HipDevice:
    """Device context (CudaContext peer, src/cuda.rs:158-192)."""

    def __init__(self, device: int = 0):
        self._lib = _abi.lib()
        h = C.c_void_p()
        _abi.call(self._lib.pssa_hip_init, device, C.byref(h))
        self.handle = h
        # Objects holding native state tied to this context; closed first.
        self._children = weakref.WeakSet()

    def close(self) -> None:
        if self.handle:
            for child in list(self._children):
                child.close()
            self._lib.pssa_hip_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass

    def backend_label(self) -> str:
        buf = C.create_string_buffer(256)
        self._lib.pssa_hip_device_name(self.handle, buf, 256)
        return buf.value.decode()

    def synchronize(self) -> None:
        _abi.call(self._lib.pssa_hip_synchronize, self.handle)

    # -- device buffers for the resident entry points ---------------------------
    def upload(self, array: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(array)
        buf = DeviceBuffer(self, a.nbytes, a.shape, a.dtype)
        _abi.call(self._lib.pssa_hip_memcpy, self.handle, C.c_void_p(buf.ptr), a.ctypes.data_as(C.c_void_p),
                  a.nbytes, _abi.H2D)
        return buf

    def empty(self, shape, dtype) -> "DeviceBuffer":
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        return DeviceBuffer(self, n, tuple(shape), np.dtype(dtype))

    # -- GpuDispatch::try_dispatch_gemm_into (src/backend.rs:1049-1085) -------
    def try_dispatch_gemm(self, x, w, m: int, n: int, k: int, batch: int = 1,
                          w_dtype: str = "f32", resident: bool = False) -> np.ndarray:
        """y = x w^T.  The library keeps a device copy of `w` keyed by its host
        address and length.  With `resident` the copy stays current for later
        calls with the same array, as a model parameter would (the caller
        invalidates it after changing the data in place); otherwise it is
        marked stale after the call, since a temporary array's address can be
        reused by other data."""
        x = _f32(x).ravel()
        if w_dtype == "f32":
            wb = _f32(w).ravel()
            code, wlen = _abi.F32, wb.size
        elif w_dtype == "bf16":
            wb = np.ascontiguousarray(w, dtype=np.uint16).ravel()
            code, wlen = _abi.BF16, wb.size
        else:
            raise ValueError("w_dtype must be 'f32' or 'bf16'")
        if resident and not np.shares_memory(wb, np.asarray(w)):
            raise ValueError("a resident weight must be a contiguous array of the weight dtype")
        y = np.empty(batch * m * n, dtype=np.float32)
        try:
            _abi.call(self._lib.pssa_hip_gemm_xwt, self.handle, _abi.ptr(x), x.size,
                      wb.ctypes.data_as(C.c_void_p), wlen, code, m, n, k, batch, _abi.ptr(y), y.size)
        finally:
            if not resident:
                self.invalidate_weights_only([wb])
        return y

    # -- GpuDispatch::gemm_nn_into / gemm_tn_accumulate_into
    #    (src/backend.rs:1152-1184) ------------------------------------------
    def gemm_nn(self, a, b, m: int, k: int, n: int) -> np.ndarray:
        """out[m, n] = a[m, k] b[k, n]."""
        a, b = _f32(a).ravel(), _f32(b).ravel()
        out = np.empty(m * n, np.float32)
        _abi.call(self._lib.pssa_hip_gemm_nn, self.handle, _abi.ptr(a), a.size, _abi.ptr(b), b.size, m, k, n,
                  _abi.ptr(out), out.size)
        return out

    def gemm_tn_accumulate(self, a, b, m: int, k: int, n: int, out: np.ndarray) -> None:
        """out[k, n] += a[m, k]^T b[m, n] (out: contiguous float32, updated in place)."""
        a, b = _f32(a).ravel(), _f32(b).ravel()
        if out.dtype != np.float32 or not out.flags.c_contiguous:
            raise ValueError("out must be a contiguous float32 array")
        _abi.call(self._lib.pssa_hip_gemm_tn_accumulate, self.handle, _abi.ptr(a), a.size, _abi.ptr(b), b.size,
                  m, k, n, _abi.ptr(out), out.size)

    # -- weight residency (GpuDispatch::invalidate_weights[_only],
    #    src/backend.rs:1113-1134) ------------------------------------------
    def invalidate_weights(self) -> None:
        self._lib.pssa_hip_invalidate_weights(self.handle)

    def invalidate_weights_only(self, arrays) -> None:
        """Marks the cached copies of these host arrays stale (keyed by data
        address and element count)."""
        keys = (_abi.WeightKey * max(len(arrays), 1))()
        for i, a in enumerate(arrays):
            keys[i].ptr, keys[i].len = a.ctypes.data, a.size
        _abi.call(self._lib.pssa_hip_invalidate_weights_only, self.handle, keys, len(arrays))

    def weight_cache_stats(self) -> dict:
        e, c, b = C.c_size_t(), C.c_size_t(), C.c_size_t()
        self._lib.pssa_hip_weight_cache_stats(self.handle, C.byref(e), C.byref(c), C.byref(b))
        return {"entries": e.value, "current": c.value, "bytes": b.value}

    def softplus_in_place(self, values: np.ndarray) -> None:
        assert values.dtype == np.float32 and values.flags.c_contiguous
        _abi.call(self._lib.pssa_hip_softplus_in_place, self.handle, _abi.ptr(values), values.size)

    # -- GpuDispatch::ssm_forward (src/backend.rs:1213-1244) -------------------
    def ssm_forward(self, delta, b_proj, x_norm, rates, c_proj, initial, seq_len: int, d_m: int,
                    d_s: int, materialize: bool = True):
        """Returns (bar_a, bar_b, states, y_ssm, final_state); the first three are
        None when materialize is False."""
        delta, b_proj, x_norm = _f32(delta).ravel(), _f32(b_proj).ravel(), _f32(x_norm).ravel()
        rates, c_proj, initial = _f32(rates).ravel(), _f32(c_proj).ravel(), _f32(initial).ravel()
        w = d_m * d_s
        y = np.empty(seq_len * d_m, np.float32)
        fin = np.empty(w, np.float32)
        bar_a = np.empty(seq_len * w, np.float32) if materialize else None
        bar_b = np.empty(seq_len * w, np.float32) if materialize else None
        states = np.empty((seq_len + 1) * w, np.float32) if materialize else None
        _abi.call(self._lib.pssa_hip_ssm_forward, self.handle, _abi.ptr(delta), delta.size, None,
                  _abi.ptr(b_proj), b_proj.size, _abi.ptr(x_norm), x_norm.size, _abi.ptr(rates),
                  rates.size, None, _abi.ptr(c_proj), c_proj.size, _abi.ptr(initial), initial.size,
                  seq_len, d_m, d_s, _abi.ptr(bar_a), _abi.ptr(bar_b), _abi.ptr(states), _abi.ptr(y),
                  y.size, _abi.ptr(fin))
        return bar_a, bar_b, states, y, fin

    # -- GpuDispatch::memory_forward (src/backend.rs:1345-1385) ----------------
    def memory_forward(self, x_norm, y_ssm, w_qx, w_qh, w_gate, w_proj, keys, norm_sq, values,
                       seq_len: int, d_m: int, d_k: int, d_val: int, capacity: int, count: int,
                       tau: float, top_k: int = 0) -> dict:
        args = [_f32(a).ravel() for a in (x_norm, y_ssm, w_qx, w_qh, w_gate, w_proj, keys, norm_sq, values)]
        out = {
            "q_euc": np.empty(seq_len * d_k, np.float32),
            "q_pnc": np.empty(seq_len * d_k, np.float32),
            "q_norm": np.empty(seq_len, np.float32),
            "weights": np.empty(seq_len * capacity, np.float32),
            "m_val": np.empty(seq_len * d_val, np.float32),
            "g_mem": np.empty(seq_len * d_val, np.float32),
            "m_proj": np.empty(seq_len * d_val, np.float32),
            "m_inj": np.empty(seq_len * d_val, np.float32),
        }
        _abi.call(self._lib.pssa_hip_memory_forward, self.handle, *[_abi.ptr(a) for a in args],
                  seq_len, d_m, d_k, d_val, capacity, count, tau, top_k,
                  *[_abi.ptr(out[k]) for k in ("q_euc", "q_pnc", "q_norm", "weights", "m_val",
                                              "g_mem", "m_proj", "m_inj")])
        return out

    # -- GpuDispatch::ssm_forward_resident + memory_forward_after_ssm
    #    (src/backend.rs:1186-1211, 1246-1289) --------------------------------
    def ssm_forward_resident(self, delta, b_proj, x_norm, rates, c_proj, initial, seq_len: int, d_m: int,
                             d_s: int) -> None:
        args = [_f32(a).ravel() for a in (delta, b_proj, x_norm, rates, c_proj, initial)]
        delta, b_proj, x_norm, rates, c_proj, initial = args
        _abi.call(self._lib.pssa_hip_ssm_forward_resident, self.handle, _abi.ptr(delta), delta.size, None,
                  _abi.ptr(b_proj), b_proj.size, _abi.ptr(x_norm), x_norm.size, _abi.ptr(rates), rates.size,
                  _abi.ptr(c_proj), c_proj.size, _abi.ptr(initial), initial.size, seq_len, d_m, d_s)

    def memory_forward_after_ssm(self, x_norm, w_qx, w_qh, w_gate, w_proj, keys, norm_sq, values,
                                 seq_len: int, d_m: int, d_k: int, d_val: int, capacity: int, count: int,
                                 tau: float, d_s: int, top_k: int = 0) -> dict:
        """memory_forward on the resident tape; also returns that tape
        (bar_a, bar_b, states, y_ssm)."""
        args = [_f32(a).ravel() for a in (x_norm, w_qx, w_qh, w_gate, w_proj, keys, norm_sq, values)]
        w = d_m * d_s
        out = {
            "bar_a": np.empty(seq_len * w, np.float32),
            "bar_b": np.empty(seq_len * w, np.float32),
            "states": np.empty((seq_len + 1) * w, np.float32),
            "y_ssm": np.empty(seq_len * d_m, np.float32),
            "q_euc": np.empty(seq_len * d_k, np.float32),
            "q_pnc": np.empty(seq_len * d_k, np.float32),
            "q_norm": np.empty(seq_len, np.float32),
            "weights": np.empty(seq_len * capacity, np.float32),
            "m_val": np.empty(seq_len * d_val, np.float32),
            "g_mem": np.empty(seq_len * d_val, np.float32),
            "m_proj": np.empty(seq_len * d_val, np.float32),
            "m_inj": np.empty(seq_len * d_val, np.float32),
        }
        _abi.call(self._lib.pssa_hip_memory_forward_after_ssm, self.handle, *[_abi.ptr(a) for a in args],
                  seq_len, d_m, d_k, d_val, capacity, count, tau, top_k, *[_abi.ptr(v) for v in out.values()])
        return out

    # -- batched retrieve_soft_into (src/memory.rs:344-426) --------------------
    def retrieve(self, q_pnc, keys, norm_sq, values, count: int, tau: float, top_k: int = 0,
                 want_weights: bool = False):
        q_pnc, keys, norm_sq, values = (_f32(a) for a in (q_pnc, keys, norm_sq, values))
        n_q, d_key = q_pnc.shape
        capacity, d_val = values.shape
        out_val = np.empty((n_q, d_val), np.float32)
        out_min = np.empty(n_q, np.float32)
        out_idx = np.empty((n_q, top_k), np.uint32) if top_k > 0 else None
        out_w = np.empty((n_q, capacity), np.float32) if want_weights else None
        _abi.call(self._lib.pssa_hip_retrieve, self.handle, _abi.ptr(q_pnc), n_q, _abi.ptr(keys),
                  _abi.ptr(norm_sq), _abi.ptr(values), capacity, count, d_key, d_val, tau, top_k,
                  _abi.ptr(out_val), _abi.ptr(out_min),
                  None if out_idx is None else _abi.ptr(out_idx, C.c_uint32), _abi.ptr(out_w))
        return out_val, out_min, out_idx, out_w

    # -- retrieve_hybrid_into (src/memory.rs:568-660) --------------------------
    def retrieve_hybrid(self, q_pnc, keys, norm_sq, values, count: int, tau: float, gate, age, lam: float,
                        top_k: int = 0, want_weights: bool = False):
        """Hybrid read of every query against one bank state; gate/age [count]
        are the bank's hybrid_gate / hybrid_age.  Returns as `retrieve`."""
        q_pnc, keys, norm_sq, values = (_f32(a) for a in (q_pnc, keys, norm_sq, values))
        gate = _f32(np.asarray(gate, np.float32)[:count])
        age = np.ascontiguousarray(np.asarray(age)[:count], dtype=np.uint64)
        n_q, d_key = q_pnc.shape
        capacity, d_val = values.shape
        out_val = np.empty((n_q, d_val), np.float32)
        out_min = np.empty(n_q, np.float32)
        out_idx = np.empty((n_q, top_k), np.uint32) if top_k > 0 else None
        out_w = np.empty((n_q, capacity), np.float32) if want_weights else None
        _abi.call(self._lib.pssa_hip_retrieve_hybrid, self.handle, _abi.ptr(q_pnc), n_q, _abi.ptr(keys),
                  _abi.ptr(norm_sq), _abi.ptr(values), capacity, count, d_key, d_val, tau, top_k,
                  _abi.ptr(gate), _abi.ptr(age, C.c_uint64), lam, _abi.ptr(out_val), _abi.ptr(out_min),
                  None if out_idx is None else _abi.ptr(out_idx, C.c_uint32), _abi.ptr(out_w))
        return out_val, out_min, out_idx, out_w

    def retrieve_resident(self, q_ptr: int, n_q: int, keys_ptr: int, norm_sq_ptr: int, values_ptr: int,
                          capacity: int, count: int, d_key: int, d_val: int, tau: float, top_k: int,
                          out_val_ptr: int, out_min_ptr: int | None = None, out_idx_ptr: int | None = None) -> None:
        """retrieve on device buffers (asynchronous on the context stream)."""
        vp = C.c_void_p
        _abi.call(self._lib.pssa_hip_retrieve_resident, self.handle, vp(q_ptr), n_q, vp(keys_ptr), vp(norm_sq_ptr),
                  vp(values_ptr), capacity, count, d_key, d_val, tau, top_k, vp(out_val_ptr),
                  vp(out_min_ptr) if out_min_ptr else None, vp(out_idx_ptr) if out_idx_ptr else None)

    def retrieve_resident_noalloc(self, q_ptr: int, n_q: int, keys_ptr: int, norm_sq_ptr: int, values_ptr: int,
                                  capacity: int, count: int, d_key: int, d_val: int, tau: float, top_k: int,
                                  out_val_ptr: int, out_min_ptr: int | None = None,
                                  out_idx_ptr: int | None = None) -> None:
        """retrieve_resident with no device allocation: the exact top-k path's
        scratch is the device's static array (shared by every call on the GPU;
        overlapping calls race)."""
        vp = C.c_void_p
        _abi.call(self._lib.pssa_hip_retrieve_resident_noalloc, self.handle, vp(q_ptr), n_q, vp(keys_ptr),
                  vp(norm_sq_ptr), vp(values_ptr), capacity, count, d_key, d_val, tau, top_k, vp(out_val_ptr),
                  vp(out_min_ptr) if out_min_ptr else None, vp(out_idx_ptr) if out_idx_ptr else None)

    def dense_scan(self, a, b, h0=None):
        a, b = _f32(a), _f32(b)
        batch, L, s = b.shape
        assert a.shape == (batch, L, s, s)
        h = np.empty((batch, L, s), np.float32)
        h0p = None if h0 is None else _abi.ptr(_f32(h0))
        _abi.call(self._lib.pssa_hip_dense_scan, self.handle, _abi.ptr(a), _abi.ptr(b), h0p, batch, L, s,
                  _abi.ptr(h))
        return h

    def dense_scan_resident(self, a_ptr: int, b_ptr: int, h0_ptr: int | None, batch: int, L: int, s: int,
                            h_ptr: int) -> None:
        _abi.call(self._lib.pssa_hip_dense_scan_resident, self.handle, C.c_void_p(a_ptr), C.c_void_p(b_ptr),
                  C.c_void_p(h0_ptr) if h0_ptr else None, batch, L, s, C.c_void_p(h_ptr))

    def dense_scan_reserve(self, batch: int, L: int, s: int) -> None:
        """Sizes the context's scratch for dense scans up to this shape, so that
        dense_scan_resident then runs without allocating."""
        _abi.call(self._lib.pssa_hip_dense_scan_reserve, self.handle, batch, L, s)


class DeviceBuffer:
    """A device allocation made through the C ABI (freed on close/GC)."""

    def __init__(self, device: HipDevice, nbytes: int, shape, dtype):
        self.device = device
        self.shape, self.dtype, self.nbytes = tuple(shape), np.dtype(dtype), nbytes
        p = C.c_void_p()
        _abi.call(device._lib.pssa_hip_device_alloc, device.handle, max(nbytes, 1), C.byref(p))
        self.ptr = p.value
        device._children.add(self)

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        _abi.call(self.device._lib.pssa_hip_memcpy, self.device.handle, out.ctypes.data_as(C.c_void_p),
                  C.c_void_p(self.ptr), self.nbytes, _abi.D2H)
        return out

    def write(self, array: np.ndarray, offset_bytes: int = 0) -> None:
        a = np.ascontiguousarray(array)
        assert offset_bytes + a.nbytes <= self.nbytes
        _abi.call(self.device._lib.pssa_hip_memcpy, self.device.handle, C.c_void_p(self.ptr + offset_bytes),
                  a.ctypes.data_as(C.c_void_p), a.nbytes, _abi.H2D)

    def close(self) -> None:
        if self.ptr and self.device.handle:
            self.device._lib.pssa_hip_device_free(self.device.handle, C.c_void_p(self.ptr))
        self.ptr = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass


@dataclass
class Sequence:
    """One training sequence of a batch (Sequence, src/sequence_batch.rs:21-28)."""
    lane: int
    inputs: object
    targets: object
    reset: bool = False


class PSSALayer:
    """Device-resident PSSA model with `lanes` independent recurrent carries."""

    def __init__(self, device: HipDevice, weights: ModelWeights, lanes: int = 1,
                 max_tokens: int | None = None, weight_dtype: str = "f32"):
        self.device = device
        self.cfg = weights.cfg
        self.lanes = lanes
        self.max_tokens = max_tokens or lanes
        lib = device._lib
        self._lib = lib
        w, keep = weights.c_view()
        m = C.c_void_p()
        code = _abi.F32 if weight_dtype == "f32" else _abi.BF16
        _abi.call(lib.pssa_hip_model_load, device.handle, C.byref(w), code, C.byref(m))
        self.model = m
        del keep
        ln = C.c_void_p()
        try:
            _abi.call(lib.pssa_hip_lanes_create, device.handle, m, lanes, self.max_tokens, C.byref(ln))
        except Exception:
            lib.pssa_hip_model_free(m)
            raise
        self.handle = ln
        device._children.add(self)

    def close(self) -> None:
        if getattr(self, "handle", None):
            self._lib.pssa_hip_lanes_free(self.handle)
            self.handle = None
        if getattr(self, "model", None):
            self._lib.pssa_hip_model_free(self.model)
            self.model = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def reset_recurrent_state(self) -> None:
        _abi.call(self._lib.pssa_hip_lanes_reset, self.handle)

    def carry_shape(self):
        """[lanes, depth, d*s], or [lanes, depth, loops, d*s] with loops > 1."""
        ds = self.cfg.d_latent * self.cfg.d_state
        loops = getattr(self, "loops", 1)
        return (self.lanes, self.cfg.depth, ds) if loops == 1 else (self.lanes, self.cfg.depth, loops, ds)

    def set_loops(self, loops: int) -> None:
        """set_loops (src/pssa.rs:2171-2184): `loops` passes per block and
        token, each with its own carry (loop 0 keeps the current one)."""
        _abi.call(self._lib.pssa_hip_lanes_set_loops, self.handle, loops)
        self.loops = loops

    def get_carry(self) -> np.ndarray:
        out = np.empty(self.carry_shape(), np.float32)
        _abi.call(self._lib.pssa_hip_lanes_get_carry, self.handle, _abi.ptr(out), out.size)
        return out

    def set_carry(self, carry) -> None:
        carry = _f32(carry)
        assert carry.shape == self.carry_shape()
        _abi.call(self._lib.pssa_hip_lanes_set_carry, self.handle, _abi.ptr(carry), carry.size)

    def prefill_inference(self, token_ids, want_logits: bool = True):
        """token_ids [n_lanes, T] (or [T] for one lane).  Returns the last
        token's logits [n_lanes, V] (None when want_logits is False)."""
        ids = np.ascontiguousarray(np.atleast_2d(np.asarray(token_ids)), dtype=np.uint32)
        n_lanes, T = ids.shape
        logits = np.empty((n_lanes, self.cfg.d_vocab), np.float32) if want_logits else None
        _abi.call(self._lib.pssa_hip_prefill, self.handle, _abi.ptr(ids, C.c_uint32), n_lanes, T,
                  _abi.ptr(logits), 0 if logits is None else logits.size)
        self._staged = (n_lanes, T)
        return logits

    def prefill_cancellable(self, token_ids, cancelled, chunk: int = 1, want_logits: bool = True):
        """prefill_inference with the reference's cancellation callback
        (src/pssa.rs:2399-2418): `cancelled()` is asked before every `chunk`
        tokens.  Returns (finished, processed tokens per lane, logits or None);
        on cancellation the logits are not produced."""
        ids = np.ascontiguousarray(np.atleast_2d(np.asarray(token_ids)), dtype=np.uint32)
        n_lanes, T = ids.shape
        logits = np.empty((n_lanes, self.cfg.d_vocab), np.float32) if want_logits else None
        cb = _abi.CANCEL_FN(lambda _user: 1 if cancelled() else 0)
        done = C.c_size_t(0)
        buf = C.create_string_buffer(1024)
        rc = self._lib.pssa_hip_prefill_cancellable(
            self.handle, _abi.ptr(ids, C.c_uint32), n_lanes, T, chunk, cb, None, _abi.ptr(logits),
            0 if logits is None else logits.size, C.byref(done), buf, C.sizeof(buf))
        if rc == _abi.CANCELLED:
            return False, int(done.value), None
        if rc != _abi.OK:
            raise _abi.HipError(rc, buf.value.decode(errors="replace"))
        self._staged = (n_lanes, T)
        return True, int(done.value), logits

    def prefill_ragged(self, sequences, want_logits: bool = True):
        """prefill_inference with its own prompt length per lane: sequences[i]
        (a 1-D id array, at least one id) runs on lane i.  Returns the last
        logits of every lane [n_lanes, V]."""
        seqs = [np.ascontiguousarray(np.asarray(q).ravel(), dtype=np.uint32) for q in sequences]
        ids = np.ascontiguousarray(np.concatenate(seqs) if seqs else np.zeros(0, np.uint32), dtype=np.uint32)
        lens = np.array([q.size for q in seqs], np.uint64)
        logits = np.empty((len(seqs), self.cfg.d_vocab), np.float32) if want_logits else None
        _abi.call(self._lib.pssa_hip_prefill_ragged, self.handle, _abi.ptr(ids, C.c_uint32),
                  _abi.ptr(lens, C.c_uint64), len(seqs), _abi.ptr(logits), 0 if logits is None else logits.size)
        self._staged = (len(seqs), 0)
        return logits

    def forward_inference(self, ids):
        """One token per lane; returns logits [n_lanes, V]."""
        ids = np.ascontiguousarray(np.atleast_1d(np.asarray(ids)), dtype=np.uint32)
        logits = np.empty((ids.size, self.cfg.d_vocab), np.float32)
        _abi.call(self._lib.pssa_hip_forward_inference, self.handle, _abi.ptr(ids, C.c_uint32), ids.size,
                  _abi.ptr(logits), logits.size)
        return logits

    # -- SequenceBatch::forward (src/sequence_batch.rs:233-384) -----------------
    def batch_forward(self, sequences, want_token_losses: bool = False, want_logits: bool = False):
        """Training forward of a batch of sequences, each on its own lane.
        `sequences` holds `Sequence`s (or (lane, inputs, targets[, reset])
        tuples).  Returns the token-mean loss, plus the per-token losses
        [tokens] and logits [tokens, V] in packed order when asked."""
        seqs = [s if isinstance(s, Sequence) else Sequence(*s) for s in sequences]
        keep = []
        arr = (_abi.Sequence * max(len(seqs), 1))()
        tokens = 0
        for i, s in enumerate(seqs):
            ids = np.ascontiguousarray(np.asarray(s.inputs).ravel(), dtype=np.uint32)
            tg = np.ascontiguousarray(np.asarray(s.targets).ravel(), dtype=np.uint32)
            if ids.size != tg.size:
                raise ValueError("each sequence needs matching input/target lengths")
            keep += [ids, tg]
            arr[i].lane, arr[i].len, arr[i].reset = s.lane, ids.size, 1 if s.reset else 0
            arr[i].inputs, arr[i].targets = _abi.ptr(ids, C.c_uint32), _abi.ptr(tg, C.c_uint32)
            tokens += ids.size
        loss = C.c_float()
        tl = np.empty(tokens, np.float32) if want_token_losses else None
        lg = np.empty((tokens, self.cfg.d_vocab), np.float32) if want_logits else None
        _abi.call(self._lib.pssa_hip_batch_forward, self.handle, arr, len(seqs), C.byref(loss),
                  _abi.ptr(tl), 0 if tl is None else tl.size, _abi.ptr(lg), 0 if lg is None else lg.size)
        del keep
        out = [float(loss.value)]
        if want_token_losses:
            out.append(tl)
        if want_logits:
            out.append(lg)
        return out[0] if len(out) == 1 else tuple(out)

    # -- greedy decode (forward_inference + sample, src/pssa.rs:2387-2391,
    #    src/inference.rs:123-127) ------------------------------------------
    def decode(self, steps: int, first_ids=None, n_lanes: int | None = None, plastic: bool = False,
               graph: bool = False, want_logits: bool = False):
        """Generates `steps` greedy tokens on lanes 0..n_lanes-1.  first_ids=None
        continues the last prefill as the reference's generate loop does
        (src/inference.rs:367-379): row 0 is the greedy choice from the
        prefill's logits and each later row costs a forward step of the row
        before it.  Given first_ids, every row is the choice after a forward
        step of the previous token (first_ids for row 0); a continuation of a
        decode passes its last row.  Returns ids [steps, n_lanes] (and the
        logits of the last choice [n_lanes, V] when want_logits)."""
        if first_ids is not None:
            first = np.ascontiguousarray(np.atleast_1d(np.asarray(first_ids)), dtype=np.uint32)
            n_lanes = first.size
            fp_ = _abi.ptr(first, C.c_uint32)
        else:
            if n_lanes is None:
                n_lanes = self._staged[0] if getattr(self, "_staged", None) else self.lanes
            fp_ = None
        out = np.empty((steps, n_lanes), np.uint32)
        logits = np.empty((n_lanes, self.cfg.d_vocab), np.float32) if want_logits else None
        flags = (_abi.DECODE_PLASTIC if plastic else 0) | (_abi.DECODE_GRAPH if graph else 0)
        _abi.call(self._lib.pssa_hip_decode, self.handle, fp_, n_lanes, steps, flags,
                  _abi.ptr(out, C.c_uint32), out.size, _abi.ptr(logits), 0 if logits is None else logits.size)
        self._staged = None
        return (out, logits) if want_logits else out

    def get_taps(self, layer: int, n_lanes: int) -> dict:
        """Block `layer`'s taps of the last plastic decode step over n_lanes lanes:
        q_pnc [n, k], z_final [n, d], adapter output [n, d], activations [n, r]."""
        c = self.cfg
        out = {"q_pnc": np.empty((n_lanes, c.d_mem_key), np.float32),
               "z_final": np.empty((n_lanes, c.d_latent), np.float32),
               "ad_out": np.empty((n_lanes, c.d_latent), np.float32),
               "act": np.empty((n_lanes, c.adapter_rank), np.float32)}
        _abi.call(self._lib.pssa_hip_lanes_get_taps, self.handle, layer, n_lanes, _abi.ptr(out["q_pnc"]),
                  _abi.ptr(out["z_final"]), _abi.ptr(out["ad_out"]), _abi.ptr(out["act"]))
        return out

    def set_repetition_penalty(self, penalty: float) -> None:
        """InferenceConfig::repetition_penalty for the greedy choice (1 = off)."""
        _abi.call(self._lib.pssa_hip_lanes_set_repetition_penalty, self.handle, penalty)

    def set_sampling(self, temperature: float, top_p: float = 0.85, top_k: int = 24, seed: int = 1337) -> None:
        """InferenceConfig::{temperature, top_p, top_k} for the lanes' choice
        (sample(), src/inference.rs:128-178); temperature 0 is greedy.  Every
        lane's generator restarts from SimpleRng::new(seed)."""
        _abi.call(self._lib.pssa_hip_lanes_set_sampling, self.handle, temperature, top_p, top_k, seed)

    def get_plastic(self, layer: int) -> dict:
        """One block's adapter fast weights and bank state as held on the device."""
        c = self.cfg
        d, k, C_, r = c.d_latent, c.d_mem_key, c.mem_capacity, c.adapter_rank
        out = {
            "adapter_up": np.empty((d, r), np.float32),
            "mem_keys": np.empty((C_, k), np.float32),
            "mem_values": np.empty((C_, d), np.float32),
            "mem_norm_sq": np.empty(C_, np.float32),
            "mem_confidence": np.empty(C_, np.float32),
            "mem_last_seen": np.empty(C_, np.uint64),
        }
        cnt, head, step = C.c_uint64(), C.c_uint64(), C.c_uint64()
        _abi.call(self._lib.pssa_hip_model_get_plastic, self.model, layer, _abi.ptr(out["adapter_up"]),
                  _abi.ptr(out["mem_keys"]), _abi.ptr(out["mem_values"]), _abi.ptr(out["mem_norm_sq"]),
                  _abi.ptr(out["mem_confidence"]), _abi.ptr(out["mem_last_seen"], C.c_uint64),
                  C.byref(cnt), C.byref(head), C.byref(step))
        out.update(mem_count=int(cnt.value), mem_write_head=int(head.value), step=int(step.value))
        return out

    def set_hybrid_read(self, enabled: bool, lam: float) -> None:
        """set_hybrid_read on every block (src/pssa.rs:2232-2243)."""
        _abi.call(self._lib.pssa_hip_model_set_hybrid_read, self.model, 1 if enabled else 0, lam)

    def set_memory_top_k(self, top_k: int | None) -> None:
        """set_memory_top_k on every block (src/pssa.rs:2215-2226); None = full read."""
        if top_k is not None and top_k <= 0:
            raise ValueError("memory top-k must be positive")
        _abi.call(self._lib.pssa_hip_model_set_memory_top_k, self.model, 0 if top_k is None else top_k)

    def set_value_cap(self, cap: float | None) -> None:
        """set_value_cap on every block of the loaded model (src/memory.rs:121-134)."""
        _abi.call(self._lib.pssa_hip_model_set_value_cap, self.model, 0.0 if cap is None else cap)

    def get_hybrid(self, layer: int):
        """One block's (hybrid_gate [C], hybrid_age [C]) as held on the device."""
        C_ = self.cfg.mem_capacity
        gate = np.empty(C_, np.float32)
        age = np.empty(C_, np.uint64)
        _abi.call(self._lib.pssa_hip_model_get_hybrid, self.model, layer, _abi.ptr(gate), _abi.ptr(age, C.c_uint64))
        return gate, age

    # -- device-resident measurement path ------------------------------------
    def stage_ids(self, token_ids) -> None:
        ids = np.ascontiguousarray(np.atleast_2d(np.asarray(token_ids)), dtype=np.uint32)
        _abi.call(self._lib.pssa_hip_lanes_stage_ids, self.handle, _abi.ptr(ids, C.c_uint32), *ids.shape)
        self._staged = ids.shape

    def prefill_staged(self) -> None:
        _abi.call(self._lib.pssa_hip_lanes_prefill_staged, self.handle)

    def read_logits(self) -> np.ndarray:
        n_lanes = self._staged[0]
        out = np.empty((n_lanes, self.cfg.d_vocab), np.float32)
        _abi.call(self._lib.pssa_hip_lanes_read_logits, self.handle, _abi.ptr(out), out.size)
        return out

    def set_stage_timing(self, enable: bool) -> None:
        self._lib.pssa_hip_lanes_stage_times(self.handle, 1 if enable else 0, None, None, 0)

    def stage_times(self) -> dict:
        names = (C.c_char_p * 32)()
        ms = (C.c_float * 32)()
        n = self._lib.pssa_hip_lanes_stage_times(self.handle, -1, names, ms, 32)
        return {names[i].decode(): float(ms[i]) for i in range(n)}
