"""ctypes binding of include/pssa_hip.h (libpssa_hip.so, built in-tree).

Loading fails loudly when the library is missing: there is no CPU fallback
for the HIP path.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpssa_hip.so")

OK = 0
EINVAL = -1
ENODEV = -2
ENOMEM = -3
EDEVICE = -4
EUNSUPPORTED = -5

F32 = 0
BF16 = 1
INIT_REFERENCE = 0
INIT_BASELINE = 1
H2D, D2H, D2D = 0, 1, 2
DECODE_PLASTIC = 1
DECODE_GRAPH = 2

fp = C.POINTER(C.c_float)
u64p = C.POINTER(C.c_uint64)
u32p = C.POINTER(C.c_uint32)
sz = C.c_size_t
err_t = C.c_char_p


class Config(C.Structure):
    _fields_ = [
        ("depth", C.c_uint64),
        ("d_vocab", C.c_uint64),
        ("d_latent", C.c_uint64),
        ("d_state", C.c_uint64),
        ("d_mem_key", C.c_uint64),
        ("mem_capacity", C.c_uint64),
        ("adapter_rank", C.c_uint64),
        ("tau_mem", C.c_float),
        ("_pad", C.c_uint32),
    ]


BLOCK_FLOAT_FIELDS = [
    "norm_gamma", "norm_beta", "a_raw", "w_delta", "w_b", "w_c", "w_qx", "w_qh", "w_gate",
    "w_proj", "adapter_down", "adapter_up", "adapter_slow", "mlp_w1", "mlp_w2", "mem_keys",
    "mem_values", "mem_norm_sq", "mem_confidence",
]


class Block(C.Structure):
    _fields_ = [(n, fp) for n in BLOCK_FLOAT_FIELDS] + [
        ("mem_last_seen", u64p),
        ("mem_count", C.c_uint64),
        ("mem_write_head", C.c_uint64),
        ("mem_hybrid_gate", fp),
        ("mem_hybrid_age", u64p),
        ("mem_hybrid_enabled", C.c_uint32),
        ("mem_hybrid_lam", C.c_float),
        ("mem_top_k", C.c_uint64),
        ("mem_value_cap", C.c_float),
        ("_pad", C.c_uint32),
    ]


class Weights(C.Structure):
    _fields_ = [
        ("cfg", Config),
        ("embed", fp),
        ("unembed", fp),
        ("blocks", C.POINTER(Block)),
    ]


# pssa_hip_cancel_fn: int (*)(void* user)
CANCEL_FN = C.CFUNCTYPE(C.c_int, C.c_void_p)
CANCELLED = 1


class WeightKey(C.Structure):
    """pssa_hip_weight_key: (host address, element count) of a cached weight."""
    _fields_ = [("ptr", C.c_void_p), ("len", C.c_size_t)]


class Sequence(C.Structure):
    """pssa_hip_sequence (Sequence, src/sequence_batch.rs:21-28)."""
    _fields_ = [
        ("lane", C.c_uint64),
        ("inputs", C.POINTER(C.c_uint32)),
        ("targets", C.POINTER(C.c_uint32)),
        ("len", C.c_uint64),
        ("reset", C.c_uint32),
        ("_pad", C.c_uint32),
    ]


class HipError(RuntimeError):
    """A libpssa_hip call failed; `code` is the PSSA_HIP_* status."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code
        self.fatal = code == EDEVICE


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m pssa_amd.build` "
            "(the HIP path has no CPU fallback)")
    L = C.CDLL(LIB_PATH)
    vp = C.c_void_p
    pp = C.POINTER(vp)
    sig = {
        "pssa_hip_abi_version": ([], C.c_int),
        "pssa_hip_init": ([C.c_int, pp, err_t, sz], C.c_int),
        "pssa_hip_destroy": ([vp], None),
        "pssa_hip_device_name": ([vp, err_t, sz], C.c_int),
        "pssa_hip_is_fatal": ([C.c_int], C.c_int),
        "pssa_hip_synchronize": ([vp, err_t, sz], C.c_int),
        "pssa_hip_device_alloc": ([vp, sz, pp, err_t, sz], C.c_int),
        "pssa_hip_device_free": ([vp, vp], None),
        "pssa_hip_memcpy": ([vp, vp, vp, sz, C.c_int, err_t, sz], C.c_int),
        "pssa_hip_weights_init": ([C.POINTER(Weights), C.c_uint64, C.c_int, u64p, err_t, sz], C.c_int),
        "pssa_hip_weights_populate_banks": ([C.POINTER(Weights), C.c_uint64, C.c_uint64, C.c_float, err_t, sz], C.c_int),
        "pssa_hip_weights_set_value_cap": ([C.POINTER(Weights), C.c_float, err_t, sz], C.c_int),
        "pssa_hip_gemm_xwt": ([vp, fp, sz, vp, sz, C.c_int, sz, sz, sz, sz, fp, sz, err_t, sz], C.c_int),
        "pssa_hip_softplus_in_place": ([vp, fp, sz, err_t, sz], C.c_int),
        "pssa_hip_gemm_nn": ([vp, fp, sz, fp, sz, sz, sz, sz, fp, sz, err_t, sz], C.c_int),
        "pssa_hip_gemm_tn_accumulate": ([vp, fp, sz, fp, sz, sz, sz, sz, fp, sz, err_t, sz], C.c_int),
        "pssa_hip_invalidate_weights": ([vp], None),
        "pssa_hip_invalidate_weights_only": ([vp, C.POINTER(WeightKey), sz, err_t, sz], C.c_int),
        "pssa_hip_weight_cache_stats": ([vp, C.POINTER(sz), C.POINTER(sz), C.POINTER(sz)], C.c_int),
        "pssa_hip_ssm_forward": ([vp, fp, sz, fp, fp, sz, fp, sz, fp, sz, fp, fp, sz, fp, sz, sz, sz, sz,
                                  fp, fp, fp, fp, sz, fp, err_t, sz], C.c_int),
        "pssa_hip_ssm_forward_resident": ([vp, fp, sz, fp, fp, sz, fp, sz, fp, sz, fp, sz, fp, sz, sz, sz, sz,
                                           err_t, sz], C.c_int),
        "pssa_hip_memory_forward_after_ssm": ([vp] + [fp] * 8 + [sz] * 6 + [C.c_float, sz] + [fp] * 12
                                               + [err_t, sz], C.c_int),
        "pssa_hip_memory_forward": ([vp, fp, fp, fp, fp, fp, fp, fp, fp, fp, sz, sz, sz, sz, sz, sz,
                                     C.c_float, sz, fp, fp, fp, fp, fp, fp, fp, fp, err_t, sz], C.c_int),
        "pssa_hip_retrieve": ([vp, fp, sz, fp, fp, fp, sz, sz, sz, sz, C.c_float, sz, fp, fp, u32p, fp,
                               err_t, sz], C.c_int),
        "pssa_hip_retrieve_hybrid": ([vp, fp, sz, fp, fp, fp, sz, sz, sz, sz, C.c_float, sz, fp, u64p, C.c_float,
                                      fp, fp, u32p, fp, err_t, sz], C.c_int),
        "pssa_hip_model_set_hybrid_read": ([vp, C.c_int, C.c_float, err_t, sz], C.c_int),
        "pssa_hip_model_get_hybrid": ([vp, sz, fp, u64p, err_t, sz], C.c_int),
        "pssa_hip_retrieve_resident": ([vp, vp, sz, vp, vp, vp, sz, sz, sz, sz, C.c_float, sz, vp, vp, vp,
                                        err_t, sz], C.c_int),
        "pssa_hip_retrieve_resident_noalloc": ([vp, vp, sz, vp, vp, vp, sz, sz, sz, sz, C.c_float, sz, vp, vp, vp,
                                                err_t, sz], C.c_int),
        "pssa_hip_dense_scan": ([vp, fp, fp, fp, sz, sz, sz, fp, err_t, sz], C.c_int),
        "pssa_hip_dense_scan_resident": ([vp, vp, vp, vp, sz, sz, sz, vp, err_t, sz], C.c_int),
        "pssa_hip_dense_scan_reserve": ([vp, sz, sz, sz, err_t, sz], C.c_int),
        "pssa_hip_model_load": ([vp, C.POINTER(Weights), C.c_int, pp, err_t, sz], C.c_int),
        "pssa_hip_model_free": ([vp], None),
        "pssa_hip_lanes_create": ([vp, vp, sz, sz, pp, err_t, sz], C.c_int),
        "pssa_hip_lanes_free": ([vp], None),
        "pssa_hip_lanes_reset": ([vp, err_t, sz], C.c_int),
        "pssa_hip_lanes_get_carry": ([vp, fp, sz, err_t, sz], C.c_int),
        "pssa_hip_lanes_set_carry": ([vp, fp, sz, err_t, sz], C.c_int),
        "pssa_hip_prefill": ([vp, u32p, sz, sz, fp, sz, err_t, sz], C.c_int),
        "pssa_hip_forward_inference": ([vp, u32p, sz, fp, sz, err_t, sz], C.c_int),
        "pssa_hip_prefill_ragged": ([vp, u32p, u64p, sz, fp, sz, err_t, sz], C.c_int),
        "pssa_hip_prefill_cancellable": ([vp, u32p, sz, sz, sz, CANCEL_FN, vp, fp, sz, C.POINTER(sz), err_t, sz],
                                         C.c_int),
        "pssa_hip_lanes_set_repetition_penalty": ([vp, C.c_float, err_t, sz], C.c_int),
        "pssa_hip_lanes_get_taps": ([vp, sz, sz, fp, fp, fp, fp, err_t, sz], C.c_int),
        "pssa_hip_lanes_set_sampling": ([vp, C.c_float, C.c_float, sz, C.c_uint64, err_t, sz], C.c_int),
        "pssa_hip_lanes_set_loops": ([vp, sz, err_t, sz], C.c_int),
        "pssa_hip_model_set_memory_top_k": ([vp, sz, err_t, sz], C.c_int),
        "pssa_hip_model_set_value_cap": ([vp, C.c_float, err_t, sz], C.c_int),
        "pssa_hip_batch_forward": ([vp, C.POINTER(Sequence), sz, fp, fp, sz, fp, sz, err_t, sz], C.c_int),
        "pssa_hip_lanes_stage_ids": ([vp, u32p, sz, sz, err_t, sz], C.c_int),
        "pssa_hip_lanes_prefill_staged": ([vp, err_t, sz], C.c_int),
        "pssa_hip_lanes_read_logits": ([vp, fp, sz, err_t, sz], C.c_int),
        "pssa_hip_lanes_stage_times": ([vp, C.c_int, C.POINTER(C.c_char_p), fp, sz], C.c_int),
        "pssa_hip_decode": ([vp, u32p, sz, sz, C.c_int, u32p, sz, fp, sz, err_t, sz], C.c_int),
        "pssa_hip_model_get_plastic": ([vp, sz, fp, fp, fp, fp, fp, u64p, u64p, u64p, u64p, err_t, sz], C.c_int),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _lib = L
    return L


def exported_symbols() -> list[str]:
    """Entry points declared in include/pssa_hip.h (parsed from the header)."""
    import re

    hdr = os.path.join(os.path.dirname(HERE), "include", "pssa_hip.h")
    text = open(hdr).read()
    return sorted(set(re.findall(r"\b(pssa_hip_[a-z0-9_]+)\s*\(", text)))


def call(fn, *args) -> None:
    """Calls an entry point whose last two arguments are (err, err_len)."""
    buf = C.create_string_buffer(1024)
    rc = fn(*args, buf, C.sizeof(buf))
    if rc != OK:
        raise HipError(rc, buf.value.decode(errors="replace"))


def ptr(a, ctype=C.c_float):
    """ctypes pointer to a numpy array's data (None passes NULL)."""
    if a is None:
        return None
    return a.ctypes.data_as(C.POINTER(ctype))
