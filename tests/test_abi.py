"""The C ABI library loads on any host and exports exactly what
include/pssa_hip.h declares; validation errors are reported before any device
work, with the reference's messages where it has them (src/backend.rs:11-39)."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

from pssa_amd import _abi


def test_library_exports_every_declared_symbol():
    lib = _abi.lib()
    declared = _abi.exported_symbols()
    assert len(declared) >= 25
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", _abi.LIB_PATH], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T pssa_hip_" in line}
    assert exported == set(declared), exported ^ set(declared)
    assert lib.pssa_hip_abi_version() == 1


def test_library_links_no_oracle_and_no_torch():
    out = subprocess.run(["ldd", _abi.LIB_PATH], capture_output=True, text=True).stdout
    # Library names only (the hex load addresses can contain any substring).
    names = [line.split()[0] for line in out.splitlines() if line.strip()]
    assert not any(("oracle" in n or "torch" in n or n.startswith("libc10")) for n in names), names
    assert any("amdhip64" in n for n in names), names


def test_init_rejects_a_missing_device():
    lib = _abi.lib()
    h = C.c_void_p()
    buf = C.create_string_buffer(256)
    rc = lib.pssa_hip_init(999, C.byref(h), buf, 256)
    assert rc == _abi.ENODEV and not h.value
    assert buf.value


def test_fatal_classification():
    lib = _abi.lib()
    assert lib.pssa_hip_is_fatal(_abi.EDEVICE) == 1
    for code in (_abi.OK, _abi.EINVAL, _abi.ENODEV, _abi.ENOMEM, _abi.EUNSUPPORTED):
        assert lib.pssa_hip_is_fatal(code) == 0


def test_validation_happens_before_device_work():
    lib = _abi.lib()
    x = np.ones(6, np.float32)
    y = np.full(4, 7.0, np.float32)
    buf = C.create_string_buffer(256)
    rc = lib.pssa_hip_gemm_xwt(None, _abi.ptr(x), 6, x.ctypes.data_as(C.c_void_p), 6, _abi.F32, 2, 2, 3, 1,
                               _abi.ptr(y), 4, buf, 256)
    assert rc == _abi.EINVAL
    assert np.all(y == 7.0)  # outputs untouched
    rc = lib.pssa_hip_ssm_forward(None, None, 0, None, None, 0, None, 0, None, 0, None, None, 0, None, 0,
                                  0, 0, 0, None, None, None, None, 0, None, buf, 256)
    assert rc == _abi.EINVAL


def test_weights_init_validates_and_fills():
    from pssa_amd import ModelWeights, PSSAConfig

    cfg = PSSAConfig(depth=3, d_vocab=9, d_latent=8, d_state=4, d_mem_key=2, mem_capacity=5)
    w = ModelWeights.init(cfg, 0, "reference")
    # Seed 0 is remapped by SimpleRng::new (src/linalg.rs:9).
    assert w.rng_state != 0
    assert np.all(np.abs(w.blocks[2].w_delta) <= np.sqrt(6 / 16))
    assert not w.blocks[1].mlp_w2.any()
    w.populate_banks(3)
    for b in w.blocks:
        assert b.mem_count == 5 and b.mem_write_head == 0
        assert np.all(b.mem_norm_sq < 0.81) and np.all(b.mem_norm_sq >= 0)
    with pytest.raises(ValueError):
        ModelWeights.init(cfg, 0, "nope")
    # Inserting past capacity advances the ring head (src/memory.rs:280-287).
    w.populate_banks(4, count=2)
    assert w.blocks[0].mem_count == 5 and w.blocks[0].mem_write_head == 2


def test_parameter_count_matches_reference_formula():
    from pssa_amd import PSSAConfig

    # 2 V d + depth (7 d^2 + (3 s + 2 k + 34) d) (docs/stacked-depth.md:33-34).
    for cfg in (PSSAConfig(depth=12, d_vocab=16384, d_latent=768, d_state=256, d_mem_key=32),
                PSSAConfig(depth=2, d_vocab=8192, d_latent=128, d_state=64, d_mem_key=32)):
        d, s, k = cfg.d_latent, cfg.d_state, cfg.d_mem_key
        assert cfg.parameter_count() == 2 * cfg.d_vocab * d + cfg.depth * (7 * d * d + (3 * s + 2 * k + 34) * d)


def test_header_is_plain_c():
    hdr = os.path.join(os.path.dirname(_abi.HERE), "include", "pssa_hip.h")
    out = subprocess.run(["gcc", "-fsyntax-only", "-x", "c", "-std=c99", "-Wall", "-Werror", hdr],
                         capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
