"""The allocation-free retrieval entry point (pssa_hip_retrieve_resident_noalloc)
against the allocating one (pssa_hip_retrieve_resident) through the C ABI:
two calls in a row, the second smaller, each bit-identical in indices,
minimum distances and readout.  The second call runs after the first has
left its contents in the shared static scratch."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print("[no-alloc]", *a, flush=True)
    sys.stdout.flush()


def ball(rng, n, dim, max_r=0.9):
    v = rng.standard_normal((n, dim))
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    return (v * rng.uniform(0.0, max_r, (n, 1))).astype(np.float32)


def squared_norms(keys):
    # Any valid bank norm (both entry points read the same input): f64 sums as f32.
    return (keys.astype(np.float64) ** 2).sum(axis=1).astype(np.float32)


def run_both(hip, q, keys, nsq, vals, capacity, count, k):
    n_q, dk = q.shape
    dv = vals.shape[1]
    bufs = [hip.upload(a) for a in (q, keys, nsq, vals)]
    outs = {}
    for name in ("resident", "noalloc"):
        out, mn, idx = hip.empty((n_q, dv), np.float32), hip.empty((n_q,), np.float32), hip.empty((n_q, k), np.uint32)
        fn = hip.retrieve_resident if name == "resident" else hip.retrieve_resident_noalloc
        fn(bufs[0].ptr, n_q, bufs[1].ptr, bufs[2].ptr, bufs[3].ptr, capacity, count, dk, dv, 0.1, k,
           out.ptr, mn.ptr, idx.ptr)
        hip.synchronize()
        outs[name] = (out.to_host(), mn.to_host(), idx.to_host())
        for b in (out, mn, idx):
            b.close()
    for b in bufs:
        b.close()
    return outs["resident"], outs["noalloc"]


def test_noalloc_retrieval_matches_the_allocating_entry_point_twice(hip):
    rng = np.random.default_rng(7)
    # Call 1: several 8192-query passes through the static scratch (config 4 widths).
    C1, dk1, n1, k1 = 512, 768, 20000, 8
    keys, vals = ball(rng, C1, dk1), ball(rng, C1, dk1)
    q = ball(rng, n1, dk1)
    nsq = squared_norms(keys)
    say(f"call 1: {n1} queries, d_key {dk1}, {C1} slots, top-{k1}")
    (r_out, r_min, r_idx), (g_out, g_min, g_idx) = run_both(hip, q, keys, nsq, vals, C1, C1, k1)
    np.testing.assert_array_equal(g_idx, r_idx)
    np.testing.assert_array_equal(g_min.view(np.uint32), r_min.view(np.uint32))
    np.testing.assert_array_equal(g_out.view(np.uint32), r_out.view(np.uint32))
    assert np.all(r_idx < C1)

    # Call 2: smaller queries, keys and bank; the scratch still holds call 1's rows.
    C2, cnt2, dk2, dv2, n2, k2 = 400, 300, 256, 96, 5000, 5
    keys2 = np.zeros((C2, dk2), np.float32)
    vals2 = np.zeros((C2, dv2), np.float32)
    keys2[:cnt2], vals2[:cnt2] = ball(rng, cnt2, dk2), ball(rng, cnt2, dv2)
    q2 = ball(rng, n2, dk2)
    nsq2 = np.zeros(C2, np.float32)
    nsq2[:cnt2] = squared_norms(keys2[:cnt2])
    say(f"call 2: {n2} queries, d_key {dk2}, {cnt2} of {C2} slots, top-{k2}")
    (r_out, r_min, r_idx), (g_out, g_min, g_idx) = run_both(hip, q2, keys2, nsq2, vals2, C2, cnt2, k2)
    np.testing.assert_array_equal(g_idx, r_idx)
    np.testing.assert_array_equal(g_min.view(np.uint32), r_min.view(np.uint32))
    np.testing.assert_array_equal(g_out.view(np.uint32), r_out.view(np.uint32))
    assert np.all(r_idx < cnt2)


def test_noalloc_retrieval_validates_before_running(hip):
    import ctypes as C

    from pssa_amd import _abi

    lib = _abi.lib()
    buf = C.create_string_buffer(256)
    rc = lib.pssa_hip_retrieve_resident_noalloc(hip.handle, None, 4, None, None, None, 8, 8, 16, 16, C.c_float(0.1),
                                                2, None, None, None, buf, 256)
    assert rc == _abi.EINVAL and b"null buffer" in buf.value


def _free_device_bytes():
    import ctypes as C

    hip_rt = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(0), C.c_size_t(0)
    assert hip_rt.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def test_noalloc_retrieval_allocates_nothing_on_a_fresh_context():
    """On a context of its own, the allocation-free entry point runs first:
    device memory in use does not move across a config-4-sized call (a
    smaller call before it loads the kernels), while the allocating entry
    point's first call of the same shape grows the context's scratch by
    tens of MB, which shows the measurement sees such a growth."""
    from pssa_amd import HipDevice

    rng = np.random.default_rng(11)
    C1, dk, n, k = 512, 768, 20000, 8
    keys, vals = ball(rng, C1, dk), ball(rng, C1, dk)
    q = ball(rng, n, dk)
    nsq = squared_norms(keys)
    dev = HipDevice(0)
    bufs = [dev.upload(a) for a in (q, keys, nsq, vals)]
    outs = [dev.empty((n, dk), np.float32), dev.empty((n,), np.float32), dev.empty((n, k), np.uint32)]

    def call(fn, n_q):
        fn(bufs[0].ptr, n_q, bufs[1].ptr, bufs[2].ptr, bufs[3].ptr, C1, C1, dk, dk, 0.1, k,
           outs[0].ptr, outs[1].ptr, outs[2].ptr)
        dev.synchronize()

    say("fresh context: warm-up call, 64 queries")
    call(dev.retrieve_resident_noalloc, 64)
    free0 = _free_device_bytes()
    say(f"fresh context: {n} queries through the allocation-free entry point")
    call(dev.retrieve_resident_noalloc, n)
    free1 = _free_device_bytes()
    idx = outs[2].to_host()
    say(f"fresh context: the allocating entry point, same shape")
    call(dev.retrieve_resident, n)
    free2 = _free_device_bytes()
    np.testing.assert_array_equal(outs[2].to_host(), idx)
    for b in bufs + outs:
        b.close()
    dev.close()
    say(f"device bytes in use: +{free0 - free1} (allocation-free), +{free1 - free2} (allocating)")
    assert abs(free0 - free1) < (1 << 20)
    assert free1 - free2 >= (16 << 20)
