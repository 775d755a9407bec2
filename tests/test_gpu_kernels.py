"""Kernel-level parity on the GPU, through the C ABI, against the CPU oracle.

Gates: fp32 max normwise relative error 1e-4, bf16 weights 2e-2; retrieved
slot indices bit-exact.  Small shapes run first."""
import numpy as np
import pytest

from conftest import assert_parity, elem_rel_err, rel_err
from oracle import oracle as O
from pssa_amd import bf16_round
from pssa_amd._abi import HipError
from test_oracle_closed_forms import F32_MIN_SUB, bank, cuda_ssm_fixture

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


# ------------------------------------------------------------------- GEMM
@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (7, 5, 3), (33, 17, 9), (128, 128, 64), (130, 257, 768),
                                   (300, 2096, 768)])
def test_gemm_f32_matches_oracle(hip, m, n, k):
    say("gemm f32", m, n, k)
    rng = np.random.default_rng(m * 1000 + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    y = hip.try_dispatch_gemm(x, w, m, n, k).reshape(m, n)
    assert rel_err(y, O.gemm_xwt(x, w)) < 1e-5


@pytest.mark.parametrize("n", [768, 1024])
def test_gemm_f32_few_rows_equal_tiled_rows_bitwise(hip, n):
    """A product of few token rows runs one wave per 32 x 32 (or 64 x 32)
    tile; a wide one the 128 x 128 tiles.  Both follow the same MFMA order
    over K, so the first rows of a 16384-row product equal the same rows
    computed alone, bit for bit (the prefill / decode identity of fp32
    models rests on it)."""
    say("gemm f32 few rows == tiled", n)
    rng = np.random.default_rng(n)
    m, k = 16384, 768
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    big = hip.try_dispatch_gemm(x, w, m, n, k).reshape(m, n)
    for rows in (1, 37, 64):
        few = hip.try_dispatch_gemm(np.ascontiguousarray(x[:rows]), w, rows, n, k).reshape(rows, n)
        np.testing.assert_array_equal(few.view(np.uint32), big[:rows].view(np.uint32))
    assert rel_err(big[:64], O.gemm_xwt(x[:64], w)) < 1e-5


@pytest.mark.parametrize("n,k", [(768, 768), (1056, 768), (1000, 128), (736, 800), (1024, 800)])
def test_gemm_bf16_few_rows_equal_tiled_rows_bitwise(hip, n, k):
    """bf16 weights: few token rows run one wave per 32 x 32 tile, with
    64-wide K slabs through an LDS ring when K % 64 == 0 (768) and through a
    register ring otherwise (800: a partial last slab); many rows run the
    128 x 128 direct-to-LDS tiles.  All feed the same fragments to the same
    MFMA sequence over K, so the rows agree bit for bit (the prefill / decode
    identity of bf16 models rests on it)."""
    say("gemm bf16 few rows == tiled", n, k)
    rng = np.random.default_rng(n + k)
    m = 16384
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = bf16_round((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    wbits = (w.view(np.uint32) >> 16).astype(np.uint16)
    big = hip.try_dispatch_gemm(x, wbits, m, n, k, w_dtype="bf16").reshape(m, n)
    for rows in (1, 37, 64, 256):
        few = hip.try_dispatch_gemm(np.ascontiguousarray(x[:rows]), wbits, rows, n, k, w_dtype="bf16").reshape(rows, n)
        np.testing.assert_array_equal(few.view(np.uint32), big[:rows].view(np.uint32))
    exact = bf16_round(x[:64]).astype(np.float64) @ w.astype(np.float64).T
    assert rel_err(big[:64], exact) < 1e-5


@pytest.mark.parametrize("m,n", [(16461, 1000), (16384 + 5, 2096), (4200, 772)])
def test_gemm_bf16_tiled_partial_tiles_bitwise(hip, m, n):
    """The tiled kernel's epilogue stages each 32 x 32 tile through LDS;
    tiles cut off by M or N load clamped rows and columns and store only
    what is in range.  Rows at both ends of a product whose last row and
    column tiles are partial (772 columns: a last tile of one 4-column
    chunk) equal the few-row kernel's bit for bit."""
    say("gemm bf16 partial tiles", m, n)
    k = 768
    rng = np.random.default_rng(m + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = bf16_round((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    wbits = (w.view(np.uint32) >> 16).astype(np.uint16)
    big = hip.try_dispatch_gemm(x, wbits, m, n, k, w_dtype="bf16").reshape(m, n)
    for r0, rows in ((0, 37), (m - 37, 37), (m - 128 - 3, 64)):
        few = hip.try_dispatch_gemm(np.ascontiguousarray(x[r0:r0 + rows]), wbits, rows, n, k,
                                    w_dtype="bf16").reshape(rows, n)
        np.testing.assert_array_equal(few.view(np.uint32), big[r0:r0 + rows].view(np.uint32))
    exact = bf16_round(x[-64:]).astype(np.float64) @ w.astype(np.float64).T
    assert rel_err(big[-64:], exact) < 1e-5


@pytest.mark.parametrize("m,n,k,batch", [(5, 9, 8, 1), (64, 130, 776, 2), (257, 96, 768, 1), (31, 3, 20, 3)])
def test_gemm_bf16_weights(hip, m, n, k, batch):
    say("gemm bf16", m, n, k, batch)
    rng = np.random.default_rng(n)
    x = rng.standard_normal((batch * m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    wb = bf16_round(w)
    wbits = (wb.view(np.uint32) >> 16).astype(np.uint16)
    y = hip.try_dispatch_gemm(x, wbits, m, n, k, batch, w_dtype="bf16").reshape(batch * m, n)
    # Exact products of bf16 operands, fp32 accumulation.
    exact = bf16_round(x).astype(np.float64) @ wb.astype(np.float64).T
    assert rel_err(y, exact) < 1e-5
    assert rel_err(y, O.gemm_xwt(x, w)) < 2e-2


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (7, 5, 3), (130, 64, 257), (300, 768, 96)])
def test_gemm_nn_and_tn_accumulate(hip, m, k, n):
    """gemm_nn_into and gemm_tn_accumulate_into (src/backend.rs:1152-1184)
    against the oracle's GEMM on transposed operands; failed validation
    leaves the output untouched."""
    say("gemm nn / tn", m, k, n)
    rng = np.random.default_rng(m + 7 * k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = (rng.standard_normal((k, n)) * 0.1).astype(np.float32)
    got = hip.gemm_nn(a, b, m, k, n).reshape(m, n)
    ref = O.gemm_xwt(a, np.ascontiguousarray(b.T))
    assert rel_err(got, ref) < 1e-4
    bm = (rng.standard_normal((m, n)) * 0.1).astype(np.float32)
    out = rng.standard_normal((k, n)).astype(np.float32)
    base = out.copy()
    hip.gemm_tn_accumulate(a, bm, m, k, n, out)
    ref = base + O.gemm_xwt(np.ascontiguousarray(a.T), np.ascontiguousarray(bm.T))
    assert rel_err(out, ref) < 1e-4
    keep = out.copy()
    with pytest.raises(HipError, match="operand lengths"):
        hip.gemm_tn_accumulate(a[:, :-1] if k > 1 else a[:0], bm, m, k, n, out)
    np.testing.assert_array_equal(out, keep)


def test_gemm_weight_cache_follows_invalidation(hip):
    """try_dispatch_gemm_into keeps the weight on the device keyed by host
    address and length (CudaContext::weight_buffer, src/cuda.rs:198-227): a
    resident weight changed in place keeps its device copy until it is
    invalidated (src/cuda.rs:229-252); a temporary weight is never reused."""
    say("gemm weight cache")
    rng = np.random.default_rng(5)
    m, n, k = 70, 96, 64
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    w_old = w.copy()
    s0 = hip.weight_cache_stats()
    y1 = hip.try_dispatch_gemm(x, w, m, n, k, resident=True)
    s1 = hip.weight_cache_stats()
    assert s1["entries"] == s0["entries"] + 1 and s1["current"] == s0["current"] + 1
    w *= 2.0  # in place: same address and length
    np.testing.assert_array_equal(hip.try_dispatch_gemm(x, w, m, n, k, resident=True), y1)
    hip.invalidate_weights_only([np.zeros(5, np.float32)])  # another key: nothing changes
    np.testing.assert_array_equal(hip.try_dispatch_gemm(x, w, m, n, k, resident=True), y1)
    hip.invalidate_weights_only([w])
    np.testing.assert_array_equal(hip.try_dispatch_gemm(x, w, m, n, k, resident=True), 2.0 * y1)
    w[:] = w_old
    hip.invalidate_weights()
    assert hip.weight_cache_stats()["current"] == 0
    np.testing.assert_array_equal(hip.try_dispatch_gemm(x, w, m, n, k, resident=True), y1)
    for scale in (4.0, 0.5):  # temporaries (exact scalings), possibly at one recycled address
        np.testing.assert_array_equal(hip.try_dispatch_gemm(x, w * np.float32(scale), m, n, k),
                                      np.float32(scale) * y1)
    assert hip.weight_cache_stats()["current"] == 1


def test_gemm_shape_errors_leave_output_untouched(hip):
    from pssa_amd._abi import HipError

    with pytest.raises(HipError, match="GEMM operand lengths"):
        hip.try_dispatch_gemm(np.ones(5, np.float32), np.ones(6, np.float32), 2, 3, 2)


# -------------------------------------------------------------------- SSM
def test_ssm_reference_fixture(hip):
    """tests/backend_cuda.rs:97-160 (L=7, d=3, s=2) with every tape output."""
    say("ssm fixture 7x3x2")
    L, dm, ds, delta, b, x, rates, c, init = cuda_ssm_fixture()
    bar_a, bar_b, states, y, fin = hip.ssm_forward(delta, b, x, rates, c, init, L, dm, ds)
    ra, rb, rs, ry = O.ssm_forward(delta, b, x, rates, c, init, L, dm, ds)
    assert rel_err(bar_a, ra) < 1e-6
    assert rel_err(bar_b, rb) < 1e-6
    assert rel_err(states, rs) < 1e-5
    assert rel_err(y, ry) < 1e-5
    np.testing.assert_array_equal(states[: dm * ds], init)
    assert rel_err(fin, rs[L * dm * ds:]) < 1e-5


def test_ssm_len64_stride4096_covers_all_channels(hip):
    """tests/backend_cuda.rs:262-340: patterned L=64, d=256, s=16."""
    say("ssm patterned 64x256x16")
    L, dm, ds = 64, 256, 16
    i = np.arange(L * dm)
    delta = np.float32(0.01 + (i % 19) * 0.001)
    b = np.float32((np.arange(L * ds) % 13) * 0.002 - 0.01)
    x = np.float32((i % 23) * 0.01 - 0.1)
    rates = np.float32(-0.01 - (np.arange(dm * ds) % 7) * 0.001)
    c = np.float32((np.arange(L * ds) % 11) * 0.003 - 0.01)
    init = np.float32((np.arange(dm * ds) % 17) * 0.001 - 0.008)
    bar_a, bar_b, states, y, fin = hip.ssm_forward(delta, b, x, rates, c, init, L, dm, ds)
    ra, rb, rs, ry = O.ssm_forward(delta, b, x, rates, c, init, L, dm, ds)
    assert rel_err(y, ry) < 1e-5 and rel_err(states, rs) < 1e-5
    assert states[0] == init[0]
    stride = dm * ds
    assert abs(states[L * stride + stride - 1] - rs[L * stride + stride - 1]) < 1e-6


@pytest.mark.parametrize("L,dm,ds", [(1, 1, 1), (17, 5, 3), (300, 100, 256), (33, 130, 64), (40, 64, 300)])
def test_ssm_random_shapes(hip, L, dm, ds):
    say("ssm random", L, dm, ds)
    rng = np.random.default_rng(L + dm + ds)
    delta = np.float32(np.log1p(np.exp(rng.standard_normal(L * dm))))
    b = rng.standard_normal(L * ds).astype(np.float32) * 0.3
    x = rng.standard_normal(L * dm).astype(np.float32)
    rates = -np.float32(np.log1p(np.exp(rng.standard_normal(dm * ds))))
    c = rng.standard_normal(L * ds).astype(np.float32) * 0.3
    init = rng.standard_normal(dm * ds).astype(np.float32) * 0.1
    _, _, _, y, fin = hip.ssm_forward(delta, b, x, rates, c, init, L, dm, ds, materialize=False)
    ra, rb, rs, ry = O.ssm_forward(delta, b, x, rates, c, init, L, dm, ds)
    assert rel_err(y, ry) < 1e-5
    assert rel_err(fin, rs[L * dm * ds:]) < 1e-5


def test_ssm_softplus_and_rate_tails(hip):
    """tests/numeric_recurrence.rs:48-137: tiny delta from the softplus tail and a
    huge delta against a tiny rate keep the state finite and exact to ~1e-6."""
    say("ssm tails")
    for raw in (-17.0, -20.0):
        delta = np.float32([np.log1p(np.exp(np.float64(raw)))] * 2)
        _, _, _, y, fin = hip.ssm_forward(delta, np.float32([1.0, 1.0]), np.float32([1.0, 1.0]),
                                          np.float32([-0.5]), np.float32([1.0, 1.0]), np.float32([0.0]), 2, 1, 1,
                                          materialize=False)
        assert fin[0] > 0 and abs(fin[0] / (2 * float(delta[0])) - 1) < 2e-6
    for raw in (-17.0, -20.0):
        rate = -np.float32(np.log1p(np.exp(np.float64(raw))))
        delta = np.float32([1e7, 1e7])
        _, _, _, y, fin = hip.ssm_forward(delta, np.float32([0.0, 0.0]), np.float32([1.0, 1.0]),
                                          np.float32([rate]), np.float32([1.0, 1.0]), np.float32([1.0]), 2, 1, 1,
                                          materialize=False)
        expected = np.exp(-1e7 * np.float64(-rate)) ** 2
        assert abs(fin[0] - expected) < 2e-6


# --------------------------------------------------------------- retrieval
def ball(rng, n, dim, rmax=0.9):
    d = rng.standard_normal((n, dim))
    return (d / np.linalg.norm(d, axis=1, keepdims=True) * rng.uniform(0, rmax, (n, 1))).astype(np.float32)


def test_retrieve_closed_forms(hip):
    """tests/memory_expansion.rs:53-93 and tests/memory_projection.rs:40-54."""
    say("retrieve closed forms")
    K, N, V, count = bank(5, [[0.0], [0.1], [0.6]], [[2.0], [4.0], [100.0]])
    out, mn, idx, w = hip.retrieve(np.float32([[0.0]]), K, N, V, count, 1.0, top_k=1, want_weights=True)
    assert out[0, 0] == 2.0 and idx[0, 0] == 0
    np.testing.assert_array_equal(w[0], np.float32([1, 0, 0, 0, 0]))
    full, _, _, wf = hip.retrieve(np.float32([[0.0]]), K, N, V, count, 1.0, top_k=0, want_weights=True)
    for k in (3, 9):
        out, _, _, w = hip.retrieve(np.float32([[0.0]]), K, N, V, count, 1.0, top_k=k, want_weights=True)
        assert rel_err(out, full) < 1e-6 and rel_err(w, wf) < 1e-6
    K, N, V, count = bank(4, [[0.2], [-0.2]], [[1.0], [2.0]])
    out, _, idx, w = hip.retrieve(np.float32([[0.0]]), K, N, V, count, F32_MIN_SUB, top_k=1, want_weights=True)
    assert out[0, 0] == 1.0 and idx[0, 0] == 0  # exact tie -> lower slot
    K, N, V, count = bank(3, [[0.5], [-0.5], [0.75]], [[1.0, 2.0], [3.0, -2.0], [100.0, 100.0]])
    out, _, _, w = hip.retrieve(np.float32([[0.0]]), K, N, V, count, F32_MIN_SUB, top_k=0, want_weights=True)
    np.testing.assert_array_equal(w[0], np.float32([0.5, 0.5, 0.0]))
    np.testing.assert_array_equal(out[0], np.float32([2.0, 0.0]))
    K, N, V, count = bank(4, np.zeros((0, 1)), np.zeros((0, 1)))
    out, mn, idx, w = hip.retrieve(np.float32([[0.0]]), K, N, V, 0, 0.5, top_k=1, want_weights=True)
    assert out[0, 0] == 0.0 and not w.any() and idx[0, 0] == 0xFFFFFFFF


@pytest.mark.parametrize("n_q,C,dk,dv,k", [(1, 3, 2, 4, 2), (500, 512, 32, 48, 8), (300, 512, 768, 96, 8),
                                           (257, 100, 7, 5, 1)])
def test_retrieve_top_k_indices_bit_exact(hip, n_q, C, dk, dv, k):
    say("retrieve top-k", n_q, C, dk, dv, k)
    rng = np.random.default_rng(C + dk)
    keys = ball(rng, C, dk)
    vals = ball(rng, C, dv)
    q = ball(rng, n_q, dk)
    q[0] = keys[min(3, C - 1)]  # exact hit: distance 0
    K, N, V, count = bank(C, keys, vals)
    out, mn, idx, _ = hip.retrieve(q, K, N, V, count, 0.1, top_k=k)
    r_out, r_min, r_idx = O.retrieve_batch(K, N, V, count, q, 0.1, k, threads=8)
    np.testing.assert_array_equal(idx, r_idx)
    np.testing.assert_array_equal(mn.view(np.uint32), r_min.view(np.uint32))
    assert rel_err(out, r_out) < 1e-5


@pytest.mark.parametrize("n_q,cap,count,dk,dv,k,dup", [(130, 512, 512, 36, 40, 8, "all"),
                                                      (200, 600, 65, 64, 16, 64, "blocks"),
                                                      (96, 512, 300, 768, 64, 8, "blocks")])
def test_ranked_top_k_ties_and_job_batches(hip, n_q, cap, count, dk, dv, k, dup):
    """The pruned top-k path with exact distance ties.  "all": every slot
    holds the same key, so every slot is a candidate and a workgroup's
    exact-distance jobs exceed one batch; ties go to the lower slots.
    "blocks": runs of duplicated keys and queries that hit keys exactly.
    Covers k = 64 of 65 slots, a capacity past the occupied 512 slots, a key
    width that is not a multiple of the slab and a partial last workgroup."""
    say("ranked top-k ties", n_q, cap, count, dk, dv, k, dup)
    rng = np.random.default_rng(count + dk)
    keys = ball(rng, count, dk)
    if dup == "all":
        keys[:] = keys[0]
    else:
        keys[10:40] = keys[5]
        keys[50:52] = keys[7]
    vals = ball(rng, count, dv)
    q = ball(rng, n_q, dk)
    q[0], q[1], q[2] = keys[5], keys[7], keys[count - 1]
    K, N, V, cnt = bank(cap, keys, vals)
    out, mn, idx, w = hip.retrieve(q, K, N, V, cnt, 0.1, top_k=k, want_weights=True)
    r_out, r_min, r_idx = O.retrieve_batch(K, N, V, cnt, q, 0.1, k, threads=8)
    np.testing.assert_array_equal(idx, r_idx)
    np.testing.assert_array_equal(mn.view(np.uint32), r_min.view(np.uint32))
    assert rel_err(out, r_out) < 1e-5
    if dup == "all":
        assert np.all(idx == np.arange(k, dtype=np.uint32))
    for i in range(n_q):
        nz = np.flatnonzero(w[i])
        assert set(nz.tolist()) <= set(idx[i].tolist())
    np.testing.assert_allclose(w.sum(axis=1), 1.0, rtol=1e-5)


def test_retrieve_config4_every_index_bit_exact(hip):
    """Config 4 at full size on device buffers: 512 x 768 bank, 32768 queries,
    top-8.  Every index and every minimum distance equals the oracle's bit
    for bit; the readout within 1e-5."""
    say("retrieve config4 full")
    rng = np.random.default_rng(4)
    C_, dk, nq, k = 512, 768, 32768, 8
    keys, vals, q = ball(rng, C_, dk), ball(rng, C_, dk), ball(rng, nq, dk)
    nsq = np.array([O.squared_norm(x) for x in keys], np.float32)
    bufs = [hip.upload(a) for a in (q, keys, nsq, vals)]
    out, mn, idx = hip.empty((nq, dk), np.float32), hip.empty((nq,), np.float32), hip.empty((nq, k), np.uint32)
    hip.retrieve_resident(bufs[0].ptr, nq, bufs[1].ptr, bufs[2].ptr, bufs[3].ptr, C_, C_, dk, dk, 0.1, k,
                          out.ptr, mn.ptr, idx.ptr)
    hip.synchronize()
    g_out, g_min, g_idx = out.to_host(), mn.to_host(), idx.to_host()
    for b in bufs + [out, mn, idx]:
        b.close()
    r_out, r_min, r_idx = O.retrieve_batch(keys, nsq, vals, C_, q, 0.1, k, threads=16)
    np.testing.assert_array_equal(g_idx, r_idx)
    np.testing.assert_array_equal(g_min.view(np.uint32), r_min.view(np.uint32))
    assert rel_err(g_out, r_out) < 1e-5


def test_retrieve_full_soft_read(hip):
    say("retrieve full soft read")
    rng = np.random.default_rng(11)
    keys, vals, q = ball(rng, 200, 16), ball(rng, 200, 24), ball(rng, 64, 16)
    K, N, V, count = bank(256, keys, vals)
    out, mn, _, w = hip.retrieve(q, K, N, V, count, 0.1, top_k=0, want_weights=True)
    r_out, r_min, _ = O.retrieve_batch(K, N, V, count, q, 0.1, 0)
    assert rel_err(out, r_out) < 1e-5
    np.testing.assert_array_equal(mn.view(np.uint32), r_min.view(np.uint32))
    assert not w[:, count:].any()
    np.testing.assert_allclose(w.sum(axis=1), 1.0, rtol=1e-5)


def test_memory_forward_stage_matches_oracle(hip):
    """GpuDispatch::memory_forward composition against the oracle's per-token
    steps (src/pssa.rs:1147-1172)."""
    say("memory_forward stage")
    rng = np.random.default_rng(12)
    L, d, k, C, count = 40, 24, 6, 16, 12
    xn = rng.standard_normal((L, d)).astype(np.float32)
    y = rng.standard_normal((L, d)).astype(np.float32) * 0.3
    wqx, wqh = (rng.standard_normal((k, d)) * 0.1).astype(np.float32), (rng.standard_normal((k, d)) * 0.1).astype(np.float32)
    wg, wp = (rng.standard_normal((d, d)) * 0.1).astype(np.float32), (rng.standard_normal((d, d)) * 0.1).astype(np.float32)
    K, N, V, count = bank(C, ball(rng, count, k), ball(rng, count, d))
    for top_k in (0, 4):
        out = hip.memory_forward(xn, y, wqx, wqh, wg, wp, K, N, V, L, d, k, d, C, count, 0.1, top_k)
        qe = O.gemm_xwt(xn, wqx) + O.gemm_xwt(y, wqh)
        assert rel_err(out["q_euc"].reshape(L, k), qe) < 1e-5
        qp = np.stack([O.project(r)[0] for r in qe])
        assert rel_err(out["q_pnc"].reshape(L, k), qp) < 1e-5
        mv = np.stack([O.retrieve(K, N, V, count, qp[t], 0.1, top_k)[0] for t in range(L)])
        assert rel_err(out["m_val"].reshape(L, d), mv) < 1e-4
        g = 1 / (1 + np.exp(-O.gemm_xwt(xn, wg).astype(np.float64)))
        assert rel_err(out["g_mem"].reshape(L, d), g) < 1e-5
        mp = mv.astype(np.float64) @ wp.T.astype(np.float64)
        assert rel_err(out["m_inj"].reshape(L, d), g * mp) < 1e-4


def test_resident_ssm_then_memory_equals_the_two_stages(hip):
    """ssm_forward_resident + memory_forward_after_ssm (src/backend.rs:
    1186-1289) give the outputs of ssm_forward + memory_forward bit for bit;
    the tape is consumed, and a missing or mismatched tape is an error."""
    say("resident ssm -> memory")
    rng = np.random.default_rng(21)
    L, d, s, k, C = 37, 32, 24, 6, 16
    delta = rng.uniform(0.01, 0.5, (L, d)).astype(np.float32)
    bp, cp = rng.standard_normal((L, s)).astype(np.float32), rng.standard_normal((L, s)).astype(np.float32)
    xn = rng.standard_normal((L, d)).astype(np.float32)
    rates = -rng.uniform(0.1, 2.0, d * s).astype(np.float32)
    h0 = (rng.standard_normal(d * s) * 0.1).astype(np.float32)
    wqx, wqh = (rng.standard_normal((k, d)) * 0.1).astype(np.float32), (rng.standard_normal((k, d)) * 0.1).astype(np.float32)
    wg, wp = (rng.standard_normal((d, d)) * 0.1).astype(np.float32), (rng.standard_normal((d, d)) * 0.1).astype(np.float32)
    K, N, V, count = bank(C, ball(rng, 12, k), ball(rng, 12, d))
    mem = (wqx, wqh, wg, wp, K, N, V, L, d, k, d, C, count, 0.1)
    with pytest.raises(HipError, match="no resident SSM tape"):
        hip.memory_forward_after_ssm(xn, *mem, d_s=s)
    bar_a, bar_b, states, y, _ = hip.ssm_forward(delta, bp, xn, rates, cp, h0, L, d, s)
    ref = hip.memory_forward(xn, y, *mem, top_k=4)
    hip.ssm_forward_resident(delta[:-1], bp[:-1], xn[:-1], rates, cp[:-1], h0, L - 1, d, s)
    with pytest.raises(HipError, match="no resident SSM tape"):
        hip.memory_forward_after_ssm(xn, *mem, d_s=s)  # L rows against an (L-1)-row tape
    hip.ssm_forward_resident(delta, bp, xn, rates, cp, h0, L, d, s)
    got = hip.memory_forward_after_ssm(xn, *mem, d_s=s, top_k=4)
    for name, want in [("bar_a", bar_a), ("bar_b", bar_b), ("states", states), ("y_ssm", y)] + list(ref.items()):
        np.testing.assert_array_equal(got[name], want, err_msg=name)
    with pytest.raises(HipError, match="no resident SSM tape"):
        hip.memory_forward_after_ssm(xn, *mem, d_s=s)


# -------------------------------------------------------------- dense scan
@pytest.mark.parametrize("B,L,s", [(1, 1, 1), (3, 100, 5), (2, 257, 16), (4, 300, 33), (5, 200, 64),
                                   (2, 1, 64), (3, 7, 64), (2, 8, 64), (2, 9, 64), (3, 10, 64), (1, 17, 64)])
def test_dense_scan_matches_oracle(hip, B, L, s):
    say("dense scan", B, L, s)
    rng = np.random.default_rng(B * L + s)
    q, _ = np.linalg.qr(rng.standard_normal((B, L, s, s)))
    a = (q * rng.uniform(0.8, 0.99, (B, L, 1, s))).astype(np.float32)
    b = rng.standard_normal((B, L, s)).astype(np.float32)
    h0 = rng.standard_normal((B, s)).astype(np.float32)
    h = hip.dense_scan(a, b, h0)
    ref = O.dense_scan(a, b, h0, threads=4)
    assert rel_err(h, ref) < 1e-4


@pytest.mark.parametrize("B,L", [(1, 256), (3, 300), (2, 513), (5, 1000)])
def test_dense_scan_two_level_matches_oracle(hip, B, L):
    """d_state 64 and at least two windows of 128 steps take the chunked
    two-level schedule (composed sub-chunk maps on the matrix cores, exact
    fp32 re-runs); ragged last windows leave sub-chunks partial or empty."""
    say("dense scan two-level", B, L)
    s = 64
    rng = np.random.default_rng(B * L)
    q, _ = np.linalg.qr(rng.standard_normal((B, L, s, s)))
    a = (q * rng.uniform(0.8, 0.99, (B, L, 1, s))).astype(np.float32)
    b = rng.standard_normal((B, L, s)).astype(np.float32)
    h0 = rng.standard_normal((B, s)).astype(np.float32)
    h = hip.dense_scan(a, b, h0)
    ref = O.dense_scan(a, b, h0, threads=4)
    assert_parity(h, ref, 1e-4, f"two-level {B}x{L}")


def test_dense_scan_two_level_replays_when_a_map_is_not_finite(hip):
    """An infinite transition entry (sequence 1, step 170 = window 1,
    sub-chunk 1) makes that sub-chunk's composed map non-finite: it is marked
    unusable and the later sub-chunks of the window replay it in fp32.  The
    states before the entry match the sequential recurrence, every state
    from it on is non-finite as in the recurrence, and the other sequences
    are unaffected."""
    say("dense scan two-level fallback")
    B, L, s = 3, 400, 64
    rng = np.random.default_rng(77)
    q, _ = np.linalg.qr(rng.standard_normal((B, L, s, s)))
    a = (q * rng.uniform(0.8, 0.99, (B, L, 1, s))).astype(np.float32)
    a[1, 170, 5, 9] = np.inf
    b = rng.standard_normal((B, L, s)).astype(np.float32)
    h = hip.dense_scan(a, b, None)
    with np.errstate(invalid="ignore", over="ignore"):
        ref = O.dense_scan(a, b, None, threads=4)
    for i in (0, 2):
        assert_parity(h[i], ref[i], 1e-4, f"sequence {i}")
    assert_parity(h[1, :170], ref[1, :170], 1e-4, "sequence 1 before the entry")
    assert not np.isfinite(ref[1, 171:]).any()
    assert not np.isfinite(h[1, 171:]).any()
    np.testing.assert_array_equal(np.isfinite(h[1, 170]), np.isfinite(ref[1, 170]))


@pytest.mark.parametrize("kind", ["orthogonal", "expanding"])
def test_dense_scan_two_level_non_contracting_transitions(hip, kind):
    """Transitions that do not contract: A_t orthogonal (u = 1), or A_t =
    Q_t diag(u_t) with u_t ~ U[1.0, 1.004] (the state grows about e^4 over
    the sequence).  Their composed maps are not used (Frobenius norm above
    1); the sub-chunks are replayed in fp32, so the 2048-step scan meets the
    fp32 gate against the sequential recurrence.  The resident entry point
    runs the same shape after dense_scan_reserve."""
    say("dense scan two-level non-contracting", kind)
    B, T, s = 4, 2048, 64
    rng = np.random.default_rng(31 if kind == "orthogonal" else 32)
    pool = householder_pool(rng, B * T, s)
    if kind == "orthogonal":
        a = pool
    else:
        a = pool * (1.0 + 0.004 * rng.random((B * T, 1, s), dtype=np.float32))
    a = np.ascontiguousarray(a.reshape(B, T, s, s), dtype=np.float32)
    b = rng.standard_normal((B, T, s)).astype(np.float32)
    h = hip.dense_scan(a, b, None)
    ref = O.dense_scan(a, b, None, threads=4)
    for i in range(B):
        assert_parity(h[i], ref[i], 1e-4, f"{kind} sequence {i}")
    hip.dense_scan_reserve(B, T, s)
    a_dev, b_dev, h_dev = hip.upload(a), hip.upload(b), hip.empty((B, T, s), np.float32)
    hip.dense_scan_resident(a_dev.ptr, b_dev.ptr, None, B, T, s, h_dev.ptr)
    np.testing.assert_array_equal(h_dev.to_host(), h)
    for buf in (a_dev, b_dev, h_dev):
        buf.close()


def householder_pool(rng, n, s):
    """n random orthogonal matrices, each a product of two Householder
    reflections (the pool config 2's transitions are drawn from)."""
    v1 = rng.standard_normal((n, s)).astype(np.float32)
    v2 = rng.standard_normal((n, s)).astype(np.float32)
    v1 /= np.linalg.norm(v1, axis=1, keepdims=True)
    v2 /= np.linalg.norm(v2, axis=1, keepdims=True)
    dot = np.einsum("ns,ns->n", v1, v2)[:, None, None]
    q = -2.0 * v1[:, :, None] * v1[:, None, :] - 2.0 * v2[:, :, None] * v2[:, None, :] \
        + 4.0 * dot * v1[:, :, None] * v2[:, None, :]
    q[:, np.arange(s), np.arange(s)] += 1.0
    return q.astype(np.float32)


def test_dense_scan_config2_full_workload(hip):
    """Config 2 at its full size: 64 sequences x 2048 steps, d_state 64,
    A_t = Q_t diag(u_t) (Q_t orthogonal, u_t ~ U[0.8, 0.99]^64), b_t ~ N(0, 1),
    h_0 = 0.  Every sequence against the sequential recurrence."""
    say("dense scan config 2 full")
    B, T, s = 64, 2048, 64
    rng = np.random.default_rng(12)
    pool = householder_pool(rng, 8192, s)
    a = np.empty((B * T, s, s), np.float32)
    for c0 in range(0, B * T, 8192):
        a[c0:c0 + 8192] = pool * (0.8 + 0.19 * rng.random((8192, 1, s), dtype=np.float32))
    a = a.reshape(B, T, s, s)
    b = rng.standard_normal((B, T, s)).astype(np.float32)
    h = hip.dense_scan(a, b, None)
    ref = O.dense_scan(a, b, None, threads=16)
    for i in range(B):
        assert_parity(h[i], ref[i], 1e-4, f"sequence {i}")


def test_softplus_in_place_matches_oracle(hip):
    """GpuDispatch::softplus_in_place (src/backend.rs:1419-1428) against the
    reference's softplus (src/linalg.rs:548-551) over both branches, the
    x > 20 cut and the far tails."""
    say("softplus_in_place")
    rng = np.random.default_rng(3)
    # Down to -87, where e^x is still a normal float.
    x = np.concatenate([rng.standard_normal(5000) * 6, np.linspace(-87, 60, 3001), [0.0, 20.0, 20.000002, 19.999998,
                        -1e-30, 1e-30, -87.0]]).astype(np.float32)
    got = x.copy()
    hip.softplus_in_place(got)
    ref = np.array([O.softplus(v) for v in x], np.float32)
    np.testing.assert_array_equal(got[x > 20], x[x > 20])
    assert elem_rel_err(got, ref, floor=1e-37) < 2e-6
