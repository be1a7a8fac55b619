"""GPU: the allocation-free GEMM entry point (sulimo_hip_enqueue_gemm_q4_0_f16_noalloc)
against the allocating one (sulimo_hip_enqueue_gemm_q4_0_f16) through the C ABI.

Its scratch (the weights' GEMM layout and the K-split partial sums) is the library's
static per-device array, which keeps the previous call's contents: two calls in a
row, the second with smaller operands, and the first shape again after it, must each
equal the allocating entry point's output bit for bit (same kernels, same plan), and
stay within the oracle's error bound. A matrix too large for the array is refused on
the host.
"""
import ctypes

import numpy as np
import pytest

import oracle
from sulimo_amd import hip
from sulimo_amd import synthetic as S
from tests.test_gpu_gemm import f16_weight_bound

pytestmark = pytest.mark.gpu


def _operands(ctx, seed, m_out, k, n_tok):
    t = S.random_q4(np.random.default_rng(seed), m_out, k)
    x = S.random_activations(seed + 1, (n_tok, k))
    bufs = (hip.HipBuffer.from_host(ctx, t.scales, True), hip.HipBuffer.from_host(ctx, t.quants, True),
            hip.HipBuffer.from_host(ctx, x, True))
    return t, x, bufs


def test_noalloc_gemm_matches_allocating_entry_point(ctx):
    # (m_out, k, n_tok): the up-projection GEMM at 128 tokens, then a smaller one
    shapes = [(8960, 1536, 128), (1536, 1536, 37), (8960, 1536, 128)]
    ops = {}
    for i, (m_out, k, n_tok) in enumerate(shapes):
        print(f"no-alloc GEMM call {i}: m_out {m_out} k {k} n_tok {n_tok}", flush=True)
        if (m_out, k, n_tok) not in ops:
            ops[(m_out, k, n_tok)] = _operands(ctx, 100 + i, m_out, k, n_tok)
        t, x, (sb, qb, xb) = ops[(m_out, k, n_tok)]
        out_a = hip.HipBuffer.device_only(ctx, n_tok * m_out * 2)
        out_b = hip.HipBuffer.device_only(ctx, n_tok * m_out * 2)
        hip.enqueue_gemm_q4_0_f16_noalloc(ctx, sb, qb, xb, out_b, m_out, k, n_tok)
        hip.enqueue_gemm_q4_0_f16(ctx, sb, qb, xb, out_a, m_out, k, n_tok)
        ctx.wait()
        ya = out_a.download(np.uint16, (n_tok, m_out))
        yb = out_b.download(np.uint16, (n_tok, m_out))
        assert np.array_equal(ya, yb), f"call {i} differs from the allocating entry point"
        ref = oracle.gemm_q4_0_f16_scalar_reference(t.scales, t.quants, x, m_out, k, n_tok)
        err = np.abs(yb.view(np.float16).astype(np.float64) - ref.astype(np.float64))
        assert np.all(err <= f16_weight_bound(x, t.scales, t.quants, ref))
        out_a.release()
        out_b.release()
    for _, _, bufs in ops.values():
        for b in bufs:
            b.release()


def _free_device_bytes():
    rt = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert rt.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_noalloc_gemm_allocates_nothing(ctx):
    """The device's free memory is unchanged by two no-alloc calls on freshly uploaded
    weights (24.8 MB in the GEMM layout, which the allocating entry point would build
    and cache), and the allocating call that follows does lower it: the probe sees an
    allocation of that size. Two contexts, each on its own stream, then call the entry
    point back to back: the library orders them, and both outputs equal the allocating
    entry point's."""
    m_out, k, n_tok = 28672, 1536, 64
    t, x, (sb, qb, xb) = _operands(ctx, 300, m_out, k, n_tok)
    outs = [hip.HipBuffer.device_only(ctx, n_tok * m_out * 2) for _ in range(3)]
    t2, x2, (sb2, qb2, xb2) = _operands(ctx, 310, 1536, 1536, 37)
    o2 = hip.HipBuffer.device_only(ctx, 37 * 1536 * 2)
    o2_ref = hip.HipBuffer.device_only(ctx, 37 * 1536 * 2)
    # a first call loads the kernels' code objects (run alone, this test is their first user)
    hip.enqueue_gemm_q4_0_f16_noalloc(ctx, sb2, qb2, xb2, o2, 1536, 1536, 37)
    ctx.wait()
    before = _free_device_bytes()
    hip.enqueue_gemm_q4_0_f16_noalloc(ctx, sb, qb, xb, outs[0], m_out, k, n_tok)
    hip.enqueue_gemm_q4_0_f16_noalloc(ctx, sb, qb, xb, outs[1], m_out, k, n_tok)
    ctx.wait()
    after = _free_device_bytes()
    print(f"no-alloc: free device memory {before} -> {after} bytes", flush=True)
    assert after == before
    hip.enqueue_gemm_q4_0_f16(ctx, sb, qb, xb, outs[2], m_out, k, n_tok)
    ctx.wait()
    assert _free_device_bytes() < after
    want = outs[2].download(np.uint16, (n_tok, m_out))
    assert np.array_equal(outs[0].download(np.uint16, (n_tok, m_out)), want)
    assert np.array_equal(outs[1].download(np.uint16, (n_tok, m_out)), want)
    # two contexts (two streams) issuing no-alloc calls back to back
    other = hip.HipContext.new(0)
    try:
        hip.enqueue_gemm_q4_0_f16_noalloc(ctx, sb, qb, xb, outs[0], m_out, k, n_tok)
        hip.enqueue_gemm_q4_0_f16_noalloc(other, sb2, qb2, xb2, o2, 1536, 1536, 37)
        other.wait()
        ctx.wait()
    finally:
        other.release()
    hip.enqueue_gemm_q4_0_f16(ctx, sb2, qb2, xb2, o2_ref, 1536, 1536, 37)
    ctx.wait()
    assert np.array_equal(outs[0].download(np.uint16, (n_tok, m_out)), want)
    assert np.array_equal(o2.download(np.uint16, (37, 1536)), o2_ref.download(np.uint16, (37, 1536)))
    for b in (sb, qb, xb, sb2, qb2, xb2, o2, o2_ref, *outs):
        b.release()


def test_noalloc_gemm_rejects_matrices_beyond_the_scratch(ctx):
    """The LM head (151936 x 1536: 131 MB in the GEMM layout) exceeds the 64 MiB array:
    refused before anything is launched."""
    m_out, k, n_tok = 151936, 1536, 1
    sb = hip.HipBuffer.device_only(ctx, m_out * k // 32 * 2)
    qb = hip.HipBuffer.device_only(ctx, m_out * k // 32 * 16)
    xb = hip.HipBuffer.device_only(ctx, n_tok * k * 2)
    ob = hip.HipBuffer.device_only(ctx, n_tok * m_out * 2)
    with pytest.raises(hip.HipError) as e:
        hip.enqueue_gemm_q4_0_f16_noalloc(ctx, sb, qb, xb, ob, m_out, k, n_tok)
    assert e.value.code == hip.ERR_INVALID_ARGUMENT and "at most" in e.value.message
    for b in (sb, qb, xb, ob):
        b.release()
