"""GPU parity of the per-op entry points (sulimo_hip_enqueue_*, sulimo_hip_embed_tokens)
against the oracle's restatement of the reference kernels (kernels/prefill.cl) and
CPU path. Integer outputs (Q8_0 codes and scales, embedding f16 bits) are bit-exact.
"""
import numpy as np
import pytest

import oracle
from sulimo_amd import hip
from sulimo_amd import synthetic as S
from tests.helpers import cosine, max_rel_err, prefill_act_fill

pytestmark = pytest.mark.gpu


def up(ctx, a, ro=True):
    return hip.HipBuffer.from_host(ctx, np.ascontiguousarray(a), ro)


def f16_close(got, want, ulps=1):
    """|got - want| <= ulps f16 ulps of want (elementwise)."""
    g = got.astype(np.float64)
    w = want.astype(np.float64)
    ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
    return bool(np.all(np.abs(g - w) <= ulps * ulp + 1e-7))


@pytest.mark.parametrize("d,n", [(1536, 37), (3072, 8), (64, 5)])
def test_rmsnorm(ctx, d, n):
    rng = np.random.default_rng(d + n)
    x = rng.standard_normal((n, d)).astype(np.float16)
    w = (1 + rng.normal(0, 0.02, d)).astype(np.float32)
    xb, wb, ob = up(ctx, x), up(ctx, w), hip.HipBuffer.device_only(ctx, n * d * 2)
    hip.enqueue_rmsnorm(ctx, xb, wb, ob, d, 1e-6, n)
    got = ob.download(np.float16, (n, d))
    want = oracle.cl_rmsnorm_f16_f32w(x, w, d, 1e-6, n)
    assert f16_close(got, want, 1)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("heads,hd,base,start", [(12, 128, 1e6, 5), (8, 128, 5e5, 1500), (2, 64, 1e4, 0),
                                                 (12, 128, 1e6, 4000)])
def test_rope(ctx, mode, heads, hd, base, start):
    """rope_f16 (kernels/prefill.cl:32-68), bit for bit given the device's cos/sin.

    1. The device's (cos, sin) table against float64 trig of the float64 angle
       pos / base^(2i/rope_dim): the f32 angle carries a few ulps of rounding, so the
       bound grows with the angle (8 * theta * 2^-24 + 2^-22).
    2. The rotation with those values, products rounded to f32 before the add
       (rot_sub / rot_add: x0 c - x1 s, x0 s + x1 c), then one f16 rounding, equals the
       device's output bit for bit. Norm mode pairs (2i, 2i+1), NeoX (i, i + d/2).
    3. The oracle's rope_f16 with glibc trig stays within the table's error."""
    n = 33
    half = hd // 2
    rng = np.random.default_rng(heads + hd + mode + start)
    v = (rng.standard_normal((n, heads, hd)) * 2).astype(np.float16)
    vb = up(ctx, v, ro=False)
    hip.enqueue_rope(ctx, vb, heads, hd, hd, base, mode, start, n)
    got = vb.download(np.float16, (n, heads, hd))
    tb = hip.HipBuffer.device_only(ctx, n * half * 8)
    hip.rope_table(ctx, hd, base, start, n, tb)
    tab = tb.download(np.float32, (n, half, 2))
    tb.release()
    theta = (start + np.arange(n, dtype=np.float64))[:, None] * float(base) ** (-2.0 * np.arange(half) / hd)
    bound = 8.0 * theta * 2.0 ** -24 + 2.0 ** -22
    assert np.all(np.abs(tab[..., 0] - np.cos(theta)) <= bound)
    assert np.all(np.abs(tab[..., 1] - np.sin(theta)) <= bound)
    i = np.arange(half)
    i0, i1 = (2 * i, 2 * i + 1) if mode == 0 else (i, i + half)
    x = v.astype(np.float32)
    c, s = tab[:, None, :, 0], tab[:, None, :, 1]
    v0, v1 = x[:, :, i0], x[:, :, i1]
    want = x.copy()
    want[:, :, i0] = v0 * c - v1 * s
    want[:, :, i1] = v0 * s + v1 * c
    assert np.array_equal(got.view(np.uint16), want.astype(np.float16).view(np.uint16))
    ref = oracle.cl_rope_f16(v, heads, hd, hd, base, mode, start, n).astype(np.float64)
    amp = np.abs(v.astype(np.float64)).max()
    tol = 2 * amp * bound.max() + np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got.astype(np.float64) - ref) <= tol)


def _kv_case(ctx, act, start, cap, bpb, n):
    ring0 = np.random.default_rng(5).integers(0, 256, cap * bpb * 34, dtype=np.uint8)  # sentinel bytes
    ab, kb = up(ctx, act), up(ctx, ring0.copy(), ro=False)
    hip.enqueue_kv_store(ctx, ab, kb, start, cap, bpb, n)
    got = kb.download(np.uint8, ring0.shape)
    want = oracle.cl_kv_store_q8_0(act, ring0, start, cap, bpb, n)
    return got, want


def test_kv_store_reference_pattern_bit_exact(ctx):
    """test_prefill.rs:56-192 (16 tokens x 8 blocks, start 5, capacity 64), tightened to
    byte equality of the whole ring (untouched slots keep their bytes)."""
    n, bpb, cap, start = 16, 8, 64, 5
    act = prefill_act_fill(n * bpb * 32).reshape(n, bpb * 32)
    got, want = _kv_case(ctx, act, start, cap, bpb, n)
    assert np.array_equal(got, want)


def test_kv_store_special_blocks_and_wrap(ctx):
    """Zero block (d=0, codes 0), exact .5 ties (round half away from zero), +-amax ->
    +-127, f16-subnormal scales, negative zero; positions wrap at capacity."""
    # 12 tokens on 8 slots: tokens 0-3 are overwritten by tokens 8-11 (last writer wins).
    n, bpb, cap, start = 12, 4, 8, 5
    act = np.random.default_rng(9).standard_normal((n, bpb * 32)).astype(np.float16)
    act[4, :32] = 0
    ties = np.arange(-16, 16, dtype=np.float32) + 0.5
    act[5, :32] = np.concatenate([[127.0], ties[1:]]).astype(np.float16)  # d = 1 -> id = 1: x.5 ties
    act[6, :32] = (np.linspace(-1, 1, 32) * 1.2e-4).astype(np.float16)  # d ~ 9.4e-7: f16 subnormal
    act[7, :32] = -0.0
    act[8, 32:64] = np.float16(-65504.0)
    got, want = _kv_case(ctx, act, start, cap, bpb, n)
    assert np.array_equal(got, want)
    # pin: the tie block rounds away from zero (2.5 -> 3, -2.5 -> -3)
    blk = want.reshape(cap, bpb, 34)[(start + 5) % cap, 0]
    codes = blk[2:].view(np.int8)
    x = act[5, :32].astype(np.float32)
    assert np.array_equal(codes, (np.sign(x) * np.floor(np.abs(x) + 0.5)).astype(np.int8))


def test_silu_mul_and_add(ctx):
    rng = np.random.default_rng(3)
    g = (rng.standard_normal(10007) * 3).astype(np.float16)
    u = rng.standard_normal(10007).astype(np.float16)
    gb, ub, ob = up(ctx, g), up(ctx, u), hip.HipBuffer.device_only(ctx, g.nbytes)
    hip.enqueue_silu_mul(ctx, gb, ub, ob, g.size)
    assert f16_close(ob.download(np.float16, g.shape), oracle.cl_silu_mul_f16(g, u), 1)
    ab = up(ctx, g, ro=False)
    hip.enqueue_add(ctx, ab, ub, g.size)
    assert np.array_equal(ab.download(np.float16, g.shape).view(np.uint16),
                          oracle.cl_add_f16(g, u).view(np.uint16))


def test_logits_final(ctx):
    rng = np.random.default_rng(4)
    V, D, n = 4096, 512, 7
    w = S.random_q4(rng, V, D)
    x = rng.standard_normal((n, D)).astype(np.float16)
    xb, sb, qb = up(ctx, x), up(ctx, w.scales), up(ctx, w.quants)
    lb = hip.HipBuffer.device_only(ctx, V * 4)
    hip.enqueue_logits_final(ctx, xb, sb, qb, lb, V, D, n - 1)
    got = lb.download(np.float32, (V,))
    want = oracle.cl_logits_f16_output(x, w.scales, w.quants, V, D, n - 1)
    assert max_rel_err(got, want) <= 2e-3


def test_embed_tokens_bit_exact(ctx):
    """Device gather == lookup_token_embedding_f16 (scheduler.rs:329-374), every bit."""
    rng = np.random.default_rng(6)
    V, D = 1000, 1536
    t = S.random_q4(rng, V, D)
    toks = rng.integers(0, V, 64, dtype=np.uint32)
    toks[:3] = [0, V - 1, 17]
    sb, qb = up(ctx, t.scales), up(ctx, t.quants)
    xb = hip.HipBuffer.device_only(ctx, 64 * D * 2)
    hip.embed_tokens(ctx, sb, qb, toks, D, V, xb)
    got = xb.download(np.float16, (64, D))
    want = np.stack([oracle.lookup_token_embedding_f16(t.scales, t.quants, D, int(k)) for k in toks])
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    with pytest.raises(hip.HipError):
        hip.embed_tokens(ctx, sb, qb, np.array([V], np.uint32), D, V, xb)


def _ring(rng, cap, hkv, hd):
    """A Q8_0 ring filled with quantized N(0,1) K values (kv_cache.rs layout)."""
    vals = rng.standard_normal((cap, hkv * hd)).astype(np.float32)
    return oracle.quantize_f32_to_q8_0(vals)


@pytest.mark.parametrize("hq,hkv,hd,n,start,cap", [
    (12, 2, 128, 100, 0, 256),     # Qwen2.5 grouping, fresh prompt
    (12, 2, 128, 64, 37, 256),     # resumed at start_pos 37
    (6, 2, 128, 70, 0, 128),       # Llama grouping (3 q heads per kv head)
    (4, 4, 64, 40, 3, 64),         # MHA, head_dim 64
    (12, 2, 128, 50, 200, 128),    # window of the last `capacity` positions (ring wrap)
    # long key ranges: query blocks split over several workgroups and merged
    (12, 2, 128, 7, 1500, 2048),   # a few queries after a long context
    (12, 2, 128, 1024, 0, 1024),   # long fresh prompt
    (6, 2, 128, 300, 900, 1024),   # Llama grouping, resumed, near the window edge
    (4, 4, 64, 200, 2000, 256),    # head_dim 64, ring wrap with split blocks
])
def test_attention_prefill(ctx, hq, hkv, hd, n, start, cap):
    rng = np.random.default_rng(hq * 7 + n + start)
    q = rng.standard_normal((n, hq, hd)).astype(np.float16)
    kr, vr = _ring(rng, cap, hkv, hd), _ring(rng, cap, hkv, hd)
    qb, kb, vb = up(ctx, q), up(ctx, kr), up(ctx, vr)
    ob = hip.HipBuffer.device_only(ctx, q.nbytes)
    hip.enqueue_attention_prefill(ctx, qb, kb, vb, ob, start, cap, hq, hkv, hd, n)
    got = ob.download(np.float16, q.shape).astype(np.float32)
    want = oracle.attention_prefill_f32(q.astype(np.float32), kr, vr, start, cap, hq, hkv, hd, n).reshape(q.shape)
    assert np.max(np.abs(got - want)) <= 1e-2 * max(1.0, float(np.abs(want).max()))
    assert cosine(got, want) >= 0.9999


@pytest.mark.parametrize("hq,hkv,hd,n,cap", [(12, 2, 128, 2048, 2048),   # Qwen2.5-1.5B, 2048-token prompt
                                            (24, 8, 128, 4096, 4096)])  # Llama-3.2-3B, 4096-token prompt
def test_attention_prefill_headline_shapes(ctx, hq, hkv, hd, n, cap):
    """The attention of the benchmark steps from position 0 (split query blocks plus the
    merge), against the oracle. q ~ 3 N(0,1) makes the softmax peaked (scores of std 3),
    so uniform weights, a wrong head map or a missing causal mask change the output."""
    rng = np.random.default_rng(hq + n)
    q = (3.0 * rng.standard_normal((n, hq, hd))).astype(np.float16)
    kr, vr = _ring(rng, cap, hkv, hd), _ring(rng, cap, hkv, hd)
    qb, kb, vb = up(ctx, q), up(ctx, kr), up(ctx, vr)
    ob = hip.HipBuffer.device_only(ctx, q.nbytes)
    hip.enqueue_attention_prefill(ctx, qb, kb, vb, ob, 0, cap, hq, hkv, hd, n)
    got = ob.download(np.float16, q.shape).astype(np.float32)
    for b in (qb, kb, vb, ob):
        b.release()
    want = oracle.attention_prefill_f32(q.astype(np.float32), kr, vr, 0, cap, hq, hkv, hd, n).reshape(q.shape)
    err = float(np.max(np.abs(got - want)))
    print(f"attention {hq}/{hkv} heads, {n} queries: max abs err {err:.3e}, |out| max {np.abs(want).max():.3f}")
    assert max_rel_err(got, want) <= 1e-2
    assert err <= 4e-3 * max(1.0, float(np.abs(want).max()))
    assert cosine(got, want) >= 0.99999


@pytest.mark.parametrize("hq,hkv,hd,n,start,cap", [
    (12, 2, 128, 2048, 0, 2048),   # the 2048-token prompt's attention (one key half per workgroup)
    (12, 2, 128, 512, 1024, 2048),  # third 512-token micro-batch (two key halves per workgroup)
    (12, 2, 128, 7, 1500, 2048),   # a few queries after a long context: many pieces per block
    (6, 2, 128, 300, 900, 1024),   # Llama grouping, resumed
    (4, 4, 64, 200, 2000, 256),    # head_dim 64, ring wrap
])
def test_attention_split_merge_paths_bit_identical(ctx, hq, hkv, hd, n, start, cap):
    """Split query blocks merged by the last workgroup of each block (device-scope
    record stores and an arrival counter per block and query wave) give the same bits
    as the separate merge kernel, on three calls in a row (each in-kernel merge leaves
    its counters at zero for the next call)."""
    rng = np.random.default_rng(hq * 11 + n + start)
    q = (3.0 * rng.standard_normal((n, hq, hd))).astype(np.float16)
    kr, vr = _ring(rng, cap, hkv, hd), _ring(rng, cap, hkv, hd)
    qb, kb, vb = up(ctx, q), up(ctx, kr), up(ctx, vr)
    ob = hip.HipBuffer.device_only(ctx, q.nbytes)

    def run():
        hip.enqueue_attention_prefill(ctx, qb, kb, vb, ob, start, cap, hq, hkv, hd, n)
        return ob.download(np.float16, q.shape).view(np.uint16).copy()

    try:
        inkernel = [run() for _ in range(3)]
        ctx.set_attention_merge_kernel(True)
        separate = run()
    finally:
        ctx.set_attention_merge_kernel(False)
    for b in (qb, kb, vb, ob):
        b.release()
    for r in inkernel:
        assert np.array_equal(r, separate)
    want = oracle.attention_prefill_f32(q.astype(np.float32), kr, vr, start, cap, hq, hkv, hd, n).reshape(q.shape)
    assert max_rel_err(separate.view(np.float16).astype(np.float32), want) <= 1e-2


def test_buffer_leak_cycle(ctx):
    """active_cl_mem_count returns to its baseline after create/release cycles
    (test_m4_scheduler.rs:286-365)."""
    base = hip.active_buffer_count()
    for _ in range(50):
        b = hip.HipBuffer.device_only(ctx, 1 << 20)
        b.release()
    assert hip.active_buffer_count() == base


def test_map_read_roundtrip(ctx):
    host = np.arange(1000, dtype=np.float32)
    b = hip.HipBuffer.from_host(ctx, host)
    b.upload(np.full(10, -1.0, np.float32), offset=40)
    view = b.map_read()
    assert view is host and np.all(host[10:20] == -1.0) and host[9] == 9.0 and host[20] == 20.0
    b.unmap()
