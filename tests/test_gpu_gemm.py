"""GPU parity of the Q4_0 x f16 GEMM (sulimo_hip_enqueue_gemm_q4_0_f16 and the
timed sulimo_hip_gemm_q4_0_f16) against the oracle and an fp32 reference.

Mirrors crates/sulimo-ocl/tests/test_gemm.rs:59-216 (shapes, fills, max rel err
<= 2e-3 with denominator max(|ref|,1), cosine >= 0.9999) and adds the benchmark
shapes (M tokens x K x N outputs) with the 1e-2 bound against fp32.
"""
import numpy as np
import pytest

import oracle
from sulimo_amd import hip
from sulimo_amd import synthetic as S
from tests.helpers import cosine, gemm_pattern_fill, max_rel_err

pytestmark = pytest.mark.gpu


def run_gemm(ctx, scales, quants, x, m_out, k, n_tok):
    sb = hip.HipBuffer.from_host(ctx, np.ascontiguousarray(scales), True)
    qb = hip.HipBuffer.from_host(ctx, np.ascontiguousarray(quants), True)
    xb = hip.HipBuffer.from_host(ctx, np.ascontiguousarray(x), True)
    ob = hip.HipBuffer.device_only(ctx, max(n_tok, 1) * m_out * 2)
    hip.enqueue_gemm_q4_0_f16(ctx, sb, qb, xb, ob, m_out, k, n_tok)
    ctx.wait()
    y = ob.download(np.float16, (n_tok, m_out))
    for b in (sb, qb, xb, ob):
        b.release()
    return y


def test_dequant_bit_exact_one_hot(ctx):
    """One-hot activations make Y = W^T exactly: every Q4_0 code, nibble position
    and scale (incl. f16-subnormal scales) must dequantize to f16((q-8)*d) bit for
    bit (repack.rs:107-131 semantics)."""
    rng = np.random.default_rng(11)
    m_out, k = 256, 256
    w = S.random_q4(rng, m_out, k)
    special = np.array([2.0 ** -20, 2.0 ** -24, 6.1e-5, 1.0, 1000.0], np.float32).astype(np.float16)
    w.scales.ravel()[: special.size] = special
    # every byte value appears in the first 16 blocks
    w.quants.reshape(-1, 16)[:16] = np.arange(256, dtype=np.uint8).reshape(16, 16)
    x = np.eye(k, dtype=np.float16)  # token t = e_t
    y = run_gemm(ctx, w.scales, w.quants, x, m_out, k, k)
    deq = oracle.dequant_q4_0_soa(w.scales, w.quants).reshape(m_out, k)
    want = deq.T.astype(np.float16)
    assert np.array_equal(y.view(np.uint16), want.view(np.uint16))


def f16_weight_bound(x, scales, quants, ref):
    """Error model of the MFMA path: each weight is dequantized once to f16 (unit roundoff
    u = 2^-11) before an f32-accumulated f16 MFMA, so |y - ref| <= u * (|X| @ |W|^T). A K
    split across workgroups stores each partial sum p_s once as f16 before the f32 sum,
    adding at most u * sum_s |p_s| <= u * (|X| @ |W|^T); then one f16 ulp of the output
    rounding. The f32 accumulation error (~K * 2^-24) is below it."""
    w = np.abs(oracle.dequant_q4_0_soa(scales, quants).reshape(scales.shape[0], -1)).astype(np.float64)
    s = np.abs(x.astype(np.float64)) @ w.T
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    return 2.0 * 2.0 ** -11 * s + ulp + 1e-6


@pytest.mark.parametrize("n_tok,k,m_out", [(8, 256, 256), (32, 512, 512), (128, 512, 1024), (512, 1024, 1024)])
def test_reference_patterns(ctx, n_tok, k, m_out):
    """test_gemm.rs:75-214 shapes and fills against gemm_q4_0_f16_scalar_reference.
    The reference's own 2e-3 gate assumes f32 weights; these fills cancel heavily
    (outputs near 0 from sums of +-1 terms), so the check is the f16-weight error
    model above, plus the 1e-2 bound and the reference's cosine >= 0.9999."""
    scales, quants, x = gemm_pattern_fill(m_out, k, n_tok)
    y = run_gemm(ctx, scales, quants, x, m_out, k, n_tok)
    ref = oracle.gemm_q4_0_f16_scalar_reference(scales, quants, x, m_out, k, n_tok)
    err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
    assert np.all(err <= f16_weight_bound(x, scales, quants, ref))
    assert max_rel_err(y, ref) <= 1e-2
    assert cosine(y, ref) >= 0.9999


SHAPES = {  # (K, N) of the Qwen2.5-1.5B layer linears, and the Llama-3.2-3B QKV
    "q_o": (1536, 1536), "k_v": (1536, 256), "gate_up": (1536, 8960), "down": (8960, 1536),
    "l3b_qkv": (3072, 5120),
}


EDGE_M = (37, 1000, 3071)  # the non-tile-multiple token counts of the edge-shape stress


@pytest.mark.parametrize("M,name", [(128, "gate_up"), (512, "q_o"), (512, "k_v"), (512, "gate_up"),
                                    (512, "down"), (1, "down"), (8, "q_o"), (1536, "down"),
                                    (1536, "l3b_qkv")]
                         + [(M, name) for M in EDGE_M for name in ("q_o", "k_v", "gate_up", "down")])
def test_benchmark_shapes_vs_fp32(ctx, M, name):
    """Benchmark shapes (nibbles uniform, d in [0.002, 0.02], x ~ N(0,1)) against an
    fp32 reference: max rel err <= 1e-2 (denominator max(|ref|,1)). The shapes cover the
    planner's tiles: 32 x 128 with four K parts inside the workgroup (M <= 512 q/o/k/v),
    64 x 128 with and without two parts (gate/up at M = 128 and 512, q/o at M = 1000),
    K splits across workgroups (down at M = 512), and 128 x 256 with two parts (down,
    also split across workgroups, and the Llama QKV at M = 1536). All four layer shapes
    run at each of M = 37, 1000 and 3071, where the last token tile is partly empty."""
    K, N = SHAPES[name]
    rng = np.random.default_rng(1000 + M + K + N)
    w = S.random_q4(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float16)
    y = run_gemm(ctx, w.scales, w.quants, x, N, K, M)
    ref = x.astype(np.float32) @ w.dequant_f32().T
    assert max_rel_err(y, ref) <= 1e-2
    assert cosine(y, ref) >= 0.9999


@pytest.mark.parametrize("M,K,N", [(4096, 1536, 8960), (4000, 1536, 8864), (4096, 3072, 8192), (1920, 1536, 8960)])
def test_persistent_tile_chain(ctx, M, K, N):
    """Shapes with more tiles than the GPU holds at once and k stages a multiple of the
    3-slot ring (24 and 48): the launch keeps only resident workgroups, each running a
    strided run of its XCD's tiles and loading the next tile's first stages under the
    current tile's epilogue. The second shape has ragged rows and columns; the last has
    only slightly more tiles than resident workgroups and XCD ranges of unequal length,
    so most workgroups run one tile and a few chain two. Against fp32 within 1e-2."""
    rng = np.random.default_rng(9000 + M + K + N)
    w = S.random_q4(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float16)
    y = run_gemm(ctx, w.scales, w.quants, x, N, K, M)
    ref = x.astype(np.float32) @ w.dequant_f32().T
    assert max_rel_err(y, ref) <= 1e-2
    assert cosine(y, ref) >= 0.9999


@pytest.mark.parametrize("M", [1, 8, 37])
def test_lm_head_shape(ctx, M):
    """LM-head GEMM K=1536, N=151936 at small M (the HBM-bound regime)."""
    K, N = 1536, 151936
    rng = np.random.default_rng(77 + M)
    w = S.random_q4(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float16)
    y = run_gemm(ctx, w.scales, w.quants, x, N, K, M)
    ref = x.astype(np.float32) @ w.dequant_f32().T
    assert max_rel_err(y, ref) <= 1e-2


@pytest.mark.parametrize("n_tok,k,m_out", [(8, 96, 40), (33, 800, 72), (130, 2080, 264)])
def test_odd_block_counts_and_ragged_rows(ctx, n_tok, k, m_out):
    """K = 32 * odd (the GEMM's last 64-wide k stage holds one block) and row counts
    that do not fill the 32-row weight panels: against the oracle's scalar reference
    with the f16-weight error model, and against fp32 within 1e-2."""
    rng = np.random.default_rng(5000 + k + m_out)
    w = S.random_q4(rng, m_out, k)
    x = rng.standard_normal((n_tok, k)).astype(np.float16)
    y = run_gemm(ctx, w.scales, w.quants, x, m_out, k, n_tok)
    ref = oracle.gemm_q4_0_f16_scalar_reference(w.scales, w.quants, x, m_out, k, n_tok)
    err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
    assert np.all(err <= f16_weight_bound(x, w.scales, w.quants, ref))
    assert max_rel_err(y, x.astype(np.float32) @ w.dequant_f32().T) <= 1e-2


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("k,m_out", [(800, 72), (1536, 256), (96, 40)])
def test_gemv_small_m(ctx, M, k, m_out):
    """Up to 4 tokens take the GEMV (no MFMA): odd block counts and ragged rows against
    the oracle's scalar reference with the f16-weight error model, and fp32 within 1e-2."""
    rng = np.random.default_rng(9000 + M * 7 + k + m_out)
    w = S.random_q4(rng, m_out, k)
    x = rng.standard_normal((M, k)).astype(np.float16)
    y = run_gemm(ctx, w.scales, w.quants, x, m_out, k, M)
    ref = oracle.gemm_q4_0_f16_scalar_reference(w.scales, w.quants, x, m_out, k, M)
    err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
    assert np.all(err <= f16_weight_bound(x, w.scales, w.quants, ref))
    assert max_rel_err(y, x.astype(np.float32) @ w.dequant_f32().T) <= 1e-2


@pytest.mark.parametrize("M", [1, 2, 4])
def test_gemv_one_hot_bit_exact(ctx, M):
    """GEMV dequant is bit-exact: token t = e_(3t+1) reads column 3t+1 of W^T exactly."""
    rng = np.random.default_rng(31 + M)
    m_out, k = 96, 160
    w = S.random_q4(rng, m_out, k)
    w.quants.reshape(-1, 16)[:16] = np.arange(256, dtype=np.uint8).reshape(16, 16)
    x = np.zeros((M, k), np.float16)
    cols = [3 * t + 1 for t in range(M)]
    for t, c in enumerate(cols):
        x[t, c] = 1.0
    y = run_gemm(ctx, w.scales, w.quants, x, m_out, k, M)
    deq = oracle.dequant_q4_0_soa(w.scales, w.quants).reshape(m_out, k)
    assert np.array_equal(y.view(np.uint16), deq[:, cols].T.astype(np.float16).view(np.uint16))


def test_panel_copy_follows_uploads(ctx):
    """The GEMM reads a panel copy of the weights built from the SoA buffers on first
    use; overwriting the buffers must be seen by the next GEMM (bit-exact one-hot
    readback before and after)."""
    rng = np.random.default_rng(21)
    m_out, k = 64, 128
    w1, w2 = S.random_q4(rng, m_out, k), S.random_q4(rng, m_out, k)
    sb = hip.HipBuffer.from_host(ctx, w1.scales, True)
    qb = hip.HipBuffer.from_host(ctx, w1.quants, True)
    xb = hip.HipBuffer.from_host(ctx, np.eye(k, dtype=np.float16), True)
    ob = hip.HipBuffer.device_only(ctx, k * m_out * 2)
    got = []
    for w in (w1, w2):
        sb.upload(w.scales)
        qb.upload(w.quants)
        hip.enqueue_gemm_q4_0_f16(ctx, sb, qb, xb, ob, m_out, k, k)
        ctx.wait()
        got.append(ob.download(np.float16, (k, m_out)))
    for b in (sb, qb, xb, ob):
        b.release()
    for w, y in zip((w1, w2), got):
        want = oracle.dequant_q4_0_soa(w.scales, w.quants).reshape(m_out, k).T.astype(np.float16)
        assert np.array_equal(y.view(np.uint16), want.view(np.uint16))


def test_timed_gemm_profile(ctx):
    """gemm_q4_0_f16 (gemm.rs:28-102): waited launch with a GPU-time profile."""
    scales, quants, x = gemm_pattern_fill(1024, 1024, 512)
    sb = hip.HipBuffer.from_host(ctx, scales, True)
    qb = hip.HipBuffer.from_host(ctx, quants, True)
    xb = hip.HipBuffer.from_host(ctx, x, True)
    ob = hip.HipBuffer.device_only(ctx, 512 * 1024 * 2)
    p = hip.gemm_q4_0_f16(ctx, sb, qb, xb, ob, 1024, 1024, 512)
    assert p.duration_seconds > 0 and p.gflops > 0
    y = ob.download(np.float16, (512, 1024))
    ref = oracle.gemm_q4_0_f16_scalar_reference(scales, quants, x, 1024, 1024, 512)
    err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
    assert np.all(err <= f16_weight_bound(x, scales, quants, ref))


def test_gemm_rejects_bad_shapes(ctx):
    """gemm.rs:39-40 asserts K % 32 == 0 and M % 8 == 0; undersized buffers are
    rejected on the host before any launch."""
    scales, quants, x = gemm_pattern_fill(64, 64, 4)
    sb = hip.HipBuffer.from_host(ctx, scales, True)
    qb = hip.HipBuffer.from_host(ctx, quants, True)
    xb = hip.HipBuffer.from_host(ctx, x, True)
    ob = hip.HipBuffer.device_only(ctx, 4 * 64 * 2)
    with pytest.raises(hip.HipError) as e:
        hip.enqueue_gemm_q4_0_f16(ctx, sb, qb, xb, ob, 64, 48, 4)
    assert e.value.code == hip.ERR_INVALID_ARGUMENT
    with pytest.raises(hip.HipError) as e:
        hip.enqueue_gemm_q4_0_f16(ctx, sb, qb, xb, ob, 60, 64, 4)
    assert e.value.code == hip.ERR_INVALID_ARGUMENT
    with pytest.raises(hip.HipError) as e:
        hip.enqueue_gemm_q4_0_f16(ctx, sb, qb, xb, ob, 64, 64, 8)  # x and out too small
    assert e.value.code == hip.ERR_INVALID_ARGUMENT
