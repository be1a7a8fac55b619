"""Shared comparison helpers and deterministic fills for the parity tests."""
import numpy as np


def max_rel_err(got, ref) -> float:
    """max |g - r| / max(|r|, 1): the reference's metric (crates/sulimo-ocl/tests/test_gemm.rs:45-57)."""
    g = np.asarray(got, dtype=np.float64).ravel()
    r = np.asarray(ref, dtype=np.float64).ravel()
    return float(np.max(np.abs(g - r) / np.maximum(np.abs(r), 1.0))) if g.size else 0.0


def cosine(a, b) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    return float(a @ b / (na * nb)) if na > 0 and nb > 0 else 0.0


def gemm_pattern_fill(m: int, k: int, n: int):
    """Deterministic fills of crates/sulimo-ocl/tests/test_gemm.rs:110-127 (m outputs,
    k inputs, n tokens): d = 0.05 + 0.01*(i%13), q = (3i)%16 | ((7i+1)%16) << 4,
    x = ((i%19) - 9) * 0.1."""
    nb = m * k // 32
    i = np.arange(nb)
    scales = (0.05 + 0.01 * (i % 13)).astype(np.float32).astype(np.float16).reshape(m, k // 32)
    j = np.arange(nb * 16)
    quants = (((3 * j) % 16) | ((((7 * j) + 1) % 16) << 4)).astype(np.uint8).reshape(m, k // 32, 16)
    t = np.arange(n * k)
    x = (((t % 19).astype(np.float32) - 9.0) * 0.1).astype(np.float16).reshape(n, k)
    return scales, quants, x


def prefill_act_fill(total: int) -> np.ndarray:
    """Activation fill of crates/sulimo-ocl/tests/test_prefill.rs:83-89:
    f16(5*sin(0.17 i) + ((i % 7) - 3))."""
    i = np.arange(total, dtype=np.float32)
    return (np.sin(i * np.float32(0.17)) * np.float32(5.0) + ((np.arange(total) % 7) - 3).astype(np.float32)).astype(np.float16)


def kv_within_one_step(dev_ring, ref_ring, slots, bpp):
    """test_prefill.rs:829-860 with an explicit error model. The device's K/V inputs differ
    from the oracle's by the GEMM's rounding (f16 weights), so block scales may differ by a
    few f16 ulps and codes by one step: codes within +-1, scales within 0.4 %, and every
    dequantized value within one step plus the scale mismatch on the largest code."""
    g = dev_ring.reshape(-1, bpp)[slots].reshape(-1, 34)
    r = ref_ring.reshape(-1, bpp)[slots].reshape(-1, 34)
    dg = g[:, :2].copy().view(np.float16).astype(np.float32)
    dr = r[:, :2].copy().view(np.float16).astype(np.float32)
    cg = g[:, 2:].view(np.int8).astype(np.int32)
    cr = r[:, 2:].view(np.int8).astype(np.int32)
    if np.abs(cg - cr).max() > 1:
        return False
    if np.any(np.abs(dg - dr) > 4e-3 * np.maximum(dr, 1e-30)):
        return False
    bound = 1.05 * np.maximum(dg, dr) + 127.0 * np.abs(dg - dr) + 1e-4
    return bool(np.all(np.abs(cg * dg - cr * dr) <= bound))


def ulp_perturb(x16, frac: float = 0.1, seed: int = 1):
    """Moves a random `frac` of the entries of an f16 array by one ulp (up or down at
    random): the input change used to measure how far the fp32 reference moves by
    itself, the noise floor of a model-level comparison."""
    x16 = np.asarray(x16, dtype=np.float16)
    rng = np.random.default_rng(seed)
    pick = rng.random(x16.shape) < frac
    toward = np.where(rng.random(x16.shape) < 0.5, np.float16(np.inf), np.float16(-np.inf))
    out = np.where(pick, np.nextafter(x16, toward), x16).astype(np.float16)
    assert np.all(np.isfinite(out))
    return out


def normwise_err(got, ref) -> float:
    """||g - r|| / ||r|| over all elements."""
    g = np.asarray(got, dtype=np.float64).ravel()
    r = np.asarray(ref, dtype=np.float64).ravel()
    return float(np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30))


def ring_values(ring, slots, bpp):
    """f32 values code * f16(d) of the Q8_0 ring blocks at `slots` (kv_cache.rs layout)."""
    b = np.asarray(ring).reshape(-1, bpp)[slots].reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)
    return b[:, 2:].view(np.int8).astype(np.float32) * d
