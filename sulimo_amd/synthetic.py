"""Seeded random-init Q4_0 models and inputs of the shapes the benchmarks name.

The weights are in the loader's Q4_0 SoA split (crates/sulimo-core/src/loader.rs:141-160,
repack.rs:45-80): per tensor ``scales`` f16 [rows, cols/32] and ``quants`` u8
[rows, cols/32, 16]. Distributions: nibbles uniform 0..15, d uniform in
[0.002, 0.02] rounded to f16, norm weights 1 + N(0, 0.02) in f32, activations
f16 N(0, 1), token ids uniform in [0, vocab). Every tensor draws from its own
child stream of ``numpy.random.SeedSequence(seed)`` in declaration order.

With those distributions every weight has mean -0.5*d, so one layer collapses the
residual stream onto one position-independent direction and every position of a deep
model has the same top-1 token. ``make_model(..., zero_mean=True)`` draws the same
nibbles and scale magnitudes and gives each block's scale a random sign (the Q4_0
format allows any f16 d): zero-mean weights, position-dependent logits. At the
prescribed magnitudes every projection multiplies the RMS of its input by about
0.056 * sqrt(K) (2.2 at K = 1536), attention scores have a standard deviation near 5,
and the network amplifies rounding noise: moving 10 % of the input embeddings by one
f16 ulp moves the fp32 reference's own residual stream by up to 0.9 (max |g - r| /
max(|r|, 1)) after one layer. ``unit_gain=True`` scales each matrix's d range to
[a, 10a] with a = 1 / (sqrt(21.5 * 37) * sqrt(K)), so that its weights have RMS
1/sqrt(K) and the projection keeps the RMS of its input, as in a trained model
(E[(q-8)^2] = 21.5, E[d^2] = 37 a^2). The benchmark keeps the prescribed distribution;
the model-level parity tests use all three.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass(frozen=True)
class ModelConfig:
    """The ModelConfig fields the prefill reads (crates/sulimo-core/src/model_config.rs:59-80)."""
    n_layers: int
    embd: int
    ffn: int
    n_head: int
    n_head_kv: int
    head_dim: int
    rope_dim: int
    vocab: int
    rope_base: float
    eps: float
    rope_mode: int  # 0 = Norm (Llama), 1 = NeoX (Qwen2)

    @property
    def q_dim(self):
        return self.n_head * self.head_dim

    @property
    def kv_dim(self):
        return self.n_head_kv * self.head_dim

    @property
    def kv_bytes_per_pos(self):
        return self.n_head_kv * (self.head_dim // 32) * 34


# Qwen2.5-1.5B shape (28 layers, 1536 hidden, 12/2 heads, ffn 8960, vocab 151936, theta 1e6).
QWEN25_1_5B = ModelConfig(28, 1536, 8960, 12, 2, 128, 128, 151936, 1e6, 1e-6, 1)
# Llama-3.2-3B shape (28 layers, 3072 hidden, 24/8 heads, ffn 8192, vocab 128256, theta 5e5).
LLAMA32_3B = ModelConfig(28, 3072, 8192, 24, 8, 128, 128, 128256, 5e5, 1e-5, 0)


@dataclass
class Q4Tensor:
    scales: np.ndarray  # f16 [rows, cols/32]
    quants: np.ndarray  # u8 [rows, cols/32, 16]

    @property
    def rows(self):
        return self.scales.shape[0]

    @property
    def cols(self):
        return self.scales.shape[1] * 32

    def dequant_f32(self) -> np.ndarray:
        """W[rows, cols] = (q - 8) * d (repack.rs:107-131 element order)."""
        q = self.quants.astype(np.int16)
        lo = (q & 15) - 8
        hi = (q >> 4) - 8
        w = np.concatenate([lo, hi], axis=-1).astype(np.float32)  # [rows, nb, 32]
        w *= self.scales.astype(np.float32)[..., None]
        return w.reshape(self.rows, self.cols)


def random_q4(rng: np.random.Generator, rows: int, cols: int, d_lo=0.002, d_hi=0.02,
              signed: bool = False) -> Q4Tensor:
    """Nibbles uniform in 0..15, d uniform in [d_lo, d_hi] rounded to f16. signed gives
    every block's d a random sign, drawn after the nibbles, so the magnitudes and nibbles
    equal those of the unsigned draw from the same generator state."""
    assert cols % 32 == 0
    nb = cols // 32
    scales = rng.uniform(d_lo, d_hi, size=(rows, nb)).astype(np.float16)
    quants = np.frombuffer(rng.bytes(rows * nb * 16), dtype=np.uint8).reshape(rows, nb, 16).copy()
    if signed:
        scales = np.where(rng.integers(0, 2, size=(rows, nb)) == 1, -scales, scales).astype(np.float16)
    return Q4Tensor(scales, quants)


@dataclass
class HostLayer:
    attn_norm: np.ndarray
    q: Q4Tensor
    k: Q4Tensor
    v: Q4Tensor
    o: Q4Tensor
    ffn_norm: np.ndarray
    gate: Q4Tensor
    up: Q4Tensor
    down: Q4Tensor
    # Optional tensors of the CPU path (forward_pass.rs:250-272): f32 q/k/v biases
    # (Qwen2) and per-head RMSNorm weights of q and k (QK-norm), None when absent.
    q_bias: np.ndarray | None = None
    k_bias: np.ndarray | None = None
    v_bias: np.ndarray | None = None
    q_norm: np.ndarray | None = None
    k_norm: np.ndarray | None = None


@dataclass
class HostModel:
    cfg: ModelConfig
    token_embd: Q4Tensor
    output_norm: np.ndarray
    output: Q4Tensor
    layers: list = field(default_factory=list)


def _norm(rng, n):
    return (1.0 + rng.normal(0.0, 0.02, size=n)).astype(np.float32)


def unit_gain_d_range(cols: int):
    """d range [a, 10a] for Q4_0 weights of RMS 1/sqrt(cols): RMS(q - 8) = sqrt(21.5),
    RMS(d) = sqrt(37) * a for d uniform in [a, 10a]."""
    a = 1.0 / (np.sqrt(21.5 * 37.0) * np.sqrt(cols))
    return a, 10.0 * a


def make_model(cfg: ModelConfig, seed: int, tie_embeddings: bool = True, biases: bool = False,
               qk_norm: bool = False, zero_mean: bool = False, unit_gain: bool = False,
               exact_f16_weights: bool = False, qk_gain: float = 1.0) -> HostModel:
    """Random-init model. With tie_embeddings the LM head is token_embd (Qwen2.5
    ties them; the engine falls back to token_embd when output.weight is absent,
    crates/sulimo-engine/src/forward_pass.rs:58). biases adds q/k/v biases ~N(0, 0.5)
    and qk_norm per-head norm weights ~1+N(0, 0.1), from their own seed stream (the
    other tensors are the same as without them). zero_mean gives every Q4_0 block scale
    a random sign (same nibbles and magnitudes as without it); unit_gain (with zero_mean)
    scales every matrix's d range to unit_gain_d_range(cols). exact_f16_weights clears
    the low 3 mantissa bits of every d, so that every weight (q - 8) * d (at most 3
    significant bits times 8) is an exact f16 number: an f16-operand GEMM then uses the
    same weights as an f32 one. qk_gain multiplies the d range of the q and k projections
    (attention scores scale with its square)."""
    assert zero_mean or not unit_gain, "unit_gain needs zero_mean"
    ss = np.random.SeedSequence(seed)
    kids = iter(ss.spawn(4 + 9 * cfg.n_layers))
    rng = lambda: np.random.default_rng(next(kids))  # noqa: E731

    def q4(r, rows, cols, gain=1.0):
        lo, hi = unit_gain_d_range(cols) if unit_gain else (0.002, 0.02)
        t = random_q4(r, rows, cols, gain * lo, gain * hi, signed=zero_mean)
        if exact_f16_weights:
            t.scales = (t.scales.view(np.uint16) & np.uint16(0xFFF8)).view(np.float16)
        return t

    D, F = cfg.embd, cfg.ffn
    token_embd = q4(rng(), cfg.vocab, D)
    output_norm = _norm(rng(), D)
    out_rng = rng()
    output = token_embd if tie_embeddings else q4(out_rng, cfg.vocab, D)
    layers = []
    for _ in range(cfg.n_layers):
        layers.append(HostLayer(
            attn_norm=_norm(rng(), D), q=q4(rng(), cfg.q_dim, D, qk_gain), k=q4(rng(), cfg.kv_dim, D, qk_gain),
            v=q4(rng(), cfg.kv_dim, D), o=q4(rng(), D, cfg.q_dim), ffn_norm=_norm(rng(), D),
            gate=q4(rng(), F, D), up=q4(rng(), F, D), down=q4(rng(), D, F)))
    if biases or qk_norm:
        er = np.random.default_rng(np.random.SeedSequence([seed, 0xB1A5]))
        for L in layers:
            if biases:
                L.q_bias = er.normal(0.0, 0.5, cfg.q_dim).astype(np.float32)
                L.k_bias = er.normal(0.0, 0.5, cfg.kv_dim).astype(np.float32)
                L.v_bias = er.normal(0.0, 0.5, cfg.kv_dim).astype(np.float32)
            if qk_norm:
                L.q_norm = (1.0 + er.normal(0.0, 0.1, cfg.head_dim)).astype(np.float32)
                L.k_norm = (1.0 + er.normal(0.0, 0.1, cfg.head_dim)).astype(np.float32)
    return HostModel(cfg, token_embd, output_norm, output, layers)


def random_tokens(seed: int, n: int, vocab: int) -> np.ndarray:
    return np.random.default_rng(seed).integers(0, vocab, size=n, dtype=np.uint32)


def random_activations(seed: int, shape) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float16)


def embed_host(hm: HostModel, tokens: np.ndarray) -> np.ndarray:
    """f16 token embeddings as lookup_token_embedding_f16 (scheduler.rs:329-374):
    f16(d * (q - 8)) per element."""
    t = hm.token_embd
    rows = np.asarray(tokens, dtype=np.int64)
    q = t.quants[rows].astype(np.int16)
    w = np.concatenate([(q & 15) - 8, (q >> 4) - 8], axis=-1).astype(np.float32)
    w *= t.scales[rows].astype(np.float32)[..., None]
    return w.reshape(len(rows), hm.cfg.embd).astype(np.float16)
