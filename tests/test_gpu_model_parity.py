"""Model-level GPU parity on zero-mean weights, where the checks can fail.

On the prescribed weight distribution (nibbles uniform in 0..15, d > 0) every weight has
mean -0.5*d: one layer collapses the residual stream onto one position-independent
direction and every position has the same top-1 token, so model-level top-1 and logit
checks cannot see attention, RoPE or masking mistakes. These tests use the same Q4_0
format with a random sign on every block scale (``zero_mean``), in these variants:

* ``signed``: the prescribed magnitudes d in [0.002, 0.02]. Every projection multiplies
  the RMS of its input by about 2.2 and attention scores have a standard deviation near
  5: distinct top-1 tokens at 98 % of 2048 positions, and a network that amplifies
  rounding noise.
* ``unit_gain``: d ranges scaled so that every projection keeps the RMS of its input
  (as in a trained model); scores of standard deviation near 1. Well conditioned, but
  attention over many keys averages, so at full depth the top-1 tokens repeat across
  positions (21 % distinct); ``qk_gain=2`` sharpens attention (distinct top-1 tokens)
  at the price of conditioning.
* ``unit_gain_exact``: unit_gain with d rounded to 8 significant bits, so that every
  weight (q - 8) * d is an exact f16 number and the device's f16 MFMA operands equal the
  oracle's f32 weights. What is left between the two is the order of f32 sums, the f16
  attention window f16(code * d) against the oracle's f32 code * d, f16 softmax
  numerators, and the device's exp2/rcp/trig.

The noise floor. The fp32 oracle rounds to f16 at every GEMM input and output, as the
reference's own test oracle does (crates/sulimo-ocl/tests/test_prefill.rs:582-885); an
implementation that rounds one of those values differently by one ulp differs from it.
Each test runs the oracle twice: on the prompt's embeddings and on the same embeddings
with 10 % of the entries moved by one f16 ulp. How far the oracle moves by itself
(top-1 agreement, residual stream, normed rows, logits, K/V ring) is printed beside the
device's distance from it, and the device must stay within that floor: top-1 at 99.5 %
or at the floor less two sampling errors, distances within 1.5x (normwise) or 2x
(elementwise max |g - r| / max(|r|, 1), the metric of
crates/sulimo-ocl/tests/test_gemm.rs:45-57) of the oracle's own. At 28 layers the
oracle keeps 87 % of its own top-1 tokens on ``signed`` (its residual stream moves by
27 in that metric) and 98 % on ``unit_gain`` (0.36), so the fixed bar of 99.5 % top-1
at vocabulary 151936 is below every floor that informative data has; the fixed 1e-2
bars are checked normwise on the unit-gain models and for the last-token logits. A
mistake in attention, RoPE or masking moves top-1 agreement to a few percent (the
oracle with RoPE base 1e4 instead of 1e6 keeps 2-3 % of its top-1 tokens on
``unit_gain``), far outside any floor.

Each test checks that its data is not degenerate: the oracle's per-position argmax takes
distinct values at >= 90 % of positions where top-1 is the gate, and the
position-dependent part of the residual stream carries >= 1/3 of its norm where hidden
states are.

Op order: crates/sulimo-ocl/src/prefill.rs:362-560; gates of
crates/sulimo-ocl/tests/test_prefill.rs:829-885 (KV within one step, argmax, cosine).
"""
import dataclasses
import os

import numpy as np
import pytest

import oracle
from sulimo_amd import hip
from sulimo_amd import synthetic as S
from tests.helpers import cosine, kv_within_one_step, max_rel_err, normwise_err, ring_values, ulp_perturb

pytestmark = pytest.mark.gpu

QWEN = S.QWEN25_1_5B
T = 2048
VARIANTS = {
    "signed": dict(zero_mean=True),
    "unit_gain": dict(zero_mean=True, unit_gain=True),
    "unit_gain_exact": dict(zero_mean=True, unit_gain=True, exact_f16_weights=True),
}


def _threads():
    try:
        return max(1, min(16, len(os.sched_getaffinity(0))))
    except AttributeError:
        return max(1, min(16, os.cpu_count() or 1))


def _gaps(logits):
    """Top-1 minus top-2 logit of each row, in units of the row's logit std."""
    part = np.partition(logits, -2, axis=1)
    return (part[:, -1] - part[:, -2]) / np.std(logits, axis=1)


def _guard_distinct(arg, what):
    frac = len(set(np.asarray(arg).tolist())) / len(arg)
    print(f"{what}: oracle argmax distinct at {frac:.2%} of {len(arg)} positions", flush=True)
    assert frac >= 0.9, f"degenerate data: the oracle's top-1 takes {frac:.1%} distinct values"


def _ring_f16(ring, n, hkv, hd):
    """f16(code * f16(d)) of ring positions [0, n) as [hkv, n, hd] (kv_cache.rs layout)."""
    b = ring[:n * hkv * (hd // 32) * 34].reshape(n, hkv, hd // 32, 34)
    d = b[..., :2].copy().view(np.float16).astype(np.float32)
    codes = b[..., 2:].view(np.int8).astype(np.float32)
    return (codes * d).astype(np.float16).reshape(n, hkv, hd).transpose(1, 0, 2).copy()


def _vt_cols(n):
    """Stored column of window position j in a V^T row: slots 4-7 and 8-11 of every
    group of 16 swapped."""
    j = np.arange(n)
    s = j & 15
    return (j & ~15) + np.where(s & 4, np.where(s & 8, s, s + 4), np.where(s & 8, s - 4, s))


def _truncate(hm, n_layers):
    cfg = dataclasses.replace(hm.cfg, n_layers=n_layers)
    return S.HostModel(cfg, hm.token_embd, hm.output_norm, hm.output, hm.layers[:n_layers])


def _oracle_pair(hm, toks, cap):
    """The oracle on the prompt and on the one-ulp-perturbed prompt: (clean, perturbed),
    each (all logits, h_final, x_final, kv)."""
    x0 = S.embed_host(hm, toks)
    om = oracle.OracleModel(hm)
    out = []
    for x in (x0, ulp_perturb(x0)):
        kv = oracle.OracleKv(hm.cfg, cap)
        lg, h, xf = oracle.prefill_reference(om, kv, x, 0, all_logits=True, want_h=True, want_x=True)
        out.append((lg, h, xf, kv))
    return out


def _report(what, name, g_arg, g_last, g_x, g_h, clean, pert):
    """Device-vs-oracle and oracle-vs-oracle(perturbed) distances, printed side by side."""
    r_all, r_h, r_x, _ = clean
    p_all, p_h, p_x, _ = pert
    r_arg, p_arg = np.argmax(r_all, axis=1), np.argmax(p_all, axis=1)
    scale = float(np.abs(r_all[-1]).max())
    m = {
        "top1": (float(np.mean(g_arg == r_arg)), float(np.mean(p_arg == r_arg))),
        "x_max_rel": (max_rel_err(g_x, r_x), max_rel_err(p_x, r_x)),
        "x_norm": (normwise_err(g_x, r_x), normwise_err(p_x, r_x)),
        "h_max_rel": (max_rel_err(g_h, r_h), max_rel_err(p_h, r_h)),
        "h_norm": (normwise_err(g_h, r_h), normwise_err(p_h, r_h)),
        "logits": (float(np.max(np.abs(g_last - r_all[-1]))) / scale,
                   float(np.max(np.abs(p_all[-1] - r_all[-1]))) / scale),
    }
    gaps = _gaps(r_all)
    miss = np.nonzero(g_arg != r_arg)[0]
    print(f"{what} [{name}]: device vs oracle | oracle vs oracle on 1-ulp-perturbed input", flush=True)
    for k, (dv, fl) in m.items():
        print(f"    {k:9s} {dv:.4e} | {fl:.4e}", flush=True)
    print(f"    oracle top-2 gap in logit std: median {np.median(gaps):.4f}; at the device's "
          f"{miss.size} disagreements: median {np.median(gaps[miss]) if miss.size else 0:.5f}, "
          f"max {gaps[miss].max() if miss.size else 0:.5f}; last-token logits cos "
          f"{cosine(g_last, r_all[-1]):.6f}", flush=True)
    return m, r_arg


def _top1_bar(floor, n):
    """The top-1 bar: 99.5 %, or, where the oracle's own agreement under a one-ulp input
    change (floor) is lower, that floor less two of its sampling errors and one position."""
    return min(0.995, floor - 2.0 * np.sqrt(floor * (1.0 - floor) / n) - 1.0 / n)


def _check_floor(m, n):
    """The device within the oracle's own noise floor: top-1 at the bar above, distances
    at most twice the oracle's (normwise 1.5x), last logits within 1e-2 of scale or twice
    the floor."""
    assert m["top1"][0] >= _top1_bar(m["top1"][1], n)
    assert m["x_norm"][0] <= 1.5 * m["x_norm"][1]
    assert m["h_norm"][0] <= 1.5 * m["h_norm"][1]
    assert m["x_max_rel"][0] <= 2.0 * m["x_max_rel"][1]
    assert m["h_max_rel"][0] <= 2.0 * m["h_max_rel"][1]
    assert m["logits"][0] <= max(1e-2, 2.0 * m["logits"][1])


def _guard_spread(x, what):
    """Hidden states that differ by position: the part of x that varies over positions
    carries at least a third of its energy (on the prescribed weights it is below 1 %)."""
    x = np.asarray(x, dtype=np.float64)
    frac = float(np.linalg.norm(x - x.mean(axis=0)) / np.linalg.norm(x))
    print(f"{what}: position-dependent share of the residual stream {frac:.3f}", flush=True)
    assert frac >= 1.0 / 3.0, f"degenerate data: residual stream {frac:.3f} position-dependent"


def _device_prefill(ctx, hm, toks, cap, window_check=False):
    """One-ubatch device prefill: per-position top-1, last logits, scratch.x and scratch.h
    (f16 [n, embd]), and a copy of the K/V rings. window_check compares the kept f16
    attention window of every layer with the ring, bit for bit."""
    n, c = len(toks), hm.cfg
    dm = hip.DeviceModel(ctx, hm, cap, n)
    dm.embed(toks)
    ab = hip.HipBuffer.device_only(ctx, n * 4)
    dm.execute_prefill_ubatch(0, n, argmax_all=ab)
    out = dict(arg=ab.download(np.int32, (n,)), last=dm.logits(),
               x=dm.scratch_bufs["x"].download(np.float16, (n, c.embd)),
               h=dm.scratch_bufs["h"].download(np.float16, (n, c.embd)))
    dm.kv_sync_to_host(0, cap)
    out["k"], out["v"] = [a.copy() for a in dm.kv_host()[0]], [a.copy() for a in dm.kv_host()[1]]
    if window_check:
        # The f16 window the attention read, written by the q/k/v GEMM's RoPE + Q8_0 store
        # epilogue and kept for the next ubatch: every entry equals f16(code * f16(d)) of
        # the ring (K rows, and the transposed V in its stored column order).
        col = _vt_cols(n)
        for l in range(c.n_layers):
            wk, wvt, vlen = dm.kv_window(l)
            assert vlen == n
            want_k = _ring_f16(out["k"][l], n, c.n_head_kv, c.head_dim)
            want_v = _ring_f16(out["v"][l], n, c.n_head_kv, c.head_dim)
            assert np.array_equal(wk[:, :n].view(np.uint16), want_k.view(np.uint16)), f"K window of layer {l}"
            assert np.array_equal(wvt[:, :, col].view(np.uint16), want_v.transpose(0, 2, 1).view(np.uint16)), \
                f"V window of layer {l}"
    ab.release()
    dm.release()
    return out


def test_zero_mean_full_depth_2048(ctx):
    """Qwen2.5-1.5B shape at full depth (28 layers, vocab 151936), a 2048-token prompt in
    one ubatch, on the signed model (distinct top-1 tokens): per-position top-1 at all
    2048 positions, last-token logits, the final residual stream (scratch.x) and the
    output-normed rows (scratch.h) against the oracle, within its floor; the kept f16
    attention window of every layer bit-exact against the ring; K/V of the first layer
    within one Q8_0 step (deeper layers carry the floor)."""
    hm = S.make_model(QWEN, 40, **VARIANTS["signed"])
    toks = S.random_tokens(41, T, QWEN.vocab)
    print("full depth [signed]: device prefill of 2048 tokens, one ubatch", flush=True)
    g = _device_prefill(ctx, hm, toks, T, window_check=True)
    print("full depth [signed]: oracle prefill, clean and perturbed (all positions)", flush=True)
    clean, pert = _oracle_pair(hm, toks, T)
    m, r_arg = _report("full depth", "signed", g["arg"], g["last"], g["x"], g["h"], clean, pert)
    _guard_distinct(r_arg, "full depth [signed]")
    _check_floor(m, T)
    okv = clean[3]
    slots = np.arange(T)
    assert kv_within_one_step(g["k"][0], okv.k[0], slots, QWEN.kv_bytes_per_pos), "K of layer 0"
    assert kv_within_one_step(g["v"][0], okv.v[0], slots, QWEN.kv_bytes_per_pos), "V of layer 0"


@pytest.mark.parametrize("variant", ["unit_gain", "unit_gain_exact"])
def test_unit_gain_full_depth_hidden_states(ctx, variant):
    """The same full-depth prompt on the unit-gain models, whose floor is low enough for
    fixed bars: the final residual stream and the normed rows within 1e-2 normwise, the
    last-token logits within 1e-2 of their scale, every metric within the oracle's floor.
    (At this depth the unit-gain model's top-1 tokens repeat across positions, so top-1
    agreement is printed and held to the floor only.)"""
    hm = S.make_model(QWEN, 40, **VARIANTS[variant])
    toks = S.random_tokens(41, T, QWEN.vocab)
    g = _device_prefill(ctx, hm, toks, T)
    clean, pert = _oracle_pair(hm, toks, T)
    m, r_arg = _report("full depth", variant, g["arg"], g["last"], g["x"], g["h"], clean, pert)
    print(f"full depth [{variant}]: oracle argmax distinct at {len(set(r_arg.tolist())) / T:.2%}")
    _guard_spread(clean[2], f"full depth [{variant}]")
    _check_floor(m, T)
    assert m["x_norm"][0] <= 1e-2 and m["h_norm"][0] <= 1e-2
    assert m["logits"][0] <= 1e-2


@pytest.mark.parametrize("n_layers", [1, 2, 4])
def test_residual_after_layers(ctx, n_layers):
    """The residual stream after layer 1, 2 and 4 of the unit-gain model (cut there, so
    that the device's final scratch.x is that layer's output) and the output-normed rows
    against the oracle at all 2048 positions: within 1e-2 normwise, last logits within
    1e-2 of scale, and every metric within the oracle's floor."""
    hm = _truncate(S.make_model(QWEN, 40, **VARIANTS["unit_gain"]), n_layers)
    toks = S.random_tokens(41, T, QWEN.vocab)
    g = _device_prefill(ctx, hm, toks, T)
    clean, pert = _oracle_pair(hm, toks, T)
    m, r_arg = _report(f"{n_layers} layer(s)", "unit_gain", g["arg"], g["last"], g["x"], g["h"], clean, pert)
    print(f"{n_layers} layer(s): oracle argmax distinct at {len(set(r_arg.tolist())) / T:.2%}")
    _guard_spread(clean[2], f"{n_layers} layer(s)")
    _check_floor(m, T)
    assert m["logits"][0] <= 1e-2
    assert m["x_norm"][0] <= 1e-2 and m["h_norm"][0] <= 1e-2


def test_4_layers_vs_forward_token(ctx):
    """Device per-position top-1 against forward_token (the reference's CPU path,
    forward_pass.rs:190-417) at 512 positions of a 4-layer Qwen2.5-1.5B-width model with
    the full vocabulary (unit gain, q/k gain 2: peaked attention, distinct top-1 tokens).
    forward_token quantizes every matvec input to Q8_0 (kv_cache.rs:162-193); the device
    and the fp32 oracle do not, so both disagree with it at near-ties. The device must
    agree with forward_token as often as the fp32 oracle does (within the bar of the
    sampling error), and logits cosine >= 0.99 everywhere."""
    cfg = dataclasses.replace(QWEN, n_layers=4)
    n = 512
    hm = S.make_model(cfg, 50, **VARIANTS["unit_gain"], qk_gain=2.0)
    toks = S.random_tokens(51, n, cfg.vocab)
    dm = hip.DeviceModel(ctx, hm, n, n)
    dm.embed(toks)
    lb = hip.HipBuffer.device_only(ctx, n * cfg.vocab * 4)
    ab = hip.HipBuffer.device_only(ctx, n * 4)
    dm.execute_prefill_ubatch(0, n, logits_all=lb, argmax_all=ab)
    g_all = lb.download(np.float32, (n, cfg.vocab))
    g_arg = ab.download(np.int32, (n,))
    lb.release()
    ab.release()
    dm.release()
    assert np.array_equal(g_arg, np.argmax(g_all, axis=1))
    om = oracle.OracleModel(hm)
    r_all = oracle.prefill_reference(om, oracle.OracleKv(cfg, n), S.embed_host(hm, toks), 0, all_logits=True)
    r_arg = np.argmax(r_all, axis=1)
    _guard_distinct(r_arg, "forward_token")
    threads = _threads()
    print(f"forward_token: 512 positions on {threads} threads", flush=True)
    kv = oracle.OracleKv(cfg, n)
    f_all = np.stack([oracle.forward_token(om, kv, int(t), p, threads=threads) for p, t in enumerate(toks)])
    f_arg = np.argmax(f_all, axis=1)
    g_agree, r_agree = g_arg == f_arg, r_arg == f_arg
    gap_f = _gaps(f_all)
    cos = np.array([cosine(g_all[i], f_all[i]) for i in range(n)])
    cos_r = np.array([cosine(r_all[i], f_all[i]) for i in range(n)])
    print(f"forward_token: top-1 agreement with it: device {g_agree.mean():.4%}, fp32 oracle "
          f"{r_agree.mean():.4%}; device vs oracle {np.mean(g_arg == r_arg):.4%}; logits cosine with it "
          f"min/median: device {cos.min():.5f}/{np.median(cos):.6f}, oracle {cos_r.min():.5f}/"
          f"{np.median(cos_r):.6f}; forward_token top-2 gap in logit std: median {np.median(gap_f):.4f}, at "
          f"the device's disagreements {np.round(np.sort(gap_f[~g_agree]), 4).tolist()}", flush=True)
    assert cos.min() >= min(0.99, cos_r.min() - 0.005)
    assert np.median(cos) >= np.median(cos_r) - 1e-3
    assert g_agree.mean() >= _top1_bar(r_agree.mean(), n)


def test_resume_wrap_qwen_widths(ctx):
    """Edge resume at Qwen2.5-1.5B widths (hidden 1536, 12/2 heads, head_dim 128, FFN
    8960, 2 layers, vocab 32768 so that 2560 random top-1 tokens can be distinct;
    unit gain, q/k gain 2): three ubatches of 512, then 1024 new tokens into the
    capacity-2048 ring, which wrap at 2048 (staged K/V, sliding window of the last 2048
    positions). Every ubatch against the oracle run the same way: logits of all
    positions within 1e-2 of their scale or the oracle's floor, top-1 at the bar of the
    floor; at the end the first layer's ring within one Q8_0 step everywhere, the second
    layer's values (which carry the first layer's noise) within 1.5x the floor normwise."""
    cfg = dataclasses.replace(QWEN, n_layers=2, vocab=32768)
    hm = S.make_model(cfg, 60, **VARIANTS["unit_gain"], qk_gain=2.0)
    chunks = [512, 512, 512, 1024]
    toks = S.random_tokens(61, sum(chunks), cfg.vocab)
    cap = 2048
    dm = hip.DeviceModel(ctx, hm, cap, max(chunks))
    om = oracle.OracleModel(hm)
    okv, pkv = oracle.OracleKv(cfg, cap), oracle.OracleKv(cfg, cap)
    pos = 0
    args = []
    for m in chunks:
        t = toks[pos:pos + m]
        dm.embed(t)
        lb = hip.HipBuffer.device_only(ctx, m * cfg.vocab * 4)
        ab = hip.HipBuffer.device_only(ctx, m * 4)
        dm.execute_prefill_ubatch(pos, m, logits_all=lb, argmax_all=ab)
        g_all = lb.download(np.float32, (m, cfg.vocab))
        g_arg = ab.download(np.int32, (m,))
        lb.release()
        ab.release()
        x = S.embed_host(hm, t)
        r_all = oracle.prefill_reference(om, okv, x, pos, all_logits=True)
        p_all = oracle.prefill_reference(om, pkv, ulp_perturb(x, seed=pos), pos, all_logits=True)
        r_arg = np.argmax(r_all, axis=1)
        scale = float(np.abs(r_all).max())
        err = float(np.max(np.abs(g_all - r_all))) / scale
        floor_err = float(np.max(np.abs(p_all - r_all))) / scale
        agree = float(np.mean(g_arg == r_arg))
        floor = float(np.mean(np.argmax(p_all, axis=1) == r_arg))
        print(f"resume ubatch at {pos} (+{m}): logits max err {err:.3e} of scale (floor {floor_err:.3e}), "
              f"top-1 {agree:.4%} (floor {floor:.4%})", flush=True)
        assert err <= max(1e-2, 2.0 * floor_err)
        assert agree >= _top1_bar(floor, m)
        args.append(r_arg)
        pos += m
    _guard_distinct(np.concatenate(args), "resume")
    dm.kv_sync_to_host(0, cap)
    dk, dv = dm.kv_host()
    slots = np.arange(cap)
    assert kv_within_one_step(dk[0], okv.k[0], slots, dm.bpp), "K of layer 0"
    assert kv_within_one_step(dv[0], okv.v[0], slots, dm.bpp), "V of layer 0"
    for l in range(1, cfg.n_layers):
        for name, dev, ref, per in (("K", dk[l], okv.k[l], pkv.k[l]), ("V", dv[l], okv.v[l], pkv.v[l])):
            r = ring_values(ref, slots, dm.bpp)
            e_dev = normwise_err(ring_values(dev, slots, dm.bpp), r)
            e_floor = normwise_err(ring_values(per, slots, dm.bpp), r)
            print(f"resume ring {name} of layer {l}: normwise {e_dev:.3e} (floor {e_floor:.3e})", flush=True)
            assert e_dev <= 1.5 * e_floor, f"{name} of layer {l}"
    dm.release()
