#!/usr/bin/env python3
"""Prefill benchmark on one MI355X: tokens/s of a full 2048-token prefill of a
random-init Qwen2.5-1.5B-shaped Q4_0 model (28 layers, hidden 1536, 12/2 heads,
head_dim 128, FFN 8960, vocab 151936, Q8_0 KV ring of 2048 positions, last-token
logits), plus the Q4_0 GEMM throughput at the one-layer M=512 shapes.

One step = device embedding gather of the 2048 prompt ids (2 bytes per token up) +
execute_prefill_ubatch (all 28 layers, final norm, LM head of the last token) ending in
its blocking wait + the read of the f32 last-token logits into their host mirror (the
engine's map_read after every prompt, crates/sulimo-engine/src/engine.rs:273-283): the
wall from the prompt upload to the logits on the host. Weights, KV ring and scratch are
resident in HBM before timing starts. The library replays each ubatch's launches from
captured HIP graphs (its default); extra.eager_launches is the same step with every
kernel launched one by one, extra.device_resident the step without the logits read.

Prints one JSON line. Before the W warm-up steps, untimed steps run for at least
half a second so that the GPU clock has left its idle state (counted under
extra.prewarm). `value` is the rate of K timed steps with nothing else on the
stream; extra.ubatch512 is the same prompt in the reference's default micro-batches
of 512 tokens, and extra.layer_m512_fused the per-layer time of their Q4_0 linears as
the prefill runs them (QKV with the RoPE + KV-store epilogue, o, gate/up with SwiGLU,
down with its residual + norm reduction). `roofline` is the Q4_0 GEMM kernel (the
dominant kernel: the gate/up projection with its SwiGLU epilogue; extra.gemm_all_roofline
is the same figure over every GEMM launch of the step, the definition `roofline` had
before it covered the dominant kernel alone), with its per-launch
GPU time taken from a hipEvent pair that each of its launches stamps with the kernel's
own start and end (hipExtLaunchKernelGGL) over K more identical steps (the other
launches of those steps sit between recorded events, which slow the steps, so they
are kept out of `value`); `traffic` is its HBM bytes per launch from the committed
rocprofv3 counter summary. `cpu_baseline` times the CPU oracle's restatement of the
reference forward_token (AVX2, one pinned core, plus an all-cores extension) on a
bounded sample of the same prompt.
extra.llama3b_4x4096 is the prefill rate of a Llama-3.2-3B-shaped model (28 layers,
hidden 3072, 24/8 heads, FFN 8192, vocab 128256) over 4 independent prompts of 4096
tokens, each in one ubatch on a ring of 4096 positions.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_F16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
PEAK_HBM_GBS = 8000.0
SEED_MODEL = 0x5EED0002
SEED_TOKENS = 0x5EED1002
METRIC = "prefill tokens/s (Qwen2.5-1.5B Q4_0, 2048 tok)"


PREWARM_S = 0.5


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--prompt", type=int, default=2048)
    ap.add_argument("--ubatch", type=int, default=2048)
    ap.add_argument("--cpu-sample", type=int, default=48, help="positions timed for the CPU baseline (0 = skip)")
    ap.add_argument("--no-gemm", action="store_true", help="skip the per-shape GEMM table")
    ap.add_argument("--no-llama", action="store_true", help="skip the Llama-3.2-3B 4 x 4096 prefill rate")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch every kernel one by one instead of replaying captured HIP graphs (for tools "
                         "that trace kernel dispatches)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB three times (the known-size "
                         "reference for FETCH_SIZE/WRITE_SIZE counter passes) and exit")
    return ap.parse_args()


def copy_calibration(mib: int):
    """Three device copies of `mib` MiB (torch's copy kernel), nothing else on the GPU."""
    import torch
    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "copies": 3}), flush=True)


def traffic_from_profiles(key: str):
    """HBM bytes (read + written) per launch of one kernel from the committed rocprofv3
    --pmc summary of the same workload, if present."""
    p = os.path.join(ROOT, "profiles", "gemm_q4_0_prefill2048_pmc.json")
    if not os.path.exists(p):
        return None
    try:
        with open(p) as f:
            return float(json.load(f)["hbm_bytes_per_launch"][key])
    except (OSError, ValueError, KeyError, TypeError):
        return None


def gemm_table(ctx, hip, S):
    """TFLOP/s of each Q4_0 linear of one Qwen2.5-1.5B layer at M=512, of the
    up-projection at M=128, 2048 and 4096 and of the Llama-3.2-3B up-projection at
    M=4096 (whole rounds of tiles: the kernel's rate without a partial last round),
    hipEvent-timed over 20 back-to-back launches."""
    rng = np.random.default_rng(0x5EED0001)
    shapes = [("q_proj", 512, 1536, 1536), ("k_proj", 512, 1536, 256), ("v_proj", 512, 1536, 256),
              ("o_proj", 512, 1536, 1536), ("gate_proj", 512, 1536, 8960), ("up_proj", 512, 1536, 8960),
              ("down_proj", 512, 8960, 1536), ("up_proj_m128", 128, 1536, 8960),
              ("up_proj_m2048", 2048, 1536, 8960), ("up_proj_m4096", 4096, 1536, 8960),
              ("llama3b_up_proj_m4096", 4096, 3072, 8192), ("lm_head_m1", 1, 1536, 151936)]
    out = {}
    tot_flop, tot_ms = 0.0, 0.0
    for name, M, K, N in shapes:
        w = S.random_q4(rng, N, K)
        x = rng.standard_normal((M, K)).astype(np.float16)
        bufs = [hip.HipBuffer.from_host(ctx, w.scales, True), hip.HipBuffer.from_host(ctx, w.quants, True),
                hip.HipBuffer.from_host(ctx, x, True), hip.HipBuffer.device_only(ctx, M * N * 2)]
        # warm: at least 30 ms of this shape, so that the clock has left the previous
        # shape's level
        ctx.wait()
        tw = time.perf_counter()
        while time.perf_counter() - tw < 0.03:
            for _ in range(10):
                hip.enqueue_gemm_q4_0_f16(ctx, *bufs, N, K, M)
            ctx.wait()
        it = 20
        ctx.timer_start()
        for _ in range(it):
            hip.enqueue_gemm_q4_0_f16(ctx, *bufs, N, K, M)
        ms = ctx.timer_stop() / it
        flop = 2.0 * M * N * K
        byts = N * K * 18 / 32 + 2 * M * K + 2 * M * N
        tf = flop / (ms * 1e-3) / 1e12
        out[name] = {"M": M, "K": K, "N": N, "us": round(ms * 1e3, 2), "tflops": round(tf, 1),
                     "frac_mfma_peak": round(tf / PEAK_F16_TFLOPS, 4),
                     "gbs": round(byts / (ms * 1e-3) / 1e9, 1)}
        if M == 512:
            tot_flop += flop
            tot_ms += ms
        for b in bufs:
            b.release()
    out["layer_m512_total"] = {"us": round(tot_ms * 1e3, 2), "tflops": round(tot_flop / (tot_ms * 1e-3) / 1e12, 1),
                               "frac_mfma_peak": round(tot_flop / (tot_ms * 1e-3) / 1e12 / PEAK_F16_TFLOPS, 4)}
    return out


def llama_rate(ctx, hip, S, T=4096, prompts=4):
    """Tokens/s of 4 independent 4096-token prefills (one ubatch each, ring of 4096) of a
    random-init Llama-3.2-3B-shaped Q4_0 model, after one untimed pass over the prompts."""
    cfg = S.LLAMA32_3B
    hm = S.make_model(cfg, 0x5EED0003)
    toks = [S.random_tokens(0x5EED1003 + i, T, cfg.vocab) for i in range(prompts)]
    dm = hip.DeviceModel(ctx, hm, capacity=T, max_n=T)

    def run():
        for tk in toks:
            dm.embed(tk)
            dm.execute_prefill_ubatch(0, T)
        ctx.wait()
    run()
    t0 = time.perf_counter()
    run()
    wall = time.perf_counter() - t0
    dm.release()
    return {"value": round(prompts * T / wall, 1), "unit": "tokens/s", "ms_per_prompt": round(wall / prompts * 1e3, 3),
            "config": f"llama-3.2-3b-shaped q4_0, {prompts} prompts x {T} tokens, one ubatch each, ring {T}, last-token logits"}


def cpu_baseline(hm, tokens, n_pos: int):
    """forward_token (crates/sulimo-engine/src/forward_pass.rs:190-417) restated in the
    oracle, on one pinned core: per-token time at n_pos evenly spaced positions of the
    prompt with a pre-filled Q8_0 ring; tokens/s = 1 / mean per-token time."""
    import oracle
    cfg = hm.cfg
    allowed = sorted(os.sched_getaffinity(0))
    cpu = allowed[0]
    os.sched_setaffinity(0, {cpu})
    om = oracle.OracleModel(hm)
    cap = len(tokens)
    rng = np.random.default_rng(7)
    ring = lambda: oracle.quantize_f32_to_q8_0(rng.standard_normal(cap * cfg.kv_dim).astype(np.float32))  # noqa: E731
    kv = oracle.OracleKv(cfg, cap, k=[ring() for _ in range(cfg.n_layers)], v=[ring() for _ in range(cfg.n_layers)])
    pos = [int(p) for p in np.linspace(0, cap - 1, n_pos).round()]
    oracle.forward_token(om, kv, int(tokens[pos[0]]), pos[0])  # warm caches / page in weights
    times = []
    for p in pos:
        t0 = time.perf_counter()
        oracle.forward_token(om, kv, int(tokens[p]), p)
        times.append(time.perf_counter() - t0)
    mean = float(np.mean(times))
    # Extension: every matvec's rows split over the usable cores (at most 16, the box's
    # CPU share), as the reference's ThreadPool::execute_parallel splits them.
    os.sched_setaffinity(0, set(allowed))
    threads = max(1, min(16, len(allowed)))
    t0 = time.perf_counter()
    for p in pos:
        oracle.forward_token(om, kv, int(tokens[p]), p, threads=threads)
    mean_mt = (time.perf_counter() - t0) / len(pos)
    return {"value": round(1.0 / mean, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
            "cpu_model": cpu_model(), "usable_cpus": len(allowed),
            "sample": f"forward_token (AVX2 Q4_0.Q8_0, per-token LM head) at {n_pos} evenly spaced positions "
                      f"of the {cap}-token prompt on a pre-filled Q8_0 ring, 1 pinned core; "
                      f"mean {mean * 1e3:.1f} ms/token, est. full prefill {mean * cap:.1f} s",
            "all_cores": {"value": round(1.0 / mean_mt, 3), "unit": "tokens/s", "threads": threads,
                          "note": "extension: the same positions with every matvec's rows split over the "
                                  f"threads; mean {mean_mt * 1e3:.1f} ms/token"}}


def cpu_model() -> str:
    """The host CPU's model name (first processor in /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    a = parse()
    if a.copy_calibration:
        copy_calibration(a.copy_calibration)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only: the prefill path runs on a single MI355X "
              f"(requested --gpus {a.gpus}, WORLD_SIZE {world}); multi-GPU runs are not part of this build.",
              file=sys.stderr)
        sys.exit(2)

    from sulimo_amd import hip
    from sulimo_amd import synthetic as S

    cfg = S.QWEN25_1_5B
    T = a.prompt
    ctx = hip.HipContext.get_or_init(0)
    ctx.set_graph_replay(not a.no_graph)
    hm = S.make_model(cfg, SEED_MODEL)
    tokens = S.random_tokens(SEED_TOKENS, T, cfg.vocab)
    dm = hip.DeviceModel(ctx, hm, capacity=T, max_n=min(a.ubatch, T))

    logits_buf = dm.scratch_bufs["logits"]

    def step(read_logits=True):
        pos = 0
        while pos < T:
            m = min(a.ubatch, T - pos)
            dm.embed(tokens[pos:pos + m])
            dm.execute_prefill_ubatch(pos, m)
            pos += m
        if read_logits:
            logits_buf.map_read()  # blocking D2H of the last-token logits into the host mirror
            logits_buf.unmap()

    def timed_steps(**kw):
        ctx.wait()
        t = time.perf_counter()
        for _ in range(a.steps):
            step(**kw)
        ctx.wait()
        return time.perf_counter() - t

    # The GPU clock ramps up from idle over a few hundred ms: untimed steps for at least
    # PREWARM_S (counted in the output) before the W warm-up steps proper.
    prewarm_steps, tp = 0, time.perf_counter()
    while prewarm_steps == 0 or time.perf_counter() - tp < PREWARM_S:
        step()
        ctx.wait()
        prewarm_steps += 1
    for _ in range(a.warmup):
        step()
    ctx.wait()

    # Timed region: K steps, nothing but the prefill on the stream.
    wall = timed_steps()
    ms_per_step = wall / a.steps * 1e3
    value = T * a.steps / wall
    # The same steps without the logits read, and with eager launches instead of replay.
    wall_dev = timed_steps(read_logits=False)
    ctx.set_graph_replay(False)
    for _ in range(a.warmup):
        step()
    wall_eager = timed_steps()
    ctx.set_graph_replay(not a.no_graph)

    # Kernel timing: the same K steps again with a hipEvent pair per launch on the
    # library's stream. The GEMM kernels stamp their pair with their own start and end
    # (hipExtLaunchKernel); the other launches sit between event records, which add gaps
    # between kernels, so these steps are slower and are not `value`.
    ctx.set_profiling(True)
    ctx.wait()
    t1 = time.perf_counter()
    for _ in range(a.steps):
        step()
    ctx.wait()
    wall_ev = time.perf_counter() - t1
    st = ctx.prefill_stats()
    ctx.set_profiling(False)

    # The dominant kernel: the gate/up GEMM with the SwiGLU epilogue (one launch per layer,
    # 2*M*(2*ffn)*hidden FLOPs each, the largest share of the step).
    g = st.gemm_gate_up
    gu_us = g.total_ms / max(g.launches, 1) * 1e3
    gu_flop = g.flop / max(g.launches, 1)
    gu_tf = gu_flop / (gu_us * 1e-6) / 1e12 if gu_us > 0 else 0.0
    roofline = {"kernel": "gemm_q4_kernel, gate/up projection with the SwiGLU epilogue "
                          f"(M={min(a.ubatch, T)} tokens, N=2x{cfg.ffn}, K={cfg.embd})",
                "bound": "mfma", "achieved": round(gu_tf, 2), "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(gu_tf / PEAK_F16_TFLOPS, 4), "traffic": traffic_from_profiles("gate_up"),
                "launches_per_step": int(g.launches // max(a.steps, 1)), "avg_launch_us": round(gu_us, 2),
                "flop_per_launch": gu_flop,
                "timing": f"hipEvent pair stamped by every gate/up kernel (hipExtLaunchKernel) over "
                          f"{a.steps} further identical steps ({wall_ev / a.steps * 1e3:.3f} ms/step "
                          f"with the per-launch events)"}

    def cls(k):
        return {"ms_per_step": round(k.total_ms / a.steps, 3), "launches_per_step": int(k.launches // a.steps),
                "tflops": round(k.flop / (k.total_ms * 1e-3) / 1e12, 2) if k.total_ms > 0 and k.flop > 0 else None,
                "frac_mfma_peak": round(k.flop / (k.total_ms * 1e-3) / 1e12 / PEAK_F16_TFLOPS, 4)
                if k.total_ms > 0 and k.flop > 0 else None,
                "gbs": round(k.bytes / (k.total_ms * 1e-3) / 1e9, 1) if k.total_ms > 0 else None}

    gall = st.gemm
    gall_tf = gall.flop / (gall.total_ms * 1e-3) / 1e12 if gall.total_ms > 0 else 0.0
    extra = {"device_resident": {"value": round(T * a.steps / wall_dev, 1), "unit": "tokens/s",
                                 "ms_per_step": round(wall_dev / a.steps * 1e3, 3),
                                 "note": "the step without the last-token logits read"},
             "eager_launches": {"value": round(T * a.steps / wall_eager, 1), "unit": "tokens/s",
                                "ms_per_step": round(wall_eager / a.steps * 1e3, 3),
                                "note": "the step with graph replay off (every kernel launched one by one)"},
             "gemm_all_roofline": {"achieved": round(gall_tf, 2), "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                                   "frac": round(gall_tf / PEAK_F16_TFLOPS, 4),
                                   "launches_per_step": int(gall.launches // max(a.steps, 1)),
                                   "note": "every Q4_0 GEMM launch of the step (QKV, o, gate/up, down with "
                                           "their K-split reductions, LM head), stamped kernel times"},
             "kernel_classes": {"gemm": cls(st.gemm), "gemm_qkv": cls(st.gemm_qkv), "gemm_o": cls(st.gemm_o),
                                "gemm_gate_up": cls(st.gemm_gate_up), "gemm_down": cls(st.gemm_down),
                                "gemm_lm_head": cls(st.gemm_lm_head), "attention": cls(st.attention),
                                "norm": cls(st.norm), "rope_kv": cls(st.rope_kv),
                                "note": "GEMM classes: the kernels' own start-to-end times (stamped "
                                        "events); split GEMMs (o, down) run from the partial-sum kernel's "
                                        "start to the K-split reduction's end, gap included. Other classes: "
                                        "event records around the launch, which add a dispatch gap each"},
             "value_with_event_records": round(T * a.steps / wall_ev, 1),
             "prewarm": {"steps": prewarm_steps, "min_seconds": PREWARM_S},
             "device": ctx.device_info.arch_name.decode()}
    # The same prompt in the reference's default micro-batch of 512 tokens.
    if a.ubatch != 512 and T > 512:
        def step512():
            for pos in range(0, T, 512):
                m = min(512, T - pos)
                dm.embed(tokens[pos:pos + m])
                dm.execute_prefill_ubatch(pos, m)
            logits_buf.map_read()
            logits_buf.unmap()
        for _ in range(a.warmup):
            step512()
        ctx.wait()
        t2 = time.perf_counter()
        for _ in range(a.steps):
            step512()
        ctx.wait()
        w512 = time.perf_counter() - t2
        extra["ubatch512"] = {"value": round(T * a.steps / w512, 1), "unit": "tokens/s",
                              "ms_per_step": round(w512 / a.steps * 1e3, 3),
                              "config": f"the {T}-token prompt in {-(-T // 512)} micro-batches of 512"}
        # The layer's linears at M=512 as the prefill runs them (QKV in one launch with the
        # RoPE + KV-store epilogue, o with the residual, gate/up with SwiGLU, down split
        # with its residual + RMSNorm reduction), per-launch events over the same steps.
        ctx.set_profiling(True)
        ctx.wait()
        for _ in range(a.steps):
            step512()
        ctx.wait()
        s5 = ctx.prefill_stats()
        ctx.set_profiling(False)
        n_layer_runs = a.steps * -(-T // 512) * cfg.n_layers
        us = s5.gemm.total_ms * 1e3 / n_layer_runs
        fl = 2.0 * 512 * cfg.embd * (cfg.q_dim + 2 * cfg.kv_dim + cfg.q_dim + 2 * cfg.ffn) + 2.0 * 512 * cfg.ffn * cfg.embd
        extra["layer_m512_fused"] = {
            "us": round(us, 2), "tflops": round(fl / (us * 1e-6) / 1e12, 1),
            "frac_mfma_peak": round(fl / (us * 1e-6) / 1e12 / PEAK_F16_TFLOPS, 4),
            "note": "GEMM-class time of the 512-token micro-batches per layer (includes the "
                    "last-token LM head once per micro-batch, about 1 %)"}
    if not a.no_gemm:
        extra["gemm_shapes"] = gemm_table(ctx, hip, S)
    dm.release()
    if not a.no_llama:
        extra["llama3b_4x4096"] = llama_rate(ctx, hip, S)

    cpu = None
    if a.cpu_sample > 0:
        cpu = cpu_baseline(hm, tokens, a.cpu_sample)

    line = {"metric": METRIC, "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1, "steps": a.steps,
            "warmup": a.warmup, "ms_per_step": round(ms_per_step, 3), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f16",
            "data": "synthetic: random-init Qwen2.5-1.5B-shaped Q4_0 weights (nibbles uniform, d~U[0.002,0.02]), "
                    "uniform token ids",
            "config": {"workload": f"qwen2.5-1.5b-shaped q4_0 prefill, {T}-token prompt, batch 1, last-token logits",
                       "layers": cfg.n_layers, "hidden": cfg.embd, "heads": f"{cfg.n_head}/{cfg.n_head_kv}",
                       "ffn": cfg.ffn, "vocab": cfg.vocab, "kv_cache": f"q8_0 ring, capacity {T}",
                       "ubatch": a.ubatch, "prompt_tokens": T},
            "roofline": roofline, "cpu_baseline": cpu, "extra": extra}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
