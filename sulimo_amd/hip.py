"""ctypes binding of libsulimo_hip.so, mirroring the public API of the
reference's ``sulimo-ocl`` crate (crates/sulimo-ocl/src/lib.rs:15-29):
contexts, zero-copy-style buffers, ``enqueue_*`` ops, ``gemm_q4_0_f16``,
``execute_prefill_ubatch`` and the waiter.

Errors follow ``OclError`` (crates/sulimo-ocl/src/program.rs:27-40): every
failing call raises :class:`HipError` carrying the C status code and message.
The library must be built (``python -m sulimo_amd.build``); there is no
fallback path, a missing library raises at import of this module's ``lib()``.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsulimo_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "sulimo_hip.h")

OK = 0
ERR_DEVICE_NOT_FOUND = -1
ERR_DRIVER = -2
ERR_BUILD_FAILED = -3
ERR_ZERO_COPY = -4
ERR_EXECUTION_FAILED = -5
ERR_IO = -6
ERR_INVALID_ARGUMENT = -7

_ERR_NAMES = {
    ERR_DEVICE_NOT_FOUND: "DeviceNotFound", ERR_DRIVER: "Driver", ERR_BUILD_FAILED: "BuildFailed",
    ERR_ZERO_COPY: "ZeroCopyViolation", ERR_EXECUTION_FAILED: "ExecutionFailed", ERR_IO: "Io",
    ERR_INVALID_ARGUMENT: "InvalidArgument",
}


class HipError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{_ERR_NAMES.get(code, code)}: {message}")
        self.code = code
        self.message = message


_lib = None


def lib():
    """Loads libsulimo_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HipError(ERR_BUILD_FAILED, f"{LIB_PATH} is missing; run python -m sulimo_amd.build")
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def header_functions() -> list[str]:
    """Names of the functions declared in include/sulimo_hip.h."""
    text = open(HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sulimo_hip_[a-z0-9_]+)\s*\(", text)))


# ---- structs (include/sulimo_hip.h) ----

class DeviceInfo(C.Structure):
    _fields_ = [("device_name", C.c_char * 256), ("arch_name", C.c_char * 64),
                ("driver_version", C.c_char * 64), ("device_index", C.c_int32),
                ("compute_units", C.c_int32), ("clock_khz", C.c_int32),
                ("wavefront_size", C.c_int32), ("global_mem_bytes", C.c_size_t),
                ("lds_bytes_per_block", C.c_size_t), ("host_unified_memory", C.c_int32),
                ("has_fp16", C.c_int32)]


class ProbeResult(C.Structure):
    _fields_ = [("available", C.c_int32), ("info", DeviceInfo), ("reason", C.c_char * 256)]


class GemmProfile(C.Structure):
    _fields_ = [("duration_seconds", C.c_double), ("gflops", C.c_double),
                ("kernel_variant", C.c_char_p)]


class ModelConfigC(C.Structure):
    _fields_ = [("n_layers", C.c_int32), ("embd", C.c_int32), ("ffn", C.c_int32),
                ("n_head", C.c_int32), ("n_head_kv", C.c_int32), ("head_dim", C.c_int32),
                ("rope_dim", C.c_int32), ("vocab", C.c_int32), ("rope_base", C.c_float),
                ("eps", C.c_float), ("rope_mode", C.c_int32)]


_BP = C.c_void_p  # sulimo_hip_buffer*


class LayerTensorsC(C.Structure):
    _fields_ = [(n, _BP) for n in (
        "attn_norm", "attn_q_scales", "attn_q_quants", "attn_k_scales", "attn_k_quants",
        "attn_v_scales", "attn_v_quants", "attn_out_scales", "attn_out_quants", "ffn_norm",
        "ffn_gate_scales", "ffn_gate_quants", "ffn_up_scales", "ffn_up_quants",
        "ffn_down_scales", "ffn_down_quants",
        # optional (NULL when absent): q/k/v biases, QK-norm weights
        "attn_q_bias", "attn_k_bias", "attn_v_bias", "attn_q_norm", "attn_k_norm")]


class ModelTensorsC(C.Structure):
    _fields_ = [("output_norm", _BP), ("output_scales", _BP), ("output_quants", _BP),
                ("layers", C.POINTER(LayerTensorsC)), ("n_layers", C.c_int32)]


class KvCacheC(C.Structure):
    _fields_ = [("k_buffers", C.POINTER(_BP)), ("v_buffers", C.POINTER(_BP)),
                ("n_layers", C.c_int32), ("capacity", C.c_size_t),
                ("head_count_kv", C.c_size_t), ("head_dim", C.c_size_t)]


class PrefillScratchC(C.Structure):
    _fields_ = [(n, _BP) for n in ("x", "h", "q", "k", "v", "attn_out", "ffn_gate", "ffn_up",
                                   "ffn_swiglu", "ffn_down", "logits")] + [("max_n", C.c_size_t)]


class PrefillOutputsC(C.Structure):
    _fields_ = [("logits_all", _BP), ("argmax_all", _BP), ("unfused", C.c_int32)]


class KernelStat(C.Structure):
    _fields_ = [("launches", C.c_uint64), ("total_ms", C.c_double), ("flop", C.c_double),
                ("bytes", C.c_double)]


class PrefillStats(C.Structure):
    _fields_ = [("gemm", KernelStat), ("attention", KernelStat), ("norm", KernelStat),
                ("rope_kv", KernelStat), ("other", KernelStat), ("prefill_calls", C.c_uint64),
                ("gemm_qkv", KernelStat), ("gemm_o", KernelStat), ("gemm_gate_up", KernelStat),
                ("gemm_down", KernelStat), ("gemm_lm_head", KernelStat)]


def _declare(L):
    I32, SZ, P, F = C.c_int32, C.c_size_t, C.c_void_p, C.c_float
    sig = {
        "sulimo_hip_get_or_init": (I32, [I32, C.POINTER(P)]),
        "sulimo_hip_context_new": (I32, [I32, C.POINTER(P)]),
        "sulimo_hip_context_release": (I32, [P]),
        "sulimo_hip_finish": (I32, [P]),
        "sulimo_hip_get_device_info": (I32, [P, C.POINTER(DeviceInfo)]),
        "sulimo_hip_probe": (I32, [C.POINTER(ProbeResult)]),
        "sulimo_hip_last_error": (C.c_char_p, []),
        "sulimo_hip_buffer_create": (I32, [P, P, SZ, I32, C.POINTER(P)]),
        "sulimo_hip_buffer_release": (I32, [P]),
        "sulimo_hip_active_buffer_count": (SZ, []),
        "sulimo_hip_buffer_size": (SZ, [P]),
        "sulimo_hip_buffer_device_ptr": (P, [P]),
        "sulimo_hip_buffer_host_ptr": (P, [P]),
        "sulimo_hip_buffer_upload": (I32, [P, P, SZ, SZ, P]),
        "sulimo_hip_buffer_download": (I32, [P, P, SZ, SZ, P]),
        "sulimo_hip_buffer_map_read": (I32, [P, P, C.POINTER(P)]),
        "sulimo_hip_buffer_unmap": (I32, [P, P, P]),
        "sulimo_hip_enqueue_gemm_q4_0_f16": (I32, [P, P, P, P, P, SZ, SZ, SZ]),
        "sulimo_hip_enqueue_gemm_q4_0_f16_noalloc": (I32, [P, P, P, P, P, SZ, SZ, SZ]),
        "sulimo_hip_enqueue_rmsnorm": (I32, [P, P, P, P, SZ, F, SZ]),
        "sulimo_hip_enqueue_rope": (I32, [P, P, SZ, SZ, SZ, F, I32, SZ, SZ]),
        "sulimo_hip_enqueue_kv_store": (I32, [P, P, P, SZ, SZ, SZ, SZ]),
        "sulimo_hip_enqueue_attention_prefill": (I32, [P, P, P, P, P, SZ, SZ, SZ, SZ, SZ, SZ]),
        "sulimo_hip_enqueue_silu_mul": (I32, [P, P, P, P, SZ]),
        "sulimo_hip_enqueue_add": (I32, [P, P, P, SZ]),
        "sulimo_hip_enqueue_logits_final": (I32, [P, P, P, P, P, SZ, SZ, SZ]),
        "sulimo_hip_wait": (I32, [P]),
        "sulimo_hip_gemm_q4_0_f16": (I32, [P, P, P, P, P, SZ, SZ, SZ, C.POINTER(GemmProfile)]),
        "sulimo_hip_execute_prefill_ubatch": (I32, [P, C.POINTER(ModelConfigC), C.POINTER(ModelTensorsC),
                                                   C.POINTER(KvCacheC), C.POINTER(PrefillScratchC), SZ, SZ]),
        "sulimo_hip_execute_prefill_ubatch_ex": (I32, [P, C.POINTER(ModelConfigC), C.POINTER(ModelTensorsC),
                                                      C.POINTER(KvCacheC), C.POINTER(PrefillScratchC), SZ, SZ,
                                                      C.POINTER(PrefillOutputsC)]),
        "sulimo_hip_embed_tokens": (I32, [P, P, P, P, SZ, SZ, SZ, P]),
        "sulimo_hip_kv_sync_to_host": (I32, [P, C.POINTER(KvCacheC), SZ, SZ]),
        "sulimo_hip_kv_sync_from_host": (I32, [P, C.POINTER(KvCacheC), SZ, SZ]),
        "sulimo_hip_kv_window_download": (I32, [P, C.POINTER(KvCacheC), I32, P, SZ, C.POINTER(SZ),
                                                C.POINTER(C.c_int64), C.POINTER(I32), C.POINTER(I32)]),
        "sulimo_hip_rope_table": (I32, [P, SZ, F, SZ, SZ, P]),
        "sulimo_hip_set_profiling": (I32, [P, I32]),
        "sulimo_hip_set_graph_replay": (I32, [P, I32]),
        "sulimo_hip_set_attention_merge_kernel": (I32, [P, I32]),
        "sulimo_hip_get_prefill_stats": (I32, [P, C.POINTER(PrefillStats)]),
        "sulimo_hip_timer_start": (I32, [P]),
        "sulimo_hip_timer_stop": (I32, [P, C.POINTER(C.c_float)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _check(rc: int):
    if rc != OK:
        raise HipError(rc, lib().sulimo_hip_last_error().decode(errors="replace"))


def probe() -> ProbeResult:
    """probe() (crates/sulimo-ocl/src/probe.rs): never raises."""
    r = ProbeResult()
    _check(lib().sulimo_hip_probe(C.byref(r)))
    return r


def active_buffer_count() -> int:
    """active_cl_mem_count (buffer.rs:21-23)."""
    return int(lib().sulimo_hip_active_buffer_count())


class HipContext:
    """OclContext: one device, one in-order stream."""

    def __init__(self, handle: int, owned: bool):
        self.handle = C.c_void_p(handle)
        self._owned = owned

    @classmethod
    def get_or_init(cls, device: int = 0) -> "HipContext":
        h = C.c_void_p()
        _check(lib().sulimo_hip_get_or_init(device, C.byref(h)))
        return cls(h.value, owned=False)

    @classmethod
    def new(cls, device: int = 0) -> "HipContext":
        h = C.c_void_p()
        _check(lib().sulimo_hip_context_new(device, C.byref(h)))
        return cls(h.value, owned=True)

    def release(self):
        if self._owned and self.handle:
            _check(lib().sulimo_hip_context_release(self.handle))
            self.handle = C.c_void_p()

    def finish(self):
        _check(lib().sulimo_hip_finish(self.handle))

    def wait(self):
        """wait_event_zero_spin (waiter.rs:39-82)."""
        _check(lib().sulimo_hip_wait(self.handle))

    @property
    def device_info(self) -> DeviceInfo:
        i = DeviceInfo()
        _check(lib().sulimo_hip_get_device_info(self.handle, C.byref(i)))
        return i

    def set_graph_replay(self, enable: bool):
        _check(lib().sulimo_hip_set_graph_replay(self.handle, 1 if enable else 0))

    def set_attention_merge_kernel(self, enable: bool):
        """Merge split attention blocks in a separate kernel (True) or in the last
        workgroup to finish each block (False, the default)."""
        _check(lib().sulimo_hip_set_attention_merge_kernel(self.handle, 1 if enable else 0))

    def set_profiling(self, enable: bool):
        """Per-launch hipEvent timing of execute_prefill_ubatch (clears the statistics)."""
        _check(lib().sulimo_hip_set_profiling(self.handle, 1 if enable else 0))

    def prefill_stats(self) -> PrefillStats:
        st = PrefillStats()
        _check(lib().sulimo_hip_get_prefill_stats(self.handle, C.byref(st)))
        return st

    def timer_start(self):
        _check(lib().sulimo_hip_timer_start(self.handle))

    def timer_stop(self) -> float:
        ms = C.c_float()
        _check(lib().sulimo_hip_timer_stop(self.handle, C.byref(ms)))
        return float(ms.value)


class HipBuffer:
    """OclBuffer: an HBM allocation mirroring a host numpy array (or device-only)."""

    def __init__(self, ctx: HipContext, handle: int, host: np.ndarray | None, nbytes: int):
        self.ctx = ctx
        self.handle = C.c_void_p(handle)
        self.host = host  # keeps the host mirror alive
        self.nbytes = nbytes

    @classmethod
    def from_host(cls, ctx: HipContext, arr: np.ndarray, read_only: bool = False) -> "HipBuffer":
        """OclBuffer::from_host_ptr (buffer.rs:42-115): uploads arr, keeps it as the mirror."""
        if not arr.flags["C_CONTIGUOUS"]:
            raise ValueError("host mirror must be C-contiguous")
        h = C.c_void_p()
        _check(lib().sulimo_hip_buffer_create(ctx.handle, arr.ctypes.data_as(C.c_void_p), arr.nbytes,
                                              1 if read_only else 0, C.byref(h)))
        return cls(ctx, h.value, arr, arr.nbytes)

    @classmethod
    def device_only(cls, ctx: HipContext, nbytes: int) -> "HipBuffer":
        h = C.c_void_p()
        _check(lib().sulimo_hip_buffer_create(ctx.handle, None, nbytes, 0, C.byref(h)))
        return cls(ctx, h.value, None, nbytes)

    def upload(self, arr: np.ndarray, offset: int = 0):
        arr = np.ascontiguousarray(arr)
        _check(lib().sulimo_hip_buffer_upload(self.ctx.handle, self.handle, offset, arr.nbytes,
                                              arr.ctypes.data_as(C.c_void_p)))

    def download(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        _check(lib().sulimo_hip_buffer_download(self.ctx.handle, self.handle, offset, out.nbytes,
                                                out.ctypes.data_as(C.c_void_p)))
        return out

    def map_read(self) -> np.ndarray:
        """OclBuffer::map_read (buffer.rs:128-145): refreshes and returns the host mirror."""
        p = C.c_void_p()
        _check(lib().sulimo_hip_buffer_map_read(self.ctx.handle, self.handle, C.byref(p)))
        return self.host

    def unmap(self):
        _check(lib().sulimo_hip_buffer_unmap(self.ctx.handle, self.handle,
                                             self.host.ctypes.data_as(C.c_void_p) if self.host is not None else None))

    def release(self):
        if self.handle:
            _check(lib().sulimo_hip_buffer_release(self.handle))
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            if self.handle and _lib is not None:
                _lib.sulimo_hip_buffer_release(self.handle)
                self.handle = C.c_void_p()
        except Exception:
            pass


# ---- per-op enqueue (crates/sulimo-ocl/src/prefill.rs:67-330) ----

def _h(b):
    return b.handle if b is not None else None


def enqueue_gemm_q4_0_f16(ctx, scales, quants, x, out, m, k, n):
    _check(lib().sulimo_hip_enqueue_gemm_q4_0_f16(ctx.handle, _h(scales), _h(quants), _h(x), _h(out), m, k, n))


def enqueue_gemm_q4_0_f16_noalloc(ctx, scales, quants, x, out, m, k, n):
    """The same GEMM with no device allocation: its scratch is the library's static
    per-device array (calls that overlap on one GPU race)."""
    _check(lib().sulimo_hip_enqueue_gemm_q4_0_f16_noalloc(ctx.handle, _h(scales), _h(quants), _h(x), _h(out),
                                                          m, k, n))


def gemm_q4_0_f16(ctx, scales, quants, x, out, m, k, n) -> GemmProfile:
    """gemm_q4_0_f16 (crates/sulimo-ocl/src/gemm.rs:28-102): waited and timed."""
    p = GemmProfile()
    _check(lib().sulimo_hip_gemm_q4_0_f16(ctx.handle, _h(scales), _h(quants), _h(x), _h(out), m, k, n,
                                          C.byref(p)))
    return p


def enqueue_rmsnorm(ctx, x, w, out, d, eps, n):
    _check(lib().sulimo_hip_enqueue_rmsnorm(ctx.handle, _h(x), _h(w), _h(out), d, eps, n))


def enqueue_rope(ctx, vec, head_count, head_dim, rope_dim, freq_base, mode, start_pos, n):
    _check(lib().sulimo_hip_enqueue_rope(ctx.handle, _h(vec), head_count, head_dim, rope_dim, freq_base,
                                         mode, start_pos, n))


def enqueue_kv_store(ctx, act, kv_cache, start_pos, capacity, blocks_per_pos, n):
    _check(lib().sulimo_hip_enqueue_kv_store(ctx.handle, _h(act), _h(kv_cache), start_pos, capacity,
                                             blocks_per_pos, n))


def enqueue_attention_prefill(ctx, q, k_cache, v_cache, out, start_pos, capacity, head_count,
                              head_count_kv, head_dim, n):
    _check(lib().sulimo_hip_enqueue_attention_prefill(ctx.handle, _h(q), _h(k_cache), _h(v_cache), _h(out),
                                                      start_pos, capacity, head_count, head_count_kv,
                                                      head_dim, n))


def enqueue_silu_mul(ctx, gate, up, out, total_elements):
    _check(lib().sulimo_hip_enqueue_silu_mul(ctx.handle, _h(gate), _h(up), _h(out), total_elements))


def enqueue_add(ctx, a, b, total_elements):
    _check(lib().sulimo_hip_enqueue_add(ctx.handle, _h(a), _h(b), total_elements))


def enqueue_logits_final(ctx, x_all, scales, quants, logits, vocab_size, embd_dim, token_idx):
    _check(lib().sulimo_hip_enqueue_logits_final(ctx.handle, _h(x_all), _h(scales), _h(quants), _h(logits),
                                                 vocab_size, embd_dim, token_idx))


def rope_table(ctx, rope_dim, freq_base, start_pos, n, table):
    """The (cos, sin) f32 pairs of a ubatch's rotations, [n][rope_dim/2][2], into table."""
    _check(lib().sulimo_hip_rope_table(ctx.handle, rope_dim, freq_base, start_pos, n, _h(table)))


def embed_tokens(ctx, embd_scales, embd_quants, tokens: np.ndarray, embd, vocab, x):
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    _check(lib().sulimo_hip_embed_tokens(ctx.handle, _h(embd_scales), _h(embd_quants),
                                         t.ctypes.data_as(C.c_void_p), t.size, embd, vocab, _h(x)))


# ---- whole-model device state (OclEngineState, crates/sulimo-engine/src/scheduler.rs:62-244) ----

@dataclass
class DevQ4:
    scales: HipBuffer
    quants: HipBuffer


class DeviceModel:
    """Uploads a host model (sulimo_amd.synthetic.HostModel) and owns the
    prefill state: weights, the Q8_0 ring per layer and the ubatch scratch."""

    def __init__(self, ctx: HipContext, hm, capacity: int, max_n: int, kv_host=None):
        c = hm.cfg
        self.ctx, self.hm, self.cfg = ctx, hm, c
        self.capacity, self.max_n = capacity, max_n

        def q4(t):
            return DevQ4(HipBuffer.from_host(ctx, t.scales, True), HipBuffer.from_host(ctx, t.quants, True))

        self.layers = []
        lt = (LayerTensorsC * c.n_layers)()
        for i, L in enumerate(hm.layers):
            d = dict(attn_norm=HipBuffer.from_host(ctx, L.attn_norm, True), q=q4(L.q), k=q4(L.k), v=q4(L.v),
                     o=q4(L.o), ffn_norm=HipBuffer.from_host(ctx, L.ffn_norm, True), gate=q4(L.gate),
                     up=q4(L.up), down=q4(L.down))
            opt = []
            for name in ("q_bias", "k_bias", "v_bias", "q_norm", "k_norm"):
                a = getattr(L, name, None)
                if a is not None:
                    d[name] = HipBuffer.from_host(ctx, a, True)
                opt.append(d[name].handle if a is not None else None)
            self.layers.append(d)
            lt[i] = LayerTensorsC(d["attn_norm"].handle, d["q"].scales.handle, d["q"].quants.handle,
                                  d["k"].scales.handle, d["k"].quants.handle, d["v"].scales.handle,
                                  d["v"].quants.handle, d["o"].scales.handle, d["o"].quants.handle,
                                  d["ffn_norm"].handle, d["gate"].scales.handle, d["gate"].quants.handle,
                                  d["up"].scales.handle, d["up"].quants.handle, d["down"].scales.handle,
                                  d["down"].quants.handle, *opt)
        self._lt = lt
        self.token_embd = q4(hm.token_embd)
        self.output = self.token_embd if hm.output is hm.token_embd else q4(hm.output)
        self.output_norm = HipBuffer.from_host(ctx, hm.output_norm, True)
        self.tensors = ModelTensorsC(self.output_norm.handle, self.output.scales.handle,
                                     self.output.quants.handle, lt, c.n_layers)
        self.cfg_c = ModelConfigC(c.n_layers, c.embd, c.ffn, c.n_head, c.n_head_kv, c.head_dim, c.rope_dim,
                                  c.vocab, c.rope_base, c.eps, c.rope_mode)
        # KV ring: host mirror per layer (the engine's KvCache slices) + device copy
        bpp = c.n_head_kv * (c.head_dim // 32) * 34
        self.bpp = bpp
        if kv_host is None:
            kv_host = ([np.zeros(capacity * bpp, np.uint8) for _ in range(c.n_layers)],
                       [np.zeros(capacity * bpp, np.uint8) for _ in range(c.n_layers)])
        self.kv_k = [HipBuffer.from_host(ctx, a) for a in kv_host[0]]
        self.kv_v = [HipBuffer.from_host(ctx, a) for a in kv_host[1]]
        self._kp = (C.c_void_p * c.n_layers)(*[b.handle.value for b in self.kv_k])
        self._vp = (C.c_void_p * c.n_layers)(*[b.handle.value for b in self.kv_v])
        self.kv = KvCacheC(self._kp, self._vp, c.n_layers, capacity, c.n_head_kv, c.head_dim)
        # ubatch scratch (scheduler.rs:190-233 sizes)
        D, F, qd, kvd = c.embd, c.ffn, c.n_head * c.head_dim, c.n_head_kv * c.head_dim
        self.x_host = np.zeros((max_n, D), np.float16)
        self.logits_host = np.zeros(c.vocab, np.float32)
        sb = {
            "x": HipBuffer.from_host(ctx, self.x_host), "h": HipBuffer.device_only(ctx, max_n * D * 2),
            "q": HipBuffer.device_only(ctx, max_n * qd * 2), "k": HipBuffer.device_only(ctx, max_n * kvd * 2),
            "v": HipBuffer.device_only(ctx, max_n * kvd * 2),
            "attn_out": HipBuffer.device_only(ctx, max_n * qd * 2),
            "ffn_swiglu": HipBuffer.device_only(ctx, max_n * F * 2),
            "logits": HipBuffer.from_host(ctx, self.logits_host),
        }
        self.scratch_bufs = sb
        self.scratch = PrefillScratchC(sb["x"].handle, sb["h"].handle, sb["q"].handle, sb["k"].handle,
                                       sb["v"].handle, sb["attn_out"].handle, None, None,
                                       sb["ffn_swiglu"].handle, None, sb["logits"].handle, max_n)

    def embed(self, tokens: np.ndarray):
        """Device embedding gather into scratch.x (replaces scheduler.rs:329-374)."""
        embed_tokens(self.ctx, self.token_embd.scales, self.token_embd.quants, tokens, self.cfg.embd,
                     self.cfg.vocab, self.scratch_bufs["x"])

    def _unfused_scratch(self):
        """f16 gate, up and down buffers the unfused validation mode writes."""
        if "ffn_gate" not in self.scratch_bufs:
            c, sb = self.cfg, self.scratch_bufs
            for name, w in (("ffn_gate", c.ffn), ("ffn_up", c.ffn), ("ffn_down", c.embd)):
                sb[name] = HipBuffer.device_only(self.ctx, self.max_n * w * 2)
            self.scratch.ffn_gate = sb["ffn_gate"].handle
            self.scratch.ffn_up = sb["ffn_up"].handle
            self.scratch.ffn_down = sb["ffn_down"].handle

    def execute_prefill_ubatch(self, start_pos: int, n: int, logits_all: HipBuffer | None = None,
                               argmax_all: HipBuffer | None = None, unfused: bool = False):
        """execute_prefill_ubatch (prefill.rs:337-566). unfused runs every op as its own
        kernel (validation of the fused GEMM epilogues)."""
        if unfused:
            self._unfused_scratch()
        if logits_all is None and argmax_all is None and not unfused:
            _check(lib().sulimo_hip_execute_prefill_ubatch(self.ctx.handle, C.byref(self.cfg_c),
                                                           C.byref(self.tensors), C.byref(self.kv),
                                                           C.byref(self.scratch), start_pos, n))
        else:
            o = PrefillOutputsC(_h(logits_all), _h(argmax_all), 1 if unfused else 0)
            _check(lib().sulimo_hip_execute_prefill_ubatch_ex(self.ctx.handle, C.byref(self.cfg_c),
                                                              C.byref(self.tensors), C.byref(self.kv),
                                                              C.byref(self.scratch), start_pos, n, C.byref(o)))

    def logits(self) -> np.ndarray:
        return self.scratch_bufs["logits"].map_read().copy()

    def kv_sync_to_host(self, start_pos: int, n: int):
        _check(lib().sulimo_hip_kv_sync_to_host(self.ctx.handle, C.byref(self.kv), start_pos, n))

    def kv_sync_from_host(self, start_pos: int, n: int):
        _check(lib().sulimo_hip_kv_sync_from_host(self.ctx.handle, C.byref(self.kv), start_pos, n))

    def kv_host(self):
        return [b.host for b in self.kv_k], [b.host for b in self.kv_v]

    def kv_window(self, layer: int):
        """The f16 attention window kept for `layer` (sulimo_hip_kv_window_download):
        returns (K [n_head_kv, pad, head_dim], V^T rows [n_head_kv, head_dim, v_row_stride]
        in the stored column order, valid_len)."""
        c = self.cfg
        nbytes, vlen = C.c_size_t(), C.c_int64()
        pad, vst = C.c_int32(), C.c_int32()
        _check(lib().sulimo_hip_kv_window_download(self.ctx.handle, C.byref(self.kv), layer, None, 0,
                                                   C.byref(nbytes), C.byref(vlen), C.byref(pad),
                                                   C.byref(vst)))
        raw = np.zeros(nbytes.value // 2, np.float16)
        _check(lib().sulimo_hip_kv_window_download(self.ctx.handle, C.byref(self.kv), layer,
                                                   raw.ctypes.data_as(C.c_void_p), raw.nbytes,
                                                   C.byref(nbytes), C.byref(vlen), C.byref(pad),
                                                   C.byref(vst)))
        hkv, hd, p, s = c.n_head_kv, c.head_dim, pad.value, vst.value
        k = raw[:hkv * p * hd].reshape(hkv, p, hd)
        vt = raw[hkv * p * hd:hkv * p * hd + hkv * hd * s].reshape(hkv, hd, s)
        return k, vt, int(vlen.value)

    def prefill_tokens(self, tokens: np.ndarray, start_pos: int = 0, ubatch: int | None = None) -> np.ndarray:
        """The engine's GPU prefill loop (engine.rs:217-286) without context repack:
        embed + execute_prefill_ubatch per micro-batch; returns the last logits."""
        ub = ubatch or self.max_n
        pos, off, n = start_pos, 0, len(tokens)
        while off < n:
            m = min(ub, n - off)
            self.embed(tokens[off:off + m])
            self.execute_prefill_ubatch(pos, m)
            pos += m
            off += m
        return self.logits()

    def release(self):
        for d in self.layers:
            for v in d.values():
                if isinstance(v, DevQ4):
                    v.scales.release(); v.quants.release()
                else:
                    v.release()
        for b in [self.output_norm, self.token_embd.scales, self.token_embd.quants, self.output.scales,
                  self.output.quants, *self.kv_k, *self.kv_v, *self.scratch_bufs.values()]:
            b.release()
