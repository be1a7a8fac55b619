"""CPU oracle for the Q4_0 prefill path -- TEST INFRASTRUCTURE ONLY.

ctypes bindings to ``oracle/liboracle.so`` (built from ``oracle/oracle.c`` by
``oracle/Makefile``), a C restatement of Sulimo's CPU path and of the reference
GPU kernels' formulas. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` import this package; the product
(``sulimo_amd``) never does.

Every wrapper names the reference function it restates; the C file carries the
file:line citations. Arrays are numpy; f16 data is passed as ``np.float16``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile oracle/liboracle.so with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-C", _HERE, "-B" if force else "liboracle.so"], check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = C.c_void_p
_SZ = C.c_size_t
_I = C.c_int
_F = C.c_float


class OrcConfig(C.Structure):
    _fields_ = [("n_layers", C.c_int32), ("embd", C.c_int32), ("ffn", C.c_int32),
                ("n_head", C.c_int32), ("n_head_kv", C.c_int32), ("head_dim", C.c_int32),
                ("rope_dim", C.c_int32), ("vocab", C.c_int32), ("rope_base", C.c_float),
                ("eps", C.c_float), ("rope_mode", C.c_int32)]


class OrcQ4(C.Structure):
    _fields_ = [("scales", _P), ("quants", _P)]


class OrcLayer(C.Structure):
    _fields_ = [("attn_norm", _P), ("q", OrcQ4), ("k", OrcQ4), ("v", OrcQ4), ("o", OrcQ4),
                ("ffn_norm", _P), ("gate", OrcQ4), ("up", OrcQ4), ("down", OrcQ4),
                ("q_bias", _P), ("k_bias", _P), ("v_bias", _P), ("q_norm", _P), ("k_norm", _P)]


class OrcModel(C.Structure):
    _fields_ = [("cfg", OrcConfig), ("token_embd", OrcQ4), ("output_norm", _P),
                ("output", OrcQ4), ("layers", C.POINTER(OrcLayer))]


class OrcKv(C.Structure):
    _fields_ = [("k", C.POINTER(C.c_void_p)), ("v", C.POINTER(C.c_void_p)), ("capacity", _SZ)]


def _declare(L):
    sig = {
        "orc_f16_to_f32": (_F, [C.c_uint16]),
        "orc_f32_to_f16": (C.c_uint16, [_F]),
        "orc_repack_q4_0_aos_to_soa": (C.c_int64, [_P, _SZ, _P, _SZ, _P, _SZ]),
        "orc_dequant_q4_0_aos": (None, [_P, _SZ, _P]),
        "orc_dequant_q4_0_soa": (None, [_P, _P, _SZ, _P]),
        "orc_quantize_f32_to_q8_0": (None, [_P, _SZ, _P]),
        "orc_dequant_q8_0": (None, [_P, _SZ, _P]),
        "orc_gemm_q4_0_f16_scalar_reference": (None, [_P, _P, _P, _SZ, _SZ, _SZ, _P]),
        "orc_vec_dot_q4_0_q8_0_scalar": (_F, [_P, _P, _P, _SZ]),
        "orc_vec_dot_q4_0_q8_0_avx2": (_F, [_P, _P, _P, _SZ]),
        "orc_matvec_q4_0_q8_0_avx2": (None, [_P, _P, _P, _SZ, _SZ, _P]),
        "orc_rmsnorm_scalar": (None, [_P, _P, _F, _SZ, _P]),
        "orc_rmsnorm_avx2": (None, [_P, _P, _F, _SZ, _P]),
        "orc_rope_head_scalar": (None, [_P, _SZ, _SZ, _F, _I]),
        "orc_softmax_scalar": (None, [_P, _SZ]),
        "orc_swiglu_scalar": (None, [_P, _P, _SZ, _P]),
        "orc_causal_gqa_decode_scalar": (None, [_P, _P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ,
                                                _P, _P, _P]),
        "orc_cl_rmsnorm_f16_f32w": (None, [_P, _P, _P, _I, _F, _I]),
        "orc_cl_rope_f16": (None, [_P, _I, _I, _I, _F, _I, _I, _I]),
        "orc_cl_kv_store_q8_0": (None, [_P, _P, _I, _I, _I, _I]),
        "orc_cl_silu_mul_f16": (None, [_P, _P, _P, _I]),
        "orc_cl_add_f16": (None, [_P, _P, _I]),
        "orc_cl_logits_f16_output": (None, [_P, _P, _P, _P, _I, _I, _I]),
        "orc_attention_prefill_f32": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I]),
        "orc_lookup_token_embedding_f16": (None, [_P, _P, _SZ, C.c_uint32, _P]),
        "orc_forward_token": (_I, [C.POINTER(OrcModel), C.POINTER(OrcKv), C.c_uint32, _SZ, _P]),
        "orc_forward_token_mt": (_I, [C.POINTER(OrcModel), C.POINTER(OrcKv), C.c_uint32, _SZ, _P, _I]),
        "orc_prefill_reference": (_I, [C.POINTER(OrcModel), C.POINTER(OrcKv), _P, _SZ, _SZ, _I,
                                       _P, _P, _P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(C.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _f16(a):
    return np.ascontiguousarray(a, dtype=np.float16)


# ---- Q4_0 / Q8_0 formats -------------------------------------------------

def repack_q4_0_aos_to_soa(aos: np.ndarray):
    """repack.rs:45-80. Returns (scales u8[2*nb], quants u8[16*nb])."""
    aos = np.ascontiguousarray(aos, dtype=np.uint8)
    nb = aos.size // 18
    sc = np.zeros(nb * 2, np.uint8)
    qu = np.zeros(nb * 16, np.uint8)
    r = lib().orc_repack_q4_0_aos_to_soa(_p(aos), aos.size, _p(sc), sc.size, _p(qu), qu.size)
    if r < 0:
        raise ValueError(f"repack error {r}")
    return sc, qu


def dequant_q4_0_aos(aos: np.ndarray) -> np.ndarray:
    aos = np.ascontiguousarray(aos, dtype=np.uint8)
    nb = aos.size // 18
    out = np.zeros(nb * 32, np.float32)
    lib().orc_dequant_q4_0_aos(_p(aos), nb, _p(out))
    return out


def dequant_q4_0_soa(scales: np.ndarray, quants: np.ndarray) -> np.ndarray:
    """repack.rs:107-131: f32 weights, blocks in storage order."""
    sc = np.ascontiguousarray(scales).view(np.uint8)
    qu = np.ascontiguousarray(quants, dtype=np.uint8)
    nb = qu.size // 16
    out = np.zeros(nb * 32, np.float32)
    lib().orc_dequant_q4_0_soa(_p(sc), _p(qu), nb, _p(out))
    return out


def quantize_f32_to_q8_0(x: np.ndarray) -> np.ndarray:
    """kv_cache.rs:162-193: u8[34 * n/32]."""
    x = _f32(x).ravel()
    out = np.zeros(x.size // 32 * 34, np.uint8)
    lib().orc_quantize_f32_to_q8_0(_p(x), x.size, _p(out))
    return out


def dequant_q8_0(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint8).ravel()
    nb = b.size // 34
    out = np.zeros(nb * 32, np.float32)
    lib().orc_dequant_q8_0(_p(b), nb, _p(out))
    return out


# ---- GEMM / CPU kernels --------------------------------------------------

def gemm_q4_0_f16_scalar_reference(scales, quants, x, m: int, k: int, n: int) -> np.ndarray:
    """gemm.rs:106-147 (reference naming: m outputs, k inputs, n tokens). f16 [n, m]."""
    sc = np.ascontiguousarray(scales).view(np.uint8)
    qu = np.ascontiguousarray(quants, dtype=np.uint8)
    x = _f16(x)
    out = np.zeros((n, m), np.float16)
    lib().orc_gemm_q4_0_f16_scalar_reference(_p(sc), _p(qu), _p(x), m, k, n, _p(out))
    return out


def vec_dot_q4_0_q8_0(w_scales, w_quants, x_q8, nblocks: int, avx2: bool = True) -> float:
    f = lib().orc_vec_dot_q4_0_q8_0_avx2 if avx2 else lib().orc_vec_dot_q4_0_q8_0_scalar
    return float(f(_p(np.ascontiguousarray(w_scales).view(np.uint8)),
                   _p(np.ascontiguousarray(w_quants, dtype=np.uint8)),
                   _p(np.ascontiguousarray(x_q8, dtype=np.uint8)), nblocks))


def matvec_q4_0_q8_0(w_scales, w_quants, x_q8, rows: int, cols: int) -> np.ndarray:
    out = np.zeros(rows, np.float32)
    lib().orc_matvec_q4_0_q8_0_avx2(_p(np.ascontiguousarray(w_scales).view(np.uint8)),
                                    _p(np.ascontiguousarray(w_quants, dtype=np.uint8)),
                                    _p(np.ascontiguousarray(x_q8, dtype=np.uint8)), rows, cols,
                                    _p(out))
    return out


def rmsnorm(x, w, eps: float, avx2: bool = False) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    out = np.zeros_like(x)
    f = lib().orc_rmsnorm_avx2 if avx2 else lib().orc_rmsnorm_scalar
    f(_p(x), _p(w), eps, x.size, _p(out))
    return out


def rope_head(vec, pos: int, rope_dim: int, freq_base: float, mode: int) -> np.ndarray:
    v = _f32(vec).copy()
    lib().orc_rope_head_scalar(_p(v), pos, rope_dim, freq_base, mode)
    return v


def softmax(x) -> np.ndarray:
    v = _f32(x).copy()
    lib().orc_softmax_scalar(_p(v), v.size)
    return v


def swiglu(gate, up) -> np.ndarray:
    g, u = _f32(gate), _f32(up)
    out = np.zeros_like(g)
    lib().orc_swiglu_scalar(_p(g), _p(u), g.size, _p(out))
    return out


def causal_gqa_decode(q, k_ring, v_ring, bytes_per_pos, capacity, first_pos, context_len,
                      head_count, head_count_kv, head_dim) -> np.ndarray:
    q = _f32(q)
    out = np.zeros(head_count * head_dim, np.float32)
    scores = np.zeros(max(context_len, 1), np.float32)
    deq = np.zeros(head_dim, np.float32)
    lib().orc_causal_gqa_decode_scalar(_p(q), _p(np.ascontiguousarray(k_ring, dtype=np.uint8)),
                                       _p(np.ascontiguousarray(v_ring, dtype=np.uint8)),
                                       bytes_per_pos, capacity, first_pos, context_len,
                                       head_count, head_count_kv, head_dim, _p(scores), _p(deq),
                                       _p(out))
    return out


# ---- reference GPU kernels restated --------------------------------------

def cl_rmsnorm_f16_f32w(x, w, d: int, eps: float, n: int) -> np.ndarray:
    x, w = _f16(x), _f32(w)
    out = np.zeros_like(x)
    lib().orc_cl_rmsnorm_f16_f32w(_p(x), _p(w), _p(out), d, eps, n)
    return out


def cl_rope_f16(vec, head_count, head_dim, rope_dim, freq_base, mode, start_pos, n) -> np.ndarray:
    v = _f16(vec).copy()
    lib().orc_cl_rope_f16(_p(v), head_count, head_dim, rope_dim, freq_base, mode, start_pos, n)
    return v


def cl_kv_store_q8_0(act, kv, start_pos, capacity, blocks_per_pos, n) -> np.ndarray:
    a = _f16(act)
    out = np.ascontiguousarray(kv, dtype=np.uint8).copy()
    lib().orc_cl_kv_store_q8_0(_p(a), _p(out), start_pos, capacity, blocks_per_pos, n)
    return out


def cl_silu_mul_f16(gate, up) -> np.ndarray:
    g, u = _f16(gate), _f16(up)
    out = np.zeros_like(g)
    lib().orc_cl_silu_mul_f16(_p(g), _p(u), _p(out), g.size)
    return out


def cl_add_f16(a, b) -> np.ndarray:
    a2, b2 = _f16(a).copy(), _f16(b)
    lib().orc_cl_add_f16(_p(a2), _p(b2), a2.size)
    return a2


def cl_logits_f16_output(x_all, scales, quants, m, k, token_idx) -> np.ndarray:
    out = np.zeros(m, np.float32)
    lib().orc_cl_logits_f16_output(_p(_f16(x_all)), _p(np.ascontiguousarray(scales).view(np.uint8)),
                                   _p(np.ascontiguousarray(quants, dtype=np.uint8)), _p(out), m, k,
                                   token_idx)
    return out


def attention_prefill_f32(q, k_ring, v_ring, start_pos, capacity, head_count, head_count_kv,
                          head_dim, n) -> np.ndarray:
    q = _f32(q)
    out = np.zeros((n, head_count * head_dim), np.float32)
    lib().orc_attention_prefill_f32(_p(q), _p(np.ascontiguousarray(k_ring, dtype=np.uint8)),
                                    _p(np.ascontiguousarray(v_ring, dtype=np.uint8)), _p(out),
                                    start_pos, capacity, head_count, head_count_kv, head_dim, n)
    return out


def lookup_token_embedding_f16(scales, quants, embd: int, token: int) -> np.ndarray:
    out = np.zeros(embd, np.float16)
    lib().orc_lookup_token_embedding_f16(_p(np.ascontiguousarray(scales).view(np.uint8)),
                                         _p(np.ascontiguousarray(quants, dtype=np.uint8)), embd,
                                         token, _p(out))
    return out


# ---- whole model ----------------------------------------------------------

class OracleModel:
    """Holds ctypes views of a host model (``sulimo_amd.synthetic.HostModel``)."""

    def __init__(self, hm):
        c = hm.cfg
        self.hm = hm
        self.cfg = OrcConfig(c.n_layers, c.embd, c.ffn, c.n_head, c.n_head_kv, c.head_dim,
                             c.rope_dim, c.vocab, c.rope_base, c.eps, c.rope_mode)

        def q4(t):
            return OrcQ4(_p(t.scales.view(np.uint8)), _p(t.quants))

        layers = (OrcLayer * c.n_layers)()
        for i, L in enumerate(hm.layers):
            opt = [None if a is None else _p(a) for a in (L.q_bias, L.k_bias, L.v_bias, L.q_norm, L.k_norm)]
            layers[i] = OrcLayer(_p(L.attn_norm), q4(L.q), q4(L.k), q4(L.v), q4(L.o),
                                 _p(L.ffn_norm), q4(L.gate), q4(L.up), q4(L.down), *opt)
        self._layers = layers
        self.model = OrcModel(self.cfg, q4(hm.token_embd), _p(hm.output_norm), q4(hm.output),
                              layers)


class OracleKv:
    """Host Q8_0 ring (kv_cache.rs layout): per layer u8[capacity * bytes_per_pos]."""

    def __init__(self, cfg, capacity: int, k=None, v=None):
        self.capacity = capacity
        self.bpp = cfg.n_head_kv * (cfg.head_dim // 32) * 34
        self.k = k if k is not None else [np.zeros(capacity * self.bpp, np.uint8)
                                          for _ in range(cfg.n_layers)]
        self.v = v if v is not None else [np.zeros(capacity * self.bpp, np.uint8)
                                          for _ in range(cfg.n_layers)]
        self._kp = (C.c_void_p * cfg.n_layers)(*[a.ctypes.data for a in self.k])
        self._vp = (C.c_void_p * cfg.n_layers)(*[a.ctypes.data for a in self.v])
        self.s = OrcKv(self._kp, self._vp, capacity)


def forward_token(om: OracleModel, kv: OracleKv, token: int, pos: int, threads: int = 1) -> np.ndarray:
    """forward_pass.rs:190-417: f32 logits of one token. threads = 1 is the reference's
    single-core path; more threads split every matvec's rows (bit-identical result)."""
    out = np.zeros(om.cfg.vocab, np.float32)
    if threads == 1:
        rc = lib().orc_forward_token(C.byref(om.model), C.byref(kv.s), token, pos, _p(out))
    else:
        rc = lib().orc_forward_token_mt(C.byref(om.model), C.byref(kv.s), token, pos, _p(out), threads)
    if rc:
        raise MemoryError("orc_forward_token failed")
    return out


def prefill_reference(om: OracleModel, kv: OracleKv, x_in, start_pos: int, all_logits=False,
                      want_h=False, want_x=False):
    """fp32 reference prefill (prefill.rs:362-560 op order, test_prefill.rs rounding).
    Returns the logits; with want_h and/or want_x a tuple (logits[, h_final][, x_final]):
    h_final the f32 output-normed hidden states [n, embd], x_final the f32 residual stream
    after the last layer [n, embd] (scratch.x and scratch.h of the device prefill)."""
    x_in = _f16(x_in)
    n = x_in.shape[0]
    V = om.cfg.vocab
    logits = np.zeros((n, V) if all_logits else (V,), np.float32)
    h = np.zeros((n, om.cfg.embd), np.float32) if want_h else None
    xf = np.zeros((n, om.cfg.embd), np.float32) if want_x else None
    rc = lib().orc_prefill_reference(C.byref(om.model), C.byref(kv.s), _p(x_in), start_pos, n,
                                     1 if all_logits else 0, _p(logits),
                                     _p(h) if h is not None else None,
                                     _p(xf) if xf is not None else None)
    if rc:
        raise MemoryError("orc_prefill_reference failed")
    if not (want_h or want_x):
        return logits
    return (logits,) + ((h,) if want_h else ()) + ((xf,) if want_x else ())
