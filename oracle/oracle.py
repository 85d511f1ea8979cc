"""ORACLE loader — test infrastructure only.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this module, and only as the checker. It wraps the C restatement
of the reference sampler (``oracle/sampler_ref.c``; see that file's header
for the reference file:line each function follows).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


class OrConfig(C.Structure):
    _fields_ = [
        ("temperature", C.c_double),
        ("top_p", C.c_double),
        ("min_p", C.c_double),
        ("typical_p", C.c_double),
        ("repetition_penalty", C.c_double),
        ("frequency_penalty", C.c_double),
        ("presence_penalty", C.c_double),
        ("top_k", C.c_int32),
        ("repetition_window", C.c_int32),
    ]


class OrTrace(C.Structure):
    _fields_ = [
        ("maximum", C.c_double),
        ("total", C.c_double),
        ("probability", C.c_double),
        ("cumulative_at_cut", C.c_double),
        ("cumulative_before_cut", C.c_double),
        ("cursor_start", C.c_double),
        ("candidate_total", C.c_double),
        ("candidates", C.c_int64),
        ("greedy", C.c_int32),
        ("fallback_last", C.c_int32),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        dp, fp, ip = C.POINTER(C.c_double), C.POINTER(C.c_float), C.POINTER(C.c_int32)
        L.or_sample_token.restype = C.c_int32
        L.or_sample_token.argtypes = [dp, C.c_int64, ip, C.c_int64, C.POINTER(OrConfig), C.c_double,
                                      C.POINTER(OrTrace)]
        L.or_sample_token_f32.restype = C.c_int32
        L.or_sample_token_f32.argtypes = [fp, C.c_int64, ip, C.c_int64, C.POINTER(OrConfig), C.c_double,
                                          C.POINTER(OrTrace)]
        L.or_token_log_prob.restype = C.c_double
        L.or_token_log_prob.argtypes = [dp, C.c_int64, C.c_int64]
        L.or_exp.restype = C.c_double
        L.or_exp.argtypes = [C.c_double]
        L.or_log.restype = C.c_double
        L.or_log.argtypes = [C.c_double]
        L.or_draw.restype = C.c_double
        L.or_draw.argtypes = [C.c_int64, C.c_uint64]
        L.or_softcap_row.restype = None
        L.or_softcap_row.argtypes = [fp, C.c_int64, C.c_double, fp]
        L.or_draws.restype = None
        L.or_draws.argtypes = [C.c_int64, C.c_uint64, C.c_int64, dp]
        u8p = C.POINTER(C.c_uint8)
        L.or_viable_states.restype = None
        L.or_viable_states.argtypes = [ip, C.c_int32, u8p, u8p]
        L.or_dfa_legal_mask.restype = None
        L.or_dfa_legal_mask.argtypes = [ip, u8p, C.c_int32, C.POINTER(C.c_int64), u8p, C.c_int64, C.c_int32,
                                        C.POINTER(C.c_uint32)]
        L.or_mask_logits.restype = None
        L.or_mask_logits.argtypes = [fp, C.c_int64, ip, C.c_int64, ip, C.c_int64, fp]
        u32p = C.POINTER(C.c_uint32)
        L.or_pack_int2_rows.restype = C.c_int
        L.or_pack_int2_rows.argtypes = [u8p, C.c_int64, C.c_int64, u32p]
        L.or_unpack_int2.restype = C.c_int
        L.or_unpack_int2.argtypes = [u32p, C.c_int64]
        L.or_apply_srq.restype = C.c_double
        L.or_apply_srq.argtypes = [C.c_double, C.c_double]
        L.or_qat_linear_int2.restype = None
        L.or_qat_linear_int2.argtypes = [fp, u32p, fp, C.c_int64, C.c_int64, C.c_double, C.c_double, fp]
        L.or_repack_block_major.restype = None
        L.or_repack_block_major.argtypes = [u32p, C.c_int64, C.c_int64, u32p]
        _lib = L
    return _lib


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(C.POINTER(ctype))


@dataclass
class Decoding:
    """The DecodingConfig fields the sampler reads (src/runtime/decoding.ts:1-14)."""

    temperature: float = 0.8
    topK: int = 40
    topP: float = 0.95
    minP: float = 0.0
    typicalP: float = 1.0
    repetitionPenalty: float = 1.05
    repetitionWindow: int = 64
    frequencyPenalty: float = 0.0
    presencePenalty: float = 0.0

    def c(self) -> OrConfig:
        return OrConfig(self.temperature, self.topP, self.minP, self.typicalP, self.repetitionPenalty,
                        self.frequencyPenalty, self.presencePenalty, int(self.topK), int(self.repetitionWindow))


def sample_token(logits, history, cfg: Decoding, uniform: float):
    """sampleToken with random() == uniform. Returns (token, trace). token -1 = reference throws."""
    L = lib()
    if isinstance(logits, np.ndarray) and logits.dtype == np.float32:
        x = np.ascontiguousarray(logits)
        h = np.ascontiguousarray(np.asarray(history, dtype=np.int32))
        tr = OrTrace()
        c = cfg.c()
        t = L.or_sample_token_f32(_ptr(x, C.c_float), x.size, _ptr(h, C.c_int32), h.size, C.byref(c),
                                  float(uniform), C.byref(tr))
        return int(t), tr
    x = np.ascontiguousarray(np.asarray(logits, dtype=np.float64))
    h = np.ascontiguousarray(np.asarray(history, dtype=np.int32))
    tr = OrTrace()
    c = cfg.c()
    t = L.or_sample_token(_ptr(x, C.c_double), x.size, _ptr(h, C.c_int32), h.size, C.byref(c), float(uniform),
                          C.byref(tr))
    return int(t), tr


def token_log_probability(logits, token: int) -> float:
    x = np.ascontiguousarray(np.asarray(logits, dtype=np.float64))
    return float(lib().or_token_log_prob(_ptr(x, C.c_double), x.size, int(token)))


def js_exp(x: float) -> float:
    return float(lib().or_exp(float(x)))


def js_log(x: float) -> float:
    return float(lib().or_log(float(x)))


def draw(seed: int, index: int) -> float:
    return float(lib().or_draw(int(seed), int(index)))


def draws(seed: int, first: int, count: int) -> np.ndarray:
    out = np.empty(count, dtype=np.float64)
    lib().or_draws(int(seed), int(first), int(count), _ptr(out, C.c_double))
    return out


def softcap(x, cap: float) -> np.ndarray:
    """cap * tanh(x / cap) per element, binary32 in and out (the engine's
    final-logit softcap; closed form only, the reference never applies one)."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    out = np.empty_like(a)
    lib().or_softcap_row(_ptr(a, C.c_float), a.size, float(cap), _ptr(out, C.c_float))
    return out


def viable_states(next_table: np.ndarray, finals: np.ndarray) -> np.ndarray:
    nt = np.ascontiguousarray(next_table, dtype=np.int32)
    f = np.ascontiguousarray(finals, dtype=np.uint8)
    out = np.zeros(nt.shape[0], dtype=np.uint8)
    lib().or_viable_states(_ptr(nt, C.c_int32), nt.shape[0], _ptr(f, C.c_uint8), _ptr(out, C.c_uint8))
    return out


def dfa_legal_mask(next_table, viable, offsets, byte_data, state: int) -> np.ndarray:
    nt = np.ascontiguousarray(next_table, dtype=np.int32)
    vi = np.ascontiguousarray(viable, dtype=np.uint8)
    off = np.ascontiguousarray(offsets, dtype=np.int64)
    by = np.ascontiguousarray(byte_data, dtype=np.uint8)
    if by.size == 0:
        by = np.zeros(1, dtype=np.uint8)
    V = off.size - 1
    out = np.zeros((V + 31) // 32, dtype=np.uint32)
    lib().or_dfa_legal_mask(_ptr(nt, C.c_int32), _ptr(vi, C.c_uint8), nt.shape[0], _ptr(off, C.c_int64),
                            _ptr(by, C.c_uint8), V, int(state), _ptr(out, C.c_uint32))
    return out


def mask_logits(logits, legal, termination) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(logits, dtype=np.float32))
    lg = np.ascontiguousarray(np.asarray(legal, dtype=np.int32))
    tm = np.ascontiguousarray(np.asarray(termination, dtype=np.int32))
    out = np.empty_like(x)
    lib().or_mask_logits(_ptr(x, C.c_float), x.size, _ptr(lg, C.c_int32), lg.size, _ptr(tm, C.c_int32), tm.size,
                         _ptr(out, C.c_float))
    return out


def mask_bits_to_ids(mask: np.ndarray, V: int) -> np.ndarray:
    bits = np.unpackbits(mask.view(np.uint8), bitorder="little")[:V]
    return np.nonzero(bits)[0].astype(np.int32)


# ------------------------------------------------ int2 QAT linear (qat_ref.c)
def pack_int2_rows(codes, out_features: int, in_features: int) -> np.ndarray:
    """packInt2Rows (src/reference/qat-linear.ts:45-71); raises the reference's errors."""
    if in_features % 16 != 0:
        raise ValueError("Int2 input width must be divisible by 16")
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    if c.size != out_features * in_features:
        raise ValueError("Int2 code count does not match the matrix shape")
    words = np.zeros(c.size // 16, dtype=np.uint32)
    if lib().or_pack_int2_rows(_ptr(c, C.c_uint8), out_features, in_features, _ptr(words, C.c_uint32)) == -1:
        raise ValueError("Int2 codes must be between 0 and 3")
    return words


def unpack_int2(words, index: int) -> int:
    w = np.ascontiguousarray(words, dtype=np.uint32)
    return int(lib().or_unpack_int2(_ptr(w, C.c_uint32), index))


def apply_srq(value: float, scale: float) -> float:
    return float(lib().or_apply_srq(value, scale))


def qat_linear_int2(inputs, words, row_scales, in_features: int, out_features: int, input_scale: float = 0.0,
                    output_scale: float = 0.0) -> np.ndarray:
    """cpuQatLinear with bits 2 (src/reference/qat-linear.ts:78-116) over row-major words."""
    x = np.ascontiguousarray(inputs, dtype=np.float32)
    w = np.ascontiguousarray(words, dtype=np.uint32)
    sc = np.ascontiguousarray(row_scales, dtype=np.float32)
    assert x.size == in_features and sc.size == out_features and w.size * 16 == in_features * out_features
    out = np.zeros(out_features, dtype=np.float32)
    lib().or_qat_linear_int2(_ptr(x, C.c_float), _ptr(w, C.c_uint32), _ptr(sc, C.c_float), in_features, out_features,
                             input_scale, output_scale, _ptr(out, C.c_float))
    return out


def repack_block_major(words, out_features: int, in_features: int) -> np.ndarray:
    w = np.ascontiguousarray(words, dtype=np.uint32)
    out = np.zeros_like(w)
    lib().or_repack_block_major(_ptr(w, C.c_uint32), out_features, in_features, _ptr(out, C.c_uint32))
    return out
