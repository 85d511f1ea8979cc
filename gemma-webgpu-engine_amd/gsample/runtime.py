"""ctypes binding of libgsample and the batched Sampler.

Device buffers are torch tensors on the context's device; every sampling
decision is made by the HIP kernels behind the C ABI.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from .config import DecodingConfig, validate_decoding_config

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
# GSAMPLE_CHECKED=1 loads the checked build (range checks on the finish's
# array indices; a violation flags the row GS_FLAG_INDEX_CHECK and replays it
# on the exact path)
LIB_PATH = os.path.join(PKG, "lib", "libgsample_checked.so" if os.environ.get("GSAMPLE_CHECKED") == "1"
                        else "libgsample.so")

GS_F32, GS_BF16 = 0, 1
GS_QAT_ROW_MAJOR, GS_QAT_BLOCK_MAJOR = 0, 1
GS_RNG_SEEDED, GS_RNG_EXPLICIT = 0, 1
GS_ROW_FORCE_EXACT = 1
GS_BATCH_FULL_DRAWS = 1  # gs_batch.hints: a row may take a full-vocabulary draw
GS_BATCH_FUSED_HEAD = 2  # gs_batch.hints: gs_lmhead_sample computes the chunk statistics in the head
GS_FORCED_TERMINATION, GS_FORCED_EXTRA = 1, 2
GS_FLAG_TOPP_TIE = 1
GS_FLAG_EXACT_PATH = 2
GS_FLAG_NEAR_TIE = 4
GS_FLAG_DEAD_END = 8
GS_FLAG_NONFINITE = 16
GS_FLAG_EMPTY_CANDIDATES = 32
GS_FLAG_GREEDY = 64
GS_FLAG_UNSUPPORTED = 128
GS_FLAG_INVALID_SLOT = 256
GS_FLAG_INDEX_CHECK = 512  # a workspace index failed its range check (row replayed exactly)

GS_OK = 0
GS_ERR_DEAD_END = 4
GS_ERR_CONSTRAINT_VIOLATION = 5
GS_ERR_TOKEN_RANGE = 6


class GSampleError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class RowConfig(C.Structure):
    """gs_row_config (include/gsample.h)."""

    _fields_ = [
        ("temperature", C.c_double),
        ("top_p", C.c_double),
        ("min_p", C.c_double),
        ("typical_p", C.c_double),
        ("repetition_penalty", C.c_double),
        ("frequency_penalty", C.c_double),
        ("presence_penalty", C.c_double),
        ("softcap", C.c_double),
        ("uniform", C.c_double),
        ("seed", C.c_int64),
        ("draw_index", C.c_uint64),
        ("top_k", C.c_int32),
        ("repetition_window", C.c_int32),
        ("rng_mode", C.c_int32),
        ("mask_slot", C.c_int32),
        ("accepting", C.c_int32),
        ("options", C.c_int32),
    ]


class RowResult(C.Structure):
    _fields_ = [("token", C.c_int32), ("flags", C.c_uint32), ("probability", C.c_double)]


class Batch(C.Structure):
    _fields_ = [
        ("logits", C.c_void_p),
        ("row_stride", C.c_int64),
        ("dtype", C.c_int32),
        ("rows", C.c_int32),
        ("configs", C.c_void_p),
        ("history_offsets", C.c_void_p),
        ("history_ids", C.c_void_p),
        ("forced_offsets", C.c_void_p),
        ("forced_ids", C.c_void_p),
        ("forced_kinds", C.c_void_p),
        ("mask_table", C.c_void_p),
        ("mask_slots", C.c_int32),
        ("hints", C.c_int32),
        ("results", C.c_void_p),
    ]


ROW_CONFIG_DTYPE = np.dtype([
    ("temperature", "<f8"), ("top_p", "<f8"), ("min_p", "<f8"), ("typical_p", "<f8"),
    ("repetition_penalty", "<f8"), ("frequency_penalty", "<f8"), ("presence_penalty", "<f8"),
    ("softcap", "<f8"), ("uniform", "<f8"), ("seed", "<i8"), ("draw_index", "<u8"), ("top_k", "<i4"),
    ("repetition_window", "<i4"), ("rng_mode", "<i4"), ("mask_slot", "<i4"), ("accepting", "<i4"),
    ("options", "<i4"),
])
RESULT_DTYPE = np.dtype([("token", "<i4"), ("flags", "<u4"), ("probability", "<f8")])
assert ROW_CONFIG_DTYPE.itemsize == C.sizeof(RowConfig)
assert RESULT_DTYPE.itemsize == C.sizeof(RowResult)

EXPORTED_SYMBOLS = (
    "gs_abi_version", "gs_device_count", "gs_seeded_random", "gs_js_exp", "gs_js_log", "gs_softcap",
    "gs_validate_configs", "gs_create", "gs_destroy", "gs_last_error", "gs_synchronize", "gs_stream",
    "gs_sample", "gs_sample_noalloc", "gs_sample_sync", "gs_token_log_prob", "gs_token_log_prob_host", "gs_set_vocab", "gs_set_dfa",
    "gs_build_masks", "gs_dfa_advance", "gs_dfa_accepting", "gs_lmhead", "gs_lmhead_sample", "gs_qat_lmhead", "gs_qat_lmhead_sample", "gs_timing_begin",
    "gs_timing_end", "gs_check_exp2",
)

# kernel stages reported by gs_timing_end (include/gsample.h GS_STAGE_*)
STAGES = ("lmhead", "scan", "finish", "exact", "deep")

_lib = None


def library():
    """Load libgsample.so; raises when it has not been built (no CPU fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise GSampleError(-1, f"libgsample.so is not built ({LIB_PATH}); run __graft_entry__.build()")
    L = C.CDLL(LIB_PATH)
    vp, i32, i64, u64 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64
    L.gs_abi_version.restype = C.c_int
    L.gs_device_count.argtypes = [C.POINTER(C.c_int)]
    L.gs_seeded_random.restype = C.c_double
    L.gs_seeded_random.argtypes = [i64, u64]
    L.gs_js_exp.restype = C.c_double
    L.gs_js_exp.argtypes = [C.c_double]
    L.gs_js_log.restype = C.c_double
    L.gs_js_log.argtypes = [C.c_double]
    L.gs_softcap.restype = C.c_float
    L.gs_softcap.argtypes = [C.c_float, C.c_double]
    L.gs_validate_configs.argtypes = [vp, vp, i32]
    L.gs_create.argtypes = [C.c_int, i32, i32, C.POINTER(vp)]
    L.gs_destroy.argtypes = [vp]
    L.gs_last_error.restype = C.c_char_p
    L.gs_last_error.argtypes = [vp]
    L.gs_synchronize.argtypes = [vp]
    L.gs_stream.restype = vp
    L.gs_stream.argtypes = [vp]
    L.gs_sample.argtypes = [vp, C.POINTER(Batch), vp]
    L.gs_sample_sync.argtypes = [vp, C.POINTER(Batch), vp]
    L.gs_sample_noalloc.argtypes = [C.POINTER(Batch), i32, vp]
    L.gs_token_log_prob.argtypes = [vp, vp, i32, i32, i64, vp, vp, vp]
    L.gs_token_log_prob_host.argtypes = [vp, vp, i32, vp, vp]
    L.gs_set_vocab.argtypes = [vp, vp, vp, i64]
    L.gs_set_dfa.argtypes = [vp, i32, vp, vp]
    L.gs_build_masks.argtypes = [vp, vp, i32, vp, vp]
    L.gs_dfa_advance.argtypes = [vp, vp, vp, i32, vp]
    L.gs_dfa_accepting.argtypes = [vp, i32, C.POINTER(C.c_int32)]
    L.gs_lmhead.argtypes = [vp, vp, vp, i32, i32, C.c_float, vp, vp]
    L.gs_lmhead_sample.argtypes = [vp, vp, vp, i32, C.c_float, vp, C.POINTER(Batch), vp]
    L.gs_qat_lmhead.argtypes = [vp, vp, i32, i32, vp, i32, vp, C.c_float, C.c_float, vp, vp]
    L.gs_qat_lmhead_sample.argtypes = [vp, vp, i32, vp, i32, vp, C.c_float, C.c_float, vp, C.POINTER(Batch), vp]
    L.gs_timing_begin.argtypes = [vp, i32]
    L.gs_timing_end.argtypes = [vp, vp, vp]
    L.gs_check_exp2.argtypes = [vp, C.c_float, C.c_float, C.POINTER(C.c_double), C.POINTER(C.c_float)]
    _lib = L
    return L


def js_exp(x: float) -> float:
    return float(library().gs_js_exp(float(x)))


def js_log(x: float) -> float:
    return float(library().gs_js_log(float(x)))


def softcap(x: float, cap: float) -> float:
    return float(library().gs_softcap(float(x), float(cap)))


class SeededRandom:
    """SeededRandom (src/runtime/sampling.ts:3-16): next() is the library's
    counter-based Mulberry32 draw, the same function the kernels evaluate."""

    def __init__(self, seed: int):
        self.seed = int(seed)
        self.index = 0

    def next(self) -> float:
        v = float(library().gs_seeded_random(self.seed, self.index))
        self.index += 1
        return v

    __call__ = next


def _np_ptr(a: np.ndarray):
    return C.c_void_p(a.ctypes.data)


def row_config(config: DecodingConfig, *, seed: Optional[int] = None, draw_index: int = 0,
               uniform: Optional[float] = None, softcap_value: float = 0.0, mask_slot: int = -1,
               accepting: bool = False, force_exact: bool = False) -> np.void:
    """One gs_row_config from a DecodingConfig (sampling fields only)."""
    c = np.zeros((), dtype=ROW_CONFIG_DTYPE)
    c["temperature"] = config.temperature
    c["top_p"] = config.topP
    c["min_p"] = config.minP
    c["typical_p"] = config.typicalP
    c["repetition_penalty"] = config.repetitionPenalty
    c["frequency_penalty"] = config.frequencyPenalty
    c["presence_penalty"] = config.presencePenalty
    c["softcap"] = softcap_value
    c["top_k"] = config.topK
    c["repetition_window"] = config.repetitionWindow
    if uniform is not None:
        c["rng_mode"] = GS_RNG_EXPLICIT
        c["uniform"] = uniform
    else:
        c["rng_mode"] = GS_RNG_SEEDED
        c["seed"] = config.seed if seed is None else seed
        c["draw_index"] = draw_index
    c["mask_slot"] = mask_slot
    c["accepting"] = 1 if accepting else 0
    c["options"] = GS_ROW_FORCE_EXACT if force_exact else 0
    return c


@dataclass
class SampleOutput:
    tokens: np.ndarray
    probabilities: np.ndarray
    flags: np.ndarray


def full_draw_rows(cfg: np.ndarray) -> bool:
    """Whether any packed row config may take a full-vocabulary draw
    (temperature > 0, topK 0, topP 1, no min-p or typical-p, no mask): the
    batch hint GS_BATCH_FULL_DRAWS (include/gsample.h)."""
    c = np.asarray(cfg).reshape(-1)
    return bool(np.any((c["temperature"] > 0) & (c["top_k"] <= 0) & (c["top_p"] >= 1) & ~(c["min_p"] > 0)
                       & (c["typical_p"] >= 1) & (c["mask_slot"] < 0)))


def _csr(lists: Optional[Sequence[Sequence[int]]], rows: int):
    if lists is None:
        return None, None
    offsets = np.zeros(rows + 1, dtype=np.int64)
    for i, l in enumerate(lists):
        offsets[i + 1] = offsets[i] + len(l)
    ids = np.zeros(max(1, int(offsets[-1])), dtype=np.int32)
    pos = 0
    for l in lists:
        ids[pos:pos + len(l)] = np.asarray(l, dtype=np.int32)
        pos += len(l)
    return offsets, ids


class Sampler:
    """A libgsample context on one GPU: batched sampling, masks, lm_head."""

    def __init__(self, vocab_size: int = 262144, max_rows: int = 256, device: int = 0):
        import torch

        self.torch = torch
        self.lib = library()
        self.vocab = int(vocab_size)
        self.max_rows = int(max_rows)
        self.device = torch.device("cuda", device)
        ctx = C.c_void_p()
        st = self.lib.gs_create(device, self.vocab, self.max_rows, C.byref(ctx))
        if st != GS_OK:
            raise GSampleError(st, f"gs_create failed with status {st}")
        self.ctx = ctx
        self.mask_words = (self.vocab + 31) // 32

    # -- plumbing ------------------------------------------------------
    def close(self):
        if getattr(self, "ctx", None):
            self.lib.gs_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, st: int):
        if st != GS_OK:
            raise GSampleError(st, self.lib.gs_last_error(self.ctx).decode())

    def stream_ptr(self) -> int:
        return int(self.lib.gs_stream(self.ctx) or 0)

    def synchronize(self):
        self._check(self.lib.gs_synchronize(self.ctx))

    def to_device(self, a: np.ndarray):
        t = self.torch.from_numpy(np.ascontiguousarray(a))
        return t.to(self.device)

    def validate(self, configs: np.ndarray):
        cfg = np.ascontiguousarray(configs, dtype=ROW_CONFIG_DTYPE)
        self._check(self.lib.gs_validate_configs(self.ctx, _np_ptr(cfg), cfg.size))

    # -- batched sampling ------------------------------------------------
    def prepare(self, logits, configs: np.ndarray, histories=None, forced=None, mask_table=None,
                hints: Optional[int] = None):
        """Device-side batch for gs_sample; returns (Batch, keepalive). hints:
        the GS_BATCH_* bits, by default GS_BATCH_FULL_DRAWS when a row may take
        a full-vocabulary draw."""
        torch = self.torch
        rows = int(logits.shape[0])
        if logits.dtype == torch.float32:
            dtype = GS_F32
        elif logits.dtype == torch.bfloat16:
            dtype = GS_BF16
        else:
            raise GSampleError(1, "logits must be float32 or bfloat16")
        if logits.device != self.device:
            raise GSampleError(1, "logits must live on the sampler's device")
        if logits.stride(1) != 1:
            raise GSampleError(1, "logits rows must be contiguous")
        cfg = np.ascontiguousarray(configs, dtype=ROW_CONFIG_DTYPE).reshape(-1)
        if cfg.size != rows:
            raise GSampleError(1, "one config per row")
        keep = [logits]
        d_cfg = self.to_device(cfg.view(np.uint8))
        keep.append(d_cfg)
        b = Batch()
        b.logits = logits.data_ptr()
        # a one-row view may carry any leading stride; only its row is read
        b.row_stride = logits.stride(0) if rows > 1 else max(logits.stride(0), int(logits.shape[1]))
        b.dtype = dtype
        b.rows = rows
        b.configs = d_cfg.data_ptr()
        b.hints = (GS_BATCH_FULL_DRAWS if full_draw_rows(cfg) else 0) if hints is None else int(hints)
        if histories is not None:
            if isinstance(histories, tuple):
                off, ids = histories
            else:
                off, ids = _csr(histories, rows)
            d_off, d_ids = self.to_device(np.asarray(off, np.int64)), self.to_device(np.asarray(ids, np.int32))
            keep += [d_off, d_ids]
            b.history_offsets, b.history_ids = d_off.data_ptr(), d_ids.data_ptr()
        if forced is not None:
            off, ids, kinds = forced
            d_off = self.to_device(np.asarray(off, np.int64))
            d_ids = self.to_device(np.asarray(ids, np.int32))
            d_kinds = self.to_device(np.asarray(kinds, np.uint8))
            keep += [d_off, d_ids, d_kinds]
            b.forced_offsets, b.forced_ids, b.forced_kinds = d_off.data_ptr(), d_ids.data_ptr(), d_kinds.data_ptr()
        if mask_table is not None:
            keep.append(mask_table)
            b.mask_table = mask_table.data_ptr()
            b.mask_slots = int(mask_table.shape[0])
        results = torch.empty((rows, 2), dtype=torch.float64, device=self.device)  # 16 bytes per row
        keep.append(results)
        b.results = results.data_ptr()
        return b, keep

    def launch(self, batch: Batch, stream: Optional[int] = None):
        """gs_sample on `stream` (a hipStream_t handle), else on the context's
        stream after torch's current stream has drained."""
        if stream is None:
            self.torch.cuda.current_stream(self.device).synchronize()
        self._check(self.lib.gs_sample(self.ctx, C.byref(batch), C.c_void_p(stream or 0)))

    def sample(self, logits, configs: np.ndarray, histories=None, forced=None, mask_table=None,
               raise_on_failure: bool = True, hints: Optional[int] = None) -> SampleOutput:
        b, keep = self.prepare(logits, configs, histories, forced, mask_table, hints)
        self.torch.cuda.current_stream(self.device).synchronize()
        out = np.zeros(b.rows, dtype=RESULT_DTYPE)
        st = self.lib.gs_sample_sync(self.ctx, C.byref(b), _np_ptr(out))
        if st != GS_OK and raise_on_failure:
            self._check(st)
        del keep
        return SampleOutput(out["token"].copy(), out["probability"].copy(), out["flags"].copy())

    # -- tokenLogProbability -------------------------------------------
    def token_log_probability(self, logits, tokens) -> np.ndarray:
        torch = self.torch
        rows = int(logits.shape[0])
        dtype = GS_BF16 if logits.dtype == torch.bfloat16 else GS_F32
        toks = self.to_device(np.asarray(tokens, dtype=np.int32))
        out = torch.empty(rows, dtype=torch.float64, device=self.device)
        self._check(self.lib.gs_token_log_prob(self.ctx, C.c_void_p(logits.data_ptr()), dtype, rows,
                                               logits.stride(0), C.c_void_p(toks.data_ptr()),
                                               C.c_void_p(out.data_ptr()), None))
        self.synchronize()
        return out.cpu().numpy()

    # -- self-check ----------------------------------------------------
    def check_exp2(self, lo: float, hi: float):
        """(largest relative error, where) of the hardware binary32 exp2 over
        every binary32 in [lo, hi] (gs_check_exp2)."""
        err, y = C.c_double(), C.c_float()
        self._check(self.lib.gs_check_exp2(self.ctx, lo, hi, C.byref(err), C.byref(y)))
        return err.value, y.value

    # -- constraints ---------------------------------------------------
    def set_vocab(self, offsets: np.ndarray, data: np.ndarray):
        off = np.ascontiguousarray(offsets, dtype=np.int64)
        by = np.ascontiguousarray(data, dtype=np.uint8)
        if by.size == 0:
            by = np.zeros(1, np.uint8)
        self._check(self.lib.gs_set_vocab(self.ctx, _np_ptr(off), _np_ptr(by), int(off[-1])))

    def set_dfa(self, next_table: np.ndarray, finals: np.ndarray):
        nt = np.ascontiguousarray(next_table, dtype=np.int32)
        fi = np.ascontiguousarray(finals, dtype=np.uint8)
        self._check(self.lib.gs_set_dfa(self.ctx, nt.shape[0], _np_ptr(nt), _np_ptr(fi)))

    def build_masks(self, states: Sequence[int]):
        st = np.ascontiguousarray(np.asarray(states, dtype=np.int32))
        table = self.torch.zeros((max(1, st.size), self.mask_words), dtype=self.torch.int32, device=self.device)
        self._check(self.lib.gs_build_masks(self.ctx, _np_ptr(st), st.size, C.c_void_p(table.data_ptr()), None))
        return table

    def dfa_advance(self, states: Sequence[int], tokens: Sequence[int]) -> np.ndarray:
        s = np.ascontiguousarray(np.asarray(states, dtype=np.int32))
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        out = np.zeros_like(s)
        self._check(self.lib.gs_dfa_advance(self.ctx, _np_ptr(s), _np_ptr(t), s.size, _np_ptr(out)))
        return out

    def dfa_accepting(self, state: int) -> bool:
        v = C.c_int32()
        self._check(self.lib.gs_dfa_accepting(self.ctx, int(state), C.byref(v)))
        return bool(v.value)

    # -- kernel timing ---------------------------------------------------
    def timing_begin(self, max_calls: int):
        """Launch every kernel of the next `max_calls` calls with start/stop HIP events."""
        self._check(self.lib.gs_timing_begin(self.ctx, int(max_calls)))

    def timing_end(self) -> dict:
        """{stage: (summed ms, calls)} for the calls timed since timing_begin."""
        ms = np.zeros(len(STAGES), dtype=np.float64)
        calls = np.zeros(len(STAGES), dtype=np.int32)
        self._check(self.lib.gs_timing_end(self.ctx, _np_ptr(ms), _np_ptr(calls)))
        return {name: (float(ms[i]), int(calls[i])) for i, name in enumerate(STAGES)}

    # -- lm_head ---------------------------------------------------------
    def lmhead(self, hidden, weight, softcap_value: float = 0.0, out=None, stream: Optional[int] = None):
        torch = self.torch
        m, width = int(hidden.shape[0]), int(hidden.shape[1])
        if out is None:
            out = torch.empty((m, self.vocab), dtype=torch.float32, device=self.device)
        if stream is None:
            # the context's stream does not order against torch's: finish torch's
            # work on the inputs first and the kernel before `out` is handed back
            torch.cuda.current_stream(self.device).synchronize()
        self._check(self.lib.gs_lmhead(self.ctx, C.c_void_p(hidden.data_ptr()), C.c_void_p(weight.data_ptr()), m,
                                       width, float(softcap_value), C.c_void_p(out.data_ptr()),
                                       C.c_void_p(stream or 0)))
        if stream is None:
            self.synchronize()
        return out

    def qat_lmhead(self, x, packed_codes, row_scales, layout: int = 0, input_scale: float = 0.0,
                   output_scale: float = 0.0, out=None, stream: Optional[int] = None):
        """gs_qat_lmhead: the int2 QAT LM head (cpuQatLinear, src/reference/qat-linear.ts:78-148).
        x: f32 [M][width]; packed_codes: int32/uint32 words (GS_QAT_ROW_MAJOR [V][width/16] or
        GS_QAT_BLOCK_MAJOR [width/64][V][4]); row_scales: f32 [V]; all on the device."""
        torch = self.torch
        m, width = int(x.shape[0]), int(x.shape[1])
        if out is None:
            out = torch.empty((m, self.vocab), dtype=torch.float32, device=self.device)
        if stream is None:
            torch.cuda.current_stream(self.device).synchronize()
        self._check(self.lib.gs_qat_lmhead(self.ctx, C.c_void_p(x.data_ptr()), m, width,
                                           C.c_void_p(packed_codes.data_ptr()), int(layout),
                                           C.c_void_p(row_scales.data_ptr()), float(input_scale),
                                           float(output_scale), C.c_void_p(out.data_ptr()), C.c_void_p(stream or 0)))
        if stream is None:
            self.synchronize()
        return out

    def qat_lmhead_sample(self, x, packed_codes, row_scales, logits_scratch, configs: np.ndarray, layout: int = 0,
                          input_scale: float = 0.0, output_scale: float = 0.0, histories=None, forced=None,
                          mask_table=None) -> "SampleOutput":
        """gs_qat_lmhead_sample: the int2 QAT head into `logits_scratch` ([rows][V] f32), then the
        sampler on it, one call; returns the rows' results."""
        b, keep = self.prepare(logits_scratch, configs, histories, forced, mask_table)
        self.torch.cuda.current_stream(self.device).synchronize()
        self._check(self.lib.gs_qat_lmhead_sample(self.ctx, C.c_void_p(x.data_ptr()), int(x.shape[1]),
                                                  C.c_void_p(packed_codes.data_ptr()), int(layout),
                                                  C.c_void_p(row_scales.data_ptr()), float(input_scale),
                                                  float(output_scale), C.c_void_p(logits_scratch.data_ptr()),
                                                  C.byref(b), None))
        self.synchronize()
        res = keep[-1].cpu().numpy().view(np.uint8).reshape(-1)[: b.rows * 16].view(RESULT_DTYPE)
        del keep
        return SampleOutput(res["token"].copy(), res["probability"].copy(), res["flags"].copy())

    def qat_lmhead_sample_launch(self, x, packed_codes, row_scales, logits_scratch, batch: Batch, layout: int = 0,
                                 input_scale: float = 0.0, output_scale: float = 0.0, stream: Optional[int] = None):
        """gs_qat_lmhead_sample on `stream`: the int2 QAT head into `logits_scratch`, then the sampler."""
        if stream is None:
            self.torch.cuda.current_stream(self.device).synchronize()
        self._check(self.lib.gs_qat_lmhead_sample(self.ctx, C.c_void_p(x.data_ptr()), int(x.shape[1]),
                                                  C.c_void_p(packed_codes.data_ptr()), int(layout),
                                                  C.c_void_p(row_scales.data_ptr()), float(input_scale),
                                                  float(output_scale), C.c_void_p(logits_scratch.data_ptr()),
                                                  C.byref(batch), C.c_void_p(stream or 0)))

    def lmhead_sample(self, hidden, weight, softcap_value: float, logits_scratch, configs: np.ndarray,
                      histories=None, forced=None, mask_table=None, fused: bool = False) -> "SampleOutput":
        """gs_lmhead_sample: the bf16 lm_head into `logits_scratch` ([rows][V] f32), then the
        sampler, one call; returns the rows' results. fused: GS_BATCH_FUSED_HEAD (the head
        computes the chunk statistics itself)."""
        b, keep = self.prepare(logits_scratch, configs, histories, forced, mask_table)
        if fused:
            b.hints |= GS_BATCH_FUSED_HEAD
        self.lmhead_sample_launch(hidden, weight, softcap_value, logits_scratch, b)
        self.synchronize()
        res = keep[-1].cpu().numpy().view(np.uint8).reshape(-1)[: b.rows * 16].view(RESULT_DTYPE)
        del keep
        return SampleOutput(res["token"].copy(), res["probability"].copy(), res["flags"].copy())

    def lmhead_sample_launch(self, hidden, weight, softcap_value: float, logits_scratch, batch: Batch,
                             stream: Optional[int] = None):
        """gs_lmhead_sample: lm_head into `logits_scratch`, then the sampler on it."""
        width = int(hidden.shape[1])
        if stream is None:
            self.torch.cuda.current_stream(self.device).synchronize()
        self._check(self.lib.gs_lmhead_sample(self.ctx, C.c_void_p(hidden.data_ptr()), C.c_void_p(weight.data_ptr()),
                                              width, float(softcap_value), C.c_void_p(logits_scratch.data_ptr()),
                                              C.byref(batch), C.c_void_p(stream or 0)))


_default_sampler: Optional[Sampler] = None


def _sampler_for(vocab: int) -> Sampler:
    global _default_sampler
    if _default_sampler is None or _default_sampler.vocab != vocab:
        if _default_sampler is not None:
            _default_sampler.close()
        _default_sampler = Sampler(vocab_size=vocab, max_rows=8)
    return _default_sampler


def sample_token(raw_logits, history: Sequence[int], config: DecodingConfig, random) -> int:
    """sampleToken(rawLogits, history, config, random) (src/runtime/sampling.ts:18-65)
    on the GPU. random() is called once, only when temperature is not 0, as the
    reference does; its value is handed to the kernel."""
    import torch

    x = np.asarray(raw_logits, dtype=np.float32).reshape(-1)
    if x.size == 0:
        raise GSampleError(3, "Cannot sample empty logits")
    # the session validates before any sampleToken call
    # (src/runtime/generation-config.ts:62-70); so does this entry point
    check = validate_decoding_config({f: getattr(config, f) for f in (
        "temperature", "topK", "topP", "minP", "typicalP", "repetitionPenalty", "repetitionWindow",
        "frequencyPenalty", "presencePenalty")})
    if not check["ok"]:
        raise GSampleError(2, "Invalid Gemma decoding config: " + "; ".join(check["errors"]))
    s = _sampler_for(int(x.size))
    u = None if config.temperature == 0 else float(random())
    cfg = row_config(config, uniform=u if u is not None else 0.0)
    if u is None:
        cfg["rng_mode"] = GS_RNG_EXPLICIT
    logits = torch.from_numpy(x.copy()).reshape(1, -1).to(s.device)
    out = s.sample(logits, cfg.reshape(1), histories=[list(history)])
    return int(out.tokens[0])


def token_log_probability(raw_logits, token: int) -> float:
    """tokenLogProbability (src/runtime/sampling.ts:67-80) on the GPU."""
    x = np.ascontiguousarray(np.asarray(raw_logits, dtype=np.float32).reshape(1, -1))
    s = _sampler_for(int(x.shape[1]))
    if not isinstance(token, (int, np.integer)) or token < 0 or token >= x.shape[1]:
        raise GSampleError(GS_ERR_TOKEN_RANGE, f"Token {token} is outside logits length {x.shape[1]}")
    out = np.zeros(1, dtype=np.float64)
    t = np.array([token], dtype=np.int32)
    s._check(s.lib.gs_token_log_prob_host(s.ctx, _np_ptr(x), 1, _np_ptr(t), _np_ptr(out)))
    return float(out[0])
