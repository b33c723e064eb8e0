"""gwenedeg_amd: the MI355X backend of gwenedeg's forward hot path, from Python.

The product is the C-ABI library ``lib/libgwenedeg_amd.so`` (include/gwenedeg_gpu.h): the forward half of the
reference's runq.h (rq_model_load, rq_seq_*, rq_ctx_*, rq_decode, rq_prefill, rq_forward_batch) on gfx950 kernels.
This module binds it with ctypes and mirrors that interface one to one (same names, argument meaning, error codes):

    m = Model(path)                      # rq_model_load (no tokenizer: token ids in, logits out)
    s = m.seq(capacity)                  # rq_seq_new (f16 KV cache in device memory)
    c = m.ctx(max_batch, max_ctx)        # rq_ctx_new
    lg = c.decode(s, token)              # rq_decode -> logits (numpy copy)
    lg = c.prefill(s, tokens, mode)      # rq_prefill
    lg = c.forward_batch([Segment(...)]) # rq_forward_batch

Errors raise RqError carrying the RQ_ERR_* code and rq_ctx_error's text. There is no CPU fallback: importing the
module without the built library raises ImportError (build it with __graft_entry__.build()).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(_HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libgwenedeg_amd.so")
SYNTH_PATH = os.path.join(LIB_DIR, "libgwsynth.so")

RQ_OK, RQ_ERR_ARG, RQ_ERR_NOMEM, RQ_ERR_CONTEXT, RQ_ERR_STATE, RQ_ERR_LOAD, RQ_ERR_IO, RQ_ERR_MISMATCH = 0, -1, -2, -3, -4, -5, -6, -7
RQ_LOGITS_NONE, RQ_LOGITS_LAST, RQ_LOGITS_ALL = 0, 1, 2
RQ_KV_F32, RQ_KV_BF16, RQ_KV_F16, RQ_KV_Q8, RQ_KV_Q4, RQ_KV_Q4K4 = 0, 1, 2, 3, 8, 9  # runq.h:214
# the bf16 dot-product attention types (runq.h:214, KV_DOT 4)
RQ_KV_BF16_DOT, RQ_KV_F16_DOT, RQ_KV_Q8_DOT, RQ_KV_Q4_DOT, RQ_KV_Q4K4_DOT = 5, 6, 7, 12, 13
RQ_BATCH_MAX = 512
GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 8, 12, 14


class RqError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what} (code {code})")
        self.code = code


# One HIP runtime per process. torch ships its own libamdhip64 (same soname, loaded by path); when the library is
# loaded first it binds the system runtime, torch then loads a second copy, and the second runtime to initialise finds
# no device. Importing torch first (when it is installed) makes the library bind to torch's copy.
try:
    import torch  # noqa: F401
except ImportError:
    pass


def _load(path: str) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise ImportError(f"gwenedeg_amd: {path} is not built (run __graft_entry__.build())")
    return ctypes.CDLL(path)


lib = _load(LIB_PATH)


lib.gw_exact_mode.restype = ctypes.c_int
lib.gw_exact_mode.argtypes = []


def exact_mode() -> int:
    """gw_exact_mode: bits 0 and 1 set when the device reproduces the reference's host float operations bit for bit
    (after a load); bit 2: libmvec's expf by its method, no table"""
    return lib.gw_exact_mode()


class RqModelOpts(ctypes.Structure):  # runq.h:63-81
    _fields_ = [("ctx_len", ctypes.c_int), ("tokenizer_only", ctypes.c_int), ("no_tokenizer", ctypes.c_int),
                ("mem", ctypes.c_double), ("kv_bits", ctypes.c_int), ("page_cache", ctypes.c_int),
                ("checkpoints", ctypes.c_int), ("repack", ctypes.c_int)]


class RqModelInfo(ctypes.Structure):  # runq.h:132-146
    _fields_ = [(n, ctypes.c_int) for n in ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "head_dim",
                                            "vocab_size", "seq_len", "ctx_max", "group_size", "shared_classifier",
                                            "gguf", "bos", "eos")] + \
               [("warning", ctypes.c_char_p), ("chat", ctypes.c_int), ("rope_theta", ctypes.c_float),
                ("linear_layers", ctypes.c_int), ("fingerprint", ctypes.c_ulonglong)]


class RqSegment(ctypes.Structure):  # runq.h:364-374
    _fields_ = [("seq", ctypes.c_void_p), ("tokens", ctypes.POINTER(ctypes.c_int)), ("n", ctypes.c_int),
                ("logits", ctypes.c_int), ("hidden", ctypes.POINTER(ctypes.c_float)),
                ("h_in", ctypes.POINTER(ctypes.c_float))]


_P, _I, _F = ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_float)
_sig = {
    "rq_strerror": (ctypes.c_char_p, [_I]),
    "rq_model_load": (_P, [ctypes.c_char_p, ctypes.POINTER(RqModelOpts), ctypes.c_char_p, ctypes.c_size_t]),
    "rq_model_free": (None, [_P]),
    "rq_model_info": (None, [_P, ctypes.POINTER(RqModelInfo)]),
    "rq_seq_new": (_P, [_P, _I, _I, ctypes.POINTER(_I)]),
    "rq_seq_free": (None, [_P]),
    "rq_seq_reset": (None, [_P]),
    "rq_seq_truncate": (_I, [_P, _I]),
    "rq_seq_len": (_I, [_P]),
    "rq_seq_capacity": (_I, [_P]),
    "rq_seq_tokens": (ctypes.POINTER(_I), [_P]),
    "rq_seq_copy": (_I, [_P, _P, _I]),
    "rq_seq_fill_synthetic": (_I, [_P, _I, ctypes.c_ulonglong]),
    "rq_seq_common_prefix": (_I, [_P, ctypes.POINTER(_I), _I]),
    "rq_seq_save": (_I, [_P, ctypes.c_char_p]),
    "rq_seq_load": (_I, [_P, ctypes.c_char_p, _I]),
    "rq_seq_release": (_I, [_P, _I]),
    "rq_seq_kv_bytes": (ctypes.c_size_t, [_P, _I]),
    "rq_seq_resident": (None, [_P, _P]),
    "gw_seq_lazy": (_I, [_I]),
    "gw_seq_device_bytes": (ctypes.c_size_t, [_P]),
    "rq_ctx_new": (_P, [_P, _I, _I, ctypes.POINTER(_I)]),
    "rq_ctx_free": (None, [_P]),
    "rq_ctx_error": (ctypes.c_char_p, [_P]),
    "rq_ctx_max_batch": (_I, [_P]),
    "rq_decode": (_I, [_P, _P, _I, ctypes.POINTER(_F)]),
    "rq_decode_hidden": (_I, [_P, _P, _I, ctypes.POINTER(_F), _F, _F]),
    "rq_prefill": (_I, [_P, _P, ctypes.POINTER(_I), _I, _I, _F, ctypes.POINTER(_F)]),
    "fw_rows": (_I, [_P, _P, ctypes.POINTER(_I), _I, _I, _F, ctypes.POINTER(_F), _F, _F]),
    "rq_forward_batch": (_I, [_P, ctypes.POINTER(RqSegment), _I, _F, ctypes.POINTER(_F)]),
    "rq_logits_hash": (ctypes.c_ulonglong, [_F, _I]),
    "gw_ctx_argmax": (_I, [_P, ctypes.POINTER(_I), _I]),
    "gw_ctx_stream": (_P, [_P]),
    "gw_decode_argmax": (_I, [_P, _P, _I, ctypes.POINTER(_I)]),
    "gw_decode_greedy": (_I, [_P, _P, _I, _I, ctypes.POINTER(_I)]),
    "gw_forward_batch_device": (_I, [_P, ctypes.POINTER(RqSegment), _I]),
    "gw_ctx_profile_enable": (_I, [_P, _I]),
    "gw_ctx_gemv_sweep": (_I, [_P, _I, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I)]),
    "gw_ctx_profile_launches": (ctypes.c_long, [_P, _I]),
    "gw_ctx_kernel_timing": (_I, [_P, _I]),
    "gw_ctx_kernel_times": (_I, [_P, _I, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_double),
                                 ctypes.POINTER(ctypes.c_long), _I]),
    "rq_ctx_profile": (_I, [_P, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_double), _I]),
    "gw_q8_pack": (_I, [_P, _I, _I, _P, _P, _P]),
    "gw_quantize": (_I, [_P, _I, _I, _P, _P, _P]),
    "gw_q8_matmul": (_I, [_P, _P, _P, _I, _I, _P, _P, _I, _P]),
    "gw_q8_block_sums": (_I, [_P, _P, _I, _I, _P, _I, _P]),
    "gw_kq_matmul": (_I, [_P, _I, _P, _I, _I, _P, _P, _I, _P]),
    "gw_topk_rows": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P]),
    "gw_matmul_tile_rows": (_I, [_I]),
    "gw_kq32_quads": (_I, [_I]),
    "gw_kq32_step": (_I, [_I]),
    "gw_kq_small_kernel": (_I, [_I]),
    "gw_q8_batch_kernel": (_I, [_I]),
    "gw_q8_gemm_kernel": (_I, [_I]),
    "gw_gemv_warm_next": (_I, [_I]),
    "gw_ctx_topk": (_I, [_P, _I, _I, _F, ctypes.POINTER(_I)]),
    "gw_ctx_topk_noalloc": (_I, [_P, _I, _I, _F, ctypes.POINTER(_I)]),
    "gw_sample_topk": (_I, [_F, ctypes.POINTER(_I), _I, ctypes.c_float, ctypes.c_float, ctypes.POINTER(ctypes.c_ulonglong)]),
}
for _name, (_res, _args) in _sig.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args

EXPORTED = tuple(_sig)


def _iptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int))


def _fptr(a: Optional[np.ndarray]):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)) if a is not None else None


class Model:
    """rq_model_load / rq_model_free / rq_model_info (runq.h:87-147)."""

    def __init__(self, path: str, ctx_len: int = 0, repack: int = 0):
        opts = RqModelOpts(ctx_len=ctx_len, no_tokenizer=1, mem=-1.0, repack=repack)
        err = ctypes.create_string_buffer(512)
        self._h = lib.rq_model_load(path.encode(), ctypes.byref(opts), err, 512)
        if not self._h:
            raise RqError(RQ_ERR_LOAD, f"rq_model_load: {err.value.decode(errors='replace')}")
        self.info = RqModelInfo()
        lib.rq_model_info(self._h, ctypes.byref(self.info))
        self.vocab = self.info.vocab_size
        self.dim = self.info.dim

    def seq(self, capacity: int = 0, kv_type: int = RQ_KV_F16) -> "Seq":
        return Seq(self, capacity, kv_type)

    def ctx(self, max_batch: int = RQ_BATCH_MAX, max_ctx: int = 0) -> "Ctx":
        return Ctx(self, max_batch, max_ctx)

    def close(self):
        if self._h:
            lib.rq_model_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class RqSeqMem(ctypes.Structure):  # runq.h:152-157
    _fields_ = [("kv", ctypes.c_size_t), ("state", ctypes.c_size_t), ("checkpoints", ctypes.c_int), ("total", ctypes.c_size_t)]


class Seq:
    """rq_seq_* (runq.h:222-282): a sequence and its device KV cache."""

    def __init__(self, model: Model, capacity: int = 0, kv_type: int = RQ_KV_F16):
        e = ctypes.c_int(0)
        self.model = model
        self._h = lib.rq_seq_new(model._h, capacity, kv_type, ctypes.byref(e))
        if not self._h:
            raise RqError(e.value, "rq_seq_new")

    def __len__(self):
        return lib.rq_seq_len(self._h)

    @property
    def capacity(self) -> int:
        return lib.rq_seq_capacity(self._h)

    def tokens(self) -> np.ndarray:
        n = len(self)
        p = lib.rq_seq_tokens(self._h)
        return np.ctypeslib.as_array(p, shape=(n,)).copy() if n else np.zeros(0, np.int32)

    def reset(self):
        lib.rq_seq_reset(self._h)

    def truncate(self, n: int):
        r = lib.rq_seq_truncate(self._h, n)
        if r != RQ_OK:
            raise RqError(r, "rq_seq_truncate")

    def copy_from(self, src: "Seq", n: int):
        r = lib.rq_seq_copy(self._h, src._h, n)
        if r != RQ_OK:
            raise RqError(r, "rq_seq_copy")

    def fill_synthetic(self, n: int, seed: int = 1):
        r = lib.rq_seq_fill_synthetic(self._h, n, seed)
        if r != RQ_OK:
            raise RqError(r, "rq_seq_fill_synthetic")

    def save(self, path: str):
        """rq_seq_save (runq.h:293): the sequence in the reference's saved-sequence format"""
        r = lib.rq_seq_save(self._h, path.encode())
        if r != RQ_OK:
            raise RqError(r, "rq_seq_save")

    def load(self, path: str, n: int):
        """rq_seq_load (runq.h:314): the first n positions of a saved sequence"""
        r = lib.rq_seq_load(self._h, path.encode(), n)
        if r != RQ_OK:
            raise RqError(r, "rq_seq_load")

    def release(self, keep: int = 0):
        """rq_seq_release (runq.h:270): the memory past max(keep, len) goes"""
        r = lib.rq_seq_release(self._h, keep)
        if r != RQ_OK:
            raise RqError(r, "rq_seq_release")

    def resident(self) -> RqSeqMem:
        """rq_seq_resident (runq.h:274)"""
        out = RqSeqMem()
        lib.rq_seq_resident(self._h, ctypes.byref(out))
        return out

    def kv_bytes(self, n: int) -> int:
        """rq_seq_kv_bytes (runq.h:277)"""
        return lib.rq_seq_kv_bytes(self._h, n)

    def device_bytes(self) -> int:
        """gw_seq_device_bytes: the device memory the K / V caches hold now"""
        return lib.gw_seq_device_bytes(self._h)

    def close(self):
        if self._h:
            lib.rq_seq_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class Segment:
    """RqSegment (runq.h:364-374): n tokens appended to seq at its next positions."""
    seq: Seq
    tokens: Sequence[int]
    logits: int = RQ_LOGITS_LAST
    hidden: bool = False


class Ctx:
    """rq_ctx_* and the forward passes (runq.h:325-375)."""

    def __init__(self, model: Model, max_batch: int = RQ_BATCH_MAX, max_ctx: int = 0):
        e = ctypes.c_int(0)
        self.model = model
        self._h = lib.rq_ctx_new(model._h, max_batch, max_ctx, ctypes.byref(e))
        if not self._h:
            raise RqError(e.value, "rq_ctx_new")

    def _check(self, r: int, what: str):
        if r != RQ_OK:
            raise RqError(r, f"{what}: {lib.rq_ctx_error(self._h).decode(errors='replace')}")

    @property
    def max_batch(self) -> int:
        return lib.rq_ctx_max_batch(self._h)

    @property
    def stream(self) -> int:
        return lib.gw_ctx_stream(self._h) or 0

    def decode(self, seq: Seq, token: int, logits: bool = True) -> Optional[np.ndarray]:
        p = ctypes.POINTER(ctypes.c_float)()
        self._check(lib.rq_decode(self._h, seq._h, int(token), ctypes.byref(p) if logits else None), "rq_decode")
        return np.ctypeslib.as_array(p, shape=(self.model.vocab,)).copy() if logits else None

    def decode_hidden(self, seq: Seq, token: int):
        p = ctypes.POINTER(ctypes.c_float)()
        hid = np.zeros(self.model.dim, np.float32)
        self._check(lib.rq_decode_hidden(self._h, seq._h, int(token), ctypes.byref(p), _fptr(hid), None), "rq_decode_hidden")
        return np.ctypeslib.as_array(p, shape=(self.model.vocab,)).copy(), hid

    def prefill(self, seq: Seq, tokens, mode: int = RQ_LOGITS_LAST) -> Optional[np.ndarray]:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.zeros((len(t), self.model.vocab), np.float32) if mode == RQ_LOGITS_ALL else None
        p = ctypes.POINTER(ctypes.c_float)()
        self._check(lib.rq_prefill(self._h, seq._h, _iptr(t), len(t), mode, _fptr(out), ctypes.byref(p)), "rq_prefill")
        if mode == RQ_LOGITS_ALL:
            return out
        if mode == RQ_LOGITS_LAST:
            return np.ctypeslib.as_array(p, shape=(self.model.vocab,)).copy()
        return None

    def prefill_hidden(self, seq: Seq, tokens, mode: int = RQ_LOGITS_LAST):
        """fw_rows: rq_prefill plus every row's final hidden state. Returns (logits as prefill returns them, hidden rows
        (n x dim))"""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.zeros((len(t), self.model.vocab), np.float32) if mode == RQ_LOGITS_ALL else None
        hid = np.zeros((len(t), self.model.dim), np.float32)
        p = ctypes.POINTER(ctypes.c_float)()
        self._check(lib.fw_rows(self._h, seq._h, _iptr(t), len(t), mode, _fptr(out), ctypes.byref(p), _fptr(hid), None), "fw_rows")
        if mode == RQ_LOGITS_ALL:
            return out, hid
        if mode == RQ_LOGITS_LAST:
            return np.ctypeslib.as_array(p, shape=(self.model.vocab,)).copy(), hid
        return None, hid

    def forward_batch(self, segments: Sequence[Segment]):
        """Returns (logits rows in row order or None, hidden arrays per segment (or None))."""
        n = len(segments)
        arr = (RqSegment * n)()
        keep = []
        nsel = 0
        hids = []
        for i, sg in enumerate(segments):
            t = np.ascontiguousarray(sg.tokens, dtype=np.int32)
            keep.append(t)
            h = np.zeros((len(t), self.model.dim), np.float32) if sg.hidden else None
            hids.append(h)
            arr[i] = RqSegment(sg.seq._h, _iptr(t), len(t), sg.logits, _fptr(h), None)
            nsel += len(t) if sg.logits == RQ_LOGITS_ALL else (1 if sg.logits == RQ_LOGITS_LAST else 0)
        out = np.zeros((max(nsel, 1), self.model.vocab), np.float32)
        p = ctypes.POINTER(ctypes.c_float)()
        self._check(lib.rq_forward_batch(self._h, arr, n, _fptr(out), ctypes.byref(p)), "rq_forward_batch")
        return (out[:nsel] if nsel else None), hids

    def forward_batch_argmax(self, segments: Sequence[Segment]) -> np.ndarray:
        """gw_forward_batch_device + gw_ctx_argmax: the greedy token of every selected row, chosen on the device"""
        n = len(segments)
        arr = (RqSegment * n)()
        keep = []
        nsel = 0
        for i, sg in enumerate(segments):
            t = np.ascontiguousarray(sg.tokens, dtype=np.int32)
            keep.append(t)
            arr[i] = RqSegment(sg.seq._h, _iptr(t), len(t), sg.logits, None, None)
            nsel += len(t) if sg.logits == RQ_LOGITS_ALL else (1 if sg.logits == RQ_LOGITS_LAST else 0)
        self._check(lib.gw_forward_batch_device(self._h, arr, n), "gw_forward_batch_device")
        return self.argmax(nsel) if nsel else np.zeros(0, np.int32)

    def decode_argmax(self, seq: Seq, token: int) -> int:
        """gw_decode_argmax: a decode step whose greedy next token is chosen on the device"""
        nxt = ctypes.c_int(0)
        self._check(lib.gw_decode_argmax(self._h, seq._h, int(token), ctypes.byref(nxt)), "gw_decode_argmax")
        return nxt.value

    def decode_greedy(self, seq: Seq, token: int, n: int) -> np.ndarray:
        """gw_decode_greedy: n greedy steps from token, the tokens chosen on the device (one wait for all n)"""
        out = np.zeros(n, np.int32)
        self._check(lib.gw_decode_greedy(self._h, seq._h, int(token), int(n), _iptr(out)), "gw_decode_greedy")
        return out

    def profile(self, on: bool = True):
        self._check(lib.gw_ctx_profile_enable(self._h, 1 if on else 0), "gw_ctx_profile_enable")

    def profile_read(self) -> dict:
        """{class: (seconds, launches)} since profile(True)"""
        names = (ctypes.c_char_p * 16)()
        secs = (ctypes.c_double * 16)()
        n = lib.rq_ctx_profile(self._h, names, secs, 16)
        return {names[i].decode(): (secs[i], lib.gw_ctx_profile_launches(self._h, i)) for i in range(n)}

    def kernel_timing(self, on: bool = True):
        """gw_ctx_kernel_timing: every later kernel launch of the passes records its own start / stop"""
        self._check(lib.gw_ctx_kernel_timing(self._h, 1 if on else 0), "gw_ctx_kernel_timing")

    def kernel_times(self, multi: bool = False) -> dict:
        """{class: (kernel seconds, launches)} of the one-row passes (multi False) or of the passes of several rows,
        since kernel_timing(True) (gw_ctx_kernel_times)"""
        names = (ctypes.c_char_p * 16)()
        secs = (ctypes.c_double * 16)()
        cnt = (ctypes.c_long * 16)()
        n = lib.gw_ctx_kernel_times(self._h, 1 if multi else 0, names, secs, cnt, 16)
        if n < 0:
            self._check(n, "gw_ctx_kernel_times")
        return {names[i].decode(): (secs[i], cnt[i]) for i in range(n)}

    def gemv_sweep(self, reps: int = 1):
        """gw_ctx_gemv_sweep: (seconds per sweep, weight bytes per sweep, launches per sweep)"""
        t, b, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_int()
        self._check(lib.gw_ctx_gemv_sweep(self._h, reps, ctypes.byref(t), ctypes.byref(b), ctypes.byref(n)), "gw_ctx_gemv_sweep")
        return t.value, b.value, n.value

    def topk(self, n: int, k: int):
        """gw_ctx_topk: the k best logits of the first n rows on the device and their ids, (n x k) each"""
        vals, idx = np.zeros((n, k), np.float32), np.zeros((n, k), np.int32)
        self._check(lib.gw_ctx_topk(self._h, n, k, _fptr(vals), _iptr(idx)), "gw_ctx_topk")
        return vals, idx

    def argmax(self, n: int = 1) -> np.ndarray:
        """gw_ctx_argmax: device-side greedy tokens of the last pass's first n logits rows."""
        t = np.zeros(n, np.int32)
        self._check(lib.gw_ctx_argmax(self._h, _iptr(t), n), "gw_ctx_argmax")
        return t

    def close(self):
        if self._h:
            lib.rq_ctx_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def logits_hash(lg: np.ndarray) -> int:
    a = np.ascontiguousarray(lg, dtype=np.float32)
    return int(lib.rq_logits_hash(_fptr(a), a.size))
