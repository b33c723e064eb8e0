"""Python binding of the oracle (liboracle.so, oracle.c) and of the reference drivers built in oracle/_ref.

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it as the checker.
"""
from __future__ import annotations

import ctypes
import json
import os
import subprocess
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")
REF_DRIVER = os.path.join(REF_DIR, "ref_driver")
REF_Q8OP = os.path.join(REF_DIR, "ref_q8op")
REF_SAMPLE = os.path.join(REF_DIR, "ref_sample")
Q2_K, IQ4_XS = 10, 23  # (ggml type numbers: the types run by iquants.h's kernels, with the codebook i-quants below)
IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ3_S, IQ2_S, IQ1_M = 16, 17, 18, 19, 21, 22, 29
IQ_TYPES = (Q2_K, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ3_S, IQ2_S, IQ4_XS, IQ1_M)

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built (make -C oracle oracle)")
        L = ctypes.CDLL(LIB_PATH)
        P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        sig = {
            "or_fp16_to_f32": (F, [ctypes.c_uint16]),
            "or_f32_f16": (ctypes.c_uint16, [F]),
            "or_quantize": (None, [P, P, P, I]),
            "or_dot_q8": (F, [P, P, P, P, I]),
            "or_q8_matmul": (None, [P, P, P, P, P, I, I, I]),
            "or_q8_block_sums": (None, [P, P, P, I, I, I]),
            "or_q8_from_blocks": (None, [P, P, P, ctypes.c_size_t]),
            "or_kq_dequant_row": (None, [I, P, I, P]),
            "or_kq_matmul": (None, [I, P, P, P, P, I, I, I]),
            "or_kq_act_prep": (None, [P, P, P, I]),
            "or_exp_att": (F, [F]),
            "or_kv_tile": (ctypes.c_size_t, [I, I, I, I]),
            "or_attention": (None, [P, P, P, P, I, I, I, I, F]),
            "or_attention_block": (None, [P, P, P, P, P, I, I, I, I, I, F]),
            "or_att_combine": (None, [P, I, P, ctypes.c_size_t, I]),
            "or_rms_scale": (F, [P, I]),
            "or_rsqrt_ref": (F, [F]),
            "or_set_swiglu_host": (None, [I]),
            "or_rmsnorm": (None, [P, P, P, I]),
            "or_silu_exp": (F, [F]),
            "or_rope_row": (None, [P, I, I, F]),
            "or_swiglu": (None, [P, P, I]),
            "or_model_load": (P, [ctypes.c_char_p, I, ctypes.c_char_p, ctypes.c_size_t]),
            "or_model_free": (None, [P]),
            "or_model_dims": (None, [P, P]),
            "or_model_att_scale": (F, [P]),
            "or_seq_new": (P, [P]),
            "or_seq_new_kv": (P, [P, I]),
            "or_seq_new_type": (P, [P, I]),
            "or_seq_free": (None, [P]),
            "or_seq_len": (I, [P]),
            "or_seq_truncate": (None, [P, I]),
            "or_seq_copy": (None, [P, P, I]),
            "or_seq_cache": (P, [P, I, I]),
            "or_forward_token": (I, [P, P, I, P, P]),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _lib = L
    return _lib


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def quantize(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    q = np.zeros(x.shape, np.int8)
    s = np.zeros(x.shape[:-1] + (x.shape[-1] // 32,), np.float32)
    rows = x.reshape(-1, x.shape[-1])
    qr, sr = q.reshape(rows.shape), s.reshape(rows.shape[0], -1)
    for i in range(rows.shape[0]):
        lib().or_quantize(_p(qr[i]), _p(sr[i]), _p(rows[i]), rows.shape[1])
    return q, s


def q8_matmul(wq, ws, xq, xs):
    N, K = wq.shape
    M = xq.shape[0]
    out = np.zeros((M, N), np.float32)
    lib().or_q8_matmul(_p(out), _p(np.ascontiguousarray(wq)), _p(np.ascontiguousarray(ws, np.float32)),
                       _p(np.ascontiguousarray(xq)), _p(np.ascontiguousarray(xs, np.float32)), M, N, K)
    return out


def q8_block_sums(wq, xq):
    N, K = wq.shape
    M = xq.shape[0]
    out = np.zeros((M, N, K // 32), np.int32)
    lib().or_q8_block_sums(_p(out), _p(np.ascontiguousarray(wq)), _p(np.ascontiguousarray(xq)), M, N, K)
    return out


def kq_matmul(typ, blocks, xq, xs, N, K):
    M = xq.shape[0]
    out = np.zeros((M, N), np.float32)
    lib().or_kq_matmul(typ, _p(out), _p(np.ascontiguousarray(blocks)), _p(np.ascontiguousarray(xq)),
                       _p(np.ascontiguousarray(xs, np.float32)), M, N, K)
    return out


def kq_dequant_row(typ, blocks, n):
    y = np.zeros(n, np.float32)
    lib().or_kq_dequant_row(typ, _p(np.ascontiguousarray(blocks)), n, _p(y))
    return y


class Model:
    """The oracle's whole forward pass (or_forward_token: one row at a time, decode semantics)."""

    def __init__(self, path: str, cap: int = 0):
        err = ctypes.create_string_buffer(256)
        self._h = lib().or_model_load(path.encode(), cap, err, 256)
        if not self._h:
            raise RuntimeError(f"or_model_load: {err.value.decode()}")
        d = np.zeros(8, np.int32)
        lib().or_model_dims(self._h, _p(d))
        self.dim, self.hidden, self.n_layers, self.n_heads, self.n_kv_heads, self.head_dim, self.vocab, self.kv_len = \
            (int(v) for v in d)

    def seq(self, bf16: bool = False, kv_type: int = None) -> "Seq":
        """kv_type (runq.h:214: 0 f32, 1 bf16, 2 f16, ...) when given, else f16 (or bf16)"""
        return Seq(self, bf16, kv_type)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().or_model_free(self._h)
            self._h = None


class Seq:
    def __init__(self, m: Model, bf16: bool = False, kv_type: int = None):
        self.m = m
        self._h = lib().or_seq_new_type(m._h, kv_type) if kv_type is not None else lib().or_seq_new_kv(m._h, 1 if bf16 else 0)
        if not self._h:
            raise RuntimeError(f"or_seq_new: kv type {kv_type}")

    def __len__(self):
        return lib().or_seq_len(self._h)

    def forward(self, token: int, logits: bool = True, trace: bool = False):
        lg = np.zeros(self.m.vocab, np.float32) if logits else None
        tr = np.zeros((self.m.n_layers, self.m.dim), np.float32) if trace else None
        r = lib().or_forward_token(self.m._h, self._h, int(token), _p(lg), _p(tr))
        if r != 0:
            raise RuntimeError("or_forward_token failed")
        return (lg, tr) if trace else lg

    def copy_from(self, src: "Seq", n: int):
        lib().or_seq_copy(self._h, src._h, n)

    def truncate(self, n: int):
        lib().or_seq_truncate(self._h, n)

    def cache(self, layer: int, v: int) -> np.ndarray:
        n = self.m.kv_len * self.m.n_kv_heads * self.m.head_dim
        p = lib().or_seq_cache(self._h, layer, v)
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint16)), shape=(n,)).copy()

    def __del__(self):
        if getattr(self, "_h", None):
            lib().or_seq_free(self._h)
            self._h = None


def have_ref() -> bool:
    return os.path.exists(REF_DRIVER) and os.path.exists(REF_Q8OP)


def run_ref_driver(model: str, ids: np.ndarray, workdir: str, steps: int = 0, threads: int = 0, cap: int = 0,
                   batch: int = 512, all_logits: bool = False, batch_decode: int = 0, reps: int = 1, kv: bool = False,
                   hidden: bool = False, kv_type: int = 2, timeout: float = 600):
    """The reference's own CPU path (oracle/_ref/ref_driver) on a GGUF file and token ids: returns (info JSON,
    logits rows written, generated tokens, KV file path or None)."""
    os.makedirs(workdir, exist_ok=True)
    ids_path = os.path.join(workdir, "ids.bin")
    np.ascontiguousarray(ids, np.int32).tofile(ids_path)
    lg_path, tok_path, kv_path = (os.path.join(workdir, n) for n in ("logits.bin", "tokens.bin", "kv.seq"))
    cmd = [REF_DRIVER, "-m", model, "--ids", ids_path, "--steps", str(steps), "-b", str(batch),
           "--logits", lg_path, "--tokens", tok_path, "--reps", str(reps)]
    if threads:
        cmd += ["-t", str(threads)]
    if cap:
        cmd += ["-c", str(cap)]
    if all_logits:
        cmd += ["--all-logits"]
    if batch_decode:
        cmd += ["--batch-decode", str(batch_decode)]
    if kv:
        cmd += ["--kv", kv_path]
    if kv_type != 2:  # (RQ_KV_F16, the default)
        cmd += ["--kv-type", str(kv_type)]
    hid_path = os.path.join(workdir, "hidden.bin")
    if hidden:
        cmd += ["--hidden", hid_path]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    if r.returncode != 0:
        raise RuntimeError(f"ref_driver failed: {r.stderr[-2000:]}")
    info = json.loads(r.stdout.strip().splitlines()[-1])
    lg = np.fromfile(lg_path, np.float32).reshape(-1, info["vocab"])
    if hidden:  # (token by token: the rows' logits and final hidden states)
        return info, lg, np.fromfile(hid_path, np.float32).reshape(-1, info["dim"]), None
    toks = np.fromfile(tok_path, np.int32) if os.path.exists(tok_path) and os.path.getsize(tok_path) else np.zeros(0, np.int32)
    return info, lg, toks, (kv_path if kv else None)


def run_ref_plan(model: str, plan: str, workdir: str, threads: int = 0, cap: int = 0, kv_type: int = 2,
                 timeout: float = 900):
    """The reference's own CPU path on a script of passes (ref_driver --plan: sequences loaded from saved KV files,
    prefix copies, rq_forward_batch passes with greedy feeds; the command list is in oracle/ref_driver.c): returns
    (info JSON, every selected logits row in pass order, the tokens the greedy feeds chose)."""
    os.makedirs(workdir, exist_ok=True)
    plan_path, lg_path, tok_path = (os.path.join(workdir, n) for n in ("plan.txt", "plan_logits.bin", "plan_tokens.bin"))
    with open(plan_path, "w") as f:
        f.write(plan)
    cmd = [REF_DRIVER, "-m", model, "--plan", plan_path, "--logits", lg_path, "--tokens", tok_path]
    if threads:
        cmd += ["-t", str(threads)]
    if cap:
        cmd += ["-c", str(cap)]
    if kv_type != 2:
        cmd += ["--kv-type", str(kv_type)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    if r.returncode != 0:
        raise RuntimeError(f"ref_driver --plan failed: {r.stderr[-2000:]}")
    info = json.loads(r.stdout.strip().splitlines()[-1])
    lg = np.fromfile(lg_path, np.float32).reshape(-1, info["vocab"])
    toks = np.fromfile(tok_path, np.int32) if os.path.getsize(tok_path) else np.zeros(0, np.int32)
    return info, lg, toks


def run_ref_q8op(workdir: str, wq, ws, xq, xs, reps: int = 0, threads: int = 1, copies: int = 1, timeout: float = 600):
    """The reference's q8p_gemv_rows / q8p_gemm_item on given int8 inputs: returns (out M x N, timing JSON or None;
    timed runs rotate over `copies` packed copies of W)."""
    os.makedirs(workdir, exist_ok=True)
    N, K = wq.shape
    M = xq.shape[0]
    paths = [os.path.join(workdir, n) for n in ("w.bin", "ws.bin", "x.bin", "xs.bin", "out.bin")]
    for a, p in zip((wq, ws, xq, xs), paths):
        np.ascontiguousarray(a).tofile(p)
    cmd = [REF_Q8OP, "q8", *paths[:4], str(M), str(N), str(K), paths[4], str(reps), str(threads), str(copies)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    if r.returncode != 0:
        raise RuntimeError(f"ref_q8op failed: {r.stderr[-2000:]}")
    out = np.fromfile(paths[4], np.float32).reshape(M, N)
    t = json.loads(r.stdout.strip().splitlines()[-1]) if reps > 0 else None
    return out, t


def run_ref_kq(workdir: str, typ: int, blocks, xq, xs, N: int, K: int, timeout: float = 600):
    os.makedirs(workdir, exist_ok=True)
    M = xq.shape[0]
    paths = [os.path.join(workdir, n) for n in ("blk.bin", "x.bin", "xs.bin", "out.bin")]
    for a, p in zip((blocks, xq, xs), paths):
        np.ascontiguousarray(a).tofile(p)
    mode = "iq" if typ in IQ_TYPES else "kq"  # (Q2_K and the i-quants: iquants.h's packing and kernels)
    cmd = [REF_Q8OP, mode, str(typ), *paths[:3], str(M), str(N), str(K), paths[3]]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    if r.returncode != 0:
        raise RuntimeError(f"ref_q8op {mode} failed: {r.stderr[-2000:]}")
    return np.fromfile(paths[3], np.float32).reshape(M, N)


def run_ref_iq_dequant(workdir: str, typ: int, blocks, nblk: int, timeout: float = 120):
    """the reference's iq_dequant_row (iquants.h:217) on nblk blocks of an i-quant type: 256 nblk floats"""
    os.makedirs(workdir, exist_ok=True)
    pb, po = os.path.join(workdir, "dq_blk.bin"), os.path.join(workdir, "dq_out.bin")
    np.ascontiguousarray(blocks).tofile(pb)
    r = subprocess.run([REF_Q8OP, "iqdq", str(typ), pb, str(nblk), po], capture_output=True, text=True, timeout=timeout)
    if r.returncode != 0:
        raise RuntimeError(f"ref_q8op iqdq failed: {r.stderr[-2000:]}")
    return np.fromfile(po, np.float32)


def run_ref_sample(workdir: str, logits, k: int, temperature: float, topp: float, rng: int, timeout: float = 120):
    """the reference's sample_topk (sampler.c, oracle/_ref/ref_sample) on each row of logits with the coin of
    rq_rng_f32: (tokens, the RNG state after the last draw)"""
    os.makedirs(workdir, exist_ok=True)
    lp = os.path.join(workdir, "sample_logits.bin")
    x = np.ascontiguousarray(logits, np.float32)
    x.tofile(lp)
    cmd = [REF_SAMPLE, lp, str(x.shape[0]), str(x.shape[1]), str(k), repr(float(temperature)), repr(float(topp)), str(rng)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    if r.returncode != 0:
        raise RuntimeError(f"ref_sample failed: {r.stderr[-2000:]}")
    out = json.loads(r.stdout.strip().splitlines()[-1])
    return [int(t) for t in out["tokens"]], int(out["rng"], 16)
