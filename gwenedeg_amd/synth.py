"""Seeded synthetic Qwen3-shaped GGUF files (random-init weights of the named architecture; no network, no
checkpoint): the inputs of the parity tests and of bench.py. Written by lib/libgwsynth.so (csrc/gw_synth.c), a host
library of its own (no GPU needed), multithreaded, deterministic for a given (shape, types, seed).

Shapes: qwen3_0_6b (config 1), qwen3_4b_q4km (config 3), qwen3_8b (configs 4 and 5), and
small test shapes.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
_PATH = os.path.join(_HERE, "lib", "libgwsynth.so")

Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_XS = 8, 10, 11, 12, 13, 14, 23
IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ3_S, IQ2_S, IQ1_M = 16, 17, 18, 19, 21, 22, 29


class GwSynthCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in "dim hidden n_layers n_heads n_kv_heads head_dim vocab ctx_len".split()] + \
        [("rope_theta", ctypes.c_float), ("tied", ctypes.c_int), ("type_default", ctypes.c_int)] + \
        [(n, ctypes.c_int) for n in "type_embd type_out type_q type_k type_v type_o type_gate type_up type_down".split()] + \
        [("std", ctypes.c_float), ("norm_value", ctypes.c_float), ("tokenizer", ctypes.c_int)]


SHAPES = {
    # config 1: Qwen3-0.6B-shaped dense decoder, Q8_0, tied classifier
    "qwen3_0_6b": dict(dim=1024, hidden=3072, n_layers=28, n_heads=16, n_kv_heads=8, head_dim=128, vocab=151936,
                       ctx_len=40960, tied=1, type_default=Q8_0),
    # config 3: Qwen3-4B-shaped Q4_K_M: Q4_K on q/k/o/gate/up and token_embd, Q6_K on v/down/output
    "qwen3_4b_q4km": dict(dim=2560, hidden=9728, n_layers=36, n_heads=32, n_kv_heads=8, head_dim=128, vocab=151936,
                          ctx_len=40960, tied=0, type_default=Q4_K, type_v=Q6_K, type_down=Q6_K, type_out=Q6_K),
    # configs 4 / 5 (and the bench): Qwen3-8B-shaped Q8_0, untied classifier
    "qwen3_8b": dict(dim=4096, hidden=12288, n_layers=36, n_heads=32, n_kv_heads=8, head_dim=128, vocab=151936,
                     ctx_len=40960, tied=0, type_default=Q8_0),
    # test shapes (parity against the oracle in seconds)
    "tiny": dict(dim=256, hidden=512, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=128, vocab=1000, ctx_len=4096,
                 tied=1, type_default=Q8_0),
    "tiny_gqa4": dict(dim=512, hidden=1024, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=128, vocab=2048,
                      ctx_len=4096, tied=0, type_default=Q8_0),
    "tiny_kq": dict(dim=512, hidden=1024, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=128, vocab=2048,
                    ctx_len=4096, tied=0, type_default=Q4_K, type_v=Q6_K, type_down=Q6_K, type_out=Q6_K),
    # Q5_K_M-style (Q5_K with Q6_K on v / down / output) and Q3_K_M-style (Q3_K with Q5_K on v / down, Q6_K output)
    "tiny_q5k": dict(dim=512, hidden=1024, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=128, vocab=2048,
                     ctx_len=4096, tied=0, type_default=Q5_K, type_v=Q6_K, type_down=Q6_K, type_out=Q6_K),
    "tiny_q3k": dict(dim=512, hidden=1024, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=128, vocab=2048,
                     ctx_len=4096, tied=0, type_default=Q3_K, type_v=Q5_K, type_down=Q5_K, type_out=Q6_K),
    # IQ4_XS-style (the i-quant IQ4_XS on every matrix and the embedding, Q6_K output)
    "tiny_iq4xs": dict(dim=512, hidden=1024, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=128, vocab=2048,
                       ctx_len=4096, tied=0, type_default=IQ4_XS, type_out=Q6_K),
    # the codebook i-quants, each on every matrix and the embedding (Q6_K output), one shape per type
    **{f"tiny_{n.lower()}": dict(dim=512, hidden=1024, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=128, vocab=2048,
                                 ctx_len=4096, tied=0, type_default=t, type_out=Q6_K)
       for n, t in (("IQ2_XXS", IQ2_XXS), ("IQ2_XS", IQ2_XS), ("IQ2_S", IQ2_S), ("IQ3_XXS", IQ3_XXS), ("IQ3_S", IQ3_S),
                    ("IQ1_S", IQ1_S), ("IQ1_M", IQ1_M))},
    # Q2_K-style (Q2_K on most matrices and the embedding, Q4_K on v, Q6_K output)
    "tiny_q2k": dict(dim=512, hidden=1024, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=128, vocab=2048,
                     ctx_len=4096, tied=0, type_default=Q2_K, type_v=Q4_K, type_out=Q6_K),
    # head sizes below 128: 8 query heads on one KV head (hd 64), plain multi-head attention (hd 32)
    "tiny_hd64": dict(dim=256, hidden=512, n_layers=2, n_heads=8, n_kv_heads=1, head_dim=64, vocab=1000, ctx_len=4096,
                      tied=1, type_default=Q8_0),
    # 16 query heads on one KV head (hd 64): the attention's items of more than 8 query vectors per row
    "tiny_kv16": dict(dim=256, hidden=512, n_layers=2, n_heads=16, n_kv_heads=1, head_dim=64, vocab=1024, ctx_len=4096,
                      tied=1, type_default=Q8_0),
    "tiny_hd32": dict(dim=256, hidden=768, n_layers=2, n_heads=8, n_kv_heads=8, head_dim=32, vocab=1000, ctx_len=4096,
                      tied=0, type_default=Q8_0),
}


def write_gguf(path: str, shape: str | dict, seed: int = 1, threads: int = 0, **over) -> str:
    """Writes the synthetic model `shape` (a SHAPES key or a dict of GwSynthCfg fields) to path; returns path."""
    if not os.path.exists(_PATH):
        raise ImportError(f"{_PATH} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_PATH)
    lib.gw_synth_gguf.restype = ctypes.c_int
    lib.gw_synth_gguf.argtypes = [ctypes.c_char_p, ctypes.POINTER(GwSynthCfg), ctypes.c_ulonglong, ctypes.c_int]
    d = dict(SHAPES[shape]) if isinstance(shape, str) else dict(shape)
    d.update(over)
    cfg = GwSynthCfg(**d)
    if threads <= 0:
        threads = min(16, os.cpu_count() or 1)
    r = lib.gw_synth_gguf(path.encode(), ctypes.byref(cfg), seed, threads)
    if r != 0:
        raise RuntimeError(f"gw_synth_gguf({path}) failed: {r}")
    return path


def synth_library() -> ctypes.CDLL:
    lib = ctypes.CDLL(_PATH)
    lib.gw_synth_encode_row.restype = None
    lib.gw_synth_encode_row.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
    lib.gw_synth_row_bytes.restype = ctypes.c_size_t
    lib.gw_synth_row_bytes.argtypes = [ctypes.c_int, ctypes.c_int]
    return lib
