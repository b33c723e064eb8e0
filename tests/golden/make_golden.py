"""Writes the golden vectors of tests/test_oracle.py::test_golden_vectors from the reference's own kernels, compiled
from its sources (oracle/_ref/ref_q8op: q8p_gemv_rows / q8p_gemm_item of kernels_avx512.h, the K-quant dot of
kquants.h, and for Q2_K and the i-quants iq_rows and iq_dequant_row of iquants.h), on seeded inputs. These kernels are integer sums plus IEEE fp32 roundings, so the vectors hold on any host.

Usage: python tests/golden/make_golden.py   (needs oracle/_ref built: make -C oracle ref, with the reference's tree)
"""
import ctypes
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as orc  # noqa: E402
from gwenedeg_amd import synth  # noqa: E402


def main():
    if not orc.have_ref():
        sys.exit("make_golden: oracle/_ref is not built")
    rng = np.random.default_rng(20240601)
    out = {}
    with tempfile.TemporaryDirectory() as wd:
        for M in (1, 6):  # the GEMV and the GEMM item
            N, K = 32, 512
            wq = rng.integers(-127, 128, (N, K), dtype=np.int8)
            ws = np.abs(rng.standard_normal((N, K // 32)) * 1e-3).astype(np.float16).astype(np.float32)
            xq = rng.integers(-127, 128, (M, K), dtype=np.int8)
            xs = np.abs(rng.standard_normal((M, K // 32))).astype(np.float32)
            ref, _ = orc.run_ref_q8op(wd, wq, ws, xq, xs)
            out.update({f"q8_m{M}_wq": wq, f"q8_m{M}_ws": ws, f"q8_m{M}_xq": xq, f"q8_m{M}_xs": xs, f"q8_m{M}_out": ref})
        lib = synth.synth_library()
        for typ in (12, 14):
            N, K, M = 16, 512, 3
            w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
            blk = np.zeros((N, lib.gw_synth_row_bytes(typ, K)), np.uint8)
            for n in range(N):
                lib.gw_synth_encode_row(typ, blk[n].ctypes.data_as(ctypes.c_void_p), w[n].ctypes.data_as(ctypes.c_void_p), K)
            xq = rng.integers(-127, 128, (M, K), dtype=np.int8)
            xs = np.abs(rng.standard_normal((M, K // 32))).astype(np.float32)
            ref = orc.run_ref_kq(wd, typ, blk, xq, xs, N, K)
            out.update({f"kq{typ}_blk": blk, f"kq{typ}_xq": xq, f"kq{typ}_xs": xs, f"kq{typ}_out": ref})
        # Q2_K and the i-quants: the reference's iq_rows (its AVX-512 kernels) and iq_dequant_row (its codebooks)
        rng2 = np.random.default_rng(20261202)
        for typ in orc.IQ_TYPES:
            N, K, M = 16, 512, 3
            w = (rng2.standard_normal((N, K)) * 0.02).astype(np.float32)
            blk = np.zeros((N, lib.gw_synth_row_bytes(typ, K)), np.uint8)
            for n in range(N):
                lib.gw_synth_encode_row(typ, blk[n].ctypes.data_as(ctypes.c_void_p), w[n].ctypes.data_as(ctypes.c_void_p), K)
            xq = rng2.integers(-127, 128, (M, K), dtype=np.int8)
            xs = np.abs(rng2.standard_normal((M, K // 32))).astype(np.float32)
            ref = orc.run_ref_kq(wd, typ, blk, xq, xs, N, K)
            dq = orc.run_ref_iq_dequant(wd, typ, blk, N * K // 256)
            out.update({f"iq{typ}_blk": blk, f"iq{typ}_xq": xq, f"iq{typ}_xs": xs, f"iq{typ}_out": ref, f"iq{typ}_dq": dq})
    path = os.path.join(HERE, "ref_kernels.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
