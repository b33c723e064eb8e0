"""Benchmark of the forward hot path on one MI355X: decode + prefill tok/s of a Qwen3-8B-shaped Q8_0 model.

One step = the run shape of the reference's config 1 on the metric's model: reset the sequence, prefill a 512-token
prompt of seeded random ids (rq_prefill, one 512-row pass), then 128 greedy decode steps (rq_decode with the argmax on
the device, gw_decode_argmax). value = (512 + 128) tokens per step / seconds per step, whole job (one GPU).
Weights: random-init, N(0, 0.02) then Q8_0 (a synthetic GGUF written by gwenedeg_amd.synth, seeded); no checkpoint.

Also on the JSON line:
  roofline      the dominant kernel, the decode GEMV (k_gemv_q8 on one activation row): the decode step's weight
                matmuls run back to back (gw_ctx_gemv_sweep) and timed with HIP events on the context's stream;
                achieved = file-format weight bytes per launch / average launch duration, against 8 TB/s HBM
  cpu_baseline  the reference's own CPU path (oracle/_ref/ref_driver, -Ofast AVX-512 VNNI) on the same GGUF file and
                prompt, all host cores, a bounded sample (the 512-token prefill + 32 decode steps), scaled to one step

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--prompt 512] [--gen 128] [--no-cpu-baseline]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--gen", type=int, default=128)
    ap.add_argument("--shape", default="qwen3_8b")
    ap.add_argument("--model", default="")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-decode", type=int, default=32)
    ap.add_argument("--workdir", default=os.environ.get("GW_BENCH_DIR", "/dev/shm/gwenedeg_bench" if os.path.isdir("/dev/shm")
                                                                      else "/tmp/gwenedeg_bench"))
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {a.gpus} is not supported (use --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import torch
    import gwenedeg_amd as gw
    from gwenedeg_amd import synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    os.makedirs(a.workdir, exist_ok=True)
    path = a.model or os.path.join(a.workdir, f"{a.shape}_seed{a.seed}.gguf")
    if not os.path.exists(path):
        t0 = time.time()
        synth.write_gguf(path, a.shape, seed=a.seed)
        log(f"synthetic {a.shape} GGUF written in {time.time() - t0:.1f} s: {os.path.getsize(path) / 1e9:.2f} GB")
    cap = (a.prompt + a.gen + 255) // 256 * 256
    t0 = time.time()
    m = gw.Model(path, ctx_len=cap)
    log(f"model loaded to the device in {time.time() - t0:.1f} s")
    c = m.ctx(max_batch=min(512, max(a.prompt, 2)), max_ctx=cap)
    s = m.seq(cap)
    ids = np.random.default_rng(a.seed).integers(0, m.vocab, a.prompt).astype(np.int32)

    def step():
        s.reset()
        t0 = time.perf_counter()
        c.prefill(s, ids, mode=gw.RQ_LOGITS_LAST)
        tok = int(c.argmax(1)[0])
        t1 = time.perf_counter()
        toks = [tok]
        for _ in range(a.gen):
            tok = c.decode_argmax(s, tok)
            toks.append(tok)
        t2 = time.perf_counter()
        return t1 - t0, t2 - t1, toks

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    tp, td = [], []
    t_start = time.perf_counter()
    for _ in range(a.steps):
        p, d, toks = step()
        tp.append(p)
        td.append(d)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    ms_per_step = 1e3 * elapsed / a.steps
    value = a.steps * (a.prompt + a.gen) / elapsed
    prefill_tok_s = a.prompt / (sum(tp) / len(tp))
    decode_tok_s = a.gen / (sum(td) / len(td))

    # roofline of the dominant kernel: the decode GEMV, on the model's own weights (8 GB per sweep: no cache reuse)
    c.gemv_sweep(1)
    sw_s, sw_bytes, sw_n = c.gemv_sweep(3)
    achieved = sw_bytes / sw_s / 1e9
    # per-class device time of one profiled decode step (HIP events; classes of rq_ctx_profile)
    c.profile(True)
    s.truncate(a.prompt)
    c.decode_argmax(s, 1)
    prof = {k: round(v[0] * 1e3, 4) for k, v in c.profile_read().items() if v[1]}
    c.profile(False)

    out = {
        "metric": "decode + prefill tok/s (Qwen3-8B-shape Q8_0, 1 GPU); % HBM / int8-MFMA peak",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 x int8 -> int32, fp32 fold (Q8_0 weights, f16 KV)",
        "data": "synthetic: random-init N(0,0.02) weights quantized to Q8_0, seeded random prompt ids",
        "config": {"workload": f"{a.shape} Q8_0: {a.prompt}-token prefill + {a.gen} greedy decode steps per step, f16 KV",
                   "prompt": a.prompt, "gen": a.gen, "global_batch": 1, "seq_len": a.prompt + a.gen},
        "prefill_tok_s": round(prefill_tok_s, 1),
        "decode_tok_s": round(decode_tok_s, 2),
        "decode_ms_per_token": round(1e3 / decode_tok_s, 4),
        "roofline": {"bound": "hbm", "kernel": "k_gemv_q8<1,4> (decode GEMV, one activation row)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "launches_per_step": sw_n, "bytes_per_step": sw_bytes,
                     "avg_launch_us": round(1e6 * sw_s / sw_n, 3),
                     "algorithmic_bytes_per_launch": round(sw_bytes / sw_n)},
        "profile_ms_per_decode_step": prof,
        "tokens_head": toks[:8],
    }
    if not a.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(path, ids, a)
    print(json.dumps(out), flush=True)


def cpu_baseline(path, ids, a):
    """The reference's CPU path on the same file and prompt (oracle/_ref/ref_driver): the prefill + cpu_decode steps,
    all host cores; the step time is estimated as prefill + gen x the measured per-token decode time"""
    from oracle import oracle as orc
    if not os.path.exists(orc.REF_DRIVER):
        return {"value": None, "unit": "tok/s", "cores": 0, "kind": "reference",
                "sample": "oracle/_ref/ref_driver not built (needs the reference tree at build time)"}
    cores = len(os.sched_getaffinity(0))
    t0 = time.time()
    info, _, _, _ = orc.run_ref_driver(path, ids, os.path.join(a.workdir, "cpu"), steps=a.cpu_decode, threads=cores,
                                       cap=(a.prompt + a.cpu_decode + 255) // 256 * 256, timeout=900)
    wall = time.time() - t0
    per_tok = info["decode_s"] / max(1, a.cpu_decode)
    step_s = info["prefill_s"] + a.gen * per_tok
    return {"value": round((a.prompt + a.gen) / step_s, 3), "unit": "tok/s", "cores": cores, "kind": "reference",
            "sample": f"the reference's CPU path (oracle/_ref/ref_driver, -Ofast AVX-512 VNNI, {cores} threads) on the same "
                      f"GGUF: {a.prompt}-token prefill + {a.cpu_decode} greedy decode steps, step time = prefill + "
                      f"{a.gen} x per-token decode ({wall:.0f} s wall incl. load)",
            "prefill_tok_s": round(info["prefill_tok_s"], 2), "decode_tok_s": round(info["decode_tok_s"], 3)}


if __name__ == "__main__":
    main()
