"""Benchmark of the forward hot path on one MI355X: decode + prefill tok/s of a Qwen3-8B-shaped Q8_0 model.

One step = the run shape of the reference's config 1 on the metric's model: reset the sequence, prefill a 512-token
prompt of seeded random ids (rq_prefill, one 512-row pass), then 128 greedy decode steps (gw_decode_greedy: rq_decode
with the argmax on the device, each step's token fed to the next on the device, one wait for the 128). value = (512 + 128) tokens per step / seconds per step, whole job (one GPU), inputs
(weights, prompt ids) resident on the device before the timed region starts.
Weights: random-init, N(0, 0.02) then Q8_0 (a synthetic GGUF written by gwenedeg_amd.synth, seeded); no checkpoint.

Also on the JSON line:
  roofline          the dominant kernel, the decode GEMV (k_gemv1: every weight matmul of a decode step, 145 launches
                    per token at 8B, about three quarters of the decode kernel time): right after the timed region, a
                    replica of the timed step (same prompt, same tokens) in which every kernel records its own start
                    and stop (hipExtLaunchKernel's events on the context's stream: the dispatch's timestamps; they
                    cost host time per launch, so that step is not the timed one); achieved = file-format weight
                    bytes (Q8_0: 34 bytes per 32 weights) per launch / average launch duration, against 8 TB/s. traffic: HBM bytes per launch measured by rocprofv3 FETCH_SIZE +
                    WRITE_SIZE (scaled by a copy kernel of known size), read from profiles/decode_gemv_traffic.json
  roofline_prefill  the prefill GEMM (k_gemm_q8l, the 512-row matmuls) of the same step: 2 ops per weight per row
                    against 5.0 POPS dense int8, with the bound the exact per-32 float fold sets on the VALU (the
                    SwiGLU + quantize after w1 / w3 is its own kernel, in kernel_ms_prefill's swiglu+quant)
  cpu_baseline      the reference's own CPU path (oracle/_ref/ref_driver, -Ofast AVX-512 VNNI) on the same GGUF file,
                    prompt and step (512-token prefill + 128 greedy decode steps), all host threads, best of 3 runs

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--prompt 512] [--gen 128] [--no-cpu-baseline]
       python bench.py --probe [--gen N]   (for rocprofv3 counter runs: warm-up, then one prefill + N decode steps and a
                                            1 GiB negation, the calibration kernel of the traffic figures; no timing)
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
# the prefill GEMM's exact fold (val = val + (ws * xs) * (float) isum per output and group of 32, each op rounded):
# ws * xs from an outer-product MFMA, then 3 VALU lane-ops (convert, multiply, add) per 64 int8 ops; 256 CUs x 64 fp32
# lanes x 2.4 GHz = 39.3 T lane-ops/s
FOLD_BOUND_TOPS = 256 * 64 * 2.4e9 / 3 * 64 / 1e12
GEMV_CLASSES = ("matmul qkv", "matmul wo", "matmul w1+w3", "matmul w2", "classifier")


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
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--probe", action="store_true")
    ap.add_argument("--kv-type", type=int, default=2,
                    help="batch32_4b / long_8b: the sequences' KV cache type (runq.h:214; default 2, RQ_KV_F16); another "
                         "type's line carries no cpu_baseline")
    ap.add_argument("--workload", default="step", choices=["step", "op_q8", "batch32_4b", "long_8b", "cb_8b", "batch32_8b"],
                    help="step: the metric's workload (default); op_q8: the isolated 12288 x 4096 Q8_0 operator of the "
                         "reference's config 2; batch32_4b / long_8b: the batched decode of configs 3 / 4; batch32_8b: "
                         "config 3's 32 sequences x 2048 positions on the 8B-shaped Q8_0 model; cb_8b: config 5's "
                         "continuous-batching steps; each a JSON line of its own")
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
    if a.workload == "cb_8b":
        continuous(torch, gw, synth, a)
        return
    if a.workload == "op_q8":
        op_q8(torch, gw, a)
        return
    if a.workload != "step":
        batched(torch, gw, synth, a)
        return
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

    if a.probe:
        probe(torch, gw, c, s, ids, a)
        return

    def step():
        s.reset()
        t0 = time.perf_counter()
        c.prefill(s, ids, mode=gw.RQ_LOGITS_LAST)
        tok = int(c.argmax(1)[0])
        t1 = time.perf_counter()
        toks = [tok] + [int(t) for t in c.decode_greedy(s, tok, a.gen)]
        t2 = time.perf_counter()
        return t1 - t0, t2 - t1, toks

    c.kernel_timing(True)  # (the event pool is created here, outside the timed region)
    for _ in range(a.warmup):
        step()
    c.kernel_timing(False)
    torch.cuda.synchronize()
    tp, td, step_ms = [], [], []
    t_start = time.perf_counter()
    for i in range(a.steps):
        t0 = time.perf_counter()
        p, d, toks = step()
        step_ms.append(round(1e3 * (time.perf_counter() - t0), 3))
        tp.append(p)
        td.append(d)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    ms_per_step = 1e3 * elapsed / a.steps
    value = a.steps * (a.prompt + a.gen) / elapsed
    prefill_tok_s = a.prompt / (sum(tp) / len(tp))
    decode_tok_s = a.gen / (sum(td) / len(td))
    # a replica of the timed step (same prompt, same tokens) in which every kernel records its own start / stop: the
    # kernels' durations (the events cost host time per launch, so this step itself is not timed)
    c.kernel_timing(True)
    _, _, toks_r = step()
    dec = c.kernel_times(multi=False)  # its decode passes
    pre = c.kernel_times(multi=True)   # its prefill pass
    c.kernel_timing(False)
    assert toks_r == toks, "the replica step chose other tokens"

    # roofline of the dominant kernel (the decode GEMV) and of the prefill GEMM, from those kernel times
    info = m.info
    q, kv = info.n_heads * info.head_dim, info.n_kv_heads * info.head_dim
    layer_w = info.dim * (q + 2 * kv) + q * info.dim + 3 * info.hidden_dim * info.dim
    cls_w = info.vocab_size * info.dim
    tok_bytes = (info.n_layers * layer_w + cls_w) * 34 / 32  # Q8_0 file bytes per decode token
    g_s = sum(dec[k][0] for k in GEMV_CLASSES)
    g_n = sum(dec[k][1] for k in GEMV_CLASSES)
    dec_s = sum(v[0] for v in dec.values())
    achieved = a.gen * tok_bytes / g_s / 1e9
    pre_ops = 2.0 * a.prompt * info.n_layers * layer_w  # the 512-row matmuls (the classifier takes one row)
    m_s = sum(pre[k][0] for k in GEMV_CLASSES[:4])
    m_n = sum(pre[k][1] for k in GEMV_CLASSES[:4])
    tops = pre_ops / m_s / 1e12
    sampling = sampling_cost(c)
    sw_s, sw_bytes, sw_n = c.gemv_sweep(2)

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
        "step_ms": step_ms,
        "roofline": {"bound": "hbm", "kernel": "k_gemv1 (decode GEMV: qkv, wo, w1+w3, w2, classifier)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_per_launch(),
                     "launches": g_n, "avg_launch_us": round(1e6 * g_s / g_n, 3),
                     "algorithmic_bytes_per_launch": round(a.gen * tok_bytes / g_n),
                     "bytes_per_token": tok_bytes, "share_of_decode_kernel_time": round(g_s / dec_s, 4),
                     "measured": "each kernel's own start / stop (hipExtLaunchKernel events on the context's stream) "
                                 f"over the {a.gen} decode passes of a replica of the timed step, run after it",
                     "sweep_gbs": round(sw_bytes / sw_s / 1e9, 1)},
        "roofline_prefill": {"bound": "mfma", "kernel": "k_gemm_q8 (prefill GEMM, 512 rows)",
                             "achieved": round(tops, 1), "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
                             "frac": round(tops / INT8_PEAK_TOPS, 4), "launches": m_n,
                             "avg_launch_us": round(1e6 * m_s / m_n, 3),
                             "algorithmic_ops_per_launch": round(pre_ops / m_n),
                             "fold_bound_tops": round(FOLD_BOUND_TOPS, 1),
                             "frac_of_fold_bound": round(tops / FOLD_BOUND_TOPS, 4),
                             "note": "the four matmuls' launches (qkv, wo, w1 / w3, w2); the SwiGLU and its "
                                     "quantization after w1 / w3 run in their own kernel (swiglu+quant)"},
        "kernel_us_per_decode_token": {k: round(v[0] * 1e6 / a.gen, 2) for k, v in dec.items() if v[1]},
        "kernel_ms_prefill": {k: round(v[0] * 1e3, 3) for k, v in pre.items() if v[1]},
        "tokens_head": toks[:8],
        "sampling_topk40": sampling,
    }
    if not a.no_cpu_baseline:
        cb = cpu_baseline(path, ids, a)
        ref_toks = cb.pop("tokens", None)
        if ref_toks is not None:  # greedy identity on the metric's own workload: the tokens fed at each decode step
            cb["greedy_tokens_identical"] = ref_toks == toks[:len(ref_toks)]
        out["cpu_baseline"] = cb
    print(json.dumps(out), flush=True)


BATCHED = {  # the reference's configs 3 and 4 (and config 3's batch on the 8B shape): shape, sequences, cached positions per sequence, timed decode steps,
    # timed steps of the CPU baseline
    "batch32_4b": ("qwen3_4b_q4km", 32, 2048, 16, 48),
    "long_8b": ("qwen3_8b", 8, 32768, 8, 12),
    "batch32_8b": ("qwen3_8b", 32, 2048, 16, 16),  # (config 3's batch on the 8B-shaped Q8_0 model: Q8_0 at 32 rows)
}


def batched(torch, gw, synth, a):
    """Batched greedy decode: nseq sequences with `ctx` cached positions each (rq_seq_fill_synthetic: the K / V of a
    prefix, whose cost does not depend on the values, runq.h:721-726), then decode passes of one row per sequence
    (gw_forward_batch_device + gw_ctx_argmax: rq_forward_batch with the greedy choice on the device). value = rows per
    second; the HBM bytes of a step = the weights' file bytes + the K / V bytes the attention reads"""
    shape, nseq, ctx, steps, cpu_steps = BATCHED[a.workload]
    steps = a.steps if a.steps != 3 else steps
    os.makedirs(a.workdir, exist_ok=True)
    path = os.path.join(a.workdir, f"{shape}_seed{a.seed}.gguf")
    if not os.path.exists(path):
        synth.write_gguf(path, shape, seed=a.seed)
    cap = ctx + steps + a.warmup + 16
    m = gw.Model(path, ctx_len=cap)
    c = m.ctx(max_batch=max(nseq, 2), max_ctx=cap)
    seqs = [m.seq(cap, kv_type=a.kv_type) for _ in range(nseq)]
    for i, sq in enumerate(seqs):
        sq.fill_synthetic(ctx, seed=a.seed + i)
    toks = [int(t) for t in np.random.default_rng(a.seed).integers(0, m.vocab, nseq)]

    def one():
        nonlocal toks
        toks = [int(t) for t in c.forward_batch_argmax([gw.Segment(sq, [t], gw.RQ_LOGITS_LAST) for sq, t in zip(seqs, toks)])]

    for _ in range(a.warmup):
        one()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        one()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    c.kernel_timing(True)
    one()
    kt = c.kernel_times(multi=True)
    c.kernel_timing(False)
    info = m.info
    # K and V bytes per position (the tiles' bytes per dim: f32 4, 16-bit 2, q8 17 / 16, q4 9 / 16; a dot-product type
    # its base type's)
    base = a.kv_type & ~4 if a.kv_type in (5, 6, 7, 12, 13) else a.kv_type
    kb, vb = {0: (4, 4), 1: (2, 2), 2: (2, 2), 3: (17 / 16, 17 / 16), 8: (17 / 16, 9 / 16), 9: (9 / 16, 9 / 16)}[base]
    kv_pos = info.n_layers * info.n_kv_heads * info.head_dim * (kb + vb)
    mean_ctx = ctx + a.warmup + steps + 0.5
    kv_bytes = nseq * mean_ctx * kv_pos
    w_bytes = weight_file_bytes(path)
    step_s = el / steps
    att_s = kt.get("attention", (0, 0))[0]
    out = {
        "metric": f"batched greedy decode rows/s ({a.workload}: " + {"batch32_4b": "the reference's config 3",
                                                                       "long_8b": "the reference's config 4",
                                                                       "batch32_8b": "config 3's batch on the 8B shape"}[a.workload] + ", 1 GPU)",
        "value": round(nseq * steps / el, 2), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": a.warmup,
        "ms_per_step": round(1e3 * step_s, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": f"int8 x int8 -> int32, fp32 fold; KV type {a.kv_type}" + (" (f16)" if a.kv_type == 2 else ""),
        "data": "synthetic weights; K / V of the prefixes by rq_seq_fill_synthetic",
        "config": {"workload": f"{shape}: {nseq} sequences x {ctx} cached positions, one row per sequence per step",
                   "global_batch": nseq, "seq_len": ctx},
        "hbm_bytes_per_step": {"weights": w_bytes, "kv_read": kv_bytes},
        "achieved_gbs": round((w_bytes + kv_bytes) / step_s / 1e9, 1),
        "attention": {"kernel_ms_per_step": round(att_s * 1e3, 3),
                      "kv_gbs": round(kv_bytes / att_s / 1e9, 1) if att_s else None},
        "kernel_ms_per_step": {k: round(v[0] * 1e3, 3) for k, v in kt.items() if v[1]},
    }
    if not a.no_cpu_baseline and a.kv_type == 2:
        # the same shape on the reference: nseq sequences filled to ctx positions, one untimed pass, then cpu_steps
        # timed greedy passes of one row per sequence
        t0 = [int(t) for t in np.random.default_rng(a.seed).integers(0, m.vocab, nseq)]
        ln = [f"seqs {nseq} {ctx + cpu_steps + 16}"] + [f"fill {i} {ctx} {a.seed + i}" for i in range(nseq)]
        for r in range(cpu_steps + 1):
            ln.append(f"pass {nseq}")
            ln += [f"seg {i} {gw.RQ_LOGITS_LAST} 1 {t0[i] if r == 0 else -1}" for i in range(nseq)]
        out["cpu_baseline"] = plan_baseline(path, "\n".join(ln) + "\n", a, ctx + cpu_steps + 16,
                                            [[k] for k in range(1, cpu_steps + 1)], nseq,
                                            f"{nseq} sequences x {ctx} cached positions (rq_seq_fill_synthetic), one untimed "
                                            f"pass, then {cpu_steps} greedy passes of {nseq} one-row segments")
    print(json.dumps(out), flush=True)


def continuous(torch, gw, synth, a):
    """Config 5: continuous batching on the 8B-shaped Q8_0 model. A step is what the reference's engine runs for 48
    decoding sequences and 2 prompt chunks of 512 tokens (engine.c:3027-3255: decode rows first, then prompt chunks
    within the budget): 1,072 rows in passes of at most RQ_BATCH_MAX = 512 rows (rq_forward_batch with the greedy
    choice on the device): [48 decode rows + 464 prompt rows], [48 + 464], [48]. The decoding sequences start at
    contexts uniform in [256, 8192] (rq_seq_fill_synthetic); prompts are 2,048 tokens, two prompt slots each taking a
    512-token chunk per step, and a finished prompt starts a new request: one in four begins with the 1,024-token shared
    prefix copied from the cache (rq_seq_copy) and prefills the rest. value = rows per second; per-step latency"""
    shape, ndec, chunk, prompt, prefix = "qwen3_8b", 48, 512, 2048, 1024
    steps = a.steps if a.steps != 3 else 40
    rng = np.random.default_rng(a.seed)
    os.makedirs(a.workdir, exist_ok=True)
    path = os.path.join(a.workdir, f"{shape}_seed{a.seed}.gguf")
    if not os.path.exists(path):
        synth.write_gguf(path, shape, seed=a.seed)
    ctxs = rng.integers(256, 8193, ndec)
    cap = 8192 + steps + a.warmup + 16
    m = gw.Model(path, ctx_len=max(cap, prompt + 16))
    c = m.ctx(max_batch=512, max_ctx=max(cap, prompt + 16))
    dec = [m.seq(cap) for _ in range(ndec)]
    for i, sq in enumerate(dec):
        sq.fill_synthetic(int(ctxs[i]), seed=a.seed + i)
    shared = m.seq(prompt + 16)
    shared.fill_synthetic(prefix, seed=a.seed + 999)
    slots = [m.seq(prompt + 16) for _ in range(2)]
    toks = [int(t) for t in rng.integers(0, m.vocab, ndec)]
    nreq, nshared = [0], [0]

    def start(sq):
        # a new request in a prompt slot: one in four starts from the shared prefix
        nreq[0] += 1
        if nreq[0] % 4 == 0:
            sq.copy_from(shared, prefix)
            nshared[0] += 1
        else:
            sq.reset()

    for sq in slots:
        start(sq)

    def one_step():
        nonlocal toks
        # this step's prompt rows: 512 from each slot (a prompt ending here: its last row's logits)
        rows = []
        for sq in slots:
            n0 = len(sq)
            ids = [int(t) for t in rng.integers(0, m.vocab, chunk)]
            rows.append((sq, ids, n0 + chunk >= prompt))
        dsegs = [gw.Segment(sq, [t], gw.RQ_LOGITS_LAST) for sq, t in zip(dec, toks)]
        budget, passes, cur = 512, [], list(dsegs)
        used = len(cur)
        for sq, ids, last in rows:
            o = 0
            while o < len(ids):
                take = min(budget - used, len(ids) - o)
                end = o + take == len(ids)
                cur.append(gw.Segment(sq, ids[o:o + take], gw.RQ_LOGITS_LAST if (end and last) else gw.RQ_LOGITS_NONE))
                used += take
                o += take
                if used == budget:
                    passes.append(cur)
                    cur, used = [], 0
        if cur:
            passes.append(cur)
        for i, segs in enumerate(passes):
            out = c.forward_batch_argmax(segs)
            if i == 0:
                toks = [int(t) for t in out[:ndec]]
        for sq, _, last in rows:
            if last:
                start(sq)

    for _ in range(a.warmup):
        one_step()
    lat = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        t1 = time.perf_counter()
        one_step()
        lat.append(time.perf_counter() - t1)
    el = time.perf_counter() - t0
    lat = np.sort(np.array(lat))
    rows_per_step = ndec + 2 * chunk
    out = {
        "metric": "continuous-batching tok/s and per-step latency (cb_8b: the reference's config 5, 1 GPU)",
        "value": round(rows_per_step * steps / el, 1), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": a.warmup,
        "ms_per_step": round(1e3 * el / steps, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 x int8 -> int32, fp32 fold; f16 KV", "data": "synthetic weights, random prompt ids; the decoding "
                "sequences' K / V by rq_seq_fill_synthetic",
        "config": {"workload": f"{shape}: per step {ndec} decode rows at contexts U[256, 8192] + 2 x {chunk} prompt rows "
                               f"(prompts of {prompt}, 1 in 4 from a {prefix}-token shared prefix), passes of <= 512 rows",
                   "global_batch": rows_per_step, "seq_len": 8192},
        "step_latency_ms": {"p50": round(1e3 * float(lat[len(lat) // 2]), 3), "p90": round(1e3 * float(lat[int(0.9 * (len(lat) - 1))]), 3),
                            "max": round(1e3 * float(lat[-1]), 3)},
        "decode_tok_s": round(ndec * steps / el, 1), "prompt_tok_s": round(2 * chunk * steps / el, 1),
        "requests_started": nreq[0], "requests_from_shared_prefix": nshared[0],
    }
    if not a.no_cpu_baseline:
        out["cpu_baseline"] = cb_cpu_baseline(path, a, ctxs, ndec, chunk, prompt, prefix, m.vocab)
    print(json.dumps(out), flush=True)


def cb_cpu_baseline(path, a, ctxs, ndec, chunk, prompt, prefix, vocab):
    """Config 5 on the reference: three steps of the device's shape (48 decode rows at the same contexts + two 512-token
    prompt chunks, passes of <= 512 rows); slot A continues a request started from the 1,024-token shared prefix
    (rq_seq_copy), slot B a fresh one; when A's prompt ends (step 2) a fresh request takes its slot. Steps 2 and 3 are
    timed (step 1 warms the host's caches and pages)"""
    import gwenedeg_amd as gw
    rng = np.random.default_rng(a.seed + 5)
    S, A, B, C = ndec, ndec + 1, ndec + 2, ndec + 3  # shared prefix, the three prompt requests
    ln = [f"seqs {ndec + 4} {8192 + 32}"] + [f"fill {i} {int(ctxs[i])} {a.seed + i}" for i in range(ndec)]
    ln += [f"fill {S} {prefix} {a.seed + 999}", f"copy {A} {S} {prefix}"]
    pos = {A: prefix, B: 0, C: 0}
    slots, npass, groups = [A, B], 0, []
    for step in range(3):
        segs = [(i, gw.RQ_LOGITS_LAST, "1 " + (str(int(rng.integers(0, vocab))) if step == 0 else "-1")) for i in range(ndec)]
        used, passes, cur = ndec, [], segs
        for k, sq in enumerate(slots):
            ids = [int(t) for t in rng.integers(0, vocab, chunk)]
            last = pos[sq] + chunk >= prompt
            o = 0
            while o < chunk:
                take = min(512 - used, chunk - o)
                mode = gw.RQ_LOGITS_LAST if (o + take == chunk and last) else gw.RQ_LOGITS_NONE
                cur.append((sq, mode, f"{take} " + " ".join(map(str, ids[o:o + take]))))
                used += take
                o += take
                if used == 512:
                    passes.append(cur)
                    cur, used = [], 0
            pos[sq] += chunk
            if last:
                slots[k] = C
        if cur:
            passes.append(cur)
        for segs_ in passes:
            ln.append(f"pass {len(segs_)}")
            ln += [f"seg {i} {mode} {rest}" for i, mode, rest in segs_]
        groups.append(list(range(npass, npass + len(passes))))
        npass += len(passes)
    return plan_baseline(path, "\n".join(ln) + "\n", a, 8192 + 32, groups[1:], ndec + 2 * chunk,
                         f"config 5's step three times ({ndec} decode rows at the device's contexts + 2 x {chunk} prompt "
                         f"rows, passes of <= 512 rows), steps 2 and 3 timed", timeout=1800)



def weight_file_bytes(path):
    """the file bytes of the GGUF's matrices (everything but the header and the f32 norms: the tensors data section)"""
    return float(os.path.getsize(path))


def traffic_per_launch():
    """HBM bytes per decode-GEMV launch from the committed counter summary (rocprofv3 FETCH_SIZE + WRITE_SIZE, each
    scaled by what the counter reads for a copy of known size), or None where it is absent"""
    f = os.path.join(ROOT, "profiles", "decode_gemv_traffic.json")
    try:
        with open(f) as fh:
            return json.load(fh)["traffic_bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        return None


def probe(torch, gw, c, s, ids, a):
    """the workload of the counter runs: one warm-up pass, then one prefill and a.gen decode steps as the timed step
    runs them, then the calibration kernel (a 1 GiB float32 negation: read once, written once)"""
    c.prefill(s, ids[:16], mode=gw.RQ_LOGITS_LAST)
    s.reset()
    c.prefill(s, ids, mode=gw.RQ_LOGITS_LAST)
    c.decode_greedy(s, int(c.argmax(1)[0]), a.gen)
    src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.neg(src, out=dst)  # one elementwise kernel: 1 GiB read, 1 GiB written
    torch.cuda.synchronize()
    log(f"probe done: prefill {len(ids)} + {a.gen} decode steps, copy of {src.numel() * 4} bytes")


def sampling_cost(c, k=40, reps=1000, warm=500, temperature=0.7, topp=0.9):
    """Host wall time per token of top-k sampling on the last decode pass's logits row, after the timed region: the
    device top-k (gw_ctx_topk: two kernels writing k (value, id) pairs into pinned host memory, one synchronisation)
    averaged over reps calls after warm calls (the first few hundred calls of a process run slower: cold_us, the
    average of the first 100), and the host draw (gw_sample_topk). Outside the metric; an error is reported, not
    raised."""
    import ctypes
    import gwenedeg_amd as gw
    try:
        t0 = time.perf_counter()
        for i in range(warm):
            c.topk(1, k)
            if i == 99:
                t_cold = (time.perf_counter() - t0) / 100
        t0 = time.perf_counter()
        for _ in range(reps):
            vals, idx = c.topk(1, k)
        t_dev = (time.perf_counter() - t0) / reps
        st = ctypes.c_ulonglong(0x9E3779B97F4A7C15)
        fp, ip = vals.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), idx.ctypes.data_as(ctypes.POINTER(ctypes.c_int))
        t0 = time.perf_counter()
        for _ in range(reps):
            tok = gw.lib.gw_sample_topk(fp, ip, k, temperature, topp, ctypes.byref(st))
        t_draw = (time.perf_counter() - t0) / reps
        return {"device_topk_us": round(t_dev * 1e6, 2), "cold_us": round(t_cold * 1e6, 2),
                "host_draw_us": round(t_draw * 1e6, 2), "k": k,
                "temperature": temperature, "top_p": topp, "last_token": int(tok)}
    except Exception as e:  # noqa: BLE001 - a side figure must not cost the bench line
        return {"error": str(e)}


def host_cpu():
    """The host the CPU baseline runs on: CPU model, the physical cores of this process's CPU set (distinct (package,
    core) pairs: the reference's threads, one per core, as its own benchmarks run it), logical CPUs, 1-minute load"""
    cpus = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in cpus:
        t = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            with open(t + "physical_package_id") as f1, open(t + "core_id") as f2:
                cores.add((f1.read().strip(), f2.read().strip()))
        except OSError:
            cores.add(("?", str(c)))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "physical_cores": len(cores), "logical_cpus": len(cpus),
            "load_1min": round(os.getloadavg()[0], 2)}


def _stats(xs):
    xs = sorted(xs)
    n = len(xs)
    return xs[0], (xs[n // 2] if n % 2 else 0.5 * (xs[n // 2 - 1] + xs[n // 2]))


def cpu_baseline(path, ids, a):
    """The reference's CPU path on the same file, prompt and step (oracle/_ref/ref_driver): the 512-token prefill and
    the gen greedy decode steps, one thread per physical core, best and median of cpu_reps runs (about 10 s of CPU
    work at 8B)"""
    from oracle import oracle as orc
    if not os.path.exists(orc.REF_DRIVER):
        return {"value": None, "unit": "tok/s", "cores": 0, "kind": "reference",
                "sample": "oracle/_ref/ref_driver not built (needs the reference tree at build time)"}
    host = host_cpu()
    cores = host["physical_cores"]
    log(f"cpu baseline: the reference's step on {cores} threads ...")
    t0 = time.time()
    info, _, toks, _ = orc.run_ref_driver(path, ids, os.path.join(a.workdir, "cpu"), steps=a.gen, threads=cores,
                                          cap=(a.prompt + a.gen + 255) // 256 * 256, reps=a.cpu_reps, timeout=900)
    wall = time.time() - t0
    best, med = _stats(info["run_s"])
    n = a.prompt + a.gen
    return {"value": round(n / best, 3), "unit": "tok/s", "cores": info["threads"], "kind": "reference",
            "sample": f"the reference's CPU path (oracle/_ref/ref_driver, -Ofast AVX-512 VNNI, {info['threads']} threads, one per "
                      f"physical core) on the same GGUF and prompt: the whole step ({a.prompt}-token prefill + {a.gen} greedy "
                      f"decode steps), best of {a.cpu_reps} runs ({wall:.0f} s wall incl. load)",
            "median": round(n / med, 3), **host,
            "prefill_tok_s": round(info["prefill_tok_s"], 2), "decode_tok_s": round(info["decode_tok_s"], 3),
            "tokens": [int(t) for t in toks]}


def plan_baseline(path, plan, a, cap, timed, rows, what, timeout=1500):
    """The reference's CPU path on a script of passes (ref_driver --plan: synthetic caches by rq_seq_fill_synthetic,
    rq_forward_batch passes with greedy feeds), one thread per physical core: `timed` lists the groups of passes
    (indices into the run's passes) that each make one timed step of `rows` rows; value = rows / best step time"""
    from oracle import oracle as orc
    if not os.path.exists(orc.REF_DRIVER):
        return {"value": None, "unit": "tok/s", "cores": 0, "kind": "reference",
                "sample": "oracle/_ref/ref_driver not built (needs the reference tree at build time)"}
    host = host_cpu()
    log(f"cpu baseline: the reference on {what} ...")
    t0 = time.time()
    info, _, _ = orc.run_ref_plan(path, plan, os.path.join(a.workdir, "cpu_plan"), threads=host["physical_cores"], cap=cap,
                                  timeout=timeout)
    wall = time.time() - t0
    steps = [sum(info["pass_s"][k] for k in g) for g in timed]
    best, med = _stats(steps)
    return {"value": round(rows / best, 3), "unit": "tok/s", "cores": info["threads"], "kind": "reference",
            "sample": f"the reference's CPU path (oracle/_ref/ref_driver --plan, {info['threads']} threads, one per physical "
                      f"core) on the same GGUF: {what}; best of {len(steps)} timed steps ({wall:.0f} s wall incl. load and "
                      "cache fill)", "median": round(rows / med, 3), "step_ms": [round(1e3 * x, 1) for x in steps], **host}


OP_N, OP_K, OP_COPIES = 12288, 4096, 8


def op_q8(torch, gw, a):
    """Config 2: the isolated Q8_0 operator, W = 12288 x 4096 (int8 codes uniform in [-127, 127], fp16 scales
    |N(0, 1e-3)|), X = M rows of N(0, 1) quantized per 32 on the device (gw_quantize), out = M x 12288 fp32, at M = 1
    (the decode GEMV, k_gemv1), 8 (k_gemv_mr), 64 and 512 (k_gemm_q8). OP_COPIES copies of W in device memory (428 MB,
    more than the 256 MB memory-side cache) and each launch takes the next copy, as a model's matrices follow one
    another. gw_q8_matmul on torch's current stream, timed with its events over reps launches after a warm-up.
    Beside each M: the reference's q8p_gemv_rows / q8p_gemm_item on the same int8 inputs (oracle/_ref/ref_q8op), one
    thread per physical core, OP_COPIES rotated packed copies, best and median; its output must equal the device's bit
    for bit. value = the M = 1 GEMV's HBM GB/s (file bytes: 34 per 32 weights)"""
    N, K = OP_N, OP_K
    rng = np.random.default_rng(a.seed)
    wq = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    ws16 = np.abs(rng.normal(0, 1e-3, size=(N, K // 32))).astype(np.float16)
    W0, WS0 = torch.from_numpy(wq).cuda(), torch.from_numpy(ws16.view(np.int16)).cuda()
    Ws = [W0] + [W0.clone() for _ in range(OP_COPIES - 1)]
    WSs = [WS0] + [WS0.clone() for _ in range(OP_COPIES - 1)]
    st = torch.cuda.current_stream()
    sp = st.cuda_stream
    w_bytes = N * K * 34 / 32
    host = host_cpu() if not a.no_cpu_baseline else None
    have_ref = False
    if not a.no_cpu_baseline:
        from oracle import oracle as orc
        have_ref = os.path.exists(orc.REF_Q8OP)
    per_m = []
    for M in (1, 8, 64, 512):
        x = torch.from_numpy(rng.normal(0, 1, size=(M, K)).astype(np.float32)).cuda()
        xq = torch.empty((M, K), dtype=torch.int8, device="cuda")
        xs = torch.empty((M, K // 32), dtype=torch.float32, device="cuda")
        assert gw.lib.gw_quantize(x.data_ptr(), M, K, xq.data_ptr(), xs.data_ptr(), sp) == 0
        out = torch.empty((M, N), dtype=torch.float32, device="cuda")

        def launch(r):
            e = gw.lib.gw_q8_matmul(out.data_ptr(), Ws[r % OP_COPIES].data_ptr(), WSs[r % OP_COPIES].data_ptr(), N, K,
                                    xq.data_ptr(), xs.data_ptr(), M, sp)
            assert e == 0, f"gw_q8_matmul: {e}"

        reps = 256 if M <= 8 else 128 if M <= 64 else 64
        for r in range(2 * OP_COPIES):
            launch(r)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for r in range(reps):
            launch(r)
        e1.record(st)
        torch.cuda.synchronize()
        us = 1e3 * e0.elapsed_time(e1) / reps
        ops = 2.0 * M * N * K
        row = {"M": M, "us_per_op": round(us, 3), "hbm_gbs": round(w_bytes / us / 1e3, 1),
               "hbm_frac": round(w_bytes / us / 1e3 / HBM_PEAK_GBS, 4), "tops": round(ops / us / 1e6, 2),
               "mfma_frac": round(ops / us / 1e6 / INT8_PEAK_TOPS, 4), "reps": reps}
        if have_ref:
            launch(0)  # (copy 0: the inputs written below)
            torch.cuda.synchronize()
            got = out.cpu().numpy()
            wd = os.path.join(a.workdir, "op_q8")
            ref, t = orc.run_ref_q8op(wd, wq, ws16.astype(np.float32), xq.cpu().numpy(), xs.cpu().numpy(),
                                      reps=max(8, min(200, int(2e4 / (M + 8)))), threads=host["physical_cores"],
                                      copies=OP_COPIES)
            row["bit_exact_vs_reference"] = bool(np.array_equal(got.view(np.uint32), ref.view(np.uint32)))
            row["cpu"] = {"best_us": round(1e6 * t["best_s"], 1), "median_us": round(1e6 * t["median_s"], 1),
                          "threads": t["threads"], "reps": t["reps"], "copies": t["copies"],
                          "hbm_gbs_equiv": round(w_bytes / t["best_s"] / 1e9, 1), "tops": round(ops / t["best_s"] / 1e12, 3)}
            row["speedup_vs_cpu_best"] = round(1e6 * t["best_s"] / us, 1)
        per_m.append(row)
        log(f"op_q8 M={M}: {row}")
    m1, m512 = per_m[0], per_m[-1]
    out = {
        "metric": "isolated Q8_0 matmul 12288 x 4096 (the reference's config 2, 1 GPU): M = 1 GEMV HBM GB/s",
        "value": m1["hbm_gbs"], "unit": "GB/s", "n_gpus": 1, "steps": m1["reps"], "warmup": 2 * OP_COPIES,
        "ms_per_step": round(m1["us_per_op"] / 1e3, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 x int8 -> int32, fp32 fold (Q8_0)",
        "data": "synthetic: int8 codes uniform in [-127, 127], fp16 scales |N(0, 1e-3)|, X ~ N(0, 1) quantized per 32",
        "config": {"workload": f"Q8_0 W {N} x {K} ({OP_COPIES} rotated copies), M = 1, 8, 64, 512", "global_batch": 1,
                   "seq_len": 1},
        "roofline": {"bound": "hbm", "kernel": "k_gemv1 (M = 1)", "achieved": m1["hbm_gbs"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": m1["hbm_frac"], "traffic": None,
                     "algorithmic_bytes_per_launch": w_bytes},
        "roofline_gemm": {"bound": "mfma", "kernel": "k_gemm_q8 (M = 512)", "achieved": m512["tops"], "peak": INT8_PEAK_TOPS,
                          "unit": "TOP/s", "frac": m512["mfma_frac"], "fold_bound_tops": round(FOLD_BOUND_TOPS, 1)},
        "per_m": per_m,
    }
    if have_ref:
        out["cpu_baseline"] = {"value": m1["cpu"]["hbm_gbs_equiv"], "unit": "GB/s", "cores": m1["cpu"]["threads"],
                               "kind": "reference",
                               "sample": f"the reference's q8p_gemv_rows (M = 1) / q8p_gemm_item (oracle/_ref/ref_q8op) on the "
                                         f"same int8 inputs, {m1['cpu']['threads']} threads, {OP_COPIES} rotated packed copies "
                                         "of W; per M in per_m[].cpu", **host}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
