"""The BASELINE configurations 3, 4 and 5 at their workload shapes (reduced depth only) against the reference's own
CPU path: the device fills the sequences' caches (rq_seq_fill_synthetic), saves them (rq_seq_save: the reference's
file format), and the reference loads the same files (ref_driver --plan: rq_seq_load, rq_seq_copy, rq_forward_batch
passes with greedy feeds). The same passes then run on both sides, and every selected logits row must be equal bit for
bit, with the same greedy tokens:
  config 3: Qwen3-4B-shaped Q4_K_M, 32 sequences at ~2,048 cached positions, 8 batched passes of 32 one-row
            segments (the 9..32-row K-quant GEMM, k_gemm_kq32, inside a model pass);
  config 4: Qwen3-8B-shaped Q8_0, 8 sequences at ~32,768 cached positions, 4 batched passes of 8 one-row segments
            (128 key blocks per row: the batched attention and the combine kernel at their real size);
  config 5: Qwen3-8B-shaped Q8_0, the continuous-batching step of engine.c:3027-3255 twice: 48 decode rows at
            contexts U[256, 8192] and two 512-token prompt chunks (one continuing a 1,024-token prefix copied from the
            cache) in passes of <= 512 rows, [48 + 464], [48 + 464], [48]; every row also against its sequence run
            alone."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LAST, ALL, NONE = 1, 2, 0


@pytest.fixture(scope="module")
def gw():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import gwenedeg_amd
    return gwenedeg_amd


@pytest.fixture(scope="module")
def orc():
    from oracle import oracle
    if not oracle.have_ref():
        pytest.skip("oracle/_ref (the reference's CPU path) is not built")
    return oracle


@pytest.fixture(scope="module")
def model_8b_1l(tmp_path_factory):
    """the Qwen3-8B shape, one layer, the full vocabulary (untied classifier)"""
    from gwenedeg_amd import synth
    d = dict(synth.SHAPES["qwen3_8b"], n_layers=1)
    path = str(tmp_path_factory.mktemp("w8b") / "qwen3_8b_1l.gguf")
    synth.write_gguf(path, d, seed=31)
    return path


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _threads():
    return min(16, len(os.sched_getaffinity(0)))


class Plan:
    """the same passes on the device and, as ref_driver --plan text, on the reference"""

    def __init__(self, c, seqs, cap):
        self.c, self.seqs = c, seqs
        self.lines = [f"seqs {len(seqs)} {cap}"]
        self.last = {}  # sequence index -> its last selected logits row (for a greedy feed)
        self.rows, self.fed = [], []

    def load(self, i, path):
        self.lines.append(f"load {i} {path}")

    def copy(self, i, j, n):
        self.seqs[i].copy_from(self.seqs[j], n)
        self.lines.append(f"copy {i} {j} {n}")

    def run(self, segs):
        """segs: (sequence index, RQ_LOGITS_* mode, token list, or None for the greedy feed of one token)"""
        import gwenedeg_amd as gw
        self.lines.append(f"pass {len(segs)}")
        dev = []
        for i, mode, toks in segs:
            if toks is None:
                t = int(np.argmax(self.last[i]))
                self.fed.append(t)
                toks, txt = [t], "-1"
            else:
                txt = " ".join(str(int(t)) for t in toks)
            self.lines.append(f"seg {i} {mode} {len(toks)} {txt}")
            dev.append(gw.Segment(self.seqs[i], [int(t) for t in toks], mode))
        lg, _ = self.c.forward_batch(dev)
        r = 0
        for i, mode, toks in segs:
            n = 1 if toks is None else len(toks)
            sel = n if mode == ALL else 1 if mode == LAST else 0
            if sel:
                self.last[i] = lg[r + sel - 1]
            r += sel
        if lg is not None:
            self.rows.append(lg)
        return lg

    def text(self):
        return "\n".join(self.lines) + "\n"

    def check(self, orc, path, workdir, cap, kv_type=2):
        info, rlg, rtok = orc.run_ref_plan(path, self.text(), workdir, threads=_threads(), cap=cap, kv_type=kv_type)
        ours = np.concatenate(self.rows)
        assert rlg.shape == ours.shape, (rlg.shape, ours.shape)
        assert [int(t) for t in rtok] == self.fed, "greedy tokens"
        bad = np.nonzero(~np.all(_bits(ours) == _bits(rlg), axis=1))[0]
        assert bad.size == 0, f"{bad.size} rows differ, first {bad[0]}: max diff {np.abs(ours[bad[0]] - rlg[bad[0]]).max()}"
        return info


def _save_all(seqs, lens, tmp, tag, seed0):
    files = []
    for i, (sq, n) in enumerate(zip(seqs, lens)):
        sq.fill_synthetic(int(n), seed=seed0 + i)
        f = os.path.join(tmp, f"{tag}{i}.seq")
        sq.save(f)
        files.append(f)
    return files


def _rm(files):
    for f in files:
        try:
            os.remove(f)
        except OSError:
            pass


def test_config4_batch8_at_32k_vs_reference(gw, orc, tmp_path, model_8b_1l):
    """config 4: 8 sequences at 32,768 - 5 i cached positions (each its own K / V), 4 batched greedy passes of 8
    one-row segments: every logits row bit for bit against the reference's rq_forward_batch on the same caches"""
    m = gw.Model(model_8b_1l, ctx_len=32832)
    if gw.exact_mode() & 3 != 3:
        pytest.skip("this host does not provide the reference's float operations (AVX-512)")
    cap, ns = 32832, 8
    seqs = [m.seq(cap) for _ in range(ns)]
    files = _save_all(seqs, [32768 - 5 * i for i in range(ns)], str(tmp_path), "c4_", 500)
    try:
        c = m.ctx(max_batch=512, max_ctx=cap)
        p = Plan(c, seqs, cap)
        for i, f in enumerate(files):
            p.load(i, f)
        toks = [int(t) for t in np.random.default_rng(4).integers(0, m.vocab, ns)]
        p.run([(i, LAST, [toks[i]]) for i in range(ns)])
        for _ in range(3):
            p.run([(i, LAST, None) for i in range(ns)])
        p.check(orc, model_8b_1l, str(tmp_path / "ref"), cap)
        assert len(p.fed) == 3 * ns
    finally:
        _rm(files)


@pytest.mark.parametrize("kvt", [3, 9, 5, 7, 0])  # RQ_KV_Q8, RQ_KV_Q4K4, RQ_KV_BF16_DOT, RQ_KV_Q8_DOT, RQ_KV_F32
def test_long_context_kv_types_vs_reference(gw, orc, tmp_path, model_8b_1l, kvt):
    """config 4's pass on the f32, quantized and dot-product caches (k_attn_q over 32 key blocks): 4 sequences at
    8,192 - 7 i cached positions of the type (rq_seq_fill_synthetic stores them as the type stores a row), saved and
    loaded by the reference, then 3 batched greedy passes of 4 one-row segments: every logits row bit for bit"""
    m = gw.Model(model_8b_1l, ctx_len=8256)
    if gw.exact_mode() & 3 != 3:
        pytest.skip("this host does not provide the reference's float operations (AVX-512)")
    cap, ns = 8256, 4
    seqs = [m.seq(cap, kv_type=kvt) for _ in range(ns)]
    files = _save_all(seqs, [8192 - 7 * i for i in range(ns)], str(tmp_path), f"lk{kvt}_", 700)
    try:
        c = m.ctx(max_batch=64, max_ctx=cap)
        p = Plan(c, seqs, cap)
        for i, f in enumerate(files):
            p.load(i, f)
        toks = [int(t) for t in np.random.default_rng(6).integers(0, m.vocab, ns)]
        p.run([(i, LAST, [toks[i]]) for i in range(ns)])
        for _ in range(2):
            p.run([(i, LAST, None) for i in range(ns)])
        p.check(orc, model_8b_1l, str(tmp_path / "ref"), cap, kv_type=kvt)
    finally:
        _rm(files)


def test_config3_batch32_q4km_vs_reference(gw, orc, tmp_path):
    """config 3: the Qwen3-4B-shaped Q4_K_M model (2 layers), 32 sequences at 2,048 - 3 i cached positions, 8 batched
    greedy passes of 32 one-row segments (k_gemm_kq32 on every matrix of the pass): bit for bit against the
    reference"""
    from gwenedeg_amd import synth
    d = dict(synth.SHAPES["qwen3_4b_q4km"], n_layers=2)
    path = str(tmp_path / "q4km.gguf")
    synth.write_gguf(path, d, seed=33)
    m = gw.Model(path, ctx_len=2112)
    if gw.exact_mode() & 3 != 3:
        pytest.skip("this host does not provide the reference's float operations (AVX-512)")
    cap, ns = 2112, 32
    seqs = [m.seq(cap) for _ in range(ns)]
    files = _save_all(seqs, [2048 - 3 * i for i in range(ns)], str(tmp_path), "c3_", 700)
    try:
        c = m.ctx(max_batch=512, max_ctx=cap)
        p = Plan(c, seqs, cap)
        for i, f in enumerate(files):
            p.load(i, f)
        toks = [int(t) for t in np.random.default_rng(3).integers(0, m.vocab, ns)]
        p.run([(i, LAST, [toks[i]]) for i in range(ns)])
        for _ in range(7):
            p.run([(i, LAST, None) for i in range(ns)])
        p.check(orc, path, str(tmp_path / "ref"), cap)
    finally:
        _rm(files)


def test_config5_continuous_batching_passes_vs_reference(gw, orc, tmp_path, model_8b_1l):
    """config 5: two continuous-batching steps (engine.c:3027-3255) on the 8B shape with the full vocabulary: 48 decode
    rows at contexts U[256, 8192], prompt slot A continuing a 1,024-token prefix copied from the cache (rq_seq_copy)
    and fresh slot B, 512 prompt tokens each per step, in passes of <= 512 rows ([48 decode + 464 of A], [48 of A + 464
    of B], [48 of B]); each prompt segment's last row and every decode row selected. Every row bit for bit against the
    reference's passes, and against the same sequence run alone on the device (same chunks, no batch-mates)"""
    m = gw.Model(model_8b_1l, ctx_len=8208)
    if gw.exact_mode() & 3 != 3:
        pytest.skip("this host does not provide the reference's float operations (AVX-512)")
    cap, nd = 8208, 48
    rng = np.random.default_rng(5)
    lens = [int(x) for x in rng.integers(256, 8193, nd)]
    # sequences: 0..47 decoding, 48 the shared prefix, 49 slot A, 50 slot B
    seqs = [m.seq(cap) for _ in range(nd + 3)]
    files = _save_all(seqs[:nd + 1], lens + [1024], str(tmp_path), "c5_", 900)
    try:
        c = m.ctx(max_batch=512, max_ctx=cap)
        p = Plan(c, seqs, cap)
        for i, f in enumerate(files):
            p.load(i, f)
        A, B = nd + 1, nd + 2
        # the same sequences alone: twins of the decoding ones and of the slots
        twins = [m.seq(cap) for _ in range(nd)]
        for tw, sq, n in zip(twins, seqs, lens):
            tw.copy_from(sq, n)
        p.copy(A, nd, 1024)
        ta, tb = m.seq(cap), m.seq(cap)
        ta.copy_from(seqs[nd], 1024)
        toks = [int(t) for t in rng.integers(0, m.vocab, nd)]
        for step in range(2):
            ca = [int(t) for t in rng.integers(0, m.vocab, 512)]
            cb = [int(t) for t in rng.integers(0, m.vocab, 512)]
            dec = [(i, LAST, [toks[i]] if step == 0 else None) for i in range(nd)]
            l1 = p.run(dec + [(A, LAST, ca[:464])])
            l2 = p.run([(A, LAST, ca[464:]), (B, LAST, cb[:464])])
            l3 = p.run([(B, LAST, cb[464:])])
            fed = toks if step == 0 else p.fed[-nd:]
            alone = [c.forward_batch([gw.Segment(tw, [t], LAST)])[0][0] for tw, t in zip(twins, fed)]
            for sq, chunks, got in ((ta, (ca[:464], ca[464:]), (l1[nd], l2[0])), (tb, (cb[:464], cb[464:]), (l2[1], l3[0]))):
                for ch, g in zip(chunks, got):
                    a = c.forward_batch([gw.Segment(sq, ch, LAST)])[0][0]
                    assert np.array_equal(_bits(a), _bits(g)), f"step {step}: a prompt chunk differs from its run alone"
            for i in range(nd):
                assert np.array_equal(_bits(alone[i]), _bits(l1[i])), f"step {step}: decode row {i} differs from its run alone"
            toks = None
        info = p.check(orc, model_8b_1l, str(tmp_path / "ref"), cap)
        assert info["passes"] == 6 and info["rows"] == 2 * (nd + 1024)
    finally:
        _rm(files)
