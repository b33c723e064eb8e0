/* Driver of the reference's own CPU path (test infrastructure: compiled against the reference's runq.h and
 * linked with its library objects by oracle/Makefile into oracle/_ref/ref_driver; never part of the product).
 *
 * It runs what the parity tests and the CPU baseline need, through the public API only (runq.h):
 *   prefill of the ids in a file (rq_prefill, chunks of max_batch rows), then greedy decode steps (rq_decode +
 *   rq_sample at temperature 0: sampler.c:40-60's first maximum), optionally writing every logits row it
 *   produced (float32), the generated tokens (int32) and the KV cache of the sequence (rq_seq_save's file:
 *   the blocks "as in memory", seqfile.c:8-27), and timing each phase (best of --reps runs; run_s: every run's
 *   prefill + decode wall time).
 *   --batch-decode N: N independent sequences, each prefilled with the same prompt, then --steps batched decode
 *   passes of one row per sequence (rq_forward_batch, RQ_LOGITS_LAST each: batch_decode_worker).
 *   --hidden FILE: instead, the prompt token by token through rq_decode_hidden (runq.h:350), every row's logits and
 *   final hidden state (after output_norm, dim floats) written.
 *   --kv-type T: the sequences' KV cache type (runq.h:214; default RQ_KV_F16).
 *   --plan FILE: instead, a script of passes over sequences loaded from saved KV files (the configs' pass shapes on
 *   caches the device filled: run_plan below); --ids is not read then.
 * Output: one JSON line on stdout. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "runq.h"

static void die(const char *what, int e, RqCtx *c) {
    fprintf(stderr, "ref_driver: %s failed: %s%s%s\n", what, rq_strerror(e), c ? ": " : "", c ? rq_ctx_error(c) : "");
    exit(1);
}

static int *read_ids(const char *path, int *n) {
    FILE *f = fopen(path, "rb");
    if (!f) { perror(path); exit(1); }
    fseek(f, 0, SEEK_END);
    long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    int *v = malloc(sz > 0 ? (size_t)sz : 4);
    if (!v || fread(v, 1, (size_t)sz, f) != (size_t)sz) { perror(path); exit(1); }
    fclose(f);
    *n = (int)(sz / 4);
    return v;
}

static void write_all(FILE *f, const void *p, size_t n) {
    if (f && fwrite(p, 1, n, f) != n) { perror("write"); exit(1); }
}

/* --plan: a text script, one command per line
 *   seqs N CAP              N sequences of capacity CAP (the --kv-type cache)
 *   load I PATH             rq_seq_load of the whole saved sequence PATH into sequence I (rq_seq_file_info's length)
 *   copy I J N              rq_seq_copy: sequence I := the first N positions of sequence J
 *   fill I N SEED           rq_seq_fill_synthetic: sequence I := N cached positions of synthetic K / V (runq.h:726)
 *   pass NSEG               one rq_forward_batch of the NSEG segments on the next NSEG lines:
 *   seg I MODE N T1 .. TN   N tokens for sequence I, RQ_LOGITS_* MODE; a token -1 is the first maximum of the last
 *                           logits row this run produced for sequence I (the greedy feed, sampler.c:40-60)
 * Every selected logits row goes to --logits in pass order, every token a -1 stood for to --tokens; the JSON line
 * lists each pass's rq_forward_batch wall time (pass_s). */
static int run_plan(RqModel *m, RqCtx *c, int V, int kv_type, const char *plan, FILE *lf, FILE *tf) {
    FILE *f = fopen(plan, "r");
    if (!f) { perror(plan); return 1; }
    char cmd[32], path[4096];
    int ns = 0, e, passes = 0, rows = 0, tcap = 64;
    RqSeq **sq = NULL;
    double *pass_s = malloc((size_t)tcap * sizeof(double));
    float *out = malloc((size_t)RQ_BATCH_MAX * V * sizeof(float)), **last = NULL;
    RqSegment *sg = malloc((size_t)RQ_BATCH_MAX * sizeof(RqSegment));
    int *sgi = malloc((size_t)RQ_BATCH_MAX * sizeof(int)); /* each segment's sequence index */
    if (!out || !sg || !sgi || !pass_s) { perror("malloc"); return 1; }
    while (fscanf(f, "%31s", cmd) == 1) {
        if (!strcmp(cmd, "seqs")) {
            int cap;
            if (fscanf(f, "%d %d", &ns, &cap) != 2 || ns < 1) { fprintf(stderr, "plan: bad seqs\n"); return 1; }
            sq = calloc((size_t)ns, sizeof(RqSeq *));
            last = calloc((size_t)ns, sizeof(float *));
            for (int i = 0; i < ns; i++)
                if (!(sq[i] = rq_seq_new(m, cap, kv_type, &e))) die("rq_seq_new", e, NULL);
        } else if (!strcmp(cmd, "load")) {
            int i;
            RqSeqFile fi;
            int *ft = NULL;
            if (fscanf(f, "%d %4095s", &i, path) != 2 || i < 0 || i >= ns) { fprintf(stderr, "plan: bad load\n"); return 1; }
            if ((e = rq_seq_file_info(m, path, &fi, &ft)) != RQ_OK) die("rq_seq_file_info", e, NULL);
            free(ft);
            if ((e = rq_seq_load(sq[i], path, fi.len)) != RQ_OK) die("rq_seq_load", e, NULL);
        } else if (!strcmp(cmd, "copy")) {
            int i, j, n;
            if (fscanf(f, "%d %d %d", &i, &j, &n) != 3 || i < 0 || i >= ns || j < 0 || j >= ns) {
                fprintf(stderr, "plan: bad copy\n");
                return 1;
            }
            if ((e = rq_seq_copy(sq[i], sq[j], n)) != RQ_OK) die("rq_seq_copy", e, NULL);
        } else if (!strcmp(cmd, "fill")) {
            int i, n;
            unsigned long long seed;
            if (fscanf(f, "%d %d %llu", &i, &n, &seed) != 3 || i < 0 || i >= ns) { fprintf(stderr, "plan: bad fill\n"); return 1; }
            if ((e = rq_seq_fill_synthetic(sq[i], n, seed)) != RQ_OK) die("rq_seq_fill_synthetic", e, NULL);
        } else if (!strcmp(cmd, "pass")) {
            int nseg, nt = 0;
            if (fscanf(f, "%d", &nseg) != 1 || nseg < 1 || nseg > RQ_BATCH_MAX) { fprintf(stderr, "plan: bad pass\n"); return 1; }
            int *all = malloc((size_t)RQ_BATCH_MAX * sizeof(int)), nsel = 0;
            for (int k = 0; k < nseg; k++) {
                int i, mode, n;
                if (fscanf(f, "%31s %d %d %d", cmd, &i, &mode, &n) != 4 || strcmp(cmd, "seg") || i < 0 || i >= ns || n < 1 ||
                    nt + n > RQ_BATCH_MAX) {
                    fprintf(stderr, "plan: bad segment\n");
                    return 1;
                }
                for (int j = 0; j < n; j++) {
                    if (fscanf(f, "%d", &all[nt + j]) != 1) { fprintf(stderr, "plan: bad token\n"); return 1; }
                    if (all[nt + j] < 0) { /* the greedy feed */
                        if (!last[i]) { fprintf(stderr, "plan: no logits row yet for sequence %d\n", i); return 1; }
                        int best = 0;
                        for (int v = 1; v < V; v++)
                            if (last[i][v] > last[i][best]) best = v;
                        all[nt + j] = best;
                        write_all(tf, &best, sizeof(int));
                    }
                }
                sg[k] = (RqSegment){ sq[i], all + nt, n, mode, NULL, NULL };
                sgi[k] = i;
                nt += n;
                nsel += mode == RQ_LOGITS_ALL ? n : mode == RQ_LOGITS_LAST;
            }
            double t0 = rq_now();
            if ((e = rq_forward_batch(c, sg, nseg, nsel ? out : NULL, NULL)) != RQ_OK) die("rq_forward_batch", e, c);
            if (passes == tcap && !(pass_s = realloc(pass_s, (size_t)(tcap *= 2) * sizeof(double)))) { perror("realloc"); return 1; }
            pass_s[passes] = rq_now() - t0;
            write_all(lf, out, (size_t)nsel * V * sizeof(float));
            for (int k = 0, r = 0; k < nseg; k++) { /* each sequence's last row of this pass, for a later greedy feed */
                int i = sgi[k], sel = sg[k].logits == RQ_LOGITS_ALL ? sg[k].n : sg[k].logits == RQ_LOGITS_LAST;
                if (sel) {
                    if (!last[i]) last[i] = malloc((size_t)V * sizeof(float));
                    memcpy(last[i], out + (size_t)(r + sel - 1) * V, (size_t)V * sizeof(float));
                }
                r += sel;
            }
            free(all);
            passes++;
            rows += nt;
        } else {
            fprintf(stderr, "plan: unknown command %s\n", cmd);
            return 1;
        }
    }
    fclose(f);
    printf("{\"threads\": %d, \"vocab\": %d, \"passes\": %d, \"rows\": %d, \"pass_s\": [", rq_threads(), V, passes, rows);
    for (int i = 0; i < passes; i++) printf("%s%.6f", i ? ", " : "", pass_s[i]);
    printf("]}\n");
    for (int i = 0; i < ns; i++) {
        rq_seq_free(sq[i]);
        free(last[i]);
    }
    free(sq); free(last); free(out); free(sg); free(sgi); free(pass_s);
    return 0;
}

int main(int argc, char **argv) {
    const char *model = NULL, *ids_path = NULL, *logits_path = NULL, *tokens_path = NULL, *kv_path = NULL, *hidden_path = NULL,
               *plan = NULL;
    int threads = 0, cap = 0, maxb = 512, steps = 0, reps = 1, all_logits = 0, nbd = 0, kv_type = RQ_KV_F16;
    for (int i = 1; i < argc; i++) {
        const char *a = argv[i], *v = i + 1 < argc ? argv[i + 1] : NULL;
        if (!strcmp(a, "-m") && v) model = v, i++;
        else if (!strcmp(a, "-t") && v) threads = atoi(v), i++;
        else if (!strcmp(a, "-c") && v) cap = atoi(v), i++;
        else if (!strcmp(a, "-b") && v) maxb = atoi(v), i++;
        else if (!strcmp(a, "--ids") && v) ids_path = v, i++;
        else if (!strcmp(a, "--steps") && v) steps = atoi(v), i++;
        else if (!strcmp(a, "--reps") && v) reps = atoi(v), i++;
        else if (!strcmp(a, "--logits") && v) logits_path = v, i++;
        else if (!strcmp(a, "--tokens") && v) tokens_path = v, i++;
        else if (!strcmp(a, "--kv") && v) kv_path = v, i++;
        else if (!strcmp(a, "--batch-decode") && v) nbd = atoi(v), i++;
        else if (!strcmp(a, "--all-logits")) all_logits = 1;
        else if (!strcmp(a, "--hidden") && v) hidden_path = v, i++;
        else if (!strcmp(a, "--kv-type") && v) kv_type = atoi(v), i++;
        else if (!strcmp(a, "--plan") && v) plan = v, i++;
        else { fprintf(stderr, "ref_driver: bad argument %s\n", a); return 2; }
    }
    if (!model || (!ids_path && !plan)) { fprintf(stderr, "usage: ref_driver -m MODEL --ids FILE [--steps K] ...\n"); return 2; }
    const char *warn = rq_threads_init(threads);
    if (warn) fprintf(stderr, "ref_driver: %s\n", warn);
    char err[512];
    RqModelOpts mo;
    memset(&mo, 0, sizeof mo);
    mo.no_tokenizer = 1;
    mo.mem = -1;
    mo.ctx_len = cap;
    RqModel *m = rq_model_load(model, &mo, err, sizeof err);
    if (!m) { fprintf(stderr, "ref_driver: load: %s\n", err); return 1; }
    RqModelInfo info;
    rq_model_info(m, &info);
    int V = info.vocab_size, e, n;
    if (plan) {
        RqCtx *pc = rq_ctx_new(m, RQ_BATCH_MAX, cap, &e);
        if (!pc) die("rq_ctx_new", e, NULL);
        FILE *lf = logits_path ? fopen(logits_path, "wb") : NULL, *tf = tokens_path ? fopen(tokens_path, "wb") : NULL;
        if ((logits_path && !lf) || (tokens_path && !tf)) { perror("output"); return 1; }
        int r = run_plan(m, pc, V, kv_type, plan, lf, tf);
        if (lf) fclose(lf);
        if (tf) fclose(tf);
        rq_ctx_free(pc);
        rq_model_free(m);
        return r;
    }
    int *ids = read_ids(ids_path, &n);
    int ns = nbd > 0 ? nbd : 1;
    if (nbd > 0 && maxb < ns) maxb = ns;
    RqCtx *c = rq_ctx_new(m, maxb, cap, &e);
    if (!c) die("rq_ctx_new", e, NULL);
    RqSeq **sq = calloc((size_t)ns, sizeof(RqSeq *));
    for (int i = 0; i < ns; i++)
        if (!(sq[i] = rq_seq_new(m, cap, kv_type, &e))) die("rq_seq_new", e, NULL);
    FILE *lf = logits_path ? fopen(logits_path, "wb") : NULL, *tf = tokens_path ? fopen(tokens_path, "wb") : NULL;
    if ((logits_path && !lf) || (tokens_path && !tf)) { perror("output"); return 1; }
    float *out = malloc((size_t)(all_logits ? n : ns) * V * sizeof(float));
    int *tok = malloc((size_t)ns * sizeof(int));
    RqSegment *sg = malloc((size_t)ns * sizeof(RqSegment));
    RqSampling smp = { 0 };
    double tp_best = 1e30, td_best = 1e30, *run_s = malloc((size_t)(reps > 0 ? reps : 1) * sizeof(double));
    for (int r = 0; r < reps; r++) {
        int last = r == reps - 1; /* outputs of the last run only */
        for (int i = 0; i < ns; i++) rq_seq_reset(sq[i]);
        double t0 = rq_now();
        float *lg = NULL;
        if (hidden_path) { /* the prompt token by token through rq_decode_hidden: every row's logits and final hidden state */
            FILE *hf = fopen(hidden_path, "wb");
            float *hid = malloc((size_t)info.dim * sizeof(float));
            if (!hf || !hid) { perror(hidden_path); return 1; }
            for (int j = 0; j < n; j++) {
                if ((e = rq_decode_hidden(c, sq[0], ids[j], &lg, hid, NULL)) != RQ_OK) die("rq_decode_hidden", e, c);
                write_all(lf, lg, (size_t)V * sizeof(float));
                write_all(hf, hid, (size_t)info.dim * sizeof(float));
            }
            fclose(hf);
            free(hid);
            printf("{\"threads\": %d, \"vocab\": %d, \"dim\": %d, \"prompt\": %d, \"fingerprint\": \"%016llx\"}\n", rq_threads(), V,
                   info.dim, n, (unsigned long long)info.fingerprint);
            if (lf) fclose(lf);
            return 0;
        }
        for (int i = 0; i < ns; i++) {
            if ((e = rq_prefill(c, sq[i], ids, n, all_logits ? RQ_LOGITS_ALL : RQ_LOGITS_LAST, all_logits ? out : NULL, &lg)) != RQ_OK)
                die("rq_prefill", e, c);
            if (last) write_all(lf, lg, (size_t)(all_logits ? n : 1) * V * sizeof(float));
            tok[i] = rq_sample(c, sq[i], lg + (size_t)(all_logits ? n - 1 : 0) * V, &smp);
        }
        double t1 = rq_now();
        for (int s = 0; s < steps; s++) {
            if (last) write_all(tf, tok, (size_t)ns * sizeof(int));
            if (nbd > 0) {
                for (int i = 0; i < ns; i++) sg[i] = (RqSegment){ sq[i], &tok[i], 1, RQ_LOGITS_LAST, NULL, NULL };
                if ((e = rq_forward_batch(c, sg, ns, out, NULL)) != RQ_OK) die("rq_forward_batch", e, c);
                if (last) write_all(lf, out, (size_t)ns * V * sizeof(float));
                for (int i = 0; i < ns; i++) tok[i] = rq_sample(c, sq[i], out + (size_t)i * V, &smp);
            } else {
                if ((e = rq_decode(c, sq[0], tok[0], &lg)) != RQ_OK) die("rq_decode", e, c);
                if (last) write_all(lf, lg, (size_t)V * sizeof(float));
                tok[0] = rq_sample(c, sq[0], lg, &smp);
            }
        }
        double t2 = rq_now();
        tp_best = t1 - t0 < tp_best ? t1 - t0 : tp_best;
        td_best = t2 - t1 < td_best ? t2 - t1 : td_best;
        run_s[r] = t2 - t0;
    }
    if (kv_path && (e = rq_seq_save(sq[0], kv_path)) != RQ_OK) die("rq_seq_save", e, NULL);
    if (lf) fclose(lf);
    if (tf) fclose(tf);
    printf("{\"threads\": %d, \"vocab\": %d, \"prompt\": %d, \"seqs\": %d, \"steps\": %d, \"prefill_s\": %.6f, "
           "\"decode_s\": %.6f, \"prefill_tok_s\": %.3f, \"decode_tok_s\": %.3f, \"fingerprint\": \"%016llx\", \"run_s\": [",
           rq_threads(), V, n, ns, steps, tp_best, td_best, tp_best > 0 ? (double)n * ns / tp_best : 0.0,
           td_best > 0 && steps ? (double)steps * ns / td_best : 0.0, (unsigned long long)info.fingerprint);
    for (int r = 0; r < reps; r++) printf("%s%.6f", r ? ", " : "", run_s[r]);
    printf("]}\n");
    free(run_s);
    for (int i = 0; i < ns; i++) rq_seq_free(sq[i]);
    rq_ctx_free(c);
    rq_model_free(m);
    free(ids); free(out); free(tok); free(sg); free(sq);
    return 0;
}
