/* A C host of the library, as the reference's own programs are (tests/api_test.c, bench_batch.c): it includes the
 * public header, links libgwenedeg_amd.so and drives the forward path through the rq_* calls only (no Python, no
 * torch). Used by tests/test_c_host.py.
 *
 *   c_driver MODEL IDS_FILE STEPS OUT_FILE
 * prefills the int32 ids of IDS_FILE (rq_prefill, RQ_LOGITS_LAST), then STEPS greedy decode steps (rq_decode; the
 * first maximum of the logits, the reference's sample_argmax, sampler.c:40-60), and writes every logits row it got
 * (float32, vocab each) to OUT_FILE. Prints one line: the tokens and rq_logits_hash of the last row. */
#include <stdio.h>
#include <stdlib.h>

#include "gwenedeg_gpu.h"

static int first_max(const float *v, int n) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

int main(int argc, char **argv) {
    if (argc != 5) {
        fprintf(stderr, "usage: %s MODEL IDS_FILE STEPS OUT_FILE\n", argv[0]);
        return 2;
    }
    FILE *f = fopen(argv[2], "rb");
    if (!f) { perror(argv[2]); return 1; }
    fseek(f, 0, SEEK_END);
    long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    int n = (int)(sz / 4), steps = atoi(argv[3]);
    int *ids = malloc((size_t)(n > 0 ? n : 1) * sizeof(int));
    if (!ids || fread(ids, 4, (size_t)n, f) != (size_t)n) { perror("read ids"); return 1; }
    fclose(f);

    char err[256] = "";
    RqModelOpts o = { 0 };
    o.ctx_len = n + steps + 1;
    o.no_tokenizer = 1;
    o.mem = -1.0;
    RqModel *m = rq_model_load(argv[1], &o, err, sizeof err);
    if (!m) { fprintf(stderr, "rq_model_load: %s\n", err); return 1; }
    RqModelInfo info;
    rq_model_info(m, &info);
    int e = RQ_OK, V = info.vocab_size;
    RqSeq *s = rq_seq_new(m, n + steps + 1, RQ_KV_F16, &e);
    if (!s) { fprintf(stderr, "rq_seq_new: %s\n", rq_strerror(e)); return 1; }
    RqCtx *c = rq_ctx_new(m, 64, n + steps + 1, &e);
    if (!c) { fprintf(stderr, "rq_ctx_new: %s\n", rq_strerror(e)); return 1; }
    FILE *out = fopen(argv[4], "wb");
    if (!out) { perror(argv[4]); return 1; }

    float *lg = NULL;
    if ((e = rq_prefill(c, s, ids, n, RQ_LOGITS_LAST, NULL, &lg)) != RQ_OK) {
        fprintf(stderr, "rq_prefill: %s: %s\n", rq_strerror(e), rq_ctx_error(c));
        return 1;
    }
    printf("tokens");
    for (int i = 0; i <= steps; i++) {
        if (fwrite(lg, sizeof(float), (size_t)V, out) != (size_t)V) { perror("write"); return 1; }
        int tok = first_max(lg, V);
        printf(" %d", tok);
        if (i == steps) break;
        if ((e = rq_decode(c, s, tok, &lg)) != RQ_OK) {
            fprintf(stderr, "rq_decode: %s: %s\n", rq_strerror(e), rq_ctx_error(c));
            return 1;
        }
    }
    printf(" hash %llu len %d\n", rq_logits_hash(lg, V), rq_seq_len(s));
    fclose(out);
    rq_ctx_free(c);
    rq_seq_free(s);
    rq_model_free(m);
    free(ids);
    return 0;
}
