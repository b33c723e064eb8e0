/* A host program of the reference's own host modules (test infrastructure: tests/test_host_modules.py builds it).
 *
 * It is linked twice from this one source:
 *   ours: libgwenedeg_amd.so (the forward half of runq.h) with the reference's sampler.o, threads.o, spec.o, chat.o,
 *         tokenizer.o and gguf.o compiled unmodified from its sources (oracle/_ref), plus the two model.c helpers
 *         those objects name (below, GW_HOST_STUBS: chat templates and the loader's error exit, never reached without
 *         a tokenizer);
 *   ref:  the reference's whole CPU library (oracle/_ref: model, gguf, forward, tokenizer, sampler, chat, threads,
 *         spec, seqfile).
 * Both runs print the same JSON only if the reference's modules read this library's RqModel / RqSeq fields and drive
 * its passes exactly as they drive the reference's: the sampler (rq_sample, rq_sample_batch: each sequence's RNG
 * state, sampler.c:307-368), the generation loop (rq_generate, chat.c:385-415, with rq_logits_hash of every logits
 * row it samples from) and the speculative loop with prompt lookup (rq_generate_spec, spec.c:404-600: verify passes
 * of several rows through rq_forward_batch, rollbacks by rq_seq_truncate; its output must be rq_generate's).
 *
 *   host_modules MODEL IDS_FILE
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "gwenedeg_gpu.h"

/* the host modules' API (runq.h:376-653, the reference's layouts; tests/test_host_modules.py checks them against
 * runq.h where the reference tree exists) */
typedef struct {
    float temperature;
    float topp;
    const unsigned char *allow;
    int top_k;
} RqSampling;
int rq_sample(RqCtx *c, RqSeq *s, float *logits, const RqSampling *cfg);
int rq_sample_batch(RqCtx *c, RqSeq *const *seqs, float *logits, int n, const RqSampling *cfg, int ncfg, int *tokens);
typedef struct {
    int (*on_token)(void *user, int token);
    void (*on_logits)(void *user, int pos, const float *logits);
    void *user;
} RqCallbacks;
typedef struct {
    int n_prompt, n_gen;
    int stop;
    double t_prefill, t_gen;
} RqGenStats;
int rq_generate(RqCtx *c, RqSeq *s, const int *tokens, int n, const RqSampling *cfg, int max_new, const RqCallbacks *cb,
                RqGenStats *st);
typedef struct {
    int k;
    float tau;
    int lookup;
    int lookup_min;
    const struct RqPassCost *cost, *dcost;
    int (*guess_hook)(void *user, int pos, int depth, int guess, float p1);
    void *hook_user;
    double prior;
} RqSpecOpts;
typedef struct {
    RqGenStats gen;
    int passes, drafted, accepted, draft_steps, refed;
    double t_draft, t_verify;
    int lookup_passes, lookup_drafted, lookup_accepted;
    int mtp_rows, mtp_approx;
} RqSpecStats;
int rq_generate_spec(RqCtx *c, RqSeq *s, RqCtx *dc, RqSeq *ds, const int *tokens, int n, const RqSampling *cfg,
                     int max_new, const RqSpecOpts *o, const RqCallbacks *cb, RqSpecStats *st);
int rq_spec_check(const RqModel *target, const RqModel *draft, char *err, size_t errlen);

#ifdef GW_HOST_STUBS
/* model.c's two helpers that chat.o and tokenizer.o name (model.c:12, :803): the chat templates' generation suffix
 * and the loader's error exit. A maintainer keeps them with the chat templates on the host; without a tokenizer
 * (no_tokenizer, these synthetic files) neither is reached */
const char *chat_gen_suffix(const RqModel *m, int thinking) {
    (void)m;
    (void)thinking;
    return "";
}
void load_fail(void *e, const char *fmt, ...) {
    (void)e;
    fprintf(stderr, "host_modules: load_fail reached: %s\n", fmt);
    abort();
}
#endif

#define MAX_GEN 32

typedef struct {
    int n;
    int pos[4 * MAX_GEN];
    unsigned long long hash[4 * MAX_GEN];
} Trace;

static int V;

static void on_logits(void *user, int pos, const float *logits) {
    Trace *t = user;
    if (t->n < 4 * MAX_GEN) {
        t->pos[t->n] = pos;
        t->hash[t->n++] = rq_logits_hash(logits, V);
    }
}

static void die(const char *what, int e, RqCtx *c) {
    fprintf(stderr, "host_modules: %s: %s %s\n", what, rq_strerror(e), c ? rq_ctx_error(c) : "");
    exit(1);
}

static void print_trace(const Trace *t) {
    printf("[");
    for (int i = 0; i < t->n; i++) printf("%s[%d, \"%016llx\"]", i ? ", " : "", t->pos[i], t->hash[i]);
    printf("]");
}

#include <stddef.h>
static void layouts(void) {
    /* the sizes and offsets of the API types declared above (no device work: the CPU check of the declarations) */
#define L(t, f) printf(#t "." #f " %zu\n", offsetof(t, f))
    printf("RqSampling %zu\nRqCallbacks %zu\nRqGenStats %zu\nRqSpecOpts %zu\nRqSpecStats %zu\n", sizeof(RqSampling),
           sizeof(RqCallbacks), sizeof(RqGenStats), sizeof(RqSpecOpts), sizeof(RqSpecStats));
    L(RqSampling, topp); L(RqSampling, allow); L(RqSampling, top_k); L(RqCallbacks, on_logits); L(RqCallbacks, user);
    L(RqGenStats, stop); L(RqGenStats, t_prefill); L(RqGenStats, t_gen); L(RqSpecOpts, lookup); L(RqSpecOpts, lookup_min);
    L(RqSpecOpts, cost); L(RqSpecOpts, dcost); L(RqSpecOpts, guess_hook); L(RqSpecOpts, hook_user); L(RqSpecOpts, prior);
    L(RqSpecStats, passes); L(RqSpecStats, refed); L(RqSpecStats, t_draft); L(RqSpecStats, t_verify);
    L(RqSpecStats, lookup_passes); L(RqSpecStats, lookup_accepted); L(RqSpecStats, mtp_approx);
#undef L
}

int main(int argc, char **argv) {
    if (argc == 2 && !strcmp(argv[1], "--layouts")) {
        layouts();
        return 0;
    }
    if (argc != 3) {
        fprintf(stderr, "usage: %s MODEL IDS_FILE | --layouts\n", argv[0]);
        return 2;
    }
    FILE *f = fopen(argv[2], "rb");
    if (!f) { perror(argv[2]); return 1; }
    fseek(f, 0, SEEK_END);
    int n = (int)(ftell(f) / 4);
    fseek(f, 0, SEEK_SET);
    int *ids = malloc((size_t)(n > 0 ? n : 1) * sizeof(int));
    if (n < 8 || !ids || fread(ids, 4, (size_t)n, f) != (size_t)n) { fprintf(stderr, "bad ids\n"); return 1; }
    fclose(f);

    char err[512] = "";
    RqModelOpts mo;
    memset(&mo, 0, sizeof mo);
    mo.ctx_len = 512;
    mo.no_tokenizer = 1;
    mo.mem = -1.0;
    RqModel *m = rq_model_load(argv[1], &mo, err, sizeof err);
    if (!m) { fprintf(stderr, "host_modules: load: %s\n", err); return 1; }
    RqModelInfo info;
    rq_model_info(m, &info);
    V = info.vocab_size;
    int e = RQ_OK;
    RqCtx *c = rq_ctx_new(m, 64, 512, &e);
    if (!c) die("rq_ctx_new", e, NULL);
    RqSeq *s[4];
    for (int i = 0; i < 4; i++)
        if (!(s[i] = rq_seq_new(m, 512, RQ_KV_F16, &e))) die("rq_seq_new", e, NULL);
    printf("{");

    /* 1. the sampler on 8 logits rows of a prefill: greedy, top-k, top-p, both, the full distribution; each setting
     * from the same seed, the tokens and the RNG state after the draws */
    const int R = 8;
    float *rows = malloc((size_t)R * V * sizeof(float)), *row = malloc((size_t)V * sizeof(float));
    if ((e = rq_prefill(c, s[0], ids, R, RQ_LOGITS_ALL, rows, NULL)) != RQ_OK) die("rq_prefill", e, c);
    const RqSampling cfgs[5] = { { 0.0f, 0.0f, NULL, 0 }, { 0.8f, 0.0f, NULL, 40 }, { 0.7f, 0.9f, NULL, 0 },
                                 { 1.0f, 0.85f, NULL, 20 }, { 1.3f, 0.0f, NULL, 0 } };
    printf("\"sample\": [");
    for (int k = 0; k < 5; k++) {
        rq_seq_seed(s[0], 1000 + k);
        printf("%s{\"tokens\": [", k ? ", " : "");
        for (int r = 0; r < R; r++) {
            memcpy(row, rows + (size_t)r * V, (size_t)V * sizeof(float));
            int t = rq_sample(c, s[0], row, &cfgs[k]);
            printf("%s%d", r ? ", " : "", t);
        }
        printf("], \"rng\": \"%016llx\"}", *rq_seq_rng(s[0]));
    }
    printf("], ");
    /* rq_sample_batch: four rows, each with its sequence's RNG and its own setting */
    for (int i = 0; i < 4; i++) rq_seq_seed(s[i], 77 + i);
    int bt[4];
    if ((e = rq_sample_batch(c, s, rows, 4, &cfgs[1], 4, bt)) != RQ_OK) die("rq_sample_batch", e, c);
    printf("\"sample_batch\": [%d, %d, %d, %d], \"batch_rng\": [", bt[0], bt[1], bt[2], bt[3]);
    for (int i = 0; i < 4; i++) printf("%s\"%016llx\"", i ? ", " : "", *rq_seq_rng(s[i]));
    printf("], ");

    /* 2. rq_generate and 3. rq_generate_spec with prompt lookup (no draft model: k 0), greedy and sampled, on fresh
     * sequences from the same seed: the tokens, the on_logits trace and the loop's counters */
    static Trace tg, ts;
    /* (greedy falls into a loop the lookup guesses; the top-3 setting mostly repeats and sometimes leaves it: guesses
     * accepted and refused, the refused ones rolled back) */
    const RqSampling gcfg[3] = { { 0.0f, 0.0f, NULL, 0 }, { 0.9f, 0.95f, NULL, 50 }, { 0.5f, 0.0f, NULL, 3 } };
    printf("\"generate\": [");
    for (int k = 0; k < 3; k++) {
        RqCallbacks cb = { NULL, on_logits, &tg };
        RqGenStats gs;
        memset(&tg, 0, sizeof tg);
        rq_seq_reset(s[1]);
        rq_seq_seed(s[1], 4242);
        if ((e = rq_generate(c, s[1], ids, n, &gcfg[k], MAX_GEN, &cb, &gs)) != RQ_OK) die("rq_generate", e, c);
        printf("%s{\"n_gen\": %d, \"stop\": %d, \"rng\": \"%016llx\", \"tokens\": [", k ? ", " : "", gs.n_gen, gs.stop,
               *rq_seq_rng(s[1]));
        const int *tk = rq_seq_tokens(s[1]);
        for (int i = n; i < rq_seq_len(s[1]); i++) printf("%s%d", i > n ? ", " : "", tk[i]);
        printf("], \"logits\": ");
        print_trace(&tg);

        RqSpecOpts so;
        memset(&so, 0, sizeof so);
        so.lookup = 6;
        RqSpecStats ss;
        memset(&ss, 0, sizeof ss);
        cb.user = &ts;
        memset(&ts, 0, sizeof ts);
        rq_seq_reset(s[2]);
        rq_seq_seed(s[2], 4242);
        if ((e = rq_generate_spec(c, s[2], NULL, NULL, ids, n, &gcfg[k], MAX_GEN, &so, &cb, &ss)) != RQ_OK)
            die("rq_generate_spec", e, c);
        printf(", \"spec\": {\"n_gen\": %d, \"stop\": %d, \"rng\": \"%016llx\", \"passes\": %d, \"lookup_passes\": %d, "
               "\"lookup_drafted\": %d, \"lookup_accepted\": %d, \"same_tokens\": %d, \"logits\": ", ss.gen.n_gen,
               ss.gen.stop, *rq_seq_rng(s[2]), ss.passes, ss.lookup_passes, ss.lookup_drafted, ss.lookup_accepted,
               rq_seq_len(s[2]) == rq_seq_len(s[1]) &&
                   !memcmp(rq_seq_tokens(s[2]), rq_seq_tokens(s[1]), (size_t)rq_seq_len(s[1]) * sizeof(int)));
        print_trace(&ts);
        printf("}}");
    }
    printf("], ");
    /* 4. a draft model without its tokenizer is refused (spec.c:48: RQ_ERR_STATE), as the reference refuses it */
    printf("\"spec_check\": %d}\n", rq_spec_check(m, m, err, sizeof err));
    free(rows);
    free(row);
    free(ids);
    for (int i = 0; i < 4; i++) rq_seq_free(s[i]);
    rq_ctx_free(c);
    rq_model_free(m);
    return 0;
}
