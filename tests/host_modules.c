/* A host program of the reference's own host modules (test infrastructure: tests/test_host_modules.py builds it).
 *
 * It is linked twice from this one source:
 *   ours: libgwenedeg_amd.so (the forward half of runq.h, the weight path of model.c and its chat-template helpers)
 *         with the reference's sampler.o, threads.o, spec.o, chat.o, tokenizer.o and gguf.o compiled unmodified from
 *         its sources (oracle/_ref);
 *   ref:  the reference's whole CPU library (oracle/_ref: model, gguf, forward, tokenizer, sampler, chat, threads,
 *         spec, seqfile).
 * Both runs print the same JSON only if the reference's modules read this library's RqModel / RqSeq fields and drive
 * its passes exactly as they drive the reference's: the sampler (rq_sample, rq_sample_batch: each sequence's RNG
 * state, sampler.c:307-368), the generation loop (rq_generate, chat.c:385-415, with rq_logits_hash of every logits
 * row it samples from) and the speculative loop with prompt lookup (rq_generate_spec, spec.c:404-600: verify passes
 * of several rows through rq_forward_batch, rollbacks by rq_seq_truncate; its output must be rq_generate's).
 *
 * With --tok (a model file with a tokenizer block), the model is loaded with its tokenizer, which the library builds
 * through the host's tokenizer.o / gguf.o at rq_model_load (model.c:1010-1016), and a last section prints what the
 * text side gives on it: rq_model_info's bos / eos / chat variant, rq_chat_check, rq_tokenize and rq_token_bytes,
 * rq_chat_render of a conversation in both thinking modes, rq_generate from that prompt (stopping at an end token)
 * and its reply through rq_detok_push / rq_detok_flush.
 *
 * With --tokenizer-only, the model is loaded with RqModelOpts.tokenizer_only (no weights, no device: this mode runs
 * on any host) and the text side is printed without the reply.
 *
 *   host_modules MODEL IDS_FILE [--tok] | MODEL --tokenizer-only
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

/* the tokenizer and chat API (runq.h:408-500), the reference's tokenizer.o and chat.o */
typedef struct {
    int *v;
    int n, cap;
} RqTokens;
void rq_tokens_free(RqTokens *t);
int rq_tokenize(const RqModel *m, const char *text, long len, RqTokens *out);
const char *rq_token_bytes(const RqModel *m, int token, int *len);
int rq_is_end_token(const RqModel *m, int token);
int rq_token_is_added(const RqModel *m, int token);
typedef struct {
    unsigned char b[8];
    int n;
} RqDetok;
int rq_detok_push(const RqModel *m, RqDetok *d, int token, char *out, size_t cap);
int rq_detok_flush(RqDetok *d, char *out, size_t cap);
enum { RQ_ROLE_SYSTEM = 0, RQ_ROLE_USER = 1, RQ_ROLE_ASSISTANT = 2 };
typedef struct {
    int role;
    const char *content;
} RqMessage;
int rq_chat_render(const RqModel *m, const RqMessage *msgs, int n, int thinking, RqTokens *out);

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

static void print_ids(const RqTokens *t) {
    printf("[");
    for (int i = 0; i < t->n; i++) printf("%s%d", i ? ", " : "", t->v[i]);
    printf("]");
}

static void print_hex(const char *p, int n) {
    printf("\"");
    for (int i = 0; i < n; i++) printf("%02x", (unsigned char)p[i]);
    printf("\"");
}

static int collect(void *user, int token) {
    RqTokens *t = user;
    if (t->n < t->cap) t->v[t->n++] = token;
    return 0;
}

static void text_side(RqModel *m, RqCtx *c, RqSeq *s) {
    /* 5. the tokenizer and the chat templates the library built at rq_model_load, and a chat reply generated from
     * them (--tok) */
    char err[512];
    RqModelInfo mi;
    rq_model_info(m, &mi);
    printf(", \"tok\": {\"bos\": %d, \"eos\": %d, \"chat\": \"%s\", \"check\": [%d, %d], \"end\": [%d, %d, %d], "
           "\"added\": [%d, %d], \"tokenize\": [", mi.bos, mi.eos, rq_chat_name(mi.chat), rq_chat_check(m, 0, err, sizeof err),
           rq_chat_check(m, 1, err, sizeof err), rq_is_end_token(m, mi.eos), rq_is_end_token(m, mi.bos),
           rq_is_end_token(m, 300), rq_token_is_added(m, mi.eos), rq_token_is_added(m, 300));
    static const char *const texts[3] = { "Hello world, the answer is 42.\n\nWhat do you think about the model?",
                                          "<|im_start|>user\nwhy would you write that?<|im_end|>\n",
                                          "  the  people   2024 ...  \t\xc3\xa9t\xc3\xa9 \xe2\x82\xac" "5" };
    for (int k = 0; k < 3; k++) {
        RqTokens t = { NULL, 0, 0 };
        int e = rq_tokenize(m, texts[k], -1, &t);
        printf("%s{\"rc\": %d, \"ids\": ", k ? ", " : "", e);
        print_ids(&t);
        char back[512];
        int nb = 0;
        for (int i = 0; i < t.n; i++) {
            int len = 0;
            const char *b = rq_token_bytes(m, t.v[i], &len);
            if (nb + len < (int)sizeof back) memcpy(back + nb, b, (size_t)len), nb += len;
        }
        printf(", \"round_trip\": %d}", nb == (int)strlen(texts[k]) && !memcmp(back, texts[k], (size_t)nb));
        rq_tokens_free(&t);
    }
    printf("], \"render\": [");
    const RqMessage conv[4] = { { RQ_ROLE_SYSTEM, "You are a helpful model." }, { RQ_ROLE_USER, "What is the answer?" },
                                { RQ_ROLE_ASSISTANT, "The answer is 42." }, { RQ_ROLE_USER, "Why would you think that?" } };
    RqTokens prompt = { NULL, 0, 0 };
    for (int th = 0; th < 2; th++) {
        RqTokens t = { NULL, 0, 0 };
        int e = rq_chat_render(m, conv, 4, th, &t);
        printf("%s{\"rc\": %d, \"ids\": ", th ? ", " : "", e);
        print_ids(&t);
        printf("}");
        if (!th) prompt = t;
        else rq_tokens_free(&t);
    }
    if (!c) { /* (tokenizer_only: no passes) */
        printf("]}");
        rq_tokens_free(&prompt);
        return;
    }
    /* the reply: greedy, until an end token or 24 tokens */
    static int buf[64];
    RqTokens reply = { buf, 0, 24 };
    RqCallbacks cb = { collect, NULL, &reply };
    RqGenStats gs;
    memset(&gs, 0, sizeof gs);
    const RqSampling greedy = { 0.0f, 0.0f, NULL, 0 };
    rq_seq_reset(s);
    int e = rq_generate(c, s, prompt.v, prompt.n, &greedy, 24, &cb, &gs);
    printf("], \"reply\": {\"rc\": %d, \"n_gen\": %d, \"stop\": %d, \"ids\": ", e, gs.n_gen, gs.stop);
    print_ids(&reply);
    char text[4096];
    int nt = 0;
    RqDetok d;
    memset(&d, 0, sizeof d);
    for (int i = 0; i < reply.n; i++) nt += rq_detok_push(m, &d, reply.v[i], text + nt, sizeof text - (size_t)nt);
    nt += rq_detok_flush(&d, text + nt, sizeof text - (size_t)nt);
    printf(", \"text\": ");
    print_hex(text, nt);
    printf("}}");
    rq_tokens_free(&prompt);
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
    printf("RqTokens %zu\nRqDetok %zu\nRqMessage %zu\n", sizeof(RqTokens), sizeof(RqDetok), sizeof(RqMessage));
    L(RqTokens, n); L(RqTokens, cap); L(RqDetok, n); L(RqMessage, content);
#undef L
}

int main(int argc, char **argv) {
    if (argc == 2 && !strcmp(argv[1], "--layouts")) {
        layouts();
        return 0;
    }
    if (argc == 3 && !strcmp(argv[2], "--tokenizer-only")) {
        /* the header and the tokenizer only (RqModelOpts.tokenizer_only, model.c:893-922): no weights, no device; a
         * context or a sequence of it is refused (RQ_ERR_STATE) */
        char err[512] = "";
        RqModelOpts mo;
        memset(&mo, 0, sizeof mo);
        mo.tokenizer_only = 1;
        RqModel *m = rq_model_load(argv[1], &mo, err, sizeof err);
        if (!m) {
            printf("{\"load\": \"%s\"}\n", err);
            return 0;
        }
        int ec = 0, es = 0;
        RqCtx *c = rq_ctx_new(m, 1, 64, &ec);
        RqSeq *q = rq_seq_new(m, 64, RQ_KV_F16, &es);
        printf("{\"ctx\": [%d, %d], \"seq\": [%d, %d]", c != NULL, ec, q != NULL, es);
        text_side(m, NULL, NULL);
        printf("}\n");
        rq_model_free(m);
        return 0;
    }
    if (argc != 3 && !(argc == 4 && !strcmp(argv[3], "--tok"))) {
        fprintf(stderr, "usage: %s MODEL IDS_FILE [--tok] | --layouts\n", argv[0]);
        return 2;
    }
    const int tok = argc == 4;
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
    mo.no_tokenizer = !tok;
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
    /* 4. a draft model without its tokenizer is refused (spec.c:48: RQ_ERR_STATE), as the reference refuses it; with
     * the tokenizers of two models of one vocabulary it is accepted */
    printf("\"spec_check\": %d", rq_spec_check(m, m, err, sizeof err));
    if (tok) text_side(m, c, s[3]);
    printf("}\n");
    free(rows);
    free(row);
    free(ids);
    for (int i = 0; i < 4; i++) rq_seq_free(s[i]);
    rq_ctx_free(c);
    rq_model_free(m);
    return 0;
}
