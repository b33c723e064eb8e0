/* The host side of model.c that the reference's host modules keep calling when this library replaces model.o: the
 * loader's error exit, the chat templates, and the tokenizer of rq_model_load (model.c:1010-1016, :893-922).
 *
 * The tokenizer itself is not rebuilt here. The host program links the reference's own tokenizer.o, gguf.o and
 * threads.o (they stay on the host: rq_tokenize, rq_token_bytes, rq_detok_*, chat.c's rendering all read RqModel.tok);
 * this file calls their build entry points (gguf_parse, gguf_chat_variant, gguf_sampling, build_tokenizer_gguf,
 * free_tokenizer) through weak references. Linked with those objects, rq_model_load fills RqModel.tok, .chat, the
 * recommended sampling and the templates at the reference's offsets and sets has_tok, as the reference does. Loaded
 * by a program without them (the Python binding, a host that only runs passes), the references stay null and the model
 * loads without a tokenizer, as RqModelOpts.no_tokenizer gives; RqModelInfo.warning says why. */
#include <setjmp.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "gw_internal.h"

/* LoadErr (internal.h:187): where load_fail formats its message, and the jump back to the loader */
typedef struct {
    jmp_buf jb;
    char *msg;
    size_t len;
} GwLoadErr;

/* Gguf (internal.h:198-205): the GGUF directory gguf_parse fills (the mapped file, its key / value and tensor
 * entries, the error exit); used here only while the tokenizer is built, then freed */
typedef struct {
    const uint8_t *map;
    uint64_t size;
    const char *path;
    uint32_t version;
    uint64_t alignment, data_off;
    void *kv;
    uint64_t n_kv;
    void *t;
    uint64_t n_t;
    GwLoadErr *err;
} GwRefGguf;

_Static_assert(sizeof(GwLoadErr) == 216 && offsetof(GwLoadErr, msg) == 200, "LoadErr layout (internal.h:187)");
_Static_assert(sizeof(GwRefGguf) == 88 && offsetof(GwRefGguf, kv) == 48 && offsetof(GwRefGguf, err) == 80,
               "Gguf layout (internal.h:198-205)");

/* the host's gguf.o / tokenizer.o (null where the program does not link them) */
void gguf_parse(GwRefGguf *g) __attribute__((weak));
int gguf_chat_variant(const GwRefGguf *g) __attribute__((weak));
int gguf_sampling(const GwRefGguf *g, float *temp, float *topp, int *topk) __attribute__((weak));
void build_tokenizer_gguf(GwRefTokenizer *t, const GwRefGguf *g, int vocab_size) __attribute__((weak));
void free_tokenizer(GwRefTokenizer *t) __attribute__((weak));

void load_fail(GwLoadErr *e, const char *fmt, ...) {
    /* model.c:12-18: the message into the loader's buffer, then back to the loader (gguf.o's gguf_fail and
     * tokenizer.o's allocation failures end here) */
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(e->msg, e->len, fmt, ap);
    va_end(ap);
    longjmp(e->jb, 1);
}

/* The chat turns of a GGUF model (model.c:790-796): Qwen3's ChatML strings with one %s, and the generation prompt's
 * think block. They are the text the model was trained on, so they are the reference's byte for byte */
#define GW_TMPL_SYS "<|im_start|>system\n%s<|im_end|>\n"
#define GW_TMPL_USER "<|im_start|>user\n%s<|im_end|>\n<|im_start|>assistant\n"
#define GW_TMPL_NOTHINK "<think>\n\n</think>\n\n"
#define GW_TMPL_THINK "<think>\n"

const char *rq_chat_name(int v) {
    /* runq.h:459 (model.c:798-801) */
    return v == RQ_CHAT_INSTRUCT ? "instruct-2507" : v == RQ_CHAT_THINKING ? "thinking-2507" : v == RQ_CHAT_QWEN35 ? "qwen3.5"
         : v == RQ_CHAT_QWEN38 ? "qwen3.8" : "qwen3";
}

const char *chat_gen_suffix(const RqModel *m, int thinking) {
    /* model.c:803-809: what the generation prompt adds after the assistant header, by variant and thinking mode */
    if (m->chat == RQ_CHAT_INSTRUCT) return "";
    if (m->chat == RQ_CHAT_THINKING || m->chat == RQ_CHAT_QWEN35 || m->chat == RQ_CHAT_QWEN38)
        return thinking ? GW_TMPL_THINK : GW_TMPL_NOTHINK;
    return thinking ? "" : GW_TMPL_NOTHINK;
}

int rq_chat_check(const RqModel *m, int thinking, char *err, size_t errlen) {
    /* runq.h (model.c:851-862): the templates of that thinking mode are usable */
    thinking = thinking != 0;
    if (!m->has_tok) {
        snprintf(err, errlen, "model loaded without a tokenizer");
        return RQ_ERR_STATE;
    }
    if (m->tmpl_missing[thinking][0]) {
        snprintf(err, errlen, "%s", m->tmpl_missing[thinking]);
        return RQ_ERR_LOAD;
    }
    return RQ_OK;
}

int gw_host_tokenizer_linked(void) {
    return gguf_parse && gguf_chat_variant && gguf_sampling && build_tokenizer_gguf && free_tokenizer;
}

static int build_guarded(RqModel *m0, GwRefGguf *g0, GwLoadErr *e) {
    /* the build with its error exit (only volatile locals are live across the setjmp): 0 after a load_fail */
    RqModel *volatile m = m0;
    GwRefGguf *volatile g = g0;
    if (setjmp(e->jb)) return 0;
    gguf_parse(g);
    m->chat = gguf_chat_variant(g);
    m->samp_set = gguf_sampling(g, &m->samp_temp, &m->samp_topp, &m->samp_topk);
    build_tokenizer_gguf(&m->tok, g, m->config.vocab_size);
    return 1;
}

int gw_host_tokenizer(RqModel *m, const char *path, const void *map, size_t size, char *err, size_t errlen) {
    /* model.c:1010-1016 (GGUF): the tokenizer from the file's metadata, the chat variant, the recommended sampling, then
     * the templates (model.c:827-836, GGUF: the variant's generation prompt); RQ_OK with has_tok 1, or RQ_ERR_LOAD with
     * the reference's message in err and nothing left allocated. m->config.vocab_size: the embedding rows */
    if (!gw_host_tokenizer_linked()) return RQ_ERR_STATE;
    GwLoadErr *e = calloc(1, sizeof *e);
    GwRefGguf *g = calloc(1, sizeof *g);
    if (!e || !g) {
        free(e);
        free(g);
        snprintf(err, errlen, "malloc failed!");
        return RQ_ERR_NOMEM;
    }
    e->msg = err;
    e->len = errlen;
    g->map = map;
    g->size = size;
    g->path = path;
    g->err = e;
    int ok = build_guarded(m, g, e);
    free(g->kv);
    free(g->t);
    free(g);
    free(e);
    if (!ok) {
        free_tokenizer(&m->tok);
        memset(&m->tok, 0, sizeof m->tok);
        m->chat = 0;
        m->samp_set = 0;
        return RQ_ERR_LOAD;
    }
    m->has_tok = 1;
    for (int t = 0; t < 2; t++) {
        m->tmpl_missing[t][0] = 0;
        snprintf(m->user_tmpl[t], sizeof m->user_tmpl[t], "%s%s", GW_TMPL_USER, chat_gen_suffix(m, t));
        snprintf(m->sys_tmpl[t], sizeof m->sys_tmpl[t], "%s", GW_TMPL_SYS);
    }
    return RQ_OK;
}

void gw_host_free_tokenizer(RqModel *m) {
    if (m->has_tok && free_tokenizer) free_tokenizer(&m->tok);
    m->has_tok = 0;
}
