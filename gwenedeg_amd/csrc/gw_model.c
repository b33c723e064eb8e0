/* Model load for the MI355X backend: rq_model_load / rq_model_free / rq_model_info (runq.h:87-147) and the small
 * process-wide helpers of runq.h (rq_strerror, rq_now, rq_threads*, rq_kv_*, rq_logits_hash).
 *
 * The GGUF file (llama.cpp's format v2 / v3, qwen3 architecture) is mapped, its metadata checked the way the
 * reference's gguf_config does (gguf.c:230-336: eps 1e-6, heads a multiple of kv heads, key = value length, no
 * RoPE scaling), and its matrices (tensor names of model.c:269-299) are copied to the device once and repacked there:
 *   Q8_0: the 34-byte blocks split into int8 codes (row-major) + fp16 scales (k_q8_unpack): 34 bytes per 32 weights
 *         as in the file; wq / wk / wv fused into one (qd + 2 kv_dim) x dim matrix, w1 / w3 into one 2 hidden x dim
 *         matrix when all are Q8_0 (one GEMV launch each)
 *   Q4_K / Q6_K: the file's blocks as they are (the kernels decode them)
 * The norms (F32) go to one device buffer; the RoPE cos / sin table of every position up to the context cap is
 * computed here on the host with rope_row's expressions (forward.c:1248-1264) and uploaded (seq_len x head_dim fp32).
 */
#define _GNU_SOURCE
#include <fcntl.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

#include "gw_internal.h"

/* ----------------------------------------------------------------------------------------- helpers */

const char *rq_strerror(int e) {
    switch (e) {
    case RQ_OK: return "ok";
    case RQ_ERR_ARG: return "invalid argument";
    case RQ_ERR_NOMEM: return "out of memory";
    case RQ_ERR_CONTEXT: return "context full";
    case RQ_ERR_STATE: return "invalid state";
    case RQ_ERR_LOAD: return "load failed";
    case RQ_ERR_IO: return "I/O error";
    case RQ_ERR_MISMATCH: return "mismatch";
    default: return "unknown error";
    }
}

double rq_mem_available(void) {
    /* runq.h:172-173: MemAvailable of /proc/meminfo in bytes, -1 where unknown */
    FILE *f = fopen("/proc/meminfo", "r");
    char line[256];
    long long kb = -1;
    while (f && fgets(line, sizeof(line), f))
        if (sscanf(line, "MemAvailable: %lld kB", &kb) == 1) break;
    if (f) fclose(f);
    return kb >= 0 ? (double)kb * 1024.0 : -1.0;
}

RqModel *rq_mtp_load(const RqModel *target, const RqMtpOpts *o, char *err, size_t errlen) {
    /* runq.h:100-112: MTP views are Qwen3.5's; a Qwen3 model has no MTP block */
    (void)target;
    (void)o;
    if (err && errlen) snprintf(err, errlen, "no MTP block (MTP views are Qwen3.5's; this library loads Qwen3 models)");
    return NULL;
}

int rq_repack_info(const RqModel *m, RqRepackInfo *info) {
    /* runq.h:175-195 (model.c:1402-1438) for the device: per type among IQ3_S, IQ3_XXS (repackable) and IQ1_S, IQ1_M,
     * over the matmul weights (the classifier, then every layer's q, k, v, o, gate, up, down) */
    memset(info, 0, sizeof(*info));
    if (!m || !m->has_weights) return RQ_ERR_STATE;
    info->available = 1;
    info->weights = m->dev_bytes;
    static const int types[RQ_REPACK_TYPES] = { GW_IQ3_S, GW_IQ3_XXS, GW_IQ1_S, GW_IQ1_M };
    static const int bits[RQ_REPACK_TYPES] = { RQ_REPACK_IQ3_S, RQ_REPACK_IQ3_XXS, 0, 0 };
    static const char *const names[RQ_REPACK_TYPES] = { "IQ3_S", "IQ3_XXS", "IQ1_S", "IQ1_M" };
    double all = 0;
    const GwMat **mats = malloc(((size_t)7 * m->n_layers + 1) * sizeof(*mats));
    int nm = 0;
    if (!mats) return RQ_ERR_NOMEM;
    if (!m->tied) mats[nm++] = &m->cls;
    for (int l = 0; l < m->n_layers; l++) {
        const GwLayer *y = &m->layer[l];
        for (int i = 0; i < y->nqkv; i++) mats[nm++] = &y->qkv[i];
        mats[nm++] = &y->wo;
        for (int i = 0; i < y->nw13; i++) mats[nm++] = &y->w13[i];
        mats[nm++] = &y->w2;
    }
    for (int i = 0; i < nm; i++) all += (double)mats[i]->rows * mats[i]->cols;
    for (int j = 0; j < RQ_REPACK_TYPES; j++) {
        RqRepackType *x = &info->t[info->n];
        for (int i = 0; i < nm; i++) {
            const GwMat *w = mats[i];
            if ((w->type & ~GW_IQ_R) != types[j]) continue;
            const size_t nblk = (size_t)w->rows * (w->cols / 256);
            x->mats++;
            x->share += (double)w->rows * w->cols / all;
            x->bytes += nblk * (size_t)gw_kq_dev_bytes(w->type);
            x->repacked = w->type != types[j];
            x->extra += bits[j] ? nblk * (size_t)(GW_IQ3R_DEV - gw_kq_dev_bytes(types[j]))
                                : nblk * (size_t)(gw_kq_dev_bytes(types[j]) - gw_kq_file_bytes(types[j]));
        }
        if (!x->mats) continue;
        x->type = names[j];
        x->bit = bits[j];
        if (x->bit && !x->repacked) info->extra += x->extra;
        info->n++;
    }
    free(mats);
    return RQ_OK;
}

int rq_dequant_rows(const RqModel *m, const char *name, size_t name_len, long r0, long nr, float **rows, float **packed,
                    int *ncols, int *npacked, char *err, size_t errlen) {
    /* runq.h:716-720 (a test hook reading the file's blocks): the file is not kept after the load here */
    (void)m, (void)name, (void)name_len, (void)r0, (void)nr, (void)ncols;
    if (rows) *rows = NULL;
    if (packed) *packed = NULL;
    if (npacked) *npacked = 0;
    if (err && errlen) snprintf(err, errlen, "rq_dequant_rows: the weights live in device memory; the file is not kept");
    return RQ_ERR_STATE;
}

double rq_now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

const char *rq_threads_init(int n) { (void)n; return NULL; }
int rq_threads(void) { return 1; }

const char *rq_kv_name(int t) {
    static const char *name[] = { "f32", "bf16", "f16", "q8", "?", "bf16-dot", "f16-dot", "q8-dot", "q4", "q4k4", "?", "?",
                                  "q4-dot", "q4k4-dot" };
    return t >= 0 && t < 14 ? name[t] : "?";
}

int rq_kv_parse(const char *s) {
    for (int t = 0; t < 14; t++)
        if (s && strcmp(rq_kv_name(t), "?") && !strcmp(s, rq_kv_name(t))) return t;
    return RQ_ERR_ARG;
}

int rq_kv_bits(int t) {
    const char *n = rq_kv_name(t);
    if (!strcmp(n, "?")) return 0;
    int e = t & ~4;
    return e == RQ_KV_F32 ? 32 : e == RQ_KV_Q8 ? 8 : e == RQ_KV_Q4 ? 6 : e == RQ_KV_Q4K4 ? 4 : 16;
}

unsigned long long rq_logits_hash(const float *logits, int n) {
    /* FNV-1a over the bytes (runq.h:559-561) */
    unsigned long long h = 1469598103934665603ull;
    const unsigned char *p = (const unsigned char *)logits;
    for (size_t i = 0; i < (size_t)n * sizeof(float); i++) {
        h ^= p[i];
        h *= 1099511628211ull;
    }
    return h;
}

int gw_hip_fail(char *err, size_t errlen, const char *what, hipError_t e) {
    if (err && errlen) snprintf(err, errlen, "%s: %s", what, hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? RQ_ERR_NOMEM : RQ_ERR_STATE;
}

int gw_device_init(char *err, size_t errlen) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n < 1) {
        if (err && errlen) snprintf(err, errlen, "no HIP device (%s)", e != hipSuccess ? hipGetErrorString(e) : "0 devices");
        return RQ_ERR_STATE;
    }
    return RQ_OK;
}

/* ------------------------------------------------------------------------------------------- GGUF */

typedef struct { const char *key; size_t klen; uint32_t type, atype; uint64_t n; size_t off; } Kv;
typedef struct { const char *name; size_t nlen; uint32_t nd, type; uint64_t ne[4]; uint64_t off, size; } Tn;
typedef struct {
    const uint8_t *map; size_t size; Kv *kv; uint64_t nkv; Tn *t; uint64_t nt; size_t data;
} Gguf;

static const size_t gv_size[13] = { 1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8 };

static int take(const Gguf *g, size_t *p, void *dst, size_t n) {
    if (n > g->size || *p > g->size - n) return 0;
    if (dst) memcpy(dst, g->map + *p, n);
    *p += n;
    return 1;
}

static size_t type_row_bytes(uint32_t type, uint64_t k, int *ok) {
    *ok = 1;
    switch (type) {
    case GW_F32: return (size_t)k * 4;
    case GW_Q8_0: if (k % 32) break; return (size_t)k / 32 * 34;
    case GW_Q2_K: case GW_Q3_K: case GW_Q4_K: case GW_Q5_K: case GW_Q6_K: case GW_IQ4_XS: case GW_IQ2_XXS: case GW_IQ2_XS:
    case GW_IQ2_S: case GW_IQ3_XXS: case GW_IQ3_S: case GW_IQ1_S: case GW_IQ1_M:
        if (k % 256) break;
        return (size_t)k / 256 * (size_t)gw_kq_file_bytes((int)type);
    default: break;
    }
    *ok = 0;
    return 0;
}

static int gguf_parse(Gguf *g, char *err, size_t errlen) {
    size_t p = 0;
    uint32_t magic = 0, ver = 0;
    if (!take(g, &p, &magic, 4) || magic != 0x46554747u) { snprintf(err, errlen, "not a GGUF file (bad magic)"); return 0; }
    if (!take(g, &p, &ver, 4) || (ver != 2 && ver != 3)) { snprintf(err, errlen, "unsupported GGUF version %u", ver); return 0; }
    if (!take(g, &p, &g->nt, 8) || !take(g, &p, &g->nkv, 8) || g->nt > 65536 || g->nkv > 65536) {
        snprintf(err, errlen, "corrupt GGUF header");
        return 0;
    }
    g->kv = calloc(g->nkv + 1, sizeof(Kv));
    g->t = calloc(g->nt + 1, sizeof(Tn));
    if (!g->kv || !g->t) { snprintf(err, errlen, "malloc failed"); return 0; }
    uint64_t align = 32;
    for (uint64_t i = 0; i < g->nkv; i++) {
        Kv *kv = &g->kv[i];
        uint64_t kl;
        if (!take(g, &p, &kl, 8) || kl > g->size - p) goto bad;
        kv->key = (const char *)g->map + p;
        kv->klen = kl;
        p += kl;
        if (!take(g, &p, &kv->type, 4)) goto bad;
        kv->n = 1;
        uint32_t et = kv->type;
        if (kv->type == 9) {
            if (!take(g, &p, &kv->atype, 4) || !take(g, &p, &kv->n, 8)) goto bad;
            et = kv->atype;
        }
        if (et >= 13 || et == 9) goto bad;
        kv->off = p;
        for (uint64_t j = 0; j < kv->n; j++) {
            if (et == 8) {
                uint64_t sl;
                if (!take(g, &p, &sl, 8) || !take(g, &p, NULL, sl)) goto bad;
            } else if (!take(g, &p, NULL, gv_size[et])) goto bad;
        }
        if (kl == 17 && !memcmp(kv->key, "general.alignment", 17) && kv->type == 4) {
            uint32_t a;
            memcpy(&a, g->map + kv->off, 4);
            if (!a || (a & (a - 1))) goto bad;
            align = a;
        }
    }
    for (uint64_t i = 0; i < g->nt; i++) {
        Tn *t = &g->t[i];
        uint64_t nl;
        if (!take(g, &p, &nl, 8) || nl > g->size - p) goto bad;
        t->name = (const char *)g->map + p;
        t->nlen = nl;
        p += nl;
        if (!take(g, &p, &t->nd, 4) || t->nd < 1 || t->nd > 4) goto bad;
        for (uint32_t d = 0; d < 4; d++) {
            t->ne[d] = 1;
            if (d < t->nd && (!take(g, &p, &t->ne[d], 8) || t->ne[d] == 0 || t->ne[d] > (1ull << 32))) goto bad;
        }
        if (!take(g, &p, &t->type, 4) || !take(g, &p, &t->off, 8)) goto bad;
        int ok;
        size_t rb = type_row_bytes(t->type, t->ne[0], &ok);
        t->size = ok ? rb * t->ne[1] * t->ne[2] * t->ne[3] : (uint64_t)-1;
    }
    g->data = (p + align - 1) / align * align;
    for (uint64_t i = 0; i < g->nt; i++) {
        Tn *t = &g->t[i];
        if (t->off % align || g->data > g->size || t->off > g->size - g->data ||
            (t->size != (uint64_t)-1 && t->size > g->size - g->data - t->off))
            goto bad;
        t->off += g->data;
    }
    return 1;
bad:
    snprintf(err, errlen, "truncated or corrupt GGUF file");
    return 0;
}

static const Kv *gguf_kv(const Gguf *g, const char *key) {
    size_t n = strlen(key);
    for (uint64_t i = 0; i < g->nkv; i++)
        if (g->kv[i].klen == n && !memcmp(g->kv[i].key, key, n)) return &g->kv[i];
    return NULL;
}

static int gguf_int(const Gguf *g, const char *key, int64_t *v) {
    const Kv *kv = gguf_kv(g, key);
    if (!kv) return 0;
    const uint8_t *p = g->map + kv->off;
    switch (kv->type) {
    case 0: *v = *p; return 1;
    case 1: *v = (int8_t)*p; return 1;
    case 2: { uint16_t x; memcpy(&x, p, 2); *v = x; return 1; }
    case 3: { int16_t x; memcpy(&x, p, 2); *v = x; return 1; }
    case 4: { uint32_t x; memcpy(&x, p, 4); *v = x; return 1; }
    case 5: { int32_t x; memcpy(&x, p, 4); *v = x; return 1; }
    case 10: { uint64_t x; memcpy(&x, p, 8); *v = (int64_t)x; return 1; }
    case 11: { int64_t x; memcpy(&x, p, 8); *v = x; return 1; }
    default: return 0;
    }
}

static int gguf_float(const Gguf *g, const char *key, float *v) {
    const Kv *kv = gguf_kv(g, key);
    if (!kv) return 0;
    if (kv->type == 6) { memcpy(v, g->map + kv->off, 4); return 1; }
    if (kv->type == 12) { double d; memcpy(&d, g->map + kv->off, 8); *v = (float)d; return 1; }
    return 0;
}

static const char *gguf_str(const Gguf *g, const char *key, size_t *n) {
    const Kv *kv = gguf_kv(g, key);
    if (!kv || kv->type != 8) return NULL;
    uint64_t l;
    memcpy(&l, g->map + kv->off, 8);
    *n = (size_t)l;
    return (const char *)g->map + kv->off + 8;
}

static const Tn *gguf_tensor(const Gguf *g, const char *name) {
    size_t n = strlen(name);
    for (uint64_t i = 0; i < g->nt; i++)
        if (g->t[i].nlen == n && !memcmp(g->t[i].name, name, n)) return &g->t[i];
    return NULL;
}

/* ------------------------------------------------------------------------------------------- load */

typedef struct {
    Gguf g;
    char *err;
    size_t errlen;
    uint8_t *stage;     /* device staging buffer for a tensor's file bytes */
    int repack;         /* RqModelOpts.repack for the matrices being loaded (0: the embedding table) */
    size_t stage_bytes;
    RqModel *m;
} Loader;

static int lfail(Loader *L, int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(L->err, L->errlen, fmt, ap);
    va_end(ap);
    return code;
}

static int dmalloc(Loader *L, void **p, size_t n) {
    hipError_t e = hipMalloc(p, n ? n : 16);
    if (e != hipSuccess) { *p = NULL; return gw_hip_fail(L->err, L->errlen, "hipMalloc (weights)", e); }
    L->m->dev_bytes += n;
    return RQ_OK;
}

static const Tn *need(Loader *L, const char *name, uint64_t ne0, uint64_t ne1, int *rc) {
    const Tn *t = gguf_tensor(&L->g, name);
    if (!t) { *rc = lfail(L, RQ_ERR_LOAD, "GGUF: tensor %s not found", name); return NULL; }
    if ((ne1 && (t->nd != 2 || t->ne[0] != ne0 || t->ne[1] != ne1)) || (!ne1 && (t->nd != 1 || t->ne[0] != ne0))) {
        *rc = lfail(L, RQ_ERR_LOAD, "GGUF: tensor %s has shape [%llu, %llu], need [%llu, %llu]", name,
                    (unsigned long long)t->ne[0], (unsigned long long)(t->nd > 1 ? t->ne[1] : 0), (unsigned long long)ne0,
                    (unsigned long long)ne1);
        return NULL;
    }
    if (t->size == (uint64_t)-1) { *rc = lfail(L, RQ_ERR_LOAD, "GGUF: tensor %s: unsupported type %u", name, t->type); return NULL; }
    return t;
}

static int stage(Loader *L, const Tn *t) {
    /* the tensor's file bytes into the device staging buffer */
    hipError_t e = hipMemcpy(L->stage, L->g.map + t->off, t->size, hipMemcpyHostToDevice);
    return e == hipSuccess ? RQ_OK : gw_hip_fail(L->err, L->errlen, "hipMemcpy (weights)", e);
}

/* matrix `name` (rows x cols): Q8_0 unpacked into dst's codes / scales from row r0 on (dst pre-allocated for Q8_0), or
 * with il > 0 interleaved with another matrix in blocks of il rows (this one's rows at offset off of each block pair);
 * K-quants: the blocks copied (dst allocated here) */
static int load_mat_il(Loader *L, GwMat *dst, int r0, const char *name, int rows, int cols, int il, int off) {
    int rc = RQ_OK;
    const Tn *t = need(L, name, (uint64_t)cols, (uint64_t)rows, &rc);
    if (!t) return rc;
    if (t->type == GW_Q8_0) {
        if (dst->type != GW_Q8_0) return lfail(L, RQ_ERR_LOAD, "GGUF: %s: internal type mismatch", name);
        if ((rc = stage(L, t)) != RQ_OK) return rc;
        if (gw_k_q8_unpack(L->stage, (size_t)rows * (cols / 32), dst->codes + (size_t)r0 * cols, dst->scales + (size_t)r0 * (cols / 32),
                           cols / 32, il, off, 0))
            return lfail(L, RQ_ERR_STATE, "GGUF: %s: repack kernel failed", name);
        hipError_t e = hipDeviceSynchronize();
        return e == hipSuccess ? RQ_OK : gw_hip_fail(L->err, L->errlen, "repack", e);
    }
    if (!GW_IS_KQ((int)t->type)) return lfail(L, RQ_ERR_LOAD, "GGUF: %s: ggml type %u not supported", name, t->type);
    if (r0 != 0 || dst->rows != rows) return lfail(L, RQ_ERR_LOAD, "GGUF: %s: internal shape mismatch", name);
    dst->type = (int)t->type;
    /* RqModelOpts.repack (model.c:360-364): IQ3_XXS / IQ3_S as 4-bit codes */
    const int rbit = dst->type == GW_IQ3_S ? RQ_REPACK_IQ3_S : dst->type == GW_IQ3_XXS ? RQ_REPACK_IQ3_XXS : 0;
    if (rbit && L->repack > 0 && (L->repack & (RQ_REPACK_ALL | rbit))) dst->type |= GW_IQ_R;
    const int fb = gw_kq_file_bytes(dst->type), db = gw_kq_dev_bytes(dst->type);
    size_t nblk = t->size / (size_t)fb;
    dst->bstride = db;
    if ((rc = dmalloc(L, (void **)&dst->blocks, nblk * (size_t)db)) != RQ_OK) return rc;
    if (fb == db) { /* Q4_K, Q5_K: the file's blocks as they are */
        hipError_t e = hipMemcpy(dst->blocks, L->g.map + t->off, t->size, hipMemcpyHostToDevice);
        return e == hipSuccess ? RQ_OK : gw_hip_fail(L->err, L->errlen, "hipMemcpy (weights)", e);
    }
    /* Q6_K, Q3_K, Q2_K: staged as the file's blocks, then padded to a 16-byte multiple each (aligned loads); the
     * i-quants: staged, then their fields reordered (gw_iq.h) */
    if ((rc = stage(L, t)) != RQ_OK) return rc;
    if (gw_k_kq_to_dev(L->stage, nblk, dst->type, dst->blocks, 0))
        return lfail(L, RQ_ERR_STATE, "GGUF: %s: repack kernel failed", name);
    hipError_t e = hipDeviceSynchronize();
    return e == hipSuccess ? RQ_OK : gw_hip_fail(L->err, L->errlen, "repack", e);
}

static int alloc_q8(Loader *L, GwMat *w, int rows, int cols) {
    w->type = GW_Q8_0;
    w->rows = rows;
    w->cols = cols;
    int rc = dmalloc(L, (void **)&w->codes, (size_t)rows * cols);
    /* (rounded up to 4 bytes: the decode GEMV reads each scale as its aligned 32-bit word) */
    if (rc == RQ_OK) rc = dmalloc(L, (void **)&w->scales, ((size_t)rows * (cols / 32) * 2 + 3) & ~(size_t)3);
    return rc;
}

static int load_mat(Loader *L, GwMat *dst, int r0, const char *name, int rows, int cols) {
    return load_mat_il(L, dst, r0, name, rows, cols, 0, 0);
}

static int tensor_type(Loader *L, const char *name) {
    const Tn *t = gguf_tensor(&L->g, name);
    return t ? (int)t->type : -1;
}

/* a group of matrices fused into one when all are Q8_0 (rows stacked), else each its own */
static int load_group(Loader *L, GwMat *out, int *nout, int n, const char *const *names, const int *rows, int cols, int il) {
    /* n matrices of `cols` columns: all Q8_0 -> one matrix of their rows stacked (il = 0) or, for n = 2 of equal rows,
     * interleaved in blocks of il rows; else n matrices as they are */
    int all_q8 = 1, tot = 0, rc;
    for (int i = 0; i < n; i++) {
        all_q8 &= tensor_type(L, names[i]) == GW_Q8_0;
        tot += rows[i];
    }
    if (all_q8) {
        *nout = 1;
        if ((rc = alloc_q8(L, &out[0], tot, cols)) != RQ_OK) return rc;
        if (il && (n != 2 || rows[0] != rows[1] || rows[0] % il)) return lfail(L, RQ_ERR_LOAD, "GGUF: %s: cannot interleave", names[0]);
        for (int i = 0, r0 = 0; i < n; r0 += rows[i], i++)
            if ((rc = load_mat_il(L, &out[0], il ? 0 : r0, names[i], rows[i], cols, il, il * i)) != RQ_OK) return rc;
        return RQ_OK;
    }
    *nout = n;
    for (int i = 0; i < n; i++) {
        out[i].rows = rows[i];
        out[i].cols = cols;
        out[i].type = tensor_type(L, names[i]);
        if (out[i].type == GW_Q8_0 && (rc = alloc_q8(L, &out[i], rows[i], cols)) != RQ_OK) return rc;
        if ((rc = load_mat(L, &out[i], 0, names[i], rows[i], cols)) != RQ_OK) return rc;
    }
    return RQ_OK;
}

static int load_single(Loader *L, GwMat *w, const char *name, int rows, int cols) {
    int rc;
    w->rows = rows;
    w->cols = cols;
    w->type = tensor_type(L, name);
    if (w->type == GW_Q8_0 && (rc = alloc_q8(L, w, rows, cols)) != RQ_OK) return rc;
    return load_mat(L, w, 0, name, rows, cols);
}

static void free_mat(GwMat *w) {
    if (w->codes) hipFree(w->codes);
    if (w->scales) hipFree(w->scales);
    if (w->blocks) hipFree(w->blocks);
    memset(w, 0, sizeof(*w));
}

void rq_model_free(RqModel *m) {
    if (!m) return;
    gw_host_free_tokenizer(m);
    if (m->layer)
        for (int l = 0; l < m->n_layers; l++) {
            for (int i = 0; i < 3; i++) free_mat(&m->layer[l].qkv[i]);
            free_mat(&m->layer[l].wo);
            for (int i = 0; i < 2; i++) free_mat(&m->layer[l].w13[i]);
            free_mat(&m->layer[l].w2);
        }
    free(m->layer);
    if (!m->tied) free_mat(&m->cls);
    free_mat(&m->embd);
    if (m->norms) hipFree(m->norms);
    if (m->rope) hipFree(m->rope);
    free(m);
}

static unsigned long long fingerprint(const uint8_t *map, size_t size) {
    /* model.c:949-953: FNV-1a 64 over the file size's 8 bytes (little-endian), its first MiB and its last 64 KiB: the
     * owner of saved sequences (rq_seq_save) and RqModelInfo.fingerprint, equal to the reference's for the same file */
    unsigned long long h = 1469598103934665603ull, sz = (unsigned long long)size;
    size_t a = size < (1u << 20) ? size : (1u << 20), b = size < 65536 ? size : 65536;
    for (int i = 0; i < 8; i++) h = (h ^ ((sz >> (8 * i)) & 0xffu)) * 1099511628211ull;
    for (size_t i = 0; i < a; i++) h = (h ^ map[i]) * 1099511628211ull;
    for (size_t i = size - b; i < size; i++) h = (h ^ map[i]) * 1099511628211ull;
    return h;
}

static void rope_table(float *cs, int hd, int npos, float log_theta) {
    /* rope_row (forward.c:1248-1264) for positions 0..npos-1, with the libm calls the reference's build makes there:
     * expf, and one sincosf for the cosf / sinf pair */
    for (int pos = 0; pos < npos; pos++, cs += hd)
        for (int j = 0; j < hd / 2; j++) {
            float freq = expf(log_theta * (-(float)j / (hd / 2))), c, sn;
            sincosf(pos * freq, &sn, &c);
            cs[j] = c;
            cs[j + hd / 2] = sn;
        }
}


RqModel *rq_model_load(const char *path, const RqModelOpts *o, char *err, size_t errlen) {
    char dummy[8];
    if (!err) err = dummy, errlen = sizeof dummy;
    err[0] = 0;
    RqModelOpts opts;
    memset(&opts, 0, sizeof opts);
    if (o) opts = *o;
    if (opts.tokenizer_only && !gw_host_tokenizer_linked()) {
        snprintf(err, errlen, "tokenizer_only: the program does not link the tokenizer (tokenizer.o, gguf.o, threads.o)");
        return NULL;
    }
    if (!opts.tokenizer_only && (gw_device_init(err, errlen) != RQ_OK || gw_exact_init(err, errlen) != RQ_OK ||
                                 gw_iq_init(err, errlen) != RQ_OK))
        return NULL;
    Loader L;
    memset(&L, 0, sizeof L);
    L.err = err;
    L.errlen = errlen;
    int fd = open(path, O_RDONLY);
    if (fd < 0) { snprintf(err, errlen, "cannot open %s", path); return NULL; }
    struct stat st;
    if (fstat(fd, &st) || st.st_size < 64) { snprintf(err, errlen, "%s: not a model file", path); close(fd); return NULL; }
    L.g.size = (size_t)st.st_size;
    void *map = mmap(NULL, L.g.size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) { snprintf(err, errlen, "%s: mmap failed", path); return NULL; }
    L.g.map = map;
    RqModel *m = calloc(1, sizeof(RqModel));
    int rc = RQ_OK;
    if (!m) { snprintf(err, errlen, "malloc failed"); goto out; }
    L.m = m;
    if (!gguf_parse(&L.g, err, errlen)) { rc = RQ_ERR_LOAD; goto out; }
    size_t n;
    const char *arch = gguf_str(&L.g, "general.architecture", &n);
    if (!arch || n != 5 || memcmp(arch, "qwen3", 5)) { rc = lfail(&L, RQ_ERR_LOAD, "architecture is not supported (need qwen3)"); goto out; }
    static const char *keys[7] = { "qwen3.block_count", "qwen3.embedding_length", "qwen3.feed_forward_length",
                                   "qwen3.attention.head_count", "qwen3.attention.head_count_kv", "qwen3.context_length",
                                   "qwen3.attention.key_length" };
    int64_t v[7];
    for (int i = 0; i < 7; i++) {
        if (!gguf_int(&L.g, keys[i], &v[i])) {
            if (i < 6) { rc = lfail(&L, RQ_ERR_LOAD, "metadata %s missing", keys[i]); goto out; }
            v[i] = v[1] / v[3];
        }
        if (v[i] < 1 || v[i] > (1 << 20)) { rc = lfail(&L, RQ_ERR_LOAD, "metadata %s out of range", keys[i]); goto out; }
    }
    int64_t vl = v[6];
    if (gguf_int(&L.g, "qwen3.attention.value_length", &vl) && vl != v[6]) {
        rc = lfail(&L, RQ_ERR_LOAD, "attention key_length != value_length is not supported");
        goto out;
    }
    float theta = 0, eps = 0;
    if (!gguf_float(&L.g, "qwen3.rope.freq_base", &theta) || !(theta >= 1e3f && theta <= 1e9f)) {
        rc = lfail(&L, RQ_ERR_LOAD, "qwen3.rope.freq_base missing or out of range (1e3 .. 1e9)");
        goto out;
    }
    if (!gguf_float(&L.g, "qwen3.attention.layer_norm_rms_epsilon", &eps) || eps != 1e-6f) {
        rc = lfail(&L, RQ_ERR_LOAD, "qwen3.attention.layer_norm_rms_epsilon must be 1e-6");
        goto out;
    }
    const char *rs = gguf_str(&L.g, "qwen3.rope.scaling.type", &n);
    if (rs && !(n == 4 && !memcmp(rs, "none", 4))) { rc = lfail(&L, RQ_ERR_LOAD, "RoPE scaling is not supported"); goto out; }
    m->n_layers = (int)v[0];
    m->dim = (int)v[1];
    m->hidden = (int)v[2];
    m->n_heads = (int)v[3];
    m->n_kv_heads = (int)v[4];
    m->ctx_max = (int)v[5];
    m->head_dim = (int)v[6];
    const Tn *emb = gguf_tensor(&L.g, "token_embd.weight");
    if (!emb || emb->nd != 2 || emb->ne[0] != (uint64_t)m->dim || emb->ne[1] > (1u << 24)) {
        rc = lfail(&L, RQ_ERR_LOAD, "tensor token_embd.weight missing or not [embedding_length, vocab]");
        goto out;
    }
    m->vocab = (int)emb->ne[1];
    m->tied = gguf_tensor(&L.g, "output.weight") == NULL;
    int hd = m->head_dim, nh = m->n_heads, nkv = m->n_kv_heads, dim = m->dim, H = m->hidden, qd = nh * hd, kvd = nkv * hd;
    /* the shapes the kernels take (forward_model_init, forward.c:127-144, plus the device kernels' limits) */
    if (nh % nkv || hd % 32 || hd > 128 || 256 % hd || dim % 256 || H % 256 || qd % 256 || (nh / nkv) > 16 || dim > 16384 || qd > 4096 || H > 65536) {
        rc = lfail(&L, RQ_ERR_LOAD, "unsupported shape (dim %d, hidden %d, heads %d / %d, head_dim %d)", dim, H, nh, nkv, hd);
        goto out;
    }
    int cap = opts.ctx_len > 0 ? opts.ctx_len : (m->ctx_max < RQ_CTX_DEFAULT_MAX ? m->ctx_max : RQ_CTX_DEFAULT_MAX);
    if (cap > m->ctx_max && opts.ctx_len <= 0) cap = m->ctx_max;
    m->seq_len = cap;
    m->rope_theta = theta;
    m->log_theta = (float)log((double)theta);
    m->att_scale = gw_rsqrt_host((float)hd); /* forward.c:137 as compiled: 1.0f / sqrtf(head_dim) */
    m->fingerprint = fingerprint(L.g.map, L.g.size);
    /* the reference's view of the model (its host modules read these: the layout note in gw_internal.h) */
    m->config = (GwRefConfig){ 0, 0, m->dim, m->hidden, m->n_layers, m->n_heads, m->n_kv_heads, m->vocab, m->seq_len,
                               m->head_dim, m->tied, 32 };
    m->ref_fp = m->fingerprint;
    m->is_gguf = 1;
    if (opts.tokenizer_only) goto tokenizer;
    /* device staging: the largest tensor */
    size_t big = 0;
    for (uint64_t i = 0; i < L.g.nt; i++)
        if (L.g.t[i].size != (uint64_t)-1 && L.g.t[i].size > big) big = L.g.t[i].size;
    hipError_t he = hipMalloc((void **)&L.stage, big);
    if (he != hipSuccess) { rc = gw_hip_fail(err, errlen, "hipMalloc (staging)", he); goto out; }
    m->layer = calloc((size_t)m->n_layers, sizeof(GwLayer));
    if (!m->layer) { rc = lfail(&L, RQ_ERR_NOMEM, "malloc failed"); goto out; }
    if ((rc = load_single(&L, &m->embd, "token_embd.weight", m->vocab, dim)) != RQ_OK) goto out;
    m->repack = opts.repack > 0 ? opts.repack : 0;
    L.repack = m->repack; /* (the matmul weights from here on) */
    if (m->tied) m->cls = m->embd;
    else if ((rc = load_single(&L, &m->cls, "output.weight", m->vocab, dim)) != RQ_OK) goto out;
    char nm[3][96];
    for (int l = 0; l < m->n_layers; l++) {
        GwLayer *y = &m->layer[l];
        snprintf(nm[0], 96, "blk.%d.attn_q.weight", l);
        snprintf(nm[1], 96, "blk.%d.attn_k.weight", l);
        snprintf(nm[2], 96, "blk.%d.attn_v.weight", l);
        const char *qkvn[3] = { nm[0], nm[1], nm[2] };
        int qkvr[3] = { qd, kvd, kvd };
        if ((rc = load_group(&L, y->qkv, &y->nqkv, 3, qkvn, qkvr, dim, 0)) != RQ_OK) goto out;
        snprintf(nm[0], 96, "blk.%d.attn_output.weight", l);
        if ((rc = load_single(&L, &y->wo, nm[0], dim, qd)) != RQ_OK) goto out;
        snprintf(nm[0], 96, "blk.%d.ffn_gate.weight", l);
        snprintf(nm[1], 96, "blk.%d.ffn_up.weight", l);
        const char *w13n[2] = { nm[0], nm[1] };
        int w13r[2] = { H, H };
        if ((rc = load_group(&L, y->w13, &y->nw13, 2, w13n, w13r, dim, GW_W13_IL)) != RQ_OK) goto out;
        y->w13_il = y->nw13 == 1 ? GW_W13_IL : 0;
        snprintf(nm[0], 96, "blk.%d.ffn_down.weight", l);
        if ((rc = load_single(&L, &y->w2, nm[0], dim, H)) != RQ_OK) goto out;
    }
    for (int l = 0; l < m->n_layers && !m->kq; l++)
        m->kq = m->layer[l].nqkv > 1 || m->layer[l].nw13 > 1 || m->layer[l].wo.type != GW_Q8_0 || m->layer[l].w2.type != GW_Q8_0;
    m->kq |= m->embd.type != GW_Q8_0 || m->cls.type != GW_Q8_0;
    /* norms: [att L x dim | ffn L x dim | q L x hd | k L x hd | final dim] */
    {
        size_t nf = (size_t)2 * m->n_layers * dim + (size_t)2 * m->n_layers * hd + dim;
        float *hn = malloc(nf * sizeof(float));
        if (!hn) { rc = lfail(&L, RQ_ERR_NOMEM, "malloc failed"); goto out; }
        size_t o2 = 0;
        struct { const char *fmt; int len; } nn[4] = { { "blk.%d.attn_norm.weight", dim }, { "blk.%d.ffn_norm.weight", dim },
                                                     { "blk.%d.attn_q_norm.weight", hd }, { "blk.%d.attn_k_norm.weight", hd } };
        for (int k = 0; k < 4 && rc == RQ_OK; k++)
            for (int l = 0; l < m->n_layers; l++) {
                snprintf(nm[0], 96, nn[k].fmt, l);
                const Tn *t = need(&L, nm[0], (uint64_t)nn[k].len, 0, &rc);
                if (!t) break;
                if (t->type != GW_F32) { rc = lfail(&L, RQ_ERR_LOAD, "GGUF: %s must be F32", nm[0]); break; }
                memcpy(hn + o2, L.g.map + t->off, (size_t)nn[k].len * 4);
                o2 += nn[k].len;
            }
        const Tn *t = rc == RQ_OK ? need(&L, "output_norm.weight", (uint64_t)dim, 0, &rc) : NULL;
        if (t && t->type != GW_F32) rc = lfail(&L, RQ_ERR_LOAD, "GGUF: output_norm.weight must be F32");
        if (rc == RQ_OK) {
            memcpy(hn + o2, L.g.map + t->off, (size_t)dim * 4);
            if ((rc = dmalloc(&L, (void **)&m->norms, nf * 4)) == RQ_OK) {
                he = hipMemcpy(m->norms, hn, nf * 4, hipMemcpyHostToDevice);
                if (he != hipSuccess) rc = gw_hip_fail(err, errlen, "hipMemcpy (norms)", he);
            }
        }
        free(hn);
        if (rc != RQ_OK) goto out;
        for (int l = 0; l < m->n_layers; l++) {
            m->layer[l].att_norm = m->norms + (size_t)l * dim;
            m->layer[l].ffn_norm = m->norms + (size_t)(m->n_layers + l) * dim;
            m->layer[l].q_norm = m->norms + (size_t)2 * m->n_layers * dim + (size_t)l * hd;
            m->layer[l].k_norm = m->norms + (size_t)2 * m->n_layers * dim + (size_t)(m->n_layers + l) * hd;
        }
        m->final_norm = m->norms + (size_t)2 * m->n_layers * dim + (size_t)2 * m->n_layers * hd;
    }
    {
        size_t nr = (size_t)m->seq_len * hd;
        float *cs = malloc(nr * sizeof(float));
        if (!cs) { rc = lfail(&L, RQ_ERR_NOMEM, "malloc failed"); goto out; }
        rope_table(cs, hd, m->seq_len, m->log_theta);
        if ((rc = dmalloc(&L, (void **)&m->rope, nr * 4)) == RQ_OK) {
            he = hipMemcpy(m->rope, cs, nr * 4, hipMemcpyHostToDevice);
            if (he != hipSuccess) rc = gw_hip_fail(err, errlen, "hipMemcpy (rope)", he);
        }
        free(cs);
        if (rc != RQ_OK) goto out;
    }
    hipGetDevice(&m->device);
    m->has_weights = 1;
tokenizer:
    /* model.c:1010-1016: the tokenizer unless no_tokenizer (the host's tokenizer.o / gguf.o, gw_host.c) */
    if (!opts.no_tokenizer) {
        if (gw_host_tokenizer_linked()) rc = gw_host_tokenizer(m, path, L.g.map, L.g.size, err, errlen);
        else
            snprintf(m->warning, sizeof m->warning, "no tokenizer: the program does not link tokenizer.o / gguf.o "
                                                    "(token ids only, as RqModelOpts.no_tokenizer)");
    }
out:
    if (L.stage) hipFree(L.stage);
    free(L.g.kv);
    free(L.g.t);
    munmap(map, L.g.size);
    if (rc != RQ_OK) {
        if (!err[0]) snprintf(err, errlen, "%s", rq_strerror(rc));
        rq_model_free(m);
        return NULL;
    }
    return m;
}

void rq_model_info(const RqModel *m, RqModelInfo *info) {
    memset(info, 0, sizeof(*info));
    info->dim = m->dim;
    info->hidden_dim = m->hidden;
    info->n_layers = m->n_layers;
    info->n_heads = m->n_heads;
    info->n_kv_heads = m->n_kv_heads;
    info->head_dim = m->head_dim;
    info->vocab_size = m->vocab;
    info->seq_len = m->seq_len;
    info->ctx_max = m->ctx_max;
    info->group_size = 32;
    info->shared_classifier = m->tied;
    info->gguf = 1;
    info->bos = m->has_tok ? (int)m->tok.bos_token_id : -1;
    info->eos = m->has_tok ? (int)m->tok.eos_token_id : -1;
    info->warning = m->warning[0] ? m->warning : NULL;
    info->chat = m->chat;
    info->rope_theta = m->rope_theta;
    info->fingerprint = m->fingerprint;
}
