/* Saved sequences (runq.h:283-314): the reference's KV disk tier (seqfile.c) over this library's device cache. The file
 * format is the reference's, version 1, so that files move between the two: a 4 KiB header (SfHdr below), the tokens at
 * 4 KiB, then per layer its K blocks and its V blocks (the first nblk blocks of 256 positions, as the cache holds them:
 * the tiled layout of forward.c:1894-1899, which the device cache keeps byte for byte), each section at a multiple of
 * 4 KiB. The blocks go through a host staging buffer (device to host on save, host to device on load), one (layer, K /
 * V) section at a time. Qwen3 only: no recurrent state, no checkpoints; f16 or bf16 KV. Plain buffered I/O, written as
 * path.tmp, synced and renamed (a reader never sees a partial file). */
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include "gw_internal.h"

#define SF_ALIGN 4096
#define SF_VERSION 1
#define SF_CK_MAX 32
static const char sf_magic[8] = { 'R', 'Q', 'S', 'E', 'Q', '\r', '\n', 0x1a };

typedef struct { /* seqfile.c:31-40, version 1: the on-disk header (little-endian, 264 bytes) */
    char magic[8];
    uint32_t version, endian;
    uint64_t model_fp;
    int32_t n_attn, kv_dim, n_kv_heads, head_dim, att_p, att_t, att, kv_esz, n_lin, len, nblk, nck;
    int32_t ck[SF_CK_MAX];
    uint64_t ssm_bytes, ssm_stride, blk_bytes;
    uint64_t off_kv, off_ssm, file_bytes, rng;
    uint64_t hash;
} SfHdr;
_Static_assert(sizeof(SfHdr) == 264, "the saved sequence header's layout");

static uint64_t sf_round(uint64_t n) { return (n + SF_ALIGN - 1) / SF_ALIGN * SF_ALIGN; }

static uint64_t fnv(uint64_t h, const void *p, size_t n) {
    const uint8_t *b = p;
    for (size_t i = 0; i < n; i++) h = (h ^ b[i]) * 1099511628211ull;
    return h;
}

static uint64_t sf_hash(const SfHdr *h, const int *tokens) {
    /* the header with hash 0, then the tokens */
    SfHdr c = *h;
    c.hash = 0;
    return fnv(fnv(1469598103934665603ull, &c, sizeof(c)), tokens, (size_t)h->len * sizeof(int));
}

/* a block's bytes of K (kv 0) or V: ATT_P / ATT_T x n_kv tiles (seqfile.c:49-53) */
static uint64_t sf_blk(const RqModel *m, int kvt, int kv) {
    return (uint64_t)(GW_ATT_P / GW_ATT_T) * m->n_kv_heads * gw_kv_tile_bytes(kvt, m->head_dim, kv);
}
static int sf_type_ok(int kvt) { return gw_kv_ok(kvt); }

static void sf_shape(const RqModel *m, int len, int kvt, SfHdr *h) {
    /* every field but rng and hash, as the reference writes them for this model, length and cache type */
    memset(h, 0, sizeof(*h));
    memcpy(h->magic, sf_magic, 8);
    h->version = SF_VERSION;
    h->endian = 0x01020304;
    h->model_fp = m->fingerprint;
    h->n_attn = m->n_layers;
    h->kv_dim = m->n_kv_heads * m->head_dim;
    h->n_kv_heads = m->n_kv_heads;
    h->head_dim = m->head_dim;
    h->att_p = GW_ATT_P;
    h->att_t = GW_ATT_T;
    h->att = kvt;
    h->kv_esz = (int32_t)(gw_kv_tile_bytes(kvt, m->head_dim, 1) / ((size_t)GW_ATT_T * m->head_dim)); /* (V's, rounded down) */
    h->len = len;
    h->nblk = (len + GW_ATT_P - 1) / GW_ATT_P;
    h->blk_bytes = sf_blk(m, kvt, 0);
    h->off_kv = SF_ALIGN + sf_round((uint64_t)len * sizeof(int));
    h->off_ssm = h->off_kv + (uint64_t)m->n_layers * h->nblk * (h->blk_bytes + sf_blk(m, kvt, 1));
    h->file_bytes = h->off_ssm;
}

static int sf_rw(int fd, int wr, void *buf, size_t n, uint64_t off) {
    /* all n bytes at off; 0, or -1 (a short read past the end included) */
    char *p = buf;
    while (n) {
        ssize_t r = wr ? pwrite(fd, p, n, (off_t)off) : pread(fd, p, n, (off_t)off);
        if (r <= 0) return -1;
        p += r, off += (uint64_t)r, n -= (size_t)r;
    }
    return 0;
}

static int sf_blocks(const RqSeq *s, int fd, int wr, const SfHdr *h, int nblk) {
    /* the first nblk blocks of every (layer, K / V) between the device cache and the file (the file's sections hold
     * h->nblk blocks each), through one host buffer of a section */
    const RqModel *m = s->m;
    const uint64_t bk = sf_blk(m, s->kvt, 0), bv = sf_blk(m, s->kvt, 1);
    void *buf = NULL;
    int rc = 0;
    if (!nblk) return 0;
    if (hipHostMalloc(&buf, (size_t)nblk * (bk > bv ? bk : bv), hipHostMallocDefault) != hipSuccess) return RQ_ERR_NOMEM;
    for (int l = 0; l < m->n_layers && !rc; l++)
        for (int kv = 0; kv < 2 && !rc; kv++) {
            size_t bytes = (size_t)nblk * (kv ? bv : bk);
            uint8_t *dev = (uint8_t *)gw_seq_layer(s, l, kv);
            uint64_t off = h->off_kv + (uint64_t)h->nblk * ((uint64_t)l * (bk + bv) + (kv ? bk : 0));
            if (wr) {
                if (hipMemcpy(buf, dev, bytes, hipMemcpyDeviceToHost) != hipSuccess) rc = RQ_ERR_STATE;
                else if (sf_rw(fd, 1, buf, bytes, off)) rc = RQ_ERR_IO;
            } else {
                if (sf_rw(fd, 0, buf, bytes, off)) rc = RQ_ERR_IO;
                else if (hipMemcpy(dev, buf, bytes, hipMemcpyHostToDevice) != hipSuccess) rc = RQ_ERR_STATE;
            }
        }
    (void)hipHostFree(buf);
    return rc;
}

int rq_seq_save(const RqSeq *s, const char *path) {
    /* seqfile.c:236-297 (runq.h:283-293) */
    if (!s || !path || s->len < 1) return RQ_ERR_ARG;
    SfHdr h;
    sf_shape(s->m, s->len, s->kvt, &h);
    h.rng = s->rng;
    h.hash = sf_hash(&h, s->tokens);
    size_t pl = strlen(path), hn = (size_t)h.off_kv;
    char *tmp = malloc(pl + 5), *head = calloc(1, hn);
    int rc = RQ_ERR_NOMEM, fd = -1;
    if (!tmp || !head) goto done;
    memcpy(tmp, path, pl);
    memcpy(tmp + pl, ".tmp", 5);
    memcpy(head, &h, sizeof(h));
    memcpy(head + SF_ALIGN, s->tokens, (size_t)s->len * sizeof(int));
    rc = RQ_ERR_IO;
    if ((fd = open(tmp, O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644)) < 0) goto done;
    if (posix_fallocate(fd, 0, (off_t)h.file_bytes) || sf_rw(fd, 1, head, hn, 0)) goto fail; /* (a full disk fails here) */
    if ((rc = sf_blocks(s, fd, 1, &h, h.nblk)) != 0) goto fail;
    rc = RQ_ERR_IO;
    if (fdatasync(fd)) goto fail;
    if (close(fd)) { fd = -1; goto fail; }
    fd = -1;
    if (rename(tmp, path)) goto fail;
    rc = RQ_OK;
    goto done;
fail:
    if (fd >= 0) close(fd);
    fd = -1;
    unlink(tmp);
done:
    free(tmp);
    free(head);
    return rc;
}

long long rq_seq_save_bytes(const RqSeq *s) {
    if (!s || s->len < 1) return 0;
    SfHdr h;
    sf_shape(s->m, s->len, s->kvt, &h);
    return (long long)h.file_bytes;
}

static int sf_open_check(const RqModel *m, const char *path, int *fd, SfHdr *h, int **tokens) {
    /* open path, read its header and tokens, check them against m (seqfile.c:182-228: the shape, the derived fields,
     * the size, the hash): RQ_OK with *fd open and *tokens malloc'd, else nothing left open or allocated */
    struct stat st;
    int rc = RQ_ERR_IO;
    *tokens = NULL;
    if ((*fd = open(path, O_RDONLY | O_CLOEXEC)) < 0) return RQ_ERR_IO;
    if (fstat(*fd, &st) || (uint64_t)st.st_size < SF_ALIGN || sf_rw(*fd, 0, h, sizeof(*h), 0)) goto fail;
    rc = RQ_ERR_MISMATCH;
    int lmax = m->seq_len;
    if (h->len < 1 || h->len > lmax) goto fail;
    SfHdr w;
    sf_shape(m, h->len, sf_type_ok(h->att) ? h->att : RQ_KV_F16, &w);
    w.rng = h->rng;
    w.hash = h->hash;
    if (memcmp(&w, h, sizeof(w)) || (uint64_t)st.st_size != h->file_bytes) goto fail;
    rc = RQ_ERR_NOMEM;
    if (!(*tokens = malloc((size_t)h->len * sizeof(int)))) goto fail;
    rc = RQ_ERR_IO;
    if (sf_rw(*fd, 0, *tokens, (size_t)h->len * sizeof(int), SF_ALIGN)) goto fail;
    rc = RQ_ERR_MISMATCH;
    if (sf_hash(h, *tokens) != h->hash) goto fail;
    for (int i = 0; i < h->len; i++)
        if ((*tokens)[i] < 0 || (*tokens)[i] >= m->vocab) goto fail;
    return RQ_OK;
fail:
    free(*tokens);
    *tokens = NULL;
    close(*fd);
    *fd = -1;
    return rc;
}

int rq_seq_file_info(const RqModel *m, const char *path, RqSeqFile *info, int **tokens) {
    /* seqfile.c:306-337 (runq.h:295-305) */
    if (!m || !path || !info) return RQ_ERR_ARG;
    SfHdr h;
    int fd, *tk, rc = sf_open_check(m, path, &fd, &h, &tk);
    if (rc != RQ_OK) return rc;
    close(fd);
    memset(info, 0, sizeof(*info));
    info->len = h.len;
    info->kv_type = h.att;
    info->bytes = (long long)h.file_bytes;
    if (tokens) *tokens = tk;
    else free(tk);
    return RQ_OK;
}

int rq_seq_file_keep(const RqSeqFile *f, int n) {
    /* runq.h:306-308: Qwen3 keeps n itself, clamped to [0, len] */
    return n < 0 ? 0 : n > f->len ? f->len : n;
}

int rq_seq_load(RqSeq *dst, const char *path, int n) {
    /* seqfile.c:340-399 (runq.h:309-314): dst := the first n positions of the saved sequence (only the blocks up to
     * them read), its RNG the saved one; RQ_ERR_IO leaves dst empty */
    if (!dst || !path || n < 0 || n > dst->cap) return RQ_ERR_ARG;
    SfHdr h;
    int fd, *tk, rc = sf_open_check(dst->m, path, &fd, &h, &tk);
    if (rc != RQ_OK) return rc;
    if (n > h.len) {
        rc = RQ_ERR_ARG;
    } else if (h.att != dst->kvt) { /* (the cache's type is the sequence's: runq.h:309-314) */
        rc = RQ_ERR_MISMATCH;
    } else {
        dst->len = 0;
        rc = gw_seq_map(dst, n) != RQ_OK ? RQ_ERR_NOMEM : sf_blocks(dst, fd, 0, &h, (n + GW_ATT_P - 1) / GW_ATT_P);
        if (rc == RQ_OK) {
            memcpy(dst->tokens, tk, (size_t)n * sizeof(int));
            dst->len = n;
            if (n > dst->hwm) dst->hwm = n;
            dst->rng = h.rng;
            dst->hvalid = n; /* (seqfile.c:385; no view here, so no kept hidden state: hpos -1) */
            dst->hpos = -1;
        }
    }
    close(fd);
    free(tk);
    return rc;
}
