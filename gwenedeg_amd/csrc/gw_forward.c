/* The forward passes on the device: sequences (RqSeq: a KV cache in device memory), compute contexts (RqCtx: device
 * activations, one HIP stream) and rq_decode / rq_prefill / rq_forward_batch (runq.h:222-375).
 *
 * One pass = n rows (each a token of some sequence at that sequence's next position) through every layer:
 *   embed -> per layer: [residual +] rmsnorm + quantize -> q / k / v matmul -> QK-norm + RoPE + K / V store ->
 *   attention partials per (row block, kv head, 256-position block) -> combine + quantize -> wo matmul ->
 *   residual + rmsnorm + quantize -> w1 / w3 matmul -> SwiGLU + quantize -> w2 matmul
 *   -> final residual + rmsnorm + quantize of the selected rows -> classifier -> logits to the host.
 * A one-row pass of an all-Q8_0 model (decode) runs the fused sequence instead: per layer qkv matmul (rmsnorm +
 * quantize in its prologue) -> QK-norm + RoPE + K / V store -> attention partials -> wo matmul (combine + quantize in
 * its prologue, + residual) -> w1 / w3 matmul (rmsnorm + quantize in its prologue, SwiGLU in its epilogue) -> w2 matmul
 * (quantize in its prologue, + residual), and the classifier's GEMV computes the final rmsnorm + quantize itself: the
 * same arithmetic, four kernels fewer per layer.
 * The same kernels run every row whatever its batch-mates (decode is a one-row pass), and each output is computed
 * whole in a fixed order, so a sequence's results do not depend on what it is batched with (runq.h:22-24).
 * Errors: every argument is validated before any device work (forward.c:3775-3800), so a failed pass changes nothing;
 * HIP failures come back as RQ_ERR_NOMEM / RQ_ERR_STATE with the text in rq_ctx_error.
 */
#define _GNU_SOURCE
#include <stdarg.h>
#include <stdio.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "gw_internal.h"

#define GW_KT_MAX 32768 /* timed launches held before a collection (gw_ctx_kernel_timing) */
#define HIPCHK(c, what, x) do { hipError_t e_ = (x); if (e_ != hipSuccess) return ctx_hip(c, what, e_); } while (0)

static int ctx_fail(RqCtx *c, int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(c->err, sizeof(c->err), fmt, ap);
    va_end(ap);
    return code;
}

static int ctx_hip(RqCtx *c, const char *what, hipError_t e) {
    return gw_hip_fail(c->err, sizeof(c->err), what, e);
}

/* ---------------------------------------------------------------------------------------- sequences */

/* bytes of one layer's K (kv 0) or V cache: kv_len / 16 x n_kv tiles */
static size_t seq_layer_bytes(const RqSeq *s, int kv) {
    return (size_t)s->kv_len / GW_ATT_T * s->m->n_kv_heads * gw_kv_tile_bytes(s->kvt, s->m->head_dim, kv);
}
#define seq_layer gw_seq_layer

/* Lazy device memory (HIP virtual memory). A sequence reserves the address range of its capacity at rq_seq_new and
 * maps physical memory in chunks of GW_SEQ_CHUNK bytes per layer and half as positions are first written (gw_seq_map,
 * called before every pass, copy, fill and load); rq_seq_release unmaps the chunks past the kept positions. So a
 * sequence of a large capacity holds only what it has used, as the reference's host memory does (its pages are touched
 * on first write and given back by madvise, forward.c:474-510). A chunk serves 2 MiB / (block bytes) 256-position
 * blocks: 4 of a layer's blocks (1,024 positions) for 8 KV heads of 128 f16 values */
#define GW_SEQ_CHUNK ((size_t)2 << 20)
static int seq_lazy = 1; /* gw_seq_lazy */

int gw_seq_lazy(int on) {
    int prev = seq_lazy;
    if (on >= 0) seq_lazy = on ? 1 : 0;
    return prev;
}

/* a layer's chunks that hold positions 0 .. n - 1 (whole 256-position blocks: the attention kernels read whole
 * blocks) */
static int seq_chunks(const RqSeq *s, int n, int kv) {
    size_t nb = ((size_t)(n < 0 ? 0 : n) + GW_ATT_P - 1) / GW_ATT_P;
    size_t bytes = nb * (GW_ATT_P / GW_ATT_T) * s->m->n_kv_heads * gw_kv_tile_bytes(s->kvt, s->m->head_dim, kv);
    return (int)((bytes + s->vm_chunk - 1) / s->vm_chunk);
}

static void vm_props(const RqSeq *s, hipMemAllocationProp *prop, hipMemAccessDesc *acc) {
    memset(prop, 0, sizeof(*prop));
    prop->type = hipMemAllocationTypePinned;
    prop->requestedHandleType = hipMemHandleTypeNone;
    prop->location.type = hipMemLocationTypeDevice;
    prop->location.id = s->m->device;
    if (acc) {
        memset(acc, 0, sizeof(*acc));
        acc->location = prop->location;
        acc->flags = hipMemAccessFlagsProtReadWrite;
    }
}

/* unmap and free chunks [from, to) of layer l's half kv (the ones mapped) */
static void vm_unmap(RqSeq *s, int kv, int l, int from, int to) {
    uint8_t *base = (uint8_t *)(kv ? s->vc : s->kc) + (size_t)l * s->lstride[kv];
    hipMemGenericAllocationHandle_t *h = s->vm_h[kv] + (size_t)l * s->vm_max[kv];
    for (int i = to - 1; i >= from; i--)
        if (h[i]) {
            (void)hipMemUnmap(base + (size_t)i * s->vm_chunk, s->vm_chunk);
            (void)hipMemRelease(h[i]);
            h[i] = NULL;
        }
}

int gw_seq_map(RqSeq *s, int n) {
    if (!s->vmm) return RQ_OK;
    n = n > s->cap ? s->cap : n;
    hipMemAllocationProp prop;
    hipMemAccessDesc acc;
    vm_props(s, &prop, &acc);
    for (int kv = 0; kv < 2; kv++) {
        int want = seq_chunks(s, n, kv), have = s->vm_n[kv];
        if (want <= have) continue;
        for (int l = 0; l < s->m->n_layers; l++) {
            uint8_t *base = (uint8_t *)(kv ? s->vc : s->kc) + (size_t)l * s->lstride[kv];
            hipMemGenericAllocationHandle_t *h = s->vm_h[kv] + (size_t)l * s->vm_max[kv];
            for (int i = have; i < want; i++) {
                void *a = base + (size_t)i * s->vm_chunk;
                if (hipMemCreate(&h[i], s->vm_chunk, &prop, 0) != hipSuccess) {
                    h[i] = NULL;
                    goto fail;
                }
                if (hipMemMap(a, s->vm_chunk, 0, h[i], 0) != hipSuccess) {
                    (void)hipMemRelease(h[i]);
                    h[i] = NULL;
                    goto fail;
                }
                if (hipMemSetAccess(a, s->vm_chunk, &acc, 1) != hipSuccess) {
                    (void)hipMemUnmap(a, s->vm_chunk);
                    (void)hipMemRelease(h[i]);
                    h[i] = NULL;
                    goto fail;
                }
            }
            continue;
        fail: /* (this half back to what it was: the chunks mapped by this call go) */
            for (int j = 0; j <= l; j++) vm_unmap(s, kv, j, have, want);
            (void)hipGetLastError();
            return RQ_ERR_NOMEM;
        }
        s->vm_n[kv] = want;
    }
    return RQ_OK;
}

size_t gw_seq_device_bytes(const RqSeq *s) {
    if (!s) return 0;
    if (!s->vmm) return (size_t)s->m->n_layers * (seq_layer_bytes(s, 0) + seq_layer_bytes(s, 1));
    return (size_t)s->m->n_layers * ((size_t)s->vm_n[0] + (size_t)s->vm_n[1]) * s->vm_chunk;
}

static int seq_reserve(RqSeq *s) {
    /* the lazy layout: each half's address range (layer strides in whole chunks), nothing mapped; 1 where the device
     * has no virtual memory management (the caller allocates whole), else RQ_OK / RQ_ERR_NOMEM */
    const RqModel *m = s->m;
    int ok = 0;
    size_t g = 0;
    hipMemAllocationProp prop;
    vm_props(s, &prop, NULL);
    if (hipDeviceGetAttribute(&ok, hipDeviceAttributeVirtualMemoryManagementSupported, m->device) != hipSuccess || !ok ||
        (hipMemGetAllocationGranularity(&g, &prop, hipMemAllocationGranularityRecommended) != hipSuccess &&
         hipMemGetAllocationGranularity(&g, &prop, hipMemAllocationGranularityMinimum) != hipSuccess) || !g) {
        (void)hipGetLastError();
        return 1;
    }
    s->vm_chunk = (GW_SEQ_CHUNK + g - 1) / g * g;
    s->vmm = 1;
    for (int kv = 0; kv < 2; kv++) {
        s->lstride[kv] = (seq_layer_bytes(s, kv) + s->vm_chunk - 1) / s->vm_chunk * s->vm_chunk;
        s->vm_max[kv] = (int)(s->lstride[kv] / s->vm_chunk);
        s->vm_h[kv] = calloc((size_t)m->n_layers * s->vm_max[kv], sizeof(hipMemGenericAllocationHandle_t));
        void *base = NULL;
        if (!s->vm_h[kv]) return RQ_ERR_NOMEM;
        if (hipMemAddressReserve(&base, (size_t)m->n_layers * s->lstride[kv], s->vm_chunk, NULL, 0) != hipSuccess) {
            (void)hipGetLastError();
            return RQ_ERR_NOMEM;
        }
        if (kv) s->vc = base;
        else s->kc = base;
    }
    return RQ_OK;
}

RqSeq *rq_seq_new(const RqModel *m, int capacity, int kv_type, int *err) {
    int e = RQ_OK;
    RqSeq *s = NULL;
    if (!m || !m->has_weights) { e = RQ_ERR_STATE; goto fail; } /* (forward.c:641: a tokenizer-only model) */
    if (capacity <= 0) capacity = m->seq_len;
    /* f16 and bf16 caches (the fp32 attention on the exactly converted values, runq.h:204-213); f32, the rotated q8 / q4
     * ones and the dot-product types with head_dim a power of two, 32 .. 128 */
    int hd = m->head_dim, qok = hd >= 32 && hd <= 128 && !(hd & (hd - 1));
    if (capacity > m->seq_len || !gw_kv_ok(kv_type) || (gw_kv_att_q(kv_type) && !qok)) {
        e = RQ_ERR_ARG;
        goto fail;
    }
    s = calloc(1, sizeof(RqSeq));
    if (!s) { e = RQ_ERR_NOMEM; goto fail; }
    s->m = m;
    s->kvt = kv_type;
    s->cap = capacity;
    s->kv_len = (capacity + GW_ATT_P - 1) / GW_ATT_P * GW_ATT_P;
    s->att_nb = s->kv_len / GW_ATT_P;
    s->nck = 2;   /* (RQ_SEQ_CK, internal.h:66) */
    s->hpos = -1; /* (not an MTP view's sequence) */
    if ((e = seq_lazy ? seq_reserve(s) : 1) < 0) goto fail;
    if (e > 0) { /* (whole: one allocation per half) */
        e = RQ_OK;
        s->vmm = 0;
        s->lstride[0] = seq_layer_bytes(s, 0);
        s->lstride[1] = seq_layer_bytes(s, 1);
        if (hipMalloc((void **)&s->kc, (size_t)m->n_layers * s->lstride[0]) != hipSuccess ||
            hipMalloc((void **)&s->vc, (size_t)m->n_layers * s->lstride[1]) != hipSuccess) {
            e = RQ_ERR_NOMEM;
            goto fail;
        }
    }
    s->tokens = malloc((size_t)capacity * sizeof(int));
    if (!s->tokens) { e = RQ_ERR_NOMEM; goto fail; }
    if (err) *err = RQ_OK;
    return s;
fail:
    rq_seq_free(s);
    if (err) *err = e;
    return NULL;
}

void rq_seq_free(RqSeq *s) {
    if (!s) return;
    if (s->vmm) {
        if (s->vm_n[0] || s->vm_n[1]) (void)hipDeviceSynchronize(); /* (no pass may still read what goes) */
        for (int kv = 0; kv < 2; kv++) {
            if (s->vm_h[kv])
                for (int l = 0; l < s->m->n_layers; l++) vm_unmap(s, kv, l, 0, s->vm_max[kv]);
            void *base = kv ? (void *)s->vc : (void *)s->kc;
            if (base) (void)hipMemAddressFree(base, (size_t)s->m->n_layers * s->lstride[kv]);
            free(s->vm_h[kv]);
        }
    } else {
        if (s->kc) hipFree(s->kc);
        if (s->vc) hipFree(s->vc);
    }
    free(s->tokens);
    free(s);
}

/* the length grows to n (the high-water mark with it: internal.h:400-411's seq_grow) */
static void seq_grow(RqSeq *s, int n) {
    if (n > s->hwm) s->hwm = n;
    s->len = n;
}

/* an MTP view's rows past n are gone (internal.h:383-393: hvalid = min(hvalid, n), hpos past n - 1 -> -1) */
static void seq_cut_view_state(RqSeq *s, int n) {
    if (s->hvalid > n) s->hvalid = n;
    if (s->hpos > n - 1) s->hpos = -1;
}

void rq_seq_reset(RqSeq *s) {
    s->len = 0;
    seq_cut_view_state(s, 0);
}

int rq_seq_truncate(RqSeq *s, int n) {
    if (n < 0 || n > s->len) return RQ_ERR_ARG;
    s->len = n;
    seq_cut_view_state(s, n);
    return RQ_OK;
}

int rq_seq_keep(const RqSeq *s, int n) { return n < 0 || n > s->len ? RQ_ERR_ARG : n; }
int rq_seq_checkpoint_at(RqSeq *s, int pos) { (void)s; (void)pos; return RQ_OK; }
int rq_seq_checkpoint_rows(RqSeq *s, int pos, int n) { (void)s; (void)pos; (void)n; return RQ_OK; }
void rq_seq_checkpoint_rows_drop(RqSeq *s) { (void)s; }
int rq_seq_set_checkpoints(RqSeq *s, int n) {
    /* runq.h:250-252 (forward.c:360-373): the slot count is kept (spec.c reads and restores it); a Qwen3 sequence holds
     * no checkpoint in them */
    if (n < 1 || n > RQ_CHECKPOINTS_MAX) return RQ_ERR_ARG;
    s->nck = n;
    return RQ_OK;
}
int rq_seq_checkpoints(const RqSeq *s, int *pos, int max) { (void)s; (void)pos; (void)max; return 0; }
int rq_seq_len(const RqSeq *s) { return s->len; }
int rq_seq_capacity(const RqSeq *s) { return s->cap; }
const int *rq_seq_tokens(const RqSeq *s) { return s->tokens; }
void rq_seq_seed(RqSeq *s, unsigned long long seed) { s->rng = seed; }
unsigned long long *rq_seq_rng(RqSeq *s) { return &s->rng; }

int rq_seq_common_prefix(const RqSeq *s, const int *tokens, int n) {
    int L = 0;
    while (L < s->len && L < n && s->tokens[L] == tokens[L]) L++;
    return L;
}

int rq_seq_release(RqSeq *s, int keep) {
    /* forward.c:474-510: the memory past max(keep, len) (capped at the capacity) goes, the high-water mark drops to it.
     * A lazy sequence unmaps its chunks past that position's whole blocks; one allocated whole keeps its memory */
    if (!s || keep < 0) return RQ_ERR_ARG;
    int k = keep > s->len ? keep : s->len;
    k = k > s->cap ? s->cap : k;
    if (s->vmm && (seq_chunks(s, k, 0) < s->vm_n[0] || seq_chunks(s, k, 1) < s->vm_n[1])) {
        (void)hipDeviceSynchronize(); /* (no pass may still read what goes) */
        for (int kv = 0; kv < 2; kv++) {
            int w = seq_chunks(s, k, kv);
            if (w >= s->vm_n[kv]) continue;
            for (int l = 0; l < s->m->n_layers; l++) vm_unmap(s, kv, l, w, s->vm_n[kv]);
            s->vm_n[kv] = w;
        }
    }
    if (k < s->hwm) s->hwm = k;
    return RQ_OK;
}

/* Qwen3.5's checkpoints: a Qwen3 sequence holds none (runq.h:257-259) */
int rq_seq_checkpoint_drop(RqSeq *s, int pos) { (void)s; (void)pos; return RQ_ERR_ARG; }

void rq_seq_resident(const RqSeq *s, RqSeqMem *out) {
    /* runq.h:271-274 (forward.c:455-462): kv = rq_seq_kv_bytes up to the high-water mark. A lazy sequence's device
     * memory is that within a chunk per layer and half (gw_seq_device_bytes); one allocated whole holds its capacity */
    memset(out, 0, sizeof(*out));
    if (!s) return;
    out->kv = rq_seq_kv_bytes(s, s->vmm ? s->hwm : s->cap);
    out->total = out->kv;
}

size_t rq_seq_kv_bytes(const RqSeq *s, int n) {
    n = n < 0 ? 0 : n > s->cap ? s->cap : n;
    size_t nb = ((size_t)n + GW_ATT_P - 1) / GW_ATT_P, hd = (size_t)s->m->head_dim;
    return (size_t)s->m->n_layers * nb * (GW_ATT_P / GW_ATT_T) * s->m->n_kv_heads *
               (gw_kv_tile_bytes(s->kvt, (int)hd, 0) + gw_kv_tile_bytes(s->kvt, (int)hd, 1)) + (size_t)s->cap * sizeof(int);
}

int rq_seq_copy(RqSeq *dst, const RqSeq *src, int n) {
    /* forward.c:553-576: dst := the first n positions of src (whole blocks below n, then the last block's tiles up to
     * position n - 1 per kv head: the tiled layout of forward.c:1894-1899), device to device */
    if (!dst || !src || dst == src || dst->m != src->m || dst->kvt != src->kvt || n < 0 || n > src->len || n > dst->cap)
        return RQ_ERR_ARG;
    const RqModel *m = src->m;
    int nkv = m->n_kv_heads, hd = m->head_dim, full = n / GW_ATT_P, rem = n % GW_ATT_P, tpb = GW_ATT_P / GW_ATT_T;
    size_t ntl = (size_t)(rem + GW_ATT_T - 1) / GW_ATT_T;
    if (gw_seq_map(dst, n) != RQ_OK) return RQ_ERR_NOMEM;
    for (int l = 0; l < m->n_layers && n > 0; l++)
        for (int kv = 0; kv < 2; kv++) {
            const size_t tb = gw_kv_tile_bytes(src->kvt, hd, kv); /* (tiles in order: block, head, tile) */
            const uint8_t *sb = (const uint8_t *)seq_layer(src, l, kv);
            uint8_t *db = (uint8_t *)seq_layer(dst, l, kv);
            if (full && hipMemcpy(db, sb, (size_t)full * tpb * nkv * tb, hipMemcpyDeviceToDevice) != hipSuccess)
                return RQ_ERR_STATE;
            for (int h = 0; h < nkv && rem; h++) {
                size_t o = ((size_t)full * nkv + h) * tpb * tb;
                if (hipMemcpy(db + o, sb + o, ntl * tb, hipMemcpyDeviceToDevice) != hipSuccess) return RQ_ERR_STATE;
            }
        }
    memcpy(dst->tokens, src->tokens, (size_t)n * sizeof(int));
    seq_grow(dst, n);
    dst->hvalid = src->hvalid;
    dst->hpos = src->hpos;
    seq_cut_view_state(dst, n);
    return RQ_OK;
}

int rq_seq_fill_synthetic(RqSeq *s, int n, unsigned long long seed) {
    /* runq.h:721-726: n positions of pseudo-random K / V (|K| < 4, |V| < 1), arbitrary valid tokens */
    if (!s || n < 1 || n > s->cap) return RQ_ERR_ARG;
    if (gw_seq_map(s, n) != RQ_OK) return RQ_ERR_NOMEM;
    size_t nb = ((size_t)n + GW_ATT_P - 1) / GW_ATT_P, per = nb * GW_ATT_P * s->m->n_kv_heads * s->m->head_dim;
    for (int l = 0; l < s->m->n_layers; l++) {
        unsigned long long sl = seed + (unsigned long long)l * 0x1000193ull;
        int e = gw_kv_quant(s->kvt) || s->kvt == RQ_KV_F32
                    ? gw_k_fill_synthetic_q(seq_layer(s, l, 0), seq_layer(s, l, 1), s->kvt, (int)(nb * GW_ATT_P),
                                            s->m->n_kv_heads, s->m->head_dim, sl, 0)
                    : gw_k_fill_synthetic(seq_layer(s, l, 0), seq_layer(s, l, 1), per, sl, gw_kv_base(s->kvt) == RQ_KV_BF16, 0);
        if (e) return RQ_ERR_STATE;
    }
    if (hipDeviceSynchronize() != hipSuccess) return RQ_ERR_STATE;
    for (int i = 0; i < n; i++) s->tokens[i] = (int)((seed + (unsigned long long)i * 7919u) % (unsigned long long)s->m->vocab);
    seq_grow(s, n);
    seq_cut_view_state(s, n);
    return RQ_OK;
}

/* ----------------------------------------------------------------------------------------- contexts */

static void dfree(void *p) { if (p) hipFree(p); }

void rq_ctx_free(RqCtx *c) {
    if (!c) return;
    void *d[] = { c->x, c->xb, c->qkv, c->hb, c->part, c->logits_d, c->hid_d, c->xq, c->hq, c->xs, c->hs, c->argmax_d, c->argmax_scr, c->meta_d,
                  c->gtok_d, c->gpos_d, c->topk_scr };
    for (size_t i = 0; i < sizeof d / sizeof d[0]; i++) dfree(d[i]);
    if (c->meta_h) hipHostFree(c->meta_h);
    if (c->logits) hipHostFree(c->logits);
    if (c->lg_h) hipHostFree(c->lg_h);
    if (c->g_h) hipHostFree(c->g_h);
    if (c->topk_h) hipHostFree(c->topk_h);
    if (c->ev) {
        for (int i = 0; i < 2048; i++)
            if (c->ev[i]) hipEventDestroy(c->ev[i]);
        free(c->ev);
        free(c->ev_class);
    }
    if (c->kt_ev) {
        if (c->kt_n) hipStreamSynchronize(c->stream);
        for (int i = 0; i < 2 * GW_KT_MAX; i++)
            if (c->kt_ev[i]) hipEventDestroy(c->kt_ev[i]);
        free(c->kt_ev);
        free(c->kt_cls);
    }
    if (c->stream) hipStreamDestroy(c->stream);
    free(c->smp);
    free(c->smp_t);
    free(c);
}

static int ctx_part(RqCtx *c, int rows, int nb) {
    /* the attention partials buffer for rows x n_heads x nb blocks of (head_dim + 2) floats */
    const RqModel *m = c->m;
    size_t need = (size_t)rows * m->n_heads * nb * (m->head_dim + 2) * sizeof(float);
    if (nb > c->att_nb || need > c->part_bytes) {
        int nbn = nb > c->att_nb ? nb : c->att_nb;
        /* the combine kernel keeps the coefficient and l of every block of its wave's heads in LDS */
        if ((size_t)(m->head_dim < 64 ? 64 / m->head_dim : 1) * 2 * (size_t)nbn * sizeof(float) > 65536)
            return ctx_fail(c, RQ_ERR_ARG, "context of %d positions too long for %d heads (attention combine)",
                            nbn * GW_ATT_P, m->n_heads);
        int B = c->nb_max > 1 ? c->nb_max : 1;
        size_t bytes = (size_t)B * m->n_heads * nbn * (m->head_dim + 2) * sizeof(float);
        HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));
        dfree(c->part);
        c->part = NULL;
        HIPCHK(c, "hipMalloc (attention partials)", hipMalloc((void **)&c->part, bytes));
        c->part_bytes = bytes;
        c->att_nb = nbn;
    }
    c->pstride = c->att_nb * (m->head_dim + 2);
    return RQ_OK;
}

static int ctx_meta(RqCtx *c, size_t bytes) {
    if (bytes <= c->meta_bytes) return RQ_OK;
    HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));
    dfree(c->meta_d);
    if (c->meta_h) hipHostFree(c->meta_h);
    c->meta_d = c->meta_h = NULL;
    c->meta_bytes = 0;
    size_t nb = bytes * 2;
    HIPCHK(c, "hipMalloc (pass metadata)", hipMalloc(&c->meta_d, nb));
    HIPCHK(c, "hipHostMalloc (pass metadata)", hipHostMalloc(&c->meta_h, nb, hipHostMallocDefault));
    c->meta_bytes = nb;
    return RQ_OK;
}

static int ctx_lg(RqCtx *c, size_t rows) {
    if (rows <= c->lg_h_rows) return RQ_OK;
    if (c->lg_h) hipHostFree(c->lg_h);
    if (c->g_h) hipHostFree(c->g_h);
    c->lg_h = NULL;
    c->lg_h_rows = 0;
    HIPCHK(c, "hipHostMalloc (logits)", hipHostMalloc((void **)&c->lg_h, rows * c->m->vocab * sizeof(float), hipHostMallocDefault));
    c->lg_h_rows = rows;
    return RQ_OK;
}

static size_t ctx_bytes(const RqModel *m, int B, int max_ctx) {
    /* what rq_ctx_new allocates for B rows and max_ctx positions (device buffers, the attention partials, the host
     * logits row) */
    size_t dim = m->dim, H = m->hidden, qd = (size_t)m->n_heads * m->head_dim, kvd = (size_t)m->n_kv_heads * m->head_dim;
    size_t kmax = dim > qd ? dim : qd;
    kmax = H > kmax ? H : kmax;
    size_t row = dim * 4 * 3 + (qd + 2 * kvd) * 4 + 2 * H * 4 + kmax + kmax / 32 * 4 + H + H / 32 * 4 + (size_t)m->vocab * 4 + 4 + 512;
    size_t nb = ((size_t)max_ctx + GW_ATT_P - 1) / GW_ATT_P;
    return (size_t)B * row + (size_t)B * m->n_heads * nb * (m->head_dim + 2) * 4 + (size_t)m->vocab * 4;
}

int rq_seq_mem(const RqModel *m, int capacity, int kv_type, RqSeqMem *mem) {
    /* model.c:765-772: one sequence's memory at its capacity (RQ_ERR_ARG as rq_seq_new): the K / V halves in device
     * memory (whole 256-position blocks) and the token array; no recurrent state (Qwen3). A lazy sequence maps it as
     * it grows, so this is its bound */
    memset(mem, 0, sizeof(*mem));
    if (!m || !m->has_weights) return RQ_ERR_STATE;
    if (capacity <= 0) capacity = m->seq_len;
    int hd = m->head_dim, qok = hd >= 32 && hd <= 128 && !(hd & (hd - 1));
    if (capacity > m->seq_len || !gw_kv_ok(kv_type) || (gw_kv_att_q(kv_type) && !qok))
        return RQ_ERR_ARG;
    size_t kv_len = ((size_t)capacity + GW_ATT_P - 1) / GW_ATT_P * GW_ATT_P;
    mem->kv = (size_t)m->n_layers * kv_len / GW_ATT_T * m->n_kv_heads *
                  (gw_kv_tile_bytes(kv_type, hd, 0) + gw_kv_tile_bytes(kv_type, hd, 1)) + (size_t)capacity * sizeof(int);
    mem->total = mem->kv;
    return RQ_OK;
}

int rq_model_mem(const RqModel *m, RqModelMem *mem) {
    /* model.c:758-763 over this library's memory: weights = the device copies of the matrices, norms and tables of the
     * model; runtime = a context of RQ_BATCH_MAX rows at the model's context length plus the exactness tables each
     * device holds (288 MiB); seq = one sequence of that length. No budget is checked (budget 0, budget_src 0); a
     * one-row pass reads every weight (read = weights) */
    memset(mem, 0, sizeof(*mem));
    if (!m || !m->has_weights) return RQ_ERR_STATE;
    mem->weights = m->dev_bytes;
    mem->runtime = ctx_bytes(m, RQ_BATCH_MAX, m->seq_len) + ((size_t)288 << 20);
    rq_seq_mem(m, m->seq_len, RQ_KV_F16, &mem->seq);
    mem->total = mem->weights + mem->runtime + mem->seq.total;
    mem->read = mem->weights;
    return RQ_OK;
}

int rq_pass_times(const RqModel *m, int reps, double *t1, double *t4) {
    /* runq.h:196-199: a decode step and a 4-row pass with every row's logits at position 32 (rq_seq_fill_synthetic),
     * the fastest of reps each after a warm-up, seconds; its own context and sequence */
    if (!m || reps < 1 || !t1 || !t4) return RQ_ERR_ARG;
    if (!m->has_weights) return RQ_ERR_STATE;
    int e = RQ_OK;
    RqCtx *c = rq_ctx_new(m, 4, 64, &e);
    if (!c) return e;
    RqSeq *s = rq_seq_new(m, 64, RQ_KV_F16, &e);
    float *out = malloc((size_t)4 * m->vocab * sizeof(float));
    if (!s || !out) e = e != RQ_OK ? e : RQ_ERR_NOMEM;
    const int toks[4] = { 1, 2, 3, 4 };
    double b1 = 1e30, b4 = 1e30;
    for (int r = -1; r < reps && e == RQ_OK; r++) { /* (r = -1: the warm-up) */
        float *lg = NULL;
        if ((e = rq_seq_fill_synthetic(s, 32, 1)) != RQ_OK) break;
        double t = rq_now();
        if ((e = rq_decode(c, s, 1, &lg)) != RQ_OK) break;
        t = rq_now() - t;
        if (r >= 0 && t < b1) b1 = t;
        if ((e = rq_seq_fill_synthetic(s, 32, 1)) != RQ_OK) break;
        t = rq_now();
        if ((e = rq_prefill(c, s, toks, 4, RQ_LOGITS_ALL, out, NULL)) != RQ_OK) break;
        t = rq_now() - t;
        if (r >= 0 && t < b4) b4 = t;
    }
    free(out);
    rq_seq_free(s);
    rq_ctx_free(c);
    if (e == RQ_OK) *t1 = b1, *t4 = b4;
    return e;
}

RqCtx *rq_ctx_new(const RqModel *m, int nb_max, int max_ctx, int *err) {
    int e = RQ_ERR_NOMEM;
    RqCtx *c = NULL;
    if (!m || !m->has_weights) { e = RQ_ERR_STATE; goto fail; } /* (forward.c:152: a tokenizer-only model) */
    c = calloc(1, sizeof(RqCtx));
    if (!c) goto fail;
    c->m = m;
    c->nb_max = nb_max < 0 ? 0 : nb_max > RQ_BATCH_MAX ? RQ_BATCH_MAX : nb_max;
    int B = c->nb_max > 1 ? c->nb_max : 1;
    int dim = m->dim, H = m->hidden, qd = m->n_heads * m->head_dim, kvd = m->n_kv_heads * m->head_dim;
    c->kmax = dim > qd ? dim : qd;
    c->kmax = H > c->kmax ? H : c->kmax;
    c->ldqkv = qd + 2 * kvd;
    if (hipStreamCreate(&c->stream) != hipSuccess) { e = RQ_ERR_STATE; goto fail; }
#define DM(p, n) if (hipMalloc((void **)&(p), (size_t)(n)) != hipSuccess) goto fail
    DM(c->x, (size_t)B * dim * 4);
    DM(c->xb, (size_t)B * dim * 4);
    DM(c->qkv, (size_t)B * c->ldqkv * 4);
    DM(c->hb, (size_t)B * 2 * H * 4);
    DM(c->xq, (size_t)B * c->kmax);
    DM(c->xs, (size_t)B * (c->kmax / 32) * 4);
    DM(c->hq, (size_t)B * H);
    DM(c->hs, (size_t)B * (H / 32) * 4);
    DM(c->logits_d, (size_t)B * m->vocab * 4);
    DM(c->hid_d, (size_t)B * dim * 4);
    DM(c->argmax_d, (size_t)B * 4);
    DM(c->argmax_scr, (size_t)B * 512);
#undef DM
    if (hipHostMalloc((void **)&c->logits, (size_t)m->vocab * 4, hipHostMallocDefault) != hipSuccess) goto fail;
    if (max_ctx <= 0 || max_ctx > m->seq_len) max_ctx = m->seq_len;
    if (ctx_part(c, B, (max_ctx + GW_ATT_P - 1) / GW_ATT_P) != RQ_OK) goto fail;
    if (err) *err = RQ_OK;
    return c;
fail:
    rq_ctx_free(c);
    if (err) *err = e;
    return NULL;
}

/* the accessors the reference's sampler.c links against (internal.h:326-328, forward.c:772-784): its host scratch
 * (vocab x 8 bytes, and nt such rows for rq_sample_batch) and the vocabulary size */
void *ctx_sampler_scratch(RqCtx *c) {
    if (!c->smp) c->smp = malloc((size_t)c->m->vocab * 8);
    return c->smp;
}

void *ctx_sampler_scratch_threads(RqCtx *c, int nt) {
    if (nt > c->smp_nt) {
        void *p = malloc((size_t)nt * c->m->vocab * 8);
        if (!p) return NULL;
        free(c->smp_t);
        c->smp_t = p;
        c->smp_nt = nt;
    }
    return c->smp_t;
}

int ctx_vocab(const RqCtx *c) { return c->m->vocab; }

int rq_ctx_max_batch(const RqCtx *c) { return c->nb_max; }
const char *rq_ctx_error(const RqCtx *c) { return c->err; }
void *gw_ctx_stream(RqCtx *c) { return c->stream; }

/* ---------------------------------------------------------------------------------------- profiling */

static const char *pf_name[GW_PF_N] = { "embed", "rmsnorm+quant", "matmul qkv", "qk-norm+rope+kv", "attention", "combine+quant",
                                        "matmul wo", "matmul w1+w3", "swiglu+quant", "matmul w2", "classifier" };
#define GW_EV_MAX 2048

int gw_ctx_profile_enable(RqCtx *c, int on) {
    if (on && !c->ev) {
        c->ev = calloc(GW_EV_MAX, sizeof(hipEvent_t));
        c->ev_class = calloc(GW_EV_MAX, sizeof(int));
        if (!c->ev || !c->ev_class) return ctx_fail(c, RQ_ERR_NOMEM, "malloc failed");
        for (int i = 0; i < GW_EV_MAX; i++)
            if (hipEventCreate(&c->ev[i]) != hipSuccess) return ctx_fail(c, RQ_ERR_STATE, "hipEventCreate failed");
    }
    c->prof_on = on;
    memset(c->prof_s, 0, sizeof c->prof_s);
    memset(c->prof_n, 0, sizeof c->prof_n);
    return RQ_OK;
}

int rq_ctx_profile(const RqCtx *c, const char **names, double *seconds, int max) {
    /* runq.h:336-338: device time per kernel class, summed over the passes since gw_ctx_profile_enable */
    if (!c->ev) return 0;
    int n = max < GW_PF_N ? max : GW_PF_N;
    for (int i = 0; i < n; i++) {
        names[i] = pf_name[i];
        seconds[i] = c->prof_s[i];
    }
    return n;
}

long gw_ctx_profile_launches(const RqCtx *c, int cls) { return cls >= 0 && cls < GW_PF_N ? c->prof_n[cls] : 0; }

static void kt_next(RqCtx *c, int cls);

static void pf_mark(RqCtx *c, int cls) {
    /* before the kernel(s) of class cls (cls -1: the end mark): a marker event (profiling), the timing pair of the next
     * launch (kernel timing) */
    c->kt_cur = cls;
    if (cls >= 0) kt_next(c, cls);
    if (!c->prof_on || c->nev >= GW_EV_MAX) return;
    hipEventRecord(c->ev[c->nev], c->stream);
    c->ev_class[c->nev++] = cls;
}

static void pf_collect(RqCtx *c) {
    /* after the pass's synchronization: each interval to the class of the kernel it started with */
    for (int i = 0; i + 1 < c->nev; i++) {
        float ms = 0;
        if (c->ev_class[i] >= 0 && hipEventElapsedTime(&ms, c->ev[i], c->ev[i + 1]) == hipSuccess) {
            c->prof_s[c->ev_class[i]] += ms * 1e-3;
            c->prof_n[c->ev_class[i]]++;
        }
    }
    c->nev = 0;
}

/* kernel timing: the matmuls' own start / stop timestamps (hipExtLaunchKernel events), no markers between kernels */

static int kt_collect(RqCtx *c) {
    if (!c->kt_n) return RQ_OK;
    HIPCHK(c, "hipStreamSynchronize (kernel timing)", hipStreamSynchronize(c->stream));
    for (int i = 0; i < c->kt_n; i++) {
        float ms = 0;
        if (hipEventElapsedTime(&ms, c->kt_ev[2 * i], c->kt_ev[2 * i + 1]) == hipSuccess) {
            c->kt_s[c->kt_cls[i]] += ms * 1e-3;
            c->kt_cnt[c->kt_cls[i]]++;
        }
    }
    c->kt_n = 0;
    return RQ_OK;
}

static void kt_next(RqCtx *c, int cls) {
    /* the next matmul launch (of class cls) is timed */
    if (!c->kt_on) return;
    if (c->kt_n == GW_KT_MAX && kt_collect(c) != RQ_OK) return;
    gw_time_next_launch(c->kt_ev[2 * c->kt_n], c->kt_ev[2 * c->kt_n + 1]);
    c->kt_cls[c->kt_n++] = (unsigned char)(cls + 16 * c->kt_multi);
}

int gw_ctx_kernel_timing(RqCtx *c, int on) {
    if (on && !c->kt_ev) {
        c->kt_ev = calloc(2 * GW_KT_MAX, sizeof(hipEvent_t));
        c->kt_cls = calloc(GW_KT_MAX, 1);
        if (!c->kt_ev || !c->kt_cls) return ctx_fail(c, RQ_ERR_NOMEM, "malloc failed");
        for (int i = 0; i < 2 * GW_KT_MAX; i++)
            HIPCHK(c, "hipEventCreate", hipEventCreate(&c->kt_ev[i]));
    }
    int rc = kt_collect(c);
    c->kt_on = on;
    memset(c->kt_s, 0, sizeof c->kt_s);
    memset(c->kt_cnt, 0, sizeof c->kt_cnt);
    return rc;
}

int gw_ctx_kernel_times(RqCtx *c, int multi, const char **names, double *seconds, long *launches, int max) {
    if (multi < 0 || multi > 1) return ctx_fail(c, RQ_ERR_ARG, "multi %d", multi);
    if (kt_collect(c) != RQ_OK) return RQ_ERR_STATE;
    int n = max < GW_PF_N ? max : GW_PF_N;
    for (int i = 0; i < n; i++) {
        if (names) names[i] = pf_name[i];
        if (seconds) seconds[i] = c->kt_s[16 * multi + i];
        if (launches) launches[i] = c->kt_cnt[16 * multi + i];
    }
    return n;
}

/* ------------------------------------------------------------------------------------------- passes */

static int fused_shape(const RqModel *m) {
    /* an all-Q8_0 model whose matrices fit the fused single-row GEMVs of gw_gemv.hip */
    int dim = m->dim, H = m->hidden, q = m->n_heads * m->head_dim;
    return !m->kq && dim <= 4096 && H <= 12288 && q <= 4096 && dim % 64 == 0 && H % 64 == 0 && q % 64 == 0;
}

typedef struct { int x, y, z, w; } Item; /* attention work item: first row, rows, kv head, key block */

typedef struct {
    int n, nsel, want_hidden;
    int tok[GW_RMAX], pos[GW_RMAX], sel[GW_RMAX];
    RqSeq *seq[GW_RMAX];
    float *hid[GW_RMAX];     /* per row: where its hidden state goes, or NULL */
} Pass;

static int run_mm(RqCtx *c, const GwMat *w, int nmat, const int8_t *xq, const float *xs, int ldx, int M, float *out, int ldo,
                  int mode) {
    /* the matrices side by side in out's columns; two neighbours of one K-quant type share a launch where the kernel
     * allows (gw_k_matmul2) */
    for (int i = 0, col = 0; i < nmat;) {
        if (i) kt_next(c, c->kt_cur); /* (the first launch's pair is set by the class mark) */
        int two = i + 1 < nmat, e = -1;
        if (two) e = gw_k_matmul2(&w[i], &w[i + 1], w[i].rows, xq, xs, ldx, M, out + col, ldo, mode, c->stream);
        if (e == -1) {
            two = 0;
            e = gw_k_matmul(&w[i], xq, xs, ldx, M, out + col, ldo, mode, c->stream);
        }
        if (e) return ctx_fail(c, RQ_ERR_STATE, "matmul launch failed (%d x %d, type %d)", w[i].rows, w[i].cols, w[i].type);
        col += w[i].rows + (two ? w[i + 1].rows : 0);
        i += two ? 2 : 1;
    }
    return RQ_OK;
}

#define KCHK(x) do { if (x) return ctx_fail(c, RQ_ERR_STATE, "kernel launch failed: %s", #x); } while (0)

static int fused_layer(RqCtx *c, int l, RqSeq *sq, int pos, const int *pos_d) {
    /* layer l of the one-row pass of an all-Q8_0 model (the fused decode sequence, x in place): qkv GEMV (rmsnorm +
     * quantize prologue) -> attention (QK-norm, RoPE, K / V store inside) -> wo GEMV (combine prologue, + residual) ->
     * w1 / w3 GEMV (rmsnorm prologue, SwiGLU epilogue) -> w2 GEMV (+ residual). pos: the row's position (pos_d: the
     * same on the device, for the combine kernel past GW_GV_NBMAX key blocks) */
    const RqModel *m = c->m;
    const GwLayer *y = &m->layer[l];
    hipStream_t s = c->stream;
    int nh = m->n_heads, hd = m->head_dim, nb = pos / GW_ATT_P + 1;
    /* (the matmul after w2: the next layer's qkv, or after the last layer the classifier) */
    const GwMat *nx = l + 1 < m->n_layers ? &m->layer[l + 1].qkv[0] : &m->cls;
    const int nxr = l + 1 < m->n_layers ? GW_GV_R_QKV : GW_GV_R_CLS;
    pf_mark(c, GW_PF_QKV);
    KCHK(gw_k_gemv1_norm(&y->qkv[0], GW_GV_R_QKV, c->x, y->att_norm, c->qkv, 0, 0, &y->wo, GW_GV_R_WO, s));
    pf_mark(c, GW_PF_ATT);
    KCHK(gw_k_attn_decode(c->qkv, nh, m->n_kv_heads, hd, m->att_scale, y->q_norm, y->k_norm, m->rope, pos,
                          seq_layer(sq, l, 0), seq_layer(sq, l, 1), c->part,
                          c->pstride, sq->kvt == RQ_KV_BF16, s));
    if (nb <= GW_GV_NBMAX) {
        pf_mark(c, GW_PF_WO);
        KCHK(gw_k_gemv1_combine(&y->wo, GW_GV_R_WO, c->part, c->pstride, hd, nb, c->x, 1, &y->w13[0], GW_GV_R_W13, s));
    } else {
        pf_mark(c, GW_PF_COMBINE);
        KCHK(gw_k_attn_combine_quant(c->part, c->pstride, nh, hd, pos_d, 1, nb, c->xq, c->xs, c->kmax, NULL, s));
        pf_mark(c, GW_PF_WO);
        KCHK(gw_k_gemv1_q(&y->wo, GW_GV_R_WO, c->xq, c->xs, c->x, 1, &y->w13[0], GW_GV_R_W13, s));
    }
    pf_mark(c, GW_PF_W13);
    KCHK(gw_k_gemv1_norm(&y->w13[0], GW_GV_R_W13, c->x, y->ffn_norm, c->hb, 0, y->w13_il, &y->w2, GW_GV_R_W2, s));
    pf_mark(c, GW_PF_W2);
    KCHK(gw_k_gemv1_qf(&y->w2, GW_GV_R_W2, c->hb, c->x, 1, nx, nxr, s));
    return RQ_OK;
}

static int fw_pass(RqCtx *c, Pass *P, float *out) {
    /* the rows of P through the model (every validation done by the caller); out: nsel x vocab logits (host), or
     * NULL with nsel == 0 */
    const RqModel *m = c->m;
    int n = P->n, L = m->n_layers, nh = m->n_heads, nkv = m->n_kv_heads, hd = m->head_dim, dim = m->dim, H = m->hidden;
    int kv_mul = nh / nkv, rb = 16 / kv_mul > 0 ? 16 / kv_mul : 1, rc;
    /* (the items of the caches k_attn_q serves (f32, quantized, dot-product): <= 8 query vectors where one row's fit, so
     * its LDS holds 3 blocks per CU; nqm: its vector bound) */
    int nqm = kv_mul <= 8 ? 8 : 16, rbq = 8 / kv_mul > 0 ? 8 / kv_mul : rb;
#define ROWS_OF(t) (gw_kv_att_q(t) ? rbq : rb)
    /* attention items: row blocks of <= rb (rbq) consecutive rows of one sequence, per kv head and key block */
    int nbmax = 1, nitems = 0;
    for (int b = 0; b < n; b++) {
        int nb = (P->pos[b] + 1 + GW_ATT_P - 1) / GW_ATT_P;
        nbmax = nb > nbmax ? nb : nbmax;
        if ((b + 1 == n || P->seq[b + 1] != P->seq[b]) && gw_seq_map(P->seq[b], P->pos[b] + 1) != RQ_OK)
            return ctx_fail(c, RQ_ERR_NOMEM, "no device memory for the KV cache up to position %d", P->pos[b]);
    }
    if ((rc = ctx_part(c, n, nbmax)) != RQ_OK) return rc;
    for (int b = 0; b < n;) {
        int e = b + 1;
        while (e < n && e - b < ROWS_OF(P->seq[b]->kvt) && P->seq[e] == P->seq[b] && P->pos[e] == P->pos[e - 1] + 1) e++;
        nitems += nkv * ((P->pos[e - 1] + 1 + GW_ATT_P - 1) / GW_ATT_P);
        b = e;
    }
    /* metadata block: tok, pos, sel (int), kc / vc tables per layer (pointers), items */
    size_t o_tok = 0, o_pos = o_tok + (size_t)n * 4, o_sel = o_pos + (size_t)n * 4, o_kbf = o_sel + (size_t)n * 4;
    size_t o_ptr = (o_kbf + (size_t)n * 4 + 15) / 16 * 16;
    size_t o_items = o_ptr + (size_t)2 * L * n * sizeof(void *), total = o_items + (size_t)nitems * sizeof(Item);
    if ((rc = ctx_meta(c, total)) != RQ_OK) return rc;
    HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream)); /* (the pinned block may still feed a copy) */
    uint8_t *h = c->meta_h, *d = c->meta_d;
    memcpy(h + o_tok, P->tok, (size_t)n * 4);
    memcpy(h + o_pos, P->pos, (size_t)n * 4);
    memcpy(h + o_sel, P->sel, (size_t)n * 4);
    /* (each row's cache type; rows of bf16 caches, rows of f32, quantized or dot-product ones (k_attn_q), rows to
     * unrotate) */
    int *kvt = (int *)(h + o_kbf), nbf = 0, nqz = 0, nrot = 0;
    for (int b = 0; b < n; b++) {
        kvt[b] = P->seq[b]->kvt;
        nbf += kvt[b] == RQ_KV_BF16;
        nqz += gw_kv_att_q(kvt[b]);
        nrot += gw_kv_quant(kvt[b]);
    }
    uint16_t **ptr = (uint16_t **)(h + o_ptr);
    for (int l = 0; l < L; l++)
        for (int b = 0; b < n; b++) {
            ptr[(size_t)l * n + b] = seq_layer(P->seq[b], l, 0);
            ptr[(size_t)(L + l) * n + b] = seq_layer(P->seq[b], l, 1);
        }
    /* the items in six groups, each launched with its own query-vector bound: the f16 caches', then the bf16
     * caches'; in each, the row blocks of <= 4 query vectors (decode rows: the narrow kernel, two blocks per CU), then
     * the wider ones (prompt row blocks). A pass of both kinds of rows would otherwise run every decode row's items in
     * the 16-vector kernel. Then the f32 and quantized caches', and the dot-product types' (k_attn_q) */
    Item *it = (Item *)(h + o_items);
    int gcnt[6] = { 0, 0, 0, 0, 0, 0 }, gnq[6] = { 1, 1, 1, 1, 1, 1 };
    for (int grp = 0, k = 0; grp < 6; grp++)
        for (int b = 0; b < n;) {
            int e = b + 1;
            while (e < n && e - b < ROWS_OF(kvt[b]) && P->seq[e] == P->seq[b] && P->pos[e] == P->pos[e - 1] + 1) e++;
            int nb = (P->pos[e - 1] + 1 + GW_ATT_P - 1) / GW_ATT_P, nq = (e - b) * kv_mul;
            int kg = gw_kv_dot(kvt[b]) ? 5 : gw_kv_att_q(kvt[b]) ? 4 : 2 * (kvt[b] == RQ_KV_BF16) + (nq > 4);
            if (kg == grp) {
                for (int g = 0; g < nkv; g++)
                    for (int kb = 0; kb < nb; kb++) it[k++] = (Item){ b, e - b, g, kb };
                gcnt[grp] += nkv * nb;
                gnq[grp] = nq > gnq[grp] ? nq : gnq[grp];
            }
            b = e;
        }
#undef ROWS_OF
    HIPCHK(c, "hipMemcpyAsync (pass metadata)", hipMemcpyAsync(d, h, total, hipMemcpyHostToDevice, c->stream));
    const int *tok_d = (const int *)(d + o_tok), *pos_d = (const int *)(d + o_pos), *sel_d = (const int *)(d + o_sel);
    const int *kvt_d = (const int *)(d + o_kbf);
    uint16_t *const *kc_d = (uint16_t *const *)(d + o_ptr), *const *vc_d = kc_d + (size_t)L * n;
    const void *items_d = d + o_items;
    hipStream_t s = c->stream;
    int K = c->kmax;

    c->nev = 0;
    c->kt_multi = n > 1;
    pf_mark(c, GW_PF_EMBED);
    if (m->embd.type == GW_Q8_0) KCHK(gw_k_embed_q8(c->x, dim, (const uint8_t *)m->embd.codes, m->embd.scales, tok_d, n, s));
    else KCHK(gw_k_embed_kq(c->x, dim, m->embd.type, m->embd.blocks, m->embd.bstride, tok_d, n, s));
    /* one row of an all-Q8_0 model: the fused decode sequence (gw_gemv.hip: each matmul computes its activation from
     * the producer's fp32 output; the residual adds go straight into x) */
    int fused = n == 1 && fused_shape(m) && !nqz, fused_att = fused && (hd == 128 || hd == 64 || hd == 32);
    for (int l = 0; l < L; l++) {
        const GwLayer *y = &m->layer[l];
        if (fused_att) {
            if ((rc = fused_layer(c, l, P->seq[0], P->pos[0], pos_d)) != RQ_OK) return rc;
            continue;
        }
        if (fused) {
            pf_mark(c, GW_PF_QKV);
            KCHK(gw_k_gemv1_norm(&y->qkv[0], GW_GV_R_QKV, c->x, y->att_norm, c->qkv, 0, 0, NULL, 0, s));
        } else {
            pf_mark(c, GW_PF_NORM);
            KCHK(gw_k_rmsnorm_quant(c->x, l ? c->xb : NULL, dim, y->att_norm, NULL, n, c->xq, c->xs, K, NULL, s));
            pf_mark(c, GW_PF_QKV);
            if ((rc = run_mm(c, y->qkv, y->nqkv, c->xq, c->xs, K, n, c->qkv, c->ldqkv, 0)) != RQ_OK) return rc;
        }
        pf_mark(c, GW_PF_ROPE);
        KCHK(gw_k_qknorm_rope_store(c->qkv, c->ldqkv, n, nh, nkv, hd, y->q_norm, y->k_norm, m->rope, pos_d,
                                    kc_d + (size_t)l * n, vc_d + (size_t)l * n, nbf || nqz ? kvt_d : NULL, s));
        pf_mark(c, GW_PF_ATT);
        for (int grp = 0, off = 0; grp < 6; off += gcnt[grp], grp++) {
            if (!gcnt[grp]) continue;
            if (grp >= 4)
                KCHK(gw_k_attn_q((const Item *)items_d + off, gcnt[grp], c->qkv, c->ldqkv, nh, nkv, hd, m->att_scale, pos_d,
                                 kc_d + (size_t)l * n, vc_d + (size_t)l * n, kvt_d, grp == 5, nqm, c->part,
                                 c->pstride, s));
            else
                KCHK(gw_k_attn_part((const Item *)items_d + off, gcnt[grp], gnq[grp], c->qkv, c->ldqkv, nh, nkv, hd,
                                    m->att_scale, pos_d, kc_d + (size_t)l * n, vc_d + (size_t)l * n, c->part, c->pstride,
                                    grp >> 1, s));
        }
        if (fused) {
            if (nbmax <= GW_GV_NBMAX) {
                pf_mark(c, GW_PF_WO);
                KCHK(gw_k_gemv1_combine(&y->wo, GW_GV_R_WO, c->part, c->pstride, hd, nbmax, c->x, 1, NULL, 0, s));
            } else {
                pf_mark(c, GW_PF_COMBINE);
                KCHK(gw_k_attn_combine_quant(c->part, c->pstride, nh, hd, pos_d, n, nbmax, c->xq, c->xs, K, NULL, s));
                pf_mark(c, GW_PF_WO);
                KCHK(gw_k_gemv1_q(&y->wo, GW_GV_R_WO, c->xq, c->xs, c->x, 1, NULL, 0, s));
            }
            pf_mark(c, GW_PF_W13);
            KCHK(gw_k_gemv1_norm(&y->w13[0], GW_GV_R_W13, c->x, y->ffn_norm, c->hb, 0, y->w13_il, NULL, 0, s));
            pf_mark(c, GW_PF_W2);
            KCHK(gw_k_gemv1_qf(&y->w2, GW_GV_R_W2, c->hb, c->x, 1, NULL, 0, s));
            continue;
        }
        pf_mark(c, GW_PF_COMBINE);
        /* (rows of quantized caches: the combined o' into the free qkv buffer, then o = D H o' / hd quantized over theirs) */
        KCHK(gw_k_attn_combine_quant(c->part, c->pstride, nh, hd, pos_d, n, nbmax, c->xq, c->xs, K, nrot ? c->qkv : NULL, s));
        if (nrot) KCHK(gw_k_unrot_quant(c->qkv, n, nh, hd, kvt_d, c->xq, c->xs, K, s));
        pf_mark(c, GW_PF_WO);
        if ((rc = run_mm(c, &y->wo, 1, c->xq, c->xs, K, n, c->xb, dim, 0)) != RQ_OK) return rc;
        pf_mark(c, GW_PF_NORM);
        KCHK(gw_k_rmsnorm_quant(c->x, c->xb, dim, y->ffn_norm, NULL, n, c->xq, c->xs, K, NULL, s));
        pf_mark(c, GW_PF_W13);
        /* (the SwiGLU and its quantization in their own kernel: measured faster than in the GEMM's epilogue, whose table
         * reads wait at the end of each block) */
        if ((rc = run_mm(c, y->w13, y->nw13, c->xq, c->xs, K, n, c->hb, 2 * H, 0)) != RQ_OK) return rc;
        pf_mark(c, GW_PF_SWIGLU);
        KCHK(gw_k_swiglu_quant(c->hb, H, y->w13_il, n, c->hq, c->hs, s));
        pf_mark(c, GW_PF_W2);
        if ((rc = run_mm(c, &y->w2, 1, c->hq, c->hs, H, n, c->xb, dim, 0)) != RQ_OK) return rc;
    }
    int resid_done = fused; /* (the fused sequence leaves no pending residual in xb) */
    if (P->want_hidden) { /* every row's final hidden state (the normed row), then the logits rows below */
        KCHK(gw_k_rmsnorm_quant(c->x, resid_done ? NULL : c->xb, dim, m->final_norm, NULL, n, c->xq, c->xs, K, c->hid_d, s));
        resid_done = 1;
    }
    if (fused && P->nsel == 1 && !P->want_hidden) { /* the final rmsnorm computed by the classifier's GEMV itself */
        pf_mark(c, GW_PF_CLS);
        KCHK(gw_k_gemv1_norm(&m->cls, GW_GV_R_CLS, c->x, m->final_norm, c->logits_d, 0, 0, NULL, 0, s));
    } else if (P->nsel > 0) {
        pf_mark(c, GW_PF_NORM);
        KCHK(gw_k_rmsnorm_quant(c->x, resid_done ? NULL : c->xb, dim, m->final_norm, sel_d, P->nsel, c->xq, c->xs, K, NULL, s));
        pf_mark(c, GW_PF_CLS);
        if ((rc = run_mm(c, &m->cls, 1, c->xq, c->xs, K, P->nsel, c->logits_d, m->vocab, 0)) != RQ_OK) return rc;
    }
    pf_mark(c, -1);
    if (P->want_hidden) {
        HIPCHK(c, "hipStreamSynchronize (pass)", hipStreamSynchronize(s));
        for (int b = 0; b < n; b++)
            if (P->hid[b])
                HIPCHK(c, "hipMemcpy (hidden)", hipMemcpy(P->hid[b], c->hid_d + (size_t)b * dim, (size_t)dim * 4, hipMemcpyDeviceToHost));
    }
    if (P->nsel > 0 && out) {
        size_t bytes = (size_t)P->nsel * m->vocab * 4;
        if (out == c->logits) {
            HIPCHK(c, "hipMemcpyAsync (logits)", hipMemcpyAsync(out, c->logits_d, bytes, hipMemcpyDeviceToHost, s));
            HIPCHK(c, "hipStreamSynchronize (pass)", hipStreamSynchronize(s));
        } else {
            if ((rc = ctx_lg(c, (size_t)P->nsel)) != RQ_OK) return rc;
            HIPCHK(c, "hipMemcpyAsync (logits)", hipMemcpyAsync(c->lg_h, c->logits_d, bytes, hipMemcpyDeviceToHost, s));
            HIPCHK(c, "hipStreamSynchronize (pass)", hipStreamSynchronize(s));
            memcpy(out, c->lg_h, bytes);
        }
    } else {
        HIPCHK(c, "hipStreamSynchronize (pass)", hipStreamSynchronize(s));
    }
    if (c->prof_on) pf_collect(c);
    c->last_nsel = P->nsel;
    return RQ_OK;
}

static int check_seq(RqCtx *c, const RqSeq *s) {
    if (!s) return ctx_fail(c, RQ_ERR_ARG, "no sequence");
    if (s->m != c->m) return ctx_fail(c, RQ_ERR_ARG, "sequence of another model");
    return RQ_OK;
}

static int decode_one(RqCtx *c, RqSeq *s, int token, float *logits, float *hidden) {
    static Pass P; /* (large: not on the stack; one pass at a time per process, as the reference's pool) */
    P.n = 1;
    P.tok[0] = token;
    P.pos[0] = s->len;
    P.seq[0] = s;
    P.sel[0] = 0;
    P.nsel = logits ? 1 : 0;
    P.want_hidden = hidden != NULL;
    P.hid[0] = hidden;
    int rc = fw_pass(c, &P, logits);
    if (rc != RQ_OK) return rc;
    s->tokens[s->len] = token;
    seq_grow(s, s->len + 1);
    return RQ_OK;
}

int rq_decode(RqCtx *c, RqSeq *s, int token, float **logits) {
    c->err[0] = 0;
    int e = check_seq(c, s);
    if (e != RQ_OK) return e;
    if (token < 0 || token >= c->m->vocab) return ctx_fail(c, RQ_ERR_ARG, "token %d out of range", token);
    if (s->len >= s->cap) return ctx_fail(c, RQ_ERR_CONTEXT, "sequence full (%d positions)", s->cap);
    e = decode_one(c, s, token, logits ? c->logits : NULL, NULL);
    if (logits) *logits = e == RQ_OK ? c->logits : NULL;
    return e;
}

int gw_decode_argmax(RqCtx *c, RqSeq *s, int token, int *next) {
    /* rq_decode + the greedy next token on the device (sample_argmax, sampler.c:40-60): the logits stay on the
     * device (gw_ctx_argmax reads them again if wanted) */
    c->err[0] = 0;
    int e = check_seq(c, s);
    if (e != RQ_OK) return e;
    if (!next) return ctx_fail(c, RQ_ERR_ARG, "no output for the token");
    if (token < 0 || token >= c->m->vocab) return ctx_fail(c, RQ_ERR_ARG, "token %d out of range", token);
    if (s->len >= s->cap) return ctx_fail(c, RQ_ERR_CONTEXT, "sequence full (%d positions)", s->cap);
    static Pass P;
    P.n = 1;
    P.tok[0] = token;
    P.pos[0] = s->len;
    P.seq[0] = s;
    P.sel[0] = 0;
    P.nsel = 1;
    P.want_hidden = 0;
    P.hid[0] = NULL;
    if ((e = fw_pass(c, &P, NULL)) != RQ_OK) return e;
    s->tokens[s->len] = token;
    seq_grow(s, s->len + 1);
    return gw_ctx_argmax(c, next, 1);
}

int gw_decode_greedy(RqCtx *c, RqSeq *s, int token, int n, int *tokens) {
    /* n greedy decode steps from token (the generation loop of chat.c:348 with sample_argmax, sampler.c:40-60):
     * tokens[i] = the first maximum of step i's logits, the token step i + 1 is fed. The token of each step stays on the
     * device (the argmax kernel writes it where the next step's embedding reads it), so the n passes are enqueued
     * without waiting for each other and the host waits once. The same kernels and results as n gw_decode_argmax calls;
     * a model outside the fused decode shapes, or a sequence whose cache k_attn_decode does not read (f32, quantized,
     * dot-product: their attention is k_attn_q's), runs exactly those calls */
    c->err[0] = 0;
    int e = check_seq(c, s);
    if (e != RQ_OK) return e;
    const RqModel *m = c->m;
    if (n < 1 || !tokens) return ctx_fail(c, RQ_ERR_ARG, "bad greedy arguments (n %d)", n);
    if (token < 0 || token >= m->vocab) return ctx_fail(c, RQ_ERR_ARG, "token %d out of range", token);
    if (s->len + n > s->cap) return ctx_fail(c, RQ_ERR_CONTEXT, "%d steps at position %d: past the capacity %d", n, s->len, s->cap);
    int hd = m->head_dim;
    if (!(fused_shape(m) && (hd == 128 || hd == 64 || hd == 32)) || gw_kv_att_q(s->kvt)) {
        for (int i = 0; i < n; i++) {
            if ((e = gw_decode_argmax(c, s, i ? tokens[i - 1] : token, &tokens[i])) != RQ_OK) return e;
        }
        return RQ_OK;
    }
    if (n > c->g_cap) {
        HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(c->stream));
        dfree(c->gtok_d);
        dfree(c->gpos_d);
        if (c->g_h) hipHostFree(c->g_h);
        c->gtok_d = c->gpos_d = c->g_h = NULL;
        c->g_cap = 0;
        HIPCHK(c, "hipMalloc (greedy tokens)", hipMalloc((void **)&c->gtok_d, (size_t)(n + 1) * sizeof(int)));
        HIPCHK(c, "hipMalloc (greedy positions)", hipMalloc((void **)&c->gpos_d, (size_t)n * sizeof(int)));
        HIPCHK(c, "hipHostMalloc (greedy staging)", hipHostMalloc((void **)&c->g_h, (size_t)(2 * n + 1) * sizeof(int), 0));
        c->g_cap = n;
    }
    int p0 = s->len;
    if ((e = ctx_part(c, 1, (p0 + n - 1) / GW_ATT_P + 1)) != RQ_OK) return e;
    if (gw_seq_map(s, p0 + n) != RQ_OK)
        return ctx_fail(c, RQ_ERR_NOMEM, "no device memory for the KV cache up to position %d", p0 + n - 1);
    hipStream_t st = c->stream;
    HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(st)); /* (the staging may still be read by a previous call) */
    c->g_h[0] = token;
    for (int i = 0; i < n; i++) c->g_h[1 + i] = p0 + i;
    HIPCHK(c, "hipMemcpyAsync (greedy token)", hipMemcpyAsync(c->gtok_d, c->g_h, sizeof(int), hipMemcpyHostToDevice, st));
    HIPCHK(c, "hipMemcpyAsync (greedy positions)", hipMemcpyAsync(c->gpos_d, c->g_h + 1, (size_t)n * sizeof(int),
                                                                  hipMemcpyHostToDevice, st));
    c->kt_multi = 0;
    for (int i = 0; i < n; i++) {
        c->nev = 0;
        pf_mark(c, GW_PF_EMBED);
        KCHK(gw_k_embed_q8(c->x, m->dim, (const uint8_t *)m->embd.codes, m->embd.scales, c->gtok_d + i, 1, st));
        for (int l = 0; l < m->n_layers; l++)
            if ((e = fused_layer(c, l, s, p0 + i, c->gpos_d + i)) != RQ_OK) return e;
        pf_mark(c, GW_PF_CLS);
        KCHK(gw_k_gemv1_norm(&m->cls, GW_GV_R_CLS, c->x, m->final_norm, c->logits_d, 0, 0, NULL, 0, st));
        pf_mark(c, -1);
        KCHK(gw_k_argmax(c->logits_d, m->vocab, m->vocab, 1, c->gtok_d + i + 1, c->argmax_scr, st));
        if (c->prof_on) { /* (profiling: each pass's intervals, as the passes of fw_pass) */
            HIPCHK(c, "hipStreamSynchronize", hipStreamSynchronize(st));
            pf_collect(c);
        }
    }
    HIPCHK(c, "hipMemcpyAsync (greedy tokens)", hipMemcpyAsync(c->g_h, c->gtok_d + 1, (size_t)n * sizeof(int),
                                                               hipMemcpyDeviceToHost, st));
    HIPCHK(c, "hipStreamSynchronize (greedy)", hipStreamSynchronize(st));
    memcpy(tokens, c->g_h, (size_t)n * sizeof(int));
    for (int i = 0; i < n; i++) s->tokens[p0 + i] = i ? tokens[i - 1] : token;
    seq_grow(s, p0 + n);
    c->last_nsel = 1;
    return RQ_OK;
}

int rq_decode_hidden(RqCtx *c, RqSeq *s, int token, float **logits, float *hidden, const float *h_in) {
    c->err[0] = 0;
    if (logits) *logits = NULL;
    int e = check_seq(c, s);
    if (e != RQ_OK) return e;
    if (h_in) return ctx_fail(c, RQ_ERR_ARG, "h_in on a model that is not an MTP view");
    if (token < 0 || token >= c->m->vocab) return ctx_fail(c, RQ_ERR_ARG, "token %d out of range", token);
    if (s->len >= s->cap) return ctx_fail(c, RQ_ERR_CONTEXT, "sequence full (%d positions)", s->cap);
    e = decode_one(c, s, token, logits ? c->logits : NULL, hidden);
    if (logits && e == RQ_OK) *logits = c->logits;
    return e;
}

static int fw_batch(RqCtx *c, const RqSegment *sg, int nseg, float *out, float **logits, int on_device) {
    /* forward.c:3762-3878's contract: validation first, rows in segment order, selected rows' logits to out in row
     * order (one selected row and out NULL: the context's buffer); on_device: the logits rows stay on the device */
    static Pass P;
    const RqModel *m = c->m;
    int n = 0, nsel = 0, any_all = 0;
    c->err[0] = 0;
    if (logits) *logits = NULL;
    if (c->nb_max <= 1) return ctx_fail(c, RQ_ERR_STATE, "context without batch buffers (max_batch %d)", c->nb_max);
    if (nseg < 1 || nseg > c->nb_max) return ctx_fail(c, RQ_ERR_ARG, "bad segment count %d", nseg);
    for (int i = 0; i < nseg; i++) {
        RqSeq *s = sg[i].seq;
        int e = check_seq(c, s);
        if (e != RQ_OK) return e;
        if (sg[i].n < 1 || n + sg[i].n > c->nb_max || sg[i].logits < RQ_LOGITS_NONE || sg[i].logits > RQ_LOGITS_ALL)
            return ctx_fail(c, RQ_ERR_ARG, "rq_forward_batch: bad segment %d (n %d, %d rows so far, max_batch %d)", i, sg[i].n, n,
                            c->nb_max);
        if (s->len + sg[i].n > s->cap)
            return ctx_fail(c, RQ_ERR_CONTEXT, "rq_forward_batch: %d tokens at position %d past the capacity %d", sg[i].n, s->len,
                            s->cap);
        for (int j = 0; j < i; j++)
            if (sg[j].seq == s) return ctx_fail(c, RQ_ERR_ARG, "sequence in segments %d and %d", j, i);
        for (int j = 0; j < sg[i].n; j++)
            if (sg[i].tokens[j] < 0 || sg[i].tokens[j] >= m->vocab) return ctx_fail(c, RQ_ERR_ARG, "token %d out of range", sg[i].tokens[j]);
        if (sg[i].h_in) return ctx_fail(c, RQ_ERR_ARG, "rq_forward_batch: segment %d: h_in on a model that is not an MTP view", i);
        n += sg[i].n;
        nsel += sg[i].logits == RQ_LOGITS_ALL ? sg[i].n : sg[i].logits == RQ_LOGITS_LAST;
        any_all |= sg[i].logits == RQ_LOGITS_ALL;
    }
    int gemv = nsel == 1 && !any_all && !out;
    if (nsel > 0 && !out && !gemv && !on_device) return ctx_fail(c, RQ_ERR_ARG, "logits of %d rows need an output buffer", nsel);
    if (gemv) out = c->logits;
    if (on_device) out = NULL;
    P.n = n;
    P.nsel = 0;
    P.want_hidden = 0;
    for (int i = 0, b = 0; i < nseg; i++)
        for (int j = 0; j < sg[i].n; j++, b++) {
            P.tok[b] = sg[i].tokens[j];
            P.pos[b] = sg[i].seq->len + j;
            P.seq[b] = sg[i].seq;
            P.hid[b] = sg[i].hidden ? sg[i].hidden + (size_t)j * m->dim : NULL;
            P.want_hidden |= sg[i].hidden != NULL;
            if (sg[i].logits == RQ_LOGITS_ALL || (sg[i].logits == RQ_LOGITS_LAST && j == sg[i].n - 1)) P.sel[P.nsel++] = b;
        }
    int e = fw_pass(c, &P, nsel ? out : NULL);
    if (e != RQ_OK) return e;
    for (int i = 0; i < nseg; i++) {
        RqSeq *s = sg[i].seq;
        memcpy(s->tokens + s->len, sg[i].tokens, (size_t)sg[i].n * sizeof(int));
        seq_grow(s, s->len + sg[i].n);
    }
    if (logits) *logits = nsel ? out : NULL;
    return RQ_OK;
}

int rq_forward_batch(RqCtx *c, const RqSegment *sg, int nseg, float *out, float **logits) {
    return fw_batch(c, sg, nseg, out, logits, 0);
}

int gw_forward_batch_device(RqCtx *c, const RqSegment *sg, int nseg) {
    /* rq_forward_batch with the selected rows' logits left on the device (gw_ctx_argmax chooses their greedy tokens):
     * the batched decode step of a serving loop without the vocab-size copy per row */
    return fw_batch(c, sg, nseg, NULL, NULL, 1);
}

int fw_rows(RqCtx *c, RqSeq *s, const int *tokens, int n, int mode, float *out, float **logits, float *hidden, const float *h_in) {
    /* forward.c:3880-3916: tokens at positions len.. in chunks of max_batch rows, or token by token through the decode
     * path (max_batch <= 1), the same results either way; every row's final hidden state (the normed row, dim floats)
     * into hidden when given. h_in (an MTP view's input rows, Qwen3.5) is refused: no model here is such a view */
    int V = c->m->vocab, dim = c->m->dim, e = check_seq(c, s);
    c->err[0] = 0;
    if (logits) *logits = NULL;
    if (e != RQ_OK) return e;
    if (n < 1 || mode < RQ_LOGITS_NONE || mode > RQ_LOGITS_ALL || (mode == RQ_LOGITS_ALL && !out))
        return ctx_fail(c, RQ_ERR_ARG, "bad prefill arguments (n %d, mode %d)", n, mode);
    if (h_in) return ctx_fail(c, RQ_ERR_ARG, "h_in on a model that is not an MTP view");
    if (s->len + n > s->cap) return ctx_fail(c, RQ_ERR_CONTEXT, "%d tokens at position %d: past the capacity %d", n, s->len, s->cap);
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= V) return ctx_fail(c, RQ_ERR_ARG, "token %d out of range", tokens[i]);
    float *lg = NULL;
    if (c->nb_max <= 1) {
        for (int i = 0; i < n && e == RQ_OK; i++) {
            int want = mode == RQ_LOGITS_ALL || (mode == RQ_LOGITS_LAST && i == n - 1);
            e = decode_one(c, s, tokens[i], want ? c->logits : NULL, hidden ? hidden + (size_t)i * dim : NULL);
            if (mode == RQ_LOGITS_ALL && e == RQ_OK) memcpy(out + (size_t)i * V, c->logits, (size_t)V * sizeof(float));
        }
        lg = mode == RQ_LOGITS_ALL ? out : mode == RQ_LOGITS_LAST ? c->logits : NULL;
    } else {
        int nb = c->nb_max;
        for (int i = 0; i < n && e == RQ_OK; i += nb) {
            int k = n - i < nb ? n - i : nb;
            RqSegment sg = { s, tokens + i, k,
                             mode == RQ_LOGITS_ALL ? RQ_LOGITS_ALL : mode == RQ_LOGITS_LAST && i + k == n ? RQ_LOGITS_LAST : RQ_LOGITS_NONE,
                             hidden ? hidden + (size_t)i * dim : NULL, NULL };
            e = rq_forward_batch(c, &sg, 1, mode == RQ_LOGITS_ALL ? out + (size_t)i * V : NULL, &lg);
        }
        lg = mode == RQ_LOGITS_ALL ? out : lg;
    }
    if (logits && e == RQ_OK) *logits = lg;
    return e;
}

int rq_prefill(RqCtx *c, RqSeq *s, const int *tokens, int n, int mode, float *out, float **logits) {
    return fw_rows(c, s, tokens, n, mode, out, logits, NULL, NULL);
}

int gw_ctx_gemv_sweep(RqCtx *c, int reps, double *seconds, double *bytes, int *launches) {
    /* the weight matmuls of one decode step (every layer's q / k / v, wo, w1 / w3, w2, then the classifier), launched
     * as a one-row pass launches them (an all-Q8_0 model: the fused GEMVs with their prologues and epilogues, the
     * attention combine over one key block), back to back on the context's stream, reps times, between two HIP
     * events: the device time of the decode path's weight streaming without the other kernels between them. The
     * inputs are whatever the context's buffers hold (the kernels' time does not depend on the values); the outputs go
     * to the context's scratch rows. *bytes: the file-format bytes of those weights per sweep (Q8_0 34 / 32, Q4_K
     * 144 / 256, Q6_K 210 / 256 per weight); *launches: kernels per sweep */
    const RqModel *m = c->m;
    if (reps < 1) return ctx_fail(c, RQ_ERR_ARG, "reps %d", reps);
    double b = 0;
    int nl = 0, rc, fused = fused_shape(m);
    hipStream_t s = c->stream;
    hipEvent_t e0, e1;
    HIPCHK(c, "hipEventCreate", hipEventCreate(&e0));
    HIPCHK(c, "hipEventCreate", hipEventCreate(&e1));
    HIPCHK(c, "hipEventRecord", hipEventRecord(e0, s));
    for (int r = 0; r < reps; r++) {
        for (int l = 0; l < m->n_layers; l++) {
            const GwLayer *y = &m->layer[l];
            if (fused) {
                const int last = l + 1 == m->n_layers;
                KCHK(gw_k_gemv1_norm(&y->qkv[0], GW_GV_R_QKV, c->x, y->att_norm, c->qkv, 0, 0, &y->wo, GW_GV_R_WO, s));
                KCHK(gw_k_gemv1_combine(&y->wo, GW_GV_R_WO, c->part, c->pstride, m->head_dim, 1, c->xb, 0, &y->w13[0],
                                        GW_GV_R_W13, s));
                KCHK(gw_k_gemv1_norm(&y->w13[0], GW_GV_R_W13, c->x, y->ffn_norm, c->hb, 0, y->w13_il, &y->w2, GW_GV_R_W2, s));
                KCHK(gw_k_gemv1_qf(&y->w2, GW_GV_R_W2, c->hb, c->xb, 0, last ? &m->cls : &m->layer[l + 1].qkv[0],
                                   last ? GW_GV_R_CLS : GW_GV_R_QKV, s));
                continue;
            }
            if ((rc = run_mm(c, y->qkv, y->nqkv, c->xq, c->xs, c->kmax, 1, c->qkv, c->ldqkv, 0)) != RQ_OK) return rc;
            if ((rc = run_mm(c, &y->wo, 1, c->xq, c->xs, c->kmax, 1, c->xb, m->dim, 0)) != RQ_OK) return rc;
            if ((rc = run_mm(c, y->w13, y->nw13, c->xq, c->xs, c->kmax, 1, c->hb, 2 * m->hidden, 0)) != RQ_OK) return rc;
            if ((rc = run_mm(c, &y->w2, 1, c->hq, c->hs, m->hidden, 1, c->xb, m->dim, 0)) != RQ_OK) return rc;
        }
        if (fused) KCHK(gw_k_gemv1_norm(&m->cls, GW_GV_R_CLS, c->x, m->final_norm, c->logits_d, 0, 0, NULL, 0, s));
        else if ((rc = run_mm(c, &m->cls, 1, c->xq, c->xs, c->kmax, 1, c->logits_d, m->vocab, 0)) != RQ_OK) return rc;
    }
    HIPCHK(c, "hipEventRecord", hipEventRecord(e1, s));
    HIPCHK(c, "hipEventSynchronize", hipEventSynchronize(e1));
    float ms = 0;
    hipEventElapsedTime(&ms, e0, e1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    for (int l = 0; l < m->n_layers; l++) {
        const GwLayer *y = &m->layer[l];
        const GwMat *ws[7] = { &y->qkv[0], y->nqkv > 1 ? &y->qkv[1] : NULL, y->nqkv > 2 ? &y->qkv[2] : NULL, &y->wo, &y->w13[0],
                               y->nw13 > 1 ? &y->w13[1] : NULL, &y->w2 };
        for (int i = 0; i < 7; i++)
            if (ws[i]) {
                b += gw_mat_file_bytes(ws[i]);
                nl++;
            }
    }
    b += gw_mat_file_bytes(&m->cls);
    nl++;
    if (seconds) *seconds = ms * 1e-3 / reps;
    if (bytes) *bytes = b;
    if (launches) *launches = nl;
    return RQ_OK;
}

int gw_ctx_topk(RqCtx *c, int n, int k, float *vals, int *idx) {
    /* the k best logits of each of the first n rows on the device (sampler.c:186-217's candidates c_0 .. c_{k-1}:
     * larger first, the lower index first on ties): vals / idx, n x k each (host) */
    int rows = c->last_nsel;
    if (rows <= 0 || n < 1 || n > rows) return ctx_fail(c, RQ_ERR_STATE, "no logits rows on the device (%d)", rows);
    if (k < 1 || k > 64 || k >= c->m->vocab || !vals || !idx) return ctx_fail(c, RQ_ERR_ARG, "top-k %d", k);
    /* each buffer on first use, for the context's rows (one for a context of max_batch 0 or 1, whose decode leaves one
     * row); one that failed before is tried again, never launched on as null. The outputs: pinned host memory mapped
     * for the device, written by the selection kernel itself (no copy after it) */
    const size_t B = c->nb_max > 1 ? (size_t)c->nb_max : 1, ob = B * 64 * 4;
    if (!c->topk_scr && hipMalloc(&c->topk_scr, B * 64 * 64 * 8) != hipSuccess) return ctx_fail(c, RQ_ERR_NOMEM, "top-k scratch");
    if (!c->topk_h) {
        void *h = NULL, *d = NULL;
        if (hipHostMalloc(&h, 2 * ob, hipHostMallocMapped) != hipSuccess) return ctx_fail(c, RQ_ERR_NOMEM, "top-k outputs");
        if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess || !d) {
            hipHostFree(h);
            return ctx_fail(c, RQ_ERR_STATE, "top-k outputs: no device address");
        }
        c->topk_h = h;
        c->topk_v = (float *)d;
        c->topk_i = (int *)((char *)d + ob);
    }
    if (gw_k_topk(c->logits_d, c->m->vocab, c->m->vocab, n, k, c->topk_v, c->topk_i, c->topk_scr, c->stream))
        return ctx_fail(c, RQ_ERR_STATE, "top-k launch failed");
    HIPCHK(c, "hipStreamSynchronize (top-k)", hipStreamSynchronize(c->stream));
    memcpy(vals, c->topk_h, (size_t)n * k * 4);
    memcpy(idx, (char *)c->topk_h + ob, (size_t)n * k * 4);
    return RQ_OK;
}

int gw_ctx_topk_noalloc(RqCtx *c, int n, int k, float *vals, int *idx) {
    /* gw_ctx_topk without any allocation: the candidates and the device outputs live in the device's static scratch
     * array (gw_kernels.hip), at most GW_TOPK_NA_ROWS rows per call; calls that overlap on one device race */
    int rows = c->last_nsel;
    if (rows <= 0 || n < 1 || n > rows) return ctx_fail(c, RQ_ERR_STATE, "no logits rows on the device (%d)", rows);
    if (n > GW_TOPK_NA_ROWS)
        return ctx_fail(c, RQ_ERR_ARG, "top-k without allocation: %d rows, at most %d per call", n, GW_TOPK_NA_ROWS);
    if (k < 1 || k > 64 || k >= c->m->vocab || !vals || !idx) return ctx_fail(c, RQ_ERR_ARG, "top-k %d", k);
    float *vd = NULL;
    int *id = NULL;
    int e = gw_k_topk_noalloc(c->logits_d, c->m->vocab, c->m->vocab, n, k, &vd, &id, c->stream);
    if (e) return ctx_hip(c, "top-k (no allocation)", (hipError_t)e);
    HIPCHK(c, "hipMemcpyAsync (top-k)", hipMemcpyAsync(vals, vd, (size_t)n * k * 4, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, "hipMemcpyAsync (top-k)", hipMemcpyAsync(idx, id, (size_t)n * k * 4, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, "hipStreamSynchronize (top-k)", hipStreamSynchronize(c->stream));
    return RQ_OK;
}

int gw_sample_topk(const float *vals, const int *idx, int k, float temperature, float topp, unsigned long long *rng) {
    /* sample_topk (sampler.c:186-256) from its candidates (gw_ctx_topk's row): w_j = expf((x_j - x_0) * (1 / T)),
     * S = w_0 + .. in order, the nucleus by prefix sums against topp * S, the draw r = coin * W with coin the next
     * xorshift draw of *rng (sampler.c:258-269); the token. temperature > 0 */
    if (!vals || !idx || !rng || k < 1 || k > 64 || !(temperature > 0)) return RQ_ERR_ARG;
    *rng ^= *rng >> 12;
    *rng ^= *rng << 25;
    *rng ^= *rng >> 27;
    const float coin = (float)((unsigned)((*rng * 0x2545F4914F6CDD1Dull) >> 32) >> 8) / 16777216.0f;
    float w[64];
    const float mx = vals[0], inv_t = 1.0f / temperature;
    volatile float vs = 0;
    for (int j = 0; j < k; j++) {
        w[j] = expf((vals[j] - mx) * inv_t);
        vs = vs + w[j];
    }
    float sum = vs, cum = 0, wsum = sum;
    int m = k;
    if (topp > 0 && topp < 1) {
        const float t = topp * sum;
        for (int j = 0; j < k; j++) {
            cum += w[j];
            if (cum > t) { m = j + 1; wsum = cum; break; }
        }
    }
    const float r = coin * wsum;
    float cdf = 0;
    int last = 0;
    for (int j = 0; j < m; j++) {
        cdf += w[j];
        if (r < cdf) return idx[j];
        if (w[j] > 0) last = j;
    }
    return idx[last];
}

int gw_ctx_argmax(RqCtx *c, int *tokens, int n) {
    int rows = c->last_nsel;
    if (rows <= 0 || n < 1 || n > rows) return ctx_fail(c, RQ_ERR_STATE, "no logits rows on the device (%d)", rows);
    if (gw_k_argmax(c->logits_d, c->m->vocab, c->m->vocab, n, c->argmax_d, c->argmax_scr, c->stream))
        return ctx_fail(c, RQ_ERR_STATE, "argmax launch failed");
    HIPCHK(c, "hipMemcpyAsync (argmax)", hipMemcpyAsync(tokens, c->argmax_d, (size_t)n * 4, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, "hipStreamSynchronize (argmax)", hipStreamSynchronize(c->stream));
    return RQ_OK;
}
