/* Internal declarations of the MI355X backend: the model / sequence / context objects behind the rq_* API and the
 * C-ABI launchers of the gfx950 kernels (gw_kernels.hip, gw_gemm.hip). */
#ifndef GW_INTERNAL_H
#define GW_INTERNAL_H

#ifndef __HIP_PLATFORM_AMD__
#define __HIP_PLATFORM_AMD__
#endif
#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#include "gwenedeg_gpu.h"

#ifdef __cplusplus
extern "C" {
#endif

enum { GW_F32 = 0, GW_Q8_0 = 8, GW_Q2_K = 10, GW_Q3_K = 11, GW_Q4_K = 12, GW_Q5_K = 13, GW_Q6_K = 14, GW_IQ2_XXS = 16,
       GW_IQ2_XS = 17, GW_IQ3_XXS = 18, GW_IQ1_S = 19, GW_IQ3_S = 21, GW_IQ2_S = 22, GW_IQ4_XS = 23, GW_IQ1_M = 29 }; /* ggml type numbers */

#define GW_ATT_T 16   /* positions per KV cache tile */
#define GW_ATT_P 256  /* positions per attention block */
#define GW_RMAX 512   /* rows per pass (RQ_BATCH_MAX) */
#define GW_W13_IL 4 /* w1 / w3 rows interleaved in the fused Q8_0 matrix (blocks of 4) */
#define GW_GEMV_MAX_ROWS 32 /* activation rows up to which a Q8_0 matmul takes the batched GEMV (else the MFMA GEMM) */
#define GW_Q4K_BYTES 144    /* bytes of a Q4_K super-block (256 weights), file and device */
#define GW_Q5K_BYTES 176    /* Q5_K, file and device */
#define GW_Q6K_BYTES 210    /* bytes of a Q6_K super-block in the file */
#define GW_Q6K_DEV 224      /* ... on the device: the file's 210 bytes padded to a 16-byte multiple (aligned loads) */
#define GW_Q3K_BYTES 110    /* Q3_K in the file */
#define GW_Q3K_DEV 112      /* ... on the device, padded as Q6_K */
#define GW_Q2K_BYTES 84     /* Q2_K in the file */
#define GW_Q2K_DEV 96       /* ... on the device, padded as Q6_K */
#define GW_IQ4XS_BYTES 136  /* IQ4_XS in the file */
#define GW_IQ4XS_DEV 144    /* ... on the device: the nibbles, the 8 S = ls - 32 as int8, D as fp32, padding (gw_iq.h) */
/* the codebook i-quants (iquants.h:12-27), file and device bytes per super-block (gw_iq.h: the fields reordered so a
 * half-group's are aligned dwords, d at the end, 2 bytes of padding; IQ1_M as the file) */
#define GW_IQ2XXS_BYTES 66
#define GW_IQ2XXS_DEV 68
#define GW_IQ2XS_BYTES 74
#define GW_IQ2XS_DEV 76
#define GW_IQ2S_BYTES 82
#define GW_IQ2S_DEV 84
#define GW_IQ3XXS_BYTES 98
#define GW_IQ3XXS_DEV 100
#define GW_IQ3S_BYTES 110
#define GW_IQ3S_DEV 112
#define GW_IQ1S_BYTES 50
#define GW_IQ1S_DEV 52
#define GW_IQ1M_BYTES 56
#define GW_IQ1M_DEV 56
#define GW_IS_CB(t) ((t) == GW_IQ2_XXS || (t) == GW_IQ2_XS || (t) == GW_IQ2_S || (t) == GW_IQ3_XXS || (t) == GW_IQ3_S || \
                     (t) == GW_IQ1_S || (t) == GW_IQ1_M)
/* RqModelOpts.repack (runq.h:76-82): IQ3_XXS / IQ3_S matmul weights held as 4-bit codes instead (internal types, never
 * in a file: the IQ_R bit of iquants.h:101-107), IQ4_XS's layout with a code table of their own (gw_iq.h) */
#define GW_IQ_R 0x100
enum { GW_IQ3_XXS_R = GW_IQ_R | GW_IQ3_XXS, GW_IQ3_S_R = GW_IQ_R | GW_IQ3_S };
#define GW_IQ3R_DEV 144
/* the super-block types (256 values; the matmul kernels' K-quant paths): Q2_K .. Q6_K and the i-quants */
#define GW_IS_KQ(t) (((t) >= GW_Q2_K && (t) <= GW_Q6_K) || (t) == GW_IQ4_XS || GW_IS_CB(t) || (t) == GW_IQ3_XXS_R || \
                     (t) == GW_IQ3_S_R)

/* KV cache types (runq.h:214): the rotated 8-bit / 4-bit ones, and the bytes of a tile (16 positions x hd of one kv
 * head) of K (is_v 0) or V: f32 64 hd, 16-bit 32 hd, q8 17 hd, q4 9 hd (RQ_KV_Q4: K q8, V q4; RQ_KV_Q4K4: both q4) */
/* ... and their bf16 dot-product types (the KV_DOT bit 4: RQ_KV_BF16_DOT 5, F16_DOT 6, Q8_DOT 7, Q4_DOT 12, Q4K4_DOT 13),
 * stored as their base type (the bf16-dot V in position pairs) */
static inline int gw_kv_dot(int kvt) { return kvt == 5 || kvt == 6 || kvt == 7 || kvt == 12 || kvt == 13; }
static inline int gw_kv_base(int kvt) { return gw_kv_dot(kvt) ? kvt & ~4 : kvt; }
static inline int gw_kv_quant(int kvt) {
    int b = gw_kv_base(kvt);
    return b == RQ_KV_Q8 || b == RQ_KV_Q4 || b == RQ_KV_Q4K4;
}
/* a type the device keeps: every type of runq.h:214 (f32, f16, bf16, the quantized ones, the dot-product types) */
static inline int gw_kv_ok(int kvt) {
    return kvt == RQ_KV_F32 || kvt == RQ_KV_F16 || kvt == RQ_KV_BF16 || gw_kv_quant(kvt) || gw_kv_dot(kvt);
}
/* the types whose attention runs in k_attn_q (the f16 / bf16 caches have their own kernels), which need a power-of-two
 * head_dim of 32 .. 128 */
static inline int gw_kv_att_q(int kvt) { return kvt == RQ_KV_F32 || gw_kv_quant(kvt) || gw_kv_dot(kvt); }
static inline size_t gw_kv_tile_bytes(int kvt, int hd, int is_v) {
    int b = gw_kv_base(kvt), q4 = b == RQ_KV_Q4K4 || (b == RQ_KV_Q4 && is_v);
    return (size_t)hd * (kvt == RQ_KV_F32 ? 64 : !gw_kv_quant(kvt) ? 32 : q4 ? 9 : 17);
}

/* a K-quant super-block's bytes in the file and on the device (0: not a K-quant) */
static inline int gw_kq_file_bytes(int type) {
    switch (type) {
    case GW_Q2_K: return GW_Q2K_BYTES;
    case GW_Q3_K: return GW_Q3K_BYTES;
    case GW_Q4_K: return GW_Q4K_BYTES;
    case GW_Q5_K: return GW_Q5K_BYTES;
    case GW_Q6_K: return GW_Q6K_BYTES;
    case GW_IQ4_XS: return GW_IQ4XS_BYTES;
    case GW_IQ2_XXS: return GW_IQ2XXS_BYTES;
    case GW_IQ2_XS: return GW_IQ2XS_BYTES;
    case GW_IQ2_S: return GW_IQ2S_BYTES;
    case GW_IQ3_XXS: return GW_IQ3XXS_BYTES;
    case GW_IQ3_S: return GW_IQ3S_BYTES;
    case GW_IQ1_S: return GW_IQ1S_BYTES;
    case GW_IQ1_M: return GW_IQ1M_BYTES;
    case GW_IQ3_XXS_R: return GW_IQ3XXS_BYTES;
    case GW_IQ3_S_R: return GW_IQ3S_BYTES;
    }
    return 0;
}
static inline int gw_kq_dev_bytes(int type) {
    switch (type) {
    case GW_Q2_K: return GW_Q2K_DEV;
    case GW_Q3_K: return GW_Q3K_DEV;
    case GW_Q6_K: return GW_Q6K_DEV;
    case GW_IQ4_XS: return GW_IQ4XS_DEV;
    case GW_IQ2_XXS: return GW_IQ2XXS_DEV;
    case GW_IQ2_XS: return GW_IQ2XS_DEV;
    case GW_IQ2_S: return GW_IQ2S_DEV;
    case GW_IQ3_XXS: return GW_IQ3XXS_DEV;
    case GW_IQ3_S: return GW_IQ3S_DEV;
    case GW_IQ1_S: return GW_IQ1S_DEV;
    case GW_IQ1_M: return GW_IQ1M_DEV;
    case GW_IQ3_XXS_R: case GW_IQ3_S_R: return GW_IQ3R_DEV;
    }
    return gw_kq_file_bytes(type);
}

/* A weight matrix on the device (rows x cols). Q8_0: int8 codes, row-major, and fp16 scales (cols / 32 per row),
 * the file's bytes split (34 bytes per 32 weights, as the file). K-quants: the file's super-blocks, row-major, each
 * bstride bytes apart (Q4_K 144, Q5_K 176; Q6_K 224: the file's 210 bytes and 14 of padding; Q3_K 112: 110 and 2;
 * Q2_K 96: 84 and 12);
 * the i-quants: their super-blocks with the fields reordered for aligned loads (gw_iq.h) */
typedef struct {
    int type, rows, cols;
    int8_t *codes;
    uint16_t *scales;
    uint8_t *blocks;
    int bstride;
} GwMat;

typedef struct {
    GwMat qkv[3];  /* Q8_0 model: qkv[0] = [wq | wk | wv] rows fused; K-quants: wq, wk, wv (types may differ) */
    int nqkv;
    GwMat wo;
    GwMat w13[2];  /* Q8_0: w13[0] = w1 and w3 fused, rows interleaved in blocks of GW_W13_IL (w1 rows 4i..4i+3, then
                    * w3 rows 4i..4i+3): one 8-row tile holds both halves of 4 SwiGLU outputs; K-quants: w1, w3 */
    int nw13, w13_il; /* w13_il: GW_W13_IL when fused, else 0 */
    GwMat w2;
    float *att_norm, *ffn_norm, *q_norm, *k_norm; /* device */
} GwLayer;

/* The reference's host modules that stay on the host (sampler.c, spec.c, chat.c, tokenizer.c's rq_token_bytes) read some
 * RqModel / RqSeq fields directly (internal.h:229-306, :353-398), compiled against the reference's layout. So both
 * structs begin with that layout as gcc lays it out on x86-64 (RqModel 9,208 bytes, RqSeq 1,832): the fields those
 * modules read sit at the reference's offsets, with this library's values, and every other byte of that prefix stays
 * zero. This library's own fields follow the prefix. The offsets are checked at compile time below and against the
 * reference's internal.h by tests/test_abi.py */
typedef struct { /* Config (internal.h:72-86): the first 48 bytes of the reference's RqModel */
    int magic_number, version, dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len, head_dim,
        shared_classifier, group_size;
} GwRefConfig;

/* Tokenizer (internal.h:207-224): built in place by the host's tokenizer.o (build_tokenizer_gguf), read by its
 * rq_tokenize / rq_token_bytes / rq_detok_* and by chat.c; this library reads bos / eos (rq_model_info) only */
typedef struct {
    char **vocab;
    int *vocab_len;
    float *merge_scores;
    int vocab_size;
    unsigned int max_token_length, bos_token_id, eos_token_id;
    char *vocab_data;
    int32_t *hash_ids;
    uint32_t *hash_tags;
    uint32_t hash_mask;
    int byte_token[256];
    int *added;
    int n_added;
    unsigned char added_first[256];
    int marks35;
} GwRefTokenizer;

#define GW_REF_MODEL_BYTES 9208
#define GW_REF_SEQ_BYTES 1832

struct RqModel {
    /* the reference's prefix (the readers: spec.c:32-54 config.vocab_size, :271-326 config.dim, :48 has_tok, :219 hy.on,
     * :292-330 mtp_of; sampler.c:328-331 samp_*; chat.c:38-295 chat, has_tok, the templates; tokenizer.c:812 has_tok) */
    GwRefConfig config;            /* @0: this model's shape, group_size 32 */
    unsigned char ref0_[280 - 48];
    GwRefTokenizer tok;            /* @280: the host's tokenizer (has_tok), else zero */
    unsigned char ref0b_[1752 - 1648];
    uint64_t ref_fp;               /* @1752: the file's fingerprint (model.c:949-953) */
    int has_weights, has_tok, is_gguf; /* @1760: weights on the device (0: tokenizer_only); the tokenizer built (the
                                        * host linked tokenizer.o, no_tokenizer 0); 1 */
    int gs_counted_;               /* @1772: 0 */
    char warning[256];             /* @1776: a load-time warning (RqModelInfo.warning), or "" */
    unsigned char ref1_[2080 - 2032];
    int hy_on;                     /* @2080: Hybrid.on, 0 (Qwen3: no linear-attention layers) */
    unsigned char ref2_[2684 - 2084];
    int chat;                      /* @2684: RQ_CHAT_* (gguf_chat_variant of the host's gguf.o; 0 without a tokenizer) */
    unsigned char ref3_[2768 - 2688];
    float samp_temp, samp_topp;    /* @2768: the file's recommended sampling (gguf_sampling; none without a tokenizer) */
    int samp_topk, samp_set;
    char user_tmpl[2][1024], sys_tmpl[2][1024], tmpl_missing[2][1088]; /* @2784, @4832, @6880: the chat templates */
    const RqModel *mtp_of;         /* @9056: NULL (not an MTP view) */
    unsigned char ref4_[GW_REF_MODEL_BYTES - 9064];
    /* this library's own */
    int dim, hidden, n_layers, n_heads, n_kv_heads, head_dim, vocab, seq_len, ctx_max, tied;
    float rope_theta, log_theta, att_scale;
    unsigned long long fingerprint;
    GwMat embd, cls;
    GwLayer *layer;
    float *final_norm;
    float *rope;       /* device: seq_len rows of head_dim floats (cos | sin) */
    float *norms;      /* the one allocation the norms live in */
    size_t dev_bytes;  /* device memory held by the weights */
    int repack;        /* RqModelOpts.repack (> 0: RQ_REPACK_* bits; else 0) */
    int kq;            /* a K-quant matrix present */
    int device;
};

struct RqSeq {
    /* the reference's prefix (the readers: spec.c:219 / :426 / :590 nck, :292-402 len, tokens, hvalid, hpos, hprev;
     * sampler.c:321-323 rng; chat.c:357 m) */
    const RqModel *m;  /* @0 */
    int cap;           /* @8: positions */
    int kv_len;        /* @12: cap rounded up to whole 256-position blocks (the cache layout) */
    int att_nb;        /* @16: kv_len / 256 */
    int kvt;           /* @20: RQ_KV_F16, RQ_KV_BF16, RQ_KV_Q8, RQ_KV_Q4 or RQ_KV_Q4K4 */
    unsigned char ref0_[80 - 24];
    int len;           /* @80: positions in the cache */
    int hwm;           /* @84 */
    unsigned char ref1_[96 - 88];
    int *tokens;       /* @96: host, cap tokens */
    unsigned char ref2_[120 - 104];
    int nck;           /* @120: checkpoint slots (rq_seq_set_checkpoints; RQ_SEQ_CK 2 at rq_seq_new). Qwen3 keeps no
                        * checkpoint: the count is only kept */
    unsigned char ref3_[1808 - 124];
    unsigned long long rng; /* @1808: the sampler's xorshift state */
    int hvalid, hpos;  /* @1816: an MTP view's state (spec.c); 0 and -1 here (no sequence is a view's) */
    float *hprev;      /* @1824: NULL */
    /* this library's own */
    uint16_t *kc, *vc; /* device: per layer kv_len x kv_dim 16-bit values (f16, or bf16 when kvt is); the quantized
                        * types: per layer kv_len / 16 x n_kv tiles of gw_kv_tile_bytes each, in the same tile order.
                        * Layer l's at l x lstride[kv] bytes (gw_seq_layer) */
    size_t lstride[2];  /* a layer's stride in kc (0) / vc (1): its bytes, rounded up to whole chunks when lazy */
    /* lazy memory (vmm 1): kc / vc are reserved address ranges; the first vm_n[kv] chunks of vm_chunk bytes of every
     * layer are mapped, each its own physical allocation vm_h[kv][l x vm_max[kv] + i] (gw_seq_map maps, rq_seq_release
     * unmaps). vmm 0: one hipMalloc per half, all of it */
    int vmm, vm_n[2], vm_max[2];
    size_t vm_chunk;
    hipMemGenericAllocationHandle_t *vm_h[2];
};

/* layer l's K (kv 0) or V (kv 1) cache base */
static inline uint16_t *gw_seq_layer(const RqSeq *s, int l, int kv) {
    return (uint16_t *)((uint8_t *)(kv ? s->vc : s->kc) + (size_t)l * s->lstride[kv]);
}
/* make positions 0 .. n - 1 of every layer writable (a lazy sequence maps the chunks not yet mapped): RQ_OK, or
 * RQ_ERR_NOMEM with nothing newly mapped in the half that failed */
int gw_seq_map(RqSeq *s, int n);

/* gw_host.c: model.c's host side (the tokenizer through the host's tokenizer.o / gguf.o, the chat templates) */
int gw_host_tokenizer_linked(void);
int gw_host_tokenizer(RqModel *m, const char *path, const void *map, size_t size, char *err, size_t errlen);
void gw_host_free_tokenizer(RqModel *m);

#ifndef __cplusplus
_Static_assert(sizeof(GwRefConfig) == 48, "Config");
_Static_assert(sizeof(GwRefTokenizer) == 1368 && offsetof(GwRefTokenizer, bos_token_id) == 32 &&
               offsetof(GwRefTokenizer, n_added) == 1104, "Tokenizer: the reference's layout");
_Static_assert(offsetof(struct RqModel, tok) == 280 && offsetof(struct RqModel, warning) == 1776 &&
               offsetof(struct RqModel, ref_fp) == 1752 && offsetof(struct RqModel, has_tok) == 1764 &&
               offsetof(struct RqModel, hy_on) == 2080 && offsetof(struct RqModel, chat) == 2684 &&
               offsetof(struct RqModel, samp_temp) == 2768 && offsetof(struct RqModel, samp_set) == 2780 &&
               offsetof(struct RqModel, user_tmpl) == 2784 && offsetof(struct RqModel, sys_tmpl) == 4832 &&
               offsetof(struct RqModel, tmpl_missing) == 6880 && offsetof(struct RqModel, mtp_of) == 9056 &&
               offsetof(struct RqModel, dim) == GW_REF_MODEL_BYTES, "RqModel: the reference's offsets");
_Static_assert(offsetof(struct RqSeq, cap) == 8 && offsetof(struct RqSeq, kvt) == 20 && offsetof(struct RqSeq, len) == 80 &&
               offsetof(struct RqSeq, tokens) == 96 && offsetof(struct RqSeq, nck) == 120 &&
               offsetof(struct RqSeq, rng) == 1808 && offsetof(struct RqSeq, hvalid) == 1816 &&
               offsetof(struct RqSeq, hpos) == 1820 && offsetof(struct RqSeq, hprev) == 1824 &&
               offsetof(struct RqSeq, kc) == GW_REF_SEQ_BYTES, "RqSeq: the reference's offsets");
#endif

struct RqCtx {
    const RqModel *m;
    int nb_max, att_nb;
    hipStream_t stream;
    /* device activations, nb_max rows */
    float *x, *xb, *qkv, *hb, *part, *logits_d, *hid_d;
    int8_t *xq, *hq;
    float *xs, *hs;
    int *argmax_d;
    void *argmax_scr;
    void *topk_scr; /* gw_ctx_topk's scratch (allocated at its first call): nb_max x 64 x 64 keys */
    void *topk_h;   /* ... and its outputs, in pinned host memory the selection kernel writes directly: nb_max x 64
                     * values, then nb_max x 64 indices */
    float *topk_v;  /* (the device addresses of those two) */
    int *topk_i;
    int kmax, ldqkv, pstride;
    size_t part_bytes;
    /* per-pass row metadata: one device block, filled from one pinned host block */
    void *meta_d, *meta_h;
    size_t meta_bytes;
    float *logits;     /* host: vocab floats (rq_decode's buffer) */
    float *lg_h;       /* pinned host staging of logits rows */
    size_t lg_h_rows;
    char err[256];
    int last_nsel;     /* logits rows the last pass left on the device (gw_ctx_argmax) */
    int *gtok_d, *gpos_d, *g_h; /* gw_decode_greedy: tokens and positions on the device, pinned staging; g_cap steps */
    int g_cap;
    void *smp, *smp_t; /* host scratch of the reference's sampler (ctx_sampler_scratch[_threads]): vocab x 8 bytes */
    int smp_nt;
    /* profiling (gw_ctx_profile_enable): HIP events around each kernel class of a pass, summed per class */
    int prof_on, nev;
    hipEvent_t *ev;
    int *ev_class;
    double prof_s[16];
    long prof_n[16];
    /* kernel timing (gw_ctx_kernel_timing): each matmul launch records its own start / stop (a pair of the pool),
     * collected when the pool is full or read; per class: summed seconds and launches */
    int kt_on, kt_n, kt_cur, kt_multi; /* kt_cur: the class of the kernels being launched (set with the profiling
                                        * marks); kt_multi: the pass has several rows */
    hipEvent_t *kt_ev;
    unsigned char *kt_cls;
    double kt_s[32];                   /* [multi][class] */
    long kt_cnt[32];
};

enum { GW_PF_EMBED, GW_PF_NORM, GW_PF_QKV, GW_PF_ROPE, GW_PF_ATT, GW_PF_COMBINE, GW_PF_WO, GW_PF_W13, GW_PF_SWIGLU, GW_PF_W2,
       GW_PF_CLS, GW_PF_N };

/* the file-format bytes of a matrix (Q8_0 34 per 32 weights, K-quants their super-block's bytes per 256) */
static inline double gw_mat_file_bytes(const GwMat *w) {
    double n = (double)w->rows * w->cols;
    return w->type == GW_Q8_0 ? n * 34 / 32 : GW_IS_KQ(w->type) ? n * gw_kq_file_bytes(w->type) / 256 : n * 4;
}

/* model / device helpers (gw_model.c) */
int gw_device_init(char *err, size_t errlen);
/* the reference's host-specific arithmetic (gw_exact.c): tables measured on this host, installed per device */
#define GW_RSQRT_MAXBITS_H 14
int gw_exact_init(char *err, size_t errlen);
int gw_exact_mode(void);        /* bit 0: 1 / sqrtf reproduced, bit 1: SwiGLU reproduced */
float gw_rsqrt_host(float t);   /* the reference's 1.0f / sqrtf(t) on this host */
float gw_exp_mvec(float x);     /* libmvec's expf by its method: the device's exp_mvec */
int gw_k_set_exact(const float *rsq, int bits, const uint64_t *rcp, const uint8_t *expd); /* gw_kernels.hip's copy */
int gw_v_set_exact(const float *rsq, int bits, const uint64_t *rcp, const uint8_t *expd); /* gw_gemv.hip's copy */
/* the i-quant codebooks on the current device (gw_gemm.hip's kernels); gw_iq_init: expanded from gw_iq_tables.h once
 * per process, installed once per device (the current one) */
int gw_g_set_iq(const uint64_t *iq2xxs, const uint64_t *iq2xs, const uint64_t *iq2s, const uint64_t *iq1s,
                const uint32_t *iq3xxs, const uint32_t *iq3s);
int gw_iq_init(char *err, size_t errlen);
/* vrcp14ps of d >= 1 from the compact table (one word per RCP_BLK_BITS-bit block of mantissas: the block's first value
 * and the value after its one step, as bits above 0.5's, and the step's offset): the result's bits */
#define RCP_BLK_BITS 7
static inline uint32_t gw_rcp_bits(const uint64_t *blk, uint32_t v) {
    const uint32_t m = v & 0x7fffffu;
    const uint64_t w = blk[m >> RCP_BLK_BITS];
    const uint32_t f = 0x3f000000u + (uint32_t)((m & ((1u << RCP_BLK_BITS) - 1)) < ((w >> 48) & 0xffu) ? w : w >> 24) % (1u << 24);
    return f - (((v >> 23) - 127u) << 23);
}
int gw_hip_fail(char *err, size_t errlen, const char *what, hipError_t e);

/* kernels (gw_kernels.hip) */
int gw_k_embed_q8(float *x, int dim, const uint8_t *codes, const uint16_t *scales, const int *tok, int n, hipStream_t s);
int gw_k_embed_kq(float *x, int dim, int type, const uint8_t *blocks, int bstride, const int *tok, int n, hipStream_t s);
/* nblk super-blocks of type (the file's bytes at src) -> the device layout at dst (gw_kq_dev_bytes apart): Q6_K, Q3_K
 * zero-padded, the i-quants' fields reordered (gw_iq.h); a type whose layouts are equal: a copy */
int gw_k_kq_to_dev(const uint8_t *src, size_t nblk, int type, uint8_t *dst, hipStream_t s);
int gw_k_rmsnorm_quant(float *x, const float *d, int dim, const float *w, const int *sel, int n, int8_t *xq, float *xs,
                       int ldq, float *hid, hipStream_t s);
int gw_k_qknorm_rope_store(float *qkv, int ldqkv, int n, int nh, int nkv, int hd, const float *qn, const float *kn,
                           const float *rope, const int *pos, uint16_t *const *kc, uint16_t *const *vc,
                           const int *kvt, hipStream_t s); /* kvt: per row, its cache type (runq.h:214; NULL: all f16) */
/* the attention partials of items on the f32 and quantized caches (RQ_KV_F32, Q8, Q4, Q4K4; dot 0) or on the dot-product
 * types (dot 1: every item's row one of them); kvt: each row's type; hd a power of two, 32 .. 128; nqm: the most query
 * vectors an item holds, 8 or 16 */
int gw_k_attn_q(const void *items, int nitems, const float *qkv, int ldqkv, int nh, int nkv, int hd, float scale, const int *pos,
                uint16_t *const *kc, uint16_t *const *vc, const int *kvt, int dot, int nqm, float *part, int pstride,
                hipStream_t s);
/* the rows of quantized caches: o = D H o' / hd from the combined attention att (n rows of nh hd), quantized into aq / as */
int gw_k_unrot_quant(const float *att, int n, int nh, int hd, const int *kvt, int8_t *aq, float *as, int ldq, hipStream_t s);
int gw_k_attn_part(const void *items, int nitems, int nq_max, const float *qkv, int ldqkv, int nh, int nkv, int hd, float scale,
                   const int *pos, uint16_t *const *kc, uint16_t *const *vc, float *part, int pstride, int kbf, hipStream_t s);
/* the one-row pass's attention with its QK-norm, RoPE and K / V store (hd 32, 64 or 128; pos: the row's position;
 * kl / vl: its sequence's K / V cache of the layer) */
int gw_k_attn_decode(const float *qkv, int nh, int nkv, int hd, float scale, const float *qn, const float *kn, const float *rope,
                     int pos, uint16_t *kl, uint16_t *vl, float *part, int pstride, int kbf, hipStream_t s);
/* the rows' attention from their key blocks' partials, quantized for wo (nbmax: the most key blocks of any row) */
int gw_k_attn_combine_quant(const float *part, int pstride, int nh, int hd, const int *pos, int n, int nbmax, int8_t *aq,
                            float *as, int ldq, float *att_out, hipStream_t s);
/* hb row: [h (H) | h2 (H)] (il = 0) or blocks of il h then il h2 (w1 / w3 rows interleaved by il) */
int gw_k_swiglu_quant(const float *hb, int H, int il, int n, int8_t *hq, float *hs, hipStream_t s);
int gw_k_quant_rows(const float *x, int n, int ldxf, int rows, int8_t *q, float *sc, int ldq, hipStream_t s);
int gw_k_argmax(const float *lg, int n, int ld, int rows, int *out, void *scratch, hipStream_t s); /* scratch: rows x 512 B */
/* the k best of each row in sample_topk's order (larger first, lower index on ties); scratch rows x 32 KiB, k <= 64 */
int gw_k_topk(const float *lg, int n, int ld, int rows, int k, float *vals, int *idx, void *scratch, hipStream_t s);
/* the same on the current device's static scratch array (no allocation; rows <= GW_TOPK_NA_ROWS): *vals / *idx, device
 * pointers into that array, get the rows x k outputs */
#define GW_TOPK_NA_ROWS 16
int gw_k_topk_noalloc(const float *lg, int n, int ld, int rows, int k, float **vals, int **idx, hipStream_t s);
/* GGUF Q8_0 blocks (gpr per row) -> codes + scales; il > 0: source row i to row (i / il) 2 il + off + i % il (two
 * matrices interleaved in blocks of il rows) */
int gw_k_q8_unpack(const uint8_t *blocks, size_t nblk, int8_t *codes, uint16_t *scales, int gpr, int il, int off, hipStream_t s);
int gw_k_fill_synthetic(uint16_t *kc, uint16_t *vc, size_t n, unsigned long long seed, int bf, hipStream_t s);
/* the quantized caches' synthetic rows (|K| < 4, |V| < 1 before the rotation): positions 0 .. npos - 1 of one layer's K
 * and V caches (kc / vc: the layer's bases), stored as k_qknorm_rope_store stores them */
int gw_k_fill_synthetic_q(void *kc, void *vc, int kvt, int npos, int nkv, int hd, unsigned long long seed, hipStream_t s);

/* the single-row Q8_0 GEMV with the activation's producer fused in front (gw_gemv.hip): out[row] (+)= W row . act for
 * R rows per tile (2, 4, 8, 16); act = the quantized row (q), rmsnorm(x, nw) (norm), the fp32 row x (qf) or the attention
 * combine of part over the row's nb <= GW_GV_NBMAX key blocks (combine); W Q8_0, W->cols % 64 == 0, <= 12288 (4096 for
 * R = 16), under 2 GiB. norm with swiglu_il = GW_W13_IL (R = 8, w1 / w3 interleaved): out[j] = swiglu(h_j, h2_j) */
#define GW_GV_NBMAX 4
#define GW_GV_R_QKV 4  /* weight rows per tile of the fused decode matmuls */
#define GW_GV_R_WO 4
#define GW_GV_R_W13 8
#define GW_GV_R_W2 2
#define GW_GV_R_CLS 8
/* nx, nR: the matmul launched next on the stream and its R (NULL: none, or not known); the blocks of this launch
 * warm its first tiles in L2 once their own loads are done (gw_gemv_warm_next) */
int gw_k_gemv1_q(const GwMat *w, int R, const int8_t *xq, const float *xs, float *out, int mode, const GwMat *nx, int nR,
                 hipStream_t s);
int gw_k_gemv1_norm(const GwMat *w, int R, const float *x, const float *nw, float *out, int mode, int swiglu_il,
                    const GwMat *nx, int nR, hipStream_t s);
int gw_k_gemv1_qf(const GwMat *w, int R, const float *x, float *out, int mode, const GwMat *nx, int nR, hipStream_t s);
int gw_k_gemv1_combine(const GwMat *w, int R, const float *part, int pstride, int hd, int nb, float *out, int mode,
                       const GwMat *nx, int nR, hipStream_t s);

/* per-launch kernel timing (gw_ctx_kernel_timing): gw_time_next_launch(a, b) makes the next matmul launch (k_gemv1,
 * k_gemm_q8, k_gemv_mr) record its own start and stop in events a and b (hipExtLaunchKernel's events: the
 * dispatch's timestamps, no extra packets on the stream); each launcher takes the pair once (gw_take_launch_events) */
void gw_time_next_launch(hipEvent_t a, hipEvent_t b);
void gw_take_launch_events(hipEvent_t *a, hipEvent_t *b);

/* the matmul dispatch (gw_gemm.hip): out[m * ldo + row] (+)= W row . X row m for M rows, any supported type */
int gw_k_matmul(const GwMat *w, const int8_t *xq, const float *xs, int ldx, int M, float *out, int ldo, int mode,
                hipStream_t s);
/* a and b (out from column col_b) in one launch where the kernel allows (two K-quant matrices of one type and width,
 * 9 .. 32 rows); else -1, nothing launched */
int gw_k_matmul2(const GwMat *a, const GwMat *b, int col_b, const int8_t *xq, const float *xs, int ldx, int M, float *out,
                 int ldo, int mode, hipStream_t s);

#ifdef __cplusplus
}
#endif
#endif
