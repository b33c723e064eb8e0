/* gwenedeg_gpu.h: the C ABI of the MI355X backend of gwenedeg's forward hot path (libgwenedeg_amd.so).
 *
 * The entry points are the forward half of the reference's public API, src/runq.h, with the same names, argument
 * meaning, return codes and error behaviour, so that runq.h's callers (engine, CLI, chat, speculative loop, tests)
 * link against this library instead of the reference's forward.c / model.c weight path. Each declaration cites the
 * runq.h line it replaces. Types are laid out exactly as runq.h's (same fields, order and widths).
 *
 * Scope of the device implementation: Qwen3 dense models (GGUF, Q8_0 / Q2_K .. Q6_K / IQ1_S .. IQ4_XS matrices), the f16, bf16,
 * q8, q4 and q4k4 KV caches (RQ_KV_F16, RQ_KV_BF16, RQ_KV_Q8, RQ_KV_Q4, RQ_KV_Q4K4), their bf16 dot-product types
 * (RQ_KV_BF16_DOT, F16_DOT, Q8_DOT, Q4_DOT, Q4K4_DOT) and RQ_KV_F32, one GPU, one HIP stream per context. Calls are synchronous at return
 * (logits valid on the host), as the reference's are. Results are bit-identical for any batch composition: a row's
 * logits do not depend on the rows it is batched with (the device kernels compute each output whole, in a fixed order).
 *
 * Extensions without a counterpart in runq.h are prefixed gw_ (below), e.g. the isolated Q8_0 operator of the
 * reference's kernels_avx512.h and device-side greedy sampling.
 */
#ifndef GWENEDEG_GPU_H
#define GWENEDEG_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* runq.h:35-44 */
enum {
    RQ_OK = 0,
    RQ_ERR_ARG = -1,
    RQ_ERR_NOMEM = -2,
    RQ_ERR_CONTEXT = -3,
    RQ_ERR_STATE = -4,
    RQ_ERR_LOAD = -5,
    RQ_ERR_IO = -6,
    RQ_ERR_MISMATCH = -7,
};
const char *rq_strerror(int err);  /* runq.h:45 */
double rq_now(void);               /* runq.h:46 */
const char *rq_threads_init(int n); /* runq.h:53: accepted, no effect (the device runs the passes) */
int rq_threads(void);              /* runq.h:54 */

typedef struct RqModel RqModel;
typedef struct RqSeq RqSeq;
typedef struct RqCtx RqCtx;

#define RQ_CTX_DEFAULT_MAX 40960 /* runq.h:61 */

/* runq.h:63-81 (same layout). tokenizer_only and no_tokenizer as the reference (model.c:1010-1016, :893-922): the
 * tokenizer is built by the host's own tokenizer.o / gguf.o when the program links them (rq_chat_check below).
 * repack as the reference (model.c:360-364): the IQ3_XXS / IQ3_S matmul weights held as 4-bit codes on the device
 * (144 bytes per 256 weights against 100 / 112: no codebook lookups in the kernels), the same values and results;
 * RQ_REPACK_ALL or the type bits; the embedding table keeps the file's type (a tied classifier with it).
 * page_cache / checkpoints are accepted and ignored here: the file is read once, Qwen3 has no recurrent state */
typedef struct {
    int ctx_len;
    int tokenizer_only;
    int no_tokenizer;
    double mem;
    int kv_bits;
    int page_cache;
    int checkpoints;
    int repack;
} RqModelOpts;
enum { RQ_REPACK_ALL = 1, RQ_REPACK_IQ3_S = 2, RQ_REPACK_IQ3_XXS = 4 }; /* runq.h:83 */

/* runq.h:87-88: a GGUF file (qwen3; Q8_0, Q2_K .. Q6_K and the i-quants IQ1_S .. IQ4_XS as matrices and embedding),
 * its weights repacked into device memory.
 * Unless opts->no_tokenizer, the tokenizer, chat variant, recommended sampling and chat templates too, where the
 * program links the reference's tokenizer.o, gguf.o and threads.o (their build entry points are weak references
 * here); without them the model loads without a tokenizer and RqModelInfo.warning says so. tokenizer_only: no
 * weights, no device (needs those objects) */
RqModel *rq_model_load(const char *path, const RqModelOpts *opts, char *err, size_t errlen);
void rq_model_free(RqModel *m);

/* the chat-template side of model.c that the reference's chat.o, cli.o, serve.o and tools.o call (runq.h:458-459;
 * model.c:798-862) */
enum { RQ_CHAT_HYBRID = 0, RQ_CHAT_INSTRUCT = 1, RQ_CHAT_THINKING = 2, RQ_CHAT_QWEN35 = 3, RQ_CHAT_QWEN38 = 4 };
const char *rq_chat_name(int variant);                                      /* runq.h:459 */
int rq_chat_check(const RqModel *m, int thinking, char *err, size_t errlen); /* runq.h:502 */
const char *chat_gen_suffix(const RqModel *m, int thinking);                /* internal.h (model.c:803): chat.o */

/* runq.h:132-147 */
typedef struct {
    int dim, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim, vocab_size;
    int seq_len;
    int ctx_max;
    int group_size;
    int shared_classifier;
    int gguf;
    int bos, eos;
    const char *warning;
    int chat;
    float rope_theta;
    int linear_layers;
    unsigned long long fingerprint;
} RqModelInfo;
void rq_model_info(const RqModel *m, RqModelInfo *info);

/* memory estimates: runq.h:150-171 (the layouts are runq.h's). This library counts device memory: the weights' device
 * copies, a context of RQ_BATCH_MAX rows plus the 288 MiB of exactness tables per device, and a sequence's K / V
 * halves; there is no recurrent state, no checkpoint and no budget check (budget 0, budget_src 0) */
typedef struct {
    size_t kv;
    size_t state;
    int checkpoints;
    size_t total;
} RqSeqMem; /* runq.h:152-157 */
typedef struct {
    size_t weights;
    size_t runtime;
    RqSeqMem seq;
    size_t total;
    double budget;
    int budget_src;
    size_t read;
} RqModelMem; /* runq.h:158-167 */
int rq_model_mem(const RqModel *m, RqModelMem *mem);                          /* runq.h:168 */
int rq_seq_mem(const RqModel *m, int capacity, int kv_type, RqSeqMem *mem);    /* runq.h:171 */
double rq_mem_available(void);                                                /* runq.h:173 */
/* runq.h:175-195 (model.c:1402-1438): available 1 (the device has kernels for the repacked IQ3 codes); per type of the
 * matmul weights among IQ3_S, IQ3_XXS (their RqModelOpts.repack bits) and IQ1_S, IQ1_M (bit 0): the matrices, their
 * share of the values, their device bytes now, and extra = what the repack adds to the device layout's bytes (IQ1:
 * the device layout's bytes over the file's); weights = the device bytes */
#define RQ_REPACK_TYPES 4
typedef struct {
    const char *type;
    int bit;
    int repacked;
    int mats;
    double share;
    size_t bytes, extra;
} RqRepackType;
typedef struct {
    int available;
    int n;
    RqRepackType t[RQ_REPACK_TYPES];
    size_t weights;
    size_t extra;
} RqRepackInfo;
int rq_repack_info(const RqModel *m, RqRepackInfo *info);                     /* runq.h:195 */
/* runq.h:196-199: a decode step and a 4-row all-logits pass at position 32, the fastest of reps, seconds */
int rq_pass_times(const RqModel *m, int reps, double *t1, double *t4);
/* MTP views (runq.h:100-112) are Qwen3.5's: NULL, with the reason in err */
typedef struct {
    int vocab;
    double mem;
} RqMtpOpts;
RqModel *rq_mtp_load(const RqModel *target, const RqMtpOpts *o, char *err, size_t errlen);
/* runq.h:716-720's test hook: RQ_ERR_STATE (the file is not kept after the load) */
int rq_dequant_rows(const RqModel *m, const char *name, size_t name_len, long r0, long nr, float **rows, float **packed,
                    int *ncols, int *npacked, char *err, size_t errlen);

/* runq.h:214-219 */
enum { RQ_KV_F32 = 0, RQ_KV_BF16 = 1, RQ_KV_F16 = 2, RQ_KV_Q8 = 3, RQ_KV_BF16_DOT = 5, RQ_KV_F16_DOT = 6, RQ_KV_Q8_DOT = 7,
       RQ_KV_Q4 = 8, RQ_KV_Q4K4 = 9, RQ_KV_Q4_DOT = 12, RQ_KV_Q4K4_DOT = 13, RQ_KV_DEFAULT = RQ_KV_F16 };
const char *rq_kv_name(int kv_type); /* runq.h:216 */
int rq_kv_parse(const char *name);   /* runq.h:217 */
int rq_kv_bits(int kv_type);         /* runq.h:218 */

/* sequences: runq.h:222-282 (the KV cache lives in device memory, in the reference's tiled layout) */
RqSeq *rq_seq_new(const RqModel *m, int capacity, int kv_type, int *err); /* runq.h:222 */
void rq_seq_free(RqSeq *s);                                               /* runq.h:223 */
void rq_seq_reset(RqSeq *s);                                              /* runq.h:224 */
int rq_seq_truncate(RqSeq *s, int n);                                     /* runq.h:229 */
int rq_seq_keep(const RqSeq *s, int n);                                   /* runq.h:230 */
int rq_seq_checkpoint_at(RqSeq *s, int pos);                              /* runq.h:239: Qwen3, a no-op */
int rq_seq_checkpoint_rows(RqSeq *s, int pos, int n);                     /* runq.h:247: Qwen3, a no-op */
void rq_seq_checkpoint_rows_drop(RqSeq *s);                               /* runq.h:248 */
int rq_seq_set_checkpoints(RqSeq *s, int n);                              /* runq.h:252 */
int rq_seq_checkpoints(const RqSeq *s, int *pos, int max);                /* runq.h:256: 0 */
int rq_seq_checkpoint_drop(RqSeq *s, int pos);                            /* runq.h:259: RQ_ERR_ARG (none held) */
int rq_seq_len(const RqSeq *s);                                           /* runq.h:260 */
int rq_seq_capacity(const RqSeq *s);                                      /* runq.h:261 */
const int *rq_seq_tokens(const RqSeq *s);                                 /* runq.h:262 */
int rq_seq_common_prefix(const RqSeq *s, const int *tokens, int n);       /* runq.h:263 */
int rq_seq_release(RqSeq *s, int keep);                                   /* runq.h:270 */
void rq_seq_resident(const RqSeq *s, RqSeqMem *out);                      /* runq.h:274: all of its device K / V */
size_t rq_seq_kv_bytes(const RqSeq *s, int n);                            /* runq.h:277 */
int rq_seq_copy(RqSeq *dst, const RqSeq *src, int n);                     /* runq.h:282: device-to-device */

/* Saved sequences, the KV disk tier (runq.h:283-314; seqfile.c's file format, version 1, so files move between this
 * library and the reference for the same model file): rq_seq_save writes positions 0..len-1 (tokens, K / V blocks
 * through a host staging buffer, the RNG state) as path.tmp, synced, then renamed to path; rq_seq_load restores the
 * first n positions. RQ_ERR_IO, RQ_ERR_MISMATCH (another model file, shape or KV type; a corrupt header) */
#define RQ_CHECKPOINTS_MAX 32
typedef struct {
    int len;
    int kv_type;
    int linear;
    int n_ck;
    int ck[RQ_CHECKPOINTS_MAX];
    long long bytes;
} RqSeqFile; /* runq.h:295-302 */
int rq_seq_save(const RqSeq *s, const char *path);                                  /* runq.h:293 */
long long rq_seq_save_bytes(const RqSeq *s);                                        /* runq.h:294 */
int rq_seq_file_info(const RqModel *m, const char *path, RqSeqFile *info, int **tokens); /* runq.h:305 */
int rq_seq_file_keep(const RqSeqFile *f, int n);                                    /* runq.h:308 */
int rq_seq_load(RqSeq *dst, const char *path, int n);                               /* runq.h:314 */
void rq_seq_seed(RqSeq *s, unsigned long long seed);                      /* runq.h:315 */
unsigned long long *rq_seq_rng(RqSeq *s);                                 /* runq.h:319 */
int rq_seq_fill_synthetic(RqSeq *s, int n, unsigned long long seed);      /* runq.h:726 */

/* contexts: runq.h:325-338 */
#define RQ_BATCH_MAX 512
RqCtx *rq_ctx_new(const RqModel *m, int max_batch, int max_ctx, int *err); /* runq.h:332 */
void rq_ctx_free(RqCtx *c);                                                /* runq.h:333 */
int rq_ctx_max_batch(const RqCtx *c);                                      /* runq.h:334 */
const char *rq_ctx_error(const RqCtx *c);                                  /* runq.h:335 */
int rq_ctx_profile(const RqCtx *c, const char **names, double *seconds, int max); /* runq.h:338 */

/* forward passes: runq.h:341-375 */
enum { RQ_LOGITS_NONE = 0, RQ_LOGITS_LAST = 1, RQ_LOGITS_ALL = 2 };
int rq_decode(RqCtx *c, RqSeq *s, int token, float **logits);                                            /* runq.h:346 */
int rq_decode_hidden(RqCtx *c, RqSeq *s, int token, float **logits, float *hidden, const float *h_in);  /* runq.h:350 */
int rq_prefill(RqCtx *c, RqSeq *s, const int *tokens, int n, int mode, float *out, float **logits);      /* runq.h:355 */
typedef struct {
    RqSeq *seq;
    const int *tokens;
    int n;
    int logits;
    float *hidden;
    const float *h_in;
} RqSegment; /* runq.h:364-374 */
int rq_forward_batch(RqCtx *c, const RqSegment *seg, int nseg, float *out, float **logits); /* runq.h:375 */

/* runq.h:561 */
unsigned long long rq_logits_hash(const float *logits, int n);

/* The reference's internal accessors that its sampler.c links against (internal.h:326-328, defined in forward.c:772-784):
 * the context's host scratch of vocab x 8 bytes (and of nt such rows for rq_sample_batch; NULL: no memory) and the
 * vocabulary size. They let sampler.c (rq_sample, rq_sample_batch) run unchanged on this library's contexts */
void *ctx_sampler_scratch(RqCtx *c);
void *ctx_sampler_scratch_threads(RqCtx *c, int nt);
int ctx_vocab(const RqCtx *c);

/* The reference's internal prefill with hidden rows that its spec.c links against (internal.h:339, forward.c:3880-3916):
 * rq_prefill's rows (chunks of max_batch, or token by token with max_batch <= 1) with every row's final hidden state
 * (the final-normed row, dim floats) into hidden (n x dim; NULL: none). h_in, an MTP view's input rows (Qwen3.5),
 * is refused with RQ_ERR_ARG: no model loaded here is such a view. rq_prefill is fw_rows without hidden and h_in */
int fw_rows(RqCtx *c, RqSeq *s, const int *tokens, int n, int mode, float *out, float **logits, float *hidden, const float *h_in);

/* ------------------------------------------------------------------------------------- extensions (gw_) */

/* Device-side greedy sampling of a pass's logits rows: the first maximum of each row (the reference's
 * sample_argmax, sampler.c:40-60, run on the logits before they leave the device). After rq_decode /
 * rq_forward_batch on c: tokens[j] = argmax of selected row j, j < n (n <= the rows the last pass selected).
 * RQ_ERR_STATE if the last pass produced no logits */
int gw_ctx_argmax(RqCtx *c, int *tokens, int n);

/* Top-k on the device (sampler.c:186-217): for the first n logits rows of the context's last pass (as gw_ctx_argmax),
 * the k largest logits of each row and their token ids, larger first and the lower id first on ties (the reference's
 * candidate order c_0 .. c_{k-1}), into vals / idx (host, n x k each); 1 <= k <= 64, k < vocab. 64 x 8 bytes per row
 * cross the bus instead of the row's logits. No counterpart in runq.h: a sampler over the candidates replaces
 * rq_sample_batch's top-k rows (engine.c:3230-3253) */
int gw_ctx_topk(RqCtx *c, int n, int k, float *vals, int *idx);
/* gw_ctx_topk without any allocation, for callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops that forbid hipMalloc): the same results; no counterpart in the reference. The candidates and the device
 * outputs live in a static array of 520 KiB per device (held until the process ends), so at most 16 rows per call
 * (n > 16: RQ_ERR_ARG); every call on a device uses the same array, so calls that overlap on one device race */
int gw_ctx_topk_noalloc(RqCtx *c, int n, int k, float *vals, int *idx);
/* sample_topk (sampler.c:186-256) on such a row's candidates, with temperature > 0, top-p topp (<= 0 or >= 1: off) and
 * the sequence's RNG state (rq_seq_rng, runq.h:319; advanced by one draw as rq_sample does): the same token as the
 * reference's rq_sample with cfg->top_k = k on the full row; RQ_ERR_ARG for bad arguments */
int gw_sample_topk(const float *vals, const int *idx, int k, float temperature, float topp, unsigned long long *rng);

/* rq_decode (runq.h:346) followed by the greedy choice on the device: *next = the first maximum of the row's logits,
 * which stay on the device (no vocab-size copy per step; gw_ctx_argmax can read them again). The decode loop of a
 * greedy generation (rq_gen_step + sample_argmax, chat.c:348, sampler.c:40) without the logits transfer */
int gw_decode_argmax(RqCtx *c, RqSeq *s, int token, int *next);

/* n greedy decode steps from token (the generation loop of chat.c:348 with sample_argmax, sampler.c:40-60):
 * tokens[i] = the first maximum of step i's logits, the token fed to step i + 1; the sequence grows by n (token,
 * tokens[0 .. n - 2] are its new tokens). Each step's token stays on the device, so the n passes run back to back and
 * the host waits once. Results equal n gw_decode_argmax calls. RQ_ERR_CONTEXT past the capacity, nothing done */
int gw_decode_greedy(RqCtx *c, RqSeq *s, int token, int n, int *tokens);

/* rq_forward_batch (runq.h:375) with the selected rows' logits left on the device instead of copied to the host: the
 * batched decode step of a serving loop (engine.c:3230-3253 samples every row), followed by gw_ctx_argmax for greedy
 * rows. Same validation and errors as rq_forward_batch */
int gw_forward_batch_device(RqCtx *c, const RqSegment *seg, int nseg);

/* Per-kernel-class device time (the GPU counterpart of the reference's -DRUNQ_PROFILE phases, forward.c:13-24):
 * gw_ctx_profile_enable(c, 1) resets the counters and brackets each kernel class of every later pass with HIP events
 * on the context's stream; rq_ctx_profile then returns the classes' names and summed seconds, and
 * gw_ctx_profile_launches the number of intervals of class i (its launches). 0 turns it off */
int gw_ctx_profile_enable(RqCtx *c, int on);

/* The weight matmuls of one decode step (per layer q / k / v, wo, w1 / w3, w2; then the classifier), launched as a
 * one-row pass launches them (all-Q8_0 models: the fused GEMVs), back to back, reps times, timed with HIP events on
 * the context's stream: *seconds per sweep, *bytes = their file-format weight bytes (the algorithmic bytes of a decode
 * step's weight streaming), *launches per sweep. Inputs are the context's buffers as they are (call it after a pass);
 * outputs go to its scratch rows. The counterpart of the reference's pass timing (rq_pass_times, runq.h:196-199) for
 * the GEMV alone */
int gw_ctx_gemv_sweep(RqCtx *c, int reps, double *seconds, double *bytes, int *launches);
long gw_ctx_profile_launches(const RqCtx *c, int cls);

/* Kernel timing, for roofline figures: gw_ctx_kernel_timing(c, 1) resets the counters and makes every later kernel of
 * c's passes record its own start and stop (hipExtLaunchKernel's events: the dispatch's timestamps, no packets between
 * kernels, so the passes run as they do untimed); 0 turns it off. gw_ctx_kernel_times synchronizes c's stream and
 * returns, per kernel class of rq_ctx_profile's names (embed, matmul qkv, attention, ..., classifier), the summed
 * kernel seconds and launches of the one-row passes (multi 0: decode) or of the passes of several rows (multi 1:
 * prefill, batches); the return value is the class count */
int gw_ctx_kernel_timing(RqCtx *c, int on);
int gw_ctx_kernel_times(RqCtx *c, int multi, const char **names, double *seconds, long *launches, int max);

/* The isolated Q8_0 operator (the reference's kernels_avx512.h q8p_pack_blocks :113, q8p_gemv_rows :286 and
 * q8p_gemm_item :235, and forward.c's quantize :803), on device pointers, on the given HIP stream (NULL: the null
 * stream); asynchronous. Return RQ_OK or RQ_ERR_ARG (shapes: N % 16 == 0, K % 32 == 0) / RQ_ERR_STATE (launch failed).
 *   gw_q8_pack:     nblk GGUF Q8_0 blocks (34 bytes each, row-major: N rows of K / 32 blocks) -> codes (N x K int8) and
 *                   fp16 scales (N x K / 32), the device layout
 *   gw_quantize:    M rows of K fp32 -> int8 codes + fp32 scales per group of 32 (forward.c:803-836)
 *   gw_q8_matmul:   out[m * N + n] = W row n . X row m, m < M: exact int32 sums per group, the fold
 *                   val = val + (ws * xs) * (float) isum in group order (forward.c:906-916), bit-identical to the
 *                   reference's q8p_gemv_rows / q8p_gemm_item on the same int8 inputs
 *   gw_q8_block_sums: isum[(m * N + n) * (K / 32) + g], the exact int32 sum of group g (for the bit-exact check) */
int gw_q8_pack(const void *blocks, int N, int K, int8_t *codes, uint16_t *scales, void *stream);
int gw_quantize(const float *x, int M, int K, int8_t *xq, float *xs, void *stream);
int gw_q8_matmul(float *out, const int8_t *codes, const uint16_t *scales, int N, int K, const int8_t *xq, const float *xs,
                 int M, void *stream);
int gw_q8_block_sums(int32_t *isum, const int8_t *codes, int N, int K, const int8_t *xq, int M, void *stream);

/* The K-quant operator on the file's blocks (kquants.h:79-109's definition; type 11 Q3_K, 12 Q4_K, 13 Q5_K, 14 Q6_K;
 * and iquants.h:49-57's for type 10 Q2_K and 23 IQ4_XS): out[m * N + n], blocks: N rows of K / 256 blocks, device memory */
int gw_kq_matmul(float *out, int type, const void *blocks, int N, int K, const int8_t *xq, const float *xs, int M,
                 void *stream);

/* The top-k selection of gw_ctx_topk on device logits (sample_topk's candidate order, sampler.c:186-217: the k
 * largest values of each row, ties to the lower index, larger first; -0 ties +0, NaN after -inf): rows rows of n
 * values, ld floats apart; vals / idx: rows x k (device memory); scratch: rows x 32 KiB of device memory. 1 <= k <= 64,
 * k < n <= 262144. RQ_OK, RQ_ERR_ARG (nothing launched) or RQ_ERR_STATE; asynchronous on stream */
int gw_topk_rows(const float *logits, int n, int ld, int rows, int k, float *vals, int *idx, void *scratch, void *stream);

/* The row tile of the MFMA GEMMs (prefill and batched rows: k_gemm_q8 for Q8_0 above 32 rows, k_gemm_kq for Q4_K /
 * Q6_K above 32 rows): 0 chosen per launch (64-row tiles when they give each SIMD several waves, else 32; a K-quant
 * matrix too narrow for 64 blocks takes the batched GEMV; the default), 32 or 64 forced (and the K-quant GEMM
 * taken whatever the width). Returns the previous setting, or -1 (and changes nothing) for another value. A tuning
 * and test hook with no counterpart in runq.h; results do not depend on it */
int gw_matmul_tile_rows(int rows);

/* The kernel of the Q8_0 matmuls of 2 .. 32 activation rows (batched decode rows): 0 chosen per launch (the default:
 * the MFMA GEMM above 16 rows, above 8 for matrices of 8,192 rows or more, above 12 for 6,144 or more at K <= 4,096, and
 * where K <= 4,096 and K % 512 == 0 above 8 for 6,144 rows or more and above 12 for 4,096 or more; else the batched GEMV
 * in passes of 8 rows), 1 the batched GEMV, 2 the MFMA GEMM (its kernel as gw_q8_gemm_kernel chooses).
 * Returns the previous setting, or -1 (and changes nothing) for another value. A tuning and test hook with no
 * counterpart in runq.h; results do not depend on it */
int gw_q8_batch_kernel(int k);

/* The kernel of the Q8_0 MFMA GEMM (K % 128 == 0): 0 chosen per launch (the default: k_gemm_q8t of 32 x 32 tiles with
 * 512-byte stages where they are at most one per CU and K % 512 == 0, with 256-byte stages where they are at most 1.5
 * per CU, of 64 x 64 where those are at most one per CU; else up to 32 rows k_gemm_q8f, above
 * k_gemm_q8l with 128-column tiles where they give 3 blocks per CU, else 64), 1 k_gemm_q8f (4 waves, stages staged
 * through registers, 32-row tiles up to 32 rows), 2 / 3 k_gemm_q8l with 128 / 64-column tiles (8 / 4 waves of 32 x 32
 * tiles, stages copied into LDS by the buffer unit), 4 / 5 k_gemm_q8t of 64 x 64 tiles (16 waves of 16 x 16 tiles) with
 * stages of 256 bytes of K where K % 256 == 0, else 128 / with 128, 6 / 7 k_gemm_q8t of 32 x 32 / 32 x 16 tiles (256-byte
 * stages where K % 256 == 0, else the 64 x 64 tiles' 128-byte ones), 8 k_gemm_q8t of 32 x 32 tiles with 512-byte
 * stages where K % 512 == 0 (else as 6). Returns the previous setting, or -1 (and changes nothing) for another value.
 * A tuning and test hook with no counterpart in runq.h; results do not depend on it */
int gw_q8_gemm_kernel(int k);

/* The kernel of the 9 .. 32-row K-quant GEMM (Q4_K / Q6_K, batched decode rows): 0 k_gemm_kq32 (32-row tiles, the
 * groups spread over 8 waves, the terms exchanged in LDS; the default), 1 k_gemm_kq16 (each wave on 16 weight rows x 16
 * activation rows over all of K, the fold in registers). Returns the previous setting, or -1 (and changes
 * nothing) for another value. A tuning and test hook with no counterpart in runq.h; results do not depend on it */
int gw_kq_small_kernel(int kq16);

/* The activation-row quads (of 8 rows) per block of the 9 .. 32-row K-quant GEMM (k_gemm_kq32): 0 the default (4: a
 * block folds all 32 rows of its weight tile), 1 or 2 forced (more blocks, each folding fewer outputs), 4 forced. Returns the previous setting, or -1 (and changes nothing) for another value. A tuning and
 * test hook with no counterpart in runq.h; results do not depend on it */
int gw_kq32_quads(int nqr);

/* The super-blocks per step of the 9 .. 32-row K-quant GEMM (k_gemm_kq32): 0 the default (1), 1 or 2 forced (2: 16
 * waves, each on one group of one of the step's two super-blocks, half the steps). Returns the previous setting, or -1
 * (and changes nothing) for another value. A tuning and test hook with no counterpart in runq.h; results do not depend
 * on it */
int gw_kq32_step(int sb);

/* Whether each decode GEMV, once its blocks have issued their last weight loads, warms the first weight tiles of the
 * matmul launched after it (the next layer's included) in L2: 1 on (the default), 0 off, a negative value only
 * queries. Returns the previous setting. A tuning and test hook with no counterpart in runq.h; results do not depend
 * on it */
int gw_gemv_warm_next(int on);

/* How rq_seq_new gives a sequence its device KV memory: 1 lazily (the default, where the device has HIP virtual memory
 * management): the address range of the capacity reserved, memory mapped in 2 MiB chunks per layer and half (K / V)
 * as positions are first written, the chunks past max(keep, len) unmapped by rq_seq_release, so a sequence holds what
 * it has used (the reference's host pages behave so, forward.c:474-510); 0 all of it allocated at rq_seq_new.
 * Sequences made before a change keep theirs. A negative value only queries; returns the previous setting. No
 * counterpart in runq.h; results do not depend on it */
int gw_seq_lazy(int on);

/* The device bytes s's K / V caches hold now: its mapped chunks (lazy), or the whole allocation */
size_t gw_seq_device_bytes(const RqSeq *s);

/* The context's stream (a hipStream_t), for callers that time the passes with events on it */
void *gw_ctx_stream(RqCtx *c);

/* Which of the reference's host-specific float operations the device reproduces, measured on this host at the first
 * rq_model_load (no counterpart in runq.h): bit 0 its 1.0f / sqrtf (rsqrtss + Newton: rmsnorm forward.c:896,
 * QK-norm, the attention scale forward.c:137), bit 1 its SwiGLU (libmvec vector expf, vrcp14ps + Newton,
 * forward.c:1953-1958). Bits 0 and 1 both set: the device's results equal the reference's CPU path on this host bit
 * for bit; otherwise the missing operation falls back to IEEE (sqrtf, division) and the attention's exp. Bit 2 (with
 * bit 1): the host's libmvec expf equals its published method on every input checked, so the device needs no table
 * of differences. 0 before any model load */
int gw_exact_mode(void);

#ifdef __cplusplus
}
#endif
#endif
