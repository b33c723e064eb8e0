/* The oracle: a plain-C restatement of the reference's arithmetic for the forward hot path.
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the checker; the product (gwenedeg_amd) never links, calls or falls back to it.
 * Every function names the reference file:line it follows (paths relative to the reference tree). */
#ifndef GW_ORACLE_H
#define GW_ORACLE_H
#include <stddef.h>
#include <stdint.h>

/* element formats */
float or_fp16_to_f32(uint16_t h);   /* kquants.h:143-156 */
uint16_t or_f32_f16(float f);       /* forward.c:1325-1344 */

/* activation quantization, per group of 32 (forward.c:803-836) */
void or_quantize(int8_t *q, float *s, const float *x, int n);

/* Q8_0: exact int32 sum per group, then val = val + (ws * xs) * (float) isum in group order
 * (forward.c:906-916 as compiled; kernels_avx512.h:157-162). out[m * N + n] = W row n . X row m */
float or_dot_q8(const int8_t *wq, const float *ws, const int8_t *xq, const float *xs, int k);
void or_q8_matmul(float *out, const int8_t *wq, const float *ws, const int8_t *xq, const float *xs, int M, int N, int K);
void or_q8_block_sums(int32_t *isum, const int8_t *wq, const int8_t *xq, int M, int N, int K); /* [m][n][g] */
/* Q8_0 file blocks (34 bytes: fp16 d, 32 int8) -> codes + fp32 scales (model.c:47-59) */
void or_q8_from_blocks(int8_t *q, float *s, const uint8_t *blk, size_t nblk);

/* K-quants and IQ4_XS on GGUF blocks: the definition of kquants.h:79-109 (types 11-14) and iquants.h:49-57 (types 10, 23) */
void or_kq_dequant_row(int type, const uint8_t *blk, int n, float *y); /* kquants.h:222-251 */
void or_kq_matmul(int type, float *out, const uint8_t *blocks, const int8_t *xq, const float *xs, int M, int N, int K);
void or_kq_act_prep(float *xf, const int8_t *xq, const float *xs, int n); /* kquants.h:392-400 */

/* attention (kernels_avx512.h:1084-1131, forward.c:1301-1431) */
float or_exp_att(float x);
size_t or_kv_tile(int t, int h, int n_kv, int hd); /* forward.c:1894-1899 */
/* one query vector over positions 0..n-1 of kv head h of one layer's tiled f16 caches (kc, vc: the layer's base) */
void or_attention(float *out, const float *q, const uint16_t *kc, const uint16_t *vc, int n, int h, int n_kv, int hd,
                  float scale);
/* the partial result of block b (positions 256 b .. min(n, 256 b + 256) - 1): o[hd] unnormalized, ml = {m, l} */
void or_attention_block(float *o, float *ml, const float *q, const uint16_t *kc, const uint16_t *vc, int n, int b, int h,
                        int n_kv, int hd, float scale);
void or_att_combine(float *out, int nb, const float *part, size_t stride, int hd); /* forward.c:1405-1431 */

/* norms, RoPE, SwiGLU (forward.c:886-901, :1248-1284, :1953-1958) */
float or_rsqrt_ref(float t);      /* the reference's 1.0f / sqrtf on this host: rsqrtss + Newton */
float or_rms_scale(const float *x, int n);
void or_rmsnorm(float *o, const float *x, const float *w, int n);
float or_silu_exp(float x);
void or_rope_row(float *cs, int hd, int pos, float log_theta);
void or_qk_norm_rope(float *v, int n_heads, const float *w, int hd, const float *cs);
void or_swiglu(float *hb, const float *hb2, int n);
void or_set_swiglu_host(int on); /* 1: SwiGLU with this host's libmvec expf + rcp14 (the reference's exact bits) */

/* the whole forward pass of one row (decode_worker, forward.c:2568-2813) on a model read from a GGUF file */
typedef struct OrModel OrModel;
typedef struct OrSeq OrSeq;
OrModel *or_model_load(const char *path, int cap, char *err, size_t errlen);
void or_model_free(OrModel *m);
/* dim, hidden, n_layers, n_heads, n_kv_heads, head_dim, vocab, kv_len (capacity rounded up to 256) */
void or_model_dims(const OrModel *m, int *d8);
float or_model_att_scale(const OrModel *m);
OrSeq *or_seq_new(const OrModel *m);
OrSeq *or_seq_new_kv(const OrModel *m, int bf16); /* bf16 1: a bf16 cache (RQ_KV_BF16) */
/* a cache of type kv_type (runq.h:214: 2 f16, 1 bf16, 3 q8, 8 q4, 9 q4k4; the quantized ones forward.c:1609-1790; + 4:
 * the bf16 dot-product attention on them, kernels_avx512.h:1439-1475) */
OrSeq *or_seq_new_type(const OrModel *m, int kv_type);
const uint8_t *or_seq_cache_q(const OrSeq *s, int layer, int v); /* a quantized cache's layer base, else NULL */
uint16_t or_f32_bf16(float f);
void or_seq_free(OrSeq *s);
int or_seq_len(const OrSeq *s);
void or_seq_truncate(OrSeq *s, int n);
void or_seq_copy(OrSeq *dst, const OrSeq *src, int n);
/* the layer's K / V cache base (kv_len * kv_dim f16 values each, the tiled layout) */
const uint16_t *or_seq_cache(const OrSeq *s, int layer, int v);
uint16_t *or_seq_cache_mut(OrSeq *s, int layer, int v);
void or_seq_set_len(OrSeq *s, int n);
/* token at the next position; logits (vocab floats) if not NULL; trace (n_layers * dim floats: the residual stream
 * after each layer) if not NULL. 0 on success */
int or_forward_token(const OrModel *m, OrSeq *s, int token, float *logits, float *trace);

#endif
