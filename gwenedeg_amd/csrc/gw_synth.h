/* Seeded synthetic Qwen3-shaped GGUF writer (test and benchmark input; see gw_synth.c). */
#ifndef GW_SYNTH_H
#define GW_SYNTH_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
typedef struct {
    int dim, hidden, n_layers, n_heads, n_kv_heads, head_dim, vocab, ctx_len;
    float rope_theta;  /* 0: 1e6 */
    int tied;          /* 1: classifier tied to token_embd (no output.weight) */
    int type_default;  /* ggml type of the matmul tensors: 8 Q8_0 (0: Q8_0), 12 Q4_K, 14 Q6_K */
    int type_embd, type_out, type_q, type_k, type_v, type_o, type_gate, type_up, type_down; /* 0: type_default */
    float std;         /* 0: 0.02 */
    float norm_value;  /* 0: 1.0 */
    int tokenizer;     /* 1: a tokenizer block (byte-level BPE, gpt2 / qwen2, ChatML added tokens) */
} GwSynthCfg;
/* 0 on success; -1 bad shape, -2 no memory, -3 I/O, -4 threads */
int gw_synth_gguf(const char *path, const GwSynthCfg *cfg, unsigned long long seed, int nthreads);
size_t gw_synth_row_bytes(int type, int k);
void gw_synth_encode_row(int type, uint8_t *out, const float *x, int k);
#ifdef __cplusplus
}
#endif
#endif
