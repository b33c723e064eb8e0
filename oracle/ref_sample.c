/* Test driver (never part of the product): the reference's own top-k sampler (sampler.c: rq_rng_f32 and
 * sample_topk, compiled from its sources with its flags) on rows of logits, for tests/test_oracle.py.
 *   ref_sample LOGITS ROWS V K TEMPERATURE TOPP RNG
 * LOGITS: ROWS x V float32. Per row, in order: coin = rq_rng_f32(&rng), token = sample_topk(row, V, K, T, TOPP, ...,
 * coin). Prints {"tokens": [...], "rng": "<hex>"} (the state after the last draw). */
#include <stdio.h>
#include <stdlib.h>

#include "runq.h"

/* sampler.c:8-11 and :186 (file-scope there, no header): the candidate type and the sampler */
typedef struct {
    float prob;
    int index;
} ProbIndex;
int sample_topk(const float *x, int n, int k, float temperature, float topp, ProbIndex *pi, float coin);

int main(int argc, char **argv) {
    if (argc != 8) { fprintf(stderr, "usage: ref_sample LOGITS ROWS V K TEMPERATURE TOPP RNG\n"); return 2; }
    int rows = atoi(argv[2]), V = atoi(argv[3]), k = atoi(argv[4]);
    float T = strtof(argv[5], NULL), topp = strtof(argv[6], NULL);
    unsigned long long rng = strtoull(argv[7], NULL, 0);
    FILE *f = fopen(argv[1], "rb");
    float *x = malloc((size_t)rows * V * sizeof(float));
    ProbIndex *pi = malloc((size_t)V * sizeof(ProbIndex));
    if (!f || !x || !pi || fread(x, sizeof(float), (size_t)rows * V, f) != (size_t)rows * V) { perror("ref_sample"); return 1; }
    fclose(f);
    printf("{\"tokens\": [");
    for (int r = 0; r < rows; r++) {
        float coin = rq_rng_f32(&rng);
        printf("%s%d", r ? ", " : "", sample_topk(x + (size_t)r * V, V, k, T, topp, pi, coin));
    }
    printf("], \"rng\": \"%llx\"}\n", rng);
    return 0;
}
