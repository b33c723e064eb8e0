/* The reference's own AVX-512 matmul kernels on given inputs (test infrastructure: compiled by oracle/Makefile
 * against the reference's kernels_avx512.h / kquants.h where they lie, into oracle/_ref/ref_q8op; never part of
 * the product). Pins the oracle's matmul fold to the reference's code bit for bit, and times the isolated Q8_0
 * op on the host cores as the CPU baseline.
 *   ref_q8op q8 W WS X XS M N K OUT [reps threads copies]
 *       W: N x K int8 codes, WS: N x K/32 fp32 weight scales (q8_from_blocks, model.c:47-59), X: M x K int8,
 *       XS: M x K/32 fp32 activation scales. Packs W (q8p_pack_blocks, kernels_avx512.h:113), then M = 1:
 *       q8p_gemv_rows (:286), M > 1: q8p_gemm_item (:235) over every (32-row tile, chunk) item; OUT: M x N fp32.
 *       reps > 0: also times reps runs on `threads` threads (items split evenly), prints JSON seconds per run (best,
 *       mean, median); run r reads packed copy r % copies of W (copies > 1: more weight bytes than the host's caches
 *       hold, as a model's matrices follow one another).
 *   ref_q8op kq TYPE BLK X XS M N K OUT
 *       BLK: N rows of K / 256 GGUF K-quant blocks (TYPE 11 Q3_K, 12 Q4_K, 13 Q5_K, 14 Q6_K), packed by kq_pack_blocks
 *       (kquants.h:253) and multiplied by the generic kq_dot (:608) with kq_act_prep's xf (:392).
 *   ref_q8op iq TYPE BLK X XS M N K OUT
 *       BLK: N rows of K / 256 GGUF blocks (TYPE 10 Q2_K, 16 IQ2_XXS, 17 IQ2_XS, 18 IQ3_XXS, 19 IQ1_S, 21 IQ3_S, 22 IQ2_S,
 *       23 IQ4_XS, 29 IQ1_M), packed by iq_pack_blocks (iquants.h:503) and multiplied by iq_rows (:1478), the forward's
 *       dispatch (the AVX-512 kernels of this build), with the activation sums of 16 of kq512_c16 (kernels_avx512.h:342).
 *   ref_q8op iqdq TYPE BLK NBLK OUT
 *       NBLK blocks of one of those types dequantized by iq_dequant_row (iquants.h:217): OUT 256 NBLK fp32.
 * All files raw little-endian arrays. */
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "kernels_avx512.h"
#include "iquants.h"

int rq_iq_gather = 0; /* (model.c:9: the VBMI decode, as the forward runs it) */

#ifndef RUNQ_VNNI
#error "needs the AVX-512 VNNI kernels (an AVX-512 VNNI -march)"
#endif

static void *slurp(const char *p, size_t need) {
    FILE *f = fopen(p, "rb");
    if (!f) { perror(p); exit(1); }
    void *v = aligned_alloc(64, (need + 63) / 64 * 64);
    if (!v || fread(v, 1, need, f) != need) { fprintf(stderr, "ref_q8op: %s: short read\n", p); exit(1); }
    fclose(f);
    return v;
}

static double now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + 1e-9 * ts.tv_nsec;
}

typedef struct {
    float *out; const uint8_t *wp; const int8_t *x; const float *xs; const int32_t *corr;
    int M, N, K, nbi, nchunk, it0, it1;
} Part;

static void run_part(const Part *p) {
    if (p->M == 1) {
        q8p_gemv_rows(p->out, p->x, p->xs, p->corr, p->wp, p->K, 32, p->it0, p->it1);
        return;
    }
    for (int it = p->it0; it < p->it1; it++)
        q8p_gemm_item(p->out, p->N, p->wp, p->N, it / p->nchunk, it % p->nchunk, p->nbi, p->x, p->xs, p->K, p->M, p->K, 32,
                      p->corr);
}

static void *part_thread(void *a) { run_part(a); return NULL; }

int main(int argc, char **argv) {
    if (argc >= 10 && !strcmp(argv[1], "q8")) {
        int M = atoi(argv[6]), N = atoi(argv[7]), K = atoi(argv[8]);
        int reps = argc > 10 ? atoi(argv[10]) : 0, nt = argc > 11 ? atoi(argv[11]) : 1, ncp = argc > 12 ? atoi(argv[12]) : 1;
        if (M < 1 || N % 32 || K % 32) { fprintf(stderr, "ref_q8op: bad shape\n"); return 2; }
        int8_t *W = slurp(argv[2], (size_t)N * K), *X = slurp(argv[4], (size_t)M * K);
        float *WS = slurp(argv[3], (size_t)N * (K / 32) * 4), *XS = slurp(argv[5], (size_t)M * (K / 32) * 4);
        uint8_t *wp = aligned_alloc(64, q8p_size(N, K, 32));
        q8p_pack_blocks(wp, W, WS, N / 16, K, 32);
        int32_t *corr = malloc((size_t)M * (K / 32) * sizeof(int32_t));
        for (int b = 0; b < M; b++)
            q8p_gemv_corr(corr + (size_t)b * (K / 32), X + (size_t)b * K, K, 32);
        float *out = calloc((size_t)M * N, sizeof(float));
        int ntile = N / 32, nbi = q8p_nb(M, ntile, nt), nchunk = (M + nbi - 1) / nbi;
        int nitems = M == 1 ? N / 16 : ntile * nchunk;
        Part one = { out, wp, X, XS, corr, M, N, K, nbi, nchunk, 0, nitems };
        run_part(&one);
        FILE *f = fopen(argv[9], "wb");
        if (!f || fwrite(out, sizeof(float), (size_t)M * N, f) != (size_t)M * N) { perror(argv[9]); return 1; }
        fclose(f);
        if (reps > 0) {
            if (nt < 1) nt = 1;
            if (nt > 256) nt = 256;
            if (ncp < 1) ncp = 1;
            if (ncp > 64) ncp = 64;
            const size_t pb = q8p_size(N, K, 32);
            uint8_t **cp = malloc((size_t)ncp * sizeof(uint8_t *));
            cp[0] = wp;
            for (int i = 1; i < ncp; i++) {
                if (!(cp[i] = aligned_alloc(64, (pb + 63) / 64 * 64))) { perror("copies"); return 1; }
                memcpy(cp[i], wp, pb);
            }
            Part *pp = malloc((size_t)nt * sizeof(Part));
            pthread_t *th = malloc((size_t)nt * sizeof(pthread_t));
            double best = 1e30, tot = 0, *ts = malloc((size_t)reps * sizeof(double));
            for (int r = 0; r < reps; r++) {
                double t0 = now();
                for (int i = 0; i < nt; i++) {
                    pp[i] = one;
                    pp[i].wp = cp[r % ncp];
                    pp[i].it0 = (int)((long)nitems * i / nt);
                    pp[i].it1 = (int)((long)nitems * (i + 1) / nt);
                    pthread_create(&th[i], NULL, part_thread, &pp[i]);
                }
                for (int i = 0; i < nt; i++) pthread_join(th[i], NULL);
                double t = now() - t0;
                best = t < best ? t : best;
                tot += t;
                ts[r] = t;
            }
            for (int i = 1; i < reps; i++) /* (insertion sort: the median) */
                for (int j = i; j > 0 && ts[j - 1] > ts[j]; j--) {
                    double x = ts[j];
                    ts[j] = ts[j - 1];
                    ts[j - 1] = x;
                }
            const double med = reps % 2 ? ts[reps / 2] : 0.5 * (ts[reps / 2 - 1] + ts[reps / 2]);
            printf("{\"op\": \"q8\", \"M\": %d, \"N\": %d, \"K\": %d, \"threads\": %d, \"reps\": %d, \"copies\": %d, "
                   "\"best_s\": %.9f, \"mean_s\": %.9f, \"median_s\": %.9f}\n", M, N, K, nt, reps, ncp, best, tot / reps, med);
        }
        return 0;
    }
    if (argc >= 10 && !strcmp(argv[1], "kq")) {
        int type = atoi(argv[2]), M = atoi(argv[6]), N = atoi(argv[7]), K = atoi(argv[8]);
        if (type < GGML_Q3_K || type > GGML_Q6_K || M < 1 || N % 16 || K % 256) { fprintf(stderr, "ref_q8op: bad kq args\n"); return 2; }
        size_t bb = (size_t)kq_block_bytes(type) * (K / 256);
        uint8_t *blk = slurp(argv[3], (size_t)N * bb);
        int8_t *X = slurp(argv[4], (size_t)M * K);
        float *XS = slurp(argv[5], (size_t)M * (K / 32) * 4);
        uint8_t *kp = aligned_alloc(64, (kq_size(type, N, K) + 63) / 64 * 64);
        kq_pack_blocks(type, kp, blk, N / 16, K);
        float *xf = malloc((size_t)M * (K / 32) * sizeof(float));
        for (int b = 0; b < M; b++)
            kq_act_prep(xf + (size_t)b * (K / 32), X + (size_t)b * K, XS + (size_t)b * (K / 32), K);
        float *out = calloc((size_t)M * N, sizeof(float));
        for (int rb = 0; rb < N / 16; rb++)
            for (int b = 0; b < M; b += KQ_NC) {
                int nc = M - b < KQ_NC ? M - b : KQ_NC;
                kq_dot(type, out + (size_t)b * N + rb * 16, N, kp + (size_t)rb * (K / 256) * kq_sb_bytes(type), K, nc,
                       X + (size_t)b * K, K, XS + (size_t)b * (K / 32), K / 32, xf + (size_t)b * (K / 32), K / 32);
            }
        FILE *f = fopen(argv[9], "wb");
        if (!f || fwrite(out, sizeof(float), (size_t)M * N, f) != (size_t)M * N) { perror(argv[9]); return 1; }
        fclose(f);
        return 0;
    }
    if (argc >= 10 && !strcmp(argv[1], "iq")) {
        int type = atoi(argv[2]), M = atoi(argv[6]), N = atoi(argv[7]), K = atoi(argv[8]);
        if (!iq_type(type) || type & IQ_R || M < 1 || N % 16 || K % 256) { fprintf(stderr, "ref_q8op: bad iq args\n"); return 2; }
        uint8_t *blk = slurp(argv[3], (size_t)N * (K / 256) * iq_block_bytes(type));
        int8_t *X = slurp(argv[4], (size_t)M * K);
        float *XS = slurp(argv[5], (size_t)M * (K / 32) * 4);
        uint8_t *kp = aligned_alloc(64, (iq_size(type, N, K) + 63) / 64 * 64);
        iq_pack_blocks(type, kp, blk, N / 16, K);
        int32_t *c16 = malloc((size_t)M * (K / 16) * sizeof(int32_t));
        for (int b = 0; b < M; b++) kq512_c16(c16 + (size_t)b * (K / 16), X + (size_t)b * K, K);
        float *out = calloc((size_t)M * N, sizeof(float));
        iq_rows(type, out, N, X, K, XS, c16, M, kp, K, 0, N / 16);
        FILE *f = fopen(argv[9], "wb");
        if (!f || fwrite(out, sizeof(float), (size_t)M * N, f) != (size_t)M * N) { perror(argv[9]); return 1; }
        fclose(f);
        return 0;
    }
    if (argc >= 6 && !strcmp(argv[1], "iqdq")) { /* iq_dequant_row (iquants.h:217): NBLK blocks of TYPE -> 256 NBLK floats */
        int type = atoi(argv[2]), nblk = atoi(argv[4]);
        if (!iq_type(type) || type & IQ_R || nblk < 1) { fprintf(stderr, "ref_q8op: bad iqdq args\n"); return 2; }
        uint8_t *blk = slurp(argv[3], (size_t)nblk * iq_block_bytes(type));
        float *y = malloc((size_t)nblk * 256 * sizeof(float));
        iq_dequant_row(type, blk, 256 * nblk, y);
        FILE *f = fopen(argv[5], "wb");
        if (!f || fwrite(y, sizeof(float), (size_t)nblk * 256, f) != (size_t)nblk * 256) { perror(argv[5]); return 1; }
        fclose(f);
        return 0;
    }
    fprintf(stderr, "usage: ref_q8op q8 W WS X XS M N K OUT [reps threads] | kq|iq TYPE BLK X XS M N K OUT | iqdq TYPE BLK NBLK OUT\n");
    return 2;
}
