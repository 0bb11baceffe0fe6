/*
 * TEST INFRASTRUCTURE ONLY -- the oracle's stand-in for matrixmultiply::sgemm
 * (third-party crate matrixmultiply 0.3, called from
 * oxionnx-ops/src/math_typed.rs:61-77 and conv/conv2d.rs:923-938,1165-1180).
 * The crate is not vendored in the reference; its published algorithm is a
 * packed, cache-blocked GEMM with an FMA microkernel, restated here as a
 * blocked i-k-j loop that the compiler vectorises with FMA (this file is
 * built with -ffp-contract=fast).  Rows are split across threads the way
 * parallel_sgemm does (conv/conv2d.rs:1132-1183); K-accumulation order does
 * not depend on the split, so the result is the same for any thread count.
 */
#include "oracle.h"
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    int64_t m0, m1, k, n;
    const float* a; int64_t rsa, csa;
    const float* b; int64_t rsb, csb;
    float* c; int64_t rsc;
} job_t;

#define NB 512
#define KB 256

static void* run(void* p) {
    job_t* j = (job_t*)p;
    int64_t k = j->k, n = j->n;
    float* bpack = (float*)malloc(sizeof(float) * KB * NB);
    for (int64_t i = j->m0; i < j->m1; ++i) memset(j->c + i * j->rsc, 0, sizeof(float) * (size_t)n);
    for (int64_t nb = 0; nb < n; nb += NB) {
        int64_t nw = n - nb < NB ? n - nb : NB;
        for (int64_t kb = 0; kb < k; kb += KB) {
            int64_t kw = k - kb < KB ? k - kb : KB;
            for (int64_t p = 0; p < kw; ++p)
                for (int64_t q = 0; q < nw; ++q)
                    bpack[p * NB + q] = j->b[(kb + p) * j->rsb + (nb + q) * j->csb];
            for (int64_t i = j->m0; i < j->m1; ++i) {
                float* crow = j->c + i * j->rsc + nb;
                for (int64_t p = 0; p < kw; ++p) {
                    float av = j->a[i * j->rsa + (kb + p) * j->csa];
                    const float* br = bpack + p * NB;
                    for (int64_t q = 0; q < nw; ++q) crow[q] += av * br[q];
                }
            }
        }
    }
    free(bpack);
    return NULL;
}

void orc_sgemm(int64_t m, int64_t k, int64_t n,
               const float* a, int64_t rsa, int64_t csa,
               const float* b, int64_t rsb, int64_t csb,
               float* c, int64_t rsc, int nthreads) {
    if (m <= 0 || n <= 0) return;
    if (nthreads < 1) nthreads = 1;
    /* parallel_sgemm's gate: split rows only when m >= 2*threads and the
     * work reaches 64^3 (conv/conv2d.rs:588,866-903). */
    if ((double)m * (double)k * (double)n < 64.0 * 64 * 64 || m < 2 * (int64_t)nthreads) nthreads = 1;
    job_t* jobs = (job_t*)calloc((size_t)nthreads, sizeof(job_t));
    pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
    int64_t chunk = (m + nthreads - 1) / nthreads;
    int used = 0;
    for (int t = 0; t < nthreads; ++t) {
        int64_t m0 = t * chunk, m1 = m0 + chunk < m ? m0 + chunk : m;
        if (m0 >= m) break;
        jobs[t] = (job_t){m0, m1, k, n, a, rsa, csa, b, rsb, csb, c, rsc};
        used++;
    }
    for (int t = 1; t < used; ++t) pthread_create(&th[t], NULL, run, &jobs[t]);
    run(&jobs[0]);
    for (int t = 1; t < used; ++t) pthread_join(th[t], NULL);
    free(jobs); free(th);
}
