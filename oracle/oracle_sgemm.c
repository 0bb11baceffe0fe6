/*
 * TEST INFRASTRUCTURE ONLY -- the oracle's stand-in for matrixmultiply::sgemm
 * (third-party crate matrixmultiply 0.3, called from
 * oxionnx-ops/src/math_typed.rs:61-77 and conv/conv2d.rs:923-938,1165-1180).
 * The crate is not vendored in the reference.  Its published algorithm is the
 * Goto / BLIS packed GEMM: B is packed into KC x NR column panels, A into
 * MC x KC row panels of MR rows, and a register-blocked FMA microkernel
 * accumulates an MR x NR block of C over one KC slab.  That is what is
 * restated here, with an AVX2 / FMA 6 x 16 microkernel (twelve 8-lane
 * accumulators); matrixmultiply's own f32 FMA kernel is 8 x 8 with KC 256,
 * so the two differ in blocking, not in kind.  Rows are split across threads
 * the way parallel_sgemm does (conv/conv2d.rs:1132-1183); the accumulation
 * order of an element does not depend on the split, so the result is the
 * same for any thread count.
 */
#include "oracle.h"
#include <immintrin.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    int64_t m0, m1, k, n;
    const float* a; int64_t rsa, csa;
    const float* b; int64_t rsb, csb;
    float* c; int64_t rsc;
} job_t;

#define MR 6
#define NR 16
#define KC 256
#define MC 120
#define NC 2048

static int64_t min64(int64_t x, int64_t y) { return x < y ? x : y; }

/* B[0..kc, 0..nc) into panels of NR columns: panel j holds kc rows of NR. */
static void pack_b(const float* b, int64_t rsb, int64_t csb, int64_t kc, int64_t nc, float* bp) {
    for (int64_t jp = 0; jp < nc; jp += NR) {
        const int64_t nw = min64(NR, nc - jp);
        float* dst = bp + jp * kc;
        for (int64_t p = 0; p < kc; ++p) {
            const float* src = b + p * rsb + jp * csb;
            int64_t q = 0;
            for (; q < nw; ++q) dst[p * NR + q] = src[q * csb];
            for (; q < NR; ++q) dst[p * NR + q] = 0.0f;
        }
    }
}

/* A[0..mc, 0..kc) into panels of MR rows: panel i holds kc columns of MR. */
static void pack_a(const float* a, int64_t rsa, int64_t csa, int64_t mc, int64_t kc, float* ap) {
    for (int64_t ip = 0; ip < mc; ip += MR) {
        const int64_t mw = min64(MR, mc - ip);
        float* dst = ap + ip * kc;
        for (int64_t p = 0; p < kc; ++p) {
            int64_t r = 0;
            for (; r < mw; ++r) dst[p * MR + r] = a[(ip + r) * rsa + p * csa];
            for (; r < MR; ++r) dst[p * MR + r] = 0.0f;
        }
    }
}

/* C[0..mw, 0..nw) += Apanel * Bpanel over kc. */
static void micro(int64_t kc, const float* ap, const float* bp, float* c, int64_t rsc, int64_t mw, int64_t nw) {
    __m256 acc[MR][2];
    for (int r = 0; r < MR; ++r) acc[r][0] = acc[r][1] = _mm256_setzero_ps();
    for (int64_t p = 0; p < kc; ++p) {
        const __m256 b0 = _mm256_loadu_ps(bp + p * NR), b1 = _mm256_loadu_ps(bp + p * NR + 8);
        for (int r = 0; r < MR; ++r) {
            const __m256 av = _mm256_broadcast_ss(ap + p * MR + r);
            acc[r][0] = _mm256_fmadd_ps(av, b0, acc[r][0]);
            acc[r][1] = _mm256_fmadd_ps(av, b1, acc[r][1]);
        }
    }
    if (mw == MR && nw == NR) {
        for (int r = 0; r < MR; ++r) {
            float* cr = c + r * rsc;
            _mm256_storeu_ps(cr, _mm256_add_ps(_mm256_loadu_ps(cr), acc[r][0]));
            _mm256_storeu_ps(cr + 8, _mm256_add_ps(_mm256_loadu_ps(cr + 8), acc[r][1]));
        }
        return;
    }
    float tmp[MR][NR];
    for (int r = 0; r < MR; ++r) {
        _mm256_storeu_ps(tmp[r], acc[r][0]);
        _mm256_storeu_ps(tmp[r] + 8, acc[r][1]);
    }
    for (int64_t r = 0; r < mw; ++r)
        for (int64_t q = 0; q < nw; ++q) c[r * rsc + q] += tmp[r][q];
}

static void* run(void* arg) {
    job_t* j = (job_t*)arg;
    const int64_t k = j->k, n = j->n;
    float* bp = (float*)aligned_alloc(64, sizeof(float) * KC * NC);
    float* ap = (float*)aligned_alloc(64, sizeof(float) * MC * KC);
    for (int64_t i = j->m0; i < j->m1; ++i) memset(j->c + i * j->rsc, 0, sizeof(float) * (size_t)n);
    for (int64_t jc = 0; jc < n; jc += NC) {
        const int64_t nc = min64(NC, n - jc);
        for (int64_t pc = 0; pc < k; pc += KC) {
            const int64_t kc = min64(KC, k - pc);
            pack_b(j->b + pc * j->rsb + jc * j->csb, j->rsb, j->csb, kc, nc, bp);
            for (int64_t ic = j->m0; ic < j->m1; ic += MC) {
                const int64_t mc = min64(MC, j->m1 - ic);
                pack_a(j->a + ic * j->rsa + pc * j->csa, j->rsa, j->csa, mc, kc, ap);
                for (int64_t jr = 0; jr < nc; jr += NR)
                    for (int64_t ir = 0; ir < mc; ir += MR)
                        micro(kc, ap + ir * kc, bp + jr * kc, j->c + (ic + ir) * j->rsc + jc + jr, j->rsc,
                              min64(MR, mc - ir), min64(NR, nc - jr));
            }
        }
    }
    free(bp);
    free(ap);
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
