/*
 * CPU oracle for the FP32 attention path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only as the
 * checker (or, for cpu_baseline, as the timed CPU port of the reference path). The product path
 * (rocmkernels_amd, libROCmKernels.Kernels.Shared.so) never calls it and has no CPU fallback.
 *
 * oracle_attention() restates the reference's own CPU reference, ReferenceAttention in
 * ROCmKernels.Tests/AttentionTests.cpp:28-125, in plain C with the same arithmetic and order:
 *   - scores in double: dot(q, k) accumulated in double over the features, times scale = 1/sqrt(D)
 *     (AttentionTests.cpp:33,63-67);
 *   - maximum via `max = (max < s) ? s : max` starting at -inf (std::max, :51,68);
 *   - probabilities exp(s - max) in double, 0 when max is -inf; total in double (:71-75);
 *   - lse = {(float)max or -inf, (float)total} (:78-79);
 *   - output = (float)(sum_k p_k v_k / total) or 0 when total is not > 0, skipping p == 0 terms (:81-92);
 *   - delta = sum upstream * (float output) in double (:94-97);
 *   - per key with p != 0: probability = p/total, valueScore in double, derivative = probability*(valueScore - delta),
 *     and every gradient term is cast to float and accumulated in float in (batch, head, query, key, column)
 *     order (:99-119).
 * Masks follow :54 (key mask [batch][keys], shared across heads) and :57 (|query - key| > radius excluded when
 * radius >= 0). Two extensions, both exact restatements of visibility rather than new arithmetic:
 *   - causal (flags bit 0): key > query is excluded, as the extra predicate beside :57;
 *   - the key loop visits only the window [max(0, q - r), min(keys, q + r + 1)) (and key <= q when causal):
 *     keys outside it have score -inf and probability exactly 0 in the reference loop, so they add nothing.
 * Inputs are packed [batch][head][token][D], as the reference assumes (:48-49,61-62).
 *
 * The driver splits the work over `threads` POSIX threads: whole (batch, head) pairs when gradients are wanted, and
 * 64-query chunks of pairs for a forward only. Pairs are independent, query rows of a forward are too, and the float
 * gradient accumulation order within a pair is unchanged, so results are bit-identical for any thread count.
 *
 * Parity pins for this file live in tests/test_oracle.py (closed forms, invariants, finite differences, an
 * independent float64 matrix formulation, and torch float64 autograd fixtures in tests/golden/).
 */
#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

/* ORACLE_MUTATION plants one known mistake so tests/test_oracle.py can show that its pins catch it:
 * 1 drops the -delta term, 2 flips the sign of dK, 3 reads K in place of V for the output, 4 squares the scale.
 * Normal builds leave it at 0. */
#ifndef ORACLE_MUTATION
#define ORACLE_MUTATION 0
#endif

typedef struct {
    const float *q, *k, *v, *upstream;
    const uint8_t *mask;
    float *output, *lse, *gq, *gk, *gv, *delta;
    int width, batch, heads, queries, keys, radius, causal;
    int next; /* next task (a pair, or a query chunk of one), taken under the lock */
    pthread_mutex_t lock;
} Job;

static void key_window(const Job *job, const int query, int *first, int *last) {
    int lo = 0, hi = job->keys;
    if (job->radius >= 0) {
        lo = query - job->radius > 0 ? query - job->radius : 0;
        hi = query + job->radius + 1 < hi ? query + job->radius + 1 : hi;
    }
    if (job->causal && query + 1 < hi) hi = query + 1;
    if (hi < lo) hi = lo;
    *first = lo;
    *last = hi;
}

/* Queries [query_begin, query_end) of one (batch, head) pair. */
static void run_pair(const Job *job, const int batch, const int head, const int query_begin, const int query_end, double *scores,
        double *probabilities) {
    const int D = job->width;
    const double scale = 1.0 / sqrt((double)D);
    const size_t pair = (size_t)batch * job->heads + head;
    const float *q = job->q + pair * job->queries * D;
    const float *k = job->k + pair * job->keys * D;
    const float *v = job->v + pair * job->keys * D;
    const uint8_t *mask = job->mask + (size_t)batch * job->keys;

    for (int query = query_begin; query < query_end; ++query) {
        const float *qrow = q + (size_t)query * D;
        int first, last;
        key_window(job, query, &first, &last);

        double maximum = -INFINITY;
        for (int key = first; key < last; ++key) {
            scores[key] = -INFINITY;
            if (!mask[key]) continue;
            const float *krow = k + (size_t)key * D;
            double dot = 0;
            for (int c = 0; c < D; ++c) dot += (double)qrow[c] * krow[c];
            scores[key] = ORACLE_MUTATION == 4 ? dot * scale * scale : dot * scale;
            maximum = maximum < scores[key] ? scores[key] : maximum;
        }

        double total = 0;
        for (int key = first; key < last; ++key) {
            probabilities[key] = maximum == -INFINITY ? 0.0 : exp(scores[key] - maximum);
            total += probabilities[key];
        }

        const size_t row = pair * job->queries + query;
        if (job->lse) {
            job->lse[row * 2] = maximum == -INFINITY ? -INFINITY : (float)maximum;
            job->lse[row * 2 + 1] = (float)total;
        }

        float *orow = job->output + row * D;
        for (int c = 0; c < D; ++c) {
            double value = 0;
            for (int key = first; key < last; ++key) {
                if (probabilities[key] == 0.0) continue;
                value += probabilities[key] * (ORACLE_MUTATION == 3 ? k : v)[(size_t)key * D + c];
            }
            orow[c] = (float)(total > 0 ? value / total : 0.0);
        }

        if (!job->upstream) continue;
        const float *urow = job->upstream + row * D;
        double delta = 0;
        for (int c = 0; c < D; ++c) delta += (double)urow[c] * orow[c];
        if (job->delta) job->delta[row] = (float)delta;

        float *gqrow = job->gq + row * D;
        for (int key = first; key < last; ++key) {
            if (probabilities[key] == 0.0) continue;
            const float *krow = k + (size_t)key * D;
            const float *vrow = v + (size_t)key * D;
            const double probability = probabilities[key] / total;
            double value_score = 0;
            for (int c = 0; c < D; ++c) value_score += (double)urow[c] * vrow[c];
            const double derivative = probability * (value_score - (ORACLE_MUTATION == 1 ? 0.0 : delta));
            float *gkrow = job->gk + (pair * job->keys + key) * D;
            float *gvrow = job->gv + (pair * job->keys + key) * D;
            for (int c = 0; c < D; ++c) {
                gqrow[c] += (float)(derivative * krow[c] * scale);
                gkrow[c] += (float)((ORACLE_MUTATION == 2 ? -derivative : derivative) * qrow[c] * scale);
                gvrow[c] += (float)(probability * urow[c]);
            }
        }
    }
}

enum { kForwardChunk = 64 };

static void *worker(void *arg) {
    Job *job = (Job *)arg;
    double *scores = (double *)malloc(sizeof(double) * (size_t)job->keys);
    double *probabilities = (double *)malloc(sizeof(double) * (size_t)job->keys);
    if (!scores || !probabilities) {
        free(scores);
        free(probabilities);
        return (void *)1;
    }
    /* A task is a (pair, query chunk). The backward accumulates dK/dV over all queries of a pair, so it keeps one task
     * per pair (the float accumulation order of every gradient is then fixed); the forward's rows are independent and
     * are cut into chunks of kForwardChunk queries, which keeps every thread busy when pairs are fewer than threads or
     * not a multiple of them. */
    const int chunk = job->upstream ? job->queries : kForwardChunk;
    const int chunks = (job->queries + chunk - 1) / chunk;
    for (;;) {
        pthread_mutex_lock(&job->lock);
        const int task = job->next++;
        pthread_mutex_unlock(&job->lock);
        if (task >= job->batch * job->heads * chunks) break;
        const int pair = task / chunks, part = task % chunks;
        const int end = (part + 1) * chunk < job->queries ? (part + 1) * chunk : job->queries;
        run_pair(job, pair / job->heads, pair % job->heads, part * chunk, end, scores, probabilities);
    }
    free(scores);
    free(probabilities);
    return NULL;
}

/*
 * Forward (and, when upstream is non-NULL, backward) of FP32 attention with head width `width`.
 * output/lse/gradients/delta are packed and written in full; gradient buffers are zeroed first.
 * lse, delta may be NULL. Returns 0 on success, -1 on invalid arguments or allocation failure.
 */
int oracle_attention(const float *q, const float *k, const float *v, const uint8_t *mask, const float *upstream, int width,
        int batch, int heads, int queries, int keys, int radius, int causal, float *output, float *lse, float *gq, float *gk,
        float *gv, float *delta, int threads) {
    if (!q || !k || !v || !mask || !output || width <= 0 || batch <= 0 || heads <= 0 || queries <= 0 || keys <= 0) return -1;
    if (upstream && (!gq || !gk || !gv)) return -1;
    if (upstream) {
        const size_t qn = (size_t)batch * heads * queries * width, kn = (size_t)batch * heads * keys * width;
        for (size_t i = 0; i < qn; ++i) gq[i] = 0.0f;
        for (size_t i = 0; i < kn; ++i) {
            gk[i] = 0.0f;
            gv[i] = 0.0f;
        }
    }
    Job job = {q, k, v, upstream, mask, output, lse, gq, gk, gv, delta, width, batch, heads, queries, keys, radius, causal, 0,
            PTHREAD_MUTEX_INITIALIZER};
    if (threads < 1) threads = 1;
    const long long tasks = (long long)batch * heads * (upstream ? 1 : (queries + kForwardChunk - 1) / kForwardChunk);
    if (threads > tasks) threads = (int)tasks;
    pthread_t *pool = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
    if (!pool) return -1;
    int failed = 0, started = 0;
    for (int t = 1; t < threads; ++t) {
        if (pthread_create(&pool[t], NULL, worker, &job) != 0) break;
        ++started;
    }
    if (worker(&job) != NULL) failed = 1;
    for (int t = 1; t <= started; ++t) {
        void *result = NULL;
        pthread_join(pool[t], &result);
        if (result != NULL) failed = 1;
    }
    free(pool);
    return failed ? -1 : 0;
}
