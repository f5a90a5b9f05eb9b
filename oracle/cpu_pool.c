/*
 * CPU oracle: the worker pool behind the lut product's thread split
 * (cq_oracle.c's parallel(), the restatement of algo-tensor's
 * tensor.Parallel). TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Workers persist between products, spin briefly for the next one and then
 * sleep, so a split costs a wake-up of a few hundred nanoseconds while
 * products follow each other, as goroutines on spinning Ps do. A run of p
 * pieces uses the caller (piece 0) and workers 1 .. p-1 (piece w); the
 * caller returns once every one of them has checked in, so no worker is
 * still inside a run when the next one is published.
 */
#include <immintrin.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>

#include "oracle.h"

enum { MAX_WORKERS = 63, SPINS = 20000 };

static pthread_mutex_t g_mu = PTHREAD_MUTEX_INITIALIZER;
static pthread_cond_t g_cv = PTHREAD_COND_INITIALIZER;
static int g_workers;                 /* started, never stopped */
static _Atomic uint64_t g_word;       /* generation << 8 | pieces of the current run */
static _Atomic int g_checked;         /* workers done with the current run */
static uint64_t g_gen;                /* caller side */
static orc_piece_fn g_fn;             /* the run, written before g_word is published */
static void *g_ctx;
static int g_n;
static _Thread_local int t_worker;    /* nonzero on a pool thread */
static uint64_t g_seen0[MAX_WORKERS + 1]; /* worker w starts after generation g_seen0[w] */

static void piece(int w, int pieces) {
    g_fn(g_ctx, (int)((long long)g_n * w / pieces), (int)((long long)g_n * (w + 1) / pieces));
}

static void *worker(void *arg) {
    const int w = (int)(intptr_t)arg;
    t_worker = 1;
    uint64_t seen = g_seen0[w]; /* the last run published before this worker was created */
    for (;;) {
        uint64_t wd;
        int spins = 0;
        while (((wd = atomic_load_explicit(&g_word, memory_order_acquire)) >> 8) == seen) {
            if (++spins < SPINS) {
                _mm_pause();
                continue;
            }
            pthread_mutex_lock(&g_mu);
            while ((atomic_load_explicit(&g_word, memory_order_acquire) >> 8) == seen) pthread_cond_wait(&g_cv, &g_mu);
            pthread_mutex_unlock(&g_mu);
            spins = 0;
        }
        seen = wd >> 8;
        const int pieces = (int)(wd & 0xff);
        if (w < pieces) {
            piece(w, pieces);
            atomic_fetch_add_explicit(&g_checked, 1, memory_order_release);
        }
    }
    return 0;
}

int orc_pool_reserve(int threads) {
    int want = threads - 1;
    if (want > MAX_WORKERS) want = MAX_WORKERS;
    while (g_workers < want) {
        pthread_t th;
        g_seen0[g_workers + 1] = g_gen; /* reserve runs between runs, on the caller's thread */
        if (pthread_create(&th, 0, worker, (void *)(intptr_t)(g_workers + 1))) return -1;
        pthread_detach(th);
        g_workers++;
    }
    return 0;
}

void orc_pool_run(int n, int pieces, orc_piece_fn fn, void *ctx) {
    if (pieces > g_workers + 1) pieces = g_workers + 1;
    if (pieces <= 1 || t_worker) {
        fn(ctx, 0, n);
        return;
    }
    g_fn = fn;
    g_ctx = ctx;
    g_n = n;
    atomic_store_explicit(&g_checked, 0, memory_order_relaxed);
    g_gen++;
    atomic_store_explicit(&g_word, g_gen << 8 | (uint64_t)pieces, memory_order_release);
    pthread_mutex_lock(&g_mu);
    pthread_cond_broadcast(&g_cv);
    pthread_mutex_unlock(&g_mu);
    piece(0, pieces);
    while (atomic_load_explicit(&g_checked, memory_order_acquire) < pieces - 1) _mm_pause();
}
